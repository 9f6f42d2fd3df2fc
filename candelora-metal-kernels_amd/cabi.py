"""ctypes binding of the C ABI in include/cmk_iq2.h (libcmk_iq2.so).

This is the binding a Python caller of the library uses; the Rust crate's
equivalent is the `extern "C"` block in src/hip/ffi.rs.
Loading fails loudly when the library has not been built: there is no CPU or
PyTorch fallback behind this module.
"""

from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libcmk_iq2.so")

CMK_OK = 0
CMK_ERR_INVALID_ARGUMENT = -1
CMK_ERR_UNSUPPORTED = -2
CMK_ERR_HIP = -3
CMK_ERR_NO_DEVICE = -4

CMK_F32, CMK_F16, CMK_BF16 = 0, 1, 2
CMK_IQ2_XXS, CMK_IQ2_XS, CMK_IQ2_S, CMK_IQ3_S = 0, 1, 2, 3
CMK_ACT_QUANT_OFF, CMK_ACT_QUANT_W8A8, CMK_ACT_QUANT_W4A8 = 0, 1, 2

# Every symbol include/cmk_iq2.h declares (checked by tests/test_abi.py).
EXPORTED = (
    "cmk_iq2_matmul",
    "cmk_iq2_matmul_noalloc",
    "cmk_iq2_matmul_workspace_size",
    "cmk_iq2_dequantize",
    "cmk_iq2_split_gguf_blocks",
    "cmk_swiglu",
    "cmk_iq2_matmul_swiglu",
    "cmk_last_error",
    "cmk_abi_version",
    "cmk_iq2_matmul_path",
    "cmk_device_count",
    "cmk_set_device",
    "cmk_device_props",
    "cmk_malloc",
    "cmk_free",
    "cmk_memcpy_htod",
    "cmk_memcpy_dtoh",
    "cmk_memset",
    "cmk_stream_create",
    "cmk_stream_destroy",
    "cmk_stream_synchronize",
    "cmk_device_synchronize",
    "cmk_event_create",
    "cmk_event_destroy",
    "cmk_event_record",
    "cmk_event_elapsed_ms",
)


class CmkError(RuntimeError):
    """A non-zero cmk_status, carrying cmk_last_error()'s message."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python candelora-metal-kernels_amd/build.py` "
            "(the IQ2_XXS path has no fallback)")
    L = ctypes.CDLL(LIB_PATH)
    P, S, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    L.cmk_iq2_matmul.argtypes = [P, I, S, S, P, S, P, S, S, S, I, I, I, P, P, S, P]
    L.cmk_iq2_matmul.restype = I
    L.cmk_iq2_matmul_noalloc.argtypes = [P, I, S, S, P, S, P, S, S, S, I, I, I, P, P]
    L.cmk_iq2_matmul_noalloc.restype = I
    L.cmk_iq2_matmul_workspace_size.argtypes = [I, S, S, S, I, I, ctypes.POINTER(S)]
    L.cmk_iq2_matmul_workspace_size.restype = I
    L.cmk_iq2_dequantize.argtypes = [P, S, P, S, S, S, I, I, P, P]
    L.cmk_iq2_split_gguf_blocks.argtypes = [P, S, S, I, P, S, P, S, P]
    L.cmk_iq2_split_gguf_blocks.restype = I
    L.cmk_swiglu.argtypes = [P, P, S, I, P, P]
    L.cmk_swiglu.restype = I
    L.cmk_iq2_matmul_swiglu.argtypes = [P, I, S, S, P, S, P, S, S, S, P, S, P, P, S, P]
    L.cmk_iq2_matmul_swiglu.restype = I
    L.cmk_iq2_dequantize.restype = I
    L.cmk_last_error.argtypes = []
    L.cmk_last_error.restype = ctypes.c_char_p
    L.cmk_abi_version.restype = I
    L.cmk_iq2_matmul_path.argtypes = [I, S, S, S, I]
    L.cmk_iq2_matmul_path.restype = I
    L.cmk_device_count.argtypes = [ctypes.POINTER(I)]
    L.cmk_set_device.argtypes = [I]
    L.cmk_device_props.argtypes = [ctypes.c_char_p, S, ctypes.POINTER(I), ctypes.POINTER(S),
                                   ctypes.POINTER(I), ctypes.POINTER(I)]
    L.cmk_malloc.argtypes = [ctypes.POINTER(P), S]
    L.cmk_free.argtypes = [P]
    L.cmk_memcpy_htod.argtypes = [P, P, S, P]
    L.cmk_memcpy_dtoh.argtypes = [P, P, S, P]
    L.cmk_memset.argtypes = [P, I, S, P]
    L.cmk_stream_create.argtypes = [ctypes.POINTER(P)]
    L.cmk_stream_destroy.argtypes = [P]
    L.cmk_stream_synchronize.argtypes = [P]
    L.cmk_event_create.argtypes = [ctypes.POINTER(P)]
    L.cmk_event_destroy.argtypes = [P]
    L.cmk_event_record.argtypes = [P, P]
    L.cmk_event_elapsed_ms.argtypes = [P, P, ctypes.POINTER(ctypes.c_float)]
    _lib = L
    return L


def last_error() -> str:
    return lib().cmk_last_error().decode()


def check(rc: int) -> None:
    if rc != CMK_OK:
        raise CmkError(rc, last_error())


def matmul_raw(x_ptr, x_dtype, x_len, m, wb_ptr, wb_len, ws_ptr, ws_len, out_dim, in_dim,
               out_ptr, variant=CMK_IQ2_XXS, mode=CMK_ACT_QUANT_OFF, strict=False,
               workspace_ptr=None, workspace_bytes=0, stream=None) -> None:
    check(lib().cmk_iq2_matmul(x_ptr, x_dtype, x_len, m, wb_ptr, wb_len, ws_ptr, ws_len, out_dim,
                               in_dim, variant, mode, 1 if strict else 0, out_ptr, workspace_ptr,
                               workspace_bytes, stream))


def matmul_noalloc_raw(x_ptr, x_dtype, x_len, m, wb_ptr, wb_len, ws_ptr, ws_len, out_dim, in_dim,
                       out_ptr, variant=CMK_IQ2_XXS, mode=CMK_ACT_QUANT_OFF, strict=False,
                       stream=None) -> None:
    """cmk_iq2_matmul_noalloc: the library's own per-device scratch instead of a
    workspace argument (up to NOALLOC_SCRATCH_BYTES)."""
    check(lib().cmk_iq2_matmul_noalloc(x_ptr, x_dtype, x_len, m, wb_ptr, wb_len, ws_ptr, ws_len,
                                       out_dim, in_dim, variant, mode, 1 if strict else 0,
                                       out_ptr, stream))


NOALLOC_SCRATCH_BYTES = 32 << 20  # CMK_IQ2_NOALLOC_SCRATCH_BYTES


def workspace_size(x_dtype, m, out_dim, in_dim, variant=CMK_IQ2_XXS,
                   mode=CMK_ACT_QUANT_OFF) -> int:
    n = ctypes.c_size_t(0)
    check(lib().cmk_iq2_matmul_workspace_size(x_dtype, m, out_dim, in_dim, variant, mode,
                                              ctypes.byref(n)))
    return n.value


def split_gguf_raw(blocks_ptr, blocks_len, n_blocks, variant, wb_ptr, wb_len, ws_ptr, ws_len,
                   stream=None) -> None:
    check(lib().cmk_iq2_split_gguf_blocks(blocks_ptr, blocks_len, n_blocks, variant, wb_ptr,
                                          wb_len, ws_ptr, ws_len, stream))


def swiglu_raw(gate_ptr, up_ptr, n, out_ptr, out_dtype=CMK_F32, stream=None) -> None:
    check(lib().cmk_swiglu(gate_ptr, up_ptr, n, out_dtype, out_ptr, stream))


def matmul_swiglu_raw(x_ptr, x_dtype, x_len, m, wb_ptr, wb_len, ws_ptr, ws_len, out_dim, in_dim,
                      gate_ptr, gate_len, out_ptr, workspace_ptr=None, workspace_bytes=0,
                      stream=None) -> None:
    check(lib().cmk_iq2_matmul_swiglu(x_ptr, x_dtype, x_len, m, wb_ptr, wb_len, ws_ptr, ws_len,
                                      out_dim, in_dim, gate_ptr, gate_len, out_ptr, workspace_ptr,
                                      workspace_bytes, stream))


def dequantize_raw(wb_ptr, wb_len, ws_ptr, ws_len, out_dim, in_dim, out_ptr,
                   out_dtype=CMK_F16, variant=CMK_IQ2_XXS, stream=None) -> None:
    check(lib().cmk_iq2_dequantize(wb_ptr, wb_len, ws_ptr, ws_len, out_dim, in_dim, variant,
                                   out_dtype, out_ptr, stream))


def matmul_path(x_dtype, m, out_dim, in_dim, mode=CMK_ACT_QUANT_OFF) -> str:
    return "gemm" if lib().cmk_iq2_matmul_path(x_dtype, m, out_dim, in_dim, mode) == 1 else "gemv"


def device_props() -> dict:
    name = ctypes.create_string_buffer(256)
    cu, mclk, bus = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
    lds = ctypes.c_size_t(0)
    check(lib().cmk_device_props(name, 256, ctypes.byref(cu), ctypes.byref(lds), ctypes.byref(mclk),
                                 ctypes.byref(bus)))
    return {"name": name.value.decode(), "cu_count": cu.value, "lds_bytes": lds.value,
            "mem_clock_khz": mclk.value, "mem_bus_bits": bus.value}


class Event:
    """A HIP event created through the C ABI (timing on any stream)."""

    def __init__(self):
        h = ctypes.c_void_p()
        check(lib().cmk_event_create(ctypes.byref(h)))
        self.h = h

    def record(self, stream=None):
        check(lib().cmk_event_record(self.h, stream))

    def elapsed_ms(self, later: "Event") -> float:
        ms = ctypes.c_float(0)
        check(lib().cmk_event_elapsed_ms(self.h, later.h, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.h:
                lib().cmk_event_destroy(self.h)
        except Exception:
            pass
