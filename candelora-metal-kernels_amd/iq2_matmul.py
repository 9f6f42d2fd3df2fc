"""PyTorch-tensor binding of the IQ2 op, with the reference's signatures.

Mirrors the public functions of src/iq2_matmul.rs:535-670 (iq2_matmul,
iq2_matmul_with_activation_quant, iq2_dequantize_to_f16, iq2_xxs_matmul and the
xs/s/iq3_s wrappers) and their argument rules (:170-311): x is rank 1 ([K] ->
[N]) or rank 2 ([M, K] -> [M, N]) in f32/f16/bf16 and is made contiguous;
weight_bytes / weight_scales are contiguous uint8 tensors at least as large as
the format requires; the output is a fresh f32 tensor.  PyTorch only supplies
device memory and the current stream; all arithmetic runs in libcmk_iq2.so.
Errors raise Iq2MatmulError with the reference's message texts.
"""

from __future__ import annotations

import enum

import torch

from . import cabi
from .activation_quant import ActivationQuantConfig, ActivationQuantMode


class Iq2MatmulVariant(enum.IntEnum):
    Iq2Xxs = cabi.CMK_IQ2_XXS
    Iq2Xs = cabi.CMK_IQ2_XS
    Iq2S = cabi.CMK_IQ2_S
    Iq3S = cabi.CMK_IQ3_S


class Iq2MatmulError(RuntimeError):
    pass


_DTYPES = {torch.float32: cabi.CMK_F32, torch.float16: cabi.CMK_F16,
           torch.bfloat16: cabi.CMK_BF16}
_DTYPE_NAMES = {torch.float32: "F32", torch.float16: "F16", torch.bfloat16: "BF16",
                torch.uint8: "U8", torch.float64: "F64", torch.int64: "I64", torch.int32: "I32",
                torch.uint32: "U32"}


def _dtype_name(dt) -> str:
    return _DTYPE_NAMES.get(dt, str(dt))


def _stream(t: torch.Tensor):
    return ctypes_stream(torch.cuda.current_stream(t.device))


def ctypes_stream(s) -> int:
    return int(s.cuda_stream)


def _parse_x_shape(x: torch.Tensor, in_dim: int):
    # src/iq2_matmul.rs:170-195
    if x.dim() == 1:
        if x.shape[0] != in_dim:
            raise Iq2MatmulError(
                f"iq2_matmul input mismatch: x dim={x.shape[0]} expected in_dim={in_dim}")
        return x.reshape(1, in_dim), 1, True
    if x.dim() == 2:
        if x.shape[1] != in_dim:
            raise Iq2MatmulError(
                f"iq2_matmul input mismatch: x last dim={x.shape[1]} expected in_dim={in_dim}")
        return x, x.shape[0], False
    raise Iq2MatmulError(f"iq2_matmul expects x rank 1 or 2, got shape {list(x.shape)}")


def _check_weights(op: str, x, weight_bytes, weight_scales):
    if weight_bytes.dtype != torch.uint8 or weight_scales.dtype != torch.uint8:
        raise Iq2MatmulError(
            f"{op} expects U8 weight bytes/scales, got bytes={_dtype_name(weight_bytes.dtype)}, "
            f"scales={_dtype_name(weight_scales.dtype)}")
    if not weight_bytes.is_contiguous() or not weight_scales.is_contiguous():
        raise Iq2MatmulError(f"{op} expects contiguous layouts")


def _matmul(x, weight_bytes, weight_scales, out_dim, in_dim, variant, mode, strict=False):
    if out_dim == 0 or in_dim == 0:
        raise Iq2MatmulError("iq2_matmul expects non-zero dimensions")
    if x.device.type != "cuda":
        raise Iq2MatmulError("iq2_matmul requires a HIP device")
    if weight_bytes.device != x.device or weight_scales.device != x.device:
        raise Iq2MatmulError(
            f"iq2_matmul device mismatch: x={x.device}, bytes={weight_bytes.device}, "
            f"scales={weight_scales.device}")
    _check_weights("iq2_matmul", x, weight_bytes, weight_scales)
    x2, m, squeeze = _parse_x_shape(x, in_dim)
    x2 = x2.contiguous()
    if x2.dtype not in _DTYPES:
        name = "iq2_matmul_w8a8" if mode == ActivationQuantMode.W8A8 else "iq2_matmul"
        raise Iq2MatmulError(f"{name} unsupported x dtype: {_dtype_name(x2.dtype)}")
    out = torch.empty((m, out_dim), dtype=torch.float32, device=x.device)
    if m > 0:
        xd = _DTYPES[x2.dtype]
        ws_bytes = cabi.workspace_size(xd, m, out_dim, in_dim, int(variant), int(mode))
        work = (torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None)
        try:
            cabi.matmul_raw(x2.data_ptr(), xd, x2.numel(), m, weight_bytes.data_ptr(),
                            weight_bytes.numel(), weight_scales.data_ptr(), weight_scales.numel(),
                            out_dim, in_dim, out.data_ptr(), int(variant), int(mode), strict,
                            work.data_ptr() if work is not None else None, ws_bytes, _stream(x))
        except cabi.CmkError as e:
            raise Iq2MatmulError(str(e)) from None
    return out.squeeze(0) if squeeze else out


def iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, variant):
    """src/iq2_matmul.rs:536-553."""
    return _matmul(x, weight_bytes, weight_scales, out_dim, in_dim, variant,
                   ActivationQuantMode.Off)


def iq2_matmul_with_activation_quant(x, weight_bytes, weight_scales, out_dim, in_dim, variant,
                                     activation_quant: ActivationQuantConfig):
    """src/iq2_matmul.rs:559-591."""
    mode = activation_quant.mode
    if mode == ActivationQuantMode.W4A8:
        if activation_quant.strict:
            raise Iq2MatmulError(
                "activation quant mode W4A8 requested in strict mode, but W4A8 kernel path is "
                "not implemented yet")
        mode = ActivationQuantMode.Off
    return _matmul(x, weight_bytes, weight_scales, out_dim, in_dim, variant, mode)


def iq2_dequantize_to_f16(weight_bytes, weight_scales, out_dim, in_dim, variant,
                          out_dtype=torch.float16):
    """src/iq2_matmul.rs:594-602; out_dtype f16 as in the reference (bf16/f32 also accepted)."""
    if out_dim == 0 or in_dim == 0:
        raise Iq2MatmulError("iq2_dequantize_to_f16 expects non-zero dimensions")
    if weight_bytes.device.type != "cuda":
        raise Iq2MatmulError("iq2_dequantize_to_f16 requires a HIP device")
    if weight_scales.device != weight_bytes.device:
        raise Iq2MatmulError(
            f"iq2_dequantize_to_f16 device mismatch: bytes={weight_bytes.device}, "
            f"scales={weight_scales.device}")
    _check_weights("iq2_dequantize_to_f16", None, weight_bytes, weight_scales)
    out = torch.empty((out_dim, in_dim), dtype=out_dtype, device=weight_bytes.device)
    try:
        cabi.dequantize_raw(weight_bytes.data_ptr(), weight_bytes.numel(),
                            weight_scales.data_ptr(), weight_scales.numel(), out_dim, in_dim,
                            out.data_ptr(), _DTYPES[out_dtype], int(variant),
                            _stream(weight_bytes))
    except cabi.CmkError as e:
        raise Iq2MatmulError(str(e)) from None
    return out


# bytes / scales per 256-weight block (src/iq2_matmul.rs:13-29)
_BLOCK_SIZES = {Iq2MatmulVariant.Iq2Xxs: (64, 2), Iq2MatmulVariant.Iq2Xs: (64, 10),
                Iq2MatmulVariant.Iq2S: (72, 10), Iq2MatmulVariant.Iq3S: (104, 6)}


def iq2_split_gguf_blocks(blocks, variant):
    """GGUF (ggml) blocks -> (weight_bytes, weight_scales), the split pair the
    matmul and dequantisation take (src/iq2_matmul.rs:13-17).  `blocks` is a flat
    U8 device tensor of whole ggml blocks ({d; codes; scales}: 66, 74, 82 or 110
    bytes).  No counterpart in the reference, whose callers split the blocks
    themselves."""
    variant = Iq2MatmulVariant(variant)
    if blocks.device.type != "cuda":
        raise Iq2MatmulError("split_gguf_blocks requires a HIP device")
    if blocks.dtype != torch.uint8 or not blocks.is_contiguous():
        raise Iq2MatmulError("split_gguf_blocks expects a contiguous U8 tensor")
    cb, sb = _BLOCK_SIZES[variant]
    if blocks.numel() % (cb + sb):
        raise Iq2MatmulError(
            f"split_gguf_blocks: {blocks.numel()} bytes is not a whole number of "
            f"{cb + sb}-byte blocks")
    n = blocks.numel() // (cb + sb)
    wb = torch.empty(n * cb, dtype=torch.uint8, device=blocks.device)
    ws = torch.empty(n * sb, dtype=torch.uint8, device=blocks.device)
    try:
        cabi.split_gguf_raw(blocks.data_ptr(), blocks.numel(), n, int(variant), wb.data_ptr(),
                            wb.numel(), ws.data_ptr(), ws.numel(), _stream(blocks))
    except cabi.CmkError as e:
        raise Iq2MatmulError(str(e)) from None
    return wb, ws


def swiglu(gate, up, out_dtype=torch.float32):
    """h = silu(gate) * up elementwise (fp32 in, f32/f16/bf16 out): the step
    between the gate/up and the down projection.  No counterpart in the
    reference, whose callers compose it from candle ops."""
    if gate.device.type != "cuda" or up.device != gate.device:
        raise Iq2MatmulError("swiglu requires gate and up on one HIP device")
    if gate.dtype != torch.float32 or up.dtype != torch.float32:
        raise Iq2MatmulError("swiglu expects F32 gate and up")
    if gate.shape != up.shape or not gate.is_contiguous() or not up.is_contiguous():
        raise Iq2MatmulError("swiglu expects contiguous gate and up of one shape")
    out = torch.empty(gate.shape, dtype=out_dtype, device=gate.device)
    try:
        cabi.swiglu_raw(gate.data_ptr(), up.data_ptr(), gate.numel(), out.data_ptr(),
                        _DTYPES[out_dtype], _stream(gate))
    except cabi.CmkError as e:
        raise Iq2MatmulError(str(e)) from None
    return out


def iq2_matmul_swiglu(x, weight_bytes, weight_scales, out_dim, in_dim, gate):
    """silu(gate) * iq2_xxs_matmul(x, ...): the up projection of a gated MLP
    with the swiglu step in its epilogue, so the step needs no launch of its
    own.  Equal, bit for bit, to swiglu(gate, iq2_xxs_matmul(x, ...)).  gate is
    F32 shaped like the output ([out_dim] or [m, out_dim]); m <= 16.  No
    counterpart in the reference, whose callers
    compose the MLP from candle ops."""
    if x.device.type != "cuda" or gate.device != x.device:
        raise Iq2MatmulError("matmul_swiglu requires x and gate on one HIP device")
    if weight_bytes.device != x.device or weight_scales.device != x.device:
        raise Iq2MatmulError("matmul_swiglu requires the weights on the device of x")
    _check_weights("matmul_swiglu", x, weight_bytes, weight_scales)
    x2, m, squeeze = _parse_x_shape(x, in_dim)
    x2 = x2.contiguous()
    if x2.dtype not in _DTYPES:
        raise Iq2MatmulError(f"iq2_matmul unsupported x dtype: {_dtype_name(x2.dtype)}")
    if gate.dtype != torch.float32 or gate.numel() != m * out_dim:
        raise Iq2MatmulError("matmul_swiglu expects an F32 gate shaped like the output")
    g = gate.contiguous()
    out = torch.empty((m, out_dim), dtype=torch.float32, device=x.device)
    if m > 0:
        xd = _DTYPES[x2.dtype]
        # the workspace iq2_xxs_matmul takes (the multi-row kernel's split over
        # K), so that both run the same launch
        ws_bytes = cabi.workspace_size(xd, m, out_dim, in_dim)
        work = (torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None)
        try:
            cabi.matmul_swiglu_raw(x2.data_ptr(), xd, x2.numel(), m,
                                   weight_bytes.data_ptr(), weight_bytes.numel(),
                                   weight_scales.data_ptr(), weight_scales.numel(), out_dim,
                                   in_dim, g.data_ptr(), g.numel(), out.data_ptr(),
                                   work.data_ptr() if work is not None else None, ws_bytes,
                                   _stream(x))
        except cabi.CmkError as e:
            raise Iq2MatmulError(str(e)) from None
    return out.squeeze(0) if squeeze else out


def iq2_xxs_matmul(x, weight_bytes, weight_scales, out_dim, in_dim):
    return iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, Iq2MatmulVariant.Iq2Xxs)


def iq2_xs_matmul(x, weight_bytes, weight_scales, out_dim, in_dim):
    return iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, Iq2MatmulVariant.Iq2Xs)


def iq2_s_matmul(x, weight_bytes, weight_scales, out_dim, in_dim):
    return iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, Iq2MatmulVariant.Iq2S)


def iq3_s_matmul(x, weight_bytes, weight_scales, out_dim, in_dim):
    return iq2_matmul(x, weight_bytes, weight_scales, out_dim, in_dim, Iq2MatmulVariant.Iq3S)
