"""TEST INFRASTRUCTURE ONLY: ctypes wrapper around the C oracle (iq2xxs_oracle.c).

The oracle is a CPU restatement of the reference crate's scalar CPU reference
for the IQ2_XXS matmul (src/iq2_matmul.rs:761-883, 1025-1063 of
Steboss/candelora-metal-kernels) and of the Metal element decode
(src/metal_src/iq2_matmul.metal:701-734, 868-887).  It is the checker for the
HIP kernels and the CPU baseline in bench.py.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this file.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "libiq2xxs_oracle.so")

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc, no FMA contraction)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        S = ctypes.c_size_t
        L.oracle_tables.argtypes = [P, P, P]
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = ctypes.c_float
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_lcg_fill.argtypes = [P, S, ctypes.c_uint32]
        L.oracle_deterministic_x.argtypes = [P, S]
        L.oracle_force_f16_one_per_block.argtypes = [P, S, S]
        L.oracle_iq2xxs_matmul_reference.argtypes = [P, S, S, S, P, P, P]
        L.oracle_iq2xxs_matmul_reference_mt.argtypes = [P, S, S, S, P, P, P, ctypes.c_int]
        L.oracle_iq2xxs_matmul_reference_mt.restype = ctypes.c_int
        L.oracle_rowwise_qdq_w8a8.argtypes = [P, S, S, P]
        L.oracle_iq2xxs_matmul_reference_w8a8.argtypes = [P, S, S, S, P, P, P]
        L.oracle_iq2xxs_dequantize_f32.argtypes = [P, P, S, S, P]
        L.oracle_iq2xxs_dequantize_f16.argtypes = [P, P, S, S, P]
        L.oracle_iq2xxs_dequantize_bf16.argtypes = [P, P, S, S, P]
        L.oracle_iq2xxs_matmul_f64.argtypes = [P, S, S, S, P, P, P, P]
        I = ctypes.c_int
        L.oracle_iq_bytes_per_block.argtypes = [I]
        L.oracle_iq_bytes_per_block.restype = S
        L.oracle_iq_scales_per_block.argtypes = [I]
        L.oracle_iq_scales_per_block.restype = S
        L.oracle_iq_grid.argtypes = [I, P]
        L.oracle_iq_grid.restype = S
        L.oracle_iq_matmul_reference.argtypes = [I, P, S, S, S, P, P, P]
        L.oracle_iq_matmul_reference_w8a8.argtypes = [I, P, S, S, S, P, P, P]
        L.oracle_iq_dequantize_f32.argtypes = [I, P, P, S, S, P]
        L.oracle_iq_dequantize_f16.argtypes = [I, P, P, S, S, P]
        L.oracle_iq_dequantize_bf16.argtypes = [I, P, P, S, S, P]
        L.oracle_iq_matmul_f64.argtypes = [I, P, S, S, S, P, P, P, P]
        L.oracle_gguf_block_bytes.argtypes = [I]
        L.oracle_gguf_block_bytes.restype = S
        L.oracle_gguf_to_split.argtypes = [I, P, S, P, P]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def tables():
    """(kmask[8] u8, ksigns[128] u8, grid[256] u64) as decoded by the oracle."""
    km = np.zeros(8, np.uint8)
    ks = np.zeros(128, np.uint8)
    gr = np.zeros(256, np.uint64)
    lib().oracle_tables(_p(km), _p(ks), _p(gr))
    return km, ks, gr


def f16_to_f32(h: int) -> float:
    return lib().oracle_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().oracle_f32_to_f16(f)


def f32_to_bf16(f: float) -> int:
    return lib().oracle_f32_to_bf16(f)


def lcg_fill(n: int, seed: int) -> np.ndarray:
    out = np.zeros(n, np.uint8)
    lib().oracle_lcg_fill(_p(out), n, seed & 0xFFFFFFFF)
    return out


def deterministic_x(n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    lib().oracle_deterministic_x(_p(out), n)
    return out


def force_f16_one_per_block(scales: np.ndarray, scales_per_block: int = 2) -> np.ndarray:
    s = np.array(scales, dtype=np.uint8, copy=True)
    lib().oracle_force_f16_one_per_block(_p(s), s.size, scales_per_block)
    return s


def matmul_reference(x, m, out_dim, in_dim, wb, ws) -> np.ndarray:
    x = _f32(x)
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((m, out_dim), np.float32)
    lib().oracle_iq2xxs_matmul_reference(_p(x), m, out_dim, in_dim, _p(wb), _p(ws), _p(out))
    return out


def matmul_reference_mt(x, m, out_dim, in_dim, wb, ws, threads=0):
    x = _f32(x)
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((m, out_dim), np.float32)
    used = lib().oracle_iq2xxs_matmul_reference_mt(
        _p(x), m, out_dim, in_dim, _p(wb), _p(ws), _p(out), threads)
    return out, used


def rowwise_qdq_w8a8(x, m, in_dim) -> np.ndarray:
    x = _f32(x)
    out = np.zeros((m, in_dim), np.float32)
    lib().oracle_rowwise_qdq_w8a8(_p(x), m, in_dim, _p(out))
    return out


def matmul_reference_w8a8(x, m, out_dim, in_dim, wb, ws) -> np.ndarray:
    x = _f32(x)
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((m, out_dim), np.float32)
    lib().oracle_iq2xxs_matmul_reference_w8a8(_p(x), m, out_dim, in_dim, _p(wb), _p(ws), _p(out))
    return out


def dequantize_f32(wb, ws, out_dim, in_dim) -> np.ndarray:
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((out_dim, in_dim), np.float32)
    lib().oracle_iq2xxs_dequantize_f32(_p(wb), _p(ws), out_dim, in_dim, _p(out))
    return out


def dequantize_f16_bits(wb, ws, out_dim, in_dim) -> np.ndarray:
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((out_dim, in_dim), np.uint16)
    lib().oracle_iq2xxs_dequantize_f16(_p(wb), _p(ws), out_dim, in_dim, _p(out))
    return out


def dequantize_bf16_bits(wb, ws, out_dim, in_dim) -> np.ndarray:
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((out_dim, in_dim), np.uint16)
    lib().oracle_iq2xxs_dequantize_bf16(_p(wb), _p(ws), out_dim, in_dim, _p(out))
    return out


def matmul_f64(x, m, out_dim, in_dim, wb, ws):
    """fp64-accumulated outputs and the per-output scale sum_k |x_k w_nk|."""
    x = _f32(x)
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((m, out_dim), np.float64)
    sc = np.zeros((m, out_dim), np.float64)
    lib().oracle_iq2xxs_matmul_f64(_p(x), m, out_dim, in_dim, _p(wb), _p(ws), _p(out), _p(sc))
    return out, sc


# ---- all four variants (iq_variants_oracle.c; variant 0 = IQ2_XXS) ----------

IQ2_XXS, IQ2_XS, IQ2_S, IQ3_S = 0, 1, 2, 3


def bytes_per_block(variant: int) -> int:
    return lib().oracle_iq_bytes_per_block(variant)


def scales_per_block(variant: int) -> int:
    return lib().oracle_iq_scales_per_block(variant)


def grid(variant: int) -> np.ndarray:
    """The variant's decoded codebook (u64 values; IQ3_S entries are u32)."""
    n = lib().oracle_iq_grid(variant, None)
    out = np.zeros(n, np.uint64)
    lib().oracle_iq_grid(variant, _p(out))
    return out


def variant_matmul_reference(variant, x, m, out_dim, in_dim, wb, ws) -> np.ndarray:
    x = _f32(x)
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((m, out_dim), np.float32)
    lib().oracle_iq_matmul_reference(variant, _p(x), m, out_dim, in_dim, _p(wb), _p(ws), _p(out))
    return out


def variant_matmul_reference_w8a8(variant, x, m, out_dim, in_dim, wb, ws) -> np.ndarray:
    x = _f32(x)
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((m, out_dim), np.float32)
    lib().oracle_iq_matmul_reference_w8a8(variant, _p(x), m, out_dim, in_dim, _p(wb), _p(ws),
                                          _p(out))
    return out


def variant_dequantize_f32(variant, wb, ws, out_dim, in_dim) -> np.ndarray:
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((out_dim, in_dim), np.float32)
    lib().oracle_iq_dequantize_f32(variant, _p(wb), _p(ws), out_dim, in_dim, _p(out))
    return out


def variant_dequantize_f16_bits(variant, wb, ws, out_dim, in_dim) -> np.ndarray:
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((out_dim, in_dim), np.uint16)
    lib().oracle_iq_dequantize_f16(variant, _p(wb), _p(ws), out_dim, in_dim, _p(out))
    return out


def variant_dequantize_bf16_bits(variant, wb, ws, out_dim, in_dim) -> np.ndarray:
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((out_dim, in_dim), np.uint16)
    lib().oracle_iq_dequantize_bf16(variant, _p(wb), _p(ws), out_dim, in_dim, _p(out))
    return out


def variant_matmul_f64(variant, x, m, out_dim, in_dim, wb, ws):
    x = _f32(x)
    wb, ws = _u8(wb), _u8(ws)
    out = np.zeros((m, out_dim), np.float64)
    sc = np.zeros((m, out_dim), np.float64)
    lib().oracle_iq_matmul_f64(variant, _p(x), m, out_dim, in_dim, _p(wb), _p(ws), _p(out), _p(sc))
    return out, sc


def gguf_block_bytes(variant: int) -> int:
    return lib().oracle_gguf_block_bytes(variant)


def gguf_to_split(variant, blocks, n_blocks):
    """ggml AoS blocks -> (weight_bytes, weight_scales) as the reference splits them."""
    blocks = _u8(blocks)
    wb = np.zeros(n_blocks * bytes_per_block(variant), np.uint8)
    ws = np.zeros(n_blocks * scales_per_block(variant), np.uint8)
    lib().oracle_gguf_to_split(variant, _p(blocks), n_blocks, _p(wb), _p(ws))
    return wb, ws


def reference_case_inputs(m=2, out_dim=7, in_dim=320, bytes_seed=0xA11CE5ED,
                          scales_seed=0xC0FFEE12, tail=0x5A):
    """Inputs of the reference's parity_case (src/iq2_matmul.rs:1071-1086):
    LCG weight bytes/scales, d forced to 1.0, last weight byte pinned, and
    deterministic_x.  w8a8_smoke_case uses seeds 0x0BADC0DE/0xD15EA5ED, tail 0xC3,
    out_dim 6 (:1136-1146)."""
    bpr = -(-in_dim // 256)
    nb = out_dim * bpr
    wb = lcg_fill(nb * 64, bytes_seed)
    ws = force_f16_one_per_block(lcg_fill(nb * 2, scales_seed), 2)
    if wb.size:
        wb[-1] = tail
    x = deterministic_x(m * in_dim).reshape(m, in_dim)
    return x, wb, ws
