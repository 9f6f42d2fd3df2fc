"""Seeded synthetic IQ2_XXS inputs (numpy, vectorised, portable).

Two generators:

* The reference's own test/bench inputs: `lcg_fill` (src/iq2_matmul.rs:765-773,
  examples/iq2_matmul_bench.rs:215-223: state = state*1664525 + 1013904223 mod
  2^32, emit state >> 24), `deterministic_x` (src/iq2_matmul.rs:775-779) and
  `force_f16_one_per_block` (:781-787), restated here with a jump-ahead form of
  the LCG so large buffers are generated without a Python loop.

* The benchmark generator for the headline configurations: counter-based
  splitmix64 streams, so any slice can be generated independently:
    - per super-block: d = f16_rne(|z| * 1e-3), z ~ N(0,1) by Box-Muller in
      float64 from two draws of the "d" stream;
    - per 32-weight sub-block: one draw r of the "q" stream gives the four
      codebook indices (bytes 0..3 of r, uniform in 0..255), four 7-bit sign
      indices (bits 32+7i..38+7i, uniform in 0..127) and the 4-bit scale
      (bits 60..63, uniform in 0..15); aux_s = s0|s1<<7|s2<<14|s3<<21|scale<<28;
    - activations: z ~ N(0,1) (Box-Muller, cosine branch) as fp32 (or rounded
      to f16/bf16).
  Default seeds: weights 0x1D2C0FFE, activations 0x5EED.
"""

from __future__ import annotations

import numpy as np

QK = 256
BYTES_PER_BLOCK = 64
SCALES_PER_BLOCK = 2

WEIGHT_SEED = 0x1D2C0FFE
X_SEED = 0x5EED

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)


# ---------------------------------------------------------------- reference LCG

def lcg_fill(n: int, seed: int) -> np.ndarray:
    """u8[n] of the reference LCG.  state_i = A^i*seed + C*(A^i - 1)/(A - 1) computed
    as running products/sums in wrapping uint32 arithmetic."""
    if n == 0:
        return np.zeros(0, np.uint8)
    a = np.full(n, 1664525, dtype=np.uint32)
    with np.errstate(over="ignore"):
        apow = np.cumprod(a, dtype=np.uint32)  # A^(i+1)
        # sum_{k=0}^{i} A^k  = 1 + A + ... + A^i
        geo = np.empty(n, np.uint32)
        geo[0] = 1
        if n > 1:
            geo[1:] = np.cumsum(apow[:-1], dtype=np.uint32) + np.uint32(1)
        state = apow * np.uint32(seed & 0xFFFFFFFF) + np.uint32(1013904223) * geo
    return (state >> np.uint32(24)).astype(np.uint8)


def deterministic_x(n: int) -> np.ndarray:
    i = np.arange(n, dtype=np.int64)
    return ((((i * 17) % 41).astype(np.float32) - np.float32(20.0)) / np.float32(13.0)).astype(
        np.float32)


def force_f16_one_per_block(scales: np.ndarray, scales_per_block: int = SCALES_PER_BLOCK):
    s = np.array(scales, dtype=np.uint8, copy=True)
    nfull = (s.size // scales_per_block) * scales_per_block
    v = s[:nfull].reshape(-1, scales_per_block)
    v[:, 0] = 0x00
    v[:, 1] = 0x3C
    return s


def reference_case(m=2, out_dim=7, in_dim=320, bytes_seed=0xA11CE5ED, scales_seed=0xC0FFEE12,
                   tail=0x5A):
    """(x[m,in_dim] f32, weight_bytes u8, weight_scales u8) of the reference's
    parity_case (src/iq2_matmul.rs:1071-1086).  w8a8_smoke_case uses out_dim=6,
    seeds 0x0BADC0DE / 0xD15EA5ED and tail 0xC3 (:1136-1146)."""
    bpr = -(-in_dim // QK)
    nb = out_dim * bpr
    wb = lcg_fill(nb * BYTES_PER_BLOCK, bytes_seed)
    ws = force_f16_one_per_block(lcg_fill(nb * SCALES_PER_BLOCK, scales_seed))
    if wb.size:
        wb[-1] = tail
    x = deterministic_x(m * in_dim).reshape(m, in_dim)
    return x, wb, ws


def reference_bench_case(m, out_dim, in_dim):
    """Inputs of examples/iq2_matmul_bench.rs:257-273 (seeds xor'ed with the dims)."""
    return reference_case(m, out_dim, in_dim, bytes_seed=(0xA11CE5ED ^ out_dim) & 0xFFFFFFFF,
                          scales_seed=(0xC0FFEE12 ^ in_dim) & 0xFFFFFFFF)


# bytes of codes / scales per 256-weight block of each format (src/iq2_matmul.rs:13-29)
VARIANT_BLOCK_SIZES = {0: (64, 2), 1: (64, 10), 2: (72, 10), 3: (104, 6)}


def reference_bench_case_variant(variant, m, out_dim, in_dim):
    """examples/iq2_matmul_bench.rs:257-273 for any format: LCG codes and
    scales (seeds xor'ed with the dims) sized by the format's block sizes,
    every block's d = f16 1.0, the last code byte 0x5A, deterministic x."""
    bpb, spb = VARIANT_BLOCK_SIZES[variant]
    nb = out_dim * (-(-in_dim // QK))
    wb = lcg_fill(nb * bpb, (0xA11CE5ED ^ out_dim) & 0xFFFFFFFF)
    ws = force_f16_one_per_block(lcg_fill(nb * spb, (0xC0FFEE12 ^ in_dim) & 0xFFFFFFFF), spb)
    if wb.size:
        wb[-1] = 0x5A
    x = deterministic_x(m * in_dim).reshape(m, in_dim)
    return x, wb, ws


# ---------------------------------------------------------------- splitmix64

def splitmix64(seed: int, start: int, n: int) -> np.ndarray:
    """Outputs start .. start+n-1 of the splitmix64 sequence seeded with `seed`."""
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def _normal(seed: int, start: int, n: int) -> np.ndarray:
    r = splitmix64(seed, 2 * start, 2 * n)
    u1 = ((r[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53  # (0, 1]
    u2 = (r[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53          # [0, 1)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def _f32_to_f16_bits(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).view(np.uint16)  # numpy rounds to nearest even


def _f32_to_bf16_bits(v: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) & 0x8000 | 0x7FC0).astype(np.uint16)
    return r


def synthetic_weights(out_dim: int, in_dim: int, seed: int = WEIGHT_SEED):
    """(weight_bytes u8[out_dim*bpr*64], weight_scales u8[out_dim*bpr*2])."""
    bpr = -(-in_dim // QK)
    nb = out_dim * bpr
    d = (np.abs(_normal(seed ^ 0xD15C0DE5, 0, nb)) * 1e-3).astype(np.float32)
    scales = _f32_to_f16_bits(d).view(np.uint8)
    r = splitmix64(seed ^ 0x5EB10C5, 0, nb * 8)
    aux_g = (r & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    aux_s = (((r >> np.uint64(32)) & np.uint64(0x0FFFFFFF)) |
             (((r >> np.uint64(60)) & np.uint64(0xF)) << np.uint64(28))).astype(np.uint32)
    words = np.empty(nb * 16, np.uint32)
    words[0::2] = aux_g
    words[1::2] = aux_s
    return words.view(np.uint8).copy(), scales.copy()


def synthetic_x(m: int, in_dim: int, seed: int = X_SEED, dtype: str = "f32") -> np.ndarray:
    """Activations N(0,1): f32 array, or the uint16 bit patterns for 'f16'/'bf16'."""
    z = _normal(seed, 0, m * in_dim).astype(np.float32).reshape(m, in_dim)
    if dtype == "f32":
        return z
    if dtype == "f16":
        return _f32_to_f16_bits(z)
    if dtype == "bf16":
        return _f32_to_bf16_bits(z)
    raise ValueError(dtype)
