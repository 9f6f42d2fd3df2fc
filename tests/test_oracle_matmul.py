"""Pins the oracle's matmul and dequantisation.

  * dequantize: every element equals the closed form +-d*(2s+1)*g/8, evaluated in
    exact rational arithmetic from the raw bytes with the reference's table
    values (tests/golden/reference_tables.json); special cases d = 0, scale
    nibble 0, codebook index 0 and subnormal d;
  * f16 / bf16 dequantisation = one RNE rounding of the exact value;
  * matmul: a one-hot x = e_k returns column k of the dequantised weights
    exactly; numpy float64 matmul with the dequantised matrix agrees within the
    fp32 summation bound K*2^-23*sum|x*w|; the fp64 helper agrees to 1e-12;
    padding columns of a partial final block never contribute;
  * the committed golden outputs of the reference's in-test cases are reproduced.
"""

import json
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

from conftest import REPO

TABLES = json.load(open(os.path.join(REPO, "tests", "golden", "reference_tables.json")))
CASES = json.load(open(os.path.join(REPO, "tests", "golden", "reference_cases.json")))
GRID = [int(v, 16) for v in TABLES["iq2xxs_grid"]]
KSIGNS = TABLES["ksigns_iq2xs"]


def closed_form(wb, ws, out_dim, in_dim):
    """Exact rational dequantised weights from the format definition."""
    bpr = -(-in_dim // 256)
    out = [[None] * in_dim for _ in range(out_dim)]
    for n in range(out_dim):
        for c in range(in_dim):
            blk, lc = divmod(c, 256)
            b = n * bpr + blk
            dbits = int(ws[2 * b]) | (int(ws[2 * b + 1]) << 8)
            d = Fraction(float(np.array([dbits], np.uint16).view(np.float16)[0]))
            ib32, w = divmod(lc, 32)
            g, j = divmod(w, 8)
            base = b * 64 + ib32 * 8
            aux_g = int.from_bytes(bytes(wb[base:base + 4]), "little")
            aux_s = int.from_bytes(bytes(wb[base + 4:base + 8]), "little")
            s = aux_s >> 28
            mag = (GRID[(aux_g >> (8 * g)) & 0xFF] >> (8 * j)) & 0xFF
            neg = (KSIGNS[(aux_s >> (7 * g)) & 0x7F] >> j) & 1
            v = d * (2 * s + 1) * mag / 8
            out[n][c] = -v if neg else v
    return out


def _rand_weights(rng, out_dim, in_dim, d_scale=1e-3):
    bpr = -(-in_dim // 256)
    nb = out_dim * bpr
    wb = rng.integers(0, 256, nb * 64, dtype=np.uint8)
    d = (np.abs(rng.standard_normal(nb)) * d_scale).astype(np.float16)
    return wb, d.view(np.uint8).copy()


@pytest.mark.parametrize("out_dim,in_dim", [(3, 320), (2, 256), (1, 41)])
def test_dequant_closed_form_exact(oracle, out_dim, in_dim):
    rng = np.random.default_rng(out_dim * 1000 + in_dim)
    wb, ws = _rand_weights(rng, out_dim, in_dim, d_scale=1.0)
    got = oracle.dequantize_f32(wb, ws, out_dim, in_dim)
    ref = closed_form(wb, ws, out_dim, in_dim)
    for n in range(out_dim):
        for c in range(in_dim):
            assert Fraction(float(got[n, c])) == ref[n][c], (n, c)


def test_dequant_special_cases(oracle):
    wb = np.zeros(64, np.uint8)
    ws = np.zeros(2, np.uint8)
    assert np.all(oracle.dequantize_f32(wb, ws, 1, 256) == 0)  # d = 0
    ws = np.array([0x00, 0x3C], np.uint8)  # d = 1.0; codes 0, signs 0, scale 0
    v = oracle.dequantize_f32(wb, ws, 1, 256)
    assert np.all(v == np.float32(8 * 1 / 8))  # grid 0 = all 8s, dl = d/8
    ws = np.array([0x01, 0x00], np.uint8)  # smallest subnormal d = 2^-24
    wb2 = wb.copy()
    wb2[7] = 0xF0  # sub-block 0: scale nibble 15 -> (2s+1) = 31
    v = oracle.dequantize_f32(wb2, ws, 1, 256)
    assert v[0, 0] == np.float32(2.0 ** -24 * 31 * 8 / 8)
    assert v[0, 32] == np.float32(2.0 ** -24 * 1)


def test_dequant_f16_bf16_are_single_rne(oracle):
    rng = np.random.default_rng(3)
    wb, ws = _rand_weights(rng, 9, 512)
    f32 = oracle.dequantize_f32(wb, ws, 9, 512)
    assert np.array_equal(oracle.dequantize_f16_bits(wb, ws, 9, 512),
                          f32.astype(np.float16).view(np.uint16))
    bf = torch.from_numpy(f32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.dequantize_bf16_bits(wb, ws, 9, 512), bf)


@pytest.mark.parametrize("k", [0, 1, 7, 8, 31, 32, 255, 256, 300, 319])
def test_matmul_one_hot_returns_column(oracle, k):
    rng = np.random.default_rng(11)
    wb, ws = _rand_weights(rng, 5, 320, d_scale=1.0)
    x = np.zeros((1, 320), np.float32)
    x[0, k] = 1.0
    y = oracle.matmul_reference(x, 1, 5, 320, wb, ws)
    col = oracle.dequantize_f32(wb, ws, 5, 320)[:, k]
    assert np.array_equal(y[0], col)


@pytest.mark.parametrize("m,out_dim,in_dim", [(2, 7, 320), (3, 16, 1024), (1, 33, 4096)])
def test_matmul_vs_numpy_f64(oracle, m, out_dim, in_dim):
    rng = np.random.default_rng(in_dim)
    wb, ws = _rand_weights(rng, out_dim, in_dim)
    x = rng.standard_normal((m, in_dim)).astype(np.float32)
    y = oracle.matmul_reference(x, m, out_dim, in_dim, wb, ws)
    w = oracle.dequantize_f32(wb, ws, out_dim, in_dim).astype(np.float64)
    y64 = x.astype(np.float64) @ w.T
    bound = in_dim * 2.0 ** -23 * (np.abs(x.astype(np.float64)) @ np.abs(w).T)
    assert np.all(np.abs(y - y64) <= bound + 1e-30)
    f64, sc = oracle.matmul_f64(x, m, out_dim, in_dim, wb, ws)
    assert np.allclose(f64, y64, rtol=1e-12, atol=1e-12 * np.max(sc))
    assert np.allclose(sc, np.abs(x.astype(np.float64)) @ np.abs(w).T, rtol=1e-12)


def test_padding_columns_never_contribute(oracle):
    rng = np.random.default_rng(5)
    wb, ws = _rand_weights(rng, 4, 300)  # bpr = 2, second block covers cols 256..511
    x = rng.standard_normal((2, 300)).astype(np.float32)
    y = oracle.matmul_reference(x, 2, 4, 300, wb, ws)
    wb2 = wb.copy()
    for n in range(4):
        blk = n * 2 + 1
        # sub-blocks 2..7 of the partial block (cols >= 320) and the tail of sub-block 1
        wb2[blk * 64 + 16: blk * 64 + 64] = rng.integers(0, 256, 48, dtype=np.uint8)
    assert np.array_equal(y, oracle.matmul_reference(x, 2, 4, 300, wb2, ws))


def test_w8a8_is_reference_on_qdq(oracle):
    rng = np.random.default_rng(9)
    wb, ws = _rand_weights(rng, 6, 512)
    x = (rng.standard_normal((3, 512)) * 4).astype(np.float32)
    a = oracle.matmul_reference_w8a8(x, 3, 6, 512, wb, ws)
    b = oracle.matmul_reference(oracle.rowwise_qdq_w8a8(x, 3, 512), 3, 6, 512, wb, ws)
    assert np.array_equal(a, b)


def test_mt_baseline_is_bit_identical(oracle):
    rng = np.random.default_rng(2)
    wb, ws = _rand_weights(rng, 64, 768)
    x = rng.standard_normal((2, 768)).astype(np.float32)
    a = oracle.matmul_reference(x, 2, 64, 768, wb, ws)
    b, used = oracle.matmul_reference_mt(x, 2, 64, 768, wb, ws, threads=4)
    assert used >= 1
    assert np.array_equal(a, b)


def test_golden_reference_cases(oracle):
    pc = CASES["parity_case"]
    x, wb, ws = oracle.reference_case_inputs(pc["m"], pc["out_dim"], pc["in_dim"],
                                             pc["bytes_seed"], pc["scales_seed"], pc["tail"])
    y = oracle.matmul_reference(x, pc["m"], pc["out_dim"], pc["in_dim"], wb, ws)
    assert list(y.view(np.uint32).ravel()) == pc["out_f32_bits"]
    yq = oracle.matmul_reference_w8a8(x, pc["m"], pc["out_dim"], pc["in_dim"], wb, ws)
    assert list(yq.view(np.uint32).ravel()) == pc["out_w8a8_f32_bits"]
    sm = CASES["w8a8_smoke_case"]
    x, wb, ws = oracle.reference_case_inputs(sm["m"], sm["out_dim"], sm["in_dim"],
                                             sm["bytes_seed"], sm["scales_seed"], sm["tail"])
    yq = oracle.matmul_reference_w8a8(x, sm["m"], sm["out_dim"], sm["in_dim"], wb, ws)
    assert list(yq.view(np.uint32).ravel()) == sm["out_w8a8_f32_bits"]
    assert np.all(np.isfinite(yq))


def test_package_generator_matches_oracle_reference_case(oracle, inputs):
    x1, wb1, ws1 = oracle.reference_case_inputs()
    x2, wb2, ws2 = inputs.reference_case()
    assert np.array_equal(x1, x2) and np.array_equal(wb1, wb2) and np.array_equal(ws1, ws2)


def test_synthetic_generator_properties(inputs):
    wb, ws = inputs.synthetic_weights(64, 4096)
    assert wb.size == 64 * 16 * 64 and ws.size == 64 * 16 * 2
    d = ws.view(np.float16).astype(np.float64)
    assert np.all(d >= 0)
    assert 0.6e-3 < d.mean() < 1.0e-3  # E|N(0,1)| * 1e-3 = 0.798e-3
    frac_sub = np.mean(d < 6.103515625e-05)
    assert 0.02 < frac_sub < 0.08  # ~4.9% fp16-subnormal d
    aux_s = wb.view(np.uint32)[1::2]
    scales = aux_s >> 28
    assert set(np.unique(scales)) == set(range(16))
    x = inputs.synthetic_x(4, 4096)
    assert abs(float(x.mean())) < 0.05 and 0.95 < float(x.std()) < 1.05
    # deterministic: same seed, same bytes; different seed, different bytes
    assert np.array_equal(inputs.synthetic_weights(64, 4096)[0], wb)
    assert not np.array_equal(inputs.synthetic_weights(64, 4096, seed=1)[0], wb)
