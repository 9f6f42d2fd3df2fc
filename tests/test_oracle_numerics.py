"""Pins the oracle's scalar building blocks against independent implementations:
IEEE conversions (numpy / torch), the reference LCG (a jump-ahead form and
hand-derived values), deterministic_x, and the W8A8 quant-dequant special cases."""

import numpy as np
import pytest
import torch


def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _edge_f32():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.996, 65520.0, 65536.0, 1e30, -1e30,
            2.0 ** -14, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -26, 3 * 2.0 ** -26,
            5.960464477539063e-08, 6.097555160522461e-05, 1.0009765625, 1.00048828125,
            1.0014648437500, 2049.0, 2051.0, float("inf"), float("-inf"), 1e-45]
    rng = np.random.default_rng(7)
    r = rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(
        -9, 6, 20000).astype(np.float32)
    ties = (np.arange(1, 2000, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10)
    return np.concatenate([np.array(vals, np.float32), r.astype(np.float32), ties])


def test_f32_to_f16_rne(oracle):
    v = _edge_f32()
    ref = v.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(x)) for x in v], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_f32_to_bf16_rne(oracle):
    v = _edge_f32()
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle.f32_to_bf16(float(x)) for x in v], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_lcg_matches_jump_ahead_and_hand_values(oracle, inputs):
    # Hand-derived: seed 0 -> state 1013904223 = 0x3C6EF35F -> first byte 0x3C.
    s = 0
    expect = []
    for _ in range(5):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        expect.append(s >> 24)
    assert expect[0] == 0x3C
    assert list(oracle.lcg_fill(5, 0)) == expect
    for seed in (0, 1, 0xA11CE5ED, 0xC0FFEE12, 0x0BADC0DE, 0xD15EA5ED, 0xFFFFFFFF):
        for n in (1, 2, 7, 1000, 40961):
            assert np.array_equal(oracle.lcg_fill(n, seed), inputs.lcg_fill(n, seed)), (seed, n)


def test_deterministic_x(oracle, inputs):
    n = 5000
    i = np.arange(n)
    ref = ((((i * 17) % 41).astype(np.float32) - np.float32(20)) / np.float32(13)).astype(
        np.float32)
    assert np.array_equal(oracle.deterministic_x(n), ref)
    assert np.array_equal(inputs.deterministic_x(n), ref)
    assert oracle.deterministic_x(1)[0] == np.float32(-20.0 / 13.0)


def test_force_f16_one(oracle, inputs):
    s = np.arange(11, dtype=np.uint8)  # trailing partial chunk stays untouched
    got = oracle.force_f16_one_per_block(s, 2)
    assert list(got) == [0, 0x3C] * 5 + [10]
    assert np.array_equal(inputs.force_f16_one_per_block(s, 2), got)


def _qdq_numpy(x):
    x = np.asarray(x, np.float32)
    mx = np.max(np.abs(x)) if x.size else np.float32(0)
    inv = np.float32(1.0) if mx < np.float32(1e-8) else np.float32(127.0) / np.float32(mx)
    t = (x * inv).astype(np.float32)
    q = (np.sign(t) * np.floor(np.abs(t) + np.float32(0.5))).astype(np.float32)  # half away
    q = np.clip(q, -127, 127).astype(np.float32)
    return (q / inv).astype(np.float32)


def test_qdq_special_cases(oracle):
    # inv = 1: ties must round away from zero (banker's rounding would differ)
    row = np.array([127.0, 0.5, -0.5, 1.5, -2.5, 63.5, -126.5, 0.0], np.float32)
    got = oracle.rowwise_qdq_w8a8(row, 1, row.size)[0]
    assert list(got) == [127.0, 1.0, -1.0, 2.0, -3.0, 64.0, -127.0, 0.0]
    # all-zero row -> inv 1 -> zeros; tiny row below 1e-8 -> inv 1 -> rounds to 0
    z = oracle.rowwise_qdq_w8a8(np.zeros(9, np.float32), 1, 9)[0]
    assert np.all(z == 0)
    tiny = oracle.rowwise_qdq_w8a8(np.full(4, 5e-9, np.float32), 1, 4)[0]
    assert np.all(tiny == 0)
    # +-max map to +-127/inv
    r = np.array([3.0, -3.0, 1.0], np.float32)
    g = oracle.rowwise_qdq_w8a8(r, 1, 3)[0]
    inv = np.float32(127.0) / np.float32(3.0)
    assert g[0] == np.float32(np.float32(127.0) / inv) and g[1] == -g[0]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_qdq_random_rows_match_numpy(oracle, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((4, 333)) * rng.uniform(0.01, 100, (4, 1))).astype(np.float32)
    got = oracle.rowwise_qdq_w8a8(x, 4, 333)
    for r in range(4):
        assert np.array_equal(got[r], _qdq_numpy(x[r]))
