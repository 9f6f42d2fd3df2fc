"""Pins the oracle's IQ2_XS / IQ2_S / IQ3_S restatement (oracle/iq_variants_oracle.c).

Checks, independent of the restatement's code:
  * codebooks: SHA-256 of the decoded little-endian images equal the digests
    recorded from the reference's table text (tests/golden/
    reference_variant_tables.json, src/metal_src/iq2_tables.metal:86-541);
    the values equal that fixture and, where /root/reference exists, the live
    text; value sets {8, 25, 43} / odd 1..15; ascending and unique; the kernels'
    compact copies (csrc/iq_variants_format.h) decode to the same tables;
  * dequantisation, one field at a time: a block of zero bytes with d = 1 is
    all ones (grid entry 0 is all 8s resp. all 1s, scale nibble 0); then a
    scale nibble, a codebook index (including its high bits) or a sign field is
    set at one position and exactly the columns that field governs change, to
    the value the format fixes (closed form with the fixture's grid bytes);
  * matmul: x = e_k gives column k of the dequantised matrix exactly; random x
    agrees with float64 x @ W^T to fp32 rounding, including a partial final
    super-block; W8A8 equals the plain reference on qdq(x).
"""

import hashlib
import json
import os
import re
import struct
from fractions import Fraction

import numpy as np
import pytest

from conftest import PKG_DIR, REPO

GOLDEN = os.path.join(REPO, "tests", "golden", "reference_variant_tables.json")
REF_TABLES = "/root/reference/src/metal_src/iq2_tables.metal"
XS, S, S3 = 1, 2, 3
NAMES = {XS: "iq2xs_grid", S: "iq2s_grid", S3: "iq3s_grid"}
SIZES = {XS: (64, 10), S: (72, 10), S3: (104, 6)}  # bytes / scales per block


def golden():
    return json.load(open(GOLDEN))


def image(v, values):
    fmt = "<I" if v == S3 else "<Q"
    return hashlib.sha256(b"".join(struct.pack(fmt, int(g)) for g in values)).hexdigest()


@pytest.mark.parametrize("v", [XS, S, S3])
def test_codebook_digest_and_values(oracle, v):
    g = golden()
    name = NAMES[v]
    vals = [int(t) for t in oracle.grid(v)]
    assert vals == [int(t, 16) for t in g[name]]
    assert image(v, vals) == g["sha256"][name]
    if os.path.exists(REF_TABLES):
        src = open(REF_TABLES).read()
        i = src.index(", %s," % name)
        j = src.index("\n", i)
        k = src.index("GGML_TABLE_END()", j)
        text = [int(t, 0) for t in re.split(r"[,\s]+", src[j:k]) if t.strip()]
        assert text == vals


@pytest.mark.parametrize("v", [XS, S, S3])
def test_codebook_invariants(oracle, v):
    vals = [int(t) for t in oracle.grid(v)]
    n = {XS: 512, S: 1024, S3: 512}[v]
    assert len(vals) == n and len(set(vals)) == n and vals == sorted(vals)
    nb, allowed = (4, set(range(1, 16, 2))) if v == S3 else (8, {8, 25, 43})
    for g in vals:
        assert {(g >> (8 * j)) & 0xFF for j in range(nb)} <= allowed
        assert g >> (8 * nb) == 0
    assert vals[0] == (0x01010101 if v == S3 else 0x0808080808080808)


def test_product_codebooks_match_oracle(oracle):
    src = open(os.path.join(PKG_DIR, "csrc", "iq_variants_format.h")).read()
    for v, macro in ((XS, "CMK_IQ2XS_GRID_CODES"), (S, "CMK_IQ2S_GRID_CODES"),
                     (S3, "CMK_IQ3S_GRID_CODES")):
        i = src.index("#define " + macro)
        j = src.find("\n\n", i)
        j = len(src) if j < 0 else j
        codes = [int(t, 16) for t in re.findall(r"0x[0-9a-fA-F]+", src[i:j])]
        dec = []
        for c in codes:
            val = 0
            if v == S3:
                for jj in range(4):
                    val |= (2 * ((c >> (3 * jj)) & 7) + 1) << (8 * jj)
            else:
                for jj in range(8):
                    val |= [8, 25, 43][(c >> (2 * jj)) & 3] << (8 * jj)
            dec.append(val)
        assert dec == [int(t) for t in oracle.grid(v)]


# ---- dequantisation, one field at a time -------------------------------------

ONE_F16 = (0x00, 0x3C)


def zero_block(v, d_bits=ONE_F16):
    bpb, spb = SIZES[v]
    wb = np.zeros(bpb, np.uint8)
    ws = np.zeros(spb, np.uint8)
    ws[0], ws[1] = d_bits
    return wb, ws


def dq(oracle, v, wb, ws):
    return oracle.variant_dequantize_f32(v, wb, ws, 1, 256)[0]


def grid_bytes(v, idx):
    g = int(golden()[NAMES[v]][idx], 16)
    return [(g >> (8 * j)) & 0xFF for j in range(4 if v == S3 else 8)]


def ksigns(i):
    return i | ((bin(i).count("1") & 1) << 7)


@pytest.mark.parametrize("v", [XS, S, S3])
def test_zero_block_is_all_ones(oracle, v):
    wb, ws = zero_block(v)
    assert np.all(dq(oracle, v, wb, ws) == 1.0)


@pytest.mark.parametrize("v", [XS, S, S3])
def test_scale_nibbles(oracle, v):
    """Nibble value 5 at each position scales exactly the columns it governs:
    IQ2 formats (0.5 + 5) / 4 * 8 = 11, IQ3_S (1 + 2 * 5) * 1 = 11."""
    positions = []
    if v in (XS, S):
        for ib32 in range(8):
            for half in range(2):  # low nibble: first 16 weights, high: last 16
                positions.append((2 + ib32, 4 * half, range(32 * ib32 + 16 * half,
                                                             32 * ib32 + 16 * half + 16)))
    else:
        for ib32 in range(8):
            positions.append((2 + ib32 // 2, 4 * (ib32 % 2), range(32 * ib32, 32 * ib32 + 32)))
    for byte, shift, cols in positions:
        wb, ws = zero_block(v)
        ws[byte] = 5 << shift
        got = dq(oracle, v, wb, ws)
        want = np.ones(256, np.float32)
        want[list(cols)] = 11.0
        assert np.array_equal(got, want), (byte, shift)


def test_iq2xs_index_and_sign_fields(oracle):
    rng = np.random.default_rng(1)
    for _ in range(40):
        ib32, w = int(rng.integers(8)), int(rng.integers(4))
        idx, si = int(rng.integers(512)), int(rng.integers(128))
        wb, ws = zero_block(XS)
        word = idx | (si << 9)
        wb[8 * ib32 + 2 * w] = word & 0xFF
        wb[8 * ib32 + 2 * w + 1] = word >> 8
        got = dq(oracle, XS, wb, ws)
        want = np.ones(256, np.float32)
        g, sg = grid_bytes(XS, idx), ksigns(si)
        for j in range(8):  # dl = (0.5 + 0) / 4 = 1/8
            want[32 * ib32 + 8 * w + j] = (g[j] / 8.0) * (-1.0 if (sg >> j) & 1 else 1.0)
        assert np.array_equal(got, want), (ib32, w, idx, si)


def test_iq2s_index_high_bits_and_signs(oracle):
    rng = np.random.default_rng(2)
    for _ in range(60):
        ib32, grp = int(rng.integers(8)), int(rng.integers(4))  # group = 8 weights
        idx, sbyte = int(rng.integers(1024)), int(rng.integers(256))
        wb, ws = zero_block(S)
        wb[4 * ib32 + grp] = idx & 0xFF          # qs: low byte of the index
        wb[64 + ib32] = (idx >> 8) << (2 * grp)   # qh: two high bits per group
        wb[32 + 4 * ib32 + grp] = sbyte           # sign byte of the group
        got = dq(oracle, S, wb, ws)
        want = np.ones(256, np.float32)
        g = grid_bytes(S, idx)
        for j in range(8):
            want[32 * ib32 + 8 * grp + j] = (g[j] / 8.0) * (-1.0 if (sbyte >> j) & 1 else 1.0)
        assert np.array_equal(got, want), (ib32, grp, idx, sbyte)


def test_iq3s_index_high_bits_and_signs(oracle):
    rng = np.random.default_rng(3)
    for _ in range(60):
        ib32, grp, half = int(rng.integers(8)), int(rng.integers(4)), int(rng.integers(2))
        idx, sbyte = int(rng.integers(512)), int(rng.integers(256))
        wb, ws = zero_block(S3)
        e = 2 * grp + half                       # entry of 4 weights within the sub-block
        wb[8 * ib32 + e] = idx & 0xFF             # qs: low byte
        wb[64 + ib32] = (idx >> 8) << e           # qh: one high bit per entry
        wb[72 + 4 * ib32 + grp] = sbyte           # one sign byte per group of 8
        got = dq(oracle, S3, wb, ws)
        want = np.ones(256, np.float32)
        g = grid_bytes(S3, idx)
        for j in range(8):  # the group's other entry stays at index 0 (all 1s)
            mag = g[j - 4 * half] if (j // 4) == half else 1
            want[32 * ib32 + 8 * grp + j] = mag * (-1.0 if (sbyte >> j) & 1 else 1.0)
        assert np.array_equal(got, want), (ib32, grp, half, idx, sbyte)


@pytest.mark.parametrize("v", [XS, S, S3])
def test_dequant_is_exact_product(oracle, v):
    """Random blocks: every value is d * (scale factor) * g with g from the
    fixture grid, i.e. exactly representable; f16/bf16 outputs are one RNE of
    it."""
    rng = np.random.default_rng(10 + v)
    bpb, spb = SIZES[v]
    nb = 2 * 3
    wb = rng.integers(0, 256, nb * bpb, dtype=np.uint8)
    ws = rng.integers(0, 256, nb * spb, dtype=np.uint8)
    for b in range(nb):  # finite d in a moderate range
        ws[b * spb + 1] = int(rng.integers(0x10, 0x40))
    f32 = oracle.variant_dequantize_f32(v, wb, ws, 3, 512)
    d = np.array([np.frombuffer(bytes(ws[b * spb:b * spb + 2]), np.float16)[0] for b in range(nb)])
    mags = {abs(float(t)) for t in f32.ravel()}
    allowed = set()
    levels = range(1, 16, 2) if v == S3 else (8, 25, 43)
    for dd in d:
        for nib in range(16):
            f = Fraction(float(dd)) * ((1 + 2 * nib) if v == S3 else Fraction(2 * nib + 1, 8))
            allowed.update(float(f * lv) for lv in levels)
    assert mags <= allowed
    f16 = oracle.variant_dequantize_f16_bits(v, wb, ws, 3, 512)
    assert np.array_equal(f16, f32.astype(np.float16).view(np.uint16))


# ---- matmul --------------------------------------------------------------------

def random_weights(v, out_dim, in_dim, seed):
    rng = np.random.default_rng(seed)
    bpb, spb = SIZES[v]
    nb = out_dim * (-(-in_dim // 256))
    wb = rng.integers(0, 256, nb * bpb, dtype=np.uint8)
    ws = rng.integers(0, 256, nb * spb, dtype=np.uint8)
    for b in range(nb):
        ws[b * spb] = int(rng.integers(256))
        ws[b * spb + 1] = int(rng.integers(0x10, 0x20))  # d ~ 1e-3 .. 1e-2
    return wb, ws


@pytest.mark.parametrize("v", [XS, S, S3])
def test_matmul_one_hot_columns(oracle, v):
    out_dim, in_dim = 5, 320
    wb, ws = random_weights(v, out_dim, in_dim, 20 + v)
    w = oracle.variant_dequantize_f32(v, wb, ws, out_dim, in_dim)
    for k in (0, 7, 31, 32, 255, 256, 319):
        x = np.zeros((1, in_dim), np.float32)
        x[0, k] = 1.0
        y = oracle.variant_matmul_reference(v, x, 1, out_dim, in_dim, wb, ws)
        assert np.array_equal(y[0], w[:, k]), k


@pytest.mark.parametrize("v", [XS, S, S3])
@pytest.mark.parametrize("in_dim", [512, 300])
def test_matmul_matches_float64(oracle, v, in_dim):
    m, out_dim = 3, 6
    wb, ws = random_weights(v, out_dim, in_dim, 30 + v + in_dim)
    x = np.random.default_rng(40 + v).standard_normal((m, in_dim)).astype(np.float32)
    y = oracle.variant_matmul_reference(v, x, m, out_dim, in_dim, wb, ws)
    w = oracle.variant_dequantize_f32(v, wb, ws, out_dim, in_dim).astype(np.float64)
    ref = x.astype(np.float64) @ w.T
    scale = np.abs(x).astype(np.float64) @ np.abs(w).T
    assert np.all(np.abs(y - ref) <= 1e-6 * scale + 1e-30)
    f64, sc = oracle.variant_matmul_f64(v, x, m, out_dim, in_dim, wb, ws)
    assert np.allclose(f64, ref, rtol=1e-12, atol=1e-12 * scale.max())
    assert np.allclose(sc, scale, rtol=1e-12)


@pytest.mark.parametrize("v", [XS, S, S3])
def test_matmul_w8a8_is_reference_on_qdq(oracle, v):
    m, out_dim, in_dim = 2, 4, 256
    wb, ws = random_weights(v, out_dim, in_dim, 50 + v)
    x = np.random.default_rng(60 + v).standard_normal((m, in_dim)).astype(np.float32)
    y = oracle.variant_matmul_reference_w8a8(v, x, m, out_dim, in_dim, wb, ws)
    xq = oracle.rowwise_qdq_w8a8(x, m, in_dim)
    assert np.array_equal(y, oracle.variant_matmul_reference(v, xq, m, out_dim, in_dim, wb, ws))


# ---- GGUF (ggml) block layout ----------------------------------------------------
# ggml's block structs (ggml-common.h, QK_K = 256), restated as numpy structured
# dtypes: the fp16 d first, then the codes, then the packed scales.
GGUF_DTYPES = {
    0: np.dtype([("d", "<u2"), ("qs", "u1", 64)]),
    XS: np.dtype([("d", "<u2"), ("qs", "u1", 64), ("scales", "u1", 8)]),
    S: np.dtype([("d", "<u2"), ("qs", "u1", 64), ("qh", "u1", 8), ("scales", "u1", 8)]),
    S3: np.dtype([("d", "<u2"), ("qs", "u1", 64), ("qh", "u1", 8), ("signs", "u1", 32),
                  ("scales", "u1", 4)]),
}


@pytest.mark.parametrize("v", [0, XS, S, S3])
def test_gguf_block_sizes(oracle, v):
    assert oracle.gguf_block_bytes(v) == GGUF_DTYPES[v].itemsize == {0: 66, XS: 74, S: 82,
                                                                      S3: 110}[v]
    assert oracle.gguf_block_bytes(v) == oracle.bytes_per_block(v) + oracle.scales_per_block(v)


@pytest.mark.parametrize("v", [0, XS, S, S3])
def test_gguf_split_fields(oracle, v):
    """d and the packed scales go to weight_scales (d first, as the reference's
    decoders read it, src/iq2_matmul.rs:857,888), the codes in struct order to
    weight_bytes; assembling the blocks back from the pair is the identity."""
    dt = GGUF_DTYPES[v]
    n = 37
    raw = np.random.default_rng(70 + v).integers(0, 256, n * dt.itemsize, dtype=np.uint8)
    rec = raw.view(dt)
    wb, ws = oracle.gguf_to_split(v, raw, n)
    codes = [f for f in dt.names if f not in ("d", "scales")]
    want_b = np.concatenate([np.concatenate([rec[f][i].ravel() for f in codes]) for i in range(n)])
    assert np.array_equal(wb, want_b)
    ws2 = ws.reshape(n, -1)
    assert np.array_equal(ws2[:, :2].copy().view("<u2").ravel(), rec["d"])
    if "scales" in dt.names:
        assert np.array_equal(ws2[:, 2:], rec["scales"])
    # inverse: rebuild the ggml blocks from the pair
    back = np.zeros(n, dt)
    back["d"] = ws2[:, :2].copy().view("<u2").ravel()
    off = 0
    wb2 = wb.reshape(n, -1)
    for f in codes:
        k = dt.fields[f][0].shape[0]
        back[f] = wb2[:, off:off + k]
        off += k
    if "scales" in dt.names:
        back["scales"] = ws2[:, 2:]
    assert np.array_equal(back.view(np.uint8), raw)
