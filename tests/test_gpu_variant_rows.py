"""GPU parity of the IQ2_XS / IQ2_S / IQ3_S matmuls on the multi-row decode
kernel (the one IQ2_XXS uses for 2..16 rows, with a format policy per variant),
and of all three at m = 1 on the one-row GEMV.

With weight_bytes 16-byte and weight_scales 2-byte aligned, every m runs
there, in launches of up to 16 activation rows (at m = 1 with K in whole
1024-column slices: the one-row GEMV).  The reference computes each
output on its own (iq2_matmul.metal:242-434, 501-699), so the bar is the
IQ2_XXS GEMV's: against the fp64 oracle product of the same x (W8A8: of the
fake-quantised x), cond <= 1e-5 and rel <= 1e-3 (definitions in
test_gpu_variants.py).  Shapes cover ragged 32-row groups, partial
super-blocks, K in several LDS slices, more row groups than workgroups,
unaligned x, more than 8 rows, and non-finite activations (output classes
exactly as the oracle's).
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from test_gpu_edges import NONFINITE, classes  # noqa: E402
from test_gpu_variants import errors, random_weights, to_dev, variant_enum  # noqa: E402

XS, S, S3 = 1, 2, 3
VARIANTS = [XS, S, S3]
NAMES = {XS: "iq2_xs", S: "iq2_s", S3: "iq3_s"}


@pytest.fixture(scope="module")
def dev(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg.cabi.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


def _x(m, in_dim, seed):
    return np.random.default_rng(seed).standard_normal((m, in_dim)).astype(np.float32)


def _check(pkg, oracle, v, xt, wb, ws, out_dim, in_dim, dev, w8a8=False):
    m = xt.shape[0]
    xf = xt.float().cpu().numpy()
    if w8a8:
        cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
        y = pkg.iq2_matmul_with_activation_quant(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim,
                                                 in_dim, variant_enum(pkg, v), cfg)
        xf = oracle.rowwise_qdq_w8a8(xf, m, in_dim)
    else:
        y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                           variant_enum(pkg, v))
    y = y.cpu().numpy()
    y64, sc = oracle.variant_matmul_f64(v, xf, m, out_dim, in_dim, wb, ws)
    cond, rel = errors(y, y64, sc)
    assert cond <= 1e-5 and rel <= 1e-3, (NAMES[v], m, out_dim, in_dim, cond, rel)
    return y


@pytest.mark.parametrize("v", VARIANTS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [1, 2, 5, 8, 12, 16, 21])
def test_variant_rows_ragged_shapes(pkg, oracle, dev, v, dtype, m):
    """1000 rows (the last 32-row group has 8), K = 2000 (a partial super-block);
    up to 16 activation rows per launch (21: a launch of 16 and one of 5)."""
    out_dim, in_dim = 1000, 2000
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 31 * v + m)
    xt = to_dev(_x(m, in_dim, 10 * v + m), dev).to(dtype)
    _check(pkg, oracle, v, xt, wb, ws, out_dim, in_dim, dev)


@pytest.mark.parametrize("v", VARIANTS)
@pytest.mark.parametrize("m,in_dim", [(8, 16384), (3, 14336), (1, 4096)])
def test_variant_rows_k_in_several_slices(pkg, oracle, dev, v, m, in_dim):
    """K beyond one LDS slice of digits (and the config-1 gate shape's K)."""
    out_dim = 512
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 7 * v + in_dim)
    xt = to_dev(_x(m, in_dim, v), dev)
    _check(pkg, oracle, v, xt, wb, ws, out_dim, in_dim, dev)


@pytest.mark.parametrize("v", VARIANTS)
def test_variant_rows_chunk_loop(pkg, oracle, dev, v):
    """More 32-row groups than 16 per workgroup on every CU: workgroups loop
    over chunks and keep their tables."""
    m, out_dim, in_dim = 3, 140000, 256
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 50 + v)
    xt = to_dev(_x(m, in_dim, 60 + v), dev)
    _check(pkg, oracle, v, xt, wb, ws, out_dim, in_dim, dev)


@pytest.mark.parametrize("v", VARIANTS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_variant_rows_unaligned_x_element_loads(pkg, oracle, dev, v, dtype):
    """x one element past a 16-byte boundary and K odd: activations are read
    element by element."""
    m, out_dim, in_dim = 6, 300, 1001
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 70 + v)
    x = to_dev(_x(m, in_dim, 80 + v), dev).to(dtype)
    big = torch.zeros(m * in_dim + 1, dtype=dtype, device=dev)
    big[1:] = x.reshape(-1)
    xt = big[1:].view(m, in_dim)
    assert xt.data_ptr() % 16 != 0
    _check(pkg, oracle, v, xt, wb, ws, out_dim, in_dim, dev)


@pytest.mark.parametrize("v", VARIANTS)
@pytest.mark.parametrize("m", [1, 4, 7, 20, 32, 40])
def test_variant_rows_w8a8(pkg, oracle, dev, v, m):
    """W8A8: int8 q, up to 32 rows per launch (40: 32 + 8)."""
    out_dim, in_dim = 777, 3000
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 90 + v + m)
    xt = to_dev(_x(m, in_dim, 95 + v + m), dev).to(torch.float16)
    _check(pkg, oracle, v, xt, wb, ws, out_dim, in_dim, dev, w8a8=True)


@pytest.mark.parametrize("v", VARIANTS)
def test_variant_rows_many_rows_in_groups_of_sixteen(pkg, oracle, dev, v):
    """m = 21: launches of 16 and 5 rows, each equal to the same rows
    multiplied on their own."""
    m, out_dim, in_dim = 21, 640, 1536
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 120 + v)
    x = _x(m, in_dim, 130 + v)
    y = _check(pkg, oracle, v, to_dev(x, dev), wb, ws, out_dim, in_dim, dev)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    for r0, r1 in ((0, 16), (16, 21)):
        yg = pkg.iq2_matmul(to_dev(x[r0:r1], dev), wbt, wst, out_dim, in_dim,
                            variant_enum(pkg, v)).cpu().numpy()
        assert np.array_equal(yg, y[r0:r1]), (r0, r1)


@pytest.mark.parametrize("v", VARIANTS)
@pytest.mark.parametrize("pattern", ["nan", "posinf", "both_inf", "inf_and_nan"])
def test_variant_rows_nonfinite_x(pkg, oracle, dev, v, pattern):
    """A NaN or infinite activation in row 0 of two: output classes as the
    oracle's (inf * a zero weight, d = 0, gives NaN), finite outputs to the bar."""
    m, out_dim, in_dim = 2, 1024, 4096
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 140 + v)
    spb = oracle.scales_per_block(v)
    bpr = in_dim // 256
    block = NONFINITE[pattern][0][0] // 256
    zero_rows = [3, 17, out_dim - 1]
    ws = ws.copy()
    for r in zero_rows:
        ws[spb * (r * bpr + block)] = 0
        ws[spb * (r * bpr + block) + 1] = 0
    x = _x(m, in_dim, 150 + v)
    for c, val in NONFINITE[pattern]:
        x[0, c] = val
    y = pkg.iq2_matmul(to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       variant_enum(pkg, v)).cpu().numpy()
    ref = oracle.variant_matmul_reference(v, x, m, out_dim, in_dim, wb, ws)
    assert np.array_equal(classes(y), classes(ref)), pattern
    if pattern == "posinf":
        assert np.all(np.isnan(y[0, zero_rows]))
    fin = classes(ref) == 0
    y64, sc = oracle.variant_matmul_f64(v, np.where(np.isfinite(x), x, 0.0).astype(np.float32), m,
                                        out_dim, in_dim, wb, ws)
    cond, rel = errors(y[fin], y64[fin], sc[fin])
    assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)


# ----------------- IQ2_XS, IQ2_S and IQ3_S at m = 1: the one-row GEMV
# (K in whole 1024-column slices, 16-byte aligned x, weight_scales 4-byte and
# weight_bytes 16-byte (IQ2_XS) / 8-byte aligned)

@pytest.mark.parametrize("v", [XS, S, S3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("out_dim,in_dim", [(14336, 4096), (4096, 14336), (777, 3072)])
def test_one_row_vs_oracle(pkg, oracle, dev, v, dtype, out_dim, in_dim):
    """BASELINE config 1's gate/up and down shapes, and a ragged row count."""
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 160 + v + in_dim % 97)
    xt = to_dev(_x(1, in_dim, 170 + out_dim % 89), dev).to(dtype)
    _check(pkg, oracle, v, xt, wb, ws, out_dim, in_dim, dev)


@pytest.mark.parametrize("v", [XS, S, S3])
def test_one_row_w8a8(pkg, oracle, dev, v):
    out_dim, in_dim = 2048, 4096
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 181 + v)
    xt = to_dev(_x(1, in_dim, 182), dev)
    _check(pkg, oracle, v, xt, wb, ws, out_dim, in_dim, dev, w8a8=True)


@pytest.mark.parametrize("v", [XS, S, S3])
@pytest.mark.parametrize("pattern", ["nan", "posinf", "both_inf", "inf_and_nan"])
def test_one_row_nonfinite_x(pkg, oracle, dev, v, pattern):
    """A NaN or an infinity in x at m = 1: output classes exactly the
    oracle's (inf times a zero weight, d = 0, gives NaN)."""
    m, out_dim, in_dim = 1, 1024, 4096
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 190 + v)
    spb = oracle.scales_per_block(v)
    bpr = in_dim // 256
    block = NONFINITE[pattern][0][0] // 256
    zero_rows = [3, 17, out_dim - 1]
    ws = ws.copy()
    for r in zero_rows:
        ws[spb * (r * bpr + block)] = 0
        ws[spb * (r * bpr + block) + 1] = 0
    x = _x(m, in_dim, 191)
    for c, val in NONFINITE[pattern]:
        x[0, c] = val
    y = pkg.iq2_matmul(to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       variant_enum(pkg, v)).cpu().numpy()
    ref = oracle.variant_matmul_reference(v, x, m, out_dim, in_dim, wb, ws)
    assert np.array_equal(classes(y), classes(ref)), pattern
    fin = classes(ref) == 0
    if fin.any():  # (a NaN in the only row makes every output NaN)
        y64, sc = oracle.variant_matmul_f64(
            v, np.where(np.isfinite(x), x, 0.0).astype(np.float32), m, out_dim, in_dim, wb, ws)
        cond, rel = errors(y[fin], y64[fin], sc[fin])
        assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)


@pytest.mark.parametrize("v", [XS, S, S3])
def test_one_row_equals_its_own_row_in_a_pair(pkg, oracle, dev, v):
    """The one-row GEMV (m = 1) and the multi-row kernel (m = 2) on the same
    row agree to the GEMV bar (they sum in different orders)."""
    out_dim, in_dim = 2048, 4096
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 200 + v)
    x = _x(2, in_dim, 201)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    y1 = pkg.iq2_matmul(to_dev(x[:1], dev), wbt, wst, out_dim, in_dim,
                        variant_enum(pkg, v)).cpu().numpy()
    y2 = pkg.iq2_matmul(to_dev(x, dev), wbt, wst, out_dim, in_dim,
                        variant_enum(pkg, v)).cpu().numpy()
    y64, sc = oracle.variant_matmul_f64(v, x[:1], 1, out_dim, in_dim, wb, ws)
    for y in (y1, y2[:1]):
        cond, rel = errors(y, y64, sc)
        assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)
