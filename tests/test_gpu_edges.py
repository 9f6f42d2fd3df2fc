"""GPU parity at the edges: non-finite activations, uneven k splits of the MFMA
GEMM, and the Llama-3-70B layer's projections at M=128.

Non-finite x.  The reference's loop (src/iq2_matmul.rs:789-809,
iq2_matmul.metal:8-28) adds x_c * w_rc in fp32, so one NaN activation makes
every output of its row NaN, an infinity makes an output +-inf (NaN where its
weight is 0, i.e. d = 0, or where infinities of both signs meet).  The tests
compare the class of every output (finite / +inf / -inf / NaN) with the oracle's
exactly, and the finite outputs with the usual bars.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from test_gpu_parity import errors, f16_weights, to_dev, x_as_f32, x_tensor  # noqa: E402


@pytest.fixture(scope="module")
def dev(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg.cabi.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


def classes(y):
    """0 finite, 1 +inf, 2 -inf, 3 NaN."""
    y = np.asarray(y)
    return np.where(np.isnan(y), 3, np.where(np.isposinf(y), 1, np.where(np.isneginf(y), 2, 0)))


# Non-finite patterns: (column, value) pairs written into row 0 of x.
NONFINITE = {
    "nan": [(100, np.nan)],
    "posinf": [(2049, np.inf)],
    "neginf": [(7, -np.inf)],
    "both_inf": [(300, np.inf), (3000, -np.inf)],
    "inf_and_nan": [(5, np.inf), (4095, np.nan)],
}


def _weights_with_zero_d(inputs, out_dim, in_dim, zero_rows, block):
    """Seeded weights with d = 0 in `block` of the given rows (their weights
    in that block are 0, so an infinite x there gives inf * 0 = NaN)."""
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    ws = ws.copy()
    bpr = (in_dim + 255) // 256
    for r in zero_rows:
        ws[2 * (r * bpr + block)] = 0
        ws[2 * (r * bpr + block) + 1] = 0
    return wb, ws


@pytest.mark.parametrize("pattern", sorted(NONFINITE))
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,out_dim,in_dim", [(1, 14336, 4096), (1, 4096, 14336), (2, 1024, 4096)])
def test_gemv_nonfinite_x(pkg, oracle, inputs, dev, pattern, dtype, m, out_dim, in_dim):
    """Config-1 shapes (gate/up and down) and a two-row case on the GEMV."""
    zero_rows = [3, 17, out_dim - 1]
    cols = [c for c, _ in NONFINITE[pattern]]
    wb, ws = _weights_with_zero_d(inputs, out_dim, in_dim, zero_rows, cols[0] // 256)
    x = inputs.synthetic_x(m, in_dim)
    for c, v in NONFINITE[pattern]:
        x[0, c % in_dim] = v
    xt = x_tensor(x, dtype, dev)
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F32, m, out_dim, in_dim) == "gemv"
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    xf = x_as_f32(xt)
    ref, _ = oracle.matmul_reference_mt(xf, m, out_dim, in_dim, wb, ws)
    assert np.array_equal(classes(y), classes(ref)), pattern
    if pattern in ("posinf", "neginf"):  # the d = 0 rows meet inf * 0
        assert np.all(np.isnan(y[0, zero_rows]))
    fin = classes(ref) == 0
    if fin.any():
        y64, sc = oracle.matmul_f64(np.where(np.isfinite(xf), xf, 0.0), m, out_dim, in_dim, wb, ws)
        cond, rel = errors(y[fin], y64[fin], sc[fin])
        assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)


@pytest.mark.parametrize("m", [1, 3, 40])
def test_w8a8_nonfinite_x(pkg, oracle, inputs, dev, m):
    """W8A8 with an infinite activation (row 0: inv = 0, so every q / inv of
    the row is NaN or infinite) and a NaN (row 1: NaN through the clamp, as in
    the reference's CPU path): output classes exactly as the oracle's, the
    finite rows to the GEMV bar (m = 1: the one-row kernel, 3: the int8
    multi-row kernel, 40: the GEMM)."""
    out_dim, in_dim = 1024, 4096
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    x = inputs.synthetic_x(m, in_dim)
    x[0, 5] = np.inf
    if m > 1:
        x[1, 77] = np.nan
    dtype = torch.float16 if m == 40 else torch.float32
    xt = x_tensor(x, dtype, dev)
    cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
    y = pkg.iq2_matmul_with_activation_quant(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim,
                                             in_dim, pkg.Iq2MatmulVariant.Iq2Xxs, cfg)
    y = y.cpu().numpy()
    xf = x_as_f32(xt)
    ref = oracle.matmul_reference_w8a8(xf, m, out_dim, in_dim, wb, ws)
    assert np.array_equal(classes(y), classes(ref))
    assert np.all(np.isnan(y[0])) and (m == 1 or np.all(np.isnan(y[1])))
    if m == 3:  # (the GEMM's numerics have their own tests)
        xq = oracle.rowwise_qdq_w8a8(xf[2:], 1, in_dim)
        y64, sc = oracle.matmul_f64(xq, 1, out_dim, in_dim, wb, ws)
        cond, rel = errors(y[2:], y64, sc)
        assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)


def _check_classes_and_finite(oracle, y, xf, wb, ws, out_dim, in_dim, w8a8=False):
    """Output classes exactly the oracle's; finite outputs to the GEMV bar
    against the fp64 product (non-finite activations set aside)."""
    m = xf.shape[0]
    if w8a8:
        ref = oracle.matmul_reference_w8a8(xf, m, out_dim, in_dim, wb, ws)
    else:
        ref, _ = oracle.matmul_reference_mt(xf, m, out_dim, in_dim, wb, ws)
    assert np.array_equal(classes(y), classes(ref))
    fin = classes(ref) == 0
    rows = [r for r in range(m) if fin[r].all()]
    if rows:
        xr = xf[rows]
        if w8a8:
            xr = oracle.rowwise_qdq_w8a8(xr, len(rows), in_dim)
        y64, sc = oracle.matmul_f64(np.ascontiguousarray(xr), len(rows), out_dim, in_dim, wb, ws)
        cond, rel = errors(y[rows], y64, sc)
        assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)
    return ref


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [12, 16])
def test_gemv_rows_nonfinite_high_rows(pkg, oracle, inputs, dev, dtype, m):
    """The 16-row decode kernel keeps rows 8-15 in a second A operand with
    their own flags: a NaN in row 9, +inf in row 11 and -inf in row m-1 reach
    exactly those output rows, as in the reference's loop; rows 0-7 and the
    other high rows stay finite."""
    out_dim, in_dim = 1024, 4096
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F32, m, out_dim, in_dim) == "gemv"
    wb, ws = _weights_with_zero_d(inputs, out_dim, in_dim, [5, 600], 3)
    x = inputs.synthetic_x(m, in_dim, seed=m)
    x[9, 100] = np.nan
    x[11, 2049] = np.inf
    x[m - 1, 7] = -np.inf
    xt = x_tensor(x, dtype, dev)
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    _check_classes_and_finite(oracle, y, x_as_f32(xt), wb, ws, out_dim, in_dim)
    assert np.all(np.isnan(y[9]))
    assert np.all(np.isfinite(y[:8]))


def test_w8a8_rows_nonfinite_high_rows(pkg, oracle, inputs, dev):
    """W8A8 with 20 rows on the 32-row int8 decode kernel: an infinity in row
    17 (inv = 0: every output of the row is NaN) and a NaN in row 9; the other
    rows to the GEMV bar against the reference's quantised activations."""
    m, out_dim, in_dim = 20, 1024, 4096
    cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F32, m, out_dim, in_dim,
                                pkg.cabi.CMK_ACT_QUANT_W8A8) == "gemv"
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    x = inputs.synthetic_x(m, in_dim, seed=20)
    x[17, 5] = np.inf
    x[9, 300] = np.nan
    xt = x_tensor(x, torch.float32, dev)
    y = pkg.iq2_matmul_with_activation_quant(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim,
                                             in_dim, pkg.Iq2MatmulVariant.Iq2Xxs, cfg)
    y = y.cpu().numpy()
    _check_classes_and_finite(oracle, y, x_as_f32(xt), wb, ws, out_dim, in_dim, w8a8=True)
    assert np.all(np.isnan(y[17])) and np.all(np.isnan(y[9]))


def test_matmul_swiglu_nonfinite_high_rows(pkg, inputs, dev):
    """silu(gate) * (x . w) with 13 rows: an infinity in row 10 of x (the
    fix-up path of the high rows) and a NaN gate in row 12 give the bits of
    the matmul followed by swiglu."""
    m, k, n = 13, 4096, 1024
    wu, su = inputs.synthetic_weights(n, k, seed=41)
    wut, sut = to_dev(wu, dev), to_dev(su, dev)
    x = torch.from_numpy(inputs.synthetic_x(m, k, seed=42)).to(dev)
    x[10, 77] = float("inf")
    gate = torch.from_numpy(inputs.synthetic_x(m, n, seed=43)).to(dev)
    gate[12, 5] = float("nan")
    ref = pkg.swiglu(gate, pkg.iq2_xxs_matmul(x, wut, sut, n, k))
    got = pkg.iq2_matmul_swiglu(x, wut, sut, n, k, gate)
    assert torch.equal(torch.isnan(ref), torch.isnan(got))
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    assert torch.equal(ref[fin], got[fin])
    assert not torch.isfinite(got[10]).all()


@pytest.mark.parametrize("pattern", ["nan", "posinf", "both_inf"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_gemm_nonfinite_x(pkg, oracle, inputs, dev, pattern, dtype):
    """The MFMA GEMM (f32 rows staged, f16 / bf16 x as given): a NaN or an
    infinity in row 0 of x reaches row 0 of the output as in the reference;
    the other rows stay finite."""
    m, out_dim, in_dim = 40, 512, 4096
    zero_rows = [3, 17]
    cols = [c for c, _ in NONFINITE[pattern]]
    wb, ws = _weights_with_zero_d(inputs, out_dim, in_dim, zero_rows, cols[0] // 256)
    x = inputs.synthetic_x(m, in_dim)
    for c, v in NONFINITE[pattern]:
        x[0, c] = v
    xt = x_tensor(x, dtype, dev)
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F32, m, out_dim, in_dim) == "gemm"
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    ref, _ = oracle.matmul_reference_mt(x_as_f32(xt), m, out_dim, in_dim, wb, ws)
    assert np.array_equal(classes(y), classes(ref)), pattern
    assert np.all(np.isfinite(y[1:]))


def test_gemm_uneven_k_split_stops_at_row_end(pkg, oracle, inputs, dev):
    """64 rows x 1024 columns give 8 tiles of 128 x 128, so k = 1792 (7 blocks)
    is split 3 + 3 + 1.  The last split must stop after its one block: weight
    row r + 1 starts right after row r's last block, and a NaN scale there must
    not reach output column r."""
    m, out_dim, in_dim = 64, 1024, 1792
    bpr = 7
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    ws = ws.copy()
    nan_row = 101
    for blk in range(bpr):  # every block of row nan_row has a NaN scale
        ws[2 * (nan_row * bpr + blk)] = 0x00
        ws[2 * (nan_row * bpr + blk) + 1] = 0x7E
    assert pkg.cabi.workspace_size(pkg.cabi.CMK_F16, m, out_dim, in_dim) == 3 * m * out_dim * 4
    xt = x_tensor(inputs.synthetic_x(m, in_dim), torch.float16, dev)
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    assert np.all(np.isnan(y[:, nan_row]))
    others = np.ones(out_dim, bool)
    others[nan_row] = False
    assert np.all(np.isfinite(y[:, others]))
    w = f16_weights(oracle, wb, ws, out_dim, in_dim)[others]
    x64 = x_as_f32(xt).astype(np.float64)
    cond, rel = errors(y[:, others], x64 @ w.T, np.abs(x64) @ np.abs(w).T)
    assert cond <= 1e-4 and rel <= 1e-2, (cond, rel)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_gemm_k_split_workspace_garbage(pkg, inputs, dev, dtype):
    """The k-split partials live in the caller's workspace: filled with 0xFF
    bytes, and reused by a second call, it gives the same bits as a fresh
    workspace (every partial is written before the split-order sum reads it)."""
    m, out_dim, in_dim = 128, 1024, 8192  # eight 128 x 128 tiles, k split in 16
    cabi = pkg.cabi
    xd = cabi.CMK_F32 if dtype == torch.float32 else cabi.CMK_F16
    assert cabi.matmul_path(xd, m, out_dim, in_dim) == "gemm"
    need = cabi.workspace_size(xd, m, out_dim, in_dim)
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=21)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    xt = x_tensor(inputs.synthetic_x(m, in_dim, seed=22), dtype, dev)
    ref = pkg.iq2_matmul(xt, wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs)
    work = torch.full((need,), 0xFF, dtype=torch.uint8, device=dev)
    for _ in range(2):
        out = torch.full((m, out_dim), float("nan"), dtype=torch.float32, device=dev)
        cabi.matmul_raw(xt.data_ptr(), xd, xt.numel(), m, wbt.data_ptr(), wbt.numel(),
                        wst.data_ptr(), wst.numel(), out_dim, in_dim, out.data_ptr(),
                        workspace_ptr=work.data_ptr(), workspace_bytes=need,
                        stream=torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


# BASELINE config 4 at M=128: q / o (8192 x 8192), gate / up (K=8192, N=28672)
# and down (K=28672, N=8192); k / v (N=1024) are in test_gpu_parity.
CONFIG4_M128 = [(8192, 8192), (28672, 8192), (8192, 28672)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("out_dim,in_dim", CONFIG4_M128)
def test_config4_m128_vs_device_dequant(pkg, inputs, dev, dtype, out_dim, in_dim):
    """Full-size config-4 projections at M=128 on the MFMA GEMM (with the k
    split these shapes take): against an fp64 product with the device
    dequantisation to f16 (bit-exact with the oracle, tested elsewhere)."""
    m = 128
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=11)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    xt = x_tensor(inputs.synthetic_x(m, in_dim, seed=12), dtype, dev)
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F32, m, out_dim, in_dim) == "gemm"
    y = pkg.iq2_matmul(xt, wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs).double()
    w = pkg.iq2_dequantize_to_f16(wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs,
                                  out_dtype=torch.float16).double()
    x64 = xt.double()
    y64 = x64 @ w.T
    sc = x64.abs() @ w.abs().T
    cond, rel = errors(y.cpu().numpy(), y64.cpu().numpy(), sc.cpu().numpy())
    # f32 rows are staged as f16 head / tail pairs (x to about 2^-22): the
    # error is the fp32 accumulation's; f16 x is exact in the MFMA.
    assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)
    del w, x64, y64, sc


# Shapes whose plan takes 256 x 128 tiles (the GEMM rows 129-256 and N near
# 8192, where 112-column tiles leave CUs idle): ragged N, K not a multiple of
# 256 or of a 32-column stage, a partial row tile, f32 rows staged as head /
# tail pairs (m = 100: 200 GEMM rows), bf16 rows staged as scaled f16, W8A8.
TILES_256x128 = [(200, 8000, 4096, torch.float16, False), (150, 8000, 3000, torch.bfloat16, False),
                 (100, 8192, 4104, torch.float32, False), (130, 8100, 2560, torch.float16, True)]


@pytest.mark.parametrize("m,out_dim,in_dim,dtype,w8a8", TILES_256x128)
def test_gemm_256x128_tiles(pkg, oracle, inputs, dev, m, out_dim, in_dim, dtype, w8a8):
    """The 256 x 128 tiles against an fp64 product with the device
    dequantisation to f16 (W8A8: of the reference's quantised rows), at the
    bars of the other GEMM shapes."""
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=m)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    xt = x_tensor(inputs.synthetic_x(m, in_dim, seed=m + 1), dtype, dev)
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F32, m, out_dim, in_dim) == "gemm"
    w = pkg.iq2_dequantize_to_f16(wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs,
                                  out_dtype=torch.float16).double()
    if w8a8:
        cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
        y = pkg.iq2_matmul_with_activation_quant(xt, wbt, wst, out_dim, in_dim,
                                                 pkg.Iq2MatmulVariant.Iq2Xxs, cfg).double()
        x64 = torch.from_numpy(
            oracle.rowwise_qdq_w8a8(x_as_f32(xt), m, in_dim).astype(np.float64)).to(dev)
    else:
        y = pkg.iq2_matmul(xt, wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs).double()
        x64 = xt.double()
    y64 = x64 @ w.T
    sc = x64.abs() @ w.abs().T
    cond, rel = errors(y.cpu().numpy(), y64.cpu().numpy(), sc.cpu().numpy())
    # W8A8 divides the fp32 sums of q * w by inv where the reference rounds
    # q / inv first: the bars of test_gpu_parity's W8A8 GEMM test.
    if w8a8:
        assert cond <= 1e-4 and rel <= 1e-2, (cond, rel)
    else:
        assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)
