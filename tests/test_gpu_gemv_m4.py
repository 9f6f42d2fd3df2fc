"""The one-row GEMV's 2-4 row launch (iq2xxs_gemv.hip, kM4) against the fp64
oracle.  The dispatch sends m = 2..4 there when out_dim <= 16 per CU (4096 on
the 256 CUs of MI355X), and m = 2 also at larger out_dim when K <= 4096 (its
packed two-operand form in mode Off), provided the rows of x are 16-byte
aligned, every digitisation task fits in registers at once (m * 32 *
ceil(K/256) <= 2048), one chunk of row groups per workgroup suffices and the
LDS holds m rows of digits.  The shapes below reach it (14336 x 4096 at m = 2
only; at m = 3, 4 it checks the multi-row kernel).  Bars as in
test_gpu_parity.py (cond <= 1e-5, rel <= 1e-3 against the exact-weight fp64
product; W8A8 against the reference's quantised activations), output classes
exactly the oracle's for non-finite activations."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from test_gpu_edges import _check_classes_and_finite, classes  # noqa: E402
from test_gpu_parity import errors, to_dev, x_as_f32, x_tensor  # noqa: E402

SHAPES = [(4096, 4096), (1024, 4096), (4096, 2048), (37, 256), (300, 1000), (2048, 8192),
          (14336, 4096)]


def _fits(m, k):
    return m * 32 * ((k + 255) // 256) <= 2048
_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.fixture(scope="module")
def dev(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg.cabi.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


def _run(pkg, xt, wb, ws, n, k, w8a8):
    mode = pkg.ActivationQuantMode.W8A8 if w8a8 else pkg.ActivationQuantMode.Off
    cfg = pkg.ActivationQuantConfig(mode, False)
    return pkg.iq2_matmul_with_activation_quant(xt, wb, ws, n, k, pkg.Iq2MatmulVariant.Iq2Xxs,
                                                cfg).cpu().numpy()


# (m, n, k): every shape at every m whose digitisation tasks fit the launch
# (m * 32 * ceil(K/256) <= 2048; 2048 x 8192 only at m = 2)
_MNK = [(m, n, k) for m in (2, 3, 4) for n, k in SHAPES if _fits(m, k)]


@pytest.mark.parametrize("w8a8", [False, True], ids=["off", "w8a8"])
@pytest.mark.parametrize("dtype", sorted(_DT))
@pytest.mark.parametrize("m,n,k", _MNK)
def test_m4_vs_oracle(pkg, oracle, inputs, dev, m, n, k, dtype, w8a8):
    wb, ws = inputs.synthetic_weights(n, k, seed=m * 7 + n + k)
    xt = x_tensor(inputs.synthetic_x(m, k, seed=m + 1), _DT[dtype], dev)
    y = _run(pkg, xt, to_dev(wb, dev), to_dev(ws, dev), n, k, w8a8).reshape(m, n)
    xf = np.ascontiguousarray(x_as_f32(xt), np.float32)
    if w8a8:
        xf = oracle.rowwise_qdq_w8a8(xf, m, k)
    y64, sc = oracle.matmul_f64(np.ascontiguousarray(xf, np.float32), m, n, k, wb, ws)
    cond, rel = errors(y, y64, sc)
    assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)
    # each row as the one-row kernel computes it alone: the same digits and
    # integer sums, fp32 combination in another order
    y1 = _run(pkg, xt[1:2].contiguous(), to_dev(wb, dev), to_dev(ws, dev), n, k, w8a8)
    np.testing.assert_allclose(y[1], y1.reshape(n), rtol=1e-5, atol=1e-5 * np.abs(y1).max())


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("m", [2, 4])
def test_m4_nonfinite_rows(pkg, oracle, inputs, dev, m, dtype):
    """A NaN in the last row and +-inf in the first (where a d = 0 block meets
    inf * 0): every class as the oracle's, the finite rows to the bar."""
    n, k = 1024, 4096
    wb, ws = inputs.synthetic_weights(n, k)
    ws = ws.copy()
    bpr = k // 256
    for r in (5, 900):  # d = 0 in block 1 of these rows
        ws[2 * (r * bpr + 1)] = 0
        ws[2 * (r * bpr + 1) + 1] = 0
    x = inputs.synthetic_x(m, k)
    x[0, 300] = np.inf
    x[0, 3000] = -np.inf
    x[m - 1, 17] = np.nan
    xt = x_tensor(x, _DT[dtype], dev)
    y = _run(pkg, xt, to_dev(wb, dev), to_dev(ws, dev), n, k, False).reshape(m, n)
    _check_classes_and_finite(oracle, y, x_as_f32(xt), wb, ws, n, k)
    assert np.all(np.isnan(y[m - 1])) and np.isnan(y[0, 5]) and np.isnan(y[0, 900])


def test_m4_w8a8_infinite_row(pkg, oracle, inputs, dev):
    """W8A8: an infinite activation makes its row's inv 0, so every output of
    the row is NaN; the other rows keep their own scales."""
    n, k, m = 4096, 4096, 3
    wb, ws = inputs.synthetic_weights(n, k)
    x = inputs.synthetic_x(m, k)
    x[1, 2049] = np.inf
    xt = x_tensor(x, torch.float32, dev)
    y = _run(pkg, xt, to_dev(wb, dev), to_dev(ws, dev), n, k, True).reshape(m, n)
    _check_classes_and_finite(oracle, y, x_as_f32(xt), wb, ws, n, k, w8a8=True)
    assert np.all(np.isnan(y[1])) and np.isfinite(y[[0, 2]]).all()


@pytest.mark.parametrize("m", [2, 3, 4])
def test_m4_swiglu_epilogue(pkg, inputs, dev, m):
    """silu(gate) * up in the 2-4 row launch's epilogue equals the matmul
    followed by cmk_swiglu, bit for bit."""
    n, k = 4096, 4096
    wb, ws = inputs.synthetic_weights(n, k)
    xt = x_tensor(inputs.synthetic_x(m, k), torch.float32, dev)
    gate = torch.randn(m, n, device=dev)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    fused = pkg.iq2_matmul_swiglu(xt, wbt, wst, n, k, gate).cpu().numpy()
    up = pkg.iq2_matmul(xt, wbt, wst, n, k, pkg.Iq2MatmulVariant.Iq2Xxs)
    composed = pkg.swiglu(gate, up.reshape(m, n)).cpu().numpy()
    assert np.array_equal(fused.reshape(m, n).view(np.uint32),
                          composed.reshape(m, n).view(np.uint32))


def test_m4_deterministic(pkg, inputs, dev):
    n, k, m = 4096, 4096, 4
    wb, ws = inputs.synthetic_weights(n, k)
    xt = x_tensor(inputs.synthetic_x(m, k), torch.float32, dev)
    a = _run(pkg, xt, to_dev(wb, dev), to_dev(ws, dev), n, k, False)
    b = _run(pkg, xt, to_dev(wb, dev), to_dev(ws, dev), n, k, False)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
