"""GPU tests of the multi-row decode kernel's split over K.

When the 32-row groups leave CUs idle (N <= 4096 on 256 CUs), each row
group's K range is cut into parts, one workgroup each; the part that arrives
last on the row group's arrival word (in the caller's workspace) adds the
parts' sums in part order.  The split is optional: without the workspace the
launch runs unsplit.  Checked here against the fp64 oracle (the GEMV bar:
cond <= 1e-5, rel <= 1e-3), split against unsplit, determinism, a workspace
holding garbage (the arrival words need no initial value), replays of a
captured launch (one epoch for every replay), non-finite activations in
different parts, W8A8 and IQ2_XS.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from test_gpu_edges import _check_classes_and_finite  # noqa: E402
from test_gpu_parity import errors, to_dev, x_as_f32, x_tensor  # noqa: E402
from test_gpu_variants import random_weights  # noqa: E402

_XD = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


@pytest.fixture(scope="module")
def dev(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg.cabi.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


class Call:
    """One launch through the C ABI with an explicit workspace (or none)."""

    def __init__(self, cabi, xt, wbt, wst, out_dim, in_dim, workspace, mode=0, variant=0):
        self.cabi, self.xt, self.wbt, self.wst = cabi, xt, wbt, wst
        self.out_dim, self.in_dim, self.mode, self.variant = out_dim, in_dim, mode, variant
        self.ws = workspace
        self.out = torch.empty((xt.shape[0], out_dim), dtype=torch.float32, device=xt.device)

    def __call__(self, stream=None):
        ws = self.ws
        self.cabi.matmul_raw(
            self.xt.data_ptr(), _XD[self.xt.dtype], self.xt.numel(), self.xt.shape[0],
            self.wbt.data_ptr(), self.wbt.numel(), self.wst.data_ptr(), self.wst.numel(),
            self.out_dim, self.in_dim, self.out.data_ptr(), variant=self.variant, mode=self.mode,
            workspace_ptr=ws.data_ptr() if ws is not None else None,
            workspace_bytes=ws.numel() if ws is not None else 0, stream=stream)
        return self.out


def _workspace(cabi, xd, m, out_dim, in_dim, dev, fill=None, mode=0, variant=0):
    n = cabi.workspace_size(xd, m, out_dim, in_dim, variant=variant, mode=mode)
    assert n > 0, "this shape should split over K"
    ws = torch.empty(n, dtype=torch.uint8, device=dev)
    if fill is not None:
        ws.copy_(torch.from_numpy(fill(n)).to(dev))
    return ws


def _bar(oracle, y, xf, wb, ws, out_dim, in_dim):
    m = xf.shape[0]
    y64, sc = oracle.matmul_f64(np.ascontiguousarray(xf), m, out_dim, in_dim, wb, ws)
    cond, rel = errors(y, y64, sc)
    assert cond <= 1e-5 and rel <= 1e-3, (m, out_dim, in_dim, cond, rel)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,out_dim,in_dim", [(12, 4096, 4096), (16, 4096, 4096), (2, 4096, 14336),
                                              (8, 4096, 14336), (16, 1024, 8192), (13, 1000, 8192),
                                              (16, 2048, 4096)])
def test_split_matches_oracle_and_unsplit(pkg, oracle, inputs, dev, dtype, m, out_dim, in_dim):
    cabi = pkg.cabi
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=m)
    xt = x_tensor(inputs.synthetic_x(m, in_dim, seed=50 + m), dtype, dev)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    split = Call(cabi, xt, wbt, wst, out_dim, in_dim,
                 _workspace(cabi, _XD[dtype], m, out_dim, in_dim, dev))
    unsplit = Call(cabi, xt, wbt, wst, out_dim, in_dim, None)
    ys = split().cpu().numpy()
    yu = unsplit().cpu().numpy()
    xf = x_as_f32(xt)
    _bar(oracle, ys, xf, wb, ws, out_dim, in_dim)
    _bar(oracle, yu, xf, wb, ws, out_dim, in_dim)
    # the same digit products summed in another order: fp32 rounding apart
    scale = np.abs(yu).max()
    assert np.abs(ys - yu).max() <= 1e-5 * scale


def test_split_deterministic_with_garbage_workspace(pkg, inputs, dev):
    """Workspaces holding zeros, 0xFF bytes and random bytes give the same bits,
    call after call (the arrival words are tagged with each launch's epoch and
    cleared by the last part)."""
    cabi = pkg.cabi
    m, out_dim, in_dim = 16, 4096, 4096
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=3)
    xt = x_tensor(inputs.synthetic_x(m, in_dim, seed=4), torch.float32, dev)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    rng = np.random.default_rng(7)
    fills = [lambda n: np.zeros(n, np.uint8), lambda n: np.full(n, 0xFF, np.uint8),
             lambda n: rng.integers(0, 256, n, dtype=np.uint8)]
    ref = None
    for fill in fills:
        c = Call(cabi, xt, wbt, wst, out_dim, in_dim,
                 _workspace(cabi, 0, m, out_dim, in_dim, dev, fill=fill))
        for _ in range(3):
            y = c().clone()
            if ref is None:
                ref = y
            assert torch.equal(y, ref)
        # every arrival word is clear after the launch
        torch.cuda.synchronize()
        n_rg = (out_dim + 31) // 32
        words = c.ws[: 8 * n_rg].view(torch.int64)
        assert int(words.abs().sum()) == 0


def test_split_graph_replays(pkg, inputs, dev):
    """A captured split launch keeps one epoch: each replay starts from the
    arrival words the previous launch cleared.  Eager split launches of other
    inputs on the same workspace run between the replays."""
    cabi = pkg.cabi
    m, out_dim, in_dim = 4, 4096, 14336
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=11)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    work = _workspace(cabi, 0, m, out_dim, in_dim, dev)
    xa = x_tensor(inputs.synthetic_x(m, in_dim, seed=12), torch.float32, dev)
    xb = x_tensor(inputs.synthetic_x(m, in_dim, seed=13), torch.float32, dev)
    ca = Call(cabi, xa, wbt, wst, out_dim, in_dim, work)
    cb = Call(cabi, xb, wbt, wst, out_dim, in_dim, work)
    ya = ca().clone()
    yb = cb().clone()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    ca.out.zero_()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        ca(stream=stream.cuda_stream)
    for i in range(4):
        ca.out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ca.out, ya), f"replay {i}"
        assert torch.equal(cb().clone(), yb), f"eager launch after replay {i}"
        torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_split_nonfinite_in_different_parts(pkg, oracle, inputs, dev, dtype):
    """N = 4096, K = 4096 with 12 rows splits in two parts of 2048 columns: a
    NaN only in the second part (row 1), +inf only in the first (row 2), -inf
    in both (row 3).  The last part combines the parts' row masks, so each row
    gets exactly the oracle's classes whichever part arrives last."""
    m, out_dim, in_dim = 12, 4096, 4096
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=21)
    x = inputs.synthetic_x(m, in_dim, seed=22)
    x[1, 3000] = np.nan
    x[2, 100] = np.inf
    x[3, 5] = -np.inf
    x[3, 4000] = -np.inf
    xt = x_tensor(x, dtype, dev)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    c = Call(pkg.cabi, xt, wbt, wst, out_dim, in_dim,
             _workspace(pkg.cabi, _XD[dtype], m, out_dim, in_dim, dev))
    y = c().cpu().numpy()
    _check_classes_and_finite(oracle, y, x_as_f32(xt), wb, ws, out_dim, in_dim)
    assert np.all(np.isnan(y[1]))
    assert np.all(np.isfinite(y[[0, 4, 11]]))


@pytest.mark.parametrize("m,in_dim", [(4, 14336), (20, 4096)])
def test_split_w8a8(pkg, oracle, inputs, dev, m, in_dim):
    """True-int8 W8A8 rows (8- and 32-row instantiations) split over K: the
    parts add raw integer-product sums; 1 / (8 inv) is applied once after."""
    cabi = pkg.cabi
    out_dim = 4096
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=30 + m)
    x = inputs.synthetic_x(m, in_dim, seed=40 + m)
    xt = x_tensor(x, torch.float32, dev)
    c = Call(cabi, xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
             _workspace(cabi, 0, m, out_dim, in_dim, dev, mode=cabi.CMK_ACT_QUANT_W8A8),
             mode=cabi.CMK_ACT_QUANT_W8A8)
    y = c().cpu().numpy()
    xq = oracle.rowwise_qdq_w8a8(x_as_f32(xt), m, in_dim)
    _bar(oracle, y, xq, wb, ws, out_dim, in_dim)


def test_split_w8a8_infinite_row(pkg, oracle, inputs, dev):
    """W8A8: an infinite activation makes its row's every output NaN (its q /
    inv is NaN in every column), found in either part."""
    cabi = pkg.cabi
    m, out_dim, in_dim = 17, 4096, 4096
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=51)
    x = inputs.synthetic_x(m, in_dim, seed=52)
    x[2, 3500] = np.inf
    xt = x_tensor(x, torch.float32, dev)
    c = Call(cabi, xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
             _workspace(cabi, 0, m, out_dim, in_dim, dev, mode=cabi.CMK_ACT_QUANT_W8A8),
             mode=cabi.CMK_ACT_QUANT_W8A8)
    y = c().cpu().numpy()
    _check_classes_and_finite(oracle, y, x_as_f32(xt), wb, ws, out_dim, in_dim, w8a8=True)
    assert np.all(np.isnan(y[2]))


def test_split_iq2_xs_rows(pkg, oracle, inputs, dev):
    """IQ2_XS on the multi-row kernel at N = 4096 takes the same split."""
    cabi = pkg.cabi
    m, out_dim, in_dim = 16, 4096, 4096
    wb, ws = random_weights(oracle, 1, out_dim, in_dim, seed=61)
    xt = x_tensor(inputs.synthetic_x(m, in_dim, seed=62), torch.float32, dev)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    split = Call(cabi, xt, wbt, wst, out_dim, in_dim,
                 _workspace(cabi, 0, m, out_dim, in_dim, dev, variant=cabi.CMK_IQ2_XS),
                 variant=cabi.CMK_IQ2_XS)
    unsplit = Call(cabi, xt, wbt, wst, out_dim, in_dim, None, variant=cabi.CMK_IQ2_XS)
    ys = split().cpu().numpy()
    yu = unsplit().cpu().numpy()
    y64, sc = oracle.variant_matmul_f64(1, x_as_f32(xt), m, out_dim, in_dim, wb, ws)
    for y in (ys, yu):
        cond, rel = errors(y, y64, sc)
        assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)
