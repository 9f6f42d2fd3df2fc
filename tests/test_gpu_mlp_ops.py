"""GPU check of the MLP step h = silu(gate) * up (no reference counterpart: it
is checked against the definition silu(g) = g / (1 + e^-g) evaluated in
float64).  Bars: f32 output within 4 ulp of the float64 value (expf and one
division, one product); f16 / bf16 output equal to the RNE of the kernel's own
f32 result and within one unit in the last place of the float64 value;
special values: silu(0) = 0, silu(-1000) = -0, silu(+inf) = +inf, silu(-inf)
and NaN give NaN; and the full MLP chain gate, up, swiglu, down against the oracle."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg.cabi.lib()
    return torch.device("cuda:0")


def silu_mul64(g, u):
    g = g.astype(np.float64)
    return g / (1.0 + np.exp(-g)) * u.astype(np.float64)


@pytest.mark.parametrize("n", [1, 3, 4, 1000, 14336, 4 * 14336 + 3])
def test_swiglu_f32(pkg, dev, n):
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    h = pkg.swiglu(torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev)).cpu().numpy()
    ref = silu_mul64(g, u)
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(h - ref) <= 4 * ulp + 1e-38), np.max(np.abs(h - ref) / ulp)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_swiglu_half_outputs(pkg, dev, dtype):
    n = 4099
    rng = np.random.default_rng(7)
    g = (rng.standard_normal(n) * 3).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    gt, ut = torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev)
    h32 = pkg.swiglu(gt, ut)
    h = pkg.swiglu(gt, ut, out_dtype=dtype)
    assert h.dtype == dtype
    assert torch.equal(h.cpu(), h32.cpu().to(dtype))  # one RNE of the f32 result
    ref = torch.from_numpy(silu_mul64(g, u))
    assert torch.allclose(h.double().cpu(), ref, rtol=2 ** -7 if dtype == torch.bfloat16 else 2 ** -10,
                          atol=1e-6)


def test_swiglu_special_values(pkg, dev):
    g = np.array([0.0, -np.inf, np.inf, np.nan, -100.0, 100.0, -1000.0], np.float32)
    u = np.array([5.0, 2.0, 3.0, 1.0, 1.0, 1.0, 1.0], np.float32)
    h = pkg.swiglu(torch.from_numpy(g).to(dev), torch.from_numpy(u).to(dev)).cpu().numpy()
    assert h[0] == 0.0
    assert np.isnan(h[1])  # -inf / (1 + inf), as -inf * sigmoid(-inf) = -inf * 0
    assert h[2] == np.inf
    assert np.isnan(h[3])
    assert abs(h[4]) < 1e-40 and h[5] == 100.0
    assert h[6] == 0.0 and np.signbit(h[6])  # exp(1000) overflows: -1000 / inf = -0


def test_swiglu_unaligned(pkg, dev):
    n = 1001
    rng = np.random.default_rng(9)
    g = torch.from_numpy(rng.standard_normal(n + 1).astype(np.float32)).to(dev)
    u = torch.from_numpy(rng.standard_normal(n + 1).astype(np.float32)).to(dev)
    a = pkg.swiglu(g[1:], u[1:])  # 4-byte aligned views: scalar path
    b = pkg.swiglu(g[1:].clone(), u[1:].clone())  # 16-byte aligned: vector path
    assert torch.equal(a, b)


def test_mlp_chain_against_oracle(pkg, oracle, inputs, dev):
    """gate, up (K=512 -> N=384), swiglu, down (384 -> 512) at M=1 against the
    oracle matmuls and a float64 swiglu."""
    k, n = 512, 384
    wg, sg = inputs.synthetic_weights(n, k, seed=11)
    wu, su = inputs.synthetic_weights(n, k, seed=12)
    wd, sd = inputs.synthetic_weights(k, n, seed=13)
    x = inputs.synthetic_x(1, k, seed=14)
    td = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    V = pkg.Iq2MatmulVariant.Iq2Xxs
    g = pkg.iq2_matmul(td(x), td(wg), td(sg), n, k, V)
    u = pkg.iq2_matmul(td(x), td(wu), td(su), n, k, V)
    h = pkg.swiglu(g, u)
    y = pkg.iq2_matmul(h, td(wd), td(sd), k, n, V).cpu().numpy()
    g64, _ = oracle.matmul_f64(x, 1, n, k, wg, sg)
    u64, _ = oracle.matmul_f64(x, 1, n, k, wu, su)
    h64 = (g64 / (1.0 + np.exp(-g64)) * u64).astype(np.float32)
    y64, scale = oracle.matmul_f64(h64, 1, k, n, wd, sd)
    err = np.abs(y - y64)
    assert np.max(err / np.maximum(scale, 1e-30)) <= 1e-4
    big = np.abs(y64) >= 1e-2 * np.abs(y64).max()
    assert np.max(err[big] / np.abs(y64[big])) <= 1e-3



@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("m", [1, 3, 8, 13])
@pytest.mark.parametrize("k,n", [(4096, 14336), (14336, 512), (1000, 300)])
def test_matmul_swiglu_equals_matmul_then_swiglu(pkg, inputs, dev, m, k, n, dtype):
    """The up projection with silu(gate) * u in its epilogue gives the same
    bits as the matmul followed by cmk_swiglu (one fp32 expression on the same
    sums)."""
    wu, su = inputs.synthetic_weights(n, k, seed=21)
    x = torch.from_numpy(inputs.synthetic_x(m, k, seed=22)).to(dev).to(dtype)
    gate = torch.from_numpy(inputs.synthetic_x(m, n, seed=23)).to(dev)
    wut, sut = torch.from_numpy(wu).to(dev), torch.from_numpy(su).to(dev)
    ref = pkg.swiglu(gate, pkg.iq2_xxs_matmul(x, wut, sut, n, k))
    got = pkg.iq2_matmul_swiglu(x, wut, sut, n, k, gate)
    assert torch.equal(ref, got)
    if m == 1:  # rank-1 x and gate give a rank-1 output
        got1 = pkg.iq2_matmul_swiglu(x[0], wut, sut, n, k, gate[0])
        assert got1.shape == (n,) and torch.equal(got1, ref[0])


@pytest.mark.parametrize("m,k,n", [(1, 4096, 1024), (2, 4096, 1024), (4, 14336, 4096)])
def test_matmul_swiglu_nonfinite(pkg, inputs, dev, m, k, n):
    """A NaN activation (the set-aside fix-up path) and a NaN / infinite gate
    reach the output as through the matmul then swiglu (K = 14336 at N = 4096:
    the multi-row kernel splits K, and the last part applies the gate after
    the fix-up)."""
    wu, su = inputs.synthetic_weights(n, k, seed=31)
    wut, sut = torch.from_numpy(wu).to(dev), torch.from_numpy(su).to(dev)
    x = torch.from_numpy(inputs.synthetic_x(m, k, seed=32)).to(dev)
    x[m - 1, 77] = float("inf")
    gate = torch.from_numpy(inputs.synthetic_x(m, n, seed=33)).to(dev)
    gate[0, 5] = float("nan")
    gate[0, 6] = -float("inf")
    ref = pkg.swiglu(gate, pkg.iq2_xxs_matmul(x, wut, sut, n, k))
    got = pkg.iq2_matmul_swiglu(x, wut, sut, n, k, gate)
    assert torch.equal(torch.isnan(ref), torch.isnan(got))
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    assert torch.equal(ref[fin], got[fin])


def test_matmul_swiglu_rejects_gemm_shapes(pkg, inputs, dev):
    wu, su = inputs.synthetic_weights(64, 256)
    x = torch.zeros((17, 256), dtype=torch.float32, device=dev)
    gate = torch.zeros((17, 64), dtype=torch.float32, device=dev)
    with pytest.raises(pkg.Iq2MatmulError, match="decode-shaped"):
        pkg.iq2_matmul_swiglu(x, torch.from_numpy(wu).to(dev), torch.from_numpy(su).to(dev), 64,
                              256, gate)
