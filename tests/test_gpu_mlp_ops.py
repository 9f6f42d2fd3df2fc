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
