"""Seeded random shapes through the public matmul, against the fp64 oracle.

Each case draws a format, an activation mode and dtype, m, N and K (ragged
and aligned, short and long K, m from 1 to 40) from a fixed seed, so every
dispatch path is reached: the one-row GEMV, the multi-row decode kernel with
and without its split over K (uneven part counts included), the MFMA GEMM
with and without its k split, and the portable kernels.  Bars as in
test_gpu_parity.py: the GEMV family and the portable kernels against the
exact-weight fp64 product (cond <= 1e-5, rel <= 1e-3); the GEMM, whose
weights are f16, against the same product within the weights' unit roundoff
(cond <= 2^-11 + 1e-5).  Every case also runs twice and must give the same
bits.  The case's parameters are in its test id.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from test_gpu_parity import W_ROUNDOFF, errors, to_dev, x_as_f32, x_tensor  # noqa: E402
from test_gpu_variants import random_weights  # noqa: E402

_DTYPES = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
_NAMES = ["iq2_xxs", "iq2_xs", "iq2_s", "iq3_s"]


def _draw_cases(n_cases=120, seed=2026):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n_cases:
        variant = int(rng.choice(4, p=[0.64, 0.12, 0.12, 0.12]))
        w8a8 = bool(rng.random() < 0.2)
        dtype = str(rng.choice(["f32", "f16", "bf16"]))
        r = rng.random()
        m = 1 if r < 0.3 else int(rng.integers(2, 17)) if r < 0.75 else int(rng.integers(17, 41))
        n = int(rng.choice([rng.integers(1, 300), 32 * rng.integers(1, 160),
                            rng.integers(300, 5000)]))
        k = int(rng.choice([rng.integers(1, 2000), 8 * rng.integers(250, 2500),
                            256 * rng.integers(1, 64)]))
        if m * n * k > 2e8 or n * k > 4e7:  # (the fp64 oracle stays within a second)
            continue
        cases.append((variant, w8a8, dtype, m, n, k))
    return cases


CASES = _draw_cases()


def _case_id(c):
    v, w8a8, dtype, m, n, k = c
    return f"{_NAMES[v]}-{'w8a8' if w8a8 else 'off'}-{dtype}-m{m}-n{n}-k{k}"


@pytest.fixture(scope="module")
def dev(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg.cabi.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


@pytest.mark.parametrize("case", CASES, ids=[_case_id(c) for c in CASES])
def test_random_shape(pkg, oracle, inputs, dev, case):
    variant, w8a8, dtype, m, n, k = case
    seed = 7 * m + 13 * n + k
    if variant == 0:
        wb, ws = inputs.synthetic_weights(n, k, seed=seed)
    else:
        wb, ws = random_weights(oracle, variant, n, k, seed)
    xt = x_tensor(inputs.synthetic_x(m, k, seed=seed + 1), _DTYPES[dtype], dev)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    ve = pkg.Iq2MatmulVariant(variant)

    def run():
        if w8a8:
            cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
            return pkg.iq2_matmul_with_activation_quant(xt, wbt, wst, n, k, ve, cfg)
        return pkg.iq2_matmul(xt, wbt, wst, n, k, ve)

    y = run().cpu().numpy().reshape(m, n)
    y2 = run().cpu().numpy().reshape(m, n)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32)), "not deterministic"

    xf = x_as_f32(xt)
    if w8a8:
        xf = oracle.rowwise_qdq_w8a8(np.ascontiguousarray(xf), m, k)
    xf = np.ascontiguousarray(xf, np.float32)
    if variant == 0:
        y64, sc = oracle.matmul_f64(xf, m, n, k, wb, ws)
    else:
        y64, sc = oracle.variant_matmul_f64(variant, xf, m, n, k, wb, ws)
    cond, rel = errors(y, y64, sc)
    xd = {"f32": pkg.cabi.CMK_F32, "f16": pkg.cabi.CMK_F16, "bf16": pkg.cabi.CMK_BF16}[dtype]
    mode = pkg.cabi.CMK_ACT_QUANT_W8A8 if w8a8 else pkg.cabi.CMK_ACT_QUANT_OFF
    path = pkg.cabi.matmul_path(xd, m, n, k, mode) if variant == 0 else "variant"
    if path == "gemm":
        assert cond <= W_ROUNDOFF["f16"] + 1e-5, (path, cond, rel)
    else:
        assert cond <= 1e-5 and rel <= 1e-3, (path, cond, rel)
