"""GPU parity of the multi-row GEMV (2 to 8 activation rows per launch, more
rows in groups of 8): every weight is decoded once and multiplied against all
the rows by one v_mfma_i32_32x32x32_i8.

The reference computes each output independently (iq2_matmul.metal:188-240),
so the bar is the one-row kernel's: against the fp64 oracle product of the
same x, cond <= 1e-5 and rel <= 1e-3.  Shapes cover ragged 32-row groups,
partial super-blocks, K in several LDS slices, more row groups than
workgroups (the chunk loop), unaligned x (element loads), W8A8 and the
row-independence of the results.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

from test_gpu_parity import errors, to_dev, x_as_f32, x_tensor  # noqa: E402


@pytest.fixture(scope="module")
def dev(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg.cabi.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


def _check(pkg, oracle, xt, wb, ws, out_dim, in_dim, dev, w8a8=False):
    m = xt.shape[0]
    if w8a8:
        cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
        y = pkg.iq2_matmul_with_activation_quant(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim,
                                                 in_dim, pkg.Iq2MatmulVariant.Iq2Xxs, cfg)
        xf = oracle.rowwise_qdq_w8a8(x_as_f32(xt), m, in_dim)
    else:
        y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                           pkg.Iq2MatmulVariant.Iq2Xxs)
        xf = x_as_f32(xt)
    y = y.cpu().numpy()
    y64, sc = oracle.matmul_f64(xf, m, out_dim, in_dim, wb, ws)
    cond, rel = errors(y, y64, sc)
    assert cond <= 1e-5 and rel <= 1e-3, (m, out_dim, in_dim, cond, rel)
    return y


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [2, 3, 4, 5, 7, 8])
def test_rows_ragged_shapes(pkg, oracle, inputs, dev, dtype, m):
    """1000 rows (the last 32-row group has 8), K = 2000 (a partial super-block)."""
    out_dim, in_dim = 1000, 2000
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F32, m, out_dim, in_dim) == "gemv"
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=m)
    xt = x_tensor(inputs.synthetic_x(m, in_dim, seed=100 + m), dtype, dev)
    _check(pkg, oracle, xt, wb, ws, out_dim, in_dim, dev)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_rows_unaligned_x_element_loads(pkg, oracle, inputs, dev, dtype):
    """x one element past a 16-byte boundary and K odd: activations are read
    element by element."""
    m, out_dim, in_dim = 6, 300, 1001
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    x = x_tensor(inputs.synthetic_x(m, in_dim), dtype, dev)
    big = torch.zeros(m * in_dim + 1, dtype=dtype, device=dev)
    big[1:] = x.reshape(-1)
    xt = big[1:].view(m, in_dim)
    assert xt.data_ptr() % 16 != 0
    _check(pkg, oracle, xt, wb, ws, out_dim, in_dim, dev)


@pytest.mark.parametrize("m,in_dim", [(8, 16384), (3, 14336), (6, 28672)])
def test_rows_k_in_several_slices(pkg, oracle, inputs, dev, m, in_dim):
    """K beyond one LDS slice of digits: the slices are digitised in turn while
    the next slice's weights are in flight."""
    out_dim = 512
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    xt = x_tensor(inputs.synthetic_x(m, in_dim), torch.float32, dev)
    _check(pkg, oracle, xt, wb, ws, out_dim, in_dim, dev)


def test_rows_chunk_loop(pkg, oracle, inputs, dev):
    """More 32-row groups than 16 per CU: workgroups loop over chunks."""
    m, out_dim, in_dim = 3, 140000, 256
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    xt = x_tensor(inputs.synthetic_x(m, in_dim), torch.float32, dev)
    _check(pkg, oracle, xt, wb, ws, out_dim, in_dim, dev)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("m", [3, 8])
def test_rows_w8a8(pkg, oracle, inputs, dev, dtype, m):
    out_dim, in_dim = 2048, 4096
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    xt = x_tensor(inputs.synthetic_x(m, in_dim), dtype, dev)
    _check(pkg, oracle, xt, wb, ws, out_dim, in_dim, dev, w8a8=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("m", [6, 12, 20, 32])
def test_rows_w8a8_int8_rows(pkg, oracle, inputs, dev, dtype, m):
    """W8A8 feeds q itself as one int8 plane per activation row, so one launch
    of the multi-row kernel serves up to 32 rows (33 on: the GEMM)."""
    out_dim, in_dim = 1000, 3000
    cd = pkg.cabi.CMK_F32 if dtype == torch.float32 else pkg.cabi.CMK_F16
    w8 = pkg.cabi.CMK_ACT_QUANT_W8A8
    assert pkg.cabi.matmul_path(cd, m, out_dim, in_dim, w8) == "gemv"
    assert pkg.cabi.matmul_path(cd, 33, out_dim, in_dim, w8) == "gemm"
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=m)
    xt = x_tensor(inputs.synthetic_x(m, in_dim, seed=200 + m), dtype, dev)
    _check(pkg, oracle, xt, wb, ws, out_dim, in_dim, dev, w8a8=True)


def test_rows_results_independent_of_other_rows(pkg, inputs, dev):
    """Rows 0-4 of an 8-row launch equal a 5-row launch of the same rows, and
    repeated launches agree bit for bit: each row's digits, scales and sums do
    not depend on the other rows."""
    out_dim, in_dim = 14336, 4096
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    x = to_dev(inputs.synthetic_x(8, in_dim), dev)
    a = pkg.iq2_xxs_matmul(x, wbt, wst, out_dim, in_dim)
    b = pkg.iq2_xxs_matmul(x, wbt, wst, out_dim, in_dim)
    assert torch.equal(a, b)
    c = pkg.iq2_xxs_matmul(x[:5].contiguous(), wbt, wst, out_dim, in_dim)
    assert torch.equal(a[:5], c)
    x2 = x.clone()
    x2[5:] *= -3.0
    d = pkg.iq2_xxs_matmul(x2, wbt, wst, out_dim, in_dim)
    assert torch.equal(a[:5], d[:5])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m", [9, 13, 16])
def test_rows_sixteen_rows_in_one_launch(pkg, oracle, inputs, dev, dtype, m):
    """Up to 16 rows take the exact-weight GEMV, in one launch that decodes
    every weight once (two A operands of 8 rows x 4 digit planes)."""
    out_dim, in_dim = 4096, 4096
    cd = {torch.float32: pkg.cabi.CMK_F32, torch.float16: pkg.cabi.CMK_F16,
          torch.bfloat16: pkg.cabi.CMK_BF16}[dtype]
    assert pkg.cabi.matmul_path(cd, m, out_dim, in_dim) == "gemv"
    assert pkg.cabi.matmul_path(cd, 17, out_dim, in_dim) == "gemm"
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    xt = x_tensor(inputs.synthetic_x(m, in_dim), dtype, dev)
    y = _check(pkg, oracle, xt, wb, ws, out_dim, in_dim, dev)
    # rows do not see each other: a row's result is the same with the other
    # rows changed (the second operand's rows 8.. scaled)
    x2 = xt.clone()
    x2[8:] *= -3.0
    y2 = pkg.iq2_matmul(x2, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                        pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    assert np.array_equal(y[:8], y2[:8])
