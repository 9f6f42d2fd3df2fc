"""GPU parity of the HIP path against the CPU oracle (gfx950 only).

Bars:
  * dequantisation: bit-exact (f16, bf16, f32) against the oracle;
  * reference in-test cases (src/iq2_matmul.rs:1065-1253): |gpu - oracle| <= 2e-3
    (mode Off) and <= 3e-3 (W8A8), the reference's own tolerances;
  * GEMV (x f32 or any x at small m): error measured against the fp64-accumulated
    oracle with two metrics, both written in the asserts:
      cond  = max_i |y_i - y64_i| / sum_k |x_k w_ik|   (<= 1e-5, fp32 class)
      rel   = max over outputs with |y64_i| >= 1e-2 max|y64| of |y_i - y64_i|/|y64_i|
              (<= 1e-3, the GEMV bar)
  * MFMA GEMM (large m; every row set runs on f16 weights, bf16 x staged as
    scaled f16): against x @ dequant_f16(W)^T in fp64 with cond <= 1e-4 and
    rel <= 1e-2 (the GEMM bar); and against the reference's path on the same
    inputs (the fp64 oracle with exact weights) within the weights' unit
    roundoff, cond <= 2^-11 + 1e-5, since each weight is one RNE of its exact
    value.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg.cabi.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def x_tensor(x_f32, dtype, dev):
    t = torch.from_numpy(np.ascontiguousarray(x_f32)).to(dev)
    return t.to(dtype)


def x_as_f32(xt):
    return xt.float().cpu().numpy()


def errors(y, y64, scale):
    y = np.asarray(y, np.float64)
    cond = float(np.max(np.abs(y - y64) / np.maximum(scale, 1e-300)))
    big = np.abs(y64) >= 1e-2 * np.max(np.abs(y64))
    rel = float(np.max(np.abs(y - y64)[big] / np.abs(y64[big]))) if big.any() else 0.0
    return cond, rel


# Unit roundoff of the GEMM's weights: each is one RNE of its exact value
# (f16: 11 significant bits, bf16: 8), so against the exact product
# |y - y_exact| <= u * sum_k |x_k w_k| plus the fp32 accumulation.
W_ROUNDOFF = {"f16": 2.0 ** -11, "bf16": 2.0 ** -8}


def check_vs_reference_path(oracle, y, x_f32, wb, ws, out_dim, in_dim, wfmt):
    """The GEMM against the reference's path on the same inputs: the fp64
    oracle product with exact weights (x_f32: the activations the reference
    multiplies, W8A8 already quantised)."""
    m = x_f32.shape[0]
    if m * out_dim * in_dim > 6e8:
        return None  # (the single-threaded fp64 oracle would take tens of seconds)
    y64, sc = oracle.matmul_f64(np.ascontiguousarray(x_f32, np.float32), m, out_dim, in_dim, wb,
                                ws)
    cond, rel = errors(y, y64, sc)
    assert cond <= W_ROUNDOFF[wfmt] + 1e-5, (wfmt, cond, rel)
    return cond, rel


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("out_dim,in_dim", [(7, 320), (64, 4096), (5, 41), (3, 300), (33, 8192)])
def test_dequant_bit_exact(pkg, oracle, inputs, dev, out_dim, in_dim):
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=out_dim * 31 + in_dim)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    f16 = pkg.iq2_dequantize_to_f16(wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs)
    assert f16.dtype == torch.float16 and tuple(f16.shape) == (out_dim, in_dim)
    got = f16.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, oracle.dequantize_f16_bits(wb, ws, out_dim, in_dim))
    bf = pkg.iq2_dequantize_to_f16(wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs,
                                   out_dtype=torch.bfloat16)
    got = bf.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, oracle.dequantize_bf16_bits(wb, ws, out_dim, in_dim))
    f32 = pkg.iq2_dequantize_to_f16(wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs,
                                    out_dtype=torch.float32)
    assert np.array_equal(f32.cpu().numpy().view(np.uint32),
                          oracle.dequantize_f32(wb, ws, out_dim, in_dim).view(np.uint32))


def test_dequant_reference_case_matches_golden(pkg, oracle, dev):
    import hashlib
    import json
    import os
    from conftest import REPO
    pc = json.load(open(os.path.join(REPO, "tests", "golden", "reference_cases.json")))["parity_case"]
    _, wb, ws = oracle.reference_case_inputs()
    f16 = pkg.iq2_dequantize_to_f16(to_dev(wb, dev), to_dev(ws, dev), 7, 320,
                                    pkg.Iq2MatmulVariant.Iq2Xxs)
    bits = f16.cpu().view(torch.int16).numpy().view(np.uint16)
    assert hashlib.sha256(bits.tobytes()).hexdigest() == pc["dequant_f16_sha256"]


# ------------------------------------------------------------------ reference cases

@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_cpu_vs_hip_parity_iq2_xxs(pkg, oracle, dev, dtype):
    x, wb, ws = oracle.reference_case_inputs()
    xt = x_tensor(x, dtype, dev)
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), 7, 320, pkg.Iq2MatmulVariant.Iq2Xxs)
    torch.cuda.synchronize()
    ref = oracle.matmul_reference(x_as_f32(xt), 2, 7, 320, wb, ws)
    diff = np.abs(y.cpu().numpy() - ref)
    assert diff.max() <= 2e-3, diff.max()  # src/iq2_matmul.rs:1113,1121


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_cpu_vs_hip_parity_w8a8_iq2_xxs(pkg, oracle, dev, dtype):
    x, wb, ws = oracle.reference_case_inputs()
    xt = x_tensor(x, dtype, dev)
    cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
    y = pkg.iq2_matmul_with_activation_quant(xt, to_dev(wb, dev), to_dev(ws, dev), 7, 320,
                                             pkg.Iq2MatmulVariant.Iq2Xxs, cfg)
    ref = oracle.matmul_reference_w8a8(x_as_f32(xt), 2, 7, 320, wb, ws)
    diff = np.abs(y.cpu().numpy() - ref)
    assert diff.max() <= 3e-3, diff.max()  # src/iq2_matmul.rs:1239,1247


def test_w8a8_kernel_smoke_iq2_xxs(pkg, oracle, dev):
    x, wb, ws = oracle.reference_case_inputs(2, 6, 320, 0x0BADC0DE, 0xD15EA5ED, 0xC3)
    cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
    y = pkg.iq2_matmul_with_activation_quant(to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev), 6,
                                             320, pkg.Iq2MatmulVariant.Iq2Xxs, cfg)
    yh = y.cpu().numpy()
    assert yh.shape == (2, 6) and np.all(np.isfinite(yh))


def test_w4a8_non_strict_runs_as_off_and_strict_errors(pkg, oracle, dev):
    x, wb, ws = oracle.reference_case_inputs()
    args = (to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev), 7, 320, pkg.Iq2MatmulVariant.Iq2Xxs)
    off = pkg.iq2_matmul(*args)
    w4 = pkg.iq2_matmul_with_activation_quant(
        *args, pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W4A8, False))
    assert torch.equal(off, w4)
    with pytest.raises(pkg.Iq2MatmulError, match="strict mode"):
        pkg.iq2_matmul_with_activation_quant(
            *args, pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W4A8, True))


# ------------------------------------------------------------------ GEMV (small m)

GEMV_CASES = [
    (1, 4096, 4096),     # config 0
    (1, 14336, 4096),    # config 1 gate/up
    (1, 4096, 14336),    # config 1 down
    (4, 4096, 4096),     # config 2: M in {4, 8, 16} x N in {4096, 14336}, K=4096
    (4, 14336, 4096),
    (8, 4096, 4096),
    (8, 14336, 4096),
    (16, 4096, 4096),    # (f32 x keeps the exact-weight GEMV up to 16 rows)
    (16, 14336, 4096),
    (9, 512, 4096),
    (16, 512, 4096),
    (8, 1024, 4096),
    (3, 13, 300),        # ragged N, partial block
    (1, 6, 41),          # K < one sub-block
    (2, 1028, 28672),    # config 4 down-proj K
    (1, 28672, 8192),    # config 4 gate/up at M=1: four row chunks per workgroup
    (1, 8192, 28672),    # config 4 down at M=1: several chunks, digits in more than one round
    (1, 8192, 8192),     # config 4 q/o at M=1
    (1, 1024, 8192),     # config 4 k/v at M=1: one row group per workgroup, waves without a tile
]

# BASELINE config 4 (Llama-3-70B layer) at M=1: every projection shape, with
# f16 and bf16 activations as well as f32.
CONFIG4_M1 = [(8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("out_dim,in_dim", CONFIG4_M1)
def test_gemv_config4_m1_half_x(pkg, oracle, inputs, dev, dtype, out_dim, in_dim):
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    xt = x_tensor(inputs.synthetic_x(1, in_dim), dtype, dev)
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F16, 1, out_dim, in_dim) == "gemv"
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    y64, sc = oracle.matmul_f64(x_as_f32(xt), 1, out_dim, in_dim, wb, ws)
    cond, rel = errors(y, y64, sc)
    assert cond <= 1e-5 and rel <= 1e-3, (out_dim, in_dim, cond, rel)


@pytest.mark.parametrize("m,out_dim,in_dim", GEMV_CASES)
def test_gemv_f32_vs_fp64_oracle(pkg, oracle, inputs, dev, m, out_dim, in_dim):
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    x = inputs.synthetic_x(m, in_dim)
    y = pkg.iq2_matmul(to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    y64, sc = oracle.matmul_f64(x, m, out_dim, in_dim, wb, ws)
    cond, rel = errors(y, y64, sc)
    assert cond <= 1e-5, cond
    assert rel <= 1e-3, rel


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemv_half_x(pkg, oracle, inputs, dev, dtype):
    m, out_dim, in_dim = 1, 2048, 4096
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    xt = x_tensor(inputs.synthetic_x(m, in_dim), dtype, dev)
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    y64, sc = oracle.matmul_f64(x_as_f32(xt), m, out_dim, in_dim, wb, ws)
    cond, rel = errors(y, y64, sc)
    assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)


def test_gemv_w8a8_vs_oracle(pkg, oracle, inputs, dev):
    m, out_dim, in_dim = 2, 4096, 4096
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    x = inputs.synthetic_x(m, in_dim)
    cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
    y = pkg.iq2_matmul_with_activation_quant(to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev),
                                             out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs,
                                             cfg).cpu().numpy()
    xq = oracle.rowwise_qdq_w8a8(x, m, in_dim)
    y64, sc = oracle.matmul_f64(xq, m, out_dim, in_dim, wb, ws)
    cond, rel = errors(y, y64, sc)
    assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)


def test_rank1_x_and_empty_m(pkg, oracle, inputs, dev):
    wb, ws = inputs.synthetic_weights(64, 512)
    x = inputs.synthetic_x(1, 512)
    y1 = pkg.iq2_matmul(to_dev(x[0], dev), to_dev(wb, dev), to_dev(ws, dev), 64, 512,
                        pkg.Iq2MatmulVariant.Iq2Xxs)
    assert tuple(y1.shape) == (64,)
    y2 = pkg.iq2_matmul(to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev), 64, 512,
                        pkg.Iq2MatmulVariant.Iq2Xxs)
    assert torch.equal(y1, y2[0])
    y0 = pkg.iq2_matmul(torch.zeros((0, 512), device=dev), to_dev(wb, dev), to_dev(ws, dev), 64,
                        512, pkg.Iq2MatmulVariant.Iq2Xxs)
    assert tuple(y0.shape) == (0, 64)
    with pytest.raises(pkg.Iq2MatmulError, match="rank 1 or 2"):
        pkg.iq2_matmul(torch.zeros((1, 1, 512), device=dev), to_dev(wb, dev), to_dev(ws, dev),
                       64, 512, pkg.Iq2MatmulVariant.Iq2Xxs)


def test_unaligned_weights_take_portable_path(pkg, oracle, inputs, dev):
    m, out_dim, in_dim = 2, 37, 512
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    big_b = torch.zeros(wb.size + 1, dtype=torch.uint8, device=dev)
    big_b[1:] = to_dev(wb, dev)
    x = inputs.synthetic_x(m, in_dim)
    y = pkg.iq2_matmul(to_dev(x, dev), big_b[1:], to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    y64, sc = oracle.matmul_f64(x, m, out_dim, in_dim, wb, ws)
    cond, rel = errors(y, y64, sc)
    assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)


def test_deterministic(pkg, inputs, dev):
    wb, ws = inputs.synthetic_weights(4096, 4096)
    x = to_dev(inputs.synthetic_x(1, 4096), dev)
    a = pkg.iq2_xxs_matmul(x, to_dev(wb, dev), to_dev(ws, dev), 4096, 4096)
    b = pkg.iq2_xxs_matmul(x, to_dev(wb, dev), to_dev(ws, dev), 4096, 4096)
    assert torch.equal(a, b)


# ------------------------------------------------------------------ MFMA GEMM (large m)

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,out_dim,in_dim", [(512, 1024, 4096), (100, 300, 1000), (17, 64, 320)])
def test_gemm_vs_dequant_matmul(pkg, oracle, inputs, dev, dtype, m, out_dim, in_dim):
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    xt = x_tensor(inputs.synthetic_x(m, in_dim), dtype, dev)
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F16, m, out_dim, in_dim) == "gemm"
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    # f16 weights for both activation types (bf16 rows are staged as f16)
    w = oracle.dequantize_f16_bits(wb, ws, out_dim, in_dim).view(np.float16).astype(np.float64)
    x64 = x_as_f32(xt).astype(np.float64)
    y64 = x64 @ w.T
    sc = np.abs(x64) @ np.abs(w).T
    cond, rel = errors(y, y64, sc)
    assert cond <= 1e-4 and rel <= 1e-2, (cond, rel)
    check_vs_reference_path(oracle, y, x_as_f32(xt), wb, ws, out_dim, in_dim, "f16")


def test_gemm_w8a8(pkg, oracle, inputs, dev):
    m, out_dim, in_dim = 64, 256, 1024
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    xt = x_tensor(inputs.synthetic_x(m, in_dim) * 3, torch.float16, dev)
    cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
    y = pkg.iq2_matmul_with_activation_quant(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim,
                                             in_dim, pkg.Iq2MatmulVariant.Iq2Xxs,
                                             cfg).cpu().numpy()
    xq = oracle.rowwise_qdq_w8a8(x_as_f32(xt), m, in_dim).astype(np.float64)
    w = oracle.dequantize_f16_bits(wb, ws, out_dim, in_dim).view(np.float16).astype(np.float64)
    y64 = xq @ w.T
    cond, rel = errors(y, y64, np.abs(xq) @ np.abs(w).T)
    assert cond <= 1e-4 and rel <= 1e-2, (cond, rel)
    check_vs_reference_path(oracle, y, xq.astype(np.float32), wb, ws, out_dim, in_dim, "f16")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,out_dim,in_dim", [(300, 2000, 2048), (129, 230, 264)])
def test_gemm_ragged_tiles(pkg, oracle, inputs, dev, dtype, m, out_dim, in_dim):
    """Partial row and column tiles of both tile widths, K not a multiple of 256."""
    test_gemm_vs_dequant_matmul(pkg, oracle, inputs, dev, dtype, m, out_dim, in_dim)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("out_dim,in_dim", [(14336, 4096), (4096, 14336)])
def test_gemm_full_size_vs_device_dequant(pkg, inputs, dev, dtype, out_dim, in_dim):
    """Prefill shapes at full size (m = 512): the GEMM against an fp64 product with
    the device dequantisation to f16 (bit-exact with the oracle, tested above)."""
    m = 512
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=5)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    xt = x_tensor(inputs.synthetic_x(m, in_dim, seed=6), dtype, dev)
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F16, m, out_dim, in_dim) == "gemm"
    y = pkg.iq2_matmul(xt, wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs).double()
    w = pkg.iq2_dequantize_to_f16(wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs,
                                  out_dtype=torch.float16).double()
    x64 = xt.double()
    y64 = x64 @ w.T
    sc = x64.abs() @ w.abs().T
    cond, rel = errors(y.cpu().numpy(), y64.cpu().numpy(), sc.cpu().numpy())
    assert cond <= 1e-4 and rel <= 1e-2, (cond, rel)


def test_gemm_w8a8_bf16_ragged(pkg, oracle, inputs, dev):
    m, out_dim, in_dim = 200, 450, 768
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    xt = x_tensor(inputs.synthetic_x(m, in_dim) * 3, torch.bfloat16, dev)
    cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
    y = pkg.iq2_matmul_with_activation_quant(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim,
                                             in_dim, pkg.Iq2MatmulVariant.Iq2Xxs,
                                             cfg).cpu().numpy()
    xq = oracle.rowwise_qdq_w8a8(x_as_f32(xt), m, in_dim).astype(np.float64)
    w = f16_weights(oracle, wb, ws, out_dim, in_dim)  # (q is written as f16)
    y64 = xq @ w.T
    check_vs_reference_path(oracle, y, xq.astype(np.float32), wb, ws, out_dim, in_dim, "f16")
    cond, rel = errors(y, y64, np.abs(xq) @ np.abs(w).T)
    assert cond <= 1e-4 and rel <= 1e-2, (cond, rel)


# ------------------------------------------------- rows staged for the GEMM (m > 16)

def test_gemm_bf16_rows_staged_as_f16(pkg, oracle, inputs, dev):
    """bf16 x on the GEMM: each row is scaled by the power of two that brings
    its largest magnitude into [2^14, 2^15) and staged as f16 (exact), so rows
    far outside f16's range keep their values and the product runs on f16
    weights: within 2^-11 of the exact product (normwise), row by row."""
    m, out_dim, in_dim = 40, 512, 2048
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=21)
    x = inputs.synthetic_x(m, in_dim, seed=22)
    x[0] *= 1e20
    x[1] *= 1e-20
    x[2] = 0.0
    xt = x_tensor(x, torch.bfloat16, dev)
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_BF16, m, out_dim, in_dim) == "gemm"
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    xf = x_as_f32(xt)
    assert np.all(y[2] == 0.0) and np.all(np.isfinite(y))
    for r in (0, 1, 3, m - 1):
        check_vs_reference_path(oracle, y[r:r + 1], xf[r:r + 1], wb, ws, out_dim, in_dim, "f16")


def f16_weights(oracle, wb, ws, out_dim, in_dim):
    return oracle.dequantize_f16_bits(wb, ws, out_dim, in_dim).view(np.float16).astype(np.float64)


@pytest.mark.parametrize("m,out_dim,in_dim", [(17, 4096, 4096), (17, 64, 320),
                                               (128, 1024, 8192), (300, 230, 1000)])
def test_gemm_f32_rows_staged(pkg, oracle, inputs, dev, m, out_dim, in_dim):
    """f32 x beyond the GEMV's rows (16): v = x * 2^e per row (e brings the row's
    largest magnitude into [2^14, 2^15)) is staged as an f16 head rne(v) and an
    f16 tail rne(v - head), two GEMM rows whose products the epilogue sums and
    divides by 2^e.  The pair carries x to about 2^-22, so against the fp64
    product of the unrounded x with the f16-dequantised W (what the MFMA GEMM
    multiplies) the error stays at the fp32-accumulation level: cond <= 1e-5,
    rel <= 1e-3 (a single f16 rounding of x reads rel 1.4e-2 at 128x1024x8192)."""
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    x = inputs.synthetic_x(m, in_dim)
    # rows far outside f16's range both ways, and an all-zero row
    x[0] *= 1e6
    x[1] *= 1e-9
    x[2] = 0.0
    assert pkg.cabi.matmul_path(pkg.cabi.CMK_F32, m, out_dim, in_dim) == "gemm"
    y = pkg.iq2_matmul(to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim,
                       pkg.Iq2MatmulVariant.Iq2Xxs).cpu().numpy()
    w = f16_weights(oracle, wb, ws, out_dim, in_dim)
    x64 = x.astype(np.float64)
    y64 = x64 @ w.T
    assert np.all(y[2] == 0.0)
    for rows in (slice(0, 1), slice(1, 2), slice(3, m)):  # each row band against its own scale
        cond, rel = errors(y[rows], y64[rows], np.abs(x64[rows]) @ np.abs(w).T)
        assert cond <= 1e-5 and rel <= 1e-3, (rows, cond, rel)
        check_vs_reference_path(oracle, y[rows], x[rows], wb, ws, out_dim, in_dim, "f16")


def test_gemm_f32_rows_w8a8(pkg, oracle, inputs, dev):
    m, out_dim, in_dim = 64, 256, 1024
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    x = inputs.synthetic_x(m, in_dim) * 3
    cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
    y = pkg.iq2_matmul_with_activation_quant(to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev),
                                             out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs,
                                             cfg).cpu().numpy()
    xq = oracle.rowwise_qdq_w8a8(x, m, in_dim).astype(np.float64)
    w = f16_weights(oracle, wb, ws, out_dim, in_dim)
    y64 = xq @ w.T
    cond, rel = errors(y, y64, np.abs(xq) @ np.abs(w).T)
    assert cond <= 1e-4 and rel <= 1e-2, (cond, rel)
    check_vs_reference_path(oracle, y, xq.astype(np.float32), wb, ws, out_dim, in_dim, "f16")


def test_gemm_k_split_deterministic(pkg, oracle, inputs, dev):
    """Eight tiles (m=128, out_dim=1024) split k=8192 in 16: the partials are
    summed in split order, so repeated launches agree bit for bit."""
    m, out_dim, in_dim = 128, 1024, 8192
    assert pkg.cabi.workspace_size(pkg.cabi.CMK_F16, m, out_dim, in_dim) > 0
    wb, ws = inputs.synthetic_weights(out_dim, in_dim)
    xt = x_tensor(inputs.synthetic_x(m, in_dim), torch.float16, dev)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    a = pkg.iq2_matmul(xt, wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs)
    b = pkg.iq2_matmul(xt, wbt, wst, out_dim, in_dim, pkg.Iq2MatmulVariant.Iq2Xxs)
    assert torch.equal(a, b)
    w = f16_weights(oracle, wb, ws, out_dim, in_dim)
    x64 = x_as_f32(xt).astype(np.float64)
    cond, rel = errors(a.cpu().numpy(), x64 @ w.T, np.abs(x64) @ np.abs(w).T)
    assert cond <= 1e-4 and rel <= 1e-2, (cond, rel)
