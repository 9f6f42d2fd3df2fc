"""GPU parity of the IQ2_XS / IQ2_S / IQ3_S path against the CPU oracle.

Bars (as for IQ2_XXS):
  * dequantisation: bit-exact (f16, bf16, f32) against the oracle, for aligned
    and unaligned weight buffers;
  * the reference's in-test cases for every variant (src/iq2_matmul.rs:
    1065-1253, 1255-1313): |gpu - exact| <= 2e-3 (mode Off), <= 3e-3 (W8A8),
    and |gpu - oracle| within that bar plus the oracle's own distance from the
    exact product (the reference sums in one fixed fp32 order; see
    _reference_bar);
  * matmul at other shapes, against the fp64-accumulated oracle:
      cond = max_i |y_i - y64_i| / sum_k |x_k w_ik|   (<= 1e-5)
      rel  = max over outputs with |y64_i| >= 1e-2 max|y64| of |y_i - y64_i|/|y64_i|
             (<= 1e-3, the GEMV bar).
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

XS, S, S3 = 1, 2, 3
VARIANTS = [XS, S, S3]


@pytest.fixture(scope="module")
def dev(pkg):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pkg.cabi.lib()  # fail loudly when the HIP library is missing
    return torch.device("cuda:0")


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def variant_enum(pkg, v):
    return pkg.Iq2MatmulVariant(v)


def reference_case(oracle, v, m=2, out_dim=7, in_dim=320, bseed=0xA11CE5ED, sseed=0xC0FFEE12,
                   tail=0x5A):
    """parity_case / w8a8_smoke_case inputs (src/iq2_matmul.rs:1071-1086,1136-1146)
    sized by the variant's bytes / scales per block."""
    bpr = -(-in_dim // 256)
    nb = out_dim * bpr
    spb = oracle.scales_per_block(v)
    wb = oracle.lcg_fill(nb * oracle.bytes_per_block(v), bseed)
    ws = oracle.force_f16_one_per_block(oracle.lcg_fill(nb * spb, sseed), spb)
    wb[-1] = tail
    x = oracle.deterministic_x(m * in_dim).reshape(m, in_dim)
    return x, wb, ws


def random_weights(oracle, v, out_dim, in_dim, seed):
    rng = np.random.default_rng(seed)
    nb = out_dim * (-(-in_dim // 256))
    bpb, spb = oracle.bytes_per_block(v), oracle.scales_per_block(v)
    wb = rng.integers(0, 256, nb * bpb, dtype=np.uint8)
    ws = rng.integers(0, 256, nb * spb, dtype=np.uint8)
    ws[1::spb] = rng.integers(0x10, 0x20, nb, dtype=np.uint8)  # d ~ 1e-3 .. 1e-2, finite
    return wb, ws


def errors(y, y64, scale):
    y = np.asarray(y, np.float64)
    cond = float(np.max(np.abs(y - y64) / np.maximum(scale, 1e-300)))
    big = np.abs(y64) >= 1e-2 * np.max(np.abs(y64))
    rel = float(np.max(np.abs(y - y64)[big] / np.abs(y64[big]))) if big.any() else 0.0
    return cond, rel


def _reference_bar(y, ref, y64, bar):
    """The reference's bar (src/iq2_matmul.rs:1113,1121 and 1239,1247) holds
    its GPU kernel, which sums in the CPU loop's order, to `bar` of the CPU
    result.  This GPU path sums in another order, and with d = 1 the outputs
    reach a few thousand, where the CPU loop's own fp32 result is ~2e-3 from
    the exact product (IQ3_S: 2.2e-3).  So the GPU result is held to `bar` of
    the exact product, and to `bar` plus the CPU loop's own distance from it
    of the CPU result."""
    y = np.asarray(y, np.float64)
    own = float(np.max(np.abs(np.asarray(ref, np.float64) - y64)))
    assert float(np.max(np.abs(y - y64))) <= bar
    assert float(np.max(np.abs(y - ref))) <= bar + own


@pytest.mark.parametrize("v", VARIANTS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_cpu_vs_hip_parity(pkg, oracle, dev, v, dtype):
    x, wb, ws = reference_case(oracle, v)
    xt = to_dev(x, dev).to(dtype)
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), 7, 320, variant_enum(pkg, v))
    torch.cuda.synchronize()
    xf = xt.float().cpu().numpy()
    ref = oracle.variant_matmul_reference(v, xf, 2, 7, 320, wb, ws)
    y64, _ = oracle.variant_matmul_f64(v, xf, 2, 7, 320, wb, ws)
    _reference_bar(y.cpu().numpy(), ref, y64, 2e-3)


@pytest.mark.parametrize("v", VARIANTS)
def test_cpu_vs_hip_parity_w8a8(pkg, oracle, dev, v):
    x, wb, ws = reference_case(oracle, v)
    cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
    y = pkg.iq2_matmul_with_activation_quant(to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev), 7,
                                             320, variant_enum(pkg, v), cfg)
    ref = oracle.variant_matmul_reference_w8a8(v, x, 2, 7, 320, wb, ws)
    y64, _ = oracle.variant_matmul_f64(v, oracle.rowwise_qdq_w8a8(x, 2, 320), 2, 7, 320, wb, ws)
    _reference_bar(y.cpu().numpy(), ref, y64, 3e-3)


@pytest.mark.parametrize("v", VARIANTS)
def test_w8a8_kernel_smoke(pkg, oracle, dev, v):
    x, wb, ws = reference_case(oracle, v, 2, 6, 320, 0x0BADC0DE, 0xD15EA5ED, 0xC3)
    cfg = pkg.ActivationQuantConfig(pkg.ActivationQuantMode.W8A8, False)
    y = pkg.iq2_matmul_with_activation_quant(to_dev(x, dev), to_dev(wb, dev), to_dev(ws, dev), 6,
                                             320, variant_enum(pkg, v), cfg)
    yh = y.cpu().numpy()
    assert yh.shape == (2, 6) and np.all(np.isfinite(yh))


@pytest.mark.parametrize("v", VARIANTS)
@pytest.mark.parametrize("out_dim,in_dim", [(7, 320), (64, 4096), (5, 41), (3, 300)])
def test_dequant_bit_exact(pkg, oracle, dev, v, out_dim, in_dim):
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 100 * v + out_dim + in_dim)
    wbt, wst = to_dev(wb, dev), to_dev(ws, dev)
    ve = variant_enum(pkg, v)
    f16 = pkg.iq2_dequantize_to_f16(wbt, wst, out_dim, in_dim, ve)
    assert f16.dtype == torch.float16 and tuple(f16.shape) == (out_dim, in_dim)
    got = f16.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, oracle.variant_dequantize_f16_bits(v, wb, ws, out_dim, in_dim))
    bf = pkg.iq2_dequantize_to_f16(wbt, wst, out_dim, in_dim, ve, out_dtype=torch.bfloat16)
    got = bf.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, oracle.variant_dequantize_bf16_bits(v, wb, ws, out_dim, in_dim))
    f32 = pkg.iq2_dequantize_to_f16(wbt, wst, out_dim, in_dim, ve, out_dtype=torch.float32)
    assert np.array_equal(f32.cpu().numpy().view(np.uint32),
                          oracle.variant_dequantize_f32(v, wb, ws, out_dim, in_dim).view(np.uint32))


@pytest.mark.parametrize("v", VARIANTS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,out_dim,in_dim", [(1, 64, 4096), (3, 33, 1000), (6, 17, 512)])
def test_matmul_parity(pkg, oracle, dev, v, dtype, m, out_dim, in_dim):
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 7 * v + m + in_dim)
    x = np.random.default_rng(v + m).standard_normal((m, in_dim)).astype(np.float32)
    xt = to_dev(x, dev).to(dtype)
    y = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim, variant_enum(pkg, v))
    y64, scale = oracle.variant_matmul_f64(v, xt.float().cpu().numpy(), m, out_dim, in_dim, wb, ws)
    cond, rel = errors(y.cpu().numpy(), y64, scale)
    assert cond <= 1e-5, cond
    assert rel <= 1e-3, rel


@pytest.mark.parametrize("v", VARIANTS)
def test_unaligned_weight_buffers(pkg, oracle, dev, v):
    """Code and scale bytes at odd device addresses: the matmul runs on the
    byte-load kernel (aligned buffers take the multi-row decode kernel), both
    within the bars; dequantisation gives the same bits."""
    out_dim, in_dim, m = 9, 512, 2
    wb, ws = random_weights(oracle, v, out_dim, in_dim, 900 + v)
    x = np.random.default_rng(v).standard_normal((m, in_dim)).astype(np.float32)
    xt = to_dev(x, dev)
    ve = variant_enum(pkg, v)
    wbig = torch.zeros(wb.size + 1, dtype=torch.uint8, device=dev)
    sbig = torch.zeros(ws.size + 1, dtype=torch.uint8, device=dev)
    wbig[1:] = to_dev(wb, dev)
    sbig[1:] = to_dev(ws, dev)
    y_al = pkg.iq2_matmul(xt, to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim, ve)
    y_un = pkg.iq2_matmul(xt, wbig[1:], sbig[1:], out_dim, in_dim, ve)
    y64, scale = oracle.variant_matmul_f64(v, x, m, out_dim, in_dim, wb, ws)
    for y in (y_al, y_un):
        cond, rel = errors(y.cpu().numpy(), y64, scale)
        assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)
    d_al = pkg.iq2_dequantize_to_f16(to_dev(wb, dev), to_dev(ws, dev), out_dim, in_dim, ve)
    d_un = pkg.iq2_dequantize_to_f16(wbig[1:], sbig[1:], out_dim, in_dim, ve)
    assert torch.equal(d_al, d_un)


@pytest.mark.parametrize("v", [0, XS, S, S3])
@pytest.mark.parametrize("n_blocks", [1, 37, 4096 * 3 + 5])
def test_split_gguf_blocks_bit_exact(pkg, oracle, dev, v, n_blocks):
    gb = oracle.gguf_block_bytes(v)
    raw = np.random.default_rng(v + n_blocks).integers(0, 256, n_blocks * gb, dtype=np.uint8)
    wb, ws = pkg.iq2_split_gguf_blocks(to_dev(raw, dev), variant_enum(pkg, v))
    ref_b, ref_s = oracle.gguf_to_split(v, raw, n_blocks)
    assert np.array_equal(wb.cpu().numpy(), ref_b)
    assert np.array_equal(ws.cpu().numpy(), ref_s)


@pytest.mark.parametrize("v", [0, XS, S, S3])
def test_gguf_blocks_to_matmul(pkg, oracle, dev, v):
    """ggml blocks -> split on the GPU -> matmul equals the oracle on the
    oracle's split of the same blocks."""
    out_dim, in_dim, m = 11, 512, 2
    n_blocks = out_dim * 2
    gb = oracle.gguf_block_bytes(v)
    rng = np.random.default_rng(300 + v)
    raw = rng.integers(0, 256, n_blocks * gb, dtype=np.uint8)
    raw[1::gb] = rng.integers(0x10, 0x20, n_blocks, dtype=np.uint8)  # d (bytes 0-1): finite
    wb, ws = pkg.iq2_split_gguf_blocks(to_dev(raw, dev), variant_enum(pkg, v))
    x = rng.standard_normal((m, in_dim)).astype(np.float32)
    y = pkg.iq2_matmul(to_dev(x, dev), wb, ws, out_dim, in_dim, variant_enum(pkg, v))
    rb, rs = oracle.gguf_to_split(v, raw, n_blocks)
    y64, scale = oracle.variant_matmul_f64(v, x, m, out_dim, in_dim, rb, rs)
    cond, rel = errors(y.cpu().numpy(), y64, scale)
    assert cond <= 1e-5 and rel <= 1e-3, (cond, rel)


@pytest.mark.parametrize("v", [0, S3])
def test_split_gguf_blocks_unaligned_outputs(pkg, cabi, oracle, dev, v):
    """Outputs at odd addresses (byte stores) match the aligned split."""
    n = 513
    gb = oracle.gguf_block_bytes(v)
    raw = np.random.default_rng(5 + v).integers(0, 256, n * gb, dtype=np.uint8)
    src = to_dev(raw, dev)
    cb, sb = oracle.bytes_per_block(v), oracle.scales_per_block(v)
    wbig = torch.zeros(n * cb + 1, dtype=torch.uint8, device=dev)
    sbig = torch.zeros(n * sb + 1, dtype=torch.uint8, device=dev)
    cabi.split_gguf_raw(src.data_ptr(), src.numel(), n, v, wbig.data_ptr() + 1, n * cb,
                        sbig.data_ptr() + 1, n * sb, None)
    torch.cuda.synchronize()
    ref_b, ref_s = oracle.gguf_to_split(v, raw, n)
    assert np.array_equal(wbig[1:].cpu().numpy(), ref_b)
    assert np.array_equal(sbig[1:].cpu().numpy(), ref_s)
