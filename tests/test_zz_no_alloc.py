"""cmk_iq2_matmul_noalloc against cmk_iq2_matmul through the C ABI.

The allocation-free entry point runs the same kernels as cmk_iq2_matmul with
the library's per-device scratch array in place of a caller's workspace, so the
outputs must be bit-identical.  Two calls in a row, the second on a smaller
input, on shapes whose launch needs scratch (the MFMA GEMM's staged f32 rows,
the W8A8 row scales and staged rows, and k-split partials).  Arguments that
need more than the array holds are refused before anything is launched.
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


def _run_pair(cabi, dev, inputs, m, out_dim, in_dim, x_dtype, mode):
    wb, ws = inputs.synthetic_weights(out_dim, in_dim, seed=m * 7 + out_dim)
    x = inputs.synthetic_x(m, in_dim, seed=m + in_dim)
    xt = torch.from_numpy(x).to(dev)
    if x_dtype == cabi.CMK_F16:
        xt = xt.half()
    wbt = torch.from_numpy(wb).to(dev)
    wst = torch.from_numpy(ws).to(dev)
    need = cabi.workspace_size(x_dtype, m, out_dim, in_dim, mode=mode)
    assert 0 < need <= cabi.NOALLOC_SCRATCH_BYTES, need
    work = torch.empty((need,), dtype=torch.uint8, device=dev)
    ref = torch.full((m, out_dim), float("nan"), dtype=torch.float32, device=dev)
    got = torch.full((m, out_dim), float("nan"), dtype=torch.float32, device=dev)
    args = (xt.data_ptr(), x_dtype, xt.numel(), m, wbt.data_ptr(), wbt.numel(), wst.data_ptr(),
            wst.numel(), out_dim, in_dim)
    cabi.matmul_raw(*args, ref.data_ptr(), mode=mode, workspace_ptr=work.data_ptr(),
                    workspace_bytes=need)
    cabi.matmul_noalloc_raw(*args, got.data_ptr(), mode=mode)
    torch.cuda.synchronize()
    return ref, got


# (m, out_dim, in_dim, x dtype, mode) pairs: each second case is smaller
CASES = [
    ((64, 1024, 4096, "f32", "off"), (24, 512, 2048, "f32", "off")),
    ((40, 768, 4096, "f16", "w8a8"), (20, 256, 1024, "f16", "w8a8")),
    ((128, 1024, 8192, "f16", "off"), (96, 512, 2048, "f16", "off")),
]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_workspace_entry_point(pkg, inputs, dev, first, second):
    cabi = pkg.cabi
    dt = {"f32": cabi.CMK_F32, "f16": cabi.CMK_F16}
    md = {"off": cabi.CMK_ACT_QUANT_OFF, "w8a8": cabi.CMK_ACT_QUANT_W8A8}
    for m, n, k, x_dtype, mode in (first, second):
        assert cabi.matmul_path(dt[x_dtype], m, n, k) == "gemm"
        ref, got = _run_pair(cabi, dev, inputs, m, n, k, dt[x_dtype], md[mode])
        assert torch.isfinite(ref).all()
        assert torch.equal(ref, got), (m, n, k, x_dtype, mode)


def test_noalloc_gemv_needs_no_scratch(pkg, inputs, dev):
    """The decode path needs no scratch: the same call on an m=1 shape."""
    cabi = pkg.cabi
    m, n, k = 1, 2048, 4096
    assert cabi.workspace_size(cabi.CMK_F32, m, n, k) == 0
    wb, ws = inputs.synthetic_weights(n, k)
    xt = torch.from_numpy(inputs.synthetic_x(m, k)).to(dev)
    wbt, wst = torch.from_numpy(wb).to(dev), torch.from_numpy(ws).to(dev)
    ref = torch.empty((m, n), dtype=torch.float32, device=dev)
    got = torch.empty((m, n), dtype=torch.float32, device=dev)
    args = (xt.data_ptr(), cabi.CMK_F32, xt.numel(), m, wbt.data_ptr(), wbt.numel(),
            wst.data_ptr(), wst.numel(), n, k)
    cabi.matmul_raw(*args, ref.data_ptr())
    cabi.matmul_noalloc_raw(*args, got.data_ptr())
    torch.cuda.synchronize()
    assert torch.equal(ref, got)


def test_noalloc_refuses_more_than_its_scratch(pkg, dev):
    """512 f32 rows of 16384 are staged as 2 x 512 x 16384 f16 values (32 MiB)
    plus the row scales: more than the array holds.  Refused with a message,
    nothing launched (the pointers are never dereferenced)."""
    cabi = pkg.cabi
    m, n, k = 512, 14336, 16384
    assert cabi.workspace_size(cabi.CMK_F32, m, n, k) > cabi.NOALLOC_SCRATCH_BYTES
    bpr = (k + 255) // 256
    fake = 1 << 20  # 16-byte aligned stand-in addresses, never used
    with pytest.raises(cabi.CmkError, match="cmk_iq2_matmul_noalloc needs"):
        cabi.matmul_noalloc_raw(fake, cabi.CMK_F32, m * k, m, fake, n * bpr * 64, fake,
                                n * bpr * 2, n, k, fake)
