"""cmk_iq2_matmul_noalloc against cmk_iq2_matmul through the C ABI.

The allocation-free entry point runs the same kernels as cmk_iq2_matmul with
the library's per-device scratch array in place of a caller's workspace, so the
outputs must be bit-identical.  Two calls in a row, the second on a smaller
input, on shapes whose launch needs scratch (the MFMA GEMM's staged f32 rows,
the W8A8 row scales and staged rows, and k-split partials).  Arguments that
need more than the array holds are refused before anything is launched.
"""

import os
import subprocess
import sys

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


@pytest.mark.parametrize("m", [1, 3])
def test_noalloc_gemv_needs_no_scratch(pkg, inputs, dev, m):
    """The decode paths need no scratch: the same call on the one-row GEMV
    (m=1) and its 2-4 row launch (m=3)."""
    cabi = pkg.cabi
    n, k = 2048, 4096
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


def _graph_case(cabi, inputs, dev, m, n, k, seed):
    wb, ws = inputs.synthetic_weights(n, k, seed=seed)
    xt = torch.from_numpy(inputs.synthetic_x(m, k, seed=seed + 1)).to(dev)
    wbt, wst = torch.from_numpy(wb).to(dev), torch.from_numpy(ws).to(dev)
    args = (xt.data_ptr(), cabi.CMK_F32, xt.numel(), m, wbt.data_ptr(), wbt.numel(),
            wst.data_ptr(), wst.numel(), n, k)
    return (xt, wbt, wst), args


def test_noalloc_graph_replays_match(pkg, inputs, dev):
    """cmk_iq2_matmul_noalloc captured in a HIP graph (torch.cuda.graph) on a
    shape whose launch uses the scratch array (f32 rows staged as f16 head /
    tail pairs): four replays, each after an eager noalloc call of another
    shape that overwrites the array, every replay bit-identical to
    cmk_iq2_matmul with a workspace of its own."""
    cabi = pkg.cabi
    m, n, k = 64, 1024, 4096
    keep, args = _graph_case(cabi, inputs, dev, m, n, k, seed=5)
    keep2, args2 = _graph_case(cabi, inputs, dev, 48, 768, 2048, seed=9)
    need = cabi.workspace_size(cabi.CMK_F32, m, n, k)
    assert cabi.matmul_path(cabi.CMK_F32, m, n, k) == "gemm" and need > 0
    work = torch.empty((need,), dtype=torch.uint8, device=dev)
    ref = torch.empty((m, n), dtype=torch.float32, device=dev)
    cabi.matmul_raw(*args, ref.data_ptr(), workspace_ptr=work.data_ptr(), workspace_bytes=need)
    other = torch.empty((48, 768), dtype=torch.float32, device=dev)
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        cabi.matmul_noalloc_raw(*args, out.data_ptr(), stream=s.cuda_stream)  # eager warm-up
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        cabi.matmul_noalloc_raw(*args, out.data_ptr(), stream=s.cuda_stream)
    torch.cuda.synchronize()
    for rep in range(4):
        out.fill_(float("nan"))
        cabi.matmul_noalloc_raw(*args2, other.data_ptr())  # overwrites the scratch array
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), rep
    del keep, keep2


_FIRST_CALL_UNDER_CAPTURE = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
from tests.conftest import load_package
pkg = load_package()
cabi, inputs = pkg.cabi, pkg.inputs
dev = torch.device("cuda:0")
m, n, k = 64, 1024, 4096
wb, ws = inputs.synthetic_weights(n, k, seed=5)
xt = torch.from_numpy(inputs.synthetic_x(m, k, seed=6)).to(dev)
wbt, wst = torch.from_numpy(wb).to(dev), torch.from_numpy(ws).to(dev)
args = (xt.data_ptr(), cabi.CMK_F32, xt.numel(), m, wbt.data_ptr(), wbt.numel(),
        wst.data_ptr(), wst.numel(), n, k)
need = cabi.workspace_size(cabi.CMK_F32, m, n, k)
work = torch.empty((need,), dtype=torch.uint8, device=dev)
ref = torch.empty((m, n), dtype=torch.float32, device=dev)
cabi.matmul_raw(*args, ref.data_ptr(), workspace_ptr=work.data_ptr(), workspace_bytes=need)
out = torch.full((m, n), float("nan"), dtype=torch.float32, device=dev)
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):  # the first noalloc call of the process
    cabi.matmul_noalloc_raw(*args, out.data_ptr(), stream=s.cuda_stream)
torch.cuda.synchronize()
for rep in range(3):
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), rep
print("first call under capture: ok", flush=True)
"""


def test_noalloc_first_call_under_capture(pkg, dev):
    """In a fresh process, the first cmk_iq2_matmul_noalloc call (which looks
    up the device's scratch address) happens inside stream capture; the graph
    replays give cmk_iq2_matmul's bits (one child process, one GPU user)."""
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE, repo],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    assert "first call under capture: ok" in r.stdout
