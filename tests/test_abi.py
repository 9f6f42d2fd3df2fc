"""The C ABI on the host: the library loads, exports every symbol that
include/cmk_iq2.h declares, and rejects invalid arguments with the reference's
error texts before touching any device (so these run without a GPU)."""

import ctypes
import os
import re

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "cmk_iq2.h")


def declared_symbols():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(cmk_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol(cabi):
    L = cabi.lib()
    syms = declared_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(L, s), s
    assert sorted(cabi.EXPORTED) == syms
    assert L.cmk_abi_version() == 3


NULL = None


def call(cabi, **kw):
    args = dict(x=NULL, x_dtype=0, x_len=0, m=1, wb=NULL, wb_len=1 << 20, ws=NULL, ws_len=1 << 20,
                out_dim=7, in_dim=320, variant=0, mode=0, strict=0, out=NULL, work=NULL,
                work_bytes=0, stream=NULL)
    args.update(kw)
    rc = cabi.lib().cmk_iq2_matmul(args["x"], args["x_dtype"], args["x_len"], args["m"],
                                   args["wb"], args["wb_len"], args["ws"], args["ws_len"],
                                   args["out_dim"], args["in_dim"], args["variant"], args["mode"],
                                   args["strict"], args["out"], args["work"], args["work_bytes"],
                                   args["stream"])
    return rc, cabi.last_error()


def test_zero_dims(cabi):
    for od, idim in ((0, 320), (7, 0)):
        rc, msg = call(cabi, out_dim=od, in_dim=idim)
        assert rc == cabi.CMK_ERR_INVALID_ARGUMENT
        assert msg == "iq2_matmul expects non-zero dimensions"


def test_w4a8_strict_and_fallback(cabi):
    rc, msg = call(cabi, mode=cabi.CMK_ACT_QUANT_W4A8, strict=1)
    assert rc == cabi.CMK_ERR_UNSUPPORTED
    assert msg == ("activation quant mode W4A8 requested in strict mode, but W4A8 kernel path is "
                   "not implemented yet")
    # non-strict W4A8 runs as Off: it reaches the Off path's own checks
    rc, msg = call(cabi, mode=cabi.CMK_ACT_QUANT_W4A8, strict=0, out_dim=0)
    assert msg == "iq2_matmul expects non-zero dimensions"


# bytes / scales per block of each variant (src/iq2_matmul.rs:13-29,39-57)
VARIANT_SIZES = {0: (64, 2), 1: (64, 10), 2: (72, 10), 3: (104, 6)}


def test_variant_size_checks(cabi):
    """Every variant is served; its buffers are checked against its own block
    sizes with the reference's texts (src/iq2_matmul.rs:238-259)."""
    for v, (bpb, spb) in VARIANT_SIZES.items():
        need_b, need_s = 7 * 2 * bpb, 7 * 2 * spb
        rc, msg = call(cabi, variant=v, wb_len=need_b - 1)
        assert rc == cabi.CMK_ERR_INVALID_ARGUMENT
        assert msg == f"iq2_matmul weight_bytes too small: got {need_b - 1} expected at least {need_b}"
        rc, msg = call(cabi, variant=v, wb_len=need_b, ws_len=need_s - 1)
        assert msg == (f"iq2_matmul weight_scales too small: got {need_s - 1} expected at least "
                       f"{need_s}")
        # exact sizes pass the size checks and stop at the missing x buffer
        rc, msg = call(cabi, variant=v, wb_len=need_b, ws_len=need_s)
        assert msg == "iq2_matmul x too small: got 0 expected at least 320"
    rc, msg = call(cabi, variant=9)
    assert rc == cabi.CMK_ERR_INVALID_ARGUMENT and msg == "invalid iq2 variant: 9"


def test_bad_dtype(cabi):
    rc, msg = call(cabi, x_dtype=7)
    assert rc == cabi.CMK_ERR_INVALID_ARGUMENT and msg == "iq2_matmul unsupported x dtype: 7"
    rc, msg = call(cabi, x_dtype=7, mode=cabi.CMK_ACT_QUANT_W8A8)
    assert msg == "iq2_matmul_w8a8 unsupported x dtype: 7"


def test_buffer_sizes(cabi):
    # N=7, K=320 -> 7 rows x 2 blocks: 896 bytes, 28 scale bytes (src/iq2_matmul.rs:237-259)
    rc, msg = call(cabi, wb_len=895, ws_len=28)
    assert rc == cabi.CMK_ERR_INVALID_ARGUMENT
    assert msg == "iq2_matmul weight_bytes too small: got 895 expected at least 896"
    rc, msg = call(cabi, wb_len=896, ws_len=27)
    assert msg == "iq2_matmul weight_scales too small: got 27 expected at least 28"
    rc, msg = call(cabi, wb_len=896, ws_len=28, x_len=639, m=2)
    assert msg == "iq2_matmul x too small: got 639 expected at least 640"
    rc, msg = call(cabi, wb_len=896, ws_len=28, x_len=640, m=2)
    assert msg == "iq2_matmul null pointer argument"


def test_overflow_and_u32_limits(cabi):
    rc, msg = call(cabi, out_dim=1 << 62, in_dim=1 << 40)
    assert msg == "iq2_matmul bytes size overflow"
    rc, msg = call(cabi, m=1 << 32, out_dim=1, in_dim=256, wb_len=64, ws_len=2)
    assert msg == "m too large"
    rc, msg = call(cabi, m=1, out_dim=1 << 32, in_dim=256, wb_len=1 << 40, ws_len=1 << 40)
    assert msg == "out_dim too large"


def test_empty_activation_is_a_noop(cabi):
    rc, msg = call(cabi, m=0, wb_len=896, ws_len=28)
    assert rc == cabi.CMK_OK and msg == ""


def test_dequantize_validation(cabi):
    L = cabi.lib()

    def dq(**kw):
        a = dict(wb=NULL, wbl=896, ws=NULL, wsl=28, od=7, idim=320, v=0, dt=1, out=NULL)
        a.update(kw)
        rc = L.cmk_iq2_dequantize(a["wb"], a["wbl"], a["ws"], a["wsl"], a["od"], a["idim"], a["v"],
                                  a["dt"], a["out"], NULL)
        return rc, cabi.last_error()

    assert dq(od=0)[1] == "iq2_dequantize_to_f16 expects non-zero dimensions"
    assert dq(wbl=10)[1] == ("iq2_dequantize_to_f16 weight_bytes too small: got 10 expected at "
                             "least 896")
    assert dq(wsl=1)[1] == ("iq2_dequantize_to_f16 weight_scales too small: got 1 expected at "
                            "least 28")
    # IQ2_S: 72 + 10 bytes per block
    assert dq(v=2)[1] == ("iq2_dequantize_to_f16 weight_bytes too small: got 896 expected at "
                          "least 1008")
    assert dq(v=2, wbl=1008)[1] == ("iq2_dequantize_to_f16 weight_scales too small: got 28 "
                                    "expected at least 140")
    assert dq(v=3, wbl=1456, wsl=84)[1] == "iq2_dequantize_to_f16 null pointer argument"
    assert "unsupported output dtype" in dq(dt=5)[1]
    assert dq()[1] == "iq2_dequantize_to_f16 null pointer argument"


def test_workspace_and_path_queries(cabi):
    assert cabi.workspace_size(cabi.CMK_F16, 512, 14336, 4096) == 0
    # W8A8 on the GEMM path: row scales (256-byte aligned) + quantised activations
    assert (cabi.workspace_size(cabi.CMK_F16, 512, 14336, 4096, mode=cabi.CMK_ACT_QUANT_W8A8)
            == 2048 + 512 * 4096 * 2)
    assert cabi.workspace_size(cabi.CMK_F32, 1, 4096, 4096, mode=cabi.CMK_ACT_QUANT_OFF) == 0
    assert cabi.matmul_path(cabi.CMK_F16, 512, 14336, 4096) == "gemm"
    assert cabi.matmul_path(cabi.CMK_BF16, 17, 14336, 4096) == "gemm"
    assert cabi.matmul_path(cabi.CMK_BF16, 9, 14336, 4096) == "gemv"
    assert cabi.matmul_path(cabi.CMK_F16, 16, 14336, 4096) == "gemv"
    assert cabi.matmul_path(cabi.CMK_F16, 8, 14336, 4096) == "gemv"
    assert cabi.matmul_path(cabi.CMK_F32, 1, 14336, 4096) == "gemv"
    # f32 rows keep the exact-weight GEMV up to 16 rows; beyond, they are
    # staged for the GEMM: row scales plus f16 head / tail row pairs (mode Off)
    # or the f16 W8A8 rows
    assert cabi.matmul_path(cabi.CMK_F32, 8, 14336, 4096) == "gemv"
    assert cabi.matmul_path(cabi.CMK_F32, 9, 14336, 4096) == "gemv"
    assert cabi.matmul_path(cabi.CMK_F32, 16, 14336, 4096) == "gemv"
    assert cabi.matmul_path(cabi.CMK_F32, 17, 14336, 4096) == "gemm"
    assert cabi.workspace_size(cabi.CMK_F32, 16, 14336, 4096) == 0
    # (+ the k-split partials where the tiles cannot fill half of the 256 CUs:
    # 256 staged rows x 8192 -> 64 tiles of 256 x 128, k split in 4 (8 blocks each):
    # 256 x 112 tiles would be 74 split in 3 (11 blocks each, 222 workgroups))
    assert (cabi.workspace_size(cabi.CMK_F32, 128, 8192, 8192)
            == 512 + 2 * 128 * 8192 * 2 + 4 * 128 * 8192 * 4)
    # N = 28672 keeps 256 x 112 (256 tiles, no split); N = 1024 too (10 tiles
    # split in 16, where 256 x 128 gives 8 tiles split in 16)
    assert cabi.workspace_size(cabi.CMK_F32, 128, 28672, 8192) == 512 + 2 * 128 * 8192 * 2
    assert (cabi.workspace_size(cabi.CMK_F32, 128, 1024, 8192)
            == 512 + 2 * 128 * 8192 * 2 + 16 * 128 * 1024 * 4)
    # 64 rows x 4096 -> 32 tiles, 16 blocks per row split in 8 (two blocks each)
    assert (cabi.workspace_size(cabi.CMK_F32, 64, 4096, 4096, mode=cabi.CMK_ACT_QUANT_W8A8)
            == 256 + 64 * 4096 * 2 + 8 * 64 * 4096 * 4)
    # half x: partials only; 8 tiles of 128 x 1024, 32 blocks per row split in 16
    assert cabi.workspace_size(cabi.CMK_F16, 128, 1024, 8192) == 16 * 128 * 1024 * 4
    # 256 tiles (the M=512 prefill shape) or too few blocks: no split; bf16
    # rows are staged as scaled f16 (row scales + the rows) for f16 weights
    assert cabi.workspace_size(cabi.CMK_BF16, 17, 64, 320) == 256 + 17 * 320 * 2
    # in_dim % 8 != 0 keeps f32 rows off the GEMM: the multi-row kernel in
    # launches of 16 rows, too short a K to split
    assert cabi.matmul_path(cabi.CMK_F32, 64, 300, 1001) == "gemv"
    assert cabi.workspace_size(cabi.CMK_F32, 64, 300, 1001) == 0
    # the multi-row kernel's split over K (optional workspace) where it pays:
    # N = 4096 has 128 row groups of 32 on 256 CUs -> 2 parts, taken by the
    # 16-row launches at K = 4096 (arrival words, part masks, the parts' sums)
    # and by every launch at K >= 12288; N = 14336 fills the CUs
    for m in (2, 4, 8):
        assert cabi.workspace_size(cabi.CMK_F32, m, 4096, 4096) == 0
    for m in (12, 16):
        assert cabi.workspace_size(cabi.CMK_F32, m, 4096, 4096) == 1024 + 1024 + 2 * m * 4096 * 4
    for m in (2, 8):
        assert cabi.workspace_size(cabi.CMK_F32, m, 4096, 14336) == 1024 + 1024 + 2 * m * 4096 * 4
    for m in (2, 16):
        assert cabi.workspace_size(cabi.CMK_F32, m, 14336, 4096) == 0
    # W8A8: the 32-row launches (m > 8) split at K = 4096, the 8-row ones not
    assert (cabi.workspace_size(cabi.CMK_F32, 32, 4096, 4096, mode=cabi.CMK_ACT_QUANT_W8A8)
            == 1024 + 1024 + 2 * 32 * 4096 * 4)
    # (the 8-row ones: the portable path's row scales only, reported in case
    # unaligned weights send the call there)
    assert cabi.workspace_size(cabi.CMK_F32, 8, 4096, 4096, mode=cabi.CMK_ACT_QUANT_W8A8) == 256
    # N = 1024: 32 row groups -> 8 parts, taken at K = 8192 by 16-row launches
    assert cabi.workspace_size(cabi.CMK_F16, 16, 1024, 8192) == 256 + 1024 + 8 * 16 * 1024 * 4
    assert cabi.workspace_size(cabi.CMK_F16, 16, 1024, 4096) == 0
    # IQ2_XS rows take the same split
    assert (cabi.workspace_size(cabi.CMK_F32, 16, 4096, 4096, variant=cabi.CMK_IQ2_XS)
            == 1024 + 1024 + 2 * 16 * 4096 * 4)
    with pytest.raises(cabi.CmkError):
        cabi.workspace_size(cabi.CMK_F16, 1, 0, 4096)


def test_split_gguf_blocks_argument_errors(cabi):
    L = cabi.lib()

    def sp(**kw):
        a = dict(src=NULL, sl=0, n=3, v=1, wb=NULL, wbl=1 << 20, ws=NULL, wsl=1 << 20)
        a.update(kw)
        rc = L.cmk_iq2_split_gguf_blocks(a["src"], a["sl"], a["n"], a["v"], a["wb"], a["wbl"],
                                         a["ws"], a["wsl"], NULL)
        return rc, cabi.last_error()

    assert sp(v=7)[1] == "invalid iq2 variant: 7"
    assert sp(sl=221)[1] == "split_gguf_blocks blocks too small: got 221 expected at least 222"
    assert sp(sl=222, wbl=191)[1] == ("split_gguf_blocks weight_bytes too small: got 191 expected "
                                      "at least 192")
    assert sp(sl=222, wsl=29)[1] == ("split_gguf_blocks weight_scales too small: got 29 expected "
                                     "at least 30")
    assert sp(sl=222)[1] == "split_gguf_blocks null pointer argument"
    assert sp(n=0)[0] == cabi.CMK_OK


def test_swiglu_argument_errors(cabi):
    L = cabi.lib()
    assert L.cmk_swiglu(NULL, NULL, 4, 7, NULL, NULL) == cabi.CMK_ERR_INVALID_ARGUMENT
    assert cabi.last_error() == "swiglu unsupported output dtype: 7"
    assert L.cmk_swiglu(NULL, NULL, 4, 0, NULL, NULL) == cabi.CMK_ERR_INVALID_ARGUMENT
    assert cabi.last_error() == "swiglu null pointer argument"
    assert L.cmk_swiglu(NULL, NULL, 0, 0, NULL, NULL) == cabi.CMK_OK



def test_rust_ffi_declarations_match_header():
    """The Rust binding (not built here) declares only functions of the header,
    each with the header's parameter count."""
    import re
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    rs = open(os.path.join(repo, "candelora-metal-kernels_amd", "rust", "src", "hip",
                           "ffi.rs")).read()
    hdr = open(os.path.join(repo, "include", "cmk_iq2.h")).read()

    def params(text, name, open_pat):
        m = re.search(open_pat % re.escape(name), text)
        assert m, name
        depth, i = 1, m.end()
        while depth:
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        body = text[m.end():i - 1].strip()
        return 0 if body in ("", "void") else body.count(",") + 1

    names = re.findall(r"pub fn (cmk_\w+)\(", rs)
    assert len(names) >= 10
    for n in names:
        assert params(rs, n, r"pub fn %s\(") == params(hdr, n, r"\b%s\("), n
