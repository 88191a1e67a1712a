"""CPU tier: the C ABI library and the Python API's host logic.

No kernel runs here: the library is loaded, its exports are compared with
include/cuda_llm_abi.h, and calls that must be rejected before any launch are
made with dummy pointers (they never reach the GPU).
"""
import ctypes
import os
import re

import pytest
import torch

import cuda_amd._lib as L
import cuda_llm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cuda_llm_abi.h")


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(ca_\w+)\s*\(([^;{]*?)\)\s*;", text):
        params = [p.strip() for p in m.group(3).split(",") if p.strip() and p.strip() != "void"]
        decls[m.group(2)] = params
    return decls


@pytest.fixture(scope="module")
def lib():
    return L.load()


def test_library_exports_every_declared_symbol(lib):
    decls = _header_functions()
    assert len(decls) >= 8
    for name in decls:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"


def test_binding_table_matches_header():
    decls = _header_functions()
    assert set(decls) == set(L.SIGNATURES)
    for name, params in decls.items():
        assert len(params) == len(L.SIGNATURES[name][1]), name


def test_version_and_workspace_sizes(lib):
    assert b"gfx950" in lib.ca_version()
    # a split is 64 pages of 16 tokens; one split needs no workspace, otherwise
    # N * Hq * splits * (D + 1) floats
    assert lib.ca_decode_workspace_bytes(4, 8, 128, 1024) == 0
    assert lib.ca_decode_workspace_bytes(4, 8, 128, 1025) == 4 * 8 * 2 * 129 * 4
    assert lib.ca_decode_workspace_bytes(64, 32, 128, 8192) == 64 * 32 * 8 * 129 * 4
    assert lib.ca_decode_workspace_bytes(256, 32, 128, 32768) == 256 * 32 * 32 * 129 * 4
    assert lib.ca_decode_workspace_bytes(0, 32, 128, 32768) == 0


P = ctypes.c_void_p(16)  # aligned dummy pointer: never dereferenced on these paths


def _status(name, *args):
    return getattr(L.load(), name)(*args)


def test_prefill_rejects_bad_arguments():
    st = _status("ca_flash_attention_fwd", L.CA_BF16, P, P, P, P, 1, 4, 4, 64, 96, 0.1, 0, None)
    assert st == L.CA_INVALID_ARGUMENT and b"head_dim" in L.load().ca_last_error()
    # float32 is a supported dtype here (the reference instantiates float), so
    # the other checks still apply to it
    st = _status("ca_flash_attention_fwd", L.CA_F32, P, P, P, P, 1, 4, 4, 64, 96, 0.1, 0, None)
    assert st == L.CA_INVALID_ARGUMENT and b"head_dim" in L.load().ca_last_error()
    st = _status("ca_flash_attention_fwd", 7, P, P, P, P, 1, 4, 4, 64, 64, 0.1, 0, None)
    assert st == L.CA_INVALID_ARGUMENT and b"dtype" in L.load().ca_last_error()
    st = _status("ca_flash_attention_fwd", L.CA_BF16, P, P, P, P, 1, 6, 4, 64, 64, 0.1, 0, None)
    assert st == L.CA_INVALID_ARGUMENT and b"multiple" in L.load().ca_last_error()
    st = _status("ca_flash_attention_fwd", L.CA_BF16, ctypes.c_void_p(18), P, P, P, 1, 4, 4, 64,
                 64, 0.1, 0, None)
    assert st == L.CA_INVALID_ARGUMENT and b"aligned" in L.load().ca_last_error()
    # empty problems are a no-op success
    assert _status("ca_flash_attention_fwd", L.CA_BF16, P, P, P, P, 0, 4, 4, 64, 64, 0.1, 0, None) == L.CA_OK


def test_backward_entry_points_validate():
    lib = L.load()
    assert lib.ca_flash_attention_bwd_workspace_bytes(2, 8, 100) == 2 * 8 * 100 * 8
    assert lib.ca_flash_attention_bwd_workspace_bytes(0, 8, 100) == 0
    args = [L.CA_BF16, P, P, P, P, P, P, P, P, P, 1, 4, 2, 64, 64, 0.1, 1, P, 1 << 20, None]
    bad_dtype = list(args)
    bad_dtype[0] = 7
    assert _status("ca_flash_attention_bwd", *bad_dtype) == L.CA_INVALID_ARGUMENT
    small_ws = list(args)
    small_ws[18] = 16
    assert _status("ca_flash_attention_bwd", *small_ws) == L.CA_INVALID_ARGUMENT
    assert b"workspace" in lib.ca_last_error()
    bad_heads = list(args)
    bad_heads[12] = 3
    assert _status("ca_flash_attention_bwd", *bad_heads) == L.CA_INVALID_ARGUMENT
    no_lse = list(args)
    no_lse[6] = None
    assert _status("ca_flash_attention_bwd", *no_lse) == L.CA_INVALID_ARGUMENT
    empty = list(args)
    empty[13] = 0
    assert _status("ca_flash_attention_bwd", *empty) == L.CA_OK
    fwd = [L.CA_BF16, P, P, P, P, None, 1, 4, 4, 64, 64, 0.1, 0, None]
    assert _status("ca_flash_attention_fwd_lse", *fwd) == L.CA_INVALID_ARGUMENT
    assert b"lse" in lib.ca_last_error()


def test_rope_entry_validates():
    lib = L.load()
    # 16-bit: the rotated k (q is rotated as the prefill loads it); float32:
    # the rotated q (256-byte aligned), then k
    n = lib.ca_rope_workspace_bytes(L.CA_BF16, 2, 8, 2, 100, 64)
    assert n == 2 * 2 * 100 * 64 * 2
    n32 = lib.ca_rope_workspace_bytes(L.CA_F32, 2, 8, 2, 100, 64)
    assert n32 == ((2 * 8 * 100 * 64 * 4 + 255) // 256) * 256 + 2 * 2 * 100 * 64 * 4
    args = [L.CA_BF16, P, P, P, P, P, P, 2, 8, 2, 100, 64, 0.1, 1, P, n, None]
    small = list(args)
    small[15] = n - 1
    assert _status("ca_fused_rope_flash_attention", *small) == L.CA_INVALID_ARGUMENT
    assert b"workspace" in lib.ca_last_error()
    no_tab = list(args)
    no_tab[4] = None
    assert _status("ca_fused_rope_flash_attention", *no_tab) == L.CA_INVALID_ARGUMENT
    odd_tab = list(args)
    odd_tab[5] = ctypes.c_void_p(16 + 4)  # the tables are read 16 bytes at a time
    assert _status("ca_fused_rope_flash_attention", *odd_tab) == L.CA_INVALID_ARGUMENT
    assert b"aligned" in lib.ca_last_error()


def test_kv_append_validates():
    lib = L.load()
    args = [L.CA_BF16, 0, P, P, P, P, None, None, 0, P, P, None, 2, 2, 128, 4, 8, 100, None]
    bad_kind = list(args)
    bad_kind[1] = 5
    assert _status("ca_paged_kv_append", *bad_kind) == L.CA_INVALID_ARGUMENT
    fp8_no_scale = list(args)
    fp8_no_scale[1] = 1
    assert _status("ca_paged_kv_append", *fp8_no_scale) == L.CA_INVALID_ARGUMENT
    assert b"k_scale" in lib.ca_last_error()
    f32 = list(args)
    f32[0] = L.CA_F32
    assert _status("ca_paged_kv_append", *f32) == L.CA_UNSUPPORTED
    bad_d = list(args)
    bad_d[14] = 96
    assert _status("ca_paged_kv_append", *bad_d) == L.CA_INVALID_ARGUMENT
    nothing = list(args)
    nothing[15] = 0
    assert _status("ca_paged_kv_append", *nothing) == L.CA_OK


def test_stream_read_validates():
    assert _status("ca_stream_read", None, 1024, P, None) == L.CA_INVALID_ARGUMENT
    assert _status("ca_stream_read", P, 1000, P, None) == L.CA_INVALID_ARGUMENT
    assert b"aligned" in L.load().ca_last_error()
    assert _status("ca_stream_read", P, 0, None, None) == L.CA_OK  # nothing to read


def test_paged_rejects_bad_arguments():
    args = [L.CA_BF16, P, P, P, P, P, P, 2, 8, 2, 128, 4, 16, 10, 0.1, None, 0, None]
    bad_page = list(args)
    bad_page[12] = 8
    assert _status("ca_paged_attention", *bad_page) == L.CA_INVALID_ARGUMENT
    assert b"page_size" in L.load().ca_last_error()
    # 4 blocks x 16 = 64 tokens: one split, no workspace needed -> the size check passes;
    # 200 blocks needs a workspace
    long = list(args)
    long[11] = 200
    assert _status("ca_paged_attention", *long) == L.CA_INVALID_ARGUMENT
    assert b"workspace" in L.load().ca_last_error()
    fp8 = [L.CA_BF16, P, P, P, None, None, 1, P, P, P, 2, 8, 2, 128, 4, 16, 10, 0.1, None, 0, None]
    assert _status("ca_fp8_paged_attention", *fp8) == L.CA_INVALID_ARGUMENT
    # float32 queries are accepted (the reference instantiates
    # dispatch_fp8_paged_attention<float, float>, fp8_paged_attention_
    # instantiations.cu:4): they reach the same argument checks
    fp8_f32 = list(fp8)
    fp8_f32[0] = L.CA_F32
    assert _status("ca_fp8_paged_attention", *fp8_f32) == L.CA_INVALID_ARGUMENT
    assert b"scale" in L.load().ca_last_error()
    fp8_bad_dtype = list(fp8)
    fp8_bad_dtype[0] = 7
    assert _status("ca_fp8_paged_attention", *fp8_bad_dtype) == L.CA_INVALID_ARGUMENT
    assert b"dtype" in L.load().ca_last_error()


def test_mxfp8_rejects_bad_arguments():
    E8, F32 = L.CA_SCALE_E8M0, L.CA_SCALE_F32
    ws = L.load().ca_mx_workspace_bytes(E8, 1, 2, 64, 128)
    assert ws == 1 * 2 * 64 * 128 * 2  # the bf16 V
    wsf = L.load().ca_mx_workspace_bytes(F32, 1, 2, 64, 128)
    assert wsf == ws + 2 * 512         # + q/k scale bytes (256-aligned)
    assert L.load().ca_mx_workspace_bytes(E8, 1, 2, 64, 64) == 0
    assert L.load().ca_mx_workspace_bytes(7, 1, 2, 64, 128) == 0

    def mx(*over, **kw):
        a = dict(dt=L.CA_BF16, kind=E8, d=128, ws=P, wsb=ws, ks=P, qs=P)
        a.update(kw)
        return _status("ca_fused_microscaled_attention", a["dt"], P, a["qs"], P, a["ks"], P, P, a["kind"],
                       P, 1, 2, 64, a["d"], 0.1, 1, a["ws"], a["wsb"], None)
    assert mx(d=64) == L.CA_INVALID_ARGUMENT
    assert mx(dt=L.CA_F32) == L.CA_UNSUPPORTED
    assert mx(kind=5) == L.CA_INVALID_ARGUMENT
    assert b"scale kind" in L.load().ca_last_error()
    assert mx(wsb=ws - 1) == L.CA_INVALID_ARGUMENT
    assert b"workspace" in L.load().ca_last_error()
    assert mx(kind=F32) == L.CA_INVALID_ARGUMENT  # the float form needs the larger workspace
    assert mx(ks=ctypes.c_void_p(18)) == L.CA_INVALID_ARGUMENT
    assert b"aligned" in L.load().ca_last_error()
    assert mx(qs=ctypes.c_void_p(17)) == L.CA_INVALID_ARGUMENT      # e8m0 q scales too: dword loads
    assert b"aligned" in L.load().ca_last_error()


def test_python_api_requires_device_tensors():
    q = torch.randn(1, 2, 8, 64)
    with pytest.raises(RuntimeError, match="Inputs must be on CUDA"):
        cuda_llm.flash_attention(q, q, q)
    with pytest.raises(RuntimeError, match="Inputs must be on CUDA"):
        cuda_llm.flash_decode(q[:, :, :1], q, q)
    bt = torch.zeros(1, 1, dtype=torch.int32)
    lens = torch.ones(1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="on CUDA"):
        cuda_llm.paged_attention(q[:, :, 0], torch.zeros(1, 2, 64, 16), torch.zeros(1, 2, 64, 16), bt, lens)


def test_mx_scale_conversion():
    b = torch.randint(100, 150, (3, 4), dtype=torch.uint8)
    assert torch.equal(cuda_llm.mx_scales_to_e8m0(b), b)
    f = torch.ldexp(torch.ones(3, 4), b.to(torch.int32) - 127)
    assert torch.equal(cuda_llm.mx_scales_to_e8m0(f), b)
    assert torch.equal(cuda_llm.mx_scales_to_e8m0(b.view(torch.float8_e8m0fnu)), b)
    with pytest.raises(RuntimeError, match="powers of two"):
        cuda_llm.mx_scales_to_e8m0(torch.full((2,), 3.0))


def test_reference_module_name_imports():
    """The reference's callers `import fused_online_softmax_cuda` (tests/
    conftest.py:25, setup.py:128 there): the module exists and binds the
    attention entry points of fused_softmax_binding.cpp:721-809 to this
    build's functions; names outside the attention forward path raise
    AttributeError (as in a reference build compiled without them)."""
    import importlib
    m = importlib.import_module("fused_online_softmax_cuda")
    for name in ("flash_attention_forward", "flash_attention_v3_hopper", "fused_gqa_forward",
                 "async_flash_decode", "paged_attention_forward", "fp8_paged_attention_forward",
                 "fused_rope_flash_attention", "flash_attention_backward"):
        assert getattr(m, name) is getattr(cuda_llm, name), name
    for name in ("forward", "fused_mla_forward", "fused_llama_megablock", "no_such_thing"):
        with pytest.raises(AttributeError):
            getattr(m, name)
    q = torch.randn(1, 2, 8, 64)
    with pytest.raises(RuntimeError, match="Inputs must be on CUDA"):
        m.flash_attention_forward(q, q, q)


def test_check_block_tables_argument_checks():
    """ca_check_block_tables rejects bad sizes before touching device memory."""
    assert _status("ca_check_block_tables", P, P, -1, 4, 10, 16, None) == L.CA_INVALID_ARGUMENT
    assert _status("ca_check_block_tables", P, P, 2, 4, 10, 0, None) == L.CA_INVALID_ARGUMENT
    assert _status("ca_check_block_tables", None, None, 2, 4, 10, 16, None) == L.CA_INVALID_ARGUMENT
    assert b"null" in L.load().ca_last_error()
    assert _status("ca_check_block_tables", None, None, 0, 4, 10, 16, None) == L.CA_OK


def test_check_mx_scales_argument_checks():
    """ca_check_mx_scales rejects bad sizes, null and misaligned pointers
    before touching device memory; an empty shape is OK."""
    assert _status("ca_check_mx_scales", P, P, P, -1, 2, 8, 128, None) == L.CA_INVALID_ARGUMENT
    assert _status("ca_check_mx_scales", P, P, P, 1, 2, 8, 100, None) == L.CA_INVALID_ARGUMENT
    assert _status("ca_check_mx_scales", None, P, P, 1, 2, 8, 128, None) == L.CA_INVALID_ARGUMENT
    assert b"null" in L.load().ca_last_error()
    assert _status("ca_check_mx_scales", ctypes.c_void_p(18), P, P, 1, 2, 8, 128, None) == L.CA_INVALID_ARGUMENT
    assert b"aligned" in L.load().ca_last_error()
    assert _status("ca_check_mx_scales", None, None, None, 1, 2, 0, 128, None) == L.CA_OK
