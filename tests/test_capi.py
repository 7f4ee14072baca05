"""CPU checks of the C ABI: the library loads, exports every declared symbol,
and the argument-validation paths return the documented status codes without
touching a GPU (no compute call is made here)."""
import ctypes as C
import os
import re

import pytest

from supersonic_amd import kernel_ffi as K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol(lib):
    names = K.header_functions()
    assert len(names) >= 17
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(K.SIGNATURES)


def test_library_exports_exactly_the_header():
    """The shipped .so exports the header's functions and nothing else of its
    own (no probe or trace entry points)."""
    import shutil
    import subprocess
    nm = shutil.which("nm") or "/usr/bin/nm"
    out = subprocess.run([nm, "-D", "--defined-only", K.LIB_PATH], capture_output=True, text=True, check=True).stdout
    funcs = {ln.split()[-1] for ln in out.splitlines() if len(ln.split()) == 3 and ln.split()[1] == "T"}
    ours = {f for f in funcs if f.startswith(("supersonic_", "ssa_"))}
    assert ours == set(K.header_functions())


def test_reference_symbols_are_declared():
    """The drop-in set: every reference bridge symbol on the path
    (prefill_ffi.rs:635-950) is declared with the reference's name."""
    need = {
        "supersonic_qwen35_hip_full_attention_prefill", "supersonic_qwen35_4b_hip_full_attention_prefill",
        "supersonic_qwen35_hip_full_attention_decode_flat", "supersonic_qwen35_hip_full_attention_decode_flat_strided",
        "supersonic_qwen35_4b_hip_quantize_kv_to_fp8", "supersonic_qwen35_hip_rms_norm", "supersonic_qwen35_hip_cast",
        "supersonic_qwen35_hip_apply_rope_prefill", "supersonic_qwen35_hip_transpose_shd_hsd",
        "supersonic_qwen35_hip_sigmoid_mul", "supersonic_qwen35_hip_split_qgate",
    }
    assert need <= set(K.header_functions())


def test_kv_cache_struct_layout_matches_header():
    text = open(os.path.join(ROOT, "include", "supersonic_attn.h")).read()
    body = re.search(r"typedef struct supersonic_kv_cache \{(.*?)\}", text, re.S).group(1)
    fields = re.findall(r"(\w+);", body)
    assert fields == [f[0] for f in K.KvCacheDesc._fields_]
    assert C.sizeof(K.KvCacheDesc) == 8 * 5 + 8 * 3 + 4 * 2 + 8 * 3


def test_version(lib):
    assert K.version().startswith("supersonic-attn-gfx950")


@pytest.mark.parametrize("fn,args,code", [
    ("supersonic_qwen35_hip_full_attention_prefill", (9, 0, 1, 1, 1, 1, 1, 64, 1, 1.0, 0, None, None, None, None), 64),
    ("supersonic_qwen35_hip_full_attention_prefill", (2, 0, 1, 1, 1, 1, 1, 0, 1, 1.0, 0, None, None, None, None), 14),
    ("supersonic_qwen35_hip_full_attention_prefill", (2, 0, 1, 1, 1, 1, 1, 1024, 1, 1.0, 0, None, None, None, None), 14),
    ("supersonic_qwen35_hip_full_attention_decode_flat", (1, 0, 1, 1, 1, 1, 256, 1, 1.0, None, None, None, None), 400),
    ("supersonic_qwen35_hip_full_attention_decode_flat", (2, 0, 1, 1, 1, 1, 512, 1, 1.0, None, None, None, None), 401),
    ("supersonic_qwen35_hip_full_attention_decode_flat_strided",
     (2, 0, 1, 1, 1, 10, 5, 256, 1, 1.0, None, None, None, None), 401),
    ("supersonic_qwen35_4b_hip_quantize_kv_to_fp8", (0, 0, None, None, None, 1, 1, 256, 1, 0), 256),
    ("supersonic_qwen35_hip_rms_norm", (5, 0, 1, 1, 1e-6, 1, None, None, None), 74),
    ("supersonic_qwen35_hip_cast", (5, 2, 0, 1, None, None), 137),
    ("supersonic_qwen35_hip_cast", (2, 5, 0, 1, None, None), 137),
    ("supersonic_qwen35_hip_apply_rope_prefill", (5, 0, 1, 1, 64, 16, None, None, None), 310),
    ("supersonic_qwen35_hip_transpose_shd_hsd", (5, 0, 1, 1, 1, None, None), 320),
    ("supersonic_qwen35_hip_sigmoid_mul", (5, 0, 1, None, None, None), 350),
    ("supersonic_qwen35_hip_split_qgate", (5, 0, 1, 1, 1, None, None, None), 370),
    ("supersonic_qwen35_4b_hip_matmul_rhs_transposed_tiled", (1, 0, 1, 1, 1, 8, None, None, None), 272),
    ("supersonic_qwen35_4b_hip_matmul_rhs_transposed_tiled", (0, 0, 1, 1, 1, 8, None, None, None), 272),
    ("supersonic_qwen35_hip_element_add", (5, 0, 1, None, None, None), 300),
])
def test_validation_status_codes(lib, fn, args, code):
    assert getattr(lib, fn)(*args) == code


def test_fused_entry_validation(lib):
    desc = K.KvCacheDesc()
    p = 0x1000  # never dereferenced: validation fails first
    dec = lambda kvd, hd, rot, q=p: lib.supersonic_attn_gfx950_decode(
        0, None, kvd, 1, 8, 2, hd, rot, 16, 1e-6, 0.0625, q, p, p, p, p, p, p, p, C.byref(desc), p, None, 0)
    assert dec(7, 256, 64) == K.ERR["DTYPE"]
    assert dec(2, 256, 64, q=None) == K.ERR["NULL"]
    assert dec(2, 256, 63) == K.ERR["ROTARY"]
    assert dec(2, 256, 64) == K.ERR["NULL"]          # the cache view has no K pointer
    desc.k = desc.v = p
    assert dec(3, 256, 64) == K.ERR["NULL"]          # fp8 without scale pointers
    assert dec(2, 96, 32) == K.ERR["HEAD_DIM"]
    desc.block_table = p
    desc.page_size = 40
    desc.max_pages_per_seq = 4
    assert dec(2, 256, 64) == K.ERR["CACHE"]         # pages must hold whole 16-token blocks
    desc.block_table = None
    pre = lambda kvd, hq, hkv, hd, rot: lib.supersonic_attn_gfx950_prefill(
        0, None, kvd, hq, hkv, hd, rot, 16, 0, 1e-6, 0.0625, p, p, p, p, p, p, p, C.byref(desc), p, None, 0)
    assert pre(9, 16, 4, 256, 64) == K.ERR["DTYPE"]
    assert pre(2, 16, 5, 256, 64) == K.ERR["HEADS"]
    assert pre(2, 16, 4, 200, 64) == K.ERR["HEAD_DIM"]
    assert pre(2, 16, 4, 256, 40) == K.ERR["ROTARY"]
    att = lambda kvd: lib.supersonic_attn_gfx950_decode_attend(0, None, kvd, 1, 8, 2, 256, 16, 0.0625, None, p,
                                                               C.byref(desc), None, p, None, 0)
    assert att(2) == K.ERR["NULL"]


def test_projection_entry_validation(lib):
    p = 0x1000  # never dereferenced: validation fails first
    op = lambda hd, rows, hid, adim, attn=p, w=p, h=p: lib.supersonic_attn_gfx950_o_proj_residual(
        0, None, hd, rows, hid, adim, attn, w, h, None, 0)
    assert op(0, 8, 64, 64) == K.ERR["DTYPE"]          # f16 hidden is not a reference layout
    assert op(2, 8, 64, 64, h=None) == K.ERR["NULL"]
    assert op(1, 8, 64, 64, w=None) == K.ERR["NULL"]
    assert op(2, 1 << 31, 64, 64) == K.ERR["RANGE"]
    assert op(2, 0, 64, 64, attn=None, w=None, h=None) == 0  # nothing to do
    qkv = lambda hd, hid, nq=64, nkv=16, x=p, kw=p: lib.supersonic_attn_gfx950_qkv_proj(
        0, None, hd, 4, hid, nq, nkv, 1e-6, x, p, p, kw, p, p, p, p, None, 0)
    assert qkv(0, 64) == K.ERR["DTYPE"]
    assert qkv(2, 64, x=None) == K.ERR["NULL"]
    assert qkv(1, 64, kw=None) == K.ERR["NULL"]
    assert qkv(2, 60) == K.ERR["RANGE"]                # rows are read 16 bytes at a time
    assert qkv(2, 0) == K.ERR["RANGE"]


def test_mixed_workspace_size_is_host_only(lib):
    """The mixed step's workspace: 2 KiB of claim counters, then the decode's and the
    chunk's workspaces, each rounded up to 256 bytes (no GPU call; the tensors are
    only read for their shapes and pointers)."""
    import torch
    Hq, Hkv, D, S, B = 16, 2, 256, 300, 3
    cache = K.KvCache(torch.zeros(1, Hkv, 8, D, dtype=torch.bfloat16), torch.zeros(1, Hkv, 8, D, dtype=torch.bfloat16))
    chunk = {"q_proj": torch.zeros(S, 1), "k_new": None, "v_new": None, "cache": cache, "out": None,
             "chunk_start": 40}
    dec = {"q_proj": torch.zeros(B, 1), "k_new": None, "v_new": None, "positions": None, "cache": cache,
           "out": None, "max_kv_len": 5000}
    r256 = lambda n: (n + 255) // 256 * 256
    dws = r256(K.decode_workspace_size(B, Hq, Hkv, D, 5000))
    pws = r256(K.prefill_workspace_size(False, Hkv, D, S, 40))
    assert K.mixed_workspace_size(False, Hq, Hkv, D, chunk, dec) == 2048 + dws + pws
    assert K.mixed_workspace_size(False, Hq, Hkv, D, chunk, None) == 2048 + pws
    assert K.mixed_workspace_size(False, Hq, Hkv, D, None, dec) == 2048 + dws
    assert K.mixed_workspace_size(False, Hq, Hkv, D, None, None) == 2048


def test_workspace_size_is_host_only(lib):
    n = K.decode_workspace_size(1, 16, 4, 256, 32769)
    assert n > 16 * 256 * 4
    assert K.decode_workspace_size(8, 16, 4, 256, 32769) >= n
    # prefill: the V^T staging of every position (x2 with an fp8 cache)
    assert K.prefill_workspace_size(False, 4, 256, 4096, 0) == 4 * 256 * 4096 * 2
    assert K.prefill_workspace_size(True, 4, 256, 100, 30) == 2 * 4 * 256 * 192 * 2
    # projections: decode rows need only the k-split counters/partials (or nothing)
    assert K.o_proj_workspace_size(8, 4096, 4096) < (1 << 22)
    assert K.qkv_proj_workspace_size(8, 4096, 8192, 1024) >= 8 * 4096 * 2
    # GEMM-sized rows: the hand-written GEMM adds into the hidden rows in place
    assert 0 < K.o_proj_workspace_size(100, 4096, 4096) <= 4096
    assert K.qkv_proj_workspace_size(100, 4096, 8192, 1024) >= 100 * 4096 * 2


@pytest.mark.parametrize("rot,max_pos,theta", [(64, 70000, 1.0e7), (32, 4097, 1.0e4), (128, 513, 1.0e6)])
def test_rope_tables_match_oracle(lib, rot, max_pos, theta):
    """The library's host table builder equals the oracle's RotaryTables::build
    restatement (itself pinned by a float64 brute force) bit for bit."""
    from oracle import attn_oracle as O
    import torch
    cos, sin = K.rope_tables(rot, max_pos, theta)
    rc, rs = O.rope_tables(rot, max_pos, theta)
    assert torch.equal(cos.view(torch.int16), rc.view(torch.int16))
    assert torch.equal(sin.view(torch.int16), rs.view(torch.int16))


def test_rope_tables_validation(lib):
    assert lib.supersonic_attn_rope_tables(63, 4, 1e4, None, None) == K.ERR["ROTARY"]
    assert lib.supersonic_attn_rope_tables(64, 4, 0.0, None, None) == K.ERR["ROTARY"]
    assert lib.supersonic_attn_rope_tables(64, 4, 1e4, None, None) == K.ERR["NULL"]


def test_qkv_proj_rope_validation(lib):
    p = 0x1000  # never dereferenced: validation fails first
    desc = K.KvCacheDesc()
    f = lambda hd=2, hdim=256, hq=16, hkv=4, rot=64, x=p, cache=None: lib.supersonic_attn_gfx950_qkv_proj_rope(
        0, None, hd, 4, 512, hq, hkv, hdim, rot, 1e-6, 1e-6, x, p, p, p, p, p, p, p, p, p, p, p, p, p,
        cache, None, 0)
    assert f(hd=0) == K.ERR["DTYPE"]
    assert f(hdim=100) == K.ERR["HEAD_DIM"]
    assert f(hkv=5) == K.ERR["HEADS"]
    assert f(rot=63) == K.ERR["ROTARY"]
    assert f(x=None) == K.ERR["NULL"]
    desc.k = desc.v = p
    desc.k_scale = desc.v_scale = p
    assert f(cache=C.byref(desc)) == K.ERR["CACHE"]   # fp8 caches are not appended here
    assert K.qkv_proj_rope_workspace_size(8, 4096, 16, 4, 256) > 8 * 4096 * 2
