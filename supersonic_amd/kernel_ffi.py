"""Host-side binding of the gfx950 attention library (ctypes over the C ABI).

Mirrors the safe wrappers of the reference crate ``kernel-ffi``
(crates/kernel-ffi/src/prefill_ffi.rs): same function names, argument order
and meaning, ``ScalarType`` dtype codes, and a ``GpuError`` raised with the
same message shape (``"<op> failed: <status>"``, prefill_ffi.rs:1283-1290)
whenever the C function returns a non-zero status.

Buffers are torch tensors used only as device memory (``data_ptr``); nothing
here computes.  If the shared library is missing this module raises on load:
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from dataclasses import dataclass
from typing import Optional, Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("SUPERSONIC_ATTN_LIB") or os.path.join(HERE, "libsupersonic_attn.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "supersonic_attn.h")


class GpuError(RuntimeError):
    """Non-zero status from the C ABI (mirrors gpu_hal::GpuError)."""

    def __init__(self, op: str, status: int):
        super().__init__(f"{op} failed: {status}")
        self.op = op
        self.status = status


class ScalarType:
    """``ScalarType::kernel_dtype_code`` (crates/gpu-hal/src/scalar_type.rs:25-32)."""
    F16 = 0
    F32 = 1
    BF16 = 2


KV_BF16 = 2
KV_FP8_E4M3 = 3

ERR = {
    "DTYPE": 1001, "HEAD_DIM": 1002, "HEADS": 1003, "NULL": 1004, "ROTARY": 1005,
    "WORKSPACE": 1006, "LAUNCH": 1007, "SYNC": 1008, "RANGE": 1009, "CACHE": 1010,
    "COOPERATIVE": 1011,
}
WAIT_LAYER_BARRIER = 1
WAIT_DECODE_MERGE = 2
WAIT_GEMM_TAIL = 4


class KvCacheDesc(C.Structure):
    """``supersonic_kv_cache`` (include/supersonic_attn.h)."""
    _fields_ = [
        ("k", C.c_void_p), ("v", C.c_void_p), ("k_scale", C.c_void_p), ("v_scale", C.c_void_p),
        ("block_table", C.c_void_p),
        ("seq_stride", C.c_int64), ("head_stride", C.c_int64), ("page_stride", C.c_int64),
        ("page_size", C.c_int32), ("max_pages_per_seq", C.c_int32),
        ("scale_seq_stride", C.c_int64), ("scale_head_stride", C.c_int64), ("scale_page_stride", C.c_int64),
    ]


_sz = C.c_size_t
_p = C.c_void_p
_i = C.c_int
_f = C.c_float


class PrefillChunkDesc(C.Structure):
    """``supersonic_prefill_chunk`` (include/supersonic_attn.h)."""
    _fields_ = [("chunk_len", C.c_size_t), ("chunk_start", C.c_size_t), ("q_proj", C.c_void_p),
                ("k_new", C.c_void_p), ("v_new", C.c_void_p), ("cache", C.POINTER(KvCacheDesc)),
                ("out", C.c_void_p)]


class DecodeBatchDesc(C.Structure):
    """``supersonic_decode_batch`` (include/supersonic_attn.h)."""
    _fields_ = [("batch", C.c_size_t), ("max_kv_len", C.c_size_t), ("q_proj", C.c_void_p),
                ("k_new", C.c_void_p), ("v_new", C.c_void_p), ("positions", C.c_void_p),
                ("cache", C.POINTER(KvCacheDesc)), ("out", C.c_void_p)]


SIGNATURES = {
    "supersonic_qwen35_hip_full_attention_prefill":
        [_i, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _f, _sz, _p, _p, _p, _p],
    "supersonic_qwen35_4b_hip_full_attention_prefill":
        [_i, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _f, _sz, _p, _p, _p, _p],
    "supersonic_qwen35_hip_full_attention_decode_flat":
        [_i, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _f, _p, _p, _p, _p],
    "supersonic_qwen35_hip_full_attention_decode_flat_strided":
        [_i, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _f, _p, _p, _p, _p],
    "supersonic_qwen35_4b_hip_quantize_kv_to_fp8":
        [_i, _sz, _p, _p, _p, _i, _i, _i, _i, _i],
    "supersonic_qwen35_hip_rms_norm": [_i, _sz, _sz, _sz, _f, _i, _p, _p, _p],
    "supersonic_qwen35_hip_cast": [_i, _i, _sz, _sz, _p, _p],
    "supersonic_qwen35_hip_apply_rope_prefill": [_i, _sz, _sz, _sz, _sz, _sz, _p, _p, _p],
    "supersonic_qwen35_hip_transpose_shd_hsd": [_i, _sz, _sz, _sz, _sz, _p, _p],
    "supersonic_qwen35_hip_sigmoid_mul": [_i, _sz, _sz, _p, _p, _p],
    "supersonic_qwen35_hip_split_qgate": [_i, _sz, _sz, _sz, _sz, _p, _p, _p],
    "supersonic_qwen35_4b_hip_matmul_rhs_transposed_tiled": [_i, _sz, _sz, _i, _i, _i, _p, _p, _p],
    "supersonic_qwen35_hip_element_add": [_i, _sz, _sz, _p, _p, _p],
    "supersonic_attn_gfx950_decode_workspace_size": [_sz, _sz, _sz, _sz, _sz],
    "supersonic_attn_gfx950_decode":
        [_sz, _p, _i, _sz, _sz, _sz, _sz, _sz, _sz, _f, _f,
         _p, _p, _p, _p, _p, _p, _p, _p, C.POINTER(KvCacheDesc), _p, _p, _sz],
    "supersonic_attn_gfx950_decode_noalloc":
        [_sz, _p, _i, _sz, _sz, _sz, _sz, _sz, _sz, _f, _f,
         _p, _p, _p, _p, _p, _p, _p, _p, C.POINTER(KvCacheDesc), _p],
    "supersonic_attn_gfx950_decode_attend":
        [_sz, _p, _i, _sz, _sz, _sz, _sz, _sz, _f, _p, _p, C.POINTER(KvCacheDesc), _p, _p, _p, _sz],
    "supersonic_attn_gfx950_prefill_workspace_size": [_i, _sz, _sz, _sz, _sz],
    "supersonic_attn_gfx950_prefill":
        [_sz, _p, _i, _sz, _sz, _sz, _sz, _sz, _sz, _f, _f,
         _p, _p, _p, _p, _p, _p, _p, C.POINTER(KvCacheDesc), _p, _p, _sz],
    "supersonic_attn_gfx950_mixed_workspace_size":
        [_i, _sz, _sz, _sz, C.POINTER(PrefillChunkDesc), C.POINTER(DecodeBatchDesc)],
    "supersonic_attn_gfx950_mixed":
        [_sz, _p, _i, _sz, _sz, _sz, _sz, _f, _f, _p, _p, _p, _p, C.POINTER(PrefillChunkDesc),
         C.POINTER(DecodeBatchDesc), _p, _sz],
    "supersonic_attn_gfx950_o_proj_workspace_size": [_sz, _sz, _sz],
    "supersonic_attn_gfx950_o_proj_residual": [_sz, _p, _i, _sz, _sz, _sz, _p, _p, _p, _p, _sz],
    "supersonic_attn_gfx950_qkv_proj_workspace_size": [_sz, _sz, _sz, _sz],
    "supersonic_attn_gfx950_qkv_proj":
        [_sz, _p, _i, _sz, _sz, _sz, _sz, _f, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz],
    "supersonic_attn_gfx950_qkv_proj_rope_workspace_size": [_sz, _sz, _sz, _sz, _sz],
    "supersonic_attn_gfx950_qkv_proj_rope":
        [_sz, _p, _i, _sz, _sz, _sz, _sz, _sz, _sz, _f, _f, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
         _p, _p, _p, _p, C.POINTER(KvCacheDesc), _p, _sz],
    "supersonic_attn_gfx950_decode_layer_workspace_size": [_sz, _sz, _sz, _sz, _sz, _sz],
    "supersonic_attn_gfx950_decode_layer":
        [_sz, _p, _i, _i, _sz, _sz, _sz, _sz, _sz, _sz, _sz, _f, _f, _f, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
         _p, C.POINTER(KvCacheDesc), _p, _sz],
    "supersonic_attn_gfx950_quantize_kv_fp8_ocp": [_sz, _p, _p, _p, _p, _i, _i, _i, _i, _i],
    "supersonic_attn_gfx950_set_profile_events": [_p, _p],
    "supersonic_attn_gfx950_wait_status": [_sz, _p, C.POINTER(C.c_uint32)],
    "supersonic_attn_rope_tables": [_sz, _sz, C.c_double, _p, _p],
    "supersonic_attn_version": [],
}
RESTYPES = {"supersonic_attn_gfx950_decode_workspace_size": _sz, "supersonic_attn_gfx950_mixed_workspace_size": _sz, "supersonic_attn_gfx950_prefill_workspace_size": _sz,
            "supersonic_attn_gfx950_o_proj_workspace_size": _sz, "supersonic_attn_gfx950_qkv_proj_workspace_size": _sz,
            "supersonic_attn_gfx950_qkv_proj_rope_workspace_size": _sz,
            "supersonic_attn_gfx950_decode_layer_workspace_size": _sz, "supersonic_attn_version": C.c_char_p,
            "supersonic_attn_gfx950_set_profile_events": None}

_LIB = None


def load(path: str = LIB_PATH):
    """Load the HIP library (once).  Raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m supersonic_amd.build` "
            "(the attention path has no CPU fallback)")
    lib = C.CDLL(path)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = RESTYPES.get(name, C.c_int)
    _LIB = lib
    return lib


def header_functions(path: str = HEADER) -> list:
    """Names of every function the public header declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(supersonic_\w+)\s*\(", text, flags=re.M)))


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    return t.data_ptr()


def _check(op: str, status: int):
    if status != 0:
        raise GpuError(op, status)


def _stream_ptr(stream) -> Optional[int]:
    if stream is None:
        return None
    return int(stream.cuda_stream) if hasattr(stream, "cuda_stream") else int(stream)


# --------------------------------------------------------------------------
# Drop-in wrappers (prefill_ffi.rs names)
# --------------------------------------------------------------------------
def full_attention_prefill(ordinal, dtype, batch_size, q_heads, kv_heads, q_len, kv_len, head_dim, scale,
                           seqlen_offset, query, key, value, out):
    """prefill_ffi.rs:1206-1292 (the HIP branch)."""
    num_kv_groups = q_heads // kv_heads
    st = load().supersonic_qwen35_hip_full_attention_prefill(
        dtype, ordinal, batch_size, q_heads, kv_heads, q_len, kv_len, head_dim, num_kv_groups, scale,
        seqlen_offset, _ptr(query), _ptr(key), _ptr(value), _ptr(out))
    _check("full_attention_prefill", st)


def full_attention_decode_flat(ordinal, dtype, batch_size, q_heads, kv_heads, kv_len, head_dim, scale,
                               query, key, value, out):
    """prefill_ffi.rs:1353-1392."""
    st = load().supersonic_qwen35_hip_full_attention_decode_flat(
        dtype, ordinal, batch_size, q_heads, kv_heads, kv_len, head_dim, q_heads // kv_heads, scale,
        _ptr(query), _ptr(key), _ptr(value), _ptr(out))
    _check("full_attention_decode_flat", st)


def full_attention_decode_flat_strided(ordinal, dtype, batch_size, q_heads, kv_heads, kv_len, kv_stride,
                                       head_dim, scale, query, key, value, out):
    """prefill_ffi.rs:1396-1453 (HIP now implements it)."""
    st = load().supersonic_qwen35_hip_full_attention_decode_flat_strided(
        dtype, ordinal, batch_size, q_heads, kv_heads, kv_len, kv_stride, head_dim, q_heads // kv_heads,
        scale, _ptr(query), _ptr(key), _ptr(value), _ptr(out))
    _check("full_attention_decode_flat_strided", st)


def quantize_kv_to_fp8(ordinal, dtype, src, dst_fp8, dst_scale, num_kv_heads, seq_len, head_dim, max_t,
                       pos_offset):
    """prefill_ffi.rs:3199-3231."""
    st = load().supersonic_qwen35_4b_hip_quantize_kv_to_fp8(
        dtype, ordinal, _ptr(src), _ptr(dst_fp8), _ptr(dst_scale), num_kv_heads, seq_len, head_dim, max_t,
        pos_offset)
    _check("quantize_kv_to_fp8", st)


def rms_norm_rows(ordinal, dtype, rows, cols, eps, input, weight, output, add_unit_offset=True):
    """prefill_ffi.rs rms_norm_rows / rms_norm_rows_plain."""
    st = load().supersonic_qwen35_hip_rms_norm(dtype, ordinal, rows, cols, eps, 1 if add_unit_offset else 0,
                                               _ptr(input), _ptr(weight), _ptr(output))
    _check("rms_norm", st)


def cast(ordinal, input_dtype, output_dtype, total_elems, input, output):
    st = load().supersonic_qwen35_hip_cast(input_dtype, output_dtype, ordinal, total_elems, _ptr(input),
                                           _ptr(output))
    _check("cast", st)


def apply_rope_prefill(ordinal, dtype, seq_len, num_heads, head_dim, rotary_dim, cos_table, sin_table,
                       pos_offset, data):
    """prefill_ffi.rs:2773-2830: the table pointers are offset by pos_offset rows."""
    half_rot = rotary_dim // 2
    esz = cos_table.element_size()
    off = pos_offset * half_rot * esz
    st = load().supersonic_qwen35_hip_apply_rope_prefill(
        dtype, ordinal, seq_len, num_heads, head_dim, half_rot, cos_table.data_ptr() + off,
        sin_table.data_ptr() + off, _ptr(data))
    _check("apply_rope_prefill", st)


def transpose_shd_hsd(ordinal, dtype, s, h, d, src, dst):
    _check("transpose_shd_hsd", load().supersonic_qwen35_hip_transpose_shd_hsd(dtype, ordinal, s, h, d,
                                                                               _ptr(src), _ptr(dst)))


def sigmoid_mul(ordinal, dtype, total_elems, data, gate, out):
    _check("sigmoid_mul", load().supersonic_qwen35_hip_sigmoid_mul(dtype, ordinal, total_elems, _ptr(data),
                                                                   _ptr(gate), _ptr(out)))


def split_qgate(ordinal, dtype, s, num_heads, head_dim, src, query_out, gate_out):
    _check("split_qgate", load().supersonic_qwen35_hip_split_qgate(dtype, ordinal, s, num_heads, head_dim,
                                                                   _ptr(src), _ptr(query_out), _ptr(gate_out)))


def matmul_rhs_transposed(ordinal, dtype, batch_elems, m, n, k, lhs, rhs, out):
    """``out[b] = lhs[b] . rhs[b]^T`` (prefill_ffi.rs:2104-2195 binding the tiled bridge)."""
    _check("matmul_rhs_transposed", load().supersonic_qwen35_4b_hip_matmul_rhs_transposed_tiled(
        dtype, ordinal, batch_elems, m, n, k, _ptr(lhs), _ptr(rhs), _ptr(out)))


def element_add(ordinal, dtype, total_elems, lhs, rhs, out):
    _check("element_add", load().supersonic_qwen35_hip_element_add(dtype, ordinal, total_elems, _ptr(lhs),
                                                                   _ptr(rhs), _ptr(out)))


# --------------------------------------------------------------------------
# Native fused entry points
# --------------------------------------------------------------------------
@dataclass
class KvCache:
    """A KV cache the fused entry points read and append to.

    Contiguous mode: ``k``/``v`` are ``[B, Hkv, cap, D]`` (bf16, or uint8 e4m3
    with ``k_scale``/``v_scale`` ``[B, Hkv, cap]`` f32).  Paged mode:
    ``k``/``v`` are ``[num_pages, Hkv, page_size, D]``, scales
    ``[num_pages, Hkv, page_size]`` and ``block_table`` ``[B, max_pages]`` int32."""
    k: object
    v: object
    k_scale: object = None
    v_scale: object = None
    block_table: object = None

    def desc(self) -> KvCacheDesc:
        d = KvCacheDesc()
        d.k, d.v = self.k.data_ptr(), self.v.data_ptr()
        d.k_scale = _ptr(self.k_scale)
        d.v_scale = _ptr(self.v_scale)
        if self.block_table is None:
            B, H, cap, D = self.k.shape
            d.block_table = None
            d.seq_stride, d.head_stride, d.page_stride = H * cap * D, cap * D, 0
            d.page_size, d.max_pages_per_seq = 0, 0
            d.scale_seq_stride, d.scale_head_stride, d.scale_page_stride = H * cap, cap, 0
        else:
            P, H, ps, D = self.k.shape
            d.block_table = self.block_table.data_ptr()
            d.seq_stride, d.head_stride, d.page_stride = 0, ps * D, H * ps * D
            d.page_size, d.max_pages_per_seq = ps, self.block_table.shape[1]
            d.scale_seq_stride, d.scale_head_stride, d.scale_page_stride = 0, ps, H * ps
        return d

    @property
    def fp8(self) -> bool:
        return self.k_scale is not None


def decode_workspace_size(batch, q_heads, kv_heads, head_dim, max_kv_len) -> int:
    return int(load().supersonic_attn_gfx950_decode_workspace_size(batch, q_heads, kv_heads, head_dim,
                                                                   max_kv_len))


def fused_decode(ordinal, q_proj, k_new, v_new, q_norm_w, k_norm_w, cos_table, sin_table, positions,
                 cache: KvCache, out, *, q_heads, kv_heads, head_dim, rotary_dim, max_kv_len, eps=1e-6,
                 scale=None, workspace=None, stream=None):
    """``supersonic_attn_gfx950_decode``: one decode step for every sequence."""
    B = q_proj.shape[0]
    scale = head_dim ** -0.5 if scale is None else scale
    desc = cache.desc()
    st = load().supersonic_attn_gfx950_decode(
        ordinal, _stream_ptr(stream), KV_FP8_E4M3 if cache.fp8 else KV_BF16, B, q_heads, kv_heads, head_dim,
        rotary_dim, max_kv_len, eps, scale, _ptr(q_proj), _ptr(k_new), _ptr(v_new), _ptr(q_norm_w),
        _ptr(k_norm_w), _ptr(cos_table), _ptr(sin_table), _ptr(positions), C.byref(desc), _ptr(out),
        _ptr(workspace), 0 if workspace is None else workspace.numel() * workspace.element_size())
    _check("fused_decode", st)


def fused_decode_noalloc(ordinal, q_proj, k_new, v_new, q_norm_w, k_norm_w, cos_table, sin_table, positions,
                         cache: KvCache, out, *, q_heads, kv_heads, head_dim, rotary_dim, max_kv_len, eps=1e-6,
                         scale=None, stream=None):
    """``supersonic_attn_gfx950_decode_noalloc``: one decode step, no workspace, no allocation."""
    B = q_proj.shape[0]
    scale = head_dim ** -0.5 if scale is None else scale
    desc = cache.desc()
    st = load().supersonic_attn_gfx950_decode_noalloc(
        ordinal, _stream_ptr(stream), KV_FP8_E4M3 if cache.fp8 else KV_BF16, B, q_heads, kv_heads, head_dim,
        rotary_dim, max_kv_len, eps, scale, _ptr(q_proj), _ptr(k_new), _ptr(v_new), _ptr(q_norm_w),
        _ptr(k_norm_w), _ptr(cos_table), _ptr(sin_table), _ptr(positions), C.byref(desc), _ptr(out))
    _check("fused_decode_noalloc", st)


def decode_attend(ordinal, q, kv_lens, cache: KvCache, out, *, q_heads, kv_heads, head_dim, max_kv_len,
                  scale=None, gate=None, workspace=None, stream=None):
    """``supersonic_attn_gfx950_decode_attend``: attention over an existing cache."""
    B = q.shape[0]
    scale = head_dim ** -0.5 if scale is None else scale
    desc = cache.desc()
    st = load().supersonic_attn_gfx950_decode_attend(
        ordinal, _stream_ptr(stream), KV_FP8_E4M3 if cache.fp8 else KV_BF16, B, q_heads, kv_heads, head_dim,
        max_kv_len, scale, _ptr(q), _ptr(kv_lens), C.byref(desc), _ptr(gate), _ptr(out), _ptr(workspace),
        0 if workspace is None else workspace.numel() * workspace.element_size())
    _check("decode_attend", st)


def _ws(workspace):
    return _ptr(workspace), 0 if workspace is None else workspace.numel() * workspace.element_size()


def prefill_workspace_size(fp8, kv_heads, head_dim, chunk_len, chunk_start) -> int:
    return int(load().supersonic_attn_gfx950_prefill_workspace_size(KV_FP8_E4M3 if fp8 else KV_BF16, kv_heads,
                                                                     head_dim, chunk_len, chunk_start))


def o_proj_workspace_size(rows, hidden_dim, attn_dim) -> int:
    return int(load().supersonic_attn_gfx950_o_proj_workspace_size(rows, hidden_dim, attn_dim))


def qkv_proj_workspace_size(rows, hidden_dim, q_out_dim, kv_out_dim) -> int:
    return int(load().supersonic_attn_gfx950_qkv_proj_workspace_size(rows, hidden_dim, q_out_dim, kv_out_dim))


def fused_prefill(ordinal, q_proj, k_new, v_new, q_norm_w, k_norm_w, cos_table, sin_table, cache: KvCache,
                  out, *, q_heads, kv_heads, head_dim, rotary_dim, chunk_start=0, eps=1e-6, scale=None,
                  stream=None, workspace=None):
    """``supersonic_attn_gfx950_prefill``: one prefill chunk of sequence 0 of ``cache``."""
    S = q_proj.shape[0]
    scale = head_dim ** -0.5 if scale is None else scale
    desc = cache.desc()
    st = load().supersonic_attn_gfx950_prefill(
        ordinal, _stream_ptr(stream), KV_FP8_E4M3 if cache.fp8 else KV_BF16, q_heads, kv_heads, head_dim,
        rotary_dim, S, chunk_start, eps, scale, _ptr(q_proj), _ptr(k_new), _ptr(v_new), _ptr(q_norm_w),
        _ptr(k_norm_w), _ptr(cos_table), _ptr(sin_table), C.byref(desc), _ptr(out), *_ws(workspace))
    _check("fused_prefill", st)


def _mixed_descs(chunk, decode):
    """ctypes descriptors (and the cache descriptors they point at) of a mixed step."""
    keep = []
    cd = dd = None
    if chunk is not None:
        cdesc = chunk["cache"].desc()
        keep.append(cdesc)
        cd = PrefillChunkDesc(chunk["q_proj"].shape[0], chunk.get("chunk_start", 0), _ptr(chunk["q_proj"]),
                              _ptr(chunk["k_new"]), _ptr(chunk["v_new"]), C.pointer(cdesc), _ptr(chunk["out"]))
    if decode is not None:
        ddesc = decode["cache"].desc()
        keep.append(ddesc)
        dd = DecodeBatchDesc(decode["q_proj"].shape[0], decode["max_kv_len"], _ptr(decode["q_proj"]),
                             _ptr(decode["k_new"]), _ptr(decode["v_new"]), _ptr(decode["positions"]),
                             C.pointer(ddesc), _ptr(decode["out"]))
    return cd, dd, keep


def mixed_workspace_size(fp8, q_heads, kv_heads, head_dim, chunk=None, decode=None) -> int:
    cd, dd, _keep = _mixed_descs(chunk, decode)
    return int(load().supersonic_attn_gfx950_mixed_workspace_size(
        KV_FP8_E4M3 if fp8 else KV_BF16, q_heads, kv_heads, head_dim, C.byref(cd) if cd else None,
        C.byref(dd) if dd else None))


def fused_mixed(ordinal, q_norm_w, k_norm_w, cos_table, sin_table, *, chunk=None, decode=None, q_heads, kv_heads,
                head_dim, rotary_dim, eps=1e-6, scale=None, stream=None, workspace=None):
    """``supersonic_attn_gfx950_mixed``: a prefill chunk and a decode batch of one layer at the same time.

    ``chunk``: dict(q_proj, k_new, v_new, cache, out, chunk_start); ``decode``: dict(q_proj, k_new, v_new,
    positions, cache, out, max_kv_len).  The results are those of ``fused_prefill`` and ``fused_decode``."""
    scale = head_dim ** -0.5 if scale is None else scale
    cd, dd, _keep = _mixed_descs(chunk, decode)
    fp8 = (chunk or decode)["cache"].fp8
    st = load().supersonic_attn_gfx950_mixed(
        ordinal, _stream_ptr(stream), KV_FP8_E4M3 if fp8 else KV_BF16, q_heads, kv_heads, head_dim, rotary_dim, eps,
        scale, _ptr(q_norm_w), _ptr(k_norm_w), _ptr(cos_table), _ptr(sin_table), C.byref(cd) if cd else None,
        C.byref(dd) if dd else None, *_ws(workspace))
    _check("fused_mixed", st)


def o_proj_residual(ordinal, attn, o_proj_w, hidden, stream=None, workspace=None):
    """``hidden = bf16(hidden + bf16(attn . o_proj_w^T))`` in place; hidden bf16 or f32."""
    import torch
    rows, attn_dim = attn.shape
    hidden_dim = o_proj_w.shape[0]
    assert o_proj_w.shape[1] == attn_dim and tuple(hidden.shape) == (rows, hidden_dim)
    assert attn.dtype == torch.bfloat16 and o_proj_w.dtype == torch.bfloat16
    assert attn.is_contiguous() and o_proj_w.is_contiguous() and hidden.is_contiguous()
    hd = {torch.bfloat16: ScalarType.BF16, torch.float32: ScalarType.F32}[hidden.dtype]
    _check("o_proj_residual", load().supersonic_attn_gfx950_o_proj_residual(
        ordinal, _stream_ptr(stream), hd, rows, hidden_dim, attn_dim, _ptr(attn), _ptr(o_proj_w), _ptr(hidden),
        *_ws(workspace)))


def qkv_proj(ordinal, hidden, input_norm_w, q_proj_w, k_proj_w, v_proj_w, q_proj_out, k_out, v_out, eps=1e-6,
             stream=None, workspace=None):
    """Input RMSNorm (1 + w) + Q/K/V projections: the fused decode's q_proj / k_new / v_new."""
    import torch
    rows, hid = hidden.shape
    nq, nkv = q_proj_w.shape[0], k_proj_w.shape[0]
    assert input_norm_w.shape == (hid,) and q_proj_w.shape[1] == hid and k_proj_w.shape == (nkv, hid)
    assert v_proj_w.shape == (nkv, hid) and tuple(q_proj_out.shape) == (rows, nq)
    assert tuple(k_out.shape) == (rows, nkv) and tuple(v_out.shape) == (rows, nkv)
    for t in (input_norm_w, q_proj_w, k_proj_w, v_proj_w, q_proj_out, k_out, v_out):
        assert t.dtype == torch.bfloat16 and t.is_contiguous()
    assert hidden.is_contiguous()
    hd = {torch.bfloat16: ScalarType.BF16, torch.float32: ScalarType.F32}[hidden.dtype]
    _check("qkv_proj", load().supersonic_attn_gfx950_qkv_proj(
        ordinal, _stream_ptr(stream), hd, rows, hid, nq, nkv, eps, _ptr(hidden), _ptr(input_norm_w),
        _ptr(q_proj_w), _ptr(k_proj_w), _ptr(v_proj_w), _ptr(q_proj_out), _ptr(k_out), _ptr(v_out),
        *_ws(workspace)))


def qkv_proj_rope(ordinal, hidden, input_norm_w, q_proj_w, k_proj_w, v_proj_w, q_norm_w, k_norm_w, cos_table,
                  sin_table, positions, q_out, gate_out, k_out, v_out, *, q_heads, kv_heads, head_dim, rotary_dim,
                  eps=1e-6, qk_eps=1e-6, cache: Optional["KvCache"] = None, workspace=None, stream=None):
    """``supersonic_attn_gfx950_qkv_proj_rope``: input norm + projections + QK norm + RoPE (+ cache append)."""
    import torch
    rows, hid = hidden.shape
    hd = {torch.bfloat16: ScalarType.BF16, torch.float32: ScalarType.F32}[hidden.dtype]
    desc = cache.desc() if cache is not None else None
    _check("qkv_proj_rope", load().supersonic_attn_gfx950_qkv_proj_rope(
        ordinal, _stream_ptr(stream), hd, rows, hid, q_heads, kv_heads, head_dim, rotary_dim, eps, qk_eps,
        _ptr(hidden), _ptr(input_norm_w), _ptr(q_proj_w), _ptr(k_proj_w), _ptr(v_proj_w), _ptr(q_norm_w),
        _ptr(k_norm_w), _ptr(cos_table), _ptr(sin_table), _ptr(positions), _ptr(q_out), _ptr(gate_out),
        _ptr(k_out), _ptr(v_out), None if desc is None else C.byref(desc), *_ws(workspace)))


def qkv_proj_rope_workspace_size(rows, hidden_dim, q_heads, kv_heads, head_dim) -> int:
    return int(load().supersonic_attn_gfx950_qkv_proj_rope_workspace_size(rows, hidden_dim, q_heads, kv_heads,
                                                                         head_dim))


def decode_layer_workspace_size(batch, hidden_dim, q_heads, kv_heads, head_dim, max_kv_len) -> int:
    return int(load().supersonic_attn_gfx950_decode_layer_workspace_size(batch, hidden_dim, q_heads, kv_heads,
                                                                        head_dim, max_kv_len))


def decode_layer(ordinal, hidden, input_norm_w, q_proj_w, k_proj_w, v_proj_w, q_norm_w, k_norm_w, o_proj_w,
                 cos_table, sin_table, positions, cache: "KvCache", workspace, *, q_heads, kv_heads, head_dim,
                 rotary_dim, max_kv_len, eps=1e-6, qk_eps=1e-6, scale=None, stream=None):
    """``supersonic_attn_gfx950_decode_layer``: the persistent one-kernel decode layer (hidden updated in place)."""
    import torch
    B, hid = hidden.shape
    scale = head_dim ** -0.5 if scale is None else scale
    hd = {torch.bfloat16: ScalarType.BF16, torch.float32: ScalarType.F32}[hidden.dtype]
    desc = cache.desc()
    _check("decode_layer", load().supersonic_attn_gfx950_decode_layer(
        ordinal, _stream_ptr(stream), hd, KV_FP8_E4M3 if cache.fp8 else KV_BF16, B, hid, q_heads, kv_heads,
        head_dim, rotary_dim, max_kv_len, eps, qk_eps, scale, _ptr(hidden), _ptr(input_norm_w), _ptr(q_proj_w),
        _ptr(k_proj_w), _ptr(v_proj_w), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(o_proj_w), _ptr(cos_table),
        _ptr(sin_table), _ptr(positions), C.byref(desc), *_ws(workspace)))


def quantize_kv_fp8_ocp(ordinal, src, dst_fp8, dst_scale, num_kv_heads, seq_len, head_dim, max_t, pos_offset,
                        stream=None):
    st = load().supersonic_attn_gfx950_quantize_kv_fp8_ocp(
        ordinal, _stream_ptr(stream), _ptr(src), _ptr(dst_fp8), _ptr(dst_scale), num_kv_heads, seq_len,
        head_dim, max_t, pos_offset)
    _check("quantize_kv_fp8_ocp", st)


def set_profile_events(before, after):
    """Arm the benchmark hook with two torch.cuda.Event (enable_timing=True)."""
    load().supersonic_attn_gfx950_set_profile_events(None if before is None else before.cuda_event,
                                                     None if after is None else after.cuda_event)


def wait_status(ordinal=0, stream=None) -> int:
    """``supersonic_attn_gfx950_wait_status``: synchronise ``stream``, return and
    clear the SUPERSONIC_WAIT_* bits of bounded waits that gave up since the last call."""
    bits = C.c_uint32(0)
    _check("wait_status", load().supersonic_attn_gfx950_wait_status(ordinal, _stream_ptr(stream), C.byref(bits)))
    return int(bits.value)


def rope_tables(rotary_dim, max_pos, theta):
    """``supersonic_attn_rope_tables``: host (CPU) bf16 tensors ``(cos, sin)`` of
    shape ``[max_pos, rotary_dim // 2]``, built by the library."""
    import torch
    half = rotary_dim // 2
    cos = torch.empty(max_pos, half, dtype=torch.bfloat16)
    sin = torch.empty(max_pos, half, dtype=torch.bfloat16)
    _check("rope_tables", load().supersonic_attn_rope_tables(rotary_dim, max_pos, float(theta), _ptr(cos),
                                                             _ptr(sin)))
    return cos, sin


def version() -> str:
    return load().supersonic_attn_version().decode()
