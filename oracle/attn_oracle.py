"""torch fp32 restatement of the full-attention hot path.  TEST INFRASTRUCTURE ONLY.

Every function names the reference code it restates.  bf16 rounding happens
exactly where the reference stores a bf16 tensor (or calls
``bf16_round_rne_f32``); everything between two such points is fp32.

Shapes use the reference's names: B batch, Hq / Hkv query / kv heads,
D head_dim, S prefill tokens, L kv length, G = Hq / Hkv.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import fp8_codec

F32 = torch.float32
BF16 = torch.bfloat16


def bf16r(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (RNE) and widen back to fp32 (``bf16_round_rne_f32``,
    full_attention_4b.hip:139-153)."""
    return x.to(BF16).to(F32)


# ---------------------------------------------------------------------------
# a3: RoPE tables and rotation
# ---------------------------------------------------------------------------
def rope_tables(rotary_dim: int, max_pos: int, theta: float):
    """``RotaryTables::build`` (crates/qwen35/src/rotary.rs:15-46): angles in
    float64, ``inv_freq_i = theta^(-2i/rotary_dim)``, each entry rounded to bf16.
    Returns ``(cos, sin)`` bf16 ``[max_pos, rotary_dim/2]``."""
    half = rotary_dim // 2
    i = torch.arange(half, dtype=torch.float64)
    freq = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64), 2.0 * i / rotary_dim)
    pos = torch.arange(max_pos, dtype=torch.float64)
    ang = pos[:, None] * freq[None, :]
    return torch.cos(ang).to(BF16), torch.sin(ang).to(BF16)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rotary_dim: int,
               positions: torch.Tensor) -> torch.Tensor:
    """Rotate-half partial RoPE, ``pfx_apply_rope_prefill_kernel``
    (kernels/prefill_helpers.hip:79-108) and the megakernel decode step
    (full_attention_4b.hip:5193-5224).

    ``x``: ``[..., S, H, D]`` fp32 holding bf16 values; ``positions``: ``[S]``
    int64 (or broadcastable to the S axis).  Pairs ``(i, i + rotary_dim/2)`` for
    ``i < rotary_dim/2``; dims ``>= rotary_dim`` are untouched.  Output is
    bf16-rounded (the kernels store T / call bf16_round)."""
    half = rotary_dim // 2
    if half == 0:
        return x.clone()
    c = cos.to(F32)[positions][:, None, :]  # [S, 1, half]
    s = sin.to(F32)[positions][:, None, :]
    x0 = x[..., :half]
    x1 = x[..., half:rotary_dim]
    out = x.clone()
    out[..., :half] = x0 * c - x1 * s
    out[..., half:rotary_dim] = x0 * s + x1 * c
    return bf16r(out)


# ---------------------------------------------------------------------------
# a1, a2, a9: split, RMSNorm, gate
# ---------------------------------------------------------------------------
def split_qgate(q_proj: torch.Tensor, num_heads: int, head_dim: int):
    """``pfx_split_qgate_kernel`` (prefill_helpers.hip:239-257): per head the
    q_proj row holds ``[q_h (D) | gate_h (D)]`` (HF ``view(H, 2D).chunk(2)``,
    oracle/qwen36_moe_oracle.py:349-365).  ``[S, H*2D] -> ([S,H,D], [S,H,D])``."""
    S = q_proj.shape[0]
    v = q_proj.reshape(S, num_heads, 2 * head_dim)
    return v[..., :head_dim].clone(), v[..., head_dim:].clone()


def rms_norm_rows(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-6,
                  add_unit_offset: bool = True) -> torch.Tensor:
    """``supersonic_qwen35_rms_norm_kernel`` (full_attention.hip:2507-2560) and the
    megakernel QK-norm (full_attention_4b.hip:5142-5191):
    ``x * rsqrt(mean(x^2) + eps) * (w + 1)``, fp32 math, bf16 output."""
    xf = x.to(F32)
    inv = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    wf = w.to(F32) + (1.0 if add_unit_offset else 0.0)
    return bf16r(xf * inv * wf)


def sigmoid_mul(data: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """``pfx_sigmoid_mul_kernel`` (prefill_helpers.hip:183-195) and the decode gate
    (full_attention_4b.hip:5464-5470): ``bf16(data * sigmoid(gate))``."""
    return bf16r(data.to(F32) * torch.sigmoid(gate.to(F32)))


# ---------------------------------------------------------------------------
# a7, a8: attention cores
# ---------------------------------------------------------------------------
def attention_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                      seqlen_offset: int) -> torch.Tensor:
    """Causal GQA prefill, ``supersonic_qwen35_full_attention_prefill_kernel``
    (full_attention.hip:246-361).  ``q [B,Hq,S,D]``, ``k,v [B,Hkv,L,D]``; query row
    ``p`` attends keys ``t < min(L, seqlen_offset + p + 1)``; a row with no keys
    is 0.  Head map ``h_kv = h // (Hq/Hkv)``.  Returns fp32 ``[B,Hq,S,D]``."""
    B, Hq, S, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = torch.zeros(B, Hq, S, D, dtype=F32)
    pos = torch.arange(S)
    limit = torch.clamp(seqlen_offset + pos + 1, max=L)  # [S]
    mask = torch.arange(L)[None, :] < limit[:, None]     # [S, L]
    has_key = limit > 0
    # rows are independent: blocks of query rows bound the [G, rows, L] score memory
    rb = max(1, min(S, (1 << 27) // max(1, G * L)))
    for b in range(B):
        for hk in range(Hkv):
            kf = k[b, hk].to(F32)
            vf = v[b, hk].to(F32)
            for r0 in range(0, S, rb):
                r1 = min(S, r0 + rb)
                qf = q[b, hk * G:(hk + 1) * G, r0:r1].to(F32)         # [G,rows,D]
                s = torch.matmul(qf, kf.T) * scale                    # [G,rows,L]
                s = s.masked_fill(~mask[r0:r1], float("-inf"))
                hk_rows = has_key[r0:r1][None, :, None]
                s = torch.where(hk_rows, s, torch.zeros_like(s))
                p = torch.softmax(s, dim=-1)
                p = torch.where(hk_rows, p, torch.zeros_like(p))
                out[b, hk * G:(hk + 1) * G, r0:r1] = torch.matmul(p, vf)
    return out


def attention_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_len, scale: float
                     ) -> torch.Tensor:
    """Single-query GQA attention, ``pfx_full_attention_decode_flat_kernel``
    (prefill_helpers.hip:319-404) and the megakernel core
    (full_attention_4b.hip:5401-5454).  ``q [B,Hq,D]``; ``k,v [B,Hkv,T,D]`` (T may
    exceed the live length); ``kv_len`` int or per-sequence list.  Keys
    ``t < kv_len[b]``; zero keys give 0.  Returns fp32 ``[B,Hq,D]``."""
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    lens = [int(kv_len)] * B if isinstance(kv_len, (int, np.integer)) else [int(x) for x in kv_len]
    out = torch.zeros(B, Hq, D, dtype=F32)
    for b in range(B):
        n = lens[b]
        if n <= 0:
            continue
        for hk in range(Hkv):
            kf = k[b, hk, :n].to(F32)
            vf = v[b, hk, :n].to(F32)
            qf = q[b, hk * G:(hk + 1) * G].to(F32)
            p = torch.softmax((qf @ kf.T) * scale, dim=-1)
            out[b, hk * G:(hk + 1) * G] = p @ vf
    return out


# ---------------------------------------------------------------------------
# a5, a6: FP8 KV quantisation
# ---------------------------------------------------------------------------
def quantize_kv_to_fp8(src: torch.Tensor, codec: str = "ref"):
    """``quantize_kv_to_fp8_kernel`` (full_attention_4b.hip:4786-4829) over
    ``src [Hkv, S, D]`` (bf16): per (head, position) ``scale = max(absmax/448,
    1e-12)``, ``code = e4m3(x * (1/scale))``.  Returns ``(codes uint8 [Hkv,S,D],
    scale f32 [Hkv,S])`` as torch tensors."""
    codes, scale = fp8_codec.quantize_rows(src.to(F32).numpy(), codec)
    return torch.from_numpy(codes), torch.from_numpy(scale)


def dequantize_kv(codes: torch.Tensor, scale: torch.Tensor, codec: str) -> torch.Tensor:
    """FP8 K/V as the megakernel reads them: ``bf16(lut[code] * scale)``
    (full_attention_4b.hip:5354-5356, :5382-5384)."""
    lut = torch.from_numpy(np.nan_to_num(
        fp8_codec.ocp_decode_table() if codec == "ocp" else fp8_codec.ref_decode_table(), nan=0.0))
    return bf16r(lut[codes.long()] * scale[..., None].to(F32))


# ---------------------------------------------------------------------------
# Fused layer cores (what the fused entry points compute)
# ---------------------------------------------------------------------------
@dataclass
class LayerShape:
    q_heads: int
    kv_heads: int
    head_dim: int
    rotary_dim: int
    eps: float = 1e-6

    @property
    def groups(self) -> int:
        return self.q_heads // self.kv_heads

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)


def prep_qk(shape: LayerShape, q_proj, k_raw, q_norm_w, k_norm_w, cos, sin, positions):
    """Split -> per-head RMSNorm -> partial RoPE for ``q_proj [S, Hq*2D]`` and
    ``k_raw [S, Hkv*D]`` at ``positions [S]``.  The prefill chain's steps 2, 4-6
    (crates/runner/src/prefill_engine.rs:1978-2096) and the megakernel's
    steps B-C (full_attention_4b.hip:5142-5224).  Returns fp32 tensors of bf16
    values ``q [S,Hq,D]``, ``gate [S,Hq,D]``, ``k [S,Hkv,D]``."""
    S = q_proj.shape[0]
    D = shape.head_dim
    q, gate = split_qgate(q_proj.to(F32), shape.q_heads, D)
    k = k_raw.to(F32).reshape(S, shape.kv_heads, D)
    q = rms_norm_rows(q, q_norm_w, shape.eps)
    k = rms_norm_rows(k, k_norm_w, shape.eps)
    q = apply_rope(q, cos, sin, shape.rotary_dim, positions)
    k = apply_rope(k, cos, sin, shape.rotary_dim, positions)
    return q, gate, k


def prefill_layer(shape: LayerShape, q_proj, k_raw, v_raw, q_norm_w, k_norm_w, cos, sin,
                  chunk_start: int = 0, k_prev=None, v_prev=None):
    """Full-attention core of one prefill chunk, ``prefill_full_attention_layer``
    (prefill_engine.rs:1912-2310) without the projections: split, QK norm, RoPE at
    ``chunk_start + s``, causal attention over ``[k_prev | k_chunk]``, cast to
    bf16, sigmoid gate.  ``q_proj [S, Hq*2D]``, ``k_raw, v_raw [S, Hkv*D]``,
    ``k_prev, v_prev [Hkv, chunk_start, D]`` (the cached prefix).

    Returns ``(out [S, Hq*D] bf16-valued fp32, k_chunk [Hkv,S,D], v_chunk [Hkv,S,D])``."""
    S = q_proj.shape[0]
    D, Hq, Hkv = shape.head_dim, shape.q_heads, shape.kv_heads
    pos = torch.arange(chunk_start, chunk_start + S)
    q, gate, k = prep_qk(shape, q_proj, k_raw, q_norm_w, k_norm_w, cos, sin, pos)
    v = bf16r(v_raw.to(F32)).reshape(S, Hkv, D)
    k_chunk = k.permute(1, 0, 2).contiguous()
    v_chunk = v.permute(1, 0, 2).contiguous()
    if chunk_start > 0:
        k_all = torch.cat([k_prev.to(F32), k_chunk], dim=1)
        v_all = torch.cat([v_prev.to(F32), v_chunk], dim=1)
    else:
        k_all, v_all = k_chunk, v_chunk
    attn = attention_prefill(q.permute(1, 0, 2)[None], k_all[None], v_all[None], shape.scale,
                             chunk_start)[0]                      # [Hq,S,D] fp32
    attn = bf16r(attn).permute(1, 0, 2)                            # cast + transpose back
    out = sigmoid_mul(attn, gate).reshape(S, Hq * D)
    return out, k_chunk, v_chunk


def decode_layer(shape: LayerShape, q_proj, k_raw, v_raw, q_norm_w, k_norm_w, cos, sin,
                 positions, k_cache, v_cache, k_scale=None, v_scale=None, codec: str = "ocp"):
    """One decode step of the full-attention core, the megakernel's steps B-F
    (full_attention_4b.hip:5109-5470), for ``B`` sequences.

    ``q_proj [B, Hq*2D]``, ``k_raw, v_raw [B, Hkv*D]``; ``positions [B]`` is the
    slot of the new token (= cached length before the step).  ``k_cache,
    v_cache``: list of per-sequence ``[Hkv, cap, D]`` tensors, bf16 (``k_scale`` is
    None) or uint8 e4m3 codes with ``k_scale, v_scale`` lists of ``[Hkv, cap]`` f32.
    The caches are updated in place at ``positions[b]``: bf16 values, or codes and
    scales from the per-(token, head) absmax quantiser (:5228-5281).

    Attention covers ``t <= positions[b]``; cached FP8 rows are read as
    ``bf16(lut[code] * scale)``, the new token unquantised (:5351-5353).
    Returns ``out [B, Hq*D]`` (bf16-valued fp32): ``bf16(bf16(attn) * sigmoid(gate))``."""
    B = q_proj.shape[0]
    D, Hq, Hkv, G = shape.head_dim, shape.q_heads, shape.kv_heads, shape.groups
    pos = torch.as_tensor(positions, dtype=torch.long)
    q, gate, k = prep_qk(shape, q_proj, k_raw, q_norm_w, k_norm_w, cos, sin, pos)
    v = bf16r(v_raw.to(F32)).reshape(B, Hkv, D)
    fp8 = k_scale is not None
    out = torch.zeros(B, Hq * D, dtype=F32)
    for b in range(B):
        p = int(pos[b])
        if fp8:
            kc, ks = quantize_kv_to_fp8(k[b][:, None, :].to(BF16), codec)
            vc, vs = quantize_kv_to_fp8(v[b][:, None, :].to(BF16), codec)
            k_cache[b][:, p] = kc[:, 0]
            v_cache[b][:, p] = vc[:, 0]
            k_scale[b][:, p] = ks[:, 0]
            v_scale[b][:, p] = vs[:, 0]
            kk = dequantize_kv(k_cache[b][:, :p + 1], k_scale[b][:, :p + 1], codec)
            vv = dequantize_kv(v_cache[b][:, :p + 1], v_scale[b][:, :p + 1], codec)
            kk[:, p] = k[b]
            vv[:, p] = v[b]
        else:
            k_cache[b][:, p] = k[b].to(k_cache[b].dtype)
            v_cache[b][:, p] = v[b].to(v_cache[b].dtype)
            kk = k_cache[b][:, :p + 1].to(F32)
            vv = v_cache[b][:, :p + 1].to(F32)
        attn = attention_decode(q[b][None], kk[None], vv[None], p + 1, shape.scale)[0]  # [Hq,D]
        out[b] = sigmoid_mul(bf16r(attn), gate[b]).reshape(Hq * D)
    return out


# ---------------------------------------------------------------------------
# Seeded synthetic inputs (same generator on CPU for oracle and GPU runs)
# ---------------------------------------------------------------------------
# ---------------------------------------------------------------------------
# f1: output projection and residual add
# ---------------------------------------------------------------------------
def matmul_rhs_transposed(lhs: torch.Tensor, rhs: torch.Tensor) -> torch.Tensor:
    """``out[b, m, n] = bf16(sum_k lhs[b, m, k] * rhs[b, n, k])``, fp32 accumulation:
    ``supersonic_qwen35_matmul_rhs_transposed_tiled_kernel`` (full_attention_4b.hip:2513-2575,
    bridge full_attention_bridge_4b.cpp:3584-3611).  That kernel gives rhs its own
    batch dimension (``rhs_base = batch * n * k``); the host fallback
    (metal_host.rs:213-245) shares one ``[n, k]`` rhs.  Both agree at batch 1."""
    return bf16r(torch.matmul(lhs.to(F32), rhs.to(F32).transpose(-1, -2)))


def element_add(lhs: torch.Tensor, rhs: torch.Tensor) -> torch.Tensor:
    """``pfx_element_add_kernel`` (prefill_helpers.hip:59-68): fp32 add, one rounding
    to the element type (here bf16)."""
    return bf16r(lhs.to(F32) + rhs.to(F32))


def o_proj_residual(attn: torch.Tensor, w: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
    """Output projection plus residual, two roundings: ``add = bf16(attn . w_j)`` then
    ``hidden = bf16(hidden + add)``.  Decode: megakernel step G
    (full_attention_4b.hip:5481-5577, bf16 weights :5551-5568, the two
    ``bf16_round_rne_f32_finite`` at :5572-5574).  Prefill: ``matmul_proj`` to a bf16
    buffer, then ``residual_add`` (prefill_engine.rs:2308-2334, 419-429)."""
    return element_add(hidden, matmul_rhs_transposed(attn, w))


def qkv_proj(hidden: torch.Tensor, norm_w: torch.Tensor, wq: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor,
             eps: float = 1e-6):
    """Input RMSNorm then the Q/K/V projections, each rounded to bf16: decode
    megakernel (full_attention_4b.hip:4942-4967 norm, :5019-5101 projections into
    ``proj_buf`` with ``bf16_round_rne_f32_finite``); prefill ``rms_norm_rows_model``
    + ``matmul_proj`` (prefill_engine.rs:1951-2117).  Returns ``(q_proj, k, v)``."""
    normed = rms_norm_rows(hidden, norm_w, eps)
    return matmul_rhs_transposed(normed, wq), matmul_rhs_transposed(normed, wk), matmul_rhs_transposed(normed, wv)


def randn_bf16(gen: torch.Generator, *shape, std: float = 1.0, mean: float = 0.0) -> torch.Tensor:
    return (torch.randn(*shape, generator=gen, dtype=F32) * std + mean).to(BF16)


def norm_weights(gen: torch.Generator, head_dim: int):
    """Q/K norm weights ~N(1, 0.02) used with the ``(1 + w)`` convention
    (effective scale ~2), as stated for the benchmark configs."""
    return randn_bf16(gen, head_dim, std=0.02, mean=1.0), randn_bf16(gen, head_dim, std=0.02, mean=1.0)
