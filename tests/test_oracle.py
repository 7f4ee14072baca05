"""Pins the CPU oracle before anything is checked against it.

Each oracle function is checked against at least one of: the reference's own
known-answer tests (restated under tests/golden/), the float64 brute force in
``oracle.brute`` (an independent implementation), closed forms and invariants,
or torch's own float8 implementation.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import attn_oracle as O
from oracle import brute

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


def t(a, *shape):
    return torch.tensor(a, dtype=torch.float32).reshape(*shape)


# ---------------------------------------------------------------- RMSNorm
def test_rmsnorm_reference_known_answer():
    g = load("rmsnorm_known_answer.json")
    out = O.rms_norm_rows(t(g["input"], 1, 2), t(g["weight"], 2), eps=g["eps"],
                          add_unit_offset=g["add_unit_offset"])
    assert np.allclose(out.numpy().ravel(), g["expected"], atol=g["tolerance"])


def test_rmsnorm_matches_brute_and_plain_variant():
    gen = torch.Generator().manual_seed(1)
    x = O.randn_bf16(gen, 5, 64).float()
    w = O.randn_bf16(gen, 64, std=0.1).float()
    out = O.rms_norm_rows(x, w, 1e-6)
    for r in range(5):
        exp = brute.bf16_round(np.array(brute.rms_norm_row(x[r].numpy(), w.numpy(), 1e-6), np.float32))
        assert np.array_equal(out[r].numpy(), exp)
    plain = O.rms_norm_rows(x, w, 1e-6, add_unit_offset=False)
    # with a zero weight the plain variant is exactly zero, the unit-offset one is x/rms
    z = O.rms_norm_rows(x, torch.zeros(64), 0.0, add_unit_offset=True)
    assert torch.allclose(z.pow(2).mean(-1), torch.ones(5), rtol=1e-2)
    assert torch.all(O.rms_norm_rows(x, torch.zeros(64), 0.0, add_unit_offset=False) == 0)
    assert not torch.equal(plain, out)


# ---------------------------------------------------------------- config / RoPE
def test_config_known_answer():
    g = load("config_known_answer.json")
    shape = O.LayerShape(q_heads=16, kv_heads=g["num_key_value_heads"], head_dim=g["head_dim"],
                         rotary_dim=int(g["head_dim"] * g["partial_rotary_factor"]))
    assert shape.rotary_dim == g["rotary_dim"]
    kv_bytes = 2 * g["num_full_attention_layers"] * shape.kv_heads * shape.head_dim * 2
    assert kv_bytes == g["kv_bytes_per_token_bf16"]


def test_rope_tables_match_brute_bitwise():
    cos, sin = O.rope_tables(64, 300, 1.0e7)
    bc, bs = brute.rope_tables(64, 300, 1.0e7)
    assert np.array_equal(cos.float().numpy(), bc)
    assert np.array_equal(sin.float().numpy(), bs)
    # i = 0 has inv_freq 1: the angle is the position itself
    assert np.array_equal(cos[:, 0].float().numpy(),
                          brute.bf16_round(np.cos(np.arange(300)).astype(np.float32)))


def test_rope_invariants():
    gen = torch.Generator().manual_seed(2)
    S, H, D, rot = 9, 3, 64, 16
    x = O.randn_bf16(gen, S, H, D).float()
    cos, sin = O.rope_tables(rot, 64, 1.0e7)
    y0 = O.apply_rope(x, cos, sin, rot, torch.zeros(S, dtype=torch.long))
    assert torch.equal(y0, x)                              # position 0 is the identity
    pos = torch.arange(20, 20 + S)
    y = O.apply_rope(x, cos, sin, rot, pos)
    assert torch.equal(y[..., rot:], x[..., rot:])         # pass-through dims untouched
    half = rot // 2
    n0 = x[..., :half] ** 2 + x[..., half:rot] ** 2
    n1 = y[..., :half] ** 2 + y[..., half:rot] ** 2
    assert torch.allclose(n0, n1, rtol=3e-2, atol=1e-2)   # rotation preserves pair norms
    for s in range(S):
        for h in range(H):
            exp = brute.bf16_round(np.array(brute.rope_row(x[s, h].numpy(), cos[pos[s]].float().numpy(),
                                                           sin[pos[s]].float().numpy(), rot), np.float32))
            assert np.array_equal(y[s, h].numpy(), exp)
    # the sign convention: x0*c - x1*s on the low half (rotate_half)
    e = torch.zeros(1, 1, D)
    e[0, 0, half] = 1.0
    r = O.apply_rope(e, cos, sin, rot, torch.tensor([5]))
    assert r[0, 0, 0] == -sin[5, 0].float() and r[0, 0, half] == cos[5, 0].float()


# ---------------------------------------------------------------- attention
@pytest.mark.parametrize("name", ["prefill_tiny.json", "prefill_clamped.json"])
def test_prefill_matches_golden(name):
    g = load(name)
    q = t(g["q"], g["B"], g["Hq"], g["S"], g["D"])
    k = t(g["k"], g["B"], g["Hkv"], g["L"], g["D"])
    v = t(g["v"], g["B"], g["Hkv"], g["L"], g["D"])
    out = O.attention_prefill(q, k, v, g["scale"], g["seqlen_offset"])
    ref = np.array(g["out"]).reshape(out.shape)
    assert np.abs(out.numpy() - ref).max() < 2e-6


def test_decode_matches_golden():
    g = load("decode_tiny.json")
    q = t(g["q"], g["B"], g["Hq"], g["D"])
    k = t(g["k"], g["B"], g["Hkv"], g["T"], g["D"])
    v = t(g["v"], g["B"], g["Hkv"], g["T"], g["D"])
    out = O.attention_decode(q, k, v, g["lens"], g["scale"])
    assert np.abs(out.numpy() - np.array(g["out"]).reshape(out.shape)).max() < 2e-6


def test_attention_invariants():
    gen = torch.Generator().manual_seed(3)
    D = 32
    v = O.randn_bf16(gen, 1, 1, 1, D).float()
    k = O.randn_bf16(gen, 1, 1, 1, D).float()
    q = O.randn_bf16(gen, 1, 2, 1, D).float()
    # a single key returns its value (reference check full_attn_phase.cuh:759-789)
    assert torch.equal(O.attention_prefill(q, k, v, 0.1, 0)[0, :, 0], v[0, 0, 0].expand(2, D))
    # identical keys -> the mean of the values
    L = 7
    kk = k.expand(1, 1, L, D).contiguous()
    vv = O.randn_bf16(gen, 1, 1, L, D).float()
    out = O.attention_decode(q[:, :, 0], kk, vv, L, 0.3)
    assert torch.allclose(out[0, 0], vv[0, 0].mean(0), atol=1e-6)
    # no visible key -> 0 (kv_len = 0 with offset 0 is an empty row)
    z = O.attention_prefill(q, k[:, :, :0], v[:, :, :0], 0.1, 0)
    assert torch.all(z == 0)
    # GQA head map h_kv = h // G: swapping kv heads swaps the head groups
    q4 = O.randn_bf16(gen, 1, 4, 3, D).float()
    k2 = O.randn_bf16(gen, 1, 2, 3, D).float()
    v2 = O.randn_bf16(gen, 1, 2, 3, D).float()
    a = O.attention_prefill(q4, k2, v2, 0.2, 0)
    b = O.attention_prefill(q4[:, [2, 3, 0, 1]], k2[:, [1, 0]], v2[:, [1, 0]], 0.2, 0)
    assert torch.allclose(a[:, [2, 3, 0, 1]], b)


def test_prefill_last_row_equals_decode():
    """Row p of a causal prefill with offset o is a decode over o+p+1 keys."""
    gen = torch.Generator().manual_seed(4)
    q = O.randn_bf16(gen, 1, 4, 6, 64).float()
    k = O.randn_bf16(gen, 1, 2, 10, 64).float()
    v = O.randn_bf16(gen, 1, 2, 10, 64).float()
    pre = O.attention_prefill(q, k, v, 0.125, 4)
    for p in range(6):
        dec = O.attention_decode(q[:, :, p], k, v, 4 + p + 1, 0.125)
        assert torch.allclose(pre[:, :, p], dec, atol=1e-6)


def test_split_lse_merge_identity():
    """The split-K decomposition the GPU decode uses: per split (m, l, o) then a
    log-sum-exp merge equals the unsplit softmax."""
    gen = torch.Generator().manual_seed(5)
    L, D = 333, 64
    q = O.randn_bf16(gen, D).float()
    k = O.randn_bf16(gen, L, D).float()
    v = O.randn_bf16(gen, L, D).float()
    s = (k @ q) * 0.125
    full = torch.softmax(s, 0) @ v
    parts = []
    for lo in range(0, L, 50):
        ss = s[lo:lo + 50]
        m = ss.max()
        p = torch.exp(ss - m)
        parts.append((m, p.sum(), p @ v[lo:lo + 50]))
    M = max(m for m, _, _ in parts)
    num = sum(torch.exp(m - M) * o for m, _, o in parts)
    den = sum(torch.exp(m - M) * l for m, l, _ in parts)
    assert torch.allclose(num / den, full, atol=1e-6)


# ---------------------------------------------------------------- fused layers
def test_fused_decode_step_matches_golden():
    g = load("fused_decode_tiny.json")
    D, Hq, Hkv, pos = g["D"], g["Hq"], g["Hkv"], g["pos"]
    shape = O.LayerShape(Hq, Hkv, D, g["rotary_dim"], g["eps"])
    cos, sin = O.rope_tables(g["rotary_dim"], pos + 1, g["theta"])
    cap = pos + 3
    kc = torch.zeros(Hkv, cap, D, dtype=torch.bfloat16)
    vc = torch.zeros(Hkv, cap, D, dtype=torch.bfloat16)
    kc[:, :pos] = t(g["cache_k"], Hkv, pos, D).bfloat16()
    vc[:, :pos] = t(g["cache_v"], Hkv, pos, D).bfloat16()
    out = O.decode_layer(shape, t(g["q_proj"], 1, Hq * 2 * D), t(g["k_raw"], 1, Hkv * D),
                         t(g["v_raw"], 1, Hkv * D), t(g["q_norm_w"], D), t(g["k_norm_w"], D),
                         cos, sin, [pos], [kc], [vc])
    assert torch.equal(kc[:, pos].float().reshape(-1), t(g["k_rot_expected"], Hkv * D))
    assert torch.equal(vc[:, pos].float().reshape(-1), t(g["v_raw"], Hkv * D))
    ref = np.array(g["out"])
    diff = np.abs(out.numpy().ravel() - ref)
    # both sides round to bf16 at the same points; the fp32-vs-fp64 attention can
    # flip a final bf16 rounding by one ulp
    assert diff.max() <= 2 ** -7 * np.abs(ref).max() and (diff > 0).mean() < 0.05


def test_prefill_chunk_then_decode_consistency():
    """A prefill chunk's last row equals the decode step at that position run on the
    prefix the chunk left in the cache (the two reference paths agree)."""
    gen = torch.Generator().manual_seed(6)
    shape = O.LayerShape(4, 2, 64, 16)
    S = 9
    qp = O.randn_bf16(gen, S, 4 * 128)
    kr = O.randn_bf16(gen, S, 2 * 64)
    vr = O.randn_bf16(gen, S, 2 * 64)
    qw, kw = O.norm_weights(gen, 64)
    cos, sin = O.rope_tables(16, 64, 1e7)
    out, kch, vch = O.prefill_layer(shape, qp, kr, vr, qw, kw, cos, sin, 0)
    kc = torch.zeros(2, 16, 64, dtype=torch.bfloat16)
    vc = torch.zeros(2, 16, 64, dtype=torch.bfloat16)
    kc[:, :S - 1] = kch[:, :S - 1].bfloat16()
    vc[:, :S - 1] = vch[:, :S - 1].bfloat16()
    dec = O.decode_layer(shape, qp[S - 1:], kr[S - 1:], vr[S - 1:], qw, kw, cos, sin, [S - 1], [kc], [vc])
    assert torch.equal(kc[:, S - 1].float(), kch[:, S - 1])
    assert torch.allclose(dec[0], out[S - 1], atol=2 ** -7)


def test_chunked_prefill_equals_single_chunk():
    gen = torch.Generator().manual_seed(7)
    shape = O.LayerShape(4, 1, 64, 16)
    S = 12
    qp = O.randn_bf16(gen, S, 4 * 128)
    kr = O.randn_bf16(gen, S, 64)
    vr = O.randn_bf16(gen, S, 64)
    qw, kw = O.norm_weights(gen, 64)
    cos, sin = O.rope_tables(16, 64, 1e7)
    full, kf, vf = O.prefill_layer(shape, qp, kr, vr, qw, kw, cos, sin, 0)
    a, ka, va = O.prefill_layer(shape, qp[:5], kr[:5], vr[:5], qw, kw, cos, sin, 0)
    b, kb, vb = O.prefill_layer(shape, qp[5:], kr[5:], vr[5:], qw, kw, cos, sin, 5, ka, va)
    assert torch.equal(torch.cat([ka, kb], 1), kf)
    assert torch.allclose(torch.cat([a, b]), full, atol=2 ** -7)
