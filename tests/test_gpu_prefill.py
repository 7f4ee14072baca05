"""GPU parity of the causal prefill path through the C ABI (MFMA kernel)."""
import json
import os

import pytest
import torch

from gpu_util import DEV, TOL_BF16, announce, check, fp8_rows, gen
from oracle import fp8_codec
from oracle import attn_oracle as O
from supersonic_amd import kernel_ffi as K

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def dropin(q, k, v, off, dtype=K.ScalarType.BF16):
    B, Hq, S, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    out = torch.full((B, Hq, S, D), float("nan"), dtype=torch.float32, device=DEV)
    K.full_attention_prefill(0, dtype, B, Hq, Hkv, S, L, D, D ** -0.5, off, q.to(DEV), k.to(DEV), v.to(DEV), out)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("name", ["prefill_tiny.json", "prefill_clamped.json"])
def test_prefill_golden(name):
    announce(f"prefill golden {name}")
    g = json.load(open(os.path.join(GOLD, name)))
    B, Hq, Hkv, S, L, D = g["B"], g["Hq"], g["Hkv"], g["S"], g["L"], g["D"]
    q = torch.tensor(g["q"]).reshape(B, Hq, S, D).bfloat16()
    k = torch.tensor(g["k"]).reshape(B, Hkv, L, D).bfloat16()
    v = torch.tensor(g["v"]).reshape(B, Hkv, L, D).bfloat16()
    out = dropin(q, k, v, g["seqlen_offset"])
    check(out, torch.tensor(g["out"]).reshape(B, Hq, S, D), (1e-2, 1e-3), name)


@pytest.mark.parametrize("dtype", [K.ScalarType.BF16, K.ScalarType.F16, K.ScalarType.F32])
@pytest.mark.parametrize("B,Hq,Hkv,S,off,D", [
    (1, 4, 2, 300, 0, 256), (2, 8, 2, 129, 40, 128), (1, 2, 1, 64, 0, 64), (1, 16, 4, 200, 1000, 256),
    (1, 2, 2, 1, 5, 256),
])
def test_prefill_dropin_matches_oracle(dtype, B, Hq, Hkv, S, off, D):
    announce(f"prefill dropin dtype={dtype} B={B} Hq={Hq} Hkv={Hkv} S={S} off={off} D={D}")
    tdt = {K.ScalarType.BF16: torch.bfloat16, K.ScalarType.F16: torch.float16, K.ScalarType.F32: torch.float32}[dtype]
    g = gen(61)
    L = off + S
    q = torch.randn(B, Hq, S, D, generator=g).to(tdt)
    k = torch.randn(B, Hkv, L, D, generator=g).to(tdt)
    v = torch.randn(B, Hkv, L, D, generator=g).to(tdt)
    out = dropin(q, k, v, off, dtype)
    ref = O.attention_prefill(q.float(), k.float(), v.float(), D ** -0.5, off)
    check(out, ref, TOL_BF16 if dtype != K.ScalarType.F32 else (1e-4, 1e-5), "prefill")


@pytest.mark.parametrize("dtype", [K.ScalarType.BF16, K.ScalarType.F16])
@pytest.mark.parametrize("B,Hq,Hkv,S,off,D", [
    (1, 4, 2, 300, 0, 80), (2, 8, 2, 129, 40, 96), (1, 16, 4, 200, 100, 192), (1, 2, 1, 70, 3, 36),
    (1, 4, 2, 65, 10, 320), (1, 2, 2, 33, 0, 512), (1, 2, 1, 17, 4, 500),
])
def test_prefill_dropin_general_head_sizes(dtype, B, Hq, Hkv, S, off, D):
    """Head sizes other than 64/128/256, up to 512, as the reference's prefill
    takes any head_dim <= 8 x wave size (full_attention_bridge.cpp:86-88):
    zero-padded copies on the MFMA kernel up to 256, the f32 kernel above."""
    announce(f"prefill dropin general dtype={dtype} B={B} Hq={Hq} Hkv={Hkv} S={S} off={off} D={D}")
    tdt = torch.bfloat16 if dtype == K.ScalarType.BF16 else torch.float16
    g = gen(63)
    L = off + S
    q = torch.randn(B, Hq, S, D, generator=g).to(tdt)
    k = torch.randn(B, Hkv, L, D, generator=g).to(tdt)
    v = torch.randn(B, Hkv, L, D, generator=g).to(tdt)
    out = dropin(q, k, v, off, dtype)
    ref = O.attention_prefill(q.float(), k.float(), v.float(), D ** -0.5, off)
    check(out, ref, TOL_BF16, f"prefill D={D}")


def test_prefill_kv_shorter_than_causal_limit():
    """kv_len < seqlen_offset + q_len: every row is clamped to kv_len keys."""
    announce("prefill clamp")
    g = gen(62)
    q = O.randn_bf16(g, 1, 4, 150, 128)
    k = O.randn_bf16(g, 1, 2, 90, 128)
    v = O.randn_bf16(g, 1, 2, 90, 128)
    out = dropin(q, k, v, 20)
    check(out, O.attention_prefill(q, k, v, 128 ** -0.5, 20), TOL_BF16, "clamp")


def test_prefill_empty_kv_gives_zeros():
    q = torch.randn(1, 2, 5, 64).bfloat16()
    k = torch.zeros(1, 1, 0, 64).bfloat16()
    out = torch.full((1, 2, 5, 64), 7.0, device=DEV)
    K.full_attention_prefill(0, 2, 1, 2, 1, 5, 0, 64, 0.125, 0, q.to(DEV), torch.zeros(64, device=DEV),
                             torch.zeros(64, device=DEV), out)
    torch.cuda.synchronize()
    assert torch.all(out == 0)


def fused_case(seed, S, Hq, Hkv, D, rot, chunk_start=0, cap=None):
    g = gen(seed)
    cap = cap or (chunk_start + S)
    c = dict(q_proj=O.randn_bf16(g, S, Hq * 2 * D), k_new=O.randn_bf16(g, S, Hkv * D),
             v_new=O.randn_bf16(g, S, Hkv * D))
    c["qw"], c["kw"] = O.norm_weights(g, D)
    c["cos"], c["sin"] = O.rope_tables(rot, cap + 1, 1.0e7)
    c["shape"] = O.LayerShape(Hq, Hkv, D, rot)
    c["prefix_k"] = O.randn_bf16(g, Hkv, chunk_start, D)
    c["prefix_v"] = O.randn_bf16(g, Hkv, chunk_start, D)
    return c


def run_fused_prefill(c, chunk_start, cache):
    sh = c["shape"]
    S = c["q_proj"].shape[0]
    out = torch.full((S, sh.q_heads * sh.head_dim), float("nan"), dtype=torch.bfloat16, device=DEV)
    K.fused_prefill(0, c["q_proj"].to(DEV), c["k_new"].to(DEV), c["v_new"].to(DEV), c["qw"].to(DEV),
                    c["kw"].to(DEV), c["cos"].to(DEV), c["sin"].to(DEV), cache, out, q_heads=sh.q_heads,
                    kv_heads=sh.kv_heads, head_dim=sh.head_dim, rotary_dim=sh.rotary_dim, chunk_start=chunk_start)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("S,Hq,Hkv,D,rot,start", [
    (512, 16, 4, 256, 64, 0), (200, 8, 2, 128, 32, 0), (333, 16, 4, 256, 64, 700), (64, 4, 1, 64, 32, 3),
    # rotary halves of 48 (the LDS-staged prologue), 64, 128 (operand-layout
    # prologue, partner chunks 2 and 4 apart) and a full-width rotation at D 128
    (160, 4, 1, 256, 96, 50), (160, 4, 1, 256, 128, 50), (130, 8, 2, 256, 256, 17), (96, 4, 2, 128, 128, 0),
])
def test_fused_prefill_matches_oracle(S, Hq, Hkv, D, rot, start):
    announce(f"fused prefill S={S} Hq={Hq} Hkv={Hkv} D={D} start={start}")
    c = fused_case(71, S, Hq, Hkv, D, rot, start)
    cap = start + S + 37
    kc = torch.zeros(1, Hkv, cap, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc[0, :, :start] = c["prefix_k"]
    vc[0, :, :start] = c["prefix_v"]
    cache = K.KvCache(kc.to(DEV), vc.to(DEV))
    out = run_fused_prefill(c, start, cache)
    ref, kch, vch = O.prefill_layer(c["shape"], c["q_proj"], c["k_new"], c["v_new"], c["qw"], c["kw"], c["cos"],
                                    c["sin"], start, c["prefix_k"], c["prefix_v"])
    check(out, ref, TOL_BF16, "fused prefill")
    kd = (cache.k[0, :, start:start + S].float().cpu() - kch).abs()
    assert kd.max().item() <= 2 ** -7 * kch.abs().max().item()
    assert torch.equal(cache.v[0, :, start:start + S].float().cpu(), vch)


def test_fused_prefill_paged():
    announce("fused prefill paged")
    S, Hq, Hkv, D, rot, ps = 400, 16, 2, 256, 64, 64
    start = 128
    c = fused_case(72, S, Hq, Hkv, D, rot, start)
    npages = (start + S + ps - 1) // ps
    perm = torch.randperm(npages + 3, generator=gen(9))[:npages].to(torch.int32)
    kp = torch.zeros(npages + 3, Hkv, ps, D, dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    for t in range(start):
        kp[perm[t // ps], :, t % ps] = c["prefix_k"][:, t]
        vp[perm[t // ps], :, t % ps] = c["prefix_v"][:, t]
    cache = K.KvCache(kp.to(DEV), vp.to(DEV), block_table=perm.reshape(1, -1).to(DEV))
    out = run_fused_prefill(c, start, cache)
    ref, _, vch = O.prefill_layer(c["shape"], c["q_proj"], c["k_new"], c["v_new"], c["qw"], c["kw"], c["cos"],
                                  c["sin"], start, c["prefix_k"], c["prefix_v"])
    check(out, ref, TOL_BF16, "paged prefill")
    t = start + 5
    assert torch.equal(cache.v[int(perm[t // ps]), :, t % ps].float().cpu(), vch[:, 5])


def test_fused_prefill_config3_full_size():
    """Config 3: 4096 tokens, 16/4 heads, D 256, fused norm/RoPE/gate."""
    announce("fused prefill config 3 S=4096")
    S, Hq, Hkv, D, rot = 4096, 16, 4, 256, 64
    c = fused_case(73, S, Hq, Hkv, D, rot)
    cache = K.KvCache(torch.zeros(1, Hkv, S, D, dtype=torch.bfloat16, device=DEV),
                      torch.zeros(1, Hkv, S, D, dtype=torch.bfloat16, device=DEV))
    out = run_fused_prefill(c, 0, cache)
    torch.set_num_threads(max(1, os.cpu_count() or 1))
    ref, _, _ = O.prefill_layer(c["shape"], c["q_proj"], c["k_new"], c["v_new"], c["qw"], c["kw"], c["cos"],
                                c["sin"], 0)
    check(out, ref, TOL_BF16, "config3")


@pytest.mark.parametrize("S,Hq,Hkv,D,rot,start", [(200, 8, 2, 128, 32, 130), (64, 4, 1, 256, 64, 0)])
def test_fused_prefill_fp8_cache(S, Hq, Hkv, D, rot, start):
    """FP8 (OCP e4m3) cache: the prefix is read back dequantised, the chunk's own
    K/V enter the attention unquantised (the reference runs prefill in bf16 and
    quantises the cache afterwards), and the appended codes and scales are the
    oracle quantiser's, bit for bit."""
    announce(f"fused prefill fp8 S={S} Hq={Hq} Hkv={Hkv} D={D} start={start}")
    c = fused_case(74, S, Hq, Hkv, D, rot, start)
    cap = start + S + 7
    kq = torch.zeros(1, Hkv, cap, D, dtype=torch.uint8)
    vq = torch.zeros_like(kq)
    ks = torch.zeros(1, Hkv, cap, dtype=torch.float32)
    vs = torch.zeros_like(ks)
    pk, pks = fp8_rows(c["prefix_k"])
    pv, pvs = fp8_rows(c["prefix_v"])
    kq[0, :, :start], ks[0, :, :start] = pk, pks
    vq[0, :, :start], vs[0, :, :start] = pv, pvs
    cache = K.KvCache(kq.to(DEV), vq.to(DEV), ks.to(DEV), vs.to(DEV))
    out = run_fused_prefill(c, start, cache)
    # prefix as the kernel reads it: codes times scale, rounded to bf16
    deq = lambda q, sc: (torch.from_numpy(fp8_codec.decode(q.numpy())) * sc[..., None]).bfloat16().float()
    ref, kch, vch = O.prefill_layer(c["shape"], c["q_proj"], c["k_new"], c["v_new"], c["qw"], c["kw"], c["cos"],
                                    c["sin"], start, deq(pk, pks), deq(pv, pvs))
    check(out, ref, TOL_BF16, "fused prefill fp8")
    # V reaches the cache unchanged, so its codes and scales are the quantiser's bit for bit
    ev, evs = fp8_rows(vch)
    assert torch.equal(cache.v[0, :, start:start + S].cpu(), ev)
    assert torch.equal(cache.v_scale[0, :, start:start + S].cpu(), evs)
    # K passes through norm and RoPE, whose bf16 results may differ from the oracle's by
    # one ulp: scales agree to that ulp, and the dequantised rows to one e4m3 step
    ek, eks = fp8_rows(kch)
    gk, gks = cache.k[0, :, start:start + S].cpu(), cache.k_scale[0, :, start:start + S].cpu()
    assert torch.allclose(gks, eks, rtol=2 ** -7, atol=0)
    assert (gk == ek).float().mean().item() > 0.98
    kd = deq(gk, gks) - kch
    assert kd.abs().max().item() <= 2 ** -3 * kch.abs().amax(-1).max().item()
    assert torch.equal(cache.k[0, :, :start].cpu(), pk)  # the prefix is untouched


def test_fused_prefill_fp8_full_size():
    """The fp8-KV lane at the bench shape: a 4096-token chunk after a 4096-token
    OCP e4m3 prefix, 16/4 heads, D 256.  The oracle covers three blocks of 128
    query rows (the first, the middle and the last of the chunk, each over its
    whole causal key range of up to 8192 keys) for every head; the bar is the
    bf16 one, since the prefix enters both sides dequantised the same way."""
    S, start, Hq, Hkv, D, rot = 4096, 4096, 16, 4, 256, 64
    announce(f"fused prefill fp8 full size S={S} start={start}")
    c = fused_case(75, S, Hq, Hkv, D, rot, start)
    cap = start + S
    pk, pks = fp8_rows(c["prefix_k"])
    pv, pvs = fp8_rows(c["prefix_v"])
    kq = torch.zeros(1, Hkv, cap, D, dtype=torch.uint8)
    vq = torch.zeros_like(kq)
    ks = torch.zeros(1, Hkv, cap, dtype=torch.float32)
    vs = torch.zeros_like(ks)
    kq[0, :, :start], ks[0, :, :start] = pk, pks
    vq[0, :, :start], vs[0, :, :start] = pv, pvs
    cache = K.KvCache(kq.to(DEV), vq.to(DEV), ks.to(DEV), vs.to(DEV))
    out = run_fused_prefill(c, start, cache).float().cpu()
    deq = lambda q, sc: (torch.from_numpy(fp8_codec.decode(q.numpy())) * sc[..., None]).bfloat16().float()
    sh = c["shape"]
    pos = torch.arange(start, start + S)
    q, gate, k = O.prep_qk(sh, c["q_proj"], c["k_new"], c["qw"], c["kw"], c["cos"], c["sin"], pos)
    v = O.bf16r(c["v_new"].float()).reshape(S, Hkv, D)
    k_all = torch.cat([deq(pk, pks), k.permute(1, 0, 2)], dim=1)[None]
    v_all = torch.cat([deq(pv, pvs), v.permute(1, 0, 2)], dim=1)[None]
    torch.set_num_threads(max(1, os.cpu_count() or 1))
    for r0 in (0, S // 2, S - 128):
        qb = q[r0:r0 + 128].permute(1, 0, 2)[None]
        attn = O.attention_prefill(qb, k_all, v_all, sh.scale, start + r0)[0]
        ref = O.sigmoid_mul(O.bf16r(attn).permute(1, 0, 2), gate[r0:r0 + 128]).reshape(128, Hq * D)
        check(out[r0:r0 + 128], ref, TOL_BF16, f"fp8 prefill rows {r0}..{r0 + 127}")
