"""supersonic_attn_gfx950_mixed: a prefill chunk and a decode batch of one layer in
one call, with the CU split (the decode planned for fewer workgroups, the chunk on
a second stream with the dynamic item schedule; its workgroup count from the
estimate or set by SUPERSONIC_MIXED_DECODE_WGS) and one after the other
(SUPERSONIC_MIXED_DECODE_WGS=0), each checked against the oracle.  The config-5
full-size case lives in test_gpu_configs.py."""
import pytest
import torch

from gpu_util import DEV, TOL_BF16, TOL_FP8, announce, check, dev, fp8_rows, gen, make_decode_case, oracle_decode
from oracle import attn_oracle as O
from oracle import fp8_codec
from supersonic_amd import kernel_ffi as K

pytestmark = pytest.mark.gpu


def _deq(q, sc):
    """e4m3 codes times their row scale, rounded to bf16 (the prefix as the kernels read it)."""
    return (torch.from_numpy(fp8_codec.decode(q.numpy())) * sc[..., None]).bfloat16().float()


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("split_wgs", [None, "0", "24"])
def test_mixed_matches_oracle(fp8, split_wgs, monkeypatch):
    """A 200-token chunk after a 130-token prefix (8/2 heads, D 128, rotary 32) and
    5 ragged decodes share the layer weights and one call; the chunk's sequence
    and the decodes have their own caches.  Checked against the oracle's prefill
    and decode steps, including the appended K/V (V bit for bit)."""
    if split_wgs is None:
        monkeypatch.delenv("SUPERSONIC_MIXED_DECODE_WGS", raising=False)
    else:
        monkeypatch.setenv("SUPERSONIC_MIXED_DECODE_WGS", split_wgs)
    Hq, Hkv, D, rot, S, start = 8, 2, 128, 32, 200, 130
    lens = [37, 300, 1, 1000, 513]
    B = len(lens)
    announce(f"mixed fp8={fp8} split_wgs={split_wgs}: chunk {S}@{start} + {B} decodes")
    dc = make_decode_case(81, B, Hq, Hkv, D, rot, lens, cap=max(lens) + 1 + 16, fp8=fp8)
    g = gen(82)
    qp_c = O.randn_bf16(g, S, Hq * 2 * D)
    kn_c = O.randn_bf16(g, S, Hkv * D)
    vn_c = O.randn_bf16(g, S, Hkv * D)
    pre_k = O.randn_bf16(g, Hkv, start, D)
    pre_v = O.randn_bf16(g, Hkv, start, D)
    cap_c = start + S + 5
    if fp8:
        kq = torch.zeros(1, Hkv, cap_c, D, dtype=torch.uint8)
        vq = torch.zeros_like(kq)
        ksc = torch.zeros(1, Hkv, cap_c, dtype=torch.float32)
        vsc = torch.zeros_like(ksc)
        pk, pks = fp8_rows(pre_k)
        pv, pvs = fp8_rows(pre_v)
        kq[0, :, :start], ksc[0, :, :start] = pk, pks
        vq[0, :, :start], vsc[0, :, :start] = pv, pvs
        chunk_cache = K.KvCache(kq.to(DEV), vq.to(DEV), ksc.to(DEV), vsc.to(DEV))
        dec_cache = K.KvCache(dev(dc["k"]), dev(dc["v"]), dev(dc["ks"]), dev(dc["vs"]))
        pre_k_ref, pre_v_ref = _deq(pk, pks), _deq(pv, pvs)
    else:
        kc = torch.zeros(1, Hkv, cap_c, D, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        kc[0, :, :start], vc[0, :, :start] = pre_k, pre_v
        chunk_cache = K.KvCache(kc.to(DEV), vc.to(DEV))
        dec_cache = K.KvCache(dev(dc["k"]), dev(dc["v"]))
        pre_k_ref, pre_v_ref = pre_k.float(), pre_v.float()
    # one rope table long enough for both parts
    cos, sin = O.rope_tables(rot, max(max(lens), start + S) + 2, 1.0e7)
    dc["cos"], dc["sin"] = cos, sin
    out_c = torch.full((S, Hq * D), float("nan"), dtype=torch.bfloat16, device=DEV)
    out_d = torch.full((B, Hq * D), float("nan"), dtype=torch.bfloat16, device=DEV)
    chunk = {"q_proj": qp_c.to(DEV), "k_new": kn_c.to(DEV), "v_new": vn_c.to(DEV), "cache": chunk_cache,
             "out": out_c, "chunk_start": start}
    dec = {"q_proj": dev(dc["q_proj"]), "k_new": dev(dc["k_new"]), "v_new": dev(dc["v_new"]),
           "positions": dev(dc["pos"]), "cache": dec_cache, "out": out_d, "max_kv_len": max(lens) + 1}
    ws = torch.zeros(K.mixed_workspace_size(fp8, Hq, Hkv, D, chunk, dec), dtype=torch.uint8, device=DEV)
    torch.cuda.synchronize()
    K.fused_mixed(0, dev(dc["qw"]), dev(dc["kw"]), cos.to(DEV), sin.to(DEV), chunk=chunk, decode=dec, q_heads=Hq,
                  kv_heads=Hkv, head_dim=D, rotary_dim=rot, workspace=ws)
    torch.cuda.synchronize()
    assert int(ws[:2048].count_nonzero()) == 0, "claim counters not left at zero"

    # decodes
    ref_d, _, v_ref, _, vs_ref = oracle_decode(dc)
    check(out_d, ref_d, TOL_FP8 if fp8 else TOL_BF16, "mixed decode")
    for b, l in enumerate(lens):
        assert torch.equal(dec_cache.v[b, :, l].cpu(), v_ref[b, :, l])
        if fp8:
            assert torch.equal(dec_cache.v_scale[b, :, l].cpu(), vs_ref[b, :, l])
    # the chunk (prefix read back as the kernel reads it)
    ref_c, _, vch = O.prefill_layer(O.LayerShape(Hq, Hkv, D, rot), qp_c, kn_c, vn_c, dc["qw"], dc["kw"], cos, sin,
                                    start, pre_k_ref, pre_v_ref)
    check(out_c, ref_c, TOL_BF16, "mixed chunk")
    if fp8:
        ev, evs = fp8_rows(vch)
        assert torch.equal(chunk_cache.v[0, :, start:start + S].cpu(), ev)
        assert torch.equal(chunk_cache.v_scale[0, :, start:start + S].cpu(), evs)
    else:
        assert torch.equal(chunk_cache.v[0, :, start:start + S].float().cpu(), vch)


def test_mixed_one_part_matches_the_single_calls(monkeypatch):
    """A mixed call with an empty decode batch is the prefill call, and one with an
    empty chunk the decode call (same outputs bit for bit; the decode under
    SUPERSONIC_DECODE_DETERMINISTIC, whose split order is fixed)."""
    import os
    Hq, Hkv, D, rot, S = 8, 2, 128, 32, 150
    announce("mixed with one part empty")
    monkeypatch.delenv("SUPERSONIC_MIXED_DECODE_WGS", raising=False)
    g = gen(83)
    qp = O.randn_bf16(g, S, Hq * 2 * D).to(DEV)
    kn = O.randn_bf16(g, S, Hkv * D).to(DEV)
    vn = O.randn_bf16(g, S, Hkv * D).to(DEV)
    qw, kw = (t.to(DEV) for t in O.norm_weights(g, D))
    cos, sin = (t.to(DEV) for t in O.rope_tables(rot, 2000, 1.0e7))

    def new_cache():
        return K.KvCache(torch.zeros(1, Hkv, S, D, dtype=torch.bfloat16, device=DEV),
                         torch.zeros(1, Hkv, S, D, dtype=torch.bfloat16, device=DEV))
    c1, c2 = new_cache(), new_cache()
    o1 = torch.empty(S, Hq * D, dtype=torch.bfloat16, device=DEV)
    o2 = torch.empty_like(o1)
    K.fused_prefill(0, qp, kn, vn, qw, kw, cos, sin, c1, o1, q_heads=Hq, kv_heads=Hkv, head_dim=D, rotary_dim=rot)
    K.fused_mixed(0, qw, kw, cos, sin, chunk={"q_proj": qp, "k_new": kn, "v_new": vn, "cache": c2, "out": o2},
                  decode=None, q_heads=Hq, kv_heads=Hkv, head_dim=D, rotary_dim=rot)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert torch.equal(c1.k, c2.k) and torch.equal(c1.v, c2.v)

    lens = [100, 1500, 7]
    dc = make_decode_case(84, len(lens), Hq, Hkv, D, rot, lens, cap=1600)
    os.environ["SUPERSONIC_DECODE_DETERMINISTIC"] = "1"
    try:
        outs = []
        for use_mixed in (False, True):
            cache = K.KvCache(dev(dc["k"]), dev(dc["v"]))
            out = torch.empty(len(lens), Hq * D, dtype=torch.bfloat16, device=DEV)
            args = [dev(dc[k]) for k in ("q_proj", "k_new", "v_new")]
            if use_mixed:
                K.fused_mixed(0, dev(dc["qw"]), dev(dc["kw"]), dev(dc["cos"]), dev(dc["sin"]), chunk=None,
                              decode={"q_proj": args[0], "k_new": args[1], "v_new": args[2],
                                      "positions": dev(dc["pos"]), "cache": cache, "out": out,
                                      "max_kv_len": max(lens) + 1},
                              q_heads=Hq, kv_heads=Hkv, head_dim=D, rotary_dim=rot)
            else:
                K.fused_decode(0, *args, dev(dc["qw"]), dev(dc["kw"]), dev(dc["cos"]), dev(dc["sin"]),
                               dev(dc["pos"]), cache, out, q_heads=Hq, kv_heads=Hkv, head_dim=D, rotary_dim=rot,
                               max_kv_len=max(lens) + 1)
            torch.cuda.synchronize()
            outs.append((out, cache))
    finally:
        del os.environ["SUPERSONIC_DECODE_DETERMINISTIC"]
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1].k, outs[1][1].k) and torch.equal(outs[0][1].v, outs[1][1].v)
