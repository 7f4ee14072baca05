"""GPU parity at the BASELINE workloads that bench.py times, through the C ABI.

Each case runs the fused entry point at the benchmark's own shape, lengths and
seeds, and checks the result against the CPU oracle on identical inputs:

* config 2 at batch 1, 32 768 cached tokens (the B=1 split plan);
* config 4: FP8 e4m3 cache, batch 16, lengths ~ U[1024, 16384] (the ragged
  device-side split plan the benchmark times);
* config 5: one 8192-token prefill chunk and 32 decode sequences with lengths
  ~ U[512, 65536] sharing one block-paged cache of 64-token pages, the two
  calls back to back on one stream.

Large inputs are drawn on the GPU from seeded generators and copied to the host
for the oracle (the values are identical on both sides).  Tolerances: BF16 KV
max-abs 2e-2 / mean-abs 2e-3, FP8 KV 4e-2 / 4e-3; appended V rows bit-exact.
"""
import os

import pytest
import torch

from gpu_util import DEV, TOL_BF16, TOL_FP8, announce, check, dev, make_decode_case, oracle_decode
from oracle import attn_oracle as O
from supersonic_amd import kernel_ffi as K

pytestmark = pytest.mark.gpu


def gpu_randn(seed, *shape):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(*shape, generator=g, device=DEV, dtype=torch.float32).to(torch.bfloat16)


def fused_decode(case_dev, cache, B, Hq, Hkv, D, rot, max_len, stream=None):
    out = torch.full((B, Hq * D), float("nan"), dtype=torch.bfloat16, device=DEV)
    if stream is not None:
        stream.wait_stream(torch.cuda.current_stream())  # the fill above runs on the current stream
    K.fused_decode(0, case_dev["q_proj"], case_dev["k_new"], case_dev["v_new"], case_dev["qw"], case_dev["kw"],
                   case_dev["cos"], case_dev["sin"], case_dev["pos"], cache, out, q_heads=Hq, kv_heads=Hkv,
                   head_dim=D, rotary_dim=rot, max_kv_len=max_len, stream=stream)
    return out


def test_config2_batch1_32k():
    """Config 2 at B=1, L=32768: 16/4 heads, D 256, bf16 KV."""
    announce("config 2 B=1 L=32768")
    torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))
    case = make_decode_case(52, 1, 16, 4, 256, 64, [32768])
    cache = K.KvCache(dev(case["k"]), dev(case["v"]))
    cd = {k: dev(case[k]) for k in ("q_proj", "k_new", "v_new", "qw", "kw", "cos", "sin", "pos")}
    out = fused_decode(cd, cache, 1, 16, 4, 256, 64, 32769)
    torch.cuda.synchronize()
    ref, k_ref, v_ref, _, _ = oracle_decode(case)
    check(out, ref, TOL_BF16, "config2 B=1")
    assert torch.equal(cache.v[0, :, 32768].cpu(), v_ref[0, :, 32768])


def fp8_bulk(x):
    """Per-(token, head) absmax e4m3 codes of a large bf16 tensor on the GPU (input
    generation only: scale = max(absmax / 448, 1e-12), code = e4m3(x * (1 / scale)))."""
    xf = x.float()
    sc = (xf.abs().amax(-1) / 448.0).clamp(min=1e-12)
    codes = (xf * (1.0 / sc)[..., None]).to(torch.float8_e4m3fn).view(torch.uint8)
    return codes, sc.contiguous()


def test_config4_fp8_batch16_ragged():
    """Config 4: FP8 e4m3 KV with fp32 per-(token, head) scales, 16/4 heads, D 256,
    batch 16 with the benchmark's lengths (seed 4, U[1024, 16384])."""
    lens = torch.randint(1024, 16385, (16,), generator=torch.Generator().manual_seed(4)).tolist()
    announce(f"config 4 fp8 B=16 lens sum={sum(lens)}")
    torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))
    B, Hq, Hkv, D, rot, cap = 16, 16, 4, 256, 64, 16385
    case = make_decode_case(53, B, Hq, Hkv, D, rot, [0] * B, cap=1)  # small tensors; caches below
    case["cos"], case["sin"] = O.rope_tables(rot, cap + 1, 1.0e7)
    case["pos"] = torch.tensor(lens, dtype=torch.int32)
    kq, ks = fp8_bulk(gpu_randn(530, B, Hkv, cap, D))
    vq, vs = fp8_bulk(gpu_randn(531, B, Hkv, cap, D))
    case.update(k=kq.cpu(), v=vq.cpu(), ks=ks.cpu(), vs=vs.cpu())
    cache = K.KvCache(kq, vq, ks, vs)
    cd = {k: dev(case[k]) for k in ("q_proj", "k_new", "v_new", "qw", "kw", "cos", "sin", "pos")}
    out = fused_decode(cd, cache, B, Hq, Hkv, D, rot, max(lens) + 1)
    torch.cuda.synchronize()
    ref, k_ref, v_ref, ks_ref, vs_ref = oracle_decode(case, codec="ocp")
    check(out, ref, TOL_FP8, "config4 fp8")
    for b, p in enumerate(lens):
        assert torch.equal(cache.v[b, :, p].cpu(), v_ref[b, :, p])
        assert torch.equal(cache.v_scale[b, :, p].cpu(), vs_ref[b, :, p])


@pytest.mark.parametrize("mode", ["serial", "concurrent"])
def test_config5_mixed_paged_batch(mode, monkeypatch):
    """Config 5: 16/2 heads, D 256, bf16, one block-paged pool of 64-token pages
    holding an 8192-token prefill chunk (offset 0) and 32 decode sequences with
    the benchmark's lengths (seed 5, U[512, 65536]), both checked against the
    oracle.  serial: prefill then decode on one stream.  concurrent: one mixed
    call with the CU split (the decode planned for the estimate's workgroups
    (160 here), the chunk on a second stream with the dynamic schedule), made
    twice on a caller workspace, the second time with the decode on 96
    workgroups: the second call gives the same chunk output bit for bit and
    leaves the claim counters at zero."""
    Hq, Hkv, D, rot, ps, S = 16, 2, 256, 64, 64, 8192
    lens = torch.randint(512, 65537, (32,), generator=torch.Generator().manual_seed(5)).tolist()
    B = len(lens)
    announce(f"config 5: chunk {S} + {B} paged decodes, lens sum={sum(lens)}")
    torch.set_num_threads(max(1, min(16, os.cpu_count() or 1)))
    shape = O.LayerShape(Hq, Hkv, D, rot)
    g = torch.Generator().manual_seed(54)
    max_pos = max(max(lens) + 1, S) + 1
    cos, sin = O.rope_tables(rot, max_pos, 1.0e7)
    qw, kw = O.norm_weights(g, D)

    # page pool: the chunk's pages first, then each sequence's, in a random order
    chunk_pages = S // ps
    seq_pages = [(l + 1 + ps - 1) // ps for l in lens]
    total = chunk_pages + sum(seq_pages)
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(55)).to(torch.int32)
    kpool = torch.zeros(total, Hkv, ps, D, dtype=torch.bfloat16, device=DEV)
    vpool = torch.zeros_like(kpool)
    chunk_bt = perm[:chunk_pages].reshape(1, -1)
    maxp = max(seq_pages)
    dec_bt = torch.zeros(B, maxp, dtype=torch.int32)
    k_host, v_host = [], []
    at = chunk_pages
    for b, l in enumerate(lens):
        n = seq_pages[b]
        pages = perm[at:at + n]
        at += n
        dec_bt[b, :n] = pages
        kb = gpu_randn(1000 + 2 * b, Hkv, n * ps, D)
        vb = gpu_randn(1001 + 2 * b, Hkv, n * ps, D)
        pl = pages.to(DEV).long()
        kpool[pl] = kb.reshape(Hkv, n, ps, D).permute(1, 0, 2, 3)
        vpool[pl] = vb.reshape(Hkv, n, ps, D).permute(1, 0, 2, 3)
        k_host.append(kb.cpu())
        v_host.append(vb.cpu())

    # inputs of the two calls
    qp_c = O.randn_bf16(g, S, Hq * 2 * D)
    kn_c = O.randn_bf16(g, S, Hkv * D)
    vn_c = O.randn_bf16(g, S, Hkv * D)
    qp_d = O.randn_bf16(g, B, Hq * 2 * D)
    kn_d = O.randn_bf16(g, B, Hkv * D)
    vn_d = O.randn_bf16(g, B, Hkv * D)
    pos = torch.tensor(lens, dtype=torch.int32)

    st = torch.cuda.Stream()
    cos_d, sin_d, qw_d, kw_d = cos.to(DEV), sin.to(DEV), qw.to(DEV), kw.to(DEV)
    chunk_cache = K.KvCache(kpool, vpool, block_table=chunk_bt.to(DEV))
    dec_cache = K.KvCache(kpool, vpool, block_table=dec_bt.to(DEV))
    out_c = torch.full((S, Hq * D), float("nan"), dtype=torch.bfloat16, device=DEV)
    args_c = [t.to(DEV) for t in (qp_c, kn_c, vn_c)]
    args_d = {"q_proj": qp_d.to(DEV), "k_new": kn_d.to(DEV), "v_new": vn_d.to(DEV), "qw": qw_d, "kw": kw_d,
              "cos": cos_d, "sin": sin_d, "pos": pos.to(DEV)}
    torch.cuda.synchronize()
    if mode == "serial":
        K.fused_prefill(0, *args_c, qw_d, kw_d, cos_d, sin_d, chunk_cache, out_c, q_heads=Hq, kv_heads=Hkv,
                        head_dim=D, rotary_dim=rot, chunk_start=0, stream=st)
        out_d = fused_decode(args_d, dec_cache, B, Hq, Hkv, D, rot, max(lens) + 1, stream=st)
        st.synchronize()
    else:
        out_d = torch.full((B, Hq * D), float("nan"), dtype=torch.bfloat16, device=DEV)
        chunk = {"q_proj": args_c[0], "k_new": args_c[1], "v_new": args_c[2], "cache": chunk_cache, "out": out_c,
                 "chunk_start": 0}
        dec = {"q_proj": args_d["q_proj"], "k_new": args_d["k_new"], "v_new": args_d["v_new"],
               "positions": args_d["pos"], "cache": dec_cache, "out": out_d, "max_kv_len": max(lens) + 1}
        ws = torch.zeros(K.mixed_workspace_size(False, Hq, Hkv, D, chunk, dec), dtype=torch.uint8, device=DEV)
        monkeypatch.delenv("SUPERSONIC_MIXED_DECODE_WGS", raising=False)
        K.fused_mixed(0, qw_d, kw_d, cos_d, sin_d, chunk=chunk, decode=dec, q_heads=Hq, kv_heads=Hkv, head_dim=D,
                      rotary_dim=rot, stream=st, workspace=ws)
        st.synchronize()
        assert int(ws[:2048].count_nonzero()) == 0, "claim counters not left at zero"
        first_c = out_c.clone()
        first_d = out_d.clone()
        out_c.fill_(float("nan"))
        monkeypatch.setenv("SUPERSONIC_MIXED_DECODE_WGS", "96")
        K.fused_mixed(0, qw_d, kw_d, cos_d, sin_d, chunk=chunk, decode=dec, q_heads=Hq, kv_heads=Hkv, head_dim=D,
                      rotary_dim=rot, stream=st, workspace=ws)
        st.synchronize()
        monkeypatch.delenv("SUPERSONIC_MIXED_DECODE_WGS")
        assert int(ws[:2048].count_nonzero()) == 0, "claim counters not left at zero"
        assert torch.equal(out_c, first_c), "second mixed call: chunk output differs"
        check(out_d, first_d.float().cpu(), TOL_BF16, "config5 decode, second mixed call")

    # decode sequences against the oracle
    ref_d = O.decode_layer(shape, qp_d, kn_d, vn_d, qw, kw, cos, sin, pos.long(), k_host, v_host)
    check(out_d, ref_d, TOL_BF16, "config5 decode")
    for b, l in enumerate(lens):
        pg = int(dec_bt[b, l // ps])
        assert torch.equal(vpool[pg, :, l % ps].cpu(), v_host[b][:, l])
    del k_host, v_host

    # the chunk against the oracle, and its K/V rows in the pool
    ref_c, kch, vch = O.prefill_layer(shape, qp_c, kn_c, vn_c, qw, kw, cos, sin, 0)
    check(out_c, ref_c, TOL_BF16, "config5 prefill chunk")
    pages = chunk_bt[0].to(DEV).long()
    vrows = vpool[pages].permute(1, 0, 2, 3).reshape(Hkv, S, D).float().cpu()
    assert torch.equal(vrows, vch)
    krows = kpool[pages].permute(1, 0, 2, 3).reshape(Hkv, S, D).float().cpu()
    assert (krows - kch).abs().max().item() <= 2 ** -7 * kch.abs().max().item()
