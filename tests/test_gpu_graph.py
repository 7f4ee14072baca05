"""A whole decode layer (input norm + Q/K/V projections, fused attention step,
output projection + residual), a fused prefill chunk and a mixed call (two
streams forked and joined inside the capture) captured into a HIP graph
through torch.cuda.CUDAGraph.  The entry points allocate nothing once
their workspaces exist and record no memset nodes.  The prefill is
deterministic, so its replays equal the eager result bit for bit; the decode
waves claim 16-token blocks dynamically, so the fp32 order of their merge and
the running max against which each probability is rounded to bf16 (the PV
operand) vary between any two runs, eager or replayed: its replays are held to
two bf16 ulps of the eager result (and most entries identical) plus an absolute
2^-8 (entries near zero come from cancellation, and their own ulp is far
below the summation-order error of the terms).  Replays are
separated by eager work (the hidden state is reset, outputs are read back)."""
import pytest
import torch

from gpu_util import DEV, announce, gen
from oracle import attn_oracle as O
from supersonic_amd import kernel_ffi as K

pytestmark = pytest.mark.gpu


def decode_layer_inputs(B, Hq, Hkv, D, rot, hid, L, seed):
    g = gen(seed)
    d = dict(hidden=O.randn_bf16(g, B, hid), nw=O.randn_bf16(g, hid, std=0.1))
    d["wq"], d["wk"], d["wv"] = (O.randn_bf16(g, n, hid, std=hid ** -0.5) for n in (Hq * 2 * D, Hkv * D, Hkv * D))
    d["wo"] = O.randn_bf16(g, hid, Hq * D, std=(Hq * D) ** -0.5)
    d["qw"], d["kw"] = O.norm_weights(g, D)
    d["cos"], d["sin"] = O.rope_tables(rot, L + 2, 1.0e7)
    d["kc"] = O.randn_bf16(g, B, Hkv, L + 1, D)
    d["vc"] = O.randn_bf16(g, B, Hkv, L + 1, D)
    return {k: v.to(DEV) for k, v in d.items()}


def make_layer(B, Hq, Hkv, D, rot, hid, L, seed, stream):
    d = decode_layer_inputs(B, Hq, Hkv, D, rot, hid, L, seed)
    pos = torch.tensor([L - 3 * b for b in range(B)], dtype=torch.int32, device=DEV)
    cache = K.KvCache(d["kc"], d["vc"])
    q_proj = torch.empty(B, Hq * 2 * D, dtype=torch.bfloat16, device=DEV)
    k_new = torch.empty(B, Hkv * D, dtype=torch.bfloat16, device=DEV)
    v_new = torch.empty_like(k_new)
    attn = torch.empty(B, Hq * D, dtype=torch.bfloat16, device=DEV)
    hidden = d["hidden"].clone()

    def layer():
        K.qkv_proj(0, hidden, d["nw"], d["wq"], d["wk"], d["wv"], q_proj, k_new, v_new, stream=stream)
        K.fused_decode(0, q_proj, k_new, v_new, d["qw"], d["kw"], d["cos"], d["sin"], pos, cache, attn,
                       q_heads=Hq, kv_heads=Hkv, head_dim=D, rotary_dim=rot, max_kv_len=L + 1, stream=stream)
        K.o_proj_residual(0, attn, d["wo"], hidden, stream=stream)
    return layer, hidden, d["hidden"], attn


@pytest.mark.parametrize("B,Hq,Hkv,hid,L", [(1, 8, 2, 1024, 2048), (8, 16, 4, 4096, 4000)])
def test_decode_layer_graph_replays_match_eager(B, Hq, Hkv, hid, L):
    announce(f"decode layer graph B={B} Hq={Hq} Hkv={Hkv} hidden={hid} L={L}")
    s = torch.cuda.Stream()
    layer, hidden, hidden0, attn = make_layer(B, Hq, Hkv, 256, 64, hid, L, 91, s)
    with torch.cuda.stream(s):
        layer()  # eager: workspaces are allocated here, before the capture
    s.synchronize()
    eager_h, eager_a = hidden.clone(), attn.clone()
    g = torch.cuda.CUDAGraph()
    hidden.copy_(hidden0)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        layer()
    for r in range(3):
        hidden.copy_(hidden0)
        attn.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_close_ulps(attn, eager_a, f"replay {r}: attention", floor=2.0 ** -8)
        # a near-zero residual sum has a small ulp: the floor is the projection's scale
        assert_close_ulps(hidden, eager_h, f"replay {r}: hidden", floor=2.0 ** -6)


def assert_close_ulps(out, ref, name, floor=0.0):
    x, y = out.float(), ref.float()
    ulp = torch.exp2(torch.floor(torch.log2(y.abs().clamp_min(2.0 ** -100))) - 7)
    bad = (x - y).abs() > 2 * ulp + floor
    assert not bad.any(), f"{name}: {int(bad.sum())} entries beyond 2 ulps, max diff {(x - y).abs().max().item():.3e}"
    assert (x == y).float().mean().item() > 0.75, f"{name}: too few identical entries"


def test_decode_eager_runs_agree_to_ulps():
    """Two eager runs of the same step: the dynamic block claiming changes only
    the fp32 summation order."""
    announce("decode eager repeat")
    s = torch.cuda.Stream()
    layer, hidden, hidden0, attn = make_layer(8, 16, 4, 256, 64, 4096, 4000, 93, s)
    outs = []
    for _ in range(2):
        hidden.copy_(hidden0)
        with torch.cuda.stream(s):
            layer()
        s.synchronize()
        outs.append(attn.clone())
    assert_close_ulps(outs[1], outs[0], "eager repeat", floor=2.0 ** -8)


def test_decode_deterministic_runs_are_identical(monkeypatch):
    """SUPERSONIC_DECODE_DETERMINISTIC=1: a static block order, so two eager
    runs of the same step give the same bits."""
    announce("decode deterministic repeat")
    monkeypatch.setenv("SUPERSONIC_DECODE_DETERMINISTIC", "1")
    s = torch.cuda.Stream()
    layer, hidden, hidden0, attn = make_layer(8, 16, 4, 256, 64, 4096, 4000, 94, s)
    outs = []
    for _ in range(3):
        hidden.copy_(hidden0)
        with torch.cuda.stream(s):
            layer()
        s.synchronize()
        outs.append(attn.clone())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_prefill_graph_replays_match_eager():
    announce("prefill graph")
    S, Hq, Hkv, D, rot, start = 300, 16, 4, 256, 64, 200
    g0 = gen(92)
    qp = O.randn_bf16(g0, S, Hq * 2 * D).to(DEV)
    kr = O.randn_bf16(g0, S, Hkv * D).to(DEV)
    vr = O.randn_bf16(g0, S, Hkv * D).to(DEV)
    qw, kw = (t.to(DEV) for t in O.norm_weights(g0, D))
    cos, sin = (t.to(DEV) for t in O.rope_tables(rot, start + S + 1, 1.0e7))
    kc = O.randn_bf16(g0, 1, Hkv, start + S, D).to(DEV)
    vc = O.randn_bf16(g0, 1, Hkv, start + S, D).to(DEV)
    cache = K.KvCache(kc, vc)
    out = torch.empty(S, Hq * D, dtype=torch.bfloat16, device=DEV)
    s = torch.cuda.Stream()

    def step():
        K.fused_prefill(0, qp, kr, vr, qw, kw, cos, sin, cache, out, q_heads=Hq, kv_heads=Hkv, head_dim=D,
                        rotary_dim=rot, chunk_start=start, stream=s)
    with torch.cuda.stream(s):
        step()
    s.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    for r in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"


def test_first_call_captured_with_caller_workspaces():
    """Every entry point of a decode layer and a prefill chunk captured into a
    graph on its FIRST call at a new size, with caller-owned workspaces (sized by
    the *_workspace_size queries, zero-filled once): nothing is allocated or
    synchronised inside the capture, and the replays agree with eager runs that
    use the library's own workspaces."""
    announce("first-call capture with caller workspaces")
    B, Hq, Hkv, D, rot, hid, L = 2, 16, 4, 256, 64, 2048, 1500
    s = torch.cuda.Stream()
    d = decode_layer_inputs(B, Hq, Hkv, D, rot, hid, L, 95)
    pos = torch.tensor([L, L - 7], dtype=torch.int32, device=DEV)
    q_proj = torch.empty(B, Hq * 2 * D, dtype=torch.bfloat16, device=DEV)
    k_new = torch.empty(B, Hkv * D, dtype=torch.bfloat16, device=DEV)
    v_new = torch.empty_like(k_new)
    attn = torch.empty(B, Hq * D, dtype=torch.bfloat16, device=DEV)
    S, start = 200, 64
    g0 = gen(96)
    qp = O.randn_bf16(g0, S, Hq * 2 * D).to(DEV)
    kr = O.randn_bf16(g0, S, Hkv * D).to(DEV)
    vr = O.randn_bf16(g0, S, Hkv * D).to(DEV)
    pout = torch.empty(S, Hq * D, dtype=torch.bfloat16, device=DEV)
    zeros = lambda n: torch.zeros(max(int(n), 1), dtype=torch.uint8, device=DEV)
    ws = dict(qkv=zeros(K.qkv_proj_workspace_size(B, hid, Hq * 2 * D, Hkv * D)),
              dec=zeros(K.decode_workspace_size(B, Hq, Hkv, D, L + 1)),
              op=zeros(K.o_proj_workspace_size(B, hid, Hq * D)),
              pre=zeros(K.prefill_workspace_size(False, Hkv, D, S, start)))

    def run(hidden, cache, pcache, use_ws):
        w = ws if use_ws else {}
        K.qkv_proj(0, hidden, d["nw"], d["wq"], d["wk"], d["wv"], q_proj, k_new, v_new, stream=s,
                   workspace=w.get("qkv"))
        K.fused_decode(0, q_proj, k_new, v_new, d["qw"], d["kw"], d["cos"], d["sin"], pos, cache, attn,
                       q_heads=Hq, kv_heads=Hkv, head_dim=D, rotary_dim=rot, max_kv_len=L + 1, stream=s,
                       workspace=w.get("dec"))
        K.o_proj_residual(0, attn, d["wo"], hidden, stream=s, workspace=w.get("op"))
        K.fused_prefill(0, qp, kr, vr, d["qw"], d["kw"], d["cos"], d["sin"], pcache, pout, q_heads=Hq,
                        kv_heads=Hkv, head_dim=D, rotary_dim=rot, chunk_start=start, stream=s,
                        workspace=w.get("pre"))

    pk = O.randn_bf16(g0, 1, Hkv, start + S, D).to(DEV)
    pv = O.randn_bf16(g0, 1, Hkv, start + S, D).to(DEV)
    hidden = d["hidden"].clone()
    cache = K.KvCache(d["kc"].clone(), d["vc"].clone())
    pcache = K.KvCache(pk.clone(), pv.clone())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run(hidden, cache, pcache, True)
    # eager reference with library-owned workspaces
    e_hidden = d["hidden"].clone()
    e_cache = K.KvCache(d["kc"].clone(), d["vc"].clone())
    e_pcache = K.KvCache(pk.clone(), pv.clone())
    with torch.cuda.stream(s):
        run(e_hidden, e_cache, e_pcache, False)
    s.synchronize()
    e_attn, e_pout = attn.clone(), pout.clone()
    for r in range(3):
        hidden.copy_(d["hidden"])
        attn.zero_()
        pout.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_close_ulps(attn, e_attn, f"replay {r}: attention", floor=2.0 ** -8)
        assert_close_ulps(hidden, e_hidden, f"replay {r}: hidden", floor=2.0 ** -6)
        assert torch.equal(pout, e_pout), f"replay {r}: prefill"
        assert int(ws["dec"][:65536].count_nonzero()) == 0


def test_mixed_call_graph_replays_match_eager(monkeypatch):
    """A mixed call in its CU-split mode (the decode on 32 workgroups from the
    capturing stream, the chunk on the library stream, forked and joined by
    events) captured after one eager call (which creates the library stream),
    on a caller workspace: every replay gives the eager chunk output bit for bit
    and the decode under SUPERSONIC_DECODE_DETERMINISTIC bit for bit, and the
    claim counters are back at zero after each replay."""
    monkeypatch.setenv("SUPERSONIC_MIXED_DECODE_WGS", "32")
    monkeypatch.setenv("SUPERSONIC_DECODE_DETERMINISTIC", "1")
    Hq, Hkv, D, rot, S, start = 8, 2, 128, 32, 300, 64
    lens = [700, 33, 1500]
    announce("mixed call graph")
    g = gen(95)
    qw, kw = (t.to(DEV) for t in O.norm_weights(g, D))
    cos, sin = (t.to(DEV) for t in O.rope_tables(rot, 2000, 1.0e7))
    kc = torch.zeros(1, Hkv, start + S, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    kc[0, :, :start] = O.randn_bf16(g, Hkv, start, D)
    vc[0, :, :start] = O.randn_bf16(g, Hkv, start, D)
    kc0, vc0 = kc.to(DEV), vc.to(DEV)
    dk0 = O.randn_bf16(g, len(lens), Hkv, 1600, D).to(DEV)
    dv0 = O.randn_bf16(g, len(lens), Hkv, 1600, D).to(DEV)
    chunk_cache = K.KvCache(kc0.clone(), vc0.clone())
    dec_cache = K.KvCache(dk0.clone(), dv0.clone())
    out_c = torch.empty(S, Hq * D, dtype=torch.bfloat16, device=DEV)
    out_d = torch.empty(len(lens), Hq * D, dtype=torch.bfloat16, device=DEV)
    chunk = {"q_proj": O.randn_bf16(g, S, Hq * 2 * D).to(DEV), "k_new": O.randn_bf16(g, S, Hkv * D).to(DEV),
             "v_new": O.randn_bf16(g, S, Hkv * D).to(DEV), "cache": chunk_cache, "out": out_c, "chunk_start": start}
    dec = {"q_proj": O.randn_bf16(g, len(lens), Hq * 2 * D).to(DEV),
           "k_new": O.randn_bf16(g, len(lens), Hkv * D).to(DEV), "v_new": O.randn_bf16(g, len(lens), Hkv * D).to(DEV),
           "positions": torch.tensor(lens, dtype=torch.int32, device=DEV), "cache": dec_cache, "out": out_d,
           "max_kv_len": max(lens) + 1}
    ws = torch.zeros(K.mixed_workspace_size(False, Hq, Hkv, D, chunk, dec), dtype=torch.uint8, device=DEV)
    s = torch.cuda.Stream()

    def call():
        K.fused_mixed(0, qw, kw, cos, sin, chunk=chunk, decode=dec, q_heads=Hq, kv_heads=Hkv, head_dim=D,
                      rotary_dim=rot, stream=s, workspace=ws)
    torch.cuda.synchronize()
    call()  # eager (creates the library stream)
    s.synchronize()
    eager_c, eager_d = out_c.clone(), out_d.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        call()
    for r in range(3):
        out_c.zero_()
        out_d.zero_()
        chunk_cache.k.copy_(kc0)
        chunk_cache.v.copy_(vc0)
        dec_cache.k.copy_(dk0)
        dec_cache.v.copy_(dv0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_c, eager_c), f"replay {r}: chunk"
        assert torch.equal(out_d, eager_d), f"replay {r}: decodes"
        assert int(ws[:2048].count_nonzero()) == 0, f"replay {r}: claim counters"
