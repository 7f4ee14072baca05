"""GPU parity of the persistent decode layer (supersonic_attn_gfx950_decode_layer)
through the C ABI against the oracle's layer chain: input RMSNorm + Q/K/V
projections (oracle.qkv_proj), the decode step (oracle.decode_layer: QK norm,
RoPE, KV append, attention, gate) and o_proj + residual (oracle.o_proj_residual).

Bar: the updated hidden rows within 2e-2 x max(1, max|ref|) max-abs and 2e-3
mean-abs (BF16 KV; 4e-2 / 4e-3 for FP8 KV, as the decode tests state); the
appended V rows (the layer's own projection) within two bf16 ulps + 2^-10 of
the oracle's (the bar of the projection tests), at least 75% identical (the input
norm is summed in another order than the oracle's, which moves a few more roundings).  Two calls in a row on one workspace check that the
barrier and split counters are left at zero."""
import pytest
import torch

from gpu_util import DEV, announce, dev, fp8_rows, gen
from oracle import attn_oracle as O
from supersonic_amd import kernel_ffi as K

pytestmark = pytest.mark.gpu


def layer_case(seed, B, Hq, Hkv, D, rot, hid, lens, fp8=False, hidden_f32=False, page=None, max_extra=0):
    g = gen(seed)
    cap = max(lens) + 1
    if page:
        cap = (cap + page - 1) // page * page
    c = dict(B=B, Hq=Hq, Hkv=Hkv, D=D, rot=rot, hid=hid, lens=lens, fp8=fp8, page=page, max_extra=max_extra)
    c["hidden"] = O.randn_bf16(g, B, hid)
    c["nw"] = O.randn_bf16(g, hid, std=0.1)
    c["wq"], c["wk"], c["wv"] = (O.randn_bf16(g, n, hid, std=hid ** -0.5) for n in (Hq * 2 * D, Hkv * D, Hkv * D))
    c["wo"] = O.randn_bf16(g, hid, Hq * D, std=(Hq * D) ** -0.5)
    c["qw"], c["kw"] = O.norm_weights(g, D)
    c["cos"], c["sin"] = O.rope_tables(rot, cap + 1, 1.0e7)
    kc = O.randn_bf16(g, B, Hkv, cap, D)
    vc = O.randn_bf16(g, B, Hkv, cap, D)
    if fp8:
        c["k"], c["ks"] = fp8_rows(kc)
        c["v"], c["vs"] = fp8_rows(vc)
    else:
        c["k"], c["v"], c["ks"], c["vs"] = kc, vc, None, None
    c["hidden_dtype"] = torch.float32 if hidden_f32 else torch.bfloat16
    return c


def paged(c):
    """The contiguous cache of case c as a pool of pages in a shuffled order plus a block table."""
    ps, B, Hkv = c["page"], c["B"], c["Hkv"]
    per = c["k"].shape[2] // ps
    perm = torch.randperm(B * per, generator=gen(7))
    def pool(t):
        if t is None:
            return None
        out = torch.zeros((B * per, Hkv, ps) + tuple(t.shape[3:]), dtype=t.dtype)
        for b in range(B):
            for j in range(per):
                out[int(perm[b * per + j])] = t[b, :, j * ps:(j + 1) * ps]
        return out
    bt = torch.tensor([[int(perm[b * per + j]) for j in range(per)] for b in range(B)], dtype=torch.int32)
    return pool(c["k"]), pool(c["v"]), pool(c["ks"]), pool(c["vs"]), bt


def appended_v(c, cache, b, p):
    if not c["page"]:
        return cache.v[b, :, p].cpu()
    ps = c["page"]
    return cache.v[int(c["bt"][b, p // ps]), :, p % ps].cpu()


def run_layer(c, ws):
    if c["page"]:
        k, v, ks, vs, c["bt"] = paged(c)
        cache = K.KvCache(dev(k), dev(v), dev(ks), dev(vs), block_table=c["bt"].to(DEV))
    else:
        cache = K.KvCache(dev(c["k"]), dev(c["v"]), dev(c["ks"]), dev(c["vs"]))
    h = c["hidden"].to(c["hidden_dtype"]).to(DEV)
    pos = torch.tensor(c["lens"], dtype=torch.int32, device=DEV)
    K.decode_layer(0, h, dev(c["nw"]), dev(c["wq"]), dev(c["wk"]), dev(c["wv"]), dev(c["qw"]), dev(c["kw"]),
                   dev(c["wo"]), dev(c["cos"]), dev(c["sin"]), pos, cache, ws, q_heads=c["Hq"], kv_heads=c["Hkv"],
                   head_dim=c["D"], rotary_dim=c["rot"], max_kv_len=max(c["lens"]) + 1 + c["max_extra"])
    torch.cuda.synchronize()
    return h.float().cpu(), cache


def oracle_layer(c):
    B = c["B"]
    shape = O.LayerShape(c["Hq"], c["Hkv"], c["D"], c["rot"])
    rq, rk, rv = O.qkv_proj(c["hidden"], c["nw"], c["wq"], c["wk"], c["wv"])
    k = c["k"].clone()
    v = c["v"].clone()
    ks = None if c["ks"] is None else [c["ks"][b].clone() for b in range(B)]
    vs = None if c["vs"] is None else [c["vs"][b].clone() for b in range(B)]
    ra = O.decode_layer(shape, rq, rk, rv, c["qw"], c["kw"], c["cos"], c["sin"], c["lens"],
                        [k[b] for b in range(B)], [v[b] for b in range(B)], ks, vs, codec="ocp")
    return O.o_proj_residual(ra, c["wo"], c["hidden"]), v


def check_layer(c, out, cache, ref, v_ref):
    d = (out - ref).abs()
    scale = max(1.0, ref.abs().max().item())
    tol = (4e-2, 4e-3) if c["fp8"] else (2e-2, 2e-3)
    assert d.max().item() <= tol[0] * scale and d.mean().item() <= tol[1], \
        f"layer: max {d.max().item():.3e} mean {d.mean().item():.3e}"
    for b, p in enumerate(c["lens"]):
        # the appended V row is this layer's own projection: within the projection's
        # rounding (fp32 summation order) of the oracle's (fp8: one code)
        got, want = appended_v(c, cache, b, p), v_ref[b, :, p]
        if c["fp8"]:
            assert (got.int() - want.int()).abs().max().item() <= 1 or (got != want).float().mean().item() < 0.02
        else:
            gf, wf = got.float(), want.float()
            ulp = torch.exp2(torch.floor(torch.log2(wf.abs().clamp_min(2.0 ** -100))) - 7)
            assert bool(((gf - wf).abs() <= 2 * ulp + 2.0 ** -10).all()), (gf - wf).abs().max().item()
            assert (gf == wf).float().mean().item() > 0.75


CASES = {
    "config1": dict(B=1, Hq=8, Hkv=2, D=256, rot=64, hid=1024, lens=[2048]),
    # one sequence whose max_kv_len overstates its length: the layer's guess
    # of the decode work items (and of which workgroups skip phase 1) is wrong
    "config1_loose_max_kv_len": dict(B=1, Hq=8, Hkv=2, D=256, rot=64, hid=1024, lens=[2048], max_extra=5000),
    "one_short_sequence": dict(B=1, Hq=16, Hkv=4, D=256, rot=64, hid=2048, lens=[40]),
    "one_sequence_fp8_paged": dict(B=1, Hq=8, Hkv=2, D=256, rot=64, hid=1024, lens=[3000], fp8=True, page=64),
    "config2_b4_ragged": dict(B=4, Hq=16, Hkv=4, D=256, rot=64, hid=4096, lens=[3000, 17, 1500, 0]),
    "d128": dict(B=2, Hq=8, Hkv=2, D=128, rot=32, hid=2048, lens=[700, 2100]),
    "fp8": dict(B=2, Hq=16, Hkv=4, D=256, rot=64, hid=2048, lens=[1200, 333], fp8=True),
    "f32_hidden": dict(B=3, Hq=8, Hkv=2, D=256, rot=64, hid=1024, lens=[64, 65, 900], hidden_f32=True),
    "paged": dict(B=3, Hq=16, Hkv=4, D=256, rot=64, hid=2048, lens=[700, 64, 1500], page=64),
    "paged_fp8": dict(B=2, Hq=8, Hkv=2, D=128, rot=32, hid=1024, lens=[1000, 129], fp8=True, page=64),
    # 16 x 16 (sequence, kv head) pairs on a 256-workgroup grid, lengths for
    # which four chunk-growth steps of the plan still leave 272 items: the
    # layer must fall back to one split per sequence, not drop 16 items
    "many_kv_heads_ragged": dict(B=16, Hq=16, Hkv=16, D=128, rot=32, hid=2048,
                                 lens=[1105, 672, 613, 2390, 1186, 1479, 1618, 2247, 532, 1202, 471, 1959, 2993, 982,
                                       198, 1262]),
}


@pytest.mark.parametrize("name", list(CASES))
def test_decode_layer_matches_oracle_chain(name):
    kw = CASES[name]
    announce(f"persistent decode layer {name}: {kw}")
    c = layer_case(130, **kw)
    ws = torch.zeros(K.decode_layer_workspace_size(c["B"], c["hid"], c["Hq"], c["Hkv"], c["D"], max(c["lens"]) + 1),
                     dtype=torch.uint8, device=DEV)
    out, cache = run_layer(c, ws)
    ref, v_ref = oracle_layer(c)
    check_layer(c, out, cache, ref, v_ref)
    assert int(ws[:256].count_nonzero()) == 0, "barrier counters not reset"


def test_decode_layer_twice_on_one_workspace():
    """Two layers back to back on one workspace, the second smaller: the barrier
    and split counters each call leaves at zero serve the next."""
    cs = [layer_case(131, B=4, Hq=16, Hkv=4, D=256, rot=64, hid=4096, lens=[1000, 2000, 5, 4095]),
          layer_case(132, B=1, Hq=8, Hkv=2, D=256, rot=64, hid=1024, lens=[300])]
    n = max(K.decode_layer_workspace_size(c["B"], c["hid"], c["Hq"], c["Hkv"], c["D"], max(c["lens"]) + 1) for c in cs)
    ws = torch.zeros(n, dtype=torch.uint8, device=DEV)
    for i, c in enumerate(cs):
        announce(f"persistent decode layer, call {i}")
        out, cache = run_layer(c, ws)
        ref, v_ref = oracle_layer(c)
        check_layer(c, out, cache, ref, v_ref)


def test_decode_layer_rejects_unsupported_shapes():
    lib = K.load()
    z = torch.zeros(64, device=DEV)
    p = z.data_ptr()
    desc = K.KvCacheDesc()
    desc.k = desc.v = p
    call = lambda B, hid, hq=8, hkv=2, hd=256: lib.supersonic_attn_gfx950_decode_layer(
        0, None, 2, 2, B, hid, hq, hkv, hd, 64, 100, 1e-6, 1e-6, 0.0625, p, p, p, p, p, p, p, p, p, p, p,
        K.C.byref(desc), p, 1 << 30)
    assert call(17, 1024) == K.ERR["RANGE"]           # more rows than the staged weight stream takes
    assert call(8, 8192) == K.ERR["RANGE"]            # rows * hidden > 32768
    assert call(1, 1024, hq=16, hkv=2) == K.ERR["HEADS"]
    assert call(1, 1024, hd=64) == K.ERR["HEAD_DIM"]


def test_decode_layer_expired_barrier_is_reported(monkeypatch):
    """The host presets barrier 0's counter so that its flag is never raised and
    shortens the poll bound: every wait on it gives up after a few polls (the
    kernel still exits normally), the error word reports it, every counter and
    flag is back at zero, and the next call on the same workspace is correct
    and reports nothing."""
    c = layer_case(133, B=1, Hq=8, Hkv=2, D=256, rot=64, hid=1024, lens=[2048])
    ws = torch.zeros(K.decode_layer_workspace_size(c["B"], c["hid"], c["Hq"], c["Hkv"], c["D"], max(c["lens"]) + 1),
                     dtype=torch.uint8, device=DEV)
    assert K.wait_status() == 0
    ws[:4].view(torch.int32).fill_(0x40000000)  # barrier 0 counter: the arrivals never reach the grid size
    monkeypatch.setenv("SUPERSONIC_WAIT_POLLS", "16")
    announce("persistent decode layer with barrier 0 held (forced give-up)")
    run_layer(c, ws)
    bits = K.wait_status()
    assert bits & K.WAIT_LAYER_BARRIER, bits
    assert int(ws[:256].count_nonzero()) == 0, "counters not reset after a wait gave up"
    monkeypatch.delenv("SUPERSONIC_WAIT_POLLS")
    announce("persistent decode layer after the forced give-up")
    c = layer_case(134, B=1, Hq=8, Hkv=2, D=256, rot=64, hid=1024, lens=[2048])
    out, cache = run_layer(c, ws)
    assert K.wait_status() == 0
    ref, v_ref = oracle_layer(c)
    check_layer(c, out, cache, ref, v_ref)
