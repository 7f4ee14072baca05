"""GPU parity of the output projection + residual through the C ABI: the
drop-in GEMM (`matmul_rhs_transposed_tiled`), the drop-in `element_add` and the
native `o_proj_residual`.

Bar: every bf16 result is within one bf16 ulp of the oracle's (fp32
accumulation in a different order can move a rounding by one ulp); with the
residual, one ulp of the projection plus one ulp of the sum.  Adds are
bit-exact."""
import json
import os

import pytest
import torch

from gpu_util import DEV, announce, gen
from oracle import attn_oracle as O
from supersonic_amd import kernel_ffi as K

pytestmark = pytest.mark.gpu
G = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "proj_known_answer.json")))


def ulp(x):
    x = x.float().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(x)) - 7)


def assert_ulps(out, ref, slack, name):
    d = (out.float().cpu() - ref.float()).abs()
    bad = d > slack
    assert not bad.any(), f"{name}: {int(bad.sum())} entries off, worst {d.max().item():.3e}"


def dropin_matmul(lhs, rhs):
    batch, m, k = lhs.shape
    n = rhs.shape[1]
    out = torch.full((batch, m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    K.matmul_rhs_transposed(0, K.ScalarType.BF16, batch, m, n, k, lhs.to(DEV), rhs.to(DEV), out)
    torch.cuda.synchronize()
    return out.cpu()


def test_matmul_known_answer():
    announce("matmul known answer")
    g = G["matmul"]
    out = dropin_matmul(torch.tensor([g["lhs"]]).bfloat16(), torch.tensor([g["rhs"]]).bfloat16())
    assert torch.allclose(out[0].float(), torch.tensor(g["expected"]), atol=g["tolerance"])


@pytest.mark.parametrize("batch,m,n,k", [
    (1, 1, 64, 4096), (1, 8, 4096, 4096), (1, 17, 100, 264), (2, 16, 40, 72), (1, 64, 48, 512),
    (1, 65, 128, 256), (1, 300, 96, 200), (1, 5, 33, 100), (2, 130, 64, 96),
    (2, 8, 4096, 1024), (3, 16, 2048, 2048),  # the LDS-staged kernel with a batch dimension
    # the tiled GEMM: partial tiles in m, n and k, n not a multiple of 8 (scalar
    # epilogue), k not a multiple of 8 (the one-thread-per-output kernel), batch
    (1, 700, 1000, 520), (1, 257, 100, 264), (2, 300, 264, 136), (1, 40, 24, 36), (1, 512, 768, 1024),
])
def test_matmul_matches_oracle(batch, m, n, k):
    announce(f"matmul batch={batch} m={m} n={n} k={k}")
    g = gen(81)
    lhs = O.randn_bf16(g, batch, m, k)
    rhs = O.randn_bf16(g, batch, n, k, std=k ** -0.5)
    out = dropin_matmul(lhs, rhs)
    ref = O.matmul_rhs_transposed(lhs, rhs)
    assert_ulps(out, ref, ulp(ref) + 1e-6, "matmul")


def test_matmul_tail_split():
    """More tiles than CUs with a short last round: the tail tiles run as two
    half-k workgroups whose fp32 partials meet through the workspace.  Two calls
    in a row (the second of another shape and tail) check that each call leaves
    the hand-over flags cleared; the partial last k-tile sits in the second half."""
    for seed, (m, n, k) in enumerate([(4096, 4608, 512), (4100, 4608, 520), (4096, 4608, 512)]):
        announce(f"matmul tail split m={m} n={n} k={k}")
        g = gen(90 + seed)
        lhs = O.randn_bf16(g, 1, m, k)
        rhs = O.randn_bf16(g, 1, n, k, std=k ** -0.5)
        out = dropin_matmul(lhs, rhs)
        ref = O.matmul_rhs_transposed(lhs, rhs)
        assert_ulps(out, ref, ulp(ref) + 1e-6, f"matmul tail split {m}x{n}x{k}")


@pytest.mark.parametrize("m,k", [(12, 2728), (15, 2184), (16, 2048)])
def test_matmul_lds_staging_padded_rows(m, k, monkeypatch):
    """The LDS-staged kernel with rows whose padded end, m * k + 8 (m - 1), passes
    32768 elements: the surplus 16-byte chunks of the staging loop must not land
    inside a row."""
    announce(f"matmul lds staging m={m} k={k}")
    monkeypatch.setenv("SUPERSONIC_PROJ_SKINNY_MAX_M", "16")
    g = gen(84)
    lhs = O.randn_bf16(g, 1, m, k)
    rhs = O.randn_bf16(g, 1, 4096, k, std=k ** -0.5)
    out = dropin_matmul(lhs, rhs)
    ref = O.matmul_rhs_transposed(lhs, rhs)
    assert_ulps(out, ref, ulp(ref) + 1e-6, "matmul lds staging")


def test_matmul_empty_k_gives_zeros():
    out = torch.full((1, 3, 5), 7.0, dtype=torch.bfloat16, device=DEV)
    K.matmul_rhs_transposed(0, K.ScalarType.BF16, 1, 3, 5, 0, torch.zeros(8, device=DEV),
                            torch.zeros(8, device=DEV), out)
    torch.cuda.synchronize()
    assert torch.all(out == 0)


def test_matmul_rejects_other_dtypes():
    x = torch.zeros(16, device=DEV)
    with pytest.raises(K.GpuError) as e:
        K.matmul_rhs_transposed(0, K.ScalarType.F32, 1, 1, 1, 1, x, x, x)
    assert e.value.status == 272


@pytest.mark.parametrize("dtype,tdt", [(K.ScalarType.BF16, torch.bfloat16), (K.ScalarType.F16, torch.float16),
                                       (K.ScalarType.F32, torch.float32)])
def test_element_add(dtype, tdt):
    announce(f"element_add {tdt}")
    g = G["element_add"]
    a, b = torch.tensor(g["lhs"]).to(tdt), torch.tensor(g["rhs"]).to(tdt)
    out = torch.empty_like(a, device=DEV)
    K.element_add(0, dtype, 4, a.to(DEV), b.to(DEV), out)
    torch.cuda.synchronize()
    assert torch.allclose(out.cpu().float(), torch.tensor(g["expected"]), atol=g["tolerance"])
    gg = gen(82)
    a = torch.randn(100003, generator=gg).to(tdt)
    b = torch.randn(100003, generator=gg).to(tdt)
    out = torch.empty_like(a, device=DEV)
    K.element_add(0, dtype, a.numel(), a.to(DEV), b.to(DEV), out)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), (a.float() + b.float()).to(tdt))


def run_o_proj(attn, w, hidden):
    h = hidden.to(DEV)
    K.o_proj_residual(0, attn.to(DEV), w.to(DEV), h)
    torch.cuda.synchronize()
    return h.cpu()


def test_o_proj_known_answer():
    announce("o_proj known answer")
    g = G["matmul_residual"]
    out = run_o_proj(torch.tensor(g["lhs"]).bfloat16(), torch.tensor(g["rhs"]).bfloat16(),
                     torch.tensor(g["residual"]).bfloat16())
    assert torch.allclose(out.float(), torch.tensor(g["expected"]), atol=g["tolerance"])


@pytest.mark.parametrize("k", [2, 32])
def test_o_proj_two_roundings(k):
    """k=2 takes the GEMM path, k=32 the fused kernel: both round the projection first."""
    g = G["double_rounding"]
    attn = torch.zeros(1, k)
    attn[0, :2] = torch.tensor(g["attn"][0])
    w = torch.zeros(1, k)
    w[0, :2] = 1.0
    for dt in (torch.bfloat16, torch.float32):
        out = run_o_proj(attn.bfloat16(), w.bfloat16(), torch.tensor(g["hidden"]).to(dt))
        assert out.item() == g["expected"][0][0], (k, dt, out.item())


@pytest.mark.parametrize("rows,hidden_dim,attn_dim,max_m", [
    (8, 4096, 4096, None), (1, 2048, 4096, None), (16, 4096, 4096, None), (64, 256, 1024, None),
    (33, 300, 520, None), (100, 256, 512, None), (3, 64, 36, None),
    # the streaming kernel with 2..4 row blocks, and its k split over workgroups
    (16, 4096, 4096, 64), (33, 300, 520, 64), (64, 256, 1024, 64), (12, 512, 8192, None), (40, 512, 8192, 64),
    # the tiled GEMM with the residual epilogue after a tail split (288 tiles)
    (4096, 4608, 512, None),
])
@pytest.mark.parametrize("hdt", [torch.bfloat16, torch.float32])
def test_o_proj_residual_matches_oracle(rows, hidden_dim, attn_dim, max_m, hdt, monkeypatch):
    announce(f"o_proj rows={rows} hidden={hidden_dim} attn={attn_dim} max_m={max_m} hidden dtype {hdt}")
    if max_m is not None:
        monkeypatch.setenv("SUPERSONIC_PROJ_SKINNY_MAX_M", str(max_m))
    g = gen(83)
    attn = O.randn_bf16(g, rows, attn_dim)
    w = O.randn_bf16(g, hidden_dim, attn_dim, std=attn_dim ** -0.5)
    hidden = O.randn_bf16(g, rows, hidden_dim).to(hdt)
    out = run_o_proj(attn, w, hidden)
    add = O.matmul_rhs_transposed(attn, w)
    ref = O.o_proj_residual(attn, w, hidden)
    assert out.dtype == hdt
    assert torch.equal(out.float(), O.bf16r(out.float()))  # f32 hidden keeps bf16 values
    assert_ulps(out, ref, ulp(add) + ulp(ref) + 1e-6, "o_proj")
    assert (out.float() == ref).float().mean().item() > 0.95


@pytest.mark.parametrize("max_m", [None, "64", "0"])
def test_o_proj_repeated_calls(max_m, monkeypatch):
    """Back-to-back calls on one stream, the second smaller: the split-k arrival
    counters return to zero and the shared workspace carries nothing over."""
    announce(f"o_proj repeated calls max_m={max_m}")
    if max_m is not None:
        monkeypatch.setenv("SUPERSONIC_PROJ_SKINNY_MAX_M", max_m)
    g = gen(84)
    for rows, hid, adim in [(8, 512, 8192), (8, 512, 8192), (5, 256, 4096)]:
        attn = O.randn_bf16(g, rows, adim)
        w = O.randn_bf16(g, hid, adim, std=adim ** -0.5)
        hidden = O.randn_bf16(g, rows, hid)
        out = run_o_proj(attn, w, hidden)
        ref = O.o_proj_residual(attn, w, hidden)
        assert_ulps(out, ref, ulp(O.matmul_rhs_transposed(attn, w)) + ulp(ref) + 1e-6, f"o_proj {rows}x{hid}")


@pytest.mark.parametrize("max_m", ["64", "0"])
def test_matmul_batched_paths(max_m, monkeypatch):
    announce(f"matmul batched max_m={max_m}")
    monkeypatch.setenv("SUPERSONIC_PROJ_SKINNY_MAX_M", max_m)
    g = gen(85)
    lhs = O.randn_bf16(g, 3, 20, 512)
    rhs = O.randn_bf16(g, 3, 72, 512, std=512 ** -0.5)
    out = dropin_matmul(lhs, rhs)
    ref = O.matmul_rhs_transposed(lhs, rhs)
    assert_ulps(out, ref, ulp(ref) + 1e-6, "batched matmul")


def run_qkv(hidden, nw, wq, wk, wv, eps=1e-6):
    rows = hidden.shape[0]
    outs = [torch.full((rows, w.shape[0]), float("nan"), dtype=torch.bfloat16, device=DEV) for w in (wq, wk, wv)]
    K.qkv_proj(0, hidden.to(DEV), nw.to(DEV), wq.to(DEV), wk.to(DEV), wv.to(DEV), *outs, eps=eps)
    torch.cuda.synchronize()
    return [o.cpu() for o in outs]


@pytest.mark.parametrize("rows,hid,nq,nkv", [
    (8, 4096, 8192, 1024), (1, 2048, 8192, 512), (16, 1000, 512, 128), (3, 4096, 1024, 256),
    (40, 1024, 512, 128), (8, 512, 1000, 72),
])
@pytest.mark.parametrize("hdt", [torch.bfloat16, torch.float32])
def test_qkv_proj_matches_oracle(rows, hid, nq, nkv, hdt):
    """Fused kernel (<= 16 rows, widths % 16) and the norm + hipBLASLt path."""
    announce(f"qkv_proj rows={rows} hidden={hid} q={nq} kv={nkv} hidden dtype {hdt}")
    g = gen(86)
    hidden = O.randn_bf16(g, rows, hid).to(hdt)
    nw = O.randn_bf16(g, hid, std=0.1)
    wq, wk, wv = (O.randn_bf16(g, n, hid, std=hid ** -0.5) for n in (nq, nkv, nkv))
    outs = run_qkv(hidden, nw, wq, wk, wv)
    refs = O.qkv_proj(hidden.float(), nw, wq, wk, wv)
    for name, out, ref in zip("qkv", outs, refs):
        # the normed row may round differently by one bf16 ulp in a few places
        # (hardware rsqrt), which moves a projection by far less than its ulp
        assert_ulps(out, ref, 2 * ulp(ref) + 2.0 ** -10, f"qkv {name}")
        assert (out.float() == ref).float().mean().item() > 0.9, name


@pytest.mark.parametrize("caller_ws", [False, True])
def test_qkv_proj_gemm_tail_split(caller_ws):
    """A prefill-sized Q/K/V: 640 GEMM tiles, the last 128 split along k, with
    the library's workspace or the caller's (zero-filled once, reused)."""
    rows, hid, nq, nkv = 4096, 1024, 8192, 1024
    announce(f"qkv_proj tail split rows={rows} caller workspace {caller_ws}")
    g = gen(87)
    hidden = O.randn_bf16(g, rows, hid)
    nw = O.randn_bf16(g, hid, std=0.1)
    wq, wk, wv = (O.randn_bf16(g, n, hid, std=hid ** -0.5) for n in (nq, nkv, nkv))
    ws = None
    if caller_ws:
        ws = torch.zeros(K.qkv_proj_workspace_size(rows, hid, nq, nkv), dtype=torch.uint8, device=DEV)
    refs = O.qkv_proj(hidden.float(), nw, wq, wk, wv)
    for _ in range(2):
        outs = [torch.full((rows, w.shape[0]), float("nan"), dtype=torch.bfloat16, device=DEV) for w in (wq, wk, wv)]
        K.qkv_proj(0, hidden.to(DEV), nw.to(DEV), wq.to(DEV), wk.to(DEV), wv.to(DEV), *outs, workspace=ws)
        torch.cuda.synchronize()
        for name, out, ref in zip("qkv", outs, refs):
            out = out.cpu()
            # two roundings apart (summation order, near a power of two the
            # larger binade's step), plus a normed element one bf16 ulp away
            # (hardware rsqrt): over 4096 rows some row's largest element
            # (|x| ~ 5, ulp 2^-5) flips, moving its outputs by up to
            # 2^-5 * |w| (|w| < 0.12 here), below 2^-8
            big = torch.maximum(out.float().abs(), ref.float().abs())
            assert_ulps(out, ref, 2 * ulp(big) + 2.0 ** -8, f"qkv tail split {name}")
            assert (out.float() == ref).float().mean().item() > 0.9, name


def test_decode_layer_chain():
    """qkv_proj -> fused decode -> o_proj + residual on device, against the oracle's
    chain (config-1 heads, a 4096-wide hidden state, B = 4, 300 cached tokens)."""
    announce("decode layer chain")
    g = gen(87)
    B, Hq, Hkv, D, rot, hid, L = 4, 8, 2, 256, 64, 4096, 300
    shape = O.LayerShape(Hq, Hkv, D, rot)
    hidden = O.randn_bf16(g, B, hid)
    nw = O.randn_bf16(g, hid, std=0.1)
    wq, wk, wv = (O.randn_bf16(g, n, hid, std=hid ** -0.5) for n in (Hq * 2 * D, Hkv * D, Hkv * D))
    wo = O.randn_bf16(g, hid, Hq * D, std=(Hq * D) ** -0.5)
    qw, kw = O.norm_weights(g, D)
    cos, sin = O.rope_tables(rot, L + 2, 1.0e7)
    kc = O.randn_bf16(g, B, Hkv, L + 1, D)
    vc = O.randn_bf16(g, B, Hkv, L + 1, D)
    pos = torch.tensor([L, L - 7, 100, 1], dtype=torch.int32)

    q_proj, k_new, v_new = (t.to(DEV) for t in run_qkv(hidden, nw, wq, wk, wv))
    cache = K.KvCache(kc.to(DEV), vc.to(DEV))
    attn = torch.zeros(B, Hq * D, dtype=torch.bfloat16, device=DEV)
    K.fused_decode(0, q_proj, k_new, v_new, qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV), pos.to(DEV), cache,
                   attn, q_heads=Hq, kv_heads=Hkv, head_dim=D, rotary_dim=rot, max_kv_len=L + 1)
    h = hidden.to(DEV)
    K.o_proj_residual(0, attn, wo.to(DEV), h)
    torch.cuda.synchronize()

    rq, rk, rv = O.qkv_proj(hidden, nw, wq, wk, wv)
    ra = O.decode_layer(shape, rq, rk, rv, qw, kw, cos, sin, pos.tolist(), [kc[b].clone() for b in range(B)],
                        [vc[b].clone() for b in range(B)])
    rh = O.o_proj_residual(ra, wo, hidden)
    d = (h.float().cpu() - rh).abs()
    assert d.max().item() <= 2e-2 * max(1.0, rh.abs().max().item()) and d.mean().item() <= 2e-3, \
        f"chain: max {d.max().item():.3e} mean {d.mean().item():.3e}"


def run_qkv_rope(hidden, nw, wq, wk, wv, qw, kw, cos, sin, pos, Hq, Hkv, D, rot, cache=None):
    rows = hidden.shape[0]
    mk = lambda n: torch.full((rows, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    q, gate, k, v = mk(Hq * D), mk(Hq * D), mk(Hkv * D), mk(Hkv * D)
    K.qkv_proj_rope(0, hidden.to(DEV), nw.to(DEV), wq.to(DEV), wk.to(DEV), wv.to(DEV), qw.to(DEV), kw.to(DEV),
                    cos.to(DEV), sin.to(DEV), pos.to(DEV), q, gate, k, v, q_heads=Hq, kv_heads=Hkv, head_dim=D,
                    rotary_dim=rot, cache=cache)
    torch.cuda.synchronize()
    return q.cpu(), gate.cpu(), k.cpu(), v.cpu()


@pytest.mark.parametrize("rows,hid,Hq,Hkv,D,rot", [
    (8, 4096, 16, 4, 256, 64),    # config-2 decode step: fused epilogue
    (1, 2048, 8, 2, 256, 64),     # config-1 heads
    (4, 1024, 8, 2, 128, 32),     # head_dim 128
    (16, 4096, 16, 4, 256, 64),   # rows * hidden > 32768: projections, then the norm/RoPE kernel
    (40, 1024, 8, 2, 256, 64),    # GEMM rows
    (3, 512, 4, 2, 64, 16),       # head_dim 64
])
@pytest.mark.parametrize("with_cache", [False, True])
def test_qkv_proj_rope_matches_oracle(rows, hid, Hq, Hkv, D, rot, with_cache):
    """Input norm + Q/K/V projections + per-head QK RMSNorm + partial RoPE (+ KV append)
    against the oracle's qkv_proj followed by prep_qk.  The projection may round a
    value one bf16 ulp apart from the oracle (fp32 summation order), which the norm
    and RoPE carry: q / k within 4 ulps of the result plus 2^-4 absolute (a rotated
    pair can cancel, leaving a small result off by an ulp of its ~2-4 sized inputs),
    v and gate within 2 ulps; at least 80% identical; the appended cache rows equal
    the returned k / v bit for bit."""
    announce(f"qkv_proj_rope rows={rows} hidden={hid} Hq={Hq} Hkv={Hkv} D={D} cache={with_cache}")
    g = gen(88)
    shape = O.LayerShape(Hq, Hkv, D, rot)
    hidden = O.randn_bf16(g, rows, hid)
    nw = O.randn_bf16(g, hid, std=0.1)
    wq, wk, wv = (O.randn_bf16(g, n, hid, std=hid ** -0.5) for n in (Hq * 2 * D, Hkv * D, Hkv * D))
    qw, kw = O.norm_weights(g, D)
    cos, sin = O.rope_tables(rot, 5000, 1.0e7)
    pos = torch.randint(0, 4999, (rows,), generator=g).to(torch.int32)
    cache = None
    if with_cache:
        cache = K.KvCache(torch.zeros(rows, Hkv, 5000, D, dtype=torch.bfloat16, device=DEV),
                          torch.zeros(rows, Hkv, 5000, D, dtype=torch.bfloat16, device=DEV))
    q, gate, k, v = run_qkv_rope(hidden, nw, wq, wk, wv, qw, kw, cos, sin, pos, Hq, Hkv, D, rot, cache)
    rq, rk, rv = O.qkv_proj(hidden, nw, wq, wk, wv)
    oq, og, ok = O.prep_qk(shape, rq, rk, qw, kw, cos, sin, pos.long())
    for name, out, ref, n_ulp, floor in (("q", q, oq.reshape(rows, -1), 4, 2.0 ** -4),
                                         ("k", k, ok.reshape(rows, -1), 4, 2.0 ** -4),
                                         ("gate", gate, og.reshape(rows, -1), 2, 2.0 ** -9), ("v", v, rv, 2, 2.0 ** -9)):
        assert_ulps(out, ref, n_ulp * ulp(ref) + floor, f"qkv_rope {name}")
        assert (out.float() == ref).float().mean().item() > 0.8, name
    if with_cache:
        for r in range(rows):
            p = int(pos[r])
            assert torch.equal(cache.k[r, :, p].cpu(), k[r].reshape(Hkv, D))
            assert torch.equal(cache.v[r, :, p].cpu(), v[r].reshape(Hkv, D))


def test_decode_layer_chain_fused_projection():
    """qkv_proj_rope (with the KV append) -> decode_attend (gate) -> o_proj + residual
    against the oracle's decode-layer chain (config-2 heads, hidden 4096, B = 4)."""
    announce("decode layer chain, fused projection")
    g = gen(89)
    B, Hq, Hkv, D, rot, hid, L = 4, 16, 4, 256, 64, 4096, 700
    shape = O.LayerShape(Hq, Hkv, D, rot)
    hidden = O.randn_bf16(g, B, hid)
    nw = O.randn_bf16(g, hid, std=0.1)
    wq, wk, wv = (O.randn_bf16(g, n, hid, std=hid ** -0.5) for n in (Hq * 2 * D, Hkv * D, Hkv * D))
    wo = O.randn_bf16(g, hid, Hq * D, std=(Hq * D) ** -0.5)
    qw, kw = O.norm_weights(g, D)
    cos, sin = O.rope_tables(rot, L + 2, 1.0e7)
    kc = O.randn_bf16(g, B, Hkv, L + 1, D)
    vc = O.randn_bf16(g, B, Hkv, L + 1, D)
    pos = torch.tensor([L, L - 9, 250, 0], dtype=torch.int32)
    cache = K.KvCache(kc.to(DEV), vc.to(DEV))
    q, gate, _, _ = (t.to(DEV) for t in run_qkv_rope(hidden, nw, wq, wk, wv, qw, kw, cos, sin, pos, Hq, Hkv, D, rot,
                                                      cache))
    attn = torch.zeros(B, Hq * D, dtype=torch.bfloat16, device=DEV)
    K.decode_attend(0, q.reshape(B, Hq, D), (pos + 1).to(DEV), cache, attn, q_heads=Hq, kv_heads=Hkv, head_dim=D,
                    max_kv_len=L + 1, gate=gate)
    h = hidden.to(DEV)
    K.o_proj_residual(0, attn, wo.to(DEV), h)
    torch.cuda.synchronize()
    rq, rk, rv = O.qkv_proj(hidden, nw, wq, wk, wv)
    ra = O.decode_layer(shape, rq, rk, rv, qw, kw, cos, sin, pos.tolist(), [kc[b].clone() for b in range(B)],
                        [vc[b].clone() for b in range(B)])
    check_a = (attn.float().cpu() - ra).abs()
    assert check_a.max().item() <= 2e-2 and check_a.mean().item() <= 2e-3, f"attn {check_a.max().item():.3e}"
    rh = O.o_proj_residual(ra, wo, hidden)
    d = (h.float().cpu() - rh).abs()
    assert d.max().item() <= 2e-2 * max(1.0, rh.abs().max().item()) and d.mean().item() <= 2e-3, \
        f"chain: max {d.max().item():.3e} mean {d.mean().item():.3e}"


def test_gemm_tail_expired_handover_is_reported(monkeypatch):
    """The host presets one tail tile's consumed count ahead of its produced count,
    so that tile's second k half never sees its first half, and shortens the
    poll bound: the wait gives up, the kernel exits normally and the error word
    reports it.  A normal call on the re-zeroed workspace is then correct,
    reports nothing and leaves every tile's two counts equal."""
    rows, hid, nq, nkv = 4096, 1024, 8192, 1024
    g = gen(88)
    hidden = O.randn_bf16(g, rows, hid)
    nw = O.randn_bf16(g, hid, std=0.1)
    wq, wk, wv = (O.randn_bf16(g, n, hid, std=hid ** -0.5) for n in (nq, nkv, nkv))
    args = [t.to(DEV) for t in (hidden, nw, wq, wk, wv)]
    ws = torch.zeros(K.qkv_proj_workspace_size(rows, hid, nq, nkv), dtype=torch.uint8, device=DEV)
    counts = ws[rows * hid * 2:rows * hid * 2 + 8192].view(torch.int32)  # the GEMM's region follows the normed rows
    outs = [torch.empty((rows, w.shape[0]), dtype=torch.bfloat16, device=DEV) for w in (wq, wk, wv)]
    assert K.wait_status() == 0
    counts[1] = 1  # tile 0: consumed 1, produced 0
    monkeypatch.setenv("SUPERSONIC_WAIT_POLLS", "16")
    announce("qkv_proj tail hand-over held (forced give-up)")
    K.qkv_proj(0, *args, *outs, workspace=ws)
    assert K.wait_status() & K.WAIT_GEMM_TAIL
    monkeypatch.delenv("SUPERSONIC_WAIT_POLLS")
    ws.zero_()
    announce("qkv_proj after the forced give-up")
    K.qkv_proj(0, *args, *outs, workspace=ws)
    assert K.wait_status() == 0
    c = counts.cpu().view(-1, 2)
    assert bool((c[:, 0] == c[:, 1]).all()) and int(c[:, 0].max()) == 1
    refs = O.qkv_proj(hidden.float(), nw, wq, wk, wv)
    for name, out, ref in zip("qkv", outs, refs):
        out = out.cpu()
        big = torch.maximum(out.float().abs(), ref.float().abs())
        assert_ulps(out, ref, 2 * ulp(big) + 2.0 ** -8, f"qkv after give-up {name}")
