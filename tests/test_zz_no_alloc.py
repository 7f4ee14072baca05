"""The allocation-free decode entry point (supersonic_attn_gfx950_decode_noalloc)
against supersonic_attn_gfx950_decode on the same inputs, through the C ABI:
two calls in a row on one GPU, the second with a smaller batch and shorter
contexts (its split counters and partials reuse the same device scratch array).

Bar: both outputs against the CPU oracle within the BF16 tolerance (max-abs
2e-2, mean-abs 2e-3), each other within two bf16 ulps plus 2^-8 (the split
waves claim blocks dynamically, so fp32 summation order differs between any
two runs), appended V rows bit-exact; a shape whose partials exceed the
8 MiB scratch array is rejected with SUPERSONIC_ERR_WORKSPACE."""
import pytest
import torch

from gpu_util import DEV, TOL_BF16, announce, check, dev, make_decode_case, oracle_decode
from supersonic_amd import kernel_ffi as K

pytestmark = pytest.mark.gpu


def run(case, noalloc):
    B = case["q_proj"].shape[0]
    sh = case["shape"]
    cache = K.KvCache(dev(case["k"]), dev(case["v"]))
    out = torch.full((B, sh.q_heads * sh.head_dim), float("nan"), dtype=torch.bfloat16, device=DEV)
    fn = K.fused_decode_noalloc if noalloc else K.fused_decode
    fn(0, dev(case["q_proj"]), dev(case["k_new"]), dev(case["v_new"]), dev(case["qw"]), dev(case["kw"]),
       dev(case["cos"]), dev(case["sin"]), dev(case["pos"]), cache, out, q_heads=sh.q_heads,
       kv_heads=sh.kv_heads, head_dim=sh.head_dim, rotary_dim=sh.rotary_dim,
       max_kv_len=int(case["pos"].max()) + 1)
    torch.cuda.synchronize()
    return out, cache


def close_ulps(x, y, floor=2.0 ** -8):
    x, y = x.float().cpu(), y.float().cpu()
    ulp = torch.exp2(torch.floor(torch.log2(y.abs().clamp_min(2.0 ** -100))) - 7)
    return bool(((x - y).abs() <= 2 * ulp + floor).all())


def test_noalloc_decode_matches_decode_twice():
    for i, (B, lens) in enumerate([(8, [32768, 100, 5000, 17, 32000, 2048, 0, 777]), (2, [1500, 64])]):
        announce(f"noalloc decode call {i}: B={B} lens={lens}")
        case = make_decode_case(120 + i, B, 16, 4, 256, 64, lens)
        ref, _, v_ref, _, _ = oracle_decode(case)
        out_n, cache_n = run(case, True)
        out_w, _ = run(case, False)
        check(out_n, ref, TOL_BF16, f"noalloc call {i}")
        check(out_w, ref, TOL_BF16, f"decode call {i}")
        assert close_ulps(out_n, out_w), f"call {i}: noalloc and decode differ beyond summation order"
        for b, p in enumerate(lens):
            assert torch.equal(cache_n.v[b, :, p].cpu(), v_ref[b, :, p])


def test_noalloc_rejects_shapes_beyond_scratch():
    lib = K.load()
    z = torch.zeros(64, device=DEV)
    p = z.data_ptr()
    desc = K.KvCacheDesc()
    desc.k = desc.v = p
    # 4096 sequences x 64 heads: the partials need far more than 8 MiB
    rc = lib.supersonic_attn_gfx950_decode_noalloc(0, None, 2, 4096, 64, 4, 256, 64, 65536, 1e-6, 0.0625,
                                                   p, p, p, p, p, p, p, p, K.C.byref(desc), p)
    assert rc == K.ERR["WORKSPACE"]
