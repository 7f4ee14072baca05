"""The o_proj + residual oracle against the reference's known answers, float64
brute force and the rounding sequence of the megakernel's step G."""
import json
import os

import numpy as np
import torch

from oracle import attn_oracle as O
from oracle import brute

GOLD = os.path.join(os.path.dirname(__file__), "golden")
G = json.load(open(os.path.join(GOLD, "proj_known_answer.json")))


def t(x):
    return torch.tensor(x, dtype=torch.float32)


def test_matmul_known_answer():
    g = G["matmul"]
    out = O.matmul_rhs_transposed(t(g["lhs"]), t(g["rhs"]))
    assert np.allclose(out.numpy(), g["expected"], atol=g["tolerance"])


def test_matmul_residual_known_answer():
    g = G["matmul_residual"]
    out = O.o_proj_residual(t(g["lhs"]), t(g["rhs"]), t(g["residual"]))
    assert np.allclose(out.numpy(), g["expected"], atol=g["tolerance"])


def test_element_add_known_answer():
    g = G["element_add"]
    assert np.allclose(O.element_add(t(g["lhs"]), t(g["rhs"])).numpy(), g["expected"], atol=g["tolerance"])


def test_two_roundings():
    """The residual is added to the bf16-rounded projection, not to the fp32 sum."""
    g = G["double_rounding"]
    out = O.o_proj_residual(t(g["attn"]), t(g["w"]), t(g["hidden"]))
    assert out.item() == g["expected"][0][0]
    single = O.bf16r(t(g["hidden"]) + t(g["attn"]) @ t(g["w"]).T)
    assert single.item() == g["single_rounding"][0][0]


def test_brute_force_case():
    g = G["brute"]
    m, n, k = g["m"], g["n"], g["k"]
    out = O.o_proj_residual(t(g["attn"]).reshape(m, k), t(g["w"]).reshape(n, k), t(g["hidden"]).reshape(m, n))
    exp = np.array(g["expected"], dtype=np.float32).reshape(m, n)
    # fp32 accumulation order may move a bf16 result by one ulp against the float64 sum
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exp), 1e-30))) - 7)
    assert np.all(np.abs(out.numpy() - exp) <= ulp)
    assert np.mean(out.numpy() == exp) > 0.9


def test_matmul_batched_rhs_and_brute():
    """Batch b pairs lhs[b] with rhs[b]; each entry is the rounded float64 dot."""
    gen = torch.Generator().manual_seed(5)
    lhs = O.randn_bf16(gen, 2, 3, 24)
    rhs = O.randn_bf16(gen, 2, 4, 24)
    out = O.matmul_rhs_transposed(lhs, rhs)
    for b in range(2):
        dot = lhs[b].double().numpy() @ rhs[b].double().numpy().T
        exp = brute.bf16_round(dot.astype(np.float32))
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exp), 1e-30))) - 7)
        assert np.all(np.abs(out[b].numpy() - exp) <= ulp)
    assert not torch.equal(out[1], O.matmul_rhs_transposed(lhs[1:], rhs[:1])[0])


def test_qkv_proj_against_brute_force():
    """Input norm (1 + w) then three projections, each entry the float64 dot of
    the bf16-rounded normed row (brute.rms_norm_row restates the norm in float64)."""
    gen = torch.Generator().manual_seed(6)
    hid = O.randn_bf16(gen, 2, 64)
    nw = O.randn_bf16(gen, 64, std=0.1)
    wq, wk, wv = (O.randn_bf16(gen, n, 64, std=0.125) for n in (32, 16, 16))
    q, k, v = O.qkv_proj(hid, nw, wq, wk, wv, 1e-6)
    for r in range(2):
        normed = brute.bf16_round(np.array(brute.rms_norm_row(hid[r].float().numpy(), nw.float().numpy(), 1e-6), np.float32))
        for got, w in ((q, wq), (k, wk), (v, wv)):
            exp = brute.bf16_round((w.double().numpy() @ normed.astype(np.float64)).astype(np.float32))
            ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exp), 1e-30))) - 7)
            assert np.all(np.abs(got[r].numpy() - exp) <= ulp)
