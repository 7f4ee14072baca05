"""Shared helpers of the GPU parity tests (inputs, tolerance checks)."""
import math
import os
import sys

import numpy as np
import torch

from oracle import attn_oracle as O
from oracle import fp8_codec

DEV = "cuda:0"

# BF16 KV tolerances vs the fp32 oracle (max-abs, mean-abs).
TOL_BF16 = (2e-2, 2e-3)
# FP8 KV: the GPU scales the score (K) and p (V) instead of rounding the
# dequantised element to bf16 first, so each cached element differs from the
# oracle's bf16(lut * scale) by up to half a bf16 ulp; stated looser bound.
TOL_FP8 = (4e-2, 4e-3)


def gen(seed):
    return torch.Generator().manual_seed(seed)


def announce(msg):
    print(f"[gpu-test] {msg}", flush=True)
    sys.stdout.flush()


def check(out, ref, tol=TOL_BF16, name=""):
    d = (out.detach().float().cpu() - ref.float()).abs()
    mx, mean = d.max().item(), d.mean().item()
    assert mx <= tol[0] and mean <= tol[1], f"{name}: max-abs {mx:.3e} (<= {tol[0]}), mean-abs {mean:.3e} (<= {tol[1]})"
    return mx, mean


def fp8_rows(x: torch.Tensor, codec="ocp"):
    """Quantise float rows [..., D] -> (uint8 codes, f32 scales) as torch tensors."""
    c, s = fp8_codec.quantize_rows(x.float().numpy(), codec)
    return torch.from_numpy(c), torch.from_numpy(s)


def make_decode_case(seed, B, Hq, Hkv, D, rot, lens, cap=None, fp8=False, theta=1.0e7):
    """Seeded inputs of one fused decode step; lens[b] = cached tokens (= position)."""
    g = gen(seed)
    cap = cap or (max(lens) + 1)
    q_proj = O.randn_bf16(g, B, Hq * 2 * D)
    k_new = O.randn_bf16(g, B, Hkv * D)
    v_new = O.randn_bf16(g, B, Hkv * D)
    qw, kw = O.norm_weights(g, D)
    cos, sin = O.rope_tables(rot, cap + 1, theta)
    kc = O.randn_bf16(g, B, Hkv, cap, D)
    vc = O.randn_bf16(g, B, Hkv, cap, D)
    case = dict(q_proj=q_proj, k_new=k_new, v_new=v_new, qw=qw, kw=kw, cos=cos, sin=sin,
                pos=torch.tensor(lens, dtype=torch.int32), shape=O.LayerShape(Hq, Hkv, D, rot))
    if fp8:
        kq, ks = fp8_rows(kc)
        vq, vs = fp8_rows(vc)
        case.update(k=kq, v=vq, ks=ks, vs=vs)
    else:
        case.update(k=kc, v=vc, ks=None, vs=None)
    return case


def oracle_decode(case, codec="ocp"):
    """Run the oracle on CPU copies; returns (out [B, Hq*D], caches after the step)."""
    B = case["q_proj"].shape[0]
    k = case["k"].clone()
    v = case["v"].clone()
    ks = None if case["ks"] is None else case["ks"].clone()
    vs = None if case["vs"] is None else case["vs"].clone()
    out = O.decode_layer(case["shape"], case["q_proj"], case["k_new"], case["v_new"], case["qw"], case["kw"],
                         case["cos"], case["sin"], case["pos"].long(), [k[b] for b in range(B)],
                         [v[b] for b in range(B)],
                         None if ks is None else [ks[b] for b in range(B)],
                         None if vs is None else [vs[b] for b in range(B)], codec=codec)
    return out, k, v, ks, vs


def dev(t):
    return None if t is None else t.to(DEV)
