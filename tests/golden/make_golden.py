"""Write the committed golden fixtures under tests/golden/.

Expected values come from ``oracle.brute`` (float64 loops, independent of the
torch oracle) and from the reference's own known-answer tests, restated as data:

* ``rmsnorm_known_answer.json``: crates/kernel-ffi/src/prefill_ffi.rs:3253-3291
  (input [3, 4], weight [0.5, -0.5], eps 0, unit offset, tolerance 0.02).
* ``config_known_answer.json``: crates/qwen35/src/config.rs:201-259 (head_dim
  256, partial_rotary_factor 0.25 -> rotary_dim 64, rope_theta 1e7, 16 full
  attention layers x 4 kv heads -> kv_bytes_per_token(2) = 65536).
* ``proj_known_answer.json``: crates/kernel-ffi/src/metal_native.rs:4307-4338
  (matmul_rhs_transposed), :4430-4469 (matmul + residual), :5807-5827
  (element_add, bf16), plus a float64 brute-force o_proj + residual case and a
  case whose answer depends on the reference's two roundings.

Inputs are seeded bf16 values (stored as float lists; every value is exact).
Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import brute  # noqa: E402


def bf16_randn(rng, *shape, std=1.0, mean=0.0):
    return brute.bf16_round((rng.standard_normal(shape) * std + mean).astype(np.float32))


def dump(name, obj):
    with open(os.path.join(HERE, name), "w") as f:
        json.dump(obj, f, separators=(",", ":"))


def tolist(a):
    return np.asarray(a, dtype=np.float64).ravel().tolist()


def main():
    rng = np.random.default_rng(20260101)

    dump("rmsnorm_known_answer.json", {
        "source": "crates/kernel-ffi/src/prefill_ffi.rs:3253-3291",
        "input": [3.0, 4.0], "weight": [0.5, -0.5], "eps": 0.0, "add_unit_offset": True,
        "expected": [3.0 / math.sqrt(12.5) * 1.5, 4.0 / math.sqrt(12.5) * 0.5],
        "tolerance": 0.02,
    })

    dump("config_known_answer.json", {
        "source": "crates/qwen35/src/config.rs:201-259",
        "head_dim": 256, "partial_rotary_factor": 0.25, "rotary_dim": 64,
        "rope_theta": 1.0e7, "num_full_attention_layers": 16, "num_key_value_heads": 4,
        "kv_bytes_per_token_bf16": 65536,
    })

    # Causal prefill with a cached prefix (seqlen_offset 3) and GQA 4:2.
    B, Hq, Hkv, S, D, off = 1, 4, 2, 6, 64, 3
    L = off + S
    q = bf16_randn(rng, B, Hq, S, D)
    k = bf16_randn(rng, B, Hkv, L, D)
    v = bf16_randn(rng, B, Hkv, L, D)
    scale = 1.0 / math.sqrt(D)
    out = brute.prefill(q, k, v, scale, off)
    dump("prefill_tiny.json", {
        "B": B, "Hq": Hq, "Hkv": Hkv, "S": S, "L": L, "D": D, "seqlen_offset": off, "scale": scale,
        "q": tolist(q), "k": tolist(k), "v": tolist(v), "out": tolist(out),
    })

    # Prefill where kv_len < seqlen_offset + S: the causal limit clamps to kv_len.
    B, Hq, Hkv, S, D, off, L = 1, 2, 1, 5, 64, 4, 6
    q = bf16_randn(rng, B, Hq, S, D)
    k = bf16_randn(rng, B, Hkv, L, D)
    v = bf16_randn(rng, B, Hkv, L, D)
    out = brute.prefill(q, k, v, 1.0 / math.sqrt(D), off)
    dump("prefill_clamped.json", {
        "B": B, "Hq": Hq, "Hkv": Hkv, "S": S, "L": L, "D": D, "seqlen_offset": off,
        "scale": 1.0 / math.sqrt(D),
        "q": tolist(q), "k": tolist(k), "v": tolist(v), "out": tolist(out),
    })

    # Ragged decode, G = 4, two sequences in a cache of capacity 16.
    B, Hq, Hkv, T, D = 2, 8, 2, 16, 64
    lens = [16, 5]
    q = bf16_randn(rng, B, Hq, D)
    k = bf16_randn(rng, B, Hkv, T, D)
    v = bf16_randn(rng, B, Hkv, T, D)
    out = brute.decode(q, k, v, lens, 1.0 / math.sqrt(D))
    dump("decode_tiny.json", {
        "B": B, "Hq": Hq, "Hkv": Hkv, "T": T, "D": D, "lens": lens, "scale": 1.0 / math.sqrt(D),
        "q": tolist(q), "k": tolist(k), "v": tolist(v), "out": tolist(out),
    })

    # One fused decode step (norm -> RoPE -> append -> attention -> gate), bf16 cache.
    Hq, Hkv, D, rot, theta, pos, eps = 4, 1, 64, 16, 1.0e7, 7, 1e-6
    q_proj = bf16_randn(rng, Hq * 2 * D)
    k_raw = bf16_randn(rng, Hkv * D)
    v_raw = bf16_randn(rng, Hkv * D)
    qw = bf16_randn(rng, D, std=0.02, mean=1.0)
    kw = bf16_randn(rng, D, std=0.02, mean=1.0)
    cache_k = bf16_randn(rng, Hkv, pos, D)
    cache_v = bf16_randn(rng, Hkv, pos, D)
    cos, sin = brute.rope_tables(rot, pos + 1, theta)
    qh = [brute.bf16_round(np.array(brute.rope_row(
        brute.bf16_round(np.array(brute.rms_norm_row(q_proj[h * 2 * D:h * 2 * D + D], qw, eps), np.float32)),
        cos[pos], sin[pos], rot), np.float32)) for h in range(Hq)]
    gate = [q_proj[h * 2 * D + D:(h + 1) * 2 * D] for h in range(Hq)]
    kh = [brute.bf16_round(np.array(brute.rope_row(
        brute.bf16_round(np.array(brute.rms_norm_row(k_raw[h * D:(h + 1) * D], kw, eps), np.float32)),
        cos[pos], sin[pos], rot), np.float32)) for h in range(Hkv)]
    vh = [v_raw[h * D:(h + 1) * D] for h in range(Hkv)]
    out = []
    G = Hq // Hkv
    for h in range(Hq):
        keys = list(cache_k[h // G]) + [kh[h // G]]
        vals = list(cache_v[h // G]) + [vh[h // G]]
        a = brute.bf16_round(np.array(brute.attend(qh[h], keys, vals, 1.0 / math.sqrt(D)), np.float32))
        out.extend(brute.bf16_round(np.array(
            [a[d] * brute.sigmoid(float(gate[h][d])) for d in range(D)], np.float32)).tolist())
    dump("fused_decode_tiny.json", {
        "Hq": Hq, "Hkv": Hkv, "D": D, "rotary_dim": rot, "theta": theta, "pos": pos, "eps": eps,
        "q_proj": tolist(q_proj), "k_raw": tolist(k_raw), "v_raw": tolist(v_raw),
        "q_norm_w": tolist(qw), "k_norm_w": tolist(kw),
        "cache_k": tolist(cache_k), "cache_v": tolist(cache_v),
        "k_rot_expected": tolist(np.array(kh)), "out": out,
    })

    # Output projection + residual (o_proj row after the gate).
    kat_lhs = [[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]]
    kat_rhs = [[1.0, 0.0, 1.0], [0.5, -1.0, 2.0]]
    m, n, k = 3, 5, 40
    attn = bf16_randn(rng, m, k)
    w = bf16_randn(rng, n, k, std=0.2)
    hid = bf16_randn(rng, m, n)
    dot = attn.astype(np.float64) @ w.astype(np.float64).T
    add = brute.bf16_round(dot.astype(np.float32))
    res = brute.bf16_round((hid.astype(np.float32) + add).astype(np.float32))
    dump("proj_known_answer.json", {
        "matmul": {"source": "crates/kernel-ffi/src/metal_native.rs:4307-4338", "lhs": kat_lhs, "rhs": kat_rhs,
                   "expected": [[4.0, 4.5], [10.0, 9.0]], "tolerance": 0.02},
        "matmul_residual": {"source": "crates/kernel-ffi/src/metal_native.rs:4430-4469", "lhs": kat_lhs,
                            "rhs": kat_rhs, "residual": [[0.25, -0.5], [1.0, 2.0]],
                            "expected": [[4.25, 4.0], [11.0, 11.0]], "tolerance": 0.02},
        "element_add": {"source": "crates/kernel-ffi/src/metal_native.rs:5807-5827",
                        "lhs": [1.0, -2.0, 0.5, 10.0], "rhs": [0.25, 3.0, -0.25, -1.5],
                        "expected": [1.25, 1.0, 0.25, 8.5], "tolerance": 0.02},
        # hidden 1 + bf16(2^-8 + 2^-20) = 1 + 2^-8, a tie that rounds to even (1.0);
        # a single rounding of 1 + 2^-8 + 2^-20 would give 1 + 2^-7.
        "double_rounding": {"attn": [[2.0 ** -8, 2.0 ** -20]], "w": [[1.0, 1.0]], "hidden": [[1.0]],
                            "expected": [[1.0]], "single_rounding": [[1.0 + 2.0 ** -7]]},
        "brute": {"attn": tolist(attn), "w": tolist(w), "hidden": tolist(hid), "m": m, "n": n, "k": k,
                  "expected": tolist(res)},
    })


if __name__ == "__main__":
    main()
