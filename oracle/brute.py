"""Float64 brute force for tiny shapes.  TEST INFRASTRUCTURE ONLY.

An independent implementation (plain python loops over numpy float64 scalars,
no torch) used to pin ``attn_oracle``: a dropped term, a wrong sign, a
transposed operand or an off-by-one in the causal limit in either one shows up
as a mismatch.  Runs in well under a second for the shapes the tests use.
"""
from __future__ import annotations

import math

import numpy as np


def bf16_round(x) -> np.ndarray:
    """Round float32 values to bf16, ties to even, by bit manipulation."""
    a = np.asarray(x, dtype=np.float32)
    bits = a.view(np.uint32).astype(np.uint64)
    bias = 0x7FFF + ((bits >> 16) & 1)
    out = ((bits + bias) & 0xFFFF0000).astype(np.uint32)
    return out.view(np.float32)


def rope_tables(rotary_dim: int, max_pos: int, theta: float):
    half = rotary_dim // 2
    cos = np.zeros((max_pos, half), np.float32)
    sin = np.zeros((max_pos, half), np.float32)
    for p in range(max_pos):
        for i in range(half):
            ang = p * (1.0 / theta ** (2.0 * i / rotary_dim))
            cos[p, i] = math.cos(ang)
            sin[p, i] = math.sin(ang)
    return bf16_round(cos), bf16_round(sin)


def rms_norm_row(x, w, eps, unit_offset=True):
    x = [float(t) for t in x]
    ms = sum(t * t for t in x) / len(x)
    inv = 1.0 / math.sqrt(ms + eps)
    return [x[i] * inv * (float(w[i]) + (1.0 if unit_offset else 0.0)) for i in range(len(x))]


def rope_row(x, cos_row, sin_row, rotary_dim):
    half = rotary_dim // 2
    y = list(map(float, x))
    for i in range(half):
        a, b = float(x[i]), float(x[i + half])
        y[i] = a * float(cos_row[i]) - b * float(sin_row[i])
        y[i + half] = b * float(cos_row[i]) + a * float(sin_row[i])
    return y


def attend(qrow, keys, vals, scale):
    """softmax(q.k * scale) @ v over the given key rows, two-pass, float64."""
    if len(keys) == 0:
        return [0.0] * len(qrow)
    scores = [sum(float(a) * float(b) for a, b in zip(qrow, k)) * scale for k in keys]
    m = max(scores)
    w = [math.exp(s - m) for s in scores]
    z = sum(w)
    D = len(vals[0])
    return [sum(w[t] * float(vals[t][d]) for t in range(len(keys))) / z for d in range(D)]


def prefill(q, k, v, scale, seqlen_offset):
    """q [B,Hq,S,D], k/v [B,Hkv,L,D] -> [B,Hq,S,D] float64 (causal)."""
    B, Hq, S, D = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Hq, S, D))
    for b in range(B):
        for h in range(Hq):
            hk = h // G
            for p in range(S):
                n = min(L, seqlen_offset + p + 1)
                out[b, h, p] = attend(q[b, h, p], k[b, hk, :n], v[b, hk, :n], scale)
    return out


def decode(q, k, v, lens, scale):
    """q [B,Hq,D], k/v [B,Hkv,T,D], per-sequence lengths -> [B,Hq,D] float64."""
    B, Hq, D = q.shape
    G = Hq // k.shape[1]
    out = np.zeros((B, Hq, D))
    for b in range(B):
        for h in range(Hq):
            n = int(lens[b])
            out[b, h] = attend(q[b, h], k[b, h // G, :n], v[b, h // G, :n], scale)
    return out


def sigmoid(x):
    return 1.0 / (1.0 + math.exp(-x))
