"""Benchmark of the gfx950 full-attention hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--skip-extra]

Headline (``value``): BASELINE config 2, the Qwen3.5-9B decode attention at
32k context, batch 8: one *step* is one ``supersonic_attn_gfx950_decode`` call
(QK RMSNorm + partial RoPE + KV append + split-K attention + LSE merge +
sigmoid gate) for all 8 sequences.  ``value`` is algorithmic bytes per step
(K+V of 32768 cached tokens per sequence, plus q, gate and out) / measured
time per step, in GB/s.  Inputs are synthetic N(0,1)
tensors resident in HBM before the timed region; the KV caches (1.07 GB) are
larger than the 256 MB last-level cache, so every step streams HBM.

``roofline`` is for the dominant kernel (``decode_split_kernel``), timed live
with HIP events recorded on its launch stream around each launch.
``cpu_baseline`` is the repo's torch fp32 oracle timed on this host for the
same workload.  ``extra`` holds the other BASELINE configs (config 1 decode, config 2 B=1,
causal prefill at 4096 tokens, FP8-KV ragged decode, mixed paged batch).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_JSON = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")


def measured_traffic(workload: str):
    """HBM bytes per launch of the workload's dominant kernel, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes (calibrated against a
    plain copy; profiles/hbm_traffic_pmc.md holds the commands), or
    None when no measurement is on file."""
    try:
        with open(TRAFFIC_JSON) as f:
            return json.load(f).get(workload, {}).get("traffic_bytes")
    except (OSError, ValueError):
        return None
MALL_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-extra", action="store_true")
    ap.add_argument("--only", default="", help="run one workload: decode8|decode_cfg1|decode1|prefill|prefill_fp8|fp8|mixed|qkv|qkv_rope|oproj|layer_graph|copy|read")
    return ap.parse_args()


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", args.gpus))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: the attention hot path is "
                                   "single-GPU; "
                                   f"got --gpus {args.gpus}"}))
        sys.exit(2)

    import torch
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from supersonic_amd import kernel_ffi as K
    K.load()
    torch.cuda.init()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    W = Workloads(torch, K, dev, args.steps, args.warmup)
    if args.only:
        r = getattr(W, args.only)()
        print(json.dumps(r, indent=None))
        return

    head = W.decode8()
    out = {
        "metric": "decode attn GB/s (% of 8 TB/s HBM); prefill attn TFLOPS (% MFMA peak)",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "BASELINE config 2: Qwen3.5-9B decode attention, fused QK-norm/RoPE/KV-append/"
                        "split-K/gate, bf16 KV cache",
            "batch": 8, "q_heads": 16, "kv_heads": 4, "head_dim": 256, "rotary_dim": 64,
            "kv_len": 32768, "bytes_per_step": head["bytes"],
        },
        "roofline": head["roofline"],
    }
    if not args.skip_cpu:
        out["cpu_baseline"] = W.cpu_decode8()
    if not args.skip_extra:
        out["extra"] = {k: getattr(W, k)() for k in ("decode_cfg1", "decode1", "prefill", "prefill_fp8", "fp8", "mixed",
                                                          "qkv", "qkv_rope", "oproj", "proj_gemm", "prefill_layer", "layer_graph",
                                                          "read")}
    print(json.dumps(out))


class Workloads:
    def __init__(self, torch, K, dev, steps, warmup):
        self.torch, self.K, self.dev = torch, K, dev
        self.steps, self.warmup = steps, warmup

    # ------------------------------------------------------------ helpers
    def randn(self, *shape, dtype=None, seed=0):
        torch = self.torch
        g = torch.Generator(device=self.dev).manual_seed(seed)
        return torch.randn(*shape, generator=g, device=self.dev, dtype=torch.float32).to(dtype or torch.bfloat16)

    def events(self, n):
        torch = self.torch
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
        for e in evs:
            e.record()  # creates the underlying hipEvent_t
        torch.cuda.synchronize()
        return evs

    def timed(self, step, n_copies=1, warmup=None):
        """Run warmup + steps of `step(i)`; returns whole-step ms and the
        dominant kernel's mean ms.  The whole-step time comes from `steps` steps
        with nothing but the workload between two events; the kernel time from
        another `steps` steps with an event pair armed around the kernel (the
        event records add about 10 us between kernels, so they stay out of the
        whole-step timing)."""
        torch, K = self.torch, self.K
        for i in range(self.warmup if warmup is None else max(warmup, self.warmup)):
            step(i % n_copies)
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for i in range(self.steps):
            step(i % n_copies)
        t1.record()
        torch.cuda.synchronize()
        step_ms = t0.elapsed_time(t1) / self.steps
        kb = self.events(self.steps)
        ka = self.events(self.steps)
        for i in range(self.steps):
            K.set_profile_events(kb[i], ka[i])
            step(i % n_copies)
        torch.cuda.synchronize()
        K.set_profile_events(None, None)
        kern = [kb[i].elapsed_time(ka[i]) for i in range(self.steps)]
        return step_ms, statistics.mean(kern), kern

    @staticmethod
    def decode_bytes(lens, Hq, Hkv, D, kv_esz, scale_bytes=0):
        kv = sum(lens) * Hkv * (D * kv_esz + scale_bytes) * 2
        qgo = len(lens) * (Hq * 2 * D * 2 + Hq * D * 2)
        return kv, kv + qgo

    def make_decode(self, B, lens, Hq, Hkv, D, rot, fp8=False, cap=None, seed=1, paged_ps=None):
        torch, K = self.torch, self.K
        cap = cap or (max(lens) + 1)
        q_proj = self.randn(B, Hq * 2 * D, seed=seed)
        k_new = self.randn(B, Hkv * D, seed=seed + 1)
        v_new = self.randn(B, Hkv * D, seed=seed + 2)
        qw = (self.randn(D, seed=seed + 3).float() * 0.02 + 1).bfloat16()
        kw = (self.randn(D, seed=seed + 4).float() * 0.02 + 1).bfloat16()
        cos, sin = K.rope_tables(rot, cap + 1, 1.0e7)
        pos = torch.tensor(lens, dtype=torch.int32, device=self.dev)
        per_cache = B * Hkv * cap * D * (1 if fp8 else 2) * 2
        n_copies = max(1, min(8, math.ceil(2 * MALL_BYTES / per_cache)))
        caches = []
        for c in range(n_copies):
            if paged_ps:
                pages_per = cap // paged_ps
                shape = (B * pages_per, Hkv, paged_ps, D)
                bt = torch.randperm(B * pages_per, device=self.dev).to(torch.int32).reshape(B, pages_per)
            else:
                shape = (B, Hkv, cap, D)
                bt = None
            kk = self.randn(*shape, seed=100 + 2 * c)
            vv = self.randn(*shape, seed=101 + 2 * c)
            if fp8:
                ks = (kk.float().abs().amax(-1) / 448).clamp(min=1e-12)
                vs = (vv.float().abs().amax(-1) / 448).clamp(min=1e-12)
                kq = (kk.float() / ks[..., None]).to(torch.float8_e4m3fn).view(torch.uint8)
                vq = (vv.float() / vs[..., None]).to(torch.float8_e4m3fn).view(torch.uint8)
                del kk, vv
                caches.append(K.KvCache(kq, vq, ks.contiguous(), vs.contiguous(), bt))
            else:
                caches.append(K.KvCache(kk, vv, block_table=bt))
        out = torch.empty(B, Hq * D, dtype=torch.bfloat16, device=self.dev)
        ws = torch.zeros(K.decode_workspace_size(B, Hq, Hkv, D, max(lens) + 1), dtype=torch.uint8, device=self.dev)
        args = dict(q_proj=q_proj, k_new=k_new, v_new=v_new, qw=qw, kw=kw, cos=cos.to(self.dev),
                    sin=sin.to(self.dev), pos=pos, out=out, ws=ws)

        def step(i):
            K.fused_decode(0, args["q_proj"], args["k_new"], args["v_new"], args["qw"], args["kw"], args["cos"],
                           args["sin"], args["pos"], caches[i], args["out"], q_heads=Hq, kv_heads=Hkv,
                           head_dim=D, rotary_dim=rot, max_kv_len=max(lens) + 1, workspace=args["ws"])
        self.last_decode = (args, caches)
        return step, n_copies

    def decode_result(self, name, B, lens, Hq, Hkv, D, rot, fp8=False, paged_ps=None, cap=None, traffic_key=None):
        step, n = self.make_decode(B, lens, Hq, Hkv, D, rot, fp8=fp8, paged_ps=paged_ps, cap=cap)
        step_ms, kern_pair_ms, _ = self.timed(step, n)
        # A step is one launch of the kernel, so its mean launch duration is the
        # back-to-back time of the steps (events only around the whole run); an
        # event pair armed around every launch adds its own ~2 us, reported as
        # kernel_ms_event_pairs.
        kern_ms = step_ms
        kv_bytes, bytes_step = self.decode_bytes(lens, Hq, Hkv, D, 1 if fp8 else 2, 4 if fp8 else 0)
        traffic = measured_traffic(traffic_key) if traffic_key else None
        # dominant kernel's algorithmic bytes: K+V (+scales) and q
        kern_bytes = kv_bytes + B * Hq * D * 2
        ach = kern_bytes / (kern_ms * 1e-3) / 1e9
        self.torch.cuda.empty_cache()
        return {
            "workload": name, "gbs": bytes_step / (step_ms * 1e-3) / 1e9, "ms_per_step": step_ms,
            "bytes": bytes_step, "kernel_ms": kern_ms, "kernel_ms_event_pairs": kern_pair_ms, "cache_copies": n,
            "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic,
                         "kernel": "decode_split_kernel", "bytes_per_launch": kern_bytes},
        }

    # ------------------------------------------------------------ workloads
    def decode8(self):
        return self.decode_result("config 2, B=8, L=32768", 8, [32768] * 8, 16, 4, 256, 64, traffic_key="decode8")

    def decode_cfg1(self):
        """Config 1: Qwen3.5-0.8B-like decode, B=1, 8/2 heads, 2048 cached tokens."""
        r = self.decode_result("config 1, B=1, Hq 8, Hkv 2, L=2048", 1, [2048], 8, 2, 256, 64, traffic_key="decode_cfg1")
        r["gbs"] = round(r["gbs"], 2)
        return r

    def decode1(self):
        r = self.decode_result("config 2, B=1, L=32768", 1, [32768], 16, 4, 256, 64, traffic_key="decode1")
        r["gbs"] = round(r["gbs"], 2)
        return r

    def fp8(self):
        torch = self.torch
        g = torch.Generator().manual_seed(4)
        lens = torch.randint(1024, 16385, (16,), generator=g).tolist()
        r = self.decode_result("config 4, FP8 e4m3 KV, B=16, L~U[1024,16384]", 16, lens, 16, 4, 256, 64,
                               fp8=True, cap=16385, traffic_key="fp8")
        r["lens_sum"] = sum(lens)
        return r

    def prefill_case(self, S, Hq, Hkv, D, rot, start=0, seed=7, paged_ps=None):
        torch, K = self.torch, self.K
        q_proj = self.randn(S, Hq * 2 * D, seed=seed)
        k_new = self.randn(S, Hkv * D, seed=seed + 1)
        v_new = self.randn(S, Hkv * D, seed=seed + 2)
        qw = (self.randn(D, seed=seed + 3).float() * 0.02 + 1).bfloat16()
        kw = (self.randn(D, seed=seed + 4).float() * 0.02 + 1).bfloat16()
        cos, sin = K.rope_tables(rot, start + S + 1, 1.0e7)
        cos, sin = cos.to(self.dev), sin.to(self.dev)
        L = start + S
        if paged_ps:
            npg = (L + paged_ps - 1) // paged_ps
            cache = K.KvCache(torch.zeros(npg, Hkv, paged_ps, D, dtype=torch.bfloat16, device=self.dev),
                              torch.zeros(npg, Hkv, paged_ps, D, dtype=torch.bfloat16, device=self.dev),
                              block_table=torch.randperm(npg, device=self.dev).to(torch.int32).reshape(1, -1))
        else:
            cache = K.KvCache(torch.zeros(1, Hkv, L, D, dtype=torch.bfloat16, device=self.dev),
                              torch.zeros(1, Hkv, L, D, dtype=torch.bfloat16, device=self.dev))
        out = torch.empty(S, Hq * D, dtype=torch.bfloat16, device=self.dev)

        def step(i):
            K.fused_prefill(0, q_proj, k_new, v_new, qw, kw, cos, sin, cache, out, q_heads=Hq, kv_heads=Hkv,
                            head_dim=D, rotary_dim=rot, chunk_start=start)
        self.last_prefill = {"q_proj": q_proj, "k_new": k_new, "v_new": v_new, "cache": cache, "out": out,
                             "chunk_start": start}
        return step

    @staticmethod
    def causal_flops(S, Hq, D, start=0):
        # QK^T + PV over the causal lower triangle including the diagonal
        keys = sum(min(start + p + 1, start + S) for p in range(S)) if start else S * (S + 1) // 2
        return 4 * Hq * D * keys

    def sdpa_reference_ms(self, S, Hq, Hkv, D):
        """torch's own causal scaled_dot_product_attention (its flash-attention
        backend on this build) on the same shape, attention only (no norm, RoPE or
        gate), median of 10: a reference point, never part of the library."""
        torch = self.torch
        q = self.randn(1, Hq, S, D, seed=70)
        k = self.randn(1, Hkv, S, D, seed=71).repeat_interleave(Hq // Hkv, 1)
        v = self.randn(1, Hkv, S, D, seed=72).repeat_interleave(Hq // Hkv, 1)
        f = lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        ts = []
        for _ in range(10):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            f()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        return statistics.median(ts)

    def prefill(self):
        S, Hq, Hkv, D, rot = 4096, 16, 4, 256, 64
        step = self.prefill_case(S, Hq, Hkv, D, rot)
        step_ms, kern_ms, _ = self.timed(step)
        fl = self.causal_flops(S, Hq, D)
        ach = fl / (kern_ms * 1e-3) / 1e12
        sdpa_ms = self.sdpa_reference_ms(S, Hq, Hkv, D)
        return {"workload": "config 3, causal prefill S=4096, 16/4 heads, D=256, fused norm/RoPE/gate",
                "tflops_step": fl / (step_ms * 1e-3) / 1e12, "ms_per_step": step_ms, "kernel_ms": kern_ms,
                "flops": fl, "torch_sdpa_ms": round(sdpa_ms, 4),
                "torch_sdpa_tflops": round(fl / (sdpa_ms * 1e-3) / 1e12, 1),
                "roofline": {"bound": "mfma", "achieved": round(ach, 1), "peak": BF16_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4),
                             "traffic": measured_traffic("prefill"), "kernel": "prefill_kernel"}}

    def prefill_layer(self):
        """One prefill chunk of a full-attention layer end to end on this
        library, config 3's shape (4096 tokens, hidden 4096, 16/4 heads of 256):
        input norm + Q/K/V (hand-written GEMM), the fused attention (QK norm,
        RoPE, cache append, causal MFMA attention, gate) and o_proj + residual
        (GEMM with the residual add in its epilogue), back to back on one
        stream; the whole chunk is timed by events."""
        torch, K = self.torch, self.K
        S, hid, Hq, Hkv, D, rot = 4096, 4096, 16, 4, 256, 64
        hidden = self.randn(S, hid, seed=60)
        nw = (self.randn(hid, seed=61) * 0.1).to(torch.bfloat16)
        wq, wk, wv = ((self.randn(n, hid, seed=62 + i) * hid ** -0.5).to(torch.bfloat16).contiguous()
                      for i, n in enumerate((Hq * 2 * D, Hkv * D, Hkv * D)))
        wo = (self.randn(hid, Hq * D, seed=65) * (Hq * D) ** -0.5).to(torch.bfloat16).contiguous()
        q_proj = torch.empty(S, Hq * 2 * D, dtype=torch.bfloat16, device=self.dev)
        k_new = torch.empty(S, Hkv * D, dtype=torch.bfloat16, device=self.dev)
        v_new = torch.empty(S, Hkv * D, dtype=torch.bfloat16, device=self.dev)
        qw = (self.randn(D, seed=66).float() * 0.02 + 1).bfloat16()
        kw = (self.randn(D, seed=67).float() * 0.02 + 1).bfloat16()
        cos, sin = (t.to(self.dev) for t in K.rope_tables(rot, S + 1, 1.0e7))
        cache = K.KvCache(torch.zeros(1, Hkv, S, D, dtype=torch.bfloat16, device=self.dev),
                          torch.zeros(1, Hkv, S, D, dtype=torch.bfloat16, device=self.dev))
        attn = torch.empty(S, Hq * D, dtype=torch.bfloat16, device=self.dev)
        h = hidden.clone()
        ws = torch.zeros(K.prefill_workspace_size(False, Hkv, D, S, 0), dtype=torch.uint8, device=self.dev)

        def step(i):
            K.qkv_proj(0, h, nw, wq, wk, wv, q_proj, k_new, v_new)
            K.fused_prefill(0, q_proj, k_new, v_new, qw, kw, cos, sin, cache, attn, q_heads=Hq, kv_heads=Hkv,
                            head_dim=D, rotary_dim=rot, chunk_start=0, workspace=ws)
            K.o_proj_residual(0, attn, wo, h)
        for _ in range(self.warmup):
            step(0)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(self.steps):
            step(0)
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / self.steps
        proj_fl = 2.0 * S * hid * (Hq * 2 * D + 2 * Hkv * D) + 2.0 * S * Hq * D * hid
        attn_fl = self.causal_flops(S, Hq, D)
        return {"workload": "prefill layer, 4096-token chunk: norm + Q/K/V GEMM, fused attention, o_proj GEMM + "
                            "residual (config 3 shape, hidden 4096)",
                "ms_per_step": ms, "flops": proj_fl + attn_fl,
                "tflops": (proj_fl + attn_fl) / (ms * 1e-3) / 1e12,
                "frac_of_bf16_peak": (proj_fl + attn_fl) / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}

    def prefill_fp8(self):
        """FP8 (OCP e4m3) KV lane of the fused prefill: a 4096-token chunk after a
        4096-token cached prefix (Qwen3.5-9B shape, 16/4 heads, D 256).  The prefix
        is read as codes x scale (bf16), the chunk unquantised; the chunk's K/V are
        appended as e4m3 codes + scales.  Roofline of the MFMA attention kernel;
        stage_ms = the step time minus the attention kernel's event-pair time,
        which come from two passes: besides the K/V staging pass (norm + RoPE +
        append of the chunk, dequantised prefix K and V^T) it carries the
        difference in the long MFMA kernel's clock between the passes (several
        per cent), so rocprof's time of kv_stage_kernel is the staging's own."""
        torch, K = self.torch, self.K
        S, start, Hq, Hkv, D, rot = 4096, 4096, 16, 4, 256, 64
        L = start + S
        q_proj = self.randn(S, Hq * 2 * D, seed=31)
        k_new = self.randn(S, Hkv * D, seed=32)
        v_new = self.randn(S, Hkv * D, seed=33)
        qw = (self.randn(D, seed=34).float() * 0.02 + 1).bfloat16()
        kw = (self.randn(D, seed=35).float() * 0.02 + 1).bfloat16()
        cos, sin = (t.to(self.dev) for t in K.rope_tables(rot, L + 1, 1.0e7))
        kk = self.randn(1, Hkv, L, D, seed=36)
        vv = self.randn(1, Hkv, L, D, seed=37)
        ks = (kk.float().abs().amax(-1) / 448).clamp(min=1e-12)
        vs = (vv.float().abs().amax(-1) / 448).clamp(min=1e-12)
        kq = (kk.float() / ks[..., None]).to(torch.float8_e4m3fn).view(torch.uint8)
        vq = (vv.float() / vs[..., None]).to(torch.float8_e4m3fn).view(torch.uint8)
        del kk, vv
        cache = K.KvCache(kq, vq, ks.contiguous(), vs.contiguous())
        out = torch.empty(S, Hq * D, dtype=torch.bfloat16, device=self.dev)
        ws = torch.zeros(K.prefill_workspace_size(True, Hkv, D, S, start), dtype=torch.uint8, device=self.dev)

        def step(i):
            K.fused_prefill(0, q_proj, k_new, v_new, qw, kw, cos, sin, cache, out, q_heads=Hq, kv_heads=Hkv,
                            head_dim=D, rotary_dim=rot, chunk_start=start, workspace=ws)
        step_ms, kern_ms, _ = self.timed(step)
        fl = self.causal_flops(S, Hq, D, start)
        ach = fl / (kern_ms * 1e-3) / 1e12
        torch.cuda.empty_cache()
        return {"workload": "FP8 e4m3 KV prefill: 4096-token chunk after a 4096-token fp8 prefix, 16/4 heads, D 256",
                "tflops_step": fl / (step_ms * 1e-3) / 1e12, "ms_per_step": step_ms, "kernel_ms": kern_ms,
                "stage_ms": step_ms - kern_ms, "flops": fl,
                "roofline": {"bound": "mfma", "achieved": round(ach, 1), "peak": BF16_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(ach / BF16_PEAK_TFLOPS, 4),
                             "traffic": measured_traffic("prefill_fp8"),
                             "kernel": "prefill_kernel (bf16 MFMA over the dequantised prefix)"}}

    def mixed(self):
        """Config 5: one 8192-token prefill chunk + 32 decode sequences, 16/2 heads,
        paged KV with 64-token pages.  The step is one mixed call (the decodes on a
        share of the CUs, the chunk beside them); the two separate calls and the
        mixed call with the two parts one after the other are timed beside it."""
        torch, K = self.torch, self.K
        Hq, Hkv, D, rot = 16, 2, 256, 64
        g = torch.Generator().manual_seed(5)
        lens = torch.randint(512, 65537, (32,), generator=g).tolist()
        # Every mode of this leg is timed after 50 warm-up steps: in a fresh
        # process the first 20-40 mixed calls with the CU split run at about
        # the two calls' speed (0.84 against 0.74-0.76 ms), later ones settle.
        wu = 50
        pstep = self.prefill_case(8192, Hq, Hkv, D, rot, seed=9, paged_ps=64)
        p_ms, p_kern, _ = self.timed(pstep, warmup=wu)
        dstep, n = self.make_decode(32, lens, Hq, Hkv, D, rot, paged_ps=64, cap=65600, seed=11)
        d_ms, _, _ = self.timed(dstep, n, warmup=wu)
        d_kern = d_ms  # one launch a step: back-to-back launch time (see decode_result)

        def both(i):
            pstep(i)
            dstep(i % n)
        serial_ms, _, _ = self.timed(both, n, warmup=wu)
        # one mixed call: decode on a share of the CUs, the chunk beside it
        dargs, dcaches = self.last_decode
        chunk = self.last_prefill
        decs = [{"q_proj": dargs["q_proj"], "k_new": dargs["k_new"], "v_new": dargs["v_new"],
                 "positions": dargs["pos"], "cache": c, "out": dargs["out"], "max_kv_len": max(lens) + 1}
                for c in dcaches]
        mws = torch.zeros(K.mixed_workspace_size(False, Hq, Hkv, D, chunk, decs[0]), dtype=torch.uint8,
                          device=self.dev)

        def conc(i):
            K.fused_mixed(0, dargs["qw"], dargs["kw"], dargs["cos"], dargs["sin"], chunk=chunk, decode=decs[i % n],
                          q_heads=Hq, kv_heads=Hkv, head_dim=D, rotary_dim=rot, workspace=mws)
        import os
        saved = os.environ.pop("SUPERSONIC_MIXED_DECODE_WGS", None)
        tot_ms, _, _ = self.timed(conc, n, warmup=wu)
        # the same call with the two parts one after the other
        os.environ["SUPERSONIC_MIXED_DECODE_WGS"] = "0"
        seq_ms, _, _ = self.timed(conc, n, warmup=wu)
        del os.environ["SUPERSONIC_MIXED_DECODE_WGS"]
        if saved is not None:
            os.environ["SUPERSONIC_MIXED_DECODE_WGS"] = saved
        fl = self.causal_flops(8192, Hq, D)
        kv_bytes, d_bytes = self.decode_bytes(lens, Hq, Hkv, D, 2)
        self.torch.cuda.empty_cache()
        return {"workload": "config 5, 8192-token chunk + 32 paged decode seqs (16/2 heads, pages of 64), "
                            "one mixed call (decode and chunk at once on disjoint CUs)",
                "ms_per_step": tot_ms, "two_calls_ms_per_step": serial_ms, "one_after_other_ms_per_step": seq_ms,
                "prefill_kernel_ms": p_kern, "decode_kernel_ms": d_kern,
                "prefill_tflops": fl / (p_kern * 1e-3) / 1e12,
                "prefill_frac": fl / (p_kern * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                "decode_gbs": (kv_bytes + 32 * Hq * D * 2) / (d_kern * 1e-3) / 1e9,
                "decode_frac": (kv_bytes + 32 * Hq * D * 2) / (d_kern * 1e-3) / 1e9 / HBM_PEAK_GBS,
                # the step's combined bound max(bytes / HBM peak, flops / MFMA peak)
                # against the measured step (one mixed call)
                "combined_bound_ms": max((kv_bytes + 32 * Hq * D * 2) / (HBM_PEAK_GBS * 1e9),
                                         fl / (BF16_PEAK_TFLOPS * 1e12)) * 1e3,
                "combined_frac": max((kv_bytes + 32 * Hq * D * 2) / (HBM_PEAK_GBS * 1e9),
                                     fl / (BF16_PEAK_TFLOPS * 1e12)) * 1e3 / tot_ms,
                "lens_sum": sum(lens)}

    def oproj(self):
        """Output projection + residual after the attention, config-2 decode step:
        8 rows, attn 16x256 = 4096 -> hidden 4096 (Qwen3.5-9B hidden size), bf16
        weights.  16 weight copies (512 MB) rotate so no step finds W in the
        256 MB last-level cache, as across a model's layers."""
        torch, K = self.torch, self.K
        rows, hid, adim, copies = 8, 4096, 4096, 16
        ws = [self.randn(hid, adim, seed=20 + c) * (adim ** -0.5) for c in range(copies)]
        ws = [w.to(torch.bfloat16).contiguous() for w in ws]
        attn = self.randn(rows, adim, seed=40)
        hidden = self.randn(rows, hid, seed=41)

        def step(i):
            K.o_proj_residual(0, attn, ws[i], hidden)
        step_ms, kern_pair_ms, _ = self.timed(step, copies)
        kern_ms = step_ms  # one launch a step: back-to-back launch time (see decode_result)
        kern_bytes = hid * adim * 2 + rows * adim * 2 + rows * hid * 4
        ach = kern_bytes / (kern_ms * 1e-3) / 1e9
        del ws
        torch.cuda.empty_cache()
        return {"workload": "o_proj + residual, 8 rows, 4096 -> 4096, bf16", "ms_per_step": step_ms,
                "kernel_ms": kern_ms, "kernel_ms_event_pairs": kern_pair_ms, "bytes": kern_bytes,
                "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic("oproj"),
                             "kernel": "skinny_lds_kernel",
                             "bytes_per_launch": kern_bytes}}

    def proj_gemm(self):
        """Prefill-sized projections on the hand-written MFMA GEMM, config 3's
        chunk (4096 rows, hidden 4096, 16/4 heads of 256): input norm + Q/K/V
        (one GEMM, three column segments) and o_proj + residual (the residual
        add in the GEMM epilogue).  The same calls routed to hipBLASLt
        (SUPERSONIC_PROJ_GEMM=hipblaslt) are timed alongside for comparison."""
        import os
        torch, K = self.torch, self.K
        rows, hid, nq, nkv, adim = 4096, 4096, 8192, 1024, 4096
        hidden = self.randn(rows, hid, seed=50)
        nw = (self.randn(hid, seed=51) * 0.1).to(torch.bfloat16)
        wq, wk, wv = ((self.randn(n, hid, seed=52 + i) * hid ** -0.5).to(torch.bfloat16).contiguous()
                      for i, n in enumerate((nq, nkv, nkv)))
        wo = (self.randn(hid, adim, seed=55) * adim ** -0.5).to(torch.bfloat16).contiguous()
        attn = self.randn(rows, adim, seed=56)
        outs = [torch.empty(rows, n, dtype=torch.bfloat16, device=self.dev) for n in (nq, nkv, nkv)]
        qkv_flops = 2.0 * rows * hid * (nq + 2 * nkv)
        o_flops = 2.0 * rows * adim * hid
        res = {"workload": "prefill projections, 4096 rows: norm + Q/K/V 4096 -> 8192 + 2x1024 and "
                           "o_proj 4096 -> 4096 + residual, bf16"}
        for label, env in (("", None), ("hipblaslt_", "hipblaslt")):
            if env:
                os.environ["SUPERSONIC_PROJ_GEMM"] = env
            try:
                _, q_ms, _ = self.timed(lambda i: K.qkv_proj(0, hidden, nw, wq, wk, wv, *outs))
                h = hidden.clone()
                _, o_ms, _ = self.timed(lambda i: K.o_proj_residual(0, attn, wo, h))
            finally:
                os.environ.pop("SUPERSONIC_PROJ_GEMM", None)
            res[label + "qkv_ms"] = q_ms
            res[label + "qkv_tflops"] = qkv_flops / (q_ms * 1e-3) / 1e12
            res[label + "oproj_ms"] = o_ms
            res[label + "oproj_tflops"] = o_flops / (o_ms * 1e-3) / 1e12
        ach = o_flops / (res["oproj_ms"] * 1e-3) / 1e12
        res["roofline"] = {"bound": "mfma", "achieved": round(ach, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                           "frac": round(ach / BF16_PEAK_TFLOPS, 4), "traffic": measured_traffic("gemm_oproj"),
                           "kernel": "gemm_bt_kernel (o_proj + residual epilogue)"}
        return res

    def qkv(self):
        """Input norm + Q/K/V projections of a config-2 decode step: 8 rows,
        hidden 4096 -> q_proj 16x2x256 = 8192, k/v 4x256 = 1024 each, bf16
        weights (84 MB; 4 copies rotate past the 256 MB last-level cache)."""
        torch, K = self.torch, self.K
        rows, hid, nq, nkv, copies = 8, 4096, 8192, 1024, 4
        ws = [[(self.randn(n, hid, seed=60 + 3 * c + i) * (hid ** -0.5)).to(torch.bfloat16).contiguous()
               for i, n in enumerate((nq, nkv, nkv))] for c in range(copies)]
        hidden = self.randn(rows, hid, seed=70)
        nw = self.randn(hid, seed=71) * 0.1
        outs = [torch.empty(rows, n, dtype=torch.bfloat16, device=self.dev) for n in (nq, nkv, nkv)]

        nwb = nw.to(torch.bfloat16)

        def step(i):
            K.qkv_proj(0, hidden, nwb, *ws[i], *outs)
        step_ms, kern_ms, _ = self.timed(step, copies)
        kern_bytes = (nq + 2 * nkv) * hid * 2 + rows * hid * 2 + hid * 2 + rows * (nq + 2 * nkv) * 2
        ach = kern_bytes / (kern_ms * 1e-3) / 1e9
        del ws
        torch.cuda.empty_cache()
        return {"workload": "input norm + Q/K/V projections, 8 rows, 4096 -> 8192 + 2x1024, bf16",
                "ms_per_step": step_ms, "kernel_ms": kern_ms, "bytes": kern_bytes,
                "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(ach / HBM_PEAK_GBS, 4),
                             "traffic": measured_traffic("qkv"),  # the projection kernel's bytes (the norm kernel: 128 KB)
                             "kernel": "input_norm_kernel + skinny_lds_kernel (3 segments), events around both",
                             "bytes_per_launch": kern_bytes}}

    def qkv_rope(self):
        """The fused projection of a config-2 decode step: input norm + Q/K/V
        projections + per-head QK RMSNorm + partial RoPE + bf16 KV append (8 rows,
        hidden 4096, 16/4 heads, D 256), 4 weight copies rotating past the MALL."""
        torch, K = self.torch, self.K
        rows, hid, Hq, Hkv, D, rot, copies, L = 8, 4096, 16, 4, 256, 64, 4, 32768
        nq, nkv = Hq * 2 * D, Hkv * D
        ws = [[(self.randn(n, hid, seed=60 + 3 * c + i) * (hid ** -0.5)).to(torch.bfloat16).contiguous()
               for i, n in enumerate((nq, nkv, nkv))] for c in range(copies)]
        hidden = self.randn(rows, hid, seed=70)
        nwb = (self.randn(hid, seed=71) * 0.1).to(torch.bfloat16)
        qw = (self.randn(D, seed=72).float() * 0.02 + 1).bfloat16()
        kw = (self.randn(D, seed=73).float() * 0.02 + 1).bfloat16()
        cos, sin = (t.to(self.dev) for t in K.rope_tables(rot, L + 1, 1.0e7))
        pos = torch.full((rows,), L, dtype=torch.int32, device=self.dev)
        cache = K.KvCache(torch.zeros(rows, Hkv, 64, D, dtype=torch.bfloat16, device=self.dev),
                          torch.zeros(rows, Hkv, 64, D, dtype=torch.bfloat16, device=self.dev),
                          block_table=torch.zeros(rows, L // 64 + 1, dtype=torch.int32, device=self.dev))
        mk = lambda n: torch.empty(rows, n, dtype=torch.bfloat16, device=self.dev)
        q, gate, k, v = mk(Hq * D), mk(Hq * D), mk(nkv), mk(nkv)
        wsp = torch.zeros(K.qkv_proj_rope_workspace_size(rows, hid, Hq, Hkv, D), dtype=torch.uint8, device=self.dev)

        def step(i):
            K.qkv_proj_rope(0, hidden, nwb, *ws[i], qw, kw, cos, sin, pos, q, gate, k, v, q_heads=Hq, kv_heads=Hkv,
                            head_dim=D, rotary_dim=rot, cache=cache, workspace=wsp)
        step_ms, kern_ms, _ = self.timed(step, copies)
        kern_bytes = (nq + 2 * nkv) * hid * 2 + rows * hid * 2 + hid * 2 + rows * (nq + 2 * nkv) * 2
        ach = kern_bytes / (kern_ms * 1e-3) / 1e9
        del ws
        torch.cuda.empty_cache()
        return {"workload": "input norm + Q/K/V projections + QK norm + RoPE + KV append, 8 rows, 4096 -> 16/4 heads",
                "ms_per_step": step_ms, "kernel_ms": kern_ms, "bytes": kern_bytes,
                "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": measured_traffic("qkv_rope"),
                             "kernel": "input_norm_kernel + skinny_lds_kernel (fused norm/RoPE epilogue), events around both",
                             "bytes_per_launch": kern_bytes}}

    def layer_graph(self):
        """One decode layer (input norm + Q/K/V projections, fused attention step,
        o_proj + residual) per step, eager launches against a HIP graph replay of
        the same launches: config 1 heads (B=1, 8/2 heads, 2048 cached tokens,
        hidden 1024) and config 2 (B=8, 16/4 heads, 32768 cached, hidden 4096)."""
        torch, K = self.torch, self.K
        res = {}
        for name, (B, Hq, Hkv, hid, L) in {"config1": (1, 8, 2, 1024, 2048),
                                           "config2_b8": (8, 16, 4, 4096, 32768)}.items():
            D, rot = 256, 64
            g = torch.Generator().manual_seed(5)
            hidden0 = self.randn(B, hid, seed=80)
            nw = (self.randn(hid, seed=81) * 0.1).to(torch.bfloat16)
            wq, wk, wv = ((self.randn(n, hid, seed=82 + i) * hid ** -0.5).to(torch.bfloat16)
                          for i, n in enumerate((Hq * 2 * D, Hkv * D, Hkv * D)))
            wo = (self.randn(hid, Hq * D, seed=85) * (Hq * D) ** -0.5).to(torch.bfloat16)
            qw = (self.randn(D, seed=88).float() * 0.02 + 1).bfloat16()
            kw = (self.randn(D, seed=89).float() * 0.02 + 1).bfloat16()
            cos, sin = (t.to(self.dev) for t in K.rope_tables(rot, L + 2, 1.0e7))
            kc = self.randn(B, Hkv, L + 1, D, seed=86)
            vc = self.randn(B, Hkv, L + 1, D, seed=87)
            cache = K.KvCache(kc, vc)
            pos = torch.full((B,), L, dtype=torch.int32, device=self.dev)
            q_proj = torch.empty(B, Hq * 2 * D, dtype=torch.bfloat16, device=self.dev)
            k_new = torch.empty(B, Hkv * D, dtype=torch.bfloat16, device=self.dev)
            v_new = torch.empty_like(k_new)
            attn = torch.empty(B, Hq * D, dtype=torch.bfloat16, device=self.dev)
            hidden = hidden0.clone()
            st = torch.cuda.Stream()

            def layer():
                K.qkv_proj(0, hidden, nw, wq, wk, wv, q_proj, k_new, v_new, stream=st)
                K.fused_decode(0, q_proj, k_new, v_new, qw, kw, cos, sin, pos, cache, attn, q_heads=Hq,
                               kv_heads=Hkv, head_dim=D, rotary_dim=rot, max_kv_len=L + 1, stream=st)
                K.o_proj_residual(0, attn, wo, hidden, stream=st)

            def timed_on_stream(fn):
                with torch.cuda.stream(st):
                    for _ in range(self.warmup):
                        fn()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(st)
                    for _ in range(self.steps):
                        fn()
                    e1.record(st)
                st.synchronize()
                return e0.elapsed_time(e1) / self.steps

            eager_ms = timed_on_stream(layer)
            graph = torch.cuda.CUDAGraph()
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=st):
                layer()
            graph_ms = timed_on_stream(graph.replay)
            # the same layer as one persistent kernel
            lws = torch.zeros(K.decode_layer_workspace_size(B, hid, Hq, Hkv, D, L + 1), dtype=torch.uint8,
                              device=self.dev)

            def persistent():
                K.decode_layer(0, hidden, nw, wq, wk, wv, qw, kw, wo, cos, sin, pos, cache, lws, q_heads=Hq,
                               kv_heads=Hkv, head_dim=D, rotary_dim=rot, max_kv_len=L + 1, stream=st)
            pers_ms = timed_on_stream(persistent)
            # the same kernel through an ordinary launch (no co-residency guarantee)
            os.environ["SUPERSONIC_LAYER_LAUNCH"] = "plain"
            try:
                plain_ms = timed_on_stream(persistent)
            finally:
                del os.environ["SUPERSONIC_LAYER_LAUNCH"]
            res[name] = {"eager_us_per_layer": round(eager_ms * 1e3, 2), "graph_us_per_layer": round(graph_ms * 1e3, 2),
                         "persistent_us_per_layer": round(pers_ms * 1e3, 2),
                         "persistent_plain_launch_us_per_layer": round(plain_ms * 1e3, 2), "launches_per_layer": 4}
            del kc, vc, cache, graph
            torch.cuda.empty_cache()
        return {"workload": "decode layer (input norm + Q/K/V projections, fused decode, o_proj + residual): eager "
                            "launches vs HIP graph replay vs the persistent one-kernel layer", **res}

    def copy(self):
        """Plain device copy of known size, to calibrate FETCH_SIZE/WRITE_SIZE counters."""
        torch = self.torch
        n = 512 << 20
        a = torch.empty(n, dtype=torch.uint8, device=self.dev)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        return {"workload": "copy", "bytes": n}

    def read(self):
        """Plain streaming reads of each decode config's byte count, for scale
        next to the decode legs: torch's int64 sum over a device buffer of that
        size (rotating over copies so that no read is served by the 256 MB
        MALL), median of 20 timed reads, and the same bytes over the decode
        leg's kernel time would read at that rate."""
        torch = self.torch
        out = {}
        for name, nbytes in (("decode_cfg1", 4198400), ("decode1", 134225920), ("fp8", 305144352),
                             ("decode8", 1073807360)):
            copies = max(1, min(8, (512 << 20) // nbytes + 1))
            bufs = [torch.ones(nbytes // 8, dtype=torch.int64, device=self.dev) for _ in range(copies)]
            for i in range(5):
                bufs[i % copies].sum()
            torch.cuda.synchronize()
            ts = []
            for i in range(20):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                bufs[i % copies].sum()
                e1.record()
                torch.cuda.synchronize()
                ts.append(e0.elapsed_time(e1))
            ms = statistics.median(ts)
            out[name] = {"bytes": nbytes, "ms": round(ms, 5), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)}
            del bufs
            torch.cuda.empty_cache()
        return {"workload": "plain streaming reads (torch int64 sum) of each decode leg's bytes", **out}

    def cpu_decode8(self):
        """The torch fp32 oracle on this host's cores: one config-2 B=8 step."""
        import torch
        from oracle import attn_oracle as O  # the CPU baseline is the oracle itself
        torch.set_num_threads(min(16, os.cpu_count() or 1))
        g = torch.Generator().manual_seed(3)
        B, Hq, Hkv, D, rot, L = 8, 16, 4, 256, 64, 32768
        shape = O.LayerShape(Hq, Hkv, D, rot)
        q_proj = O.randn_bf16(g, B, Hq * 2 * D)
        k_new = O.randn_bf16(g, B, Hkv * D)
        v_new = O.randn_bf16(g, B, Hkv * D)
        qw, kw = O.norm_weights(g, D)
        cos, sin = O.rope_tables(rot, L + 1, 1.0e7)
        kc = [O.randn_bf16(g, Hkv, L + 1, D) for _ in range(B)]
        vc = [O.randn_bf16(g, Hkv, L + 1, D) for _ in range(B)]
        pos = [L] * B
        O.decode_layer(shape, q_proj, k_new, v_new, qw, kw, cos, sin, pos, kc, vc)  # warm-up
        times = []
        t_end = time.perf_counter() + 30.0
        while len(times) < 5 and (len(times) < 2 or time.perf_counter() < t_end):
            t = time.perf_counter()
            O.decode_layer(shape, q_proj, k_new, v_new, qw, kw, cos, sin, pos, kc, vc)
            times.append(time.perf_counter() - t)
        med = statistics.median(times)
        _, bytes_step = self.decode_bytes([L] * B, Hq, Hkv, D, 2)
        return {"value": round(bytes_step / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
                "kind": "port", "seconds_per_step": round(med, 4),
                "sample": f"oracle.attn_oracle.decode_layer (torch fp32) on one full config-2 B=8 step, "
                          f"median of {len(times)} runs after 1 warm-up"}


if __name__ == "__main__":
    main()
