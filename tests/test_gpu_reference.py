"""The reference's own HIP kernels (built from /root/reference by oracle/Makefile
into oracle/_ref/) as a checker, on the GPU:

* they pin the CPU oracle to the reference's actual behaviour (the FP8 encoder
  byte for byte, the causal prefill semantics within fp32 tolerance);
* they show the drop-in library matches the reference symbol for symbol.

``decode_flat`` is not run: launched with 32 threads on a wave64 GPU, its
``__shfl_down(v, 32)`` reduction (prefill_helpers.hip:48-53) reads lanes
outside the workgroup, so the reference itself is only meaningful on wave32
hardware; that entry point stays pinned by the oracle, the float64 brute force
and the golden vectors instead.
"""
import ctypes as C
import os

import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, check, gen
from oracle import attn_oracle as O
from supersonic_amd import kernel_ffi as K

pytestmark = pytest.mark.gpu
REF_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref")


def _lib(name):
    path = os.path.join(REF_DIR, name)
    if not os.path.exists(path):
        pytest.skip(f"{path} not built (needs /root/reference at build time)")
    return C.CDLL(path)


@pytest.fixture(scope="module")
def ref_fa():
    return _lib("libref_full_attention.so")


@pytest.fixture(scope="module")
def ref_fa4b():
    return _lib("libref_full_attention_4b.so")


@pytest.fixture(scope="module")
def ref_ph():
    return _lib("libref_prefill_helpers.so")


def P(t):
    return C.c_void_p(t.data_ptr())


def test_reference_fp8_quantiser_bytes(ref_fa4b):
    """Reference encoder == oracle restatement == drop-in, byte for byte,
    including the exponent-14 saturation (|x/scale| >= 248 -> 0x7E)."""
    announce("reference quantize_kv_to_fp8")
    g = gen(91)
    Hkv, S, D, maxT, off = 4, 96, 256, 128, 9
    src = O.randn_bf16(g, Hkv, S, D)
    src[2, 5] = 0.0
    src[1, 1, :6] = torch.tensor([1e-4, -2.5e-3, 0.3, 250.0, -447.0, 300.0]).bfloat16()
    codes_ref = torch.zeros(Hkv, maxT, D, dtype=torch.uint8, device=DEV)
    scale_ref = torch.zeros(Hkv, maxT, dtype=torch.float32, device=DEV)
    f = ref_fa4b.supersonic_qwen35_4b_hip_quantize_kv_to_fp8
    f.argtypes = [C.c_int, C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p] + [C.c_int] * 5
    assert f(2, 0, P(src.to(DEV)), P(codes_ref), P(scale_ref), Hkv, S, D, maxT, off) == 0
    codes_o, scale_o = O.quantize_kv_to_fp8(src, "ref")
    assert torch.equal(codes_ref[:, off:off + S].cpu(), codes_o)
    assert torch.equal(scale_ref[:, off:off + S].cpu(), scale_o)
    ours = torch.zeros_like(codes_ref)
    ours_s = torch.zeros_like(scale_ref)
    K.quantize_kv_to_fp8(0, K.ScalarType.BF16, src.to(DEV), ours, ours_s, Hkv, S, D, maxT, off)
    assert torch.equal(ours.cpu(), codes_ref.cpu()) and torch.equal(ours_s.cpu(), scale_ref.cpu())


@pytest.mark.parametrize("dtype", [2, 0, 1])
@pytest.mark.parametrize("B,Hq,Hkv,S,off,D", [(1, 8, 2, 160, 0, 256), (2, 4, 1, 70, 33, 128)])
def test_reference_prefill_semantics(ref_fa, dtype, B, Hq, Hkv, S, off, D):
    """Reference prefill kernel vs the oracle (pins causal limit, GQA map,
    scale) and vs the drop-in MFMA kernel."""
    announce(f"reference prefill dtype={dtype} B={B} S={S} off={off} D={D}")
    tdt = {2: torch.bfloat16, 0: torch.float16, 1: torch.float32}[dtype]
    g = gen(92)
    L = off + S
    q = torch.randn(B, Hq, S, D, generator=g).to(tdt)
    k = torch.randn(B, Hkv, L, D, generator=g).to(tdt)
    v = torch.randn(B, Hkv, L, D, generator=g).to(tdt)
    out_ref = torch.zeros(B, Hq, S, D, device=DEV)
    f = ref_fa.supersonic_qwen35_hip_full_attention_prefill
    f.argtypes = [C.c_int] + [C.c_size_t] * 8 + [C.c_float, C.c_size_t] + [C.c_void_p] * 4
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    assert f(dtype, 0, B, Hq, Hkv, S, L, D, Hq // Hkv, D ** -0.5, off, P(qd), P(kd), P(vd), P(out_ref)) == 0
    oracle = O.attention_prefill(q.float(), k.float(), v.float(), D ** -0.5, off)
    check(out_ref, oracle, (1e-4, 1e-5), "reference vs oracle")
    ours = torch.zeros_like(out_ref)
    K.full_attention_prefill(0, dtype, B, Hq, Hkv, S, L, D, D ** -0.5, off, qd, kd, vd, ours)
    torch.cuda.synchronize()
    check(ours, out_ref.cpu(), (2e-2, 2e-3) if dtype != 1 else (1e-4, 1e-5), "drop-in vs reference")


def test_reference_rms_norm_and_cast(ref_fa):
    announce("reference rms_norm / cast")
    g = gen(93)
    x = O.randn_bf16(g, 64, 256).to(DEV)
    w = O.randn_bf16(g, 256, std=0.1).to(DEV)
    a = torch.zeros(64, 256, dtype=torch.bfloat16, device=DEV)
    b = torch.zeros_like(a)
    f = ref_fa.supersonic_qwen35_hip_rms_norm
    f.argtypes = [C.c_int, C.c_size_t, C.c_size_t, C.c_size_t, C.c_float, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    for unit in (1, 0):
        assert f(2, 0, 64, 256, 1e-6, unit, P(x), P(w), P(a)) == 0
        K.rms_norm_rows(0, 2, 64, 256, 1e-6, x, w, b, add_unit_offset=bool(unit))
        d = (a.float() - b.float()).abs()
        # same formula, different reduction order: at most one bf16 ulp apart
        assert (d <= 2 ** -7 * a.float().abs() + 1e-30).all() and (d > 0).float().mean() < 0.01
        o = O.rms_norm_rows(x.float().cpu(), w.cpu(), 1e-6, add_unit_offset=bool(unit))
        assert ((a.float().cpu() - o).abs() <= 2 ** -7 * o.abs() + 1e-30).all()
    c = ref_fa.supersonic_qwen35_hip_cast
    c.argtypes = [C.c_int, C.c_int, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p]
    f32r = torch.zeros(64, 256, device=DEV)
    f32o = torch.zeros_like(f32r)
    assert c(2, 1, 0, x.numel(), P(x), P(f32r)) == 0
    K.cast(0, 2, 1, x.numel(), x, f32o)
    assert torch.equal(f32r, f32o)


def test_reference_prefill_chain_helpers(ref_ph):
    """RoPE, split q/gate, sigmoid gate and the transpose: drop-in == reference."""
    announce("reference rope/split/sigmoid/transpose")
    g = gen(94)
    S, H, D, rot, off = 37, 4, 256, 64, 500
    cos, sin = O.rope_tables(rot, off + S, 1.0e7)
    cosd, sind = cos.to(DEV), sin.to(DEV)
    x = O.randn_bf16(g, S, H, D).to(DEV)
    xr, xo = x.clone(), x.clone()
    f = ref_ph.supersonic_qwen35_hip_apply_rope_prefill
    f.argtypes = [C.c_int, C.c_size_t] + [C.c_size_t] * 4 + [C.c_void_p] * 3
    offb = off * (rot // 2) * 2
    assert f(2, 0, S, H, D, rot // 2, C.c_void_p(cosd.data_ptr() + offb), C.c_void_p(sind.data_ptr() + offb), P(xr)) == 0
    K.apply_rope_prefill(0, 2, S, H, D, rot, cosd, sind, off, xo)
    torch.cuda.synchronize()
    d = (xr.float() - xo.float()).abs()
    assert (d <= 2 ** -7 * xr.float().abs() + 1e-30).all() and (d > 0).float().mean() < 0.01
    src = O.randn_bf16(g, S, H * 2 * D).to(DEV)
    qr, gr = torch.zeros(S, H, D, dtype=torch.bfloat16, device=DEV), torch.zeros(S, H, D, dtype=torch.bfloat16, device=DEV)
    qo, go = torch.zeros_like(qr), torch.zeros_like(gr)
    s = ref_ph.supersonic_qwen35_hip_split_qgate
    s.argtypes = [C.c_int, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p]
    assert s(2, 0, S, H, D, P(src), P(qr), P(gr)) == 0
    K.split_qgate(0, 2, S, H, D, src, qo, go)
    assert torch.equal(qr, qo) and torch.equal(gr, go)
    m = ref_ph.supersonic_qwen35_hip_sigmoid_mul
    m.argtypes = [C.c_int, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p, C.c_void_p]
    mr, mo = torch.zeros_like(qr), torch.zeros_like(qr)
    assert m(2, 0, qr.numel(), P(qr), P(gr), P(mr)) == 0
    K.sigmoid_mul(0, 2, qr.numel(), qr, gr, mo)
    d = (mr.float() - mo.float()).abs()
    assert (d <= 2 ** -7 * mr.float().abs() + 1e-30).all() and (d > 0).float().mean() < 0.01
    t = ref_ph.supersonic_qwen35_hip_transpose_shd_hsd
    t.argtypes = [C.c_int, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p]
    tr, to = torch.zeros(H, S, D, dtype=torch.bfloat16, device=DEV), torch.zeros(H, S, D, dtype=torch.bfloat16, device=DEV)
    assert t(2, 0, S, H, D, P(qr), P(tr)) == 0
    K.transpose_shd_hsd(0, 2, S, H, D, qr, to)
    assert torch.equal(tr, to)
