"""GPU parity of the drop-in prefill-chain helpers and the FP8 quantisers."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, announce, gen
from oracle import attn_oracle as O
from oracle import fp8_codec
from supersonic_amd import kernel_ffi as K

pytestmark = pytest.mark.gpu
BF = K.ScalarType.BF16


def ulp_close(a, b, frac=0.01):
    """bf16 results equal except for rare one-ulp differences from fp32 op order."""
    a = a.float().cpu()
    b = b.float().cpu()
    d = (a - b).abs()
    assert (d <= 2 ** -7 * b.abs().clamp(min=1e-30) + 1e-30).all(), f"max diff {d.max()}"
    assert (d > 0).float().mean().item() <= frac


def test_rms_norm():
    announce("rms_norm")
    g = gen(81)
    x = O.randn_bf16(g, 300, 256)
    w = O.randn_bf16(g, 256, std=0.1)
    out = torch.zeros(300, 256, dtype=torch.bfloat16, device=DEV)
    K.rms_norm_rows(0, BF, 300, 256, 1e-6, x.to(DEV), w.to(DEV), out)
    ulp_close(out, O.rms_norm_rows(x.float(), w, 1e-6))
    K.rms_norm_rows(0, BF, 300, 256, 1e-6, x.to(DEV), w.to(DEV), out, add_unit_offset=False)
    ulp_close(out, O.rms_norm_rows(x.float(), w, 1e-6, add_unit_offset=False))


def test_rms_norm_known_answer():
    x = torch.tensor([[3.0, 4.0]]).bfloat16().to(DEV)
    w = torch.tensor([0.5, -0.5]).bfloat16().to(DEV)
    out = torch.zeros(1, 2, dtype=torch.bfloat16, device=DEV)
    K.rms_norm_rows(0, BF, 1, 2, 0.0, x, w, out)
    exp = torch.tensor([3.0 / 12.5 ** 0.5 * 1.5, 4.0 / 12.5 ** 0.5 * 0.5])
    assert (out.float().cpu()[0] - exp).abs().max() <= 0.02


def test_rope_with_offset():
    announce("rope")
    g = gen(82)
    S, H, D, rot, off = 77, 4, 256, 64, 1000
    x = O.randn_bf16(g, S, H, D)
    cos, sin = O.rope_tables(rot, off + S, 1.0e7)
    data = x.to(DEV)
    K.apply_rope_prefill(0, BF, S, H, D, rot, cos.to(DEV), sin.to(DEV), off, data)
    ulp_close(data, O.apply_rope(x.float(), cos, sin, rot, torch.arange(off, off + S)))


def test_split_transpose_sigmoid_cast():
    announce("split/transpose/sigmoid/cast")
    g = gen(83)
    S, H, D = 33, 4, 64
    src = O.randn_bf16(g, S, H * 2 * D)
    q = torch.zeros(S, H, D, dtype=torch.bfloat16, device=DEV)
    gt = torch.zeros_like(q)
    K.split_qgate(0, BF, S, H, D, src.to(DEV), q, gt)
    eq, eg = O.split_qgate(src.float(), H, D)
    assert torch.equal(q.float().cpu(), eq) and torch.equal(gt.float().cpu(), eg)
    t = torch.zeros(H, S, D, dtype=torch.bfloat16, device=DEV)
    K.transpose_shd_hsd(0, BF, S, H, D, q, t)
    assert torch.equal(t.cpu(), q.cpu().permute(1, 0, 2))
    o = torch.zeros_like(q)
    K.sigmoid_mul(0, BF, q.numel(), q, gt, o)
    ulp_close(o, O.sigmoid_mul(eq, eg))
    f = torch.zeros(S, H, D, dtype=torch.float32, device=DEV)
    K.cast(0, BF, K.ScalarType.F32, q.numel(), q, f)
    assert torch.equal(f.cpu(), eq)
    b2 = torch.zeros_like(q)
    K.cast(0, K.ScalarType.F32, BF, q.numel(), f, b2)
    assert torch.equal(b2.cpu(), q.cpu())


def test_quantize_kv_reference_codec_bit_exact():
    """Drop-in quantiser: bytes and scales identical to the reference encoder."""
    announce("quantize ref codec")
    g = gen(84)
    Hkv, S, D, maxT, off = 4, 100, 256, 160, 17
    src = O.randn_bf16(g, Hkv, S, D)
    src[0, 0] = 0.0
    src[1, 3, :8] = torch.tensor([1e-4, -3e-3, 250.0, -447.0, 2.0 ** -9, 0.5, -0.0, 300.0]).bfloat16()
    dst = torch.zeros(Hkv, maxT, D, dtype=torch.uint8, device=DEV)
    sc = torch.zeros(Hkv, maxT, dtype=torch.float32, device=DEV)
    K.quantize_kv_to_fp8(0, BF, src.to(DEV), dst, sc, Hkv, S, D, maxT, off)
    codes, scale = O.quantize_kv_to_fp8(src, "ref")
    assert torch.equal(dst[:, off:off + S].cpu(), codes)
    assert torch.equal(sc[:, off:off + S].cpu(), scale)
    assert torch.all(dst[:, :off] == 0) and torch.all(dst[:, off + S:] == 0)


def test_quantize_kv_ocp_codec_bit_exact():
    announce("quantize ocp codec")
    g = gen(85)
    Hkv, S, D = 2, 64, 256
    src = O.randn_bf16(g, Hkv, S, D)
    dst = torch.zeros(Hkv, S, D, dtype=torch.uint8, device=DEV)
    sc = torch.zeros(Hkv, S, dtype=torch.float32, device=DEV)
    K.quantize_kv_fp8_ocp(0, src.to(DEV), dst, sc, Hkv, S, D, S, 0)
    torch.cuda.synchronize()
    codes, scale = O.quantize_kv_to_fp8(src, "ocp")
    assert torch.equal(sc.cpu(), scale)
    assert torch.equal(dst.cpu(), codes)


def test_quantize_bad_dtype():
    assert K.load().supersonic_qwen35_4b_hip_quantize_kv_to_fp8(0, 0, None, None, None, 1, 1, 256, 1, 0) == 256
