"""Pins both e4m3 codecs of ``oracle.fp8_codec``.

OCP e4m3fn is pinned against ``torch.float8_e4m3fn`` (an independent
implementation) exhaustively over all codes and on dense random inputs.  The
reference codec (kernels/full_attention_4b.hip:118-132, :205-232) is pinned by
expectations derived by hand from that source, value by value, below.
"""
import numpy as np
import pytest
import torch

from oracle import attn_oracle as O
from oracle import fp8_codec as F

# (value, OCP code, reference code), each code worked out by hand:
#   reference subnormal step is 1.52587890625e-2 / 8, values below 1/8 of that
#   flush to 0; normal exponents are clamped to 14, so |x| >= 248 -> 0x7E.
HAND = [
    (0.0, 0x00, 0x00), (-0.0, 0x80, 0x00), (1e-30, 0x00, 0x00),
    (2.0 ** -10, 0x00, 0x00),            # OCP: tie between 0 and 2^-9 -> even (0)
    (2.0 ** -9, 0x01, 0x01),             # ref: rint(1.024) = 1
    (1.5 * 2.0 ** -9, 0x02, 0x02),       # OCP tie -> even code 2; ref rint(1.536) = 2
    (0.0152, 0x08, 0x08),                # ref: rint(7.969) = 8 -> smallest normal
    (0.015625, 0x08, 0x08), (0.0175, 0x09, 0x09),
    (1.0, 0x38, 0x38), (1.0625, 0x38, 0x38), (1.1875, 0x3A, 0x3A),
    (3.0, 0x44, 0x44), (17.0, 0x58, 0x58),
    (239.0, 0x77, 0x77), (240.0, 0x77, 0x77), (247.9, 0x77, 0x77),
    (248.0, 0x78, 0x7E),                 # OCP rounds up to 256; ref overflows exponent 14
    (255.9, 0x78, 0x7E), (256.0, 0x78, 0x7E), (300.0, 0x79, 0x7E), (447.0, 0x7E, 0x7E),
    (448.0, 0x7E, 0x7E), (460.0, 0x7E, 0x7E), (1000.0, 0x7E, 0x7E),
    (-0.3, 0xAA, 0xAA), (-250.0, 0xF8, 0xFE), (-448.0, 0xFE, 0xFE),
]


def test_hand_derived_codes():
    x = np.array([h[0] for h in HAND], np.float32)
    assert F.ocp_encode(x).tolist() == [h[1] for h in HAND]
    assert F.ref_encode(x).tolist() == [h[2] for h in HAND]


def test_ocp_table_matches_torch_exhaustively():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    tv = codes.view(torch.float8_e4m3fn).float().numpy()
    ours = F.ocp_decode_table()
    nan = np.isnan(tv)
    assert np.array_equal(nan, np.isnan(ours))
    assert np.array_equal(tv[~nan], ours[~nan])
    assert nan.sum() == 2 and ours[0x7E] == 448.0 and ours[0x08] == 2.0 ** -6 and ours[1] == 2.0 ** -9


def test_ocp_encode_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(200000) * s for s in (1e-3, 0.1, 1, 30, 200)]).astype(np.float32)
    x = np.concatenate([x, F.ocp_decode_table()[:0x7F],            # every grid point
                        (F.ocp_decode_table()[:0x7E] + F.ocp_decode_table()[1:0x7F]) / 2])  # every midpoint
    x = np.clip(x, -448, 448).astype(np.float32)
    tv = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(F.ocp_encode(x), tv)


def test_ref_decode_table_spot_values():
    tab = F.ref_decode_table()
    assert tab[0x00] == 0.0 and tab[0x80] == 0.0
    assert tab[0x01] == np.float32(1.52587890625e-2 / 8)     # not 2^-9: the reference constant
    assert tab[0x07] == np.float32(7 * 1.52587890625e-2 / 8)
    assert tab[0x08] == 2.0 ** -6 and tab[0x38] == 1.0 and tab[0x7E] == 448.0
    assert tab[0x7F] == 0.0 and tab[0xFF] == 0.0                # NaN codes read as 0
    assert tab[0xFE] == -448.0 and tab[0x78] == 256.0           # exponent 15 still decodes
    # normals agree with OCP, subnormals are 125/128 of OCP's
    ocp = F.ocp_decode_table()
    normal = [c for c in range(256) if (c >> 3) & 0xF and (c & 0x7F) != 0x7F]
    assert np.array_equal(tab[normal], ocp[normal])
    sub = [c for c in range(1, 8)]
    assert np.allclose(tab[sub] / ocp[sub], 125 / 128)


def test_ref_encode_roundtrips_its_own_grid():
    tab = F.ref_decode_table()
    codes = np.array([c for c in range(256) if ((c >> 3) & 0xF) <= 14 and (c & 0x7F) not in (0,)], np.uint8)
    assert np.array_equal(F.ref_encode(tab[codes]), codes)


def test_quantize_rows_invariants():
    rng = np.random.default_rng(1)
    x = O.bf16r(torch.from_numpy(rng.standard_normal((4, 5, 256)).astype(np.float32))).numpy()
    x[0, 0] = 0.0
    for codec in ("ocp", "ref"):
        codes, scale = F.quantize_rows(x, codec)
        assert scale[0, 0] == np.float32(1e-12) and np.all(codes[0, 0] == 0)
        am = np.argmax(np.abs(x), -1)
        peak = np.take_along_axis(codes, am[..., None], -1)[..., 0]
        assert np.all((peak[1:] & 0x7F) == 0x7E)             # |q(absmax)| = 448
        assert np.allclose(scale[1:], np.abs(x[1:]).max(-1) / 448, rtol=1e-6)
    # OCP dequantisation error is bounded by half an e4m3 ulp (2^-4 relative)
    codes, scale = F.quantize_rows(x, "ocp")
    deq = F.decode(codes, "ocp") * scale[..., None]
    assert np.all(np.abs(deq - x) <= np.abs(x) * 2.0 ** -4 + scale[..., None] * 2.0 ** -10 + 1e-30)


@pytest.mark.parametrize("codec", ["ocp", "ref"])
def test_torch_wrapper_matches_rows(codec):
    rng = np.random.default_rng(2)
    src = torch.from_numpy(rng.standard_normal((2, 3, 64)).astype(np.float32)).bfloat16()
    c, s = O.quantize_kv_to_fp8(src, codec)
    c2, s2 = F.quantize_rows(src.float().numpy(), codec)
    assert np.array_equal(c.numpy(), c2) and np.array_equal(s.numpy(), s2)
