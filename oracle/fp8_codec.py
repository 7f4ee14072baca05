"""FP8 e4m3 codecs restated on the CPU (numpy).  TEST INFRASTRUCTURE ONLY.

Two codecs live on this path:

* ``ocp``: OCP FP8 e4m3fn (bias 7, no infinities, 0x7F/0xFF = NaN, largest
  finite 448, round-to-nearest-even, subnormal step 2^-9).  gfx950 converts this
  format in hardware and ``torch.float8_e4m3fn`` implements it, so it is the
  codec of the native fused paths.
* ``ref``: the reference's hand-rolled codec,
  ``kernels/full_attention_4b.hip:118-132`` (decode) and ``:205-232`` (encode).
  It differs from OCP in two places that the restatement keeps on purpose:
    - subnormals use the step ``1.52587890625e-2 / 8`` (= 125/65536) instead
      of 2^-9 (= 128/65536), ``:126`` and ``:210-216``;
    - the normal-range exponent is clamped to 14 (``:222``), so every
      magnitude that would need exponent field 15 and every magnitude that
      rounds up out of exponent 14 (|x| >= 248) is encoded as 0x7E (= 448).
  The drop-in ``supersonic_qwen35_4b_hip_quantize_kv_to_fp8`` reproduces these
  bytes exactly; the decode LUT is ``fp8_e4m3_to_float`` (``:118-132``).

Arithmetic is done in float32 where the reference computes in float32 so the
restatement is bit-faithful (the divisions by powers of two are exact; the one
rounded float32 step is the subnormal ``val / 1.52587890625e-2f * 8.0f``).
"""
from __future__ import annotations

import numpy as np

REF_SUBNORMAL = np.float32(1.52587890625e-2)  # full_attention_4b.hip:126
E4M3_MAX = 448.0


def ocp_decode_table() -> np.ndarray:
    """All 256 OCP e4m3fn codes decoded to float32 (NaN for 0x7F/0xFF)."""
    codes = np.arange(256, dtype=np.uint32)
    sign = np.where(codes & 0x80, -1.0, 1.0)
    exp = (codes >> 3) & 0xF
    man = (codes & 0x7).astype(np.float64)
    mag = np.where(exp == 0, man * 2.0 ** -9, (1.0 + man / 8.0) * np.exp2(exp.astype(np.float64) - 7.0))
    out = (sign * mag).astype(np.float32)
    out[(codes & 0x7F) == 0x7F] = np.nan
    return out


def ref_decode_table() -> np.ndarray:
    """The reference decode LUT, ``fp8_e4m3_to_float`` (full_attention_4b.hip:118-132).

    NaN codes decode to 0; subnormals use the 1.52587890625e-2 constant."""
    codes = np.arange(256, dtype=np.uint32)
    sign = (codes >> 7) & 1
    exp = (codes >> 3) & 0xF
    man = (codes & 0x7).astype(np.float32)
    sub = (man / np.float32(8.0)) * REF_SUBNORMAL
    nrm = (np.float32(1.0) + man / np.float32(8.0)) * np.exp2(exp.astype(np.float32) - np.float32(7.0))
    val = np.where(exp == 0, sub, nrm).astype(np.float32)
    val = np.where(sign == 1, -val, val)
    val[(codes == 0x7F) | (codes == 0xFF)] = 0.0
    return val.astype(np.float32)


def ocp_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> OCP e4m3fn codes, round-to-nearest-even, saturating at +-448.

    Independent of torch so it can pin ``torch.float8_e4m3fn``: every code's
    value is a grid point, and the nearest grid point (ties to the even code)
    is picked by searching the sorted positive grid."""
    x = np.asarray(x, dtype=np.float32)
    table = ocp_decode_table()[:0x7F].astype(np.float64)  # codes 0..0x7E, increasing
    a = np.minimum(np.abs(x.astype(np.float64)), E4M3_MAX)
    hi = np.searchsorted(table, a, side="left")  # first grid point >= a
    hi = np.clip(hi, 0, 0x7E)
    lo = np.clip(hi - 1, 0, 0x7E)
    d_lo = a - table[lo]
    d_hi = table[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(a == table[hi], hi, code).astype(np.uint8)
    neg = np.signbit(x)
    return (code | np.where(neg, 0x80, 0)).astype(np.uint8)


def ref_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> codes with the reference encoder ``float_to_fp8_e4m3``
    (full_attention_4b.hip:205-232), branch for branch."""
    v = np.asarray(x, dtype=np.float32)
    sign = np.where(v < 0, 0x80, 0).astype(np.uint32)
    a = np.abs(v).astype(np.float32)
    out = np.zeros(a.shape, dtype=np.uint32)

    sat = a >= np.float32(448.0)                                   # :209
    tiny = (~sat) & (a < REF_SUBNORMAL * np.float32(0.125))        # :210
    sub = (~sat) & (~tiny) & (a < np.float32(0.015625))            # :212
    nrm = ~(sat | tiny | sub)

    out[sat] = 0x7E
    out[tiny] = 0
    if np.any(sub):
        m = np.rint((a[sub] / REF_SUBNORMAL) * np.float32(8.0)).astype(np.int64)   # :213
        m = np.maximum(m, 0)
        out[sub] = np.where(m >= 8, 0x08, m).astype(np.uint32)      # :215-216
    if np.any(nrm):
        an = a[nrm]
        _, e2 = np.frexp(an)                 # an = f * 2^e2, f in [0.5, 1)
        e = (e2 - 1) + 7                     # floor(log2(an)) + 7, :219-220
        e = np.clip(e, 1, 14)                # :221-222
        pow2 = np.ldexp(np.float32(1.0), e - 7).astype(np.float32)
        m = np.rint((an / pow2 - np.float32(1.0)) * np.float32(8.0)).astype(np.int64)  # :224
        m = np.maximum(m, 0)
        carry = m >= 8
        e = np.where(carry, e + 1, e)
        m = np.where(carry, 0, m)
        code = (e.astype(np.uint32) << 3) | m.astype(np.uint32)
        code = np.where(e > 14, 0x7E, code)                        # :229
        out[nrm] = code
    return (out | sign).astype(np.uint8)


def decode(codes: np.ndarray, codec: str = "ocp") -> np.ndarray:
    table = ocp_decode_table() if codec == "ocp" else ref_decode_table()
    return table[np.asarray(codes, dtype=np.uint8).astype(np.int64)]


def encode(x: np.ndarray, codec: str = "ocp") -> np.ndarray:
    return ocp_encode(x) if codec == "ocp" else ref_encode(x)


def quantize_rows(x: np.ndarray, codec: str = "ocp"):
    """Per-row (token, head) absmax quantisation of a ``[..., D]`` float array.

    ``scale = max(absmax / 448, 1e-12)`` and ``code = e4m3(x * (1/scale))``,
    computed in float32 exactly as ``quantize_kv_to_fp8_kernel``
    (full_attention_4b.hip:4786-4829): the reciprocal is rounded once and the
    element is multiplied by it.  Returns ``(codes uint8 [..., D], scale f32 [...])``."""
    x = np.asarray(x, dtype=np.float32)
    absmax = np.max(np.abs(x), axis=-1)
    scale = np.maximum(absmax / np.float32(448.0), np.float32(1e-12)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    return encode(x * inv[..., None], codec), scale
