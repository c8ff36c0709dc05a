"""Bit-level numerics shared by the CPU oracle (test infrastructure only).

This module is part of the parity oracle.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product path never does.

It restates, with numpy float32 arithmetic (every operation IEEE
round-to-nearest-even, no fused multiply-add), the scalar helpers that the HIP
kernels in ``community_kv_amd/csrc/ckv_numerics.h`` implement with the same
operation sequence:

* ``f32_to_f16_bits`` / ``ordered_fp16_key`` -- the fp16 score key of the
  reference selector (``descriptor_selection.cu:30-33``,
  ``tests/community_kv/attention/kernels/test_centroid_selection.py:27-33``).
* ``f32_to_bf16`` -- round-to-nearest-even bf16 storage.
* ``f32_to_e4m3`` / ``e4m3_to_f32`` -- OCP FP8 E4M3 (``float8_e4m3fn``) with the
  reference's +-448 saturation (``graph/partition.py:452-454``,
  ``tests/community_kv/graph/test_state.py:120-124``).
* ``ckv_exp`` / ``ckv_log`` -- deterministic exp/log used by the online update
  and the split merge.  Method: Cody-Waite range reduction (W. J. Cody and
  W. Waite, "Software Manual for the Elementary Functions", 1980) with a
  Taylor polynomial for exp, and the atanh series log(m) = 2*atanh((m-1)/(m+1))
  for log.  Both are pinned against ``numpy.exp``/``numpy.log`` in the tests.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32

# ---------------------------------------------------------------------------
# fp16 / bf16
# ---------------------------------------------------------------------------


def f32_to_f16_bits(x) -> np.ndarray:
    """fp32 -> IEEE half bits, round-to-nearest-even (numpy's cast)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def ordered_fp16_key(bits) -> np.ndarray:
    """Order-preserving 16-bit key of fp16 bits (descriptor_selection.cu:30-33)."""
    bits = np.asarray(bits, dtype=np.uint16)
    flip = np.where((bits & np.uint16(0x8000)) != 0, np.uint16(0xFFFF), np.uint16(0x8000))
    return (bits ^ flip).astype(np.uint16)


def f32_to_bf16(x) -> np.ndarray:
    """fp32 -> bf16 (returned as fp32 values), round-to-nearest-even, NaN kept."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    # round half to even on the 16 dropped bits; only NaN bit patterns can wrap
    # around 2^32 here, and they are replaced below
    with np.errstate(over="ignore"):
        rounded = (bits + (np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1)))) & np.uint32(0xFFFF0000)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, (bits | np.uint32(0x00400000)) & np.uint32(0xFFFF0000), rounded)
    return rounded.astype(np.uint32).view(np.float32)


def bf16_bits(x) -> np.ndarray:
    return (f32_to_bf16(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << np.uint32(16)).astype(np.uint32).view(np.float32)


# ---------------------------------------------------------------------------
# FP8 E4M3 (OCP "fn": no infinities, 0x7F/0xFF are NaN, max finite 448)
# ---------------------------------------------------------------------------

E4M3_MAX = 448.0


def _e4m3_table() -> np.ndarray:
    table = np.zeros(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exponent = (code >> 3) & 0xF
        mantissa = code & 0x7
        if exponent == 0xF and mantissa == 0x7:
            table[code] = np.nan
        elif exponent == 0:
            table[code] = sign * (mantissa / 8.0) * 2.0 ** -6
        else:
            table[code] = sign * (1.0 + mantissa / 8.0) * 2.0 ** (exponent - 7)
    return table


E4M3_TABLE = _e4m3_table()


def e4m3_to_f32(codes) -> np.ndarray:
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def f32_to_e4m3(x) -> np.ndarray:
    """fp32 -> E4M3 codes: clamp to +-448 then round-to-nearest-even.

    Restates ``tensor.clamp(-448, 448).to(torch.float8_e4m3fn)``
    (graph/partition.py:452-454).  NaN maps to 0x7F.
    """
    x = np.asarray(x, dtype=np.float32)
    sign = np.where(np.signbit(x), np.uint8(0x80), np.uint8(0))
    a = np.minimum(np.abs(x).astype(np.float64), E4M3_MAX)
    out = np.zeros(x.shape, dtype=np.uint8)
    # Subnormals: quantum 2^-9.
    sub = a < 2.0 ** -6
    q_sub = np.rint(a * 512.0)  # exact scaling by a power of two; rint is half-even
    out = np.where(sub, q_sub.astype(np.uint8), out)
    # Normals.
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(sub, 1.0, a)))
    m = np.where(sub, 1.0, a) / np.exp2(e)
    # guard log2 rounding at exact powers of two
    fix_lo = m < 1.0
    e = np.where(fix_lo, e - 1, e)
    m = np.where(fix_lo, m * 2.0, m)
    fix_hi = m >= 2.0
    e = np.where(fix_hi, e + 1, e)
    m = np.where(fix_hi, m / 2.0, m)
    q = np.rint((m - 1.0) * 8.0)
    carry = q >= 8.0
    e = np.where(carry, e + 1, e)
    q = np.where(carry, 0.0, q)
    normal_code = ((e + 7).astype(np.int64) << 3) | q.astype(np.int64)
    out = np.where(sub, out, normal_code.astype(np.uint8))
    out = (out | sign).astype(np.uint8)
    out = np.where(np.isnan(x), np.uint8(0x7F), out)
    return out.astype(np.uint8)


# ---------------------------------------------------------------------------
# Deterministic exp / log (identical operation sequence to ckv_numerics.h)
# ---------------------------------------------------------------------------

LOG2E = F32(1.44269504088896340736)
LN2_HI = F32(0.693145751953125)  # 0x3F317200: 15 significant bits, n*LN2_HI exact
LN2_LO = F32(1.42860682030941723212e-6)
EXP_C = [F32(1.0 / 5040.0), F32(1.0 / 720.0), F32(1.0 / 120.0), F32(1.0 / 24.0),
         F32(1.0 / 6.0), F32(0.5), F32(1.0), F32(1.0)]
LOG_C = [F32(2.0 / 11.0), F32(2.0 / 9.0), F32(2.0 / 7.0), F32(2.0 / 5.0), F32(2.0 / 3.0), F32(2.0)]
SQRT2 = F32(1.41421356237309504880)


def ckv_exp(x) -> np.ndarray:
    """exp(x) in float32 with a fixed operation order (no FMA)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        t = (x * LOG2E).astype(np.float32)
        n = np.rint(t).astype(np.float32)
        n_c = np.clip(n, F32(-200.0), F32(200.0)).astype(np.float32)
        r = (x - (n_c * LN2_HI).astype(np.float32)).astype(np.float32)
        r = (r - (n_c * LN2_LO).astype(np.float32)).astype(np.float32)
        p = EXP_C[0]
        for c in EXP_C[1:]:
            p = ((p * r).astype(np.float32) + c).astype(np.float32)
        ni = n_c.astype(np.int64)
        scale = ((np.clip(ni, -126, 127) + 127).astype(np.uint32) << np.uint32(23)).view(np.float32)
        y = (p * scale).astype(np.float32)
    y = np.where(ni < -125, F32(0.0), y)
    y = np.where(ni > 127, F32(np.inf), y)
    y = np.where(np.isnan(x), F32(np.nan), y)
    y = np.where(x == -np.inf, F32(0.0), y)
    y = np.where(x == np.inf, F32(np.inf), y)
    return y.astype(np.float32)


def ckv_log(x) -> np.ndarray:
    """log(x) for positive normal float32 x, fixed operation order (no FMA)."""
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    e = ((bits >> np.uint32(23)) & np.uint32(0xFF)).astype(np.int32) - 127
    m = ((bits & np.uint32(0x007FFFFF)) | np.uint32(0x3F800000)).view(np.float32)
    big = m > SQRT2
    m = np.where(big, (m * F32(0.5)).astype(np.float32), m).astype(np.float32)
    e = np.where(big, e + 1, e)
    f = (m - F32(1.0)).astype(np.float32)
    s = (f / (m + F32(1.0)).astype(np.float32)).astype(np.float32)
    s2 = (s * s).astype(np.float32)
    p = LOG_C[0]
    for c in LOG_C[1:]:
        p = ((p * s2).astype(np.float32) + c).astype(np.float32)
    logm = (s * p).astype(np.float32)
    ef = e.astype(np.float32)
    y = ((ef * LN2_HI).astype(np.float32) + ((ef * LN2_LO).astype(np.float32) + logm).astype(np.float32)).astype(np.float32)
    y = np.where(x == 0, F32(-np.inf), y)
    y = np.where(x == np.inf, F32(np.inf), y)
    y = np.where((x < 0) | np.isnan(x), F32(np.nan), y)
    return y.astype(np.float32)
