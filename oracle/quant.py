"""Oracle: the reference's weight formats, restated in numpy (TEST INFRASTRUCTURE).

int4  — spider_moe/quant.py:89-143 (quantize_int4 / dequantize_int4):
        symmetric, per group of ``g`` elements along the LAST dim (the GEMM-K
        dim of an nn.Linear weight [out, in]); scale = max(amax, 1e-8) / 7;
        q = clamp(round_half_even(w / scale), -8, 7); byte i of a row holds
        element 2i in the low nibble and 2i+1 in the high nibble
        (quant.py:108-110); dequant sign-extends nibbles (quant.py:132-133)
        and multiplies by the group scale.  ``g`` falls back to the row
        length when it does not divide it (quant.py:99-100).
fp8   — spider_moe/quant.py:146-169 (quantize_fp8_with_scale_tensor /
        dequantize_fp8_with_scale_tensor) with a per-output-channel scale
        (amax over K / 448, as compute_fp8_scale quant.py:30-33 does per
        tensor).  The cast is torch's float32 -> float8_e4m3fn: round to
        nearest even, no saturation (|x| > 464 becomes NaN; 0x7F/0xFF are
        the NaN codes, the format has no infinities).

Pins (tests/test_oracle_quant.py):
  * the e4m3 encoder/decoder against torch's own float8_e4m3fn cast over all
    256 codes and a dense sweep including every rounding midpoint;
  * int4 against hand-computed bytes and the closed-form invariants
    (q in [-7, 7] from the quantizer, -8 only through dequant of 0x8 nibbles,
    round trip error <= scale/2 elementwise, mean error < 0.15 at g=32 as in
    tests/test_quant_fp8_int4.py:30-36 of the reference);
  * golden bytes written by the reference's own quantize_int4
    (tests/golden/quant_int4.npz).
"""
from __future__ import annotations

import numpy as np

FP8_E4M3_MAX = 448.0


# ---------------------------------------------------------------- int4 ----
def int4_group(n: int, group_size: int) -> int:
    """Effective group size (quant.py:99-100)."""
    if group_size <= 0 or n % group_size != 0:
        return n
    return group_size


def int4_quantize(weight: np.ndarray, group_size: int = 64):
    """Return (packed uint8 [..., n/2], scales float32 [..., n/g], g)."""
    w = np.asarray(weight, dtype=np.float32)
    *lead, n = w.shape
    if n % 2:
        raise ValueError("last dimension must be even for INT4 packing")
    g = int4_group(n, group_size)
    rows = w.reshape(-1, n // g, g)
    amax = np.abs(rows).max(axis=-1)
    scales = (np.maximum(amax, np.float32(1e-8)) / np.float32(7.0)).astype(np.float32)
    q = np.round(rows / scales[..., None]).clip(-8, 7).astype(np.int8).reshape(-1, n)
    lo = (q[:, 0::2].astype(np.int16) & 0xF).astype(np.uint8)
    hi = (q[:, 1::2].astype(np.int16) & 0xF).astype(np.uint8)
    packed = (lo | (hi << 4)).astype(np.uint8).reshape(*lead, n // 2)
    return packed, scales.reshape(*lead, n // g), g


def int4_unpack(packed: np.ndarray) -> np.ndarray:
    """Signed int8 values [..., 2*half] from packed bytes."""
    p = np.asarray(packed, dtype=np.uint8)
    lo = (p & 0xF).astype(np.int8)
    hi = ((p >> 4) & 0xF).astype(np.int8)
    lo = np.where(lo >= 8, lo - 16, lo).astype(np.int8)
    hi = np.where(hi >= 8, hi - 16, hi).astype(np.int8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def int4_dequantize(packed: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """float32 weights: q * scale per group (scales may be fp16 or fp32)."""
    q = int4_unpack(packed).astype(np.float32)
    *lead, n = q.shape
    g = group_size
    s = np.asarray(scales).astype(np.float32).reshape(*lead, n // g, 1)
    return (q.reshape(*lead, n // g, g) * s).reshape(*lead, n)


# ----------------------------------------------------------------- fp8 ----
def fp8_e4m3_decode(bits: np.ndarray) -> np.ndarray:
    """float32 value of each e4m3fn code (bias 7, no inf, 0x7F/0xFF NaN)."""
    b = np.asarray(bits, dtype=np.uint8).astype(np.int32)
    sign = np.where(b & 0x80, -1.0, 1.0)
    exp = (b >> 3) & 0xF
    man = b & 0x7
    normal = sign * (1.0 + man / 8.0) * np.exp2(exp - 7.0)
    sub = sign * (man / 8.0) * np.exp2(-6.0)
    val = np.where(exp == 0, sub, normal)
    val = np.where((b & 0x7F) == 0x7F, np.nan, val)
    return val.astype(np.float32)


def _round_half_even(x: np.ndarray) -> np.ndarray:
    return np.round(x)  # numpy rounds half to even


def fp8_e4m3_encode(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> e4m3fn code, NaN above 464."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64)  # exact widening
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.int32)
    a = np.abs(x)
    out = np.zeros(a.shape, dtype=np.int32)
    nan = np.isnan(a) | (a > 464.0)
    small = a < 2.0 ** -6
    # subnormals: value = m * 2^-9, m in [0, 8]; m == 8 is the smallest normal
    m_sub = _round_half_even(np.where(small, a, 0.0) / 2.0 ** -9).astype(np.int32)
    # normals
    with np.errstate(divide="ignore", invalid="ignore"):
        e = np.floor(np.log2(np.where(small | nan, 1.0, a))).astype(np.int32)
    frac = np.where(small | nan, 1.0, a) / np.exp2(e.astype(np.float64))
    # guard log2 rounding at exact powers of two
    adj_hi = frac >= 2.0
    adj_lo = frac < 1.0
    e = e + adj_hi.astype(np.int32) - adj_lo.astype(np.int32)
    frac = np.where(small | nan, 1.0, a) / np.exp2(e.astype(np.float64))
    m = _round_half_even((frac - 1.0) * 8.0).astype(np.int32)
    carry = m == 8
    e = e + carry.astype(np.int32)
    m = np.where(carry, 0, m)
    normal_code = ((e + 7) << 3) | m
    out = np.where(small, m_sub, normal_code)
    out = np.where(nan, 0x7F, out)
    return (out | sign).astype(np.uint8)


def fp8_quantize_per_channel(w: np.ndarray):
    """w [..., N, K] -> (codes uint8 [..., N, K], scale float32 [..., N]).

    scale = max(amax_K / 448, 1e-12)  (compute_fp8_scale per output channel,
    quant.py:30-33; the 1e-12 clamp is quant.py:158).
    """
    w = np.asarray(w, dtype=np.float32)
    amax = np.abs(w).max(axis=-1)
    scale = np.maximum(amax / np.float32(FP8_E4M3_MAX), np.float32(1e-12)).astype(np.float32)
    codes = fp8_e4m3_encode((w / scale[..., None]).astype(np.float32))
    return codes, scale


def fp8_dequantize_per_channel(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """float32 weights = decode(code) * scale  (quant.py:161-169)."""
    return (fp8_e4m3_decode(codes) * np.asarray(scale, np.float32)[..., None]).astype(np.float32)
