"""Pins for oracle/quant.py: fp8-e4m3 against torch's own cast, int4 against
the reference's quantize_int4 bytes, hand-computed nibbles and closed forms."""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import quant as Q


def test_fp8_decode_all_codes_match_torch():
    codes = np.arange(256, dtype=np.uint8)
    ours = Q.fp8_e4m3_decode(codes)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(theirs)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], theirs[~nan])
    assert nan.sum() == 2  # 0x7F and 0xFF


def test_fp8_encode_matches_torch_on_midpoints_and_sweep():
    # every representable value, every midpoint between neighbours, +-1 ulp
    vals = Q.fp8_e4m3_decode(np.arange(256, dtype=np.uint8))
    vals = np.unique(vals[np.isfinite(vals)])
    mids = (vals[:-1].astype(np.float64) + vals[1:]) / 2
    mids = mids.astype(np.float32)
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)),
                           np.nextafter(mids, np.float32(-np.inf))])
    rng = np.random.default_rng(0)
    sweep = np.concatenate([
        vals, mids, near,
        rng.standard_normal(20000).astype(np.float32) * 50,
        rng.standard_normal(5000).astype(np.float32) * 1e-3,
        np.array([448.0, 464.0, 464.0001, 470.0, 480.0, 1e6, -464.0, -465.0,
                  2.0 ** -9, 2.0 ** -10, 2.0 ** -10 * 1.0001, 0.0, -0.0], np.float32)])
    ours = Q.fp8_e4m3_encode(sweep)
    theirs = torch.from_numpy(sweep).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    # compare decoded values (NaN codes compare as NaN; +-0 by bits)
    assert np.array_equal(ours, theirs), sweep[ours != theirs][:10]


def test_fp8_per_channel_quantize_roundtrip_bound():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((3, 16, 64)) * 0.02).astype(np.float32)
    codes, scale = Q.fp8_quantize_per_channel(w)
    assert scale.shape == (3, 16)
    deq = Q.fp8_dequantize_per_channel(codes, scale)
    # e4m3 has 3 mantissa bits: relative error <= 2^-4 for normals
    rel = np.abs(deq - w) / np.maximum(np.abs(w), scale[..., None] * 2.0 ** -6)
    assert rel.max() <= 2.0 ** -4 + 1e-6
    # the channel maximum maps exactly to 448 * scale
    amax = np.abs(w).max(-1)
    assert np.allclose(np.abs(deq).max(-1), amax, rtol=1e-6)


def test_int4_hand_vector():
    # one group of 8: amax 3.5 -> scale 0.5 -> q = w / 0.5
    w = np.array([[0.0, 1.0, -1.0, 0.5, -0.5, 0.25, 3.5, -3.5]], np.float32)
    packed, scales, g = Q.int4_quantize(w, group_size=8)
    assert g == 8 and scales[0, 0] == np.float32(0.5)
    q = [0, 2, -2, 1, -1, 0, 7, -7]   # 0.25/0.5 = 0.5 rounds half-to-even -> 0
    nib = [v & 0xF for v in q]
    expect = [nib[0] | nib[1] << 4, nib[2] | nib[3] << 4, nib[4] | nib[5] << 4, nib[6] | nib[7] << 4]
    assert packed[0].tolist() == expect
    assert np.array_equal(Q.int4_unpack(packed)[0], np.array(q, np.int8))
    # nibble 0x8 decodes to -8 (only reachable through dequant)
    assert Q.int4_unpack(np.array([[0x88]], np.uint8)).tolist() == [[-8, -8]]


def test_int4_closed_form_invariants():
    rng = np.random.default_rng(2)
    w = rng.standard_normal((6, 256)).astype(np.float32)
    for gs in (32, 64, 128):
        packed, scales, g = Q.int4_quantize(w, gs)
        q = Q.int4_unpack(packed)
        assert q.min() >= -7 and q.max() <= 7
        deq = Q.int4_dequantize(packed, scales, g)
        s = np.repeat(scales, g, axis=-1)
        assert np.all(np.abs(deq - w) <= s / 2 + 1e-6)
    # reference's own bound (tests/test_quant_fp8_int4.py:30-36)
    w4 = rng.standard_normal((4, 64)).astype(np.float32)
    p, s, g = Q.int4_quantize(w4, 32)
    assert np.abs(Q.int4_dequantize(p, s, g) - w4).mean() < 0.15
    # group fallback when it does not divide the row (quant.py:99-100)
    assert Q.int4_group(256, 48) == 256 and Q.int4_group(256, 0) == 256


def test_int4_matches_reference_bytes():
    z = np.load(os.path.join(GOLDEN, "quant_int4.npz"))
    w = z["w"]
    for gs in (32, 64, 128, 48):
        packed, scales, g = Q.int4_quantize(w, gs)
        assert g == int(z[f"g{gs}/group"])
        assert np.array_equal(packed, z[f"g{gs}/packed"])
        assert np.array_equal(scales, z[f"g{gs}/scales"])
        assert np.array_equal(Q.int4_dequantize(packed, scales, g), z[f"g{gs}/deq"])


def test_planted_int4_nibble_order_mistake_is_caught():
    """A swapped nibble order must fail the reference-bytes check."""
    z = np.load(os.path.join(GOLDEN, "quant_int4.npz"))
    packed, _, _ = Q.int4_quantize(z["w"], 64)
    swapped = ((packed & 0xF) << 4) | (packed >> 4)
    assert not np.array_equal(swapped.astype(np.uint8), z["g64/packed"])
