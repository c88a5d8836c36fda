"""Pins for the oracle's warm-tier codecs (CPU)."""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import codec

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_scale_division_is_rounding_invariant():
    # f16(d / 255) is the same whether the division is IEEE fp32 (ATen CPU)
    # or a multiply by the fp32 reciprocal (ATen CUDA scalar-divisor path),
    # for every finite non-negative fp16 d -- so the reference's scale has
    # one value on either device.
    d = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    a = (d / np.float32(255.0)).astype(np.float16)
    b = (d * (np.float32(1.0) / np.float32(255.0))).astype(np.float16)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_ref_constant_row_uses_unit_scale():
    x = np.full((1, 1, 1, 8), 3.7, np.float16)
    q, s, z = codec.quantize_ref_u8(x)
    assert s.item() == 1.0                      # torch.where(scale == 0, 1, scale)
    assert z.item() == -4.0                     # -round(3.7 / 1)
    assert (q == 0).all()                       # clamp(round(3.7) - 4, 0, 255)


def test_ref_positive_row_negative_zero_point():
    x = np.linspace(1.0, 2.0, 64).astype(np.float16).reshape(1, 64)
    q, s, z = codec.quantize_ref_u8(x)
    assert z.item() < 0
    assert q.min() == 0 and q.max() == 255
    # dequant error bounded by ~half a step (+ fp16 rounding of the ops)
    deq = codec.dequantize_ref_u8(q, s, z).astype(np.float32)
    assert np.abs(deq - x.astype(np.float32)).max() <= s.item() * 0.5 + 2e-3


def test_ref_half_even_ties():
    # scale = 1: (max - min) = 255 exactly; x / 1 = x; rint half to even.
    x = np.array([[0.0, 255.0, 2.5, 3.5, 100.5, 101.5]], np.float16)
    q, s, z = codec.quantize_ref_u8(x)
    assert s.item() == 1.0 and z.item() == 0.0
    assert q.tolist() == [[0, 255, 2, 4, 100, 102]]


def test_ref_double_rounding_through_fp16():
    # torch.round(tensor / scale) rounds the quotient to fp16 first: find a
    # row where that differs from rounding the fp32 quotient directly and
    # check the oracle follows the fp16 path.
    rng = np.random.default_rng(3)
    for _ in range(2000):
        row = rng.uniform(-3, 3, 16).astype(np.float16)
        q, s, z = codec.quantize_ref_u8(row[None])
        sf = np.float32(s.item())
        quo32 = row.astype(np.float32) / sf
        quo16 = quo32.astype(np.float16).astype(np.float32)
        diff = np.rint(quo16) != np.rint(quo32)
        if diff.any():
            i = int(np.argmax(diff))
            expect = np.clip(np.float32(np.float16(np.rint(quo16[i]) + np.float32(z.item()))), 0, 255)
            assert q[0, i] == int(expect)
            return
    pytest.fail("no double-rounding case found")


def test_ref_codec_matches_golden_vectors():
    path = os.path.join(GOLDEN, "codec_ref_u8.npz")
    if not os.path.exists(path):
        pytest.skip("golden vectors not generated")
    g = np.load(path)
    q, s, z = codec.quantize_ref_u8(g["x"])
    assert np.array_equal(q, g["q"])
    assert np.array_equal(s.view(np.uint16), g["scale"].view(np.uint16))
    assert np.array_equal(z.view(np.uint16), g["zero"].view(np.uint16))
    deq = codec.dequantize_ref_u8(g["q"], g["scale"], g["zero"])
    assert np.array_equal(deq.view(np.uint16), g["deq"].view(np.uint16))


def test_absmax_endpoints_and_error_bound():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 3, 16, 32)).astype(np.float16)
    q, s = codec.quantize_absmax_i8(x)
    assert q.dtype == np.int8 and s.shape == (5, 3)
    amax = np.abs(x.astype(np.float32)).max(axis=(-2, -1))
    np.testing.assert_array_equal(s, (amax / np.float32(127)).astype(np.float32))
    # the largest |x| of every tile maps to +-127
    assert (np.abs(q.astype(np.int32)).max(axis=(-2, -1)) == 127).all()
    deq = codec.dequantize_absmax_i8(q, s)
    err = np.abs(deq - x.astype(np.float32))
    assert (err <= s[..., None, None] * 0.5 * (1 + 1e-6)).all()


def test_absmax_zero_block_and_brute_force():
    z = np.zeros((1, 1, 2, 4), np.float16)
    q, s = codec.quantize_absmax_i8(z)
    assert s.item() == 0.0 and (q == 0).all()
    # brute force: every code is the integer in [-127, 127] nearest to x / s
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((1, 1, 4, 4)) * 3).astype(np.float16)
    q, s = codec.quantize_absmax_i8(x)
    sv = np.float32(s.item())
    for v, c in zip(x.ravel(), q.ravel()):
        r = np.float32(v) / sv
        cands = np.arange(-127, 128)
        best = cands[np.argmin(np.abs(cands - np.float64(r)))]
        if abs(abs(np.float64(r) - np.floor(np.float64(r))) - 0.5) > 1e-9:
            assert c == best
