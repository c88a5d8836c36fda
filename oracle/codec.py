"""Warm-tier codecs (oracle; test infrastructure only).

Two formats:

1. Reference format -- ``quantize_fp16_to_int8`` / ``dequantize_int8_to_fp16``
   (tierkv_policy.py:21-44).  Per (token, head) asymmetric min/max over the
   last dim, uint8 codes, fp16 scale and fp16 zero point.  Every ATen half op
   computes in fp32 and rounds to fp16, so the restatement rounds after every
   binary op:

       scale = f16(f16(max - min) / 255)        (1.0 where it is 0)
       zp    = f16(-rint(f16(min / scale)))
       q     = u8(clamp(f16(rint(f16(x / scale)) + zp), 0, 255))
       deq   = f16(f16(f16(q) - zp) * scale)

   ``f16(d / 255)`` is identical whether the division is IEEE or a multiply
   by the fp32 reciprocal (ATen CUDA's scalar-divisor path): an exhaustive
   check over all finite fp16 ``d`` is in tests/test_oracle_codec.py.
   Pinned by golden vectors written from the reference function itself
   (tests/golden/make_golden.py) and by closed-form special cases.

2. Block absmax format (the reference has no symmetric
   quantizer).  Per (block, kv head) over block_size x head_dim:

       s = fp32(max|x|) / 127      (IEEE fp32 division)
       q = int8(clamp(rint(fp32(x) / s), -127, 127))     (0 where s == 0)
       deq = fp32(q) * s

   Pinned by brute force on tiny blocks and closed-form special cases.
"""

from __future__ import annotations

import numpy as np

F16 = np.float16
F32 = np.float32


def _f16(x):
    return np.asarray(x, dtype=F32).astype(F16)


def quantize_ref_u8(x):
    """Restates quantize_fp16_to_int8 (tierkv_policy.py:21-36).

    x: float16 array [..., D].  Returns (codes uint8 [..., D],
    scale float16 [..., 1], zero_point float16 [..., 1]).
    """
    x = np.asarray(x).astype(F16)
    xf = x.astype(F32)
    mn = x.min(axis=-1, keepdims=True).astype(F32)           # amin (exact)
    mx = x.max(axis=-1, keepdims=True).astype(F32)           # amax (exact)
    rng = _f16(mx - mn).astype(F32)                          # half sub
    scale = _f16(rng / F32(255.0))                           # half / 255.0
    scale = np.where(scale == F16(0), F16(1.0), scale)       # torch.where(scale == 0, 1, scale)
    sf = scale.astype(F32)
    zp = _f16(-np.rint(_f16(mn / sf).astype(F32)))           # -(round(min / scale))
    r = np.rint(_f16(xf / sf).astype(F32))                   # round(x / scale)
    s = _f16(r + zp.astype(F32)).astype(F32)                 # + zero_point
    q = np.clip(s, 0.0, 255.0).astype(np.uint8)              # clamp, .to(uint8)
    return q, scale, zp


def dequantize_ref_u8(q, scale, zp):
    """Restates dequantize_int8_to_fp16 (tierkv_policy.py:39-44)."""
    qf = np.asarray(q).astype(F16).astype(F32)
    d = _f16(qf - np.asarray(zp, dtype=F16).astype(F32)).astype(F32)
    return _f16(d * np.asarray(scale, dtype=F16).astype(F32))


def dequantize_ref_u8_fp32(q, scale, zp):
    """The decode kernel's fp32 dequant: (q - zp) * scale in fp32
    (tierkv_triton.py:101-102; eager reference tierkv_triton.py:762-767)."""
    qf = np.asarray(q).astype(F32)
    return (qf - np.asarray(zp, dtype=F16).astype(F32)) * np.asarray(scale, dtype=F16).astype(F32)


def quantize_absmax_i8(x, reduce_axes=(-2, -1)):
    """Symmetric int8 absmax codec over ``reduce_axes`` (default: the
    [block_size, head_dim] tile of a [..., H_kv, block_size, D] block).

    Returns (codes int8, scale float32 with reduce_axes dropped)."""
    xf = np.asarray(x).astype(F16).astype(F32)
    amax = np.abs(xf).max(axis=reduce_axes, keepdims=True)
    s = (amax / F32(127.0)).astype(F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(xf / s)
    r = np.where(s == 0, F32(0), r)
    q = np.clip(r, -127, 127).astype(np.int8)
    return q, np.squeeze(s, axis=reduce_axes).astype(F32)


def dequantize_absmax_i8(q, s, reduce_axes=(-2, -1)):
    """fp32(q) * s with s broadcast over ``reduce_axes``."""
    s = np.asarray(s, dtype=F32)
    for ax in sorted(a % np.ndim(q) for a in reduce_axes):
        s = np.expand_dims(s, ax)
    return np.asarray(q).astype(F32) * s
