"""CPU restatement of the reference MXFP4 codec (test infrastructure only).

Format (reference ``tinyinfer/quantization/quantize_mxfp4.py:20-25, 233-253``):

* weight ``W[out, in]`` is cut into blocks of 32 consecutive input features;
* every element becomes a 4-bit e2m1 code ``s m2 m1 m0`` (sign in bit 3,
  magnitude index into {0, .5, 1, 1.5, 2, 3, 4, 6});
* codes are packed two per byte, the element with the even column index in
  the low nibble: ``packed[r, j] = c[r, 2j] | c[r, 2j+1] << 4`` ->
  uint8 ``[out, in/2]``;
* each block stores one e8m0 byte ``e + 127`` -> uint8 ``[out, in/32]``,
  decoding to ``2**(byte-127)``; byte 255 is NaN.

Byte arithmetic is numpy; the exponent choice goes through torch's CPU
``log2`` exactly as the reference does, because that is where its rounding
is defined (third-party dependency: PyTorch, pinned only as ``torch>=2.4`` in
the reference's ``pyproject.toml:11``; this container has 2.10.0).
"""

from __future__ import annotations

import numpy as np
import torch

# e2m1 magnitudes indexed by the 3-bit magnitude code
# (reference quantize_mxfp4.py:21).
E2M1_MAGNITUDE = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
# Decision points between consecutive magnitudes (reference quantize_mxfp4.py:22).
E2M1_MIDPOINT = (E2M1_MAGNITUDE[:-1] + E2M1_MAGNITUDE[1:]) / np.float32(2.0)
BLOCK = 32
E8M0_BIAS = 127
E8M0_NAN = 255


def decode_e2m1(codes) -> np.ndarray:
    """4-bit codes -> float32 values (reference ``dequantize_chunk``,
    quantize_mxfp4.py:80-82; GPU form ``decode_e2m1`` utils.h:115-127).
    Code 8 decodes to -0.0."""
    c = np.asarray(codes, dtype=np.uint8)
    mag = E2M1_MAGNITUDE[c & 7]
    return np.where((c & 8) != 0, -mag, mag).astype(np.float32)


def decode_e8m0(scale_bytes, nan_ok: bool = False) -> np.ndarray:
    """e8m0 bytes -> float32 ``2**(b-127)``.

    The reference CPU decoder rejects byte 255 (quantize_mxfp4.py:75-76); its
    GPU decoder returns a quiet NaN for it (utils.h:87-92).  ``nan_ok``
    selects the GPU behaviour.  Byte 0 is 2**-127, an fp32 subnormal.
    """
    b = np.asarray(scale_bytes, dtype=np.uint8)
    if not nan_ok and np.any(b == E8M0_NAN):
        raise ValueError("E8M0 NaN scale detected (255)")
    out = np.ldexp(np.float32(1.0), b.astype(np.int32) - E8M0_BIAS).astype(np.float32)
    return np.where(b == E8M0_NAN, np.float32(np.nan), out).astype(np.float32)


def unpack_codes(packed) -> np.ndarray:
    """uint8 ``[rows, K/2]`` -> uint8 codes ``[rows, K]`` (low nibble first)."""
    p = np.asarray(packed, dtype=np.uint8)
    codes = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    codes[..., 0::2] = p & 0x0F
    codes[..., 1::2] = p >> 4
    return codes


def pack_codes(codes) -> np.ndarray:
    """uint8 codes ``[rows, K]`` -> packed ``[rows, K/2]`` (low nibble first)."""
    c = np.asarray(codes, dtype=np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def dequantize_chunk(packed, scale, nan_ok: bool = False) -> np.ndarray:
    """Decode ``packed [rows, K/2]`` + ``scale [rows, K/32]`` to float32
    ``[rows, K]`` (reference quantize_mxfp4.py:67-85).  Every finite result is
    exact in fp32 and in bf16."""
    p = np.asarray(packed, dtype=np.uint8)
    s = np.asarray(scale, dtype=np.uint8)
    if p.ndim != 2 or s.ndim != 2 or p.shape[0] != s.shape[0]:
        raise ValueError("packed/scale shape mismatch")
    rows, half_k = p.shape
    k = 2 * half_k
    if k % BLOCK or s.shape[1] != k // BLOCK:
        raise ValueError("scale shape mismatch")
    vals = decode_e2m1(unpack_codes(p)).reshape(rows, k // BLOCK, BLOCK)
    mult = decode_e8m0(s, nan_ok=nan_ok)[..., None]
    with np.errstate(over="ignore", invalid="ignore"):
        return (vals * mult).astype(np.float32).reshape(rows, k)


def dequantize_chunk_torch(packed, scale) -> torch.Tensor:
    """The same decode as torch CPU ops on torch tensors, the way the
    reference's CPU path runs it (quantize_mxfp4.py:67-85: nibbles split,
    table lookup, sign select, ``ldexp`` of the block exponent, one multiply
    per block): this is the form the CPU baseline times, since torch spreads
    it over the host's threads.  Raises on byte 255 like the reference.
    Bit-identical to ``dequantize_chunk`` (tests/test_oracle_codec.py)."""
    p = torch.as_tensor(np.asarray(packed, dtype=np.uint8)) if not isinstance(packed, torch.Tensor) else packed
    s = torch.as_tensor(np.asarray(scale, dtype=np.uint8)) if not isinstance(scale, torch.Tensor) else scale
    if p.ndim != 2 or s.ndim != 2 or p.shape[0] != s.shape[0]:
        raise ValueError("packed/scale shape mismatch")
    rows, half_k = p.shape
    k = 2 * half_k
    if k % BLOCK or s.shape[1] != k // BLOCK:
        raise ValueError("scale shape mismatch")
    if bool((s == E8M0_NAN).any()):
        raise ValueError("E8M0 NaN scale detected (255)")
    codes = torch.stack((p & 0x0F, p >> 4), dim=-1).reshape(rows, k)
    mag = torch.from_numpy(E2M1_MAGNITUDE)[(codes & 7).long()]
    vals = torch.where(codes >= 8, -mag, mag)
    mult = torch.ldexp(torch.ones(s.shape, dtype=torch.float32), s.to(torch.int32) - E8M0_BIAS)
    return (vals.reshape(rows, k // BLOCK, BLOCK) * mult.unsqueeze(-1)).reshape(rows, k)


def block_exponent(amax: np.ndarray) -> np.ndarray:
    """Shared exponent per block: ``ceil(log2(amax / 6))`` evaluated with
    torch's fp32 CPU ops, 0 for all-zero blocks (quantize_mxfp4.py:42-46)."""
    a = torch.from_numpy(np.ascontiguousarray(amax, dtype=np.float32))
    nonzero = a > 0
    safe = torch.where(nonzero, a, torch.ones_like(a))
    e = torch.ceil(torch.log2(safe / 6.0)).to(torch.int32)
    e = torch.where(nonzero, e, torch.zeros_like(e))
    return e.numpy()


def e2m1_round(magnitude: np.ndarray) -> np.ndarray:
    """Round non-negative fp32 magnitudes (already clamped to <= 6) to the
    nearest e2m1 magnitude code, ties to the even code
    (quantize_mxfp4.py:53-59).  The upper code of midpoints 0.75, 1.75 and
    3.5 is even, so those ties round up; the rest round down."""
    m = np.asarray(magnitude, dtype=np.float32)
    code = np.zeros(m.shape, dtype=np.uint8)
    for lower, mid in enumerate(E2M1_MIDPOINT):
        upper_is_even = (lower + 1) % 2 == 0
        up = (m > mid) | ((m == mid) & upper_is_even)
        code += up.astype(np.uint8)
    return code


def quantize_chunk(weight):
    """Quantize ``[rows, K]`` fp32/fp16/bf16 weights into
    (packed uint8 ``[rows, K/2]``, scale uint8 ``[rows, K/32]``)
    (reference quantize_mxfp4.py:28-64).

    Raises ``ValueError`` for a bad shape, non-finite input, or a block
    exponent outside [-127, 127], as the reference does.
    """
    t = weight if isinstance(weight, torch.Tensor) else torch.from_numpy(np.asarray(weight))
    if t.ndim != 2 or t.shape[1] % BLOCK:
        raise ValueError(f"expected [rows,K], K multiple of 32; got {tuple(t.shape)}")
    x = t.to(dtype=torch.float32).contiguous().numpy()
    if not np.isfinite(x).all():
        raise ValueError("non-finite weights (NaN/Inf) are not supported")
    rows, k = x.shape
    blocks = x.reshape(rows, k // BLOCK, BLOCK)
    amax = np.abs(blocks).max(axis=-1) if k else np.zeros((rows, 0), np.float32)
    e = block_exponent(amax)
    if np.any((e < -E8M0_BIAS) | (e > E8M0_BIAS)):
        raise ValueError("E8M0 exponent out of representable range [-127,127]")
    # x / 2**e in fp32 (exact unless the quotient is subnormal, where fp32
    # division rounds to nearest even, as torch's division does).
    divisor = np.ldexp(np.float32(1.0), e).astype(np.float32)[..., None]
    scaled = (blocks / divisor).astype(np.float32)
    mag = np.minimum(np.abs(scaled), np.float32(6.0))
    code = e2m1_round(mag) | (np.signbit(scaled).astype(np.uint8) << 3)
    packed = pack_codes(code.reshape(rows, k))
    scale = (e + E8M0_BIAS).astype(np.uint8)
    return np.ascontiguousarray(packed), np.ascontiguousarray(scale)


def quantize_weight(w):
    """Whole-matrix convenience wrapper (the reference quantizes in row
    chunks of 128, quantize_mxfp4.py:188-192; rows are independent, so the
    chunking does not change the bytes)."""
    return quantize_chunk(w)
