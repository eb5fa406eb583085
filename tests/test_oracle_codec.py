"""Pins the CPU oracle's MXFP4 codec (oracle/mxfp4.py) against checks that do
not share its code: the OCP MX field definitions, torch's own e8m0 dtype, a
brute-force nearest-code search, an exact model of the exponent choice, and
hand-built bytes.  The reference ships no codec tests or vectors
(reference ``.gitignore:22``; nothing in ``docs/``)."""

import math
import struct

import numpy as np
import pytest
import torch

from oracle import mxfp4 as ox


def ocp_e2m1_value(code: int) -> float:
    """OCP MX v1.0 E2M1: 1 sign, 2 exponent (bias 1), 1 mantissa bit;
    exponent field 0 is subnormal: 2**(1-1) * (m/2)."""
    s, e, m = (code >> 3) & 1, (code >> 1) & 3, code & 1
    mag = (m / 2.0) if e == 0 else 2.0 ** (e - 1) * (1.0 + m / 2.0)
    return -mag if s else mag


def f32_bits(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def test_e2m1_table_matches_ocp_fields():
    got = ox.decode_e2m1(np.arange(16))
    want = np.array([ocp_e2m1_value(c) for c in range(16)], dtype=np.float32)
    assert np.array_equal(f32_bits(got), f32_bits(want))
    assert np.signbit(got[8]) and got[8] == 0.0  # code 8 is -0.0


def test_e8m0_matches_torch_float8_e8m0fnu():
    b = np.arange(255, dtype=np.uint8)
    want = torch.from_numpy(b).view(torch.float8_e8m0fnu).float().numpy()
    assert np.array_equal(f32_bits(ox.decode_e8m0(b)), f32_bits(want))
    # byte 0 is 2**-127, an fp32 subnormal, not zero
    assert f32_bits(ox.decode_e8m0(np.uint8(0))) == 0x00400000
    with pytest.raises(ValueError):
        ox.decode_e8m0(np.array([255], np.uint8))
    assert np.isnan(ox.decode_e8m0(np.array([255], np.uint8), nan_ok=True)[0])
    assert np.isnan(torch.tensor([255], dtype=torch.uint8).view(torch.float8_e8m0fnu).float()[0])


def exhaustive_pairs():
    """Every (code, scale byte) pair: one row per scale byte, the 16 codes
    repeated twice to fill a 32-element block."""
    codes = np.tile(np.arange(16, dtype=np.uint8), 2)
    packed = np.tile(ox.pack_codes(codes[None, :]), (255, 1))
    scale = np.arange(255, dtype=np.uint8)[:, None]
    return packed, scale


def test_dequant_exhaustive_known_answers():
    packed, scale = exhaustive_pairs()
    got = ox.dequantize_chunk(packed, scale)
    assert got.shape == (255, 32) and got.dtype == np.float32
    for b in range(255):
        sc = math.ldexp(1.0, b - 127)
        for j in range(32):
            v = ocp_e2m1_value(j % 16) * sc          # exact in float64
            want = np.float32(v)                       # exact (or +-inf) in fp32
            assert f32_bits(got[b, j]) == f32_bits(want), (b, j)


def test_dequant_values_are_exact_in_bf16():
    packed, scale = exhaustive_pairs()
    f = ox.dequantize_chunk(packed, scale)
    t = torch.from_numpy(f)
    back = t.to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(f32_bits(back), f32_bits(f))
    # overflow points at byte 254 (scale 2**127): 1.5 * 2**127 is the last
    # finite magnitude, 2 * 2**127 and above are +-inf
    assert np.isfinite(f[254, 3]) and f[254, 3] == np.float32(1.5 * 2.0 ** 127)
    assert np.isinf(f[254, 4]) and f[254, 4] > 0
    assert np.isinf(f[254, 15]) and f[254, 15] < 0


def test_torch_form_of_dequant_is_bit_identical():
    """The torch-ops decode the CPU baseline times gives the numpy decode's
    bits on the exhaustive code x byte table and on random blocks, and
    raises on byte 255 and bad shapes like it."""
    packed, scale = exhaustive_pairs()
    a = ox.dequantize_chunk(packed, scale)
    b = ox.dequantize_chunk_torch(packed, scale).numpy()
    assert b.dtype == np.float32 and np.array_equal(f32_bits(a), f32_bits(b))
    rng = np.random.default_rng(5)
    p = rng.integers(0, 256, (37, 96), dtype=np.uint8)
    s = rng.integers(0, 255, (37, 6), dtype=np.uint8)
    assert np.array_equal(f32_bits(ox.dequantize_chunk(p, s)),
                          f32_bits(ox.dequantize_chunk_torch(torch.from_numpy(p), torch.from_numpy(s)).numpy()))
    with pytest.raises(ValueError):
        ox.dequantize_chunk_torch(np.zeros((1, 16), np.uint8), np.array([[255]], np.uint8))
    with pytest.raises(ValueError):
        ox.dequantize_chunk_torch(np.zeros((1, 16), np.uint8), np.zeros((1, 2), np.uint8))


def test_hand_built_bytes():
    # 0x21: low nibble 1 (0.5) first, high nibble 2 (1.0) second
    p = np.full((1, 16), 0x21, np.uint8)
    got = ox.dequantize_chunk(p, np.array([[127]], np.uint8))
    assert got[0, 0] == 0.5 and got[0, 1] == 1.0
    # 0x8F: first element code 15 (-6), second code 8 (-0.0); scale 2**-3
    p = np.full((1, 16), 0x8F, np.uint8)
    got = ox.dequantize_chunk(p, np.array([[124]], np.uint8))
    assert got[0, 0] == -0.75 and got[0, 1] == 0.0 and np.signbit(got[0, 1])
    # scale column b covers elements 32b..32b+31
    p = np.full((1, 32), 0x22, np.uint8)
    got = ox.dequantize_chunk(p, np.array([[127, 130]], np.uint8))
    assert np.all(got[0, :32] == 1.0) and np.all(got[0, 32:] == 8.0)


def test_dequant_rejects_nan_scale_and_bad_shapes():
    with pytest.raises(ValueError):
        ox.dequantize_chunk(np.zeros((1, 16), np.uint8), np.array([[255]], np.uint8))
    with pytest.raises(ValueError):
        ox.dequantize_chunk(np.zeros((1, 16), np.uint8), np.zeros((1, 2), np.uint8))
    with pytest.raises(ValueError):
        ox.dequantize_chunk(np.zeros((1, 8), np.uint8), np.zeros((1, 1), np.uint8))


# ---------------------------------------------------------------- quantizer

def exact_exponent(amax: np.float32) -> int:
    """ceil of the correctly rounded fp32 log2 of fl32(amax/6).

    The reference evaluates ``ceil(torch.log2(amax / 6.0))`` in fp32.  For a
    quotient ``y = 2**k * (1+f)`` the exact ceil is ``k`` when ``f == 0`` and
    ``k+1`` otherwise, except that a correctly rounded fp32 log2 returns the
    integer ``k`` itself while ``log2(1+f)`` stays under half an fp32 ulp of
    ``k``; then the ceil is ``k``.  Evaluated here in float64."""
    if amax == 0:
        return 0
    y = np.float32(amax) / np.float32(6.0)          # fp32 division, RNE
    yf = float(y)
    m, k = math.frexp(yf)                           # yf = m * 2**k, m in [0.5, 1)
    k -= 1                                          # yf = (2m) * 2**k
    frac = 2.0 * m - 1.0
    if frac == 0.0:
        return k
    v = k + math.log1p(frac) / math.log(2.0)
    r = float(np.float32(v))
    return int(math.ceil(r))


def brute_force_block(x: np.ndarray):
    """Quantize one 32-block by exhaustive search over the 8 magnitudes,
    ties to the even code, using ``exact_exponent``."""
    amax = np.float32(np.max(np.abs(x)))
    e = exact_exponent(amax)
    divisor = np.float32(math.ldexp(1.0, e))
    codes = []
    for v in x:
        s = np.float32(v) / divisor
        mag = min(abs(float(s)), 6.0)
        best, best_err = None, None
        for c in range(8):
            err = abs(mag - float(ox.E2M1_MAGNITUDE[c]))
            if best is None or err < best_err or (err == best_err and c % 2 == 0):
                best, best_err = c, err
        codes.append(best | (8 if np.signbit(s) else 0))
    return np.array(codes, np.uint8), e + 127


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_quantizer_matches_brute_force_random(seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(6, 256, generator=g) * 0.02)
    w[0, :32] *= 1e3          # large block
    w[1, 32:64] *= 1e-20      # tiny block
    w[2, 64:96] = 0.0         # zero block
    w[3, 96:128] = -0.0       # negative zero block
    packed, scale = ox.quantize_chunk(w)
    codes = ox.unpack_codes(packed)
    x = w.numpy()
    for r in range(x.shape[0]):
        for b in range(x.shape[1] // 32):
            c, s = brute_force_block(x[r, 32 * b:32 * b + 32])
            assert s == scale[r, b], (r, b)
            assert np.array_equal(c, codes[r, 32 * b:32 * b + 32]), (r, b)


def test_exponent_model_equals_torch_log2_in_every_binade():
    """The oracle's exponent goes through torch.log2; it must agree with the
    correctly-rounded model at and just above every power of two, where a
    faithful-but-not-correctly-rounded log2 could differ."""
    amax = []
    for k in range(-124, 128):
        for j in range(0, 40):
            y = math.ldexp(1.0 + j * 2.0 ** -23, k)
            a = np.float32(np.float32(y) * np.float32(6.0))
            if np.isfinite(a) and a > 0:
                amax.append(a)
                amax.append(np.nextafter(a, np.float32(np.inf)))
                amax.append(np.nextafter(a, np.float32(0)))
    amax = np.array(amax, dtype=np.float32)
    got = ox.block_exponent(amax)
    want = np.array([exact_exponent(a) for a in amax])
    assert np.array_equal(got, want)


def test_quantizer_special_cases():
    # all-zero block: byte 127, codes 0, and code 8 for -0.0
    w = np.zeros((1, 32), np.float32)
    w[0, 5] = -0.0
    p, s = ox.quantize_chunk(w)
    c = ox.unpack_codes(p)[0]
    assert s[0, 0] == 127 and c[5] == 8 and np.all(np.delete(c, 5) == 0)
    # amax exactly 6 * 2**e -> exponent e, element codes 7
    for e in (-10, -1, 0, 3):
        w = np.full((1, 32), 6.0 * 2.0 ** e, np.float32)
        p, s = ox.quantize_chunk(w)
        assert s[0, 0] == 127 + e and np.all(ox.unpack_codes(p) == 7)
    # ties: scale 1 (amax 6); midpoints 0.25,1.25,2.5,5 round down, 0.75,1.75,3.5 up
    w = np.zeros((1, 32), np.float32)
    w[0, :8] = [6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    w[0, 8:16] = -w[0, :8]
    p, s = ox.quantize_chunk(w)
    c = ox.unpack_codes(p)[0]
    assert s[0, 0] == 127
    assert list(c[:8]) == [7, 0, 2, 2, 4, 4, 6, 6]
    assert list(c[8:16]) == [15, 8, 10, 10, 12, 12, 14, 14]  # -0.25 -> code 8 (-0)
    # a negative value that rounds to zero keeps its sign bit
    w = np.zeros((1, 32), np.float32)
    w[0, 0], w[0, 1] = 6.0, -0.1
    c = ox.unpack_codes(ox.quantize_chunk(w)[0])[0]
    assert c[1] == 8


def test_quantizer_clamps_above_six():
    # amax/6 rounds so that log2 lands on an integer from above:
    # y = 2**-7 * (1 + 2**-23) has ceil(log2) == -7 under correct rounding,
    # so amax / 2**-7 slightly exceeds 6 and is clamped to code 7.
    y = np.float32(math.ldexp(1.0 + 2.0 ** -23, -7))
    a = np.float32(y * np.float32(6.0))
    assert np.float32(a / np.float32(6.0)) == y
    w = np.zeros((1, 32), np.float32)
    w[0, 0] = a
    p, s = ox.quantize_chunk(w)
    assert s[0, 0] == 127 - 7
    assert ox.unpack_codes(p)[0, 0] == 7
    assert np.float32(a / np.float32(2.0 ** -7)) > 6.0


def test_quantizer_errors():
    with pytest.raises(ValueError):
        ox.quantize_chunk(np.zeros((2, 48), np.float32))
    with pytest.raises(ValueError):
        ox.quantize_chunk(np.zeros((2,), np.float32).reshape(1, 2, 1)[0])
    for bad in (np.nan, np.inf, -np.inf):
        w = np.zeros((1, 32), np.float32)
        w[0, 3] = bad
        with pytest.raises(ValueError):
            ox.quantize_chunk(w)
    w = np.full((1, 32), 3.0e38, np.float32)       # e = ceil(log2(5e37)) = 126 -> ok
    ox.quantize_chunk(w)
    w = np.full((1, 32), 1.0e-44, np.float32)      # e < -127 -> error
    with pytest.raises(ValueError):
        ox.quantize_chunk(w)


def test_quantizer_idempotent_and_error_bound():
    g = torch.Generator().manual_seed(11)
    w = torch.randn(64, 512, generator=g) * 0.02
    p, s = ox.quantize_chunk(w)
    d = ox.dequantize_chunk(p, s)
    # values are a fixed point; codes need not be (a block whose scaled amax
    # rounds to 3 re-quantizes with exponent e-1 and doubled codes)
    p2, s2 = ox.quantize_chunk(d)
    assert np.array_equal(f32_bits(ox.dequantize_chunk(p2, s2)), f32_bits(d))
    assert np.all((s2 == s) | (s2 == s - 1))
    # |deq - x| <= half the local grid gap * 2**e (gap <= 2 at the top of the grid)
    x = w.numpy().reshape(64, 16, 32)
    scale = ox.decode_e8m0(s)[..., None]
    err = np.abs(d.reshape(64, 16, 32) - x) / scale
    assert np.all(err <= 1.0 + 1e-6)
    # sign symmetry: quantize(-x) flips exactly the sign bits
    pn, sn = ox.quantize_chunk(-w)
    assert np.array_equal(sn, s)
    assert np.array_equal(ox.unpack_codes(pn), ox.unpack_codes(p) ^ 8)


def test_quantizer_accepts_bf16_and_fp16():
    g = torch.Generator().manual_seed(3)
    w = torch.randn(4, 64, generator=g) * 0.02
    for dt in (torch.bfloat16, torch.float16):
        a = ox.quantize_chunk(w.to(dt))
        b = ox.quantize_chunk(w.to(dt).float())
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
