"""GPU parity of the device codec against the CPU oracle: dequantization is
bit-exact over every (code, scale byte) pair, and the quantizer is bit-exact
on random and adversarial blocks.  Both go through the C ABI."""

import math

import numpy as np
import pytest
import torch

from oracle import mxfp4 as ox
from tests.helpers import banner

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


def bits32(t):
    return t.detach().cpu().contiguous().view(torch.int32).numpy()


def exhaustive():
    codes = np.tile(np.arange(16, dtype=np.uint8), 2)
    packed = np.tile(ox.pack_codes(codes[None, :]), (256, 1))
    scale = np.arange(256, dtype=np.uint8)[:, None]
    return packed, scale


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_dequant_exhaustive_bit_exact(capi, out_dtype):
    banner(f"dequant exhaustive {out_dtype}")
    packed, scale = exhaustive()
    got = capi.dequant(torch.from_numpy(packed).cuda(), torch.from_numpy(scale).cuda(), out_dtype)
    torch.cuda.synchronize()
    want = ox.dequantize_chunk(packed, scale, nan_ok=True)       # fp32
    g = got.float().cpu().numpy()
    finite_rows = slice(0, 255)
    assert np.array_equal(g[finite_rows].view(np.uint32), want[finite_rows].view(np.uint32))
    # byte 255: NaN, as the reference GPU decode produces
    assert np.all(np.isnan(g[255]))


def test_dequant_random_matrix_bit_exact(capi):
    banner("dequant random 1000x4096")
    rng = np.random.default_rng(0)
    packed = rng.integers(0, 256, size=(1000, 2048), dtype=np.uint8)
    scale = rng.integers(100, 140, size=(1000, 128), dtype=np.uint8)
    scale[::7, ::5] = rng.integers(0, 255, size=scale[::7, ::5].shape, dtype=np.uint8)
    p, s = torch.from_numpy(packed).cuda(), torch.from_numpy(scale).cuda()
    want = ox.dequantize_chunk(packed, scale)
    for dt in (torch.float32, torch.bfloat16):
        got = capi.dequant(p, s, dt).float().cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), dt


def test_dequant_python_wrapper_matches_reference_errors():
    from tinyinfer_amd.quantization import dequantize_chunk
    p = torch.zeros(2, 16, dtype=torch.uint8)
    s = torch.full((2, 1), 255, dtype=torch.uint8)
    with pytest.raises(ValueError, match="255"):
        dequantize_chunk(p, s)
    s[:] = 127
    out = dequantize_chunk(p, s)
    assert out.device.type == "cpu" and out.shape == (2, 32) and torch.count_nonzero(out) == 0


def adversarial_weights():
    """Blocks at the exponent edges, ties, zeros, -0, subnormals and huge values."""
    rows = []
    for k in range(-120, 126, 7):
        for j in (0, 1, 2, 5, 11, 22, 23, 45):
            y = np.float32(math.ldexp(1.0 + j * 2.0 ** -23, k))
            a = np.float32(y * np.float32(6.0))
            for amax in (a, np.nextafter(a, np.float32(np.inf)), np.nextafter(a, np.float32(0))):
                blk = np.linspace(-1.0, 1.0, 32, dtype=np.float32) * amax
                blk[7] = amax
                rows.append(blk)
    ties = np.zeros(32, np.float32)
    ties[:8] = [6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    ties[8:16] = -ties[:8]
    rows.append(ties)
    z = np.zeros(32, np.float32)
    z[3] = -0.0
    rows.append(z)
    sub = np.full(32, 3e-39, np.float32)            # subnormal elements; amax
    sub[0] = -1e-39                                  # 2e-38 keeps e = -127 in range
    sub[1] = 2e-38
    sub[2] = -1.4e-45
    rows.append(sub)
    big = np.full(32, 1e30, np.float32)
    big[1] = 1e-30                                   # underflows after scaling
    big[2] = -1e-45
    rows.append(big)
    w = np.stack(rows).astype(np.float32)            # [R, 32]
    pad = (-w.shape[0]) % 4
    w = np.concatenate([w, np.zeros((pad, 32), np.float32)])
    return w.reshape(-1, 128)


def test_quantizer_bit_exact_random(capi):
    banner("quantize random 512x4096 fp32/bf16/fp16")
    g = torch.Generator().manual_seed(123)
    w = torch.randn(512, 4096, generator=g) * 0.02
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        wd = w.to(dt)
        p, s, f = capi.quantize(wd.cuda())
        torch.cuda.synchronize()
        pr, sr = ox.quantize_chunk(wd)
        assert int(f.item()) == 0
        assert np.array_equal(p.cpu().numpy(), pr), dt
        assert np.array_equal(s.cpu().numpy(), sr), dt


def test_quantizer_bit_exact_adversarial(capi):
    banner("quantize adversarial")
    w = adversarial_weights()
    p, s, f = capi.quantize(torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    pr, sr = ox.quantize_chunk(w)
    assert int(f.item()) == 0
    assert np.array_equal(s.cpu().numpy(), sr)
    assert np.array_equal(p.cpu().numpy(), pr)


def test_quantizer_errors_match_reference():
    from tinyinfer_amd.quantization import quantize_chunk
    banner("quantize errors")
    w = torch.zeros(4, 64)
    w[1, 5] = float("nan")
    with pytest.raises(ValueError, match="non-finite"):
        quantize_chunk(w)
    w[1, 5] = float("inf")
    with pytest.raises(ValueError, match="non-finite"):
        quantize_chunk(w)
    w = torch.full((4, 64), 1e-44)
    with pytest.raises(ValueError, match="exponent"):
        quantize_chunk(w)
    with pytest.raises(ValueError):
        quantize_chunk(torch.zeros(4, 48))
    # the flags word is cleared per call: a good call after a bad one passes
    p, s = quantize_chunk(torch.ones(4, 64))
    assert p.device.type == "cpu"
    pr, sr = ox.quantize_chunk(torch.ones(4, 64))
    assert np.array_equal(p.numpy(), pr) and np.array_equal(s.numpy(), sr)


def test_roundtrip_device_codec_full_size(capi):
    """quantize -> dequantize on the GPU at an 8B weight shape: dequant is a
    fixed point of quantize (values), checked entirely on the device."""
    banner("codec roundtrip 12288x4096")
    g = torch.Generator(device="cuda").manual_seed(1000)
    w = torch.randn(12288, 4096, generator=g, device="cuda") * 0.02
    p, s, f = capi.quantize(w)
    d = capi.dequant(p, s, torch.float32)
    p2, s2, f2 = capi.quantize(d)
    d2 = capi.dequant(p2, s2, torch.float32)
    torch.cuda.synchronize()
    assert int(f.item()) == 0 and int(f2.item()) == 0
    assert torch.equal(d.view(torch.int32), d2.view(torch.int32))
    # error bound: |deq - w| <= 2^e (half the widest grid gap, 2, times 2^e / 2... <= 1 * 2^e)
    sc = torch.ldexp(torch.ones_like(s, dtype=torch.float32), s.to(torch.int32) - 127)
    err = ((d - w).abs().reshape(12288, 128, 32) / sc.unsqueeze(-1)).max()
    assert float(err) <= 1.0
