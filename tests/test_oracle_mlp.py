"""Pins the CPU oracle's MLP forms (oracle/mlp.py): an independent pure-Python
brute force on tiny shapes (decodes nibbles itself from the packed bytes,
no shared code with oracle.mxfp4), exact power-of-two scale invariance,
permutation invariance, and zero weights."""

import math

import numpy as np
import pytest
import torch

from oracle import mlp as om
from oracle import mxfp4 as ox


def make_mlp(m, h, i, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, h, generator=g).to(dtype)
    mats = []
    for rows, cols in ((i, h), (i, h), (h, i)):
        w = torch.randn(rows, cols, generator=g) * 0.02
        mats.extend(ox.quantize_chunk(w))
    return x, mats


def brute_force(x, mats):
    """Pure-Python loops straight from the packed bytes."""
    table = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]

    def weight(packed, scale, r, k):
        byte = int(packed[r, k // 2])
        code = (byte >> 4) if (k % 2) else (byte & 15)
        v = table[code & 7] * math.ldexp(1.0, int(scale[r, k // 32]) - 127)
        return -v if code & 8 else v

    gp, gs, up, us, dp, ds = mats
    xs = x.to(torch.float64).tolist()
    m, h = len(xs), len(xs[0])
    i = gp.shape[0]
    out = [[0.0] * h for _ in range(m)]
    for t in range(m):
        hid = []
        for r in range(i):
            g = sum(xs[t][k] * weight(gp, gs, r, k) for k in range(h))
            u = sum(xs[t][k] * weight(up, us, r, k) for k in range(h))
            hid.append(g / (1.0 + math.exp(-g)) * u)
        for n in range(h):
            out[t][n] = sum(hid[r] * weight(dp, ds, n, r) for r in range(i))
    return np.array(out)


def test_fp64_matches_brute_force():
    x, mats = make_mlp(2, 32, 64, seed=5)
    bf = brute_force(x, mats)
    got = om.mlp_fp64(x, *mats)
    assert np.allclose(got, bf, rtol=1e-12, atol=1e-15)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_reference_and_kernel_semantics_close_to_fp64(dtype):
    x, mats = make_mlp(3, 64, 96, seed=1, dtype=dtype)
    truth = om.mlp_fp64(x, *mats)
    for fn in (om.mlp_reference, om.mlp_kernel_semantics):
        out = fn(x, *mats)
        assert out.dtype == dtype and out.shape == (3, 64)
        st = om.parity_stats(out, torch.from_numpy(truth))
        assert om.within_tolerance(st), (fn.__name__, st)
    # kernel semantics rounds twice (h, out); each bf16 rounding is <= 2**-9
    st = om.parity_stats(om.mlp_kernel_semantics(x, *mats), torch.from_numpy(truth))
    assert st["rel_max_err"] < 2e-2 and st["cos"] > 0.99999


def test_down_scale_plus_one_doubles_output_exactly():
    x, mats = make_mlp(4, 64, 128, seed=2)
    gp, gs, up, us, dp, ds = mats
    base = om.mlp_reference(x, *mats)
    dbl = om.mlp_reference(x, gp, gs, up, us, dp, (ds + 1).astype(np.uint8))
    assert torch.equal(dbl, base * 2)


def test_intermediate_block_permutation_invariance():
    x, mats = make_mlp(3, 64, 128, seed=3)
    gp, gs, up, us, dp, ds = mats
    i = gp.shape[0]
    perm_blocks = np.array([2, 0, 3, 1])               # permute 32-feature blocks
    rows = np.concatenate([np.arange(32) + 32 * b for b in perm_blocks])
    dp_b = dp.reshape(dp.shape[0], i // 32, 16)[:, perm_blocks].reshape(dp.shape)
    ds_b = ds[:, perm_blocks]
    a = om.mlp_fp64(x, *mats)
    b = om.mlp_fp64(x, gp[rows], gs[rows], up[rows], us[rows], dp_b, ds_b)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-14)


def test_zero_gate_gives_zero_output():
    x, mats = make_mlp(2, 64, 64, seed=4)
    gp, gs, up, us, dp, ds = mats
    zero = np.zeros_like(gp)
    out = om.mlp_reference(x, zero, gs, up, us, dp, ds)
    assert torch.count_nonzero(out) == 0


def test_parity_stats_detects_a_transposed_operand():
    """A plausible mistake (down applied transposed on a square shape) must
    fail the task's tolerance."""
    x, mats = make_mlp(4, 64, 64, seed=6)
    gp, gs, up, us, dp, ds = mats
    ref = om.mlp_reference(x, *mats)
    wd = om.dequant_weight(dp, ds, torch.float32)
    g = torch.nn.functional.linear(x.float(), om.dequant_weight(gp, gs, torch.float32))
    u = torch.nn.functional.linear(x.float(), om.dequant_weight(up, us, torch.float32))
    wrong = torch.nn.functional.linear(torch.nn.functional.silu(g) * u, wd.T.contiguous())
    assert not om.within_tolerance(om.parity_stats(wrong, ref))
    right = torch.nn.functional.linear(torch.nn.functional.silu(g) * u, wd)
    assert om.within_tolerance(om.parity_stats(right, ref))


# ---------------------------------------------------------------- RMSNorm
# rmsnorm_reference restates tinyinfer/csrc/rmsnorm.cu:10-54.  Pinned by an
# fp64 brute force (within one bf16 rounding), by torch's own rms_norm
# routine, by exact power-of-two scale invariance at eps = 0, and by a planted
# mistake (mean over the wrong length) that the fp64 check must reject.

def _rms_fp64(x, w, eps):
    x64 = x.to(torch.float64)
    return w.to(torch.float64) * x64 / torch.sqrt((x64 * x64).mean(-1, keepdim=True) + eps)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rmsnorm_reference_matches_fp64_within_one_rounding(dtype):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(5, 256, generator=g).to(dtype)
    w = (1.0 + 0.1 * torch.randn(256, generator=g)).to(dtype)
    out = om.rmsnorm_reference(x, w, 1e-6).to(torch.float64)
    ref = _rms_fp64(x, w, 1e-6)
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    assert float(((out - ref).abs() / ref.abs().clamp_min(1e-30)).max()) <= ulp


def test_rmsnorm_reference_matches_torch_rms_norm():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(7, 512, generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn(512, generator=g)).to(torch.bfloat16)
    lib = torch.nn.functional.rms_norm(x.float(), (512,), w.float(), 1e-6).to(torch.bfloat16)
    out = om.rmsnorm_reference(x, w, 1e-6)
    diff = (out.float() - lib.float()).abs()
    # same math, fp32 summation orders differ: at most one bf16 ulp, almost always equal
    assert float((diff / lib.float().abs().clamp_min(1e-30)).max()) <= 2.0 ** -7
    assert float((out == lib).float().mean()) > 0.99


def test_rmsnorm_reference_power_of_two_invariance():
    g = torch.Generator().manual_seed(13)
    x = torch.randn(3, 128, generator=g).to(torch.bfloat16)
    w = torch.randn(128, generator=g).to(torch.bfloat16)
    a = om.rmsnorm_reference(x, w, 0.0)
    b = om.rmsnorm_reference(x * 8, w, 0.0)       # x and sum scale by 8 and 64: inv by 1/8
    assert torch.equal(a, b)


def test_rmsnorm_planted_mistake_is_caught():
    g = torch.Generator().manual_seed(14)
    x = torch.randn(4, 256, generator=g).to(torch.bfloat16)
    w = torch.ones(256, dtype=torch.bfloat16)
    x32 = x.float()
    wrong = (x32 * torch.rsqrt((x32 * x32).sum(-1, keepdim=True) / 255.0 + 1e-6)).to(torch.bfloat16)
    ref = _rms_fp64(x, w, 1e-6)
    rel = float(((wrong.to(torch.float64) - ref).abs() / ref.abs().clamp_min(1e-30)).max())
    assert rel > 2.0 ** -9                        # a length off by one is visible above the rounding


def test_decoder_mlp_reference_composition():
    """x + mlp(rmsnorm(x)): with zero gate weights the MLP is zero and the
    output is x itself; otherwise it is the two reference ops composed."""
    x, mats = make_mlp(3, 64, 96, seed=15)
    w = (1.0 + 0.1 * torch.randn(64, generator=torch.Generator().manual_seed(16))).to(torch.bfloat16)
    gp, gs, up, us, dp, ds = mats
    zero = np.zeros_like(gp)
    same = om.decoder_mlp_reference(x, w, 1e-6, zero, gs, up, us, dp, ds)
    assert torch.equal(same, x)
    out = om.decoder_mlp_reference(x, w, 1e-6, *mats)
    y = om.mlp_reference(om.rmsnorm_reference(x, w, 1e-6), *mats)
    assert torch.equal(out, (x.float() + y.float()).to(torch.bfloat16))
