"""Shared helpers for the GPU parity tests (imported by test modules)."""

from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import mlp as om
from oracle import mxfp4 as ox


def banner(msg: str) -> None:
    """Name the case before a GPU step, flushed, so a crash log says where it was."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def make_case(m, h, i, seed=0, dtype=torch.bfloat16, std=0.02):
    """Seeded CPU inputs quantized by the oracle: (x, [gp, gs, up, us, dp, ds]) numpy/torch on CPU."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, h, generator=g).to(dtype)
    mats = []
    for rows, cols in ((i, h), (i, h), (h, i)):
        w = torch.randn(rows, cols, generator=g) * std
        mats.extend(ox.quantize_chunk(w))
    return x, mats


def to_dev(x, mats):
    return x.cuda(), [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in mats]


def assert_parity(out, ref, what=""):
    st = om.parity_stats(out, ref)
    assert om.within_tolerance(st), f"{what}: {st}"
    return st


def torch_fp32_reference(x, gp, gs, up, us, dp, ds, acc=torch.float32):
    """GPU fp32 reference of the dequant-then-matmul path, built from plain
    torch ops (table lookup + ldexp, as the reference dequantize_chunk does),
    sharing no code with the HIP kernels. h is rounded to x.dtype as in the
    reference (its tmp buffer has the activation dtype).  ``acc=float64``
    gives the same composition with float64 sums (a second reference that
    differs from the first only in its summation error)."""
    lut = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], device=x.device)

    def deq(p, s):
        codes = torch.stack([p & 15, p >> 4], dim=-1).reshape(p.shape[0], -1)
        v = lut[(codes & 7).long()]
        v = torch.where((codes & 8) != 0, -v, v)
        sc = torch.ldexp(torch.ones_like(s, dtype=torch.float32), s.to(torch.int32) - 127)
        return (v.reshape(p.shape[0], -1, 32) * sc.unsqueeze(-1)).reshape(p.shape[0], -1).to(acc)

    xf = x.to(acc)
    g = xf @ deq(gp, gs).T
    u = xf @ deq(up, us).T
    h = (torch.nn.functional.silu(g) * u).to(x.dtype).to(acc)
    return (h @ deq(dp, ds).T).to(x.dtype)
