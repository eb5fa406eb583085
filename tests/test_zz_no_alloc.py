"""GPU: the allocation-free entry point tinyinfer_mlp_forward_mxfp4_noalloc,
called through the C ABI, against tinyinfer_mlp_forward_mxfp4 on the same
inputs.  Two calls in a row per case, the second with fewer tokens (the
fixed scratch array keeps the first call's contents): the split-K tile
kernels (8B at 64 then 16 tokens, 32B at 64 then 3), the GEMM path with a
split K (8B at 512 then 160 tokens), and a call whose tile kernels would
need more than the array holds, which is refused with TI_ERR_SCRATCH before
any launch."""

import ctypes

import pytest
import torch

from oracle import mlp as om
from tests.helpers import banner

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


def _call(capi, fn, x, w, out, tmp):
    n, h = x.shape
    i = w[0].shape[0]
    st = fn(x.data_ptr(), *[t.data_ptr() for t in w], n, h, i, tmp.data_ptr(), out.data_ptr(), capi.TI_DTYPE_BF16,
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return st


def _pair(capi, x, w):
    lib = capi.lib()
    n, h = x.shape
    i = w[0].shape[0]
    outs = []
    for fn in (lib.tinyinfer_mlp_forward_mxfp4, lib.tinyinfer_mlp_forward_mxfp4_noalloc):
        out = torch.full((n, h), 3.0, dtype=torch.bfloat16, device="cuda")
        tmp = torch.full((n, i), 3.0, dtype=torch.bfloat16, device="cuda")
        st = _call(capi, fn, x, w, out, tmp)
        assert st == capi.TI_OK, capi.status_string(st)
        outs.append((out, tmp))
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("shape,ms,bitwise", [
    ((4096, 12288), (64, 16), True),     # tile kernels: split-K partials in scratch
    ((5120, 25600), (64, 3), True),      # 32B gate_up at 64 tokens: 62.5 MiB of partials
    ((4096, 12288), (512, 160), False),  # GEMM path, K split only as far as scratch holds
])
def test_noalloc_matches_allocating_entry(capi, shape, ms, bitwise):
    from tinyinfer_amd.workloads import activations, quantized_weights
    h, i = shape
    w = quantized_weights(h, i, layer=3)
    for m in ms:
        banner(f"noalloc h={h} i={i} m={m}")
        x = activations(m, h, seed=40 + m)
        (a, ta), (b, tb) = _pair(capi, x, w)
        st = om.parity_stats(b.cpu(), a.cpu())
        assert st["finite"] and st["rel_max_err"] < 5e-3 and st["cos"] > 0.99999, (m, st)
        assert om.within_tolerance(st)
        if bitwise:
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), m
            assert torch.equal(ta.view(torch.int16), tb.view(torch.int16)), m


def test_noalloc_refuses_calls_beyond_its_scratch(capi):
    """hidden 8192, intermediate 32768 at 64 tokens: the tile gate_up would
    keep 8 K ranges x 64 tokens x 2 x 32768 rows of fp32 partials (128 MiB)."""
    banner("noalloc refuses 128 MiB of partials")
    h, i, m = 8192, 32768, 64
    w = [torch.zeros((i, h // 2), dtype=torch.uint8, device="cuda"),
         torch.full((i, h // 32), 127, dtype=torch.uint8, device="cuda"),
         torch.zeros((i, h // 2), dtype=torch.uint8, device="cuda"),
         torch.full((i, h // 32), 127, dtype=torch.uint8, device="cuda"),
         torch.zeros((h, i // 2), dtype=torch.uint8, device="cuda"),
         torch.full((h, i // 32), 127, dtype=torch.uint8, device="cuda")]
    x = torch.zeros((m, h), dtype=torch.bfloat16, device="cuda")
    out = torch.full((m, h), 3.0, dtype=torch.bfloat16, device="cuda")
    tmp = torch.full((m, i), 3.0, dtype=torch.bfloat16, device="cuda")
    st = _call(capi, capi.lib().tinyinfer_mlp_forward_mxfp4_noalloc, x, w, out, tmp)
    torch.cuda.synchronize()
    assert st == capi.TI_ERR_SCRATCH, capi.status_string(st)
    assert "scratch" in capi.status_string(st)
    assert bool((out == 3.0).all()) and bool((tmp == 3.0).all())
    # a smaller call right after it runs normally
    (a, _), (b, _) = _pair(capi, x[:8].contiguous(), w)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
