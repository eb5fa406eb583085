"""GPU: the two fusions beyond the reference's single call.

* residual + MLP(x) with the add in the down stage's epilogue
  (``tinyinfer_mlp_forward_mxfp4_residual``): on every kernel path it equals,
  bit for bit, the plain MLP followed by torch's bf16/fp16 add (what the
  reference's ``hidden_states = residual + hidden_states`` computes), also
  in place (output written over the residual).
* One MXFP4 linear on the down-stage kernels (``tinyinfer_mxfp4_linear``):
  against exact sums of the oracle's dequantized weights rounded once, for
  the Qwen3 qkv/o-proj/lm-head-like shapes, plus its residual form and the
  ``LinearMXFP4.forward`` / torch-extension wrappers."""

import pytest
import torch

from oracle import mxfp4 as ox
from tests.helpers import assert_parity, banner, make_case, to_dev
from tests.test_gpu_stream import check_close, down_semantics

pytestmark = pytest.mark.gpu

AUTO, SKINNY, GEMM, DECODE = 0, 1, 2, 3


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


def _added(res, y):
    return (res.float() + y.float()).to(res.dtype)


@pytest.mark.parametrize("m,h,i,path,dtype", [
    (1, 1024, 3072, AUTO, torch.bfloat16),        # stream kernels
    (4, 2048, 6144, AUTO, torch.float16),         # stream kernels, fp16
    (2, 1024, 3072, DECODE, torch.bfloat16),      # fused decode kernel
    (24, 1024, 1536, SKINNY, torch.bfloat16),     # skinny kernels
    (16, 1024, 3072, AUTO, torch.bfloat16),       # tile kernels: one-launch gate_up, down + reduce
    (40, 2048, 6144, SKINNY, torch.bfloat16),     # tile kernels: both stages split + reduce
    (300, 1024, 1536, GEMM, torch.bfloat16),      # ring GEMM, unsplit down
    (160, 2048, 6144, GEMM, torch.bfloat16),      # ring GEMM, split-K down + reduce
    (130, 1024, 1536, GEMM, torch.float16),       # register-staged GEMM (fp16)
])
def test_residual_mlp_equals_mlp_then_add(capi, m, h, i, path, dtype):
    banner(f"residual mlp m={m} h={h} i={i} path={path} {dtype}")
    x, mats = make_case(m, h, i, seed=m + h, dtype=dtype)
    xd, md = to_dev(x, mats)
    res = torch.randn(m, h, generator=torch.Generator().manual_seed(7)).to(dtype).cuda()
    plain = capi.mlp_forward(xd, *md, path=path)
    fused = capi.mlp_forward(xd, *md, path=path, residual=res)
    inplace = res.clone()
    capi.mlp_forward(xd, *md, path=path, residual=inplace, out=inplace)
    torch.cuda.synchronize()
    want = _added(res, plain)
    assert torch.equal(fused.view(torch.int16), want.view(torch.int16))
    assert torch.equal(inplace.view(torch.int16), want.view(torch.int16))


def test_residual_torch_extension(capi):
    from tinyinfer_amd.extension import load_extension
    banner("residual torch extension")
    x, mats = make_case(3, 512, 1024, seed=11)
    xd, md = to_dev(x, mats)
    res = torch.randn(3, 512, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).cuda()
    ext = load_extension()
    a = ext.mlp_forward_mxfp4_residual(xd, *md, res)
    b = _added(res, ext.mlp_forward_mxfp4(xd, *md))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    with pytest.raises(RuntimeError, match="residual must match"):
        ext.mlp_forward_mxfp4_residual(xd, *md, res[:2].contiguous())


@pytest.mark.parametrize("m,k,r,dtype", [
    (1, 4096, 6144, torch.bfloat16), (7, 4096, 4096, torch.bfloat16), (200, 2048, 2048, torch.bfloat16),
    (3, 1024, 151936, torch.bfloat16), (96, 1536, 512, torch.bfloat16), (16, 4096, 4096, torch.bfloat16),
    (48, 2048, 2048, torch.bfloat16),
    # fp16 activations through the same kernel families
    (1, 4096, 6144, torch.float16), (2, 4096, 4096, torch.float16), (5, 2048, 2048, torch.float16),
    (16, 4096, 4096, torch.float16), (300, 2048, 2048, torch.float16)])
def test_linear_against_exact_sums(capi, m, k, r, dtype):
    banner(f"linear m={m} k={k} r={r} {dtype}")
    g = torch.Generator().manual_seed(k + r)
    w = torch.randn(r, k, generator=g) * 0.02
    p, s = ox.quantize_chunk(w)
    x = torch.randn(m, k, generator=g).to(dtype)
    pd, sd = torch.from_numpy(p).cuda(), torch.from_numpy(s).cuda()
    y = capi.linear(x.cuda(), pd, sd)
    torch.cuda.synchronize()
    check_close(y.cpu(), down_semantics(x, p, s), f"linear {m}x{k}->{r}")
    res = torch.randn(m, r, generator=g).to(dtype).cuda()
    yr = capi.linear(x.cuda(), pd, sd, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(yr.view(torch.int16), _added(res, y).view(torch.int16))


def test_linear_module_forward():
    from tinyinfer_amd.linear import LinearMXFP4
    banner("LinearMXFP4.forward")
    g = torch.Generator().manual_seed(5)
    lin = LinearMXFP4(1024, 2048, bias=True, dtype=torch.bfloat16, device="cuda")
    w = torch.randn(2048, 1024, generator=g) * 0.02
    p, s = ox.quantize_chunk(w)
    lin.weight_packed.data.copy_(torch.from_numpy(p))
    lin.weight_scale.data.copy_(torch.from_numpy(s))
    lin.bias.data.copy_(torch.randn(2048, generator=g).to(torch.bfloat16))
    x = torch.randn(2, 3, 1024, generator=g).to(torch.bfloat16)
    y = lin(x.cuda())
    assert y.shape == (2, 3, 2048) and y.dtype == torch.bfloat16
    ref = down_semantics(x.reshape(6, 1024), p, s).float() + lin.bias.detach().cpu().float()
    assert_parity(y.reshape(6, 2048).cpu(), ref, "LinearMXFP4.forward")
