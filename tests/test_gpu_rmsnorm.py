"""GPU: the decoder layer's MLP half with the RMSNorm prologue fused
(``tinyinfer_mlp_forward_mxfp4_rmsnorm``: x + MLP(RMSNorm(x)), the reference's
``post_attention_layernorm -> mlp -> residual add``, tinyinfer/models/qwen3.py:210-219)
and the RMSNorm op alone (``tinyinfer_rmsnorm`` / ``_C.rmsnorm_forward``, the
reference's tinyinfer/csrc/rmsnorm.cu).

Checked against the CPU oracle's restatement of the reference (oracle/mlp.py
``rmsnorm_reference`` / ``decoder_mlp_reference``) at the task's bar, and
internally: the normalized rows match the oracle within one rounding (fp32
sums in a different order can move a value across a rounding boundary), and
on every path the output equals, bit for bit, the plain MLP with residual run
on the normalized rows the call itself produced."""

import pytest
import torch

from oracle import mlp as om
from tests.helpers import assert_parity, banner, make_case, to_dev

pytestmark = pytest.mark.gpu

AUTO, SKINNY, GEMM, DECODE = 0, 1, 2, 3
EPS = 1e-6


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


def norm_weight(h, dtype, seed=3):
    g = torch.Generator().manual_seed(seed)
    return (1.0 + 0.1 * torch.randn(h, generator=g)).to(dtype)


def assert_within_one_rounding(out, ref, what):
    """Every value equal or one rounding step apart, almost all equal."""
    o, r = out.cpu().float(), ref.cpu().float()
    ulp = 2.0 ** -7 if out.dtype == torch.bfloat16 else 2.0 ** -10
    rel = ((o - r).abs() / r.abs().clamp_min(1e-30)).max()
    same = (out.cpu() == ref.cpu()).float().mean()
    assert float(rel) <= ulp and float(same) > 0.99, f"{what}: max rel {float(rel):.3g}, equal {float(same):.4f}"


@pytest.mark.parametrize("rows,h,dtype", [(1, 4096, torch.bfloat16), (7, 5120, torch.bfloat16),
                                          (300, 1024, torch.bfloat16), (5, 2048, torch.float16)])
def test_rmsnorm_op(capi, rows, h, dtype):
    banner(f"rmsnorm rows={rows} h={h} {dtype}")
    x = torch.randn(rows, h, generator=torch.Generator().manual_seed(rows + h)).to(dtype)
    w = norm_weight(h, dtype)
    out = capi.rmsnorm(x.cuda(), w.cuda(), EPS)
    torch.cuda.synchronize()
    assert_within_one_rounding(out, om.rmsnorm_reference(x, w, EPS), f"rmsnorm {rows}x{h}")


def test_rmsnorm_torch_extension(capi):
    from tinyinfer_amd.extension import load_extension
    banner("rmsnorm _C")
    C = load_extension()
    x = torch.randn(2, 3, 1024, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).cuda()
    w = norm_weight(1024, torch.bfloat16).cuda()
    out = C.rmsnorm_forward(x, w, EPS)
    torch.cuda.synchronize()
    assert out.shape == x.shape
    assert torch.equal(out.view(torch.int16), capi.rmsnorm(x, w, EPS).view(torch.int16))
    with pytest.raises(RuntimeError, match="weight size must match input last dimension"):
        C.rmsnorm_forward(x, w[:512], EPS)
    with pytest.raises(RuntimeError, match="RMSNorm supports fp16 and bf16 only"):
        C.rmsnorm_forward(x.float(), w.float(), EPS)


@pytest.mark.parametrize("m,h,i,path,dtype", [
    (1, 1024, 3072, AUTO, torch.bfloat16),        # row kernels, norm in gate_up's prologue
    (1, 4096, 12288, AUTO, torch.float16),        # the same, fp16 (x normalized and kept as fp16)
    (2, 2048, 6144, AUTO, torch.float16),         # row-pair kernels, norm in the prologue, fp16
    (4, 2048, 6144, AUTO, torch.float16),         # stream kernels (gate_up) and row-pair (down), fp16
    (8, 1024, 3072, SKINNY, torch.bfloat16),      # stream kernels at their token limit
    (8, 2560, 3072, SKINNY, torch.bfloat16),      # x beyond the preload registers: norm from LDS
    (2, 1024, 3072, DECODE, torch.bfloat16),      # norm kernel + fused decode kernel
    (24, 1024, 1536, SKINNY, torch.bfloat16),     # norm kernel + skinny kernels
    (300, 1024, 1536, GEMM, torch.bfloat16),      # norm kernel + ring GEMM
    (130, 1024, 1536, GEMM, torch.float16),       # norm kernel + ring GEMM, fp16
])
def test_decoder_mlp_half(capi, m, h, i, path, dtype):
    banner(f"rmsnorm mlp m={m} h={h} i={i} path={path} {dtype}")
    x, mats = make_case(m, h, i, seed=m + i, dtype=dtype)
    w = norm_weight(h, dtype)
    xd, md = to_dev(x, mats)
    wd = w.cuda()
    out, xn = capi.mlp_forward_rmsnorm(xd, wd, EPS, *md, path=path)
    torch.cuda.synchronize()
    # the oracle: the reference's ops composed on the CPU
    assert_parity(out.cpu(), om.decoder_mlp_reference(x, w, EPS, *mats), f"m={m} path={path}")
    assert_within_one_rounding(xn, om.rmsnorm_reference(x, w, EPS), f"xn m={m} path={path}")
    # bit-identical to the unfused composition on the same normalized rows
    plain = capi.mlp_forward(xn, *md, path=path, residual=xd)
    inplace = xd.clone()
    capi.mlp_forward_rmsnorm(inplace, wd, EPS, *md, out=inplace, path=path)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
    assert torch.equal(inplace.view(torch.int16), out.view(torch.int16))


def test_decoder_mlp_half_qwen3_8b_decode(capi):
    """BASELINE's 8B decode shape on the fused prologue (M = 1), and the
    torch extension's entry point."""
    from tinyinfer_amd.extension import load_extension
    from tinyinfer_amd.workloads import activations, quantized_weights
    banner("rmsnorm mlp 8B m=1")
    mats = quantized_weights(4096, 12288, layer=0)
    x = activations(1, 4096)
    w = norm_weight(4096, torch.bfloat16).cuda()
    out, xn = capi.mlp_forward_rmsnorm(x, w, EPS, *mats)
    ref = om.decoder_mlp_reference(x.cpu(), w.cpu(), EPS, *[t.cpu() for t in mats])
    assert_parity(out.cpu(), ref, "8B m=1")
    via_c = load_extension().mlp_forward_mxfp4_rmsnorm(x, w, EPS, *mats)
    torch.cuda.synchronize()
    assert torch.equal(via_c.view(torch.int16), out.view(torch.int16))


def test_decoder_mlp_half_refusals(capi):
    banner("rmsnorm mlp refusals")
    x, mats = make_case(2, 512, 1024, seed=1)
    xd, md = to_dev(x, mats)
    w = norm_weight(512, torch.bfloat16).cuda()
    base = torch.empty(513, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(capi.TinyInferError) as e:
        capi.mlp_forward_rmsnorm(xd, base[1:], EPS, *md)          # misaligned norm weight
    assert e.value.status == capi.TI_ERR_MISALIGNED
    L = capi.lib()
    st = L.tinyinfer_mlp_forward_mxfp4_rmsnorm(
        xd.data_ptr(), w.data_ptr(), EPS, *[t.data_ptr() for t in md], 2, 512, 1024, None,
        torch.empty(2, 1024, dtype=torch.bfloat16, device="cuda").data_ptr(),
        torch.empty(2, 512, dtype=torch.bfloat16, device="cuda").data_ptr(), capi.TI_DTYPE_BF16, AUTO, None)
    assert st == capi.TI_ERR_INVALID_ARG                           # no xn workspace
    with pytest.raises(ValueError):
        capi.mlp_forward_rmsnorm(xd, w[:256], EPS, *md)
