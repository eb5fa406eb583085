"""GPU parity of BASELINE's Qwen3-32B MLP stack workload (hidden 5120,
intermediate 25600, residual add between layers), on its first two layers:
``x <- x + MLP_l(x)`` through the C ABI (AUTO path; the residual fused into
the down epilogue in place, or added by torch) against the same
composition over a plain PyTorch fp32 reference of each MLP, with the
residual rounded to bf16 after every layer as the reference does."""

import pytest
import torch

from tests.helpers import assert_parity, banner, torch_fp32_reference

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,fused", [(1, True), (3, True), (160, True), (1, False), (160, False)])
def test_qwen3_32b_two_layer_stack(m, fused):
    from tinyinfer_amd import capi
    from tinyinfer_amd.workloads import SHAPES, activations, mlp_stack_step, quantized_weights
    shp = SHAPES["qwen3-32b"]
    banner(f"32B stack m={m} fused={fused}")
    layers = [quantized_weights(shp.hidden, shp.inter, layer=l) for l in range(2)]
    x0 = activations(m, shp.hidden)
    x = x0.clone()
    out = torch.empty_like(x0)
    tmp = torch.empty((m, shp.inter), dtype=x0.dtype, device="cuda")
    mlp_stack_step(capi, x, layers, out, tmp, fused_residual=fused)
    ref = x0.clone()
    for w in layers:
        ref = (ref.float() + torch_fp32_reference(ref, *w).float()).to(torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.isfinite(x.float()).all()
    assert_parity(x, ref, f"32B stack m={m}")
    # the MLP part alone (the residual dominates the sum)
    assert_parity(x.float() - x0.float(), ref.float() - x0.float(), f"32B stack m={m} increments")
