"""GPU parity sweep of the AUTO path over every token count from 1 to 70 and a
few prefill sizes, in bf16 and fp16, at the Qwen3-0.6B and Qwen3-1.7B MLP
shapes: whichever kernel family the dispatch picks for a count (row,
row-pair, stream, tile, ring GEMM, and their per-stage mixes), the MLP output
is held to the task's bar against a plain-PyTorch fp32 reference of the
dequant-then-matmul path on the same device (h rounded to the activation
dtype as the reference's tmp buffer does).  Weights come from the device
quantizer with the workload seeds."""

import pytest
import torch

from oracle import mlp as om
from tests.helpers import banner, torch_fp32_reference

pytestmark = pytest.mark.gpu

COUNTS = list(range(1, 71)) + [96, 97, 130, 257]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("h,i", [(1024, 3072), (2048, 6144)])
def test_auto_path_every_token_count(h, i, dtype):
    from tinyinfer_amd import capi
    from tinyinfer_amd.workloads import quantized_weights
    banner(f"sweep h={h} i={i} {dtype}")
    mats = quantized_weights(h, i, layer=3, generator="cuda")
    worst = 0.0
    for m in COUNTS:
        g = torch.Generator(device="cuda").manual_seed(1000 + m)
        x = torch.randn(m, h, generator=g, device="cuda").to(dtype)
        out = capi.mlp_forward(x, *mats)
        st = om.parity_stats(out, torch_fp32_reference(x, *mats))
        assert om.within_tolerance(st), (m, st)
        worst = max(worst, st["rel_max_err"])
    print(f"h={h} i={i} {dtype}: worst rel_max_err {worst:.3e} over {len(COUNTS)} token counts")
