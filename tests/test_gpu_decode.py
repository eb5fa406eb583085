"""GPU parity of the fused single-launch decode kernel (TI_PATH_DECODE):
gate_up, SiLU*up and down in one launch; workgroups publish their rows of h
and an epoch flag, and start down once every flag carries this launch's
epoch.

Checked against the CPU oracle (the reference's torch dequant-then-matmul
path) at the task's bar, against the two-launch paths, for both activation
dtypes, every token count it accepts (1..4), the BASELINE shapes, repeated
calls and graph replays (the epoch must advance by exactly one per launch),
and its refusal of calls it does not support."""

import numpy as np
import pytest
import torch

from oracle import mlp as om
from tests.helpers import assert_parity, banner, make_case, to_dev, torch_fp32_reference

pytestmark = pytest.mark.gpu

DECODE, SKINNY = 3, 1


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


@pytest.fixture(autouse=True)
def no_barrier_timeouts(capi):
    yield
    assert capi.decode_barrier_timeouts() == 0


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_decode_token_counts_small_shape(capi, m):
    banner(f"decode m={m} h=512 i=1536")
    x, mats = make_case(m, 512, 1536, seed=300 + m)
    ref = om.mlp_reference(x, *mats)
    xd, md = to_dev(x, mats)
    out = capi.mlp_forward(xd, *md, path=DECODE)
    torch.cuda.synchronize()
    assert out.shape == ref.shape and out.dtype == torch.bfloat16
    assert_parity(out.cpu(), ref, f"decode m={m}")
    # against exact sums with the kernel rounding points: a few bf16 ulps
    st = om.parity_stats(out.cpu(), om.mlp_kernel_semantics(x, *mats))
    assert st["rel_max_err"] < 5e-3 and st["cos"] > 0.99999, st


@pytest.mark.parametrize("h,i", [(1536, 512), (512, 4096), (2560, 1024), (1024, 5120), (768, 2048),
                                 (256, 2304)])
def test_decode_shapes(capi, h, i):
    """Waves with no K segment or a partial unit, fewer down row groups than
    workgroups, several gate_up row groups per workgroup; shapes outside the
    kernel's range (K not a multiple of 512, too many down units) must be
    refused, never run wrong."""
    for m in (1, 3):
        banner(f"decode shape h={h} i={i} m={m}")
        x, mats = make_case(m, h, i, seed=h + i + m)
        ref = om.mlp_reference(x, *mats)
        xd, md = to_dev(x, mats)
        try:
            out = capi.mlp_forward(xd, *md, path=DECODE)
        except capi.TinyInferError as e:
            assert e.status == capi.TI_ERR_UNSUPPORTED
            continue
        assert_parity(out.cpu(), ref, f"h={h} i={i} m={m}")


def test_decode_tmp_holds_h(capi):
    """The fused path leaves SiLU(g)*u in tmp, as the reference's tmp buffer."""
    banner("decode tmp")
    x, mats = make_case(2, 512, 1024, seed=9)
    xd, md = to_dev(x, mats)
    tmp = torch.empty((2, 1024), dtype=torch.bfloat16, device="cuda")
    capi.mlp_forward(xd, *md, tmp=tmp, path=DECODE)
    tmp_sk = capi.gate_up(xd, *md[:4], path=SKINNY)
    torch.cuda.synchronize()
    st = om.parity_stats(tmp.cpu(), tmp_sk.cpu())
    assert st["rel_max_err"] < 1e-2 and st["cos"] > 0.99999, st


@pytest.mark.parametrize("m", [1, 4])
def test_decode_config1_qwen3_1p7b(capi, m):
    banner(f"decode 1.7B m={m}")
    x, mats = make_case(m, 2048, 6144, seed=100 + m)
    ref = om.mlp_reference(x, *mats)
    xd, md = to_dev(x, mats)
    out = capi.mlp_forward(xd, *md, path=DECODE)
    assert_parity(out.cpu(), ref, f"1.7B m={m}")
    auto = capi.mlp_forward(xd, *md)          # the streaming kernels at this size
    assert_parity(auto.cpu(), ref, f"1.7B m={m} auto")


def test_decode_config0_qwen3_0p6b(capi):
    banner("decode 0.6B m=4")
    x, mats = make_case(4, 1024, 3072, seed=1)
    xd, md = to_dev(x, mats)
    out = capi.mlp_forward(xd, *md, path=DECODE)
    assert_parity(out.cpu(), om.mlp_reference(x, *mats), "0.6B m=4")


@pytest.mark.parametrize("m", [1, 4])
def test_decode_qwen3_8b(capi, m):
    from tinyinfer_amd.workloads import activations, quantized_weights
    banner(f"decode 8B m={m}")
    mats = quantized_weights(4096, 12288, layer=0)
    x = activations(m, 4096)
    ref = torch_fp32_reference(x, *mats)
    out = capi.mlp_forward(x, *mats, path=DECODE)
    assert_parity(out, ref, f"decode 8B m={m}")
    sk = capi.mlp_forward(x, *mats, path=SKINNY)
    st = om.parity_stats(out, sk)
    assert st["rel_max_err"] < 1e-2 and st["cos"] > 0.99999, st


def test_decode_qwen3_32b_m1(capi):
    """Qwen3-32B layer shape (hidden 5120, intermediate 25600): down's K range
    per wave (100 segments over 8 waves) is beyond the fused kernel, which
    refuses it; AUTO serves it on the two-launch path."""
    from tinyinfer_amd.workloads import activations, quantized_weights
    banner("decode 32B m=1")
    mats = quantized_weights(5120, 25600, layer=0)
    x = activations(1, 5120)
    ref = torch_fp32_reference(x, *mats)
    with pytest.raises(capi.TinyInferError) as e:
        capi.mlp_forward(x, *mats, path=DECODE)
    assert e.value.status == capi.TI_ERR_UNSUPPORTED
    assert_parity(capi.mlp_forward(x, *mats), ref, "32B m=1 auto")


def test_decode_fp16(capi):
    for m in (1, 3):
        banner(f"decode fp16 m={m}")
        x, mats = make_case(m, 512, 1536, seed=60 + m, dtype=torch.float16)
        xd, md = to_dev(x, mats)
        out = capi.mlp_forward(xd, *md, path=DECODE)
        assert out.dtype == torch.float16
        assert_parity(out.cpu(), om.mlp_reference(x, *mats), f"fp16 m={m}")


def test_decode_repeated_calls_and_graph_replays(capi):
    """The flags need no reset: many calls in a row, alternating with other
    kernels, and replays of a captured graph all give the same bits."""
    banner("decode repeat + graph")
    x, mats = make_case(2, 1024, 3072, seed=5)
    xd, md = to_dev(x, mats)
    first = capi.mlp_forward(xd, *md, path=DECODE).clone()
    for i in range(50):
        out = capi.mlp_forward(xd, *md, path=DECODE)
        if i % 10 == 0:
            capi.mlp_forward(xd, *md, path=SKINNY)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), first.view(torch.int16))
    out_g = torch.empty_like(first)
    tmp_g = torch.empty((2, 3072), dtype=torch.bfloat16, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        capi.mlp_forward(xd, *md, out=out_g, tmp=tmp_g, path=DECODE)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(3):
            capi.mlp_forward(xd, *md, out=out_g, tmp=tmp_g, path=DECODE)
    for _ in range(5):
        out_g.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g.view(torch.int16), first.view(torch.int16))
        capi.mlp_forward(xd, *md, path=SKINNY)   # eager work between replays
    del g


def test_decode_refuses_what_it_does_not_support(capi):
    banner("decode refusals")
    # 5 and 9 tokens, hidden or intermediate not a multiple of 512, the stage
    # entry points
    for m, h, i in ((5, 512, 1024), (9, 512, 1024), (2, 96, 512), (2, 512, 160), (2, 768, 1024)):
        x, mats = make_case(m, h, i, seed=m)
        xd, md = to_dev(x, mats)
        with pytest.raises(capi.TinyInferError) as e:
            capi.mlp_forward(xd, *md, path=DECODE)
        assert e.value.status == capi.TI_ERR_UNSUPPORTED
        auto = capi.mlp_forward(xd, *md)                 # auto falls back
        assert_parity(auto.cpu(), om.mlp_reference(x, *mats), f"fallback m={m} h={h} i={i}")
    x, mats = make_case(2, 512, 1024, seed=3)
    xd, md = to_dev(x, mats)
    with pytest.raises(capi.TinyInferError) as e:
        capi.gate_up(xd, *md[:4], path=DECODE)
    assert e.value.status == capi.TI_ERR_UNSUPPORTED
    # tmp must be 16-byte aligned on every path (vector loads of h)
    base = torch.empty(2 * 1024 + 1, dtype=torch.bfloat16, device="cuda")
    tmp_bad = base[1:].view(2, 1024)
    for path in (0, 1, 2, DECODE):
        with pytest.raises(capi.TinyInferError) as e:
            capi.mlp_forward(xd, *md, tmp=tmp_bad, path=path)
        assert e.value.status == capi.TI_ERR_MISALIGNED
