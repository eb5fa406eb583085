"""GPU parity of the prefill GEMM path (TI_PATH_GEMM, and TI_PATH_AUTO at
N >= 96): the direct-to-LDS ring kernels for bf16 activations with hidden and
intermediate multiples of 512 (bf16 and fp16), the register-staged GEMM
otherwise.

Each stage is called through its C-ABI entry point and compared with the CPU
oracle at the kernel's rounding points (exact sums, h rounded once to the
activation dtype): a few bf16 ulps. Cases: partial token tiles, the Qwen3
block shapes, scale bytes outside the hardware conversion's exact range,
fp16 activations (the ring's fp16 MFMA path, fp16-subnormal weights, and
its exact hi + lo path for scale bytes below fp16's range),
bit-reproducibility, and the
split-K form of the ring kernels (fp32 partials over K ranges summed in a
fixed order by a reduce kernel) that runs when the output tiles alone would
leave CUs idle, for every tile or for the tiles past the last full round of
workgroups only (the tail split)."""  

import os

import numpy as np
import pytest
import torch

from oracle import mlp as om
from tests.helpers import banner, make_case, to_dev
from tests.test_gpu_stream import check_close, down_semantics, h_semantics

pytestmark = pytest.mark.gpu

GEMM = 2


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


def run_gemm_stages(capi, x, mats, what, cols=None):
    xd, md = to_dev(x, mats)
    gp, gs, up, us, dp, ds = mats
    h = capi.gate_up(xd, *md[:4], path=GEMM)
    torch.cuda.synchronize()
    h_ref = h_semantics(x, gp, gs, up, us)
    check_close(h.cpu(), h_ref, f"{what} gate_up")
    out = capi.down(h_ref.to("cuda"), md[4], md[5], path=GEMM)
    torch.cuda.synchronize()
    out, out_ref = out.cpu(), down_semantics(h_ref, dp, ds)
    if cols is not None:
        out, out_ref = out[:, cols], out_ref[:, cols]
    check_close(out, out_ref, f"{what} down")
    return out, out_ref


@pytest.mark.parametrize("m", [16, 33, 64, 96, 130, 256, 300, 513])
def test_gemm_partial_token_tiles(capi, m):
    """Token counts around the tile sizes (64-token tiles up to 64 tokens,
    then 128 and 256), with partial last tiles."""
    banner(f"gemm m={m} h=1024 i=1536")
    x, mats = make_case(m, 1024, 1536, seed=1000 + m)
    run_gemm_stages(capi, x, mats, f"m={m}")


@pytest.mark.parametrize("h,i,m", [(1024, 3072, 128), (2048, 6144, 200), (4096, 12288, 256), (4096, 12288, 24)])
def test_gemm_qwen3_shapes(capi, h, i, m):
    """Qwen3-0.6B, 1.7B and 8B MLP shapes."""
    banner(f"gemm qwen3 h={h} i={i} m={m}")
    x, mats = make_case(m, h, i, seed=h + m)
    run_gemm_stages(capi, x, mats, f"h={h} i={i} m={m}")


def test_gemm_scale_bytes_outside_fast_range(capi):
    """Scale bytes 0, 1, 253 and 254 take the exact dequantisation of a K step;
    other steps of the same tiles stay on the hardware conversion."""
    banner("gemm exact-scale branch")
    x, mats = make_case(160, 1024, 2048, seed=91)
    gp, gs, up, us, dp, ds = [np.array(a) for a in mats]
    gs[3, 0] = 0
    gs[700, 5] = 1
    us[11, 31] = 1
    for row, blk, byte in ((17, 9, 253), (900, 60, 254)):
        ds[row, blk] = byte
        dp[row, blk * 16:(blk + 1) * 16] = 0
        dp[row, blk * 16 + 3] = 0x10
    mats = [gp, gs, up, us, dp, ds]
    big = [17, 900]
    _, ref = run_gemm_stages(capi, x, mats, "exact-scale big rows", cols=big)
    assert torch.isfinite(ref.float()).all() and ref.float().abs().min() > 1e30
    run_gemm_stages(capi, x, mats, "exact-scale other rows", cols=[c for c in range(1024) if c not in big])


def test_gemm_fp16_activations(capi):
    banner("gemm fp16")
    x, mats = make_case(130, 1024, 1536, seed=5, dtype=torch.float16)
    run_gemm_stages(capi, x, mats, "fp16")


@pytest.mark.parametrize("h,i,m", [(4096, 12288, 256), (2048, 6144, 200), (1024, 3072, 1100)])
def test_gemm_fp16_qwen3_shapes(capi, h, i, m):
    """fp16 activations on the ring kernels (fp16 MFMAs on weights converted to
    fp16, split K at 8B M=256), at the Qwen3 shapes."""
    banner(f"gemm fp16 qwen3 h={h} i={i} m={m}")
    x, mats = make_case(m, h, i, seed=h + m + 1, dtype=torch.float16)
    run_gemm_stages(capi, x, mats, f"fp16 h={h} i={i} m={m}")


def _isolate_block(dp, ds, rows, blk, byte):
    """Down rows whose only nonzero weights are one 32-element block with the
    given scale byte (the other blocks keep their scale bytes, codes zero)."""
    for row in rows:
        dp[row, :] = 0
        dp[row, blk * 16:(blk + 1) * 16] = (np.arange(16) * 17).astype(np.uint8)   # codes c | c << 4
        ds[row, blk] = byte


def _ulps_f16(a, b):
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    return (ia - ib).abs().max().item()


def test_gemm_fp16_subnormal_weights(capi):
    """Scale bytes 104..113 make fp16 subnormal weights on the fast path (the
    whole tile stays on it): rows that read only such a block equal the exact
    sum rounded to fp16 within one unit (a flush to zero would give 0)."""
    banner("gemm fp16 subnormal weights")
    x, mats = make_case(160, 1024, 2048, seed=93, dtype=torch.float16)
    gp, gs, up, us, dp, ds = [np.array(a) for a in mats]
    rows = {5: 104, 333: 107, 1000: 113}
    for row, byte in rows.items():
        _isolate_block(dp, ds, [row], 7, byte)
    mats = [gp, gs, up, us, dp, ds]
    assert ((ds >= 104) & (ds <= 140)).all() and ((gs >= 104) & (gs <= 140)).all()
    out, ref = run_gemm_stages(capi, x, mats, "fp16 subnormal weights", cols=[c for c in range(1024) if c not in rows])
    xd, md = to_dev(x, mats)
    h_ref = h_semantics(x, gp, gs, up, us)
    o = capi.down(h_ref.to("cuda"), md[4], md[5], path=GEMM).cpu()
    o_ref = down_semantics(h_ref, dp, ds)
    for row in rows:
        assert o_ref[:, row].float().abs().max() > 0
        assert _ulps_f16(o[:, row], o_ref[:, row]) <= 1, row


def test_gemm_fp16_scales_outside_fp16_range(capi):
    """A scale byte below 104 (weights below fp16's range) sends its tiles to
    the exact bf16 weights against the activations' bf16 hi + lo parts: the
    whole output within tolerance, the isolated rows exact to one unit."""
    banner("gemm fp16 hi/lo path")
    x, mats = make_case(160, 1024, 2048, seed=94, dtype=torch.float16)
    gp, gs, up, us, dp, ds = [np.array(a) for a in mats]
    gs[40, 3] = 90
    us[1500, 20] = 95
    rows = [9, 600]
    _isolate_block(dp, ds, rows, 11, 103)
    mats = [gp, gs, up, us, dp, ds]
    run_gemm_stages(capi, x, mats, "fp16 hi/lo", cols=[c for c in range(1024) if c not in rows])
    xd, md = to_dev(x, mats)
    h_ref = h_semantics(x, gp, gs, up, us)
    o = capi.down(h_ref.to("cuda"), md[4], md[5], path=GEMM).cpu()
    o_ref = down_semantics(h_ref, dp, ds)
    for row in rows:
        assert o_ref[:, row].float().abs().max() > 0
        assert _ulps_f16(o[:, row], o_ref[:, row]) <= 1, row


def test_gemm_fp16_infinite_activation_on_the_hi_lo_path(capi):
    """An infinite fp16 activation on the exact hi + lo path (every down tile
    sent there by one scale byte below fp16's range per row) multiplies as
    IEEE has it: +-inf where its weight is nonzero, NaN where it is zero, as in
    the oracle; the other tokens stay finite and within the bar."""
    banner("gemm fp16 inf activation, hi/lo path")
    x, mats = make_case(160, 1024, 2048, seed=95, dtype=torch.float16)
    gp, gs, up, us, dp, ds = [np.array(a) for a in mats]
    ds[:, 0] = 103
    h_ref = h_semantics(x, gp, gs, up, us)
    h_ref[0, 100] = float("inf")
    dpt, dst = torch.from_numpy(dp).cuda(), torch.from_numpy(ds).cuda()
    o = capi.down(h_ref.cuda(), dpt, dst, path=GEMM).cpu().float()
    o_ref = down_semantics(h_ref, dp, ds).float()
    assert torch.equal(torch.isnan(o[0]), torch.isnan(o_ref[0]))
    assert torch.equal(torch.isinf(o[0]), torch.isinf(o_ref[0])) and torch.isinf(o_ref[0]).any()
    inf = torch.isinf(o_ref[0])
    assert torch.equal(torch.sign(o[0][inf]), torch.sign(o_ref[0][inf]))
    check_close(o[1:].to(torch.float16), o_ref[1:].to(torch.float16), "finite tokens")


def test_gemm_deterministic_and_full_call(capi):
    """Two calls give the same bits; the full entry point equals its stages."""
    banner("gemm determinism")
    x, mats = make_case(300, 2048, 6144, seed=8)
    xd, md = to_dev(x, mats)
    a = capi.mlp_forward(xd, *md, path=GEMM)
    b = capi.mlp_forward(xd, *md, path=GEMM)
    tmp = capi.gate_up(xd, *md[:4], path=GEMM)
    c = capi.down(tmp, *md[4:], path=GEMM)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(a.view(torch.int16), c.view(torch.int16))
    check_close(a.cpu(), om.mlp_kernel_semantics(x, *mats), "1.7B m=300 full")


@pytest.mark.parametrize("m", [96, 128, 384, 512])
def test_gemm_split_k_qwen3_8b(capi, m):
    """Qwen3-8B shapes at token counts whose tiles leave CUs idle: down has 16
    output tiles per 128 tokens, so its K (12288) is split."""
    banner(f"gemm split-K qwen3-8b m={m}")
    x, mats = make_case(m, 4096, 12288, seed=77 + m)
    run_gemm_stages(capi, x, mats, f"8B m={m}")


@pytest.mark.parametrize("ksplit", [1, 2, 3, 5])
def test_gemm_forced_split_counts(capi, ksplit):
    """Every split count gives the oracle's result within tolerance, also
    uneven ranges (5 ranges over 6 blocks of 512 K) and no split at all."""
    banner(f"gemm forced ksplit={ksplit}")
    x, mats = make_case(200, 3072, 3072, seed=600 + ksplit)
    with capi.option("TINYINFER_RING_KSPLIT", ksplit):
        run_gemm_stages(capi, x, mats, f"ksplit={ksplit}")


def test_gemm_split_deterministic(capi):
    """Split results are bit-reproducible and close to the unsplit ones."""
    banner("gemm split determinism")
    x, mats = make_case(160, 2048, 6144, seed=31)
    xd, md = to_dev(x, mats)
    with capi.option("TINYINFER_RING_KSPLIT", 4):
        a = capi.mlp_forward(xd, *md, path=GEMM)
        b = capi.mlp_forward(xd, *md, path=GEMM)
    with capi.option("TINYINFER_RING_KSPLIT", 1):
        c = capi.mlp_forward(xd, *md, path=GEMM)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    check_close(a.cpu(), c.cpu().float(), "split vs unsplit")


@pytest.mark.parametrize("m,dtype,row0", [
    (300, torch.bfloat16, 10880),    # 288 gate_up tiles: 255 whole + 33 in 7 K ranges
    (257, torch.bfloat16, 10880),    # the same split, one token in the last token tile
    (384, torch.float16, 10880),
])
def test_gemm_tail_split_qwen3_8b(capi, m, dtype, row0):
    """Qwen3-8B gate_up at token counts whose tiles leave the last round of
    workgroups part-empty: the tiles past the last full round are split over
    K (TINYINFER_RING_TAIL), where the cost model prefers that to splitting
    every tile or none.  Both stages match the oracle; the output rows of the
    whole tiles are bit-identical to the unsplit kernel's
    (TINYINFER_RING_KSPLIT=1), the split band within the tolerance, and the
    split call is bit-reproducible."""
    banner(f"gemm tail split qwen3-8b m={m} {dtype}")
    x, mats = make_case(m, 4096, 12288, seed=90 + m, dtype=dtype)
    run_gemm_stages(capi, x, mats, f"8B m={m} tail split")
    xd, md = to_dev(x, mats)
    a = capi.gate_up(xd, *md[:4], path=GEMM)
    b = capi.gate_up(xd, *md[:4], path=GEMM)
    with capi.option("TINYINFER_RING_KSPLIT", 1):       # every tile whole
        c = capi.gate_up(xd, *md[:4], path=GEMM)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(a[:, :row0].view(torch.int16), c[:, :row0].view(torch.int16))
    assert not torch.equal(a[:, row0:].view(torch.int16), c[:, row0:].view(torch.int16)), "band not split"
    check_close(a[:, row0:].cpu(), c[:, row0:].cpu().float(), "split band vs unsplit")


def test_gemm_tail_split_graph_replays(capi):
    """A graph captured on a stream that already ran the tail-split call
    replays it bit-identically, with eager work between replays."""
    banner("gemm tail split graph replays")
    m = 300
    x, mats = make_case(m, 4096, 12288, seed=45)
    xd, md = to_dev(x, mats)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out = torch.empty((m, 4096), dtype=torch.bfloat16, device="cuda")
    tmp = torch.empty((m, 12288), dtype=torch.bfloat16, device="cuda")
    with torch.cuda.stream(s):
        capi.mlp_forward(xd, *md, out=out, tmp=tmp, path=GEMM)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        capi.mlp_forward(xd, *md, out=out, tmp=tmp, path=GEMM)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
        capi.mlp_forward(xd[:200].contiguous(), *md, path=GEMM)
        torch.cuda.synchronize()
    del g
    check_close(eager.cpu(), om.mlp_kernel_semantics(x, *mats), "tail split full call")


def test_gemm_split_k_graph_replays(capi):
    """Graphs: on a capture stream that already ran the call eagerly, the
    split kernels and their workspace are captured, and every replay (with
    eager work between them) gives the eager bits; on a fresh capture stream
    the call is captured unsplit, still within tolerance of the oracle."""
    banner("gemm split-K graph replays")
    x, mats = make_case(160, 2048, 6144, seed=44)
    xd, md = to_dev(x, mats)
    ref = om.mlp_kernel_semantics(x, *mats)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out = torch.empty((160, 2048), dtype=torch.bfloat16, device="cuda")
    tmp = torch.empty((160, 6144), dtype=torch.bfloat16, device="cuda")
    with torch.cuda.stream(s):
        capi.mlp_forward(xd, *md, out=out, tmp=tmp, path=GEMM)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    check_close(eager.cpu(), ref, "eager split")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(3):
            capi.mlp_forward(xd, *md, out=out, tmp=tmp, path=GEMM)
    for _ in range(4):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
        capi.mlp_forward(xd, *md, path=GEMM)          # eager work between replays
        torch.cuda.synchronize()
    del g
    g2 = torch.cuda.CUDAGraph()
    out2 = torch.empty_like(out)
    with torch.cuda.graph(g2):                        # a fresh capture stream
        capi.mlp_forward(xd, *md, out=out2, tmp=tmp, path=GEMM)
    for _ in range(2):
        out2.zero_()
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        check_close(out2.cpu(), ref, "fresh-stream capture")
    del g2
