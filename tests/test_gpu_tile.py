"""GPU parity of the split-K tile kernels (9..80 bf16 or fp16 tokens, K a
multiple of 1024): TI_PATH_SKINNY and TI_PATH_AUTO run them for small batches
the decode kernels do not take.

Each stage is checked against the CPU oracle with the kernel's rounding
points (exact fp32 sums, h rounded once), as for the decode kernels.  The
cases cover one to five 16-token column tiles with a partial last one, one
K range (Qwen3-0.6B gate_up) and 25 of them, a grid with fewer row groups
than waves, scale bytes outside the hardware conversion's exact range (NaN
included), fp16 activations (fp16 MFMAs, fp16-subnormal weights, and the
exact hi + lo form for scale bytes below fp16's range), the residual, and the
dispatch (TINYINFER_TILE=0 switches the kernels off)."""


import numpy as np
import pytest
import torch

from oracle import mlp as om
from tests.helpers import assert_parity, banner, make_case, to_dev
from tests.test_gpu_rowstream import kernel_names, stages
from tests.test_gpu_stream import check_close, h_semantics

pytestmark = pytest.mark.gpu

AUTO, SKINNY = 0, 1


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


@pytest.mark.parametrize("m", [9, 16, 17, 33, 48, 64, 72, 80])
@pytest.mark.parametrize("h,i", [
    (4096, 12288),   # Qwen3-8B: gate_up 4 K ranges, down 12
    (1024, 3072),    # Qwen3-0.6B: gate_up one K range (48 workgroups), down 3
    (2048, 1024),    # down: one range of 128 row groups, fewer than a full grid's waves
    (1024, 25600),   # down: 25 K ranges
])
def test_tile_stage_shapes(capi, m, h, i):
    banner(f"tile stages m={m} h={h} i={i}")
    x, mats = make_case(m, h, i, seed=17 * h + i + m)
    stages(capi, x, mats, f"m={m} h={h} i={i}")


def test_tile_scale_bytes_outside_fast_range(capi):
    """Scale bytes 0, 1, 253, 254 and 255 (NaN) send their row group to the
    exact dequantisation; a NaN block poisons only its own output row, for
    every token."""
    banner("tile exact-scale branch")
    x, mats = make_case(20, 4096, 2048, seed=81)
    gp, gs, up, us, dp, ds = [np.array(a) for a in mats]
    gs[3, 0] = 0
    gs[700, 5] = 1
    us[11, 100] = 1
    for row, blk, byte in ((17, 9, 253), (900, 60, 254)):
        ds[row, blk] = byte
        dp[row, blk * 16:(blk + 1) * 16] = 0
        dp[row, blk * 16 + 3] = 0x10
    mats = [gp, gs, up, us, dp, ds]
    big = [17, 900]
    rest = [c for c in range(4096) if c not in big]
    stages(capi, x, mats, "exact-scale rows", cols=rest)
    out, ref = stages(capi, x, mats, "exact-scale big rows", cols=big)
    assert torch.isfinite(ref.float()).all() and ref.float().abs().min() > 1e30
    ds[1500, 33] = 255
    rest = [c for c in rest if c != 1500]
    h_ref = h_semantics(x, gp, gs, up, us)
    y = capi.down(h_ref.cuda(), torch.from_numpy(dp).cuda(), torch.from_numpy(ds).cuda(), path=SKINNY)
    torch.cuda.synchronize()
    y = y.cpu().float()
    assert torch.isnan(y[:, 1500]).all() and torch.isfinite(y[:, rest]).all()


@pytest.mark.parametrize("m", [16, 40])
def test_tile_full_call_residual(capi, m):
    """The AUTO entry point with a residual equals the two stages plus torch's
    residual add bit for bit, and the reference composition within the
    parity bar."""
    banner(f"tile full call + residual m={m}")
    x, mats = make_case(m, 4096, 12288, seed=500 + m)
    xd, md = to_dev(x, mats)
    res = torch.randn(m, 4096, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16).cuda()
    full = capi.mlp_forward(xd, *md, path=AUTO, residual=res)
    tmp = capi.gate_up(xd, *md[:4], path=AUTO)
    out = capi.down(tmp, *md[4:], path=AUTO)
    torch.cuda.synchronize()
    ref = (out.float() + res.float()).to(torch.bfloat16)
    assert torch.equal(full.view(torch.int16), ref.view(torch.int16))
    check_close(out.cpu(), om.mlp_kernel_semantics(x, *mats), f"m={m} full")
    assert_parity(full.cpu(), (om.mlp_reference(x, *mats).float() + res.cpu().float()).to(torch.bfloat16),
                  f"m={m} + residual")


def test_tile_dispatch_and_switch(capi):
    """AUTO runs the tile kernels for 16 tokens at the 8B shape (gate_up in one
    launch, down as tile kernel + reduce); TINYINFER_TILE=0 sends the call to
    the GEMM path, and both agree within the parity bar."""
    banner("tile dispatch")
    x, mats = make_case(16, 4096, 12288, seed=600)
    xd, md = to_dev(x, mats)
    out, names = {}, {}
    for flag in ("1", "0"):
        with capi.option("TINYINFER_TILE", int(flag)):
            names[flag] = kernel_names(lambda: out.__setitem__(flag, capi.mlp_forward(xd, *md, path=AUTO)))
    ref = om.mlp_kernel_semantics(x, *mats)
    check_close(out["1"].cpu(), ref, "tile kernels")
    check_close(out["0"].cpu(), ref, "GEMM path")
    if not names["1"]:
        pytest.skip("the profiler recorded no kernels here; parity checked, dispatch not")
    assert sum("tile_gu_kernel" in n for n in names["1"]) == 1, names["1"]
    assert sum("tile_kernel" in n for n in names["1"]) == 1, names["1"]
    assert sum("tile_reduce" in n for n in names["1"]) == 1, names["1"]
    assert not any("tile_kernel" in n or "tile_gu_kernel" in n for n in names["0"]), names["0"]


@pytest.mark.parametrize("m,h,i", [
    (9, 4096, 12288), (16, 4096, 12288),   # four K ranges, one block per workgroup iteration
    (24, 2048, 6144), (32, 2048, 6144),    # two ranges, two column tiles
    (20, 1024, 3072),                      # one range, four blocks per iteration
])
def test_tile_gate_up_in_one_launch(capi, m, h, i):
    """gate_up with all of x in LDS runs as one launch that adds the K ranges'
    partial tiles in LDS: bit-identical to the split kernel + reduce (the same
    partials added in the same order; TINYINFER_TILE_GU=0), and one kernel
    instead of two."""
    banner(f"tile gate_up one launch m={m} h={h} i={i}")
    x, mats = make_case(m, h, i, seed=900 + m + h)
    xd, md = to_dev(x, mats)
    out, names = {}, {}
    for flag in ("1", "0"):
        with capi.option("TINYINFER_TILE_GU", int(flag)):
            names[flag] = kernel_names(lambda: out.__setitem__(flag, capi.gate_up(xd, *md[:4], path=SKINNY)))
    assert torch.equal(out["1"].view(torch.int16), out["0"].view(torch.int16))
    check_close(out["1"].cpu(), h_semantics(x, *mats[:4]), f"m={m} gate_up")
    if names["1"]:
        assert sum("tile_gu_kernel" in n for n in names["1"]) == 1, names["1"]
        assert not any("tile_reduce" in n for n in names["1"]), names["1"]
        assert sum("tile_reduce" in n for n in names["0"]) == 1, names["0"]


@pytest.mark.parametrize("m", [9, 16, 33, 64])
@pytest.mark.parametrize("h,i", [(4096, 12288), (1024, 3072), (1024, 25600)])
def test_tile_fp16_stage_shapes(capi, m, h, i):
    """fp16 activations on the tile kernels (fp16 MFMAs on weights converted to
    fp16), at one to four column tiles and 1..25 K ranges."""
    banner(f"tile fp16 stages m={m} h={h} i={i}")
    x, mats = make_case(m, h, i, seed=31 * h + i + m, dtype=torch.float16)
    stages(capi, x, mats, f"fp16 m={m} h={h} i={i}")


@pytest.mark.parametrize("m", [16, 48])
def test_tile_fp16_scale_paths(capi, m):
    """fp16 with scale bytes 104..113 (fp16-subnormal weights, still the fp16
    MFMA path) and below 104 (those row groups on exact bf16 weights against
    the activations' bf16 hi and lo parts): every other output within the
    bar, the rows that read only such a block exact to one fp16 unit."""
    from tests.test_gpu_gemm import _isolate_block, _ulps_f16
    from tests.test_gpu_stream import down_semantics
    banner(f"tile fp16 scale paths m={m}")
    x, mats = make_case(m, 1024, 2048, seed=97 + m, dtype=torch.float16)
    gp, gs, up, us, dp, ds = [np.array(a) for a in mats]
    gs[40, 3] = 90
    us[1500, 20] = 95
    rows = {5: 104, 333: 109, 600: 103, 1000: 113}
    for row, byte in rows.items():
        _isolate_block(dp, ds, [row], 7, byte)
    mats = [gp, gs, up, us, dp, ds]
    stages(capi, x, mats, "fp16 scale paths", cols=[c for c in range(1024) if c not in rows])
    xd, md = to_dev(x, mats)
    h_ref = h_semantics(x, gp, gs, up, us)
    o = capi.down(h_ref.cuda(), md[4], md[5], path=SKINNY).cpu()
    o_ref = down_semantics(h_ref, dp, ds)
    for row in rows:
        assert o_ref[:, row].float().abs().max() > 0
        assert _ulps_f16(o[:, row], o_ref[:, row]) <= 1, row


@pytest.mark.parametrize("m,h,i", [(16, 4096, 12288), (24, 2048, 6144)])
def test_tile_fp16_gate_up_in_one_launch(capi, m, h, i):
    """fp16 gate_up in one launch is bit-identical to the split kernel + reduce."""
    banner(f"tile fp16 gate_up one launch m={m} h={h} i={i}")
    x, mats = make_case(m, h, i, seed=950 + m + h, dtype=torch.float16)
    xd, md = to_dev(x, mats)
    out = {}
    for flag in (1, 0):
        with capi.option("TINYINFER_TILE_GU", flag):
            out[flag] = capi.gate_up(xd, *md[:4], path=SKINNY)
    torch.cuda.synchronize()
    assert torch.equal(out[1].view(torch.int16), out[0].view(torch.int16))
    check_close(out[1].cpu(), h_semantics(x, *mats[:4]), f"fp16 m={m} gate_up")


@pytest.mark.parametrize("m", [16, 40])
def test_tile_graph_replays(capi, m):
    """Graphs: on a capture stream that already ran the call eagerly (so its
    workspace exists) the tile kernels are captured, and every replay, with
    eager work between replays, gives the eager bits (16 tokens: one-launch
    gate_up + down with its reduce; 40: both stages split + reduce). On a
    fresh capture stream the workspace cannot be allocated: the call is
    captured on another kernel family, still within tolerance."""
    banner(f"tile graph replays m={m}")
    x, mats = make_case(m, 4096, 12288, seed=700 + m)
    xd, md = to_dev(x, mats)
    ref = om.mlp_kernel_semantics(x, *mats)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out = torch.empty((m, 4096), dtype=torch.bfloat16, device="cuda")
    tmp = torch.empty((m, 12288), dtype=torch.bfloat16, device="cuda")
    with torch.cuda.stream(s):
        capi.mlp_forward(xd, *md, out=out, tmp=tmp, path=AUTO)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = out.clone()
    check_close(eager.cpu(), ref, "eager tile")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(2):
            capi.mlp_forward(xd, *md, out=out, tmp=tmp, path=AUTO)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
        capi.mlp_forward(xd, *md, path=AUTO)          # eager work between replays
        torch.cuda.synchronize()
    del g
    g2 = torch.cuda.CUDAGraph()
    out2 = torch.empty_like(out)
    with torch.cuda.graph(g2):                        # a fresh capture stream
        capi.mlp_forward(xd, *md, out=out2, tmp=tmp, path=AUTO)
    for _ in range(2):
        out2.zero_()
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        check_close(out2.cpu(), ref, "fresh-stream capture")
