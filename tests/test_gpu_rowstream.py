"""GPU parity of the row-streaming kernels (one token, one launch per MLP
stage): TI_PATH_SKINNY and TI_PATH_AUTO run them for N == 1 when K % 128 == 0
and the stage's K fits the chunk limits (a wave holds at most 4 chunks of 2048
K elements for gate_up, 6 for down; with fp16 activations 2 and 3; a row is
shared by at most 2 waves for gate_up, 4 for down).

Each stage is checked against the CPU oracle with the kernel's rounding
points (exact sums, h rounded once), as for the 8-row stream kernels.  The
shapes cover the kernel's edge cases: a last chunk with fewer than 64 blocks
(K not a multiple of 2048), waves with no row and waves with many, every
instantiated chunk count, scale bytes outside the hardware conversion's exact
range (NaN included), fp16 activations (fp16 MFMAs; fp16-subnormal weights;
the exact hi + lo form for scale bytes below fp16's range), the residual and
the RMSNorm prologue.  TINYINFER_ROWSTREAM=0 switches the library back to the 8-row
stream kernels for N == 1, which the last tests compare against."""


import numpy as np
import pytest
import torch

from oracle import mlp as om
from tests.helpers import assert_parity, banner, make_case, to_dev
from tests.test_gpu_stream import check_close, down_semantics, h_semantics

pytestmark = pytest.mark.gpu

SKINNY = 1


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


def stages(capi, x, mats, what, cols=None):
    xd, md = to_dev(x, mats)
    gp, gs, up, us, dp, ds = mats
    h = capi.gate_up(xd, *md[:4], path=SKINNY)
    torch.cuda.synchronize()
    h_ref = h_semantics(x, gp, gs, up, us)
    check_close(h.cpu(), h_ref, f"{what} gate_up")
    out = capi.down(h_ref.cuda(), md[4], md[5], path=SKINNY)
    torch.cuda.synchronize()
    out_ref = down_semantics(h_ref, dp, ds)
    out = out.cpu()
    if cols is not None:
        out, out_ref = out[:, cols], out_ref[:, cols]
    check_close(out, out_ref, f"{what} down")
    return out, out_ref


@pytest.mark.parametrize("h,i", [
    (2048, 6144),    # one full chunk per gate_up row; down: 3 chunks
    (4096, 12288),   # Qwen3-8B: 2 chunks (gate_up), 6 chunks (down)
    (2560, 9728),    # Qwen3-4B: last chunk 16 of 64 blocks; down 5 chunks, last 48 blocks
    (1152, 5120),    # one partial chunk of 36 blocks; down 2.5 chunks
    (8192, 1024),    # gate_up at its 4-chunk limit
    (10240, 1024),   # gate_up beyond it: two waves per row (2 + 3 chunks); down 1 chunk
    (3072, 128),     # 16 workgroups, one row per wave; down K = 128: a 4-block chunk
    (1024, 32768),   # 16 rows per wave on a 256-CU part
    (1024, 16384),   # down K = 16384: two waves per row, 4 chunks each
    (5120, 25600),   # Qwen3-32B: gate_up 2.5 chunks; down 12.5 chunks over four waves (3, 3, 3, 4)
])
def test_rowstream_stage_shapes(capi, h, i):
    banner(f"rowstream stages h={h} i={i}")
    x, mats = make_case(1, h, i, seed=11 * h + i)
    stages(capi, x, mats, f"h={h} i={i}")


def test_rowstream_scale_bytes_outside_fast_range(capi):
    """Scale bytes 0, 1, 253, 254 and 255 (NaN) send their row to the exact
    dequantisation branch; a NaN block poisons only its own output row."""
    banner("rowstream exact-scale branch")
    x, mats = make_case(1, 4096, 2048, seed=78)
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
    # a NaN block (the oracle's CPU decoder refuses byte 255): its row only
    ds[1500, 33] = 255
    rest = [c for c in rest if c != 1500]
    h_ref = h_semantics(x, gp, gs, up, us)
    y = capi.down(h_ref.cuda(), torch.from_numpy(dp).cuda(), torch.from_numpy(ds).cuda(), path=SKINNY)
    torch.cuda.synchronize()
    y = y.cpu().float()
    assert torch.isnan(y[0, 1500]) and torch.isfinite(y[0, rest]).all()


@pytest.mark.parametrize("h,i", [(1024, 3072), (2560, 6144), (6144, 2048), (1024, 8192), (4096, 12288),
                                 (8192, 6144), (2048, 24576)])
def test_rowstream_fp16(capi, h, i):
    banner(f"rowstream fp16 h={h} i={i}")
    x, mats = make_case(1, h, i, seed=31 + h, dtype=torch.float16)
    stages(capi, x, mats, f"fp16 h={h} i={i}")


def test_rowstream_fp16_scale_paths(capi):
    """fp16 with scale bytes 104..113 (fp16-subnormal weights, fp16 MFMAs)
    and below 104 (those rows on exact bf16 weights against x's bf16 hi and
    lo parts): every other output within the bar, the rows that read only
    such a block exact to one fp16 unit."""
    from tests.test_gpu_gemm import _isolate_block, _ulps_f16
    banner("rowstream fp16 scale paths")
    x, mats = make_case(1, 2048, 6144, seed=77, dtype=torch.float16)
    gp, gs, up, us, dp, ds = [np.array(a) for a in mats]
    gs[40, 3] = 90
    us[1500, 20] = 95
    rows = {5: 104, 333: 109, 600: 103, 1000: 113}
    for row, byte in rows.items():
        _isolate_block(dp, ds, [row], 7, byte)
    mats = [gp, gs, up, us, dp, ds]
    stages(capi, x, mats, "fp16 scale paths", cols=[c for c in range(2048) if c not in rows])
    xd, md = to_dev(x, mats)
    h_ref = h_semantics(x, gp, gs, up, us)
    o = capi.down(h_ref.cuda(), md[4], md[5], path=SKINNY).cpu()
    o_ref = down_semantics(h_ref, dp, ds)
    for row in rows:
        assert o_ref[:, row].float().abs().max() > 0
        assert _ulps_f16(o[:, row], o_ref[:, row]) <= 1, row


def test_rowstream_residual_and_full_call(capi):
    """The full entry point with a residual equals the two stages plus the
    residual add, bit for bit, and the oracle's composition."""
    banner("rowstream full call + residual")
    x, mats = make_case(1, 4096, 12288, seed=5)
    xd, md = to_dev(x, mats)
    res = torch.randn(1, 4096, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).cuda()
    full = capi.mlp_forward(xd, *md, path=SKINNY, residual=res)
    tmp = capi.gate_up(xd, *md[:4], path=SKINNY)
    out = capi.down(tmp, *md[4:], path=SKINNY)
    torch.cuda.synchronize()
    ref = (out.float() + res.float()).to(torch.bfloat16)
    assert torch.equal(full.view(torch.int16), ref.view(torch.int16))
    check_close(out.cpu(), om.mlp_kernel_semantics(x, *mats), "8B full")


def test_rowstream_rmsnorm_prologue(capi):
    """x + MLP(RMSNorm(x)) at one token: the norm runs in the gate_up kernel's
    prologue; xn is within one rounding of the oracle's norm and the output
    equals the unfused MLP on that xn, bit for bit."""
    banner("rowstream rmsnorm prologue")
    x, mats = make_case(1, 4096, 12288, seed=41)
    xd, md = to_dev(x, mats)
    w = (torch.rand(4096, generator=torch.Generator().manual_seed(3)) + 0.5).to(torch.bfloat16)
    out, xn = capi.mlp_forward_rmsnorm(xd, w.cuda(), 1e-6, *md, path=SKINNY)
    torch.cuda.synchronize()
    xn_ref = om.rmsnorm_reference(x, w, 1e-6)
    rel = ((xn.cpu().float() - xn_ref.float()).abs() / xn_ref.float().abs().clamp_min(1e-30)).max()
    assert float(rel) <= 2 ** -7, f"xn max rel {float(rel)}"
    plain = capi.mlp_forward(xn, *md, path=SKINNY, residual=xd)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
    # the oracle's own norm may round an element of xn the other way, and the
    # residual add rounds once more
    assert_parity(out.cpu(), om.decoder_mlp_reference(x, w, 1e-6, *mats), "norm + mlp")


def kernel_names(fn):
    """Names of the GPU kernels `fn` launches, from torch's profiler."""
    from torch.profiler import ProfilerActivity, profile
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    return [e.name for e in prof.events()]


def test_rowstream_matches_item_stream_kernels(capi):
    """Both decode kernel families agree within the parity bar at one token,
    and TINYINFER_ROWSTREAM picks which one runs."""
    banner("rowstream vs 8-row stream kernels")
    x, mats = make_case(1, 4096, 12288, seed=123)
    xd, md = to_dev(x, mats)
    out = {}
    names = {}
    for flag in ("1", "0"):
        with capi.option("TINYINFER_ROWSTREAM", int(flag)):
            names[flag] = kernel_names(lambda: out.__setitem__(flag, capi.mlp_forward(xd, *md, path=SKINNY)))
    ref = om.mlp_kernel_semantics(x, *mats)
    check_close(out["1"].cpu(), ref, "row kernels")
    check_close(out["0"].cpu(), ref, "item kernels")
    if not names["1"]:
        pytest.skip("the profiler recorded no kernels here; parity checked, dispatch not")
    assert sum("rowstream_kernel" in n for n in names["1"]) == 2, names["1"]
    assert not any("rowstream_kernel" in n for n in names["0"]), names["0"]
    assert sum("stream_kernel<" in n for n in names["0"]) == 2, names["0"]


@pytest.mark.parametrize("split", ["1", "2", "4"])
def test_rowstream_down_split_override(capi, split):
    """TINYINFER_ROW_SPLIT_DOWN picks how many waves share a down row (the
    8B down stage has 6 chunks: 6, 3 + 3 or 1 + 2 + 1 + 2); every choice
    agrees with the oracle and sums its parts in a fixed order."""
    banner(f"rowstream down split {split}")
    x, mats = make_case(1, 4096, 12288, seed=321)
    xd, md = to_dev(x, mats)
    with capi.option("TINYINFER_ROW_SPLIT_DOWN", int(split)):
        h = capi.gate_up(xd, *md[:4], path=SKINNY)
        out = capi.down(h, *md[4:], path=SKINNY)
        again = capi.down(h, *md[4:], path=SKINNY)
        torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    check_close(out.cpu(), down_semantics(h.cpu(), mats[4], mats[5]), f"split {split}")


def test_rowstream_gateup_split_with_norm(capi):
    """gate_up split over two waves per row (TINYINFER_ROW_SPLIT_GATEUP=2) with
    the RMSNorm prologue: each wave normalizes and writes its own chunks of
    xn, and the output equals the unfused MLP on that xn, bit for bit."""
    banner("rowstream gate_up split 2 + norm")
    x, mats = make_case(1, 4096, 12288, seed=55)
    xd, md = to_dev(x, mats)
    w = (torch.rand(4096, generator=torch.Generator().manual_seed(4)) + 0.5).to(torch.bfloat16)
    with capi.option("TINYINFER_ROW_SPLIT_GATEUP", 2):
        out, xn = capi.mlp_forward_rmsnorm(xd, w.cuda(), 1e-6, *md, path=SKINNY)
        plain = capi.mlp_forward(xn, *md, path=SKINNY, residual=xd)
        torch.cuda.synchronize()
    xn_ref = om.rmsnorm_reference(x, w, 1e-6)
    rel = ((xn.cpu().float() - xn_ref.float()).abs() / xn_ref.float().abs().clamp_min(1e-30)).max()
    assert float(rel) <= 2 ** -7, f"xn max rel {float(rel)}"
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
    assert_parity(out.cpu(), om.decoder_mlp_reference(x, w, 1e-6, *mats), "split norm + mlp")


@pytest.mark.parametrize("h,i", [
    (4096, 12288),   # Qwen3-8B at two tokens: gate_up 2 chunks, down 3 + 3
    (2560, 9728),    # partial chunks
    (2048, 6144),    # Qwen3-1.7B
    (1024, 25600),   # down over four waves (3, 3, 3, 4 chunks)
    (1024, 4096),    # down 2 chunks, one wave per row
])
def test_rowstream_two_tokens(capi, h, i):
    """Two tokens (bf16) with the row-pair kernels off: the down stage runs on
    the row kernels, two MFMA passes over each dequantized operand, one per
    token's activations (gate_up on the 8-row stream kernel)."""
    banner(f"rowstream two tokens h={h} i={i}")
    x, mats = make_case(2, h, i, seed=5 * h + i)
    with capi.option("TINYINFER_ROWPAIR", 0):
        stages(capi, x, mats, f"m=2 h={h} i={i}")


@pytest.fixture
def rowpair_off(capi):
    with capi.option("TINYINFER_ROWPAIR", 0):
        yield


def test_rowstream_two_tokens_norm_residual(capi, rowpair_off):
    """x + MLP(RMSNorm(x)) at two tokens (row-pair kernels off): per-token
    norm sums in the prologue, per-token residual in the epilogue; equal to
    the unfused composition."""
    banner("rowstream two tokens norm + residual")
    x, mats = make_case(2, 4096, 12288, seed=77)
    xd, md = to_dev(x, mats)
    w = (torch.rand(4096, generator=torch.Generator().manual_seed(8)) + 0.5).to(torch.bfloat16)
    out, xn = capi.mlp_forward_rmsnorm(xd, w.cuda(), 1e-6, *md, path=SKINNY)
    plain = capi.mlp_forward(xn, *md, path=SKINNY, residual=xd)
    names = kernel_names(lambda: capi.mlp_forward(xn, *md, path=SKINNY, residual=xd))
    torch.cuda.synchronize()
    xn_ref = om.rmsnorm_reference(x, w, 1e-6)
    rel = ((xn.cpu().float() - xn_ref.float()).abs() / xn_ref.float().abs().clamp_min(1e-30)).max()
    assert float(rel) <= 2 ** -7, f"xn max rel {float(rel)}"
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
    assert_parity(out.cpu(), om.decoder_mlp_reference(x, w, 1e-6, *mats), "m=2 norm + mlp")
    if names:
        assert sum("rowstream_kernel" in n for n in names) == 1, names   # down
