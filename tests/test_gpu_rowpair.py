"""GPU parity of the row-pair kernels (2..4 bf16 or fp16 tokens, one launch
per MLP stage): TI_PATH_SKINNY and TI_PATH_AUTO run them for 2 <= N <= 4 when K % 128
== 0 and a wave's share of a row pair fits its registers.

Each stage is checked against the CPU oracle with the kernel's rounding
points (exact sums, h rounded once), as for the other decode kernels.  The
shapes cover the kernel's edge cases: a last chunk with fewer than 32 blocks
(K not a multiple of 1024), waves with no pair and waves with many, one to
four waves per pair, an odd token count (the second MFMA pass half empty),
scale bytes outside the hardware conversion's exact range (NaN included),
fp16 activations (fp16 MFMAs, fp16-subnormal weights, the exact hi + lo form
below fp16's range), the residual and the RMSNorm prologue.  TINYINFER_ROWPAIR=0 switches the
library back to the row / 8-row stream kernels, which the last tests compare
against."""


import numpy as np
import pytest
import torch

from oracle import mlp as om
from tests.helpers import assert_parity, banner, make_case, to_dev
from tests.test_gpu_rowstream import kernel_names, stages
from tests.test_gpu_stream import check_close, h_semantics

pytestmark = pytest.mark.gpu

SKINNY = 1


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("h,i", [
    (4096, 12288),   # Qwen3-8B: gate_up 4 chunks (3-4 tokens: stream kernel), down 12 over four waves
    (2560, 9728),    # Qwen3-4B: last chunk 16 of 32 blocks; down 9.5 chunks over four waves
    (1152, 5120),    # one chunk and a 4-block chunk; down 5 chunks
    (8192, 1024),    # gate_up 8 chunks: two waves per pair (3-4 tokens: stream kernel)
    (10240, 1024),   # gate_up 10 chunks over four waves (3, 2, 3, 2) at two tokens; down one chunk
    (3072, 128),     # down K = 128: a 4-block chunk; 64 gate_up pairs, most waves idle
    (1024, 32768),   # 8 pairs per wave on a 256-CU part
    (1024, 3072),    # Qwen3-0.6B: 512 down pairs split over two waves each to fill the CUs
])
def test_rowpair_stage_shapes(capi, m, h, i):
    banner(f"rowpair stages m={m} h={h} i={i}")
    x, mats = make_case(m, h, i, seed=13 * h + i + m)
    stages(capi, x, mats, f"m={m} h={h} i={i}")


@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("h,i", [(4096, 12288), (1152, 5120), (1024, 3072), (3072, 128)])
def test_rowpair_fp16_stage_shapes(capi, m, h, i):
    """fp16 activations (fewer chunks per wave than bf16: stages beyond them
    run on the other decode kernels, also checked here)."""
    banner(f"rowpair fp16 stages m={m} h={h} i={i}")
    x, mats = make_case(m, h, i, seed=19 * h + i + m, dtype=torch.float16)
    stages(capi, x, mats, f"fp16 m={m} h={h} i={i}")


def test_rowpair_fp16_runs_here_and_scale_paths(capi):
    """At two fp16 tokens the down stage of a 2048 x 6144 MLP runs on the
    row-pair kernels; scale bytes 104..113 (fp16-subnormal weights) and
    below 104 (exact hi + lo form): every other output within the bar, the
    rows that read only such a block exact to one fp16 unit."""
    from tests.test_gpu_gemm import _isolate_block, _ulps_f16
    from tests.test_gpu_stream import down_semantics
    banner("rowpair fp16 scale paths")
    x, mats = make_case(2, 2048, 6144, seed=78, dtype=torch.float16)
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
    names = kernel_names(lambda: capi.down(h_ref.cuda(), md[4], md[5], path=SKINNY))
    o = capi.down(h_ref.cuda(), md[4], md[5], path=SKINNY).cpu()
    o_ref = down_semantics(h_ref, dp, ds)
    for row in rows:
        assert o_ref[:, row].float().abs().max() > 0
        assert _ulps_f16(o[:, row], o_ref[:, row]) <= 1, row
    if names:
        assert any("rowpair_kernel" in n for n in names), names


def test_rowpair_fp16_norm_residual(capi):
    """The fused layer half in fp16 at two tokens: xn within one fp16 rounding
    of the oracle's norm, the output bit-identical to the unfused composition."""
    banner("rowpair fp16 norm + residual")
    x, mats = make_case(2, 4096, 12288, seed=71, dtype=torch.float16)
    xd, md = to_dev(x, mats)
    w = (torch.rand(4096, generator=torch.Generator().manual_seed(3)) + 0.5).to(torch.float16)
    out, xn = capi.mlp_forward_rmsnorm(xd, w.cuda(), 1e-6, *md, path=SKINNY)
    plain = capi.mlp_forward(xn, *md, path=SKINNY, residual=xd)
    torch.cuda.synchronize()
    xn_ref = om.rmsnorm_reference(x, w, 1e-6)
    rel = ((xn.cpu().float() - xn_ref.float()).abs() / xn_ref.float().abs().clamp_min(1e-30)).max()
    assert float(rel) <= 2 ** -10, f"xn max rel {float(rel)}"
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
    assert_parity(out.cpu(), om.decoder_mlp_reference(x, w, 1e-6, *mats), "fp16 norm + mlp")


def test_rowpair_falls_back_beyond_its_registers(capi):
    """Down K = 25600 is 25 chunks: more than four waves' registers hold, so
    that stage runs on the other decode kernels; the gate_up stage still runs
    here.  Both agree with the oracle."""
    banner("rowpair fallback (down K = 25600)")
    x, mats = make_case(2, 1024, 25600, seed=99)
    stages(capi, x, mats, "m=2 h=1024 i=25600")


def test_rowpair_scale_bytes_outside_fast_range(capi):
    """Scale bytes 0, 1, 253, 254 and 255 (NaN) send their pair to the exact
    dequantisation branch; a NaN block poisons only its own output row, for
    every token, and not the other row of its pair."""
    banner("rowpair exact-scale branch")
    x, mats = make_case(3, 4096, 2048, seed=79)
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


@pytest.mark.parametrize("m,h,i", [
    (2, 4096, 12288), (3, 4096, 12288), (4, 4096, 12288),
    (2, 10240, 1024),   # gate_up over four waves per pair: each normalizes and writes its chunks of xn
])
def test_rowpair_norm_residual(capi, m, h, i):
    """x + MLP(RMSNorm(x)): per-token norm sums in the gate_up prologue,
    per-token residual in the down epilogue; xn within one rounding of the
    oracle's norm, the output equal to the unfused composition bit for bit."""
    banner(f"rowpair norm + residual m={m} h={h} i={i}")
    x, mats = make_case(m, h, i, seed=70 + m + h)
    xd, md = to_dev(x, mats)
    w = (torch.rand(h, generator=torch.Generator().manual_seed(m)) + 0.5).to(torch.bfloat16)
    out, xn = capi.mlp_forward_rmsnorm(xd, w.cuda(), 1e-6, *md, path=SKINNY)
    plain = capi.mlp_forward(xn, *md, path=SKINNY, residual=xd)
    torch.cuda.synchronize()
    xn_ref = om.rmsnorm_reference(x, w, 1e-6)
    rel = ((xn.cpu().float() - xn_ref.float()).abs() / xn_ref.float().abs().clamp_min(1e-30)).max()
    assert float(rel) <= 2 ** -7, f"xn max rel {float(rel)}"
    assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
    assert_parity(out.cpu(), om.decoder_mlp_reference(x, w, 1e-6, *mats), f"m={m} norm + mlp")


@pytest.mark.parametrize("m,launches", [(2, 2), (4, 1)])
def test_rowpair_matches_other_decode_kernels(capi, m, launches):
    """The row-pair kernels and the kernels they replace agree within the
    parity bar, and TINYINFER_ROWPAIR picks which run (8B at four tokens:
    the down stage only; its gate_up runs on the 8-row stream kernel)."""
    banner(f"rowpair vs other decode kernels m={m}")
    x, mats = make_case(m, 4096, 12288, seed=400 + m)
    xd, md = to_dev(x, mats)
    out, names = {}, {}
    for flag in ("1", "0"):
        with capi.option("TINYINFER_ROWPAIR", int(flag)):
            names[flag] = kernel_names(lambda: out.__setitem__(flag, capi.mlp_forward(xd, *md, path=SKINNY)))
    ref = om.mlp_kernel_semantics(x, *mats)
    check_close(out["1"].cpu(), ref, "row-pair kernels")
    check_close(out["0"].cpu(), ref, "other kernels")
    if not names["1"]:
        pytest.skip("the profiler recorded no kernels here; parity checked, dispatch not")
    assert sum("rowpair_kernel" in n for n in names["1"]) == launches, names["1"]
    assert not any("rowpair_kernel" in n for n in names["0"]), names["0"]
