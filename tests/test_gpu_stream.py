"""GPU parity of the streaming decode GEMV kernels (one launch per MLP stage,
N <= 8 tokens, hidden and intermediate multiples of 512, at most 8 K
segments of 256 per wave): the kernels TI_PATH_SKINNY and TI_PATH_AUTO run
for decode-sized calls.

Each stage is called through its own C-ABI entry point and checked against
the CPU oracle with the kernel's rounding points (exact sums, h rounded once
to the activation dtype): a few bf16 ulps. The shapes are chosen for the
kernel's edge cases: waves with no K segment or a partial last unit, units
spanning two row-group parts, fewer row groups than CUs and many row groups
per workgroup, scale bytes outside the hardware conversion's exact range, and
fp16 activations (fp16 MFMAs, fp16-subnormal weights, and the exact hi + lo
form for scale bytes below fp16's range)."""

import numpy as np
import pytest
import torch

from oracle import mlp as om
from oracle.mxfp4 import dequantize_chunk
from tests.helpers import banner, make_case, to_dev

pytestmark = pytest.mark.gpu

SKINNY = 1


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


@pytest.fixture(autouse=True)
def stream_kernels_only(capi):
    """The row and row-pair kernels take 1..4 tokens when they are on; these
    tests keep them off so that every case runs on the 8-row stream kernels."""
    with capi.option("TINYINFER_ROWSTREAM", 0), capi.option("TINYINFER_ROWPAIR", 0):
        yield


def h_semantics(x, gp, gs, up, us):
    """Exact gate/up sums, SiLU(g)*u rounded once to the activation dtype."""
    x64 = x.to(torch.float64).numpy()
    wg = dequantize_chunk(np.asarray(gp), np.asarray(gs)).astype(np.float64)
    wu = dequantize_chunk(np.asarray(up), np.asarray(us)).astype(np.float64)
    h = om._round_to(om._silu64(x64 @ wg.T) * (x64 @ wu.T), x.dtype)
    return torch.from_numpy(h).to(x.dtype)


def down_semantics(h, dp, ds):
    h64 = h.to(torch.float64).numpy()
    wd = dequantize_chunk(np.asarray(dp), np.asarray(ds)).astype(np.float64)
    return torch.from_numpy((h64 @ wd.T).astype(np.float32)).to(h.dtype)


def check_close(out, ref, what):
    st = om.parity_stats(out, ref)
    assert st["rel_max_err"] < 5e-3 and st["cos"] > 0.99999, f"{what}: {st}"


def run_stages(capi, x, mats, what, cols=None):
    """Both stages on the device; `cols` restricts the down check to those
    output columns (None: all)."""
    xd, md = to_dev(x, mats)
    gp, gs, up, us, dp, ds = mats
    h = capi.gate_up(xd, *md[:4], path=SKINNY)
    torch.cuda.synchronize()
    h_ref = h_semantics(x, gp, gs, up, us)
    check_close(h.cpu(), h_ref, f"{what} gate_up")
    # down from the oracle's h, so the two stages are checked independently
    out = capi.down(h_ref.cuda(), md[4], md[5], path=SKINNY)
    torch.cuda.synchronize()
    out_ref = down_semantics(h_ref, dp, ds)
    out = out.cpu()
    if cols is not None:
        out, out_ref = out[:, cols], out_ref[:, cols]
    check_close(out, out_ref, f"{what} down")
    return out, out_ref


@pytest.mark.parametrize("h,i", [
    (512, 1536),    # gate_up: 2 segments over 8 waves (6 waves have none); down: 6 segments
    (1536, 512),    # gate_up: 6 segments, some waves empty; down: 2 segments
    (2560, 1024),   # 10 segments: runs of 1 and 2 (partial units)
    (1024, 5120),   # down: 20 segments, runs of 2 and 3 in units of 3
    (5120, 1024),   # gate_up: runs of 2 and 3 -> two units per row group
    (512, 64),      # 8 row groups: fewer than CUs
])
@pytest.mark.parametrize("m", [1, 3, 8])
def test_stream_stage_shapes(capi, h, i, m):
    banner(f"stream stages h={h} i={i} m={m}")
    x, mats = make_case(m, h, i, seed=7 * h + i + m)
    run_stages(capi, x, mats, f"h={h} i={i} m={m}")


@pytest.mark.parametrize("m", [1, 2, 5, 8])
def test_stream_many_row_groups_per_workgroup(capi, m):
    """32768 rows of gate/up: 16 row groups per workgroup on a 256-CU part,
    the LDS scale block and the output staging at their largest here."""
    banner(f"stream many row groups m={m}")
    x, mats = make_case(m, 512, 32768, seed=900 + m)
    run_stages(capi, x, mats, f"rows=32768 m={m}")


def test_stream_scale_bytes_outside_fast_range(capi):
    """Scale bytes 0, 1, 253 and 254 take the exact dequantisation branch of
    the unit (products are subnormal or near the top of the range); every
    other block stays on the hardware conversion."""
    banner("stream exact-scale branch")
    x, mats = make_case(2, 1024, 2048, seed=77)
    gp, gs, up, us, dp, ds = [np.array(a) for a in mats]
    gs[3, 0] = 0
    gs[700, 5] = 1
    us[11, 2] = 1
    # large scales on down: one nonzero code (0.5) in the block keeps the
    # output finite (0.5 * 2^126 or 2^127 times an h of order 0.1)
    for row, blk, byte in ((17, 9, 253), (900, 60, 254)):
        ds[row, blk] = byte
        dp[row, blk * 16:(blk + 1) * 16] = 0
        dp[row, blk * 16 + 3] = 0x10        # element 7 of the block: code 1
    mats = [gp, gs, up, us, dp, ds]
    # the two huge rows on their own, then every other row at its own scale
    big = [17, 900]
    out, ref = run_stages(capi, x, mats, "exact-scale big rows", cols=big)
    assert torch.isfinite(ref.float()).all() and ref.float().abs().min() > 1e30
    rest = [c for c in range(1024) if c not in big]
    run_stages(capi, x, mats, "exact-scale other rows", cols=rest)


def test_stream_fp16_activations(capi):
    banner("stream fp16")
    x, mats = make_case(4, 1024, 3072, seed=31, dtype=torch.float16)
    run_stages(capi, x, mats, "fp16")


@pytest.mark.parametrize("m", [3, 8])
def test_stream_fp16_qwen3_8b(capi, m):
    banner(f"stream fp16 8B m={m}")
    x, mats = make_case(m, 4096, 12288, seed=33 + m, dtype=torch.float16)
    run_stages(capi, x, mats, f"fp16 8B m={m}")


def test_stream_fp16_scale_paths(capi):
    """fp16 with scale bytes 104..113 (fp16-subnormal weights, fp16 MFMAs) and
    below 104 (those units on exact bf16 weights against the activations'
    bf16 hi and lo parts): every other output within the bar, the rows that
    read only such a block exact to one fp16 unit."""
    from tests.test_gpu_gemm import _isolate_block, _ulps_f16
    banner("stream fp16 scale paths")
    x, mats = make_case(5, 2048, 6144, seed=79, dtype=torch.float16)
    gp, gs, up, us, dp, ds = [np.array(a) for a in mats]
    gs[40, 3] = 90
    us[1500, 20] = 95
    rows = {5: 104, 333: 109, 600: 103, 1000: 113}
    for row, byte in rows.items():
        _isolate_block(dp, ds, [row], 7, byte)
    mats = [gp, gs, up, us, dp, ds]
    run_stages(capi, x, mats, "fp16 scale paths", cols=[c for c in range(2048) if c not in rows])
    xd, md = to_dev(x, mats)
    h_ref = h_semantics(x, gp, gs, up, us)
    o = capi.down(h_ref.cuda(), md[4], md[5], path=SKINNY).cpu()
    o_ref = down_semantics(h_ref, dp, ds)
    for row in rows:
        assert o_ref[:, row].float().abs().max() > 0
        assert _ulps_f16(o[:, row], o_ref[:, row]) <= 1, row


def test_stream_full_call_matches_stages(capi):
    """The full entry point on the decode path gives the same bits as its two
    stage entry points."""
    banner("stream full vs stages")
    x, mats = make_case(1, 4096, 12288, seed=5)
    xd, md = to_dev(x, mats)
    tmp_full = torch.empty((1, 12288), dtype=xd.dtype, device="cuda")
    full = capi.mlp_forward(xd, *md, tmp=tmp_full, path=SKINNY)
    tmp = capi.gate_up(xd, *md[:4], path=SKINNY)
    out = capi.down(tmp, *md[4:], path=SKINNY)
    torch.cuda.synchronize()
    assert torch.equal(tmp.view(torch.int16), tmp_full.view(torch.int16))
    assert torch.equal(out.view(torch.int16), full.view(torch.int16))
    check_close(full.cpu(), om.mlp_kernel_semantics(x, *mats), "8B full")
