"""Benchmark of the MXFP4 weight-only Qwen3 MLP on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

Headline workload (BASELINE.json metric): the Qwen3-8B-shaped MLP
(hidden 4096, intermediate 12288) at M=1 decode, reported as algorithmic HBM
GB/s (``value``), and at M=2048 prefill, reported as bf16 TFLOP/s
(``prefill``).  A step is one MLP call (gate_up + SiLU*up + down) over one
batch of seeded synthetic activations, with the weight set rotated every step
over enough independently seeded sets (>= 2 x 256 MiB) that the 256 MB
Infinity Cache cannot hold them: every step streams its weights from HBM.

Timing: W untimed warm-up steps, then a HIP graph of exactly K steps is
replayed R = max(10, ceil(200 / K)) times, each replay bracketed by HIP
events on the stream the kernels run on (torch's current stream, which the C
ABI is handed) and by device synchronizations.  Per-step time of a replay =
its event time / K; ``ms_per_step`` and ``value`` come from the median over
the R replays (>= 200 timed MLP calls), ``us_per_step_p10_p50_p90`` from the
same replays.  The dominant kernel (the gate_up stage) is timed the same way
on its own for the ``roofline`` object, at M=1 and at M=2048.

``hot_cache`` (and ``prefill.hot_cache_us_per_call``) repeats the timing
with one weight set reused every call, so the weights sit in the MALL:
labelled as such, never the headline.  ``prefill.vendor_bf16_gemm`` times
torch's bf16 GEMM (hipBLASLt) on bf16 weights of the same shapes, an
achievable matrix-core reference; ``device_max_clock_mhz`` is rocminfo's.

``points`` holds the other BASELINE configurations, each timed the same way
with its own rotated weight sets: Qwen3-1.7B at M=1/4/8, Qwen3-8B at
M=16/64/256/512, and the Qwen3-32B 64-layer stack at M=1/512.
``cpu_baseline`` times the CPU restatement of the reference's torch
dequant-then-matmul path (the oracle) on this host: the whole call at 8B
M=1 and M=2048 (per-call dequant + matmul, and matmul only), and per other
configuration the dequant and the matmul-only parts.

Work per MLP call:  bytes = 3*H*I*(1/2 + 1/32) + 4*M*H,  flops = 6*M*H*I.
Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
MALL_BYTES = 256 * 2 ** 20     # Infinity Cache
PROFILE_DIR = os.path.join(ROOT, "profiles")
MIN_TIMED_CALLS = 200          # timed MLP calls per reported figure
MIN_REPLAYS = 10

METRIC = "MXFP4 MLP GB/s (M=1) & TFLOP/s (M=2048), Qwen3-8B shape, % of peak"
NORM_EPS = 1e-6                # Qwen3's rms_norm_eps


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100, help="MLP calls per timed graph replay")
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--config", default="qwen3-8b")
    p.add_argument("--m", type=int, default=1, help="headline token count")
    p.add_argument("--prefill-m", type=int, default=2048, help="prefill token count (0: skip)")
    p.add_argument("--quick", action="store_true", help="headline, roofline and prefill only (no points)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=30.0, help="CPU baseline budget (whole run)")
    p.add_argument("--copy-probe", action="store_true",
                   help="only run a 256 MiB device copy (calibrates rocprof FETCH/WRITE_SIZE)")
    p.add_argument("--only", choices=["decode", "gate_up", "down", "prefill", "prefill_gate_up", "prefill_down",
                                      "norm_mlp"], default=None,
                   help="run a single timed loop (for rocprofv3 runs)")
    p.add_argument("--path", type=int, default=0,
                   help="kernel path for --only runs (0 auto, 1 skinny/stream, 2 GEMM, 3 fused decode)")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----------------------------------------------------------------- inputs

def weight_sets(shape, min_bytes=2 * MALL_BYTES, generator="cpu"):
    """Independently seeded quantized weight sets whose total exceeds
    ``min_bytes`` (set s uses the seeds of layer s: 1000+3*s+{0,1,2}), drawn
    with torch's CPU generator as BASELINE specifies, quantized on the GPU."""
    from tinyinfer_amd.workloads import quantized_weights, weight_bytes
    per = weight_bytes(shape.hidden, shape.inter)
    n = max(1, math.ceil(min_bytes / per))
    return [quantized_weights(shape.hidden, shape.inter, layer=s, generator=generator) for s in range(n)]


def quantiles(v):
    s = sorted(v)
    pick = lambda q: s[min(len(s) - 1, int(round(q * (len(s) - 1))))]
    return pick(0.1), pick(0.5), pick(0.9)


def replays_for(steps: int) -> int:
    return max(MIN_REPLAYS, math.ceil(MIN_TIMED_CALLS / max(1, steps)))


class Runner:
    """Graph-captured loops of MLP calls (full MLP or one stage)."""

    def __init__(self, capi, x, sets, kind, path=0):
        import torch
        self.capi, self.x, self.sets, self.kind, self.path = capi, x, sets, kind, path
        m, h = x.shape
        i = sets[0][0].shape[0]
        self.tmp = torch.empty((m, i), dtype=x.dtype, device=x.device)
        self.out = torch.empty((m, h), dtype=x.dtype, device=x.device)
        if kind in ("norm_mlp", "norm_then_mlp"):
            g = torch.Generator(device="cpu").manual_seed(17)
            self.nw = (1.0 + 0.1 * torch.randn(h, generator=g)).to(x.dtype).to(x.device)
            self.xn = torch.empty((m, h), dtype=x.dtype, device=x.device)

    def step(self, s):
        c, w = self.capi, self.sets[s % len(self.sets)]
        if self.kind == "mlp":
            c.mlp_forward(self.x, *w, out=self.out, tmp=self.tmp, path=self.path)
        elif self.kind == "norm_mlp":          # RMSNorm in the MLP's prologue, residual in its epilogue
            c.mlp_forward_rmsnorm(self.x, self.nw, NORM_EPS, *w, out=self.out, tmp=self.tmp, xn=self.xn,
                                  path=self.path)
        elif self.kind == "norm_then_mlp":     # the same layer half with the norm as its own kernel
            c.rmsnorm(self.x, self.nw, NORM_EPS, out=self.xn)
            c.mlp_forward(self.xn, *w, out=self.out, tmp=self.tmp, path=self.path, residual=self.x)
        elif self.kind == "gate_up":
            c.gate_up(self.x, *w[:4], tmp=self.tmp, path=self.path)
        else:
            c.down(self.tmp, *w[4:], out=self.out, path=self.path)

    def warm(self, n):
        import torch
        for s in range(n):
            self.step(s)
        torch.cuda.synchronize()

    def graph(self, steps):
        import torch
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.step(0)                      # first call on this stream outside capture
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        # capture on the warmed stream: the library's split-K workspace for it
        # exists (allocation cannot happen during capture)
        with torch.cuda.graph(g, stream=side):
            for s in range(steps):
                self.step(s)
        torch.cuda.synchronize()
        return g

    def time_graph(self, steps, reps=None):
        """Per-step milliseconds of each of `reps` timed replays of one
        `steps`-call graph (after one untimed replay), and the wall time of
        the timed replays."""
        import torch
        reps = reps or replays_for(steps)
        g = self.graph(steps)
        g.replay()                            # warm replay
        torch.cuda.synchronize()
        per = []
        t0 = time.perf_counter()
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record()
            g.replay()
            b.record()
            torch.cuda.synchronize()
            per.append(a.elapsed_time(b) / steps)
        wall = time.perf_counter() - t0
        del g
        return per, wall


def gpu_max_clock_mhz():
    """The GPU agent's maximum engine clock as rocminfo reports it (run as a
    child process before this process touches the GPU), or None."""
    import subprocess
    try:
        out = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=60).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    agent, clocks = "", []
    for line in out.splitlines():
        t = line.strip()
        if t.startswith("Name:"):
            agent = t.split(":", 1)[1].strip()
        elif t.startswith("Max Clock Freq. (MHz):") and agent.startswith("gfx"):
            try:
                clocks.append(int(t.split(":", 1)[1].strip()))
            except ValueError:
                pass
    return max(clocks) if clocks else None


def vendor_gemm_reference(shape, m, steps=20):
    """torch's bf16 GEMM (hipBLASLt) on bf16 weights of the MLP's shapes at M
    tokens -- gate and up as one [2I, H] product, down as [H, I] -- timed with
    events around ``steps`` calls after a warm-up: an achievable matrix-core
    reference for the prefill roofline, not this library's work."""
    import torch
    import torch.nn.functional as F
    h_, i_ = shape.hidden, shape.inter
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(m, h_, generator=g, device="cuda").to(torch.bfloat16)
    w_gu = (0.02 * torch.randn(2 * i_, h_, generator=g, device="cuda")).to(torch.bfloat16)
    hh = torch.randn(m, i_, generator=g, device="cuda").to(torch.bfloat16)
    w_d = (0.02 * torch.randn(h_, i_, generator=g, device="cuda")).to(torch.bfloat16)

    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / steps * 1e3

    gu_us = timed(lambda: F.linear(x, w_gu))
    dn_us = timed(lambda: F.linear(hh, w_d))
    flops = 6.0 * m * h_ * i_
    del x, w_gu, hh, w_d
    torch.cuda.empty_cache()
    return {"what": "torch bf16 F.linear (hipBLASLt) on bf16 weights of the same shapes: achievable MFMA "
                    "reference, not MXFP4", "m": m, "gate_up_us": round(gu_us, 2), "down_us": round(dn_us, 2),
            "tflops": round(flops / ((gu_us + dn_us) * 1e-6) / 1e12, 1)}


def eager_call_us(runner, calls=200):
    """Python-call wall time per MLP call (eager, incl. host overhead)."""
    import torch
    runner.warm(20)
    t0 = time.perf_counter()
    for s in range(calls):
        runner.step(s)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / calls * 1e6


# ----------------------------------------------------------------- CPU baseline

def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _timed(fn, runs, budget_s):
    """Median seconds of ``fn`` after one warm-up: ``runs`` runs, fewer (at
    least two) when the budget runs out."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= 2 and time.perf_counter() > t_end:
            break
    return statistics.median(times), len(times)


def cpu_baseline(budget_s, quick):
    """The oracle's restatement of the reference torch CPU path (weights
    decoded with torch ops to fp32 then bf16, three F.linear calls,
    SiLU*up) on this host's cores.  Whole calls at the headline shape (8B)
    at M=1 and M=2048: (i) per-call dequant + matmul, (ii) matmul only on
    pre-dequantized bf16 weights.  For the other configurations the two
    parts are timed separately (the dequant once per shape, the matmul per
    M) and (i) is their sum; for the 32B stack the dequant is timed on a
    quarter of one layer's rows and the matmul on one whole layer, both
    scaled to 64 layers.  The packed weights are the GPU runs' own (same
    seeds), copied to the host; only the CPU work is timed."""
    import torch
    from oracle import mlp as om
    from tinyinfer_amd.workloads import SHAPES, activations, alg_bytes, alg_flops, quantized_weights

    torch.set_num_threads(os.cpu_count() or 1)
    t_start = time.perf_counter()

    def mats_for(shp, generator):
        return [a.cpu() for a in quantized_weights(shp.hidden, shp.inter, layer=0, generator=generator)]

    def dequant_all(mats, rows=None):
        return tuple(om.dequant_weight(mats[2 * j][:rows], mats[2 * j + 1][:rows], torch.bfloat16, "torch")
                     for j in range(3))

    res = {"unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
           "os_cpu_count": os.cpu_count(), "cpu_model": _cpu_model()}
    h8 = SHAPES["qwen3-8b"]
    mats8 = mats_for(h8, "cpu")
    whole = {}
    for m in (1, 2048):
        x = activations(m, h8.hidden, device="cpu")
        t_i, n_i = _timed(lambda: om.mlp_reference(x, *mats8, impl="torch"), 5, budget_s * 0.15)
        wts = dequant_all(mats8)
        t_ii, n_ii = _timed(lambda: om.mlp_reference(x, *mats8, weights=wts), 5, budget_s * 0.1)
        b, f = alg_bytes(m, h8.hidden, h8.inter), alg_flops(m, h8.hidden, h8.inter)
        whole[m] = {"config": h8.name, "m": m, "ms_per_call": round(t_i * 1e3, 3), "runs": n_i,
                    "gbs": round(b / t_i / 1e9, 3), "tflops": round(f / t_i / 1e12, 4),
                    "matmul_only_ms": round(t_ii * 1e3, 3), "matmul_only_runs": n_ii,
                    "matmul_only_gbs": round(b / t_ii / 1e9, 3), "matmul_only_tflops": round(f / t_ii / 1e12, 4)}
        log(f"cpu {h8.name} M={m}: {t_i * 1e3:.1f} ms/call, matmul only {t_ii * 1e3:.1f} ms")
    w1 = whole[1]
    res.update({"value": w1["gbs"], "ms_per_call": w1["ms_per_call"], "matmul_only_gbs": w1["matmul_only_gbs"],
                "prefill": whole[2048]})
    res["sample"] = (f"{w1['runs']} whole calls of the torch CPU dequant-then-matmul path at {h8.name} M=1 "
                     f"(median {w1['ms_per_call']:.1f} ms/call) and {whole[2048]['runs']} at M=2048 "
                     f"(median {whole[2048]['ms_per_call']:.1f} ms/call), each after one warm-up; "
                     "matmul-only variants on pre-dequantized bf16 weights beside them")
    if quick:
        return res
    pts = []
    rest = max(4.0, budget_s - (time.perf_counter() - t_start))
    plan = (("qwen3-1.7b", (1, 4, 8), "cpu", None), ("qwen3-8b", (16, 64, 256, 512), "cpu", None),
            ("qwen3-32b", (1, 512), "cuda", 4))
    for name, ms_, gen, frac in plan:
        shp = SHAPES[name]
        mats = mats8 if name == h8.name else mats_for(shp, gen)
        if frac is None:
            t_dq, n_dq = _timed(lambda: dequant_all(mats), 3, rest / 10)
        else:   # a quarter of each matrix's rows, scaled by 4 (elementwise work)
            part = [a[: a.shape[0] // frac] for a in mats]
            t_dq, n_dq = _timed(lambda: dequant_all(part), 3, rest / 10)
            t_dq *= frac
        wts = dequant_all(mats)
        scale = shp.layers
        for m in ms_:
            x = activations(m, shp.hidden, device="cpu")
            t_mm, n_mm = _timed(lambda: om.mlp_reference(x, *mats, weights=wts), 5, rest / 20)
            t_i = (t_dq + t_mm) * scale
            b = shp.layers * alg_bytes(m, shp.hidden, shp.inter)
            f = shp.layers * alg_flops(m, shp.hidden, shp.inter)
            note = "dequant and matmul timed separately, summed"
            if shp.layers > 1:
                note += (f"; one layer timed (dequant on 1/{frac} of its rows x{frac}), x{shp.layers} layers "
                         "(extrapolated)")
            pts.append({"config": name + (f" x{shp.layers} layers" if shp.layers > 1 else ""), "m": m,
                        "ms_per_call": round(t_i * 1e3, 3), "gbs": round(b / t_i / 1e9, 3),
                        "tflops": round(f / t_i / 1e12, 4), "matmul_only_ms": round(t_mm * scale * 1e3, 3),
                        "matmul_only_gbs": round(b / (t_mm * scale) / 1e9, 3),
                        "dequant_ms": round(t_dq * scale * 1e3, 3), "runs": [n_dq, n_mm], "note": note})
            log(f"cpu {name} M={m}: {t_i * 1e3:.1f} ms/call (dequant {t_dq * scale * 1e3:.1f})")
        del mats, wts
    res["points"] = pts
    return res


# ----------------------------------------------------------------- profiles

def committed_profile(name):
    """A JSON summary committed under profiles/ (rocprofv3 counters of a
    kernel on a workload, with the commands that produced it); None if absent."""
    try:
        with open(os.path.join(PROFILE_DIR, name)) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def committed_traffic(kernel, workload):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration), committed under
    profiles/ as traffic_<kernel>_<workload>.json; None if absent."""
    rec = committed_profile(f"traffic_{kernel}_{workload}.json")
    return rec.get("bytes_per_launch") if rec else None


# ----------------------------------------------------------------- GPU points

def measure_point(capi, shape, m, sets, steps, path=0):
    from tinyinfer_amd.workloads import activations, alg_bytes, alg_flops
    x = activations(m, shape.hidden, device="cuda")
    r = Runner(capi, x, sets, "mlp", path)
    r.warm(5)
    per, _ = r.time_graph(steps)
    p10, ms, p90 = quantiles(per)
    b, f = alg_bytes(m, shape.hidden, shape.inter), alg_flops(m, shape.hidden, shape.inter)
    return {"config": shape.name, "m": m, "us_per_call": round(ms * 1e3, 3),
            "us_p10_p90": [round(p10 * 1e3, 3), round(p90 * 1e3, 3)],
            "gbs": round(b / ms / 1e6, 1), "tflops": round(f / ms / 1e9, 2),
            "hbm_frac": round(b / ms / 1e6 / HBM_PEAK_GBS, 4),
            "mfma_frac": round(f / ms / 1e9 / BF16_PEAK_TFLOPS, 4),
            "tok_s": round(m / (ms * 1e-3), 1), "timed_calls": steps * len(per), "weight_sets": len(sets)}


def measure_stack(capi, m, layers, reps=5):
    """BASELINE's Qwen3-32B config: 64 MLP layers (hidden 5120, intermediate
    25600, ~13.4 GB of MXFP4 weights, far beyond the MALL) with the residual
    add between layers; one graph per pass (x reset from x0 inside it).  On
    these synthetic weights the plain stack overflows bf16 after a few layers
    (the MLP is quadratic in x); the speed of the kernels does not depend on
    the activation values."""
    import torch
    from tinyinfer_amd.workloads import SHAPES, activations, alg_bytes, alg_flops, mlp_stack_step
    shp = SHAPES["qwen3-32b"]
    x0 = activations(m, shp.hidden, device="cuda")
    x = x0.clone()
    out = torch.empty_like(x0)
    tmp = torch.empty((m, shp.inter), dtype=x0.dtype, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        mlp_stack_step(capi, x, layers, out, tmp)           # warm-up pass on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        x.copy_(x0)
        mlp_stack_step(capi, x, layers, out, tmp)
    g.replay()
    torch.cuda.synchronize()
    per = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        per.append(a.elapsed_time(b))
    del g
    p10, ms, p90 = quantiles(per)
    byt = shp.layers * alg_bytes(m, shp.hidden, shp.inter)
    fl = shp.layers * alg_flops(m, shp.hidden, shp.inter)
    return {"config": f"{shp.name} x{shp.layers} layers + residual", "m": m, "ms_per_pass": round(ms, 4),
            "ms_p10_p90": [round(p10, 4), round(p90, 4)],
            "tok_s": round(m / (ms * 1e-3), 1), "gbs": round(byt / ms / 1e6, 1),
            "hbm_frac": round(byt / ms / 1e6 / HBM_PEAK_GBS, 4), "tflops": round(fl / ms / 1e9, 2),
            "mfma_frac": round(fl / ms / 1e9 / BF16_PEAK_TFLOPS, 4), "timed_calls": reps * shp.layers,
            "note": "residual add fused into each layer's down epilogue (in place), included in the time; "
                    "weights drawn with the GPU generator (64 x 3 seeded N(0,0.02) matrices)"}


def stage_roofline(capi, x, sets, steps, m, shape, bound):
    """The gate_up stage (the MLP's dominant kernel) timed alone; down beside it."""
    h, i = shape.hidden, shape.inter
    gu = Runner(capi, x, sets, "gate_up")
    gu.warm(3)
    gu_ms = statistics.median(gu.time_graph(steps)[0])
    dn = Runner(capi, x, sets, "down")
    dn.warm(3)
    dn_ms = statistics.median(dn.time_graph(steps)[0])
    workload = f"{shape.name}-m{m}"
    if bound == "hbm":
        gu_bytes = 2 * i * h // 2 + 2 * i * h // 32 + 2 * m * h + 2 * m * i
        ach = gu_bytes / (gu_ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": committed_traffic("gate_up", workload),
                "kernel": ("gate_up stage: rowstream_kernel (1 KB single-row loads, MFMA diagonal dot "
                           "products, SiLU*up epilogue)" if m == 1 else "gate_up stage"),
                "us_per_launch": round(gu_ms * 1e3, 3), "alg_bytes_per_launch": gu_bytes,
                "down_us_per_launch": round(dn_ms * 1e3, 3)}
    gu_flops = 4 * m * h * i
    ach = gu_flops / (gu_ms * 1e-3) / 1e12
    busy = committed_profile(f"mfma_gate_up_gemm_{workload}.json")
    return {"bound": "mfma", "achieved": round(ach, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(ach / BF16_PEAK_TFLOPS, 4), "traffic": committed_traffic("gate_up_gemm", workload),
            "kernel": "gate_up stage: gemm_ring_kernel (direct-to-LDS ring, dequant to bf16, "
                      "v_mfma_f32_32x32x16_bf16, SiLU*up epilogue)",
            "us_per_launch": round(gu_ms * 1e3, 3), "alg_flops_per_launch": gu_flops,
            "down_us_per_launch": round(dn_ms * 1e3, 3),
            "down_tflops": round(2 * m * h * i / (dn_ms * 1e-3) / 1e12, 1),
            "mfma_busy": busy.get("mfma_busy") if busy else None}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported here "
              "(the MXFP4 MLP would shard as tensor parallelism over the intermediate dimension; "
              "no multi-GPU figure is produced in this build).", file=sys.stderr)
        sys.exit(2)
    clock_mhz = gpu_max_clock_mhz() if not (args.only or args.copy_probe) else None
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a gfx950 GPU (none visible)", file=sys.stderr)
        sys.exit(1)
    from tinyinfer_amd import capi
    from tinyinfer_amd.extension import load_extension
    from tinyinfer_amd.workloads import SHAPES, activations, alg_bytes, quantized_weights

    capi.lib()
    load_extension()
    torch.cuda.set_device(0)
    dev_name = torch.cuda.get_device_properties(0).name

    if args.copy_probe:
        n = 256 * 2 ** 20
        a = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "launches": 5}))
        return

    shape = SHAPES[args.config]
    m = args.m
    t_setup = time.perf_counter()
    sets = weight_sets(shape)
    torch.cuda.synchronize()
    log(f"{len(sets)} weight sets of {shape.name} ready in {time.perf_counter() - t_setup:.1f}s on {dev_name}")
    x = activations(m, shape.hidden, device="cuda")

    if args.only:
        kind = {"decode": "mlp", "gate_up": "gate_up", "down": "down", "prefill": "mlp",
                "prefill_gate_up": "gate_up", "prefill_down": "down", "norm_mlp": "norm_mlp"}[args.only]
        mm = args.prefill_m if args.only.startswith("prefill") else m
        r = Runner(capi, activations(mm, shape.hidden, device="cuda"), sets, kind, path=args.path)
        r.warm(args.warmup)
        per, _ = r.time_graph(args.steps, reps=1)
        print(json.dumps({"only": args.only, "m": mm, "us_per_call": round(per[0] * 1e3, 3)}))
        return

    # -- headline: R replays of a K-step graph of the M=m MLP -----------------
    runner = Runner(capi, x, sets, "mlp")
    runner.warm(args.warmup)
    per, wall = runner.time_graph(args.steps)
    p10, ms_step, p90 = quantiles(per)
    b1 = alg_bytes(m, shape.hidden, shape.inter)
    value = b1 / (ms_step * 1e-3) / 1e9
    log(f"M={m}: {ms_step * 1e3:.2f} us/step (median of {len(per)} replays x {args.steps} steps), "
        f"{value:.1f} GB/s")
    py_us = eager_call_us(runner)
    roofline = stage_roofline(capi, x, sets, args.steps, m, shape, "hbm")
    # hot cache: one weight set reused every call (80 MB at 8B: resident in
    # the 256 MB MALL), reported beside the rotated headline, never as it
    hot = Runner(capi, x, sets[:1], "mlp")
    hot.warm(5)
    hot_ms = statistics.median(hot.time_graph(args.steps)[0])
    hot_cache = {"what": "one weight set reused every call (weights MALL-resident); not the headline",
                 "m": m, "us_per_call": round(hot_ms * 1e3, 3), "gbs": round(b1 / (hot_ms * 1e-3) / 1e9, 1)}
    del hot

    # -- the decoder layer's MLP half: RMSNorm + MLP + residual ----------------
    nm = Runner(capi, x, sets, "norm_mlp")
    nm.warm(3)
    nm_ms = statistics.median(nm.time_graph(args.steps)[0])
    sp = Runner(capi, x, sets, "norm_then_mlp")
    sp.warm(3)
    sep_ms = statistics.median(sp.time_graph(args.steps)[0])
    decoder_half = {"what": "x + MLP(RMSNorm(x)) per call, M=%d" % m,
                    "fused_us": round(nm_ms * 1e3, 3), "norm_kernel_then_mlp_us": round(sep_ms * 1e3, 3)}
    log(f"decoder half: fused {nm_ms * 1e3:.2f} us, norm kernel + MLP {sep_ms * 1e3:.2f} us")

    # -- prefill headline -------------------------------------------------------
    prefill = None
    if args.prefill_m:
        psteps = min(args.steps, 20)
        pt = measure_point(capi, shape, args.prefill_m, sets, psteps)
        xp = activations(args.prefill_m, shape.hidden, device="cuda")
        prefill = {"m": args.prefill_m, "tflops": pt["tflops"], "frac": pt["mfma_frac"],
                   "us_per_call": pt["us_per_call"], "us_p10_p90": pt["us_p10_p90"], "gbs": pt["gbs"],
                   "tok_s": pt["tok_s"], "timed_calls": pt["timed_calls"],
                   "roofline": stage_roofline(capi, xp, sets, psteps, args.prefill_m, shape, "mfma")}
        hp = Runner(capi, xp, sets[:1], "mlp")
        hp.warm(2)
        hp_ms = statistics.median(hp.time_graph(psteps)[0])
        prefill["hot_cache_us_per_call"] = round(hp_ms * 1e3, 3)
        del hp, xp
        prefill["vendor_bf16_gemm"] = vendor_gemm_reference(shape, args.prefill_m)
        log(f"M={args.prefill_m}: {pt['us_per_call']:.1f} us/call, {pt['tflops']:.1f} TFLOP/s")

    points = []
    if not args.quick:
        for mm in (16, 64, 256, 512):
            points.append(measure_point(capi, shape, mm, sets, 50 if mm <= 64 else 20))
            log(json.dumps(points[-1]))
        del sets
        torch.cuda.empty_cache()
        shp = SHAPES["qwen3-1.7b"]
        st = weight_sets(shp)
        for mm in (1, 4, 8):
            points.append(measure_point(capi, shp, mm, st, args.steps))
            log(json.dumps(points[-1]))
        del st
        torch.cuda.empty_cache()
        shp = SHAPES["qwen3-32b"]
        t0 = time.perf_counter()
        layers = [quantized_weights(shp.hidden, shp.inter, layer=l, generator="cuda") for l in range(shp.layers)]
        torch.cuda.synchronize()
        log(f"{shp.layers} layers of {shp.name} ready in {time.perf_counter() - t0:.1f}s")
        for mm in (1, 512):
            points.append(measure_stack(capi, mm, layers))
            log(json.dumps(points[-1]))
        del layers
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        log(f"timing the CPU baseline (~{args.cpu_seconds:.0f}s)")
        cpu = cpu_baseline(args.cpu_seconds, args.quick)

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded N(0,0.02) weights (torch CPU generator) quantized to MXFP4 on device, "
                "N(0,1) bf16 activations",
        "config": {"workload": f"{shape.name} MXFP4 MLP (hidden {shape.hidden}, intermediate {shape.inter}) "
                               f"decode M={m}, {len(runner.sets)} rotated weight sets",
                   "hidden": shape.hidden, "intermediate": shape.inter, "m": m},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "timed_calls": args.steps * len(per), "replays": len(per),
        "us_per_step_p10_p50_p90": [round(1e3 * q, 3) for q in (p10, ms_step, p90)],
        "wall_ms_timed_region": round(wall * 1e3, 3),
        "python_call_us": round(py_us, 2),
        "hot_cache": hot_cache,
        "roofline": roofline,
        "decoder_half": decoder_half,
        "prefill": prefill,
        "cpu_baseline": cpu,
        "points": points or None,
        "device": dev_name,
        "device_max_clock_mhz": clock_mhz,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
