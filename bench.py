"""Benchmark of the MXFP4 weight-only Qwen3 MLP on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--all]

Headline workload (BASELINE.json metric): the Qwen3-8B-shaped MLP
(hidden 4096, intermediate 12288) at M=1 decode, reported as algorithmic HBM
GB/s (``value``), and at M=2048 prefill, reported as bf16 TFLOP/s
(``prefill``).  A step is one MLP call (gate_up + SiLU*up + down) over one
batch of seeded synthetic activations, with the weight set rotated every step
over enough independently seeded sets (>= 2 x 256 MiB) that the 256 MB
Infinity Cache cannot hold them: every step streams its weights from HBM.

Timing: W untimed warm-up steps, then exactly K steps captured in one HIP
graph and replayed once between two device synchronizations (the graph keeps
host launch overhead out of the M=1 number); HIP events on the stream the
kernels run on (torch's current stream, which the C ABI is handed) bracket
the replay.  The dominant kernel (the gate_up stage) is timed the same way
on its own for the ``roofline`` object.  ``cpu_baseline`` times the CPU
restatement of the reference's torch dequant-then-matmul path (the oracle)
on a bounded sample of the same workload on this host.

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

METRIC = "MXFP4 MLP GB/s (M=1) & TFLOP/s (M=2048), Qwen3-8B shape, % of peak"
NORM_EPS = 1e-6                # Qwen3's rms_norm_eps


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000, help="timed M=1 steps (one MLP call each)")
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--config", default="qwen3-8b")
    p.add_argument("--m", type=int, default=1, help="headline token count")
    p.add_argument("--prefill-m", type=int, default=2048, help="prefill token count (0: skip)")
    p.add_argument("--prefill-steps", type=int, default=100)
    p.add_argument("--all", action="store_true",
                   help="also measure every other BASELINE config (1.7B decode, 8B M=256/512, 32B 64-layer stack) "
                        "and 8B small batches (M=16, 64)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline sample budget")
    p.add_argument("--copy-probe", action="store_true",
                   help="only run a 256 MiB device copy (calibrates rocprof FETCH/WRITE_SIZE)")
    p.add_argument("--only", choices=["decode", "gate_up", "down", "prefill", "norm_mlp"], default=None,
                   help="run a single timed loop (for rocprofv3 runs)")
    p.add_argument("--path", type=int, default=0,
                   help="kernel path for --only runs (0 auto, 1 skinny/stream, 2 GEMM, 3 fused decode)")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ----------------------------------------------------------------- inputs

def weight_sets(shape, min_bytes=2 * MALL_BYTES):
    """Independently seeded quantized weight sets whose total exceeds
    ``min_bytes`` (layer index = set index -> seeds 1000+3*set+{0,1,2})."""
    from tinyinfer_amd.workloads import quantized_weights, weight_bytes
    per = weight_bytes(shape.hidden, shape.inter)
    n = max(1, math.ceil(min_bytes / per))
    sets = [quantized_weights(shape.hidden, shape.inter, layer=s, generator="cuda") for s in range(n)]
    return sets


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

    def time_graph(self, steps, reps=1):
        """Per-step milliseconds of `reps` replays of a `steps`-call graph."""
        import torch
        g = self.graph(steps)
        g.replay()                            # warm replay
        torch.cuda.synchronize()
        per = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record()
            g.replay()
            b.record()
            torch.cuda.synchronize()
            per.append(a.elapsed_time(b) / steps)
        del g
        return per


def eager_call_us(runner, calls=200):
    """Python-call wall time per MLP call (eager, incl. host overhead)."""
    import torch
    for s in range(20):
        runner.step(s)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(calls):
        runner.step(s)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / calls * 1e6


# ----------------------------------------------------------------- CPU baseline

def cpu_baseline(shape, m, budget_s):
    """The oracle's restatement of the reference torch CPU path, timed on a
    bounded sample: per-call dequant + F.linear x3 (bf16) at the headline
    shape and M, repeated until ``budget_s`` of CPU work."""
    import torch
    from oracle import mlp as om
    from tinyinfer_amd.workloads import activations, alg_bytes, random_weights
    from oracle import mxfp4 as ox

    mats = []
    for w in random_weights(shape.hidden, shape.inter, layer=0, generator="cpu"):
        mats.extend(ox.quantize_chunk(w))
    x = activations(m, shape.hidden, device="cpu")
    om.mlp_reference(x, *mats)                       # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 2 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        om.mlp_reference(x, *mats)
        times.append(time.perf_counter() - t0)
        if len(times) >= 2 and time.perf_counter() > t_end:
            break
    t = statistics.median(times)
    # matmul-only variant (pre-dequantized bf16 weights)
    wts = tuple(om.dequant_weight(mats[2 * j], mats[2 * j + 1], x.dtype) for j in range(3))
    om.mlp_reference(x, *mats, weights=wts)
    mm = []
    for _ in range(5):
        t0 = time.perf_counter()
        om.mlp_reference(x, *mats, weights=wts)
        mm.append(time.perf_counter() - t0)
    t_mm = statistics.median(mm)
    b = alg_bytes(m, shape.hidden, shape.inter)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(b / t / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{len(times)} calls of the torch CPU dequant-then-matmul path at {shape.name} "
                   f"M={m} (median {t * 1e3:.1f} ms/call); matmul-only with pre-dequantized bf16 weights "
                   f"{t_mm * 1e3:.1f} ms/call = {b / t_mm / 1e9:.3f} GB/s"),
        "ms_per_call": round(t * 1e3, 3),
        "matmul_only_gbs": round(b / t_mm / 1e9, 3),
        "os_cpu_count": os.cpu_count(),
        "cpu_model": model,
    }


# ----------------------------------------------------------------- traffic

def committed_traffic(kernel, workload):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration), committed under
    profiles/ as traffic_<kernel>_<workload>.json; None if absent."""
    path = os.path.join(PROFILE_DIR, f"traffic_{kernel}_{workload}.json")
    try:
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


# ----------------------------------------------------------------- main

def measure_point(capi, shape, m, sets, steps, path=0, reps=3):
    import torch
    from tinyinfer_amd.workloads import activations, alg_bytes, alg_flops
    x = activations(m, shape.hidden, device="cuda")
    r = Runner(capi, x, sets, "mlp", path)
    per = r.time_graph(steps, reps=reps)
    ms = statistics.median(per)
    b, f = alg_bytes(m, shape.hidden, shape.inter), alg_flops(m, shape.hidden, shape.inter)
    return {"config": shape.name, "m": m, "us_per_call": round(ms * 1e3, 3),
            "gbs": round(b / ms / 1e6, 1), "tflops": round(f / ms / 1e9, 2),
            "hbm_frac": round(b / ms / 1e6 / HBM_PEAK_GBS, 4),
            "mfma_frac": round(f / ms / 1e9 / BF16_PEAK_TFLOPS, 4),
            "tok_s": round(m / (ms * 1e-3), 1), "steps": steps, "weight_sets": len(sets)}


def measure_stack(capi, m, reps=5):
    """BASELINE's Qwen3-32B config: 64 MLP layers (hidden 5120, intermediate
    25600, ~13.4 GB of MXFP4 weights, far beyond the MALL) with the residual
    add between layers; one graph per pass (x reset from x0 inside it)."""
    import torch
    from tinyinfer_amd.workloads import SHAPES, activations, alg_bytes, alg_flops, mlp_stack_step, quantized_weights
    shp = SHAPES["qwen3-32b"]
    layers = [quantized_weights(shp.hidden, shp.inter, layer=l, generator="cuda") for l in range(shp.layers)]
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
    del g, layers
    torch.cuda.empty_cache()
    ms = statistics.median(per)
    byt = shp.layers * alg_bytes(m, shp.hidden, shp.inter)
    fl = shp.layers * alg_flops(m, shp.hidden, shp.inter)
    return {"config": f"{shp.name} x{shp.layers} layers + residual", "m": m, "ms_per_pass": round(ms, 4),
            "tok_s": round(m / (ms * 1e-3), 1), "gbs": round(byt / ms / 1e6, 1),
            "hbm_frac": round(byt / ms / 1e6 / HBM_PEAK_GBS, 4), "tflops": round(fl / ms / 1e9, 2),
            "mfma_frac": round(fl / ms / 1e9 / BF16_PEAK_TFLOPS, 4), "reps": reps,
            "note": "residual add fused into each layer's down epilogue (in place), included in the time"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported here "
              "(the MXFP4 MLP would shard as tensor parallelism over the intermediate dimension; "
              "no multi-GPU figure is produced in this build).", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a gfx950 GPU (none visible)", file=sys.stderr)
        sys.exit(1)
    from tinyinfer_amd import capi
    from tinyinfer_amd.extension import load_extension
    from tinyinfer_amd.workloads import SHAPES, activations, alg_bytes, alg_flops

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
                "norm_mlp": "norm_mlp"}[args.only]
        mm = args.prefill_m if args.only == "prefill" else m
        r = Runner(capi, activations(mm, shape.hidden, device="cuda"), sets, kind, path=args.path)
        for s in range(args.warmup):
            r.step(s)
        torch.cuda.synchronize()
        per = r.time_graph(args.steps, reps=1)
        print(json.dumps({"only": args.only, "m": mm, "us_per_call": round(per[0] * 1e3, 3)}))
        return

    # -- headline: K steps of the M=m MLP, one graph, one replay -------------
    runner = Runner(capi, x, sets, "mlp")
    for s in range(args.warmup):
        runner.step(s)
    torch.cuda.synchronize()
    g = runner.graph(args.steps)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    g.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_total = ev0.elapsed_time(ev1)
    ms_step = ms_total / args.steps
    del g
    b1 = alg_bytes(m, shape.hidden, shape.inter)
    value = b1 / (ms_step * 1e-3) / 1e9
    log(f"M={m}: {ms_step * 1e3:.2f} us/step, {value:.1f} GB/s")
    # distribution over further replays (10 replays of a K/10-step graph)
    dist = runner.time_graph(max(1, args.steps // 10), reps=10)
    py_us = eager_call_us(runner)

    # -- dominant kernel: the gate_up stage alone ------------------------------
    gu = Runner(capi, x, sets, "gate_up")
    gu_ms = statistics.median(gu.time_graph(args.steps, reps=3))
    h, i = shape.hidden, shape.inter
    gu_bytes = 2 * i * h // 2 + 2 * i * h // 32 + 2 * m * h + 2 * m * i
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    dn = Runner(capi, x, sets, "down")
    dn_ms = statistics.median(dn.time_graph(args.steps, reps=3))
    workload = f"{shape.name}-m{m}"
    roofline = {"bound": "hbm", "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": committed_traffic("gate_up", workload),
                "kernel": ("gate_up stage: rowstream_kernel (1 KB single-row loads, MFMA diagonal dot "
                           "products, SiLU*up epilogue)" if m == 1 else
                           "gate_up stage: stream_kernel (row-group dequant GEMV on MFMA, SiLU*up epilogue)"
                           if m <= 8 else "gate_up stage: skinny dequant MFMA kernel"),
                "us_per_launch": round(gu_ms * 1e3, 3), "alg_bytes_per_launch": gu_bytes,
                "down_us_per_launch": round(dn_ms * 1e3, 3)}

    # -- the decoder layer's MLP half: RMSNorm + MLP + residual ----------------
    # fused (norm in gate_up's prologue, residual in down's epilogue) against
    # the norm as a kernel of its own in front of the MLP-with-residual
    nm_ms = statistics.median(Runner(capi, x, sets, "norm_mlp").time_graph(args.steps, reps=3))
    sep_ms = statistics.median(Runner(capi, x, sets, "norm_then_mlp").time_graph(args.steps, reps=3))
    decoder_half = {"what": "x + MLP(RMSNorm(x)) per call, M=%d" % m,
                    "fused_us": round(nm_ms * 1e3, 3), "norm_kernel_then_mlp_us": round(sep_ms * 1e3, 3)}
    log(f"decoder half: fused {nm_ms * 1e3:.2f} us, norm kernel + MLP {sep_ms * 1e3:.2f} us")

    # -- prefill headline -------------------------------------------------------
    prefill = None
    if args.prefill_m:
        pt = measure_point(capi, shape, args.prefill_m, sets, args.prefill_steps)
        prefill = {"m": args.prefill_m, "tflops": pt["tflops"], "frac": pt["mfma_frac"],
                   "us_per_call": pt["us_per_call"], "gbs": pt["gbs"], "tok_s": pt["tok_s"]}
        log(f"M={args.prefill_m}: {pt['us_per_call']:.1f} us/call, {pt['tflops']:.1f} TFLOP/s")

    points = []
    if args.all:
        for name, ms_ in (("qwen3-1.7b", (1, 4, 8)), ("qwen3-8b", (16, 64, 256, 512))):
            shp = SHAPES[name]
            st = sets if name == shape.name else weight_sets(shp)
            for mm in ms_:
                points.append(measure_point(capi, shp, mm, st, 200 if mm <= 8 else 50))
                log(json.dumps(points[-1]))
            del st
        torch.cuda.empty_cache()
        for mm in (1, 512):
            points.append(measure_stack(capi, mm))
            log(json.dumps(points[-1]))

    cpu = None
    if not args.no_cpu:
        log(f"timing the CPU baseline (~{args.cpu_seconds:.0f}s)")
        cpu = cpu_baseline(shape, m, args.cpu_seconds)

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 6),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded N(0,0.02) weights quantized to MXFP4 on device, N(0,1) bf16 activations",
        "config": {"workload": f"{shape.name} MXFP4 MLP (hidden {shape.hidden}, intermediate {shape.inter}) "
                               f"decode M={m}, {len(sets)} rotated weight sets",
                   "hidden": shape.hidden, "intermediate": shape.inter, "m": m},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "us_per_step_p10_p50_p90": [round(1e3 * q, 3) for q in _quantiles(dist)],
        "wall_ms_timed_region": round(wall_ms, 3),
        "python_call_us": round(py_us, 2),
        "roofline": roofline,
        "decoder_half": decoder_half,
        "prefill": prefill,
        "cpu_baseline": cpu,
        "points": points or None,
        "device": dev_name,
    }
    print(json.dumps(line), flush=True)


def _quantiles(v):
    s = sorted(v)
    pick = lambda q: s[min(len(s) - 1, int(round(q * (len(s) - 1))))]
    return pick(0.1), pick(0.5), pick(0.9)


if __name__ == "__main__":
    main()
