"""CPU checks of bench.py's contract (no GPU needed).

* ``--gpus N`` with N > 1 exits with status 2 and says that only one GPU is
  measured; with no GPU visible the script exits with status 1 and a message
  rather than a traceback.
* The algorithmic work per call is the one BASELINE's configurations are
  quoted on: bytes = 3·H·I/2 + 3·H·I/32 + 4·M·H and flops = 6·M·H·I, checked
  against the figures of the configuration table it was derived from (8B
  M=1: 80,232,448 B; M=2048: 113,770,496 B and 6.185e11 flop; 1.7B M=1:
  20,062,208 B; the 32B 64-layer stack at M=1: 13,370,654,720 B).
* Every reported figure comes from at least 200 timed calls and 10 replays,
  and p10 <= p50 <= p90.
* The rocminfo clock parser takes the GPU agent's line, not the CPU's.
"""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from tinyinfer_amd.workloads import SHAPES, alg_bytes, alg_flops  # noqa: E402


def _run(args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True,
                          text=True, timeout=300, env=e, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run(["--gpus", "2"])
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_no_gpu_exits_cleanly():
    # hides any GPU from HIP so the check holds on a GPU box too
    r = _run(["--quick", "--no-cpu"], env={"HIP_VISIBLE_DEVICES": "", "ROCR_VISIBLE_DEVICES": ""})
    assert r.returncode == 1, r.stderr[-2000:]
    assert "needs a gfx950 GPU" in r.stderr
    assert "Traceback" not in r.stderr


@pytest.mark.parametrize("config,m,nbytes", [("qwen3-8b", 1, 80_232_448), ("qwen3-8b", 256, 84_410_368),
                                             ("qwen3-8b", 512, 88_604_672), ("qwen3-8b", 2048, 113_770_496),
                                             ("qwen3-1.7b", 1, 20_062_208), ("qwen3-1.7b", 4, 20_086_784),
                                             ("qwen3-1.7b", 8, 20_119_552), ("qwen3-0.6b", 16, 5_079_040)])
def test_algorithmic_bytes_match_the_configuration_table(config, m, nbytes):
    s = SHAPES[config]
    assert alg_bytes(m, s.hidden, s.inter) == nbytes


def test_algorithmic_flops_and_the_32b_stack():
    s8 = SHAPES["qwen3-8b"]
    assert alg_flops(2048, s8.hidden, s8.inter) == 6 * 2048 * 4096 * 12288
    assert abs(alg_flops(2048, s8.hidden, s8.inter) - 6.185e11) / 6.185e11 < 1e-3
    s32 = SHAPES["qwen3-32b"]
    assert s32.layers * alg_bytes(1, s32.hidden, s32.inter) == 13_370_654_720
    assert s32.layers * alg_bytes(512, s32.hidden, s32.inter) == 14_040_432_640


@pytest.mark.parametrize("steps", [1, 2, 20, 100, 1000])
def test_at_least_200_timed_calls(steps):
    reps = bench.replays_for(steps)
    assert reps >= bench.MIN_REPLAYS >= 10
    assert reps * steps >= 200


def test_quantiles_are_ordered_and_from_the_sample():
    v = [5.0, 1.0, 3.0, 2.0, 4.0, 9.0, 7.0, 8.0, 6.0, 10.0]
    p10, p50, p90 = bench.quantiles(v)
    assert p10 <= p50 <= p90 and {p10, p50, p90} <= set(v)
    assert bench.quantiles([4.2]) == (4.2, 4.2, 4.2)


def test_rocminfo_clock_is_the_gpu_agents(monkeypatch):
    sample = """
*******
Agent 1
*******
  Name:                    AMD EPYC 9575F 64-Core Processor
  Max Clock Freq. (MHz):   3300
*******
Agent 2
*******
  Name:                    gfx950
  Max Clock Freq. (MHz):   2400
"""

    class Done:
        stdout = sample

    monkeypatch.setattr(subprocess, "run", lambda *a, **k: Done())
    assert bench.gpu_max_clock_mhz() == 2400

    def missing(*a, **k):
        raise FileNotFoundError("rocminfo")

    monkeypatch.setattr(subprocess, "run", missing)
    assert bench.gpu_max_clock_mhz() is None
