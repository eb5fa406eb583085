"""Writes the committed golden fixtures under tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

* ``mlp_small.npz``: a seeded MLP (M=5, hidden=256, intermediate=512) with
  weights N(0, 0.02) quantized by the oracle; stores the inputs, the oracle
  reference output (torch CPU bf16 dequant-then-matmul path) and the
  kernel-semantics output (exact sums, h and out rounded to bf16).
* ``configs.json``: SHA-256 digests of the packed/scale bytes that the
  seeded generation gives for the configs[0] shape (Qwen3-0.6B block), and of
  the oracle reference output at M=16, so drift in the codec or the oracle
  shows up as a digest mismatch.

The reference implementation is not imported: every vector here comes from
the oracle, which tests/test_oracle_*.py pin independently.
"""

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import mlp as om  # noqa: E402
from oracle import mxfp4 as ox  # noqa: E402


def seeded_case(m, h, i, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, h, generator=g).to(torch.bfloat16)
    mats = []
    for rows, cols in ((i, h), (i, h), (h, i)):
        w = torch.randn(rows, cols, generator=g) * 0.02
        mats.extend(ox.quantize_chunk(w))
    return x, mats


def config0_case():
    """configs[0] with the workload seeds: weights 1000/1001/1002, x seed 7."""
    mats = []
    for seed, (rows, cols) in zip((1000, 1001, 1002), ((3072, 1024), (3072, 1024), (1024, 3072))):
        g = torch.Generator().manual_seed(seed)
        w = torch.randn(rows, cols, generator=g) * 0.02
        mats.extend(ox.quantize_chunk(w))
    g = torch.Generator().manual_seed(7)
    x = torch.randn(16, 1024, generator=g).to(torch.bfloat16)
    return x, mats


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main():
    x, mats = seeded_case(5, 256, 512, seed=2024)
    ref = om.mlp_reference(x, *mats)
    ks = om.mlp_kernel_semantics(x, *mats)
    np.savez_compressed(
        os.path.join(HERE, "mlp_small.npz"),
        x_bf16=bf16_bits(x), gp=mats[0], gs=mats[1], up=mats[2], us=mats[3], dp=mats[4], ds=mats[5],
        out_reference_bf16=bf16_bits(ref), out_kernel_semantics_bf16=bf16_bits(ks))

    x0, m0 = config0_case()
    ref0 = om.mlp_reference(x0, *m0)
    record = {
        "config": "qwen3-0.6b block: x [16,1024] seed 7; gate/up [3072,1024] seeds 1000/1001; down [1024,3072] seed 1002",
        "sha256": {k: sha(a) for k, a in zip(("gp", "gs", "up", "us", "dp", "ds"), m0)},
        "x_sha256": sha(bf16_bits(x0)),
        "out_reference_sha256": sha(bf16_bits(ref0)),
        "out_reference_abs_max": float(ref0.float().abs().max()),
    }
    with open(os.path.join(HERE, "configs.json"), "w") as f:
        json.dump(record, f, indent=2)
        f.write("\n")
    np.save(os.path.join(HERE, "config0_out_reference_bf16.npy"), bf16_bits(ref0))
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
