"""The CPU oracle reproduces the committed golden fixtures (tests/golden/)."""

import hashlib
import json
import os

import numpy as np
import torch

from oracle import mlp as om
from tests.golden.make_golden import bf16_bits, config0_case, sha

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_mlp_small_fixture_reproduces():
    z = np.load(os.path.join(GOLDEN, "mlp_small.npz"))
    x = torch.from_numpy(z["x_bf16"].view(np.int16)).view(torch.bfloat16)
    mats = [z[k] for k in ("gp", "gs", "up", "us", "dp", "ds")]
    assert np.array_equal(bf16_bits(om.mlp_reference(x, *mats)), z["out_reference_bf16"])
    assert np.array_equal(bf16_bits(om.mlp_kernel_semantics(x, *mats)), z["out_kernel_semantics_bf16"])


def test_config0_digests_reproduce():
    rec = json.load(open(os.path.join(GOLDEN, "configs.json")))
    x, mats = config0_case()
    for k, a in zip(("gp", "gs", "up", "us", "dp", "ds"), mats):
        assert sha(a) == rec["sha256"][k], k
    assert sha(bf16_bits(x)) == rec["x_sha256"]
    ref = om.mlp_reference(x, *mats)
    assert sha(bf16_bits(ref)) == rec["out_reference_sha256"]
    assert np.array_equal(np.load(os.path.join(GOLDEN, "config0_out_reference_bf16.npy")), bf16_bits(ref))
