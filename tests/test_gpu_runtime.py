"""GPU: the library's shared host state under use.

* First calls from two host threads at once (a fresh process, so the device
  properties, options and workspaces are initialised by whichever thread
  gets there first), each on its own stream, each result checked against
  the oracle.
* The split-K workspace: its limit sends calls to kernels that need less (or
  none) with the same results, and release_workspaces frees it.
* The fused decode kernel's wait: a wait bound of zero polls (forced from the
  host; every kernel still ends) makes the wait give up, which poisons the
  path: later TI_PATH_DECODE calls leave their outputs alone until
  decode_reset, after which the path gives the oracle's result again.
"""

import os
import subprocess
import sys

import pytest
import torch

from oracle import mlp as om
from tests.helpers import assert_parity, banner, make_case, to_dev
from tests.test_gpu_stream import check_close

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
AUTO, SKINNY, GEMM, DECODE = 0, 1, 2, 3

TWO_THREADS = r'''
import sys, threading
sys.path.insert(0, {root!r})
import torch
from oracle import mlp as om
from tests.helpers import make_case, to_dev
from tinyinfer_amd import capi
cases = [(1, 4096, 12288, 0), (16, 4096, 12288, 0), (4, 2048, 6144, 0), (200, 1024, 3072, 0), (40, 2048, 6144, 2)]
prepared = []
for m, h, i, path in cases:
    x, mats = make_case(m, h, i, seed=m + h)
    prepared.append((x, mats) + tuple(to_dev(x, mats)) + (path,))
torch.cuda.synchronize()
results = {{}}
barrier = threading.Barrier(2)
def run(idx):
    s = torch.cuda.Stream()
    barrier.wait()
    with torch.cuda.stream(s):
        for k in range(idx, len(prepared), 2):
            x, mats, xd, md, path = prepared[k]
            results[k] = capi.mlp_forward(xd, *md, path=path)
    s.synchronize()
ts = [threading.Thread(target=run, args=(j,)) for j in range(2)]
for t in ts: t.start()
for t in ts: t.join()
for k, (x, mats, xd, md, path) in enumerate(prepared):
    st = om.parity_stats(results[k].cpu(), om.mlp_kernel_semantics(x, *mats))
    assert st["rel_max_err"] < 5e-3 and st["cos"] > 0.99999, (k, st)
    print("case", k, "ok", flush=True)
print("two threads ok", flush=True)
'''


def test_first_calls_from_two_threads():
    banner("first calls from two threads (subprocess)")
    out = subprocess.run([sys.executable, "-c", TWO_THREADS.format(root=ROOT)], cwd=ROOT, capture_output=True,
                         text=True, timeout=240)
    print(out.stdout[-2000:], out.stderr[-2000:], flush=True)
    assert out.returncode == 0 and "two threads ok" in out.stdout


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    return c


def test_workspace_limit_and_release(capi):
    """16 tokens at 8B take the split-K tile kernels (workspace); with a zero
    limit they fall back to kernels without one, within the same bar; 160
    tokens on the ring GEMM split K only while the workspace allows it."""
    banner("workspace limit and release")
    for m in (16, 160):
        x, mats = make_case(m, 4096, 12288, seed=70 + m)
        xd, md = to_dev(x, mats)
        ref = om.mlp_kernel_semantics(x, *mats)
        a = capi.mlp_forward(xd, *md)
        torch.cuda.synchronize()
        held, limit = capi.workspace_info()
        assert 0 < held and limit == 512 << 20
        with capi.option("TINYINFER_WORKSPACE_MB", 0):
            assert capi.workspace_info()[1] == 0
            b = capi.mlp_forward(xd, *md)
        capi.release_workspaces()
        assert capi.workspace_info()[0] == 0
        c = capi.mlp_forward(xd, *md)
        torch.cuda.synchronize()
        assert capi.workspace_info()[0] > 0
        check_close(a.cpu(), ref, f"m={m} with workspace")
        check_close(b.cpu(), ref, f"m={m} without workspace")
        assert torch.equal(a.view(torch.int16), c.view(torch.int16))


def test_decode_wait_bound_poisons_until_reset(capi):
    banner("fused decode: forced wait timeout, poison, reset")
    x, mats = make_case(1, 1024, 3072, seed=12)
    xd, md = to_dev(x, mats)
    ref = om.mlp_reference(x, *mats)
    capi.decode_reset()
    assert capi.decode_barrier_timeouts() == 0
    good = capi.mlp_forward(xd, *md, path=DECODE)
    torch.cuda.synchronize()
    assert_parity(good.cpu(), ref, "decode before")
    with capi.option("TINYINFER_DECODE_SPIN", 0):
        for _ in range(3):                # a zero bound gives up unless every flag is already there
            capi.mlp_forward(xd, *md, path=DECODE)
            torch.cuda.synchronize()
            if capi.decode_barrier_timeouts() > 0:
                break
    n = capi.decode_barrier_timeouts()
    if n == 0:
        pytest.skip("every workgroup arrived before the first poll three times; timeout not exercised")
    out = torch.full_like(good, 7.0)
    tmp = torch.full((1, 3072), 7.0, dtype=torch.bfloat16, device="cuda")
    capi.mlp_forward(xd, *md, out=out, tmp=tmp, path=DECODE)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()) and bool((tmp == 7.0).all()), "poisoned path wrote its outputs"
    assert capi.decode_barrier_timeouts() == n
    capi.decode_reset()
    assert capi.decode_barrier_timeouts() == 0
    again = capi.mlp_forward(xd, *md, path=DECODE)
    torch.cuda.synchronize()
    assert torch.equal(again.view(torch.int16), good.view(torch.int16))
