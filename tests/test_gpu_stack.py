"""GPU parity of BASELINE's Qwen3-32B MLP stack workload (hidden 5120,
intermediate 25600, residual add between layers).

* Two layers at 1, 3, 160 and 512 tokens: ``x <- x + MLP_l(x)`` through the C
  ABI (AUTO path; the residual fused into the down epilogue in place, or
  added by torch) against the same composition over a plain PyTorch fp32
  reference of each MLP, with the residual rounded to bf16 after every layer
  as the reference does (tinyinfer/models/qwen3.py:219).
* The full 64-layer pass at 1 and 512 tokens, through ``mlp_stack_step``.
  On N(0, 0.02) weights and N(0, 1) activations the plain stack squares its
  scale every layer (the MLP is quadratic in x) and overflows bf16 at layer 5,
  after which every value is inf or NaN.  So each layer is checked on its own
  input: the pass is replayed layer by layer, every increment that has a
  finite input is compared with the fp32 reference MLP of that layer on the
  same input, and the replay's final bits equal the one-call pass's.
* The 64 decoder-layer MLP halves ``x <- x + MLP_l(RMSNorm_l(x))`` (the model's
  own structure, qwen3.py:210-219, which keeps every MLP input at unit RMS),
  end to end against the fp32 reference composed with the same roundings.
"""

import pytest
import torch

from oracle import mlp as om
from tests.helpers import assert_parity, banner, torch_fp32_reference

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _layers(n):
    from tinyinfer_amd.workloads import SHAPES, quantized_weights
    shp = SHAPES["qwen3-32b"]
    return shp, [quantized_weights(shp.hidden, shp.inter, layer=l) for l in range(n)]


@pytest.mark.parametrize("m,fused", [(1, True), (3, True), (160, True), (512, True), (1, False), (160, False),
                                     (512, False)])
def test_qwen3_32b_two_layer_stack(m, fused):
    from tinyinfer_amd import capi
    from tinyinfer_amd.workloads import activations, mlp_stack_step
    banner(f"32B stack m={m} fused={fused}")
    shp, layers = _layers(2)
    x0 = activations(m, shp.hidden)
    x = x0.clone()
    out = torch.empty_like(x0)
    tmp = torch.empty((m, shp.inter), dtype=x0.dtype, device="cuda")
    mlp_stack_step(capi, x, layers, out, tmp, fused_residual=fused)
    ref = x0.clone()
    for w in layers:
        ref = (ref.float() + torch_fp32_reference(ref, *w).float()).to(torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.isfinite(x.float()).all()
    assert_parity(x, ref, f"32B stack m={m}")
    # the MLP part alone (the residual dominates the sum)
    assert_parity(x.float() - x0.float(), ref.float() - x0.float(), f"32B stack m={m} increments")


@pytest.fixture(scope="module")
def stack64():
    """The 64 seeded layers of the 32B workload (13.4 GB of MXFP4 weights)."""
    shp, layers = _layers(64)
    yield shp, layers
    del layers
    torch.cuda.empty_cache()


@pytest.mark.parametrize("m", [1, 512])
def test_qwen3_32b_full_stack_per_layer(stack64, m):
    from tinyinfer_amd import capi
    from tinyinfer_amd.workloads import activations, mlp_stack_step
    shp, layers = stack64
    banner(f"32B 64-layer stack m={m}")
    x0 = activations(m, shp.hidden)
    tmp = torch.empty((m, shp.inter), dtype=x0.dtype, device="cuda")
    out = torch.empty_like(x0)
    full = x0.clone()
    mlp_stack_step(capi, full, layers, out, tmp)                   # the benchmark's pass, one call
    x = x0.clone()
    checked = 0
    for l, w in enumerate(layers):
        xin = x.clone()
        mlp_stack_step(capi, x, [w], out, tmp)                     # the same calls, one layer at a time
        if not torch.isfinite(xin.float()).all():
            continue
        ref = torch_fp32_reference(xin, *w)
        inc = x.float() - xin.float()
        if not torch.isfinite(ref.float()).all() or not torch.isfinite(x.float()).all():
            continue                                               # the bf16 overflow of the sum itself
        ref_sum = (xin.float() + ref.float()).to(torch.bfloat16)
        assert_parity(x, ref_sum, f"32B layer {l} m={m}")
        assert_parity(inc, ref_sum.float() - xin.float(), f"32B layer {l} m={m} increment")
        checked += 1
    torch.cuda.synchronize()
    assert checked >= 4, checked
    assert torch.equal(full.view(torch.int16), x.view(torch.int16))


def _assert_increment(x, ref, xin, what):
    """The layer's MLP part: |x - ref| within the task's bar of the
    reference increment plus one bf16 rounding of the sum (x and ref are
    both rounded residual sums, so a one-ulp difference of the sum is not an
    error of the MLP)."""
    d = (x.float() - ref.float()).abs()
    inc = (ref.float() - xin.float()).abs().max()
    a = ref.float().abs().clamp_min(2.0 ** -126)
    ulp = torch.exp2(torch.floor(torch.log2(a)) - 7)
    bad = d > 2e-2 * inc + ulp
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} values, worst {float((d - 2e-2 * inc - ulp).max())}"


def _decoder_ref(x, nw, w, h, acc=torch.float32):
    """fp32 reference of one decoder-layer MLP half on x: the RMSNorm
    (fp32 sums, (w*x)*inv, rounded), the MLP (h rounded), the residual sum
    rounded -- the roundings of tinyinfer/models/qwen3.py:210-219.  ``acc``
    is the type the sums run in."""
    r32 = x.to(acc)
    inv = torch.rsqrt((r32 * r32).sum(-1, keepdim=True) / h + EPS)
    xr = ((nw.to(acc) * r32) * inv).to(torch.bfloat16)
    return (r32 + torch_fp32_reference(xr, *w, acc=acc).to(acc)).to(torch.bfloat16)


@pytest.mark.parametrize("m", [1, 512])
def test_qwen3_32b_64_decoder_mlp_halves(stack64, m):
    """Every layer against the fp32 reference on that layer's own input (the
    task's bar), the one-call pass bit-identical to the layer-by-layer
    replay, and the 64-layer result against the reference composed end to
    end.  End to end the bar is relative to how far two references apart
    only in their summation error drift (fp32 and fp64 sums, the same
    roundings): the MLP is quadratic in its input, so a relative difference
    in x grows by about 1 + 2|MLP(x)|/|x| per layer (a factor of several in
    the first layers, where |x| is small), and one rounding that lands on the
    other side of a bf16 boundary early is amplified along the stack, for any
    two implementations that sum in different orders."""
    from tinyinfer_amd import capi
    from tinyinfer_amd.workloads import activations, decoder_stack_step, norm_weight
    shp, layers = stack64
    banner(f"32B 64 decoder MLP halves m={m}")
    nws = [norm_weight(shp.hidden, l) for l in range(len(layers))]
    x0 = activations(m, shp.hidden)
    tmp = torch.empty((m, shp.inter), dtype=x0.dtype, device="cuda")
    xn = torch.empty_like(x0)
    full = x0.clone()
    decoder_stack_step(capi, full, layers, nws, tmp, xn, EPS)     # one call, 64 layers
    x = x0.clone()
    for l, (w, nw) in enumerate(zip(layers, nws)):
        xin = x.clone()
        decoder_stack_step(capi, x, [w], [nw], tmp, xn, EPS)
        ref = _decoder_ref(xin, nw, w, shp.hidden)
        assert_parity(x, ref, f"32B decoder layer {l} m={m}")
        _assert_increment(x, ref, xin, f"32B decoder layer {l} m={m}")
    torch.cuda.synchronize()
    assert torch.equal(full.view(torch.int16), x.view(torch.int16))
    ref, ref64 = x0.clone(), x0.clone()
    for w, nw in zip(layers, nws):
        ref = _decoder_ref(ref, nw, w, shp.hidden)
        ref64 = _decoder_ref(ref64, nw, w, shp.hidden, torch.float64)
    st = om.parity_stats(x, ref)
    drift = om.parity_stats(ref64, ref)
    print(f"64 layers m={m}: kernels vs fp32 reference {st}; fp64 vs fp32 reference {drift}", flush=True)
    assert st["finite"] and drift["finite"]
    assert 1.0 - st["cos"] <= 4.0 * (1.0 - drift["cos"]) + 1e-4, (st, drift)
    assert st["rel_max_err"] <= 4.0 * drift["rel_max_err"] + 2e-2, (st, drift)
