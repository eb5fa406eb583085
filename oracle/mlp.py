"""CPU restatements of the reference MXFP4 MLP (test infrastructure only).

``out = down( silu(x @ gate^T) * (x @ up^T) )`` with all three weights in
MXFP4 (see ``oracle.mxfp4``).

Three forms:

* ``mlp_reference``: the reference's torch CPU dequant-then-matmul path.
  Weights are dequantized to fp32 and cast to the activation dtype, then
  ``F.linear`` (reference ``tinyinfer/layers/linear.py:19-21``),
  ``silu(gate) * up`` (``tinyinfer/layers/activation.py:7-11``) and
  ``F.linear`` again, composed as in ``tinyinfer/models/qwen3.py:155-158``.
  Every intermediate is stored in the activation dtype.  This is the parity
  target named by the task and the timed CPU baseline.
* ``mlp_kernel_semantics``: the rounding points of the reference GPU kernels
  (``tinyinfer/csrc/mlp_fp4.cu:79-142, 365-426``): gate/up sums and the
  SiLU product are exact (fp64 here), ``h`` is rounded once to the
  activation dtype (``mlp_fp4.cu:140``), the down sum is exact and rounded
  once (``mlp_fp4.cu:424``).
* ``mlp_fp64``: everything in float64, no intermediate rounding.

And the MLP's two neighbours in the decoder layer
(``tinyinfer/models/qwen3.py:210-219``):

* ``rmsnorm_reference``: the reference's RMSNorm op, ``rmsnorm_forward``
  (``tinyinfer/layers/layernorm.py:15-23`` -> ``tinyinfer/csrc/rmsnorm.cu:10-54``):
  per row the sum of squares in fp32, ``inv = rsqrt(sum / hidden + eps)``,
  ``out = round(w * x * inv)`` evaluated as ``(w * x) * inv`` in fp32.
* ``decoder_mlp_reference``: ``x + mlp(rmsnorm(x))`` with the sum of the two
  activation-dtype tensors rounded once, as torch adds them
  (``qwen3.py:219``).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from .mxfp4 import dequantize_chunk, dequantize_chunk_torch


def _as_tensor(a) -> torch.Tensor:
    return a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))


def dequant_weight(packed, scale, dtype=torch.bfloat16, impl: str = "numpy") -> torch.Tensor:
    """fp32 dequant then cast to the activation dtype (exact for bf16).
    ``impl="torch"`` decodes with torch CPU ops (the reference's own form,
    multi-threaded; same bits)."""
    if impl == "torch":
        return dequantize_chunk_torch(_as_tensor(packed).cpu(), _as_tensor(scale).cpu()).to(dtype)
    w32 = dequantize_chunk(_as_tensor(packed).cpu().numpy(), _as_tensor(scale).cpu().numpy())
    return torch.from_numpy(w32).to(dtype)


def mlp_reference(x, gp, gs, up, us, dp, ds, weights=None, impl: str = "numpy") -> torch.Tensor:
    """Reference torch CPU path; returns a CPU tensor of ``x``'s dtype.

    ``weights`` may carry pre-dequantized ``(Wg, Wu, Wd)`` in the activation
    dtype to time the matmul-only variant; ``impl`` picks the decode form of
    ``dequant_weight``."""
    xt = _as_tensor(x).cpu()
    dt = xt.dtype
    if weights is None:
        wg = dequant_weight(gp, gs, dt, impl)
        wu = dequant_weight(up, us, dt, impl)
        wd = dequant_weight(dp, ds, dt, impl)
    else:
        wg, wu, wd = weights
    g = F.linear(xt, wg)
    u = F.linear(xt, wu)
    h = F.silu(g) * u
    return F.linear(h, wd)


def rmsnorm_reference(x, w, eps: float) -> torch.Tensor:
    """The reference's rmsnorm kernel (rmsnorm.cu:10-54) on the CPU, fp32
    inside, rounded once to x's dtype."""
    xt = _as_tensor(x).cpu()
    x32 = xt.to(torch.float32)
    w32 = _as_tensor(w).cpu().to(torch.float32)
    ssum = (x32 * x32).sum(dim=-1, keepdim=True)                        # rmsnorm.cu:24-28, fp32
    inv = torch.rsqrt(ssum / float(xt.shape[-1]) + np.float32(eps))     # rmsnorm.cu:45
    return ((w32 * x32) * inv).to(xt.dtype)                             # rmsnorm.cu:51-53


def decoder_mlp_reference(x, w_norm, eps: float, gp, gs, up, us, dp, ds) -> torch.Tensor:
    """``x + Qwen3MLP(post_attention_layernorm(x))`` (qwen3.py:210-219)."""
    xt = _as_tensor(x).cpu()
    y = mlp_reference(rmsnorm_reference(xt, w_norm, eps), gp, gs, up, us, dp, ds)
    return (xt.to(torch.float32) + y.to(torch.float32)).to(xt.dtype)


def _silu64(v: np.ndarray) -> np.ndarray:
    return v / (1.0 + np.exp(-v))


def _round_to(a64: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Round float64 values to ``dtype`` through fp32, the accumulator type
    of the reference kernels (fp32 sum, then one round to the activation
    dtype, mlp_fp4.cu:140)."""
    return torch.from_numpy(a64.astype(np.float32)).to(dtype).to(torch.float64).numpy()


def mlp_kernel_semantics(x, gp, gs, up, us, dp, ds) -> torch.Tensor:
    """Exact sums, ``h`` and ``out`` rounded once to the activation dtype."""
    xt = _as_tensor(x).cpu()
    dt = xt.dtype
    x64 = xt.to(torch.float64).numpy()
    wg = dequantize_chunk(_as_tensor(gp).numpy(), _as_tensor(gs).numpy()).astype(np.float64)
    wu = dequantize_chunk(_as_tensor(up).numpy(), _as_tensor(us).numpy()).astype(np.float64)
    wd = dequantize_chunk(_as_tensor(dp).numpy(), _as_tensor(ds).numpy()).astype(np.float64)
    g = x64 @ wg.T
    u = x64 @ wu.T
    h = _round_to(_silu64(g) * u, dt)
    out = h @ wd.T
    return torch.from_numpy(out.astype(np.float32)).to(dt)


def mlp_fp64(x, gp, gs, up, us, dp, ds) -> np.ndarray:
    """Float64 everywhere (brute-force ground truth for tiny shapes)."""
    x64 = _as_tensor(x).cpu().to(torch.float64).numpy()
    wg = dequantize_chunk(_as_tensor(gp).numpy(), _as_tensor(gs).numpy()).astype(np.float64)
    wu = dequantize_chunk(_as_tensor(up).numpy(), _as_tensor(us).numpy()).astype(np.float64)
    wd = dequantize_chunk(_as_tensor(dp).numpy(), _as_tensor(ds).numpy()).astype(np.float64)
    return (_silu64(x64 @ wg.T) * (x64 @ wu.T)) @ wd.T


def parity_stats(out, ref) -> dict:
    """The task's bar: ``max|out-ref| <= 2e-2 * max|ref|`` and cosine >= 0.9999."""
    o = _as_tensor(out).detach().cpu().to(torch.float64).flatten()
    r = _as_tensor(ref).detach().cpu().to(torch.float64).flatten()
    max_ref = float(r.abs().max()) if r.numel() else 0.0
    max_err = float((o - r).abs().max()) if r.numel() else 0.0
    denom = float(o.norm() * r.norm())
    cos = float((o @ r) / denom) if denom > 0 else (1.0 if float(o.norm()) == float(r.norm()) else 0.0)
    return {"max_err": max_err, "max_ref": max_ref, "rel_max_err": max_err / max_ref if max_ref else max_err,
            "cos": cos, "finite": bool(torch.isfinite(o).all())}


def within_tolerance(stats: dict, rel: float = 2e-2, cos_min: float = 0.9999) -> bool:
    return stats["finite"] and stats["max_err"] <= rel * stats["max_ref"] and stats["cos"] >= cos_min
