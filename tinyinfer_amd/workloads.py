"""Benchmark/test workloads: the MLP shapes of the target configurations,
their algorithmic byte and flop counts, and seeded synthetic inputs.

Shapes: Qwen3 hidden/intermediate sizes.  Work per MLP call:
  bytes = 3*H*I/2 (e2m1 nibbles) + 3*H*I/32 (e8m0 scales) + 2*M*H (x) + 2*M*H (out)
  flops = 6*M*H*I   (three GEMMs; the SiLU*up epilogue is not counted)
The h round trip (4*M*I bytes) is not counted, since a fused kernel need not
make it.

Synthetic inputs: weights N(0, 0.02) with seeds 1000 + 3*layer + {0 gate,
1 up, 2 down}, quantized with the device quantizer; activations N(0, 1) with
seed 7, cast to the activation dtype.  ``generator="cpu"`` draws with
torch's CPU generator (tests, small shapes); ``"cuda"`` draws on the GPU
(benchmark, multi-GB weight sets).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class MlpShape:
    name: str
    hidden: int
    inter: int
    layers: int = 1


SHAPES = {
    "qwen3-0.6b": MlpShape("qwen3-0.6b", 1024, 3072),
    "qwen3-1.7b": MlpShape("qwen3-1.7b", 2048, 6144),
    "qwen3-8b": MlpShape("qwen3-8b", 4096, 12288),
    "qwen3-32b": MlpShape("qwen3-32b", 5120, 25600, 64),
}

WEIGHT_STD = 0.02
X_SEED = 7
NORM_EPS = 1e-6          # Qwen3's rms_norm_eps


def weight_bytes(h: int, i: int) -> int:
    return 3 * h * i // 2 + 3 * h * i // 32


def alg_bytes(m: int, h: int, i: int) -> int:
    return weight_bytes(h, i) + 4 * m * h


def alg_flops(m: int, h: int, i: int) -> int:
    return 6 * m * h * i


def weight_seeds(layer: int):
    base = 1000 + 3 * layer
    return base, base + 1, base + 2


def _randn(shape, seed: int, generator: str, device) -> torch.Tensor:
    g = torch.Generator(device=generator).manual_seed(seed)
    return torch.randn(shape, generator=g, device=generator, dtype=torch.float32)


def random_weights(h: int, i: int, layer: int = 0, generator: str = "cpu"):
    """fp32 N(0, 0.02) gate [i,h], up [i,h], down [h,i] on ``generator``'s device."""
    sg, su, sd = weight_seeds(layer)
    return (_randn((i, h), sg, generator, None) * WEIGHT_STD,
            _randn((i, h), su, generator, None) * WEIGHT_STD,
            _randn((h, i), sd, generator, None) * WEIGHT_STD)


def quantized_weights(h: int, i: int, layer: int = 0, generator: str = "cuda", device="cuda"):
    """(gate_packed, gate_scale, up_packed, up_scale, down_packed, down_scale) on
    ``device``, quantized by the device quantizer."""
    from .quantization import quantize_chunk
    out = []
    for w in random_weights(h, i, layer, generator):
        p, s = quantize_chunk(w.to(device))
        out.extend((p, s))
        del w
    return tuple(out)


def activations(m: int, h: int, dtype=torch.bfloat16, seed: int = X_SEED, generator: str = "cpu", device="cuda"):
    return _randn((m, h), seed, generator, None).to(dtype).to(device)


def mlp_stack_step(capi, x, layers, out, tmp, fused_residual=True):
    """One pass of the Qwen3-32B MLP stack workload: ``x <- x + MLP_l(x)`` for
    every layer, in the activation dtype, rounded as the reference's
    ``hidden_states = residual + hidden_states``.  With ``fused_residual`` the
    add happens in the down stage's epilogue, in place on ``x`` (the MLP has
    read x before down writes it); otherwise it is torch's add of ``out``.
    ``out``/``tmp`` are [M, H] / [M, I] buffers reused by every layer."""
    for w in layers:
        if fused_residual:
            capi.mlp_forward(x, *w, out=x, tmp=tmp, residual=x)
        else:
            capi.mlp_forward(x, *w, out=out, tmp=tmp)
            x.add_(out)
    return x


def norm_weight(h: int, layer: int = 0, dtype=torch.bfloat16, device="cuda") -> torch.Tensor:
    """A post-attention RMSNorm weight for ``layer``: 1 + N(0, 0.1), seed 2000 + layer."""
    return (1.0 + 0.1 * _randn((h,), 2000 + layer, "cpu", None)).to(dtype).to(device)


def decoder_stack_step(capi, x, layers, norm_ws, tmp, xn, eps: float = NORM_EPS):
    """One pass over the decoder layers' MLP halves, in place on ``x``:
    ``x <- x + MLP_l(RMSNorm_l(x))`` for every layer (the reference decoder
    layer's ``post_attention_layernorm -> mlp -> residual add``,
    tinyinfer/models/qwen3.py:210-219), each layer one call of the fused
    entry point.  The norm keeps every MLP's input at unit RMS, so the
    residual stream grows only as a random walk over the 64 layers; the plain
    stack of ``mlp_stack_step`` squares its scale every layer and overflows
    bf16 within a few layers on N(0, 0.02) weights."""
    for w, nw in zip(layers, norm_ws):
        capi.mlp_forward_rmsnorm(x, nw, eps, *w, out=x, tmp=tmp, xn=xn)
    return x
