"""Tiny synthetic Qwen3 checkpoints for the checkpoint tests."""

from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import torch


def tiny_config(layers=2, hidden=64, inter=96, heads=4, kv_heads=2, vocab=32, tied=False):
    return {"model_type": "qwen3", "num_hidden_layers": layers, "hidden_size": hidden,
            "intermediate_size": inter, "vocab_size": vocab, "num_attention_heads": heads,
            "num_key_value_heads": kv_heads, "head_dim": hidden // heads, "tie_word_embeddings": tied}


def module_config(cfg):
    return SimpleNamespace(**{k: cfg[k] for k in ("hidden_size", "intermediate_size", "num_hidden_layers",
                                                   "vocab_size", "num_attention_heads", "num_key_value_heads",
                                                   "head_dim")})


def hf_tensors(cfg, seed=0, dtype=torch.bfloat16, full_attn=False, lm_head=False):
    """A Qwen3-like state dict: MLP weights plus non-MLP tensors (a q_proj
    only, or with ``full_attn`` all four attention projections; an untied
    ``lm_head`` with ``lm_head``)."""
    g = torch.Generator().manual_seed(seed)
    h, i = cfg["hidden_size"], cfg["intermediate_size"]
    q = cfg["num_attention_heads"] * cfg["head_dim"]
    kv = cfg["num_key_value_heads"] * cfg["head_dim"]
    t = {"model.embed_tokens.weight": torch.randn(cfg["vocab_size"], h, generator=g).to(dtype),
         "model.norm.weight": torch.ones(h, dtype=dtype)}
    if lm_head:
        t["lm_head.weight"] = (torch.randn(cfg["vocab_size"], h, generator=g) * 0.02).to(dtype)
    for layer in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{layer}."
        t[p + "self_attn.q_proj.weight"] = (torch.randn(q, h, generator=g) * (0.02 if full_attn else 1.0)).to(dtype)
        if full_attn:
            t[p + "self_attn.k_proj.weight"] = (torch.randn(kv, h, generator=g) * 0.02).to(dtype)
            t[p + "self_attn.v_proj.weight"] = (torch.randn(kv, h, generator=g) * 0.02).to(dtype)
            t[p + "self_attn.o_proj.weight"] = (torch.randn(h, q, generator=g) * 0.02).to(dtype)
            t[p + "self_attn.q_norm.weight"] = torch.ones(cfg["head_dim"], dtype=dtype)
        t[p + "post_attention_layernorm.weight"] = torch.ones(h, dtype=dtype)
        t[p + "mlp.gate_proj.weight"] = (torch.randn(i, h, generator=g) * 0.02).to(dtype)
        t[p + "mlp.up_proj.weight"] = (torch.randn(i, h, generator=g) * 0.02).to(dtype)
        t[p + "mlp.down_proj.weight"] = (torch.randn(h, i, generator=g) * 0.02).to(dtype)
    return t


def write_hf(path: Path, cfg, tensors, shards=1):
    """Write a source checkpoint: config.json, an auxiliary text file, and the
    tensors in ``shards`` safetensors files (with an index when > 1)."""
    from safetensors.torch import save_file
    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps(cfg))
    (path / "tokenizer_config.json").write_text("{}")
    (path / "README.md").write_text("not copied (suffix)")
    names = sorted(tensors)
    weight_map = {}
    for s in range(shards):
        part = {n: tensors[n].contiguous() for n in names[s::shards]}
        fname = "model.safetensors" if shards == 1 else f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file(part, str(path / fname), metadata={"format": "pt"})
        weight_map.update({n: fname for n in part})
    if shards > 1:
        (path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))


def oracle_mxfp4_tensors(tensors, groups=("mlp",), tied=False):
    """The MXFP4 checkpoint's tensors, quantized by the CPU oracle: the MLP
    weights (the reference's format), and with ``groups`` also the attention
    projections and ``lm_head`` (from ``model.embed_tokens.weight`` when
    ``tied``)."""
    import re

    from oracle import mxfp4 as ox
    pats = {"mlp": r"mlp\.(gate_proj|up_proj|down_proj)", "attn": r"self_attn\.(q_proj|k_proj|v_proj|o_proj)"}
    pat = re.compile(r"^model\.layers\.(\d+)\.(" + "|".join(pats[g] for g in groups if g in pats) + r")\.weight$")

    def q(base, t):
        p, s = ox.quantize_chunk(t)
        out[base + ".weight_packed"] = torch.from_numpy(np.asarray(p))
        out[base + ".weight_scale"] = torch.from_numpy(np.asarray(s))

    out = {}
    for n, t in tensors.items():
        if pat.fullmatch(n) or (n == "lm_head.weight" and "lm_head" in groups):
            q(n[:-len(".weight")], t)
        else:
            out[n] = t
        if tied and "lm_head" in groups and n == "model.embed_tokens.weight":
            q("lm_head", t)
    return out
