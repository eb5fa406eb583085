"""Tiny synthetic Qwen3 checkpoints for the checkpoint tests."""

from __future__ import annotations

import json
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import torch


def tiny_config(layers=2, hidden=64, inter=96):
    return {"model_type": "qwen3", "num_hidden_layers": layers, "hidden_size": hidden,
            "intermediate_size": inter, "vocab_size": 32}


def module_config(cfg):
    return SimpleNamespace(hidden_size=cfg["hidden_size"], intermediate_size=cfg["intermediate_size"],
                           num_hidden_layers=cfg["num_hidden_layers"])


def hf_tensors(cfg, seed=0, dtype=torch.bfloat16):
    """A Qwen3-like state dict: MLP weights plus a few non-MLP tensors."""
    g = torch.Generator().manual_seed(seed)
    h, i = cfg["hidden_size"], cfg["intermediate_size"]
    t = {"model.embed_tokens.weight": torch.randn(cfg["vocab_size"], h, generator=g).to(dtype),
         "model.norm.weight": torch.ones(h, dtype=dtype)}
    for layer in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{layer}."
        t[p + "self_attn.q_proj.weight"] = torch.randn(h, h, generator=g).to(dtype)
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


def oracle_mxfp4_tensors(tensors):
    """The MXFP4 checkpoint's tensors, quantized by the CPU oracle."""
    import re

    from oracle import mxfp4 as ox
    pat = re.compile(r"^model\.layers\.(\d+)\.mlp\.(gate_proj|up_proj|down_proj)\.weight$")
    out = {}
    for n, t in tensors.items():
        if pat.fullmatch(n):
            p, s = ox.quantize_chunk(t)
            out[n[:-len(".weight")] + ".weight_packed"] = torch.from_numpy(np.asarray(p))
            out[n[:-len(".weight")] + ".weight_scale"] = torch.from_numpy(np.asarray(s))
        else:
            out[n] = t
    return out
