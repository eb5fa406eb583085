"""MXFP4 checkpoint loading (the MLP part of the reference's
``tinyinfer/utils/loader.py``) and ``quantization_config.json`` handling,
on the CPU: checkpoints here are written by the test from the oracle's
quantization in the reference's key layout."""

import json

import pytest
import torch

from tests.ckpt_helpers import hf_tensors, module_config, oracle_mxfp4_tensors, tiny_config
from tinyinfer_amd import checkpoint as ck


def _save(path, tensors):
    from safetensors.torch import save_file
    path.mkdir(parents=True, exist_ok=True)
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(path / "model.safetensors"))


def test_load_mlp_weights_one_to_one(tmp_path):
    cfg = tiny_config()
    q = oracle_mxfp4_tensors(hf_tensors(cfg))
    _save(tmp_path, q)
    stack = ck.Qwen3MLPStack(module_config(cfg))
    rep = ck.load_mlp_weights(stack, tmp_path)
    assert len(rep.loaded) == 2 * 3 * 2 and not rep.missing and not rep.unexpected
    assert "model.embed_tokens.weight" in rep.skipped
    for layer in range(2):
        mlp = stack.mlp(layer)
        for proj in ("gate_proj", "up_proj", "down_proj"):
            lin = getattr(mlp, proj)
            base = f"model.layers.{layer}.mlp.{proj}."
            assert torch.equal(lin.weight_packed.data, q[base + "weight_packed"])
            assert torch.equal(lin.weight_scale.data, q[base + "weight_scale"])


def test_load_mlp_weights_strict_errors(tmp_path):
    cfg = tiny_config()
    q = oracle_mxfp4_tensors(hf_tensors(cfg))
    # a missing projection
    miss = dict(q)
    del miss["model.layers.1.mlp.up_proj.weight_scale"]
    _save(tmp_path / "a", miss)
    with pytest.raises(RuntimeError, match="missing"):
        ck.load_mlp_weights(ck.Qwen3MLPStack(module_config(cfg)), tmp_path / "a")
    rep = ck.load_mlp_weights(ck.Qwen3MLPStack(module_config(cfg)), tmp_path / "a", strict=False)
    assert rep.missing == ["model.layers.1.mlp.up_proj.weight_scale"]
    # an unquantized MLP weight (a bf16 checkpoint given to the MXFP4 model)
    _save(tmp_path / "b", hf_tensors(cfg))
    with pytest.raises(RuntimeError, match="unexpected"):
        ck.load_mlp_weights(ck.Qwen3MLPStack(module_config(cfg)), tmp_path / "b")
    # a layer the model does not have
    extra = dict(q)
    extra["model.layers.7.mlp.gate_proj.weight_packed"] = q["model.layers.0.mlp.gate_proj.weight_packed"].clone()
    _save(tmp_path / "c", extra)
    with pytest.raises(RuntimeError, match="unexpected"):
        ck.load_mlp_weights(ck.Qwen3MLPStack(module_config(cfg)), tmp_path / "c")
    # shape mismatch
    bad = dict(q)
    bad["model.layers.0.mlp.down_proj.weight_packed"] = bad["model.layers.0.mlp.down_proj.weight_packed"][:, :-1].contiguous()
    _save(tmp_path / "d", bad)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        ck.load_mlp_weights(ck.Qwen3MLPStack(module_config(cfg)), tmp_path / "d")
    with pytest.raises(FileNotFoundError):
        ck.load_mlp_weights(ck.Qwen3MLPStack(module_config(cfg)), tmp_path / "empty")


def test_resolve_quantization(tmp_path):
    assert ck.resolve_quantization(tmp_path, "none") is None
    assert ck.resolve_quantization(tmp_path, "mxfp4") == "mxfp4"
    assert ck.resolve_quantization(tmp_path, "auto") is None          # no config file
    (tmp_path / "quantization_config.json").write_text(json.dumps(ck.quantization_config("qwen3", 2, 10, 5)))
    assert ck.resolve_quantization(tmp_path, "auto") == "mxfp4"
    (tmp_path / "quantization_config.json").write_text(json.dumps({"quantization": "int8"}))
    with pytest.raises(ValueError, match="Unsupported quantization"):
        ck.resolve_quantization(tmp_path, "auto")


def test_quantization_config_record():
    """The format identifiers the reference's checkpoints carry
    (quantize_mxfp4.py:233-253)."""
    qc = ck.quantization_config("qwen3", 36, 1000, 266)
    assert qc["format"] == "tinyinfer_mxfp4_weight_only_v1" and qc["quantization"] == "mxfp4"
    assert qc["block_size"] == 32 and qc["weight_key_suffixes"] == ["weight_packed", "weight_scale"]
    assert qc["packed_nibble_order"] == "first_element_low_nibble"
    assert qc["scale_encoding"] == "stored_byte = unbiased_exponent + 127"
    assert qc["source_num_hidden_layers"] == 36 and qc["quantized_mlp_weight_bytes"] == 266
    assert list(qc)[0] == "format" and list(qc)[-1] == "note" and len(qc) == 19


def test_writer_refuses_bad_inputs(tmp_path):
    src = tmp_path / "src"
    src.mkdir()
    with pytest.raises(FileNotFoundError, match="config.json"):
        ck.quantize_checkpoint(src, tmp_path / "out")
    (src / "config.json").write_text(json.dumps({"model_type": "llama", "num_hidden_layers": 1}))
    with pytest.raises(ValueError, match="model_type=qwen3"):
        ck.quantize_checkpoint(src, tmp_path / "out")
    with pytest.raises(ValueError, match="non-nested"):
        ck.quantize_checkpoint(src, src / "sub")
    (tmp_path / "full").mkdir()
    (tmp_path / "full" / "x").write_text("x")
    with pytest.raises(FileExistsError):
        ck.quantize_checkpoint(src, tmp_path / "full")
