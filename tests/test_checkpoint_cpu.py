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
    with pytest.raises(ValueError, match="separate directories"):
        ck.quantize_checkpoint(src, src / "sub")
    (tmp_path / "full").mkdir()
    (tmp_path / "full" / "x").write_text("x")
    with pytest.raises(FileExistsError):
        ck.quantize_checkpoint(src, tmp_path / "full")


def _write(path, tensors, shards=1, cfg=None):
    from tests.ckpt_helpers import write_hf
    write_hf(path, cfg or tiny_config(), tensors, shards=shards)


def test_plan_reports_every_problem_before_writing(tmp_path):
    """The planning pass reads only headers and lists all problems at once:
    a layer without up_proj, a weight whose input features are not a
    multiple of 32, a key in two shards; nothing is written."""
    from safetensors.torch import save_file
    cfg = tiny_config()
    t = hf_tensors(cfg)
    del t["model.layers.1.mlp.up_proj.weight"]
    t["model.layers.0.mlp.down_proj.weight"] = torch.zeros(64, 80, dtype=torch.bfloat16)
    _write(tmp_path / "src", t, shards=2, cfg=cfg)
    dup = {"model.norm.weight": torch.ones(64, dtype=torch.bfloat16)}
    save_file(dup, str(tmp_path / "src" / "model-00003-of-00003.safetensors"))
    idx = json.loads((tmp_path / "src" / "model.safetensors.index.json").read_text())
    idx["weight_map"]["model.norm.weight.extra"] = "model-00003-of-00003.safetensors"
    (tmp_path / "src" / "model.safetensors.index.json").write_text(json.dumps(idx))
    with pytest.raises(ValueError) as e:
        ck.quantize_checkpoint(tmp_path / "src", tmp_path / "dst")
    msg = str(e.value)
    assert "layer 1 lacks mlp.up_proj" in msg
    assert "model.layers.0.mlp.down_proj.weight: shape [64, 80]" in msg
    assert "model.norm.weight appears in" in msg
    assert not (tmp_path / "dst").exists()


def test_plan_module_groups(tmp_path):
    """Opt-in groups: the attention projections of every layer, and lm_head
    (its own weight, or the tied embedding); a group the checkpoint cannot
    fill is refused."""
    cfg = tiny_config(tied=True)
    _write(tmp_path / "a", hf_tensors(cfg, full_attn=True), cfg=cfg)
    plan = ck.plan_conversion(tmp_path / "a", ("mlp", "attn", "lm_head"))
    bases = sorted(t.base for t in plan.all_targets())
    assert len(bases) == 2 * 7 + 1 and "lm_head" in bases
    assert "model.layers.1.self_attn.k_proj" in bases
    assert [t.key for t in plan.all_targets() if t.base == "lm_head"] == ["model.embed_tokens.weight"]
    cfg2 = tiny_config()
    _write(tmp_path / "b", hf_tensors(cfg2, full_attn=True), cfg=cfg2)
    with pytest.raises(ValueError, match="no lm_head.weight"):
        ck.plan_conversion(tmp_path / "b", ("mlp", "lm_head"))
    _write(tmp_path / "c", hf_tensors(cfg2), cfg=cfg2)            # q_proj only
    with pytest.raises(ValueError, match="lacks self_attn.k_proj, self_attn.o_proj, self_attn.v_proj"):
        ck.plan_conversion(tmp_path / "c", ("mlp", "attn"))
    with pytest.raises(ValueError, match="module groups"):
        ck.plan_conversion(tmp_path / "c", ("mlp", "embed"))


def test_load_attention_and_lm_head(tmp_path):
    """q/k/v go into row ranges of the merged qkv_proj, o_proj and lm_head
    one to one; a missing k_proj leaves qkv_proj incomplete."""
    cfg = tiny_config()
    q = oracle_mxfp4_tensors(hf_tensors(cfg, full_attn=True, lm_head=True), ("mlp", "attn", "lm_head"))
    _save(tmp_path / "a", q)
    mod = ck.Qwen3MXFP4Linears(module_config(cfg), ("mlp", "attn", "lm_head"))
    rep = ck.load_mxfp4_weights(mod, tmp_path / "a")
    assert not rep.missing and not rep.unexpected and "model.embed_tokens.weight" in rep.skipped
    for layer in range(2):
        a = mod.attn(layer)
        p = f"model.layers.{layer}.self_attn."
        for kind in ("packed", "scale"):
            want = torch.cat([q[p + f"{s}_proj.weight_{kind}"] for s in "qkv"])
            assert torch.equal(getattr(a.qkv_proj, f"weight_{kind}").data, want)
            assert torch.equal(getattr(a.o_proj, f"weight_{kind}").data, q[p + f"o_proj.weight_{kind}"])
    assert torch.equal(mod.lm_head.weight_packed.data, q["lm_head.weight_packed"])
    miss = dict(q)
    del miss["model.layers.0.self_attn.k_proj.weight_scale"]
    _save(tmp_path / "b", miss)
    rep = ck.load_mxfp4_weights(ck.Qwen3MXFP4Linears(module_config(cfg), ("mlp", "attn", "lm_head")),
                                tmp_path / "b", strict=False)
    assert rep.missing == ["model.layers.0.self_attn.qkv_proj.weight_scale"]
    # a dense q_proj given to a model that holds attention in MXFP4 is unexpected
    dense = dict(q)
    dense["model.layers.0.self_attn.q_proj.weight"] = torch.zeros(64, 64, dtype=torch.bfloat16)
    _save(tmp_path / "c", dense)
    with pytest.raises(RuntimeError, match="unexpected"):
        ck.load_mxfp4_weights(ck.Qwen3MXFP4Linears(module_config(cfg), ("mlp", "attn", "lm_head")), tmp_path / "c")
