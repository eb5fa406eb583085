"""GPU: the MXFP4 checkpoint writer (device quantizer) produces the
reference's files byte for byte (codes and scales equal to the oracle's
quantization, everything else copied), and a checkpoint it wrote loads into
the MLP modules and runs through the C ABI within the parity bar."""

import json

import pytest
import torch

from oracle import mlp as om
from tests.ckpt_helpers import hf_tensors, module_config, oracle_mxfp4_tensors, tiny_config, write_hf
from tests.helpers import assert_parity, banner
from tinyinfer_amd import checkpoint as ck

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shards,dtype,chunk", [(2, torch.bfloat16, 40), (1, torch.float32, 128)])
def test_writer_matches_oracle_bytes(tmp_path, shards, dtype, chunk):
    from safetensors import safe_open
    banner(f"checkpoint writer shards={shards} {dtype}")
    cfg = tiny_config()
    src_t = hf_tensors(cfg, seed=3, dtype=dtype)
    write_hf(tmp_path / "src", cfg, src_t, shards=shards)
    report = ck.quantize_checkpoint(tmp_path / "src", tmp_path / "dst", chunk_rows=chunk, log=lambda *_: None)
    dst = tmp_path / "dst"
    want = oracle_mxfp4_tensors(src_t)
    got = {}
    for f in sorted(dst.glob("*.safetensors")):
        with safe_open(str(f), framework="pt", device="cpu") as r:
            got.update({k: r.get_tensor(k) for k in r.keys()})
    assert set(got) == set(want)
    for k in want:
        assert got[k].dtype == want[k].dtype and torch.equal(got[k], want[k]), k
    src_files = sorted(p.name for p in (tmp_path / "src").glob("*.safetensors"))
    assert sorted(p.name for p in dst.glob("*.safetensors")) == src_files
    if shards > 1:
        idx = json.loads((dst / "model.safetensors.index.json").read_text())
        assert set(idx["weight_map"]) == set(want) and idx["metadata"]["total_size"] > 0
    else:
        assert not (dst / "model.safetensors.index.json").exists()
    mlp_keys = [k for k in src_t if ck.MLP_PATTERN.fullmatch(k)]
    orig = sum(src_t[k].numel() * src_t[k].element_size() for k in mlp_keys)
    quant = sum(want[k].numel() for k in want if ck.MLP_QUANT_PATTERN.fullmatch(k))
    qc = json.loads((dst / "quantization_config.json").read_text())
    assert qc == ck.quantization_config("qwen3", 2, orig, quant)
    rep = json.loads((dst / "mxfp4_report.json").read_text())
    assert rep == json.loads(json.dumps(report))
    assert rep["num_quantized_matrices"] == 6 and len(rep["tensor_errors"]) == 6
    assert all(0 < e["rmse"] < 0.01 for e in rep["tensor_errors"])
    assert (dst / "config.json").exists() and (dst / "tokenizer_config.json").exists()
    assert not (dst / "README.md").exists()
    assert ck.resolve_quantization(dst) == "mxfp4"


def test_written_checkpoint_runs(tmp_path):
    banner("checkpoint load + forward")
    cfg = tiny_config(layers=2, hidden=512, inter=1024)
    src_t = hf_tensors(cfg, seed=5)
    write_hf(tmp_path / "src", cfg, src_t)
    ck.quantize_checkpoint(tmp_path / "src", tmp_path / "dst", log=lambda *_: None)
    stack = ck.Qwen3MLPStack(module_config(cfg)).to("cuda")
    rep = ck.load_mlp_weights(stack, tmp_path / "dst")
    assert len(rep.loaded) == 12 and not rep.missing
    want = oracle_mxfp4_tensors(src_t)
    x = torch.randn(3, 512, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    for layer in range(2):
        out = stack.mlp(layer)(x.cuda())
        p = f"model.layers.{layer}.mlp."
        mats = [want[p + f"{proj}.weight_{kind}"] for proj in ("gate_proj", "up_proj", "down_proj")
                for kind in ("packed", "scale")]
        assert_parity(out.cpu(), om.mlp_reference(x, *mats), f"layer {layer}")


@pytest.mark.parametrize("tied", [False, True])
def test_writer_attention_and_lm_head(tmp_path, tied):
    """Opt-in groups: attention projections and lm_head (its own weight, or
    the tied embedding) converted to the oracle's bytes, the record lists
    them, and the converted linears loaded into the reference's module
    layout (q/k/v merged) compute within the parity bar."""
    from safetensors import safe_open
    import torch.nn.functional as F
    from tests.ckpt_helpers import module_config
    banner(f"checkpoint attention + lm_head tied={tied}")
    cfg = tiny_config(hidden=512, inter=1024, heads=8, kv_heads=2, vocab=2048, tied=tied)
    src_t = hf_tensors(cfg, seed=9, full_attn=True, lm_head=not tied)
    write_hf(tmp_path / "src", cfg, src_t, shards=2)
    groups = ("mlp", "attn", "lm_head")
    rep = ck.quantize_checkpoint(tmp_path / "src", tmp_path / "dst", groups=groups, chunk_rows=100,
                                 log=lambda *_: None)
    want = oracle_mxfp4_tensors(src_t, groups, tied=tied)
    got = {}
    for f in sorted((tmp_path / "dst").glob("*.safetensors")):
        with safe_open(str(f), framework="pt", device="cpu") as r:
            got.update({k: r.get_tensor(k) for k in r.keys()})
    assert set(got) == set(want)
    for k in want:
        assert got[k].dtype == want[k].dtype and torch.equal(got[k], want[k]), k
    assert rep["num_quantized_matrices"] == 2 * 7 + 1
    qc = json.loads((tmp_path / "dst" / "quantization_config.json").read_text())
    assert qc["target_modules"][-5:] == ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                         "self_attn.o_proj", "lm_head"]
    mod = ck.Qwen3MXFP4Linears(module_config(cfg), groups).to("cuda")
    ck.load_mxfp4_weights(mod, tmp_path / "dst")
    x = torch.randn(5, 512, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)

    def ref(base, inp):
        w = om.dequant_weight(want[base + ".weight_packed"], want[base + ".weight_scale"], torch.bfloat16)
        return F.linear(inp, w)

    for layer in range(2):
        a = mod.attn(layer)
        p = f"model.layers.{layer}.self_attn."
        q, k, v = a.qkv_proj.split_qkv(a.qkv_proj(x.cuda()))
        for name, y in (("q", q), ("k", k), ("v", v)):
            assert_parity(y.cpu(), ref(p + f"{name}_proj", x), f"layer {layer} {name}_proj")
        h = torch.randn(5, 512, generator=torch.Generator().manual_seed(layer)).to(torch.bfloat16)
        assert_parity(a.o_proj(h.cuda()).cpu(), ref(p + "o_proj", h), f"layer {layer} o_proj")
    assert_parity(mod.lm_head(x.cuda()).cpu(), ref("lm_head", x), "lm_head")
