"""MXFP4 checkpoints: writing them from a Hugging Face Qwen3 checkpoint, and
loading their MLP weights into this package's modules.

The on-disk format is the reference's, byte for byte, so checkpoints move
between the two implementations in both directions:

* ``quantize_checkpoint`` follows ``tinyinfer/quantization/quantize_mxfp4.py``
  (``main``, ``:141-266``): every ``model.layers.N.mlp.{gate,up,down}_proj.weight``
  becomes ``...weight_packed`` (uint8 ``[out, in/2]``) and ``...weight_scale``
  (uint8 ``[out, in/32]``), all other tensors are copied, one output shard per
  input shard, ``model.safetensors.index.json`` when there are several,
  ``quantization_config.json`` with the reference's field values
  (``:233-253``), ``mxfp4_report.json`` (``:255-263``), and the small text files
  of the source directory.  The MXFP4 codes come from the device quantizer
  (bit-exact with the reference's ``quantize_chunk``), so this needs a gfx950
  GPU; the reference's CPU script writes the same bytes.
* ``load_mlp_weights`` is the MLP part of ``tinyinfer/utils/loader.py``
  (``load_weights``, ``:40-131``): checkpoint names map 1:1 onto parameter names
  (``model.layers.N.mlp.gate_proj.weight_packed`` ...), shapes are checked, and
  a report lists what was loaded, missing, skipped or unexpected.
* ``resolve_quantization`` reads ``quantization_config.json`` as the
  reference's harnesses do (``tinyinfer/quantization/PPL.py:23-35``).
"""

from __future__ import annotations

import json
import math
import re
import shutil
from dataclasses import dataclass, field
from pathlib import Path

import torch
from torch import nn

from .mlp import Qwen3MLP

MLP_PATTERN = re.compile(r"^model\.layers\.(\d+)\.mlp\.(gate_proj|up_proj|down_proj)\.weight$")
MLP_QUANT_PATTERN = re.compile(r"^model\.layers\.(\d+)\.mlp\.(gate_proj|up_proj|down_proj)\.weight_(packed|scale)$")
MLP_PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
COPY_SUFFIXES = {".json", ".txt", ".model", ".tiktoken", ".jinja", ".vocab", ".py"}

FORMAT = "tinyinfer_mxfp4_weight_only_v1"


def quantization_config(model_type: str, n_layers: int, original_bytes: int, quantized_bytes: int) -> dict:
    """The ``quantization_config.json`` record, field for field as the
    reference writes it (``quantize_mxfp4.py:233-253``)."""
    return {
        "format": FORMAT,
        "quantization": "mxfp4",
        "target_modules": ["mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"],
        "block_size": 32,
        "axis": "input_features_last_dim",
        "value_format": "fp4_e2m1",
        "scale_format": "e8m0",
        "scale_selection": "ceil_log2_amax_over_6",
        "rounding": "nearest_ties_to_even",
        "packed_dtype": "uint8",
        "packed_nibble_order": "first_element_low_nibble",
        "scale_dtype": "uint8_raw_e8m0_exponent",
        "scale_encoding": "stored_byte = unbiased_exponent + 127",
        "weight_key_suffixes": ["weight_packed", "weight_scale"],
        "source_model_type": model_type,
        "source_num_hidden_layers": n_layers,
        "original_mlp_weight_bytes": original_bytes,
        "quantized_mlp_weight_bytes": quantized_bytes,
        "note": "Custom checkpoint; standard transformers.from_pretrained does not support this layout without a custom loader",
    }


def resolve_quantization(model_path, requested: str = "auto"):
    """``"none"`` -> None, ``"mxfp4"`` -> ``"mxfp4"``; otherwise the
    ``quantization`` field of ``quantization_config.json`` (None without the
    file); anything other than None/"mxfp4" there raises ``ValueError``."""
    if requested == "none":
        return None
    if requested == "mxfp4":
        return "mxfp4"
    path = Path(model_path) / "quantization_config.json"
    if not path.is_file():
        return None
    quantization = json.loads(path.read_text(encoding="utf-8")).get("quantization")
    if quantization not in (None, "mxfp4"):
        raise ValueError(f"Unsupported quantization: {quantization}")
    return quantization


# ----------------------------------------------------------------- writing

def _check_config(source: Path) -> tuple[dict, int]:
    path = source / "config.json"
    if not path.exists():
        raise FileNotFoundError(f"missing config.json: {path}")
    config = json.loads(path.read_text(encoding="utf-8"))
    if config.get("model_type") != "qwen3":
        raise ValueError(f"Expected model_type=qwen3, got {config.get('model_type')!r}")
    if config.get("num_experts") or config.get("num_local_experts"):
        raise ValueError("MoE model not supported by this dense-Qwen3 MLP quantizer")
    return config, int(config["num_hidden_layers"])


def _input_shards(source: Path) -> list[Path]:
    index_path = source / "model.safetensors.index.json"
    if index_path.exists():
        names = sorted(set(json.loads(index_path.read_text(encoding="utf-8"))["weight_map"].values()))
        if not names:
            raise ValueError("empty weight_map")
        shards = [source / n for n in names]
        missing = [str(p) for p in shards if not p.is_file()]
        if missing:
            raise FileNotFoundError(f"Missing source shards: {missing}")
        return shards
    if (source / "model.safetensors").is_file():
        return [source / "model.safetensors"]
    shards = sorted(source.glob("model-*-of-*.safetensors"))
    if not shards:
        raise FileNotFoundError("No HF safetensors checkpoint found")
    return shards


def _copy_auxiliary(source: Path, dest: Path) -> None:
    for item in source.iterdir():
        if not item.is_file() or item.name in {"model.safetensors.index.json", "quantization_config.json"}:
            continue
        if item.name.endswith(".safetensors") or item.suffix not in COPY_SUFFIXES:
            continue
        shutil.copy2(item, dest / item.name)


def quantize_checkpoint(source, dest, chunk_rows: int = 128, verify: bool = True, log=print) -> dict:
    """Write the MXFP4 checkpoint of the Qwen3 checkpoint at ``source`` into the
    empty or new directory ``dest``; returns the report written to
    ``mxfp4_report.json``.  Rows are quantized ``chunk_rows`` at a time on the
    current GPU; ``verify`` decodes them again and records the error."""
    from safetensors import safe_open
    from safetensors.torch import save_file

    from .quantization import dequantize_chunk, quantize_chunk

    source = Path(source).expanduser().resolve()
    dest = Path(dest).expanduser().resolve()
    if chunk_rows <= 0:
        raise ValueError("--chunk-rows must be positive")
    if not source.is_dir():
        raise NotADirectoryError(source)
    if source == dest or source in dest.parents or dest in source.parents:
        raise ValueError("Input/output must be separate, non-nested directories")
    if dest.exists() and any(dest.iterdir()):
        raise FileExistsError(f"Output directory must be empty: {dest}")
    config, n_layers = _check_config(source)
    shards = _input_shards(source)
    dest.mkdir(parents=True, exist_ok=True)
    _copy_auxiliary(source, dest)
    out_map: dict[str, str] = {}
    seen: set[str] = set()
    counts: dict[int, set[str]] = {}
    num_quantized = original_bytes = compressed_bytes = 0
    errors = []
    for shard_index, path in enumerate(shards, start=1):
        output: dict[str, torch.Tensor] = {}
        log(f"[{shard_index}/{len(shards)}] {path.name}")
        with safe_open(str(path), framework="pt", device="cpu") as reader:
            for key in reader.keys():
                if key in seen:
                    raise ValueError(f"duplicate tensor key across shards: {key}")
                seen.add(key)
                tensor = reader.get_tensor(key)
                match = MLP_PATTERN.fullmatch(key)
                if match is None:
                    output[key] = tensor.contiguous()
                    continue
                layer, proj = int(match.group(1)), match.group(2)
                if layer < 0 or layer >= n_layers or proj in counts.setdefault(layer, set()):
                    raise ValueError(f"duplicate/invalid MLP weight: {key}")
                if tensor.ndim != 2 or tensor.shape[1] % 32:
                    raise ValueError(f"{key}: require 2D [out,in] and in % 32 == 0; got {tuple(tensor.shape)}")
                if tensor.dtype not in (torch.float32, torch.float16, torch.bfloat16):
                    raise ValueError(f"{key}: unsupported dtype {tensor.dtype}")
                packed_parts, scale_parts = [], []
                sq = ab = 0.0
                mx = 0.0
                total = 0
                for start in range(0, tensor.shape[0], chunk_rows):
                    chunk = tensor[start:start + chunk_rows].to("cuda")
                    packed, scale = quantize_chunk(chunk)
                    packed_parts.append(packed.cpu())
                    scale_parts.append(scale.cpu())
                    if verify:
                        diff = dequantize_chunk(packed, scale).float() - chunk.float()
                        sq += float(diff.double().square().sum())
                        ab += float(diff.double().abs().sum())
                        mx = max(mx, float(diff.abs().max()))
                        total += chunk.numel()
                packed_t = torch.cat(packed_parts, dim=0)
                scale_t = torch.cat(scale_parts, dim=0)
                base = key[:-len(".weight")]
                output[base + ".weight_packed"] = packed_t
                output[base + ".weight_scale"] = scale_t
                counts[layer].add(proj)
                num_quantized += 1
                original_bytes += tensor.numel() * tensor.element_size()
                compressed_bytes += packed_t.numel() + scale_t.numel()
                if verify:
                    err = {"tensor": key, "mae": ab / total, "rmse": math.sqrt(sq / total), "max_abs": mx}
                    errors.append(err)
                    log(f"  {key}: {tuple(tensor.shape)} | MAE={err['mae']:.6g} RMSE={err['rmse']:.6g}")
                else:
                    log(f"  {key}: {tuple(tensor.shape)}")
        save_file(output, str(dest / path.name), metadata={"format": "pt"})
        for k in output:
            if k in out_map:
                raise ValueError(f"duplicate output key: {k}")
            out_map[k] = path.name
        del output
    incomplete = {layer: sorted(set(MLP_PROJECTIONS) - counts.get(layer, set())) for layer in range(n_layers)
                  if counts.get(layer, set()) != set(MLP_PROJECTIONS)}
    if incomplete:
        raise ValueError(f"Incomplete MLP projections; refusing to finalize checkpoint: {incomplete}")
    if len(shards) > 1:
        size = sum((dest / p.name).stat().st_size for p in shards)
        (dest / "model.safetensors.index.json").write_text(
            json.dumps({"metadata": {"total_size": size}, "weight_map": out_map}, indent=2, ensure_ascii=False) + "\n",
            encoding="utf-8")
    qc = quantization_config(config["model_type"], n_layers, original_bytes, compressed_bytes)
    (dest / "quantization_config.json").write_text(json.dumps(qc, indent=2, ensure_ascii=False) + "\n",
                                                   encoding="utf-8")
    report = {
        "num_quantized_matrices": num_quantized,
        "num_layers": n_layers,
        "mlp_original_bytes": original_bytes,
        "mlp_quantized_bytes": compressed_bytes,
        "mlp_compression_ratio": original_bytes / compressed_bytes if compressed_bytes else float("nan"),
        "tensor_errors": errors,
    }
    (dest / "mxfp4_report.json").write_text(json.dumps(report, indent=2, ensure_ascii=False) + "\n",
                                            encoding="utf-8")
    return report


# ----------------------------------------------------------------- loading

class _Layer(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.mlp = Qwen3MLP(config, quantization="mxfp4")


class Qwen3MLPStack(nn.Module):
    """The MLP blocks of a Qwen3 model under the reference's parameter names
    (``model.layers.N.mlp.{gate,up,down}_proj.weight_{packed,scale}``), so an
    MXFP4 checkpoint loads into it 1:1.  ``config`` needs ``hidden_size``,
    ``intermediate_size`` and ``num_hidden_layers``."""

    def __init__(self, config):
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList(_Layer(config) for _ in range(config.num_hidden_layers))

    def mlp(self, layer: int) -> Qwen3MLP:
        return self.model.layers[layer].mlp


@dataclass
class LoadReport:
    loaded: list = field(default_factory=list)
    missing: list = field(default_factory=list)
    unexpected: list = field(default_factory=list)
    skipped: list = field(default_factory=list)


def iter_checkpoint(model_path):
    """(name, tensor) of every tensor of the checkpoint's ``*.safetensors``
    files, in file-name order (CPU tensors)."""
    from safetensors import safe_open
    path = Path(model_path).expanduser().resolve()
    files = sorted(path.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no .safetensors files found under {path}")
    for f in files:
        with safe_open(str(f), framework="pt", device="cpu") as reader:
            for name in reader.keys():
                yield name, reader.get_tensor(name)


def load_mlp_weights(module: nn.Module, model_path, strict: bool = True) -> LoadReport:
    """Copy the checkpoint's MXFP4 MLP tensors into ``module``'s parameters of
    the same names (shapes checked, bytes copied to the parameters' device).
    Tensors outside the MLPs (attention, norms, embeddings) are reported as
    ``skipped``; MLP tensors with no matching parameter as ``unexpected``;
    MLP parameters the checkpoint lacks as ``missing``.  ``strict`` raises on
    missing or unexpected MLP tensors."""
    params = dict(module.named_parameters())
    mlp_params = {n for n, p in params.items() if MLP_QUANT_PATTERN.fullmatch(n)}
    report = LoadReport()
    loaded = set()
    for name, tensor in iter_checkpoint(model_path):
        if not MLP_QUANT_PATTERN.fullmatch(name):
            (report.unexpected if MLP_PATTERN.fullmatch(name) else report.skipped).append(name)
            continue
        if name not in params:
            report.unexpected.append(name)
            continue
        param = params[name]
        if tuple(param.shape) != tuple(tensor.shape):
            raise RuntimeError(f"shape mismatch for {name}: parameter={tuple(param.shape)} "
                               f"checkpoint={tuple(tensor.shape)}")
        if tensor.dtype != torch.uint8:
            raise RuntimeError(f"{name}: expected uint8, got {tensor.dtype}")
        param.data.copy_(tensor.to(device=param.device))
        loaded.add(name)
        report.loaded.append(name)
    report.missing = sorted(mlp_params - loaded)
    if strict and (report.missing or report.unexpected):
        raise RuntimeError(f"MXFP4 checkpoint does not match the model: missing={report.missing[:8]} "
                           f"unexpected={report.unexpected[:8]}")
    return report


def main(argv=None) -> None:
    """Command line of the writer, with the reference script's arguments
    (``quantize_mxfp4.py:86-92``): ``python -m tinyinfer_amd.checkpoint
    --input HF_DIR --output NEW_DIR [--chunk-rows 128] [--no-verify]``."""
    import argparse
    p = argparse.ArgumentParser(description="MXFP4 weight-only quantization of Qwen3 MLP checkpoints (gfx950 GPU)")
    p.add_argument("--input", required=True, type=Path, help="Original HF Qwen3 directory")
    p.add_argument("--output", required=True, type=Path, help="New checkpoint directory (must be empty)")
    p.add_argument("--chunk-rows", type=int, default=128, help="Rows processed at once")
    p.add_argument("--verify", action=argparse.BooleanOptionalAction, default=True,
                   help="Decode and measure quantization error")
    a = p.parse_args(argv)
    rep = quantize_checkpoint(a.input, a.output, chunk_rows=a.chunk_rows, verify=a.verify,
                              log=lambda m: print(m, flush=True))
    o, q = rep["mlp_original_bytes"], rep["mlp_quantized_bytes"]
    print(f"\nDONE: {rep['num_quantized_matrices']} matrices, {o / 2**20:.2f} MiB -> {q / 2**20:.2f} MiB"
          f" ({o / q:.3f}x). Output: {Path(a.output).expanduser().resolve()}", flush=True)


if __name__ == "__main__":
    main()
