"""MXFP4 checkpoints on the GPU: converting a Hugging Face Qwen3 checkpoint,
and loading the result into this package's modules.

File format -- shared with the reference (tinyinfer/quantization/
quantize_mxfp4.py:20-25, 203-204, 233-263), so checkpoints move between the
two implementations in both directions:

* a converted weight ``<base>.weight`` ``[out, in]`` is stored as
  ``<base>.weight_packed`` (uint8 ``[out, in/2]``, e2m1 codes, first element
  in the low nibble) and ``<base>.weight_scale`` (uint8 ``[out, in/32]``,
  e8m0 byte per 32 input features); every other tensor is kept as it is;
* the output has the source's shard files (same names, same split of the
  tensors), ``model.safetensors.index.json`` when there is more than one,
  ``quantization_config.json`` (``quantization_config``) and
  ``mxfp4_report.json`` (``build_report``).

The reference converts the MLP weights only (``mlp.{gate,up,down}_proj``);
that is the default here too and gives the reference's files byte for
byte.  Opt-in module groups extend the same format to the attention
projections (``self_attn.{q,k,v,o}_proj``) and to ``lm_head`` (taken from
``model.embed_tokens.weight`` when the checkpoint ties the two), listed in
``target_modules``.

How the converter works (``convert``): a planning pass reads only the
safetensors headers of every shard and checks the whole conversion -- keys
unique across shards, every target 2-D with ``in % 32 == 0`` and a float
dtype, every layer complete -- and reports every problem it finds at once,
before anything is written.  The writing pass then streams: per shard, per
tensor, a target goes to the GPU in row blocks, the device quantizer
(bit-exact with the reference's ``quantize_chunk``) writes its codes and
scales straight into slices of one device buffer, and the error statistics
are accumulated on the device; the host synchronizes once per tensor.

Loading (``load_mxfp4_weights``): checkpoint names map onto the parameters
of the reference model's modules -- ``mlp.*`` and ``o_proj``/``lm_head``
one to one, ``q_proj``/``k_proj``/``v_proj`` into row ranges of the merged
``qkv_proj`` (tinyinfer/layers/linear.py:58-77; MXFP4 rows are independent,
so rows concatenate byte for byte).
"""

from __future__ import annotations

import fnmatch
import json
import re
import shutil
from dataclasses import dataclass, field
from pathlib import Path

import torch
from torch import nn

from .linear import LinearMXFP4
from .mlp import Qwen3MLP

FORMAT_TAG = "tinyinfer_mxfp4_weight_only_v1"
BLOCK = 32

# module groups that can be stored in MXFP4 (names relative to a decoder
# layer, or to the model root for lm_head); "mlp" is the reference's format
MODULE_GROUPS = {
    "mlp": ("mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"),
    "attn": ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj"),
    "lm_head": ("lm_head",),
}
DEFAULT_GROUPS = ("mlp",)

# checkpoint names of the MLP weights, dense and converted
MLP_PATTERN = re.compile(r"^model\.layers\.(\d+)\.mlp\.(gate_proj|up_proj|down_proj)\.weight$")
MLP_QUANT_PATTERN = re.compile(r"^model\.layers\.(\d+)\.mlp\.(gate_proj|up_proj|down_proj)\.weight_(packed|scale)$")
_LAYER_WEIGHT = re.compile(r"^model\.layers\.(\d+)\.(.+)\.weight$")
_QUANT_NAME = re.compile(r"^(.+)\.weight_(packed|scale)$")

# files of the source directory that a loader or tokenizer reads
_AUX_FILES = ("config.json", "generation_config.json", "tokenizer*", "vocab*", "merges.txt",
              "special_tokens_map.json", "added_tokens.json", "chat_template*", "*.model", "*.tiktoken")
_WRITTEN = ("model.safetensors.index.json", "quantization_config.json", "mxfp4_report.json")


def quantization_config(model_type: str, n_layers: int, original_bytes: int, quantized_bytes: int,
                        groups=DEFAULT_GROUPS) -> dict:
    """The ``quantization_config.json`` record (format fields and values as
    the reference writes them, quantize_mxfp4.py:233-253).  With the default
    groups it is the reference's record; other groups add their modules to
    ``target_modules`` and their bytes to the two byte counts."""
    modules = [m for g in groups for m in MODULE_GROUPS[g]]
    return {
        "format": FORMAT_TAG,
        "quantization": "mxfp4",
        "target_modules": modules,
        "block_size": BLOCK,
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


def build_report(n_matrices: int, n_layers: int, original_bytes: int, quantized_bytes: int, errors: list) -> dict:
    """The ``mxfp4_report.json`` record (the reference's fields,
    quantize_mxfp4.py:255-263)."""
    return {
        "num_quantized_matrices": n_matrices,
        "num_layers": n_layers,
        "mlp_original_bytes": original_bytes,
        "mlp_quantized_bytes": quantized_bytes,
        "mlp_compression_ratio": original_bytes / quantized_bytes if quantized_bytes else float("nan"),
        "tensor_errors": errors,
    }


def resolve_quantization(model_path, requested: str = "auto"):
    """What the reference's harnesses pass as ``quantization``
    (tinyinfer/quantization/PPL.py:23-35): ``"none"`` -> None, ``"mxfp4"`` ->
    ``"mxfp4"``, ``"auto"`` -> the ``quantization`` field of the directory's
    ``quantization_config.json`` (None without one).  Any other recorded
    value raises ``ValueError("Unsupported quantization: ...")``."""
    if requested in ("none", "mxfp4"):
        return None if requested == "none" else "mxfp4"
    record = Path(model_path) / "quantization_config.json"
    if not record.is_file():
        return None
    value = json.loads(record.read_text(encoding="utf-8")).get("quantization")
    if value is not None and value != "mxfp4":
        raise ValueError(f"Unsupported quantization: {value}")
    return value


# ----------------------------------------------------------------- planning

@dataclass
class Target:
    """One weight to convert: ``key`` in shard ``shard`` (or, for a tied
    lm_head, ``model.embed_tokens.weight`` written again under ``base``)."""
    key: str
    base: str                 # output names: base + ".weight_packed" / ".weight_scale"
    group: str
    shape: tuple
    dtype: str


@dataclass
class ConversionPlan:
    source: Path
    config: dict
    n_layers: int
    groups: tuple
    shards: list                                        # source shard paths, output in the same order
    keys: dict = field(default_factory=dict)            # shard path -> its tensor names
    targets: dict = field(default_factory=dict)         # tensor name -> Target
    extra: dict = field(default_factory=dict)           # shard path -> [Target] written beside its tensors

    def all_targets(self):
        yield from self.targets.values()
        for ts in self.extra.values():
            yield from ts


_FLOAT_DTYPES = {"F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16}


def _source_shards(source: Path) -> list:
    """The checkpoint's weight files: those its index names (in order of
    first mention), else model.safetensors, else the model-*-of-* files."""
    index = source / "model.safetensors.index.json"
    if index.is_file():
        files = []
        for name in json.loads(index.read_text(encoding="utf-8")).get("weight_map", {}).values():
            if name not in files:
                files.append(name)
        if not files:
            raise ValueError(f"{index} maps no tensors")
        absent = [f for f in files if not (source / f).is_file()]
        if absent:
            raise FileNotFoundError(f"{index} names shard files that do not exist: {absent}")
        return [source / f for f in files]
    single = source / "model.safetensors"
    if single.is_file():
        return [single]
    files = sorted(source.glob("model-*-of-*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no safetensors weights in {source}")
    return files


def _target_base(key: str, groups) -> tuple | None:
    """(group, output base) when ``key`` is a weight of a selected group."""
    if key == "lm_head.weight":
        return ("lm_head", "lm_head") if "lm_head" in groups else None
    m = _LAYER_WEIGHT.fullmatch(key)
    if not m:
        return None
    for g in groups:
        if m.group(2) in MODULE_GROUPS[g]:
            return g, key[: -len(".weight")]
    return None


def plan_conversion(source, groups=DEFAULT_GROUPS) -> ConversionPlan:
    """Read the config and every shard's header; check the conversion as a
    whole.  Raises with every problem found (not only the first)."""
    from safetensors import safe_open

    source = Path(source).expanduser().resolve()
    if not source.is_dir():
        raise NotADirectoryError(f"source checkpoint is not a directory: {source}")
    unknown = [g for g in groups if g not in MODULE_GROUPS]
    if unknown or not groups:
        raise ValueError(f"module groups must be among {sorted(MODULE_GROUPS)}, got {list(groups)}")
    cfg_path = source / "config.json"
    if not cfg_path.is_file():
        raise FileNotFoundError(f"the source has no config.json: {cfg_path}")
    config = json.loads(cfg_path.read_text(encoding="utf-8"))
    if config.get("model_type") != "qwen3":
        raise ValueError(f"only dense Qwen3 checkpoints convert (model_type=qwen3); this one is "
                         f"{config.get('model_type')!r}")
    if config.get("num_experts") or config.get("num_local_experts"):
        raise ValueError("mixture-of-experts checkpoints are not supported: their MLPs are expert banks")
    n_layers = int(config["num_hidden_layers"])
    plan = ConversionPlan(source, config, n_layers, tuple(groups), _source_shards(source))

    problems = []
    where = {}
    headers = {}
    for shard in plan.shards:
        with safe_open(str(shard), framework="pt", device="cpu") as f:
            names = list(f.keys())
            plan.keys[shard] = names
            for k in names:
                if k in where:
                    problems.append(f"{k} appears in {where[k].name} and {shard.name}")
                    continue
                where[k] = shard
                if _target_base(k, groups) or k == "model.embed_tokens.weight":
                    sl = f.get_slice(k)
                    headers[k] = (tuple(sl.get_shape()), sl.get_dtype())

    seen = {}                                             # layer -> set of converted modules
    for k, shard in where.items():
        tb = _target_base(k, groups)
        if tb is None:
            continue
        group, base = tb
        shape, dtype = headers[k]
        if len(shape) != 2 or shape[1] % BLOCK:
            problems.append(f"{k}: shape {list(shape)} is not [out, in] with in a multiple of {BLOCK}")
        if dtype not in _FLOAT_DTYPES:
            problems.append(f"{k}: dtype {dtype} is not F32, F16 or BF16")
        if group != "lm_head":
            layer = int(_LAYER_WEIGHT.fullmatch(k).group(1))
            if layer >= n_layers:
                problems.append(f"{k}: layer {layer} is beyond num_hidden_layers={n_layers}")
            seen.setdefault(layer, set()).add(_LAYER_WEIGHT.fullmatch(k).group(2))
        plan.targets[k] = Target(k, base, group, shape, dtype)
    layer_modules = [m for g in groups if g != "lm_head" for m in MODULE_GROUPS[g]]
    for layer in range(n_layers):
        lacking = sorted(set(layer_modules) - seen.get(layer, set()))
        if lacking:
            problems.append(f"layer {layer} lacks {', '.join(lacking)}")
    if "lm_head" in groups and "lm_head.weight" not in where:
        emb = "model.embed_tokens.weight"
        if config.get("tie_word_embeddings") and emb in where:
            shape, dtype = headers[emb]
            if len(shape) != 2 or shape[1] % BLOCK or dtype not in _FLOAT_DTYPES:
                problems.append(f"{emb} (tied lm_head): cannot convert shape {list(shape)} dtype {dtype}")
            plan.extra.setdefault(where[emb], []).append(Target(emb, "lm_head", "lm_head", shape, dtype))
        else:
            problems.append("lm_head was requested but the checkpoint has no lm_head.weight "
                            "(and does not tie it to model.embed_tokens.weight)")
    if problems:
        raise ValueError("cannot convert this checkpoint:\n  " + "\n  ".join(problems))
    return plan


# ----------------------------------------------------------------- writing

class _DeviceQuantizer:
    """Row blocks of one weight through the device quantizer into one
    device buffer; error sums stay on the device until ``finish``."""

    def __init__(self, rows: int, cols: int, verify: bool):
        from . import capi
        self.capi = capi
        self.packed = torch.empty((rows, cols // 2), dtype=torch.uint8, device="cuda")
        self.scale = torch.empty((rows, cols // BLOCK), dtype=torch.uint8, device="cuda")
        self.flags = []
        self.verify = verify
        self.sums = torch.zeros(3, dtype=torch.float64, device="cuda")   # |d|, d^2, max|d|

    def add(self, start: int, block: torch.Tensor) -> None:
        capi = self.capi
        w = block.to("cuda", non_blocking=True).contiguous()
        if w.dtype not in _FLOAT_DTYPES.values():
            w = w.float()
        codes = {torch.float32: capi.TI_DTYPE_F32, torch.bfloat16: capi.TI_DTYPE_BF16,
                 torch.float16: capi.TI_DTYPE_F16}
        rows, cols = w.shape
        p = self.packed[start:start + rows]
        s = self.scale[start:start + rows]
        flag = torch.empty(1, dtype=torch.int32, device="cuda")
        st = capi.lib().tinyinfer_mxfp4_quantize(w.data_ptr(), codes[w.dtype], rows, cols, p.data_ptr(),
                                                 s.data_ptr(), flag.data_ptr(), capi._stream_handle())
        if st != capi.TI_OK:
            raise capi.TinyInferError(st, "tinyinfer_mxfp4_quantize")
        self.flags.append(flag)
        if self.verify:
            d = capi.dequant(p, s, torch.float32) - w.float()
            a = d.abs()
            self.sums[0] += a.sum(dtype=torch.float64)
            self.sums[1] += d.double().square().sum()
            self.sums[2] = torch.maximum(self.sums[2], a.max().double())

    def finish(self, key: str, numel: int):
        """(packed, scale) on the host, and the error record (or None);
        raises where the reference's quantizer raises."""
        bits = 0
        for v in torch.cat(self.flags).tolist():      # the one synchronization of the tensor
            bits |= int(v)
        if bits & self.capi.TI_QFLAG_NONFINITE:
            raise ValueError(f"{key}: non-finite weights (NaN/Inf) cannot be quantized")
        if bits & self.capi.TI_QFLAG_EXP_RANGE:
            raise ValueError(f"{key}: a block's scale exponent falls outside the e8m0 range [-127, 127]")
        err = None
        if self.verify:
            mae, sq, mx = self.sums.tolist()
            err = {"tensor": key, "mae": mae / numel, "rmse": (sq / numel) ** 0.5, "max_abs": mx}
        return self.packed.cpu(), self.scale.cpu(), err


def _quantize_on_device(tensor: torch.Tensor, key: str, chunk_rows: int, verify: bool):
    q = _DeviceQuantizer(tensor.shape[0], tensor.shape[1], verify)
    for start in range(0, tensor.shape[0], chunk_rows):
        q.add(start, tensor[start:start + chunk_rows])
    return q.finish(key, tensor.numel())


def _check_destination(source: Path, dest: Path) -> None:
    if dest == source or source in dest.parents or dest in source.parents:
        raise ValueError(f"source and destination must be separate directories, neither inside the "
                         f"other: {source} / {dest}")
    if dest.exists() and (not dest.is_dir() or any(dest.iterdir())):
        raise FileExistsError(f"destination is not an empty directory: {dest}")


def _copy_side_files(source: Path, dest: Path) -> list:
    copied = []
    for f in sorted(source.iterdir()):
        if f.is_file() and f.name not in _WRITTEN and any(fnmatch.fnmatch(f.name, p) for p in _AUX_FILES):
            shutil.copy2(f, dest / f.name)
            copied.append(f.name)
    return copied


def convert(source, dest, groups=DEFAULT_GROUPS, chunk_rows: int = 4096, verify: bool = True, log=print) -> dict:
    """Convert the Qwen3 checkpoint at ``source`` into an MXFP4 checkpoint in
    the new or empty directory ``dest`` (see the module docstring); returns
    the report also written to ``mxfp4_report.json``."""
    from safetensors import safe_open
    from safetensors.torch import save_file

    if chunk_rows < 1:
        raise ValueError(f"chunk_rows must be at least 1, got {chunk_rows}")
    src = Path(source).expanduser().resolve()
    dest = Path(dest).expanduser().resolve()
    _check_destination(src, dest)
    plan = plan_conversion(src, groups)
    if not torch.cuda.is_available():
        raise RuntimeError("the MXFP4 converter quantizes on a gfx950 GPU; none is visible")
    dest.mkdir(parents=True, exist_ok=True)
    log(f"{plan.source.name}: {len(plan.shards)} shard(s), {sum(1 for _ in plan.all_targets())} weights to "
        f"convert ({', '.join(plan.groups)}); side files: {', '.join(_copy_side_files(plan.source, dest))}")

    weight_map = {}
    n_mats = orig = quant = 0
    errors = []
    for i, shard in enumerate(plan.shards, 1):
        tensors = {}
        with safe_open(str(shard), framework="pt", device="cpu") as f:
            work = [(k, plan.targets.get(k)) for k in plan.keys[shard]] + [(t.key, t) for t in plan.extra.get(shard, [])]
            for k, target in work:
                t = f.get_tensor(k)
                if target is None:
                    tensors[k] = t.contiguous()
                    continue
                packed, scale, err = _quantize_on_device(t, target.key, chunk_rows, verify)
                tensors[target.base + ".weight_packed"] = packed
                tensors[target.base + ".weight_scale"] = scale
                n_mats += 1
                orig += t.numel() * t.element_size()
                quant += packed.numel() + scale.numel()
                if err is not None:
                    err["tensor"] = target.base + ".weight"
                    errors.append(err)
                    log(f"  {err['tensor']} {list(t.shape)}: mae {err['mae']:.3g} rmse {err['rmse']:.3g} "
                        f"max {err['max_abs']:.3g}")
        save_file(tensors, str(dest / shard.name), metadata={"format": "pt"})
        weight_map.update((name, shard.name) for name in tensors)
        log(f"[{i}/{len(plan.shards)}] wrote {shard.name} ({len(tensors)} tensors)")
        del tensors

    if len(plan.shards) > 1:
        total = sum((dest / s.name).stat().st_size for s in plan.shards)
        index = {"metadata": {"total_size": total}, "weight_map": dict(sorted(weight_map.items()))}
        (dest / "model.safetensors.index.json").write_text(json.dumps(index, indent=2) + "\n", encoding="utf-8")
    record = quantization_config(plan.config["model_type"], plan.n_layers, orig, quant, plan.groups)
    (dest / "quantization_config.json").write_text(json.dumps(record, indent=2) + "\n", encoding="utf-8")
    report = build_report(n_mats, plan.n_layers, orig, quant, errors)
    (dest / "mxfp4_report.json").write_text(json.dumps(report, indent=2) + "\n", encoding="utf-8")
    return report


def quantize_checkpoint(source, dest, chunk_rows: int = 4096, verify: bool = True, log=print,
                        groups=DEFAULT_GROUPS) -> dict:
    """``convert`` under the name of the reference script's job
    (tinyinfer/quantization/quantize_mxfp4.py)."""
    return convert(source, dest, groups=groups, chunk_rows=chunk_rows, verify=verify, log=log)


# ----------------------------------------------------------------- loading

class _QKV(LinearMXFP4):
    """The reference's merged q/k/v projection (QKVParallelLinear,
    tinyinfer/layers/linear.py:58-77) with MXFP4 weights: rows [0, q) are
    q_proj, then k_proj, then v_proj."""

    def __init__(self, hidden: int, q_size: int, kv_size: int):
        super().__init__(hidden, q_size + 2 * kv_size)
        self.q_size, self.kv_size = q_size, kv_size

    def shard_rows(self, shard: str) -> tuple:
        start = {"q": 0, "k": self.q_size, "v": self.q_size + self.kv_size}[shard]
        return start, start + (self.q_size if shard == "q" else self.kv_size)

    def split_qkv(self, y: torch.Tensor):
        return torch.split(y, [self.q_size, self.kv_size, self.kv_size], dim=-1)


class _Attn(nn.Module):
    def __init__(self, config):
        super().__init__()
        heads, kv_heads = int(config.num_attention_heads), int(config.num_key_value_heads)
        head_dim = int(getattr(config, "head_dim", None) or config.hidden_size // heads)
        self.qkv_proj = _QKV(config.hidden_size, heads * head_dim, kv_heads * head_dim)
        self.o_proj = LinearMXFP4(heads * head_dim, config.hidden_size)


class _Layer(nn.Module):
    def __init__(self, config, groups):
        super().__init__()
        if "mlp" in groups:
            self.mlp = Qwen3MLP(config, quantization="mxfp4")
        if "attn" in groups:
            self.self_attn = _Attn(config)


class Qwen3MXFP4Linears(nn.Module):
    """The linears of a Qwen3 model that a checkpoint keeps in MXFP4, under
    the reference model's parameter names: ``model.layers.N.mlp.*_proj``,
    ``model.layers.N.self_attn.{qkv,o}_proj`` and ``lm_head``, for the chosen
    module groups.  ``config`` needs ``hidden_size``, ``intermediate_size``
    and ``num_hidden_layers`` (and the head counts for ``attn``, the
    ``vocab_size`` for ``lm_head``)."""

    def __init__(self, config, groups=DEFAULT_GROUPS):
        super().__init__()
        self.groups = tuple(groups)
        self.model = nn.Module()
        self.model.layers = nn.ModuleList(_Layer(config, groups) for _ in range(config.num_hidden_layers))
        if "lm_head" in groups:
            self.lm_head = LinearMXFP4(config.hidden_size, config.vocab_size)

    def mlp(self, layer: int) -> Qwen3MLP:
        return self.model.layers[layer].mlp

    def attn(self, layer: int) -> _Attn:
        return self.model.layers[layer].self_attn


class Qwen3MLPStack(Qwen3MXFP4Linears):
    """The MLP blocks only (the reference's checkpoint contents)."""

    def __init__(self, config):
        super().__init__(config, ("mlp",))


@dataclass
class LoadReport:
    loaded: list = field(default_factory=list)
    missing: list = field(default_factory=list)
    unexpected: list = field(default_factory=list)
    skipped: list = field(default_factory=list)


def iter_checkpoint(model_path):
    """(name, CPU tensor) for every tensor of the directory's safetensors
    files, file by file in name order."""
    from safetensors import safe_open
    root = Path(model_path).expanduser().resolve()
    files = sorted(root.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"{root} holds no .safetensors files")
    for path in files:
        with safe_open(str(path), framework="pt", device="cpu") as f:
            for name in f.keys():
                yield name, f.get_tensor(name)


_QKV_SHARD = re.compile(r"^(model\.layers\.\d+\.self_attn\.)([qkv])_proj\.(weight_packed|weight_scale)$")


def load_mxfp4_weights(module: nn.Module, model_path, strict: bool = True) -> LoadReport:
    """Copy an MXFP4 checkpoint's converted tensors into ``module``'s
    parameters (see the module docstring for the name mapping), checking
    shapes and dtypes.  Tensors the checkpoint keeps dense (embeddings,
    norms) are ``skipped``; converted tensors, or dense weights of modules
    ``module`` holds in MXFP4, with no parameter to go to are ``unexpected``;
    converted parameters the checkpoint does not fill are ``missing``.
    ``strict`` raises on missing or unexpected tensors."""
    params = dict(module.named_parameters())
    wanted = {n for n in params if n.endswith(".weight_packed") or n.endswith(".weight_scale")}
    filled = {}                                   # parameter name -> rows filled (q/k/v) or None (whole)
    report = LoadReport()

    def dense_counterpart(name):
        """A dense weight of a module the model holds in MXFP4."""
        if not name.endswith(".weight"):
            return False
        base = name[: -len(".weight")]
        qkv = re.fullmatch(r"(model\.layers\.\d+\.self_attn\.)[qkv]_proj", base)
        return (base + ".weight_packed") in params or bool(qkv and qkv.group(1) + "qkv_proj.weight_packed" in params)

    for name, t in iter_checkpoint(model_path):
        m = _QKV_SHARD.fullmatch(name)
        if m:
            target = f"{m.group(1)}qkv_proj.{m.group(3)}"
            if target not in params:
                report.unexpected.append(name)
                continue
            mod = module.get_submodule(target.rsplit(".", 1)[0])
            r0, r1 = mod.shard_rows(m.group(2))
            dst = params[target].data[r0:r1]
        elif _QUANT_NAME.fullmatch(name):
            if name not in params:
                report.unexpected.append(name)
                continue
            dst = params[name].data
            target, r0, r1 = name, 0, params[name].shape[0]
        else:
            (report.unexpected if dense_counterpart(name) else report.skipped).append(name)
            continue
        if t.dtype != torch.uint8:
            raise RuntimeError(f"{name} is {t.dtype}; converted MXFP4 tensors are uint8")
        if tuple(t.shape) != tuple(dst.shape):
            raise RuntimeError(f"{name}: the checkpoint holds {list(t.shape)}, the model expects "
                               f"{list(dst.shape)} (shape mismatch)")
        dst.copy_(t.to(dst.device))
        filled.setdefault(target, []).append((r0, r1))
        report.loaded.append(name)
    for n in sorted(wanted):
        rows = sorted(filled.get(n, []))
        covered, end = True, 0
        for r0, r1 in rows:
            covered = covered and r0 == end
            end = r1
        if not rows or not covered or end != params[n].shape[0]:
            report.missing.append(n)
    if strict and (report.missing or report.unexpected):
        raise RuntimeError(f"the MXFP4 checkpoint and the model disagree: missing {report.missing[:8]}, "
                           f"unexpected {report.unexpected[:8]}")
    return report


def load_mlp_weights(module: nn.Module, model_path, strict: bool = True) -> LoadReport:
    """``load_mxfp4_weights`` for a module that holds only the MLPs."""
    return load_mxfp4_weights(module, model_path, strict)


def main(argv=None) -> None:
    """``python -m tinyinfer_amd.checkpoint --input HF_DIR --output NEW_DIR
    [--chunk-rows N] [--no-verify] [--modules mlp,attn,lm_head]`` (the
    reference script's arguments, quantize_mxfp4.py:86-92, plus the module
    groups)."""
    import argparse
    ap = argparse.ArgumentParser(description="Convert a Qwen3 checkpoint to MXFP4 weights on a gfx950 GPU")
    ap.add_argument("--input", required=True, type=Path, help="Hugging Face Qwen3 checkpoint directory")
    ap.add_argument("--output", required=True, type=Path, help="new or empty output directory")
    ap.add_argument("--chunk-rows", type=int, default=4096, help="weight rows sent to the GPU at a time")
    ap.add_argument("--verify", action=argparse.BooleanOptionalAction, default=True,
                    help="decode again and record the quantization error per weight")
    ap.add_argument("--modules", default="mlp", help="comma-separated groups among: " + ", ".join(MODULE_GROUPS))
    a = ap.parse_args(argv)
    groups = tuple(g for g in a.modules.split(",") if g)
    rep = convert(a.input, a.output, groups=groups, chunk_rows=a.chunk_rows, verify=a.verify,
                  log=lambda m: print(m, flush=True))
    o, q = rep["mlp_original_bytes"], rep["mlp_quantized_bytes"]
    print(f"{rep['num_quantized_matrices']} weights: {o / 2 ** 20:.1f} MiB -> {q / 2 ** 20:.1f} MiB "
          f"({rep['mlp_compression_ratio']:.2f}x) in {Path(a.output).expanduser().resolve()}", flush=True)


if __name__ == "__main__":
    main()
