"""CPU-side checks of the boundary: the C-ABI library loads and exports every
function that include/tinyinfer_mxfp4.h declares, argument validation that
happens before any device work returns the documented status codes, and the
torch wrapper raises the reference's messages for non-device inputs."""

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tinyinfer_mxfp4.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tinyinfer_\w+)\s*\(", text)))


def declared_macros():
    return dict((m, int(v)) for m, v in re.findall(r"#define\s+(TI_\w+)\s+(\d+)u?\b", open(HEADER).read()))


@pytest.fixture(scope="module")
def capi():
    from tinyinfer_amd import capi as c
    if not os.path.exists(c.LIB_PATH):
        pytest.fail("libtinyinfer_mxfp4.so is not built; run python -m tinyinfer_amd.build")
    return c


def test_library_exports_every_declared_symbol(capi):
    names = declared_functions()
    assert len(names) >= 6
    handle = ctypes.CDLL(capi.LIB_PATH)
    for n in names:
        assert hasattr(handle, n), n
    # the Python binding covers the same set
    assert set(names) == set(capi.SIGNATURES)


def test_python_constants_match_header(capi):
    for name, value in declared_macros().items():
        assert getattr(capi, name) == value, name


def test_abi_version_and_status_strings(capi):
    assert capi.lib().tinyinfer_mxfp4_abi_version() == 7
    assert capi.status_string(0) == "ok"
    assert "32" in capi.status_string(capi.TI_ERR_BAD_SHAPE)
    assert capi.status_string(999) == "unknown status"


def test_tuning_options(capi):
    """Options start from the environment (read once) and change through the
    C ABI; unknown names and out-of-range values are refused; the context
    manager restores the previous value."""
    assert capi.get_option("TINYINFER_TILE") in (0, 1)
    before = capi.get_option("TINYINFER_RING_KSPLIT")
    with capi.option("TINYINFER_RING_KSPLIT", 5):
        assert capi.get_option("TINYINFER_RING_KSPLIT") == 5
    assert capi.get_option("TINYINFER_RING_KSPLIT") == before
    for name, bad in (("TINYINFER_ROW_SPLIT_DOWN", 3), ("TINYINFER_RING_NW_GU", 6), ("TINYINFER_TILE", 2),
                      ("TINYINFER_RING_KSPLIT", -1), ("TINYINFER_NO_SUCH_OPTION", 1)):
        with pytest.raises(capi.TinyInferError) as e:
            capi.set_option(name, bad)
        assert e.value.status == capi.TI_ERR_INVALID_ARG
    assert capi.lib().tinyinfer_mxfp4_set_option(None, 1) == capi.TI_ERR_INVALID_ARG
    held, limit = capi.workspace_info()
    assert held >= 0 and limit == capi.get_option("TINYINFER_WORKSPACE_MB") << 20


def test_options_from_environment_read_once():
    """A fresh process takes the options from its environment."""
    import subprocess
    import sys
    code = ("from tinyinfer_amd import capi; "
            "print(capi.get_option('TINYINFER_TILE'), capi.get_option('TINYINFER_ROW_SPLIT_DOWN'), "
            "capi.get_option('TINYINFER_RING_NW_GU'))")
    env = dict(os.environ, TINYINFER_TILE="0", TINYINFER_ROW_SPLIT_DOWN="2", TINYINFER_RING_NW_GU="5")
    out = subprocess.run([sys.executable, "-c", code], cwd=ROOT, env=env, capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    # an invalid value (5 waves) leaves the default
    assert out.stdout.split() == ["0", "2", "8"]


def test_validation_before_device_work(capi):
    L = capi.lib()
    f = L.tinyinfer_mlp_forward_mxfp4
    p = 0x1000  # never dereferenced: validation fails first
    # null pointer
    assert f(None, p, p, p, p, p, p, 1, 64, 64, p, p, 1, None) == capi.TI_ERR_INVALID_ARG
    # zero sizes
    assert f(p, p, p, p, p, p, p, 0, 64, 64, p, p, 1, None) == capi.TI_ERR_INVALID_ARG
    # hidden / intermediate not multiples of 32
    assert f(p, p, p, p, p, p, p, 1, 48, 64, p, p, 1, None) == capi.TI_ERR_BAD_SHAPE
    assert f(p, p, p, p, p, p, p, 1, 64, 80, p, p, 1, None) == capi.TI_ERR_BAD_SHAPE
    # fp32 activations are not supported (reference: FP16/BF16 only)
    assert f(p, p, p, p, p, p, p, 1, 64, 64, p, p, 2, None) == capi.TI_ERR_BAD_DTYPE
    # forced path out of range
    g = L.tinyinfer_mlp_forward_mxfp4_path
    assert g(p, p, p, p, p, p, p, 1, 64, 64, p, p, 1, 7, None) in (capi.TI_ERR_INVALID_ARG,)
    # stage entry points: the pointers of the other stage may be null
    gu = L.tinyinfer_mlp_gate_up_mxfp4
    assert gu(p, p, p, p, None, 1, 64, 64, p, 1, 0, None) == capi.TI_ERR_INVALID_ARG
    assert gu(p, p, p, p, p, 1, 64, 40, p, 1, 0, None) == capi.TI_ERR_BAD_SHAPE
    assert gu(p, p, p, p, p, 1, 64, 64, p, 2, 0, None) == capi.TI_ERR_BAD_DTYPE
    dn = L.tinyinfer_mlp_down_mxfp4
    assert dn(p, p, None, 1, 64, 64, p, 1, 0, None) == capi.TI_ERR_INVALID_ARG
    assert dn(p, p, p, 0, 64, 64, p, 1, 0, None) == capi.TI_ERR_INVALID_ARG
    assert dn(p, p, p, 1, 64, 64, p, 1, 4, None) == capi.TI_ERR_INVALID_ARG
    # residual MLP: null residual, misaligned residual; linear: null X, shapes, misaligned residual
    rf = L.tinyinfer_mlp_forward_mxfp4_residual
    assert rf(p, p, p, p, p, p, p, 1, 64, 64, p, None, p, 1, 0, None) == capi.TI_ERR_INVALID_ARG
    assert rf(p, p, p, p, p, p, p, 1, 64, 64, p, p + 2, p, 1, 0, None) == capi.TI_ERR_MISALIGNED
    assert rf(p, p, p, p, p, p, p, 1, 64, 64, p, p, p, 1, 9, None) == capi.TI_ERR_INVALID_ARG
    li = L.tinyinfer_mxfp4_linear
    assert li(None, p, p, 1, 64, 64, None, p, 1, 0, None) == capi.TI_ERR_INVALID_ARG
    assert li(p, p, p, 1, 48, 64, None, p, 1, 0, None) == capi.TI_ERR_BAD_SHAPE
    assert li(p, p, p, 1, 64, 40, None, p, 1, 0, None) == capi.TI_ERR_BAD_SHAPE
    assert li(p, p, p, 1, 64, 64, p + 8, p, 1, 0, None) == capi.TI_ERR_MISALIGNED
    assert li(p, p + 1, p, 1, 64, 64, None, p, 1, 0, None) == capi.TI_ERR_MISALIGNED
    # decoder MLP half with the RMSNorm prologue: null norm weight / xn, misaligned norm weight
    nf = L.tinyinfer_mlp_forward_mxfp4_rmsnorm
    assert nf(p, None, 1e-6, p, p, p, p, p, p, 1, 64, 64, p, p, p, 1, 0, None) == capi.TI_ERR_INVALID_ARG
    assert nf(p, p, 1e-6, p, p, p, p, p, p, 1, 64, 64, None, p, p, 1, 0, None) == capi.TI_ERR_INVALID_ARG
    assert nf(p, p + 4, 1e-6, p, p, p, p, p, p, 1, 64, 64, p, p, p, 1, 0, None) == capi.TI_ERR_MISALIGNED
    assert nf(p, p, 1e-6, p, p, p, p, p, p, 1, 48, 64, p, p, p, 1, 0, None) == capi.TI_ERR_BAD_SHAPE
    assert nf(p, p, 1e-6, p, p, p, p, p, p, 1, 64, 64, p, p, p, 1, 5, None) == capi.TI_ERR_INVALID_ARG
    rn = L.tinyinfer_rmsnorm
    assert rn(None, p, 1e-6, 1, 64, p, 1, None) == capi.TI_ERR_INVALID_ARG
    assert rn(p, p, 1e-6, 1, 60, p, 1, None) == capi.TI_ERR_BAD_SHAPE
    assert rn(p, p, 1e-6, 1, 64, p, 2, None) == capi.TI_ERR_BAD_DTYPE
    assert rn(p, p + 2, 1e-6, 1, 64, p, 1, None) == capi.TI_ERR_MISALIGNED
    assert L.tinyinfer_mxfp4_dequant(p, p, 4, 48, p, 2, None) == capi.TI_ERR_BAD_SHAPE
    assert L.tinyinfer_mxfp4_dequant(p, p, 4, 64, p, 0, None) == capi.TI_ERR_BAD_DTYPE
    assert L.tinyinfer_mxfp4_quantize(p, 2, 4, 64, p, p, None, None) == capi.TI_ERR_INVALID_ARG


def test_no_device_reports_no_device(capi):
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    p = 0x1000
    st = capi.lib().tinyinfer_mlp_forward_mxfp4(p, p, p, p, p, p, p, 1, 64, 64, p, p, 1, None)
    assert st == capi.TI_ERR_NO_DEVICE
    assert capi.lib().tinyinfer_mlp_down_mxfp4(p, p, p, 1, 64, 64, p, 1, 0, None) == capi.TI_ERR_NO_DEVICE


def _cpu_inputs(m=2, h=64, i=96, xdtype=torch.bfloat16):
    u8 = torch.uint8
    return [torch.zeros(m, h, dtype=xdtype), torch.zeros(i, h // 2, dtype=u8), torch.zeros(i, h // 32, dtype=u8),
            torch.zeros(i, h // 2, dtype=u8), torch.zeros(i, h // 32, dtype=u8),
            torch.zeros(h, i // 2, dtype=u8), torch.zeros(h, i // 32, dtype=u8)]


def test_torch_wrapper_rejects_host_tensors_with_reference_message():
    from tinyinfer_amd.extension import load_extension
    C = load_extension()
    args = _cpu_inputs()
    with pytest.raises(RuntimeError, match="X must be a CUDA tensor"):
        C.mlp_forward_mxfp4(*args)
    names = ["X", "gate", "gate_scale", "up", "up_scale", "down", "down_scale"]
    assert C.mlp_forward_mxfp4.__doc__.startswith("mlp_forward_mxfp4(X: torch.Tensor, gate: torch.Tensor")
    for n in names:
        assert f"{n}: torch.Tensor" in C.mlp_forward_mxfp4.__doc__


def test_rmsnorm_wrappers_reject_host_tensors_with_reference_message():
    from tinyinfer_amd.extension import load_extension
    C = load_extension()
    with pytest.raises(RuntimeError, match="input must be a CUDA tensor"):
        C.rmsnorm_forward(torch.zeros(2, 64, dtype=torch.bfloat16), torch.ones(64, dtype=torch.bfloat16), 1e-6)
    args = _cpu_inputs()
    with pytest.raises(RuntimeError, match="X must be a CUDA tensor"):
        C.mlp_forward_mxfp4_rmsnorm(args[0], torch.ones(64, dtype=torch.bfloat16), 1e-6, *args[1:])


def test_load_extension_is_cached():
    from tinyinfer_amd.extension import load_extension
    assert load_extension() is load_extension()


def test_qwen3_mlp_parameters_match_reference_layout():
    from tinyinfer_amd.mlp import Qwen3MLP, qwen3_config
    m = Qwen3MLP(qwen3_config(64, 96), quantization="mxfp4")
    assert m.gate_proj.weight_packed.shape == (96, 32) and m.gate_proj.weight_scale.shape == (96, 2)
    assert m.up_proj.weight_packed.shape == (96, 32) and m.up_proj.weight_scale.shape == (96, 2)
    assert m.down_proj.weight_packed.shape == (64, 48) and m.down_proj.weight_scale.shape == (64, 3)
    for p in m.parameters():
        assert p.dtype == torch.uint8 and not p.requires_grad
    keys = sorted(m.state_dict())
    assert keys == sorted(f"{a}_proj.weight_{b}" for a in ("gate", "up", "down") for b in ("packed", "scale"))
    with pytest.raises(NotImplementedError):
        Qwen3MLP(qwen3_config(64, 96), quantization=None)


def test_quant_config_record_matches_reference_format():
    from tinyinfer_amd.quantization import QUANT_CONFIG
    assert QUANT_CONFIG["format"] == "tinyinfer_mxfp4_weight_only_v1"
    assert QUANT_CONFIG["block_size"] == 32
    assert QUANT_CONFIG["packed_nibble_order"] == "first_element_low_nibble"
    assert QUANT_CONFIG["scale_encoding"] == "stored_byte = unbiased_exponent + 127"


def test_host_quantizer_wrapper_validates_shape_first():
    from tinyinfer_amd.quantization import quantize_chunk, dequantize_chunk
    with pytest.raises(ValueError):
        quantize_chunk(torch.zeros(2, 48))
    with pytest.raises(ValueError):
        dequantize_chunk(torch.zeros(1, 16, dtype=torch.uint8), torch.zeros(1, 2, dtype=torch.uint8))


def test_workload_accounting():
    from tinyinfer_amd.workloads import alg_bytes, alg_flops
    assert alg_bytes(1, 4096, 12288) == 80_232_448
    assert alg_bytes(2048, 4096, 12288) == 113_770_496
    assert alg_bytes(16, 1024, 3072) == 5_079_040
    assert alg_flops(2048, 4096, 12288) == 618_475_290_624
    assert 64 * alg_bytes(1, 5120, 25600) == 13_370_654_720
