"""ctypes binding of the C ABI (``include/tinyinfer_mxfp4.h``).

This is the binding a non-torch host (or a test) uses: every entry point
takes raw device pointers, sizes and a stream handle.  ``torch`` tensors are
accepted by the convenience wrappers only to read ``data_ptr()`` and the
current stream; nothing crosses the boundary as a torch type.
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtinyinfer_mxfp4.so")

TI_OK = 0
TI_ERR_INVALID_ARG = 1
TI_ERR_BAD_SHAPE = 2
TI_ERR_BAD_DTYPE = 3
TI_ERR_HIP = 4
TI_ERR_NO_DEVICE = 5
TI_ERR_TOO_LARGE = 6
TI_ERR_MISALIGNED = 7
TI_ERR_UNSUPPORTED = 8
TI_ERR_SCRATCH = 9

TI_DTYPE_F16 = 0
TI_DTYPE_BF16 = 1
TI_DTYPE_F32 = 2

TI_PATH_AUTO = 0
TI_PATH_SKINNY = 1
TI_PATH_GEMM = 2
TI_PATH_DECODE = 3

TI_QFLAG_NONFINITE = 1
TI_QFLAG_EXP_RANGE = 2

# name -> (restype, argtypes); mirrors include/tinyinfer_mxfp4.h
_vp, _u8p, _sz, _int = ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
SIGNATURES = {
    "tinyinfer_mlp_forward_mxfp4": (_int, [_vp, _u8p, _u8p, _u8p, _u8p, _u8p, _u8p, _sz, _sz, _sz, _vp, _vp, _int, _vp]),
    "tinyinfer_mlp_forward_mxfp4_noalloc": (_int, [_vp, _u8p, _u8p, _u8p, _u8p, _u8p, _u8p, _sz, _sz, _sz, _vp, _vp, _int,
                                                   _vp]),
    "tinyinfer_mlp_forward_mxfp4_path": (_int, [_vp, _u8p, _u8p, _u8p, _u8p, _u8p, _u8p, _sz, _sz, _sz, _vp, _vp, _int, _int, _vp]),
    "tinyinfer_mlp_gate_up_mxfp4": (_int, [_vp, _u8p, _u8p, _u8p, _u8p, _sz, _sz, _sz, _vp, _int, _int, _vp]),
    "tinyinfer_mlp_down_mxfp4": (_int, [_vp, _u8p, _u8p, _sz, _sz, _sz, _vp, _int, _int, _vp]),
    "tinyinfer_mlp_forward_mxfp4_residual": (_int, [_vp, _u8p, _u8p, _u8p, _u8p, _u8p, _u8p, _sz, _sz, _sz, _vp, _vp,
                                                    _vp, _int, _int, _vp]),
    "tinyinfer_mlp_forward_mxfp4_rmsnorm": (_int, [_vp, _vp, ctypes.c_float, _u8p, _u8p, _u8p, _u8p, _u8p, _u8p,
                                                   _sz, _sz, _sz, _vp, _vp, _vp, _int, _int, _vp]),
    "tinyinfer_rmsnorm": (_int, [_vp, _vp, ctypes.c_float, _sz, _sz, _vp, _int, _vp]),
    "tinyinfer_mxfp4_linear": (_int, [_vp, _u8p, _u8p, _sz, _sz, _sz, _vp, _vp, _int, _int, _vp]),
    "tinyinfer_mxfp4_dequant": (_int, [_u8p, _u8p, _sz, _sz, _vp, _int, _vp]),
    "tinyinfer_mxfp4_quantize": (_int, [_vp, _int, _sz, _sz, _u8p, _u8p, _vp, _vp]),
    "tinyinfer_mxfp4_diagnostics": (_int, [ctypes.c_void_p]),
    "tinyinfer_mxfp4_decode_reset": (_int, []),
    "tinyinfer_mxfp4_set_option": (_int, [ctypes.c_char_p, _int]),
    "tinyinfer_mxfp4_get_option": (_int, [ctypes.c_char_p, ctypes.c_void_p]),
    "tinyinfer_mxfp4_workspace_info": (_int, [ctypes.c_void_p, ctypes.c_void_p]),
    "tinyinfer_mxfp4_release_workspaces": (_int, []),
    "tinyinfer_mxfp4_status_string": (ctypes.c_char_p, [_int]),
    "tinyinfer_mxfp4_abi_version": (_int, []),
}


class TinyInferError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what} failed: {status_string(status)} (status {status})")


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run: python -m tinyinfer_amd.build")
    handle = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


def status_string(status: int) -> str:
    return lib().tinyinfer_mxfp4_status_string(int(status)).decode()


def _check(status: int, what: str) -> None:
    if status != TI_OK:
        raise TinyInferError(status, what)


def _stream_handle(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _act_code(dtype) -> int:
    import torch
    if dtype == torch.bfloat16:
        return TI_DTYPE_BF16
    if dtype == torch.float16:
        return TI_DTYPE_F16
    raise ValueError("MXFP4 MLP only supports FP16 and BF16 activations")


def mlp_forward(x, gp, gs, up, us, dp, ds, out=None, tmp=None, path: int = TI_PATH_AUTO, stream=None,
                residual=None):
    """Run the MLP through the C ABI on torch-owned device buffers.

    ``out``/``tmp`` may be preallocated ([N, hidden] / [N, intermediate] in
    ``x``'s dtype); they are allocated when omitted.  With ``residual``
    ([N, hidden], may be ``out`` itself) the result is ``residual + MLP(x)``,
    added in the down stage's epilogue.  Returns ``out``."""
    import torch
    n, hidden = x.shape
    inter = gp.shape[0]
    if out is None:
        out = torch.empty((n, hidden), dtype=x.dtype, device=x.device)
    if tmp is None:
        tmp = torch.empty((n, inter), dtype=x.dtype, device=x.device)
    if residual is None:
        st = lib().tinyinfer_mlp_forward_mxfp4_path(
            x.data_ptr(), gp.data_ptr(), gs.data_ptr(), up.data_ptr(), us.data_ptr(), dp.data_ptr(), ds.data_ptr(),
            n, hidden, inter, tmp.data_ptr(), out.data_ptr(), _act_code(x.dtype), int(path), _stream_handle(stream))
        _check(st, "tinyinfer_mlp_forward_mxfp4")
    else:
        if tuple(residual.shape) != (n, hidden) or residual.dtype != x.dtype or not residual.is_contiguous():
            raise ValueError("residual must be a contiguous [N, hidden] tensor of x's dtype")
        st = lib().tinyinfer_mlp_forward_mxfp4_residual(
            x.data_ptr(), gp.data_ptr(), gs.data_ptr(), up.data_ptr(), us.data_ptr(), dp.data_ptr(), ds.data_ptr(),
            n, hidden, inter, tmp.data_ptr(), residual.data_ptr(), out.data_ptr(), _act_code(x.dtype), int(path),
            _stream_handle(stream))
        _check(st, "tinyinfer_mlp_forward_mxfp4_residual")
    return out


def mlp_forward_rmsnorm(x, norm_w, eps, gp, gs, up, us, dp, ds, out=None, tmp=None, xn=None,
                        path: int = TI_PATH_AUTO, stream=None):
    """The decoder layer's MLP half: ``out = x + MLP(RMSNorm(x))`` with the
    norm in the MLP's prologue.  ``xn`` ([N, hidden], allocated when omitted)
    receives the normalized rows; ``out`` may be ``x`` itself.  Returns
    ``(out, xn)``."""
    import torch
    n, hidden = x.shape
    inter = gp.shape[0]
    if tuple(norm_w.shape) != (hidden,) or norm_w.dtype != x.dtype or not norm_w.is_contiguous():
        raise ValueError("norm_w must be a contiguous [hidden] tensor of x's dtype")
    if out is None:
        out = torch.empty((n, hidden), dtype=x.dtype, device=x.device)
    if tmp is None:
        tmp = torch.empty((n, inter), dtype=x.dtype, device=x.device)
    if xn is None:
        xn = torch.empty((n, hidden), dtype=x.dtype, device=x.device)
    st = lib().tinyinfer_mlp_forward_mxfp4_rmsnorm(
        x.data_ptr(), norm_w.data_ptr(), float(eps), gp.data_ptr(), gs.data_ptr(), up.data_ptr(), us.data_ptr(),
        dp.data_ptr(), ds.data_ptr(), n, hidden, inter, xn.data_ptr(), tmp.data_ptr(), out.data_ptr(),
        _act_code(x.dtype), int(path), _stream_handle(stream))
    _check(st, "tinyinfer_mlp_forward_mxfp4_rmsnorm")
    return out, xn


def rmsnorm(x, w, eps, out=None, stream=None):
    """RMSNorm of the rows of x ([..., hidden]) with weight w ([hidden])."""
    import torch
    hidden = x.shape[-1]
    rows = x.numel() // hidden
    if out is None:
        out = torch.empty_like(x)
    st = lib().tinyinfer_rmsnorm(x.data_ptr(), w.data_ptr(), float(eps), rows, hidden, out.data_ptr(),
                                 _act_code(x.dtype), _stream_handle(stream))
    _check(st, "tinyinfer_rmsnorm")
    return out


def linear(x, w, ws, out=None, residual=None, path: int = TI_PATH_AUTO, stream=None):
    """One MXFP4 linear layer: out = x w^T (+ residual) [N, out_features],
    w [out_features, in_features/2] packed, ws [out_features, in_features/32]."""
    import torch
    n, k = x.shape
    r = w.shape[0]
    if out is None:
        out = torch.empty((n, r), dtype=x.dtype, device=x.device)
    if residual is not None and (tuple(residual.shape) != (n, r) or residual.dtype != x.dtype
                                 or not residual.is_contiguous()):
        raise ValueError("residual must be a contiguous [N, out_features] tensor of x's dtype")
    st = lib().tinyinfer_mxfp4_linear(
        x.data_ptr(), w.data_ptr(), ws.data_ptr(), n, k, r, residual.data_ptr() if residual is not None else None,
        out.data_ptr(), _act_code(x.dtype), int(path), _stream_handle(stream))
    _check(st, "tinyinfer_mxfp4_linear")
    return out


def gate_up(x, gp, gs, up, us, tmp=None, path: int = TI_PATH_AUTO, stream=None):
    """The gate_up stage alone: returns tmp = SiLU(x gate^T) * (x up^T) [N, intermediate]."""
    import torch
    n, hidden = x.shape
    inter = gp.shape[0]
    if tmp is None:
        tmp = torch.empty((n, inter), dtype=x.dtype, device=x.device)
    st = lib().tinyinfer_mlp_gate_up_mxfp4(
        x.data_ptr(), gp.data_ptr(), gs.data_ptr(), up.data_ptr(), us.data_ptr(), n, hidden, inter,
        tmp.data_ptr(), _act_code(x.dtype), int(path), _stream_handle(stream))
    _check(st, "tinyinfer_mlp_gate_up_mxfp4")
    return tmp


def down(tmp, dp, ds, out=None, path: int = TI_PATH_AUTO, stream=None):
    """The down stage alone: returns out = tmp down^T [N, hidden]."""
    import torch
    n, inter = tmp.shape
    hidden = dp.shape[0]
    if out is None:
        out = torch.empty((n, hidden), dtype=tmp.dtype, device=tmp.device)
    st = lib().tinyinfer_mlp_down_mxfp4(
        tmp.data_ptr(), dp.data_ptr(), ds.data_ptr(), n, hidden, inter, out.data_ptr(),
        _act_code(tmp.dtype), int(path), _stream_handle(stream))
    _check(st, "tinyinfer_mlp_down_mxfp4")
    return out


def decode_barrier_timeouts() -> int:
    """Grid-barrier timeouts of the fused decode kernel on the current device."""
    v = ctypes.c_uint32(0)
    _check(lib().tinyinfer_mxfp4_diagnostics(ctypes.byref(v)), "tinyinfer_mxfp4_diagnostics")
    return int(v.value)


def decode_reset() -> None:
    """Clear the fused decode kernel's cross-workgroup state (synchronous)."""
    _check(lib().tinyinfer_mxfp4_decode_reset(), "tinyinfer_mxfp4_decode_reset")


def set_option(name: str, value: int) -> None:
    """Set a tuning option (see tinyinfer_mxfp4_set_option) for every later call."""
    _check(lib().tinyinfer_mxfp4_set_option(name.encode(), int(value)), f"tinyinfer_mxfp4_set_option({name})")


def get_option(name: str) -> int:
    v = ctypes.c_int(0)
    _check(lib().tinyinfer_mxfp4_get_option(name.encode(), ctypes.byref(v)), f"tinyinfer_mxfp4_get_option({name})")
    return int(v.value)


class option:
    """Context manager: ``with option("TINYINFER_TILE", 0): ...`` sets a tuning
    option for the block and restores the previous value after it."""

    def __init__(self, name: str, value: int):
        self.name, self.value = name, int(value)

    def __enter__(self):
        self.prev = get_option(self.name)
        set_option(self.name, self.value)
        return self

    def __exit__(self, *exc):
        set_option(self.name, self.prev)
        return False


def workspace_info():
    """(bytes held by split-K workspaces over all devices/streams, limit per buffer)."""
    held, limit = ctypes.c_size_t(0), ctypes.c_size_t(0)
    _check(lib().tinyinfer_mxfp4_workspace_info(ctypes.byref(held), ctypes.byref(limit)),
           "tinyinfer_mxfp4_workspace_info")
    return int(held.value), int(limit.value)


def release_workspaces() -> None:
    """Synchronize and free every split-K workspace (no earlier graph may be replayed afterwards)."""
    _check(lib().tinyinfer_mxfp4_release_workspaces(), "tinyinfer_mxfp4_release_workspaces")


def dequant(packed, scale, out_dtype=None, stream=None):
    import torch
    out_dtype = out_dtype or torch.float32
    rows, half_k = packed.shape
    out = torch.empty((rows, 2 * half_k), dtype=out_dtype, device=packed.device)
    code = TI_DTYPE_F32 if out_dtype == torch.float32 else TI_DTYPE_BF16
    st = lib().tinyinfer_mxfp4_dequant(packed.data_ptr(), scale.data_ptr(), rows, 2 * half_k, out.data_ptr(),
                                       code, _stream_handle(stream))
    _check(st, "tinyinfer_mxfp4_dequant")
    return out


def quantize(w, stream=None):
    """Device quantizer; returns (packed, scale, flags) device tensors."""
    import torch
    codes = {torch.float32: TI_DTYPE_F32, torch.bfloat16: TI_DTYPE_BF16, torch.float16: TI_DTYPE_F16}
    rows, k = w.shape
    packed = torch.empty((rows, k // 2), dtype=torch.uint8, device=w.device)
    scale = torch.empty((rows, k // 32), dtype=torch.uint8, device=w.device)
    flags = torch.empty((1,), dtype=torch.int32, device=w.device)
    st = lib().tinyinfer_mxfp4_quantize(w.data_ptr(), codes[w.dtype], rows, k, packed.data_ptr(),
                                        scale.data_ptr(), flags.data_ptr(), _stream_handle(stream))
    _check(st, "tinyinfer_mxfp4_quantize")
    return packed, scale, flags
