"""fxgpu.abi: ctypes mirror of include/fx_abi.h and the libfxforge.so loader.

The C ABI is the only way the fxlm/fxgpu ops reach the GPU: every op wrapper
allocates its tensors through torch's caching allocator, then passes raw device
pointers, sizes and the current torch stream to one ``fx_*`` entry point.
There is no other code path: when the library is missing, ``lib()`` raises.
"""
import ctypes
import os
import threading

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_ROOT, "libfxforge.so")
HEADER_PATH = os.path.join(os.path.dirname(_PKG_ROOT), "include", "fx_abi.h")

FX_EINVAL = -1
FX_ABI_VERSION = 5
MAX_TENSORS = 64
ADAMW_NOALLOC_SCRATCH_BYTES = 1 << 20   # FX_ADAMW_NOALLOC_SCRATCH_BYTES

c_void_p = ctypes.c_void_p
c_int32 = ctypes.c_int32
c_int64 = ctypes.c_int64
c_float = ctypes.c_float


class fxCEArgs(ctypes.Structure):
    """Mirror of ``fxCEArgs`` (fx_abi.h)."""
    _fields_ = [
        ("logits", c_void_p), ("target", c_void_p), ("grad", c_void_p),
        ("row_loss", c_void_p), ("mul", c_void_p),
        ("N", c_int64), ("V", c_int64), ("ld", c_int64), ("ldg", c_int64),
        ("ignore_index", c_int64),
    ]


class fxTensorList(ctypes.Structure):
    """Mirror of ``fxTensorList`` (fx_abi.h)."""
    _fields_ = [
        ("g", c_void_p * MAX_TENSORS),
        ("off", c_int64 * MAX_TENSORS),
        ("n", c_int64 * MAX_TENSORS),
        ("wd", c_int32 * MAX_TENSORS),
        ("count", c_int32),
    ]


class fxAdamWState(ctypes.Structure):
    """Mirror of ``fxAdamWState`` (fx_abi.h)."""
    _fields_ = [
        ("master", c_void_p), ("m", c_void_p), ("v", c_void_p), ("p16", c_void_p),
        ("step", c_void_p), ("found_inf", c_void_p), ("grad_norm", c_void_p),
        ("scale", c_void_p), ("growth", c_void_p), ("work", c_void_p),
        ("lr", c_float), ("beta1", c_float), ("beta2", c_float), ("eps", c_float),
        ("weight_decay", c_float), ("max_grad_norm", c_float),
        ("growth_factor", c_float), ("backoff_factor", c_float),
        ("growth_interval", c_int32),
    ]


class fxAttnArgs(ctypes.Structure):
    """Mirror of ``fxAttnArgs`` (fx_abi.h)."""
    _fields_ = [
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p),
        ("o", c_void_p), ("dout", c_void_p), ("o_out", c_void_p),
        ("dq", c_void_p), ("dk", c_void_p), ("dv", c_void_p),
        ("lse", c_void_p), ("lse_out", c_void_p), ("delta", c_void_p),
        ("qsb", c_int64), ("qst", c_int64), ("qsh", c_int64),
        ("ksb", c_int64), ("kst", c_int64), ("ksh", c_int64),
        ("vsb", c_int64), ("vst", c_int64), ("vsh", c_int64),
        ("dqb", c_int64), ("dqt", c_int64), ("dqh", c_int64),
        ("dkb", c_int64), ("dkt", c_int64), ("dkh", c_int64),
        ("dvb", c_int64), ("dvt", c_int64), ("dvh", c_int64),
        ("B", c_int32), ("T", c_int32), ("H", c_int32),
        ("D", c_int32), ("scale", c_float), ("causal", c_int32),
    ]


class fxAttnDecodeArgs(ctypes.Structure):
    _fields_ = [
        ("q", c_void_p), ("k", c_void_p), ("v", c_void_p), ("lens", c_void_p),
        ("o", c_void_p), ("lse", c_void_p), ("work", c_void_p),
        ("qsb", c_int64), ("qsh", c_int64), ("ksb", c_int64), ("kst", c_int64), ("ksh", c_int64),
        ("vsb", c_int64), ("vst", c_int64), ("vsh", c_int64),
        ("B", c_int32), ("H", c_int32), ("Tmax", c_int32), ("D", c_int32),
        ("scale", c_float),
        ("knew", c_void_p), ("vnew", c_void_p),
        ("knb", c_int64), ("knh", c_int64), ("vnb", c_int64), ("vnh", c_int64),
    ]


class fxLinearArgs(ctypes.Structure):
    _fields_ = [
        ("X", c_void_p), ("ldx", c_int64), ("W", c_void_p), ("bias", c_void_p),
        ("res", c_void_p), ("ldres", c_int64), ("norm_w", c_void_p),
        ("Y", c_void_p), ("H", c_void_p),
        ("M", c_int64), ("N", c_int64), ("K", c_int64),
        ("eps", c_float), ("act", c_int32),
    ]


_P = c_void_p
# name -> (restype, argtypes); must list exactly the functions of fx_abi.h
SIGNATURES = {
    "fx_abi_version": (c_int32, []),
    "fx_last_error": (ctypes.c_char_p, []),
    "fx_fill_f32": (c_int32, [_P, c_int64, c_float, _P]),
    "fx_rms_norm_fwd": (c_int32, [_P, _P, _P, _P, c_int64, c_int32, c_float, _P]),
    "fx_rms_norm_fwd_add": (c_int32, [_P, _P, _P, _P, _P, _P, c_int64, c_int32, c_float, _P]),
    "fx_rms_norm_bwd_workspace": (c_int64, [c_int64, c_int32]),
    "fx_rms_norm_bwd": (c_int32, [_P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int32, _P]),
    "fx_rms_norm_bwd_add": (c_int32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int32, _P]),
    "fx_ce_inv_nvalid": (c_int32, [_P, c_int64, c_int64, _P, c_float, _P, _P, _P]),
    "fx_ce_fwd_grad": (c_int32, [ctypes.POINTER(fxCEArgs), _P]),
    "fx_ce_loss_finalize": (c_int32, [_P, c_int64, _P, _P, _P]),
    "fx_ce_scale_grad": (c_int32, [_P, c_int64, _P, _P, c_int32, _P]),
    "fx_ce_lin_grad_scale": (c_int32, [_P, c_int64, _P, c_int64, _P, _P, c_float, _P, _P, _P]),
    "fx_ce_lin_grad_scale_bf16w": (c_int32, [_P, c_int64, _P, c_int64, _P, _P, c_float, _P, _P, _P]),
    "fx_ce_lin_grad_scale_inplace": (c_int32, [_P, c_int64, _P, c_int64, _P, _P, c_float, _P]),
    "fx_adamw_workspace": (c_int64, [ctypes.POINTER(fxTensorList), c_int32]),
    "fx_adamw_step": (c_int32, [ctypes.POINTER(fxAdamWState), ctypes.POINTER(fxTensorList),
                                c_int32, _P]),
    "fx_adamw_step_noalloc": (c_int32, [ctypes.POINTER(fxAdamWState), ctypes.POINTER(fxTensorList),
                                        c_int32, _P]),
    "fx_attn_fwd": (c_int32, [ctypes.POINTER(fxAttnArgs), _P]),
    "fx_attn_bwd": (c_int32, [ctypes.POINTER(fxAttnArgs), _P]),
    "fx_attn_decode_workspace": (c_int64, [c_int32, c_int32, c_int32, c_int32]),
    "fx_attn_decode": (c_int32, [ctypes.POINTER(fxAttnDecodeArgs), _P]),
    "fx_linear_fwd": (c_int32, [_P, c_int64, _P, c_int64, c_int64, _P, _P, _P, _P, _P,
                                c_int64, c_int64, c_int64, c_int32, _P]),
    "fx_linear_fwd_ex": (c_int32, [_P, _P]),
    "fx_gelu_bwd": (c_int32, [_P, _P, _P, c_int64, _P]),
    "fx_gelu_bwd_gate": (c_int32, [_P, _P, _P, c_int64, _P]),
    "fx_embedding_bwd_workspace": (c_int64, [c_int64, c_int64, c_int64]),
    "fx_embedding_bwd": (c_int32, [_P, c_int64, _P, c_int64, _P, c_int64, c_int64, _P, _P]),
    "fx_linear_dgrad": (c_int32, [_P, c_int64, _P, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64, _P]),
    "fx_linear_dgrad_gate": (c_int32, [_P, c_int64, _P, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64,
                                       _P]),
    "fx_linear_wgrad_workspace": (c_int64, [c_int64, c_int64, c_int64]),
    "fx_linear_wgrad": (c_int32, [_P, c_int64, _P, c_int64, _P, c_int64, _P, c_int64, c_int64, c_int64,
                                  _P]),
    "fx_lce_workspace": (c_int64, [c_int64, c_int64, c_int64]),
    "fx_lce_fwd": (c_int32, [_P, c_int64, _P, _P, c_int64, _P, _P, _P, c_int64, c_int64, c_int64, _P]),
    "fx_lce_grad": (c_int32, [_P, c_int64, _P, _P, c_int64, _P, _P, _P, c_int64, c_int64, c_int64, c_int64,
                              _P]),
}

_LIB = None
_LOCK = threading.Lock()


def lib():
    """Load libfxforge.so once (raises RuntimeError when it was not built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"libfxforge.so not found at {LIB_PATH}: build it first "
                    "(python __graft_entry__.py build, or "
                    "python radeon-igpu-forge_amd/csrc/build.py)")
            import torch  # noqa: F401  (torch's HIP runtime must be the one bound)
            h = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                f = getattr(h, name)
                f.restype = res
                f.argtypes = args
            v = h.fx_abi_version()
            if v != FX_ABI_VERSION:
                raise RuntimeError(f"libfxforge.so ABI {v} != expected {FX_ABI_VERSION}")
            _LIB = h
    return _LIB


_FUNCS = {}


def call(name, *args):
    """Call ``fx_<name>``; a non-zero return raises RuntimeError with the library message.
    The bound functions are looked up once (the GPT step makes ~400 calls)."""
    f = _FUNCS.get(name)
    if f is None:
        f = _FUNCS[name] = getattr(lib(), name)
    rc = f(*args)
    if rc != 0:
        msg = lib().fx_last_error().decode(errors="replace")
        if rc == FX_EINVAL:
            raise ValueError(msg)
        raise RuntimeError(f"{name} failed: hipError={rc} ({msg})")


def ptr(t):
    """Device pointer of a tensor as an int (None -> NULL); the argtypes convert it."""
    return None if t is None else t.data_ptr()


def stream_of(t):
    """The current torch stream on t's device, as a hipStream_t handle (an int): torch's
    raw-stream query, without building a Stream object (2.2 -> 0.1 us per call); the
    public Stream object where a torch build does not have that query."""
    import torch
    dev = t.device.index if t.device.index is not None else torch.cuda.current_device()
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is None:
        return torch.cuda.current_stream(dev).cuda_stream
    return raw(dev)
