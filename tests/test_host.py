"""Host-side logic of the Python surface (CPU only): argument validation raises
the reference's error classes before any kernel call, and the small pure-Python
helpers (layout, chunking) follow the reference."""
import pytest
import torch
from torch import nn

from oracle import adamw as oadam


def test_norm_validation():
    from fxlm.norm import rms_norm
    x = torch.randn(4, 16).bfloat16()
    w = torch.ones(16).bfloat16()
    with pytest.raises(TypeError):
        rms_norm(x.float(), w)          # dtype
    with pytest.raises(TypeError):
        rms_norm(x, w)                  # device (cpu)


def test_ce_validation():
    from fxlm.cross_entropy import _check_lin, _check_logits
    lg = torch.randn(4, 8).bfloat16()
    tg = torch.zeros(4, dtype=torch.int64)
    with pytest.raises(TypeError):
        _check_logits(lg.half(), tg)
    with pytest.raises(TypeError):
        _check_logits(lg, tg)           # cpu tensors
    with pytest.raises(TypeError):
        _check_lin(lg, lg, tg)


def test_attention_validation():
    from fxlm.attention import _check_qkv
    q = torch.randn(1, 8, 2, 32).bfloat16()
    with pytest.raises(ValueError):
        _check_qkv(q, q, q)             # head_dim 32
    q = torch.randn(1, 8, 2, 64).bfloat16()
    with pytest.raises(ValueError):
        _check_qkv(q, q[:, :4], q)      # shape mismatch
    with pytest.raises(TypeError):
        _check_qkv(q, q, q)             # cpu tensors
    with pytest.raises(TypeError):
        _check_qkv(q.half(), q.half(), q.half())


def test_flat_adamw_requires_cuda_fp32():
    from fxlm.optim import FlatAdamW, _align8
    with pytest.raises(TypeError):
        FlatAdamW(nn.Linear(4, 4))      # cpu parameters
    with pytest.raises(ValueError):
        FlatAdamW(nn.Module())          # no parameters
    for n in (0, 1, 7, 8, 9, 37, 2048):
        assert _align8(n) == oadam.align8(n) and _align8(n) % 8 == 0 and _align8(n) >= n


def test_linear_ce_auto_chunk():
    from fxlm.cross_entropy import _auto_chunk
    c = _auto_chunk(768, 50304)
    assert c % 256 == 0 and c * 50304 * 2 <= 2 << 30 and c >= 16384   # cfg5 runs as one chunk
    assert _auto_chunk(64, 10 ** 9) == 256


def test_hip_kernel_surface():
    from fxgpu import hip_kernel
    for name in ("compile_kernel", "compile_module", "launch", "amdhip", "hiprtc", "_INC", "_BIN"):
        assert hasattr(hip_kernel, name)


def test_hiprtc_compile_error_raises_with_log(capsys):
    # ml/fxgpu/hip_kernel.py:59-69: the compiler log is printed with a "[hiprtc log]"
    # prefix and a failed compile raises RuntimeError before anything is loaded
    from fxgpu import hip_kernel
    src = 'extern "C" __global__ void bad(float* p) { p[0] = undeclared_name; }'
    with pytest.raises(RuntimeError, match="hiprtcCompileProgram failed"):
        hip_kernel.compile_module(src, ["bad"])
    out = capsys.readouterr().out
    assert "[hiprtc log]" in out and "undeclared_name" in out


def test_lazy_exports():
    import fxgpu
    import fxlm
    for name in fxlm.__all__:
        assert getattr(fxlm, name) is not None
    for name in ("FusedGatherLinear", "fused_gather_linear", "setup_env", "require_gpu"):
        assert getattr(fxgpu, name) is not None

