"""fxgpu.hip_kernel: hiprtc + ctypes harness for raw HIP kernels on gfx950.

Same API as the reference loader (ml/fxgpu/hip_kernel.py:16-145):
``compile_kernel``, ``compile_module``, ``launch`` and the module attributes
``amdhip``, ``hiprtc``, ``_INC`` and ``_BIN``.  Differences:

* Linux/ROCm paths: the HIP runtime and hiprtc are the ones torch already
  loaded (``torch/lib``), the include directory is ``$ROCM_PATH/include``.
* The default architecture is gfx950 (MI355X); compiled code objects are cached
  per (source, name list, options) so a module is built once per process.
* The fxlm/fxgpu ops themselves do not JIT-compile: they call the prebuilt
  C-ABI library (``fxgpu.abi``).  This module stays for user kernels and for
  the loader smoke test.
"""
import ctypes
import glob
import hashlib
import os

import torch

DEFAULT_ARCH = "gfx950"


def _torch_lib_dir():
    return os.path.join(os.path.dirname(torch.__file__), "lib")


def _rocm_root():
    return os.environ.get("ROCM_PATH") or os.environ.get("HIP_PATH") or "/opt/rocm"


def _find_lib(pattern):
    """First match of pattern under torch/lib, then $ROCM_PATH/lib."""
    for d in (_torch_lib_dir(), os.path.join(_rocm_root(), "lib")):
        hits = sorted(h for h in glob.glob(os.path.join(d, pattern))
                      if "builtins" not in os.path.basename(h))
        if hits:
            return hits[0]
    raise RuntimeError(
        f"{pattern} not found under {_torch_lib_dir()} or {_rocm_root()}/lib")


_BIN = os.path.dirname(_find_lib("libamdhip64.so*"))
_INC = os.path.join(_rocm_root(), "include")
if not os.path.exists(os.path.join(_INC, "hip", "hip_runtime.h")):
    raise RuntimeError(f"HIP headers not found under {_INC} (set ROCM_PATH)")

amdhip = ctypes.CDLL(_find_lib("libamdhip64.so*"))
hiprtc = ctypes.CDLL(_find_lib("libhiprtc.so*"))

_vp = ctypes.c_void_p
hiprtc.hiprtcCreateProgram.argtypes = [ctypes.POINTER(_vp), ctypes.c_char_p, ctypes.c_char_p,
                                       ctypes.c_int, _vp, _vp]
hiprtc.hiprtcCompileProgram.argtypes = [_vp, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
hiprtc.hiprtcGetProgramLogSize.argtypes = [_vp, ctypes.POINTER(ctypes.c_size_t)]
hiprtc.hiprtcGetProgramLog.argtypes = [_vp, ctypes.c_char_p]
hiprtc.hiprtcGetCodeSize.argtypes = [_vp, ctypes.POINTER(ctypes.c_size_t)]
hiprtc.hiprtcGetCode.argtypes = [_vp, ctypes.c_char_p]
hiprtc.hiprtcDestroyProgram.argtypes = [ctypes.POINTER(_vp)]
amdhip.hipModuleLoadData.argtypes = [ctypes.POINTER(_vp), _vp]
amdhip.hipModuleGetFunction.argtypes = [ctypes.POINTER(_vp), _vp, ctypes.c_char_p]
amdhip.hipModuleLaunchKernel.argtypes = [_vp] + [ctypes.c_uint] * 6 + [
    ctypes.c_uint, _vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp)]

_CODE_CACHE = {}   # (sha1(src), opts) -> code object bytes
_MOD_CACHE = {}    # (sha1(src), opts, device) -> module handle


def _chk(err, what):
    if err != 0:
        raise RuntimeError(f"{what} failed: hipError={err}")


def _compile(src, arch, extra_opts):
    opts = [f"--offload-arch={arch}", f"-I{_INC}", "-O3"] + list(extra_opts or [])
    key = (hashlib.sha1(src.encode()).hexdigest(), tuple(opts))
    if key in _CODE_CACHE:
        return key, _CODE_CACHE[key]
    prog = _vp()
    _chk(hiprtc.hiprtcCreateProgram(ctypes.byref(prog), src.encode(), b"k.hip", 0, None, None),
         "hiprtcCreateProgram")
    arr = (ctypes.c_char_p * len(opts))(*[o.encode() for o in opts])
    err = hiprtc.hiprtcCompileProgram(prog, len(opts), arr)
    logsize = ctypes.c_size_t()
    hiprtc.hiprtcGetProgramLogSize(prog, ctypes.byref(logsize))
    if logsize.value > 1:
        log = ctypes.create_string_buffer(logsize.value)
        hiprtc.hiprtcGetProgramLog(prog, log)
        print("[hiprtc log]", log.value.decode(errors="replace"))
    if err != 0:
        hiprtc.hiprtcDestroyProgram(ctypes.byref(prog))
        raise RuntimeError(f"hiprtcCompileProgram failed: {err}")
    size = ctypes.c_size_t()
    _chk(hiprtc.hiprtcGetCodeSize(prog, ctypes.byref(size)), "GetCodeSize")
    code = ctypes.create_string_buffer(size.value)
    _chk(hiprtc.hiprtcGetCode(prog, code), "GetCode")
    hiprtc.hiprtcDestroyProgram(ctypes.byref(prog))
    _CODE_CACHE[key] = code.raw
    return key, code.raw


def _load(key, code):
    mkey = key + (torch.cuda.current_device(),)
    if mkey not in _MOD_CACHE:
        module = _vp()
        buf = ctypes.create_string_buffer(code, len(code))
        _chk(amdhip.hipModuleLoadData(ctypes.byref(module), buf), "hipModuleLoadData")
        _MOD_CACHE[mkey] = module
    return _MOD_CACHE[mkey]


def _get_func(module, name):
    func = _vp()
    _chk(amdhip.hipModuleGetFunction(ctypes.byref(func), module, name.encode()),
         f"hipModuleGetFunction({name})")
    return func


def compile_kernel(src: str, name: str, arch: str = DEFAULT_ARCH, extra_opts=None):
    """Compile src with hiprtc; return (module, function) ctypes handles."""
    key, code = _compile(src, arch, extra_opts)
    module = _load(key, code)
    return module, _get_func(module, name)


def compile_module(src: str, names, arch: str = DEFAULT_ARCH, extra_opts=None):
    """One hiprtc compile for several kernels: {name: function}."""
    key, code = _compile(src, arch, extra_opts)
    module = _load(key, code)
    return {name: _get_func(module, name) for name in names}


def launch(func, grid, block, args, shared=0, stream=None):
    """args: list of ctypes values, passed by reference as kernelParams."""
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    params = (_vp * len(args))()
    for i, a in enumerate(args):
        params[i] = ctypes.cast(ctypes.byref(a), _vp)
    _chk(amdhip.hipModuleLaunchKernel(
        func, grid[0], grid[1], grid[2], block[0], block[1], block[2],
        shared, _vp(stream), params, None), "hipModuleLaunchKernel")


FILL42_SRC = r"""
extern "C" __global__ void fill42(float* p, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 42.0f;
}
"""


def smoke(n=1000):
    """Loader smoke test: a hiprtc-compiled kernel writes 42 into a torch tensor."""
    x = torch.zeros(n, device="cuda")
    _mod, fn = compile_kernel(FILL42_SRC, "fill42")
    launch(fn, ((n + 255) // 256, 1, 1), (256, 1, 1),
           [ctypes.c_void_p(x.data_ptr()), ctypes.c_int(n)])
    torch.cuda.synchronize()
    if not bool((x == 42).all()):
        raise RuntimeError("fill42 failed")
    return x


if __name__ == "__main__":
    smoke()
    print("hiprtc harness OK: fill42 wrote 42s to a torch tensor")
