"""Build libfxforge.so, the gfx950 kernel library behind fxlm/fxgpu.

    python radeon-igpu-forge_amd/csrc/build.py [--report]

Every ``*.hip`` file in this directory is one translation unit, compiled in
parallel by hipcc for gfx950 only and linked into
``radeon-igpu-forge_amd/libfxforge.so`` (written to a temporary name and
renamed, so a concurrent loader never sees a half-written file).
``--report`` adds ``-Rpass-analysis=kernel-resource-usage`` so hipcc prints
VGPR/AGPR/SGPR, scratch (spill) and LDS use per kernel, then a one-line summary per
kernel; it exits with status 1 if any kernel uses scratch.

``resource_usage()`` compiles every source with that report into a temporary directory
(the library is left alone) and returns the figures per kernel; the CPU test suite fails
when any kernel of the library spills to scratch.  A spill is the failure the reference
gated on at run time (``ml/fxlm/kernel_regs.py:1-12``: a 1.3 KB/lane spill made its
attention backward 10-30x slower, ``ml/docs/HIZ_NOTLARI.md:228-245``); here it is caught
at build time, from the compiler's own report.
"""
import concurrent.futures
import os
import re
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
OUT = os.path.join(PKG, "libfxforge.so")
OBJ_DIR = os.path.join(HERE, "_build")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
    # keep MFMA accumulators in VGPRs: the softmax works on them directly, without
    # v_accvgpr_read/write copies each tile
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def _hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    for cand in (os.path.join(rocm, "bin", "hipcc"), shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set ROCM_PATH)")


def sources():
    return sorted(os.path.join(HERE, f) for f in os.listdir(HERE) if f.endswith(".hip"))


def _compile(hipcc, src, report, obj_dir=None):
    obj = os.path.join(obj_dir or OBJ_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc] + FLAGS + (["-Rpass-analysis=kernel-resource-usage"] if report else []) \
        + ["-c", src, "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    log = "\n".join(l for l in (p.stdout + p.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{log}")
    return obj, log


def build(verbose=False, report=False, jobs=None):
    """Compile every .hip source and link libfxforge.so; returns its path."""
    hipcc = _hipcc()
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    objs = []
    with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
        for obj, log in ex.map(lambda s: _compile(hipcc, s, report), srcs):
            objs.append(obj)
            if log.strip() and (verbose or report):
                print(log)
    tmp = OUT + f".tmp{os.getpid()}"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stdout}{p.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources")
    return OUT


_REMARK = re.compile(r"remark: +(.+?): (\S+) \[-Rpass-analysis=kernel-resource-usage\]")


def parse_resource_report(log):
    """{mangled kernel name: {field: value}} from hipcc's kernel-resource-usage remarks
    (fields as hipcc names them: "VGPRs", "AGPRs", "ScratchSize [bytes/lane]",
    "Occupancy [waves/SIMD]", "LDS Size [bytes/block]", ...; values as ints where they are)."""
    out, cur = {}, None
    for line in log.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        key, val = m.group(1).strip(), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
            continue
        if cur is not None:
            cur[key] = int(val) if val.lstrip("-").isdigit() else val
    return out


def resource_usage(jobs=None):
    """Compile every source with the resource report (objects in a temporary directory,
    the library untouched); returns {mangled kernel name: fields}."""
    hipcc = _hipcc()
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    usage = {}
    with tempfile.TemporaryDirectory() as tmp:
        with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
            for _, log in ex.map(lambda s: _compile(hipcc, s, True, tmp), srcs):
                usage.update(parse_resource_report(log))
    return usage


def _demangle(names):
    try:
        p = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True)
        out = p.stdout.splitlines()
        if len(out) == len(names):
            return out
    except OSError:
        pass
    return list(names)


if __name__ == "__main__":
    build(verbose="--report" not in sys.argv)
    if "--report" in sys.argv:
        usage = resource_usage()
        names = sorted(usage)
        bad = 0
        for n, d in zip(names, _demangle(names)):
            f = usage[n]
            scratch = f.get("ScratchSize [bytes/lane]", 0)
            bad += scratch > 0
            print(f"vgpr {f.get('VGPRs', '?'):>3} agpr {f.get('AGPRs', '?'):>3} scratch {scratch:>5} "
                  f"occupancy {f.get('Occupancy [waves/SIMD]', '?'):>2} lds {f.get('LDS Size [bytes/block]', '?'):>6}  {d}")
        print(f"{len(names)} kernels, {bad} with scratch")
        sys.exit(1 if bad else 0)
