"""Register spill gate (CPU): no kernel of libfxforge.so may use scratch memory.

The reference learned this the hard way: a 1.3 KB/lane spill made its attention
backward 10-30x slower (`ml/docs/HIZ_NOTLARI.md:228-245`), after which it parsed
each compiled kernel's descriptor at run time (`ml/fxlm/kernel_regs.py:1-12,57-93`).
Here the same fact comes from the compiler: every source is compiled with
hipcc's kernel-resource-usage report and each kernel's ScratchSize must be 0.
Every template instantiation in the library is checked, not only the ones the
cfg shapes select, so a width or epilogue variant that spills fails here.
"""
import importlib.util
import os

import pytest

from conftest import ROOT

BUILD = os.path.join(ROOT, "radeon-igpu-forge_amd", "csrc", "build.py")
SCRATCH = "ScratchSize [bytes/lane]"


def _build_module():
    spec = importlib.util.spec_from_file_location("fx_build", BUILD)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def build():
    return _build_module()


def test_parser_reads_hipcc_remarks(build):
    # two kernels as hipcc reports them; the second spills
    log = "\n".join([
        "a.hip:3:1: remark: Function Name: _Z1fv [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:3:1: remark:     VGPRs: 40 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:3:1: remark:     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:3:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:3:1: remark:     Occupancy [waves/SIMD]: 8 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark: Function Name: _Z1gv [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: remark:     ScratchSize [bytes/lane]: 52 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:9:1: warning: something else",
    ])
    usage = build.parse_resource_report(log)
    assert set(usage) == {"_Z1fv", "_Z1gv"}
    assert usage["_Z1fv"][SCRATCH] == 0 and usage["_Z1fv"]["VGPRs"] == 40
    assert usage["_Z1gv"][SCRATCH] == 52


def test_no_kernel_uses_scratch(build):
    usage = build.resource_usage()
    # every source's kernels were reported (attention, CE, norm, AdamW, GEMMs, decode,
    # embedding: 240 instantiations when this test was written)
    assert len(usage) >= 200, sorted(usage)
    missing = [n for n, f in usage.items() if SCRATCH not in f]
    assert not missing, f"no scratch figure reported for {missing}"
    spilled = {n: f[SCRATCH] for n, f in usage.items() if f[SCRATCH] > 0}
    assert not spilled, f"kernels spill to scratch (bytes/lane): {spilled}"
    for fam in ("attn_fwd_kernel", "attn_bwd_dq_kernel", "attn_bwd_dkv_kernel", "ce_row_kernel",
                "rms_bwd_lds_kernel", "rms_bwd_wide_kernel", "adamw_update", "gemm_fast_kernel",
                "gemm_wgrad_fast_kernel", "gemm_dgrad_fast_kernel", "gemm_bias_act_kernel", "lce_stats_kernel",
                "attn_decode_kernel", "emb_part_kernel", "emb_final_kernel"):
        assert any(fam in n for n in usage), f"{fam} missing from the report"
