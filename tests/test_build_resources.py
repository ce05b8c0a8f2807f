"""The build refuses grouped-GEMM kernels that use scratch memory or spill
vector registers: their main loop counts its buffer->LDS loads by hand, out of
the compiler's sight, and assumes no compiler-generated memory traffic."""

import subprocess

import pytest

from placemoe_amd import build

REMARKS = """\
x.hip:10:1: remark: Function Name: _ZN12_GLOBAL__N_119grouped_gemm_kernelILi0EEEvv [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     VGPRs: 250 [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     ScratchSize [bytes/lane]: {scratch} [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     SGPRs Spill: 38 [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     VGPRs Spill: {spill} [-Rpass-analysis=kernel-resource-usage]
x.hip:10:1: remark:     LDS Size [bytes/block]: 157712 [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark: Function Name: _Z10other_kernv [-Rpass-analysis=kernel-resource-usage]
x.hip:20:1: remark:     ScratchSize [bytes/lane]: 64 [-Rpass-analysis=kernel-resource-usage]
"""


def test_parse_resource_usage():
    recs = build.parse_resource_usage(REMARKS.format(scratch=0, spill=0))
    assert [r["name"] for r in recs] == ["_ZN12_GLOBAL__N_119grouped_gemm_kernelILi0EEEvv", "_Z10other_kernv"]
    assert recs[0] == {"name": recs[0]["name"], "vgprs": 250, "agprs": 0, "scratch": 0, "sgpr_spill": 38,
                       "vgpr_spill": 0}
    assert recs[1]["scratch"] == 64


@pytest.mark.parametrize("scratch,spill", [(0, 0), (24, 0), (24, 6), (0, 2)])
def test_check_no_scratch(scratch, spill):
    recs = build.parse_resource_usage(REMARKS.format(scratch=scratch, spill=spill))
    pat = build.RESOURCE_CHECKED["grouped_gemm.hip"]
    if scratch == 0 and spill == 0:
        build.check_no_scratch(recs, pat, "x.hip")  # the other kernel's scratch is not checked
    else:
        with pytest.raises(RuntimeError, match="scratch"):
            build.check_no_scratch(recs, pat, "x.hip")


def test_unreadable_report_fails():
    with pytest.raises(RuntimeError, match="names no kernel"):
        build.check_no_scratch([], build.RESOURCE_CHECKED["grouped_gemm.hip"], "x.hip")


def _compile_remarks(src, tmp_path, extra=()):
    obj = tmp_path / "k.o"
    cmd = [build.hipcc(), *build.HIP_FLAGS, *extra, build.RESOURCE_FLAG, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    return build.parse_resource_usage(proc.stderr)


def test_planted_scratch_kernel_is_caught(tmp_path):
    """A kernel that indexes a private array at run time lives in scratch;
    the compiled report must say so and the check must refuse it."""
    src = tmp_path / "planted.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "__global__ void grouped_gemm_planted(float* o, const int* idx) {\n"
        "  float a[512];\n"
        "  for (int i = 0; i < 512; ++i) a[i] = o[i * 64 + threadIdx.x];\n"
        "  o[threadIdx.x] = a[idx[threadIdx.x] & 511];\n"
        "}\n"
    )
    recs = _compile_remarks(src, tmp_path)
    assert any(r["name"].endswith("grouped_gemm_plantedPfPKi") and r["scratch"] > 0 for r in recs), recs
    with pytest.raises(RuntimeError, match="scratch"):
        build.check_no_scratch(recs, build.RESOURCE_CHECKED["grouped_gemm.hip"], "planted.hip")


@pytest.mark.parametrize("extra", [(), ("-DPMX_TILE_TAB=2",)], ids=["shipped", "tiletab2"])
def test_shipped_gemm_kernels_have_no_scratch(extra, tmp_path):
    recs = _compile_remarks(build.CSRC / "grouped_gemm.hip", tmp_path, extra)
    gemm = [r for r in recs if "grouped_gemm" in r["name"]]
    assert sum("grouped_gemm_kernel" in r["name"] for r in gemm) >= 13, [r["name"] for r in recs]
    assert sum("grouped_gemm_w4_kernel" in r["name"] for r in gemm) >= 4, [r["name"] for r in recs]
    build.check_no_scratch(recs, build.RESOURCE_CHECKED["grouped_gemm.hip"], "grouped_gemm.hip")
    assert all(r["scratch"] == 0 and r["vgpr_spill"] == 0 for r in gemm)
