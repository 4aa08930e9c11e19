"""CPU guards against the two GPU-fault patterns this library has met: an
inline-asm vector memory instruction issued without the wait states the
compiler cannot insert for it, and an asm load whose destination registers
end up in scratch memory.  The checks run over the committed sources and the
resource-usage remarks the build leaves next to each object
(``kempnerforge_amd/csrc/Makefile``), and each check is shown to fire on a
deliberately broken input."""

from __future__ import annotations

import glob
import os
import subprocess

import pytest

import asm_guard as g


def test_vmem_asm_opens_with_wait_states():
    bad = [v for name, text in g.sources().items() for v in g.check_asm(text, name)]
    assert not bad, "\n".join(bad)


def test_every_vmem_asm_is_found():
    # the direct-to-LDS loads exist, so the scan sees them (not vacuously green)
    found = [(name, line) for name, text in g.sources().items()
             for line, tpl, _ in g.asm_statements(text) if "global_load_lds" in tpl]
    assert len(found) >= 3, found


def test_checker_flags_missing_wait_states():
    text = '__device__ void f(uint32_t o, const void* b) {\n' \
           '  asm volatile("global_load_lds_dwordx4 %0, %1" : : "v"(o), "s"(b) : "memory");\n}\n'
    bad = g.check_asm(text)
    assert len(bad) == 1 and "KF_VMEM_ASM_NOPS" in bad[0] and ":2:" in bad[0]


def test_checker_flags_asm_load_into_registers():
    text = ('__device__ void f(u32x4* r, uint32_t o, const void* b) {\n'
            '  /* comment with asm("x") in it */\n'
            '  asm volatile(KF_VMEM_ASM_NOPS "global_load_dwordx4 %0, %1, %2"\n'
            '               : "=v"(r[1]) : "v"(o), "s"(b) : "memory");\n}\n')
    bad = g.check_asm(text)
    assert len(bad) == 1 and "register outputs" in bad[0]
    # the same load with the nops and no outputs passes; non-memory asm is ignored
    assert not g.check_asm('asm volatile(KF_VMEM_ASM_NOPS "global_load_lds_dword %0, %1" '
                           ': : "v"(o), "s"(b), "{m0}"(l) : "memory");')
    assert not g.check_asm('asm volatile("s_waitcnt vmcnt(0)" ::: "memory");')
    assert not g.check_asm('asm volatile("" : "+v"(x));')


def test_reachability_follows_calls():
    text = ('__device__ __forceinline__ void dma(uint32_t o, const void* b) {\n'
            '  asm volatile(KF_VMEM_ASM_NOPS "global_load_lds_dword %0, %1" : : "v"(o), "s"(b));\n'
            '}\n'
            'template <int N> __device__ void stage(int x) { dma(x, nullptr); }\n'
            'template <int D>\n__global__ __launch_bounds__(256, 2) void uses_kernel(int x) {\n'
            '  auto l = [&](int y) { stage<D>(y); };\n  l(x);\n}\n'
            '__global__ void plain_kernel(int* p) { p[0] = 1; }\n')
    reach = g.dma_functions({"t.hip": text})
    assert {"dma", "stage", "uses_kernel"} <= reach and "plain_kernel" not in reach
    assert g.kernels({"t.hip": text}) == {"uses_kernel", "plain_kernel"}


REMARKS_BAD = """\
kf_x.hip:10:1: remark: Function Name: _ZN2kf12_GLOBAL__N_111uses_kernelILi128EEEvi [-Rpass-analysis=kernel-resource-usage]
   10 | void uses_kernel(int x) {
      | ^
kf_x.hip:10:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
kf_x.hip:10:1: remark:     ScratchSize [bytes/lane]: 16 [-Rpass-analysis=kernel-resource-usage]
kf_x.hip:10:1: remark:     SGPRs Spill: 2 [-Rpass-analysis=kernel-resource-usage]
kf_x.hip:10:1: remark:     VGPRs Spill: 3 [-Rpass-analysis=kernel-resource-usage]
kf_x.hip:20:1: remark: Function Name: _ZN2kf12_GLOBAL__N_112plain_kernelEPi [-Rpass-analysis=kernel-resource-usage]
kf_x.hip:20:1: remark:     ScratchSize [bytes/lane]: 64 [-Rpass-analysis=kernel-resource-usage]
"""


def test_checker_flags_scratch_in_dma_kernel():
    r = g.parse_remarks(REMARKS_BAD)
    assert r["_ZN2kf12_GLOBAL__N_111uses_kernelILi128EEEvi"]["ScratchSize"] == 16
    bad = g.check_scratch(r, {"uses_kernel"})
    assert len(bad) == 1 and bad[0].startswith("uses_kernel")  # plain_kernel has no asm
    assert not g.check_scratch(g.parse_remarks(REMARKS_BAD.replace(": 16 [", ": 0 [")
                                               .replace("Spill: 3", "Spill: 0")),
                               {"uses_kernel"})


def _remarks_files():
    files = sorted(glob.glob(os.path.join(g.OBJ, "*.remarks")))
    want = {os.path.splitext(n)[0] for n in os.listdir(g.CSRC) if n.endswith(".hip")}
    if {os.path.splitext(os.path.basename(f))[0] for f in files} >= want:
        return files
    # not built here yet: compile the objects (the remarks come with them)
    subprocess.run(["make", "-C", g.CSRC, "-j", str(min(8, os.cpu_count() or 1)), "remarks"],
                   check=True, stdout=subprocess.DEVNULL)
    return sorted(glob.glob(os.path.join(g.OBJ, "*.remarks")))


def test_dma_kernels_use_no_scratch():
    texts = g.sources()
    dma = g.dma_functions(texts) & g.kernels(texts)
    assert {"bwd_dkdv_kernel", "bwd_dq_ds_kernel", "fwd32_kernel"} <= dma
    files = _remarks_files()
    if not files:
        pytest.skip("no resource-usage remarks (library not built)")
    seen, bad = set(), []
    for f in files:
        r = g.parse_remarks(open(f).read())
        seen |= {g.source_name(m, dma) for m in r} - {None}
        bad += g.check_scratch(r, dma)
    assert seen == dma, f"kernels without remarks: {sorted(dma - seen)}"
    assert not bad, "\n".join(bad)
