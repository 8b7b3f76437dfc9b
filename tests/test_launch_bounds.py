"""Launch geometry of every kernel of the built liblq.so against its compiled metadata (CPU; reads the library's own
gfx950 code objects, tests/lq_codeobj.py).

  * the workgroup size each launch site uses (tests/lq_codeobj.LAUNCH_BLOCK, from leapquant_amd/csrc/*.hip) equals the
    kernel's compiled maximum (__launch_bounds__): a kernel is never launched with more threads than its registers
    were allocated for;
  * its static LDS fits a workgroup on a CU (160 KiB), and the workgroups per CU that LDS and registers allow are at
    least one, so every launch can make progress;
  * the kernels of the benchmark's hot path (the one-launch GDN decode, the four-wave GDN and KDA flushes, the KDA
    step) keep the residency they are tuned for (four workgroups per CU for the 256-thread ones, eight for the KDA
    step).
"""
import os
import shutil

import pytest

from tests import lq_codeobj as C

pytestmark = pytest.mark.skipif(not os.path.exists(C.LIB) or not os.path.exists(C.READELF) or not shutil.which("c++filt"),
                                reason="needs the built liblq.so, llvm-readelf and c++filt")


@pytest.fixture(scope="module")
def kernels():
    ks = C.kernels()
    assert ks, "no gfx950 code object found in liblq.so"
    return ks


def _per_cu(k):
    """Workgroups of kernel k that fit one CU at once (LDS and registers; wave64, four SIMDs)."""
    waves = k["block"] // 64
    regs = -(-(k["vgpr"] + k["agpr"]) // 8) * 8                     # allocation granule of 8
    waves_per_simd = min(8, C.VGPRS_PER_SIMD_LANE // max(regs, 1))
    by_regs = (4 * waves_per_simd) // waves
    by_lds = C.LDS_PER_CU // k["lds"] if k["lds"] else 64
    return min(by_regs, by_lds)


def test_every_kernel_has_a_known_launch_site(kernels):
    fams = {C.family(k["name"]) for k in kernels}
    assert fams <= set(C.LAUNCH_BLOCK), fams - set(C.LAUNCH_BLOCK)


def test_launch_block_equals_the_compiled_bound(kernels):
    bad = [(k["name"], k["block"], C.launch_block(k)) for k in kernels if C.launch_block(k) != k["block"]]
    assert not bad, bad


def test_lds_and_registers_fit(kernels):
    for k in kernels:
        assert k["lds"] <= C.LDS_PER_CU, (k["name"], k["lds"])
        assert k["vgpr"] + k["agpr"] <= C.VGPRS_PER_SIMD_LANE, k["name"]
        assert _per_cu(k) >= 1, k["name"]


def test_hot_kernels_keep_their_residency(kernels):
    def find(pattern):
        hit = [k for k in kernels if pattern in k["name"]]
        assert hit, pattern
        return hit
    for k in find("gdn_step_kernel<128, 128, 2, false, true, 4, false>") + find("flush4_kernel<128, 128, 1, false>"):
        assert _per_cu(k) >= 4 and k["scratch"] <= 8, (k["name"], _per_cu(k), k["scratch"])
    for k in find("flush4_kernel<128, 128, 1, true>"):        # KDA: a few loop-invariant values spilled per head
        assert _per_cu(k) >= 4 and k["scratch"] <= 64, (k["name"], _per_cu(k), k["scratch"])
    for k in find("kda_step_kernel"):
        assert _per_cu(k) >= 8 and k["scratch"] == 0, (k["name"], _per_cu(k), k["scratch"])
