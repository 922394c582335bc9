"""Kernel resources at build time (host only): no HIP kernel of the library uses scratch memory or
spills registers. The tile kernels' waits count their vector-memory operations exactly (static
issue order), and a spill would add uncounted ones. The remarks come from the library's own build
(hipcc -Rpass-analysis=kernel-resource-usage, one build/<unit>.res per HIP unit)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mxfp6-gemm_amd")
sys.path.insert(0, PKG)
import check_resources as cr  # noqa: E402

BUILD = os.path.join(PKG, "build")


def test_no_kernel_uses_scratch():
    files, kernels = cr.collect(BUILD)
    assert files, "no build/*.res: build the library (make -C mxfp6-gemm_amd) first"
    # every tile-kernel family is present, so a unit that stopped producing remarks is noticed
    fams = {cr.family(n) for n in kernels}
    assert {"wide_kernel", "slab_kernel", "direct_kernel", "reduce_splitk_kernel"} <= fams, fams
    assert sum(cr.family(n) == "wide_kernel" for n in kernels) >= 100
    bad = cr.violations(kernels)
    assert not bad, bad[:5]
    # the wide kernels hold their accumulators in AGPRs and stay within one wave per SIMD's file
    for n, r in kernels.items():
        assert r["vgpr"] <= 256 and r["agpr"] <= 256, (n, r)


def test_planted_spill_is_caught(tmp_path):
    """A remarks file with a 4-byte scratch kernel and one with a VGPR spill both fail the check;
    a clean one passes."""
    def remarks(name, scratch, vspill):
        f = "csrc/hip/x.hpp:1:1: remark: "
        tail = " [-Rpass-analysis=kernel-resource-usage]\n"
        return (f + f"Function Name: {name}" + tail + f + "    VGPRs: 200" + tail +
                f + "    AGPRs: 256" + tail + f + f"    ScratchSize [bytes/lane]: {scratch}" + tail +
                f + "    Dynamic Stack: False" + tail + f + "    SGPRs Spill: 0" + tail +
                f + f"    VGPRs Spill: {vspill}" + tail)
    for i, (s, v, want_bad) in enumerate(((0, 0, False), (4, 0, True), (0, 3, True))):
        d = tmp_path / str(i)
        d.mkdir()
        (d / "u.res").write_text(remarks(f"_ZN9mxfp6_dev11wide_kernelILi{i}E", s, v))
        files, kernels = cr.collect(str(d))
        assert len(kernels) == 1
        assert bool(cr.violations(kernels)) == want_bad
        assert (cr.main(["x", str(d)]) == 1) == want_bad
