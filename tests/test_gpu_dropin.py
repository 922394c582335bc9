"""The reference's C++ API from a compiled caller (tests/cpp/dropin_gemm.cpp): host quantisation
and layouts from include/mxfp6/preprocess.hpp, then choose_tile / gemm_workspace_size / gemm from
include/mxfp6/gemm.hpp, linked against libmxfp6gemm.so only. The program checks D against an FP64
dot of the dequantised operands and exits non-zero on a mismatch.
"""
import os
import subprocess

import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp")
BINS = {"shared": os.path.join(HERE, "dropin_gemm"),
        "static": os.path.join(HERE, "dropin_gemm_static")}


@pytest.mark.parametrize("M,N,K,out_type,link,ws", [
    (256, 256, 1024, 0, "shared", "ref"),     # the small benchmark workload, FP32
    (512, 384, 960, 1, "shared", "ref"),      # K-tail (kpad 1152)
    (384, 1280, 4160, 2, "static", "ref"),
    (96, 512, 8192, 1, "shared", "ref"),      # M a multiple of 32 only: skinny tile, split K
    (2048, 1024, 16384, 1, "static", "ref"),  # narrow N, long K: split K with the workspace
    # N/32 = 260 is not a multiple of 3: the router must not pick a three-block-per-wave
    # N-masked tile, whose last scale group the header's tile_scale would not produce
    (512, 8320, 8192, 1, "shared", "ref"),
    (512, 8320, 8192, 1, "static", "preferred"),
    (2048, 8192, 4096, 1, "shared", "preferred"),  # a plan that repacks A into the workspace
    (2048, 8192, 4096, 2, "static", "ref"),        # the same plan on row-major A
    # N a multiple of 32 but not of 128 (last tile column masked): N/32 = 125 and 85 are odd, so
    # a grouping of two or four blocks would leave a partial scale group that the header's
    # tile_scale drops and the masked kernel reads
    (4096, 4000, 8192, 1, "shared", "ref"),
    (4096, 4000, 8192, 2, "static", "ref"),
    (256, 2720, 8192, 1, "shared", "ref"),
    (256, 2720, 8192, 0, "static", "preferred"),
])
def test_cpp_caller(M, N, K, out_type, link, ws):
    exe = BINS[link]
    if not os.path.exists(exe):
        pytest.fail(f"{exe} missing: build it with __graft_entry__.build() or make -C tests/cpp")
    say(f"dropin_gemm ({link}) {M} {N} {K} {out_type} {ws}")
    r = subprocess.run([exe, str(M), str(N), str(K), str(out_type), ws], capture_output=True,
                       text=True, timeout=120)
    say("  " + r.stdout.strip())
    assert r.returncode == 0, r.stdout + r.stderr
