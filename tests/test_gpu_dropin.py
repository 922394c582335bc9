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

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "dropin_gemm")


@pytest.mark.parametrize("M,N,K,out_type", [
    (256, 256, 1024, 0),     # the small benchmark workload, FP32
    (512, 384, 960, 1),      # K-tail (kpad 1152)
    (384, 1280, 4160, 2),
    (96, 512, 8192, 1),      # M a multiple of 32 only: skinny tile, split K
    (2048, 1024, 16384, 1),  # narrow N, long K: split K with the workspace
])
def test_cpp_caller(M, N, K, out_type):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} missing: build it with __graft_entry__.build() or make -C tests/cpp")
    say(f"dropin_gemm {M} {N} {K} {out_type}")
    r = subprocess.run([BIN, str(M), str(N), str(K), str(out_type)], capture_output=True,
                       text=True, timeout=120)
    say("  " + r.stdout.strip())
    assert r.returncode == 0, r.stdout + r.stderr
