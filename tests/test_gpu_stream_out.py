"""Plans that stream D: an unsplit plan on a wide tile whose operands fit in the 256 MiB
last-level cache but whose operands and D together do not writes D with nontemporal stores
(mxfp6_gemm_streams_output). The values are the same as with plain stores: every case here is
checked bit for bit against the direct kernel with the same scale grouping (a kernel with plain
stores and the same MFMA sequence), masked and unmasked, FP16, BF16 and FP32.
"""
import pytest
import torch

import checks
import mxfp6_amd as mx
from gpu_util import DevProblem, run_direct, run_routed, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K,out_type", [
    (2048, 102272, 1024, mx.OUT_F16),   # 256x256 wide tile, last tile column masked
    (1024, 102272, 2048, mx.OUT_BF16),
    (4096, 16384, 1024, mx.OUT_F32),
    (8192, 12288, 192, mx.OUT_F32),     # a single K-tile: the 256x256 tile's single-K-tile kernel
    (8192, 12288, 576, mx.OUT_F32),     # three K-tiles: its three-K-tile kernel
])
def test_routed_streaming_plan_equals_direct_kernel(M, N, K, out_type):
    # block scales spread so that FP32 bits depend on the K order (compared bit for bit)
    p = checks.spread_scales(mx.make_problem(M, N, K, seed=M + 11 * N + K), seed=K)
    tile = mx.choose_tile(M, N, p.Kp)
    assert mx.splitk_segments(M, N, p.Kp) == 1
    assert mx.streams_output(out_type, M, N, p.Kp, p.a_row_bytes), "plan does not stream D"
    dp = DevProblem(p, tile)
    say(f"  {M}x{N}x{K} {mx.OUT_NAMES[out_type]} tile {tile}: D streamed")
    D = run_routed(dp, out_type)
    R = run_direct(dp, out_type)
    assert (D.view("u4") == R.view("u4")).all(), "streamed D differs from the direct kernel"
    del dp
    torch.cuda.empty_cache()

