"""The 32 x 32 tile (tiny_kernel.hpp): K split over a workgroup's four waves, operands loaded up
front, the partial blocks summed in LDS in segment order. Its output is bit for bit that of any
split plan with the same segments and the 1 x 1 scale grouping: the direct kernel's split on
multiples of 64, the 32 x 128 slab tile's split on ragged shapes; and it meets the FP64 oracle's
bar."""
import numpy as np
import pytest

import checks
import mxfp6_amd as mx
import gpu_util as g

pytestmark = pytest.mark.gpu

TINY = (32, 32, 1, 1)
T3 = {"dist_a": mx.DIST_STUDENT_T3, "dist_b": mx.DIST_STUDENT_T3}


@pytest.mark.parametrize("M,N", [(256, 256), (64, 512), (512, 128), (2048, 1024)])
@pytest.mark.parametrize("K,S", [(192, 1), (384, 2), (576, 3), (768, 4), (1152, 4), (1344, 2),
                                 (2112, 3), (3072, 4), (768, 1), (3072, 8), (4224, 6),
                                 (4224, 8), (8256, 11), (8256, 16), (12288, 16)])
def test_tiny_bitwise_equals_direct_split(M, N, K, S):
    """K-tile counts 1 to 64 in 1 to 16 segments of at most four K-tiles (segments of uneven
    length among them: 7 in 2, 11 in 3, 22 in 6, 43 in 11; past four segments a wave computes
    several in turn), on grids of 32 to 2048 blocks (an explicit plan runs the tile past the
    router's grid limit)."""
    seed = M + 3 * N + K + S
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=seed), seed=seed)
    dp = g.DevProblem(p, TINY)
    Dt = g.run_explicit(dp, mx.OUT_F32, splits=S)
    Dd = g.run_direct(dp, mx.OUT_F32, splits=S)
    assert np.array_equal(Dt.view(np.uint32), Dd.view(np.uint32))


@pytest.mark.parametrize("M,N,K,S", [(100, 200, 960, 3), (33, 97, 192, 1), (250, 31, 1344, 2),
                                     (1, 1, 3072, 4), (100, 200, 4224, 8), (1000, 300, 4224, 6),
                                     (1000, 300, 8256, 11), (1000, 300, 2112, 3)])
def test_tiny_ragged_equals_slab_split(M, N, K, S):
    """Ragged shapes (the last block row / column masked) against the 32 x 128 slab tile's split
    plan with the same segments (the same 1 x 1 grouping, the same sums); A loaded directly on the
    smallest grids and at S = 11 on 320 blocks, staged by eight waves (28 blocks, S = 8) or four
    (320 blocks, S = 6 and S = 3)."""
    seed = M * 7 + N + K
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=seed), seed=seed)
    dt = g.DevProblem(p, TINY)
    ds = g.DevProblem(p, (32, 128, 1, 1))
    Dt = g.run_explicit(dt, mx.OUT_F32, splits=S)
    Ds = g.run_explicit(ds, mx.OUT_F32, splits=S)
    assert np.array_equal(Dt.view(np.uint32), Ds.view(np.uint32))


@pytest.mark.parametrize("out_type", [mx.OUT_F32, mx.OUT_F16, mx.OUT_BF16])
def test_tiny_output_types_against_oracle(out_type):
    import oracle
    M, N, K = 256, 256, 1024  # the 256 x 256 x 1024 workload; kpad(1024) = 1152, 6 K-tiles
    p = mx.make_problem(M, N, K, seed=21)
    dp = g.DevProblem(p, TINY)
    R, ab = oracle.problem_f64(p)
    for S in (2, 4):
        D = g.run_explicit(dp, out_type, splits=S)
        checks.check(D, R, ab, out_type)
    # 16-bit outputs are the FP32 output rounded to nearest-even
    D32 = g.run_explicit(dp, mx.OUT_F32, splits=4)
    if out_type == mx.OUT_F16:
        want = D32.astype(np.float16).astype(np.float32)
        assert np.array_equal(g.run_explicit(dp, out_type, splits=4).view(np.uint32), want.view(np.uint32))
    elif out_type == mx.OUT_BF16:
        want = checks.round_bf16(D32)
        assert np.array_equal(g.run_explicit(dp, out_type, splits=4).view(np.uint32), want.view(np.uint32))
