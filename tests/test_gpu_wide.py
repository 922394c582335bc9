"""The wide tiles (four waves side by side, B streamed straight into registers, A staged in LDS one
K-tile per row): 128 x 512, 128 x 384, 128 x 256 and 256 x 256. Each is bit for bit equal to the
direct kernel (same MFMAs, same K order) with row-major A (staged as copied, and staged in
swizzled 12-byte units: explicit layout 3) and repacked A, unsplit and split on both XCD maps;
equal to the 256x256 slab kernel on ragged (masked) shapes (the same MFMA sequence per output
block, whatever the scale grouping of the layouts); all output types against the FP64 oracle."""
import numpy as np
import pytest

import checks
import mxfp6_amd as mx
import gpu_util as g

# Operands of the bit-for-bit comparisons between two computations: Student-t(3) codes with every
# block scale lowered by a random exponent in [0, 12] (checks.spread_scales), so that FP32 sums of
# the scaled products round and a different K order changes bits
# (with the generator's own scales the partial sums stay exact; test_gpu_gemm.py
# test_bitwise_operands_see_the_k_order).
T3 = {"dist_a": mx.DIST_STUDENT_T3, "dist_b": mx.DIST_STUDENT_T3}

pytestmark = pytest.mark.gpu

WIDE_TILES = [(128, 512, 4, 4), (128, 384, 4, 3), (128, 256, 4, 2), (256, 256, 4, 2)]


@pytest.mark.parametrize("WIDE", WIDE_TILES)
@pytest.mark.parametrize("tm,tn,K", [(2, 2, 2112), (1, 1, 192), (1, 4, 4224), (3, 3, 3456),
                                     (2, 1, 384), (1, 2, 576)])
@pytest.mark.parametrize("a_layout", [0, 1, 3])
def test_wide_bitwise_equals_direct(WIDE, tm, tn, K, a_layout):
    """tm x tn tiles (M, N multiples of 256 and of the tile); the K-tile counts 11, 1, 22, 18, 2
    and 3: the K loop runs passes of six K-tiles and leaves after any of them (11 and 22 end
    mid-pass, 18 on a pass boundary); with 2 and 3 K-tiles most prefetches are clamped to the last
    K-tile."""
    M, N = 256 * tm, WIDE[1] * tn
    seed = M + N + K + a_layout
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=seed), seed=seed)
    dp = g.DevProblem(p, WIDE)
    Dw = g.run_explicit(dp, mx.OUT_F32, a_layout=a_layout)
    Dd = g.run_direct(dp, mx.OUT_F32)
    assert np.array_equal(Dw.view(np.uint32), Dd.view(np.uint32))


@pytest.mark.parametrize("WIDE", WIDE_TILES)
@pytest.mark.parametrize("S", [2, 3, 8])
@pytest.mark.parametrize("M,tn", [(512, 2), (2048, 2)])
def test_wide_split_bitwise_equals_direct_split(WIDE, M, tn, S):
    """Split grids: at most 128 tiles hand each XCD whole K segments, more use the grid order;
    every partial lands in its segment's slot either way."""
    N = WIDE[1] * tn
    K = 4224  # 22 K-tiles: uneven segments
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=S * 7 + M), seed=S * 7 + M)
    dp = g.DevProblem(p, WIDE)
    for a_layout in (0, 1, 3):
        Dw = g.run_explicit(dp, mx.OUT_F32, splits=S, a_layout=a_layout)
        Dd = g.run_direct(dp, mx.OUT_F32, splits=S)
        assert np.array_equal(Dw.view(np.uint32), Dd.view(np.uint32)), a_layout


@pytest.mark.parametrize("WIDE", WIDE_TILES)
@pytest.mark.parametrize("S,K", [(1, 192), (3, 576), (6, 1152), (1, 384), (3, 1152), (2, 1152),
                                 (3, 1728)])
def test_wide_single_k_tile_segments(WIDE, S, K):
    """Every K segment one, two or three K-tiles (the short path, or for 128 x 512 and 256 x 256
    their short-path instantiations, three K-tiles on 256 x 256 only; the swizzled staging has no
    short path of its own and runs its main loop): bit for bit the direct kernel, rows (both
    stagings) and repacked A."""
    M, N = 512, WIDE[1] * 2
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=S * 11 + K), seed=S * 11 + K)
    dp = g.DevProblem(p, WIDE)
    for a_layout in (0, 1, 3):
        Dw = g.run_explicit(dp, mx.OUT_F32, splits=S, a_layout=a_layout)
        Dd = g.run_direct(dp, mx.OUT_F32, splits=S)
        assert np.array_equal(Dw.view(np.uint32), Dd.view(np.uint32)), a_layout


@pytest.mark.parametrize("WIDE", WIDE_TILES)
@pytest.mark.parametrize("K", [192, 384, 576])
def test_wide_short_path_lowp_outputs(WIDE, K):
    """Unsplit K of one to three K-tiles (the short path, or the short-path instantiations of
    128 x 512 (one or two) and 256 x 256 (one to three)) with 16-bit outputs: FP32 equals the direct kernel bit for bit, and
    FP16 / BF16 equal that FP32 rounded to nearest-even on the host, rows (both stagings) and
    repacked A."""
    M, N = 512, WIDE[1] * 2
    p = mx.make_problem(M, N, K, dist_a=mx.DIST_STUDENT_T3, dist_b=mx.DIST_STUDENT_T3,
                        seed=K * 5 + WIDE[1])
    dp = g.DevProblem(p, WIDE)
    Dd = g.run_direct(dp, mx.OUT_F32)
    for a_layout in (0, 1, 3):
        D32 = g.run_explicit(dp, mx.OUT_F32, a_layout=a_layout)
        assert np.array_equal(D32.view(np.uint32), Dd.view(np.uint32)), a_layout
        D16 = g.run_explicit(dp, mx.OUT_F16, a_layout=a_layout)
        want16 = D32.astype(np.float16).astype(np.float32)
        assert np.array_equal(D16.view(np.uint32), want16.view(np.uint32)), a_layout
        Db16 = g.run_explicit(dp, mx.OUT_BF16, a_layout=a_layout)
        assert np.array_equal(Db16.view(np.uint32), checks.round_bf16(D32).view(np.uint32)), a_layout


@pytest.mark.parametrize("WIDE", WIDE_TILES)
@pytest.mark.parametrize("M,N,K", [(300, 700, 960), (97, 1000, 2112), (129, 513, 384),
                                   (1, 33, 192)])
def test_wide_masked_equals_slab_masked(WIDE, M, N, K):
    """Ragged shapes run the wide tile masked; its FP32 output equals the masked 256x256 slab
    kernel's (same scale grouping, same K order) bit for bit, and both meet the oracle bar."""
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=M * 7 + N), seed=M * 7 + N)
    dw = g.DevProblem(p, WIDE)
    ds = g.DevProblem(p, (256, 256, 4, 4))
    for a_layout, S in ((0, 1), (1, 1), (0, 3)):
        if S > p.Kp // 192:
            continue
        Dw = g.run_explicit(dw, mx.OUT_F32, splits=S, a_layout=a_layout)
        Ds = g.run_explicit(ds, mx.OUT_F32, splits=S, a_layout=a_layout)
        assert np.array_equal(Dw.view(np.uint32), Ds.view(np.uint32)), (a_layout, S)
    import oracle
    R, ab = oracle.problem_f64(p)
    checks.check(Dw, R, ab, mx.OUT_F32)


@pytest.mark.parametrize("WIDE", WIDE_TILES)
@pytest.mark.parametrize("out_type", [0, 1, 2])
def test_wide_output_types_against_oracle(WIDE, out_type):
    import oracle
    M, N, K = 256, 1024, 960  # K-tail: kpad(960) = 1152
    p = mx.make_problem(M, N, K, **T3, seed=13)
    dp = g.DevProblem(p, WIDE)
    R, ab = oracle.problem_f64(p)
    for a_layout in (0, 1):
        D = g.run_explicit(dp, out_type, a_layout=a_layout)
        checks.check(D, R, ab, out_type)
