"""GPU parity of the MXFP6 GEMM against the FP64 oracle (tolerances in tests/checks.py).

Inputs: the seeded PCG32 workload generator with the OCP MX scale rule; A compact
(A_row_bytes = packed(K), a_compact_end_pad) unless stated; outputs poisoned with 0x5A so an
unwritten element fails. Every launch goes through the library's C ABI.
"""
import numpy as np
import pytest

import checks
import mxfp6_amd as mx

pytestmark = pytest.mark.gpu

# Operands of the bit-for-bit comparisons between two computations: Student-t(3) codes with every
# block scale lowered by a random exponent in [0, 12] (checks.spread_scales), so that FP32 sums of
# the scaled products round and a different K order changes bits
# (with the generator's own scales the partial sums stay exact;
# test_bitwise_operands_see_the_k_order).
T3 = {"dist_a": mx.DIST_STUDENT_T3, "dist_b": mx.DIST_STUDENT_T3}


@pytest.fixture(scope="module")
def g():
    import gpu_util
    return gpu_util


def _oracle(orc, p, rows=None):
    return orc.problem_f64(p, rows=rows)


# ---- the small benchmark workload, routed ------------------------------------------------------

def test_small_config_fp32(g, orc):
    """256x256x1024, FP32 out, N(0,1): the CPU-runnable benchmark workload, full check."""
    p = mx.make_problem(256, 256, 1024)
    dp = g.DevProblem(p, mx.choose_tile(256, 256, p.Kp))
    D = g.run_routed(dp, mx.OUT_F32)
    R, ab = _oracle(orc, p)
    rel = checks.check_f32(D, R, ab)
    g.say(f"    normwise max|D-R|/max|R| = {rel:.3e}")


@pytest.mark.parametrize("out_type", [0, 1, 2])
@pytest.mark.parametrize("M,N,K", [(128, 128, 192), (256, 384, 768), (384, 256, 960),
                                   (512, 768, 1152),
                                   # 128x128x4224 and 256x256x4096: 22 K-tiles in 8
                                   # segments of the 32x32 tile, two per wave in turn
                                   (128, 128, 4224), (512, 512, 2048), (256, 256, 4096)])
def test_routed_small_shapes(g, orc, out_type, M, N, K):
    p = mx.make_problem(M, N, K, seed=M * 3 + N * 7 + K)
    dp = g.DevProblem(p, mx.choose_tile(M, N, p.Kp))
    D = g.run_routed(dp, out_type)
    R, ab = _oracle(orc, p)
    checks.check(D, R, ab, out_type)


@pytest.mark.parametrize("tile", [(128, 128, 2, 2), (128, 256, 2, 4), (128, 384, 4, 3),
                                  (256, 256, 4, 4), (256, 256, 2, 4),
                                  (256, 192, 4, 3), (128, 512, 4, 4)])
@pytest.mark.parametrize("out_type", [0, 1, 2])
def test_forced_tiles(g, orc, tile, out_type):
    M, N, K = 256, 1536, 960  # every tile divides 256 x 1536; K-tail: kpad(960) = 1152
    p = mx.make_problem(M, N, K, **T3, seed=11)
    D = g.run_forced(g.DevProblem(p, tile), out_type)
    R, ab = _oracle(orc, p)
    checks.check(D, R, ab, out_type)


def test_bitwise_operands_see_the_k_order(g):
    """The bit-for-bit tests compare two computations of the same sums; they catch a kernel that
    adds the right terms in another order only if the operands make FP32 rounding depend on the
    order. The direct kernel, unsplit against split in three (the same products, summed per
    segment and then across segments), shows that the spread scales do: at least 10% of the
    outputs differ in their bits. With the generator's own scales (N(0,1) and Student-t(3) codes)
    no output differs: every partial sum is exact."""
    M, N, K = 256, 256, 4224
    diff = {}
    for name, dist, spread in (("spread", mx.DIST_STUDENT_T3, True),
                               ("t3", mx.DIST_STUDENT_T3, False),
                               ("normal", mx.DIST_NORMAL, False)):
        p = mx.make_problem(M, N, K, dist_a=dist, dist_b=dist, seed=97)
        if spread:
            checks.spread_scales(p, seed=97)
        dp = g.DevProblem(p, (128, 128, 2, 2))
        D1 = g.run_direct(dp, mx.OUT_F32)
        D3 = g.run_direct(dp, mx.OUT_F32, splits=3)
        assert np.all(np.isfinite(D1)) and np.all(np.isfinite(D3))
        diff[name] = int(np.count_nonzero(D1.view(np.uint32) != D3.view(np.uint32)))
    assert diff["spread"] >= M * N // 10, diff
    assert diff["t3"] == 0 and diff["normal"] == 0, diff


@pytest.mark.parametrize("tile", [(128, 128, 2, 2), (128, 256, 2, 4), (128, 384, 4, 3),
                                  (256, 256, 4, 4), (256, 256, 2, 4),
                                  (256, 192, 4, 3)])
def test_pipelined_kernel_bitwise_equals_direct(g, tile):
    """Both kernels add the same MFMA results in the same K order, so FP32 outputs are equal
    bit for bit (covers every wave block, slab and stage of the pipelined kernel)."""
    M, N, K = 512, 768, 2112  # 11 K-tiles: odd count, both ring stages, peeled tail
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=71), seed=71)
    dp = g.DevProblem(p, tile)
    Dt = g.run_forced(dp, mx.OUT_F32)
    Dd = g.run_direct(dp, mx.OUT_F32)
    assert np.array_equal(Dt.view(np.uint32), Dd.view(np.uint32))


def test_pipelined_split_bitwise_equals_direct_split(g):
    # a shape routed to a split on a pipelined tile (not the 32 x 32 one, tested in test_gpu_tiny)
    M, N, K = g.routed_shape([(512, 512, 4224), (768, 768, 3072), (1024, 512, 4224)],
                             lambda t, S, rp: S > 1 and t != (32, 32, 1, 1))
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=81), seed=81)
    t = mx.choose_tile(M, N, p.Kp)
    S = mx.splitk_segments(M, N, p.Kp)
    dp = g.DevProblem(p, t)
    Dr = g.run_routed(dp, mx.OUT_F32)
    Dd = g.run_direct(dp, mx.OUT_F32, splits=S)
    assert np.array_equal(Dr.view(np.uint32), Dd.view(np.uint32))


@pytest.mark.parametrize("tile", [(128, 256, 2, 4), (128, 384, 4, 3), (256, 256, 4, 4),
                                  (256, 256, 2, 4), (256, 192, 4, 3)])
@pytest.mark.parametrize("S,a_layout", [(3, 0), (8, 1)])
def test_segment_per_xcd_split_bitwise_equals_direct_split(g, tile, S, a_layout):
    """Split grids of at most 128 tiles of at least 128 x 256 hand each XCD whole K segments
    (the workgroup -> (tile, segment) map differs from the grid's); every partial must still land
    in its segment's slot, so the result equals the direct kernel's split bit for bit."""
    M, N, K = 512, 768, 4224  # 22 K-tiles: uneven segments for S = 3 and 8
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=83), seed=83)
    dp = g.DevProblem(p, tile)
    Dr = g.run_explicit(dp, mx.OUT_F32, splits=S, a_layout=a_layout)
    Dd = g.run_direct(dp, mx.OUT_F32, splits=S)
    assert np.array_equal(Dr.view(np.uint32), Dd.view(np.uint32))


# ---- M not a multiple of 128: the skinny tiles ------------------------------------------------

SKINNY = [(32, 128, 1, 1), (32, 256, 1, 2), (64, 128, 2, 1), (64, 256, 2, 2)]


@pytest.mark.parametrize("out_type", [0, 1, 2])
@pytest.mark.parametrize("M,N,K", [(32, 128, 192), (64, 256, 1024), (96, 384, 960),
                                   (160, 256, 2048), (224, 512, 4096), (32, 4096, 8192)])
def test_routed_skinny_m(g, orc, out_type, M, N, K):
    """M not a multiple of 128 routes to the 32- and 64-row tiles (the 32 x 32 one among them on
    grids of at most two 32 x 32 blocks per CU with up to 28-64 K-tiles, by the grid); the routed
    output meets the oracle's bar."""
    p = mx.make_problem(M, N, K, seed=M * 5 + N + K)
    t = mx.choose_tile(M, N, p.Kp)
    assert tuple(t) in SKINNY + [(32, 32, 1, 1)]
    D = g.run_routed(g.DevProblem(p, t), out_type)
    R, ab = _oracle(orc, p)
    checks.check(D, R, ab, out_type)


@pytest.mark.parametrize("tile", SKINNY)
def test_skinny_tiles_bitwise_equal_direct(g, tile):
    """Every skinny tile, row-major and repacked A, unsplit and split: the same MFMAs in the same
    K order as the direct kernel, so FP32 outputs are equal bit for bit."""
    M, N, K = 192, 512, 2112  # 11 K-tiles: odd count, ring wrap, peeled tail
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=91), seed=91)
    dp = g.DevProblem(p, tile)
    Dd = g.run_direct(dp, mx.OUT_F32)
    for a_layout in (0, 1):
        Dt = g.run_explicit(dp, mx.OUT_F32, a_layout=a_layout)
        assert np.array_equal(Dt.view(np.uint32), Dd.view(np.uint32)), a_layout
    Dds = g.run_direct(dp, mx.OUT_F32, splits=5)
    Dts = g.run_explicit(dp, mx.OUT_F32, splits=5, a_layout=1)
    assert np.array_equal(Dts.view(np.uint32), Dds.view(np.uint32))


# ---- A repacked into the preshuffled layout ------------------------------------------------------

@pytest.mark.parametrize("tile", [(128, 128, 2, 2), (128, 256, 2, 4), (128, 384, 4, 3),
                                  (256, 256, 4, 4), (256, 256, 2, 4),
                                  (256, 192, 4, 3)])
def test_repacked_a_bitwise_equals_direct(g, tile):
    """The kernel reading the repacked A multiplies the same operands in the same order."""
    M, N, K = 512, 768, 2112
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=72), seed=72)
    dp = g.DevProblem(p, tile)
    Dr = g.run_explicit(dp, mx.OUT_F32, a_layout=1)
    Dd = g.run_direct(dp, mx.OUT_F32)
    assert np.array_equal(Dr.view(np.uint32), Dd.view(np.uint32))


def test_repacked_a_split_bitwise_equals_direct_split(g):
    M, N, K = 512, 512, 3072
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=82), seed=82)
    dp = g.DevProblem(p, (128, 128, 2, 2))
    Dr = g.run_explicit(dp, mx.OUT_F32, splits=3, a_layout=1)
    Dd = g.run_direct(dp, mx.OUT_F32, splits=3)
    assert np.array_equal(Dr.view(np.uint32), Dd.view(np.uint32))


@pytest.mark.parametrize("compact", [True, False])
def test_device_preshuffle_matches_host_preshuffle(g, orc, compact):
    """The on-device row preshuffle (the A repack) gives the host preshuffle_B's bytes, for
    compact rows (over-read into the next row / end pad, as the kernels read them) and padded."""
    import torch
    M, K = 256, 960
    p = mx.make_problem(M, 128, K, seed=5, compact=compact)
    src = torch.from_numpy(p.a_packed).cuda()
    dst = torch.full((M * p.Kp // 4 * 3,), 0x5A, dtype=torch.uint8, device="cuda")
    rc = mx.preshuffle_rows(src.data_ptr(), p.a_row_bytes, M, p.Kp, dst.data_ptr())
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    host = orc.preshuffle_b(p.a_packed, M, p.Kp, p.a_row_bytes)
    assert np.array_equal(dst.cpu().numpy(), host)


def test_preshuffled_a_input(g):
    """A handed over already preshuffled (layout 2) gives the repack path's bits."""
    import torch
    M, N, K = 256, 512, 1536
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=24), seed=24)
    dp = g.DevProblem(p, (256, 256, 4, 4))
    ash = torch.empty(M * p.Kp // 4 * 3, dtype=torch.uint8, device="cuda")
    assert mx.preshuffle_rows(dp.a.data_ptr(), p.a_row_bytes, M, p.Kp, ash.data_ptr()) == 0
    D2 = g.run_explicit(dp, mx.OUT_F32, a_layout=2, a_dev=ash)
    D1 = g.run_explicit(dp, mx.OUT_F32, a_layout=1)
    assert np.array_equal(D1.view(np.uint32), D2.view(np.uint32))


def test_routed_repack_and_fallback(g, orc):
    """A shape the router repacks A for: full workspace (repack) and none (row-major A) give
    the same bits and pass the oracle."""
    # among the smallest shapes the router repacks A for
    M, N, K = g.routed_shape([(M, N, K) for K in (8192, 16384) for M in (384, 512, 640, 768, 1024)
                              for N in (4096, 5120, 5504, 6144, 6784, 8192)],
                             lambda t, S, rp: rp)
    p = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=23), seed=23)
    assert mx.repacks_a(M, N, p.Kp)
    dp = g.DevProblem(p, mx.choose_tile(M, N, p.Kp))
    rows = np.r_[0:8, 380:388, M - 8:M]
    R, ab = orc.problem_f64(p, rows=rows)
    D1 = g.run_routed(dp, mx.OUT_F32, with_ws=True)
    D0 = g.run_routed(dp, mx.OUT_F32, with_ws=False)
    checks.check_f32(D1[rows], R, ab)
    assert np.array_equal(D1.view(np.uint32), D0.view(np.uint32))


# ---- the direct kernel (independent implementation) ------------------------------------------

@pytest.mark.parametrize("groups", [(1, 1), (2, 2), (4, 3), (2, 4), (4, 4)])
@pytest.mark.parametrize("out_type", [0, 1, 2])
def test_direct_kernel(g, orc, groups, out_type):
    M, N, K = 256, 384, 1024
    if (N // 32) % groups[1] or (M // 32) % groups[0]:
        pytest.skip("grouping does not divide")
    p = mx.make_problem(M, N, K, seed=sum(groups) + out_type)
    dp = g.DevProblem(p, (128, 128) + groups)
    D = g.run_direct(dp, out_type)
    R, ab = _oracle(orc, p)
    checks.check(D, R, ab, out_type)


@pytest.mark.parametrize("splits", [2, 3, 5])
def test_direct_split_k(g, orc, splits):
    p = mx.make_problem(256, 256, 3072, seed=splits)
    dp = g.DevProblem(p, (128, 128, 2, 2))
    D = g.run_direct(dp, mx.OUT_F16, splits=splits)
    R, ab = _oracle(orc, p)
    checks.check(D, R, ab, mx.OUT_F16)


# ---- split-K through the router -----------------------------------------------------------------

def test_routed_split_k_and_fallback(g, orc):
    M, N, K = 512, 512, 3072
    p = mx.make_problem(M, N, K, seed=21)
    S = mx.splitk_segments(M, N, p.Kp)
    assert S > 1
    dp = g.DevProblem(p, mx.choose_tile(M, N, p.Kp))
    R, ab = _oracle(orc, p)
    for out_type in (0, 1, 2):
        D = g.run_routed(dp, out_type, with_ws=True)
        checks.check(D, R, ab, out_type)
    # no workspace: runs unsplit (stderr warning), same bar
    D = g.run_routed(dp, mx.OUT_F32, with_ws=False)
    checks.check(D, R, ab, mx.OUT_F32)


def test_split_k_uneven_segments_large_k(g, orc):
    """Narrow N, large K: the split path with k_tiles % S != 0 (checked on sampled rows)."""
    M, N, K = 2048, 1024, 12256  # kpad 12288 = 64 K-tiles
    p = mx.make_problem(M, N, K, seed=31)
    S = mx.splitk_segments(M, N, p.Kp)
    assert S > 1
    dp = g.DevProblem(p, mx.choose_tile(M, N, p.Kp))
    rows = np.r_[0:8, 1000:1008, M - 8:M]
    R, ab = _oracle(orc, p, rows)
    D = g.run_routed(dp, mx.OUT_F32)
    checks.check(D[rows], R, ab, mx.OUT_F32)


# ---- layout variants and failure behaviour ------------------------------------------------------

def test_compact_and_padded_a_agree(g):
    M, N, K = 256, 256, 928
    pc = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=41, compact=True), seed=41)
    pp = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=41, compact=False), seed=41)
    assert np.array_equal(pc.a_codes_view(), pp.a_codes_view())
    t = mx.choose_tile(M, N, pc.Kp)
    Dc = g.run_routed(g.DevProblem(pc, t), mx.OUT_F32)
    Dp = g.run_routed(g.DevProblem(pp, t), mx.OUT_F32)
    assert np.array_equal(Dc.view(np.uint32), Dp.view(np.uint32))


@pytest.mark.parametrize("pad", [4, 8, 16])
def test_row_stride_alignments(g, pad):
    """A rows at a stride of packed(Kp) + pad bytes (4-, 8- and 16-byte aligned rows): the
    row-major paths (the routed plan, the plan without a workspace, a pipelined tile), the repack
    path (its 4/8/16-byte load variants) and the device preshuffle all give the bits of the
    padded-row problem."""
    import dataclasses
    import torch
    M, N, K = 256, 2048, 992  # Kp 1152; the repack is forced through the explicit plan
    pp = checks.spread_scales(mx.make_problem(M, N, K, **T3, seed=43, compact=False), seed=43)
    rb = pp.a_row_bytes + pad
    a = np.zeros(M * rb, dtype=np.uint8)
    a.reshape(M, rb)[:, :pp.a_row_bytes] = pp.a_packed[:M * pp.a_row_bytes].reshape(M, -1)
    ps = dataclasses.replace(pp, a_packed=a, a_row_bytes=rb)
    t = mx.choose_tile(M, N, pp.Kp)
    dpp, dps = g.DevProblem(pp, t), g.DevProblem(ps, t)
    # with a workspace the routed plan; without one (a split plan then runs unsplit) another
    for with_ws in (True, False):
        ref = g.run_routed(dpp, mx.OUT_F32, with_ws=with_ws)
        got = g.run_routed(dps, mx.OUT_F32, with_ws=with_ws)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), with_ws
    # a pipelined tile, row-major and repacked (the 32 x 32 tile reads row-major A only)
    tp = (128, 128, 2, 2)
    ref_p = g.run_explicit(g.DevProblem(pp, tp), mx.OUT_F32)
    dps_p = g.DevProblem(ps, tp)
    for a_layout in (0, 1):
        got = g.run_explicit(dps_p, mx.OUT_F32, a_layout=a_layout)
        assert np.array_equal(got.view(np.uint32), ref_p.view(np.uint32)), a_layout
    ash_p = torch.empty(M * pp.Kp // 4 * 3, dtype=torch.uint8, device="cuda")
    ash_s = torch.empty_like(ash_p)
    assert mx.preshuffle_rows(dpp.a.data_ptr(), pp.a_row_bytes, M, pp.Kp, ash_p.data_ptr()) == 0
    assert mx.preshuffle_rows(dps.a.data_ptr(), rb, M, pp.Kp, ash_s.data_ptr()) == 0
    torch.cuda.synchronize()
    assert torch.equal(ash_p, ash_s)


def test_nan_scale_poisons_its_row(g, orc):
    M, N, K = 256, 256, 768
    p = mx.make_problem(M, N, K, seed=51)
    p.a_scales[77, 5] = 255  # E8M0 NaN in one A block
    dp = g.DevProblem(p, mx.choose_tile(M, N, p.Kp))
    D = g.run_routed(dp, mx.OUT_F32)
    R, ab = _oracle(orc, p)
    assert np.isnan(D[77]).all()
    checks.check_f32(D, R, ab)


def test_stream_entry_point(g, orc):
    import torch
    p = mx.make_problem(256, 512, 1152, seed=61)
    dp = g.DevProblem(p, mx.choose_tile(256, 512, p.Kp))
    s = torch.cuda.Stream()
    D = g.run_routed(dp, mx.OUT_BF16, stream=s)
    R, ab = _oracle(orc, p)
    checks.check(D, R, ab, mx.OUT_BF16)


# ---- cross-library parity with the reference GPU library ----------------------------------------

@pytest.mark.parametrize("M,N,K,out_type", [(512, 512, 768, 0), (768, 1280, 960, 1),
                                            (4096, 4096, 768, 1), (2048, 1024, 12288, 0)])
def test_reference_library_same_inputs(g, orc, ref_lib, M, N, K, out_type):
    """Our D and the reference library's D on the same operands (each with the scale grouping
    of its own router) both meet the oracle bar; when both split K the same way (same segment
    count, hence the same MFMA sequence and reduction order) they are bit-identical."""
    import ctypes as C
    import torch
    p = mx.make_problem(M, N, K, seed=M * 3 + N * 7 + K)
    ours = g.run_routed(g.DevProblem(p, mx.choose_tile(M, N, p.Kp)), out_type)
    t = (C.c_int * 4)()
    ref_lib.ref_choose_tile(M, N, p.Kp, t)
    dr = g.DevProblem(p, tuple(t))
    D = dr.out(out_type)
    wsb = ref_lib.ref_gemm_workspace_size(M, N, p.Kp)
    ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device="cuda")
    a, b, sa, sb = dr.ptrs()
    g.say(f"  reference library {M}x{N}x{K} tile {tuple(t)} ws {wsb}")
    ref_lib.ref_gemm(out_type, M, N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes,
                     p.b_row_bytes, ws.data_ptr() if wsb else None, wsb)
    torch.cuda.synchronize()
    theirs = g.to_f32(D, out_type, M, N)
    rows = np.r_[0:16, M // 2:M // 2 + 16, M - 16:M]
    R, ab = _oracle(orc, p, rows)
    checks.check(ours[rows], R, ab, out_type)
    checks.check(theirs[rows], R, ab, out_type)
    same = float((ours.view(np.uint32) == theirs.view(np.uint32)).mean())
    s_ours = mx.splitk_segments(M, N, p.Kp)
    s_ref = wsb // (M * N * 4) if wsb else 1
    g.say(f"    segments ours {s_ours} reference {s_ref}; bit-identical to the reference library: "
          f"{100 * same:.2f}% of elements")
    if s_ours == s_ref:
        assert same == 1.0


# ---- FP16/BF16 epilogue: exactly the rounded FP32 result ------------------------------------

@pytest.mark.parametrize("tile", [(256, 256, 4, 4), (256, 256, 2, 4), (256, 192, 4, 3),
                                  (128, 384, 4, 3), (128, 256, 2, 4), (128, 128, 2, 2),
                                  (64, 256, 2, 2), (32, 256, 1, 2), (64, 128, 2, 1),
                                  (32, 128, 1, 1), (128, 512, 4, 4), (128, 256, 4, 2),
                                  (256, 256, 4, 2)])
@pytest.mark.parametrize("M,N", [(256, 768), (512, 1536), (289, 418), (97, 419)])
def test_lowp_output_is_rounded_f32(g, tile, M, N):
    """Every tile, unsplit: the FP16 and BF16 outputs equal the FP32 output of the same plan
    rounded to nearest-even on the host, bit for bit (the lane-pair exchange of the 16-bit
    epilogue moves every value to its row and column; N odd takes the element stores)."""
    import torch
    K = 1056
    p = mx.make_problem(M, N, K, dist_a=mx.DIST_STUDENT_T3, dist_b=mx.DIST_STUDENT_T3,
                        seed=M + N)
    dp = g.DevProblem(p, tile)
    D32 = g.run_explicit(dp, mx.OUT_F32)
    D16 = g.run_explicit(dp, mx.OUT_F16)
    Db16 = g.run_explicit(dp, mx.OUT_BF16)
    want16 = D32.astype(np.float16).astype(np.float32)
    assert np.array_equal(D16.view(np.uint32), want16.view(np.uint32))
    wantb = checks.round_bf16(D32)
    assert np.array_equal(Db16.view(np.uint32), wantb.view(np.uint32))
