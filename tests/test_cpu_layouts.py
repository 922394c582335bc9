"""Operand and scale layouts (CPU only): library == oracle == reference, byte for byte, plus
permutation invariants that follow from the layout definitions."""
import numpy as np
import pytest


@pytest.mark.parametrize("dim,K", [(32, 192), (128, 1152), (96, 384), (256, 4032)])
def test_preprocess_scale_three_ways(mx, orc, ref_lib, dim, K):
    rng = np.random.default_rng(dim + K)
    s = rng.integers(0, 255, (dim, K // 32), dtype=np.uint8)
    o = orc.preprocess_scale(s, dim, K)
    assert np.array_equal(mx.preprocess_scale(s, dim, K), o)
    r = np.empty_like(o)
    ref_lib.ref_preprocess_scale(s.ctypes.data, dim, K, r.ctypes.data)
    assert np.array_equal(r, o)
    # a permutation of the scales: same multiset
    assert np.array_equal(np.sort(o), np.sort(s.ravel()))


@pytest.mark.parametrize("group", [1, 2, 3, 4])
@pytest.mark.parametrize("dim,K", [(384, 1152), (768, 576)])
def test_tile_scale_three_ways(mx, orc, ref_lib, group, dim, K):
    if (dim // 32) % group:
        pytest.skip("group must divide dim/32")
    rng = np.random.default_rng(group * 7 + dim)
    s = rng.integers(0, 255, (dim, K // 32), dtype=np.uint8)
    ps = orc.preprocess_scale(s, dim, K)
    o = orc.tile_scale(ps, dim, K, group)
    assert np.array_equal(mx.tile_scale(ps, dim, K, group), o)
    r = np.empty_like(o)
    assert ref_lib.ref_tile_scale(s.ctypes.data, dim, K, group, 3, r.ctypes.data) == o.size
    assert np.array_equal(r, o)
    # fused multi-threaded path used for device uploads
    assert np.array_equal(mx.prepare_scales(s, dim, K, group), o)
    # padding bytes are zero, the rest is a permutation of the scales
    gp = (group + 3) // 4 * 4
    body = o.reshape(-1, gp)
    assert (body[:, group:] == 0).all()
    assert np.array_equal(np.sort(body[:, :group].ravel()), np.sort(s.ravel()))


@pytest.mark.parametrize("N,K", [(32, 64), (64, 192), (160, 1152)])
def test_preshuffle_three_ways(mx, orc, ref_lib, N, K):
    rng = np.random.default_rng(N * K)
    packed = rng.integers(0, 256, N * K // 4 * 3, dtype=np.uint8)
    scales = np.full((N, K // 32), 127, dtype=np.uint8)
    o = orc.preshuffle_b(packed, N, K, K // 4 * 3)
    assert np.array_equal(mx.preshuffle_b(packed, N, K), o)
    assert np.array_equal(mx.prepare_b(packed, N, K, K // 4 * 3), o)
    r = np.empty_like(o)
    ref_lib.ref_preshuffle_b(packed.ctypes.data, scales.ctypes.data, N, K, r.ctypes.data)
    assert np.array_equal(r, o)
    assert np.array_equal(np.sort(o), np.sort(packed))


def test_preshuffle_wide_rows(mx, orc):
    # rows longer than packed(K) (a padded B^T): only the first packed(K) bytes are used
    N, K, rb = 64, 192, 200
    rng = np.random.default_rng(0)
    packed = rng.integers(0, 256, N * rb, dtype=np.uint8)
    assert np.array_equal(mx.prepare_b(packed, N, K, rb), orc.preshuffle_b(packed, N, K, rb))


def test_pad_scales_and_end_pad(mx, orc, ref_lib):
    rng = np.random.default_rng(1)
    for K in (32, 160, 192, 224, 1024, 105728):
        s = rng.integers(0, 255, (5, K // 32), dtype=np.uint8)
        o = orc.pad_scales_k(s, 5, K)
        assert np.array_equal(mx.pad_scales_k(s, 5, K), o)
        r = np.empty_like(o)
        ref_lib.ref_pad_scales_k(s.ctypes.data, 5, K, r.ctypes.data)
        assert np.array_equal(r, o)
        assert mx.a_compact_end_pad(K) == ref_lib.ref_a_compact_end_pad(K) == \
            (mx.kpad(K) - K) // 4 * 3
        assert mx.kpad(K) == ref_lib.ref_kpad(K)


def test_problem_layouts_consistent(mx, orc):
    p = mx.make_problem(256, 384, 1024)
    bsh, sa, sb = p.layouts((128, 384, 4, 3))
    assert np.array_equal(bsh, orc.preshuffle_b(p.b_packed, p.N, p.Kp, p.b_row_bytes))
    assert np.array_equal(sa, orc.tile_scale(orc.preprocess_scale(p.a_scales, p.M, p.Kp), p.M, p.Kp, 4))
    assert np.array_equal(sb, orc.tile_scale(orc.preprocess_scale(p.b_scales, p.N, p.Kp), p.N, p.Kp, 3))
    # compact A: rows of packed(K), end pad present, K-tail scales 127
    assert p.a_row_bytes == 768 and p.a_packed.size == 256 * 768 + mx.a_compact_end_pad(1024)
    assert (p.a_scales[:, 32:] == 127).all() and (p.b_scales[:, 32:] == 127).all()
