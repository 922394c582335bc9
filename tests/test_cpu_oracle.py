"""Pinning the oracle's GEMM (CPU only).

o_gemm_f64 is checked against a library routine (numpy float64 matmul of operands dequantised
from the OCP value table), against closed forms, and against the reference's own CPU GEMM within
the FP32 rounding bound; o_gemm_f32_seq must equal the reference's CPU GEMM bit for bit.
Planted mistakes (in the oracle's output, on the CPU) must trip the parity checks.
"""
import json
import os

import numpy as np
import pytest

import checks

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _table():
    with open(os.path.join(GOLD, "e2m3_table.json")) as f:
        m = json.load(f)["magnitudes"]
    return np.array(m + [-x for x in m], dtype=np.float64)


def _dequant_np(packed, row_bytes, scales, rows, K):
    """numpy dequantisation from the bit layout and the value table."""
    t = _table()
    b = np.lib.stride_tricks.as_strided(packed, shape=(rows, K // 4 * 3), strides=(row_bytes, 1))
    g = b.reshape(rows, K // 4, 3).astype(np.uint32)
    w = g[..., 0] | (g[..., 1] << 8) | (g[..., 2] << 16)
    codes = np.stack([(w >> (6 * i)) & 63 for i in range(4)], axis=-1).reshape(rows, K)
    sc = np.exp2(scales[:, :K // 32].astype(np.float64) - 127)
    return t[codes] * np.repeat(sc, 32, axis=1)


@pytest.mark.parametrize("M,N,K,dist", [(64, 96, 256, 0), (128, 64, 1024, 2), (32, 32, 4032, 1)])
def test_f64_equals_numpy_matmul(mx, orc, M, N, K, dist):
    p = mx.make_problem(M, N, K, dist_a=dist, dist_b=dist, seed=M + N + K)
    D, ab = orc.problem_f64(p)
    a = _dequant_np(p.a_packed, p.a_row_bytes, p.a_scales, M, K)
    b = _dequant_np(p.b_packed, p.b_row_bytes, p.b_scales, N, K)
    R = a @ b.T
    assert np.allclose(D, R, rtol=0, atol=1e-12 * (np.abs(a) @ np.abs(b).T).max())
    assert np.allclose(ab, np.abs(a) @ np.abs(b).T, rtol=1e-12)


def test_f64_closed_forms(orc):
    M, N, K = 32, 32, 256
    ones = np.array([8, 8, 8, 8], dtype=np.uint8)  # code 8 = 1.0
    pk = orc.pack(np.tile(ones, K // 4))
    a = np.tile(pk, M)
    b = np.tile(pk, N)
    sa = np.full((M, K // 32), 127, dtype=np.uint8)
    sb = np.full((N, K // 32), 127, dtype=np.uint8)
    sa[:, 0] = 130   # block 0 of A scaled by 8
    sb[3, :] = 126   # row 3 of B halved
    D, ab = orc.gemm_f64(a, K // 4 * 3, sa, b, K // 4 * 3, sb, M, N, K)
    want = np.full((M, N), (K - 32) + 32 * 8.0)
    want[:, 3] /= 2
    assert np.array_equal(D, want) and np.array_equal(ab, want)
    # a NaN scale poisons exactly its row
    sa[5, 2] = 255
    D, _ = orc.gemm_f64(a, K // 4 * 3, sa, b, K // 4 * 3, sb, M, N, K)
    assert np.isnan(D[5]).all() and not np.isnan(np.delete(D, 5, axis=0)).any()


def test_f32_seq_bit_exact_with_reference(mx, orc, ref_lib):
    M, N, K = 48, 64, 1024
    p = mx.make_problem(M, N, K, compact=False, seed=3)
    Df = orc.gemm_f32_seq(p.a_packed, p.a_row_bytes, p.a_scales, p.b_packed, p.b_row_bytes,
                          p.b_scales, M, N, K)
    # the reference function on dense [rows][K] operands
    a = np.ascontiguousarray(p.a_codes_view())
    b = np.ascontiguousarray(p.b_codes_view())
    sa = np.ascontiguousarray(p.a_scales[:, :K // 32])
    sb = np.ascontiguousarray(p.b_scales[:, :K // 32])
    R = np.empty((M, N), dtype=np.float32)
    ref_lib.ref_gemm_cpu(a.ctypes.data, sa.ctypes.data, b.ctypes.data, sb.ctypes.data, M, N, K,
                         R.ctypes.data)
    assert np.array_equal(Df.view(np.uint32), R.view(np.uint32))
    # and the FP64 oracle agrees with the reference's FP32 result within FP32 rounding
    D, ab = orc.problem_f64(p)
    assert (np.abs(R - D) <= K * 2.0 ** -24 * ab).all()


def test_f32_seq_split_equals_whole(mx, orc):
    p = mx.make_problem(32, 48, 576, seed=13)
    D = orc.gemm_f32_seq(p.a_packed, p.a_row_bytes, p.a_scales, p.b_packed, p.b_row_bytes,
                         p.b_scales, 32, 48, 576)
    bf = orc.dequant_f32(p.b_packed, p.b_row_bytes, p.b_scales, 48, 576)
    rows = [3, 0, 31]
    Ds = orc.gemm_f32_seq_deq(p.a_packed, p.a_row_bytes, p.a_scales, bf, 32, 48, 576, rows)
    assert np.array_equal(Ds.view(np.uint32), D[rows].view(np.uint32))


def test_f64_row_subset_equals_full(mx, orc):
    p = mx.make_problem(96, 128, 576, seed=9)
    D, ab = orc.problem_f64(p)
    rows = [0, 17, 95, 40]
    Ds, abs_ = orc.problem_f64(p, rows=rows)
    assert np.array_equal(Ds, D[rows]) and np.array_equal(abs_, ab[rows])


def test_checks_catch_planted_mistakes(mx, orc):
    p = mx.make_problem(64, 64, 1024, seed=5)
    R, ab = orc.problem_f64(p)
    checks.check_f32(R.astype(np.float32), R, ab)          # the FP32 rounding of R passes
    bad = R.copy()
    bad[3, 7] += 1e-4 * ab[3, 7]                          # a dropped / extra term
    with pytest.raises(AssertionError):
        checks.check_f32(bad, R, ab)
    with pytest.raises(AssertionError):                   # a transposed operand
        checks.check_f32(R.T.copy(), R, ab)
    r16 = R.astype(np.float32).astype(np.float16).astype(np.float32)
    checks.check_lowp(r16, R, "f16")
    with pytest.raises(AssertionError):                   # 2 ulp off
        e = r16.copy()
        e[0, 0] = np.nextafter(np.nextafter(np.float16(e[0, 0]), np.float16(1e4)), np.float16(1e4))
        checks.check_lowp(e, R, "f16")
    b16 = checks.round_bf16(R.astype(np.float32))
    checks.check_lowp(b16, R, "bf16")
    with pytest.raises(AssertionError):
        checks.check_lowp(-b16 + 1e-3, R, "bf16")


@pytest.mark.parametrize("out_type", [0, 1, 2])
def test_checksums_catch_planted_mistakes(mx, orc, out_type):
    """The whole-output checksums of the full-size GPU tests pass on the oracle's own D (rounded
    to the output format) and fail on a zeroed 32x32 block, two swapped 128-column tiles, one
    row scaled by 2 (a wrong scale), and a doubled K segment in one 32x32 block."""
    M, N, K = 256, 384, 1024
    p = mx.make_problem(M, N, K, seed=11 + out_type)
    R, _ = orc.problem_f64(p)
    r32 = R.astype(np.float32)
    D = {0: r32, 1: r32.astype(np.float16).astype(np.float32),
         2: checks.round_bf16(r32)}[out_type].astype(np.float64)
    Af = orc.dequant_f32(p.a_packed, p.a_row_bytes, p.a_scales, M, K)
    Bf = orc.dequant_f32(p.b_packed, p.b_row_bytes, p.b_scales, N, K)

    def run(d):
        return checks.check_checksums(d.sum(0), d.sum(1), np.abs(d).sum(0), np.abs(d).sum(1),
                                      float(d.sum()), Af, Bf, out_type)

    run(D)
    half = orc.gemm_f64(p.a_packed, p.a_row_bytes, p.a_scales, p.b_packed, p.b_row_bytes,
                        p.b_scales, M, N, K // 2)[0]
    planted = []
    z = D.copy(); z[64:96, 32:64] = 0; planted.append(z)                 # block never written
    s = D.copy(); s[:, 0:128], s[:, 128:256] = D[:, 128:256], D[:, 0:128]; planted.append(s)
    w = D.copy(); w[100] *= 2; planted.append(w)                          # wrong scale on a row
    dk = D.copy(); dk[0:32, 0:32] += half[0:32, 0:32]; planted.append(dk)  # K half counted twice
    for bad in planted:
        with pytest.raises(AssertionError):
            run(bad)
