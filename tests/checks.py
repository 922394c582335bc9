"""Parity bars of the MXFP6 GEMM against the FP64 oracle (R = exact dot of the dequantised
operands over the nominal K, accumulated in FP64).

  FP32 output: |D - R| <= 1e-5 * sum_k |a_k b_k|      (per element; relative to the magnitude of
               the terms, so cancellation in R does not make the bound vanish)
               and max|D - R| / max|R| <= 1e-5        (normwise over the elements compared)
  FP16/BF16:   |D - rn(R32)| <= 1 ulp(rn(R32))          R32 = float32(R), rn = round to nearest
               even in the output format, ulp = spacing of that format at |rn(R32)|
NaN in R (a 0xFF scale) requires NaN in D.
"""
import numpy as np

F32_RTOL = 1e-5


def _nan_ok(D, R):
    rn = np.isnan(R)
    assert np.array_equal(np.isnan(D), rn), "NaN pattern differs from the oracle"
    return ~rn


def check_f32(D, R, absdot, rtol=F32_RTOL):
    D = np.asarray(D, dtype=np.float64)
    ok = _nan_ok(D, R)
    err = np.abs(D - R)[ok]
    bound = rtol * absdot[ok]
    bad = err > bound
    assert not bad.any(), (f"{bad.sum()} elements exceed {rtol}*sum|ab|; worst excess "
                           f"{(err - bound).max():.3e}")
    if not err.size:
        return 0.0
    rmax = float(np.abs(R[ok]).max())
    if rmax == 0.0:
        assert err.max() == 0.0, "nonzero output where the oracle is all zero"
        return 0.0
    rel = float(err.max() / rmax)
    assert rel <= rtol, f"normwise max|D-R|/max|R| = {rel:.3e} exceeds {rtol}"
    return rel


def round_bf16(x32: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16, returned as float32 (finite inputs)."""
    u = x32.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def ulp_bf16(x32: np.ndarray) -> np.ndarray:
    return np.spacing(np.abs(x32).astype(np.float32)) * np.float32(65536.0)


def check_lowp(D, R, kind):
    """D: device output converted to float32 (exact for f16/bf16)."""
    D = np.asarray(D, dtype=np.float32)
    ok = _nan_ok(D, R)
    r32 = R.astype(np.float32)
    if kind == "f16":
        e = r32.astype(np.float16)
        ulp = np.spacing(np.abs(e)).astype(np.float32)
        e = e.astype(np.float32)
    elif kind == "bf16":
        e = round_bf16(r32)
        ulp = ulp_bf16(e)
    else:
        raise ValueError(kind)
    diff = np.abs(D.astype(np.float64) - e.astype(np.float64))[ok]
    bad = diff > ulp.astype(np.float64)[ok]
    assert not bad.any(), f"{bad.sum()} elements differ by more than 1 ulp from rn(R32)"
    exact = float((diff == 0).mean()) if diff.size else 1.0
    return exact


def check(D, R, absdot, out_type):
    if out_type == 0:
        return check_f32(D, R, absdot)
    return check_lowp(D, R, "f16" if out_type == 1 else "bf16")


# ---- whole-output checksums (full-size workloads) ------------------------------------------------

# half an ulp of each output format relative to |D| (normal range), and its subnormal step
HALF_ULP = {0: (0.0, 0.0), 1: (2.0 ** -11, 2.0 ** -24), 2: (2.0 ** -8, 2.0 ** -133)}


def spread_scales(p, span=12, seed=0):
    """Lower every E8M0 block scale of both operands of problem p by its own random exponent in
    [0, span] (kept >= 1), in place, and drop p's cached layouts. The products summed along K then
    span about 2^(2 span) in magnitude while none grows (no FP16 overflow), so FP32 sums round and
    their bits depend on the order of the additions: the operands of the bit-for-bit comparisons
    between two computations. (With the generator's own scales, which follow each block's maximum,
    the FP32 sums of the scaled products stay exact whatever the order.)"""
    rng = np.random.default_rng(seed)
    for sc in (p.a_scales, p.b_scales):
        off = rng.integers(-span, 1, size=sc.shape)
        sc[...] = np.clip(sc.astype(np.int32) + off, 1, 254).astype(np.uint8)
    p.tiles.clear()
    return p


def _gemv64(X32, v64, chunk=1024):
    """X (float32 [R][K]) @ v (float64 [K]) in float64, a block of rows at a time."""
    out = np.empty(X32.shape[0], dtype=np.float64)
    for r in range(0, X32.shape[0], chunk):
        out[r:r + chunk] = X32[r:r + chunk].astype(np.float64) @ v64
    return out


def check_checksums(col_sum, row_sum, col_abs, row_abs, total, Af, Bf, out_type):
    """Row and column sums of D (float64 sums of the output values, and of their magnitudes)
    against FP64 GEMVs of the exactly dequantised operands Af [M][K] and Bf = B^T [N][K]:
    column sums = (1^T A) B, row sums = A (B 1), total = 1^T A B 1. Each row or column may differ
    by the sum of its elements' bars: 1e-5 * sum|ab| for the FP32 accumulation, half an ulp of
    the output format per element and the format's smallest subnormal step. Returns the largest
    error / bound ratio over columns and rows."""
    M, N = Af.shape[0], Bf.shape[0]
    sA = Af.sum(axis=0, dtype=np.float64)
    sB = Bf.sum(axis=0, dtype=np.float64)
    col_pred = _gemv64(Bf, sA)
    row_pred = _gemv64(Af, sB)
    col_ab = _gemv64(np.abs(Bf), np.abs(Af).sum(axis=0, dtype=np.float64))
    row_ab = _gemv64(np.abs(Af), np.abs(Bf).sum(axis=0, dtype=np.float64))
    rel, sub = HALF_ULP[out_type]
    col_bound = F32_RTOL * col_ab + rel * np.asarray(col_abs) + sub * M
    row_bound = F32_RTOL * row_ab + rel * np.asarray(row_abs) + sub * N
    col_err = np.abs(np.asarray(col_sum) - col_pred)
    row_err = np.abs(np.asarray(row_sum) - row_pred)
    assert (col_err <= col_bound).all(), (
        f"{(col_err > col_bound).sum()} column sums off; worst column "
        f"{int(np.argmax(col_err - col_bound))}")
    assert (row_err <= row_bound).all(), (
        f"{(row_err > row_bound).sum()} row sums off; worst row {int(np.argmax(row_err - row_bound))}")
    tot_pred = float(sA @ sB)
    assert abs(total - tot_pred) <= col_bound.sum(), f"total {total} vs {tot_pred}"
    return float((col_err / col_bound).max()), float((row_err / row_bound).max())
