"""Parity bars of the MXFP6 GEMM against the FP64 oracle (R = exact dot of the dequantised
operands over the nominal K, accumulated in FP64).

  FP32 output: |D - R| <= 1e-5 * sum_k |a_k b_k|      (per element; relative to the magnitude of
               the terms, so cancellation in R does not make the bound vanish)
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
    denom = max(np.abs(R[ok]).max(), 1e-300) if ok.any() else 1.0
    return float(err.max() / denom) if err.size else 0.0


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
