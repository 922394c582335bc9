"""ctypes binding of the MXFP6 oracle -- TEST INFRASTRUCTURE ONLY.

Loads oracle/liboracle.so (the C restatement, see oracle.h for what each function restates
and how it is pinned) and, when present, oracle/_ref/libmxfp6ref.so (the reference library
compiled from its own sources). Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of
bench.py use this module, as the checker or the CPU baseline; the product never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libmxfp6ref.so")

_vp = C.c_void_p
_SIG = {
    "o_fp6_decode": (C.c_double, [C.c_uint8]),
    "o_fp6_encode": (C.c_uint8, [C.c_float]),
    "o_e8m0_decode": (C.c_double, [C.c_uint8]),
    "o_pack": (None, [_vp, C.c_int, _vp]),
    "o_unpack": (None, [_vp, C.c_int, _vp]),
    "o_quantize_ref": (None, [_vp, C.c_int, C.c_int, _vp, _vp]),
    "o_quantize_ocp": (None, [_vp, C.c_int, C.c_int, _vp, _vp]),
    "o_pad_scales_k": (None, [_vp, C.c_int, C.c_int, _vp]),
    "o_preprocess_scale": (None, [_vp, C.c_int, C.c_int, _vp]),
    "o_tile_scale_bytes": (C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "o_tile_scale": (None, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp]),
    "o_preshuffle_b": (None, [_vp, C.c_int, C.c_int, C.c_size_t, _vp]),
    "o_choose_tile_ref": (None, [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int)]),
    "o_splitk_s_ref": (C.c_int, [C.c_int, C.c_int, C.c_int]),
    "o_gemm_f64": (C.c_int, [_vp, C.c_size_t, _vp, C.c_int, _vp, C.c_size_t, _vp, C.c_int,
                             C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp, C.c_int]),
    "o_gemm_f32_seq": (C.c_int, [_vp, C.c_size_t, _vp, C.c_int, _vp, C.c_size_t, _vp, C.c_int,
                                 C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp, C.c_int]),
    "o_dequant_f32": (C.c_int, [_vp, C.c_size_t, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "o_gemm_f32_seq_deq": (C.c_int, [_vp, C.c_size_t, _vp, C.c_int, _vp, C.c_int, C.c_int,
                                     C.c_int, _vp, C.c_int, _vp, C.c_int]),
}
_REF_SIG = {
    "ref_fp6_decode": (C.c_float, [C.c_uint8]),
    "ref_fp6_encode": (C.c_uint8, [C.c_float]),
    "ref_e8m0_decode": (C.c_float, [C.c_uint8]),
    "ref_e8m0_encode": (C.c_uint8, [C.c_float]),
    "ref_pack": (None, [_vp, C.c_int, _vp]),
    "ref_unpack": (None, [_vp, C.c_int, _vp]),
    "ref_a_compact_end_pad": (C.c_int, [C.c_int]),
    "ref_kpad": (C.c_int, [C.c_int]),
    "ref_pad_scales_k": (None, [_vp, C.c_int, C.c_int, _vp]),
    "ref_quantize": (None, [_vp, C.c_int, C.c_int, _vp, _vp]),
    "ref_preprocess_b": (None, [_vp, C.c_int, C.c_int, _vp, _vp]),
    "ref_dequantize": (None, [_vp, _vp, C.c_int, C.c_int, _vp]),
    "ref_preprocess_scale": (None, [_vp, C.c_int, C.c_int, _vp]),
    "ref_tile_scale": (C.c_size_t, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp]),
    "ref_preshuffle_b": (None, [_vp, _vp, C.c_int, C.c_int, _vp]),
    "ref_gemm_cpu": (None, [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, _vp]),
    "ref_choose_tile": (None, [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int)]),
    "ref_gemm_workspace_size": (C.c_size_t, [C.c_int, C.c_int, C.c_int]),
    "ref_gemm": (None, [C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_int,
                        C.c_int, _vp, C.c_size_t]),
    "ref_gemm_force_tile": (None, [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int), _vp,
                                   _vp, _vp, _vp, _vp, C.c_int, C.c_int]),
}

_o = None
_r = None


def _load(path, sig):
    h = C.CDLL(path)
    for name, (res, args) in sig.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    return h


def lib():
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run make -C oracle")
        _o = _load(ORACLE_SO, _SIG)
    return _o


def ref():
    """The reference library (None when it was not built)."""
    global _r
    if _r is None and os.path.exists(REF_SO):
        _r = _load(REF_SO, _REF_SIG)
    return _r


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def gemm_f64(a_packed, a_row_bytes, a_scales, b_packed, b_row_bytes, b_scales, M, N, K,
             rows=None, nthreads=0):
    """(D, absdot) float64 [nrows, N] over the nominal K for the listed A rows (all if None)."""
    a_scales = np.ascontiguousarray(a_scales)
    b_scales = np.ascontiguousarray(b_scales)
    ridx = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    nr = M if ridx is None else len(ridx)
    D = np.empty((nr, N), dtype=np.float64)
    ab = np.empty((nr, N), dtype=np.float64)
    rc = lib().o_gemm_f64(_p(a_packed), a_row_bytes, _p(a_scales), a_scales.shape[1],
                          _p(b_packed), b_row_bytes, _p(b_scales), b_scales.shape[1], M, N, K,
                          None if ridx is None else _p(ridx), nr, _p(D), _p(ab), nthreads)
    if rc != 0:
        raise RuntimeError(f"o_gemm_f64 failed ({rc})")
    return D, ab


def gemm_f32_seq(a_packed, a_row_bytes, a_scales, b_packed, b_row_bytes, b_scales, M, N, K,
                 rows=None, nthreads=0):
    a_scales = np.ascontiguousarray(a_scales)
    b_scales = np.ascontiguousarray(b_scales)
    ridx = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    nr = M if ridx is None else len(ridx)
    D = np.empty((nr, N), dtype=np.float32)
    rc = lib().o_gemm_f32_seq(_p(a_packed), a_row_bytes, _p(a_scales), a_scales.shape[1],
                              _p(b_packed), b_row_bytes, _p(b_scales), b_scales.shape[1], M, N, K,
                              None if ridx is None else _p(ridx), nr, _p(D), nthreads)
    if rc != 0:
        raise RuntimeError(f"o_gemm_f32_seq failed ({rc})")
    return D


def dequant_f32(packed, row_bytes, scales, rows, K):
    scales = np.ascontiguousarray(scales)
    out = np.empty((rows, K), dtype=np.float32)
    if lib().o_dequant_f32(_p(packed), row_bytes, _p(scales), scales.shape[1], rows, K, _p(out)):
        raise RuntimeError("o_dequant_f32 failed")
    return out


def gemm_f32_seq_deq(a_packed, a_row_bytes, a_scales, bf, M, N, K, rows, nthreads=0):
    a_scales = np.ascontiguousarray(a_scales)
    ridx = np.ascontiguousarray(rows, dtype=np.int32)
    D = np.empty((len(ridx), N), dtype=np.float32)
    if lib().o_gemm_f32_seq_deq(_p(a_packed), a_row_bytes, _p(a_scales), a_scales.shape[1],
                                _p(bf), M, N, K, _p(ridx), len(ridx), _p(D), nthreads):
        raise RuntimeError("o_gemm_f32_seq_deq failed")
    return D


def problem_f64(p, rows=None, nthreads=0):
    """Oracle D (float64) and sum|a*b| of an mxfp6_amd.Problem over its nominal K."""
    return gemm_f64(p.a_packed, p.a_row_bytes, p.a_scales, p.b_packed, p.b_row_bytes, p.b_scales,
                    p.M, p.N, p.K, rows, nthreads)


def choose_tile_ref(M, N, Kp):
    t = (C.c_int * 4)()
    lib().o_choose_tile_ref(M, N, Kp, t)
    return tuple(t)


def splitk_s_ref(M, N, Kp):
    return lib().o_splitk_s_ref(M, N, Kp)


def preprocess_scale(scales, dim, K):
    out = np.empty((dim // 32) * (K // 64) * 64, dtype=np.uint8)
    lib().o_preprocess_scale(_p(np.ascontiguousarray(scales)), dim, K, _p(out))
    return out


def tile_scale(ps, dim, K, group, subs=3):
    out = np.empty(lib().o_tile_scale_bytes(dim, K, group, subs), dtype=np.uint8)
    lib().o_tile_scale(_p(np.ascontiguousarray(ps)), dim, K, group, subs, _p(out))
    return out


def preshuffle_b(packed, N, K, row_bytes):
    out = np.empty((N // 32) * (K // 64) * 1536, dtype=np.uint8)
    lib().o_preshuffle_b(_p(np.ascontiguousarray(packed)), N, K, row_bytes, _p(out))
    return out


def pad_scales_k(scales, dim, K):
    Kp = (K + 191) // 192 * 192
    out = np.empty((dim, Kp // 32), dtype=np.uint8)
    lib().o_pad_scales_k(_p(np.ascontiguousarray(scales)), dim, K, _p(out))
    return out


def quantize_ref(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    r, c = x.shape
    packed = np.empty(r * c // 4 * 3, dtype=np.uint8)
    scales = np.empty((r, c // 32), dtype=np.uint8)
    lib().o_quantize_ref(_p(x), r, c, _p(packed), _p(scales))
    return packed, scales


def quantize_ocp(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    r, c = x.shape
    packed = np.empty(r * c // 4 * 3, dtype=np.uint8)
    scales = np.empty((r, c // 32), dtype=np.uint8)
    lib().o_quantize_ocp(_p(x), r, c, _p(packed), _p(scales))
    return packed, scales


def pack(codes):
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(codes.size // 4 * 3, dtype=np.uint8)
    lib().o_pack(_p(codes), codes.size, _p(out))
    return out


def unpack(packed, n):
    out = np.empty(n, dtype=np.uint8)
    lib().o_unpack(_p(np.ascontiguousarray(packed, dtype=np.uint8)), n, _p(out))
    return out
