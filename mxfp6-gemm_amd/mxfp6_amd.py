"""Python binding of libmxfp6gemm (ctypes over the C ABI in include/mxfp6_gemm.h).

The library is the product: this module only marshals pointers. It loads
``lib/libmxfp6gemm.so`` next to this file and raises if it is missing -- there is no
fallback implementation. Device memory is plain integers (device addresses), e.g.
``torch.Tensor.data_ptr()``.

Host helpers build the operands of a GEMM problem in the public layouts (the same
layouts as the reference's include/mxfp6/preprocess.hpp):
  * A: packed E2M3 codes, row-major, compact rows of packed(K) bytes + a_compact_end_pad(K),
    raw scales [M][K/32] extended to [M][Kp/32] with code 127;
  * B: packed B^T [N][packed(Kp)] with a zero K-tail, raw scales [N][Kp/32];
  * kernel layouts: preshuffled B and tiled scales for a tile's (MPW, NPW).
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmxfp6gemm.so")

OUT_F32, OUT_F16, OUT_BF16 = 0, 1, 2
OUT_NAMES = {OUT_F32: "f32", OUT_F16: "f16", OUT_BF16: "bf16"}
OUT_BYTES = {OUT_F32: 4, OUT_F16: 2, OUT_BF16: 2}
DIST_NORMAL, DIST_UNIFORM, DIST_STUDENT_T3 = 0, 1, 2
K_TILE = 192

STATUS = {0: "OK", 1: "ERR_NULL", 2: "ERR_SHAPE", 3: "ERR_OUT_TYPE", 4: "ERR_TILE",
          5: "ERR_ARG", 6: "ERR_HIP", 7: "ERR_SCRATCH"}
NOALLOC_SCRATCH_BYTES = 128 << 20  # MXFP6_NOALLOC_SCRATCH_BYTES

# Every C symbol declared in include/mxfp6_gemm.h: (restype, argtypes).
_u8p = C.POINTER(C.c_uint8)
_vp = C.c_void_p
SIGNATURES = {
    "mxfp6_kpad": (C.c_int, [C.c_int]),
    "mxfp6_choose_tile": (C.c_int, [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int)]),
    "mxfp6_gemm_workspace_size": (C.c_size_t, [C.c_int, C.c_int, C.c_int]),
    "mxfp6_gemm_preferred_workspace_size": (C.c_size_t, [C.c_int, C.c_int, C.c_int]),
    "mxfp6_clock_sample_async": (C.c_int, [_vp, C.c_int, _vp]),
    "mxfp6_splitk_segments": (C.c_int, [C.c_int, C.c_int, C.c_int]),
    "mxfp6_gemm": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp,
                             C.c_int, C.c_int, _vp, C.c_size_t]),
    "mxfp6_gemm_async": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp,
                                   C.c_int, C.c_int, _vp, C.c_size_t, _vp]),
    "mxfp6_gemm_noalloc_async": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp,
                                           _vp, C.c_int, C.c_int, _vp]),
    "mxfp6_gemm_force_tile": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int),
                                        _vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, _vp]),
    "mxfp6_gemm_explicit": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int),
                                      C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_int, _vp,
                                      C.c_size_t, _vp]),
    "mxfp6_gemm_repacks_a": (C.c_int, [C.c_int, C.c_int, C.c_int]),
    "mxfp6_gemm_streams_output": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "mxfp6_gemm_tune": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                  C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                  C.c_size_t, C.c_int, C.c_void_p, C.POINTER(C.c_int),
                                  C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "mxfp6_gemm_tuned_plan": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int),
                                        C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "mxfp6_gemm_tune_reset": (None, []),
    "mxfp6_gemm_tune_save": (C.c_int, [C.c_char_p, C.POINTER(C.c_int)]),
    "mxfp6_gemm_tune_load": (C.c_int, [C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "mxfp6_gemm_plan": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_size_t,
                                  C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int)]),
    "mxfp6_plan_workspace_size": (C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "mxfp6_preshuffle_rows_async": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    "mxfp6_quantize_async": (C.c_int, [_vp, C.c_int, C.c_int, _vp, C.c_size_t, _vp, C.c_int, _vp]),
    "mxfp6_prepare_a_async": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, C.c_size_t, _vp,
                                        _vp]),
    "mxfp6_prepare_a_preshuffled_async": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp,
                                                    _vp]),
    "mxfp6_prepare_b_async": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp]),
    "mxfp6_tile_scales_async": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    "mxfp6_preshuffled_bytes": (C.c_size_t, [C.c_int, C.c_int]),
    "mxfp6_tiled_scale_bytes": (C.c_size_t, [C.c_int, C.c_int, C.c_int]),
    "mxfp6_gemm_direct": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp,
                                    _vp, _vp, _vp, _vp, C.c_int, C.c_int, _vp, C.c_size_t, _vp]),
    "mxfp6_fp6_e2m3_to_float": (C.c_float, [C.c_uint8]),
    "mxfp6_float_to_fp6_e2m3": (C.c_uint8, [C.c_float]),
    "mxfp6_e8m0_to_float": (C.c_float, [C.c_uint8]),
    "mxfp6_float_to_e8m0": (C.c_uint8, [C.c_float]),
    "mxfp6_pack_fp6": (C.c_int, [_vp, C.c_int, _vp]),
    "mxfp6_unpack_fp6": (C.c_int, [_vp, C.c_int, _vp]),
    "mxfp6_a_compact_end_pad": (C.c_int, [C.c_int]),
    "mxfp6_pad_scales_k": (C.c_int, [_vp, C.c_int, C.c_int, _vp]),
    "mxfp6_quantize": (C.c_int, [_vp, C.c_int, C.c_int, _vp, _vp]),
    "mxfp6_dequantize": (C.c_int, [_vp, _vp, C.c_int, C.c_int, _vp]),
    "mxfp6_preprocess_b": (C.c_int, [_vp, C.c_int, C.c_int, _vp, _vp]),
    "mxfp6_preprocess_scale": (C.c_int, [_vp, C.c_int, C.c_int, _vp]),
    "mxfp6_preshuffle_b": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp]),
    "mxfp6_tile_scale_bytes": (C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "mxfp6_tile_scale": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp]),
    "mxfp6_gen_operand": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_double, C.c_uint64,
                                    C.c_uint64, _vp, C.c_size_t, _vp, C.c_int, C.c_int]),
    "mxfp6_gen_values": (C.c_int, [C.c_int, C.c_int, C.c_int, C.c_double, C.c_uint64,
                                   C.c_uint64, _vp, C.c_int]),
    "mxfp6_prepare_b": (C.c_int, [_vp, C.c_int, C.c_int, C.c_size_t, _vp, C.c_int]),
    "mxfp6_prepare_scales": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int]),
}

_lib = None


class Mxfp6Error(RuntimeError):
    pass


def lib() -> C.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise Mxfp6Error(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                             "(make -C mxfp6-gemm_amd)")
        h = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise Mxfp6Error(f"{what} failed: {STATUS.get(rc, rc)}")


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def packed_bytes(n: int) -> int:
    return n // 4 * 3


def kpad(K: int) -> int:
    return lib().mxfp6_kpad(K)


def choose_tile(M: int, N: int, Kp: int) -> tuple:
    t = (C.c_int * 4)()
    _check(lib().mxfp6_choose_tile(M, N, Kp, t), "choose_tile")
    return tuple(t)


def workspace_size(M: int, N: int, Kp: int) -> int:
    """gemm_workspace_size: the split-K partials only (the reference's meaning)."""
    return lib().mxfp6_gemm_workspace_size(M, N, Kp)


def preferred_workspace_size(M: int, N: int, Kp: int) -> int:
    """The routed plan's whole workspace: split-K partials plus the repacked A when it repacks."""
    return lib().mxfp6_gemm_preferred_workspace_size(M, N, Kp)


def splitk_segments(M: int, N: int, Kp: int) -> int:
    return lib().mxfp6_splitk_segments(M, N, Kp)


def a_compact_end_pad(K: int) -> int:
    return lib().mxfp6_a_compact_end_pad(K)


# ---- GEMM launches (device addresses as ints) ---------------------------------------------------

def gemm(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, ws=0, ws_bytes=0, stream=None,
         B_row_bytes=0) -> int:
    """mxfp6_gemm_async; returns the status (0 on success)."""
    return lib().mxfp6_gemm_async(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes,
                                  B_row_bytes, ws or None, ws_bytes, stream)


def gemm_noalloc(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, stream=None,
                 B_row_bytes=0) -> int:
    """mxfp6_gemm_noalloc_async: no workspace argument, no device allocation (the library's
    per-GPU scratch); returns the status."""
    return lib().mxfp6_gemm_noalloc_async(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes,
                                          B_row_bytes, stream)


def gemm_null_stream(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, ws=0, ws_bytes=0,
                     B_row_bytes=0) -> int:
    return lib().mxfp6_gemm(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, B_row_bytes,
                            ws or None, ws_bytes)


def gemm_force_tile(out_type, M, N, Kp, tile, dA, dBsh, dsA, dsB, dD, A_row_bytes, stream=None):
    t = (C.c_int * 4)(*tile)
    return lib().mxfp6_gemm_force_tile(out_type, M, N, Kp, t, dA, dBsh, dsA, dsB, dD,
                                       A_row_bytes, 0, stream)


# A layouts of an explicit plan (mxfp6_gemm_explicit): row-major, repacked by the plan, already
# preshuffled, row-major staged in LDS in 12-byte units (wide tiles dividing M x N only)
A_ROWS, A_REPACK, A_PRESHUFFLED, A_ROWS_SWIZZLED = 0, 1, 2, 3


def gemm_explicit(out_type, M, N, Kp, tile, splits, dA, dBsh, dsA, dsB, dD, A_row_bytes, ws=0,
                  ws_bytes=0, stream=None, a_layout=A_ROWS):
    t = (C.c_int * 4)(*tile)
    return lib().mxfp6_gemm_explicit(out_type, M, N, Kp, t, splits, a_layout, dA, dBsh, dsA, dsB,
                                     dD, A_row_bytes, ws or None, ws_bytes, stream)


def repacks_a(M, N, Kp):
    """Whether gemm() repacks A into the preshuffled layout for this shape."""
    return bool(lib().mxfp6_gemm_repacks_a(M, N, Kp))


def gemm_tune(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, ws=0, ws_bytes=0,
              candidates=4, stream=None):
    """Times the router's best-predicted plans on these operands and keeps the fastest for later
    gemm() calls of the shape; returns (status, (tile, splits, a_repack))."""
    t = (C.c_int * 4)()
    s, r = C.c_int(0), C.c_int(0)
    rc = lib().mxfp6_gemm_tune(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, ws or None,
                               ws_bytes, candidates, stream, t, C.byref(s), C.byref(r))
    return rc, (tuple(t), s.value, bool(r.value))


def tuned_plan(out_type, M, N, Kp):
    """(tile, splits, a_repack) chosen by gemm_tune for this shape, or None."""
    t = (C.c_int * 4)()
    s, r = C.c_int(0), C.c_int(0)
    if not lib().mxfp6_gemm_tuned_plan(out_type, M, N, Kp, t, C.byref(s), C.byref(r)):
        return None
    return tuple(t), s.value, bool(r.value)


def tune_reset():
    lib().mxfp6_gemm_tune_reset()


def tune_save(path):
    """Writes the measured plans to `path`; returns how many."""
    n = C.c_int(0)
    rc = lib().mxfp6_gemm_tune_save(os.fsencode(path), C.byref(n))
    if rc != 0:
        raise OSError(f"mxfp6_gemm_tune_save({path}): {STATUS.get(rc, rc)}")
    return n.value


def tune_load(path):
    """Adds the plans of a tune_save file; returns (loaded, skipped)."""
    a, b = C.c_int(0), C.c_int(0)
    rc = lib().mxfp6_gemm_tune_load(os.fsencode(path), C.byref(a), C.byref(b))
    if rc != 0:
        raise OSError(f"mxfp6_gemm_tune_load({path}): {STATUS.get(rc, rc)}")
    return a.value, b.value


def gemm_plan(out_type, M, N, Kp, ws_bytes):
    """(tile, splits, a_repack) that gemm() runs for this shape with a workspace of ws_bytes."""
    t = (C.c_int * 4)()
    s, r = C.c_int(0), C.c_int(0)
    rc = lib().mxfp6_gemm_plan(out_type, M, N, Kp, ws_bytes, t, C.byref(s), C.byref(r))
    if rc != 0:
        raise ValueError(f"mxfp6_gemm_plan: {STATUS.get(rc, rc)}")
    return tuple(t), s.value, bool(r.value)


def streams_output(out_type, M, N, Kp, A_row_bytes):
    """Whether gemm()'s plan writes D with nontemporal stores for this call."""
    return bool(lib().mxfp6_gemm_streams_output(out_type, M, N, Kp, A_row_bytes))


def plan_workspace_size(M, N, Kp, splits, a_repack):
    return lib().mxfp6_plan_workspace_size(M, N, Kp, splits, int(a_repack))


def clock_sample(d_out, nwg, stream=None):
    """mxfp6_clock_sample_async: nwg x 4 uint64 records (cycles, 100 MHz reference, XCD, HW id)."""
    return lib().mxfp6_clock_sample_async(d_out, nwg, stream)


def clock_between(a, b):
    """Mean graphics clock (MHz) per XCD between two clock samples a and b (uint64 arrays of
    shape [nwg, 4] from clock_sample): for each CU seen in both samples, its cycle difference over
    its reference difference times 100 MHz, averaged over the XCD's CUs. Returns {xcd: MHz}."""
    import numpy as np

    def per_cu(s):
        d = {}
        for cyc, ref, xcc, hw in np.asarray(s, dtype=np.uint64).tolist():
            d[(int(xcc), (int(hw) >> 8) & 0xFF)] = (int(cyc), int(ref))
        return d

    da, db = per_cu(a), per_cu(b)
    acc = {}
    for key in da.keys() & db.keys():
        (c0, r0), (c1, r1) = da[key], db[key]
        if r1 > r0:
            acc.setdefault(key[0], []).append((c1 - c0) / (r1 - r0) * 100.0)
    return {x: sum(v) / len(v) for x, v in sorted(acc.items())}


def preshuffle_rows(src, row_bytes, rows, Kp, dst, stream=None):
    """On-device preshuffle of row-major packed rows (device pointers), preshuffle_B's layout."""
    return lib().mxfp6_preshuffle_rows_async(src, row_bytes, rows, Kp, dst, stream)


def quantize_dev(dx, rows, cols, dpacked, packed_row_bytes, dscales, scale_cols, stream=None):
    """quantize_to_mxfp6 on the device (device pointers); returns the status."""
    return lib().mxfp6_quantize_async(dx, rows, cols, dpacked, packed_row_bytes, dscales,
                                      scale_cols, stream)


def prepare_a_dev(dA, M, K, group, dpacked, a_row_bytes, dtiled, stream=None):
    """float A[M][K] -> packed rows + tiled scales at kpad(K) on the device; returns the status."""
    return lib().mxfp6_prepare_a_async(dA, M, K, group, dpacked, a_row_bytes, dtiled, stream)


def prepare_a_preshuffled_dev(dA, M, K, group, dash, dtiled, stream=None):
    return lib().mxfp6_prepare_a_preshuffled_async(dA, M, K, group, dash, dtiled, stream)


def prepare_b_dev(dB, K, N, group, dbsh, dtiled, stream=None):
    """float B[K][N] -> preshuffled B^T + tiled scales at kpad(K) on the device; returns the
    status."""
    return lib().mxfp6_prepare_b_async(dB, K, N, group, dbsh, dtiled, stream)


def tile_scales_dev(dscales, dim, K, ld, group, dtiled, stream=None):
    """Raw scales [dim][ld] -> tiled at kpad(K) on the device; returns the status."""
    return lib().mxfp6_tile_scales_async(dscales, dim, K, ld, group, dtiled, stream)


def preshuffled_bytes(dim, K):
    return lib().mxfp6_preshuffled_bytes(dim, K)


def tiled_scale_bytes(dim, K, group):
    return lib().mxfp6_tiled_scale_bytes(dim, K, group)


def gemm_direct(out_type, M, N, Kp, mpw, npw, dA, dBsh, dsA, dsB, dD, A_row_bytes, splits=1,
                ws=0, ws_bytes=0, stream=None):
    return lib().mxfp6_gemm_direct(out_type, M, N, Kp, mpw, npw, dA, dBsh, dsA, dsB, dD,
                                   A_row_bytes, splits, ws or None, ws_bytes, stream)


# ---- host formats -------------------------------------------------------------------------------

def gen_operand(rows: int, K: int, dist: int, sigma: float, seed: int, stream: int,
                row_bytes: int | None = None, scale_cols: int | None = None,
                nthreads: int = 0, extra_bytes: int = 0):
    """(packed uint8 [rows*row_bytes + extra_bytes], scales uint8 [rows, scale_cols])."""
    row_bytes = packed_bytes(K) if row_bytes is None else row_bytes
    scale_cols = K // 32 if scale_cols is None else scale_cols
    packed = np.zeros(rows * row_bytes + extra_bytes, dtype=np.uint8)
    scales = np.empty((rows, scale_cols), dtype=np.uint8)
    _check(lib().mxfp6_gen_operand(rows, K, dist, sigma, seed, stream, _ptr(packed), row_bytes,
                                   _ptr(scales), scale_cols, nthreads), "gen_operand")
    return packed, scales


def gen_values(rows: int, K: int, dist: int, sigma: float, seed: int, stream: int,
               nthreads: int = 0) -> np.ndarray:
    out = np.empty((rows, K), dtype=np.float32)
    _check(lib().mxfp6_gen_values(rows, K, dist, sigma, seed, stream, _ptr(out), nthreads),
           "gen_values")
    return out


def prepare_b(packed: np.ndarray, N: int, Kp: int, row_bytes: int, nthreads: int = 0) -> np.ndarray:
    """Preshuffled B^T: ceil(N/32) tiles of 32 columns (zero codes past N)."""
    out = np.empty(-(-N // 32) * (Kp // 64) * 1536, dtype=np.uint8)
    _check(lib().mxfp6_prepare_b(_ptr(packed), N, Kp, row_bytes, _ptr(out), nthreads),
           "prepare_b")
    return out


def prepare_scales(scales: np.ndarray, dim: int, Kp: int, group: int, nthreads: int = 0) -> np.ndarray:
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    assert scales.size == dim * (Kp // 32)
    out = np.empty(tiled_scale_bytes(dim, Kp, group), dtype=np.uint8)
    _check(lib().mxfp6_prepare_scales(_ptr(scales), dim, Kp, group, _ptr(out), nthreads),
           "prepare_scales")
    return out


def quantize(mat: np.ndarray):
    mat = np.ascontiguousarray(mat, dtype=np.float32)
    rows, cols = mat.shape
    packed = np.empty(rows * packed_bytes(cols), dtype=np.uint8)
    scales = np.empty((rows, cols // 32), dtype=np.uint8)
    _check(lib().mxfp6_quantize(_ptr(mat), rows, cols, _ptr(packed), _ptr(scales)), "quantize")
    return packed, scales


def dequantize(packed: np.ndarray, scales: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.float32)
    _check(lib().mxfp6_dequantize(_ptr(np.ascontiguousarray(packed)),
                                  _ptr(np.ascontiguousarray(scales)), rows, cols, _ptr(out)),
           "dequantize")
    return out


def preprocess_b(B: np.ndarray):
    B = np.ascontiguousarray(B, dtype=np.float32)
    K, N = B.shape
    packed = np.empty(N * packed_bytes(K), dtype=np.uint8)
    scales = np.empty((N, K // 32), dtype=np.uint8)
    _check(lib().mxfp6_preprocess_b(_ptr(B), K, N, _ptr(packed), _ptr(scales)), "preprocess_b")
    return packed, scales


def preprocess_scale(scales: np.ndarray, dim: int, K: int) -> np.ndarray:
    out = np.empty((dim // 32) * (K // 64) * 64, dtype=np.uint8)
    _check(lib().mxfp6_preprocess_scale(_ptr(np.ascontiguousarray(scales)), dim, K, _ptr(out)),
           "preprocess_scale")
    return out


def tile_scale(pscale: np.ndarray, dim: int, K: int, group: int, subs: int = 3) -> np.ndarray:
    out = np.empty(lib().mxfp6_tile_scale_bytes(dim, K, group, subs), dtype=np.uint8)
    _check(lib().mxfp6_tile_scale(_ptr(np.ascontiguousarray(pscale)), dim, K, group, subs,
                                  _ptr(out)), "tile_scale")
    return out


def preshuffle_b(packed: np.ndarray, N: int, K: int, row_bytes: int | None = None) -> np.ndarray:
    row_bytes = packed_bytes(K) if row_bytes is None else row_bytes
    out = np.empty((N // 32) * (K // 64) * 1536, dtype=np.uint8)
    _check(lib().mxfp6_preshuffle_b(_ptr(np.ascontiguousarray(packed)), N, K, row_bytes,
                                    _ptr(out)), "preshuffle_b")
    return out


def pad_scales_k(scales: np.ndarray, dim: int, K: int) -> np.ndarray:
    out = np.empty((dim, kpad(K) // 32), dtype=np.uint8)
    _check(lib().mxfp6_pad_scales_k(_ptr(np.ascontiguousarray(scales)), dim, K, _ptr(out)),
           "pad_scales_k")
    return out


# ---- a whole GEMM problem -------------------------------------------------------------------------

@dataclass
class Problem:
    """Host operands of D[M,N] = A[M,K] B[K,N] in the public layouts.

    a_packed: compact A rows (A_row_bytes = packed(K)) + a_compact_end_pad(K) bytes, or padded
    rows of packed(Kp) when compact=False; a_scales [M][Kp/32] (tail 127);
    b_packed: B^T rows [N][packed(Kp)] with zero K-tail; b_scales [N][Kp/32] (tail 127).
    """
    M: int
    N: int
    K: int
    Kp: int
    a_packed: np.ndarray
    a_scales: np.ndarray
    a_row_bytes: int
    b_packed: np.ndarray
    b_scales: np.ndarray
    tiles: dict = field(default_factory=dict)

    @property
    def b_row_bytes(self) -> int:
        return packed_bytes(self.Kp)

    def a_codes_view(self) -> np.ndarray:
        """A packed codes as [M][packed(K)] (drops the end pad / K-tail)."""
        pk = packed_bytes(self.K)
        return np.lib.stride_tricks.as_strided(
            self.a_packed, shape=(self.M, pk), strides=(self.a_row_bytes, 1))

    def b_codes_view(self) -> np.ndarray:
        return self.b_packed.reshape(self.N, self.b_row_bytes)[:, :packed_bytes(self.K)]

    def layouts(self, tile, nthreads: int = 0):
        """(bsh, sa_tiled, sb_tiled) for a tile (MT, NT, MPW, NPW); cached per scale grouping."""
        key = (tile[2], tile[3])
        if "bsh" not in self.tiles:
            self.tiles["bsh"] = prepare_b(self.b_packed, self.N, self.Kp, self.b_row_bytes, nthreads)
        if key not in self.tiles:
            self.tiles[key] = (prepare_scales(self.a_scales, self.M, self.Kp, tile[2], nthreads),
                               prepare_scales(self.b_scales, self.N, self.Kp, tile[3], nthreads))
        return (self.tiles["bsh"],) + self.tiles[key]


def make_problem(M: int, N: int, K: int, dist_a=DIST_NORMAL, sigma_a=1.0, dist_b=DIST_NORMAL,
                 sigma_b=1.0, seed: int = 0x4D584636, compact: bool = True,
                 nthreads: int = 0) -> Problem:
    """Synthetic operands: A from PCG32 stream 1, B^T from stream 2 of `seed`."""
    Kp = kpad(K)
    if compact:
        a_row = packed_bytes(K)
        a_packed, a_sc = gen_operand(M, K, dist_a, sigma_a, seed, 1, a_row, Kp // 32, nthreads,
                                     extra_bytes=a_compact_end_pad(K))
    else:
        a_row = packed_bytes(Kp)
        a_packed, a_sc = gen_operand(M, K, dist_a, sigma_a, seed, 1, a_row, Kp // 32, nthreads)
    b_packed, b_sc = gen_operand(N, K, dist_b, sigma_b, seed, 2, packed_bytes(Kp), Kp // 32,
                                 nthreads)
    return Problem(M, N, K, Kp, a_packed, a_sc, a_row, b_packed, b_sc)
