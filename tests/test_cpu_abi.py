"""The C-ABI library loads and exports every symbol include/*.h declares (no GPU needed);
argument checks reject bad calls before any device work."""
import glob
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(mxfp6_\w+)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_entry_points():
    d = _declared()
    for n in ("mxfp6_gemm", "mxfp6_choose_tile", "mxfp6_gemm_workspace_size", "mxfp6_kpad",
              "mxfp6_gemm_force_tile", "mxfp6_preshuffle_b", "mxfp6_tile_scale"):
        assert n in d


def test_library_exports_every_declared_symbol(mx):
    out = subprocess.run(["nm", "-D", "--defined-only", mx.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = sorted(_declared() - exported)
    assert not missing, missing
    # the binding covers every declared symbol too
    assert _declared() <= set(mx.SIGNATURES)


def test_cpp_drop_in_symbols_exported(mx):
    out = subprocess.run(["nm", "-D", "-C", "--defined-only", mx.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    for sig in ("mxfp6::choose_tile(int, int, int)", "mxfp6::gemm_workspace_size(int, int, int)",
                "mxfp6::gemm(mxfp6::OutType, int, int, int, void const*, void const*, "
                "unsigned char const*, unsigned char const*, void*, int, int, void*, unsigned long)",
                "mxfp6::gemm_force_tile(mxfp6::OutType, int, int, int, mxfp6::TileChoice, "
                "void const*, void const*, unsigned char const*, unsigned char const*, void*, "
                "int, int)"):
        assert sig in out, sig


def test_argument_checks_reject_before_launch(mx):
    p = 0x1000  # never dereferenced: every call below must fail validation first
    assert mx.gemm(0, 128, 128, 192, 0, p, p, p, p, 144) == 1            # null A
    assert mx.gemm(3, 128, 128, 192, p, p, p, p, p, 144) == 3            # bad out type
    assert mx.gemm(0, 0, 128, 192, p, p, p, p, p, 144) == 2              # M = 0
    assert mx.gemm(0, 128, -5, 192, p, p, p, p, p, 144) == 2             # N < 0
    assert mx.gemm(0, 128, 128, 200, p, p, p, p, p, 144) == 2            # Kp % 192
    assert mx.gemm(0, 128, 128, 192, p, p, p, p, p, 6) == 2              # A row too short
    assert mx.gemm(0, 128, 128, 192, p, p, p, p, p, 146) == 2            # A row misaligned
    assert mx.gemm_force_tile(0, 128, 128, 192, (128, 384, 4, 3), p, p, p, p, p, 144) == 4
    assert mx.gemm_force_tile(0, 256, 256, 192, (256, 128, 4, 2), p, p, p, p, p, 144) == 4  # not instantiated
    assert mx.gemm_force_tile(0, 100, 128, 192, (128, 128, 2, 2), p, p, p, p, p, 144) == 4  # ragged
    assert mx.gemm_explicit(0, 100, 100, 192, (256, 128, 4, 2), 1, p, p, p, p, p, 144) == 4
    assert mx.gemm_explicit(0, 100, 100, 192, (128, 128, 2, 2), 2, p, p, p, p, p, 144) == 5  # no ws
    # the swizzled staging of row-major A: wide tiles that divide M x N only, and no layout past it
    sw = mx.A_ROWS_SWIZZLED
    assert mx.gemm_explicit(0, 256, 256, 192, (128, 128, 2, 2), 1, p, p, p, p, p, 144,
                            a_layout=sw) == 5                                        # slab tile
    assert mx.gemm_explicit(0, 256, 384, 192, (256, 256, 4, 2), 1, p, p, p, p, p, 144,
                            a_layout=sw) == 5                                        # masked N
    assert mx.gemm_explicit(0, 200, 512, 192, (128, 512, 4, 4), 1, p, p, p, p, p, 144,
                            a_layout=sw) == 5                                        # masked M
    assert mx.gemm_explicit(0, 256, 256, 192, (256, 256, 4, 2), 1, p, p, p, p, p, 144,
                            a_layout=sw + 1) == 5                                    # no layout 4
    # the 32 x 32 tile: at most 16 segments of at most 4 K-tiles, row-major A
    assert mx.gemm_explicit(0, 256, 256, 1152, (32, 32, 1, 1), 1, p, p, p, p, p, 864) == 5  # 6 > 4
    assert mx.gemm_explicit(0, 256, 256, 3456, (32, 32, 1, 1), 4, p, p, p, p, p, 2592,
                            ws=p, ws_bytes=1 << 30) == 5                             # 18 in 4
    assert mx.gemm_explicit(0, 256, 256, 12480, (32, 32, 1, 1), 16, p, p, p, p, p, 9360,
                            ws=p, ws_bytes=1 << 30) == 5                             # 65 in 16
    assert mx.gemm_explicit(0, 256, 256, 13056, (32, 32, 1, 1), 17, p, p, p, p, p, 9792,
                            ws=p, ws_bytes=1 << 30) == 5                             # 17 segments
    assert mx.gemm_explicit(0, 256, 256, 576, (32, 32, 1, 1), 1, p, p, p, p, p, 432,
                            a_layout=mx.A_REPACK, ws=p, ws_bytes=1 << 30) == 5       # repack
    assert mx.gemm_force_tile(0, 256, 256, 1152, (32, 32, 1, 1), p, p, p, p, p, 864) == 4
    assert mx.gemm_direct(0, 128, 128, 192, 5, 2, p, p, p, p, p, 144) == 5
    assert mx.gemm_direct(0, 128, 128, 192, 2, 2, p, p, p, p, p, 144, splits=2) == 5
    assert mx.gemm_direct(0, 96, 128, 192, 1, 1, p, p, p, p, p, 144) == 2   # M % 64
    assert mx.gemm_direct(0, 128, 100, 192, 1, 1, p, p, p, p, p, 144) == 2  # N % 64


def test_prep_argument_checks_reject_before_launch(mx):
    p = 0x1000  # 16-byte aligned, never dereferenced
    assert mx.quantize_dev(0, 4, 64, p, 48, p, 2) == 1                  # null input
    assert mx.quantize_dev(p, 0, 48, p, 48, p, 2) == 2                  # no rows
    assert mx.quantize_dev(p, 4, 64, p, 44, p, 2) == 2                  # row shorter than codes
    assert mx.quantize_dev(p, 4, 40, p, 44, p, 2) == 2                  # ragged K: 2 blocks
    assert mx.quantize_dev(p, 4, 64, p, 50, p, 2) == 2                  # row stride % 4
    assert mx.quantize_dev(p, 4, 40, p, 48, p, 1) == 2                  # too few scale columns
    assert mx.quantize_dev(p + 2, 4, 64, p, 48, p, 2) == 5              # input not 4-byte aligned
    assert mx.prepare_a_dev(p, 0, 64, 2, p, 48, p) == 2                 # M = 0
    assert mx.prepare_a_dev(p, 96, 40, 2, p, 44, p) == 2                # row shorter than codes
    assert mx.prepare_a_dev(p, 128, 64, 5, p, 48, p) == 5               # group
    assert mx.prepare_a_preshuffled_dev(0, 64, 64, 2, p, p) == 1        # null input
    assert mx.prepare_a_preshuffled_dev(p, 0, 64, 2, p, p) == 2         # M = 0
    assert mx.prepare_a_preshuffled_dev(p, 64, 64, 0, p, p) == 5        # group
    assert mx.prepare_a_preshuffled_dev(p, 64, 64, 2, p + 8, p) == 5    # A^sh not 16-byte aligned
    assert mx.prepare_b_dev(p, 64, 0, 2, p, p) == 2                     # N = 0
    assert mx.prepare_b_dev(p, -1, 64, 2, p, p) == 2                    # K < 0
    assert mx.prepare_b_dev(p, 64, 64, 2, p + 8, p) == 5                # Bsh not 16-byte aligned
    assert mx.tile_scales_dev(p, 64, 64, 1, 2, p) == 2                  # ld < ceil(K/32)
    assert mx.tile_scales_dev(p, 64, 40, 1, 2, p) == 2
    assert mx.tile_scales_dev(0, 64, 64, 2, 2, p) == 1
    # layout sizes at kpad(K); ragged dims round up to 32-row blocks and whole scale groups
    assert mx.preshuffled_bytes(0, 64) == 0
    assert mx.preshuffled_bytes(64, 1000) == 2 * (1152 // 64) * 1536
    assert mx.preshuffled_bytes(50, 992) == 2 * (1152 // 64) * 1536
    assert mx.tiled_scale_bytes(96, 992, 3) == 1 * (1152 // 192) * 64 * 3 * 4
    assert mx.tiled_scale_bytes(96, 992, 2) == 2 * (1152 // 192) * 64 * 3 * 4
    assert mx.tiled_scale_bytes(1, 33, 4) == 1 * 1 * 64 * 3 * 4


def test_tile_scale_rejects_partial_groups(mx):
    """The C ABI's tile_scale (the header's floor-over-groups layout) accepts only groupings that
    divide dim/32: a partial last group would be dropped, and a masked tile reads it."""
    import ctypes as C
    import numpy as np
    assert mx.lib().mxfp6_tile_scale_bytes(416, 192, 3, 3) == 0       # 13 blocks, group 3
    assert mx.lib().mxfp6_tile_scale_bytes(384, 192, 3, 3) == 4 * 1 * 64 * 3 * 4
    buf = np.zeros(1 << 16, dtype=np.uint8)
    ptr = buf.ctypes.data_as(C.c_void_p)
    assert mx.lib().mxfp6_tile_scale(ptr, 416, 192, 3, 3, ptr) == 5
    assert mx.lib().mxfp6_tile_scale(ptr, 384, 192, 3, 3, ptr) == 0


def test_noalloc_rejects_before_device_work(mx):
    """mxfp6_gemm_noalloc_async checks its arguments, then that the plan's split-K partials fit
    its scratch, before touching the device: a shape whose partials exceed the 128 MiB scratch is
    rejected with MXFP6_ERR_SCRATCH."""
    p = 0x1000  # never dereferenced
    Kp = mx.kpad(105728)
    rb = Kp // 4 * 3
    assert mx.gemm_noalloc(0, 4096, 6144, Kp, 0, p, p, p, p, rb) == 1      # null A
    assert mx.gemm_noalloc(5, 4096, 6144, Kp, p, p, p, p, p, rb) == 3      # bad out type
    assert mx.workspace_size(4096, 6144, Kp) > mx.NOALLOC_SCRATCH_BYTES
    assert mx.gemm_noalloc(1, 4096, 6144, Kp, p, p, p, p, p, rb) == 7      # partials too large
