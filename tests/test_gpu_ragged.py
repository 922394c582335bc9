"""GPU parity on ragged shapes: M not a multiple of 32, N not a multiple of 128, K not a multiple
of 32 (the reference needs M and N multiples of 128 and K of 32; README.md:265-279).

The library runs such shapes on masked tiles (grid ceil(M/MT) x ceil(N/NT); copies past the last
row, 32-row block or scale group of an operand repeat the last one; stores only inside M x N)
over operand layouts extended with zero rows: ceil(N/32) preshuffled 32-column tiles, scales
tiled over whole groups of 32 * group rows with code 127 for the added rows. A K that is not a
multiple of 32 is quantised as if zero-padded to one.

Expected values come from the oracle on the zero-padded operands: the ragged layouts must equal
the reference layouts (oracle restatements of preprocess_B, pad_scales_k, preprocess_scale,
preshuffle_B, tile_scale) of the operand padded with zero rows / columns, and D must match the
FP64 oracle GEMM of the quantised operands to the usual bar (tests/checks.py). Every D and
workspace buffer carries a guard region past its end, filled with a pattern that must survive
the call (a masked store or copy that escapes the shape fails the test).
"""
import numpy as np
import pytest
import torch

import checks
import mxfp6_amd as mx
import oracle
from gpu_util import DevProblem, TORCH_OUT, say

pytestmark = pytest.mark.gpu

GUARD = 4096
TILES = [(256, 256, 4, 4), (256, 256, 2, 4), (256, 192, 4, 3), (128, 384, 4, 3),
         (128, 256, 2, 4), (128, 128, 2, 2), (64, 256, 2, 2), (32, 256, 1, 2), (64, 128, 2, 1),
         (32, 128, 1, 1)]


def _kpad(K):
    return (K + 191) // 192 * 192


def _buf(nbytes, fill):
    return torch.full((nbytes + GUARD,), fill, dtype=torch.uint8, device="cuda")


def _guard_ok(t, nbytes, fill, what):
    tail = t[nbytes:].cpu().numpy()
    assert (tail == fill).all(), f"{what}: bytes written past the end"


def _gemm(dp, out_type, explicit=None, splits=1, a_layout=0, a_dev=None):
    """Routed gemm (explicit None) or the explicit plan (tile, splits, a_layout); D as float32."""
    p = dp.p
    n = p.M * p.N * mx.OUT_BYTES[out_type]
    if explicit is None:
        ws_bytes = mx.preferred_workspace_size(p.M, p.N, p.Kp)
    else:
        ws_bytes = mx.plan_workspace_size(p.M, p.N, p.Kp, splits, a_layout == 1)
    D = _buf(n, 0x5A)
    ws = _buf(max(ws_bytes, 4), 0x3C)
    a, b, sa, sb = dp.ptrs()
    if a_dev is not None:
        a = a_dev.data_ptr()
    say(f"  {'routed' if explicit is None else explicit} {p.M}x{p.N}x{p.K} (Kp {p.Kp}) out "
        f"{mx.OUT_NAMES[out_type]} S {splits} A {a_layout} ws {ws_bytes}")
    if explicit is None:
        rc = mx.gemm(out_type, p.M, p.N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes,
                     ws.data_ptr(), ws_bytes)
    else:
        rc = mx.gemm_explicit(out_type, p.M, p.N, p.Kp, explicit, splits, a, b, sa, sb,
                              D.data_ptr(), p.a_row_bytes, ws.data_ptr() if ws_bytes else 0,
                              ws_bytes, a_layout=a_layout)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    _guard_ok(D, n, 0x5A, "D")
    _guard_ok(ws, max(ws_bytes, 4), 0x3C, "workspace")
    return D[:n].view(TORCH_OUT[out_type]).float().reshape(p.M, p.N).cpu().numpy()


def _rows(M, cap=48):
    """Every row of a small M; for a large one the first, last and a spread of rows between."""
    if M <= cap:
        return None
    return np.unique(np.r_[0:4, M - 4:M, np.linspace(0, M - 1, cap - 8).astype(int)])


def _check(D, p, out_type):
    rows = _rows(p.M)
    R, ab = oracle.problem_f64(p, rows=rows)
    checks.check(D if rows is None else D[rows], R, ab, out_type)


# ---- routed gemm() on ragged M x N ------------------------------------------------------------

RAGGED = [(1, 1, 64), (7, 50, 192), (33, 100, 992), (100, 129, 2048), (127, 300, 4096),
          (200, 1000, 1056), (257, 8191, 1024), (4095, 129, 8192), (77, 300, 32768),
          (300, 77, 65536), (8191, 8191, 1024), (3000, 5000, 4096)]


@pytest.mark.parametrize("out_type", [0, 1, 2])
@pytest.mark.parametrize("M,N,K", RAGGED)
def test_routed_ragged(out_type, M, N, K):
    p = mx.make_problem(M, N, K, seed=M * 7 + N * 3 + K)
    t = mx.choose_tile(M, N, p.Kp)
    D = _gemm(DevProblem(p, t), out_type)
    _check(D, p, out_type)


# ---- every tile masked, every A layout, unsplit and split ---------------------------------------

@pytest.mark.parametrize("tile", TILES)
def test_every_tile_masked(tile):
    """M and N leave a partial last tile row and column for every tile; row-major, repacked and
    preshuffled A give the same bits unsplit, and the split runs match the oracle."""
    M, N, K = 289, 419, 2080  # 11 K-tiles; M = 9 * 32 + 1, N = 3 * 128 + 35
    p = mx.make_problem(M, N, K, dist_a=mx.DIST_STUDENT_T3, dist_b=mx.DIST_STUDENT_T3, seed=5)
    checks.spread_scales(p, seed=5)  # FP32 bits that depend on the K order
    dp = DevProblem(p, tile)
    ash = torch.empty(mx.preshuffled_bytes(M, K), dtype=torch.uint8, device="cuda")
    assert mx.preshuffle_rows(dp.a.data_ptr(), p.a_row_bytes, M, p.Kp, ash.data_ptr()) == 0
    D0 = _gemm(dp, 0, explicit=tile)
    _check(D0, p, 0)
    for a_layout, a_dev in ((1, None), (2, ash)):
        D = _gemm(dp, 0, explicit=tile, a_layout=a_layout, a_dev=a_dev)
        assert np.array_equal(D.view(np.uint32), D0.view(np.uint32)), a_layout
    for out_type in (1, 2):
        _check(_gemm(dp, out_type, explicit=tile, splits=4, a_layout=1), p, out_type)


# ---- device quantisation and layouts on ragged sizes ----------------------------------------

def _padded(x, rows, cols):
    z = np.zeros((rows, cols), np.float32)
    z[:x.shape[0], :x.shape[1]] = x
    return z


def _expected_a(x, M, K, group):
    """Packed rows (first M, of packed(kpad K) bytes) and tiled scales of x zero-padded to whole
    scale groups of rows and to a multiple of 32 values."""
    Kp, K32 = _kpad(K), -(-K // 32) * 32
    MG = -(-M // (32 * group)) * (32 * group)
    po, so = oracle.quantize_ref(_padded(x, MG, K32))
    rows = np.zeros((MG, Kp // 4 * 3), np.uint8)
    rows[:, :K32 // 4 * 3] = po.reshape(MG, -1)
    tiled = oracle.tile_scale(oracle.preprocess_scale(oracle.pad_scales_k(so, MG, K32), MG, Kp),
                              MG, Kp, group)
    return rows[:M], tiled


def _expected_b(B, K, N, group):
    """Preshuffled B^T (ceil(N/32) tiles) and tiled scales of B zero-padded the same way."""
    Kp, K32 = _kpad(K), -(-K // 32) * 32
    NG = -(-N // (32 * group)) * (32 * group)
    N32 = -(-N // 32) * 32
    po, so = oracle.quantize_ref(_padded(np.ascontiguousarray(B.T), NG, K32))
    rows = np.zeros((NG, Kp // 4 * 3), np.uint8)
    rows[:, :K32 // 4 * 3] = po.reshape(NG, -1)
    bsh = oracle.preshuffle_b(np.ascontiguousarray(rows[:N32]), N32, Kp, Kp // 4 * 3)
    tiled = oracle.tile_scale(oracle.preprocess_scale(oracle.pad_scales_k(so, NG, K32), NG, Kp),
                              NG, Kp, group)
    return bsh, tiled


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def _host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("M,K,group", [(1, 1, 1), (33, 40, 4), (100, 1000, 2), (127, 4097, 3),
                                       (65, 8190, 4)])
def test_prepare_a_ragged(M, K, group):
    say(f"prepare_a ragged M={M} K={K} group={group}")
    rng = np.random.default_rng(M * 31 + K)
    x = rng.standard_normal((M, K)).astype(np.float32) * np.float32(3.0)
    want_rows, want_t = _expected_a(x, M, K, group)
    rb = want_rows.shape[1]
    assert mx.tiled_scale_bytes(M, K, group) == want_t.size
    dp = _buf(M * rb, 0xA5)
    dt = _buf(want_t.size, 0xA5)
    assert mx.prepare_a_dev(_dev(x).data_ptr(), M, K, group, dp.data_ptr(), rb, dt.data_ptr()) == 0
    _guard_ok(dp, M * rb, 0xA5, "packed A")
    _guard_ok(dt, want_t.size, 0xA5, "tiled A scales")
    assert np.array_equal(_host(dp[:M * rb]).reshape(M, rb), want_rows)
    assert np.array_equal(_host(dt[:want_t.size]), want_t)


@pytest.mark.parametrize("K,N,group", [(1, 1, 1), (40, 33, 4), (1000, 100, 2), (4097, 129, 3),
                                       (8190, 65, 4)])
def test_prepare_b_ragged(K, N, group):
    say(f"prepare_b ragged K={K} N={N} group={group}")
    rng = np.random.default_rng(K * 7 + N)
    B = rng.standard_normal((K, N)).astype(np.float32)
    want_b, want_t = _expected_b(B, K, N, group)
    assert mx.preshuffled_bytes(N, K) == want_b.size
    assert mx.tiled_scale_bytes(N, K, group) == want_t.size
    db = _buf(want_b.size, 0xA5)
    dt = _buf(want_t.size, 0xA5)
    assert mx.prepare_b_dev(_dev(B).data_ptr(), K, N, group, db.data_ptr(), dt.data_ptr()) == 0
    _guard_ok(db, want_b.size, 0xA5, "preshuffled B")
    _guard_ok(dt, want_t.size, 0xA5, "tiled B scales")
    assert np.array_equal(_host(db[:want_b.size]), want_b)
    assert np.array_equal(_host(dt[:want_t.size]), want_t)


@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 33), (9, 1001), (3, 4094), (4, 40), (2, 4100)])
def test_quantize_ragged_cols(rows, cols):
    """Raw quantisation of a row length that is not a multiple of 32 (scalar or float4 loads)."""
    say(f"quantize ragged rows={rows} cols={cols}")
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    nb = -(-cols // 32)
    po, so = oracle.quantize_ref(_padded(x, rows, nb * 32))
    rb, sc = nb * 24 + 8, nb + 2
    dp = _buf(rows * rb, 0xA5)
    ds = _buf(rows * sc, 0xA5)
    assert mx.quantize_dev(_dev(x).data_ptr(), rows, cols, dp.data_ptr(), rb, ds.data_ptr(),
                           sc) == 0
    _guard_ok(dp, rows * rb, 0xA5, "packed")
    _guard_ok(ds, rows * sc, 0xA5, "scales")
    got_p = _host(dp[:rows * rb]).reshape(rows, rb)
    got_s = _host(ds[:rows * sc]).reshape(rows, sc)
    assert np.array_equal(got_p[:, :nb * 24], po.reshape(rows, -1))
    assert not got_p[:, nb * 24:].any()
    assert np.array_equal(got_s[:, :nb], so)
    assert (got_s[:, nb:] == 127).all()


@pytest.mark.parametrize("dim,K,ld,group", [(1, 1, 1, 1), (33, 40, 2, 4), (100, 1000, 40, 3)])
def test_tile_scales_ragged(dim, K, ld, group):
    say(f"tile_scales ragged dim={dim} K={K} ld={ld} group={group}")
    rng = np.random.default_rng(dim * 3 + K)
    raw = rng.integers(0, 255, size=(dim, ld), dtype=np.uint8)
    Kp, nb = _kpad(K), -(-K // 32)
    G = -(-dim // (32 * group)) * (32 * group)
    full = np.full((G, nb), 127, np.uint8)
    full[:dim] = raw[:, :nb]
    want = oracle.tile_scale(oracle.preprocess_scale(oracle.pad_scales_k(full, G, nb * 32), G, Kp),
                             G, Kp, group)
    dt = _buf(want.size, 0xA5)
    assert mx.tile_scales_dev(_dev(raw.reshape(-1)).data_ptr(), dim, K, ld, group,
                              dt.data_ptr()) == 0
    _guard_ok(dt, want.size, 0xA5, "tiled scales")
    assert np.array_equal(_host(dt[:want.size]), want)


@pytest.mark.parametrize("M,N,K,out_type", [(45, 77, 1000, 0), (300, 260, 3001, 1),
                                            (1, 129, 33, 2)])
def test_gemm_on_device_prepared_ragged(M, N, K, out_type):
    """Float operands of any size -> device preparation -> routed gemm; D matches the FP64 oracle
    of the same quantised operands (zero-padded to 32-value blocks)."""
    say(f"device-prepared ragged gemm {M}x{N}x{K} out {out_type}")
    Kp, K32 = _kpad(K), -(-K // 32) * 32
    t = mx.choose_tile(M, N, Kp)
    rng = np.random.default_rng(M + N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    rb = Kp // 4 * 3
    da = torch.empty(M * rb, dtype=torch.uint8, device="cuda")
    dsa = torch.empty(mx.tiled_scale_bytes(M, K, t[2]), dtype=torch.uint8, device="cuda")
    db = torch.empty(mx.preshuffled_bytes(N, K), dtype=torch.uint8, device="cuda")
    dsb = torch.empty(mx.tiled_scale_bytes(N, K, t[3]), dtype=torch.uint8, device="cuda")
    assert mx.prepare_a_dev(_dev(A).data_ptr(), M, K, t[2], da.data_ptr(), rb, dsa.data_ptr()) == 0
    assert mx.prepare_b_dev(_dev(B).data_ptr(), K, N, t[3], db.data_ptr(), dsb.data_ptr()) == 0
    ws_bytes = mx.preferred_workspace_size(M, N, Kp)
    ws = _buf(max(ws_bytes, 4), 0x3C)
    n = M * N * mx.OUT_BYTES[out_type]
    D = _buf(n, 0x5A)
    rc = mx.gemm(out_type, M, N, Kp, da.data_ptr(), db.data_ptr(), dsa.data_ptr(), dsb.data_ptr(),
                 D.data_ptr(), rb, ws.data_ptr(), ws_bytes)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    _guard_ok(D, n, 0x5A, "D")
    _guard_ok(ws, max(ws_bytes, 4), 0x3C, "workspace")
    Dh = D[:n].view(TORCH_OUT[out_type]).float().reshape(M, N).cpu().numpy()
    pa, sa = oracle.quantize_ref(_padded(A, M, K32))
    pb, sb = oracle.quantize_ref(_padded(np.ascontiguousarray(B.T), N, K32))
    R, ab = oracle.gemm_f64(pa, K32 // 4 * 3, sa, pb, K32 // 4 * 3, sb, M, N, K32)
    checks.check(Dh, R, ab, out_type)
