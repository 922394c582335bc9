"""GPU parity of the device quantisation and layout kernels against the oracle.

Every output is byte data and must be bit-identical to the oracle's restatement of the
reference's host functions (quantize_to_mxfp6, preprocess_B, pad_scales_k, preprocess_scale,
preshuffle_B, tile_scale; reference include/mxfp6/preprocess.hpp), which the CPU tests pin to
the reference library itself. When oracle/_ref is built, the quantiser is also compared with the
reference's own quantize_to_mxfp6 directly. The last test runs the GEMM on device-prepared
operands and requires the same D bits as on host-prepared ones.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import say

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _kpad(K):
    return (K + 191) // 192 * 192


def specials_matrix(rows, cols, seed):
    """Normal values with per-block magnitudes from 2^-140 to 2^120, plus blocks of special
    cases: zeros, subnormals, negative values that round to zero, E2M3 ties, saturation at the
    scale's rounding boundary, exact powers of two times 7.5."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    nb = cols // 32
    mag = np.exp2(rng.integers(-140, 121, size=(rows, nb))).astype(np.float32)
    x = (x.reshape(rows, nb, 32) * mag[:, :, None]).reshape(rows, cols).astype(np.float32)
    blocks = x.reshape(rows, nb, 32)
    specials = [
        np.zeros(32, np.float32),
        np.full(32, np.float32(1e-44)) * np.sign(rng.standard_normal(32)).astype(np.float32),
        np.concatenate([[np.float32(7.5)], -np.full(31, np.float32(0.01))]).astype(np.float32),
        (np.arange(32, dtype=np.float32) - 16) / 16,            # every k/16: ties between codes
        np.float32(7.5) * np.float32(1 + 2**-23) * np.ones(32, np.float32),  # need rounds to 1
        np.float32(7.5 * 2**-3) * np.linspace(-1, 1, 32).astype(np.float32),
        np.concatenate([[np.float32(3e38)], rng.standard_normal(31).astype(np.float32)]),
        -np.zeros(32, np.float32),
    ]
    for i, blk in enumerate(specials):
        r, b = divmod(i * 7 + 3, nb)
        if r < rows:
            blocks[r, b] = blk
    return x


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("rows,cols,pad_bytes,extra_cols", [
    (3, 32, 0, 0), (5, 2080, 0, 3), (7, 4160, 4, 0), (64, 8192, 96, 2), (33, 992, 8, 7),
])
def test_quantize_rows_equals_oracle(mx, rows, cols, pad_bytes, extra_cols):
    say(f"quantize rows={rows} cols={cols} pad={pad_bytes} extra={extra_cols}")
    x = specials_matrix(rows, cols, seed=rows * 1000 + cols)
    po, so = oracle.quantize_ref(x)
    r = oracle.ref()
    if r is not None:  # the reference's own quantize_to_mxfp6 on the same input
        pr = np.empty_like(po)
        sr = np.empty_like(so)
        r.ref_quantize(x.ctypes.data, rows, cols, pr.ctypes.data, sr.ctypes.data)
        assert np.array_equal(pr, po) and np.array_equal(sr, so)
    rb = cols // 4 * 3 + pad_bytes
    sc = cols // 32 + extra_cols
    dx = to_dev(x)
    dp = torch.full((rows * rb,), 0xA5, dtype=torch.uint8, device=DEV)
    ds = torch.full((rows * sc,), 0xA5, dtype=torch.uint8, device=DEV)
    assert mx.quantize_dev(dx.data_ptr(), rows, cols, dp.data_ptr(), rb, ds.data_ptr(), sc) == 0
    got_p = host(dp).reshape(rows, rb)
    got_s = host(ds).reshape(rows, sc)
    assert np.array_equal(got_p[:, :cols // 4 * 3], po.reshape(rows, -1))
    assert not got_p[:, cols // 4 * 3:].any()
    assert np.array_equal(got_s[:, :cols // 32], so)
    assert (got_s[:, cols // 32:] == 127).all()


@pytest.mark.parametrize("M,K,group,row_mode", [
    (32, 32, 1, "compact"), (128, 992, 4, "compact"), (96, 1024, 3, "padded"),
    (256, 2080, 2, "padded"), (64, 8256, 2, "compact"), (384, 192, 3, "padded"),
])
def test_prepare_a_equals_oracle(mx, M, K, group, row_mode):
    say(f"prepare_a M={M} K={K} group={group} rows={row_mode}")
    Kp = _kpad(K)
    x = specials_matrix(M, K, seed=M * 7 + K)
    po, so = oracle.quantize_ref(x)
    rb = K // 4 * 3 if row_mode == "compact" else Kp // 4 * 3
    want_p = np.zeros((M, rb), np.uint8)
    want_p[:, :K // 4 * 3] = po.reshape(M, -1)
    want_t = oracle.tile_scale(oracle.preprocess_scale(oracle.pad_scales_k(so, M, K), M, Kp),
                               M, Kp, group)
    assert mx.tiled_scale_bytes(M, K, group) == want_t.size
    dx = to_dev(x)
    dp = torch.full((M * rb,), 0xA5, dtype=torch.uint8, device=DEV)
    dt = torch.full((want_t.size,), 0xA5, dtype=torch.uint8, device=DEV)
    assert mx.prepare_a_dev(dx.data_ptr(), M, K, group, dp.data_ptr(), rb, dt.data_ptr()) == 0
    assert np.array_equal(host(dp).reshape(M, rb), want_p)
    assert np.array_equal(host(dt), want_t)


def expected_b(B, K, N, group):
    """preprocess_B, zero K-tail to kpad(K), preshuffle_B; scales padded and tiled."""
    Kp = _kpad(K)
    po, so = oracle.quantize_ref(np.ascontiguousarray(B.T))
    rows = np.zeros((N, Kp // 4 * 3), np.uint8)
    rows[:, :K // 4 * 3] = po.reshape(N, -1)
    bsh = oracle.preshuffle_b(rows, N, Kp, Kp // 4 * 3)
    tiled = oracle.tile_scale(oracle.preprocess_scale(oracle.pad_scales_k(so, N, K), N, Kp),
                              N, Kp, group)
    return bsh, tiled


@pytest.mark.parametrize("K,N,group", [
    (32, 32, 1), (192, 128, 4), (992, 96, 3), (1024, 256, 2), (2080, 64, 2), (8256, 384, 3),
])
def test_prepare_b_equals_oracle(mx, K, N, group):
    say(f"prepare_b K={K} N={N} group={group}")
    B = specials_matrix(K, N, seed=K * 3 + N)
    want_b, want_t = expected_b(B, K, N, group)
    assert mx.preshuffled_bytes(N, K) == want_b.size
    r = oracle.ref()
    if r is not None and K % 64 == 0 and K == _kpad(K):  # the reference's own preshuffle_B
        po, so = oracle.quantize_ref(np.ascontiguousarray(B.T))
        rb = np.empty_like(want_b)
        r.ref_preshuffle_b(po.ctypes.data, so.ctypes.data, N, K, rb.ctypes.data)
        assert np.array_equal(rb, want_b)
    dB = to_dev(B)
    db = torch.full((want_b.size,), 0xA5, dtype=torch.uint8, device=DEV)
    dt = torch.full((want_t.size,), 0xA5, dtype=torch.uint8, device=DEV)
    assert mx.prepare_b_dev(dB.data_ptr(), K, N, group, db.data_ptr(), dt.data_ptr()) == 0
    assert np.array_equal(host(db), want_b)
    assert np.array_equal(host(dt), want_t)


@pytest.mark.parametrize("dim,K,ld,group", [(32, 32, 1, 1), (128, 992, 40, 4), (96, 8256, 258, 3),
                                            (256, 2048, 64, 2)])
def test_tile_scales_equals_oracle(mx, dim, K, ld, group):
    say(f"tile_scales dim={dim} K={K} ld={ld} group={group}")
    rng = np.random.default_rng(dim + K)
    raw = rng.integers(0, 255, size=(dim, ld), dtype=np.uint8)
    Kp = _kpad(K)
    want = oracle.tile_scale(
        oracle.preprocess_scale(oracle.pad_scales_k(np.ascontiguousarray(raw[:, :K // 32]), dim, K),
                                dim, Kp), dim, Kp, group)
    ds = to_dev(raw.reshape(-1))
    dt = torch.full((want.size,), 0xA5, dtype=torch.uint8, device=DEV)
    assert mx.tile_scales_dev(ds.data_ptr(), dim, K, ld, group, dt.data_ptr()) == 0
    assert np.array_equal(host(dt), want)


@pytest.mark.parametrize("M,N,K,out_type", [(256, 512, 2080, 1), (512, 1024, 4096, 2)])
def test_gemm_on_device_prepared_operands(mx, M, N, K, out_type):
    """D from device-prepared A and B equals D from the same operands prepared on the host."""
    say(f"gemm on device-prepared operands {M}x{N}x{K} out {out_type}")
    Kp = _kpad(K)
    tile = mx.choose_tile(M, N, Kp)
    rng = np.random.default_rng(M + N + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    # host preparation through the oracle
    pa, sa = oracle.quantize_ref(A)
    a_rows = np.zeros((M, Kp // 4 * 3), np.uint8)
    a_rows[:, :K // 4 * 3] = pa.reshape(M, -1)
    sa_t = oracle.tile_scale(oracle.preprocess_scale(oracle.pad_scales_k(sa, M, K), M, Kp),
                             M, Kp, tile[2])
    bsh, sb_t = expected_b(B, K, N, tile[3])
    rb = Kp // 4 * 3
    # device preparation
    dA, dB = to_dev(A), to_dev(B)
    da = torch.empty(M * rb, dtype=torch.uint8, device=DEV)
    dsa = torch.empty(sa_t.size, dtype=torch.uint8, device=DEV)
    db = torch.empty(bsh.size, dtype=torch.uint8, device=DEV)
    dsb = torch.empty(sb_t.size, dtype=torch.uint8, device=DEV)
    assert mx.prepare_a_dev(dA.data_ptr(), M, K, tile[2], da.data_ptr(), rb, dsa.data_ptr()) == 0
    assert mx.prepare_b_dev(dB.data_ptr(), K, N, tile[3], db.data_ptr(), dsb.data_ptr()) == 0
    ws_bytes = mx.preferred_workspace_size(M, N, Kp)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=DEV)
    ob = mx.OUT_BYTES[out_type]

    def run(a, b, s_a, s_b):
        D = torch.full((M * N * ob,), 0x5A, dtype=torch.uint8, device=DEV)
        rc = mx.gemm(out_type, M, N, Kp, a.data_ptr(), b.data_ptr(), s_a.data_ptr(),
                     s_b.data_ptr(), D.data_ptr(), rb, ws.data_ptr(), ws_bytes)
        assert rc == 0
        return host(D)

    d_dev = run(da, db, dsa, dsb)
    d_host = run(to_dev(a_rows.reshape(-1)), to_dev(bsh), to_dev(sa_t), to_dev(sb_t))
    assert np.array_equal(d_dev, d_host)


@pytest.mark.parametrize("M,K,group", [(32, 64, 1), (100, 1000, 2), (256, 2080, 4), (97, 8192, 3)])
def test_prepare_a_preshuffled(mx, M, K, group):
    """A quantised straight into the preshuffled layout equals the device preshuffle of
    prepare_a's padded rows and the oracle's preshuffle of the quantised rows (zero rows up to
    the next 32); the scales equal prepare_a's; and a GEMM reading it (a_layout 2) gives the bits
    of the routed GEMM on the row-major A."""
    say(f"prepare_a preshuffled M={M} K={K} group={group}")
    Kp = _kpad(K)
    rb = Kp // 4 * 3
    x = specials_matrix(M, K, seed=M * 13 + K) if K % 32 == 0 else None
    x = np.random.default_rng(M + K).standard_normal((M, K)).astype(np.float32) if x is None else x
    dx = to_dev(x)
    nts = mx.tiled_scale_bytes(M, K, group)
    rows = torch.empty(M * rb, dtype=torch.uint8, device=DEV)
    t_rows = torch.empty(nts, dtype=torch.uint8, device=DEV)
    assert mx.prepare_a_dev(dx.data_ptr(), M, K, group, rows.data_ptr(), rb, t_rows.data_ptr()) == 0
    nsh = mx.preshuffled_bytes(M, K)
    via_rows = torch.empty(nsh, dtype=torch.uint8, device=DEV)
    assert mx.preshuffle_rows(rows.data_ptr(), rb, M, Kp, via_rows.data_ptr()) == 0
    ash = torch.full((nsh + 256,), 0xA5, dtype=torch.uint8, device=DEV)
    t_sh = torch.full((nts,), 0xA5, dtype=torch.uint8, device=DEV)
    assert mx.prepare_a_preshuffled_dev(dx.data_ptr(), M, K, group, ash.data_ptr(),
                                        t_sh.data_ptr()) == 0
    got = host(ash)
    assert (got[nsh:] == 0xA5).all()
    assert np.array_equal(got[:nsh], host(via_rows))
    assert np.array_equal(host(t_sh), host(t_rows))
    M32, K32 = -(-M // 32) * 32, -(-K // 32) * 32
    xz = np.zeros((M32, K32), np.float32)
    xz[:M, :K] = x
    po, _ = oracle.quantize_ref(xz)
    padded = np.zeros((M32, rb), np.uint8)
    padded[:, :K32 // 4 * 3] = po.reshape(M32, -1)
    assert np.array_equal(got[:nsh], oracle.preshuffle_b(padded, M32, Kp, rb))
    # the GEMM on it: N = 256, B prepared on the device, the tile the router picks
    N = 256
    tile = mx.choose_tile(M, N, Kp)
    if tile[2] != group:
        return
    B = np.random.default_rng(K).standard_normal((K, N)).astype(np.float32)
    db = torch.empty(mx.preshuffled_bytes(N, K), dtype=torch.uint8, device=DEV)
    dsb = torch.empty(mx.tiled_scale_bytes(N, K, tile[3]), dtype=torch.uint8, device=DEV)
    assert mx.prepare_b_dev(to_dev(B).data_ptr(), K, N, tile[3], db.data_ptr(), dsb.data_ptr()) == 0
    D1 = torch.empty(M * N * 4, dtype=torch.uint8, device=DEV)
    D2 = torch.empty(M * N * 4, dtype=torch.uint8, device=DEV)
    wsb = mx.workspace_size(M, N, Kp)
    ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device=DEV)
    assert mx.gemm(0, M, N, Kp, rows.data_ptr(), db.data_ptr(), t_rows.data_ptr(), dsb.data_ptr(),
                   D1.data_ptr(), rb, ws.data_ptr(), wsb) == 0
    # the plan gemm() runs with that workspace (the routed scale grouping, row-major A)
    ftile, S, _ = mx.gemm_plan(0, M, N, Kp, wsb)
    assert ftile[2:] == tuple(tile)[2:]
    wse = mx.plan_workspace_size(M, N, Kp, S, 0)
    wsx = torch.empty(max(wse, 4), dtype=torch.uint8, device=DEV)
    assert mx.gemm_explicit(0, M, N, Kp, ftile, S, ash.data_ptr(), db.data_ptr(), t_sh.data_ptr(),
                            dsb.data_ptr(), D2.data_ptr(), rb, wsx.data_ptr() if wse else 0, wse,
                            a_layout=2) == 0
    assert np.array_equal(host(D1), host(D2))
