"""Measured plan selection (mxfp6_gemm_tune): the router's best-predicted plans of a shape are
timed on the caller's operands and the fastest kept for the process.

Checked: the chosen plan keeps choose_tile's scale grouping; gemm() afterwards runs it (D bit for
bit equal to the explicit plan) and D meets the oracle bar on sampled rows; a workspace too small
for the chosen plan makes gemm() fall back to the router's plan (bit-equal to that explicit plan);
mxfp6_gemm_tune_reset forgets the choice.
"""
import numpy as np
import pytest
import torch

import checks
import mxfp6_amd as mx
from gpu_util import DevProblem, run_explicit, say, to_f32

pytestmark = pytest.mark.gpu

# the tiles with a pipelined-kernel instantiation (slab and wide kernels)
IMPLEMENTED = [(128, 128, 2, 2), (128, 256, 2, 4), (128, 384, 4, 3), (256, 256, 4, 4),
               (256, 192, 4, 3), (128, 512, 4, 4), (128, 256, 4, 2), (256, 256, 4, 2)]


@pytest.fixture(autouse=True)
def clean_table():
    mx.tune_reset()
    yield
    mx.tune_reset()


def _gemm(dp, ot, ws_bytes):
    p = dp.p
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device="cuda")
    D = dp.out(ot)
    a, b, sa, sb = dp.ptrs()
    rc = mx.gemm(ot, p.M, p.N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes,
                 ws.data_ptr() if ws_bytes else 0, ws_bytes)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    return to_f32(D, ot, p.M, p.N)


@pytest.mark.parametrize("M,N,K", [(8192, 1024, 16384), (1536, 1536, 5120), (1024, 4096, 1024),
                                   (512, 2048, 8192), (256, 256, 1024), (256, 256, 4096)])
def test_tuned_plan_is_used_and_correct(orc, M, N, K):
    ot = mx.OUT_F16
    p = mx.make_problem(M, N, K, seed=M + 3 * N + 5 * K)
    routed = tuple(mx.choose_tile(M, N, p.Kp))
    dp = DevProblem(p, routed)
    wsb = mx.preferred_workspace_size(M, N, p.Kp)
    ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device="cuda")
    D = dp.out(ot)
    a, b, sa, sb = dp.ptrs()
    rc, (tile, S, rp) = mx.gemm_tune(ot, M, N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes,
                                     ws.data_ptr() if wsb else 0, wsb, candidates=4)
    assert rc == 0, mx.STATUS.get(rc, rc)
    say(f"  {M}x{N}x{K}: router {routed} S {mx.splitk_segments(M, N, p.Kp)} repack "
        f"{mx.repacks_a(M, N, p.Kp)} -> measured {tile} S {S} repack {rp}")
    assert mx.tuned_plan(ot, M, N, p.Kp) == (tile, S, rp)
    assert tile[2:] == routed[2:], "the measured plan must keep the scale grouping"
    assert mx.plan_workspace_size(M, N, p.Kp, S, int(rp)) <= wsb

    got = _gemm(dp, ot, wsb)
    dp_t = DevProblem(p, tile) if tile != routed else dp
    want = run_explicit(dp_t, ot, splits=S, a_layout=1 if rp else 0)
    assert (got.view("u4") == want.view("u4")).all(), "gemm() did not run the measured plan"
    rows = np.r_[0:2, M // 2, M - 2:M]
    R, ab = orc.gemm_f64(p.a_packed, p.a_row_bytes, p.a_scales, p.b_packed, p.b_row_bytes,
                         p.b_scales, M, N, K, rows=rows)
    checks.check(got[rows], R, ab, ot)

    # gemm_workspace_size's workspace (the router's partials only), too small for the measured
    # plan: the plan mxfp6_gemm_plan names for it (routed scale grouping, fits the workspace)
    small = mx.workspace_size(M, N, p.Kp)
    if mx.plan_workspace_size(M, N, p.Kp, S, int(rp)) > small:
        ft, fs, frp = mx.gemm_plan(ot, M, N, p.Kp, small)
        assert ft[2:] == routed[2:] and not frp
        got_small = _gemm(dp, ot, small)
        dp_f = DevProblem(p, ft) if ft != routed else dp
        want_r = run_explicit(dp_f, ot, splits=fs, a_layout=0)
        assert (got_small.view("u4") == want_r.view("u4")).all(), "no fallback to the router"
        say(f"    with the router's workspace: {ft} S {fs}")

    mx.tune_reset()
    assert mx.tuned_plan(ot, M, N, p.Kp) is None


def test_loaded_plan_is_used(orc, tmp_path):
    """A plan from a measured-plan file (mxfp6_gemm_tune_load) is what gemm() runs: bit-equal to
    the same plan run explicitly, within the oracle bar on sampled rows."""
    ot = mx.OUT_F16
    M, N, K = 2048, 2048, 16384
    p = mx.make_problem(M, N, K, seed=99)
    routed = tuple(mx.choose_tile(M, N, p.Kp))
    # a tile with the routed scale grouping that has a kernel and divides the shape, other than
    # the routed tile where there is one (a router refit may change the routed grouping)
    same = [t for t in IMPLEMENTED if t[2:] == routed[2:] and M % t[0] == 0 and N % t[1] == 0]
    tile = next((t for t in same if t != routed), routed)
    plan = (tile, 2, False)
    f = tmp_path / "plans.txt"
    f.write_text(f"{ot} {M} {N} {p.Kp} {plan[0][0]} {plan[0][1]} {plan[0][2]} {plan[0][3]} "
                 f"{plan[1]} 0\n")
    assert mx.tune_load(str(f)) == (1, 0)
    assert mx.gemm_plan(ot, M, N, p.Kp, mx.plan_workspace_size(M, N, p.Kp, 2, 0)) == plan
    dp = DevProblem(p, routed)
    got = _gemm(dp, ot, mx.plan_workspace_size(M, N, p.Kp, 2, 0))
    want = run_explicit(DevProblem(p, plan[0]), ot, splits=2, a_layout=0)
    assert (got.view("u4") == want.view("u4")).all(), "gemm() did not run the loaded plan"
    rows = np.r_[0:2, M // 2, M - 2:M]
    R, ab = orc.gemm_f64(p.a_packed, p.a_row_bytes, p.a_scales, p.b_packed, p.b_row_bytes,
                         p.b_scales, M, N, K, rows=rows)
    checks.check(got[rows], R, ab, ot)
