"""Plans for a workspace that does not hold the routed plan (mxfp6_gemm_plan): gemm() then runs the
fastest predicted plan with the routed scale grouping that fits, here a different tile. Checked
bit for bit against that plan run explicitly and against the routed tile run unsplit on
row-major A (unsplit plans of one grouping issue the same MFMAs in the same K order), and against
the oracle on sampled rows; the reference-sized workspace keeps the routed split."""
import numpy as np
import pytest
import torch

import checks
import mxfp6_amd as mx
from gpu_util import DevProblem, run_explicit, say, to_f32

pytestmark = pytest.mark.gpu


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


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 16384), (1536, 1536, 24576)])
def test_no_workspace_runs_the_best_fitting_plan(orc, M, N, K):
    ot = mx.OUT_F16
    p = mx.make_problem(M, N, K, seed=M + N + K)
    routed = tuple(mx.choose_tile(M, N, p.Kp))
    S = mx.splitk_segments(M, N, p.Kp)
    ft, fs, frp = mx.gemm_plan(ot, M, N, p.Kp, 0)
    say(f"  {M}x{N}x{K}: routed {routed} S {S}; without a workspace {ft} S {fs} repack {frp}")
    assert S > 1 and fs == 1 and not frp and ft[2:] == routed[2:] and ft != routed
    dp = DevProblem(p, routed)
    got = _gemm(dp, ot, 0)
    want = run_explicit(DevProblem(p, ft), ot, splits=1, a_layout=0)
    same_grouping = run_explicit(dp, ot, splits=1, a_layout=0)
    assert (got.view("u4") == want.view("u4")).all()
    assert (got.view("u4") == same_grouping.view("u4")).all()
    rows = np.r_[0:2, M // 2, M - 2:M]
    R, ab = orc.gemm_f64(p.a_packed, p.a_row_bytes, p.a_scales, p.b_packed, p.b_row_bytes,
                         p.b_scales, M, N, K, rows=rows)
    checks.check(got[rows], R, ab, ot)
    # gemm_workspace_size's workspace: the routed split
    wsr = mx.workspace_size(M, N, p.Kp)
    assert mx.gemm_plan(ot, M, N, p.Kp, wsr)[1] == S
    got_r = _gemm(dp, ot, wsr)
    want_r = run_explicit(dp, ot, splits=S, a_layout=0)
    assert (got_r.view("u4") == want_r.view("u4")).all()
