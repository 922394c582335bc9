"""The reference's own GPU test cases (tests/test_gemm.cpp:402-442), shape for shape, through this
library: each case runs the same kind of call the reference test makes (routed gemm with padded or
compact A, forced tiles, a workspace handed over when none is needed) and is checked against the
FP64 oracle at this build's bar (tests/checks.py), not the reference's 2e-2 * max|R|. Outputs are
poisoned with 0x5A, as the reference does, and D carries a guard region past its end.

The reference forces its 128x128 and 128x384 kernels (verify_128x128 / verify_128x384); here the
same shapes are forced onto the same tiles with gemm_force_tile. Its NMASK cases (N a multiple of
128 but not of 256, :438-442) additionally run a masked 256x256 explicitly, the reference's route
for them.
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


def _run(dp, out_type, how, tile=None, ws_bytes=None):
    p = dp.p
    n = p.M * p.N * mx.OUT_BYTES[out_type]
    D = torch.full((n + GUARD,), 0x5A, dtype=torch.uint8, device="cuda")
    a, b, sa, sb = dp.ptrs()
    say(f"  {how} {p.M}x{p.N}x{p.K} (Kp {p.Kp}) tile {tile or dp.tile} A_row_bytes {p.a_row_bytes}")
    if how == "routed":
        wsb = mx.preferred_workspace_size(p.M, p.N, p.Kp) if ws_bytes is None else ws_bytes
        ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device="cuda")
        rc = mx.gemm(out_type, p.M, p.N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes,
                     ws.data_ptr() if wsb else 0, wsb)
    elif how == "forced":
        rc = mx.gemm_force_tile(out_type, p.M, p.N, p.Kp, tile, a, b, sa, sb, D.data_ptr(),
                                p.a_row_bytes)
    else:  # explicit, unsplit, row-major A
        rc = mx.gemm_explicit(out_type, p.M, p.N, p.Kp, tile, 1, a, b, sa, sb, D.data_ptr(),
                              p.a_row_bytes)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    assert (D[n:].cpu().numpy() == 0x5A).all(), "write past the end of D"
    return D[:n].view(TORCH_OUT[out_type]).float().reshape(p.M, p.N).cpu().numpy()


def _check(D, p, out_type=mx.OUT_F32):
    rows = None if p.M <= 512 else np.unique(np.r_[0:8, p.M // 2 - 4:p.M // 2 + 4, p.M - 8:p.M,
                                                  np.linspace(0, p.M - 1, 24).astype(int)])
    R, ab = oracle.problem_f64(p, rows=rows)
    checks.check(D if rows is None else D[rows], R, ab, out_type)


# verify(M, N, K): routed, padded A rows (test_gemm.cpp:402-404, 433, 437, 441-442)
@pytest.mark.parametrize("M,N,K", [(512, 512, 768), (768, 1280, 960), (4096, 4096, 768),
                                   (128, 384, 3072), (256, 384, 32768), (512, 640, 960),
                                   (256, 1408, 384)])
def test_verify_routed(M, N, K):
    p = mx.make_problem(M, N, K, compact=False, seed=M * 3 + N * 7 + K)
    D = _run(DevProblem(p, mx.choose_tile(M, N, p.Kp)), mx.OUT_F32, "routed")
    _check(D, p)


# verify_compact(M, N, K): routed, compact A + end pad, real K-tails, split-K (:407-414)
@pytest.mark.parametrize("M,N,K", [(4096, 4096, 224), (768, 1280, 224), (512, 512, 160),
                                   (2048, 1024, 12288), (2048, 1024, 3808), (2048, 1024, 6304)])
def test_verify_compact(M, N, K):
    p = mx.make_problem(M, N, K, compact=True, seed=M * 5 + N * 11 + K * 2)
    D = _run(DevProblem(p, mx.choose_tile(M, N, p.Kp)), mx.OUT_F32, "routed")
    _check(D, p)


# verify_128x128 / verify_128x384: forced tiles (:417-428), incl. the 10x3 XCD-remap remainder grid
@pytest.mark.parametrize("tile,M,N,K", [((128, 128, 2, 2), 256, 256, 768),
                                        ((128, 128, 2, 2), 384, 512, 1536),
                                        ((128, 384, 4, 3), 256, 384, 768),
                                        ((128, 384, 4, 3), 384, 768, 960),
                                        ((128, 384, 4, 3), 1280, 1152, 384)])
def test_verify_forced(tile, M, N, K):
    p = mx.make_problem(M, N, K, compact=False, seed=M * 3 + N * 7 + K)
    D = _run(DevProblem(p, tile), mx.OUT_F32, "forced", tile=tile)
    _check(D, p)


# verify(128, 384, 3072, force_ws=true): a workspace handed over where none is needed (:433-434)
def test_verify_workspace_handed_over():
    M, N, K = 128, 384, 3072
    p = mx.make_problem(M, N, K, compact=False, seed=M * 3 + N * 7 + K)
    dp = DevProblem(p, mx.choose_tile(M, N, p.Kp))
    D0 = _run(dp, mx.OUT_F32, "routed")
    D1 = _run(dp, mx.OUT_F32, "routed", ws_bytes=16 * M * N * 4 + M * p.Kp)
    assert np.array_equal(D0.view(np.uint32), D1.view(np.uint32))
    _check(D1, p)


# the NMASK cases on the reference's own route: 256x256 over ceil(N/256) tile columns (:438-442)
@pytest.mark.parametrize("M,N,K", [(512, 640, 960), (256, 1408, 384)])
@pytest.mark.parametrize("out_type", [0, 1, 2])
def test_nmask_256x256(M, N, K, out_type):
    p = mx.make_problem(M, N, K, compact=False, seed=M * 3 + N * 7 + K)
    D = _run(DevProblem(p, (256, 256, 4, 4)), out_type, "explicit", tile=(256, 256, 4, 4))
    _check(D, p, out_type)
