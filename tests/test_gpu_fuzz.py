"""Seeded random shapes through the routed gemm(), against the FP64 oracle.

Twenty-four shapes drawn once from a fixed seed: M and N log-uniform in [32, 4096] (a third of
them rounded to multiples of 128, a third to multiples of 32 and 128, the rest ragged), K a
multiple of 32 up to 8192; and eight shapes that reach the routes small random shapes rarely do.
The output type cycles through FP32, FP16 and BF16. Each runs with the workspace the router asks
for (so the plans it picks are exercised: big and skinny tiles, N-masked and ragged tiles,
split-K on either XCD map, repacked A) and again with no
workspace (the documented fallback to the unsplit, unrepacked plan), and is checked against the
FP64 oracle at this build's bar (tests/checks.py) on every row of a small M, or on 48 spread rows.
Outputs and workspaces carry guard regions that must survive the call. The same shapes run again
on operands whose FP32 sums depend on the order of the additions (FP32 out, tests/checks.py
spread_scales), where the two workspaces that run the same split must also agree bit for bit.
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


# shapes that reach routes random small shapes rarely do: the wide tiles (256x256, 128x512,
# 128x384, 128x256) unsplit and split, with and without a masked last column, the 128x128 tile
# split and not, and a ragged skinny one (the router's picks move when its model is refitted, so
# the list is wide rather than one shape per route)
ROUTES = [(5504, 1536, 1024), (5504, 384, 16384), (896, 4352, 1024), (384, 10112, 1024),
          (128, 5504, 8192), (768, 11008, 1024), (6656, 1152, 1024), (4608, 384, 16384),
          (768, 10880, 16384), (2304, 7296, 1024), (6016, 2688, 1024), (384, 5504, 1024),
          (5504, 128, 8192), (2047, 1000, 4096), (3072, 4096, 2048), (1536, 1536, 24576),
          (1024, 16384, 16384)]


def _shapes(n=24, seed=20261201):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M, N = (int(round(2 ** rng.uniform(5, 12))) for _ in range(2))
        if i % 3 == 0:
            M, N = max(128, M // 128 * 128), max(128, N // 128 * 128)
        elif i % 3 == 1:
            M, N = max(32, M // 32 * 32), max(128, N // 128 * 128)
        K = int(rng.integers(1, 257)) * 32
        out.append((M, N, K, i % 3))
    return out + [(M, N, K, i % 3) for i, (M, N, K) in enumerate(ROUTES)]


def _run(dp, out_type, with_ws):
    """with_ws: "preferred" (the plan's whole workspace), "split" (gemm_workspace_size's bytes,
    the split-K partials only: A read row-major) or False (no workspace: never split)."""
    p = dp.p
    n = p.M * p.N * mx.OUT_BYTES[out_type]
    size = mx.preferred_workspace_size if with_ws == "preferred" else mx.workspace_size
    ws_bytes = size(p.M, p.N, p.Kp) if with_ws else 0
    D = torch.full((n + GUARD,), 0x5A, dtype=torch.uint8, device="cuda")
    ws = torch.full((max(ws_bytes, 4) + GUARD,), 0x3C, dtype=torch.uint8, device="cuda")
    a, b, sa, sb = dp.ptrs()
    say(f"  routed {p.M}x{p.N}x{p.K} (Kp {p.Kp}) tile {dp.tile} S "
        f"{mx.splitk_segments(p.M, p.N, p.Kp)} repack {mx.repacks_a(p.M, p.N, p.Kp)} out "
        f"{mx.OUT_NAMES[out_type]} ws {ws_bytes}")
    rc = mx.gemm(out_type, p.M, p.N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes,
                 ws.data_ptr() if ws_bytes else 0, ws_bytes)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    assert (D[n:].cpu().numpy() == 0x5A).all(), "write past the end of D"
    assert (ws[max(ws_bytes, 4):].cpu().numpy() == 0x3C).all(), "write past the workspace"
    return D[:n].view(TORCH_OUT[out_type]).float().reshape(p.M, p.N).cpu().numpy()


@pytest.mark.parametrize("M,N,K,out_type", _shapes())
def test_routed_random_shape(M, N, K, out_type):
    p = mx.make_problem(M, N, K, seed=M * 131 + N * 17 + K)
    dp = DevProblem(p, mx.choose_tile(M, N, p.Kp))
    rows = None if M <= 48 else np.unique(np.r_[0:4, M - 4:M,
                                                 np.linspace(0, M - 1, 40).astype(int)])
    R, ab = oracle.problem_f64(p, rows=rows)
    for with_ws in ("preferred", "split", False):
        D = _run(dp, out_type, with_ws)
        checks.check(D if rows is None else D[rows], R, ab, out_type)


@pytest.mark.parametrize("M,N,K,_", _shapes())
def test_routed_random_shape_order_sensitive(M, N, K, _):
    """The same shapes on operands whose FP32 sums depend on the order of the additions (block
    scales lowered by random exponents, checks.spread_scales), FP32 out: each run within the FP32
    bar of the FP64 oracle, and the plan's whole workspace and the split-only one (the same K
    segments, A repacked or read row-major) bit for bit equal."""
    seed = M * 131 + N * 17 + K + 1
    p = checks.spread_scales(mx.make_problem(M, N, K, seed=seed), seed=seed)
    dp = DevProblem(p, mx.choose_tile(M, N, p.Kp))
    rows = None if M <= 48 else np.unique(np.r_[0:4, M - 4:M,
                                                 np.linspace(0, M - 1, 40).astype(int)])
    R, ab = oracle.problem_f64(p, rows=rows)
    out = {}
    for with_ws in ("preferred", "split", False):
        D = _run(dp, mx.OUT_F32, with_ws)
        checks.check(D if rows is None else D[rows], R, ab, mx.OUT_F32)
        out[with_ws] = D
    assert np.array_equal(out["preferred"].view(np.uint32), out["split"].view(np.uint32))
