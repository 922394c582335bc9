"""Graph capture of the routed GEMM.

A caller that replays its work through HIP graphs (a serving loop, a launch-bound inner loop)
captures mxfp6_gemm_async's launches on its own stream. The library allocates, frees,
synchronises and clears nothing on the way, so every route captures as plain kernel nodes: one
tile-kernel launch; the A repack then the tile kernel; the tile kernel then the split-K reduce;
and the no-allocation entry point's scratch-backed plans. Each replay must equal the eager call
bit for bit. Eager work and synchronisations run between the replays, and D is overwritten with
a poison pattern before each one, so a replay that wrote nothing (or only part of D) fails.
"""
import pytest
import torch

import mxfp6_amd as mx
from gpu_util import DevProblem, routed_shape, say

pytestmark = pytest.mark.gpu

# (candidate shapes, wanted route): the first candidate the router sends down the route is used
ROUTES = {
    "one launch": ([(M, N, 2048) for M in (512, 1024) for N in (1024, 2048)],
                   lambda t, S, rp: S == 1 and not rp),
    "split-K": ([(M, N, K) for K in (16384, 32768) for M in (512, 1024) for N in (512, 768, 1024)],
                lambda t, S, rp: S > 1),
    "A repacked": ([(1024, N, K) for K in (16384, 32768) for N in (5120, 8192, 16384)],
                   lambda t, S, rp: rp),
    # the 32 x 32 tile: K split over each workgroup's waves, one segment per wave and two in turn
    "32x32 split": ([(256, 256, 1024)], lambda t, S, rp: t == (32, 32, 1, 1) and 1 < S <= 4),
    "32x32 two segments per wave": ([(512, 512, 4096), (256, 256, 4096)],
                                    lambda t, S, rp: t == (32, 32, 1, 1) and S > 4),
}
REPLAYS = 3


def _capture_and_replay(launch, D, eager):
    """Captures launch() on a side stream, replays it REPLAYS times (poisoning D and running
    unrelated eager work first) and checks each replay against the eager output."""
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        launch(side)
    torch.cuda.synchronize()
    scratch = torch.empty(1 << 20, dtype=torch.float32, device="cuda")
    for r in range(REPLAYS):
        D.fill_(0x5A + r)
        scratch.normal_()
        float(scratch.sum())  # eager work and a synchronisation between the replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(D, eager), f"replay {r + 1} differs from the eager call"
        say(f"    replay {r + 1}: equal to the eager call")


@pytest.mark.parametrize("route", sorted(ROUTES))
@pytest.mark.parametrize("out_type", [mx.OUT_F16, mx.OUT_F32])
def test_captured_gemm_replays_equal_eager(route, out_type):
    M, N, K = routed_shape(*ROUTES[route])
    p = mx.make_problem(M, N, K, seed=M + 5 * N + K)
    dp = DevProblem(p, mx.choose_tile(M, N, p.Kp))
    S, rp = mx.splitk_segments(M, N, p.Kp), mx.repacks_a(M, N, p.Kp)
    ws_bytes = mx.preferred_workspace_size(M, N, p.Kp)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device="cuda")
    say(f"  {route}: {M}x{N}x{K} out {mx.OUT_NAMES[out_type]} tile {dp.tile} S {S} repack {rp} "
        f"ws {ws_bytes}")
    a, b, sa, sb = dp.ptrs()

    def launch(stream, D):
        rc = mx.gemm(out_type, M, N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes,
                     ws.data_ptr() if ws_bytes else 0, ws_bytes, stream=stream.cuda_stream)
        assert rc == 0, mx.STATUS.get(rc, rc)

    eager = dp.out(out_type)
    launch(torch.cuda.current_stream(), eager)
    torch.cuda.synchronize()
    D = dp.out(out_type)
    _capture_and_replay(lambda s: launch(s, D), D, eager)


@pytest.mark.parametrize("route", ["split-K", "A repacked"])
def test_captured_noalloc_gemm_replays_equal_eager(route):
    M, N, K = routed_shape(*ROUTES[route])
    p = mx.make_problem(M, N, K, seed=M + 7 * N + K)
    dp = DevProblem(p, mx.choose_tile(M, N, p.Kp))
    say(f"  no-alloc {route}: {M}x{N}x{K} tile {dp.tile} S {mx.splitk_segments(M, N, p.Kp)} "
        f"repack {mx.repacks_a(M, N, p.Kp)}")
    a, b, sa, sb = dp.ptrs()

    def launch(stream, D):
        rc = mx.gemm_noalloc(mx.OUT_F16, M, N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes,
                             stream=stream.cuda_stream)
        assert rc == 0, mx.STATUS.get(rc, rc)

    eager = dp.out(mx.OUT_F16)
    launch(torch.cuda.current_stream(), eager)
    torch.cuda.synchronize()
    D = dp.out(mx.OUT_F16)
    _capture_and_replay(lambda s: launch(s, D), D, eager)
