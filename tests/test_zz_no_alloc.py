"""The no-allocation entry point (mxfp6_gemm_noalloc_async) through the C ABI: its output equals
mxfp6_gemm_async's with the plan's whole workspace, bit for bit, on two calls in a row, the second
on a smaller input (the scratch keeps the first call's bytes, which the second must not read); the
second call leaves the device's free memory unchanged."""
import numpy as np
import pytest
import torch

import mxfp6_amd as mx
from gpu_util import DevProblem, say

pytestmark = pytest.mark.gpu

# (M, N, K, out_type) pairs, larger first
SEQUENCES = {
    # split-K: the 2048x1024x105728 workload (8 segments, 64 MiB of partials), then a smaller split
    "split": [(2048, 1024, 105728, 1), (512, 1024, 32768, 0)],
    # A repacked into the scratch (24 MiB), then a plan that repacks a smaller A (12 MiB); the
    # shapes are the first of short lists that the router repacks A for
    "repack": [(1024, 16384, 32768, 2), (1024, 16384, 16384, 1)],
    # 3 segments of partials (120 MiB) fit, the repacked A beside them does not: A read row-major
    "split_no_room_for_repack": [(2048, 5120, 105728, 2), (256, 256, 1024, 0)],
}


def _with_workspace(dp, ot):
    p = dp.p
    wsb = mx.preferred_workspace_size(p.M, p.N, p.Kp)
    ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device="cuda")
    D = dp.out(ot)
    a, b, sa, sb = dp.ptrs()
    rc = mx.gemm(ot, p.M, p.N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes,
                 ws.data_ptr() if wsb else 0, wsb)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    return D


def _no_alloc(dp, ot):
    p = dp.p
    D = dp.out(ot)
    a, b, sa, sb = dp.ptrs()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    rc = mx.gemm_noalloc(ot, p.M, p.N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    return D, free0, torch.cuda.mem_get_info()[0]


def _sequence(kind):
    if kind != "repack":
        return SEQUENCES[kind]
    from gpu_util import routed_shape
    big = routed_shape([(1024, N, K) for K in (32768, 65536) for N in (16384, 8192, 5120)],
                       lambda t, S, rp: rp and S == 1)
    small = routed_shape([(M, N, 16384) for M in (1024, 2048) for N in (16384, 8192, 5120)],
                         lambda t, S, rp: rp and S == 1)
    return [big + (2,), small + (1,)]


@pytest.mark.parametrize("kind", sorted(SEQUENCES))
def test_noalloc_equals_workspace_path_twice(kind):
    for i, (M, N, K, ot) in enumerate(_sequence(kind)):
        p = mx.make_problem(M, N, K, seed=M + 3 * N + 7 * K)
        dp = DevProblem(p, mx.choose_tile(M, N, p.Kp))
        S, rp = mx.splitk_segments(M, N, p.Kp), mx.repacks_a(M, N, p.Kp)
        say(f"  no-alloc call {i + 1} ({kind}): {M}x{N}x{K} out {mx.OUT_NAMES[ot]} tile {dp.tile} "
            f"S {S} repack {rp} partials {mx.workspace_size(M, N, p.Kp)} B")
        assert mx.workspace_size(M, N, p.Kp) <= mx.NOALLOC_SCRATCH_BYTES
        if kind == "repack":
            assert rp, "the repack sequence needs plans that repack A"
        want = _with_workspace(dp, ot)
        got, free0, free1 = _no_alloc(dp, ot)
        assert torch.equal(got, want), f"{kind} call {i + 1}: outputs differ"
        if i > 0:
            assert free1 == free0, f"free device memory changed by {free0 - free1} bytes"
        del dp, want, got
        torch.cuda.empty_cache()
