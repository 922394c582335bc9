"""Concurrent calls: one host thread per stream, each stream with its own operands, output and
workspace, four routes at once (split-K, A repacked into the workspace, one wide-tile launch, a
skinny tile). The host code keeps only a per-thread plan cache and the kernels share nothing but
the inputs' read-only memory, so every concurrent result must equal the same call made alone, bit
for bit. (ctypes releases the GIL around each library call, so the threads do call the library
at the same time.)
"""
import threading

import pytest
import torch

import mxfp6_amd as mx
from gpu_util import DevProblem, routed_shape, say

pytestmark = pytest.mark.gpu

ROUTES = [
    ([(M, N, K) for K in (16384, 32768) for M in (512, 1024) for N in (512, 768, 1024)],
     lambda t, S, rp: S > 1),
    ([(1024, N, K) for K in (16384, 32768) for N in (5120, 8192, 16384)],
     lambda t, S, rp: rp),
    ([(M, N, 4096) for M in (2048, 3072) for N in (2048, 4096)],
     lambda t, S, rp: t[0] == 256 and S == 1 and not rp),
    ([(M, N, 4096) for M in (96, 160, 224) for N in (1024, 2048)],
     lambda t, S, rp: t[0] < 128),
]
ROUNDS = 4


class Call:
    def __init__(self, i, shape):
        M, N, K = shape
        self.p = mx.make_problem(M, N, K, seed=17 * i + M + N + K)
        self.dp = DevProblem(self.p, mx.choose_tile(M, N, self.p.Kp))
        self.ws_bytes = mx.preferred_workspace_size(M, N, self.p.Kp)
        self.ws = torch.empty(max(self.ws_bytes, 4), dtype=torch.uint8, device="cuda")
        self.D = self.dp.out(mx.OUT_F16)
        self.stream = torch.cuda.Stream()
        self.desc = (f"{M}x{N}x{K} tile {self.dp.tile} S {mx.splitk_segments(M, N, self.p.Kp)} "
                     f"repack {mx.repacks_a(M, N, self.p.Kp)}")

    def launch(self, stream):
        p = self.p
        a, b, sa, sb = self.dp.ptrs()
        rc = mx.gemm(mx.OUT_F16, p.M, p.N, p.Kp, a, b, sa, sb, self.D.data_ptr(), p.a_row_bytes,
                     self.ws.data_ptr() if self.ws_bytes else 0, self.ws_bytes,
                     stream=stream.cuda_stream)
        return rc


def test_concurrent_streams_equal_sequential_calls():
    calls = [Call(i, routed_shape(*r)) for i, r in enumerate(ROUTES)]
    expected = []
    for c in calls:
        say(f"  alone: {c.desc}")
        assert c.launch(torch.cuda.current_stream()) == 0
        torch.cuda.synchronize()
        expected.append(c.D.clone())
    for r in range(ROUNDS):
        for c in calls:
            c.D.fill_(0x5A + r)
        torch.cuda.synchronize()
        rcs = [None] * len(calls)

        def worker(k):
            rcs[k] = calls[k].launch(calls[k].stream)

        threads = [threading.Thread(target=worker, args=(k,)) for k in range(len(calls))]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        torch.cuda.synchronize()
        assert rcs == [0] * len(calls), rcs
        for c, e in zip(calls, expected):
            assert torch.equal(c.D, e), f"round {r + 1}: {c.desc} differs from the call alone"
        say(f"  round {r + 1}: four concurrent calls equal the calls alone")
