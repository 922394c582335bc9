"""Same-session throughput of this library against the reference GPU library (oracle/_ref, built
from the reference's own sources) on the five benchmark workloads, same device operands.

Each side runs its own router (choose_tile / workspace) on identical packed operands; outputs are
spot-checked against the FP64 oracle so a fast wrong result cannot pass. Timing follows the
reference's methodology (warm-up, then the best mean of repetitions of 20 back-to-back launches).
On the five benchmark workloads the goal is >= 1.0x; the assertion allows 3% for run-to-run noise
(>= 0.97x). The off-benchmark shapes include known short-K losses (0.91-0.98x measured), so they are
guarded at >= 0.85x only. Set MXFP6_PERF_LOG=<file> to append one JSON line per workload.
"""
import ctypes as C
import json
import os

import numpy as np
import pytest

import checks
import mxfp6_amd as mx

pytestmark = pytest.mark.gpu

SEED = 0x4D584636
WORKLOADS = {
    "c1": (256, 256, 1024, mx.OUT_F32, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "c2": (8192, 8192, 8192, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "c3": (2048, 6144, 16128, mx.OUT_F16, (mx.DIST_NORMAL, 2.0), (mx.DIST_UNIFORM, 1.0)),
    "c4": (2048, 1024, 105728, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "c5": (2048, 5120, 105728, mx.OUT_BF16, (mx.DIST_STUDENT_T3, 1.0), (mx.DIST_STUDENT_T3, 1.0)),
    # shapes outside the benchmark set, from the bands the reference's benchmark notes list as
    # its weakest (benchmark_results.md:246-259: grids too small for the GPU at short K, mid N)
    "s2048x2048x2048": (2048, 2048, 2048, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "s2048x1024x1024": (2048, 1024, 1024, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "s2048x512x2560": (2048, 512, 2560, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "s2048x1024x4096": (2048, 1024, 4096, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "s1024x4096x8192": (1024, 4096, 8192, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "s4096x4096x1024": (4096, 4096, 1024, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    # N a multiple of 128 but not of 256: the reference's masked 256x256 route (NMASK,
    # src/kernel.hpp:144-154; README.md:270-279 quotes N = 102272)
    "s8192x896x8192": (8192, 896, 8192, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "s4096x2432x8192": (4096, 2432, 8192, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "s2048x102272x1024": (2048, 102272, 1024, mx.OUT_F16, (mx.DIST_NORMAL, 1.0),
                          (mx.DIST_NORMAL, 1.0)),
}


def _best_ms(torch, fn, reps=4, n=20, warm=8):
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b) / n)
    return best


@pytest.mark.parametrize("name", sorted(WORKLOADS))
def test_throughput_vs_reference_library(orc, ref_lib, name):
    import torch
    from gpu_util import say, TORCH_OUT

    M, N, K, ot, (da, sa_), (db, sb_) = WORKLOADS[name]
    p = mx.make_problem(M, N, K, da, sa_, db, sb_,
                        seed=SEED ^ (int(name[1:]) if name[0] == "c" else M + N + K))
    flops = 2.0 * M * N * K
    dA = torch.from_numpy(p.a_packed).cuda()
    D = torch.empty(M * N * mx.OUT_BYTES[ot], dtype=torch.uint8, device="cuda")
    rows = np.r_[0:4, M // 2:M // 2 + 4, M - 4:M]
    R, ab = orc.problem_f64(p, rows=rows)
    ridx = torch.from_numpy(rows).cuda()

    def check(label):
        got = D.view(TORCH_OUT[ot]).float().reshape(M, N)[ridx].cpu().numpy()
        checks.check(got, R, ab, ot)

    # this library, its own route
    t = mx.choose_tile(M, N, p.Kp)
    bsh, sa, sb = p.layouts(t)
    dB, dsa, dsb = (torch.from_numpy(x).cuda() for x in (bsh, sa, sb))
    wsb = mx.preferred_workspace_size(M, N, p.Kp)
    ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device="cuda")

    def ours():
        rc = mx.gemm(ot, M, N, p.Kp, dA.data_ptr(), dB.data_ptr(), dsa.data_ptr(), dsb.data_ptr(),
                     D.data_ptr(), p.a_row_bytes, ws.data_ptr() if wsb else 0, wsb)
        assert rc == 0, mx.STATUS.get(rc, rc)

    say(f"  {name}: ours tile {tuple(t)} S {mx.splitk_segments(M, N, p.Kp)} "
        f"repack {mx.repacks_a(M, N, p.Kp)}")
    D.fill_(0x5A)
    ours()
    torch.cuda.synchronize()
    check("ours")
    ms_ours = _best_ms(torch, ours)
    del dB, dsa, dsb, ws

    # the reference library, its own route and workspace
    tr = (C.c_int * 4)()
    ref_lib.ref_choose_tile(M, N, p.Kp, tr)
    tr = tuple(tr)
    bsh, sa, sb = p.layouts(tr)
    dB, dsa, dsb = (torch.from_numpy(x).cuda() for x in (bsh, sa, sb))
    wsr = ref_lib.ref_gemm_workspace_size(M, N, p.Kp)
    wsr_t = torch.empty(max(wsr, 4), dtype=torch.uint8, device="cuda")

    def ref():
        ref_lib.ref_gemm(ot, M, N, p.Kp, dA.data_ptr(), dB.data_ptr(), dsa.data_ptr(),
                         dsb.data_ptr(), D.data_ptr(), p.a_row_bytes, p.b_row_bytes,
                         wsr_t.data_ptr() if wsr else None, wsr)

    say(f"  {name}: reference tile {tr}")
    D.fill_(0x5A)
    ref()
    torch.cuda.synchronize()
    check("reference")
    ms_ref = _best_ms(torch, ref)

    tf_o, tf_r = flops / ms_ours / 1e9, flops / ms_ref / 1e9
    say(f"  {name} {M}x{N}x{K}: ours {ms_ours * 1e3:8.1f} us {tf_o:7.1f} TF | reference "
        f"{ms_ref * 1e3:8.1f} us {tf_r:7.1f} TF | ratio {tf_o / tf_r:.3f}")
    log = os.environ.get("MXFP6_PERF_LOG")
    if log:
        with open(log, "a") as f:
            f.write(json.dumps({"workload": name, "M": M, "N": N, "K": K, "ours_us": ms_ours * 1e3,
                                "ours_tflops": tf_o, "ref_us": ms_ref * 1e3, "ref_tflops": tf_r,
                                "ratio": tf_o / tf_r, "ours_tile": list(t),
                                "ref_tile": list(tr)}) + "\n")
    floor = 0.97 if name[0] == "c" else 0.85
    assert tf_o >= floor * tf_r, f"{name}: {tf_o / tf_r:.3f}x the reference (floor {floor})"
