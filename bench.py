"""Benchmark of libmxfp6gemm on one MI355X: MXFP6 GEMM TFLOPs and fraction of the dense MXFP6
MFMA peak.

A step is one mxfp6_gemm_async call: the whole hot path the router picks for the shape (for the
default workload: one launch of the 256x256 tile kernel with four waves side by side, reading
row-major A), over operands already resident in HBM, with the plan's whole workspace
(mxfp6_gemm_preferred_workspace_size). Default workload: M = N = K = 8192, FP16 out, A and B
drawn from N(0,1) with the seeded PCG32 generator and quantised with the OCP MX rule.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--all] [--no-cpu]
                  [--no-ref]
  python bench.py --prep      (device operand preparation: float -> MXFP6 device layouts, GB/s)
  python bench.py --power S   (board power and clocks over S seconds of back-to-back GEMMs of the
                               workload, this library then the reference library; amd-smi)
  python bench.py --roof [S]  (the MFMA-only diagnostic kernel against the workload's GEMM: the
                               cycles per MFMA and the board's power roof, each sustained S s)
  python bench.py --ab PLANS [--config cN] [--repeat R]  (explicit plans MTxNTxMPWxNPW[:S[:r|p|s]]
                               of a workload against each other and the routed plan, R rounds,
                               order rotated)
  python bench.py --e2e [--all]  (float A to D on the device: quantise to row-major A + the routed
                                  gemm, against quantise to preshuffled A + the same plan)
  python bench.py --map [SHAPES|second] [--repeat R]  (this library against the reference library,
                               shape by shape: MxNxK,... or the default map of 154 shapes, FP16
                               out; R > 1: R more runs per library, alternating their order)

Prints one JSON line per workload (only the default one unless --all). The headline `value` is
the mean over exactly K timed steps after W warm-up steps. The per_config comparisons (below) run
before it, on the GPU only, so its W warm-ups follow seconds of GEMMs rather than an idle MI355X
near 160 MHz, whose clock would still be ramping through a short timed loop; the CPU baselines
run after it. `sclk_mhz` reports the clock the loop ran at. Besides the contract fields it reports:
  sclk_mhz      the mean graphics clock over the timed loop (each XCD's shader cycle counter
                against the 100 MHz reference counter, read by the library's clock sample just
                before and just after the loop, outside its events; mean over the XCDs), and
                frac_at_sclk = value / (4,194,304 flop/clk x sclk), the fraction of the dense
                MXFP6 MFMA peak at the clock the chip actually ran;
  roofline      the dominant kernel (the tile kernel) against the dense MXFP6 MFMA peak: its
                algorithmic flops per launch / its average launch duration, timed live with HIP
                events on the launch stream in a second loop of K steps that issues the step's
                two launches separately (repack, then the tile kernel on the repacked A);
                traffic = HBM bytes per launch from the committed rocprofv3 counter summary of
                the same kernel and workload (FETCH_SIZE + WRITE_SIZE scaled by the copy-kernel
                calibration), null when no summary matches;
  vs_baseline   value / the reference GPU library's TFLOPs on the same operands in this process
                (oracle/_ref/libmxfp6ref.so, built from the reference's own sources; its own
                router and workspace), timed by the reference's method (tests/test_gemm.cpp:33-55:
                8 warm-ups, best mean of 4 x 20 back-to-back launches) after the headline loop
                (and again, with the other workloads, in per_config before it);
  per_config    the five workloads, this library and the reference library each timed by that
                same method on identical operands: TFLOPs, fraction of 10.1 PF, ratio, and for the
                split-K workload the algorithmic HBM GB/s;
  cpu_baseline  the reference CPU GEMM's arithmetic on this host's CPU share (OMP_NUM_THREADS
                threads, else every CPU the process may use; the count is in `cores`): for the
                headline a bounded sample of A rows scaled to the whole GEMM, and in each
                per_config entry the same for that workload (the small one in full).
The reference library and the oracle are baselines only: nothing here routes the measured GEMM
through them.
"""
import argparse
import json
import os
import re
import subprocess
import sys
import threading
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mxfp6-gemm_amd"))

import numpy as np  # noqa: E402

import mxfp6_amd as mx  # noqa: E402

SEED = 0x4D584636
# MI355X published dense MXFP6 / MXFP4 MFMA peak (TFLOP/s) and HBM bandwidth (GB/s)
PEAK_TFLOPS = 10100.0
PEAK_HBM_GBS = 8000.0
# dense MXFP6 MFMA flops per clock: 256 CUs x 4 SIMDs x 131,072 flop per 32-cycle 32x32x64 MFMA
FLOP_PER_CLK = 256 * 4 * 2 * 32 * 32 * 64 // 32

# name -> (M, N, K, out_type, (dist_a, sigma_a), (dist_b, sigma_b), description)
CONFIGS = {
    "c1": (256, 256, 1024, mx.OUT_F32, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0),
           "A,B ~ N(0,1)"),
    "c2": (8192, 8192, 8192, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0),
           "A,B ~ N(0,1)"),
    "c3": (2048, 6144, 16128, mx.OUT_F16, (mx.DIST_NORMAL, 2.0), (mx.DIST_UNIFORM, 1.0),
           "A ~ N(0,4) (sigma 2), B ~ U[-1,1]"),
    "c4": (2048, 1024, 105728, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0),
           "A,B ~ N(0,1)"),
    "c5": (2048, 5120, 105728, mx.OUT_BF16, (mx.DIST_STUDENT_T3, 1.0),
           (mx.DIST_STUDENT_T3, 1.0), "A,B ~ Student-t(3)"),
}
PROFILES = os.path.join(ROOT, "profiles")
# the tiles run by wide_kernel (four waves side by side, B loaded into registers); the others by
# slab_kernel
WIDE_TILES = {(128, 512, 4, 4), (128, 384, 4, 3), (128, 256, 4, 2), (256, 256, 4, 2)}
METRIC = "MXFP6 GEMM TFLOPs (FP16 out) and % of MXFP6 MFMA peak, 1xMI355X"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def alg_bytes(M, N, K, out_type):
    """Algorithmic HBM bytes of one GEMM: packed A and B, one scale byte per 32 elements, D."""
    return (M + N) * K * 3 // 4 + (M + N) * K // 32 + M * N * mx.OUT_BYTES[out_type]


def workload_name(M, N, K, out_type):
    return f"mxfp6_gemm_{M}x{N}x{K}_{mx.OUT_NAMES[out_type]}"


def profiled_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` on `workload` from profiles/*_pmc.txt (lines
    'workload: ...', 'kernel: ...', 'hbm_bytes_per_launch: N'), or None."""
    if not os.path.isdir(PROFILES):
        return None
    for fn in sorted(os.listdir(PROFILES)):
        if not fn.endswith("_pmc.txt"):
            continue
        with open(os.path.join(PROFILES, fn)) as f:
            txt = f.read()
        w = re.search(r"^workload:\s*(\S+)", txt, re.M)
        k = re.search(r"^kernel:\s*(.+)$", txt, re.M)
        b = re.search(r"^hbm_bytes_per_launch:\s*([0-9.eE+]+)", txt, re.M)
        if w and k and b and w.group(1) == workload and k.group(1).strip() == kernel:
            return float(b.group(1))
    return None


class ClockProbe:
    """The graphics clock over a region of GPU work, from two clock samples of the library
    (mxfp6_clock_sample_async: each of 256 one-wave workgroups reads its CU's shader cycle
    counter and the 100 MHz reference counter) launched on the same stream just before and just
    after the region, outside its timing events. stop() returns the mean over the XCDs (MHz)."""

    NWG = 256

    def __init__(self):
        import torch
        self.bufs = [torch.zeros(self.NWG * 4, dtype=torch.int64, device="cuda:0")
                     for _ in range(2)]
        self.per_xcd = None

    def _sample(self, i, stream):
        if mx.clock_sample(self.bufs[i].data_ptr(), self.NWG, stream.cuda_stream) != 0:
            raise RuntimeError("clock sample failed")

    def start(self, stream):
        self._sample(0, stream)

    def stop(self, stream):
        import torch
        self._sample(1, stream)
        torch.cuda.synchronize()
        a, b = (t.cpu().numpy().reshape(self.NWG, 4) for t in self.bufs)
        self.per_xcd = mx.clock_between(a, b)
        if not self.per_xcd:
            return None
        return round(sum(self.per_xcd.values()) / len(self.per_xcd), 1)


def frac_at(tflops, mhz):
    """Fraction of the dense MXFP6 MFMA peak at the given graphics clock."""
    return round(tflops * 1e12 / (FLOP_PER_CLK * mhz * 1e6), 4) if mhz else None


def host_threads():
    """Threads for the CPU baseline: the process's CPU share. OMP_NUM_THREADS when set (a GPU box
    gives one GPU's jobs 16 host threads and sets it so), else the CPUs this process may run on;
    never more than the latter."""
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    try:
        want = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        want = 0
    return max(1, min(avail, want) if want > 0 else avail)


def cpu_baseline(p, target_cpu_s=12.0):
    """The reference CPU GEMM's arithmetic (tests/reference.hpp: dequantise both operands to FP32,
    then one sequential FP32 dot per output; the oracle's restatement, pinned bit-exact to the
    reference function) on the same operands, on this host's cores. B is dequantised once (timed);
    the dots are timed on a bounded sample of A rows and scaled by M / rows (their cost is exactly
    linear in the number of rows); a workload whose dots fit the time target runs in full."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    threads = host_threads()
    t0 = time.perf_counter()
    bf = oracle.dequant_f32(p.b_packed, p.b_row_bytes, p.b_scales, p.N, p.K)
    t_deq = time.perf_counter() - t0
    t0 = time.perf_counter()
    oracle.gemm_f32_seq_deq(p.a_packed, p.a_row_bytes, p.a_scales, bf, p.M, p.N, p.K,
                            np.zeros(1, dtype=np.int32), nthreads=1)
    per_row = max(time.perf_counter() - t0, 1e-5)
    nrows = int(min(p.M, max(threads, round(target_cpu_s / per_row))))
    nrows = max(threads, nrows // threads * threads)
    rows = np.linspace(0, p.M - 1, nrows).astype(np.int32)
    t0 = time.perf_counter()
    oracle.gemm_f32_seq_deq(p.a_packed, p.a_row_bytes, p.a_scales, bf, p.M, p.N, p.K, rows,
                            nthreads=threads)
    t_rows = time.perf_counter() - t0
    full = t_deq + t_rows * p.M / nrows
    whole = nrows == p.M
    return {"value": round(2.0 * p.M * p.N * p.K / full / 1e12, 6), "unit": "TFLOP/s",
            "cores": threads, "host_cpus": os.cpu_count(), "kind": "port", "full": whole,
            "sample": f"B dequantised once ({t_deq:.2f} s, 1 thread) + dots of "
                      + (f"all {p.M} A rows x {p.N} columns ({t_rows:.3f} s on {threads} threads): "
                         f"{full:.3f} s per GEMM" if whole else
                         f"{nrows} of {p.M} A rows x {p.N} columns ({t_rows:.2f} s on {threads} "
                         f"threads), scaled x{p.M / nrows:.1f}: {full:.1f} s per GEMM")}


def copy_calibration(mib=256, reps=5):
    """A plain device copy of known size (torch's copy kernel), for scaling the FETCH_SIZE and
    WRITE_SIZE counters: each launch reads and writes exactly `mib` MiB."""
    import torch
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] copy calibration: {reps} copies of {mib} MiB")


def reference_library():
    """The reference GPU library built from its own sources (oracle/_ref), or None."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    try:
        import oracle
        return oracle.ref()
    except Exception as e:
        log(f"[bench] reference library unavailable: {e}")
        return None


def best_of(fn, stream, reps=4, n=20, warm=8):
    """The reference's timing method (tests/test_gemm.cpp:33-55): `warm` calls, then `reps`
    repetitions of `n` back-to-back calls between two events; returns (best mean, median mean)
    in milliseconds and the graphics clock (MHz) over the best repetition (clock samples taken
    right outside its events, so no host-side gap between repetitions dilutes it)."""
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    means, clocks = [], []
    clock = ClockProbe()
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        clock.start(stream)
        a.record(stream)
        for _ in range(n):
            fn()
        b.record(stream)
        clocks.append(clock.stop(stream))
        means.append(a.elapsed_time(b) / n)
    best = int(np.argmin(means))
    return means[best], float(np.median(means)), clocks[best]


class Workload:
    """Device operands of one workload for this library's route and, when the reference library
    is given, for the reference library's own route (its scale grouping and workspace)."""

    def __init__(self, name, ref=None, shape=None):
        """name: a CONFIGS workload; or shape = (M, N, K): FP16 out, A and B from N(0,1)."""
        import torch
        if shape is None:
            M, N, K, ot, (da, sa_), (db, sb_), desc = CONFIGS[name]
            seed = SEED ^ int(name[1:])
        else:
            (M, N, K), ot = shape, mx.OUT_F16
            (da, sa_), (db, sb_), desc = (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0), "A,B ~ N(0,1)"
            seed = SEED ^ (M * 7 + N * 3 + K)
        self.name, self.M, self.N, self.K, self.ot, self.desc = name, M, N, K, ot, desc
        t0 = time.perf_counter()
        p = mx.make_problem(M, N, K, da, sa_, db, sb_, seed=seed)
        self.p = p
        dev = torch.device("cuda:0")
        self.tile = mx.choose_tile(M, N, p.Kp)
        self.S = mx.splitk_segments(M, N, p.Kp)
        self.repack = mx.repacks_a(M, N, p.Kp)
        bsh, sa, sb = p.layouts(self.tile)
        self.dA = torch.from_numpy(p.a_packed).to(dev)
        self.dB, self.dsa, self.dsb = (torch.from_numpy(x).to(dev) for x in (bsh, sa, sb))
        self.D = torch.empty(M * N * mx.OUT_BYTES[ot], dtype=torch.uint8, device=dev)
        self.ws_bytes = mx.preferred_workspace_size(M, N, p.Kp)
        self.ws = torch.empty(max(self.ws_bytes, 4), dtype=torch.uint8, device=dev)
        self.ref = ref
        if ref is not None:
            import ctypes as C
            tr = (C.c_int * 4)()
            ref.ref_choose_tile(M, N, p.Kp, tr)
            self.ref_tile = tuple(tr)
            if self.ref_tile == tuple(self.tile):
                self.rB, self.rsa, self.rsb = self.dB, self.dsa, self.dsb
            else:
                rbsh, rsa, rsb = p.layouts(self.ref_tile)
                self.rB, self.rsa, self.rsb = (torch.from_numpy(x).to(dev)
                                               for x in (rbsh, rsa, rsb))
            self.rws_bytes = ref.ref_gemm_workspace_size(M, N, p.Kp)
            self.rws = torch.empty(max(self.rws_bytes, 4), dtype=torch.uint8, device=dev)
            self.rD = torch.empty_like(self.D)
        self.flops = 2.0 * M * N * K
        log(f"[bench] {name}: {M}x{N}x{K} (Kp {p.Kp}) tile {self.tile} S {self.S} repack A "
            f"{self.repack} ws {self.ws_bytes} B; inputs ready in {time.perf_counter() - t0:.1f} s")

    def ours(self, stream):
        rc = mx.gemm(self.ot, self.M, self.N, self.p.Kp, self.dA.data_ptr(), self.dB.data_ptr(),
                     self.dsa.data_ptr(), self.dsb.data_ptr(), self.D.data_ptr(),
                     self.p.a_row_bytes, self.ws.data_ptr() if self.ws_bytes else 0,
                     self.ws_bytes, stream=stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(f"mxfp6_gemm failed: {mx.STATUS.get(rc, rc)}")

    def theirs(self, stream):
        # the reference API launches on the null stream; the timing events go on that stream too
        self.ref.ref_gemm(self.ot, self.M, self.N, self.p.Kp, self.dA.data_ptr(),
                          self.rB.data_ptr(), self.rsa.data_ptr(), self.rsb.data_ptr(),
                          self.rD.data_ptr(), self.p.a_row_bytes, self.p.b_row_bytes,
                          self.rws.data_ptr() if self.rws_bytes else None, self.rws_bytes)

    def agree(self):
        """Loose sanity check between the two libraries' outputs (full parity is the tests'
        job): the largest difference relative to the largest magnitude."""
        import torch
        tt = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}[self.ot]
        a = self.D.view(tt).float()
        b = self.rD.view(tt).float()
        return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def compare(w, stream):
    """This library and the reference library on the same operands, by the reference's timing
    method, one after the other, with the clock each ran at."""
    import torch
    null = torch.cuda.default_stream()
    ms_o, med_o, sclk_o = best_of(lambda: w.ours(stream), stream)
    out = {"workload": workload_name(w.M, w.N, w.K, w.ot), "tile": list(w.tile),
           "splitk": w.S, "a_repacked": w.repack, "us": round(ms_o * 1e3, 2),
           "tflops": round(w.flops / ms_o / 1e9, 1),
           "frac": round(w.flops / ms_o / 1e9 / PEAK_TFLOPS, 4),
           "median_us": round(med_o * 1e3, 2), "sclk_mhz": sclk_o,
           "frac_at_sclk": frac_at(w.flops / ms_o / 1e9, sclk_o)}
    if w.S > 1:
        # algorithmic bytes, and with the split-K partials written and read back
        ab = alg_bytes(w.M, w.N, w.K, w.ot)
        out["hbm_gbs_alg"] = round(ab / ms_o / 1e6, 1)
        out["hbm_gbs_alg_with_partials"] = round(
            (ab + 2 * 4 * w.S * w.M * w.N) / ms_o / 1e6, 1)
    if w.ref is not None:
        ms_r, med_r, sclk_r = best_of(lambda: w.theirs(null), null)
        tf_r = w.flops / ms_r / 1e9
        out.update({"ref_tile": list(w.ref_tile), "ref_us": round(ms_r * 1e3, 2),
                    "ref_tflops": round(tf_r, 1), "ref_median_us": round(med_r * 1e3, 2),
                    "ref_sclk_mhz": sclk_r,
                    "ratio": round(ms_r / ms_o, 3), "max_rel_diff_vs_ref": w.agree()})
    log(f"[bench] {w.name}: ours {out['us']} us ({out['tflops']} TF, {sclk_o} MHz)" +
        (f" | reference {out['ref_us']} us ({out['ref_tflops']} TF, {out['ref_sclk_mhz']} MHz)"
         f" | ratio {out['ratio']}"
         if w.ref is not None else ""))
    return out


def headline(name, steps, warmup, ref, w=None):
    """The contract measurement of one workload: `warmup` untimed steps, then exactly `steps`
    steps between two synchronisations; then the dominant kernel timed alone. w: the workload's
    operands when already on the device."""
    import torch
    if w is None:
        w = Workload(name, ref)
    M, N, K, p = w.M, w.N, w.K, w.p
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        w.ours(stream)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    clock = ClockProbe()
    clock.start(stream)
    w0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        w.ours(stream)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - w0) * 1e3
    sclk = clock.stop(stream)
    sclk_xcd = clock.per_xcd
    ms = ev0.elapsed_time(ev1) / steps
    tflops = w.flops / (ms * 1e-3) / 1e12

    # dominant kernel: the same launches issued one by one, HIP events around the tile kernel
    kernel_name = "wide_kernel" if tuple(w.tile) in WIDE_TILES else "slab_kernel"
    if w.S == 1 and w.repack:
        ash = torch.empty(mx.preshuffled_bytes(M, p.Kp), dtype=torch.uint8, device="cuda:0")
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(steps)]
        sp = stream.cuda_stream

        def split_step(i):
            # what gemm() does for this plan, launch by launch: repack A, then the tile kernel
            # reading the repacked copy (A layout 2)
            if mx.preshuffle_rows(w.dA.data_ptr(), p.a_row_bytes, M, p.Kp, ash.data_ptr(), sp):
                raise RuntimeError("repack failed")
            if i >= 0:
                evs[i][0].record(stream)
            rc = mx.gemm_explicit(w.ot, M, N, p.Kp, w.tile, 1, ash.data_ptr(), w.dB.data_ptr(),
                                  w.dsa.data_ptr(), w.dsb.data_ptr(), w.D.data_ptr(),
                                  p.a_row_bytes, stream=sp, a_layout=mx.A_PRESHUFFLED)
            if rc != 0:
                raise RuntimeError(f"mxfp6_gemm_explicit failed: {mx.STATUS.get(rc, rc)}")
            if i >= 0:
                evs[i][1].record(stream)

        for _ in range(max(2, warmup // 2)):
            split_step(-1)
        torch.cuda.synchronize()
        clock.start(stream)
        for i in range(steps):
            split_step(i)
        torch.cuda.synchronize()
        k_sclk = clock.stop(stream)
        k_ms = sum(a.elapsed_time(b) for a, b in evs) / steps
        kernel_scope = "tile kernel alone (repack of A timed outside)"
    else:
        k_ms, k_sclk = ms, sclk
        kernel_scope = "whole step (" + ("tile kernel + split-K reduce" if w.S > 1 else
                                         "tile kernel") + ")"
    k_tflops = w.flops / (k_ms * 1e-3) / 1e12
    log(f"[bench] {name}: {ms * 1e3:.1f} us/step over {steps} steps ({tflops:.1f} TFLOP/s, "
        f"sclk {sclk} MHz), tile kernel {k_ms * 1e3:.1f} us ({k_tflops:.1f} TFLOP/s, sclk "
        f"{k_sclk} MHz), wall {wall_ms:.1f} ms")
    workload = workload_name(M, N, K, w.ot)
    out = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp6_e2m3 (fp32 accumulate)",
        "data": "synthetic",
        "config": {"workload": workload, "M": M, "N": N, "K": K, "Kp": p.Kp,
                   "out": mx.OUT_NAMES[w.ot], "inputs": w.desc, "tile": list(w.tile),
                   "splitk": w.S, "a_repacked": w.repack, "a_layout": "compact row-major",
                   "workspace_bytes": w.ws_bytes, "parallelism": "single GPU"},
        "pct_of_peak": round(100.0 * tflops / PEAK_TFLOPS, 2),
        "sclk_mhz": sclk,
        "sclk_mhz_per_xcd": [round(v, 1) for v in sclk_xcd.values()] if sclk_xcd else None,
        "frac_at_sclk": frac_at(tflops, sclk),
        "hbm_gbs_alg": round(alg_bytes(M, N, K, w.ot) / (ms * 1e-3) / 1e9, 1),
        "roofline": {"bound": "mfma", "achieved": round(k_tflops, 2), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(k_tflops / PEAK_TFLOPS, 4),
                     "traffic": profiled_traffic(workload, kernel_name), "kernel": kernel_name,
                     "scope": kernel_scope, "kernel_ms": round(k_ms, 6), "sclk_mhz": k_sclk,
                     "frac_at_sclk": frac_at(k_tflops, k_sclk)},
    }
    return w, out


def run(names, steps, warmup, with_cpu, with_ref, per_config):
    import torch
    ref = reference_library() if with_ref else None
    lines = []
    cpu_done = {}
    # The per-workload comparisons (GPU launches only) run before the headline, its operands
    # already on the device, so the headline's warm-up and timed steps follow seconds of GEMMs
    # instead of an idle GPU near 160 MHz; the CPU baselines run last.
    pc, probs, ready = {}, {}, {}
    if per_config:
        # the headline's own workload last: the timed loop then follows the same GEMM (after a
        # different one, the 20-step loop ran at 1356 MHz against 1496 in that comparison)
        ready[names[0]] = Workload(names[0], ref)
        for n in sorted(CONFIGS, key=lambda c: (c == names[0], c)):
            w = ready[n] if n in ready else Workload(n, ref)
            pc[n] = compare(w, torch.cuda.current_stream())
            probs[n] = w.p
            if n not in ready:
                del w
                torch.cuda.empty_cache()
    for n in names:
        w, out = headline(n, steps, warmup, ref, ready.pop(n, None))
        if ref is not None:
            c = compare(w, torch.cuda.current_stream())
            out["vs_baseline"] = round(out["value"] / c["ref_tflops"], 3)
            out["baseline"] = {
                "kind": "reference GPU library (libmxfp6gemm built from its own sources), same "
                        "process, same operands, its own router; timed by its own method "
                        "(8 warm-ups, best mean of 4 x 20 launches)",
                "value": c["ref_tflops"], "unit": "TFLOP/s", "tile": c["ref_tile"],
                "ours_same_method_tflops": c["tflops"], "ratio_same_method": c["ratio"]}
        probs.setdefault(n, w.p)
        lines.append((w, out))
        del w
        torch.cuda.empty_cache()
    if with_cpu:
        log(f"[bench] {names[0]}: CPU baseline ...")
        lines[0][1]["cpu_baseline"] = cpu_done[names[0]] = cpu_baseline(probs[names[0]])
    if per_config:
        for n in sorted(CONFIGS):
            if with_cpu:
                # every workload beside the reference CPU path (the headline's own sample where
                # it was just taken; the small workload runs in full)
                if n not in cpu_done:
                    log(f"[bench] {n}: CPU baseline ...")
                    cpu_done[n] = cpu_baseline(probs[n])
                pc[n]["cpu_baseline"] = cpu_done[n]
        lines[0][1]["per_config"] = {n: pc[n] for n in sorted(pc)}
    for _, out in lines:
        print(json.dumps(out), flush=True)


def run_prep(steps, warmup):
    """Operand preparation on the device at the default workload's size: float A[8192][8192] ->
    packed rows + tiled scales (prepare_a), float B[8192][8192] -> preshuffled B^T + tiled scales
    (prepare_b), one step = both calls. Algorithmic bytes per value: 4 read, 0.75 + 1/32 written
    (padded to kpad(K) = 8256)."""
    import torch

    M = N = K = 8192
    Kp = mx.kpad(K)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(SEED)
    A = torch.randn(M, K, device=dev, generator=g)
    B = torch.randn(K, N, device=dev, generator=g)
    rb = Kp // 4 * 3
    pa = torch.empty(M * rb, dtype=torch.uint8, device=dev)
    ta = torch.empty(mx.tiled_scale_bytes(M, K, 4), dtype=torch.uint8, device=dev)
    pb = torch.empty(mx.preshuffled_bytes(N, K), dtype=torch.uint8, device=dev)
    tb = torch.empty(mx.tiled_scale_bytes(N, K, 4), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    calls = {
        "prep_rows_kernel": lambda: mx.prepare_a_dev(A.data_ptr(), M, K, 4, pa.data_ptr(), rb,
                                                     ta.data_ptr(), sp),
        "prep_b_kernel": lambda: mx.prepare_b_dev(B.data_ptr(), K, N, 4, pb.data_ptr(),
                                                  tb.data_ptr(), sp),
    }
    for _ in range(warmup):
        for c in calls.values():
            assert c() == 0
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        for k, c in calls.items():
            if c() != 0:
                raise RuntimeError(f"{k} failed")
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # each kernel alone: `steps` back-to-back launches between two events on the launch stream
    k_ms = {}
    for k, c in calls.items():
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(steps):
            c()
        b.record(stream)
        torch.cuda.synchronize()
        k_ms[k] = a.elapsed_time(b) / steps
    per_op = M * K * 4 + M * Kp * 3 // 4 + M * Kp // 32  # A and B have the same shape
    gbs = 2 * per_op / (ms * 1e-3) / 1e9
    dom = max(k_ms, key=k_ms.get)
    achieved = per_op / (k_ms[dom] * 1e-3) / 1e9
    workload = f"mxfp6_prepare_{M}x{K}"
    log(f"[bench] prepare: {ms * 1e3:.1f} us/step; " +
        ", ".join(f"{k} {v * 1e3:.1f} us ({per_op / (v * 1e-3) / 1e9:.0f} GB/s)"
                  for k, v in k_ms.items()))
    return {
        "metric": "MXFP6 operand preparation (quantize + device layouts) GB/s, 1xMI355X",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32 -> mxfp6_e2m3", "data": "synthetic",
        "config": {"workload": workload, "A": [M, K], "B": [K, N], "Kp": Kp, "group": 4,
                   "inputs": "N(0,1) float32", "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                     "traffic": profiled_traffic(workload, dom), "kernel": dom,
                     "kernel_ms": round(k_ms[dom], 6)},
    }


def default_map():
    """154 shapes: M in {1024, 2048, 4096, 8192} x N in {1024, 4096, 8192} x K in {1024 ... 16384},
    four more (the reference's weakest bands: short K on a wide grid, N a multiple of 128 but
    not of 256, a small square), and 90 drawn with a fixed seed (M, N multiples of 128, K from 256 to 65536,
    between 1 GFLOP and 1.2 TFLOP)."""
    import random
    shapes = [(M, N, K) for M in (1024, 2048, 4096, 8192) for N in (1024, 4096, 8192)
              for K in (1024, 2048, 4096, 8192, 16384)]
    shapes += [(2048, 102272, 1024), (8192, 896, 8192), (4096, 2432, 8192), (2048, 2048, 2048)]
    rng = random.Random(20261202)
    ms = [128, 256, 384, 512, 640, 768, 1024, 1280, 1536, 2048, 3072, 4096, 6144]
    ns = [128, 256, 384, 640, 896, 1152, 1536, 2176, 2560, 3072, 3584, 5120, 6144, 7168, 10240,
          14336]
    ks = [256, 512, 768, 1536, 2048, 3072, 5120, 6144, 12288, 24576, 32768, 65536]
    drawn = set()
    while len(drawn) < 90:
        M, N, K = rng.choice(ms), rng.choice(ns), rng.choice(ks)
        if 1e9 <= 2.0 * M * N * K <= 1.2e12:
            drawn.add((M, N, K))
    return shapes + [s for s in sorted(drawn) if s not in shapes]


def second_map():
    """160 shapes drawn with another seed from other sizes than default_map's (N multiples of
    384 among them, K up to 73728, M up to 16384), between 1 GFLOP and 1.5 TFLOP: a check that
    the router's and kernels' standing against the reference holds off the shapes they were
    tuned on."""
    import random
    rng = random.Random(777)
    ms = [128, 256, 384, 512, 768, 1024, 1536, 2048, 2560, 3072, 4096, 5120, 6144, 8192, 12288,
          16384]
    ns = [256, 384, 768, 1152, 1536, 2304, 3072, 3840, 4608, 5376, 6144, 7680, 9216, 10752, 12288,
          13824, 18432, 24576]
    ks = [256, 512, 1024, 1536, 2304, 3072, 4608, 6144, 9216, 12288, 18432, 24576, 36864, 49152,
          73728]
    drawn = set()
    while len(drawn) < 160:
        M, N, K = rng.choice(ms), rng.choice(ns), rng.choice(ks)
        if 1e9 <= 2.0 * M * N * K <= 1.5e12:
            drawn.add((M, N, K))
    return sorted(drawn)


def run_map(spec, repeat=1):
    """This library and the reference library on the same operands, shape by shape, by the
    reference's timing method (compare()); one JSON line per shape, then a summary line. With
    repeat > 1 each shape is timed `repeat` more times per library, alternating which library
    runs first, and the line also carries both series and the ratio of their medians."""
    import torch
    ref = reference_library()
    if ref is None:
        raise SystemExit("--map needs the reference library (oracle/_ref/libmxfp6ref.so)")
    if spec == "second":
        shapes = second_map()
    elif spec:
        txt = open(spec).read() if os.path.exists(spec) else spec
        shapes = [tuple(int(v) for v in t.strip().split("x")) for t in txt.split(",") if t.strip()]
    else:
        shapes = default_map()
    stream = torch.cuda.current_stream()
    ratios = []
    for i, sh in enumerate(shapes):
        w = Workload(f"{sh[0]}x{sh[1]}x{sh[2]}", ref, shape=sh)
        c = compare(w, stream)
        line = {"shape": list(sh), "tile": c["tile"], "splitk": c["splitk"],
                "a_repacked": c["a_repacked"], "us": c["us"], "ref_tile": c["ref_tile"],
                "ref_us": c["ref_us"], "ratio": c["ratio"]}
        if repeat > 1:
            null = torch.cuda.default_stream()
            runs = {"ours": [], "ref": []}
            for r in range(repeat):
                order = [("ours", lambda: w.ours(stream), stream),
                         ("ref", lambda: w.theirs(null), null)]
                for tag, fn, s in (order if r % 2 == 0 else order[::-1]):
                    runs[tag].append(round(best_of(fn, s)[0] * 1e3, 2))
            line.update({"repeat_us": runs["ours"], "repeat_ref_us": runs["ref"],
                         "ratio_median": round(float(np.median(runs["ref"])) /
                                               float(np.median(runs["ours"])), 3)})
        ratios.append(line.get("ratio_median", c["ratio"]))
        print(json.dumps(line), flush=True)
        del w
        torch.cuda.empty_cache()
    gm = float(np.exp(np.mean(np.log(ratios))))
    print(json.dumps({"shapes": len(ratios), "geomean_ratio": round(gm, 3),
                      "min_ratio": min(ratios), "max_ratio": max(ratios),
                      "below_1": int(sum(r < 1.0 for r in ratios))}), flush=True)


def smi_power_clock():
    """amd-smi's socket power (W) and the mean graphics clock over the XCDs (MHz) of the one
    visible GPU, or None (no amd-smi, no reading, or more than one GPU listed)."""
    try:
        out = subprocess.run(["amd-smi", "metric", "--power", "--clock"], capture_output=True,
                             text=True, timeout=30).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    if len(re.findall(r"^GPU:", out, re.M)) != 1:
        return None
    pw = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", out)
    clks = [int(x) for x in re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*(\d+)\s*MHz", out)]
    if not pw:
        return None
    return float(pw.group(1)), (sum(clks) / len(clks) if clks else None)


def power_cap_w():
    """The board's power cap (W) as rocm-smi reports it, or None."""
    try:
        out = subprocess.run(["rocm-smi", "--showmaxpower"], capture_output=True, text=True,
                             timeout=30).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    caps = re.findall(r"Max Graphics Package Power \(W\):\s*([0-9.]+)", out)
    return float(caps[0]) if len(caps) == 1 else None


def run_power(name, seconds):
    """Back-to-back GEMMs of one workload for `seconds` (after 2 s of the same), this library and
    then the reference library on the same operands, sampling amd-smi's socket power and clocks
    every 0.25 s in a thread: where the board sits against its power limit while each runs."""
    import torch
    ref = reference_library()
    w = Workload(name, ref)
    stream = torch.cuda.current_stream()
    out = {"metric": "board power and clocks during back-to-back MXFP6 GEMMs, 1xMI355X",
           "workload": workload_name(w.M, w.N, w.K, w.ot), "seconds": seconds,
           "power_cap_w": power_cap_w()}
    runs = [("this_library", lambda: w.ours(stream))]
    if ref is not None:
        runs.append(("reference_library", lambda: w.theirs(stream)))
    for label, fn in runs:
        t0 = time.time()
        while time.time() - t0 < 2.0:
            for _ in range(20):
                fn()
            torch.cuda.synchronize()
        samples, done = [], threading.Event()

        def sample():
            while not done.is_set():
                r = smi_power_clock()
                if r is not None:
                    samples.append(r)
                done.wait(0.25)
        th = threading.Thread(target=sample)
        th.start()
        calls, t1 = 0, time.time()
        while time.time() - t1 < seconds:
            for _ in range(20):
                fn()
            torch.cuda.synchronize()
            calls += 20
        el = time.time() - t1
        done.set()
        th.join()
        pw = [s[0] for s in samples]
        ck = [s[1] for s in samples if s[1] is not None]
        out[label] = {"calls": calls, "us_per_call": round(el / calls * 1e6, 1),
                      "tflops": round(w.flops * calls / el / 1e12, 1),
                      "socket_power_w_mean": round(sum(pw) / len(pw), 1) if pw else None,
                      "socket_power_w_max": max(pw) if pw else None,
                      "gfx_clock_mhz_mean": round(sum(ck) / len(ck), 1) if ck else None,
                      "samples": len(samples)}
        if pw and out[label]["gfx_clock_mhz_mean"]:
            out[label]["joules_per_pflop"] = round(
                out[label]["socket_power_w_mean"] / (out[label]["tflops"] / 1000.0), 1)
    return out


def run_ab(name, plans, repeat):
    """Explicit plans of one workload against each other (and the routed plan), on the same
    operands, each timed by the reference's method (compare()'s best_of), `repeat` rounds with
    the order rotating every round; prints one JSON line with every plan's series and median.
    plans: "MTxNTxMPWxNPW[:S[:r|p|s]]" separated by commas (S K segments; r: A repacked by the
    plan, the repack timed with it; p: A repacked once beforehand, the tile kernel alone on the
    preshuffled copy; s: row-major A staged in LDS in 12-byte units, swizzled, wide tiles)."""
    import torch
    w = Workload(name)
    M, N, Kp, p = w.M, w.N, w.p.Kp, w.p
    stream = torch.cuda.current_stream()
    dev = torch.device("cuda:0")
    entries = [("routed", lambda: w.ours(stream))]
    keep = []
    ash = None
    for spec in plans.split(","):
        parts = spec.strip().split(":")
        tile = tuple(int(v) for v in parts[0].split("x"))
        S = int(parts[1]) if len(parts) > 1 else 1
        lay = {"r": mx.A_REPACK, "p": mx.A_PRESHUFFLED, "s": mx.A_ROWS_SWIZZLED}.get(
            parts[2] if len(parts) > 2 else "", mx.A_ROWS)
        a_ptr = w.dA.data_ptr()
        if lay == mx.A_PRESHUFFLED:
            # A repacked once here, outside the timing: the tile kernel alone on preshuffled A
            if ash is None:
                ash = torch.empty(mx.preshuffled_bytes(M, Kp), dtype=torch.uint8, device=dev)
                if mx.preshuffle_rows(w.dA.data_ptr(), p.a_row_bytes, M, Kp, ash.data_ptr(),
                                      stream.cuda_stream):
                    raise RuntimeError("repack failed")
            a_ptr = ash.data_ptr()
        _, sa, sb = p.layouts(tile)
        dsa, dsb = torch.from_numpy(sa).to(dev), torch.from_numpy(sb).to(dev)
        wsb = mx.plan_workspace_size(M, N, Kp, S, lay == mx.A_REPACK)
        ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device=dev)
        keep.append((dsa, dsb, ws))

        def fn(tile=tile, S=S, lay=lay, a_ptr=a_ptr, dsa=dsa, dsb=dsb, ws=ws, wsb=wsb):
            rc = mx.gemm_explicit(w.ot, M, N, Kp, tile, S, a_ptr, w.dB.data_ptr(),
                                  dsa.data_ptr(), dsb.data_ptr(), w.D.data_ptr(), p.a_row_bytes,
                                  ws.data_ptr() if wsb else 0, wsb, stream=stream.cuda_stream,
                                  a_layout=lay)
            if rc != 0:
                raise RuntimeError(f"plan {tile} S {S}: {mx.STATUS.get(rc, rc)}")
        entries.append((spec.strip(), fn))
    series = {k: [] for k, _ in entries}
    for r in range(repeat):
        order = entries[r % len(entries):] + entries[:r % len(entries)]
        for k, fn in order:
            series[k].append(round(best_of(fn, stream)[0] * 1e3, 2))
    out = {"workload": workload_name(M, N, w.K, w.ot), "routed": {"tile": list(w.tile),
           "splitk": w.S, "a_repacked": w.repack}, "repeat": repeat,
           "method": "best mean of 4 x 20 launches after 8 warm-ups per run; plan order rotated "
                     "every run", "us": series,
           "median_us": {k: float(np.median(v)) for k, v in series.items()}}
    return out


def run_e2e(names):
    """Float A to D on the device, two ways, for each workload: quantise A into row-major rows
    (mxfp6_prepare_a_async) and run the routed gemm() on them (with its preferred workspace, so
    that it repacks where the router does), against quantising A straight into the preshuffled
    layout (mxfp6_prepare_a_preshuffled_async) and running the router's tile and split on it as
    an explicit plan (A layout 2). B is prepared once beforehand (a weight); each path is timed
    by the reference's method (best_of), both calls per step. FP32 A from N(0, sigma) of the
    workload, B from N(0, 1): the timing does not depend on the values."""
    import torch
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    out = {}
    for name in names:
        M, N, K, ot, (_, sa_), _, _ = CONFIGS[name]
        Kp = mx.kpad(K)
        tile = mx.choose_tile(M, N, Kp)
        S = mx.splitk_segments(M, N, Kp)
        g = torch.Generator(device=dev)
        g.manual_seed(SEED ^ int(name[1:]))
        A = torch.randn(M, K, device=dev, generator=g) * sa_
        B = torch.randn(K, N, device=dev, generator=g)
        rb = Kp // 4 * 3
        bsh = torch.empty(mx.preshuffled_bytes(N, K), dtype=torch.uint8, device=dev)
        tsb = torch.empty(mx.tiled_scale_bytes(N, K, tile[3]), dtype=torch.uint8, device=dev)
        if mx.prepare_b_dev(B.data_ptr(), K, N, tile[3], bsh.data_ptr(), tsb.data_ptr(), sp):
            raise RuntimeError("prepare_b failed")
        del B
        rows = torch.empty(M * rb, dtype=torch.uint8, device=dev)
        ash = torch.empty(mx.preshuffled_bytes(M, K), dtype=torch.uint8, device=dev)
        tsa = torch.empty(mx.tiled_scale_bytes(M, K, tile[2]), dtype=torch.uint8, device=dev)
        D = torch.empty(M * N * mx.OUT_BYTES[ot], dtype=torch.uint8, device=dev)
        wsr = mx.preferred_workspace_size(M, N, Kp)
        wse = mx.plan_workspace_size(M, N, Kp, S, False)
        ws = torch.empty(max(wsr, wse, 4), dtype=torch.uint8, device=dev)

        def via_rows():
            if mx.prepare_a_dev(A.data_ptr(), M, K, tile[2], rows.data_ptr(), rb,
                                tsa.data_ptr(), sp):
                raise RuntimeError("prepare_a failed")
            if mx.gemm(ot, M, N, Kp, rows.data_ptr(), bsh.data_ptr(), tsa.data_ptr(),
                       tsb.data_ptr(), D.data_ptr(), rb, ws.data_ptr(), wsr, stream=sp):
                raise RuntimeError("gemm failed")

        def via_preshuffled():
            if mx.prepare_a_preshuffled_dev(A.data_ptr(), M, K, tile[2], ash.data_ptr(),
                                            tsa.data_ptr(), sp):
                raise RuntimeError("prepare_a_preshuffled failed")
            if mx.gemm_explicit(ot, M, N, Kp, tile, S, ash.data_ptr(), bsh.data_ptr(),
                                tsa.data_ptr(), tsb.data_ptr(), D.data_ptr(), rb,
                                ws.data_ptr() if wse else 0, wse, stream=sp, a_layout=mx.A_PRESHUFFLED):
                raise RuntimeError("explicit gemm failed")

        t_rows = best_of(via_rows, stream)[0] * 1e3
        t_pre = best_of(via_preshuffled, stream)[0] * 1e3
        out[name] = {"workload": workload_name(M, N, K, ot), "tile": list(tile), "splitk": S,
                     "routed_repacks_a": bool(mx.repacks_a(M, N, Kp)),
                     "rows_then_gemm_us": round(t_rows, 1),
                     "preshuffled_then_explicit_us": round(t_pre, 1),
                     "ratio": round(t_rows / t_pre, 3)}
        log(f"[bench] e2e {name}: {out[name]}")
        del A, rows, ash, tsa, tsb, bsh, D, ws
        torch.cuda.empty_cache()
    return out


def diag_library():
    """libmxfp6diag.so (the MFMA-only diagnostic kernel), loaded with ctypes."""
    import ctypes as C
    path = os.path.join(ROOT, "mxfp6-gemm_amd", "lib", "libmxfp6diag.so")
    if not os.path.exists(path):
        raise SystemExit(f"{path} missing: build with make -C mxfp6-gemm_amd")
    lib = C.CDLL(path)
    f = lib.mxfp6_diag_mfma_roof_async
    f.restype = C.c_int
    f.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_int,
                  C.c_void_p, C.c_void_p]
    return lib


def run_roof(name, steps, warmup, seconds):
    """The MFMA-only diagnostic against the GEMM of one workload, in one process: the MFMA stream
    of the workload's tile kernel (its grid, its K slabs, 16 accumulators per wave for the 256x256
    tile) with every data path taken out, on the workload's real operand codes and scales. Both
    are timed like the headline (warmup, then `steps` launches between events, the clock sampled
    around them), and then each sustained for `seconds` with amd-smi sampling the board's power
    and clock. The diagnostic's cycle count per MFMA (from each wave's s_memtime) shows the issue
    rate of back-to-back MFMAs; its sustained rate is what the board's power limit leaves of the
    dense MXFP6 peak: the practical roof of any tile kernel on this board."""
    import torch
    w = Workload(name)
    if tuple(w.tile[:2]) not in ((256, 256), (128, 384)) or w.S != 1:
        raise SystemExit(f"--roof: workload {name} is not an unsplit 256x256 or 128x384 route")
    lib = diag_library()
    shape = 0 if tuple(w.tile[:2]) == (256, 256) else 1
    mb, npw = (8, 2) if shape == 0 else (4, 3)
    wgs = -(-w.M // w.tile[0]) * -(-w.N // w.tile[1])
    slabs = w.p.Kp // 64
    cyc = torch.zeros(wgs * 4, dtype=torch.int64, device="cuda:0")
    stream = torch.cuda.current_stream()
    op_blocks = w.dB.numel() // 1536
    sc_dwords = w.dsb.numel() // 4

    def roof():
        if lib.mxfp6_diag_mfma_roof_async(shape, w.dB.data_ptr(), op_blocks, w.dsb.data_ptr(),
                                          sc_dwords, cyc.data_ptr(), wgs, slabs, None,
                                          stream.cuda_stream):
            raise RuntimeError("mfma roof launch failed")

    mfma_flops = float(wgs) * 4 * slabs * mb * npw * 2 * 32 * 32 * 64
    out = {"metric": "MFMA-only roof vs GEMM, 1xMI355X", "workload": workload_name(w.M, w.N, w.K, w.ot),
           "tile": list(w.tile), "roof_grid": wgs, "roof_slabs": slabs,
           "roof_mfmas_per_wave": slabs * mb * npw, "steps": steps, "warmup": warmup,
           "power_cap_w": power_cap_w()}
    for label, fn, flops in (("mfma_only", roof, mfma_flops), ("gemm", lambda: w.ours(stream), w.flops)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        clock = ClockProbe()
        clock.start(stream)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        sclk = clock.stop(stream)
        ms = e0.elapsed_time(e1) / steps
        tf = flops / ms / 1e9
        r = {"us": round(ms * 1e3, 2), "tflops": round(tf, 1), "frac": round(tf / PEAK_TFLOPS, 4),
             "sclk_mhz": sclk, "frac_at_sclk": frac_at(tf, sclk)}
        if label == "mfma_only":
            c = cyc.cpu().numpy().astype(np.float64)
            r["cycles_per_mfma_mean"] = round(float(c.mean()) / (slabs * mb * npw), 2)
            r["cycles_per_mfma_min"] = round(float(c.min()) / (slabs * mb * npw), 2)
        out[label] = r
        log(f"[bench] roof {label}: {r}")
    if seconds > 0:
        for label, fn, flops in (("mfma_only", roof, mfma_flops), ("gemm", lambda: w.ours(stream), w.flops)):
            samples, done = [], threading.Event()

            def sample():
                while not done.is_set():
                    v = smi_power_clock()
                    if v is not None:
                        samples.append(v)
                    done.wait(0.25)
            t0 = time.time()
            while time.time() - t0 < 1.0:
                for _ in range(20):
                    fn()
                torch.cuda.synchronize()
            th = threading.Thread(target=sample)
            th.start()
            calls, t1 = 0, time.time()
            while time.time() - t1 < seconds:
                for _ in range(20):
                    fn()
                torch.cuda.synchronize()
                calls += 20
            el = time.time() - t1
            done.set()
            th.join()
            pw = [v[0] for v in samples]
            ck = [v[1] for v in samples if v[1] is not None]
            tf = flops * calls / el / 1e12
            out[label]["sustained"] = {
                "seconds": round(el, 1), "calls": calls, "tflops": round(tf, 1),
                "frac": round(tf / PEAK_TFLOPS, 4),
                "socket_power_w_mean": round(sum(pw) / len(pw), 1) if pw else None,
                "gfx_clock_mhz_mean": round(sum(ck) / len(ck), 1) if ck else None,
                "samples": len(samples)}
            log(f"[bench] roof {label} sustained: {out[label]['sustained']}")
    out["gemm_over_roof"] = round(out["gemm"]["tflops"] / out["mfma_only"]["tflops"], 4)
    if "sustained" in out["gemm"]:
        out["gemm_over_roof_sustained"] = round(out["gemm"]["sustained"]["tflops"] /
                                                out["mfma_only"]["sustained"]["tflops"], 4)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--all", action="store_true",
                    help="a headline line for every workload (vs_baseline each)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-ref", action="store_true",
                    help="skip the reference library baseline (vs_baseline null)")
    ap.add_argument("--no-per-config", action="store_true",
                    help="skip the per-workload comparison block")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run the 256 MiB copy kernel that calibrates the HBM byte counters")
    ap.add_argument("--prep", action="store_true",
                    help="time the device operand preparation (quantize + layouts) instead")
    ap.add_argument("--power", type=float, default=0.0, metavar="SECONDS",
                    help="board power and clocks over SECONDS of back-to-back GEMMs instead")
    ap.add_argument("--roof", type=float, default=None, nargs="?", const=5.0, metavar="SECONDS",
                    help="the MFMA-only diagnostic kernel against the workload's GEMM instead "
                         "(timed like the headline, then each sustained for SECONDS, default 5)")
    ap.add_argument("--ab", default=None, metavar="PLANS",
                    help="explicit plans of the workload against each other and the routed plan "
                         "instead (MTxNTxMPWxNPW[:S[:r|p|s]],...; r: repacked A, p: A "
                         "preshuffled beforehand, s: row-major A staged swizzled; with --repeat R "
                         "rounds)")
    ap.add_argument("--e2e", action="store_true",
                    help="float A to D on the device instead: quantise to row-major A + the routed "
                         "gemm against quantise to preshuffled A + the same plan (the workload, or "
                         "with --all the four large ones)")
    ap.add_argument("--map", nargs="?", const="", default=None, metavar="SHAPES",
                    help="this library against the reference library shape by shape instead "
                         "(MxNxK,... or a file of them; 'second': 160 other shapes; "
                         "default: 154 shapes)")
    ap.add_argument("--repeat", type=int, default=1, metavar="R",
                    help="with --map: time each shape R more times per library, alternating "
                         "which runs first, and summarise by the ratio of the medians")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py runs on exactly one GPU; --gpus {a.gpus} is not supported (the MXFP6 "
              "GEMM here is a single-GPU library; multi-GPU sharding is design-only).",
              file=sys.stderr)
        sys.exit(2)
    if a.copy_calibration:
        copy_calibration()
        return
    if a.prep:
        print(json.dumps(run_prep(a.steps, a.warmup)), flush=True)
        return
    if a.power > 0:
        print(json.dumps(run_power(a.config, a.power)), flush=True)
        return
    if a.e2e:
        print(json.dumps(run_e2e(["c2", "c3", "c4", "c5"] if a.all else [a.config])), flush=True)
        return
    if a.ab is not None:
        print(json.dumps(run_ab(a.config, a.ab, max(a.repeat, 1))), flush=True)
        return
    if a.roof is not None:
        print(json.dumps(run_roof(a.config, a.steps, a.warmup, a.roof)), flush=True)
        return
    if a.map is not None:
        run_map(a.map, a.repeat)
        return
    names = sorted(CONFIGS, key=lambda n: n != a.config) if a.all else [a.config]
    run(names, a.steps, a.warmup, not a.no_cpu, not a.no_ref, not a.no_per_config and not a.all)


if __name__ == "__main__":
    main()
