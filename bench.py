"""Benchmark of libmxfp6gemm on one MI355X: MXFP6 GEMM TFLOPs and fraction of the dense MXFP6
MFMA peak.

A step is one mxfp6_gemm_async call: the whole hot path the router picks for the shape (for the
default workload: the repack of A into the preshuffled layout, then the 256x256 tile kernel),
over operands already resident in HBM. Default workload: M = N = K = 8192, FP16 out, A and B
drawn from N(0,1) with the seeded PCG32 generator and quantised with the OCP MX rule.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2] [--all] [--no-cpu]
  python bench.py --prep      (device operand preparation: float -> MXFP6 device layouts, GB/s)

Prints one JSON line per workload (only the default one unless --all). Besides the contract
fields it reports:
  roofline      the dominant kernel (the tile kernel) against the dense MXFP6 MFMA peak: its
                algorithmic flops per launch / its average launch duration, timed live with HIP
                events on the launch stream in a second loop of K steps that issues the step's
                two launches separately (repack, then the tile kernel on the repacked A);
                traffic = HBM bytes per launch from the committed rocprofv3 counter summary of
                the same kernel and workload (FETCH_SIZE + WRITE_SIZE scaled by the copy-kernel
                calibration), null when no summary matches;
  cpu_baseline  the reference CPU GEMM's arithmetic on this host (a bounded sample, scaled).
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mxfp6-gemm_amd"))

import numpy as np  # noqa: E402

import mxfp6_amd as mx  # noqa: E402

SEED = 0x4D584636
# MI355X published dense MXFP6 / MXFP4 MFMA peak (TFLOP/s) and HBM bandwidth (GB/s)
PEAK_TFLOPS = 10100.0
PEAK_HBM_GBS = 8000.0

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


def cpu_baseline(p, target_cpu_s=12.0):
    """The reference CPU GEMM's arithmetic (tests/reference.hpp: dequantise both operands to FP32,
    then one sequential FP32 dot per output; the oracle's restatement, pinned bit-exact to the
    reference function) on the same operands, on this host's cores. B is dequantised once (timed);
    the dots are timed on a bounded sample of A rows and scaled by M / rows (their cost is exactly
    linear in the number of rows)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    threads = max(1, min(16, os.cpu_count() or 1))
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
    return {"value": round(2.0 * p.M * p.N * p.K / full / 1e12, 6), "unit": "TFLOP/s",
            "cores": threads, "kind": "port",
            "sample": f"B dequantised once ({t_deq:.2f} s, 1 thread) + dots of {nrows} of {p.M} "
                      f"A rows x {p.N} columns ({t_rows:.2f} s on {threads} threads), "
                      f"scaled x{p.M / nrows:.1f}: {full:.1f} s per GEMM"}


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


def run_config(name, steps, warmup, with_cpu):
    import torch

    M, N, K, out_type, (da, sa_), (db, sb_), desc = CONFIGS[name]
    cfg_idx = int(name[1:])
    t0 = time.perf_counter()
    p = mx.make_problem(M, N, K, da, sa_, db, sb_, seed=SEED ^ cfg_idx)
    tile = mx.choose_tile(M, N, p.Kp)
    S = mx.splitk_segments(M, N, p.Kp)
    repack = mx.repacks_a(M, N, p.Kp)
    bsh, sa, sb = p.layouts(tile)
    dev = torch.device("cuda:0")
    dA = torch.from_numpy(p.a_packed).to(dev)
    dB = torch.from_numpy(bsh).to(dev)
    dsa = torch.from_numpy(sa).to(dev)
    dsb = torch.from_numpy(sb).to(dev)
    D = torch.empty(M * N * mx.OUT_BYTES[out_type], dtype=torch.uint8, device=dev)
    ws_bytes = mx.workspace_size(M, N, p.Kp)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    log(f"[bench] {name}: {M}x{N}x{K} (Kp {p.Kp}) tile {tile} S {S} repack A {repack} "
        f"ws {ws_bytes} B; inputs ready in {time.perf_counter() - t0:.1f} s")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    args = (out_type, M, N, p.Kp, dA.data_ptr(), dB.data_ptr(), dsa.data_ptr(), dsb.data_ptr(),
            D.data_ptr(), p.a_row_bytes, ws.data_ptr() if ws_bytes else 0, ws_bytes)

    def step():
        rc = mx.gemm(*args, stream=sp)
        if rc != 0:
            raise RuntimeError(f"mxfp6_gemm failed: {mx.STATUS.get(rc, rc)}")

    flops = 2.0 * M * N * K
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # timed region: exactly `steps` steps between two synchronisations
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - w0) * 1e3
    ms = ev0.elapsed_time(ev1) / steps
    tflops = flops / (ms * 1e-3) / 1e12

    # dominant kernel: the same launches issued one by one, HIP events around the tile kernel
    kernel_name = "slab_kernel"
    if S == 1 and repack:
        ash = torch.empty(M * p.Kp // 4 * 3, dtype=torch.uint8, device=dev)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(steps)]

        def split_step(i):
            # what gemm() does for this plan, launch by launch: repack A, then the tile kernel
            # reading the repacked copy (A layout 2)
            if mx.preshuffle_rows(dA.data_ptr(), p.a_row_bytes, M, p.Kp, ash.data_ptr(), sp):
                raise RuntimeError("repack failed")
            if i >= 0:
                evs[i][0].record(stream)
            rc = mx.gemm_explicit(out_type, M, N, p.Kp, tile, 1, ash.data_ptr(), dB.data_ptr(),
                                  dsa.data_ptr(), dsb.data_ptr(), D.data_ptr(), p.a_row_bytes,
                                  stream=sp, a_layout=mx.A_PRESHUFFLED)
            if rc != 0:
                raise RuntimeError(f"mxfp6_gemm_explicit failed: {mx.STATUS.get(rc, rc)}")
            if i >= 0:
                evs[i][1].record(stream)

        for _ in range(max(2, warmup // 2)):
            split_step(-1)
        torch.cuda.synchronize()
        for i in range(steps):
            split_step(i)
        torch.cuda.synchronize()
        k_ms = sum(a.elapsed_time(b) for a, b in evs) / steps
        kernel_scope = "tile kernel alone (repack of A timed outside)"
    else:
        k_ms = ms
        kernel_scope = "whole step (" + ("tile kernel + split-K reduce" if S > 1 else
                                         "tile kernel") + ")"
    k_tflops = flops / (k_ms * 1e-3) / 1e12

    log(f"[bench] {name}: {ms * 1e3:.1f} us/step over {steps} steps ({tflops:.1f} TFLOP/s), "
        f"tile kernel {k_ms * 1e3:.1f} us ({k_tflops:.1f} TFLOP/s), wall {wall_ms:.1f} ms")
    workload = workload_name(M, N, K, out_type)
    traffic = profiled_traffic(workload, kernel_name)
    out = {
        "metric": "MXFP6 GEMM TFLOPs (FP16 out) and % of MXFP6 MFMA peak, 1xMI355X",
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
                   "out": mx.OUT_NAMES[out_type], "inputs": desc, "tile": list(tile),
                   "splitk": S, "a_repacked": repack, "a_layout": "compact row-major",
                   "parallelism": "single GPU"},
        "pct_of_peak": round(100.0 * tflops / PEAK_TFLOPS, 2),
        "hbm_gbs_alg": round(alg_bytes(M, N, K, out_type) / (ms * 1e-3) / 1e9, 1),
        "roofline": {"bound": "mfma", "achieved": round(k_tflops, 2), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(k_tflops / PEAK_TFLOPS, 4),
                     "traffic": traffic, "kernel": kernel_name, "scope": kernel_scope,
                     "kernel_ms": round(k_ms, 6)},
    }
    if with_cpu:
        log(f"[bench] {name}: CPU baseline ...")
        out["cpu_baseline"] = cpu_baseline(p)
    return out


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # long enough for the power controller's clock transient at the start of a burst of GEMMs
    # to settle (tens of milliseconds on MI355X)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--all", action="store_true", help="every workload, one JSON line each")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-clock", action="store_true", help=argparse.SUPPRESS)  # accepted, no-op
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run the 256 MiB copy kernel that calibrates the HBM byte counters")
    ap.add_argument("--prep", action="store_true",
                    help="time the device operand preparation (quantize + layouts) instead")
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
    names = sorted(CONFIGS) if a.all else [a.config]
    for n in names:
        print(json.dumps(run_config(n, a.steps, a.warmup, not a.no_cpu)), flush=True)


if __name__ == "__main__":
    main()
