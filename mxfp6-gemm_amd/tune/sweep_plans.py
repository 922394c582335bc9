"""Measure every execution plan of libmxfp6gemm on the GPU, for re-fitting the router's model.

A plan is (tile, K segments S, A layout: 0 row-major, 1 repacked first; a tile that does not
divide M x N runs masked); each is timed through
mxfp6_gemm_explicit on FP16 output as the best mean of 3 x 20 back-to-back launches after 5
warm-ups. One JSON line per shape: {"shape": [M, N, K], "plans": [[us, tile, S, a_layout], ...]}
sorted by time.

  python mxfp6-gemm_amd/tune/sweep_plans.py 2048x2048x2048,8192x8192x8192 out.jsonl
  python mxfp6-gemm_amd/tune/sweep_plans.py SHAPES out.jsonl --tiles 128x512x4x4
      (only the plans of the listed tiles)
  python mxfp6-gemm_amd/tune/sweep_plans.py --merge base.jsonl new.jsonl merged.jsonl
      (each shape of base with the plans of the tiles measured in new replaced by new's)
"""
import json
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import torch  # noqa: E402

import mxfp6_amd as mx  # noqa: E402

TILES = [(128, 128, 2, 2), (128, 256, 2, 4), (128, 384, 4, 3), (256, 256, 4, 4), (256, 192, 4, 3),
         (128, 512, 4, 4), (128, 256, 4, 2), (256, 256, 4, 2), (64, 256, 2, 2), (32, 256, 1, 2),
         (64, 128, 2, 1), (32, 128, 1, 1)]
SPLITS = (1, 2, 3, 4, 6, 8, 12, 16)


def best_us(fn, reps=3, n=20, warm=5):
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
    return best * 1e3


def sweep(M, N, K, tiles=TILES):
    p = mx.make_problem(M, N, K, seed=7)
    kt = p.Kp // mx.K_TILE
    dA = torch.from_numpy(p.a_packed).cuda()
    D = torch.empty(M * N * 2, dtype=torch.uint8, device="cuda")
    res = []
    regular = M % 32 == 0 and N % 128 == 0
    for t in tiles:
        # the plans the router considers: on a regular shape (M % 32 == 0, N % 128 == 0) the
        # tiles whose MT divides M, N masked when NT does not divide it; on a ragged shape every
        # tile. The skinny tiles (fewer than 128 rows) are measured on M % 128 == 0 shapes only
        # up to 2048 workgroups (they lose on larger grids, and take long there).
        if regular and M % t[0]:
            continue
        if t[0] < 128 and M % 128 == 0 and -(-M // t[0]) * -(-N // t[1]) > 2048:
            continue
        bsh, sa, sb = p.layouts(t)
        dB, dsa, dsb = (torch.from_numpy(x).cuda() for x in (bsh, sa, sb))
        for S in SPLITS:
            if S > kt or (S > 1 and -(-M // t[0]) * -(-N // t[1]) * S > 2048):
                continue
            for rp in (0, 1):
                wsb = mx.plan_workspace_size(M, N, p.Kp, S, rp)
                ws = torch.empty(max(wsb, 4), dtype=torch.uint8, device="cuda")

                def fn():
                    rc = mx.gemm_explicit(mx.OUT_F16, M, N, p.Kp, t, S, dA.data_ptr(),
                                          dB.data_ptr(), dsa.data_ptr(), dsb.data_ptr(),
                                          D.data_ptr(), p.a_row_bytes, ws.data_ptr(), wsb,
                                          a_layout=rp)
                    assert rc == 0, mx.STATUS.get(rc, rc)

                res.append((best_us(fn), list(t), S, rp))
    res.sort()
    return {"shape": [M, N, K], "plans": [list(r) for r in res]}


def merge(base_path, new_path, out_path):
    new = {}
    for line in open(new_path):
        rec = json.loads(line)
        new[tuple(rec["shape"])] = rec["plans"]
    with open(out_path, "w") as out:
        for line in open(base_path):
            rec = json.loads(line)
            plans = new.get(tuple(rec["shape"]))
            if plans is not None:
                tiles = {tuple(pl[1]) for pl in plans}
                rec["plans"] = sorted([pl for pl in rec["plans"] if tuple(pl[1]) not in tiles] +
                                      plans)
            out.write(json.dumps(rec) + "\n")


def main():
    if sys.argv[1] == "--merge":
        merge(*sys.argv[2:5])
        return
    shapes = [tuple(int(v) for v in s.split("x")) for s in sys.argv[1].split(",")]
    tiles = TILES
    if "--tiles" in sys.argv:
        tiles = [tuple(int(v) for v in t.split("x"))
                 for t in sys.argv[sys.argv.index("--tiles") + 1].split(",")]
    with open(sys.argv[2], "a") as out:
        for M, N, K in shapes:
            rec = sweep(M, N, K, tiles)
            best = rec["plans"][0]
            print(f"{M}x{N}x{K}: best {best[0]:.1f} us tile {tuple(best[1])} S {best[2]} "
                  f"a_layout {best[3]} ({len(rec['plans'])} plans)", flush=True)
            out.write(json.dumps(rec) + "\n")
            out.flush()


if __name__ == "__main__":
    main()
