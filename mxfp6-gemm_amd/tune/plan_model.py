"""The router's plan-time model (csrc/host/plan.cpp plan_time_us / best_plan) in Python, and its
least-squares fit to measured plans (sweep_plans.py output).

  python mxfp6-gemm_amd/tune/plan_model.py [plans.jsonl ...]   # refit, print the constants and
                                                              # how close the picks come to the
                                                              # measured best plan per shape
The constants in CONSTANTS are the ones compiled into plan.hpp; tests check that this model and
the library's router pick the same plans.
"""
import json
import math
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CUS = 256
K_TILE = 192
MAX_SPLITS = 16
TILES = [(256, 256, 4, 4), (256, 192, 4, 3), (128, 384, 4, 3), (128, 256, 2, 4), (128, 128, 2, 2)]
SKINNY = [(64, 256, 2, 2), (32, 256, 1, 2), (64, 128, 2, 1), (32, 128, 1, 1)]
NAMES = ["T_LAUNCH", "T_WG", "T_SLAB_MIN", "T_MFMA", "T_COPY_KB", "T_OUT_KB", "REPACK_BYTES_PER_US",
         "SPLIT_BYTES_PER_US", "A_ROWS_COST"]
CONSTANTS = {"T_LAUNCH": 2.61668, "T_WG": 1.17567, "T_SLAB_MIN": 0.187174, "T_MFMA": 0.00709531,
             "T_COPY_KB": 0.0153215, "T_OUT_KB": 0.0256923, "REPACK_BYTES_PER_US": 5.5e6,
             "SPLIT_BYTES_PER_US": 4.4079e6, "A_ROWS_COST": 0.581966}
# the repack rate is the repack kernel's measured one, not fitted
FIXED = {"REPACK_BYTES_PER_US": 5.5e6}
# plans within NEAR x the best of their shape weigh 1 in the fit, the others FAR_WEIGHT: the fit
# should rank the contenders, not predict every hopeless plan
NEAR, FAR_WEIGHT = 1.3, 0.2
PLAN_MIN_GAIN = 0.01


def plan_time_us(c, tile, M, N, Kp, S, repack):
    MT, NT = tile[0], tile[1]
    wg = -(-M // MT) * -(-N // NT) * S
    occ = 2 if (MT, NT) in ((128, 128), (32, 128)) else 1
    cap = CUS * occ
    waves = (wg + cap - 1) // cap
    per_cu = max(1, -(-min(wg, cap) // CUS))  # workgroups on the busiest CU
    mfmas = tile[2] * tile[3]
    slabs = (Kp // 64) / S
    copy_kb = (MT * 48.0 * (1.0 if repack else 1.0 + c["A_ROWS_COST"]) + NT // 32 * 1536.0) / 1024.0
    t_slab = max(c["T_SLAB_MIN"], per_cu * (c["T_MFMA"] * mfmas + c["T_COPY_KB"] * copy_kb))
    out_kb = MT * NT * (4.0 if S > 1 else 2.0) / 1024.0
    t_wg = c["T_WG"] + slabs * t_slab + c["T_OUT_KB"] * out_kb * per_cu
    t = c["T_LAUNCH"] + waves * t_wg
    if repack:
        t += c["T_LAUNCH"] + 2.0 * (-(-M // 32) * 32) * (Kp // 4 * 3.0) / c["REPACK_BYTES_PER_US"]
    if S > 1:
        t += c["T_LAUNCH"] + (4.0 * S * M * N + 2.0 * M * N) / c["SPLIT_BYTES_PER_US"]
    return t


def best_plan(c, M, N, Kp):
    """(tile, S, repack) with the least predicted time, visiting plans from the simplest and
    requiring a PLAN_MIN_GAIN lead to replace an earlier one (as plan.cpp does). Regular shapes
    (M % 32 == 0, N % 128 == 0) take the tiles whose MT divides M, the 32- and 64-row ones
    included (the last tile column masked when NT does not divide N, visited after every dividing
    plan) whose scale grouping divides the shape; ragged ones any tile, masked."""
    best, best_t = ((128, 128, 2, 2), 1, False), None
    kt = Kp // K_TILE
    regular = M % 32 == 0 and N % 128 == 0
    cands = (SKINNY if M % 128 else TILES + SKINNY) if regular else TILES + SKINNY
    for masked in ((False, True) if regular else (None,)):
        for rp in (False, True):
            for S in range(1, min(MAX_SPLITS, kt) + 1):
                for tile in cands:
                    if regular and (M % tile[0] or bool(N % tile[1]) != masked):
                        continue
                    # the header's tile_scale holds whole scale groups only
                    if regular and ((M // 32) % tile[2] or (N // 32) % tile[3]):
                        continue
                    t = plan_time_us(c, tile, M, N, Kp, S, rp)
                    if best_t is None or t < best_t * (1.0 - PLAN_MIN_GAIN):
                        best, best_t = (tile, S, rp), t
    return best


def load(paths):
    recs = []
    for p in paths:
        with open(p) as f:
            recs += [json.loads(line) for line in f if line.strip()]
    return recs


def fit(recs, start):
    import numpy as np
    from scipy.optimize import minimize

    names = [n for n in NAMES if n not in FIXED]

    def loss(x):
        c = dict(zip(names, np.abs(x)))
        c.update(FIXED)
        s = 0.0
        for r in recs:
            M, N, K = r["shape"]
            Kp = (K + K_TILE - 1) // K_TILE * K_TILE
            best = r["plans"][0][0]
            for us, tile, S, rp in r["plans"]:
                w = 1.0 if us < NEAR * best else FAR_WEIGHT
                s += w * (math.log(plan_time_us(c, tile, M, N, Kp, S, rp)) - math.log(us)) ** 2
        return s

    x0 = np.array([start[n] for n in names])
    res = minimize(loss, x0, method="Nelder-Mead",
                   options={"maxiter": 40000, "xatol": 1e-7, "fatol": 1e-9})
    c = dict(zip(names, [float(v) for v in np.abs(res.x)]))
    c.update(FIXED)
    return c, float(res.fun)


def evaluate(c, recs):
    """Measured time of the model's pick / measured best, per shape whose pick was measured."""
    out = []
    for r in recs:
        M, N, K = r["shape"]
        Kp = (K + K_TILE - 1) // K_TILE * K_TILE
        tile, S, rp = best_plan(c, M, N, Kp)
        meas = [p[0] for p in r["plans"] if tuple(p[1]) == tile and p[2] == S and p[3] == int(rp)]
        if meas:
            out.append((tuple(r["shape"]), meas[0] / r["plans"][0][0]))
    return out


def main():
    paths = sys.argv[1:] or [os.path.join(HERE, "plans_mi355x.jsonl")]
    recs = load(paths)
    # the constants are fitted on the shapes with M % 128 == 0 (every tile measured on them)
    fit_recs = [r for r in recs if r["shape"][0] % 128 == 0]
    c, l = fit(fit_recs, CONSTANTS)
    print("fitted constants (log-time loss %.3f over %d shapes):" % (l, len(fit_recs)))
    for n in NAMES:
        print(f"  {n:14s} {c[n]:.6g}")
    for label, sel in (("M % 128 == 0", lambda s: s[0] % 128 == 0),
                       ("skinny M", lambda s: s[0] % 128 != 0)):
        ev = [(s, g) for s, g in evaluate(c, recs) if sel(s)]
        if ev:
            gm = math.exp(sum(math.log(g) for _, g in ev) / len(ev))
            print(f"{label}: picks measured for {len(ev)} shapes: geomean {gm:.3f}x of the best, "
                  f"worst {max(g for _, g in ev):.3f}x")


if __name__ == "__main__":
    main()
