"""The router's plan-time model (csrc/host/plan.cpp plan_time_us / best_plan) in Python, and its
fit to measured plans (plans_mi355x.jsonl: one JSON line per shape with every plan's measured
time on one MI355X), which scores the plans the model picks.

  python mxfp6-gemm_amd/tune/plan_model.py [plans.jsonl ...]   # refit, print the constants and
                                                              # how close the picks come to the
                                                              # measured best plan per shape
  python mxfp6-gemm_amd/tune/plan_model.py --no-fit            # the same for CONSTANTS
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
SPLIT_CHOICES = (1, 2, 3, 4, 6, 8, 12, 16)
# the routed tiles (256x192 is implemented but not routed: plan.cpp kCands)
TILES = [(256, 256, 4, 4), (128, 384, 4, 3), (128, 256, 2, 4), (128, 128, 2, 2), (128, 512, 4, 4),
         (128, 256, 4, 2), (256, 256, 4, 2)]
# the 32 x 32 tile (tiny_kernel.hpp): routed by a measured rule ahead of the model (plan.cpp
# tiny_routed): at most two 32 x 32 blocks per CU and 2 to 28 K-tiles; on at most one block per CU
# up to 32, and up to 64 on at least a quarter as many blocks as CUs; in ceil(K-tiles / 4)
# segments up to 16 K-tiles (8 at 13-16 on at most one block per CU) and max(8, ceil(K-tiles / 4))
# past that (tiny_segments)
TINY = (32, 32, 1, 1)
# the tiles whose B goes straight to registers (wide_kernel.hpp)
WIDE = {(128, 512, 4, 4), (128, 384, 4, 3), (128, 256, 4, 2), (256, 256, 4, 2)}
SKINNY = [(64, 256, 2, 2), (32, 256, 1, 2), (64, 128, 2, 1), (32, 128, 1, 1)]
NAMES = ["T_LAUNCH", "T_WG", "T_SLAB_MIN", "T_MFMA", "T_COPY_KB", "T_BREG_KB", "T_L2_KB",
         "T_OUT_KB", "REPACK_BYTES_PER_US", "SPLIT_BYTES_PER_US", "A_ROWS_COST", "A_ROWS_COST_WIDE",
         "A_ROWS_LONG"]
CONSTANTS = {"T_LAUNCH": 2.40452, "T_WG": 0.806055, "T_SLAB_MIN": 0.183313, "T_MFMA": 0.00394993,
             "T_COPY_KB": 0.0165642, "T_BREG_KB": 0.00831597, "T_L2_KB": 7.1085e-05,
             "T_OUT_KB": 0.0216756, "REPACK_BYTES_PER_US": 5.5e6, "SPLIT_BYTES_PER_US": 4.05965e+06,
             "A_ROWS_COST": 0.572519, "A_ROWS_COST_WIDE": 0.0675946, "A_ROWS_LONG": 0.158036}
# the repack rate is the repack kernel's measured one, not fitted
FIXED = {"REPACK_BYTES_PER_US": 5.5e6}
# the fit: summed log(measured time of the pick / measured best) per shape (the benchmark
# workloads BENCH_WEIGHT x), plus REG_WEIGHT x the log-time least squares of every measured plan,
# those within NEAR x the best of their shape weighing 1, the others FAR_WEIGHT; a pick that was
# not measured counts UNMEASURED
NEAR, FAR_WEIGHT, REG_WEIGHT, BENCH_WEIGHT, UNMEASURED = 1.3, 0.2, 0.1, 5.0, 1.3
BENCH = {(256, 256, 1024), (8192, 8192, 8192), (2048, 6144, 16128), (2048, 1024, 105728),
         (2048, 5120, 105728)}
PLAN_MIN_GAIN = 0.01


def _features(tile, M, N, Kp, S, repack):
    MT, NT = tile[0], tile[1]
    wg = -(-M // MT) * -(-N // NT) * S
    occ = 2 if (MT, NT) in ((128, 128), (32, 128)) else 1
    cap = CUS * occ
    active = min(wg, cap)
    return dict(waves=(wg + cap - 1) // cap, active=active, per_cu=max(1, -(-active // CUS)),
                mfmas=MT // 32 * (NT // 32) // 4, slabs=(Kp // 64) / S, wide=tuple(tile) in WIDE,
                repack=bool(repack), akb=MT * 48.0 / 1024.0, bkb=NT // 32 * 1536.0 / 1024.0,
                out_kb=MT * NT * (4.0 if S > 1 else 2.0) / 1024.0, split=S > 1,
                rep_bytes=2.0 * (-(-M // 32) * 32) * (Kp // 4 * 3.0),
                long_rows=math.log2(max(1.0, Kp / 8192.0)),
                split_bytes=4.0 * S * M * N + 2.0 * M * N)


def _time(c, f, xp=None):
    """plan.cpp plan_time_us over one plan's features (scalars) or arrays of them (xp = numpy)."""
    where = (lambda q, a, b: a if q else b) if xp is None else xp.where
    mx = max if xp is None else xp.maximum
    a_cost = where(f["repack"], 1.0, 1.0 + where(f["wide"], c["A_ROWS_COST_WIDE"], c["A_ROWS_COST"]) +
                   c["A_ROWS_LONG"] * f["long_rows"])
    a_kb = f["akb"] * a_cost
    work = c["T_COPY_KB"] * a_kb + where(f["wide"], c["T_BREG_KB"], c["T_COPY_KB"]) * f["bkb"]
    t_slab = mx(mx(c["T_SLAB_MIN"], f["per_cu"] * (c["T_MFMA"] * f["mfmas"] + work)),
                f["active"] * c["T_L2_KB"] * (a_kb + f["bkb"]))
    t_wg = c["T_WG"] + f["slabs"] * t_slab + c["T_OUT_KB"] * f["out_kb"] * f["per_cu"]
    t = c["T_LAUNCH"] + f["waves"] * t_wg
    t = t + where(f["repack"], c["T_LAUNCH"] + f["rep_bytes"] / c["REPACK_BYTES_PER_US"], 0.0)
    t = t + where(f["split"], c["T_LAUNCH"] + f["split_bytes"] / c["SPLIT_BYTES_PER_US"], 0.0)
    return t


def plan_time_us(c, tile, M, N, Kp, S, repack):
    return _time(c, _features(tile, M, N, Kp, S, repack))


def candidates(M, N, Kp):
    """The plans best_plan visits, in its order. Regular shapes (M % 32 == 0, N % 128 == 0) take
    the tiles whose MT divides M, the 32- and 64-row ones included (the last tile column masked
    when NT does not divide N, visited after every dividing plan); ragged ones any tile, masked.
    On every shape the scale grouping divides each dimension that is a whole number of
    32-blocks."""
    kt = Kp // K_TILE
    regular = M % 32 == 0 and N % 128 == 0
    cands = (SKINNY if M % 128 else TILES + SKINNY) if regular else TILES + SKINNY
    out = []
    for masked in ((False, True) if regular else (None,)):
        for rp in (False, True):
            for S in SPLIT_CHOICES:
                if S > kt:
                    continue
                for tile in cands:
                    if regular and (M % tile[0] or bool(N % tile[1]) != masked):
                        continue
                    # the header's tile_scale holds whole scale groups only: on a dimension
                    # of whole 32-blocks the grouping must divide dim / 32
                    if (M % 32 == 0 and (M // 32) % tile[2]) or \
                            (N % 32 == 0 and (N // 32) % tile[3]):
                        continue
                    out.append((tile, S, rp))
    return out


def _pick(times):
    """Index of the router's pick: visiting in order, a plan replaces the current one only with a
    PLAN_MIN_GAIN lead."""
    bi = 0
    while True:
        later = [i for i in range(bi + 1, len(times)) if times[i] < times[bi] * (1.0 - PLAN_MIN_GAIN)]
        if not later:
            return bi
        bi = later[0]


def tiny_routed(M, N, Kp):
    kt = Kp // K_TILE
    blocks = -(-M // 32) * -(-N // 32)
    if blocks > 2 * CUS or kt < 2:
        return False
    if blocks > CUS:
        return kt <= 28
    return kt <= 32 or (kt <= 64 and 4 * blocks >= CUS)


def tiny_segments(M, N, Kp):
    kt = Kp // K_TILE
    if kt > 16:
        return max(8, -(-kt // 4))
    return 8 if kt > 12 and -(-M // 32) * -(-N // 32) <= CUS else -(-kt // 4)


def best_plan(c, M, N, Kp):
    """(tile, S, repack) with the least predicted time, as plan.cpp best_plan (the 32 x 32 tile's
    rule first)."""
    if tiny_routed(M, N, Kp):
        return (TINY, tiny_segments(M, N, Kp), False)
    cands = candidates(M, N, Kp)
    if not cands:
        return ((128, 128, 2, 2), 1, False)
    return cands[_pick([plan_time_us(c, t, M, N, Kp, S, rp) for t, S, rp in cands])]


def load(paths):
    recs = []
    for p in paths:
        with open(p) as f:
            recs += [json.loads(line) for line in f if line.strip()]
    return recs


def fit(recs, start, restarts=12, seed=0):
    """Pick-aware fit (see the weights above) by Nelder-Mead from a least-squares start, with
    perturbed restarts; returns (constants, objective)."""
    import numpy as np
    from scipy.optimize import minimize

    names = [n for n in NAMES if n not in FIXED]
    feats, segs = [], []
    for r in recs:
        M, N, K = r["shape"]
        Kp = (K + K_TILE - 1) // K_TILE * K_TILE
        meas = {(tuple(p[1]), p[2], p[3]): p[0] for p in r["plans"]}
        best = r["plans"][0][0]
        st = len(feats)
        for tile, S, rp in candidates(M, N, Kp):
            f = _features(tile, M, N, Kp, S, rp)
            f["meas"] = meas.get((tuple(tile), S, int(rp)), float("nan"))
            feats.append(f)
        segs.append((st, len(feats), best, BENCH_WEIGHT if tuple(r["shape"]) in BENCH else 1.0))
    F = {k: np.array([f[k] for f in feats], dtype=float) for k in feats[0]}
    for k in ("wide", "repack", "split"):
        F[k] = F[k] > 0
    has = ~np.isnan(F["meas"])
    logm = np.log(np.where(has, F["meas"], 1.0))
    regw = np.zeros(len(feats))
    for st, en, best, w in segs:
        regw[st:en] = np.where(F["meas"][st:en] < NEAR * best, 1.0, FAR_WEIGHT) * w
    regw = regw * has

    def consts(x):
        c = dict(zip(names, np.abs(x)))
        c.update(FIXED)
        return c

    def reg_loss(x):
        d = np.log(np.maximum(_time(consts(x), F, np), 1e-9)) - logm
        return float(np.sum(regw * d * d))

    def total(x):
        t = _time(consts(x), F, np)
        s = 0.0
        for st, en, best, w in segs:
            tt = t[st:en]
            bi = 0
            while True:
                later = np.nonzero(tt[bi + 1:] < tt[bi] * (1.0 - PLAN_MIN_GAIN))[0]
                if len(later) == 0:
                    break
                bi += 1 + int(later[0])
            m = F["meas"][st + bi]
            s += w * math.log(m / best if m == m else UNMEASURED)
        d = np.log(np.maximum(t, 1e-9)) - logm
        return s + REG_WEIGHT * float(np.sum(regw * d * d))

    x = np.array([start[n] for n in names])
    x = minimize(reg_loss, x, method="Nelder-Mead",
                 options={"maxiter": 20000, "xatol": 1e-8, "fatol": 1e-10}).x
    best_x, best_f = x, total(x)
    rng = np.random.default_rng(seed)
    for k in range(restarts):
        x0 = best_x * (1 + 0.1 * rng.standard_normal(len(best_x))) if k else best_x
        r = minimize(total, x0, method="Nelder-Mead",
                     options={"maxiter": 6000, "xatol": 1e-9, "fatol": 1e-12})
        if r.fun < best_f:
            best_x, best_f = r.x, r.fun
    return consts(best_x), float(best_f)


def evaluate(c, recs):
    """Measured time of the model's pick / measured best, per shape (nan: the pick was not
    measured)."""
    out = []
    for r in recs:
        M, N, K = r["shape"]
        Kp = (K + K_TILE - 1) // K_TILE * K_TILE
        tile, S, rp = best_plan(c, M, N, Kp)
        meas = [p[0] for p in r["plans"] if tuple(p[1]) == tile and p[2] == S and p[3] == int(rp)]
        out.append((tuple(r["shape"]), meas[0] / r["plans"][0][0] if meas else float("nan")))
    return out


def main():
    paths = sys.argv[1:] or [os.path.join(HERE, "plans_mi355x.jsonl")]
    recs = load([p for p in paths if p != "--no-fit"] or [os.path.join(HERE, "plans_mi355x.jsonl")])
    # the constants are fitted on the shapes with M % 128 == 0 (every tile measured on them) that
    # the model routes (not those of the 32 x 32 tile's rule)
    def modelled(r):
        M, N, K = r["shape"]
        return M % 128 == 0 and not tiny_routed(M, N, (K + K_TILE - 1) // K_TILE * K_TILE)
    fit_recs = [r for r in recs if modelled(r)]
    if "--no-fit" in sys.argv:
        c = CONSTANTS
    else:
        c, l = fit(fit_recs, CONSTANTS)
        print("fitted constants (objective %.3f over %d shapes):" % (l, len(fit_recs)))
        for n in NAMES:
            print(f"  {n:20s} {c[n]:.6g}")
    for label, sel in (("M % 128 == 0", lambda s: s[0] % 128 == 0),
                       ("skinny M or ragged", lambda s: s[0] % 128 != 0)):
        ev = [(s, g) for s, g in evaluate(c, recs) if sel(s)]
        meas = [g for _, g in ev if g == g]
        if meas:
            gm = math.exp(sum(math.log(g) for g in meas) / len(meas))
            print(f"{label}: {len(ev)} shapes, picks measured for {len(meas)}: geomean "
                  f"{gm:.3f}x of the best, worst {max(meas):.3f}x")
    for s, g in evaluate(c, recs):
        if s in BENCH:
            print(f"  benchmark {s}: pick {best_plan(c, s[0], s[1], (s[2] + K_TILE - 1) // K_TILE * K_TILE)}"
                  f" at {g:.3f}x of the best")


if __name__ == "__main__":
    main()
