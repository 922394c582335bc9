// Host plan of libmxfp6gemm: shape router, split-K planner, argument checks and the public entry
// points (C++ API of include/mxfp6/gemm.hpp and the GEMM part of the C ABI in
// include/mxfp6_gemm.h). Plain C++17 with no HIP header: every device action goes through the
// thin launch layer declared in hip_layer.h.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <mutex>
#include <vector>

#include "../hip_layer.h"
#include "mxfp6/gemm.hpp"
#include "mxfp6_gemm.h"
#include "plan.hpp"

namespace mxfp6 {
namespace plan {

// ---- router ------------------------------------------------------------------------------
//
// Candidate tiles (4 waves per workgroup):
//   256x256, waves 2x2, each wave 128x128 -> MPW 4, NPW 4   (16 MFMAs per wave per 64-wide slab)
//   256x192, waves 2x2, each wave 128x96  -> MPW 4, NPW 3   (12; built, not routed: kCands)
//   128x256, waves 2x2, each wave  64x128 -> MPW 2, NPW 4   (8)
//   128x128, waves 2x2, each wave  64x64  -> MPW 2, NPW 2   (4; two workgroups fit a CU's LDS)
// the wide tiles (waves 1x4, B straight into registers, A staged in LDS one K-tile at a time):
//   128x512, each wave 128x128            -> MPW 4, NPW 4   (16)
//   128x384, each wave 128x96             -> MPW 4, NPW 3   (12)
//   128x256, each wave 128x64             -> MPW 4, NPW 2   (8)
//   256x256, each wave 256x64             -> MPW 4, NPW 2   (16; A scales in two groups of 4)
// and the skinny tiles (waves 1x4), the only ones for M not a multiple of 128 (M a multiple of
// 32), and on small grids faster than the big ones for any M (C1, 256x256x1024: 32x128 6.2 us
// against 7.2 us on 128x128 and 8.2 us on the 128x256 wide tile):
//   64x256 (MPW 2, NPW 2), 32x256 (1, 2), 64x128 (2, 1), 32x128 (1, 1; two per CU)
// Ragged shapes (M not a multiple of 32 or N not a multiple of 128) take any of the eleven tiles,
// the last tile row and column masked (wg counts the partial tiles).
// A plan is (tile, K segments S from SPLIT_CHOICES, A repacked or not); the router takes the plan
// with the least predicted time. The time model (microseconds, MI355X) follows the kernel's
// structure:
//   wg       = ceil(M / MT) * ceil(N / NT) workgroups per K segment;
//   waves    = ceil(wg * S / (CUS * occupancy)) rounds of workgroups;
//   active   = min(wg * S, CUS * occupancy) workgroups in flight;
//   per_cu   = ceil(active / CUS) workgroups on the busiest CU;
//              (CUS: the current device's compute units, 256 on an MI355X)
//   kb       = KiB a workgroup moves per 64-wide K slab: A (MT * 48 bytes, times 1 + A_ROWS_COST
//              when read row-major: a copy touches ~3 cache lines per 128 bytes instead of 1,
//              plus A_ROWS_LONG per doubling of Kp past 8192: rows further apart cost more) and
//              B (NT / 32 * 1536 bytes);
//   t_slab   = max(T_SLAB_MIN, per_cu * (T_MFMA * mfmas + T_COPY_KB * kb),
//                  active * T_L2_KB * kb) per slab: a latency floor (the ring keeps several slabs
//              in flight), the CU's MFMA and global->LDS copy work shared by the workgroups
//              resident on it, and the chip's L2 -> CU delivery shared by every workgroup in
//              flight; the wide tiles load B into registers (T_BREG_KB per KiB) and copy A at
//              their own row-major cost (A_ROWS_COST_WIDE: a K-tile row is 144 contiguous bytes);
//   t_wg     = T_WG + slabs * t_slab + T_OUT_KB * output KiB * per_cu;
//   t        = T_LAUNCH + waves * t_wg, plus for a repack T_LAUNCH + its bytes (A read and written)
//              at REPACK_BYTES_PER_US, and for a split T_LAUNCH + the partials written and read
//              back at SPLIT_BYTES_PER_US.
// The constants are fitted to every plan of the 82 measured shapes (one MI355X; M from 32 to
// 8192, N from 77 to 102272, K from 1024 to 105728, ragged and skinny shapes included), choosing
// the plan, not predicting every time: the fit minimises the summed log of (measured time of the
// model's pick / measured best) over the shapes with M % 128 == 0, the five benchmark workloads
// weighing 5x, plus 0.1x the log-time least squares of the plans within 1.3x of their shape's
// best (0.2x weight for the others); the repack rate is the repack kernel's measured one. The
// pick is then within 1.8% of the measured best on average over the 66 shapes with M % 128 == 0,
// 19% at worst (2048x8192x1024, a short-K shape whose plans trade places between machines), and
// the best on four of the five benchmark workloads (2048x6144x16128: 6% behind the 128x384
// tile on the sweep's machine); on the 16 skinny-M and ragged shapes within 2.3% on average,
// 10% at worst.
size_t split_bytes(int M, int N, int S);
size_t plan_bytes(int M, int N, int Kp, int S, bool repack);

// Whether a workspace of ws_bytes holds a plan's buffers: the split-K partials (exactly
// gemm_workspace_size's bytes for the routed split), or the partials rounded to 256 bytes and the
// repacked A after them.
bool plan_fits(int M, int N, int Kp, int S, bool repack, size_t ws_bytes) {
    return ws_bytes >= (repack ? plan_bytes(M, N, Kp, S, true) : split_bytes(M, N, S));
}

namespace {
struct Plan {
    TileChoice tc;
    int S;
    bool repack;
};
// 256x192 (slab kernel) is implemented but not routed: the best measured plan on 1 of 194 swept
// shapes (by 3.5%), while the model picked it, repacked, on shapes where 128x384 on row-major A
// is 4-10% faster (2048x12288x4096, 3072x6144x8192, 6144x6144x8192, 2048x9216x16384)
const TileChoice kCands[] = {{256, 256, 4, 4}, {128, 384, 4, 3}, {128, 256, 2, 4},
                             {128, 128, 2, 2}, {128, 512, 4, 4}, {128, 256, 4, 2},
                             {256, 256, 4, 2}};
const TileChoice kSkinny[] = {{64, 256, 2, 2}, {32, 256, 1, 2}, {64, 128, 2, 1}, {32, 128, 1, 1}};

// The tiles of the wide kernel (B loaded into registers, A staged per K-tile).
bool is_wide(const TileChoice& tc) {
    return (tc.MT == 128 && tc.NT == 512 && tc.MPW == 4 && tc.NPW == 4) ||
           (tc.MT == 128 && tc.NT == 384 && tc.MPW == 4 && tc.NPW == 3) ||
           (tc.MT == 128 && tc.NT == 256 && tc.MPW == 4 && tc.NPW == 2) ||
           (tc.MT == 256 && tc.NT == 256 && tc.MPW == 4 && tc.NPW == 2);
}

double plan_time_us(const TileChoice& tc, int M, int N, int Kp, int S, bool repack, int CUS) {
    const long wg = (long)((M + tc.MT - 1) / tc.MT) * ((N + tc.NT - 1) / tc.NT) * S;
    const int occ = (tc.NT == 128 && (tc.MT == 128 || tc.MT == 32)) ? 2 : 1;  // per CU (LDS)
    const long cap = (long)CUS * occ;
    const long waves = (wg + cap - 1) / cap;
    const long active = std::min(wg, cap);
    const long per_cu = std::max(1L, (active + CUS - 1) / CUS);  // on the busiest CU
    const int mfmas = tc.MT / 32 * (tc.NT / 32) / 4;  // per wave per slab (4 waves)
    const double slabs = (double)(Kp / 64) / S;
    const bool wide = is_wide(tc);
    const double long_rows = std::log2(std::max(1.0, Kp / 8192.0));
    const double a_cost =
        repack ? 1.0 : 1.0 + (wide ? A_ROWS_COST_WIDE : A_ROWS_COST) + A_ROWS_LONG * long_rows;
    const double a_kb = tc.MT * 48.0 * a_cost / 1024.0, b_kb = tc.NT / 32 * 1536.0 / 1024.0;
    const double work = T_COPY_KB * a_kb + (wide ? T_BREG_KB : T_COPY_KB) * b_kb;
    const double t_slab = std::max({T_SLAB_MIN, (double)per_cu * (T_MFMA * mfmas + work),
                                    (double)active * T_L2_KB * (a_kb + b_kb)});
    const double out_kb = tc.MT * tc.NT * (S > 1 ? 4.0 : 2.0) / 1024.0;
    const double t_wg = T_WG + slabs * t_slab + T_OUT_KB * out_kb * per_cu;
    double t = T_LAUNCH + (double)waves * t_wg;
    if (repack) t += T_LAUNCH + 2.0 * ((M + 31) / 32 * 32) * (Kp / 4 * 3.0) / REPACK_BYTES_PER_US;
    if (S > 1) t += T_LAUNCH + (4.0 * S * M * N + 2.0 * M * N) / SPLIT_BYTES_PER_US;
    return t;
}

bool shape_ok(int M, int N, int Kp) {
    return M > 0 && N > 0 && Kp > 0 && Kp % K_TILE == 0;
}

// M x N tiled by whole 32-row and 128-column blocks (the reference's shapes and the skinny-M
// ones); other shapes are ragged and run masked tiles.
bool regular(int M, int N) {
    return M % 32 == 0 && N % 128 == 0;
}

const int kNCands = (int)(sizeof(kCands) / sizeof(kCands[0]));
const int kNSkinny = (int)(sizeof(kSkinny) / sizeof(kSkinny[0]));

// The least-time plan. Candidates are visited from the simplest (no split, no repack) and a
// plan needs a PLAN_MIN_GAIN lead to displace an earlier one, so near-ties keep the plan with
// fewer launches and less workspace. Regular shapes take the tiles whose MT divides M, with the
// last tile column masked when NT does not divide N (the reference's NMASK route,
// src/kernel.hpp:144-154, for any tile: N = 102272 runs 256x256 over ceil(N/256) columns instead
// of 128x128); ragged shapes any of the ten, big tiles first. Shapes gemm() rejects get the
// trivial plan.
// Calls f(tile, S, repack) for every plan the router considers for (M, N, Kp), in its visiting
// order: big tiles first, then the skinny ones; on regular shapes only the tiles whose MT divides
// M (so M % 128 != 0 leaves the skinny ones), the dividing tiles first, then (pass 1) the
// N-masked ones.
template <typename F>
void visit_plans(int M, int N, int Kp, F&& f) {
    const int k_tiles = Kp / K_TILE;
    const bool reg = regular(M, N);
    for (int pass = 0; pass < (reg ? 2 : 1); pass++)
        for (int rp = 0; rp < 2; rp++)
            for (const int S : SPLIT_CHOICES)
                for (int ci = 0; ci < kNCands + kNSkinny && S <= k_tiles; ci++) {
                    const TileChoice& tc = ci < kNCands ? kCands[ci] : kSkinny[ci - kNCands];
                    if (reg && (M % tc.MT != 0 || (N % tc.NT != 0) != (pass == 1))) continue;
                    // a dimension that is a whole number of 32-blocks may have its scales tiled
                    // by the header's tile_scale, which holds floor(dim / (32 * group)) whole
                    // groups, while a masked tile reads up to group ceil(dim / (32 * group)) - 1:
                    // the grouping must divide dim / 32 (N = 4000, 125 blocks, excludes NPW 2
                    // and 4; an N-masked 128x384, NPW 3, needs (N / 32) % 3 == 0). Ragged
                    // dimensions cannot go through the header and take the C ABI's ceil layout.
                    if ((M % 32 == 0 && (M / 32) % tc.MPW != 0) ||
                        (N % 32 == 0 && (N / 32) % tc.NPW != 0))
                        continue;
                    f(tc, S, rp != 0);
                }
}

// The 32 x 32 tile (tiny_kernel.hpp): K split over a workgroup's waves, the segments summed and
// stored by all of them. Routed by a measured rule ahead of the model, which has no term for it:
// grids that fit the chip in one round (two four-wave workgroups per CU) with 2 to 28 K-tiles,
// and on grids of one workgroup per CU (eight waves, A staged) up to 32 K-tiles, up to 64 on
// those of at least a quarter as many blocks as CUs; up to 16 K-tiles in the fewest segments of
// at most four K-tiles (one a wave), except 13-16 K-tiles on one workgroup per CU in 8 (eight
// waves, A staged), and past 16 in max(8, ceil(K-tiles / 4)) (A staged through LDS, two
// segments a wave at most). Against the routed pipelined plans, same sessions: 2-16
// K-tiles, 26 shapes: 3-36% faster (256 x 256 x 1024 6.09 -> 3.88 us, 256 x 256 x 3072 8.22 ->
// 6.30, 1024 x 512 x 1024 6.34 -> 5.42); slower with one K-tile (3.69 -> 3.77) and on grids of
// three blocks per CU, which take a second round (1536 x 512 x 1024 6.41 -> 7.29). 17-28 K-tiles
// (8 segments): 512 x 512 x 4096 11.09 -> 5.34, 1024 x 512 x 4096 13.65 -> 8.59, 96 x 4096 x 4096
// 12.55 -> 10.92. 29-32 on one workgroup per CU: 256 x 256 x 6144 8.77 -> 5.84, 128 x 128 x 6144
// 7.07 -> 5.71, 512 x 512 x 5568 11.54 -> 6.11; on two, mixed (1024 x 512 x 6144 15.16 -> 10.28,
// 128 x 4096 x 6144 15.06 -> 16.77). 33-64 on 64-256 blocks: 512 x 512 x 8192 13.49 -> 8.05, 64 x
// 2048 x 8192 10.70 -> 7.83, 32 x 8192 x 12288 19.16 -> 16.56, 256 x 256 x 12288 10.00 -> 9.61;
// on 16 blocks slower (128 x 128 x 12288 8.36 -> 9.36). The fewest segments measured best or
// within 3% up to 12 K-tiles (256 x 256 x 1024 3.88, 3.99 and 4.09 us in 2, 3 and 4; 6 and 8
// segments 1-7% slower on 8-12 K-tiles but for one 16-block grid); 8 beat 4 at 13-16 K-tiles on
// all nine grids of 4-256 blocks measured (64 x 64 x 3072 5.95 -> 4.42 us, 256 x 256 x 3072 4.92 ->
// 4.76); 8 beat 6 on all six 22-K-tile shapes, 11 beat 16 at 43 K-tiles on four of four.
// The 32 x 32 tile splits K over its waves: at most 16 segments of at most 4 K-tiles, on
// row-major A (tiny_kernel.hpp).
bool tiny_plan_ok(const TileChoice& tc, int Kp, int S, int a_layout) {
    if (tc.MT != 32 || tc.NT != 32) return true;
    const int kt = Kp / K_TILE;
    return a_layout == MXFP6_A_ROWS && S >= 1 && S <= 16 && (kt + S - 1) / S <= 4;
}

const TileChoice kTiny = {32, 32, 1, 1};

bool is_tiny(const TileChoice& tc) {
    return tc.MT == kTiny.MT && tc.NT == kTiny.NT && tc.MPW == kTiny.MPW && tc.NPW == kTiny.NPW;
}

bool tiny_routed(int M, int N, int Kp, int cus) {
    const long blocks = (long)((M + 31) / 32) * ((N + 31) / 32);
    const int kt = Kp / K_TILE;
    if (blocks > 2L * cus || kt < 2) return false;
    if (blocks > cus) return kt <= 28;
    return kt <= 32 || (kt <= 64 && 4 * blocks >= cus);
}

int tiny_segments(int M, int N, int Kp, int cus) {
    const long blocks = (long)((M + 31) / 32) * ((N + 31) / 32);
    const int kt = Kp / K_TILE;
    if (kt > 16) return std::max(8, (kt + 3) / 4);
    return kt > 12 && blocks <= cus ? 8 : (kt + 3) / 4;
}

Plan best_plan(int M, int N, int Kp, int cus) {
    Plan best = {{128, 128, 2, 2}, 1, false};
    if (!shape_ok(M, N, Kp)) return best;
    if (tiny_routed(M, N, Kp, cus)) return {kTiny, tiny_segments(M, N, Kp, cus), false};
    double best_t = -1.0;
    visit_plans(M, N, Kp, [&](const TileChoice& tc, int S, bool rp) {
        const double t = plan_time_us(tc, M, N, Kp, S, rp, cus);
        if (best_t < 0 || t < best_t * (1.0 - PLAN_MIN_GAIN)) {
            best = {tc, S, rp};
            best_t = t;
        }
    });
    return best;
}

// The least-time row-major plan with the scale grouping of `grouping` and S K segments: what
// gemm() runs when the caller's workspace does not hold the routed plan (S = the routed split
// with gemm_workspace_size's workspace, 1 with none). For a given S every tile of a grouping gives
// the same output bits (each K segment's MFMAs in the same K order, the same reduction).
Plan best_fitting_plan(int M, int N, int Kp, int cus, const TileChoice& grouping, int S_fixed) {
    // the 32 x 32 tile itself where it can run the split (its plans never repack)
    if (is_tiny(grouping) && tiny_plan_ok(grouping, Kp, S_fixed, MXFP6_A_ROWS))
        return {grouping, S_fixed, false};
    Plan best = {grouping, S_fixed, false};
    double best_t = -1.0;
    visit_plans(M, N, Kp, [&](const TileChoice& tc, int S, bool rp) {
        if (tc.MPW != grouping.MPW || tc.NPW != grouping.NPW || S != S_fixed || rp) return;
        const double t = plan_time_us(tc, M, N, Kp, S, rp, cus);
        if (best_t < 0 || t < best_t * (1.0 - PLAN_MIN_GAIN)) {
            best = {tc, S, rp};
            best_t = t;
        }
    });
    return best;
}

// best_plan evaluates the model for every (tile, split, layout): a few microseconds of host time,
// as long as a small GEMM runs on the GPU. gemm() and the routing queries look the plan up in a
// per-thread cache of the last shapes instead (16 entries indexed by a hash of the shape; no
// lock, and the plan of a shape on a device never changes). The key includes the compute-unit
// count of the current device, which the HIP layer reads once per device.
// The cached entry of a shape: the routed plan, and the plans gemm() falls back to with
// gemm_workspace_size's workspace (ref_ws) and with none (no_ws).
struct Routed {
    Plan plan, ref_ws, no_ws;
};

const Routed& cached_routes(int M, int N, int Kp) {
    struct Entry {
        int M, N, Kp, cus;
        Routed r;
        bool valid;
    };
    thread_local Entry cache[16] = {};
    const int reported = mxfp6_hip_device_cus();
    const int cus = reported > 0 ? reported : DEFAULT_CUS;
    const unsigned h = ((unsigned)M * 73856093u ^ (unsigned)N * 19349663u ^ (unsigned)Kp * 83492791u) >> 4;
    Entry& e = cache[h % 16];
    if (!e.valid || e.M != M || e.N != N || e.Kp != Kp || e.cus != cus) {
        const Plan pl = best_plan(M, N, Kp, cus);
        const Plan none = best_fitting_plan(M, N, Kp, cus, pl.tc, 1);
        const Plan ref = pl.S > 1 ? best_fitting_plan(M, N, Kp, cus, pl.tc, pl.S) : none;
        e = {M, N, Kp, cus, {pl, ref, none}, true};
    }
    return e.r;
}

Plan cached_plan(int M, int N, int Kp) {
    return cached_routes(M, N, Kp).plan;
}

// ---- measured plans (mxfp6_gemm_tune) ----------------------------------------------------------
// tune() times the router's best-predicted plans of a shape on the caller's operands and keeps the
// fastest for the process; gemm() then runs it whenever the call's workspace holds it. The table
// is shared by all threads (a mutex, skipped while it is empty).
struct Tuned {
    int out_type, M, N, Kp;
    Plan plan;
};
std::mutex g_tuned_mu;
std::vector<Tuned> g_tuned;
std::atomic<int> g_n_tuned{0};

bool find_tuned(int out_type, int M, int N, int Kp, Plan* out) {
    if (g_n_tuned.load(std::memory_order_acquire) == 0) return false;
    std::lock_guard<std::mutex> lk(g_tuned_mu);
    for (const Tuned& t : g_tuned)
        if (t.out_type == out_type && t.M == M && t.N == N && t.Kp == Kp) {
            *out = t.plan;
            return true;
        }
    return false;
}

void store_tuned(int out_type, int M, int N, int Kp, const Plan& p) {
    std::lock_guard<std::mutex> lk(g_tuned_mu);
    for (Tuned& t : g_tuned)
        if (t.out_type == out_type && t.M == M && t.N == N && t.Kp == Kp) {
            t.plan = p;
            return;
        }
    g_tuned.push_back({out_type, M, N, Kp, p});
    g_n_tuned.store((int)g_tuned.size(), std::memory_order_release);
}
}  // namespace

TileChoice route(int M, int N, int Kp) {
    return cached_plan(M, N, Kp).tc;
}

size_t split_bytes(int M, int N, int S) {
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
}

// The repacked A: ceil(M / 32) whole 32-row blocks.
size_t repack_bytes(int M, int Kp) {
    return (size_t)((M + 31) / 32 * 32) * (size_t)(Kp / 4 * 3);
}

size_t plan_bytes(int M, int N, int Kp, int S, bool repack) {
    const size_t sb = (split_bytes(M, N, S) + 255) / 256 * 256;
    return sb + (repack ? repack_bytes(M, Kp) : 0);
}

bool route_repacks(int M, int N, int Kp) {
    return shape_ok(M, N, Kp) && cached_plan(M, N, Kp).repack;
}

int splitk_segments(int M, int N, int Kp) {
    return shape_ok(M, N, Kp) ? cached_plan(M, N, Kp).S : 1;
}

// gemm_workspace_size: the split-K partials of the routed plan, 0 when it is not split (the
// reference's meaning, src/dispatch.hpp:55-59). With exactly that workspace gemm() runs the plan
// on row-major A.
size_t workspace_bytes(int M, int N, int Kp) {
    return split_bytes(M, N, splitk_segments(M, N, Kp));
}

// The workspace of the routed plan in full: the split-K partials, then (at the next 256-byte
// boundary) the repacked A when the plan repacks. gemm() given at least this much runs the plan
// with the repack; the output is the same bits either way.
size_t preferred_workspace_bytes(int M, int N, int Kp) {
    const int S = splitk_segments(M, N, Kp);
    const bool rp = route_repacks(M, N, Kp);
    return (S > 1 || rp) ? plan_bytes(M, N, Kp, S, rp) : 0;
}

// ---- argument checks -----------------------------------------------------------------------

int check_common(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
                 const void* dsA, const void* dsB, const void* dD, int A_row_bytes) {
    if (out_type < 0 || out_type > 2) return MXFP6_ERR_OUT_TYPE;
    if (!dA || !dBsh || !dsA || !dsB || !dD) return MXFP6_ERR_NULL;
    if (M <= 0 || N <= 0 || Kp <= 0 || Kp % K_TILE != 0) return MXFP6_ERR_SHAPE;
    // A rows are read for packed(Kp) bytes from row * A_row_bytes; a compact row (packed(K),
    // K > Kp - K_TILE) is at most packed(K_TILE - 32) = 120 bytes shorter than packed(Kp).
    const long packed_kp = (long)Kp / 4 * 3;
    if (A_row_bytes <= 0 || A_row_bytes % 4 != 0 || A_row_bytes < packed_kp - 120)
        return MXFP6_ERR_SHAPE;
    return MXFP6_OK;
}

const char* status_text(int st) {
    switch (st) {
        case MXFP6_OK: return "ok";
        case MXFP6_ERR_NULL: return "null pointer argument";
        case MXFP6_ERR_SHAPE: return "unsupported shape (M, N > 0; Kp a multiple of 192; A_row_bytes)";
        case MXFP6_ERR_OUT_TYPE: return "out_type must be F32, F16 or BF16";
        case MXFP6_ERR_TILE: return "tile not implemented or does not divide the shape";
        case MXFP6_ERR_ARG: return "invalid argument";
        case MXFP6_ERR_HIP: return "HIP launch error";
        case MXFP6_ERR_SCRATCH: return "split-K partials exceed the no-allocation scratch";
        default: return "unknown status";
    }
}

// ---- launch ----------------------------------------------------------------------------------

bool streams_output(int out_type, int M, int N, int Kp, const TileChoice& tc, int S, bool repack,
                    int A_row_bytes) {
    // the split-K partials are read back and the reduce writes D; the other tiles' kernel keeps
    // plain stores
    if (S > 1 || !is_wide(tc)) return false;
    const double packed = Kp / 4 * 3.0;
    const double in = (double)M * A_row_bytes + (repack ? ((M + 31) / 32 * 32) * packed : 0.0) +
                      (double)N * packed + (double)(M + N) * (Kp / 32);
    const double out = (double)M * N * (out_type == 0 ? 4 : 2);  // FP32 or a 16-bit type
    return in <= LLC_BYTES && in + out > STREAM_FOOTPRINT_BYTES;
}

// ws: the workspace of the plan (S, a_layout): split partials first, then (MXFP6_A_REPACK) the
// repacked A at the next 256-byte boundary.
int run(int out_type, int M, int N, int Kp, const TileChoice& tc, int S, int a_layout, int kernel,
        const void* dA, const void* dBsh, const uint8_t* dsA, const uint8_t* dsB, void* dD,
        int A_row_bytes, void* ws, void* stream) {
    mxfp6_launch_desc d;
    d.kernel = kernel;
    d.out_type = out_type;
    d.M = M;
    d.N = N;
    d.Kp = Kp;
    d.MT = tc.MT;
    d.NT = tc.NT;
    d.mpw = tc.MPW;
    d.npw = tc.NPW;
    d.splits = S;
    d.A_row_bytes = A_row_bytes;
    d.A = dA;
    d.Bsh = dBsh;
    d.sA = dsA;
    d.sB = dsB;
    d.D = dD;
    d.ws = S > 1 ? static_cast<float*>(ws) : nullptr;
    d.a_layout = a_layout;
    d.Ash = a_layout == MXFP6_A_REPACK
                ? static_cast<uint8_t*>(ws) + (split_bytes(M, N, S) + 255) / 256 * 256
                : nullptr;
    d.out_stream = kernel == MXFP6_KERNEL_TILE && a_layout != MXFP6_A_ROWS_SWIZZLED &&
                           streams_output(out_type, M, N, Kp, tc, S, a_layout == MXFP6_A_REPACK,
                                          A_row_bytes)
                       ? 1
                       : 0;
    d.stream = stream;
    const int rc = mxfp6_hip_launch(&d);
    return rc == 0 ? MXFP6_OK : rc == 1 ? MXFP6_ERR_TILE : MXFP6_ERR_HIP;
}

int kernel_for(const TileChoice& tc) {
    return mxfp6_hip_has_tile(tc.MT, tc.NT, tc.MPW, tc.NPW) ? MXFP6_KERNEL_TILE
                                                            : MXFP6_KERNEL_DIRECT;
}

Plan plan_for(int out_type, int M, int N, int Kp, size_t ws_bytes, bool* unsplit);

int gemm_checked(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
                 const uint8_t* dsA, const uint8_t* dsB, void* dD, int A_row_bytes, void* ws,
                 size_t ws_bytes, void* stream) {
    const int st = check_common(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes);
    if (st != MXFP6_OK) return st;
    if (ws == nullptr) ws_bytes = 0;
    bool unsplit = false;
    const Plan pl = plan_for(out_type, M, N, Kp, ws_bytes, &unsplit);
    if (unsplit)
        std::fprintf(stderr,
                     "[mxfp6] %dx%dx%d: split-K over %d segments needs a %zu-byte workspace, "
                     "got %zu; running unsplit. Size it with gemm_workspace_size().\n",
                     M, N, Kp, splitk_segments(M, N, Kp), workspace_bytes(M, N, Kp), ws_bytes);
    const int kernel = kernel_for(pl.tc);
    const bool rp = pl.repack && kernel == MXFP6_KERNEL_TILE;
    if (kernel != MXFP6_KERNEL_TILE && (M % 64 != 0 || N % 64 != 0)) return MXFP6_ERR_TILE;
    return run(out_type, M, N, Kp, pl.tc, pl.S, rp ? MXFP6_A_REPACK : MXFP6_A_ROWS, kernel, dA,
               dBsh, dsA, dsB, dD, A_row_bytes, ws, stream);
}

// The plan gemm() runs for a workspace of ws_bytes: a measured plan of the shape when the
// workspace holds it; else the routed plan when the workspace holds it; else, on row-major A, the
// fastest predicted tile with the routed scale grouping for the routed split when ws_bytes holds
// its partials (gemm_workspace_size's workspace), or unsplit (*unsplit set when the routed plan
// was split: the reference's warning case). Falling back changes neither the scale layout the
// caller prepared nor the output bits of the routed plan when the split is kept.
Plan plan_for(int out_type, int M, int N, int Kp, size_t ws_bytes, bool* unsplit) {
    if (unsplit != nullptr) *unsplit = false;
    Plan tuned;
    if (find_tuned(out_type, M, N, Kp, &tuned) &&
        plan_fits(M, N, Kp, tuned.S, tuned.repack, ws_bytes))
        return tuned;
    const Routed& r = cached_routes(M, N, Kp);
    const Plan& pl = r.plan;
    if (plan_fits(M, N, Kp, pl.S, pl.repack, ws_bytes)) return pl;
    if (ws_bytes >= split_bytes(M, N, pl.S)) return r.ref_ws;
    if (unsplit != nullptr) *unsplit = pl.S > 1;
    return r.no_ws;
}

namespace {
struct TuneCall {
    int out_type, M, N, Kp, A_row_bytes;
    Plan plan;
    const void *dA, *dBsh;
    const uint8_t *dsA, *dsB;
    void *dD, *ws, *stream;
};

int tune_launch(void* ctx) {
    const TuneCall& c = *static_cast<const TuneCall*>(ctx);
    return run(c.out_type, c.M, c.N, c.Kp, c.plan.tc, c.plan.S,
               c.plan.repack ? MXFP6_A_REPACK : MXFP6_A_ROWS, kernel_for(c.plan.tc), c.dA, c.dBsh,
               c.dsA, c.dsB, c.dD, c.A_row_bytes, c.ws, c.stream);
}
}  // namespace

int tune(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh, const uint8_t* dsA,
         const uint8_t* dsB, void* dD, int A_row_bytes, void* ws, size_t ws_bytes,
         int candidates, void* stream, int tile_out[4], int* splits_out, int* repack_out) {
    const int st = check_common(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes);
    if (st != MXFP6_OK) return st;
    if (candidates < 1) return MXFP6_ERR_ARG;
    if (ws == nullptr) ws_bytes = 0;
    const Plan routed = cached_plan(M, N, Kp);
    if (kernel_for(routed.tc) != MXFP6_KERNEL_TILE) return MXFP6_ERR_TILE;
    const int reported = mxfp6_hip_device_cus();
    const int cus = reported > 0 ? reported : DEFAULT_CUS;
    // the candidates: the plans with the routed tile's scale grouping (the caller's scales are
    // tiled for it) whose workspace fits, by predicted time
    struct Ranked {
        double t;
        Plan plan;
    };
    std::vector<Ranked> ranked;
    // the routed plan is always measured (the 32 x 32 tile is not among the model's plans), and
    // for the 32 x 32 tile the nearest valid segment counts below and above the routed one next
    // (their times are within a few percent of each other, in an order that varies by box)
    if (plan_fits(M, N, Kp, routed.S, routed.repack, ws_bytes)) ranked.push_back({-1.0, routed});
    if (is_tiny(routed.tc)) {
        for (int dir = -1; dir <= 1; dir += 2)
            for (int S = routed.S + dir; S >= 1 && S <= 16; S += dir)
                if (tiny_plan_ok(routed.tc, Kp, S, MXFP6_A_ROWS)) {
                    if (plan_fits(M, N, Kp, S, false, ws_bytes))
                        ranked.push_back({-0.5, {routed.tc, S, false}});
                    break;
                }
    }
    visit_plans(M, N, Kp, [&](const TileChoice& tc, int S, bool rp) {
        if (tc.MT == routed.tc.MT && tc.NT == routed.tc.NT && S == routed.S && rp == routed.repack)
            return;
        if (tc.MPW != routed.tc.MPW || tc.NPW != routed.tc.NPW) return;
        if (kernel_for(tc) != MXFP6_KERNEL_TILE) return;
        if (!plan_fits(M, N, Kp, S, rp, ws_bytes)) return;
        ranked.push_back({plan_time_us(tc, M, N, Kp, S, rp, cus), {tc, S, rp}});
    });
    std::stable_sort(ranked.begin(), ranked.end(),
                     [](const Ranked& a, const Ranked& b) { return a.t < b.t; });
    if (ranked.size() > (size_t)candidates) ranked.resize((size_t)candidates);
    if (ranked.empty()) return MXFP6_ERR_ARG;
    Plan best = ranked[0].plan;
    float best_ms = -1.0f;
    for (const Ranked& r : ranked) {
        TuneCall c = {out_type, M, N, Kp, A_row_bytes, r.plan, dA, dBsh, dsA, dsB, dD, ws, stream};
        // about 2 ms of launches per candidate, at least 3
        const int reps = std::max(3, std::min(50, (int)(2000.0 / std::max(1.0, r.t))));
        float ms = 0.0f;
        const int rc = mxfp6_hip_time(tune_launch, &c, stream, 2, reps, &ms);
        if (rc != 0) return rc == 2 ? MXFP6_ERR_HIP : rc;
        if (best_ms < 0 || ms < best_ms) {
            best_ms = ms;
            best = r.plan;
        }
    }
    store_tuned(out_type, M, N, Kp, best);
    if (tile_out) {
        tile_out[0] = best.tc.MT;
        tile_out[1] = best.tc.NT;
        tile_out[2] = best.tc.MPW;
        tile_out[3] = best.tc.NPW;
    }
    if (splits_out) *splits_out = best.S;
    if (repack_out) *repack_out = best.repack ? 1 : 0;
    return MXFP6_OK;
}

int tuned(int out_type, int M, int N, int Kp, int tile_out[4], int* splits_out, int* repack_out) {
    Plan p;
    if (!find_tuned(out_type, M, N, Kp, &p)) return 0;
    if (tile_out) {
        tile_out[0] = p.tc.MT;
        tile_out[1] = p.tc.NT;
        tile_out[2] = p.tc.MPW;
        tile_out[3] = p.tc.NPW;
    }
    if (splits_out) *splits_out = p.S;
    if (repack_out) *repack_out = p.repack ? 1 : 0;
    return 1;
}

int plan_info(int out_type, int M, int N, int Kp, size_t ws_bytes, int tile_out[4],
              int* splits_out, int* repack_out) {
    const Plan pl = plan_for(out_type, M, N, Kp, ws_bytes, nullptr);
    tile_out[0] = pl.tc.MT;
    tile_out[1] = pl.tc.NT;
    tile_out[2] = pl.tc.MPW;
    tile_out[3] = pl.tc.NPW;
    *splits_out = pl.S;
    *repack_out = pl.repack && kernel_for(pl.tc) == MXFP6_KERNEL_TILE ? 1 : 0;
    return MXFP6_OK;
}

void tune_reset() {
    std::lock_guard<std::mutex> lk(g_tuned_mu);
    g_tuned.clear();
    g_n_tuned.store(0, std::memory_order_release);
}

// The measured plans as text, one per line after a comment line:
//   out_type M N Kp MT NT MPW NPW S repack
int tune_save(const char* path, int* count) {
    std::vector<Tuned> copy;
    {
        std::lock_guard<std::mutex> lk(g_tuned_mu);
        copy = g_tuned;
    }
    FILE* f = std::fopen(path, "w");
    if (f == nullptr) return MXFP6_ERR_ARG;
    bool ok = std::fprintf(f, "# libmxfp6gemm measured plans: out_type M N Kp MT NT MPW NPW S "
                              "repack\n") > 0;
    for (const Tuned& t : copy)
        ok = ok && std::fprintf(f, "%d %d %d %d %d %d %d %d %d %d\n", t.out_type, t.M, t.N, t.Kp,
                                t.plan.tc.MT, t.plan.tc.NT, t.plan.tc.MPW, t.plan.tc.NPW,
                                t.plan.S, t.plan.repack ? 1 : 0) > 0;
    ok = std::fclose(f) == 0 && ok;
    if (count != nullptr) *count = ok ? (int)copy.size() : 0;
    return ok ? MXFP6_OK : MXFP6_ERR_ARG;
}

// Adds the plans of a tune_save file to the table. A line is taken only if it names a tile the
// kernels implement, a split the shape allows, and the scale grouping choose_tile returns for the
// shape on this device (the caller's scales are tiled for that grouping); others are counted as
// skipped, as are malformed lines.
int tune_load(const char* path, int* loaded, int* skipped) {
    FILE* f = std::fopen(path, "r");
    if (f == nullptr) return MXFP6_ERR_ARG;
    int n_ok = 0, n_skip = 0;
    char line[256];
    while (std::fgets(line, sizeof line, f) != nullptr) {
        if (line[0] == '#' || line[0] == '\n') continue;
        int v[10];
        if (std::sscanf(line, "%d %d %d %d %d %d %d %d %d %d", &v[0], &v[1], &v[2], &v[3], &v[4],
                        &v[5], &v[6], &v[7], &v[8], &v[9]) != 10) {
            n_skip++;
            continue;
        }
        const int ot = v[0], M = v[1], N = v[2], Kp = v[3], S = v[8], rp = v[9];
        const TileChoice tc = {v[4], v[5], v[6], v[7]};
        bool ok = ot >= 0 && ot <= 2 && shape_ok(M, N, Kp) && S >= 1 && S <= Kp / K_TILE &&
                  (rp == 0 || rp == 1) && kernel_for(tc) == MXFP6_KERNEL_TILE;
        if (ok) {
            const TileChoice r = route(M, N, Kp);
            ok = r.MPW == tc.MPW && r.NPW == tc.NPW;
        }
        if (!ok) {
            n_skip++;
            continue;
        }
        store_tuned(ot, M, N, Kp, {tc, S, rp != 0});
        n_ok++;
    }
    std::fclose(f);
    if (loaded != nullptr) *loaded = n_ok;
    if (skipped != nullptr) *skipped = n_skip;
    return MXFP6_OK;
}

bool tile_divides(const int tile[4], int M, int N) {
    return tile[0] > 0 && tile[1] > 0 && M % tile[0] == 0 && N % tile[1] == 0 &&
           tile[2] >= 1 && tile[2] <= 4 && tile[3] >= 1 && tile[3] <= 4 &&
           (M / 32) % tile[2] == 0 && (N / 32) % tile[3] == 0;
}

// A tile the explicit plan may run on any M x N: a partial last tile row or column is masked.
bool tile_valid(const int tile[4]) {
    return tile[0] > 0 && tile[1] > 0 && tile[2] >= 1 && tile[2] <= 4 && tile[3] >= 1 &&
           tile[3] <= 4;
}

}  // namespace plan

// ---- C++ API (include/mxfp6/gemm.hpp) ---------------------------------------------------------

TileChoice choose_tile(int M, int N, int Kp) {
    return plan::route(M, N, Kp);
}

size_t gemm_workspace_size(int M, int N, int Kp) {
    return plan::workspace_bytes(M, N, Kp);
}

void gemm(OutType ot, int M, int N, int Kp, const void* dA, const void* dBsh, const uint8_t* dsA,
          const uint8_t* dsB, void* dD, int A_row_bytes, int B_row_bytes, void* ws,
          size_t ws_bytes) {
    (void)B_row_bytes;
    const int st = plan::gemm_checked((int)ot, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, ws,
                                      ws_bytes, nullptr);
    if (st != MXFP6_OK)
        std::fprintf(stderr, "[mxfp6] gemm %dx%dx%d not launched: %s\n", M, N, Kp,
                     plan::status_text(st));
}

// Test hook with the reference's signature (src/gemm.cpp:89-107; not in the public header).
void gemm_force_tile(OutType ot, int M, int N, int Kp, TileChoice tc, const void* dA,
                     const void* dBsh, const uint8_t* dsA, const uint8_t* dsB, void* dD,
                     int A_row_bytes, int B_row_bytes) {
    const int tile[4] = {tc.MT, tc.NT, tc.MPW, tc.NPW};
    const int st = mxfp6_gemm_force_tile((int)ot, M, N, Kp, tile, dA, dBsh, dsA, dsB, dD,
                                         A_row_bytes, B_row_bytes, nullptr);
    if (st != MXFP6_OK)
        std::fprintf(stderr, "[mxfp6] gemm_force_tile %dx%dx%d (%dx%d) not launched: %s\n", M, N,
                     Kp, tc.MT, tc.NT, plan::status_text(st));
}

}  // namespace mxfp6

// ---- C ABI: GEMM part of include/mxfp6_gemm.h -------------------------------------------------

using namespace mxfp6;

extern "C" int mxfp6_kpad(int K) {
    return kpad(K);
}

extern "C" int mxfp6_choose_tile(int M, int N, int Kp, int tile[4]) {
    if (!tile) return MXFP6_ERR_NULL;
    const TileChoice tc = plan::route(M, N, Kp);
    tile[0] = tc.MT;
    tile[1] = tc.NT;
    tile[2] = tc.MPW;
    tile[3] = tc.NPW;
    return MXFP6_OK;
}

extern "C" size_t mxfp6_gemm_workspace_size(int M, int N, int Kp) {
    return plan::workspace_bytes(M, N, Kp);
}

extern "C" size_t mxfp6_gemm_preferred_workspace_size(int M, int N, int Kp) {
    return plan::preferred_workspace_bytes(M, N, Kp);
}

extern "C" int mxfp6_splitk_segments(int M, int N, int Kp) {
    return plan::splitk_segments(M, N, Kp);
}

extern "C" int mxfp6_gemm(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
                          const uint8_t* dsA, const uint8_t* dsB, void* dD, int A_row_bytes,
                          int B_row_bytes, void* ws, size_t ws_bytes) {
    (void)B_row_bytes;
    return plan::gemm_checked(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, ws,
                              ws_bytes, nullptr);
}

extern "C" int mxfp6_gemm_async(int out_type, int M, int N, int Kp, const void* dA,
                                const void* dBsh, const uint8_t* dsA, const uint8_t* dsB, void* dD,
                                int A_row_bytes, int B_row_bytes, void* ws, size_t ws_bytes,
                                void* stream) {
    (void)B_row_bytes;
    return plan::gemm_checked(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, ws,
                              ws_bytes, stream);
}

extern "C" int mxfp6_gemm_noalloc_async(int out_type, int M, int N, int Kp, const void* dA,
                                        const void* dBsh, const uint8_t* dsA, const uint8_t* dsB,
                                        void* dD, int A_row_bytes, int B_row_bytes, void* stream) {
    (void)B_row_bytes;
    const int st = plan::check_common(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes);
    if (st != MXFP6_OK) return st;
    // the plan's split-K partials must fit; a plan that also repacks A runs as planned only when
    // the repacked A fits beside them (gemm_checked runs the fastest plan of the routed scale
    // grouping that fits the partials otherwise)
    if (plan::workspace_bytes(M, N, Kp) > MXFP6_NOALLOC_SCRATCH_BYTES) return MXFP6_ERR_SCRATCH;
    size_t cap = 0;
    void* scratch = mxfp6_hip_scratch(&cap);
    if (scratch == nullptr) return MXFP6_ERR_HIP;
    return plan::gemm_checked(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, scratch,
                              cap, stream);
}

extern "C" int mxfp6_gemm_force_tile(int out_type, int M, int N, int Kp, const int tile[4],
                                     const void* dA, const void* dBsh, const uint8_t* dsA,
                                     const uint8_t* dsB, void* dD, int A_row_bytes,
                                     int B_row_bytes, void* stream) {
    (void)B_row_bytes;
    if (!tile) return MXFP6_ERR_NULL;
    const int st = plan::check_common(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes);
    if (st != MXFP6_OK) return st;
    if (!plan::tile_divides(tile, M, N)) return MXFP6_ERR_TILE;
    const TileChoice tc = {tile[0], tile[1], tile[2], tile[3]};
    if (!mxfp6_hip_has_tile(tc.MT, tc.NT, tc.MPW, tc.NPW)) return MXFP6_ERR_TILE;
    if (!plan::tiny_plan_ok(tc, Kp, 1, MXFP6_A_ROWS)) return MXFP6_ERR_TILE;
    return plan::run(out_type, M, N, Kp, tc, 1, MXFP6_A_ROWS, MXFP6_KERNEL_TILE, dA, dBsh, dsA,
                     dsB, dD, A_row_bytes, nullptr, stream);
}

extern "C" int mxfp6_gemm_explicit(int out_type, int M, int N, int Kp, const int tile[4],
                                   int splits, int a_layout, const void* dA, const void* dBsh,
                                   const uint8_t* dsA, const uint8_t* dsB, void* dD,
                                   int A_row_bytes, void* ws, size_t ws_bytes, void* stream) {
    if (!tile) return MXFP6_ERR_NULL;
    const int st = plan::check_common(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes);
    if (st != MXFP6_OK) return st;
    if (!plan::tile_valid(tile)) return MXFP6_ERR_TILE;
    const TileChoice tc = {tile[0], tile[1], tile[2], tile[3]};
    if (!mxfp6_hip_has_tile(tc.MT, tc.NT, tc.MPW, tc.NPW)) return MXFP6_ERR_TILE;
    if (splits < 1 || splits > Kp / K_TILE || a_layout < MXFP6_A_ROWS ||
        a_layout > MXFP6_A_ROWS_SWIZZLED)
        return MXFP6_ERR_ARG;
    // the swizzled staging of row-major A exists for the wide tiles, unmasked
    if (a_layout == MXFP6_A_ROWS_SWIZZLED && (!plan::is_wide(tc) || !plan::tile_divides(tile, M, N)))
        return MXFP6_ERR_ARG;
    if (!plan::tiny_plan_ok(tc, Kp, splits, a_layout)) return MXFP6_ERR_ARG;
    const bool repack = a_layout == MXFP6_A_REPACK;
    if ((splits > 1 || repack) &&
        (ws == nullptr || ws_bytes < plan::plan_bytes(M, N, Kp, splits, repack)))
        return MXFP6_ERR_ARG;
    return plan::run(out_type, M, N, Kp, tc, splits, a_layout, MXFP6_KERNEL_TILE, dA, dBsh, dsA,
                     dsB, dD, A_row_bytes, ws, stream);
}

extern "C" int mxfp6_gemm_direct(int out_type, int M, int N, int Kp, int mpw, int npw,
                                 const void* dA, const void* dBsh, const uint8_t* dsA,
                                 const uint8_t* dsB, void* dD, int A_row_bytes, int splits,
                                 void* ws, size_t ws_bytes, void* stream) {
    const int st = plan::check_common(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes);
    if (st != MXFP6_OK) return st;
    if (M % 64 != 0 || N % 64 != 0) return MXFP6_ERR_SHAPE;  // its workgroups are 64x64
    if (mpw < 1 || mpw > 4 || npw < 1 || npw > 4 || (M / 32) % mpw != 0 || (N / 32) % npw != 0)
        return MXFP6_ERR_ARG;
    if (splits < 1 || splits > Kp / K_TILE) return MXFP6_ERR_ARG;
    if (splits > 1 && (ws == nullptr || ws_bytes < (size_t)splits * M * N * sizeof(float)))
        return MXFP6_ERR_ARG;
    const TileChoice tc = {128, 128, mpw, npw};
    return plan::run(out_type, M, N, Kp, tc, splits, MXFP6_A_ROWS, MXFP6_KERNEL_DIRECT, dA, dBsh,
                     dsA, dsB, dD, A_row_bytes, splits > 1 ? ws : nullptr, stream);
}

extern "C" int mxfp6_gemm_repacks_a(int M, int N, int Kp) {
    return plan::route_repacks(M, N, Kp) ? 1 : 0;
}

extern "C" int mxfp6_gemm_streams_output(int out_type, int M, int N, int Kp, int A_row_bytes) {
    if (M <= 0 || N <= 0 || Kp <= 0 || Kp % K_TILE != 0) return 0;
    return plan::streams_output(out_type, M, N, Kp, plan::route(M, N, Kp),
                                plan::splitk_segments(M, N, Kp), plan::route_repacks(M, N, Kp),
                                A_row_bytes)
               ? 1
               : 0;
}

extern "C" int mxfp6_gemm_tune(int out_type, int M, int N, int Kp, const void* dA,
                               const void* dBsh, const uint8_t* dsA, const uint8_t* dsB, void* dD,
                               int A_row_bytes, void* ws, size_t ws_bytes, int candidates,
                               void* stream, int tile[4], int* splits, int* a_repack) {
    return plan::tune(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, ws, ws_bytes,
                      candidates, stream, tile, splits, a_repack);
}

extern "C" int mxfp6_gemm_tuned_plan(int out_type, int M, int N, int Kp, int tile[4], int* splits,
                                     int* a_repack) {
    return plan::tuned(out_type, M, N, Kp, tile, splits, a_repack);
}

extern "C" void mxfp6_gemm_tune_reset(void) {
    plan::tune_reset();
}

extern "C" int mxfp6_gemm_tune_save(const char* path, int* count) {
    if (path == nullptr) return MXFP6_ERR_NULL;
    return plan::tune_save(path, count);
}

extern "C" int mxfp6_gemm_tune_load(const char* path, int* loaded, int* skipped) {
    if (path == nullptr) return MXFP6_ERR_NULL;
    return plan::tune_load(path, loaded, skipped);
}

extern "C" int mxfp6_gemm_plan(int out_type, int M, int N, int Kp, size_t ws_bytes, int tile[4],
                               int* splits, int* a_repack) {
    if (out_type < 0 || out_type > 2 || M <= 0 || N <= 0 || Kp <= 0 || Kp % K_TILE != 0)
        return MXFP6_ERR_ARG;
    if (tile == nullptr || splits == nullptr || a_repack == nullptr) return MXFP6_ERR_NULL;
    return plan::plan_info(out_type, M, N, Kp, ws_bytes, tile, splits, a_repack);
}

extern "C" size_t mxfp6_plan_workspace_size(int M, int N, int Kp, int splits, int a_repack) {
    if (M <= 0 || N <= 0 || Kp <= 0 || splits < 1) return 0;
    if (splits == 1 && !a_repack) return 0;
    return plan::plan_bytes(M, N, Kp, splits, a_repack != 0);
}

extern "C" int mxfp6_clock_sample_async(uint64_t* d_out, int nwg, void* stream) {
    if (!d_out) return MXFP6_ERR_NULL;
    if (nwg < 1 || nwg > 65536) return MXFP6_ERR_ARG;
    return mxfp6_hip_clock_sample(d_out, nwg, stream) == 0 ? MXFP6_OK : MXFP6_ERR_HIP;
}

extern "C" int mxfp6_preshuffle_rows_async(const void* src, int row_bytes, int rows, int Kp,
                                           void* dst, void* stream) {
    if (!src || !dst) return MXFP6_ERR_NULL;
    if (rows <= 0 || Kp <= 0 || Kp % K_TILE != 0) return MXFP6_ERR_SHAPE;
    if (row_bytes <= 0 || row_bytes % 4 != 0 || row_bytes < Kp / 4 * 3 - 120) return MXFP6_ERR_SHAPE;
    return mxfp6_hip_repack(src, row_bytes, rows, Kp, dst, stream) == 0 ? MXFP6_OK : MXFP6_ERR_HIP;
}
