// Host plan of libmxfp6gemm: shape router, split-K planner, argument checks and the public entry
// points (C++ API of include/mxfp6/gemm.hpp and the GEMM part of the C ABI in
// include/mxfp6_gemm.h). Plain C++17 with no HIP header: every device action goes through the
// thin launch layer declared in hip_layer.h.
#include <cstdio>

#include "../hip_layer.h"
#include "mxfp6/gemm.hpp"
#include "mxfp6_gemm.h"
#include "plan.hpp"

namespace mxfp6 {
namespace plan {

// ---- router ------------------------------------------------------------------------------
//
// Candidate tiles (each an instantiation of the pipelined kernel, 4 waves per workgroup, one
// workgroup per CU):
//   256x256, waves 2x2, each wave 128x128 -> MPW 4, NPW 4   (work 4 units of 128x128)
//   256x192, waves 2x2, each wave 128x96  -> MPW 4, NPW 3   (3 units)
//   128x384, waves 1x4, each wave 128x96  -> MPW 4, NPW 3   (3 units)
//   128x256, waves 2x2, each wave  64x128 -> MPW 2, NPW 4   (2 units)
//   128x128, waves 2x2, each wave  64x64  -> MPW 2, NPW 2   (1 unit)
// The kernel is bound by the per-CU global->LDS copy rate (64 B/clk per CU on MI355X), so the
// tiles that move the fewest operand bytes per flop, 256x256 and 256x192, are preferred whenever
// one divides the shape and its (split) grid has at least BIG_TILE_MIN_WG workgroups: measured on
// MI355X they beat a smaller tile that fills every CU. Between the two, and otherwise among all
// candidates that divide the shape, workgroup-starved grids are split along K (split_for) and the
// cost of a candidate is the number of CU waves its (split) grid needs times the work of one
// workgroup: ceil(wg * S / CUS) * units / S. The cheapest wins; ties go to the earlier (larger)
// tile.
namespace {
struct Cand {
    TileChoice tc;
    int units;
};
const Cand kCands[] = {{{256, 256, 4, 4}, 4}, {{256, 192, 4, 3}, 3}, {{128, 384, 4, 3}, 3},
                       {{128, 256, 2, 4}, 2}, {{128, 128, 2, 2}, 1}};
constexpr int N_BIG = 2;  // kCands[0 .. N_BIG) are the big tiles

// K segments for a tile on (M, N, Kp), from a time model: a (split) grid of wg * S workgroups
// takes ceil(wg * S / CUS) CU waves of t_tile / S each (t_tile: one workgroup over all of K at
// CU_RATE), and every segment adds one FP32 write and read of an M x N partial at PARTIAL_BW.
// S runs up to MAX_SPLITS with at least MIN_TILES_PER_SEG K-tiles per segment; a split must beat
// S = 1 by SPLIT_MIN_GAIN. Measured at 2048x5120x105728 (160 workgroups of 256x256): S = 1, 3, 4,
// 6, 8 take 792, 688, 746, 734, 763 us, and the model picks S = 3; 2048x1024x105728 gets S = 8.
int split_for(const TileChoice& tc, int M, int N, int Kp) {
    const long wg = (long)(M / tc.MT) * (N / tc.NT);
    const int k_tiles = Kp / K_TILE;
    if (wg <= 0) return 1;
    const double t_tile = (double)k_tiles * 2.0 * tc.MT * tc.NT * K_TILE / CU_RATE;
    const double t_part = 2.0 * M * N * sizeof(float) / PARTIAL_BW;
    const double base = (double)((wg + CUS - 1) / CUS) * t_tile;
    int best = 1;
    double best_cost = base * (1.0 - SPLIT_MIN_GAIN);
    for (int S = 2; S <= MAX_SPLITS && k_tiles / S >= MIN_TILES_PER_SEG; S++) {
        const double cost = (double)((wg * S + CUS - 1) / CUS) * t_tile / S + S * t_part;
        if (cost < best_cost) {
            best = S;
            best_cost = cost;
        }
    }
    return best;
}
}  // namespace

TileChoice route(int M, int N, int Kp) {
    TileChoice best = {128, 128, 2, 2};
    double best_cost = -1;
    // shapes gemm() rejects (M, N multiples of 128, Kp of K_TILE) get the smallest tile, no split
    if (M <= 0 || N <= 0 || Kp <= 0 || M % 128 != 0 || N % 128 != 0 || Kp % K_TILE != 0)
        return best;
    auto cost_of = [&](const Cand& c) {
        const long wg = (long)(M / c.tc.MT) * (N / c.tc.NT);
        const int S = split_for(c.tc, M, N, Kp);
        return (double)((wg * S + CUS - 1) / CUS) * c.units / S;
    };
    for (int i = 0; i < N_BIG; i++) {
        const Cand& c = kCands[i];
        if (M % c.tc.MT != 0 || N % c.tc.NT != 0) continue;
        if ((long)(M / c.tc.MT) * (N / c.tc.NT) * split_for(c.tc, M, N, Kp) < BIG_TILE_MIN_WG)
            continue;
        const double cost = cost_of(c);
        if (best_cost < 0 || cost < best_cost - 1e-9) {
            best = c.tc;
            best_cost = cost;
        }
    }
    if (best_cost >= 0) return best;
    for (const Cand& c : kCands) {
        if (M % c.tc.MT != 0 || N % c.tc.NT != 0) continue;
        const double cost = cost_of(c);
        if (best_cost < 0 || cost < best_cost - 1e-9) {
            best = c.tc;
            best_cost = cost;
        }
    }
    return best;
}

// Whether A is first repacked into the preshuffled operand layout (an HBM-bound pass over A).
// A row-major A costs the tile kernel's copies one 128-byte cache line per 48 useful bytes of a
// row and slab; repacked, every copy is a contiguous 1 KiB. The pass pays when the kernel re-reads
// each A row band many times, i.e. when the output has many tile columns.
bool repack_for(const TileChoice& tc, int M, int N, int Kp) {
    (void)M;
    (void)Kp;
    return N / tc.NT >= REPACK_MIN_TILE_COLS;
}

size_t split_bytes(int M, int N, int S) {
    return S > 1 ? (size_t)S * (size_t)M * (size_t)N * sizeof(float) : 0;
}

size_t repack_bytes(int M, int Kp) {
    return (size_t)M * (size_t)(Kp / 4 * 3);
}

size_t plan_bytes(int M, int N, int Kp, int S, bool repack) {
    const size_t sb = (split_bytes(M, N, S) + 255) / 256 * 256;
    return sb + (repack ? repack_bytes(M, Kp) : 0);
}

bool route_repacks(int M, int N, int Kp) {
    if (M <= 0 || N <= 0 || Kp <= 0 || M % 128 != 0 || N % 128 != 0 || Kp % K_TILE != 0)
        return false;
    const TileChoice tc = route(M, N, Kp);
    if (M % tc.MT != 0 || N % tc.NT != 0) return false;
    return repack_for(tc, M, N, Kp);
}

int splitk_segments(int M, int N, int Kp) {
    if (M <= 0 || N <= 0 || Kp <= 0 || M % 128 != 0 || N % 128 != 0 || Kp % K_TILE != 0) return 1;
    const TileChoice tc = route(M, N, Kp);
    if (M % tc.MT != 0 || N % tc.NT != 0) return 1;
    return split_for(tc, M, N, Kp);
}

size_t workspace_bytes(int M, int N, int Kp) {
    const int S = splitk_segments(M, N, Kp);
    const bool rp = route_repacks(M, N, Kp);
    return (S > 1 || rp) ? plan_bytes(M, N, Kp, S, rp) : 0;
}

// ---- argument checks -----------------------------------------------------------------------

int check_common(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
                 const void* dsA, const void* dsB, const void* dD, int A_row_bytes) {
    if (out_type < 0 || out_type > 2) return MXFP6_ERR_OUT_TYPE;
    if (!dA || !dBsh || !dsA || !dsB || !dD) return MXFP6_ERR_NULL;
    if (M <= 0 || N <= 0 || M % 128 != 0 || N % 128 != 0) return MXFP6_ERR_SHAPE;
    if (Kp <= 0 || Kp % K_TILE != 0) return MXFP6_ERR_SHAPE;
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
        case MXFP6_ERR_SHAPE: return "unsupported shape (M, N multiples of 128; Kp multiple of 192; A_row_bytes)";
        case MXFP6_ERR_OUT_TYPE: return "out_type must be F32, F16 or BF16";
        case MXFP6_ERR_TILE: return "tile not implemented or does not divide the shape";
        case MXFP6_ERR_ARG: return "invalid argument";
        case MXFP6_ERR_HIP: return "HIP launch error";
        default: return "unknown status";
    }
}

// ---- launch ----------------------------------------------------------------------------------

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
    d.stream = stream;
    const int rc = mxfp6_hip_launch(&d);
    return rc == 0 ? MXFP6_OK : rc == 1 ? MXFP6_ERR_TILE : MXFP6_ERR_HIP;
}

int kernel_for(const TileChoice& tc) {
    return mxfp6_hip_has_tile(tc.MT, tc.NT, tc.MPW, tc.NPW) ? MXFP6_KERNEL_TILE
                                                            : MXFP6_KERNEL_DIRECT;
}

int gemm_checked(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
                 const uint8_t* dsA, const uint8_t* dsB, void* dD, int A_row_bytes, void* ws,
                 size_t ws_bytes, void* stream) {
    const int st = check_common(out_type, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes);
    if (st != MXFP6_OK) return st;
    const TileChoice tc = route(M, N, Kp);
    if (N % tc.NT != 0 || M % tc.MT != 0) return MXFP6_ERR_TILE;
    int S = split_for(tc, M, N, Kp);
    bool rp = repack_for(tc, M, N, Kp);
    const int kernel = kernel_for(tc);
    if (kernel != MXFP6_KERNEL_TILE) rp = false;
    if (ws == nullptr) ws_bytes = 0;
    // A workspace too small for the repacked A drops the repack (a pure speed choice); one too
    // small for the split-K partials as well runs unsplit, with the reference's warning.
    if (rp && ws_bytes < plan_bytes(M, N, Kp, S, true)) rp = false;
    if (S > 1 && ws_bytes < plan_bytes(M, N, Kp, S, false)) {
        std::fprintf(stderr,
                     "[mxfp6] %dx%dx%d: split-K over %d segments needs a %zu-byte workspace, "
                     "got %zu; running unsplit. Size it with gemm_workspace_size().\n",
                     M, N, Kp, S, split_bytes(M, N, S), ws_bytes);
        S = 1;
    }
    return run(out_type, M, N, Kp, tc, S, rp ? MXFP6_A_REPACK : MXFP6_A_ROWS, kernel, dA, dBsh, dsA,
               dsB, dD, A_row_bytes, ws, stream);
}

bool tile_divides(const int tile[4], int M, int N) {
    return tile[0] > 0 && tile[1] > 0 && M % tile[0] == 0 && N % tile[1] == 0 &&
           tile[2] >= 1 && tile[2] <= 4 && tile[3] >= 1 && tile[3] <= 4 &&
           (M / 32) % tile[2] == 0 && (N / 32) % tile[3] == 0;
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
    if (!plan::tile_divides(tile, M, N)) return MXFP6_ERR_TILE;
    const TileChoice tc = {tile[0], tile[1], tile[2], tile[3]};
    if (!mxfp6_hip_has_tile(tc.MT, tc.NT, tc.MPW, tc.NPW)) return MXFP6_ERR_TILE;
    if (splits < 1 || splits > Kp / K_TILE || a_layout < MXFP6_A_ROWS ||
        a_layout > MXFP6_A_PRESHUFFLED)
        return MXFP6_ERR_ARG;
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

extern "C" size_t mxfp6_plan_workspace_size(int M, int N, int Kp, int splits, int a_repack) {
    if (M <= 0 || N <= 0 || Kp <= 0 || splits < 1) return 0;
    if (splits == 1 && !a_repack) return 0;
    return plan::plan_bytes(M, N, Kp, splits, a_repack != 0);
}

extern "C" int mxfp6_preshuffle_rows_async(const void* src, int row_bytes, int rows, int Kp,
                                           void* dst, void* stream) {
    if (!src || !dst) return MXFP6_ERR_NULL;
    if (rows <= 0 || rows % 32 != 0 || Kp <= 0 || Kp % K_TILE != 0) return MXFP6_ERR_SHAPE;
    if (row_bytes <= 0 || row_bytes % 4 != 0 || row_bytes < Kp / 4 * 3 - 120) return MXFP6_ERR_SHAPE;
    return mxfp6_hip_repack(src, row_bytes, rows, Kp, dst, stream) == 0 ? MXFP6_OK : MXFP6_ERR_HIP;
}
