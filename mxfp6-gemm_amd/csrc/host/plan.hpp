// Internal declarations of the host plan (router, split-K planner, checks).
#pragma once
#include <cstddef>
#include <cstdint>

#include "mxfp6/gemm.hpp"

namespace mxfp6 {
namespace plan {

// MI355X: 256 compute units (8 XCDs x 32 CUs).
constexpr int CUS = 256;
// Split-K model (see split_for): shortest segment in K-tiles of 192, most segments, the dense
// MXFP6 rate of one CU under full load (MI355X at its power limit: ~3.35 PF / 256 CUs), the
// bandwidth of the partials' round trip, and the least gain a split must promise.
constexpr int MIN_TILES_PER_SEG = 8;
constexpr int MAX_SPLITS = 16;
constexpr double CU_RATE = 13e12;
constexpr double PARTIAL_BW = 5e12;
constexpr double SPLIT_MIN_GAIN = 0.05;
// Smallest (split) grid for which the 256x256 tile is taken without comparing costs.
constexpr long BIG_TILE_MIN_WG = 64;
// Tile columns (N / NT) from which A is repacked to the preshuffled layout first.
constexpr int REPACK_MIN_TILE_COLS = 8;

TileChoice route(int M, int N, int Kp);
int splitk_segments(int M, int N, int Kp);
size_t workspace_bytes(int M, int N, int Kp);
bool route_repacks(int M, int N, int Kp);
size_t plan_bytes(int M, int N, int Kp, int S, bool repack);
int check_common(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
                 const void* dsA, const void* dsB, const void* dD, int A_row_bytes);
const char* status_text(int st);

}  // namespace plan
}  // namespace mxfp6
