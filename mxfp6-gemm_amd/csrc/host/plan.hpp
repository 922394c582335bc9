// Internal declarations of the host plan (router, split-K planner, checks).
#pragma once
#include <cstddef>
#include <cstdint>

#include "mxfp6/gemm.hpp"

namespace mxfp6 {
namespace plan {

// MI355X: 256 compute units (8 XCDs x 32 CUs).
constexpr int CUS = 256;
// Shortest K segment of a split, in K-tiles of 192.
constexpr int MIN_TILES_PER_SEG = 8;
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
