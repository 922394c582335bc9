// Internal declarations of the host plan (router, split-K planner, checks).
#pragma once
#include <cstddef>
#include <cstdint>

#include "mxfp6/gemm.hpp"

namespace mxfp6 {
namespace plan {

// Compute units the router plans for when the HIP runtime reports no device (a host without a
// GPU): MI355X's 256 (8 XCDs x 32 CUs). On a device the count is read from it (plan.cpp).
constexpr int DEFAULT_CUS = 256;
// Plan-time model of the router (plan.cpp): fitted on MI355X measurements, microseconds.
constexpr int SPLIT_CHOICES[] = {1, 2, 3, 4, 6, 8, 12, 16};  // K segments considered
constexpr double T_LAUNCH = 2.40452;       // one kernel launch (and its ramp), back to back
constexpr double T_WG = 0.806055;           // fixed cost of one workgroup
constexpr double T_SLAB_MIN = 0.183313;      // latency floor of one 64-wide K slab
constexpr double T_MFMA = 0.00394993;        // per MFMA per wave per slab, per workgroup on the busiest CU
constexpr double T_COPY_KB = 0.0165642;      // per KiB copied global->LDS per slab, per workgroup
constexpr double T_BREG_KB = 0.00831597;     // per KiB of B loaded into registers per slab (wide tiles)
constexpr double T_L2_KB = 7.1085e-05;     // per KiB per slab of every workgroup in flight (L2 -> CUs)
constexpr double T_OUT_KB = 0.0216756;      // per KiB of output (FP16 tile or FP32 partial) per workgroup
constexpr double REPACK_BYTES_PER_US = 5.5e6;        // A repack traffic (measured kernel rate)
constexpr double SPLIT_BYTES_PER_US = 4059650.0;   // split-K partials written and read back
constexpr double A_ROWS_COST = 0.572519;    // extra copy cost per byte of a row-major A slab
constexpr double A_ROWS_COST_WIDE = 0.0675946;  // the same for the wide tiles' K-tile chunks
constexpr double A_ROWS_LONG = 0.158036;    // more per doubling of Kp past 8192 (row-major A)
constexpr double PLAN_MIN_GAIN = 0.01;     // lead a more complex plan needs over a simpler one
// An unsplit plan on a wide tile writes D with nontemporal stores when the bytes it reads (operands, scales, the
// repacked A) fit in MI355X's 256 MiB last-level cache (Infinity Cache) but those and D together
// exceed STREAM_FOOTPRINT_BYTES: D then no longer evicts the operands the tiles re-read. Measured:
// streaming D 6-22% faster above the footprint (8192x16384x2048, 4096x51200x1024,
// 16384x16384x4096, 1024x102272x2048, 2048x102272x1024), plain stores 5-12% faster below it
// (8192x8192x2048, 8192x12288x2048, 2048x51200x1024), no difference once the operands alone
// exceed the cache (2048x102272x4096).
constexpr double LLC_BYTES = 268435456.0;
constexpr double STREAM_FOOTPRINT_BYTES = 280e6;

TileChoice route(int M, int N, int Kp);
int splitk_segments(int M, int N, int Kp);
size_t workspace_bytes(int M, int N, int Kp);
size_t preferred_workspace_bytes(int M, int N, int Kp);
bool route_repacks(int M, int N, int Kp);
bool streams_output(int out_type, int M, int N, int Kp, const TileChoice& tc, int S, bool repack,
                    int A_row_bytes);
int tune(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh, const uint8_t* dsA,
         const uint8_t* dsB, void* dD, int A_row_bytes, void* ws, size_t ws_bytes,
         int candidates, void* stream, int tile_out[4], int* splits_out, int* repack_out);
int tuned(int out_type, int M, int N, int Kp, int tile_out[4], int* splits_out, int* repack_out);
void tune_reset();
int tune_save(const char* path, int* count);
int tune_load(const char* path, int* loaded, int* skipped);
int plan_info(int out_type, int M, int N, int Kp, size_t ws_bytes, int tile_out[4],
              int* splits_out, int* repack_out);
size_t plan_bytes(int M, int N, int Kp, int S, bool repack);
int check_common(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
                 const void* dsA, const void* dsB, const void* dD, int A_row_bytes);
const char* status_text(int st);

}  // namespace plan
}  // namespace mxfp6
