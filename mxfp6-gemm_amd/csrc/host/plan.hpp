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
// Plan-time model of the router (plan.cpp): least-squares fit on MI355X, microseconds.
constexpr int MAX_SPLITS = 16;             // K segments considered
constexpr double T_LAUNCH = 2.61668;       // one kernel launch (and its ramp), back to back
constexpr double T_WG = 1.17567;           // fixed cost of one workgroup
constexpr double T_SLAB_MIN = 0.187174;      // latency floor of one 64-wide K slab
constexpr double T_MFMA = 0.00709531;        // per MFMA per wave per slab, per workgroup on the busiest CU
constexpr double T_COPY_KB = 0.0153215;      // per KiB copied global->LDS per slab, per workgroup
constexpr double T_OUT_KB = 0.0256923;      // per KiB of output (FP16 tile or FP32 partial) per workgroup
constexpr double REPACK_BYTES_PER_US = 5.5e6;        // A repack traffic (measured kernel rate)
constexpr double SPLIT_BYTES_PER_US = 4.4079e6;   // split-K partials written and read back
constexpr double A_ROWS_COST = 0.581966;    // extra copy cost per byte of a row-major A slab
constexpr double PLAN_MIN_GAIN = 0.01;     // lead a more complex plan needs over a simpler one

TileChoice route(int M, int N, int Kp);
int splitk_segments(int M, int N, int Kp);
size_t workspace_bytes(int M, int N, int Kp);
size_t preferred_workspace_bytes(int M, int N, int Kp);
bool route_repacks(int M, int N, int Kp);
size_t plan_bytes(int M, int N, int Kp, int S, bool repack);
int check_common(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
                 const void* dsA, const void* dsB, const void* dD, int A_row_bytes);
const char* status_text(int st);

}  // namespace plan
}  // namespace mxfp6
