#pragma once
// libmxfp6gemm — public C++ API of the MI355X (gfx950) MXFP6 GEMM.
//
//   D[M,N] = A[M,K] · B[K,N]
//
// A and B are MXFP6: 6-bit FP6 E2M3 codes, four codes packed into three bytes, with one
// E8M0 (power-of-two) scale per 32-element block along K. D is FP32, FP16 or BF16.
//
// The declarations below keep the exact names, signatures and meaning of the reference
// library's public header (include/mxfp6/gemm.hpp:25-64 in eeezio/mxfp6-gemm), so a caller
// of that library recompiles and links against this one unchanged. The header is
// device-free: no HIP include, so plain host C++ can use it.
//
// Inputs are device buffers prepared on the host with mxfp6/preprocess.hpp:
//   * A packed row-major, A_row_bytes per row (compact packed(K) rows or padded packed(Kp));
//   * B transposed to B^T[N][Kp] (zero K-tail), then preshuffle_B;
//   * A scales and B scales laid out by preprocess_scale + tile_scale, grouped with
//     choose_tile(M,N,Kp).MPW (A) and .NPW (B), where Kp is the same value passed to gemm().
#include <cstddef>
#include <cstdint>

namespace mxfp6 {

enum class OutType { F32, F16, BF16 };

// K is consumed in slabs of K_TILE elements; callers pass Kp = kpad(K). The padded tail must
// be zero on B (preprocess_B over a zero-padded float B gives that), which nulls whatever A
// holds there. A's scale tail must not contain the E8M0 NaN code 0xFF.
constexpr int K_TILE = 192;
inline int kpad(int K) {
    return (K + K_TILE - 1) / K_TILE * K_TILE;
}

// The tile the library runs (M,N,Kp) on, and the scale grouping its kernel reads:
// MT x NT output tile per workgroup; MPW / NPW = number of 32-row blocks of A / 32-column
// blocks of B held by one wave. tile_scale() must be called with group = MPW for A's
// scales and group = NPW for B's. Kp is required and must equal the Kp given to gemm().
struct TileChoice {
    int MT, NT, MPW, NPW;
};
TileChoice choose_tile(int M, int N, int Kp);

// Bytes of FP32 split-K workspace gemm() uses for (M, N, Kp); 0 when the shape is not split.
// The buffer is owned by the caller (allocate once, reuse; one per concurrent stream). A larger
// workspace (mxfp6_gemm_preferred_workspace_size in mxfp6_gemm.h) also lets gemm() repack A into
// the layout its kernel reads fastest; the output is the same bits.
size_t gemm_workspace_size(int M, int N, int Kp);

// Launches D = A·B on the null stream; asynchronous to the host.
//   dA   packed MXFP6 A, A_row_bytes per row; the kernel reads packed(Kp) bytes per row
//   dBsh preshuffled B^T (preshuffle_B)
//   dsA  A scales, tile_scale(preprocess_scale(.., M, Kp), MPW, 3)
//   dsB  B scales, tile_scale(preprocess_scale(.., N, Kp), NPW, 3)
//   dD   M x N row-major output of element type ot (float / __half / __hip_bfloat16)
//   B_row_bytes is accepted for interface compatibility; B is addressed via its preshuffle.
//   ws / ws_bytes: split-K workspace sized by gemm_workspace_size(); (nullptr, 0) never
//   splits. A shape that would split with a missing or short workspace runs unsplit and a
//   warning goes to stderr. Extra workspace bytes beyond the partials may hold a repacked copy
//   of A (see gemm_workspace_size).
void gemm(OutType ot, int M, int N, int Kp, const void* dA, const void* dBsh, const uint8_t* dsA,
          const uint8_t* dsB, void* dD, int A_row_bytes, int B_row_bytes, void* ws, size_t ws_bytes);

}  // namespace mxfp6
