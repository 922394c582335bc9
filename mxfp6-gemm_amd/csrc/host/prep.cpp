// C ABI of the device quantisation and layout kernels: argument checks and the plan of blocks to
// write; the kernels themselves are in csrc/hip/prep_kernel.hpp behind the HIP launch layer.
// Reference counterparts (include/mxfp6/preprocess.hpp): quantize_to_mxfp6 (:51-97),
// preprocess_B (:112-118), pad_scales_k (:32-38), preprocess_scale (:136-162), preshuffle_B
// (:182-207), tile_scale (:216-233); the reference runs them on the host only.
#include <algorithm>
#include <cstdint>

#include "hip_layer.h"
#include "mxfp6_gemm.h"

namespace {

constexpr int K_TILE = 192;
constexpr int SUBS = 3;  // 64-wide K slabs per scale K-tile

int kpad_of(int K) { return (K + K_TILE - 1) / K_TILE * K_TILE; }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int status_of(int hip_rc) { return hip_rc == 0 ? MXFP6_OK : MXFP6_ERR_HIP; }

// Blocks of 24 bytes (32 codes) a row of row_bytes spans, rounded up.
int row_blocks(size_t row_bytes) { return (int)((row_bytes + 23) / 24); }

// 32-blocks of K values (the last one zero-padded when K % 32 != 0) and their packed bytes.
int kblocks(int K) { return (K + 31) / 32; }
size_t packed_k(int K) { return (size_t)kblocks(K) * 24; }

}  // namespace

// Ragged sizes (beyond the reference, which needs K % 32 == 0 and whole 32-row blocks): a K that
// is not a multiple of 32 is quantised as if zero-padded to one (its last block holds fewer
// values); rows or columns that do not fill a scale group (32 * group) or a 32-column tile are
// completed with zero rows (codes 0, scale 127) in the tiled scales and the preshuffled operand.

extern "C" int mxfp6_quantize_async(const float* d_x, int rows, int cols, void* d_packed,
                                    size_t packed_row_bytes, uint8_t* d_scales, int scale_cols,
                                    void* stream) {
    if (!d_x || !d_packed || !d_scales) return MXFP6_ERR_NULL;
    if (rows <= 0 || cols <= 0) return MXFP6_ERR_SHAPE;
    if (packed_row_bytes < packed_k(cols) || packed_row_bytes % 4 != 0) return MXFP6_ERR_SHAPE;
    if (scale_cols < kblocks(cols)) return MXFP6_ERR_SHAPE;
    if (!aligned(d_x, 4) || !aligned(d_packed, 4)) return MXFP6_ERR_ARG;
    const int nblk = std::max(scale_cols, row_blocks(packed_row_bytes));
    return status_of(mxfp6_hip_quantize_rows(d_x, rows, cols, nblk, d_packed, packed_row_bytes, 0,
                                             d_scales, 0, scale_cols, 1, K_TILE, stream));
}

extern "C" int mxfp6_prepare_a_async(const float* d_A, int M, int K, int group, void* d_packed,
                                     size_t a_row_bytes, uint8_t* d_tiled, void* stream) {
    if (!d_A || !d_packed || !d_tiled) return MXFP6_ERR_NULL;
    if (group < 1 || group > 4) return MXFP6_ERR_ARG;
    if (M <= 0 || K <= 0) return MXFP6_ERR_SHAPE;
    if (a_row_bytes < packed_k(K) || a_row_bytes % 4 != 0) return MXFP6_ERR_SHAPE;
    if (!aligned(d_A, 4) || !aligned(d_packed, 4)) return MXFP6_ERR_ARG;
    const int Kp = kpad_of(K);
    const int nblk = std::max(Kp / 32, row_blocks(a_row_bytes));
    return status_of(mxfp6_hip_quantize_rows(d_A, M, K, nblk, d_packed, a_row_bytes, 0, d_tiled, 1,
                                             Kp / 32, group, Kp, stream));
}

extern "C" int mxfp6_prepare_a_preshuffled_async(const float* d_A, int M, int K, int group,
                                                 void* d_ash, uint8_t* d_tiled, void* stream) {
    if (!d_A || !d_ash || !d_tiled) return MXFP6_ERR_NULL;
    if (group < 1 || group > 4) return MXFP6_ERR_ARG;
    if (M <= 0 || K <= 0) return MXFP6_ERR_SHAPE;
    if (!aligned(d_A, 4) || !aligned(d_ash, 16)) return MXFP6_ERR_ARG;
    const int Kp = kpad_of(K);
    return status_of(mxfp6_hip_quantize_rows(d_A, M, K, Kp / 32, d_ash, 0, 1, d_tiled, 1, Kp / 32,
                                             group, Kp, stream));
}

extern "C" int mxfp6_prepare_b_async(const float* d_B, int K, int N, int group, void* d_bsh,
                                     uint8_t* d_tiled, void* stream) {
    if (!d_B || !d_bsh || !d_tiled) return MXFP6_ERR_NULL;
    if (group < 1 || group > 4) return MXFP6_ERR_ARG;
    if (N <= 0 || K <= 0) return MXFP6_ERR_SHAPE;
    if (!aligned(d_B, 4) || !aligned(d_bsh, 16)) return MXFP6_ERR_ARG;
    return status_of(mxfp6_hip_prepare_b(d_B, K, N, kpad_of(K), group, d_bsh, d_tiled, stream));
}

extern "C" int mxfp6_tile_scales_async(const uint8_t* d_scales, int dim, int K, int ld, int group,
                                       uint8_t* d_tiled, void* stream) {
    if (!d_scales || !d_tiled) return MXFP6_ERR_NULL;
    if (group < 1 || group > 4) return MXFP6_ERR_ARG;
    if (dim <= 0 || K <= 0 || ld < kblocks(K)) return MXFP6_ERR_SHAPE;
    return status_of(mxfp6_hip_tile_scales(d_scales, dim, kblocks(K), ld, kpad_of(K), group,
                                           d_tiled, stream));
}

extern "C" size_t mxfp6_preshuffled_bytes(int dim, int K) {
    if (dim <= 0 || K <= 0) return 0;
    return (size_t)((dim + 31) / 32) * (size_t)(kpad_of(K) / 64) * 1536;
}

extern "C" size_t mxfp6_tiled_scale_bytes(int dim, int K, int group) {
    if (dim <= 0 || K <= 0 || group < 1 || group > 4) return 0;
    const int gp = (group + 3) / 4 * 4;
    const size_t groups = (size_t)((dim + 32 * group - 1) / (32 * group));
    return groups * (size_t)(kpad_of(K) / K_TILE) * 64 * SUBS * gp;
}
