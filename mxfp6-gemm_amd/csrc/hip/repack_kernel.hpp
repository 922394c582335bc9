// Repack of a row-major packed MXFP6 operand into the preshuffled operand layout.
//
// Source: `rows` rows of packed FP6 codes, row r at src + r * row_bytes, read for packed(Kp) =
// 48 * k64n bytes (a compact row shorter than that is over-read into the next row or the
// buffer's end pad, exactly as the GEMM kernels read it; those bytes meet B's zero K-tail).
// Destination: ceil(rows / 32) row blocks (rows past `rows` in the last block are zero codes);
// for each 32-row block mb and 64-wide K slab kk, one 1536-byte tile at
// (mb * k64n + kk) * 1536 holding the slab in MFMA operand order: lane t = 32h + i (row 32mb + i,
// K-half h) owns the row's bytes 48kk + 24h .. +23, the first 16 at 16t, the last 8 at
// 1024 + 8t. This is the layout preshuffle_B gives B^T, so a repacked A is read by the same
// contiguous copies and linear LDS reads as B.
//
// HBM-bound transpose through LDS: a workgroup takes one 32-row block and REPACK_KK consecutive
// slabs. It reads the block's 32 row segments of 48 * REPACK_KK bytes with coalesced loads (VEC
// bytes per lane, consecutive lanes on consecutive bytes of a row; VEC = 16, 8 or 4 by the row
// alignment) into LDS, then writes the REPACK_KK output tiles, one contiguous run, with 16-byte
// stores whose pieces it gathers from LDS.
#pragma once
#include "device_common.hpp"

namespace mxfp6_dev {

// K slabs per workgroup: 8 (12 KiB of LDS) measured 5.9 TB/s on MI355X at 8192 x 8256 against
// 5.0 for 16 and 3.6 for 32 (more, smaller workgroups overlap one's loads with another's stores)
constexpr int REPACK_KK = 8;
constexpr int REPACK_THREADS = 256;
constexpr int REPACK_SEG = 48 * REPACK_KK;  // bytes of one row segment (384)

template <int VEC>
__global__ void __launch_bounds__(REPACK_THREADS)
    repack_rows_kernel(const uint8_t* __restrict__ src, int row_bytes, int rows, int k64n,
                       uint8_t* __restrict__ dst) {
    __shared__ __attribute__((aligned(16))) uint8_t seg[32 * REPACK_SEG];
    const int mb = blockIdx.y;
    const int kk0 = blockIdx.x * REPACK_KK;
    const int nkk = min(REPACK_KK, k64n - kk0);
    const int seg_bytes = nkk * SLAB_BYTES;
    const uint8_t* rows0 = src + (size_t)mb * 32 * row_bytes + (size_t)kk0 * SLAB_BYTES;
    const int nrows = min(32, rows - mb * 32);  // rows of this block that exist

    // phase 1: 32 row segments -> LDS (row-major, REPACK_SEG bytes per row)
    const int per_row = seg_bytes / VEC;
    for (int c = threadIdx.x; c < 32 * per_row; c += REPACK_THREADS) {
        const int i = c / per_row, o = (c - i * per_row) * VEC;
        const uint8_t* s = rows0 + (size_t)i * row_bytes + o;
        uint8_t* d = seg + i * REPACK_SEG + o;
        if (i >= nrows) {
            for (int b = 0; b < VEC; b += 4) *reinterpret_cast<int*>(d + b) = 0;
            continue;
        }
        if constexpr (VEC == 16)
            *reinterpret_cast<v4i*>(d) = *reinterpret_cast<const v4i*>(s);
        else if constexpr (VEC == 8)
            *reinterpret_cast<v2i*>(d) = *reinterpret_cast<const v2i*>(s);
        else
            *reinterpret_cast<int*>(d) = *reinterpret_cast<const int*>(s);
    }
    __syncthreads();

    // phase 2: output chunk c (16 bytes) of tile j: lanes u < 64 take their first 16 bytes,
    // chunks 64..95 the last 8 bytes of lanes 2p and 2p+1
    uint8_t* out = dst + ((size_t)mb * k64n + kk0) * OPBLK_BYTES;
    for (int c = threadIdx.x; c < nkk * 96; c += REPACK_THREADS) {
        const int j = c / 96, u = c - j * 96;
        v2i lo, hi;
        if (u < 64) {
            const uint8_t* s = seg + (u & 31) * REPACK_SEG + j * SLAB_BYTES + 24 * (u >> 5);
            lo = *reinterpret_cast<const v2i*>(s);
            hi = *reinterpret_cast<const v2i*>(s + 8);
        } else {
            const int t = 2 * (u - 64), i = t & 31, h = t >> 5;
            const uint8_t* s = seg + i * REPACK_SEG + j * SLAB_BYTES + 24 * h + 16;
            lo = *reinterpret_cast<const v2i*>(s);
            hi = *reinterpret_cast<const v2i*>(s + REPACK_SEG);
        }
        // ordinary (temporal) loads and stores: the tile kernel reads the copy right after, and
        // what stays cached of it helps (C3-sized A 1-3% faster end to end than with
        // nontemporal accesses; unchanged at 8192^3 and at 2048 x 105728)
        *reinterpret_cast<v4i*>(out + (size_t)c * 16) = v4i{lo.x, lo.y, hi.x, hi.y};
    }
}

// Launch: the widest load the source rows' alignment allows.
inline hipError_t repack_rows_launch(const uint8_t* src, int row_bytes, int rows, int k64n,
                                     uint8_t* dst, hipStream_t st) {
    const dim3 grid((unsigned)((k64n + REPACK_KK - 1) / REPACK_KK), (unsigned)((rows + 31) / 32));
    const uintptr_t align = reinterpret_cast<uintptr_t>(src) | (uintptr_t)row_bytes;
    auto* k = align % 16 == 0 ? repack_rows_kernel<16>
              : align % 8 == 0 ? repack_rows_kernel<8>
                               : repack_rows_kernel<4>;
    return launch_kernel(k, grid, dim3(REPACK_THREADS), st, src, row_bytes, rows, k64n, dst);
}

}  // namespace mxfp6_dev
