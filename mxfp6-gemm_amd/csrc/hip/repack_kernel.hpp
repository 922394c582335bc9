// Repack of a row-major packed MXFP6 operand into the preshuffled operand layout.
//
// Source: `rows` rows of packed FP6 codes, row r at src + r * row_bytes, read for packed(Kp) =
// 48 * k64n bytes (a compact row shorter than that is over-read into the next row or the
// buffer's end pad, exactly as the GEMM kernels read it; those bytes meet B's zero K-tail).
// Destination: for each 32-row block mb and 64-wide K slab kk, one 1536-byte tile at
// (mb * k64n + kk) * 1536 holding the slab in MFMA operand order: lane t = 32h + i (row 32mb + i,
// K-half h) owns the row's bytes 48kk + 24h .. +23, the first 16 at 16t, the last 8 at
// 1024 + 8t. This is the layout preshuffle_B gives B^T, so a repacked A is read by the same
// contiguous copies and linear LDS reads as B.
//
// HBM-bound: each workgroup writes KK consecutive tiles of one row block (a contiguous run) and
// reads the matching contiguous 48*KK-byte span of each of its 32 rows. Loads are 4-byte (rows
// are only 4-byte aligned), stores are 16-byte.
#pragma once
#include "device_common.hpp"

namespace mxfp6_dev {

constexpr int REPACK_KK = 12;       // K slabs per workgroup
constexpr int REPACK_THREADS = 256;

__global__ void __launch_bounds__(REPACK_THREADS)
    repack_rows_kernel(const uint8_t* __restrict__ src, int row_bytes, int k64n,
                       uint8_t* __restrict__ dst) {
    const int mb = blockIdx.y;
    const int kk0 = blockIdx.x * REPACK_KK;
    const int nkk = min(REPACK_KK, k64n - kk0);
    const int chunks = nkk * 96;  // 16-byte output chunks of this workgroup
    const uint8_t* rows0 = src + (size_t)mb * 32 * row_bytes;
    uint8_t* out = dst + ((size_t)mb * k64n + kk0) * OPBLK_BYTES;
    for (int c = threadIdx.x; c < chunks; c += REPACK_THREADS) {
        const int j = c / 96, u = c - j * 96;
        const int kbyte = (kk0 + j) * SLAB_BYTES;
        uint32_t w[4];
        if (u < 64) {
            // lane u's first 16 bytes
            const int i = u & 31, h = u >> 5;
            const uint32_t* s = reinterpret_cast<const uint32_t*>(rows0 + (size_t)i * row_bytes + kbyte + 24 * h);
            w[0] = s[0], w[1] = s[1], w[2] = s[2], w[3] = s[3];
        } else {
            // the last 8 bytes of lanes 2p and 2p+1 (same K-half, rows i and i+1)
            const int t = 2 * (u - 64), i = t & 31, h = t >> 5;
            const uint32_t* s0 = reinterpret_cast<const uint32_t*>(rows0 + (size_t)i * row_bytes + kbyte + 24 * h + 16);
            const uint32_t* s1 = reinterpret_cast<const uint32_t*>(rows0 + (size_t)(i + 1) * row_bytes + kbyte + 24 * h + 16);
            w[0] = s0[0], w[1] = s0[1], w[2] = s1[0], w[3] = s1[1];
        }
        *reinterpret_cast<v4i*>(out + (size_t)c * 16) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    }
}

}  // namespace mxfp6_dev
