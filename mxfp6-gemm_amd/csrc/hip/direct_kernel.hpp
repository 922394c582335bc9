// Direct MXFP6 kernel: one wave per 32x32 output block, operands loaded straight from global
// memory in the public layouts (no LDS, no pipelining). It is the simplest correct reading of
// the operand/scale contract and accepts any scale grouping, so it serves as the fallback for
// tiles the pipelined kernel does not instantiate and as an independent GPU cross-check of it.
#pragma once
#include "device_common.hpp"

namespace mxfp6_dev {

// Grid (M/64, N/64, S), 256 threads: wave w of a workgroup computes 32-row block
// 2*blockIdx.x + w/2 and 32-column block 2*blockIdx.y + w%2 over K segment blockIdx.z.
// Requires M % 64 == 0, N % 64 == 0, Kp % 192 == 0, A_row_bytes % 4 == 0.
template <typename OutT, bool SPLIT>
__global__ void __launch_bounds__(256)
    direct_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ Bsh,
                  const uint8_t* __restrict__ sA, const uint8_t* __restrict__ sB,
                  OutT* __restrict__ D, float* __restrict__ ws, int M, int N, int Kp,
                  int A_row_bytes, int mpw, int npw, int S) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int mb = blockIdx.x * 2 + (wave >> 1);
    const int nb = blockIdx.y * 2 + (wave & 1);
    const int k64n = Kp / 64, k_tiles = Kp / 192;
    int kt0 = 0, nkt = k_tiles;
    if (SPLIT) split_segment(k_tiles, S, (int)blockIdx.z, kt0, nkt);

    const int gpa = (mpw + 3) & ~3, gpb = (npw + 3) & ~3;
    // operand row / column of this lane and its K half
    const uint8_t* arow = A + (size_t)(mb * 32 + (lane & 31)) * A_row_bytes + (lane >> 5) * 24;
    const uint8_t* bcol = Bsh + (size_t)nb * k64n * OPBLK_BYTES;
    // tiled scales: byte (((g*k_tiles + kt)*64 + lane)*3 + sub)*gp + j for block g*group + j
    const uint8_t* sa = sA + ((size_t)(mb / mpw) * k_tiles * 64 + lane) * SUBS * gpa + (mb % mpw);
    const uint8_t* sb = sB + ((size_t)(nb / npw) * k_tiles * 64 + lane) * SUBS * gpb + (nb % npw);

    v16f acc = {};
    for (int kt = kt0; kt < kt0 + nkt; kt++) {
#pragma unroll
        for (int sub = 0; sub < SUBS; sub++) {
            const int q = kt * SUBS + sub;
            const uint32_t* pa = reinterpret_cast<const uint32_t*>(arow + (size_t)q * SLAB_BYTES);
            v8i a = {(int)pa[0], (int)pa[1], (int)pa[2], (int)pa[3], (int)pa[4], (int)pa[5], 0, 0};
            const uint8_t* tb = bcol + (size_t)q * OPBLK_BYTES;
            const v4i b0 = *reinterpret_cast<const v4i*>(tb + lane * 16);
            const v2i b1 = *reinterpret_cast<const v2i*>(tb + 1024 + lane * 8);
            v8i b = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, 0, 0};
            const size_t so = ((size_t)kt * 64 * SUBS + sub);
            const int sav = sa[so * gpa];
            const int sbv = sb[so * gpb];
            acc = mfma_fp6<0, 0>(acc, a, b, sav, sbv);
        }
    }

    const int n = nb * 32 + (lane & 31);
    const int m0 = mb * 32 + 4 * (lane >> 5);
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const size_t idx = (size_t)(m0 + 8 * g + r) * N + n;
            if (SPLIT)
                ws[(size_t)blockIdx.z * M * N + idx] = acc[4 * g + r];
            else
                D[idx] = cvt_out<OutT>(acc[4 * g + r]);
        }
}

}  // namespace mxfp6_dev
