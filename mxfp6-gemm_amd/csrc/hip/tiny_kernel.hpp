// Tiny-shape kernel of libmxfp6gemm (tile {32, 32, 1, 1}): one workgroup per 32 x 32 block of D,
// its four waves splitting K. Wave w computes K segment w of S (split_segment, S <= 4, at most
// TINY_MAX_KT K-tiles per segment) as one MFMA accumulation from zero in K order, with every
// A, B and scale load of its segment issued before its first MFMA (the operands of up to 12
// slabs held in registers: one memory latency per call instead of one per K slab); the S
// partial blocks then meet in LDS and the four waves sum them, a quarter of the block each, in
// segment order from zero, ((0 + P0) + P1) + ..., as the split-K reduce does (reduce_kernel.hpp),
// and store D. The output
// therefore has the bits of any S-segment split plan with a 1 x 1 scale grouping, with no
// workspace and no second launch.
// For grids of a few dozen blocks and short K (the latency floor: 256 x 256 x 1024 runs on 64 of
// the 256 CUs), where a pipelined tile spends its time on per-slab copy issue and barriers.
// A is row-major (a lane reads its row's 24 bytes of a slab as a 16- and an 8-byte load at
// 8-byte alignment, as the direct kernel's compiled loads do), B
// preshuffled, scales tiled with groups of one 32-block. MASK: the last block row / column
// clamps its A row and masks its stores (the layouts hold whole 32-blocks). The conversion to
// FP16 / BF16 is cvt_out's round to nearest-even, the split-K reduce's.
#pragma once

#include "../hip_layer.h"
#include "device_common.hpp"
#include "lds_dma.hpp"

namespace mxfp6_dev {

constexpr int TINY_MAX_KT = 4;  // K-tiles per segment (operands of 12 slabs in registers)

template <typename OutT, bool MASK>
__global__ void __launch_bounds__(256)
    tiny_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ Bsh,
                const uint8_t* __restrict__ sA, const uint8_t* __restrict__ sB,
                OutT* __restrict__ D, int M, int N, int Kp, int A_row_bytes, int S) {
    constexpr int MAXKT = TINY_MAX_KT;
    __shared__ float part[4][16][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int mb = blockIdx.x, nb = blockIdx.y;
    const int k64n = Kp / 64, k_tiles = Kp / 192;
    int kt0 = 0, nkt = 0;
    if (wave < S) split_segment(k_tiles, S, wave, kt0, nkt);

    // A: the lane's row (the last valid one past M) and K half; B: block nb; scales: group mb / nb
    int row = mb * 32 + (lane & 31);
    if (MASK) row = min(row, M - 1);
    const rsrc_t a_rs = raw_rsrc(opaque_gptr(A));
    const int v_a = (int)opaque_v((uint32_t)(row * A_row_bytes + (lane >> 5) * 24));
    const rsrc_t b_rs = raw_rsrc(opaque_gptr(Bsh + (size_t)nb * k64n * OPBLK_BYTES));
    const rsrc_t sa_rs = raw_rsrc(opaque_gptr(sA + (size_t)mb * k_tiles * 64 * 12));
    const rsrc_t sb_rs = raw_rsrc(opaque_gptr(sB + (size_t)nb * k_tiles * 64 * 12));
    const int v_b0 = (int)opaque_v(16 * lane), v_b1 = (int)opaque_v(1024 + 8 * lane);
    const int v_sc = (int)opaque_v(12 * lane);

    v8i RA[MAXKT][SUBS], RB[MAXKT][SUBS];
    v3i SA[MAXKT], SB[MAXKT];
#pragma unroll
    for (int c = 0; c < MAXKT; c++) {
        if (c < nkt) {
            const int kt = kt0 + c;
            SA[c] = __builtin_bit_cast(v3i, __builtin_amdgcn_raw_buffer_load_b96(sa_rs, v_sc, kt * 768, 0));
            SB[c] = __builtin_bit_cast(v3i, __builtin_amdgcn_raw_buffer_load_b96(sb_rs, v_sc, kt * 768, 0));
#pragma unroll
            for (int s = 0; s < SUBS; s++) {
                const int ka = kt * (SUBS * SLAB_BYTES);
                const v4i x01 = __builtin_bit_cast(
                    v4i, __builtin_amdgcn_raw_buffer_load_b128(a_rs, v_a + s * SLAB_BYTES, ka, 0));
                const v2i x2 = __builtin_bit_cast(
                    v2i, __builtin_amdgcn_raw_buffer_load_b64(a_rs, v_a + s * SLAB_BYTES + 16, ka, 0));
                const v4i x2w = __builtin_shufflevector(x2, x2, 0, 1, -1, -1);
                RA[c][s] = __builtin_shufflevector(x01, x2w, 0, 1, 2, 3, 4, 5, -1, -1);
                const int kb = kt * (SUBS * OPBLK_BYTES);
                const v4i y0 = __builtin_bit_cast(
                    v4i, __builtin_amdgcn_raw_buffer_load_b128(b_rs, v_b0 + s * OPBLK_BYTES, kb, 0));
                const v2i y1 = __builtin_bit_cast(
                    v2i, __builtin_amdgcn_raw_buffer_load_b64(b_rs, v_b1 + s * OPBLK_BYTES, kb, 0));
                const v4i y1w = __builtin_shufflevector(y1, y1, 0, 1, -1, -1);
                RB[c][s] = __builtin_shufflevector(y0, y1w, 0, 1, 2, 3, 4, 5, -1, -1);
            }
        }
    }
    v16f acc = {};
#pragma unroll
    for (int c = 0; c < MAXKT; c++) {
        if (c < nkt) {
            acc = mfma_fp6<0, 0>(acc, RA[c][0], RB[c][0], SA[c].x, SB[c].x);
            acc = mfma_fp6<0, 0>(acc, RA[c][1], RB[c][1], SA[c].y, SB[c].y);
            acc = mfma_fp6<0, 0>(acc, RA[c][2], RB[c][2], SA[c].z, SB[c].z);
        }
    }
#pragma unroll
    for (int e = 0; e < 16; e++) part[wave][e][lane] = acc[e];
    __syncthreads();
    // the sums and stores split over the four waves: wave w takes elements 4 w .. 4 w + 3 of each
    // lane (rows 8 w + 4 (l / 32) + r, r < 4, column l % 32 of the block); one wave storing all
    // sixteen took 2.1 us of a 4.2 us workgroup at 256 x 256 x 1024, four take about a quarter
    const int col = nb * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int e = 4 * wave + r;
        float x = 0.f;
        for (int w = 0; w < S; w++) x += part[w][e][lane];
        const int row = mb * 32 + 8 * wave + 4 * (lane >> 5) + r;
        if (!MASK || (row < M && col < N)) D[(size_t)row * N + col] = cvt_out<OutT>(x);
    }
}

// One launch: grid ceil(M/32) x ceil(N/32), 256 threads; d->splits segments (1 to 4, each at
// most TINY_MAX_KT K-tiles: the host plan guarantees it); row-major A only. Returns 0, or 2.
template <typename OutT>
int tiny_launch(const mxfp6_launch_desc* d, hipStream_t st) {
    const int kt = d->Kp / 192;
    if (d->a_layout != MXFP6_A_ROWS || d->splits < 1 || d->splits > 4 ||
        (kt + d->splits - 1) / d->splits > TINY_MAX_KT)
        return 2;
    const dim3 grid((unsigned)((d->M + 31) / 32), (unsigned)((d->N + 31) / 32));
    const bool mask = d->M % 32 != 0 || d->N % 32 != 0;
    const uint8_t* A = static_cast<const uint8_t*>(d->A);
    const uint8_t* B = static_cast<const uint8_t*>(d->Bsh);
    OutT* D = static_cast<OutT*>(d->D);
    const hipError_t e =
        mask ? launch_kernel(tiny_kernel<OutT, true>, grid, dim3(256), st, A, B, d->sA, d->sB, D,
                             d->M, d->N, d->Kp, d->A_row_bytes, d->splits)
             : launch_kernel(tiny_kernel<OutT, false>, grid, dim3(256), st, A, B, d->sA, d->sB, D,
                             d->M, d->N, d->Kp, d->A_row_bytes, d->splits);
    return e == hipSuccess ? 0 : 2;
}

}  // namespace mxfp6_dev
