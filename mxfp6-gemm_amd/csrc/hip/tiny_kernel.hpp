// Tiny-shape kernel of libmxfp6gemm (tile {32, 32, 1, 1}): one workgroup per 32 x 32 block of D,
// its NW waves (4 or 8) splitting K. The K-tiles form S segments (split_segment, S <=
// TINY_MAX_SEG, at most TINY_MAX_KT K-tiles each); wave w computes segments w, w + NW, ... in turn,
// each as one MFMA accumulation from zero in K order with every A, B and scale load of the segment
// issued before its first MFMA (the operands of up to 12 slabs held in registers: one memory
// latency per segment instead of one per K slab). The waves then sum the S partial blocks from
// LDS, a share of the block each, in segment order from zero, ((0 + P0) + P1) + ..., as the split-K
// reduce does (reduce_kernel.hpp), and store D. The output therefore has the bits of any S-segment
// split plan with a 1 x 1 scale grouping, with no workspace and no second launch.
// For grids of at most a few hundred blocks (the latency floor: 256 x 256 x 1024 runs on 64 of
// the 256 CUs), where a pipelined tile spends its time on per-slab copy issue and barriers.
// A is row-major. Read straight into the MFMA layout (a lane takes its row's 24 bytes of a slab as
// a 16- and an 8-byte load at 8-byte alignment, as the direct kernel's compiled loads do) every
// load touches all 32 rows of the block; where many waves a CU load A that bounds the kernel, so
// the STAGED instantiations read each segment's A along its rows instead (consecutive lanes on
// consecutive 16-byte pieces of a row, a few cache lines per load; 256 x 256 x 4096 7.2 -> 4.6 us
// with such loads in a timing probe), copy it into the wave's own LDS region and read it back in
// the MFMA layout; their segments' partial blocks wait in registers until every wave is done with
// its region, which then holds them. Four instantiations (tiny_launch picks one):
//   MULTI = false, NW = 4, direct A: S <= 4 on the smallest grids (one segment a wave, 16 KiB LDS);
//   STAGED, NW = 8: S > 4 on grids of at most one workgroup per CU (two segments a wave at most;
//     twice the loads in flight at the occupancy of two waves per SIMD);
//   STAGED, NW = 4: S <= 8 otherwise (two workgroups a CU);
//   MULTI, NW = 4, direct A: S = 9-16 on grids past one workgroup per CU (partials in LDS).
// B preshuffled, scales tiled with groups of one 32-block. MASK: the last block row / column
// clamps its A row and masks its stores (the layouts hold whole 32-blocks). The conversion to
// FP16 / BF16 is cvt_out's round to nearest-even, the split-K reduce's.
#pragma once

#include "../hip_layer.h"
#include "device_common.hpp"
#include "lds_dma.hpp"

namespace mxfp6_dev {

constexpr int TINY_MAX_KT = 4;    // K-tiles per segment (operands of 12 slabs in registers)
constexpr int TINY_MAX_SEG = 16;  // segments per workgroup (their partials: 64 KiB of LDS)
// a wave's staged A: 32 rows of up to 576 bytes (4 K-tiles), rows 592 bytes apart (16-byte
// aligned rows; the MFMA-layout reads of 32 rows then fall on distinct bank pairs)
constexpr int TINY_AROW = TINY_MAX_KT * 144 + 16;
constexpr int TINY_AREG = 32 * TINY_AROW;

// One K segment (K-tiles kt0 .. kt0 + nkt - 1, nkt <= TINY_MAX_KT) of the 32 x 32 block: every
// load issued, then the MFMAs in K order from zero.
__device__ __forceinline__ v16f tiny_segment(rsrc_t a_rs, rsrc_t b_rs, rsrc_t sa_rs, rsrc_t sb_rs,
                                             int v_a, int v_b0, int v_b1, int v_sc, int kt0,
                                             int nkt) {
    constexpr int MAXKT = TINY_MAX_KT;
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
    return acc;
}

// One K segment as tiny_segment, with A staged through the wave's LDS region `stage` (TINY_AREG
// bytes, rows TINY_AROW apart): copy i moves LDS piece p = 64 i + l (16 bytes, lane l) from
// 16-byte piece p % 37 of row p / 37 of the segment's A (piece 36 is the row's padding, pieces past
// 9 nkt are not copied; rows past a_rows repeat the last valid one). The copies go first, then the
// B and scale loads (8 per K-tile), so waiting until at most 8 nkt loads are outstanding leaves the
// copies landed; then lane l reads row l % 32's 24 bytes of each slab at K half l / 32.
template <bool MASK>
__device__ __forceinline__ v16f tiny_segment_staged(const uint8_t* a_seg, int A_row_bytes,
                                                    int a_rows, char* stage, rsrc_t b_rs,
                                                    rsrc_t sa_rs, rsrc_t sb_rs, int v_b0, int v_b1,
                                                    int v_sc, int lane, int kt0, int nkt) {
    constexpr int MAXKT = TINY_MAX_KT;
    constexpr int RP = TINY_AROW / 16;              // 37 LDS pieces a row
    constexpr int NI = (32 * RP + 63) / 64;         // 19 copies
    static_assert(RP == 9 * MAXKT + 1, "one padding piece a row");
    const int nch = 9 * nkt;
    // this wave's reads of the region for its previous segment are done before the copies
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const uint32_t st = lds_u32(stage);
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int p = 64 * i + lane;
        const int r = p / RP, c = p - RP * r;
        if (p < 32 * RP && c < nch) {
            const int rr = MASK ? min(r, a_rows - 1) : r;
            dma16(st + 1024 * i, a_seg, opaque_v((uint32_t)(rr * A_row_bytes + 16 * c)));
        }
    }
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
    // the copies have landed once at most the 8 nkt later loads are outstanding (in-order count)
    switch (nkt) {
        case 1: wait_vmcnt<8>(); break;
        case 2: wait_vmcnt<16>(); break;
        case 3: wait_vmcnt<24>(); break;
        default: wait_vmcnt<32>(); break;
    }
    const char* rd = stage + (lane & 31) * TINY_AROW + (lane >> 5) * 24;
#pragma unroll
    for (int c = 0; c < MAXKT; c++) {
        if (c < nkt) {
#pragma unroll
            for (int s = 0; s < SUBS; s++) {
                const char* q = rd + c * 144 + s * 48;
                const v2i x0 = *reinterpret_cast<const v2i*>(q);
                const v2i x1 = *reinterpret_cast<const v2i*>(q + 8);
                const v2i x2 = *reinterpret_cast<const v2i*>(q + 16);
                const v4i x01 = __builtin_shufflevector(x0, x1, 0, 1, 2, 3);
                const v4i x2w = __builtin_shufflevector(x2, x2, 0, 1, -1, -1);
                RA[c][s] = __builtin_shufflevector(x01, x2w, 0, 1, 2, 3, 4, 5, -1, -1);
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
    return acc;
}

// two waves per SIMD: two four-wave workgroups, or one eight-wave workgroup, per CU
template <typename OutT, bool MASK, bool MULTI, int NW, bool STAGED>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
    tiny_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ Bsh,
                const uint8_t* __restrict__ sA, const uint8_t* __restrict__ sB,
                OutT* __restrict__ D, int M, int N, int Kp, int A_row_bytes, int S) {
    static_assert(NW == 4 || (MULTI && NW == 8 && STAGED), "four waves, or eight staging A");
    static_assert(!STAGED || MULTI, "A is staged by the looping instantiations");
    // staged: each wave's staged A, then the partial blocks (at most two segments a wave);
    // otherwise the partial blocks
    constexpr int NSEG = 2;
    static_assert(!STAGED || NSEG * NW * 16 * 64 * 4 <= NW * TINY_AREG, "partials fit the stage");
    __shared__ __align__(16) char lds[STAGED ? NW * TINY_AREG : (MULTI ? TINY_MAX_SEG : 4) * 16 * 64 * 4];
    float(*part)[16][64] = reinterpret_cast<float(*)[16][64]>(lds);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int mb = blockIdx.x, nb = blockIdx.y;
    const int k64n = Kp / 64, k_tiles = Kp / 192;

    // A: the block row's 32 rows from a 64-bit base (32-bit offsets then stay within the block
    // whatever M), the lane's row (the last valid one past M) and K half; B: block nb; scales:
    // group mb / nb
    int a_row = lane & 31;
    if (MASK) a_row = min(a_row, M - 1 - mb * 32);
    const rsrc_t a_rs = raw_rsrc(opaque_gptr(A + (size_t)mb * 32 * A_row_bytes));
    const int v_a = (int)opaque_v((uint32_t)(a_row * A_row_bytes + (lane >> 5) * 24));
    const rsrc_t b_rs = raw_rsrc(opaque_gptr(Bsh + (size_t)nb * k64n * OPBLK_BYTES));
    const rsrc_t sa_rs = raw_rsrc(opaque_gptr(sA + (size_t)mb * k_tiles * 64 * 12));
    const rsrc_t sb_rs = raw_rsrc(opaque_gptr(sB + (size_t)nb * k_tiles * 64 * 12));
    const int v_b0 = (int)opaque_v(16 * lane), v_b1 = (int)opaque_v(1024 + 8 * lane);
    const int v_sc = (int)opaque_v(12 * lane);

    if constexpr (STAGED) {
        // wave w: segments w and w + NW (S <= 2 NW), A staged in its own LDS region; the partial
        // blocks stay in registers until every wave is done with its region
        const uint8_t* a_blk = A + (size_t)mb * 32 * A_row_bytes;
        v16f acc[NSEG];
#pragma unroll
        for (int k = 0; k < NSEG; k++) {
            const int seg = wave + k * NW;
            if (seg < S) {
                int kt0, nkt;
                split_segment(k_tiles, S, seg, kt0, nkt);
                acc[k] = tiny_segment_staged<MASK>(a_blk + kt0 * 144, A_row_bytes, M - mb * 32,
                                                   lds + wave * TINY_AREG, b_rs, sa_rs, sb_rs, v_b0,
                                                   v_b1, v_sc, lane, kt0, nkt);
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < NSEG; k++) {
            const int seg = wave + k * NW;
            if (seg < S) {
#pragma unroll
                for (int e = 0; e < 16; e++) part[seg][e][lane] = acc[k][e];
            }
        }
    } else if constexpr (MULTI) {
        // wave w: segments w, w + 4, ... in turn, each partial to its own LDS block
        for (int seg = wave; seg < S; seg += NW) {
            int kt0, nkt;
            split_segment(k_tiles, S, seg, kt0, nkt);
            const v16f acc = tiny_segment(a_rs, b_rs, sa_rs, sb_rs, v_a, v_b0, v_b1, v_sc, kt0, nkt);
#pragma unroll
            for (int e = 0; e < 16; e++) part[seg][e][lane] = acc[e];
        }
    } else {
        // wave w: segment w (waves past S write a zero block that is never read)
        int kt0 = 0, nkt = 0;
        if (wave < S) split_segment(k_tiles, S, wave, kt0, nkt);
        const v16f acc = tiny_segment(a_rs, b_rs, sa_rs, sb_rs, v_a, v_b0, v_b1, v_sc, kt0, nkt);
#pragma unroll
        for (int e = 0; e < 16; e++) part[wave][e][lane] = acc[e];
    }
    __syncthreads();
    // the sums and stores split over the waves: wave w takes elements EPW w .. EPW w + EPW - 1 of
    // each lane (element e: row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32 of the block); one
    // wave storing all sixteen took 2.1 us of a 4.2 us workgroup at 256 x 256 x 1024, four take
    // about a quarter
    constexpr int EPW = 16 / NW;
    const int col = nb * 32 + (lane & 31);
#pragma unroll
    for (int r = 0; r < EPW; r++) {
        const int e = EPW * wave + r;
        float x = 0.f;
        for (int w = 0; w < S; w++) x += part[w][e][lane];
        const int row = mb * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (!MASK || (row < M && col < N)) D[(size_t)row * N + col] = cvt_out<OutT>(x);
    }
}

// One launch: grid ceil(M/32) x ceil(N/32), 256 or 512 threads; d->splits segments (1 to
// TINY_MAX_SEG, each at most TINY_MAX_KT K-tiles: the host plan guarantees it); row-major A only.
// Returns 0, or 2.
template <typename OutT>
int tiny_launch(const mxfp6_launch_desc* d, hipStream_t st) {
    const int kt = d->Kp / 192;
    if (d->a_layout != MXFP6_A_ROWS || d->splits < 1 || d->splits > TINY_MAX_SEG ||
        (kt + d->splits - 1) / d->splits > TINY_MAX_KT)
        return 2;
    const dim3 grid((unsigned)((d->M + 31) / 32), (unsigned)((d->N + 31) / 32));
    const bool mask = d->M % 32 != 0 || d->N % 32 != 0;
    const uint8_t* A = static_cast<const uint8_t*>(d->A);
    const uint8_t* B = static_cast<const uint8_t*>(d->Bsh);
    OutT* D = static_cast<OutT*>(d->D);
    // S <= 4: one segment a wave, A staged by four waves once the grid's blocks times K-tiles
    // reach twice the CUs (below that, a few waves a CU with short segments, the direct loads
    // were 1-5% faster: 256 x 256 x 1024, 256 x 256 x 384; above it staging was 14-34% faster:
    // 1024 x 512 x 1024, 256 x 256 x 3072, 1024 x 512 x 3072); past four segments A is staged,
    // by eight waves where the grid leaves one workgroup per CU (two segments a wave at most),
    // else by four up to S = 8; four waves with A loaded directly take S = 9-16 on larger grids
    const bool multi = d->splits > 4;
    const int reported = mxfp6_hip_device_cus();
    const long cus = reported > 0 ? reported : 256;
    const long blocks = (long)grid.x * grid.y;
    const bool eight = multi && blocks <= cus;
    const bool staged4 = multi ? !eight && d->splits <= 8 : blocks * kt >= 2 * cus;
    auto k = eight     ? (mask ? tiny_kernel<OutT, true, true, 8, true> : tiny_kernel<OutT, false, true, 8, true>)
             : staged4 ? (mask ? tiny_kernel<OutT, true, true, 4, true> : tiny_kernel<OutT, false, true, 4, true>)
             : multi   ? (mask ? tiny_kernel<OutT, true, true, 4, false> : tiny_kernel<OutT, false, true, 4, false>)
                       : (mask ? tiny_kernel<OutT, true, false, 4, false> : tiny_kernel<OutT, false, false, 4, false>);
    const hipError_t e = launch_kernel(k, grid, dim3(eight ? 512 : 256), st, A, B, d->sA, d->sB, D,
                                       d->M, d->N, d->Kp, d->A_row_bytes, d->splits);
    return e == hipSuccess ? 0 : 2;
}

}  // namespace mxfp6_dev
