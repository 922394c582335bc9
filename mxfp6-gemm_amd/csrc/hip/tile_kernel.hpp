// LDS-pipelined MXFP6 tile kernel for gfx950.
//
// One workgroup = 4 waves (256 threads) computes an MT x NT tile of D; wave (wm, wn) of a
// WM x WN wave grid owns MPW x NPW 32x32 blocks (MPW = MT/32/WM, NPW = NT/32/WN), accumulated in
// FP32 AGPRs by v_mfma_scale_f32_32x32x64_f8f6f4 (FP6 E2M3 x FP6 E2M3, per-lane E8M0 scales).
//
// K is walked in K-tiles of 192 (three 64-wide slabs, the scale layout's grouping). Both operands
// of a K-tile are copied global -> LDS by the direct-to-LDS DMA (global_load_lds_dwordx4), double
// buffered: the copy of K-tile t+1 is issued right after the barrier that opens K-tile t and has
// the whole MFMA work of K-tile t to land.
//   B: its preshuffled layout is already in MFMA operand order (per 32x64 block: lane t's 16
//      bytes at 16t, its last 8 bytes at 1024+8t), so a K-tile of one 32-column block is a
//      contiguous 4608-byte run copied verbatim; operand reads are linear ds_read_b128 + b64.
//   A: rows of 144 bytes (the K-tile's 192 codes), copied row-major with 16-byte chunks
//      (coalesced global reads); the operand of lane l is 24 bytes at row l%32, byte 24*(l/32)
//      of the slab.
//   Scales: per wave and K-tile one dwordx3 per operand from the tiled-scale layout (group =
//      MPW for A, NPW for B); dword `sub` holds the scale bytes of the wave's blocks for slab
//      `sub`, and the MFMA's op_sel picks the block's byte, so no shifts are needed.
// Epilogue: lane l of block (mi, ni) holds column l%32 and rows 8g + 4(l/32) + r; D row-major.
// Split-K (SPLIT): blockIdx.z selects a K segment and FP32 partials go to ws[z][M][N].
#pragma once
#include "../hip_layer.h"
#include "device_common.hpp"

namespace mxfp6_dev {

constexpr int KT_ELEMS = 192;        // K per K-tile
constexpr int KT_ROW_BYTES = 144;    // packed bytes of one row per K-tile
constexpr int KT_CHUNKS = 9;         // 16-byte chunks per row per K-tile
constexpr int BLK_TILE_BYTES = 4608; // one 32-column B block per K-tile (3 x 1536)

typedef __attribute__((address_space(3))) void lds_void;

// Issue the DMA of `total` 16-byte chunks; chunk c of the workgroup's list goes to LDS
// lds_base + 16*c, from the global address src(c). Thread tid handles c = i*256 + tid.
template <int TOTAL, class Src>
__device__ __forceinline__ void dma_chunks(char* lds_base, int wave, int lane, Src src) {
#pragma unroll
    for (int i = 0; i < (TOTAL + 255) / 256; i++) {
        const int c0 = i * 256 + wave * 64;  // first chunk of this wave (wave-uniform)
        const int c = c0 + lane;
        if ((TOTAL % 256 == 0) || c < TOTAL) {
            __builtin_amdgcn_global_load_lds(src(c), (lds_void*)(lds_base + c0 * 16), 16, 0, 0);
        }
    }
}

template <int MT, int NT, int WM, int WN, typename OutT, bool SPLIT>
__global__ void __launch_bounds__(256, 1)
    tile_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ Bsh,
                const uint8_t* __restrict__ sA, const uint8_t* __restrict__ sB,
                OutT* __restrict__ D, float* __restrict__ ws, int M, int N, int Kp,
                int A_row_bytes, int S) {
    constexpr int MPW = MT / 32 / WM, NPW = NT / 32 / WN;
    static_assert(WM * WN == 4, "4 waves per workgroup");
    static_assert(MPW >= 1 && MPW <= 4 && NPW >= 1 && NPW <= 4, "scale groups hold <= 4 blocks");
    constexpr int A_STAGE = MT * KT_ROW_BYTES, B_STAGE = NT * KT_ROW_BYTES;
    constexpr int A_CHUNKS = MT * KT_CHUNKS, B_CHUNKS = NT * KT_CHUNKS;
    __shared__ __attribute__((aligned(16))) char lds_a[2][A_STAGE];
    __shared__ __attribute__((aligned(16))) char lds_b[2][B_STAGE];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WN, wn = wave % WN;
    const int wg_m = blockIdx.x, wg_n = blockIdx.y;
    const int k64n = Kp / 64, k_tiles = Kp / KT_ELEMS;
    int kt0 = 0, nkt = k_tiles;
    if (SPLIT) split_segment(k_tiles, S, (int)blockIdx.z, kt0, nkt);

    const uint8_t* a_rows = A + (size_t)wg_m * MT * A_row_bytes;
    const uint8_t* b_cols = Bsh + (size_t)wg_n * (NT / 32) * k64n * OPBLK_BYTES;
    // tiled scales of this wave: group (wg_m*WM + wm) of A, (wg_n*WN + wn) of B; 12 bytes per
    // (K-tile, lane)
    const uint8_t* sa_w = sA + ((size_t)(wg_m * WM + wm) * k_tiles * 64 + lane) * 12;
    const uint8_t* sb_w = sB + ((size_t)(wg_n * WN + wn) * k_tiles * 64 + lane) * 12;

    auto issue_tile = [&](int kt, int buf) {
        const size_t a_k = (size_t)kt * KT_ROW_BYTES;
        dma_chunks<A_CHUNKS>(lds_a[buf], wave, lane, [&](int c) {
            const int row = c / KT_CHUNKS, part = c - row * KT_CHUNKS;
            return (const void*)(a_rows + (size_t)row * A_row_bytes + a_k + part * 16);
        });
        const size_t b_k = (size_t)kt * 3 * OPBLK_BYTES;
        dma_chunks<B_CHUNKS>(lds_b[buf], wave, lane, [&](int c) {
            const int blk = c / (BLK_TILE_BYTES / 16), r = c - blk * (BLK_TILE_BYTES / 16);
            return (const void*)(b_cols + (size_t)blk * k64n * OPBLK_BYTES + b_k + r * 16);
        });
    };
    auto load_scales = [&](int kt, v3i& sa, v3i& sb) {
        sa = *reinterpret_cast<const v3i*>(sa_w + (size_t)kt * 64 * 12);
        sb = *reinterpret_cast<const v3i*>(sb_w + (size_t)kt * 64 * 12);
    };

    v16f acc[MPW][NPW];
#pragma unroll
    for (int i = 0; i < MPW; i++)
#pragma unroll
        for (int j = 0; j < NPW; j++) acc[i][j] = v16f{};

    // operand byte offsets inside a stage
    const int a_off = (wm * MPW * 32 + (lane & 31)) * KT_ROW_BYTES + (lane >> 5) * 24;
    const int b_off = wn * NPW * BLK_TILE_BYTES + lane * 16;
    const int b_off2 = wn * NPW * BLK_TILE_BYTES + 1024 + lane * 8;

    v3i sa_cur, sb_cur, sa_nxt, sb_nxt;
    issue_tile(kt0, 0);
    load_scales(kt0, sa_cur, sb_cur);

    for (int i = 0; i < nkt; i++) {
        const int buf = i & 1;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (i + 1 < nkt) {
            issue_tile(kt0 + i + 1, buf ^ 1);
            load_scales(kt0 + i + 1, sa_nxt, sb_nxt);
        }
        const char* la = lds_a[buf];
        const char* lb = lds_b[buf];
#pragma unroll
        for (int s = 0; s < 3; s++) {
            v8i a[MPW], b[NPW];
#pragma unroll
            for (int mi = 0; mi < MPW; mi++) {
                const char* p = la + a_off + mi * 32 * KT_ROW_BYTES + s * 48;
                const v2i x0 = *reinterpret_cast<const v2i*>(p);
                const v2i x1 = *reinterpret_cast<const v2i*>(p + 8);
                const v2i x2 = *reinterpret_cast<const v2i*>(p + 16);
                a[mi] = v8i{x0.x, x0.y, x1.x, x1.y, x2.x, x2.y, 0, 0};
            }
#pragma unroll
            for (int ni = 0; ni < NPW; ni++) {
                const v4i y0 = *reinterpret_cast<const v4i*>(lb + b_off + ni * BLK_TILE_BYTES + s * OPBLK_BYTES);
                const v2i y1 = *reinterpret_cast<const v2i*>(lb + b_off2 + ni * BLK_TILE_BYTES + s * OPBLK_BYTES);
                b[ni] = v8i{y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, 0, 0};
            }
            const int sav = sa_cur[s], sbv = sb_cur[s];
#pragma unroll
            for (int ni = 0; ni < NPW; ni++)
#pragma unroll
                for (int mi = 0; mi < MPW; mi++) {
                    // op_sel selects byte mi of the A scale dword and byte ni of the B one
                    switch (mi * 4 + ni) {
#define MX_CASE(I, J) \
    case I * 4 + J: acc[mi][ni] = mfma_fp6<I, J>(acc[mi][ni], a[mi], b[ni], sav, sbv); break;
                        MX_CASE(0, 0) MX_CASE(0, 1) MX_CASE(0, 2) MX_CASE(0, 3)
                        MX_CASE(1, 0) MX_CASE(1, 1) MX_CASE(1, 2) MX_CASE(1, 3)
                        MX_CASE(2, 0) MX_CASE(2, 1) MX_CASE(2, 2) MX_CASE(2, 3)
                        MX_CASE(3, 0) MX_CASE(3, 1) MX_CASE(3, 2) MX_CASE(3, 3)
#undef MX_CASE
                    }
                }
        }
        sa_cur = sa_nxt;
        sb_cur = sb_nxt;
    }

    // epilogue
    const int m_w = wg_m * MT + wm * MPW * 32 + 4 * (lane >> 5);
    const int n_w = wg_n * NT + wn * NPW * 32 + (lane & 31);
#pragma unroll
    for (int mi = 0; mi < MPW; mi++)
#pragma unroll
        for (int ni = 0; ni < NPW; ni++)
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const size_t idx = (size_t)(m_w + mi * 32 + 8 * g + r) * N + n_w + ni * 32;
                    if (SPLIT)
                        ws[(size_t)blockIdx.z * M * N + idx] = acc[mi][ni][4 * g + r];
                    else
                        D[idx] = cvt_out<OutT>(acc[mi][ni][4 * g + r]);
                }
}

// ---- instantiations and launch -------------------------------------------------------------------

inline bool tile_supported(int MT, int NT, int mpw, int npw) {
    return (MT == 128 && NT == 128 && mpw == 2 && npw == 2) ||
           (MT == 128 && NT == 256 && mpw == 2 && npw == 4) ||
           (MT == 128 && NT == 384 && mpw == 4 && npw == 3) ||
           (MT == 256 && NT == 256 && mpw == 4 && npw == 4);
}

template <int MT, int NT, int WM, int WN, typename OutT>
int tile_launch_t(const mxfp6_launch_desc* d, hipStream_t st) {
    const dim3 grid((unsigned)(d->M / MT), (unsigned)(d->N / NT), (unsigned)d->splits);
    const uint8_t* A = static_cast<const uint8_t*>(d->A);
    const uint8_t* B = static_cast<const uint8_t*>(d->Bsh);
    if (d->splits > 1)
        tile_kernel<MT, NT, WM, WN, float, true><<<grid, dim3(256), 0, st>>>(
            A, B, d->sA, d->sB, nullptr, d->ws, d->M, d->N, d->Kp, d->A_row_bytes, d->splits);
    else
        tile_kernel<MT, NT, WM, WN, OutT, false><<<grid, dim3(256), 0, st>>>(
            A, B, d->sA, d->sB, static_cast<OutT*>(d->D), nullptr, d->M, d->N, d->Kp,
            d->A_row_bytes, 1);
    return 0;
}

template <typename OutT>
int tile_launch(const mxfp6_launch_desc* d, hipStream_t st) {
    if (!tile_supported(d->MT, d->NT, d->mpw, d->npw)) return 1;
    if (d->MT == 128 && d->NT == 128) return tile_launch_t<128, 128, 2, 2, OutT>(d, st);
    if (d->MT == 128 && d->NT == 256) return tile_launch_t<128, 256, 2, 2, OutT>(d, st);
    if (d->MT == 128 && d->NT == 384) return tile_launch_t<128, 384, 1, 4, OutT>(d, st);
    return tile_launch_t<256, 256, 2, 2, OutT>(d, st);
}

}  // namespace mxfp6_dev
