// LDS-pipelined MXFP6 tile kernel for gfx950.
//
// One workgroup = 4 waves (256 threads) computes an MT x NT tile of D; wave (wm, wn) of a
// WM x WN wave grid owns MPW x NPW 32x32 blocks (MPW = MT/32/WM, NPW = NT/32/WN), accumulated in
// FP32 AGPRs by v_mfma_scale_f32_32x32x64_f8f6f4 (FP6 E2M3 x FP6 E2M3, per-lane E8M0 scales).
//
// K is walked in K-tiles of 192 (three 64-wide slabs, the scale layout's grouping). Both operands
// of a K-tile are copied global -> LDS by the direct-to-LDS DMA (global_load_lds_dwordx4) into a
// two-stage ring.
//   B: its preshuffled layout is already in MFMA operand order (per 32x64 block: lane t's first
//      16 bytes at 16t, its last 8 at 1024+8t), so one 32-column block of a K-tile is a
//      contiguous 4608-byte run copied verbatim; operand reads are linear ds_read_b128 + b64.
//   A: rows of 144 bytes (the K-tile's 192 codes) copied row-major in 16-byte chunks (coalesced
//      global reads); lane l's operand is 24 bytes at row l%32, byte 24*(l/32) of the slab.
//   Scales: the tiled-scale layout (group = MPW for A, NPW for B) keeps one group's scales of a
//      K-tile in a contiguous 768-byte run (64 lanes x 3 dwords), so the workgroup's WM + WN runs
//      ride the same DMA into the stage; a wave reads dword `sub` of its lane for slab `sub`, and
//      the MFMA's op_sel picks the block's byte inside it.
// Schedule per K-tile t (stage t%2), software-pipelined by one slab:
//      read slab1 | MFMA slab0 | read slab2 | MFMA slab1 | wait own DMA, barrier, DMA(t+2) into
//      this stage, read slab0 of t+1 | MFMA slab2
// so the barrier, the DMA issue and the first LDS reads of the next K-tile overlap the last
// slab's MFMAs, and the copy of K-tile t+1 has a whole K-tile of MFMA work to land.
// The DMA is inline asm (M0 + global_load_lds in one statement): the compiler sees neither an
// LDS store it cannot tell apart from the other stage's ds_reads (it would wait for the next
// K-tile's copy before every read) nor any pending vector load in the main loop (its loop-merge
// waits would do the same). The waits are explicit: each wave drains its own copies (vmcnt(0))
// before the barrier that publishes a stage. The loop is peeled so its body has no branches.
// Workgroup order: with XG > 0 the linear workgroup id is remapped so the workgroups running at
// the same time on one XCD (ids congruent mod 8) cover an XG-row band of output tiles, sharing
// A and B tiles in that XCD's L2.
// Epilogue: lane l of block (mi, ni) holds column l%32 and rows 8g + 4(l/32) + r; D row-major.
// Split-K (SPLIT): blockIdx.z selects a K segment; FP32 partials go to ws[z][M][N].
#pragma once
#include <type_traits>

#include "../hip_layer.h"
#include "device_common.hpp"

namespace mxfp6_dev {

constexpr int KT_ELEMS = 192;         // K per K-tile
constexpr int KT_ROW_BYTES = 144;     // packed bytes of one row per K-tile
constexpr int KT_CHUNKS = 9;          // 16-byte chunks per row per K-tile
constexpr int BLK_TILE_BYTES = 4608;  // one 32-column B block per K-tile (3 x 1536)
constexpr int NXCD = 8;               // MI355X: 8 XCDs, workgroup id i runs on XCD i % 8

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// 16 bytes per lane global -> LDS: lane l's bytes go to LDS m0 + 16*l. `lds` must be uniform.
__device__ __forceinline__ void dma16(uint32_t lds, const void* gbase, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds), "v"(voff), "s"(gbase)
                 : "memory");
}

// Same with a per-lane 64-bit global address.
__device__ __forceinline__ void dma16_flat(uint32_t lds, const void* gaddr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds), "v"(gaddr)
                 : "memory");
}

typedef __attribute__((address_space(3))) const char* lds_cptr;

// Returns x unchanged, hidden from the optimizer (forces a VGPR, defeats offset folding).
__device__ __forceinline__ uint32_t opaque_v(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ void wait_vmcnt0() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Bijective map of the linear workgroup id onto (tile_m, tile_n) such that each XCD receives a
// contiguous run of the grouped order (groups of XG tile rows, tile_m fastest).
__device__ __forceinline__ void xcd_tile(int gm, int gn, int XG, int pid, int& tm, int& tn) {
    const int total = gm * gn;
    const int per = total / NXCD, rem = total % NXCD;
    const int x = pid % NXCD, j = pid / NXCD;
    const int L = x < rem ? x * (per + 1) + j : rem * (per + 1) + (x - rem) * per + j;
    const int band = XG * gn;
    const int grp = L / band, rows = min(XG, gm - grp * XG), w = L - grp * band;
    tm = grp * XG + w % rows;
    tn = w / rows;
}

template <int MT, int NT, int WM, int WN, int XG, typename OutT, bool SPLIT>
__global__ void __launch_bounds__(64 * WM * WN, 1)
    tile_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ Bsh,
                const uint8_t* __restrict__ sA, const uint8_t* __restrict__ sB,
                OutT* __restrict__ D, float* __restrict__ ws, int M, int N, int Kp,
                int A_row_bytes, int S) {
    constexpr int MPW = MT / 32 / WM, NPW = NT / 32 / WN;
    constexpr int NWAVES = WM * WN, THREADS = 64 * NWAVES;
    static_assert(NWAVES == 4 || NWAVES == 8, "4 or 8 waves per workgroup");
    static_assert(MPW >= 1 && MPW <= 4 && NPW >= 1 && NPW <= 4, "scale groups hold <= 4 blocks");
    constexpr int A_STAGE = MT * KT_ROW_BYTES, B_STAGE = NT * KT_ROW_BYTES;
    constexpr int SC_GROUP = 64 * 12;  // one scale group per K-tile: 64 lanes x 3 dwords
    constexpr int SC_STAGE = (WM + WN) * SC_GROUP;
    constexpr int SC_CHUNKS = SC_STAGE / 16;
    // the scale copy is one instruction; lanes past SC_CHUNKS inside a partly used wave land in
    // this pad, waves entirely past it in the dummy area
    constexpr int SC_PAD = (64 - SC_CHUNKS % 64) % 64 * 16;
    constexpr int STAGE = A_STAGE + B_STAGE + SC_STAGE + SC_PAD;
    // 1 KiB sink for the lanes of waves with no chunk in a partial DMA instruction: they copy a
    // valid source there instead of branching around the copy (a branch would split the loop
    // body into blocks and let the compiler sink MFMAs past the stage barrier)
    constexpr int DUMMY = 2 * STAGE;
    constexpr int A_CHUNKS = MT * KT_CHUNKS, B_CHUNKS = NT * KT_CHUNKS;
    static_assert(SC_CHUNKS <= THREADS, "one DMA instruction for the scales");
    constexpr int A_ISS = (A_CHUNKS + THREADS - 1) / THREADS;
    constexpr int B_ISS = (B_CHUNKS + THREADS - 1) / THREADS;
    constexpr int B_BLK_CHUNKS = BLK_TILE_BYTES / 16;
    __shared__ __attribute__((aligned(1024))) char lds[2 * STAGE + 1024];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WN, wn = wave % WN;
    int wg_m = blockIdx.x, wg_n = blockIdx.y;
    if constexpr (XG > 0) {
        if (!SPLIT || ((gridDim.x * gridDim.y) % NXCD) == 0)
            xcd_tile((int)gridDim.x, (int)gridDim.y, XG, (int)(blockIdx.y * gridDim.x + blockIdx.x),
                     wg_m, wg_n);
    }
    const int k64n = Kp / 64, k_tiles = Kp / KT_ELEMS;
    int kt0 = 0, nkt = k_tiles;
    if (SPLIT) split_segment(k_tiles, S, (int)blockIdx.z, kt0, nkt);

    const uint8_t* a_base = A + (size_t)wg_m * MT * A_row_bytes;
    const uint8_t* b_base = Bsh + (size_t)wg_n * (NT / 32) * k64n * OPBLK_BYTES;

    // per-thread DMA source offsets (constant across K-tiles; the K-tile moves the base)
    uint32_t a_voff[A_ISS], b_voff[B_ISS];
#pragma unroll
    for (int i = 0; i < A_ISS; i++) {
        const int c = (i * THREADS + tid) % A_CHUNKS, row = c / KT_CHUNKS, part = c - row * KT_CHUNKS;
        a_voff[i] = (uint32_t)(row * A_row_bytes + part * 16);
    }
#pragma unroll
    for (int i = 0; i < B_ISS; i++) {
        const int c = (i * THREADS + tid) % B_CHUNKS, blk = c / B_BLK_CHUNKS, r = c - blk * B_BLK_CHUNKS;
        b_voff[i] = (uint32_t)(blk * k64n * OPBLK_BYTES + r * 16);
    }
    // scale chunk of this thread: group tid/48 of [A groups of the workgroup | B groups],
    // 16 bytes at r*16 of that group's 768-byte run for a K-tile (tiled-scale layout:
    // byte ((g*k_tiles + kt)*64 + lane)*12 + 4*sub + j)
    const uint8_t* sc_src;
    {
        const int t = tid < SC_CHUNKS ? tid : SC_CHUNKS - 1;
        const int grp = t / 48, r = t - grp * 48;
        const int g = grp < WM ? wg_m * WM + grp : wg_n * WN + (grp - WM);
        sc_src = (grp < WM ? sA : sB) + (size_t)g * k_tiles * SC_GROUP + r * 16;
    }
    const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(lds_u32(lds) + wave * 1024);
    const uint32_t lds_dummy = __builtin_amdgcn_readfirstlane(lds_u32(lds) + DUMMY);
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);

    // DMA instruction j (0 <= j < N_DMA) of K-tile kt into stage st: A chunks, B chunks, scales
    constexpr int N_DMA = A_ISS + B_ISS + 1;
    auto dma_op = [&](int j, int kt, int st) {
        const uint32_t la = lds_wave + st * STAGE, lb = la + A_STAGE, ls = lb + B_STAGE;
        if (j < A_ISS) {
            const bool live = A_CHUNKS % THREADS == 0 || j * THREADS + wave_u * 64 < A_CHUNKS;
            dma16(live ? la + j * THREADS * 16 : lds_dummy, a_base + (size_t)kt * KT_ROW_BYTES,
                  a_voff[j]);
        } else if (j < A_ISS + B_ISS) {
            const int i = j - A_ISS;
            const bool live = B_CHUNKS % THREADS == 0 || i * THREADS + wave_u * 64 < B_CHUNKS;
            dma16(live ? lb + i * THREADS * 16 : lds_dummy, b_base + (size_t)kt * BLK_TILE_BYTES,
                  b_voff[i]);
        } else {
            dma16_flat(wave_u * 64 < SC_CHUNKS ? ls : lds_dummy, sc_src + (size_t)kt * SC_GROUP);
        }
    };
    auto issue_tile = [&](int kt, int st) {
#pragma unroll
        for (int j = 0; j < N_DMA; j++) dma_op(j, kt, st);
    };

    // operand byte offsets inside a stage
    const int a_off = (wm * MPW * 32 + (lane & 31)) * KT_ROW_BYTES + (lane >> 5) * 24;
    const int b_off = A_STAGE + wn * NPW * BLK_TILE_BYTES + lane * 16;
    const int b_off2 = A_STAGE + wn * NPW * BLK_TILE_BYTES + 1024 + lane * 8;
    const int sa_off = A_STAGE + B_STAGE + wm * SC_GROUP + lane * 12;
    const int sb_off = A_STAGE + B_STAGE + (WM + wn) * SC_GROUP + lane * 12;

    struct Slab {
        v8i a[MPW], b[NPW];
        int sa, sb;
    };
    // LDS operand reads. Each operand's byte offset goes through opaque_v(): with no common
    // provable base the backend cannot fuse reads of different operands into ds_read2 forms,
    // whose results it would then have to copy into each operand's 6-register tuple (each copy
    // waiting on its read). A: one 24-byte (three 8-byte) read; B: 16 + 8 bytes.
    const lds_cptr lds3 = (lds_cptr)lds;
    auto read_slab = [&](int st, int s, Slab& R) {
        const uint32_t base = st * STAGE;
#pragma unroll
        for (int mi = 0; mi < MPW; mi++) {
            const uint32_t o = opaque_v(base + a_off + mi * 32 * KT_ROW_BYTES + s * 48);
            const v6i_a8 x = *reinterpret_cast<const __attribute__((address_space(3))) v6i_a8*>(lds3 + o);
            R.a[mi] = __builtin_shufflevector(x, x, 0, 1, 2, 3, 4, 5, -1, -1);
        }
#pragma unroll
        for (int ni = 0; ni < NPW; ni++) {
            const uint32_t o = opaque_v(base + b_off + ni * BLK_TILE_BYTES + s * OPBLK_BYTES);
            const v4i y0 = *reinterpret_cast<const __attribute__((address_space(3))) v4i*>(lds3 + o);
            const v2i y1 = *reinterpret_cast<const __attribute__((address_space(3))) v2i*>(lds3 + o + (1024 - 8 * lane));
            const v4i y1w = __builtin_shufflevector(y1, y1, 0, 1, -1, -1);
            R.b[ni] = __builtin_shufflevector(y0, y1w, 0, 1, 2, 3, 4, 5, -1, -1);
        }
        R.sa = *reinterpret_cast<const __attribute__((address_space(3))) int*>(lds3 + base + sa_off + s * 4);
        R.sb = *reinterpret_cast<const __attribute__((address_space(3))) int*>(lds3 + base + sb_off + s * 4);
    };

    v16f acc[MPW][NPW];
#pragma unroll
    for (int i = 0; i < MPW; i++)
#pragma unroll
        for (int j = 0; j < NPW; j++) acc[i][j] = v16f{};

    // MFMA k of a slab: block (mi, ni) = (k % MPW, k / MPW); op_sel picks byte mi of the A
    // scale dword and byte ni of the B scale dword
    auto mfma_one = [&](const Slab& R, int k) {
        const int mi = k % MPW, ni = k / MPW;
        switch (mi * 4 + ni) {
#define MX_CASE(I, J) \
    case I * 4 + J: acc[I % MPW][J % NPW] = mfma_fp6<I, J>(acc[I % MPW][J % NPW], R.a[I % MPW], R.b[J % NPW], R.sa, R.sb); break;
            MX_CASE(0, 0) MX_CASE(0, 1) MX_CASE(0, 2) MX_CASE(0, 3)
            MX_CASE(1, 0) MX_CASE(1, 1) MX_CASE(1, 2) MX_CASE(1, 3)
            MX_CASE(2, 0) MX_CASE(2, 1) MX_CASE(2, 2) MX_CASE(2, 3)
            MX_CASE(3, 0) MX_CASE(3, 1) MX_CASE(3, 2) MX_CASE(3, 3)
#undef MX_CASE
        }
    };
    constexpr int NMF = MPW * NPW;
    auto mfma_slab = [&](const Slab& R) {
#pragma unroll
        for (int k = 0; k < NMF; k++) mfma_one(R, k);
    };

    Slab R0, R1, R2;
    // K-tile i from stage i%2; NEXT: K-tile i+1 follows (barrier + slab 0 read); DMA2: K-tile
    // i+2 exists and is copied into this stage once every wave is done with it.
    auto ktile = [&](int i, auto next_tag, auto dma2_tag) {
        constexpr bool NEXT = decltype(next_tag)::value, DMA2 = decltype(dma2_tag)::value;
        const int st = i & 1;
        // phase boundaries are scheduling barriers: each phase's LDS reads overlap the
        // previous slab's MFMAs, and no MFMA drifts across the stage barrier
        read_slab(st, 1, R1);
        mfma_slab(R0);
        __builtin_amdgcn_sched_barrier(0);
        read_slab(st, 2, R2);
        mfma_slab(R1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NEXT) {
            wait_vmcnt0();    // this wave's copy of K-tile i+1 has landed
            __syncthreads();  // every wave's copy landed; every wave finished reading stage st
            read_slab(st ^ 1, 0, R0);
            if constexpr (DMA2) {
                // the copy of K-tile i+2 into this stage, spread over the slab's MFMAs
                constexpr int PER = (N_DMA + NMF - 1) / NMF;
#pragma unroll
                for (int k = 0; k < NMF; k++) {
                    mfma_one(R2, k);
#pragma unroll
                    for (int j = k * PER; j < (k + 1) * PER && j < N_DMA; j++)
                        dma_op(j, kt0 + i + 2, st);
                    __builtin_amdgcn_sched_barrier(0);
                }
                return;
            }
        }
        mfma_slab(R2);
        __builtin_amdgcn_sched_barrier(0);
    };
    using T = std::true_type;
    using F = std::false_type;

    // prologue: K-tile 0 resident, K-tile 1 in flight, slab 0 of K-tile 0 in registers
    issue_tile(kt0, 0);
    wait_vmcnt0();
    __syncthreads();
    if (nkt > 1) issue_tile(kt0 + 1, 1);
    read_slab(0, 0, R0);
    int i = 0;
    for (; i + 2 < nkt; i++) ktile(i, T{}, T{});
    if (i + 1 < nkt) ktile(i++, T{}, F{});
    ktile(i, F{}, F{});

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

// (MT, NT, MPW, NPW) -> wave grid: the scale grouping fixes how many 32-blocks one wave holds,
// so it also selects between the 4-wave and 8-wave instantiation of a tile.
inline bool tile_supported(int MT, int NT, int mpw, int npw) {
    return (MT == 128 && NT == 128 && mpw == 2 && npw == 2) ||
           (MT == 128 && NT == 256 && mpw == 2 && npw == 4) ||
           (MT == 128 && NT == 384 && mpw == 4 && npw == 3) ||
           (MT == 256 && NT == 256 && mpw == 4 && npw == 4) ||
           (MT == 256 && NT == 256 && mpw == 2 && npw == 4);
}

template <int MT, int NT, int WM, int WN, int XG, typename OutT>
int tile_launch_t(const mxfp6_launch_desc* d, hipStream_t st) {
    const dim3 grid((unsigned)(d->M / MT), (unsigned)(d->N / NT), (unsigned)d->splits);
    const dim3 block(64 * WM * WN);
    const uint8_t* A = static_cast<const uint8_t*>(d->A);
    const uint8_t* B = static_cast<const uint8_t*>(d->Bsh);
    if (d->splits > 1)
        tile_kernel<MT, NT, WM, WN, XG, float, true><<<grid, block, 0, st>>>(
            A, B, d->sA, d->sB, nullptr, d->ws, d->M, d->N, d->Kp, d->A_row_bytes, d->splits);
    else
        tile_kernel<MT, NT, WM, WN, XG, OutT, false><<<grid, block, 0, st>>>(
            A, B, d->sA, d->sB, static_cast<OutT*>(d->D), nullptr, d->M, d->N, d->Kp,
            d->A_row_bytes, 1);
    return 0;
}

template <typename OutT>
int tile_launch(const mxfp6_launch_desc* d, hipStream_t st) {
    if (!tile_supported(d->MT, d->NT, d->mpw, d->npw)) return 1;
    if (d->MT == 128 && d->NT == 128) return tile_launch_t<128, 128, 2, 2, 4, OutT>(d, st);
    if (d->MT == 128 && d->NT == 256) return tile_launch_t<128, 256, 2, 2, 4, OutT>(d, st);
    if (d->MT == 128 && d->NT == 384) return tile_launch_t<128, 384, 1, 4, 4, OutT>(d, st);
    if (d->mpw == 2) return tile_launch_t<256, 256, 4, 2, 4, OutT>(d, st);
    return tile_launch_t<256, 256, 2, 2, 4, OutT>(d, st);
}

}  // namespace mxfp6_dev
