// Tile kernel of libmxfp6gemm for gfx950: an LDS ring of 64-wide K slabs.
//
// One workgroup computes an MT x NT tile of D with WM x WN waves; wave (wm, wn) owns MPW x NPW
// 32x32 blocks, accumulated in FP32 AGPRs by v_mfma_scale_f32_32x32x64_f8f6f4 (FP6 E2M3 x FP6
// E2M3, per-lane E8M0 scales picked by op_sel). K is walked in slabs of 64 (48 packed bytes per
// row). The LDS ring holds NS slabs; a stage holds the slab's A operand blocks, its B blocks and
// the workgroup's scale dwords for the slab:
//   B  preshuffled (preshuffle_B): one 32x64 block is a contiguous 1536-byte tile already in MFMA
//      operand order (lane t: 16 bytes at 16t, 8 bytes at 1024 + 8t), copied verbatim and read
//      with linear ds_read_b128 + ds_read_b64 (conflict-free).
//   A  either repacked into the same preshuffled layout (ASH; the repack kernel runs first) and
//      then handled exactly like B, or row-major (A_row_bytes per row): each row's 48 bytes copied
//      in 16-byte chunks, lane l reading 24 bytes at row l%32, byte 24*(l/32) (ds_read_b64 x3,
//      two-way bank conflicts, and a copy touches ~30 cache lines per KiB instead of 8).
//   scales  the tiled-scale layout keeps lane l's three slab dwords of a K-tile together; one
//      4-byte LDS copy per scale group gathers the slab's dword of every lane.
// Copies are global_load_lds (direct to LDS). Per slab every wave issues the same D copy
// instructions (waves with nothing to copy in a partial instruction copy into a dummy LDS area
// instead of branching), spread over the slab's MFMAs, so that:
//   * the in-order issue of MFMAs never stalls behind a burst of copies or LDS reads;
//   * NS - 2 slabs are in flight ahead of the one being multiplied;
//   * a wave waits only for its own copies of the next slab: vmcnt((NS - 3) * D) is exact.
// Schedule of slab q (registers R[q%2] hold slab q, read during slab q-1):
//     wait (own copies of slab q+1) | barrier | MFMAs of slab q, interleaved with the copy of
//     slab q+NS-1 into stage (q-1)%NS and the reads of slab q+1 into R[(q+1)%2]
// The barrier certifies slab q+1 (every wave's copies landed) and frees stage (q-1)%NS: every
// wave has issued the MFMAs of slab q-1, so its reads of that stage have completed. The reads of
// slab q, issued during slab q-1, may still be in flight at the barrier; nothing waits for them
// before the MFMAs that use them. The steady-state loop body is branch-free; the last NS slabs
// run a tail step with runtime conditions.
// Workgroup order: with XG > 0 the linear workgroup id is remapped so the workgroups running at
// the same time on one XCD cover an XG-row band of output tiles (shared A and B lines in that
// XCD's L2). Split-K grids of at most 128 tiles of at least 128 x 256 instead give each XCD whole
// K segments (xcd_split_tile): with few large tiles per segment, a slice of every segment leaves
// an XCD's L2 serving many distinct A and B streams (measured at 2048 x 1024 x 105728, 8 segments:
// 214 -> 197 us). Epilogue: lane l of block (mi, ni) holds column l%32 and rows 8g + 4(l/32) + r;
// D row-major; with SPLIT, FP32 partials of K segment z go to ws[z][M][N].
// Ragged shapes (MASK: MT does not divide M or NT does not divide N): the grid is
// ceil(M/MT) x ceil(N/NT), and the operand layouts hold ceil(M/32) and ceil(N/32) 32-row blocks
// (scale groups: ceil over MPW / NPW blocks). The last tile row and column copy clamped sources
// (a block, row or scale group past the end reads the last one that exists), so every copy stays
// inside the operands; the epilogue stores only rows < M and columns < N. The clamping sits in
// the per-workgroup copy offsets, so the K loop is the same as for a dividing tile.
#pragma once

#include "../hip_layer.h"
#include "device_common.hpp"
#include "epilogue.hpp"
#include "lds_dma.hpp"
#include "repack_kernel.hpp"
#include "slab_run.hpp"
#include "wide_kernel.hpp"

namespace mxfp6_dev {

template <int MT, int NT, int WM, int WN, int NS>
struct SlabGeom {
    static constexpr int MPW = MT / 32 / WM, NPW = NT / 32 / WN;
    static constexpr int NWAVES = WM * WN, THREADS = 64 * NWAVES;
    static constexpr int A_BYTES = MT * SLAB_BYTES;           // A rows of one slab
    // the stage's A area rounded up to whole 1 KiB wave copies (a 32-row tile has 1.5 KiB; the
    // last wave's extra chunks land in the padding)
    static constexpr int A_STAGE = (A_BYTES + 1023) / 1024 * 1024;
    static constexpr int B_BYTES = NT / 32 * OPBLK_BYTES;      // B blocks of one slab
    static constexpr int SC_GROUPS = WM + WN;                  // scale groups of the workgroup
    static constexpr int SC_BYTES = SC_GROUPS * 256;           // one dword per lane per group
    static constexpr int STAGE = A_STAGE + B_BYTES + SC_BYTES;
    static constexpr int A_CHUNKS = A_BYTES / 16, B_CHUNKS = B_BYTES / 16;
    static constexpr int A_ISS = (A_STAGE / 16 + THREADS - 1) / THREADS;
    static constexpr int B_ISS = (B_CHUNKS + THREADS - 1) / THREADS;
    static constexpr int SC_ISS = (SC_GROUPS + NWAVES - 1) / NWAVES;
    static constexpr int D = A_ISS + B_ISS + SC_ISS;           // copy instructions per wave per slab
    static constexpr int LDS = NS * STAGE + 1024;              // + dummy sink
    static_assert(B_BYTES % 1024 == 0, "whole-wave chunks");
    static_assert(STAGE % 16 == 0, "16-byte aligned stages");
    static_assert(NS >= 4 && (NS - 2) * D <= 63, "vmcnt range");
};

template <int MT, int NT, int WM, int WN, int NS, int XG, typename OutT, bool SPLIT, bool ASH,
          bool MASK>
__global__ void __launch_bounds__(64 * WM * WN, 1)
    slab_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ Bsh,
                const uint8_t* __restrict__ sA, const uint8_t* __restrict__ sB,
                OutT* __restrict__ D, float* __restrict__ ws, int M, int N, int Kp,
                int A_row_bytes, int S) {
    using G = SlabGeom<MT, NT, WM, WN, NS>;
    constexpr int MPW = G::MPW, NPW = G::NPW, THREADS = G::THREADS, STAGE = G::STAGE;
    static_assert(G::NWAVES == 4 || G::NWAVES == 8, "4 or 8 waves per workgroup");
    static_assert(MPW >= 1 && MPW <= 4 && NPW >= 1 && NPW <= 4, "scale groups hold <= 4 blocks");
    static_assert(NS >= 3, "ring depth");
    __shared__ __attribute__((aligned(1024))) char lds[G::LDS];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WN, wn = wave % WN;
    int wg_m = blockIdx.x, wg_n = blockIdx.y, wg_z = SPLIT ? (int)blockIdx.z : 0;
    if constexpr (XG > 0) {
        const int gm = (int)gridDim.x, gn = (int)gridDim.y;
        if (SPLIT && MT * NT >= 128 * 256 && gm * gn <= 128)
            xcd_split_tile(gm, gn, S, XG, (int)((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x),
                           wg_m, wg_n, wg_z);
        else if (!SPLIT || (gm * gn) % NXCD == 0)
            xcd_tile(gm, gn, XG, (int)(blockIdx.y * gridDim.x + blockIdx.x), wg_m, wg_n);
    }
    const int k64n = Kp / 64, k_tiles = Kp / 192;
    int kt0 = 0, nkt = k_tiles;
    if (SPLIT) split_segment(k_tiles, S, wg_z, kt0, nkt);
    const int q0 = kt0 * 3, nq = nkt * 3;  // first slab and slab count of this workgroup

    const uint8_t* a_base = ASH ? A + (size_t)wg_m * (MT / 32) * k64n * OPBLK_BYTES
                                : A + (size_t)wg_m * MT * A_row_bytes;
    const uint8_t* b_base = Bsh + (size_t)wg_n * (NT / 32) * k64n * OPBLK_BYTES;
    // MASK: the last row / block / scale group of the operands that this tile may read (relative
    // to the tile's first); past them the copies repeat the last one (never stored)
    const int a_row_last = M - 1 - wg_m * MT;
    const int a_blk_last = (M + 31) / 32 - 1 - wg_m * (MT / 32);
    const int b_blk_last = (N + 31) / 32 - 1 - wg_n * (NT / 32);
    const int sa_grp_last = ((M + 31) / 32 + MPW - 1) / MPW - 1;
    const int sb_grp_last = ((N + 31) / 32 + NPW - 1) / NPW - 1;

    // per-thread copy sources (offsets from the slab's base, constant across slabs)
    uint32_t a_voff[G::A_ISS], b_voff[G::B_ISS];
#pragma unroll
    for (int i = 0; i < G::A_ISS; i++) {
        const int c = (i * THREADS + tid) % G::A_CHUNKS;
        if (ASH) {
            int blk = c / 96;
            const int r = c - blk * 96;
            if (MASK) blk = min(blk, a_blk_last);
            a_voff[i] = (uint32_t)(blk * k64n * OPBLK_BYTES + r * 16);
        } else {
            int row = c / 3;
            const int part = c - row * 3;
            if (MASK) row = min(row, a_row_last);
            a_voff[i] = (uint32_t)(row * A_row_bytes + part * 16);
        }
    }
#pragma unroll
    for (int i = 0; i < G::B_ISS; i++) {
        const int c = (i * THREADS + tid) % G::B_CHUNKS, b = c / 96, r = c - b * 96;
        const int blk = MASK ? min(b, b_blk_last) : b;
        b_voff[i] = (uint32_t)(blk * k64n * OPBLK_BYTES + r * 16);
    }
    // scale gather: wave w copies group i*NWAVES + w of [A groups | B groups]; lane l's dword of
    // slab q lives at ((g*k_tiles + q/3)*64 + l)*12 + 4*(q%3) of that group's tiled scales
    const uint8_t* sc_src[G::SC_ISS];
#pragma unroll
    for (int i = 0; i < G::SC_ISS; i++) {
        int grp = i * G::NWAVES + wave;
        if (grp >= G::SC_GROUPS) grp = G::SC_GROUPS - 1;  // dummy copy: valid source
        int g = grp < WM ? wg_m * WM + grp : wg_n * WN + (grp - WM);
        if (MASK) g = min(g, grp < WM ? sa_grp_last : sb_grp_last);
        sc_src[i] = (grp < WM ? sA : sB) + ((size_t)g * k_tiles * 64 + lane) * 12;
    }
    const uint32_t lds0 = lds_u32(lds);
    const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(lds0 + wave * 1024);
    const uint32_t lds_sc_wave = __builtin_amdgcn_readfirstlane(lds0 + G::A_STAGE + G::B_BYTES + wave * 256);
    const uint32_t lds_dummy = __builtin_amdgcn_readfirstlane(lds0 + NS * STAGE);
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);

    // copy instruction j (0 <= j < D) of global slab q into stage st
    auto dma_op = [&](int j, int q, int st) {
        const uint32_t so = st * STAGE;
        if (j < G::A_ISS) {
            const bool live = (G::A_STAGE / 16) % THREADS == 0 || j * THREADS + wave_u * 64 < G::A_STAGE / 16;
            dma16(live ? lds_wave + so + j * THREADS * 16 : lds_dummy,
                  a_base + (size_t)q * (ASH ? OPBLK_BYTES : SLAB_BYTES), a_voff[j]);
        } else if (j < G::A_ISS + G::B_ISS) {
            const int i = j - G::A_ISS;
            const bool live = G::B_CHUNKS % THREADS == 0 || i * THREADS + wave_u * 64 < G::B_CHUNKS;
            dma16(live ? lds_wave + so + G::A_STAGE + i * THREADS * 16 : lds_dummy,
                  b_base + (size_t)q * OPBLK_BYTES, b_voff[i]);
        } else {
            const int i = j - G::A_ISS - G::B_ISS;
            const bool live = i * G::NWAVES + wave_u < G::SC_GROUPS;
            dma4_flat(live ? lds_sc_wave + so + i * G::NWAVES * 256 : lds_dummy,
                      sc_src[i] + (size_t)(q / 3) * 768 + (q % 3) * 4);
        }
    };

    // Operand reads. Per slab every operand kind gets one base address (hidden from the compiler,
    // so it neither re-derives it per read nor fuses reads of different kinds); the blocks of a
    // kind are immediate offsets from it.
    const lds_cptr lds3 = (lds_cptr)lds;
    const int a_off = ASH ? wm * MPW * OPBLK_BYTES + lane * 16
                          : (wm * MPW * 32 + (lane & 31)) * SLAB_BYTES + (lane >> 5) * 24;
    const int b_off = G::A_STAGE + wn * NPW * OPBLK_BYTES + lane * 16;
    const int sa_off = G::A_STAGE + G::B_BYTES + wm * 256 + lane * 4;
    const int sb_off = G::A_STAGE + G::B_BYTES + (WM + wn) * 256 + lane * 4;
    struct Slab {
        v8i a[MPW], b[NPW];
        int sa, sb;
    };
    struct Bases {
        uint32_t a16, a8, b16, b8, sa, sb;
    };
    // the preshuffled blocks: lane t reads 16 bytes at 16t and 8 bytes at 1024 + 8t
    auto slab_bases = [&](uint32_t base) {
        Bases r;
        r.a16 = opaque_v(base + a_off);
        r.a8 = ASH ? opaque_v(base + a_off + 1024 - 8 * lane) : 0u;
        r.b16 = opaque_v(base + b_off);
        r.b8 = opaque_v(base + b_off + 1024 - 8 * lane);
        r.sa = opaque_v(base + sa_off);
        r.sb = opaque_v(base + sb_off);
        return r;
    };
    // Operand reads of one slab as items: item 0 = both scale dwords, then the A and B operands in
    // the order the slab's MFMAs first use them (MFMA k multiplies a[k % MPW] by b[k / MPW]).
    constexpr int ITEMS = 1 + MPW + NPW;
    auto read_item = [&](int item, const Bases& bs, Slab& R) {
        if (item == 0) {
            R.sa = *reinterpret_cast<const __attribute__((address_space(3))) int*>(lds3 + bs.sa);
            R.sb = *reinterpret_cast<const __attribute__((address_space(3))) int*>(lds3 + bs.sb);
            return;
        }
        // items: 1 = A0, 2 = B0, 3 .. MPW+1 = A1 .. A(MPW-1), MPW+2 .. = B1 .. B(NPW-1)
        int kind_b, idx;
        if (item == 1) {
            kind_b = 0, idx = 0;
        } else if (item == 2) {
            kind_b = 1, idx = 0;
        } else if (item < 2 + MPW) {
            kind_b = 0, idx = item - 2;
        } else {
            kind_b = 1, idx = item - 1 - MPW;
        }
        if (!kind_b && ASH) {
            const v4i y0 = *reinterpret_cast<const __attribute__((address_space(3))) v4i*>(lds3 + bs.a16 + idx * OPBLK_BYTES);
            const v2i y1 = *reinterpret_cast<const __attribute__((address_space(3))) v2i*>(lds3 + bs.a8 + idx * OPBLK_BYTES);
            const v4i y1w = __builtin_shufflevector(y1, y1, 0, 1, -1, -1);
            R.a[idx] = __builtin_shufflevector(y0, y1w, 0, 1, 2, 3, 4, 5, -1, -1);
        } else if (!kind_b) {
            const uint32_t o = opaque_v(bs.a16 + idx * 32 * SLAB_BYTES);
            const v6i_a8 x = *reinterpret_cast<const __attribute__((address_space(3))) v6i_a8*>(lds3 + o);
            R.a[idx] = __builtin_shufflevector(x, x, 0, 1, 2, 3, 4, 5, -1, -1);
        } else {
            const v4i y0 = *reinterpret_cast<const __attribute__((address_space(3))) v4i*>(lds3 + bs.b16 + idx * OPBLK_BYTES);
            const v2i y1 = *reinterpret_cast<const __attribute__((address_space(3))) v2i*>(lds3 + bs.b8 + idx * OPBLK_BYTES);
            const v4i y1w = __builtin_shufflevector(y1, y1, 0, 1, -1, -1);
            R.b[idx] = __builtin_shufflevector(y0, y1w, 0, 1, 2, 3, 4, 5, -1, -1);
        }
    };
    auto read_slab = [&](int st, Slab& R) {
        const Bases bs = slab_bases(st * STAGE);
#pragma unroll
        for (int i = 0; i < ITEMS; i++) read_item(i, bs, R);
    };

    v16f acc[MPW][NPW];
#pragma unroll
    for (int i = 0; i < MPW; i++)
#pragma unroll
        for (int j = 0; j < NPW; j++) acc[i][j] = v16f{};
    constexpr int NMF = MPW * NPW;
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

    Slab R0, R1;
    // Steady-state slab q: multiply Rc (slab q) while reading slab q+1 into Rn and copying slab
    // q+NS-1 into stage (q-1)%NS. Every wave has issued D copies per slab, so after the copies of
    // slab q+1 exactly NS-3 newer slabs are in flight: vmcnt((NS-3)*D) leaves only them pending.
    // Placement in the MFMA sequence: the copies spread over the first half of the slab's MFMAs
    // (copy j after MFMA j * (NMF/2) / D), the operand reads over the second half (item i after
    // MFMA NMF/2 + i * (NMF/2) / ITEMS). No wave issues a burst of LDS or vector-memory
    // instructions (with one wave per SIMD, a wave blocked on a full queue idles its MFMA unit),
    // and the copies' LDS writes and the operand reads do not compete for the LDS at the same time
    // (measured at 8192^3: 810 cycles per slab against 890 with both spread over the whole slab).
    auto slab_step = [&](int q, Slab& Rc, Slab& Rn) {
        const int st = (q + NS - 1) % NS;
        wait_vmcnt<(NS - 3) * G::D>();
        ring_barrier();  // slab q+1 landed for every wave; every wave is done reading stage st
        const uint32_t rbase = ((q + 1) % NS) * STAGE;
        Bases bs;
#pragma unroll
        for (int k = 0; k < NMF; k++) {
            mfma_one(Rc, k);
            if (k == NMF / 2) bs = slab_bases(rbase);
#pragma unroll
            for (int i = 0; i < ITEMS; i++)
                if (NMF / 2 + i * (NMF / 2) / ITEMS == k) read_item(i, bs, Rn);
#pragma unroll
            for (int j = 0; j < G::D; j++)
                if (j * (NMF / 2) / G::D == k) dma_op(j, q0 + q + NS - 1, st);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Tail slab q (the last NS slabs): the same with runtime conditions, full waits and the
    // remaining copies issued in one block.
    auto tail_step = [&](int q, Slab& Rc, Slab& Rn) {
        if (q + 1 < nq) {
            wait_vmcnt0();
            ring_barrier();
            read_slab((q + 1) % NS, Rn);
            if (q + NS - 1 < nq) {
#pragma unroll
                for (int j = 0; j < G::D; j++) dma_op(j, q0 + q + NS - 1, (q + NS - 1) % NS);
            }
        }
#pragma unroll
        for (int k = 0; k < NMF; k++) mfma_one(Rc, k);
    };

    // prologue: slabs 0..min(NS-1, nq)-1 in flight, slab 0 resident and read
    const int pro = nq < NS - 1 ? nq : NS - 1;
    for (int q = 0; q < pro; q++)
#pragma unroll
        for (int j = 0; j < G::D; j++) dma_op(j, q0 + q, q);
    if (pro == NS - 1)
        wait_vmcnt<(NS - 2) * G::D>();
    else
        wait_vmcnt0();
    ring_barrier();
    read_slab(0, R0);

    int q = 0;
    // two slabs per iteration keep the register roles static; the body is branch-free
    for (; q + NS < nq; q += 2) {
        slab_step(q, R0, R1);
        slab_step(q + 1, R1, R0);
    }
    for (; q < nq; q += 2) {
        tail_step(q, R0, R1);
        if (q + 1 < nq) tail_step(q + 1, R1, R0);
    }

    // epilogue
    wait_vmcnt0();
    store_tile<MPW, NPW, OutT, SPLIT, MASK>(acc, D, ws, M, N,
                                             wg_m * MT + wm * MPW * 32 + 4 * (lane >> 5),
                                             wg_n * NT + wn * NPW * 32 + (lane & 31), lane, wg_z);
}

// ---- launch ----------------------------------------------------------------------------------

// One launch of the tile kernel; KT is the kernel's output type (float for the split-K partials).
template <int MT, int NT, int WM, int WN, int XG, int NS, typename KT, bool SPLIT, bool ASH,
          bool MASK>
hipError_t slab_kernel_launch(const mxfp6_launch_desc* d, const uint8_t* A, hipStream_t st) {
    const dim3 grid((unsigned)((d->M + MT - 1) / MT), (unsigned)((d->N + NT - 1) / NT),
                    (unsigned)d->splits);
    return launch_kernel(slab_kernel<MT, NT, WM, WN, NS, XG, KT, SPLIT, ASH, MASK>, grid,
                         dim3(64 * WM * WN), st, A, static_cast<const uint8_t*>(d->Bsh), d->sA,
                         d->sB, SPLIT ? nullptr : static_cast<KT*>(d->D),
                         SPLIT ? d->ws : nullptr, d->M, d->N, d->Kp, d->A_row_bytes,
                         SPLIT ? d->splits : 1);
}

// Ring depth per tile: as many slabs as fit 160 KiB of LDS (128 x 128 and 32 x 128: half of it,
// two workgroups per CU). MASK when the tile does not divide M x N. Returns 0, or 2 when a launch
// fails.
template <int MT, int NT, int WM, int WN, int XG, int NS, typename KT, bool SPLIT>
int slab_launch_t(const mxfp6_launch_desc* d, hipStream_t st) {
    static_assert(SlabGeom<MT, NT, WM, WN, NS>::LDS <= 160 * 1024, "LDS budget");
    if (d->a_layout == MXFP6_A_ROWS_SWIZZLED) return 2;  // a staging of the wide tiles only
    const bool mask = d->M % MT != 0 || d->N % NT != 0;
    const uint8_t* A = static_cast<const uint8_t*>(d->A);
    if (d->a_layout == MXFP6_A_REPACK) {
        // repack A into the preshuffled layout, then run the kernel on it
        if (repack_rows_launch(A, d->A_row_bytes, d->M, d->Kp / 64, static_cast<uint8_t*>(d->Ash),
                               st) != hipSuccess)
            return 2;
        A = static_cast<const uint8_t*>(d->Ash);
    }
    hipError_t e;
    if (d->a_layout == MXFP6_A_ROWS) {
        if (mask)
            e = slab_kernel_launch<MT, NT, WM, WN, XG, NS, KT, SPLIT, false, true>(d, A, st);
        else
            e = slab_kernel_launch<MT, NT, WM, WN, XG, NS, KT, SPLIT, false, false>(d, A, st);
    } else {
        if (mask)
            e = slab_kernel_launch<MT, NT, WM, WN, XG, NS, KT, SPLIT, true, true>(d, A, st);
        else
            e = slab_kernel_launch<MT, NT, WM, WN, XG, NS, KT, SPLIT, true, false>(d, A, st);
    }
    return e == hipSuccess ? 0 : 2;
}

// The wide tiles (four waves side by side, B straight to registers): the A repack first when
// asked, MASK when the tile does not divide M x N. Three LDS chunk buffers; XCD groups of 8 tile
// rows for the 128-row tiles (4 buffers and groups of 4 or 16 rows measured within run-to-run
// noise on 8192^3, 2048x1024x105728 and 2048x6144x16128 for 128 x 512), 4 for 256 x 256.
constexpr int WIDE_NB = 3;
// an unsplit plan may write D with nontemporal stores (d->out_stream): its own instantiation, so
// that the kernels with plain stores keep a single epilogue
template <int MB, int NPW, int XG, typename KT, bool SPLIT, bool ASH, bool MASK>
hipError_t wide_launch_st(const mxfp6_launch_desc* d, const uint8_t* A, hipStream_t st) {
    if constexpr (!SPLIT) {
        if (d->out_stream)
            return wide_kernel_launch<MB, NPW, WIDE_NB, XG, KT, SPLIT, ASH, MASK, true>(d, A, st);
    }
    return wide_kernel_launch<MB, NPW, WIDE_NB, XG, KT, SPLIT, ASH, MASK, false>(d, A, st);
}

template <int MB, int NPW, int XG, typename KT, bool SPLIT>
int wide_launch_t(const mxfp6_launch_desc* d, hipStream_t st) {
    using G = WideGeom<MB, NPW, WIDE_NB>;
    static_assert(G::LDS <= 160 * 1024 && WideGeom<MB, NPW, WIDE_NB, true>::LDS <= 160 * 1024,
                  "LDS budget");
    const bool mask = d->M % G::MT != 0 || d->N % G::NT != 0;
    // the swizzled staging of row-major A: unmasked tiles, plain stores
    if (d->a_layout == MXFP6_A_ROWS_SWIZZLED && (mask || d->out_stream)) return 2;
    const uint8_t* A = static_cast<const uint8_t*>(d->A);
    if (d->a_layout == MXFP6_A_REPACK) {
        if (repack_rows_launch(A, d->A_row_bytes, d->M, d->Kp / 64, static_cast<uint8_t*>(d->Ash),
                               st) != hipSuccess)
            return 2;
        A = static_cast<const uint8_t*>(d->Ash);
    }
    hipError_t e;
    if (d->a_layout == MXFP6_A_ROWS || d->a_layout == MXFP6_A_ROWS_SWIZZLED)
        e = mask ? wide_launch_st<MB, NPW, XG, KT, SPLIT, false, true>(d, A, st)
                 : wide_launch_st<MB, NPW, XG, KT, SPLIT, false, false>(d, A, st);
    else
        e = mask ? wide_launch_st<MB, NPW, XG, KT, SPLIT, true, true>(d, A, st)
                 : wide_launch_st<MB, NPW, XG, KT, SPLIT, true, false>(d, A, st);
    return e == hipSuccess ? 0 : 2;
}

// Tile dispatch (declared in slab_run.hpp; instantiated once per (KT, SPLIT) in its own
// translation unit: slab_split.hip, slab_f32.hip, slab_f16.hip, slab_bf16.hip).
template <typename KT, bool SPLIT>
int slab_run(const mxfp6_launch_desc* d, hipStream_t st) {
    if (!tile_supported(d->MT, d->NT, d->mpw, d->npw)) return 1;
    // wide tiles: four waves side by side (TileChoice MPW 4 = the A scale group)
    if (d->MT == 128 && d->NT == 512) return wide_launch_t<4, 4, 8, KT, SPLIT>(d, st);
    if (d->MT == 128 && d->NT == 256 && d->mpw == 4) return wide_launch_t<4, 2, 8, KT, SPLIT>(d, st);
    if (d->MT == 256 && d->NT == 256 && d->npw == 2) return wide_launch_t<8, 2, 4, KT, SPLIT>(d, st);
    if (d->MT == 128 && d->NT == 384) return wide_launch_t<4, 3, 8, KT, SPLIT>(d, st);
    // skinny tiles: one wave row, four wave columns, a deeper ring
    if (d->MT == 32 && d->NT == 128) return slab_launch_t<32, 128, 1, 4, 4, 8, KT, SPLIT>(d, st);
    if (d->MT == 32 && d->NT == 256) return slab_launch_t<32, 256, 1, 4, 4, 8, KT, SPLIT>(d, st);
    if (d->MT == 64 && d->NT == 128) return slab_launch_t<64, 128, 1, 4, 4, 8, KT, SPLIT>(d, st);
    if (d->MT == 64 && d->NT == 256) return slab_launch_t<64, 256, 1, 4, 4, 8, KT, SPLIT>(d, st);
    if (d->MT == 128 && d->NT == 128) return slab_launch_t<128, 128, 2, 2, 4, 6, KT, SPLIT>(d, st);
    if (d->MT == 128 && d->NT == 256) return slab_launch_t<128, 256, 2, 2, 4, 8, KT, SPLIT>(d, st);
    if (d->MT == 256 && d->NT == 192) return slab_launch_t<256, 192, 2, 2, 4, 6, KT, SPLIT>(d, st);
    if (d->mpw == 2) return slab_launch_t<256, 256, 4, 2, 4, 6, KT, SPLIT>(d, st);
    return slab_launch_t<256, 256, 2, 2, 4, 6, KT, SPLIT>(d, st);
}

}  // namespace mxfp6_dev
