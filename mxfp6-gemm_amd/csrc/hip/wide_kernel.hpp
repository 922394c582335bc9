// Wide tile kernels of libmxfp6gemm for gfx950: four waves side by side, B straight into registers.
//
// A workgroup computes an MT x NT tile of D with MT = 32 MB and NT = 4 * 32 NPW; wave w owns all
// MT rows and columns [32 NPW w, 32 NPW (w + 1)) of the tile: MB x NPW blocks of 32x32, FP32
// accumulators in AGPRs, fed by v_mfma_scale_f32_32x32x64_f8f6f4 (FP6 E2M3 x FP6 E2M3 with per-lane
// E8M0 scales). Four shapes are built:
//   128 x 512 (MB 4, NPW 4), 128 x 384 (MB 4, NPW 3), 128 x 256 (MB 4, NPW 2) and 256 x 256 (MB 8,
//   NPW 2; A scales in two groups of four 32-row blocks).
// No B block is needed by two waves, so
//   B  streams straight from the preshuffled layout into the wave's MFMA operand registers: per
//      64-wide K slab and block, one 16-byte load (lane t: bytes 16t) and one 8-byte load (bytes
//      1024 + 8t) of the block's 1536-byte tile, each a contiguous piece of memory. The operands
//      sit in a ring of three register slots; slot s holds slab 3c + s of K-tile c, and the loads
//      of slab q + 3 are issued during slab q, a block's two loads right after the last MFMA that
//      reads the block. The scales (tiled layout: a lane's three slab dwords of a K-tile are
//      contiguous) come one K-tile ahead, one 12-byte load per scale group at the start of K-tile
//      c for K-tile c + 1, into registers moved to the current set when K-tile c ends.
//   A  (the MT rows, needed by every wave) is staged in LDS one K-tile at a time: a chunk holds,
//      per row, the K-tile's 144 contiguous bytes of the row-major operand (or, for A repacked
//      into the preshuffled layout, the K-tile's three 1536-byte tiles of each 32-row block),
//      MT x 144 bytes, copied with direct-to-LDS 16-byte loads (global_load_lds_dwordx4). A row's
//      144 bytes at a 16-byte offset span two 128-byte cache lines where a 64-wide slab copy of 48
//      bytes takes 1-2 per slab, so row-major A costs about half the L2 requests of a per-slab
//      copy. Chunks go through a ring of NB LDS buffers: chunk c + NB - 1 is copied during K-tile
//      c (the wave's copies spread over the K-tile's three slabs; a chunk of 128 rows is 18 wave
//      copies, two dummies keep the count per wave uniform), and a wave reads each slab's A
//      operand blocks during the previous slab into a register set: three sets (one per slab of a
//      K-tile) for MB 4, two alternating sets for MB 8. The K loop runs passes of six K-tiles, so
//      the chunk buffer (period 3), the A set and the scale set (period 2) of every step are
//      compile-time constants.
// One workgroup barrier per K-tile, at the start of its last slab: before it, each wave waits for
// its own copies of the next chunk (vmcnt, exact: the issue order is static) and for its LDS reads
// (lgkmcnt(0)); after it the next chunk is complete for every wave and the chunk read before the
// current one is free for the copies of K-tile c + NB - 1. The B loads and scale loads are
// ordinary loads whose waits the compiler places before the MFMAs that use them.
// Prefetches past the workgroup's last K-tile are clamped to that K-tile (valid addresses, data
// never used), so the K loop has no branch. A workgroup with a single K-tile, or a 128 x 256 one
// with up to three (K <= 576, or a split segment that short), takes a short path instead: every
// K-tile's chunk, scales and B operands (a register set per K-tile) are requested before the
// first MFMA, so no K-tile waits out a memory latency for B loads issued during the one before
// it, and no clamped prefetch is issued (128 x 512 runs segments of one or two K-tiles and
// 256 x 256 of one to three in instantiations of their own, ONE = 1, 2 or 3, unmasked only: with
// the path in their main kernel the masked and repacked-A instantiations would spill, and so
// would a masked ONE; three K-tiles of 128 x 512 would issue more loads up front than vmcnt
// counts). With every CU requesting its first K-tiles at once, the main loop's one-K-tile lead
// leaves each of the first K-tiles waiting on a loaded memory system; up front, the latencies
// overlap (256 x 256, three K-tiles: 8192 x 4096 x 512 42.1 us in the main loop).
// MASK (ragged M or N) clamps the copy and load sources
// of the last tile row and column and masks the stores, as in the slab kernel.
// SWZ (explicit plans only, never routed; row-major A, unmasked) stages a chunk row as twelve
// 12-byte units in 16-byte LDS slots (global_load_lds_dwordx3), the slots of row r permuted by
// XOR with (r / 4) % 4: a lane's 24-byte operand is then two 16-byte-aligned ds_read_b128 (four
// bytes of each unused), and the 16 lanes one LDS cycle serves read 16 distinct slot positions,
// so the operand reads are free of bank conflicts, for a third more copy instructions and a third
// more LDS per chunk (48 instead of 36 KiB at 256 rows).
#pragma once

#include <type_traits>

#include "../hip_layer.h"
#include "device_common.hpp"
#include "epilogue.hpp"
#include "lds_dma.hpp"

namespace mxfp6_dev {

// Static schedule of one wave in slab s (0..2) of a K-tile. In the order a step issues them:
// MFMA k; (s = 0, k = 0) the scale loads of the next K-tile; the slab's next A copy when k is a
// copy position; the two loads of B block k / MB when MFMA k was its last use in the slab
// (k % MB == MB - 1); the LDS read of an A block of the next slab when k is a read position.
template <int MB_, int NPW_, int NB_, bool SWZ_ = false>
struct WideGeom {
    static constexpr int MB = MB_, NPW = NPW_, NB = NB_;
    static constexpr bool SWZ = SWZ_;                            // 12-byte units, swizzled rows
    static constexpr int MT = 32 * MB, NT = 4 * 32 * NPW, NWAVES = 4, THREADS = 256;
    static constexpr int GA = MB < 4 ? MB : 4;                   // A scale group (blocks)
    static constexpr int NGA = MB / GA;                          // A scale groups per tile
    static constexpr int NMF = MB * NPW;                         // MFMAs per wave per slab
    static constexpr int NSET = MB <= 4 ? 3 : 2;                 // A operand register sets
    static constexpr int CHUNK = MT * SUBS * SLAB_BYTES;         // one K-tile of A
    // wave copies per chunk: of 1 KiB, or (SWZ) of 64 12-byte units, 12 per row
    static constexpr int COPIES = SWZ ? MT * 12 / 64 : CHUNK / 1024;
    static constexpr int A_ISS = (COPIES + NWAVES - 1) / NWAVES; // copies per wave per chunk
    // LDS buffer stride: room for every wave's A_ISS copies, so the copies that a chunk does
    // not need (128-row tiles: 18 real of 20) land in the buffer's own unread tail
    static constexpr int CST = A_ISS * NWAVES * 1024;
    static constexpr int LDS = NB * CST;
    // copies of slab s, and the MFMA after which copy j of a slab is issued
    static constexpr int cps(int s) { return A_ISS / SUBS + (s < A_ISS % SUBS ? 1 : 0); }
    static constexpr int CSTEP = cps(0) <= 2 ? NMF / 4 : NMF / cps(0);
    static constexpr int copy_k(int j) { return 1 + j * CSTEP; }
    static constexpr bool b_load_at(int k) { return k % MB == MB - 1; }
    // MFMA after which the read of A block i of the next slab is issued
    static constexpr int read_k(int i) { return NSET == 3 ? NMF / 2 + i : i * (NMF / MB); }
    static constexpr int ops_in_slab(int s) { return (s == 0 ? NGA + 1 : 0) + cps(s) + 2 * NPW; }
    static constexpr int ops_in_ktile() { return ops_in_slab(0) + ops_in_slab(1) + ops_in_slab(2); }
    static constexpr int b_ops_from(int k0) {
        int n = 0;
        for (int k = k0; k < NMF; k++) n += b_load_at(k) ? 2 : 0;
        return n;
    }
    // Before the barrier at the start of slab 2 of K-tile c, the wave's copies of chunk c + 1
    // (issued during K-tile c + 2 - NB, the last one in its slab 2) must have landed; issued
    // after that copy: the B loads of the rest of that slab, NB - 3 whole K-tiles, and slabs 0
    // and 1 of K-tile c.
    static constexpr int CHUNK_WAIT = b_ops_from(copy_k(cps(2) - 1)) + (NB - 3) * ops_in_ktile() +
                                      ops_in_slab(0) + ops_in_slab(1);
    // In the prologue: after chunk 0's copies, those of chunks 1 .. NB - 2, the scale loads of
    // K-tile 0 and the B loads of its three slabs.
    static constexpr int PRO_WAIT = (NB - 2) * A_ISS + NGA + 1 + SUBS * 2 * NPW;
    // One to three K-tiles (wide_kernel's short path): everything is loaded up front, K-tile by
    // K-tile its chunk, scales and B operands; the operations issued after chunk c's copies
    static constexpr int short_wait(int nk, int c) {
        return NGA + 1 + SUBS * 2 * NPW + (nk - 1 - c) * (A_ISS + NGA + 1 + SUBS * 2 * NPW);
    }
    // the short path holds a set of B operands per K-tile: up to three K-tiles on the 128 x 256
    // tile, one on 128 x 384; none on 128 x 512 and 256 x 256, whose masked and repacked-A
    // instantiations would then spill (the registers are allocated for the whole kernel)
    static constexpr int SHORT_MAX = MB == 4 && NPW == 2 ? 3 : MB == 4 && NPW == 3 ? 1 : 0;
    static_assert(MB == 4 || MB == 8, "128 or 256 rows");
    static_assert(NPW >= 1 && NPW <= 4, "B scale group holds <= 4 blocks");
    // NB = 3: the prologue issues chunk 1 before the loop, and the count above then holds for
    // it too (more loads follow chunk 1 in the prologue, the B loads of slabs 1 and 2, than
    // follow a chunk's last copy in the loop)
    static_assert(NB == 3, "three chunk buffers");
    static_assert(cps(0) + cps(1) + cps(2) == A_ISS && cps(2) >= 1, "copies per K-tile");
    static_assert(copy_k(cps(0) - 1) < NMF, "copy positions");
    static_assert(read_k(MB - 1) < NMF, "read positions");
    static_assert(CHUNK_WAIT <= 63 && PRO_WAIT <= 63, "vmcnt range");
    static_assert(short_wait(SHORT_MAX > 0 ? SHORT_MAX : 1, 0) <= 63, "vmcnt range (short path)");
};

// acc[mi][ni] += A(mi) * B(ni) with the scale bytes mi % 4 of sa and ni of sb (op_sel must be a
// constant: mi and ni are known at compile time wherever this is called from an unrolled loop).
template <int MB, int NPW>
__device__ __forceinline__ void wide_mfma(v16f (&acc)[MB][NPW], int mi, int ni, const v8i& a,
                                          const v8i& b, int sa, int sb) {
    switch (mi * 4 + ni) {
#define WX_CASE(I, J)                                                                   \
    case I * 4 + J:                                                                     \
        if constexpr (I < MB && J < NPW) acc[I][J] = mfma_fp6<I % 4, J>(acc[I][J], a, b, sa, sb); \
        break;
#define WX_ROW(I) WX_CASE(I, 0) WX_CASE(I, 1) WX_CASE(I, 2) WX_CASE(I, 3)
        WX_ROW(0) WX_ROW(1) WX_ROW(2) WX_ROW(3) WX_ROW(4) WX_ROW(5) WX_ROW(6) WX_ROW(7)
#undef WX_ROW
#undef WX_CASE
    }
}

template <int MB_, int NPW_, int NB_, int XG, typename OutT, bool SPLIT, bool ASH, bool MASK,
          bool STREAM, int ONE = 0, bool SWZ = false>
__global__ void __launch_bounds__(256, 1)
    wide_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ Bsh,
                const uint8_t* __restrict__ sA, const uint8_t* __restrict__ sB,
                OutT* __restrict__ D, float* __restrict__ ws, int M, int N, int Kp,
                int A_row_bytes, int S) {
    using G = WideGeom<MB_, NPW_, NB_, SWZ>;
    static_assert(!SWZ || (!ASH && !MASK && ONE == 0), "SWZ: row-major A, unmasked tiles");
    constexpr int MT = G::MT, NT = G::NT, MB = G::MB, NPW = G::NPW, NB = G::NB;
    constexpr int NGA = G::NGA, GA = G::GA, NSET = G::NSET, NMF = G::NMF;
    constexpr int CHUNK = G::CHUNK;
    __shared__ __attribute__((aligned(1024))) char lds[G::LDS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int wg_m = blockIdx.x, wg_n = blockIdx.y, wg_z = SPLIT ? (int)blockIdx.z : 0;
    if constexpr (XG > 0) {
        const int gm = (int)gridDim.x, gn = (int)gridDim.y;
        if (SPLIT && gm * gn <= 128)
            xcd_split_tile(gm, gn, S, XG,
                           (int)((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x),
                           wg_m, wg_n, wg_z);
        else if (!SPLIT || (gm * gn) % NXCD == 0)
            xcd_tile(gm, gn, XG, (int)(blockIdx.y * gridDim.x + blockIdx.x), wg_m, wg_n);
    }
    const int k64n = Kp / 64, k_tiles = Kp / 192;
    int kt0 = 0, nkt = k_tiles;
    if (SPLIT) split_segment(k_tiles, S, wg_z, kt0, nkt);
    const int kt_last = kt0 + nkt - 1;

    // ---- A chunk copies: copy i of this wave fills bytes [1024 j, 1024 j + 1024) of a chunk,
    // j = 4 i + wave; lane l's 16 bytes land at 1024 j + 16 l
    const int a_row_last = M - 1 - wg_m * MT;                     // MASK: last valid row
    const int a_blk_last = (M + 31) / 32 - 1 - wg_m * (MT / 32);  // MASK: last valid block
    const uint8_t* a_tile = ASH ? A + (size_t)wg_m * (MT / 32) * k64n * OPBLK_BYTES
                                : A + (size_t)wg_m * MT * A_row_bytes;
    uint32_t a_voff[G::A_ISS];
#pragma unroll
    for (int i = 0; i < G::A_ISS; i++) {
        const int j = i * G::NWAVES + wave;
        const int x = (j < G::COPIES ? j : 0) * 1024 + 16 * lane;  // dummies copy chunk byte 16 l
        if (ASH) {
            int blk = x / (SUBS * OPBLK_BYTES);
            const int rest = x - blk * (SUBS * OPBLK_BYTES);
            if (MASK) blk = min(blk, a_blk_last);
            a_voff[i] = (uint32_t)(blk * k64n * OPBLK_BYTES + rest);
        } else if (SWZ) {
            // LDS slot p = 64 j + l of the chunk holds unit u = v ^ ((r / 4) % 4) of row r = p / 12,
            // v = p % 12 (bytes 12 u of the row's K-tile)
            const int p = j * 64 + lane, row = p / 12;
            const int u = (p - row * 12) ^ ((row >> 2) & 3);
            a_voff[i] = (uint32_t)(row * A_row_bytes + 12 * u);
        } else {
            int row = x / (SUBS * SLAB_BYTES);
            const int col = x - row * (SUBS * SLAB_BYTES);
            if (MASK) row = min(row, a_row_last);
            a_voff[i] = (uint32_t)(row * A_row_bytes + col);
        }
    }
    const uint32_t lds0 = lds_u32(lds);
    // LDS destination of copy i in buffer 0 (scalar); buffer b adds b * CST in the copy itself
    uint32_t a_dst[G::A_ISS];
#pragma unroll
    for (int i = 0; i < G::A_ISS; i++)
        a_dst[i] = __builtin_amdgcn_readfirstlane(lds0 + (i * G::NWAVES + wave) * 1024);
    // copy i of chunk kt (absolute K-tile, clamped to the segment) into LDS buffer BUF
    auto a_copy = [&](int i, int kt, auto bufc) {
        constexpr int BUF = decltype(bufc)::value;
        const uint8_t* src = a_tile + (size_t)kt * (ASH ? SUBS * OPBLK_BYTES : SUBS * SLAB_BYTES);
        if constexpr (SWZ)
            dma12_at<BUF * G::CST>(a_dst[i], src, a_voff[i]);
        else
            dma16_at<BUF * G::CST>(a_dst[i], src, a_voff[i]);
    };

    // ---- B operand and scale loads of this wave
    const int b_blk_last = (N + 31) / 32 - 1;
    const int sa_grp_last = ((M + 31) / 32 + GA - 1) / GA - 1;
    const int sb_grp_last = ((N + 31) / 32 + NPW - 1) / NPW - 1;
    // The B operand and scale loads are buffer loads: a resource per B block column and per scale
    // group (base address in SGPRs), the lane's part as a constant VGPR offset, the K-tile as a
    // scalar offset and the slab as the instruction's immediate, so a load needs no address
    // arithmetic of its own. The bases are hidden from the optimizer (opaque_gptr): the loads then
    // keep their order relative to the asm copies and are not merged across them.
    rsrc_t b_rs[NPW];
#pragma unroll
    for (int ni = 0; ni < NPW; ni++) {
        int blk = wg_n * (NT / 32) + wave * NPW + ni;
        if (MASK) blk = min(blk, b_blk_last);
        b_rs[ni] = raw_rsrc(opaque_gptr(Bsh + (size_t)blk * k64n * OPBLK_BYTES));
    }
    // the lane's scale dwords of a K-tile (the dword of slab s at + 4 s), per A group and for B
    rsrc_t sa_rs[NGA];
#pragma unroll
    for (int g = 0; g < NGA; g++) {
        int ga = wg_m * NGA + g;
        if (MASK) ga = min(ga, sa_grp_last);
        sa_rs[g] = raw_rsrc(opaque_gptr(sA + (size_t)ga * k_tiles * 64 * 12));
    }
    int gb = wg_n * G::NWAVES + wave;
    if (MASK) gb = min(gb, sb_grp_last);
    const rsrc_t sb_rs = raw_rsrc(opaque_gptr(sB + (size_t)gb * k_tiles * 64 * 12));
    const int v_b0 = (int)opaque_v(16 * lane), v_b1 = (int)opaque_v(1024 + 8 * lane);
    const int v_sc = (int)opaque_v(12 * lane);

    // slab s of K-tile kt, block ni, into v
    auto load_b = [&](v8i& v, int ni, int kt, int s) {
        const int so = kt * (SUBS * OPBLK_BYTES);
        const v4i y0 = __builtin_bit_cast(
            v4i, __builtin_amdgcn_raw_buffer_load_b128(b_rs[ni], v_b0 + s * OPBLK_BYTES, so, 0));
        const v2i y1 = __builtin_bit_cast(
            v2i, __builtin_amdgcn_raw_buffer_load_b64(b_rs[ni], v_b1 + s * OPBLK_BYTES, so, 0));
        const v4i y1w = __builtin_shufflevector(y1, y1, 0, 1, -1, -1);
        v = __builtin_shufflevector(y0, y1w, 0, 1, 2, 3, 4, 5, -1, -1);
    };
    // the lane's three slab scale dwords of K-tile kt, for each A group and for B
    auto load_scales = [&](v3i (&a)[NGA], v3i& b, int kt) {
#pragma unroll
        for (int g = 0; g < NGA; g++)
            a[g] = __builtin_bit_cast(v3i, __builtin_amdgcn_raw_buffer_load_b96(sa_rs[g], v_sc, kt * 768, 0));
        b = __builtin_bit_cast(v3i, __builtin_amdgcn_raw_buffer_load_b96(sb_rs, v_sc, kt * 768, 0));
    };

    // ---- A operand reads (LDS): slab s of the chunk in buffer BUF, block mi. The addresses are
    // per-buffer (repacked A: two per buffer) or per-(buffer, block) (row-major A) base VGPRs
    // computed once, plus the slab's offset as the instructions' immediate: no address arithmetic
    // per read (a ds_read2_b64 reaches 2040 bytes past its base, a row-major block's three slabs
    // 96 + 16).
    const lds_cptr lds3 = (lds_cptr)lds;
    const uint32_t a_rd = ASH ? (uint32_t)(lane * 16)
                              : (uint32_t)((lane & 31) * SUBS * SLAB_BYTES + (lane >> 5) * 24);
    // (the masked instantiations hold clamp values besides: one base per buffer for row-major A,
    // and the block's offset added per read, so that they stay within the register file)
    // (SWZ: lane t reads units 4 s + 2 h and 4 s + 2 h + 1 of row t % 32 of the block, h = t / 32,
    // in slots 4 s + ((2 h + e) ^ q) of the row, e = 0, 1, q = ((t % 32) / 4) % 4: two bases per
    // buffer, the block's and slab's offsets as the reads' immediates)
    constexpr bool PER_BLOCK = !ASH && !MASK && !SWZ;
    constexpr int NBASE = ASH || SWZ ? 2 : PER_BLOCK ? MB : 1;
    const uint32_t q4 = ((lane & 31) >> 2) & 3, h2 = (lane >> 5) * 2;
    uint32_t a_base[NB][NBASE];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int i = 0; i < NBASE; i++)
            a_base[b][i] = ASH   ? opaque_v(b * G::CST + (i == 0 ? a_rd : 1024u + 8u * lane))
                           : SWZ ? opaque_v(b * G::CST + 192u * (lane & 31) + 16u * ((h2 + i) ^ q4))
                                 : opaque_v(b * G::CST + i * 32 * SUBS * SLAB_BYTES + a_rd);
    auto read_a = [&](v8i& dst, auto bufc, int s, int mi) {
        constexpr int BUF = decltype(bufc)::value;
        if constexpr (ASH) {
            const int o = (mi * SUBS + s) * OPBLK_BYTES;
            const v4i y0 = *reinterpret_cast<const __attribute__((address_space(3))) v4i*>(
                lds3 + a_base[BUF][0] + o);
            const v2i y1 = *reinterpret_cast<const __attribute__((address_space(3))) v2i*>(
                lds3 + a_base[BUF][1] + o);
            const v4i y1w = __builtin_shufflevector(y1, y1, 0, 1, -1, -1);
            dst = __builtin_shufflevector(y0, y1w, 0, 1, 2, 3, 4, 5, -1, -1);
        } else if constexpr (SWZ) {
            const int o = mi * 32 * 192 + s * 64;
            const v4i x0 = *reinterpret_cast<const __attribute__((address_space(3))) v4i*>(
                lds3 + a_base[BUF][0] + o);
            const v4i x1 = *reinterpret_cast<const __attribute__((address_space(3))) v4i*>(
                lds3 + a_base[BUF][1] + o);
            dst = __builtin_shufflevector(x0, x1, 0, 1, 2, 4, 5, 6, -1, -1);
        } else {
            const uint32_t o = PER_BLOCK ? a_base[BUF][PER_BLOCK ? mi : 0] + s * SLAB_BYTES
                                         : opaque_v(a_base[BUF][0] + mi * 32 * SUBS * SLAB_BYTES +
                                                    s * SLAB_BYTES);
            const v6i_a8 x = *reinterpret_cast<const __attribute__((address_space(3))) v6i_a8*>(lds3 + o);
            dst = __builtin_shufflevector(x, x, 0, 1, 2, 3, 4, 5, -1, -1);
        }
    };

    v16f acc[MB][NPW];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NPW; j++) acc[i][j] = v16f{};

    v8i RB[SUBS][NPW];        // B operands, slot s = slab s of a K-tile
    v8i RA[NSET][MB];         // A operands
    v3i sc_a[2][NGA], sc_b[2];  // scale dwords of K-tiles of even and of odd index

    if constexpr (G::SHORT_MAX > 0 || ONE > 0) {
        // One K-tile, or on the 128 x 256 tile up to three (K <= 576, or a split segment that
        // short): every K-tile's chunk, scales and B operands (a register set per K-tile) are
        // requested before the first MFMA, so no K-tile waits for loads issued during the one
        // before it; nothing is clamped, and the last K-tile needs no barrier. Chunk c goes to
        // LDS buffer c.
        auto short_path = [&](auto nk) {
            constexpr int NK = decltype(nk)::value;
            static_assert(G::short_wait(NK, 0) <= 63, "vmcnt range (short path)");
            v8i RBk[NK][SUBS][NPW];
            v3i ska[NK][NGA], skb[NK];
            static_for<NK>([&](auto cc) {
                constexpr int c = decltype(cc)::value;
#pragma unroll
                for (int i = 0; i < G::A_ISS; i++) a_copy(i, kt0 + c, cc);
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
                load_scales(ska[c], skb[c], kt0 + c);
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int s = 0; s < SUBS; s++)
#pragma unroll
                    for (int ni = 0; ni < NPW; ni++) {
                        load_b(RBk[c][s][ni], ni, kt0 + c, s);
                        asm volatile("" ::: "memory");
                        __builtin_amdgcn_sched_barrier(0);
                    }
            });
            wait_vmcnt<G::short_wait(NK, 0)>();  // chunk 0 landed
            ring_barrier();
#pragma unroll
            for (int mi = 0; mi < MB; mi++) read_a(RA[0][mi], std::integral_constant<int, 0>{}, 0, mi);
            // K-tile C from LDS buffer C; slab s uses A set s (three sets) or (3 C + s) % 2 (two)
            auto step = [&](auto cc) {
                constexpr int C = decltype(cc)::value;
                constexpr bool MORE = C + 1 < NK;
#pragma unroll
                for (int s = 0; s < SUBS; s++) {
                    if (MORE && s == SUBS - 1) {
                        // chunk C + 1 complete for every wave
                        wait_vmcnt<G::short_wait(NK, MORE ? C + 1 : 0)>();
                        ring_barrier();
                    }
                    const int cur = NSET == 3 ? s : (3 * C + s) % 2;
                    const int nxt = NSET == 3 ? (s + 1) % 3 : (3 * C + s + 1) % 2;
                    const int rs = s + 1 < SUBS ? s + 1 : 0;
#pragma unroll
                    for (int k = 0; k < NMF; k++) {
                        const int ni = k / MB, mi = k % MB;
                        const int g = mi / GA;
                        const int sa = s == 0 ? ska[C][g].x : s == 1 ? ska[C][g].y : ska[C][g].z;
                        const int sb = s == 0 ? skb[C].x : s == 1 ? skb[C].y : skb[C].z;
                        wide_mfma<MB, NPW>(acc, mi, ni, RA[cur][mi], RBk[C][s][ni], sa, sb);
#pragma unroll
                        for (int i = 0; i < MB; i++)
                            if (k == G::read_k(i) && (MORE || s + 1 < SUBS)) {
                                // slab s + 1 of chunk C, or slab 0 of chunk C + 1
                                if (s + 1 < SUBS)
                                    read_a(RA[nxt][i], cc, rs, i);
                                else if constexpr (MORE)
                                    read_a(RA[nxt][i], std::integral_constant<int, C + 1>{}, rs, i);
                            }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            };
            step(std::integral_constant<int, 0>{});
            if constexpr (NK >= 2) step(std::integral_constant<int, 1>{});
            if constexpr (NK == 3) step(std::integral_constant<int, 2>{});
            const int le = lane_id();  // recomputed: no lane value stays live across the K loop
            store_tile<MB, NPW, OutT, SPLIT, MASK, STREAM>(acc, D, ws, M, N,
                                                        wg_m * MT + 4 * (le >> 5),
                                                        wg_n * NT + wave * NPW * 32 + (le & 31),
                                                        le, wg_z);
        };
        if constexpr (ONE > 0) {
            // the instantiation for segments of ONE K-tiles of the tiles without the path in their
            // main kernel: nothing of the main loop is compiled in (the code below is unreachable)
            short_path(std::integral_constant<int, ONE>{});
            return;
        }
        if (nkt == 1) {
            short_path(std::integral_constant<int, 1>{});
            return;
        }
        if constexpr (G::SHORT_MAX >= 3) {
            if (nkt == 2) {
                short_path(std::integral_constant<int, 2>{});
                return;
            }
            if (nkt == 3) {
                short_path(std::integral_constant<int, 3>{});
                return;
            }
        }
    }

    // prologue: what the first MFMAs need first (chunk 0, the scales of K-tile 0, the B operands
    // of its slab 0), then chunks 1 .. NB-2 and the B operands of slabs 1 and 2 (the compiler,
    // which places the B waits, then sees at least the count of loads in flight on entry to the
    // loop that it sees around it; the empty asm statements keep it from merging or reordering the
    // loads). PRO_WAIT counts the same operations after chunk 0 in either order.
    using I0 = std::integral_constant<int, 0>;
#pragma unroll
    for (int i = 0; i < G::A_ISS; i++) a_copy(i, kt0, I0{});
    load_scales(sc_a[0], sc_b[0], kt0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < SUBS; s++) {
#pragma unroll
        for (int ni = 0; ni < NPW; ni++) {
            load_b(RB[s][ni], ni, kt0, s);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
        if (s == 0) {
            static_for<NB - 2>([&](auto cc) {
                constexpr int C = decltype(cc)::value + 1;
#pragma unroll
                for (int i = 0; i < G::A_ISS; i++)
                    a_copy(i, min(kt0 + C, kt_last), std::integral_constant<int, C>{});
            });
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    wait_vmcnt<G::PRO_WAIT>();  // chunk 0 landed
    ring_barrier();
#pragma unroll
    for (int mi = 0; mi < MB; mi++) read_a(RA[0][mi], I0{}, 0, mi);

    // K-tile c = T (mod 6) of the pass: chunk in LDS buffer BUF = T % NB, scales in set Q = T % 2
    // (the next K-tile's go to the other set), and with two A register sets slab s uses set
    // (3 Q + s) % 2 (with three, set s). Everything that rotates is a compile-time constant.
    auto ktile = [&](int c, auto tt) {
        constexpr int T = decltype(tt)::value;
        constexpr int BUF = T % NB, NBUF = (T + 1) % NB, CBUF = (T + NB - 1) % NB;
        constexpr int Q = T % 2;
        using BufC = std::integral_constant<int, BUF>;
        using NBufC = std::integral_constant<int, NBUF>;
        using CBufC = std::integral_constant<int, CBUF>;
        const int kt_copy = min(kt0 + c + NB - 1, kt_last);
        const int kt_next = min(kt0 + c + 1, kt_last);
#pragma unroll
        for (int s = 0; s < SUBS; s++) {
            if (s == SUBS - 1) {
                // chunk c + 1 complete for every wave before its first slab is read below; every
                // wave's reads of chunk c - 1 are complete, so its buffer may take chunk c + NB - 1
                wait_vmcnt<G::CHUNK_WAIT>();
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                ring_barrier();
            }
            const int cur = NSET == 3 ? s : (3 * Q + s) % 2;           // set of slab s
            const int nxt = NSET == 3 ? (s + 1) % 3 : (3 * Q + s + 1) % 2;  // of the next slab
            const int rs = s + 1 < SUBS ? s + 1 : 0;
            int ci = 0;  // copies of this slab so far
            const int c0 = s == 0 ? 0 : s == 1 ? G::cps(0) : G::cps(0) + G::cps(1);
#pragma unroll
            for (int k = 0; k < NMF; k++) {
                const int ni = k / MB, mi = k % MB;
                const int g = mi / GA;
                const int sa = s == 0 ? sc_a[Q][g].x : s == 1 ? sc_a[Q][g].y : sc_a[Q][g].z;
                const int sb = s == 0 ? sc_b[Q].x : s == 1 ? sc_b[Q].y : sc_b[Q].z;
                wide_mfma<MB, NPW>(acc, mi, ni, RA[cur][mi], RB[s][ni], sa, sb);
                if (s == 0 && k == 0) load_scales(sc_a[1 - Q], sc_b[1 - Q], kt_next);
                if (ci < G::cps(s) && k == G::copy_k(ci)) {
                    a_copy(c0 + ci, kt_copy, CBufC{});
                    ci++;
                }
                if (G::b_load_at(k)) load_b(RB[s][ni], ni, kt_next, s);
                // slab s + 1 of this K-tile, or slab 0 of the next, goes to RA[nxt]
#pragma unroll
                for (int i = 0; i < MB; i++)
                    if (k == G::read_k(i)) {
                        if (s + 1 < SUBS)
                            read_a(RA[nxt][i], BufC{}, rs, i);
                        else
                            read_a(RA[nxt][i], NBufC{}, rs, i);
                    }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    // passes of six K-tiles (the buffer rotates with period NB = 3, the sets with period 2); a
    // K loop of any length leaves after the K-tile that completes it
    int c = 0;
    bool done = false;
    while (!done) {
        static_for<6>([&](auto tt) {
            if (done) return;
            ktile(c, tt);
            done = ++c == nkt;
        });
    }

    // epilogue (the clamped prefetches of the last K-tiles are drained first); STREAM: D written
    // with nontemporal stores
    wait_vmcnt0();
    const int le = lane_id();  // recomputed: no lane value stays live across the K loop
    store_tile<MB, NPW, OutT, SPLIT, MASK, STREAM>(acc, D, ws, M, N, wg_m * MT + 4 * (le >> 5),
                                                wg_n * NT + wave * NPW * 32 + (le & 31), le,
                                                wg_z);
}

// One launch of a wide kernel (grid ceil(M/MT) x ceil(N/NT) x splits, 256 threads).
template <int MB, int NPW, int NB, int XG, typename KT, bool SPLIT, bool ASH, bool MASK,
          bool STREAM>
hipError_t wide_kernel_launch(const mxfp6_launch_desc* d, const uint8_t* A, hipStream_t st) {
    using G = WideGeom<MB, NPW, NB>;
    const dim3 grid((unsigned)((d->M + G::MT - 1) / G::MT), (unsigned)((d->N + G::NT - 1) / G::NT),
                    (unsigned)d->splits);
    if constexpr (!ASH && !MASK && !STREAM) {
        // row-major A staged swizzled (explicit plans): the main kernel for every segment length
        if (d->a_layout == MXFP6_A_ROWS_SWIZZLED)
            return launch_kernel(wide_kernel<MB, NPW, NB, XG, KT, SPLIT, false, false, false, 0, true>,
                                 grid, dim3(G::THREADS), st, A,
                                 static_cast<const uint8_t*>(d->Bsh), d->sA, d->sB,
                                 SPLIT ? nullptr : static_cast<KT*>(d->D), SPLIT ? d->ws : nullptr,
                                 d->M, d->N, d->Kp, d->A_row_bytes, SPLIT ? d->splits : 1);
    }
    if constexpr (G::SHORT_MAX == 0 && !MASK) {
        // every K segment one to three K-tiles: the short-path instantiations (not for masked
        // tiles, whose instantiations of it would spill; three K-tiles on 256 x 256 only, where
        // the loads issued up front still fit the vmcnt range)
        if constexpr (G::short_wait(3, 0) <= 63)
            if (d->Kp / 192 == 3 * d->splits)
                return launch_kernel(wide_kernel<MB, NPW, NB, XG, KT, SPLIT, ASH, MASK, STREAM, 3>,
                                     grid, dim3(G::THREADS), st, A,
                                     static_cast<const uint8_t*>(d->Bsh), d->sA, d->sB,
                                     SPLIT ? nullptr : static_cast<KT*>(d->D),
                                     SPLIT ? d->ws : nullptr, d->M, d->N, d->Kp, d->A_row_bytes,
                                     SPLIT ? d->splits : 1);
        if (d->Kp / 192 == 2 * d->splits)
            return launch_kernel(wide_kernel<MB, NPW, NB, XG, KT, SPLIT, ASH, MASK, STREAM, 2>,
                                 grid, dim3(G::THREADS), st, A,
                                 static_cast<const uint8_t*>(d->Bsh), d->sA, d->sB,
                                 SPLIT ? nullptr : static_cast<KT*>(d->D), SPLIT ? d->ws : nullptr,
                                 d->M, d->N, d->Kp, d->A_row_bytes, SPLIT ? d->splits : 1);
        if (d->Kp / 192 == d->splits)
            return launch_kernel(wide_kernel<MB, NPW, NB, XG, KT, SPLIT, ASH, MASK, STREAM, 1>,
                                 grid, dim3(G::THREADS), st, A,
                                 static_cast<const uint8_t*>(d->Bsh), d->sA, d->sB,
                                 SPLIT ? nullptr : static_cast<KT*>(d->D), SPLIT ? d->ws : nullptr,
                                 d->M, d->N, d->Kp, d->A_row_bytes, SPLIT ? d->splits : 1);
    }
    return launch_kernel(wide_kernel<MB, NPW, NB, XG, KT, SPLIT, ASH, MASK, STREAM>, grid,
                         dim3(G::THREADS), st, A, static_cast<const uint8_t*>(d->Bsh), d->sA,
                         d->sB, SPLIT ? nullptr : static_cast<KT*>(d->D), SPLIT ? d->ws : nullptr,
                         d->M, d->N, d->Kp, d->A_row_bytes, SPLIT ? d->splits : 1);
}

}  // namespace mxfp6_dev
