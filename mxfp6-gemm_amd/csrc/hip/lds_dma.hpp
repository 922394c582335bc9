// gfx950 building blocks of the LDS-pipelined kernels: direct-to-LDS copies (global_load_lds),
// explicit vector-memory waits, opaque LDS offsets and the XCD-aware workgroup order.
//
// The copies are inline asm (M0 + global_load_lds in one statement) so the compiler sees neither an
// LDS store it could not tell apart from other stages' ds_reads (it would wait for every copy
// before every read) nor a pending vector load (its loop-merge waits would do the same); the
// kernels keep the vector-memory count themselves (s_waitcnt vmcnt).
#pragma once
#include <utility>

#include "device_common.hpp"

namespace mxfp6_dev {

constexpr int NXCD = 8;  // MI355X: 8 XCDs, workgroup id i runs on XCD i % 8

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

// dma16 into LDS lds + OFF: M0 is set from the scalar base plus the constant in one SALU
// instruction (a kernel's ring position is a compile-time constant).
template <int OFF>
__device__ __forceinline__ void dma16_at(uint32_t lds, const void* gbase, uint32_t voff) {
    if constexpr (OFF == 0)
        dma16(lds, gbase, voff);
    else
        asm volatile("s_add_u32 m0, %0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                     :
                     : "s"(lds), "v"(voff), "s"(gbase), "n"(OFF)
                     : "memory");
}

// 12 bytes per lane global -> LDS: lane l's bytes go to LDS m0 + OFF + 16*l (the instruction keeps a
// 16-byte LDS stride per lane; the last 4 bytes of each slot are not written).
template <int OFF>
__device__ __forceinline__ void dma12_at(uint32_t lds, const void* gbase, uint32_t voff) {
    if constexpr (OFF == 0)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx3 %1, %2"
                     :
                     : "s"(lds), "v"(voff), "s"(gbase)
                     : "memory");
    else
        asm volatile("s_add_u32 m0, %0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx3 %1, %2"
                     :
                     : "s"(lds), "v"(voff), "s"(gbase), "n"(OFF)
                     : "memory");
}

// Same with a per-lane 64-bit global address.
__device__ __forceinline__ void dma16_flat(uint32_t lds, const void* gaddr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds), "v"(gaddr)
                 : "memory");
}

// 4 bytes per lane global -> LDS: lane l's dword goes to LDS m0 + 4*l.
__device__ __forceinline__ void dma4_flat(uint32_t lds, const void* gaddr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
                 :
                 : "s"(lds), "v"(gaddr)
                 : "memory");
}

// f(std::integral_constant<int, I>) for I = 0 .. N-1, in order (a loop whose index is a
// compile-time constant in its body).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Buffer resource of a raw (untyped, unstrided) buffer at `base` with no effective bound: buffer
// loads through it take a VGPR offset, an SGPR offset and an immediate, with no 64-bit address
// arithmetic per load.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t raw_rsrc(const __attribute__((address_space(1))) uint8_t* base) {
    // dword 3: 32-bit data format (required for untyped loads on gfx9), no swizzle, no index
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, -1, 0x00020000);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier without the LDS fence of __syncthreads (which waits for every outstanding LDS
// read of the wave). The memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_barrier" ::: "memory"); }

typedef __attribute__((address_space(3))) const char* lds_cptr;

// Returns x unchanged, hidden from the optimizer (forces a VGPR, defeats offset folding).
__device__ __forceinline__ uint32_t opaque_v(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}

typedef __attribute__((address_space(1))) const uint8_t* gbl_cptr;

// Returns p as a global-memory pointer with its provenance hidden from the optimizer: loads through
// it are no longer known to read memory nothing writes, so they keep their order relative to asm
// statements with a memory clobber (and are not merged across them).
__device__ __forceinline__ gbl_cptr opaque_gptr(const uint8_t* p) {
    gbl_cptr g = (gbl_cptr)p;
    asm volatile("" : "+s"(g));
    return g;
}

__device__ __forceinline__ void wait_vmcnt0() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Position of workgroup pid in an XCD-major order of `total` workgroups: workgroups are dispatched
// to the XCDs round-robin (pid % NXCD), so XCD x receives the contiguous run of positions
// [x * per (+ remainder), ...) in dispatch order. A bijection of [0, total).
__device__ __forceinline__ int xcd_position(int total, int pid) {
    const int per = total / NXCD, rem = total % NXCD;
    const int x = pid % NXCD, j = pid / NXCD;
    return x < rem ? x * (per + 1) + j : rem * (per + 1) + (x - rem) * per + j;
}

// Tile of position L in the grouped order of a gm x gn tile grid: groups of XG tile rows, tile_m
// fastest inside a group.
__device__ __forceinline__ void grouped_tile(int gm, int gn, int XG, int L, int& tm, int& tn) {
    const int band = XG * gn;
    const int grp = L / band, rows = min(XG, gm - grp * XG), w = L - grp * band;
    tm = grp * XG + w % rows;
    tn = w / rows;
}

// Bijective map of the linear workgroup id onto (tile_m, tile_n) such that each XCD receives a
// contiguous run of the grouped order.
__device__ __forceinline__ void xcd_tile(int gm, int gn, int XG, int pid, int& tm, int& tn) {
    grouped_tile(gm, gn, XG, xcd_position(gm * gn, pid), tm, tn);
}

// Split-K variant: the S K segments of a gm x gn grid are laid end to end (segment-major) and
// each XCD receives a contiguous run of that order, so an XCD holds whole K segments (or a
// contiguous part of one) instead of a slice of every segment. pid counts over all S * gm * gn
// workgroups; z is the K segment.
__device__ __forceinline__ void xcd_split_tile(int gm, int gn, int S, int XG, int pid, int& tm,
                                               int& tn, int& z) {
    const int T = gm * gn, L = xcd_position(T * S, pid);
    z = L / T;
    grouped_tile(gm, gn, XG, L - z * T, tm, tn);
}

}  // namespace mxfp6_dev
