// Epilogue shared by the tile kernels: a wave's MPW x NPW block of FP32 accumulators to D (FP32,
// FP16 or BF16, row-major, ld = N) or, for a split-K segment, to its FP32 partials ws[z][M][N].
// Lane l of block (mi, ni) holds column n_w + 32 ni and rows m_w + 32 mi + 8 g + r in
// acc[mi][ni][4 g + r], with m_w = (first row of the wave) + 4 (l / 32) and n_w = (first column of
// the wave) + l % 32. MASK stores only rows < M and columns < N. NT writes D with nontemporal
// stores (streamed past the caches, for plans whose D would evict the operands the tiles re-read).
#pragma once
#include "device_common.hpp"

namespace mxfp6_dev {

// *p = v, nontemporal when NT
template <bool NT, typename T>
__device__ __forceinline__ void store_out(T* p, T v) {
    if constexpr (!NT)
        *p = v;
    else if constexpr (sizeof(T) == 2)
        __builtin_nontemporal_store((uint16_t)half_bits(v), reinterpret_cast<uint16_t*>(p));
    else
        __builtin_nontemporal_store(v, p);
}

template <int MPW, int NPW, typename OutT, bool SPLIT, bool MASK, bool NT = false>
__device__ __forceinline__ void store_tile(const v16f (&acc)[MPW][NPW], OutT* __restrict__ D,
                                           float* __restrict__ ws, int M, int N, int m_w, int n_w,
                                           int lane, int wg_z) {
    if constexpr (!SPLIT && sizeof(OutT) == 2) {
        if (!MASK || (N & 1) == 0) {
            // 16-bit output in 4-byte stores: lanes 2k and 2k+1 (columns c, c+1) trade halves so
            // that the even lane holds rows +0 and +2 of both columns and the odd lane rows +1
            // and +3 (one quad_perm DPP move and three byte permutes per 4 values), halving the
            // store instructions. The conversions are the per-element ones of cvt_out.
            const bool odd = (lane & 1) != 0;
            const uint32_t sel_send = odd ? 0x05040100u : 0x07060302u;
            const uint32_t sel_a = odd ? 0x03020504u : 0x05040100u;
            const uint32_t sel_b = odd ? 0x03020706u : 0x07060100u;
            const int m_p = m_w + (lane & 1), n_p = n_w & ~1;
#pragma unroll
            for (int mi = 0; mi < MPW; mi++)
#pragma unroll
                for (int ni = 0; ni < NPW; ni++)
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const v16f& a = acc[mi][ni];
                        const uint32_t p01 = half_bits(cvt_out<OutT>(a[4 * g])) |
                                             (half_bits(cvt_out<OutT>(a[4 * g + 1])) << 16);
                        const uint32_t p23 = half_bits(cvt_out<OutT>(a[4 * g + 2])) |
                                             (half_bits(cvt_out<OutT>(a[4 * g + 3])) << 16);
                        const uint32_t send = __builtin_amdgcn_perm(p23, p01, sel_send);
                        const uint32_t recv = (uint32_t)__builtin_amdgcn_mov_dpp(
                            (int)send, 0xB1, 0xF, 0xF, false);  // quad_perm [1, 0, 3, 2]
                        const uint32_t oa = __builtin_amdgcn_perm(recv, p01, sel_a);
                        const uint32_t ob = __builtin_amdgcn_perm(recv, p23, sel_b);
                        const int m = m_p + mi * 32 + 8 * g, n = n_p + ni * 32;
                        if (MASK && n >= N) continue;  // n even and N even: n + 1 < N as well
                        uint32_t* d0 = reinterpret_cast<uint32_t*>(D + (size_t)m * N + n);
                        if (!MASK || m < M) store_out<NT>(d0, oa);
                        if (!MASK || m + 2 < M)
                            store_out<NT>(reinterpret_cast<uint32_t*>(D + (size_t)(m + 2) * N + n), ob);
                    }
            return;
        }
    }
#pragma unroll
    for (int mi = 0; mi < MPW; mi++)
#pragma unroll
        for (int ni = 0; ni < NPW; ni++)
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m_w + mi * 32 + 8 * g + r, n = n_w + ni * 32;
                    if (MASK && (m >= M || n >= N)) continue;
                    const size_t idx = (size_t)m * N + n;
                    if (SPLIT)
                        ws[(size_t)wg_z * M * N + idx] = acc[mi][ni][4 * g + r];
                    else
                        store_out<NT>(D + idx, cvt_out<OutT>(acc[mi][ni][4 * g + r]));
                }
}

}  // namespace mxfp6_dev
