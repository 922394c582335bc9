// Split-K second stage: D[i] = (OutT)(((0 + P[0][i]) + P[1][i]) + ... + P[S-1][i]) over the FP32
// partial layers P[s] = ws + s*total, in fixed segment order (bit-reproducible, and the same
// summation order as the reference's reduce_splitk, src/kernel.hpp:305-313).
// HBM-bound: reads S*total*4 bytes and writes total*sizeof(OutT) bytes. With VEC = 4 each thread
// handles 4 consecutive elements with 16-byte loads (total a multiple of 4); VEC = 1 (a ragged
// M x N) one element per thread. The loads of up to 8 segments are issued before their sums, so
// a thread waits for one memory latency per 8 segments rather than one per segment (the adds
// keep the segment order). The partials are read once, with nontemporal loads: cached, they
// would push the operands out of the Infinity Cache, which a following call on the same
// operands then reads from HBM again (2048 x 1024 x 105728, 8 segments, back to back: 162.6 ->
// 150.1 us per call; other split shapes within +-1%).
#pragma once
#include "device_common.hpp"

namespace mxfp6_dev {

template <typename OutT, int VEC>
__global__ void __launch_bounds__(256)
    reduce_splitk_kernel(const float* __restrict__ ws, OutT* __restrict__ D, size_t total, int S) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * VEC;
    if (i >= total) return;
    constexpr int BATCH = 8;
    if constexpr (VEC == 1) {
        float acc = 0.f;
        for (int s0 = 0; s0 < S; s0 += BATCH) {
            float p[BATCH];
#pragma unroll
            for (int j = 0; j < BATCH; j++)
                if (s0 + j < S) p[j] = __builtin_nontemporal_load(ws + (size_t)(s0 + j) * total + i);
#pragma unroll
            for (int j = 0; j < BATCH; j++)
                if (s0 + j < S) acc += p[j];
        }
        D[i] = cvt_out<OutT>(acc);
    } else {
        v4f acc = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < S; s0 += BATCH) {
            v4f p[BATCH];
#pragma unroll
            for (int j = 0; j < BATCH; j++)
                if (s0 + j < S)
                    p[j] = __builtin_nontemporal_load(
                        reinterpret_cast<const v4f*>(ws + (size_t)(s0 + j) * total + i));
#pragma unroll
            for (int j = 0; j < BATCH; j++)
                if (s0 + j < S) acc += p[j];
        }
        if constexpr (sizeof(OutT) == 4) {
            *reinterpret_cast<v4f*>(D + i) = acc;
        } else {
            OutT o[4] = {cvt_out<OutT>(acc.x), cvt_out<OutT>(acc.y), cvt_out<OutT>(acc.z),
                         cvt_out<OutT>(acc.w)};
            *reinterpret_cast<v2i*>(D + i) = *reinterpret_cast<const v2i*>(o);
        }
    }
}

}  // namespace mxfp6_dev
