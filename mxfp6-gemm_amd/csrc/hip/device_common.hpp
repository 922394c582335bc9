// Device-side building blocks shared by the MXFP6 kernels (gfx950 / CDNA4 only).
#pragma once
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <tuple>

namespace mxfp6_dev {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v3i __attribute__((ext_vector_type(3)));
typedef float v16f __attribute__((ext_vector_type(16)));
// 24 bytes (one FP6 MFMA operand of a lane), 8-byte aligned
typedef int v6i_a8 __attribute__((__vector_size__(24), __aligned__(8)));
// 12 bytes, 4-byte aligned (one ds_read_b96)
typedef int v3i_a4 __attribute__((__vector_size__(12), __aligned__(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned v6u __attribute__((ext_vector_type(6)));

// Bytes of one packed 64-element K slab of a row (64 codes * 6 bits).
constexpr int SLAB_BYTES = 48;
// Bytes of one preshuffled 32x64 B tile and of one MFMA operand block (32 rows x 64 K).
constexpr int OPBLK_BYTES = 1536;
// K slabs (of 64) per scale K-tile: the scale layout groups 3 slabs (K_TILE = 192).
constexpr int SUBS = 3;

// D += A_blk * B_blk^T for one 32x32 output block over 64 K, FP6 E2M3 x FP6 E2M3 with per-lane
// E8M0 scales. a / b: lane l holds the 32 codes (24 bytes, 6 dwords) of row l%32 for K
// [32*(l/32), +32) of its operand block. Result layout: lane l holds column l%32 of the block,
// rows 8*g + 4*(l/32) + r in acc[4*g + r]. SA / SB select the scale byte inside sa / sb.
template <int SA, int SB>
__device__ __forceinline__ v16f mfma_fp6(v16f acc, v8i a, v8i b, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc, 2, 2, SA, sa, SB, sb);
}

// The lane's index in its wave (mbcnt over a full mask), computed afresh rather than kept live.
__device__ __forceinline__ int lane_id() {
    return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

template <typename OutT>
__device__ __forceinline__ OutT cvt_out(float v);
template <>
__device__ __forceinline__ float cvt_out<float>(float v) {
    return v;
}
template <>
__device__ __forceinline__ __half cvt_out<__half>(float v) {
    return __float2half_rn(v);
}
template <>
__device__ __forceinline__ __hip_bfloat16 cvt_out<__hip_bfloat16>(float v) {
    return __float2bfloat16(v);
}

// The 16 bits of an FP16 / BF16 value, zero-extended.
template <typename T>
__device__ __forceinline__ uint32_t half_bits(T h) {
    static_assert(sizeof(T) == 2, "16-bit type");
    return __builtin_bit_cast(uint16_t, h);
}

// Launches kernel k on stream st through hipLaunchKernel and returns that launch's own status, so
// an entry point's status neither reports nor clears an error left by an earlier runtime call of
// the caller's (as reading hipGetLastError after a <<<>>> launch would). The arguments are
// converted to the kernel's parameter types first.
template <typename... KArgs, typename... Args>
inline hipError_t launch_kernel(void (*k)(KArgs...), dim3 grid, dim3 block, hipStream_t st,
                                Args... args) {
    static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count");
    std::tuple<KArgs...> a(args...);
    return std::apply(
        [&](auto&... v) {
            void* p[] = {static_cast<void*>(&v)...};
            return hipLaunchKernel(reinterpret_cast<const void*>(k), grid, block, p, 0, st);
        },
        a);
}

// First K-tile and K-tile count of split segment z when k_tiles tiles are divided into S
// segments: the first k_tiles % S segments take one extra tile.
__device__ __forceinline__ void split_segment(int k_tiles, int S, int z, int& kt0, int& nkt) {
    const int base = k_tiles / S, rem = k_tiles % S;
    kt0 = z * base + (z < rem ? z : rem);
    nkt = base + (z < rem ? 1 : 0);
}

}  // namespace mxfp6_dev
