// HIP launch layer: maps a host plan (mxfp6_launch_desc) onto kernel instantiations, grids and
// a stream. This file, the tile kernel's instantiation units (slab_*.hip) and the kernels they
// include are the only HIP code in the library.
#include <algorithm>
#include <atomic>

#include "../hip_layer.h"
#include "direct_kernel.hpp"
#include "prep_kernel.hpp"
#include "reduce_kernel.hpp"
#include "repack_kernel.hpp"
#include "slab_run.hpp"
#include "tiny_kernel.hpp"

using namespace mxfp6_dev;

namespace {

// Every launcher returns 0, 1 (no kernel for the descriptor) or 2 (a launch failed).
int status_of(hipError_t e) {
    return e == hipSuccess ? 0 : 2;
}

template <typename OutT>
int launch_reduce(const mxfp6_launch_desc* d, hipStream_t st) {
    const size_t total = (size_t)d->M * d->N;
    OutT* D = static_cast<OutT*>(d->D);
    if (total % 4 == 0)
        return status_of(launch_kernel(reduce_splitk_kernel<OutT, 4>,
                                       dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), st,
                                       d->ws, D, total, d->splits));
    return status_of(launch_kernel(reduce_splitk_kernel<OutT, 1>,
                                   dim3((unsigned)((total + 255) / 256)), dim3(256), st, d->ws, D,
                                   total, d->splits));
}

template <typename OutT>
int launch_direct(const mxfp6_launch_desc* d, hipStream_t st) {
    const dim3 grid((unsigned)(d->M / 64), (unsigned)(d->N / 64), (unsigned)d->splits);
    const uint8_t* A = static_cast<const uint8_t*>(d->A);
    const uint8_t* B = static_cast<const uint8_t*>(d->Bsh);
    if (d->splits > 1) {
        if (launch_kernel(direct_kernel<float, true>, grid, dim3(256), st, A, B, d->sA, d->sB,
                          nullptr, d->ws, d->M, d->N, d->Kp, d->A_row_bytes, d->mpw, d->npw,
                          d->splits) != hipSuccess)
            return 2;
        return launch_reduce<OutT>(d, st);
    }
    return status_of(launch_kernel(direct_kernel<OutT, false>, grid, dim3(256), st, A, B, d->sA,
                                   d->sB, static_cast<OutT*>(d->D), nullptr, d->M, d->N, d->Kp,
                                   d->A_row_bytes, d->mpw, d->npw, 1));
}

template <typename OutT>
int launch_typed(const mxfp6_launch_desc* d, hipStream_t st) {
    switch (d->kernel) {
        case MXFP6_KERNEL_DIRECT:
            return launch_direct<OutT>(d, st);
        case MXFP6_KERNEL_TILE: {
            // the 32 x 32 tile: K split over the workgroup's waves, reduced in LDS (no workspace)
            if (d->MT == 32 && d->NT == 32) return tiny_launch<OutT>(d, st);
            if (d->splits <= 1) return slab_run<OutT, false>(d, st);
            const int rc = slab_run<float, true>(d, st);
            return rc != 0 ? rc : launch_reduce<OutT>(d, st);
        }
        default:
            return 1;
    }
}

}  // namespace

extern "C" int mxfp6_hip_launch(const mxfp6_launch_desc* d) {
    hipStream_t st = static_cast<hipStream_t>(d->stream);
    int rc;
    switch (d->out_type) {
        case 0:
            rc = launch_typed<float>(d, st);
            break;
        case 1:
            rc = launch_typed<__half>(d, st);
            break;
        case 2:
            rc = launch_typed<__hip_bfloat16>(d, st);
            break;
        default:
            return 1;
    }
    return rc;
}

extern "C" int mxfp6_hip_repack(const void* src, int row_bytes, int rows, int Kp, void* dst,
                                void* stream) {
    return status_of(repack_rows_launch(static_cast<const uint8_t*>(src), row_bytes, rows, Kp / 64,
                                        static_cast<uint8_t*>(dst),
                                        static_cast<hipStream_t>(stream)));
}

// Clock sample: lane 0 of each one-wave workgroup stores the shader clock counter (s_memtime,
// counting at the XCD's current graphics clock), the 100 MHz reference counter (s_memrealtime),
// the XCD id and the hardware id (shader engine, shader array and CU in bits 8..15) of where it
// ran. The counters are read once per workgroup; the stores are ordinary vector stores.
__global__ void clock_sample_kernel(uint64_t* out) {
    const uint64_t cyc = __builtin_amdgcn_s_memtime();
    const uint64_t ref = __builtin_amdgcn_s_memrealtime();
    uint32_t xcc, hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    if (threadIdx.x == 0) {
        uint64_t* o = out + (size_t)blockIdx.x * 4;
        o[0] = cyc;
        o[1] = ref;
        o[2] = xcc;
        o[3] = hw;
    }
}

extern "C" int mxfp6_hip_clock_sample(uint64_t* out, int nwg, void* stream) {
    return status_of(launch_kernel(clock_sample_kernel, dim3((unsigned)nwg), dim3(64),
                                   static_cast<hipStream_t>(stream), out));
}

extern "C" int mxfp6_hip_time(int (*launch)(void* ctx), void* ctx, void* stream, int warm, int reps,
                              float* ms) {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    hipEvent_t a = nullptr, b = nullptr;
    if (hipEventCreate(&a) != hipSuccess) return 2;
    if (hipEventCreate(&b) != hipSuccess) {
        (void)hipEventDestroy(a);
        return 2;
    }
    int rc = 0;
    for (int i = 0; i < warm && rc == 0; i++) rc = launch(ctx);
    if (rc == 0 && hipEventRecord(a, st) != hipSuccess) rc = 2;
    for (int i = 0; i < reps && rc == 0; i++) rc = launch(ctx);
    if (rc == 0 && hipEventRecord(b, st) != hipSuccess) rc = 2;
    float t = 0.0f;
    if (rc == 0 && (hipEventSynchronize(b) != hipSuccess || hipEventElapsedTime(&t, a, b) != hipSuccess))
        rc = 2;
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    if (rc == 0) *ms = t / (float)(reps > 0 ? reps : 1);
    return rc;
}

extern "C" int mxfp6_hip_device_cus(void) {
    // per device: 0 = not read yet, -1 = the query failed
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev >= 64) dev = 63;
    int c = cus[dev].load(std::memory_order_relaxed);
    if (c == 0) {
        int v = 0;
        c = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
                ? v
                : -1;
        cus[dev].store(c, std::memory_order_relaxed);
    }
    return c > 0 ? c : 0;
}

extern "C" int mxfp6_hip_has_tile(int MT, int NT, int mpw, int npw) {
    return tile_supported(MT, NT, mpw, npw) ? 1 : 0;
}

// Rows of the tiled scale layout: dim rounded up to whole groups of 32 * group rows.
static int rows_in_groups(int dim, int group) {
    return (dim + 32 * group - 1) / (32 * group) * (32 * group);
}

extern "C" int mxfp6_hip_quantize_rows(const float* x, int rows, int cols, int nblk, void* packed,
                                       size_t row_bytes, int preshuffled, uint8_t* scales,
                                       int scale_mode, int ncols, int group, int Kp, void* stream) {
    // one wave per (row, 64 value blocks); the last chunk of a row also writes its K-tail blocks;
    // one block per lane: more, smaller one-wave workgroups beat 2 or 4 blocks per lane (8192^2:
    // 76 us against 100 and 163 us; the LDS per workgroup bounds the waves per CU)
    const int vblk = (cols + 31) / 32;
    const int chunks = (vblk + PREP_BLKS_PER_WAVE - 1) / PREP_BLKS_PER_WAVE;
    const int rows32 = (rows + 31) / 32 * 32;
    int rows_out = scale_mode ? rows_in_groups(rows, group) : rows;
    if (preshuffled) rows_out = std::max(rows_out, rows32);
    const PackedOut po{static_cast<uint8_t*>(packed), row_bytes, preshuffled ? Kp / 64 : 0, rows32};
    const ScaleOut so{scales, scale_mode, ncols, group, Kp / 192};
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool v4 = cols % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (preshuffled && scale_mode == 1) {
        // one whole output tile per wave (coalesced stores): 32-row blocks x 4 slabs per workgroup
        const dim3 g((unsigned)((Kp / 64 + PSH_SLABS - 1) / PSH_SLABS), (unsigned)(rows_out / 32));
        uint8_t* ash = static_cast<uint8_t*>(packed);
        return status_of(launch_kernel(v4 ? prep_rows_preshuffled_kernel<true>
                                          : prep_rows_preshuffled_kernel<false>,
                                       g, dim3(64 * PSH_SLABS), st, x, rows, cols, Kp / 64, ash,
                                       rows32, so));
    }
    const dim3 grid((unsigned)((size_t)rows_out * chunks));
    return status_of(launch_kernel(v4 ? prep_rows_kernel<true> : prep_rows_kernel<false>, grid,
                                   dim3(64), st, x, cols, nblk, po, so, chunks, rows));
}

extern "C" int mxfp6_hip_prepare_b(const float* B, int K, int N, int Kp, int group, void* bsh,
                                   uint8_t* tiled, void* stream) {
    const int NG = rows_in_groups(N, group);
    const unsigned nchunks = (unsigned)((NG + PREP_THREADS - 1) / PREP_THREADS), kchunks = (unsigned)(Kp / 32);
    return status_of(launch_kernel(prep_b_kernel, dim3(nchunks * kchunks), dim3(PREP_THREADS),
                                   static_cast<hipStream_t>(stream), B, K, N, NG, Kp, group,
                                   static_cast<uint8_t*>(bsh), tiled, (int)nchunks));
}

extern "C" int mxfp6_hip_tile_scales(const uint8_t* s, int dim, int vblk, int ld, int Kp,
                                     int group, uint8_t* tiled, void* stream) {
    const int dim_out = rows_in_groups(dim, group);
    const size_t total = (size_t)dim_out * (Kp / 32);
    const unsigned blocks = (unsigned)std::min<size_t>((total + PREP_THREADS - 1) / PREP_THREADS, 65536);
    return status_of(launch_kernel(tile_scales_kernel, dim3(blocks), dim3(PREP_THREADS),
                                   static_cast<hipStream_t>(stream), s, dim, dim_out, vblk, ld, Kp,
                                   group, tiled));
}
