// A caller of the reference's C++ API, written the way the reference's quick start uses it
// (README.md:144-196): host quantisation and layouts from include/mxfp6/preprocess.hpp,
// hipMalloc'ed operands, then choose_tile / gemm_workspace_size / gemm from include/mxfp6/gemm.hpp
// on the null stream. It is compiled against this repository's headers and linked with
// libmxfp6gemm.so only, so it shows that a reference caller relinks without source changes.
//
// D is compared with an FP64 dot of the dequantised operands over the nominal K, on every row of
// a small M and on 16 spread rows of a large one: |D - R| <= 1e-5 * sum|a b| (FP32 accumulation)
// plus one unit in the last place of the output format at |R| (FP16: 2^-10 |R|, BF16: 2^-7 |R|)
// plus the format's smallest subnormal step.
//
//   dropin_gemm M N K out_type(0 = F32, 1 = F16, 2 = BF16) [ws]   -> exit status 0 when D passes
//   ws: "ref" (default) allocates gemm_workspace_size() bytes, as a reference caller does;
//       "preferred" allocates mxfp6_gemm_preferred_workspace_size() bytes (include/mxfp6_gemm.h),
//       which also holds the repacked A on the shapes whose plan repacks.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "mxfp6/gemm.hpp"
#include "mxfp6/preprocess.hpp"
#include "mxfp6_gemm.h"
#include <cstring>

using namespace mxfp6;

#define HIP_OK(x)                                                                     \
    do {                                                                              \
        hipError_t e_ = (x);                                                          \
        if (e_ != hipSuccess) {                                                       \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));              \
            std::exit(2);                                                             \
        }                                                                             \
    } while (0)

// Deterministic test values: a 64-bit LCG, sums of uniforms (roughly normal), with per-row
// magnitudes spread over 2^-4 .. 2^4 so the E8M0 scales vary.
static std::vector<float> values(int rows, int cols, uint64_t seed) {
    std::vector<float> v((size_t)rows * cols);
    uint64_t s = seed * 6364136223846793005ULL + 1442695040888963407ULL;
    auto next = [&]() {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        return (double)(s >> 11) / 9007199254740992.0;
    };
    for (int r = 0; r < rows; r++) {
        const double mag = std::ldexp(1.0, (int)(next() * 9.0) - 4);
        for (int c = 0; c < cols; c++)
            v[(size_t)r * cols + c] = (float)(mag * (next() + next() + next() - 1.5));
    }
    return v;
}

static double out_value(const std::vector<uint8_t>& D, OutType ot, size_t i) {
    switch (ot) {
        case OutType::F32: return reinterpret_cast<const float*>(D.data())[i];
        case OutType::F16: return (double)__half2float(reinterpret_cast<const __half*>(D.data())[i]);
        default: return (double)__bfloat162float(reinterpret_cast<const __hip_bfloat16*>(D.data())[i]);
    }
}

int main(int argc, char** argv) {
    if (argc != 5 && argc != 6) {
        std::fprintf(stderr, "usage: %s M N K out_type [ref|preferred]\n", argv[0]);
        return 2;
    }
    const bool preferred_ws = argc == 6 && std::strcmp(argv[5], "preferred") == 0;
    const int M = std::atoi(argv[1]), N = std::atoi(argv[2]), K = std::atoi(argv[3]);
    const OutType ot = (OutType)std::atoi(argv[4]);
    const size_t ob = ot == OutType::F32 ? 4 : 2;

    const int Kp = kpad(K);
    const TileChoice tc = choose_tile(M, N, Kp);

    // 1. host quantisation: A compact over K, B over Kp with a zero K-tail
    const std::vector<float> A = values(M, K, 11);
    std::vector<float> B((size_t)Kp * N, 0.0f);
    {
        const std::vector<float> b = values(K, N, 22);
        std::copy(b.begin(), b.end(), B.begin());
    }
    const QuantizedMatrix Aq = quantize_to_mxfp6(A.data(), M, K);
    const QuantizedMatrix Bq = preprocess_B(B.data(), Kp, N);

    // 2. kernel layouts
    const PreshuffledB Bsh = preshuffle_B(Bq);
    const TiledScale sA = tile_scale(
        preprocess_scale(pad_scales_k(Aq.scales.data(), M, K).data(), M, Kp), tc.MPW, K_TILE / 64);
    const TiledScale sB = tile_scale(preprocess_scale(Bq.scales.data(), N, Kp), tc.NPW, K_TILE / 64);

    // 3. device buffers (A: compact rows + the end pad its last row's K-tail read needs)
    const size_t a_bytes = (size_t)M * Aq.packed_row_bytes + a_compact_end_pad(K);
    void *dA, *dBsh, *dD, *ws = nullptr;
    uint8_t *dsA, *dsB;
    HIP_OK(hipMalloc(&dA, a_bytes));
    HIP_OK(hipMemset(dA, 0, a_bytes));
    HIP_OK(hipMemcpy(dA, Aq.packed_data.data(), (size_t)M * Aq.packed_row_bytes, hipMemcpyHostToDevice));
    HIP_OK(hipMalloc(&dBsh, Bsh.data.size()));
    HIP_OK(hipMemcpy(dBsh, Bsh.data.data(), Bsh.data.size(), hipMemcpyHostToDevice));
    HIP_OK(hipMalloc(&dsA, sA.data.size()));
    HIP_OK(hipMemcpy(dsA, sA.data.data(), sA.data.size(), hipMemcpyHostToDevice));
    HIP_OK(hipMalloc(&dsB, sB.data.size()));
    HIP_OK(hipMemcpy(dsB, sB.data.data(), sB.data.size(), hipMemcpyHostToDevice));
    HIP_OK(hipMalloc(&dD, (size_t)M * N * ob));
    HIP_OK(hipMemset(dD, 0x5A, (size_t)M * N * ob));
    const size_t ws_bytes = preferred_ws ? mxfp6_gemm_preferred_workspace_size(M, N, Kp)
                                         : gemm_workspace_size(M, N, Kp);
    if (ws_bytes) HIP_OK(hipMalloc(&ws, ws_bytes));

    // 4. launch
    gemm(ot, M, N, Kp, dA, dBsh, dsA, dsB, dD, Aq.packed_row_bytes, Bq.packed_row_bytes, ws,
         ws_bytes);
    HIP_OK(hipDeviceSynchronize());
    std::vector<uint8_t> D((size_t)M * N * ob);
    HIP_OK(hipMemcpy(D.data(), dD, D.size(), hipMemcpyDeviceToHost));

    // FP64 reference of the dequantised operands over the nominal K
    std::vector<float> Ad((size_t)M * K), Bd((size_t)N * Kp);
    dequantize_mxfp6(Aq, Ad.data());
    dequantize_mxfp6(Bq, Bd.data());
    std::vector<int> rows;
    if (M <= 64) {
        for (int r = 0; r < M; r++) rows.push_back(r);
    } else {
        for (int i = 0; i < 16; i++) rows.push_back((int)((long)i * (M - 1) / 15));
    }
    const double ulp = ot == OutType::F32 ? 0.0 : ot == OutType::F16 ? std::ldexp(1.0, -10)
                                                                     : std::ldexp(1.0, -7);
    const double tiny = ot == OutType::F32 ? 0.0 : ot == OutType::F16 ? std::ldexp(1.0, -24)
                                                                      : std::ldexp(1.0, -133);
    long bad = 0;
    double worst = 0.0;
    for (int r : rows)
        for (int n = 0; n < N; n++) {
            double acc = 0.0, mag = 0.0;
            for (int k = 0; k < K; k++) {
                const double p = (double)Ad[(size_t)r * K + k] * (double)Bd[(size_t)n * Kp + k];
                acc += p;
                mag += std::fabs(p);
            }
            const double got = out_value(D, ot, (size_t)r * N + n);
            const double bound = 1e-5 * mag + ulp * std::fabs(acc) + tiny;
            const double err = std::fabs(got - acc);
            if (!(err <= bound)) bad++;
            if (bound > 0 && err / bound > worst) worst = err / bound;
        }
    std::printf("dropin_gemm %dx%dx%d out %d: tile %dx%d (%d,%d), workspace %zu B, %zu rows "
                "checked, worst error / bound %.3f, %ld failures\n",
                M, N, K, (int)ot, tc.MT, tc.NT, tc.MPW, tc.NPW, ws_bytes, rows.size(), worst, bad);
    HIP_OK(hipFree(dA));
    HIP_OK(hipFree(dBsh));
    HIP_OK(hipFree(dsA));
    HIP_OK(hipFree(dsB));
    HIP_OK(hipFree(dD));
    if (ws) HIP_OK(hipFree(ws));
    return bad == 0 ? 0 : 1;
}
