// C ABI of the host-side formats and layouts (include/mxfp6/types.hpp, preprocess.hpp) and the
// synthetic workload generator of the benchmarks. Plain C++17, no HIP.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "mxfp6/preprocess.hpp"
#include "mxfp6/types.hpp"
#include "mxfp6_gemm.h"

using namespace mxfp6;

namespace {

// Run fn(i) for i in [0, n) on up to nthreads threads (contiguous chunks).
template <class F>
void parallel_for(size_t n, int nthreads, F fn) {
    if (nthreads <= 0) nthreads = (int)std::max(1u, std::thread::hardware_concurrency());
    if ((size_t)nthreads > n) nthreads = (int)std::max<size_t>(1, n);
    if (nthreads == 1) {
        for (size_t i = 0; i < n; i++) fn(i);
        return;
    }
    std::vector<std::thread> pool;
    const size_t chunk = (n + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        const size_t b = t * chunk, e = std::min(n, b + chunk);
        if (b >= e) break;
        pool.emplace_back([=] {
            for (size_t i = b; i < e; i++) fn(i);
        });
    }
    for (auto& th : pool) th.join();
}

// PCG32 (M. E. O'Neill, "PCG: A Family of Simple Fast Space-Efficient Statistically Good
// Algorithms for Random Number Generation", 2014; pcg32_random_r / pcg32_srandom_r /
// pcg32_advance_r of the pcg-c-basic distribution): 64-bit LCG state, XSH-RR 32-bit output.
struct Pcg32 {
    static constexpr uint64_t MULT = 6364136223846793005ULL;
    uint64_t state = 0, inc = 1;

    Pcg32(uint64_t seed, uint64_t stream) {
        inc = (stream << 1) | 1u;
        next();
        state += seed;
        next();
    }
    uint32_t next() {
        const uint64_t old = state;
        state = old * MULT + inc;
        const uint32_t xs = (uint32_t)(((old >> 18) ^ old) >> 27);
        const uint32_t rot = (uint32_t)(old >> 59);
        return (xs >> rot) | (xs << ((32u - rot) & 31u));
    }
    // Jump ahead by delta steps: state <- MULT^delta * state + inc * (MULT^delta - 1)/(MULT - 1),
    // by binary decomposition of delta (Brown, "Random number generation with arbitrary
    // strides", 1994).
    void advance(uint64_t delta) {
        uint64_t cur_mult = MULT, cur_plus = inc, acc_mult = 1, acc_plus = 0;
        while (delta) {
            if (delta & 1) {
                acc_mult *= cur_mult;
                acc_plus = acc_plus * cur_mult + cur_plus;
            }
            cur_plus = (cur_mult + 1) * cur_plus;
            cur_mult *= cur_mult;
            delta >>= 1;
        }
        state = acc_mult * state + acc_plus;
    }
    // Uniform double in [0, 1) with 53 random bits from two draws.
    double uniform53() {
        const uint32_t a = next() >> 5, b = next() >> 6;
        return (a * 67108864.0 + b) * (1.0 / 9007199254740992.0);
    }
};

// Draws consumed per generated value.
int draws_per_value(int dist) {
    switch (dist) {
        case MXFP6_DIST_NORMAL: return 2;      // Box-Muller: 2 uniforms (4 draws) per 2 values
        case MXFP6_DIST_UNIFORM: return 2;     // 1 uniform
        case MXFP6_DIST_STUDENT_T3: return 8;  // 4 normals
        default: return -1;
    }
}

// Box-Muller: two independent N(0,1) from two uniforms.
inline void box_muller(Pcg32& g, double& z0, double& z1) {
    const double u1 = 1.0 - g.uniform53();  // (0, 1]
    const double u2 = g.uniform53();
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double th = 6.283185307179586476925286766559 * u2;
    z0 = r * std::cos(th);
    z1 = r * std::sin(th);
}

// Values of one row (K even) into out[0..K).
void gen_row(int K, int dist, double sigma, uint64_t seed, uint64_t stream, size_t row,
             float* out) {
    Pcg32 g(seed, stream);
    g.advance((uint64_t)row * (uint64_t)K * (uint64_t)draws_per_value(dist));
    if (dist == MXFP6_DIST_NORMAL) {
        for (int k = 0; k < K; k += 2) {
            double z0, z1;
            box_muller(g, z0, z1);
            out[k] = (float)(sigma * z0);
            out[k + 1] = (float)(sigma * z1);
        }
    } else if (dist == MXFP6_DIST_UNIFORM) {
        for (int k = 0; k < K; k++) out[k] = (float)(sigma * (2.0 * g.uniform53() - 1.0));
    } else {
        // Student-t, 3 degrees of freedom: Z / sqrt(chi2_3 / 3), chi2_3 = sum of 3 squared normals.
        for (int k = 0; k < K; k++) {
            double z, a, b, c;
            box_muller(g, z, a);
            box_muller(g, b, c);
            out[k] = (float)(sigma * z / std::sqrt((a * a + b * b + c * c) / 3.0));
        }
    }
}

// OCP MX scale of a block: E8M0 code of 2^(floor(log2 amax) - 2), clamped to [0, 254];
// an all-zero block -> 127.
inline uint8_t ocp_scale_code(float amax) {
    if (!(amax > 0.0f)) return 127;
    int e;
    std::frexp(amax, &e);  // amax = m * 2^e, m in [0.5, 1): floor(log2 amax) = e - 1
    const int code = (e - 1 - 2) + 127;
    return (uint8_t)std::min(std::max(code, 0), 254);
}

void quantize_row_ocp(const float* x, int K, uint8_t* packed, uint8_t* scales) {
    uint8_t codes[32];
    for (int blk = 0; blk < K / 32; blk++) {
        const float* v = x + 32 * blk;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(v[i]));
        const uint8_t sc = ocp_scale_code(amax);
        scales[blk] = sc;
        const int e = (int)sc - 127;
        for (int i = 0; i < 32; i++) codes[i] = float_to_fp6_e2m3(std::ldexp(v[i], -e));
        pack_fp6(codes, 32, packed + 24 * blk);
    }
}

}  // namespace

// ---- element formats ------------------------------------------------------------------------

extern "C" float mxfp6_fp6_e2m3_to_float(uint8_t code) {
    return fp6_e2m3_to_float(code);
}
extern "C" uint8_t mxfp6_float_to_fp6_e2m3(float v) {
    return float_to_fp6_e2m3(v);
}
extern "C" float mxfp6_e8m0_to_float(uint8_t code) {
    return e8m0_to_float(code);
}
extern "C" uint8_t mxfp6_float_to_e8m0(float v) {
    return float_to_e8m0(v);
}
extern "C" int mxfp6_pack_fp6(const uint8_t* vals, int n, uint8_t* packed) {
    if (!vals || !packed) return MXFP6_ERR_NULL;
    if (n < 0 || n % 4 != 0) return MXFP6_ERR_ARG;
    pack_fp6(vals, n, packed);
    return MXFP6_OK;
}
extern "C" int mxfp6_unpack_fp6(const uint8_t* packed, int n, uint8_t* vals) {
    if (!vals || !packed) return MXFP6_ERR_NULL;
    if (n < 0 || n % 4 != 0) return MXFP6_ERR_ARG;
    unpack_fp6(packed, n, vals);
    return MXFP6_OK;
}

// ---- layouts ----------------------------------------------------------------------------------

extern "C" int mxfp6_a_compact_end_pad(int K) {
    return a_compact_end_pad(K);
}

extern "C" int mxfp6_pad_scales_k(const uint8_t* scales, int dim, int K, uint8_t* out) {
    if (!scales || !out) return MXFP6_ERR_NULL;
    if (dim < 0 || K <= 0 || K % 32 != 0) return MXFP6_ERR_ARG;
    const std::vector<uint8_t> v = pad_scales_k(scales, dim, K);
    std::memcpy(out, v.data(), v.size());
    return MXFP6_OK;
}

extern "C" int mxfp6_quantize(const float* mat, int rows, int cols, uint8_t* packed,
                              uint8_t* scales) {
    if (!mat || !packed || !scales) return MXFP6_ERR_NULL;
    if (rows < 0 || cols <= 0 || cols % 32 != 0) return MXFP6_ERR_ARG;
    const QuantizedMatrix q = quantize_to_mxfp6(mat, rows, cols);
    std::memcpy(packed, q.packed_data.data(), q.packed_data.size());
    std::memcpy(scales, q.scales.data(), q.scales.size());
    return MXFP6_OK;
}

extern "C" int mxfp6_dequantize(const uint8_t* packed, const uint8_t* scales, int rows, int cols,
                                float* out) {
    if (!packed || !scales || !out) return MXFP6_ERR_NULL;
    if (rows < 0 || cols <= 0 || cols % 32 != 0) return MXFP6_ERR_ARG;
    QuantizedMatrix q;
    q.rows = rows;
    q.cols = cols;
    q.packed_row_bytes = fp6_packed_bytes(cols);
    q.scale_cols = cols / 32;
    q.packed_data.assign(packed, packed + (size_t)rows * q.packed_row_bytes);
    q.scales.assign(scales, scales + (size_t)rows * q.scale_cols);
    dequantize_mxfp6(q, out);
    return MXFP6_OK;
}

extern "C" int mxfp6_preprocess_b(const float* B, int K, int N, uint8_t* packed, uint8_t* scales) {
    if (!B || !packed || !scales) return MXFP6_ERR_NULL;
    if (N < 0 || K <= 0 || K % 32 != 0) return MXFP6_ERR_ARG;
    const QuantizedMatrix q = preprocess_B(B, K, N);
    std::memcpy(packed, q.packed_data.data(), q.packed_data.size());
    std::memcpy(scales, q.scales.data(), q.scales.size());
    return MXFP6_OK;
}

extern "C" int mxfp6_preprocess_scale(const uint8_t* scales, int dim, int K, uint8_t* out) {
    if (!scales || !out) return MXFP6_ERR_NULL;
    if (dim <= 0 || dim % 32 != 0 || K <= 0 || K % 64 != 0) return MXFP6_ERR_ARG;
    const PreprocessedScale ps = preprocess_scale(scales, dim, K);
    std::memcpy(out, ps.data.data(), ps.data.size());
    return MXFP6_OK;
}

extern "C" int mxfp6_preshuffle_b(const uint8_t* packed, int N, int K, int row_bytes,
                                  uint8_t* out) {
    if (!packed || !out) return MXFP6_ERR_NULL;
    if (N <= 0 || N % 32 != 0 || K <= 0 || K % 64 != 0 || row_bytes < K / 4 * 3)
        return MXFP6_ERR_ARG;
    return mxfp6_prepare_b(packed, N, K, (size_t)row_bytes, out, 1);
}

// The header's tile_scale keeps floor(dim / (32 * group)) whole groups and drops the rest; the
// C ABI accepts only groupings that divide dim / 32, so its buffer is exactly the layout the
// kernels read (mxfp6_tiled_scale_bytes sizes the zero-extended layout of any grouping).
static bool tile_scale_args_ok(int dim, int K, int group, int subs) {
    return dim > 0 && dim % 32 == 0 && K > 0 && K % 64 == 0 && group >= 1 && subs >= 1 &&
           (dim / 32) % group == 0;
}

extern "C" size_t mxfp6_tile_scale_bytes(int dim, int K, int group, int subs) {
    if (!tile_scale_args_ok(dim, K, group, subs)) return 0;
    const size_t gp = (size_t)((group + 3) / 4 * 4);
    return (size_t)(dim / 32 / group) * (size_t)(K / 64 / subs) * 64 * subs * gp;
}

extern "C" int mxfp6_tile_scale(const uint8_t* pscale, int dim, int K, int group, int subs,
                                uint8_t* out) {
    if (!pscale || !out) return MXFP6_ERR_NULL;
    if (!tile_scale_args_ok(dim, K, group, subs)) return MXFP6_ERR_ARG;
    PreprocessedScale ps;
    ps.dim = dim;
    ps.K = K;
    ps.num_tiles = dim / 32;
    ps.k64_iters = K / 64;
    ps.data.assign(pscale, pscale + (size_t)ps.num_tiles * ps.k64_iters * 64);
    const TiledScale ts = tile_scale(ps, group, subs);
    std::memcpy(out, ts.data.data(), ts.data.size());
    return MXFP6_OK;
}

// ---- synthetic operands ---------------------------------------------------------------------

extern "C" int mxfp6_gen_values(int rows, int K, int dist, double sigma, uint64_t seed,
                                uint64_t stream, float* out, int nthreads) {
    if (!out) return MXFP6_ERR_NULL;
    if (rows < 0 || K <= 0 || K % 32 != 0 || draws_per_value(dist) < 0) return MXFP6_ERR_ARG;
    parallel_for((size_t)rows, nthreads, [&](size_t r) {
        gen_row(K, dist, sigma, seed, stream, r, out + r * (size_t)K);
    });
    return MXFP6_OK;
}

extern "C" int mxfp6_gen_operand(int rows, int K, int dist, double sigma, uint64_t seed,
                                 uint64_t stream, uint8_t* packed, size_t row_bytes,
                                 uint8_t* scales, int scale_cols, int nthreads) {
    if (!packed || !scales) return MXFP6_ERR_NULL;
    if (rows < 0 || K <= 0 || K % 32 != 0 || draws_per_value(dist) < 0) return MXFP6_ERR_ARG;
    if (row_bytes < (size_t)(K / 4 * 3) || scale_cols < K / 32) return MXFP6_ERR_ARG;
    parallel_for((size_t)rows, nthreads, [&](size_t r) {
        std::vector<float> x((size_t)K);
        gen_row(K, dist, sigma, seed, stream, r, x.data());
        uint8_t* prow = packed + r * row_bytes;
        uint8_t* srow = scales + r * (size_t)scale_cols;
        quantize_row_ocp(x.data(), K, prow, srow);
        std::memset(prow + K / 4 * 3, 0, row_bytes - (size_t)(K / 4 * 3));
        std::memset(srow + K / 32, 127, (size_t)(scale_cols - K / 32));
    });
    return MXFP6_OK;
}

extern "C" int mxfp6_prepare_b(const uint8_t* packed, int N, int Kp, size_t b_row_bytes,
                               uint8_t* bsh, int nthreads) {
    if (!packed || !bsh) return MXFP6_ERR_NULL;
    if (N <= 0 || Kp <= 0 || Kp % 64 != 0 || b_row_bytes < (size_t)(Kp / 4 * 3))
        return MXFP6_ERR_ARG;
    const size_t k64n = (size_t)(Kp / 64);
    // ceil(N / 32) tiles; rows past N in the last one are zero codes
    parallel_for((size_t)((N + 31) / 32), nthreads, [&](size_t nt) {
        for (size_t q = 0; q < k64n; q++) {
            uint8_t* tile = bsh + (nt * k64n + q) * 1536;
            for (size_t t = 0; t < 64; t++) {
                const size_t n = nt * 32 + (t & 31);
                if (n >= (size_t)N) {
                    std::memset(tile + 16 * t, 0, 16);
                    std::memset(tile + 1024 + 8 * t, 0, 8);
                    continue;
                }
                const uint8_t* src = packed + n * b_row_bytes + q * 48 + (t >> 5) * 24;
                std::memcpy(tile + 16 * t, src, 16);
                std::memcpy(tile + 1024 + 8 * t, src + 16, 8);
            }
        }
    });
    return MXFP6_OK;
}

extern "C" int mxfp6_prepare_scales(const uint8_t* scales, int dim, int Kp, int group,
                                    uint8_t* tiled, int nthreads) {
    if (!scales || !tiled) return MXFP6_ERR_NULL;
    if (dim <= 0 || Kp <= 0 || Kp % 192 != 0 || group < 1 || group > 4) return MXFP6_ERR_ARG;
    const size_t sc = (size_t)(Kp / 32), k_tiles = (size_t)(Kp / 192), gp = 4;
    // ceil(dim / (32 * group)) groups; rows past dim are zero rows (code 127)
    parallel_for((size_t)((dim + 32 * group - 1) / (32 * group)), nthreads, [&](size_t g) {
        for (size_t kt = 0; kt < k_tiles; kt++)
            for (size_t lane = 0; lane < 64; lane++)
                for (size_t sub = 0; sub < 3; sub++) {
                    uint8_t* dst = tiled + (((g * k_tiles + kt) * 64 + lane) * 3 + sub) * gp;
                    for (size_t j = 0; j < gp; j++) {
                        if (j >= (size_t)group) {
                            dst[j] = 0;
                            continue;
                        }
                        const size_t row = (g * group + j) * 32 + (lane & 31);
                        dst[j] = row < (size_t)dim
                                     ? scales[row * sc + 2 * (kt * 3 + sub) + (lane >> 5)]
                                     : 127;
                    }
                }
    });
    return MXFP6_OK;
}
