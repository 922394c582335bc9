#pragma once
// Host-side quantisation and operand / scale layouts for mxfp6::gemm (header-only).
//
// Every function here keeps the name, signature and byte layout of the reference's
// include/mxfp6/preprocess.hpp (eeezio/mxfp6-gemm), because the layouts are part of the
// drop-in contract: a buffer prepared for the reference library is a valid input here.
// Indexing uses size_t throughout so multi-GiB operands do not overflow.
//
// Layout summary (k64 = one 64-element K slab, 32-block = 32 rows of A or columns of B):
//   preprocess_scale : out[(tile*(K/64) + k64)*64 + lane] = scales[tile*32 + lane%32][2*k64 + lane/32]
//   tile_scale       : out[(((g*k_tiles + kt)*64 + lane)*subs + sub)*group_pad + j]
//                        = ps[((g*group + j)*(K/64) + kt*subs + sub)*64 + lane],  zero for j >= group
//   preshuffle_B     : tile (nt, k64) of 1536 bytes at (nt*(K/64) + k64)*1536; lane t in 0..63 holds
//                      the 24 bytes of B^T row nt*32 + t%32 at K offset k64*64 + (t/32)*32:
//                      bytes 0..15 at 16*t, bytes 16..23 at 1024 + 8*t.
#include <algorithm>
#include <cassert>
#include <cmath>
#include <cstring>
#include <vector>

#include "mxfp6/gemm.hpp"  // K_TILE, kpad
#include "mxfp6/types.hpp"

namespace mxfp6 {

// ---- compact-A K padding (reference preprocess.hpp:12-38) ---------------------------------
// The kernel reads packed(Kp) bytes of every A row starting at row * A_row_bytes. With a compact
// A (A_row_bytes = packed(K)) the last row's read runs past the data by this many bytes, which
// the caller over-allocates (contents irrelevant: B's zero K-tail nulls them).
inline int a_compact_end_pad(int K) {
    return fp6_packed_bytes(kpad(K)) - fp6_packed_bytes(K);
}

// Scales [dim][K/32] -> [dim][kpad(K)/32]; the added blocks get code 127 (2^0), never NaN.
inline std::vector<uint8_t> pad_scales_k(const uint8_t* scales, int dim, int K) {
    const size_t sc = (size_t)(K / 32), scp = (size_t)(kpad(K) / 32);
    std::vector<uint8_t> out((size_t)dim * scp, (uint8_t)127);
    for (size_t r = 0; r < (size_t)dim; r++) std::memcpy(&out[r * scp], scales + r * sc, sc);
    return out;
}

// ---- quantisation (reference preprocess.hpp:40-118) -----------------------------------------

struct QuantizedMatrix {
    std::vector<uint8_t> packed_data;  // [rows][packed_row_bytes]
    std::vector<uint8_t> scales;       // [rows][scale_cols]
    int rows, cols;
    int packed_row_bytes;  // fp6_packed_bytes(cols)
    int scale_cols;        // cols / 32
};

// E8M0 code of the smallest power of two s with amax / s <= 7.5 (i.e. 2^ceil(log2(amax/7.5))),
// clamped to [0, 254]; an all-zero block gets 127.
inline uint8_t mx_block_scale_code(float amax) {
    if (amax == 0.0f) return 127;
    const float need = amax / 7.5f;
    int e;
    const float sig = std::frexp(need, &e);  // need = sig * 2^e, sig in [0.5, 1)
    if (sig == 0.5f) e -= 1;                 // exact power of two: 2^(e-1) == need suffices
    const int code = std::min(std::max(e + 127, 0), 254);
    return (uint8_t)code;
}

// Quantise a row-major float matrix [rows][cols] (cols % 32 == 0) block by block: per 32
// consecutive elements of a row, scale = mx_block_scale_code(max |x|), codes = E2M3(x / scale).
inline QuantizedMatrix quantize_to_mxfp6(const float* mat, int rows, int cols) {
    assert(cols % 32 == 0);
    QuantizedMatrix q;
    q.rows = rows;
    q.cols = cols;
    q.packed_row_bytes = fp6_packed_bytes(cols);
    q.scale_cols = cols / 32;
    q.packed_data.assign((size_t)rows * q.packed_row_bytes, 0);
    q.scales.assign((size_t)rows * q.scale_cols, 0);
    uint8_t codes[32];
    for (size_t r = 0; r < (size_t)rows; r++) {
        const float* row = mat + r * (size_t)cols;
        for (int blk = 0; blk < q.scale_cols; blk++) {
            const float* x = row + 32 * blk;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
            const uint8_t sc = mx_block_scale_code(amax);
            q.scales[r * q.scale_cols + blk] = sc;
            const float s = e8m0_to_float(sc);
            for (int i = 0; i < 32; i++) codes[i] = float_to_fp6_e2m3(x[i] / s);
            pack_fp6(codes, 32, &q.packed_data[r * q.packed_row_bytes + (size_t)24 * blk]);
        }
    }
    return q;
}

inline void dequantize_mxfp6(const QuantizedMatrix& q, float* out) {
    std::vector<uint8_t> codes((size_t)q.cols);
    for (size_t r = 0; r < (size_t)q.rows; r++) {
        unpack_fp6(&q.packed_data[r * q.packed_row_bytes], q.cols, codes.data());
        for (int c = 0; c < q.cols; c++)
            out[r * q.cols + c] =
                fp6_e2m3_to_float(codes[c]) * e8m0_to_float(q.scales[r * q.scale_cols + c / 32]);
    }
}

// B[K][N] (row-major) -> quantised B^T[N][K].
inline QuantizedMatrix preprocess_B(const float* B, int K, int N) {
    assert(K % 32 == 0);
    std::vector<float> bt((size_t)N * K);
    for (size_t k = 0; k < (size_t)K; k++)
        for (size_t n = 0; n < (size_t)N; n++) bt[n * K + k] = B[k * N + n];
    return quantize_to_mxfp6(bt.data(), N, K);
}

// ---- scale layout in MFMA lane order (reference preprocess.hpp:120-162) ---------------------

struct PreprocessedScale {
    std::vector<uint8_t> data;  // [num_tiles][k64_iters][64]
    int dim, K;
    int num_tiles;  // dim / 32
    int k64_iters;  // K / 64
};

inline PreprocessedScale preprocess_scale(const uint8_t* scales, int dim, int K) {
    assert(dim % 32 == 0 && K % 64 == 0);
    PreprocessedScale ps;
    ps.dim = dim;
    ps.K = K;
    ps.num_tiles = dim / 32;
    ps.k64_iters = K / 64;
    ps.data.resize((size_t)ps.num_tiles * ps.k64_iters * 64);
    const size_t sc = (size_t)(K / 32);
    size_t o = 0;
    for (size_t t = 0; t < (size_t)ps.num_tiles; t++)
        for (size_t k64 = 0; k64 < (size_t)ps.k64_iters; k64++)
            for (size_t lane = 0; lane < 64; lane++)
                ps.data[o++] = scales[(t * 32 + (lane & 31)) * sc + 2 * k64 + (lane >> 5)];
    return ps;
}

// ---- B preshuffle (reference preprocess.hpp:164-207) ---------------------------------------

struct PreshuffledB {
    std::vector<uint8_t> data;  // [n_tiles][k64_iters][1536]
    int N, K;
    int n_tiles;    // N / 32
    int k64_iters;  // K / 64
};

inline PreshuffledB preshuffle_B(const QuantizedMatrix& B_q) {
    assert(B_q.rows % 32 == 0 && B_q.cols % 64 == 0);
    PreshuffledB pb;
    pb.N = B_q.rows;
    pb.K = B_q.cols;
    pb.n_tiles = B_q.rows / 32;
    pb.k64_iters = B_q.cols / 64;
    pb.data.resize((size_t)pb.n_tiles * pb.k64_iters * 1536);
    for (size_t nt = 0; nt < (size_t)pb.n_tiles; nt++)
        for (size_t k64 = 0; k64 < (size_t)pb.k64_iters; k64++) {
            uint8_t* tile = &pb.data[(nt * pb.k64_iters + k64) * 1536];
            for (size_t t = 0; t < 64; t++) {
                const uint8_t* src = &B_q.packed_data[(nt * 32 + (t & 31)) * B_q.packed_row_bytes +
                                                      k64 * 48 + (t >> 5) * 24];
                std::memcpy(tile + 16 * t, src, 16);
                std::memcpy(tile + 1024 + 8 * t, src + 16, 8);
            }
        }
    return pb;
}

// ---- scale grouping per wave (reference preprocess.hpp:209-233) ---------------------------

struct TiledScale {
    std::vector<uint8_t> data;
};

inline TiledScale tile_scale(const PreprocessedScale& ps, int group, int subs) {
    const size_t gp = (size_t)((group + 3) / 4 * 4);
    const size_t k_tiles = (size_t)(ps.k64_iters / subs);
    const size_t ng = (size_t)(ps.num_tiles / group);
    TiledScale ts;
    ts.data.assign(ng * k_tiles * 64 * subs * gp, 0);
    for (size_t g = 0; g < ng; g++)
        for (size_t kt = 0; kt < k_tiles; kt++)
            for (size_t lane = 0; lane < 64; lane++)
                for (size_t sub = 0; sub < (size_t)subs; sub++) {
                    uint8_t* dst = &ts.data[(((g * k_tiles + kt) * 64 + lane) * subs + sub) * gp];
                    for (size_t j = 0; j < (size_t)group; j++)
                        dst[j] = ps.data[((g * group + j) * ps.k64_iters + kt * subs + sub) * 64 + lane];
                }
    return ts;
}

}  // namespace mxfp6
