// C entry points over the reference implementation (eeezio/mxfp6-gemm), compiled from the
// reference's own sources under /root/reference into oracle/_ref/. TEST INFRASTRUCTURE ONLY:
// the reference's header-only formats/layouts/CPU GEMM pin the oracle's restatement, its router
// pins the oracle's router, and its GPU library gives the cross-library parity check.
// This file holds no reference code; it only adapts calls to plain C signatures.
#include <cstring>
#include <vector>

#include "mxfp6/gemm.hpp"
#include "mxfp6/preprocess.hpp"
#include "mxfp6/types.hpp"
#include "reference.hpp"

namespace mxfp6 {
// Test-only symbol of the reference library (src/gemm.cpp:89-107), not in its header.
void gemm_force_tile(OutType ot, int M, int N, int Kp, TileChoice tc, const void* dA,
                     const void* dBsh, const uint8_t* dsA, const uint8_t* dsB, void* dD,
                     int A_row_bytes, int B_row_bytes);
}  // namespace mxfp6

using namespace mxfp6;

static QuantizedMatrix qm(const uint8_t* packed, const uint8_t* scales, int rows, int cols) {
    QuantizedMatrix q;
    q.rows = rows;
    q.cols = cols;
    q.packed_row_bytes = fp6_packed_bytes(cols);
    q.scale_cols = cols / 32;
    q.packed_data.assign(packed, packed + (size_t)rows * q.packed_row_bytes);
    q.scales.assign(scales, scales + (size_t)rows * q.scale_cols);
    return q;
}

extern "C" {
float ref_fp6_decode(uint8_t c) { return fp6_e2m3_to_float(c); }
uint8_t ref_fp6_encode(float v) { return float_to_fp6_e2m3(v); }
float ref_e8m0_decode(uint8_t c) { return e8m0_to_float(c); }
uint8_t ref_e8m0_encode(float v) { return float_to_e8m0(v); }
void ref_pack(const uint8_t* codes, int n, uint8_t* packed) { pack_fp6(codes, n, packed); }
void ref_unpack(const uint8_t* packed, int n, uint8_t* codes) { unpack_fp6(packed, n, codes); }
int ref_a_compact_end_pad(int K) { return a_compact_end_pad(K); }
int ref_kpad(int K) { return kpad(K); }

void ref_pad_scales_k(const uint8_t* scales, int dim, int K, uint8_t* out) {
    std::vector<uint8_t> v = pad_scales_k(scales, dim, K);
    std::memcpy(out, v.data(), v.size());
}
void ref_quantize(const float* mat, int rows, int cols, uint8_t* packed, uint8_t* scales) {
    QuantizedMatrix q = quantize_to_mxfp6(mat, rows, cols);
    std::memcpy(packed, q.packed_data.data(), q.packed_data.size());
    std::memcpy(scales, q.scales.data(), q.scales.size());
}
void ref_preprocess_b(const float* B, int K, int N, uint8_t* packed, uint8_t* scales) {
    QuantizedMatrix q = preprocess_B(B, K, N);
    std::memcpy(packed, q.packed_data.data(), q.packed_data.size());
    std::memcpy(scales, q.scales.data(), q.scales.size());
}
void ref_dequantize(const uint8_t* packed, const uint8_t* scales, int rows, int cols, float* out) {
    dequantize_mxfp6(qm(packed, scales, rows, cols), out);
}
void ref_preprocess_scale(const uint8_t* scales, int dim, int K, uint8_t* out) {
    PreprocessedScale ps = preprocess_scale(scales, dim, K);
    std::memcpy(out, ps.data.data(), ps.data.size());
}
size_t ref_tile_scale(const uint8_t* scales, int dim, int K, int group, int subs, uint8_t* out) {
    // tile_scale over preprocess_scale(scales[dim][K/32]); out may be NULL to query the size
    TiledScale ts = tile_scale(preprocess_scale(scales, dim, K), group, subs);
    if (out) std::memcpy(out, ts.data.data(), ts.data.size());
    return ts.data.size();
}
void ref_preshuffle_b(const uint8_t* packed, const uint8_t* scales, int N, int K, uint8_t* out) {
    PreshuffledB pb = preshuffle_B(qm(packed, scales, N, K));
    std::memcpy(out, pb.data.data(), pb.data.size());
}
// tests/reference.hpp:14-29 on A[M][K] and B^T[N][K] (dense packed rows of 3K/4 bytes)
void ref_gemm_cpu(const uint8_t* a_packed, const uint8_t* a_scales, const uint8_t* b_packed,
                  const uint8_t* b_scales, int M, int N, int K, float* D) {
    mxfp6_gemm_ref(qm(a_packed, a_scales, M, K), qm(b_packed, b_scales, N, K), D, M, K, N);
}

void ref_choose_tile(int M, int N, int Kp, int* t) {
    TileChoice tc = choose_tile(M, N, Kp);
    t[0] = tc.MT; t[1] = tc.NT; t[2] = tc.MPW; t[3] = tc.NPW;
}
size_t ref_gemm_workspace_size(int M, int N, int Kp) { return gemm_workspace_size(M, N, Kp); }
void ref_gemm(int ot, int M, int N, int Kp, const void* dA, const void* dBsh, const uint8_t* dsA,
              const uint8_t* dsB, void* dD, int A_row_bytes, int B_row_bytes, void* ws,
              size_t ws_bytes) {
    gemm((OutType)ot, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, B_row_bytes, ws, ws_bytes);
}
void ref_gemm_force_tile(int ot, int M, int N, int Kp, const int* t, const void* dA,
                         const void* dBsh, const uint8_t* dsA, const uint8_t* dsB, void* dD,
                         int A_row_bytes, int B_row_bytes) {
    gemm_force_tile((OutType)ot, M, N, Kp, TileChoice{t[0], t[1], t[2], t[3]}, dA, dBsh, dsA, dsB,
                    dD, A_row_bytes, B_row_bytes);
}
}
