/* MXFP6 GEMM oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of the reference's (eeezio/mxfp6-gemm) formats, layouts, router and CPU
 * GEMM, used as the checker of libmxfp6gemm. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker or the CPU baseline;
 * the product never calls it.
 *
 * Each function names the reference file:line it restates and how it is pinned (the test in
 * tests/ that checks it against something other than itself). Status of every function:
 *   o_fp6_decode          types.hpp:13-24      pinned: OCP MX v1.0 E2M3 value table (golden fixture)
 *   o_fp6_encode          types.hpp:26-72      pinned: brute-force nearest search here + _ref encoder
 *   o_e8m0_decode         types.hpp:78-81      pinned: closed form 2^(u-127), 255 = NaN
 *   o_pack / o_unpack     types.hpp:97-123     pinned: bit-level KAT fixture + _ref packers
 *   o_quantize_ref        preprocess.hpp:51-97 pinned: _ref quantize_to_mxfp6 (byte-exact)
 *   o_quantize_ocp        BASELINE config rule pinned: brute force over exponents (tests)
 *   o_preprocess_scale    preprocess.hpp:136-162 pinned: _ref (byte-exact) + permutation checks
 *   o_tile_scale          preprocess.hpp:216-233 pinned: _ref (byte-exact)
 *   o_preshuffle_b        preprocess.hpp:182-207 pinned: _ref (byte-exact)
 *   o_choose_tile_ref     gemm.cpp:12-59       pinned: reference's 30-case table + _ref sweep
 *   o_splitk_s_ref        dispatch.hpp:30-59   pinned: _ref gemm_workspace_size sweep
 *   o_gemm_f64            reference.hpp:14-29 semantics in FP64; pinned: numpy float64 matmul,
 *                         _ref mxfp6_gemm_ref within FP32 error, closed-form cases
 *   o_gemm_f32_seq        reference.hpp:14-29 (FP32 sequential); pinned: _ref mxfp6_gemm_ref
 *                         bit-exact
 */
#ifndef MXFP6_ORACLE_H
#define MXFP6_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

double o_fp6_decode(uint8_t code);
uint8_t o_fp6_encode(float v);
double o_e8m0_decode(uint8_t code);
void o_pack(const uint8_t* codes, int n, uint8_t* packed);
void o_unpack(const uint8_t* packed, int n, uint8_t* codes);

void o_quantize_ref(const float* x, int rows, int cols, uint8_t* packed, uint8_t* scales);
void o_quantize_ocp(const float* x, int rows, int cols, uint8_t* packed, uint8_t* scales);

void o_pad_scales_k(const uint8_t* scales, int dim, int K, uint8_t* out);
void o_preprocess_scale(const uint8_t* scales, int dim, int K, uint8_t* out);
size_t o_tile_scale_bytes(int dim, int K, int group, int subs);
void o_tile_scale(const uint8_t* ps, int dim, int K, int group, int subs, uint8_t* out);
void o_preshuffle_b(const uint8_t* packed, int N, int K, size_t row_bytes, uint8_t* out);

void o_choose_tile_ref(int M, int N, int Kp, int tile[4]);
int o_splitk_s_ref(int M, int N, int Kp);

/* D[i][n] = sum_{k<K} a(row_i, k) * b(n, k) in FP64 for the listed A rows (rows == NULL: all M),
 * with absdot[i][n] = sum |a b| (may be NULL). A packed with stride a_row_bytes, scales with
 * stride a_scale_cols; B^T packed [N] rows of b_row_bytes, scales stride b_scale_cols. Exact
 * per 32-block (integer arithmetic), FP64 across blocks. nthreads <= 0: all cores. */
int o_gemm_f64(const uint8_t* a_packed, size_t a_row_bytes, const uint8_t* a_scales,
               int a_scale_cols, const uint8_t* b_packed, size_t b_row_bytes,
               const uint8_t* b_scales, int b_scale_cols, int M, int N, int K,
               const int* rows, int nrows, double* D, double* absdot, int nthreads);

/* The reference CPU GEMM's arithmetic: dequantise to FP32, then acc += a*b over k = 0..K-1 in
 * FP32, one accumulator per output, for the listed A rows. */
int o_gemm_f32_seq(const uint8_t* a_packed, size_t a_row_bytes, const uint8_t* a_scales,
                   int a_scale_cols, const uint8_t* b_packed, size_t b_row_bytes,
                   const uint8_t* b_scales, int b_scale_cols, int M, int N, int K,
                   const int* rows, int nrows, float* D, int nthreads);

/* The two halves of o_gemm_f32_seq: dequantise rows to FP32 once, then the sequential dots of
 * the listed A rows against the dequantised B^T bf[N][K]. */
int o_dequant_f32(const uint8_t* packed, size_t row_bytes, const uint8_t* scales,
                  int scale_cols, int rows, int K, float* out);
int o_gemm_f32_seq_deq(const uint8_t* a_packed, size_t a_row_bytes, const uint8_t* a_scales,
                       int a_scale_cols, const float* bf, int M, int N, int K, const int* rows,
                       int nrows, float* D, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
