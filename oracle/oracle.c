/* MXFP6 GEMM oracle -- TEST INFRASTRUCTURE ONLY (see oracle.h for scope and pinning).
 * Plain C11 + pthreads. Restates the reference (eeezio/mxfp6-gemm) from its sources:
 * include/mxfp6/types.hpp, include/mxfp6/preprocess.hpp, src/gemm.cpp, src/dispatch.hpp,
 * tests/reference.hpp. Written for clarity over speed, except the GEMM loops, which must finish
 * full-width sampled rows of the benchmark shapes in seconds. */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ---- FP6 E2M3 / E8M0 (types.hpp:9-95) -------------------------------------------------- */

/* value = (-1)^s * (e == 0 ? m/8 : (1 + m/8) * 2^(e-1)), s = bit 5, e = bits 4:3, m = bits 2:0 */
double o_fp6_decode(uint8_t code) {
    const int s = (code >> 5) & 1, e = (code >> 3) & 3, m = code & 7;
    const double mag = e == 0 ? m / 8.0 : (1.0 + m / 8.0) * ldexp(1.0, e - 1);
    return s ? -mag : mag;
}

/* Nearest representable magnitude by exhaustive search over the 32 magnitude codes; a tie goes
 * to the even code (= even mantissa). |v| > 7.5 saturates. The sign bit follows v < 0. */
uint8_t o_fp6_encode(float v) {
    const uint8_t sign = v < 0.0f ? 0x20 : 0x00;
    double a = fabs((double)v);
    if (a == 0.0 || isnan(a)) return sign;
    if (a > 7.5) a = 7.5;
    int best = 0;
    double bestd = INFINITY;
    for (int c = 0; c < 32; c++) {
        const double d = fabs(a - o_fp6_decode((uint8_t)c));
        if (d < bestd || (d == bestd && (c & 1) == 0 && (best & 1) == 1)) {
            best = c;
            bestd = d;
        }
    }
    return (uint8_t)(sign | best);
}

double o_e8m0_decode(uint8_t code) {
    return code == 255 ? NAN : ldexp(1.0, (int)code - 127);
}

/* code j occupies bits [6j, 6j+6) of the little-endian bit string of the packed bytes */
void o_pack(const uint8_t* codes, int n, uint8_t* packed) {
    memset(packed, 0, (size_t)n / 4 * 3);
    for (int j = 0; j < n; j++)
        for (int i = 0; i < 6; i++) {
            const int bit = 6 * j + i;
            if ((codes[j] >> i) & 1) packed[bit >> 3] |= (uint8_t)(1u << (bit & 7));
        }
}

void o_unpack(const uint8_t* packed, int n, uint8_t* codes) {
    for (int j = 0; j < n; j++) {
        uint8_t c = 0;
        for (int i = 0; i < 6; i++) {
            const int bit = 6 * j + i;
            c |= (uint8_t)(((packed[bit >> 3] >> (bit & 7)) & 1) << i);
        }
        codes[j] = c;
    }
}

/* ---- quantisers ------------------------------------------------------------------------------ */

static float block_amax(const float* x) {
    float m = 0.0f;
    for (int i = 0; i < 32; i++) m = fmaxf(m, fabsf(x[i])); /* NaN ignored */
    return m;
}

static int clamp_code(int c) {
    return c < 0 ? 0 : c > 254 ? 254 : c;
}

static void encode_block(const float* x, int e, uint8_t* packed) {
    uint8_t codes[32];
    for (int i = 0; i < 32; i++) codes[i] = o_fp6_encode((float)ldexp((double)x[i], -e));
    o_pack(codes, 32, packed);
}

/* Reference rule (preprocess.hpp:62-94): scale = smallest power of two >= amax / 7.5f
 * (the quotient computed in FP32), searched over exponents; zero block -> 127. */
void o_quantize_ref(const float* x, int rows, int cols, uint8_t* packed, uint8_t* scales) {
    const int nb = cols / 32;
    for (size_t r = 0; r < (size_t)rows; r++)
        for (int b = 0; b < nb; b++) {
            const float* v = x + r * cols + 32 * b;
            const float amax = block_amax(v);
            int code = 127;
            if (amax != 0.0f) {
                const float need = amax / 7.5f;
                int e = -160;
                while (ldexp(1.0, e) < (double)need) e++;
                code = clamp_code(e + 127);
            }
            scales[r * nb + b] = (uint8_t)code;
            encode_block(v, code - 127, packed + r * ((size_t)cols / 4 * 3) + 24 * b);
        }
}

/* BASELINE workload rule (OCP MX v1.0 section 6.3): scale = 2^(floor(log2 amax) - emax_elem),
 * emax_elem = 2 for E2M3; floor(log2) found by search over exponents; zero block -> 127. */
void o_quantize_ocp(const float* x, int rows, int cols, uint8_t* packed, uint8_t* scales) {
    const int nb = cols / 32;
    for (size_t r = 0; r < (size_t)rows; r++)
        for (int b = 0; b < nb; b++) {
            const float* v = x + r * cols + 32 * b;
            const float amax = block_amax(v);
            int code = 127;
            if (amax > 0.0f) {
                int e = 200;
                while (ldexp(1.0, e) > (double)amax) e--;
                code = clamp_code(e - 2 + 127);
            }
            scales[r * nb + b] = (uint8_t)code;
            encode_block(v, code - 127, packed + r * ((size_t)cols / 4 * 3) + 24 * b);
        }
}

/* ---- layouts (preprocess.hpp:26-38, 136-162, 182-207, 216-233) ---------------------------- */

void o_pad_scales_k(const uint8_t* scales, int dim, int K, uint8_t* out) {
    const int sc = K / 32, scp = (K + 191) / 192 * 192 / 32;
    for (int r = 0; r < dim; r++)
        for (int c = 0; c < scp; c++)
            out[(size_t)r * scp + c] = c < sc ? scales[(size_t)r * sc + c] : 127;
}

void o_preprocess_scale(const uint8_t* scales, int dim, int K, uint8_t* out) {
    const int tiles = dim / 32, k64n = K / 64, sc = K / 32;
    for (int t = 0; t < tiles; t++)
        for (int q = 0; q < k64n; q++)
            for (int lane = 0; lane < 64; lane++) {
                const int row = t * 32 + lane % 32, col = 2 * q + lane / 32;
                out[((size_t)t * k64n + q) * 64 + lane] = scales[(size_t)row * sc + col];
            }
}

size_t o_tile_scale_bytes(int dim, int K, int group, int subs) {
    const int gp = (group + 3) / 4 * 4;
    return (size_t)(dim / 32 / group) * (size_t)(K / 64 / subs) * 64 * (size_t)subs * gp;
}

void o_tile_scale(const uint8_t* ps, int dim, int K, int group, int subs, uint8_t* out) {
    const int gp = (group + 3) / 4 * 4, k64n = K / 64, ktn = k64n / subs, ng = dim / 32 / group;
    memset(out, 0, o_tile_scale_bytes(dim, K, group, subs));
    for (int g = 0; g < ng; g++)
        for (int kt = 0; kt < ktn; kt++)
            for (int lane = 0; lane < 64; lane++)
                for (int sub = 0; sub < subs; sub++)
                    for (int j = 0; j < group; j++) {
                        const size_t dst = ((((size_t)g * ktn + kt) * 64 + lane) * subs + sub) * gp + j;
                        const size_t src = (((size_t)g * group + j) * k64n + kt * subs + sub) * 64 + lane;
                        out[dst] = ps[src];
                    }
}

void o_preshuffle_b(const uint8_t* packed, int N, int K, size_t row_bytes, uint8_t* out) {
    const int k64n = K / 64;
    for (int nt = 0; nt < N / 32; nt++)
        for (int q = 0; q < k64n; q++) {
            uint8_t* tile = out + ((size_t)nt * k64n + q) * 1536;
            for (int t = 0; t < 64; t++) {
                const uint8_t* src = packed + (size_t)(nt * 32 + t % 32) * row_bytes + (size_t)q * 48 + (t / 32) * 24;
                memcpy(tile + 16 * t, src, 16);
                memcpy(tile + 1024 + 8 * t, src + 16, 8);
            }
        }
}

/* ---- reference router and split plan (gemm.cpp:12-59, dispatch.hpp:30-59) ------------------ */

static void set_tile(int t[4], int mt, int nt, int mpw, int npw) {
    t[0] = mt;
    t[1] = nt;
    t[2] = mpw;
    t[3] = npw;
}

void o_choose_tile_ref(int M, int N, int Kp, int t[4]) {
    const int CU = 256, LARGEK = 32768;
    const int wg256 = (M / 256) * (N / 256);
    if (wg256 < CU && M % 128 == 0 && N % 384 == 0) {
        const int wg384 = (M / 128) * (N / 384), wg256g = (M / 128) * (N / 256);
        if (wg384 >= CU && 3 * ((wg384 + CU - 1) / CU) < 2 * ((wg256g + CU - 1) / CU)) {
            set_tile(t, 128, 384, 4, 3);
            return;
        }
    }
    if (wg256 < CU && M % 128 == 0 && N % 128 == 0 && Kp >= LARGEK && (M / 128) * (N / 128) >= CU) {
        set_tile(t, 128, 128, 2, 2);
        return;
    }
    if (wg256 < CU && M % 128 == 0 && N % 256 == 0) { set_tile(t, 128, 256, 2, 4); return; }
    if (M % 256 == 0 && N % 256 == 0) { set_tile(t, 256, 256, 4, 4); return; }
    if (M % 128 == 0 && N % 256 == 0) { set_tile(t, 128, 256, 2, 4); return; }
    if (M % 128 == 0 && N % 384 == 0) { set_tile(t, 128, 384, 4, 3); return; }
    if (M % 256 == 0 && N % 128 == 0) { set_tile(t, 256, 256, 4, 4); return; }
    if (M % 128 == 0 && N % 128 == 0) { set_tile(t, 128, 128, 2, 2); return; }
    set_tile(t, 256, 256, 4, 4);
}

int o_splitk_s_ref(int M, int N, int Kp) {
    int t[4];
    o_choose_tile_ref(M, N, Kp, t);
    if (t[1] == 384 || t[1] == 128) return 1;
    if (N % t[1] != 0) return 1;
    const int k_tiles = (Kp / 64) / 3, base = (M / t[0]) * (N / t[1]);
    int S = 1;
    if (base > 0 && base < 256 && k_tiles >= 16) {
        S = (256 + base - 1) / base;
        if (S > k_tiles / 8) S = k_tiles / 8;
        if (S < 1) S = 1;
    }
    return S;
}

/* ---- GEMM ------------------------------------------------------------------------------------ */

/* Every E2M3 value times 8 is an integer in [-60, 60]. */
static void decode_row_i8(const uint8_t* packed, int K, int8_t* out) {
    static int8_t lut[64];
    static int ready = 0;
    if (!ready) {
        for (int c = 0; c < 64; c++) lut[c] = (int8_t)lrint(o_fp6_decode((uint8_t)c) * 8.0);
        ready = 1;
    }
    for (int g = 0; g < K / 4; g++) {
        const uint32_t w = packed[3 * g] | ((uint32_t)packed[3 * g + 1] << 8) | ((uint32_t)packed[3 * g + 2] << 16);
        for (int i = 0; i < 4; i++) out[4 * g + i] = lut[(w >> (6 * i)) & 63];
    }
}

typedef struct {
    const uint8_t *ap, *as, *bp, *bs;
    size_t arb, brb;
    int asc, bsc, M, N, K;
    const int* rows;
    int nrows;
    const int8_t* bi8; /* [N][K] */
    double *D, *absdot;
    float* Df;
    int next, nthreads;
    pthread_mutex_t mu;
} gemm_job;

static int take_row(gemm_job* j) {
    pthread_mutex_lock(&j->mu);
    const int i = j->next < j->nrows ? j->next++ : -1;
    pthread_mutex_unlock(&j->mu);
    return i;
}

static void* f64_worker(void* arg) {
    gemm_job* j = (gemm_job*)arg;
    const int K = j->K, nb = K / 32;
    int8_t* ai = (int8_t*)malloc((size_t)K);
    double* sa = (double*)malloc(sizeof(double) * nb);
    for (int i; (i = take_row(j)) >= 0;) {
        const int m = j->rows ? j->rows[i] : i;
        decode_row_i8(j->ap + (size_t)m * j->arb, K, ai);
        for (int b = 0; b < nb; b++) sa[b] = o_e8m0_decode(j->as[(size_t)m * j->asc + b]);
        for (int n = 0; n < j->N; n++) {
            const int8_t* bi = j->bi8 + (size_t)n * K;
            const uint8_t* bsr = j->bs + (size_t)n * j->bsc;
            double acc = 0.0, aacc = 0.0;
            for (int b = 0; b < nb; b++) {
                int s = 0, sabs = 0;
                for (int k = 32 * b; k < 32 * b + 32; k++) {
                    const int p = ai[k] * bi[k];
                    s += p;
                    sabs += p < 0 ? -p : p;
                }
                const double w = sa[b] * o_e8m0_decode(bsr[b]) / 64.0;
                if (s != 0 || isnan(w)) acc += (double)s * w;
                if (sabs != 0 || isnan(w)) aacc += (double)sabs * w;
            }
            j->D[(size_t)i * j->N + n] = acc;
            if (j->absdot) j->absdot[(size_t)i * j->N + n] = aacc;
        }
    }
    free(ai);
    free(sa);
    return NULL;
}

static void run_pool(gemm_job* j, void* (*fn)(void*)) {
    int nt = j->nthreads > 0 ? j->nthreads : (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (nt < 1) nt = 1;
    if (nt > 64) nt = 64;
    pthread_t th[64];
    pthread_mutex_init(&j->mu, NULL);
    j->next = 0;
    for (int t = 0; t < nt; t++) pthread_create(&th[t], NULL, fn, j);
    for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
    pthread_mutex_destroy(&j->mu);
}

int o_gemm_f64(const uint8_t* a_packed, size_t a_row_bytes, const uint8_t* a_scales,
               int a_scale_cols, const uint8_t* b_packed, size_t b_row_bytes,
               const uint8_t* b_scales, int b_scale_cols, int M, int N, int K, const int* rows,
               int nrows, double* D, double* absdot, int nthreads) {
    if (K % 32 != 0) return 1;
    int8_t* bi8 = (int8_t*)malloc((size_t)N * K);
    if (!bi8) return 2;
    for (int n = 0; n < N; n++) decode_row_i8(b_packed + (size_t)n * b_row_bytes, K, bi8 + (size_t)n * K);
    gemm_job j;
    memset(&j, 0, sizeof j);
    j.ap = a_packed; j.as = a_scales; j.bp = b_packed; j.bs = b_scales;
    j.arb = a_row_bytes; j.brb = b_row_bytes; j.asc = a_scale_cols; j.bsc = b_scale_cols;
    j.M = M; j.N = N; j.K = K; j.rows = rows; j.nrows = rows ? nrows : M;
    j.bi8 = bi8; j.D = D; j.absdot = absdot; j.nthreads = nthreads;
    run_pool(&j, f64_worker);
    free(bi8);
    return 0;
}

/* FP32 dequantised row: fp6 value (float) times e8m0 scale (float), as reference.hpp:20-22 via
 * dequantize_mxfp6 (preprocess.hpp:100-109). */
static void dequant_row_f32(const uint8_t* packed, const uint8_t* scales, int K, float* out) {
    static float lut[64];
    static int ready = 0;
    if (!ready) {
        for (int c = 0; c < 64; c++) lut[c] = (float)o_fp6_decode((uint8_t)c);
        ready = 1;
    }
    for (int g = 0; g < K / 4; g++) {
        const uint32_t w = packed[3 * g] | ((uint32_t)packed[3 * g + 1] << 8) | ((uint32_t)packed[3 * g + 2] << 16);
        const float s = (float)o_e8m0_decode(scales[(4 * g) / 32]);
        for (int i = 0; i < 4; i++) out[4 * g + i] = lut[(w >> (6 * i)) & 63] * s;
    }
}

typedef struct {
    gemm_job* j;
    const float* bf; /* [N][K] */
} f32_ctx;

static void* f32_worker(void* arg) {
    f32_ctx* c = (f32_ctx*)arg;
    gemm_job* j = c->j;
    const int K = j->K;
    float* a = (float*)malloc(sizeof(float) * K);
    for (int i; (i = take_row(j)) >= 0;) {
        const int m = j->rows ? j->rows[i] : i;
        dequant_row_f32(j->ap + (size_t)m * j->arb, j->as + (size_t)m * j->asc, K, a);
        for (int n = 0; n < j->N; n++) {
            const float* b = c->bf + (size_t)n * K;
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc += a[k] * b[k];
            j->Df[(size_t)i * j->N + n] = acc;
        }
    }
    free(a);
    return NULL;
}

static void* f32_trampoline(void* arg) {
    return f32_worker(arg);
}

int o_dequant_f32(const uint8_t* packed, size_t row_bytes, const uint8_t* scales,
                  int scale_cols, int rows, int K, float* out) {
    if (K % 32 != 0) return 1;
    dequant_row_f32(packed, scales, 32, out); /* initialise the table on this thread */
    for (int r = 0; r < rows; r++)
        dequant_row_f32(packed + (size_t)r * row_bytes, scales + (size_t)r * scale_cols, K,
                        out + (size_t)r * K);
    return 0;
}

int o_gemm_f32_seq_deq(const uint8_t* a_packed, size_t a_row_bytes, const uint8_t* a_scales,
                       int a_scale_cols, const float* bf, int M, int N, int K, const int* rows,
                       int nrows, float* D, int nthreads) {
    if (K % 32 != 0) return 1;
    float tmp[32];
    dequant_row_f32(a_packed, a_scales, 32, tmp); /* initialise the table before the threads */
    gemm_job j;
    memset(&j, 0, sizeof j);
    j.ap = a_packed; j.as = a_scales; j.arb = a_row_bytes; j.asc = a_scale_cols;
    j.M = M; j.N = N; j.K = K; j.rows = rows; j.nrows = rows ? nrows : M;
    j.Df = D; j.nthreads = nthreads;
    f32_ctx c = {&j, bf};
    int nt = nthreads > 0 ? nthreads : (int)sysconf(_SC_NPROCESSORS_ONLN);
    if (nt < 1) nt = 1;
    if (nt > 64) nt = 64;
    pthread_t th[64];
    pthread_mutex_init(&j.mu, NULL);
    for (int t = 0; t < nt; t++) pthread_create(&th[t], NULL, f32_trampoline, &c);
    for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
    pthread_mutex_destroy(&j.mu);
    return 0;
}

int o_gemm_f32_seq(const uint8_t* a_packed, size_t a_row_bytes, const uint8_t* a_scales,
                   int a_scale_cols, const uint8_t* b_packed, size_t b_row_bytes,
                   const uint8_t* b_scales, int b_scale_cols, int M, int N, int K,
                   const int* rows, int nrows, float* D, int nthreads) {
    if (K % 32 != 0) return 1;
    float* bf = (float*)malloc(sizeof(float) * (size_t)N * K);
    if (!bf) return 2;
    o_dequant_f32(b_packed, b_row_bytes, b_scales, b_scale_cols, N, K, bf);
    const int rc = o_gemm_f32_seq_deq(a_packed, a_row_bytes, a_scales, a_scale_cols, bf, M, N, K,
                                      rows, nrows, D, nthreads);
    free(bf);
    return rc;
}
