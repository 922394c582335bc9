/* libmxfp6gemm — C ABI of the MI355X (gfx950) MXFP6 GEMM.
 *
 * Plain C: pointers, ints and sizes only, no C++ or HIP types, so any FFI (ctypes, cgo, JNI,
 * N-API) binds it. Each entry point names the reference interface it stands for
 * (eeezio/mxfp6-gemm, path:line). The C++ API of include/mxfp6/gemm.hpp is exported from the
 * same library and calls the same code.
 *
 * Conventions
 *   - Functions returning int return an mxfp6_status (0 = success). The reference API has no
 *     status; these codes are additive. Invalid arguments are reported, never launched.
 *   - Device pointers (d*, ws) are caller-owned device memory; nothing here allocates or frees
 *     device memory.
 *   - `stream` is a hipStream_t passed as void*; NULL is the null stream.
 *   - out_type: 0 = FP32, 1 = FP16, 2 = BF16 (the order of mxfp6::OutType).
 */
#ifndef MXFP6_GEMM_H
#define MXFP6_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mxfp6_status {
    MXFP6_OK = 0,
    MXFP6_ERR_NULL = 1,      /* a required pointer is NULL */
    MXFP6_ERR_SHAPE = 2,     /* M, N, Kp or a row stride violates the kernel's requirements */
    MXFP6_ERR_OUT_TYPE = 3,  /* out_type not in {0, 1, 2} */
    MXFP6_ERR_TILE = 4,      /* tile not implemented, or it does not divide the shape */
    MXFP6_ERR_ARG = 5,       /* other invalid argument */
    MXFP6_ERR_HIP = 6,       /* the HIP runtime reported an error at launch */
    MXFP6_ERR_SCRATCH = 7    /* mxfp6_gemm_noalloc_async: the plan's split-K partials exceed
                                MXFP6_NOALLOC_SCRATCH_BYTES */
} mxfp6_status;

/* ---- GEMM (reference include/mxfp6/gemm.hpp, src/gemm.cpp) -------------------------------- */

/* kpad(K): K rounded up to a multiple of K_TILE = 192.   Replaces gemm.hpp:30-33. */
int mxfp6_kpad(int K);

/* choose_tile(M, N, Kp) -> tile[4] = {MT, NT, MPW, NPW}.   Replaces gemm.hpp:46 / gemm.cpp:12-59. */
int mxfp6_choose_tile(int M, int N, int Kp, int tile[4]);

/* gemm_workspace_size(M, N, Kp): bytes of FP32 split-K partials gemm() uses for (M, N, Kp)
 * (splits * M * N * 4), 0 when the shape is not split.   Replaces gemm.hpp:53 / gemm.cpp:61-63
 * (same meaning). */
size_t mxfp6_gemm_workspace_size(int M, int N, int Kp);

/* The routed plan's whole workspace: the split-K partials, then (at the next 256-byte boundary)
 * ceil(M/32)*32 * packed(Kp) bytes when the plan repacks A into the preshuffled operand layout
 * first (mxfp6_gemm_repacks_a); 0 when the plan needs neither. gemm() given at least this much
 * runs the repack; given only mxfp6_gemm_workspace_size's bytes it reads A row-major: the same
 * output bits, slower on the shapes that repack. No counterpart in the reference (its kernels
 * read A row-major). */
size_t mxfp6_gemm_preferred_workspace_size(int M, int N, int Kp);

/* Number of K segments gemm() uses for (M, N, Kp) when given a sufficient workspace.
 * Replaces src/dispatch.hpp:30-53 (detail::splitk_S). */
int mxfp6_splitk_segments(int M, int N, int Kp);

/* gemm(ot, M, N, Kp, dA, dBsh, dsA, dsB, dD, A_row_bytes, B_row_bytes, ws, ws_bytes) on the
 * null stream. Same arguments and semantics as gemm.hpp:63-64 / gemm.cpp:65-83 on the
 * reference's shapes (M, N multiples of 128). Beyond the reference, any M, N >= 1: M a multiple
 * of 32 routes to 32- and 64-row tiles, and a tile that does not divide M x N runs with its last
 * tile row / column masked (the reference's NMASK, src/kernel.hpp:144-154, generalised). The
 * operand layouts then hold ceil(dim/32) 32-row blocks and whole scale groups, completed with
 * zero rows (codes 0, scale code 127): mxfp6_preshuffled_bytes / mxfp6_tiled_scale_bytes size
 * them, mxfp6_prepare_* and mxfp6_prepare_b / mxfp6_prepare_scales produce them. The scales are
 * tiled with the MPW / NPW choose_tile returns for the shape. Plus a status: a shape that would
 * split with a NULL or short workspace runs unsplit (stderr warning, status MXFP6_OK), as the
 * reference does. A workspace of at least mxfp6_gemm_preferred_workspace_size bytes also holds
 * the repacked A; a shorter one (such as exactly mxfp6_gemm_workspace_size's) skips the repack:
 * same result, slower. */
int mxfp6_gemm(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
               const uint8_t* dsA, const uint8_t* dsB, void* dD, int A_row_bytes, int B_row_bytes,
               void* ws, size_t ws_bytes);

/* mxfp6_gemm on an explicit HIP stream (additive; the reference has no stream argument). */
int mxfp6_gemm_async(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
                     const uint8_t* dsA, const uint8_t* dsB, void* dD, int A_row_bytes,
                     int B_row_bytes, void* ws, size_t ws_bytes, void* stream);

/* Size of the device scratch of mxfp6_gemm_noalloc_async: 128 MiB per GPU. */
#define MXFP6_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)

/* mxfp6_gemm_async without a workspace argument, and without any device allocation or free (no
 * hipMalloc, hipFree or allocating library call): the split-K partials, and the repacked A when it
 * fits beside them, go to a device array of MXFP6_NOALLOC_SCRATCH_BYTES that the library holds
 * per GPU from the first such call on that GPU until the process ends. Same plan and the same
 * output bits as mxfp6_gemm_async with mxfp6_gemm_preferred_workspace_size bytes, except that a
 * repacked A that does not fit is read row-major instead (with the routed split, possibly on
 * another tile of the routed scale grouping: the same bits). A shape whose split-K
 * partials (mxfp6_gemm_workspace_size) exceed the scratch is rejected with MXFP6_ERR_SCRATCH,
 * before any device work. Every call on a GPU shares that GPU's scratch: calls that overlap on one
 * GPU (concurrent streams or host threads) race; serialise them. The first call on a GPU looks the
 * scratch's device address up (hipGetSymbolAddress, which may load the code object): make it
 * outside stream capture, e.g. once eagerly at set-up; later calls may be captured into a HIP
 * graph. No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). */
int mxfp6_gemm_noalloc_async(int out_type, int M, int N, int Kp, const void* dA,
                             const void* dBsh, const uint8_t* dsA, const uint8_t* dsB, void* dD,
                             int A_row_bytes, int B_row_bytes, void* stream);

/* gemm_force_tile: run the tile {MT, NT, MPW, NPW} given by the caller instead of the router's
 * choice, unsplit. Test-only in the reference (src/gemm.cpp:85-107, not in its header); the
 * scales must be tiled with this tile's MPW/NPW. Rejects tiles the library does not implement
 * and tiles that do not divide M x N (mxfp6_gemm_explicit runs those masked), and the 32 x 32
 * tile past four K-tiles (its unsplit limit). */
int mxfp6_gemm_force_tile(int out_type, int M, int N, int Kp, const int tile[4], const void* dA,
                          const void* dBsh, const uint8_t* dsA, const uint8_t* dsB, void* dD,
                          int A_row_bytes, int B_row_bytes, void* stream);

/* Run an explicit plan: the pipelined kernel with tile {MT, NT, MPW, NPW} (masked when it does
 * not divide M x N), `splits` K segments and an A layout: 0 = row-major A (A_row_bytes per row); 1 = repack row-major A into the workspace in
 * the preshuffled operand layout first, then read that; 2 = dA already holds A in the preshuffled
 * layout (mxfp6_preshuffle_rows_async output; A_row_bytes is then only checked); 3 = row-major A
 * as 0, staged in LDS in 12-byte units whose slots are swizzled per row (operand reads free of
 * bank conflicts; the four wide tiles only, dividing M x N, else MXFP6_ERR_ARG; same output bits
 * as 0; never routed: measured no faster). The tile {32, 32, 1, 1} splits K over a workgroup's
 * waves (small grids): row-major A, at most 16 segments of at most 4 K-tiles, else MXFP6_ERR_ARG;
 * the same bits as the other split plans of that grouping. Needs ws of
 * mxfp6_plan_workspace_size(M, N, Kp, splits, a_layout == 1) bytes. For tuning, benchmarks and
 * callers that keep A preshuffled; the scales must be tiled with this tile's MPW/NPW. No
 * counterpart in the reference (it is the reference's gemm_force_tile, src/gemm.cpp:89-107, plus a
 * split count and the A layout). */
int mxfp6_gemm_explicit(int out_type, int M, int N, int Kp, const int tile[4], int splits,
                        int a_layout, const void* dA, const void* dBsh, const uint8_t* dsA,
                        const uint8_t* dsB, void* dD, int A_row_bytes, void* ws, size_t ws_bytes,
                        void* stream);

/* Whether gemm() repacks A for (M, N, Kp) when its workspace allows. No counterpart in the
 * reference (its kernels read A row-major). */
int mxfp6_gemm_repacks_a(int M, int N, int Kp);

/* Measured plan selection. No counterpart in the reference (its router is a fixed rule).
 *
 * mxfp6_gemm_tune times up to `candidates` plans for (out_type, M, N, Kp) -- the routed plan
 * first (where it is the 32 x 32 tile, then that tile at the nearest valid segment counts below
 * and above), then the router's best-predicted ones with choose_tile's scale grouping (the
 * operands' scales are tiled for it), each whose workspace fits ws_bytes -- on the caller's
 * operands (D is overwritten), and keeps the fastest for
 * the process: later gemm() calls of the shape and output type run it whenever their workspace
 * holds it (else the router's plan). It waits for `stream`, so it must not be called during graph
 * capture. The chosen plan is returned in tile, *splits and *a_repack (each may be NULL). A
 * different plan may sum K in another order: D stays within the same tolerance of the exact
 * result, but its low bits may differ from the router's plan. */
int mxfp6_gemm_tune(int out_type, int M, int N, int Kp, const void* dA, const void* dBsh,
                    const uint8_t* dsA, const uint8_t* dsB, void* dD, int A_row_bytes, void* ws,
                    size_t ws_bytes, int candidates, void* stream, int tile[4], int* splits,
                    int* a_repack);

/* The measured plan of (out_type, M, N, Kp): 1 and the plan in tile, *splits, *a_repack (each may
 * be NULL) if mxfp6_gemm_tune chose one, else 0. */
int mxfp6_gemm_tuned_plan(int out_type, int M, int N, int Kp, int tile[4], int* splits,
                          int* a_repack);

/* Forgets every measured plan (gemm() runs the router's plans again). */
void mxfp6_gemm_tune_reset(void);

/* Writes the measured plans to a text file (a comment line, then one plan per line: out_type M N
 * Kp MT NT MPW NPW S repack) and their number to *count (may be NULL); MXFP6_ERR_ARG when the
 * file cannot be written. mxfp6_gemm_tune_load adds such a file's plans to the table, so that a
 * serving process can start with the plans an earlier run measured: a plan is taken only if its
 * tile is implemented, its split fits the shape and its scale grouping is the one choose_tile
 * returns for the shape on this device; *loaded and *skipped (may be NULL) count the lines taken
 * and left. MXFP6_ERR_ARG when the file cannot be read. No counterpart in the reference. */
int mxfp6_gemm_tune_save(const char* path, int* count);
int mxfp6_gemm_tune_load(const char* path, int* loaded, int* skipped);

/* The plan gemm() runs for (out_type, M, N, Kp) with a workspace of ws_bytes: tile {MT, NT, MPW,
 * NPW}, K segments and whether A is repacked first. A measured plan when the workspace holds it,
 * else the routed plan when the workspace holds it, else, on row-major A, the fastest predicted
 * tile with the routed scale grouping (the tile choose_tile returns fixes the scale layout) for the
 * routed split when ws_bytes holds its partials (gemm_workspace_size's bytes), or unsplit. For a
 * given split, the tiles of one scale grouping give the same output bits. No counterpart in the reference (its
 * dispatch runs choose_tile's tile, unsplit when the workspace is short, src/dispatch.hpp:74-87). */
int mxfp6_gemm_plan(int out_type, int M, int N, int Kp, size_t ws_bytes, int tile[4], int* splits,
                    int* a_repack);

/* Whether the routed plan for (out_type, M, N, Kp, A_row_bytes) writes D with nontemporal stores
 * (unsplit plans whose operands fit in MI355X's 256 MiB last-level cache but whose operands and D
 * together do not). The answer is for the plan gemm() runs with the preferred workspace
 * (mxfp6_gemm_preferred_workspace_size) and no measured plan registered for the shape; a measured
 * plan or a shorter workspace can run another plan, whose stores are decided the same way from
 * that plan. No counterpart in the reference (its epilogue stores are plain); D's values are the
 * same either way. */
int mxfp6_gemm_streams_output(int out_type, int M, int N, int Kp, int A_row_bytes);

/* Workspace bytes of an explicit plan (0 when splits == 1 and a_repack == 0). */
size_t mxfp6_plan_workspace_size(int M, int N, int Kp, int splits, int a_repack);

/* On-device preshuffle of `rows` row-major packed rows, each read for packed(Kp) bytes from
 * src + r * row_bytes, into dst (ceil(rows/32) * 32 * packed(Kp) bytes; rows past `rows` in the
 * last 32-row block are zero codes) in the layout of preshuffle_B (reference
 * include/mxfp6/preprocess.hpp:182-207, which runs on the host). Used by gemm() to repack A;
 * applied to B^T it gives preshuffle_B's output on the GPU. */
int mxfp6_preshuffle_rows_async(const void* src, int row_bytes, int rows, int Kp, void* dst,
                                void* stream);

/* The direct kernel (one wave per 32x32 block, operands read straight from global memory, any
 * scale grouping mpw/npw in 1..4) with an explicit K split count; M and N multiples of 64. A
 * second, independent GPU implementation used to cross-check the pipelined kernels; no
 * counterpart in the reference. splits > 1 needs ws of splits*M*N*4 bytes. */
int mxfp6_gemm_direct(int out_type, int M, int N, int Kp, int mpw, int npw, const void* dA,
                      const void* dBsh, const uint8_t* dsA, const uint8_t* dsB, void* dD,
                      int A_row_bytes, int splits, void* ws, size_t ws_bytes, void* stream);

/* Clock sample, a measurement aid: nwg one-wave workgroups (1..65536) each record, at
 * d_out[4*i .. 4*i+3], the shader clock counter (s_memtime, which counts at the current graphics
 * clock of the XCD the workgroup ran on), the 100 MHz reference counter (s_memrealtime), the XCD
 * id and the hardware id (shader engine, shader array and CU in bits 8..15). Two samples around
 * a region of GPU work give each XCD's mean graphics clock over it: the cycle difference over the
 * reference difference times 100 MHz, pairing workgroups that ran on the same CU (each CU's
 * cycle counter has its own fixed offset). Asynchronous on `stream`. No counterpart in the
 * reference (its benchmarks read the clock from the SMI tools). */
int mxfp6_clock_sample_async(uint64_t* d_out, int nwg, void* stream);

/* ---- element formats (reference include/mxfp6/types.hpp) ---------------------------------- */

float mxfp6_fp6_e2m3_to_float(uint8_t code);    /* types.hpp:13-24 */
uint8_t mxfp6_float_to_fp6_e2m3(float v);       /* types.hpp:26-72 */
float mxfp6_e8m0_to_float(uint8_t code);        /* types.hpp:78-81 */
uint8_t mxfp6_float_to_e8m0(float v);           /* types.hpp:83-92 */
int mxfp6_pack_fp6(const uint8_t* vals, int n, uint8_t* packed);   /* types.hpp:97-117 */
int mxfp6_unpack_fp6(const uint8_t* packed, int n, uint8_t* vals); /* types.hpp:104-122 */

/* ---- host layouts (reference include/mxfp6/preprocess.hpp) -------------------------------- */

/* a_compact_end_pad(K).   preprocess.hpp:26-28 */
int mxfp6_a_compact_end_pad(int K);

/* pad_scales_k: scales[dim][K/32] -> out[dim][kpad(K)/32], tail code 127.   preprocess.hpp:32-38 */
int mxfp6_pad_scales_k(const uint8_t* scales, int dim, int K, uint8_t* out);

/* quantize_to_mxfp6: mat[rows][cols] -> packed[rows][3*cols/4], scales[rows][cols/32].
 * preprocess.hpp:51-97 */
int mxfp6_quantize(const float* mat, int rows, int cols, uint8_t* packed, uint8_t* scales);

/* dequantize_mxfp6: packed + scales -> out[rows][cols].   preprocess.hpp:100-109 */
int mxfp6_dequantize(const uint8_t* packed, const uint8_t* scales, int rows, int cols, float* out);

/* preprocess_B: B[K][N] row-major -> quantised B^T: packed[N][3*K/4], scales[N][K/32].
 * preprocess.hpp:112-118 */
int mxfp6_preprocess_b(const float* B, int K, int N, uint8_t* packed, uint8_t* scales);

/* preprocess_scale: scales[dim][K/32] -> out[dim/32][K/64][64].   preprocess.hpp:136-162 */
int mxfp6_preprocess_scale(const uint8_t* scales, int dim, int K, uint8_t* out);

/* preshuffle_B: packed B^T[N][row_bytes] (row_bytes >= 3*K/4) -> out[N/32][K/64][1536].
 * preprocess.hpp:182-207 (the reference reads rows of exactly 3*K/4 bytes). */
int mxfp6_preshuffle_b(const uint8_t* packed, int N, int K, int row_bytes, uint8_t* out);

/* tile_scale: preprocess_scale output for (dim, K) -> grouped layout.   preprocess.hpp:216-233
 * group must divide dim / 32 (the header's tile_scale drops a partial last group, which a masked
 * tile would read): otherwise mxfp6_tile_scale_bytes returns 0 and mxfp6_tile_scale
 * MXFP6_ERR_ARG. mxfp6_prepare_scales / mxfp6_tiled_scale_bytes give the zero-extended layout of
 * any grouping. */
size_t mxfp6_tile_scale_bytes(int dim, int K, int group, int subs);
int mxfp6_tile_scale(const uint8_t* pscale, int dim, int K, int group, int subs, uint8_t* out);

/* ---- the same formats produced on the device (one HBM pass over float operands) ------------
 * The reference has host loops only; these are their device counterparts, bit-identical to them.
 * Inputs and outputs are device pointers; the calls are asynchronous on `stream`. Beyond the
 * reference (which needs K % 32 == 0 and whole 32-row blocks), any sizes >= 1: a K that is not a
 * multiple of 32 is quantised as if zero-padded to one (nb = ceil(K/32) blocks, 24 bytes each),
 * and dims that do not fill a 32-row block or a scale group are completed with zero rows
 * (codes 0, scale code 127) in the preshuffled and tiled outputs. Float inputs are 4-byte
 * aligned (16-byte aligned with a row length that is a multiple of 4 reads them as float4). */

/* quantize_to_mxfp6 (preprocess.hpp:51-97) of row-major float d_x[rows][cols]: row r's
 * 24 * ceil(cols/32) code bytes at d_packed + r * packed_row_bytes (at least that, a multiple of 4;
 * the bytes past the codes are set to 0), scales at d_scales[r * scale_cols + c]
 * (scale_cols >= ceil(cols/32); columns past the values set to 127, as pad_scales_k, :32-38,
 * does). */
int mxfp6_quantize_async(const float* d_x, int rows, int cols, void* d_packed,
                         size_t packed_row_bytes, uint8_t* d_scales, int scale_cols, void* stream);

/* A operand ready for mxfp6_gemm: quantize_to_mxfp6 of d_A[M][K] into rows of a_row_bytes
 * (>= 24 * ceil(K/32), a multiple of 4; bytes past the codes zero: a_row_bytes = 3*kpad(K)/4
 * gives padded rows with a zero K-tail), and the scales padded to kpad(K) and tiled as
 * tile_scale(preprocess_scale(pad_scales_k(..)), group, 3) (:32-38, :136-162, :216-233) with
 * group = the tile's MPW. d_tiled holds mxfp6_tiled_scale_bytes(M, K, group) bytes. */
int mxfp6_prepare_a_async(const float* d_A, int M, int K, int group, void* d_packed,
                          size_t a_row_bytes, uint8_t* d_tiled, void* stream);

/* A operand straight into the preshuffled operand layout (the bytes mxfp6_preshuffle_rows_async
 * would make of mxfp6_prepare_a_async's rows, i.e. preshuffle_B's layout, :182-207, applied to A)
 * in d_ash (mxfp6_preshuffled_bytes(M, K) bytes, 16-byte aligned), scales as mxfp6_prepare_a_async.
 * For mxfp6_gemm_explicit with a_layout = 2: a caller that quantises A on the device skips the
 * repack of A. No counterpart in the reference (its A is row-major only). */
int mxfp6_prepare_a_preshuffled_async(const float* d_A, int M, int K, int group, void* d_ash,
                                      uint8_t* d_tiled, void* stream);

/* B operand ready for mxfp6_gemm from row-major float d_B[K][N]: preprocess_B (:112-118), K
 * padded to kpad(K) with zero codes, preshuffle_B (:182-207) into d_bsh
 * (mxfp6_preshuffled_bytes(N, K) bytes, 16-byte aligned), and the scales tiled as for A with
 * group = the tile's NPW. */
int mxfp6_prepare_b_async(const float* d_B, int K, int N, int group, void* d_bsh,
                          uint8_t* d_tiled, void* stream);

/* Scales already quantised: d_scales[dim][ld] (ceil(K/32) valid columns) -> padded to kpad(K)
 * and tiled (group) as above. */
int mxfp6_tile_scales_async(const uint8_t* d_scales, int dim, int K, int ld, int group,
                            uint8_t* d_tiled, void* stream);

/* Sizes of the device layouts at kpad(K): preshuffled operand (ceil(dim/32) * kpad(K)/64 * 1536)
 * and tiled scales (tile_scale(.., group, 3) over ceil(dim / (32 * group)) groups). 0 for
 * dim, K < 1 or a group outside 1..4. */
size_t mxfp6_preshuffled_bytes(int dim, int K);
size_t mxfp6_tiled_scale_bytes(int dim, int K, int group);

/* ---- synthetic operands (the benchmark workloads) ----------------------------------------- */

/* Distributions of mxfp6_gen_operand. */
enum { MXFP6_DIST_NORMAL = 0, MXFP6_DIST_UNIFORM = 1, MXFP6_DIST_STUDENT_T3 = 2 };

/* Fill rows x K values (K % 32 == 0) from a PCG32 stream (O'Neill; state seeded by (seed,
 * stream), row r starting at draw r * draws_per_row so rows are independent of the thread
 * count) and quantise every 32-block with the OCP MX rule: scale = 2^(floor(log2 amax) - 2),
 * codes = nearest E2M3 of x / scale (saturating at 7.5), all-zero block -> code 127.
 *   dist: MXFP6_DIST_NORMAL (N(0, sigma^2)), MXFP6_DIST_UNIFORM (U[-sigma, sigma]),
 *         MXFP6_DIST_STUDENT_T3 (sigma * t with 3 degrees of freedom)
 *   packed: rows x row_bytes bytes; row r's codes at r * row_bytes, 3*K/4 bytes; bytes past
 *           3*K/4 in a row (up to row_bytes) are set to 0 (a zero K-tail)
 *   scales: rows x scale_cols bytes; columns past K/32 set to 127
 *   nthreads <= 0 uses the hardware concurrency. */
int mxfp6_gen_operand(int rows, int K, int dist, double sigma, uint64_t seed, uint64_t stream,
                      uint8_t* packed, size_t row_bytes, uint8_t* scales, int scale_cols,
                      int nthreads);

/* The same values as mxfp6_gen_operand before quantisation (float), for tests. */
int mxfp6_gen_values(int rows, int K, int dist, double sigma, uint64_t seed, uint64_t stream,
                     float* out, int nthreads);

/* Prepare kernel-ready device-layout buffers on the host from raw packed codes and scales:
 *   B: packed B^T[N][b_row_bytes] (Kp codes per row) -> preshuffled bsh
 *      (ceil(N/32) * Kp/64 * 1536 B; zero codes past N)
 *   scales[dim][Kp/32] -> tiled (preprocess_scale then tile_scale(group, 3)) over
 *      ceil(dim / (32 * group)) groups (code 127 past dim).
 * Multi-threaded versions of preshuffle_B and tile_scale(preprocess_scale(..)), extended to
 * ragged dims as the device producers are. */
int mxfp6_prepare_b(const uint8_t* packed, int N, int Kp, size_t b_row_bytes, uint8_t* bsh,
                    int nthreads);
int mxfp6_prepare_scales(const uint8_t* scales, int dim, int Kp, int group, uint8_t* tiled,
                         int nthreads);

#ifdef __cplusplus
}
#endif

#endif /* MXFP6_GEMM_H */
