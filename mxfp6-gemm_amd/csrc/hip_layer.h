/* Internal C ABI between the device-free host plan (csrc/host, plain C++) and the HIP launch
 * layer (csrc/hip). The host plan decides tile, split and checks every argument; the HIP layer
 * only maps the plan onto a kernel instantiation, a grid and a stream. */
#ifndef MXFP6_HIP_LAYER_H
#define MXFP6_HIP_LAYER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* How the tile kernel finds A. */
enum mxfp6_a_layout {
    MXFP6_A_ROWS = 0,
    MXFP6_A_REPACK = 1,
    MXFP6_A_PRESHUFFLED = 2,
    MXFP6_A_ROWS_SWIZZLED = 3
};

/* Kernel families of the HIP layer. */
enum mxfp6_kernel_id {
    MXFP6_KERNEL_DIRECT = 0, /* one wave per 32x32 block, operands straight from global memory */
    MXFP6_KERNEL_TILE = 1    /* LDS-pipelined tile kernel, tile given by (MT, NT) */
};

typedef struct mxfp6_launch_desc {
    int kernel;        /* mxfp6_kernel_id */
    int out_type;      /* 0 FP32, 1 FP16, 2 BF16 */
    int M, N, Kp;      /* Kp % 192 == 0 */
    int MT, NT;        /* workgroup tile (MXFP6_KERNEL_TILE) */
    int mpw, npw;      /* scale grouping of sA / sB (32-blocks per group) */
    int splits;        /* K segments; > 1 writes FP32 partials to ws then reduces into D */
    int A_row_bytes;
    const void* A;
    const void* Bsh;
    const uint8_t* sA;
    const uint8_t* sB;
    void* D;
    float* ws;         /* splits * M * N floats when splits > 1 */
    int a_layout;      /* MXFP6_A_ROWS: A row-major (A_row_bytes per row);
                          MXFP6_A_REPACK: repack A into Ash first, the kernel reads Ash;
                          MXFP6_A_PRESHUFFLED: A is already in the preshuffled operand layout;
                          MXFP6_A_ROWS_SWIZZLED: row-major A, staged in LDS in 12-byte units
                          (wide tiles that divide M x N, plain stores; explicit plans only) */
    void* Ash;         /* MXFP6_A_REPACK: M * packed(Kp) bytes */
    int out_stream;    /* 1: the wide tile kernel writes D with nontemporal stores (unsplit plans
                          whose D would evict the operands from the last-level cache) */
    void* stream;      /* hipStream_t */
} mxfp6_launch_desc;

/* Returns 0 on success, 1 when no kernel instantiation matches the descriptor, 2 when the HIP
 * runtime reports a launch error. */
int mxfp6_hip_launch(const mxfp6_launch_desc* d);

/* Repacks rows (rows % 32 == 0) of a row-major packed operand, read for packed(Kp) bytes each,
 * into the preshuffled operand layout at dst (rows * packed(Kp) bytes). 0 ok, 2 launch error. */
int mxfp6_hip_repack(const void* src, int row_bytes, int rows, int Kp, void* dst, void* stream);

/* The no-allocation scratch of the current device (csrc/hip/scratch.hip): its device address,
 * read with hipGetSymbolAddress on the first call per device, and its size in *bytes; NULL when
 * the runtime cannot provide it. */
void* mxfp6_hip_scratch(size_t* bytes);

/* Clock sample (see mxfp6_clock_sample_async in include/mxfp6_gemm.h). 0 ok, 2 launch error. */
int mxfp6_hip_clock_sample(uint64_t* out, int nwg, void* stream);

/* Compute units of the current HIP device (hipDeviceAttributeMultiprocessorCount, read once per
 * device), or 0 when the runtime reports no device. */
int mxfp6_hip_device_cus(void);

/* Calls launch(ctx) `warm` times, then `reps` times between two events recorded on `stream`, and
 * waits for the second: *ms = the mean time per call. Returns 0, 2 on a HIP error, or launch's
 * own nonzero status. */
int mxfp6_hip_time(int (*launch)(void* ctx), void* ctx, void* stream, int warm, int reps, float* ms);

/* Whether the tile kernel has an instantiation for MT x NT with scale grouping (mpw, npw). */
int mxfp6_hip_has_tile(int MT, int NT, int mpw, int npw);

/* Quantisation and layout kernels (csrc/hip/prep_kernel.hpp). All return 0 ok, 2 launch error.
 *
 * Row-major float x[rows][cols] (4-byte aligned; 16-byte aligned with cols % 4 == 0 reads float4):
 * for each row r and block c < nblk, the codes of values 32c .. 32c+31 (zero past cols; zero bytes
 * for a block past the values) go to packed + r * row_bytes + 24c, cut at row_bytes (row_bytes % 4
 * == 0) -- or, with preshuffled != 0, to the preshuffled operand layout at Kp (nblk = Kp / 32,
 * ceil(rows / 32) 32-row blocks, the rows past `rows` zero codes); scale column c < ncols goes to
 * scales[r * ncols + c] (scale_mode 0) or to the tile_scale(group, 3) layout at Kp (scale_mode 1,
 * ncols = Kp / 32), code 127 for a block without values. */
int mxfp6_hip_quantize_rows(const float* x, int rows, int cols, int nblk, void* packed,
                            size_t row_bytes, int preshuffled, uint8_t* scales, int scale_mode,
                            int ncols, int group, int Kp, void* stream);

/* Row-major float B[K][N] -> preshuffled B^T at Kp (N/32 * Kp/64 * 1536 bytes) and its scales
 * in the tile_scale(group, 3) layout at Kp. N % (32 * group) == 0. */
int mxfp6_hip_prepare_b(const float* B, int K, int N, int Kp, int group, void* bsh,
                        uint8_t* tiled, void* stream);

/* Raw scales s[dim][ld] (vblk valid columns) -> tile_scale(group, 3) layout at Kp. */
int mxfp6_hip_tile_scales(const uint8_t* s, int dim, int vblk, int ld, int Kp, int group,
                          uint8_t* tiled, void* stream);

#ifdef __cplusplus
}
#endif

#endif
