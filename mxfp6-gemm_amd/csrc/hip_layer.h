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
enum mxfp6_a_layout { MXFP6_A_ROWS = 0, MXFP6_A_REPACK = 1, MXFP6_A_PRESHUFFLED = 2 };

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
                          MXFP6_A_PRESHUFFLED: A is already in the preshuffled operand layout */
    void* Ash;         /* MXFP6_A_REPACK: M * packed(Kp) bytes */
    void* stream;      /* hipStream_t */
} mxfp6_launch_desc;

/* Returns 0 on success, 1 when no kernel instantiation matches the descriptor, 2 when the HIP
 * runtime reports a launch error. */
int mxfp6_hip_launch(const mxfp6_launch_desc* d);

/* Repacks rows (rows % 32 == 0) of a row-major packed operand, read for packed(Kp) bytes each,
 * into the preshuffled operand layout at dst (rows * packed(Kp) bytes). 0 ok, 2 launch error. */
int mxfp6_hip_repack(const void* src, int row_bytes, int rows, int Kp, void* dst, void* stream);

/* Whether the tile kernel has an instantiation for MT x NT with scale grouping (mpw, npw). */
int mxfp6_hip_has_tile(int MT, int NT, int mpw, int npw);

#ifdef __cplusplus
}
#endif

#endif
