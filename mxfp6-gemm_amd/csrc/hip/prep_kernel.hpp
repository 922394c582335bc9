// Quantisation and layout kernels: float operands -> the GEMM's device formats in one HBM pass.
//
// The GEMM consumes three formats (reference include/mxfp6/preprocess.hpp):
//   packed rows   FP6 E2M3 codes, 4 codes in 3 bytes LSB-first (types.hpp:97-117), one E8M0
//                 scale per 32 consecutive values of a row (quantize_to_mxfp6, :51-97);
//   preshuffled B B^T quantised (preprocess_B, :112-118), padded to Kp with zero codes and cut into
//                 1536-byte tiles per (32 columns, 64-wide K slab) in MFMA operand order
//                 (preshuffle_B, :182-207): lane t = 32h + i holds column i's 32-block 2q + h,
//                 its first 16 packed bytes at 16t, the last 8 at 1024 + 8t;
//   tiled scales  scales padded to Kp with code 127 (pad_scales_k, :32-38), put in MFMA lane
//                 order (preprocess_scale, :136-162) and grouped (tile_scale(group, 3), :216-233):
//                 the scale of (row r, 32-block c) sits at byte
//                 ((((g * ktn + kt) * 64 + lane) * 3 + sub) * gp + j), with t = r / 32,
//                 lane = r % 32 + 32 * (c % 2), q = c / 2, g = t / group, j = t % group,
//                 kt = q / 3, sub = q % 3, ktn = Kp / 192, gp = group rounded up to 4 (the
//                 gp - group pad bytes of every dword are zero).
//
// Quantisation rule (quantize_to_mxfp6): per 32-block amax = max |x|; a zero block gets code 127;
// otherwise need = amax / 7.5 (FP32 division) and the scale is the smallest power of two >= need,
// code = clamp(log2(scale) + 127, 0, 254). Every value is divided by the scale (here multiplied
// by its reciprocal, a power of two in [2^-126, 2^127]: the same correctly rounded quotient) and
// encoded by float_to_fp6_e2m3 (types.hpp:26-72): magnitude saturated at 7.5, round to nearest
// E2M3 with ties to the even code, sign from q < 0 (so a negative quotient that rounds to zero
// keeps code 0x20, and a zero quotient gives 0x00).
//
// Kernels (all HBM-bound; algorithmic bytes = 4 per value read + 0.75 per value and 1/32 per
// scale written):
//   prep_rows_kernel  row-major float [rows][cols] -> packed rows (+ zero tail up to row_bytes) and
//                     scales, raw [rows][scale_cols] (tail columns 127) or tiled at Kp. A
//                     one-wave workgroup takes 64 consecutive 32-blocks of one row: coalesced
//                     float4 loads into LDS, then lane l quantises block l; the chunk's 1536
//                     packed bytes go back through LDS and out as 16-byte stores (6 strided
//                     dword stores per lane before: 82 -> 65 us at 8192 x 8192).
//   prep_rows_preshuffled_kernel  row-major float A -> the preshuffled operand layout + tiled
//                     scales: a workgroup stages 32 rows x 4 slabs in LDS, each wave then writes
//                     one whole 1536-byte tile (lane t: row t % 32, 32-block half t / 32).
//   prep_b_kernel     row-major float B [K][N] -> preshuffled B^T at Kp + tiled scales. Lane n of
//                     a wave takes column n and one 32-block: 32 loads each coalesced across the
//                     wave's 64 consecutive columns; its 24 bytes land at 16t / 1024 + 8t of the
//                     column's tile, so the wave's stores are contiguous too.
//   tile_scales_kernel raw scales [dim][ld] (ceil(K/32) valid columns) -> tiled at Kp.
#pragma once
#include "device_common.hpp"

namespace mxfp6_dev {

// Scale code of a 32-block from its amax (quantize_to_mxfp6, preprocess.hpp:62-94).
__device__ __forceinline__ int mx_scale_code(float amax) {
    if (amax == 0.0f) return 127;
    const float need = amax / 7.5f;
    int e;
    const float sig = __builtin_frexpf(need, &e);  // need = sig * 2^e, sig in [0.5, 1)
    if (sig == 0.5f) e -= 1;                       // an exact power of two is its own scale
    return min(max(e + 127, 0), 254);
}

// 1 / 2^(code - 127) for codes 0..253 (a normal float; code 254 needs amax > FLT_MAX).
__device__ __forceinline__ float inv_scale(int code) {
    return __uint_as_float((uint32_t)(254 - code) << 23);
}

// The quotient x / scale as the reference forms it, with -0.0 turned into +0.0: the reference
// takes the sign from q < 0, so a zero quotient always encodes as code 0x00, while the hardware
// conversion keeps the sign bit of -0.0. A nonzero quotient is unchanged by + 0.0, and the
// product is not contracted into an FMA (which would keep the sign of an underflowing product).
__device__ __forceinline__ float scaled_quotient(float x, float inv) {
#pragma clang fp contract(off)
    return x * inv + 0.0f;
}

// Quantise 32 values into 6 packed dwords (code i at bits 6i .. 6i+5, LSB-first); returns the
// scale code. The E2M3 encoding is v_cvt_scalef32_2xpk16_fp6_f32 (scale 1.0) on the quotients:
// round to nearest with ties to even, magnitude saturated at 7.5, the sign kept for a value that
// rounds to zero -- float_to_fp6_e2m3 (types.hpp:26-72) exactly; the instruction interleaves its
// two 16-value sources (output i comes from source i % 2, element i / 2).
__device__ __forceinline__ int quant32(const float (&v)[32], uint32_t (&w)[6]) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const int code = mx_scale_code(amax);
    const float inv = inv_scale(code);
    v16f even, odd;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        even[i] = scaled_quotient(v[2 * i], inv);
        odd[i] = scaled_quotient(v[2 * i + 1], inv);
    }
    const v6u h = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(even, odd, 1.0f);
#pragma unroll
    for (int d = 0; d < 6; d++) w[d] = h[d];
    return code;
}

// Byte offset of the tiled scale of (row r, 32-block c); see the file comment.
__device__ __forceinline__ size_t tiled_scale_off(int r, int c, int group, int gp, int ktn) {
    const int t = r >> 5, lane = (r & 31) + ((c & 1) << 5), q = c >> 1;
    const int g = t / group, j = t - g * group, kt = q / 3, sub = q - kt * 3;
    return ((((size_t)g * ktn + kt) * 64 + lane) * 3 + sub) * gp + j;
}

// Store one tiled scale byte; the last row block of a group also clears the dword's pad bytes.
__device__ __forceinline__ void put_tiled_scale(uint8_t* tiled, int r, int c, int group, int ktn,
                                                int code) {
    const int gp = (group + 3) & ~3;
    const size_t o = tiled_scale_off(r, c, group, gp, ktn);
    tiled[o] = (uint8_t)code;
    if (((r >> 5) % group) == group - 1)
        for (int j = 1; j < gp - group + 1; j++) tiled[o + j] = 0;
}

constexpr int PREP_THREADS = 256;
constexpr int PREP_BLKS_PER_WAVE = 64;

// Scale output of prep_rows_kernel: raw [rows][ncols] or tiled (group, ktn) with ncols = Kp / 32.
struct ScaleOut {
    uint8_t* p;
    int tiled;       // 0 raw, 1 tiled
    int ncols;       // scale columns written per row (raw: also the row stride)
    int group, ktn;  // tiled
};

// Packed output of prep_rows_kernel: row-major rows of row_bytes (k64n == 0), or the preshuffled
// operand layout (k64n > 0 slabs per 32-row block; rows32 = rows rounded up to 32, the rows past the
// data written as zero codes).
struct PackedOut {
    uint8_t* p;
    size_t row_bytes;
    int k64n, rows32;
};

// Packed codes of block c of row r and its scale column c (if c < so.ncols). Row-major: bytes
// [24c, 24c + 24) of the row, cut at row_bytes (a multiple of 4), data rows only. Preshuffled:
// the block's 24 bytes at 16t and 1024 + 8t of tile (r / 32, c / 2), t = r % 32 + 32 (c % 2).
__device__ __forceinline__ void put_block(const PackedOut& po, const ScaleOut& so, int r, int c,
                                          bool data, const uint32_t (&w)[6], int code) {
    if (po.k64n > 0) {
        if (r < po.rows32 && c < 2 * po.k64n) {
            const int t = (r & 31) + ((c & 1) << 5);
            uint8_t* tile = po.p + ((size_t)(r >> 5) * po.k64n + (c >> 1)) * OPBLK_BYTES;
            *reinterpret_cast<v4i*>(tile + 16 * t) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            *reinterpret_cast<v2i*>(tile + 1024 + 8 * t) = v2i{(int)w[4], (int)w[5]};
        }
    } else {
        const size_t o = (size_t)24 * c;
        if (data && o < po.row_bytes) {
            uint32_t* dst = reinterpret_cast<uint32_t*>(po.p + (size_t)r * po.row_bytes + o);
            const int nd = (int)min((size_t)6, (po.row_bytes - o) / 4);
#pragma unroll
            for (int d = 0; d < 6; d++)
                if (d < nd) dst[d] = w[d];
        }
    }
    if (c < so.ncols) {
        if (so.tiled)
            put_tiled_scale(so.p, r, c, so.group, so.ktn, code);
        else
            so.p[(size_t)r * so.ncols + c] = (uint8_t)code;
    }
}

// One wave per workgroup (no barrier across waves); workgroup = task (row r, chunk), row-major,
// r < rows_out, chunk < chunks = ceil(vblk / 64) with vblk = ceil(cols / 32) the blocks holding
// values. A task quantises the value blocks 64 chunk .. +63 of its row (lane l: block
// 64 chunk + l); the last chunk also writes the blocks vblk .. nblk-1 past the values (zero
// codes, scale 127), so no workgroup is spent on a K-tail alone. Rows rows .. rows_out-1 are zero
// rows that complete the last 32-row block of a preshuffled output and the last scale group of a
// tiled one (zero codes, scale 127). Block c of row r (c < nblk) writes the codes of values
// 32c .. 32c+31 (zero past cols) as put_block places them, and the scale column c if
// c < so.ncols. V4: cols % 4 == 0 and x 16-byte aligned (float4 loads);
// otherwise one float per lane per load.
template <bool V4>
__global__ void __launch_bounds__(64)
    prep_rows_kernel(const float* __restrict__ x, int cols, int nblk, PackedOut po, ScaleOut so,
                     int chunks, int rows) {
    constexpr int BPW = PREP_BLKS_PER_WAVE;  // blocks per task, one per lane
    __shared__ __attribute__((aligned(16))) float stage[BPW * 33];
    const int lane = threadIdx.x;
    const int r = (int)(blockIdx.x / (unsigned)chunks);
    const int chunk = (int)(blockIdx.x - (unsigned)r * chunks);
    const bool data = r < rows;
    const int blk0 = chunk * BPW;
    const int vblk = (cols + 31) / 32;
    const float* xr = x + (size_t)r * cols;
    // coalesced loads of the task's values, block-padded in LDS
    if (data) {
        if constexpr (V4) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int p = 4 * (lane + 64 * j);  // value index within the task's range
                const int b = p >> 5, i = p & 31, e = blk0 * 32 + p;
                v4f v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (e < cols) v = *reinterpret_cast<const v4f*>(xr + e);
                stage[b * 33 + i] = v[0];
                stage[b * 33 + i + 1] = v[1];
                stage[b * 33 + i + 2] = v[2];
                stage[b * 33 + i + 3] = v[3];
            }
        } else {
#pragma unroll 8
            for (int j = 0; j < 32; j++) {
                const int p = lane + 64 * j, e = blk0 * 32 + p;
                stage[(p >> 5) * 33 + (p & 31)] = e < cols ? xr[e] : 0.0f;
            }
        }
    }
    __syncthreads();
    const int c = blk0 + lane;
    // a whole chunk of value blocks into 16-byte aligned row-major rows: staged in LDS and stored
    // as 16-byte contiguous pieces
    const bool full = po.k64n == 0 && data && (po.row_bytes % 16) == 0 && blk0 + BPW <= vblk &&
                      (size_t)24 * (blk0 + BPW) <= po.row_bytes;
    if (full) {
        uint32_t w[6];
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = stage[lane * 33 + i];
        const int code = quant32(v, w);
        __syncthreads();
        uint32_t* ob = reinterpret_cast<uint32_t*>(stage);
#pragma unroll
        for (int d = 0; d < 6; d++) ob[lane * 6 + d] = w[d];
        __syncthreads();
        uint8_t* dst = po.p + (size_t)r * po.row_bytes + (size_t)24 * blk0;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int q = lane + 64 * k;
            if (q < BPW * 24 / 16)
                *reinterpret_cast<v4i*>(dst + 16 * q) = *reinterpret_cast<const v4i*>(ob + 4 * q);
        }
        if (c < so.ncols) {
            if (so.tiled)
                put_tiled_scale(so.p, r, c, so.group, so.ktn, code);
            else
                so.p[(size_t)r * so.ncols + c] = (uint8_t)code;
        }
    } else if (c < nblk) {
        uint32_t w[6] = {0, 0, 0, 0, 0, 0};
        int code = 127;
        if (data && c < vblk) {
            float v[32];
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = stage[lane * 33 + i];
            code = quant32(v, w);
        }
        put_block(po, so, r, c, data, w, code);
    }
    if (chunk == chunks - 1) {
        const uint32_t z[6] = {0, 0, 0, 0, 0, 0};
        for (int cz = blk0 + BPW + lane; cz < nblk; cz += 64)
            put_block(po, so, r, cz, data, z, 127);
    }
}

// Row-major float A -> the preshuffled operand layout, one output tile per wave. Workgroup
// (32-row block mb, 4 slabs from s0 = 4 * blockIdx.x): its 32 rows x 256 values are loaded with
// coalesced float4 loads (each row's 1 KiB contiguous) into LDS; wave w then quantises slab s0 + w:
// lane t = 32h + i takes row 32mb + i, 32-block 2(s0 + w) + h, and its 24 bytes land at 16t and
// 1024 + 8t of tile (mb, s0 + w), so each wave writes one whole 1536-byte tile with two
// contiguous stores. Rows >= rows (up to the 32-row block) and values >= cols are zeros; the
// scales go to the tiled layout (scale_mode 1) as in prep_rows_kernel, rows up to the group
// multiple written by the workgroups of the extra blocks (grid.y = ceil(rows_out / 32)).
// V4: cols % 4 == 0 and x 16-byte aligned.
constexpr int PSH_SLABS = 4;
template <bool V4>
__global__ void __launch_bounds__(64 * PSH_SLABS)
    prep_rows_preshuffled_kernel(const float* __restrict__ x, int rows, int cols, int k64n,
                                 uint8_t* __restrict__ ash, int rows32, ScaleOut so) {
    constexpr int BLK = 2 * PSH_SLABS;  // 32-value blocks per row in the workgroup's range
    // rows BLK * 33 + 1 dwords apart: the quantising reads (lane = row i, block half h) then hit
    // distinct banks for the 32 rows (a stride of BLK * 33 = 264 mapped rows i and i + 8 to one
    // bank: 79 -> 68 us at 8192 x 8192)
    __shared__ float stage[32][BLK * 33 + 1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int mb = blockIdx.y, s0 = blockIdx.x * PSH_SLABS;
    const int c0 = 2 * s0;  // first block
    // loads: wave w takes rows 8w .. 8w+7; per row 256 values = 64 float4, one per lane
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = wave * 8 + j, r = mb * 32 + i;
        const int p = 4 * lane;  // value index in the row's range
        const int e = c0 * 32 + p;
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (r < rows) {
            const float* xr = x + (size_t)r * cols;
            if constexpr (V4) {
                if (e < cols) {
                    const v4f q = *reinterpret_cast<const v4f*>(xr + e);
                    v[0] = q[0], v[1] = q[1], v[2] = q[2], v[3] = q[3];
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (e + k < cols) v[k] = xr[e + k];
            }
        }
        const int b = p >> 5, o = p & 31;
#pragma unroll
        for (int k = 0; k < 4; k++) stage[i][b * 33 + o + k] = v[k];
    }
    __syncthreads();
    const int s = s0 + wave;
    if (s >= k64n) return;
    const int i = lane & 31, h = lane >> 5, r = mb * 32 + i, c = 2 * s + h;
    const int vblk = (cols + 31) / 32;
    uint32_t w[6] = {0, 0, 0, 0, 0, 0};
    int code = 127;
    if (r < rows && c < vblk) {
        float v[32];
#pragma unroll
        for (int k = 0; k < 32; k++) v[k] = stage[i][(2 * wave + h) * 33 + k];
        code = quant32(v, w);
    }
    if (r < rows32) {
        uint8_t* tile = ash + ((size_t)mb * k64n + s) * OPBLK_BYTES;
        *reinterpret_cast<v4i*>(tile + 16 * lane) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        *reinterpret_cast<v2i*>(tile + 1024 + 8 * lane) = v2i{(int)w[4], (int)w[5]};
    }
    if (c < so.ncols) put_tiled_scale(so.p, r, c, so.group, so.ktn, code);
}

// grid: nchunks * kchunks workgroups, nchunks = ceil(NG / 256), kchunks = Kp / 32: workgroup
// (nb, kc) = 32-block kc of 256 consecutive columns, 64 per wave, K-block major (the four waves
// read 1 KiB of each row together: 60 -> 56 us at 8192 x 8192 against 64 columns x 4 blocks).
// Columns N .. NG-1 (NG = N rounded up to whole scale groups of 32 * group columns) are zero
// columns: they complete the last 32-column tile of bsh and the last scale group. Values past K
// in the last 32-block are zero.
__global__ void __launch_bounds__(PREP_THREADS)
    prep_b_kernel(const float* __restrict__ B, int K, int N, int NG, int Kp, int group,
                  uint8_t* __restrict__ bsh, uint8_t* __restrict__ tiled, int nchunks) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int kc = (int)(blockIdx.x / nchunks), nb = (int)(blockIdx.x - (unsigned)kc * nchunks);
    const int n = nb * PREP_THREADS + wave * 64 + lane;
    const int c = kc;
    if (c >= Kp / 32 || n >= NG) return;
    uint32_t w[6] = {0, 0, 0, 0, 0, 0};
    int code = 127;
    if (n < N && 32 * c < K) {
        float v[32];
        const float* src = B + (size_t)32 * c * N + n;
        const int kv = min(32, K - 32 * c);  // values of this block
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = i < kv ? src[(size_t)i * N] : 0.0f;
        code = quant32(v, w);
    }
    if (n < (N + 31) / 32 * 32) {
        const int k64n = Kp / 64, t = (n & 31) + ((c & 1) << 5);
        uint8_t* tile = bsh + ((size_t)(n >> 5) * k64n + (c >> 1)) * OPBLK_BYTES;
        *reinterpret_cast<v4i*>(tile + 16 * t) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        *reinterpret_cast<v2i*>(tile + 1024 + 8 * t) = v2i{(int)w[4], (int)w[5]};
    }
    put_tiled_scale(tiled, n, c, group, Kp / 192, code);
}

// grid-stride over dim_out * Kp/32 (row-major over (r, c)); rows dim .. dim_out-1 complete the
// last scale group (code 127, zero values).
__global__ void __launch_bounds__(PREP_THREADS)
    tile_scales_kernel(const uint8_t* __restrict__ s, int dim, int dim_out, int vblk, int ld,
                       int Kp, int group, uint8_t* __restrict__ tiled) {
    const int nb = Kp / 32;
    const size_t total = (size_t)dim_out * nb;
    for (size_t e = (size_t)blockIdx.x * PREP_THREADS + threadIdx.x; e < total;
         e += (size_t)gridDim.x * PREP_THREADS) {
        const int r = (int)(e / nb), c = (int)(e - (size_t)r * nb);
        const int code = (r < dim && c < vblk) ? s[(size_t)r * ld + c] : 127;
        put_tiled_scale(tiled, r, c, group, Kp / 192, code);
    }
}

}  // namespace mxfp6_dev
