// MFMA-only diagnostic of libmxfp6gemm (not a GEMM, never routed; built into libmxfp6diag.so, which
// only bench.py loads): the block-scaled FP6 MFMA stream of a tile kernel with every data path
// taken out, on real operands. It answers two questions a GEMM's timing cannot:
//   * how many shader cycles one v_mfma_scale_f32_32x32x64_f8f6f4 (FP6 x FP6) takes when a wave
//     issues them back to back on independent accumulators (the per-wave s_memtime cycle count
//     over the loop, divided by the MFMAs issued), and
//   * what the board's power limit leaves of the dense MXFP6 peak when every SIMD of the chip runs
//     nothing but MFMAs (the launch's time and the clock it ran at): the practical roof of a GEMM
//     on this board, above which no tile kernel can go whatever its data paths cost.
// Each wave holds MB A operand blocks and NPW B operand blocks (real FP6 codes read once from a
// caller buffer, e.g. a preshuffled B of the benchmark workload) and the scale dwords of its lane,
// and runs `slabs` rounds of MB x NPW MFMAs into MB x NPW accumulators of 32x32 FP32 (AGPRs; one
// wave per SIMD, as the tile kernels). Round r pairs accumulator (i, j) with A block (i + r) % MB
// and B block (j + r) % NPW, so the operands entering every MFMA change from round to round like
// a GEMM's (the switching activity, and so the power, of real data). Lane 0 of each wave stores the
// wave's loop cycle count with an ordinary vector store; the accumulators are stored only when the
// caller asks (acc_out), never in a timing run.
#include "../hip/device_common.hpp"

namespace mxfp6_dev {

template <int MB, int NPW>
__global__ void __launch_bounds__(256, 1)
    mfma_roof_kernel(const uint8_t* __restrict__ ops, int op_blocks,
                     const uint32_t* __restrict__ scales, int scale_dwords,
                     long long* __restrict__ cycles, int slabs, float* __restrict__ acc_out) {
    // the wave id is scalar, and the lane id is recomputed after the loop (mbcnt), so nothing but
    // the operands and scales stays live in VGPRs across it
    const int wid = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    v8i a[MB], b[NPW];
    // the wave's MB + NPW consecutive operand blocks, from a whole group of them in the buffer
    const uint8_t* base =
        ops + (size_t)(wid % (op_blocks / (MB + NPW))) * (MB + NPW) * OPBLK_BYTES;
    auto load_op = [&](v8i& v, int blk) {
        const uint8_t* p = base + blk * OPBLK_BYTES;
        const v4i y0 = *reinterpret_cast<const v4i*>(p + 16 * lane);
        const v2i y1 = *reinterpret_cast<const v2i*>(p + 1024 + 8 * lane);
        // an FP6 operand is 6 dwords; the last two of the 8-dword register tuple are unused
        const v4i y1w = __builtin_shufflevector(y1, y1, 0, 1, -1, -1);
        v = __builtin_shufflevector(y0, y1w, 0, 1, 2, 3, 4, 5, -1, -1);
    };
#pragma unroll
    for (int i = 0; i < MB; i++) load_op(a[i], i);
#pragma unroll
    for (int j = 0; j < NPW; j++) load_op(b[j], MB + j);
    const int sc0 = (int)(((unsigned)wid * 64u) % (unsigned)scale_dwords);
    const int sa = (int)scales[(sc0 + lane) % scale_dwords];
    const int sb = (int)scales[(sc0 + lane + 32) % scale_dwords];

    v16f acc[MB][NPW];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NPW; j++) acc[i][j] = v16f{};

    // one round: every accumulator once, A block (i + R) % MB and B block (j + R) % NPW
    auto round = [&](auto rr) {
        constexpr int R = decltype(rr)::value;
#pragma unroll
        for (int j = 0; j < NPW; j++)
#pragma unroll
            for (int i = 0; i < MB; i++) {
                const v8i& x = a[(i + R) % MB];
                const v8i& y = b[(j + R) % NPW];
                switch ((i % 4) * 4 + j % 4) {
#define ROOF_CASE(SA, SB) \
    case SA * 4 + SB: acc[i][j] = mfma_fp6<SA, SB>(acc[i][j], x, y, sa, sb); break;
                    ROOF_CASE(0, 0) ROOF_CASE(0, 1) ROOF_CASE(0, 2) ROOF_CASE(0, 3)
                    ROOF_CASE(1, 0) ROOF_CASE(1, 1) ROOF_CASE(1, 2) ROOF_CASE(1, 3)
                    ROOF_CASE(2, 0) ROOF_CASE(2, 1) ROOF_CASE(2, 2) ROOF_CASE(2, 3)
                    ROOF_CASE(3, 0) ROOF_CASE(3, 1) ROOF_CASE(3, 2) ROOF_CASE(3, 3)
#undef ROOF_CASE
                }
            }
    };
    const long long t0 = (long long)__builtin_amdgcn_s_memtime();
    int s = 0;
    for (; s + 3 <= slabs; s += 3) {
        round(std::integral_constant<int, 0>{});
        round(std::integral_constant<int, 1>{});
        round(std::integral_constant<int, 2>{});
    }
    for (; s < slabs; s++) round(std::integral_constant<int, 0>{});
    const long long t1 = (long long)__builtin_amdgcn_s_memtime();
    const int l = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    if (l == 0) cycles[wid] = t1 - t0;
    // with `acc_out` the accumulators are stored (block by block, 16 floats per lane, as a tile
    // kernel's FP32 epilogue); a timing run passes none, and the stores are then skipped, but
    // the compiler cannot drop an MFMA whose result it may have to store
    if (acc_out != nullptr) {
        float* o = acc_out + ((size_t)wid * MB * NPW * 64 + l) * 16;
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int j = 0; j < NPW; j++) {
                v4f* d = reinterpret_cast<v4f*>(o + (size_t)(i * NPW + j) * 64 * 16);
#pragma unroll
                for (int q = 0; q < 4; q++)
                    d[q] = v4f{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                               acc[i][j][4 * q + 3]};
            }
    }
}

}  // namespace mxfp6_dev

// grid: `workgroups` workgroups of four waves; every wave issues slabs * MB * NPW MFMAs, each
// 2 * 32 * 32 * 64 flop. ops: op_blocks (>= 11) blocks of 1536 bytes of FP6 operand codes; scales:
// scale_dwords dwords of E8M0 scale bytes; cycles: workgroups * 4 int64 (shader cycles of each
// wave's MFMA loop); acc_out: null (timing), or workgroups * 4 * MB * NPW * 1024 floats that
// receive every wave's accumulators. shape 0: MB 8, NPW 2 (the 256x256 wide tile's
// 16 accumulators per wave); 1: MB 4, NPW 3 (128x384). Returns 0, or 1 on a bad argument or a
// failed launch.
extern "C" int mxfp6_diag_mfma_roof_async(int shape, const void* ops, int op_blocks,
                                          const void* scales, int scale_dwords,
                                          long long* cycles, int workgroups, int slabs,
                                          float* acc_out, void* stream) {
    using namespace mxfp6_dev;
    if (!ops || !scales || !cycles || op_blocks < 11 || scale_dwords < 1 ||
        workgroups < 1 || slabs < 1)
        return 1;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* sc = static_cast<const uint32_t*>(scales);
    const auto* op = static_cast<const uint8_t*>(ops);
    hipError_t e;
    if (shape == 0)
        e = launch_kernel(mfma_roof_kernel<8, 2>, dim3((unsigned)workgroups), dim3(256), st, op,
                          op_blocks, sc, scale_dwords, cycles, slabs, acc_out);
    else if (shape == 1)
        e = launch_kernel(mfma_roof_kernel<4, 3>, dim3((unsigned)workgroups), dim3(256), st, op,
                          op_blocks, sc, scale_dwords, cycles, slabs, acc_out);
    else
        return 1;
    return e == hipSuccess ? 0 : 1;
}
