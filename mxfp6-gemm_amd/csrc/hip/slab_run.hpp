// Declarations of the tile kernel's launch entry (definitions in slab_kernel.hpp). The launch
// code of each kernel output type is compiled in a translation unit of its own (slab_split.hip,
// slab_f32.hip, slab_f16.hip, slab_bf16.hip), so the instantiations build in parallel and
// launch.hip compiles none of them.
#pragma once
#include "../hip_layer.h"
#include "device_common.hpp"

namespace mxfp6_dev {

// (MT, NT, MPW, NPW) -> wave grid: the scale grouping fixes how many 32-blocks one wave holds,
// so it also selects between the 4-wave and 8-wave instantiation of a tile.
inline bool tile_supported(int MT, int NT, int mpw, int npw) {
    return (MT == 32 && NT == 32 && mpw == 1 && npw == 1) ||  // tiny_kernel.hpp (launch.hip)
           (MT == 32 && NT == 128 && mpw == 1 && npw == 1) ||
           (MT == 32 && NT == 256 && mpw == 1 && npw == 2) ||
           (MT == 64 && NT == 128 && mpw == 2 && npw == 1) ||
           (MT == 64 && NT == 256 && mpw == 2 && npw == 2) ||
           (MT == 128 && NT == 128 && mpw == 2 && npw == 2) ||
           (MT == 128 && NT == 256 && mpw == 2 && npw == 4) ||
           (MT == 128 && NT == 384 && mpw == 4 && npw == 3) ||
           (MT == 128 && NT == 512 && mpw == 4 && npw == 4) ||
           (MT == 128 && NT == 256 && mpw == 4 && npw == 2) ||
           (MT == 256 && NT == 256 && mpw == 4 && npw == 2) ||
           (MT == 256 && NT == 256 && mpw == 4 && npw == 4) ||
           (MT == 256 && NT == 192 && mpw == 4 && npw == 3) ||
           (MT == 256 && NT == 256 && mpw == 2 && npw == 4);
}

// Runs the descriptor's plan on the tile kernel (after the A repack when a_layout asks for it):
// KT = the kernel's output type, SPLIT = FP32 partials of d->splits K segments into d->ws (KT =
// float). Returns 0, 1 when no instantiation matches the tile, 2 when a launch fails.
template <typename KT, bool SPLIT>
int slab_run(const mxfp6_launch_desc* d, hipStream_t st);

extern template int slab_run<float, true>(const mxfp6_launch_desc*, hipStream_t);
extern template int slab_run<float, false>(const mxfp6_launch_desc*, hipStream_t);
extern template int slab_run<__half, false>(const mxfp6_launch_desc*, hipStream_t);
extern template int slab_run<__hip_bfloat16, false>(const mxfp6_launch_desc*, hipStream_t);

}  // namespace mxfp6_dev
