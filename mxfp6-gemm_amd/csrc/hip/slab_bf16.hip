// Tile kernel instantiations: BF16 output.
#include "slab_kernel.hpp"

namespace mxfp6_dev {
template int slab_run<__hip_bfloat16, false>(const mxfp6_launch_desc*, hipStream_t);
}  // namespace mxfp6_dev
