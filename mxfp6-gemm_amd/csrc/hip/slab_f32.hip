// Tile kernel instantiations: FP32 output.
#include "slab_kernel.hpp"

namespace mxfp6_dev {
template int slab_run<float, false>(const mxfp6_launch_desc*, hipStream_t);
}  // namespace mxfp6_dev
