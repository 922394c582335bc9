// Tile kernel instantiations: FP16 output.
#include "slab_kernel.hpp"

namespace mxfp6_dev {
template int slab_run<__half, false>(const mxfp6_launch_desc*, hipStream_t);
}  // namespace mxfp6_dev
