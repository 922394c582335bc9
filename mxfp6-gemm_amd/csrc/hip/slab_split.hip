// Tile kernel instantiations: split-K FP32 partials (every output type).
#include "slab_kernel.hpp"

namespace mxfp6_dev {
template int slab_run<float, true>(const mxfp6_launch_desc*, hipStream_t);
}  // namespace mxfp6_dev
