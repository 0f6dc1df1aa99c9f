// Decode-GEMV kernel instantiations for K=2 bits per weight.
#define TRELLIS_GEMV_INSTANTIATE
#include "gemv_launch.h"

namespace trellis {
template int launch_gemv_k<2>(int, int, int, const GemvGroupArgs&, hipStream_t);
}  // namespace trellis
