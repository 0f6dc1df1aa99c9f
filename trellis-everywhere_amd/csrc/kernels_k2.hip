// Decode-matmul kernel instantiations for K=2 bits per weight.
#define TRELLIS_KERNELS_INSTANTIATE
#include "launch.h"

namespace trellis {
template int launch_gemv_k<2>(int, int, int, const LinArgs&, hipStream_t);
template int launch_bgemm_k<2>(int, int, int, const LinArgs&, hipStream_t);
}  // namespace trellis
