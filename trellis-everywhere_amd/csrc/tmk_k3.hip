// Decode-to-MFMA kernel instantiations for K=3 bits per weight.
#define TRELLIS_TMK_INSTANTIATE
#include "tmk_launch.h"

namespace trellis {
template int launch_tmk_k<3>(int, int, const TmkArgs&, hipStream_t);
template int launch_gemv_k<3>(int, int, const TmkArgs&, hipStream_t);
template int launch_bgemm_k<3>(int, int, const TmkArgs&, hipStream_t);
}  // namespace trellis
