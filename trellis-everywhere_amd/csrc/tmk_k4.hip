// Decode-to-MFMA kernel instantiations for K=4 bits per weight.
#define TRELLIS_TMK_INSTANTIATE
#include "tmk_launch.h"

namespace trellis {
template int launch_tmk_k<4>(int, int, const TmkArgs&, hipStream_t);
template int launch_gemv_k<4>(int, int, const TmkArgs&, hipStream_t);
template int launch_bgemm_k<4>(int, int, const TmkArgs&, hipStream_t);
}  // namespace trellis
