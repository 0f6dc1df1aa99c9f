// gemv_launch.h — host launchers of the persistent grouped decode-GEMV, one translation
// unit per K (gemv_k2.hip, gemv_k3.hip, gemv_k4.hip) so the instantiations build in
// parallel.
#pragma once

#include <hip/hip_runtime.h>

#include "gemv.h"

namespace trellis {

// Launch gemv_group_kernel<K, cb, nb, tpw> (nb in {1,2,4,8}, tpw in {4,8}) on a
// persistent grid of min(items, CUs x resident workgroups per CU). Returns 0 or a
// trellis_status code.
template <int K>
int launch_gemv_k(int cb, int nb, int tpw, const GemvGroupArgs& g, hipStream_t st);

#ifdef TRELLIS_GEMV_INSTANTIATE
inline int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  return cus;
}

template <int K, int CB, int NB, int TPW>
static int launch_one(const GemvGroupArgs& g, hipStream_t st) {
  // resident workgroups per CU of this instantiation (registers/LDS limited), cached
  static int per_cu = 0;
  if (per_cu == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_group_kernel<K, CB, NB, TPW>, 256, 0) !=
            hipSuccess || n < 1)
      n = 1;
    per_cu = n < 4 ? n : 4;
  }
  int cus = device_cus();
  if (cus <= 0) return 13;
  long long grid = static_cast<long long>(cus) * per_cu;
  if (grid > g.total) grid = g.total;
  hipLaunchKernelGGL((gemv_group_kernel<K, CB, NB, TPW>), dim3(static_cast<unsigned>(grid)),
                     dim3(256), 0, st, g);
  return hipGetLastError() == hipSuccess ? 0 : 13;
}

template <int K, int CB, int NB>
static int launch_tpw(int tpw, const GemvGroupArgs& g, hipStream_t st) {
  return tpw == 4 ? launch_one<K, CB, NB, 4>(g, st) : launch_one<K, CB, NB, 8>(g, st);
}

template <int K, int CB>
static int launch_nb(int nb, int tpw, const GemvGroupArgs& g, hipStream_t st) {
  switch (nb) {
    case 1: return launch_tpw<K, CB, 1>(tpw, g, st);
    case 2: return launch_tpw<K, CB, 2>(tpw, g, st);
    case 4: return launch_tpw<K, CB, 4>(tpw, g, st);
    default: return launch_tpw<K, CB, 8>(tpw, g, st);
  }
}

template <int K>
int launch_gemv_k(int cb, int nb, int tpw, const GemvGroupArgs& g, hipStream_t st) {
  switch (cb) {
    case CB_MCG: return launch_nb<K, CB_MCG>(nb, tpw, g, st);
    case CB_3INST: return launch_nb<K, CB_3INST>(nb, tpw, g, st);
    default: return launch_nb<K, CB_1MAD>(nb, tpw, g, st);
  }
}
#endif

}  // namespace trellis
