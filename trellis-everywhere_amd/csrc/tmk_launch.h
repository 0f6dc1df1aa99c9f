// tmk_launch.h — host launchers of the decode-to-MFMA kernels, one translation unit per
// K (tmk_k2.hip, tmk_k3.hip, tmk_k4.hip) so the instantiations build in parallel.
#pragma once

#include <hip/hip_runtime.h>

#include "bgemm.h"
#include "gemv.h"
#include "tmk.h"

namespace trellis {

// tmk_kernel<K, cb, ks> over g.total items (the x fold has been launched before it).
// Returns 0 or a trellis_status code.
template <int K>
int launch_tmk_k(int cb, int ks, const TmkArgs& g, hipStream_t st);

// gemv_kernel<K, cb, kc> over g.total items (batch 1, k-ranges of g.kr tiles).
template <int K>
int launch_gemv_k(int cb, int kc, const TmkArgs& g, hipStream_t st);

// bgemm_kernel<K, cb, nc> over g.total items (the x fold has been launched before it).
template <int K>
int launch_bgemm_k(int cb, int nc, const TmkArgs& g, hipStream_t st);

// bfold_kernel<cb, nc> over nfold workgroups (after a split-K bgemm_kernel).
int launch_bfold(int cb, int nc, int nfold, const TmkArgs& g, hipStream_t st);

#ifdef TRELLIS_BFOLD_DEFINE
template <int CB>
static int launch_bfold_cb(int nc, int nfold, const TmkArgs& g, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(nfold));
  switch (nc) {
    case 1: hipLaunchKernelGGL((bfold_kernel<CB, 1>), grid, dim3(256), 0, st, g); break;
    case 2: hipLaunchKernelGGL((bfold_kernel<CB, 2>), grid, dim3(256), 0, st, g); break;
    case 4: hipLaunchKernelGGL((bfold_kernel<CB, 4>), grid, dim3(256), 0, st, g); break;
    default: hipLaunchKernelGGL((bfold_kernel<CB, 8>), grid, dim3(256), 0, st, g); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 13;
}

int launch_bfold(int cb, int nc, int nfold, const TmkArgs& g, hipStream_t st) {
  switch (cb) {
    case CB_MCG: return launch_bfold_cb<CB_MCG>(nc, nfold, g, st);
    case CB_3INST: return launch_bfold_cb<CB_3INST>(nc, nfold, g, st);
    default: return launch_bfold_cb<CB_1MAD>(nc, nfold, g, st);
  }
}
#endif

#ifdef TRELLIS_TMK_INSTANTIATE
template <int K, int CB, int XB>
static int launch_ks(int ks, const TmkArgs& g, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(g.total));
  switch (ks) {
    case 4: hipLaunchKernelGGL((tmk_kernel<K, CB, 4, XB>), grid, dim3(256), 0, st, g); break;
    case 8: hipLaunchKernelGGL((tmk_kernel<K, CB, 8, XB>), grid, dim3(256), 0, st, g); break;
    case 16: hipLaunchKernelGGL((tmk_kernel<K, CB, 16, XB>), grid, dim3(256), 0, st, g); break;
    default: hipLaunchKernelGGL((tmk_kernel<K, CB, 32, XB>), grid, dim3(256), 0, st, g); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 13;
}

template <int K, int CB>
static int launch_xb(int ks, const TmkArgs& g, hipStream_t st) {
  return g.batch == 1 ? launch_ks<K, CB, 1>(ks, g, st) : launch_ks<K, CB, TMK_MAX_BATCH>(ks, g, st);
}

template <int K>
int launch_tmk_k(int cb, int ks, const TmkArgs& g, hipStream_t st) {
  switch (cb) {
    case CB_MCG: return launch_xb<K, CB_MCG>(ks, g, st);
    case CB_3INST: return launch_xb<K, CB_3INST>(ks, g, st);
    default: return launch_xb<K, CB_1MAD>(ks, g, st);
  }
}

template <int K, int CB>
static int launch_gemv_kc(int kc, const TmkArgs& g, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(g.total));
  if (kc == 8)
    hipLaunchKernelGGL((gemv_kernel<K, CB, 8, GEMV_PF>), grid, dim3(64 * GEMV_WAVES), 0, st, g);
  else
    hipLaunchKernelGGL((gemv_kernel<K, CB, 16, GEMV_PF>), grid, dim3(64 * GEMV_WAVES), 0, st, g);
  return hipGetLastError() == hipSuccess ? 0 : 13;
}

template <int K>
int launch_gemv_k(int cb, int kc, const TmkArgs& g, hipStream_t st) {
  switch (cb) {
    case CB_MCG: return launch_gemv_kc<K, CB_MCG>(kc, g, st);
    case CB_3INST: return launch_gemv_kc<K, CB_3INST>(kc, g, st);
    default: return launch_gemv_kc<K, CB_1MAD>(kc, g, st);
  }
}

template <int K, int CB>
static int launch_bgemm_nc(int nc, const TmkArgs& g, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(g.total));
  switch (nc) {
    case 1: hipLaunchKernelGGL((bgemm_kernel<K, CB, 1>), grid, dim3(256), 0, st, g); break;
    case 2: hipLaunchKernelGGL((bgemm_kernel<K, CB, 2>), grid, dim3(256), 0, st, g); break;
    case 4: hipLaunchKernelGGL((bgemm_kernel<K, CB, 4>), grid, dim3(256), 0, st, g); break;
    default: hipLaunchKernelGGL((bgemm_kernel<K, CB, 8>), grid, dim3(256), 0, st, g); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 13;
}

template <int K>
int launch_bgemm_k(int cb, int nc, const TmkArgs& g, hipStream_t st) {
  switch (cb) {
    case CB_MCG: return launch_bgemm_nc<K, CB_MCG>(nc, g, st);
    case CB_3INST: return launch_bgemm_nc<K, CB_3INST>(nc, g, st);
    default: return launch_bgemm_nc<K, CB_1MAD>(nc, g, st);
  }
}
#endif

}  // namespace trellis
