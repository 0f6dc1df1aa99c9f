// launch.h — host launchers of the decode-matmul kernels, one translation unit per K
// (kernels_k2.hip, kernels_k3.hip, kernels_k4.hip) so the instantiations build in parallel.
// Every launcher returns 0 or TRELLIS_ERR_LAUNCH.
#pragma once

#include <hip/hip_runtime.h>

#include "bgemm.h"
#include "common.h"
#include "gemv.h"

namespace trellis {

// gemv_kernel<K, cb, V, kc, nb> over g.total items (batch g.batch <= GEMV_MAX_NB, nb the
// smallest of 1, 2, 4, 8, 16 that holds it, gemv_nb; k-ranges of g.kr <= gemv_kr_max(nb)
// tiles).
constexpr int GEMV_MAX_NB = 16;
constexpr int gemv_nb(int batch) { return batch <= 1 ? 1 : batch == 2 ? 2 : batch <= 4 ? 4 : batch <= 8 ? 8 : 16; }
template <int K>
int launch_gemv_k(int cb, int V, int kc, const LinArgs& g, hipStream_t st);

// bgemm_kernel<K, cb, V, nc, g.mma_f16> over g.total items (the x fold has been launched
// before it).
template <int K>
int launch_bgemm_k(int cb, int V, int nc, const LinArgs& g, hipStream_t st);

// bfold_kernel<cb, nc> over nfold (block, column block) jobs of 4 * nc workgroups each
// (after a split-K bgemm_kernel).
int launch_bfold(int cb, int nc, int nfold, const LinArgs& g, hipStream_t st);

#ifdef TRELLIS_BFOLD_DEFINE
template <int CB>
static int launch_bfold_cb(int nc, int nfold, const LinArgs& g, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(nfold * 4 * nc));
  const bool one = g.nmat == 1;
  switch (nc) {
    case 1:
      if (one) hipLaunchKernelGGL((bfold_kernel<CB, 1, true>), grid, dim3(256), 0, st, g);
      else hipLaunchKernelGGL((bfold_kernel<CB, 1, false>), grid, dim3(256), 0, st, g);
      break;
    case 2:
      if (one) hipLaunchKernelGGL((bfold_kernel<CB, 2, true>), grid, dim3(256), 0, st, g);
      else hipLaunchKernelGGL((bfold_kernel<CB, 2, false>), grid, dim3(256), 0, st, g);
      break;
    case 4:
      if (one) hipLaunchKernelGGL((bfold_kernel<CB, 4, true>), grid, dim3(256), 0, st, g);
      else hipLaunchKernelGGL((bfold_kernel<CB, 4, false>), grid, dim3(256), 0, st, g);
      break;
    default:
      if (one) hipLaunchKernelGGL((bfold_kernel<CB, 8, true>), grid, dim3(256), 0, st, g);
      else hipLaunchKernelGGL((bfold_kernel<CB, 8, false>), grid, dim3(256), 0, st, g);
      break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 13;
}

int launch_bfold(int cb, int nc, int nfold, const LinArgs& g, hipStream_t st) {
  switch (cb) {
    case CB_MCG: return launch_bfold_cb<CB_MCG>(nc, nfold, g, st);
    case CB_3INST: return launch_bfold_cb<CB_3INST>(nc, nfold, g, st);
    default: return launch_bfold_cb<CB_1MAD>(nc, nfold, g, st);
  }
}
#endif

#ifdef TRELLIS_KERNELS_INSTANTIATE
template <int K, int CB, int V, int NB>
static int launch_gemv_nb(int kc, const LinArgs& g, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(g.total));
  // 16 rows: stages of 8 tiles (two 16-tile ring slots do not fit beside their activations)
  constexpr int KC_WIDE = NB == 16 ? 8 : 16;
  const bool one = g.nmat == 1;
  if (kc == 8) {
    if (one) hipLaunchKernelGGL((gemv_kernel<K, CB, V, 8, NB, true>), grid, dim3(64 * GEMV_WAVES), 0, st, g);
    else hipLaunchKernelGGL((gemv_kernel<K, CB, V, 8, NB, false>), grid, dim3(64 * GEMV_WAVES), 0, st, g);
  } else {
    if (one) hipLaunchKernelGGL((gemv_kernel<K, CB, V, KC_WIDE, NB, true>), grid, dim3(64 * GEMV_WAVES), 0, st, g);
    else hipLaunchKernelGGL((gemv_kernel<K, CB, V, KC_WIDE, NB, false>), grid, dim3(64 * GEMV_WAVES), 0, st, g);
  }
  return hipGetLastError() == hipSuccess ? 0 : 13;
}

template <int K, int CB, int V>
static int launch_gemv_kc(int kc, const LinArgs& g, hipStream_t st) {
  switch (gemv_nb(g.batch)) {
    case 1: return launch_gemv_nb<K, CB, V, 1>(kc, g, st);
    case 2: return launch_gemv_nb<K, CB, V, 2>(kc, g, st);
    case 4: return launch_gemv_nb<K, CB, V, 4>(kc, g, st);
    case 8: return launch_gemv_nb<K, CB, V, 8>(kc, g, st);
    default: return launch_gemv_nb<K, CB, V, 16>(kc, g, st);
  }
}

template <int K, int CB>
static int launch_gemv_v(int V, int kc, const LinArgs& g, hipStream_t st) {
  return V == 2 ? launch_gemv_kc<K, CB, 2>(kc, g, st) : launch_gemv_kc<K, CB, 1>(kc, g, st);
}

template <int K>
int launch_gemv_k(int cb, int V, int kc, const LinArgs& g, hipStream_t st) {
  switch (cb) {
    case CB_MCG: return launch_gemv_v<K, CB_MCG>(V, kc, g, st);
    case CB_3INST: return launch_gemv_v<K, CB_3INST>(V, kc, g, st);
    default: return launch_gemv_v<K, CB_1MAD>(V, kc, g, st);
  }
}

template <int K, int CB, int V, int F16>
static int launch_bgemm_nc(int nc, const LinArgs& g, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(g.total));
  const bool one = g.nmat == 1;
#define TRELLIS_BG_LAUNCH(NCV) \
  if (one) hipLaunchKernelGGL((bgemm_kernel<K, CB, V, NCV, F16, true>), grid, dim3(64 * BgWaves<NCV, F16>::WV), 0, st, g); \
  else hipLaunchKernelGGL((bgemm_kernel<K, CB, V, NCV, F16, false>), grid, dim3(64 * BgWaves<NCV, F16>::WV), 0, st, g);
  switch (nc) {
    case 1: TRELLIS_BG_LAUNCH(1) break;
    case 2: TRELLIS_BG_LAUNCH(2) break;
    case 4: TRELLIS_BG_LAUNCH(4) break;
    default: TRELLIS_BG_LAUNCH(8) break;
  }
#undef TRELLIS_BG_LAUNCH
  return hipGetLastError() == hipSuccess ? 0 : 13;
}

template <int K, int CB, int V>
static int launch_bgemm_f(int nc, const LinArgs& g, hipStream_t st) {
  return g.mma_f16 ? launch_bgemm_nc<K, CB, V, 1>(nc, g, st) : launch_bgemm_nc<K, CB, V, 0>(nc, g, st);
}

template <int K, int CB>
static int launch_bgemm_v(int V, int nc, const LinArgs& g, hipStream_t st) {
  return V == 2 ? launch_bgemm_f<K, CB, 2>(nc, g, st) : launch_bgemm_f<K, CB, 1>(nc, g, st);
}

template <int K>
int launch_bgemm_k(int cb, int V, int nc, const LinArgs& g, hipStream_t st) {
  switch (cb) {
    case CB_MCG: return launch_bgemm_v<K, CB_MCG>(V, nc, g, st);
    case CB_3INST: return launch_bgemm_v<K, CB_3INST>(V, nc, g, st);
    default: return launch_bgemm_v<K, CB_1MAD>(V, nc, g, st);
  }
}
#endif

}  // namespace trellis
