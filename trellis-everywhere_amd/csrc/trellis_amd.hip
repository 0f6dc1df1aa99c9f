// trellis_amd.hip — C ABI (include/trellis_amd.h) and launchers of the gfx950 trellis
// kernels: the bit-exact tile decode and the fused decode-GEMV.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>

#include "trellis_amd.h"
#include "decode.h"
#include "gemv.h"

using namespace trellis;

namespace {

// ---------------------------------------------------------------- decode kernel
// One thread per tile row: the same window + codebook code the matmul kernels run,
// storing each value's exact fp32 (the fp16 halves summed in fp32).
template <int K, int CB, int PAR>
__device__ __forceinline__ void decode_tile_row(const uint32_t* tp, int nw, int r, float* out) {
  const int w0 = row_word0<K>(r);
  const uint32_t W0 = tp[w0];
  const uint32_t W1 = tp[(w0 + 1) % nw];
  const uint32_t W2 = tp[(w0 + 2) % nw];
  float v[16];
  decode_row<K, PAR, CB>(W0, W1, W2, [&](int c, uint32_t raw) { v[c] = cb_exact<CB>(raw); });
  float4* o = reinterpret_cast<float4*>(out);
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

template <int K, int CB>
__global__ __launch_bounds__(256) void decode_tiles_kernel(const uint32_t* __restrict__ bits,
                                                           int nw, uint32_t tile0, uint32_t ntiles,
                                                           float* __restrict__ out) {
  const uint32_t lt = blockIdx.x * 16u + (threadIdx.x >> 4);
  const int r = threadIdx.x & 15;
  if (lt >= ntiles) return;
  const uint32_t* tp = bits + static_cast<size_t>(tile0 + lt) * nw;
  float* o = out + static_cast<size_t>(lt) * 256 + r * 16;
  if (r & 1)
    decode_tile_row<K, CB, 1>(tp, nw, r, o);
  else
    decode_tile_row<K, CB, 0>(tp, nw, r, o);
}

// ---------------------------------------------------------------- validation
bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

int fit_block(int d, int cap) {
  int b = 1;
  while (b < cap && d % (b * 2) == 0) b *= 2;
  return b;
}

int validate(const trellis_desc* W) {
  if (!W || !W->bits) return TRELLIS_ERR_NULL;
  if (W->n_out <= 0 || W->k_in <= 0 || W->n_out % 16 || W->k_in % 16) return TRELLIS_ERR_SHAPE;
  if (W->K < 2 || W->K > 4) return TRELLIS_ERR_K;
  if (W->V != 1) return TRELLIS_ERR_V;
  if (W->codebook < 0 || W->codebook > 2) return TRELLIS_ERR_CODEBOOK;
  if (W->nwords != 256 * W->K / 32) return TRELLIS_ERR_NWORDS;
  if (!is_pow2(W->block_in) || W->block_in < 16 || W->block_in > 128 || W->k_in % W->block_in)
    return TRELLIS_ERR_BLOCK;
  if (!is_pow2(W->block_out) || W->block_out < 16 || W->block_out > 128 ||
      W->n_out % W->block_out)
    return TRELLIS_ERR_BLOCK;
  if (reinterpret_cast<uintptr_t>(W->bits) % 16) return TRELLIS_ERR_ALIGN;
  return TRELLIS_OK;
}

int validate_fold(const trellis_desc* W) {
  if (!W->su || !W->sv || !W->isc_scaled || !W->osc) return TRELLIS_ERR_NULL;
  return TRELLIS_OK;
}

// ---------------------------------------------------------------- GEMV plan
constexpr int GEMV_MAX_NB = 8;
constexpr int GEMV_MAX_KS = 64;

struct GemvPlan {
  int nb;     // batch rows per launch (1, 2, 4, 8)
  int kS;     // tile columns per workgroup
  int S;      // k-slices
  int n_ob;   // 128-row output blocks
  size_t ws;  // workspace bytes
};

int env_int(const char* name, int dflt) {
  const char* s = std::getenv(name);
  return s ? std::atoi(s) : dflt;
}

int pick_ks(int n_ob, int tiles_in, int block_in) {
  const int forced = env_int("TRELLIS_GEMV_KS", 0);
  const int target_wg = env_int("TRELLIS_GEMV_TARGET_WG", 1024);
  int best = -1;
  // valid kS: divides tiles_in, slice holds whole Hadamard blocks, fits LDS
  for (int ks = 1; ks <= GEMV_MAX_KS && ks <= tiles_in; ++ks) {
    if (tiles_in % ks || (ks * 16) % block_in) continue;
    if (forced > 0 && ks == forced) return ks;
    const int wg = n_ob * (tiles_in / ks);
    if (wg >= target_wg || best < 0) best = ks;  // largest kS that still meets the target
  }
  return best;
}

GemvPlan gemv_plan(const trellis_desc* W, int batch) {
  GemvPlan p;
  const int b = batch < GEMV_MAX_NB ? batch : GEMV_MAX_NB;
  p.nb = b <= 1 ? 1 : b <= 2 ? 2 : b <= 4 ? 4 : 8;
  p.n_ob = (W->n_out + 127) / 128;
  const int tiles_in = W->k_in / 16;
  p.kS = pick_ks(p.n_ob, tiles_in, W->block_in);
  p.S = tiles_in / p.kS;
  p.ws = 0;
  if (p.S > 1) {
    const size_t tickets = (static_cast<size_t>(p.n_ob) * 4 + 255) & ~static_cast<size_t>(255);
    p.ws = tickets + static_cast<size_t>(p.n_ob) * p.S * p.nb * 128 * sizeof(float);
  }
  return p;
}

size_t gemv_lds_bytes(int nb, int kS) {
  return static_cast<size_t>(nb) * kS * 16 * 4 + 3 * static_cast<size_t>(nb) * 128 * 4;
}

template <int K, int CB>
int launch_gemv_nb(int nb, const GemvArgs& a, int grid, size_t lds, hipStream_t st) {
  switch (nb) {
    case 1: hipLaunchKernelGGL((gemv_kernel<K, CB, 1>), dim3(grid), dim3(256), lds, st, a); break;
    case 2: hipLaunchKernelGGL((gemv_kernel<K, CB, 2>), dim3(grid), dim3(256), lds, st, a); break;
    case 4: hipLaunchKernelGGL((gemv_kernel<K, CB, 4>), dim3(grid), dim3(256), lds, st, a); break;
    default: hipLaunchKernelGGL((gemv_kernel<K, CB, 8>), dim3(grid), dim3(256), lds, st, a); break;
  }
  return hipGetLastError() == hipSuccess ? TRELLIS_OK : TRELLIS_ERR_LAUNCH;
}

template <int K>
int launch_gemv_k(int cb, int nb, const GemvArgs& a, int grid, size_t lds, hipStream_t st) {
  switch (cb) {
    case CB_MCG: return launch_gemv_nb<K, CB_MCG>(nb, a, grid, lds, st);
    case CB_3INST: return launch_gemv_nb<K, CB_3INST>(nb, a, grid, lds, st);
    default: return launch_gemv_nb<K, CB_1MAD>(nb, a, grid, lds, st);
  }
}

int launch_gemv(const trellis_desc* W, int cb, int nb, const GemvArgs& a, int grid, size_t lds,
                hipStream_t st) {
  switch (W->K) {
    case 2: return launch_gemv_k<2>(cb, nb, a, grid, lds, st);
    case 3: return launch_gemv_k<3>(cb, nb, a, grid, lds, st);
    default: return launch_gemv_k<4>(cb, nb, a, grid, lds, st);
  }
}

template <int K>
int launch_decode_k(int cb, const uint32_t* bits, int nw, uint32_t t0, uint32_t nt, float* out,
                    hipStream_t st) {
  const dim3 grid((nt + 15) / 16);
  switch (cb) {
    case CB_MCG:
      hipLaunchKernelGGL((decode_tiles_kernel<K, CB_MCG>), grid, dim3(256), 0, st, bits, nw, t0, nt, out);
      break;
    case CB_3INST:
      hipLaunchKernelGGL((decode_tiles_kernel<K, CB_3INST>), grid, dim3(256), 0, st, bits, nw, t0, nt, out);
      break;
    default:
      hipLaunchKernelGGL((decode_tiles_kernel<K, CB_1MAD>), grid, dim3(256), 0, st, bits, nw, t0, nt, out);
      break;
  }
  return hipGetLastError() == hipSuccess ? TRELLIS_OK : TRELLIS_ERR_LAUNCH;
}

}  // namespace

// ---------------------------------------------------------------- C ABI
extern "C" {

const char* trellis_version(void) { return "trellis-amd 0.1 gfx950"; }

const char* trellis_strerror(int status) {
  switch (status) {
    case TRELLIS_OK: return "ok";
    case TRELLIS_ERR_NULL: return "a required pointer is NULL";
    case TRELLIS_ERR_SHAPE: return "n_out and k_in must be positive multiples of 16";
    case TRELLIS_ERR_BLOCK: return "Hadamard block must be a power of 2 in [16,128] dividing its dim";
    case TRELLIS_ERR_K: return "bits per weight K must be 2, 3 or 4";
    case TRELLIS_ERR_V: return "only V=1 is supported";
    case TRELLIS_ERR_CODEBOOK: return "unknown codebook id";
    case TRELLIS_ERR_NWORDS: return "nwords must equal 256*K/32";
    case TRELLIS_ERR_ALIGN: return "bits must be 16-byte aligned and strides must cover a row";
    case TRELLIS_ERR_DTYPE: return "x/y dtype must be TRELLIS_F32 or TRELLIS_F16";
    case TRELLIS_ERR_WORKSPACE: return "workspace missing or too small";
    case TRELLIS_ERR_BATCH: return "batch must be >= 1";
    case TRELLIS_ERR_RANGE: return "tile range outside the matrix";
    case TRELLIS_ERR_LAUNCH: return "HIP kernel launch failed";
    default: return "unknown trellis status";
  }
}

int trellis_workspace_bytes(const trellis_desc* W, int batch, size_t* bytes) {
  if (!bytes) return TRELLIS_ERR_NULL;
  const int v = validate(W);
  if (v) return v;
  if (batch < 1) return TRELLIS_ERR_BATCH;
  *bytes = gemv_plan(W, batch).ws;
  return TRELLIS_OK;
}

int trellis_decode_tiles(const trellis_desc* W, uint32_t tile_begin, uint32_t ntiles, float* out,
                         void* stream) {
  const int v = validate(W);
  if (v) return v;
  if (!out) return TRELLIS_ERR_NULL;
  const uint64_t total = static_cast<uint64_t>(W->n_out / 16) * (W->k_in / 16);
  if (static_cast<uint64_t>(tile_begin) + ntiles > total) return TRELLIS_ERR_RANGE;
  if (ntiles == 0) return TRELLIS_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (W->K) {
    case 2: return launch_decode_k<2>(W->codebook, W->bits, W->nwords, tile_begin, ntiles, out, st);
    case 3: return launch_decode_k<3>(W->codebook, W->bits, W->nwords, tile_begin, ntiles, out, st);
    default: return launch_decode_k<4>(W->codebook, W->bits, W->nwords, tile_begin, ntiles, out, st);
  }
}

int trellis_packed_linear(const trellis_desc* W, const void* x, int64_t ldx, int batch,
                          int x_dtype, void* y, int64_t ldy, int y_dtype, void* workspace,
                          size_t ws_bytes, void* stream) {
  int v = validate(W);
  if (v) return v;
  v = validate_fold(W);
  if (v) return v;
  if (!x || !y) return TRELLIS_ERR_NULL;
  if (batch < 1) return TRELLIS_ERR_BATCH;
  if ((x_dtype != TRELLIS_F32 && x_dtype != TRELLIS_F16) ||
      (y_dtype != TRELLIS_F32 && y_dtype != TRELLIS_F16))
    return TRELLIS_ERR_DTYPE;
  if (batch > 1 && (ldx < W->k_in || ldy < W->n_out)) return TRELLIS_ERR_ALIGN;
  const GemvPlan p = gemv_plan(W, batch);
  if (p.ws > 0 && (!workspace || ws_bytes < p.ws)) return TRELLIS_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);

  GemvArgs a;
  a.bits = W->bits;
  a.su = W->su;
  a.sv = W->sv;
  a.isc = W->isc_scaled;
  a.osc = W->osc;
  a.ldx = ldx;
  a.ldy = ldy;
  a.n = W->n_out;
  a.k = W->k_in;
  a.nwords = W->nwords;
  a.tiles_in = W->k_in / 16;
  a.kS = p.kS;
  a.S = p.S;
  a.block_in = W->block_in;
  a.block_out = W->block_out;
  a.x_f16 = x_dtype == TRELLIS_F16;
  a.y_f16 = y_dtype == TRELLIS_F16;
  const size_t tickets = (static_cast<size_t>(p.n_ob) * 4 + 255) & ~static_cast<size_t>(255);
  a.tickets = p.S > 1 ? static_cast<unsigned*>(workspace) : nullptr;
  a.part = p.S > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + tickets) : nullptr;
  const size_t xes = a.x_f16 ? 2 : 4, yes = a.y_f16 ? 2 : 4;
  const size_t lds = gemv_lds_bytes(p.nb, p.kS);
  const int grid = p.n_ob * p.S;
  for (int b0 = 0; b0 < batch; b0 += p.nb) {
    a.batch = batch - b0 < p.nb ? batch - b0 : p.nb;
    a.x = static_cast<const char*>(x) + static_cast<size_t>(b0) * ldx * xes;
    a.y = static_cast<char*>(y) + static_cast<size_t>(b0) * ldy * yes;
    v = launch_gemv(W, W->codebook, p.nb, a, grid, lds, st);
    if (v) return v;
  }
  return TRELLIS_OK;
}

}  // extern "C"
