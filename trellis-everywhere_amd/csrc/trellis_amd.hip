// trellis_amd.hip — C ABI (include/trellis_amd.h) and launchers of the gfx950 trellis
// kernels: the bit-exact tile decode and the fused decode-GEMV.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>

#include "trellis_amd.h"
#include "decode.h"
#include "gemv_launch.h"

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

int env_int(const char* name, int dflt) {
  const char* s = std::getenv(name);
  return s ? std::atoi(s) : dflt;
}

struct GroupPlan {
  int nb;              // batch rows per launch (1, 2, 4, 8)
  int tpw;             // tiles per wave: a work item covers kS = 2*tpw tile columns
  int total;           // work items over the group
  int n_ob[GEMV_MAX_GROUP], S[GEMV_MAX_GROUP];
  size_t ws_off[GEMV_MAX_GROUP];  // workspace offset of matrix i (tickets, then partials)
  size_t ws;           // workspace bytes
};

// A work item is one 128-row output block x one k-slice of 2*tpw tile columns. tpw = 8
// unless the group has too few items to occupy every CU several times over;
// TRELLIS_GEMV_TPW forces 4 or 8.
GroupPlan group_plan(const trellis_desc* const* W, int count, int batch) {
  GroupPlan p;
  const int b = batch < GEMV_MAX_NB ? batch : GEMV_MAX_NB;
  p.nb = b <= 1 ? 1 : b <= 2 ? 2 : b <= 4 ? 4 : 8;
  auto items = [&](int tpw) {
    long long t = 0;
    for (int i = 0; i < count; ++i)
      t += static_cast<long long>((W[i]->n_out + 127) / 128) *
           ((W[i]->k_in / 16 + 2 * tpw - 1) / (2 * tpw));
    return t;
  };
  const int forced = env_int("TRELLIS_GEMV_TPW", 0);
  p.tpw = forced == 4 || forced == 8 ? forced : (items(8) >= 2048 ? 8 : 4);
  p.total = 0;
  p.ws = 0;
  for (int i = 0; i < count; ++i) {
    p.n_ob[i] = (W[i]->n_out + 127) / 128;
    p.S[i] = (W[i]->k_in / 16 + 2 * p.tpw - 1) / (2 * p.tpw);
    p.total += p.n_ob[i] * p.S[i];
    p.ws_off[i] = p.ws;
    if (p.S[i] > 1) {
      const size_t tickets = (static_cast<size_t>(p.n_ob[i]) * 4 + 255) & ~static_cast<size_t>(255);
      p.ws += tickets + static_cast<size_t>(p.n_ob[i]) * p.S[i] * p.nb * 128 * sizeof(float);
    }
  }
  return p;
}

int launch_gemv(int K, int cb, int nb, int tpw, const GemvGroupArgs& g, hipStream_t st) {
  switch (K) {
    case 2: return launch_gemv_k<2>(cb, nb, tpw, g, st);
    case 3: return launch_gemv_k<3>(cb, nb, tpw, g, st);
    default: return launch_gemv_k<4>(cb, nb, tpw, g, st);
  }
}

int validate_group(const trellis_desc* const* W, int count) {
  if (!W || count < 1) return TRELLIS_ERR_NULL;
  if (count > GEMV_MAX_GROUP) return TRELLIS_ERR_GROUP;
  for (int i = 0; i < count; ++i) {
    int v = validate(W[i]);
    if (v) return v;
    v = validate_fold(W[i]);
    if (v) return v;
    if (W[i]->K != W[0]->K || W[i]->codebook != W[0]->codebook) return TRELLIS_ERR_GROUP;
  }
  return TRELLIS_OK;
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
    case TRELLIS_ERR_GROUP: return "a group holds 1..8 linears sharing K and codebook";
    default: return "unknown trellis status";
  }
}

int trellis_workspace_bytes_group(const trellis_desc* const* W, int count, int batch,
                                  size_t* bytes) {
  if (!bytes) return TRELLIS_ERR_NULL;
  const int v = validate_group(W, count);
  if (v) return v;
  if (batch < 1) return TRELLIS_ERR_BATCH;
  *bytes = group_plan(W, count, batch).ws;
  return TRELLIS_OK;
}

int trellis_workspace_bytes(const trellis_desc* W, int batch, size_t* bytes) {
  if (!bytes) return TRELLIS_ERR_NULL;
  const int v = validate(W);
  if (v) return v;
  if (batch < 1) return TRELLIS_ERR_BATCH;
  *bytes = group_plan(&W, 1, batch).ws;
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

int trellis_packed_linear_group(const trellis_desc* const* W, int count, const void* const* x,
                                 const int64_t* ldx, int batch, int x_dtype, void* const* y,
                                 const int64_t* ldy, int y_dtype, void* workspace,
                                 size_t ws_bytes, void* stream) {
  int v = validate_group(W, count);
  if (v) return v;
  if (!x || !y || !ldx || !ldy) return TRELLIS_ERR_NULL;
  if (batch < 1) return TRELLIS_ERR_BATCH;
  if ((x_dtype != TRELLIS_F32 && x_dtype != TRELLIS_F16) ||
      (y_dtype != TRELLIS_F32 && y_dtype != TRELLIS_F16))
    return TRELLIS_ERR_DTYPE;
  for (int i = 0; i < count; ++i) {
    if (!x[i] || !y[i]) return TRELLIS_ERR_NULL;
    if (batch > 1 && (ldx[i] < W[i]->k_in || ldy[i] < W[i]->n_out)) return TRELLIS_ERR_ALIGN;
    // activations are read as aligned u32 words
    if (reinterpret_cast<uintptr_t>(x[i]) % 4) return TRELLIS_ERR_ALIGN;
    if (x_dtype == TRELLIS_F16 && batch > 1 && ldx[i] % 2) return TRELLIS_ERR_ALIGN;
  }
  const GroupPlan p = group_plan(W, count, batch);
  if (p.ws > 0 && (!workspace || ws_bytes < p.ws)) return TRELLIS_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);

  GemvGroupArgs g;
  std::memset(&g, 0, sizeof(g));
  g.nmat = count;
  g.total = p.total;
  g.nwords = W[0]->nwords;
  g.x_f16 = x_dtype == TRELLIS_F16;
  g.y_f16 = y_dtype == TRELLIS_F16;
  int item0 = 0;
  for (int i = 0; i < count; ++i) {
    GemvMat& m = g.m[i];
    m.bits = W[i]->bits;
    m.su = W[i]->su;
    m.sv = W[i]->sv;
    m.isc = W[i]->isc_scaled;
    m.osc = W[i]->osc;
    m.ldx = ldx[i];
    m.ldy = ldy[i];
    m.n = W[i]->n_out;
    m.k = W[i]->k_in;
    m.tiles_in = W[i]->k_in / 16;
    m.block_in = W[i]->block_in;
    m.block_out = W[i]->block_out;
    m.n_ob = p.n_ob[i];
    m.S = p.S[i];
    m.item0 = item0;
    item0 += p.n_ob[i] * p.S[i];
    if (p.S[i] > 1) {
      char* base = static_cast<char*>(workspace) + p.ws_off[i];
      const size_t tickets = (static_cast<size_t>(p.n_ob[i]) * 4 + 255) & ~static_cast<size_t>(255);
      m.tickets = reinterpret_cast<unsigned*>(base);
      m.part = reinterpret_cast<float*>(base + tickets);
    }
  }
  const size_t xes = g.x_f16 ? 2 : 4, yes = g.y_f16 ? 2 : 4;
  for (int b0 = 0; b0 < batch; b0 += p.nb) {
    g.batch = batch - b0 < p.nb ? batch - b0 : p.nb;
    for (int i = 0; i < count; ++i) {
      g.m[i].x = static_cast<const char*>(x[i]) + static_cast<size_t>(b0) * ldx[i] * xes;
      g.m[i].y = static_cast<char*>(y[i]) + static_cast<size_t>(b0) * ldy[i] * yes;
    }
    v = launch_gemv(W[0]->K, W[0]->codebook, p.nb, p.tpw, g, st);
    if (v) return v;
  }
  return TRELLIS_OK;
}

int trellis_packed_linear(const trellis_desc* W, const void* x, int64_t ldx, int batch,
                          int x_dtype, void* y, int64_t ldy, int y_dtype, void* workspace,
                          size_t ws_bytes, void* stream) {
  return trellis_packed_linear_group(&W, 1, &x, &ldx, batch, x_dtype, &y, &ldy, y_dtype,
                                     workspace, ws_bytes, stream);
}

}  // extern "C"
