// trellis_amd.hip — C ABI (include/trellis_amd.h): validation, launch planning, the
// bit-exact tile decode kernel and the dispatch to the decode-matmul kernels (gemv_kernel at
// batch 1 to 4 and, where use_gemv picks it, 5 to 16; xfold_kernel + bgemm_kernel
// (+ bfold_kernel) otherwise).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "trellis_amd.h"
#include "decode.h"
#define TRELLIS_XFOLD_DEFINE
#define TRELLIS_BFOLD_DEFINE
#include "launch.h"
#include "embed.h"
#include "encode.h"

using namespace trellis;

namespace {

// ---------------------------------------------------------------- decode kernel
// One wave per tile, lane l = (tile row r = l%16, column group g = l/16): the same
// decode_quad the matmul kernels run, each value stored as its exact fp32 (the fp16
// halves summed in fp32; 1MAD divided as the reference does).
template <int K, int CB, int V>
__global__ __launch_bounds__(256) void decode_tiles_kernel(const uint32_t* __restrict__ bits,
                                                           uint32_t tile0, uint32_t ntiles,
                                                           float* __restrict__ out) {
  const uint32_t lt = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (lt >= ntiles) return;
  const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const uint32_t* tp = bits + static_cast<size_t>(tile0 + lt) * (8 * K);
  const QuadPos qp = quad_pos_v<K, V>(r, g);
  uint32_t raw[4];
  decode_quad<K, CB, V>(tp[qp.wa], tp[qp.wb], qp.sh, raw);
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = cb_exact<CB>(raw[q]);
  *reinterpret_cast<float4*>(out + static_cast<size_t>(lt) * 256 + 16 * r + 4 * g) =
      make_float4(v[0], v[1], v[2], v[3]);
}

// Zero n words (the split-K ticket header of a call on the static scratch below). A kernel,
// not hipMemsetAsync, so that a caller may capture the call in a HIP graph.
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* __restrict__ p, unsigned n) {
  const unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i < n) p[i] = 0u;
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
  if (W->V != 1 && W->V != 2) return TRELLIS_ERR_V;
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

// ---------------------------------------------------------------- plan
int env_int(const char* name, int dflt) {
  const char* s = std::getenv(name);
  return s ? std::atoi(s) : dflt;
}

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

struct GroupPlan {
  int nb;              // batch rows per launch
  int gemv;            // batch-1 gemv_kernel (else bgemm_kernel)
  int nc, ncb;         // bgemm: 16-column chunks per workgroup, column blocks
  int kr;              // gemv / bgemm: tile columns per k-range
  int kc;              // gemv: tile columns per pipeline stage (8 or 16)
  int total;           // work items over the group
  int folds;           // x-fold jobs over the group
  int n_ob[MAX_GROUP], S[MAX_GROUP];
  size_t off_tickets[MAX_GROUP], off_part[MAX_GROUP], off_xf[MAX_GROUP];
  size_t header;       // bytes of the ticket header at the start of the workspace
  size_t ws;           // workspace bytes
};

// CUs of the current device, asked of the runtime once per device (the planners consult it
// several times per call)
int device_cus() {
  constexpr int MAX_DEVICES = 64;
  static std::atomic<int> cached[MAX_DEVICES];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev >= 0 && dev < MAX_DEVICES) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  if (dev >= 0 && dev < MAX_DEVICES) cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Batch 1 to 4, and 5 to 16 where the group is narrow (gemv_kernel): a work item is one
// 128-row output block x one k-range of kr tile columns (kr a multiple of 8, so a k-range
// holds whole 128-column fold chunks, and at most gemv_kr_max(nb)), run by one 16-wave
// workgroup; one workgroup fits a CU. kr minimises an estimate of the launch time in
// 2.4 GHz cycles: rounds of items over the CUs x the decode of 8 bands x kr/2 tiles per wave
// at ~50 cycles per tile with four waves per SIMD (above 4 rows, plus the fold of kr x 16
// activations of every row in each workgroup), plus ~2 us of split-K epilogue (publish,
// ticket, reduce) and ~0.1 us of ticket contention per slice when kr does not cover k, plus
// a first-load latency for every round after the first. TRELLIS_GEMV_KR forces a value.
int gemv_kr(const trellis_desc* const* W, int count, int batch) {
  const int nb = gemv_nb(batch), krm = gemv_kr_max(nb);
  int maxt = 0;
  for (int i = 0; i < count; ++i) maxt = W[i]->k_in / 16 > maxt ? W[i]->k_in / 16 : maxt;
  const int cap = ((maxt + 7) / 8) * 8 < krm ? ((maxt + 7) / 8) * 8 : krm;
  const int forced = env_int("TRELLIS_GEMV_KR", 0);
  if (forced >= 8 && forced <= krm && forced % 8 == 0) return forced;
  // the per-workgroup fold of every row (~2 model units per tile column and row)
  const long long per_kr = 100 + (nb > 4 ? 2 * nb : 0);
  const long long cus = device_cus();
  int best = 8;
  long long best_cost = -1;
  for (int kr = 8; kr <= cap; kr += 8) {
    long long items = 0;
    int smax = 1;
    for (int i = 0; i < count; ++i) {
      const int S = (W[i]->k_in / 16 + kr - 1) / kr;
      items += static_cast<long long>((W[i]->n_out + 127) / 128) * S;
      smax = S > smax ? S : smax;
    }
    const long long rounds = (items + cus - 1) / cus;
    const long long cost = rounds * kr * per_kr + (smax > 1 ? 4800 + 240 * smax : 0) +
                           (rounds - 1) * 3600;
    if (best_cost < 0 || cost < best_cost) {
      best = kr;
      best_cost = cost;
    }
  }
  return best;
}

// Batch >= 2 (bgemm_kernel): NC 16-column batch chunks per workgroup (up to 128 columns),
// a work item is one 128-row block x one column block x one k-range of kr tile columns
// (a multiple of the k-step: 16 tiles at 16 columns, 8 up to 64 and in the fp16-weight
// mode, else 6), run by one workgroup per CU (16 waves; 12 for the exact mode's 128-column
// blocks). kr minimises ceil(items/CUs) x the per-SIMD work of an item (2 bands x kr tiles
// x (decode ~61 + NC MFMAs x ~19 cycles; fp16-weight mode ~75 + NC x ~10; ~225 for the
// exact mode's 128-column blocks at three waves per SIMD, fitted to a sweep of both widths
// on the 8B block's launches at 128-512 rows, where it picks the faster width for all but
// q/k/v at 128 and 192 rows, ~3 us each)) plus, with split-K,
// the bfold_kernel launch (~1.5 us) and the partial blocks it moves (S x rows x NB x 4
// bytes written and read at ~2.5 KB per cycle), plus a start-up latency per round after
// the first. TRELLIS_BGEMM_KR forces a value, TRELLIS_BGEMM_NC the column-block width.
static int bgemm_kr_cost(const trellis_desc* const* W, int count, int batch, int nc, bool f16,
                         long long* cost) {
  int maxt = 0;
  for (int i = 0; i < count; ++i) maxt = W[i]->k_in / 16 > maxt ? W[i]->k_in / 16 : maxt;
  const int kt = f16 ? 8 : nc == 1 ? 16 : nc <= 4 ? 8 : 6;   // BgStep<nc, f16>::KT
  // per band-tile SIMD cycles: the decode and NC MFMAs (the fp16-weight mode decodes a
  // little more and issues half the MFMAs)
  const long long tile_cost = f16 ? 75 + 10 * nc : nc == 8 ? 225 : 61 + 19 * nc;
  const int cap = ((maxt + kt - 1) / kt) * kt;
  const long long cus = device_cus();
  const long long ncb = (batch + 16 * nc - 1) / (16 * nc);
  const int forced = env_int("TRELLIS_BGEMM_KR", 0);
  const bool force = forced >= kt && forced % kt == 0;
  int best = cap;
  long long best_cost = -1;
  for (int kr = force ? (forced < cap ? forced : cap) : kt; kr <= cap; kr += kt) {
    long long items = 0, part_bytes = 0;
    int smax = 1;
    for (int i = 0; i < count; ++i) {
      const int S = (W[i]->k_in / 16 + kr - 1) / kr;
      const long long n_ob = (W[i]->n_out + 127) / 128;
      items += n_ob * ncb * S;
      smax = S > smax ? S : smax;
      if (S > 1) part_bytes += static_cast<long long>(S) * n_ob * ncb * 128 * 16 * nc * 4;
    }
    if (smax > 16 && !force) continue;
    const long long rounds = (items + cus - 1) / cus;
    const long long epi = smax > 1 ? 3600 + 2 * part_bytes / 2500 : 0;
    const long long c = rounds * kr * 2 * tile_cost + epi + (rounds - 1) * 3600;
    if (best_cost < 0 || c < best_cost) {
      best = kr;
      best_cost = c;
    }
    if (force) break;
  }
  *cost = best_cost;
  return best;
}

int bgemm_kr(const trellis_desc* const* W, int count, int batch, int nc, bool f16) {
  long long cost;
  return bgemm_kr_cost(W, count, batch, nc, f16, &cost);
}

// Column-block width: 16, 32 or 64 columns up to batch 64; above, the fp16-weight mode
// takes 128, and the exact mode 64 (four waves per SIMD) or 128 (three waves per SIMD, each
// tile decoded half as often), whichever the cost model above finds cheaper for the group
// (8B block at batch 512: q/k/v and gate+up at 128 columns, 100 -> 87 and 277 -> 243 us;
// o stays at 64, where 128 measured 53 -> 57 us; one gate projection at batch 96 stays at 64,
// at 256 takes 128: 92 -> 76 us).
int bgemm_nc(const trellis_desc* const* W, int count, int batch, bool f16) {
  const int forced = env_int("TRELLIS_BGEMM_NC", 0);
  if (forced == 1 || forced == 2 || forced == 4 || forced == 8) return forced;
  if (batch <= 16) return 1;
  if (batch <= 32) return 2;
  if (batch <= 64) return 4;
  if (f16) return 8;
  long long c4, c8;
  bgemm_kr_cost(W, count, batch, 4, false, &c4);
  bgemm_kr_cost(W, count, batch, 8, false, &c8);
  return c8 < c4 ? 8 : 4;
}

// The decode-GEMV for batch 1 to 4, and for 5 to 16 when its items at the longest k-range
// (gemv_kr_max) fit one round on the CUs: every workgroup folds the activations of its
// k-range for all rows, and the cap on the k-range that the rows' LDS imposes multiplies
// the items of a long k or a wide group; otherwise the batched path, with its two extra
// launches (x fold, split-K fold), is faster (measured on the 8B block: the gemv wins for
// q/k/v, o and down at batch 5 to 16, by 1-5 us per launch; gate+up needs two or more
// rounds and loses by 4-15 us). TRELLIS_SMALL_BATCH_GEMV
// = 1 / 0 forces the choice for batch 5 to 16.
bool use_gemv(const trellis_desc* const* W, int count, int batch) {
  if (batch <= 4) return true;
  if (batch > GEMV_MAX_NB) return false;
  const int forced = env_int("TRELLIS_SMALL_BATCH_GEMV", -1);
  if (forced == 0 || forced == 1) return forced == 1;
  const int krm = gemv_kr_max(gemv_nb(batch));
  long long items = 0;
  for (int i = 0; i < count; ++i)
    items += static_cast<long long>((W[i]->n_out + 127) / 128) * ((W[i]->k_in / 16 + krm - 1) / krm);
  return items <= device_cus();
}

GroupPlan group_plan(const trellis_desc* const* W, int count, int batch, bool f16) {
  GroupPlan p;
  p.gemv = use_gemv(W, count, batch);
  p.nb = batch;
  p.nc = bgemm_nc(W, count, batch, f16);
  p.ncb = p.gemv ? 1 : (batch + 16 * p.nc - 1) / (16 * p.nc);
  p.kr = p.gemv ? gemv_kr(W, count, batch) : bgemm_kr(W, count, batch, p.nc, f16);
  // tiles per decode-GEMV stage: 16, or 8 for short k-ranges and for launches that split k
  // (a workgroup's first stage lands sooner: the 8B block's q/k/v and down launches
  // 0.2-0.7 us faster each at batch 1 to 8)
  bool split = false;
  for (int i = 0; i < count; ++i) split = split || W[i]->k_in / 16 > p.kr;
  p.kc = p.kr >= 32 && !(p.gemv && split) ? 16 : 8;
  {
    const int kc = env_int("TRELLIS_GEMV_KC", 0);
    if (p.gemv && (kc == 8 || kc == 16) && kc <= p.kr) p.kc = kc;
  }
  // 16 rows: two 16-tile ring slots do not fit beside the rows' activations, so the
  // kernel's stages are 8 tiles; the plan says so too
  if (p.gemv && gemv_nb(batch) == 16) p.kc = 8;
  p.total = 0;
  p.folds = 0;
  // Workspace: a header of counters whose layout depends only on the members' shapes (one
  // split-K ticket per 128-row block of every member); every call leaves them at zero.
  // Plans for other batch sizes reuse the same workspace, so their data (partial sums,
  // folded activations) only ever lies past the header, and a ticket never starts from
  // another plan's data.
  p.ws = 0;
  for (int i = 0; i < count; ++i) {
    p.n_ob[i] = (W[i]->n_out + 127) / 128;
    p.off_tickets[i] = p.ws;
    p.ws += align256(static_cast<size_t>(p.n_ob[i]) * 4);
  }
  p.header = p.ws;
  // partial sums per (block, slice): the gemv's NB batch rows, or bgemm's 16 * NC
  const int part_cols = p.gemv ? gemv_nb(batch) : 16 * p.nc;
  for (int i = 0; i < count; ++i) {
    p.S[i] = (W[i]->k_in / 16 + p.kr - 1) / p.kr;
    p.total += p.n_ob[i] * p.ncb * p.S[i];
    p.folds += p.nb * ((W[i]->k_in + 127) / 128);
    p.off_part[i] = p.ws;
    if (p.S[i] > 1)
      p.ws += align256(static_cast<size_t>(p.n_ob[i]) * p.ncb * p.S[i] * part_cols * 128 *
                       sizeof(float));
    p.off_xf[i] = p.ws;
    if (!p.gemv) p.ws += align256(static_cast<size_t>(p.nb) * W[i]->k_in * 4);
  }
  return p;
}

// The pipelined decode-GEMV (its x fold is fused): batch 1 to 4, and 5 to 16 where
// use_gemv picks it.
int launch_gemv(int K, int cb, int V, int kc, const LinArgs& g, hipStream_t st) {
  switch (K) {
    case 2: return launch_gemv_k<2>(cb, V, kc, g, st);
    case 3: return launch_gemv_k<3>(cb, V, kc, g, st);
    default: return launch_gemv_k<4>(cb, V, kc, g, st);
  }
}

// The x fold of every member (the batched path), written once to the workspace.
int launch_xfold(LinArgs& g, int folds, hipStream_t st) {
  const int items = g.total;
  g.total = folds;
  const dim3 grid(static_cast<unsigned>((folds + 3) / 4));
  const bool one = g.nmat == 1;
  if (xfold_rows(g.batch) == 4) {
    if (one) hipLaunchKernelGGL((xfold_kernel<4, true>), grid, dim3(256), 0, st, g);
    else hipLaunchKernelGGL((xfold_kernel<4, false>), grid, dim3(256), 0, st, g);
  } else {
    if (one) hipLaunchKernelGGL((xfold_kernel<1, true>), grid, dim3(256), 0, st, g);
    else hipLaunchKernelGGL((xfold_kernel<1, false>), grid, dim3(256), 0, st, g);
  }
  g.total = items;
  return hipGetLastError() == hipSuccess ? TRELLIS_OK : TRELLIS_ERR_LAUNCH;
}

// The batched path: the x fold, the decode-once batched kernel, and (split-K) its reduction.
int launch_bgemm(int K, int cb, int V, int nc, LinArgs& g, int folds, int nfold, hipStream_t st) {
  int v = launch_xfold(g, folds, st);
  if (v) return v;
  switch (K) {
    case 2: v = launch_bgemm_k<2>(cb, V, nc, g, st); break;
    case 3: v = launch_bgemm_k<3>(cb, V, nc, g, st); break;
    default: v = launch_bgemm_k<4>(cb, V, nc, g, st); break;
  }
  if (v || nfold == 0) return v;
  return launch_bfold(cb, nc, nfold, g, st);
}

int validate_group(const trellis_desc* const* W, int count) {
  if (!W || count < 1) return TRELLIS_ERR_NULL;
  if (count > MAX_GROUP) return TRELLIS_ERR_GROUP;
  for (int i = 0; i < count; ++i) {
    int v = validate(W[i]);
    if (v) return v;
    v = validate_fold(W[i]);
    if (v) return v;
    if (W[i]->K != W[0]->K || W[i]->codebook != W[0]->codebook || W[i]->V != W[0]->V)
      return TRELLIS_ERR_GROUP;
  }
  return TRELLIS_OK;
}

template <int K, int V>
int launch_decode_kv(int cb, const uint32_t* bits, uint32_t t0, uint32_t nt, float* out,
                     hipStream_t st) {
  const dim3 grid((nt + 3) / 4);
  switch (cb) {
    case CB_MCG:
      hipLaunchKernelGGL((decode_tiles_kernel<K, CB_MCG, V>), grid, dim3(256), 0, st, bits, t0, nt, out);
      break;
    case CB_3INST:
      hipLaunchKernelGGL((decode_tiles_kernel<K, CB_3INST, V>), grid, dim3(256), 0, st, bits, t0, nt, out);
      break;
    default:
      hipLaunchKernelGGL((decode_tiles_kernel<K, CB_1MAD, V>), grid, dim3(256), 0, st, bits, t0, nt, out);
      break;
  }
  return hipGetLastError() == hipSuccess ? TRELLIS_OK : TRELLIS_ERR_LAUNCH;
}

template <int K>
int launch_decode_k(int cb, int V, const uint32_t* bits, uint32_t t0, uint32_t nt, float* out,
                    hipStream_t st) {
  return V == 2 ? launch_decode_kv<K, 2>(cb, bits, t0, nt, out, st)
                : launch_decode_kv<K, 1>(cb, bits, t0, nt, out, st);
}

template <int K, int V>
int launch_embed_kv(int cb, const EmbedArgs& a, unsigned grid, hipStream_t st) {
  switch (cb) {
    case CB_MCG: hipLaunchKernelGGL((embed_kernel<K, CB_MCG, V>), dim3(grid), dim3(256), 0, st, a); break;
    case CB_3INST: hipLaunchKernelGGL((embed_kernel<K, CB_3INST, V>), dim3(grid), dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((embed_kernel<K, CB_1MAD, V>), dim3(grid), dim3(256), 0, st, a); break;
  }
  return hipGetLastError() == hipSuccess ? TRELLIS_OK : TRELLIS_ERR_LAUNCH;
}

template <int K>
int launch_embed_k(int cb, int V, const EmbedArgs& a, unsigned grid, hipStream_t st) {
  return V == 2 ? launch_embed_kv<K, 2>(cb, a, grid, st) : launch_embed_kv<K, 1>(cb, a, grid, st);
}

// Viterbi encoder: one workgroup per CU, persistent over the tiles.
unsigned encode_grid(uint32_t ntiles) {
  const unsigned cus = static_cast<unsigned>(device_cus());
  return ntiles < cus ? ntiles : cus;
}

template <int K>
int launch_encode_k(int cb, const VitArgs& a, unsigned grid, hipStream_t st) {
  switch (cb) {
    case CB_MCG: hipLaunchKernelGGL((viterbi_kernel<K, CB_MCG>), dim3(grid), dim3(VIT_THREADS), 0, st, a); break;
    case CB_3INST: hipLaunchKernelGGL((viterbi_kernel<K, CB_3INST>), dim3(grid), dim3(VIT_THREADS), 0, st, a); break;
    default: hipLaunchKernelGGL((viterbi_kernel<K, CB_1MAD>), dim3(grid), dim3(VIT_THREADS), 0, st, a); break;
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
    case TRELLIS_ERR_V: return "V (weights per trellis step) must be 1 or 2";
    case TRELLIS_ERR_CODEBOOK: return "unknown codebook id";
    case TRELLIS_ERR_NWORDS: return "nwords must equal 256*K/32";
    case TRELLIS_ERR_ALIGN: return "bits must be 16-byte aligned and strides must cover a row";
    case TRELLIS_ERR_DTYPE: return "x/y dtype must be TRELLIS_F32 or TRELLIS_F16";
    case TRELLIS_ERR_WORKSPACE: return "workspace missing or too small";
    case TRELLIS_ERR_BATCH: return "batch must be >= 1";
    case TRELLIS_ERR_RANGE: return "tile range outside the matrix";
    case TRELLIS_ERR_LAUNCH: return "HIP kernel launch failed";
    case TRELLIS_ERR_GROUP: return "a group holds 1..8 linears sharing K, V and codebook";
    case TRELLIS_ERR_FLAGS: return "unknown flag bits";
    case TRELLIS_ERR_SCRATCH:
      return "the call needs more workspace than the no-allocation entry point's static scratch "
             "(TRELLIS_NOALLOC_SCRATCH_BYTES)";
    case TRELLIS_ERR_CAPTURE:
      return "the first no-allocation call on a device must not be made under stream capture "
             "(it looks up the device's scratch address)";
    default: return "unknown trellis status";
  }
}

int trellis_workspace_bytes_group(const trellis_desc* const* W, int count, int batch,
                                  size_t* bytes) {
  if (!bytes) return TRELLIS_ERR_NULL;
  const int v = validate_group(W, count);
  if (v) return v;
  if (batch < 1) return TRELLIS_ERR_BATCH;
  // either MFMA mode's plan fits (their k-ranges, hence partial buffers, may differ)
  const size_t a = group_plan(W, count, batch, false).ws, b = group_plan(W, count, batch, true).ws;
  *bytes = a > b ? a : b;
  return TRELLIS_OK;
}

int trellis_workspace_bytes(const trellis_desc* W, int batch, size_t* bytes) {
  if (!bytes) return TRELLIS_ERR_NULL;
  const int v = validate(W);
  if (v) return v;
  if (batch < 1) return TRELLIS_ERR_BATCH;
  return trellis_workspace_bytes_group(&W, 1, batch, bytes);
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
    case 2: return launch_decode_k<2>(W->codebook, W->V, W->bits, tile_begin, ntiles, out, st);
    case 3: return launch_decode_k<3>(W->codebook, W->V, W->bits, tile_begin, ntiles, out, st);
    default: return launch_decode_k<4>(W->codebook, W->V, W->bits, tile_begin, ntiles, out, st);
  }
}

int trellis_embed_rows(const trellis_desc* W, const int32_t* tokens, int ntok, void* out,
                       int64_t ldo, int out_dtype, void* stream) {
  const int v = validate(W);
  if (v) return v;
  if (ntok < 0) return TRELLIS_ERR_BATCH;
  if (ntok == 0) return TRELLIS_OK;
  if (!tokens || !out) return TRELLIS_ERR_NULL;
  if (out_dtype != TRELLIS_F32 && out_dtype != TRELLIS_F16) return TRELLIS_ERR_DTYPE;
  if (ntok > 1 && ldo < W->k_in) return TRELLIS_ERR_ALIGN;
  EmbedArgs a;
  a.bits = W->bits;
  a.su = W->su;
  a.sv = W->sv;
  a.isc = W->isc_scaled;
  a.osc = W->osc;
  a.tokens = tokens;
  a.out = out;
  a.ldo = ntok > 1 ? ldo : W->k_in;
  a.n = W->n_out;
  a.k = W->k_in;
  a.tiles_in = W->k_in / 16;
  a.block_in = W->block_in;
  a.block_out = W->block_out;
  a.nblk = W->k_in / W->block_in;
  a.nrm = (1.0f / std::sqrt(static_cast<float>(W->block_in))) *
          (1.0f / std::sqrt(static_cast<float>(W->block_out)));
  a.out_f16 = out_dtype == TRELLIS_F16;
  const uint64_t grid = static_cast<uint64_t>(ntok) * a.nblk;
  if (grid > 0x7FFFFFFFull) return TRELLIS_ERR_BATCH;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (W->K) {
    case 2: return launch_embed_k<2>(W->codebook, W->V, a, static_cast<unsigned>(grid), st);
    case 3: return launch_embed_k<3>(W->codebook, W->V, a, static_cast<unsigned>(grid), st);
    default: return launch_embed_k<4>(W->codebook, W->V, a, static_cast<unsigned>(grid), st);
  }
}

int trellis_encode_workspace_bytes(int K, uint32_t ntiles, size_t* bytes) {
  if (!bytes) return TRELLIS_ERR_NULL;
  if (K < 2 || K > 4) return TRELLIS_ERR_K;
  *bytes = static_cast<size_t>(encode_grid(ntiles)) * vit_bp_bytes(K);
  return TRELLIS_OK;
}

int trellis_encode_tiles(const float* w, uint32_t ntiles, int K, int codebook, uint32_t* bits,
                         float* dq, void* workspace, size_t ws_bytes, void* stream) {
  if (K < 2 || K > 4) return TRELLIS_ERR_K;
  if (codebook < TRELLIS_CB_MCG || codebook > TRELLIS_CB_1MAD) return TRELLIS_ERR_CODEBOOK;
  if (ntiles == 0) return TRELLIS_OK;
  if (!w || !bits) return TRELLIS_ERR_NULL;
  const unsigned grid = encode_grid(ntiles);
  if (!workspace || ws_bytes < static_cast<size_t>(grid) * vit_bp_bytes(K))
    return TRELLIS_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return TRELLIS_ERR_ALIGN;
  VitArgs a;
  a.w = w;
  a.bits = bits;
  a.dq = dq;
  a.bp = static_cast<uint32_t*>(workspace);
  a.ntiles = ntiles;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (K) {
    case 2: return launch_encode_k<2>(codebook, a, grid, st);
    case 3: return launch_encode_k<3>(codebook, a, grid, st);
    default: return launch_encode_k<4>(codebook, a, grid, st);
  }
}

}  // extern "C"

namespace {

// The static scratch of trellis_packed_linear_group_noalloc: a workspace that no call
// allocates. Each GPU the library runs on holds its own copy until the process ends. Its
// host-side name is not a device address: host code uses only the per-device address that
// hipGetSymbolAddress returns (scratch_ptr).
constexpr size_t NOALLOC_SCRATCH_BYTES = TRELLIS_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[MAX_DEVICES] = {};

// The current device's address of `scratch`, looked up once per device (that device
// current) and kept. The look-up may load the code object, which is not a stream-ordered
// operation: a first call under stream capture is refused instead (TRELLIS_ERR_CAPTURE).
int scratch_ptr(hipStream_t st, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return TRELLIS_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
      return TRELLIS_ERR_CAPTURE;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return TRELLIS_ERR_LAUNCH;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return TRELLIS_OK;
}

// trellis_packed_linear_group_ex, and with noalloc its variant on the static scratch: the
// plan must fit NOALLOC_SCRATCH_BYTES, and the ticket header, which an earlier call on the
// scratch may have covered with its data, is cleared before the launches.
int packed_linear_group(const trellis_desc* const* W, int count, const void* const* x,
                        const int64_t* ldx, int batch, int x_dtype, void* const* y,
                        const int64_t* ldy, int y_dtype, void* workspace, size_t ws_bytes,
                        int flags, void* stream, bool noalloc) {
  int v = validate_group(W, count);
  if (v) return v;
  if (flags & ~TRELLIS_MMA_F16) return TRELLIS_ERR_FLAGS;
  // the flag concerns the batched MFMA kernel only (the decode-GEMV is exact)
  const bool f16 = (flags & TRELLIS_MMA_F16) != 0 && !use_gemv(W, count, batch);
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
    // the kernels address a call's activations through 32-bit byte ranges
    const int64_t xes = x_dtype == TRELLIS_F16 ? 2 : 4;
    if (static_cast<int64_t>(batch) * (batch > 1 ? ldx[i] : W[i]->k_in) * xes >= (int64_t(1) << 31))
      return TRELLIS_ERR_SHAPE;
  }
  const GroupPlan p = group_plan(W, count, batch, f16);
  if (noalloc) {
    if (p.ws > NOALLOC_SCRATCH_BYTES) return TRELLIS_ERR_SCRATCH;
    v = scratch_ptr(static_cast<hipStream_t>(stream), &workspace);
    if (v) return v;
    ws_bytes = NOALLOC_SCRATCH_BYTES;
  }
  if (!workspace || ws_bytes < p.ws) return TRELLIS_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return TRELLIS_ERR_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);

  LinArgs g;
  std::memset(&g, 0, sizeof(g));
  g.nmat = count;
  g.total = p.total;
  g.nwords = W[0]->nwords;
  g.x_f16 = x_dtype == TRELLIS_F16;
  g.y_f16 = y_dtype == TRELLIS_F16;
  g.kr = p.kr;
  g.mma_f16 = f16;
  int item0 = 0;
  char* ws = static_cast<char*>(workspace);
  for (int i = 0; i < count; ++i) {
    LinMat& m = g.m[i];
    m.bits = W[i]->bits;
    m.su = W[i]->su;
    m.sv = W[i]->sv;
    m.isc = W[i]->isc_scaled;
    m.osc = W[i]->osc;
    m.ldx = ldx[i];
    m.ldy = ldy[i];
    m.n = W[i]->n_out;
    m.k = W[i]->k_in;
    m.xfw = f16 ? ((W[i]->k_in + 31) / 32) * 16 : W[i]->k_in;
    m.tiles_in = W[i]->k_in / 16;
    m.block_in = W[i]->block_in;
    m.block_out = W[i]->block_out;
    // the same correctly rounded fp32 sqrt and divide the kernels would do
    m.nrm_in = 1.0f / std::sqrt(static_cast<float>(W[i]->block_in));
    m.nrm_out = 1.0f / std::sqrt(static_cast<float>(W[i]->block_out));
    m.n_ob = p.n_ob[i];
    m.S = p.S[i];
    // exact for item * S < 2^32: items < 2^20 and S <= 256 here
    m.s_inv = p.S[i] > 1 ? static_cast<unsigned>((0x100000000ULL + p.S[i] - 1) / p.S[i]) : 0u;
    m.item0 = item0;
    item0 += p.n_ob[i] * p.ncb * p.S[i];
    m.tickets = reinterpret_cast<unsigned*>(ws + p.off_tickets[i]);
    m.part = reinterpret_cast<float*>(ws + p.off_part[i]);
    m.xf = reinterpret_cast<uint32_t*>(ws + p.off_xf[i]);
  }
  // the members' item ranges must tile the grid exactly
  if (item0 != p.total) return TRELLIS_ERR_LAUNCH;
  // bfold_kernel jobs: one per (block, column block) of every split-K member
  int nfold = 0;
  for (int i = 0; i < count; ++i) {
    g.m[i].fold0 = nfold;
    if (!p.gemv && p.S[i] > 1) nfold += p.n_ob[i] * p.ncb;
  }
  if (env_int("TRELLIS_PLAN_LOG", 0))
    std::fprintf(stderr, "trellis plan: batch=%d members=%d mode=%s kr=%d kc=%d nc=%d ncb=%d "
                         "items=%d S0=%d ws=%zu\n",
                 batch, count, p.gemv ? "gemv" : f16 ? "bgemm-f16" : "bgemm", p.kr, p.kc, p.nc,
                 p.ncb, p.total, p.S[0], p.ws);
  if (noalloc && p.gemv) {
    // only the decode-GEMV's split-K tickets must start at zero (the batched path writes
    // its folded activations and partial sums before reading them)
    bool tickets = false;
    for (int i = 0; i < count; ++i) tickets = tickets || p.S[i] > 1;
    const unsigned words = static_cast<unsigned>(p.header / 4);
    if (tickets && words > 0) {
      hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, st,
                         static_cast<uint32_t*>(workspace), words);
      if (hipGetLastError() != hipSuccess) return TRELLIS_ERR_LAUNCH;
    }
  }
  const size_t xes = g.x_f16 ? 2 : 4, yes = g.y_f16 ? 2 : 4;
  for (int b0 = 0; b0 < batch; b0 += p.nb) {
    g.batch = batch - b0 < p.nb ? batch - b0 : p.nb;
    int chunk0 = 0;
    for (int i = 0; i < count; ++i) {
      g.m[i].x = static_cast<const char*>(x[i]) + static_cast<size_t>(b0) * ldx[i] * xes;
      g.m[i].y = static_cast<char*>(y[i]) + static_cast<size_t>(b0) * ldy[i] * yes;
      g.m[i].chunk0 = chunk0;
      chunk0 += ((g.batch + xfold_rows(g.batch) - 1) / xfold_rows(g.batch)) * ((W[i]->k_in + 127) / 128);
    }
    v = p.gemv ? launch_gemv(W[0]->K, W[0]->codebook, W[0]->V, p.kc, g, st)
               : launch_bgemm(W[0]->K, W[0]->codebook, W[0]->V, p.nc, g, chunk0, nfold, st);
    if (v) return v;
  }
  return TRELLIS_OK;
}

}  // namespace

extern "C" {

int trellis_packed_linear_group_ex(const trellis_desc* const* W, int count, const void* const* x,
                                   const int64_t* ldx, int batch, int x_dtype, void* const* y,
                                   const int64_t* ldy, int y_dtype, void* workspace,
                                   size_t ws_bytes, int flags, void* stream) {
  return packed_linear_group(W, count, x, ldx, batch, x_dtype, y, ldy, y_dtype, workspace,
                             ws_bytes, flags, stream, false);
}

int trellis_packed_linear_group_noalloc(const trellis_desc* const* W, int count,
                                        const void* const* x, const int64_t* ldx, int batch,
                                        int x_dtype, void* const* y, const int64_t* ldy,
                                        int y_dtype, int flags, void* stream) {
  return packed_linear_group(W, count, x, ldx, batch, x_dtype, y, ldy, y_dtype, nullptr, 0,
                             flags, stream, true);
}

int trellis_packed_linear_group(const trellis_desc* const* W, int count, const void* const* x,
                                 const int64_t* ldx, int batch, int x_dtype, void* const* y,
                                 const int64_t* ldy, int y_dtype, void* workspace,
                                 size_t ws_bytes, void* stream) {
  return trellis_packed_linear_group_ex(W, count, x, ldx, batch, x_dtype, y, ldy, y_dtype,
                                        workspace, ws_bytes, 0, stream);
}

int trellis_packed_linear_ex(const trellis_desc* W, const void* x, int64_t ldx, int batch,
                             int x_dtype, void* y, int64_t ldy, int y_dtype, void* workspace,
                             size_t ws_bytes, int flags, void* stream) {
  return trellis_packed_linear_group_ex(&W, 1, &x, &ldx, batch, x_dtype, &y, &ldy, y_dtype,
                                        workspace, ws_bytes, flags, stream);
}

int trellis_packed_linear(const trellis_desc* W, const void* x, int64_t ldx, int batch,
                          int x_dtype, void* y, int64_t ldy, int y_dtype, void* workspace,
                          size_t ws_bytes, void* stream) {
  return trellis_packed_linear_ex(W, x, ldx, batch, x_dtype, y, ldy, y_dtype, workspace,
                                  ws_bytes, 0, stream);
}

}  // extern "C"
