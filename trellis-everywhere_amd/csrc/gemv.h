// gemv.h — persistent, grouped decode-GEMV for gfx950 (batch 1..8) with the
// incoherence-processing fold fused on both sides (web/packed.js:163-182 runs it as seven
// dispatches per linear).
//
// Work items
//   One launch serves a group of up to GEMV_MAX_GROUP packed linears (e.g. q/k/v, or
//   gate/up, which share an input; or any set of independent linears). Each matrix is cut
//   into items = (128-row output block ob, k-slice sl of kS = 2*TPW tile columns); the
//   out-dim Hadamard block is <= 128, so a 128-row block is closed under the output fold.
//   The grid is persistent (a few workgroups per CU) and workgroup g takes items
//   g, g + grid, g + 2*grid, ...
//
// Inside an item (256 threads = 4 wave64)
//   Wave w: row parity PAR = w & 1, k-half kh = w >> 1. Lane l: band l>>3, tile row
//   r = 2*(l&7) + PAR; every lane owns ONE output row and the TPW tiles of its k-half.
//   Parity is wave-uniform, so every window shift is a compile-time constant (decode.h).
//   The activations of the slice are folded first, xf = Hb_k(isc_scaled*su*x), by lane
//   shuffles, and kept in LDS as fp16 (x,x) pairs read by broadcast. The MAC is
//   v_dot2_f32_f16(pair, (x,x), acc) = hi*x + lo*x with fp32 accumulation, so the
//   weight's exact fp32 value hi+lo is never rounded. The two k-halves are summed in LDS
//   in a fixed order.
//
// Pipeline (per workgroup, one item per iteration)
//   1. fold the activations of item i (prefetched during item i-1)
//   2. prefetch item i+1: its 2-3 packed words per tile row and its activations, pinned
//      ahead of the decode by a compiler memory barrier
//   3. decode + MAC of item i
//   4. wait for all earlier memory traffic (it was issued a whole decode ago)
//   5. if the ticket taken two items ago said "last": sum that output block's partials
//      in slice order (deterministic), apply y = sv*osc*Hb_n(t), reset its ticket
//   6. take the ticket of the item stored one iteration ago (result read next time)
//   7. publish item i's partial sums (or, with a single k-slice, fold and store y now)
//   Tickets are deferred so no store/atomic round trip sits between two decodes; the
//   only exposed latencies are the first prefetch, the 1-in-S "last" reads and the drain.
//   Everything exchanged between workgroups uses agent-scope atomic accesses (coherent
//   across the XCDs' separate L2s, write-through on store) and explicit vmcnt waits: no
//   __threadfence(), whose buffer_wbl2/buffer_inv would write back and invalidate L2.
#pragma once

#include "decode.h"

namespace trellis {

constexpr int GEMV_MAX_GROUP = 8;

struct GemvMat {
  const uint32_t* bits;
  const float* su;
  const float* sv;
  const float* isc;     // isc_scaled = f32(isc) * scale
  const float* osc;
  const void* x;
  void* y;
  float* part;          // [n_ob][S][NB][128] partial sums (S > 1)
  unsigned* tickets;    // [n_ob] arrival counters (S > 1), zero between calls
  long long ldx, ldy;
  int n, k, tiles_in, block_in, block_out;
  int n_ob, S;
  int item0;            // first group-wide item index of this matrix
};

struct GemvGroupArgs {
  GemvMat m[GEMV_MAX_GROUP];
  int nmat;
  int total;            // items over all matrices
  int nwords;
  int batch;            // rows of x handled by this launch (<= NB)
  int x_f16, y_f16;
};

// Activation i of an f16 or f32 array, read as the aligned u32 word holding it so the
// load is branch-free (f16 arrays must be 4-byte aligned with an even row stride).
__device__ __forceinline__ uint32_t load_act_word(const void* p, long long i, int is_f16) {
  const long long byte = is_f16 ? ((2 * i) & ~3LL) : 4 * i;
  return *reinterpret_cast<const uint32_t*>(static_cast<const char*>(p) + byte);
}

__device__ __forceinline__ float act_value(uint32_t w, long long i, int is_f16) {
  if (!is_f16) return __builtin_bit_cast(float, w);
  const uint16_t h = static_cast<uint16_t>((i & 1) ? (w >> 16) : (w & 0xFFFFu));
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Butterflies of a normalized-free block Hadamard (block B <= 128) on a 128-element
// chunk held as lo = e[lane], hi = e[lane + 64].
__device__ __forceinline__ void fwht_chunk(float& lo, float& hi, int B, int lane) {
  for (int h = 1; h < B && h < 64; h <<= 1) {
    const float plo = __shfl_xor(lo, h);
    const float phi = __shfl_xor(hi, h);
    const bool upper = (lane & h) != 0;
    lo = upper ? plo - lo : lo + plo;
    hi = upper ? phi - hi : hi + phi;
  }
  if (B == 128) {
    const float a = lo, b = hi;
    lo = a + b;
    hi = a - b;
  }
}

__device__ __forceinline__ uint32_t dup_half(float v) {
  const _Float16 h = static_cast<_Float16>(v);
  const uint16_t u = __builtin_bit_cast(uint16_t, h);
  return (static_cast<uint32_t>(u) << 16) | u;
}

// Position of one item.
struct Item {
  int mi, ob, sl;
};

__device__ __forceinline__ Item locate(const GemvGroupArgs& g, int it) {
  int mi = 0;
#pragma unroll
  for (int j = 1; j < GEMV_MAX_GROUP; ++j)
    if (j < g.nmat && it >= g.m[j].item0) mi = j;
  const int local = it - g.m[mi].item0;
  return {mi, local / g.m[mi].S, local % g.m[mi].S};
}

// Registers prefetched for one item: this lane's packed words and its share of the
// slice's activations (x word, su, isc for two elements per fold job).
template <int NB, int TPW>
struct Prefetch {
  static constexpr int M = 32 * TPW;
  static constexpr int NCH = (M + 127) / 128;
  static constexpr int JOBS = (NB * NCH + 3) / 4;  // fold jobs per wave
  uint32_t W[TPW][3];
  uint32_t xw[JOBS][2];
  float su[JOBS][2], is[JOBS][2];
};

template <int K, int NB, int TPW>
__device__ __forceinline__ void prefetch(const GemvGroupArgs& g, const Item& t,
                                         Prefetch<NB, TPW>& p) {
  const GemvMat& m = g.m[t.mi];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int par = wave & 1, kh = wave >> 1;
  const int bandl = lane >> 3, r = 2 * (lane & 7) + par;
  const int rows = min(128, m.n - t.ob * 128);
  const int band = t.ob * 8 + (bandl * 16 + r < rows ? bandl : 0);  // idle lanes re-read
  const int nw = g.nwords;
  const int w0 = row_word0<K>(r);
  const int i0 = w0, i1 = (w0 + 1) % nw, i2 = (w0 + 2) % nw;
  const uint32_t* bandp = m.bits + static_cast<size_t>(band) * m.tiles_in * nw;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    // a partial last slice re-reads its last tile; its activations are zero in LDS
    const int col = min(t.sl * 2 * TPW + kh + 2 * j, m.tiles_in - 1);
    const uint32_t* tp = bandp + static_cast<size_t>(col) * nw;
    p.W[j][0] = __builtin_nontemporal_load(tp + i0);
    p.W[j][1] = __builtin_nontemporal_load(tp + i1);
    p.W[j][2] = __builtin_nontemporal_load(tp + i2);
  }
  constexpr int M = Prefetch<NB, TPW>::M, NCH = Prefetch<NB, TPW>::NCH;
  const int kcol0 = t.sl * M;
  const int kvalid = min(M, m.k - kcol0);
#pragma unroll
  for (int q = 0; q < Prefetch<NB, TPW>::JOBS; ++q) {
    const int job = wave + 4 * q;
    const int b = min(job / NCH, g.batch - 1), ch = job % NCH;
    const int e0 = ch * 128 + lane;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ci = kcol0 + min(e0 + 64 * h, kvalid - 1);
      p.xw[q][h] = load_act_word(m.x, b * m.ldx + ci, g.x_f16);
      p.su[q][h] = m.su[ci];
      p.is[q][h] = m.isc[ci];
    }
  }
}

// xf of the item's slice into LDS xs[NB][M] as (x,x) fp16 pairs; for 1MAD also the sum
// of the rounded xf of each batch row (xsum).
template <int CB, int NB, int TPW>
__device__ __forceinline__ void fold_x(const GemvGroupArgs& g, const Item& t,
                                       const Prefetch<NB, TPW>& p, uint32_t* xs, float* xpart,
                                       float* xsum) {
  const GemvMat& m = g.m[t.mi];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  constexpr int M = Prefetch<NB, TPW>::M, NCH = Prefetch<NB, TPW>::NCH;
  const int kcol0 = t.sl * M;
  const int kvalid = min(M, m.k - kcol0);
  const float nrm = 1.0f / sqrtf(static_cast<float>(m.block_in));
#pragma unroll
  for (int q = 0; q < Prefetch<NB, TPW>::JOBS; ++q) {
    const int job = wave + 4 * q;
    if (job >= NB * NCH) break;  // wave-uniform
    const int b = job / NCH, ch = job % NCH;
    const int e0 = ch * 128 + lane, e1 = e0 + 64;
    const bool live = b < g.batch;
    const long long xi0 = min(b, g.batch - 1) * m.ldx + kcol0 + min(e0, kvalid - 1);
    const long long xi1 = min(b, g.batch - 1) * m.ldx + kcol0 + min(e1, kvalid - 1);
    float lo = (live && e0 < kvalid) ? act_value(p.xw[q][0], xi0, g.x_f16) * p.su[q][0] * p.is[q][0] : 0.0f;
    float hi = (live && e1 < kvalid) ? act_value(p.xw[q][1], xi1, g.x_f16) * p.su[q][1] * p.is[q][1] : 0.0f;
    fwht_chunk(lo, hi, m.block_in, lane);
    const uint32_t plo = dup_half(lo * nrm), phi = dup_half(hi * nrm);
    if (e0 < M) xs[b * M + e0] = plo;
    if (e1 < M) xs[b * M + e1] = phi;
    if constexpr (CB == CB_1MAD) {
      float s = static_cast<float>(__builtin_bit_cast(half2_t, plo).x) +
                static_cast<float>(__builtin_bit_cast(half2_t, phi).x);
      for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
      if (lane == 0) xpart[job] = s;
    }
  }
  __syncthreads();
  if constexpr (CB == CB_1MAD) {
    if (threadIdx.x < NB) {
      float s = 0.0f;
      for (int ch = 0; ch < NCH; ++ch) s += xpart[threadIdx.x * NCH + ch];
      xsum[threadIdx.x] = s;
    }
  }
}

template <int K, int PAR, int CB, int NB, int TPW>
__device__ __forceinline__ void decode_mac(const uint32_t* __restrict__ xs, int kh,
                                           const uint32_t (&W)[TPW][3], float (&acc)[NB]) {
  constexpr int M = 32 * TPW;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int col = (kh + 2 * j) * 16;  // column inside the slice
    if constexpr (NB == 1) {
      uint32_t xq[16];
      const uint4* src = reinterpret_cast<const uint4*>(xs + col);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 v = src[q];
        xq[4 * q] = v.x;
        xq[4 * q + 1] = v.y;
        xq[4 * q + 2] = v.z;
        xq[4 * q + 3] = v.w;
      }
      decode_row<K, PAR, CB>(W[j][0], W[j][1], W[j][2], [&](int c, uint32_t raw) {
        half2_t wv;
        if constexpr (CB == CB_1MAD)
          wv = half2_t{static_cast<_Float16>(static_cast<float>(raw)), static_cast<_Float16>(0.0f)};
        else
          wv = __builtin_bit_cast(half2_t, raw);
        acc[0] = __builtin_amdgcn_fdot2(wv, __builtin_bit_cast(half2_t, xq[c]), acc[0], false);
      });
    } else {
      decode_row<K, PAR, CB>(W[j][0], W[j][1], W[j][2], [&](int c, uint32_t raw) {
        half2_t wv;
        if constexpr (CB == CB_1MAD)
          wv = half2_t{static_cast<_Float16>(static_cast<float>(raw)), static_cast<_Float16>(0.0f)};
        else
          wv = __builtin_bit_cast(half2_t, raw);
#pragma unroll
        for (int b = 0; b < NB; ++b)
          acc[b] = __builtin_amdgcn_fdot2(wv, __builtin_bit_cast(half2_t, xs[b * M + col + c]),
                                          acc[b], false);
      });
    }
  }
}

// y = sv * osc * Hb_n(t) for the 128-row block `ob` of matrix m; t in LDS [NB][128].
template <int NB>
__device__ __forceinline__ void out_fold(const GemvGroupArgs& g, const GemvMat& m, const float* t,
                                         int ob) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rows = min(128, m.n - ob * 128);
  const float nrm = 1.0f / sqrtf(static_cast<float>(m.block_out));
  for (int b = wave; b < g.batch; b += 4) {
    float lo = lane < rows ? t[b * 128 + lane] : 0.0f;
    float hi = lane + 64 < rows ? t[b * 128 + lane + 64] : 0.0f;
    fwht_chunk(lo, hi, m.block_out, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int rl = lane + 64 * j;
      if (rl < rows) {
        const int row = ob * 128 + rl;
        const float v = (j ? hi : lo) * nrm * m.osc[row] * m.sv[row];
        const long long o = static_cast<long long>(b) * m.ldy + row;
        if (g.y_f16)
          static_cast<_Float16*>(m.y)[o] = static_cast<_Float16>(v);
        else
          static_cast<float*>(m.y)[o] = v;
      }
    }
  }
}

// The last arriving item of an output block: sum its S partials in slice order, divide
// for 1MAD, fold, store y, reset the ticket. Uses ft[NB*128] and red[2*NB*128] in LDS.
template <int CB, int NB>
__device__ __forceinline__ void finish_block(const GemvGroupArgs& g, const Item& t, float* ft,
                                             float* red) {
  const GemvMat& m = g.m[t.mi];
  const float* obpart = m.part + static_cast<size_t>(t.ob) * m.S * NB * 128;
  constexpr int E = NB * 128;
  constexpr int SPLIT = E < 256 ? 256 / E : 1;  // threads per element
  for (int i0 = 0; i0 < E; i0 += 256 / SPLIT) {
    const int i = i0 + threadIdx.x / SPLIT;
    const int h = threadIdx.x % SPLIT;
    float v = 0.0f;
    for (int s0 = h; s0 < m.S; s0 += 8 * SPLIT) {
      float q[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int s = s0 + u * SPLIT;
        q[u] = s < m.S ? __hip_atomic_load(obpart + static_cast<size_t>(s) * E + i,
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                       : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) v += q[u];
    }
    red[h * E + i] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < E; i += 256) {
    float v = 0.0f;
    for (int h = 0; h < SPLIT; ++h) v += red[h * E + i];
    if constexpr (CB == CB_1MAD) v = v / 147.800537109375f;
    ft[i] = v;
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(m.tickets + t.ob, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  out_fold<NB>(g, m, ft, t.ob);
}

template <int K, int CB, int NB, int TPW>
__device__ __forceinline__ void run_item(const GemvGroupArgs& g, const Item& cur, int nxt,
                                         const Prefetch<NB, TPW>& pc, Prefetch<NB, TPW>& pn,
                                         int& p1, int& p2, unsigned& tk2, uint32_t* xs, float* red,
                                         float* tt, float* ft, float* xsum, unsigned* flag) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int par = wave & 1, kh = wave >> 1;
  const int rl = (lane >> 3) * 16 + 2 * (lane & 7) + par;

  // 1. activations of this item
  fold_x<CB, NB, TPW>(g, cur, pc, xs, red, xsum);
  __syncthreads();
  // 2. prefetch the next item, pinned ahead of the decode
  if (nxt < g.total) prefetch<K, NB, TPW>(g, locate(g, nxt), pn);
  asm volatile("" ::: "memory");
  // 3. decode + MAC; k-halves summed in a fixed order
  float acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
  if (par == 0)
    decode_mac<K, 0, CB, NB, TPW>(xs, kh, pc.W, acc);
  else
    decode_mac<K, 1, CB, NB, TPW>(xs, kh, pc.W, acc);
#pragma unroll
  for (int b = 0; b < NB; ++b) red[(kh * NB + b) * 128 + rl] = acc[b];
  __syncthreads();
  for (int i = threadIdx.x; i < NB * 128; i += 256) {
    float v = red[i] + red[NB * 128 + i];
    if constexpr (CB == CB_1MAD) v -= 510.0f * xsum[i >> 7];
    tt[i] = v;
  }
  // 4. everything issued before (the previous item's partial stores and ticket, this
  //    prefetch) is complete after this wait
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // 5. the ticket taken one iteration ago
  if (threadIdx.x == 0) {
    unsigned last = 0u;
    if (p2 >= 0) last = tk2 == static_cast<unsigned>(g.m[locate(g, p2).mi].S - 1) ? 1u : 0u;
    *flag = last;
  }
  __syncthreads();
  if (*flag) finish_block<CB, NB>(g, locate(g, p2), ft, red);
  // 6. ticket of the item stored one iteration ago (its stores completed at step 4)
  p2 = p1;
  if (p2 >= 0 && threadIdx.x == 0) {
    const Item t = locate(g, p2);
    tk2 = __hip_atomic_fetch_add(g.m[t.mi].tickets + t.ob, 1u, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
  }
  // 7. publish this item
  const GemvMat& m = g.m[cur.mi];
  if (m.S > 1) {
    float* mypart = m.part + (static_cast<size_t>(cur.ob) * m.S + cur.sl) * NB * 128;
    for (int i = threadIdx.x; i < NB * 128; i += 256)
      __hip_atomic_store(mypart + i, tt[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    p1 = g.m[cur.mi].item0 + cur.ob * m.S + cur.sl;
  } else {
    if constexpr (CB == CB_1MAD)
      for (int i = threadIdx.x; i < NB * 128; i += 256) tt[i] = tt[i] / 147.800537109375f;
    __syncthreads();
    out_fold<NB>(g, m, tt, cur.ob);
    p1 = -1;
  }
  __syncthreads();
}

template <int K, int CB, int NB, int TPW>
__global__ __launch_bounds__(256) void gemv_group_kernel(GemvGroupArgs g) {
  constexpr int M = 32 * TPW;
  __shared__ __align__(16) uint32_t xs[NB * M];  // (x,x) pairs of the slice
  __shared__ float red[2 * NB * 128];
  __shared__ float tt[NB * 128];
  __shared__ float ft[NB * 128];
  __shared__ float xsum[NB];
  __shared__ unsigned flag;

  int p1 = -1, p2 = -1;   // item stored last iteration / item whose ticket is pending
  unsigned tk2 = 0u;      // pending ticket value (thread 0)
  Prefetch<NB, TPW> pa, pb;
  int it = blockIdx.x;
  if (it < g.total) prefetch<K, NB, TPW>(g, locate(g, it), pa);
  // two items per loop trip so the prefetch buffers alternate without copies
  while (it < g.total) {
    run_item<K, CB, NB, TPW>(g, locate(g, it), it + gridDim.x, pa, pb, p1, p2, tk2, xs, red,
                             tt, ft, xsum, &flag);
    it += gridDim.x;
    if (it >= g.total) break;
    run_item<K, CB, NB, TPW>(g, locate(g, it), it + gridDim.x, pb, pa, p1, p2, tk2, xs, red,
                             tt, ft, xsum, &flag);
    it += gridDim.x;
  }
  // drain: the pending ticket, then the last stored item
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (threadIdx.x == 0) {
    unsigned last = 0u;
    if (p2 >= 0) last = tk2 == static_cast<unsigned>(g.m[locate(g, p2).mi].S - 1) ? 1u : 0u;
    flag = last;
  }
  __syncthreads();
  if (flag) finish_block<CB, NB>(g, locate(g, p2), ft, red);
  if (p1 >= 0) {
    __syncthreads();
    if (threadIdx.x == 0) {
      const Item t = locate(g, p1);
      const unsigned v = __hip_atomic_fetch_add(g.m[t.mi].tickets + t.ob, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      flag = v == static_cast<unsigned>(g.m[t.mi].S - 1) ? 1u : 0u;
    }
    __syncthreads();
    if (flag) finish_block<CB, NB>(g, locate(g, p1), ft, red);
  }
}

}  // namespace trellis
