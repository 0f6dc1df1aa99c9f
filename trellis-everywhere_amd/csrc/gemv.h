// gemv.h — batch-1..8 decode-GEMV for gfx950 with the incoherence-processing fold
// fused on both sides (web/packed.js:163-182 does the same as seven dispatches).
//
// Work decomposition
//   A workgroup (256 threads = 4 wave64) owns one 128-row output block `ob` (8 bands of
//   16 rows, the out-dim Hadamard block is <= 128) and one k-slice of kS tile columns.
//   Wave w: row parity PAR = w & 1, k-half kh = w >> 1. Lane l: band l>>3, tile row
//   r = 2*(l&7) + PAR. So every lane owns ONE output row and walks the tiles of its
//   k-half (columns kh, kh+2, ...), decoding its 16-window tile row per step and
//   accumulating one fp32 dot product per batch row. Row parity is wave-uniform, which
//   makes every window shift a compile-time constant (decode.h).
//   Each step a lane reads 2-3 u32 words of its tile (the 96-byte K=3 tiles of one wave
//   step sit in 8 bands x ~1 cache line each), and 16 fp16 activations, duplicated as
//   (x,x) half pairs, from LDS by broadcast (the whole wave shares the tile column).
//   The MAC is v_dot2_f32_f16(pair, (x,x), acc): hi*x + lo*x with fp32 accumulation, so
//   the weight's exact fp32 value hi+lo is never rounded.
//
// Prologue (per workgroup, its k-slice only): xf = Hb_k(isc_scaled * su * x), one
//   128-element chunk per wave pass, butterflies by lane shuffles, stored to LDS as
//   fp16 (x,x) pairs.
// Epilogue: the two k-halves are summed in LDS in a fixed order. With one k-slice the
//   block applies y = sv*osc*Hb_n(t) itself; otherwise it writes its 128 partial sums to
//   the workspace, and the last block of the output block (atomic ticket) sums the
//   slices in slice order, applies the output fold and resets the ticket to zero.
#pragma once

#include "decode.h"

namespace trellis {

struct GemvArgs {
  const uint32_t* bits;
  const float* su;
  const float* sv;
  const float* isc;  // isc_scaled
  const float* osc;
  const void* x;
  void* y;
  float* part;          // [n_ob][S][NB][128] partial sums (S > 1)
  unsigned* tickets;    // [n_ob] arrival counters (S > 1), zero between calls
  long long ldx, ldy;
  int n, k, nwords, tiles_in;
  int kS;               // tile columns per workgroup
  int S;                // k-slices
  int block_in, block_out;
  int batch;            // rows of x handled by this launch (<= NB)
  int x_f16, y_f16;
};

__device__ __forceinline__ float load_act(const void* p, long long i, int is_f16) {
  return is_f16 ? static_cast<float>(static_cast<const _Float16*>(p)[i])
                : static_cast<const float*>(p)[i];
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

template <int K, int PAR, int CB, int NB>
__device__ __forceinline__ void gemv_main(const GemvArgs& a, const uint32_t* __restrict__ xs,
                                          int M, int band, int r, int kh, float (&acc)[NB]) {
  const int nw = a.nwords;
  const int w0 = row_word0<K>(r);
  const int i0 = w0, i1 = (w0 + 1) % nw, i2 = (w0 + 2) % nw;
  constexpr bool NEED_W2 = row_needs_w2<K, PAR>();
  const int c0 = blockIdx.x % a.S * a.kS;
  const uint32_t* tp = a.bits + (static_cast<size_t>(band) * a.tiles_in + c0 + kh) * nw;
  const size_t step = 2 * static_cast<size_t>(nw);
  const int nsteps = (a.kS - kh + 1) >> 1;

  uint32_t W0 = 0, W1 = 0, W2 = 0;
  if (nsteps > 0) {
    W0 = __builtin_nontemporal_load(tp + i0);
    W1 = __builtin_nontemporal_load(tp + i1);
    if constexpr (NEED_W2) W2 = __builtin_nontemporal_load(tp + i2);
  }
  for (int s = 0; s < nsteps; ++s) {
    // prefetch the next tile of this k-half
    const uint32_t* np = (s + 1 < nsteps) ? tp + step : tp;
    const uint32_t N0 = __builtin_nontemporal_load(np + i0);
    const uint32_t N1 = __builtin_nontemporal_load(np + i1);
    uint32_t N2 = 0;
    if constexpr (NEED_W2) N2 = __builtin_nontemporal_load(np + i2);

    const int col = (kh + 2 * s) * 16;  // column inside the slice
    // 16 (x,x) pairs per batch row: 4 broadcast ds_read_b128 each
    uint32_t xq[NB][16];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const uint4* src = reinterpret_cast<const uint4*>(xs + b * M + col);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 v = src[q];
        xq[b][4 * q + 0] = v.x;
        xq[b][4 * q + 1] = v.y;
        xq[b][4 * q + 2] = v.z;
        xq[b][4 * q + 3] = v.w;
      }
    }
    if constexpr (CB == CB_1MAD) {
      decode_row<K, PAR, CB>(W0, W1, W2, [&](int c, uint32_t y) {
        const half2_t wy = {static_cast<_Float16>(static_cast<float>(y)), static_cast<_Float16>(0.0f)};
#pragma unroll
        for (int b = 0; b < NB; ++b)
          acc[b] = __builtin_amdgcn_fdot2(wy, __builtin_bit_cast(half2_t, xq[b][c]), acc[b], false);
      });
    } else {
      decode_row<K, PAR, CB>(W0, W1, W2, [&](int c, uint32_t pr) {
        const half2_t wp = __builtin_bit_cast(half2_t, pr);
#pragma unroll
        for (int b = 0; b < NB; ++b)
          acc[b] = __builtin_amdgcn_fdot2(wp, __builtin_bit_cast(half2_t, xq[b][c]), acc[b], false);
      });
    }
    W0 = N0;
    W1 = N1;
    W2 = N2;
    tp = np;
  }
}

// Output fold of one 128-row block held in LDS t[NB][128]: Hb_n, then *osc*sv.
template <int NB>
__device__ __forceinline__ void out_fold(const GemvArgs& a, float* t, int ob, int rows) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float nrm = 1.0f / sqrtf(static_cast<float>(a.block_out));
  for (int b = wave; b < a.batch; b += 4) {
    float lo = lane < rows ? t[b * 128 + lane] : 0.0f;
    float hi = lane + 64 < rows ? t[b * 128 + lane + 64] : 0.0f;
    fwht_chunk(lo, hi, a.block_out, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int rl = lane + 64 * j;
      if (rl < rows) {
        const int row = ob * 128 + rl;
        const float v = (j ? hi : lo) * nrm * a.osc[row] * a.sv[row];
        const long long o = static_cast<long long>(b) * a.ldy + row;
        if (a.y_f16)
          static_cast<_Float16*>(a.y)[o] = static_cast<_Float16>(v);
        else
          static_cast<float*>(a.y)[o] = v;
      }
    }
  }
}

template <int K, int CB, int NB>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  extern __shared__ __align__(16) uint32_t smem[];
  const int M = a.kS * 16;
  uint32_t* xs = smem;                                         // [NB][M] (x,x) pairs
  float* red = reinterpret_cast<float*>(smem + NB * M);        // [2][NB][128]
  float* tt = red + 2 * NB * 128;                              // [NB][128]
  __shared__ float xsum[NB];
  __shared__ unsigned last_flag;

  const int ob = blockIdx.x / a.S;
  const int sl = blockIdx.x % a.S;
  const int kcol0 = sl * a.kS * 16;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;

  // ---- prologue: xf = Hb_k(isc*su*x) for this k-slice, fp16 (x,x) pairs in LDS
  {
    const float nrm = 1.0f / sqrtf(static_cast<float>(a.block_in));
    const int nchunks = (M + 127) >> 7;
    float xpart = 0.0f;  // 1MAD only: sum of the fp16-rounded xf of this slice
    for (int job = wave; job < NB * nchunks; job += 4) {
      const int b = job / nchunks, ch = job % nchunks;
      const int e0 = ch * 128 + lane, e1 = e0 + 64;
      float lo = 0.0f, hi = 0.0f;
      if (b < a.batch) {
        if (e0 < M) {
          const int col = kcol0 + e0;
          lo = load_act(a.x, b * a.ldx + col, a.x_f16) * a.su[col] * a.isc[col];
        }
        if (e1 < M) {
          const int col = kcol0 + e1;
          hi = load_act(a.x, b * a.ldx + col, a.x_f16) * a.su[col] * a.isc[col];
        }
      }
      fwht_chunk(lo, hi, a.block_in, lane);
      const uint32_t plo = dup_half(lo * nrm), phi = dup_half(hi * nrm);
      if (e0 < M) xs[b * M + e0] = plo;
      if (e1 < M) xs[b * M + e1] = phi;
      if constexpr (CB == CB_1MAD) {
        float s = (e0 < M ? static_cast<float>(__builtin_bit_cast(half2_t, plo).x) : 0.0f) +
                  (e1 < M ? static_cast<float>(__builtin_bit_cast(half2_t, phi).x) : 0.0f);
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        if (lane == 0) red[job] = s;  // red is free during the prologue
      }
    }
    (void)xpart;
    __syncthreads();
    if constexpr (CB == CB_1MAD) {
      if (threadIdx.x < NB) {
        float s = 0.0f;
        for (int ch = 0; ch < nchunks; ++ch) s += red[threadIdx.x * nchunks + ch];
        xsum[threadIdx.x] = s;
      }
      __syncthreads();
    }
  }

  // ---- main loop
  const int par = wave & 1, kh = wave >> 1;
  const int bandl = lane >> 3;
  const int r = 2 * (lane & 7) + par;
  const int rl = bandl * 16 + r;                // row inside the 128-row block
  const int rows = min(128, a.n - ob * 128);    // multiple of 16
  const int band = ob * 8 + (rl < rows ? bandl : 0);  // inactive lanes re-read band 0
  float acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
  if (par == 0)
    gemv_main<K, 0, CB, NB>(a, xs, M, band, r, kh, acc);
  else
    gemv_main<K, 1, CB, NB>(a, xs, M, band, r, kh, acc);

  // ---- epilogue
#pragma unroll
  for (int b = 0; b < NB; ++b) red[(kh * NB + b) * 128 + rl] = acc[b];
  __syncthreads();
  for (int i = threadIdx.x; i < NB * 128; i += 256) {
    float v = red[i] + red[NB * 128 + i];
    if constexpr (CB == CB_1MAD) v -= 510.0f * xsum[i >> 7];
    tt[i] = v;
  }
  __syncthreads();

  if (a.S == 1) {
    if constexpr (CB == CB_1MAD)
      for (int i = threadIdx.x; i < NB * 128; i += 256) tt[i] = tt[i] / 147.800537109375f;
    __syncthreads();
    out_fold<NB>(a, tt, ob, rows);
    return;
  }

  // split-K: publish partials, last arriving block finishes the output block
  float* mypart = a.part + (static_cast<size_t>(ob) * a.S + sl) * NB * 128;
  for (int i = threadIdx.x; i < NB * 128; i += 256) mypart[i] = tt[i];
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = atomicAdd(a.tickets + ob, 1u);
    last_flag = (prev == static_cast<unsigned>(a.S - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();
  const float* obpart = a.part + static_cast<size_t>(ob) * a.S * NB * 128;
  for (int i = threadIdx.x; i < NB * 128; i += 256) {
    float v = 0.0f;
    for (int s = 0; s < a.S; ++s)
      v += __hip_atomic_load(obpart + static_cast<size_t>(s) * NB * 128 + i, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (CB == CB_1MAD) v = v / 147.800537109375f;
    tt[i] = v;
  }
  if (threadIdx.x == 0) a.tickets[ob] = 0u;
  __syncthreads();
  out_fold<NB>(a, tt, ob, rows);
}

}  // namespace trellis
