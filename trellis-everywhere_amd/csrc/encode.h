// encode.h — tail-biting trellis encoder (Viterbi) for gfx950: the counterpart of the
// reference's fused Triton encoder (src/trellis/viterbi_triton.py:34-129) and of
// qtip.viterbi_tb / _viterbi_pass (src/trellis/qtip.py:124-196), for L = 16, T = 256, V = 1.
//
// One 1024-thread workgroup per tile at a time (persistent over tiles):
//   * QTIP's two-pass tail-biting (qtip.py:124-144): pass 1 on the tile rolled by T/2,
//     unconstrained; the overlap (the top L-K bits of the state at rolled position T/2)
//     constrains pass 2 to start and end on that edge.
//   * A pass is the exact DP over the E = 2^(L-K) edges (state s = (q << (L-K)) | e, its
//     predecessor edge s >> K = (q << (L-2K)) | (e >> K)): the cost vector ping-pongs
//     between two LDS buffers (E floats each: 64 KB at K=2), one barrier per step; thread
//     j owns edges j, j + 1024, ..., and keeps the codebook values of its Q = 2^K
//     candidate states per edge in registers (they do not depend on the step).
//   * fp32 arithmetic in the reference's order without contraction, d = w - v,
//     c = d*d + cost[pred], the smallest q kept on ties, the smallest edge for the free
//     end: the same operations as the CPU restatement, so the paths agree bit for bit.
//   * Backpointers (4 bits per edge per step) go to a per-workgroup workspace region;
//     one lane walks them back, then the K-bit symbols are packed into the reference's
//     reversed stream layout (scripts/export_packed.py:27-35) with LDS atomic ORs.
#pragma once

#include "common.h"

namespace trellis {

constexpr int VIT_L = 16;
constexpr int VIT_T = 256;
constexpr int VIT_THREADS = 1024;

// Workspace bytes per workgroup: per step, each thread's edges' 4-bit backpointers in
// ceil(edges/8) words.
__host__ __device__ constexpr size_t vit_bp_bytes(int K) {
  return static_cast<size_t>(VIT_T) * ((((1 << (VIT_L - K)) / VIT_THREADS) + 7) / 8) *
         VIT_THREADS * 4;
}

struct VitArgs {
  const float* w;       // [ntiles][256] targets in tile order t = (row%16)*16 + col%16
  uint32_t* bits;       // [ntiles][8K] packed symbols
  float* dq;            // [ntiles][256] codebook value of each chosen state, or null
  uint32_t* bp;         // workspace: gridDim.x regions of vit_bp_bytes(K)
  uint32_t ntiles;
};

template <int K, int CB>
__global__ __launch_bounds__(VIT_THREADS) void viterbi_kernel(VitArgs a) {
#pragma clang fp contract(off)
  constexpr int L = VIT_L, T = VIT_T;
  constexpr int E = 1 << (L - K), Q = 1 << K;
  constexpr int EPT = E / VIT_THREADS;            // edges per thread: 16, 8, 4
  constexpr int BPW = (EPT + 7) / 8;              // backpointer words per thread per step
  constexpr int NWK = 8 * K;
  static_assert(EPT >= 1 && EPT <= 16, "edges per thread");
  __shared__ float cost[2][E];
  __shared__ float wseq[T];
  __shared__ int32_t states[T];
  __shared__ uint32_t packed[NWK];
  __shared__ int32_t edge_sh;
  const int tid = threadIdx.x;
  uint32_t* bp = a.bp + static_cast<size_t>(blockIdx.x) * (vit_bp_bytes(K) / 4);

  // the codebook values of this thread's candidate states (independent of the step)
  float cv[EPT][Q];
#pragma unroll
  for (int i = 0; i < EPT; ++i)
#pragma unroll
    for (int q = 0; q < Q; ++q)
      cv[i][q] = cb_exact<CB>(cb_raw<CB>(static_cast<uint32_t>((q << (L - K)) | (i * VIT_THREADS + tid))));

  for (uint32_t tile = blockIdx.x; tile < a.ntiles; tile += gridDim.x) {
    const float* wt = a.w + static_cast<size_t>(tile) * T;
    int overlap = -1;
    for (int pass = 0; pass < 2; ++pass) {
      // pass 0: the tile rolled by T/2 (torch.roll: wr[t] = w[(t - T/2) mod T])
      if (tid < T) wseq[tid] = pass == 0 ? wt[(tid + T / 2) % T] : wt[tid];
#pragma unroll
      for (int i = 0; i < EPT; ++i) {
        const int e = i * VIT_THREADS + tid;
        cost[0][e] = overlap < 0 || e == overlap ? 0.0f : __FLT_MAX__ / 4.0f;
      }
      __syncthreads();
      int cur = 0;
      for (int t = 0; t < T; ++t) {
        const float w_t = wseq[t];
        uint32_t word[BPW];
#pragma unroll
        for (int b = 0; b < BPW; ++b) word[b] = 0u;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
          const int e = i * VIT_THREADS + tid;
          float best = __FLT_MAX__;
          int bq = 0;
#pragma unroll
          for (int q = 0; q < Q; ++q) {
            const float d = w_t - cv[i][q];
            const float c = d * d + cost[cur][(q << (L - 2 * K)) | (e >> K)];
            if (c < best) {
              best = c;
              bq = q;
            }
          }
          cost[cur ^ 1][e] = best;
          word[i >> 3] |= static_cast<uint32_t>(bq) << (4 * (i & 7));
        }
#pragma unroll
        for (int b = 0; b < BPW; ++b)
          bp[(static_cast<size_t>(t) * BPW + b) * VIT_THREADS + tid] = word[b];
        __syncthreads();
        cur ^= 1;
      }
      // the final edge: the smallest-cost edge (ties: the smallest) or the overlap
      if (overlap < 0) {
        // per-thread best of its edges, then a workgroup argmin in edge order
        float best = __FLT_MAX__;
        int be = 0;
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
          const int e = i * VIT_THREADS + tid;
          const float c = cost[cur][e];
          if (c < best || (c == best && e < be)) {
            best = c;
            be = e;
          }
        }
        __syncthreads();   // every thread has read the final costs
        // reduce (cost, edge) pairs through the now-free other buffer
        float* rc = cost[cur ^ 1];
        int32_t* re = reinterpret_cast<int32_t*>(cost[cur ^ 1] + VIT_THREADS);
        rc[tid] = best;
        re[tid] = be;
        __syncthreads();
        for (int s = VIT_THREADS / 2; s > 0; s >>= 1) {
          if (tid < s) {
            const float c2 = rc[tid + s];
            const int e2 = re[tid + s];
            if (c2 < rc[tid] || (c2 == rc[tid] && e2 < re[tid])) {
              rc[tid] = c2;
              re[tid] = e2;
            }
          }
          __syncthreads();
        }
        if (tid == 0) edge_sh = re[0];
      } else if (tid == 0) {
        edge_sh = overlap;
      }
      // the barrier makes every thread's backpointer stores visible to the walking lane
      __syncthreads();
      if (tid == 0) {
        int e = edge_sh;
        for (int t = T - 1; t >= 0; --t) {
          const int i = e / VIT_THREADS, j = e % VIT_THREADS;
          const uint32_t wd = __builtin_nontemporal_load(
              bp + (static_cast<size_t>(t) * BPW + (i >> 3)) * VIT_THREADS + j);
          const int q = static_cast<int>((wd >> (4 * (i & 7))) & 15u);
          const int s = (q << (L - K)) | e;
          states[t] = s;
          e = s >> K;
        }
      }
      __syncthreads();
      if (pass == 0) overlap = states[T / 2] >> K;
    }
    // pass 2's states: symbols packed reversed (symbol t at stream bits (255-t)*K), and
    // the dequantized values
    if (tid < NWK) packed[tid] = 0u;
    __syncthreads();
    if (tid < T) {
      const uint32_t sym = static_cast<uint32_t>(states[tid]) & ((1u << K) - 1u);
      const int p = (T - 1 - tid) * K;
      atomicOr(&packed[p >> 5], sym << (p & 31));
      if ((p & 31) + K > 32) atomicOr(&packed[(p >> 5) + 1], sym >> (32 - (p & 31)));
      if (a.dq)
        a.dq[static_cast<size_t>(tile) * T + tid] =
            cb_exact<CB>(cb_raw<CB>(static_cast<uint32_t>(states[tid])));
    }
    __syncthreads();
    if (tid < NWK) a.bits[static_cast<size_t>(tile) * NWK + tid] = packed[tid];
    __syncthreads();
  }
}

}  // namespace trellis
