// tmk.h — decode-to-MFMA packed linear for gfx950 ("tile-MFMA"), batch 1..16, with the
// incoherence-processing fold on both sides (web/packed.js:163-182 runs it as seven
// dispatches per linear).
//
// Launches per call:
//   1. (batch > 1) xfold_kernel: xf = Hb_k(isc_scaled * su * x) for every member and
//      batch row, once, stored to the workspace as fp16 (x, x) pairs (the MFMA B-operand
//      format). At batch 1 every workgroup folds its own k-slice instead (one 128-column
//      chunk per wave, lane shuffles), which saves a launch.
//   2. tmk_kernel: the decode-matmul with the output fold.
//
// tmk_kernel work item: one matrix, one 128-row output block `ob` (8 bands of 16 rows;
// the out-dim Hadamard block is <= 128), one k-slice of KS tile columns. 4 waves; wave w
// owns bands 2w and 2w+1 for the whole slice.
//   * The slice's packed words (8 bands x KS tiles x nwords u32, contiguous per band) are
//     loaded with coalesced 16-byte loads into LDS.
//   * v_mfma_f32_16x16x32_f16 works on one 16x16 tile: lane l = (tile row r = l%16,
//     column group g = l/16) decodes the 4 windows t = 16r + 4g + q (q = 0..3). They sit in
//     one 32-bit funnel of the stream (3K+16 <= 28 bits), so one v_alignbit + one
//     v_bfe_u32 per window extract them; the state is multiplied (v_mul_lo_u32, full rate
//     on gfx950) and the lop3 (v_bitop3_b32) result IS the fp16 pair (lo, hi) of the
//     weight. Its two halves are two adjacent k elements of the A operand, and the B
//     operand holds x twice at those positions, so the MFMA accumulates (hi + lo) * x in
//     fp32: the exact codebook value is never rounded. B columns are the batch rows.
//   * Split-K epilogue: partial sums go to the workspace with agent-scope atomic stores;
//     the last workgroup of the output block (atomic ticket) sums the slices in slice
//     order (deterministic), applies y = sv * osc * Hb_n(t) and resets the ticket. No
//     __threadfence (its buffer_wbl2 / buffer_inv would write back and invalidate L2).
#pragma once

#include "decode.h"

namespace trellis {

constexpr int TMK_MAX_GROUP = 8;
constexpr int TMK_MAX_BATCH = 16;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct TmkMat {
  const uint32_t* bits;
  const float* su;
  const float* sv;
  const float* isc;     // isc_scaled = f32(isc) * scale
  const float* osc;
  const void* x;
  void* y;
  uint32_t* xf;         // workspace: [batch][k] fp16 (x,x) pairs
  float* part;          // workspace: [n_ob][S][batch][128] partial sums (S > 1)
  unsigned* tickets;    // workspace: [n_ob] arrival counters (S > 1), zero between calls
  long long ldx, ldy;
  int n, k, tiles_in, block_in, block_out;
  int n_ob, S;
  int item0;            // first group-wide work item of this matrix
  int chunk0;           // first group-wide x-fold job of this matrix
  int fold0;            // first group-wide bfold_kernel workgroup of this matrix
};

struct TmkArgs {
  TmkMat m[TMK_MAX_GROUP];
  int nmat;
  int total;            // work items (tmk_kernel) or x-fold jobs (xfold_kernel)
  int nwords;
  int batch;            // 1..16
  int x_f16, y_f16;
  int kr;               // gemv_kernel: tile columns per k-range
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

__device__ __forceinline__ int locate_fold(const TmkArgs& g, int it) {
  int mi = 0;
#pragma unroll
  for (int j = 1; j < TMK_MAX_GROUP; ++j)
    if (j < g.nmat && it >= g.m[j].fold0) mi = j;
  return mi;
}

__device__ __forceinline__ int locate_mat(const TmkArgs& g, int it, bool by_chunk) {
  int mi = 0;
#pragma unroll
  for (int j = 1; j < TMK_MAX_GROUP; ++j)
    if (j < g.nmat && it >= (by_chunk ? g.m[j].chunk0 : g.m[j].item0)) mi = j;
  return mi;
}

// ---------------------------------------------------------------- x fold
// One wave per (matrix, batch row, 128-column chunk): xf = Hb_k(isc * su * x) scaled by
// 1/sqrt(block_in), stored as (x,x) fp16 pairs. Defined in one translation unit only.
#ifdef TRELLIS_XFOLD_DEFINE
__global__ __launch_bounds__(256) void xfold_kernel(TmkArgs g) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int job = blockIdx.x * 4 + wave;
  if (job >= g.total) return;
  const int mi = locate_mat(g, job, true);
  const TmkMat& m = g.m[mi];
  const int local = job - m.chunk0;
  const int nch = (m.k + 127) / 128;
  const int b = local / nch, ch = local % nch;
  const int kvalid = min(128, m.k - ch * 128);
  const int e0 = lane, e1 = lane + 64;
  const int c0i = ch * 128 + min(e0, kvalid - 1), c1i = ch * 128 + min(e1, kvalid - 1);
  const long long x0i = b * m.ldx + c0i, x1i = b * m.ldx + c1i;
  const uint32_t w0 = load_act_word(m.x, x0i, g.x_f16);
  const uint32_t w1 = load_act_word(m.x, x1i, g.x_f16);
  const float s0 = m.su[c0i] * m.isc[c0i], s1 = m.su[c1i] * m.isc[c1i];
  float lo = e0 < kvalid ? act_value(w0, x0i, g.x_f16) * s0 : 0.0f;
  float hi = e1 < kvalid ? act_value(w1, x1i, g.x_f16) * s1 : 0.0f;
  fwht_chunk(lo, hi, m.block_in, lane);
  const float nrm = 1.0f / sqrtf(static_cast<float>(m.block_in));
  uint32_t* dst = m.xf + static_cast<size_t>(b) * m.k + ch * 128;
  if (e0 < kvalid) dst[e0] = dup_half(lo * nrm);
  if (e1 < kvalid) dst[e1] = dup_half(hi * nrm);
}
#endif

// ---------------------------------------------------------------- output fold
// y = sv * osc * Hb_n(t) for the 128-row block `ob`; t in LDS [batch][128].
__device__ __forceinline__ void tmk_out_fold(const TmkArgs& g, const TmkMat& m, const float* t,
                                             int ob, int is_1mad) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int rows = min(128, m.n - ob * 128);
  float nrm = 1.0f / sqrtf(static_cast<float>(m.block_out));
  for (int b = wave; b < g.batch; b += 4) {
    float lo = lane < rows ? t[b * 128 + lane] : 0.0f;
    float hi = lane + 64 < rows ? t[b * 128 + lane + 64] : 0.0f;
    if (is_1mad) {
      lo = lo / 147.800537109375f;
      hi = hi / 147.800537109375f;
    }
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

// ---------------------------------------------------------------- decode -> MFMA
// The A operand of one band-tile for this lane (decode_quad). 1MAD yields (y - 510) as an
// exact fp16 in the low half (the division by 147.800537109375 follows the sum).
template <int K, int CB>
__device__ __forceinline__ half8_t decode_a(uint32_t wlo, uint32_t whi, int sh) {
  uint32_t a4[4];
  decode_quad<K, CB>(wlo, whi, sh, a4);
  if constexpr (CB == CB_1MAD) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const _Float16 h = static_cast<_Float16>(static_cast<float>(static_cast<int>(a4[q]) - 510));
      a4[q] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
    }
  }
  return __builtin_bit_cast(half8_t, a4);
}

template <int K, int CB, int KS, int XB>
__global__ __launch_bounds__(256) void tmk_kernel(TmkArgs g) {
  // XB: batch rows the LDS buffers are sized for (1, or TMK_MAX_BATCH)
  constexpr int NWK = 8 * K;                    // words per tile
  constexpr int BSTRIDE = KS * NWK + 4;         // LDS words per band (padded)
  constexpr int CH16 = KS * NWK / 4;            // 16-byte chunks per band
  constexpr int LOADS = (8 * CH16 + 255) / 256; // 16-byte bit loads per thread
  constexpr int XW = KS * 16;                   // activation words per batch row
  constexpr int XLOADS = (XB * XW / 4 + 255) / 256;
  __shared__ __align__(16) uint32_t tl[8 * BSTRIDE];
  __shared__ __align__(16) uint32_t xs[XB * XW];
  __shared__ float tt[XB * 128];
  __shared__ float red[2 * 128];
  __shared__ unsigned last_flag;

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int mi = locate_mat(g, blockIdx.x, false);
  const TmkMat& m = g.m[mi];
  const int local = blockIdx.x - m.item0;
  const int ob = local / m.S, sl = local % m.S;
  const int c0 = sl * KS;
  const int rows = min(128, m.n - ob * 128);
  const int nb = rows / 16;  // live bands of this block

  // ---- packed words of the slice: coalesced 16-byte loads (tiles past k_in re-read the
  // last tile; their activations are zero)
  u32x4_t v[LOADS];
#pragma unroll
  for (int q = 0; q < LOADS; ++q) {
    const int ch = threadIdx.x + 256 * q;
    const int band = min(ch / CH16, nb - 1), off = ch % CH16;
    const int tile = min(c0 + off / (NWK / 4), m.tiles_in - 1);
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(
        m.bits + (static_cast<size_t>(ob * 8 + band) * m.tiles_in + tile) * NWK) + (off % (NWK / 4));
    v[q] = __builtin_nontemporal_load(src);
  }
  // ---- activations of the slice as (x,x) pairs. Batch 1 folds its own slice here
  // (xf = Hb_k(isc*su*x), one 128-column chunk per wave, loads issued with the bit loads);
  // larger batches read what xfold_kernel wrote.
  constexpr int NCHK = (XW + 127) / 128;        // 128-column chunks of the slice
  u32x4_t xv[XLOADS];
  uint32_t fw[2] = {0u, 0u};
  float fs[2] = {0.f, 0.f};
  const int kslice = c0 * 16;
  const int kvalid = min(XW, m.k - kslice);
  if constexpr (XB == 1) {
    if (wave < NCHK) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int e = wave * 128 + lane + 64 * h;
        const int ci = kslice + min(e, kvalid - 1);
        fw[h] = load_act_word(m.x, ci, g.x_f16);
        fs[h] = m.su[ci] * m.isc[ci];
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < XLOADS; ++q) {
      const int ch = threadIdx.x + 256 * q;
      const int b = min(ch / (XW / 4), g.batch - 1), off = ch % (XW / 4);
      const int col = min(kslice + 4 * off, m.k - 4);
      xv[q] = *reinterpret_cast<const u32x4_t*>(m.xf + static_cast<size_t>(b) * m.k + col);
      if (kslice + 4 * off >= m.k) xv[q] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
#pragma unroll
  for (int q = 0; q < LOADS; ++q) {
    const int ch = threadIdx.x + 256 * q;
    if (ch < 8 * CH16) {
      const int band = ch / CH16, off = ch % CH16;
      *reinterpret_cast<u32x4_t*>(tl + band * BSTRIDE + off * 4) = v[q];
    }
  }
  if constexpr (XB == 1) {
    if (wave < NCHK) {
      const int e0 = wave * 128 + lane;
      float lo = e0 < kvalid ? act_value(fw[0], kslice + e0, g.x_f16) * fs[0] : 0.0f;
      float hi = e0 + 64 < kvalid ? act_value(fw[1], kslice + e0 + 64, g.x_f16) * fs[1] : 0.0f;
      fwht_chunk(lo, hi, m.block_in, lane);
      const float nrm = 1.0f / sqrtf(static_cast<float>(m.block_in));
      if (e0 < XW) xs[e0] = dup_half(lo * nrm);
      if (e0 + 64 < XW) xs[e0 + 64] = dup_half(hi * nrm);
    }
  } else {
#pragma unroll
    for (int q = 0; q < XLOADS; ++q) {
      const int ch = threadIdx.x + 256 * q;
      if (ch < g.batch * XW / 4) *reinterpret_cast<u32x4_t*>(xs + 4 * ch) = xv[q];
    }
  }
  __syncthreads();

  // ---- decode + MFMA: wave w owns bands 2w, 2w+1; B = (x,x) pairs of columns 4g..4g+3,
  // batch row n = lane%16 (rows past the batch repeat the last one and are ignored)
  const int r = lane & 15, gq = lane >> 4;
  const int n = min(r, g.batch - 1);
  const QuadPos qp = quad_pos<K>(r, gq);
  float4_t acc[2] = {float4_t{0.f, 0.f, 0.f, 0.f}, float4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    const half8_t B = __builtin_bit_cast(half8_t,
        *reinterpret_cast<const u32x4_t*>(xs + n * XW + j * 16 + 4 * gq));
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const uint32_t* tp = tl + (2 * wave + bb) * BSTRIDE + j * NWK;
      const half8_t A = decode_a<K, CB>(tp[qp.wa], tp[qp.wb], qp.sh);
      acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc[bb], 0, 0, 0);
    }
  }
  // C[row 4g+i][col n] of each band -> tt[n][row]
  if (r < g.batch) {
#pragma unroll
    for (int bb = 0; bb < 2; ++bb)
#pragma unroll
      for (int i = 0; i < 4; ++i) tt[r * 128 + (2 * wave + bb) * 16 + 4 * gq + i] = acc[bb][i];
  }
  __syncthreads();

  const int E = g.batch * 128;
  if (m.S == 1) {
    tmk_out_fold(g, m, tt, ob, CB == CB_1MAD);
    return;
  }
  // ---- split-K: publish, ticket, the last block folds
  float* mypart = m.part + (static_cast<size_t>(ob) * m.S + sl) * E;
  for (int i = threadIdx.x; i < E; i += 256)
    __hip_atomic_store(mypart + i, tt[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(m.tickets + ob, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == static_cast<unsigned>(m.S - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (!last_flag) return;
  // sum the S partials of every element in slice order: for batch 1 two threads split
  // each element's slices; every thread keeps up to 16 loads in flight per round, and
  // the halves are combined in a fixed order (deterministic)
  const float* obpart = m.part + static_cast<size_t>(ob) * m.S * E;
  const int split = E < 256 ? 2 : 1;
  for (int i0 = 0; i0 < E; i0 += 256 / split) {
    const int i = i0 + threadIdx.x / split;
    const int h = threadIdx.x % split;
    float s = 0.0f;
    if (i < E) {
      for (int s0 = h; s0 < m.S; s0 += 16 * split) {
        float q[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int sidx = s0 + u * split;
          q[u] = sidx < m.S ? __hip_atomic_load(obpart + static_cast<size_t>(sidx) * E + i,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) s += q[u];
      }
    }
    if (split == 2) {
      if (i < E) red[h * 128 + i] = s;
    } else if (i < E) {
      tt[i] = s;
    }
  }
  __syncthreads();
  if (split == 2 && threadIdx.x < 128) tt[threadIdx.x] = red[threadIdx.x] + red[128 + threadIdx.x];
  if (threadIdx.x == 0)
    __hip_atomic_store(m.tickets + ob, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  tmk_out_fold(g, m, tt, ob, CB == CB_1MAD);
}

}  // namespace trellis
