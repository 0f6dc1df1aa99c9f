// gemv.h — batch-1 packed linear for gfx950: a pipelined decode-GEMV.
//
// The decode goes straight into the A operand of v_mfma_f32_16x16x32_f16 (the codebook's
// fp16 pair (hi, lo) against a duplicated activation, fp32 accumulation: common.h),
// organised for batch 1, where the decode's VALU work and fixed per-launch latencies, not
// HBM, set the time:
//
//   * Work item = one matrix x one 128-row output block (8 bands of 16 rows) x one
//     k-range of `kr` tile columns, run by one 16-wave workgroup (one per CU): waves w and
//     w + 8 own band w, each for half of the k-range, so every wave of a CU starts together
//     and none runs alone at the end.
//   * Each wave streams its half-band in stages of KC tiles. GEMV_PF stages are in flight
//     in registers (coalesced 16-byte loads); the current stage is copied to a wave-private
//     LDS buffer and decoded from there, so no barrier is needed in the main loop.
//   * Tiles are decoded GEMV_G at a time into separate A registers before their MFMAs are
//     issued: a decode then never waits for an MFMA to release its operands.
//   * The activation fold xf = Hb_k(isc_scaled * su * x) of the k-range is computed once
//     per workgroup (its loads are issued before the packed words) and kept in LDS as
//     (x, x) fp16 pairs.
//   * The two k-halves are added in LDS. With one k-range (S == 1) wave 0 applies
//     y = sv * osc * Hb_n(t) directly; with split-K it publishes the block's partial sum,
//     takes a ticket, and the last workgroup of the block adds the partials in slice order
//     (deterministic) before the fold. sv * osc is loaded at kernel start.
#pragma once

#include "common.h"

namespace trellis {

constexpr int GEMV_WAVES = 16;    // two waves per 16-row band: 128 rows per workgroup
constexpr int GEMV_MAX_KR = 256;  // tile columns per k-range (4096 activations)
constexpr int GEMV_PF = 2;        // pipeline stages in flight per wave
constexpr int GEMV_G = 4;         // tiles decoded before their MFMAs are issued

template <int K, int CB, int V, int KC, int PF>
__global__ __launch_bounds__(64 * GEMV_WAVES) void gemv_kernel(LinArgs g) {
  constexpr int NWK = 8 * K;                 // words per tile
  constexpr int SW = KC * NWK;               // words per wave-stage
  constexpr int CH = SW / 4;                 // 16-byte chunks per wave-stage
  constexpr int LOADS = (CH + 63) / 64;      // chunks per lane
  constexpr int CPT = NWK / 4;               // chunks per tile
  constexpr int FCH = GEMV_MAX_KR * 16 / 128 / GEMV_WAVES;  // fold chunks per wave (max)
  __shared__ __align__(16) uint32_t stg[GEMV_WAVES * SW];
  __shared__ __align__(16) uint32_t xs[GEMV_MAX_KR * 16];
  __shared__ float tt[2][128];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int bl = wave & 7, half = wave >> 3;     // band of the block, half of the k-range
  const int mi = locate_mat(g, blockIdx.x, false);
  const LinMat& m = g.m[mi];
  const int local = blockIdx.x - m.item0;
  const int ob = local / m.S, sl = local % m.S;
  const int c0 = sl * g.kr;                          // first tile column of the k-range
  const int ntl = min(g.kr, m.tiles_in - c0);        // tile columns in the k-range
  const int nst = (ntl + KC - 1) / KC;
  const int s_mid = (nst + 1) / 2;
  const int s_begin = half ? s_mid : 0, s_end = half ? nst : s_mid;
  const int rows = min(128, m.n - ob * 128);
  const int band = ob * 8 + min(bl, rows / 16 - 1);
  const uint32_t* bsrc = m.bits + (static_cast<size_t>(band) * m.tiles_in + c0) * NWK;
  uint32_t* mystg = stg + wave * SW;

  // ---- output scales of this block for the fold (wave 0), activation loads of the
  // k-range fold (chunk w and w + GEMV_WAVES per wave), then the first packed words: the
  // fold and the epilogue never wait behind the packed-word stream
  float so[2] = {0.f, 0.f};
  if (wave == 0) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = ob * 128 + min(lane + 64 * h, rows - 1);
      so[h] = m.sv[row] * m.osc[row];
    }
  }
  const int kcols = ntl * 16;
  const int nch = (kcols + 127) / 128;
  uint32_t fw[FCH][2];
  float fsc[FCH][2];
#pragma unroll
  for (int f = 0; f < FCH; ++f) {
    const int ch = wave + GEMV_WAVES * f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = c0 * 16 + min(ch * 128 + lane + 64 * h, kcols - 1);
      if (ch < nch) {
        fw[f][h] = load_act_word(m.x, i, g.x_f16);
        fsc[f][h] = m.su[i] * m.isc[i];
      }
    }
  }
  u32x4_t R[PF][LOADS];
  auto load_stage = [&](int s, u32x4_t (&dst)[LOADS]) {
#pragma unroll
    for (int q = 0; q < LOADS; ++q) {
      const int ch = lane + 64 * q;
      if (CH % 64 == 0 || ch < CH) {
        const int t = min(s * KC + ch / CPT, ntl - 1);
        dst[q] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4_t*>(bsrc + static_cast<size_t>(t) * NWK) + ch % CPT);
      }
    }
  };
#pragma unroll
  for (int b = 0; b < PF; ++b)
    if (s_begin + b < s_end) load_stage(s_begin + b, R[b]);

  // ---- activation fold: xf = Hb_k(isc_scaled * su * x) / sqrt(block_in) as (x,x) pairs
  {
    const float nrm = 1.0f / sqrtf(static_cast<float>(m.block_in));
#pragma unroll
    for (int f = 0; f < FCH; ++f) {
      const int ch = wave + GEMV_WAVES * f;
      if (ch < nch) {
        const int e0 = ch * 128 + lane, e1 = e0 + 64;
        float lo = e0 < kcols ? act_value(fw[f][0], c0 * 16 + e0, g.x_f16) * fsc[f][0] : 0.0f;
        float hi = e1 < kcols ? act_value(fw[f][1], c0 * 16 + e1, g.x_f16) * fsc[f][1] : 0.0f;
        fwht_chunk(lo, hi, m.block_in, lane);
        xs[e0] = dup_half(lo * nrm);
        xs[e1] = dup_half(hi * nrm);
      }
    }
  }
  __syncthreads();

  // ---- main loop: stage s is moved from registers to the wave's LDS buffer, the load
  // of stage s + PF is issued into the freed registers, then stage s is decoded
  const int r = lane & 15, gq = lane >> 4;
  const QuadPos qp = quad_pos_v<K, V>(r, gq);
  float4_t acc = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  half8_t Bv[GEMV_G];
  auto stage = [&](int s, u32x4_t (&src)[LOADS]) {
#pragma unroll
    for (int q = 0; q < LOADS; ++q) {
      const int ch = lane + 64 * q;
      if (CH % 64 == 0 || ch < CH) *reinterpret_cast<u32x4_t*>(mystg + 4 * ch) = src[q];
    }
    if (s + PF < s_end) load_stage(s + PF, src);
    const uint32_t* xst = xs + s * KC * 16 + 4 * gq;
    // G tiles at a time: their LDS reads, then their decodes into separate A registers,
    // then their MFMAs on alternating accumulators, so a decode never waits for the
    // previous MFMA to release its operand registers
    auto group = [&](int j0) {
      uint32_t wlo[GEMV_G], whi[GEMV_G];
      half8_t A[GEMV_G];
#pragma unroll
      for (int j = 0; j < GEMV_G; ++j) {
        const uint32_t* tp = mystg + (j0 + j) * NWK;
        wlo[j] = tp[qp.wa];
        whi[j] = tp[qp.wb];
      }
#pragma unroll
      for (int j = 0; j < GEMV_G; ++j)
        Bv[j] = __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4_t*>(xst + (j0 + j) * 16));
#pragma unroll
      for (int j = 0; j < GEMV_G; ++j) A[j] = decode_a<K, CB, V>(wlo[j], whi[j], qp.sh);
#pragma unroll
      for (int j = 0; j < GEMV_G; ++j) {
        if (j & 1)
          acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[j], Bv[j], acc1, 0, 0, 0);
        else
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[j], Bv[j], acc, 0, 0, 0);
      }
    };
    const int jn = ntl - s * KC;
    if (jn >= KC) {
#pragma unroll
      for (int j0 = 0; j0 < KC; j0 += GEMV_G) group(j0);
    } else {
      for (int j = 0; j < jn; ++j) {
        const half8_t B = __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4_t*>(xst + j * 16));
        const uint32_t* tp = mystg + j * NWK;
        const half8_t A = decode_a<K, CB, V>(tp[qp.wa], tp[qp.wb], qp.sh);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, acc, 0, 0, 0);
      }
    }
  };
  for (int s = s_begin; s < s_end; s += PF) {
#pragma unroll
    for (int b = 0; b < PF; ++b) {
      if (s + b < s_end) {
        stage(s + b, R[b]);
      }
    }
  }
  acc += acc1;
  // column 0 of C: lanes 0, 16, 32, 48 hold rows 4*gq + i of the band
  if (r == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) tt[half][bl * 16 + 4 * gq + i] = acc[i];
  }
  __syncthreads();
  if (wave != 0) return;

  // ---- wave 0: the two k-halves, then (split-K) publish, ticket, and in the last
  // workgroup of the block the partials in slice order; then y = sv * osc * Hb_n(t)
  float t0 = tt[0][lane] + tt[1][lane], t1 = tt[0][lane + 64] + tt[1][lane + 64];
  if (m.S > 1) {
    float* mypart = m.part + (static_cast<size_t>(ob) * m.S + sl) * 128;
    __hip_atomic_store(mypart + lane, t0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(mypart + lane + 64, t1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    unsigned prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(m.tickets + ob, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __builtin_amdgcn_readfirstlane(prev);
    if (prev != static_cast<unsigned>(m.S - 1)) return;
    const float* obpart = m.part + static_cast<size_t>(ob) * m.S * 128;
    t0 = 0.f;
    t1 = 0.f;
    for (int s0 = 0; s0 < m.S; s0 += 8) {
      float q0[8], q1[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float* p = obpart + static_cast<size_t>(min(s0 + u, m.S - 1)) * 128;
        q0[u] = __hip_atomic_load(p + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        q1[u] = __hip_atomic_load(p + lane + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (s0 + u < m.S) {
          t0 += q0[u];
          t1 += q1[u];
        }
      }
    }
    if (lane == 0) __hip_atomic_store(m.tickets + ob, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (CB == CB_1MAD) {
    t0 = t0 / 147.800537109375f;
    t1 = t1 / 147.800537109375f;
  }
  fwht_chunk(t0, t1, m.block_out, lane);
  const float nrm = 1.0f / sqrtf(static_cast<float>(m.block_out));
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rl = lane + 64 * h;
    if (rl < rows) {
      const float v = (h ? t1 : t0) * nrm * so[h];
      const long long o = ob * 128 + rl;
      if (g.y_f16)
        static_cast<_Float16*>(m.y)[o] = static_cast<_Float16>(v);
      else
        static_cast<float*>(m.y)[o] = v;
    }
  }
}

}  // namespace trellis
