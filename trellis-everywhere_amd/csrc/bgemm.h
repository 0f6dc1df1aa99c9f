// bgemm.h — batched packed linear for gfx950 (batch 2 .. prefill): decode once, reuse
// across the batch.
//
// A workgroup (4 waves) owns one 128-row output block (the out-dim Hadamard block; wave w
// owns bands 2w and 2w+1) x NB = 16*NC batch columns x one k-range of `kr` tile columns,
// walked in steps of KT tiles (8, or 4 at 128 columns):
//   * step s+1 is loaded into registers (the B tile: xf[batch cols][64] as (x, x) fp16
//     pairs written by xfold_kernel; the waves' packed words) while step s is computed,
//     then stored to the other half of a double-buffered LDS area; one barrier per step;
//   * each wave decodes a tile of each of its bands once, straight into the A operand of
//     v_mfma_f32_16x16x32_f16 (the exact (hi, lo) pair against the duplicated activation,
//     common.h), and issues NC MFMAs per band against the NC batch chunks, so the
//     decode is amortised over all NB columns and each B fragment read from LDS serves
//     both bands;
//   * the B rows are padded by 4 words so the 16 batch rows of a fragment fall in
//     different LDS banks;
//   * the epilogue stages t[NB][128] in LDS; with one k-range the workgroup applies
//     y = sv * osc * Hb_n(t) itself, otherwise it stores its partial block and
//     bfold_kernel (next launch) adds the slices in slice order (deterministic) and folds:
//     a cross-CU reduction inside the kernel would wait on device-scope round trips of
//     ~2 us each, with one workgroup's worth of loads in flight.
#pragma once

#include "common.h"

namespace trellis {

// y[b0 + b] = sv * osc * Hb_n(t[b]) for the nbv batch columns staged in LDS as
// t[b][128]; one column per wave at a time (256-thread workgroups).
template <int CB>
__device__ __forceinline__ void bg_out_fold(const LinArgs& g, const LinMat& m, const float* tl,
                                            int ob, int b0, int nbv, int rows) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float nrm = m.nrm_out;
  float so[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = ob * 128 + min(lane + 64 * h, rows - 1);
    so[h] = m.sv[row] * m.osc[row] * nrm;
  }
  for (int b = wave; b < nbv; b += 4) {
    float lo = lane < rows ? tl[b * 128 + lane] : 0.f;
    float hi = lane + 64 < rows ? tl[b * 128 + lane + 64] : 0.f;
    if (CB == CB_1MAD) {
      lo = lo / 147.800537109375f;
      hi = hi / 147.800537109375f;
    }
    fwht_chunk(lo, hi, m.block_out, lane);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rl = lane + 64 * h;
      if (rl < rows) {
        const float v = (h ? hi : lo) * so[h];
        const long long o = static_cast<long long>(b0 + b) * m.ldy + ob * 128 + rl;
        if (g.y_f16)
          static_cast<_Float16*>(m.y)[o] = static_cast<_Float16>(v);
        else
          static_cast<float*>(m.y)[o] = v;
      }
    }
  }
}

// k-step: 8 tile columns for up to 64 batch columns, 4 for 128 (LDS holds two B steps)
template <int NC> struct BgStep { static constexpr int KT = NC <= 4 ? 8 : 4; };

template <int K, int CB, int V, int NC>
__global__ __launch_bounds__(256) void bgemm_kernel(LinArgs g) {
  constexpr int NWK = 8 * K;
  constexpr int BG_KT = BgStep<NC>::KT;            // tile columns per k-step
  constexpr int BG_XW = BG_KT * 16 + 4;            // LDS words per B row (+4: bank spread)
  constexpr int NB = 16 * NC;                      // batch columns per workgroup
  constexpr int RCH = BG_KT * 4;                   // 16-byte chunks per B row per step
  constexpr int XCH = NB * RCH;                    // 16-byte B chunks per step
  constexpr int XLOADS = (XCH + 255) / 256;
  constexpr int BW = 2 * BG_KT * NWK;              // packed words per wave per step
  constexpr int BCH = BW / 4;                      // 16-byte chunks per wave per step
  constexpr int BLOADS = (BCH + 63) / 64;
  constexpr int XBUF = NB * BG_XW;                 // words per B buffer
  __shared__ __align__(16) uint32_t xsb[2 * XBUF];
  __shared__ __align__(16) uint32_t bst[2][4][BW];
  float* tl = reinterpret_cast<float*>(xsb);       // epilogue: t[NB][128] (fits in 2*XBUF)

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int mi = locate_mat(g, blockIdx.x, false);
  const LinMat& m = g.m[mi];
  const int local = blockIdx.x - m.item0;
  const int ncb = (g.batch + NB - 1) / NB;
  const int sl = local % m.S, obcb = local / m.S;
  const int ob = obcb / ncb, cb = obcb % ncb;
  const int b0 = cb * NB;                          // first batch row of this column block
  const int nbv = min(NB, g.batch - b0);           // valid batch columns
  const int c0 = sl * g.kr;
  const int ntl = min(g.kr, m.tiles_in - c0);
  const int nsteps = (ntl + BG_KT - 1) / BG_KT;
  const int rows = min(128, m.n - ob * 128);

  u32x4_t xr[XLOADS], br[BLOADS];
  auto load_step = [&](int s) {
#pragma unroll
    for (int q = 0; q < XLOADS; ++q) {
      const int ch = threadIdx.x + 256 * q;
      if (XCH % 256 == 0 || ch < XCH) {
        const int n = ch / RCH, off = ch % RCH;     // batch row, 16-byte chunk of its row
        const int col = (c0 + s * BG_KT) * 16 + off * 4;
        const bool ok = n < nbv && col < (c0 + ntl) * 16;
        const uint32_t* src = m.xf + static_cast<size_t>(b0 + min(n, nbv - 1)) * m.k +
                              min(col, m.k - 4);
        xr[q] = *reinterpret_cast<const u32x4_t*>(src);
        if (!ok) xr[q] = u32x4_t{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int q = 0; q < BLOADS; ++q) {
      const int ch = lane + 64 * q;
      if (BCH % 64 == 0 || ch < BCH) {
        const int bb = ch / (BCH / 2), rem = ch % (BCH / 2);
        const int band = ob * 8 + min(2 * wave + bb, rows / 16 - 1);
        const int tile = c0 + min(s * BG_KT + rem / (NWK / 4), ntl - 1);
        br[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(
            m.bits + (static_cast<size_t>(band) * m.tiles_in + tile) * NWK) + rem % (NWK / 4));
      }
    }
  };
  auto store_step = [&](int buf) {
#pragma unroll
    for (int q = 0; q < XLOADS; ++q) {
      const int ch = threadIdx.x + 256 * q;
      if (XCH % 256 == 0 || ch < XCH)
        *reinterpret_cast<u32x4_t*>(xsb + buf * XBUF + (ch / RCH) * BG_XW + (ch % RCH) * 4) = xr[q];
    }
#pragma unroll
    for (int q = 0; q < BLOADS; ++q) {
      const int ch = lane + 64 * q;
      if (BCH % 64 == 0 || ch < BCH) *reinterpret_cast<u32x4_t*>(&bst[buf][wave][4 * ch]) = br[q];
    }
  };

  const int r = lane & 15, gq = lane >> 4;
  const QuadPos qp = quad_pos_v<K, V>(r, gq);
  float4_t acc[2][NC];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[b][c] = float4_t{0.f, 0.f, 0.f, 0.f};

  load_step(0);
  store_step(0);
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int buf = s & 1;
    if (s + 1 < nsteps) load_step(s + 1);
    const uint32_t* xb = xsb + buf * XBUF + r * BG_XW + 4 * gq;
#pragma unroll
    for (int t = 0; t < BG_KT; ++t) {
      const uint32_t* t0 = &bst[buf][wave][t * NWK];
      const uint32_t* t1 = &bst[buf][wave][(BG_KT + t) * NWK];
      const half8_t A0 = decode_a<K, CB, V>(t0[qp.wa], t0[qp.wb], qp.sh);
      const half8_t A1 = decode_a<K, CB, V>(t1[qp.wa], t1[qp.wb], qp.sh);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const half8_t B = __builtin_bit_cast(
            half8_t, *reinterpret_cast<const u32x4_t*>(xb + c * 16 * BG_XW + t * 16));
        acc[0][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, B, acc[0][c], 0, 0, 0);
        acc[1][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, B, acc[1][c], 0, 0, 0);
      }
    }
    if (s + 1 < nsteps) store_step(buf ^ 1);
    __syncthreads();
  }

  // ---- t[batch col][row] in LDS: lane (n, gq) of band b, chunk c holds rows 4gq + i
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) tl[(c * 16 + r) * 128 + 32 * wave + 16 * b + 4 * gq + i] = acc[b][c][i];
  __syncthreads();

  if (m.S > 1) {
    // publish this slice's partial block; bfold_kernel adds the slices and folds
    float* mypart = m.part + (static_cast<size_t>(ob * ncb + cb) * m.S + sl) * NB * 128;
    for (int i = threadIdx.x; i < nbv * 32; i += 256)
      reinterpret_cast<float4_t*>(mypart)[i] = reinterpret_cast<const float4_t*>(tl)[i];
    return;
  }
  bg_out_fold<CB>(g, m, tl, ob, b0, nbv, rows);
}

// Split-K reduction of bgemm_kernel: one workgroup per (matrix, 128-row block, column
// block) adds the S partial blocks in slice order (deterministic), then folds. Runs after
// bgemm_kernel, so plain loads see its plain stores.
template <int CB, int NC>
__global__ __launch_bounds__(256) void bfold_kernel(LinArgs g) {
  constexpr int NB = 16 * NC;
  __shared__ __align__(16) float tl[NB * 128];
  const int mi = locate_fold(g, blockIdx.x);
  const LinMat& m = g.m[mi];
  const int ncb = (g.batch + NB - 1) / NB;
  const int local = blockIdx.x - m.fold0;
  const int ob = local / ncb, cb = local % ncb;
  const int b0 = cb * NB, nbv = min(NB, g.batch - b0);
  const int rows = min(128, m.n - ob * 128);
  const float4_t* part = reinterpret_cast<const float4_t*>(
      m.part + static_cast<size_t>(ob * ncb + cb) * m.S * NB * 128);
  const size_t stride = static_cast<size_t>(NB) * 32;       // float4s per slice
  for (int i0 = threadIdx.x; i0 < nbv * 32; i0 += 2 * 256) {
    float4_t a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
    const int i1 = min(i0 + 256, nbv * 32 - 1);
    for (int s0 = 0; s0 < m.S; s0 += 4) {
      float4_t q0[4], q1[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const size_t so = static_cast<size_t>(min(s0 + v, m.S - 1)) * stride;
        q0[v] = part[so + i0];
        q1[v] = part[so + i1];
      }
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (s0 + v < m.S) {
          a0 += q0[v];
          a1 += q1[v];
        }
    }
    reinterpret_cast<float4_t*>(tl)[i0] = a0;
    if (i0 + 256 < nbv * 32) reinterpret_cast<float4_t*>(tl)[i0 + 256] = a1;
  }
  __syncthreads();
  bg_out_fold<CB>(g, m, tl, ob, b0, nbv, rows);
}

}  // namespace trellis
