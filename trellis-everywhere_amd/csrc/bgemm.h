// bgemm.h — batched packed linear for gfx950 (batch 2 .. prefill): decode once, reuse
// across the batch.
//
// A workgroup of 16 waves (12 for the exact mode's 128-column blocks) owns one 128-row
// output block (the out-dim Hadamard block) x NB = 16*NC batch columns x one k-range of
// `kr` tile columns, walked in steps of KT tiles (16 at 16 columns, 8 up to 64 and in the
// fp16-weight mode, 6 for the exact mode's 128 columns). Wave w = (band group
// bg = w % NG, k-lane kl = w / NG), a band group being BW = 2 or 4 adjacent bands
// (NG = 8 / BW groups, KL = waves / NG k-lanes): the waves of a SIMD share a band group and
// split every step's tiles between them (tile j of a step belongs to k-lane j % KL), so a
// SIMD has four (or three) waves to switch between:
//   * the B tile of a step (xf[batch cols][KT*16] as (x, x) fp16 pairs written by
//     xfold_kernel) is loaded two steps ahead into registers by all the threads, stored
//     to one half of a double-buffered LDS area, and read by every wave: each fragment
//     serves the BW bands of each of the NG band groups; one barrier per step;
//   * each wave's packed words ride a two-step register ring and a wave-private LDS
//     buffer (for the lanes' window reads), as in gemv_kernel;
//   * each wave decodes a tile of each of its bands once, straight into the A operand of
//     v_mfma_f32_16x16x32_f16 (the exact (hi, lo) pair against the duplicated activation,
//     common.h), and issues NC MFMAs per band against the NC batch chunks;
//   * every load is a range-checked buffer load (batch rows past the call's, tiles past the
//     matrix read zeros), so none is clamped or skipped and the waits stay exact;
//   * the B rows are padded by 8 words (a row stride of 8 mod 64 words): the 16 batch
//     rows x 4 column groups of a fragment read then run at the LDS's full rate on gfx950
//     (measured 177 B/clk per CU, against 115 with a 4-word pad, whose rows collide);
//   * the epilogue adds the KL k-lanes' sums into t[NB][128] in LDS in k-lane order
//     (deterministic); with one k-range the workgroup applies y = sv * osc * Hb_n(t)
//     itself, otherwise it stores its partial block and bfold_kernel (next launch) adds
//     the slices in slice order and folds, one wave per batch column: reducing inside the
//     kernel leaves the whole reduction to the last workgroup of each block, behind
//     device-scope round trips, and measured slower.
#pragma once

#include "common.h"

namespace trellis {

// y[b0 + b] = sv * osc * Hb_n(t[b]) for the nbv <= NB batch columns staged in LDS as
// t[b][TLS] (rows padded to TLS), summed over NR regions NR_OFF floats apart. Wave w folds
// columns w, w + WAVES, ..: all of them at once, level by level (fwht_chunks), so their
// lane exchanges overlap (one column after another, the fold of 64 columns measured ~2 us
// at the end of every batched launch); a wave's slots past nbv repeat column nbv - 1 and
// are not stored. so[h] = sv * osc of row 128 ob + min(lane + 64 h, rows - 1), loaded by
// the caller long before (cold, their load took ~1 us when the fold issued it).
template <int CB, int WAVES, int TLS, int NR, int NR_OFF, int NB>
__device__ __forceinline__ void bg_out_fold(const LinArgs& g, const LinMat& m, const float* tl,
                                            int ob, int b0, int nbv, int rows,
                                            const float (&sov)[2]) {
  constexpr int C = (NB + WAVES - 1) / WAVES;   // columns per wave
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave >= nbv) return;
  const float nrm = m.nrm_out;
  const float so[2] = {sov[0] * nrm, sov[1] * nrm};
  const FwhtLane fl = fwht_lane(lane, m.block_out);
  float lo[C], hi[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int b = min(wave + WAVES * c, nbv - 1);
    lo[c] = tl[b * TLS + lane];
    hi[c] = tl[b * TLS + lane + 64];
#pragma unroll
    for (int q = 1; q < NR; ++q) {
      lo[c] += tl[q * NR_OFF + b * TLS + lane];
      hi[c] += tl[q * NR_OFF + b * TLS + lane + 64];
    }
    if (lane >= rows) lo[c] = 0.f;
    if (lane + 64 >= rows) hi[c] = 0.f;
    if (CB == CB_1MAD) {
      lo[c] = lo[c] / 147.800537109375f;
      hi[c] = hi[c] / 147.800537109375f;
    }
  }
  fwht_chunks<C>(lo, hi, m.block_out, lane, fl);
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int b = wave + WAVES * c;
    if (b >= nbv) break;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rl = lane + 64 * h;
      if (rl < rows) {
        const float v = (h ? hi[c] : lo[c]) * so[h];
        const long long o = static_cast<long long>(b0 + b) * m.ldy + ob * 128 + rl;
        if (g.y_f16)
          st_wt(static_cast<_Float16*>(m.y) + o, static_cast<_Float16>(v));
        else
          st_wt(static_cast<float*>(m.y) + o, v);
      }
    }
  }
}

// k-step: 16 tile columns for 16 batch columns (half the barriers; the 8B gate+up group at
// batch 16: 29.1 -> 27.9 us), 8 for up to 64, 6 for 128 (two per k-lane over three
// k-lanes; LDS holds two B steps; a k-range's last step may be partial); always 8 in the
// fp16-weight mode, whose B words are half as many per column
template <int NC, int F16> struct BgStep {
  static constexpr int KT = F16 ? 8 : NC == 1 ? 16 : NC <= 4 ? 8 : 6;
};
// waves per workgroup: 16 (four per SIMD), or 12 (three per SIMD, up to 168 registers each)
// for the exact mode's 128-column blocks, whose 8 fragments and 16 accumulators per wave
// (~150 registers) do not fit a quarter of a SIMD's registers (against 8 waves, two per
// SIMD: the 8B block at a 512 prefill 463.4 -> 452.2 us, gate+up at 128 rows 69.4 -> 64.9)
template <int NC, int F16> struct BgWaves {
  static constexpr int WV = (!F16 && NC == 8) ? 12 : 16;
};
// bands per wave: 4 at 16 batch columns (8 k-lanes: each B fragment read from LDS feeds 4
// bands instead of 2; the 8B gate+up group at batch 16 27.8 -> 26.6-27.1 us), otherwise 2
// (a band pair, 4 k-lanes: at 32 and 64 columns 4 bands measured no faster on gate+up and
// 4-6 % slower on the split-K launches, whose epilogue adds twice the k-lanes); the k-step
// must hold a tile column per k-lane
template <int NC, int F16> struct BgBands {
  static constexpr int BW = (!F16 && NC == 1) ? 4 : 2;
};
// LDS regions of the epilogue's t[NB][TLS] partial sums, one per k-lane added in the same
// round (the k-lanes' sums meet in KL / NR rounds): as many as the LDS holds beside the
// waves' packed-word buffers, up to one per k-lane. From 64 batch columns (one workgroup per
// CU whatever its LDS) the whole LDS; below that half of it, so a kernel with few registers
// keeps room for two workgroups per CU (the 8B gate+up group at batch 16, four regions
// instead of two: 26.1 -> 25.9 us, 29.2 -> 28.7 in the fp16-weight mode).
constexpr int BG_LDS_WORDS = 160 * 1024 / 4;
template <int NC> __host__ __device__ constexpr int bg_regions(int nb, int kl, int tls, int xbuf,
                                                              int other) {
  // below 64 columns the LDS stays within half a CU's, for two workgroups per CU
  const int limit = NC < 4 ? BG_LDS_WORDS / 2 : BG_LDS_WORDS;
  const int base = 2 * xbuf;
  int r = kl;
  while (r > 1 && (r * nb * tls > base ? r * nb * tls : base) + other > limit) r /= 2;
  return r;
}

// s_setprio with a value known after unrolling (the instruction takes an immediate)
__device__ __forceinline__ void setprio_n(int v) {
  if (v >= 3) __builtin_amdgcn_s_setprio(3);
  else if (v == 2) __builtin_amdgcn_s_setprio(2);
  else if (v == 1) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

template <int K, int CB, int V, int NC, int F16, bool SINGLE>
__global__ __launch_bounds__((64 * BgWaves<NC, F16>::WV)) void bgemm_kernel(LinArgs g) {
  constexpr int BG_WAVES = BgWaves<NC, F16>::WV;
  constexpr int NWK = 8 * K;
  constexpr int KT = BgStep<NC, F16>::KT;          // tile columns per k-step
  constexpr int BW = BgBands<NC, F16>::BW;         // bands per wave
  constexpr int NG = 8 / BW;                       // band groups of the block
  constexpr int KL = BG_WAVES / NG;                // k-lanes: waves of one band group
  // tiles per band per k-lane per step: exact mode, tiles kl, kl + KL, ...; fp16-weight
  // mode, the tile pair 2kl, 2kl + 1 (one MFMA per pair)
  constexpr int TPL = F16 ? 2 : KT / KL;
  static_assert(F16 || (KT % KL == 0 && TPL >= 1), "a tile column per k-lane per step");
  constexpr int WPT = F16 ? 8 : 16;                // B words per tile column and batch row
  constexpr int XW = KT * WPT + 8;                 // LDS words per B row (+8: bank spread)
  constexpr int NB = 16 * NC;                      // batch columns per workgroup
  constexpr int RCH = KT * WPT / 4;                // 16-byte chunks per B row per step
  constexpr int XCH = NB * RCH;                    // 16-byte B chunks per step
  constexpr int XLOADS = (XCH + 64 * BG_WAVES - 1) / (64 * BG_WAVES);
  constexpr int XBUF = NB * XW;                    // words per B buffer
  constexpr int CPT = NWK / 4;                     // 16-byte chunks per tile
  constexpr int BCH = BW * TPL * CPT;              // 16-byte chunks per wave per step
  constexpr int BLOADS = (BCH + 63) / 64;
  constexpr int BSW = BLOADS * 256;                // words per wave buffer: every lane's chunks
  static_assert(!F16 || (KT == 2 * KL && BW == 2), "fp16-weight mode: one tile pair per k-lane per step");
  // epilogue: t[NB][TLS] (rows padded like the B rows, so a fragment's float4 writes
  // spread over the banks) in NR regions NR_OFF floats apart over the B buffers (bg_regions:
  // k-lanes k2 .. k2 + NR - 1 add into regions 0 .. NR - 1 in round k2 / NR)
  constexpr int TLS = 136;
  constexpr int NR = bg_regions<NC>(NB, KL, TLS, XBUF, BG_WAVES * BSW);
  constexpr int NR_OFF = NB * TLS;
  constexpr int XSB = 2 * XBUF > NR * NR_OFF ? 2 * XBUF : NR * NR_OFF;
  static_assert(KL % NR == 0 && NB * TLS <= XSB, "epilogue regions");
  __shared__ __align__(16) uint32_t xsb[XSB];
  __shared__ __align__(16) uint32_t bst[BG_WAVES * BSW];
  float* tl = reinterpret_cast<float*>(xsb);

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int bg = wave % NG, kl = wave / NG;
  // a one-matrix launch (SINGLE) reads its matrix's fields in the first argument round
  const int mi = SINGLE ? 0 : locate_mat(g, blockIdx.x, false);
  const LinMat& m = g.m[mi];
  {
    // the matrix's fields that the set-up needs, loaded in one round (the argument segment
    // is cold; used one by one, the loads would go out in several dependent rounds)
    const int f_i0 = m.item0, f_s = m.S, f_t = m.tiles_in, f_n = m.n, f_xw = m.xfw;
    const int f_bt = g.batch, f_kr = g.kr;
    const uint32_t *f_b = m.bits, *f_xf = m.xf;
    const float *f_sv = m.sv, *f_os = m.osc;
    asm volatile("" ::"s"(f_i0), "s"(f_s), "s"(f_t), "s"(f_n), "s"(f_xw), "s"(f_bt), "s"(f_kr),
                 "s"(f_b), "s"(f_xf), "s"(f_sv), "s"(f_os));
  }
  const int local = blockIdx.x - m.item0;
  const int ncb = (g.batch + NB - 1) / NB;
  const int sl = local % m.S, obcb = local / m.S;
  const int ob = obcb / ncb, cb = obcb % ncb;
  const int b0 = cb * NB;                          // first batch row of this column block
  const int nbv = min(NB, g.batch - b0);           // valid batch columns
  const int c0 = sl * g.kr;
  const int ntl = min(g.kr, m.tiles_in - c0);
  const int nsteps = (ntl + KT - 1) / KT;
  const int rows = min(128, m.n - ob * 128);
  uint32_t* mystg = bst + wave * BSW;

  // B: rows b0 .. b0 + nbv - 1 of xf (a batch row past the call's reads zeros; columns
  // past the k-range feed only tiles that are not decoded)
  const rsrc_t r_x = make_rsrc(m.xf + static_cast<size_t>(b0) * m.xfw,
                               static_cast<unsigned>(nbv) * m.xfw * 4);
  unsigned xoff[XLOADS];
#pragma unroll
  for (int q = 0; q < XLOADS; ++q) {
    const int ch = threadIdx.x + 64 * BG_WAVES * q;
    const int n = ch / RCH, off = ch % RCH;        // batch row, 16-byte chunk of its row
    xoff[q] = ch < XCH ? static_cast<unsigned>((n * m.xfw + c0 * WPT + off * 4) * 4) : RSRC_OOB;
  }
  // packed words of the block's bands (bands past the matrix read zeros; the range stays
  // far below 4 GB whatever the matrix); lane chunk -> (band of the pair, tile of the
  // k-lane, chunk)
  const size_t blk0 = static_cast<size_t>(ob) * 8 * m.tiles_in * NWK;
  const int nbands = min(8, m.n / 16 - ob * 8);    // bands of this block in the matrix
  const rsrc_t r_b = make_rsrc(m.bits + blk0, static_cast<unsigned>(nbands * m.tiles_in * NWK * 4));
  unsigned boff[BLOADS];
#pragma unroll
  for (int q = 0; q < BLOADS; ++q) {
    const int ch = lane + 64 * q;
    const int bb = ch / (TPL * CPT), rem = ch % (TPL * CPT);
    const int t = rem / CPT, c = rem % CPT;
    const int tile = c0 + (F16 ? 2 * kl + t : kl + KL * t);
    boff[q] = ch < BCH ? static_cast<unsigned>(((BW * bg + bb) * m.tiles_in + tile) * NWK * 4 + c * 16)
                       : RSRC_OOB;
  }
  u32x4_t xr[2][XLOADS], br[2][BLOADS];
  auto load_step = [&](int s, u32x4_t (&xd)[XLOADS], u32x4_t (&bd)[BLOADS]) {
    // a step past the last reads nothing
    const unsigned sx = s < nsteps ? static_cast<unsigned>(s * KT * WPT * 4) : RSRC_OOB;
    const unsigned sb = s < nsteps ? static_cast<unsigned>(s * KT * NWK * 4) : RSRC_OOB;
#pragma unroll
    for (int q = 0; q < XLOADS; ++q)
      xd[q] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              r_x, static_cast<int>(xoff[q] + sx), 0, 0));
#pragma unroll
    for (int q = 0; q < BLOADS; ++q)
      bd[q] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              r_b, static_cast<int>(boff[q] + sb), 0, AUX_NT));
  };
  auto store_b = [&](int buf, const u32x4_t (&xd)[XLOADS]) {
#pragma unroll
    for (int q = 0; q < XLOADS; ++q) {
      const int ch = threadIdx.x + 64 * BG_WAVES * q;
      if (XCH % (64 * BG_WAVES) == 0 || ch < XCH)
        *reinterpret_cast<u32x4_t*>(xsb + buf * XBUF + (ch / RCH) * XW + (ch % RCH) * 4) = xd[q];
    }
  };

  // one k-range: the output fold's scales, loaded now so their latency hides behind the loop
  float sov[2] = {0.f, 0.f};
  if (m.S == 1) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = ob * 128 + min(lane + 64 * h, rows - 1);
      sov[h] = m.sv[row] * m.osc[row];
    }
  }

  const int r = lane & 15, gq = lane >> 4;
  const QuadPos qp = quad_pos_v<K, V>(r, gq);
  float4_t acc[BW][NC];
#pragma unroll
  for (int b = 0; b < BW; ++b)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[b][c] = float4_t{0.f, 0.f, 0.f, 0.f};

  load_step(0, xr[0], br[0]);
  load_step(1, xr[1], br[1]);
  store_b(0, xr[0]);
  __syncthreads();
  __builtin_amdgcn_s_setprio(3);
  // two steps per trip so the register rings keep a fixed shape; a step past the last
  // computes nothing, and its loads read nothing
  for (int s = 0; s < nsteps; s += 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int st = s + h;
      // this wave's packed words of step st to its LDS buffer; the B tile of step st + 1
      // (loaded a step ago) to the other buffer, whose step st - 1 every wave finished
      // before the last barrier: its stores drain while this step computes, instead of
      // all waves' stores queueing in front of the barrier; then refill the slots with
      // step st + 2 (the B part of this slot went to LDS a step earlier)
#pragma unroll
      for (int q = 0; q < BLOADS; ++q)
        *reinterpret_cast<u32x4_t*>(mystg + 4 * (lane + 64 * q)) = br[h][q];
      store_b(h ^ 1, xr[h ^ 1]);
      load_step(st + 2, xr[h], br[h]);
      if (st < nsteps) {
        const uint32_t* xb = xsb + h * XBUF + r * XW + 4 * gq;
        if constexpr (F16) {
          // the pair 2kl, 2kl + 1 of the step; past an odd last tile the second tile's
          // words decode to finite values that meet zero activations (xfold_kernel)
          if (st * KT + 2 * kl < ntl) {
            const uint32_t* p0 = mystg;                 // band 2bg: tiles 2kl, 2kl + 1
            const uint32_t* p1 = mystg + TPL * NWK;     // band 2bg + 1
            // the window words and the first two fragments are read before the decode, and
            // each later pair of fragments while the MFMAs of the pair before it run (read
            // just before its own MFMAs, each pair's LDS latency was exposed)
            const uint32_t w0a = p0[qp.wa], w0b = p0[qp.wb], w0c = p0[NWK + qp.wa], w0d = p0[NWK + qp.wb];
            const uint32_t w1a = p1[qp.wa], w1b = p1[qp.wb], w1c = p1[NWK + qp.wa], w1d = p1[NWK + qp.wb];
            constexpr int FP = NC < 2 ? NC : 2;         // fragments per group
            auto frag = [&](int c) {
              return __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4_t*>(xb + c * 16 * XW + kl * 16));
            };
            half8_t Bn[FP];
#pragma unroll
            for (int f = 0; f < FP; ++f) Bn[f] = frag(f);
            const half8_t A0 = decode_a_pair<K, CB, V>(w0a, w0b, w0c, w0d, qp.sh);
            const half8_t A1 = decode_a_pair<K, CB, V>(w1a, w1b, w1c, w1d, qp.sh);
#pragma unroll
            for (int c0 = 0; c0 < NC; c0 += FP) {
              half8_t Bc[FP];
#pragma unroll
              for (int f = 0; f < FP; ++f) Bc[f] = Bn[f];
              if (c0 + FP < NC) {
#pragma unroll
                for (int f = 0; f < FP; ++f) Bn[f] = frag(c0 + FP + f);
              }
#pragma unroll
              for (int f = 0; f < FP; ++f) {
                acc[0][c0 + f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A0, Bc[f], acc[0][c0 + f], 0, 0, 0);
                acc[1][c0 + f] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A1, Bc[f], acc[1][c0 + f], 0, 0, 0);
              }
              setprio_n(2 - 4 * (c0 + FP) / NC);
            }
          }
        } else {
#pragma unroll
          for (int t = 0; t < TPL; ++t) {
            const int j = kl + KL * t;               // tile of the step
            if (st * KT + j < ntl) {
              // every LDS read of the tile (window words, the NC B fragments) before the
              // decode, so the fragments' latency hides behind it (read just before each
              // MFMA pair, it was exposed)
              uint32_t wa[BW], wb[BW];
#pragma unroll
              for (int b = 0; b < BW; ++b) {
                const uint32_t* tb = mystg + (b * TPL + t) * NWK;   // band BW * bg + b
                wa[b] = tb[qp.wa];
                wb[b] = tb[qp.wb];
              }
              half8_t Bf[NC];
#pragma unroll
              for (int c = 0; c < NC; ++c)
                Bf[c] = __builtin_bit_cast(half8_t, *reinterpret_cast<const u32x4_t*>(xb + c * 16 * XW + j * 16));
              // no instruction crosses this point (the scheduler would otherwise sink each
              // fragment's read back in front of its MFMAs); with 8 chunks the fragments'
              // registers would spill
              if constexpr (NC <= 4) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
              for (int b = 0; b < BW; ++b) {
                const half8_t A = decode_a<K, CB, V>(wa[b], wb[b], qp.sh);
#pragma unroll
                for (int c = 0; c < NC; ++c)
                  acc[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bf[c], acc[b][c], 0, 0, 0);
                setprio_n(2 - (t * BW + b) * 4 / (TPL * BW));
              }
            }
          }
        }
      }
      // every wave is done with this step's buffer, and the next step's B is stored
      __syncthreads();
      __builtin_amdgcn_s_setprio(3);
    }
  }
  __builtin_amdgcn_s_setprio(0);
  // the rings' last loads (steps past the end) are not consumed: let them land
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- t[batch col][row] in LDS, k-lanes added in a fixed order: lane (n, gq) of band
  // b, chunk c holds rows 4gq .. 4gq + 3 (one float4)
  for (int k2 = 0; k2 < KL; k2 += NR) {
    if (kl >= k2 && kl < k2 + NR) {
      float* reg = tl + (kl - k2) * NR_OFF;
#pragma unroll
      for (int b = 0; b < BW; ++b)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          float4_t* p = reinterpret_cast<float4_t*>(&reg[(c * 16 + r) * TLS + 16 * (BW * bg + b) + 4 * gq]);
          *p = k2 == 0 ? acc[b][c] : *p + acc[b][c];
        }
    }
    __syncthreads();
  }

  if (m.S > 1) {
    // publish this slice's partial block (16-byte write-through stores); bfold_kernel adds
    // the slices and folds
    float* mypart = m.part + (static_cast<size_t>(ob * ncb + cb) * m.S + sl) * NB * 128;
    const float4_t* t4 = reinterpret_cast<const float4_t*>(tl);
    const rsrc_t r_p = make_rsrc(mypart, static_cast<unsigned>(nbv) * 512);
    for (int i = threadIdx.x; i < nbv * 32; i += 64 * BG_WAVES) {
      const int j = (i >> 5) * (TLS / 4) + (i & 31);
      float4_t v = t4[j];
#pragma unroll
      for (int q = 1; q < NR; ++q) v += t4[q * (NR_OFF / 4) + j];
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r_p, i * 16, 0, AUX_SC1);
    }
    return;
  }
  bg_out_fold<CB, BG_WAVES, TLS, NR, NR_OFF, NB>(g, m, tl, ob, b0, nbv, rows, sov);
}

// Split-K reduction of bgemm_kernel: one wave per (matrix, 128-row block, batch column):
// it loads that column's 128 rows of every slice at once (S slices x 2 values per lane in
// flight), adds them in slice order (deterministic), and folds y = sv * osc * Hb_n(t).
// Workgroup = 4 batch columns of one (matrix, block, column block). Runs after
// bgemm_kernel (a kernel boundary), so plain loads see its partial sums.
template <int CB, int NC, bool SINGLE>
__global__ __launch_bounds__(256) void bfold_kernel(LinArgs g) {
  constexpr int NB = 16 * NC, CG = NB / 4;        // workgroups per (block, column block)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int fi = blockIdx.x / CG, cg = blockIdx.x % CG;
  // a one-matrix launch reads its matrix's fields in the first round of argument loads
  const int mi = SINGLE ? 0 : locate_fold(g, fi);
  const LinMat& m = g.m[mi];
  const int ncb = (g.batch + NB - 1) / NB;
  const int local = fi - m.fold0;
  const int ob = local / ncb, cb = local % ncb;
  const int b0 = cb * NB, nbv = min(NB, g.batch - b0);
  const int n = cg * 4 + wave;                    // batch column of the block
  if (n >= nbv) return;
  const int rows = min(128, m.n - ob * 128);
  const int S = m.S;
  // the output scales first: their loads are in flight with the partial sums'
  float so[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = ob * 128 + min(lane + 64 * h, rows - 1);
    so[h] = m.sv[row] * m.osc[row];
  }
  const float* p = m.part + static_cast<size_t>(ob * ncb + cb) * S * NB * 128 + n * 128;
  float lo = 0.f, hi = 0.f;
  for (int s0 = 0; s0 < S; s0 += 8) {
    float q0[8], q1[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float* ps = p + static_cast<size_t>(min(s0 + v, S - 1)) * NB * 128;
      q0[v] = ps[lane];
      q1[v] = ps[lane + 64];
    }
#pragma unroll
    for (int v = 0; v < 8; ++v)
      if (s0 + v < S) {
        lo += q0[v];
        hi += q1[v];
      }
  }
  if (CB == CB_1MAD) {
    lo = lo / 147.800537109375f;
    hi = hi / 147.800537109375f;
  }
  fwht_chunk(lo, hi, m.block_out, lane);
  const float nrm = m.nrm_out;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int rl = lane + 64 * h;
    if (rl < rows) {
      const int row = ob * 128 + rl;
      const float v = (h ? hi : lo) * (so[h] * nrm);
      const long long o = static_cast<long long>(b0 + n) * m.ldy + row;
      if (g.y_f16)
        st_wt(static_cast<_Float16*>(m.y) + o, static_cast<_Float16>(v));
      else
        st_wt(static_cast<float*>(m.y) + o, v);
    }
  }
}

}  // namespace trellis
