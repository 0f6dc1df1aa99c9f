// embed.h — embedding-row lookup from a packed trellis matrix with the full restore:
// out[t, j] = W_hat[tok[t], j] (web/kernels.js:192-249 DECODE_EMBED, web/packed.js:137-146).
//
// W_hat[r, j] = sv[r] osc[r] su[j] isc_scaled[j] / sqrt(B_n B_k)
//               * sum_l H_k[j % B_k, l] * sum_c H_n[r % B_n, c] * zq[rb + c, jb + l]
// (rb, jb: first row / column of r's and j's Hadamard blocks; H entries (-1)^popcount(a&b)).
// The two Hadamard sums commute, so every weight of the B_n x B_k block is decoded once
// per (token, column block): one workgroup per (token, column block), 4 waves.
//   * wave w takes the bands b = w, w + 4 of the row block; it loads their tiles' packed
//     words as 16-byte chunks into a wave-private LDS buffer (one chunk per lane and load;
//     each lane loading its window words straight from global memory, two 4-byte gathers
//     per tile, measured slower in the batched kernel), then lane (row rl = l%16, column
//     group g = l/16) decodes 4 weights of each tile (the same window/codebook code as the
//     matmul kernels) and accumulates sign(rr, 16b + rl) * w per column, so a lane holds 4
//     columns of each of the block's tile columns. MCG/3INST: one
//     v_dot2_f32_f16 of the raw (hi, lo) fp16 pair with (sign, sign) per weight (the
//     products are exact; hi + lo is the reference's exact fp32 sum); 1MAD: the integer
//     (y - 510) * sign, exact in fp32, divided by 147.800537109375 once per output;
//   * the 16 rows of a lane group are summed by DPP butterflies (all-reduce within a
//     16-lane row), the 4 waves' column sums are added in LDS in wave order;
//   * wave 0 applies the column-side Hadamard (fwht_chunk) and the scales.
// A token id outside [0, n_out) yields a row of zeros.
#pragma once

#include "common.h"

namespace trellis {

struct EmbedArgs {
  const uint32_t* bits;
  const float* su;
  const float* sv;
  const float* isc;     // isc_scaled = f32(isc) * scale
  const float* osc;
  const int32_t* tokens;
  void* out;
  long long ldo;
  int n, k, tiles_in, block_in, block_out, nblk;   // nblk = k / block_in
  float nrm;            // 1/sqrt(block_in) * 1/sqrt(block_out), fp32
  int out_f16;
};

template <int K, int CB, int V>
__global__ __launch_bounds__(256) void embed_kernel(EmbedArgs a) {
  constexpr int NWK = 8 * K;
  constexpr int WBUF = 2 * 8 * NWK;                 // words of two bands x 8 tiles
  __shared__ float colsum[4][128];
  __shared__ __align__(16) uint32_t wbuf[4][WBUF];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int t = blockIdx.x / a.nblk, jblk = blockIdx.x % a.nblk;
  const int jb = jblk * a.block_in;                 // first column of the block
  const int tok = a.tokens[t];
  const bool ok = tok >= 0 && tok < a.n;
  const int r = ok ? tok : 0;
  const int rb = r - r % a.block_out, rr = r % a.block_out;
  const int ntc = a.block_in / 16, nbands = a.block_out / 16;
  const int rl = lane & 15, g = lane >> 4;
  const QuadPos qp = quad_pos_v<K, V>(rl, g);

  // this wave's bands' tiles of the column block to LDS: band slot s (band wave + 4s)
  // holds words [s * ntc * NWK, (s + 1) * ntc * NWK); a band past the block reads zeros
  uint32_t* mybuf = wbuf[wave];
  {
    const int cpb = ntc * NWK / 4;                  // 16-byte chunks per band
    const rsrc_t r_bits = make_rsrc(a.bits + static_cast<size_t>(rb / 16) * a.tiles_in * NWK,
                                    static_cast<unsigned>(nbands * a.tiles_in * NWK * 4));
#pragma unroll
    for (int q = 0; q < (WBUF / 4 + 63) / 64; ++q) {
      const int ch = lane + 64 * q;
      const int sb = ch / cpb, c = ch % cpb;
      const int band = wave + 4 * sb;
      const unsigned off = ch < 2 * cpb && band < nbands
                               ? static_cast<unsigned>(((band * a.tiles_in + jb / 16) * NWK + 4 * c) * 4)
                               : RSRC_OOB;
      const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                        r_bits, static_cast<int>(off), 0, AUX_NT));
      if (ch < 2 * cpb) *reinterpret_cast<u32x4_t*>(mybuf + 4 * ch) = v;
    }
  }

  float acc[8][4];
#pragma unroll
  for (int tc = 0; tc < 8; ++tc)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[tc][q] = 0.f;
  for (int b = wave; b < nbands; b += 4) {
    const int c = 16 * b + rl;                       // row within the row block
    const float sgn = (__builtin_popcount(rr & c) & 1) ? -1.f : 1.f;
    const half2_t s2 = {static_cast<_Float16>(sgn), static_cast<_Float16>(sgn)};
    const uint32_t* band = mybuf + ((b - wave) / 4) * ntc * NWK;
#pragma unroll
    for (int tc = 0; tc < 8; ++tc) {
      if (tc < ntc) {
        const uint32_t* tp = band + tc * NWK;
        uint32_t raw[4];
        decode_quad<K, CB, V>(tp[qp.wa], tp[qp.wb], qp.sh, raw);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (CB == CB_1MAD)
            acc[tc][q] += sgn * static_cast<float>(static_cast<int>(raw[q]) - 510);
          else
            acc[tc][q] = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, raw[q]), s2,
                                                acc[tc][q], false);
        }
      }
    }
  }
  // sum over the 16 rows of each lane group (a 16-lane DPP row)
#pragma unroll
  for (int tc = 0; tc < 8; ++tc)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float v = acc[tc][q];
      v += lane_xor<1>(v, lane);
      v += lane_xor<2>(v, lane);
      v += lane_xor<4>(v, lane);
      v += lane_xor<8>(v, lane);
      acc[tc][q] = v;
    }
  if (rl == 0) {
#pragma unroll
    for (int tc = 0; tc < 8; ++tc)
      if (tc < ntc)
#pragma unroll
        for (int q = 0; q < 4; ++q) colsum[wave][16 * tc + 4 * g + q] = acc[tc][q];
  }
  __syncthreads();
  if (wave != 0) return;
  float lo = 0.f, hi = 0.f;
  const int nw = nbands < 4 ? nbands : 4;
  for (int w = 0; w < nw; ++w) {
    if (lane < a.block_in) lo += colsum[w][lane];
    if (lane + 64 < a.block_in) hi += colsum[w][lane + 64];
  }
  if (CB == CB_1MAD) {
    lo = lo / 147.800537109375f;
    hi = hi / 147.800537109375f;
  }
  fwht_chunk(lo, hi, a.block_in, lane);
  const float rs = ok ? a.sv[r] * a.osc[r] * a.nrm : 0.f;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int jl = lane + 64 * h;
    if (jl < a.block_in) {
      const int j = jb + jl;
      const float v = (h ? hi : lo) * rs * a.isc[j] * a.su[j];
      const long long o = static_cast<long long>(t) * a.ldo + j;
      if (a.out_f16)
        static_cast<_Float16*>(a.out)[o] = static_cast<_Float16>(v);
      else
        static_cast<float*>(a.out)[o] = v;
    }
  }
}

}  // namespace trellis
