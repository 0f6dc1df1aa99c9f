// decode.h — gfx950 device code shared by every trellis kernel: the wrapped 16-bit
// window read from the packed stream and the three computed codebooks.
//
// Packed layout (scripts/export_packed.py:27-35): per 16x16 tile, nwords = 8K little-
// endian u32 words; bit kb of symbol t sits at stream bit (255-t)*K + kb. The state of
// position t is the 16-bit window starting at bit (255-t)*K, read with wrap-around at
// word granularity (web/kernels.js:115-122); this equals qtip.py decode_window over the
// tail-biting stream (qtip.py:82-110).
//
// Codebook arithmetic (qtip.py:32-53) uses the full-rate gfx950 v_mul_lo_u32 on the
// masked 16-bit state, then one v_bitop3_b32 for the lop3 mask/xor; its result is the
// fp16 pair (hi, lo) whose fp32 sum is the codebook value.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace trellis {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

enum { CB_MCG = 0, CB_3INST = 1, CB_1MAD = 2 };

template <int CB> struct Lcg;
template <> struct Lcg<CB_MCG> {
  static constexpr uint32_t MUL = 0xCBAC1FEDu, ADD = 0u;
};
template <> struct Lcg<CB_3INST> {
  static constexpr uint32_t MUL = 89226354u, ADD = 64248484u;
};
template <> struct Lcg<CB_1MAD> {
  static constexpr uint32_t MUL = 34038481u, ADD = 76625530u;
};

// P = state*MUL + ADD mod 2^32 for a 16-bit state (upper bits of `state` are zero).
template <int CB>
__device__ __forceinline__ uint32_t lcg_p(uint32_t state) {
  return state * Lcg<CB>::MUL + Lcg<CB>::ADD;
}

// (P & 0x8FFF8FFF) ^ 0x3B603B60: the fp16 pair (hi, lo) of MCG / 3INST (qtip.py:44,52).
__device__ __forceinline__ uint32_t lop3_pair(uint32_t p) {
  return (p & 0x8FFF8FFFu) ^ 0x3B603B60u;
}

// Byte sum of P (qtip.py:36), via v_sad_u8 against zero.
__device__ __forceinline__ uint32_t byte_sum(uint32_t p) {
  return __builtin_amdgcn_sad_u8(p, 0u, 0u);
}

// Exact fp32 codebook value from the raw per-state output: fp16 halves summed in fp32
// (exact: both halves lie in +-[0.125, 2)), or the 1MAD standardisation with an
// IEEE-rounded fp32 divide, matching torch's CPU arithmetic (qtip.py:28-29, 37).
template <int CB>
__device__ __forceinline__ float cb_exact(uint32_t raw) {
  if constexpr (CB == CB_1MAD) {
    return (static_cast<float>(raw) - 510.0f) / 147.800537109375f;
  } else {
    half2_t h = __builtin_bit_cast(half2_t, raw);
    return static_cast<float>(h.y) + static_cast<float>(h.x);
  }
}

// Raw per-state output: the fp16 pair for MCG/3INST, the byte sum for 1MAD.
template <int CB>
__device__ __forceinline__ uint32_t cb_raw(uint32_t state) {
  const uint32_t p = lcg_p<CB>(state);
  if constexpr (CB == CB_1MAD)
    return byte_sum(p);
  else
    return lop3_pair(p);
}

// The four windows t = 16r + 4g + q (q = 0..3) of one lane of a 16x16 MFMA tile (r = tile
// row, g = column group). The lowest of them (q = 3) starts at stream bit
// o3 = (252 - 16r - 4g) * K, and all four lie in the 32-bit funnel of words (wa, wb) at
// shift sh: wa = o3 >> 5, wb = (wa + 1) % nwords (the stream wraps at word granularity),
// sh = o3 & 31. Window q sits at bit K*(3-q) of the funnel.
struct QuadPos {
  int wa, wb, sh;
};

template <int K>
__device__ __forceinline__ QuadPos quad_pos(int r, int g) {
  constexpr int NW = 8 * K;
  const int o3 = (252 - 16 * r - 4 * g) * K;
  return {o3 >> 5, ((o3 >> 5) + 1) % NW, o3 & 31};
}

// V=2 (two weights per trellis step; the reference has V=1 only, this build's definition):
// the tile's stream is read as 128 steps of 2K bits, step u at stream bit (127-u)*2K; the
// state of step u gives weight 2u from the codebook's first LCG iterate and weight 2u+1 from
// the second iterate of the same 32-bit map. Lane (r, g) holds columns 4g..4g+3, i.e. steps
// u0 = 8r + 2g and u1 = u0 + 1; u1's window starts at o1 = (126 - 8r - 2g) * 2K and u0's
// sits 2K bits above it in the same funnel (16 + 2K <= 24 bits).
template <int K>
__device__ __forceinline__ QuadPos quad_pos_v2(int r, int g) {
  constexpr int NW = 8 * K;
  const int o1 = (126 - 8 * r - 2 * g) * 2 * K;
  return {o1 >> 5, ((o1 >> 5) + 1) % NW, o1 & 31};
}

template <int K, int V>
__device__ __forceinline__ QuadPos quad_pos_v(int r, int g) {
  if constexpr (V == 2)
    return quad_pos_v2<K>(r, g);
  else
    return quad_pos<K>(r, g);
}

// Output stage of a full 32-bit LCG value: lop3 pair, or 1MAD's byte sum.
template <int CB>
__device__ __forceinline__ uint32_t cb_out(uint32_t p) {
  if constexpr (CB == CB_1MAD)
    return byte_sum(p);
  else
    return lop3_pair(p);
}

// Raw codebook outputs (cb_raw) of the lane's four weights (columns 4g..4g+3).
template <int K, int CB, int V = 1>
__device__ __forceinline__ void decode_quad(uint32_t wlo, uint32_t whi, int sh, uint32_t (&raw)[4]) {
  const uint32_t u = __builtin_amdgcn_alignbit(whi, wlo, sh);
  if constexpr (V == 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t p = lcg_p<CB>((u >> (2 * K * (1 - h))) & 0xFFFFu);
      raw[2 * h] = cb_out<CB>(p);
      raw[2 * h + 1] = cb_out<CB>(p * Lcg<CB>::MUL + Lcg<CB>::ADD);
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) raw[q] = cb_raw<CB>((u >> (K * (3 - q))) & 0xFFFFu);
  }
}

}  // namespace trellis
