// decode.h — gfx950 device code shared by every trellis kernel: the wrapped 16-bit
// window read from the packed stream and the three computed codebooks.
//
// Packed layout (scripts/export_packed.py:27-35): per 16x16 tile, nwords = 8K little-
// endian u32 words; bit kb of symbol t sits at stream bit (255-t)*K + kb. The state of
// position t is the 16-bit window starting at bit (255-t)*K, read with wrap-around at
// word granularity (web/kernels.js:115-122); this equals qtip.py decode_window over the
// tail-biting stream (qtip.py:82-110).
//
// One tile row r (t = 16r + c, c = 0..15) occupies a 16*K-1+16 bit span starting at bit
// (240-16r)*K. For K = 2 and 4 that start is word aligned; for K = 3 it is at bit 16
// of its first word for even r and bit 0 for odd r. decode_row<K, PAR> therefore works
// on three consecutive words W0..W2 (word indices a, a+1, a+2 mod nwords, with
// a = ((240-16r)*K) >> 5) and every window's word pair and shift is a compile-time
// constant once K and the row parity PAR are fixed.
//
// Codebook arithmetic (qtip.py:32-53) uses the full-rate gfx950 v_mul_lo_u32 on the
// masked 16-bit state, then one v_bitop3_b32 for the lop3 mask/xor; its result is the
// fp16 pair (hi, lo) whose fp32 sum is the codebook value. Window extraction: the row's
// words are re-sliced at 16-bit granularity (W0, W0:W1>>16, W1, W1:W2>>16, W2), so every
// window lies inside one 32-bit register and costs one v_bfe_u32.
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

// Word index of the first of the three words a tile row reads.
template <int K>
__device__ __forceinline__ int row_word0(int r) {
  return ((240 - 16 * r) * K) >> 5;
}

// Bit offset of the row's lowest window (column 15) inside word W0.
template <int K, int PAR>
constexpr int row_bit0() {
  return (K == 3 && PAR == 0) ? 16 : 0;
}

// Does the row need its third word?
template <int K, int PAR>
constexpr bool row_needs_w2() {
  return row_bit0<K, PAR>() + K * 15 + 16 > 64;  // span ends beyond W1
}

// Decode the 16 windows of one tile row. f(c, raw) receives column c = 0..15 and the
// raw codebook output (cb_raw) of state t = 16r + c.
template <int K, int PAR, int CB, typename F>
__device__ __forceinline__ void decode_row(uint32_t W0, uint32_t W1, uint32_t W2, F&& f) {
  constexpr int B0 = row_bit0<K, PAR>();
  // 16-bit-aligned views of the row's 96-bit span: R[j] = bits [16j, 16j+32)
  const uint32_t R1 = __builtin_amdgcn_alignbit(W1, W0, 16);
  const uint32_t R3 = __builtin_amdgcn_alignbit(W2, W1, 16);
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const int off = B0 + K * (15 - c);
    const int j = off >> 4;
    const int s = off & 15;
    const uint32_t Rj = j == 0 ? W0 : j == 1 ? R1 : j == 2 ? W1 : j == 3 ? R3 : W2;
    const uint32_t state = (Rj >> s) & 0xFFFFu;
    f(c, cb_raw<CB>(state));
  }
}

}  // namespace trellis
