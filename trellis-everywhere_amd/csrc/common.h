// common.h — what the gfx950 trellis kernels share: launch arguments of a group of packed
// linears, activation access, the lane-shuffle block Hadamard, the batched x fold, and the
// decode of one tile straight into the A operand of v_mfma_f32_16x16x32_f16.
//
// The incoherence-processing fold (web/packed.js:163-182 runs it as seven dispatches per
// linear) is split around the decode-matmul: xf = Hb_k(isc_scaled * su * x) on the input
// side (fused in gemv_kernel at batch 1, xfold_kernel once per call for batch > 1) and
// y = sv * osc * Hb_n(t) on the output side (in the kernels' epilogues).
//
// Decode to MFMA: lane l = (tile row r = l%16, column group g = l/16) decodes the 4
// weights of columns 4g..4g+3 (decode.h). The codebook's lop3 result is the fp16 pair
// (hi, lo) of a weight; its two halves are two adjacent k elements of the A operand and
// the B operand holds the activation twice at those positions, so the MFMA accumulates
// (hi + lo) * x in fp32 and the exact codebook value (the fp32 sum of the halves,
// qtip.py:28-29) is never rounded.
#pragma once

#include "decode.h"

namespace trellis {

constexpr int MAX_GROUP = 8;   // linears per launch

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Launch arguments. The kernels read them straight from the kernel-argument segment, which is
// cold at every launch of a rotated weight set (~0.5-1 us a round trip): the fields a
// kernel's first instructions need of a matrix (its first work item and what locates the
// item, the pointers of the first loads) sit in the matrix's first 64-byte line, and the
// launch-wide fields in the first line of all.
struct alignas(64) LinMat {
  // ---- first line: item location and the pointers of the first loads
  int item0;            // first group-wide work item of this matrix
  int S;                // k-ranges (slices)
  unsigned s_inv;       // ceil(2^32 / S) for S > 1 (item / S = umulhi(item, s_inv)), else 0
  int tiles_in;
  const uint32_t* bits;
  const void* x;
  const float* su;
  const float* isc;     // isc_scaled = f32(isc) * scale
  const float* sv;
  const float* osc;
  // ---- second line
  int n, block_in, k, block_out;
  float nrm_in, nrm_out;  // 1 / sqrt(block_in), 1 / sqrt(block_out), rounded as fp32 ops
  int n_ob;
  int xfw;              // words per xf row: k ((x, x) fp16 pairs), or kp / 2 in the fp16-weight
                        // mode (kp = k rounded up to 32; fp16 values, tile pairs interleaved)
  long long ldx, ldy;
  void* y;
  float* part;          // workspace: split-K partial sums (S > 1)
  // ---- third line
  unsigned* tickets;    // workspace: [n_ob] arrival counters (batch 1, S > 1), zero between calls
  uint32_t* xf;         // workspace: [batch][xfw words] folded activations (xfold_kernel)
  int chunk0;           // first group-wide x-fold job of this matrix
  int fold0;            // first group-wide bfold_kernel job of this matrix
};

struct alignas(64) LinArgs {
  int nmat;
  int total;            // work items of the launched kernel
  int nwords;
  int batch;            // batch rows of the call
  int x_f16, y_f16;
  int kr;               // tile columns per k-range
  int mma_f16;          // batched path: codebook values rounded to fp16, one MAC per weight
  LinMat m[MAX_GROUP];
};

// Range-checked buffer loads: a buffer resource over [base, base + bytes); an offset at or
// past the end reads zeros without touching memory. Word 3 is gfx9's raw-buffer format.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           0x00020000);
}
constexpr unsigned RSRC_OOB = 0x40000000u;   // an offset past every buffer made here
constexpr int AUX_NT = 2;                    // nontemporal cache policy (gfx94x/gfx950)
constexpr int AUX_SC1 = 16;                  // agent scope (sc1): written through past the L2

// Stores of what another kernel reads (the x fold's output, split-K partial sums, every
// final output): relaxed agent-scope atomic stores, i.e. plain stores with the sc1 bit,
// which write through the XCD's L2 to the device-coherent point. The L2 then holds no
// dirty lines of them when the kernel ends, so the release at the kernel boundary has
// less to write back before the next kernel may start (8B block at batch 64: 123.1 ->
// 120.0 us; 512-token prefill in the fp16-weight mode 352 -> 345 us).
__device__ __forceinline__ void st_wt(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_wt(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_wt(_Float16* p, _Float16 v) {
  __hip_atomic_store(reinterpret_cast<unsigned short*>(p), __builtin_bit_cast(unsigned short, v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS byte address of a shared-memory pointer.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return static_cast<unsigned>(reinterpret_cast<size_t>(
      (__attribute__((address_space(3))) void*)(const_cast<void*>(p))));
}

// s_waitcnt for the vector-memory counter only (expcnt and lgkmcnt at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One 16-byte global -> LDS load per lane (gfx950 buffer_load_dwordx4 ... lds, nontemporal):
// the 16 bytes at byte offset `voff` of the buffer (zeros past its end) land at LDS byte
// address `lds_base` + 16 * lane; lds_base is wave-uniform (it goes to M0, which is saved
// and restored). Written as inline assembly because the compiler's wait-count pass cannot
// tell which LDS bytes such a load writes, and puts a wait for every outstanding load in
// front of each later LDS read; the caller waits for these loads itself (s_waitcnt vmcnt).
// Loads complete in issue order, so the compiler's own waits for earlier loads stay
// correct (they may wait longer than needed, never shorter). GFX9 needs one wait state
// between an SALU write of M0 and an LDS-DMA load that reads it; the compiler's hazard
// pass does not look inside inline assembly, so the s_nop is written here.
__device__ __forceinline__ void load_lds16(rsrc_t r, unsigned lds_base, unsigned voff) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, 0 offen nt lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_base), "v"(voff), "s"(r)
      : "memory");
}

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

// The value lane ^ H holds, without LDS: DPP for partners inside a 16-lane row
// (quad_perm for 1 and 2; for 4, a quad reversal (lane j takes j ^ 3) followed by
// row_half_mirror (lane i takes i ^ 7): (i ^ 7) ^ 3 = i ^ 4; row_ror:8 for 8) and gfx950's
// permlane swaps for 16 and 32 (with both operands equal, the first result holds the
// partner of the odd rows / upper half, the second that of the even rows / lower half).
template <int H>
__device__ __forceinline__ float lane_xor(float v, int lane) {
  const int iv = __builtin_bit_cast(int, v);
  int r;
  if constexpr (H == 1) {
    r = __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  } else if constexpr (H == 2) {
    r = __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  } else if constexpr (H == 4) {
    const int rev = __builtin_amdgcn_mov_dpp(iv, 0x1B, 0xF, 0xF, false);  // quad_perm [3,2,1,0]
    r = __builtin_amdgcn_mov_dpp(rev, 0x141, 0xF, 0xF, false);            // row_half_mirror
  } else if constexpr (H == 8) {
    r = __builtin_amdgcn_mov_dpp(iv, 0x128, 0xF, 0xF, false);  // row_ror:8 = lane i ^ 8
  } else if constexpr (H == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
    r = (lane & 16) ? static_cast<int>(p[0]) : static_cast<int>(p[1]);
  } else {
    static_assert(H == 32, "partner distance");
    const auto p = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
    r = (lane & 32) ? static_cast<int>(p[0]) : static_cast<int>(p[1]);
  }
  return __builtin_bit_cast(float, r);
}

// One butterfly level (partner distance H <= 8) on values kept with a per-lane sign: a lane
// stores st(l) = a(l) * v(l), a(l) = +-1, and the level computes st(l) + s(l) * st(l ^ H)
// with s(l) = -1 where bit H of the lane is set. As a(l ^ H) = a(l) (no earlier level
// touched bit H), that is a(l) * (v(l) + v(l ^ H)) in the lower lane and
// -a(l) * (v(l ^ H) - v(l)) in the upper one: the Hadamard butterfly, each result rounded
// once exactly as the plain add or subtract rounds it, with s(l) joining a(l). One DPP move
// and one fma per value, in place of an add, a subtract and a select.
template <int H>
__device__ __forceinline__ void butterfly(float& lo, float& hi, float s, int lane) {
  lo = __builtin_fmaf(lane_xor<H>(lo, lane), s, lo);
  hi = __builtin_fmaf(lane_xor<H>(hi, lane), s, hi);
}

// Butterfly levels 16 and 32 on both values at once: one permlane swap of (lo, hi) puts a
// butterfly pair in every lane (lanes of the lower row / half: lo's pair (l, l + H); of the
// upper: hi's pair (l - H, l)), the lane forms (lower + upper, lower - upper), and a second
// swap puts the results back in place. Signs are unchanged (both values of a pair carry
// the same a(l)).
template <int H>
__device__ __forceinline__ void butterfly_swap(float& lo, float& hi) {
  uint32_t a, b;
  if constexpr (H == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, lo),
                                                    __builtin_bit_cast(uint32_t, hi), false, false);
    a = p[0];
    b = p[1];
  } else {
    static_assert(H == 32, "partner distance");
    const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, lo),
                                                    __builtin_bit_cast(uint32_t, hi), false, false);
    a = p[0];
    b = p[1];
  }
  const float x = __builtin_bit_cast(float, a), y = __builtin_bit_cast(float, b);
  const uint32_t sum = __builtin_bit_cast(uint32_t, x + y), dif = __builtin_bit_cast(uint32_t, x - y);
  if constexpr (H == 16) {
    const auto q = __builtin_amdgcn_permlane16_swap(sum, dif, false, false);
    lo = __builtin_bit_cast(float, static_cast<uint32_t>(q[0]));
    hi = __builtin_bit_cast(float, static_cast<uint32_t>(q[1]));
  } else {
    const auto q = __builtin_amdgcn_permlane32_swap(sum, dif, false, false);
    lo = __builtin_bit_cast(float, static_cast<uint32_t>(q[0]));
    hi = __builtin_bit_cast(float, static_cast<uint32_t>(q[1]));
  }
}

// Per-lane constants of fwht_chunk for one block size: the signs s(l) of the levels 1 to 8
// and the sign bit that restores a(l) at the end (computed once, used for many chunks).
struct FwhtLane {
  float s1, s2, s4, s8;
  uint32_t flip;
};

__device__ __forceinline__ FwhtLane fwht_lane(int lane, int B) {
  auto sgn = [&](int h) { return __builtin_bit_cast(float, 0x3F800000u | (static_cast<uint32_t>(lane & h) != 0u ? 0x80000000u : 0u)); };
  return {sgn(1), sgn(2), sgn(4), sgn(8),
          static_cast<uint32_t>(__builtin_popcount(lane & ((B < 16 ? B : 16) - 1)) & 1) << 31};
}

// Butterflies of a normalized-free block Hadamard (block B <= 128, a power of 2) on a
// 128-element chunk held as lo = e[lane], hi = e[lane + 64]; pairs are exchanged in
// registers (DPP, permlane swaps), so a level costs a few VALU operations, not an LDS
// round trip. The levels 1 to 8 leave each lane's values multiplied by
// a(l) = (-1)^popcount(l & (min(B, 16) - 1)) (butterfly); one sign flip at the end
// restores them exactly. `fl` is fwht_lane(lane, B).
__device__ __forceinline__ void fwht_chunk(float& lo, float& hi, int B, int lane, const FwhtLane& fl) {
  if (B > 1) butterfly<1>(lo, hi, fl.s1, lane);
  if (B > 2) butterfly<2>(lo, hi, fl.s2, lane);
  if (B > 4) butterfly<4>(lo, hi, fl.s4, lane);
  if (B > 8) butterfly<8>(lo, hi, fl.s8, lane);
  if (B > 16) butterfly_swap<16>(lo, hi);
  if (B > 32) butterfly_swap<32>(lo, hi);
  if (B == 128) {
    const float a = lo, b = hi;
    lo = a + b;
    hi = a - b;
  }
  lo = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, lo) ^ fl.flip);
  hi = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, hi) ^ fl.flip);
}

__device__ __forceinline__ void fwht_chunk(float& lo, float& hi, int B, int lane) {
  fwht_chunk(lo, hi, B, lane, fwht_lane(lane, B));
}

// fwht_chunk on C independent chunks, level by level, so the chunks' dependent lane
// exchanges overlap instead of running one chunk after another (same operations per chunk,
// same results).
template <int C>
__device__ __forceinline__ void fwht_chunks(float (&lo)[C], float (&hi)[C], int B, int lane,
                                            const FwhtLane& fl) {
  if (B > 1)
#pragma unroll
    for (int c = 0; c < C; ++c) butterfly<1>(lo[c], hi[c], fl.s1, lane);
  if (B > 2)
#pragma unroll
    for (int c = 0; c < C; ++c) butterfly<2>(lo[c], hi[c], fl.s2, lane);
  if (B > 4)
#pragma unroll
    for (int c = 0; c < C; ++c) butterfly<4>(lo[c], hi[c], fl.s4, lane);
  if (B > 8)
#pragma unroll
    for (int c = 0; c < C; ++c) butterfly<8>(lo[c], hi[c], fl.s8, lane);
  if (B > 16)
#pragma unroll
    for (int c = 0; c < C; ++c) butterfly_swap<16>(lo[c], hi[c]);
  if (B > 32)
#pragma unroll
    for (int c = 0; c < C; ++c) butterfly_swap<32>(lo[c], hi[c]);
  if (B == 128)
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float a = lo[c], b = hi[c];
      lo[c] = a + b;
      hi[c] = a - b;
    }
#pragma unroll
  for (int c = 0; c < C; ++c) {
    lo[c] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, lo[c]) ^ fl.flip);
    hi[c] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, hi[c]) ^ fl.flip);
  }
}

__device__ __forceinline__ uint32_t dup_half(float v) {
  const _Float16 h = static_cast<_Float16>(v);
  const uint16_t u = __builtin_bit_cast(uint16_t, h);
  return (static_cast<uint32_t>(u) << 16) | u;
}

// The matrix of a group-wide job number: the last one whose first job (field F of LinMat)
// is at or below it. Every matrix's first-job field is loaded in one round, needed or not
// (the argument segment holds all MAX_GROUP entries; conditional loads went out in two
// dependent rounds from the cold segment).
template <int LinMat::*F>
__device__ __forceinline__ int locate_by(const LinArgs& g, int it) {
  int s[MAX_GROUP];
#pragma unroll
  for (int j = 1; j < MAX_GROUP; ++j) s[j] = g.m[j].*F;
  const int nm = g.nmat;
  asm volatile("" ::"s"(s[1]), "s"(s[2]), "s"(s[3]), "s"(s[4]), "s"(s[5]), "s"(s[6]), "s"(s[7]),
               "s"(nm));
  int mi = 0;
#pragma unroll
  for (int j = 1; j < MAX_GROUP; ++j)
    if (j < nm && it >= s[j]) mi = j;
  return mi;
}

__device__ __forceinline__ int locate_fold(const LinArgs& g, int it) {
  return locate_by<&LinMat::fold0>(g, it);
}

__device__ __forceinline__ int locate_mat(const LinArgs& g, int it, bool by_chunk) {
  return by_chunk ? locate_by<&LinMat::chunk0>(g, it) : locate_by<&LinMat::item0>(g, it);
}

// The fp16-weight mode's B layout: the 32 activations of a tile pair (columns 32p .. 32p+31)
// are stored as, for g = 0..3, columns 32p + 4g .. +3 then 32p + 16 + 4g .. +3, so the 16
// bytes at half 32p + 8g hold the k-slots 8g .. 8g+7 that lane group g of an MFMA fragment
// reads: the first tile's columns 4g .. 4g+3, then the second tile's (decode_a_pair).
__device__ __forceinline__ int xf_pair_slot(int e) {
  return (e & ~31) + 8 * ((e >> 2) & 3) + 4 * ((e >> 4) & 1) + (e & 3);
}

// ---------------------------------------------------------------- x fold
// xf = Hb_k(isc * su * x) scaled by 1/sqrt(block_in), stored as (x,x) fp16 pairs. One
// wave per (matrix, group of R batch rows, 128-column chunk), every load a range-checked
// buffer load issued up front. Up to 64 rows the kernel is latency-bound (a few MB): one
// row per wave gives every SIMD several waves to overlap the transform's dependent lane
// exchanges (8B gate+up fold at batch 64, alone in a graph chain: 2.7 us per launch,
// against 2.9 with 2 rows and 3.6 with 4 rows per wave). From 256 rows up a launch needs
// several rounds of waves on the CUs, each paying the start-up latency: four rows per wave
// (their scales loaded once, the rows transformed together) took the 8B block's folds at
// batch 512 from 12.5 to 9.5 us per launch on average (kernel trace), eight rows 9.7; the
// block 517 -> 503.5 us, 360 -> 347.5 in the fp16-weight mode; at 128 rows no change.
__host__ __device__ constexpr int xfold_rows(int batch) { return batch >= 256 ? 4 : 1; }
#ifdef TRELLIS_XFOLD_DEFINE
template <int XFOLD_ROWS, bool SINGLE>
__global__ __launch_bounds__(256) void xfold_kernel(LinArgs g) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int job = blockIdx.x * 4 + wave;
  if (job >= g.total) return;
  // a one-matrix launch reads its matrix's fields in the first round of argument loads
  const int mi = SINGLE ? 0 : locate_mat(g, job, true);
  const LinMat& m = g.m[mi];
  const int local = job - m.chunk0;
  const int nch = (m.k + 127) / 128;
  const int rg = local / nch, ch = local % nch;
  const int b0 = rg * XFOLD_ROWS;
  const int kvalid = min(128, m.k - ch * 128);
  const int xsh = g.x_f16 ? 1 : 2;
  const rsrc_t r_x = make_rsrc(m.x, static_cast<unsigned>(g.batch) * static_cast<unsigned>(m.ldx) << xsh);
  const rsrc_t r_su = make_rsrc(m.su, m.k * 4), r_isc = make_rsrc(m.isc, m.k * 4);
  const int e0 = ch * 128 + lane, e1 = e0 + 64;
  const float s0 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_su, e0 * 4, 0, 0)) *
                   __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_isc, e0 * 4, 0, 0));
  const float s1 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_su, e1 * 4, 0, 0)) *
                   __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_isc, e1 * 4, 0, 0));
  uint32_t w0[XFOLD_ROWS], w1[XFOLD_ROWS];
#pragma unroll
  for (int r = 0; r < XFOLD_ROWS; ++r) {
    const unsigned row = static_cast<unsigned>((b0 + r) * m.ldx);
    w0[r] = __builtin_amdgcn_raw_buffer_load_b32(r_x, static_cast<int>(((row + e0) << xsh) & ~3u), 0, 0);
    w1[r] = __builtin_amdgcn_raw_buffer_load_b32(r_x, static_cast<int>(((row + e1) << xsh) & ~3u), 0, 0);
  }
  const float nrm = m.nrm_in;
  const FwhtLane fl = fwht_lane(lane, m.block_in);
  // the rows are transformed together, level by level, so their dependent lane exchanges
  // overlap (rows past the call's were loaded as zeros and are not stored)
  float lov[XFOLD_ROWS], hiv[XFOLD_ROWS];
#pragma unroll
  for (int r = 0; r < XFOLD_ROWS; ++r) {
    // an f16 row stride is even, so the element's half within its word follows e
    lov[r] = lane < kvalid ? act_value(w0[r], e0, g.x_f16) * s0 : 0.0f;
    hiv[r] = lane + 64 < kvalid ? act_value(w1[r], e1, g.x_f16) * s1 : 0.0f;
  }
  fwht_chunks<XFOLD_ROWS>(lov, hiv, m.block_in, lane, fl);
#pragma unroll
  for (int r = 0; r < XFOLD_ROWS; ++r) {
    if (b0 + r >= g.batch) break;
    const float lo = lov[r], hi = hiv[r];
    if (g.mma_f16) {
      // fp16 values in tile-pair order (xf_pair_slot); columns k .. kp - 1 of the last
      // pair are written as zeros (lo and hi are zero there)
      _Float16* dst = reinterpret_cast<_Float16*>(m.xf + static_cast<size_t>(b0 + r) * m.xfw);
      const int kp = 2 * m.xfw;
      if (e0 < kp) st_wt(dst + xf_pair_slot(e0), static_cast<_Float16>(lo * nrm));
      if (e1 < kp) st_wt(dst + xf_pair_slot(e1), static_cast<_Float16>(hi * nrm));
    } else {
      uint32_t* dst = m.xf + static_cast<size_t>(b0 + r) * m.xfw + ch * 128;
      if (lane < kvalid) st_wt(dst + lane, dup_half(lo * nrm));
      if (lane + 64 < kvalid) st_wt(dst + lane + 64, dup_half(hi * nrm));
    }
  }
}
#endif

// ---------------------------------------------------------------- decode -> MFMA
// The A operand of one band-tile for this lane (decode_quad). 1MAD yields (y - 510) as an
// exact fp16 in the low half (the division by 147.800537109375 follows the sum).
template <int K, int CB, int V = 1>
__device__ __forceinline__ half8_t decode_a(uint32_t wlo, uint32_t whi, int sh) {
  uint32_t a4[4];
  decode_quad<K, CB, V>(wlo, whi, sh, a4);
  if constexpr (CB == CB_1MAD) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const _Float16 h = static_cast<_Float16>(static_cast<float>(static_cast<int>(a4[q]) - 510));
      a4[q] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
    }
  }
  return __builtin_bit_cast(half8_t, a4);
}

// hi + lo of two codebook pairs (hi in the upper half of each word) as one packed pair of
// fp16 sums: v_add_f16 with SDWA operand selects, one instruction per value. The fp16 add
// rounds the exact sum of the two halves to nearest even, as a cast of the reference's
// fp32 sum (qtip.py:28-29, 45, 53) to fp16 does.
__device__ __forceinline__ uint32_t add_halves2(uint32_t r0, uint32_t r1) {
  uint32_t d;
  asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:WORD_0\n\t"
      "v_add_f16_sdwa %0, %2, %2 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_1 src1_sel:WORD_0"
      : "=&v"(d)
      : "v"(r0), "v"(r1));
  return d;
}

// The A operand of a tile pair in the fp16-weight mode (one MAC per weight): k-slots
// 8g .. 8g+3 of lane (r, g) hold the first tile's columns 4g .. 4g+3, slots 8g+4 .. 8g+7
// the second tile's (xf_pair_slot lays B out to match), each codebook value rounded once
// to fp16. 1MAD's (y - 510) is an exact fp16 integer, as in decode_a.
template <int K, int CB, int V = 1>
__device__ __forceinline__ half8_t decode_a_pair(uint32_t wlo0, uint32_t whi0, uint32_t wlo1,
                                                 uint32_t whi1, int sh) {
  uint32_t a0[4], a1[4], o[4];
  decode_quad<K, CB, V>(wlo0, whi0, sh, a0);
  decode_quad<K, CB, V>(wlo1, whi1, sh, a1);
  if constexpr (CB == CB_1MAD) {
    uint32_t h[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int y = static_cast<int>(q < 4 ? a0[q] : a1[q - 4]) - 510;
      h[q] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(static_cast<float>(y)));
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = h[2 * w] | (h[2 * w + 1] << 16);
  } else {
    o[0] = add_halves2(a0[0], a0[1]);
    o[1] = add_halves2(a0[2], a0[3]);
    o[2] = add_halves2(a1[0], a1[1]);
    o[3] = add_halves2(a1[2], a1[3]);
  }
  return __builtin_bit_cast(half8_t, o);
}

}  // namespace trellis
