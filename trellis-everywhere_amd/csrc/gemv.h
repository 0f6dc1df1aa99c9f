// gemv.h — packed linear for batch 1 to 16 on gfx950: a pipelined decode-GEMV.
//
// The decode goes straight into the A operand of v_mfma_f32_16x16x32_f16 (the codebook's
// fp16 pair (hi, lo) against a duplicated activation, fp32 accumulation: common.h),
// organised for batch 1, where the decode's VALU work and fixed per-launch latencies, not
// HBM, set the time. The MFMA's 16 B columns carry NB <= 16 batch rows (column n = batch
// row n; NB = 1 at batch 1), so a few rows cost about what one does (the planner sends
// batch 5 to 16 here only when the group's items fit one round on the CUs at the shorter
// k-ranges that NB > 4 rows of folded activations in LDS allow):
//
//   * Work item = one matrix x one 128-row output block (8 bands of 16 rows) x one
//     k-range of `kr` tile columns, run by one 16-wave workgroup (one per CU): waves w and
//     w + 8 own band w, each for half of the k-range, so every wave of a CU starts together
//     and none runs alone at the end.
//   * Each wave streams its half-band in stages of KC tiles through a wave-private ring of
//     two stages in LDS: gfx950's 16-byte buffer loads write each lane's chunk straight
//     into the ring (no VGPR staging, no LDS store instruction), one stage stays in flight
//     while the other is decoded, and the wave waits only on its own loads, so no barrier
//     is needed.
//   * Tiles are decoded GEMV_G at a time into separate A registers before their MFMAs are
//     issued: a decode then never waits for an MFMA to release its operands.
//   * The activation fold xf = Hb_k(isc_scaled * su * x) of the k-range (every batch row)
//     is computed once per workgroup (its loads are issued before the packed words) and
//     kept in LDS as (x, x) fp16 pairs.
//   * The two k-halves are added in LDS. With one k-range (S == 1) wave 0 applies
//     y = sv * osc * Hb_n(t) directly; with split-K it publishes the block's partial sum,
//     takes a ticket, and the last workgroup of the block adds the partials in slice order
//     (deterministic) before the fold. Above 4 rows wave n does this for batch row n.
//     sv * osc is loaded at kernel start.
#pragma once

#include "common.h"

namespace trellis {

// Split-K publication: why relaxed agent-scope atomics plus a vmcnt wait order the partial
// sums on gfx950 (both epilogues below use this pattern).
//
// The C++/HIP memory model alone does not promise it: the ticket's fetch_add is relaxed, so
// formally nothing orders a workgroup's partial-sum stores before it. The ordering comes
// from how gfx950 executes these operations:
//   1. A relaxed agent-scope atomic store is a global store with the coherence bits set
//      (sc1): it does not stay in the XCD's own, non-coherent L2 but is written through to
//      the device-coherent point (memory side of the Infinity Fabric / MALL), where every
//      XCD reads the same bytes.
//   2. `s_waitcnt vmcnt(0)` holds the wave until each of its stores is acknowledged by that
//      point, i.e. performed for every agent. Only then is the ticket's atomic issued.
//   3. The fetch_add is itself performed at the coherent point, so the arrivals form one
//      order there; the workgroup that reads S - 1 arrives after every other slice's
//      partial sums were performed.
//   4. The last workgroup reads the partials with relaxed agent-scope atomic loads (sc1:
//      they bypass the L2's possibly stale lines) issued only after its fetch_add has
//      returned (the branch on the returned value depends on it), so they read what was
//      performed before that fetch_add.
// A formal release/acquire pair (acq_rel on the fetch_add) compiles to a write-back of the
// XCD's whole L2 before the atomic and an invalidate after it (buffer_wbl2 sc1 /
// buffer_inv sc1); a device-scope fence here (__threadfence, the same write-back and
// invalidate) measured about ten times slower than this epilogue. The pattern above moves
// only the partial sums through the coherent point. Every step is exercised by the
// determinism tests (repeated calls bit-identical at batch 1, 16 and 64).

constexpr int GEMV_WAVES = 16;    // two waves per 16-row band: 128 rows per workgroup
constexpr int GEMV_MAX_KR = 256;  // tile columns per k-range (4096 activations)
// tile columns per k-range with NB batch rows: the rows' folded activations of one k-range
// live in LDS as (x, x) pairs, 64 bytes per tile column and row
__host__ __device__ constexpr int gemv_kr_max(int nb) { return nb <= 4 ? GEMV_MAX_KR : nb <= 8 ? 128 : 96; }
constexpr int GEMV_G = 4;         // tiles decoded before their MFMAs are issued
constexpr int GEMV_LDS = 160 * 1024;   // LDS bytes per CU (one workgroup per CU)

// words of one wave's ring slot (a stage of KC tiles: every lane's 16-byte chunks, 1 KB per
// load instruction), and the rows' folded activations per batch row (8 mod 64 words apart)
__host__ __device__ constexpr int gemv_swp(int K, int KC) { return ((KC * 8 * K / 4 + 63) / 64) * 256; }
__host__ __device__ constexpr int gemv_xrow(int nb) { return nb > 1 ? gemv_kr_max(nb) * 16 + 8 : gemv_kr_max(nb) * 16; }
// stages in each wave's LDS ring: two (one decoded while the next is in flight). Deeper
// rings measured slower on the 8B block at batch 1 (four stages: 59.3 us against 57.8, the
// register-staged loads this ring replaced: 58.4), as did 32-tile stages.
constexpr int GEMV_NS = 2;
__host__ __device__ constexpr int gemv_lds_bytes(int K, int KC, int nb) {
  return 4 * (GEMV_WAVES * GEMV_NS * gemv_swp(K, KC) + nb * gemv_xrow(nb) + 2 * nb * 128 +
              gemv_kr_max(nb) / 8 + 4);
}

// rows of activations transformed together by the fold (a compile-time count for a lambda)
template <int N> struct RowGroup { static constexpr int value = N; };

template <int K, int CB, int V, int KC, int NB, bool SINGLE>
__global__ __launch_bounds__(64 * GEMV_WAVES) void gemv_kernel(LinArgs g) {
  constexpr int NWK = 8 * K;                 // words per tile
  constexpr int SW = KC * NWK;               // words per wave-stage
  constexpr int CH = SW / 4;                 // 16-byte chunks per wave-stage
  constexpr int LOADS = (CH + 63) / 64;      // chunks per lane
  constexpr int CPT = NWK / 4;               // chunks per tile
  constexpr int SWP = gemv_swp(K, KC);       // words per ring slot: every lane's chunks
  constexpr int NS = GEMV_NS;                // ring slots per wave
  constexpr int KRM = gemv_kr_max(NB);       // tile columns per k-range (max)
  constexpr int FCH = (KRM * 16 / 128 + GEMV_WAVES - 1) / GEMV_WAVES;  // fold chunks per wave
  // folded activations of the NB batch rows, rows 8 mod 64 words apart (bank spread)
  constexpr int XROW = gemv_xrow(NB);
  static_assert(NB <= GEMV_WAVES, "one wave per batch row in the epilogue");
  static_assert(SWP == LOADS * 256, "ring slot layout");
  static_assert(gemv_lds_bytes(K, KC, NB) <= GEMV_LDS, "ring, activations and sums fit the LDS");
  __shared__ __align__(16) uint32_t stg[GEMV_WAVES * NS * SWP];
  __shared__ __align__(16) uint32_t xs[NB * XROW];
  __shared__ float tt[2][NB][128];
  __shared__ unsigned ready[KRM / 8];   // per 128-column chunk of xs: rows folded
  __shared__ unsigned nready;           // chunks folded so far
  __shared__ unsigned ticket_sh;        // split-K ticket, shared with every wave (NB > 4)
  // the wave index is uniform: kept scalar, so per-wave choices are scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // The kernel arguments are cold at every launch of a rotated weight set (~0.5-1 us a round
  // trip). One round of loads finds the item's matrix; every field the first loads need is
  // then read in one second round (the empty asm that takes them all keeps the compiler from
  // issuing them one at a time, each behind its own wait), both before the start-up barrier.
  // a one-matrix launch (SINGLE: o, down) reads its matrix's fields in the first round of
  // argument loads, without the item locator's round (8B block at batch 1 48.5 -> 47.45 us)
  const int mi = SINGLE ? 0 : locate_mat(g, blockIdx.x, false);
  const LinMat& m = g.m[mi];
  {
    const int f_i0 = m.item0, f_s = m.S, f_t = m.tiles_in, f_n = m.n, f_bi = m.block_in;
    const unsigned f_si = m.s_inv;
    const uint32_t* f_b = m.bits;
    const void* f_x = m.x;
    const float *f_su = m.su, *f_is = m.isc, *f_sv = m.sv, *f_os = m.osc;
    const long long f_ldx = m.ldx;
    const float f_nrm = m.nrm_in;
    const int f_kr = g.kr, f_xh = g.x_f16, f_bt = g.batch;
    asm volatile("" ::"s"(f_i0), "s"(f_s), "s"(f_t), "s"(f_n), "s"(f_bi), "s"(f_si), "s"(f_b),
                 "s"(f_x), "s"(f_su), "s"(f_is), "s"(f_sv), "s"(f_os), "s"(f_ldx), "s"(f_nrm),
                 "s"(f_kr), "s"(f_xh), "s"(f_bt));
  }
  if (threadIdx.x < KRM / 8) ready[threadIdx.x] = 0u;
  if (threadIdx.x == 0) nready = 0u;
  __syncthreads();
  const int bl = wave & 7, half = wave >> 3;     // band of the block, half of the k-range
  const unsigned local = blockIdx.x - m.item0;
  const int ob = m.S > 1 ? static_cast<int>(__umulhi(local, m.s_inv)) : static_cast<int>(local);
  const int sl = static_cast<int>(local) - ob * m.S;
  const int c0 = sl * g.kr;                          // first tile column of the k-range
  const int ntl = min(g.kr, m.tiles_in - c0);        // tile columns in the k-range
  const int nst = (ntl + KC - 1) / KC;
  const int s_mid = (nst + 1) / 2;
  const int s_begin = half ? s_mid : 0, s_end = half ? nst : s_mid;
  const int rows = min(128, m.n - ob * 128);
  const int band = ob * 8 + min(bl, rows / 16 - 1);
  uint32_t* myring = stg + wave * NS * SWP;
  const unsigned ring_base = __builtin_amdgcn_readfirstlane(lds_addr(myring));
  const int kcols = ntl * 16;
  const int nch = (kcols + 127) / 128;
  const int nbv = NB > 1 ? min(NB, g.batch) : 1;     // batch rows of the call (<= NB)

  // ---- loads. All of them go through range-checked buffer resources: an index past the
  // block's rows, the k-range's columns or the band's tiles reads zeros without touching
  // memory, so no address is clamped, every load is issued on every path (the number in
  // flight is static and each wait covers only the loads it needs), and per-lane offsets
  // are fixed while the per-stage part is one add. Order: output scales of the block
  // (used at the end), the fold's inputs (chunks w and w + GEMV_WAVES of the k-range),
  // then the wave's first stage of packed words (the rest of its ring after the fold).
  const rsrc_t r_sv = make_rsrc(m.sv + ob * 128, rows * 4);
  const rsrc_t r_osc = make_rsrc(m.osc + ob * 128, rows * 4);
  const int xsh = g.x_f16 ? 1 : 2;                   // log2 bytes per activation
  const unsigned ldx = NB > 1 ? static_cast<unsigned>(m.ldx) : 0u;
  const rsrc_t r_x = make_rsrc(static_cast<const char*>(m.x) + (static_cast<size_t>(c0) * 16 << xsh),
                               ((nbv - 1) * ldx + static_cast<unsigned>(kcols)) << xsh);
  const rsrc_t r_su = make_rsrc(m.su + c0 * 16, kcols * 4);
  const rsrc_t r_isc = make_rsrc(m.isc + c0 * 16, kcols * 4);
  const rsrc_t r_bits = make_rsrc(m.bits + (static_cast<size_t>(band) * m.tiles_in + c0) * NWK,
                                  static_cast<unsigned>(ntl) * NWK * 4);
  float so[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int o = (lane + 64 * h) * 4;
    so[h] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_sv, o, 0, 0)) *
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_osc, o, 0, 0));
  }
  // fold jobs: the k-range's 128-column chunks, chunk ch folded by wave ch % GEMV_WAVES
  // for every batch row (spreading the (chunk, row) pairs over all the waves measured
  // slower: every wave then folds before its first decode)
  // With 16 rows (one chunk per wave at most) the rows of a chunk are split over
  // wpc = 16 / nch waves, so few chunks of many rows still keep every wave folding: wave w
  // folds rows [f_r0, f_r1) of chunk w % nch (8B block at batch 16: q/k/v and o launches
  // ~0.5 us faster; at 8 rows it measured ~0.5 us slower, so 8 rows keep a chunk per wave).
  constexpr bool SPLIT = NB > 8;
  const int wpc = SPLIT ? max(1, GEMV_WAVES / nch) : 1;
  const int f_rpw = (nbv + wpc - 1) / wpc;
  const int f_r0 = SPLIT ? (wave / nch) * f_rpw : 0;
  const int f_r1 = SPLIT ? min(nbv, f_r0 + f_rpw) : nbv;
  const int f_ch0 = SPLIT ? (wave < nch * wpc ? wave % nch : nch) : wave;
  const int njobs = SPLIT ? nch * nbv : nch;     // rows folded (SPLIT) or chunks
  uint32_t fw[FCH][NB][2];
  float fsu[FCH][2], fis[FCH][2];
#pragma unroll
  for (int f = 0; f < FCH; ++f) {
    const int ch = f_ch0 + GEMV_WAVES * f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const unsigned e = ch < nch ? ch * 128 + lane + 64 * h : RSRC_OOB / 4;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        // the wave's n-th row, batch row f_r0 + n of the call (rows past its share read zeros)
        const int r = f_r0 + n;
        const unsigned en = r < f_r1 && ch < nch ? r * ldx + e : RSRC_OOB / 4;
        fw[f][n][h] = __builtin_amdgcn_raw_buffer_load_b32(r_x, static_cast<int>(((en << xsh) & ~3u)), 0, 0);
      }
      fsu[f][h] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_su, static_cast<int>(e * 4), 0, 0));
      fis[f][h] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_isc, static_cast<int>(e * 4), 0, 0));
    }
  }
  // keeps the fold's loads ahead of the packed words in issue order
  asm volatile("" ::: "memory");
  // byte offset of this lane's 16-byte chunk within a stage (chunks past the stage's last
  // are pointed out of range), and of stage s within the band's k-range. Load q of a stage
  // writes the lanes' chunks lane + 64 q, 16 bytes each, to words 256 q + 4 lane of the
  // stage's ring slot (the slot base is wave-uniform: it goes to M0), so the slot holds the
  // stage's tiles one after another, NWK words each.
  unsigned lo_q[LOADS];
#pragma unroll
  for (int q = 0; q < LOADS; ++q) {
    const int ch = lane + 64 * q;
    lo_q[q] = CH % 64 == 0 || ch < CH ? static_cast<unsigned>(((ch / CPT) * NWK + 4 * (ch % CPT)) * 4)
                                      : RSRC_OOB;
  }
  auto load_stage = [&](int s) {
    // a stage past the wave's last one (prefetch beyond the end) reads nothing
    const unsigned soff = s < s_end ? static_cast<unsigned>(s * KC * NWK * 4) : RSRC_OOB;
    const unsigned slot = ring_base + static_cast<unsigned>((s % NS) * SWP * 4);
#pragma unroll
    for (int q = 0; q < LOADS; ++q) load_lds16(r_bits, slot + 1024 * q, lo_q[q] + soff);
  };
  // only the first stage before the fold: a smaller burst of loads at kernel start, so
  // every wave's first stage (and the fold's inputs) arrive sooner; the rest of the
  // ring follows the fold
  load_stage(s_begin);

  // ---- activation fold: xf = Hb_k(isc_scaled * su * x) / sqrt(block_in) as (x,x) pairs
  {
    const float nrm = m.nrm_in;
    const FwhtLane fl = fwht_lane(lane, m.block_in);
#pragma unroll
    for (int f = 0; f < FCH; ++f) {
      const int ch = f_ch0 + GEMV_WAVES * f;
      if (ch < nch && f_r1 > f_r0) {
        const int e0 = ch * 128 + lane, e1 = e0 + 64;
        // columns past the k-range loaded as zeros; an f16 row stride is even, so the
        // element's half within its word follows e. Rows are transformed RG at a time,
        // level by level (fwht_chunks), so their dependent lane exchanges overlap (one row
        // after another, a wave's 16-row fold took up to ~6 us at batch 16); a group's rows
        // past the wave's share were loaded as zeros and are not stored. A wave with at most
        // four rows (16 rows over four chunks) transforms them four at a time: in groups of
        // eight, half its fold was rows of zeros.
        const int nr = f_r1 - f_r0;
        auto fold_rows = [&](auto rg) {
          constexpr int RG = decltype(rg)::value;
#pragma unroll
          for (int g0 = 0; g0 < NB; g0 += RG) {
            if (g0 >= nr) continue;
            float lo[RG], hi[RG];
#pragma unroll
            for (int j = 0; j < RG; ++j) {
              lo[j] = act_value(fw[f][g0 + j][0], e0, g.x_f16) * (fsu[f][0] * fis[f][0]);
              hi[j] = act_value(fw[f][g0 + j][1], e1, g.x_f16) * (fsu[f][1] * fis[f][1]);
            }
            fwht_chunks<RG>(lo, hi, m.block_in, lane, fl);
#pragma unroll
            for (int j = 0; j < RG; ++j) {
              if (g0 + j < nr) {
                const int n = f_r0 + g0 + j;
                xs[n * XROW + e0] = dup_half(lo[j] * nrm);
                xs[n * XROW + e1] = dup_half(hi[j] * nrm);
              }
            }
          }
        };
        if constexpr (SPLIT) {
          if (nr <= 4)
            fold_rows(RowGroup<4>{});
          else
            fold_rows(RowGroup<8>{});
        } else {
          fold_rows(RowGroup<(NB < 8 ? NB : 8)>{});
        }
        // publish the chunk's rows: their xs words are written before the count
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) {
          __hip_atomic_fetch_add(&ready[ch], static_cast<unsigned>(f_r1 - f_r0), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
          __hip_atomic_fetch_add(&nready, SPLIT ? static_cast<unsigned>(f_r1 - f_r0) : 1u,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
      }
    }
  }
  // Every load the compiler knows of (output scales, the fold's inputs) and stage s_begin
  // have landed: a wait the compiler sees, so it puts none of its own (for a register a
  // skipped fold chunk never read) after the next stages' loads, which it cannot count.
  __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
#pragma unroll
  for (int b = 1; b < NS; ++b) load_stage(s_begin + b);
  // No barrier: a wave decodes a stage as soon as the chunks it covers are folded for
  // every batch row (each wait ends: every wave publishes its chunks before it decodes
  // anything); once a wave has seen every chunk done it stops checking.
  bool all_ready = false;
  auto wait_chunks = [&](int s) {
    if (all_ready || s >= s_end) return;
    const unsigned done = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(&nready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    if (done >= static_cast<unsigned>(njobs)) {
      all_ready = true;
    } else {
      const int ca = (s * KC) >> 3, cb = min((s * KC + KC - 1) >> 3, nch - 1);
      for (int c = ca; c <= cb; ++c)
        while (__builtin_amdgcn_readfirstlane(__hip_atomic_load(
                   &ready[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) < static_cast<unsigned>(nbv))
          __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  };

  // ---- main loop: wait for stage s (this wave's own loads: the NS - 1 stages issued after
  // it may still be in flight), decode it from its ring slot, then refill that slot with
  // stage s + NS
  const int r = lane & 15, gq = lane >> 4;
  const QuadPos qp = quad_pos_v<K, V>(r, gq);
  // B column r of the MFMA is batch row r (columns past the call's repeat its last row;
  // their outputs are not used)
  const uint32_t* xsr = xs + (NB > 1 ? min(r, nbv - 1) * XROW : 0);
  float4_t acc = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  half8_t Bv[GEMV_G];
  auto stage = [&](int s) {
    // loads complete in issue order: with stages s + 1 .. s + NS - 1 (LOADS each) issued
    // after stage s, at most that many may be outstanding once stage s has landed
    wait_vmcnt<(NS - 1) * LOADS>();
    asm volatile("" ::: "memory");
    wait_chunks(s);
    const uint32_t* mystg = myring + (s % NS) * SWP;
    const uint32_t* xst = xsr + s * KC * 16 + 4 * gq;
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
    // tiles of this stage: none past the wave's last stage
    const int jn = s < s_end ? ntl - s * KC : 0;
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
    // every LDS read of the slot has returned before the next stage's loads write it
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    load_stage(s + NS);
  };
  // A stage past s_end decodes nothing and its loads read nothing, so the number of loads
  // in flight stays fixed for the waits. A SIMD issues from its oldest ready wave first, so
  // left alone its first wave finishes in about half the time of its last one, and the
  // last waves run alone, with nothing to hide their latencies behind. Each wave's issue
  // priority falls by one level per quarter of its stages done, so the waves of a SIMD
  // progress together (measured ~1 us less per 8B block, mostly on the gate+up launch).
  const int tot = s_end - s_begin > 0 ? s_end - s_begin : 1;
  for (int s = s_begin; s < s_end; ++s) {
    const int lvl = (4 * (s_end - s) - 1) / tot;
    if (lvl >= 3)
      __builtin_amdgcn_s_setprio(3);
    else if (lvl == 2)
      __builtin_amdgcn_s_setprio(2);
    else if (lvl == 1)
      __builtin_amdgcn_s_setprio(1);
    else
      __builtin_amdgcn_s_setprio(0);
    stage(s);
  }
  __builtin_amdgcn_s_setprio(0);
  // the ring's last loads (stages past the end) are not consumed: let them land
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  acc += acc1;
  // column n of C (batch row n): lanes n, n + 16, n + 32, n + 48 hold rows 4*gq + i of
  // the band
  if (r < NB) {
#pragma unroll
    for (int i = 0; i < 4; ++i) tt[half][r][bl * 16 + 4 * gq + i] = acc[i];
  }
  __syncthreads();
  if constexpr (NB > 4) {
    // ---- wave n finishes batch row n: the two k-halves, then (split-K) every row's
    // partial sum published, one ticket per workgroup, and in the last workgroup of the
    // block each wave adds its row's partials in slice order; then y = sv * osc * Hb_n(t)
    const int n = wave;
    const bool mine = n < nbv;
    float t0 = 0.f, t1 = 0.f;
    if (mine) {
      t0 = tt[0][n][lane] + tt[1][n][lane];
      t1 = tt[0][n][lane + 64] + tt[1][n][lane + 64];
    }
    if (m.S > 1) {
      // partial sums [block][slice][NB][128]; published as the comment at the top of this
      // file explains (write-through atomic stores, acknowledged before the ticket)
      float* mypart = m.part + (static_cast<size_t>(ob) * m.S + sl) * NB * 128 + n * 128;
      if (mine) {
        __hip_atomic_store(mypart + lane, t0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(mypart + lane + 64, t1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();   // every row's partial sum is stored before the ticket is taken
      if (wave == 0) {
        unsigned prev = 0;
        if (lane == 0)
          prev = __hip_atomic_fetch_add(m.tickets + ob, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __builtin_amdgcn_readfirstlane(prev);
        if (lane == 0) ticket_sh = prev;
      }
      __syncthreads();
      if (ticket_sh != static_cast<unsigned>(m.S - 1)) return;
      if (wave == 0 && lane == 0)
        __hip_atomic_store(m.tickets + ob, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (!mine) return;
      const float* rowpart = m.part + static_cast<size_t>(ob) * m.S * NB * 128 + n * 128;
      t0 = 0.f;
      t1 = 0.f;
      for (int s0 = 0; s0 < m.S; s0 += 8) {
        float q0[8], q1[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float* p = rowpart + static_cast<size_t>(min(s0 + u, m.S - 1)) * NB * 128;
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
    }
    if (!mine) return;
    if (CB == CB_1MAD) {
      t0 = t0 / 147.800537109375f;
      t1 = t1 / 147.800537109375f;
    }
    fwht_chunk(t0, t1, m.block_out, lane);
    const float nrm = m.nrm_out;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rl = lane + 64 * h;
      if (rl < rows) {
        const float v = (h ? t1 : t0) * nrm * so[h];
        const long long o = n * m.ldy + ob * 128 + rl;
        if (g.y_f16)
          st_wt(static_cast<_Float16*>(m.y) + o, static_cast<_Float16>(v));
        else
          st_wt(static_cast<float*>(m.y) + o, v);
      }
    }
    return;
  }
  if (wave != 0) return;

  // ---- wave 0: the two k-halves, then (split-K) publish, ticket, and in the last
  // workgroup of the block the partials in slice order; then y = sv * osc * Hb_n(t) of
  // every batch row
  float t0[NB], t1[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    t0[n] = tt[0][n][lane] + tt[1][n][lane];
    t1[n] = tt[0][n][lane + 64] + tt[1][n][lane + 64];
  }
  if (m.S > 1) {
    // partial sums [block][slice][NB][128], published as the comment at the top of this
    // file explains (write-through atomic stores, acknowledged before the ticket)
    float* mypart = m.part + (static_cast<size_t>(ob) * m.S + sl) * NB * 128;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      if (n < nbv) {
        __hip_atomic_store(mypart + n * 128 + lane, t0[n], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(mypart + n * 128 + lane + 64, t1[n], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    unsigned prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(m.tickets + ob, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __builtin_amdgcn_readfirstlane(prev);
    if (prev != static_cast<unsigned>(m.S - 1)) return;
    const float* obpart = m.part + static_cast<size_t>(ob) * m.S * NB * 128;
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      t0[n] = 0.f;
      t1[n] = 0.f;
    }
    // up to 8 slices of every batch row in flight together: these loads miss the L2 (the
    // partials come from other XCDs), so one round trip per 8 slices, not one per row
    for (int s0 = 0; s0 < m.S; s0 += 8) {
      float q0[NB][8], q1[NB][8];
#pragma unroll
      for (int n = 0; n < NB; ++n) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          // rows past the call's repeat its last one (their sums are never stored)
          const float* p = obpart + (static_cast<size_t>(min(s0 + u, m.S - 1)) * NB + min(n, nbv - 1)) * 128;
          q0[n][u] = __hip_atomic_load(p + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          q1[n][u] = __hip_atomic_load(p + lane + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
#pragma unroll
      for (int n = 0; n < NB; ++n) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (s0 + u < m.S) {
            t0[n] += q0[n][u];
            t1[n] += q1[n][u];
          }
        }
      }
    }
    if (lane == 0) __hip_atomic_store(m.tickets + ob, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const float nrm = m.nrm_out;
  const FwhtLane fl = fwht_lane(lane, m.block_out);
  // every row's transform at once (rows past the call's hold a copy of a valid row's sums
  // and are not stored), so their lane exchanges overlap
  if (CB == CB_1MAD) {
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      t0[n] = t0[n] / 147.800537109375f;
      t1[n] = t1[n] / 147.800537109375f;
    }
  }
  fwht_chunks<NB>(t0, t1, m.block_out, lane, fl);
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    if (n >= nbv) break;
    const float a = t0[n], b = t1[n];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int rl = lane + 64 * h;
      if (rl < rows) {
        const float v = (h ? b : a) * nrm * so[h];
        const long long o = (NB > 1 ? n * m.ldy : 0) + ob * 128 + rl;
        if (g.y_f16)
          st_wt(static_cast<_Float16*>(m.y) + o, static_cast<_Float16>(v));
        else
          st_wt(static_cast<float*>(m.y) + o, v);
      }
    }
  }
}

}  // namespace trellis
