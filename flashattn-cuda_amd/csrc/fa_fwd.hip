// fa_fwd.hip — FlashAttention forward for MI355X (gfx950), fp16 in, fp32
// accumulate, O fp16 and optional logsumexp L fp32.
//
// Replaces the reference's fa3db_full_fwd_kernel and its launcher
// (cuda/flash_attn_fa3_db_full.cu:87-403) behind the C ABI in
// include/fa_mi355x.h. Same math: S = Q K^T / sqrt(D), online softmax in
// base 2 with running max m and sum l, O = P V / l, L = m ln2 + ln l
// (cuda/flash_attn_fa3_db_full.cu:202, :250-284, :319-343).
//
// Work decomposition (CDNA4):
//   * a workgroup owns 128 query rows of one (b, h), as four row groups of 32
//     rows (one wave each); a 1-D grid with an XCD-aware remap keeps the query
//     blocks of a head on one XCD so its K/V stay in that XCD's L2;
//   * K/V advance in 64-key tiles, copied global -> LDS by buffer_load ... lds
//     into double-buffered stages while the previous tiles are consumed; the
//     loops are unrolled by stage so every LDS read has a constant offset;
//   * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_f16 (fa_tile.hpp);
//   * softmax without a per-tile max reduction: P = 2^(S c - m) against the
//     running max m; the lane's tile sum bounds every P it holds, and only when
//     it exceeds 2^15 (first tile, or a much larger new maximum) is m raised
//     and O rescaled. P <= 2^15 stays inside fp16 and the fp32 accumulators.
// Two kernels share that per-wave core (RowBlock):
//   * fa_fwd_split_kernel<.., KSPLIT>: 4*KSPLIT waves; the KSPLIT waves of a
//     row group take every KSPLIT-th tile and merge their (m, l, O) through LDS
//     at the end. More waves per SIMD is what lets MFMA and VALU work of
//     different waves overlap (a single wave issues VALU work several times
//     slower than four waves sharing a SIMD);
//   * fa_fwd_pipe_kernel: one wave per row group, software-pipelined (QK of
//     tile t+1 issued alongside the softmax of tile t).
// Template flags: D in {64,128}, CAUSAL, WRITE_L (O-only when false), FULL
// (N % 128 == 0: no bounds predicates).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <type_traits>

#include "fa_mi355x.h"
#include "fa_tile.hpp"

namespace fa {

constexpr int kBR = 128;   // query rows per workgroup
constexpr int kBC = 64;    // keys per tile
constexpr int kRowGroups = kBR / 32;
// A lane's tile sum of P above this triggers a rescale; it bounds every P,
// so P stays far inside the fp16 range (65504).
constexpr float kSumLimit = 32768.0f;

// Workgroup g of `total` lands on XCD g % 8. Map it to a logical tile index
// so that each XCD gets one contiguous range of logical tiles.
__device__ __forceinline__ int xcd_remap(int g, int total) {
  const int q = total >> 3, r = total & 7;
  const int xcd = g & 7, slot = g >> 3;
  return (xcd < r) ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

// State and tile operations of one wave: 32 query rows, one lane pair per row
// (lanes l and l^32 hold the two halves of every 32-key block).
template <int D, bool CAUSAL, bool FULL>
struct RowBlock {
  static constexpr int KSTEPS = D / 16;   // QK k-steps
  static constexpr int DB = D / 32;       // O^T d-blocks

  int lane, hi, N, row_w, qrow;
  float c;
  f16x8 qf[KSTEPS];    // Q^T: the B operand of S^T = K Q^T
  f32x16 o[DB];        // O^T accumulators
  float m_run;         // running row max of S*c (log2 units), never lowered
  float l_run;         // this lane's share of the row sum at m_run

  __device__ __forceinline__ void init(const f16* Qh, int head_bytes, int lane_, int row_w_,
                                       int N_, float c_) {
    lane = lane_;
    hi = lane >> 5;
    N = N_;
    row_w = row_w_;
    qrow = row_w + (lane & 31);
    c = c_;
    // Buffer loads return zero for rows >= N.
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(Qh, head_bytes);
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(
          rq, (uint32_t)(qrow * D + 16 * kk + 8 * hi) * 2, 0, 0);
      qf[kk] = __builtin_bit_cast(f16x8, x);
    }
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = f32x16{};
    m_run = -INFINITY;
    l_run = 0.f;
  }

  // Tile t is entirely above the causal diagonal for these rows.
  __device__ __forceinline__ bool dead_tile(int t) const {
    return CAUSAL && t * kBC > row_w + 31;
  }

  // The functions below work on NB consecutive 32-key blocks of a 64-key
  // tile, starting at block kb0 (NB = 2: the whole tile).

  // S^T of the blocks: s[b] = K[32 (kb0+b) ..] Q^T.
  template <int NB>
  __device__ __forceinline__ void qk(const char* ks, int kb0, f32x16 (&s)[NB]) const {
#pragma unroll
    for (int b = 0; b < NB; ++b) s[b] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
#pragma unroll
      for (int b = 0; b < NB; ++b) s[b] = mfma32(load_k_frag<D>(ks, kb0 + b, kk, lane), qf[kk], s[b]);
    }
  }

  // The same products with the operand loads kept one k-step ahead of the
  // MFMAs and nothing moved across steps: bounds the live operand registers
  // (for kernels that run several waves per SIMD, whose other waves hide the
  // LDS latency).
  template <int NB>
  __device__ __forceinline__ void qk_lean(const char* ks, int kb0, f32x16 (&s)[NB]) const {
    f16x8 a[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      s[b] = f32x16{};
      a[b] = load_k_frag<D>(ks, kb0 + b, 0, lane);
    }
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      f16x8 n[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) n[b] = (kk + 1 < KSTEPS) ? load_k_frag<D>(ks, kb0 + b, kk + 1, lane) : a[b];
#pragma unroll
      for (int b = 0; b < NB; ++b) s[b] = mfma32(a[b], qf[kk], s[b]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < NB; ++b) a[b] = n[b];
    }
  }

  // Key of register r in block kb is key0 + 4 hi + kofs(kb, r) with a
  // compile-time kofs, so each test compares that constant against one
  // per-tile lane value (no per-register key arrays kept live).
  template <int NB>
  __device__ __forceinline__ void mask(int t, int kb0, f32x16 (&s)[NB]) const {
    const int key0 = t * kBC;
    const bool need = (!FULL && key0 + kBC > N) || (CAUSAL && key0 + kBC - 1 > row_w);
    if (need) {
      const int lane_key = key0 + 4 * hi;
      const int n_lim = N - lane_key;      // dead if kofs >= n_lim
      const int c_lim = qrow - lane_key;   // dead if kofs >  c_lim
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kofs = st_key(kb0 + b, r, 0);
          const bool dead = (!FULL && kofs >= n_lim) || (CAUSAL && kofs > c_lim);
          if (dead) s[b][r] = -INFINITY;
        }
      }
    }
  }

  // p = 2^(s c - m) into p (which may alias s); returns this lane's sum.
  template <int NB>
  __device__ __forceinline__ float expo(const f32x16 (&s)[NB], f32x16 (&p)[NB], float m) const {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[b][r] = exp2_hw(fmaf(s[b][r], c, -m));
        acc[r & 3] += p[b][r];
      }
    }
    return (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }

  // Raise m to the row max of s (both lanes of a row agree), rescale O and l.
  template <int NB>
  __device__ __forceinline__ void raise_max(const f32x16 (&s)[NB]) {
    float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
    for (int r = 2; r < 16; ++r) mx = fmaxf(mx, s[0][r]);
#pragma unroll
    for (int b = 1; b < NB; ++b) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[b][r]);
    }
    const float m_new = fmaxf(m_run, max_xor32(mx) * c);
    const float alpha = (m_new == m_run) ? 1.f : exp2_hw(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] *= alpha;
    m_run = m_new;
  }

  __device__ __forceinline__ float m_safe() const { return (m_run == -INFINITY) ? 0.f : m_run; }

  // B operands (P^T) of the PV k-steps of the blocks: two per block.
  template <int NB>
  static __device__ __forceinline__ void pack(const f32x16 (&p)[NB], f16x8 (&pf)[2 * NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      pf[2 * b] = pack_p(p[b], 0);
      pf[2 * b + 1] = pack_p(p[b], 1);
    }
  }

  // Softmax of the blocks, keeping the scores (the pipelined kernel cannot
  // reread K(t): its LDS stage is already being refilled).
  template <int NB>
  __device__ __forceinline__ void softmax_keep(const f32x16 (&s)[NB], f16x8 (&pf)[2 * NB]) {
    f32x16 p[NB];
    float rs = expo<NB>(s, p, m_run);
    if (!__all(rs <= kSumLimit)) {
      raise_max<NB>(s);
      rs = expo<NB>(s, p, m_safe());
    }
    l_run += rs;
    pack<NB>(p, pf);
  }

  // Softmax in place; on the rare slow path the scores are recomputed from
  // the K tile still resident at ks.
  template <int NB>
  __device__ __forceinline__ void softmax_inplace(f32x16 (&s)[NB], f16x8 (&pf)[2 * NB],
                                                  const char* ks, int t, int kb0) {
    float rs = expo<NB>(s, s, m_run);
    if (!__all(rs <= kSumLimit)) {
      qk_lean<NB>(ks, kb0, s);
      mask<NB>(t, kb0, s);
      raise_max<NB>(s);
      rs = expo<NB>(s, s, m_safe());
    }
    l_run += rs;
    pack<NB>(s, pf);
  }

  // O^T += V^T P^T over the PV k-steps of the blocks.
  template <int NB>
  __device__ __forceinline__ void pv(const char* vs, int kb0, const f16x8 (&pf)[2 * NB]) {
#pragma unroll
    for (int j = 0; j < 2 * NB; ++j) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
        o[db] = mfma32(load_v_frag<D>(vs, 2 * kb0 + j, db, lane), pf[j], o[db]);
    }
  }

  // PV with one (k-step, d-block) operand load in flight ahead of its MFMA.
  template <int NB>
  __device__ __forceinline__ void pv_lean(const char* vs, int kb0, const f16x8 (&pf)[2 * NB]) {
    f16x8 a = load_v_frag<D>(vs, 2 * kb0, 0, lane);
#pragma unroll
    for (int i = 0; i < 2 * NB * DB; ++i) {
      const int j = i / DB, db = i % DB;
      f16x8 n = a;
      if (i + 1 < 2 * NB * DB) n = load_v_frag<D>(vs, 2 * kb0 + (i + 1) / DB, (i + 1) % DB, lane);
      o[db] = mfma32(a, pf[j], o[db]);
      __builtin_amdgcn_sched_barrier(0);
      a = n;
    }
  }

  // Merge another wave's (m, l, O) for the same rows, read from LDS.
  __device__ __forceinline__ void merge_from(const float* src) {
    const float m2 = src[lane];
    const float l2 = src[64 + lane];
    const float M = fmaxf(m_run, m2);
    const float a1 = (m_run == M) ? 1.f : exp2_hw(m_run - M);
    const float a2 = (m2 == M) ? 1.f : exp2_hw(m2 - M);
    l_run = l_run * a1 + l2 * a2;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] = o[db][r] * a1 + src[(2 + 16 * db + r) * 64 + lane] * a2;
    }
    m_run = M;
  }

  __device__ __forceinline__ void save_to(float* dst) const {
    dst[lane] = m_run;
    dst[64 + lane] = l_run;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[(2 + 16 * db + r) * 64 + lane] = o[db][r];
    }
  }

  // Combine the two half-rows, normalise, store O (and L).
  template <bool WRITE_L>
  __device__ __forceinline__ void finish(f16* Oh, float* Lh) const {
    const float l_tot = sum_xor32(l_run);
    if (FULL || qrow < N) {
      const float inv = 1.f / l_tot;
      f16* orow = Oh + (size_t)qrow * D;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f16x2 a = cvt2(o[db][4 * g + 0] * inv, o[db][4 * g + 1] * inv);
          f16x2 b = cvt2(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
          f16x4 v4 = f16x4{a[0], a[1], b[0], b[1]};
          *reinterpret_cast<f16x4*>(orow + 32 * db + 8 * g + 4 * hi) = v4;
        }
      }
      if (WRITE_L && hi == 0) Lh[qrow] = (m_run + log2_hw(l_tot)) * kLn2;
    }
  }
};

// Per-lane DMA source offsets of 1 KiB block b of a tile: lane l writes bytes
// [16 l, 16 l + 16) of the block, so the XOR swizzle of the LDS layout is
// applied by choosing which global chunk the lane fetches.
template <int D>
__device__ __forceinline__ void dma_offsets(int b, int lane, uint32_t& koff, uint32_t& voff) {
  const int o = b * 1024 + 16 * lane;
  const int r = o / (2 * D);
  const int slot = (o % (2 * D)) / 16;
  koff = (uint32_t)(r * 2 * D + (slot ^ k_swz<D>(r)) * 16);
  voff = (uint32_t)(r * 2 * D + (slot ^ v_swz<D>(r)) * 16);
}

// Copy one 1 KiB block of tile t of a head (K or V) into dst. The buffer
// range ends at the head's last byte, so rows >= N arrive as zeros.
template <int D, bool FULL>
__device__ __forceinline__ void dma_block(const char* head, int head_bytes, int t, uint32_t dst,
                                          uint32_t off) {
  constexpr int TILE = kBC * D * 2;
  const int done = t * TILE;
  const int bytes = FULL ? TILE : min(TILE, head_bytes - done);
  dma16(make_rsrc(head + done, bytes), dst, off);
}

// As dma_block, but a tile past the end is still issued, with an empty buffer
// range (it writes zeros and reads no memory), so every wave issues the same
// number of copies per tile group and vmcnt counts stay exact.
template <int D, bool FULL>
__device__ __forceinline__ void dma_block_or_zero(const char* head, int head_bytes, int t,
                                                  bool valid, uint32_t dst, uint32_t off) {
  constexpr int TILE = kBC * D * 2;
  const int done = valid ? t * TILE : 0;
  const int bytes = !valid ? 0 : (FULL ? TILE : min(TILE, head_bytes - done));
  dma16(make_rsrc(head + done, bytes), dst, off);
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] at bits 3:0, vmcnt[5:4] at
// bits 15:14, expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// ---------------------------------------------------------------------------
// Split kernel: 4*KSPLIT waves; wave w is row group w % 4 and key slice w / 4.
// Tiles advance in groups of KSPLIT (one per key slice) through a ring of
// STAGES LDS stages, so the copy of group g+STAGES-1 is in flight while group
// g is consumed: the deeper the ring, the more of the global-memory latency
// the copies hide (all workgroups of a head request the same tile at about
// the same time, so a tile's first fetch is a miss for all of them).
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL, bool WRITE_L, bool FULL, int KSPLIT, int STAGES>
__global__ void __launch_bounds__(256 * KSPLIT)
fa_fwd_split_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                    const f16* __restrict__ V, f16* __restrict__ O,
                    float* __restrict__ L, int N, int num_qb, int total, float c) {
  constexpr int TILE = kBC * D * 2;
  constexpr int BLOCKS = TILE / 1024;                     // 1 KiB blocks per tile
  constexpr int WAVES = kRowGroups * KSPLIT;
  constexpr int LOADS = KSPLIT * BLOCKS / WAVES;          // blocks per wave per tile group
  constexpr int GROUP = KSPLIT * TILE;                    // bytes of one stage (K or V)
  constexpr int PER_GROUP = 2 * LOADS;                    // copies per wave per group
  static_assert(STAGES >= 2 && STAGES <= 4, "two to four stages");
  static_assert(2 * STAGES * GROUP <= 160 * 1024, "stages exceed the 160 KiB LDS");
  using RB = RowBlock<D, CAUSAL, FULL>;
  static_assert((KSPLIT - 1) * (2 + 16 * RB::DB) * 64 * 4 <= GROUP, "merge area too small");
  // Stage s: K part at 2*s*GROUP, V part at (2*s+1)*GROUP; each KSPLIT tiles.
  __shared__ __attribute__((aligned(1024))) char smem[2 * STAGES * GROUP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: SGPR
  const int rg = wave & (kRowGroups - 1);
  const int ks = wave / kRowGroups;

  const int logical = xcd_remap(blockIdx.x, total);
  const int bh = logical / num_qb;
  int qb = logical - bh * num_qb;
  if (CAUSAL) qb = num_qb - 1 - qb;   // longest rows dispatch first

  const size_t head = (size_t)bh * N * D;
  const int head_bytes = N * D * 2;
  const char* Kh = reinterpret_cast<const char*>(K + head);
  const char* Vh = reinterpret_cast<const char*>(V + head);
  const int q0 = qb * kBR;

  RB rb;
  rb.init(Q + head, head_bytes, lane, q0 + 32 * rg, N, c);

  // Blocks this wave copies in each tile group: tile slot within the group,
  // block within the tile, and the source offsets.
  uint32_t koff[LOADS], voff[LOADS];
  int slot_of[LOADS], blk_of[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int blk = wave * LOADS + i;
    slot_of[i] = blk / BLOCKS;
    blk_of[i] = blk % BLOCKS;
    dma_offsets<D>(blk_of[i], lane, koff[i], voff[i]);
  }

  const int kv_end = CAUSAL ? min(N, q0 + kBR) : N;
  const int n_tiles = (kv_end + kBC - 1) / kBC;
  const int n_groups = (n_tiles + KSPLIT - 1) / KSPLIT;

  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int g, int stage) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int t = g * KSPLIT + slot_of[i];
      const bool valid = t < n_tiles;
      const uint32_t at = lds0 + stage * 2 * GROUP + slot_of[i] * TILE + blk_of[i] * 1024;
      dma_block_or_zero<D, FULL>(Kh, head_bytes, t, valid, at, koff[i]);
      dma_block_or_zero<D, FULL>(Vh, head_bytes, t, valid, at + GROUP, voff[i]);
    }
  };

  // Prologue: groups 0 .. STAGES-2 in flight, then wait for all of them.
#pragma unroll
  for (int g = 0; g < STAGES - 1; ++g) {
    if (g < n_groups) issue(g, g);
  }
  wait_vmem();
  __syncthreads();
  auto step = [&](auto st, int g) {
    constexpr int ST = decltype(st)::value;     // g % STAGES
    const char* kc = smem + ST * 2 * GROUP + ks * TILE;
    const char* vc = kc + GROUP;
    // Stage (g-1) % STAGES was consumed by step g-1 (barrier at its end).
    if (g + STAGES - 1 < n_groups) issue(g + STAGES - 1, (ST + STAGES - 1) % STAGES);
    const int t = g * KSPLIT + ks;
    if (t < n_tiles && !rb.dead_tile(t)) {   // wave-uniform
      // The tile is consumed as two 32-key blocks: half the score and P
      // registers of a whole-tile pass, so more waves fit per SIMD.
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x16 s[1];
        f16x8 pf[2];
        rb.template qk<1>(kc, kb, s);
        rb.template mask<1>(t, kb, s);
        rb.template softmax_keep<1>(s, pf);
        rb.template pv<1>(vc, kb, pf);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // Wait for group g+1: the groups issued after it stay in flight.
    const int ahead = max(0, min(STAGES - 2, n_groups - 2 - g));
    if constexpr (STAGES >= 4) {
      if (ahead >= 2) wait_vmcnt<2 * PER_GROUP>();
      else if (ahead == 1) wait_vmcnt<PER_GROUP>();
      else wait_vmcnt<0>();
    } else if constexpr (STAGES == 3) {
      if (ahead >= 1) wait_vmcnt<PER_GROUP>();
      else wait_vmcnt<0>();
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();
  };
  for (int g = 0; g < n_groups; g += STAGES) {
    step(std::integral_constant<int, 0>{}, g);
    if (g + 1 < n_groups) step(std::integral_constant<int, 1>{}, g + 1);
    if constexpr (STAGES > 2) {
      if (g + 2 < n_groups) step(std::integral_constant<int, 2 % STAGES>{}, g + 2);
    }
    if constexpr (STAGES > 3) {
      if (g + 3 < n_groups) step(std::integral_constant<int, 3 % STAGES>{}, g + 3);
    }
  }

  if constexpr (KSPLIT > 1) {
    // Merge the key slices of each row group through LDS (the stages are
    // free: the last step ended with a barrier). Row group rg uses the rg-th
    // quarter of the stage memory; slice s > 0 writes record s-1 of it.
    constexpr int REC = (2 + 16 * RB::DB) * 64;   // floats per wave record
    float* area = reinterpret_cast<float*>(smem + rg * GROUP);
    if (ks > 0) rb.save_to(area + (ks - 1) * REC);
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int s2 = 1; s2 < KSPLIT; ++s2) rb.merge_from(area + (s2 - 1) * REC);
  }
  rb.template finish<WRITE_L>(O + head, L + (size_t)bh * N);
}

// ---------------------------------------------------------------------------
// Pipelined kernel: 4*KSPLIT waves; wave w is row group w % 4 and key slice
// w / 4 (as in the split kernel), and tiles advance in groups of KSPLIT. Step
// g issues the MFMAs of two different tiles of the wave's slice, QK of its
// tile in group g+1 and PV of its tile in group g-1, while the VALU computes
// the softmax of its tile in group g: none of the step's MFMAs depends on its
// VALU work, so matrix cores and VALU run side by side within one wave, and
// with KSPLIT = 2 a second wave shares each SIMD. K therefore runs two groups
// ahead of V: step g reads K(g+1) and V(g-1), and its DMA fills K(g+2) and
// V(g) into the stages those reads do not touch.
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL, bool WRITE_L, bool FULL, int KSPLIT>
__global__ void __launch_bounds__(256 * KSPLIT)
fa_fwd_pipe_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                   const f16* __restrict__ V, f16* __restrict__ O,
                   float* __restrict__ L, int N, int num_qb, int total, float c) {
  constexpr int TILE = kBC * D * 2;
  constexpr int BLOCKS = TILE / 1024;
  constexpr int WAVES = kRowGroups * KSPLIT;
  constexpr int LOADS = KSPLIT * BLOCKS / WAVES;          // blocks per wave per group
  constexpr int GROUP = KSPLIT * TILE;                    // bytes of one K or V stage
  static_assert(4 * GROUP <= 160 * 1024, "stages exceed the 160 KiB LDS");
  using RB = RowBlock<D, CAUSAL, FULL>;
  static_assert((KSPLIT - 1) * (2 + 16 * RB::DB) * 64 * 4 <= GROUP, "merge area too small");
  __shared__ __attribute__((aligned(1024))) char smem[4 * GROUP];   // [K0 | K1 | V0 | V1]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: SGPR
  const int rg = wave & (kRowGroups - 1);
  const int ks = wave / kRowGroups;

  const int logical = xcd_remap(blockIdx.x, total);
  const int bh = logical / num_qb;
  int qb = logical - bh * num_qb;
  if (CAUSAL) qb = num_qb - 1 - qb;

  const size_t head = (size_t)bh * N * D;
  const int head_bytes = N * D * 2;
  const char* Kh = reinterpret_cast<const char*>(K + head);
  const char* Vh = reinterpret_cast<const char*>(V + head);
  const int q0 = qb * kBR;

  RB rb;
  rb.init(Q + head, head_bytes, lane, q0 + 32 * rg, N, c);

  uint32_t koff[LOADS], voff[LOADS];
  int slot_of[LOADS], blk_of[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int blk = wave * LOADS + i;
    slot_of[i] = blk / BLOCKS;
    blk_of[i] = blk % BLOCKS;
    dma_offsets<D>(blk_of[i], lane, koff[i], voff[i]);
  }
  const int kv_end = CAUSAL ? min(N, q0 + kBR) : N;
  const int n_tiles = (kv_end + kBC - 1) / kBC;
  const int n_groups = (n_tiles + KSPLIT - 1) / KSPLIT;

  const uint32_t lds0 = lds_addr(smem);
  auto issue_k = [&](int g, int stage) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int t = g * KSPLIT + slot_of[i];
      dma_block_or_zero<D, FULL>(Kh, head_bytes, t, t < n_tiles,
                                 lds0 + stage * GROUP + slot_of[i] * TILE + blk_of[i] * 1024,
                                 koff[i]);
    }
  };
  auto issue_v = [&](int g, int stage) {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int t = g * KSPLIT + slot_of[i];
      dma_block_or_zero<D, FULL>(Vh, head_bytes, t, t < n_tiles,
                                 lds0 + (2 + stage) * GROUP + slot_of[i] * TILE + blk_of[i] * 1024,
                                 voff[i]);
    }
  };

  // This wave's tile in group g is g * KSPLIT + ks. A slice whose tile is past
  // the end (last group of an odd tile count) processes it fully masked
  // (P = 0), which keeps the pipeline's shape uniform.
  const int tile_of = ks;   // t = g * KSPLIT + tile_of
  auto mask_tile = [&](int t, f32x16 (&s)[2]) {
    if (t >= n_tiles) {
#pragma unroll
      for (int b = 0; b < 2; ++b) s[b] = f32x16{} - INFINITY;
    } else {
      rb.template mask<2>(t, 0, s);
    }
  };

  // Prologue: K(0), K(1) in, S(0) computed.
  f32x16 s_cur[2];
  issue_k(0, 0);
  if (n_groups > 1) issue_k(1, 1);
  wait_vmem();
  __syncthreads();
  rb.template qk<2>(smem + ks * TILE, 0, s_cur);
  mask_tile(tile_of, s_cur);

  f16x8 pf[4];   // P of the previous group's tile, packed: the B operands of its PV
  auto step = [&](auto par, auto has_prev, auto has_next, int g) {
    constexpr int PAR = decltype(par)::value;          // g & 1
    constexpr bool PREV = decltype(has_prev)::value;   // g >= 1
    constexpr bool NEXT = decltype(has_next)::value;   // g + 1 < n_groups
    if (g + 2 < n_groups) issue_k(g + 2, PAR);         // K(g) was consumed by step g-1
    issue_v(g, PAR);                                   // V(g-2) was consumed by step g-1
    const char* k_next = smem + (1 - PAR) * GROUP + ks * TILE;        // K(g+1)
    const char* v_prev = smem + (2 + (1 - PAR)) * GROUP + ks * TILE;  // V(g-1)
    f32x16 s_nxt[2];
    if constexpr (NEXT) rb.template qk<2>(k_next, 0, s_nxt);
    if constexpr (PREV) rb.template pv<2>(v_prev, 0, pf);
    rb.template softmax_keep<2>(s_cur, pf);
    if constexpr (NEXT) {
      mask_tile((g + 1) * KSPLIT + tile_of, s_nxt);
      s_cur[0] = s_nxt[0];
      s_cur[1] = s_nxt[1];
    }
    wait_vmem();
    __syncthreads();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using BT = std::true_type;
  using BF = std::false_type;
  if (n_groups == 1) {
    step(I0{}, BF{}, BF{}, 0);
  } else {
    step(I0{}, BF{}, BT{}, 0);
    int g = 1;
    for (; g + 2 < n_groups; g += 2) {
      step(I1{}, BT{}, BT{}, g);
      step(I0{}, BT{}, BT{}, g + 1);
    }
    if (n_groups - g == 2) {
      step(I1{}, BT{}, BT{}, g);
      step(I0{}, BT{}, BF{}, g + 1);
    } else {
      step(I1{}, BT{}, BF{}, g);
    }
  }
  // PV of the last group: its V landed in stage (n_groups-1) & 1 in the last step.
  rb.template pv<2>(smem + (2 + ((n_groups - 1) & 1)) * GROUP + ks * TILE, 0, pf);

  if constexpr (KSPLIT > 1) {
    // Merge the key slices of each row group through LDS (see the split kernel).
    __syncthreads();
    constexpr int REC = (2 + 16 * RB::DB) * 64;
    float* area = reinterpret_cast<float*>(smem + rg * GROUP);
    if (ks > 0) rb.save_to(area + (ks - 1) * REC);
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int s2 = 1; s2 < KSPLIT; ++s2) rb.merge_from(area + (s2 - 1) * REC);
  }
  rb.template finish<WRITE_L>(O + head, L + (size_t)bh * N);
}

// Kernel variants: 10*k + s = split kernel with KSPLIT k and s LDS stages;
// 100 + k = pipelined kernel with KSPLIT k.
constexpr int kPipe1 = 101;
constexpr int kPipe2 = 102;

template <int D, bool CAUSAL, bool WRITE_L, bool FULL, int KSPLIT, int STAGES>
static void launch_split(const f16* Q, const f16* K, const f16* V, f16* O, float* L, int N,
                         int num_qb, int total, float c, hipStream_t stream) {
  hipLaunchKernelGGL((fa_fwd_split_kernel<D, CAUSAL, WRITE_L, FULL, KSPLIT, STAGES>), dim3(total),
                     dim3(256 * KSPLIT), 0, stream, Q, K, V, O, L, N, num_qb, total, c);
}

// Variants whose LDS fits: 2 * STAGES * KSPLIT * (64 * D * 2) <= 160 KiB.
static bool variant_fits(int D, int variant) {
  if (variant == kPipe1) return true;
  if (variant == kPipe2) return 4 * 2 * (64 * D * 2) <= 160 * 1024;
  const int ks = variant / 10, st = variant % 10;
  if ((ks != 1 && ks != 2 && ks != 4) || st < 2 || st > 4) return false;
  return 2 * st * ks * (64 * D * 2) <= 160 * 1024;
}

template <int D, bool CAUSAL, bool WRITE_L, bool FULL>
static hipError_t launch_fwd(const void* q, const void* k, const void* v, void* o,
                             float* lse, int N, int num_qb, int total, float c, int variant,
                             hipStream_t stream) {
  const f16* Q = (const f16*)q;
  const f16* K = (const f16*)k;
  const f16* V = (const f16*)v;
  f16* Op = (f16*)o;
  switch (variant) {
    case kPipe1:
      hipLaunchKernelGGL((fa_fwd_pipe_kernel<D, CAUSAL, WRITE_L, FULL, 1>), dim3(total), dim3(256), 0,
                         stream, Q, K, V, Op, lse, N, num_qb, total, c);
      break;
    case kPipe2:
      hipLaunchKernelGGL((fa_fwd_pipe_kernel<D, CAUSAL, WRITE_L, FULL, 2>), dim3(total), dim3(512), 0,
                         stream, Q, K, V, Op, lse, N, num_qb, total, c);
      break;
    case 13: launch_split<D, CAUSAL, WRITE_L, FULL, 1, 3>(Q, K, V, Op, lse, N, num_qb, total, c, stream); break;
    case 14: launch_split<D, CAUSAL, WRITE_L, FULL, 1, 4>(Q, K, V, Op, lse, N, num_qb, total, c, stream); break;
    case 22: launch_split<D, CAUSAL, WRITE_L, FULL, 2, 2>(Q, K, V, Op, lse, N, num_qb, total, c, stream); break;
    case 23:
      if constexpr (D == 64) { launch_split<D, CAUSAL, WRITE_L, FULL, 2, 3>(Q, K, V, Op, lse, N, num_qb, total, c, stream); break; }
      return hipErrorInvalidValue;
    case 24:
      if constexpr (D == 64) { launch_split<D, CAUSAL, WRITE_L, FULL, 2, 4>(Q, K, V, Op, lse, N, num_qb, total, c, stream); break; }
      return hipErrorInvalidValue;
    case 42:
      if constexpr (D == 64) { launch_split<D, CAUSAL, WRITE_L, FULL, 4, 2>(Q, K, V, Op, lse, N, num_qb, total, c, stream); break; }
      return hipErrorInvalidValue;
    default:
      launch_split<D, CAUSAL, WRITE_L, FULL, 1, 2>(Q, K, V, Op, lse, N, num_qb, total, c, stream);
      break;
  }
  return hipGetLastError();
}

template <int D, bool CAUSAL>
static hipError_t dispatch_wl(const void* q, const void* k, const void* v, void* o,
                              float* lse, int N, int num_qb, int total, float c, bool full,
                              int variant, hipStream_t s) {
  if (lse) {
    return full ? launch_fwd<D, CAUSAL, true, true>(q, k, v, o, lse, N, num_qb, total, c, variant, s)
                : launch_fwd<D, CAUSAL, true, false>(q, k, v, o, lse, N, num_qb, total, c, variant, s);
  }
  return full ? launch_fwd<D, CAUSAL, false, true>(q, k, v, o, lse, N, num_qb, total, c, variant, s)
              : launch_fwd<D, CAUSAL, false, false>(q, k, v, o, lse, N, num_qb, total, c, variant, s);
}

// Variant choice (measured on MI355X; see bench.py). The environment
// variable FA_MI355X_FWD_VARIANT ("pipe<k>" or "split<k>s<s>", e.g. split1s4)
// forces one that fits D; it is read once, for measurement and tests.
static int choose_variant(int64_t D) {
  static const int forced = [] {
    const char* e = getenv("FA_MI355X_FWD_VARIANT");
    if (!e) return -1;
    int ks = 0, st = 0;
    if (sscanf(e, "pipe%d", &ks) == 1) return 100 + ks;
    if (sscanf(e, "split%ds%d", &ks, &st) == 2) return 10 * ks + st;
    return -1;
  }();
  if (forced >= 0 && variant_fits((int)D, forced)) return forced;
  // D = 64: four key slices per query block (16 waves per workgroup) keep
  // every SIMD busy even when B*H*N/128 is about one workgroup per CU.
  // D = 128: one slice, double-buffered; the larger tiles already fill it.
  return D == 64 ? 42 : 12;
}

}  // namespace fa

extern "C" int fa_fwd_f16(const void* q, const void* k, const void* v, void* o,
                          float* lse, int64_t B, int64_t H, int64_t N, int64_t D,
                          int causal, void* stream) {
  using namespace fa;
  int st = fa_validate_fwd(q, k, v, o, B, H, N, D);
  if (st != FA_OK) return st;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return FA_ERR_ALIGNMENT;
  const int num_qb = (int)((N + kBR - 1) / kBR);
  const int total = (int)(B * H * num_qb);
  const float c = (float)(1.0 / sqrt((double)D)) * kLog2e;
  const bool full = (N % kBR) == 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int variant = choose_variant(D);
  hipError_t e;
  if (D == 64) {
    e = causal ? dispatch_wl<64, true>(q, k, v, o, lse, (int)N, num_qb, total, c, full, variant, s)
               : dispatch_wl<64, false>(q, k, v, o, lse, (int)N, num_qb, total, c, full, variant, s);
  } else {
    e = causal ? dispatch_wl<128, true>(q, k, v, o, lse, (int)N, num_qb, total, c, full, variant, s)
               : dispatch_wl<128, false>(q, k, v, o, lse, (int)N, num_qb, total, c, full, variant, s);
  }
  return e == hipSuccess ? FA_OK : -(int)e;
}
