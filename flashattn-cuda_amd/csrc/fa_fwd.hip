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
// Three kernels share that per-wave core (RowBlock):
//   * fa_fwd_pp_kernel (the default): two wave groups own the even and odd
//     key tiles of the same rows and alternate, barrier by barrier, between a
//     matrix phase and a softmax phase, so each SIMD runs one wave's MFMAs
//     while the other wave's VALU work issues;
//   * fa_fwd_split_kernel<.., KSPLIT>: 4*KSPLIT waves; the KSPLIT waves of a
//     row group take every KSPLIT-th tile and merge their (m, l, O) through LDS
//     at the end;
//   * fa_fwd_pipe_kernel: one wave per row group, software-pipelined (QK of
//     tile t+1 issued alongside the softmax of tile t).
// A single wave issues VALU work about half as fast as two or more waves
// sharing a SIMD (measured: fp32 fma 2.8 ns vs 1.3-1.5 ns per instruction,
// v_exp_f32 6.7 ns vs 4.0-4.6 ns), which is what all three designs work
// around.
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
template <int D, bool CAUSAL, bool FULL, bool BF16 = false>
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
      for (int b = 0; b < NB; ++b) s[b] = mma32<BF16>(load_k_frag<D>(ks, kb0 + b, kk, lane), qf[kk], s[b]);
    }
  }

  // Key of register r in block kb is key0 + 4 hi + kofs(kb, r) with a
  // compile-time kofs, so each test compares that constant against one
  // per-tile lane limit (no per-register key arrays kept live). Keys >= N and,
  // if CAUSAL, keys > the lane's query row get -inf.
  template <int NB>
  __device__ __forceinline__ void mask_all(int t, int kb0, f32x16 (&s)[NB]) const {
    const int lane_key = t * kBC + 4 * hi;
    int lim = N - 1 - lane_key;                    // live iff kofs <= lim
    if (CAUSAL) lim = min(lim, qrow - lane_key);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (st_key(kb0 + b, r, 0) > lim) s[b][r] = -INFINITY;
      }
    }
  }

  // mask_all for the tiles that need it (the last tile of a ragged N, the
  // tiles crossing the causal diagonal); a wave-uniform branch skips the rest.
  template <int NB>
  __device__ __forceinline__ void mask(int t, int kb0, f32x16 (&s)[NB]) const {
    const int key0 = t * kBC;
    const bool need = (!FULL && key0 + kBC > N) || (CAUSAL && key0 + kBC - 1 > row_w);
    if (need) mask_all<NB>(t, kb0, s);
  }

  // p = 2^(s c - m), rounded to fp16 and packed as the B operands (P^T) of
  // the PV k-steps: two per 32-key block, in S^T register order. Returns this
  // lane's sum of the fp32 values (the normaliser keeps fp32 accuracy even
  // for short rows, where fp16 rounding of P would not average out).
  template <int NB>
  __device__ __forceinline__ float expo_pack(const f32x16 (&s)[NB], f16x8 (&pf)[2 * NB],
                                             float m) const {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f16x2 x[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = 8 * h + 2 * q;
          const float e0 = exp2_hw(fmaf(s[b][r], c, -m));
          const float e1 = exp2_hw(fmaf(s[b][r + 1], c, -m));
          acc[q] += e0 + e1;
          x[q] = cvt2x<BF16>(e0, e1);
        }
        pf[2 * b + h] = f16x8{x[0][0], x[0][1], x[1][0], x[1][1], x[2][0], x[2][1], x[3][0], x[3][1]};
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

  // Slow path of the softmax: some lane's tile sum at the running max left
  // the fp16-safe range (or is not finite: first tile, m_run = -inf). Raise
  // the max to the tile's row max and redo the exponentials.
  template <int NB>
  __device__ __forceinline__ float rescue(const f32x16 (&s)[NB], f16x8 (&pf)[2 * NB]) {
    raise_max<NB>(s);
    return expo_pack<NB>(s, pf, m_safe());
  }

  // Softmax of the blocks into packed P; the scores stay intact for the
  // slow path.
  template <int NB>
  __device__ __forceinline__ void softmax_keep(const f32x16 (&s)[NB], f16x8 (&pf)[2 * NB]) {
    float rs = expo_pack<NB>(s, pf, m_run);
    // Rare: the merge copies of P, O and l go on this edge, not the fast one.
    if (__builtin_expect(!__all(rs <= kSumLimit), 0)) rs = rescue<NB>(s, pf);
    l_run += rs;
  }

  // O^T += V^T P^T over the PV k-steps of the blocks.
  template <int NB>
  __device__ __forceinline__ void pv(const char* vs, int kb0, const f16x8 (&pf)[2 * NB]) {
#pragma unroll
    for (int j = 0; j < 2 * NB; ++j) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
        o[db] = mma32<BF16>(load_v_frag<D>(vs, 2 * kb0 + j, db, lane), pf[j], o[db]);
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
    const float inv = 1.f / l_tot;
    // Lanes l and l^32 hold the two 8-byte halves of each 16-byte chunk
    // (columns 32 db + 8 g .. +7) of the row. One permlane32 swap per
    // register of a chunk pair (g, g+1) gives lane l (hi = 0) all of chunk g
    // and lane l^32 all of chunk g+1, so every lane stores whole 16-byte
    // chunks: half the store instructions, 32 bytes of a row per lane pair.
    uint4 st[DB][2];
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        uint32_t w[2][2];   // [chunk g0 or g0+1][register]
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int g = 2 * gp + j;
          const f16x2 a = cvt2x<BF16>(o[db][4 * g + 0] * inv, o[db][4 * g + 1] * inv);
          const f16x2 b = cvt2x<BF16>(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
          w[j][0] = __builtin_bit_cast(uint32_t, a);
          w[j][1] = __builtin_bit_cast(uint32_t, b);
        }
        const auto r0 = __builtin_amdgcn_permlane32_swap(w[0][0], w[1][0], false, false);
        const auto r1 = __builtin_amdgcn_permlane32_swap(w[0][1], w[1][1], false, false);
        st[db][gp] = uint4{r0[0], r1[0], r0[1], r1[1]};
      }
    }
    if (FULL || qrow < N) {
      f16* orow = Oh + (size_t)qrow * D;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int gp = 0; gp < 2; ++gp)
          *reinterpret_cast<uint4*>(orow + 32 * db + 8 * (2 * gp + hi)) = st[db][gp];
      }
      if (WRITE_L && hi == 0) Lh[qrow] = (m_run + log2_hw(l_tot)) * kLn2;
    }
  }

  // finish<WRITE_L> with O staged through this wave's `stage` LDS area (at
  // least 32 rows of STAGE_STRIDE bytes, written and read only by this wave):
  // each lane writes its 16-byte chunks, then 8 lanes store one 128-byte
  // (D = 64) or two (D = 128) rows, so a store instruction covers whole rows
  // instead of 32-byte pieces of 32 rows.
  static constexpr int STAGE_STRIDE = 2 * D + 16;   // padded: spreads the LDS banks
  template <bool WRITE_L>
  __device__ __forceinline__ void finish_staged(f16* Oh, float* Lh, char* stage) const {
    const float l_tot = sum_xor32(l_run);
    const float inv = 1.f / l_tot;
    constexpr int CPR = D / 8;                       // 16-byte chunks per row
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        uint32_t w[2][2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int g = 2 * gp + j;
          const f16x2 a = cvt2x<BF16>(o[db][4 * g + 0] * inv, o[db][4 * g + 1] * inv);
          const f16x2 b = cvt2x<BF16>(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv);
          w[j][0] = __builtin_bit_cast(uint32_t, a);
          w[j][1] = __builtin_bit_cast(uint32_t, b);
        }
        const auto r0 = __builtin_amdgcn_permlane32_swap(w[0][0], w[1][0], false, false);
        const auto r1 = __builtin_amdgcn_permlane32_swap(w[0][1], w[1][1], false, false);
        const int chunk = 4 * db + 2 * gp + hi;      // 16-byte chunk of the row
        *reinterpret_cast<uint4*>(stage + (lane & 31) * STAGE_STRIDE + chunk * 16) =
            uint4{r0[0], r1[0], r0[1], r1[1]};
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's LDS writes landed
#pragma unroll
    for (int k = 0; k < 32 * CPR / 64; ++k) {
      const int idx = 64 * k + lane;
      const int r = idx / CPR, ch = idx % CPR;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + r * STAGE_STRIDE + ch * 16);
      if (FULL || row_w + r < N)
        *reinterpret_cast<uint4*>(Oh + (size_t)(row_w + r) * D + ch * 8) = v;
    }
    if (WRITE_L && hi == 0 && (FULL || qrow < N)) Lh[qrow] = (m_run + log2_hw(l_tot)) * kLn2;
  }

  // Split-KV epilogue: this row's fp32 O normalised over the keys of one
  // split and the natural-log LSE of those keys, at partial index `at` of a
  // row-major [rows, splits] layout. A row that saw no key gets O = 0 and
  // LSE = -inf (weight 0 in the combine).
  __device__ __forceinline__ void finish_partial(float* part_o, float* part_lse, size_t at) const {
    const float l_tot = sum_xor32(l_run);
    if (FULL || qrow < N) {
      const bool empty = l_tot == 0.f;
      const float inv = empty ? 0.f : 1.f / l_tot;
      float* orow = part_o + at * D;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 v4 = f32x4{o[db][4 * g + 0] * inv, o[db][4 * g + 1] * inv,
                                 o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv};
          *reinterpret_cast<f32x4*>(orow + 32 * db + 8 * g + 4 * hi) = v4;
        }
      }
      if (hi == 0) part_lse[at] = empty ? -INFINITY : (m_run + log2_hw(l_tot)) * kLn2;
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
                    float* __restrict__ L, Geom geo, int num_qb, int total, float c) {
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

  const HeadView hv = head_view<D>(geo, bh);
  const int N = hv.n;
  if (qb * kBR >= N) return;   // varlen: past this sequence (whole workgroup)
  const size_t head = hv.q;
  const int head_bytes = N * D * 2;
  const char* Kh = reinterpret_cast<const char*>(K + hv.kv);
  const char* Vh = reinterpret_cast<const char*>(V + hv.kv);
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
  rb.template finish<WRITE_L>(O + head, L + hv.l);
}


// ---------------------------------------------------------------------------
// Pipelined kernel: 4*KSPLIT waves; wave w is row group w % 4 and key slice
// w / 4 (as in the split kernel), and tiles advance in groups of KSPLIT.
//
// Step g issues the MFMAs of two other tiles of the wave's slice, QK of its
// tile in group g+1 and PV of its tile in group g-1, while the VALU computes
// the softmax of its tile in group g. None of the step's MFMAs depends on its
// VALU work, so the step is written as a fixed schedule of chunks, each one
// MFMA + the LDS reads of the MFMA PF places later + a slice of the softmax,
// fenced by sched_barrier: the matrix core runs while the same wave computes
// exponentials, and a 64-key step costs about max(MFMA, VALU), not the sum.
//
// K and V tiles go through rings of RING LDS slots each; K(x) and V(x) live
// in slot x % RING. Step g reads K(g+1) and V(g-1). MID_BACK MFMAs before its
// end, once all its reads are done, the step waits for its own copies of
// K(g+2) and V(g), meets the other waves at the barrier, issues the copies of
// K(g+1+RING) (into the slot of K(g+1)) and V(g+RING-1) (slot of V(g-1)), and
// reads the first operands of step g+1, so the next step starts with its
// operands in registers and each copy has about RING-1 steps to land. Copies
// of tiles past the end are still issued, with an empty buffer range (they
// write zeros and read nothing), so every wave issues the same number per
// step and the vmcnt waits are exact.
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL, bool WRITE_L, bool FULL, int KSPLIT, int RING>
__global__ void __launch_bounds__(256 * KSPLIT)
fa_fwd_pipe_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                   const f16* __restrict__ V, f16* __restrict__ O,
                   float* __restrict__ L, Geom geo, int num_qb, int total, float c) {
  constexpr int TILE = kBC * D * 2;
  constexpr int BLOCKS = TILE / 1024;
  constexpr int WAVES = kRowGroups * KSPLIT;
  constexpr int LOADS = KSPLIT * BLOCKS / WAVES;          // blocks per wave per group (K or V)
  constexpr int GROUP = KSPLIT * TILE;                    // bytes of one K or V slot
  constexpr int PER_STEP = 2 * LOADS;                     // copies per wave per step
  static_assert(RING >= 2 && RING <= 4, "two to four slots");
  static_assert(2 * RING * GROUP <= 160 * 1024, "slots exceed the 160 KiB LDS");
  using RB = RowBlock<D, CAUSAL, FULL>;
  static_assert((KSPLIT - 1) * (2 + 16 * RB::DB) * 64 * 4 <= GROUP, "merge area too small");
  constexpr int DB = RB::DB;
  constexpr int NMM = D / 8;     // MFMAs of QK (2 blocks x D/16 k-steps) = of PV (4 x DB)
  constexpr int PF = D == 64 ? 8 : 4;   // operand prefetch distance, in MFMAs
  constexpr int MID_BACK = 2;    // the step barrier sits this many MFMAs before the end
  constexpr int NSLOT = 17;      // softmax slots of a step (16 value pairs, pipelined)
  // Step 0's PF first operands are all of its own; every read of a step is
  // issued before its barrier.
  static_assert(PF <= NMM && MID_BACK >= 1 && MID_BACK <= PF, "bad step schedule");
  // K slots at [0, RING) * GROUP, V slots at [RING, 2 RING) * GROUP.
  __shared__ __attribute__((aligned(1024))) char smem[2 * RING * GROUP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: SGPR
  const int rg = wave & (kRowGroups - 1);
  const int ks = wave / kRowGroups;

  const int logical = xcd_remap(blockIdx.x, total);
  const int bh = logical / num_qb;
  int qb = logical - bh * num_qb;
  if (CAUSAL) qb = num_qb - 1 - qb;

  const HeadView hv = head_view<D>(geo, bh);
  const int N = hv.n;
  if (qb * kBR >= N) return;   // varlen: past this sequence (whole workgroup)
  const size_t head = hv.q;
  const int head_bytes = N * D * 2;
  const char* Kh = reinterpret_cast<const char*>(K + hv.kv);
  const char* Vh = reinterpret_cast<const char*>(V + hv.kv);
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
  // Per-lane offsets of the operand fragments within a tile.
  int koffs[D / 16], voffs[DB];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) koffs[kk] = k_frag_off<D>(kk, lane);
#pragma unroll
  for (int db = 0; db < DB; ++db) voffs[db] = v_frag_off<D>(db, lane);

  const int kv_end = CAUSAL ? min(N, q0 + kBR) : N;
  const int n_tiles = (kv_end + kBC - 1) / kBC;
  const int n_groups = (n_tiles + KSPLIT - 1) / KSPLIT;
  // Groups [0, g_full) hold no key >= N and, if CAUSAL, no key above the
  // workgroup's first row: their scores need no mask.
  const int lim = CAUSAL ? min(N, q0 + 1) : N;
  const int g_full = lim / (KSPLIT * kBC);

  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int x, int base_slot) {   // K(x) (base_slot 0) or V(x) (base_slot RING)
    const char* src = base_slot == 0 ? Kh : Vh;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int t = x * KSPLIT + slot_of[i];
      const uint32_t at = lds0 + (base_slot + x % RING) * GROUP + slot_of[i] * TILE + blk_of[i] * 1024;
      dma_block_or_zero<D, FULL>(src, head_bytes, t, t < n_tiles, at,
                                 base_slot == 0 ? koff[i] : voff[i]);
    }
  };
  auto k_base = [&](int x) -> const char* { return smem + (x % RING) * GROUP + ks * TILE; };
  auto v_base = [&](int x) -> const char* { return smem + (RING + x % RING) * GROUP + ks * TILE; };
  // Per-lane bases of the operand reads from K(x) and V(y).
  struct Bases {
    lds_cp k[D / 16];
    lds_cp v[DB];
  };
  auto bases = [&](int x, int y) {
    Bases r;
    // Slot bases as scalars (opaque, so no per-lane share of the slot
    // arithmetic is folded into the lane offsets).
    uint32_t kt = lds0 + (x % RING) * GROUP + ks * TILE;
    uint32_t vt = lds0 + (RING + y % RING) * GROUP + ks * TILE;
    asm("" : "+s"(kt), "+s"(vt));
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) r.k[kk] = lds_lane_base(kt + koffs[kk]);
#pragma unroll
    for (int db = 0; db < DB; ++db) r.v[db] = lds_lane_base(vt + voffs[db]);
    return r;
  };

  // Operand of MFMA m of a step. Steps with a PV alternate (even m: QK i =
  // m/2, odd m: PV i = m/2); the first step has QK only. QK i: block i % 2,
  // k-step i / 2. PV i: k-step i / DB, d-block i % DB. Consecutive MFMAs on
  // one accumulator are four (two) MFMAs apart.
  auto fetch = [&](auto prev, int m, const Bases& bs) -> f16x8 {
    constexpr bool PREV = decltype(prev)::value;
    const int i = PREV ? m >> 1 : m;
    if (!PREV || (m & 1) == 0) return lds_b128(bs.k[i / 2] + (i % 2) * 32 * 2 * D);
    return v_frag_lds<D>(bs.v[i % DB] + (i / DB) * 16 * 2 * D);
  };

  // Prologue: K(0 .. RING-1) and V(0 .. RING-3) in flight; K(0), K(1) landed.
#pragma unroll
  for (int x = 0; x < RING; ++x) issue(x, 0);
#pragma unroll
  for (int x = 0; x < RING - 2; ++x) issue(x, RING);
  wait_vmcnt<(RING - 2) * PER_STEP>();
  __syncthreads();

  f32x16 sA[2], sB[2];   // scores of the tile being softmaxed / being computed
  f16x8 pA[4], pB[4];    // packed P of the tile whose PV is pending / being made
  f16x8 a[PF];           // operands of the next step's first PF MFMAs
  rb.template qk<2>(k_base(0), 0, sA);
  __syncthreads();       // K(0) read by every wave: its slot is refilled next
  issue(RING, 0);        // step 0's copies: K(RING), V(RING-2)
  issue(RING - 2, RING);
  using BT = std::true_type;
  using BF = std::false_type;
  Bases nb = bases(1, RING - 1);   // bases of the next step (V unused in step 0)
#pragma unroll
  for (int i = 0; i < PF; ++i) a[i] = fetch(BF{}, i, nb);

  // One step. cur: S(g); nxt: S(g+1) out; pin: P(g-1); pout: P(g) out.
  auto step = [&](auto prev, auto masked, int g, f32x16 (&cur)[2], f32x16 (&nxt)[2],
                  const f16x8 (&pin)[4], f16x8 (&pout)[4]) {
    constexpr bool PREV = decltype(prev)::value;       // g >= 1
    constexpr bool MASKED = decltype(masked)::value;   // group g may need a mask
    constexpr int NM = PREV ? 2 * NMM : NMM;
    constexpr int MID = NM - MID_BACK;
    // Bases of K(g+1) (zeros past the end: harmless, unused) and V(g-1),
    // computed by the previous step.
    const Bases bs = nb;
    f16x8 op[NM];
#pragma unroll
    for (int m = 0; m < PF; ++m) op[m] = a[m];
#pragma unroll
    for (int b = 0; b < 2; ++b) nxt[b] = f32x16{};
    if constexpr (MASKED) rb.template mask_all<2>(g * KSPLIT + ks, 0, cur);
    const float m_cur = rb.m_run;
    float acc[2];
    float ex[16][2];
    // Softmax slot u: exponentials of value pair u (u < 16), then the fp16
    // pack and row-sum of pair u-1 (u >= 1), a slot after its exponentials.
    auto slot = [&](auto ui) {
      constexpr int u = decltype(ui)::value;
      if constexpr (u < 16) {
        constexpr int b = u / 8, r = 2 * (u % 8);
        ex[u][0] = exp2_hw(fmaf(cur[b][r], c, -m_cur));
        ex[u][1] = exp2_hw(fmaf(cur[b][r + 1], c, -m_cur));
      }
      if constexpr (u >= 1) {
        constexpr int p = u - 1, b = p / 8, h = (p % 8) / 4, q = p % 4;
        f16x2 x = cvt2(ex[p][0], ex[p][1]);
        // Pin the conversion to this chunk (the slow path also writes P, and
        // the compiler would otherwise sink it below the branch).
        asm volatile("" : "+v"(x));
        if constexpr (p < 2) {
          acc[p] = ex[p][0] + ex[p][1];
        } else {
          acc[p & 1] += ex[p][0] + ex[p][1];
        }
        pout[2 * b + h][2 * q] = x[0];
        pout[2 * b + h][2 * q + 1] = x[1];
      }
    };
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NM>([&](auto mi) {
      constexpr int m = decltype(mi)::value;
      if constexpr (m + PF < NM) op[m + PF] = fetch(prev, m + PF, bs);
      if constexpr (m == MID) {
        // Every LDS read of this step is issued (the barrier waits for them).
        wait_vmcnt<(RING - 2) * PER_STEP>();
        __syncthreads();
        issue(g + 1 + RING, 0);
        issue(g + RING - 1, RING);
        nb = bases(g + 2, g);
#pragma unroll
        for (int i = 0; i < PF; ++i) a[i] = fetch(BT{}, i, nb);
      }
      if constexpr (PREV) {
        constexpr int i = m >> 1;
        if constexpr ((m & 1) == 0) {
          nxt[i % 2] = mfma32(op[m], rb.qf[i / 2], nxt[i % 2]);
        } else {
          rb.o[i % DB] = mfma32(op[m], pin[i / DB], rb.o[i % DB]);
        }
      } else {
        nxt[m % 2] = mfma32(op[m], rb.qf[m / 2], nxt[m % 2]);
      }
      static_for<m * NSLOT / NM, (m + 1) * NSLOT / NM>(slot);
      __builtin_amdgcn_sched_barrier(0);
    });
    float rs = acc[0] + acc[1];
    // Rare: copies for the merge of O and P go on this edge, not the fast one.
    if (__builtin_expect(!__all(rs <= kSumLimit), 0)) rs = rb.template rescue<2>(cur, pout);
    rb.l_run += rs;
  };

  // Step 0 (no PV yet; always masked: cheap, and covers g_full == 0).
  // Odd steps then read sB / pA and write sA / pB, even steps the reverse.
  step(BF{}, BT{}, 0, sA, sB, pB, pA);
  int g = 1;
  for (; g + 1 < g_full; g += 2) {
    step(BT{}, BF{}, g, sB, sA, pA, pB);
    step(BT{}, BF{}, g + 1, sA, sB, pB, pA);
  }
  if (g < g_full) {
    step(BT{}, BF{}, g, sB, sA, pA, pB);
    ++g;
  }
  if ((g & 1) == 0 && g < n_groups) {
    step(BT{}, BT{}, g, sA, sB, pB, pA);
    ++g;
  }
  for (; g + 1 < n_groups; g += 2) {
    step(BT{}, BT{}, g, sB, sA, pA, pB);
    step(BT{}, BT{}, g + 1, sA, sB, pB, pA);
  }
  if (g < n_groups) step(BT{}, BT{}, g, sB, sA, pA, pB);

  // PV of the last group: V(n_groups-1) landed before the last step's
  // barrier; its P is in pB if n_groups-1 is odd, else in pA.
  {
    const bool odd = ((n_groups - 1) & 1) != 0;
    f16x8 pl[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) pl[j] = odd ? pB[j] : pA[j];
    rb.template pv<2>(v_base(n_groups - 1), 0, pl);
  }
  wait_vmem();   // the last steps' copies (all of empty ranges) have drained

  if constexpr (KSPLIT > 1) {
    // Merge the key slices of each row group through LDS (see the split kernel).
    __syncthreads();
    constexpr int REC = (2 + 16 * DB) * 64;
    float* area = reinterpret_cast<float*>(smem + rg * GROUP);
    if (ks > 0) rb.save_to(area + (ks - 1) * REC);
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int s2 = 1; s2 < KSPLIT; ++s2) rb.merge_from(area + (s2 - 1) * REC);
  }
  rb.template finish<WRITE_L>(O + head, L + hv.l);
}

// ---------------------------------------------------------------------------
// Ping-pong kernel: 8 waves. Wave w is row group w % 4 and group w / 4;
// group 0 owns the even key tiles and group 1 the odd ones, so waves w and
// w + 4 (one per group) share a SIMD and the same 32 query rows. Time runs
// in barrier-separated phases, and in every phase one group issues matrix
// work (its "M" phase: PV of its current tile and QK of its next one) while
// the other runs the softmax of its current tile on the VALU ("S" phase):
//
//   phase      2j                       2j+1
//   group 0    S(tile 2j)               M(PV tile 2j, QK tile 2j+2)
//   group 1    M(PV 2j-1, QK 2j+1)      S(tile 2j+1)
//
// The two waves of a SIMD then need different pipes at the same time, so
// the matrix core and the VALU overlap across waves even though the
// hardware issues oldest-wave-first; two waves of the same phase kind would
// run nearly one after the other. Each wave holds one score tile and one
// packed P tile, and each group runs its own copy of the loop (the same
// number of barriers), so neither is merged between groups.
//
// K and V tiles go through rings of RING slots (tile x in slot x % RING).
// The copies are issued by the waves in their M phase, between their MFMAs
// (their issue slots are idle while the matrix core runs): in phase 2j
// group 1 copies K tile 2j+RING-1 and V tile 2j+RING-3, in phase 2j+1 group
// 0 copies K tile 2j+RING and V tile 2j+RING-2, each into the slot of a tile
// read in step j-1; both are read RING-2 phases later. A wave waits for its
// copies at the end of the S phase just before that, so each copy has about
// RING/2 - 1 steps to land. Tiles past the end are copied with an empty
// buffer range (zeros).
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL, bool WRITE_L, bool FULL, int RING, bool BF16 = false, int TG = 2,
          int SUB = 1, bool SPLITKV = false>
__global__ void __launch_bounds__(256 * TG)
fa_fwd_pp_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                 const f16* __restrict__ V, f16* __restrict__ O,
                 float* __restrict__ L, Geom geo, int num_qb, int total, float c,
                 float* __restrict__ part_o = nullptr, float* __restrict__ part_lse = nullptr,
                 int nsplit = 1) {
  // The unit of the ring and of a phase is a tile of SUB * 64 keys: SUB
  // consecutive 64-key key tiles ("sub-tiles", the unit of masking and of the
  // copies' bounds), NB 32-key blocks.
  constexpr int TPS = TG;                      // tiles per step (one per group)
  constexpr int WAVES = kRowGroups * TG;
  static_assert(TG == 2 || TG == 4, "two or four tile groups");
  static_assert(SUB == 1 || SUB == 2, "tiles of 64 or 128 keys");
  static_assert(RING % TPS == 0 && RING >= 2 * TPS, "a ring of whole steps, two at least");
  constexpr int NB = 2 * SUB;                  // 32-key blocks per tile
  constexpr int STILE = kBC * D * 2;           // bytes of a 64-key sub-tile
  constexpr int TILE = SUB * STILE;
  constexpr int SBLOCKS = STILE / 1024;        // 1 KiB blocks per sub-tile
  constexpr int BLOCKS = TILE / 1024;          // 1 KiB blocks per tile
  constexpr int LOADS = BLOCKS / 4;            // blocks per M-phase wave per tile
  static_assert(2 * RING * TILE <= 160 * 1024, "slots exceed the 160 KiB LDS");
  using RB = RowBlock<D, CAUSAL, FULL, BF16>;
  constexpr int DB = RB::DB;
  constexpr int KSTEPS = D / 16;
  constexpr int NMM = NB * KSTEPS;             // MFMAs of one QK (= of one PV)
  constexpr int PF = (D == 64 && TG == 2) ? 8 : 4;   // operand prefetch distance, in MFMAs
  // With four groups the M phase runs its PV before its QK, so the scores
  // can take the registers of P (four waves per SIMD have 128 VGPRs each).
  constexpr bool SEQ = TG == 4;
  constexpr int REC = (2 + 16 * DB) * 64;      // floats per wave record of the merge
  static_assert((TG - 1) * kRowGroups * REC * 4 <= 2 * RING * TILE, "merge area too small");
  // K slots at [0, RING) * TILE, V slots at [RING, 2 RING) * TILE.
  __shared__ __attribute__((aligned(1024))) char smem[2 * RING * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: SGPR
  const int rg = wave & (kRowGroups - 1);
  const int grp = wave >> 2;
  const int team = grp / (TG / 2);   // team 0 starts in the S phase
  // Tile of group g in step j.
  auto tile_of = [&](int g, int j) { return TPS * j + g; };

  const int logical = xcd_remap(blockIdx.x, total);
  // Split-KV: the splits of one q-block are adjacent (same XCD, same K/V).
  const int split = SPLITKV ? logical % nsplit : 0;
  const int unit = SPLITKV ? logical / nsplit : logical;
  const int bh = unit / num_qb;
  int qb = unit - bh * num_qb;
  if (CAUSAL) qb = num_qb - 1 - qb;   // longest rows dispatch first

  const HeadView hv = head_view<D>(geo, bh);
  const int N = hv.n;
  if (qb * kBR >= N) return;   // varlen: past this sequence (whole workgroup)
  const size_t head = hv.q;
  const int head_bytes = N * D * 2;
  const int q0 = qb * kBR;

  RB rb;
  rb.init(Q + head, head_bytes, lane, q0 + 32 * rg, N, c);

  const int kv_end = CAUSAL ? min(N, q0 + kBR) : N;
  int n_sub = (kv_end + kBC - 1) / kBC;          // 64-key sub-tiles
  int n_tiles = (n_sub + SUB - 1) / SUB;
  // Split-KV: this workgroup's tiles are tb .. tb + n_tiles - 1 of the row
  // block's; K/V pointers and bounds start at tile tb, masking uses absolute
  // key positions (sub-tile offset tbs).
  int tb = 0;
  if constexpr (SPLITKV) {
    const int per = (n_tiles + nsplit - 1) / nsplit;
    tb = min(split * per, n_tiles);
    n_tiles = min(per, n_tiles - tb);
    n_sub = min(n_sub - tb * SUB, n_tiles * SUB);
    if (n_tiles == 0) {   // nothing for this split: an empty partial for every row
      if (grp == 0) rb.finish_partial(part_o, part_lse, (hv.l + rb.qrow) * nsplit + split);
      return;
    }
  }
  const int tbs = SPLITKV ? tb * SUB : 0;
  const int kv_bytes = head_bytes - tbs * (kBC * D * 2);
  const char* Kh = reinterpret_cast<const char*>(K + hv.kv) + (size_t)tbs * (kBC * D * 2);
  const char* Vh = reinterpret_cast<const char*>(V + hv.kv) + (size_t)tbs * (kBC * D * 2);
  const int n_steps = (n_tiles + TPS - 1) / TPS;   // tiles per group

  const uint32_t lds0 = lds_addr(smem);
  // This wave's share of a tile copy in its M phase: blocks rg*LOADS .. +LOADS.
  uint32_t koff[LOADS], voff[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) dma_offsets<D>((rg * LOADS + i) % SBLOCKS, lane, koff[i], voff[i]);
  // 1 KiB block b of tile t: sub-tile SUB t + b / SBLOCKS, bounded by its own
  // buffer range (zeros past the end).
  auto dma_tile_block = [&](bool is_v, int t, int b, uint32_t dst, uint32_t off) {
    int st = SUB * t + b / SBLOCKS;
    const char* src = is_v ? Vh : Kh;
    if constexpr (SUB > 1) {
      // wave-uniform, but the compiler loses track of it here: keep the
      // buffer descriptor in SGPRs explicitly
      st = __builtin_amdgcn_readfirstlane(st);
      const uintptr_t a = reinterpret_cast<uintptr_t>(src);
      const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
      const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
      src = reinterpret_cast<const char*>(((uintptr_t)hi << 32) | lo);
    }
    dma_block_or_zero<D, FULL>(src, kv_bytes, st, st < n_sub, dst, off);
  };
  // With four groups the per-lane offsets are recomputed where they are used
  // (from a lane id the compiler cannot hoist) instead of held in registers.
  auto lane_now = [&] {
    int l = lane;
    if constexpr (TG == 4) asm volatile("" : "+v"(l));
    return l;
  };
  auto copy_block = [&](bool is_v, int t, int i) {
    const uint32_t at = lds0 + ((is_v ? RING : 0) + t % RING) * TILE + (rg * LOADS + i) * 1024;
    uint32_t off = is_v ? voff[i] : koff[i];
    if constexpr (TG == 4) {
      uint32_t ko, vo;
      dma_offsets<D>((rg * LOADS + i) % SBLOCKS, lane_now(), ko, vo);
      off = is_v ? vo : ko;
    }
    dma_tile_block(is_v, t, rg * LOADS + i, at, off);
  };

  // Per-lane offsets of the operand fragments within a tile.
  int koffs[KSTEPS], voffs[DB];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) koffs[kk] = k_frag_off<D>(kk, lane);
#pragma unroll
  for (int db = 0; db < DB; ++db) voffs[db] = v_frag_off<D>(db, lane);

  // Prologue: the waves share the copies of K tiles 0 .. RING-TPS/2-1 and V
  // tiles 0 .. RING-3 TPS/2-1 (those read before the first M-phase copies
  // land), 1 KiB block by block.
  {
    constexpr int NK = RING - TPS / 2, NV = RING - 3 * TPS / 2;
    constexpr int ITEMS = (NK + NV) * BLOCKS;
#pragma unroll
    for (int it0 = 0; it0 < ITEMS; it0 += WAVES) {
      const int it = it0 + wave;
      if (ITEMS % WAVES == 0 || it < ITEMS) {
        const bool is_v = it >= NK * BLOCKS;
        const int x = (is_v ? it - NK * BLOCKS : it) / BLOCKS;
        const int blk = it % BLOCKS;
        uint32_t ko, vo;
        dma_offsets<D>(blk % SBLOCKS, lane, ko, vo);
        dma_tile_block(is_v, x, blk, lds0 + ((is_v ? RING : 0) + x) * TILE + blk * 1024,
                       is_v ? vo : ko);
      }
    }
  }
  wait_vmem();
  __syncthreads();

  f32x16 s[NB];       // scores of this wave's current tile
  f16x8 p[2 * NB];     // its packed P (one per PV k-step)
  // The two blocks of sub-tile u.
  auto sub_s = [&](int u) -> f32x16(&)[2] { return *reinterpret_cast<f32x16(*)[2]>(&s[2 * u]); };

  using BT = std::true_type;
  using BF = std::false_type;

  // M phase: PV of tile tv (P in p; skipped without PV) and QK of tile tq
  // into s, alternating, with the operand reads PF MFMAs ahead; between
  // them, this wave's share of the copies of K tile ck and V tile cv.
  auto mphase = [&](auto with_pv, int tq, int tv, int ck, int cv) {
    constexpr bool PV = decltype(with_pv)::value;
    constexpr int NM = PV ? 2 * NMM : NMM;
    constexpr int NC = 2 * LOADS;              // copies of this phase
    uint32_t kt = lds0 + (tq % RING) * TILE;
    uint32_t vt = lds0 + (RING + tv % RING) * TILE;
    asm("" : "+s"(kt), "+s"(vt));
    lds_cp kl[KSTEPS], vl[DB];
    const int ln = lane_now();
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
      kl[kk] = lds_lane_base(kt + (TG == 4 ? k_frag_off<D>(kk, ln) : koffs[kk]));
#pragma unroll
    for (int db = 0; db < DB; ++db)
      vl[db] = lds_lane_base(vt + (TG == 4 ? v_frag_off<D>(db, ln) : voffs[db]));
    // MFMA m is PV i or QK i: with PV and interleaved, even m = PV m / 2 and
    // odd m = QK m / 2; with PV and SEQ, m < NMM = PV m, else QK m - NMM;
    // without PV, QK m. QK i: block i % NB, k-step i / NB. PV i: k-step
    // i / DB, d-block i % DB.
    auto is_pv = [](int m) { return PV && (SEQ ? m < NMM : (m & 1) == 0); };
    auto idx = [](int m) { return !PV ? m : (SEQ ? (m < NMM ? m : m - NMM) : m >> 1); };
    auto fetch = [&](int m) -> f16x8 {
      const int i = idx(m);
      if (is_pv(m)) return v_frag_lds<D>(vl[i % DB] + (i / DB) * 16 * 2 * D);
      return lds_b128(kl[i / NB] + (i % NB) * 32 * 2 * D);
    };
    f16x8 op[NM];
#pragma unroll
    for (int m = 0; m < PF; ++m) op[m] = fetch(m);
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NM>([&](auto mi) {
      constexpr int m = decltype(mi)::value;
      if constexpr (m + PF < NM) op[m + PF] = fetch(m + PF);
      constexpr int i = idx(m);
      if constexpr (is_pv(m)) {
        rb.o[i % DB] = mma32<BF16>(op[m], p[i / DB], rb.o[i % DB]);
      } else if constexpr (i < NB) {
        s[i % NB] = mma32<BF16>(op[m], rb.qf[i / NB], f32x16{});   // first k-step
      } else {
        s[i % NB] = mma32<BF16>(op[m], rb.qf[i / NB], s[i % NB]);
      }
      // Copy c of this phase after MFMA (c + 1) * NM / (NC + 1).
      static_for<0, NC>([&](auto ci) {
        constexpr int cc = decltype(ci)::value;
        if constexpr ((cc + 1) * NM / (NC + 1) == m) copy_block(cc >= LOADS, cc >= LOADS ? cv : ck, cc % LOADS);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // S phase: softmax of tile t (scores in s) into p, the exponentials of a
  // value pair consumed two pairs later.
  auto sphase = [&](int t) {
    if ((TG * SUB > 2 || SPLITKV) && t >= n_tiles) {
      // A group's last tile can lie past the end: no keys, P = 0. (With two
      // groups and no split, such a tile is past N and masked anyway; past a
      // split's end its keys belong to the next split.)
#pragma unroll
      for (int j = 0; j < 2 * NB; ++j) p[j] = f16x8{};
      wait_vmcnt<(RING / TPS - 2) * 2 * LOADS>();
      return;
    }
#pragma unroll
    for (int u = 0; u < SUB; ++u) rb.template mask<2>(tbs + SUB * t + u, 0, sub_s(u));
    const float m_cur = rb.m_run;
    constexpr int PAIRS = 8 * NB;
    float ex[PAIRS][2];
    float acc[2];
    auto slot = [&](auto ui) {
      constexpr int u = decltype(ui)::value;
      if constexpr (u < PAIRS) {
        constexpr int b = u / 8, r = 2 * (u % 8);
        ex[u][0] = exp2_hw(fmaf(s[b][r], c, -m_cur));
        ex[u][1] = exp2_hw(fmaf(s[b][r + 1], c, -m_cur));
      }
      if constexpr (u >= 2) {
        constexpr int q2 = u - 2, b = q2 / 8, h = (q2 % 8) / 4, q = q2 % 4;
        const f16x2 x = cvt2x<BF16>(ex[q2][0], ex[q2][1]);
        if constexpr (q2 < 2) {
          acc[q2] = ex[q2][0] + ex[q2][1];
        } else {
          acc[q2 & 1] += ex[q2][0] + ex[q2][1];
        }
        p[2 * b + h][2 * q] = x[0];
        p[2 * b + h][2 * q + 1] = x[1];
      }
    };
    static_for<0, PAIRS + 2>(slot);
    float rs = acc[0] + acc[1];
    if (__builtin_expect(!__all(rs <= kSumLimit), 0)) rs = rb.template rescue<NB>(s, p);
    rb.l_run += rs;
    // This wave's copies of its M phase RING/2 - 1 phases of its own back;
    // those of the later M phases stay in flight.
    wait_vmcnt<(RING / TPS - 2) * 2 * LOADS>();
  };

  // A phase's register-only work must stay between its barriers: the compiler
  // may otherwise move a softmax across the barrier into the other group's
  // matrix phase. The empty volatile asm ties the scores to a point after the
  // barrier and P to a point before the next one.
  auto pin_s = [&] {
#pragma unroll
    for (int b = 0; b < NB; ++b) asm volatile("" : "+v"(s[b]));
  };
  auto pin_p = [&] {
#pragma unroll
    for (int j = 0; j < 2 * NB; ++j) asm volatile("" : "+v"(p[j]));
  };
  // M phase copies: K and V of the tiles RING - TPS after the ones it reads.
  auto mstep = [&](auto with_pv, int tq, int tv) {
    mphase(with_pv, tq, tv, tq + RING - TPS, tv + RING - TPS);
  };
  if (team == 0) {
    rb.template qk<NB>(smem + (tile_of(grp, 0) % RING) * TILE, 0, s);
    __syncthreads();                 // its slot is refilled in phase 1
    for (int j = 0; j < n_steps; ++j) {
      pin_s();
      sphase(tile_of(grp, j));
      pin_p();
      __syncthreads();
      mstep(BT{}, tile_of(grp, j + 1), tile_of(grp, j));
      __syncthreads();
    }
    __syncthreads();   // team 1's last PV
  } else {
    __syncthreads();
    // Step 0 (no PV yet) is peeled: with both M-phase forms in one loop body
    // the compiler moved the accumulators between them on every step.
    mstep(BF{}, tile_of(grp, 0), tile_of(grp, -1));
    __syncthreads();
    pin_s();
    sphase(tile_of(grp, 0));
    pin_p();
    __syncthreads();
    for (int j = 1; j < n_steps; ++j) {
      mstep(BT{}, tile_of(grp, j), tile_of(grp, j - 1));
      __syncthreads();
      pin_s();
      sphase(tile_of(grp, j));
      pin_p();
      __syncthreads();
    }
    // Phase 2n: the last PV.
    rb.template pv<NB>(smem + (RING + tile_of(grp, n_steps - 1) % RING) * TILE, 0, p);
    __syncthreads();
  }
  wait_vmem();   // copies of the last M phases

  // Merge groups 1 .. TG-1 into group 0 through LDS (the ring is free: all
  // copies have landed and every read is done).
  float* area = reinterpret_cast<float*>(smem) + rg * (TG - 1) * REC;
  __syncthreads();
  if (grp > 0) rb.save_to(area + (grp - 1) * REC);
  __syncthreads();
  if (grp > 0) return;
#pragma unroll
  for (int g = 1; g < TG; ++g) rb.merge_from(area + (g - 1) * REC);
  if constexpr (SPLITKV) {
    rb.finish_partial(part_o, part_lse, (hv.l + rb.qrow) * nsplit + split);
  } else {
    // this wave's merge record is read; its area stages the O tile
    static_assert(32 * RB::STAGE_STRIDE <= REC * 4, "O staging exceeds the merge record");
    rb.template finish_staged<WRITE_L>(O + head, L + hv.l, reinterpret_cast<char*>(area));
  }
}

// Kernel variants: 10*k + s = split kernel with KSPLIT k and s LDS stages;
// 100 + 10*r + k = pipelined kernel with KSPLIT k and a ring of r slots;
// 200 + r = ping-pong kernel with a ring of r tiles; 300 + r = ping-pong
// kernel with four tile groups (two wave teams) and a ring of r tiles;
// 400 + r = ping-pong kernel with 128-key tiles and a ring of r of them.
constexpr int kPingPong = 204;
constexpr int kPingPong4 = 308;
constexpr int kPingPongWide = 404;
constexpr int pipe_code(int ksplit, int ring) { return 100 + 10 * ring + ksplit; }

template <int D, bool CAUSAL, bool WRITE_L, bool FULL, int KSPLIT, int STAGES>
static void launch_split(const f16* Q, const f16* K, const f16* V, f16* O, float* L, Geom geo,
                         int num_qb, int total, float c, hipStream_t stream) {
  hipLaunchKernelGGL((fa_fwd_split_kernel<D, CAUSAL, WRITE_L, FULL, KSPLIT, STAGES>), dim3(total),
                     dim3(256 * KSPLIT), 0, stream, Q, K, V, O, L, geo, num_qb, total, c);
}

template <int D, bool CAUSAL, bool WRITE_L, bool FULL, int KSPLIT, int RING>
static void launch_pipe(const f16* Q, const f16* K, const f16* V, f16* O, float* L, Geom geo,
                        int num_qb, int total, float c, hipStream_t stream) {
  hipLaunchKernelGGL((fa_fwd_pipe_kernel<D, CAUSAL, WRITE_L, FULL, KSPLIT, RING>), dim3(total),
                     dim3(256 * KSPLIT), 0, stream, Q, K, V, O, L, geo, num_qb, total, c);
}

// Variants that exist and whose LDS fits in 160 KiB.
static bool variant_fits(int D, int variant) {
  const int tile = 64 * D * 2;
  if (variant == kPingPong) return true;
  if (variant == kPingPong4) return D == 64;   // 128 VGPRs per wave hold D = 64 only
  if (variant == kPingPongWide) return D == 64;   // two 128-key rings exceed the LDS at D = 128
  if (variant > 100) {
    const int ks = variant % 10, ring = (variant - 100) / 10;
    if ((ks != 1 && ks != 2) || ring < 2 || ring > 4) return false;
    return 2 * ring * ks * tile <= 160 * 1024;
  }
  const int ks = variant / 10, st = variant % 10;
  if ((ks != 1 && ks != 2 && ks != 4) || st < 2 || st > 4) return false;
  return 2 * st * ks * tile <= 160 * 1024;
}

template <int D, bool CAUSAL, bool WRITE_L, bool FULL>
static hipError_t launch_fwd(const void* q, const void* k, const void* v, void* o,
                             float* lse, Geom geo, int num_qb, int total, float c, int variant,
                             hipStream_t stream) {
  const f16* Q = (const f16*)q;
  const f16* K = (const f16*)k;
  const f16* V = (const f16*)v;
  f16* Op = (f16*)o;
  switch (variant) {
    case kPingPong:
      hipLaunchKernelGGL((fa_fwd_pp_kernel<D, CAUSAL, WRITE_L, FULL, 4>), dim3(total), dim3(512), 0,
                         stream, Q, K, V, Op, lse, geo, num_qb, total, c);
      break;
    case kPingPong4:
      if constexpr (D == 64) {
        hipLaunchKernelGGL((fa_fwd_pp_kernel<D, CAUSAL, WRITE_L, FULL, 8, false, 4>), dim3(total),
                           dim3(1024), 0, stream, Q, K, V, Op, lse, geo, num_qb, total, c);
        break;
      }
      return hipErrorInvalidValue;
    case kPingPongWide:
      if constexpr (D == 64) {
        hipLaunchKernelGGL((fa_fwd_pp_kernel<D, CAUSAL, WRITE_L, FULL, 4, false, 2, 2>),
                           dim3(total), dim3(512), 0, stream, Q, K, V, Op, lse, geo, num_qb,
                           total, c);
        break;
      }
      return hipErrorInvalidValue;
    case pipe_code(1, 2): launch_pipe<D, CAUSAL, WRITE_L, FULL, 1, 2>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break;
    case pipe_code(1, 3): launch_pipe<D, CAUSAL, WRITE_L, FULL, 1, 3>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break;
    case pipe_code(1, 4): launch_pipe<D, CAUSAL, WRITE_L, FULL, 1, 4>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break;
    case pipe_code(2, 2): launch_pipe<D, CAUSAL, WRITE_L, FULL, 2, 2>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break;
    case pipe_code(2, 3):
      if constexpr (D == 64) { launch_pipe<D, CAUSAL, WRITE_L, FULL, 2, 3>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break; }
      return hipErrorInvalidValue;
    case 13: launch_split<D, CAUSAL, WRITE_L, FULL, 1, 3>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break;
    case 14: launch_split<D, CAUSAL, WRITE_L, FULL, 1, 4>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break;
    case 22: launch_split<D, CAUSAL, WRITE_L, FULL, 2, 2>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break;
    case 23:
      if constexpr (D == 64) { launch_split<D, CAUSAL, WRITE_L, FULL, 2, 3>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break; }
      return hipErrorInvalidValue;
    case 24:
      if constexpr (D == 64) { launch_split<D, CAUSAL, WRITE_L, FULL, 2, 4>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break; }
      return hipErrorInvalidValue;
    case 42:
      if constexpr (D == 64) { launch_split<D, CAUSAL, WRITE_L, FULL, 4, 2>(Q, K, V, Op, lse, geo, num_qb, total, c, stream); break; }
      return hipErrorInvalidValue;
    default:
      launch_split<D, CAUSAL, WRITE_L, FULL, 1, 2>(Q, K, V, Op, lse, geo, num_qb, total, c, stream);
      break;
  }
  return hipGetLastError();
}

template <int D, bool CAUSAL>
static hipError_t dispatch_wl(const void* q, const void* k, const void* v, void* o,
                              float* lse, Geom geo, int num_qb, int total, float c, bool full,
                              int variant, hipStream_t s) {
  if (lse) {
    return full ? launch_fwd<D, CAUSAL, true, true>(q, k, v, o, lse, geo, num_qb, total, c, variant, s)
                : launch_fwd<D, CAUSAL, true, false>(q, k, v, o, lse, geo, num_qb, total, c, variant, s);
  }
  return full ? launch_fwd<D, CAUSAL, false, true>(q, k, v, o, lse, geo, num_qb, total, c, variant, s)
              : launch_fwd<D, CAUSAL, false, false>(q, k, v, o, lse, geo, num_qb, total, c, variant, s);
}

// Variant choice (measured on MI355X; see bench.py). The environment
// variable FA_MI355X_FWD_VARIANT ("pingpong", "pingpong4", "pingpongwide",
// "pipe<k>r<r>" or "split<k>s<s>", e.g. pipe1r3, split1s4)
// forces one that fits D; it is read once, for measurement and tests.
static int choose_variant(int64_t D) {
  static const int forced = [] {
    const char* e = getenv("FA_MI355X_FWD_VARIANT");
    if (!e) return -1;
    int ks = 0, st = 0;
    if (strcmp(e, "pingpong") == 0) return kPingPong;
    if (strcmp(e, "pingpong4") == 0) return kPingPong4;
    if (strcmp(e, "pingpongwide") == 0) return kPingPongWide;
    if (sscanf(e, "pipe%dr%d", &ks, &st) == 2) return pipe_code(ks, st);
    if (sscanf(e, "split%ds%d", &ks, &st) == 2) return 10 * ks + st;
    return -1;
  }();
  if (forced >= 0 && variant_fits((int)D, forced)) return forced;
  // The ping-pong kernel (ring of 4 tiles) is fastest at every measured
  // shape, D = 64 and 128, causal or not: one wave of each SIMD runs its
  // matrix phase while the other runs its softmax.
  return kPingPong;
}

}  // namespace fa

namespace fa {
// The forward over a head geometry with an explicit kernel variant (0: the
// default choice). Arguments are already validated.
static int fwd_run(const void* q, const void* k, const void* v, void* o, float* lse,
                   const Geom& geo, int64_t B, int64_t D, int causal, int variant, void* stream) {
  if (variant == 0) variant = choose_variant(D);
  if (!variant_fits((int)D, variant)) return FA_ERR_HEAD_DIM;
  const int num_qb = (geo.N + kBR - 1) / kBR;
  const int total = (int)(B * geo.H * num_qb);
  const float c = (float)(1.0 / sqrt((double)D)) * kLog2e;
  const bool full = geo.cu == nullptr && (geo.N % kBR) == 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  if (D == 64) {
    e = causal ? dispatch_wl<64, true>(q, k, v, o, lse, geo, num_qb, total, c, full, variant, s)
               : dispatch_wl<64, false>(q, k, v, o, lse, geo, num_qb, total, c, full, variant, s);
  } else {
    e = causal ? dispatch_wl<128, true>(q, k, v, o, lse, geo, num_qb, total, c, full, variant, s)
               : dispatch_wl<128, false>(q, k, v, o, lse, geo, num_qb, total, c, full, variant, s);
  }
  return e == hipSuccess ? FA_OK : -(int)e;
}

static int fwd_dense(const void* q, const void* k, const void* v, void* o, float* lse,
                     int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D, int causal,
                     int variant, void* stream) {
  const int st = fa_validate_fwd_gqa(q, k, v, o, B, H, H_kv, N, D);
  if (st != FA_OK) return st;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return FA_ERR_ALIGNMENT;
  const Geom geo{nullptr, (int)N, (int)H, (int)(H / H_kv), 0};
  return fwd_run(q, k, v, o, lse, geo, B, D, causal, variant, stream);
}
}  // namespace fa

namespace fa {
constexpr int kNumCUs = 256;   // MI355X

// Split-KV forward: the ping-pong kernel over (row block, split) units writes
// normalised fp32 partials and their LSEs; the decode's LSE combine, over the
// B*H*N rows, merges them into O and L. For long sequences over few heads,
// where the row blocks alone leave CUs idle.
template <int D, bool CAUSAL, bool FULL>
static hipError_t launch_splitkv(const f16* Q, const f16* K, const f16* V, f16* O, float* L,
                                 const Geom& geo, int num_qb, int units, float c, float* part_o,
                                 float* part_lse, int nsplit, int64_t rows, hipStream_t s) {
  hipLaunchKernelGGL((fa_fwd_pp_kernel<D, CAUSAL, true, FULL, 4, false, 2, 1, true>),
                     dim3(units * nsplit), dim3(512), 0, s, Q, K, V, O, L, geo, num_qb,
                     units * nsplit, c, part_o, part_lse, nsplit);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int st = fa_lse_combine_f32(part_o, part_lse, rows, 1, D, nsplit, O, L, s);
  return st == FA_OK ? hipSuccess : hipErrorInvalidValue;
}
}  // namespace fa

extern "C" int fa_fwd_splitkv_plan(int64_t B, int64_t H, int64_t N, int64_t D, int causal) {
  if (B <= 0 || H <= 0 || N <= 0 || (D != 64 && D != 128)) return 1;
  // Measured: a split pays where the row blocks leave CUs idle and each split
  // still has >= 32 key tiles (B1 H1 N16384: 122 -> 88 us with 2 splits);
  // with fewer tiles per workgroup its fixed costs and the combine pass
  // dominate (B1 H8 N1024: 11.5 -> 12.8 us + 7 us), and causal triangles did
  // not even out (B1 H8 N4096 causal: 36.5 -> 42.6 us).
  if (causal) return 1;
  const int64_t units = B * H * ((N + fa::kBR - 1) / fa::kBR);
  const int64_t tiles = (N + fa::kBC - 1) / fa::kBC;   // key tiles of a row block
  if (units >= fa::kNumCUs) return 1;
  int64_t sp = (fa::kNumCUs + units - 1) / units;
  sp = sp < tiles / 32 ? sp : tiles / 32;
  sp = sp < 8 ? sp : 8;
  return sp < 2 ? 1 : (int)sp;
}

extern "C" int64_t fa_fwd_splitkv_workspace_floats(int64_t B, int64_t H, int64_t N, int64_t D,
                                                   int64_t num_splits) {
  if (B <= 0 || H <= 0 || N <= 0 || (D != 64 && D != 128) || num_splits < 1) return 0;
  return B * H * N * num_splits * (D + 1);   // partial O, then the partial LSEs
}

extern "C" int fa_fwd_splitkv_f16(const void* q, const void* k, const void* v, void* o,
                                  float* lse, float* workspace, int64_t B, int64_t H,
                                  int64_t H_kv, int64_t N, int64_t D, int causal,
                                  int64_t num_splits, void* stream) {
  using namespace fa;
  int st = fa_validate_fwd_gqa(q, k, v, o, B, H, H_kv, N, D);
  if (st != FA_OK) return st;
  if (workspace == nullptr) return FA_ERR_NULL_POINTER;
  if (num_splits < 1 || num_splits > 16) return FA_ERR_NUM_SPLITS;
  if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0) return FA_ERR_ALIGNMENT;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return FA_ERR_ALIGNMENT;
  const int64_t num_qb = (N + kBR - 1) / kBR;
  if (B * H * num_qb > (int64_t(1) << 31) / num_splits) return FA_ERR_TOO_LARGE;
  const Geom geo{nullptr, (int)N, (int)H, (int)(H / H_kv), 0};
  const int units = (int)(B * H * num_qb);
  const float c = (float)(1.0 / sqrt((double)D)) * kLog2e;
  const bool full = (N % kBR) == 0;
  const int64_t rows = B * H * N;
  float* part_o = workspace;
  float* part_lse = workspace + rows * num_splits * D;
  const f16* Q = (const f16*)q;
  const f16* K = (const f16*)k;
  const f16* V = (const f16*)v;
  f16* Op = (f16*)o;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int ns = (int)num_splits;
  const int nq = (int)num_qb;
  hipError_t e;
#define FA_SPLITKV(DD, CC, FF) \
  launch_splitkv<DD, CC, FF>(Q, K, V, Op, lse, geo, nq, units, c, part_o, part_lse, ns, rows, s)
  if (D == 64) {
    e = causal ? (full ? FA_SPLITKV(64, true, true) : FA_SPLITKV(64, true, false))
               : (full ? FA_SPLITKV(64, false, true) : FA_SPLITKV(64, false, false));
  } else {
    e = causal ? (full ? FA_SPLITKV(128, true, true) : FA_SPLITKV(128, true, false))
               : (full ? FA_SPLITKV(128, false, true) : FA_SPLITKV(128, false, false));
  }
#undef FA_SPLITKV
  return e == hipSuccess ? FA_OK : -(int)e;
}

extern "C" int fa_fwd_f16(const void* q, const void* k, const void* v, void* o,
                          float* lse, int64_t B, int64_t H, int64_t N, int64_t D,
                          int causal, void* stream) {
  return fa::fwd_dense(q, k, v, o, lse, B, H, H, N, D, causal, 0, stream);
}

extern "C" int fa_fwd_gqa_f16(const void* q, const void* k, const void* v, void* o,
                              float* lse, int64_t B, int64_t H, int64_t H_kv, int64_t N,
                              int64_t D, int causal, void* stream) {
  return fa::fwd_dense(q, k, v, o, lse, B, H, H_kv, N, D, causal, 0, stream);
}

extern "C" int fa_fwd_varlen_f16(const void* q, const void* k, const void* v, void* o,
                                 float* lse, const int32_t* cu_seqlens, int64_t B, int64_t H,
                                 int64_t H_kv, int64_t max_seqlen, int64_t total, int64_t D,
                                 int causal, void* stream) {
  const int st = fa_validate_fwd_varlen(q, k, v, o, cu_seqlens, B, H, H_kv, max_seqlen, total, D);
  if (st != FA_OK) return st;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return FA_ERR_ALIGNMENT;
  const fa::Geom geo{cu_seqlens, (int)max_seqlen, (int)H, (int)(H / H_kv), (int)total, (int)B};
  return fa::fwd_run(q, k, v, o, lse, geo, B, D, causal, 0, stream);
}

namespace fa {
// bfloat16 forward: the default (ping-pong) kernel with bf16 operands
// (v_mfma_f32_32x32x16_bf16, P packed with v_cvt_pk_bf16_f32).
template <int D, bool CAUSAL, bool WRITE_L, bool FULL>
static void launch_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                        const Geom& geo, int num_qb, int total, float c, hipStream_t s) {
  const f16* Q = (const f16*)q;
  const f16* K = (const f16*)k;
  const f16* V = (const f16*)v;
  f16* O = (f16*)o;
  hipLaunchKernelGGL((fa_fwd_pp_kernel<D, CAUSAL, WRITE_L, FULL, 4, true>), dim3(total), dim3(512), 0,
                     s, Q, K, V, O, lse, geo, num_qb, total, c);
}

template <int D, bool CAUSAL>
static void dispatch_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                          const Geom& geo, int num_qb, int total, float c, bool full,
                          hipStream_t s) {
  if (lse) {
    if (full) launch_bf16<D, CAUSAL, true, true>(q, k, v, o, lse, geo, num_qb, total, c, s);
    else launch_bf16<D, CAUSAL, true, false>(q, k, v, o, lse, geo, num_qb, total, c, s);
  } else {
    if (full) launch_bf16<D, CAUSAL, false, true>(q, k, v, o, lse, geo, num_qb, total, c, s);
    else launch_bf16<D, CAUSAL, false, false>(q, k, v, o, lse, geo, num_qb, total, c, s);
  }
}
}  // namespace fa

extern "C" int fa_fwd_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                           int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D, int causal,
                           void* stream) {
  using namespace fa;
  const int st = fa_validate_fwd_gqa(q, k, v, o, B, H, H_kv, N, D);
  if (st != FA_OK) return st;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return FA_ERR_ALIGNMENT;
  const Geom geo{nullptr, (int)N, (int)H, (int)(H / H_kv), 0};
  const int num_qb = (int)((N + kBR - 1) / kBR);
  const int total = (int)(B * H * num_qb);
  const float c = (float)(1.0 / sqrt((double)D)) * kLog2e;
  const bool full = (N % kBR) == 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (D == 64) {
    if (causal) dispatch_bf16<64, true>(q, k, v, o, lse, geo, num_qb, total, c, full, s);
    else dispatch_bf16<64, false>(q, k, v, o, lse, geo, num_qb, total, c, full, s);
  } else {
    if (causal) dispatch_bf16<128, true>(q, k, v, o, lse, geo, num_qb, total, c, full, s);
    else dispatch_bf16<128, false>(q, k, v, o, lse, geo, num_qb, total, c, full, s);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FA_OK : -(int)e;
}

extern "C" int fa_probe_fwd_variant(const void* q, const void* k, const void* v, void* o,
                                    float* lse, int64_t B, int64_t H, int64_t N, int64_t D,
                                    int causal, int variant, void* stream) {
  if (variant <= 0) return FA_ERR_HEAD_DIM;
  return fa::fwd_dense(q, k, v, o, lse, B, H, H, N, D, causal, variant, stream);
}

extern "C" int fa_probe_default_variant(int64_t D) {
  if (D != 64 && D != 128) return 0;
  return fa::choose_variant(D);
}

extern "C" int fa_probe_fwd_variants(int* out, int max_out, int64_t D) {
  static const int all[] = {12, 13, 14, 22, 23, 24, 42, 121, 131, 141, 122, 132, 204, 308, 404};
  int n = 0;
  for (int v : all) {
    if (fa::variant_fits((int)D, v)) {
      if (out != nullptr && n < max_out) out[n] = v;
      ++n;
    }
  }
  return n;
}
