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
//   * a workgroup owns 128 query rows of one (b, h), 8 waves (64 rows with
//     four key-tile groups where 128-row blocks leave CUs idle); a 1-D grid
//     with an XCD-aware remap keeps the query blocks of a head on one XCD so
//     its K/V stay in that XCD's L2;
//   * K/V advance in 64-key tiles, copied global -> LDS by buffer_load ... lds
//     into rings of LDS slots while earlier tiles are consumed; every LDS
//     operand read has a constant offset from a per-lane base;
//   * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_f16 (fa_tile.hpp);
//   * softmax without a per-tile max reduction: P = 2^(S c - m) against the
//     running max m; the lane's tile sum bounds every P it holds, and only when
//     it exceeds 2^15 (first tile, or a much larger new maximum) is m raised
//     and O rescaled. P <= 2^15 stays inside fp16 and the fp32 accumulators.
// The kernel, fa_fwd_pp_kernel, is built on a per-wave core (RowBlock, 32
// rows): two wave groups own the even and odd key tiles of the same rows and
// alternate, barrier by barrier, between a matrix phase and a softmax phase,
// so each SIMD runs one wave's MFMAs while the other wave's VALU work issues.
// Template flags: D in {64,128}, CAUSAL, WRITE_L (O-only when false), FULL
// (N a multiple of the variant's full-tile unit: no bounds predicates), BF16,
// SPLITKV, TG (key-tile groups).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "fa_mi355x.h"
#include "fa_tile.hpp"

namespace fa {

constexpr int kBR = 128;   // query rows per workgroup
constexpr int kBC = 64;    // keys per tile
// A lane's tile sum of P above this triggers a rescale; it bounds every P,
// so P stays far inside the fp16 range (65504).
constexpr float kSumLimit = 32768.0f;

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

  // Row state without Q (the caller fills qf).
  __device__ __forceinline__ void setup(int lane_, int row_w_, int N_, float c_) {
    lane = lane_;
    hi = lane >> 5;
    N = N_;
    row_w = row_w_;
    qrow = row_w + (lane & 31);
    c = c_;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = f32x16{};
    m_run = -INFINITY;
    l_run = 0.f;
  }

  __device__ __forceinline__ void init(const f16* Qh, int head_bytes, int lane_, int row_w_,
                                       int N_, float c_) {
    setup(lane_, row_w_, N_, c_);
    // Buffer loads return zero for rows >= N.
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(Qh, head_bytes);
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(
          rq, (uint32_t)(qrow * D + 16 * kk + 8 * hi) * 2, 0, 0);
      qf[kk] = __builtin_bit_cast(f16x8, x);
    }
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

  // Merge records in LDS: m and l of the 64 lanes, then O in groups of four
  // registers, lane-major (16 bytes per lane, 1 KiB per group), so a lane
  // writes and reads its O with 16-byte accesses (conflict-free: the 64
  // lanes of an access cover 1 KiB contiguously).
  static constexpr int REC_FLOATS = (2 + 16 * DB) * 64;
  __device__ __forceinline__ static int rec_o(int g, int lane) { return 128 + (g * 64 + lane) * 4; }

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
      for (int q = 0; q < 4; ++q) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(src + rec_o(4 * db + q, lane));
#pragma unroll
        for (int e = 0; e < 4; ++e) o[db][4 * q + e] = o[db][4 * q + e] * a1 + v[e] * a2;
      }
    }
    m_run = M;
  }

  __device__ __forceinline__ void save_to(float* dst) const {
    dst[lane] = m_run;
    dst[64 + lane] = l_run;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f32x4*>(dst + rec_o(4 * db + q, lane)) =
            f32x4{o[db][4 * q], o[db][4 * q + 1], o[db][4 * q + 2], o[db][4 * q + 3]};
    }
  }

  // Parallel merge of the TG tile groups holding partial (m, l, O) for the
  // same rows: tile group P finishes part P of the O registers (groups
  // P·PG .. P·PG + PG − 1 of four registers, i.e. 16-byte chunks 2·P·PG/2 ..
  // of every row), so the TG waves merge and store at once instead of one
  // wave merging TG − 1 records. A part record holds m and l of the 64 lanes
  // and, lane-major like the full record, the parts of the other tile groups
  // (part p at slot p − (p > owner)).
  template <int TG>
  static constexpr int part_groups() { return 4 * DB / TG; }
  template <int TG>
  static constexpr int part_rec_floats() { return (2 + (TG - 1) * part_groups<TG>() * 4) * 64; }
  template <int TG>
  __device__ __forceinline__ static int part_off(int slot, int gi, int lane) {
    return 128 + ((slot * part_groups<TG>() + gi) * 64 + lane) * 4;
  }

  template <int TG>
  __device__ __forceinline__ void save_parts(float* rec, int self) const {
    constexpr int PG = part_groups<TG>();
    rec[lane] = m_run;
    rec[64 + lane] = l_run;
    static_for<0, TG>([&](auto pi) {
      constexpr int p = decltype(pi)::value;
      if (p != self) {
        const int slot = p - (p > self ? 1 : 0);
#pragma unroll
        for (int gi = 0; gi < PG; ++gi) {
          const int g = p * PG + gi;
          *reinterpret_cast<f32x4*>(rec + part_off<TG>(slot, gi, lane)) =
              f32x4{o[g / 4][4 * (g % 4)], o[g / 4][4 * (g % 4) + 1], o[g / 4][4 * (g % 4) + 2],
                    o[g / 4][4 * (g % 4) + 3]};
        }
      }
    });
  }

  // This wave's part P of the merged, normalised O tile into the row group's
  // `stage` (32 rows of STAGE_STRIDE bytes, shared by the TG waves); rec(i)
  // is tile group i's part record. Leaves the merged m and l in m_run, l_run
  // (every part computes the same values, in the same order).
  template <int TG, int P, typename Rec>
  __device__ __forceinline__ void merge_part_stage(Rec rec, char* stage) {
    constexpr int PG = part_groups<TG>();
    float mi[TG], li[TG];
#pragma unroll
    for (int i = 0; i < TG; ++i) {
      mi[i] = i == P ? m_run : rec(i)[lane];
      li[i] = i == P ? l_run : rec(i)[64 + lane];
    }
    float M = mi[0];
#pragma unroll
    for (int i = 1; i < TG; ++i) M = fmaxf(M, mi[i]);
    float a[TG];
    float l = 0.f;
#pragma unroll
    for (int i = 0; i < TG; ++i) {
      a[i] = (mi[i] == M) ? 1.f : exp2_hw(mi[i] - M);
      l += li[i] * a[i];
    }
    f32x4 acc[PG];
#pragma unroll
    for (int gi = 0; gi < PG; ++gi) {
      const int g = P * PG + gi;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[gi][e] = o[g / 4][4 * (g % 4) + e] * a[P];
    }
#pragma unroll
    for (int i = 0; i < TG; ++i) {
      if (i == P) continue;
      const int slot = P - (P > i ? 1 : 0);
#pragma unroll
      for (int gi = 0; gi < PG; ++gi) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(rec(i) + part_off<TG>(slot, gi, lane));
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[gi][e] = fmaf(v[e], a[i], acc[gi][e]);
      }
    }
    m_run = M;
    l_run = l;
    const float inv = 1.f / sum_xor32(l);
#pragma unroll
    for (int gi = 0; gi < PG; gi += 2) {
      const int g = P * PG + gi;                     // even: a pair of groups
      uint32_t w[2][2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f16x2 x0 = cvt2x<BF16>(acc[gi + j][0] * inv, acc[gi + j][1] * inv);
        const f16x2 x1 = cvt2x<BF16>(acc[gi + j][2] * inv, acc[gi + j][3] * inv);
        w[j][0] = __builtin_bit_cast(uint32_t, x0);
        w[j][1] = __builtin_bit_cast(uint32_t, x1);
      }
      const auto r0 = __builtin_amdgcn_permlane32_swap(w[0][0], w[1][0], false, false);
      const auto r1 = __builtin_amdgcn_permlane32_swap(w[0][1], w[1][1], false, false);
      const int chunk = 4 * (g / 4) + 2 * ((g % 4) / 2) + hi;   // 16-byte chunk of the row
      *reinterpret_cast<uint4*>(stage + (lane & 31) * STAGE_STRIDE + chunk * 16) =
          uint4{r0[0], r1[0], r0[1], r1[1]};
    }
  }

  // After every part is staged (a barrier): wave `self` of the TG stores its
  // share of the row group's 16-byte chunks, and tile group 0 writes L.
  template <int TG, bool WRITE_L>
  __device__ __forceinline__ void store_staged_part(f16* Oh, float* Lh, const char* stage,
                                                    int self) const {
    constexpr int CPR = D / 8;
    constexpr int PER = 32 * CPR / (64 * TG);
    static_assert(PER * 64 * TG == 32 * CPR, "whole chunks per lane");
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int idx = (k * TG + self) * 64 + lane;
      const int r = idx / CPR, ch = idx % CPR;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + r * STAGE_STRIDE + ch * 16);
      if (FULL || row_w + r < N)
        *reinterpret_cast<uint4*>(Oh + (size_t)(row_w + r) * D + ch * 8) = v;
    }
    const float l_tot = sum_xor32(l_run);   // all lanes: a cross-lane exchange
    if (WRITE_L && self == 0 && hi == 0 && (FULL || qrow < N))
      Lh[qrow] = (m_run + log2_hw(l_tot)) * kLn2;
  }

  // Rows of the O staging tile are padded by 16 bytes: spreads the LDS banks.
  static constexpr int STAGE_STRIDE = 2 * D + 16;

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

// LDS layouts of a 64-key tile, copied as 1 KiB blocks (lane l of a copy
// writes bytes [16 l, 16 l + 16) of its block, so a layout is chosen by which
// global 16-byte chunk each lane fetches):
//   * K: row-major [key][D] with the XOR swizzle of k_off;
//   * V: one block per PV operand fragment. Block b = ks * (D / 32) + db
//     holds keys 16 ks .. 16 ks + 15 as 64-byte rows of columns 32 db ..
//     32 db + 31, so the PV k-steps, in the order the matrix phases issue them
//     (k-step outer, d-block inner), read their fragments at increasing
//     addresses. With the row-major layout the d-blocks of one k-step share
//     rows and the reads alternate between them, which made the transposed
//     reads of a matrix phase ~12% slower (measured on MI355X). The
//     transposed reads of a block are conflict-free without a swizzle: the
//     32 lanes of a half wave cover 4 rows x 64 bytes, i.e. each of the 64
//     banks once.
template <int D>
__device__ __forceinline__ void dma_offsets(int b, int lane, uint32_t& koff, uint32_t& voff) {
  const int o = b * 1024 + 16 * lane;
  const int r = o / (2 * D);
  const int slot = (o % (2 * D)) / 16;
  koff = (uint32_t)(r * 2 * D + (slot ^ k_swz<D>(r)) * 16);
  constexpr int DB = D / 32;
  const int ks = b / DB, db = b % DB;
  voff = (uint32_t)((16 * ks + (lane >> 2)) * 2 * D + (4 * db + (lane & 3)) * 16);
}

// Lane offset, within a V block, of the transposed read of the block's lower
// 8 keys (the upper 8 follow at +512): lane l gets column 32 db + l % 32 of
// keys 4 (l / 32) .. + 3, the P^T key order of the S^T accumulators.
__device__ __forceinline__ int vblk_lane_off(int lane) {
  const int s = lane & 15;
  return (4 * (lane >> 5) + (s >> 2)) * 64 + 32 * ((lane >> 4) & 1) + 8 * (s & 3);
}

// The A operand (V^T) of PV fragment b, p = block b + vblk_lane_off(lane).
__device__ __forceinline__ f16x8 vblk_frag(lds_cp p) {
  const f16x4 lo = lds_tr16(p);
  const f16x4 up = lds_tr16(p + 512);
  return f16x8{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
}

// Copy one 1 KiB block of tile t of a head (K or V) into dst. The buffer
// range ends at the head's last byte, so rows >= N arrive as zeros; a tile
// past the end is still issued, with an empty buffer range (it writes zeros
// and reads no memory), so every wave issues the same number of copies per
// tile group and vmcnt counts stay exact.
template <int D, bool FULL>
__device__ __forceinline__ void dma_block_or_zero(const char* head, int head_bytes, int t,
                                                  bool valid, uint32_t dst, uint32_t off) {
  constexpr int TILE = kBC * D * 2;
  const int done = valid ? t * TILE : 0;
  const int bytes = !valid ? 0 : (FULL ? TILE : min(TILE, head_bytes - done));
  dma16(make_rsrc_s(head + done, bytes), dst, off);
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
//
// SPLITKV: the grid covers (row block, key range) units; each writes fp32
// partials normalised over its range and the range's LSE, merged by the LSE
// combine afterwards.
// ---------------------------------------------------------------------------
template <int D, bool CAUSAL, bool WRITE_L, bool FULL, int RING, bool BF16 = false,
          bool SPLITKV = false, int TG = 2>
__global__ void __launch_bounds__(512)
fa_fwd_pp_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                 const f16* __restrict__ V, f16* __restrict__ O,
                 float* __restrict__ L, Geom geo, int num_qb, int total, float c,
                 float* __restrict__ part_o = nullptr, float* __restrict__ part_lse = nullptr,
                 int nsplit = 1) {
  constexpr int NB = 2;                        // 32-key blocks per tile
  constexpr int TILE = kBC * D * 2;            // bytes of a 64-key K or V tile
  constexpr int BLOCKS = TILE / 1024;          // 1 KiB blocks per tile
  constexpr int NRG = 8 / TG;                  // row groups (32 rows each)
  constexpr int ROWS = 32 * NRG;               // query rows of the workgroup
  constexpr int LOADS = BLOCKS / NRG;          // blocks per M-phase wave per tile
  static_assert(TG == 2 || TG == 4, "two or four tile groups");
  static_assert(!SPLITKV || TG == 2, "split-KV runs with two tile groups");
  // Two steps of slots: a copy lands one step ahead of its read, and the
  // prologue's waits below are counted for this ring.
  static_assert(RING == 2 * TG, "a ring of two steps");
  static_assert(2 * RING * TILE <= 160 * 1024, "slots exceed the 160 KiB LDS");
  using RB = RowBlock<D, CAUSAL, FULL, BF16>;
  constexpr int DB = RB::DB;
  constexpr int KSTEPS = D / 16;
  constexpr int NMM = NB * KSTEPS;             // MFMAs of one QK (= of one PV)
  constexpr int PF = D == 64 ? 8 : 4;          // operand prefetch distance, in MFMAs
  constexpr int REC = RB::REC_FLOATS;          // floats per wave record of the merge
  static_assert(!SPLITKV || (TG - 1) * NRG * REC * 4 <= 2 * RING * TILE, "merge area too small");
  // K slots at [0, RING) * TILE, V slots at [RING, 2 RING) * TILE.
  __shared__ __attribute__((aligned(1024))) char smem[2 * RING * TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: SGPR
  const int rg = wave % NRG;                   // row group
  const int tg = wave / NRG;                   // tile group: tiles tg, tg + TG, ...
  const int grp = tg / (TG / 2);               // phase group; group 0 starts in the S phase
  // This wave's tile in step j.
  auto tile_of = [&](int j) { return TG * j + tg; };

  const int logical = xcd_remap(blockIdx.x, total, geo.nxcd);
  // Split-KV: the splits of one q-block are adjacent (same XCD, same K/V).
  const int split = SPLITKV ? logical % nsplit : 0;
  const int unit = SPLITKV ? logical / nsplit : logical;
  const int bh = unit / num_qb;
  int qb = unit - bh * num_qb;
  if (CAUSAL) qb = num_qb - 1 - qb;   // longest rows dispatch first

  const HeadView hv = head_view<D>(geo, bh);
  const int N = hv.n;
  if (qb * ROWS >= N) return;   // varlen: past this sequence (whole workgroup)
  const size_t head = hv.q;
  const int head_bytes = N * D * 2;
  const int q0 = qb * ROWS;

  RB rb;
  rb.init(Q + head, head_bytes, lane, q0 + 32 * rg, N, c);

  const int kv_end = CAUSAL ? min(N, q0 + ROWS) : N;
  int n_tiles = (kv_end + kBC - 1) / kBC;
  // Split-KV: this workgroup's tiles are tb .. tb + n_tiles - 1 of the row
  // block's; K/V pointers and bounds start at tile tb, masking uses absolute
  // key positions.
  int tb = 0;
  if constexpr (SPLITKV) {
    const int per = (n_tiles + nsplit - 1) / nsplit;
    tb = min(split * per, n_tiles);
    n_tiles = min(per, n_tiles - tb);
    if (n_tiles == 0) {   // nothing for this split: an empty partial for every row
      if (grp == 0) rb.finish_partial(part_o, part_lse, (hv.l + rb.qrow) * nsplit + split);
      return;
    }
  }
  const int kv_bytes = head_bytes - tb * TILE;
  const char* Kh = reinterpret_cast<const char*>(K + hv.kv) + (size_t)tb * TILE;
  const char* Vh = reinterpret_cast<const char*>(V + hv.kv) + (size_t)tb * TILE;
  // Tiles per tile group.
  const int n_steps = (n_tiles + TG - 1) / TG;

  const uint32_t lds0 = lds_addr(smem);
  // This wave's share of a tile copy in its M phase: blocks rg*LOADS .. +LOADS.
  uint32_t koff[LOADS], voff[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) dma_offsets<D>(rg * LOADS + i, lane, koff[i], voff[i]);
  // 1 KiB block b of tile t, bounded by the range (zeros past the end).
  auto dma_tile_block = [&](bool is_v, int t, uint32_t dst, uint32_t off) {
    dma_block_or_zero<D, FULL>(is_v ? Vh : Kh, kv_bytes, t, t < n_tiles, dst, off);
  };
  auto copy_block = [&](bool is_v, int t, int i) {
    const uint32_t at = lds0 + ((is_v ? RING : 0) + t % RING) * TILE + (rg * LOADS + i) * 1024;
    dma_tile_block(is_v, t, at, is_v ? voff[i] : koff[i]);
  };

  // Per-lane offsets of the operand fragments within a tile.
  int koffs[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) koffs[kk] = k_frag_off<D>(kk, lane);
  const int voff_l = vblk_lane_off(lane);

  // Prologue: the waves share the copies of K tiles 0 .. RING - TG/2 - 1 and
  // V tiles 0 .. RING - 3 TG/2 - 1 (those read before the first M-phase
  // copies land), 1 KiB block by block. (Waiting only for the K tiles of
  // step 0 here and for the rest during phase 0 measured 1-2% slower; so did,
  // by 3-6 % at every non-causal shape, group 1 copying and awaiting K tiles
  // 0 .. TG-1 while group 0 copies the rest and awaits them at the end of its
  // phase-0 softmax.)
  {
    constexpr int NK = RING - TG / 2, NV = RING - 3 * TG / 2;
    constexpr int ITEMS = (NK + NV) * BLOCKS;
#pragma unroll
    for (int it0 = 0; it0 < ITEMS; it0 += 8) {
      const int it = it0 + wave;
      if (ITEMS % 8 == 0 || it < ITEMS) {
        const bool is_v = it >= NK * BLOCKS;
        const int x = (is_v ? it - NK * BLOCKS : it) / BLOCKS;
        const int blk = it % BLOCKS;
        uint32_t ko, vo;
        dma_offsets<D>(blk, lane, ko, vo);
        dma_tile_block(is_v, x, lds0 + ((is_v ? RING : 0) + x) * TILE + blk * 1024,
                       is_v ? vo : ko);
      }
    }
  }
  wait_vmem();
  __syncthreads();

  f32x16 s[NB];       // scores of this wave's current tile
  f16x8 p[2 * NB];     // its packed P (one per PV k-step)

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
    lds_cp kl[KSTEPS];
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) kl[kk] = lds_lane_base(kt + koffs[kk]);
    const lds_cp vl = lds_lane_base(vt + voff_l);
    // MFMA m is PV i or QK i. With PV, in groups of four: QK 2j and 2j + 1
    // (the two 32-key blocks of k-step j, one Q^T operand), then PV 2j and
    // 2j + 1 (two d-blocks of one P^T operand), so consecutive MFMAs share
    // their B operand (1.6 % faster at the headline than alternating PV and
    // QK, same results: each accumulator still sums its k-steps in order);
    // every accumulator is reused four MFMAs later. Without PV, QK m. QK i:
    // block i % NB, k-step i / NB. PV i: k-step i / DB, d-block i % DB: V
    // block i.
    auto is_pv = [](int m) { return PV && (m & 3) >= 2; };
    auto idx = [](int m) { return PV ? 2 * (m >> 2) + (m & 1) : m; };
    auto fetch = [&](int m) -> f16x8 {
      const int i = idx(m);
      if (is_pv(m)) return vblk_frag(vl + i * 1024);
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
    if (SPLITKV && t >= n_tiles) {
      // A group's last tile can lie past a split's end: its keys belong to
      // the next split, so masking by N would not remove them. P = 0.
#pragma unroll
      for (int j = 0; j < 2 * NB; ++j) p[j] = f16x8{};
      wait_vmcnt<((RING - TG) / TG - 1) * 2 * LOADS>();
      return;
    }
    rb.template mask<2>(tb + t, 0, s);
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
    // This wave's copies of its M phase (RING - TG) / TG steps back; those of
    // the later M phases stay in flight.
    wait_vmcnt<((RING - TG) / TG - 1) * 2 * LOADS>();
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
  // M phase copies: K and V of the tiles RING - TG after the ones it reads
  // (the same tile group's tiles one ring turn minus a step later), into the
  // slots of the tiles it read in its previous M phase.
  auto mstep = [&](auto with_pv, int tq, int tv) {
    mphase(with_pv, tq, tv, tq + RING - TG, tv + RING - TG);
  };
  if (grp == 0) {
    rb.template qk<NB>(smem + (tile_of(0) % RING) * TILE, 0, s);
    __syncthreads();                 // its slot is refilled in phase 1
    for (int j = 0; j < n_steps; ++j) {
      pin_s();
      sphase(tile_of(j));
      pin_p();
      __syncthreads();
      mstep(BT{}, tile_of(j + 1), tile_of(j));
      __syncthreads();
    }
    __syncthreads();   // group 1's last PV
  } else {
    __syncthreads();
    // Step 0 (no PV yet) is peeled: with both M-phase forms in one loop body
    // the compiler moved the accumulators between them on every step.
    mstep(BF{}, tile_of(0), tile_of(-1));
    __syncthreads();
    pin_s();
    sphase(tile_of(0));
    pin_p();
    __syncthreads();
    for (int j = 1; j < n_steps; ++j) {
      mstep(BT{}, tile_of(j), tile_of(j - 1));
      __syncthreads();
      pin_s();
      sphase(tile_of(j));
      pin_p();
      __syncthreads();
    }
    // Phase 2n: the last PV.
    {
      const lds_cp vl = lds_lane_base(lds0 + (RING + tile_of(n_steps - 1) % RING) * TILE + voff_l);
#pragma unroll
      for (int i = 0; i < NMM; ++i) rb.o[i % DB] = mma32<BF16>(vblk_frag(vl + i * 1024), p[i / DB], rb.o[i % DB]);
    }
    __syncthreads();
  }
  wait_vmem();   // copies of the last M phases

  // Merge the tile groups' partial rows through LDS (the ring is free: all
  // copies have landed and every read is done).
  float* area = reinterpret_cast<float*>(smem);
  __syncthreads();
  // Every tile group merges and stores one part of the O columns of its
  // rows (RowBlock::merge_part_stage), through part records and a staging
  // tile per row group after them.
  constexpr int PREC = RB::template part_rec_floats<TG>();
  constexpr int RECS = TG * NRG * PREC;                 // floats of one row block's records
  constexpr int STAGE_BYTES = NRG * 32 * RB::STAGE_STRIDE;
  if constexpr (!SPLITKV) {
    static_assert(RECS * 4 + STAGE_BYTES <= 2 * RING * TILE, "merge area too small");
    auto rec = [&](int i) { return area + (i * NRG + rg) * PREC; };
    char* stage = reinterpret_cast<char*>(area + RECS) + rg * 32 * RB::STAGE_STRIDE;
    rb.template save_parts<TG>(rec(tg), tg);
    __syncthreads();
    static_for<0, TG>([&](auto pi) {
      constexpr int P = decltype(pi)::value;
      if (tg == P) rb.template merge_part_stage<TG, P>(rec, stage);
    });
    __syncthreads();
    rb.template store_staged_part<TG, WRITE_L>(O + head, L + hv.l, stage, tg);
    return;
  }
  // Split-KV: tile group 0 merges the others' records and writes the fp32
  // partial.
  if (tg > 0) rb.save_to(area + ((tg - 1) * NRG + rg) * REC);
  __syncthreads();
  if (tg > 0) return;
#pragma unroll
  for (int g = 1; g < TG; ++g) rb.merge_from(area + ((g - 1) * NRG + rg) * REC);
  rb.finish_partial(part_o, part_lse, (hv.l + rb.qrow) * nsplit + split);
}

// Kernel variants (for fa_probe_fwd_variant; the default path picks one per
// problem shape): the ping-pong kernel with two tile groups over 128 rows and
// a ring of 4 tiles (204), or with four tile groups over 64 rows and a ring
// of 8 tiles (408, D = 64: twice the workgroups for the same rows).
constexpr int kPingPong = 204;
constexpr int kPingPong4 = 408;
constexpr int kGuarded = 1000;   // probe flag: force the guarded (not full-tile) instance

// Query rows per row block, and the multiple of N that lets every tile group
// run the same number of whole tiles (the full-tile instance).
static int variant_rows(int variant) { return variant == kPingPong4 ? 64 : kBR; }
static int variant_full_n(int variant) { return variant == kPingPong4 ? 256 : kBR; }

// Variants that exist for head dimension D and the causal flag.
static bool variant_fits(int D, int variant, int causal) {
  if (variant == kPingPong) return true;
  if (variant == kPingPong4) return D == 64;
  (void)causal;
  return false;
}

// BF16: bf16 operands (v_mfma_f32_32x32x16_bf16, P packed with
// v_cvt_pk_bf16_f32) through the same kernels; the pointers carry 16-bit
// elements either way.
template <int D, bool CAUSAL, bool WRITE_L, bool FULL, bool BF16>
static hipError_t launch_fwd(const void* q, const void* k, const void* v, void* o,
                             float* lse, Geom geo, int num_qb, int total, float c, int variant,
                             hipStream_t stream) {
  const f16* Q = (const f16*)q;
  const f16* K = (const f16*)k;
  const f16* V = (const f16*)v;
  f16* Op = (f16*)o;
  switch (variant) {
    case kPingPong:
      hipLaunchKernelGGL((fa_fwd_pp_kernel<D, CAUSAL, WRITE_L, FULL, 4, BF16>), dim3(total),
                         dim3(512), 0, stream, Q, K, V, Op, lse, geo, num_qb, total, c);
      break;
    case kPingPong4:
      if constexpr (D == 64) {
        hipLaunchKernelGGL((fa_fwd_pp_kernel<D, CAUSAL, WRITE_L, FULL, 8, BF16, false, 4>),
                           dim3(total), dim3(512), 0, stream, Q, K, V, Op, lse, geo, num_qb, total, c);
        break;
      }
      return hipErrorInvalidValue;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int D, bool CAUSAL, bool BF16>
static hipError_t dispatch_wl(const void* q, const void* k, const void* v, void* o,
                              float* lse, Geom geo, int num_qb, int total, float c, bool full,
                              int variant, hipStream_t s) {
  if (lse) {
    return full ? launch_fwd<D, CAUSAL, true, true, BF16>(q, k, v, o, lse, geo, num_qb, total, c,
                                                          variant, s)
                : launch_fwd<D, CAUSAL, true, false, BF16>(q, k, v, o, lse, geo, num_qb, total, c,
                                                           variant, s);
  }
  return full ? launch_fwd<D, CAUSAL, false, true, BF16>(q, k, v, o, lse, geo, num_qb, total, c,
                                                         variant, s)
              : launch_fwd<D, CAUSAL, false, false, BF16>(q, k, v, o, lse, geo, num_qb, total, c,
                                                          variant, s);
}

// The kernel the forward runs for a problem shape (bh = B * H heads of N
// rows) on a device of `cus` compute units; nothing in the environment
// changes it. Measured on MI355X (256 CUs; D = 64, us, 128-row vs 64-row
// workgroups): where the 128-row grid leaves CUs idle the 64-row kernel wins
// (B1 H8 N2048 17.3 -> 13.8, B1 H4 N4096 29.7 -> 22.9, B1 H16 N1024 11.3 ->
// 9.6), and so it does for causal long rows on a single wave of workgroups
// (B1 H8 N4096 33.6 -> 29.0: the short row blocks finish early and free their
// CUs); from one 128-row block per CU on (non-causal) or two (causal) it
// loses (B1 H16 N2048 21.1 vs 26.5, B2 H8 N4096 causal 45.1 vs 55.5), as it
// does for causal N = 1024 (B4 H8 12.8 vs 17.6).
static int choose_variant(int64_t D, int causal, int64_t bh, int64_t N, int cus) {
  if (D != 64) return kPingPong;
  const int64_t grid = bh * ((N + kBR - 1) / kBR);
  if (grid < cus) return kPingPong4;
  if (causal && grid == cus && N >= 2048) return kPingPong4;
  return kPingPong;
}

}  // namespace fa

namespace fa {
// The forward over a head geometry with an explicit kernel variant (0: the
// default choice). Arguments are already validated.
static int fwd_run(const void* q, const void* k, const void* v, void* o, float* lse,
                   const Geom& geo_in, int64_t B, int64_t D, int causal, int variant, void* stream,
                   bool bf16 = false) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const Topology topo = stream_topology(s);
  Geom geo = geo_in;
  geo.nxcd = topo.xcds;
  // kGuarded + v: variant v through its guarded instance even where N is a
  // multiple of the row block (tests compare it bitwise with the full-tile one).
  const bool guarded = variant >= kGuarded;
  if (guarded) variant -= kGuarded;
  if (variant == 0) variant = choose_variant(D, causal, B * geo.H, geo.N, topo.cus);
  if (!variant_fits((int)D, variant, causal)) return FA_ERR_HEAD_DIM;
  const int rows = variant_rows(variant);
  const int num_qb = (geo.N + rows - 1) / rows;
  // The validation bounds the grid of 128-row blocks; 64-row blocks double it.
  if (B * geo.H * (int64_t)num_qb > (int64_t(1) << 31) - 1) return FA_ERR_TOO_LARGE;
  const int total = (int)(B * geo.H * num_qb);   // workgroups
  const float c = (float)(1.0 / sqrt((double)D)) * kLog2e;
  const bool full = !guarded && geo.cu == nullptr && (geo.N % variant_full_n(variant)) == 0;
  hipError_t e;
#define FA_FWD_DISPATCH(DD, CC, BB) \
  dispatch_wl<DD, CC, BB>(q, k, v, o, lse, geo, num_qb, total, c, full, variant, s)
  if (D == 64) {
    if (bf16) e = causal ? FA_FWD_DISPATCH(64, true, true) : FA_FWD_DISPATCH(64, false, true);
    else e = causal ? FA_FWD_DISPATCH(64, true, false) : FA_FWD_DISPATCH(64, false, false);
  } else {
    if (bf16) e = causal ? FA_FWD_DISPATCH(128, true, true) : FA_FWD_DISPATCH(128, false, true);
    else e = causal ? FA_FWD_DISPATCH(128, true, false) : FA_FWD_DISPATCH(128, false, false);
  }
#undef FA_FWD_DISPATCH
  return e == hipSuccess ? FA_OK : -(int)e;
}

static int fwd_dense(const void* q, const void* k, const void* v, void* o, float* lse,
                     int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D, int causal,
                     int variant, void* stream) {
  const int st = fa_validate_fwd_gqa(q, k, v, o, B, H, H_kv, N, D);
  if (st != FA_OK) return st;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return FA_ERR_ALIGNMENT;
  const Geom geo{nullptr, (int)N, (int)H, (int)(H / H_kv), 0, 0, 0};   // nxcd: launcher
  return fwd_run(q, k, v, o, lse, geo, B, D, causal, variant, stream);
}
}  // namespace fa

namespace fa {

// Split-KV forward: the ping-pong kernel over (row block, split) units writes
// normalised fp32 partials and their LSEs; the decode's LSE combine, over the
// B*H*N rows, merges them into O and L. For long sequences over few heads,
// where the row blocks alone leave CUs idle.
template <int D, bool CAUSAL, bool FULL>
static hipError_t launch_splitkv(const f16* Q, const f16* K, const f16* V, f16* O, float* L,
                                 const Geom& geo, int num_qb, int units, float c, float* part_o,
                                 float* part_lse, int nsplit, int64_t rows, hipStream_t s) {
  hipLaunchKernelGGL((fa_fwd_pp_kernel<D, CAUSAL, true, FULL, 4, false, true>),
                     dim3(units * nsplit), dim3(512), 0, s, Q, K, V, O, L, geo, num_qb,
                     units * nsplit, c, part_o, part_lse, nsplit);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int st = fa_lse_combine_f32(part_o, part_lse, rows, 1, D, nsplit, O, L, s);
  return st == FA_OK ? hipSuccess : hipErrorInvalidValue;
}
}  // namespace fa

namespace fa {
// Key splits for the torch forward on a device of `cus` compute units.
static int splitkv_plan(int64_t B, int64_t H, int64_t N, int64_t D, int causal, int cus) {
  if (B <= 0 || H <= 0 || N <= 0 || (D != 64 && D != 128) || cus <= 0) return 1;
  // D = 64: the 64-row kernel (chosen where 128-row blocks leave CUs idle)
  // beat every split count (us: B1 H1 N16384 79.7 vs 85.6 with 2 splits, B1 H2
  // N8192 42.0 vs 49.5, B1 H1 N8192 31.6 vs 32.0 with 4, B1 H2 N4096 18.8 vs
  // 23.1 with 4; causal B1 H2 N8192 36.0 vs 44.0, B1 H4 N4096 19.8 vs 28.9).
  if (D == 64) return 1;
  const int64_t units = B * H * ((N + kBR - 1) / kBR);
  const int64_t tiles = (N + kBC - 1) / kBC;   // key tiles of a row block
  // D = 128 splits only where the splits of every row block still fit one
  // wave of workgroups (B1 H3 N8192, 192 row blocks: 100.6 us unsplit,
  // 125.2 with 2 splits; causal 84.6 vs 95.6).
  if (2 * units > cus) return 1;
  int64_t sp = cus / units;
  sp = sp < 8 ? sp : 8;
  if (!causal) {
    // At least 32 key tiles per split (B1 H1 N16384: 156.5 -> 137.8 us with
    // 2 splits; B1 H8 N2048, 32 tiles: 27.3 vs 36.4 with 2).
    sp = sp < tiles / 32 ? sp : tiles / 32;
  } else {
    // Causal row blocks differ in length, and the longest sets the time: a
    // split evens them out down to 8 tiles per split (B1 H1 N8192 78.1 ->
    // 43.4 us with 4 splits, B1 H1 N2048 25.2 -> 17.6 with 4, B1 H2 N8192
    // 79.4 -> 68.0 with 2), but a 2-way split needs 64 tiles (B1 H4 N4096
    // 43.6 -> 41.7; B1 H8 N2048, 32 tiles: 25.9 -> 34.5).
    sp = sp < tiles / 8 ? sp : tiles / 8;
    if (sp == 2 && tiles < 64) sp = 1;
  }
  return sp < 2 ? 1 : (int)sp;
}
}  // namespace fa

extern "C" int fa_fwd_splitkv_plan(int64_t B, int64_t H, int64_t N, int64_t D, int causal) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  return fa::splitkv_plan(B, H, N, D, causal, fa::device_topology(dev).cus);
}

extern "C" int fa_probe_splitkv_plan_cus(int64_t B, int64_t H, int64_t N, int64_t D, int causal,
                                         int cus) {
  return fa::splitkv_plan(B, H, N, D, causal, cus);
}

extern "C" int fa_probe_choose_variant(int64_t D, int causal, int64_t bh, int64_t N, int cus) {
  if ((D != 64 && D != 128) || bh <= 0 || N <= 0 || cus <= 0) return 0;
  return fa::choose_variant(D, causal, bh, N, cus);
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
  Geom geo{nullptr, (int)N, (int)H, (int)(H / H_kv), 0, 0, 1};
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
  geo.nxcd = stream_topology(s).xcds;
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
  const fa::Geom geo{cu_seqlens, (int)max_seqlen, (int)H, (int)(H / H_kv), (int)total,
                       (int)B, 0};   // nxcd: launcher
  return fa::fwd_run(q, k, v, o, lse, geo, B, D, causal, 0, stream);
}

extern "C" int fa_fwd_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                           int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D, int causal,
                           void* stream) {
  using namespace fa;
  const int st = fa_validate_fwd_gqa(q, k, v, o, B, H, H_kv, N, D);
  if (st != FA_OK) return st;
  if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3u) != 0) return FA_ERR_ALIGNMENT;
  const Geom geo{nullptr, (int)N, (int)H, (int)(H / H_kv), 0, 0, 0};   // nxcd: launcher
  // The fp16 path's kernel choice for the shape, with bf16 operands.
  return fwd_run(q, k, v, o, lse, geo, B, D, causal, 0, stream, true);
}

extern "C" int fa_probe_fwd_variant(const void* q, const void* k, const void* v, void* o,
                                    float* lse, int64_t B, int64_t H, int64_t N, int64_t D,
                                    int causal, int variant, void* stream) {
  if (variant < 0) return FA_ERR_HEAD_DIM;
  return fa::fwd_dense(q, k, v, o, lse, B, H, H, N, D, causal, variant, stream);
}

extern "C" int fa_probe_default_variant(int64_t D) {
  if (D != 64 && D != 128) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  return fa::choose_variant(D, 0, 8, 4096, fa::device_topology(dev).cus);
}

extern "C" int fa_probe_fwd_variants(int* out, int max_out, int64_t D, int causal) {
  static const int all[] = {204, 408};
  int n = 0;
  for (int v : all) {
    if (fa::variant_fits((int)D, v, causal)) {
      if (out != nullptr && n < max_out) out[n] = v;
      ++n;
    }
  }
  return n;
}
