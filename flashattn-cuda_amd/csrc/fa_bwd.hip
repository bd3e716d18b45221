// fa_bwd.hip — FlashAttention backward for gfx950 (MI355X): dQ, dK, dV from
// Q, K, V, O, dO and the forward's logsumexp L.
//
// The reference's backward (cuda/flash_attn_kernel.cu:417-503, fp32 math, one
// thread per row) runs three kernels: D_i = rowsum(dO * O) (:173-191), dQ
// (:193-...) and dK/dV, each recomputing P = exp(S - L) from the saved L. This
// file keeps that decomposition — it needs no atomics and no O(N^2) storage —
// and builds each kernel on v_mfma_f32_32x32x16_f16 with fp32 accumulation:
//
//   fa_bwd_di_kernel    D_i = sum_d dO[i][d] * O[i][d] (fp32, stored negated)
//   dK/dV body          a workgroup owns 128 keys (32 per wave, K and V as
//                       register operands) and streams 64-query tiles of Q
//                       and dO (plus L, D_i) through LDS rings: S = Q K^T,
//                       dP = dO V^T, P = exp2(S c - L log2e),
//                       dS = P (dP - D_i), dV^T += dO^T P, dK^T += Q^T dS
//   dQ body             a workgroup owns 128 queries (32 per wave, Q and dO
//                       as register operands) and streams 64-key tiles of K
//                       and V: S^T = K Q^T, dP^T = V dO^T, dS^T as above,
//                       dQ^T += K^T dS^T
//
// The two bodies run as one launch (fa_bwd_fused_kernel: a workgroup takes
// one role by its block index). In each workgroup two wave groups take the
// two 32-row halves of every tile and run one phase apart, so one wave's
// MFMAs overlap the other wave's VALU work on every SIMD.
//
// P and dS are packed to fp16 straight from the score accumulators as the B
// operands of the gradient products (the reduction index is permuted the same
// way in both operands, as in the forward). Tiles read both as rows (b128)
// and transposed (ds_read_b64_tr_b16) are stored in LDS twice, once per
// swizzle, so both reads stay bank-conflict free.
#include <hip/hip_runtime.h>

#include <stdlib.h>

#include <math.h>
#include <stdint.h>


#include <type_traits>

#include "fa_mi355x.h"
#include "fa_tile.hpp"

namespace fa {
namespace bwd {

constexpr int kBQ = 64;     // rows of a streamed tile
constexpr int kBlk = 128;   // rows owned by a workgroup (32 per wave)

// Per-lane source offsets of 1 KiB block b of a 64-row tile, for the K-style
// (row reads) and V-style (transposed reads) LDS swizzles.
template <int D>
__device__ __forceinline__ void block_offsets(int b, int lane, uint32_t& koff, uint32_t& voff) {
  const int o = b * 1024 + 16 * lane;
  const int r = o / (2 * D);
  const int slot = (o % (2 * D)) / 16;
  koff = (uint32_t)(r * 2 * D + (slot ^ k_swz<D>(r)) * 16);
  voff = (uint32_t)(r * 2 * D + (slot ^ v_swz<D>(r)) * 16);
}

// A pointer the caller knows to be the same in every lane, moved to SGPRs
// (buffer resources must be scalar; selects between head pointers otherwise
// leave the compiler unsure of that).
template <typename T>
__device__ __forceinline__ const T* wave_uniform(const T* p) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  return (const T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// Copy 1 KiB block `blk` of 64-row tile t of a head (bytes head_bytes; rows
// past the end arrive as zeros) into LDS at dst, with per-lane offset off.
template <int D>
__device__ __forceinline__ void copy_block(const char* head, int head_bytes, int t, uint32_t dst,
                                           uint32_t off) {
  constexpr int TILE = kBQ * D * 2;
  const int done = t * TILE;
  const int bytes = max(0, min(TILE, head_bytes - done));
  dma16(make_rsrc(wave_uniform(head + (bytes > 0 ? done : 0)),
                  __builtin_amdgcn_readfirstlane(bytes)), dst, off);
}

// 64 floats of a row vector (L or D_i) starting at row t*64 into 256 bytes of
// LDS at dst, one per lane (rows >= n arrive as zeros). Dword copies: a head's
// row vector starts at bh*N floats, only 4-byte aligned.
__device__ __forceinline__ void copy_rowvec(const float* base, int n, int t, uint32_t dst,
                                            int lane) {
  const int done = t * kBQ;
  const int bytes = max(0, min(kBQ, n - done)) * 4;
  dma4(make_rsrc(wave_uniform(base + (bytes > 0 ? done : 0)),
                 __builtin_amdgcn_readfirstlane(bytes)), dst, (uint32_t)(4 * lane));
}

// B operand (16 x 32) of a product over D from 32 rows of a [N][D] fp16 head:
// lane l holds row (row0 + l%32), columns 16 kk + 8 (l/32) .. +7 (zeros for
// rows >= n via the buffer range).
template <int D>
__device__ __forceinline__ void load_row_operand(const f16* head, int n, int row0, int lane,
                                                 f16x8 (&out)[D / 16]) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(head, n * D * 2);
  const int row = row0 + (lane & 31);
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(
        r, (uint32_t)(row * D + 16 * kk + 8 * (lane >> 5)) * 2, 0, 0);
    out[kk] = __builtin_bit_cast(f16x8, x);
  }
}

// Store a C-layout accumulator pair-block acc[DB] (rows = 32 d of each block,
// columns = 32 rows of the output) as fp32 rows out[row][d], scaled.
template <int D>
__device__ __forceinline__ void store_transposed(float* out, int n, int row0, int lane,
                                                 const f32x16 (&acc)[D / 32], float scale) {
  const int row = row0 + (lane & 31);
  if (row >= n) return;
  float* dst = out + (size_t)row * D + 4 * (lane >> 5);
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f32x4 v = {acc[db][4 * g] * scale, acc[db][4 * g + 1] * scale, acc[db][4 * g + 2] * scale,
                 acc[db][4 * g + 3] * scale};
      *reinterpret_cast<f32x4*>(dst + 32 * db + 8 * g) = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Row terms: ND[i] = -D_i = -sum_d dO[i][d] * O[i][d] and NL[i] = -L[i] *
// log2(e), so that P = exp2(S c + NL) takes one fma and dP - D_i = dP + ND
// one add (or an MFMA chain's initial value). 8 lanes per row, one 16-byte
// chunk each per step (coalesced 128-byte runs), reduced with xor shuffles.
// ---------------------------------------------------------------------------
template <int D, bool BF16>
__global__ void __launch_bounds__(256)
fa_bwd_di_kernel(const f16* __restrict__ O, const f16* __restrict__ dO,
                 const float* __restrict__ L, float* __restrict__ ND, float* __restrict__ NL,
                 int64_t rows) {
  const int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int part = threadIdx.x & 7;
  float acc = 0.f;
  if (row < rows) {
    const f16x8* o = reinterpret_cast<const f16x8*>(O + row * D);
    const f16x8* g = reinterpret_cast<const f16x8*>(dO + row * D);
#pragma unroll
    for (int i = part; i < D / 8; i += 8) {
      const f16x8 a = o[i], b = g[i];
      if constexpr (BF16) {
        const bf16x8 ab = __builtin_bit_cast(bf16x8, a), bb = __builtin_bit_cast(bf16x8, b);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf((float)ab[e], (float)bb[e], acc);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf((float)a[e], (float)b[e], acc);
      }
    }
  }
  acc += __shfl_xor(acc, 1, 8);
  acc += __shfl_xor(acc, 2, 8);
  acc += __shfl_xor(acc, 4, 8);
  if (row < rows && part == 0) {
    ND[row] = -acc;
    NL[row] = -L[row] * kLog2e;
  }
}

// Partial accumulators of the second wave group, added into the first's
// through LDS (lane-major, conflict-free): wave slot w, NA arrays of DB
// blocks of 16 registers.
template <int NA, int DB>
__device__ __forceinline__ void group_reduce(char* smem, int grp, int slot, int lane,
                                             f32x16 (&a)[NA][DB]) {
  float* buf = reinterpret_cast<float*>(smem) + (size_t)slot * NA * DB * 16 * 64 + lane;
  __syncthreads();   // every wave is done with the staging buffers
  if (grp == 1) {
#pragma unroll
    for (int x = 0; x < NA; ++x)
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) buf[((x * DB + db) * 16 + r) * 64] = a[x][db][r];
  }
  __syncthreads();
  if (grp == 0) {
#pragma unroll
    for (int x = 0; x < NA; ++x)
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) a[x][db][r] += buf[((x * DB + db) * 16 + r) * 64];
  }
}

// ---------------------------------------------------------------------------
// dK/dV and dQ bodies (8 waves). A dK/dV workgroup owns 128 keys of one
// (b, h): wave w holds K^T and V^T of keys k0 + 32 (w % 4) .. +31 as register
// B operands, and 64-query tiles of Q and dO stream through LDS, each stored
// twice (row swizzle for the score products, transposed swizzle for the
// gradient products), with 64 floats each of NL and -D_i. A dQ workgroup
// owns 128 queries the same way (Q^T and dO^T as register operands, NL and
// -D_i lane constants) and streams 64-key tiles of K (twice) and V.
//
// The two wave groups (waves 0-3 and 4-7) hold the same keys (dK/dV) or
// queries (dQ), each takes one 32-row half of every tile, their partial sums
// are added through LDS at the end (group_reduce), and they run one phase
// apart. Each tile's work splits into the score products A (S and dP
// MFMAs), the VALU part B (P, dS, packed as B operands) and the gradient
// products C; a group's matrix phase M(j) issues C of its tile j - 1 and A
// of tile j, its softmax phase S(j) runs B of tile j. In every phase one
// group is in M and the other in S, so each SIMD overlaps one wave's MFMAs
// with the other's VALU work:
//
//   phase      2j          2j+1        ...   2T          2T+1
//   group 0    M(j)        S(j)              C(T-1)      -
//   group 1    S(j-1)      M(j)              S(T-1)      C(T-1)
//
// A group reads only its own 32-row half of every tile, so it copies only
// that half, and the row vectors into slots of its own: the groups share no
// staged data, and the barriers keep them one phase apart and sync each
// group's four waves on their copies.
//
// D = 64 (rows 32 g .. +31 of each part are its 1 KiB blocks 4 g .. 4 g + 3
// in both swizzles): tile j's stage is read
// from S(j - 1), which loads tile j's A operands into registers (M(j) then
// issues its score products without LDS waits), to M(j + 1), which reads its
// C operands. S(j) starts the copies of tile j + 3 into the stage of tile
// j - 1 (last read in M(j), before the barrier that starts S(j)) and M(j + 2)
// waits for them, leaving those of S(j + 1) in flight: a ring of 4 stages,
// with the copy issue in the VALU phase.
// ---------------------------------------------------------------------------
constexpr int kPPStages = 4;

template <int D>
constexpr int dkdv_pp_smem() {
  constexpr int STAGE = 4 * (kBQ * D * 2) + 2048;
  constexpr int RED = 4 * 2 * (D / 32) * 16 * 64 * 4;
  return kPPStages * STAGE > RED ? kPPStages * STAGE : RED;
}

template <int D>
constexpr int dq_pp_smem() {
  constexpr int STAGE = 3 * (kBQ * D * 2);
  constexpr int RED = 4 * (D / 32) * 16 * 64 * 4;
  return kPPStages * STAGE > RED ? kPPStages * STAGE : RED;
}

template <int D, bool CAUSAL, bool BF16>
__device__ __forceinline__ void dkdv_body_pp(const f16* __restrict__ Q, const f16* __restrict__ K,
                                             const f16* __restrict__ V, const f16* __restrict__ dO,
                                             const float* __restrict__ NL,
                                             const float* __restrict__ ND, float* __restrict__ dK,
                                             float* __restrict__ dV, const Geom& geo, int num_kb,
                                             int total, float c, float scale, int block,
                                             char* smem /* dkdv_pp_smem<D>() bytes */) {
  static_assert(D == 64, "a 32-row half of a tile is 4 blocks, the register budget D = 64's");
  constexpr int TILE = kBQ * D * 2;
  constexpr int BLOCKS = TILE / 1024;
  constexpr int OWN = BLOCKS / 2;              // blocks of a 32-row half
  constexpr int KSTEPS = D / 16, DB = D / 32;
  // Qk | Qv | dOk | dOv | row vectors (group g: L at +512 g, D_i at +512 g + 256)
  constexpr int STAGE = 4 * TILE + 2048;
  static_assert(kPPStages * STAGE <= 160 * 1024, "LDS");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kw = wave & 3;
  const int grp = wave >> 2;                   // also this group's query half of a tile
  const int qb = grp;
  const int hi = lane >> 5;
  const int logical = xcd_remap(block, total, geo.nxcd);
  const int bh = logical / num_kb;
  const int kb = logical - bh * num_kb;
  const int k0 = kb * kBlk;
  const int key = k0 + 32 * kw + (lane & 31);

  const HeadView hv = head_view<D>(geo, bh);
  const int N = hv.n;
  if (k0 >= N) return;   // varlen: past this sequence (whole workgroup)
  const size_t head = hv.q;
  const int head_bytes = N * D * 2;
  const char* Qh = reinterpret_cast<const char*>(Q + head);
  const char* Gh = reinterpret_cast<const char*>(dO + head);
  const float* Lh = NL + hv.l;
  const float* Dh = ND + hv.l;   // -D_i

  f16x8 kf[KSTEPS], vf[KSTEPS];   // B operands: K^T and V^T of this wave's keys
  load_row_operand<D>(K + hv.kv, N, k0 + 32 * kw, lane, kf);
  load_row_operand<D>(V + hv.kv, N, k0 + 32 * kw, lane, vf);
  f32x16 acc[2][DB];              // [0] = dV^T, [1] = dK^T (unscaled)
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    acc[0][db] = f32x16{};
    acc[1][db] = f32x16{};
  }

  const int n_qt = (N + kBQ - 1) / kBQ;
  const int t0 = CAUSAL ? k0 / kBQ : 0;   // earlier query tiles see none of these keys
  const int T = n_qt - t0;                 // tiles of this workgroup (>= 1)

  const uint32_t lds0 = lds_addr(smem);
  auto stage_of = [&](int j) { return smem + (j % kPPStages) * STAGE; };
  // This group's half of tile t into stage st: wave kw copies its 4 blocks of
  // part kw; waves 0 and 1 also copy the 64-row L and D_i vectors.
  auto issue_own = [&](int t, int st) {
    const uint32_t base = lds0 + st * STAGE;
    const char* src = kw < 2 ? Qh : Gh;
#pragma unroll
    for (int i = 0; i < OWN; ++i) {
      const int b = OWN * grp + i;
      uint32_t ko, vo;
      block_offsets<D>(b, lane, ko, vo);
      copy_block<D>(src, head_bytes, t, base + kw * TILE + b * 1024, (kw & 1) ? vo : ko);
    }
    if (kw == 0) copy_rowvec(Lh, N, t, base + 4 * TILE + 512 * grp, lane);
    if (kw == 1) copy_rowvec(Dh, N, t, base + 4 * TILE + 512 * grp + 256, lane);
  };
  // Copies run three tiles ahead: at the end of M phase j tile j + 1 must
  // have landed, and tile j + 2's copies (this wave's last issue) may still
  // be in flight.
  auto wait_next = [&](bool later_in_flight) {
    if (!later_in_flight) wait_vmem();
    else if (kw < 2) wait_vmcnt<OWN + 1>();
    else wait_vmcnt<OWN>();
  };
  issue_own(t0, 0);
  if (T > 1) issue_own(t0 + 1, 1);
  if (T > 2) issue_own(t0 + 2, 2);
  wait_next(T > 2);
  __syncthreads();

  f32x16 s = {}, dp = {};   // this wave's scores of its current tile
  f16x8 pb[2], gb[2];       // its packed P and dS (B operands of the two k-steps)
  f16x8 af[KSTEPS][2];      // A operands of its next score products (Q, dO rows)
  auto load_a = [&](int j) {   // of relative tile j
    const char* sb = stage_of(j);
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      af[kk][0] = load_k_frag<D>(sb, qb, kk, lane);
      af[kk][1] = load_k_frag<D>(sb + 2 * TILE, qb, kk, lane);
    }
  };
  // A: S = Q K^T and dP = dO V^T (C layout: register r holds query
  // qt0 + 32 qb + 8 (r/4) + 4 hi + r%4, lane l key l%32).
  auto mma_a = [&](int kk) {
    s = mma32<BF16>(af[kk][0], kf[kk], kk == 0 ? f32x16{} : s);
    dp = mma32<BF16>(af[kk][1], vf[kk], kk == 0 ? f32x16{} : dp);
  };
  // C of the tile whose stage is sb: dV^T += dO^T P and dK^T += Q^T dS; step
  // kk is k-step kk / DB, d-block kk % DB. Operands (dO^T, Q^T) read two
  // steps ahead.
  auto load_c = [&](const char* sb, int kk, f16x8 (&f)[2]) {
    const int jj = 2 * qb + kk / DB;
    f[0] = load_v_frag<D>(sb + 3 * TILE, jj, kk % DB, lane);
    f[1] = load_v_frag<D>(sb + TILE, jj, kk % DB, lane);
  };
  auto mma_c = [&](const f16x8 (&f)[2], int kk) {
    const int h = kk / DB, db = kk % DB;
    acc[0][db] = mma32<BF16>(f[0], pb[h], acc[0][db]);
    acc[1][db] = mma32<BF16>(f[1], gb[h], acc[1][db]);
  };
  // M phase of relative tile j (WITH_C: C of tile j - 1; WITH_A: A of tile
  // j); then the wait for the copies this wave started in S(j - 1).
  auto mphase = [&](int j, auto with_c, auto with_a) {
    constexpr bool WC = decltype(with_c)::value, WA = decltype(with_a)::value;
    const char* sc = stage_of(j + kPPStages - 1);
    f16x8 cf[KSTEPS][2];
    if constexpr (WC) {
      load_c(sc, 0, cf[0]);
      load_c(sc, 1, cf[1]);
    }
    static_for<0, KSTEPS>([&](auto ki) {
      constexpr int kk = decltype(ki)::value;
      if constexpr (WC && kk + 2 < KSTEPS) load_c(sc, kk + 2, cf[kk + 2]);
      if constexpr (WA) mma_a(kk);   // register operands: first, while C's land
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (WC) mma_c(cf[kk], kk);
      __builtin_amdgcn_sched_barrier(0);   // keep every product in this phase
    });
    wait_next(j + 2 < T);
  };
  // S phase of relative tile j: the copies of tile j + 3 (into the stage of
  // tile j - 1, whose last reads were this group's M phase j), P and dS into
  // pb, gb, and tile j + 1's A operands.
  auto sphase = [&](int j) {
    if (j + 3 < T) issue_own(t0 + j + 3, (j + 3) % kPPStages);
    const char* sb = stage_of(j);
    const int qt0 = (t0 + j) * kBQ;
    const float* ls = reinterpret_cast<const float*>(sb + 4 * TILE + 512 * grp);
    const float* nds = ls + 64;
    // Row vectors first (LDS reads return in order), then the next tile's A
    // operands, which land while the VALU work below runs.
    f32x4 lq[4], nd[4];
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      lq[r4] = *reinterpret_cast<const f32x4*>(ls + 32 * qb + 8 * r4 + 4 * hi);
      nd[r4] = *reinterpret_cast<const f32x4*>(nds + 32 * qb + 8 * r4 + 4 * hi);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (j + 1 < T) load_a(j + 1);
    __builtin_amdgcn_sched_barrier(0);
    f32x16 p, g;
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = exp2_hw(fmaf(s[r], c, lq[r >> 2][r & 3]));
    const bool edge = (qt0 + 32 * qb + 32 > N) || (CAUSAL && qt0 + 32 * qb < k0 + 32 * kw + 32);
    if (edge) {   // rows past N, and (causal) keys after the row
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int q = qt0 + 32 * qb + 8 * (r >> 2) + 4 * hi + (r & 3);
        p[r] = ((q >= N) || (CAUSAL && key > q)) ? 0.f : p[r];
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) g[r] = p[r] * (dp[r] + nd[r >> 2][r & 3]);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      pb[h] = pack_px<BF16>(p, h);
      gb[h] = pack_px<BF16>(g, h);
    }
  };
  // Register-only work stays in its phase (see the forward kernel).
  auto pin_s = [&] { asm volatile("" : "+v"(s), "+v"(dp)); };
  auto pin_p = [&] { asm volatile("" : "+v"(pb[0]), "+v"(pb[1]), "+v"(gb[0]), "+v"(gb[1])); };

  using BT = std::true_type;
  using BF = std::false_type;
  load_a(0);
  if (grp == 1) __syncthreads();   // phase 0: group 1 waits
  mphase(0, BF{}, BT{});
  __syncthreads();
  pin_s();
  sphase(0);
  pin_p();
  __syncthreads();
  for (int j = 1; j < T; ++j) {
    mphase(j, BT{}, BT{});
    __syncthreads();
    pin_s();
    sphase(j);
    pin_p();
    __syncthreads();
  }
  mphase(T, BT{}, BF{});   // C of the last tile
  __syncthreads();
  if (grp == 0) __syncthreads();   // phase 2T + 1: group 0 waits
  group_reduce<2, DB>(smem, grp, kw, lane, acc);
  if (grp == 0) {
    store_transposed<D>(dV + head, N, k0 + 32 * kw, lane, acc[0], 1.f);
    store_transposed<D>(dK + head, N, k0 + 32 * kw, lane, acc[1], scale);
  }
}

template <int D, bool CAUSAL, bool BF16>
__device__ __forceinline__ void dq_body_pp(const f16* __restrict__ Q, const f16* __restrict__ K,
                                           const f16* __restrict__ V, const f16* __restrict__ dO,
                                           const float* __restrict__ NL,
                                           const float* __restrict__ ND, float* __restrict__ dQ,
                                           const Geom& geo, int num_qb, int total, float c,
                                           float scale, int block,
                                           char* smem /* dq_pp_smem<D>() bytes */) {
  static_assert(D == 64, "a 32-row half of a tile is 4 blocks, the register budget D = 64's");
  constexpr int TILE = kBQ * D * 2;
  constexpr int BLOCKS = TILE / 1024;
  constexpr int OWN = BLOCKS / 2;              // blocks of a 32-row half
  constexpr int PER = 3 * OWN / 4;             // blocks per wave of a group's copies
  constexpr int KSTEPS = D / 16, DB = D / 32;
  constexpr int STAGE = 3 * TILE;              // Kk | Kv | Vk
  static_assert(3 * OWN % 4 == 0 && kPPStages * STAGE <= 160 * 1024, "copy split, LDS");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qw = wave & 3;
  const int grp = wave >> 2;                   // also this group's key half of a tile
  const int half = grp;
  const int hi = lane >> 5;
  const int logical = xcd_remap(block, total, geo.nxcd);
  const int bh = logical / num_qb;
  int qblk = logical - bh * num_qb;
  if (CAUSAL) qblk = num_qb - 1 - qblk;   // longest rows first
  const int q0 = qblk * kBlk;
  const int query = q0 + 32 * qw + (lane & 31);

  const HeadView hv = head_view<D>(geo, bh);
  const int N = hv.n;
  if (q0 >= N) return;   // varlen: past this sequence (whole workgroup)
  const size_t head = hv.q;
  const int head_bytes = N * D * 2;
  const char* Kh = reinterpret_cast<const char*>(K + hv.kv);
  const char* Vh = reinterpret_cast<const char*>(V + hv.kv);

  f16x8 qf[KSTEPS], gf[KSTEPS];   // B operands: Q^T and dO^T of this wave's queries
  load_row_operand<D>(Q + head, N, q0 + 32 * qw, lane, qf);
  load_row_operand<D>(dO + head, N, q0 + 32 * qw, lane, gf);
  const bool row_ok = query < N;
  const float nl = row_ok ? NL[hv.l + query] : 0.f;
  // dP^T starts from -D_i (a lane constant), so the chain yields dP - D_i.
  const float ndi = row_ok ? ND[hv.l + query] : 0.f;
  f32x16 acc[1][DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[0][db] = f32x16{};

  const int kv_end = CAUSAL ? min(N, q0 + kBlk) : N;
  const int T = (kv_end + kBQ - 1) / kBQ;   // >= 1
  // rows past N (last block only) and, causal, keys after the wave's first query
  const bool rows_edge = q0 + 32 * qw + 32 > N;

  const uint32_t lds0 = lds_addr(smem);
  auto stage_of = [&](int j) { return smem + (j % kPPStages) * STAGE; };
  // This group's half of tile t into stage st: 4 blocks of each of the 3
  // parts, PER consecutive ones per wave.
  auto issue_own = [&](int t, int st) {
    const uint32_t base = lds0 + st * STAGE;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int x = PER * qw + i;
      const int part = x / OWN;
      const int b = OWN * grp + x % OWN;
      uint32_t ko, vo;
      block_offsets<D>(b, lane, ko, vo);
      copy_block<D>(part < 2 ? Kh : Vh, head_bytes, t, base + part * TILE + b * 1024,
                    part == 1 ? vo : ko);
    }
  };
  // Copies run three tiles ahead (as in the dK/dV body).
  auto wait_next = [&](bool later_in_flight) {
    if (later_in_flight) wait_vmcnt<PER>();
    else wait_vmem();
  };
  issue_own(0, 0);
  if (T > 1) issue_own(1, 1);
  if (T > 2) issue_own(2, 2);
  wait_next(T > 2);
  __syncthreads();

  f32x16 s = {}, dp = {};
  f16x8 gb[2];
  f16x8 af[KSTEPS][2];   // A operands of the next score products (K, V rows)
  auto load_a = [&](const char* sb) {
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      af[kk][0] = load_k_frag<D>(sb, half, kk, lane);
      af[kk][1] = load_k_frag<D>(sb + 2 * TILE, half, kk, lane);
    }
  };
  auto mma_a = [&](int kk) {
    f32x16 dp0;
#pragma unroll
    for (int r = 0; r < 16; ++r) dp0[r] = ndi;
    s = mma32<BF16>(af[kk][0], qf[kk], kk == 0 ? f32x16{} : s);
    dp = mma32<BF16>(af[kk][1], gf[kk], kk == 0 ? dp0 : dp);
  };
  auto load_c = [&](const char* sb, int kk) {
    return load_v_frag<D>(sb + TILE, 2 * half + kk / DB, kk % DB, lane);
  };
  auto mphase = [&](int j, auto with_c, auto with_a) {
    constexpr bool WC = decltype(with_c)::value, WA = decltype(with_a)::value;
    const char* sc = stage_of(j + kPPStages - 1);
    f16x8 cf[KSTEPS];
    if constexpr (WC) {
      cf[0] = load_c(sc, 0);
      cf[1] = load_c(sc, 1);
    }
    static_for<0, KSTEPS>([&](auto ki) {
      constexpr int kk = decltype(ki)::value;
      if constexpr (WC && kk + 2 < KSTEPS) cf[kk + 2] = load_c(sc, kk + 2);
      if constexpr (WA) mma_a(kk);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (WC) acc[0][kk % DB] = mma32<BF16>(cf[kk], gb[kk / DB], acc[0][kk % DB]);
      __builtin_amdgcn_sched_barrier(0);
    });
    wait_next(j + 2 < T);
  };
  auto sphase = [&](int j) {
    if (j + 3 < T) issue_own(j + 3, (j + 3) % kPPStages);
    if (j + 1 < T) load_a(stage_of(j + 1));
    const int kt0 = j * kBQ;
    f32x16 p;
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = exp2_hw(fmaf(s[r], c, nl));
    const bool edge = rows_edge || (kt0 + 32 * half + 32 > N) ||
                      (CAUSAL && kt0 + 32 * half + 31 > q0 + 32 * qw);
    if (edge) {   // keys past N, rows past N, and (causal) keys after the row
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kidx = kt0 + 32 * half + 8 * (r >> 2) + 4 * hi + (r & 3);
        p[r] = ((kidx >= N) || (CAUSAL && kidx > query) || !row_ok) ? 0.f : p[r];
      }
    }
    f32x16 g;
#pragma unroll
    for (int r = 0; r < 16; ++r) g[r] = p[r] * dp[r];
#pragma unroll
    for (int h = 0; h < 2; ++h) gb[h] = pack_px<BF16>(g, h);
  };
  auto pin_s = [&] { asm volatile("" : "+v"(s), "+v"(dp)); };
  auto pin_p = [&] { asm volatile("" : "+v"(gb[0]), "+v"(gb[1])); };

  using BT = std::true_type;
  using BF = std::false_type;
  load_a(stage_of(0));
  if (grp == 1) __syncthreads();   // phase 0: group 1 waits
  mphase(0, BF{}, BT{});
  __syncthreads();
  pin_s();
  sphase(0);
  pin_p();
  __syncthreads();
  for (int j = 1; j < T; ++j) {
    mphase(j, BT{}, BT{});
    __syncthreads();
    pin_s();
    sphase(j);
    pin_p();
    __syncthreads();
  }
  mphase(T, BT{}, BF{});   // C of the last tile
  __syncthreads();
  if (grp == 0) __syncthreads();   // phase 2T + 1: group 0 waits
  group_reduce<1, DB>(smem, grp, qw, lane, acc);
  if (grp == 0) store_transposed<D>(dQ + head, N, q0 + 32 * qw, lane, acc[0], scale);
}

// ---------------------------------------------------------------------------
// D = 128. The phases are those of the D = 64 forms (M(j): C of tile j - 1,
// then A of tile j; S(j): B of tile j; the two groups one phase apart),
// fitted to D = 128's budgets:
//   * registers: the score products' A operands are read from LDS inside
//     the M phase (not prefetched into registers), and the M phase runs all
//     of C(j - 1) before A(j), so the packed P and dS of tile j - 1 are dead
//     before S and dP of tile j are live: the dK/dV body fits the 256 VGPRs
//     of two waves per SIMD without spilling (K^T, V^T and the two
//     accumulators alone take 192);
//   * LDS: the parts of a tile are freed at different times (the row-swizzled
//     A parts after M(j), the row vectors after S(j), the transposed C parts
//     after M(j + 1)), so each part has its own ring of slots and S(j) starts
//     A of tile j + 2, C of tile j + 1 and the row vectors of tile j + 2,
//     each into the slot its last reader has just left: two A slots, two C
//     slots and three row-vector slots (131 KiB at D = 128 for dK/dV) give
//     every copy two phases to land, issued from the VALU phase.
// A group copies and reads only its own 32-row half of every part (rows
// 32 g .. +31 are 1 KiB blocks 8 g .. 8 g + 7 in both swizzles).
// ---------------------------------------------------------------------------
template <int D>
constexpr int dkdv_pp128_smem() {
  constexpr int TILE = kBQ * D * 2;
  constexpr int RING = 2 * (2 * TILE) + 2 * (2 * TILE) + 3 * 1024;
  constexpr int RED = 4 * 2 * (D / 32) * 16 * 64 * 4;
  return RING > RED ? RING : RED;
}

template <int D>
constexpr int dq_pp128_smem() {
  constexpr int TILE = kBQ * D * 2;
  constexpr int RING = 2 * (2 * TILE) + 2 * TILE;
  constexpr int RED = 4 * (D / 32) * 16 * 64 * 4;
  return RING > RED ? RING : RED;
}

template <int D, bool CAUSAL, bool BF16>
__device__ __forceinline__ void dkdv_body_pp128(const f16* __restrict__ Q,
                                                const f16* __restrict__ K,
                                                const f16* __restrict__ V,
                                                const f16* __restrict__ dO,
                                                const float* __restrict__ NL,
                                                const float* __restrict__ ND,
                                                float* __restrict__ dK, float* __restrict__ dV,
                                                const Geom& geo, int num_kb, int total, float c,
                                                float scale, int block,
                                                char* smem /* dkdv_pp128_smem<D>() bytes */) {
  static_assert(D == 128, "a 32-row half of a tile is 8 blocks");
  constexpr int TILE = kBQ * D * 2;
  constexpr int BLOCKS = TILE / 1024;
  constexpr int OWN = BLOCKS / 2;              // blocks of a 32-row half
  constexpr int PER = OWN / 2;                 // blocks per wave of one part's half
  constexpr int KSTEPS = D / 16, DB = D / 32;
  constexpr int SLOT = 2 * TILE;               // A slot: Qk | dOk; C slot: Qv | dOv
  constexpr int C0 = 2 * SLOT;                 // C ring after the A ring
  constexpr int R0 = 4 * SLOT;                 // row vectors: group g L at +512 g, -D_i +256
  static_assert(R0 + 3 * 1024 <= dkdv_pp128_smem<D>() && dkdv_pp128_smem<D>() <= 160 * 1024,
                "ring inside the buffer, LDS");
  static_assert(2 * KSTEPS == 2 * 2 * DB, "C and A take the same number of steps");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kw = wave & 3;
  const int grp = wave >> 2;                   // also this group's query half of a tile
  const int qb = grp;
  const int hi = lane >> 5;
  const int logical = xcd_remap(block, total, geo.nxcd);
  const int bh = logical / num_kb;
  const int kb = logical - bh * num_kb;
  const int k0 = kb * kBlk;

  const HeadView hv = head_view<D>(geo, bh);
  const int N = hv.n;
  if (k0 >= N) return;   // varlen: past this sequence (whole workgroup)
  const size_t head = hv.q;
  const int head_bytes = N * D * 2;
  const char* Qh = reinterpret_cast<const char*>(Q + head);
  const char* Gh = reinterpret_cast<const char*>(dO + head);
  const float* Lh = NL + hv.l;
  const float* Dh = ND + hv.l;   // -D_i

  f16x8 kf[KSTEPS], vf[KSTEPS];   // B operands: K^T and V^T of this wave's keys
  load_row_operand<D>(K + hv.kv, N, k0 + 32 * kw, lane, kf);
  load_row_operand<D>(V + hv.kv, N, k0 + 32 * kw, lane, vf);
  f32x16 acc[2][DB];              // [0] = dV^T, [1] = dK^T (unscaled)
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    acc[0][db] = f32x16{};
    acc[1][db] = f32x16{};
  }

  const int n_qt = (N + kBQ - 1) / kBQ;
  const int t0 = CAUSAL ? k0 / kBQ : 0;   // earlier query tiles see none of these keys
  const int T = n_qt - t0;                 // tiles of this workgroup (>= 1)

  const uint32_t lds0 = lds_addr(smem);
  // Wave kw copies blocks 8 grp + 4 (kw & 1) .. +3 of part kw >> 1 (Q or dO)
  // of a ring; the per-lane offsets are recomputed per copy (volatile lane
  // id: held across the loop they would take registers the body needs).
  auto issue_part = [&](int t, uint32_t base, bool vsw) {
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const char* src = kw < 2 ? Qh : Gh;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int b = OWN * grp + PER * (kw & 1) + i;
      uint32_t ko, vo;
      block_offsets<D>(b, ln, ko, vo);
      copy_block<D>(src, head_bytes, t, base + (kw >> 1) * TILE + b * 1024, vsw ? vo : ko);
    }
  };
  auto issue_a = [&](int j) {   // A parts and row vectors of relative tile j
    issue_part(t0 + j, lds0 + (j & 1) * SLOT, false);
    const uint32_t rv = lds0 + R0 + (j % 3) * 1024 + 512 * grp;
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    if (kw == 0) copy_rowvec(Lh, N, t0 + j, rv, ln);
    if (kw == 1) copy_rowvec(Dh, N, t0 + j, rv + 256, ln);
  };
  auto issue_c = [&](int j) { issue_part(t0 + j, lds0 + C0 + (j & 1) * SLOT, true); };
  // Copies issued by this wave in one S phase: A (PER, + 1 row vector for
  // waves 0 and 1) and C (PER). The end of S(j) leaves S(j)'s copies in
  // flight and waits for the rest.
  auto wait_for = [&](bool a, bool cc) {
    if (a && cc) {
      if (kw < 2) wait_vmcnt<2 * PER + 1>();
      else wait_vmcnt<2 * PER>();
    } else if (a) {
      if (kw < 2) wait_vmcnt<PER + 1>();
      else wait_vmcnt<PER>();
    } else if (cc) {
      wait_vmcnt<PER>();
    } else {
      wait_vmem();
    }
  };
  issue_a(0);
  issue_c(0);
  if (T > 1) issue_a(1);
  wait_vmem();
  __syncthreads();

  f32x16 s = {}, dp = {};   // this wave's scores of its current tile
  f16x8 pb[2], gb[2];       // its packed P and dS (B operands of the two k-steps)
  // M phase of relative tile j: C of tile j - 1 (dV^T += dO^T P, dK^T += Q^T
  // dS; step x: k-step x / DB, d-block x % DB), then A of tile j (S = Q K^T,
  // dP = dO V^T; step x: k-step x). Operands two steps ahead.
  auto mphase = [&](int j, auto with_c, auto with_a) {
    constexpr bool WC = decltype(with_c)::value, WA = decltype(with_a)::value;
    constexpr int X0 = WC ? 0 : KSTEPS, X1 = WA ? 2 * KSTEPS : KSTEPS;
    const char* sc = smem + C0 + ((j + 1) & 1) * SLOT;   // C slot of tile j - 1
    const char* sa = smem + (j & 1) * SLOT;              // A slot of tile j
    f16x8 f[2 * KSTEPS][2];
    auto load = [&](auto xi) {
      constexpr int x = decltype(xi)::value;
      if constexpr (x < KSTEPS) {
        const int jj = 2 * qb + x / DB;
        f[x][0] = load_v_frag<D>(sc + TILE, jj, x % DB, lane);   // dO^T
        f[x][1] = load_v_frag<D>(sc, jj, x % DB, lane);          // Q^T
      } else {
        f[x][0] = load_k_frag<D>(sa, qb, x - KSTEPS, lane);          // Q rows
        f[x][1] = load_k_frag<D>(sa + TILE, qb, x - KSTEPS, lane);   // dO rows
      }
    };
    // Operands two steps ahead within each part; A's first two are loaded
    // where A starts, once C's last operands are consumed (loading them
    // during C measured 2 % slower at config 3).
    auto ahead = [&](auto xi) {
      constexpr int x = decltype(xi)::value;
      if constexpr (x < X1 && (x < KSTEPS || x >= KSTEPS + 2 || !WC)) load(xi);
    };
    static_for<X0, X0 + 2>(load);   // X1 - X0 >= KSTEPS
    static_for<X0, X1>([&](auto xi) {
      constexpr int x = decltype(xi)::value;
      if constexpr (WC && WA && x == KSTEPS) static_for<KSTEPS, KSTEPS + 2>(load);
      ahead(std::integral_constant<int, x + 2>{});
      if constexpr (x < KSTEPS) {
        acc[0][x % DB] = mma32<BF16>(f[x][0], pb[x / DB], acc[0][x % DB]);
        acc[1][x % DB] = mma32<BF16>(f[x][1], gb[x / DB], acc[1][x % DB]);
      } else {
        constexpr int kk = x - KSTEPS;
        s = mma32<BF16>(f[x][0], kf[kk], kk == 0 ? f32x16{} : s);
        dp = mma32<BF16>(f[x][1], vf[kk], kk == 0 ? f32x16{} : dp);
      }
      if constexpr (x + 1 == KSTEPS) __builtin_amdgcn_sched_barrier(0);   // C before A
    });
    __builtin_amdgcn_sched_barrier(0);   // keep every product in this phase
  };
  // S phase of relative tile j: the copies of A(j + 2), C(j + 1) and the row
  // vectors of j + 2, then P and dS into pb, gb; at the end, the wait for
  // the copies of S(j - 1) (A(j + 1), C(j): M(j + 1) reads them).
  auto sphase = [&](int j) {
    const bool ca = j + 2 < T, cc = j + 1 < T;
    if (cc) issue_c(j + 1);
    if (ca) issue_a(j + 2);
    const int qt0 = (t0 + j) * kBQ;
    const float* ls = reinterpret_cast<const float*>(smem + R0 + (j % 3) * 1024 + 512 * grp);
    const float* nds = ls + 64;
    f32x16 p, g;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const f32x4 lq = *reinterpret_cast<const f32x4*>(ls + 32 * qb + 8 * r4 + 4 * hi);
#pragma unroll
      for (int e = 0; e < 4; ++e) p[4 * r4 + e] = exp2_hw(fmaf(s[4 * r4 + e], c, lq[e]));
    }
    const bool edge = (qt0 + 32 * qb + 32 > N) || (CAUSAL && qt0 + 32 * qb < k0 + 32 * kw + 32);
    if (edge) {   // rows past N, and (causal) keys after the row
      int ln;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
      const int base = qt0 + 32 * qb + 4 * (ln >> 5);
      const int lim_n = N - base, lim_k = k0 + 32 * kw + (ln & 31) - base;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ro = 8 * (r >> 2) + (r & 3);
        p[r] = ((ro >= lim_n) || (CAUSAL && ro < lim_k)) ? 0.f : p[r];
      }
    }
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const f32x4 dq = *reinterpret_cast<const f32x4*>(nds + 32 * qb + 8 * r4 + 4 * hi);
#pragma unroll
      for (int e = 0; e < 4; ++e) g[4 * r4 + e] = p[4 * r4 + e] * (dp[4 * r4 + e] + dq[e]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      pb[h] = pack_px<BF16>(p, h);
      gb[h] = pack_px<BF16>(g, h);
    }
    wait_for(ca, cc);
  };
  auto pin_s = [&] { asm volatile("" : "+v"(s), "+v"(dp)); };
  auto pin_p = [&] { asm volatile("" : "+v"(pb[0]), "+v"(pb[1]), "+v"(gb[0]), "+v"(gb[1])); };

  using BT = std::true_type;
  using BF = std::false_type;
  if (grp == 1) __syncthreads();   // phase 0: group 1 waits
  mphase(0, BF{}, BT{});
  __syncthreads();
  pin_s();
  sphase(0);
  pin_p();
  __syncthreads();
  for (int j = 1; j < T; ++j) {
    mphase(j, BT{}, BT{});
    __syncthreads();
    pin_s();
    sphase(j);
    pin_p();
    __syncthreads();
  }
  mphase(T, BT{}, BF{});   // C of the last tile
  __syncthreads();
  if (grp == 0) __syncthreads();   // phase 2T + 1: group 0 waits
  int ln;   // the lane id again (not held across the loop)
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
  group_reduce<2, DB>(smem, grp, kw, ln, acc);
  if (grp == 0) {
    store_transposed<D>(dV + head, N, k0 + 32 * kw, ln, acc[0], 1.f);
    store_transposed<D>(dK + head, N, k0 + 32 * kw, ln, acc[1], scale);
  }
}

template <int D, bool CAUSAL, bool BF16>
__device__ __forceinline__ void dq_body_pp128(const f16* __restrict__ Q, const f16* __restrict__ K,
                                              const f16* __restrict__ V,
                                              const f16* __restrict__ dO,
                                              const float* __restrict__ NL,
                                              const float* __restrict__ ND, float* __restrict__ dQ,
                                              const Geom& geo, int num_qb, int total, float c,
                                              float scale, int block,
                                              char* smem /* dq_pp128_smem<D>() bytes */) {
  static_assert(D == 128, "a 32-row half of a tile is 8 blocks");
  constexpr int TILE = kBQ * D * 2;
  constexpr int BLOCKS = TILE / 1024;
  constexpr int OWN = BLOCKS / 2;              // blocks of a 32-row half
  constexpr int PA = OWN / 2, PC = OWN / 4;    // blocks per wave: A parts, C part
  constexpr int KSTEPS = D / 16, DB = D / 32;
  constexpr int SLOT = 2 * TILE;               // A slot: Kk | Vk
  constexpr int C0 = 2 * SLOT;                 // C slots (Kv), TILE bytes each
  static_assert(C0 + 2 * TILE <= dq_pp128_smem<D>() && dq_pp128_smem<D>() <= 160 * 1024 &&
                OWN % 4 == 0, "ring inside the buffer, LDS, copy split");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qw = wave & 3;
  const int grp = wave >> 2;                   // also this group's key half of a tile
  const int half = grp;
  const int hi = lane >> 5;
  const int logical = xcd_remap(block, total, geo.nxcd);
  const int bh = logical / num_qb;
  int qblk = logical - bh * num_qb;
  if (CAUSAL) qblk = num_qb - 1 - qblk;   // longest rows first
  const int q0 = qblk * kBlk;
  const int query = q0 + 32 * qw + (lane & 31);

  const HeadView hv = head_view<D>(geo, bh);
  const int N = hv.n;
  if (q0 >= N) return;   // varlen: past this sequence (whole workgroup)
  const size_t head = hv.q;
  const int head_bytes = N * D * 2;
  const char* Kh = reinterpret_cast<const char*>(K + hv.kv);
  const char* Vh = reinterpret_cast<const char*>(V + hv.kv);

  f16x8 qf[KSTEPS], gf[KSTEPS];   // B operands: Q^T and dO^T of this wave's queries
  load_row_operand<D>(Q + head, N, q0 + 32 * qw, lane, qf);
  load_row_operand<D>(dO + head, N, q0 + 32 * qw, lane, gf);
  const bool row_ok = query < N;
  const float nl = row_ok ? NL[hv.l + query] : 0.f;
  const float dq_i = row_ok ? ND[hv.l + query] : 0.f;   // -D_i
  f32x16 acc[1][DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[0][db] = f32x16{};

  const int kv_end = CAUSAL ? min(N, q0 + kBlk) : N;
  const int T = (kv_end + kBQ - 1) / kBQ;   // >= 1
  // rows past N (last block only) and, causal, keys after the wave's first query
  const bool rows_edge = q0 + 32 * qw + 32 > N;

  const uint32_t lds0 = lds_addr(smem);
  // A parts (Kk, Vk): wave qw copies blocks 8 grp + 4 (qw & 1) .. +3 of part
  // qw >> 1; C part (Kv): blocks 8 grp + 2 qw .. +1.
  auto issue_a = [&](int j) {
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const uint32_t base = lds0 + (j & 1) * SLOT + (qw >> 1) * TILE;
#pragma unroll
    for (int i = 0; i < PA; ++i) {
      const int b = OWN * grp + PA * (qw & 1) + i;
      uint32_t ko, vo;
      block_offsets<D>(b, ln, ko, vo);
      copy_block<D>(qw < 2 ? Kh : Vh, head_bytes, j, base + b * 1024, ko);
    }
  };
  auto issue_c = [&](int j) {
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    const uint32_t base = lds0 + C0 + (j & 1) * TILE;
#pragma unroll
    for (int i = 0; i < PC; ++i) {
      const int b = OWN * grp + PC * qw + i;
      uint32_t ko, vo;
      block_offsets<D>(b, ln, ko, vo);
      copy_block<D>(Kh, head_bytes, j, base + b * 1024, vo);
    }
  };
  auto wait_for = [&](bool a, bool cc) {
    if (a && cc) wait_vmcnt<PA + PC>();
    else if (a) wait_vmcnt<PA>();
    else if (cc) wait_vmcnt<PC>();
    else wait_vmem();
  };
  issue_a(0);
  issue_c(0);
  if (T > 1) issue_a(1);
  wait_vmem();
  __syncthreads();

  f32x16 s = {}, dp = {};
  f16x8 gb[2];
  // M phase of tile j: C of tile j - 1 (dQ^T += K^T dS^T; step x: k-step
  // x / DB, d-block x % DB), then A of tile j (S^T = K Q^T, dP^T = V dO^T).
  auto mphase = [&](int j, auto with_c, auto with_a) {
    constexpr bool WC = decltype(with_c)::value, WA = decltype(with_a)::value;
    constexpr int CX = 2 * DB;   // C steps
    constexpr int X0 = WC ? 0 : CX, X1 = WA ? CX + KSTEPS : CX;
    const char* sc = smem + C0 + ((j + 1) & 1) * TILE;   // C slot of tile j - 1
    const char* sa = smem + (j & 1) * SLOT;              // A slot of tile j
    f16x8 f[CX + KSTEPS][2];
    auto load = [&](auto xi) {
      constexpr int x = decltype(xi)::value;
      if constexpr (x < CX) {
        f[x][0] = load_v_frag<D>(sc, 2 * half + x / DB, x % DB, lane);   // K^T
      } else {
        f[x][0] = load_k_frag<D>(sa, half, x - CX, lane);          // K rows
        f[x][1] = load_k_frag<D>(sa + TILE, half, x - CX, lane);   // V rows
      }
    };
    static_for<X0, X0 + 2 < X1 ? X0 + 2 : X1>(load);
    static_for<X0, X1>([&](auto xi) {
      constexpr int x = decltype(xi)::value;
      if constexpr (x + 2 < X1) load(std::integral_constant<int, x + 2>{});
      if constexpr (x < CX) {
        acc[0][x % DB] = mma32<BF16>(f[x][0], gb[x / DB], acc[0][x % DB]);
      } else {
        constexpr int kk = x - CX;
        s = mma32<BF16>(f[x][0], qf[kk], kk == 0 ? f32x16{} : s);
        dp = mma32<BF16>(f[x][1], gf[kk], kk == 0 ? f32x16{} : dp);
      }
      if constexpr (x + 1 == CX) __builtin_amdgcn_sched_barrier(0);   // C before A
    });
    __builtin_amdgcn_sched_barrier(0);
  };
  auto sphase = [&](int j) {
    const bool ca = j + 2 < T, cc = j + 1 < T;
    if (cc) issue_c(j + 1);
    if (ca) issue_a(j + 2);
    const int kt0 = j * kBQ;
    f32x16 p;
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = exp2_hw(fmaf(s[r], c, nl));
    const bool edge = rows_edge || (kt0 + 32 * half + 32 > N) ||
                      (CAUSAL && kt0 + 32 * half + 31 > q0 + 32 * qw);
    if (edge) {   // keys past N, rows past N, and (causal) keys after the row
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kidx = kt0 + 32 * half + 8 * (r >> 2) + 4 * hi + (r & 3);
        p[r] = ((kidx >= N) || (CAUSAL && kidx > query) || !row_ok) ? 0.f : p[r];
      }
    }
    f32x16 g;
#pragma unroll
    for (int r = 0; r < 16; ++r) g[r] = p[r] * (dp[r] + dq_i);
#pragma unroll
    for (int h = 0; h < 2; ++h) gb[h] = pack_px<BF16>(g, h);
    wait_for(ca, cc);
  };
  auto pin_s = [&] { asm volatile("" : "+v"(s), "+v"(dp)); };
  auto pin_p = [&] { asm volatile("" : "+v"(gb[0]), "+v"(gb[1])); };

  using BT = std::true_type;
  using BF = std::false_type;
  if (grp == 1) __syncthreads();   // phase 0: group 1 waits
  mphase(0, BF{}, BT{});
  __syncthreads();
  pin_s();
  sphase(0);
  pin_p();
  __syncthreads();
  for (int j = 1; j < T; ++j) {
    mphase(j, BT{}, BT{});
    __syncthreads();
    pin_s();
    sphase(j);
    pin_p();
    __syncthreads();
  }
  mphase(T, BT{}, BF{});   // C of the last tile
  __syncthreads();
  if (grp == 0) __syncthreads();   // phase 2T + 1: group 0 waits
  group_reduce<1, DB>(smem, grp, qw, lane, acc);
  if (grp == 0) store_transposed<D>(dQ + head, N, q0 + 32 * qw, lane, acc[0], scale);
}

// dK/dV and dQ in one launch (both bodies take 8 waves and share one LDS
// buffer): blocks [0, total) run the dK/dV body, [total, 2 total) the dQ
// body. Each half is dispatched longest unit first, so a CU that
// finished a short dK/dV unit (late keys of a causal head) picks up a long
// dQ unit: the causal triangle's two halves even out across the CUs instead
// of each kernel waiting for its own longest unit.
template <int D, bool CAUSAL, bool BF16>
__global__ void __launch_bounds__(512)
fa_bwd_fused_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                    const f16* __restrict__ V, const f16* __restrict__ dO,
                    const float* __restrict__ NL, const float* __restrict__ ND,
                    float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ dQ,
                    Geom geo, int nb, int total, float c, float scale) {
  // One LDS buffer serves whichever body this workgroup runs.
  constexpr int SK = D == 64 ? dkdv_pp_smem<D>() : dkdv_pp128_smem<D>();
  constexpr int SQ = D == 64 ? dq_pp_smem<D>() : dq_pp128_smem<D>();
  __shared__ __attribute__((aligned(1024))) char smem[SK > SQ ? SK : SQ];
  const int blk = (int)blockIdx.x;
  if (blk < total) {
    if constexpr (D == 64) {
      dkdv_body_pp<D, CAUSAL, BF16>(Q, K, V, dO, NL, ND, dK, dV, geo, nb, total, c, scale, blk,
                                    smem);
    } else {
      dkdv_body_pp128<D, CAUSAL, BF16>(Q, K, V, dO, NL, ND, dK, dV, geo, nb, total, c, scale,
                                       blk, smem);
    }
  } else {
    if constexpr (D == 64) {
      dq_body_pp<D, CAUSAL, BF16>(Q, K, V, dO, NL, ND, dQ, geo, nb, total, c, scale, blk - total,
                                  smem);
    } else {
      dq_body_pp128<D, CAUSAL, BF16>(Q, K, V, dO, NL, ND, dQ, geo, nb, total, c, scale,
                                     blk - total, smem);
    }
  }
}

// GQA: dK, dV of KV head hk = sum over its `group` query heads of the
// per-query-head partials (fp32 [B*H, N*D] -> [B*Hkv, N*D]), four floats per
// thread.
__global__ void __launch_bounds__(256)
fa_bwd_group_sum_kernel(const float* __restrict__ part, float* __restrict__ out, int64_t head_elems,
                        int64_t kv_heads, int group) {
  const int64_t i4 = (int64_t)blockIdx.x * 256 + threadIdx.x;   // float4 index in out
  const int64_t n4 = kv_heads * head_elems / 4;
  if (i4 >= n4) return;
  const int64_t hk = (i4 * 4) / head_elems;
  const int64_t e = i4 * 4 - hk * head_elems;
  const f32x4* src = reinterpret_cast<const f32x4*>(part + (hk * group) * head_elems + e);
  const int64_t stride4 = head_elems / 4;
  f32x4 acc = src[0];
  for (int j = 1; j < group; ++j) acc += src[j * stride4];
  reinterpret_cast<f32x4*>(out)[i4] = acc;
}

// The three passes (-D_i and -L log2 e, dK/dV, dQ) and, with H_kv < H, the
// group sums. geo is dense (B heads of N rows per head) or varlen (heads of
// geo.total packed rows; units = B*H (b, h) pairs either way); `rows` is the
// number of L rows: B*H*N dense, H*total varlen.
template <int D, bool CAUSAL, bool BF16>
static hipError_t launch_bwd(const void* q, const void* k, const void* v, const void* o,
                             const void* dout, const float* lse, float* dq, float* dk, float* dv,
                             float* ws, const Geom& geo, int64_t units, int64_t rows,
                             int64_t out_heads, int64_t head_rows, hipStream_t s) {
  const float scale = (float)(1.0 / sqrt((double)D));
  const float c = scale * kLog2e;
  const f16* Q = (const f16*)q;
  const f16* K = (const f16*)k;
  const f16* V = (const f16*)v;
  const f16* O = (const f16*)o;
  const f16* G = (const f16*)dout;
  const int group = geo.group;
  float* nd = ws;
  float* nl = ws + rows;
  // GQA: per-query-head dK/dV partials in the workspace, summed per KV head.
  const int64_t part0 = (2 * rows + 3) / 4 * 4;   // 16-byte aligned start of the partials
  float* dk_q = group == 1 ? dk : ws + part0;
  float* dv_q = group == 1 ? dv : ws + part0 + rows * D;
  hipLaunchKernelGGL((fa_bwd_di_kernel<D, BF16>), dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, s, O,
                     G, lse, nd, nl, rows);
  const int nb = (geo.N + kBlk - 1) / kBlk;
  const int total = (int)(units * nb);
  // dK/dV and dQ in one launch. A causal head's short and long units even
  // out across the CUs (B1 H8 N4096 D128: 0.237 -> 0.165 ms against two
  // launches); with units of one length the one launch measured level with
  // two or slightly ahead (D = 128 non-causal, B1 H8 N4096 256.4 -> 254.5 us,
  // B4 H16 N4096 1981.8 -> 1972.3 us; same gradients bit for bit).
  hipLaunchKernelGGL((fa_bwd_fused_kernel<D, CAUSAL, BF16>), dim3(2 * total), dim3(512), 0, s,
                     Q, K, V, G, nl, nd, dk_q, dv_q, dq, geo, nb, total, c, scale);
  if (group > 1) {
    // out_heads KV heads of head_rows rows, each the sum of `group`
    // consecutive query heads' partials
    const int64_t head_elems = head_rows * D;
    const int64_t n4 = out_heads * head_elems / 4;
    const dim3 grid((unsigned)((n4 + 255) / 256));
    hipLaunchKernelGGL(fa_bwd_group_sum_kernel, grid, dim3(256), 0, s, dk_q, dk, head_elems,
                       out_heads, group);
    hipLaunchKernelGGL(fa_bwd_group_sum_kernel, grid, dim3(256), 0, s, dv_q, dv, head_elems,
                       out_heads, group);
  }
  return hipGetLastError();
}

}  // namespace bwd
}  // namespace fa

extern "C" int64_t fa_bwd_workspace_floats(int64_t B, int64_t H, int64_t N) {
  if (B <= 0 || H <= 0 || N <= 0) return 0;
  return 2 * B * H * N;   // -D_i, then -L log2(e)
}

extern "C" int64_t fa_bwd_gqa_workspace_floats(int64_t B, int64_t H, int64_t H_kv, int64_t N,
                                               int64_t D) {
  if (B <= 0 || H <= 0 || N <= 0 || H_kv <= 0 || H % H_kv != 0) return 0;
  // -D_i and -L log2(e), then (GQA only, from a 16-byte boundary) the
  // per-query-head dK and dV partials
  if (H_kv == H) return 2 * B * H * N;
  return (2 * B * H * N + 3) / 4 * 4 + 2 * B * H * N * D;
}

namespace fa {
namespace bwd {
template <bool BF16>
static int bwd_run(const void* q, const void* k, const void* v, const void* o, const void* dout,
                   const float* lse, float* dq, float* dk, float* dv, float* workspace,
                   const Geom& geo_in, int64_t units, int64_t rows, int64_t out_heads,
                   int64_t head_rows, int64_t D, int causal, void* stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  Geom geo = geo_in;
  geo.nxcd = stream_topology(s).xcds;
  hipError_t e;
  if (D == 64) {
    e = causal ? launch_bwd<64, true, BF16>(q, k, v, o, dout, lse, dq, dk, dv, workspace, geo, units, rows, out_heads, head_rows, s)
               : launch_bwd<64, false, BF16>(q, k, v, o, dout, lse, dq, dk, dv, workspace, geo, units, rows, out_heads, head_rows, s);
  } else {
    e = causal ? launch_bwd<128, true, BF16>(q, k, v, o, dout, lse, dq, dk, dv, workspace, geo, units, rows, out_heads, head_rows, s)
               : launch_bwd<128, false, BF16>(q, k, v, o, dout, lse, dq, dk, dv, workspace, geo, units, rows, out_heads, head_rows, s);
  }
  return e == hipSuccess ? FA_OK : -(int)e;
}

static int bwd_gqa(bool bf16, const void* q, const void* k, const void* v, const void* o,
                   const void* dout, const float* lse, float* dq, float* dk, float* dv,
                   float* workspace, int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D,
                   int causal, void* stream) {
  int st = fa_validate_bwd(q, k, v, o, dout, lse, dq, dk, dv, workspace, B, H, N, D);
  if (st != FA_OK) return st;
  if (H_kv <= 0 || H % H_kv != 0) return FA_ERR_KV_HEADS;
  // the partials are written and read as 16-byte vectors
  if (H_kv != H && (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0) return FA_ERR_ALIGNMENT;
  const Geom geo{nullptr, (int)N, (int)H, (int)(H / H_kv), 0, 0, 0};   // nxcd: launcher
  return bf16 ? bwd_run<true>(q, k, v, o, dout, lse, dq, dk, dv, workspace, geo, B * H,
                              B * H * N, B * H_kv, N, D, causal, stream)
              : bwd_run<false>(q, k, v, o, dout, lse, dq, dk, dv, workspace, geo, B * H,
                               B * H * N, B * H_kv, N, D, causal, stream);
}
}  // namespace bwd
}  // namespace fa

extern "C" int fa_bwd_f16(const void* q, const void* k, const void* v, const void* o,
                          const void* dout, const float* lse, float* dq, float* dk, float* dv,
                          float* workspace, int64_t B, int64_t H, int64_t N, int64_t D, int causal,
                          void* stream) {
  return fa::bwd::bwd_gqa(false, q, k, v, o, dout, lse, dq, dk, dv, workspace, B, H, H, N, D,
                          causal, stream);
}

extern "C" int fa_bwd_gqa_f16(const void* q, const void* k, const void* v, const void* o,
                              const void* dout, const float* lse, float* dq, float* dk, float* dv,
                              float* workspace, int64_t B, int64_t H, int64_t H_kv, int64_t N,
                              int64_t D, int causal, void* stream) {
  return fa::bwd::bwd_gqa(false, q, k, v, o, dout, lse, dq, dk, dv, workspace, B, H, H_kv, N, D,
                          causal, stream);
}

extern "C" int fa_bwd_bf16(const void* q, const void* k, const void* v, const void* o,
                           const void* dout, const float* lse, float* dq, float* dk, float* dv,
                           float* workspace, int64_t B, int64_t H, int64_t H_kv, int64_t N,
                           int64_t D, int causal, void* stream) {
  return fa::bwd::bwd_gqa(true, q, k, v, o, dout, lse, dq, dk, dv, workspace, B, H, H_kv, N, D,
                          causal, stream);
}

extern "C" int fa_bwd_varlen_f16(const void* q, const void* k, const void* v, const void* o,
                                 const void* dout, const float* lse, float* dq, float* dk,
                                 float* dv, float* workspace, const int32_t* cu_seqlens,
                                 int64_t B, int64_t H, int64_t H_kv, int64_t max_seqlen,
                                 int64_t total, int64_t D, int causal, void* stream) {
  const int st = fa_validate_bwd_varlen(q, k, v, o, dout, lse, dq, dk, dv, workspace, cu_seqlens,
                                        B, H, H_kv, max_seqlen, total, D);
  if (st != FA_OK) return st;
  if (total == 0) return FA_OK;
  if (H_kv != H && (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0) return FA_ERR_ALIGNMENT;
  const fa::Geom geo{cu_seqlens, (int)max_seqlen, (int)H, (int)(H / H_kv), (int)total,
                       (int)B, 0};   // nxcd: launcher
  return fa::bwd::bwd_run<false>(q, k, v, o, dout, lse, dq, dk, dv, workspace, geo, B * H,
                                 H * total, H_kv, total, D, causal, stream);
}
