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
//   fa_bwd_dkdv_kernel  a workgroup owns 128 keys (32 per wave, K and V as
//                       register operands) and streams 64-query tiles of Q
//                       and dO (plus L, D_i) through a double-buffered LDS
//                       ring: S = Q K^T, dP = dO V^T, P = exp2(S c - L log2e),
//                       dS = P (dP - D_i), dV^T += dO^T P, dK^T += Q^T dS
//   fa_bwd_dq_kernel    a workgroup owns 128 queries (32 per wave, Q and dO
//                       as register operands) and streams 64-key tiles of K
//                       and V: S^T = K Q^T, dP^T = V dO^T, dS^T as above,
//                       dQ^T += K^T dS^T
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
// dK, dV. Workgroup = 4 G waves, 128 keys of one (b, h): wave w owns keys
// k0 + 32 (w % 4) .. +31 and, with G = 2, query half w / 4 of every tile (the
// two groups' partial sums are added at the end). Query tiles of 64 rows
// stream through 2 LDS stages; each stage holds Q and dO twice (row swizzle,
// transposed swizzle) and 64 floats each of NL and -D_i.
// ---------------------------------------------------------------------------
// LDS bytes of the dK/dV body: two stages, or the group reduction's
// 2 (dK, dV) x DB x 16 floats per lane of 4 waves, whichever is larger.
template <int D, int G>
constexpr int dkdv_smem() {
  constexpr int STAGE = 4 * (kBQ * D * 2) + 2048;   // Qk | Qv | dOk | dOv | NL | -D_i
  constexpr int RED = (G - 1) * 4 * 2 * (D / 32) * 16 * 64 * 4;
  return 2 * STAGE > RED ? 2 * STAGE : RED;
}

template <int D, bool CAUSAL, int G, bool BF16>
__device__ __forceinline__ void dkdv_body(const f16* __restrict__ Q, const f16* __restrict__ K,
                                          const f16* __restrict__ V, const f16* __restrict__ dO,
                                          const float* __restrict__ NL,
                                          const float* __restrict__ ND, float* __restrict__ dK,
                                          float* __restrict__ dV, const Geom& geo, int num_kb,
                                          int total, float c, float scale, int block,
                                          char* smem /* dkdv_smem<D, G>() bytes, 1 KiB aligned */) {
  constexpr int TILE = kBQ * D * 2;
  constexpr int BLOCKS = TILE / 1024;
  constexpr int KSTEPS = D / 16, DB = D / 32;
  constexpr int STAGE = 4 * TILE + 2048;       // Qk | Qv | dOk | dOv | NL | -D_i
  constexpr int WAVES = 4 * G;
  constexpr int LOADS = 4 * BLOCKS / WAVES;    // tile blocks per wave per stage
  static_assert(4 * BLOCKS % WAVES == 0, "copy blocks split evenly over the waves");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kw = wave & 3;
  const int grp = wave >> 2;
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
  const size_t kv_head = hv.kv;   // GQA: K/V head of this query head
  load_row_operand<D>(K + kv_head, N, k0 + 32 * kw, lane, kf);
  load_row_operand<D>(V + kv_head, N, k0 + 32 * kw, lane, vf);
  f32x16 acc[2][DB];              // [0] = dV^T, [1] = dK^T (unscaled)
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    acc[0][db] = f32x16{};
    acc[1][db] = f32x16{};
  }

  // Block b = i * WAVES + wave of a stage: part b / BLOCKS of {Qk, Qv, dOk,
  // dOv}, block b % BLOCKS of that tile. The per-lane source offsets are
  // recomputed at each copy from a lane id the compiler cannot hoist: held
  // across the loop they are the first registers spilled at D = 128, and a
  // reload before each copy waits for every copy before it.
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int t, int st) {
    const uint32_t base = lds0 + st * STAGE;
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int b = i * WAVES + wave;
      const int part = b / BLOCKS;
      uint32_t ko, vo;
      block_offsets<D>(b % BLOCKS, ln, ko, vo);
      copy_block<D>(part < 2 ? Qh : Gh, head_bytes, t, base + part * TILE + (b % BLOCKS) * 1024,
                    (part & 1) ? vo : ko);
    }
    if (wave == 0) copy_rowvec(Lh, N, t, base + 4 * TILE, ln);
    if (wave == 1) copy_rowvec(Dh, N, t, base + 4 * TILE + 1024, ln);
  };

  // One 32-query block qb of the tile at sb: S = Q K^T and dP = dO V^T
  // (C layout: register r holds query qt0 + 32 qb + 8 (r/4) + 4 hi + r%4,
  // lane l key l%32), then P, dS and the two gradient products. `mid` runs
  // once the score products are issued (the next tile's copies go there, so
  // their issue overlaps the matrix cores).
  auto body = [&](const char* sb, int qt0, int qb, bool edge, auto mid) {
    const char* qk = sb;
    const char* qv = sb + TILE;
    const char* gk = sb + 2 * TILE;
    const char* gv = sb + 3 * TILE;
    const float* ls = reinterpret_cast<const float*>(sb + 4 * TILE);
    const float* ds = reinterpret_cast<const float*>(sb + 4 * TILE + 1024);
    f32x16 s = {}, dp = {};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      s = mma32<BF16>(load_k_frag<D>(qk, qb, kk, lane), kf[kk], s);
      dp = mma32<BF16>(load_k_frag<D>(gk, qb, kk, lane), vf[kk], dp);
      // D = 128: bound the operand reads in flight (registers are the limit)
      if constexpr (D == 128) if (kk % 2 == 1) __builtin_amdgcn_sched_barrier(0);
    }
    mid();
    f32x16 p, g;
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const f32x4 lq = *reinterpret_cast<const f32x4*>(ls + 32 * qb + 8 * r4 + 4 * hi);
#pragma unroll
      for (int e = 0; e < 4; ++e) p[4 * r4 + e] = exp2_hw(fmaf(s[4 * r4 + e], c, lq[e]));
    }
    if (edge) {   // rows past N, and (causal) keys after the row
      // Register r holds query base + 8 (r/4) + r%4: compare that constant
      // offset against two per-lane limits. The lane id is read here again
      // (volatile, so the key index is not held across the loop: at D = 128
      // that register is one of those the causal instance would spill).
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
      const f32x4 dq = *reinterpret_cast<const f32x4*>(ds + 32 * qb + 8 * r4 + 4 * hi);
#pragma unroll
      for (int e = 0; e < 4; ++e) g[4 * r4 + e] = p[4 * r4 + e] * (dp[4 * r4 + e] + dq[e]);
    }
    // dV^T += dO^T P and dK^T += Q^T dS over the two 16-query k-steps.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = 2 * qb + h;
      const f16x8 pb = pack_px<BF16>(p, h);
      const f16x8 gb = pack_px<BF16>(g, h);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        acc[0][db] = mma32<BF16>(load_v_frag<D>(gv, j, db, lane), pb, acc[0][db]);
        acc[1][db] = mma32<BF16>(load_v_frag<D>(qv, j, db, lane), gb, acc[1][db]);
      }
    }
  };

  const int n_qt = (N + kBQ - 1) / kBQ;
  const int t0 = CAUSAL ? k0 / kBQ : 0;   // earlier query tiles see none of these keys
  if (t0 < n_qt) {
    issue(t0, 0);
    wait_vmem();
    __syncthreads();
  }
  for (int t = t0; t < n_qt; ++t) {
    const int st = (t - t0) & 1;
    const char* sb = smem + st * STAGE;
    const int qt0 = t * kBQ;
    auto prefetch = [&] {
      if (t + 1 < n_qt) issue(t + 1, st ^ 1);
    };
#pragma unroll
    for (int i = 0; i < 2 / G; ++i) {
      const int qb = G == 2 ? grp : i;
      // masking only where a query is past N or precedes one of the keys
      const bool edge = (qt0 + 32 * qb + 32 > N) ||
                        (CAUSAL && qt0 + 32 * qb < k0 + 32 * kw + 32);
      if (i == 0) body(sb, qt0, qb, edge, prefetch);
      else body(sb, qt0, qb, edge, [] {});
    }
    wait_vmem();
    __syncthreads();
  }
  if constexpr (G == 2) group_reduce<2, DB>(smem, grp, kw, lane, acc);
  if (grp == 0) {
    store_transposed<D>(dV + head, N, k0 + 32 * kw, lane, acc[0], 1.f);
    store_transposed<D>(dK + head, N, k0 + 32 * kw, lane, acc[1], scale);
  }
}

// ---------------------------------------------------------------------------
// dQ. Workgroup = 4 G waves, 128 queries of one (b, h): wave w owns queries
// q0 + 32 (w % 4) .. +31 (Q^T and dO^T as register B operands, NL and -D_i as
// lane constants) and, with G = 2, key half w / 4 of every tile. Key tiles of
// 64 rows stream through 2 LDS stages, each holding K twice (row swizzle,
// transposed swizzle) and V once (row swizzle).
// ---------------------------------------------------------------------------
// LDS bytes of the dQ body: two stages, or the group reduction's DB x 16
// floats per lane of 4 waves, whichever is larger.
template <int D, int G>
constexpr int dq_smem() {
  constexpr int STAGE = 3 * (kBQ * D * 2);    // Kk | Kv | Vk
  constexpr int RED = (G - 1) * 4 * (D / 32) * 16 * 64 * 4;
  return 2 * STAGE > RED ? 2 * STAGE : RED;
}

template <int D, bool CAUSAL, int G, bool BF16>
__device__ __forceinline__ void dq_body(const f16* __restrict__ Q, const f16* __restrict__ K,
                                        const f16* __restrict__ V, const f16* __restrict__ dO,
                                        const float* __restrict__ NL,
                                        const float* __restrict__ ND, float* __restrict__ dQ,
                                        const Geom& geo, int num_qb, int total, float c,
                                        float scale, int block,
                                        char* smem /* dq_smem<D, G>() bytes, 1 KiB aligned */) {
  constexpr int TILE = kBQ * D * 2;
  constexpr int BLOCKS = TILE / 1024;
  constexpr int KSTEPS = D / 16, DB = D / 32;
  constexpr int STAGE = 3 * TILE;              // Kk | Kv | Vk
  constexpr int NBLK = 3 * BLOCKS;
  constexpr int WAVES = 4 * G;
  constexpr int LOADS = (NBLK + WAVES - 1) / WAVES;   // tile blocks per wave per stage

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qw = wave & 3;
  const int grp = wave >> 2;
  const int hi = lane >> 5;
  const int logical = xcd_remap(block, total, geo.nxcd);
  const int bh = logical / num_qb;
  int qb = logical - bh * num_qb;
  if (CAUSAL) qb = num_qb - 1 - qb;   // longest rows first
  const int q0 = qb * kBlk;
  const int query = q0 + 32 * qw + (lane & 31);

  const HeadView hv = head_view<D>(geo, bh);
  const int N = hv.n;
  if (q0 >= N) return;   // varlen: past this sequence (whole workgroup)
  const size_t head = hv.q;
  const int head_bytes = N * D * 2;
  const size_t kv_head = hv.kv;   // GQA: K/V head of this query head
  const char* Kh = reinterpret_cast<const char*>(K + kv_head);
  const char* Vh = reinterpret_cast<const char*>(V + kv_head);

  f16x8 qf[KSTEPS], gf[KSTEPS];   // B operands: Q^T and dO^T of this wave's queries
  load_row_operand<D>(Q + head, N, q0 + 32 * qw, lane, qf);
  load_row_operand<D>(dO + head, N, q0 + 32 * qw, lane, gf);
  const bool row_ok = query < N;
  const float nl = row_ok ? NL[hv.l + query] : 0.f;
  const float dq_i = row_ok ? ND[hv.l + query] : 0.f;   // -D_i
  f32x16 acc[1][DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[0][db] = f32x16{};

  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int t, int st) {   // offsets recomputed per copy (see the dK/dV body)
    const uint32_t base = lds0 + st * STAGE;
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int b = i * WAVES + wave;
      if (b < NBLK) {   // wave-uniform
        const int part = b / BLOCKS;
        uint32_t ko, vo;
        block_offsets<D>(b % BLOCKS, ln, ko, vo);
        copy_block<D>(part < 2 ? Kh : Vh, head_bytes, t, base + part * TILE + (b % BLOCKS) * 1024,
                      part == 1 ? vo : ko);
      }
    }
  };

  // One 32-key half of the tile at kt: S^T = K Q^T and dP^T = V dO^T
  // (register r holds key kt0 + 32 half + 8 (r/4) + 4 hi + r%4, lane l query
  // l%32), then dS^T and dQ^T += K^T dS^T. `mid` runs once the score
  // products are issued.
  auto body = [&](const char* kt, int kt0, int half, bool edge, auto mid) {
    const char* kk_t = kt;
    const char* kv_t = kt + TILE;
    const char* vk_t = kt + 2 * TILE;
    f32x16 s = {}, dp = {};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      s = mma32<BF16>(load_k_frag<D>(kk_t, half, kk, lane), qf[kk], s);
      dp = mma32<BF16>(load_k_frag<D>(vk_t, half, kk, lane), gf[kk], dp);
    }
    mid();
    f32x16 p;
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = exp2_hw(fmaf(s[r], c, nl));
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
    for (int h = 0; h < 2; ++h) {
      const int j = 2 * half + h;
      const f16x8 gb = pack_px<BF16>(g, h);
#pragma unroll
      for (int db = 0; db < DB; ++db)
        acc[0][db] = mma32<BF16>(load_v_frag<D>(kv_t, j, db, lane), gb, acc[0][db]);
    }
  };

  const int kv_end = CAUSAL ? min(N, q0 + kBlk) : N;
  const int n_kt = (kv_end + kBQ - 1) / kBQ;
  // rows past N (last block only) and, causal, keys after the wave's first query
  const bool rows_edge = q0 + 32 * qw + 32 > N;
  issue(0, 0);
  wait_vmem();
  __syncthreads();
  for (int t = 0; t < n_kt; ++t) {
    const int st = t & 1;
    const char* kt = smem + st * STAGE;
    const int kt0 = t * kBQ;
    auto prefetch = [&] {
      if (t + 1 < n_kt) issue(t + 1, st ^ 1);
    };
#pragma unroll
    for (int i = 0; i < 2 / G; ++i) {
      const int half = G == 2 ? grp : i;
      const bool edge = rows_edge || (kt0 + 32 * half + 32 > N) ||
                        (CAUSAL && kt0 + 32 * half + 31 > q0 + 32 * qw);
      if (i == 0) body(kt, kt0, half, edge, prefetch);
      else body(kt, kt0, half, edge, [] {});
    }
    wait_vmem();
    __syncthreads();
  }
  if constexpr (G == 2) group_reduce<1, DB>(smem, grp, qw, lane, acc);
  if (grp == 0) store_transposed<D>(dQ + head, N, q0 + 32 * qw, lane, acc[0], scale);
}

// ---------------------------------------------------------------------------
// Ping-pong forms of the two bodies (D = 64, 8 waves): the two wave groups of
// a workgroup hold the same keys (dK/dV) or queries (dQ), each takes one
// 32-row half of every tile, and they run one phase apart. Each tile's work
// splits into the score products A (S and dP MFMAs), the VALU part B (P,
// dS, packed as B operands) and the gradient products C; a group's matrix
// phase M(j) issues C of its tile j - 1 and A of tile j, its softmax phase
// S(j) runs B of tile j. In every phase one group is in M and the other in
// S, so each SIMD overlaps one wave's MFMAs with the other's VALU work (the
// lockstep bodies above run the two waves' MFMAs and VALU at the same time):
//
//   phase      2j          2j+1        ...   2T          2T+1
//   group 0    M(j)        S(j)              C(T-1)      -
//   group 1    S(j-1)      M(j)              S(T-1)      C(T-1)
//
// A group reads only its own 32-row half of every tile (rows 32 g .. +31 of
// each part are its 1 KiB blocks 4 g .. 4 g + 3 in both swizzles), so it
// copies only that half, and the row vectors into slots of its own: the
// groups share no staged data, and the barriers keep them one phase apart
// and sync each group's four waves on their copies. Tile j's stage is read
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

// GQA: dK, dV of KV head hk = sum over its `group` query heads of the
// per-query-head partials (fp32 [B*H, N*D] -> [B*Hkv, N*D]), four floats per
// thread.
template <int D, bool CAUSAL, int G, bool BF16>
__global__ void __launch_bounds__(256 * G)
fa_bwd_dkdv_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                   const f16* __restrict__ V, const f16* __restrict__ dO,
                   const float* __restrict__ NL, const float* __restrict__ ND,
                   float* __restrict__ dK, float* __restrict__ dV, Geom geo, int num_kb,
                   int total, float c, float scale) {
  __shared__ __attribute__((aligned(1024))) char smem[dkdv_smem<D, G>()];
  dkdv_body<D, CAUSAL, G, BF16>(Q, K, V, dO, NL, ND, dK, dV, geo, num_kb, total, c, scale,
                                (int)blockIdx.x, smem);
}

template <int D, bool CAUSAL, int G, bool BF16>
__global__ void __launch_bounds__(256 * G)
fa_bwd_dq_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                 const f16* __restrict__ V, const f16* __restrict__ dO,
                 const float* __restrict__ NL, const float* __restrict__ ND,
                 float* __restrict__ dQ, Geom geo, int num_qb, int total, float c,
                 float scale) {
  __shared__ __attribute__((aligned(1024))) char smem[dq_smem<D, G>()];
  dq_body<D, CAUSAL, G, BF16>(Q, K, V, dO, NL, ND, dQ, geo, num_qb, total, c, scale,
                              (int)blockIdx.x, smem);
}

// dK/dV and dQ in one launch (both bodies take 8 waves and share one LDS
// buffer): blocks [0, total) are the dK/dV kernel's, [total, 2 total) the dQ
// kernel's. Each
// half is dispatched longest unit first, so a CU that finished a short dK/dV
// unit (late keys of a causal head) picks up a long dQ unit: the causal
// triangle's two halves even out across the CUs instead of each kernel
// waiting for its own longest unit.
template <int D, bool CAUSAL, bool BF16>
__global__ void __launch_bounds__(512)
fa_bwd_fused_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
                    const f16* __restrict__ V, const f16* __restrict__ dO,
                    const float* __restrict__ NL, const float* __restrict__ ND,
                    float* __restrict__ dK, float* __restrict__ dV, float* __restrict__ dQ,
                    Geom geo, int nb, int total, float c, float scale) {
  // One LDS buffer serves whichever body this workgroup runs. D = 64 runs the
  // ping-pong bodies (their 4-stage rings fit the LDS only there).
  constexpr bool PP = D == 64;
  constexpr int SK = PP ? dkdv_pp_smem<D>() : dkdv_smem<D, 2>();
  constexpr int SQ = PP ? dq_pp_smem<D>() : dq_smem<D, 2>();
  __shared__ __attribute__((aligned(1024))) char smem[SK > SQ ? SK : SQ];
  const int blk = (int)blockIdx.x;
  if (blk < total) {
    if constexpr (PP) {
      dkdv_body_pp<D, CAUSAL, BF16>(Q, K, V, dO, NL, ND, dK, dV, geo, nb, total, c, scale, blk,
                                    smem);
    } else {
      dkdv_body<D, CAUSAL, 2, BF16>(Q, K, V, dO, NL, ND, dK, dV, geo, nb, total, c, scale, blk,
                                    smem);
    }
  } else {
    if constexpr (PP) {
      dq_body_pp<D, CAUSAL, BF16>(Q, K, V, dO, NL, ND, dQ, geo, nb, total, c, scale, blk - total,
                                  smem);
    } else {
      dq_body<D, CAUSAL, 2, BF16>(Q, K, V, dO, NL, ND, dQ, geo, nb, total, c, scale, blk - total,
                                  smem);
    }
  }
}

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

// Wave groups per workgroup: two (the second group takes the other half of
// every tile, so the grid stays one workgroup per 128 rows and the SIMDs get
// a second wave to overlap). At D = 128 the dK/dV body then fills the 256
// VGPRs two waves per SIMD allow (no spill once the copy offsets are
// recomputed per copy); measured on B4 H16 N4096 causal, two groups beat one
// (281 VGPRs, one wave per SIMD) by 9%.

template <int D>
constexpr int kDkdvGroups = 2;
template <int D>
constexpr int kDqGroups = 2;

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
  constexpr int GK = kDkdvGroups<D>, GQ = kDqGroups<D>;
  bool launched = false;
  // One launch where it pays (measured): at D = 64 always; at D = 128 for
  // causal heads, where a short wave of workgroups cannot even out the
  // triangle on its own (B1 H8 N4096: 0.237 -> 0.165 ms) and larger grids
  // run the same in one launch as in two (B2 H8 N4096 303.2 / 301.1 us,
  // B4 H8 600.8 / 597.2 us, B4 H16 1237.2 / 1237.9 us, B1 H16 N8192
  // 1082.9 / 1081.2 us; same gradients bit for bit). Non-causal D = 128
  // heads, whose units are all the same length, keep the two launches
  // (B4 H16 N4096: 2.36 vs 2.50 ms).
  if constexpr (GK == 2 && GQ == 2 && (D == 64 || CAUSAL)) {
    hipLaunchKernelGGL((fa_bwd_fused_kernel<D, CAUSAL, BF16>), dim3(2 * total), dim3(512), 0,
                       s, Q, K, V, G, nl, nd, dk_q, dv_q, dq, geo, nb, total, c, scale);
    launched = true;
  }
  if (!launched) {
    hipLaunchKernelGGL((fa_bwd_dkdv_kernel<D, CAUSAL, GK, BF16>), dim3(total), dim3(256 * GK), 0, s, Q, K,
                       V, G, nl, nd, dk_q, dv_q, geo, nb, total, c, scale);
    hipLaunchKernelGGL((fa_bwd_dq_kernel<D, CAUSAL, GQ, BF16>), dim3(total), dim3(256 * GQ), 0, s, Q, K, V,
                       G, nl, nd, dq, geo, nb, total, c, scale);
  }
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
  const Geom geo{nullptr, (int)N, (int)H, (int)(H / H_kv), 0};
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
  const fa::Geom geo{cu_seqlens, (int)max_seqlen, (int)H, (int)(H / H_kv), (int)total, (int)B};
  return fa::bwd::bwd_run<false>(q, k, v, o, dout, lse, dq, dk, dv, workspace, geo, B * H,
                                 H * total, H_kv, total, D, causal, stream);
}
