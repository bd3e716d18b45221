// fa_decode.hip — split-KV paged decode and its logsumexp combine for MI355X.
//
// No reference counterpart: the reference has no decode path. The math is
// attention of one query token over the keys of its sequence, read through a
// page table, computed per (sequence, head, split) as a normalised partial
// (O_s, L_s), then merged by L = log sum_s exp(L_s), O = sum_s exp(L_s - L) O_s.
//
// Pool layout: [num_pages, H_kv, 16, D] fp16 or bf16 (H_kv = H, or fewer KV heads
// shared by groups of H / H_kv query heads), so the 16 tokens of one head in a
// page are 16*D*2 contiguous bytes (4 KiB at D=128), copied into LDS as
// contiguous 1 KiB requests.
//
// Split kernel: one workgroup (4 waves) per (split, KV head, up to 16 query
// heads of its group, sequence); wave w walks pages p0+w, p0+w+4, ... and
// computes the scores of every head of the workgroup and their PV products
// on the matrix cores, so a page is read once per KV head. Each wave keeps
// its own running max/sum and fp32 partial output per head; the four waves
// merge through LDS at the end.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <mutex>

#include "fa_mi355x.h"
#include "fa_tile.hpp"

namespace fa {

constexpr int kPage = 16;
constexpr int kDecThreads = 256;
constexpr int kDecWaves = kDecThreads / 64;

// Element types of q, the pools and O: fp16, or bf16 (BF16 = true). The
// matrix products take them as 16-bit operands with fp32 accumulation; P is
// rounded to the same 16-bit type for its product with V, everything else
// is fp32.
template <bool BF16>
struct DecT {
  using e = f16;
  using v8 = f16x8;
};
template <>
struct DecT<true> {
  using e = __bf16;
  using v8 = bf16x8;
};

// Longest sequence first: grid index z (the slowest-varying one, so low z
// is dispatched first) takes the sequence of rank z by decreasing
// context length, ties by index. The longest splits then start first and the
// shortest fill the tail instead of a long sequence dispatched last running
// alone. Ranks of B <= kDecThreads contexts are computed from a copy in LDS;
// larger batches keep the identity order. Invalid (negative) lengths rank
// like any other value and are flagged by the caller as before.
__device__ __forceinline__ int sequence_of_rank(const int32_t* __restrict__ ctx_lens, int B, int z,
                                                int* sh_ctx, int* sh_seq) {
  if (B > kDecThreads) return z;
  const int t = threadIdx.x;
  if (t < B) sh_ctx[t] = ctx_lens[t];
  __syncthreads();
  if (t < B) {
    const int c = sh_ctx[t];
    int r = 0;
    for (int j = 0; j < B; ++j) {
      const int cj = sh_ctx[j];
      r += (cj > c) || (cj == c && j < t);
    }
    if (r == z) *sh_seq = t;   // ranks are a permutation: exactly one writer
  }
  __syncthreads();
  return *sh_seq;
}

// Split kernel, on the matrix cores: one workgroup (4 waves) per (split, KV
// head, up to 16 of the query heads that share it, sequence). A wave copies each
// page's K and V rows of the KV head into LDS (1 KiB per copy instruction,
// contiguous in the pool, non-temporal), then
//   S   = K Q^T   (v_mfma_f32_16x16x32: 16 tokens x 16 heads, K from LDS,
//                  Q^T in registers; heads past the group are zero columns)
//   P   = exp2(S c - m) per head column (online softmax, in registers)
//   O^T += V^T P^T (v_mfma_f32_16x16x16 per 16 columns of D: V^T read with
//                  ds_read_b64_tr_b16, P^T straight from the S accumulator)
// so each page is read once for every query head of its group. Lane l holds
// head l % 16 and tokens 4 (l / 16) .. + 3 of S, and rows 4 (l / 16) + r of
// every 16-column block of O^T for the same head, so the softmax statistics
// of a head stay in its lane column. Each wave keeps two page slots (the
// next page's copies land while the current one is computed).
//
// LDS layout of a page slot: row t (token) of 16-byte chunks, chunk c stored
// at position c ^ (t % (D / 8)), the forward's K-tile swizzle. The copies
// apply it on the source side: lane l of copy i fills LDS chunk 64 i + l from
// the page chunk it should hold. (SQ_LDS_BANK_CONFLICT still counts ~30 % of
// the LDS-active cycles, all in the K reads; the kernel waits on memory for
// ~74 % of its wave cycles, and a conflict-free variant of the swizzle for a
// 64-bank model timed the same.)
template <int D>
__device__ __forceinline__ int dec_swz(int t) { return t & (D / 8 - 1); }

template <bool BF16>
__device__ __forceinline__ f32x4 mma16k32(f16x8 a, f16x8 b, f32x4 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
}

template <bool BF16>
__device__ __forceinline__ f32x4 mma16k16(f16x4 a, f16x4 b, f32x4 c) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                     __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
}

// 16-byte copy straight into LDS with the non-temporal hint (the page is read
// once): see dma16.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_nt(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voffset), "s"(r)
               : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ float max_cols(float x) {   // max over the 4 lane groups of a column
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float sum_cols(float x) {   // sum over the 4 lane groups of a column
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

template <int D, bool BF16>
__global__ void __launch_bounds__(kDecThreads)
fa_decode_split_kernel(const typename DecT<BF16>::e* __restrict__ q,
                       const typename DecT<BF16>::e* __restrict__ kpool,
                       const typename DecT<BF16>::e* __restrict__ vpool,
                       const int32_t* __restrict__ page_table,
                       const int32_t* __restrict__ ctx_lens, float* __restrict__ part_o,
                       float* __restrict__ part_lse, int H, int Hkv, int max_pages,
                       int num_pages, int S, float c) {
  using T = DecT<BF16>;
  constexpr int PAGE = kPage * D * 2;   // bytes of one head's page
  constexpr int CPR = D / 8;            // 16-byte chunks per token row
  constexpr int KB = D / 32;            // k-steps of S = K Q^T
  constexpr int DB = D / 16;            // 16-column blocks of O^T
  constexpr int NC = PAGE / 1024;       // 1 KiB copies per page and pool
  static_assert(kDecWaves * 16 * D * 4 <= kDecWaves * 4 * PAGE, "merge area within the slots");
  __shared__ __attribute__((aligned(1024))) char smem[kDecWaves * 4 * PAGE];
  __shared__ float sh_m[kDecWaves][16];
  __shared__ float sh_l[kDecWaves][16];
  __shared__ int sh_bad;
  __shared__ int sh_ctx[kDecThreads];
  __shared__ int sh_seq;

  const int s = blockIdx.x;
  const int group = H / Hkv;
  const int ngrp = (group + 15) / 16;
  const int hk = blockIdx.y / ngrp;
  const int h0 = hk * group + 16 * (blockIdx.y % ngrp);   // first query head of this workgroup
  const int G = min(16, hk * group + group - h0);
  const int b = sequence_of_rank(ctx_lens, (int)gridDim.z, (int)blockIdx.z, sh_ctx, &sh_seq);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;

  if (tid == 0) sh_bad = 0;
  __syncthreads();

  int ctx = ctx_lens[b];
  bool bad = false;
  if (ctx < 0) { bad = true; ctx = 0; }
  int pages = (ctx + kPage - 1) / kPage;
  if (pages > max_pages) { bad = true; pages = max_pages; ctx = max_pages * kPage; }
  const int chunk = (pages + S - 1) / S;
  const int p0 = min(s * chunk, pages);
  const int p1 = min(p0 + chunk, pages);

  // Q^T operand (16x16x32 B): column col = head h0 + col, rows 8 grp .. + 7
  // of k-step kb.
  f16x8 qf[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    qf[kb] = f16x8{};
    if (col < G)
      qf[kb] = __builtin_bit_cast(f16x8, *reinterpret_cast<const typename T::v8*>(
                                             q + ((size_t)b * H + h0 + col) * D + 32 * kb + 8 * grp));
  }

  float m = -INFINITY, l = 0.f;
  f32x4 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x4{};

  // Copy offsets: lane l of copy i fills LDS chunk L = 64 i + l with page
  // chunk (L % CPR) ^ swz(row) of row L / CPR.
  uint32_t coff[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int L = 64 * i + lane, t = L / CPR;
    coff[i] = (uint32_t)((t * CPR + ((L % CPR) ^ dec_swz<D>(t))) * 16);
  }
  const uint32_t lds0 = lds_addr(smem) + (uint32_t)(wave * 4 * PAGE);   // this wave's two slots
  const int32_t* pt = page_table + (size_t)b * max_pages;
  // Page ids of the wave's pages p0 + wave + 4 k, 64 at a time: lane i of
  // pidv holds the id of page k = 64 j + i, read with readlane (a page
  // table load per page would wait for every copy in flight before it).
  int pidv = -1;
  auto page_id = [&](int k) -> int {
    if ((k & 63) == 0) {
      const int pi = p0 + wave + 4 * (k + lane);
      pidv = pi < p1 ? pt[pi] : -1;
    }
    return __builtin_amdgcn_readlane(pidv, k & 63);
  };
  // Issue the copies of the wave's k-th page into slot sl; false (nothing
  // issued) for an invalid page id.
  auto issue = [&](int k, int sl) -> bool {
    const int pid = page_id(k);
    if (pid < 0 || pid >= num_pages) return false;
    const size_t off = ((size_t)pid * Hkv + hk) * (size_t)(kPage * D);
    const auto rk = make_rsrc_s(kpool + off, PAGE);
    const auto rv = make_rsrc_s(vpool + off, PAGE);
    const uint32_t dk = lds0 + (uint32_t)(sl * 2 * PAGE);
#pragma unroll
    for (int i = 0; i < NC; ++i) dma16_nt(rk, dk + 1024 * i, coff[i]);
#pragma unroll
    for (int i = 0; i < NC; ++i) dma16_nt(rv, dk + PAGE + 1024 * i, coff[i]);
    return true;
  };

  // Per-lane LDS offsets of the operand reads within a slot.
  // K (16x16x32 A): row col, chunk 4 kb + grp.
  // V^T (16x16x16 A through ds_read_b64_tr_b16): lane (grp, s) supplies row
  // 4 grp + s / 4, 8 bytes at column 16 db + 4 (s % 4).
  const int vrow = 4 * grp + (col >> 2);
  int p = p0 + wave;
  int sl = 0, k = 0;
  bool ok = p < p1 && issue(0, 0);
  for (; p < p1; p += kDecWaves, sl ^= 1, ++k) {
    const int pn = p + kDecWaves;
    const bool ok_n = pn < p1 && issue(k + 1, sl ^ 1);
    if (ok_n) wait_vmcnt<2 * NC>(); else wait_vmem();
    if (!ok) { bad = true; ok = ok_n; continue; }
    const uint32_t ks = lds0 + (uint32_t)(sl * 2 * PAGE);
    const uint32_t vs = ks + PAGE;
    f32x4 sc = f32x4{};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const lds_cp a = (lds_cp)(size_t)(ks + (uint32_t)((col * CPR + ((4 * kb + grp) ^ dec_swz<D>(col))) * 16));
      sc = mma16k32<BF16>(lds_b128(a), qf[kb], sc);
    }
    // Scores of head col, tokens 4 grp + r of the page; slots past the
    // context get -inf (their K rows may hold anything, NaN included).
    const int tok0 = p * kPage + 4 * grp;
    float st[4];
    float mp = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      st[r] = tok0 + r < ctx ? sc[r] * c : -INFINITY;
      mp = fmaxf(mp, st[r]);
    }
    mp = max_cols(mp);
    const float m_new = fmaxf(m, mp);   // finite: token p*16 < ctx
    const float alpha = (m_new == m) ? 1.f : exp2_hw(m - m_new);
    float pr[4];
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pr[r] = exp2_hw(st[r] - m_new);
      ps += pr[r];
    }
    l = l * alpha + ps;
    m = m_new;
    const f16x2 p01 = cvt2x<BF16>(pr[0], pr[1]);
    const f16x2 p23 = cvt2x<BF16>(pr[2], pr[3]);
    const f16x4 pb = f16x4{p01[0], p01[1], p23[0], p23[1]};
    // bf16 keeps 8 significant bits of P: a second product with the rounded
    // remainder p - bf16(p) carries P to 16 (fp16's 11 are kept as they are).
    f16x4 pl = f16x4{};
    if constexpr (BF16) {
      auto up = [](f16 h) { return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, h) << 16); };
      const f16x2 l01 = cvt2x<true>(pr[0] - up(pb[0]), pr[1] - up(pb[1]));
      const f16x2 l23 = cvt2x<true>(pr[2] - up(pb[2]), pr[3] - up(pb[3]));
      pl = f16x4{l01[0], l01[1], l23[0], l23[1]};
    }
    const bool tail = p * kPage + kPage > ctx;   // wave-uniform: the sequence's last, partial page
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int cb = 2 * db + ((col & 3) >> 1);   // chunk of columns 16 db + 4 (s % 4)
      const lds_cp a = (lds_cp)(size_t)(vs + (uint32_t)((vrow * CPR + (cb ^ dec_swz<D>(vrow))) * 16 + 8 * (col & 1)));
      f16x4 va = lds_tr16(a);
      if (tail) {   // V rows past the context may hold NaN or Inf: 0 * NaN
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (tok0 + e >= ctx) va[e] = (f16)0.f;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) o[db][e] *= alpha;
      o[db] = mma16k16<BF16>(va, pb, o[db]);
      if constexpr (BF16) o[db] = mma16k16<true>(va, pl, o[db]);
    }
    ok = ok_n;
  }
  l = sum_cols(l);

  // Merge the waves through LDS (the page slots are free once every wave's
  // copies have landed and its reads are done).
  wait_vmem();
  if (bad) sh_bad = 1;
  __syncthreads();
  float* sh_o = reinterpret_cast<float*>(smem);   // [kDecWaves][16][D]
  if (col < G) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) sh_o[(wave * 16 + col) * D + 16 * db + 4 * grp + r] = o[db][r];
    if (grp == 0) { sh_m[wave][col] = m; sh_l[wave][col] = l; }
  }
  __syncthreads();

  // Thread x merges column x % D of head x / D across the waves.
  for (int x = tid; x < G * D; x += kDecThreads) {
    const int g = x / D, d = x % D;
    float M = sh_m[0][g];
#pragma unroll
    for (int w = 1; w < kDecWaves; ++w) M = fmaxf(M, sh_m[w][g]);
    float acc = 0.f, z = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) {
        const float e = (sh_m[w][g] == -INFINITY) ? 0.f : exp2_hw(sh_m[w][g] - M);
        acc += e * sh_o[(w * 16 + g) * D + d];
        z += e * sh_l[w][g];
      }
    }
    float out = (z > 0.f) ? acc / z : 0.f;
    float lse = (z > 0.f) ? (M + log2_hw(z)) * kLn2 : -INFINITY;
    if (sh_bad) { out = NAN; lse = NAN; }
    const size_t pidx = ((size_t)b * H + h0 + g) * S + s;
    part_o[pidx * D + d] = out;
    if (d == 0) part_lse[pidx] = lse;
  }
}

// One workgroup of D threads per (b, h): thread d merges column d.
template <int D, bool BF16>
__global__ void __launch_bounds__(D)
fa_lse_combine_kernel(const float* __restrict__ part_o, const float* __restrict__ part_lse,
                      typename DecT<BF16>::e* __restrict__ o, float* __restrict__ lse, int S) {
  const int bh = blockIdx.x;
  const int d = threadIdx.x;
  const float* ls = part_lse + (size_t)bh * S;
  float M = -INFINITY;
  bool nan = false;
  for (int s = 0; s < S; ++s) {
    const float x = ls[s];
    nan |= (x != x);
    M = fmaxf(M, x);
  }
  float out, L;
  if (nan) {
    out = NAN;
    L = NAN;
  } else if (M == -INFINITY) {
    out = 0.f;
    L = -INFINITY;
  } else {
    float z = 0.f;
    for (int s = 0; s < S; ++s) z += exp2_hw((ls[s] - M) * kLog2e);
    L = M + log2_hw(z) * kLn2;
    float acc = 0.f;
    const float* po = part_o + (size_t)bh * S * D + d;
    for (int s = 0; s < S; ++s) {
      const float w = exp2_hw((ls[s] - L) * kLog2e);
      acc = fmaf(w, po[(size_t)s * D], acc);
    }
    out = acc;
  }
  o[(size_t)bh * D + d] = (typename DecT<BF16>::e)out;
  if (lse != nullptr && d == 0) lse[bh] = L;
}

}  // namespace fa

namespace fa {
// Split pass with query heads h reading pool head h / (H / Hkv); arguments
// already validated.
template <bool BF16>
static int decode_split(const void* q, const void* k_pool, const void* v_pool,
                        const int32_t* page_table, const int32_t* ctx_lens, int64_t B, int64_t H,
                        int64_t Hkv, int64_t D, int64_t max_pages, int64_t num_pages,
                        int64_t num_splits, float* part_o, float* part_lse, void* stream) {
  using E = typename DecT<BF16>::e;
  if (!part_o || !part_lse) return FA_ERR_NULL_POINTER;
  const float c = (float)(1.0 / sqrt((double)D)) * kLog2e;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const E* Q = (const E*)q;
  const E* Kp = (const E*)k_pool;
  const E* Vp = (const E*)v_pool;
  // One workgroup per (split, KV head, 16 of its query heads, sequence).
  const int64_t group = H / Hkv;
  const dim3 grid((unsigned)num_splits, (unsigned)(Hkv * ((group + 15) / 16)), (unsigned)B);
  if (D == 128) {
    hipLaunchKernelGGL((fa_decode_split_kernel<128, BF16>), grid, dim3(kDecThreads), 0, s, Q, Kp,
                       Vp, page_table, ctx_lens, part_o, part_lse, (int)H, (int)Hkv,
                       (int)max_pages, (int)num_pages, (int)num_splits, c);
  } else {
    hipLaunchKernelGGL((fa_decode_split_kernel<64, BF16>), grid, dim3(kDecThreads), 0, s, Q, Kp,
                       Vp, page_table, ctx_lens, part_o, part_lse, (int)H, (int)Hkv,
                       (int)max_pages, (int)num_pages, (int)num_splits, c);
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FA_OK : -(int)e;
}

// LSE combine of [B, H, num_splits] partials into O [B, H, D] (fp16 or bf16)
// and L fp32 [B, H] (may be null).
template <bool BF16>
static int lse_combine(const float* part_o, const float* part_lse, int64_t B, int64_t H,
                       int64_t D, int64_t num_splits, void* o, float* lse, void* stream) {
  using E = typename DecT<BF16>::e;
  if (!part_o || !part_lse || !o) return FA_ERR_NULL_POINTER;
  if (D != 64 && D != 128) return FA_ERR_HEAD_DIM;
  if (B <= 0 || H <= 0) return FA_ERR_BATCH_HEADS;
  if (num_splits < 1 || num_splits > 16) return FA_ERR_NUM_SPLITS;
  if (B * H > (int64_t(1) << 31) - 1) return FA_ERR_TOO_LARGE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (D == 128) {
    hipLaunchKernelGGL((fa_lse_combine_kernel<128, BF16>), dim3((unsigned)(B * H)), dim3(128), 0,
                       s, part_o, part_lse, (E*)o, lse, (int)num_splits);
  } else {
    hipLaunchKernelGGL((fa_lse_combine_kernel<64, BF16>), dim3((unsigned)(B * H)), dim3(64), 0,
                       s, part_o, part_lse, (E*)o, lse, (int)num_splits);
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FA_OK : -(int)e;
}
}  // namespace fa

extern "C" int fa_decode_split_f16(const void* q, const void* k_pool, const void* v_pool,
                                   const int32_t* page_table, const int32_t* ctx_lens,
                                   int64_t B, int64_t H, int64_t D, int64_t page_size,
                                   int64_t max_pages, int64_t num_pages, int64_t num_splits,
                                   float* part_o, float* part_lse, void* stream) {
  int st = fa_validate_decode(q, k_pool, v_pool, page_table, ctx_lens, B, H, D, page_size,
                              max_pages, num_pages, num_splits);
  if (st != FA_OK) return st;
  return fa::decode_split<false>(q, k_pool, v_pool, page_table, ctx_lens, B, H, H, D, max_pages,
                                 num_pages, num_splits, part_o, part_lse, stream);
}

extern "C" int fa_lse_combine_f32(const float* part_o, const float* part_lse, int64_t B,
                                  int64_t H, int64_t D, int64_t num_splits, void* o,
                                  float* lse, void* stream) {
  return fa::lse_combine<false>(part_o, part_lse, B, H, D, num_splits, o, lse, stream);
}

extern "C" int fa_decode_paged_f16(const void* q, const void* k_pool, const void* v_pool,
                                   const int32_t* page_table, const int32_t* ctx_lens,
                                   int64_t B, int64_t H, int64_t D, int64_t page_size,
                                   int64_t max_pages, int64_t num_pages, int64_t num_splits,
                                   float* part_o, float* part_lse, void* o, float* lse,
                                   void* stream) {
  int st = fa_decode_split_f16(q, k_pool, v_pool, page_table, ctx_lens, B, H, D, page_size,
                               max_pages, num_pages, num_splits, part_o, part_lse, stream);
  if (st != FA_OK) return st;
  return fa_lse_combine_f32(part_o, part_lse, B, H, D, num_splits, o, lse, stream);
}

namespace fa {
template <bool BF16>
static int decode_paged_gqa(const void* q, const void* k_pool, const void* v_pool,
                            const int32_t* page_table, const int32_t* ctx_lens, int64_t B,
                            int64_t H, int64_t H_kv, int64_t D, int64_t page_size,
                            int64_t max_pages, int64_t num_pages, int64_t num_splits,
                            float* part_o, float* part_lse, void* o, float* lse, void* stream) {
  int st = fa_validate_decode(q, k_pool, v_pool, page_table, ctx_lens, B, H, D, page_size,
                              max_pages, num_pages, num_splits);
  if (st != FA_OK) return st;
  if (H_kv <= 0 || H % H_kv != 0) return FA_ERR_KV_HEADS;
  st = decode_split<BF16>(q, k_pool, v_pool, page_table, ctx_lens, B, H, H_kv, D, max_pages,
                          num_pages, num_splits, part_o, part_lse, stream);
  if (st != FA_OK) return st;
  return lse_combine<BF16>(part_o, part_lse, B, H, D, num_splits, o, lse, stream);
}
}  // namespace fa

extern "C" int fa_decode_paged_gqa_f16(const void* q, const void* k_pool, const void* v_pool,
                                       const int32_t* page_table, const int32_t* ctx_lens,
                                       int64_t B, int64_t H, int64_t H_kv, int64_t D,
                                       int64_t page_size, int64_t max_pages, int64_t num_pages,
                                       int64_t num_splits, float* part_o, float* part_lse,
                                       void* o, float* lse, void* stream) {
  return fa::decode_paged_gqa<false>(q, k_pool, v_pool, page_table, ctx_lens, B, H, H_kv, D,
                                     page_size, max_pages, num_pages, num_splits, part_o,
                                     part_lse, o, lse, stream);
}

extern "C" int fa_decode_paged_bf16(const void* q, const void* k_pool, const void* v_pool,
                                    const int32_t* page_table, const int32_t* ctx_lens,
                                    int64_t B, int64_t H, int64_t H_kv, int64_t D,
                                    int64_t page_size, int64_t max_pages, int64_t num_pages,
                                    int64_t num_splits, float* part_o, float* part_lse, void* o,
                                    float* lse, void* stream) {
  return fa::decode_paged_gqa<true>(q, k_pool, v_pool, page_table, ctx_lens, B, H, H_kv, D,
                                    page_size, max_pages, num_pages, num_splits, part_o,
                                    part_lse, o, lse, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free paged decode: the split partials (part_o, then part_lse)
// live in a file-scope device array instead of a caller workspace, for
// callers that cannot allocate device memory. The split pass writes every
// partial it owns (an empty split writes 0 and -inf), so nothing in the array
// needs clearing between calls.
namespace fa {
// One copy per GPU that loads this library, held until the process ends. In
// host code `scratch` names a host-side stand-in: only the address returned
// by hipGetSymbolAddress for the current device may reach a kernel.
static __device__ __align__(256) float scratch[FA_DECODE_SCRATCH_FLOATS];

constexpr int kScratchDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_addr[kScratchDevices];   // per device, null until resolved

// Device address of `scratch` on device `dev`, resolved on first use with
// `dev` current (then the previous current device is restored).
static int scratch_addr(int dev, float** out) {
  if (dev < 0 || dev >= kScratchDevices) return -(int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return -(int)e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return -(int)e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    const hipError_t e2 = cur != dev ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess) return -(int)e;
    if (e2 != hipSuccess) return -(int)e2;
    if (p == nullptr) return -(int)hipErrorInvalidSymbol;
    g_scratch_addr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_addr[dev];
  return FA_OK;
}
}  // namespace fa

extern "C" int fa_decode_paged_noalloc_f16(const void* q, const void* k_pool,
                                           const void* v_pool, const int32_t* page_table,
                                           const int32_t* ctx_lens, int64_t B, int64_t H,
                                           int64_t H_kv, int64_t D, int64_t page_size,
                                           int64_t max_pages, int64_t num_pages,
                                           int64_t num_splits, void* o, float* lse,
                                           void* stream) {
  int st = fa_validate_decode(q, k_pool, v_pool, page_table, ctx_lens, B, H, D, page_size,
                              max_pages, num_pages, num_splits);
  if (st != FA_OK) return st;
  if (o == nullptr) return FA_ERR_NULL_POINTER;
  if (H_kv <= 0 || H % H_kv != 0) return FA_ERR_KV_HEADS;
  // B, H, D and num_splits are bounded by the validation above, so the
  // product cannot overflow.
  if (B * H * num_splits * (D + 1) > FA_DECODE_SCRATCH_FLOATS) return FA_ERR_SCRATCH_SIZE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int dev = 0;
  hipError_t e = s != nullptr ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return -(int)e;
  float* part_o = nullptr;
  st = fa::scratch_addr(dev, &part_o);
  if (st != FA_OK) return st;
  float* part_lse = part_o + B * H * num_splits * D;
  return fa::decode_paged_gqa<false>(q, k_pool, v_pool, page_table, ctx_lens, B, H, H_kv, D,
                                     page_size, max_pages, num_pages, num_splits, part_o,
                                     part_lse, o, lse, stream);
}
