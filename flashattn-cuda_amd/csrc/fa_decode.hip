// fa_decode.hip — split-KV paged decode and its logsumexp combine for MI355X.
//
// No reference counterpart: the reference has no decode path. The math is
// attention of one query token over the keys of its sequence, read through a
// page table, computed per (sequence, head, split) as a normalised partial
// (O_s, L_s), then merged by L = log sum_s exp(L_s), O = sum_s exp(L_s - L) O_s.
//
// Pool layout: [num_pages, H_kv, 16, D] fp16 or bf16 (H_kv = H, or fewer KV heads
// shared by groups of H / H_kv query heads), so the 16 tokens of one head in a
// page are 16*D*2 contiguous bytes (4 KiB at D=128): one wave reads a page of
// one head as fully coalesced 16-byte loads.
//
// Split kernel: one workgroup (4 waves) per (split, head, sequence). Wave w
// walks pages p0+w, p0+w+4, ...; lane l covers the 16-byte chunk l % (D/8)
// of tokens l / (D/8) + (512/D) i of the page (i < D/32), so every load
// instruction reads 1 KiB of the page contiguously. Each wave keeps its own
// running max/sum and fp32 partial output; the four waves merge through LDS
// at the end.
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

// Element types of q, the pools and O: fp16, or bf16 (BF16 = true). Products
// of two 16-bit values are exact in fp32; the dot product accumulates in fp32
// (v_dot2_f32_f16 / v_dot2_f32_bf16) and everything after it is fp32.
template <bool BF16>
struct DecT {
  using e = f16;
  using v8 = f16x8;
  using v2 = f16x2;
  static __device__ __forceinline__ float dot2(v2 a, v2 b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
  }
};
template <>
struct DecT<true> {
  using e = __bf16;
  using v8 = bf16x8;
  using v2 = bf16x2;
  static __device__ __forceinline__ float dot2(v2 a, v2 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
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

template <int D, bool BF16>
__global__ void __launch_bounds__(kDecThreads)
fa_decode_split_kernel(const typename DecT<BF16>::e* __restrict__ q,
                       const typename DecT<BF16>::e* __restrict__ kpool,
                       const typename DecT<BF16>::e* __restrict__ vpool,
                       const int32_t* __restrict__ page_table,
                       const int32_t* __restrict__ ctx_lens, float* __restrict__ part_o,
                       float* __restrict__ part_lse, int H, int Hkv, int max_pages, int num_pages,
                       int S, float c) {
  using T = DecT<BF16>;
  using v8 = typename T::v8;
  using v2 = typename T::v2;
  constexpr int CH = D / 8;          // 16-byte chunks of a token row
  constexpr int TPI = 64 / CH;       // tokens per load instruction (1 KiB contiguous)
  constexpr int NI = kPage / TPI;    // load instructions per page and pool
  __shared__ float sh_o[kDecWaves][D];
  __shared__ float sh_m[kDecWaves];
  __shared__ float sh_l[kDecWaves];
  __shared__ int sh_bad;
  __shared__ int sh_ctx[kDecThreads];
  __shared__ int sh_seq;

  const int s = blockIdx.x, h = blockIdx.y;
  const int b = sequence_of_rank(ctx_lens, (int)gridDim.z, (int)blockIdx.z, sh_ctx, &sh_seq);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ch = lane % CH;    // chunk: d = 8 ch .. 8 ch + 7
  const int tl = lane / CH;    // token tl + TPI i of load instruction i

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

  v2 qv[4];
  {
    const v8 x = *reinterpret_cast<const v8*>(q + ((size_t)b * H + h) * D + 8 * ch);
#pragma unroll
    for (int e = 0; e < 4; ++e) qv[e] = v2{x[2 * e], x[2 * e + 1]};
  }

  float m = -INFINITY, l = 0.f;
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = 0.f;

  const int32_t* pt = page_table + (size_t)b * max_pages;
  const int kvh = h / (H / Hkv);
  // The wave's next page is loaded into (kn, vn) before the current one is
  // used, so one page per wave is always in flight behind the arithmetic.
  // Load instruction i of a pool reads bytes 1024 i .. 1024 i + 1023 of the
  // page (lane l: 16 bytes at 16 l), with the non-temporal hint: each page
  // is read once, and whole contiguous 1 KiB requests let the hint stream it
  // (a layout in which each instruction touched every line of the page ran
  // 57 % slower with the hint and no faster without it).
  v8 kn[NI], vn[NI];
  bool ok_n = false;
  auto load_page = [&](int p) {
    const int pid = pt[p];
    ok_n = pid >= 0 && pid < num_pages;
    if (!ok_n) return;
    const size_t base = ((size_t)pid * Hkv + kvh) * (kPage * D) + 8 * (size_t)lane;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      kn[i] = __builtin_nontemporal_load(reinterpret_cast<const v8*>(kpool + base + 512 * i));
#pragma unroll
    for (int i = 0; i < NI; ++i)
      vn[i] = __builtin_nontemporal_load(reinterpret_cast<const v8*>(vpool + base + 512 * i));
  };
  if (p0 + wave < p1) load_page(p0 + wave);
  for (int p = p0 + wave; p < p1; p += kDecWaves) {
    v8 kv[NI], vv[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      kv[i] = kn[i];
      vv[i] = vn[i];
    }
    const bool ok = ok_n;
    if (p + kDecWaves < p1) load_page(p + kDecWaves);
    if (!ok) { bad = true; continue; }
    float st[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) d = T::dot2(qv[e], v2{kv[i][2 * e], kv[i][2 * e + 1]}, d);
      st[i] = d;
    }
#pragma unroll
    for (int sh = 1; sh < CH; sh <<= 1)
#pragma unroll
      for (int i = 0; i < NI; ++i) st[i] += __shfl_xor(st[i], sh, 64);
    float mp = -INFINITY;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      st[i] *= c;
      if (p * kPage + TPI * i + tl >= ctx) {
        // A slot past the context holds whatever the pool held (NaN and
        // Inf included): its score is -inf and its V row is dropped, since
        // 0 * NaN would poison the output.
        st[i] = -INFINITY;
        vv[i] = v8{};
      }
      mp = fmaxf(mp, st[i]);
    }
#pragma unroll
    for (int sh = CH; sh < 64; sh <<= 1) mp = fmaxf(mp, __shfl_xor(mp, sh, 64));
    const float m_new = fmaxf(m, mp);   // finite: token p*16 < ctx
    const float alpha = (m_new == m) ? 1.f : exp2_hw(m - m_new);
    float pr[NI];
    float ps = 0.f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      pr[i] = exp2_hw(st[i] - m_new);
      ps += pr[i];
    }
    l = l * alpha + ps;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float a = o[e] * alpha;
#pragma unroll
      for (int i = 0; i < NI; ++i) a = fmaf(pr[i], (float)vv[i][e], a);
      o[e] = a;
    }
    m = m_new;
  }

  // Sum the token groups that share a chunk of D.
#pragma unroll
  for (int sh = CH; sh < 64; sh <<= 1) {
    l += __shfl_xor(l, sh, 64);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] += __shfl_xor(o[i], sh, 64);
  }
  if (bad) sh_bad = 1;
  if (tl == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) sh_o[wave][8 * ch + i] = o[i];
    if (ch == 0) { sh_m[wave] = m; sh_l[wave] = l; }
  }
  __syncthreads();

  const size_t pidx = ((size_t)b * H + h) * S + s;
  if (tid < D) {
    float M = sh_m[0];
#pragma unroll
    for (int w = 1; w < kDecWaves; ++w) M = fmaxf(M, sh_m[w]);
    float acc = 0.f, z = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) {
        const float e = (sh_m[w] == -INFINITY) ? 0.f : exp2_hw(sh_m[w] - M);
        acc += e * sh_o[w][tid];
        z += e * sh_l[w];
      }
    }
    float out = (z > 0.f) ? acc / z : 0.f;
    float lse = (z > 0.f) ? (M + log2_hw(z)) * kLn2 : -INFINITY;
    if (sh_bad) { out = NAN; lse = NAN; }
    part_o[pidx * D + tid] = out;
    if (tid == 0) part_lse[pidx] = lse;
  }
}

// Grouped-KV split pass: one workgroup per (split, G query heads that share
// one KV head, sequence). Each K/V page is loaded once into registers and
// used for all G heads (a lane's dot products, softmax state and output
// slice are kept per head), so a page is read once per KV head instead of
// once per query head. Waves split the pages as above and merge per head.
//
// LPT lanes share a token: with LPT = 4 a lane holds D / 4 columns of one
// token of the page; with LPT = 8 it holds D / 8 columns of two tokens
// (t and t + 8), which halves the per-head query and output registers so
// that four heads fit at D = 128.
template <int D, int G, bool BF16, int LPT = 4>
__global__ void __launch_bounds__(kDecThreads)
fa_decode_split_group_kernel(const typename DecT<BF16>::e* __restrict__ q,
                             const typename DecT<BF16>::e* __restrict__ kpool,
                             const typename DecT<BF16>::e* __restrict__ vpool,
                             const int32_t* __restrict__ page_table,
                             const int32_t* __restrict__ ctx_lens, float* __restrict__ part_o,
                             float* __restrict__ part_lse, int H, int Hkv, int max_pages,
                             int num_pages, int S, float c) {
  using T = DecT<BF16>;
  using v8 = typename T::v8;
  using v2 = typename T::v2;
  static_assert(LPT == 4 || LPT == 8, "4 or 8 lanes per token");
  constexpr int DPL = D / LPT;   // d per lane
  constexpr int NV = DPL / 8;    // 16-byte vectors per lane per row
  constexpr int TPL = LPT / 4;   // tokens per lane: tok + 8 j
  __shared__ float sh_o[kDecWaves][G][D];
  __shared__ float sh_m[kDecWaves][G];
  __shared__ float sh_l[kDecWaves][G];
  __shared__ int sh_bad;
  __shared__ int sh_ctx[kDecThreads];
  __shared__ int sh_seq;

  const int s = blockIdx.x, hg = blockIdx.y;
  const int b = sequence_of_rank(ctx_lens, (int)gridDim.z, (int)blockIdx.z, sh_ctx, &sh_seq);
  const int h0 = hg * G;                  // first query head of this workgroup
  const int hk = h0 / (H / Hkv);          // their KV head (G divides H / Hkv)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tok = lane / LPT;
  const int dq = lane % LPT;

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

  v2 qv[G][DPL / 2];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const typename T::e* qp = q + ((size_t)b * H + h0 + g) * D + dq * DPL;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      v8 x = *reinterpret_cast<const v8*>(qp + 8 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) qv[g][4 * i + e] = v2{x[2 * e], x[2 * e + 1]};
    }
  }

  float m[G], l[G];
  float o[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) o[g][i] = 0.f;
  }

  const int32_t* pt = page_table + (size_t)b * max_pages;
  for (int p = p0 + wave; p < p1; p += kDecWaves) {
    const int pid = pt[p];
    if (pid < 0 || pid >= num_pages) { bad = true; continue; }
    const size_t base = ((size_t)pid * Hkv + hk) * (kPage * D) + (size_t)tok * D + dq * DPL;
    v8 kv[TPL][NV], vv[TPL][NV];
#pragma unroll
    for (int j = 0; j < TPL; ++j) {
#pragma unroll
      for (int i = 0; i < NV; ++i) kv[j][i] = *reinterpret_cast<const v8*>(kpool + base + j * 8 * D + 8 * i);
    }
#pragma unroll
    for (int j = 0; j < TPL; ++j) {
#pragma unroll
      for (int i = 0; i < NV; ++i) vv[j][i] = *reinterpret_cast<const v8*>(vpool + base + j * 8 * D + 8 * i);
    }
    bool live[TPL];
#pragma unroll
    for (int j = 0; j < TPL; ++j) {
      live[j] = p * kPage + tok + 8 * j < ctx;
      if (!live[j]) {   // slot past the context: drop its V row (it may hold NaN or Inf)
#pragma unroll
        for (int i = 0; i < NV; ++i) vv[j][i] = v8{};
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float st[TPL];
      float mp = -INFINITY;
#pragma unroll
      for (int j = 0; j < TPL; ++j) {
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            dot = T::dot2(qv[g][4 * i + e], v2{kv[j][i][2 * e], kv[j][i][2 * e + 1]}, dot);
          }
        }
#pragma unroll
        for (int sh = 1; sh < LPT; sh <<= 1) dot += __shfl_xor(dot, sh, 64);
        st[j] = live[j] ? dot * c : -INFINITY;
        mp = fmaxf(mp, st[j]);
      }
#pragma unroll
      for (int sh = LPT; sh < 64; sh <<= 1) mp = fmaxf(mp, __shfl_xor(mp, sh, 64));
      const float m_new = fmaxf(m[g], mp);   // finite: token p*16 < ctx
      const float alpha = (m_new == m[g]) ? 1.f : exp2_hw(m[g] - m_new);
      float pr[TPL];
      float psum = 0.f;
#pragma unroll
      for (int j = 0; j < TPL; ++j) {
        pr[j] = exp2_hw(st[j] - m_new);
        psum += pr[j];
      }
      l[g] = l[g] * alpha + psum;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float acc = o[g][8 * i + e] * alpha;
#pragma unroll
          for (int j = 0; j < TPL; ++j) acc = fmaf(pr[j], (float)vv[j][i][e], acc);
          o[g][8 * i + e] = acc;
        }
      }
      m[g] = m_new;
    }
  }

#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int sh = LPT; sh < 64; sh <<= 1) {
      l[g] += __shfl_xor(l[g], sh, 64);
#pragma unroll
      for (int i = 0; i < DPL; ++i) o[g][i] += __shfl_xor(o[g][i], sh, 64);
    }
  }
  if (bad) sh_bad = 1;
  if (tok == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int i = 0; i < DPL; ++i) sh_o[wave][g][dq * DPL + i] = o[g][i];
      if (dq == 0) { sh_m[wave][g] = m[g]; sh_l[wave][g] = l[g]; }
    }
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
        acc += e * sh_o[w][g][d];
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
  // Grouped KV heads: G query heads per workgroup share each page read. At
  // D = 128 four heads take 8 lanes per token (two tokens per lane), which
  // keeps their state within the registers of three waves per SIMD; with 4
  // lanes per token they needed 256 VGPRs (one wave per SIMD: 706 us vs 507 us
  // for G = 2 on the group-of-4 pools).
  const int64_t group = H / Hkv;
  const int G = group % 4 == 0 ? 4 : (group % 2 == 0 ? 2 : 1);
  if (G > 1) {
    const dim3 ggrid((unsigned)num_splits, (unsigned)(H / G), (unsigned)B);
#define FA_DEC_GROUP(DD, GG, LL)                                                                    \
  hipLaunchKernelGGL((fa_decode_split_group_kernel<DD, GG, BF16, LL>), ggrid, dim3(kDecThreads), 0, \
                     s, Q, Kp, Vp, page_table, ctx_lens, part_o, part_lse, (int)H, (int)Hkv,         \
                     (int)max_pages, (int)num_pages, (int)num_splits, c)
    if (D == 128) {
      if (G == 4) FA_DEC_GROUP(128, 4, 8); else FA_DEC_GROUP(128, 2, 4);
    } else {
      if (G == 4) FA_DEC_GROUP(64, 4, 4); else FA_DEC_GROUP(64, 2, 4);
    }
#undef FA_DEC_GROUP
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? FA_OK : -(int)e;
  }
  dim3 grid((unsigned)num_splits, (unsigned)H, (unsigned)B);
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
