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
//   * one workgroup = 4 waves = 128 query rows of one (b, h); each wave owns
//     32 rows; a 1-D grid with an XCD-aware remap keeps the query blocks of a
//     head on one XCD so its K/V stay in that XCD's L2;
//   * K/V advance in 64-key tiles through two LDS stages (two separate LDS
//     objects, so the compiler can see that reads of one stage never alias
//     the DMA into the other); the next tile is copied global -> LDS by
//     buffer_load ... lds while the current one is consumed;
//   * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_f16 (fa_tile.hpp);
//   * softmax state per lane; the running max is only raised when a new
//     block max exceeds it by more than 2^8 (P <= 256 stays exact in fp32
//     accumulators and representable in fp16), so O is rarely rescaled;
//   * template flags: D in {64,128}, CAUSAL, WRITE_L (O-only when false),
//     FULL (N % 128 == 0: no bounds predicates).
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "fa_mi355x.h"
#include "fa_tile.hpp"

namespace fa {

constexpr int kBR = 128;   // query rows per workgroup
constexpr int kBC = 64;    // keys per tile
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr float kRescaleThreshold = 8.0f;  // log2 units

// Workgroup g of `total` lands on XCD g % 8. Map it to a logical tile index
// so that each XCD gets one contiguous range of logical tiles.
__device__ __forceinline__ int xcd_remap(int g, int total) {
  const int q = total >> 3, r = total & 7;
  const int xcd = g & 7, slot = g >> 3;
  return (xcd < r) ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

template <int D, bool CAUSAL, bool WRITE_L, bool FULL>
__global__ void __launch_bounds__(kThreads)
fa_fwd_kernel(const f16* __restrict__ Q, const f16* __restrict__ K,
              const f16* __restrict__ V, f16* __restrict__ O,
              float* __restrict__ L, int N, int num_qb, int total, float c) {
  constexpr int KSTEPS = D / 16;                  // QK k-steps
  constexpr int DB = D / 32;                      // O^T d-blocks
  constexpr int TILE = kBC * D * 2;               // bytes of one K or V tile
  constexpr int BLOCKS = TILE / 1024;             // 1 KiB DMA blocks per tile
  constexpr int LOADS = BLOCKS / kWaves;          // DMA blocks per wave per tile
  __shared__ __attribute__((aligned(1024))) char smem0[2 * TILE];   // stage 0: K|V
  __shared__ __attribute__((aligned(1024))) char smem1[2 * TILE];   // stage 1: K|V

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int hi = lane >> 5;

  const int logical = xcd_remap(blockIdx.x, total);
  const int bh = logical / num_qb;
  int qb = logical - bh * num_qb;
  if (CAUSAL) qb = num_qb - 1 - qb;   // longest rows dispatch first

  const size_t head = (size_t)bh * N * D;
  const int head_bytes = N * D * 2;
  const f16* Kh = K + head;
  const f16* Vh = V + head;

  const int q0 = qb * kBR;
  const int row_w = q0 + wave * 32;
  const int qrow = row_w + (lane & 31);

  // Q^T as the B operand of S^T = K Q^T, kept in registers for the whole loop.
  // Buffer loads return zero for rows >= N.
  f16x8 qf[KSTEPS];
  {
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(Q + head, head_bytes);
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(
          rq, (uint32_t)(qrow * D + 16 * kk + 8 * hi) * 2, 0, 0);
      qf[kk] = __builtin_bit_cast(f16x8, x);
    }
  }

  // Tile loads go global -> LDS directly. Each wave fills LOADS 1 KiB blocks
  // of the K tile and of the V tile; lane l writes bytes [16 l, 16 l + 16) of a
  // block, so the swizzle is applied by choosing which global chunk it fetches.
  uint32_t koff[LOADS], voff[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int o = (wave * LOADS + i) * 1024 + 16 * lane;
    const int r = o / (2 * D);
    const int slot = (o % (2 * D)) / 16;
    koff[i] = (uint32_t)(r * 2 * D + (slot ^ k_swz<D>(r)) * 16);
    voff[i] = (uint32_t)(r * 2 * D + (slot ^ v_swz<D>(r)) * 16);
  }
  auto issue = [&](int t, char* stage) {
    const int done = t * TILE;
    const int bytes = FULL ? TILE : min(TILE, head_bytes - done);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(reinterpret_cast<const char*>(Kh) + done, bytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(reinterpret_cast<const char*>(Vh) + done, bytes);
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      dma16(rk, stage + (wave * LOADS + i) * 1024, koff[i]);
      dma16(rv, stage + TILE + (wave * LOADS + i) * 1024, voff[i]);
    }
  };

  const int kv_end = CAUSAL ? min(N, q0 + kBR) : N;
  const int n_tiles = (kv_end + kBC - 1) / kBC;

  f32x16 o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o[db] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;

  auto compute = [&](int t, const char* ks) {
    const char* vs = ks + TILE;
    const int key0 = t * kBC;
    if (CAUSAL && key0 > row_w + 31) return;   // wave-uniform: tile fully masked
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) s[kb] = f32x16{};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) s[kb] = mfma32(load_k_frag<D>(ks, kb, kk, lane), qf[kk], s[kb]);
    }
    const bool need_mask = (!FULL && key0 + kBC > N) || (CAUSAL && key0 + kBC - 1 > row_w);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + st_key(kb, r, lane);
          const bool dead = (!FULL && key >= N) || (CAUSAL && key > qrow);
          if (dead) s[kb][r] = -INFINITY;
        }
      }
    }
    float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
    for (int r = 2; r < 16; ++r) mx = fmaxf(mx, s[0][r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[1][r]);
    mx = max_xor32(mx);
    const float mt = mx * c;
    const bool raise = mt > m_run + kRescaleThreshold;
    if (__any(raise)) {
      const float m_new = raise ? mt : m_run;
      const float alpha = (m_new == m_run) ? 1.f : exp2_hw(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] *= alpha;
      m_run = m_new;
    }
    const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
    float rs = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = exp2_hw(fmaf(s[kb][r], c, -m_use));
        s[kb][r] = p;
        rs += p;
      }
    }
    l_run += rs;
    const f16x8 pf[4] = {pack_p(s[0], 0), pack_p(s[0], 1), pack_p(s[1], 0), pack_p(s[1], 1)};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] = mfma32(load_v_frag<D>(vs, j, db, lane), pf[j], o[db]);
    }
  };

  // Two LDS stages; the loop is unrolled by two so stage offsets are constants.
  char* st0 = smem0;
  char* st1 = smem1;
  issue(0, st0);
  wait_vmem();
  __syncthreads();
  for (int t = 0; t < n_tiles; t += 2) {
    if (t + 1 < n_tiles) issue(t + 1, st1);
    compute(t, st0);
    wait_vmem();
    __syncthreads();
    if (t + 1 < n_tiles) {
      if (t + 2 < n_tiles) issue(t + 2, st0);
      compute(t + 1, st1);
      wait_vmem();
      __syncthreads();
    }
  }

  // Epilogue: combine the two half-rows, normalise, store O (and L).
  const float l_tot = sum_xor32(l_run);
  if (FULL || qrow < N) {
    const float inv = 1.f / l_tot;
    f16* orow = O + head + (size_t)qrow * D;
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
    if (WRITE_L && hi == 0) {
      const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
      L[(size_t)bh * N + qrow] = (m_use + log2_hw(l_tot)) * kLn2;
    }
  }
}

template <int D, bool CAUSAL, bool WRITE_L, bool FULL>
static hipError_t launch_fwd(const void* q, const void* k, const void* v, void* o,
                             float* lse, int N, int num_qb, int total, float c,
                             hipStream_t stream) {
  hipLaunchKernelGGL((fa_fwd_kernel<D, CAUSAL, WRITE_L, FULL>), dim3(total),
                     dim3(kThreads), 0, stream, (const f16*)q, (const f16*)k,
                     (const f16*)v, (f16*)o, lse, N, num_qb, total, c);
  return hipGetLastError();
}

template <int D, bool CAUSAL>
static hipError_t dispatch_wl(const void* q, const void* k, const void* v, void* o,
                              float* lse, int N, int num_qb, int total, float c,
                              bool full, hipStream_t s) {
  if (lse) {
    return full ? launch_fwd<D, CAUSAL, true, true>(q, k, v, o, lse, N, num_qb, total, c, s)
                : launch_fwd<D, CAUSAL, true, false>(q, k, v, o, lse, N, num_qb, total, c, s);
  }
  return full ? launch_fwd<D, CAUSAL, false, true>(q, k, v, o, lse, N, num_qb, total, c, s)
              : launch_fwd<D, CAUSAL, false, false>(q, k, v, o, lse, N, num_qb, total, c, s);
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
  hipError_t e;
  if (D == 64) {
    e = causal ? dispatch_wl<64, true>(q, k, v, o, lse, (int)N, num_qb, total, c, full, s)
               : dispatch_wl<64, false>(q, k, v, o, lse, (int)N, num_qb, total, c, full, s);
  } else {
    e = causal ? dispatch_wl<128, true>(q, k, v, o, lse, (int)N, num_qb, total, c, full, s)
               : dispatch_wl<128, false>(q, k, v, o, lse, (int)N, num_qb, total, c, full, s);
  }
  return e == hipSuccess ? FA_OK : -(int)e;
}
