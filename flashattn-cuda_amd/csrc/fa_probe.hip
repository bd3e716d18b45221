// fa_probe.hip — on-device checks of the matrix-core and LDS layouts the
// forward kernel is built on. Test support only (the forward path never calls
// these). The method follows the reference's mma probe
// (cuda/mma_probe.cu:87-254, tests/test_mma_probe.py:35-57): run a single
// matrix instruction on known operands, compare against a host product, and
// keep a negative control that must fail.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "fa_probe.h"
#include "fa_tile.hpp"

namespace fa {

// a: [32][16], b: [16][32], c: [32][32], row-major. variant 1 swaps the two
// k-halves of A only (negative control: the product must be wrong).
__global__ void probe_mfma32_kernel(const f16* a, const f16* b, float* c, int variant) {
  const int l = threadIdx.x;
  const int kh = variant ? 1 - (l >> 5) : (l >> 5);
  f16x8 av, bv;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    av[i] = a[(l & 31) * 16 + 8 * kh + i];
    bv[i] = b[(8 * (l >> 5) + i) * 32 + (l & 31)];
  }
  f32x16 acc = mfma32(av, bv, f32x16{});
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    c[(8 * (r >> 2) + 4 * (l >> 5) + (r & 3)) * 32 + (l & 31)] = acc[r];
  }
}

// a: [16][32], b: [32][16], c: [16][16]. variant 1 reverses A's k-groups.
__global__ void probe_mfma16_kernel(const f16* a, const f16* b, float* c, int variant) {
  const int l = threadIdx.x;
  const int kg = variant ? 3 - (l >> 4) : (l >> 4);
  f16x8 av, bv;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    av[i] = a[(l & 15) * 32 + 8 * kg + i];
    bv[i] = b[(8 * (l >> 4) + i) * 16 + (l & 15)];
  }
  f32x4 acc = mfma16(av, bv, f32x4{});
#pragma unroll
  for (int r = 0; r < 4; ++r) c[(4 * (l >> 4) + r) * 16 + (l & 15)] = acc[r];
}

// Raw ds_read_b64_tr_b16: LDS holds in[0..255]; lane l reads at byte 8*l.
__global__ void probe_tr16_raw_kernel(const uint16_t* in, uint16_t* out) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[256];
  const int l = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) lds[4 * l + i] = in[4 * l + i];
  __syncthreads();
  f16x4 v = lds_read_tr16(reinterpret_cast<const char*>(lds) + 8 * l);
  // Store the vector whole: extracting elements through __builtin_bit_cast was
  // observed to be miscompiled (all four lanes of the vector read element 0).
  *reinterpret_cast<f16x4*>(out + 4 * l) = v;
}

// v_permlane32_swap_b32 with both operands x = in[l]: out[l] = r0, out[64+l] = r1,
// plus the max/sum helpers the forward kernel uses: out[128+l], out[192+l].
__global__ void probe_permlane_kernel(const float* in, float* out) {
  const int l = threadIdx.x;
  const float x = in[l];
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  out[l] = __uint_as_float(r[0]);
  out[64 + l] = __uint_as_float(r[1]);
  out[128 + l] = max_xor32(x);
  out[192 + l] = sum_xor32(x);
}

// Stores a [64][D] tile with the forward kernel's K and V layouts, then reads
// every operand fragment the kernel reads.
//   kout: [2 kb][D/16 kk][64 lanes][8]    (load_k_frag)
//   vout: [4 j][D/32 db][64 lanes][8]     (load_v_frag)
template <int D>
__global__ void probe_frag_kernel(const f16* tile, f16* kout, f16* vout) {
  constexpr int TILE = 64 * D * 2;
  constexpr int CPR = D / 8;
  __shared__ __attribute__((aligned(16))) char smem[2 * TILE];
  const int l = threadIdx.x;
  for (int id = l; id < 64 * CPR; id += 64) {
    const int r = id / CPR, cc = id % CPR;
    const u32x4 x = *reinterpret_cast<const u32x4*>(tile + r * D + cc * 8);
    *reinterpret_cast<u32x4*>(smem + k_off<D>(r, cc)) = x;
    *reinterpret_cast<u32x4*>(smem + TILE + v_off<D>(r, cc)) = x;
  }
  __syncthreads();
  for (int kb = 0; kb < 2; ++kb)
    for (int kk = 0; kk < D / 16; ++kk) {
      f16x8 x = load_k_frag<D>(smem, kb, kk, l);
      *reinterpret_cast<f16x8*>(kout + (((kb * (D / 16) + kk) * 64) + l) * 8) = x;
    }
  for (int j = 0; j < 4; ++j)
    for (int db = 0; db < D / 32; ++db) {
      f16x8 x = load_v_frag<D>(smem + TILE, j, db, l);
      *reinterpret_cast<f16x8*>(vout + (((j * (D / 32) + db) * 64) + l) * 8) = x;
    }
}

// One wave, one 64-key tile, no softmax: S^T = K Q^T, P = fp16(S), O^T = V^T P^T,
// through the kernel's own layouts, loaders and packing. q: [32][D],
// k, v: [64][D], o: [32][D] fp32.
template <int D>
__global__ void probe_chain_kernel(const f16* q, const f16* k, const f16* v, float* o) {
  constexpr int TILE = 64 * D * 2;
  constexpr int CPR = D / 8;
  __shared__ __attribute__((aligned(16))) char smem[2 * TILE];
  const int l = threadIdx.x;
  for (int id = l; id < 64 * CPR; id += 64) {
    const int r = id / CPR, cc = id % CPR;
    *reinterpret_cast<u32x4*>(smem + k_off<D>(r, cc)) =
        *reinterpret_cast<const u32x4*>(k + r * D + cc * 8);
    *reinterpret_cast<u32x4*>(smem + TILE + v_off<D>(r, cc)) =
        *reinterpret_cast<const u32x4*>(v + r * D + cc * 8);
  }
  __syncthreads();
  f16x8 qf[D / 16];
  for (int kk = 0; kk < D / 16; ++kk)
    qf[kk] = *reinterpret_cast<const f16x8*>(q + (l & 31) * D + 16 * kk + 8 * (l >> 5));
  f32x16 s[2];
  for (int kb = 0; kb < 2; ++kb) {
    s[kb] = f32x16{};
    for (int kk = 0; kk < D / 16; ++kk) s[kb] = mfma32(load_k_frag<D>(smem, kb, kk, l), qf[kk], s[kb]);
  }
  f16x8 pf[4] = {pack_p(s[0], 0), pack_p(s[0], 1), pack_p(s[1], 0), pack_p(s[1], 1)};
  for (int db = 0; db < D / 32; ++db) {
    f32x16 acc = f32x16{};
    for (int j = 0; j < 4; ++j) acc = mfma32(load_v_frag<D>(smem + TILE, j, db, l), pf[j], acc);
    for (int r = 0; r < 16; ++r)
      o[(l & 31) * D + 32 * db + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3)] = acc[r];
  }
}

}  // namespace fa

static int finish() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : -(int)e;
}

extern "C" int fa_probe_mfma32(const void* a, const void* b, float* c, int variant, void* stream) {
  if (!a || !b || !c) return 1;
  hipLaunchKernelGGL(fa::probe_mfma32_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const fa::f16*)a, (const fa::f16*)b, c, variant);
  return finish();
}

extern "C" int fa_probe_mfma16(const void* a, const void* b, float* c, int variant, void* stream) {
  if (!a || !b || !c) return 1;
  hipLaunchKernelGGL(fa::probe_mfma16_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const fa::f16*)a, (const fa::f16*)b, c, variant);
  return finish();
}

extern "C" int fa_probe_tr16_raw(const void* in, void* out, void* stream) {
  if (!in || !out) return 1;
  hipLaunchKernelGGL(fa::probe_tr16_raw_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const uint16_t*)in, (uint16_t*)out);
  return finish();
}

extern "C" int fa_probe_permlane(const float* in, float* out, void* stream) {
  if (!in || !out) return 1;
  hipLaunchKernelGGL(fa::probe_permlane_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, in, out);
  return finish();
}

extern "C" int fa_probe_frags(const void* tile, void* kout, void* vout, int64_t D, void* stream) {
  if (!tile || !kout || !vout) return 1;
  if (D == 64) {
    hipLaunchKernelGGL(fa::probe_frag_kernel<64>, dim3(1), dim3(64), 0, (hipStream_t)stream,
                       (const fa::f16*)tile, (fa::f16*)kout, (fa::f16*)vout);
  } else if (D == 128) {
    hipLaunchKernelGGL(fa::probe_frag_kernel<128>, dim3(1), dim3(64), 0, (hipStream_t)stream,
                       (const fa::f16*)tile, (fa::f16*)kout, (fa::f16*)vout);
  } else {
    return 2;
  }
  return finish();
}

extern "C" int fa_probe_chain(const void* q, const void* k, const void* v, float* o, int64_t D,
                              void* stream) {
  if (!q || !k || !v || !o) return 1;
  if (D == 64) {
    hipLaunchKernelGGL(fa::probe_chain_kernel<64>, dim3(1), dim3(64), 0, (hipStream_t)stream,
                       (const fa::f16*)q, (const fa::f16*)k, (const fa::f16*)v, o);
  } else if (D == 128) {
    hipLaunchKernelGGL(fa::probe_chain_kernel<128>, dim3(1), dim3(64), 0, (hipStream_t)stream,
                       (const fa::f16*)q, (const fa::f16*)k, (const fa::f16*)v, o);
  } else {
    return 2;
  }
  return finish();
}

namespace fa {
// Streaming read of `n` 16-byte vectors folded into one word per lane
// (written only on a 2^-32 chance, so the loads stay and the stores do not
// count): the HBM read rate a plain kernel reaches, the ceiling the paged
// decode is compared with.
__global__ void __launch_bounds__(256)
probe_read_kernel(const uint4* __restrict__ p, size_t n, uint32_t* __restrict__ sink) {
  // Each workgroup streams one contiguous chunk of the buffer (the last one
  // also the remainder), 8 loads of 16 bytes per thread in flight, with the
  // non-temporal hint: measured on MI355X over 4 GiB, 7.0-7.1 TB/s, against
  // 6.2-6.3 TB/s for the same loads without the hint and 5.7-6.2 TB/s for a
  // grid-stride loop whose 8 loads lie a grid apart.
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const size_t per = n / gridDim.x;
  const size_t begin = (size_t)blockIdx.x * per;
  const size_t end = blockIdx.x + 1 == gridDim.x ? n : begin + per;
  const u4* q = reinterpret_cast<const u4*>(p);
  uint32_t acc = 0;
  size_t i = begin + threadIdx.x;
  for (; i + 7 * 256 < end; i += 8 * 256) {
    u4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(q + i + u * 256);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < end; i += 256) {
    const u4 v = __builtin_nontemporal_load(q + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

// Gather read of 4 KiB pages of two pools through a table (the paged
// decode's access pattern without its arithmetic): lane l of a wave reads
// bytes 16 l .. 16 l + 15 of each 1 KiB quarter of the page, four loads per
// pool and page, one page per wave in flight.
template <bool NT>
__global__ void __launch_bounds__(256)
probe_gather_kernel(const uint4* __restrict__ k, const uint4* __restrict__ v,
                    const int32_t* __restrict__ table, int64_t pages, int per,
                    uint32_t* __restrict__ sink) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t first = (int64_t)blockIdx.x * per;
  const int n = (int)min((int64_t)per, pages - first);
  const u4* kq = reinterpret_cast<const u4*>(k);
  const u4* vq = reinterpret_cast<const u4*>(v);
  uint32_t acc = 0;
  for (int i = wave; i < n; i += 4) {
    const int64_t pid = min(max((int64_t)table[first + i], (int64_t)0), pages - 1);
    const size_t base = (size_t)pid * 256 + lane;   // 256 16-byte vectors per page
    u4 x[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = NT ? __builtin_nontemporal_load(kq + base + 64 * j) : kq[base + 64 * j];
      x[4 + j] = NT ? __builtin_nontemporal_load(vq + base + 64 * j) : vq[base + 64 * j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= x[j][0] ^ x[j][1] ^ x[j][2] ^ x[j][3];
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;
}
}  // namespace fa

extern "C" int fa_probe_gather_bw(const void* k, const void* v, const int32_t* table,
                                  int64_t pages, int pages_per_wg, int nontemporal,
                                  uint32_t* sink, void* stream) {
  if (!k || !v || !table || !sink) return 1;
  if (pages < 1 || pages_per_wg < 1 || ((reinterpret_cast<uintptr_t>(k) |
                                         reinterpret_cast<uintptr_t>(v)) & 15u))
    return 2;
  const int64_t wgs = (pages + pages_per_wg - 1) / pages_per_wg;
  if (wgs > (int64_t(1) << 31) - 1) return 2;
  if (nontemporal)
    hipLaunchKernelGGL(fa::probe_gather_kernel<true>, dim3((unsigned)wgs), dim3(256), 0,
                       (hipStream_t)stream, (const uint4*)k, (const uint4*)v, table, pages,
                       pages_per_wg, sink);
  else
    hipLaunchKernelGGL(fa::probe_gather_kernel<false>, dim3((unsigned)wgs), dim3(256), 0,
                       (hipStream_t)stream, (const uint4*)k, (const uint4*)v, table, pages,
                       pages_per_wg, sink);
  return finish();
}

extern "C" int fa_probe_read_bw(const void* p, int64_t bytes, int blocks, uint32_t* sink,
                                void* stream) {
  if (!p || !sink) return 1;
  if (bytes < 16 || (bytes & 15) || blocks < 1 || (reinterpret_cast<uintptr_t>(p) & 15u)) return 2;
  hipLaunchKernelGGL(fa::probe_read_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)p, (size_t)(bytes / 16), sink);
  return finish();
}
