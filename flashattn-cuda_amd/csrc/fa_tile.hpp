// fa_tile.hpp — gfx950 building blocks shared by the forward kernel and the
// layout probes: MFMA wrappers, LDS tile layouts, operand loaders, P packing.
//
// Matrix-core conventions (v_mfma_f32_32x32x16_f16, one wave64):
//   A (32 x 16): lane l holds A[l % 32][8*(l/32) + i], i = 0..7
//   B (16 x 32): lane l holds B[8*(l/32) + i][l % 32], i = 0..7
//   C (32 x 32): lane l, register r holds C[8*(r/4) + 4*(l/32) + r%4][l % 32]
// The layout probes in fa_probe.hip check these on the device.
//
// The forward kernel computes S^T = K Q^T (A = K tile from LDS, B = Q held in
// registers), so lane l owns query l%32 and 16 of the 32 keys of a block; row
// statistics are in-lane plus one exchange with lane l^32. It then computes
// O^T = V^T P^T with P^T taken straight from the S^T accumulator (no LDS round
// trip): the PV reduction index is the key, so keys may be visited in any
// order as long as V^T and P^T agree. The order used is the S^T register order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

namespace fa {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Operand registers hold raw 16-bit values; BF16 selects how they are read.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <bool BF16>
__device__ __forceinline__ f32x16 mma32(f16x8 a, f16x8 b, f32x16 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return mfma32(a, b, c);
  }
}

// 2^x on the hardware transcendental unit (v_exp_f32); 2^-inf = 0.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }
// log2(x) on v_log_f32.
__device__ __forceinline__ float log2_hw(float x) { return __builtin_amdgcn_logf(x); }

// v_permlane32_swap_b32 with both operands x: element 0 of the result holds,
// in lanes 32..63, x of lane l-32 (lanes 0..31 keep x); element 1 holds, in
// lanes 0..31, x of lane l+32 (lanes 32..63 keep x). So {r0, r1} is
// {x[l], x[l^32]} in some order in every lane.
__device__ __forceinline__ float max_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float sum_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Raw buffer resource over `bytes` bytes at `base`: loads at offsets beyond
// `bytes` return zero instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// make_rsrc for a wave-uniform range that must sit in SGPRs (the inline
// asm of the LDS copies below takes the descriptor as an SGPR operand): the
// base and length go through readfirstlane, which is free when the compiler
// already holds them in SGPRs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_s(const void* base, int bytes) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const void* p = reinterpret_cast<const void*>(((uintptr_t)hi << 32) | lo);
  return make_rsrc(p, __builtin_amdgcn_readfirstlane(bytes));
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// 16 bytes per lane from global (rsrc + voffset) straight into LDS at byte
// lds + 16*lane (lds is wave-uniform). Written as inline assembly so the
// compiler does not treat it as an LDS store: it would otherwise wait for
// every DMA in flight before any LDS read it cannot prove disjoint. The
// kernels order these copies themselves (s_waitcnt vmcnt(0) + barrier before
// the data is read), and nothing else in them uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voffset), "s"(r)
               : "memory", "m0");
}

// 4 bytes per lane from global (rsrc + voffset) into LDS at byte lds + 4*lane;
// the dword form needs only 4-byte alignment of the source.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voffset), "s"(r)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(0) through the builtin, so the compiler also knows that its
// own vector-memory loads issued before this point have completed (gfx9
// encoding: vmcnt bits [3:0] and [15:14] = 0, expcnt 7, lgkmcnt 15).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// f(integral_constant<int, I>) for I = B .. E-1, expanded at compile time
// (a fixed instruction schedule must not depend on the loop unroller).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] at bits 3:0, vmcnt[5:4] at
// bits 15:14, expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// ---------------------------------------------------------------------------
// LDS tile layouts. A K or V tile is BC rows (keys) x D fp16, row stride 2*D
// bytes, stored as 16-byte chunks (8 halves). Chunk c of row r lives at chunk
// slot pos(r, c) of that row; pos is an XOR swizzle chosen so that the
// operand reads below hit distinct LDS banks within each 16-lane group.
// ---------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ int k_swz(int r) {
  if constexpr (D == 64) {
    return (r >> 1) & 7;
  } else {
    return r & 15;
  }
}

template <int D>
__device__ __forceinline__ int v_swz(int r) {
  if constexpr (D == 64) {
    return ((r >> 1) & 1) << 2;
  } else {
    return (r & 3) << 2;
  }
}

// XOR swizzles are involutions: slot = c ^ swz(r) and c = slot ^ swz(r).
template <int D>
__device__ __forceinline__ int k_slot(int r, int c) { return c ^ k_swz<D>(r); }

template <int D>
__device__ __forceinline__ int v_slot(int r, int c) { return c ^ v_swz<D>(r); }

template <int D>
__device__ __forceinline__ int k_off(int r, int c) { return r * (2 * D) + k_slot<D>(r, c) * 16; }

template <int D>
__device__ __forceinline__ int v_off(int r, int c) { return r * (2 * D) + v_slot<D>(r, c) * 16; }

// LDS pointers for the pipelined kernel's operand reads: arithmetic on them
// stays in the 32-bit LDS address space, so constant offsets fold into the
// DS instructions' offset field.
typedef const __attribute__((address_space(3))) char* lds_cp;

// A lane's base address in LDS, opaque to the optimiser: every read of the
// step is then this base plus a constant, instead of a separately hoisted
// loop-invariant offset plus the step's slot base per read.
__device__ __forceinline__ lds_cp lds_lane_base(uint32_t a) {
  asm("" : "+v"(a));
  return (lds_cp)(size_t)a;
}

__device__ __forceinline__ f16x8 lds_b128(lds_cp p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) f16x8*>(p);
}

__device__ __forceinline__ f16x4 lds_tr16(lds_cp p) {
  typedef __attribute__((address_space(3))) fp16x4_t lds_fp16x4;
  fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4*)(p));
  return __builtin_bit_cast(f16x4, v);
}

// V fragment (see load_v_frag) whose k-step-0 address is p.
template <int D>
__device__ __forceinline__ f16x8 v_frag_lds(lds_cp p) {
  f16x4 lo = lds_tr16(p);
  f16x4 up = lds_tr16(p + 8 * 2 * D);
  return f16x8{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
}

// A operand of S^T = K Q^T for key block kb (32 keys) and k-step kk (16 of D).
// The K swizzle depends on the row only modulo 16, so block kb is the block-0
// fragment shifted by 32 rows: k_frag_off(kk, lane) + 32 * kb * 2D.
template <int D>
__device__ __forceinline__ int k_frag_off(int kk, int lane) {
  return k_off<D>(lane & 31, 2 * kk + (lane >> 5));
}

template <int D>
__device__ __forceinline__ f16x8 load_k_frag(const char* ks, int kb, int kk, int lane) {
  return *reinterpret_cast<const f16x8*>(ks + 32 * kb * 2 * D + k_frag_off<D>(kk, lane));
}

// ds_read_b64_tr_b16: within each group of 16 lanes, lane s supplies the
// address of 4 consecutive halves M[s][0..3]; it receives
// out[e] = M[4*e + s/4][s%4]. If lane s points at row (k0 + s/4),
// columns (d0 + 4*(s%4)) .. +3 of a row-major [key][d] tile, lane s receives
// the column d0 + s for keys k0 .. k0+3.
__device__ __forceinline__ f16x4 lds_read_tr16(const char* p) {
  typedef __attribute__((address_space(3))) fp16x4_t lds_fp16x4;
  fp16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_fp16x4*)(p));
  return __builtin_bit_cast(f16x4, v);
}

// A operand of O^T = V^T P^T for PV k-step j (16 keys of the 64-key tile) and
// d-block db (32 of D). Slot i of lane l must hold V[key(j, i, l)][32*db + l%32]
// with key(j, i, l) = 16*j + 8*(i/4) + 4*(l/32) + i%4, the key order of the
// S^T accumulator registers (see pack_p). Lane l reads rows r0 = 4*(l/32) +
// (l%16)/4 (+16 j) and r0 + 8; the V swizzle depends on the row only modulo
// 4, so k-step j and the upper 4 keys are constant row shifts of
// v_frag_off(db, lane).
template <int D>
__device__ __forceinline__ int v_frag_off(int db, int lane) {
  const int s = lane & 15;
  const int d = 32 * db + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
  const int r0 = 4 * (lane >> 5) + (s >> 2);
  return v_off<D>(r0, d >> 3) + 8 * ((d >> 2) & 1);
}

// The fragment whose k-step j = 0 row-0 address is p (= tile + v_frag_off).
template <int D>
__device__ __forceinline__ f16x8 v_frag_at(const char* p) {
  f16x4 lo = lds_read_tr16(p);
  f16x4 up = lds_read_tr16(p + 8 * 2 * D);
  return f16x8{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
}

template <int D>
__device__ __forceinline__ f16x8 load_v_frag(const char* vs, int j, int db, int lane) {
  return v_frag_at<D>(vs + 16 * j * 2 * D + v_frag_off<D>(db, lane));
}

// Key index (within a 64-key tile) held by register r of key block kb in lane l.
__device__ __forceinline__ int st_key(int kb, int r, int lane) {
  return 32 * kb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}

// fp32 -> fp16 round-to-nearest-even, two at a time (v_cvt_pk_f16_f32).
__device__ __forceinline__ f16x2 cvt2(float a, float b) {
  return f16x2{(f16)a, (f16)b};
}

// fp32 -> 16-bit operand pair: fp16 (v_cvt_pk_f16_f32) or, with BF16,
// bfloat16 round-to-nearest-even (v_cvt_pk_bf16_f32), as raw bits.
template <bool BF16>
__device__ __forceinline__ f16x2 cvt2x(float a, float b) {
  if constexpr (BF16) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(f16x2, __builtin_convertvector(f32x2_t{a, b}, bf16x2));
  } else {
    return cvt2(a, b);
  }
}

// B operand (P^T) of PV k-step j from the S^T accumulators p[2] of a tile.
__device__ __forceinline__ f16x8 pack_p(const f32x16& p, int half_sel) {
  const int b = 8 * half_sel;
  f16x2 x0 = cvt2(p[b + 0], p[b + 1]);
  f16x2 x1 = cvt2(p[b + 2], p[b + 3]);
  f16x2 x2 = cvt2(p[b + 4], p[b + 5]);
  f16x2 x3 = cvt2(p[b + 6], p[b + 7]);
  return f16x8{x0[0], x0[1], x1[0], x1[1], x2[0], x2[1], x3[0], x3[1]};
}

// pack_p with the operand format chosen by BF16 (bfloat16 bits in the same
// register layout).
template <bool BF16>
__device__ __forceinline__ f16x8 pack_px(const f32x16& p, int half_sel) {
  const int b = 8 * half_sel;
  f16x2 x0 = cvt2x<BF16>(p[b + 0], p[b + 1]);
  f16x2 x1 = cvt2x<BF16>(p[b + 2], p[b + 3]);
  f16x2 x2 = cvt2x<BF16>(p[b + 4], p[b + 5]);
  f16x2 x3 = cvt2x<BF16>(p[b + 6], p[b + 7]);
  return f16x8{x0[0], x0[1], x1[0], x1[1], x2[0], x2[1], x3[0], x3[1]};
}

// Where the heads of one launch live. Dense: Q/O [B, H, N, D], K/V
// [B, H/group, N, D], L [B, H, N]. Varlen (cu != nullptr): sequences packed
// head-major, Q/O [H, total, D], K/V [H/group, total, D], L [H, total];
// sequence b is rows cu[b] .. cu[b+1] of every head and N is the grid's
// maximum length. Query head h reads KV head h / group (GQA / MQA).
struct Geom {
  const int32_t* cu;
  int N;
  int H;
  int group;
  int total;
  int B;       // varlen: number of sequences
  int nxcd;    // XCDs of the device the launch runs on (set by the launcher)
};

// Workgroup g of a 1-D grid of `total` lands on XCD g % nxcd (the dispatcher
// deals consecutive workgroups to the XCDs in turn). Map it to a logical index
// so that each XCD gets one contiguous range of logical indices: the row
// blocks of a head then share one XCD's L2, which serves their K/V after the
// first fetch. nxcd <= 1 (one XCD, or a partition of one) is the identity.
__device__ __forceinline__ int xcd_remap(int g, int total, int nxcd) {
  if (nxcd <= 1) return g;
  const int q = total / nxcd, r = total % nxcd;
  const int xcd = g % nxcd, slot = g / nxcd;
  return (xcd < r) ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
}

// Compute units and XCDs of a device: read once per device from the runtime
// (hipDeviceAttributeMultiprocessorCount, hipDeviceAttributeNumberOfXccs) and
// kept for later calls. A partitioned MI355X reports its own share (e.g. 32
// CUs on one XCD per partition), so the kernel choices and the XCD remap
// follow the device the launch actually runs on.
struct Topology {
  int cus;
  int xcds;
};

inline Topology device_topology(int dev) {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cache[kMaxDev];   // cus << 8 | xcds, 0 = not read yet
  const bool cacheable = dev >= 0 && dev < kMaxDev;
  if (cacheable) {
    const int v = cache[dev].load(std::memory_order_relaxed);
    if (v != 0) return Topology{v >> 8, v & 0xff};
  }
  int cus = 0, xcds = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;   // MI355X, if the runtime cannot say
  if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || xcds <= 0)
    xcds = 1;
  if (xcds > 255) xcds = 255;
  if (cacheable) cache[dev].store(cus << 8 | xcds, std::memory_order_relaxed);
  return Topology{cus, xcds};
}

// Topology of the device that runs work queued on `stream`.
inline Topology stream_topology(hipStream_t stream) {
  int dev = 0;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess && hipGetDevice(&dev) != hipSuccess) dev = 0;
  return device_topology(dev);
}

// One (b, h): element offsets of its Q/O and K/V rows, of its L row, and its
// length. Varlen bounds are clamped into [0, total] and to N, so a malformed
// cu never moves a head's buffer range outside its own rows.
struct HeadView {
  size_t q, kv, l;
  int n;
};

template <int D>
__device__ __forceinline__ HeadView head_view(const Geom& g, int bh) {
  HeadView v;
  if (g.cu == nullptr) {
    v.n = g.N;
    v.q = (size_t)bh * g.N * D;
    v.kv = (size_t)(bh / g.group) * g.N * D;
    v.l = (size_t)bh * g.N;
  } else {
    // Head-major unit order (h, then b): the grid is cut into one contiguous
    // range per XCD, and a range of whole heads holds every sequence's share
    // of the work, where a range of whole sequences would give one XCD all of
    // a long sequence.
    const int h = bh / g.B, b = bh - h * g.B;
    const int s0 = min(max(g.cu[b], 0), g.total);
    const int s1 = min(max(g.cu[b + 1], s0), g.total);
    v.n = min(s1 - s0, g.N);
    v.q = ((size_t)h * g.total + s0) * D;
    v.kv = ((size_t)(h / g.group) * g.total + s0) * D;
    v.l = (size_t)h * g.total + s0;
  }
  return v;
}

}  // namespace fa
