// fa_capi.cpp — host-only part of the C ABI: argument validation and status
// strings. No HIP call is made here, so every error path runs without a GPU.
//
// fa_validate_fwd mirrors the argument checks of the reference launcher
// fa3db_full_forward_impl (cuda/flash_attn_fa3_db_full.cu:352-363): head dim,
// N > 0, and the B*H grid limit, widened to D in {64, 128}; shape/device
// equality of Q/K/V is the binding's job because the C ABI only sees
// pointers.
#include <stdint.h>

#include "fa_mi355x.h"

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Largest element count the kernels index with 32-bit in-head offsets.
constexpr int64_t kMaxHeadElems = (int64_t(1) << 31) - 1;
constexpr int64_t kMaxGrid = (int64_t(1) << 31) - 1;

}  // namespace

extern "C" const char* fa_status_str(int status) {
  switch (status) {
    case FA_OK: return "ok";
    case FA_ERR_NULL_POINTER: return "a required pointer is NULL";
    case FA_ERR_HEAD_DIM: return "Head dimension must be 64 or 128";
    case FA_ERR_SEQ_LEN: return "N must be > 0";
    case FA_ERR_BATCH_HEADS: return "B and H must be > 0";
    case FA_ERR_ALIGNMENT: return "tensor pointers must be 16-byte aligned";
    case FA_ERR_TOO_LARGE: return "size exceeds the kernels' 32-bit index range";
    case FA_ERR_PAGE_SIZE: return "page_size must be 16";
    case FA_ERR_NUM_SPLITS: return "num_splits must be in [1, 16]";
    case FA_ERR_MAX_PAGES: return "max_pages must be > 0";
    case FA_ERR_NUM_PAGES: return "num_pages must be > 0";
    case FA_ERR_KV_HEADS: return "H must be a positive multiple of H_kv";
    case FA_ERR_SCRATCH_SIZE:
      return "B*H*num_splits*(D+1) exceeds FA_DECODE_SCRATCH_FLOATS (no-alloc decode)";
    default: break;
  }
  if (status < 0) return "HIP error (negated hipError_t)";
  return "unknown fa_mi355x status";
}

extern "C" int fa_abi_version(void) { return FA_ABI_VERSION; }

extern "C" int fa_validate_fwd(const void* q, const void* k, const void* v, const void* o,
                               int64_t B, int64_t H, int64_t N, int64_t D) {
  if (!q || !k || !v || !o) return FA_ERR_NULL_POINTER;
  if (D != 64 && D != 128) return FA_ERR_HEAD_DIM;
  if (N <= 0) return FA_ERR_SEQ_LEN;
  if (B <= 0 || H <= 0) return FA_ERR_BATCH_HEADS;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return FA_ERR_ALIGNMENT;
  // One head of K or V is addressed through a 32-bit buffer range (bytes).
  if (N * D * 2 > kMaxHeadElems) return FA_ERR_TOO_LARGE;
  if (B > kMaxGrid / H) return FA_ERR_TOO_LARGE;
  const int64_t bh = B * H;
  const int64_t num_qb = (N + 127) / 128;
  if (bh > kMaxGrid / num_qb) return FA_ERR_TOO_LARGE;
  return FA_OK;
}

// GQA: the dense checks plus the head grouping.
extern "C" int fa_validate_fwd_gqa(const void* q, const void* k, const void* v, const void* o,
                                   int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D) {
  const int st = fa_validate_fwd(q, k, v, o, B, H, N, D);
  if (st != FA_OK) return st;
  if (H_kv <= 0 || H % H_kv != 0) return FA_ERR_KV_HEADS;
  return FA_OK;
}

// Varlen: one head's packed rows are addressed with size_t offsets; one
// sequence (at most max_seqlen rows) through a 32-bit buffer range.
extern "C" int fa_validate_fwd_varlen(const void* q, const void* k, const void* v, const void* o,
                                      const int32_t* cu_seqlens, int64_t B, int64_t H,
                                      int64_t H_kv, int64_t max_seqlen, int64_t total,
                                      int64_t D) {
  if (!q || !k || !v || !o || !cu_seqlens) return FA_ERR_NULL_POINTER;
  if (D != 64 && D != 128) return FA_ERR_HEAD_DIM;
  if (max_seqlen <= 0 || total < 0) return FA_ERR_SEQ_LEN;
  if (B <= 0 || H <= 0) return FA_ERR_BATCH_HEADS;
  if (H_kv <= 0 || H % H_kv != 0) return FA_ERR_KV_HEADS;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return FA_ERR_ALIGNMENT;
  if (reinterpret_cast<uintptr_t>(cu_seqlens) & 3u) return FA_ERR_ALIGNMENT;
  if (max_seqlen * D * 2 > kMaxHeadElems || total > kMaxGrid) return FA_ERR_TOO_LARGE;
  if (B > kMaxGrid / H) return FA_ERR_TOO_LARGE;
  const int64_t num_qb = (max_seqlen + 127) / 128;
  if (B * H > kMaxGrid / num_qb) return FA_ERR_TOO_LARGE;
  return FA_OK;
}

// Mirrors the reference backward launcher's checks (cuda/flash_attn_kernel.cu:
// 425-432: CUDA tensors, head dimension), widened to D in {64, 128}, plus the
// C ABI's own pointer, alignment and index-range checks.
extern "C" int fa_validate_bwd(const void* q, const void* k, const void* v, const void* o,
                               const void* dout, const float* lse, const float* dq,
                               const float* dk, const float* dv, const float* workspace,
                               int64_t B, int64_t H, int64_t N, int64_t D) {
  if (!dout || !lse || !dq || !dk || !dv || !workspace) return FA_ERR_NULL_POINTER;
  const int st = fa_validate_fwd(q, k, v, o, B, H, N, D);
  if (st != FA_OK) return st;
  if (!aligned16(dout) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
    return FA_ERR_ALIGNMENT;
  if ((reinterpret_cast<uintptr_t>(lse) & 3u) != 0 ||
      (reinterpret_cast<uintptr_t>(workspace) & 3u) != 0)
    return FA_ERR_ALIGNMENT;
  // The row-sum kernel's grid (32 rows per workgroup) and the per-head float
  // offsets of the gradients.
  if (B * H > kMaxGrid / N) return FA_ERR_TOO_LARGE;
  if ((B * H * N + 31) / 32 > kMaxGrid) return FA_ERR_TOO_LARGE;
  return FA_OK;
}

// Varlen backward (no reference counterpart): the varlen forward's checks on
// q/k/v/o plus the backward's gradient, L and workspace pointers and the row
// grid of the D_i pass.
extern "C" int fa_validate_bwd_varlen(const void* q, const void* k, const void* v, const void* o,
                                      const void* dout, const float* lse, const float* dq,
                                      const float* dk, const float* dv, const float* workspace,
                                      const int32_t* cu_seqlens, int64_t B, int64_t H,
                                      int64_t H_kv, int64_t max_seqlen, int64_t total,
                                      int64_t D) {
  if (!dout || !lse || !dq || !dk || !dv || !workspace) return FA_ERR_NULL_POINTER;
  const int st = fa_validate_fwd_varlen(q, k, v, o, cu_seqlens, B, H, H_kv, max_seqlen, total, D);
  if (st != FA_OK) return st;
  if (!aligned16(dout) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
    return FA_ERR_ALIGNMENT;
  if ((reinterpret_cast<uintptr_t>(lse) & 3u) != 0 ||
      (reinterpret_cast<uintptr_t>(workspace) & 3u) != 0)
    return FA_ERR_ALIGNMENT;
  if (H > kMaxGrid / (total > 0 ? total : 1)) return FA_ERR_TOO_LARGE;
  if ((H * total + 31) / 32 > kMaxGrid) return FA_ERR_TOO_LARGE;
  return FA_OK;
}

// Decode arguments (no reference counterpart): pool/page-table shapes, the
// split count and the grid limits of the split pass.
extern "C" int fa_validate_decode(const void* q, const void* k_pool, const void* v_pool,
                                  const int32_t* page_table, const int32_t* ctx_lens,
                                  int64_t B, int64_t H, int64_t D, int64_t page_size,
                                  int64_t max_pages, int64_t num_pages, int64_t num_splits) {
  if (!q || !k_pool || !v_pool || !page_table || !ctx_lens) return FA_ERR_NULL_POINTER;
  if (D != 64 && D != 128) return FA_ERR_HEAD_DIM;
  if (B <= 0 || H <= 0) return FA_ERR_BATCH_HEADS;
  if (page_size != 16) return FA_ERR_PAGE_SIZE;
  if (num_splits < 1 || num_splits > 16) return FA_ERR_NUM_SPLITS;
  if (max_pages <= 0) return FA_ERR_MAX_PAGES;
  if (num_pages <= 0) return FA_ERR_NUM_PAGES;
  if (!aligned16(q) || !aligned16(k_pool) || !aligned16(v_pool)) return FA_ERR_ALIGNMENT;
  if ((reinterpret_cast<uintptr_t>(page_table) & 3u) || (reinterpret_cast<uintptr_t>(ctx_lens) & 3u))
    return FA_ERR_ALIGNMENT;
  // Grid is (num_splits, H, B); y and z are limited to 65535 on this target.
  if (H > 65535 || B > 65535) return FA_ERR_TOO_LARGE;
  if (B > kMaxHeadElems / max_pages) return FA_ERR_TOO_LARGE;
  if (max_pages > kMaxHeadElems / page_size) return FA_ERR_TOO_LARGE;
  return FA_OK;
}

// KV page writer arguments (no reference counterpart). T = 0 is a valid
// no-op; grid is (ceil(T / rows), H, B).
extern "C" int fa_validate_kv_append(const void* k_new, const void* v_new,
                                     const int32_t* page_table, const int32_t* start_pos,
                                     const int32_t* new_lens, const void* k_pool,
                                     const void* v_pool, const int32_t* bad, int64_t B, int64_t H,
                                     int64_t T, int64_t D, int64_t page_size, int64_t max_pages,
                                     int64_t num_pages) {
  // k_new/v_new may be NULL when there is nothing to copy (T = 0: an empty
  // tensor has no storage).
  if ((T != 0 && (!k_new || !v_new)) || !page_table || !start_pos || !k_pool || !v_pool)
    return FA_ERR_NULL_POINTER;
  if (D != 64 && D != 128) return FA_ERR_HEAD_DIM;
  if (T < 0) return FA_ERR_SEQ_LEN;
  if (B <= 0 || H <= 0) return FA_ERR_BATCH_HEADS;
  if (page_size != 16) return FA_ERR_PAGE_SIZE;
  if (max_pages <= 0) return FA_ERR_MAX_PAGES;
  if (num_pages <= 0) return FA_ERR_NUM_PAGES;
  if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(k_pool) || !aligned16(v_pool))
    return FA_ERR_ALIGNMENT;
  const auto a4 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; };
  if (!a4(page_table) || !a4(start_pos) || !a4(new_lens) || !a4(bad)) return FA_ERR_ALIGNMENT;
  if (H > 65535 || B > 65535) return FA_ERR_TOO_LARGE;
  if (T > kMaxGrid || max_pages > kMaxGrid || num_pages > kMaxGrid) return FA_ERR_TOO_LARGE;
  return FA_OK;
}

extern "C" int64_t fa_decode_workspace_floats(int64_t B, int64_t H, int64_t D,
                                              int64_t num_splits) {
  if (B <= 0 || H <= 0 || D <= 0 || num_splits <= 0) return 0;
  return B * H * num_splits * (D + 1);
}
