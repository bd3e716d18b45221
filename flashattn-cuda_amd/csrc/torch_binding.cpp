// torch_binding.cpp — the reference's torch-extension surface, over the C ABI.
//
// Mirrors the reference module built from cuda/flash_attn_fa3_db_full.cu:
//   forward(Q, K, V)      -> [O half [B,H,N,D], L float [B,H,N]]   (:405-408)
//   forward_only(Q, K, V) -> O                                      (:410-413)
// and the backward of the reference's first module (cuda/flash_attn_kernel.cu):
//   backward(Q, K, V, O, dO, L) -> [dQ, dK, dV] float [B,H,N,D]     (:417-503)
// with the same argument checks and messages as fa3db_full_forward_impl
// (:352-363), the same fp16 cast of the inputs (:366-368), fresh outputs on
// Q's device (:370-376) and an asynchronous launch on the current stream
// (:378-399). Additions: a `causal` flag (default false) and D = 128, plus the
// paged decode entry points. Kernels are reached only through the C ABI in
// include/fa_mi355x.h; this file makes no HIP call of its own.
#include <torch/extension.h>

#include <limits>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <vector>

#include "fa_mi355x.h"
#include "fa_probe.h"

namespace {

void* current_stream(const torch::Tensor& t) {
  return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.get_device()).stream());
}

void check_status(int st, const char* what) {
  TORCH_CHECK(st == FA_OK, what, " failed: ", fa_status_str(st), " (status ", st, ")");
}

// variant 0: the default kernel, split over the keys where
// fa_fwd_splitkv_plan asks for it (few row blocks, or causal at small B*H);
// variant > 0: one explicit kernel variant; splits > 0: that split count.
std::pair<torch::Tensor, torch::Tensor> forward_impl(torch::Tensor Q, torch::Tensor K,
                                                     torch::Tensor V, bool want_L, bool causal,
                                                     int variant = 0, int64_t splits = 0) {
  TORCH_CHECK(Q.is_cuda() && K.is_cuda() && V.is_cuda(), "Q/K/V must be CUDA tensors");
  TORCH_CHECK(Q.dim() == 4, "Q must be 4D [B, H, N, D]");
  const int64_t B = Q.size(0), H = Q.size(1), N = Q.size(2), D = Q.size(3);
  TORCH_CHECK(D == 64 || D == 128, "Head dimension must be 64 or 128");
  TORCH_CHECK(N > 0, "N must be > 0");
  TORCH_CHECK(K.dim() == 4 && V.sizes() == K.sizes() && K.size(0) == B && K.size(2) == N &&
                  K.size(3) == D,
              "K and V must have the same shape as Q (self-attention only), or [B, H_kv, N, D] "
              "with H a multiple of H_kv");
  const int64_t Hkv = K.size(1);
  TORCH_CHECK(Hkv > 0 && H % Hkv == 0, "H must be a positive multiple of K/V's head count");
  TORCH_CHECK(K.device() == Q.device() && V.device() == Q.device(),
              "Q/K/V must be on the same device");
  TORCH_CHECK(Q.is_floating_point() && K.is_floating_point() && V.is_floating_point(),
              "Q/K/V must be floating point");

  const c10::DeviceGuard guard(Q.device());
  const int64_t BH = B * H;
  auto Qh = Q.to(torch::kHalf).reshape({BH, N, D}).contiguous();
  auto Kh = K.to(torch::kHalf).reshape({B * Hkv, N, D}).contiguous();
  auto Vh = V.to(torch::kHalf).reshape({B * Hkv, N, D}).contiguous();
  auto O = torch::empty({BH, N, D}, Qh.options());
  torch::Tensor L;
  float* L_ptr = nullptr;
  if (want_L) {
    L = torch::empty({BH, N}, Qh.options().dtype(torch::kFloat));
    L_ptr = L.data_ptr<float>();
  }
  TORCH_CHECK(variant == 0 || Hkv == H, "explicit kernel variants take H_kv == H");
  const int64_t nsplit =
      variant != 0 ? 1 : (splits > 0 ? splits : fa_fwd_splitkv_plan(B, H, N, D, causal ? 1 : 0));
  int st;
  if (nsplit > 1) {
    auto ws = torch::empty({fa_fwd_splitkv_workspace_floats(B, H, N, D, nsplit)},
                           Qh.options().dtype(torch::kFloat));
    st = fa_fwd_splitkv_f16(Qh.data_ptr(), Kh.data_ptr(), Vh.data_ptr(), O.data_ptr(), L_ptr,
                            ws.data_ptr<float>(), B, H, Hkv, N, D, causal ? 1 : 0, nsplit,
                            current_stream(Qh));
  } else if (variant == 0) {
    st = fa_fwd_gqa_f16(Qh.data_ptr(), Kh.data_ptr(), Vh.data_ptr(), O.data_ptr(), L_ptr, B, H,
                        Hkv, N, D, causal ? 1 : 0, current_stream(Qh));
  } else {
    st = fa_probe_fwd_variant(Qh.data_ptr(), Kh.data_ptr(), Vh.data_ptr(), O.data_ptr(), L_ptr,
                              B, H, N, D, causal ? 1 : 0, variant, current_stream(Qh));
  }
  check_status(st, "fa_fwd_f16");
  return {O.reshape({B, H, N, D}), want_L ? L.reshape({B, H, N}) : torch::Tensor()};
}

std::vector<torch::Tensor> forward(torch::Tensor Q, torch::Tensor K, torch::Tensor V, bool causal) {
  auto r = forward_impl(Q, K, V, /*want_L=*/true, causal);
  return {r.first, r.second};
}

torch::Tensor forward_only(torch::Tensor Q, torch::Tensor K, torch::Tensor V, bool causal) {
  return forward_impl(Q, K, V, /*want_L=*/false, causal).first;
}

// forward_bf16(Q, K, V, causal=False) -> [O bf16, L float]: the bfloat16
// forward (K/V may have fewer heads, GQA). Inputs are cast to bf16. No
// reference counterpart (the reference module is fp16-only).
std::vector<torch::Tensor> forward_bf16(torch::Tensor Q, torch::Tensor K, torch::Tensor V,
                                        bool causal, bool want_L) {
  TORCH_CHECK(Q.is_cuda() && K.is_cuda() && V.is_cuda(), "Q/K/V must be CUDA tensors");
  TORCH_CHECK(Q.dim() == 4, "Q must be 4D [B, H, N, D]");
  const int64_t B = Q.size(0), H = Q.size(1), N = Q.size(2), D = Q.size(3);
  TORCH_CHECK(D == 64 || D == 128, "Head dimension must be 64 or 128");
  TORCH_CHECK(N > 0, "N must be > 0");
  TORCH_CHECK(K.dim() == 4 && V.sizes() == K.sizes() && K.size(0) == B && K.size(2) == N &&
                  K.size(3) == D,
              "K and V must be [B, H_kv, N, D] with H a multiple of H_kv");
  const int64_t Hkv = K.size(1);
  TORCH_CHECK(Hkv > 0 && H % Hkv == 0, "H must be a positive multiple of K/V's head count");
  TORCH_CHECK(K.device() == Q.device() && V.device() == Q.device(),
              "Q/K/V must be on the same device");
  const c10::DeviceGuard guard(Q.device());
  auto q = Q.to(torch::kBFloat16).contiguous();
  auto k = K.to(torch::kBFloat16).contiguous();
  auto v = V.to(torch::kBFloat16).contiguous();
  auto O = torch::empty({B, H, N, D}, q.options());
  torch::Tensor L;
  float* L_ptr = nullptr;
  if (want_L) {
    L = torch::empty({B, H, N}, q.options().dtype(torch::kFloat));
    L_ptr = L.data_ptr<float>();
  }
  const int st = fa_fwd_bf16(q.data_ptr(), k.data_ptr(), v.data_ptr(), O.data_ptr(), L_ptr, B, H,
                             Hkv, N, D, causal ? 1 : 0, current_stream(q));
  check_status(st, "fa_fwd_bf16");
  if (want_L) return {O, L};
  return {O};
}

// forward_varlen(q, k, v, cu_seqlens, max_seqlen, causal=False) -> [O, L]:
// B packed sequences, head-major: q [H, total, D], k/v [H_kv, total, D],
// cu_seqlens int32 [B+1]; O [H, total, D] fp16, L [H, total] fp32. Rows of O
// outside every sequence are left as zeros. No reference counterpart.
std::vector<torch::Tensor> forward_varlen(torch::Tensor q, torch::Tensor k, torch::Tensor v,
                                          torch::Tensor cu_seqlens, int64_t max_seqlen,
                                          bool causal) {
  TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda() && cu_seqlens.is_cuda(),
              "q/k/v/cu_seqlens must be CUDA tensors");
  TORCH_CHECK(q.dim() == 3, "q must be 3D [H, total, D]");
  const int64_t H = q.size(0), total = q.size(1), D = q.size(2);
  TORCH_CHECK(k.dim() == 3 && v.sizes() == k.sizes() && k.size(1) == total && k.size(2) == D,
              "k and v must be [H_kv, total, D] matching q");
  TORCH_CHECK(cu_seqlens.dim() == 1 && cu_seqlens.scalar_type() == torch::kInt &&
                  cu_seqlens.size(0) >= 2,
              "cu_seqlens must be int32 [B + 1]");
  const auto dev = q.device();
  TORCH_CHECK(k.device() == dev && v.device() == dev && cu_seqlens.device() == dev,
              "q/k/v/cu_seqlens must be on the same device");
  const c10::DeviceGuard guard(dev);
  const int64_t B = cu_seqlens.size(0) - 1, Hkv = k.size(0);
  auto qh = q.to(torch::kHalf).contiguous();
  auto kh = k.to(torch::kHalf).contiguous();
  auto vh = v.to(torch::kHalf).contiguous();
  auto cu = cu_seqlens.contiguous();
  // Rows outside every sequence (past cu_seqlens[B]) are not written by the
  // kernel: they keep O = 0 and L = -inf, the logsumexp of no keys.
  auto O = torch::zeros({H, total, D}, qh.options());
  auto L = torch::full({H, total}, -std::numeric_limits<float>::infinity(),
                       qh.options().dtype(torch::kFloat));
  const int st = fa_fwd_varlen_f16(qh.data_ptr(), kh.data_ptr(), vh.data_ptr(), O.data_ptr(),
                                   L.data_ptr<float>(), cu.data_ptr<int32_t>(), B, H, Hkv,
                                   max_seqlen, total, D, causal ? 1 : 0, current_stream(qh));
  check_status(st, "fa_fwd_varlen_f16");
  return {O, L};
}

// backward(Q, K, V, O, dO, L) -> [dQ, dK, dV] float32 [B,H,N,D], the module
// function of cuda/flash_attn_kernel.cu:417-503 (checks :425-432). Q/K/V/O/dO
// are cast to fp16 (O from forward() already is), L to fp32; the D_i
// workspace comes from the caching allocator.
static std::vector<torch::Tensor> backward_impl(torch::Tensor Q, torch::Tensor K,
                                                torch::Tensor V, torch::Tensor O,
                                                torch::Tensor dO, torch::Tensor L, bool causal,
                                                bool bf16) {
  TORCH_CHECK(Q.is_cuda(), "Q must be a CUDA tensor");
  TORCH_CHECK(dO.is_cuda(), "dO must be a CUDA tensor");
  TORCH_CHECK(K.is_cuda() && V.is_cuda() && O.is_cuda() && L.is_cuda(),
              "K/V/O/L must be CUDA tensors");
  TORCH_CHECK(Q.dim() == 4, "Q must be 4D [B, H, N, D]");
  const int64_t B = Q.size(0), H = Q.size(1), N = Q.size(2), D = Q.size(3);
  TORCH_CHECK(D == 64 || D == 128, "Head dimension must be 64 or 128");
  TORCH_CHECK(N > 0, "N must be > 0");
  TORCH_CHECK(O.sizes() == Q.sizes() && dO.sizes() == Q.sizes(),
              "O and dO must have the same shape as Q");
  TORCH_CHECK(K.dim() == 4 && V.sizes() == K.sizes() && K.size(0) == B && K.size(2) == N &&
                  K.size(3) == D,
              "K and V must have the same shape as Q, or [B, H_kv, N, D] with H a multiple of H_kv");
  const int64_t Hkv = K.size(1);
  TORCH_CHECK(Hkv > 0 && H % Hkv == 0, "H must be a positive multiple of K/V's head count");
  TORCH_CHECK(L.numel() == B * H * N, "L must hold B*H*N logsumexp values");
  const auto dev = Q.device();
  TORCH_CHECK(K.device() == dev && V.device() == dev && O.device() == dev && dO.device() == dev &&
                  L.device() == dev,
              "Q/K/V/O/dO/L must be on the same device");

  const c10::DeviceGuard guard(dev);
  const int64_t BH = B * H;
  const auto in_type = bf16 ? torch::kBFloat16 : torch::kHalf;
  auto half = [&](const torch::Tensor& t) { return t.to(in_type).contiguous(); };
  auto Qh = half(Q), Kh = half(K), Vh = half(V), Oh = half(O), dOh = half(dO);
  auto Lf = L.to(torch::kFloat).reshape({BH, N}).contiguous();
  auto f32 = Qh.options().dtype(torch::kFloat);
  auto dQ = torch::empty({B, H, N, D}, f32);
  auto dK = torch::empty({B, Hkv, N, D}, f32);
  auto dV = torch::empty({B, Hkv, N, D}, f32);
  auto ws = torch::empty({fa_bwd_gqa_workspace_floats(B, H, Hkv, N, D)}, f32);
  auto entry = bf16 ? fa_bwd_bf16 : fa_bwd_gqa_f16;
  const int st = entry(Qh.data_ptr(), Kh.data_ptr(), Vh.data_ptr(), Oh.data_ptr(), dOh.data_ptr(),
                       Lf.data_ptr<float>(), dQ.data_ptr<float>(), dK.data_ptr<float>(),
                       dV.data_ptr<float>(), ws.data_ptr<float>(), B, H, Hkv, N, D,
                       causal ? 1 : 0, current_stream(Qh));
  check_status(st, bf16 ? "fa_bwd_bf16" : "fa_bwd_gqa_f16");
  return {dQ, dK, dV};
}

std::vector<torch::Tensor> backward(torch::Tensor Q, torch::Tensor K, torch::Tensor V,
                                    torch::Tensor O, torch::Tensor dO, torch::Tensor L,
                                    bool causal) {
  return backward_impl(Q, K, V, O, dO, L, causal, /*bf16=*/false);
}

// backward_bf16(Q, K, V, O, dO, L, causal=False) -> [dQ, dK, dV] float32: the
// backward of forward_bf16 (inputs cast to bf16). No reference counterpart.
std::vector<torch::Tensor> backward_bf16(torch::Tensor Q, torch::Tensor K, torch::Tensor V,
                                         torch::Tensor O, torch::Tensor dO, torch::Tensor L,
                                         bool causal) {
  return backward_impl(Q, K, V, O, dO, L, causal, /*bf16=*/true);
}

// backward_varlen(q, k, v, o, dO, L, cu_seqlens, max_seqlen, causal=False) ->
// [dQ, dK, dV] float32: the backward of forward_varlen (head-major packed
// sequences, dQ [H, total, D], dK/dV [H_kv, total, D]). Rows outside every
// sequence are zeros. No reference counterpart.
std::vector<torch::Tensor> backward_varlen(torch::Tensor q, torch::Tensor k, torch::Tensor v,
                                           torch::Tensor o, torch::Tensor dO, torch::Tensor L,
                                           torch::Tensor cu_seqlens, int64_t max_seqlen,
                                           bool causal) {
  TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda() && o.is_cuda() && dO.is_cuda() &&
                  L.is_cuda() && cu_seqlens.is_cuda(),
              "q/k/v/o/dO/L/cu_seqlens must be CUDA tensors");
  TORCH_CHECK(q.dim() == 3, "q must be 3D [H, total, D]");
  const int64_t H = q.size(0), total = q.size(1), D = q.size(2);
  TORCH_CHECK(D == 64 || D == 128, "Head dimension must be 64 or 128");
  TORCH_CHECK(k.dim() == 3 && v.sizes() == k.sizes() && k.size(1) == total && k.size(2) == D,
              "k and v must be [H_kv, total, D] matching q");
  TORCH_CHECK(o.sizes() == q.sizes() && dO.sizes() == q.sizes(),
              "o and dO must have the same shape as q");
  TORCH_CHECK(L.numel() == H * total, "L must hold H*total logsumexp values");
  TORCH_CHECK(cu_seqlens.dim() == 1 && cu_seqlens.scalar_type() == torch::kInt &&
                  cu_seqlens.size(0) >= 2,
              "cu_seqlens must be int32 [B + 1]");
  const auto dev = q.device();
  TORCH_CHECK(k.device() == dev && v.device() == dev && o.device() == dev &&
                  dO.device() == dev && L.device() == dev && cu_seqlens.device() == dev,
              "all tensors must be on the same device");
  const c10::DeviceGuard guard(dev);
  const int64_t B = cu_seqlens.size(0) - 1, Hkv = k.size(0);
  TORCH_CHECK(Hkv > 0 && H % Hkv == 0, "H must be a positive multiple of k/v's head count");
  auto half = [&](const torch::Tensor& t) { return t.to(torch::kHalf).contiguous(); };
  auto qh = half(q), kh = half(k), vh = half(v), oh = half(o), gh = half(dO);
  auto Lf = L.to(torch::kFloat).reshape({H, total}).contiguous();
  auto cu = cu_seqlens.contiguous();
  auto f32 = qh.options().dtype(torch::kFloat);
  auto dQ = torch::zeros({H, total, D}, f32);
  auto dK = torch::zeros({Hkv, total, D}, f32);
  auto dV = torch::zeros({Hkv, total, D}, f32);
  const int64_t wsn = fa_bwd_gqa_workspace_floats(1, H, Hkv, total > 0 ? total : 1, D);
  // zeros: with H_kv < H the group sums also read the partials of rows
  // outside every sequence
  auto ws = torch::zeros({wsn}, f32);
  const int st = fa_bwd_varlen_f16(qh.data_ptr(), kh.data_ptr(), vh.data_ptr(), oh.data_ptr(),
                                   gh.data_ptr(), Lf.data_ptr<float>(), dQ.data_ptr<float>(),
                                   dK.data_ptr<float>(), dV.data_ptr<float>(),
                                   ws.data_ptr<float>(), cu.data_ptr<int32_t>(), B, H, Hkv,
                                   max_seqlen, total, D, causal ? 1 : 0, current_stream(qh));
  check_status(st, "fa_bwd_varlen_f16");
  return {dQ, dK, dV};
}

// Test support: the forward through one explicit kernel variant.
std::vector<torch::Tensor> probe_fwd_variant(torch::Tensor Q, torch::Tensor K, torch::Tensor V,
                                             bool causal, int64_t variant, bool want_L) {
  TORCH_CHECK(variant > 0, "variant must be > 0 (1000 + v: v's guarded instance)");
  auto r = forward_impl(Q, K, V, want_L, causal, (int)variant);
  if (want_L) return {r.first, r.second};
  return {r.first};
}

// Test support: the forward split over the keys into an explicit number of
// ranges (1 = the unsplit default kernel).
std::vector<torch::Tensor> probe_fwd_splitkv(torch::Tensor Q, torch::Tensor K, torch::Tensor V,
                                             bool causal, int64_t splits, bool want_L) {
  TORCH_CHECK(splits >= 1 && splits <= 16, "splits must be in [1, 16]");
  const int def = fa_probe_default_variant(Q.size(3));
  auto r = splits == 1 ? forward_impl(Q, K, V, want_L, causal, def)
                       : forward_impl(Q, K, V, want_L, causal, 0, splits);
  if (want_L) return {r.first, r.second};
  return {r.first};
}

std::vector<int64_t> probe_fwd_variants(int64_t D, bool causal) {
  int buf[64];
  const int n = fa_probe_fwd_variants(buf, 64, D, causal ? 1 : 0);
  return std::vector<int64_t>(buf, buf + (n < 64 ? n : 64));
}

struct DecodeArgs {
  int64_t B, H, Hkv, D, page_size, max_pages, num_pages;
};

DecodeArgs check_decode(const torch::Tensor& q, const torch::Tensor& k_pool,
                        const torch::Tensor& v_pool, const torch::Tensor& page_table,
                        const torch::Tensor& ctx_lens) {
  TORCH_CHECK(q.is_cuda() && k_pool.is_cuda() && v_pool.is_cuda() && page_table.is_cuda() &&
                  ctx_lens.is_cuda(),
              "q/k_pool/v_pool/page_table/ctx_lens must be CUDA tensors");
  TORCH_CHECK(q.dim() == 3, "q must be 3D [B, H, D]");
  TORCH_CHECK(k_pool.dim() == 4, "k_pool must be 4D [num_pages, H, page_size, D]");
  TORCH_CHECK(v_pool.sizes() == k_pool.sizes(), "v_pool must have the same shape as k_pool");
  TORCH_CHECK((q.scalar_type() == torch::kHalf || q.scalar_type() == torch::kBFloat16) &&
                  k_pool.scalar_type() == q.scalar_type() &&
                  v_pool.scalar_type() == q.scalar_type(),
              "q/k_pool/v_pool must be all float16 or all bfloat16");
  TORCH_CHECK(page_table.dim() == 2 && page_table.scalar_type() == torch::kInt,
              "page_table must be int32 [B, max_pages]");
  TORCH_CHECK(ctx_lens.dim() == 1 && ctx_lens.scalar_type() == torch::kInt,
              "ctx_lens must be int32 [B]");
  TORCH_CHECK(q.is_contiguous() && k_pool.is_contiguous() && v_pool.is_contiguous() &&
                  page_table.is_contiguous() && ctx_lens.is_contiguous(),
              "decode tensors must be contiguous");
  DecodeArgs a;
  a.B = q.size(0);
  a.H = q.size(1);
  a.D = q.size(2);
  a.num_pages = k_pool.size(0);
  a.Hkv = k_pool.size(1);
  a.page_size = k_pool.size(2);
  a.max_pages = page_table.size(1);
  TORCH_CHECK(k_pool.size(1) > 0 && a.H % k_pool.size(1) == 0 && k_pool.size(3) == a.D,
              "k_pool must be [num_pages, H_kv, page_size, D] with q's D and H a multiple of H_kv");
  TORCH_CHECK(page_table.size(0) == a.B && ctx_lens.size(0) == a.B,
              "page_table and ctx_lens must have q's batch size");
  auto dev = q.device();
  TORCH_CHECK(k_pool.device() == dev && v_pool.device() == dev && page_table.device() == dev &&
                  ctx_lens.device() == dev,
              "decode tensors must be on the same device");
  return a;
}

std::vector<torch::Tensor> decode_partials(torch::Tensor q, torch::Tensor k_pool,
                                           torch::Tensor v_pool, torch::Tensor page_table,
                                           torch::Tensor ctx_lens, int64_t num_splits) {
  const DecodeArgs a = check_decode(q, k_pool, v_pool, page_table, ctx_lens);
  TORCH_CHECK(a.Hkv == a.H, "decode_partials takes pools with H heads (use decode_paged for GQA)");
  TORCH_CHECK(q.scalar_type() == torch::kHalf,
              "decode_partials takes float16 (use decode_paged for bfloat16)");
  const c10::DeviceGuard guard(q.device());
  auto part_o = torch::empty({a.B, a.H, num_splits, a.D}, q.options().dtype(torch::kFloat));
  auto part_lse = torch::empty({a.B, a.H, num_splits}, q.options().dtype(torch::kFloat));
  const int st = fa_decode_split_f16(q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
                                     page_table.data_ptr<int32_t>(), ctx_lens.data_ptr<int32_t>(),
                                     a.B, a.H, a.D, a.page_size, a.max_pages, a.num_pages,
                                     num_splits, part_o.data_ptr<float>(),
                                     part_lse.data_ptr<float>(), current_stream(q));
  check_status(st, "fa_decode_split_f16");
  return {part_o, part_lse};
}

std::vector<torch::Tensor> lse_combine(torch::Tensor part_o, torch::Tensor part_lse) {
  TORCH_CHECK(part_o.is_cuda() && part_lse.is_cuda(), "part_o/part_lse must be CUDA tensors");
  TORCH_CHECK(part_o.dim() == 4 && part_o.scalar_type() == torch::kFloat && part_o.is_contiguous(),
              "part_o must be contiguous float32 [B, H, num_splits, D]");
  TORCH_CHECK(part_lse.dim() == 3 && part_lse.scalar_type() == torch::kFloat &&
                  part_lse.is_contiguous(),
              "part_lse must be contiguous float32 [B, H, num_splits]");
  const int64_t B = part_o.size(0), H = part_o.size(1), S = part_o.size(2), D = part_o.size(3);
  TORCH_CHECK(part_lse.size(0) == B && part_lse.size(1) == H && part_lse.size(2) == S,
              "part_lse must be [B, H, num_splits] matching part_o");
  const c10::DeviceGuard guard(part_o.device());
  auto o = torch::empty({B, H, D}, part_o.options().dtype(torch::kHalf));
  auto lse = torch::empty({B, H}, part_o.options());
  const int st = fa_lse_combine_f32(part_o.data_ptr<float>(), part_lse.data_ptr<float>(), B, H, D,
                                    S, o.data_ptr(), lse.data_ptr<float>(), current_stream(part_o));
  check_status(st, "fa_lse_combine_f32");
  return {o, lse};
}

std::vector<torch::Tensor> decode_paged(torch::Tensor q, torch::Tensor k_pool, torch::Tensor v_pool,
                                        torch::Tensor page_table, torch::Tensor ctx_lens,
                                        int64_t num_splits) {
  const DecodeArgs a = check_decode(q, k_pool, v_pool, page_table, ctx_lens);
  const c10::DeviceGuard guard(q.device());
  auto ws = torch::empty({fa_decode_workspace_floats(a.B, a.H, a.D, num_splits)},
                         q.options().dtype(torch::kFloat));
  float* part_o = ws.data_ptr<float>();
  float* part_lse = part_o + a.B * a.H * num_splits * a.D;
  auto o = torch::empty({a.B, a.H, a.D}, q.options());
  auto lse = torch::empty({a.B, a.H}, q.options().dtype(torch::kFloat));
  // O takes q's element type (fp16 or bf16).
  const bool bf16 = q.scalar_type() == torch::kBFloat16;
  const auto fn = bf16 ? fa_decode_paged_bf16 : fa_decode_paged_gqa_f16;
  const int st = fn(q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
                    page_table.data_ptr<int32_t>(), ctx_lens.data_ptr<int32_t>(), a.B, a.H, a.Hkv,
                    a.D, a.page_size, a.max_pages, a.num_pages, num_splits, part_o, part_lse,
                    o.data_ptr(), lse.data_ptr<float>(), current_stream(q));
  check_status(st, bf16 ? "fa_decode_paged_bf16" : "fa_decode_paged_gqa_f16");
  return {o, lse};
}

// kv_append(k_new, v_new, k_pool, v_pool, page_table, start_pos, new_lens=None)
// writes new rows into the pools in place and returns bad int32 [B] (1 where
// a token of the sequence had no valid page). No reference counterpart.
torch::Tensor kv_append(torch::Tensor k_new, torch::Tensor v_new, torch::Tensor k_pool,
                        torch::Tensor v_pool, torch::Tensor page_table, torch::Tensor start_pos,
                        c10::optional<torch::Tensor> new_lens) {
  TORCH_CHECK(k_new.is_cuda() && v_new.is_cuda() && k_pool.is_cuda() && v_pool.is_cuda() &&
                  page_table.is_cuda() && start_pos.is_cuda(),
              "k_new/v_new/k_pool/v_pool/page_table/start_pos must be CUDA tensors");
  TORCH_CHECK(k_new.dim() == 4 && v_new.sizes() == k_new.sizes(),
              "k_new and v_new must be [B, H, T, D] of the same shape");
  TORCH_CHECK(k_pool.dim() == 4 && v_pool.sizes() == k_pool.sizes(),
              "k_pool and v_pool must be [num_pages, H, page_size, D] of the same shape");
  TORCH_CHECK((k_new.scalar_type() == torch::kHalf || k_new.scalar_type() == torch::kBFloat16) &&
                  v_new.scalar_type() == k_new.scalar_type() &&
                  k_pool.scalar_type() == k_new.scalar_type() &&
                  v_pool.scalar_type() == k_new.scalar_type(),
              "k_new/v_new/k_pool/v_pool must be all float16 or all bfloat16");
  const int64_t B = k_new.size(0), H = k_new.size(1), T = k_new.size(2), D = k_new.size(3);
  TORCH_CHECK(k_pool.size(1) == H && k_pool.size(3) == D,
              "k_pool must be [num_pages, H, page_size, D] with k_new's H and D");
  TORCH_CHECK(page_table.dim() == 2 && page_table.scalar_type() == torch::kInt &&
                  page_table.size(0) == B,
              "page_table must be int32 [B, max_pages]");
  TORCH_CHECK(start_pos.dim() == 1 && start_pos.scalar_type() == torch::kInt &&
                  start_pos.size(0) == B,
              "start_pos must be int32 [B]");
  const int32_t* lens = nullptr;
  torch::Tensor nl;
  if (new_lens.has_value()) {
    nl = new_lens.value();
    TORCH_CHECK(nl.is_cuda() && nl.dim() == 1 && nl.scalar_type() == torch::kInt &&
                    nl.size(0) == B && nl.is_contiguous(),
                "new_lens must be a contiguous CUDA int32 [B]");
    lens = nl.data_ptr<int32_t>();
  }
  TORCH_CHECK(k_new.is_contiguous() && v_new.is_contiguous() && k_pool.is_contiguous() &&
                  v_pool.is_contiguous() && page_table.is_contiguous() && start_pos.is_contiguous(),
              "kv_append tensors must be contiguous");
  const auto dev = k_new.device();
  TORCH_CHECK(v_new.device() == dev && k_pool.device() == dev && v_pool.device() == dev &&
                  page_table.device() == dev && start_pos.device() == dev &&
                  (!nl.defined() || nl.device() == dev),
              "kv_append tensors must be on the same device");
  const c10::DeviceGuard guard(dev);
  auto bad = torch::zeros({B}, page_table.options());
  const bool bf16 = k_new.scalar_type() == torch::kBFloat16;
  const auto fn = bf16 ? fa_kv_append_bf16 : fa_kv_append_f16;
  const int st = fn(k_new.data_ptr(), v_new.data_ptr(), page_table.data_ptr<int32_t>(),
                    start_pos.data_ptr<int32_t>(), lens, k_pool.data_ptr(), v_pool.data_ptr(),
                    bad.data_ptr<int32_t>(), B, H, T, D, k_pool.size(2), page_table.size(1),
                    k_pool.size(0), current_stream(k_new));
  check_status(st, bf16 ? "fa_kv_append_bf16" : "fa_kv_append_f16");
  return bad;
}

// ---- layout probes (test support) ----
torch::Tensor probe_mfma32(torch::Tensor a, torch::Tensor b, int64_t variant) {
  TORCH_CHECK(a.is_cuda() && a.sizes() == torch::IntArrayRef({32, 16}) && a.scalar_type() == torch::kHalf);
  TORCH_CHECK(b.is_cuda() && b.sizes() == torch::IntArrayRef({16, 32}) && b.scalar_type() == torch::kHalf);
  auto ac = a.contiguous(), bc = b.contiguous();
  auto c = torch::empty({32, 32}, a.options().dtype(torch::kFloat));
  check_status(fa_probe_mfma32(ac.data_ptr(), bc.data_ptr(), c.data_ptr<float>(), (int)variant,
                               current_stream(a)), "fa_probe_mfma32");
  return c;
}

torch::Tensor probe_mfma16(torch::Tensor a, torch::Tensor b, int64_t variant) {
  TORCH_CHECK(a.is_cuda() && a.sizes() == torch::IntArrayRef({16, 32}) && a.scalar_type() == torch::kHalf);
  TORCH_CHECK(b.is_cuda() && b.sizes() == torch::IntArrayRef({32, 16}) && b.scalar_type() == torch::kHalf);
  auto ac = a.contiguous(), bc = b.contiguous();
  auto c = torch::empty({16, 16}, a.options().dtype(torch::kFloat));
  check_status(fa_probe_mfma16(ac.data_ptr(), bc.data_ptr(), c.data_ptr<float>(), (int)variant,
                               current_stream(a)), "fa_probe_mfma16");
  return c;
}

torch::Tensor probe_tr16_raw(torch::Tensor in) {
  TORCH_CHECK(in.is_cuda() && in.numel() == 256 && in.element_size() == 2);
  auto ic = in.contiguous();
  auto out = torch::empty({64, 4}, in.options());
  check_status(fa_probe_tr16_raw(ic.data_ptr(), out.data_ptr(), current_stream(in)),
               "fa_probe_tr16_raw");
  return out;
}

torch::Tensor probe_permlane(torch::Tensor in) {
  TORCH_CHECK(in.is_cuda() && in.numel() == 64 && in.scalar_type() == torch::kFloat);
  auto ic = in.contiguous();
  auto out = torch::empty({4, 64}, in.options());
  check_status(fa_probe_permlane(ic.data_ptr<float>(), out.data_ptr<float>(), current_stream(in)),
               "fa_probe_permlane");
  return out;
}

std::vector<torch::Tensor> probe_frags(torch::Tensor tile) {
  TORCH_CHECK(tile.is_cuda() && tile.dim() == 2 && tile.size(0) == 64 &&
              (tile.size(1) == 64 || tile.size(1) == 128) && tile.scalar_type() == torch::kHalf);
  const int64_t D = tile.size(1);
  auto tc = tile.contiguous();
  auto kout = torch::empty({2, D / 16, 64, 8}, tile.options());
  auto vout = torch::empty({4, D / 32, 64, 8}, tile.options());
  check_status(fa_probe_frags(tc.data_ptr(), kout.data_ptr(), vout.data_ptr(), D, current_stream(tile)),
               "fa_probe_frags");
  return {kout, vout};
}

// One streaming read of x (any dtype, contiguous, 16-byte multiple) into the
// one-word sink (int32, CUDA): the read-bandwidth probe.
void probe_read_bw(torch::Tensor x, torch::Tensor sink, int64_t blocks) {
  TORCH_CHECK(x.is_cuda() && x.is_contiguous(), "x must be a contiguous CUDA tensor");
  TORCH_CHECK(sink.is_cuda() && sink.scalar_type() == torch::kInt && sink.numel() >= 1,
              "sink must be a CUDA int32 tensor");
  const int64_t bytes = x.numel() * (int64_t)x.element_size();
  check_status(fa_probe_read_bw(x.data_ptr(), bytes, (int)blocks,
                                reinterpret_cast<uint32_t*>(sink.data_ptr<int>()), current_stream(x)),
               "fa_probe_read_bw");
}

// One gather read of the 4 KiB pages of k and v (contiguous CUDA tensors of
// equal size, a multiple of 4 KiB) in the order of table (int32, CUDA): the
// paged decode's read pattern without its arithmetic.
void probe_gather_bw(torch::Tensor k, torch::Tensor v, torch::Tensor table, torch::Tensor sink,
                     int64_t pages_per_wg, bool nontemporal) {
  TORCH_CHECK(k.is_cuda() && v.is_cuda() && k.is_contiguous() && v.is_contiguous(),
              "k and v must be contiguous CUDA tensors");
  const int64_t bytes = k.numel() * (int64_t)k.element_size();
  TORCH_CHECK(bytes == v.numel() * (int64_t)v.element_size() && bytes % 4096 == 0,
              "k and v must hold the same whole number of 4 KiB pages");
  TORCH_CHECK(table.is_cuda() && table.scalar_type() == torch::kInt && table.is_contiguous() &&
                  table.numel() == bytes / 4096,
              "table must be a contiguous CUDA int32 tensor of one entry per page");
  TORCH_CHECK(sink.is_cuda() && sink.scalar_type() == torch::kInt && sink.numel() >= 1,
              "sink must be a CUDA int32 tensor");
  check_status(fa_probe_gather_bw(k.data_ptr(), v.data_ptr(), table.data_ptr<int>(), bytes / 4096,
                                  (int)pages_per_wg, nontemporal ? 1 : 0,
                                  reinterpret_cast<uint32_t*>(sink.data_ptr<int>()),
                                  current_stream(k)),
               "fa_probe_gather_bw");
}

torch::Tensor probe_chain(torch::Tensor q, torch::Tensor k, torch::Tensor v) {
  TORCH_CHECK(q.is_cuda() && q.dim() == 2 && q.size(0) == 32 && q.scalar_type() == torch::kHalf);
  const int64_t D = q.size(1);
  TORCH_CHECK(D == 64 || D == 128);
  TORCH_CHECK(k.sizes() == torch::IntArrayRef({64, D}) && v.sizes() == torch::IntArrayRef({64, D}));
  auto qc = q.contiguous(), kc = k.contiguous(), vc = v.contiguous();
  auto o = torch::empty({32, D}, q.options().dtype(torch::kFloat));
  check_status(fa_probe_chain(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr<float>(), D,
                              current_stream(q)), "fa_probe_chain");
  return o;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("forward", &forward, "FlashAttention forward: returns [O half, L float]",
        py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("causal") = false);
  m.def("forward_only", &forward_only, "FlashAttention forward, O only",
        py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("causal") = false);
  m.def("forward_bf16", &forward_bf16, "bfloat16 forward: returns [O bf16, L float] ([O] if not want_L)",
        py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("causal") = false,
        py::arg("want_L") = true);
  m.def("forward_varlen", &forward_varlen,
        "packed variable-length forward (head-major): returns [O half, L float]", py::arg("q"),
        py::arg("k"), py::arg("v"), py::arg("cu_seqlens"), py::arg("max_seqlen"),
        py::arg("causal") = false);
  m.def("backward", &backward, "FlashAttention backward: returns [dQ, dK, dV] float",
        py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("O"), py::arg("dO"), py::arg("L"),
        py::arg("causal") = false);
  m.def("backward_bf16", &backward_bf16, "bfloat16 backward: returns [dQ, dK, dV] float",
        py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("O"), py::arg("dO"), py::arg("L"),
        py::arg("causal") = false);
  m.def("backward_varlen", &backward_varlen,
        "varlen backward: returns [dQ, dK, dV] float (head-major packed)", py::arg("q"),
        py::arg("k"), py::arg("v"), py::arg("o"), py::arg("dO"), py::arg("L"),
        py::arg("cu_seqlens"), py::arg("max_seqlen"), py::arg("causal") = false);
  m.def("kv_append", &kv_append, "write new K/V rows into the paged pools; returns bad [B]",
        py::arg("k_new"), py::arg("v_new"), py::arg("k_pool"), py::arg("v_pool"),
        py::arg("page_table"), py::arg("start_pos"), py::arg("new_lens") = py::none());
  m.def("decode_paged", &decode_paged, "split-KV paged decode (fp16 or bf16): returns [O in q's dtype, L float]",
        py::arg("q"), py::arg("k_pool"), py::arg("v_pool"), py::arg("page_table"),
        py::arg("ctx_lens"), py::arg("num_splits") = 16);
  m.def("decode_partials", &decode_partials, "split pass only: returns [part_o, part_lse]",
        py::arg("q"), py::arg("k_pool"), py::arg("v_pool"), py::arg("page_table"),
        py::arg("ctx_lens"), py::arg("num_splits") = 16);
  m.def("lse_combine", &lse_combine, "combine pass: returns [O half, L float]",
        py::arg("part_o"), py::arg("part_lse"));
  m.def("probe_mfma32", &probe_mfma32);
  m.def("probe_mfma16", &probe_mfma16);
  m.def("probe_tr16_raw", &probe_tr16_raw);
  m.def("probe_permlane", &probe_permlane);
  m.def("probe_frags", &probe_frags);
  m.def("probe_chain", &probe_chain);
  m.def("probe_read_bw", &probe_read_bw, py::arg("x"), py::arg("sink"), py::arg("blocks"));
  m.def("probe_gather_bw", &probe_gather_bw, py::arg("k"), py::arg("v"), py::arg("table"),
        py::arg("sink"), py::arg("pages_per_wg"), py::arg("nontemporal"));
  m.def("probe_fwd_variant", &probe_fwd_variant, py::arg("Q"), py::arg("K"), py::arg("V"),
        py::arg("causal") = false, py::arg("variant") = 12, py::arg("want_L") = true);
  m.def("probe_fwd_variants", &probe_fwd_variants);
  m.def("probe_fwd_splitkv", &probe_fwd_splitkv,
            "forward split over the keys into `splits` ranges ([O, L] or [O])", py::arg("Q"),
            py::arg("K"), py::arg("V"), py::arg("causal"), py::arg("splits"), py::arg("want_L"));
  m.def("probe_fwd_splitkv_plan", &fa_fwd_splitkv_plan, "split count the forward uses",
            py::arg("B"), py::arg("H"), py::arg("N"), py::arg("D"), py::arg("causal"));
  m.def("probe_default_variant", [](int64_t D) { return fa_probe_default_variant(D); });
  m.def("abi_version", &fa_abi_version);
}
