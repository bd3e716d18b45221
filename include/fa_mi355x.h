/*
 * fa_mi355x.h — C ABI of the MI355X (gfx950) FlashAttention forward and
 * backward, the split-KV paged decode and the KV-cache page writer.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * passed as void*. The library never allocates, never synchronises the host
 * and keeps no mutable global state: it is re-entrant and stream-ordered.
 * Buffers (including the decode split workspace) belong to the caller.
 *
 * Status codes: 0 = ok, > 0 = invalid argument (fa_status_str names it),
 * < 0 = a HIP error, negated (-(int)hipError_t).
 *
 * Tensor layouts (all contiguous, row-major):
 *   q, k, v, o : fp16 [B, H, N, D]        (bh = b*H + h; row stride D)
 *   lse        : fp32 [B, H, N]           natural-log logsumexp of the scaled
 *                                         logits S = q k^T / sqrt(D)
 *   k_pool,    : fp16 [num_pages, H, page_size, D]   head-major pages
 *   v_pool
 *   page_table : int32 [B, max_pages]     page ids of each sequence, in order
 *   ctx_lens   : int32 [B]                tokens per sequence
 *   part_o     : fp32 [B, H, num_splits, D]   normalised split partials
 *   part_lse   : fp32 [B, H, num_splits]      split logsumexp (-inf if empty)
 */
#ifndef FA_MI355X_H
#define FA_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 1

enum fa_status_code {
  FA_OK = 0,
  FA_ERR_NULL_POINTER = 1,   /* a required pointer is NULL */
  FA_ERR_HEAD_DIM = 2,       /* D is not 64 or 128 */
  FA_ERR_SEQ_LEN = 3,        /* N <= 0 */
  FA_ERR_BATCH_HEADS = 4,    /* B <= 0 or H <= 0 */
  FA_ERR_ALIGNMENT = 5,      /* a tensor pointer is not 16-byte aligned */
  FA_ERR_TOO_LARGE = 6,      /* a size exceeds the kernels' index range */
  FA_ERR_PAGE_SIZE = 7,      /* page_size is not 16 */
  FA_ERR_NUM_SPLITS = 8,     /* num_splits outside [1, 16] */
  FA_ERR_MAX_PAGES = 9,      /* max_pages <= 0 */
  FA_ERR_NUM_PAGES = 10,     /* num_pages <= 0 */
  FA_ERR_KV_HEADS = 11,      /* H_kv <= 0 or H not a multiple of H_kv */
  FA_ERR_SCRATCH_SIZE = 12   /* split partials exceed FA_DECODE_SCRATCH_FLOATS */
};

/* Floats of the library's own split-partials array used by
 * fa_decode_paged_noalloc_f16 (16 MiB per GPU). */
#define FA_DECODE_SCRATCH_FLOATS (((int64_t)1) << 22)

/* Human-readable name of a status code (static storage). */
const char* fa_status_str(int status);

/* FA_ABI_VERSION of the built library. */
int fa_abi_version(void);

/*
 * Host-only argument check of fa_fwd_f16 (no HIP call; runs without a GPU).
 * Replaces the argument checks of the reference launcher
 * fa3db_full_forward_impl (cuda/flash_attn_fa3_db_full.cu:352-363), widened to
 * D in {64, 128}.
 */
int fa_validate_fwd(const void* q, const void* k, const void* v, const void* o,
                    int64_t B, int64_t H, int64_t N, int64_t D);

/*
 * Attention forward: o = softmax(q k^T / sqrt(D) [+ causal mask]) v, and, if
 * lse != NULL, the per-row logsumexp. lse == NULL is the O-only variant; its o
 * is bitwise equal to the o written with lse != NULL.
 * causal != 0: query i sees keys j <= i.
 * Replaces fa3db_full_forward_impl (cuda/flash_attn_fa3_db_full.cu:349-403):
 * want_L=true <-> lse != NULL (:405-408), want_L=false <-> lse == NULL
 * (:410-413). The causal flag and D=128 have no reference counterpart.
 */
int fa_fwd_f16(const void* q, const void* k, const void* v, void* o, float* lse,
               int64_t B, int64_t H, int64_t N, int64_t D, int causal,
               void* stream);

/*
 * Host-only argument check of fa_fwd_gqa_f16: fa_validate_fwd plus
 * H_kv > 0 and H % H_kv == 0. No reference counterpart (README.md:326 lists
 * GQA/MQA as not covered).
 */
int fa_validate_fwd_gqa(const void* q, const void* k, const void* v, const void* o,
                        int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D);

/*
 * Grouped-query / multi-query forward: q, o fp16 [B, H, N, D]; k, v fp16
 * [B, H_kv, N, D]; query head h attends with key/value head h / (H / H_kv).
 * H_kv == H is fa_fwd_f16; H_kv == 1 is MQA. lse, causal and the O-only
 * contract are those of fa_fwd_f16. No reference counterpart.
 */
int fa_fwd_gqa_f16(const void* q, const void* k, const void* v, void* o, float* lse,
                   int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D, int causal,
                   void* stream);

/*
 * bfloat16 forward: q, o bf16 [B, H, N, D]; k, v bf16 [B, H_kv, N, D]
 * (H_kv == H for plain multi-head); fp32 accumulation and softmax, P rounded
 * to bf16 for the PV product; lse fp32 [B, H, N] or NULL (O-only, bitwise the
 * same o). Same argument checks as fa_fwd_gqa_f16. No reference counterpart
 * (the reference is fp16-only).
 */
int fa_fwd_bf16(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B,
                int64_t H, int64_t H_kv, int64_t N, int64_t D, int causal, void* stream);

/*
 * Host-only argument check of fa_fwd_varlen_f16: pointers (cu_seqlens
 * 4-byte aligned), D, B/H/H_kv, max_seqlen > 0, total >= 0, index ranges.
 */
int fa_validate_fwd_varlen(const void* q, const void* k, const void* v, const void* o,
                           const int32_t* cu_seqlens, int64_t B, int64_t H, int64_t H_kv,
                           int64_t max_seqlen, int64_t total, int64_t D);

/*
 * Variable-length forward over B packed sequences, head-major: q, o fp16
 * [H, total, D]; k, v fp16 [H_kv, total, D]; lse fp32 [H, total] (or NULL).
 * Sequence b is rows cu_seqlens[b] .. cu_seqlens[b+1] of every head
 * (cu_seqlens int32 [B+1], nondecreasing, cu_seqlens[B] <= total) and attends
 * only within itself (causal: row i of a sequence sees its keys j <= i).
 * max_seqlen sizes the grid and must be >= every sequence length: rows past
 * it are not computed. Bounds read from cu_seqlens are clamped into
 * [0, total], so a malformed table cannot move any access outside the
 * buffers. Rows of o and lse that belong to no sequence (rows before
 * cu_seqlens[0] or from cu_seqlens[B] on) are never written: a caller that
 * needs them defined sets O = 0 and L = -inf there itself (the torch binding
 * does). No reference counterpart (README.md:326 lists varlen as not
 * covered).
 */
int fa_fwd_varlen_f16(const void* q, const void* k, const void* v, void* o, float* lse,
                      const int32_t* cu_seqlens, int64_t B, int64_t H, int64_t H_kv,
                      int64_t max_seqlen, int64_t total, int64_t D, int causal, void* stream);

/*
 * Host-only argument check of fa_bwd_f16. Replaces the checks of the reference
 * backward launcher flash_attn_backward (cuda/flash_attn_kernel.cu:425-432),
 * widened to D in {64, 128}.
 */
int fa_validate_bwd(const void* q, const void* k, const void* v, const void* o,
                    const void* dout, const float* lse, const float* dq, const float* dk,
                    const float* dv, const float* workspace, int64_t B, int64_t H,
                    int64_t N, int64_t D);

/* Floats of the workspace fa_bwd_f16 needs: 2*B*H*N (the negated row sums -D_i, then -lse*log2(e)). */
int64_t fa_bwd_workspace_floats(int64_t B, int64_t H, int64_t N);

/*
 * Attention backward from the forward's outputs: given q, k, v, o (fp16
 * [B,H,N,D]), dout = dL/do (fp16 [B,H,N,D]) and lse (fp32 [B,H,N], the
 * forward's natural-log logsumexp), writes fp32 [B,H,N,D] gradients
 *   dq = dS k / sqrt(D),  dk = dS^T q / sqrt(D),  dv = P^T dout,
 * with P = exp(q k^T / sqrt(D) - lse) [causal-masked], dS = P * (dout v^T - D_i),
 * D_i = rowsum(dout * o). workspace: caller-provided fp32 [2*B*H*N].
 * Replaces flash_attn_backward (cuda/flash_attn_kernel.cu:417-503), which
 * takes the same six tensors (fp32 there) and returns [dQ, dK, dV]; the causal
 * flag and D = 128 have no reference counterpart.
 */
int fa_bwd_f16(const void* q, const void* k, const void* v, const void* o, const void* dout,
               const float* lse, float* dq, float* dk, float* dv, float* workspace,
               int64_t B, int64_t H, int64_t N, int64_t D, int causal, void* stream);

/*
 * Floats of the workspace fa_bwd_gqa_f16 needs: 2*B*H*N for H_kv == H, plus,
 * for H_kv < H, the per-query-head dK and dV partials (2*B*H*N*D floats from
 * the next 16-byte boundary). 0 for invalid sizes.
 */
int64_t fa_bwd_gqa_workspace_floats(int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D);

/*
 * fa_bwd_f16 with grouped KV heads: k, v fp16 [B, H_kv, N, D] (H % H_kv == 0,
 * else FA_ERR_KV_HEADS) and dk, dv fp32 [B, H_kv, N, D], each the sum over the
 * H / H_kv query heads that share the KV head. With H_kv < H the workspace
 * must be 16-byte aligned. No reference counterpart.
 */
int fa_bwd_gqa_f16(const void* q, const void* k, const void* v, const void* o, const void* dout,
                   const float* lse, float* dq, float* dk, float* dv, float* workspace,
                   int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D, int causal,
                   void* stream);

/*
 * bfloat16 backward: fa_bwd_gqa_f16 with q, k, v, o, dout in bf16 (H_kv == H
 * for plain multi-head); P and dS are rounded to bf16 for their products,
 * everything else as in the fp16 path. Workspace: fa_bwd_gqa_workspace_floats.
 * No reference counterpart.
 */
int fa_bwd_bf16(const void* q, const void* k, const void* v, const void* o, const void* dout,
                const float* lse, float* dq, float* dk, float* dv, float* workspace,
                int64_t B, int64_t H, int64_t H_kv, int64_t N, int64_t D, int causal,
                void* stream);

/*
 * Backward of fa_fwd_varlen_f16: q/o/dout [H, total, D] fp16, k/v [H_kv,
 * total, D] fp16, lse [H, total] fp32 (the forward's L), sequence b = rows
 * cu_seqlens[b] .. cu_seqlens[b+1] of every head (bounds clamped as in the
 * forward); dq [H, total, D], dk/dv [H_kv, total, D] fp32. Workspace:
 * fa_bwd_gqa_workspace_floats(1, H, H_kv, total, D) floats, 16-byte aligned
 * when H_kv < H. Rows outside every sequence are not written (with H_kv < H
 * dk/dv get the sum of the workspace's unwritten partial rows there: zero
 * the workspace first where zeros are wanted). No reference counterpart.
 */
int fa_bwd_varlen_f16(const void* q, const void* k, const void* v, const void* o,
                      const void* dout, const float* lse, float* dq, float* dk, float* dv,
                      float* workspace, const int32_t* cu_seqlens, int64_t B, int64_t H,
                      int64_t H_kv, int64_t max_seqlen, int64_t total, int64_t D, int causal,
                      void* stream);

/* Host-only argument check of fa_bwd_varlen_f16. */
int fa_validate_bwd_varlen(const void* q, const void* k, const void* v, const void* o,
                           const void* dout, const float* lse, const float* dq, const float* dk,
                           const float* dv, const float* workspace, const int32_t* cu_seqlens,
                           int64_t B, int64_t H, int64_t H_kv, int64_t max_seqlen,
                           int64_t total, int64_t D);

/*
 * Split-KV forward (no reference counterpart): fa_fwd_gqa_f16's result with
 * each 128-row block's keys cut into num_splits ranges run as separate
 * workgroups, then merged by the LSE combine (fills the GPU when B*H*N/128
 * row blocks are at most half the CUs, and evens out causal row blocks of
 * different lengths). O within the
 * forward's tolerance of the unsplit kernel; lse nullable (O only). The
 * workspace (fa_fwd_splitkv_workspace_floats floats, 16-byte aligned) holds
 * the fp32 partials. fa_fwd_splitkv_plan returns the split count the torch
 * binding uses (1: no split) for a shape on the current device (it depends on
 * the device's compute-unit count).
 */
int fa_fwd_splitkv_plan(int64_t B, int64_t H, int64_t N, int64_t D, int causal);
int64_t fa_fwd_splitkv_workspace_floats(int64_t B, int64_t H, int64_t N, int64_t D,
                                        int64_t num_splits);
int fa_fwd_splitkv_f16(const void* q, const void* k, const void* v, void* o, float* lse,
                       float* workspace, int64_t B, int64_t H, int64_t H_kv, int64_t N,
                       int64_t D, int causal, int64_t num_splits, void* stream);

/*
 * Host-only argument check of the decode entry points. No reference
 * counterpart (the reference has no decode path).
 */
int fa_validate_decode(const void* q, const void* k_pool, const void* v_pool,
                       const int32_t* page_table, const int32_t* ctx_lens,
                       int64_t B, int64_t H, int64_t D, int64_t page_size,
                       int64_t max_pages, int64_t num_pages, int64_t num_splits);

/* Floats of split workspace the caller provides: part_o then part_lse. */
int64_t fa_decode_workspace_floats(int64_t B, int64_t H, int64_t D,
                                   int64_t num_splits);

/*
 * Split pass of the paged decode: for each (sequence b, head h, split s) the
 * normalised partial attention of q[b,h] over the split's pages (QK and PV
 * on fp16 matrix-core products with fp32 accumulation; P rounded to fp16
 * for the PV product).
 * Sequence b has ceil(ctx_lens[b]/page_size) pages, divided into num_splits
 * runs of ceil(pages/num_splits) pages. An empty split writes part_o = 0 and
 * part_lse = -inf. A page id outside [0, num_pages) makes the partials of
 * the splits that touch the bad page NaN; a negative ctx_lens[b] or one
 * beyond max_pages*page_size makes every partial of that sequence NaN. No
 * memory outside the pool is read. No reference counterpart.
 */
int fa_decode_split_f16(const void* q, const void* k_pool, const void* v_pool,
                        const int32_t* page_table, const int32_t* ctx_lens,
                        int64_t B, int64_t H, int64_t D, int64_t page_size,
                        int64_t max_pages, int64_t num_pages, int64_t num_splits,
                        float* part_o, float* part_lse, void* stream);

/*
 * Combine pass: L = log sum_s exp(part_lse_s); o = sum_s exp(part_lse_s - L)
 * part_o_s, written as fp16 o [B, H, D] and fp32 lse [B, H] (lse may be NULL).
 * If every split is empty, o = 0 and lse = -inf; a NaN partial makes o and
 * lse of its (b, h) NaN. No reference counterpart.
 */
int fa_lse_combine_f32(const float* part_o, const float* part_lse,
                       int64_t B, int64_t H, int64_t D, int64_t num_splits,
                       void* o, float* lse, void* stream);

/* Split pass then combine pass, both on `stream`. No reference counterpart. */
int fa_decode_paged_f16(const void* q, const void* k_pool, const void* v_pool,
                        const int32_t* page_table, const int32_t* ctx_lens,
                        int64_t B, int64_t H, int64_t D, int64_t page_size,
                        int64_t max_pages, int64_t num_pages, int64_t num_splits,
                        float* part_o, float* part_lse, void* o, float* lse,
                        void* stream);

/*
 * fa_decode_paged_f16 with grouped KV heads: k_pool / v_pool are
 * [num_pages, H_kv, 16, D] and query head h reads pool head h / (H / H_kv)
 * (H % H_kv == 0, else FA_ERR_KV_HEADS). part_o / part_lse / o / lse are per
 * query head, as in fa_decode_paged_f16. No reference counterpart.
 */
int fa_decode_paged_gqa_f16(const void* q, const void* k_pool, const void* v_pool,
                            const int32_t* page_table, const int32_t* ctx_lens, int64_t B,
                            int64_t H, int64_t H_kv, int64_t D, int64_t page_size,
                            int64_t max_pages, int64_t num_pages, int64_t num_splits,
                            float* part_o, float* part_lse, void* o, float* lse, void* stream);

/*
 * fa_decode_paged_gqa_f16 that allocates nothing and takes no workspace: the
 * split partials go to a static device array of FA_DECODE_SCRATCH_FLOATS
 * floats that the library holds on each GPU it runs on until the process
 * ends (its address is resolved once per device, on that device's first
 * call: make that first call outside HIP graph capture; later calls record
 * only kernel launches and can be captured and replayed, which
 * tests/test_zz_no_alloc.py checks bit for bit against
 * fa_decode_paged_gqa_f16). Needs B*H*num_splits*(D+1) <=
 * FA_DECODE_SCRATCH_FLOATS, else
 * FA_ERR_SCRATCH_SIZE (B = 32, H = 32, D = 128, 16 splits uses half). Makes
 * no hipMalloc/hipFree or other allocating call. Nothing in the array has to
 * start at zero (every partial a call reads, that call wrote). All calls on
 * one GPU share the array, so calls that overlap on one GPU (different
 * streams, or host threads) race; calls on one stream are ordered. Same
 * arguments, layouts and results as fa_decode_paged_gqa_f16, bit for bit.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).
 */
int fa_decode_paged_noalloc_f16(const void* q, const void* k_pool, const void* v_pool,
                                const int32_t* page_table, const int32_t* ctx_lens, int64_t B,
                                int64_t H, int64_t H_kv, int64_t D, int64_t page_size,
                                int64_t max_pages, int64_t num_pages, int64_t num_splits,
                                void* o, float* lse, void* stream);

/*
 * fa_decode_paged_gqa_f16 for bf16 q, pools and O (same layouts and
 * arguments; QK products of bf16 pairs accumulated in fp32, P carried into
 * the PV product as two bf16 terms (~16 significant bits), softmax and merges
 * in fp32, O rounded to bf16 to nearest even). No reference counterpart (the
 * reference has neither a decode path nor bf16).
 */
int fa_decode_paged_bf16(const void* q, const void* k_pool, const void* v_pool,
                         const int32_t* page_table, const int32_t* ctx_lens, int64_t B, int64_t H,
                         int64_t H_kv, int64_t D, int64_t page_size, int64_t max_pages,
                         int64_t num_pages, int64_t num_splits, float* part_o, float* part_lse,
                         void* o, float* lse, void* stream);

/*
 * Host-only argument check of fa_kv_append_f16. No reference counterpart.
 */
int fa_validate_kv_append(const void* k_new, const void* v_new, const int32_t* page_table,
                          const int32_t* start_pos, const int32_t* new_lens, const void* k_pool,
                          const void* v_pool, const int32_t* bad, int64_t B, int64_t H,
                          int64_t T, int64_t D, int64_t page_size, int64_t max_pages,
                          int64_t num_pages);

/*
 * KV-cache page writer (append, or reshape a prefill into pages): for each
 * sequence b and new token t < n_b (n_b = new_lens[b] clamped to [0, T], or T
 * if new_lens is NULL), copies k_new[b,h,t,:] and v_new[b,h,t,:] (fp16
 * [B, H, T, D]) into k_pool / v_pool (fp16 [num_pages, H, 16, D], the layout
 * fa_decode_paged_f16 reads) at position p = start_pos[b] + t: page
 * page_table[b][p / 16], slot p % 16. Bit-exact copy. A token whose position
 * is negative or not below max_pages*16, or whose page id is outside
 * [0, num_pages), is not written; if `bad` is not NULL, bad[b] is set to 1
 * for that sequence (the caller zeroes `bad`). With T = 0 nothing is copied
 * and k_new / v_new may be NULL. Tokens of different sequences must not map
 * to the same (page, slot): such writes race. No reference
 * counterpart (the reference has no KV cache); it is the step before the
 * paged decode.
 */
int fa_kv_append_f16(const void* k_new, const void* v_new, const int32_t* page_table,
                     const int32_t* start_pos, const int32_t* new_lens, void* k_pool,
                     void* v_pool, int32_t* bad, int64_t B, int64_t H, int64_t T, int64_t D,
                     int64_t page_size, int64_t max_pages, int64_t num_pages, void* stream);

/*
 * fa_kv_append_f16 for bf16 rows and pools (same arguments; the copy moves
 * 16-bit elements without arithmetic). No reference counterpart.
 */
int fa_kv_append_bf16(const void* k_new, const void* v_new, const int32_t* page_table,
                      const int32_t* start_pos, const int32_t* new_lens, void* k_pool,
                      void* v_pool, int32_t* bad, int64_t B, int64_t H, int64_t T, int64_t D,
                      int64_t page_size, int64_t max_pages, int64_t num_pages, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FA_MI355X_H */
