/*
 * fa_probe.h — device probes of the gfx950 matrix-core and LDS layouts that
 * the forward kernel relies on. Test support only; the analogue of the
 * reference's mma probe module (cuda/mma_probe.cu:256-320, exported to Python
 * at cuda/mma_probe.cu:314-320), rebuilt for v_mfma_f32_32x32x16_f16,
 * v_mfma_f32_16x16x32_f16 and ds_read_b64_tr_b16.
 *
 * All buffers are device pointers; every probe runs one wave on `stream`.
 * Return: 0 ok, > 0 bad argument, < 0 negated hipError_t.
 *
 * Probe interface version FA_PROBE_VERSION (separate from the product ABI's
 * fa_abi_version): 2 added the causal argument of fa_probe_fwd_variants;
 * 3 removed variant 418 and added fa_probe_choose_variant and
 * fa_probe_splitkv_plan_cus (the kernel and split choices for a given
 * compute-unit count, without a device); 4 added fa_probe_gather_bw.
 */
#ifndef FA_PROBE_H
#define FA_PROBE_H

#include <stdint.h>

#define FA_PROBE_VERSION 4

#ifdef __cplusplus
extern "C" {
#endif

/* c[32][32] = a[32][16] @ b[16][32] (fp16 in, fp32 out) with the lane layout
 * the kernels assume; variant 1 swaps A's k-halves (negative control). */
int fa_probe_mfma32(const void* a, const void* b, float* c, int variant, void* stream);

/* c[16][16] = a[16][32] @ b[32][16]; variant 1 reverses A's k-groups. */
int fa_probe_mfma16(const void* a, const void* b, float* c, int variant, void* stream);

/* LDS holds the 256 halves of `in`; lane l executes ds_read_b64_tr_b16 at byte
 * offset 8*l and writes its 4 halves to out[4*l .. 4*l+3]. */
int fa_probe_tr16_raw(const void* in, void* out, void* stream);

/* v_permlane32_swap_b32 on x = in[0..63]: out[0..63] and out[64..127] are the
 * two results; out[128..191] = max(x[l], x[l^32]), out[192..255] = x[l] + x[l^32]
 * through the forward kernel's helpers. */
int fa_probe_permlane(const float* in, float* out, void* stream);

/* Stores a [64][D] fp16 tile with the forward kernel's K and V LDS layouts and
 * dumps every operand fragment the kernel reads:
 *   kout [2][D/16][64][8], vout [4][D/32][64][8] fp16. D in {64, 128}. */
int fa_probe_frags(const void* tile, void* kout, void* vout, int64_t D, void* stream);

/* One 64-key tile through the kernel's loaders and MFMA chain without softmax:
 * o[32][D] = fp16(q[32][D] @ k[64][D]^T) @ v[64][D], fp32 out. */
int fa_probe_chain(const void* q, const void* k, const void* v, float* o, int64_t D,
                   void* stream);

/* fa_fwd_f16 with an explicit kernel variant (the codes fa_probe_fwd_variants
 * lists for D, or 0 for the default), so the tests can check every variant in
 * one process. 1000 + v runs variant v through its guarded instance (bounds
 * predicates compiled in) even where N is a multiple of the 128-row block, for
 * the full-tile vs guarded identity. Returns FA_ERR_HEAD_DIM for a variant
 * that does not exist for D. */
int fa_probe_fwd_variant(const void* q, const void* k, const void* v, void* o, float* lse,
                         int64_t B, int64_t H, int64_t N, int64_t D, int causal, int variant,
                         void* stream);

/* The variant fa_fwd_f16 runs for head dimension D at the headline shape
 * (B = 1, H = 8, N = 4096, non-causal) on the current device (0 for another
 * D). 204 = ping-pong kernel with two tile groups over 128 rows (ring of 4
 * tiles), 408 = with four tile groups over 64 rows (ring of 8 tiles,
 * D = 64); the forward picks 408 for D = 64 where 128-row workgroups leave
 * CUs idle. */
int fa_probe_default_variant(int64_t D);

/* The variant the forward picks for bh = B*H heads of N rows on a device of
 * `cus` compute units (the device's own count is read at launch time).
 * 0 for a bad argument. No device needed. */
int fa_probe_choose_variant(int64_t D, int causal, int64_t bh, int64_t N, int cus);

/* fa_fwd_splitkv_plan for a device of `cus` compute units instead of the
 * current device's. No device needed. */
int fa_probe_splitkv_plan_cus(int64_t B, int64_t H, int64_t N, int64_t D, int causal, int cus);

/* Writes up to max_out variant codes that exist for head dimension D and the
 * causal flag into out (may be NULL) and returns how many there are. */
int fa_probe_fwd_variants(int* out, int max_out, int64_t D, int causal);

/* Streams `bytes` (a multiple of 16, 16-byte aligned) from device memory at p
 * with `blocks` workgroups of 256 threads, each over one contiguous chunk,
 * 16-byte non-temporal loads, 8 in flight per thread: the read bandwidth a
 * plain kernel reaches on this device, the ceiling the paged decode's split
 * pass is measured against. sink: one device uint32, written only on a
 * 2^-32 chance. 1: NULL argument, 2: bad size, alignment or grid. */
int fa_probe_read_bw(const void* p, int64_t bytes, int blocks, uint32_t* sink, void* stream);

/* Reads `pages` 4 KiB pages from each of two pools (k, v: pages * 4096
 * bytes each, 16-byte aligned) in the order of `table` (int32 page ids,
 * clamped into [0, pages)), the access pattern of the paged decode: one
 * workgroup of 4 waves per `pages_per_wg` consecutive table entries, wave w
 * taking entries w, w + 4, ...; each load instruction reads 1 KiB of a page
 * contiguously, with the non-temporal hint when `nontemporal` is non-zero.
 * The ceiling of the decode's split pass for a given table. sink as above.
 * 1: NULL argument, 2: bad size, alignment or grid. */
int fa_probe_gather_bw(const void* k, const void* v, const int32_t* table, int64_t pages,
                       int pages_per_wg, int nontemporal, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FA_PROBE_H */
