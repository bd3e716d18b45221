// fa_pages.hip — KV-cache page writer for MI355X: appends new K/V rows of each
// sequence into the paged pools the decode kernel reads.
//
// No reference counterpart (the reference has no KV cache). Pool layout is the
// decode's: [num_pages, H, 16, D] fp16, so the 16 token slots of one head in a
// page are one contiguous 16*D*2-byte run. Token t of sequence b goes to
// position p = start_pos[b] + t: page page_table[b][p / 16], slot p % 16.
//
// The work is a pure copy (HBM-bound): one lane moves one 16-byte chunk of a
// row for both K and V; a workgroup covers 256 / (D/8) consecutive tokens of
// one (b, h), so reads are contiguous and writes are contiguous within each
// page's run of 16 slots.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "fa_mi355x.h"

namespace fa {
namespace pages {

constexpr int kPageSize = 16;
constexpr int kThreads = 256;

template <int D>
__global__ void __launch_bounds__(kThreads)
fa_kv_append_kernel(const uint4* __restrict__ k_new, const uint4* __restrict__ v_new,
                    const int32_t* __restrict__ page_table, const int32_t* __restrict__ start_pos,
                    const int32_t* __restrict__ new_lens, uint4* __restrict__ k_pool,
                    uint4* __restrict__ v_pool, int32_t* __restrict__ bad, int H, int T,
                    int max_pages, int num_pages) {
  constexpr int CH = D / 8;            // 16-byte chunks per row
  constexpr int ROWS = kThreads / CH;  // tokens per workgroup
  const int h = blockIdx.y, b = blockIdx.z;
  const int t = blockIdx.x * ROWS + (int)threadIdx.x / CH;
  const int c = (int)threadIdx.x % CH;
  int n = T;
  if (new_lens) n = min(max(new_lens[b], 0), T);
  if (t >= n) return;
  const int64_t p = (int64_t)start_pos[b] + t;
  bool ok = p >= 0 && p < (int64_t)max_pages * kPageSize;
  const int pid = ok ? page_table[(size_t)b * max_pages + (size_t)(p / kPageSize)] : -1;
  ok = ok && pid >= 0 && pid < num_pages;
  if (!ok) {
    if (bad && c == 0) bad[b] = 1;   // same value from every writer: benign
    return;
  }
  const size_t src = (((size_t)b * H + h) * T + t) * CH + c;
  const size_t dst = (((size_t)pid * H + h) * kPageSize + (size_t)(p % kPageSize)) * CH + c;
  const uint4 kx = k_new[src];
  const uint4 vx = v_new[src];
  k_pool[dst] = kx;
  v_pool[dst] = vx;
}

}  // namespace pages
}  // namespace fa

extern "C" int fa_kv_append_f16(const void* k_new, const void* v_new, const int32_t* page_table,
                                const int32_t* start_pos, const int32_t* new_lens, void* k_pool,
                                void* v_pool, int32_t* bad, int64_t B, int64_t H, int64_t T,
                                int64_t D, int64_t page_size, int64_t max_pages,
                                int64_t num_pages, void* stream) {
  using namespace fa::pages;
  const int st = fa_validate_kv_append(k_new, v_new, page_table, start_pos, new_lens, k_pool,
                                       v_pool, bad, B, H, T, D, page_size, max_pages, num_pages);
  if (st != FA_OK) return st;
  if (T == 0) return FA_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int rows = kThreads / (int)(D / 8);
  const dim3 grid((unsigned)((T + rows - 1) / rows), (unsigned)H, (unsigned)B);
  if (D == 64) {
    hipLaunchKernelGGL((fa_kv_append_kernel<64>), grid, dim3(kThreads), 0, s,
                       (const uint4*)k_new, (const uint4*)v_new, page_table, start_pos, new_lens,
                       (uint4*)k_pool, (uint4*)v_pool, bad, (int)H, (int)T, (int)max_pages,
                       (int)num_pages);
  } else {
    hipLaunchKernelGGL((fa_kv_append_kernel<128>), grid, dim3(kThreads), 0, s,
                       (const uint4*)k_new, (const uint4*)v_new, page_table, start_pos, new_lens,
                       (uint4*)k_pool, (uint4*)v_pool, bad, (int)H, (int)T, (int)max_pages,
                       (int)num_pages);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? FA_OK : -(int)e;
}

// bf16 rows into bf16 pools: the kernel moves 16-byte chunks of 16-bit
// elements without arithmetic, so the fp16 path serves both element types.
extern "C" int fa_kv_append_bf16(const void* k_new, const void* v_new, const int32_t* page_table,
                                 const int32_t* start_pos, const int32_t* new_lens, void* k_pool,
                                 void* v_pool, int32_t* bad, int64_t B, int64_t H, int64_t T,
                                 int64_t D, int64_t page_size, int64_t max_pages,
                                 int64_t num_pages, void* stream) {
  return fa_kv_append_f16(k_new, v_new, page_table, start_pos, new_lens, k_pool, v_pool, bad, B,
                          H, T, D, page_size, max_pages, num_pages, stream);
}
