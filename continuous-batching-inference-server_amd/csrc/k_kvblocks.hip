// Whole-page gather / scatter between the paged K/V allocation and a
// block-major staging buffer, for the tiered block manager's spill and
// restore.  The reference moves one block (a physical page's K and V slots in
// every layer) with 2 * n_layers synchronous copies
// (src/tiered_kv_manager.cpp:69-98); here one launch moves every block of a
// batch, one workgroup per (block, layer, K|V) page, 16-byte non-temporal
// accesses (each byte is touched once, nothing is reused).
//
// Pool layout (PagedKVCache): [n_layers][2][max_pages][page_bytes].
// Staging layout: [n_pages][n_layers][2][page_bytes] -- block b's raw bytes
// are contiguous, in the reference's block byte order (layer 0 K, layer 0 V,
// layer 1 K, ...).
#include "common.hpp"

namespace cbis {
namespace {

constexpr int kCopyThreads = 256;

template <bool kGather>
__global__ __launch_bounds__(kCopyThreads) void kv_pages_kernel(u32x4_t* __restrict__ staging,
                                                                 u32x4_t* __restrict__ pools,
                                                                 const int* __restrict__ pages, int n_layers,
                                                                 int max_pages, int64_t page_units) {
  const int64_t job = blockIdx.x;  // (block, layer, K|V)
  const int b = (int)(job / (2 * n_layers));
  const int lc = (int)(job % (2 * n_layers));
  const int page = pages[b];
  if (page < 0 || page >= max_pages) return;  // rejected on the host; never dereferenced
  u32x4_t* pool_page = pools + ((int64_t)lc * max_pages + page) * page_units;
  u32x4_t* stage_page = staging + job * page_units;
  for (int64_t i = threadIdx.x; i < page_units; i += kCopyThreads) {
    if constexpr (kGather) {
      __builtin_nontemporal_store(__builtin_nontemporal_load(pool_page + i), stage_page + i);
    } else {
      __builtin_nontemporal_store(__builtin_nontemporal_load(stage_page + i), pool_page + i);
    }
  }
}

int kv_pages(bool gather, void* staging, void* pools, int n_layers, int max_pages, int64_t page_bytes,
             const int* pages, int n_pages, cbis_stream_t stream, const char* who) {
  CBIS_REQUIRE(n_pages >= 0 && n_layers > 0 && max_pages > 0 && page_bytes > 0, CBIS_ERR_INVALID,
               "%s: bad sizes (n_pages %d, n_layers %d, max_pages %d, page_bytes %lld)", who, n_pages, n_layers,
               max_pages, (long long)page_bytes);
  if (n_pages == 0) return CBIS_OK;
  CBIS_REQUIRE(page_bytes % 16 == 0, CBIS_ERR_INVALID, "%s: page_bytes %lld must be a multiple of 16", who,
               (long long)page_bytes);
  CBIS_REQUIRE(staging && pools && pages, CBIS_ERR_INVALID, "%s: null pointer", who);
  CBIS_REQUIRE(((uintptr_t)staging & 15u) == 0 && ((uintptr_t)pools & 15u) == 0 && ((uintptr_t)pages & 3u) == 0,
               CBIS_ERR_INVALID, "%s: staging / pools must be 16-byte aligned", who);
  const int64_t jobs = (int64_t)n_pages * 2 * n_layers;
  CBIS_REQUIRE(jobs < (int64_t)1 << 31, CBIS_ERR_INVALID, "%s: too many pages in one call", who);
  hipStream_t s = (hipStream_t)stream;
  if (gather)
    kv_pages_kernel<true><<<(unsigned)jobs, kCopyThreads, 0, s>>>((u32x4_t*)staging, (u32x4_t*)pools, pages, n_layers,
                                                                 max_pages, page_bytes / 16);
  else
    kv_pages_kernel<false><<<(unsigned)jobs, kCopyThreads, 0, s>>>((u32x4_t*)staging, (u32x4_t*)pools, pages, n_layers,
                                                                  max_pages, page_bytes / 16);
  return check_launch(who);
}

}  // namespace
}  // namespace cbis

using namespace cbis;

extern "C" {

int cbis_kv_pages_gather(void* staging, const void* pools, int n_layers, int max_pages, int64_t page_bytes,
                         const int* pages, int n_pages, cbis_stream_t stream) {
  return kv_pages(true, staging, const_cast<void*>(pools), n_layers, max_pages, page_bytes, pages, n_pages, stream,
                  "cbis_kv_pages_gather");
}

int cbis_kv_pages_scatter(void* pools, const void* staging, int n_layers, int max_pages, int64_t page_bytes,
                          const int* pages, int n_pages, cbis_stream_t stream) {
  return kv_pages(false, const_cast<void*>(staging), pools, n_layers, max_pages, page_bytes, pages, n_pages, stream,
                  "cbis_kv_pages_scatter");
}

}  // extern "C"
