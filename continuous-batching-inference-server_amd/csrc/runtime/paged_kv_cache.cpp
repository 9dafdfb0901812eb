// PagedKVCache: block bookkeeping of src/paged_kv_cache.cpp:5-60, bit-exact,
// separable from device memory (alloc_device = false runs without a GPU),
// and a single device arena for every layer's K and V pools.
#include <algorithm>

#include "runtime.hpp"

namespace cbis {

size_t dtype_size(int dtype) {
  switch (dtype) {
    case CBIS_F32: return 4;
    case CBIS_BF16: return 2;
    case CBIS_FP8E4M3: return 1;
    default: throw std::invalid_argument("unknown dtype " + std::to_string(dtype));
  }
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void cbis_check(int rc, const char* what) {
  if (rc != CBIS_OK) throw std::runtime_error(std::string(what) + ": " + cbis_last_error());
}

void ModelConfig::validate() const {
  if (vocab <= 0 || d_model <= 0 || n_heads <= 0 || head_dim <= 0 || n_layers <= 0 || mlp <= 0 || max_seq <= 0 ||
      page_size <= 0)
    throw std::invalid_argument("ModelConfig: every dimension must be positive");
  if (n_heads * head_dim != d_model) throw std::invalid_argument("ModelConfig: n_heads * head_dim != d_model");
  if (max_seq % page_size != 0) throw std::invalid_argument("ModelConfig: max_seq must be page-aligned");
  if (weight_dtype != CBIS_F32 && weight_dtype != CBIS_BF16 && weight_dtype != CBIS_FP8E4M3)
    throw std::invalid_argument("ModelConfig: weight dtype");
  if (kv_dtype != CBIS_F32 && kv_dtype != CBIS_BF16) throw std::invalid_argument("ModelConfig: kv dtype");
}

PagedKVCache::PagedKVCache(int num_layers, int max_pages, int page_size, int n_heads, int head_dim, int kv_dtype,
                           int pages_per_seq, bool alloc_device)
    : num_layers_(num_layers),
      max_pages_(max_pages),
      page_size_(page_size),
      n_heads_(n_heads),
      head_dim_(head_dim),
      kv_dtype_(kv_dtype),
      pages_per_seq_(pages_per_seq) {
  if (num_layers <= 0 || max_pages <= 0 || page_size <= 0 || n_heads <= 0 || head_dim <= 0 || pages_per_seq <= 0)
    throw std::invalid_argument("PagedKVCache: sizes must be positive");
  layer_bytes_ = (size_t)max_pages * page_size * n_heads * head_dim * dtype_size(kv_dtype);
  if (alloc_device) {
    const size_t total = layer_bytes_ * 2 * (size_t)num_layers;
    hip_check(hipMalloc((void**)&base_, total), "PagedKVCache: hipMalloc");
    hip_check(hipMemset(base_, 0, total), "PagedKVCache: hipMemset");
  }
  free_pages_.reserve(max_pages);
  for (int p = max_pages - 1; p >= 0; --p) free_pages_.push_back(p);
}

PagedKVCache::~PagedKVCache() {
  if (base_) (void)hipFree(base_);
}

int PagedKVCache::allocate_sequence() {
  const int id = next_seq_id_++;
  seq_pages_[id] = {};
  return id;
}

void PagedKVCache::free_sequence(int seq_id) {
  auto it = seq_pages_.find(seq_id);
  if (it == seq_pages_.end()) return;
  for (int page : it->second) free_pages_.push_back(page);
  seq_pages_.erase(it);
}

bool PagedKVCache::ensure_capacity(int seq_id, int token_pos) {
  auto& pages = seq_pages_.at(seq_id);
  const int needed = token_pos / page_size_ + 1;
  while ((int)pages.size() < needed) {
    if (free_pages_.empty()) return false;
    pages.push_back(free_pages_.back());
    free_pages_.pop_back();
  }
  return true;
}

void PagedKVCache::resolve_slot(int seq_id, int token_pos, int* physical_page, int* offset) const {
  const auto& pages = seq_pages_.at(seq_id);
  *physical_page = pages.at(token_pos / page_size_);
  *offset = token_pos % page_size_;
}

std::vector<int> PagedKVCache::page_table(int seq_id) const {
  const auto& pages = seq_pages_.at(seq_id);
  std::vector<int> table(pages_per_seq_, 0);
  for (size_t i = 0; i < pages.size() && i < table.size(); ++i) table[i] = pages[i];
  return table;
}

const std::vector<int>& PagedKVCache::pages(int seq_id) const { return seq_pages_.at(seq_id); }

void* PagedKVCache::k_base(int layer) const {
  if (!base_) throw std::logic_error("PagedKVCache: created without device pools");
  if (layer < 0 || layer >= num_layers_) throw std::out_of_range("PagedKVCache::k_base: layer");
  return base_ + (size_t)layer * 2 * layer_bytes_;
}

void* PagedKVCache::v_base(int layer) const {
  if (!base_) throw std::logic_error("PagedKVCache: created without device pools");
  if (layer < 0 || layer >= num_layers_) throw std::out_of_range("PagedKVCache::v_base: layer");
  return base_ + ((size_t)layer * 2 + 1) * layer_bytes_;
}

void PagedKVCache::fill_normal(uint64_t seed, float std, hipStream_t s) {
  if (!base_) throw std::logic_error("PagedKVCache: created without device pools");
  const int64_t n = (int64_t)(layer_bytes_ * 2 * (size_t)num_layers_ / dtype_size(kv_dtype_));
  cbis_check(cbis_fill_normal_fast(base_, kv_dtype_, n, seed, std, s), "PagedKVCache::fill_normal");
  hip_check(hipStreamSynchronize(s), "PagedKVCache::fill_normal sync");
}

}  // namespace cbis
