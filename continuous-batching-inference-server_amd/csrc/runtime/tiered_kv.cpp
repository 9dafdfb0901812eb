// Three-tier KV block manager: the API and policy of
// include/tiered_kv_manager.hpp / src/tiered_kv_manager.cpp and the host
// blob store of src/block_storage.cpp, on HIP.
//
// Block bytes leave and enter the device through cbis_kv_pages_gather /
// cbis_kv_pages_scatter: one launch and one pinned host copy per batch (per
// chunk of up to kStageBytes), instead of the reference's 2 * n_layers
// synchronous copies per block -- the restore cost its README measures
// (README.md:237-250).  Deflate / inflate of a batch's blocks runs on the
// host cores in parallel.  Eviction: score = alpha * (now - last_access) -
// beta * (fixed_ns + raw_bytes * expected_ratio * ns_per_byte) of the tier
// the block would go to (DRAM while it has room, else NVMe); the block with
// the highest score goes, ties to the smallest block id.
#include <fcntl.h>
#include <unistd.h>
#include <zlib.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cstring>
#include <set>

#include "runtime.hpp"

namespace cbis {

namespace {
constexpr size_t kStageBytes = (size_t)256 << 20;  // staging per chunk of a batch
}

// ---------------------------------------------------------------------------
// Block codec (zlib deflate at its fastest level, as src/block_storage.cpp:7-23
// settled on: K/V mantissas barely compress, so effort buys little).
// ---------------------------------------------------------------------------
std::vector<uint8_t> deflate_block(const void* data, size_t len) {
  uLongf cap = compressBound((uLong)len);
  std::vector<uint8_t> out(cap);
  const int rc = compress2(out.data(), &cap, (const Bytef*)data, (uLong)len, Z_BEST_SPEED);
  if (rc != Z_OK) throw std::runtime_error("deflate_block: zlib error " + std::to_string(rc));
  out.resize(cap);
  return out;
}

void inflate_block(const uint8_t* comp, size_t comp_len, void* out, size_t out_len) {
  uLongf n = (uLongf)out_len;
  const int rc = uncompress((Bytef*)out, &n, comp, (uLong)comp_len);
  if (rc != Z_OK) throw std::runtime_error("inflate_block: zlib error " + std::to_string(rc));
  if (n != out_len) throw std::runtime_error("inflate_block: size mismatch");
}

// ---------------------------------------------------------------------------
// NvmeBlockStore
// ---------------------------------------------------------------------------
NvmeBlockStore::NvmeBlockStore(const std::string& path) : path_(path) {
  fd_ = ::open(path.c_str(), O_RDWR | O_CREAT | O_TRUNC, 0644);
  if (fd_ < 0) throw std::runtime_error("NvmeBlockStore: cannot open " + path + ": " + std::strerror(errno));
}

NvmeBlockStore::~NvmeBlockStore() {
  if (fd_ >= 0) ::close(fd_);
}

NvmeBlockStore::Loc NvmeBlockStore::write_block(const uint8_t* data, uint32_t length) {
  const Loc loc{next_, length};
  size_t done = 0;
  while (done < length) {
    const ssize_t n = ::pwrite(fd_, data + done, length - done, (off_t)(loc.offset + done));
    if (n < 0 && errno == EINTR) continue;
    if (n <= 0) throw std::runtime_error("NvmeBlockStore::write_block: short write");
    done += (size_t)n;
  }
  next_ += length;
  return loc;
}

void NvmeBlockStore::read_block(Loc loc, uint8_t* out) const {
  size_t done = 0;
  while (done < loc.length) {
    const ssize_t n = ::pread(fd_, out + done, loc.length - done, (off_t)(loc.offset + done));
    if (n < 0 && errno == EINTR) continue;
    if (n <= 0) throw std::runtime_error("NvmeBlockStore::read_block: short read");
    done += (size_t)n;
  }
}

std::vector<uint8_t> NvmeBlockStore::read_block(Loc loc) const {
  std::vector<uint8_t> buf(loc.length);
  read_block(loc, buf.data());
  return buf;
}

// ---------------------------------------------------------------------------
// TieredKVBlockManager
// ---------------------------------------------------------------------------
TieredKVBlockManager::TieredKVBlockManager(int layer_count, int page_size, int n_heads, int head_dim,
                                           const std::string& nvme_scratch_path, size_t gpu_capacity_blocks,
                                           size_t dram_capacity_blocks, EvictionParams params, int kv_dtype)
    : layer_count_(layer_count),
      page_size_(page_size),
      n_heads_(n_heads),
      head_dim_(head_dim),
      kv_dtype_(kv_dtype),
      gpu_capacity_blocks_(gpu_capacity_blocks),
      dram_capacity_blocks_(dram_capacity_blocks),
      params_(params),
      nvme_(nvme_scratch_path) {
  if (layer_count <= 0 || page_size <= 0 || n_heads <= 0 || head_dim <= 0)
    throw std::invalid_argument("TieredKVBlockManager: sizes must be positive");
  if (kv_dtype != CBIS_F32 && kv_dtype != CBIS_BF16) throw std::invalid_argument("TieredKVBlockManager: kv dtype");
  page_bytes_ = (size_t)page_size * n_heads * head_dim * dtype_size(kv_dtype);
  raw_block_bytes_ = (size_t)layer_count * 2 * page_bytes_;
  hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "TieredKVBlockManager: stream");
}

TieredKVBlockManager::~TieredKVBlockManager() {
  if (host_stage_) (void)hipHostFree(host_stage_);
  if (host_pages_) (void)hipHostFree(host_pages_);
  if (dev_stage_) (void)hipFree(dev_stage_);
  if (dev_pages_) (void)hipFree(dev_pages_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

void TieredKVBlockManager::reserve(size_t blocks) {
  if (blocks <= stage_blocks_) return;
  if (host_stage_) hip_check(hipHostFree(host_stage_), "hipHostFree");
  if (host_pages_) hip_check(hipHostFree(host_pages_), "hipHostFree");
  if (dev_stage_) hip_check(hipFree(dev_stage_), "hipFree");
  if (dev_pages_) hip_check(hipFree(dev_pages_), "hipFree");
  host_stage_ = dev_stage_ = nullptr;
  host_pages_ = dev_pages_ = nullptr;
  stage_blocks_ = 0;
  hip_check(hipHostMalloc((void**)&host_stage_, blocks * raw_block_bytes_, 0), "TieredKVBlockManager: staging");
  hip_check(hipHostMalloc((void**)&host_pages_, blocks * sizeof(int), 0), "TieredKVBlockManager: staging");
  hip_check(hipMalloc((void**)&dev_stage_, blocks * raw_block_bytes_), "TieredKVBlockManager: staging");
  hip_check(hipMalloc((void**)&dev_pages_, blocks * sizeof(int)), "TieredKVBlockManager: staging");
  stage_blocks_ = blocks;
}

void TieredKVBlockManager::check_cache(const PagedKVCache& cache) const {
  if (!cache.has_device() || cache.num_layers() != layer_count_ || cache.page_size() != page_size_ ||
      cache.n_heads() != n_heads_ || cache.head_dim() != head_dim_ || cache.kv_dtype() != kv_dtype_)
    throw std::invalid_argument("TieredKVBlockManager: cache geometry differs from the manager's");
}

void TieredKVBlockManager::gather_to_host(PagedKVCache& cache, const std::vector<int>& pages) {
  const int n = (int)pages.size();
  if (n == 0) return;
  reserve(pages.size());
  std::memcpy(host_pages_, pages.data(), pages.size() * sizeof(int));
  hip_check(hipMemcpyAsync(dev_pages_, host_pages_, n * sizeof(int), hipMemcpyHostToDevice, stream_), "H2D pages");
  cbis_check(cbis_kv_pages_gather(dev_stage_, cache.k_base(0), layer_count_, cache.max_pages(), (int64_t)page_bytes_,
                                  dev_pages_, n, stream_),
             "kv gather");
  hip_check(hipMemcpyAsync(host_stage_, dev_stage_, n * raw_block_bytes_, hipMemcpyDeviceToHost, stream_),
            "D2H blocks");
  hip_check(hipStreamSynchronize(stream_), "gather sync");
}

void TieredKVBlockManager::scatter_from_host(PagedKVCache& cache, const std::vector<int>& pages) {
  const int n = (int)pages.size();
  if (n == 0) return;
  std::memcpy(host_pages_, pages.data(), pages.size() * sizeof(int));
  hip_check(hipMemcpyAsync(dev_pages_, host_pages_, n * sizeof(int), hipMemcpyHostToDevice, stream_), "H2D pages");
  hip_check(hipMemcpyAsync(dev_stage_, host_stage_, n * raw_block_bytes_, hipMemcpyHostToDevice, stream_),
            "H2D blocks");
  cbis_check(cbis_kv_pages_scatter(cache.k_base(0), dev_stage_, layer_count_, cache.max_pages(), (int64_t)page_bytes_,
                                   dev_pages_, n, stream_),
             "kv scatter");
  hip_check(hipStreamSynchronize(stream_), "scatter sync");
}

void TieredKVBlockManager::calibrate() {
  constexpr int kIters = 20;
  reserve(1);
  std::memset(host_stage_, 0xAB, raw_block_bytes_);
  const auto t0 = std::chrono::steady_clock::now();
  for (int i = 0; i < kIters; ++i) {
    hip_check(hipMemcpyAsync(dev_stage_, host_stage_, raw_block_bytes_, hipMemcpyHostToDevice, stream_), "H2D");
    hip_check(hipMemcpyAsync(host_stage_, dev_stage_, raw_block_bytes_, hipMemcpyDeviceToHost, stream_), "D2H");
  }
  hip_check(hipStreamSynchronize(stream_), "calibrate sync");
  const double pcie_ns = std::chrono::duration<double, std::nano>(std::chrono::steady_clock::now() - t0).count();
  params_.dram_ns_per_byte = pcie_ns / (2.0 * kIters * (double)raw_block_bytes_);
  // Disk: one real block-sized write and read through the store's file.
  const auto t1 = std::chrono::steady_clock::now();
  const NvmeBlockStore::Loc loc = nvme_.write_block(host_stage_, (uint32_t)raw_block_bytes_);
  const auto t2 = std::chrono::steady_clock::now();
  nvme_.read_block(loc, host_stage_);
  const auto t3 = std::chrono::steady_clock::now();
  const double disk_ns = std::chrono::duration<double, std::nano>(t3 - t1).count();
  (void)t2;
  params_.nvme_ns_per_byte = disk_ns / (2.0 * (double)raw_block_bytes_);
}

double TieredKVBlockManager::score(const BlockMeta& m, long now_step, Tier dest) const {
  const double staleness = (double)(now_step - m.last_access_step);
  const double comp = (double)raw_block_bytes_ * params_.expected_compression_ratio;
  const double cost = dest == Tier::DRAM ? params_.dram_fixed_ns + comp * params_.dram_ns_per_byte
                                         : params_.nvme_fixed_ns + comp * params_.nvme_ns_per_byte;
  return params_.alpha_staleness * staleness - params_.beta_restore_cost * cost;
}

void TieredKVBlockManager::admit_gpu_resident(uint64_t block_id, PagedKVCache& cache, int physical_page,
                                              long now_step) {
  check_cache(cache);
  if (physical_page < 0 || physical_page >= cache.max_pages())
    throw std::out_of_range("admit_gpu_resident: physical_page");
  if (meta_.count(block_id)) throw std::runtime_error("admit_gpu_resident: block_id is already managed (a block seen before comes back through restore)");
  if (gpu_resident_count_ >= gpu_capacity_blocks_) evict_one(now_step);
  BlockMeta m;
  m.tier = Tier::GPU;
  m.last_access_step = now_step;
  m.cache = &cache;
  m.physical_page = physical_page;
  meta_.emplace(block_id, std::move(m));
  ++gpu_resident_count_;
}

uint64_t TieredKVBlockManager::evict_one(long now_step) {
  if (gpu_resident_count_ == 0) return UINT64_MAX;
  const Tier dest = dram_resident_count_ < dram_capacity_blocks_ ? Tier::DRAM : Tier::NVME;
  uint64_t best = UINT64_MAX;
  double best_score = -1e300;
  for (const auto& kv : meta_) {  // ascending block id: ties keep the smallest
    if (kv.second.tier != Tier::GPU) continue;
    const double s = score(kv.second, now_step, dest);
    if (best == UINT64_MAX || s > best_score) {
      best = kv.first;
      best_score = s;
    }
  }
  spill(best, dest, now_step);
  return best;
}

void TieredKVBlockManager::spill(uint64_t block_id, Tier dest, long now_step) {
  spill_batch({block_id}, dest, now_step);
}

void TieredKVBlockManager::spill_batch(const std::vector<uint64_t>& ids, Tier dest, long /*now_step*/) {
  if (dest != Tier::DRAM && dest != Tier::NVME) throw std::invalid_argument("spill: destination must be DRAM or NVME");
  std::set<uint64_t> seen;
  for (uint64_t id : ids) {
    auto it = meta_.find(id);
    if (it == meta_.end()) throw std::runtime_error("spill: unknown block_id");
    if (it->second.tier != Tier::GPU) throw std::runtime_error("spill: block is not GPU-resident");
    if (!seen.insert(id).second) throw std::invalid_argument("spill: block listed twice");
  }
  const size_t chunk = std::max<size_t>(1, kStageBytes / raw_block_bytes_);
  for (size_t c0 = 0; c0 < ids.size(); c0 += chunk) {
    const size_t n = std::min(chunk, ids.size() - c0);
    // Read and deflate the chunk's blocks one cache at a time (normally all
    // of them sit in one cache: one gather, one copy).
    std::vector<std::vector<uint8_t>> comp(n);
    std::vector<char> done(n, 0);
    for (size_t i = 0; i < n; ++i) {
      if (done[i]) continue;
      PagedKVCache* cache = meta_.at(ids[c0 + i]).cache;
      std::vector<int> pages;
      std::vector<size_t> members;
      for (size_t j = i; j < n; ++j) {
        const BlockMeta& m = meta_.at(ids[c0 + j]);
        if (!done[j] && m.cache == cache) {
          pages.push_back(m.physical_page);
          members.push_back(j);
          done[j] = 1;
        }
      }
      gather_to_host(*cache, pages);
#pragma omp parallel for schedule(dynamic, 1)
      for (long long k = 0; k < (long long)members.size(); ++k)
        comp[members[k]] = deflate_block(host_stage_ + k * raw_block_bytes_, raw_block_bytes_);
    }
    for (size_t i = 0; i < n; ++i) {
      BlockMeta& m = meta_.at(ids[c0 + i]);
      --gpu_resident_count_;
      m.cache = nullptr;
      m.physical_page = -1;
      m.compressed_bytes = comp[i].size();
      if (dest == Tier::DRAM) {
        m.tier = Tier::DRAM;
        m.dram_bytes = std::move(comp[i]);
        ++dram_resident_count_;
      } else {
        m.tier = Tier::NVME;
        m.nvme_loc = nvme_.write_block(comp[i].data(), (uint32_t)comp[i].size());
      }
    }
  }
}

void TieredKVBlockManager::restore(uint64_t block_id, PagedKVCache& cache, int physical_page, long now_step) {
  restore_batch({block_id}, cache, {physical_page}, now_step);
}

void TieredKVBlockManager::restore_batch(const std::vector<uint64_t>& ids, PagedKVCache& cache,
                                         const std::vector<int>& pages, long now_step) {
  check_cache(cache);
  if (ids.size() != pages.size()) throw std::invalid_argument("restore: ids and pages differ in length");
  std::set<uint64_t> seen_ids;
  std::set<int> seen_pages;
  for (size_t i = 0; i < ids.size(); ++i) {
    if (!meta_.count(ids[i])) throw std::runtime_error("restore: unknown block_id");
    if (pages[i] < 0 || pages[i] >= cache.max_pages()) throw std::out_of_range("restore: physical_page");
    if (!seen_ids.insert(ids[i]).second) throw std::invalid_argument("restore: block listed twice");
    if (!seen_pages.insert(pages[i]).second) throw std::invalid_argument("restore: destination page listed twice");
  }
  // A GPU-resident block of the batch is read from its current page before
  // any page is written.  One restore() after another would read it after
  // the earlier blocks' writes, so a batch in which an earlier block's
  // destination is a later moved block's current page (whose bytes those
  // calls would lose) is refused rather than given other data.
  {
    std::set<int> written;
    for (size_t i = 0; i < ids.size(); ++i) {
      const BlockMeta& m = meta_.at(ids[i]);
      if (m.tier == Tier::GPU && m.cache == &cache && written.count(m.physical_page))
        throw std::invalid_argument("restore: a block's current page is an earlier block's destination");
      written.insert(pages[i]);
    }
  }
  const size_t chunk = std::max<size_t>(1, kStageBytes / raw_block_bytes_);
  for (size_t c0 = 0; c0 < ids.size(); c0 += chunk) {
    const size_t n = std::min(chunk, ids.size() - c0);
    reserve(n);
    // 1. Raw bytes of every block into staging slot i: GPU-resident blocks
    //    (moving to a new page) are read off the device first, then the
    //    colder blocks are inflated in parallel.
    std::vector<std::vector<uint8_t>> moved(n);
    for (size_t i = 0; i < n; ++i) {
      const BlockMeta& m = meta_.at(ids[c0 + i]);
      if (m.tier != Tier::GPU) continue;
      gather_to_host(*m.cache, {m.physical_page});
      moved[i].assign(host_stage_, host_stage_ + raw_block_bytes_);
    }
    std::vector<std::vector<uint8_t>> from_disk(n);
    for (size_t i = 0; i < n; ++i) {
      const BlockMeta& m = meta_.at(ids[c0 + i]);
      if (m.tier == Tier::NVME) from_disk[i] = nvme_.read_block(m.nvme_loc);
    }
#pragma omp parallel for schedule(dynamic, 1)
    for (long long i = 0; i < (long long)n; ++i) {
      const BlockMeta& m = meta_.at(ids[c0 + i]);
      uint8_t* dst = host_stage_ + i * raw_block_bytes_;
      if (m.tier == Tier::DRAM) inflate_block(m.dram_bytes.data(), m.dram_bytes.size(), dst, raw_block_bytes_);
      else if (m.tier == Tier::NVME) inflate_block(from_disk[i].data(), from_disk[i].size(), dst, raw_block_bytes_);
      else std::memcpy(dst, moved[i].data(), raw_block_bytes_);
    }
    // 2. Scatter into the destination pages and do the bookkeeping in order,
    //    as one restore() after another (src/tiered_kv_manager.cpp:173-208):
    //    block i's page is written, then a full GPU tier evicts a victim,
    //    which reads its page.  The writes of blocks [w, i] are issued as one
    //    copy and one scatter right before such an eviction (so a victim
    //    whose page is a later block's destination still spills its own
    //    bytes), the remaining ones at the end of the chunk.  Staging slots
    //    below w are done with: the victim's spill may reuse slot 0.
    size_t w = 0;
    auto flush = [&](size_t upto) {
      if (upto <= w) return;
      // scatter_from_host sends staging slots 0.. : move slots [w, upto) down.
      if (w > 0) std::memmove(host_stage_, host_stage_ + w * raw_block_bytes_, (upto - w) * raw_block_bytes_);
      scatter_from_host(cache, std::vector<int>(pages.begin() + c0 + w, pages.begin() + c0 + upto));
      w = upto;
    };
    for (size_t i = 0; i < n; ++i) {
      BlockMeta& m = meta_.at(ids[c0 + i]);
      const bool was_gpu = m.tier == Tier::GPU;
      if (m.tier == Tier::DRAM) {
        --dram_resident_count_;
        m.dram_bytes.clear();
        m.dram_bytes.shrink_to_fit();
      }
      if (!was_gpu && gpu_resident_count_ >= gpu_capacity_blocks_) {
        flush(i + 1);
        evict_one(now_step);
      }
      m.tier = Tier::GPU;
      m.cache = &cache;
      m.physical_page = pages[c0 + i];
      m.compressed_bytes = 0;
      m.last_access_step = now_step;
      if (!was_gpu) ++gpu_resident_count_;
    }
    flush(n);
  }
}

Tier TieredKVBlockManager::tier_of(uint64_t block_id) const {
  auto it = meta_.find(block_id);
  if (it == meta_.end()) throw std::runtime_error("tier_of: unknown block_id");
  return it->second.tier;
}

void TieredKVBlockManager::touch(uint64_t block_id, long now_step) {
  auto it = meta_.find(block_id);
  if (it != meta_.end()) it->second.last_access_step = now_step;
}

BlockStats TieredKVBlockManager::stats() const {
  BlockStats s;
  for (const auto& kv : meta_) {
    const BlockMeta& m = kv.second;
    s.raw_bytes_total += raw_block_bytes_;
    if (m.tier == Tier::GPU) {
      ++s.gpu_count;
    } else {
      (m.tier == Tier::DRAM ? s.dram_count : s.nvme_count) += 1;
      s.compressed_bytes_total += m.compressed_bytes;
    }
  }
  return s;
}

}  // namespace cbis
