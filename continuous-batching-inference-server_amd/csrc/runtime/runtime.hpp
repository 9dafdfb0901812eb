// Host runtime of the per-step forward, keeping the reference's C++ API:
//   ModelConfig        runtime twin of cfg:: (include/config.hpp:4-25)
//   PagedKVCache       include/paged_kv_cache.hpp:17-51
//   ModelWeights       include/model_weights.hpp:7-25
//   TransformerRunner  include/transformer.hpp:15-34
//   run_continuous     src/bench_batching.cpp:98-179
// Device work goes only through the kernels' C-ABI (cbis_kernels.h).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "cbis_kernels.h"

namespace cbis {

struct ModelConfig {
  int vocab = 1000;
  int d_model = 256;
  int n_heads = 8;
  int head_dim = 32;
  int n_layers = 4;
  int mlp = 1024;
  int max_seq = 32768;
  int page_size = 16;
  int weight_dtype = CBIS_F32;
  int kv_dtype = CBIS_F32;

  int pages_per_seq() const { return max_seq / page_size; }
  // GEMM input activations: fp32 for an fp32 model, bf16 otherwise.
  int act_dtype() const { return weight_dtype == CBIS_F32 ? CBIS_F32 : CBIS_BF16; }
  void validate() const;
};

size_t dtype_size(int dtype);
void hip_check(hipError_t e, const char* what);
void cbis_check(int rc, const char* what);

// ---------------------------------------------------------------------------
// Paged KV cache.  The bookkeeping reproduces src/paged_kv_cache.cpp:5-60
// exactly (free list [P-1 .. 0] so pop_back hands out 0, 1, 2, ...; pages of
// a freed sequence are pushed back in logical order; sequence ids are a
// monotonic counter).  Device pools: one allocation holding, per layer, a K
// pool then a V pool, each [max_pages][page_size][n_heads][head_dim].
// ---------------------------------------------------------------------------
class PagedKVCache {
 public:
  PagedKVCache(int num_layers, int max_pages, int page_size, int n_heads, int head_dim, int kv_dtype = CBIS_F32,
               int pages_per_seq = 2048, bool alloc_device = true);
  ~PagedKVCache();
  PagedKVCache(const PagedKVCache&) = delete;
  PagedKVCache& operator=(const PagedKVCache&) = delete;

  int allocate_sequence();
  void free_sequence(int seq_id);
  bool ensure_capacity(int seq_id, int token_pos);
  void resolve_slot(int seq_id, int token_pos, int* physical_page, int* offset) const;
  std::vector<int> page_table(int seq_id) const;
  const std::vector<int>& pages(int seq_id) const;  // throws std::out_of_range

  void* k_base(int layer) const;
  void* v_base(int layer) const;
  int num_free_pages() const { return (int)free_pages_.size(); }
  int max_pages() const { return max_pages_; }
  int page_size() const { return page_size_; }
  int n_heads() const { return n_heads_; }
  int head_dim() const { return head_dim_; }
  int num_layers() const { return num_layers_; }
  int kv_dtype() const { return kv_dtype_; }
  int pages_per_seq() const { return pages_per_seq_; }
  size_t pool_bytes() const { return layer_bytes_; }
  bool has_device() const { return base_ != nullptr; }
  void fill_normal(uint64_t seed, float std, hipStream_t s);

 private:
  int num_layers_, max_pages_, page_size_, n_heads_, head_dim_, kv_dtype_, pages_per_seq_;
  size_t layer_bytes_ = 0;
  uint8_t* base_ = nullptr;
  std::vector<int> free_pages_;
  std::unordered_map<int, std::vector<int>> seq_pages_;
  int next_seq_id_ = 0;
};

// ---------------------------------------------------------------------------
// Weights.  Linear weights in the config's dtype (fp32 / bf16 / fp8 e4m3 with
// a per-output-channel fp32 scale), Q/K/V fused to one [3d, d] matrix;
// embeddings fp32 (fp32 model) or bf16; biases and LayerNorm fp32.  All
// tensors live in one device arena.
// ---------------------------------------------------------------------------
struct LayerWeights {
  float *ln1_w = nullptr, *ln1_b = nullptr, *ln2_w = nullptr, *ln2_b = nullptr;
  void* wqkv = nullptr;
  float *bqkv = nullptr, *sqkv = nullptr;
  void* wo = nullptr;
  float *bo = nullptr, *so = nullptr;
  void* w1 = nullptr;
  float *b1 = nullptr, *s1 = nullptr;
  void* w2 = nullptr;
  float *b2 = nullptr, *s2 = nullptr;
};

class ModelWeights {
 public:
  ModelConfig cfg;
  void* tok_emb = nullptr;
  void* pos_emb = nullptr;
  std::vector<LayerWeights> layers;
  float *ln_f_w = nullptr, *ln_f_b = nullptr;
  void* lm_head = nullptr;
  float* lm_scale = nullptr;

  // One tensor of the device arena.
  struct Entry {
    std::string name;
    int dtype;
    size_t offset, bytes;
  };

  static std::unique_ptr<ModelWeights> synthetic(const ModelConfig& cfg, uint64_t seed, float std = 0.02f);
  static std::unique_ptr<ModelWeights> load(const std::string& path, const ModelConfig& cfg);
  // Packed checkpoint: the config, the tensor table and the arena image in
  // its stored dtypes (bf16 / fp8 codes + fp32 scales), versioned.
  void save_packed(const std::string& path) const;
  static std::unique_ptr<ModelWeights> load_packed(const std::string& path);
  // The arena's tensor table for a config (no allocation).
  static std::vector<Entry> layout(const ModelConfig& cfg);
  ~ModelWeights();
  void free_all();
  size_t device_bytes() const { return arena_bytes_; }
  int emb_dtype() const { return cfg.weight_dtype == CBIS_F32 ? CBIS_F32 : CBIS_BF16; }
  void* tensor(const std::string& name) const;

 private:
  ModelWeights() = default;
  void plan();
  uint8_t* arena_ = nullptr;
  size_t arena_bytes_ = 0;
  std::vector<Entry> table_;
  std::map<std::string, void*> named_;
};

// ---------------------------------------------------------------------------
// One flattened continuous-batch step (src/transformer.cpp:44-99).
// ---------------------------------------------------------------------------
class TransformerRunner {
 public:
  TransformerRunner(const ModelWeights& weights, PagedKVCache& cache, int max_total_rows);
  ~TransformerRunner();
  TransformerRunner(const TransformerRunner&) = delete;
  TransformerRunner& operator=(const TransformerRunner&) = delete;

  // Returns row-major [rows, vocab] logits (the reference's contract).
  std::vector<float> forward_step(const std::vector<int>& token_ids, const std::vector<int>& positions,
                                  const std::vector<int>& seq_ids);
  // Same step; returns the greedy next token of every row.  lm_head runs
  // fused with the row argmax (cbis_gemm_argmax): the logits are not stored
  // where its kernel reduces them in the epilogue.  last_margins() then holds
  // each row's top-2 margin (max logit minus the runner-up).
  std::vector<int> forward_step_greedy(const std::vector<int>& token_ids, const std::vector<int>& positions,
                                       const std::vector<int>& seq_ids);
  // Pipelined greedy steps (no reference counterpart).  enqueue_greedy
  // queues the step of forward_step_greedy and returns at once with a ticket;
  // wait_greedy(ticket) waits for that step and returns its tokens (and sets
  // last_margins / last_device_ms / last_host_ms).  token_src (empty, or one
  // entry per row) lets a row take its input token from the device: row i
  // with token_src[i] >= 0 uses the greedy token of row token_src[i] of the
  // greedy step enqueued just before this one (token_ids[i] is then
  // ignored), so a decode loop can queue step t + 1 before step t's tokens
  // reach the host.  At most two steps are outstanding: a step's buffers are
  // reused two steps later, and enqueue_greedy throws std::logic_error if
  // that step has not been waited for.
  int64_t enqueue_greedy(const std::vector<int>& token_ids, const std::vector<int>& positions,
                         const std::vector<int>& seq_ids, const std::vector<int>& token_src);
  std::vector<int> wait_greedy(int64_t ticket);
  // Empty after a plain forward_step: margins belong to greedy steps only.
  const std::vector<float>& last_margins() const { return margins_; }
  // Device time of the last step's forward (embedding, which also stages
  // the step's metadata, through lm_head and the argmax, between two events
  // on the runner's stream), in ms.
  float last_device_ms() const { return last_device_ms_; }
  // Host wall time of the last greedy step's phases, in ms: {host
  // preparation of the metadata, the forward's launch, the wait for its
  // results}.
  const double* last_host_ms() const { return host_ms_; }
  // Device logits of the last forward_step (not of a greedy step).
  const float* logits_device() const { return d_logits_; }
  hipStream_t stream() const { return stream_; }
  void set_graphs(bool on) { use_graphs_ = on; }
  // Small all-decode steps run each layer's attention and out-projection as
  // one launch (cbis_paged_attention_proj) when the model's widths allow it;
  // off: two launches, as every other step.
  void set_fused_decode(bool on) { fuse_decode_ = on; }
  // How the last step ran: {rows, decode rows, prefill tiles, sequences,
  // block-table width, max_kv bound, decode split_tokens (1 << 30: one pass
  // per row; 0: the attention library's own split)}.
  std::vector<int> last_plan() const { return signature(); }

 private:
  // One step's own buffers; consecutive steps alternate between two of them,
  // so a step can be prepared and queued while the one before it runs.
  // A step's host<->device traffic goes through pinned, coherent host memory
  // that the kernels read and write themselves: no copy commands between
  // two steps' kernels on the stream.
  struct StepBuf {
    uint8_t* h_meta = nullptr;   // the step's metadata, written by the host
    uint8_t* hd_meta = nullptr;  // h_meta's device address
    uint8_t* d_meta = nullptr;   // its device copy (staged by the embed launch)
    size_t cap = 0;
    int* h_next = nullptr;  // [M] tokens then [M] margins (fp32) of a greedy step, written by the argmax launch
    int* d_next = nullptr;  // h_next's device address (the next step's embed reads tokens there)
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;  // around the forward
    int64_t ticket = -1;    // the greedy step these buffers hold, -1 if none
    bool pending = false;   // enqueued, not yet waited for
    int M = 0;
    double host_ms[2] = {0, 0};
  };
  void prepare(int b, const int* tok, const int* pos, const int* seq, const int* src, int M);
  void enqueue_forward(int b, bool greedy, bool from_prev);
  void run_step(int b, bool greedy, bool from_prev);
  void timed_step(int b, bool greedy, bool from_prev);

  const ModelWeights& w_;
  PagedKVCache& cache_;
  ModelConfig cfg_;
  int max_rows_;
  hipStream_t stream_ = nullptr;
  float last_device_ms_ = 0.f;
  double host_ms_[3] = {0, 0, 0};
  bool use_graphs_ = true;
  bool fuse_decode_ = true;
  bool attn_proj_ok_ = false;  // the model's widths and dtypes fit cbis_paged_attention_proj

  StepBuf bufs_[2];
  int next_buf_ = 0;          // the buffers the next step takes
  int64_t tickets_ = 0;       // greedy steps enqueued so far
  int prev_greedy_rows_ = -1; // rows of the step just before, if it was greedy (its tokens can be sources)

  // activations
  float* d_x_ = nullptr;
  void* d_xn_ = nullptr;
  float* d_q_ = nullptr;
  void* d_attn_ = nullptr;
  void* d_h_ = nullptr;
  float* d_logits_ = nullptr;
  void* d_amax_ws_ = nullptr;  // cbis_gemm_argmax partials
  size_t amax_ws_bytes_ = 0;
  std::vector<float> margins_;
  void* d_ws_ = nullptr;
  size_t ws_bytes_ = 0;
  void* d_gemm_ws_ = nullptr;
  size_t gemm_ws_bytes_ = 0;

  // current step
  int M_ = 0;
  int n_decode_ = 0, n_tiles_ = 0, n_seqs_ = 0, bt_width_ = 0, max_kv_ = 0, split_tokens_ = 0;
  int fused_proj_ = 0;  // this step runs attention + out-projection as one launch per layer
  size_t meta_bytes_ = 0;
  const uint8_t* stage_src_ = nullptr;  // the step's metadata in host memory (device address) ...
  uint8_t* stage_dst_ = nullptr;        // ... and its device copy, which the step's embed launch fills
  // Read by the embed launch straight from host memory:
  const int *hd_tok_ = nullptr, *hd_pos_ = nullptr, *hd_src_ = nullptr;
  // Read from the device copy by every later launch:
  int *d_pos_ = nullptr, *d_wpage_ = nullptr, *d_woff_ = nullptr, *d_rowbt_ = nullptr, *d_drows_ = nullptr,
      *d_tiles_ = nullptr, *d_bt_ = nullptr;

  // graph cache: one executable graph per step shape signature
  struct GraphEntry {
    hipGraphExec_t exec = nullptr;
  };
  std::map<std::vector<int>, GraphEntry> graphs_;
  std::vector<int> signature() const;
};

// ---------------------------------------------------------------------------
// Three-tier KV block manager (include/tiered_kv_manager.hpp,
// include/block_storage.hpp): a block is one physical page's K and V slots in
// every layer; GPU-resident blocks live in a PagedKVCache, colder blocks are
// deflated (zlib, fastest level) into host DRAM or an append-only file.
// Same API and eviction policy as the reference; batch spill / restore move
// every block of a call with one gather / scatter launch and one host copy.
// ---------------------------------------------------------------------------
enum class Tier { GPU = 0, DRAM = 1, NVME = 2 };

struct EvictionParams {
  double alpha_staleness = 1.0;             // weight on steps since last access
  double beta_restore_cost = 1.0;           // weight on the estimated restore cost (ns)
  double expected_compression_ratio = 0.5;  // compressed / raw
  double dram_fixed_ns = 2000.0;
  double dram_ns_per_byte = 0.05;           // calibrate() measures H2D + D2H
  double nvme_fixed_ns = 50000.0;
  double nvme_ns_per_byte = 0.2;            // calibrate() measures file write + read
};

struct BlockStats {
  size_t gpu_count = 0, dram_count = 0, nvme_count = 0;
  size_t raw_bytes_total = 0;
  size_t compressed_bytes_total = 0;  // DRAM + NVMe blocks
};

std::vector<uint8_t> deflate_block(const void* data, size_t len);
void inflate_block(const uint8_t* comp, size_t comp_len, void* out, size_t out_len);

// Append-only single-file blob store (pwrite / pread on one descriptor).
class NvmeBlockStore {
 public:
  struct Loc {
    uint64_t offset = 0;
    uint32_t length = 0;
  };
  explicit NvmeBlockStore(const std::string& path);
  ~NvmeBlockStore();
  NvmeBlockStore(const NvmeBlockStore&) = delete;
  NvmeBlockStore& operator=(const NvmeBlockStore&) = delete;
  Loc write_block(const uint8_t* data, uint32_t length);
  void read_block(Loc loc, uint8_t* out) const;
  std::vector<uint8_t> read_block(Loc loc) const;
  uint64_t bytes_written() const { return next_; }
  const std::string& path() const { return path_; }

 private:
  std::string path_;
  int fd_ = -1;
  uint64_t next_ = 0;
};

class TieredKVBlockManager {
 public:
  TieredKVBlockManager(int layer_count, int page_size, int n_heads, int head_dim, const std::string& nvme_scratch_path,
                       size_t gpu_capacity_blocks, size_t dram_capacity_blocks, EvictionParams params = {},
                       int kv_dtype = CBIS_F32);
  ~TieredKVBlockManager();
  TieredKVBlockManager(const TieredKVBlockManager&) = delete;
  TieredKVBlockManager& operator=(const TieredKVBlockManager&) = delete;

  size_t raw_block_bytes() const { return raw_block_bytes_; }
  const EvictionParams& params() const { return params_; }
  void calibrate();

  void admit_gpu_resident(uint64_t block_id, PagedKVCache& cache, int physical_page, long now_step);
  uint64_t evict_one(long now_step);  // UINT64_MAX when no block is GPU-resident
  void spill(uint64_t block_id, Tier dest, long now_step);
  void restore(uint64_t block_id, PagedKVCache& cache, int physical_page, long now_step);
  // Batches: the blocks' bytes move with one gather (spill) or scatter
  // (restore) launch and one host copy; per-block bookkeeping, and the
  // evictions a restore triggers, happen in the order of `ids`.
  void spill_batch(const std::vector<uint64_t>& ids, Tier dest, long now_step);
  void restore_batch(const std::vector<uint64_t>& ids, PagedKVCache& cache, const std::vector<int>& pages,
                     long now_step);

  Tier tier_of(uint64_t block_id) const;
  void touch(uint64_t block_id, long now_step);
  bool known(uint64_t block_id) const { return meta_.count(block_id) != 0; }
  BlockStats stats() const;

 private:
  struct BlockMeta {
    Tier tier = Tier::GPU;
    long last_access_step = 0;
    size_t compressed_bytes = 0;
    PagedKVCache* cache = nullptr;
    int physical_page = -1;
    std::vector<uint8_t> dram_bytes;
    NvmeBlockStore::Loc nvme_loc{};
  };
  double score(const BlockMeta& m, long now_step, Tier dest) const;
  void check_cache(const PagedKVCache& cache) const;
  // Device <-> pinned host: every listed page of `cache` into / out of
  // host_stage_ (block i at i * raw_block_bytes_).
  void gather_to_host(PagedKVCache& cache, const std::vector<int>& pages);
  void scatter_from_host(PagedKVCache& cache, const std::vector<int>& pages);
  void reserve(size_t blocks);

  int layer_count_, page_size_, n_heads_, head_dim_, kv_dtype_;
  size_t page_bytes_, raw_block_bytes_;
  size_t gpu_capacity_blocks_, dram_capacity_blocks_;
  EvictionParams params_;
  NvmeBlockStore nvme_;
  hipStream_t stream_ = nullptr;
  size_t stage_blocks_ = 0;
  uint8_t* host_stage_ = nullptr;  // pinned
  uint8_t* dev_stage_ = nullptr;
  int* host_pages_ = nullptr;      // pinned
  int* dev_pages_ = nullptr;
  std::map<uint64_t, BlockMeta> meta_;
  size_t gpu_resident_count_ = 0;
  size_t dram_resident_count_ = 0;
};

// ---------------------------------------------------------------------------
// Continuous batching (src/bench_batching.cpp:98-179).
// ---------------------------------------------------------------------------
struct Request {
  std::vector<int> prompt;
  int decode_len = 0;
  // Admitted once this many ms have passed since the run began
  // (src/bench_batching.cpp:110-121); requests are given in arrival order.
  double arrival_ms = 0.0;
};

struct ContinuousResult {
  std::vector<std::vector<int>> tokens;  // generated tokens per request
  std::vector<double> step_ms;           // wall time of each forward step
  std::vector<double> finish_ms;         // per request: ms since the run began when its last token came back
};

// Scheduling knobs.  prefill_chunk = 0 and step_token_budget = 0 is the
// reference's policy (a slot's whole prompt in the step after admission).
struct ScheduleOptions {
  int max_slots = 16;
  int prefill_chunk = 0;      // prompt rows a slot contributes per step; 0 = the whole prompt
  int step_token_budget = 0;  // cap on prompt rows per step (decode rows always run); 0 = none
  // The run's clock in ms since it began and the wait of an idle scheduler
  // for the next arrival; unset: steady_clock and a sleep
  // (src/bench_batching.cpp:153-158).  The host-only dry run sets a virtual
  // clock.
  std::function<double()> clock_ms;
  std::function<void(double)> wait_ms;
};

// Rows of one scheduled step, in the order they were handed to the step.
struct StepRows {
  std::vector<int> tok, pos, sid;
};

// One forward step: rows (token, position, sequence) -> greedy next token
// of every row.
using StepFn = std::function<std::vector<int>(const std::vector<int>&, const std::vector<int>&,
                                              const std::vector<int>&)>;

ContinuousResult run_continuous(const StepFn& step, PagedKVCache& cache, const std::vector<Request>& reqs,
                                const ScheduleOptions& opt, std::vector<StepRows>* trace = nullptr);
ContinuousResult run_continuous(TransformerRunner& runner, PagedKVCache& cache, const std::vector<Request>& reqs,
                                const ScheduleOptions& opt);
ContinuousResult run_continuous(TransformerRunner& runner, PagedKVCache& cache, const std::vector<Request>& reqs,
                                int max_slots);

// A forward step queued without waiting for it (no reference counterpart):
// enqueue(tok, pos, sid, src) returns a ticket; a row with src[i] >= 0 takes
// as its input token the greedy token of row src[i] of the step enqueued
// just before (tok[i] is not used); wait(ticket) returns the greedy next
// token of every row of that step.
struct PipelinedStep {
  std::function<int64_t(const std::vector<int>&, const std::vector<int>&, const std::vector<int>&,
                        const std::vector<int>&)>
      enqueue;
  std::function<std::vector<int>(int64_t)> wait;
};

// run_continuous with one step in flight: step t + 1 is built and queued
// before step t's tokens come back (its decode rows name the rows of step t
// that produce their tokens), then step t's tokens are collected.  The rows,
// tokens and page order are run_continuous's for the same admissions; a
// request whose arrival falls while step t runs is seen when step t + 2 is
// built, one step later than there.  step_ms: per step, host wall time from
// the later of its enqueue and the previous collection to its collection;
// finish_ms: when the host collected the request's last token.  In the
// trace, rows that take their token from the previous step hold tok -1.
ContinuousResult run_continuous_pipelined(const PipelinedStep& step, PagedKVCache& cache,
                                          const std::vector<Request>& reqs, const ScheduleOptions& opt,
                                          std::vector<StepRows>* trace = nullptr);
ContinuousResult run_continuous_pipelined(TransformerRunner& runner, PagedKVCache& cache,
                                          const std::vector<Request>& reqs, const ScheduleOptions& opt);

}  // namespace cbis
