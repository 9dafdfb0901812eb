// extern "C" wrappers of the C++ runtime (include/cbis_runtime.h).  C++
// exceptions stop here: they become negative return codes (or NULL) with the
// message in cbis_runtime_last_error().
#include <cstring>
#include <map>

#include "cbis_runtime.h"
#include "runtime.hpp"

using namespace cbis;

struct cbis_cache {
  std::unique_ptr<PagedKVCache> impl;
};
struct cbis_weights {
  std::unique_ptr<ModelWeights> impl;
};
struct cbis_runner {
  std::unique_ptr<TransformerRunner> impl;
};
struct cbis_tiered {
  std::unique_ptr<TieredKVBlockManager> impl;
};

namespace {
thread_local std::string g_err;

template <typename F>
int guard(F&& f) {
  try {
    return f();
  } catch (const std::out_of_range& e) {
    g_err = std::string("out_of_range: ") + e.what();
    return -2;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}

template <typename T, typename F>
T* guard_ptr(F&& f) {
  try {
    return f();
  } catch (const std::exception& e) {
    g_err = e.what();
    return nullptr;
  }
}

ModelConfig to_cfg(const cbis_model_config* c) {
  if (!c) throw std::invalid_argument("null config");
  ModelConfig m;
  m.vocab = c->vocab; m.d_model = c->d_model; m.n_heads = c->n_heads; m.head_dim = c->head_dim;
  m.n_layers = c->n_layers; m.mlp = c->mlp; m.max_seq = c->max_seq; m.page_size = c->page_size;
  m.weight_dtype = c->weight_dtype; m.kv_dtype = c->kv_dtype;
  m.validate();
  return m;
}
}  // namespace

extern "C" {

const char* cbis_runtime_last_error(void) { return g_err.c_str(); }

void cbis_default_config(cbis_model_config* c) {
  ModelConfig m;
  c->vocab = m.vocab; c->d_model = m.d_model; c->n_heads = m.n_heads; c->head_dim = m.head_dim;
  c->n_layers = m.n_layers; c->mlp = m.mlp; c->max_seq = m.max_seq; c->page_size = m.page_size;
  c->weight_dtype = m.weight_dtype; c->kv_dtype = m.kv_dtype;
}

cbis_cache* cbis_cache_create(int num_layers, int max_pages, int page_size, int n_heads, int head_dim, int kv_dtype,
                              int pages_per_seq, int alloc_device) {
  return guard_ptr<cbis_cache>([&] {
    auto* c = new cbis_cache();
    try {
      c->impl.reset(new PagedKVCache(num_layers, max_pages, page_size, n_heads, head_dim, kv_dtype, pages_per_seq,
                                     alloc_device != 0));
    } catch (...) {
      delete c;
      throw;
    }
    return c;
  });
}

void cbis_cache_destroy(cbis_cache* c) { delete c; }

int cbis_cache_allocate_sequence(cbis_cache* c) { return guard([&] { return c->impl->allocate_sequence(); }); }

void cbis_cache_free_sequence(cbis_cache* c, int seq_id) { c->impl->free_sequence(seq_id); }

int cbis_cache_ensure_capacity(cbis_cache* c, int seq_id, int token_pos) {
  return guard([&] { return c->impl->ensure_capacity(seq_id, token_pos) ? 1 : 0; });
}

int cbis_cache_resolve_slot(cbis_cache* c, int seq_id, int token_pos, int* page, int* offset) {
  return guard([&] {
    c->impl->resolve_slot(seq_id, token_pos, page, offset);
    return 0;
  });
}

int cbis_cache_page_table(cbis_cache* c, int seq_id, int* out, int capacity) {
  return guard([&] {
    const std::vector<int> t = c->impl->page_table(seq_id);
    const int n = std::min<int>((int)t.size(), capacity);
    std::memcpy(out, t.data(), (size_t)n * 4);
    return n;
  });
}

int cbis_cache_seq_pages(cbis_cache* c, int seq_id, int* out, int capacity) {
  return guard([&] {
    const auto& p = c->impl->pages(seq_id);
    const int n = std::min<int>((int)p.size(), capacity);
    if (n > 0) std::memcpy(out, p.data(), (size_t)n * 4);
    return (int)p.size();
  });
}

int cbis_cache_num_free_pages(cbis_cache* c) { return c->impl->num_free_pages(); }
int cbis_cache_max_pages(cbis_cache* c) { return c->impl->max_pages(); }
int cbis_cache_page_size(cbis_cache* c) { return c->impl->page_size(); }

void* cbis_cache_k_base(cbis_cache* c, int layer) {
  return guard_ptr<void>([&] { return c->impl->k_base(layer); });
}

void* cbis_cache_v_base(cbis_cache* c, int layer) {
  return guard_ptr<void>([&] { return c->impl->v_base(layer); });
}

int cbis_cache_fill_normal(cbis_cache* c, uint64_t seed, float std) {
  return guard([&] {
    c->impl->fill_normal(seed, std, nullptr);
    return 0;
  });
}

cbis_weights* cbis_weights_synthetic(const cbis_model_config* cfg, uint64_t seed, float std) {
  return guard_ptr<cbis_weights>([&] {
    auto* w = new cbis_weights();
    try {
      w->impl = ModelWeights::synthetic(to_cfg(cfg), seed, std);
    } catch (...) {
      delete w;
      throw;
    }
    return w;
  });
}

cbis_weights* cbis_weights_load(const char* path, const cbis_model_config* cfg) {
  return guard_ptr<cbis_weights>([&] {
    auto* w = new cbis_weights();
    try {
      w->impl = ModelWeights::load(path ? path : "", to_cfg(cfg));
    } catch (...) {
      delete w;
      throw;
    }
    return w;
  });
}

int cbis_weights_save_packed(const cbis_weights* w, const char* path) {
  return guard([&] {
    w->impl->save_packed(path ? path : "");
    return 0;
  });
}

cbis_weights* cbis_weights_load_packed(const char* path, cbis_model_config* cfg_out) {
  return guard_ptr<cbis_weights>([&] {
    auto* w = new cbis_weights();
    try {
      w->impl = ModelWeights::load_packed(path ? path : "");
    } catch (...) {
      delete w;
      throw;
    }
    if (cfg_out) {
      const ModelConfig& c = w->impl->cfg;
      *cfg_out = {c.vocab, c.d_model, c.n_heads, c.head_dim, c.n_layers, c.mlp, c.max_seq, c.page_size,
                  c.weight_dtype, c.kv_dtype};
    }
    return w;
  });
}

void cbis_weights_destroy(cbis_weights* w) { delete w; }

size_t cbis_weights_device_bytes(const cbis_weights* w) { return w->impl->device_bytes(); }

void* cbis_weights_tensor(const cbis_weights* w, const char* name) {
  return guard_ptr<void>([&] { return w->impl->tensor(name ? name : ""); });
}

cbis_runner* cbis_runner_create(const cbis_weights* w, cbis_cache* c, int max_total_rows) {
  return guard_ptr<cbis_runner>([&] {
    auto* r = new cbis_runner();
    try {
      r->impl.reset(new TransformerRunner(*w->impl, *c->impl, max_total_rows));
    } catch (...) {
      delete r;
      throw;
    }
    return r;
  });
}

void cbis_runner_destroy(cbis_runner* r) { delete r; }

int cbis_runner_forward_step(cbis_runner* r, int n, const int* token_ids, const int* positions, const int* seq_ids,
                             float* logits_out) {
  return guard([&] {
    if (n < 0) throw std::invalid_argument("forward_step: n < 0");
    std::vector<int> t(token_ids, token_ids + n), p(positions, positions + n), s(seq_ids, seq_ids + n);
    const std::vector<float> lg = r->impl->forward_step(t, p, s);
    if (!lg.empty()) std::memcpy(logits_out, lg.data(), lg.size() * 4);
    return 0;
  });
}

int cbis_runner_forward_step_greedy(cbis_runner* r, int n, const int* token_ids, const int* positions,
                                    const int* seq_ids, int* next_tokens) {
  return guard([&] {
    if (n < 0) throw std::invalid_argument("forward_step_greedy: n < 0");
    std::vector<int> t(token_ids, token_ids + n), p(positions, positions + n), s(seq_ids, seq_ids + n);
    const std::vector<int> nx = r->impl->forward_step_greedy(t, p, s);
    if (!nx.empty()) std::memcpy(next_tokens, nx.data(), nx.size() * 4);
    return 0;
  });
}

int cbis_runner_enqueue_greedy(cbis_runner* r, int n, const int* token_ids, const int* positions, const int* seq_ids,
                               const int* token_src, int64_t* ticket) {
  return guard([&] {
    if (n <= 0) throw std::invalid_argument("enqueue_greedy: n must be > 0");
    if (!ticket) throw std::invalid_argument("enqueue_greedy: null ticket");
    std::vector<int> t(token_ids, token_ids + n), p(positions, positions + n), s(seq_ids, seq_ids + n);
    std::vector<int> src;
    if (token_src) src.assign(token_src, token_src + n);
    *ticket = r->impl->enqueue_greedy(t, p, s, src);
    return 0;
  });
}

int cbis_runner_wait_greedy(cbis_runner* r, int64_t ticket, int* next_tokens, int capacity) {
  return guard([&] {
    const std::vector<int> nx = r->impl->wait_greedy(ticket);
    for (int i = 0; i < capacity && i < (int)nx.size(); ++i) next_tokens[i] = nx[i];
    return (int)nx.size();
  });
}

const float* cbis_runner_logits_device(cbis_runner* r) { return r->impl->logits_device(); }

float cbis_runner_last_device_ms(const cbis_runner* r) { return r->impl->last_device_ms(); }

void cbis_runner_last_host_ms(const cbis_runner* r, double out[3]) {
  for (int i = 0; i < 3; ++i) out[i] = r->impl->last_host_ms()[i];
}

void* cbis_runner_stream(cbis_runner* r) { return (void*)r->impl->stream(); }

void cbis_runner_set_graphs(cbis_runner* r, int enable) { r->impl->set_graphs(enable != 0); }

void cbis_runner_set_fused_decode(cbis_runner* r, int enable) { r->impl->set_fused_decode(enable != 0); }

int cbis_runner_last_margins(const cbis_runner* r, float* out, int capacity) {
  return guard([&] {
    const std::vector<float>& m = r->impl->last_margins();
    for (int i = 0; i < capacity && i < (int)m.size(); ++i) out[i] = m[i];
    return (int)m.size();
  });
}

int cbis_runner_last_plan(const cbis_runner* r, int* out, int capacity) {
  return guard([&] {
    const std::vector<int> p = r->impl->last_plan();
    for (int i = 0; i < capacity && i < (int)p.size(); ++i) out[i] = p[i];
    return (int)p.size();
  });
}

namespace {
std::vector<Request> make_requests(int n_requests, const int* prompt_lens, const int* prompt_tokens,
                                   const int* decode_lens) {
  if (n_requests < 0) throw std::invalid_argument("run_continuous: n_requests < 0");
  std::vector<Request> reqs(n_requests);
  size_t off = 0;
  for (int i = 0; i < n_requests; ++i) {
    if (prompt_lens[i] < 0) throw std::invalid_argument("run_continuous: negative prompt length");
    reqs[i].prompt.assign(prompt_tokens + off, prompt_tokens + off + prompt_lens[i]);
    off += prompt_lens[i];
    reqs[i].decode_len = decode_lens[i];
  }
  return reqs;
}

void set_arrivals(std::vector<Request>& reqs, const double* arrival_ms) {
  if (arrival_ms)
    for (size_t i = 0; i < reqs.size(); ++i) reqs[i].arrival_ms = arrival_ms[i];
}

void copy_tokens(const ContinuousResult& res, int n_requests, const int* decode_lens, int* out_tokens) {
  size_t o = 0;
  for (int i = 0; i < n_requests; ++i)
    for (int j = 0; j < decode_lens[i]; ++j) out_tokens[o++] = j < (int)res.tokens[i].size() ? res.tokens[i][j] : -1;
}

ScheduleOptions options(int max_slots, int prefill_chunk, int step_token_budget) {
  ScheduleOptions opt;
  opt.max_slots = max_slots;
  opt.prefill_chunk = prefill_chunk;
  opt.step_token_budget = step_token_budget;
  return opt;
}
}  // namespace

int cbis_run_continuous(cbis_runner* r, cbis_cache* c, int n_requests, const int* prompt_lens,
                        const int* prompt_tokens, const int* decode_lens, int max_slots, int* out_tokens,
                        double* step_ms, int max_steps) {
  return cbis_run_continuous_chunked(r, c, n_requests, prompt_lens, prompt_tokens, decode_lens, max_slots, 0, 0,
                                     out_tokens, step_ms, max_steps);
}

int cbis_run_continuous_chunked(cbis_runner* r, cbis_cache* c, int n_requests, const int* prompt_lens,
                                const int* prompt_tokens, const int* decode_lens, int max_slots, int prefill_chunk,
                                int step_token_budget, int* out_tokens, double* step_ms, int max_steps) {
  return cbis_run_continuous_timed(r, c, n_requests, prompt_lens, prompt_tokens, decode_lens, nullptr, max_slots,
                                   prefill_chunk, step_token_budget, out_tokens, step_ms, max_steps, nullptr);
}

int cbis_run_continuous_timed(cbis_runner* r, cbis_cache* c, int n_requests, const int* prompt_lens,
                              const int* prompt_tokens, const int* decode_lens, const double* arrival_ms,
                              int max_slots, int prefill_chunk, int step_token_budget, int* out_tokens,
                              double* step_ms, int max_steps, double* finish_ms) {
  return guard([&] {
    std::vector<Request> reqs = make_requests(n_requests, prompt_lens, prompt_tokens, decode_lens);
    set_arrivals(reqs, arrival_ms);
    const ContinuousResult res =
        run_continuous(*r->impl, *c->impl, reqs, options(max_slots, prefill_chunk, step_token_budget));
    copy_tokens(res, n_requests, decode_lens, out_tokens);
    if (step_ms)
      for (int i = 0; i < (int)res.step_ms.size() && i < max_steps; ++i) step_ms[i] = res.step_ms[i];
    if (finish_ms)
      for (int i = 0; i < n_requests; ++i) finish_ms[i] = res.finish_ms[i];
    return (int)res.step_ms.size();
  });
}

int cbis_schedule_dry_run(cbis_cache* c, int n_requests, const int* prompt_lens, const int* prompt_tokens,
                          const int* decode_lens, int max_slots, int prefill_chunk, int step_token_budget, int vocab,
                          int* out_tokens, int* step_rows, int max_steps, int* row_tok, int* row_pos, int* row_sid,
                          int max_rows) {
  return cbis_schedule_dry_run_timed(c, n_requests, prompt_lens, prompt_tokens, decode_lens, nullptr, 1.0, max_slots,
                                     prefill_chunk, step_token_budget, vocab, out_tokens, step_rows, max_steps, row_tok,
                                     row_pos, row_sid, max_rows, nullptr);
}

namespace {
// The dry run's stand-in for a forward step: row (tok, pos, seq) -> (31 tok +
// 7 pos + 13 seq + 1) mod vocab.
int stand_in(int t, int p, int s, int vocab) {
  return (int)(((uint32_t)t * 31u + (uint32_t)p * 7u + (uint32_t)s * 13u + 1u) % (uint32_t)vocab);
}

int dry_run(cbis_cache* c, int n_requests, const int* prompt_lens, const int* prompt_tokens, const int* decode_lens,
            const double* arrival_ms, double step_time_ms, int max_slots, int prefill_chunk, int step_token_budget,
            int vocab, int* out_tokens, int* step_rows, int max_steps, int* row_tok, int* row_pos, int* row_sid,
            int max_rows, double* finish_ms, bool pipelined) {
  return guard([&] {
    if (vocab <= 0) throw std::invalid_argument("schedule_dry_run: vocab must be > 0");
    if (!(step_time_ms >= 0.0)) throw std::invalid_argument("schedule_dry_run: step_time_ms must be >= 0");
    std::vector<Request> reqs = make_requests(n_requests, prompt_lens, prompt_tokens, decode_lens);
    set_arrivals(reqs, arrival_ms);
    // Virtual clock: a step takes step_time_ms, an idle wait jumps to the arrival.
    double clock = 0.0;
    const StepFn step = [&](const std::vector<int>& t, const std::vector<int>& p, const std::vector<int>& s) {
      std::vector<int> next(t.size());
      for (size_t i = 0; i < t.size(); ++i) next[i] = stand_in(t[i], p[i], s[i], vocab);
      clock += step_time_ms;
      return next;
    };
    // Pipelined: the stand-in "device" keeps each step's outputs, resolves a
    // row's token source against the step queued before it and runs the step
    // (on the virtual clock) when it is queued.  The trace reports the
    // resolved tokens, so both modes' traces read alike.
    std::map<int64_t, std::vector<int>> outputs;
    std::vector<std::vector<int>> resolved;
    int64_t queued = 0;
    PipelinedStep pstep;
    pstep.enqueue = [&](const std::vector<int>& t, const std::vector<int>& p, const std::vector<int>& s,
                        const std::vector<int>& src) {
      std::vector<int> tok = t;
      for (size_t i = 0; i < src.size(); ++i) {
        if (src[i] < 0) continue;
        const auto prev = outputs.find(queued - 1);
        if (prev == outputs.end() || src[i] >= (int)prev->second.size())
          throw std::logic_error("schedule_dry_run: token source past the previous step");
        tok[i] = prev->second[src[i]];
      }
      outputs[queued] = step(tok, p, s);
      resolved.push_back(tok);
      outputs.erase(queued - 2);  // a source is always the step just before
      return queued++;
    };
    pstep.wait = [&](int64_t ticket) { return outputs.at(ticket); };
    std::vector<StepRows> trace;
    ScheduleOptions opt = options(max_slots, prefill_chunk, step_token_budget);
    opt.clock_ms = [&]() { return clock; };
    opt.wait_ms = [&](double ms) { clock += ms; };
    const ContinuousResult res = pipelined ? run_continuous_pipelined(pstep, *c->impl, reqs, opt, &trace)
                                           : run_continuous(step, *c->impl, reqs, opt, &trace);
    if (pipelined)
      for (size_t k = 0; k < trace.size(); ++k) trace[k].tok = resolved.at(k);
    copy_tokens(res, n_requests, decode_lens, out_tokens);
    if (finish_ms)
      for (int i = 0; i < n_requests; ++i) finish_ms[i] = res.finish_ms[i];
    int row = 0;
    for (size_t k = 0; k < trace.size(); ++k) {
      const int n = (int)trace[k].tok.size();
      if ((int)k < max_steps) step_rows[k] = n;
      for (int i = 0; i < n; ++i, ++row) {
        if (row < max_rows) {
          row_tok[row] = trace[k].tok[i];
          row_pos[row] = trace[k].pos[i];
          row_sid[row] = trace[k].sid[i];
        }
      }
    }
    return (int)trace.size();
  });
}
}  // namespace

int cbis_schedule_dry_run_timed(cbis_cache* c, int n_requests, const int* prompt_lens, const int* prompt_tokens,
                                const int* decode_lens, const double* arrival_ms, double step_time_ms, int max_slots,
                                int prefill_chunk, int step_token_budget, int vocab, int* out_tokens, int* step_rows,
                                int max_steps, int* row_tok, int* row_pos, int* row_sid, int max_rows,
                                double* finish_ms) {
  return dry_run(c, n_requests, prompt_lens, prompt_tokens, decode_lens, arrival_ms, step_time_ms, max_slots,
                 prefill_chunk, step_token_budget, vocab, out_tokens, step_rows, max_steps, row_tok, row_pos, row_sid,
                 max_rows, finish_ms, false);
}

int cbis_schedule_dry_run_pipelined(cbis_cache* c, int n_requests, const int* prompt_lens, const int* prompt_tokens,
                                    const int* decode_lens, const double* arrival_ms, double step_time_ms,
                                    int max_slots, int prefill_chunk, int step_token_budget, int vocab,
                                    int* out_tokens, int* step_rows, int max_steps, int* row_tok, int* row_pos,
                                    int* row_sid, int max_rows, double* finish_ms) {
  return dry_run(c, n_requests, prompt_lens, prompt_tokens, decode_lens, arrival_ms, step_time_ms, max_slots,
                 prefill_chunk, step_token_budget, vocab, out_tokens, step_rows, max_steps, row_tok, row_pos, row_sid,
                 max_rows, finish_ms, true);
}

int cbis_run_continuous_pipelined(cbis_runner* r, cbis_cache* c, int n_requests, const int* prompt_lens,
                                  const int* prompt_tokens, const int* decode_lens, const double* arrival_ms,
                                  int max_slots, int prefill_chunk, int step_token_budget, int* out_tokens,
                                  double* step_ms, int max_steps, double* finish_ms) {
  return guard([&] {
    std::vector<Request> reqs = make_requests(n_requests, prompt_lens, prompt_tokens, decode_lens);
    set_arrivals(reqs, arrival_ms);
    const ContinuousResult res =
        run_continuous_pipelined(*r->impl, *c->impl, reqs, options(max_slots, prefill_chunk, step_token_budget));
    copy_tokens(res, n_requests, decode_lens, out_tokens);
    if (step_ms)
      for (int i = 0; i < (int)res.step_ms.size() && i < max_steps; ++i) step_ms[i] = res.step_ms[i];
    if (finish_ms)
      for (int i = 0; i < n_requests; ++i) finish_ms[i] = res.finish_ms[i];
    return (int)res.step_ms.size();
  });
}

namespace {
Tier to_tier(int t) {
  if (t < 0 || t > 2) throw std::invalid_argument("tier must be 0 (GPU), 1 (DRAM) or 2 (NVME)");
  return (Tier)t;
}
EvictionParams to_params(const cbis_eviction_params* p) {
  EvictionParams e;
  if (p) {
    e.alpha_staleness = p->alpha_staleness;
    e.beta_restore_cost = p->beta_restore_cost;
    e.expected_compression_ratio = p->expected_compression_ratio;
    e.dram_fixed_ns = p->dram_fixed_ns;
    e.dram_ns_per_byte = p->dram_ns_per_byte;
    e.nvme_fixed_ns = p->nvme_fixed_ns;
    e.nvme_ns_per_byte = p->nvme_ns_per_byte;
  }
  return e;
}
void from_params(const EvictionParams& e, cbis_eviction_params* p) {
  *p = {e.alpha_staleness, e.beta_restore_cost, e.expected_compression_ratio, e.dram_fixed_ns,
        e.dram_ns_per_byte, e.nvme_fixed_ns, e.nvme_ns_per_byte};
}
}  // namespace

void cbis_eviction_params_default(cbis_eviction_params* p) {
  if (p) from_params(EvictionParams(), p);
}

cbis_tiered* cbis_tiered_create(int layer_count, int page_size, int n_heads, int head_dim, int kv_dtype,
                                const char* nvme_scratch_path, size_t gpu_capacity_blocks,
                                size_t dram_capacity_blocks, const cbis_eviction_params* params) {
  return guard_ptr<cbis_tiered>([&] {
    auto* t = new cbis_tiered();
    try {
      t->impl.reset(new TieredKVBlockManager(layer_count, page_size, n_heads, head_dim,
                                             nvme_scratch_path ? nvme_scratch_path : "", gpu_capacity_blocks,
                                             dram_capacity_blocks, to_params(params), kv_dtype));
    } catch (...) {
      delete t;
      throw;
    }
    return t;
  });
}

void cbis_tiered_destroy(cbis_tiered* t) { delete t; }

size_t cbis_tiered_raw_block_bytes(const cbis_tiered* t) { return t->impl->raw_block_bytes(); }

int cbis_tiered_calibrate(cbis_tiered* t) {
  return guard([&] {
    t->impl->calibrate();
    return 0;
  });
}

int cbis_tiered_params(const cbis_tiered* t, cbis_eviction_params* out) {
  return guard([&] {
    if (!out) throw std::invalid_argument("params: null output");
    from_params(t->impl->params(), out);
    return 0;
  });
}

int cbis_tiered_admit_gpu_resident(cbis_tiered* t, uint64_t block_id, cbis_cache* c, int physical_page,
                                   long now_step) {
  return guard([&] {
    t->impl->admit_gpu_resident(block_id, *c->impl, physical_page, now_step);
    return 0;
  });
}

int cbis_tiered_evict_one(cbis_tiered* t, long now_step, uint64_t* evicted) {
  return guard([&] {
    const uint64_t id = t->impl->evict_one(now_step);
    if (evicted) *evicted = id;
    return 0;
  });
}

int cbis_tiered_spill(cbis_tiered* t, uint64_t block_id, int dest_tier, long now_step) {
  return guard([&] {
    t->impl->spill(block_id, to_tier(dest_tier), now_step);
    return 0;
  });
}

int cbis_tiered_restore(cbis_tiered* t, uint64_t block_id, cbis_cache* c, int physical_page, long now_step) {
  return guard([&] {
    t->impl->restore(block_id, *c->impl, physical_page, now_step);
    return 0;
  });
}

int cbis_tiered_spill_batch(cbis_tiered* t, const uint64_t* block_ids, int n, int dest_tier, long now_step) {
  return guard([&] {
    if (n < 0 || (n > 0 && !block_ids)) throw std::invalid_argument("spill_batch: bad block list");
    t->impl->spill_batch(std::vector<uint64_t>(block_ids, block_ids + n), to_tier(dest_tier), now_step);
    return 0;
  });
}

int cbis_tiered_restore_batch(cbis_tiered* t, const uint64_t* block_ids, int n, cbis_cache* c,
                              const int* physical_pages, long now_step) {
  return guard([&] {
    if (n < 0 || (n > 0 && (!block_ids || !physical_pages)))
      throw std::invalid_argument("restore_batch: bad block list");
    t->impl->restore_batch(std::vector<uint64_t>(block_ids, block_ids + n), *c->impl,
                           std::vector<int>(physical_pages, physical_pages + n), now_step);
    return 0;
  });
}

int cbis_tiered_tier_of(const cbis_tiered* t, uint64_t block_id) {
  return guard([&] { return (int)t->impl->tier_of(block_id); });
}

int cbis_tiered_known(const cbis_tiered* t, uint64_t block_id) { return t->impl->known(block_id) ? 1 : 0; }

int cbis_tiered_touch(cbis_tiered* t, uint64_t block_id, long now_step) {
  return guard([&] {
    t->impl->touch(block_id, now_step);
    return 0;
  });
}

int cbis_tiered_stats(const cbis_tiered* t, size_t* out) {
  return guard([&] {
    if (!out) throw std::invalid_argument("stats: null output");
    const BlockStats s = t->impl->stats();
    out[0] = s.gpu_count;
    out[1] = s.dram_count;
    out[2] = s.nvme_count;
    out[3] = s.raw_bytes_total;
    out[4] = s.compressed_bytes_total;
    return 0;
  });
}

int64_t cbis_block_deflate(const void* src, size_t len, void* dst, size_t cap) {
  int64_t r = -1;
  const int rc = guard([&] {
    const std::vector<uint8_t> c = deflate_block(src, len);
    if (c.size() > cap) throw std::length_error("block_deflate: output capacity too small");
    std::memcpy(dst, c.data(), c.size());
    r = (int64_t)c.size();
    return 0;
  });
  return rc < 0 ? rc : r;
}

int cbis_block_inflate(const void* src, size_t len, void* dst, size_t out_len) {
  return guard([&] {
    inflate_block((const uint8_t*)src, len, dst, out_len);
    return 0;
  });
}

}  // extern "C"
