// Continuous batching, the iteration-level scheduler of
// src/bench_batching.cpp:98-179:
//  * free slots admit requests in order (allocate_sequence), each once its
//    arrival time has passed; with no active slot the scheduler waits for
//    the next arrival;
//  * slots are visited in order every step; a slot still feeding its prompt
//    contributes its next prompt rows (ensure_capacity per row), a slot past
//    its prompt one decode row at next_pos fed with its last generated token;
//  * after the step, the row that ends a slot's prompt, and every decode row,
//    yields the slot's next token by greedy argmax (first maximum wins,
//    src/bench_batching.cpp:66-73) -- taken on the device here;
//  * a slot completes when generated >= decode_len and frees its pages.
// With prefill_chunk = 0 and no token budget a slot's whole prompt goes in
// the step after its admission: the reference's schedule, row for row (and
// so its page allocation order).  prefill_chunk > 0 feeds at most that many
// prompt rows per slot per step (the chunked prefill of
// src/bench_tiering.cpp:78-89, mixed with the other slots' decode rows);
// step_token_budget > 0 caps the prompt rows of one step, decode rows are
// never deferred.
//
// The pipelined variant builds the same steps but queues step t + 1 before
// step t's tokens come back: a decode row names the row of the previous step
// that produces its input token, and the device reads it there.  A slot's
// completion depends only on how many tokens it has generated, so the host
// can free its pages when it queues the slot's last row; the stream runs the
// steps in order, so a later step that reuses those pages writes them only
// after that row's step is done with them.
#include <chrono>
#include <cmath>
#include <deque>
#include <thread>

#include "runtime.hpp"

namespace cbis {

namespace {

struct Slot {
  bool active = false;
  int req = -1, seq_id = -1, fed = 0, next_pos = 0, last_token = 0, generated = 0;
  int src_row = -1;  // pipelined: the row of the last queued step that yields this slot's next input token
};

void validate(const std::vector<Request>& reqs, const ScheduleOptions& opt) {
  if (opt.max_slots <= 0) throw std::invalid_argument("run_continuous: max_slots must be > 0");
  if (opt.prefill_chunk < 0 || opt.step_token_budget < 0)
    throw std::invalid_argument("run_continuous: prefill_chunk and step_token_budget must be >= 0");
  double prev_arrival = 0.0;
  for (const auto& r : reqs) {
    if (r.prompt.empty()) throw std::invalid_argument("run_continuous: empty prompt");
    if (r.decode_len <= 0) throw std::invalid_argument("run_continuous: decode_len must be > 0");
    if (!std::isfinite(r.arrival_ms) || r.arrival_ms < prev_arrival)
      throw std::invalid_argument("run_continuous: arrival_ms must be finite, >= 0 and nondecreasing");
    prev_arrival = r.arrival_ms;
  }
}

// One step's rows: (token, position, sequence) and, pipelined, the source
// row of a decode row's token (-1 elsewhere; such rows carry tok -1).
struct Rows {
  std::vector<int> tok, pos, sid, src;
  std::vector<Slot*> owner;
  std::vector<char> last;  // the row yields its slot's next token
};

class Batcher {
 public:
  Batcher(PagedKVCache& cache, const std::vector<Request>& reqs, const ScheduleOptions& opt)
      : cache_(cache), reqs_(reqs), opt_(opt), slots_(opt.max_slots) {}

  // Admits the requests that have arrived by `now` into free slots, then
  // builds every active slot's rows.  false: no slot is active.
  bool build(double now, bool device_tokens, Rows& r) {
    for (auto& s : slots_) {
      if (s.active) continue;
      if (next_req_ >= reqs_.size() || reqs_[next_req_].arrival_ms > now) break;
      s = Slot();
      s.active = true;
      s.req = (int)next_req_++;
      s.seq_id = cache_.allocate_sequence();
    }
    r = Rows();
    int prompt_rows = 0;
    for (auto& s : slots_) {
      if (!s.active) continue;
      const Request& q = reqs_[s.req];
      const int P = (int)q.prompt.size();
      if (s.fed < P) {
        int n = P - s.fed;
        if (opt_.prefill_chunk > 0) n = std::min(n, opt_.prefill_chunk);
        if (opt_.step_token_budget > 0) n = std::min(n, opt_.step_token_budget - prompt_rows);
        for (int p = s.fed; p < s.fed + n; ++p) {
          if (!cache_.ensure_capacity(s.seq_id, p)) throw std::runtime_error("run_continuous: out of KV pages");
          add(r, &s, q.prompt[p], -1, p, p == P - 1);
        }
        s.fed += std::max(n, 0);
        prompt_rows += std::max(n, 0);
        s.next_pos = s.fed;
      } else {
        if (!cache_.ensure_capacity(s.seq_id, s.next_pos)) throw std::runtime_error("run_continuous: out of KV pages");
        if (device_tokens) add(r, &s, -1, s.src_row, s.next_pos, true);
        else add(r, &s, s.last_token, -1, s.next_pos, true);
        s.next_pos += 1;
      }
    }
    bool any_active = false;
    for (const auto& s : slots_) any_active = any_active || s.active;
    if (any_active && r.tok.empty()) throw std::runtime_error("run_continuous: no runnable rows");
    return any_active;
  }

  // Counts the token row i of this step yields for its slot; true when that
  // completes the request (its pages are freed and the slot opens).
  bool yield(Rows& r, size_t i) {
    Slot* s = r.owner[i];
    s->src_row = (int)i;
    s->generated += 1;
    if (s->generated < reqs_[s->req].decode_len) return false;
    cache_.free_sequence(s->seq_id);
    s->active = false;
    return true;
  }

  // The request the next admission waits for (when no slot is active).
  double next_arrival() const { return reqs_[next_req_].arrival_ms; }

 private:
  static void add(Rows& r, Slot* s, int tok, int src, int pos, bool last) {
    r.tok.push_back(tok);
    r.src.push_back(src);
    r.pos.push_back(pos);
    r.sid.push_back(s->seq_id);
    r.owner.push_back(s);
    r.last.push_back(last);
  }

  PagedKVCache& cache_;
  const std::vector<Request>& reqs_;
  const ScheduleOptions& opt_;
  std::vector<Slot> slots_;
  size_t next_req_ = 0;
};

using Clock = std::chrono::steady_clock;

// The run's clock and an idle scheduler's wait (virtual ones when set).
struct RunClock {
  const ScheduleOptions& opt;
  Clock::time_point start = Clock::now();
  double now() const {
    return opt.clock_ms ? opt.clock_ms() : std::chrono::duration<double, std::milli>(Clock::now() - start).count();
  }
  void wait(double ms) const {
    if (ms <= 0) return;
    if (opt.wait_ms) opt.wait_ms(ms);
    else std::this_thread::sleep_for(std::chrono::duration<double, std::milli>(ms));
  }
};

}  // namespace

ContinuousResult run_continuous(const StepFn& step, PagedKVCache& cache, const std::vector<Request>& reqs,
                                const ScheduleOptions& opt, std::vector<StepRows>* trace) {
  validate(reqs, opt);
  ContinuousResult res;
  res.tokens.assign(reqs.size(), {});
  res.finish_ms.assign(reqs.size(), 0.0);
  Batcher batch(cache, reqs, opt);
  const RunClock clock{opt};
  size_t completed = 0;
  Rows r;
  while (completed < reqs.size()) {
    const double now = clock.now();
    if (!batch.build(now, false, r)) {  // nothing admitted yet: wait for the next arrival
      clock.wait(batch.next_arrival() - now);
      continue;
    }
    if (trace) trace->push_back({r.tok, r.pos, r.sid});
    const auto t0 = Clock::now();
    const std::vector<int> next = step(r.tok, r.pos, r.sid);
    res.step_ms.push_back(std::chrono::duration<double, std::milli>(Clock::now() - t0).count());
    const double step_done = clock.now();
    if (next.size() != r.tok.size()) throw std::runtime_error("run_continuous: step returned a wrong row count");
    for (size_t i = 0; i < r.tok.size(); ++i) {
      if (!r.last[i]) continue;
      Slot* s = r.owner[i];
      s->last_token = next[i];
      res.tokens[s->req].push_back(next[i]);
      const int req = s->req;
      if (batch.yield(r, i)) {
        res.finish_ms[req] = step_done;
        completed += 1;
      }
    }
  }
  return res;
}

ContinuousResult run_continuous_pipelined(const PipelinedStep& step, PagedKVCache& cache,
                                          const std::vector<Request>& reqs, const ScheduleOptions& opt,
                                          std::vector<StepRows>* trace) {
  validate(reqs, opt);
  ContinuousResult res;
  res.tokens.assign(reqs.size(), {});
  res.finish_ms.assign(reqs.size(), 0.0);
  Batcher batch(cache, reqs, opt);
  const RunClock clock{opt};
  struct InFlight {
    int64_t ticket;
    size_t rows;
    std::vector<std::pair<int, int>> yields;  // (request, row) pairs whose tokens this step produces
    std::vector<int> finished;                // requests whose last token it produces
    Clock::time_point queued;
  };
  std::deque<InFlight> inflight;
  Clock::time_point last_collect = Clock::now();
  auto collect = [&]() {
    InFlight f = std::move(inflight.front());
    inflight.pop_front();
    const std::vector<int> next = step.wait(f.ticket);
    const Clock::time_point t = Clock::now();
    res.step_ms.push_back(std::chrono::duration<double, std::milli>(t - std::max(f.queued, last_collect)).count());
    last_collect = t;
    if (next.size() != f.rows) throw std::runtime_error("run_continuous: step returned a wrong row count");
    for (const auto& y : f.yields) res.tokens[y.first].push_back(next[y.second]);
    const double done = clock.now();
    for (int q : f.finished) res.finish_ms[q] = done;
  };
  try {
    size_t queued_done = 0;  // requests whose last row has been queued
    Rows r;
    while (queued_done < reqs.size()) {
      const double now = clock.now();
      if (!batch.build(now, true, r)) {
        while (!inflight.empty()) collect();
        clock.wait(batch.next_arrival() - now);
        continue;
      }
      if (trace) trace->push_back({r.tok, r.pos, r.sid});
      InFlight f;
      f.queued = Clock::now();
      f.ticket = step.enqueue(r.tok, r.pos, r.sid, r.src);
      f.rows = r.tok.size();
      for (size_t i = 0; i < r.tok.size(); ++i) {
        if (!r.last[i]) continue;
        const int req = r.owner[i]->req;
        f.yields.push_back({req, (int)i});
        if (batch.yield(r, i)) {
          f.finished.push_back(req);
          queued_done += 1;
        }
      }
      inflight.push_back(std::move(f));
      while (inflight.size() > 1) collect();  // keep one step in flight
    }
    while (!inflight.empty()) collect();
  } catch (...) {
    // Leave no step queued behind: the step's owner may reuse its buffers.
    for (const InFlight& f : inflight) {
      try {
        (void)step.wait(f.ticket);
      } catch (...) {
      }
    }
    throw;
  }
  return res;
}

ContinuousResult run_continuous(TransformerRunner& runner, PagedKVCache& cache, const std::vector<Request>& reqs,
                                const ScheduleOptions& opt) {
  const StepFn step = [&](const std::vector<int>& t, const std::vector<int>& p, const std::vector<int>& s) {
    return runner.forward_step_greedy(t, p, s);
  };
  return run_continuous(step, cache, reqs, opt);
}

ContinuousResult run_continuous(TransformerRunner& runner, PagedKVCache& cache, const std::vector<Request>& reqs,
                                int max_slots) {
  ScheduleOptions opt;
  opt.max_slots = max_slots;
  return run_continuous(runner, cache, reqs, opt);
}

ContinuousResult run_continuous_pipelined(TransformerRunner& runner, PagedKVCache& cache,
                                          const std::vector<Request>& reqs, const ScheduleOptions& opt) {
  PipelinedStep step;
  step.enqueue = [&](const std::vector<int>& t, const std::vector<int>& p, const std::vector<int>& s,
                     const std::vector<int>& src) { return runner.enqueue_greedy(t, p, s, src); };
  step.wait = [&](int64_t ticket) { return runner.wait_greedy(ticket); };
  return run_continuous_pipelined(step, cache, reqs, opt);
}

}  // namespace cbis
