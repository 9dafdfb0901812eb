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
#include <chrono>
#include <cmath>
#include <thread>

#include "runtime.hpp"

namespace cbis {

ContinuousResult run_continuous(const StepFn& step, PagedKVCache& cache, const std::vector<Request>& reqs,
                                const ScheduleOptions& opt, std::vector<StepRows>* trace) {
  struct Slot {
    bool active = false;
    int req = -1, seq_id = -1, fed = 0, next_pos = 0, last_token = 0, generated = 0;
  };
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
  ContinuousResult res;
  res.tokens.assign(reqs.size(), {});
  res.finish_ms.assign(reqs.size(), 0.0);
  std::vector<Slot> slots(opt.max_slots);
  size_t next_req = 0;
  size_t completed = 0;
  using Clock = std::chrono::steady_clock;
  const auto start = Clock::now();
  auto now_ms = [&]() {
    return opt.clock_ms ? opt.clock_ms() : std::chrono::duration<double, std::milli>(Clock::now() - start).count();
  };
  while (completed < reqs.size()) {
    const double now = now_ms();
    for (auto& s : slots) {
      if (s.active) continue;
      if (next_req >= reqs.size() || reqs[next_req].arrival_ms > now) break;
      s = Slot();
      s.active = true;
      s.req = (int)next_req++;
      s.seq_id = cache.allocate_sequence();
    }
    std::vector<int> tok, pos, sid;
    std::vector<Slot*> owner;
    std::vector<char> last;
    int prompt_rows = 0;
    for (auto& s : slots) {
      if (!s.active) continue;
      const Request& r = reqs[s.req];
      const int P = (int)r.prompt.size();
      if (s.fed < P) {
        int n = P - s.fed;
        if (opt.prefill_chunk > 0) n = std::min(n, opt.prefill_chunk);
        if (opt.step_token_budget > 0) n = std::min(n, opt.step_token_budget - prompt_rows);
        for (int p = s.fed; p < s.fed + n; ++p) {
          if (!cache.ensure_capacity(s.seq_id, p)) throw std::runtime_error("run_continuous: out of KV pages");
          tok.push_back(r.prompt[p]);
          pos.push_back(p);
          sid.push_back(s.seq_id);
          owner.push_back(&s);
          last.push_back(p == P - 1);
        }
        s.fed += std::max(n, 0);
        prompt_rows += std::max(n, 0);
        s.next_pos = s.fed;
      } else {
        if (!cache.ensure_capacity(s.seq_id, s.next_pos)) throw std::runtime_error("run_continuous: out of KV pages");
        tok.push_back(s.last_token);
        pos.push_back(s.next_pos);
        sid.push_back(s.seq_id);
        owner.push_back(&s);
        last.push_back(1);
        s.next_pos += 1;
      }
    }
    bool any_active = false;
    for (const auto& s : slots) any_active = any_active || s.active;
    if (!any_active) {  // nothing admitted yet: wait for the next arrival (next_req < reqs.size() here)
      const double wait = reqs[next_req].arrival_ms - now;
      if (wait > 0) {
        if (opt.wait_ms) opt.wait_ms(wait);
        else std::this_thread::sleep_for(std::chrono::duration<double, std::milli>(wait));
      }
      continue;
    }
    if (tok.empty()) throw std::runtime_error("run_continuous: no runnable rows");
    if (trace) trace->push_back({tok, pos, sid});
    const auto t0 = Clock::now();
    const std::vector<int> next = step(tok, pos, sid);
    res.step_ms.push_back(std::chrono::duration<double, std::milli>(Clock::now() - t0).count());
    const double step_done = now_ms();
    if (next.size() != tok.size()) throw std::runtime_error("run_continuous: step returned a wrong row count");
    for (size_t i = 0; i < tok.size(); ++i) {
      if (!last[i]) continue;
      Slot* s = owner[i];
      s->last_token = next[i];
      s->generated += 1;
      res.tokens[s->req].push_back(next[i]);
      if (s->generated >= reqs[s->req].decode_len) {
        res.finish_ms[s->req] = step_done;
        cache.free_sequence(s->seq_id);
        s->active = false;
        completed += 1;
      }
    }
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

}  // namespace cbis
