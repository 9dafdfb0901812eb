// Continuous batching, the iteration-level scheduler of
// src/bench_batching.cpp:98-179 with every request present at t = 0:
//  * free slots admit requests in order (allocate_sequence);
//  * an un-prefilled slot contributes its whole prompt as rows at positions
//    0..P-1 (ensure_capacity per row); a prefilled slot one decode row at
//    next_pos fed with its last generated token;
//  * after the step, each slot's last row yields its next token by greedy
//    argmax (first maximum wins, :66-73) -- taken on the device here;
//  * a slot completes when generated >= decode_len and frees its pages.
#include <chrono>

#include "runtime.hpp"

namespace cbis {

ContinuousResult run_continuous(TransformerRunner& runner, PagedKVCache& cache, const std::vector<Request>& reqs,
                                int max_slots) {
  struct Slot {
    bool active = false;
    int req = -1, seq_id = -1, next_pos = 0, last_token = 0, generated = 0;
    bool prefilled = false;
  };
  if (max_slots <= 0) throw std::invalid_argument("run_continuous: max_slots must be > 0");
  ContinuousResult res;
  res.tokens.assign(reqs.size(), {});
  std::vector<Slot> slots(max_slots);
  size_t next_req = 0;
  size_t completed = 0;
  using Clock = std::chrono::steady_clock;
  while (completed < reqs.size()) {
    for (auto& s : slots) {
      if (s.active) continue;
      if (next_req >= reqs.size()) break;
      s = Slot();
      s.active = true;
      s.req = (int)next_req++;
      s.seq_id = cache.allocate_sequence();
    }
    std::vector<int> tok, pos, sid;
    std::vector<Slot*> owner;
    std::vector<char> last;
    for (auto& s : slots) {
      if (!s.active) continue;
      const Request& r = reqs[s.req];
      if (!s.prefilled) {
        for (int p = 0; p < (int)r.prompt.size(); ++p) {
          if (!cache.ensure_capacity(s.seq_id, p)) throw std::runtime_error("run_continuous: out of KV pages");
          tok.push_back(r.prompt[p]);
          pos.push_back(p);
          sid.push_back(s.seq_id);
          owner.push_back(&s);
          last.push_back(p == (int)r.prompt.size() - 1);
        }
        s.next_pos = (int)r.prompt.size();
        s.prefilled = true;
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
    if (tok.empty()) throw std::runtime_error("run_continuous: no runnable rows (empty prompt?)");
    const auto t0 = Clock::now();
    const std::vector<int> next = runner.forward_step_greedy(tok, pos, sid);
    res.step_ms.push_back(std::chrono::duration<double, std::milli>(Clock::now() - t0).count());
    for (size_t i = 0; i < tok.size(); ++i) {
      if (!last[i]) continue;
      Slot* s = owner[i];
      s->last_token = next[i];
      s->generated += 1;
      res.tokens[s->req].push_back(next[i]);
      if (s->generated >= reqs[s->req].decode_len) {
        cache.free_sequence(s->seq_id);
        s->active = false;
        completed += 1;
      }
    }
  }
  return res;
}

}  // namespace cbis
