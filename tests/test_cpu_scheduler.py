"""CPU checks of the continuous-batching scheduler (libcbis.so on the host,
no HIP call): cbis_schedule_dry_run drives run_continuous with a stand-in
step, and its per-step rows and generated tokens are compared with a
restatement of the reference's schedule (src/bench_batching.cpp:98-179) and
of its chunked-prefill extension."""
import random

import pytest
from hypothesis import given, settings, strategies as st


def _stand_in(tok, pos, sid, vocab):
    """The dry run's stand-in greedy token (include/cbis_runtime.h)."""
    return ((tok * 31 + pos * 7 + sid * 13 + 1) & 0xFFFFFFFF) % vocab


def _restated(prompts, decode_lens, vocab, max_slots, chunk=0, budget=0):
    """src/bench_batching.cpp:98-179 with every request present at t = 0:
    free slots admit requests in order (:110-119), slots are visited in
    order and contribute their prompt (:130-141) -- here at most `chunk`
    rows of it per step and at most `budget` prompt rows per step -- or one
    decode row (:142-149); the row ending a prompt and every decode row yield
    the slot's next token (:160-166); a slot completes at decode_len
    (:167-172).  Sequence ids come from a counter starting at 0."""
    slots = [None] * max_slots
    nxt, done, seq_counter = 0, 0, 0
    toks = [[] for _ in prompts]
    steps = []
    while done < len(prompts):
        for k in range(max_slots):
            if slots[k] is not None:
                continue
            if nxt >= len(prompts):
                break
            slots[k] = {"req": nxt, "sid": seq_counter, "fed": 0, "pos": 0, "last": 0, "gen": 0}
            nxt += 1
            seq_counter += 1
        rows, owners, lasts = [], [], []
        prompt_rows = 0
        for s in slots:
            if s is None:
                continue
            p = prompts[s["req"]]
            if s["fed"] < len(p):
                n = len(p) - s["fed"]
                if chunk > 0:
                    n = min(n, chunk)
                if budget > 0:
                    n = min(n, budget - prompt_rows)
                for q in range(s["fed"], s["fed"] + max(n, 0)):
                    rows.append((p[q], q, s["sid"]))
                    owners.append(s)
                    lasts.append(q == len(p) - 1)
                s["fed"] += max(n, 0)
                prompt_rows += max(n, 0)
                s["pos"] = s["fed"]
            else:
                rows.append((s["last"], s["pos"], s["sid"]))
                owners.append(s)
                lasts.append(True)
                s["pos"] += 1
        steps.append(rows)
        for (t, q, sid), s, last in zip(rows, owners, lasts):
            if not last:
                continue
            tok = _stand_in(t, q, sid, vocab)
            s["last"] = tok
            s["gen"] += 1
            toks[s["req"]].append(tok)
            if s["gen"] >= decode_lens[s["req"]]:
                slots[slots.index(s)] = None
                done += 1
    return toks, steps


def _cache(cbis, max_pages=4096):
    return cbis.PagedKVCache(4, max_pages, 16, 8, 32, "f32", alloc_device=False)


def _workload(seed, n, lo, hi, dlo, dhi, vocab=512):
    rng = random.Random(seed)
    prompts = [[rng.randrange(vocab) for _ in range(rng.randint(lo, hi))] for _ in range(n)]
    return prompts, [rng.randint(dlo, dhi) for _ in range(n)]


def test_reference_schedule_config1(cbis):
    """Config 1's shape: 8 prompts U[16,64] and 32 tokens each in 16 slots
    is one whole-prompt prefill step plus 31 decode steps of 8 rows."""
    prompts, dl = _workload(0, 8, 16, 64, 32, 32)
    c = _cache(cbis)
    toks, steps = cbis.schedule_dry_run(c, prompts, dl, 512, max_slots=16)
    rtoks, rsteps = _restated(prompts, dl, 512, 16)
    assert steps == rsteps and toks == rtoks
    assert len(steps) == 32
    assert len(steps[0]) == sum(len(p) for p in prompts)
    assert all(len(s) == 8 for s in steps[1:])
    assert c.num_free_pages() == 4096


def test_reference_schedule_slot_reuse(cbis):
    """More requests than slots: a finished slot admits the next request at
    the start of the following step."""
    prompts, dl = _workload(1, 23, 1, 40, 1, 9)
    c = _cache(cbis)
    toks, steps = cbis.schedule_dry_run(c, prompts, dl, 1000, max_slots=5)
    rtoks, rsteps = _restated(prompts, dl, 1000, 5)
    assert steps == rsteps and toks == rtoks
    assert [len(t) for t in toks] == dl
    assert c.num_free_pages() == 4096


@pytest.mark.parametrize("chunk,budget", [(1, 0), (7, 0), (16, 0), (0, 20), (16, 48), (5, 12)])
def test_chunked_prefill_schedule(cbis, chunk, budget):
    prompts, dl = _workload(2, 12, 1, 70, 1, 12)
    c = _cache(cbis)
    toks, steps = cbis.schedule_dry_run(c, prompts, dl, 777, max_slots=6, prefill_chunk=chunk,
                                        step_token_budget=budget)
    rtoks, rsteps = _restated(prompts, dl, 777, 6, chunk, budget)
    assert steps == rsteps and toks == rtoks
    # every prompt position is fed exactly once, in order, within the caps;
    # on a fresh cache sequence ids are the request indices
    fed = [[] for _ in prompts]
    for rows in steps:
        prompt_rows = [(t, q, sid) for t, q, sid in rows if q < len(prompts[sid])]
        if budget > 0:
            assert len(prompt_rows) <= budget
        for sid in {r[2] for r in prompt_rows}:
            mine = [q for t, q, s in prompt_rows if s == sid]
            assert chunk == 0 or len(mine) <= chunk
            fed[sid] += mine
        for t, q, sid in prompt_rows:
            assert t == prompts[sid][q]
    assert fed == [list(range(len(p))) for p in prompts]
    whole, _ = cbis.schedule_dry_run(_cache(cbis), prompts, dl, 777, max_slots=6)
    assert toks == whole
    assert c.num_free_pages() == 4096


@settings(max_examples=40, deadline=None)
@given(seed=st.integers(0, 10 ** 6), n=st.integers(1, 14), slots=st.integers(1, 8), chunk=st.integers(0, 20),
       budget=st.integers(0, 40))
def test_schedule_matches_restatement(cbis, seed, n, slots, chunk, budget):
    prompts, dl = _workload(seed, n, 1, 50, 1, 6)
    c = _cache(cbis)
    toks, steps = cbis.schedule_dry_run(c, prompts, dl, 300, max_slots=slots, prefill_chunk=chunk,
                                        step_token_budget=budget)
    rtoks, rsteps = _restated(prompts, dl, 300, slots, chunk, budget)
    assert steps == rsteps and toks == rtoks
    assert c.num_free_pages() == 4096


def test_schedule_rejects_bad_input(cbis):
    c = _cache(cbis)
    with pytest.raises(RuntimeError, match="empty prompt"):
        cbis.schedule_dry_run(c, [[1, 2], []], [2, 2], 100)
    with pytest.raises(RuntimeError, match="decode_len"):
        cbis.schedule_dry_run(c, [[1, 2]], [0], 100)
    with pytest.raises(RuntimeError, match="prefill_chunk"):
        cbis.schedule_dry_run(c, [[1, 2]], [1], 100, prefill_chunk=-1)
    with pytest.raises(RuntimeError, match="out of KV pages"):
        cbis.schedule_dry_run(_cache(cbis, max_pages=2), [[1] * 40], [1], 100)


def _restated_arrivals(prompts, decode_lens, arrivals, vocab, max_slots, step_ms):
    """src/bench_batching.cpp:98-179 on a virtual clock: at the top of each
    iteration free slots admit, in order, the requests whose arrival_ms has
    passed (:108-121); with no active slot the loop waits for the next
    arrival (:153-158); a forward step takes step_ms; a request finishes at
    the clock after its last step (:162-172)."""
    slots = [None] * max_slots
    nxt, done, seq_counter, clock = 0, 0, 0, 0.0
    toks = [[] for _ in prompts]
    finish = [0.0] * len(prompts)
    steps = []
    while done < len(prompts):
        now = clock
        for k in range(max_slots):
            if slots[k] is not None:
                continue
            if nxt >= len(prompts) or arrivals[nxt] > now:
                break
            slots[k] = {"req": nxt, "sid": seq_counter, "pos": 0, "pre": False, "last": 0, "gen": 0}
            nxt += 1
            seq_counter += 1
        rows, owners, lasts = [], [], []
        for s in slots:
            if s is None:
                continue
            p = prompts[s["req"]]
            if not s["pre"]:
                for q in range(len(p)):
                    rows.append((p[q], q, s["sid"]))
                    owners.append(s)
                    lasts.append(q == len(p) - 1)
                s["pos"], s["pre"] = len(p), True
            else:
                rows.append((s["last"], s["pos"], s["sid"]))
                owners.append(s)
                lasts.append(True)
                s["pos"] += 1
        if not rows:
            clock += max(0.0, arrivals[nxt] - now)
            continue
        steps.append(rows)
        clock += step_ms
        for (t, q, sid), s, last in zip(rows, owners, lasts):
            if not last:
                continue
            tok = _stand_in(t, q, sid, vocab)
            s["last"] = tok
            s["gen"] += 1
            toks[s["req"]].append(tok)
            if s["gen"] >= decode_lens[s["req"]]:
                finish[s["req"]] = clock
                slots[slots.index(s)] = None
                done += 1
    return toks, steps, finish


@settings(max_examples=30, deadline=None)
@given(seed=st.integers(0, 10 ** 6), n=st.integers(1, 12), slots=st.integers(1, 6),
       gap=st.sampled_from([0.0, 0.5, 2.0, 7.5]))
def test_arrival_schedule_matches_restatement(cbis, seed, n, slots, gap):
    """Arrival-time admission on the dry run's virtual clock (1 ms steps):
    requests arriving on a random walk of mean `gap` ms are admitted only
    once their time has passed, an idle scheduler jumps to the next arrival,
    and the finish times are the clock after each request's last step."""
    prompts, dl = _workload(seed, n, 1, 30, 1, 6)
    rng = random.Random(seed + 1)
    arrivals, t = [], 0.0
    for _ in range(n):
        t += rng.random() * 2 * gap
        arrivals.append(round(t, 3))
    c = _cache(cbis)
    toks, steps, fin = cbis.schedule_dry_run(c, prompts, dl, 300, max_slots=slots, arrival_ms=arrivals,
                                             step_time_ms=1.0)
    rtoks, rsteps, rfin = _restated_arrivals(prompts, dl, arrivals, 300, slots, 1.0)
    assert steps == rsteps and toks == rtoks
    assert fin == pytest.approx(rfin)
    assert all(f >= a for f, a in zip(fin, arrivals))
    assert c.num_free_pages() == 4096


def test_arrivals_at_zero_are_the_plain_schedule(cbis):
    prompts, dl = _workload(5, 9, 1, 40, 1, 8)
    plain = cbis.schedule_dry_run(_cache(cbis), prompts, dl, 500, max_slots=4)
    timed = cbis.schedule_dry_run(_cache(cbis), prompts, dl, 500, max_slots=4, arrival_ms=[0.0] * 9)
    assert timed[:2] == plain


def test_arrivals_rejected_when_unordered(cbis):
    with pytest.raises(RuntimeError, match="arrival_ms"):
        cbis.schedule_dry_run(_cache(cbis), [[1], [2]], [1, 1], 100, arrival_ms=[5.0, 1.0])
    with pytest.raises(RuntimeError, match="arrival_ms"):
        cbis.schedule_dry_run(_cache(cbis), [[1]], [1], 100, arrival_ms=[-1.0])


@settings(max_examples=30, deadline=None)
@given(seed=st.integers(0, 10 ** 6), n=st.integers(1, 12), slots=st.integers(1, 6), chunk=st.sampled_from([0, 1, 7]),
       budget=st.sampled_from([0, 9]), gap=st.sampled_from([0.0, 0.5, 3.0]))
def test_pipelined_schedule_is_the_synchronous_one(cbis, seed, n, slots, chunk, budget, gap):
    """The pipelined scheduler queues step t + 1 before step t's tokens are
    back; its decode rows name the previous step's row that holds their input
    token and the stand-in device resolves it there.  Steps, resolved row
    tokens, generated tokens and page use must equal the synchronous
    schedule's; a request's finish is seen one step later at most (its last
    step is collected after the next one is queued)."""
    prompts, dl = _workload(seed, n, 1, 30, 1, 6)
    rng = random.Random(seed + 2)
    arrivals, t = [], 0.0
    for _ in range(n):
        t += rng.random() * 2 * gap
        arrivals.append(round(t, 3))
    kw = dict(max_slots=slots, prefill_chunk=chunk, step_token_budget=budget, arrival_ms=arrivals, step_time_ms=1.0)
    c_sync, c_pipe = _cache(cbis), _cache(cbis)
    toks, steps, fin = cbis.schedule_dry_run(c_sync, prompts, dl, 300, **kw)
    ptoks, psteps, pfin = cbis.schedule_dry_run(c_pipe, prompts, dl, 300, pipeline=True, **kw)
    assert psteps == steps and ptoks == toks
    for f, pf in zip(fin, pfin):
        assert f <= pf <= f + 1.0
    assert c_pipe.num_free_pages() == c_sync.num_free_pages() == 4096
