"""Pipelined greedy decode through the runtime C-ABI: a step is queued
before the previous step's tokens are back, and each decode row reads its
input token on the device from the row of the previous step that produced
it (cbis_runner_enqueue_greedy's token_src).  The tokens must be those of
the synchronous path (cbis_runner_forward_step_greedy fed the same tokens
from the host) and, for config 1, python/model.py's greedy decode
(tests/golden/g2_c1_greedy.npz)."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _model(cbis, wdt, kvdt):
    cfg = cbis.ModelConfig.make(vocab=512, n_layers=2, weight_dtype=wdt, kv_dtype=kvdt, max_seq=512)
    return cbis.ModelWeights.synthetic(cfg, seed=3)


def _setup(cbis, w, kvdt, prompts):
    cache = cbis.PagedKVCache(2, 64, 16, 8, 32, kvdt, pages_per_seq=32)
    runner = cbis.TransformerRunner(w, cache, 256)
    seqs = []
    for p in prompts:
        s = cache.allocate_sequence()
        for q in range(len(p) + 8):
            assert cache.ensure_capacity(s, q)
        seqs.append(s)
    return cache, runner, seqs


@pytest.mark.parametrize("wdt,kvdt", [("f32", "f32"), ("bf16", "bf16")])
@pytest.mark.parametrize("graphs", [True, False])
def test_token_src_steps_match_synchronous_steps(cbis, wdt, kvdt, graphs):
    """Three prompts prefilled in one step, then four decode steps, each
    queued before the previous one is waited for; the last decode steps also
    carry a fresh prompt's rows (no token source) beside the decode rows.
    Every step's greedy tokens equal the synchronous runner's, fed the same
    tokens from the host."""
    w = _model(cbis, wdt, kvdt)
    rng = np.random.default_rng(11)
    prompts = [[int(t) for t in rng.integers(0, 512, n)] for n in (5, 17, 33)]
    late = [int(t) for t in rng.integers(0, 512, 9)]
    _, pr, pseq = _setup(cbis, w, kvdt, prompts + [late])
    _, sr, sseq = _setup(cbis, w, kvdt, prompts + [late])
    pr.set_graphs(graphs)
    sr.set_graphs(graphs)

    def prefill_rows(seqs):
        tok, pos, sid = [], [], []
        for p, s in zip(prompts, seqs):
            tok += p
            pos += list(range(len(p)))
            sid += [s] * len(p)
        return tok, pos, sid

    lasts = list(np.cumsum([len(p) for p in prompts]) - 1)
    # Synchronous reference: the host feeds each step's tokens.
    ref = [sr.forward_step_greedy(*prefill_rows(sseq))]
    cur = [ref[0][i] for i in lasts]
    ref_rows = []
    for k in range(4):
        tok = list(cur)
        pos = [len(p) + k for p in prompts]
        sid = list(sseq[:3])
        if k >= 2:  # the late prompt joins, fed from the host
            q = (k - 2) * 4
            tok += late[q: q + 4]
            pos += list(range(q, q + 4))
            sid += [sseq[3]] * 4
        out = sr.forward_step_greedy(tok, pos, sid)
        ref.append(out)
        ref_rows.append((tok, pos, sid))
        cur = out[:3]

    # Pipelined: queue step k + 1 before waiting for step k.
    t_prev = pr.enqueue_greedy(*prefill_rows(pseq))
    src = lasts
    got = []
    for k in range(4):
        _, pos, _ = ref_rows[k]
        tok = [-1] * 3
        s = list(src)
        sid = list(pseq[:3])
        if k >= 2:
            q = (k - 2) * 4
            tok += late[q: q + 4]
            s += [-1] * 4
            sid += [pseq[3]] * 4
        t = pr.enqueue_greedy(tok, pos, sid, token_src=s)
        got.append(pr.wait_greedy(t_prev))
        t_prev = t
        src = [0, 1, 2]
    got.append(pr.wait_greedy(t_prev))
    assert got == ref


def test_token_src_errors(cbis):
    w = _model(cbis, "f32", "f32")
    _, r, seqs = _setup(cbis, w, "f32", [[1, 2, 3]])
    s = seqs[0]
    with pytest.raises(cbis.CbisError, match="token_src needs a greedy step"):
        r.enqueue_greedy([-1], [0], [s], token_src=[0])
    t0 = r.enqueue_greedy([1, 2, 3], [0, 1, 2], [s] * 3)
    with pytest.raises(IndexError, match="token_src beyond"):
        r.enqueue_greedy([-1], [3], [s], token_src=[3])
    with pytest.raises(IndexError, match="token id out of range"):
        r.enqueue_greedy([-1], [3], [s], token_src=[-1])
    t1 = r.enqueue_greedy([-1], [3], [s], token_src=[2])
    with pytest.raises(cbis.CbisError, match="has not been waited for"):
        r.enqueue_greedy([-1], [4], [s], token_src=[0])
    with pytest.raises(cbis.CbisError, match="has not been waited for"):
        r.forward_step_greedy([5], [4], [s])
    with pytest.raises(cbis.CbisError, match="no queued greedy step"):
        r.wait_greedy(t1 + 7)
    a = r.wait_greedy(t0)
    b = r.wait_greedy(t1)
    with pytest.raises(cbis.CbisError, match="no queued greedy step"):
        r.wait_greedy(t1)  # already collected
    assert len(a) == 3 and len(b) == 1
    # The runner is still usable: the synchronous step at position 4.
    assert len(r.forward_step_greedy([b[0]], [4], [s])) == 1


@pytest.mark.parametrize("slots,chunk,budget,arrivals", [(16, 0, 0, False), (3, 0, 0, True), (16, 8, 40, False)])
def test_c1_pipelined_greedy(cbis, slots, chunk, budget, arrivals):
    """Config 1 (8 prompts U[16,64], 32 greedy tokens each) through the
    pipelined scheduler, with every request at t = 0, with arrivals over time
    and 3 slots, and with chunked prefill: tokens identical to
    python/model.py's greedy decode, every page freed."""
    g = np.load(os.path.join(GOLDEN, "g2_c1_greedy.npz"))
    n = int(g["n"])
    prompts = [[int(t) for t in g[f"prompt{i}"]] for i in range(n)]
    cfg = cbis.ModelConfig.make(vocab=512, n_layers=4, weight_dtype="f32", kv_dtype="f32")
    w = cbis.ModelWeights.synthetic(cfg, seed=0)
    cache = cbis.PagedKVCache(4, 128, 16, 8, 32, "f32")
    runner = cbis.TransformerRunner(w, cache, 512)
    arr = [5.0 + 2.0 * i for i in range(n)] if arrivals else None
    res = cbis.run_continuous(runner, cache, prompts, [32] * n, max_slots=slots, prefill_chunk=chunk,
                              step_token_budget=budget, arrival_ms=arr, pipeline=True)
    toks, step_ms = res[0], res[1]
    for i in range(n):
        assert toks[i] == [int(t) for t in g[f"gen{i}"]], i
    assert len(step_ms) >= 32
    if arrivals:
        assert all(f > a for f, a in zip(res[2], arr))
    assert cache.num_free_pages() == 128
    # The runner is left with nothing queued: a synchronous step works.
    s = cache.allocate_sequence()
    assert cache.ensure_capacity(s, 0)
    assert len(runner.forward_step_greedy([1], [0], [s])) == 1


def test_runner_closed_with_a_step_queued(cbis):
    """Closing a runner while a greedy step is still queued waits for it
    (its buffers are freed only after the stream has run it); the cache and a
    new runner over it then work, with the same tokens as before."""
    w = _model(cbis, "f32", "f32")
    cache, r, seqs = _setup(cbis, w, "f32", [[1, 2, 3, 4]])
    s = seqs[0]
    ref = r.forward_step_greedy([1, 2, 3, 4], [0, 1, 2, 3], [s] * 4)
    r.enqueue_greedy([1, 2, 3, 4], [0, 1, 2, 3], [s] * 4)
    r.enqueue_greedy([-1], [4], [s], token_src=[3])
    r.close()
    r2 = cbis.TransformerRunner(w, cache, 256)
    assert r2.forward_step_greedy([1, 2, 3, 4], [0, 1, 2, 3], [s] * 4) == ref
