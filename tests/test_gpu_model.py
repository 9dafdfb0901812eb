"""Whole-step parity of TransformerRunner::forward_step (HIP path through the
runtime C-ABI) against the golden vectors written from the reference's
python/model.py and against the CPU oracle.

Tolerances: fp32 models 1e-4 max-abs on logits; bf16 / fp8 models 2e-2
relative (per row ||d||_inf / ||ref||_inf); greedy tokens identical.
"""
import ctypes
import os

import numpy as np
import pytest

from helpers import bits_u16, check_logits as _check_logits, row_rel_err

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _ref_model(cbis, vocab=1000, n_layers=4, wdt="f32", kvdt="f32", **kw):
    cfg = cbis.ModelConfig.make(vocab=vocab, n_layers=n_layers, weight_dtype=wdt, kv_dtype=kvdt, **kw)
    return cfg, cbis.ModelWeights.synthetic(cfg, seed=0)


def test_g1_reference_dims_logits(cbis):
    """Reference model dims (V=1000, d=256, 8x32, L=4) with seeded weights:
    single-sequence prefill of lengths 1/3/7/16/31/64 as src/correctness_check.cpp
    runs it, against logits from python/model.py (tests/golden/g1_refmodel.npz)."""
    g = np.load(os.path.join(GOLDEN, "g1_refmodel.npz"))
    cfg, w = _ref_model(cbis)
    cache = cbis.PagedKVCache(4, 8 * 6 + 8, 16, 8, 32, "f32", pages_per_seq=2048)
    runner = cbis.TransformerRunner(w, cache, 128)
    worst = 0.0
    for i in range(len(g["lens"])):
        ids = [int(t) for t in g[f"ids{i}"]]
        sid = cache.allocate_sequence()
        for p in range(len(ids)):
            assert cache.ensure_capacity(sid, p)
        lg = runner.forward_step(ids, list(range(len(ids))), [sid] * len(ids))
        worst = max(worst, float(np.abs(lg - g[f"logits{i}"]).max()))
        cache.free_sequence(sid)
    assert worst < 1e-4, worst


def test_c1_greedy_continuous_batching(cbis, oracle):
    """Config 1: 8 prompts U[16,64], 32 greedy tokens each through
    the continuous-batching scheduler -- tokens identical to python/model.py's
    full-recompute greedy decode (tests/golden/g2_c1_greedy.npz)."""
    g = np.load(os.path.join(GOLDEN, "g2_c1_greedy.npz"))
    n = int(g["n"])
    prompts = [[int(t) for t in g[f"prompt{i}"]] for i in range(n)]
    cfg, w = _ref_model(cbis, vocab=512)
    cache = cbis.PagedKVCache(4, 128, 16, 8, 32, "f32")
    runner = cbis.TransformerRunner(w, cache, 512)
    toks, step_ms = cbis.run_continuous(runner, cache, prompts, [32] * n, max_slots=16)
    for i in range(n):
        assert toks[i] == [int(t) for t in g[f"gen{i}"]], i
    assert len(step_ms) == 32
    assert cache.num_free_pages() == 128  # every sequence freed its pages


def test_c1_greedy_with_arrivals(cbis, oracle):
    """Config 1's requests arriving over time (src/bench_batching.cpp:110-121:
    admitted once their arrival_ms has passed, the scheduler idling until the
    first arrives) with only 3 slots: every request's greedy tokens are still
    python/model.py's -- each row of a step is computed independently of the
    rows batched with it -- and each finishes after it arrives."""
    g = np.load(os.path.join(GOLDEN, "g2_c1_greedy.npz"))
    n = int(g["n"])
    prompts = [[int(t) for t in g[f"prompt{i}"]] for i in range(n)]
    cfg, w = _ref_model(cbis, vocab=512)
    cache = cbis.PagedKVCache(4, 128, 16, 8, 32, "f32")
    runner = cbis.TransformerRunner(w, cache, 512)
    arrivals = [5.0 + 2.0 * i for i in range(n)]
    toks, step_ms, fin = cbis.run_continuous(runner, cache, prompts, [32] * n, max_slots=3, arrival_ms=arrivals)
    for i in range(n):
        assert toks[i] == [int(t) for t in g[f"gen{i}"]], i
    assert all(f > a for f, a in zip(fin, arrivals))
    assert len(step_ms) > 32
    assert cache.num_free_pages() == 128


@pytest.mark.parametrize("chunk,budget", [(16, 0), (8, 40)])
def test_c1_chunked_prefill_greedy(cbis, oracle, chunk, budget):
    """Config 1's workload with the prompts fed in chunks (at most `chunk`
    rows per slot and `budget` prompt rows per step) beside the other slots'
    decode rows: the greedy tokens are still python/model.py's."""
    g = np.load(os.path.join(GOLDEN, "g2_c1_greedy.npz"))
    n = int(g["n"])
    prompts = [[int(t) for t in g[f"prompt{i}"]] for i in range(n)]
    cfg, w = _ref_model(cbis, vocab=512)
    cache = cbis.PagedKVCache(4, 128, 16, 8, 32, "f32")
    runner = cbis.TransformerRunner(w, cache, 512)
    toks, step_ms = cbis.run_continuous(runner, cache, prompts, [32] * n, max_slots=16, prefill_chunk=chunk,
                                        step_token_budget=budget)
    for i in range(n):
        assert toks[i] == [int(t) for t in g[f"gen{i}"]], i
    assert len(step_ms) > 32
    assert cache.num_free_pages() == 128


def test_c1_step_logits_match_golden(cbis, oracle):
    """Same workload driven step by step through forward_step: every
    generated step's last-row logits within 1e-4 of python/model.py."""
    g = np.load(os.path.join(GOLDEN, "g2_c1_greedy.npz"))
    n = int(g["n"])
    cfg, w = _ref_model(cbis, vocab=512)
    cache = cbis.PagedKVCache(4, 128, 16, 8, 32, "f32")
    runner = cbis.TransformerRunner(w, cache, 512)
    seqs = [cache.allocate_sequence() for _ in range(n)]
    prompts = [[int(t) for t in g[f"prompt{i}"]] for i in range(n)]
    tok, pos, sid, last = [], [], [], []
    for i, p in enumerate(prompts):
        for j, t in enumerate(p):
            assert cache.ensure_capacity(seqs[i], j)
            tok.append(t); pos.append(j); sid.append(seqs[i])
        last.append(len(tok) - 1)
    worst = 0.0
    nxt_pos = [len(p) for p in prompts]
    for step in range(32):
        lg = runner.forward_step(tok, pos, sid)
        rows = lg[last]
        for i in range(n):
            worst = max(worst, float(np.abs(rows[i] - g[f"logits{i}"][step]).max()))
        nxt = [int(g[f"gen{i}"][step]) for i in range(n)]  # teacher-forced on the golden tokens
        tok, pos, sid = [], [], []
        for i in range(n):
            assert cache.ensure_capacity(seqs[i], nxt_pos[i])
            tok.append(nxt[i]); pos.append(nxt_pos[i]); sid.append(seqs[i])
            nxt_pos[i] += 1
        last = list(range(n))
    assert worst < 1e-4, worst


_HIP = None


def _hip():
    global _HIP
    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so")
        _HIP.hipMemcpy.restype = ctypes.c_int
        _HIP.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return _HIP


def _d2h(dst_np, src_ptr):
    rc = _hip().hipMemcpy(dst_np.ctypes.data, src_ptr, dst_np.nbytes, 2)  # hipMemcpyDeviceToHost
    assert rc == 0


def _mid_setup(cbis, oracle, wdt, n_layers=2, max_pages=160):
    spec = oracle.ModelSpec(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=n_layers, mlp=8192,
                            max_seq=4096, weight_dtype=wdt, kv_dtype="bf16")
    cfg = cbis.ModelConfig.make(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=n_layers, mlp=8192,
                                max_seq=4096, weight_dtype=wdt, kv_dtype="bf16")
    w = cbis.ModelWeights.synthetic(cfg, seed=0)
    cache = cbis.PagedKVCache(n_layers, max_pages, 16, 64, 32, "bf16", pages_per_seq=256)
    cache.fill_normal(seed=99, std=1.0)  # synthetic cached K/V for positions before the step
    ow = oracle.synthetic_weights(spec, seed=0, pos_rows=4096)
    om = oracle.OracleModel(ow, max_pages=max_pages)
    for l in range(n_layers):
        _d2h(om.kpools[l], cache.k_base(l))
        _d2h(om.vpools[l], cache.v_base(l))
    return cfg, w, cache, om


@pytest.mark.parametrize("wdt", ["bf16", "fp8"])
def test_mid_size_mixed_step(cbis, oracle, wdt):
    """Config 4's step shape, reduced: full d=2048 / 64 heads / mlp 8192 /
    V=32000 model, 2 layers; 6 decode rows over synthetic cached K/V plus two
    prefill chunks (a fresh sequence and one with 48 cached tokens)."""
    cfg, w, cache, om = _mid_setup(cbis, oracle, wdt)
    ocache = oracle.PagedKVCacheOracle(160, pages_per_seq=256)
    runner = cbis.TransformerRunner(w, cache, 256)
    dec_kv = [300, 17, 1000, 640, 16, 129]
    tok, pos, sid, osid = [], [], [], []
    ids = oracle.uniform_int(5, 4001, 200, 0, 31999)
    k = 0
    for kv in dec_kv:  # decode rows: kv-1 cached tokens, query at position kv-1
        s, o = cache.allocate_sequence(), ocache.allocate_sequence()
        for p in range(kv):
            assert cache.ensure_capacity(s, p) and ocache.ensure_capacity(o, p)
        tok.append(int(ids[k])); pos.append(kv - 1); sid.append(s); osid.append(o); k += 1
    for cached, n in ((0, 40), (48, 37)):  # prefill chunks
        s, o = cache.allocate_sequence(), ocache.allocate_sequence()
        for p in range(cached + n):
            assert cache.ensure_capacity(s, p) and ocache.ensure_capacity(o, p)
        for p in range(cached, cached + n):
            tok.append(int(ids[k % 200])); pos.append(p); sid.append(s); osid.append(o); k += 1
    assert cache.pages(sid[0]) == ocache.seq_pages[osid[0]]  # identical allocation
    got = runner.forward_step(tok, pos, sid)
    ref = oracle.forward_step_with_cache(om, ocache, tok, pos, osid)
    err = row_rel_err(got, ref)
    assert err < 2e-2, err


def test_mid_size_step_one_pass_decode_rows(cbis, oracle):
    """The runner's one-pass decode attention: 192 decode rows (192 x 4 head
    blocks = 768 workgroups, no row over twice the mean length, as at config
    4) plus a prefill chunk, on the reduced config-4 model, against the
    oracle's forward."""
    cfg, w, cache, om = _mid_setup(cbis, oracle, "bf16", max_pages=1800)
    ocache = oracle.PagedKVCacheOracle(1800, pages_per_seq=256)
    runner = cbis.TransformerRunner(w, cache, 512)
    dec_kv = oracle.uniform_int(6, 4002, 192, 60, 110)
    tok, pos, sid, osid = [], [], [], []
    ids = oracle.uniform_int(6, 4003, 300, 0, 31999)
    k = 0
    for kv in dec_kv:
        kv = int(kv)
        s, o = cache.allocate_sequence(), ocache.allocate_sequence()
        assert cache.ensure_capacity(s, kv - 1) and ocache.ensure_capacity(o, kv - 1)
        tok.append(int(ids[k % 300])); pos.append(kv - 1); sid.append(s); osid.append(o); k += 1
    s, o = cache.allocate_sequence(), ocache.allocate_sequence()
    assert cache.ensure_capacity(s, 63) and ocache.ensure_capacity(o, 63)
    for p in range(16, 64):
        tok.append(int(ids[k % 300])); pos.append(p); sid.append(s); osid.append(o); k += 1
    got = runner.forward_step(tok, pos, sid)
    ref = oracle.forward_step_with_cache(om, ocache, tok, pos, osid)
    err = row_rel_err(got, ref)
    assert err < 2e-2, err


def test_fp8_decode_greedy_tokens(cbis, oracle):
    """Config 5's decode shape, reduced: fp8 weights, bf16 K/V, 4 sequences
    with long synthetic contexts, 4 greedy steps; tokens must match the
    oracle's wherever its top-2 margin exceeds the measured logit error."""
    cfg, w, cache, om = _mid_setup(cbis, oracle, "fp8", max_pages=600)
    ocache = oracle.PagedKVCacheOracle(600, pages_per_seq=256)
    runner = cbis.TransformerRunner(w, cache, 64)
    kvs = [2000, 1500, 4000 - 8, 900]
    seqs, oseqs = [], []
    for kv in kvs:
        s, o = cache.allocate_sequence(), ocache.allocate_sequence()
        for p in range(kv + 4):
            assert cache.ensure_capacity(s, p) and ocache.ensure_capacity(o, p)
        seqs.append(s); oseqs.append(o)
    toks = [int(t) for t in oracle.uniform_int(6, 4002, 4, 0, 31999)]
    for step in range(4):
        pos = [kv - 1 + step for kv in kvs]
        got = runner.forward_step(toks, pos, seqs)
        ref = oracle.forward_step_with_cache(om, ocache, toks, pos, oseqs)
        err = np.abs(got - ref).max(axis=1)
        assert row_rel_err(got, ref) < 2e-2
        srt = np.sort(ref, axis=1)
        margin = srt[:, -1] - srt[:, -2]
        g_tok = got.argmax(axis=1)
        r_tok = ref.argmax(axis=1)
        for i in range(4):
            if margin[i] > 2 * err[i]:
                assert g_tok[i] == r_tok[i], (step, i)
        toks = [int(t) for t in r_tok]  # teacher-force on the oracle's tokens


def test_graph_replay_matches_eager(cbis):
    """Steps replayed from a captured HIP graph give bit-identical logits to
    eager launches, across several replays with eager work in between."""
    cfg, w = _ref_model(cbis, vocab=512, n_layers=2, max_seq=512)
    cache = cbis.PagedKVCache(2, 64, 16, 8, 32, "f32", pages_per_seq=32)
    runner = cbis.TransformerRunner(w, cache, 64)
    seqs = [cache.allocate_sequence() for _ in range(4)]
    other = cache.allocate_sequence()
    for s in seqs + [other]:
        for p in range(40):
            assert cache.ensure_capacity(s, p)
    prompt_tok = list(range(10, 50))
    for s in seqs:  # fill K/V for positions 0..38
        runner.forward_step(prompt_tok[:39], list(range(39)), [s] * 39)
    step = ([1, 2, 3, 4], [39] * 4, seqs)
    runner.set_graphs(False)
    eager = runner.forward_step(*step)
    runner.set_graphs(True)
    outs = []
    for _ in range(3):
        outs.append(runner.forward_step(*step))       # graph replay
        runner.set_graphs(False)
        runner.forward_step(prompt_tok[:20], list(range(20)), [other] * 20)  # eager work in between
        runner.set_graphs(True)
    for o in outs:
        assert np.array_equal(o, eager)
    greedy = runner.forward_step_greedy(*step)
    assert greedy == [int(np.argmax(r)) for r in eager]


@pytest.mark.parametrize("wdt,kvdt,H", [("f32", "f32", 8), ("bf16", "bf16", 8), ("bf16", "bf16", 16)])
def test_fused_decode_matches_two_launches(cbis, wdt, kvdt, H):
    """Small all-decode steps run attention + out-projection as one launch
    per layer (cbis_paged_attention_proj); the same steps with the fusion
    off (two launches) give the same logits up to the projection's summation
    order and the same greedy tokens.  A step with prefill rows, or keys past
    768, takes the two launches either way."""
    cfg = cbis.ModelConfig.make(vocab=512, n_layers=2, weight_dtype=wdt, kv_dtype=kvdt, n_heads=H,
                                d_model=32 * H, max_seq=2048)
    w = cbis.ModelWeights.synthetic(cfg, seed=4)
    cache = cbis.PagedKVCache(2, 160, 16, H, 32, kvdt, pages_per_seq=64)
    runner = cbis.TransformerRunner(w, cache, 256)
    rng = np.random.default_rng(4)
    lens = [3, 17, 40, 64, 100]
    seqs = [cache.allocate_sequence() for _ in lens]
    for s, n in zip(seqs, lens):
        for p in range(n + 4):
            assert cache.ensure_capacity(s, p)
    tok = [int(t) for t in rng.integers(0, 512, sum(lens))]
    pos = [p for n in lens for p in range(n)]
    sid = [s for s, n in zip(seqs, lens) for _ in range(n)]
    runner.forward_step(tok, pos, sid)  # prefill
    assert runner.last_plan()["fused_attention_proj"] == 0
    dec = ([int(t) for t in rng.integers(0, 512, len(lens))], list(lens), seqs)
    runner.set_fused_decode(False)
    two = runner.forward_step(*dec)
    assert runner.last_plan()["fused_attention_proj"] == 0
    runner.set_fused_decode(True)
    one = runner.forward_step(*dec)  # rewrites the same K/V slots with the same values
    assert runner.last_plan()["fused_attention_proj"] == 1
    if wdt == "f32":
        assert np.abs(one - two).max() <= 1e-4 * max(1.0, float(np.abs(two).max()))
    else:  # a changed last bit can move a later bf16 rounding
        assert row_rel_err(one, two) < 1e-2
    assert runner.forward_step_greedy(*dec) == [int(np.argmax(r)) for r in one]
    assert runner.last_plan()["fused_attention_proj"] == 1
    # a row past 768 keys: two launches
    long = cache.allocate_sequence()
    assert cache.ensure_capacity(long, 1000)
    runner.forward_step([5], [1000], [long])
    assert runner.last_plan()["fused_attention_proj"] == 0


@pytest.mark.parametrize("wdt", ["bf16", "fp8", "f32"])
def test_packed_checkpoint_round_trip(cbis, tmp_path, wdt):
    """save_packed -> load_packed gives back the same config and the same
    device image (re-saving reproduces the file byte for byte), the same
    logits, and a flipped data byte fails the checksum."""
    kvdt = "f32" if wdt == "f32" else "bf16"
    H = 8 if wdt == "f32" else 16  # bf16 K/V pages are read in 16-head blocks
    cfg = cbis.ModelConfig.make(vocab=512, d_model=32 * H, n_heads=H, mlp=128 * H, n_layers=2, max_seq=1024,
                                weight_dtype=wdt, kv_dtype=kvdt)
    w = cbis.ModelWeights.synthetic(cfg, seed=5)
    p1, p2 = tmp_path / "a.cbisw", tmp_path / "b.cbisw"
    w.save_packed(str(p1))
    w2 = cbis.ModelWeights.load_packed(str(p1))
    assert [getattr(w2.cfg, f) for f, _ in cfg._fields_] == [getattr(cfg, f) for f, _ in cfg._fields_]
    assert w2.device_bytes() == w.device_bytes()
    w2.save_packed(str(p2))
    assert p1.read_bytes() == p2.read_bytes()
    ids = [int(t) for t in np.arange(37) * 13 % 512]
    outs = []
    for weights in (w, w2):
        cache = cbis.PagedKVCache(2, 16, 16, H, 32, kvdt, pages_per_seq=64)
        runner = cbis.TransformerRunner(weights, cache, 64)
        sid = cache.allocate_sequence()
        for q in range(len(ids)):
            cache.ensure_capacity(sid, q)
        outs.append(runner.forward_step(ids, list(range(len(ids))), [sid] * len(ids)))
        runner.close()
    assert np.array_equal(outs[0], outs[1])
    blob = bytearray(p1.read_bytes())
    blob[-100] ^= 0x40
    p2.write_bytes(bytes(blob))
    with pytest.raises(cbis.CbisError, match="checksum"):
        cbis.ModelWeights.load_packed(str(p2))


# --------------------------------------------------------------------------
# Whole steps at configs 4 and 5's own workloads (1-2 of their 16
# layers), the counterpart of src/correctness_check.cpp:55-94 (a full step
# diffed against the model).
# --------------------------------------------------------------------------

def _shuffle_free_lists(caches, n_pages, seed):
    """Hands every cache the same shuffled free list through the reference
    API alone (as bench.py does for configs 4 and 5): n_pages one-page
    sequences take pages 0..n-1 and are freed in a random order, so later
    allocations pop physical pages in that order."""
    perm = np.random.default_rng(seed).permutation(n_pages)
    for c in caches:
        dummies = []
        for _ in range(n_pages):
            s = c.allocate_sequence()
            assert c.ensure_capacity(s, 0)
            dummies.append(s)
        for i in perm:
            c.free_sequence(dummies[i])


def _big_setup(cbis, oracle, wdt, n_layers, max_pages, max_seq, fill_seed):
    spec = oracle.ModelSpec(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=n_layers, mlp=8192,
                            max_seq=max_seq, weight_dtype=wdt, kv_dtype="bf16")
    cfg = cbis.ModelConfig.make(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=n_layers, mlp=8192,
                                max_seq=max_seq, weight_dtype=wdt, kv_dtype="bf16")
    w = cbis.ModelWeights.synthetic(cfg, seed=0)
    cache = cbis.PagedKVCache(n_layers, max_pages, 16, 64, 32, "bf16", pages_per_seq=max_seq // 16)
    cache.fill_normal(seed=fill_seed, std=1.0)  # synthetic cached K/V for positions before the step
    om = oracle.OracleModel(oracle.synthetic_weights(spec, seed=0), max_pages=max_pages)
    for l in range(n_layers):
        _d2h(om.kpools[l], cache.k_base(l))
        _d2h(om.vpools[l], cache.v_base(l))
    ocache = oracle.PagedKVCacheOracle(max_pages, pages_per_seq=max_seq // 16)
    _shuffle_free_lists([cache, ocache], max_pages, fill_seed)
    return w, cache, om, ocache


def test_c4_step_at_config_workload(cbis, oracle):
    """Config 4's step exactly as bench.py builds it, on 2 of the 16
    layers: 192 decode rows with kv U[256, 4096] (the seed-0 draw) over a
    shuffled page table plus two 512-row prefill chunks (a fresh sequence at
    positions 0..511 and one with 512 cached tokens at 512..1023), M = 1216.
    The runner's one-pass decode rows, 64-row snake-ordered prefill tiles and
    the wave-specialised bf16 GEMMs at M = 1216 run as in the bench."""
    kv = oracle.uniform_int(0, 5001, 192, 256, 4096)
    max_pages = int(((kv + 15) // 16).sum()) + 32 + 64 + 64
    w, cache, om, ocache = _big_setup(cbis, oracle, "bf16", 2, max_pages, 4096, 1)
    runner = cbis.TransformerRunner(w, cache, 1216)
    toks = oracle.uniform_int(0, 5002, 1216, 0, 31999)
    tok, pos, sid, osid = [], [], [], []
    for i in range(192):
        s, o = cache.allocate_sequence(), ocache.allocate_sequence()
        assert cache.ensure_capacity(s, int(kv[i]) - 1) and ocache.ensure_capacity(o, int(kv[i]) - 1)
        tok.append(int(toks[i])); pos.append(int(kv[i]) - 1); sid.append(s); osid.append(o)
    for start in (0, 512):
        s, o = cache.allocate_sequence(), ocache.allocate_sequence()
        assert cache.ensure_capacity(s, start + 511) and ocache.ensure_capacity(o, start + 511)
        for p in range(start, start + 512):
            tok.append(int(toks[len(tok)])); pos.append(p); sid.append(s); osid.append(o)
    assert len(tok) == 1216
    for s, o in zip(sid, osid):
        assert cache.pages(s) == ocache.seq_pages[o]   # bit-exact allocation on the shuffled list
    got = runner.forward_step(tok, pos, sid)
    plan = runner.last_plan()
    assert plan["decode_rows"] == 192 and plan["prefill_tiles"] == 16 and plan["split_tokens"] == 1 << 30
    ref = oracle.forward_step_with_cache(om, ocache, tok, pos, osid)
    _check_logits(got, ref, "config 4 step (2 layers)")
    # The greedy form of the same step (lm_head fused with the row argmax, no
    # logits stored): the argmax and top-2 margin of the same logits, bit for bit.
    greedy = runner.forward_step_greedy(tok, pos, sid)
    assert greedy == [int(t) for t in oracle.argmax_rows(got)]
    m = runner.last_margins()
    srt = np.sort(got, axis=1)
    assert np.array_equal(m, (srt[:, -1] - srt[:, -2]).astype(np.float32))


def test_c5_decode_at_config_workload(cbis, oracle):
    """Config 5's decode on 1 of the 16 layers: fp8-e4m3 weights
    with per-channel scales, bf16 K/V, 16 sequences whose caches hold 32704
    synthetic tokens, greedy steps at positions 32704, 32705, 32706 through
    the runner's own split choice (8192-token splits: one CU's share of the
    rows' tokens) and the skinny fp8 GEMMs; teacher-forced on the oracle's
    tokens."""
    n_seq, ctx = 16, 32768 - 64
    max_pages = n_seq * 2048 + 64
    w, cache, om, ocache = _big_setup(cbis, oracle, "fp8", 1, max_pages, 32768, 5)
    runner = cbis.TransformerRunner(w, cache, 64)
    seqs, oseqs = [], []
    for _ in range(n_seq):
        s, o = cache.allocate_sequence(), ocache.allocate_sequence()
        assert cache.ensure_capacity(s, 32767) and ocache.ensure_capacity(o, 32767)
        assert cache.pages(s) == ocache.seq_pages[o]
        seqs.append(s); oseqs.append(o)
    toks = [int(t) for t in oracle.uniform_int(0, 5003, n_seq, 0, 31999)]
    for step in range(3):
        pos = [ctx + step] * n_seq
        got = runner.forward_step(toks, pos, seqs)
        assert len(runner.last_margins()) == 0  # the previous greedy step's margins are gone
        assert runner.last_plan()["split_tokens"] == 8192
        ref = oracle.forward_step_with_cache(om, ocache, toks, pos, oseqs)
        want = _check_logits(got, ref, f"config 5 step {step} (1 layer)")
        # the greedy step as bench.py runs it (fused fp8 lm_head + argmax):
        # the argmax and top-2 margin of the same logits, bit for bit
        assert runner.forward_step_greedy(toks, pos, seqs) == [int(t) for t in oracle.argmax_rows(got)]
        srt = np.sort(got, axis=1)
        assert np.array_equal(runner.last_margins(), (srt[:, -1] - srt[:, -2]).astype(np.float32))
        toks = [int(t) for t in want]


def test_runner_split_kv_decode_rows_with_prefill(cbis, oracle):
    """The runner's split sizing for decode rows that cannot fill the GPU in
    one pass but carry >= 2048 tokens per CU: 24 rows at kv U[7000, 8192]
    (one CU's share ~2850 tokens) get power-of-two 4096-token splits, two per
    row, whose merge runs inside the prefill launch of the step's 100-row
    chunk; 2 of the 16 layers of the config-4 model, shuffled page table."""
    kv = oracle.uniform_int(3, 4101, 24, 7000, 8192)
    max_pages = int(((kv + 15) // 16).sum()) + 16 + 64
    w, cache, om, ocache = _big_setup(cbis, oracle, "bf16", 2, max_pages, 8192, 3)
    runner = cbis.TransformerRunner(w, cache, 256)
    ids = oracle.uniform_int(3, 4102, 200, 0, 31999)
    tok, pos, sid, osid = [], [], [], []
    for i, k in enumerate(kv):
        s, o = cache.allocate_sequence(), ocache.allocate_sequence()
        assert cache.ensure_capacity(s, int(k) - 1) and ocache.ensure_capacity(o, int(k) - 1)
        tok.append(int(ids[i])); pos.append(int(k) - 1); sid.append(s); osid.append(o)
    s, o = cache.allocate_sequence(), ocache.allocate_sequence()
    assert cache.ensure_capacity(s, 139) and ocache.ensure_capacity(o, 139)
    for p in range(40, 140):
        tok.append(int(ids[len(tok)])); pos.append(p); sid.append(s); osid.append(o)
    got = runner.forward_step(tok, pos, sid)
    plan = runner.last_plan()
    assert plan["decode_rows"] == 24 and plan["prefill_tiles"] == 2 and plan["split_tokens"] == 4096, plan
    assert (kv > 4096).sum() >= 20   # most rows take two splits and the merge
    ref = oracle.forward_step_with_cache(om, ocache, tok, pos, osid)
    _check_logits(got, ref, "split-KV decode rows + prefill chunk (2 layers)")


@pytest.mark.parametrize("wdt,kvdt,H", [("f32", "f32", 12), ("bf16", "bf16", 8), ("bf16", "bf16", 20)])
def test_runner_any_head_count(cbis, oracle, wdt, kvdt, H):
    """Head counts that leave the attention kernels' last 1 KiB head block
    partial (8 fp32 / 16 bf16 heads per block): a step with a prefill chunk
    and decode rows, then a decode step, against the oracle."""
    D = 32 * H
    spec = oracle.ModelSpec(vocab=512, d_model=D, n_heads=H, n_layers=2, mlp=4 * D, max_seq=512, weight_dtype=wdt,
                            kv_dtype=kvdt)
    cfg = cbis.ModelConfig.make(vocab=512, d_model=D, n_heads=H, n_layers=2, mlp=4 * D, max_seq=512, weight_dtype=wdt,
                                kv_dtype=kvdt)
    w = cbis.ModelWeights.synthetic(cfg, seed=2)
    cache = cbis.PagedKVCache(2, 64, 16, H, 32, kvdt, pages_per_seq=32)
    runner = cbis.TransformerRunner(w, cache, 128)
    om = oracle.OracleModel(oracle.synthetic_weights(spec, seed=2), max_pages=64)
    ocache = oracle.PagedKVCacheOracle(64, pages_per_seq=32)
    lens = [50, 3, 20]
    seqs, oseqs = [], []
    tok, pos, sid, osid = [], [], [], []
    ids = oracle.uniform_int(2, 77, 100, 0, 511)
    for n in lens:
        s, o = cache.allocate_sequence(), ocache.allocate_sequence()
        seqs.append(s); oseqs.append(o)
        for p in range(n):
            assert cache.ensure_capacity(s, p) and ocache.ensure_capacity(o, p)
            tok.append(int(ids[len(tok)])); pos.append(p); sid.append(s); osid.append(o)
    tol = (lambda g, r: float(np.abs(g - r).max()) < 1e-4) if wdt == "f32" else \
        (lambda g, r: row_rel_err(g, r) < 2e-2)
    got = runner.forward_step(tok, pos, sid)
    ref = oracle.forward_step_with_cache(om, ocache, tok, pos, osid)
    assert tol(got, ref)
    dpos = list(lens)
    for s, o, q in zip(seqs, oseqs, dpos):
        assert cache.ensure_capacity(s, q) and ocache.ensure_capacity(o, q)
    nxt = [1, 2, 3]
    got = runner.forward_step(nxt, dpos, seqs)
    ref = oracle.forward_step_with_cache(om, ocache, nxt, dpos, oseqs)
    assert tol(got, ref)


def test_weights_bin_loader_reproduces_model_py(cbis, oracle, tmp_path):
    """ModelWeights::load (src/model_weights.cpp:41-75) on a weights.bin
    written in python/export_weights.py:42-66 order from the seed-0 weights
    of the reference dims: the G1 batch of src/correctness_check.cpp gives
    python/model.py's logits (tests/golden/g1_refmodel.npz) within 1e-4, and
    the same logits bit for bit as the synthetic weights it was written from."""
    from helpers import write_weights_bin
    g = np.load(os.path.join(GOLDEN, "g1_refmodel.npz"))
    path = tmp_path / "weights.bin"
    write_weights_bin(path, oracle.synthetic_weights(oracle.ModelSpec(), seed=0))
    cfg, w_syn = _ref_model(cbis)
    w_bin = cbis.ModelWeights.load(str(path), cfg)
    assert w_bin.device_bytes() == w_syn.device_bytes()
    outs = {}
    for name, w in (("bin", w_bin), ("syn", w_syn)):
        cache = cbis.PagedKVCache(4, 8 * 6 + 8, 16, 8, 32, "f32", pages_per_seq=2048)
        runner = cbis.TransformerRunner(w, cache, 128)
        res = []
        for i in range(len(g["lens"])):
            ids = [int(t) for t in g[f"ids{i}"]]
            s = cache.allocate_sequence()
            for p in range(len(ids)):
                assert cache.ensure_capacity(s, p)
            res.append(runner.forward_step(ids, list(range(len(ids))), [s] * len(ids)))
            cache.free_sequence(s)
        outs[name] = res
        runner.close()
        cache.close()
    worst = 0.0
    for i in range(len(g["lens"])):
        assert np.array_equal(outs["bin"][i], outs["syn"][i])
        worst = max(worst, float(np.abs(outs["bin"][i] - g[f"logits{i}"]).max()))
    print(f"weights.bin G1 max abs vs model.py {worst:.3e}", flush=True)
    assert worst < 1e-4, worst
