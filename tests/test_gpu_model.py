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

from helpers import bits_u16, row_rel_err

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
    """8 prompts U[16,64], 32 greedy tokens each through
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



def test_runner_rejects_unsupported_head_blocks(cbis):
    """bf16 K/V pages are read in 16-head blocks: an 8-head bf16 model is
    refused when the runner is built, not in the middle of a step."""
    cfg = cbis.ModelConfig.make(vocab=512, n_layers=1, max_seq=1024, weight_dtype="bf16", kv_dtype="bf16")
    w = cbis.ModelWeights.synthetic(cfg, seed=1)
    cache = cbis.PagedKVCache(1, 8, 16, 8, 32, "bf16", pages_per_seq=64)
    with pytest.raises(cbis.CbisError, match="n_heads a multiple"):
        cbis.TransformerRunner(w, cache, 16)
