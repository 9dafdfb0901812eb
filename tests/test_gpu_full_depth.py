"""Whole steps at full depth: bench.py's own config 4 step and config 5
decode on all 16 layers of the mid-size GPT, against the CPU oracle run one
layer at a time (each layer's K/V pools copied to the host only while that
layer runs: 3.6 GB for config 4, 4.3 GB for config 5, where the whole
16-layer set is 57 / 69 GB).  The counterpart of the reference's
correctness harness, which diffs the whole model's logits
(src/correctness_check.cpp:55-94).

Bar: per row ||d||_inf / ||ref||_inf <= 2e-2 over the logits,
greedy tokens equal wherever the oracle's top-2 margin exceeds twice the
row's measured error, the fused greedy path's tokens and margins bit-equal
to the argmax and top-2 of the full logits.
"""
import ctypes
import importlib.util
import os
import sys
import time

import numpy as np
import pytest

from helpers import check_logits

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("cbis_bench", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _progress(msg):
    # straight to the terminal (pytest captures stdout): a full-depth check
    # spends a minute on the host cores and says where it is
    print(msg, file=sys.__stderr__, flush=True)


class _LayerPools:
    """Host copies of one layer's K and V pools at a time (bf16 bits)."""

    def __init__(self, cache):
        self.cache = cache
        shape = (cache.max_pages(), 16, 64, 32)
        self.k = np.empty(shape, np.uint16)
        self.v = np.empty(shape, np.uint16)
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]

    def load(self, l):
        for dst, src in ((self.k, self.cache.k_base(l)), (self.v, self.cache.v_base(l))):
            assert self.hip.hipMemcpy(dst.ctypes.data, src, dst.nbytes, 2) == 0  # device to host
        return self.k, self.v


def _check_greedy(runner, tokens, got):
    """The fused greedy step's tokens and margins against the full logits."""
    srt = np.sort(got, axis=1)
    first_max = [int(i) for i in np.argmax(got, axis=1)]  # numpy's argmax keeps the first maximum
    assert tokens == first_max
    assert np.array_equal(runner.last_margins(), (srt[:, -1] - srt[:, -2]).astype(np.float32))


@pytest.mark.timeout(900)
def test_c4_step_full_depth(cbis, oracle):
    """bench.py's config 4 step exactly (c4_setup: 192 decode rows at kv
    U[256, 4096], two 512-row prefill chunks, shuffled page table, M = 1216)
    through all 16 layers: forward_step's logits against the oracle, and
    forward_step_greedy -- the call bench.py times -- against those logits."""
    bench = _bench()
    t0 = time.time()
    st = bench.c4_setup(cbis, oracle)
    runner, cache = st["runner"], st["cache"]
    tok, pos, sid = st["tok"], st["pos"], st["sid"]
    got = runner.forward_step(tok, pos, sid)
    plan = runner.last_plan()
    assert plan["decode_rows"] == 192 and plan["prefill_tiles"] == 16 and plan["split_tokens"] == 1 << 30
    _check_greedy(runner, runner.forward_step_greedy(tok, pos, sid), got)
    _progress(f"c4 full depth: GPU step done ({time.time() - t0:.0f}s)")
    spec = oracle.ModelSpec(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=16, mlp=8192,
                            max_seq=32768, weight_dtype="bf16", kv_dtype="bf16")
    om = oracle.OracleModel(oracle.synthetic_weights(spec, seed=0, pos_rows=max(pos) + 1), max_pages=1)
    _progress(f"c4 full depth: oracle weights ready ({time.time() - t0:.0f}s)")
    wpage, woff, bt, row_bt = oracle.step_tables(cache, tok, pos, sid)
    pools = _LayerPools(cache)
    x = om.embed(tok, pos)
    for l in range(16):
        kp, vp = pools.load(l)
        om.layer(l, x, pos, wpage, woff, bt, row_bt, kp, vp)
        _progress(f"c4 full depth: oracle layer {l} ({time.time() - t0:.0f}s)")
    ref = om.head(x)
    check_logits(got, ref, "config 4 step (16 layers)")


@pytest.mark.timeout(900)
def test_c5_decode_full_depth(cbis, oracle):
    """bench.py's config 5 decode (c5_setup: fp8 weights, 16 sequences at
    kv 32704, bf16 K/V, 8192-token splits) through all 16 layers for 4
    free-running greedy steps: each step feeds the GPU's own tokens of the
    step before, as run_c5 does.  The oracle is given the same tokens and
    its logits are compared at every step; where a row's margin is
    decisive its argmax is the GPU's token, so the free-running sequence is
    the oracle's own."""
    bench = _bench()
    t0 = time.time()
    st = bench.c5_setup(cbis, oracle)
    runner, cache, seqs = st["runner"], st["cache"], st["seqs"]
    n_seq, ctx, T = st["n_seq"], st["ctx"], 4
    toks = st["first"]
    steps = []
    for t in range(T):
        pos = [ctx + t] * n_seq
        got = runner.forward_step(toks, pos, seqs)
        assert runner.last_plan()["split_tokens"] == 8192
        nxt = runner.forward_step_greedy(toks, pos, seqs)  # the call run_c5 times
        _check_greedy(runner, nxt, got)
        steps.append((toks, pos, got))
        toks = nxt
    _progress(f"c5 full depth: {T} GPU steps done ({time.time() - t0:.0f}s)")
    spec = oracle.ModelSpec(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=16, mlp=8192,
                            max_seq=32768, weight_dtype="fp8", kv_dtype="bf16")
    om = oracle.OracleModel(oracle.synthetic_weights(spec, seed=0, pos_rows=ctx + T), max_pages=1)
    _progress(f"c5 full depth: oracle weights ready ({time.time() - t0:.0f}s)")
    # Layer by layer, every step of the layer in order: step t writes its
    # K/V at position ctx + t before attending, so later steps see the
    # oracle's own K/V of the earlier ones (the GPU's are overwritten).
    tables = [oracle.step_tables(cache, tk, ps, seqs) for tk, ps, _ in steps]
    xs = [om.embed(tk, ps) for tk, ps, _ in steps]
    pools = _LayerPools(cache)
    for l in range(16):
        kp, vp = pools.load(l)
        for t, (tk, ps, _) in enumerate(steps):
            om.layer(l, xs[t], ps, *tables[t], kp, vp)
        _progress(f"c5 full depth: oracle layer {l} ({time.time() - t0:.0f}s)")
    for t, (tk, ps, got) in enumerate(steps):
        check_logits(got, om.head(xs[t]), f"config 5 step {t} (16 layers, free-running)")
