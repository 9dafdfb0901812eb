"""Pins the CPU oracle (oracle/) before it is trusted as the checker:
golden vectors written from the reference's python/model.py, library
routines (numpy / torch on the CPU), closed forms, and exhaustive codec
checks.  Each check is chosen so a plausible slip (dropped bias, transposed
weight, wrong variance, wrong scale, off-by-one causal bound) fails it."""
import math
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
REF_WEIGHTS = "/root/reference/python/weights.bin"


def _prefill(oracle, om, ids):
    cache = oracle.PagedKVCacheOracle(om.kpools[0].shape[0])
    sid = cache.allocate_sequence()
    for p in range(len(ids)):
        assert cache.ensure_capacity(sid, p)
    return oracle.forward_step_with_cache(om, cache, list(ids), list(range(len(ids))), [sid] * len(ids))


def test_g1_oracle_matches_model_py(oracle):
    g = np.load(os.path.join(GOLDEN, "g1_refmodel.npz"))
    w = oracle.synthetic_weights(oracle.ModelSpec(), seed=0, pos_rows=64)
    om = oracle.OracleModel(w, max_pages=8)
    for i in range(len(g["lens"])):
        lg = _prefill(oracle, om, g[f"ids{i}"])
        assert np.abs(lg - g[f"logits{i}"]).max() < 1e-5


def test_g1_oracle_layer_by_layer(oracle):
    """The step run one layer at a time (orc_step_embed / orc_step_layer /
    orc_step_head, each layer given its own pools, as the full-depth GPU
    checks run it) against model.py's golden logits, and bit-identical to
    the whole-step call."""
    g = np.load(os.path.join(GOLDEN, "g1_refmodel.npz"))
    w = oracle.synthetic_weights(oracle.ModelSpec(), seed=0, pos_rows=64)
    for i in range(len(g["lens"])):
        ids = [int(t) for t in g[f"ids{i}"]]
        pos = list(range(len(ids)))
        whole = _prefill(oracle, oracle.OracleModel(w, max_pages=8), ids)
        om = oracle.OracleModel(w, max_pages=8)
        cache = oracle.PagedKVCacheOracle(8)
        sid = cache.allocate_sequence()
        for p in pos:
            assert cache.ensure_capacity(sid, p)
        wpage, woff, bt, row_bt = oracle.step_tables(cache, ids, pos, [sid] * len(ids))
        x = om.embed(ids, pos)
        for l in range(om.spec.n_layers):
            om.layer(l, x, pos, wpage, woff, bt, row_bt, om.kpools[l], om.vpools[l])
        lg = om.head(x)
        assert np.array_equal(lg, whole)
        assert np.abs(lg - g[f"logits{i}"]).max() < 1e-5


@pytest.mark.skipif(not os.path.exists(REF_WEIGHTS), reason="reference weights.bin not present")
def test_g1_oracle_matches_reference_weights_bin(oracle):
    """The reference's own weights.bin and export_reference batch (seed 777):
    the content of the reference.bin that src/correctness_check.cpp reads."""
    g = np.load(os.path.join(GOLDEN, "g1_weightsbin.npz"))
    w = oracle.load_weights_bin(REF_WEIGHTS, oracle.ModelSpec())
    om = oracle.OracleModel(w, max_pages=8)
    worst = 0.0
    for i in range(len(g["lens"])):
        worst = max(worst, float(np.abs(_prefill(oracle, om, g[f"ids{i}"]) - g[f"logits{i}"]).max()))
    assert worst < 5e-3  # the reference's own gate, src/correctness_check.cpp:88
    assert worst < 1e-5


def test_g2_c1_greedy_oracle(oracle):
    """Config 1 through the oracle's restatement of run_continuous with
    incremental paged attention == python/model.py's full recompute."""
    g = np.load(os.path.join(GOLDEN, "g2_c1_greedy.npz"))
    spec = oracle.ModelSpec(vocab=512)
    w = oracle.synthetic_weights(spec, seed=0, pos_rows=128)
    om = oracle.OracleModel(w, max_pages=128)
    cache = oracle.PagedKVCacheOracle(128)
    reqs = oracle.c1_requests(0)
    for i, r in enumerate(reqs):
        assert r.prompt == [int(t) for t in g[f"prompt{i}"]]
    gen, logs = oracle.run_continuous(om, cache, reqs, record_logits=True)
    for i in range(len(reqs)):
        assert gen[i] == [int(t) for t in g[f"gen{i}"]]
    worst = max(float(np.abs(row - g[f"logits{r}"][s]).max()) for s, rec in enumerate(logs) for r, row in rec.items())
    assert worst < 1e-5


@pytest.mark.parametrize("wdt", ["bf16", "fp8"])
def test_g3_mid_size_oracle(oracle, wdt):
    """Reduced mid-size GPT with bf16 / fp8 weights: the oracle without
    activation rounding matches python/model.py (fp16-stored logits); with the
    product's bf16 rounding points it stays inside the 2e-2 relative bound."""
    g = np.load(os.path.join(GOLDEN, f"g3_mid_{wdt}.npz"))
    for act in (False, True):
        spec = oracle.ModelSpec(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=2, mlp=8192,
                                max_seq=16, weight_dtype=wdt, kv_dtype="bf16" if act else "f32")
        w = oracle.synthetic_weights(spec, seed=0, pos_rows=16)
        om = oracle.OracleModel(w, max_pages=4)
        om._mdl.act_bf16 = int(act)
        for i in range(len(g["lens"])):
            lg = _prefill(oracle, om, g[f"ids{i}"])[g[f"rows{i}"]]
            ref = g[f"logits{i}"].astype(np.float64)
            rel = (np.abs(lg - ref).max(axis=1) / np.abs(ref).max(axis=1)).max()
            assert rel < (2e-2 if act else 1e-3), (act, rel)


def test_gemm_pins(oracle):
    rng = np.random.default_rng(0)
    # exact small-integer products: fp64 accumulation is exact
    X = rng.integers(-8, 8, (17, 64)).astype(np.float32)
    W = rng.integers(-8, 8, (33, 64)).astype(np.float32)
    b = rng.integers(-8, 8, 33).astype(np.float32)
    R = rng.integers(-8, 8, (17, 33)).astype(np.float32)
    Y = oracle.gemm(X, W, bias=b, residual=R)
    assert np.array_equal(Y, X.astype(np.int64) @ W.T.astype(np.int64) + b + R)
    # per-channel scale, transposed-operand slips
    s = rng.uniform(0.5, 2, 33).astype(np.float32)
    assert np.allclose(oracle.gemm(X, W, w_scale=s), (X @ W.T) * s)
    # GELU epilogue == torch's exact-erf gelu (python/model.py:50)
    import torch
    Xf = rng.standard_normal((9, 32)).astype(np.float32)
    Wf = rng.standard_normal((11, 32)).astype(np.float32)
    z = torch.from_numpy(Xf).double() @ torch.from_numpy(Wf).double().T
    assert np.allclose(oracle.gemm(Xf, Wf, gelu=True), torch.nn.functional.gelu(z).numpy(), atol=1e-12)


def test_gemm_sums_each_output_in_k_order(oracle):
    """orc_gemm runs blocks of outputs side by side on fp64 vectors; every
    output must still be the plain loop's fp64 sum over k in order (bit for
    bit), including ragged row and column blocks, K = 0 and the epilogues."""
    import math
    rng = np.random.default_rng(5)
    for M, N, K in ((1, 1, 1), (3, 5, 7), (6, 9, 33), (4, 8, 0), (9, 17, 70)):
        X = rng.standard_normal((M, K)).astype(np.float32)
        W = rng.standard_normal((N, K)).astype(np.float32)
        s = rng.uniform(0.5, 2, N).astype(np.float32)
        b = rng.standard_normal(N).astype(np.float32)
        R = rng.standard_normal((M, N)).astype(np.float32)
        for kw in ({}, {"w_scale": s, "bias": b, "gelu": True, "residual": R}):
            got = oracle.gemm(X, W, **kw)
            for m in range(M):
                for n in range(N):
                    acc = 0.0
                    for k in range(K):
                        acc += float(X[m, k]) * float(W[n, k])
                    if kw:
                        acc = acc * float(s[n]) + float(b[n])
                        acc = 0.5 * acc * (1.0 + math.erf(acc * 0.70710678118654752440)) + float(R[m, n])
                    assert got[m, n] == acc, (M, N, K, m, n, kw != {})


def test_layernorm_pins(oracle):
    import torch
    rng = np.random.default_rng(1)
    X = (rng.standard_normal((7, 256)) * 3 + 2).astype(np.float32)
    g = rng.standard_normal(256).astype(np.float32)
    b = rng.standard_normal(256).astype(np.float32)
    ref = torch.nn.functional.layer_norm(torch.from_numpy(X).double(), (256,), torch.from_numpy(g).double(),
                                         torch.from_numpy(b).double(), eps=1e-5)
    assert np.allclose(oracle.layernorm(X, g, b), ref.numpy(), atol=1e-10)
    # constant row -> beta
    assert np.allclose(oracle.layernorm(np.full((1, 256), 3.0, np.float32), g, b)[0], b)


def _dense_attention(q, k, v):
    """Tiny dense causal softmax(q k^T / sqrt(hd)) v per head, via torch on CPU."""
    import torch
    q, k, v = (torch.from_numpy(a).double() for a in (q, k, v))
    s = (q @ k.transpose(-1, -2)) / math.sqrt(q.shape[-1])
    T = q.shape[-2]
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    return (torch.softmax(s, -1) @ v).numpy()


def test_attention_pins(oracle):
    rng = np.random.default_rng(2)
    H, hd, T, P = 2, 32, 40, 8
    q = rng.standard_normal((T, H * hd)).astype(np.float32)
    kv_k = rng.standard_normal((T, H, hd)).astype(np.float32)
    kv_v = rng.standard_normal((T, H, hd)).astype(np.float32)
    table = np.array([6, 1, 3], np.int32)  # non-identity physical pages
    kp = np.zeros((P, 16, H, hd), np.float32)
    vp = np.zeros_like(kp)
    for j in range(T):
        kp[table[j // 16], j % 16] = kv_k[j]
        vp[table[j // 16], j % 16] = kv_v[j]
    out = oracle.paged_attention(q, kp, vp, np.repeat(table[None], T, 0), np.arange(T), H, hd, 16)
    dense = _dense_attention(q.reshape(T, H, hd).transpose(1, 0, 2), kv_k.transpose(1, 0, 2), kv_v.transpose(1, 0, 2))
    assert np.allclose(out.reshape(T, H, hd), dense.transpose(1, 0, 2), atol=1e-12)
    # kv_len = 1 -> v0 exactly; a dominant key -> its value
    assert np.array_equal(out[0].reshape(H, hd), kv_v[0])
    q2 = np.zeros((1, H * hd), np.float32)
    kp2, vp2 = kp.copy(), vp.copy()
    kp2[table[0], 5] = 0.0
    q2[0, :] = 50.0
    kp2[table[0], 5, :, :] = 1.0  # key 5 dominates (score 50*32/sqrt(32))
    o2 = oracle.paged_attention(q2, kp2, vp2, table[None], np.array([30]), H, hd, 16)
    assert np.allclose(o2.reshape(H, hd), vp2[table[0], 5], atol=1e-6)
    # permuting physical pages (with the table) changes nothing
    perm = np.array([3, 0, 7, 6, 5, 4, 1, 2])
    inv = np.argsort(perm)
    out_p = oracle.paged_attention(q, kp[perm], vp[perm], np.repeat(inv[table][None], T, 0), np.arange(T), H, hd, 16)
    assert np.array_equal(out, out_p)


def test_bf16_codec_matches_torch(oracle):
    import torch
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10,
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 0.0, -0.0, 3.3e38], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16_bits(x), ref)


def test_e4m3_codec_exhaustive(oracle):
    """OCP e4m3 decode of all 256 codes equals torch.float8_e4m3fn; RNE
    encode round-trips every finite code and matches torch in range; the
    scalar and vectorised encoders agree."""
    import torch
    codes = np.arange(256, dtype=np.uint8)
    tab = oracle.e4m3_table()
    tref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    finite = ~np.isnan(tref)
    assert np.array_equal(tab[finite], tref[finite]) and np.isnan(tab[~finite]).all()
    assert np.array_equal(oracle.f32_to_e4m3(tab[finite]), codes[finite])
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(20000) * rng.choice([1e-3, 0.05, 1, 30, 200], 20000)).astype(np.float32)
    x = np.clip(x, -447.9, 447.9)
    mids = ((tab[1:0x7E] + tab[2:0x7F]) / 2).astype(np.float32)  # exact ties between neighbours
    x = np.concatenate([x, mids, -mids])
    ours = oracle.f32_to_e4m3(x)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs)
    assert np.array_equal(oracle._e4m3_encode_vec(x), ours)
    assert oracle.f32_to_e4m3(np.array([1000.0, -1000.0], np.float32)).tolist() == [0x7E, 0xFE]
    # per-channel absmax quantisation: the C rows (OpenMP) and numpy agree,
    # including an all-zero row (scale 1) and a row whose max sits at a tie
    w = (rng.standard_normal((64, 300)) * 0.02).astype(np.float32)
    w[3] = 0.0
    w[5, 7] = np.float32(1.0)
    c_codes, c_scale = oracle.quantize_e4m3_rows(w)
    n_codes, n_scale = oracle.quantize_e4m3_rows_np(w)
    assert np.array_equal(c_codes, n_codes) and np.array_equal(c_scale.view(np.uint32), n_scale.view(np.uint32))
    assert c_scale[3] == 1.0 and (c_codes[3] == 0).all()
    dq = oracle.e4m3_table()[c_codes] * c_scale[:, None]
    assert np.allclose(np.abs(dq).max(axis=1)[np.arange(64) != 3], np.abs(w).max(axis=1)[np.arange(64) != 3],
                       rtol=1e-6)


def test_prng_spec(oracle):
    """The documented generator: counter-based, start offsets compose, and
    the Irwin-Hall(12) values have mean 0 / variance 1 and bounded support."""
    a = oracle.normal(0, 7, 1000)
    b = oracle.normal(0, 7, 500, start=500)
    assert np.array_equal(a[500:], b)
    z = oracle.normal(1, 9, 400000)
    assert abs(z.mean()) < 0.01 and abs(z.var() - 1.0) < 0.01 and np.abs(z).max() <= 6.0
    u = oracle.uniform_int(0, 3, 10000, 16, 64)
    assert u.min() == 16 and u.max() == 64


def _torch_cpu(oracle):
    import importlib.util
    spec = importlib.util.spec_from_file_location("torch_cpu", os.path.join(os.path.dirname(oracle.__file__),
                                                                            "torch_cpu.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_torch_cpu_step_matches_model_py(oracle):
    """The fp32 PyTorch CPU step (the cpu_baseline's forward) reproduces
    python/model.py's G1 logits through the paged pools."""
    tc = _torch_cpu(oracle)
    g = np.load(os.path.join(GOLDEN, "g1_refmodel.npz"))
    w = oracle.synthetic_weights(oracle.ModelSpec(), seed=0, pos_rows=64)
    for i in range(len(g["lens"])):
        ids = g[f"ids{i}"]
        kp = [np.zeros((8, 16, 8, 32), np.float32) for _ in range(4)]
        vp = [np.zeros((8, 16, 8, 32), np.float32) for _ in range(4)]
        cache = oracle.PagedKVCacheOracle(8)
        sid = cache.allocate_sequence()
        for p in range(len(ids)):
            assert cache.ensure_capacity(sid, p)
        pos = list(range(len(ids)))
        wp, wo, bt, rb = oracle.step_tables(cache, list(ids), pos, [sid] * len(ids))
        lg = tc.TorchCpuStep(w, kp, vp).forward_step(ids, pos, wp, wo, bt, rb).double().numpy()
        assert np.abs(lg - g[f"logits{i}"]).max() < 2e-5


@pytest.mark.parametrize("wdt", ["f32", "bf16", "fp8"])
def test_torch_cpu_step_matches_c_oracle(oracle, wdt):
    """A mixed step -- 5 decode rows over cached keys and a 20-row prefill
    chunk after 9 cached tokens, shuffled pages -- through the fp32 PyTorch
    CPU step and the fp64 C oracle: same K/V written, logits within fp32
    rounding (f32 model) or the bf16 bound."""
    tc = _torch_cpu(oracle)
    spec = oracle.ModelSpec(vocab=512, d_model=256, n_heads=8, head_dim=32, n_layers=2, mlp=1024, max_seq=256,
                            weight_dtype=wdt, kv_dtype="f32" if wdt == "f32" else "bf16")
    w = oracle.synthetic_weights(spec, seed=3, pos_rows=256)
    P = 64
    cache = oracle.PagedKVCacheOracle(P)
    rng = np.random.default_rng(7)
    rng.shuffle(cache.free)  # pages handed out in a random order
    tok, pos, sid = [], [], []
    for kv in (17, 40, 1, 96, 63):
        s = cache.allocate_sequence()
        assert cache.ensure_capacity(s, kv - 1)
        tok.append(int(rng.integers(0, 512))); pos.append(kv - 1); sid.append(s)
    s = cache.allocate_sequence()
    assert cache.ensure_capacity(s, 28)
    for p in range(9, 29):
        tok.append(int(rng.integers(0, 512))); pos.append(p); sid.append(s)
    om = oracle.OracleModel(w, max_pages=P)
    for pools in (om.kpools, om.vpools):
        for a in pools:
            vals = rng.standard_normal(a.shape).astype(np.float32)
            a[...] = vals if a.dtype == np.float32 else oracle.f32_to_bf16_bits(vals)
    kp = [a.copy() for a in om.kpools]
    vp = [a.copy() for a in om.vpools]
    wp, wo, bt, rb = oracle.step_tables(cache, tok, pos, sid)
    ref = om.forward_step(tok, pos, wp, wo, bt, rb)
    lg = tc.TorchCpuStep(w, kp, vp).forward_step(tok, pos, wp, wo, bt, rb).double().numpy()
    rel = (np.abs(lg - ref).max(axis=1) / np.abs(ref).max(axis=1)).max()
    assert rel < (1e-4 if wdt == "f32" else 2e-2), rel
    for l in range(2):  # the step's own K/V slots, as written by each
        for mine, theirs in ((kp[l], om.kpools[l]), (vp[l], om.vpools[l])):
            a = mine.astype(np.float64) if wdt == "f32" else oracle.bf16_bits_to_f32(mine).astype(np.float64)
            b = theirs.astype(np.float64) if wdt == "f32" else oracle.bf16_bits_to_f32(theirs).astype(np.float64)
            assert np.abs(a - b).max() < (1e-4 if wdt == "f32" else 0.05)
