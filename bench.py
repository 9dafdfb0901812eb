#!/usr/bin/env python3
"""Benchmark of the per-step forward on one MI355X.

Default workload (config 4): the mid-size GPT (16 layers, d 2048,
64x32 heads, MLP 8192, vocab 32000, bf16 weights with fp32 accumulation, bf16
paged K/V) running one mixed continuous-batch step of 192 decode rows
(kv_len U[256, 4096] over synthetic cached K/V) plus two 512-row prefill
chunks (a fresh sequence at positions 0..511 and a sequence with 512 cached
tokens at positions 512..1023): M = 1216 rows.  The physical page table is
shuffled (single-page sequences freed in a random order before admission).
A step is TransformerRunner::forward_step_greedy (every layer, lm_head over
all 1216 rows, device argmax); metric = decode tokens/s = 192 / step time.

Also measured live with HIP events on the runner's stream:
  * the dominant kernel, split-KV paged decode attention of one layer over the
    step's 192 decode rows (roofline: HBM, algorithmic bytes / duration);
  * the step's bf16 GEMMs at M = 1216 (MFMA roofline, reported beside).
cpu_baseline: the C oracle (a scalar-per-row fp64 restatement, OpenMP) timed
on the host on one layer of the same step plus lm_head, scaled to 16 layers.

Other modes: --config c1 (tiny fp32 GPT greedy continuous batching),
--config c2 (the isolated linear layers), --config c3 (paged decode
attention alone), --config c5 (long-context fp8 decode), --config gemm
(config 4's GEMM shapes alone), --config tiering (the tiered K/V prefix
restore); --copy-calib (a plain device copy for PMC byte calibration).
"""
import argparse
import contextlib
import ctypes
import gc
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3


def _log(*a):
    print(*a, file=sys.stderr, flush=True)


def _cbis():
    import __graft_entry__ as ge
    return ge._import_cbis()


class Events:
    """HIP events on an explicit stream (the runner's), via torch's wrappers."""

    def __init__(self, stream_handle):
        import torch
        self.torch = torch
        self.stream = torch.cuda.ExternalStream(stream_handle) if stream_handle else torch.cuda.current_stream()

    def time_graph(self, fn, iters, reps=5):
        """Per-call device time of `fn` with the host taken out: `iters`
        calls captured in one graph on a side stream, the graph replayed
        `reps` times between events (kernels that are a few microseconds
        long are otherwise bound by the Python launch rate)."""
        torch = self.torch
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            fn()  # warm (lazy loads happen outside the capture)
            side.synchronize()
            with torch.cuda.graph(g, stream=side):
                for _ in range(iters):
                    fn()
        g.replay()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            g.replay()
        e.record()
        e.synchronize()
        return s.elapsed_time(e) / (reps * iters)

    def time(self, fn, iters):
        torch = self.torch
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(self.stream):
            s.record(self.stream)
            for _ in range(iters):
                fn()
            e.record(self.stream)
        e.synchronize()
        return s.elapsed_time(e) / iters  # ms


@contextlib.contextmanager
def gc_paused():
    """Runs a timed loop with Python's cyclic garbage collector paused, as
    the standard library's timeit does (the collector runs once before).  A
    full collection of this process's heap takes 40-55 ms on the GPU box's
    host; one falling inside a 20-step region of config 4 added ~2 ms to the
    mean step while every step's device time and C++ call time stayed put."""
    gc.collect()
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def shuffled_cache(cbis, cache, n_pages, seed):
    """Hands the allocator a shuffled free list using only the reference API:
    n_pages one-page sequences take pages 0..n-1, then are freed in a random
    order (free_sequence pushes their page back), so later allocations pop
    physical pages in random order."""
    rng = np.random.default_rng(seed)
    dummies = []
    for _ in range(n_pages):
        s = cache.allocate_sequence()
        assert cache.ensure_capacity(s, 0)
        dummies.append(s)
    for i in rng.permutation(n_pages):
        cache.free_sequence(dummies[i])


def c4_setup(cbis, oracle, n_layers=16, seed=0):
    cfg = cbis.ModelConfig.make(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=n_layers, mlp=8192,
                                max_seq=32768, weight_dtype="bf16", kv_dtype="bf16")
    kv = oracle.uniform_int(seed, 5001, 192, 256, 4096)
    pages_needed = int(((kv + 15) // 16).sum()) + 32 + 64
    max_pages = pages_needed + 64
    t0 = time.time()
    w = cbis.ModelWeights.synthetic(cfg, seed=seed)
    cache = cbis.PagedKVCache(n_layers, max_pages, 16, 64, 32, "bf16", pages_per_seq=2048)
    cache.fill_normal(seed=seed + 1, std=1.0)
    shuffled_cache(cbis, cache, max_pages, seed)
    runner = cbis.TransformerRunner(w, cache, 1216)
    toks = oracle.uniform_int(seed, 5002, 1216, 0, 31999)
    tok, pos, sid, dec_seqs = [], [], [], []
    for i in range(192):
        s = cache.allocate_sequence()
        assert cache.ensure_capacity(s, int(kv[i]) - 1)  # grows the page list to cover 0..kv-1
        tok.append(int(toks[i])); pos.append(int(kv[i]) - 1); sid.append(s); dec_seqs.append(s)
    for start in (0, 512):
        s = cache.allocate_sequence()
        assert cache.ensure_capacity(s, start + 511)
        for p in range(start, start + 512):
            tok.append(int(toks[len(tok)])); pos.append(p); sid.append(s)
    _log(f"c4 setup {time.time() - t0:.1f}s: weights {w.device_bytes() / 1e9:.2f} GB, "
         f"kv pool {max_pages} pages x {n_layers} layers")
    return dict(cfg=cfg, w=w, cache=cache, runner=runner, tok=tok, pos=pos, sid=sid, kv=kv, dec_seqs=dec_seqs)


def decode_attention_timing(cbis, st, iters):
    """Times one layer's split-KV decode attention over the step's 192 decode
    rows (the dominant kernel) on the runner's stream."""
    import torch
    cache, kv = st["cache"], st["kv"]
    n, H = 192, 64
    tables = [cache.pages(s) for s in st["dec_seqs"]]
    width = max(len(t) for t in tables)
    bt = np.zeros((n, width), np.int32)
    for i, t in enumerate(tables):
        bt[i, : len(t)] = t
    dev = torch.device("cuda:0")
    BT = torch.from_numpy(bt).to(dev)
    POS = torch.from_numpy((kv - 1).astype(np.int32)).to(dev)
    # rows in the order TransformerRunner passes them: longest first
    ROWS = torch.from_numpy(np.argsort(-kv, kind="stable").astype(np.int32)).to(dev)
    q = torch.empty((n, H * 32), dtype=torch.float32, device=dev)
    cbis.check(cbis.kernels().cbis_fill_normal_fast(q.data_ptr(), cbis.F32, q.numel(), 7, 1.0, None))
    out = torch.empty((n, H * 32), dtype=torch.bfloat16, device=dev)
    d = cbis.AttnDesc()
    d.n_rows, d.n_heads, d.head_dim, d.page_size = n, H, 32, 16
    d.rows = ROWS.data_ptr()
    d.q_dtype, d.q, d.ldq = cbis.F32, q.data_ptr(), H * 32
    d.kv_dtype, d.k_pool, d.v_pool, d.num_pages = cbis.BF16, cache.k_base(0), cache.v_base(0), cache.max_pages()
    d.block_table, d.bt_stride, d.row_pos = BT.data_ptr(), width, POS.data_ptr()
    d.out_dtype, d.out, d.ldo = cbis.BF16, out.data_ptr(), H * 32
    d.max_kv_len = int(kv.max())
    # As TransformerRunner runs these rows: one pass per row (192 rows x 4 head
    # blocks = 768 workgroups >= 1.5 rounds, no row over twice the mean length).
    assert n * (H // 16) >= 768 and int(kv.max()) * n <= 2 * int(kv.sum())
    d.split_tokens = 1 << 30
    need = cbis.kernels().cbis_paged_attention_workspace_size(ctypes.byref(d))
    ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
    d.workspace, d.workspace_bytes = ws.data_ptr(), need
    torch.cuda.synchronize()
    ev = Events(st["runner"].stream())
    stream = st["runner"].stream()
    fn = lambda: cbis.check(cbis.kernels().cbis_paged_attention(ctypes.byref(d), stream))
    ev.time(fn, 3)
    ms = ev.time(fn, iters)
    kvsum = int(kv.sum())
    alg_bytes = kvsum * H * 32 * 2 * 2 + int(((kv + 15) // 16).sum()) * 4 + n * H * 32 * 4 + n * H * 32 * 2
    return ms, alg_bytes


def gemm_timing(cbis, st, iters):
    """Times the step's five bf16 GEMMs at M = 1216 on layer 0's weights with
    the epilogues the step runs them with: qkv with bias, fp32 q and the K/V
    page scatter (into layer 0's pools at the step's write slots); the
    out-projection with bias and the fp32 residual; fc1 with bias, GELU and a
    bf16 output; fc2 with bias and residual, split-K, its reduce fused with the
    next LayerNorm (cbis_gemm_layernorm); lm_head fused with the greedy argmax
    (cbis_gemm_argmax).  The split-K workspace is the one cbis_gemm asks for."""
    import torch
    w, cache = st["w"], st["cache"]
    dev = torch.device("cuda:0")
    M, D, F, V = 1216, 2048, 8192, 32000
    K_ = cbis.kernels()
    X = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
    cbis.check(K_.cbis_fill_normal_fast(X.data_ptr(), cbis.BF16, X.numel(), 9, 1.0, None))
    Q = torch.empty((M, D), dtype=torch.float32, device=dev)
    R = torch.empty((M, D), dtype=torch.float32, device=dev)
    cbis.check(K_.cbis_fill_normal_fast(R.data_ptr(), cbis.F32, R.numel(), 10, 1.0, None))
    H = torch.empty((M, F), dtype=torch.bfloat16, device=dev)
    LN = torch.empty((M, D), dtype=torch.bfloat16, device=dev)
    slots = np.array([cache.resolve_slot(s, p) for s, p in zip(st["sid"], st["pos"])], np.int32)
    WP = torch.from_numpy(np.ascontiguousarray(slots[:, 0])).to(dev)
    WO = torch.from_numpy(np.ascontiguousarray(slots[:, 1])).to(dev)
    nxt = torch.empty(M, dtype=torch.int32, device=dev)
    mar = torch.empty(M, dtype=torch.float32, device=dev)
    ev = Events(st["runner"].stream())
    stream = st["runner"].stream()
    keep = []

    def desc(N, K, wname, bias, Y, y_dtype, residual=None, gelu=False):
        d = cbis.GemmDesc()
        d.M, d.N, d.K = M, N, K
        d.x_dtype, d.X, d.ldx = cbis.BF16, X.data_ptr(), K
        d.w_dtype, d.W, d.ldw = cbis.BF16, w.tensor(wname), K
        d.bias = w.tensor(bias) if bias else None
        d.epilogue = cbis.EPI_GELU if gelu else cbis.EPI_NONE
        d.residual, d.ldr = (residual.data_ptr() if residual is not None else None), N
        d.y_dtype, d.Y, d.ldy = y_dtype, (Y.data_ptr() if Y is not None else None), N
        need = K_.cbis_gemm_workspace_size(ctypes.byref(d))
        ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
        keep.append(ws)
        d.workspace, d.workspace_bytes = ws.data_ptr(), need
        return d

    dq = desc(3 * D, D, "l0.wqkv", "l0.bqkv", Q, cbis.F32)
    dq.ldy = D
    dq.kv_col0, dq.kv_width, dq.kv_dtype, dq.page_size = D, D, cbis.BF16, 16
    dq.k_pool, dq.v_pool, dq.write_page, dq.write_offset = cache.k_base(0), cache.v_base(0), WP.data_ptr(), WO.data_ptr()
    do = desc(D, D, "l0.wo", "l0.bo", R, cbis.F32, residual=R)
    d1 = desc(F, D, "l0.w1", "l0.b1", H, cbis.BF16, gelu=True)
    d2 = desc(D, F, "l0.w2", "l0.b2", R, cbis.F32, residual=R)
    dl = desc(V, D, "lm_head", None, None, cbis.F32)
    need = K_.cbis_gemm_argmax_workspace_size(ctypes.byref(dl))
    aws = torch.empty(max(4, need // 4), dtype=torch.float32, device=dev)
    ln_w, ln_b = w.tensor("l1.ln1_w"), w.tensor("l1.ln1_b")
    calls = [
        ("qkv", dq, lambda: cbis.check(K_.cbis_gemm(ctypes.byref(dq), stream))),
        ("out", do, lambda: cbis.check(K_.cbis_gemm(ctypes.byref(do), stream))),
        ("fc1", d1, lambda: cbis.check(K_.cbis_gemm(ctypes.byref(d1), stream))),
        ("fc2+ln", d2, lambda: cbis.check(K_.cbis_gemm_layernorm(ctypes.byref(d2), ln_w, ln_b, 1e-5, cbis.BF16,
                                                                  LN.data_ptr(), D, stream))),
        ("lm_head+argmax", dl, lambda: cbis.check(K_.cbis_gemm_argmax(ctypes.byref(dl), nxt.data_ptr(),
                                                                      mar.data_ptr(), aws.data_ptr(), need,
                                                                      stream))),
    ]
    res = {}
    tot_flops = tot_ms = 0.0
    for name, d, fn in calls:
        ev.time(fn, 2)
        ms = ev.time(fn, iters)
        fl = 2.0 * M * d.N * d.K
        # per layer the four projections run once; lm_head once per step
        mult = 1 if name.startswith("lm_head") else st["cfg"].n_layers
        tot_flops += fl * mult
        tot_ms += ms * mult
        res[name] = {"ms": round(ms, 4), "tflops": round(fl / ms / 1e9, 1), "split_k_workspace": d.workspace_bytes}
    return res, tot_flops, tot_ms


def torch_step_sampler(oracle, spec, cache, tok, pos, sid):
    """The reference's CPU forward (python/model.py's operators, fp32 PyTorch:
    oracle/torch_cpu.py) on one layer of a forward step over the GPU cache's
    layer-0 K/V (copied to the host).  Returns run() -> (t_layer, t_head): the
    time of that layer over every row, and of the final LayerNorm + lm_head."""
    import torch
    import torch_cpu
    w = oracle.synthetic_weights(spec, seed=0, pos_rows=max(pos) + 1)
    P = cache.max_pages()
    kp = np.empty((P, 16, spec.n_heads, spec.head_dim), np.uint16)
    vp = np.empty_like(kp)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    for dst, src in ((kp, cache.k_base(0)), (vp, cache.v_base(0))):
        assert hip.hipMemcpy(dst.ctypes.data, src, dst.nbytes, 2) == 0
    wp, wo, bt, rb = oracle.step_tables(cache, tok, pos, sid)
    model = torch_cpu.TorchCpuStep(w, [kp], [vp])

    def run():
        with torch.no_grad():
            x = model.embed(tok, pos)
            t0 = time.perf_counter()
            x = model.layer(0, x, pos, wp, wo, bt, rb)
            t1 = time.perf_counter()
            model.head(x)
            return t1 - t0, time.perf_counter() - t1

    return run


def cpu_baseline_step(oracle, spec, cache, tok, pos, sid, decode_rows, runs=3):
    """A step's CPU time as the reference computes on the CPU (fp32 PyTorch,
    torch_step_sampler): one layer over all rows and the lm_head, each the
    median of `runs` runs after a first-touch run, scaled to 16 layers, on the
    host's threads; then one run on 1 thread.  Returns the cpu_baseline
    object (decode tokens/s of the step's decode_rows)."""
    import torch
    run = torch_step_sampler(oracle, spec, cache, tok, pos, sid)
    cores = torch.get_num_threads()
    run()
    ts = [run() for _ in range(runs)]
    tl, th = float(np.median([t[0] for t in ts])), float(np.median([t[1] for t in ts]))
    t_step = tl * 16 + th
    torch.set_num_threads(1)
    try:
        tl1, th1 = run()
    finally:
        torch.set_num_threads(cores)
    t_step1 = tl1 * 16 + th1
    return {"value": round(decode_rows / t_step, 4), "unit": "decode tokens/s", "cores": cores, "kind": "port",
            "value_1core": round(decode_rows / t_step1, 4),
            "sample": f"fp32 PyTorch CPU forward (oracle/torch_cpu.py: python/model.py's operators over the paged "
                      f"K/V) of the {len(tok)}-row step, 1 of 16 layers (median of {runs}: {tl:.3f} s) + lm_head "
                      f"({th:.3f} s), scaled to 16 layers: step {t_step:.2f} s on {cores} threads; on 1 thread "
                      f"layer {tl1:.2f} s + lm_head {th1:.2f} s -> step {t_step1:.1f} s"}


def cpu_baseline_c4(oracle, st, cbis, runs=3):
    """Config 4's step (192 decode rows + two 512-row chunks) on the host."""
    spec = oracle.ModelSpec(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=1, mlp=8192,
                            max_seq=32768, weight_dtype="bf16", kv_dtype="bf16")
    return cpu_baseline_step(oracle, spec, st["cache"], st["tok"], st["pos"], st["sid"], 192, runs)


def recorded_traffic(name):
    """HBM bytes per launch of the dominant kernel, as recorded from the two
    rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE, copy-calibrated) in
    profiles/<name>; None when no such record exists."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def machine_peaks():
    """The box's own figures beside the published peaks: CU count and
    maximum engine clock from rocminfo (bf16 dense MFMA = CUs x 4096 flop/clk
    x clock), and a measured device-to-device copy (1 GiB read + 1 GiB
    written) as the practical HBM figure."""
    import subprocess
    import torch
    out = {"published": {"hbm_gbs": HBM_PEAK_GBS, "bf16_tflops": BF16_PEAK_TFLOPS}}
    try:
        txt = subprocess.run(["rocminfo"], capture_output=True, text=True, timeout=60).stdout
        cus, mhz = None, None
        for blk in txt.split("*******"):
            if "gfx950" not in blk:
                continue
            for line in blk.splitlines():
                line = line.strip()
                if line.startswith("Compute Unit:"):
                    cus = int(line.split(":")[1])
                elif line.startswith("Max Clock Freq. (MHz):"):
                    mhz = int(line.split(":")[1])
            if cus and mhz:
                break
        if cus and mhz:
            out["rocminfo"] = {"compute_units": cus, "max_clock_mhz": mhz,
                               "bf16_dense_tflops": round(cus * 4096 * mhz * 1e6 / 1e12, 1)}
    except Exception as e:  # rocminfo missing or refused: report what is known
        out["rocminfo"] = f"unavailable ({type(e).__name__})"
    n = 1 << 28
    a = torch.ones(n, dtype=torch.float32, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s_.record()
    for _ in range(10):
        b.copy_(a)
    e_.record()
    e_.synchronize()
    ms = s_.elapsed_time(e_) / 10
    out["measured_copy_gbs"] = round(2 * n * 4 / ms / 1e6, 1)
    del a, b
    torch.cuda.empty_cache()
    return out


def run_c4(args, cbis, oracle):
    st = c4_setup(cbis, oracle)
    runner = st["runner"]
    import torch
    # The step's rows as int32 arrays (the binding passes them to the C++
    # runner without a per-element conversion); the runner redoes all of its
    # per-step host work (checks, slot resolution, block tables, one H2D copy).
    tok, pos, sid = (np.asarray(st[k], dtype=np.int32) for k in ("tok", "pos", "sid"))
    # Pipelined steps, as the pipelined scheduler runs them: step k + 1 is
    # queued before step k's tokens are waited for, and each of the 192
    # decode rows takes its input token from its own row of the step before
    # (read on the device); the prefill rows' tokens come from the host.
    src = np.full(len(tok), -1, dtype=np.int32)
    src[:192] = np.arange(192, dtype=np.int32)
    # Every step is timed twice: host wall time (synchronous: around the
    # call, which returns once the step's tokens are on the host; pipelined:
    # between consecutive steps' results) and the device time of its forward
    # between two events on the runner's stream.  The collector is paused
    # from before the warmup, whose steps absorb the idle GPU's slower first
    # step after the collection.
    def timed(pipelined):
        wall, dev, host = [], [], []
        with gc_paused():
            for _ in range(args.warmup):
                runner.forward_step_greedy(tok, pos, sid)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            if pipelined:
                prev = runner.enqueue_greedy(tok, pos, sid)
                t_last = time.perf_counter()
                for k in range(args.steps):
                    nxt = runner.enqueue_greedy(tok, pos, sid, src) if k + 1 < args.steps else None
                    runner.wait_greedy(prev)
                    t1 = time.perf_counter()
                    wall.append((t1 - t_last) * 1000.0)
                    t_last = t1
                    dev.append(runner.last_device_ms())
                    host.append(runner.last_host_ms())
                    prev = nxt
            else:
                for _ in range(args.steps):
                    t1 = time.perf_counter()
                    runner.forward_step_greedy(tok, pos, sid)
                    wall.append((time.perf_counter() - t1) * 1000.0)
                    dev.append(runner.last_device_ms())
                    host.append(runner.last_host_ms())
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
        stats = {"wall_median": float(np.median(wall)), "wall_mean": float(np.mean(wall)), "wall_min": min(wall),
                 "wall_max": max(wall), "device_median": float(np.median(dev)), "device_min": min(dev),
                 "device_max": max(dev), "region_mean": dt * 1000.0 / args.steps}
        stats = {k: round(v, 4) for k, v in stats.items()}
        mode = "pipelined" if pipelined else "synchronous"
        _log(f"c4 {mode} per-step wall ms: " + " ".join(f"{x:.3f}" for x in wall))
        _log(f"c4 {mode} per-step device ms: " + " ".join(f"{x:.3f}" for x in dev))
        med = float(np.median(wall))
        for i, (w_, d_, h_) in enumerate(zip(wall, dev, host)):
            if w_ > med + 1.0:
                _log(f"c4 {mode} slow step {i}: wall {w_:.3f} ms, device {d_:.3f} ms; host phases: prepare "
                     f"{h_[0]:.3f}, launch {h_[1]:.3f}, wait {h_[2]:.3f} ms")
        value = 192.0 * args.steps / dt
        _log(f"c4 {mode}: step median {stats['wall_median']:.3f} ms (mean over the region "
             f"{stats['region_mean']:.3f}, device median {stats['device_median']:.3f}) -> {value:.1f} decode tok/s "
             f"over the region ({1216 * args.steps / dt:.0f} rows/s)")
        return value, stats

    sync_value, sync_stats = timed(False)
    value, stats = timed(True)
    ms_step = stats["wall_median"]
    att_ms, att_bytes = decode_attention_timing(cbis, st, max(10, args.steps))
    att_gbs = att_bytes / att_ms / 1e6
    _log(f"decode attention (1 layer): {att_ms:.4f} ms, {att_bytes / 1e9:.3f} GB -> {att_gbs:.0f} GB/s")
    gem, gflops, gms = gemm_timing(cbis, st, max(10, args.steps))
    gemm_tflops = gflops / gms / 1e9
    _log(f"gemms: {json.dumps(gem)}; step total {gemm_tflops:.0f} TFLOP/s")
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_c4(oracle, st, cbis)
        _log(f"cpu baseline: {cpu}")
    peaks = machine_peaks()
    _log(f"machine: {json.dumps(peaks)}")
    return {
        "machine": peaks,
        "metric": "decode tokens/s (config 4 mixed continuous-batch step, mid-size GPT)",
        "value": round(value, 2),
        "unit": "decode tokens/s",
        "ms_per_step": round(ms_step, 4),
        "step_ms": stats,
        "synchronous": {"value": round(sync_value, 2), "step_ms": sync_stats},
        "dtype": "bf16",
        "data": "synthetic (seeded weights N(0,0.02); K/V cache N(0,1); random token ids)",
        "config": {"workload": "c4_mixed_step", "model": "gpt-mid L16 d2048 h64x32 mlp8192 V32000",
                   "decode_rows": 192, "decode_kv_len": "U[256,4096]", "prefill_chunks": "2x512 (pos 0, 512)",
                   "rows_per_step": 1216, "page_size": 16, "page_table": "shuffled", "parallelism": "none (1 GPU)",
                   "steps": "pipelined (step k + 1 queued before step k's tokens are back; decode rows take "
                            "their token from the step before on the device)"},
        "roofline": {"bound": "hbm", "kernel": "paged_decode_kernel<bf16>, one layer, one pass per row",
                     "achieved": round(att_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(att_gbs / HBM_PEAK_GBS, 4),
                     "traffic": recorded_traffic("paged_decode_c4_hbm_traffic.md"),
                     "algorithmic_bytes": att_bytes, "ms": round(att_ms, 4)},
        "gemm_roofline": {"bound": "mfma", "achieved": round(gemm_tflops, 1), "peak": BF16_PEAK_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(gemm_tflops / BF16_PEAK_TFLOPS, 4), "shapes": gem},
        "cpu_baseline": cpu,
    }


def c3_inputs(oracle, n_seq=256, lo=128, hi=2048, pool=40000, seed=0):
    """Config 3: kv_len U[lo, hi], one query per sequence at pos kv_len-1, a
    random permutation of a pool of `pool` pages as the page table."""
    kv = oracle.uniform_int(seed, 3001, n_seq, lo, hi)
    npages = (kv + 15) // 16
    perm = np.random.default_rng(seed).permutation(pool).astype(np.int32)
    bt = np.zeros((n_seq, int(npages.max())), np.int32)
    off = 0
    for i in range(n_seq):
        bt[i, : npages[i]] = perm[off: off + npages[i]]
        off += npages[i]
    return kv, bt


def run_c3(args, cbis, oracle):
    """Config 3: paged decode attention alone (fp32 K/V, 8x32 heads, 256
    sequences, kv U[128, 2048], 40,000-page pool, permuted page table)."""
    import torch
    H, P = 8, 40000
    kv, bt = c3_inputs(oracle)
    n = kv.size
    dev = torch.device("cuda:0")
    K = cbis.kernels()
    kp = torch.empty((P, 16, H, 32), dtype=torch.float32, device=dev)
    vp = torch.empty_like(kp)
    q = torch.empty((n, H * 32), dtype=torch.float32, device=dev)
    for t, sd in ((kp, 1), (vp, 2), (q, 3)):
        cbis.check(K.cbis_fill_normal_fast(t.data_ptr(), cbis.F32, t.numel(), sd, 1.0, None))
    BT = torch.from_numpy(bt).to(dev)
    POS = torch.from_numpy((kv - 1).astype(np.int32)).to(dev)
    ROWS = torch.from_numpy(np.argsort(-kv, kind="stable").astype(np.int32)).to(dev)  # longest first
    out = torch.empty((n, H * 32), dtype=torch.float32, device=dev)
    d = cbis.AttnDesc()
    d.n_rows, d.n_heads, d.head_dim, d.page_size = n, H, 32, 16
    d.rows = ROWS.data_ptr()
    d.q_dtype, d.q, d.ldq = cbis.F32, q.data_ptr(), H * 32
    d.kv_dtype, d.k_pool, d.v_pool, d.num_pages = cbis.F32, kp.data_ptr(), vp.data_ptr(), P
    d.block_table, d.bt_stride, d.row_pos = BT.data_ptr(), bt.shape[1], POS.data_ptr()
    d.out_dtype, d.out, d.ldo = cbis.F32, out.data_ptr(), H * 32
    d.max_kv_len = int(kv.max())
    need = K.cbis_paged_attention_workspace_size(ctypes.byref(d))
    ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
    d.workspace, d.workspace_bytes = ws.data_ptr(), need
    torch.cuda.synchronize()
    ev = Events(None)
    stream = torch.cuda.current_stream().cuda_stream
    fn = lambda: cbis.check(K.cbis_paged_attention(ctypes.byref(d), stream))
    ev.time(fn, args.warmup)
    ms = ev.time(fn, args.steps)
    alg = int(kv.sum()) * H * 32 * 4 * 2 + int(((kv + 15) // 16).sum()) * 4 + 2 * n * H * 32 * 4
    gbs = alg / ms / 1e6
    _log(f"c3 decode attention: {ms:.4f} ms, {alg / 1e6:.1f} MB -> {gbs:.0f} GB/s")
    cpu = None
    if not args.no_cpu:
        qh, kh, vh = q.cpu().numpy(), kp.cpu().numpy(), vp.cpu().numpy()
        t0 = time.time()
        reps = 0
        while time.time() - t0 < 10.0:
            oracle.paged_attention(qh, kh, vh, bt, kv - 1, H, 32, 16)
            reps += 1
        cpu_ms = (time.time() - t0) * 1000.0 / reps
        cpu = {"value": round(alg / cpu_ms / 1e6, 2), "unit": "GB/s", "cores": oracle.lib().orc_num_threads(),
               "kind": "port", "sample": f"oracle fp64 paged attention over the full config-3 call, {reps} reps "
                                          f"({cpu_ms:.1f} ms each)"}
    return {"metric": "paged decode attention HBM GB/s (config 3)", "value": round(gbs, 1), "unit": "GB/s",
            "ms_per_step": round(ms, 4), "dtype": "f32",
            "data": "synthetic (Q/K/V N(0,1); permuted page table)",
            "config": {"workload": "c3_paged_decode_attention", "rows": n, "heads": "8x32", "kv_len": "U[128,2048]",
                       "pool_pages": P, "page_size": 16},
            "roofline": {"bound": "hbm", "kernel": "paged_decode_kernel<f32> + split merge", "achieved": round(gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": recorded_traffic("paged_decode_c3_hbm_traffic.md"),
                         "algorithmic_bytes": alg, "ms": round(ms, 4)},
            "cpu_baseline": cpu}


def run_c1(args, cbis, oracle):
    """Config 1: tiny fp32 GPT (V=512, d=256, 8x32, L=4, MLP 1024), 8 prompts
    U[16,64], 32 greedy tokens each through the C++ continuous-batching
    scheduler (1 prefill step + 31 decode steps of 8 rows).  value = decode
    tokens / decode wall time (median of `steps` runs) of the pipelined
    scheduler, which queues each step before the previous step's tokens are
    back; the synchronous scheduler's rate is reported beside it."""
    reqs = oracle.c1_requests()
    cfg = cbis.ModelConfig.make(vocab=512, n_layers=4)
    w = cbis.ModelWeights.synthetic(cfg, seed=0)
    cache = cbis.PagedKVCache(4, 128, 16, 8, 32, "f32")
    runner = cbis.TransformerRunner(w, cache, 512)
    prompts = [r.prompt for r in reqs]
    dl = [r.decode_len for r in reqs]
    n_dec = sum(d - 1 for d in dl)
    n_prompt = sum(len(p) for p in prompts)
    rate = {}
    toks = {}
    with gc_paused():
        for pipe in (False, True):
            dec, tot = [], []
            for _ in range(max(1, args.warmup)):
                cbis.run_continuous(runner, cache, prompts, dl, pipeline=pipe)
            for _ in range(args.steps):
                toks[pipe], ms = cbis.run_continuous(runner, cache, prompts, dl, pipeline=pipe)
                # Step 0 is the prefill; the rest, in the pipelined mode the
                # intervals between consecutive steps' results, the decode.
                dec.append(sum(ms[1:]))
                tot.append(sum(ms))
            dec_ms, tot_ms = float(np.median(dec)), float(np.median(tot))
            rate[pipe] = (n_dec / dec_ms * 1000.0, dec_ms, tot_ms)
            _log(f"c1 {'pipelined' if pipe else 'synchronous'}: decode {dec_ms:.3f} ms for {n_dec} tokens -> "
                 f"{rate[pipe][0]:.0f} tok/s; whole run {tot_ms:.3f} ms "
                 f"({(n_prompt + sum(dl)) / tot_ms * 1000.0:.0f} prompt+generated tok/s)")
    assert toks[True] == toks[False], "pipelined and synchronous greedy tokens differ"
    value, dec_ms, tot_ms = rate[True]
    toks = toks[True]
    cpu = None
    if not args.no_cpu:
        # The whole workload through the same scheduler with the reference's
        # CPU forward (fp32 PyTorch, oracle/torch_cpu.py) as the step.
        import torch
        import torch_cpu
        spec = oracle.ModelSpec(vocab=512, n_layers=4, max_seq=128)
        pools = [[np.zeros((128, 16, 8, 32), np.float32) for _ in range(4)] for _ in range(2)]
        tm = torch_cpu.TorchCpuStep(oracle.synthetic_weights(spec, seed=0, pos_rows=128), *pools)
        step_s = []

        class CpuStep:
            def forward_step(self, *a):
                t = time.perf_counter()
                with torch.no_grad():
                    lg = tm.forward_step(*a).double().numpy()
                step_s.append((len(a[0]), time.perf_counter() - t))
                return lg

        t0 = time.time()
        gen, _ = oracle.run_continuous(CpuStep(), oracle.PagedKVCacheOracle(128), reqs)
        cpu_s = time.time() - t0
        dec = [t for m, t in step_s if m == len(reqs)]  # the steps of one decode row per request
        dec_s = float(np.median(dec))
        cpu = {"value": round(len(reqs) / dec_s, 2), "unit": "decode tokens/s", "cores": torch.get_num_threads(),
               "kind": "port", "tokens_match_gpu": gen == toks,
               "sample": f"fp32 PyTorch CPU step (oracle/torch_cpu.py: python/model.py's operators) through the "
                         f"same scheduler over the whole config-1 workload ({cpu_s:.2f} s, {len(step_s)} steps): "
                         f"median {len(reqs)}-row decode step {dec_s * 1e3:.3f} ms"}
    return {"metric": "decode tokens/s (config 1 tiny GPT continuous batching)", "value": round(value, 1),
            "unit": "decode tokens/s", "ms_per_step": round(dec_ms / (len(dl) and 31), 4), "dtype": "f32",
            "data": "synthetic (seeded weights N(0,0.02); prompt ids U[0,511])",
            "config": {"workload": "c1_tiny_gpt_greedy", "requests": len(dl), "prompt_len": "U[16,64]",
                       "decode_len": 32, "scheduler": "pipelined", "whole_run_ms": round(tot_ms, 3),
                       "synchronous_decode_tok_s": round(rate[False][0], 1)},
            "cpu_baseline": cpu}


def c5_setup(cbis, oracle):
    """Config 5's model, cache and sequences as run_c5 times them: fp8
    weights, a bf16 cache of 16 x 2048 + 64 pages filled N(0, 1) over a
    shuffled free list, 16 sequences owning positions 0..32767, and their
    first tokens; decode runs at positions ctx .. ctx + gen - 1."""
    n_seq, ctx, gen = 16, 32768 - 64, 64
    cfg = cbis.ModelConfig.make(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=16, mlp=8192,
                                max_seq=32768, weight_dtype="fp8", kv_dtype="bf16")
    pages = n_seq * 2048 + 64
    t0 = time.time()
    w = cbis.ModelWeights.synthetic(cfg, seed=0)
    cache = cbis.PagedKVCache(16, pages, 16, 64, 32, "bf16", pages_per_seq=2048)
    cache.fill_normal(seed=5, std=1.0)
    shuffled_cache(cbis, cache, pages, 5)
    runner = cbis.TransformerRunner(w, cache, 64)
    seqs = []
    for _ in range(n_seq):
        sid = cache.allocate_sequence()
        assert cache.ensure_capacity(sid, 32767)
        seqs.append(sid)
    _log(f"c5 setup {time.time() - t0:.1f}s: weights {w.device_bytes() / 1e9:.2f} GB, "
         f"kv {pages} pages x 16 layers ({cache.max_pages() * 16 * 2048 * 2 * 2 * 16 / 1e9:.1f} GB)")
    first = [int(t) for t in oracle.uniform_int(0, 5003, n_seq, 0, 31999)]
    return dict(cfg=cfg, w=w, cache=cache, runner=runner, seqs=seqs, first=first, n_seq=n_seq, ctx=ctx, gen=gen)


def run_c5(args, cbis, oracle):
    """Config 5: the mid-size GPT with fp8-e4m3 linear weights (per-channel
    fp32 scales) and a bf16 paged K/V cache; 16 sequences whose caches hold
    32704 synthetic tokens greedy-decode 64 tokens each at positions
    32704..32767 (the last one is kMaxSeqLen - 1).  A step is 16 rows;
    value = 16 * 64 / wall time of the 64 steps (median over `steps` runs),
    the steps pipelined (each queued before the previous one's tokens are
    back, its rows reading their tokens from it on the device); the
    synchronous loop's rate is reported beside it."""
    import torch
    st = c5_setup(cbis, oracle)
    runner, cache, seqs, first = st["runner"], st["cache"], st["seqs"], st["first"]
    n_seq, ctx, gen = st["n_seq"], st["ctx"], st["gen"]

    def run_sync():
        toks = first
        for i in range(gen):
            toks = runner.forward_step_greedy(toks, [ctx + i] * n_seq, seqs)
        return toks

    src = list(range(n_seq))

    def run_pipelined():
        prev = runner.enqueue_greedy(first, [ctx] * n_seq, seqs)
        for i in range(1, gen):
            nxt = runner.enqueue_greedy([-1] * n_seq, [ctx + i] * n_seq, seqs, src)
            runner.wait_greedy(prev)
            prev = nxt
        return runner.wait_greedy(prev)

    rate, last = {}, {}
    with gc_paused():
        for name, run in (("synchronous", run_sync), ("pipelined", run_pipelined)):
            times = []
            for _ in range(max(1, args.warmup)):
                run()
            for _ in range(args.steps):
                torch.cuda.synchronize()
                t1 = time.perf_counter()
                last[name] = run()
                torch.cuda.synchronize()
                times.append(time.perf_counter() - t1)
            dt = float(np.median(times))
            rate[name] = (n_seq * gen / dt, dt)
            _log(f"c5 {name}: {gen} steps in {dt * 1000:.2f} ms -> {rate[name][0]:.1f} tok/s "
                 f"({dt * 1000 / gen:.3f} ms/step)")
    assert last["pipelined"] == last["synchronous"], "pipelined and synchronous greedy tokens differ"
    value, dt = rate["pipelined"]
    cpu = None
    if not args.no_cpu:
        spec = oracle.ModelSpec(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=1, mlp=8192,
                                max_seq=32768, weight_dtype="fp8", kv_dtype="bf16")
        cpu = cpu_baseline_step(oracle, spec, cache, first, [ctx] * n_seq, seqs, n_seq, runs=1)
    return {"metric": "decode tokens/s (config 5 long-context fp8 decode)", "value": round(value, 2),
            "unit": "decode tokens/s", "ms_per_step": round(dt * 1000 / gen, 4), "dtype": "bf16 x fp8-e4m3",
            "data": "synthetic (fp8 weights absmax-quantised from N(0,0.02); K/V cache N(0,1))",
            "config": {"workload": "c5_long_context_fp8_decode", "sequences": n_seq, "kv_len": "32704..32767",
                       "decode_tokens": gen, "kv_cache_gb": round(16 * n_seq * 32768 * 2048 * 2 * 2 / 1e9, 1),
                       "steps": "pipelined", "synchronous_decode_tok_s": round(rate["synchronous"][0], 2)},
            "cpu_baseline": cpu}


def run_c2(args, cbis, oracle):
    """Config 2: the isolated flattened-batch linear layers of the reference
    model (d_model 256): QKV 256->768 (+bias), out-proj 256->256 (+bias),
    MLP up 256->1024 (+bias, GELU), MLP down 1024->256 (+bias, residual), at
    M in {64, 512, 4096}, fp32 and bf16 (fp32 accumulate), each call given
    the split-K workspace cbis_gemm_workspace_size asks for.  Device time per
    call from a replayed graph of `steps` calls.  value = total flops of the
    24 GEMMs / their summed time; each shape is reported with
    its TFLOP/s, bytes moved and roofline fraction (fp32: MFMA-bound against
    157.3 TFLOP/s; bf16: min(2.5 PFLOP/s, AI x 8 TB/s))."""
    import torch
    dev = torch.device("cuda:0")
    K_ = cbis.kernels()
    ev = Events(None)
    shapes = [("qkv", 768, 256, True, False, False), ("out", 256, 256, True, False, False),
              ("up", 1024, 256, True, True, False), ("down", 256, 1024, True, False, True)]
    rows, tot_fl, tot_ms = [], 0.0, 0.0
    cpu_fl = cpu_s = 0.0
    for dt in ("f32", "bf16"):
        for M in (64, 512, 4096):
            for name, N, K, has_b, gelu, has_r in shapes:
                x = torch.randn(M, K, device=dev)
                w = torch.randn(N, K, device=dev) * 0.02
                b = torch.randn(N, device=dev) * 0.02
                Y = torch.randn(M, N, device=dev)
                X = x if dt == "f32" else x.to(torch.bfloat16)
                W = w if dt == "f32" else w.to(torch.bfloat16)
                d = cbis.GemmDesc()
                d.M, d.N, d.K = M, N, K
                d.x_dtype = d.w_dtype = cbis.F32 if dt == "f32" else cbis.BF16
                d.X, d.ldx, d.W, d.ldw = X.data_ptr(), K, W.data_ptr(), K
                d.bias = b.data_ptr()
                d.epilogue = cbis.EPI_GELU if gelu else cbis.EPI_NONE
                if has_r:
                    d.residual, d.ldr = Y.data_ptr(), N
                d.y_dtype, d.Y, d.ldy = cbis.F32, Y.data_ptr(), N
                need = K_.cbis_gemm_workspace_size(ctypes.byref(d))
                ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
                d.workspace, d.workspace_bytes = ws.data_ptr(), need
                fn = lambda d=d: cbis.check(K_.cbis_gemm(ctypes.byref(d), torch.cuda.current_stream().cuda_stream))
                ms = ev.time_graph(fn, max(5, args.steps))
                fl = 2.0 * M * N * K
                es = 4 if dt == "f32" else 2
                nbytes = (M * K + N * K) * es + (N + M * N) * 4 + (M * N * 4 if has_r else 0)
                tf = fl / ms / 1e9
                if dt == "f32":
                    peak = FP32_PEAK_TFLOPS
                    bound = "mfma"
                else:
                    peak = min(BF16_PEAK_TFLOPS, fl / nbytes * HBM_PEAK_GBS / 1e3)
                    bound = "mfma" if peak == BF16_PEAK_TFLOPS else "hbm"
                rows.append({"dtype": dt, "M": M, "shape": name, "N": N, "K": K, "us": round(ms * 1000, 2),
                             "tflops": round(tf, 1), "gbs": round(nbytes / ms / 1e6, 1), "bound": bound,
                             "roofline_frac": round(tf / peak, 4)})
                tot_fl += fl
                tot_ms += ms
                if not args.no_cpu and M == 512:
                    xh, wh, bh = x.cpu().numpy(), w.cpu().numpy(), b.cpu().numpy()
                    t0 = time.time()
                    oracle.gemm(xh, wh, bias=bh, gelu=gelu)
                    cpu_s += time.time() - t0
                    cpu_fl += fl
    for r in rows:
        _log(f"c2 {r['dtype']:>4} M={r['M']:>4} {r['shape']:>4}: {r['us']:8.2f} us {r['tflops']:7.1f} TFLOP/s "
             f"{r['gbs']:7.1f} GB/s  {r['bound']} frac {r['roofline_frac']:.3f}")
    value = tot_fl / tot_ms / 1e9
    cpu = None
    if cpu_s > 0:
        cpu = {"value": round(cpu_fl / cpu_s / 1e9, 3), "unit": "GFLOP/s", "cores": oracle.lib().orc_num_threads(),
               "kind": "port", "sample": f"oracle fp64 GEMM (+bias/GELU) of the 8 M=512 shapes ({cpu_s:.1f} s)"}
    return {"metric": "flattened-batch linear layers TFLOP/s (config 2)", "value": round(value, 2), "unit": "TFLOP/s",
            "ms_per_step": round(tot_ms, 4), "dtype": "f32 and bf16 (fp32 accumulate)",
            "data": "synthetic (X N(0,1), W and bias N(0,0.02))",
            "config": {"workload": "c2_linear_layers", "d_model": 256, "M": [64, 512, 4096], "shapes": rows},
            "cpu_baseline": cpu}


def run_gemm_shapes(args, cbis, oracle):
    """Config 4's five bf16 GEMM shapes at M = 1216 on their own (random
    N(0,1) X, N(0,0.02) W, fp32 Y, the split-K workspace the runner gives
    them): a light target for rocprofv3 counter passes.  value = flop-weighted
    TFLOP/s of one layer's four projections plus lm_head."""
    import torch
    dev = torch.device("cuda:0")
    K_ = cbis.kernels()
    M = 1216
    ev = Events(None)
    stream = torch.cuda.current_stream().cuda_stream
    names = [s for s in (args.shapes or "qkv,out,fc1,fc2,lm_head").split(",")]
    dims = {"qkv": (6144, 2048), "out": (2048, 2048), "fc1": (8192, 2048), "fc2": (2048, 8192), "lm_head": (32000, 2048)}
    X = torch.empty((M, 8192), dtype=torch.bfloat16, device=dev)
    cbis.check(K_.cbis_fill_normal_fast(X.data_ptr(), cbis.BF16, X.numel(), 9, 1.0, None))
    res, fl_tot, ms_tot = {}, 0.0, 0.0
    for name in names:
        N, K = dims[name]
        W = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
        cbis.check(K_.cbis_fill_normal_fast(W.data_ptr(), cbis.BF16, W.numel(), 10, 0.02, None))
        Y = torch.empty((M, N), dtype=torch.float32, device=dev)
        d = cbis.GemmDesc()
        d.M, d.N, d.K = M, N, K
        d.x_dtype, d.X, d.ldx = cbis.BF16, X.data_ptr(), 8192
        d.w_dtype, d.W, d.ldw = cbis.BF16, W.data_ptr(), K
        d.y_dtype, d.Y, d.ldy = cbis.F32, Y.data_ptr(), N
        need = K_.cbis_gemm_workspace_size(ctypes.byref(d))
        ws = torch.empty(max(1, need // 4), dtype=torch.float32, device=dev)
        d.workspace, d.workspace_bytes = ws.data_ptr(), need
        fn = lambda d=d: cbis.check(K_.cbis_gemm(ctypes.byref(d), stream))
        ev.time(fn, max(1, args.warmup))
        ms = ev.time(fn, max(5, args.steps))
        fl = 2.0 * M * N * K
        res[name] = {"ms": round(ms, 4), "tflops": round(fl / ms / 1e9, 1)}
        fl_tot += fl
        ms_tot += ms
        _log(f"gemm {name}: {ms * 1000:.1f} us, {fl / ms / 1e9:.1f} TFLOP/s")
    value = fl_tot / ms_tot / 1e9
    return {"metric": "bf16 GEMM TFLOP/s on config 4's shapes (M=1216)", "value": round(value, 1),
            "unit": "TFLOP/s", "ms_per_step": round(ms_tot, 4), "dtype": "bf16 (fp32 accumulate)",
            "data": "synthetic (X N(0,1), W N(0,0.02))", "config": {"workload": "c4_gemm_shapes", "shapes": res},
            "roofline": {"bound": "mfma", "achieved": round(value, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(value / BF16_PEAK_TFLOPS, 4), "traffic": None},
            "cpu_baseline": None}


def run_tiering(args, cbis, oracle):
    """The reference's tiering scenario (src/bench_tiering.cpp): a
    32768-token prefix of the reference model (4 layers, 8x32 heads, fp32
    K/V: 2048 blocks of 128 KiB) spilled from the GPU to the DRAM tier and
    restored into fresh pages.  value = restored raw bytes per second of the
    batched restore (inflate on the host cores + one pinned H2D copy + one
    scatter launch per 256 MiB chunk); beside it the same restore one block
    per call (the reference's loop), the batched spill, and the scatter
    kernel alone (roofline: HBM, bytes read + written per launch)."""
    import tempfile
    import torch
    L, H, HD, PS, NB = 4, 8, 32, 16, 2048
    cache = cbis.PagedKVCache(L, 2 * NB, PS, H, HD, "f32", pages_per_seq=NB)
    cache.fill_normal(seed=11, std=1.0)
    tmp = tempfile.mkdtemp(prefix="cbis_tier_")
    mgr = cbis.TieredKVBlockManager(L, PS, H, HD, os.path.join(tmp, "scratch.nvme"), NB, NB)
    raw = mgr.raw_block_bytes()
    ids = list(range(NB))
    for b in ids:
        mgr.admit_gpu_resident(b, cache, b, 0)
    t0 = time.perf_counter()
    mgr.spill_batch(ids, "DRAM", 1)
    spill_s = time.perf_counter() - t0
    comp = mgr.stats()["compressed_bytes_total"]
    t0 = time.perf_counter()
    mgr.restore_batch(ids, cache, [NB + b for b in ids], 2)
    batch_s = time.perf_counter() - t0
    mgr.spill_batch(ids, "DRAM", 3)
    t0 = time.perf_counter()
    for b in ids:
        mgr.restore(b, cache, b, 4)
    single_s = time.perf_counter() - t0
    mgr.close()
    # the scatter kernel alone, device staging -> pages NB..2NB-1
    K_ = cbis.kernels()
    page_bytes = PS * H * HD * 4
    stage = torch.empty(NB * raw, dtype=torch.uint8, device="cuda:0")
    pages = torch.arange(NB, 2 * NB, dtype=torch.int32, device="cuda:0")
    ev = Events(None)
    stream = torch.cuda.current_stream().cuda_stream
    fn = lambda: cbis.check(K_.cbis_kv_pages_scatter(cache.k_base(0), stage.data_ptr(), L, 2 * NB, page_bytes,
                                                     pages.data_ptr(), NB, stream))
    ev.time(fn, max(1, args.warmup))
    ms = ev.time(fn, max(5, args.steps))
    kbytes = 2.0 * NB * raw
    kgbs = kbytes / ms / 1e6
    total = NB * raw
    value = total / batch_s / 1e9
    _log(f"tiering: spill {spill_s * 1e3:.1f} ms, batched restore {batch_s * 1e3:.1f} ms, "
         f"one-block restores {single_s * 1e3:.1f} ms, scatter kernel {ms * 1e3:.1f} us = {kgbs:.0f} GB/s")
    return {"metric": "DRAM-tier restore GB/s (raw K/V bytes) of a 2048-block prefix", "value": round(value, 2),
            "unit": "GB/s", "ms_per_step": round(batch_s * 1e3, 2), "dtype": "f32 K/V bytes (lossless)",
            "data": "synthetic (K/V N(0,1))",
            "config": {"workload": "tiering_prefix_restore", "blocks": NB, "block_bytes": raw,
                       "layers": L, "heads": f"{H}x{HD}", "page_size": PS,
                       "compressed_ratio": round(comp / total, 4),
                       "spill_ms": round(spill_s * 1e3, 2), "batched_restore_ms": round(batch_s * 1e3, 2),
                       "one_block_restores_ms": round(single_s * 1e3, 2),
                       "host_threads": int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()},
            "roofline": {"bound": "hbm", "kernel": "kv_pages_kernel<scatter>", "achieved": round(kgbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(kgbs / HBM_PEAK_GBS, 4),
                         "traffic": None, "algorithmic_bytes": int(kbytes), "ms": round(ms, 4)},
            "cpu_baseline": None}


def run_copy_calib(args):
    """A plain device-to-device copy of known size for PMC byte calibration."""
    import torch
    n = 1 << 28  # 1 GiB of fp32
    a = torch.ones(n, dtype=torch.float32, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    return {"metric": "copy calibration", "value": float(n * 4), "unit": "bytes read per launch"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=["c4", "c1", "c2", "c3", "c5", "gemm", "tiering"],
                    help="c4: the bench line (default); c1 / c2 / c3 / c5: the other configs; "
                         "gemm: config 4's GEMM shapes alone; tiering: the tiered K/V prefix restore")
    ap.add_argument("--shapes", default=None, help="--config gemm: comma list of qkv,out,fc1,fc2,lm_head")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--copy-calib", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every box here has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_calib:
        print(json.dumps(run_copy_calib(args)))
        return
    cbis = _cbis()
    import oracle
    if args.config != "c4":
        res = {"c1": run_c1, "c2": run_c2, "c3": run_c3, "c5": run_c5,
               "gemm": run_gemm_shapes, "tiering": run_tiering}[args.config](args, cbis, oracle)
        line = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1, "steps": args.steps,
                "warmup": args.warmup, "ms_per_step": res["ms_per_step"], "higher_is_better": True,
                "scaling": "weak", "vs_baseline": None, "dtype": res["dtype"], "data": res["data"],
                "config": res["config"], "roofline": res.get("roofline"), "cpu_baseline": res["cpu_baseline"]}
        print(json.dumps(line), flush=True)
        return
    res = run_c4(args, cbis, oracle)
    line = {"metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": res["ms_per_step"], "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": res["dtype"], "data": res["data"], "config": res["config"],
            "step_ms": res["step_ms"], "synchronous": res["synchronous"], "roofline": res["roofline"],
            "gemm_roofline": res["gemm_roofline"], "cpu_baseline": res["cpu_baseline"], "machine": res["machine"]}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
