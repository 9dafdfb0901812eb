"""CPU oracle for the per-step forward -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker (never as the thing measured or shipped).  The
product path (HIP kernels behind the C-ABI, C++ runtime) never touches it.

Contents (each restating the reference; citations are reference file:line):

* ctypes bindings of ``oracle/cbis_oracle.c`` (fp64 GEMM / LayerNorm /
  paged attention / whole forward step);
* :class:`PagedKVCacheOracle` -- ``src/paged_kv_cache.cpp:5-60`` bookkeeping
  (LIFO free list initialised [P-1..0], monotonic seq ids, zero-padded page
  tables) in plain Python;
* :func:`run_continuous` -- ``src/bench_batching.cpp:98-179`` (whole-prompt
  prefill rows, one decode row per active slot, greedy argmax with the first
  maximum winning, free at ``generated >= decode_len``);
* the synthetic weight specification (stream ids, N(0, 0.02) linear and
  embedding weights and biases, LayerNorm gamma=1 / beta=0, bf16 rounding,
  per-output-channel absmax fp8 e4m3 quantisation).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_D = ctypes.c_double


class _Layer(ctypes.Structure):
    _fields_ = [(n, _P) for n in (
        "ln1_w", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
        "ln2_w", "ln2_b", "fc1", "b1", "fc2", "b2",
        "sq", "sk", "sv", "so", "s1", "s2")]


class _Model(ctypes.Structure):
    _fields_ = [("vocab", _I), ("d_model", _I), ("n_heads", _I), ("head_dim", _I),
                ("n_layers", _I), ("mlp", _I), ("page_size", _I), ("act_bf16", _I),
                ("kv_dtype", _I), ("tok_emb", _P), ("pos_emb", _P), ("ln_f_w", _P),
                ("ln_f_b", _P), ("lm_head", _P), ("lm_scale", _P), ("layers", _P)]


def _declare(L):
    L.orc_key.restype = _U64
    L.orc_key.argtypes = [_U64, _U64]
    L.orc_u64.restype = _U64
    L.orc_u64.argtypes = [_U64, _U64]
    L.orc_normal_f32.argtypes = [_U64, _U64, _U64, _I64, _D, _P]
    L.orc_uniform_int.argtypes = [_U64, _U64, _U64, _I64, ctypes.c_int32, ctypes.c_int32, _P]
    L.orc_f32_to_bf16.restype = ctypes.c_uint16
    L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
    L.orc_bf16_to_f32.restype = ctypes.c_float
    L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_round_bf16.argtypes = [_P, _I64]
    L.orc_quantize_e4m3_rows.argtypes = [_I64, _I64, _P, _P, _P]
    L.orc_e4m3_to_f32.restype = ctypes.c_float
    L.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
    L.orc_f32_to_e4m3.restype = ctypes.c_uint8
    L.orc_f32_to_e4m3.argtypes = [ctypes.c_float]
    L.orc_gemm.argtypes = [_I, _I, _I, _P, _I, _P, _I, _P, _P, _I, _P, _I, _P, _I]
    L.orc_layernorm.argtypes = [_I, _I, _P, _I, _P, _P, _D, _P, _I]
    L.orc_embed.argtypes = [_I, _I, _P, _P, _P, _P, _P]
    L.orc_scatter_kv.argtypes = [_I, _I, _P, _P, _P, _P, _I, _P, _P, _I]
    L.orc_paged_attention.argtypes = [_I, _I, _I, _I, _P, _P, _I, _P, _I, _P, _P, _P, _I, _P, _I]
    L.orc_argmax_rows.argtypes = [_I, _I, _P, _I, _P]
    L.orc_forward_step.argtypes = [_P, _I, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P]
    L.orc_step_embed.argtypes = [_P, _I, _P, _P, _P]
    L.orc_step_layer.argtypes = [_P, _I, _I, _P, _P, _P, _P, _P, _I, _P, _P, _P]
    L.orc_step_head.argtypes = [_P, _I, _P, _P]
    L.orc_num_threads.restype = _I
    L.orc_set_num_threads.restype = _I
    L.orc_set_num_threads.argtypes = [_I]


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.int32)


# --------------------------------------------------------------------------
# PRNG and number formats
# --------------------------------------------------------------------------

def normal(seed: int, stream: int, n: int, std: float = 1.0, start: int = 0) -> np.ndarray:
    """std is an fp32 value (the product's C-ABI takes it as float); the
    variate is scaled by it in fp64 and rounded once to fp32."""
    out = np.empty(n, dtype=np.float32)
    lib().orc_normal_f32(seed, stream, start, n, float(np.float32(std)), _ptr(out))
    return out


def uniform_int(seed: int, stream: int, n: int, lo: int, hi_inclusive: int, start: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().orc_uniform_int(seed, stream, start, n, lo, hi_inclusive, _ptr(out))
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    lib().orc_round_bf16(_ptr(y), y.size)
    return y


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) of x rounded to nearest even."""
    y = round_bf16(x)
    return (y.view(np.uint32) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


_E4M3_TABLE = None


def e4m3_table() -> np.ndarray:
    global _E4M3_TABLE
    if _E4M3_TABLE is None:
        _E4M3_TABLE = np.array([lib().orc_e4m3_to_f32(i) for i in range(256)], dtype=np.float32)
    return _E4M3_TABLE


def f32_to_e4m3(x: np.ndarray) -> np.ndarray:
    f = lib().orc_f32_to_e4m3
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([f(float(v)) for v in flat], dtype=np.uint8).reshape(np.shape(x))


def quantize_e4m3_rows(w: np.ndarray):
    """Per-output-channel absmax fp8 e4m3: scale[n] = absmax(w[n,:]) / 448
    (fp32), q = e4m3_rne(w / scale).  Returns (codes uint8 [N,K], scale fp32 [N]).
    orc_quantize_e4m3_rows (C, rows in parallel); quantize_e4m3_rows_np is
    the same rule in numpy, the cross-check."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    codes = np.empty((N, K), np.uint8)
    scale = np.empty(N, np.float32)
    lib().orc_quantize_e4m3_rows(N, K, _ptr(w), _ptr(codes), _ptr(scale))
    return codes, scale


def quantize_e4m3_rows_np(w: np.ndarray):
    """quantize_e4m3_rows in numpy (vectorised encoder)."""
    w = np.asarray(w, dtype=np.float32)
    absmax = np.max(np.abs(w), axis=1).astype(np.float32)
    scale = (absmax / np.float32(448.0)).astype(np.float32)
    scale[scale == 0] = np.float32(1.0)
    scaled = (w / scale[:, None]).astype(np.float32)
    return _e4m3_encode_vec(scaled), scale


def _e4m3_encode_vec(a: np.ndarray) -> np.ndarray:
    """Vectorised twin of orc_f32_to_e4m3 (round half even, saturate 448)."""
    a = np.asarray(a, dtype=np.float32)
    sign = (np.signbit(a)).astype(np.uint8) << 7
    m = np.abs(a.astype(np.float64))
    code = np.zeros(a.shape, dtype=np.int32)
    sub = m < 2.0 ** -6
    code[sub] = np.rint(m[sub] * 512.0).astype(np.int32)
    nrm = ~sub
    mn = m[nrm]
    _, e = np.frexp(mn)
    E = e - 1
    q = np.rint(np.ldexp(mn, 3 - E))
    wrap = q == 16.0
    q[wrap] = 8.0
    E = E + wrap
    c = ((E + 7) << 3) | (q.astype(np.int32) - 8)
    code[nrm] = np.minimum(c, 0x7E)
    code[m >= 448.0] = 0x7E
    code[np.isnan(a)] = 0x7F
    return (code.astype(np.uint8) | sign).astype(np.uint8)


# --------------------------------------------------------------------------
# Kernel-level oracles (fp64)
# --------------------------------------------------------------------------

def gemm(X, W, w_scale=None, bias=None, gelu=False, residual=None) -> np.ndarray:
    X = _f32(X)
    W = _f32(W)
    M, K = X.shape
    N = W.shape[0]
    assert W.shape[1] == K
    res = _f32(residual)
    Y = np.empty((M, N), dtype=np.float64)
    lib().orc_gemm(M, N, K, _ptr(X), K, _ptr(W), K, _ptr(_f32(w_scale)), _ptr(_f32(bias)),
                   int(bool(gelu)), _ptr(res), N, _ptr(Y), N)
    return Y


def layernorm(X, g, b, eps=1e-5) -> np.ndarray:
    X = _f32(X)
    M, D = X.shape
    Y = np.empty((M, D), dtype=np.float64)
    lib().orc_layernorm(M, D, _ptr(X), D, _ptr(_f32(g)), _ptr(_f32(b)), eps, _ptr(Y), D)
    return Y


def paged_attention(q, kpool, vpool, block_table, row_pos, n_heads, head_dim, page_size,
                    row_bt=None, kv_dtype=0) -> np.ndarray:
    """q [M, H*hd] float; pools [P, page, H, hd] as float32 (kv_dtype 0) or
    uint16 bf16 bits (kv_dtype 1); block_table [R, stride] int32."""
    q = _f32(q)
    M = q.shape[0]
    bt = _i32(block_table)
    pos = _i32(row_pos)
    kp = np.ascontiguousarray(kpool)
    vp = np.ascontiguousarray(vpool)
    out = np.empty((M, n_heads * head_dim), dtype=np.float64)
    lib().orc_paged_attention(M, n_heads, head_dim, page_size, _ptr(kp), _ptr(vp), kv_dtype, _ptr(bt),
                              bt.shape[1], _ptr(_i32(row_bt)), _ptr(pos), _ptr(q), q.shape[1], _ptr(out),
                              out.shape[1])
    return out


def argmax_rows(logits) -> np.ndarray:
    lg = _f32(logits)
    out = np.empty(lg.shape[0], dtype=np.int32)
    lib().orc_argmax_rows(lg.shape[0], lg.shape[1], _ptr(lg), lg.shape[1], _ptr(out))
    return out


# --------------------------------------------------------------------------
# PagedKVCache bookkeeping, src/paged_kv_cache.cpp:5-60
# --------------------------------------------------------------------------

class PagedKVCacheOracle:
    """Allocation restated from src/paged_kv_cache.cpp (no device memory)."""

    def __init__(self, max_pages: int, page_size: int = 16, pages_per_seq: int = 2048):
        self.page_size = page_size
        self.pages_per_seq = pages_per_seq
        self.max_pages = max_pages
        self.free = list(range(max_pages - 1, -1, -1))  # :15-16, pop_back yields 0,1,2..
        self.seq_pages: dict[int, list[int]] = {}
        self.next_seq_id = 0

    def allocate_sequence(self) -> int:  # :24-28
        sid = self.next_seq_id
        self.next_seq_id += 1
        self.seq_pages[sid] = []
        return sid

    def free_sequence(self, sid: int) -> None:  # :30-35
        pages = self.seq_pages.pop(sid, None)
        if pages is None:
            return
        self.free.extend(pages)

    def ensure_capacity(self, sid: int, pos: int) -> bool:  # :37-46
        pages = self.seq_pages[sid]
        needed = pos // self.page_size + 1
        while len(pages) < needed:
            if not self.free:
                return False
            pages.append(self.free.pop())
        return True

    def resolve_slot(self, sid: int, pos: int):  # :48-53
        pages = self.seq_pages[sid]
        lp = pos // self.page_size
        if lp >= len(pages):
            raise IndexError("resolve_slot: position beyond the sequence's pages")
        return pages[lp], pos % self.page_size

    def page_table(self, sid: int) -> list[int]:  # :55-60
        pages = self.seq_pages[sid]
        t = [0] * self.pages_per_seq
        for i, p in enumerate(pages[: self.pages_per_seq]):
            t[i] = p
        return t

    def num_free_pages(self) -> int:
        return len(self.free)


# --------------------------------------------------------------------------
# Model spec and synthetic weights
# --------------------------------------------------------------------------

@dataclass
class ModelSpec:
    vocab: int = 1000
    d_model: int = 256
    n_heads: int = 8
    head_dim: int = 32
    n_layers: int = 4
    mlp: int = 1024
    max_seq: int = 32768
    page_size: int = 16
    weight_dtype: str = "f32"   # f32 | bf16 | fp8
    kv_dtype: str = "f32"       # f32 | bf16

    @property
    def act_bf16(self) -> bool:
        return self.weight_dtype != "f32"


# Stream ids of the synthetic weights (seeded N(0, std) per tensor, element
# index = row-major offset).  Mirrored by the product's ModelWeights.
STREAM_TOK_EMB = 1
STREAM_POS_EMB = 2
STREAM_LM_HEAD = 3
LAYER_STREAM_BASE = 100
LAYER_STREAM_STRIDE = 20
LAYER_TENSORS = ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "fc1", "b1", "fc2", "b2")


def layer_stream(layer: int, name: str) -> int:
    return LAYER_STREAM_BASE + LAYER_STREAM_STRIDE * layer + LAYER_TENSORS.index(name)


@dataclass
class Weights:
    """fp32 master weights plus the dequantised values the forward uses."""
    spec: ModelSpec
    master: dict = field(default_factory=dict)   # name -> fp32 array (as generated)
    used: dict = field(default_factory=dict)     # name -> fp32 array the math consumes
    scale: dict = field(default_factory=dict)    # name -> per-row fp32 scale (fp8 only)


def synthetic_weights(spec: ModelSpec, seed: int = 0, std: float = 0.02, pos_rows: int | None = None) -> Weights:
    """Generates every tensor of the spec.  pos_rows limits how many pos_emb
    rows are materialised (the values of row p do not depend on it)."""
    D, F, V = spec.d_model, spec.mlp, spec.vocab
    pr = spec.max_seq if pos_rows is None else pos_rows
    w = Weights(spec)
    m = w.master
    m["tok_emb"] = normal(seed, STREAM_TOK_EMB, V * D, std).reshape(V, D)
    m["pos_emb"] = normal(seed, STREAM_POS_EMB, pr * D, std).reshape(pr, D)
    m["lm_head"] = normal(seed, STREAM_LM_HEAD, V * D, std).reshape(V, D)
    m["ln_f_w"] = np.ones(D, np.float32)
    m["ln_f_b"] = np.zeros(D, np.float32)
    shapes = {"wq": (D, D), "bq": (D,), "wk": (D, D), "bk": (D,), "wv": (D, D), "bv": (D,),
              "wo": (D, D), "bo": (D,), "fc1": (F, D), "b1": (F,), "fc2": (D, F), "b2": (D,)}
    for l in range(spec.n_layers):
        for name, shp in shapes.items():
            m[f"l{l}.{name}"] = normal(seed, layer_stream(l, name), int(np.prod(shp)), std).reshape(shp)
        m[f"l{l}.ln1_w"] = np.ones(D, np.float32)
        m[f"l{l}.ln1_b"] = np.zeros(D, np.float32)
        m[f"l{l}.ln2_w"] = np.ones(D, np.float32)
        m[f"l{l}.ln2_b"] = np.zeros(D, np.float32)
    _derive_used(w)
    return w


def is_linear_weight(name: str) -> bool:
    base = name.split(".")[-1]
    return base in ("wq", "wk", "wv", "wo", "fc1", "fc2", "lm_head")


def _derive_used(w: Weights) -> None:
    spec = w.spec
    for name, arr in w.master.items():
        base = name.split(".")[-1]
        if spec.weight_dtype == "f32" or base.startswith("ln") or base.startswith("b"):
            w.used[name] = arr
        elif spec.weight_dtype == "bf16" or base in ("tok_emb", "pos_emb"):
            w.used[name] = round_bf16(arr)
        else:  # fp8 linear weights
            codes, sc = quantize_e4m3_rows(arr)
            w.used[name] = e4m3_table().take(codes.astype(np.intp))
            w.scale[name] = sc


def load_weights_bin(path: str, spec: ModelSpec) -> Weights:
    """python/export_weights.py:42-66 order, all fp32."""
    D, F, V = spec.d_model, spec.mlp, spec.vocab
    raw = np.fromfile(path, dtype=np.float32)
    off = 0

    def take(*shape):
        nonlocal off
        n = int(np.prod(shape))
        if off + n > raw.size:
            raise ValueError("weights.bin truncated")
        a = raw[off: off + n].reshape(shape)
        off += n
        return a

    w = Weights(spec)
    m = w.master
    m["tok_emb"] = take(V, D)
    m["pos_emb"] = take(spec.max_seq, D)
    for l in range(spec.n_layers):
        m[f"l{l}.ln1_w"] = take(D); m[f"l{l}.ln1_b"] = take(D)
        m[f"l{l}.wq"] = take(D, D); m[f"l{l}.bq"] = take(D)
        m[f"l{l}.wk"] = take(D, D); m[f"l{l}.bk"] = take(D)
        m[f"l{l}.wv"] = take(D, D); m[f"l{l}.bv"] = take(D)
        m[f"l{l}.wo"] = take(D, D); m[f"l{l}.bo"] = take(D)
        m[f"l{l}.ln2_w"] = take(D); m[f"l{l}.ln2_b"] = take(D)
        m[f"l{l}.fc1"] = take(F, D); m[f"l{l}.b1"] = take(F)
        m[f"l{l}.fc2"] = take(D, F); m[f"l{l}.b2"] = take(D)
    m["ln_f_w"] = take(D)
    m["ln_f_b"] = take(D)
    m["lm_head"] = take(V, D)
    _derive_used(w)
    return w


# --------------------------------------------------------------------------
# Whole forward step over host paged pools
# --------------------------------------------------------------------------

class OracleModel:
    """Holds ctypes views of the weights and per-layer host K/V pools."""

    def __init__(self, weights: Weights, max_pages: int):
        self.w = weights
        s = weights.spec
        self.spec = s
        kv_np = np.float32 if s.kv_dtype == "f32" else np.uint16
        shape = (max_pages, s.page_size, s.n_heads, s.head_dim)
        self.kpools = [np.zeros(shape, kv_np) for _ in range(s.n_layers)]
        self.vpools = [np.zeros(shape, kv_np) for _ in range(s.n_layers)]
        u = weights.used
        self._keep = []
        layers = (_Layer * s.n_layers)()
        for l in range(s.n_layers):
            L = layers[l]
            for f, key in (("ln1_w", "ln1_w"), ("ln1_b", "ln1_b"), ("wq", "wq"), ("bq", "bq"),
                           ("wk", "wk"), ("bk", "bk"), ("wv", "wv"), ("bv", "bv"), ("wo", "wo"),
                           ("bo", "bo"), ("ln2_w", "ln2_w"), ("ln2_b", "ln2_b"), ("fc1", "fc1"),
                           ("b1", "b1"), ("fc2", "fc2"), ("b2", "b2")):
                setattr(L, f, self._p(u[f"l{l}.{key}"]))
            for f, key in (("sq", "wq"), ("sk", "wk"), ("sv", "wv"), ("so", "wo"), ("s1", "fc1"), ("s2", "fc2")):
                sc = weights.scale.get(f"l{l}.{key}")
                setattr(L, f, self._p(sc) if sc is not None else None)
        self._layers = layers
        mdl = _Model()
        mdl.vocab, mdl.d_model, mdl.n_heads, mdl.head_dim = s.vocab, s.d_model, s.n_heads, s.head_dim
        mdl.n_layers, mdl.mlp, mdl.page_size = s.n_layers, s.mlp, s.page_size
        mdl.act_bf16 = int(s.act_bf16)
        mdl.kv_dtype = 0 if s.kv_dtype == "f32" else 1
        mdl.tok_emb = self._p(u["tok_emb"])
        mdl.pos_emb = self._p(u["pos_emb"])
        mdl.ln_f_w = self._p(u["ln_f_w"])
        mdl.ln_f_b = self._p(u["ln_f_b"])
        mdl.lm_head = self._p(u["lm_head"])
        sc = weights.scale.get("lm_head")
        mdl.lm_scale = self._p(sc) if sc is not None else None
        mdl.layers = ctypes.cast(layers, ctypes.c_void_p)
        self._mdl = mdl
        self._kp = (ctypes.c_void_p * s.n_layers)(*[p.ctypes.data for p in self.kpools])
        self._vp = (ctypes.c_void_p * s.n_layers)(*[p.ctypes.data for p in self.vpools])

    def _p(self, arr):
        a = np.ascontiguousarray(arr, dtype=np.float32)
        self._keep.append(a)
        return a.ctypes.data_as(ctypes.c_void_p)

    def forward_step(self, token_ids, positions, wpage, woff, block_table, row_bt=None) -> np.ndarray:
        """Returns [M, vocab] float64 logits; block_table [R, stride]."""
        tok = _i32(token_ids)
        pos = _i32(positions)
        M = tok.size
        bt = _i32(block_table)
        out = np.empty((M, self.spec.vocab), dtype=np.float64)
        rb = _i32(row_bt) if row_bt is not None else None
        lib().orc_forward_step(ctypes.byref(self._mdl), M, _ptr(tok), _ptr(pos), _ptr(_i32(wpage)),
                               _ptr(_i32(woff)), _ptr(bt), bt.shape[1], _ptr(rb), self._kp, self._vp,
                               _ptr(out))
        return out


    # The same step one layer at a time (orc_step_embed / orc_step_layer /
    # orc_step_head; forward_step is exactly their sequence): a caller can
    # hold one layer's pools on the host at a time.
    def embed(self, token_ids, positions) -> np.ndarray:
        """Residual stream [M, d_model] (float64) of the step's rows."""
        tok, pos = _i32(token_ids), _i32(positions)
        x = np.empty((tok.size, self.spec.d_model), dtype=np.float64)
        lib().orc_step_embed(ctypes.byref(self._mdl), tok.size, _ptr(tok), _ptr(pos), _ptr(x))
        return x

    def layer(self, l, x, positions, wpage, woff, block_table, row_bt, kpool, vpool) -> None:
        """Layer l on x in place; K/V of the rows are written into kpool /
        vpool (this layer's [P, page, H, hd] pools, float32 or uint16 bf16
        bits, contiguous) before its attention reads them."""
        assert x.dtype == np.float64 and x.flags.c_contiguous
        assert kpool.flags.c_contiguous and vpool.flags.c_contiguous
        pos, bt = _i32(positions), _i32(block_table)
        lib().orc_step_layer(ctypes.byref(self._mdl), l, x.shape[0], _ptr(x), _ptr(pos), _ptr(_i32(wpage)),
                             _ptr(_i32(woff)), _ptr(bt), bt.shape[1], _ptr(_i32(row_bt)), _ptr(kpool), _ptr(vpool))

    def head(self, x) -> np.ndarray:
        """Final LayerNorm + lm_head: [M, vocab] float64 logits."""
        out = np.empty((x.shape[0], self.spec.vocab), dtype=np.float64)
        lib().orc_step_head(ctypes.byref(self._mdl), x.shape[0], _ptr(np.ascontiguousarray(x)), _ptr(out))
        return out


def step_tables(cache, token_ids, positions, seq_ids):
    """src/transformer.cpp:51-57: each row's write slot and a compact block
    table (one row per distinct sequence, row_bt[i] its index) from a cache
    with the reference's API (resolve_slot, and pages(seq) or seq_pages).
    Returns (wpage, woff, block_table, row_bt)."""
    M = len(token_ids)
    wpage = np.empty(M, np.int32)
    woff = np.empty(M, np.int32)
    uniq = {}
    row_bt = np.empty(M, np.int32)
    for i in range(M):
        wpage[i], woff[i] = cache.resolve_slot(seq_ids[i], positions[i])
        if seq_ids[i] not in uniq:
            uniq[seq_ids[i]] = len(uniq)
        row_bt[i] = uniq[seq_ids[i]]
    pages = {s: (cache.pages(s) if hasattr(cache, "pages") else cache.seq_pages[s]) for s in uniq}
    width = max(1, max(len(p) for p in pages.values()))
    table = np.zeros((len(uniq), width), np.int32)
    for s, j in uniq.items():
        table[j, : len(pages[s])] = pages[s]
    return wpage, woff, table, row_bt


def forward_step_with_cache(model: OracleModel, cache: PagedKVCacheOracle, token_ids, positions, seq_ids):
    """src/transformer.cpp:51-57: resolve each row's write slot and page table
    from the cache (the caller already ran ensure_capacity), then run."""
    wpage, woff, table, row_bt = step_tables(cache, token_ids, positions, seq_ids)
    return model.forward_step(token_ids, positions, wpage, woff, table, row_bt)


# --------------------------------------------------------------------------
# Continuous-batching scheduler, src/bench_batching.cpp:98-179
# --------------------------------------------------------------------------

@dataclass
class Request:
    prompt: list
    decode_len: int


def run_continuous(model: OracleModel, cache: PagedKVCacheOracle, requests: list, max_slots: int = 16,
                   record_logits: bool = False):
    """All requests are taken as arrived at t=0 (the C1 workload).  Returns
    (generated tokens per request, per-step last-row logits if asked)."""
    slots = [None] * max_slots
    nxt = 0
    done = 0
    gen = [[] for _ in requests]
    step_logits = []
    while done < len(requests):
        for i in range(max_slots):
            if slots[i] is None and nxt < len(requests):
                slots[i] = {"req": nxt, "seq": cache.allocate_sequence(), "next_pos": 0,
                            "prefilled": False, "last": 0, "generated": 0}
                nxt += 1
        toks, poss, sids, owner, last = [], [], [], [], []
        for i, s in enumerate(slots):
            if s is None:
                continue
            r = requests[s["req"]]
            if not s["prefilled"]:
                for p in range(len(r.prompt)):
                    if not cache.ensure_capacity(s["seq"], p):
                        raise RuntimeError("OOM pages")
                    toks.append(r.prompt[p]); poss.append(p); sids.append(s["seq"])
                    owner.append(i); last.append(p == len(r.prompt) - 1)
                s["next_pos"] = len(r.prompt)
                s["prefilled"] = True
            else:
                if not cache.ensure_capacity(s["seq"], s["next_pos"]):
                    raise RuntimeError("OOM pages")
                toks.append(s["last"]); poss.append(s["next_pos"]); sids.append(s["seq"])
                owner.append(i); last.append(True)
                s["next_pos"] += 1
        logits = forward_step_with_cache(model, cache, toks, poss, sids)
        lf = logits.astype(np.float32)
        rec = {}
        for row in range(len(toks)):
            if not last[row]:
                continue
            i = owner[row]
            s = slots[i]
            tok = int(argmax_rows(lf[row: row + 1])[0])
            rec[s["req"]] = logits[row]
            s["last"] = tok
            s["generated"] += 1
            gen[s["req"]].append(tok)
            if s["generated"] >= requests[s["req"]].decode_len:
                cache.free_sequence(s["seq"])
                slots[i] = None
                done += 1
        if record_logits:
            step_logits.append(rec)
    return gen, step_logits


# --------------------------------------------------------------------------
# Workload generators shared by tests and bench (our own spec)
# --------------------------------------------------------------------------

STREAM_C1_PROMPT_LEN = 1001
STREAM_C1_TOKENS = 1002


def c1_requests(seed: int = 0, n: int = 8, vocab: int = 512, lo: int = 16, hi: int = 64, decode_len: int = 32):
    lens = uniform_int(seed, STREAM_C1_PROMPT_LEN, n, lo, hi)
    reqs = []
    for i in range(n):
        toks = uniform_int(seed, STREAM_C1_TOKENS, int(lens[i]), 0, vocab - 1, start=i * 4096)
        reqs.append(Request([int(t) for t in toks], decode_len))
    return reqs


def scatter_kv(K, V, kpool, vpool, wpage, woff, page_size, kv_dtype=0) -> None:
    """In place: kpool/vpool[page][slot] = K/V rows (kernels/attention.cu:7-19);
    pools float32 (kv_dtype 0) or uint16 bf16 bits (kv_dtype 1)."""
    Kd = np.ascontiguousarray(K, dtype=np.float64)
    Vd = np.ascontiguousarray(V, dtype=np.float64)
    M, D = Kd.shape
    assert kpool.flags.c_contiguous and vpool.flags.c_contiguous
    lib().orc_scatter_kv(M, D, _ptr(Kd), _ptr(Vd), _ptr(kpool), _ptr(vpool), kv_dtype, _ptr(_i32(wpage)),
                         _ptr(_i32(woff)), page_size)
