"""ctypes binding of the MI355X libraries (include/cbis_kernels.h and
include/cbis_runtime.h) with Python twins of the reference's host classes:

    PagedKVCache       include/paged_kv_cache.hpp:17-51
    ModelWeights       include/model_weights.hpp:7-25
    TransformerRunner  include/transformer.hpp:15-34
    run_continuous     src/bench_batching.cpp:98-179

The compute is the HIP code in lib/libcbis_kernels.so, reached through the
C-ABI; nothing here computes on the CPU.  Importing fails loudly when the
libraries have not been built (``make -C`` this directory, or
``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
KERNELS_SO = os.path.join(LIB_DIR, "libcbis_kernels.so")
# CBIS_RUNTIME_SO selects another build of the runtime library (the host
# sanitizer build, `make sanitize`).
RUNTIME_SO = os.environ.get("CBIS_RUNTIME_SO") or os.path.join(LIB_DIR, "libcbis.so")

F32, BF16, FP8E4M3 = 0, 1, 2
EPI_NONE, EPI_GELU = 0, 1
DTYPES = {"f32": F32, "bf16": BF16, "fp8": FP8E4M3}

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_IP = ctypes.POINTER(ctypes.c_int)


class GemmDesc(ctypes.Structure):
    _fields_ = [("M", _I), ("N", _I), ("K", _I),
                ("x_dtype", _I), ("X", _P), ("ldx", _I64),
                ("w_dtype", _I), ("W", _P), ("ldw", _I64),
                ("w_scale", _P), ("bias", _P), ("epilogue", _I),
                ("residual", _P), ("ldr", _I64),
                ("y_dtype", _I), ("Y", _P), ("ldy", _I64),
                ("kv_col0", _I), ("kv_width", _I), ("kv_dtype", _I), ("page_size", _I),
                ("k_pool", _P), ("v_pool", _P), ("write_page", _P), ("write_offset", _P),
                ("workspace", _P), ("workspace_bytes", _SZ)]


class AttnDesc(ctypes.Structure):
    _fields_ = [("n_rows", _I), ("rows", _P), ("n_heads", _I), ("head_dim", _I), ("page_size", _I),
                ("q_dtype", _I), ("q", _P), ("ldq", _I64),
                ("kv_dtype", _I), ("k_pool", _P), ("v_pool", _P), ("num_pages", _I),
                ("block_table", _P), ("bt_stride", _I64), ("row_bt", _P), ("row_pos", _P),
                ("out_dtype", _I), ("out", _P), ("ldo", _I64),
                ("max_kv_len", _I), ("split_tokens", _I), ("workspace", _P), ("workspace_bytes", _SZ),
                ("tile_pages", _I)]


class EvictionParams(ctypes.Structure):
    """include/tiered_kv_manager.hpp:40-48."""
    _fields_ = [("alpha_staleness", ctypes.c_double), ("beta_restore_cost", ctypes.c_double),
                ("expected_compression_ratio", ctypes.c_double), ("dram_fixed_ns", ctypes.c_double),
                ("dram_ns_per_byte", ctypes.c_double), ("nvme_fixed_ns", ctypes.c_double),
                ("nvme_ns_per_byte", ctypes.c_double)]


class ModelConfig(ctypes.Structure):
    _fields_ = [("vocab", _I), ("d_model", _I), ("n_heads", _I), ("head_dim", _I), ("n_layers", _I),
                ("mlp", _I), ("max_seq", _I), ("page_size", _I), ("weight_dtype", _I), ("kv_dtype", _I)]

    @classmethod
    def make(cls, vocab=1000, d_model=256, n_heads=8, head_dim=32, n_layers=4, mlp=1024, max_seq=32768,
             page_size=16, weight_dtype="f32", kv_dtype="f32"):
        return cls(vocab, d_model, n_heads, head_dim, n_layers, mlp, max_seq, page_size,
                   DTYPES[weight_dtype] if isinstance(weight_dtype, str) else weight_dtype,
                   DTYPES[kv_dtype] if isinstance(kv_dtype, str) else kv_dtype)


# Every symbol the two headers declare, with its ctypes signature.
KERNEL_SYMBOLS = {
    "cbis_last_error": (ctypes.c_char_p, []),
    "cbis_linear_forward": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "cbis_embed_lookup_add": (_I, [_P, _P, _P, _P, _P, _I, _I, _P]),
    "cbis_layernorm_forward": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "cbis_gelu_forward": (_I, [_P, _I, _I, _P]),
    "cbis_residual_add": (_I, [_P, _P, _I, _I, _P]),
    "cbis_scatter_kv_to_cache": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "cbis_fused_paged_causal_attention": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "cbis_gemm": (_I, [ctypes.POINTER(GemmDesc), _P]),
    "cbis_gemm_layernorm": (_I, [ctypes.POINTER(GemmDesc), _P, _P, _F, _I, _P, _I64, _P]),
    "cbis_layernorm_gemm": (_I, [ctypes.POINTER(GemmDesc), _P, _I64, _P, _P, _F, _P]),
    "cbis_kv_pages_gather": (_I, [_P, _P, _I, _I, ctypes.c_int64, _P, _I, _P]),
    "cbis_kv_pages_scatter": (_I, [_P, _P, _I, _I, ctypes.c_int64, _P, _I, _P]),
    "cbis_gemm_workspace_size": (_SZ, [ctypes.POINTER(GemmDesc)]),
    "cbis_gemm_layernorm_workspace_size": (_SZ, [ctypes.POINTER(GemmDesc)]),
    "cbis_gemm_argmax_workspace_size": (_SZ, [ctypes.POINTER(GemmDesc)]),
    "cbis_gemm_argmax": (_I, [ctypes.POINTER(GemmDesc), _P, _P, _P, _SZ, _P]),
    "cbis_layernorm_gemm_argmax": (_I, [ctypes.POINTER(GemmDesc), _P, _I64, _P, _P, _F, _P, _P, _P, _SZ, _P]),
    "cbis_paged_attention_workspace_size": (_SZ, [ctypes.POINTER(AttnDesc)]),
    "cbis_paged_attention": (_I, [ctypes.POINTER(AttnDesc), _P]),
    "cbis_paged_attention_static": (_I, [ctypes.POINTER(AttnDesc), _P]),
    "cbis_paged_attention_proj": (_I, [ctypes.POINTER(AttnDesc), ctypes.POINTER(GemmDesc), _P]),
    "cbis_paged_prefill_attention": (_I, [ctypes.POINTER(AttnDesc), _I, _P, _P]),
    "cbis_paged_attention_mixed": (_I, [ctypes.POINTER(AttnDesc), _I, _P, _P]),
    "cbis_embed": (_I, [_I, _I, _P, _P, _I, _P, _P, _I, _I, _P, _P]),
    "cbis_embed_from": (_I, [_I, _I, _P, _P, _P, _P, _I, _P, _P, _I, _I, _P, _P, _P, _SZ, _P]),
    "cbis_layernorm": (_I, [_I, _I, _P, _I64, _P, _P, _F, _I, _P, _I64, _P]),
    "cbis_argmax_rows": (_I, [_I, _I, _P, _I64, _P, _P]),
    "cbis_fill_normal_exact": (_I, [_P, _I, _I64, _U64, _U64, _U64, _F, _P]),
    "cbis_fill_normal_fast": (_I, [_P, _I, _I64, _U64, _F, _P]),
    "cbis_convert_f32": (_I, [_P, _I, _P, _I64, _P]),
    "cbis_quantize_fp8_rows": (_I, [_P, _P, _P, _I, _I, _P]),
}

RUNTIME_SYMBOLS = {
    "cbis_runtime_last_error": (ctypes.c_char_p, []),
    "cbis_default_config": (None, [ctypes.POINTER(ModelConfig)]),
    "cbis_cache_create": (_P, [_I, _I, _I, _I, _I, _I, _I, _I]),
    "cbis_cache_destroy": (None, [_P]),
    "cbis_cache_allocate_sequence": (_I, [_P]),
    "cbis_cache_free_sequence": (None, [_P, _I]),
    "cbis_cache_ensure_capacity": (_I, [_P, _I, _I]),
    "cbis_cache_resolve_slot": (_I, [_P, _I, _I, _IP, _IP]),
    "cbis_cache_page_table": (_I, [_P, _I, _IP, _I]),
    "cbis_cache_seq_pages": (_I, [_P, _I, _IP, _I]),
    "cbis_cache_num_free_pages": (_I, [_P]),
    "cbis_cache_max_pages": (_I, [_P]),
    "cbis_cache_page_size": (_I, [_P]),
    "cbis_cache_k_base": (_P, [_P, _I]),
    "cbis_cache_v_base": (_P, [_P, _I]),
    "cbis_cache_fill_normal": (_I, [_P, _U64, _F]),
    "cbis_weights_synthetic": (_P, [ctypes.POINTER(ModelConfig), _U64, _F]),
    "cbis_weights_load": (_P, [ctypes.c_char_p, ctypes.POINTER(ModelConfig)]),
    "cbis_weights_save_packed": (_I, [_P, ctypes.c_char_p]),
    "cbis_weights_load_packed": (_P, [ctypes.c_char_p, ctypes.POINTER(ModelConfig)]),
    "cbis_weights_destroy": (None, [_P]),
    "cbis_weights_device_bytes": (_SZ, [_P]),
    "cbis_weights_tensor": (_P, [_P, ctypes.c_char_p]),
    "cbis_runner_create": (_P, [_P, _P, _I]),
    "cbis_runner_destroy": (None, [_P]),
    "cbis_runner_forward_step": (_I, [_P, _I, _IP, _IP, _IP, ctypes.POINTER(ctypes.c_float)]),
    "cbis_runner_forward_step_greedy": (_I, [_P, _I, _IP, _IP, _IP, _IP]),
    "cbis_runner_enqueue_greedy": (_I, [_P, _I, _IP, _IP, _IP, _IP, ctypes.POINTER(ctypes.c_int64)]),
    "cbis_runner_wait_greedy": (_I, [_P, ctypes.c_int64, _IP, _I]),
    "cbis_runner_logits_device": (_P, [_P]),
    "cbis_runner_stream": (_P, [_P]),
    "cbis_runner_set_graphs": (None, [_P, _I]),
    "cbis_runner_set_fused_decode": (None, [_P, _I]),
    "cbis_runner_last_plan": (_I, [_P, _IP, _I]),
    "cbis_runner_last_device_ms": (ctypes.c_float, [_P]),
    "cbis_runner_last_host_ms": (None, [_P, ctypes.POINTER(ctypes.c_double)]),
    "cbis_runner_last_margins": (_I, [_P, ctypes.POINTER(ctypes.c_float), _I]),
    "cbis_run_continuous": (_I, [_P, _P, _I, _IP, _IP, _IP, _I, _IP, ctypes.POINTER(ctypes.c_double), _I]),
    "cbis_eviction_params_default": (None, [ctypes.POINTER(EvictionParams)]),
    "cbis_tiered_create": (_P, [_I, _I, _I, _I, _I, ctypes.c_char_p, _SZ, _SZ, ctypes.POINTER(EvictionParams)]),
    "cbis_tiered_destroy": (None, [_P]),
    "cbis_tiered_raw_block_bytes": (_SZ, [_P]),
    "cbis_tiered_calibrate": (_I, [_P]),
    "cbis_tiered_params": (_I, [_P, ctypes.POINTER(EvictionParams)]),
    "cbis_tiered_admit_gpu_resident": (_I, [_P, ctypes.c_uint64, _P, _I, ctypes.c_long]),
    "cbis_tiered_evict_one": (_I, [_P, ctypes.c_long, ctypes.POINTER(ctypes.c_uint64)]),
    "cbis_tiered_spill": (_I, [_P, ctypes.c_uint64, _I, ctypes.c_long]),
    "cbis_tiered_restore": (_I, [_P, ctypes.c_uint64, _P, _I, ctypes.c_long]),
    "cbis_tiered_spill_batch": (_I, [_P, ctypes.POINTER(ctypes.c_uint64), _I, _I, ctypes.c_long]),
    "cbis_tiered_restore_batch": (_I, [_P, ctypes.POINTER(ctypes.c_uint64), _I, _P, _IP, ctypes.c_long]),
    "cbis_tiered_tier_of": (_I, [_P, ctypes.c_uint64]),
    "cbis_tiered_known": (_I, [_P, ctypes.c_uint64]),
    "cbis_tiered_touch": (_I, [_P, ctypes.c_uint64, ctypes.c_long]),
    "cbis_tiered_stats": (_I, [_P, ctypes.POINTER(_SZ)]),
    "cbis_block_deflate": (ctypes.c_int64, [_P, _SZ, _P, _SZ]),
    "cbis_block_inflate": (_I, [_P, _SZ, _P, _SZ]),
    "cbis_run_continuous_chunked": (_I, [_P, _P, _I, _IP, _IP, _IP, _I, _I, _I, _IP,
                                         ctypes.POINTER(ctypes.c_double), _I]),
    "cbis_schedule_dry_run": (_I, [_P, _I, _IP, _IP, _IP, _I, _I, _I, _I, _IP, _IP, _I, _IP, _IP, _IP, _I]),
    "cbis_run_continuous_timed": (_I, [_P, _P, _I, _IP, _IP, _IP, ctypes.POINTER(ctypes.c_double), _I, _I, _I, _IP,
                                       ctypes.POINTER(ctypes.c_double), _I, ctypes.POINTER(ctypes.c_double)]),
    "cbis_schedule_dry_run_timed": (_I, [_P, _I, _IP, _IP, _IP, ctypes.POINTER(ctypes.c_double), ctypes.c_double, _I,
                                         _I, _I, _I, _IP, _IP, _I, _IP, _IP, _IP, _I,
                                         ctypes.POINTER(ctypes.c_double)]),
    "cbis_run_continuous_pipelined": (_I, [_P, _P, _I, _IP, _IP, _IP, ctypes.POINTER(ctypes.c_double), _I, _I, _I,
                                           _IP, ctypes.POINTER(ctypes.c_double), _I, ctypes.POINTER(ctypes.c_double)]),
    "cbis_schedule_dry_run_pipelined": (_I, [_P, _I, _IP, _IP, _IP, ctypes.POINTER(ctypes.c_double), ctypes.c_double,
                                             _I, _I, _I, _I, _IP, _IP, _I, _IP, _IP, _IP, _I,
                                             ctypes.POINTER(ctypes.c_double)]),
}

_kern = None
_rt = None


def _load(path, symbols):
    if not os.path.exists(path):
        raise ImportError(f"{path} is not built: run __graft_entry__.build() (the HIP path has no CPU fallback)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in symbols.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def kernels():
    global _kern
    if _kern is None:
        _kern = _load(KERNELS_SO, KERNEL_SYMBOLS)
    return _kern


def runtime():
    global _rt
    if _rt is None:
        kernels()
        _rt = _load(RUNTIME_SO, RUNTIME_SYMBOLS)
    return _rt


class CbisError(RuntimeError):
    pass


def check(rc, what="cbis"):
    if rc != 0:
        msg = kernels().cbis_last_error()
        raise CbisError(f"{what} failed with status {rc}: {msg.decode() if msg else ''}")


def _rt_check(rc, what):
    if rc is None or (isinstance(rc, int) and rc < 0):
        msg = runtime().cbis_runtime_last_error()
        text = msg.decode() if msg else ""
        if text.startswith("out_of_range"):
            raise IndexError(f"{what}: {text}")
        raise CbisError(f"{what}: {text}")
    return rc


def _iarr(vals):
    """int32 C view of `vals` for an `int*` argument.  A C-contiguous numpy
    int32 array is passed without a copy; anything else is converted once
    through numpy (integers outside int32 raise OverflowError).  The returned
    pointer keeps its array alive for the call."""
    a = np.ascontiguousarray(vals, dtype=np.int32)
    if a.ndim != 1:
        a = a.reshape(-1)
    if a.size == 0:
        a = np.zeros(1, dtype=np.int32)
    return a.ctypes.data_as(_IP)


# --------------------------------------------------------------------------
# Reference-API twins
# --------------------------------------------------------------------------

class PagedKVCache:
    """src/paged_kv_cache.cpp semantics; device pools optional."""

    _h = None

    def __init__(self, num_layers, max_pages, page_size=16, n_heads=8, head_dim=32, kv_dtype="f32",
                 pages_per_seq=2048, alloc_device=True):
        self._h = _rt_check(runtime().cbis_cache_create(num_layers, max_pages, page_size, n_heads, head_dim,
                                                        DTYPES[kv_dtype], pages_per_seq, int(alloc_device)),
                            "PagedKVCache")
        self.num_layers, self.n_heads, self.head_dim = num_layers, n_heads, head_dim
        self.kv_dtype, self.pages_per_seq = kv_dtype, pages_per_seq

    def close(self):
        if self._h:
            runtime().cbis_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        # At interpreter exit the module globals may already be gone; the
        # process teardown releases the device memory then.
        try:
            self.close()
        except Exception:
            pass

    def allocate_sequence(self) -> int:
        return _rt_check(runtime().cbis_cache_allocate_sequence(self._h), "allocate_sequence")

    def free_sequence(self, seq_id: int) -> None:
        runtime().cbis_cache_free_sequence(self._h, seq_id)

    def ensure_capacity(self, seq_id: int, token_pos: int) -> bool:
        return bool(_rt_check(runtime().cbis_cache_ensure_capacity(self._h, seq_id, token_pos), "ensure_capacity"))

    def resolve_slot(self, seq_id: int, token_pos: int):
        p, o = ctypes.c_int(), ctypes.c_int()
        _rt_check(runtime().cbis_cache_resolve_slot(self._h, seq_id, token_pos, ctypes.byref(p), ctypes.byref(o)),
                  "resolve_slot")
        return p.value, o.value

    def page_table(self, seq_id: int) -> list:
        buf = (ctypes.c_int * self.pages_per_seq)()
        n = _rt_check(runtime().cbis_cache_page_table(self._h, seq_id, buf, self.pages_per_seq), "page_table")
        return list(buf[:n])

    def pages(self, seq_id: int) -> list:
        n = _rt_check(runtime().cbis_cache_seq_pages(self._h, seq_id, None, 0), "pages")
        buf = (ctypes.c_int * max(1, n))()
        runtime().cbis_cache_seq_pages(self._h, seq_id, buf, n)
        return list(buf[:n])

    def num_free_pages(self) -> int:
        return runtime().cbis_cache_num_free_pages(self._h)

    def max_pages(self) -> int:
        return runtime().cbis_cache_max_pages(self._h)

    def page_size(self) -> int:
        return runtime().cbis_cache_page_size(self._h)

    def k_base(self, layer: int) -> int:
        return _rt_check(runtime().cbis_cache_k_base(self._h, layer), "k_base")

    def v_base(self, layer: int) -> int:
        return _rt_check(runtime().cbis_cache_v_base(self._h, layer), "v_base")

    def fill_normal(self, seed: int, std: float = 1.0) -> None:
        _rt_check(runtime().cbis_cache_fill_normal(self._h, seed, std), "fill_normal")


class ModelWeights:
    _h = None

    def __init__(self, handle, cfg: ModelConfig):
        self._h = handle
        self.cfg = cfg

    @classmethod
    def synthetic(cls, cfg: ModelConfig, seed: int = 0, std: float = 0.02):
        return cls(_rt_check(runtime().cbis_weights_synthetic(ctypes.byref(cfg), seed, std), "ModelWeights.synthetic"), cfg)

    @classmethod
    def load(cls, path: str, cfg: ModelConfig):
        return cls(_rt_check(runtime().cbis_weights_load(path.encode(), ctypes.byref(cfg)), "ModelWeights.load"), cfg)

    @classmethod
    def load_packed(cls, path: str):
        """A checkpoint written by save_packed; the config comes from the file."""
        cfg = ModelConfig()
        h = _rt_check(runtime().cbis_weights_load_packed(path.encode(), ctypes.byref(cfg)), "ModelWeights.load_packed")
        return cls(h, cfg)

    def save_packed(self, path: str) -> None:
        _rt_check(runtime().cbis_weights_save_packed(self._h, path.encode()), "ModelWeights.save_packed")

    def tensor(self, name: str) -> int:
        return _rt_check(runtime().cbis_weights_tensor(self._h, name.encode()), f"tensor {name}")

    def device_bytes(self) -> int:
        return runtime().cbis_weights_device_bytes(self._h)

    def close(self):
        if self._h:
            runtime().cbis_weights_destroy(self._h)
            self._h = None

    def __del__(self):
        # At interpreter exit the module globals may already be gone; the
        # process teardown releases the device memory then.
        try:
            self.close()
        except Exception:
            pass


class TransformerRunner:
    _h = None

    def __init__(self, weights: ModelWeights, cache: PagedKVCache, max_total_rows: int):
        self.weights, self.cache = weights, cache  # keep them alive
        self.vocab = weights.cfg.vocab
        self._max_rows = max_total_rows
        self._h = _rt_check(runtime().cbis_runner_create(weights._h, cache._h, max_total_rows), "TransformerRunner")

    def close(self):
        if self._h:
            runtime().cbis_runner_destroy(self._h)
            self._h = None

    def __del__(self):
        # At interpreter exit the module globals may already be gone; the
        # process teardown releases the device memory then.
        try:
            self.close()
        except Exception:
            pass

    def forward_step(self, token_ids, positions, seq_ids):
        """Returns [rows, vocab] fp32 logits as a flat list-backed ctypes array -> numpy via caller."""
        import numpy as np
        n = len(token_ids)
        out = np.empty((n, self.vocab), dtype=np.float32)
        _rt_check(runtime().cbis_runner_forward_step(self._h, n, _iarr(token_ids), _iarr(positions), _iarr(seq_ids),
                                                     out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))),
                  "forward_step")
        return out

    def forward_step_greedy(self, token_ids, positions, seq_ids):
        n = len(token_ids)
        out = (ctypes.c_int * max(1, n))()
        _rt_check(runtime().cbis_runner_forward_step_greedy(self._h, n, _iarr(token_ids), _iarr(positions),
                                                            _iarr(seq_ids), out), "forward_step_greedy")
        return list(out[:n])

    def enqueue_greedy(self, token_ids, positions, seq_ids, token_src=None) -> int:
        """Queues a greedy step without waiting; returns its ticket.  A row
        with token_src[i] >= 0 takes the greedy token of row token_src[i] of
        the greedy step enqueued just before (token_ids[i] is not used)."""
        n = len(token_ids)
        ticket = ctypes.c_int64()
        src = _iarr(token_src) if token_src is not None else None
        _rt_check(runtime().cbis_runner_enqueue_greedy(self._h, n, _iarr(token_ids), _iarr(positions), _iarr(seq_ids),
                                                       src, ctypes.byref(ticket)), "enqueue_greedy")
        return ticket.value

    def wait_greedy(self, ticket: int):
        """Waits for a queued greedy step; returns the next token of every row."""
        out = (ctypes.c_int * max(1, self._max_rows))()
        n = _rt_check(runtime().cbis_runner_wait_greedy(self._h, ticket, out, len(out)), "wait_greedy")
        return list(out[:n])

    def last_margins(self):
        """Top-2 margins of the last forward_step_greedy's rows (numpy fp32)."""
        n = _rt_check(runtime().cbis_runner_last_margins(self._h, None, 0), "last_margins")
        out = np.empty(max(1, n), dtype=np.float32)
        _rt_check(runtime().cbis_runner_last_margins(self._h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n),
                  "last_margins")
        return out[:n]

    def logits_device(self) -> int:
        return runtime().cbis_runner_logits_device(self._h)

    def last_device_ms(self) -> float:
        """Device time of the last step's forward (events on the runner's
        stream around its kernels, which move the step's metadata and
        results to and from pinned host memory themselves)."""
        return float(runtime().cbis_runner_last_device_ms(self._h))

    def last_host_ms(self):
        """Host wall time of the last greedy step's phases: (preparation,
        launch, wait for the results), ms."""
        out = (ctypes.c_double * 3)()
        runtime().cbis_runner_last_host_ms(self._h, out)
        return tuple(out)

    def stream(self) -> int:
        return runtime().cbis_runner_stream(self._h) or 0

    def set_graphs(self, enable: bool) -> None:
        runtime().cbis_runner_set_graphs(self._h, int(enable))

    def set_fused_decode(self, enable: bool) -> None:
        """Small all-decode steps run attention + out-projection as one launch
        per layer (the default) or as two."""
        runtime().cbis_runner_set_fused_decode(self._h, int(enable))

    PLAN_FIELDS = ("rows", "decode_rows", "prefill_tiles", "sequences", "bt_width", "max_kv", "split_tokens",
                   "fused_attention_proj")

    def last_plan(self) -> dict:
        """How the last step ran; split_tokens 1 << 30 = one pass per decode
        row, 0 = the attention library's automatic split."""
        out = (ctypes.c_int * len(self.PLAN_FIELDS))()
        n = _rt_check(runtime().cbis_runner_last_plan(self._h, out, len(out)), "last_plan")
        return dict(zip(self.PLAN_FIELDS, list(out[:n])))


TIERS = {"GPU": 0, "DRAM": 1, "NVME": 2}
TIER_NAMES = {v: k for k, v in TIERS.items()}


class TieredKVBlockManager:
    """include/tiered_kv_manager.hpp:50-151 on the HIP runtime; tiers are
    the strings "GPU", "DRAM", "NVME"."""

    _h = None

    def __init__(self, layer_count, page_size, n_heads, head_dim, nvme_scratch_path, gpu_capacity_blocks,
                 dram_capacity_blocks, params: "EvictionParams" = None, kv_dtype="f32"):
        self._h = _rt_check(runtime().cbis_tiered_create(layer_count, page_size, n_heads, head_dim, DTYPES[kv_dtype],
                                                         str(nvme_scratch_path).encode(), gpu_capacity_blocks,
                                                         dram_capacity_blocks,
                                                         ctypes.byref(params) if params is not None else None),
                            "TieredKVBlockManager")

    @staticmethod
    def default_params() -> "EvictionParams":
        p = EvictionParams()
        runtime().cbis_eviction_params_default(ctypes.byref(p))
        return p

    def close(self):
        if self._h:
            runtime().cbis_tiered_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def raw_block_bytes(self) -> int:
        return runtime().cbis_tiered_raw_block_bytes(self._h)

    def calibrate(self) -> None:
        _rt_check(runtime().cbis_tiered_calibrate(self._h), "calibrate")

    def params(self) -> "EvictionParams":
        p = EvictionParams()
        _rt_check(runtime().cbis_tiered_params(self._h, ctypes.byref(p)), "params")
        return p

    def admit_gpu_resident(self, block_id, cache: "PagedKVCache", physical_page, now_step):
        _rt_check(runtime().cbis_tiered_admit_gpu_resident(self._h, block_id, cache._h, physical_page, now_step),
                  "admit_gpu_resident")

    def evict_one(self, now_step):
        out = ctypes.c_uint64()
        _rt_check(runtime().cbis_tiered_evict_one(self._h, now_step, ctypes.byref(out)), "evict_one")
        return None if out.value == (1 << 64) - 1 else out.value

    def spill(self, block_id, dest, now_step):
        _rt_check(runtime().cbis_tiered_spill(self._h, block_id, TIERS[dest], now_step), "spill")

    def restore(self, block_id, cache: "PagedKVCache", physical_page, now_step):
        _rt_check(runtime().cbis_tiered_restore(self._h, block_id, cache._h, physical_page, now_step), "restore")

    def spill_batch(self, block_ids, dest, now_step):
        ids = (ctypes.c_uint64 * max(1, len(block_ids)))(*block_ids)
        _rt_check(runtime().cbis_tiered_spill_batch(self._h, ids, len(block_ids), TIERS[dest], now_step),
                  "spill_batch")

    def restore_batch(self, block_ids, cache: "PagedKVCache", physical_pages, now_step):
        ids = (ctypes.c_uint64 * max(1, len(block_ids)))(*block_ids)
        _rt_check(runtime().cbis_tiered_restore_batch(self._h, ids, len(block_ids), cache._h, _iarr(physical_pages),
                                                      now_step), "restore_batch")

    def tier_of(self, block_id) -> str:
        return TIER_NAMES[_rt_check(runtime().cbis_tiered_tier_of(self._h, block_id), "tier_of")]

    def known(self, block_id) -> bool:
        return bool(runtime().cbis_tiered_known(self._h, block_id))

    def touch(self, block_id, now_step):
        _rt_check(runtime().cbis_tiered_touch(self._h, block_id, now_step), "touch")

    def stats(self) -> dict:
        out = (_SZ * 5)()
        _rt_check(runtime().cbis_tiered_stats(self._h, out), "stats")
        return dict(zip(("gpu_count", "dram_count", "nvme_count", "raw_bytes_total", "compressed_bytes_total"),
                        list(out)))


def block_deflate(data: bytes) -> bytes:
    cap = len(data) + len(data) // 1000 + 64
    buf = ctypes.create_string_buffer(cap)
    n = runtime().cbis_block_deflate(data, len(data), buf, cap)
    if n < 0:
        _rt_check(-1, "block_deflate")
    return buf.raw[:n]


def block_inflate(comp: bytes, out_len: int) -> bytes:
    buf = ctypes.create_string_buffer(max(1, out_len))
    _rt_check(runtime().cbis_block_inflate(comp, len(comp), buf, out_len), "block_inflate")
    return buf.raw[:out_len]


def _darr(values):
    return (ctypes.c_double * max(1, len(values)))(*values)


def run_continuous(runner: TransformerRunner, cache: PagedKVCache, prompts, decode_lens, max_slots=16,
                   max_steps=4096, prefill_chunk=0, step_token_budget=0, arrival_ms=None, pipeline=False):
    """Continuous batching (src/bench_batching.cpp:98-179); prefill_chunk /
    step_token_budget > 0 feed prompts in chunks; arrival_ms (nondecreasing)
    admits request i only once that many ms of the run have passed.
    pipeline=True queues each step before the previous one's tokens come
    back (decode rows read their input token on the device): the same steps
    and tokens, with the host's work hidden behind the device's.  Returns
    (tokens per request, per-step wall ms), plus the per-request finish
    times (ms since the run began) when arrival_ms is given."""
    lens = [len(p) for p in prompts]
    flat = [t for p in prompts for t in p]
    out = (ctypes.c_int * max(1, sum(decode_lens)))()
    ms = (ctypes.c_double * max_steps)()
    fin = (ctypes.c_double * max(1, len(prompts)))()
    arr = _darr(arrival_ms) if arrival_ms is not None else None
    fn = runtime().cbis_run_continuous_pipelined if pipeline else runtime().cbis_run_continuous_timed
    n = _rt_check(fn(runner._h, cache._h, len(prompts), _iarr(lens), _iarr(flat), _iarr(decode_lens), arr, max_slots,
                     prefill_chunk, step_token_budget, out, ms, max_steps, fin), "run_continuous")
    toks, o = [], 0
    for d in decode_lens:
        toks.append(list(out[o: o + d]))
        o += d
    if arrival_ms is None:
        return toks, list(ms[: min(n, max_steps)])
    return toks, list(ms[: min(n, max_steps)]), list(fin[: len(prompts)])


def schedule_dry_run(cache: PagedKVCache, prompts, decode_lens, vocab, max_slots=16, prefill_chunk=0,
                     step_token_budget=0, max_steps=4096, max_rows=1 << 16, arrival_ms=None, step_time_ms=1.0,
                     pipeline=False):
    """The scheduler alone, on the host, with the stand-in step of
    cbis_schedule_dry_run (pipeline=True: the pipelined scheduler, whose
    rows report the tokens the stand-in device resolved).  Returns (tokens
    per request, [(tok, pos, sid) rows of each step]); with arrival_ms, on a
    virtual clock where a step takes step_time_ms, and the per-request
    finish times as a third value."""
    lens = [len(p) for p in prompts]
    flat = [t for p in prompts for t in p]
    out = (ctypes.c_int * max(1, sum(decode_lens)))()
    rows = (ctypes.c_int * max_steps)()
    rt, rp, rs = (ctypes.c_int * max_rows)(), (ctypes.c_int * max_rows)(), (ctypes.c_int * max_rows)()
    fin = (ctypes.c_double * max(1, len(prompts)))()
    arr = _darr(arrival_ms) if arrival_ms is not None else None
    fn = runtime().cbis_schedule_dry_run_pipelined if pipeline else runtime().cbis_schedule_dry_run_timed
    n = _rt_check(fn(cache._h, len(prompts), _iarr(lens), _iarr(flat), _iarr(decode_lens), arr, step_time_ms,
                     max_slots, prefill_chunk, step_token_budget, vocab, out, rows, max_steps, rt, rp, rs, max_rows,
                     fin), "schedule_dry_run")
    if n > max_steps or sum(rows[:n]) > max_rows:
        raise RuntimeError("schedule_dry_run: trace larger than the buffers")
    toks, o = [], 0
    for d in decode_lens:
        toks.append(list(out[o: o + d]))
        o += d
    steps, r = [], 0
    for k in range(n):
        steps.append([(rt[r + i], rp[r + i], rs[r + i]) for i in range(rows[k])])
        r += rows[k]
    if arrival_ms is None:
        return toks, steps
    return toks, steps, list(fin[: len(prompts)])
