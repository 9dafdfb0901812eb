"""CPU-only checks of the product's host code: PagedKVCache bookkeeping
(libcbis.so with alloc_device = 0, no HIP call) against the reference's KATs
and the oracle restatement, the C-ABI exports, and argument validation that
happens before any launch."""
import ctypes
import os
import re

import pytest
from hypothesis import given, settings, strategies as st

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _cache(cbis, max_pages, pages_per_seq=2048):
    return cbis.PagedKVCache(4, max_pages, 16, 8, 32, "f32", pages_per_seq=pages_per_seq, alloc_device=False)


# tests/correctness_test.cpp:28-90, the reference's four KATs ---------------

def test_kat_allocate_and_grow(cbis):
    c = _cache(cbis, 8)
    seq = c.allocate_sequence()
    assert c.num_free_pages() == 8
    for p in range(16):
        assert c.ensure_capacity(seq, p)
    assert c.num_free_pages() == 7
    assert c.ensure_capacity(seq, 16)
    assert c.num_free_pages() == 6
    assert c.ensure_capacity(seq, 17)
    assert c.num_free_pages() == 6
    assert c.resolve_slot(seq, 0)[1] == 0
    assert c.resolve_slot(seq, 16)[1] == 0
    assert c.resolve_slot(seq, 19)[1] == 3
    c.free_sequence(seq)
    assert c.num_free_pages() == 8


def test_kat_page_reuse_across_sequences(cbis):
    c = _cache(cbis, 2)
    a = c.allocate_sequence()
    assert c.ensure_capacity(a, 0) and c.ensure_capacity(a, 16)
    assert c.num_free_pages() == 0
    b = c.allocate_sequence()
    assert not c.ensure_capacity(b, 0)  # exhausted: false, not a crash
    c.free_sequence(a)
    assert c.num_free_pages() == 2
    assert c.ensure_capacity(b, 0)


def test_kat_page_table_padding(cbis):
    c = _cache(cbis, 4)
    s = c.allocate_sequence()
    c.ensure_capacity(s, 0)
    t = c.page_table(s)
    assert len(t) == 2048 and all(x == 0 for x in t[1:])


def test_kat_disjoint_sequences(cbis):
    c = _cache(cbis, 4)
    a, b = c.allocate_sequence(), c.allocate_sequence()
    c.ensure_capacity(a, 0)
    c.ensure_capacity(b, 0)
    assert c.page_table(a)[0] != c.page_table(b)[0]


def test_exact_allocation_order(cbis):
    """Free list [P-1..0]: pages come out 0,1,2,...; a freed sequence's pages
    return in logical order so the next ones come back LIFO-reversed."""
    c = _cache(cbis, 8)
    a = c.allocate_sequence()
    c.ensure_capacity(a, 47)
    assert c.pages(a) == [0, 1, 2]
    b = c.allocate_sequence()
    c.ensure_capacity(b, 16)
    assert c.pages(b) == [3, 4]
    c.free_sequence(a)
    d = c.allocate_sequence()
    c.ensure_capacity(d, 40)
    assert c.pages(d) == [2, 1, 0]
    assert d == 2  # monotonic ids, never reused


def test_error_paths(cbis):
    c = _cache(cbis, 4)
    s = c.allocate_sequence()
    with pytest.raises(IndexError):
        c.resolve_slot(s, 0)          # no capacity yet (reference: std::out_of_range)
    with pytest.raises(IndexError):
        c.ensure_capacity(99, 0)      # unknown sequence
    c.free_sequence(12345)            # unknown: no-op like the reference
    with pytest.raises(cbis.CbisError):
        cbis.PagedKVCache(0, 4, alloc_device=False)


@settings(max_examples=60, deadline=None)
@given(st.lists(st.tuples(st.sampled_from(["alloc", "grow", "free"]), st.integers(0, 7), st.integers(0, 200)),
                max_size=80))
def test_allocation_bit_exact_vs_oracle(cbis, oracle, ops):
    """Random operation traces: every page table and free count identical to
    the oracle's restatement of src/paged_kv_cache.cpp."""
    c = _cache(cbis, 24, pages_per_seq=16)
    o = oracle.PagedKVCacheOracle(24, pages_per_seq=16)
    live = []
    for op, k, pos in ops:
        if op == "alloc" or not live:
            a, b = c.allocate_sequence(), o.allocate_sequence()
            assert a == b
            live.append(a)
        elif op == "grow":
            s = live[k % len(live)]
            assert c.ensure_capacity(s, pos) == o.ensure_capacity(s, pos)
        else:
            s = live.pop(k % len(live))
            c.free_sequence(s)
            o.free_sequence(s)
        assert c.num_free_pages() == o.num_free_pages()
        for s in live:
            assert c.pages(s) == o.seq_pages[s]
            assert c.page_table(s) == o.page_table(s)
    owned = [p for s in live for p in c.pages(s)]
    assert len(owned) == len(set(owned))  # no page owned twice


# C-ABI ----------------------------------------------------------------------

def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cbis_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header,which", [("cbis_kernels.h", "kernels"), ("cbis_runtime.h", "runtime")])
def test_every_declared_symbol_is_exported(cbis, header, which):
    lib = getattr(cbis, which)()
    names = _declared(header)
    assert len(names) > 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    table = cbis.KERNEL_SYMBOLS if which == "kernels" else cbis.RUNTIME_SYMBOLS
    assert set(names) == set(table)  # the binding covers the whole header


def test_abi_validation_without_gpu(cbis):
    K = cbis.kernels()
    d = cbis.GemmDesc()
    d.M, d.N, d.K = 4, 8, 100
    d.x_dtype = d.w_dtype = d.y_dtype = cbis.BF16
    d.X = d.W = d.Y = 4096
    d.ldx = d.ldw = 100
    d.ldy = 8
    assert K.cbis_gemm(ctypes.byref(d), None) == 2  # K % 64
    assert b"multiple of 64" in K.cbis_last_error()
    d.K, d.ldx, d.ldw = 128, 128, 128
    d.x_dtype = cbis.F32  # fp32 activations with bf16 weights
    assert K.cbis_gemm(ctypes.byref(d), None) == 2
    assert K.cbis_gemm(None, None) == 1
    a = cbis.AttnDesc()
    a.n_rows, a.n_heads, a.head_dim, a.page_size = 4, 8, 32, 16
    a.q = a.k_pool = a.v_pool = a.block_table = a.out = a.row_pos = 4096
    a.num_pages, a.bt_stride = 10, 4
    a.max_kv_len, a.split_tokens = 4096, 64
    assert K.cbis_paged_attention(ctypes.byref(a), None) == 3  # needs a workspace
    need = K.cbis_paged_attention_workspace_size(ctypes.byref(a))
    assert need == 4 * 64 * 8 * 36 * 4
    a.n_heads = 12  # a partial last head block (8 fp32 heads per block) is fine
    assert K.cbis_paged_attention_workspace_size(ctypes.byref(a)) == 4 * 64 * 12 * 36 * 4
    assert K.cbis_paged_attention(ctypes.byref(a), None) == 3  # still only the workspace is missing
    # A split that is not a whole number of pages would count the keys of its
    # first page twice: refused.
    a.split_tokens = 100
    assert K.cbis_paged_attention_workspace_size(ctypes.byref(a)) == 0
    assert K.cbis_paged_attention(ctypes.byref(a), None) == 1
    assert b"multiple of page_size" in K.cbis_last_error()
    a.n_heads = 0
    a.split_tokens = 64
    assert K.cbis_paged_attention(ctypes.byref(a), None) == 1
    assert K.cbis_layernorm(4, 10000, 4096, 10000, 4096, 4096, 1e-5, 0, 4096, 10000, None) == 2
    # embedding tables: 16-byte fp32 / 8-byte bf16 lane loads, 16-byte stores
    assert K.cbis_embed(4, 256, 4096, 4096, cbis.F32, 4104, 4096, 10, 10, 4096, None) == 1
    assert b"aligned" in K.cbis_last_error()
    assert K.cbis_embed(4, 256, 4096, 4096, cbis.BF16, 4096, 4100, 10, 10, 4096, None) == 1
    assert K.cbis_embed(4, 256, 4096, 4096, cbis.BF16, 4096, 4096, 10, 10, 4104, None) == 1
