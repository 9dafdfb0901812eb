"""Three-tier KV block manager on the GPU: the reference's functional tests
(tests/tiered_kv_test.cpp:83-155 -- bit-identical DRAM and NVMe round
trips, cost-aware eviction, DRAM-full spill to NVMe, stats), the batched
spill / restore against one-block-at-a-time calls, and the page gather /
scatter kernels against numpy."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

_HIP = None


def _hip():
    global _HIP
    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so")
        _HIP.hipMemcpy.restype = ctypes.c_int
        _HIP.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return _HIP


def _h2d(dst, a):
    assert _hip().hipMemcpy(dst, a.ctypes.data, a.nbytes, 1) == 0


def _d2h(a, src):
    assert _hip().hipMemcpy(a.ctypes.data, src, a.nbytes, 2) == 0


L, PS, H, HD = 4, 16, 8, 32   # the reference model's cache geometry (include/config.hpp)


def _cache(cbis, max_pages, kv="f32", heads=H, layers=L):
    return cbis.PagedKVCache(layers, max_pages, PS, heads, HD, kv, pages_per_seq=64)


def _page_bytes(cache):
    return PS * cache.n_heads * HD * (4 if cache.kv_dtype == "f32" else 2)


def fill_page(cache, page, seed):
    """Writes random bytes into every layer's K and V page; returns the
    block's raw bytes in the reference's order (l0 K, l0 V, l1 K, ...)."""
    pb = _page_bytes(cache)
    rng = np.random.default_rng(seed)
    parts = []
    for l in range(cache.num_layers):
        for base in (cache.k_base(l), cache.v_base(l)):
            a = rng.uniform(-10, 10, pb // 4).astype(np.float32).view(np.uint8)
            _h2d(base + page * pb, a)
            parts.append(a)
    return np.concatenate(parts)


def read_page(cache, page):
    pb = _page_bytes(cache)
    parts = []
    for l in range(cache.num_layers):
        for base in (cache.k_base(l), cache.v_base(l)):
            a = np.empty(pb, np.uint8)
            _d2h(a, base + page * pb)
            parts.append(a)
    return np.concatenate(parts)


@pytest.fixture
def mgr_factory(cbis, tmp_path):
    made = []

    def make(gpu_cap, dram_cap, kv="f32", heads=H, params=None):
        m = cbis.TieredKVBlockManager(L, PS, heads, HD, tmp_path / f"t{len(made)}.nvme", gpu_cap, dram_cap,
                                      params=params, kv_dtype=kv)
        made.append(m)
        return m
    yield make
    for m in made:
        m.close()


# tests/tiered_kv_test.cpp:83-155 ------------------------------------------

def test_dram_roundtrip(cbis, mgr_factory):
    cache = _cache(cbis, 4)
    mgr = mgr_factory(4, 4)
    original = fill_page(cache, 0, 1)
    mgr.admit_gpu_resident(100, cache, 0, 0)
    assert mgr.tier_of(100) == "GPU"
    mgr.spill(100, "DRAM", 1)
    assert mgr.tier_of(100) == "DRAM"
    mgr.restore(100, cache, 2, 2)
    assert mgr.tier_of(100) == "GPU"
    assert np.array_equal(read_page(cache, 2), original)


def test_nvme_roundtrip(cbis, mgr_factory):
    cache = _cache(cbis, 4)
    mgr = mgr_factory(4, 4)
    original = fill_page(cache, 1, 2)
    mgr.admit_gpu_resident(200, cache, 1, 0)
    mgr.spill(200, "NVME", 1)
    assert mgr.tier_of(200) == "NVME"
    mgr.restore(200, cache, 3, 2)
    assert np.array_equal(read_page(cache, 3), original)


def test_eviction_picks_most_stale(cbis, mgr_factory):
    cache = _cache(cbis, 4)
    mgr = mgr_factory(2, 4)
    fill_page(cache, 0, 10)
    fill_page(cache, 1, 11)
    mgr.admit_gpu_resident(1, cache, 0, 0)
    mgr.admit_gpu_resident(2, cache, 1, 5)
    fill_page(cache, 2, 12)
    mgr.admit_gpu_resident(3, cache, 2, 10)
    assert (mgr.tier_of(1), mgr.tier_of(2), mgr.tier_of(3)) == ("DRAM", "GPU", "GPU")


def test_eviction_spills_to_nvme_once_dram_full(cbis, mgr_factory):
    cache = _cache(cbis, 8)
    mgr = mgr_factory(1, 1)
    fill_page(cache, 0, 20)
    mgr.admit_gpu_resident(1, cache, 0, 0)
    fill_page(cache, 1, 21)
    mgr.admit_gpu_resident(2, cache, 1, 1)
    assert mgr.tier_of(1) == "DRAM"
    fill_page(cache, 2, 22)
    mgr.admit_gpu_resident(3, cache, 2, 2)
    assert mgr.tier_of(2) == "NVME"


def test_stats(cbis, mgr_factory):
    cache = _cache(cbis, 4)
    mgr = mgr_factory(4, 4)
    fill_page(cache, 0, 30)
    mgr.admit_gpu_resident(1, cache, 0, 0)
    s = mgr.stats()
    assert s["gpu_count"] == 1 and s["raw_bytes_total"] == L * 2 * PS * H * HD * 4 == mgr.raw_block_bytes()


# beyond the reference's tests ----------------------------------------------

def test_restore_into_full_gpu_tier_evicts_stalest(cbis, mgr_factory):
    """A restore into a full GPU tier evicts the stalest resident block
    before the restored block counts as resident
    (src/tiered_kv_manager.cpp:196-198), and the evicted block's bytes come
    back intact."""
    cache = _cache(cbis, 8)
    mgr = mgr_factory(2, 8)
    orig = {}
    for b, (page, step) in {7: (0, 1), 8: (1, 3)}.items():
        orig[b] = fill_page(cache, page, b)
        mgr.admit_gpu_resident(b, cache, page, step)
    orig[9] = fill_page(cache, 2, 9)
    mgr.admit_gpu_resident(9, cache, 2, 4)             # evicts 7 (stalest)
    assert mgr.tier_of(7) == "DRAM"
    mgr.spill(9, "NVME", 5)
    orig[10] = fill_page(cache, 3, 10)
    mgr.admit_gpu_resident(10, cache, 3, 5)            # GPU tier full again
    mgr.restore(9, cache, 5, 6)                         # evicts 8 (step 3) rather than 10 (step 5)
    assert [mgr.tier_of(b) for b in (7, 8, 9, 10)] == ["DRAM", "DRAM", "GPU", "GPU"]
    assert np.array_equal(read_page(cache, 5), orig[9])
    s = mgr.stats()
    assert (s["gpu_count"], s["dram_count"], s["nvme_count"]) == (2, 2, 0)
    assert 0 < s["compressed_bytes_total"] <= 2 * mgr.raw_block_bytes() * 1.01
    mgr.restore_batch([7, 8], cache, [6, 7], 7)        # each restore evicts again
    assert np.array_equal(read_page(cache, 6), orig[7]) and np.array_equal(read_page(cache, 7), orig[8])
    assert mgr.stats()["gpu_count"] == 2


@pytest.mark.parametrize("kv,heads", [("f32", 8), ("bf16", 64)])
def test_batch_matches_single_calls(cbis, mgr_factory, kv, heads):
    """spill_batch / restore_batch leave the same tiers, stats and page
    bytes as the same calls made one block at a time, including the
    evictions that restores into a full GPU tier trigger midway."""
    caches = [_cache(cbis, 32, kv, heads), _cache(cbis, 32, kv, heads)]
    mgrs = [mgr_factory(6, 5, kv, heads), mgr_factory(6, 5, kv, heads)]
    originals = {}
    for cache, mgr in zip(caches, mgrs):
        for b in range(12):   # admissions 6..11 evict 0..4 to DRAM, 5 to NVMe
            originals[b] = fill_page(cache, b, 1000 + b)
            mgr.admit_gpu_resident(b, cache, b, b)
    assert [mgrs[0].tier_of(b) for b in range(12)] == ["DRAM"] * 5 + ["NVME"] + ["GPU"] * 6
    mgrs[0].spill_batch([6, 7, 8], "NVME", 20)
    for b in (6, 7, 8):
        mgrs[1].spill(b, "NVME", 20)
    ids = [0, 6, 3, 5, 8, 1]
    pages = [20 + i for i in range(len(ids))]
    mgrs[0].restore_batch(ids, caches[0], pages, 30)
    for b, p in zip(ids, pages):
        mgrs[1].restore(b, caches[1], p, 30)
    assert mgrs[0].stats() == mgrs[1].stats()
    assert [mgrs[0].tier_of(b) for b in range(12)] == [mgrs[1].tier_of(b) for b in range(12)]
    assert mgrs[0].tier_of(9) == "DRAM"   # evicted by the restore of block 5
    for b, p in zip(ids, pages):
        got = read_page(caches[0], p)
        assert np.array_equal(got, originals[b])
        assert np.array_equal(got, read_page(caches[1], p))
    # evicted blocks come back intact too
    mgrs[0].restore_batch([9], caches[0], [30], 40)
    assert np.array_equal(read_page(caches[0], 30), originals[9])


def test_batch_destination_aliases_evicted_victim(cbis, mgr_factory):
    """A restore batch whose later destination page is the current page of a
    block the batch's own earlier restore evicts: as with one restore() after
    another, the victim spills its own bytes before that page is written."""
    caches = [_cache(cbis, 16), _cache(cbis, 16)]
    mgrs = [mgr_factory(2, 8), mgr_factory(2, 8)]
    orig = {}
    for cache, mgr in zip(caches, mgrs):
        for b, page in ((1, 0), (2, 1), (3, 2), (4, 3)):
            orig[b] = fill_page(cache, page, 50 + b)
            mgr.admit_gpu_resident(b, cache, page, b)
        for b in (3, 4):   # blocks 1, 2 went to DRAM when 3, 4 arrived; now 3, 4 follow
            mgr.spill(b, "DRAM", 10)
        mgr.restore(2, cache, 1, 11)                   # GPU: 2 (page 1)
        fill_page(cache, 7, 99)
        mgr.admit_gpu_resident(5, cache, 7, 12)         # GPU: 2, 5 -- tier full
        orig[5] = read_page(cache, 7)
    # Restoring 3 evicts 2 (stalest, page 1); 4 is then written into page 1.
    mgrs[0].restore_batch([3, 4], caches[0], [9, 1], 20)
    mgrs[1].restore(3, caches[1], 9, 20)
    mgrs[1].restore(4, caches[1], 1, 20)
    assert mgrs[0].tier_of(2) == "DRAM" and mgrs[0].stats() == mgrs[1].stats()
    for cache, mgr in zip(caches, mgrs):
        assert np.array_equal(read_page(cache, 9), orig[3]) and np.array_equal(read_page(cache, 1), orig[4])
        mgr.restore(2, cache, 12, 30)                   # the victim's spilled bytes are its own
        assert np.array_equal(read_page(cache, 12), orig[2])


def test_batch_refuses_overwriting_a_later_moved_block(cbis, mgr_factory):
    """One restore() after another would overwrite a GPU-resident block's
    page before moving it; the batch refuses that order instead."""
    cache = _cache(cbis, 8)
    mgr = mgr_factory(4, 4)
    for b, page in ((1, 0), (2, 1)):
        fill_page(cache, page, b)
        mgr.admit_gpu_resident(b, cache, page, 0)
    with pytest.raises(cbis.CbisError, match="earlier block's destination"):
        mgr.restore_batch([1, 2], cache, [1, 5], 1)
    assert mgr.tier_of(1) == "GPU" and mgr.tier_of(2) == "GPU"
    mgr.restore_batch([2, 1], cache, [5, 1], 1)         # the order that moves 2 first is fine


def test_restore_moves_gpu_resident_block(cbis, mgr_factory):
    cache = _cache(cbis, 8)
    mgr = mgr_factory(4, 4)
    orig = fill_page(cache, 1, 5)
    mgr.admit_gpu_resident(42, cache, 1, 0)
    mgr.restore_batch([42], cache, [6], 1)
    assert mgr.tier_of(42) == "GPU" and mgr.stats()["gpu_count"] == 1
    assert np.array_equal(read_page(cache, 6), orig)


def test_manager_errors(cbis, mgr_factory):
    cache = _cache(cbis, 4)
    mgr = mgr_factory(4, 4)
    fill_page(cache, 0, 1)
    mgr.admit_gpu_resident(1, cache, 0, 0)
    with pytest.raises(cbis.CbisError, match="already managed"):
        mgr.admit_gpu_resident(1, cache, 1, 0)
    with pytest.raises(cbis.CbisError, match="unknown block_id"):
        mgr.restore(99, cache, 1, 0)
    with pytest.raises(cbis.CbisError, match="not GPU-resident"):
        mgr.spill(1, "DRAM", 1)
        mgr.spill(1, "DRAM", 1)
    with pytest.raises(IndexError):
        mgr.restore(1, cache, 4, 2)          # page out of range
    with pytest.raises(cbis.CbisError, match="listed twice"):
        mgr.restore_batch([1, 1], cache, [1, 2], 2)
    with pytest.raises(cbis.CbisError, match="geometry"):
        mgr.admit_gpu_resident(5, _cache(cbis, 4, "bf16", 16), 0, 0)
    assert mgr.stats()["gpu_count"] == 0 and mgr.evict_one(3) is None


def test_page_gather_scatter_kernels(cbis, dev):
    """cbis_kv_pages_gather / _scatter against numpy on a [L][2][P][page]
    pool; out-of-range page ids are skipped."""
    import torch
    from helpers import stream, sync
    Lx, P, pb = 3, 11, 4096
    rng = np.random.default_rng(3)
    pool_np = rng.integers(0, 256, (Lx, 2, P, pb), dtype=np.uint8)
    pool = torch.from_numpy(pool_np).to(dev)
    pages = np.array([7, 0, 10, 3], np.int32)
    pg = torch.from_numpy(pages).to(dev)
    stage = torch.zeros((len(pages), Lx, 2, pb), dtype=torch.uint8, device=dev)
    k = cbis.kernels()
    assert k.cbis_kv_pages_gather(stage.data_ptr(), pool.data_ptr(), Lx, P, pb, pg.data_ptr(), len(pages),
                                  stream()) == 0
    sync()
    want = np.stack([pool_np[:, :, p, :] for p in pages])
    assert np.array_equal(stage.cpu().numpy(), want)
    # scatter a modified staging into other pages (one id out of range)
    new = rng.integers(0, 256, stage.shape, dtype=np.uint8)
    dst_pages = np.array([1, 2, 99, 9], np.int32)
    st2 = torch.from_numpy(new).to(dev)
    dp = torch.from_numpy(dst_pages).to(dev)
    assert k.cbis_kv_pages_scatter(pool.data_ptr(), st2.data_ptr(), Lx, P, pb, dp.data_ptr(), len(dst_pages),
                                   stream()) == 0
    sync()
    expect = pool_np.copy()
    for i, p in enumerate(dst_pages):
        if 0 <= p < P:
            expect[:, :, p, :] = new[i]
    assert np.array_equal(pool.cpu().numpy(), expect)
    assert k.cbis_kv_pages_gather(stage.data_ptr(), pool.data_ptr(), Lx, P, 4095, pg.data_ptr(), 4, stream()) != 0
