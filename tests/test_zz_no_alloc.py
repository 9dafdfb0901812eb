"""cbis_paged_attention_static, the entry point that allocates nothing (its
split-KV partials live in a static device buffer): same results as
cbis_paged_attention with a caller workspace, on two calls in a row (the
second smaller, so it runs over what the first left in the buffer), and a
clear error for a call whose partials do not fit the buffer."""
import ctypes

import numpy as np
import pytest

from helpers import ptr, rng, stream, sync, to_dev

pytestmark = pytest.mark.gpu

STATIC_BYTES = 32 << 20   # CBIS_ATTN_STATIC_SCRATCH_BYTES


def _case(cbis, dev, kv, H, kv_dtype, split, seed):
    """Inputs of one decode-attention call: rows at kv_len kv over a
    permuted page table."""
    import torch
    n = len(kv)
    npages = (kv + 15) // 16
    P = int(npages.sum()) + 4
    perm = rng(seed).permutation(P).astype(np.int32)
    bt = np.zeros((n, int(npages.max())), np.int32)
    off = 0
    for i in range(n):
        bt[i, : npages[i]] = perm[off: off + npages[i]]
        off += npages[i]
    tdt = torch.float32 if kv_dtype == cbis.F32 else torch.bfloat16
    kp = torch.empty((P, 16, H, 32), dtype=tdt, device=dev)
    vp = torch.empty_like(kp)
    q = torch.empty((n, H * 32), dtype=torch.float32, device=dev)
    K = cbis.kernels()
    for t, sd, dt in ((kp, seed + 1, kv_dtype), (vp, seed + 2, kv_dtype), (q, seed + 3, cbis.F32)):
        cbis.check(K.cbis_fill_normal_fast(ptr(t), dt, t.numel(), sd, 1.0, stream()))
    d = cbis.AttnDesc()
    d.n_rows, d.n_heads, d.head_dim, d.page_size = n, H, 32, 16
    d.q_dtype, d.q, d.ldq = cbis.F32, ptr(q), H * 32
    d.kv_dtype, d.k_pool, d.v_pool, d.num_pages = kv_dtype, ptr(kp), ptr(vp), P
    BT, POS = to_dev(bt, dev), to_dev((kv - 1).astype(np.int32), dev)
    d.block_table, d.bt_stride, d.row_pos = ptr(BT), bt.shape[1], ptr(POS)
    d.out_dtype, d.ldo = cbis.F32, H * 32
    d.max_kv_len, d.split_tokens = int(kv.max()), split
    d.keep_alive = (q, kp, vp, BT, POS)
    return d


def _run_both(cbis, dev, d):
    import torch
    K = cbis.kernels()
    n, width = d.n_rows, d.n_heads * 32
    need = K.cbis_paged_attention_workspace_size(ctypes.byref(d))
    assert 0 < need <= STATIC_BYTES   # the call splits: the partials path runs
    ws = torch.empty(need // 4, dtype=torch.float32, device=dev)
    ref = torch.full((n, width), 7.0, dtype=torch.float32, device=dev)
    d.out, d.workspace, d.workspace_bytes = ptr(ref), ptr(ws), need
    cbis.check(K.cbis_paged_attention(ctypes.byref(d), stream()))
    got = torch.full((n, width), 7.0, dtype=torch.float32, device=dev)
    d.out, d.workspace, d.workspace_bytes = ptr(got), None, 0   # ignored by the static entry point
    cbis.check(K.cbis_paged_attention_static(ctypes.byref(d), stream()), "static")
    sync()
    g, r = got.cpu().numpy(), ref.cpu().numpy()
    assert (r != 7.0).all()
    assert np.array_equal(g.view(np.uint32), r.view(np.uint32))
    del ws


def test_static_scratch_matches_workspace_entry_point(cbis, dev):
    """A large bf16 call (64 heads, automatic split), then a smaller fp32 one
    (8 heads, 64-token splits) over the partials the first left behind:
    bit-identical to cbis_paged_attention both times."""
    kv1 = rng(61).integers(100, 5000, 96).astype(np.int32)
    print(f"no-alloc call 1: 96 rows, bf16 K/V, 64 heads, kv {kv1.min()}..{kv1.max()}", flush=True)
    _run_both(cbis, dev, _case(cbis, dev, kv1, 64, cbis.BF16, 0, 61))
    kv2 = np.array([1, 17, 64, 65, 300, 129, 999], np.int32)
    print("no-alloc call 2: 7 rows, fp32 K/V, 8 heads, 64-token splits", flush=True)
    _run_both(cbis, dev, _case(cbis, dev, kv2, 8, cbis.F32, 64, 62))


def test_static_scratch_too_small_is_refused(cbis, dev):
    """Partials beyond the static buffer: CBIS_ERR_WORKSPACE before any
    launch, with the sizes in the message."""
    kv = np.full(64, 4096, np.int32)
    d = _case(cbis, dev, kv, 64, cbis.BF16, 16, 63)
    K = cbis.kernels()
    need = K.cbis_paged_attention_workspace_size(ctypes.byref(d))
    assert need > STATIC_BYTES
    import torch
    out = torch.empty((64, 64 * 32), dtype=torch.float32, device=dev)
    d.out = ptr(out)
    assert K.cbis_paged_attention_static(ctypes.byref(d), stream()) == 3
    assert b"static scratch" in K.cbis_last_error()
    sync()
