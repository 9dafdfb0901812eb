"""Shared helpers for the GPU parity tests (torch is used only for device
memory and the stream handle)."""
import numpy as np


def ptr(t):
    return None if t is None else t.data_ptr()


def stream():
    import torch
    return torch.cuda.current_stream().cuda_stream


def sync():
    import torch
    torch.cuda.synchronize()


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def bf16_dev(a_f32, dev):
    """fp32 numpy -> device bf16 tensor (round to nearest even), plus the
    exact fp32 values it holds."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a_f32, dtype=np.float32)).to(dev).to(torch.bfloat16)
    return t, t.float().cpu().numpy()


def bits_u16(t):
    import torch
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def row_rel_err(got, ref):
    """max over rows of ||got - ref||_inf / ||ref||_inf (the bf16/fp8 metric)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    num = np.abs(got - ref).max(axis=-1)
    den = np.maximum(np.abs(ref).max(axis=-1), 1e-30)
    return float((num / den).max())


def check_logits(got, ref, what):
    """The bf16/fp8 parity bar: per row ||d||_inf / ||ref||_inf <= 2e-2,
    and the greedy token equal wherever the oracle's top-2 margin exceeds
    twice the row's measured error.  Returns the oracle's argmax per row."""
    err = row_rel_err(got, ref)
    abs_err = np.abs(got - ref).max(axis=1)
    srt = np.sort(ref, axis=1)
    margin = srt[:, -1] - srt[:, -2]
    sure = margin > 2 * abs_err
    agree = got.argmax(axis=1) == ref.argmax(axis=1)
    print(f"{what}: rows={len(got)} per-row rel err {err:.3e}, max abs {abs_err.max():.3e}, "
          f"argmax agrees on {int(agree.sum())}/{len(got)} ({int(sure.sum())} with margin > 2 err)", flush=True)
    assert err < 2e-2, err
    assert agree[sure].all()
    return ref.argmax(axis=1)


def rng(seed):
    return np.random.default_rng(seed)


def write_weights_bin(path, weights):
    """Writes oracle Weights' fp32 master tensors as the reference's
    weights.bin: python/export_weights.py:42-66 order, raw little-endian fp32,
    nothing else."""
    spec, m = weights.spec, weights.master
    names = ["tok_emb", "pos_emb"]
    for l in range(spec.n_layers):
        names += [f"l{l}.{n}" for n in ("ln1_w", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
                                         "ln2_w", "ln2_b", "fc1", "b1", "fc2", "b2")]
    names += ["ln_f_w", "ln_f_b", "lm_head"]
    with open(path, "wb") as f:
        for n in names:
            f.write(np.ascontiguousarray(m[n], dtype="<f4").tobytes())
