"""Writes the golden fixtures that pin the CPU oracle's whole forward step.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/gen_golden.py /root/reference

It imports the reference's ``python/model.py`` (TinyGPT, python/model.py:23-77)
-- the only definition of the forward's math end to end -- overrides its
module-level dimensions for each configuration, loads weights into it and
records inputs and logits.  Nothing of the reference is copied into the
fixtures: they hold token ids, generated tokens and logits only.

Fixtures:
  g1_refmodel.npz   reference dims (V=1000, d=256, 8x32, L=4, mlp=1024), our
                    synthetic weights (seed 0), 6 sequences of lengths
                    1/3/7/16/31/64 (python/export_weights.py:69-85 shape).
  g1_weightsbin.npz the reference's own python/weights.bin with
                    export_reference's token batch (seed 777): the
                    reference.bin content the reference gitignores.
  g2_c1_greedy.npz  config C1 (V=512): 8 prompts, 32 greedy tokens each by
                    full recompute, and every generated step's logits.
  g3_mid_bf16.npz   reduced mid-size GPT (d=2048, 64x32, mlp=8192, V=32000,
                    2 layers), bf16-rounded weights: logits of 4 rows (fp16).
  g3_mid_fp8.npz    the same with fp8-e4m3 per-channel-scaled linear weights.
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle  # noqa: E402


def import_model(ref_root):
    sys.path.insert(0, os.path.join(ref_root, "python"))
    import model  # the reference's python/model.py
    return model


def configure(model, spec):
    model.VOCAB = spec.vocab
    model.D_MODEL = spec.d_model
    model.N_HEADS = spec.n_heads
    model.HEAD_DIM = spec.head_dim
    model.N_LAYERS = spec.n_layers
    model.MLP_HIDDEN = spec.mlp
    model.MAX_SEQ_LEN = spec.max_seq


def build_torch(model, spec, weights: oracle.Weights):
    configure(model, spec)
    torch.manual_seed(0)
    m = model.TinyGPT()
    m.eval()
    u = weights.used
    sd = {}

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))

    def lin(name):
        w = u[name].astype(np.float32)
        sc = weights.scale.get(name)
        if sc is not None:
            w = (w.astype(np.float64) * sc.astype(np.float64)[:, None]).astype(np.float32)
        return t(w)

    sd["tok_emb.weight"] = t(u["tok_emb"])
    pe = np.zeros((spec.max_seq, spec.d_model), np.float32)
    pe[: u["pos_emb"].shape[0]] = u["pos_emb"]
    sd["pos_emb.weight"] = t(pe)
    for l in range(spec.n_layers):
        p = f"blocks.{l}."
        sd[p + "ln1.weight"] = t(u[f"l{l}.ln1_w"]); sd[p + "ln1.bias"] = t(u[f"l{l}.ln1_b"])
        sd[p + "ln2.weight"] = t(u[f"l{l}.ln2_w"]); sd[p + "ln2.bias"] = t(u[f"l{l}.ln2_b"])
        for tn, on, bn in (("wq", "wq", "bq"), ("wk", "wk", "bk"), ("wv", "wv", "bv"), ("wo", "wo", "bo"),
                           ("fc1", "fc1", "b1"), ("fc2", "fc2", "b2")):
            sd[p + tn + ".weight"] = lin(f"l{l}.{on}")
            sd[p + tn + ".bias"] = t(u[f"l{l}.{bn}"])
    sd["ln_f.weight"] = t(u["ln_f_w"]); sd["ln_f.bias"] = t(u["ln_f_b"])
    sd["lm_head.weight"] = lin("lm_head")
    m.load_state_dict(sd, strict=True)
    return m


@torch.no_grad()
def logits_of(m, ids):
    return m(torch.tensor([ids], dtype=torch.long))[0].numpy().astype(np.float32)


def g1_refmodel(model):
    spec = oracle.ModelSpec()
    w = oracle.synthetic_weights(spec, seed=0, pos_rows=64)
    m = build_torch(model, spec, w)
    lens = (1, 3, 7, 16, 31, 64)
    ids = [oracle.uniform_int(0, 2001, n, 0, spec.vocab - 1, start=i * 4096) for i, n in enumerate(lens)]
    out = {"lens": np.array(lens, np.int32)}
    for i, seq in enumerate(ids):
        out[f"ids{i}"] = seq.astype(np.int32)
        out[f"logits{i}"] = logits_of(m, [int(x) for x in seq])
    np.savez_compressed(os.path.join(HERE, "g1_refmodel.npz"), **out)


def g1_weightsbin(model, ref_root):
    spec = oracle.ModelSpec()
    w = oracle.load_weights_bin(os.path.join(ref_root, "python", "weights.bin"), spec)
    m = build_torch(model, spec, w)
    lens = (1, 3, 7, 16, 31, 64)
    g = torch.Generator().manual_seed(777)
    batch = torch.randint(0, spec.vocab, (len(lens), max(lens)), generator=g)
    out = {"lens": np.array(lens, np.int32)}
    for i, n in enumerate(lens):
        seq = batch[i, :n].tolist()
        out[f"ids{i}"] = np.array(seq, np.int32)
        out[f"logits{i}"] = logits_of(m, seq)
    np.savez_compressed(os.path.join(HERE, "g1_weightsbin.npz"), **out)


def g2_c1(model):
    spec = oracle.ModelSpec(vocab=512)
    w = oracle.synthetic_weights(spec, seed=0, pos_rows=128)
    m = build_torch(model, spec, w)
    reqs = oracle.c1_requests(seed=0)
    out = {"n": np.array(len(reqs), np.int32)}
    for i, r in enumerate(reqs):
        seq = list(r.prompt)
        gen, lg, margin = [], [], []
        for _ in range(r.decode_len):
            row = logits_of(m, seq)[-1]
            tok = int(torch.argmax(torch.from_numpy(row)).item())
            top2 = np.sort(row)[-2:]
            gen.append(tok); lg.append(row); margin.append(float(top2[1] - top2[0]))
            seq.append(tok)
        out[f"prompt{i}"] = np.array(r.prompt, np.int32)
        out[f"gen{i}"] = np.array(gen, np.int32)
        out[f"logits{i}"] = np.stack(lg).astype(np.float32)
        out[f"margin{i}"] = np.array(margin, np.float32)
    np.savez_compressed(os.path.join(HERE, "g2_c1_greedy.npz"), **out)


def g3_mid(model, wdtype):
    spec = oracle.ModelSpec(vocab=32000, d_model=2048, n_heads=64, head_dim=32, n_layers=2, mlp=8192,
                            weight_dtype=wdtype, kv_dtype="bf16")
    w = oracle.synthetic_weights(spec, seed=0, pos_rows=16)
    spec_t = oracle.ModelSpec(**{**spec.__dict__, "max_seq": 16})
    m = build_torch(model, spec_t, w)
    lens = (5, 9)
    out = {"lens": np.array(lens, np.int32)}
    rows = {0: (2, 4), 1: (0, 8)}
    for i, n in enumerate(lens):
        seq = oracle.uniform_int(0, 2003, n, 0, spec.vocab - 1, start=i * 4096)
        lg = logits_of(m, [int(x) for x in seq])
        out[f"ids{i}"] = seq.astype(np.int32)
        out[f"rows{i}"] = np.array(rows[i], np.int32)
        out[f"logits{i}"] = lg[list(rows[i])].astype(np.float16)
    np.savez_compressed(os.path.join(HERE, f"g3_mid_{wdtype}.npz"), **out)


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    torch.set_num_threads(8)
    model = import_model(ref_root)
    g1_refmodel(model)
    g1_weightsbin(model, ref_root)
    g2_c1(model)
    g3_mid(model, "bf16")
    g3_mid(model, "fp8")
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
