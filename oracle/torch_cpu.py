"""fp32 PyTorch-on-CPU forward of one continuous-batch step -- TEST
INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and tests/ use it).

The reference's CPU forward is python/model.py: PyTorch modules in fp32 on
the host (nn.LayerNorm, nn.Linear, F.gelu, a causal softmax attention,
python/model.py:35-70).  This module restates that forward with the same
operators, in fp32, for the server's step shape (src/transformer.cpp:44-99):
rows of many sequences, each row's K/V written into the paged pools before
its attention reads keys 0..position through the page table
(kernels/attention.cu:57-98).  Where the model's weights are bf16 or fp8 it
rounds the GEMM inputs to bf16 at the same points as the C oracle
(oracle/cbis_oracle.c orc_step_layer), so the two agree to fp32 rounding.

It exists to time a like-for-like CPU baseline (fp32, vectorised library
GEMMs on the host's cores) beside the GPU step; the fp64 C oracle stays the
checker.  Pinned against that oracle in tests/test_cpu_oracle.py
(test_torch_cpu_step_matches_c_oracle: f32 and bf16 models, decode rows and
a prefill chunk with cached keys).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def _t(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


def _bf16_round(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


class TorchCpuStep:
    """One step's forward over host pools.  weights: oracle.Weights (its
    `used` fp32 values and fp8 channel scales); kpools / vpools: per-layer
    [pages, page_size, heads, head_dim] arrays, float32 or uint16 bf16 bits
    (written in place by each layer, as the step writes its rows' K/V)."""

    def __init__(self, weights, kpools, vpools):
        self.spec = s = weights.spec
        self.kpools, self.vpools = kpools, vpools
        u, sc = weights.used, weights.scale
        self.round = s.act_bf16

        def lin(name):
            W = _t(u[name])
            if name in sc:  # fp8: dequantised values times the channel scale
                W = W * _t(sc[name])[:, None]
            return W

        self.tok_emb, self.pos_emb = _t(u["tok_emb"]), _t(u["pos_emb"])
        self.ln_f = (_t(u["ln_f_w"]), _t(u["ln_f_b"]))
        self.lm_head = lin("lm_head")
        self.layers = []
        for l in range(s.n_layers):
            p = f"l{l}."
            self.layers.append({
                "ln1": (_t(u[p + "ln1_w"]), _t(u[p + "ln1_b"])), "ln2": (_t(u[p + "ln2_w"]), _t(u[p + "ln2_b"])),
                "wq": lin(p + "wq"), "wk": lin(p + "wk"), "wv": lin(p + "wv"), "wo": lin(p + "wo"),
                "fc1": lin(p + "fc1"), "fc2": lin(p + "fc2"),
                "bq": _t(u[p + "bq"]), "bk": _t(u[p + "bk"]), "bv": _t(u[p + "bv"]), "bo": _t(u[p + "bo"]),
                "b1": _t(u[p + "b1"]), "b2": _t(u[p + "b2"])})

    def _act(self, x):
        return _bf16_round(x) if self.round else x

    def _pool(self, pool) -> torch.Tensor:
        """The pool as [slots, heads * head_dim] (bf16 bits viewed as bf16)."""
        s = self.spec
        if pool.dtype == np.uint16:
            t = torch.from_numpy(pool.view(np.int16)).view(torch.bfloat16)
        else:
            t = torch.from_numpy(pool)
        return t.reshape(-1, s.n_heads * s.head_dim)

    def embed(self, tok, pos) -> torch.Tensor:
        """python/model.py:63-66: token + position embedding."""
        return self.tok_emb[torch.as_tensor(tok, dtype=torch.long)] + self.pos_emb[torch.as_tensor(pos, dtype=torch.long)]

    def _attention(self, q, kpool, vpool, pos, block_table, row_bt) -> torch.Tensor:
        """Each row attends to keys 0..pos of its block-table row, scaled by
        1/sqrt(head_dim) and softmax-normalised (python/model.py:40-44); rows
        of one sequence share one gather of its keys, with a causal mask."""
        s = self.spec
        H, hd, ps = s.n_heads, s.head_dim, s.page_size
        kp, vp = self._pool(kpool), self._pool(vpool)
        out = torch.empty_like(q)
        pos = np.asarray(pos)
        row_bt = np.asarray(row_bt)
        for r in np.unique(row_bt):
            rows = np.nonzero(row_bt == r)[0]
            n_keys = int(pos[rows].max()) + 1
            j = np.arange(n_keys)
            slots = torch.from_numpy((block_table[r][j // ps].astype(np.int64) * ps + j % ps))
            K = kp.index_select(0, slots).to(torch.float32).reshape(n_keys, H, hd).transpose(0, 1)
            V = vp.index_select(0, slots).to(torch.float32).reshape(n_keys, H, hd).transpose(0, 1)
            Q = q[torch.from_numpy(rows)].reshape(len(rows), H, hd).transpose(0, 1)
            S = torch.matmul(Q, K.transpose(1, 2)) / float(np.sqrt(hd))
            mask = torch.from_numpy(j[None, :] > pos[rows][:, None])
            S = S.masked_fill(mask[None], float("-inf"))
            O = torch.matmul(torch.softmax(S, dim=-1), V)
            out[torch.from_numpy(rows)] = O.transpose(0, 1).reshape(len(rows), H * hd)
        return out

    def layer(self, l, x, pos, wpage, woff, block_table, row_bt) -> torch.Tensor:
        """python/model.py:48-52 (x + attn(ln1 x), then x + mlp(ln2 x)) for the
        step's rows; K/V are written into layer l's pools first."""
        s, L = self.spec, self.layers[l]
        D = s.d_model
        a = self._act(F.layer_norm(x, (D,), *L["ln1"], eps=1e-5))
        q = F.linear(a, L["wq"], L["bq"])
        k = F.linear(a, L["wk"], L["bk"])
        v = F.linear(a, L["wv"], L["bv"])
        kp, vp = self._pool(self.kpools[l]), self._pool(self.vpools[l])
        slots = torch.from_numpy(np.asarray(wpage, np.int64) * s.page_size + np.asarray(woff, np.int64))
        kp[slots] = k.to(kp.dtype)
        vp[slots] = v.to(vp.dtype)
        att = self._act(self._attention(q, self.kpools[l], self.vpools[l], pos, block_table, row_bt))
        x = x + F.linear(att, L["wo"], L["bo"])
        a = self._act(F.layer_norm(x, (D,), *L["ln2"], eps=1e-5))
        h = self._act(F.gelu(F.linear(a, L["fc1"], L["b1"])))
        return x + F.linear(h, L["fc2"], L["b2"])

    def head(self, x) -> torch.Tensor:
        """Final LayerNorm and lm_head (no bias), python/model.py:67-70."""
        a = self._act(F.layer_norm(x, (self.spec.d_model,), *self.ln_f, eps=1e-5))
        return F.linear(a, self.lm_head)

    @torch.no_grad()
    def forward_step(self, tok, pos, wpage, woff, block_table, row_bt) -> torch.Tensor:
        x = self.embed(tok, pos)
        for l in range(self.spec.n_layers):
            x = self.layer(l, x, pos, wpage, woff, block_table, row_bt)
        return self.head(x)
