"""CPU checks of the packed checkpoint reader (ModelWeights::load_packed):
files written here by an independent writer of the documented format
(include/cbis_runtime.h, csrc/runtime/model_weights.cpp) are accepted up to
the device allocation, and every malformed variant is rejected before it."""
import struct

import numpy as np
import pytest

F32, BF16, FP8 = 0, 1, 2
SIZE = {F32: 4, BF16: 2, FP8: 1}


def _layout(cfg):
    """(name, dtype, offset, bytes) of every arena tensor, 256-byte aligned,
    in the loader's order."""
    V, D, H, hd, L, F, S, ps, wd, kvd = cfg
    ed = F32 if wd == F32 else BF16
    fp8 = wd == FP8
    out, off = [], 0

    def add(name, dt, nbytes):
        nonlocal off
        out.append((name, dt, off, nbytes))
        off = (off + nbytes + 255) // 256 * 256

    add("tok_emb", ed, V * D * SIZE[ed])
    add("pos_emb", ed, S * D * SIZE[ed])
    for l in range(L):
        p = f"l{l}."
        for n in ("ln1_w", "ln1_b", "ln2_w", "ln2_b"):
            add(p + n, F32, D * 4)
        add(p + "wqkv", wd, 3 * D * D * SIZE[wd]); add(p + "bqkv", F32, 3 * D * 4)
        add(p + "wo", wd, D * D * SIZE[wd]); add(p + "bo", F32, D * 4)
        add(p + "w1", wd, F * D * SIZE[wd]); add(p + "b1", F32, F * 4)
        add(p + "w2", wd, D * F * SIZE[wd]); add(p + "b2", F32, D * 4)
        if fp8:
            add(p + "sqkv", F32, 3 * D * 4); add(p + "so", F32, D * 4)
            add(p + "s1", F32, F * 4); add(p + "s2", F32, D * 4)
    add("ln_f_w", F32, D * 4)
    add("ln_f_b", F32, D * 4)
    add("lm_head", wd, V * D * SIZE[wd])
    if fp8:
        add("lm_scale", F32, V * 4)
    return out


def _checksum(data: bytes) -> int:
    h, M = 0, (1 << 64) - 1
    words = np.frombuffer(data[: len(data) // 8 * 8], dtype="<u8")
    for w in words.tolist():
        h = (((h << 5) | (h >> 59)) & M) ^ w
        h = (h * 0x9E3779B97F4A7C15) & M
    for b in data[len(data) // 8 * 8:]:
        h = (((h << 5) | (h >> 59)) & M) ^ b
        h = (h * 0x9E3779B97F4A7C15) & M
    return h


def _write(path, cfg, *, magic=b"CBISWT01", version=1, table=None, data=None, truncate=0, bad_sum=False,
           count=None):
    table = table if table is not None else _layout(cfg)
    arena = table[-1][2] + table[-1][3]
    if data is None:
        data = bytes((i * 37 + 11) & 0xFF for i in range(arena))
    head = magic + struct.pack("<II", version, len(table) if count is None else count)
    head += struct.pack("<10i", *cfg)
    fixed = len(head)
    head += struct.pack("<QQQ", arena, 0, 0)
    for name, dt, off, nb in table:
        head += struct.pack("<H", len(name)) + name.encode() + struct.pack("<IQQ", dt, off, nb)
    data_off = (len(head) + 4095) // 4096 * 4096
    s = _checksum(data) ^ (1 if bad_sum else 0)
    head = head[:fixed] + struct.pack("<QQQ", arena, data_off, s) + head[fixed + 24:]
    blob = head + b"\0" * (data_off - len(head)) + data
    with open(path, "wb") as f:
        f.write(blob[: len(blob) - truncate])


CFG = (64, 32, 2, 16, 2, 64, 16, 16, BF16, BF16)   # vocab, d, heads, hd, layers, mlp, max_seq, page, w, kv
CFG8 = (64, 32, 2, 16, 2, 64, 16, 16, FP8, BF16)


@pytest.mark.parametrize("cfg", [CFG, CFG8])
def test_wellformed_file_reaches_allocation(cbis, tmp_path, cfg):
    """A file from this writer passes every header check; without a GPU the
    loader then stops at the device allocation."""
    p = tmp_path / "w.cbisw"
    _write(p, cfg)
    with pytest.raises(RuntimeError, match="hipMalloc"):
        cbis.ModelWeights.load_packed(str(p))


@pytest.mark.parametrize("kind,match", [
    ("magic", "bad magic"),
    ("version", "unsupported version"),
    ("count", "tensor count"),
    ("name", "tensor table differs"),
    ("offset", "tensor table differs"),
    ("dtype", "tensor table differs"),
    ("truncate", "truncated"),
    ("config", "n_heads \\* head_dim"),
])
def test_malformed_file_rejected(cbis, tmp_path, kind, match):
    p = tmp_path / "w.cbisw"
    table = _layout(CFG)
    if kind == "magic":
        _write(p, CFG, magic=b"CBISWT00")
    elif kind == "version":
        _write(p, CFG, version=2)
    elif kind == "count":
        _write(p, CFG, count=len(table) - 1)
    elif kind == "name":
        t = list(table); t[3] = ("l0.ln1_x",) + t[3][1:]
        _write(p, CFG, table=t)
    elif kind == "offset":
        t = list(table); t[5] = t[5][:2] + (t[5][2] + 256,) + t[5][3:]
        _write(p, CFG, table=t)
    elif kind == "dtype":
        t = list(table); t[-1] = (t[-1][0], FP8) + t[-1][2:]
        _write(p, CFG, table=t)
    elif kind == "truncate":
        _write(p, CFG, truncate=1)
    elif kind == "config":
        bad = list(CFG); bad[2] = 3    # n_heads * head_dim != d_model
        _write(p, tuple(bad), table=table)
    with pytest.raises(RuntimeError, match=match) as ei:
        cbis.ModelWeights.load_packed(str(p))
    assert "hipMalloc" not in str(ei.value)


def test_missing_file(cbis, tmp_path):
    with pytest.raises(RuntimeError, match="cannot open"):
        cbis.ModelWeights.load_packed(str(tmp_path / "none.cbisw"))


# The reference's weights.bin (ModelWeights::load, src/model_weights.cpp:41-75)

def test_weights_bin_size_must_match_config(cbis, oracle, tmp_path):
    """A weights.bin of exactly the config's tensors reaches the device
    allocation; one byte-count off in either direction (other dims, trailing
    bytes, truncation) is refused before it."""
    from helpers import write_weights_bin
    spec = oracle.ModelSpec(vocab=64, d_model=64, n_heads=2, n_layers=2, mlp=256, max_seq=32)
    cfg = cbis.ModelConfig.make(vocab=64, d_model=64, n_heads=2, n_layers=2, mlp=256, max_seq=32)
    p = tmp_path / "weights.bin"
    write_weights_bin(p, oracle.synthetic_weights(spec, seed=0))
    good = p.read_bytes()
    D, F, V, S = 64, 256, 64, 32
    assert len(good) == 4 * (2 * V * D + S * D + 2 * (9 * D + 4 * D * D + 2 * F * D + F) + 2 * D)
    with pytest.raises(RuntimeError, match="hipMalloc"):
        cbis.ModelWeights.load(str(p), cfg)
    for blob in (good[:-4], good + b"\0\0\0\0", good[:-1]):
        p.write_bytes(blob)
        with pytest.raises(RuntimeError, match="the config's tensors are") as ei:
            cbis.ModelWeights.load(str(p), cfg)
        assert "hipMalloc" not in str(ei.value)
    p.write_bytes(good)
    other = cbis.ModelConfig.make(vocab=64, d_model=64, n_heads=2, n_layers=3, mlp=256, max_seq=32)
    with pytest.raises(RuntimeError, match="the config's tensors are"):
        cbis.ModelWeights.load(str(p), other)
