"""CPU checks of the colder tiers' block codec (zlib deflate at its fastest
level, src/block_storage.cpp:7-31): exact round trips on K/V-like fp32 and
bf16 bytes, on incompressible and on constant blocks, and the errors a
damaged or mis-sized block raises."""
import zlib

import numpy as np
import pytest


@pytest.mark.parametrize("kind", ["f32", "bf16", "random", "zeros", "tiny"])
def test_block_round_trip(cbis, kind):
    rng = np.random.default_rng(7)
    if kind == "f32":
        raw = rng.standard_normal(4 * 2 * 16 * 8 * 32).astype(np.float32).tobytes()  # one reference block
    elif kind == "bf16":
        raw = (rng.standard_normal(2 * 16 * 64 * 32).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16).tobytes()
    elif kind == "random":
        raw = rng.integers(0, 256, 100_000, dtype=np.uint8).tobytes()
    elif kind == "zeros":
        raw = bytes(65536)
    else:
        raw = b"\x01"
    comp = cbis.block_deflate(raw)
    assert zlib.decompress(comp) == raw          # a standard zlib stream
    assert cbis.block_inflate(comp, len(raw)) == raw
    if kind == "zeros":
        assert len(comp) < len(raw) // 100


def test_block_inflate_rejects_damage(cbis):
    raw = np.arange(4096, dtype=np.float32).tobytes()
    comp = bytearray(cbis.block_deflate(raw))
    with pytest.raises(RuntimeError, match="size mismatch|zlib error"):
        cbis.block_inflate(bytes(comp), len(raw) - 4)
    comp[len(comp) // 2] ^= 0xFF
    with pytest.raises(RuntimeError, match="zlib error|size mismatch"):
        cbis.block_inflate(bytes(comp), len(raw))
