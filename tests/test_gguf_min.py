"""CPU tests of the tests' GGUF reader (tests/gguf_min.py): a split model written by the writer
reads back with every tensor's shard, dims, type and bytes; the data sections honour each file's
own general.alignment; a foreign file is refused."""
from __future__ import annotations

import numpy as np
import pytest

from tests import gguf_min as G


def test_split_model_round_trip(tmp_path):
    rng = np.random.default_rng(1)
    t1 = [("a.weight", [64, 3], G.GGML_Q2_0, rng.integers(0, 256, 3 * 18, dtype=np.uint8).tobytes()),
          ("b.weight", [5], G.GGML_F32, rng.standard_normal(5).astype(np.float32).tobytes())]
    t2 = [("c.weight", [32, 2], G.GGML_Q8_0, rng.integers(0, 256, 2 * 34, dtype=np.uint8).tobytes()),
          ("d.weight", [7, 2], G.GGML_F16, rng.standard_normal(14).astype(np.float16).tobytes())]
    p1, p2 = str(tmp_path / "m-00001-of-00002.gguf"), str(tmp_path / "m-00002-of-00002.gguf")
    G.write_gguf(p1, t1, {"split.count": 2, "general.name": "x"}, align=32)
    G.write_gguf(p2, t2, {"split.count": 2}, align=256)
    g = G.open_gguf(p1)
    assert g.shards == [p1, p2]
    assert g.meta["general.name"] == "x" and g.meta["general.alignment"] == 32
    for shard, ts in ((0, t1), (1, t2)):
        for name, dims, ty, raw in ts:
            t = g.tensor(name)
            assert (t.shard, t.dims, t.type) == (shard, dims, ty)
            assert t.nbytes() == len(raw)
            assert g.read(t) == raw
    assert g.tensor("c.weight").file_offset % 256 == 0   # shard 2's own alignment


def test_not_gguf(tmp_path):
    p = tmp_path / "x.gguf"
    p.write_bytes(b"GGML" + b"\0" * 64)
    with pytest.raises(ValueError):
        G.open_gguf(str(p))
