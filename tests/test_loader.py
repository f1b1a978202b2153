"""The expert-cache index as the loader reads it (tinygiant_amd/loader.py,
following tinygiant/cache.py:29-54): offsets, sizes and formats of every
expert, and the q4_k default for a layer without tensor_formats."""

import numpy as np

from tests._expert_cache import write_cache
from tinygiant_amd import loader as LD


def test_index_layout_and_formats(tmp_path):
    rng = np.random.default_rng(0)
    sizes = {"gate": 144 * 3, "up": 144 * 3, "down": 210 * 2}
    layers = {l: {e: {k: rng.integers(0, 256, sizes[k], dtype=np.uint8) for k in sizes} for e in (0, 1, 2, 5)}
              for l in (0, 1)}
    idx = write_cache(tmp_path, layers, 6, 256, 192, {"gate": 0, "up": 0, "down": 2}, omit_formats=(1,))
    assert LD.read_index(tmp_path) == idx
    fname, total, fmts, experts = LD.layer_layout(idx, 0)
    assert fname == "layer_000.q4.bin" and total == 4 * sum(sizes.values())
    assert fmts == {"gate": 0, "up": 0, "down": 2}
    assert [e for e, _, _ in experts] == [0, 1, 2, 5]
    blob = (tmp_path / fname).read_bytes()
    for eid, off, sz in experts:
        p = off
        for k in ("gate", "up", "down"):
            assert blob[p:p + sz[k]] == layers[0][eid][k].tobytes()
            p += sz[k]
    # no tensor_formats: every tensor reads as q4_k (tinygiant/engine.py:326-327)
    assert LD.layer_layout(idx, 1)[2] == {"gate": 0, "up": 0, "down": 0}
