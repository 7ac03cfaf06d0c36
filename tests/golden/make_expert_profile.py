"""Measured expert popularity of MiMo-V2.6-Flash's MoE layers, as a fixture.

    python tests/golden/make_expert_profile.py      # reads the reference's data file, rewrites expert_profile.npz

Source: engine/mimo_stream/data/expert_profile.npz of the reference (keys L01 .. L47, 256 int64 selection counts
per MoE layer), which the engine loads at engine/server.py:41-45 and uses to order each layer's resident slots
(engine/mimo_stream/model.py:158-167).  It is read with numpy.load(allow_pickle=False) and written here as one
int64 array `counts` [47, 256] (row i = layer L(i + 1)) plus `layers` [47], so tests and the benchmark can draw
routes with the real per-layer popularity next to the synthetic Zipf(1.1) one.  The counts are copied unchanged.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "expert_profile.npz")
SOURCE = "/root/reference/engine/mimo_stream/data/expert_profile.npz"


def main(src=SOURCE):
    z = np.load(src, allow_pickle=False)
    keys = sorted(z.files, key=lambda k: int(k[1:]))
    layers = np.array([int(k[1:]) for k in keys], np.int32)
    counts = np.stack([np.asarray(z[k], np.int64) for k in keys])
    assert counts.shape == (47, 256) and (counts >= 0).all()
    np.savez_compressed(PATH, counts=counts, layers=layers)
    print(PATH, counts.shape, int(counts.sum()))


def load():
    """(layers int32 [47], counts int64 [47, 256]) from the committed fixture."""
    with np.load(PATH, allow_pickle=False) as z:
        return z["layers"], z["counts"]


if __name__ == "__main__":
    main(*sys.argv[1:])
