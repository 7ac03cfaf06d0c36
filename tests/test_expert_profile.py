"""The measured-popularity fixture (tests/golden/expert_profile.npz, from the reference's
engine/mimo_stream/data/expert_profile.npz): 47 MoE layers x 256 selection counts, every layer the same number
of selections (tokens x top-8), and, where the reference tree is present, equal to its file."""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_expert_profile as mep  # noqa: E402


def test_fixture_shape_and_totals():
    layers, counts = mep.load()
    assert layers.tolist() == list(range(1, 48))
    assert counts.shape == (47, 256) and counts.dtype == np.int64 and (counts >= 0).all()
    tot = counts.sum(1)
    assert (tot == tot[0]).all() and tot[0] % 8 == 0          # every layer saw the same tokens, 8 routes each
    top = counts.max(1) / tot
    assert 0.02 < top.min() and top.max() < 0.11               # the most popular expert: 2.4-10.5% of routes


@pytest.mark.skipif(not os.path.exists(mep.SOURCE), reason="reference tree not present")
def test_fixture_equals_reference_file():
    layers, counts = mep.load()
    z = np.load(mep.SOURCE, allow_pickle=False)
    for i, L in enumerate(layers):
        np.testing.assert_array_equal(counts[i], z[f"L{L:02d}"])
