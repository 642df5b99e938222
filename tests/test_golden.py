"""The committed golden vectors (tests/golden/dsa_small.npz) are what the CPU
oracle computes for their inputs: regenerating them must give the same bits,
so an edit to the oracle cannot silently move the GPU tests' expectations."""

import sys
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))


def test_golden_vectors_match_the_oracle():
    import make_golden

    stored = np.load(GOLDEN / "dsa_small.npz")
    fresh = make_golden.make()
    assert sorted(stored.files) == sorted(fresh)
    for name in stored.files:
        a, b = stored[name], np.asarray(fresh[name])
        assert a.dtype == b.dtype and a.shape == b.shape, name
        assert np.array_equal(a.reshape(-1).view(np.uint8), b.reshape(-1).view(np.uint8)), name


@pytest.mark.parametrize("name", ["quant_codes", "topk_ids", "kv_cache", "mla_out_bits"])
def test_golden_outputs_are_nontrivial(name):
    data = np.load(GOLDEN / "dsa_small.npz")[name]
    assert np.unique(data).size > 8, name
