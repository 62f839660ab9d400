"""The oracle against the committed fixtures of tests/golden (regression lock:
inputs are regenerated from their seeds and must equal the stored ones, and
every stored output must be reproduced bit for bit)."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))


def test_oracle_reproduces_golden_vectors():
    import make_golden
    want = np.load(os.path.join(HERE, "golden", "oracle_golden.npz"))
    got = make_golden.compute()
    assert sorted(want.files) == sorted(got)
    for k in want.files:
        assert np.array_equal(np.asarray(got[k]), want[k]), k
