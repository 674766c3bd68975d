"""The oracle reproduces every committed golden fixture exactly (CPU)."""
import glob
import os

import numpy as np
import pytest

from golden import make_golden as G

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(HERE, "*.npz")))


def recompute(name):
    if name == "C1_full":
        return G.config_case("C1", 512)
    if name.endswith("_t64"):
        return G.config_case(name[:2], 64)
    if name == "tie_softmax_bias":
        return G.tie_case(G.O.SCORING_SOFTMAX_BIAS)
    if name == "tie_sigmoid_group":
        return G.tie_case(G.O.SCORING_SIGMOID_GROUP)
    if name == "degenerate":
        return G.degenerate_case()
    raise KeyError(name)


def test_fixture_set():
    assert set(FIXTURES) == {"C1_full", "C2_t64", "C3_t64", "C4_t64", "C5_t64",
                             "tie_softmax_bias", "tie_sigmoid_group", "degenerate"}


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_reproduces_fixture(name):
    want = np.load(os.path.join(HERE, name + ".npz"))
    got = recompute(name)
    assert set(want.files) == set(got)
    for k in want.files:
        assert np.array_equal(np.asarray(got[k]), want[k]), (name, k)
