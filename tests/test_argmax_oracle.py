"""The oracle's greedy token (first index of the maximum, the sampler's errors) pinned by
closed-form cases and against a direct loop over the reference's MTP argmax steps
(src/runtime/qwen35_mtp.cpp:300-308: start from element 0, take an element only when strictly
larger)."""
import numpy as np
import pytest

import oracle


def loop_argmax(v):
    best_i, best = 0, v[0]
    for i in range(1, len(v)):
        if v[i] > best:
            best, best_i = v[i], i
    return best_i


@pytest.mark.parametrize("v,want", [
    ([3.0], 0),
    ([1.0, 5.0, 5.0, 2.0], 1),            # ties: the first index
    ([7.0, 7.0, 7.0], 0),
    ([-3.0, -1.0, -2.0], 1),
    ([0.0, -0.0], 0),                     # -0 == 0: the first
    ([-np.inf, -5.0, -np.inf], 1),
    ([1.0, 2.0, 3.0, 4.0], 3),
])
def test_known_answers(v, want):
    i, val = oracle.greedy_token(np.array(v, np.float32))
    assert i == want and val == np.float32(v[want])


@pytest.mark.parametrize("v,msg", [([], "empty"), ([1.0, np.nan], "NaN"), ([-np.inf, -np.inf], "no finite"),
                                   ([1.0, np.inf], "no finite")])
def test_sampler_errors(v, msg):
    with pytest.raises(ValueError, match=msg):
        oracle.greedy_token(np.array(v, np.float32))


def test_matches_reference_loop_with_ties():
    rng = np.random.default_rng(5)
    for n in (1, 2, 17, 1000, 4099):
        for _ in range(20):
            v = rng.integers(-4, 5, n).astype(np.float32)  # many ties
            assert oracle.greedy_token(v)[0] == loop_argmax(v)
