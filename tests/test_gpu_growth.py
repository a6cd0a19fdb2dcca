"""GPU: the reference's growth-policy cases (tests/lossguide.rs,
tests/max_leaves.rs; growth_cases.py) grow the oracle's trees on the device,
and meet the reference's expectations themselves."""

from __future__ import annotations

import numpy as np
import pytest

from growth_cases import cases, unlimited_equals_nonbinding
from helpers import assert_same_models

pytestmark = pytest.mark.gpu

CASES = cases()


@pytest.fixture(scope="module")
def fb():
    import ferrisboost_amd as fb
    from ferrisboost_amd import _native as N

    if not N.device_available(0):
        pytest.fail("no gfx950 device: the GPU suite needs an MI355X")
    return fb


def _both(fb, oracle, x, y, p):
    kw = dict(p)
    n = kw.pop("n_rounds")
    om = oracle.train(x, y, oracle.make_params(n_rounds=n, cols_per_block=1, nthread=1, **kw))
    pm = fb.train(kw, x, y, num_boost_round=n)
    return om, pm


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_growth_case_on_the_device(fb, oracle, case):
    _, x, y, p, check = case
    om, pm = _both(fb, oracle, x, y, p)
    assert_same_models(om, pm)
    check(pm.trees())
    assert np.array_equal(pm.train_margins(y.size).view(np.uint32),
                          om.train_margins(y.size).view(np.uint32))


@pytest.mark.parametrize("host_levels", [False, True])
def test_zero_and_nonbinding_leaf_limits_match_on_the_device(fb, host_levels):
    x, y, p = unlimited_equals_nonbinding()
    kw = {k: v for k, v in p.items() if k != "n_rounds"}
    kw["hip_host_levels"] = host_levels
    a = fb.train(dict(kw, max_leaves=0), x, y, num_boost_round=p["n_rounds"])
    b = fb.train(dict(kw, max_leaves=64), x, y, num_boost_round=p["n_rounds"])
    assert_same_models(a, b)
    assert a.to_json() == b.to_json()
