"""Tree-growth cases of the reference's own tests, restated as data: each is
(name, x, y, params, expectation). The oracle must meet every expectation
(tests/test_oracle_growth.py), and the device must grow the oracle's trees
from them (tests/test_gpu_growth.py).

Sources: tests/lossguide.rs:50-147 and tests/max_leaves.rs:75-205 of the
reference. Every case uses one feature binned with 16 bins
(DenseSource::from_row_major(values, n, 1, 16, 1)), squared error, a fixed
base score, min_child_weight 0 and learning rate 0.3.
"""

from __future__ import annotations

import numpy as np

X8 = np.arange(8, dtype=np.float32)
SEPARABLE = np.array([0.0, 0.0, 1.0, 1.0, 3.0, 3.0, 4.0, 4.0], np.float32)


def _p(**kw):
    p = {"n_rounds": 1, "max_bin": 16, "eta": 0.3, "lambda": 0.0, "min_child_weight": 0.0,
         "objective": "reg:squarederror", "base_score": 0.0, "grow_policy": "lossguide",
         "max_depth": 8, "max_leaves": 0}
    p.update(kw)
    return p


def _leaves(t):
    return int((t["is_leaf"] == 1).sum())


def _split(t, i):
    return not t[i]["is_leaf"]


# (name, x, y, params, check(trees) -> None)
def cases():
    out = []

    def add(name, x, y, params, check):
        out.append((name, np.asarray(x, np.float32).reshape(-1, 1),
                    np.asarray(y, np.float32), params, check))

    y_gain = [0., 0., 1., 1., 10., 10., 14., 20.]
    y_tie = [0., 0., 1., 1., 3., 3., 4., 4.]

    def highest_gain(tr):
        t = tr[0]
        assert _leaves(t) == 3 and _split(t, 0)
        assert not _split(t, 1), "the lower-gain left candidate stays a leaf"
        assert _split(t, 2), "the higher-gain right candidate is split"

    add("lossguide_highest_gain_under_cap", X8, y_gain, _p(max_leaves=3), highest_gain)

    def tie(tr):
        t = tr[0]
        assert _leaves(t) == 3 and _split(t, 1) and not _split(t, 2), "ties go to the lower id"

    add("lossguide_tie_lower_node_id", X8, y_tie, _p(max_leaves=3), tie)

    def root_only(tr):
        assert tr[0].size == 1 and _leaves(tr[0]) == 1

    add("lossguide_depth0", X8, y_tie, _p(max_depth=0, max_leaves=0), root_only)
    add("lossguide_one_leaf_cap", X8, y_tie, _p(max_depth=8, max_leaves=1), root_only)

    x32 = np.arange(32, dtype=np.float32)
    y32 = np.array([(v // 4) ** 2 for v in range(32)], np.float32)
    def uncapped(tr):
        assert _leaves(tr[0]) > 3, "max_leaves=0 imposes no cap"

    def capped3(tr):
        assert _leaves(tr[0]) == 3

    add("lossguide_zero_cap_unlimited", x32, y32, _p(max_leaves=0), uncapped)
    add("lossguide_cap_3", x32, y32, _p(max_leaves=3), capped3)

    def depths(tr):
        t = tr[0]
        assert _leaves(t) == 4
        assert not _split(t, 1), "shallower, lower-gain candidate"
        assert _split(t, 3), "deeper, higher-gain candidate"

    add("lossguide_across_depths", X8, y_gain, _p(max_leaves=4), depths)

    # tests/max_leaves.rs: depthwise, lambda 1, base score 1.5, max_depth 6.
    def mp(**kw):
        return _p(grow_policy="depthwise", **{"lambda": 1.0, "base_score": 1.5, "max_depth": 6,
                                             **kw})

    add("depthwise_cap_1", SEPARABLE, y_tie, mp(max_leaves=1), root_only)

    def cap2(tr):
        t = tr[0]
        assert _leaves(t) == 2 and _split(t, 0) and not _split(t, 1) and not _split(t, 2)

    add("depthwise_cap_2", SEPARABLE, y_tie, mp(max_leaves=2), cap2)

    def cap3(tr):
        t = tr[0]
        assert _leaves(t) == 3 and _split(t, 0)
        assert _split(t, 1), "the left depth-one node is split first"
        assert not _split(t, 2), "the right depth-one node stays a leaf"

    add("depthwise_cap_3_node_order", SEPARABLE, y_tie, mp(max_leaves=3), cap3)

    def depth1(tr):
        t = tr[0]
        assert _leaves(t) == 2 and not _split(t, 1) and not _split(t, 2)

    add("depthwise_depth_limit_first", SEPARABLE, y_tie, mp(max_leaves=3, max_depth=1), depth1)
    add("depthwise_depth0", SEPARABLE, y_tie, mp(max_leaves=8, max_depth=0), root_only)
    def every_round(tr):
        assert len(tr) == 4 and all(_leaves(t) <= 3 for t in tr)

    add("depthwise_every_round_capped", SEPARABLE, y_tie, mp(max_leaves=3, n_rounds=4),
        every_round)

    def terminal(tr):
        t = tr[0]
        assert _leaves(t) <= 3
        assert not _split(t, 1) and _split(t, 2), "the terminal left branch counts toward the cap"

    add("depthwise_terminal_branch_counts", X8, [0., 0., 0., 0., 10., 10., 11., 12.],
        mp(max_leaves=3, max_depth=8, **{"lambda": 0.0}), terminal)
    return out


def unlimited_equals_nonbinding():
    """tests/max_leaves.rs:108-124: max_leaves 0 and 64 grow the same trees."""
    return (SEPARABLE.reshape(-1, 1), np.array([0., 0., 1., 1., 3., 3., 4., 4.], np.float32),
            {"n_rounds": 3, "max_bin": 16, "eta": 0.3, "lambda": 1.0, "min_child_weight": 0.0,
             "objective": "reg:squarederror", "base_score": 1.5, "grow_policy": "depthwise",
             "max_depth": 6})
