"""CPU: pandas DataFrame inputs of train() and Model.predict()
(python/ferrisboost/__init__.py:725-797, 923-962 name the conversion):
numeric and boolean columns as float32 with missing values NaN, `category`
columns as their positions in `categories` (NaN for a missing value) that
need enable_categorical, string and integer category lists, prediction data
bound by column name and re-coded by category value, and the input errors."""

from __future__ import annotations

import numpy as np
import pytest

pd = pytest.importorskip("pandas")

from ferrisboost_amd import frame_rows  # noqa: E402


def _frame(n=400, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, 2)).astype(np.float32)
    x[rng.random((n, 2)) < 0.1] = np.nan
    city = rng.integers(0, 4, n)
    size = rng.integers(0, 3, n)
    df = pd.DataFrame({
        "a": x[:, 0],
        "city": pd.Categorical.from_codes(np.where(rng.random(n) < 0.05, -1, city),
                                          ["rome", "oslo", "lima", "kyiv"]),
        "n": pd.array(rng.integers(-3, 9, n), dtype="Int64"),
        "flag": rng.random(n) < 0.3,
        "size": pd.Categorical.from_codes(size, [10, 20, 40]),
        "b": x[:, 1].astype(np.float64),
    })
    df.loc[rng.random(n) < 0.05, "n"] = pd.NA
    return df


def test_columns_become_float32_and_codes():
    df = _frame()
    X, names, flags, lists = frame_rows.frame_matrix(df, True)
    assert X.dtype == np.float32 and X.shape == (len(df), 6) and X.flags.c_contiguous
    assert names == ["a", "city", "n", "flag", "size", "b"]
    assert flags == [False, True, False, False, True, False]
    assert lists[1] == ["rome", "oslo", "lima", "kyiv"] and lists[4] == [10, 20, 40]
    assert lists[0] is None and lists[2] is None
    codes = df["city"].cat.codes.to_numpy()
    assert np.array_equal(np.isnan(X[:, 1]), codes < 0)
    assert np.array_equal(X[codes >= 0, 1], codes[codes >= 0].astype(np.float32))
    # integer categories train on their codes, not their values
    assert np.array_equal(X[:, 4], df["size"].cat.codes.to_numpy().astype(np.float32))
    na = df["n"].isna().to_numpy()
    assert np.array_equal(np.isnan(X[:, 2]), na)
    assert np.array_equal(X[~na, 2], df["n"].to_numpy()[~na].astype(np.float32))
    assert np.array_equal(X[:, 3], df["flag"].to_numpy().astype(np.float32))
    assert np.array_equal(X[:, 5], df["b"].to_numpy().astype(np.float32), equal_nan=True)


def test_prediction_recodes_by_value_and_binds_by_name():
    df = _frame(seed=1)
    X, names, _, lists = frame_rows.frame_matrix(df, True)
    # the same rows with the categories listed in another order and the
    # columns shuffled, plus a column the model does not use
    shuffled = df.assign(city=df["city"].cat.reorder_categories(["kyiv", "lima", "oslo", "rome"]),
                         size=df["size"].cat.reorder_categories([40, 10, 20]),
                         extra=1.0)[["extra", "b", "size", "flag", "n", "city", "a"]]
    sel = frame_rows.select_columns(shuffled, names)
    X2 = frame_rows.frame_matrix(sel, True, lists, what="predict data", scoring=True)[0]
    assert np.array_equal(X2, X, equal_nan=True)
    # a plain integer column of a feature with integer categories is looked
    # up by value
    plain = sel.assign(size=df["size"].astype(np.int64))
    X3 = frame_rows.frame_matrix(plain, True, lists, what="predict data", scoring=True,
                                 categorical=[False, True, False, False, True, False])[0]
    assert np.array_equal(X3, X, equal_nan=True)
    # without a training list, integer categories yield their values and
    # string categories their codes
    X4 = frame_rows.frame_matrix(df, True, None, scoring=True)[0]
    assert np.array_equal(X4[:, 4], df["size"].astype(np.int64).to_numpy().astype(np.float32))
    assert np.array_equal(X4[:, 1], X[:, 1], equal_nan=True)


def test_input_errors():
    df = _frame(n=50, seed=2)
    with pytest.raises(ValueError, match="enable_categorical"):
        frame_rows.frame_matrix(df, False)
    _, names, _, lists = frame_rows.frame_matrix(df, True)
    unseen = df.assign(city=pd.Categorical(["paris"] * len(df)))
    with pytest.raises(ValueError, match="'paris', which is not in the training categories"):
        frame_rows.frame_matrix(unseen, True, lists, scoring=True)
    wrong_kind = df.assign(size=df["size"].cat.rename_categories(str))
    with pytest.raises(ValueError, match="training categories are integers"):
        frame_rows.frame_matrix(wrong_kind, True, lists, scoring=True)
    with pytest.raises(ValueError, match="missing the model's feature columns"):
        frame_rows.select_columns(df.drop(columns=["b"]), names)
    with pytest.raises(ValueError, match="not a numeric feature"):
        frame_rows.frame_matrix(df.assign(s=["x"] * len(df)), True)
    with pytest.raises(ValueError, match="duplicate column names"):
        frame_rows.frame_matrix(pd.concat([df["a"], df["a"]], axis=1), True)
    with pytest.raises(ValueError, match="strings or integers"):
        frame_rows.frame_matrix(df.assign(f=pd.Categorical([0.5] * len(df))), True)
    plain = df.assign(size=np.full(len(df), 30, np.int64))
    with pytest.raises(ValueError, match="category 30"):
        frame_rows.frame_matrix(plain, True, lists, scoring=True,
                                categorical=[False, True, False, False, True, False])


def test_frames_are_told_from_other_inputs():
    assert frame_rows.is_frame(_frame(n=3))
    assert not frame_rows.is_frame(np.zeros((3, 2)))
    assert not frame_rows.is_frame(_frame(n=3)["a"])


def test_monotone_constraints_by_column_name():
    from ferrisboost_amd import _monotone

    names = ["a", "city", "b"]
    assert _monotone({"b": -1, "a": 3}, names).tolist() == [1, 0, -1]
    assert _monotone("(1,0,-1)", None).tolist() == [1, 0, -1]
    assert _monotone((0, -2), None).tolist() == [0, -1]
    assert _monotone(None, names) is None
    with pytest.raises(ValueError, match="needs column names"):
        _monotone({"a": 1}, None)
    with pytest.raises(ValueError, match=r"\['z'\] are not feature columns"):
        _monotone({"z": 1}, names)
