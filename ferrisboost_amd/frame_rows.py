"""pandas DataFrame inputs for train() and Model.predict().

A DataFrame is read column by column into the float32 row-major matrix the
array path takes (python/ferrisboost/__init__.py:725-797 names the same
conversion): numeric and boolean columns become float32 with missing values
as NaN; a `category` column is a categorical feature (enable_categorical
must be set to train one) whose code is the value's position in the column's
`categories`, NaN for a missing value. Column names become the model's
feature names, and the category lists are kept by feature so that prediction
data can list its categories in another order: predict() selects the model's
columns by name and re-codes every category column by value onto the
training codes (python/ferrisboost/__init__.py:923-962). A category outside
the training list is an error.

Categories are strings or integers, nothing else. When a prediction column
has no training list to re-code against, an integer `category` column yields
its values and a string one its codes, as a file's dictionary column is read;
a plain integer column of a categorical feature whose training categories are
integers is looked up by value.
"""

from __future__ import annotations

from typing import Sequence

import numpy as np


def is_frame(data) -> bool:
    mod = type(data).__module__ or ""
    return mod.startswith("pandas") and type(data).__name__ == "DataFrame"


def _category_list(categories, where: str) -> list:
    """A pandas categories Index -> a list of str or a list of int."""
    import pandas as pd

    if pd.api.types.is_integer_dtype(categories.dtype):
        return [int(v) for v in categories]
    values = list(categories)
    if all(isinstance(v, str) for v in values):
        return values
    raise ValueError(f"{where}: categories must be strings or integers, got {categories.dtype} "
                     "categories; convert them, e.g. with .cat.rename_categories(str)")


def _is_str_list(values: Sequence) -> bool:
    return all(isinstance(v, str) for v in values)


def _codes_f32(codes: np.ndarray) -> np.ndarray:
    out = codes.astype(np.float32)
    out[codes < 0] = np.float32("nan")
    return out


def _recode(codes: np.ndarray, values: list, ref: list, where: str) -> np.ndarray:
    """Codes into `values` (-1 missing) -> codes into the training list `ref`."""
    if values and ref and _is_str_list(values) != _is_str_list(ref):
        theirs = "strings" if _is_str_list(values) else "integers"
        ours = "strings" if _is_str_list(ref) else "integers"
        raise ValueError(f"{where}: its categories are {theirs}, the training categories are "
                         f"{ours}; the category type must match the training data")
    pos = {v: i for i, v in enumerate(ref)}
    table = np.array([pos.get(v, -1) for v in values] + [-1], np.int64)
    out = table[codes]  # code -1 picks the trailing -1
    unseen = (codes >= 0) & (out < 0)
    if unseen.any():
        v = values[int(codes[np.argmax(unseen)])]
        raise ValueError(f"{where} holds the category {v!r}, which is not in the training "
                         "categories (a category unseen in training is an error)")
    return out


def _lookup_values(values: np.ndarray, na: np.ndarray, ref: list, where: str) -> np.ndarray:
    """Plain integer values -> codes by position in an integer category list."""
    refv = np.asarray(ref, np.int64)
    order = np.argsort(refv, kind="stable")
    srt = refv[order]
    big = values > np.iinfo(np.int64).max if values.dtype.kind == "u" else np.zeros(values.shape,
                                                                                      bool)
    v = values.astype(np.int64)
    pos = np.minimum(np.searchsorted(srt, v), len(srt) - 1)
    hit = (srt[pos] == v) & ~big
    codes = np.full(values.shape, -1, np.int64)
    codes[hit] = order[pos[hit]]
    unseen = ~na & (codes < 0)
    if unseen.any():
        raise ValueError(f"{where} holds the category {int(values[np.argmax(unseen)])!r}, which "
                         "is not in the training categories (a category unseen in training is "
                         "an error)")
    return codes


def frame_matrix(df, enable_categorical: bool, refs: Sequence | None = None,
                 what: str = "data", scoring: bool = False,
                 categorical: Sequence[bool] | None = None):
    """DataFrame -> (float32 matrix, column names, categorical flags, category
    lists by column: a list for a `category` column, else None).

    refs (training category lists by column, None where a column has none)
    re-code category columns by value; scoring reads columns the way
    prediction data is read (module docstring). categorical (the model's
    flags) limits the by-value lookup of plain integer columns to
    categorical features."""
    import pandas as pd

    names = [str(c) for c in df.columns]
    if len(set(names)) != len(names):
        dups = sorted({n for n in names if names.count(n) > 1})
        raise ValueError(f"{what} has duplicate column names {dups}; column names must be unique")
    n = len(df)
    X = np.empty((n, len(names)), np.float32)
    flags: list[bool] = []
    lists: list = []
    for j, name in enumerate(names):
        s = df.iloc[:, j]
        where = f"{what} column {name!r}"
        ref = refs[j] if refs is not None and j < len(refs) else None
        if isinstance(s.dtype, pd.CategoricalDtype):
            if not enable_categorical:
                raise ValueError(f"{where} has category dtype; to train it as a categorical "
                                 "feature, set params['enable_categorical'] = True")
            values = _category_list(s.cat.categories, where)
            codes = np.asarray(s.cat.codes.to_numpy(), np.int64)
            if ref is not None:
                codes = _recode(codes, values, list(ref), where)
                X[:, j] = _codes_f32(codes)
                lists.append(list(ref))
            elif scoring and values and not _is_str_list(values):
                col = np.append(np.asarray(values, np.float64), np.nan)
                X[:, j] = col[codes].astype(np.float32)
                lists.append(None)
            else:
                X[:, j] = _codes_f32(codes)
                lists.append(values)
            flags.append(True)
            continue
        int_ref = (ref is not None and len(ref) > 0 and not _is_str_list(ref)
                   and (categorical is None or (j < len(categorical) and categorical[j])))
        if scoring and int_ref and pd.api.types.is_integer_dtype(s.dtype):
            na = np.asarray(s.isna().to_numpy(), bool)
            kind = np.dtype(getattr(s.dtype, "numpy_dtype", s.dtype)).kind
            vals = s.to_numpy(dtype=np.uint64 if kind == "u" else np.int64, na_value=0)
            X[:, j] = _codes_f32(_lookup_values(vals, na, list(ref), where))
            flags.append(True)
            lists.append(list(ref))
            continue
        try:
            X[:, j] = s.to_numpy(dtype=np.float32, na_value=np.nan)
        except (TypeError, ValueError) as e:
            raise ValueError(f"{where} has dtype {s.dtype}, which is not a numeric feature; "
                             "convert it to numeric, or to category and set "
                             "enable_categorical=True") from e
        flags.append(False)
        lists.append(None)
    return X, names, flags, lists


def select_columns(df, names: Sequence[str] | None, what: str = "predict data"):
    """The model's feature columns of df, in the model's order (extra columns
    are ignored, a missing one is an error); df unchanged without names."""
    if not names:
        return df
    cols = [str(c) for c in df.columns]
    absent = [n for n in names if n not in cols]
    if absent:
        raise ValueError(f"{what} is missing the model's feature columns {absent}")
    return df[[c for n in names for c in df.columns if str(c) == n]]
