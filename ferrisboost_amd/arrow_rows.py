"""Row readers over Parquet files and Arrow tables for train().

The reference reads Parquet column chunks with its own Rust reader and bins
them without building a float matrix in Python (src/source/parquet_source.rs,
src/source/arrow_source.rs; python/ferrisboost/__init__.py:1090-1230 names
the file and table entries). Here pyarrow decodes the row groups, and the
training call pulls row-major float32 chunks through fbt_train_rows, front to
back, once for the sketch and once for the binning: the host never holds the
whole matrix unless a host pass needs it (weighted rows, host binning).

Feature columns are every column except the label (and weight) columns, in
schema order. Numeric and boolean columns become float32 (nulls are missing);
numeric dictionary columns yield their values; string dictionary and string
columns are categorical features when enable_categorical is set, coded in the
order their values first appear in the rows, one list per feature for the
whole source (src/source/cat_recode.rs:1-30).
"""

from __future__ import annotations

import os
from typing import Callable, Iterator, Sequence

import numpy as np


def _pa():
    try:
        import pyarrow as pa
        import pyarrow.compute as pc
    except ImportError as e:  # pragma: no cover - pyarrow ships with the image
        raise ValueError("Parquet and Arrow inputs need pyarrow") from e
    return pa, pc


def is_path(data) -> bool:
    return isinstance(data, (str, os.PathLike))


# Largest category code a categorical feature holds (MAX_CAT_CODE_WIDE,
# src/data/categorical.rs): codes 0..=65533, so at most 65534 categories.
MAX_CATEGORIES = 65534


def _is_string(t) -> bool:
    pa, _ = _pa()
    return pa.types.is_string(t) or pa.types.is_large_string(t) or (
        hasattr(pa.types, "is_string_view") and pa.types.is_string_view(t))


def _named(t) -> bool:
    """A column type that carries category names: a string dictionary or a
    plain string column (cat_recode::is_named, src/source/cat_recode.rs:55-61)."""
    pa, _ = _pa()
    if pa.types.is_dictionary(t):
        return _is_string(t.value_type)
    return _is_string(t)


class CategoryCoder:
    """One feature's category names -> codes (cat_recode::Recoder,
    src/source/cat_recode.rs:1-30).

    Learning (training): a value gets the next code when a row first holds
    it, so the list is the column's first-appearance order whatever the
    dictionaries of the chunks and row groups list or in which order (the
    reference's pass 1); reading the same rows again gives the same codes.
    Fixed (prediction): values are looked up in a trained list, and a row
    holding a value outside it is an input error."""

    def __init__(self, values: Sequence[str] | None = None):
        self.learning = values is None
        self.values: list[str] = [] if values is None else list(values)
        self.index = {v: i for i, v in enumerate(self.values)}
        if len(self.index) != len(self.values):
            raise ValueError("duplicate category in a category list")

    def codes(self, col, name: str) -> np.ndarray:
        """float32 codes of a string dictionary / string column, nulls NaN."""
        pa, pc = _pa()
        if not pa.types.is_dictionary(col.type):
            col = pc.dictionary_encode(col)
        idx = col.indices.to_numpy(zero_copy_only=False)
        valid = ~np.asarray(col.is_null().to_numpy(zero_copy_only=False), bool)
        idx = np.where(valid, idx, -1).astype(np.int64)
        entries = col.dictionary.to_pylist()
        lut = np.full(len(entries), -1, np.int64)
        used = idx[valid]
        if used.size:
            # dictionary entries in the order rows first use them
            u, first = np.unique(used, return_index=True)
            for d in u[np.argsort(first, kind="stable")]:
                v = entries[int(d)]
                if v is None:
                    raise ValueError(f"column {name!r}: a dictionary entry is null; categories "
                                     "must be values")
                code = self.index.get(v)
                if code is None:
                    if not self.learning:
                        raise ValueError(f"column {name!r} holds the category {v!r}, which is not "
                                         "in the training categories (categories unseen in "
                                         "training are rejected, as in XGBoost)")
                    if len(self.values) >= MAX_CATEGORIES:
                        raise ValueError(f"column {name!r} has more than {MAX_CATEGORIES} "
                                         "categories")
                    code = len(self.values)
                    self.values.append(v)
                    self.index[v] = code
                lut[d] = code
        out = np.full(idx.size, np.nan, np.float32)
        out[valid] = lut[idx[valid]].astype(np.float32)
        return out


def _column_f32(col, name: str, categorical: bool,
                coder: CategoryCoder | None = None) -> np.ndarray:
    """One Arrow column as float32 values, nulls as NaN.

    A numeric dictionary column yields its decoded values
    (arrow_source::visit_column_f32, src/source/arrow_source.rs:126-145); a
    string dictionary or string column of a categorical feature goes through
    the feature's category coder."""
    pa, pc = _pa()
    if isinstance(col, pa.ChunkedArray):
        col = col.combine_chunks()
    t = col.type
    if _named(t):
        if not categorical or coder is None:
            if pa.types.is_dictionary(t):
                raise ValueError(f"column {name!r} is a dictionary (categorical) column; set "
                                 "params['enable_categorical'] = True to train on its categories")
            raise ValueError(f"column {name!r} has type {t}; feature columns must be numeric, "
                             "boolean or dictionary-encoded")
        return coder.codes(col, name)
    if pa.types.is_dictionary(t):
        if not (pa.types.is_integer(t.value_type) or pa.types.is_floating(t.value_type)):
            raise ValueError(f"column {name!r} is a dictionary of {t.value_type} values; "
                             "categories must be strings or integers")
        col = col.dictionary_decode()
        t = col.type
    if not (pa.types.is_integer(t) or pa.types.is_floating(t) or pa.types.is_boolean(t)):
        raise ValueError(f"column {name!r} has type {t}; feature columns must be numeric, "
                         "boolean or dictionary-encoded")
    return pc.cast(col, pa.float32()).to_numpy(zero_copy_only=False).astype(np.float32, copy=False)


def table_matrix(table, names: Sequence[str] | None, categories: Sequence | None,
                 n_features: int, missing: float) -> np.ndarray:
    """A pyarrow Table as the float32 matrix predict() scores: columns
    selected and ordered by the model's feature names when it has them, and
    named categories re-coded by value onto the model's lists (unknown
    values are an error; python/ferrisboost/__init__.py:925-975)."""
    pa, _ = _pa()
    if isinstance(table, pa.RecordBatch):
        table = pa.Table.from_batches([table])
    if names:
        absent = [c for c in names if c not in table.column_names]
        if absent:
            raise ValueError(f"predict data is missing the model's feature columns {absent}")
        table = table.select(list(names))
    if table.num_columns != n_features:
        raise ValueError(f"expected {n_features} feature columns, got {table.num_columns}")
    cols = []
    for j in range(table.num_columns):
        cats = categories[j] if categories else None
        coder = CategoryCoder(cats) if cats is not None else None
        name = table.column_names[j]
        cols.append(_column_f32(table.column(j), name, coder is not None, coder))
    X = np.stack(cols, axis=1) if cols else np.zeros((table.num_rows, 0), np.float32)
    miss = np.float32(missing)
    if not np.isnan(miss):
        X[X == miss] = np.nan
    return np.ascontiguousarray(X, np.float32)


class ArrowRows:
    """Row-major float32 chunks of the feature columns of a Parquet file or
    an Arrow table, served front to back (a read before the last position
    starts the source again)."""

    def __init__(self, data, label: str, weight: str | None, enable_categorical: bool,
                 missing: float, batch_rows: int = 1 << 16):
        pa, _ = _pa()
        if is_path(data):
            import pyarrow.parquet as pq

            self._file = pq.ParquetFile(os.fspath(data))
            schema = self._file.schema_arrow
            self.n_rows = self._file.metadata.num_rows
            self._table = None
        else:
            table = data
            if isinstance(table, pa.RecordBatchReader):
                table = table.read_all()  # one pass only: held as a table for the two passes
            if not isinstance(table, pa.Table):
                raise ValueError("data must be a numpy array, a pyarrow Table or "
                                 "RecordBatchReader, or a .parquet path")
            self._file = None
            self._table = table
            schema = table.schema
            self.n_rows = table.num_rows
        names = list(schema.names)
        # A table takes the label and weight as arrays too (every column is
        # then a feature); a file names them.
        label_col = label if isinstance(label, str) else None
        weight_col = weight if isinstance(weight, str) else None
        if label_col is None and self._file is not None:
            raise ValueError("for Parquet inputs, label names the label column")
        if weight is not None and weight_col is None and self._file is not None:
            raise ValueError("for Parquet inputs, weight names the weight column")
        for col, what in ((label_col, "label"), (weight_col, "weight")):
            if col is not None and col not in names:
                raise ValueError(f"{what} column {col!r} is not in the data (columns: "
                                 f"{', '.join(names)})")
        excluded = {label_col, weight_col} - {None}
        self.features: list[str] = [c for c in names if c not in excluded]
        if not self.features:
            raise ValueError("the data has no feature columns besides the label")
        types = [schema.field(c).type for c in self.features]
        self.categorical = np.array(
            [1 if (pa.types.is_dictionary(t) or _named(t)) else 0 for t in types], np.uint8)
        self._cat_ok = bool(enable_categorical)
        # one learning coder per named feature, kept across both passes
        self.coders: list[CategoryCoder | None] = [
            CategoryCoder() if (self._cat_ok and _named(t)) else None for t in types]
        self._missing = np.float32(missing)
        self._batch_rows = int(batch_rows)
        self._it: Iterator | None = None
        self._cur: np.ndarray | None = None
        self._cur_start = 0
        self._cur_end = 0
        self.labels = self._whole(label_col) if label_col is not None else self._given(label,
                                                                                      "label")
        if np.isnan(self.labels).any():
            raise ValueError(f"label column {label!r} has missing values" if label_col else
                             "label has missing values")
        self.weights = (None if weight is None else self._whole(weight_col)
                        if weight_col is not None else self._given(weight, "weight"))

    def _given(self, values, what: str) -> np.ndarray:
        a = np.ascontiguousarray(np.asarray(values, dtype=np.float32).reshape(-1))
        if a.shape != (self.n_rows,):
            raise ValueError(f"{what} has {a.size} rows, but the training data has "
                             f"{self.n_rows} rows")
        return a

    @property
    def n_features(self) -> int:
        return len(self.features)

    def _whole(self, name: str) -> np.ndarray:
        if self._file is not None:
            col = self._file.read(columns=[name]).column(0)
        else:
            col = self._table.column(name)
        return np.ascontiguousarray(_column_f32(col, name, False))

    def _batches(self) -> Iterator:
        if self._file is not None:
            return self._file.iter_batches(batch_size=self._batch_rows, columns=self.features)
        return iter(self._table.select(self.features).to_batches(max_chunksize=self._batch_rows))

    def _rows_of(self, batch) -> np.ndarray:
        cols = [_column_f32(batch.column(j), self.features[j], self._cat_ok, self.coders[j])
                for j in range(batch.num_columns)]
        rows = np.stack(cols, axis=1) if cols else np.zeros((batch.num_rows, 0), np.float32)
        if not np.isnan(self._missing):
            rows[rows == self._missing] = np.nan
        return np.ascontiguousarray(rows, np.float32)

    def read(self, begin: int, count: int, out: np.ndarray) -> None:
        """Fill out ([count, n_features]) with rows begin .. begin + count."""
        if self._it is None or begin < self._cur_start:
            self._it = self._batches()
            self._cur, self._cur_start, self._cur_end = None, 0, 0
        filled = 0
        while filled < count:
            row = begin + filled
            while row >= self._cur_end:
                batch = next(self._it, None)
                if batch is None:
                    raise ValueError(f"the data ended at row {self._cur_end}, before row {row}")
                self._cur = self._rows_of(batch)
                self._cur_start, self._cur_end = self._cur_end, self._cur_end + batch.num_rows
            take = min(count - filled, self._cur_end - row)
            a = row - self._cur_start
            out[filled:filled + take] = self._cur[a:a + take]
            filled += take

    def as_callback(self, errors: list) -> Callable:
        """The fbt_rows_fn for this source; an exception is kept in errors
        and the call reports failure."""
        from . import _native as N

        nf = self.n_features

        def fn(_user, begin, count, ptr):
            try:
                out = np.ctypeslib.as_array(ptr, shape=(int(count) * nf,)).reshape(int(count), nf)
                self.read(int(begin), int(count), out)
                return 0
            except BaseException as e:  # reported after the call returns
                errors.append(e)
                return 1

        return N.ROWS_FN(fn)


def categories_of(src: ArrowRows, types: Sequence[str] | None) -> list | None:
    """The learned category lists by feature (None for a feature without
    names), or None when no categorical feature has names."""
    cats = [c.values if (c is not None and (types is None or types[j] == "c")) else None
            for j, c in enumerate(src.coders)]
    return cats if any(c is not None for c in cats) else None


def feature_types_of(src: ArrowRows, given: Sequence[str] | None) -> list[str] | None:
    """feature_types for the source's features: the given list, else "c" for
    dictionary columns (None when every feature is numeric)."""
    if given is not None:
        if len(given) != src.n_features:
            raise ValueError(f"feature_types has {len(given)} entries for {src.n_features} "
                             "feature columns")
        for j, t in enumerate(given):
            if t != "c" and src.coders[j] is not None:
                raise ValueError(f"column {src.features[j]!r} holds category names, which can "
                                 "only be a categorical feature (do not declare it \"q\" in "
                                 "feature_types)")
        return list(given)
    if src.categorical.any():
        return ["c" if c else "q" for c in src.categorical]
    return None
