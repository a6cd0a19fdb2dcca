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
dictionary columns are categorical codes when enable_categorical is set.
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


def _column_f32(col, name: str, categorical: bool) -> np.ndarray:
    """One Arrow column as float32 values, nulls as NaN."""
    pa, pc = _pa()
    if isinstance(col, pa.ChunkedArray):
        col = col.combine_chunks()
    if pa.types.is_dictionary(col.type):
        if not categorical:
            raise ValueError(f"column {name!r} is a dictionary (categorical) column; set "
                             "params['enable_categorical'] = True to train on its codes")
        col = col.indices
    t = col.type
    if not (pa.types.is_integer(t) or pa.types.is_floating(t) or pa.types.is_boolean(t)):
        raise ValueError(f"column {name!r} has type {t}; feature columns must be numeric, "
                         "boolean or dictionary-encoded")
    return pc.cast(col, pa.float32()).to_numpy(zero_copy_only=False).astype(np.float32, copy=False)


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
        if not isinstance(label, str):
            raise ValueError("for Parquet and Arrow inputs, label names the label column")
        for col, what in ((label, "label"), (weight, "weight")):
            if col is not None and col not in names:
                raise ValueError(f"{what} column {col!r} is not in the data (columns: "
                                 f"{', '.join(names)})")
        excluded = {label} | ({weight} if weight is not None else set())
        self.features: list[str] = [c for c in names if c not in excluded]
        if not self.features:
            raise ValueError("the data has no feature columns besides the label")
        self.categorical = np.array(
            [1 if pa.types.is_dictionary(schema.field(c).type) else 0 for c in self.features],
            np.uint8)
        self._cat_ok = bool(enable_categorical)
        self._missing = np.float32(missing)
        self._batch_rows = int(batch_rows)
        self._it: Iterator | None = None
        self._cur: np.ndarray | None = None
        self._cur_start = 0
        self._cur_end = 0
        self.labels = self._whole(label, "label")
        if np.isnan(self.labels).any():
            raise ValueError(f"label column {label!r} has missing values")
        self.weights = None if weight is None else self._whole(weight, "weight")

    @property
    def n_features(self) -> int:
        return len(self.features)

    def _whole(self, name: str, what: str) -> np.ndarray:
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
        cols = [_column_f32(batch.column(j), self.features[j], self._cat_ok)
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


def feature_types_of(src: ArrowRows, given: Sequence[str] | None) -> list[str] | None:
    """feature_types for the source's features: the given list, else "c" for
    dictionary columns (None when every feature is numeric)."""
    if given is not None:
        if len(given) != src.n_features:
            raise ValueError(f"feature_types has {len(given)} entries for {src.n_features} "
                             "feature columns")
        return list(given)
    if src.categorical.any():
        return ["c" if c else "q" for c in src.categorical]
    return None
