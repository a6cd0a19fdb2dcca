"""CPU: the Parquet / Arrow row reader behind train()'s file and table inputs
(python/ferrisboost/__init__.py:1090-1230; the reference reads Parquet in
src/source/parquet_source.rs): feature columns in schema order without the
label and weight, nulls as NaN, integer / boolean / dictionary columns as
float32, the missing value, several row groups read front to back in
arbitrary chunk sizes and read again from the start, and the input errors."""

from __future__ import annotations

import numpy as np
import pytest

pa = pytest.importorskip("pyarrow")
pq = pytest.importorskip("pyarrow.parquet")

from ferrisboost_amd import arrow_rows  # noqa: E402


def _table(n=5000, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, 3)).astype(np.float32)
    x[rng.random((n, 3)) < 0.1] = np.nan
    cols = {f"f{j}": pa.array(x[:, j], mask=np.isnan(x[:, j])) for j in range(3)}
    ints = rng.integers(-5, 50, n).astype(np.int64)
    cols["count"] = pa.array(ints, mask=rng.random(n) < 0.05)
    cols["flag"] = pa.array(rng.random(n) < 0.3)
    cols["y"] = pa.array(rng.standard_normal(n).astype(np.float32))
    cols["w"] = pa.array(rng.uniform(0.5, 2.0, n).astype(np.float32))
    codes = rng.integers(0, 4, n)
    cols["city"] = pa.DictionaryArray.from_arrays(pa.array(codes.astype(np.int32)),
                                                  pa.array(["a", "b", "c", "d"]))
    t = pa.table(cols)
    want = np.column_stack([
        x,
        np.where(t.column("count").is_null().to_numpy(zero_copy_only=False), np.nan,
                 ints).astype(np.float32),
        t.column("flag").to_numpy().astype(np.float32),
        codes.astype(np.float32),
    ]).astype(np.float32)
    return t, want


def _read_all(src, step):
    out = np.empty((src.n_rows, src.n_features), np.float32)
    for b in range(0, src.n_rows, step):
        k = min(step, src.n_rows - b)
        src.read(b, k, out[b:b + k])
    return out


@pytest.mark.parametrize("step", [1, 999, 4096, 5000])
def test_parquet_rows_in_any_chunking(tmp_path, step):
    t, want = _table()
    path = tmp_path / "d.parquet"
    pq.write_table(t, path, row_group_size=1700)
    src = arrow_rows.ArrowRows(path, "y", "w", True, float("nan"), batch_rows=777)
    assert src.features == ["f0", "f1", "f2", "count", "flag", "city"]
    assert src.categorical.tolist() == [0, 0, 0, 0, 0, 1]
    assert np.array_equal(src.labels, t.column("y").to_numpy())
    assert np.array_equal(src.weights, t.column("w").to_numpy())
    got = _read_all(src, step)
    assert np.array_equal(got, want, equal_nan=True)
    # a second pass starts the file again
    assert np.array_equal(_read_all(src, 2048), want, equal_nan=True)


def test_tables_and_batch_readers_read_the_same_rows():
    t, want = _table(seed=1)
    for data in (t, pa.RecordBatchReader.from_batches(t.schema, t.to_batches(max_chunksize=600))):
        src = arrow_rows.ArrowRows(data, "y", None, True, float("nan"))
        assert "w" in src.features and src.weights is None
        cols = src.features
        got = _read_all(src, 1234)
        assert np.array_equal(got[:, cols.index("f1")], want[:, 1], equal_nan=True)


def test_the_missing_value_becomes_nan():
    t = pa.table({"a": pa.array(np.array([1, -999, 3, -999], np.float32)),
                  "y": pa.array(np.zeros(4, np.float32))})
    src = arrow_rows.ArrowRows(t, "y", None, False, -999.0)
    got = _read_all(src, 4)
    assert np.isnan(got[[1, 3], 0]).all() and got[[0, 2], 0].tolist() == [1.0, 3.0]


def test_input_errors(tmp_path):
    t, _ = _table(n=100)
    with pytest.raises(ValueError, match="enable_categorical"):
        src = arrow_rows.ArrowRows(t, "y", None, False, float("nan"))
        _read_all(src, 100)
    with pytest.raises(ValueError, match="label column 'nope'"):
        arrow_rows.ArrowRows(t, "nope", None, True, float("nan"))
    with pytest.raises(ValueError, match="names the label column"):
        arrow_rows.ArrowRows(t, np.zeros(100), None, True, float("nan"))
    bad = t.append_column("name", pa.array(["x"] * 100))
    with pytest.raises(ValueError, match="must be numeric"):
        src = arrow_rows.ArrowRows(bad, "y", None, True, float("nan"))
        _read_all(src, 100)
    holes = pa.table({"a": pa.array([1.0, 2.0]), "y": pa.array([1.0, None])})
    with pytest.raises(ValueError, match="missing values"):
        arrow_rows.ArrowRows(holes, "y", None, False, float("nan"))


def test_train_rejects_unknown_file_types(tmp_path):
    import ferrisboost_amd as fb

    with pytest.raises(ValueError, match="cannot tell the format"):
        fb.train({}, str(tmp_path / "d.csv"), "y")
