"""CPU: the Parquet / Arrow row reader behind train()'s file and table inputs
(python/ferrisboost/__init__.py:1090-1230; the reference reads Parquet in
src/source/parquet_source.rs): feature columns in schema order without the
label and weight, nulls as NaN, integer / boolean columns as float32,
string dictionaries and string columns as categories coded in row order,
numeric dictionaries as their values, the missing value, several row groups read front to back in
arbitrary chunk sizes and read again from the start, and the input errors."""

from __future__ import annotations

import numpy as np
import pytest

pa = pytest.importorskip("pyarrow")
pq = pytest.importorskip("pyarrow.parquet")

from ferrisboost_amd import arrow_rows  # noqa: E402


def first_appearance_codes(codes):
    """Codes renumbered in the order the rows first use them (the order
    named categories are coded in)."""
    u, first = np.unique(codes, return_index=True)
    remap = np.empty(u.max() + 1, np.int64)
    remap[u[np.argsort(first)]] = np.arange(u.size)
    return remap[codes]


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
        first_appearance_codes(codes).astype(np.float32),
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
    with pytest.raises(ValueError, match="label has 99 rows"):
        arrow_rows.ArrowRows(t, np.zeros(99), None, True, float("nan"))
    path = tmp_path / "t.parquet"
    pq.write_table(t, path)
    with pytest.raises(ValueError, match="names the label column"):
        arrow_rows.ArrowRows(path, np.zeros(100), None, True, float("nan"))
    bad = t.append_column("name", pa.array(["x"] * 100))
    with pytest.raises(ValueError, match="must be numeric"):
        src = arrow_rows.ArrowRows(bad.drop(["city"]), "y", None, False, float("nan"))
        _read_all(src, 100)
    src = arrow_rows.ArrowRows(bad, "y", None, True, float("nan"))
    with pytest.raises(ValueError, match="holds category names"):
        arrow_rows.feature_types_of(src, ["q"] * src.n_features)
    floats = t.append_column("fd", pa.DictionaryArray.from_arrays(
        pa.array(np.zeros(100, np.int32)), pa.array([True])))
    with pytest.raises(ValueError, match="categories must be strings or integers"):
        src = arrow_rows.ArrowRows(floats, "y", None, True, float("nan"))
        _read_all(src, 100)
    holes = pa.table({"a": pa.array([1.0, 2.0]), "y": pa.array([1.0, None])})
    with pytest.raises(ValueError, match="missing values"):
        arrow_rows.ArrowRows(holes, "y", None, False, float("nan"))


def test_train_rejects_unknown_file_types(tmp_path):
    import ferrisboost_amd as fb

    with pytest.raises(ValueError, match="cannot tell the format"):
        fb.train({}, str(tmp_path / "d.csv"), "y")


# ---- category names (cat_recode::Recoder, src/source/cat_recode.rs:1-30;
# numeric dictionaries, src/source/arrow_source.rs:126-145)


def _dict(codes, values):
    return pa.DictionaryArray.from_arrays(pa.array(np.asarray(codes, np.int32)), pa.array(values))


def test_chunk_dictionaries_code_by_first_appearance():
    # Two chunks whose dictionaries list different categories in different
    # orders: a category keeps one code, codes follow the rows' first use.
    c1 = _dict([0, 1, 0, 1], ["a", "b"])
    c2 = _dict([0, 1, 2, 1], ["c", "b", "a"])
    col = pa.chunked_array([c1, c2])
    t = pa.table({"k": col, "y": pa.array(np.zeros(8, np.float32))})
    src = arrow_rows.ArrowRows(t, "y", None, True, float("nan"), batch_rows=3)
    got = _read_all(src, 5)[:, 0]
    # rows: a b a b | c b a b  ->  a=0, b=1, c=2
    assert got.tolist() == [0, 1, 0, 1, 2, 1, 0, 1]
    assert src.coders[0].values == ["a", "b", "c"]
    assert np.array_equal(_read_all(src, 8)[:, 0], got)  # the second pass agrees
    assert arrow_rows.categories_of(src, None) == [["a", "b", "c"]]


def test_row_group_dictionaries_and_unused_entries(tmp_path):
    # Parquet row groups with their own dictionaries: unused entries and the
    # dictionary's order do not matter, only the order rows use the values.
    groups = [(["z", "y", "x"], [2, 2, 0]), (["x", "w"], [1, 0, 1]), (["w", "y"], [1, 0])]
    batches = [pa.record_batch({"k": _dict(c, v), "y": pa.array(np.ones(len(c), np.float32))})
               for v, c in groups]
    path = tmp_path / "g.parquet"
    with pq.ParquetWriter(path, batches[0].schema) as w:
        for b in batches:
            w.write_table(pa.Table.from_batches([b]))
    src = arrow_rows.ArrowRows(path, "y", None, True, float("nan"), batch_rows=2)
    got = _read_all(src, 3)[:, 0]
    # rows: x x z | w x w | y w  ->  x=0, z=1, w=2, y=3
    assert got.tolist() == [0, 0, 1, 2, 0, 2, 3, 2]
    assert src.coders[0].values == ["x", "z", "w", "y"]


def test_numeric_dictionaries_yield_their_values_and_strings_are_categories():
    vals = _dict([1, 0, 1, 1], pa.array([10, 20], pa.int64()))
    strings = pa.array(["q", None, "p", "q"])
    t = pa.table({"v": vals, "s": strings, "y": pa.array(np.zeros(4, np.float32))})
    src = arrow_rows.ArrowRows(t, "y", None, True, float("nan"))
    got = _read_all(src, 4)
    assert got[:, 0].tolist() == [20, 10, 20, 20]
    assert got[:, 1].tolist()[0] == 0 and np.isnan(got[1, 1]) and got[2:, 1].tolist() == [1, 0]
    assert src.categorical.tolist() == [1, 1]
    assert arrow_rows.categories_of(src, None) == [None, ["q", "p"]]


def test_prediction_tables_recode_by_value():
    cats = [None, ["q", "p"]]
    t = pa.table({"s": _dict([0, 1, 2, 0], ["p", "q", "r"]), "v": pa.array([1.5, 2.5, 3.5, 4.5])})
    with pytest.raises(ValueError, match="'r', which is not in the training categories"):
        arrow_rows.table_matrix(t, ["v", "s"], cats, 2, float("nan"))
    t = t.slice(0, 2)
    X = arrow_rows.table_matrix(t, ["v", "s"], cats, 2, float("nan"))
    assert X.tolist() == [[1.5, 1.0], [2.5, 0.0]]
    with pytest.raises(ValueError, match="missing the model's feature columns"):
        arrow_rows.table_matrix(t, ["v", "nope"], cats, 2, float("nan"))
