"""GPU: training from a Parquet file or an Arrow table (the rows streamed to
the device sketch and binning in chunks through fbt_train_rows) gives the
model that training from the same rows as a numpy matrix gives, byte for
byte: unit weights (streamed), weighted rows (gathered for the host sketch),
string dictionary columns as categorical features coded by category
whatever each chunk's dictionary, a feature the device sketch
leaves to the host (zeros of both signs among its cuts), a reader error
raised back to the caller, and a pandas DataFrame with a category column."""

from __future__ import annotations

import numpy as np
import pytest

pa = pytest.importorskip("pyarrow")
pq = pytest.importorskip("pyarrow.parquet")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fb():
    import ferrisboost_amd as fb
    from ferrisboost_amd import _native as N

    if not N.device_available(0):
        pytest.fail("no gfx950 device: the GPU suite needs an MI355X")
    return fb


@pytest.fixture
def small_reads(monkeypatch):
    # several read chunks per pass
    monkeypatch.setenv("FB_READ_ROWS", "3001")


def _data(n=20_000, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, 6)).astype(np.float32)
    x[rng.random((n, 6)) < 0.05] = np.nan
    # zeros of both signs, with zero among the cuts (left to the host sketch)
    x[:, 5] = np.where(rng.random(n) < 0.3, np.round(rng.standard_normal(n)) * 0.0,
                       rng.standard_normal(n)).astype(np.float32)
    codes = rng.integers(0, 7, n)
    y = (np.nan_to_num(x[:, 0]) + (codes % 3) * 0.7 + rng.standard_normal(n) * 0.3 > 0.5)
    return x, codes, y.astype(np.float32), rng.uniform(0.2, 2.0, n).astype(np.float32)


def _table(x, codes, y, w, categorical, weight_column=True):
    cols = {f"f{j}": pa.array(x[:, j], mask=np.isnan(x[:, j])) for j in range(x.shape[1])}
    if categorical:
        cols["c"] = pa.DictionaryArray.from_arrays(pa.array(codes.astype(np.int32)),
                                                   pa.array([f"k{i}" for i in range(7)]))
    cols["label"] = pa.array(y)
    if weight_column:
        cols["weight"] = pa.array(w)
    return pa.table(cols)


PARAMS = {"objective": "binary:logistic", "max_depth": 6, "eta": 0.3, "max_bin": 64}


@pytest.mark.parametrize("weighted", [False, True])
def test_parquet_trains_the_array_model(fb, tmp_path, small_reads, weighted):
    x, codes, y, w = _data()
    path = tmp_path / "train.parquet"
    pq.write_table(_table(x, codes, y, w, False, weight_column=weighted), path,
                   row_group_size=4096)
    m_file = fb.train(PARAMS, str(path), "label", weight="weight" if weighted else None,
                      num_boost_round=5)
    arr = np.ascontiguousarray(x)
    # feature 5 holds both zero signs and a zero cut: the device sketch leaves it to the host
    cuts = fb.sketch(arr, 64)
    z = x[:, 5][x[:, 5] == 0]
    assert (cuts.values[cuts.offsets[5]:cuts.offsets[6]] == 0).any()
    assert np.signbit(z).any() and not np.signbit(z).all()
    m_arr = fb.train(PARAMS, arr, y, weight=w if weighted else None, num_boost_round=5)
    assert m_file.to_json() == m_arr.to_json()
    assert np.array_equal(m_file.train_margins(y.size).view(np.uint32),
                          m_arr.train_margins(y.size).view(np.uint32))
    assert m_file.feature_names == [f"f{j}" for j in range(6)]
    assert bool(m_file.stats["device_sketch"]) == (not weighted)
    assert m_file.stats["device_binning"]


def _first_appearance(codes):
    u, first = np.unique(codes, return_index=True)
    remap = np.empty(u.max() + 1, np.int64)
    remap[u[np.argsort(first)]] = np.arange(u.size)
    return remap[codes]


def _chunked_dictionaries(codes, names, seed):
    """The category column as chunks whose dictionaries list the categories
    in their own orders (as Arrow chunks and Parquet row groups may)."""
    rng = np.random.default_rng(seed)
    chunks = []
    for part in np.array_split(np.arange(codes.size), 3):
        perm = rng.permutation(len(names))  # chunk dictionary position -> category
        pos = np.argsort(perm)              # category -> chunk dictionary position
        chunks.append(pa.DictionaryArray.from_arrays(
            pa.array(pos[codes[part]].astype(np.int32)), pa.array([names[i] for i in perm])))
    return pa.chunked_array(chunks)


def test_dictionary_columns_are_categorical(fb, small_reads):
    # String dictionaries are coded by category in the order rows first use
    # them (src/source/cat_recode.rs:1-30), whatever each chunk's dictionary.
    x, codes, y, w = _data(seed=1)
    t = _table(x, codes, y, w, True)
    p = dict(PARAMS, enable_categorical=True)
    m_tab = fb.train(p, t, "label", num_boost_round=5)
    arr = np.ascontiguousarray(np.column_stack([x, _first_appearance(codes).astype(np.float32),
                                                w]))
    m_arr = fb.train(dict(PARAMS, feature_types=["q"] * 6 + ["c", "q"]), arr, y,
                     num_boost_round=5)
    assert m_tab.to_json() == m_arr.to_json()
    names = [f"k{i}" for i in range(7)]
    assert m_tab.get_categories()[6] == [names[c] for c in
                                         codes[np.sort(np.unique(codes, return_index=True)[1])]]
    t2 = t.set_column(t.column_names.index("c"), "c", _chunked_dictionaries(codes, names, 5))
    m_chunks = fb.train(p, t2, "label", num_boost_round=5)
    assert m_chunks.to_json() == m_tab.to_json()
    # prediction re-codes a table's categories by value
    want = m_arr.predict(arr, output_margin=True)
    assert np.array_equal(m_tab.predict(t2, output_margin=True), want)
    with pytest.raises(ValueError, match="enable_categorical"):
        fb.train(PARAMS, t, "label", num_boost_round=1)


def test_reader_errors_reach_the_caller(fb, monkeypatch):
    from ferrisboost_amd import arrow_rows

    x, codes, y, w = _data(n=2000, seed=2)
    t = _table(x, codes, y, w, False)

    def broken(self, batch):
        raise OSError("the source went away")

    monkeypatch.setattr(arrow_rows.ArrowRows, "_rows_of", broken)
    with pytest.raises(OSError, match="went away"):
        fb.train(PARAMS, t, "label", num_boost_round=1)


def test_reader_rows_take_8bit_cells_as_arrays_do(fb):
    """At max_bin 256 a numeric feature without a missing row fills its 256
    bins into 8-bit cells. From an Arrow table the device sketch counts the
    missing values, so the table-trained context plans the same cell widths
    (the same planned bytes) as the array-trained one, and the models are
    equal byte for byte."""
    rng = np.random.default_rng(4)
    n = 30_000
    x = rng.standard_normal((n, 6)).astype(np.float32)
    x[:, 5][rng.random(n) < 0.02] = np.nan  # one feature keeps 16-bit cells
    y = (x[:, 0] + x[:, 1] * x[:, 2] > 0).astype(np.float32)
    cols = {f"f{j}": pa.array(x[:, j], mask=np.isnan(x[:, j])) for j in range(6)}
    cols["label"] = pa.array(y)
    p = dict(PARAMS, max_bin=256)
    m_tab = fb.train(p, pa.table(cols), "label", num_boost_round=4)
    m_arr = fb.train(p, np.ascontiguousarray(x), y, num_boost_round=4)
    assert m_tab.stats["device_sketch"] and m_arr.stats["device_sketch"]
    assert m_tab.stats["planned_bytes"] == m_arr.stats["planned_bytes"]
    assert m_tab.to_json() == m_arr.to_json()
    m_wide = fb.train(dict(p, hip_host_sketch=True), np.ascontiguousarray(x), y,
                      num_boost_round=4)
    assert m_wide.stats["planned_bytes"] == m_arr.stats["planned_bytes"]


def test_dataframe_trains_the_array_model(fb):
    """A pandas DataFrame trains the model its float32 matrix trains (category
    columns as their positions in `categories`, feature names from the
    columns), and prediction binds columns by name and re-codes categories
    by value."""
    pd = pytest.importorskip("pandas")
    x, codes, y, w = _data(n=20_000, seed=5)
    names = ["rome", "oslo", "lima", "kyiv", "doha", "baku", "riga"]
    df = pd.DataFrame({f"f{j}": x[:, j] for j in range(6)})
    df["c"] = pd.Categorical.from_codes(codes, names)
    p = dict(PARAMS, enable_categorical=True)
    m_df = fb.train(p, df, y, num_boost_round=5, weight=w)
    arr = np.ascontiguousarray(np.column_stack([x, codes.astype(np.float32)]))
    m_arr = fb.train(dict(PARAMS, feature_types=["q"] * 6 + ["c"]), arr, y, num_boost_round=5,
                     weight=w)
    assert m_df.feature_names == list(df.columns)
    assert m_df.get_categories()[6] == names
    assert m_df.to_json() == m_arr.to_json()
    assert np.array_equal(m_df.predict(df, output_margin=True),
                          m_arr.predict(arr, output_margin=True))
    shuffled = df.assign(c=df["c"].cat.reorder_categories(names[::-1]), extra=0.0)
    shuffled = shuffled[["extra", "c"] + [f"f{j}" for j in range(5, -1, -1)]]
    assert np.array_equal(m_df.predict(shuffled, output_margin=True),
                          m_arr.predict(arr, output_margin=True))
    # monotone constraints by column name
    m_mono = fb.train(dict(p, monotone_constraints={"f0": 1}), df, y, num_boost_round=3)
    m_mono_arr = fb.train(dict(PARAMS, feature_types=["q"] * 6 + ["c"],
                               monotone_constraints=(1, 0, 0, 0, 0, 0, 0)), arr, y,
                          num_boost_round=3)
    assert m_mono.to_json() == m_mono_arr.to_json()
    with pytest.raises(ValueError, match="enable_categorical"):
        fb.train(PARAMS, df, y, num_boost_round=1)
