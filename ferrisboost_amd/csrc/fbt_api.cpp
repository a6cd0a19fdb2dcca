// fbt_api.cpp -- C ABI of the round driver (include/fbtrain.h).

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <memory>
#include <string>

#include "fbhip.h"
#include "fbt_internal.h"

namespace fbt {
Model train(const RowSource &src, uint64_t n, uint32_t nf, const float *y, const float *w,
            const uint8_t *cat, const int8_t *mono, uint32_t n_mono, const fbt_params &p,
            const Cuts *given);
fbt_stats last_stats();
uint32_t last_round_stats(double *wall, double *ms, uint64_t *bytes, uint32_t cap);
uint32_t last_round_launches(uint64_t *launches, uint32_t cap);
}  // namespace fbt

struct fbt_model {
    fbt::Model m;
};

namespace {

thread_local std::string g_err;
thread_local double g_last_shap_ms = 0.0;

template <class F>
int guard(F &&f) {
    try {
        f();
        return FBH_OK;
    } catch (const fbt::InputError &e) {
        g_err = e.what();
        return FBH_INPUT_ERROR;
    } catch (const std::exception &e) {
        g_err = e.what();
        return FBH_RUNTIME_ERROR;
    } catch (...) {
        g_err = "unknown error";
        return FBH_RUNTIME_ERROR;
    }
}

}  // namespace

extern "C" {

size_t fbt_last_error(char *buf, size_t len) {
    if (buf && len) {
        const size_t n = std::min(len - 1, g_err.size());
        std::memcpy(buf, g_err.data(), n);
        buf[n] = 0;
    }
    return g_err.size();
}

int fbt_train(const float *x, uint64_t n_rows, uint32_t n_features, const float *labels,
              const float *weights, const uint8_t *categorical, const int8_t *monotone,
              uint32_t n_monotone, const fbt_params *params, fbt_model **out) {
    return guard([&] {
        if (!x || !labels || !params || !out) throw fbt::InputError("null argument");
        *out = nullptr;
        auto m = std::make_unique<fbt_model>();
        fbt::RowSource src;
        src.x = x;
        m->m = fbt::train(src, n_rows, n_features, labels, weights, categorical, monotone,
                          n_monotone, *params, nullptr);
        *out = m.release();
    });
}

int fbt_train_rows(fbt_rows_fn fn, void *user, uint64_t n_rows, uint32_t n_features,
                   const float *labels, const float *weights, const uint8_t *categorical,
                   const int8_t *monotone, uint32_t n_monotone, const fbt_params *params,
                   fbt_model **out) {
    return guard([&] {
        if (!fn || !labels || !params || !out) throw fbt::InputError("null argument");
        *out = nullptr;
        fbt::RowSource src;
        src.read = [&](uint64_t begin, uint64_t count, float *rows) {
            if (int rc = fn(user, begin, count, rows))
                throw fbt::InputError("the row reader failed at rows " + std::to_string(begin) +
                                      ".." + std::to_string(begin + count) + " (code " +
                                      std::to_string(rc) + ")");
        };
        auto m = std::make_unique<fbt_model>();
        m->m = fbt::train(src, n_rows, n_features, labels, weights, categorical, monotone,
                          n_monotone, *params, nullptr);
        *out = m.release();
    });
}

int fbt_train_cuts(const float *x, uint64_t n_rows, uint32_t n_features, const float *labels,
                   const float *weights, const uint8_t *categorical, const int8_t *monotone,
                   uint32_t n_monotone, const fbt_params *params, const float *cut_values,
                   const uint32_t *cut_offsets, fbt_model **out) {
    return guard([&] {
        if (!x || !labels || !params || !out || !cut_values || !cut_offsets)
            throw fbt::InputError("null argument");
        *out = nullptr;
        fbt::Cuts c;
        c.offsets.assign(cut_offsets, cut_offsets + n_features + 1);
        c.values.assign(cut_values, cut_values + c.offsets.back());
        c.categorical.assign(n_features, 0);
        for (uint32_t f = 0; f < n_features; f++)
            c.categorical[f] = categorical && categorical[f] ? 1 : 0;
        auto m = std::make_unique<fbt_model>();
        fbt::RowSource src;
        src.x = x;
        m->m = fbt::train(src, n_rows, n_features, labels, weights, categorical, monotone,
                          n_monotone, *params, &c);
        *out = m.release();
    });
}

int fbt_last_stats(fbt_stats *out) {
    return guard([&] {
        if (!out) throw fbt::InputError("null argument");
        *out = fbt::last_stats();
    });
}

uint32_t fbt_last_round_stats(double *wall_s, double *hist_ms, uint64_t *hist_bytes,
                              uint32_t capacity) {
    return fbt::last_round_stats(wall_s, hist_ms, hist_bytes, capacity);
}

uint32_t fbt_last_round_launches(uint64_t *hist_launches, uint32_t capacity) {
    return fbt::last_round_launches(hist_launches, capacity);
}

void fbt_model_free(fbt_model *m) { delete m; }
uint32_t fbt_model_n_trees(const fbt_model *m) { return (uint32_t)m->m.trees.size(); }
uint32_t fbt_model_tree_len(const fbt_model *m, uint32_t t) {
    return (uint32_t)m->m.trees[t].nodes.size();
}

void fbt_model_tree_nodes(const fbt_model *m, uint32_t t, fbt_node *out) {
    uint32_t base = 0;
    for (uint32_t k = 0; k < t; k++)
        for (const auto &n : m->m.trees[k].nodes) base += (uint32_t)n.cats.size();
    const auto &nodes = m->m.trees[t].nodes;
    for (size_t i = 0; i < nodes.size(); i++) {
        const auto &n = nodes[i];
        fbt_node o;
        std::memset(&o, 0, sizeof(o));
        o.feat = n.feat;
        o.split_cond = n.split_cond;
        o.left = n.left;
        o.right = n.right;
        o.default_left = n.default_left;
        o.is_leaf = n.is_leaf;
        o.leaf_value = n.leaf_value;
        o.gain = n.gain;
        o.sum_hess = n.sum_hess;
        o.cat_begin = base;
        o.cat_len = (uint32_t)n.cats.size();
        base += o.cat_len;
        out[i] = o;
    }
}

uint32_t fbt_model_n_cat_words(const fbt_model *m) {
    uint32_t s = 0;
    for (const auto &t : m->m.trees)
        for (const auto &n : t.nodes) s += (uint32_t)n.cats.size();
    return s;
}

void fbt_model_cat_words(const fbt_model *m, uint32_t *out) {
    for (const auto &t : m->m.trees)
        for (const auto &n : t.nodes)
            for (uint32_t w : n.cats) *out++ = w;
}

float fbt_model_base_score(const fbt_model *m) { return m->m.base_score; }
float fbt_model_base_margin(const fbt_model *m) { return m->m.base_margin(); }
uint32_t fbt_model_n_features(const fbt_model *m) { return m->m.n_features; }

int fbt_model_train_margins(const fbt_model *m, float *out, uint64_t n) {
    return guard([&] {
        if (!m || !out) throw fbt::InputError("null argument");
        const uint64_t k = m->m.n_outputs();
        if (n * k != m->m.train_margins.size()) throw fbt::InputError("row count mismatch");
        std::memcpy(out, m->m.train_margins.data(), 4 * n * k);
    });
}

uint32_t fbt_model_num_outputs(const fbt_model *m) { return m->m.n_outputs(); }

uint32_t fbt_model_quantile_alpha(const fbt_model *m, float *out, uint32_t cap) {
    const auto &a = m->m.quantile_alpha;
    if (out) std::copy(a.begin(), a.begin() + std::min<size_t>(cap, a.size()), out);
    return (uint32_t)a.size();
}

void fbt_model_class_margins(const fbt_model *m, float *out) {
    std::copy(m->m.class_margins.begin(), m->m.class_margins.end(), out);
}

uint32_t fbt_model_n_cuts(const fbt_model *m) { return (uint32_t)m->m.cuts.values.size(); }

void fbt_model_cuts(const fbt_model *m, float *values, uint32_t *offsets) {
    std::copy(m->m.cuts.values.begin(), m->m.cuts.values.end(), values);
    std::copy(m->m.cuts.offsets.begin(), m->m.cuts.offsets.end(), offsets);
}

void fbt_predict_margin(const fbt_model *m, const float *x, uint64_t n, uint32_t nf, float *out) {
    if (m->m.n_outputs() > 1) {  // Model::predict_margins_upto (src/model/tree.rs:470-480)
        const uint32_t K = m->m.n_outputs();
        for (uint64_t r = 0; r < n; r++) {
            float *o = out + r * K;
            for (uint32_t k = 0; k < K; k++) o[k] = m->m.class_margins[k];
            for (size_t t = 0; t < m->m.trees.size(); t++) o[t % K] += m->m.trees[t].leaf_value(x + r * nf);
        }
        return;
    }
    const float bm = m->m.base_margin();
    for (uint64_t r = 0; r < n; r++) {
        float acc = bm;
        for (const auto &t : m->m.trees) acc += t.leaf_value(x + r * nf);
        out[r] = acc;
    }
}

size_t fbt_model_to_json(const fbt_model *m, char *buf, size_t len) {
    const std::string s = fbt::model_to_json(m->m);
    if (buf && len) {
        const size_t n = std::min(len - 1, s.size());
        std::memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return s.size();
}

}  // extern "C"

namespace {

// The device explanation model of trees [begin, end) (GpuExplainModel::new,
// src/backend/cuda/explain.rs:186-490, over the model slice that
// iteration_range selects, src/python/mod.rs:1993-2029).
using ShapModel = std::unique_ptr<fbh_shap_model, int (*)(fbh_shap_model *)>;

void backend_fail(int rc) {
    char buf[1024];
    fbh_last_error(buf, sizeof(buf));
    if (rc == FBH_INPUT_ERROR) throw fbt::InputError(buf);
    throw fbt::RuntimeError(buf);
}

// The device model of the given trees with `bias` as the intercept of
// predictions and explanations.
ShapModel explain_model(const fbt::Model &m, const std::vector<uint32_t> &ids, float bias,
                        int device) {
    std::vector<uint32_t> offs{0}, feat, cat_off, cat_len, words;
    std::vector<float> cond, leaf, hess;
    std::vector<int32_t> left, right;
    std::vector<uint8_t> dl, is_leaf;
    for (uint32_t t : ids) {
        for (const auto &n : m.trees[t].nodes) {
            feat.push_back(n.feat);
            cond.push_back(n.split_cond);
            left.push_back(n.left);
            right.push_back(n.right);
            dl.push_back(n.default_left);
            is_leaf.push_back(n.is_leaf);
            leaf.push_back(n.leaf_value);
            hess.push_back(n.sum_hess);
            cat_off.push_back((uint32_t)words.size());
            cat_len.push_back(n.is_leaf ? 0u : (uint32_t)n.cats.size());
            if (!n.is_leaf) words.insert(words.end(), n.cats.begin(), n.cats.end());
        }
        offs.push_back((uint32_t)feat.size());
    }
    fbh_shap_model *sm = nullptr;
    const int rc = fbh_shap_model_create(device, (uint32_t)ids.size(), offs.data(), feat.data(),
                                         cond.data(), left.data(), right.data(), dl.data(),
                                         is_leaf.data(), leaf.data(), hess.data(), cat_off.data(),
                                         cat_len.data(), words.data(), (uint32_t)words.size(),
                                         m.n_features, bias, &sm);
    if (rc) backend_fail(rc);
    return ShapModel(sm, fbh_shap_model_destroy);
}

ShapModel explain_model(const fbt::Model &m, uint32_t begin, uint32_t end, int device) {
    std::vector<uint32_t> ids;
    for (uint32_t t = begin; t < end; t++) ids.push_back(t);
    return explain_model(m, ids, m.base_margin(), device);
}

// softmax_in_place (src/training/objective.rs:1308-1322): the row's largest
// margin, the double sum of expf(v - max) in order, each value divided by
// the float of that sum.
void softmax_row(float *row, uint32_t k) {
    float wmax = row[0];
    for (uint32_t i = 1; i < k; i++) wmax = std::fmax(row[i], wmax);
    double wsum = 0.0;
    for (uint32_t i = 0; i < k; i++) {
        row[i] = std::exp(row[i] - wmax);
        wsum += (double)row[i];
    }
    const float d = (float)wsum;
    for (uint32_t i = 0; i < k; i++) row[i] /= d;
}

// argmax (src/training/objective.rs:1324-1333): the first largest.
uint32_t argmax_row(const float *row, uint32_t k) {
    uint32_t best = 0;
    for (uint32_t i = 1; i < k; i++)
        if (row[i] > row[best]) best = i;
    return best;
}

// sort_row_ascending (src/training/objective.rs:1294-1306): XGBoost's
// insertion sort with a > comparison, which keeps NaN where it compares.
void sort_row_ascending(float *row, uint32_t k) {
    for (uint32_t i = 1; i < k; i++) {
        const float v = row[i];
        uint32_t pos = i;
        while (pos > 0 && row[pos - 1] > v) {
            row[pos] = row[pos - 1];
            pos--;
        }
        row[pos] = v;
    }
}

// A multiclass model's outputs: each class scored or explained by its own
// trees with its own intercept (Model::class_view, src/model/tree.rs:
// 395-425), the per-class results laid out [row][class][...].
void predict_multiclass(const fbt::Model &m, const float *x, uint64_t n_rows, uint32_t nf,
                        uint32_t output, uint32_t begin, uint32_t end, const float *base_margin,
                        int device, float *out) {
    const uint32_t K = m.n_outputs();
    if (output == FBT_OUT_LEAF) {
        if (device < 0) throw fbt::InputError("explanations run on the device; pass a device index");
        ShapModel sm = explain_model(m, begin, end, device);
        if (int rc = fbh_predict(sm.get(), x, n_rows, nullptr, FBH_PREDICT_LEAF, out)) backend_fail(rc);
        g_last_shap_ms = fbh_shap_last_ms(sm.get());
        return;
    }
    const bool scores = output == FBT_OUT_MARGIN || output == FBT_OUT_VALUE;
    if (!scores && device < 0)
        throw fbt::InputError("explanations run on the device; pass a device index");
    const uint64_t width = scores ? 1 : output == FBT_OUT_INTERACTIONS
                                            ? (uint64_t)(nf + 1) * (nf + 1)
                                            : (uint64_t)nf + 1;
    std::vector<float> margins(scores ? n_rows * K : 0), col(n_rows * width);
    double ms = 0.0;
    for (uint32_t k = 0; k < K; k++) {
        std::vector<uint32_t> ids;
        for (uint32_t t = begin; t < end; t++)
            if (t % K == k) ids.push_back(t);
        const float *bm = base_margin ? base_margin + (uint64_t)k * n_rows : nullptr;
        const float bias = m.class_margins[k];
        if (device < 0) {
            for (uint64_t r = 0; r < n_rows; r++) {
                float acc = bm ? bm[r] : bias;
                for (uint32_t t : ids) acc += m.trees[t].leaf_value(x + r * nf);
                col[r] = acc;
            }
        } else {
            ShapModel sm = explain_model(m, ids, bias, device);
            int rc = FBH_OK;
            if (scores) rc = fbh_predict(sm.get(), x, n_rows, bm, FBH_PREDICT_MARGIN, col.data());
            else if (output == FBT_OUT_CONTRIBS) rc = fbh_shap_contribs(sm.get(), x, n_rows, bm, col.data());
            else if (output == FBT_OUT_APPROX_CONTRIBS)
                rc = fbh_saabas_contribs(sm.get(), x, n_rows, bm, col.data());
            else rc = fbh_shap_interactions(sm.get(), x, n_rows, bm, col.data());
            if (rc) backend_fail(rc);
            ms += fbh_shap_last_ms(sm.get());
        }
        if (scores) {
            for (uint64_t r = 0; r < n_rows; r++) margins[r * K + k] = col[r];
        } else {
            for (uint64_t r = 0; r < n_rows; r++)
                std::memcpy(out + (r * K + k) * width, col.data() + r * width, 4 * width);
        }
    }
    g_last_shap_ms = ms;
    if (!scores) return;
    if (output == FBT_OUT_MARGIN) {
        std::memcpy(out, margins.data(), 4 * margins.size());
    } else if (m.objective == 4) {  // several quantiles: each row ascending (non-crossing)
        for (uint64_t r = 0; r < n_rows; r++) sort_row_ascending(&margins[r * K], K);
        std::memcpy(out, margins.data(), 4 * margins.size());
    } else if (m.objective == 3) {  // multi:softmax: the class index
        for (uint64_t r = 0; r < n_rows; r++) out[r] = (float)argmax_row(&margins[r * K], K);
    } else {  // multi:softprob: the probabilities
        for (uint64_t r = 0; r < n_rows; r++) softmax_row(&margins[r * K], K);
        std::memcpy(out, margins.data(), 4 * margins.size());
    }
}

}  // namespace

extern "C" {

int fbt_shap(const fbt_model *mm, const float *x, uint64_t n_rows, uint32_t n_features,
             int device, float *out) {
    return fbt_predict(mm, x, n_rows, n_features, FBT_OUT_CONTRIBS, 0,
                       mm ? (uint32_t)mm->m.trees.size() : 0, nullptr, device, out);
}

int fbt_predict(const fbt_model *mm, const float *x, uint64_t n_rows, uint32_t n_features,
                uint32_t output, uint32_t tree_begin, uint32_t tree_end, const float *base_margin,
                int device, float *out) {
    return guard([&] {
        if (!mm || (!x && n_rows) || (!out && n_rows)) throw fbt::InputError("null argument");
        const fbt::Model &m = mm->m;
        if (n_features != m.n_features)
            throw fbt::InputError("expected " + std::to_string(m.n_features) + " features, got " +
                                  std::to_string(n_features));
        if (output > FBT_OUT_INTERACTIONS) throw fbt::InputError("unknown prediction output");
        if (tree_begin > tree_end || tree_end > m.trees.size())
            throw fbt::InputError("tree range [" + std::to_string(tree_begin) + ", " +
                                  std::to_string(tree_end) + ") is outside the model's " +
                                  std::to_string(m.trees.size()) + " trees");
        // Feature values equal to f32::MAX are reserved for split boundaries
        // (src/model/tree.rs:985-990) and rejected, as in training.
        const uint64_t cells = n_rows * (uint64_t)n_features;
        for (uint64_t i = 0; i < cells; i++)
            if (x[i] == std::numeric_limits<float>::max())
                throw fbt::InputError(
                    "feature values equal to the largest float32 (3.4028235e38) are reserved "
                    "and cannot be scored");
        if (m.n_outputs() > 1) {
            predict_multiclass(m, x, n_rows, n_features, output, tree_begin, tree_end, base_margin,
                               device, out);
            return;
        }
        const bool logistic = m.objective == 1;
        if (device < 0) {
            // Host scoring (use_gpu=False): Model::predict_margin_upto and the
            // objective's transform with the host libm.
            if (output != FBT_OUT_MARGIN && output != FBT_OUT_VALUE)
                throw fbt::InputError("explanations run on the device; pass a device index");
            const float bm = m.base_margin();
            for (uint64_t r = 0; r < n_rows; r++) {
                float acc = base_margin ? base_margin[r] : bm;
                for (uint32_t t = tree_begin; t < tree_end; t++) acc += m.trees[t].leaf_value(x + r * n_features);
                out[r] = output == FBT_OUT_VALUE && logistic ? 1.0f / (1.0f + std::exp(-acc)) : acc;
            }
            return;
        }
        ShapModel sm = explain_model(m, tree_begin, tree_end, device);
        int rc = FBH_OK;
        switch (output) {
            case FBT_OUT_MARGIN:
                rc = fbh_predict(sm.get(), x, n_rows, base_margin, FBH_PREDICT_MARGIN, out);
                break;
            case FBT_OUT_VALUE:
                rc = fbh_predict(sm.get(), x, n_rows, base_margin,
                                 logistic ? FBH_PREDICT_SIGMOID : FBH_PREDICT_MARGIN, out);
                break;
            case FBT_OUT_LEAF:
                rc = fbh_predict(sm.get(), x, n_rows, nullptr, FBH_PREDICT_LEAF, out);
                break;
            case FBT_OUT_CONTRIBS:
                rc = fbh_shap_contribs(sm.get(), x, n_rows, base_margin, out);
                break;
            case FBT_OUT_APPROX_CONTRIBS:
                rc = fbh_saabas_contribs(sm.get(), x, n_rows, base_margin, out);
                break;
            default:
                rc = fbh_shap_interactions(sm.get(), x, n_rows, base_margin, out);
                break;
        }
        if (rc) backend_fail(rc);
        g_last_shap_ms = fbh_shap_last_ms(sm.get());
    });
}

int fbt_model_from_json(const char *json, size_t len, fbt_model **out) {
    return guard([&] {
        if (!json || !out) throw fbt::InputError("null argument");
        *out = nullptr;
        auto m = std::make_unique<fbt_model>();
        m->m = fbt::model_from_json(json, len);
        *out = m.release();
    });
}

uint32_t fbt_model_objective(const fbt_model *m) { return m->m.objective; }
float fbt_model_scale_pos_weight(const fbt_model *m) { return m->m.scale_pos_weight; }
uint32_t fbt_model_is_categorical(const fbt_model *m, uint32_t feat) {
    return feat < m->m.cuts.categorical.size() ? m->m.cuts.categorical[feat] : 0u;
}

double fbt_last_shap_ms(void) { return g_last_shap_ms; }

int fbt_sketch_cuts(const float *x, uint64_t n, uint32_t nf, uint32_t max_bin, const float *w,
                    const uint8_t *cat, float *values, uint32_t *offsets) {
    return guard([&] {
        if (!x || !values || !offsets) throw fbt::InputError("null argument");
        fbt::Cuts c = fbt::sketch_matrix(x, n, nf, max_bin, w, cat, 0);
        std::copy(c.values.begin(), c.values.end(), values);
        std::copy(c.offsets.begin(), c.offsets.end(), offsets);
    });
}

}  // extern "C"
