// fbt_internal.h -- host-side types of the round driver (libfbtrain.so).
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "fbtrain.h"

namespace fbt {

struct InputError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct RuntimeError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// BinCuts (src/data/columns.rs:50-360): per-feature upper-bound cuts.
struct Cuts {
    std::vector<float> values;
    std::vector<uint32_t> offsets;  // n_features + 1
    std::vector<uint8_t> categorical;
    // Numeric features of 256 bins with no missing value in the training
    // rows (empty: none known): stored in 8-bit cells, every byte a bin.
    std::vector<uint8_t> full;

    uint32_t n_features() const { return (uint32_t)offsets.size() - 1; }
    uint32_t n_cuts(uint32_t f) const { return offsets[f + 1] - offsets[f]; }
    uint32_t n_bins(uint32_t f) const { return n_cuts(f) + 1; }
    bool is_cat(uint32_t f) const { return categorical[f] != 0; }
    // BinWidth::for_feature (src/data/bins.rs:55-66): 8-bit cells up to 255
    // bins (the all-ones byte is the missing code), 16-bit beyond. Storage
    // only: a 256-bin numeric feature without missing values needs no
    // missing code, so its bins fit 8-bit cells too (same bins, half the
    // bytes the histograms read).
    uint32_t width(uint32_t f) const {
        if (n_bins(f) == 256 && !is_cat(f) && f < full.size() && full[f]) return 1;
        return n_bins(f) <= (is_cat(f) ? 254u : 255u) ? 1u : 2u;
    }
    uint32_t bin_of(uint32_t f, float v) const;
};

// Row-major f32 rows: the whole matrix in memory (x), or a reader that fills
// `count` rows from `begin` (rows are read front to back, once per pass).
struct RowSource {
    const float *x = nullptr;
    std::function<void(uint64_t begin, uint64_t count, float *out)> read;
    // Rows a pass reads at a time: about 64 MB of f32 (FB_READ_ROWS sets
    // the row count).
    static uint64_t chunk_rows(uint32_t n_features) {
        if (const char *e = std::getenv("FB_READ_ROWS")) {
            const long long v = std::atoll(e);
            if (v > 0) return (uint64_t)v;
        }
        return std::max<uint64_t>(1, (64ull << 20) / (4ull * std::max(n_features, 1u)));
    }
    // Every row, front to back, in chunks: fn(begin, count, rows).
    template <class F>
    void each_chunk(uint64_t n, uint32_t nf, F &&fn) const {
        if (x) {
            fn(0, n, x);
            return;
        }
        const uint64_t step = chunk_rows(nf);
        std::vector<float> buf(std::min(step, n) * nf);
        for (uint64_t r0 = 0; r0 < n; r0 += step) {
            const uint64_t k = std::min(step, n - r0);
            read(r0, k, buf.data());
            fn(r0, k, buf.data());
        }
    }
};

// Sketch every feature of a row-major matrix (DenseSource binning pass).
Cuts sketch_matrix(const float *x, uint64_t n_rows, uint32_t n_features, uint32_t max_bin,
                   const float *weights, const uint8_t *categorical, unsigned threads);

// The same cuts from the device sketch (fbh_sketch_*), for unit row
// weights; a feature the device leaves to the host (both zero signs) is
// sketched here.
Cuts sketch_matrix_device(int device, const RowSource &src, uint64_t n_rows,
                          uint32_t n_features, uint32_t max_bin, const uint8_t *categorical,
                          uint64_t memory_budget, unsigned threads);

// Cuts handed in by a caller (fbt_train_cuts): per feature strictly
// increasing finite values, at most max_bin - 1 for a numeric feature and
// categorical flags matching `categorical`; InputError otherwise.
void check_cuts(const Cuts &c, uint32_t n_features, uint32_t max_bin, const uint8_t *categorical);

// Column-major bins of `feats` (one width) for upload.
void bin_columns(const float *x, uint64_t n_rows, uint32_t n_features, const Cuts &cuts,
                 const std::vector<uint32_t> &feats, uint32_t width, void *out, unsigned threads);

// partition_features_by_width (src/data/columns.rs:446-463).
std::vector<std::vector<uint32_t>> blocks_by_width(const Cuts &cuts, uint32_t cols_per_block);

struct Node {
    uint32_t feat = 0;
    float split_cond = 0.0f;
    int32_t left = -1, right = -1;
    bool default_left = false;
    bool is_leaf = true;
    float leaf_value = 0.0f;
    float gain = 0.0f;
    float sum_hess = 0.0f;
    std::vector<uint32_t> cats;  // right-going set, u32 words, trailing zeros trimmed
};

struct Tree {
    std::vector<Node> nodes;
    uint32_t push_leaf(float value, float hess);
    // Tree::split_leaf (src/model/tree.rs:140-170).
    std::pair<uint32_t, uint32_t> split_leaf(uint32_t node, uint32_t feat, float cond,
                                             bool default_left, float gain, float lv, float lh,
                                             float rv, float rh);
    // Tree::set_categories: set words from 64-bit CatBits words.
    void set_categories(uint32_t node, const uint64_t *words64, uint32_t n_words64);
    float leaf_value(const float *x) const;
};

struct Model {
    std::vector<Tree> trees;
    float base_score = 0.5f;
    uint32_t objective = 1;  // 0 squared error, 1 logistic, 2 multi:softprob, 3 multi:softmax,
                             // 4 reg:quantileerror
    // A multiclass (or multi-quantile) model's per-output intercepts
    // (class_base_margins, src/model/tree.rs:256-260); tree t belongs to
    // output t % K. Empty for a single-output model.
    std::vector<float> class_margins;
    // reg:quantileerror's quantile_alpha, one per output (ascending).
    std::vector<float> quantile_alpha;
    uint32_t n_outputs() const { return class_margins.empty() ? 1u : (uint32_t)class_margins.size(); }
    uint32_t n_features = 0;
    float scale_pos_weight = 1.0f;
    Cuts cuts;
    std::vector<float> train_margins;
    float base_margin() const;
};

float base_margin_of(uint32_t objective, float base_score);
std::string model_to_json(const Model &m);
// Model::from_xgboost_json (src/model/tree.rs:754-990); InputError on a
// document the reader cannot represent.
Model model_from_json(const char *text, size_t len);

}  // namespace fbt
