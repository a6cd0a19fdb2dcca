/* oracle.h -- C ABI of the CPU oracle.
 *
 * TEST INFRASTRUCTURE ONLY. This library is a CPU restatement of the
 * FerrisBoost CPU engine (reference crate `ferrisboost` 0.1.1). Only the
 * test suite, the smoke check and the CPU-baseline leg of the benchmark load
 * it, and only to check or time against it. Nothing in the shipped package
 * links, loads or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates.
 * Parity status of each part is listed in oracle.cpp's header.
 */
#ifndef FB_ORACLE_H
#define FB_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Training parameters; field meaning follows TrainParams
 * (src/types.rs:432-660). Layout is shared with the Python test harness. */
typedef struct {
    uint32_t n_rounds;
    uint32_t max_depth;
    uint32_t max_leaves;
    uint32_t max_bin;
    float learning_rate;
    float lambda_;
    float gamma;
    float min_child_weight;
    float alpha;
    float max_delta_step;
    float scale_pos_weight;
    float subsample;
    float colsample_bytree;
    uint32_t cols_per_block;
    uint64_t seed;
    uint32_t objective;       /* 0 = reg:squarederror, 1 = binary:logistic,
                                 2 = multi:softprob, 3 = multi:softmax,
                                 4 = reg:quantileerror */
    uint32_t grow_policy;     /* 0 = depthwise, 1 = lossguide */
    uint32_t max_cat_to_onehot;
    uint32_t max_cat_threshold;
    float base_score;         /* used when has_base_score != 0 */
    uint32_t has_base_score;
    uint32_t nthread;         /* histogram worker threads (0 = 1) */
    uint32_t num_class;       /* classes of multi:softprob / multi:softmax */
    uint32_t n_quantile_alpha; /* quantiles of reg:quantileerror (one output each) */
    const float *quantile_alpha;
    const float *base_margin;  /* starting margins, class-major [outputs][n_rows]
                                  (TrainConfig::base_margin; NULL: the intercepts) */
    float colsample_bylevel;   /* (0, 1]; 0 reads as 1 */
    float colsample_bynode;    /* (0, 1]; 0 reads as 1 */
    const float *feature_weights; /* n_features column-sampling weights (NULL: uniform) */
} orc_params;

/* One tree node; same field meaning as Node (src/model/tree.rs:52-111). */
typedef struct {
    uint32_t feat;
    float split_cond;
    int32_t left;
    int32_t right;
    uint8_t default_left;
    uint8_t is_leaf;
    uint16_t pad;
    float leaf_value;
    float gain;
    float sum_hess;
    uint32_t cat_begin; /* index into the model's category-word pool */
    uint32_t cat_len;   /* u32 words (0 = numeric split or leaf) */
} orc_node;

typedef struct orc_model orc_model;

/* ---- quantizer (src/types.rs:246-385) ---- */
int orc_quantizer_from_bounds(double max_grad, double max_hess, uint64_t n_rows,
                              double out_scale[2]);
void orc_quantize(const float *gpair2n, uint64_t n, const double scale[2], int64_t *out2n,
                  int64_t out_sum[2]);
void orc_to_f64(const int64_t *fixed2n, uint64_t n, const double scale[2], double *out2n);

/* ---- sketch and binning (src/data/sketch.rs, src/data/columns.rs,
 *      src/source/dense.rs:99-290) ---- */
/* Cuts of every feature of a row-major matrix. cut_values must hold
 * n_features * max_bin floats; cut_offsets n_features + 1. */
int orc_sketch_cuts(const float *x, uint64_t n_rows, uint32_t n_features, uint32_t max_bin,
                    const float *weights, const uint8_t *categorical, float *cut_values,
                    uint32_t *cut_offsets);
/* Bin of one value (NaN -> sentinel of the feature's width). */
uint32_t orc_find_bin(const float *cut_values, const uint32_t *cut_offsets, uint32_t feat,
                      uint8_t categorical, float value);

/* ---- histogram (src/training/hist.rs:66-182) ----
 * bins: column-major [n_feats][n_rows] of width 1 or 2 bytes. rows == NULL
 * means every row. out (2 * offsets[n_feats] int64) must be zero on entry. */
void orc_hist_build(const void *bins, uint32_t width, uint64_t n_rows, uint32_t n_feats,
                    const uint32_t *offsets, const int64_t *gpair2n, const uint32_t *rows,
                    uint64_t n_sel, int64_t *out);
void orc_node_sum(const int64_t *gpair2n, const uint32_t *rows, uint64_t n_sel, uint64_t n_rows,
                  int64_t out[2]);

/* ---- split (src/training/split.rs:284-642) ---- */
typedef struct {
    uint32_t found;
    uint32_t feat;
    uint32_t bin;
    float gain;
    int64_t left[2];
    int64_t right[2];
    uint32_t missing_left;
    uint32_t n_cat_words;   /* 64-bit words in cats */
    uint64_t cats[1024];    /* right-going category set (CatBits) */
} orc_split;

/* given_weight != 0: the training path (bounded given-weight gain with node
 * bounds lo/hi and per-feature monotone constraints); 0: the plain
 * G^2/(H+lambda) path of best_split_in_block. */
void orc_best_split(const int64_t *hist, uint32_t n_feats, const uint32_t *feat_ids,
                    const uint32_t *offsets, const int64_t node_sum[2], const double scale[2],
                    const orc_params *p, const uint32_t *sampled, uint32_t n_sampled,
                    uint32_t given_weight, float lo, float hi, const int8_t *monotone,
                    uint32_t n_monotone, const uint8_t *categorical, uint32_t n_categorical,
                    orc_split *out);

/* ---- stable partition (src/training/mod.rs:5169-5430) ----
 * col: the split feature's column [n_rows] of width 1 or 2. Writes left rows
 * then right rows to out; returns the left count. */
uint64_t orc_partition(const uint32_t *rows, uint64_t n, const void *col, uint32_t width,
                       uint32_t split_bin, uint32_t missing_left, const uint64_t *cats,
                       uint32_t n_cat_words, uint32_t *out);

/* ---- training (src/training/mod.rs:1299-2376, 3357-4565; lossguide.rs) ----
 * x: row-major f32 [n_rows][n_features]. cuts may be NULL (sketched here). */
int orc_train(const float *x, uint64_t n_rows, uint32_t n_features, const float *labels,
              const float *weights, const uint8_t *categorical, const int8_t *monotone,
              uint32_t n_monotone, const orc_params *p, orc_model **out);
void orc_model_free(orc_model *m);
/* A model from node records (the layout of orc_node; cat_begin/cat_len index
 * the u32 category words) -- e.g. a model trained elsewhere, to explain it
 * on the CPU. tree_offsets has n_trees + 1 entries. */
int orc_model_from_nodes(const orc_node *nodes, const uint32_t *tree_offsets, uint32_t n_trees,
                         const uint32_t *cat_words, uint32_t n_cat_words, uint32_t objective,
                         float base_score, orc_model **out);
uint32_t orc_model_n_trees(const orc_model *m);
/* Outputs per row (num_class of a multiclass model, else 1) and the class
 * intercepts (class_base_margins, src/model/tree.rs:256-260) of a
 * multiclass model. Training margins of a multiclass model are class-major
 * (K x n), and orc_predict_margin writes n x K for it (predict_margins_upto,
 * src/model/tree.rs:470-480). */
uint32_t orc_model_num_outputs(const orc_model *m);
void orc_model_class_margins(const orc_model *m, float *out);
uint32_t orc_model_tree_len(const orc_model *m, uint32_t tree);
void orc_model_tree_nodes(const orc_model *m, uint32_t tree, orc_node *out);
uint32_t orc_model_n_cat_words(const orc_model *m);
void orc_model_cat_words(const orc_model *m, uint32_t *out);
float orc_model_base_score(const orc_model *m);
float orc_model_base_margin(const orc_model *m);
/* Training-loop wall time of the last orc_train call (seconds). */
double orc_model_train_seconds(const orc_model *m);
/* Margins of the model on row-major rows (Model::predict_margin). */
void orc_predict_margin(const orc_model *m, const float *x, uint64_t n_rows, uint32_t n_features,
                        float *out);
/* The training-set margins the training loop itself accumulated. */
void orc_model_train_margins(const orc_model *m, float *out);

/* ---- QuadratureTreeSHAP (src/model/explain.rs:116-401, 704-728) ----
 * out: [n_rows][n_features + 1]. */
int orc_shap(const orc_model *m, const float *x, uint64_t n_rows, uint32_t n_features,
             float *out);
/* Explainer::compute_with_margin (src/model/explain.rs:612-811): kind 0
 * TreeSHAP contributions [n][nf + 1], 1 Saabas contributions [n][nf + 1],
 * 2 interaction values [n][nf + 1][nf + 1], 3 leaf ids [n][n_trees];
 * margin (may be NULL) replaces the bias per row. */
int orc_explain(const orc_model *m, uint32_t kind, const float *x, uint64_t n_rows,
                uint32_t n_features, const float *margin, float *out);
void orc_quadrature_rule(float nodes[8], float weights[8]);

/* ---- colsample (src/data/colsample.rs:57-117) ---- */
uint32_t orc_sample_features(uint32_t n_features, float rate, uint64_t seed, uint64_t round,
                             uint32_t *out);

/* The collapsed summary of one numeric feature's sketch (FeatureSketch::
 * collapse, src/data/sketch.rs:183-203) after pushing col[0..n) with weights
 * (NULL: 1): (value, weight, rmin, rmax) per entry into out (4 floats each,
 * at most capacity entries). Returns the entry count. */
uint64_t orc_sketch_summary(const float *col, uint64_t n, const float *weights,
                            uint32_t max_bin, float *out, uint64_t capacity);
/* Times compress's ceiling (src/data/sketch.rs:422-424) has moved a pick
 * below the entry its target walk reached, since the library loaded. */
uint64_t orc_compress_clamps(void);

/* Objective::softmax_gradients (src/training/objective.rs:1175-1219) of class
 * k from class-major margins [k_count][n]: f32 pairs [n][2], weights may be
 * NULL. */
void orc_softmax_pairs(const float *margins, const float *labels, const float *weights,
                       uint64_t n, uint32_t k_count, uint32_t k, float *out2n);

/* validated_weights (src/data/colsample.rs:119-141): 0 = uniform sampling
 * (absent or all equal), 1 = weighted, -1 = invalid (orc_last_error). */
int orc_validated_weights(const float *weights, uint32_t n_features);
/* sample_features_weighted (src/data/colsample.rs:174-195); weights NULL =
 * the uniform sampler. */
uint32_t orc_sample_features_weighted(uint32_t n_features, float rate, uint64_t seed,
                                      uint64_t round, const float *weights, uint32_t *out);
/* NestedSampler (src/data/colsample.rs:203-286): tag 1 = level_set(base,
 * depth = idx), tag 2 = node_set(base, node = idx). */
uint32_t orc_nested_set(const uint32_t *base, uint32_t n, float bylevel, float bynode,
                        uint64_t seed, uint64_t tree, uint32_t tag, uint64_t idx,
                        const float *weights, uint32_t *out);
/* subset_key (src/data/colsample.rs:197-201). */
uint64_t orc_subset_key(uint64_t seed, uint64_t tree, uint64_t tag, uint64_t idx);

/* ---- the generators behind sampling ----
 * SplitMix64::next_u64 (src/data/colsample.rs:34-45) from `seed`, n outputs;
 * its finaliser mix (src/data/subsample.rs:44-47); row_hash (:50-55). */
void orc_splitmix64(uint64_t seed, uint64_t n, uint64_t *out);
uint64_t orc_mix64(uint64_t z);
uint64_t orc_row_hash(uint64_t row, uint64_t seed, uint64_t tree);

/* ---- row subsample (src/data/subsample.rs:1-104) ---- */
uint64_t orc_threshold_for(float rate);
int orc_row_selected(uint64_t row, uint64_t threshold, uint64_t seed, uint64_t tree);

/* ---- objective (src/training/objective.rs:37-39, 363-530) ---- */
void orc_gradients(const float *pred, const float *labels, const float *weights, uint64_t n,
                   uint32_t objective, float *out2n);
float orc_base_margin(uint32_t objective, float base_score);
float orc_estimate_base_score(const float *labels, const float *weights, uint64_t n);
/* reg:quantileerror (objective.rs:1002-1160): the round's scale
 * (sum w sqrtf|p - y| / sum w)^2, the weighted pairs of one alpha under a
 * scale, and the labels' alpha quantiles (the intercepts). */
float orc_quantile_scale(const float *pred, const float *labels, const float *weights, uint64_t n);
void orc_quantile_pairs(const float *pred, const float *labels, const float *weights, uint64_t n,
                        float alpha, float scale, float *out2n);
void orc_quantile_intercepts(const float *labels, const float *weights, uint64_t n,
                             const float *alphas, uint32_t k, float *out);

/* Logistic sigmoid 1 / (1 + expf(-x)) with the host libm (objective.rs:37-39),
 * elementwise, and its fingerprint over float bit patterns [begin, end):
 * wrapping sum of splitmix64(u ^ bits(s(u)) << 32), NaN outputs as 0x7fc00000. */
void orc_sigmoid(const float *in, uint64_t n, float *out);
uint64_t orc_sigmoid_checksum(uint64_t begin, uint64_t end, uint32_t threads);
/* The same fingerprint of the host libm's tanhf (objective.rs:1151). */
uint64_t orc_tanh_checksum(uint64_t begin, uint64_t end, uint32_t threads);

/* Message of the last failing call on this thread. */
const char *orc_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
