/* fbtrain.h -- C ABI of the host round driver (libfbtrain.so).
 *
 * The driver is the restated training state machine of FerrisBoost's
 * device="cuda" path: train_with_backend (src/training/mod.rs:1299-2376),
 * build_tree (src/training/mod.rs:3357-4565) and lossguide::grow
 * (src/training/lossguide.rs:494-700). It prepares the data exactly like
 * DenseSource (sketch -> cuts -> u8/u16 column blocks,
 * src/source/dense.rs:99-290) and runs gradients, histograms, split scans,
 * partitions, leaves and margins through the fbh_* backend (fbhip.h): the
 * exact-mode gradient (gpu_math="exact", src/training/mod.rs:2033-2087) on
 * the device with the host libm's sigmoid restated, or through the host
 * libm when the device's does not match it or the caller asks; the fast
 * mode (gpu_math="fast") with the hardware exponential. Depthwise trees,
 * and lossguide trees whose leaf cap cannot bind, grow whole on the device.
 * It never falls back to a CPU histogram or split path: without a usable
 * device, fbt_train fails with FBH_RUNTIME_ERROR.
 *
 * Status codes as fbhip.h (0 ok, 1 input error, 2 runtime error).
 */
#ifndef FBTRAIN_H
#define FBTRAIN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Training parameters: TrainParams (src/types.rs:432-660) and the Python
 * parameter surface (python/ferrisboost/__init__.py:46-200). */
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
    uint32_t objective;        /* 0 = reg:squarederror, 1 = binary:logistic,
                                  2 = multi:softprob, 3 = multi:softmax,
                                  4 = reg:quantileerror */
    uint32_t grow_policy;      /* 0 = depthwise, 1 = lossguide */
    uint32_t max_cat_to_onehot;
    uint32_t max_cat_threshold;
    float base_score;          /* used when has_base_score != 0 */
    uint32_t has_base_score;
    uint32_t nthread;          /* host threads (0 = up to 16) */
    uint32_t num_class;        /* classes of multi:softprob / multi:softmax */
    /* device-path knobs */
    int32_t device;            /* "cuda:N" */
    uint32_t gpu_math;         /* 0 = "exact" (bit-identical to the CPU engine),
                                  1 = "fast" (hardware exp in the logistic
                                  gradient: deterministic, not bit-equal) */
    uint64_t gpu_memory_budget;/* bytes, 0 = automatic */
    uint32_t tile_bytes;       /* LDS histogram tile (0 = default) */
    uint32_t rows_per_block;   /* histogram rows per workgroup (0 = default) */
    uint32_t profile;          /* 1: time histogram kernels with HIP events */
    uint32_t host_sigmoid;     /* 1: logistic sigmoid on the host every round
                                  (0: on the device once it matches the host
                                  libm on the probe inputs) */
    uint32_t host_levels;      /* 1: depthwise trees grow level by level from
                                  the host (0: whole trees on the device when
                                  every tile and column is resident) */
    uint32_t sync_round;       /* nonzero: the loop waits for the device before
                                  this round starts (a clean timing boundary;
                                  trees are otherwise collected a round late) */
    uint32_t hist_streams;     /* hist_streams: 1 or 2 streaming windows (0 = 2) */
    uint32_t resident_limit;   /* resident_blocks + 1: at most that many LDS
                                  tiles stay resident (0 = as the budget allows) */
    uint32_t host_binning;     /* 1: bin the rows on the host and upload column
                                  blocks (0: bin on the device when the plan
                                  keeps the columns resident and the budget has
                                  room for the row staging) */
    uint32_t host_sketch;      /* 1: sketch the cuts on the host (0: on the
                                  device for unit row weights when the budget
                                  has room, the same cuts either way) */
    uint32_t n_quantile_alpha; /* reg:quantileerror: quantiles (1..=64), one
                                  output and one tree a round each */
    const float *quantile_alpha; /* ascending, in [0, 1] */
    const float *base_margin;  /* per-row starting margins, class-major
                                  [outputs][n_rows], finite (XGBoost's
                                  base_margin; TrainConfig::base_margin,
                                  src/training/mod.rs:646-652); NULL: every
                                  row starts at the intercept. The intercepts
                                  are estimated and stored either way. */
    float colsample_bylevel;   /* (0, 1]: each depth's features drawn from the
                                  tree's (src/data/colsample.rs:203-286);
                                  0 reads as 1 */
    float colsample_bynode;    /* (0, 1]: each node's features drawn from its
                                  depth's; 0 reads as 1 */
    const float *feature_weights; /* n_features nonnegative weights of the
                                  column samplers (feature_weights,
                                  src/data/colsample.rs:119-195); NULL or all
                                  equal: uniform */
} fbt_params;

/* One tree node: Node (src/model/tree.rs:52-111). */
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
    uint32_t cat_begin;
    uint32_t cat_len;
} fbt_node;

/* Timing of the last training call. */
typedef struct {
    double train_seconds;     /* the round loop (gradients .. leaf deltas) */
    double setup_seconds;     /* sketch, binning, context, upload */
    double hist_kernel_ms;    /* histogram kernels (HIP events; profile=1) */
    uint64_t hist_launches;
    uint64_t hist_bytes;      /* algorithmic bytes of the histogram launches */
    double host_gradient_seconds;  /* the per-round gradient step (host and device) */
    double device_bytes;      /* bytes the backend context holds */
    uint32_t rounds;
    uint32_t device_sigmoid;  /* 1: logistic gradients used the device sigmoid */
    uint32_t n_tiles;         /* LDS tiles of the memory plan (fbh_plan) */
    uint32_t resident_tiles;  /* tiles kept in HBM; the others streamed */
    uint64_t streamed_bytes;  /* host-to-device bytes of streamed records and columns */
    uint64_t planned_bytes;   /* peak_bytes of the plan */
    uint64_t budget_bytes;    /* the budget the plan honoured */
    uint32_t device_trees;    /* trees grown whole on the device (fbh_grow_depthwise) */
    uint32_t device_binning;  /* 1: the rows were binned on the device (fbh_upload_rows) */
    double sketch_seconds;    /* the quantile sketch, part of setup_seconds */
    double bin_seconds;       /* binning and upload of the bins, part of setup_seconds */
    uint32_t device_sketch;   /* 1: the cuts came from the device sketch (fbh_sketch_*) */
} fbt_stats;

typedef struct fbt_model fbt_model;

size_t fbt_last_error(char *buf, size_t len);

/* fb.train(params, X, label, weight) on the device path. x is row-major
 * [n_rows][n_features] f32 (NaN = missing), categorical[f] != 0 marks
 * categorical features, monotone holds per-feature -1/0/1 constraints. */
int fbt_train(const float *x, uint64_t n_rows, uint32_t n_features, const float *labels,
              const float *weights, const uint8_t *categorical, const int8_t *monotone,
              uint32_t n_monotone, const fbt_params *params, fbt_model **out);
/* Training from a row reader (the Parquet / Arrow sources of the Python
 * entry, DenseSource's two passes, src/source/dense.rs:99-290): fn(user,
 * begin, count, out) fills `count` row-major f32 rows from row `begin` (NaN
 * is missing) and returns 0, or nonzero to stop with an input error. The
 * reader is called front to back in chunks of about 64 MB, once to sketch
 * the cuts and once to bin the rows, both on the device when the plan allows;
 * the matrix is gathered into host memory only where a host pass needs it
 * whole (weighted rows, whose sketch runs on the host, or host binning).
 * Labels and weights are whole arrays. The result equals fbt_train on the
 * same rows. */
typedef int (*fbt_rows_fn)(void *user, uint64_t row_begin, uint64_t n_rows, float *out);
int fbt_train_rows(fbt_rows_fn fn, void *user, uint64_t n_rows, uint32_t n_features,
                   const float *labels, const float *weights, const uint8_t *categorical,
                   const int8_t *monotone, uint32_t n_monotone, const fbt_params *params,
                   fbt_model **out);
/* fbt_train with the cuts given instead of sketched (the cut_values /
 * cut_offsets fbt_sketch_cuts returns for the same data, max_bin, weights
 * and categorical flags), so several models over one matrix share one
 * sketch. The cuts are checked (strictly increasing finite values, at most
 * max_bin - 1 per numeric feature, offsets n_features + 1 long); no
 * reference counterpart (the reference re-sketches per DenseSource). */
int fbt_train_cuts(const float *x, uint64_t n_rows, uint32_t n_features, const float *labels,
                   const float *weights, const uint8_t *categorical, const int8_t *monotone,
                   uint32_t n_monotone, const fbt_params *params, const float *cut_values,
                   const uint32_t *cut_offsets, fbt_model **out);
int fbt_last_stats(fbt_stats *out);
/* Per-round timing of the last training call: wall seconds of round r (from
 * its start to the start of round r+1, delta download and gradient pass
 * included), histogram kernel milliseconds and algorithmic bytes (the
 * latter two need params.profile = 1). Returns the number of rounds. */
uint32_t fbt_last_round_stats(double *wall_s, double *hist_ms, uint64_t *hist_bytes,
                              uint32_t capacity);
/* Histogram launches of each round of the last training call (needs
 * params.profile = 1), counted as fbt_last_round_stats counts the bytes.
 * Returns the number of rounds. */
uint32_t fbt_last_round_launches(uint64_t *hist_launches, uint32_t capacity);

void fbt_model_free(fbt_model *m);
uint32_t fbt_model_n_trees(const fbt_model *m);
uint32_t fbt_model_tree_len(const fbt_model *m, uint32_t tree);
void fbt_model_tree_nodes(const fbt_model *m, uint32_t tree, fbt_node *out);
uint32_t fbt_model_n_cat_words(const fbt_model *m);
void fbt_model_cat_words(const fbt_model *m, uint32_t *out);
float fbt_model_base_score(const fbt_model *m);
float fbt_model_base_margin(const fbt_model *m);
uint32_t fbt_model_n_features(const fbt_model *m);
/* Training-set margins the round loop accumulated: n_rows floats, or
 * num_class x n_rows class-major for a multiclass model (n_rows is the
 * training row count either way). */
int fbt_model_train_margins(const fbt_model *m, float *out, uint64_t n_rows);
/* Outputs per row (num_class of a multiclass model, the number of
 * quantile_alpha of a reg:quantileerror model, else 1) and a multi-output
 * model's per-output intercepts (class_base_margins, src/model/tree.rs:
 * 256-260; tree t belongs to output t % outputs). */
uint32_t fbt_model_num_outputs(const fbt_model *m);
void fbt_model_class_margins(const fbt_model *m, float *out);
/* A reg:quantileerror model's quantile_alpha (the Python model's
 * quantile_alpha, src/python/mod.rs:3159-3166): the count, with up to cap
 * values copied to out (may be NULL); 0 for other objectives. */
uint32_t fbt_model_quantile_alpha(const fbt_model *m, float *out, uint32_t cap);
/* Cuts the model was trained with (values, offsets n_features + 1). */
uint32_t fbt_model_n_cuts(const fbt_model *m);
void fbt_model_cuts(const fbt_model *m, float *values, uint32_t *offsets);
/* Model::predict_margin (src/model/tree.rs:486-510) on row-major rows; a
 * multiclass model writes [n_rows][num_class] (predict_margins_upto,
 * src/model/tree.rs:470-480). */
void fbt_predict_margin(const fbt_model *m, const float *x, uint64_t n_rows, uint32_t n_features,
                        float *out);
/* XGBoost-schema JSON (Model::to_xgboost_json, src/model/tree.rs:600-760).
 * Returns the length; writes at most len bytes (NUL-terminated) when buf. */
size_t fbt_model_to_json(const fbt_model *m, char *buf, size_t len);
/* pred_contribs on the device (GpuExplainModel): out [n_rows][n_features+1]. */
int fbt_shap(const fbt_model *m, const float *x, uint64_t n_rows, uint32_t n_features,
             int device, float *out);

/* Outputs of fbt_predict. */
enum {
    FBT_OUT_MARGIN = 0,          /* raw margins [n_rows] ([n_rows][K] multiclass) */
    FBT_OUT_VALUE = 1,           /* margins through the objective's link [n_rows]
                                    (multi:softprob: probabilities [n_rows][K];
                                    multi:softmax: the class index [n_rows]) */
    FBT_OUT_LEAF = 2,            /* pred_leaf: tree-local leaf ids [n_rows][trees] */
    FBT_OUT_CONTRIBS = 3,        /* pred_contribs: TreeSHAP [n_rows][n_features + 1] */
    FBT_OUT_APPROX_CONTRIBS = 4, /* approx_contribs: Saabas [n_rows][n_features + 1] */
    FBT_OUT_INTERACTIONS = 5     /* pred_interactions [n_rows][n_features + 1]^2 */
    /* A multiclass model explains each class with its own trees and
     * intercept (Model::class_view, src/model/tree.rs:395-425): contributions
     * [n_rows][K][n_features + 1], interactions [n_rows][K][...]^2. */
};
/* Model.predict (python/ferrisboost/_core.pyi:94-197, src/python/mod.rs:
 * 2667-2800) over the trees [tree_begin, tree_end) (n_trees and
 * iteration_range select them: a prefix, or the slice of
 * src/python/mod.rs:1993-2029, which keeps the model's base score). x is
 * row-major [n_rows][n_features] f32, NaN = missing; base_margin (may be
 * NULL) is XGBoost's per-row starting margin, replacing the intercept and the
 * bias of explanations. device >= 0 runs on that GPU (the GpuPredictor /
 * GpuExplainModel kernels); device < 0 scores FBT_OUT_MARGIN / FBT_OUT_VALUE
 * on the host (use_gpu=False). The logistic link is 1 / (1 + expf(-m))
 * (objective.rs:37-39, 600-614) on either side, bit for bit; softprob's is
 * the row softmax of softmax_in_place (objective.rs:1308-1322) with the host
 * libm. A multiclass model's base_margin is class-major (K x n_rows). Feature values
 * equal to the largest float32 are an input error (they are reserved for
 * split boundaries). */
int fbt_predict(const fbt_model *m, const float *x, uint64_t n_rows, uint32_t n_features,
                uint32_t output, uint32_t tree_begin, uint32_t tree_end, const float *base_margin,
                int device, float *out);
/* Model::from_xgboost_json (src/model/tree.rs:754-990, 1259-1470): a model
 * of binary:logistic or reg:squarederror trees from XGBoost-schema JSON
 * text, with the reference's checks (input error on what it cannot
 * represent). The loaded model has no cuts; it predicts and explains. */
int fbt_model_from_json(const char *json, size_t len, fbt_model **out);
/* The model's objective (0 = reg:squarederror, 1 = binary:logistic), its
 * scale_pos_weight, and whether feature `feat` is categorical. */
uint32_t fbt_model_objective(const fbt_model *m);
float fbt_model_scale_pos_weight(const fbt_model *m);
uint32_t fbt_model_is_categorical(const fbt_model *m, uint32_t feat);
/* Device time of the SHAP kernels of this thread's last fbt_shap call (ms). */
double fbt_last_shap_ms(void);

/* Sketch cuts and bins exactly as training does (tests / diagnostics).
 * cut_values holds n_features * max(max_bin, 2) floats. */
int fbt_sketch_cuts(const float *x, uint64_t n_rows, uint32_t n_features, uint32_t max_bin,
                    const float *weights, const uint8_t *categorical, float *cut_values,
                    uint32_t *cut_offsets);

#ifdef __cplusplus
}
#endif
#endif /* FBTRAIN_H */
