/* fbhip.h -- C ABI of the MI355X (gfx950) training and explanation backend.
 *
 * This is the drop-in boundary for FerrisBoost's device="cuda" path. The
 * reference binds its device backend through the Rust API of
 * src/backend/cuda/{train_ctx.rs,split_ctx.rs,explain.rs,mod.rs}; every
 * entry point below names the reference function it replaces. Signatures
 * carry plain pointers and sizes only: host buffers are borrowed for the
 * duration of the call, device memory is owned by the context and allocated
 * once at creation (worst case, like GpuTrainCtx::new_with_shape).
 *
 * Status codes: FBH_OK (0), FBH_INPUT_ERROR (1, the reference's InputError,
 * ValueError in Python, src/error.rs:1-68) and FBH_RUNTIME_ERROR (2).
 * fbh_last_error() returns the message of the last failure on the calling
 * thread. No call panics, aborts or throws across the boundary.
 *
 * Threading: one context is used by one host thread at a time; all device
 * work of a context runs in order on the context's single HIP stream.
 */
#ifndef FBHIP_H
#define FBHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { FBH_OK = 0, FBH_INPUT_ERROR = 1, FBH_RUNTIME_ERROR = 2 };

typedef struct fbh_ctx fbh_ctx;

/* A contiguous run of the device row arena: GpuRowSpan
 * (src/backend/cuda/train_ctx.rs, used by src/training/mod.rs:3253-3281). */
typedef struct {
    uint32_t offset;
    uint32_t len;
} fbh_span;

/* Feature shape of the training matrix: GpuBlockShape
 * (src/training/gpu_mem_plan.rs:95-144) flattened per feature. width[f] is
 * the stored bin width in bytes (1 = u8, 2 = u16), n_bins[f] the histogram
 * bins of feature f (cuts + 1), categorical[f] != 0 marks a categorical
 * feature (may be NULL). */
typedef struct {
    uint32_t n_features;
    const uint8_t *width;
    const uint32_t *n_bins;
    const uint8_t *categorical;
} fbh_shape;

/* Context options: SharedHistogramConfig (src/backend/cuda/mod.rs:84-208)
 * re-derived for MI355X. Zero selects the default of each field. */
typedef struct {
    uint64_t memory_budget;  /* bytes the context may allocate; 0 = free HBM
                                minus the safety reserve (gpu_memory_budget) */
    uint32_t hist_slots;     /* node histograms kept on the device at once */
    uint32_t tile_bytes;     /* LDS bytes of one histogram tile (<= 160 KiB) */
    uint32_t rows_per_block; /* rows one histogram workgroup accumulates */
    uint32_t max_cat_words;  /* 64-bit words of the widest category set */
    uint32_t stream_windows; /* hist_streams: 1 or 2 device windows of each kind
                                for streamed records and columns (2: uploads
                                overlap the kernels) */
    uint32_t resident_limit; /* resident_blocks + 1: keep at most that many LDS
                                tiles resident, streaming the rest even when
                                they would fit (0: as the budget allows) */
    uint32_t n_outputs;      /* margin columns the objective keeps: num_class
                                of a multiclass objective (0 or 1: one) */
    uint32_t reserved[3];
} fbh_config;

/* Split-scan parameters: the TrainParams fields split.rs reads
 * (src/training/split.rs:113-270, src/types.rs:432-660). */
typedef struct {
    float lambda_;
    float gamma;
    float min_child_weight;
    float alpha;
    float max_delta_step;
    uint32_t max_cat_to_onehot;
    uint32_t max_cat_threshold;
    uint32_t reserved;
} fbh_split_params;

/* One node handed to the split scan: a LevelNode (src/training/mod.rs:3239)
 * plus its histogram source (HistFrom, src/training/mod.rs:3283-3291).
 * subtract_parent < 0: accumulate the node's rows into `slot`; otherwise
 * slot = histogram(subtract_parent) - histogram(subtract_sibling), where the
 * sibling is accumulated by an earlier entry of the same call. */
typedef struct {
    fbh_span rows;
    int64_t sum[2];  /* fixed-point node sum, missing rows included */
    float lower;     /* NodeBounds (src/training/split.rs:120-160) */
    float upper;
    uint32_t slot;
    int32_t subtract_parent;
    int32_t subtract_sibling;
    uint32_t reserved;
} fbh_node;

/* The chosen split of one node: SplitCandidate
 * (src/training/split.rs:17-52), 64 bytes like the reference's packet
 * (src/backend/cuda/histogram.cu:6-11). Categorical sets are returned in a
 * separate word array at cat_offset (64-bit words, bit c of word c/64 set =
 * category c goes right). */
typedef struct {
    uint32_t found;
    uint32_t feat;
    uint32_t bin;
    uint32_t missing_left;
    float gain;
    uint32_t is_cat;
    uint32_t cat_offset;
    uint32_t n_cat_words;
    int64_t left[2];
    int64_t right[2];
} fbh_split;

/* One stable partition request (GpuPartitionSession::partition /
 * partition_categorical, src/backend/cuda/train_ctx.rs:4849-5500). */
typedef struct {
    fbh_span rows;
    uint32_t feat;
    uint32_t bin;          /* rows with bin < this go left (numeric) */
    uint32_t missing_left;
    uint32_t cat_offset;   /* into the category words passed alongside */
    uint32_t n_cat_words;  /* 0 = numeric split */
    uint32_t reserved;
} fbh_part_req;

/* ---------------------------------------------------------------- errors */
/* Copies the last error message of this thread (NUL-terminated). Returns its
 * full length. */
size_t fbh_last_error(char *buf, size_t len);
/* 1 when a usable gfx950 device is present, 0 otherwise (never errors). */
int fbh_device_available(int device);

/* ------------------------------------------------------------ lifecycle */
/* GpuTrainCtx::new_with_shape (src/backend/cuda/train_ctx.rs:728-1769):
 * allocates every device buffer of the run once. */
int fbh_ctx_create(int device, uint64_t n_rows, const fbh_shape *shape, const fbh_config *cfg,
                   fbh_ctx **out);
/* Drop of GpuTrainCtx. */
int fbh_ctx_destroy(fbh_ctx *ctx);

/* The memory plan of a context (StreamingMemModel + fill_residency,
 * src/training/gpu_mem_plan.rs:279-600, 855-880, re-derived for HBM-resident
 * LDS tiles). Everything is resident when it fits the budget; otherwise the
 * column-major copies go first, then as many tiles as fit stay resident and
 * the others stream from pinned host memory in row windows (histograms) and
 * whole columns (partitions of their features). A budget that cannot hold
 * the per-row arrays plus the streaming windows is an input error. */
typedef struct {
    uint64_t budget;                /* bytes the context may allocate */
    uint64_t fixed_bytes;           /* per-row arrays, histogram slots, tables */
    uint64_t resident_record_bytes; /* records of the resident tiles */
    uint64_t column_bytes;          /* resident column-major bins (0: none) */
    uint64_t staging_bytes;         /* streaming windows (0: nothing streams) */
    uint64_t peak_bytes;            /* the sum: what the context allocates */
    uint64_t streamed_record_bytes; /* host records streamed by one full pass */
    uint32_t n_tiles;
    uint32_t resident_tiles;
    uint32_t columns_resident;      /* 1: the partition reads resident columns */
    uint32_t window_rows;           /* rows of one streamed window */
} fbh_plan;

/* The plan fbh_ctx_create would make for this shape, configuration and free
 * device memory (no device needed; free_bytes is used when
 * cfg->memory_budget is 0, minus max(15 %, 512 MiB) of it as the reserve of
 * default_safety_reserve, src/training/gpu_mem_plan.rs:957-959). */
int fbh_plan_memory(uint64_t n_rows, const fbh_shape *shape, const fbh_config *cfg,
                    uint64_t free_bytes, fbh_plan *out);
/* The plan a context was created with. */
int fbh_ctx_plan(const fbh_ctx *ctx, fbh_plan *out);
/* Host-to-device bytes the context has streamed (records and columns of
 * streamed tiles) since its creation. */
uint64_t fbh_ctx_streamed_bytes(const fbh_ctx *ctx);
/* GpuTrainCtx::budget (src/backend/cuda/train_ctx.rs:103-242): bytes the
 * context holds on the device. */
uint64_t fbh_ctx_device_bytes(const fbh_ctx *ctx);

/* --------------------------------------------------------------- blocks */
/* GpuTrainCtx::block_session_bins / resident block upload
 * (src/backend/cuda/train_ctx.rs:3507-4052): one ColumnBlock
 * (src/data/columns.rs:9-46), column-major data[local * n_rows + row] of
 * `width` bytes per cell, features feat_ids[0..n_feats). The device re-lays
 * it into LDS-sized tiles of row records. */
int fbh_upload_block(fbh_ctx *ctx, const uint32_t *feat_ids, uint32_t n_feats, uint32_t width,
                     const void *bins);

/* Binning on the device (the quantisation half of DenseSource's ingest,
 * src/source/dense.rs:99-290, with find_bin / quantize_value,
 * src/data/columns.rs:335-356, and categorical::code_to_bin): the cuts of
 * every feature (a FeatureSketch's cuts, src/data/sketch.rs:236-275) once,
 * then row-major f32 rows in chunks. Each chunk is binned on the device
 * straight into the context's resident bin columns: NaN to the missing code
 * (all ones of the feature's width); a numeric value to the number of cuts
 * <= it; a categorical value v to v when 0 <= v < n_bins, else to the
 * unseen-category code (missing - 1). fbh_finish_rows then lays the columns
 * into the tile records, as fbh_upload_block does. The chunk's rows are
 * staged in device memory outside the memory plan: fbh_rows_staging_bytes
 * gives how much, and the calls are an input error when the budget's
 * remaining room cannot hold it or when the plan streams the columns (bin
 * on the host and use fbh_upload_block then).
 * cut_values[cut_offsets[f] .. cut_offsets[f + 1]) are feature f's cuts,
 * strictly increasing; categorical[f] (nullable) marks categorical
 * features, whose cut count is then n_bins - 1 (the codes 1..n_bins-1). */
int fbh_set_cuts(fbh_ctx *ctx, const float *cut_values, const uint32_t *cut_offsets,
                 const uint8_t *categorical);
/* Device bytes the row staging of fbh_upload_rows takes. */
uint64_t fbh_rows_staging_bytes(const fbh_ctx *ctx);
/* Rows [row0, row0 + n_rows) of the matrix, row-major with the context's
 * n_features columns (x points at row row0). */
int fbh_upload_rows(fbh_ctx *ctx, const float *x, uint64_t row0, uint64_t n_rows);
/* Every feature's tile records from its binned column; the features count
 * as uploaded from then on. */
int fbh_finish_rows(fbh_ctx *ctx);

/* The quantile sketch on the device (the sketch half of DenseSource's
 * ingest, src/source/dense.rs:99-290): SketchSet::with_categorical,
 * push_row over every row with weight 1, finalize_checked
 * (src/data/sketch.rs:440-560). The cuts equal the host sketch's bit for
 * bit: each feature's non-missing values are batched in row order, sorted
 * and merged through the same binary counter of summaries, with the same
 * f32 operations. Row weights other than 1 are not taken (sketch those on
 * the host). The one value the host leaves to its unstable sort is the sign
 * of a zero entry whose batch holds both -0.0 and +0.0 (they compare
 * equal): a numeric feature holding both signs whose cuts include a zero is
 * reported in host_features and left to the caller's host sketch.
 * The sketch is independent of any context: it allocates its own device
 * memory (fbh_sketch_device_bytes at most) and frees it at destroy. */
typedef struct fbh_sketch fbh_sketch;
/* Device bytes a sketch of these sizes takes at most; 0 when the device
 * sketch does not take them (max_bin above 1024, 2^32 rows or more). */
uint64_t fbh_sketch_device_bytes(uint64_t n_rows, uint32_t n_features, uint32_t max_bin,
                                 const uint8_t *categorical);
/* 1 when fbh_sketch_create would accept these sizes on this device
 * (fbh_sketch_device_bytes within memory_budget, or within free HBM minus
 * max(15 %, 512 MiB) when memory_budget is 0), else 0. Never errors. */
int fbh_sketch_fits(int device, uint64_t n_rows, uint32_t n_features, uint32_t max_bin,
                    const uint8_t *categorical, uint64_t memory_budget);
/* SketchSet::with_categorical (src/data/sketch.rs:452-466) for n_rows rows
 * of n_features features; categorical[f] (nullable) marks categorical
 * features. Input error when the sizes do not fit (fbh_sketch_fits). */
int fbh_sketch_create(int device, uint64_t n_rows, uint32_t n_features, uint32_t max_bin,
                      const uint8_t *categorical, uint64_t memory_budget, fbh_sketch **out);
/* SketchSet::push_row (src/data/sketch.rs:474-483) over the next n_rows
 * rows, row-major f32 (NaN is missing). At most the created row count in
 * all; x may be reused when the call returns. */
int fbh_sketch_push_rows(fbh_sketch *s, const float *x, uint64_t n_rows);
/* SketchSet::finalize_checked (src/data/sketch.rs:517-560), once: feature
 * f's cuts into cut_values[cut_offsets[f] .. cut_offsets[f + 1])
 * (n_features + 1 offsets). A categorical feature's cuts are its codes
 * 1..max_code; an invalid code (negative, fractional or above 65533) is
 * the reference's input error. host_features[f] (n_features entries) is 1
 * for a numeric feature holding both zero signs whose cuts include a zero;
 * its cuts are then left empty for the caller to sketch on the host; else
 * 0. Input error when the
 * cuts need more than values_capacity values (the offsets are set). */
int fbh_sketch_cuts(fbh_sketch *s, float *cut_values, uint64_t values_capacity,
                    uint32_t *cut_offsets, uint8_t *host_features);
/* Missing (NaN) values of every numeric feature among the rows pushed so far
 * into missing[f] (n_features entries; 0 for categorical features). The
 * trainer stores a 256-bin numeric feature with none in 8-bit cells. Has no
 * counterpart in the reference (whose bins are 32-bit). */
int fbh_sketch_missing(const fbh_sketch *s, uint64_t *missing);
int fbh_sketch_destroy(fbh_sketch *s);

/* ------------------------------------------------------------ gradients */
/* GpuTrainCtx::upload_and_quantize_gpair_sampled
 * (src/backend/cuda/train_ctx.rs:2345-2391, 3182-3343): uploads interleaved
 * f32 [grad, hess] per row, masks rows the sampler drops
 * (threshold from subsample::threshold_for; UINT64_MAX keeps all), picks the
 * power-of-two scales (GradQuantizer::try_from_bounds) and writes the i64
 * fixed-point pairs. Returns the scales and the fixed-point root sum. */
int fbh_upload_quantize_gpair(fbh_ctx *ctx, const float *gpair2n, uint64_t sample_threshold,
                              uint64_t seed, uint64_t tree, double scales_out[2],
                              int64_t root_sum_out[2]);
/* GpuTrainCtx::upload_gpair: fixed-point pairs quantized on the host. */
int fbh_upload_gpair_fixed(fbh_ctx *ctx, const int64_t *gpair2n, const double scales[2]);

/* Resident labels, gradient weights and margins (GpuTrainCtx::init_fast_math,
 * src/backend/cuda/train_ctx.rs:2964-3060): objective 0 = reg:squarederror,
 * 1 = binary:logistic; grad_weights (may be NULL) are the row weights with
 * scale_pos_weight folded in; every margin starts at base_margin. From then
 * on fbh_assign_leaves also adds each row's leaf value to its margin (the
 * same f32 addition as the host's pred += delta) and records the row's leaf
 * position (u8 when the tree has at most 256 leaves, else u16). */
int fbh_set_objective(fbh_ctx *ctx, uint32_t objective, const float *labels,
                      const float *grad_weights, float base_margin);

/* Host half of the exact-mode logistic gradient: for rows
 * [row_begin, row_begin + n) apply the last tree's leaf values (leaf_ids is
 * NULL before the first tree) to the host margins and write
 * s = 1 / (1 + expf(-margin)) per row to sigmoid_out. */
typedef void (*fbh_sigmoid_fn)(void *user, uint64_t row_begin, uint64_t n, const void *leaf_ids,
                               uint32_t id_bytes, float *sigmoid_out);

/* One round's gradient pairs, the exact-mode round of train_with_backend
 * (src/training/mod.rs:2010-2110: with_prediction_delta, gradient_of
 * :5449-5459, upload_and_quantize_gpair_sampled). Squared error is computed
 * from the device margins. Logistic with fn == NULL uses the device sigmoid
 * (fbh_sigmoid_device, bit-identical to the host libm's 1 / (1 + expf(-x)))
 * on the device margins: no host work, no per-row traffic. Logistic with a
 * callback downloads the last tree's leaf ids in chunks, calls fn per chunk
 * while later chunks are in flight and uploads the sigmoids. Either way the
 * device derives g = s - y, h = max(s(1 - s), 1e-16) (times the weight) with
 * the host's f32 operations, then masks, scales and quantizes as
 * fbh_upload_quantize_gpair. The scales are computed on the device from the
 * bounds (the floor of a correctly rounded log2, as the host's libm gives
 * it). With root_out NULL the root sum stays on the device (for
 * fbh_grow_depthwise) and the call returns once the scales are known,
 * without waiting for the quantisation. With scales_out NULL as well (the
 * callback must then be NULL) nothing comes back and the call does not wait
 * at all: the scales stay on the device for the kernels that follow, and
 * fbh_grow_collect reports invalid bounds (non-finite gradients) of the
 * round the tree was grown in, and checks the device's scales against the
 * host libm's. */
int fbh_gradient_exchange(fbh_ctx *ctx, fbh_sigmoid_fn fn, void *user, uint64_t sample_threshold,
                          uint64_t seed, uint64_t tree, double scales_out[2],
                          int64_t root_sum_out[2]);

/* gpu_math (src/python/mod.rs, TrainParams::gpu_math): 0 = "exact" (the
 * default: the device sigmoid is bit-identical to the host libm's), 1 =
 * "fast": the logistic gradient uses the hardware exponential, as the
 * reference's fast path does on its device (apply_delta_and_gradient,
 * src/backend/cuda/histogram.cu:673-783; fast_gradient_and_quantize,
 * src/backend/cuda/train_ctx.rs:2404-2512): deterministic, not bit-equal to
 * the CPU engine. A host sigmoid callback is an input error in fast mode. */
int fbh_set_gpu_math(fbh_ctx *ctx, uint32_t gpu_math);
/* The f32 gradient pairs [n][2] of `margin` under objective 0 / 1 with
 * gpu_math 0 (exact) or 1 (fast), on host buffers (weights may be NULL):
 * the per-row arithmetic of fbh_gradient_exchange, for characterisation. */
int fbh_gradient_pairs(int device, uint32_t objective, uint32_t gpu_math, const float *margin,
                       const float *labels, const float *weights, uint64_t n, float *gpair2n_out);

/* The device margins (the training margins after the assigned trees);
 * n_outputs x n_rows class-major values for a multiclass objective. */
int fbh_download_margin(fbh_ctx *ctx, float *out);
/* GpuTrainCtx::init_fast_math_rows (src/backend/cuda/train_ctx.rs:2985-3010)
 * for every objective: replaces the margins the objective call set with
 * per-row starting margins, class-major [n_outputs][n_rows] (XGBoost's
 * base_margin; TrainConfig::base_margin, src/training/mod.rs:646-652).
 * Call after fbh_set_objective / fbh_set_multiclass / fbh_set_quantile and
 * before the first gradients. */
int fbh_set_margins(fbh_ctx *ctx, const float *margins);

/* Multiclass objectives (multi:softprob / multi:softmax): the resident state
 * of train_multiclass_rounds (src/training/mod.rs:2578-2850) and its device
 * gradient (softmax_row_stats / softmax_class_gradient,
 * src/backend/cuda/histogram.cu:786-890; Objective::softmax_gradients,
 * src/training/objective.rs:1175-1219). The context keeps n_classes margin
 * columns (class-major, n_classes x n_rows), each starting at its class
 * intercept; labels are class indices; weights (may be NULL) are the sample
 * weights. The context must have been created with cfg->n_outputs equal to
 * n_classes. */
int fbh_set_multiclass(fbh_ctx *ctx, uint32_t n_classes, const float *labels,
                       const float *weights, const float *class_margins);
/* At the start of a round: every row's largest class margin (from the
 * smallest normal float up) and the sum over classes, in double, of
 * exp(margin - largest), which the round's class gradients share: each class
 * of a round takes its pairs from the margins the round started with. exp is
 * glibc's expf restated (gpu_math exact, the host's values bit for bit) or
 * the hardware exponential (fast). */
int fbh_multiclass_begin_round(fbh_ctx *ctx);
/* The output (class or quantile) the next gradient call computes the pairs
 * of and whose margin column the next tree's leaves update. */
int fbh_set_output(fbh_ctx *ctx, uint32_t output);

/* reg:quantileerror (Objective::quantile_gradient / quantile_scale,
 * src/training/objective.rs:1002-1160; train_multiclass_rounds with several
 * quantile_alpha, src/training/mod.rs:2578-2890; the fast path's
 * quantile_apply_delta_partials / quantile_reduce_scale /
 * quantile_gradient_rows, src/backend/cuda/histogram.cu:907-1077): one margin
 * column per alpha (ascending, in [0, 1]), each starting at its intercept;
 * weights (may be NULL) are the sample weights. The context must have been
 * created with cfg->n_outputs equal to n_alphas. Every fbh_gradient_exchange
 * first takes the round's scale S = (sum w sqrtf|m - y| / sum w)^2 of the
 * current output's column: gpu_math exact sums the f32 terms on the host in
 * row order in double (the reference's serial sum, bit for bit; one
 * device-to-host copy of 4 bytes a row; with several alphas, every
 * column's sum starts at the first column's call, one host thread each,
 * when n_alphas x 4 bytes a row fit the memory budget's remaining room and
 * 1 GiB, and a later column's call takes its finished sum), fast sums them
 * on the device in a
 * fixed order (deterministic). The pairs use glibc's tanhf restated, so
 * exact-mode pairs equal the host's bit for bit.
 * fbh_quantile_last_scale reads back the scale the last gradient call used. */
int fbh_set_quantile(fbh_ctx *ctx, uint32_t n_alphas, const float *alphas, const float *labels,
                     const float *weights, const float *intercepts);
int fbh_quantile_last_scale(fbh_ctx *ctx, float *scale);

/* The logistic sigmoid 1 / (1 + expf(-x)) of Objective::gradient
 * (src/training/objective.rs:37-39) with expf restated from glibc's
 * table-driven method, computed by the host compile (fbh_sigmoid_host) or on
 * the device (fbh_sigmoid_device). fbh_sigmoid_checksum fingerprints the
 * device sigmoid over the float bit patterns [begin, end) (end <= 2^32):
 * the wrapping sum of splitmix64(u ^ bits(s(u)) << 32), NaN outputs as
 * 0x7fc00000. The round driver compares device and host sigmoids on probe
 * inputs before it relies on the device. */
int fbh_sigmoid_host(const float *in, uint64_t n, float *out);
int fbh_sigmoid_device(int device, const float *in, uint64_t n, float *out);
int fbh_sigmoid_checksum(int device, uint64_t begin, uint64_t end, uint64_t *out);
/* The same fingerprint of the device tanhf (glibc's fdlibm-derived tanhf
 * restated; Objective::quantile_gradient, src/training/objective.rs:1151). */
int fbh_tanh_checksum(int device, uint64_t begin, uint64_t end, uint64_t *out);

/* ------------------------------------------------------------------ tree */
/* GpuTrainCtx::begin_tree_rows (src/backend/cuda/train_ctx.rs:1971-1993) plus
 * the tree's column plan (BlockPlan, src/training/mod.rs:3302-3463): resets
 * the row arena to 0..n_rows, zeroes the prediction delta and selects the
 * features whose histograms this tree builds (ascending global ids; NULL =
 * all features). Returns the root span. */
int fbh_begin_tree(fbh_ctx *ctx, const uint32_t *features, uint32_t n_features,
                   const int8_t *monotone, uint32_t n_monotone, fbh_span *root);

/* GpuBlockSession::split_cached_submit / split_cached_finish
 * (src/backend/cuda/split_ctx.rs:387-960) over every selected feature:
 * builds the histograms of the accumulate nodes in one batched launch
 * (hist_build_shared_planar32_batched, histogram.cu:1685-1852), derives the
 * subtract nodes (sibling subtraction), runs the split scan per
 * (node, feature) and the per-node argmax with the reference's tie rules
 * (split.rs:260-270, 631-642). enabled[i*n_features_tree + j] (may be NULL)
 * masks feature j of the tree for node i. Category sets of categorical
 * winners are copied to cat_words (capacity cat_capacity 64-bit words). */
int fbh_eval_nodes(fbh_ctx *ctx, const fbh_node *nodes, uint32_t n_nodes,
                   const fbh_split_params *params, const uint8_t *enabled, fbh_split *out,
                   uint64_t *cat_words, uint32_t cat_capacity);

/* Copies the histogram of a slot to the host (download_histograms,
 * src/backend/cuda/train_ctx.rs:4770-4817): 2 * width int64, in the tree's
 * compact feature order. Returns the width through width_out when out is
 * NULL. */
int fbh_download_histogram(fbh_ctx *ctx, uint32_t slot, int64_t *out, uint64_t *width_out);

/* GpuPartitionSession::partition_resident_multi + resolve_partitions
 * (src/backend/cuda/train_ctx.rs:4893-5196, 2007-2055): stable partition of
 * every requested span (left rows keep their order, then right rows keep
 * theirs) in place, one blocking copy of the left counts. children receives
 * (left, right) per request. */
int fbh_partition(fbh_ctx *ctx, const fbh_part_req *reqs, uint32_t n_reqs,
                  const uint64_t *cat_words, uint32_t n_cat_words, fbh_span *children);

/* One split node of fbh_partition_eval. */
typedef struct fbh_child_pair {
    uint32_t parent_slot; /* histogram slot of the split node */
    uint32_t new_slot;    /* a free slot for one child */
    uint32_t evaluate;    /* nonzero: build and scan both children */
    uint32_t reserved;
    float lower[2];       /* monotone bounds of the left and right child */
    float upper[2];
    int64_t left_sum[2];  /* fixed-point sums of the children (the split's left, right) */
    int64_t right_sum[2];
} fbh_child_pair;

/* One growth step with one host round trip: fbh_partition of the split
 * nodes, then fbh_eval_nodes of the children of every pair marked
 * `evaluate`, planned on the device from the partition's left counts.
 * Replaces partition_resident_multi + resolve_partitions +
 * finish_partition_level followed by histogram_device_batch +
 * split_cached_submit/finish of the children (train_ctx.rs:4893, 2007, 2058,
 * 4543; split_ctx.rs:387-960), as one depthwise level or one lossguide
 * expansion (lossguide.rs:73, 416-463) drives them. Of an evaluated pair the
 * smaller child (the left one on ties) accumulates into new_slot and the
 * larger one is derived in place from parent_slot; left_slot[i] receives the
 * slot the left child holds (UINT32_MAX when not evaluated). children gets
 * (left, right) per request; out gets (left, right) packets per evaluated
 * pair, in order, with their category sets in cat_out. Every slot of the
 * evaluated pairs must be used once. */
int fbh_partition_eval(fbh_ctx *ctx, const fbh_part_req *reqs, uint32_t n_reqs,
                       const uint64_t *cat_words, uint32_t n_cat_words,
                       const fbh_child_pair *pairs, const fbh_split_params *params,
                       fbh_span *children, uint32_t *left_slot, fbh_split *out,
                       uint64_t *cat_out, uint32_t cat_capacity);

/* fbh_partition_eval whose children scan only some of the tree's features:
 * enabled[(2 * e + k) * n_tree_features + j] != 0 lets child k (0 left, 1
 * right) of the e-th evaluated pair split on tree feature j (the order
 * fbh_begin_tree selected). The reference's masked split scan
 * (split_cached_features_masked, src/backend/cuda/histogram.cu:482-494; the
 * per-(node, feature) byte masks of split_ctx.rs:66) for colsample_bylevel /
 * colsample_bynode (src/training/mod.rs:3575-3638). NULL = every feature. */
int fbh_partition_eval_masked(fbh_ctx *ctx, const fbh_part_req *reqs, uint32_t n_reqs,
                              const uint64_t *cat_words, uint32_t n_cat_words,
                              const fbh_child_pair *pairs, const fbh_split_params *params,
                              const uint8_t *enabled, fbh_span *children, uint32_t *left_slot,
                              fbh_split *out, uint64_t *cat_out, uint32_t cat_capacity);

/* One node of a tree grown on the device, in the order the host grower
 * numbers them (Tree::split_leaf, src/model/tree.rs:140-170). */
typedef struct fbh_tree_node {
    uint32_t feat, bin;   /* split: feature and bin as in fbh_split */
    int32_t left, right;  /* child ids, -1 for a leaf */
    float leaf_value;     /* learning rate applied; 0 for a split node */
    float sum_hess;
    float gain;
    uint32_t flags;       /* bit 0 leaf, bit 1 missing goes left, bit 2 categorical */
    uint32_t cat_offset;  /* right-going category set: cat_words[cat_offset..+n_cat_words] */
    uint32_t n_cat_words;
    float value_as_leaf;  /* the node's leaf value (learning rate applied) had it
                             stayed a leaf; equal to leaf_value for a leaf */
    uint32_t leaf_pos;    /* a leaf's position among the leaf values (its rows'
                             leaf id); 0xFFFFFFFF for a split node or a leaf
                             without rows */
} fbh_tree_node;

/* fbh_grow_params.flags */
enum {
    /* The rows' leaf ids are computed but no leaf value is added to the
     * margins: the caller adds them with fbh_apply_leaf_values once it has
     * decided them (lossguide under a binding leaf cap, which keeps only
     * some of the grown splits). Needs a device objective. */
    FBH_GROW_DEFER_LEAVES = 1
};

typedef struct fbh_grow_params {
    uint32_t max_depth;   /* 1..=14 */
    uint32_t max_leaves;  /* 0: unlimited */
    float learning_rate;
    uint32_t flags;       /* FBH_GROW_* */
} fbh_grow_params;

/* A whole depthwise tree on the device (build_tree, src/training/mod.rs:
 * 3357-4565, driving the calls fbh_eval_nodes / fbh_partition_eval /
 * fbh_assign_leaves stand for), enqueued level after level without waiting
 * on the host: the max_leaves budget, node ids, leaf weights, monotone
 * bounds, partitions, histogram slots and the leaf assignment are decided
 * by kernels, and one copy brings the tree back. The root sum is the one
 * the gradient call returned (NULL: the one it left on the device); every
 * tile and column must be resident. Leaf
 * values come back in leaf-id order (the ids fbh_gradient_exchange hands to
 * a host sigmoid callback). */
int fbh_grow_depthwise(fbh_ctx *ctx, const fbh_grow_params *grow, const fbh_split_params *params,
                       const int64_t root_sum[2], fbh_tree_node *nodes, uint32_t node_capacity,
                       uint32_t *n_nodes, uint64_t *cat_words, uint32_t cat_capacity,
                       float *leaf_values, uint32_t leaf_capacity, uint32_t *n_leaves);
/* The same in two halves: _async enqueues the tree and returns; collect
 * waits for the oldest enqueued tree and copies it out (at most two wait).
 * A caller enqueues the next round's gradients before collecting, so the
 * host rebuilds tree r while the device computes round r + 1. root_sum may
 * be NULL after fbh_gradient_exchange with a NULL root_out: the root sum then
 * never leaves the device. */
int fbh_grow_depthwise_async(fbh_ctx *ctx, const fbh_grow_params *grow,
                             const fbh_split_params *params, const int64_t root_sum[2]);
int fbh_grow_collect(fbh_ctx *ctx, fbh_tree_node *nodes, uint32_t node_capacity,
                     uint32_t *n_nodes, uint64_t *cat_words, uint32_t cat_capacity,
                     float *leaf_values, uint32_t leaf_capacity, uint32_t *n_leaves);

/* GpuTrainCtx::assign_leaf_values for a tree grown with
 * FBH_GROW_DEFER_LEAVES (src/backend/cuda/train_ctx.rs:2128-2252, the
 * device_leaves of lossguide::grow, src/training/lossguide.rs:693-695):
 * margin[row] += values[leaf id of row] for the last grown tree, values by
 * the leaf positions fbh_grow_collect reported (n_values of them). */
int fbh_apply_leaf_values(fbh_ctx *ctx, const float *values, uint32_t n_values);

/* GpuTrainCtx::assign_leaf_values (src/backend/cuda/train_ctx.rs:2128-2252):
 * delta[row] = value for every row of each span. */
int fbh_assign_leaves(fbh_ctx *ctx, const fbh_span *spans, const float *values, uint32_t n);

/* GpuTrainCtx::download_prediction_delta (src/backend/cuda/train_ctx.rs:2215-2236). */
int fbh_download_delta(fbh_ctx *ctx, float *out);

/* Page-locked host memory (the reference's pinned staging windows,
 * FB_CUDA_PINNED, src/backend/cuda/train_ctx.rs:1129-1204): the per-round
 * delta download and gradient upload run at full link speed from it. */
int fbh_host_alloc(size_t bytes, void **out);
int fbh_host_free(void *p);
/* The current row arena (tests and diagnostics). */
int fbh_download_rows(fbh_ctx *ctx, uint32_t *out);

/* Device time of the histogram kernels since creation or the last reset, in
 * milliseconds, and their launch count (HIP events on the context stream).
 * Does not wait: launches still running are counted by a later call (after
 * any blocking call, such as fbh_download_margin, everything is counted). */
int fbh_hist_timing(fbh_ctx *ctx, double *ms_out, uint64_t *launches_out, uint64_t *bytes_out,
                    int reset);
/* Enables HIP-event timing of histogram launches (off by default). */
int fbh_set_timing(fbh_ctx *ctx, int enabled);

/* ---------------------------------------------- standalone characterization */
/* build_histogram (src/backend/cuda/mod.rs:241-497): one histogram over a
 * column-major block and a row subset (rows == NULL: all rows), on host
 * buffers. out must hold 2 * offsets[n_feats] int64. */
int fbh_build_histogram(int device, const void *bins, uint32_t width, uint64_t n_rows,
                        uint32_t n_feats, const uint32_t *offsets, const int64_t *gpair2n,
                        const uint32_t *rows, uint64_t n_sel, int64_t *out);
/* partition_rows_gpu (src/backend/cuda/mod.rs:848-892): stable partition of
 * rows by one column, on host buffers. Returns the left count. */
int fbh_partition_rows(int device, const void *col, uint32_t width, uint64_t n_rows,
                       const uint32_t *rows, uint64_t n, uint32_t split_bin,
                       uint32_t missing_left, const uint64_t *cat_words, uint32_t n_cat_words,
                       uint32_t *out, uint64_t *n_left);

/* ------------------------------------------------------------ TreeSHAP */
typedef struct fbh_shap_model fbh_shap_model;

/* GpuExplainModel::new (src/backend/cuda/explain.rs:186-490): flattened
 * single-output ensemble. Node arrays are indexed by the global node id;
 * tree_offsets[t] is the first node of tree t (n_trees + 1 entries).
 * left/right are tree-local child ids (-1 for leaves), cat_offset/cat_len
 * index cat_words (32-bit words; cat_len 0 = numeric). bias is the model's
 * margin-space base score. */
int fbh_shap_model_create(int device, uint32_t n_trees, const uint32_t *tree_offsets,
                          const uint32_t *feat, const float *split_cond, const int32_t *left,
                          const int32_t *right, const uint8_t *default_left,
                          const uint8_t *is_leaf, const float *leaf_value,
                          const float *sum_hess, const uint32_t *cat_offset,
                          const uint32_t *cat_len, const uint32_t *cat_words,
                          uint32_t n_cat_words, uint32_t n_features, float bias,
                          fbh_shap_model **out);
int fbh_shap_model_destroy(fbh_shap_model *m);
/* GpuExplainModel::compute (src/backend/cuda/explain.rs:491-843) for
 * pred_contribs: rows row-major [n_rows][n_features], optional per-row
 * margin replacing the bias, out [n_rows][n_features + 1]. */
int fbh_shap_contribs(fbh_shap_model *m, const float *rows, uint64_t n_rows,
                      const float *margin, float *out);
/* Same on device-resident buffers (no host copies): d_rows and d_out are
 * device pointers; the call is asynchronous on the model's stream when
 * sync == 0. */
int fbh_shap_contribs_device(fbh_shap_model *m, const float *d_rows, uint64_t n_rows,
                             const float *d_margin, float *d_out, int sync);
/* Milliseconds of the kernels of the model's last host call (all batches) or
 * device call with sync != 0 (HIP events): fbh_shap_contribs[_device|_noalloc],
 * fbh_shap_interactions, fbh_saabas_contribs, fbh_predict[_device]. */
double fbh_shap_last_ms(const fbh_shap_model *m);

/* Explainer::compute with Kind::Interactions (interaction_row,
 * src/model/explain.rs:762-811; device shx interaction kernels,
 * src/backend/cuda/histogram.cu:3438-3571) for pred_interactions: out
 * [n_rows][n_features + 1][n_features + 1], symmetric, each row summing to
 * the row's pred_contribs. */
int fbh_shap_interactions(fbh_shap_model *m, const float *rows, uint64_t n_rows,
                          const float *margin, float *out);
/* Explainer::compute with Kind::Contribs { approx: true } (saabas_row,
 * src/model/explain.rs:730-760; histogram.cu:4101-4181) for
 * approx_contribs: out [n_rows][n_features + 1], bias last. */
int fbh_saabas_contribs(fbh_shap_model *m, const float *rows, uint64_t n_rows,
                        const float *margin, float *out);

/* Prediction outputs of fbh_predict. */
enum { FBH_PREDICT_MARGIN = 0, FBH_PREDICT_SIGMOID = 1, FBH_PREDICT_LEAF = 2 };
/* GpuPredictor::predict_margins_from (src/backend/cuda/inference.rs:300-431;
 * kernels predict_margin_soa[_cat], src/backend/cuda/histogram.cu:2459-2494,
 * 3600-3642) and leaf_row (src/model/explain.rs:689-702) over the model's
 * trees, on host rows [n_rows][n_features]:
 *   FBH_PREDICT_MARGIN:  out[row] = (margin ? margin[row] : bias) plus every
 *                        tree's leaf, added in tree order (Model::predict_margin,
 *                        src/model/tree.rs:486-510);
 *   FBH_PREDICT_SIGMOID: the logistic link 1 / (1 + expf(-m)) of that margin
 *                        (objective.rs:37-39, 600-614), bit-identical to the
 *                        host libm's;
 *   FBH_PREDICT_LEAF:    out [n_rows][n_trees], the tree-local node id of each
 *                        tree's leaf as a float (margin unused). */
int fbh_predict(fbh_shap_model *m, const float *rows, uint64_t n_rows, const float *margin,
                uint32_t output, float *out);
/* The same on device buffers, asynchronous on the model's stream when
 * sync == 0. */
int fbh_predict_device(fbh_shap_model *m, const float *d_rows, uint64_t n_rows,
                       const float *d_margin, uint32_t output, float *d_out, int sync);

/* Bytes of device scratch fbh_shap_contribs_noalloc stages through. */
#define FBH_NOALLOC_SCRATCH_BYTES (32u << 20)
/* fbh_shap_contribs without any device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Rows, margins and contributions are staged batch by batch
 * through a fixed FBH_NOALLOC_SCRATCH_BYTES array that each device holds for
 * the life of the process (found once per device on the first call). The
 * copies in and out are ordinary (pageable) copies followed by a stream
 * synchronisation, so the call is not capturable as it stands; and the
 * kernel's private per-lane segment (its register spills) is backed by the
 * HIP runtime, which may size that backing at the kernel's first launch,
 * as for any kernel. A row
 * of more than (FBH_NOALLOC_SCRATCH_BYTES - 768) / (8 * n_features + 8)
 * features' worth of data is an input error. Results equal
 * fbh_shap_contribs bit for bit. Calls that overlap on one device share the
 * array and race: serialise them. */
int fbh_shap_contribs_noalloc(fbh_shap_model *m, const float *rows, uint64_t n_rows,
                              const float *margin, float *out);

#ifdef __cplusplus
}
#endif
#endif /* FBHIP_H */
