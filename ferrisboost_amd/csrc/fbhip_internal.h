// fbhip_internal.h -- device-side structures shared by the kernels
// (fbhip_kernels.hip) and the context that launches them (fbhip_ctx.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fbh {

constexpr int HIST_TPB = 256;      // threads of one histogram workgroup
constexpr int SPLIT_TPB = 256;     // threads of one split-scan workgroup
constexpr int PART_TPB = 256;      // threads of one partition workgroup
constexpr int PART_CHUNK = 2048;   // rows of one partition chunk (8 per thread)
// 64-bit words between the cursors of two requests of the one-pass
// partition (one 128-byte line each).
constexpr uint32_t PART_CURSOR_STRIDE = 16;
constexpr int XCDS = 8;            // MI355X accelerator complex dies
constexpr uint32_t NO_SLOT = 0xFFFFFFFFu;
constexpr uint32_t MAX_GROW_SLOTS = 16384;  // histogram slots a device-grown tree can use
constexpr uint32_t MAX_WALK_NODES = 1024;   // tree nodes the row-order leaf walk holds in LDS
// (node, feature) candidates a level decision stages in LDS for its argmax.
constexpr uint32_t DECIDE_CAND_LDS = 4096;

// One histogram tile: a group of features of one width stored as row
// records, record i at data + i * stride, feature k of the tile at byte
// k * width of the record. A tile's histogram fits the LDS tile budget.
// Tiles may share one row bundle (stride = bundle pitch, data = the tile's
// offset in it), so a scattered row costs one cache line for all of them.
struct TileDev {
    const uint8_t *data;
    uint32_t stride;     // bytes from one row's record to the next (multiple of 4)
    uint32_t width;      // 1 or 2
    uint32_t n_feat;     // features in the record
    uint32_t feat_base;  // first entry of this tile in the TileFeatDev table
    uint32_t lds_slots;  // LDS histogram slots of the tile's active features
    uint32_t rec_dwords; // record size in dwords (a launch's tiles may be smaller than its own)
};

// Interleaved tiles: 16 cells a record (8-bit cells in 16 bytes, or 16-bit
// cells of features with at most HIST_ROT_BINS bins in 32 bytes). Their LDS
// layout is slot bin * 16 + k for feature k of the tile, whatever the tile's
// bin counts. Every 16-byte 8-bit tile is interleaved.
constexpr uint32_t HIST_ROT_BINS = 256u;
constexpr uint32_t HIST_ROT_SLOTS = 16u * HIST_ROT_BINS;

// Per-feature entry of a tile for one tree.
struct TileFeatDev {
    uint32_t n_bins;    // 0 when the feature is not built this tree
    uint32_t lds_off;   // first LDS slot of the feature
    uint32_t hist_off;  // first slot of the feature in a node histogram
    // Planar tiles: the feature's two most frequent bins (HOT_NONE: none)
    // are added into 64 lane-private LDS slots each, from hot_off (first
    // bin) and hot_off + 64 (second), so the many lanes of one wave that
    // hold a frequent category do not serialise on one address; the flush
    // folds the lane slots back into their bin.
    uint32_t hot[2];
    uint32_t hot_off;
    uint32_t pad;
};
constexpr uint32_t HOT_NONE = 0xFFFFFFFFu;
constexpr uint32_t HOT_SLOTS = 128u;  // lane-private slots of a feature with hot bins

// One node of a histogram batch.
struct HistNodeDev {
    uint32_t row_off;
    uint32_t row_len;
    uint32_t chunk_begin;  // first chunk of the node in the launch
    uint32_t slot;         // output histogram slot
    uint32_t n_chunks;
    uint32_t group_begin;  // first reduction group of the node (per-chunk partials)
    uint32_t pad[2];
};

// Reduction groups of a node of n chunks (one for a node without rows).
__host__ __device__ inline uint32_t reduce_groups(uint32_t n_chunks) {
    return n_chunks <= 16u ? 1u : (n_chunks + 15u) / 16u;
}

struct ScalesDev;

struct HistLaunch {
    const TileDev *tiles;      // tiles of this launch (one width; records up to the launch's size)
    const TileFeatDev *feats;
    uint32_t n_tiles;
    const HistNodeDev *nodes;
    uint32_t n_nodes;
    const uint32_t *dev_n_nodes;  // non-null: the node count, read on the device
    uint32_t n_chunks;         // chunks of the grid (a node may use fewer)
    uint32_t chunk_rows;
    // Non-null: the launch was planned on the device and the rows per chunk
    // are read from here (chunk_rows is then unused).
    const uint32_t *dev_chunk_rows;
    uint32_t chunk_groups;     // ceil(n_chunks / XCDS)
    uint32_t linear;           // 1: linear workgroup mapping (many tiles), 0: XCD-local
    const uint32_t *rows;      // row arena
    const int64_t *gpair;      // [n_rows][2]
    int64_t *hist;             // [slots][hist_width][2]
    // Non-null: a node of several chunks stores each chunk's histogram here
    // ([chunk][hist_width][2], plain stores) for reduce_chunks_kernel,
    // instead of adding it into its slot with global atomics.
    int64_t *partials;
    // Non-null: the pairs are read as f32 [n_rows][2] and quantized here
    // with the scales at `scales`, as the gradient pass quantized gpair
    // (8 instead of 16 bytes a scattered row).
    const float *gpair_f32;
    const ScalesDev *scales;
    uint64_t hist_width;
    // Streamed tile: its records of rows [row_lo, row_hi) sit at
    // stream_data + (row - row_lo) * stride; only those rows are accumulated.
    const uint8_t *stream_data;
    uint32_t row_lo, row_hi;
    // With partials: a node of more chunks than this is summed into its slot
    // with atomics, so the launch clears the slot (REDUCE_GROUP, or
    // PAIR_MAX_CHUNKS where split_pair_kernel sums smaller nodes itself).
    uint32_t clear_above;
};

// Per-tree feature table of the split scan (compact histogram order).
struct SplitFeatDev {
    uint32_t feat;       // global feature id
    uint32_t hist_off;
    uint32_t n_bins;
    int32_t monotone;
    uint32_t categorical;
    uint32_t cat_words;  // 64-bit words of the feature's category set
    uint32_t cat_base;   // word offset of the feature's set within a node's set scratch
    uint32_t pad;
};

struct SplitNodeDev {
    int64_t sum_g, sum_h;
    float lower, upper;
    uint32_t slot;
    uint32_t pad;
};

// Quantizer scales of the current gradients in device memory: computed on
// the device from the gradient bounds, or set from the host for pairs it
// uploads already quantised. Kernels read the inverses from here, so a round
// needs no host round trip between its gradients and its tree.
struct ScalesDev {
    double scale[2];    // power-of-two scales of g and h
    double inv[2];      // their inverses
    double max_abs[2];  // the bounds they come from (0 when set from the host)
    uint32_t status;    // 0: valid; 1: non-finite or negative bounds
    uint32_t from_host; // 1: set from the host (no bounds)
    uint32_t spec_miss; // 1: a speculative gradient pass used other scales
    uint32_t pad;
};

struct SplitParamsDev {
    const ScalesDev *scales;  // quantizer scales (device memory)
    double inv_g, inv_h;      // their inverses, loaded from `scales` by each kernel on entry
    float lambda_, gamma, mcw, alpha, mds;
    uint32_t max_cat_to_onehot, max_cat_threshold;
    uint32_t n_feats;     // features of the tree
    uint32_t cat_words_per_node;
    uint32_t pad;
};

// Best candidate of one (node, feature).
struct FeatCandDev {
    float gain;
    uint32_t found;
    uint32_t bin;
    uint32_t missing_left;
    int64_t left_g, left_h;
};

// Packet of one node (layout of fbh_split).
struct SplitPacketDev {
    uint32_t found, feat, bin, missing_left;
    float gain;
    uint32_t is_cat, cat_offset, n_cat_words;
    int64_t left[2];
    int64_t right[2];
};

struct PartReqDev {
    uint32_t row_off, row_len;
    uint32_t chunk_begin, n_chunks;
    const uint8_t *data;   // tile records of the split feature
    uint32_t stride, byte_off, width;
    uint32_t bin, missing_left;
    uint32_t cat_off, n_cat_words;
    uint32_t count_base;   // index of the request's first chunk in the chunk arrays
    // The cell value that means missing: all ones of the width, except for an
    // 8-bit feature of 256 bins (no missing row, every byte a bin): 256.
    uint32_t missing;
};

// One split node of a fused partition + evaluation step: its children's
// spans come from the partition; the smaller child is accumulated into
// new_slot and the larger derived in place from parent_slot.
struct PairDev {
    uint32_t req;          // index of the node's partition request, NO_SLOT when it has no rows
    uint32_t row_off, row_len;
    uint32_t parent_slot, new_slot;
    uint32_t eval_index;   // position among evaluated pairs, NO_SLOT when not evaluated
    float lower[2], upper[2];  // bounds of the left and right child
    int64_t left_sum[2], right_sum[2];
    uint32_t left_id, right_id;  // tree node ids of the children (device-grown trees)
};

// ---- device-grown depthwise trees ----
// Counters of one tree in device memory; kernels read the counts they run
// over from here (pairs of fields are read as {count, chunks}).
struct GrowState {
    uint32_t n_level;       // evaluated nodes of the current level
    uint32_t n_split;       // split nodes of the level (partition requests, pairs)
    uint32_t part_chunks;   // partition chunks of the split nodes
    uint32_t n_eval;        // pairs whose children are evaluated (n_split or 0)
    uint32_t n_leaves;      // leaf table entries
    uint32_t leaf_chunks;   // leaf-assignment chunks
    uint32_t tree_size;     // tree nodes so far
    uint32_t leaf_count;    // leaves as the host grower counts them (max_leaves)
    uint32_t tree_cat_words;
    uint32_t error;         // bit 0: histogram slots ran out; bit 1: invalid gradient bounds
    uint32_t hist_nodes;    // accumulated nodes with rows (all levels)
    uint32_t pad;
    uint64_t hist_rows;     // accumulated rows (all levels)
    uint64_t covered;       // rows of all leaves
    ScalesDev scales;       // the scales the tree was grown with
};

// Histogram slots a partition's scatter clears for the next level's
// accumulated nodes (hist NULL: none).
struct ZeroNodesDev {
    int64_t *hist;
    uint64_t width;
    const HistNodeDev *nodes;
    const uint32_t *dev_n;  // node count, read on the device
    uint32_t force;         // clear single-chunk nodes too
    uint32_t group;         // nonzero: per-chunk partials; clear only nodes of more chunks than this
};

// Chunks of one node that one workgroup of reduce_chunks_kernel sums
// (reduce_groups).
constexpr uint32_t REDUCE_GROUP = 16;
// Chunks of an accumulated node that split_pair_kernel sums from the
// partials itself (more: reduce_chunks_kernel, atomically into the slot).
constexpr uint32_t PAIR_MAX_CHUNKS = 64;

// Column of one feature for the partition of a device-grown tree.
struct DevColumn {
    const uint8_t *data;
    uint32_t width;
    uint32_t missing;  // the cell value that means missing (256 for a full 8-bit column: none)
};


// One evaluated node of the current level.
struct LNodeDev {
    uint32_t tree_id, row_off, row_len, slot;
    int64_t sum_g, sum_h;
    float lower, upper;
    uint32_t pad[2];
};

// One tree node as the device grows it (node ids in the host grower's order).
struct TreeNodeDev {
    uint32_t feat, bin;
    int32_t left, right;
    float leaf_value, sum_hess, gain;
    uint32_t flags;  // bit 0 leaf, bit 1 default left, bit 2 categorical
    uint32_t cat_off, n_cat_words;
    uint32_t pad[2];
};

struct GrowParamsDev {
    SplitParamsDev sp;     // lambda, alpha, max_delta_step, inverse scales
    float learning_rate;
    uint32_t max_depth, max_leaves;
    uint32_t n_slots;
    uint32_t cw;           // category words per node of the split outputs
    uint32_t n_rows;
    uint32_t pad[2];
    // One-pass partition (part_split_kernel): the level decision zeroes each
    // request's cursor pair here (PART_CURSOR_STRIDE apart); null: the
    // three-pass partition.
    unsigned long long *part_cur;
};

// Rows per chunk of a device-planned histogram launch: fixed when nonzero,
// else ceil(rows / want_chunks) rounded up to 1024 and clamped to
// [min_rows, max_rows].
struct ChunkRule {
    uint32_t fixed, want_chunks, min_rows, max_rows;
    // Nodes of fewer chunks get no chunk-reduction group (split_pair_kernel
    // sums them); 0: every evaluated node gets its groups.
    uint32_t group_min_chunks;
    uint32_t pad;
};

struct LeafDev {
    uint32_t row_off, row_len, chunk_begin;
    float value;
    uint32_t id;     // position of the leaf in the caller's list
    uint32_t arena;  // 0: the row arena, 1: the second arena (device-grown trees)
};

// Flattened ensemble for TreeSHAP.
struct ShapNodeDev {
    uint32_t feat;
    float split_cond;
    int32_t left, right;   // global node ids, -1 for leaves
    float leaf_value;
    float left_weight, right_weight;  // branch_weight of each child
    uint32_t flags;        // bit 0 leaf, bit 1 default_left, bit 2 categorical
    uint32_t cat_offset, cat_len;
    uint32_t uslot;        // slot of the node's feature in its tree's unique list
    uint32_t pad;
};

// Outputs of the level plan that only a device-grown tree has (st null:
// the host drives the tree).
struct GrowDevOut {
    GrowState *st;
    LNodeDev *next;            // the next level's evaluated nodes
    TreeNodeDev *tree;         // read; leaves registered here get their position
    LeafDev *leaves;
    float *leaf_vals;
    uint32_t child_arena;      // arena holding the rows of this level's children
};

// Last-error message shared by every fbh_* entry point (thread local).
void set_last_error(const char *msg);
const char *last_error();

// ---------------------------------------------------------------- launchers
// threads_per_block is 256, 512 or 1024.
// stream: L describes one streamed tile window (see HistLaunch).
// ev_start / ev_stop (nullable) take the launch's start / end time.
// rot: the tile uses the interleaved layout (required for 8-bit 16-byte
// records, allowed for 16-bit 32-byte ones).
hipError_t launch_hist(const HistLaunch &L, int width, int rec_dwords, bool rot,
                       int threads_per_block, bool stream, size_t lds_bytes, hipEvent_t ev_start,
                       hipEvent_t ev_stop, hipStream_t s);
hipError_t launch_hist_global(const HistLaunch &L, int width, hipEvent_t ev_start,
                              hipEvent_t ev_stop, hipStream_t s);
hipError_t launch_zero_slots(int64_t *hist, uint64_t width, const uint32_t *slots, uint32_t n,
                             hipStream_t s);
// dev_n (nullable): the triple count read on the device, n its upper bound.
// Per-chunk partial histograms of the accumulated nodes into their slots:
// plain stores for nodes of 2..REDUCE_GROUP chunks (and zeros for nodes
// without rows), global atomics into the cleared slot per group of
// REDUCE_GROUP chunks for larger ones. max_groups bounds the groups of all
// nodes (HistNodeDev::group_begin numbers them).
// Nodes of fewer than min_chunks chunks are left alone (split_pair_kernel
// sums them).
hipError_t launch_reduce_chunks(int64_t *hist, uint64_t width, const int64_t *partials,
                                const HistNodeDev *nodes, uint32_t n, const uint32_t *dev_n,
                                uint32_t max_groups, uint32_t min_chunks, hipStream_t s);
hipError_t launch_subtract(int64_t *hist, uint64_t width, const uint32_t *triples, uint32_t n,
                           const uint32_t *dev_n, hipStream_t s);
// Zero the slots of accumulated nodes that need it: all when force, else
// those not written by plain stores (n_chunks != 1).
hipError_t launch_zero_nodes(int64_t *hist, uint64_t width, const HistNodeDev *nodes, uint32_t n,
                             const uint32_t *dev_n, bool force, uint32_t group, hipStream_t s);
// Device plan of a fused step: children spans (2 per pair) and the left
// child's slot per pair, the accumulated nodes (one per evaluated pair, in
// pair order), the split-scan nodes (left, right per evaluated pair) and
// the rows per chunk.
hipError_t launch_level_plan(const PairDev *pairs, uint32_t n_pairs, const uint32_t *totals,
                             ChunkRule rule, HistNodeDev *hist_nodes, SplitNodeDev *split_nodes,
                             uint32_t *spans, uint32_t *left_slot, uint32_t *chunk_rows,
                             const GrowDevOut &D, hipStream_t s);
// Device-grown depthwise trees (one workgroup each): the root, the decision
// of one level (see grow_decide_kernel) and the leaf table's chunks.
// root NULL: the root sum is the wrapping sum of n_blocks (g, h) block sums.
// clear (clear_words i64) is cleared by the same launch.
hipError_t launch_grow_prep(const GrowParamsDev &G, const int64_t *root, const int64_t *block_sums,
                            uint32_t n_blocks, uint32_t root_slot, LNodeDev *level,
                            SplitNodeDev *root_split, TreeNodeDev *tree, GrowState *st,
                            int64_t *clear, uint64_t clear_words, hipStream_t s);
// cands non-null: the level decision picks each node's best feature from
// the split scan's candidates itself (split_node_kernel not launched) and
// writes the winners' category sets to pk_cats.
struct FusedArgmaxDev {
    const FeatCandDev *cands;
    const SplitFeatDev *feats;
    const SplitNodeDev *nodes;
    const uint64_t *cat_scratch;
};
hipError_t launch_grow_decide(const GrowParamsDev &G, uint32_t depth, SplitPacketDev *pk,
                              uint64_t *pk_cats, const LNodeDev *level, TreeNodeDev *tree,
                              uint64_t *tree_cats, const int8_t *monotone, const DevColumn *cols,
                              PartReqDev *reqs, PairDev *pairs, uint32_t *triples,
                              LeafDev *leaves, float *leaf_vals, GrowState *st,
                              const FusedArgmaxDev &A, hipStream_t s);
hipError_t launch_leaf_plan(LeafDev *leaves, GrowState *st, hipStream_t s);
// Leaves of a device-grown tree by a row-order walk over the single row
// bundle (feat_off[f]: byte offset of feature f in the bundle row, bit 15 set
// for 16-bit cells); at most MAX_WALK_NODES tree nodes. Workgroup 0 writes
// each leaf's position into its node (pad[1]). margin NULL: leaf ids only.
// bytes from a device view of coherent pinned host memory to device memory,
// as a kernel in the stream.
hipError_t launch_copy_bytes(void *dst, const void *src, uint64_t bytes, hipStream_t s);
// A grown tree's state, used nodes, category words and leaf values into a
// device view of pinned host memory, in stream order.
hipError_t launch_tree_out(const GrowState *st, const TreeNodeDev *tree, uint32_t tree_cap,
                           const uint64_t *cats, uint32_t cat_cap, const float *vals,
                           uint32_t leaf_cap, uint8_t *out, uint64_t o_tree, uint64_t o_cats,
                           uint64_t o_vals, hipStream_t s);
hipError_t launch_tree_leaves(const uint8_t *bundle, uint32_t pitch, uint64_t n_rows,
                              TreeNodeDev *tree, const uint64_t *tree_cats,
                              const uint16_t *feat_off, GrowState *st, void *ids, int id_bytes,
                              float *margin, float *delta, float *leaf_vals, hipStream_t s);
// order: the tree's feature positions, n_num numeric ones of at most 256
// bins first (one wave each, 4 bins a lane), then n_wide numeric ones of at
// most 1024 (one workgroup each, 4 bins a lane), then n_cat others,
// categorical or wider (one workgroup each). sub_triples set: the sibling
// subtraction of evaluated pairs (nodes 2e, 2e + 1; triples as
// launch_subtract's) is done by the scan, which stores the larger children's
// bins when write_big (the one-workgroup features always store them).
hipError_t launch_split_feats(int64_t *hist, uint64_t hist_width, const SplitNodeDev *nodes,
                              uint32_t n_nodes, const SplitFeatDev *feats, const uint32_t *order,
                              uint32_t n_num, uint32_t n_wide, uint32_t n_cat,
                              const uint8_t *enabled, SplitParamsDev P, FeatCandDev *cands,
                              uint64_t *cat_scratch, const uint32_t *dev_n,
                              const uint32_t *sub_triples, bool write_big, hipStream_t s);
// Chunk reduction (nodes of at most REDUCE_GROUP chunks), sibling
// subtraction and split scan of evaluated pairs in one pass, for trees whose
// features are all numeric of at most 256 bins (split_pair_kernel).
hipError_t launch_split_pairs(int64_t *hist, uint64_t hist_width, const int64_t *partials,
                              const HistNodeDev *hn, const uint32_t *triples, uint32_t n_pairs,
                              const SplitNodeDev *nodes, const SplitFeatDev *feats,
                              const uint32_t *order, uint32_t n_num, const uint8_t *enabled,
                              SplitParamsDev P, FeatCandDev *cands, const uint32_t *dev_n,
                              bool write, hipStream_t s);
hipError_t launch_split_nodes(const FeatCandDev *cands, const SplitFeatDev *feats,
                              uint32_t n_nodes, SplitParamsDev P, const SplitNodeDev *nodes,
                              const uint64_t *cat_scratch, SplitPacketDev *out,
                              uint64_t *cat_out, uint32_t cat_out_words, const uint32_t *dev_n,
                              hipStream_t s);
// Pass 1 (direction flags, left count per chunk) over a group of requests
// whose chunk_begin numbers the group's own chunks; counts land at count_base.
// A device-grown level's partition with its plan: count, scan + children
// plan (one workgroup), scatter (clearing Z's slots).
hipError_t launch_partition_level(const PartReqDev *reqs, const uint32_t *dev, uint32_t grid_chunks,
                                  const uint32_t *rows_in, uint32_t *rows_out, uint8_t *flags,
                                  uint32_t *counts, uint32_t *excl, uint32_t *totals,
                                  const uint64_t *cat_words, const PairDev *pairs, ChunkRule rule,
                                  HistNodeDev *hn, SplitNodeDev *sn, uint32_t *spans,
                                  uint32_t *left_slot, uint32_t *chunk_rows, const GrowDevOut &D,
                                  const ZeroNodesDev &Z, hipStream_t s);
// The same in one pass (part_split_kernel, cursors zeroed by the level
// decision), then the children plan (left totals from the cursors into
// totals). No slot is cleared: only for levels whose histograms need none.
hipError_t launch_partition_split(const PartReqDev *reqs, const uint32_t *dev,
                                  uint32_t grid_chunks, const uint32_t *rows_in,
                                  uint32_t *rows_out, unsigned long long *cursors,
                                  uint32_t *totals,
                                  const uint64_t *cat_words, const PairDev *pairs, ChunkRule rule,
                                  HistNodeDev *hn, SplitNodeDev *sn, uint32_t *spans,
                                  uint32_t *left_slot, uint32_t *chunk_rows, const GrowDevOut &D,
                                  hipStream_t s);
hipError_t launch_partition_count(const PartReqDev *reqs, uint32_t n_reqs, uint32_t n_chunks,
                                  const uint32_t *rows, uint8_t *flags, uint32_t *chunk_counts,
                                  const uint64_t *cat_words, hipStream_t s);
// Passes 2-4 (scan, stable scatter, copy back) over all requests of the call.
hipError_t launch_partition_finish(const PartReqDev *reqs, uint32_t n_reqs, uint32_t n_chunks,
                                   uint32_t *rows, uint32_t *tmp, const uint8_t *flags,
                                   const uint32_t *chunk_counts, uint32_t *chunk_offsets,
                                   uint32_t *totals, hipStream_t s);
// id_bytes 0: delta[row] = leaf value; 1 / 2: ids[row] = leaf position as
// u8 / u16.
// dev (nullable): {leaf count, chunks} read on the device; n_chunks is then
// the grid's upper bound.
hipError_t launch_assign_leaves(const LeafDev *leaves, uint32_t n_leaves, uint32_t n_chunks,
                                const uint32_t *rows, const uint32_t *rows_alt, float *delta,
                                void *ids, int id_bytes, const uint32_t *dev, hipStream_t s);
// margin[row] += values[ids[row]] over all rows (id_bytes 1 or 2).
hipError_t launch_apply_leaves(const void *ids, int id_bytes, const float *values, uint64_t n,
                               float *margin, hipStream_t s);
// Objective gradient pairs (f32, interleaved) from a per-row source value:
// mode 0: squared error from the margin (g = p - y, h = 1);
// mode 1: from the host's sigmoid s (g = s - y, h = max(s(1 - s), 1e-16));
// mode 2: as 1 with s computed on the device from the margin;
// mode 3: as 2 with the hardware exponential (gpu_math="fast");
// modes 4/5: softmax class cls of the margins src, from the round's per-row
// statistics (launch_softmax_stats), with glibc's expf restated (4) or the
// hardware exponential (5).
// All are multiplied by the row weight when w is non-null.
hipError_t launch_gradient(const float *src, const float *y, const float *w, uint64_t n,
                           int mode, float *g2n, uint64_t threshold, uint64_t seed, uint64_t tree,
                           double *block_max, uint32_t n_blocks, hipStream_t s,
                           const float2 *stats = nullptr, uint32_t cls = 0);
// Per row of K class-major margin columns: (largest margin from the smallest
// normal float up, float of the double sum of exp(m - that)).
hipError_t launch_softmax_stats(const float *margin, uint32_t K, uint64_t n, int fast,
                                float2 *stats, hipStream_t s);
hipError_t launch_sigmoid(const float *in, uint64_t n, float *out, hipStream_t s);
hipError_t launch_sigmoid_checksum(uint64_t begin, uint64_t end, unsigned long long *out,
                                   hipStream_t s, bool tanh = false);
// reg:quantileerror: the scale's per-row terms (exact: summed on the host),
// the (scale, alpha) slot the gradient's mode 6 reads, and the fast mode's
// fixed-order device reduction into that slot (partials: 512 doubles).
hipError_t launch_quantile_terms(const float *margin, const float *y, const float *w, uint64_t n,
                                 float *out, hipStream_t s);
hipError_t launch_quantile_set(float2 *slot, float scale, float alpha, hipStream_t s);
hipError_t launch_quantile_scale_fast(const float *margin, const float *y, const float *w,
                                      uint64_t n, float alpha, double *partials, float2 *slot,
                                      hipStream_t s);
hipError_t launch_fill_f32(float *p, float v, uint64_t n, hipStream_t s);
hipError_t launch_init_rows(uint32_t *rows, float *delta, uint64_t n, hipStream_t s);
// The gradients of a round quantized in the same pass under the previous
// round's scales (still in `scales`), then the bounds and this round's
// scales, then a pass that recomputes the pairs only if the scales changed:
// fixed-point pairs and block sums as gpair_quantize would give. g2n
// non-null: the (subsample-masked) f32 pairs are written there too; fixed
// may then be null (block sums only, the pairs quantized where they are read).
hipError_t launch_gradient_spec(const float *src, const float *y, const float *w, uint64_t n,
                                int mode, uint64_t th, uint64_t seed, uint64_t tree,
                                double *block_max, uint32_t n_blocks, ScalesDev *scales,
                                int64_t *fixed, int64_t *block_sum, float *g2n, hipStream_t s,
                                const float2 *stats = nullptr, uint32_t cls = 0);
hipError_t launch_gpair_maxabs(float *g2n, uint64_t n, uint64_t threshold, uint64_t seed,
                               uint64_t tree, double *block_max, uint32_t n_blocks,
                               hipStream_t s);
hipError_t launch_reduce_bounds(const double *block_max, uint32_t n_blocks, double *out_max,
                                uint64_t n_rows, ScalesDev *scales, hipStream_t s);
hipError_t launch_set_scales(ScalesDev *scales, double scale_g, double scale_h, hipStream_t s);
hipError_t launch_gpair_quantize(const float *g2n, uint64_t n, const ScalesDev *scales,
                                 int64_t *out, int64_t *block_sum, uint32_t n_blocks,
                                 int64_t *out_sum, hipStream_t s);
// The two most frequent codes of categorical bin columns (HOT_MAX_BINS codes
// at most), counted over up to `sample` rows spread evenly: out[4 f ..] =
// (first code, second code, first count, second count), ties to the lower
// code; HOT_NONE when a column has no second code.
constexpr uint32_t HOT_MAX_BINS = 4096;
struct CatColDev {
    const uint8_t *col;
    uint32_t width, n_bins;
};
hipError_t launch_cat_hot(const CatColDev *cols, uint32_t n_cols, uint64_t n_rows, uint32_t sample,
                          uint32_t *out, hipStream_t s);
hipError_t launch_pack_feature(const uint8_t *col, uint64_t n_rows, uint32_t width, uint8_t *tile,
                               uint32_t stride, uint32_t byte_off, hipStream_t s);

// One feature of the device binning: its cuts, bin count and width, and
// its resident bin column.
struct BinFeatDev {
    const float *cuts;
    uint8_t *col;
    uint32_t n_cuts;
    uint32_t n_bins;
    uint32_t width;        // 1 or 2
    uint32_t categorical;  // 1: code_to_bin instead of the cut search
};
// Bins rows [row0, row0 + n_rows) of the row-major f32 matrix x (device
// memory, the chunk's first row at x) into the features' columns.
hipError_t launch_bin_rows(const float *x, uint64_t n_rows, uint32_t n_features, uint64_t row0,
                           const BinFeatDev *feats, hipStream_t s);

// One interleaved tile of a tree's own features, packed from the bin
// columns: row r's record at out + r * stride, cell k copied from col[k]
// when bit k of `live` is set, else zero (col[k] is then any valid column).
struct PackTileDev {
    uint8_t *out;
    uint32_t stride;
    uint32_t live;
    const uint8_t *col[16];
};
// Records of n_tiles packed tiles of `width`-byte cells (device table, in
// row-bundle order: tiles b * 8 / width ... of bundle b share its rows).
hipError_t launch_pack_tiles(const PackTileDev *tiles, uint32_t n_tiles, uint32_t width,
                             uint64_t n_rows, hipStream_t s);

// Categories the device split scan sorts in LDS (weights + order, 32 KiB).
constexpr uint32_t MAX_DEVICE_CATS = 4096;
// Distinct split features of one tree the TreeSHAP kernel accepts.
constexpr uint32_t MAX_SHAP_UNIQUE = 1024;

}  // namespace fbh
