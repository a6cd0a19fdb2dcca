// fbhip_ctx.hip -- the training context behind the fbh_* C ABI (include/fbhip.h).
//
// A context owns every device buffer of one training run, allocated once at
// creation (GpuTrainCtx::new_with_shape, src/backend/cuda/train_ctx.rs:728):
//   tiles      the training matrix as LDS-sized tiles of row records
//   gpair      i64 [n_rows][2] fixed-point gradient pairs (+ f32 staging)
//   rows       u32 [n_rows] row arena (+ temporary arena and u8 flags)
//   delta      f32 [n_rows] per-row leaf value of the current tree
//   hist       i64 [slots][width][2] node histograms kept on the device
// All work runs in order on one HIP stream; the host blocks only where a
// result must come back (scales, root sum, split packets, left counts).

#include "fb_expf.h"
#include "fbhip_internal.h"
#include "../../include/fbhip.h"

#include <algorithm>
#include <cmath>
#include <deque>
#include <future>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <cstring>
#include <limits>
#include <memory>
#include <stdexcept>
#include <thread>
#include <string>
#include <vector>

using namespace fbh;

namespace {

thread_local std::string g_err;

struct InputError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct RuntimeError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void check(hipError_t e, const char *what) {
    if (e != hipSuccess)
        throw RuntimeError(std::string(what) + ": " + hipGetErrorString(e));
}

template <class F>
int guard(F &&f) {
    try {
        f();
        return FBH_OK;
    } catch (const InputError &e) {
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

uint64_t env_u64(const char *name, uint64_t dflt) {
    const char *v = std::getenv(name);
    if (!v || !*v) return dflt;
    char *end = nullptr;
    unsigned long long x = std::strtoull(v, &end, 10);
    return (end && *end == 0) ? (uint64_t)x : dflt;
}

// Record sizes the histogram kernel is instantiated for.
uint32_t round_stride(uint32_t bytes) {
    static const uint32_t allowed[] = {4, 8, 12, 16, 32, 48, 64};
    for (uint32_t a : allowed)
        if (bytes <= a) return a;
    return 0;
}

constexpr uint32_t MAX_RECORD_BYTES = 64;
// Largest per-chunk partial histogram buffer (also bounded by the budget's
// remaining room). Wide-bin 2M x 100 needs about 360 MB at its root; with
// 256 MB its 7,440 root workgroups flushed with global atomics instead.
constexpr uint64_t MAX_PARTIAL_BYTES = 2048ull << 20;
constexpr uint32_t MAX_NODES = 16384;      // nodes of one eval / partition call
// A level of a device-grown tree partitions in one pass (part_split_kernel)
// when its partition chunks, divided by the level's node bound (2^depth),
// number at most this many. Each workgroup reserves its places with one
// atomic on its node's cursor pair, and the atomics on one cursor serialize
// (about 14 ns each measured: 74 us for 5128 chunks of one node, against
// 56 us for the count, scan and scatter passes).
constexpr uint32_t ONE_PASS_CHUNKS_PER_NODE = 512;
// Histogram slots of at least this many bytes take the one-pass chunk
// reduction, subtraction and split scan of evaluated pairs (split_pair_kernel)
// when every tree feature allows it. Measured on one box over the first 25
// rounds: 400k x 2000 (4 MB slots) 351 -> 361 rounds/s, 10.5M x 28 (114 KB
// slots) 490 -> 480.
constexpr uint64_t PAIR_PASS_MIN_SLOT_BYTES = 1u << 20;
constexpr uint32_t DEFAULT_TILE_BYTES = 64 * 1024;
// LDS of a planar tile (its bins plus the 1 KiB of lane dummies) when the
// caller sets no tile size: three workgroups then share a CU's 160 KiB,
// which the loads of tiles with few wide-bin features need (2M rows x 80
// features of 1024 bins: 254 against 340 us a histogram).
constexpr uint32_t PLANAR_TILE_BYTES = 53 * 1024;
// Device-grown trees of at most this many features pick each node's best
// split inside the level decision instead of a separate argmax launch; trees
// of at most FUSED_STAGED_FEATS do so at the levels whose candidates the
// decision stages in LDS (DECIDE_CAND_LDS).
constexpr size_t FUSED_ARGMAX_FEATS = 64;
constexpr size_t FUSED_STAGED_FEATS = 256;
// Row layouts of at most this many tiles histogram f32 pairs (fbh_ctx::f32_hist).
constexpr size_t F32_PAIR_MAX_TILES = 4;
// Rows per histogram workgroup: chosen per launch so that the launch makes
// one full wave of workgroups (HIST_WAVES), never fewer than MIN_CHUNK_ROWS
// rows: each workgroup then flushes its LDS histogram once per launch.
constexpr uint32_t MIN_CHUNK_ROWS = 4096;
// Rows per chunk at most when more than four tiles share a row bundle.
constexpr uint32_t SHARED_LINE_CHUNK_ROWS = 8192;
// Row chunks of the per-round gradient exchange (download, host work and
// upload of different chunks overlap).
constexpr int EXCHANGE_CHUNKS = 8;
constexpr uint32_t HIST_WAVES = 1;
// Device-planned launches of layouts with planar tiles plan two waves: their
// workgroups hold fewer rows each and the second wave overlaps the first's
// flushes (wide-bin 2M x 100 rounds 5-24: 545 against 571 rounds/s; the
// interleaved layouts of 10.5M x 28 and 400k x 2000 lost 7 % and 6 % with
// two).
constexpr uint32_t PLANAR_HIST_WAVES = 2;
// Host-driven evaluations (lossguide expansions, host levels) accumulate
// fewer rows per launch; two waves of workgroups measured faster there
// (wide-bin lossguide: 107 against 99 rounds/s).
constexpr uint32_t HOST_HIST_WAVES = 2;

struct DeviceBuf {
    void *p = nullptr;
    size_t bytes = 0;
};

struct PinnedBuf {
    void *p = nullptr;
    size_t bytes = 0;
    void *dev = nullptr;  // device view of a mapped (coherent) buffer
};

}  // namespace

namespace fbh {
void set_last_error(const char *msg) { g_err = msg; }
const char *last_error() { return g_err.c_str(); }
}  // namespace fbh

struct fbh_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    uint64_t n_rows = 0;
    uint32_t n_features = 0;
    std::vector<uint8_t> width, cat;
    std::vector<uint32_t> n_bins;
    uint32_t tile_bytes = DEFAULT_TILE_BYTES;
    uint32_t planar_tile_bytes = PLANAR_TILE_BYTES;
    uint32_t fixed_chunk_rows = 0;  // nonzero: rows per workgroup forced by the caller
    uint32_t shared_line_rows = SHARED_LINE_CHUNK_ROWS;
    uint32_t planar_max_feats = 0;  // nonzero: at most this many features a planar tile
    uint64_t max_partial_bytes = MAX_PARTIAL_BYTES;
    uint32_t one_pass_chunks = ONE_PASS_CHUNKS_PER_NODE;  // 0: never one pass
    bool pair_pass = true;          // split_pair_kernel where EvalPlan::pairs allows it
    bool sub_in_scan = true;        // sibling subtraction inside split_num_kernel, likewise
    uint32_t hist_tpb = 0;          // histogram threads per workgroup (0: per launch)
    uint32_t hist_waves = 0;  // 0: HIST_WAVES, PLANAR_HIST_WAVES with planar tiles
    uint32_t host_hist_waves = HOST_HIST_WAVES;
    uint32_t n_cus = 256;
    uint32_t n_slots = 0;
    uint32_t max_cat_words = 0;
    uint64_t width_max = 0;  // sum of all features' bins
    uint64_t device_bytes = 0;
    std::vector<DeviceBuf> allocs;

    struct Tile {
        uint32_t width;
        uint32_t rec;     // record bytes per row (the kernel's record size)
        uint32_t stride;  // bytes from one row's record to the next
        std::vector<uint32_t> feats;  // ascending global ids
        uint8_t *data;
        bool global;  // one feature too wide for LDS: global-memory atomics
        bool resident = true;      // records in HBM; else streamed from host
        uint8_t *host = nullptr;   // pinned host records of a streamed tile
        int32_t bundle = -1;       // row bundle holding the records, or -1
        uint32_t bundle_off = 0;   // offset of the record in the bundle row
        bool rot = false;          // interleaved LDS layout (16 cells a record)
        // The tile's records again, tile-major (row r at tm + r * rec): the
        // root of a tree whose tiles share bundle lines reads these, where
        // its rows are in order, so its chunks need no shared lines in L2.
        uint8_t *tm = nullptr;
    };
    std::vector<Tile> tiles;
    bool tm_stale = false;  // some tile's records changed after its tile-major copy was made
    // Hot bins of categorical features (TileFeatDev::hot), found once from
    // the resident bin columns after the last upload.
    std::vector<uint32_t> hot_a, hot_b;
    bool hot_ready = false;
    // Packed tiles of the current tree: with column sampling, the tree's
    // features of interleaved tiles are packed 16 to a record (from the bin
    // columns, into `pack`) when that takes at most 3/4 of the tiles that
    // hold them, so the histograms read and add no unsampled cells.
    std::vector<Tile> pack_tiles;
    uint8_t *pack = nullptr;
    uint64_t pack_bytes = 0;
    std::vector<uint32_t> pack_sig;  // features (and width marks) the pack holds now
    // Device binning (fbh_set_cuts / fbh_upload_rows): the cuts and feature
    // table, and the row staging, all outside the memory plan.
    BinFeatDev *d_binfeats = nullptr;
    float *d_cut_values = nullptr;
    float *rows_stage = nullptr;
    bool cuts_set = false;
    // Device binning under a plan that does not keep the bin columns: a
    // chunk's bins land in bin_stage (feature f's column of stage_rows()
    // cells at byte bin_off[f], 256-aligned), resident tiles are packed from
    // there and streamed tiles' records are packed in rec_stage and copied
    // to their pinned host memory.
    uint8_t *bin_stage = nullptr, *rec_stage = nullptr;
    std::vector<uint64_t> bin_off;
    uint64_t bin_stage_bytes() const {
        uint64_t cols = 0, stride = 0;
        for (uint32_t f = 0; f < n_features; f++)
            cols += (stage_rows() * width[f] + 255) & ~uint64_t(255);
        for (const auto &t : tiles)
            if (!t.resident) stride = std::max<uint64_t>(stride, t.stride);
        return cols + stage_rows() * stride + 512;
    }
    // Rows the staging holds: 64 MiB of rows, at least 64 rows.
    uint64_t stage_rows_cap = 0;  // nonzero: rows of the row staging (FB_HIP_STAGE_ROWS)
    uint64_t stage_rows() const {
        const uint64_t per = 4ull * std::max<uint32_t>(n_features, 1);
        const uint64_t cap = stage_rows_cap ? stage_rows_cap : (64ull << 20) / per;
        return std::max<uint64_t>(64, std::min<uint64_t>(n_rows, cap));
    }
    // Row bundles: consecutive LDS tiles whose records fit in one 128-byte
    // cache line share one allocation, row r's records together at data +
    // r * pitch (a power of two, so no row straddles two lines). A histogram
    // over a scattered node then fetches one line per row for the whole
    // bundle instead of one per tile, and a line holds no other row when the
    // pitch is 128 (the tiles of a bundle run side by side on one XCD). Used
    // when every tile is resident. The gradient pairs stay a separate array:
    // they are rewritten every round, and a partial-line write costs a full
    // line.
    struct Bundle {
        uint32_t pitch;
        uint8_t *data;
    };
    std::vector<Bundle> bundles;
    bool bundled = false;
    std::vector<int32_t> feat_tile, feat_pos;
    // Column-major bins of every feature, when the plan keeps them (the
    // partition reads one cell per row: rows of the nodes splitting on one
    // feature share cache lines).
    std::vector<uint8_t *> cols;
    fbh_plan plan{};
    // Streaming (plan.staging_bytes > 0): pinned host columns of the features
    // of streamed tiles, two device windows for records and two for columns,
    // a copy stream and the events that hand the windows back and forth.
    std::vector<uint8_t *> host_cols;
    uint8_t *win_rec[2] = {nullptr, nullptr};
    uint8_t *win_col[2] = {nullptr, nullptr};
    hipStream_t copy_stream = nullptr;
    hipEvent_t win_ready[4] = {}, win_free[4] = {};
    std::vector<void *> host_allocs;
    std::vector<uint8_t> uploaded;

    float *gpair_f32 = nullptr;
    // gpair_f32 holds the f32 pairs that quantize to gpair under d_scales:
    // histograms of scattered rows read those instead (half the bytes).
    bool f32_pairs = false;
    // Every tile's workgroup quantizes the pairs it reads again, so f32
    // pairs pay only with few tiles (measured: 2 tiles +3 %, 33 tiles -6 %).
    bool f32_hist() const { return tiles.size() <= F32_PAIR_MAX_TILES; }
    // launch_gradient mode of the device objective.
    int gradient_mode() const {
        if (objective == 3) return 6;
        if (objective == 2) return fast_math ? 5 : 4;
        return objective == 0 ? 0 : (fast_math ? 3 : 2);
    }
    int64_t *gpair = nullptr;
    bool root_on_device = false;  // the last quantisation's root sum is on the device
    uint32_t *rows = nullptr, *tmp = nullptr;
    uint8_t *flags = nullptr;
    float *delta = nullptr;
    int64_t *hist = nullptr;
    ScalesDev *d_scales = nullptr;  // scales of the current gradients
    int64_t *partials = nullptr;    // per-chunk partial histograms
    uint64_t partial_bytes = 0;
    unsigned long long *d_cursors = nullptr;  // cursor pairs of the one-pass partition
    // The row arena of a new tree is the identity; it is written out only
    // when something reads it (a device-grown tree walks the root without it).
    bool rows_identity = false;
    double *red_f64 = nullptr;
    int64_t *red_i64 = nullptr;
    uint32_t n_red_blocks = 8192;  // blocks of the bounds and quantisation passes

    // launch tables (device) and their pinned staging
    TileDev *d_tiles = nullptr;
    TileFeatDev *d_tilefeats = nullptr;
    SplitFeatDev *d_sfeats = nullptr;
    uint8_t *d_stage = nullptr;  // device copy of the pinned launch-table staging
    FeatCandDev *d_cands = nullptr;
    uint64_t *d_cat_scratch = nullptr;
    SplitPacketDev *d_packets = nullptr;
    uint32_t *d_counts = nullptr, *d_excl = nullptr, *d_totals = nullptr;
    LeafDev *d_leaves = nullptr;
    // Tables a fused partition + evaluation step plans on the device.
    HistNodeDev *d_lvl_hist = nullptr;
    SplitNodeDev *d_lvl_split = nullptr;
    uint32_t *d_lvl_out = nullptr;  // spans (4 per pair), then left slots (1 per pair)
    uint32_t *d_lvl_rows = nullptr; // rows per chunk of the planned launch
    // Device-grown depthwise trees (fbh_grow_depthwise): buffers sized for
    // the deepest tree asked for so far, allocated on first use.
    struct Grow {
        uint32_t depth = 0;  // capacity: trees up to this depth
        size_t level_cap = 0, tree_cap = 0, leaf_cap = 0, cat_cap = 0;
        GrowState *st = nullptr;
        LNodeDev *level[2] = {nullptr, nullptr};
        TreeNodeDev *tree = nullptr;
        uint64_t *tree_cats = nullptr;
        PartReqDev *reqs = nullptr;
        PairDev *pairs = nullptr;
        uint32_t *triples = nullptr;
        LeafDev *leaves = nullptr;
        float *leaf_vals = nullptr;
        DevColumn *cols = nullptr;
        uint16_t *feat_off = nullptr;  // byte offset of each feature in the row bundle (leaf walk)
        // The root's accumulation table (offset 0) and the monotone
        // constraints (offset 256) on the device, with the host copies they
        // were last uploaded from.
        uint8_t *root_tables = nullptr;
        HistNodeDev h_root_hn{};
        std::vector<int8_t> h_mono;
        // Two result slots (state, tree, category words, leaf values), so a
        // tree can be collected while the next one is already enqueued.
        PinnedBuf out[2];
        uint8_t *out_dev[2] = {nullptr, nullptr};  // device views of out
        hipEvent_t done[2] = {nullptr, nullptr};
        uint64_t next_slot = 0;
        struct Job {
            int slot;
            uint32_t cat_words;  // category words per node of the tree's features
        };
        std::deque<Job> pending;
    } grow;
    // offsets in the tree-table buffer
    size_t off_tilefeats = 0, off_sfeats = 0, off_order = 0, off_pack = 0, off_root = 0,
           tables_bytes = 0;
    PackTileDev *d_pack = nullptr;  // the packed tiles' sources (tree tables)
    uint32_t *d_split_order = nullptr;  // tree features: numeric positions, then categorical
    uint32_t n_split_num = 0, n_split_wide = 0, n_split_cat = 0;
    size_t stage_bytes = 0;
    uint64_t max_chunks = 0;    // capacity of the partition chunk arrays
    uint64_t cat_in_words = 0;  // capacity of the partition category words

    // Pinned staging of launch tables going to the device: a ring of slots,
    // each reused only after the copy out of it has run, so a call can
    // return while its tables are still on their way.
    static constexpr int STAGE_SLOTS = 4;
    PinnedBuf pin_stage[STAGE_SLOTS];
    hipEvent_t stage_ev[STAGE_SLOTS] = {};
    int stage_next = 0;
    PinnedBuf pin_leaves;  // leaf tables (asynchronous call)
    PinnedBuf pin_out;     // results coming back
    size_t pin_out_spans = 0;  // offset of a fused step's spans in pin_out
    hipEvent_t leaves_done = nullptr;
    bool leaves_pending = false;

    // per tree
    std::vector<uint8_t> tree_tables;  // the tree tables last sent to the device
    std::vector<uint32_t> tree_feats;
    std::vector<int64_t> hist_off;  // global feature -> compact offset, -1 if not built
    uint64_t hist_width = 0;
    std::vector<int8_t> monotone;
    struct Group {
        int width, rd;
        uint32_t tile_begin, n_tiles;
        uint32_t lds_max;
        uint32_t bytes_per_row;  // active feature bytes of the group's tiles
        bool global;
        bool rot;
    };
    std::vector<Group> groups;
    struct Streamed {
        uint32_t tile;         // index in tiles
        uint32_t entry;        // index of its TileDev in the tree's table
        uint32_t lds_slots;
        uint32_t bytes_per_row;
    };
    std::vector<Streamed> streamed;  // streamed tiles with active features this tree
    uint64_t win_flip = 0;           // alternates the record windows
    uint64_t col_flip = 0;           // alternates the column windows
    uint32_t n_windows = 2;          // streaming windows of each kind (hist_streams)
    uint32_t resident_cap = UINT32_MAX;  // tiles the plan may keep resident (resident_blocks)
    uint64_t streamed_bytes = 0;     // host-to-device bytes of streamed records and columns
    bool has_global = false;  // this tree builds a feature with global atomics
    uint32_t hist_row_bytes = 0;  // active cell bytes per row over all built tiles
    uint32_t hist_tiles = 0;      // resident tiles with features built this tree
    uint32_t line_share = 1;      // most built tiles sharing one row bundle this tree
    // The tree's root reads tile-major copies (d_root_tiles): every built
    // tile is planar, resident and has one, and its tiles share bundle lines.
    bool root_tm = false;
    TileDev *d_root_tiles = nullptr;
    uint64_t bins_active = 0;     // bins of the tree's features
    uint32_t cat_words_per_node = 0;
    bool tree_begun = false;
    double scales[2] = {1.0, 1.0};

    // objective state on the device (fbh_set_objective, fbh_set_multiclass)
    int objective = -1;                 // -1 none, 0 squared error, 1 logistic, 2 softmax,
                                        // 3 quantile
    uint32_t n_outputs = 1;             // margin columns (class-major), as planned
    uint32_t out_k = 0;                 // the column gradients read and leaves update
    float2 *softmax_stats = nullptr;    // per-row (wmax, wsum) of the round (softmax)
    float2 *quantile_slot = nullptr;    // (scale, alpha) of the current output (quantile)
    std::vector<float> alphas;          // quantile_alpha of each output
    double quantile_sum_w = 0.0;        // the serial double sum of the weights (or n)
    float quantile_scale = 0.0f;        // the last scale taken (exact mode)
    // Exact scales of several outputs, summed on host threads side by side:
    // output j's margins change only with output j's own trees, so every
    // output's sum can start when the first of them is needed.
    std::vector<std::future<double>> q_sums;  // output j's pending or finished sum
    std::vector<uint8_t> q_have;        // q_sums[j] is for output j's current margins
    float *q_terms = nullptr;           // n_outputs x n_rows terms (device)
    PinnedBuf pin_q;                    // the same terms on the host
    // A worker's error of a sum dropped before anyone took it (the first
    // one), raised by the next quantile scale instead of being lost.
    std::exception_ptr q_error;
    void q_forget(int k) {              // k < 0: every output
        for (size_t j = 0; j < q_sums.size(); j++) {
            if (k >= 0 && j != (size_t)k) continue;
            if (q_sums[j].valid()) {
                try {
                    q_sums[j].get();
                } catch (...) {
                    if (!q_error) q_error = std::current_exception();
                }
            }
            q_sums[j] = std::future<double>();
            q_have[j] = 0;
        }
    }
    void q_raise() {
        if (!q_error) return;
        std::exception_ptr e = q_error;
        q_error = nullptr;
        std::rethrow_exception(e);
    }
    float *cur_margin() const { return margin + (uint64_t)out_k * n_rows; }
    bool fast_math = false;             // gpu_math="fast": hardware exp in the logistic gradient
    float *labels = nullptr, *gweights = nullptr, *margin = nullptr;
    void *leaf_ids = nullptr;           // per-row leaf position of the last tree
    int leaf_id_bytes = 0;              // 1 or 2 for the last assigned tree
    bool ids_fresh = false;             // leaf ids not yet handed to the host
    bool leaves_deferred = false;       // the last grown tree's values are not in the margins yet
    bool has_weights = false;
    float *sig = nullptr;               // the host's per-row sigmoids (logistic)
    PinnedBuf pin_ids, pin_src;         // leaf-id download / sigmoid upload staging
    hipStream_t up_stream = nullptr;    // host-to-device copies of the exchange
    std::vector<hipEvent_t> chunk_ev;   // one per exchange chunk
    hipEvent_t up_done = nullptr;

    // timing
    bool timing = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev_pool;
    size_t ev_used = 0;
    double hist_ms = 0.0;
    uint64_t hist_launches = 0, hist_bytes = 0;

    ~fbh_ctx() { release(); }

    void release() {
        q_forget(-1);  // the sums read pin_q and wait on chunk_ev
        if (device >= 0) (void)hipSetDevice(device);
        if (stream) (void)hipStreamSynchronize(stream);
        for (auto &a : allocs)
            if (a.p) (void)hipFree(a.p);
        allocs.clear();
        for (int k = 0; k < STAGE_SLOTS; k++) {
            if (pin_stage[k].p) (void)hipHostFree(pin_stage[k].p);
            pin_stage[k].p = nullptr;
            if (stage_ev[k]) (void)hipEventDestroy(stage_ev[k]);
            stage_ev[k] = nullptr;
        }
        if (pin_leaves.p) (void)hipHostFree(pin_leaves.p);
        if (pin_out.p) (void)hipHostFree(pin_out.p);
        for (int k = 0; k < 2; k++) {
            if (grow.out[k].p) (void)hipHostFree(grow.out[k].p);
            grow.out[k].p = nullptr;
            if (grow.done[k]) (void)hipEventDestroy(grow.done[k]);
            grow.done[k] = nullptr;
        }
        if (pin_ids.p) (void)hipHostFree(pin_ids.p);
        if (pin_src.p) (void)hipHostFree(pin_src.p);
        if (pin_q.p) (void)hipHostFree(pin_q.p);
        pin_leaves.p = pin_out.p = pin_ids.p = pin_src.p = pin_q.p = nullptr;
        q_terms = nullptr;
        if (copy_stream) (void)hipStreamSynchronize(copy_stream);
        for (void *h : host_allocs) (void)hipHostFree(h);
        host_allocs.clear();
        for (int k = 0; k < 4; k++) {
            if (win_ready[k]) (void)hipEventDestroy(win_ready[k]);
            if (win_free[k]) (void)hipEventDestroy(win_free[k]);
            win_ready[k] = win_free[k] = nullptr;
        }
        if (copy_stream) (void)hipStreamDestroy(copy_stream);
        copy_stream = nullptr;
        if (up_stream) (void)hipStreamSynchronize(up_stream);
        for (auto e : chunk_ev) (void)hipEventDestroy(e);
        chunk_ev.clear();
        if (up_done) (void)hipEventDestroy(up_done);
        up_done = nullptr;
        if (up_stream) (void)hipStreamDestroy(up_stream);
        up_stream = nullptr;
        for (auto &e : ev_pool) {
            (void)hipEventDestroy(e.first);
            (void)hipEventDestroy(e.second);
        }
        ev_pool.clear();
        if (leaves_done) (void)hipEventDestroy(leaves_done);
        leaves_done = nullptr;
        if (stream) (void)hipStreamDestroy(stream);
        stream = nullptr;
    }

    template <class T>
    T *alloc(size_t count, const char *what) {
        size_t bytes = std::max<size_t>(count * sizeof(T), 256);
        void *p = nullptr;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess)
            throw RuntimeError(std::string("device allocation of ") + what + " (" +
                               std::to_string(bytes) + " bytes) failed: " + hipGetErrorString(e));
        allocs.push_back({p, bytes});
        device_bytes += bytes;
        return static_cast<T *>(p);
    }

    // Frees a buffer alloc() made, once the stream has finished with it.
    void release_alloc(void *p) {
        if (!p) return;
        sync();
        for (size_t i = 0; i < allocs.size(); i++)
            if (allocs[i].p == p) {
                (void)hipFree(p);
                device_bytes -= allocs[i].bytes;
                allocs.erase(allocs.begin() + (long)i);
                return;
            }
    }

    // Per-chunk partial histograms (see HistLaunch::partials) of `bytes`, or
    // NULL when a launch cannot use them (global or streamed tiles), they
    // would exceed MAX_PARTIAL_BYTES or the memory budget has no room left
    // for them; grown on demand. Without them launches flush with atomics.
    int64_t *partial_buffer(uint64_t bytes);

    void pinned(PinnedBuf &b, size_t bytes) {
        check(hipHostMalloc(&b.p, bytes, hipHostMallocDefault), "pinned host allocation");
        b.bytes = bytes;
    }
    // Coherent pinned memory that kernels read through its device view:
    // host-to-device sends then run as a kernel in the compute stream
    // (send_mapped) instead of a copy-engine transfer, whose handoff between
    // engines stalls the queue for tens of microseconds.
    void pinned_mapped(PinnedBuf &b, size_t bytes) {
        check(hipHostMalloc(&b.p, bytes, hipHostMallocCoherent), "pinned host allocation");
        b.bytes = bytes;
        check(hipHostGetDevicePointer(&b.dev, b.p, 0), "device view of pinned memory");
    }
    void send_mapped(void *dst, const PinnedBuf &b, size_t bytes) {
        check(launch_copy_bytes(dst, b.dev, bytes, stream), "launch tables");
    }

    uint8_t *host_alloc(size_t bytes, const char *what) {
        void *p = nullptr;
        hipError_t e = hipHostMalloc(&p, std::max<size_t>(bytes, 64), hipHostMallocDefault);
        if (e != hipSuccess)
            throw RuntimeError(std::string("pinned host allocation of ") + what + " (" +
                               std::to_string(bytes) + " bytes) failed: " + hipGetErrorString(e));
        host_allocs.push_back(p);
        return static_cast<uint8_t *>(p);
    }

    void sync() { check(hipStreamSynchronize(stream), "stream synchronize"); }

    // The row arena written out (rows in order) if the tree has not yet.
    void ensure_rows();
    // The cell value that means missing for feature f (see PartReqDev::missing).
    uint32_t missing_code(uint32_t f) const {
        return width[f] == 2 ? 0xFFFFu : (n_bins[f] > 255 ? 0x100u : 0xFFu);
    }

    // The next staging slot, once the copy that last read it has run.
    uint8_t *stage_acquire(int &slot) {
        slot = stage_next;
        stage_next = (stage_next + 1) % STAGE_SLOTS;
        check(hipEventSynchronize(stage_ev[slot]), "staging reuse");
        return static_cast<uint8_t *>(pin_stage[slot].p);
    }
    // Copies `bytes` of the slot to dst in stream order; marks the slot busy.
    void stage_send(int slot, void *dst, size_t bytes) {
        send_mapped(dst, pin_stage[slot], bytes);
        check(hipEventRecord(stage_ev[slot], stream), "event");
    }

    // Threads of a histogram workgroup of group g: 512 when the LDS lets
    // three or more workgroups share a CU (planar tiles of few wide-bin
    // features: the rows' loads then need more waves in flight; measured
    // on 2M rows x 80 features of 1024 bins, 254 against 340 us), and for
    // interleaved tiles in groups of more than F32_PAIR_MAX_TILES tiles
    // (their rows gather 16-byte pairs once a tile, and two workgroups a CU
    // leave those loads short of waves: 400k x 2000 at 1000 features a tree
    // 391 -> 408 rounds/s), else 256 (C2's two interleaved tiles: LDS-atomic
    // bound at the root, 512 threads lost 2 %).
    int hist_threads(const Group &g) const {
        if (hist_tpb) return (int)hist_tpb;
        if (g.rot) return g.n_tiles > F32_PAIR_MAX_TILES ? 512 : 256;
        const uint64_t lds = (uint64_t)(g.lds_max + 64) * 16;
        return 3 * lds <= 160u * 1024u ? 512 : 256;
    }

    // Rows per histogram workgroup for a launch accumulating acc_rows rows:
    // enough chunks for hist_waves full waves of workgroups over all tiles
    // (occupancy bounded by LDS and by 2048 threads per CU), so that each
    // workgroup flushes its LDS histogram once per many rows.
    ChunkRule chunk_rule(bool host = false, bool own_lines = false) const {
        ChunkRule R{fixed_chunk_rows, 1, MIN_CHUNK_ROWS, 1u << 24};
        uint64_t n_tiles = 0, lds_max = 0;
        bool planar = false;
        for (const auto &g : groups) {
            n_tiles += g.n_tiles;
            if (!g.global) lds_max = std::max<uint64_t>(lds_max, (uint64_t)(g.lds_max + 64) * 16);
            planar = planar || (!g.global && !g.rot);
        }
        if (n_tiles == 0) return R;
        uint64_t per_cu = lds_max ? (160u * 1024u) / lds_max : 8;
        per_cu = std::max<uint64_t>(1, std::min<uint64_t>(per_cu, 2048 / (hist_tpb ? hist_tpb : 256)));
        const uint32_t waves =
            host ? host_hist_waves
                 : (hist_waves ? hist_waves : (planar ? PLANAR_HIST_WAVES : HIST_WAVES));
        const uint64_t wgs = (uint64_t)n_cus * per_cu * waves;
        R.want_chunks = (uint32_t)std::max<uint64_t>(1, wgs / n_tiles);
        // Many tiles reading one bundle line: short chunks, so the tiles'
        // workgroups of a chunk stay close enough in the rows for the line
        // to be read once into L2 (wide-bin 2M x 100, 16 tiles a line:
        // 394 against 343 rounds/s; with 2 or 4 tiles a line the longer
        // default chunks are faster).
        if (line_share > 4 && !own_lines) R.max_rows = shared_line_rows;
        return R;
    }
    // Rows per chunk for accumulated nodes of these lengths: the smallest
    // multiple of 1024 whose chunks (ceil(len / rows) per node) fit one wave
    // of workgroups, so no launch runs a second, mostly idle wave; with more
    // nodes than the wave holds, rows / want_chunks rounded up.
    uint32_t chunk_rows_for(const uint32_t *lens, size_t n, bool host = false,
                            bool own_lines = false) const {
        const ChunkRule R = chunk_rule(host, own_lines);
        if (R.fixed) return R.fixed;
        uint64_t acc = 0, nz = 0;
        for (size_t i = 0; i < n; i++) {
            acc += lens[i];
            nz += lens[i] ? 1 : 0;
        }
        uint64_t lo = (acc + (uint64_t)R.want_chunks * 1024 - 1) / ((uint64_t)R.want_chunks * 1024);
        lo = std::max<uint64_t>(lo, 1);
        if (R.want_chunks > nz) {
            const uint64_t room = R.want_chunks - nz;
            uint64_t hi = (acc + room * 1024 - 1) / (room * 1024);
            hi = std::max(hi, lo);
            while (lo < hi) {
                const uint64_t mid = (lo + hi) / 2, rows = mid * 1024;
                uint64_t k = 0;
                for (size_t i = 0; i < n; i++) k += (lens[i] + rows - 1) / rows;
                if (k <= R.want_chunks) hi = mid;
                else lo = mid + 1;
            }
        }
        return (uint32_t)std::min<uint64_t>(std::max<uint64_t>(lo * 1024, R.min_rows), R.max_rows);
    }
    uint32_t chunk_rows_for(uint64_t rows, bool own_lines = false) const {
        const uint32_t len = (uint32_t)rows;
        return chunk_rows_for(&len, 1, false, own_lines);
    }

    // Adds the histogram time of every completed launch; pairs still in
    // flight (a tree enqueued behind the one collected) stay for later.
    void collect_timing() {
        size_t keep = 0;
        for (size_t i = 0; i < ev_used; i++) {
            if (hipEventQuery(ev_pool[i].second) != hipSuccess) {
                std::swap(ev_pool[keep], ev_pool[i]);
                keep++;
                continue;
            }
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, ev_pool[i].first, ev_pool[i].second) == hipSuccess)
                hist_ms += ms;
        }
        ev_used = keep;
    }
};

int64_t *fbh_ctx::partial_buffer(uint64_t bytes) {
    if (has_global || !streamed.empty() || bytes > max_partial_bytes) return nullptr;
    // Outside the memory plan: only within the budget's remaining room.
    if (bytes > partial_bytes && device_bytes - partial_bytes + bytes + 256 > plan.budget)
        return nullptr;
    if (bytes > partial_bytes) {
        release_alloc(partials);
        partials = alloc<int64_t>(bytes / 8 + 1, "partial histograms");
        partial_bytes = bytes;
    }
    return partials;
}

void fbh_ctx::ensure_rows() {
    if (!rows_identity) return;
    check(launch_init_rows(rows, objective >= 0 ? nullptr : delta, n_rows, stream),
          "row arena reset");
    rows_identity = false;
}

namespace {

// Features of `width` bytes that go to interleaved tiles: at least 9 of
// them (fewer fill a compact planar record better), 8-bit ones or 16-bit
// ones of at most HIST_ROT_BINS bins; none when the tile budget is below the
// interleaved layout's.
std::vector<uint32_t> rot_features(const fbh_ctx &c, uint32_t w,
                                   const std::vector<uint32_t> &feats) {
    std::vector<uint32_t> out;
    if (c.tile_bytes < DEFAULT_TILE_BYTES) return out;
    for (uint32_t f : feats)
        if (c.width[f] == w && c.n_bins[f] <= HIST_ROT_BINS) out.push_back(f);
    if (out.size() < 9) out.clear();
    return out;
}

// Interleaved tiles holding `feats` (16-cell records), the features spread
// evenly over ceil(n / 16) tiles so that no tile is left nearly empty.
template <class F>
void rot_tiles(uint32_t w, const std::vector<uint32_t> &feats, F &&emit) {
    const size_t n = feats.size(), nt = (n + 15) / 16;
    for (size_t i = 0; i < nt; i++) {
        fbh_ctx::Tile t{w, 16 * w, 16 * w, {}, nullptr, false};
        t.rot = true;
        for (size_t k = n * i / nt; k < n * (i + 1) / nt; k++) t.feats.push_back(feats[k]);
        emit(std::move(t));
    }
}

// LDS bytes of a planar feature: its bins, plus the lane slots of its hot
// bins for a categorical feature that may have them.
uint64_t feature_lds_bytes(const fbh_ctx &c, uint32_t f) {
    uint64_t b = (uint64_t)c.n_bins[f] * 16u;
    if (c.cat[f] && c.n_bins[f] >= 2 && c.n_bins[f] <= HOT_MAX_BINS) b += HOT_SLOTS * 16u;
    return b;
}

void plan_tiles(fbh_ctx &c) {
    c.feat_tile.assign(c.n_features, -1);
    c.feat_pos.assign(c.n_features, -1);
    auto push = [&](fbh_ctx::Tile t) {
        const uint32_t id = (uint32_t)c.tiles.size();
        for (size_t k = 0; k < t.feats.size(); k++) {
            c.feat_tile[t.feats[k]] = (int32_t)id;
            c.feat_pos[t.feats[k]] = (int32_t)k;
        }
        c.tiles.push_back(std::move(t));
    };
    std::vector<uint32_t> all(c.n_features);
    for (uint32_t f = 0; f < c.n_features; f++) all[f] = f;
    for (uint32_t w : {1u, 2u}) {
        const std::vector<uint32_t> rot = rot_features(c, w, all);
        std::vector<uint8_t> in_rot(c.n_features, 0);
        for (uint32_t f : rot) in_rot[f] = 1;
        rot_tiles(w, rot, push);
        fbh_ctx::Tile cur{w, 0, 0, {}, nullptr, false};
        uint64_t lds = 0;
        // Planar tiles of one width hold at most as many features as a tile
        // holds of the width's widest LDS feature, so that every workgroup of
        // a launch adds about as many cells a row (wide-bin 2M x 100: tiles of
        // 3 x 1024-bin numeric and 6 x 500-code categorical features against
        // 3 and 3, 424 against 455 rounds/s).
        uint32_t max_feats = c.planar_max_feats;
        if (!max_feats) {
            uint64_t widest = 0;
            for (uint32_t f = 0; f < c.n_features; f++) {
                const uint64_t fb = feature_lds_bytes(c, f);
                if (c.width[f] == w && !in_rot[f] && fb <= c.planar_tile_bytes - 1024u)
                    widest = std::max(widest, fb);
            }
            max_feats = widest ? (uint32_t)((c.planar_tile_bytes - 1024u) / widest) : 0u;
        }
        auto flush = [&]() {
            if (cur.feats.empty()) return;
            cur.rec = round_stride((uint32_t)cur.feats.size() * w);
            cur.stride = cur.rec;
            // an 8-bit 16-byte record is always interleaved
            cur.rot = w == 1 && cur.rec == 16 && !cur.global;
            push(cur);
            cur.feats.clear();
            cur.global = false;
            lds = 0;
        };
        for (uint32_t f = 0; f < c.n_features; f++) {
            if (c.width[f] != w || in_rot[f]) continue;
            // The tile's LDS also holds 64 per-lane dummy slots (1 KiB).
            // Tiles share planar_tile_bytes; a feature wider than that but
            // within tile_bytes takes a tile of its own.
            const uint64_t budget = c.planar_tile_bytes - 1024u;
            const uint64_t fb = feature_lds_bytes(c, f);
            if (fb > budget) {
                // A tile of its own: in LDS up to tile_bytes, else too wide
                // for LDS and accumulated in global memory.
                flush();
                cur.feats.push_back(f);
                cur.global = fb > (uint64_t)c.tile_bytes - 1024u;
                lds = fb;
                flush();
                continue;
            }
            const uint32_t rec = (uint32_t)(cur.feats.size() + 1) * w;
            if (!cur.feats.empty() && (lds + fb > budget || rec > MAX_RECORD_BYTES ||
                                       (max_feats && cur.feats.size() >= max_feats)))
                flush();
            cur.feats.push_back(f);
            lds += fb;
        }
        flush();
    }
}

// Row-bundle layout (see fbh_ctx::bundles): runs of consecutive LDS tiles
// (any width and record size) up to BUNDLE_BYTES of records each; a
// record's offset is a multiple of its load size (16 bytes for records of
// 16 or more, 8 for 8, else 4), so every load keeps its alignment. A run of
// one tile stays on its own. Returns whether any bundle was formed.
constexpr uint32_t BUNDLE_BYTES = 128;
uint32_t record_align(uint32_t rec) { return rec >= 16 ? 16u : (rec == 8 ? 8u : 4u); }

bool layout_bundles(fbh_ctx &c) {
    c.bundles.clear();
    for (auto &t : c.tiles) {
        t.bundle = -1;
        t.bundle_off = 0;
    }
    size_t i = 0;
    while (i < c.tiles.size()) {
        std::vector<uint32_t> offs{0};
        uint32_t used = c.tiles[i].rec;
        size_t j = i + 1;
        if (!c.tiles[i].global)
            while (j < c.tiles.size() && !c.tiles[j].global) {
                const uint32_t a = record_align(c.tiles[j].rec);
                const uint32_t at = (used + a - 1) / a * a;
                if (at + c.tiles[j].rec > BUNDLE_BYTES) break;
                offs.push_back(at);
                used = at + c.tiles[j].rec;
                j++;
            }
        if (j - i >= 2) {
            const int32_t b = (int32_t)c.bundles.size();
            uint32_t pitch = 16;
            while (pitch < used) pitch *= 2;
            c.bundles.push_back({pitch, nullptr});
            for (size_t k = i; k < j; k++) {
                c.tiles[k].bundle = b;
                c.tiles[k].bundle_off = offs[k - i];
            }
        }
        i = j;
    }
    return !c.bundles.empty();
}

uint32_t div_up(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// Upper bound of the chunks a device-planned launch over n_nodes accumulated
// nodes makes under the rule: at most want_chunks when they fit one wave,
// else at most rows / chunk_rows + n_nodes with chunk_rows >= rows /
// want_chunks, or rows / max_rows + n_nodes when the rows per chunk hit
// their maximum.
uint32_t rule_chunk_bound(const ChunkRule &R, uint64_t n_rows, uint32_t n_nodes) {
    const uint64_t clamp = (n_rows + R.max_rows - 1) / R.max_rows;
    return (uint32_t)(std::max<uint64_t>(R.want_chunks, clamp) + n_nodes);
}

// Per-row bytes of the arrays fbh_set_objective adds later: labels, margins,
// leaf ids, row weights and host sigmoids (a context without objective keeps
// a 4-byte delta instead, which this covers).
constexpr uint64_t OBJECTIVE_ROW_BYTES = 4 + 4 + 2 + 4 + 4;
constexpr uint64_t MAX_WINDOW_BYTES = 512ull << 20;  // one streamed record window
constexpr uint64_t MIN_WINDOW_ROWS = 65536;

uint64_t al256(uint64_t b) { return (b + 255) & ~uint64_t(255); }

// Every allocation whose size does not depend on the residency plan, in one
// place: the planner sums it (a returns nullptr), the context performs it.
template <class A>
void fixed_allocations(fbh_ctx &c, A &&a) {
    const uint64_t n = c.n_rows;
    c.gpair_f32 = static_cast<float *>(a(8 * n, "f32 gradient pairs"));
    c.gpair = static_cast<int64_t *>(a(16 * n, "fixed-point gradient pairs"));
    c.rows = static_cast<uint32_t *>(a(4 * n, "row arena"));
    c.tmp = static_cast<uint32_t *>(a(4 * n, "partition arena"));
    c.flags = static_cast<uint8_t *>(a(n, "partition flags"));
    c.hist = static_cast<int64_t *>(a(16 * (uint64_t)c.n_slots * c.width_max, "histogram slots"));
    c.d_scales = static_cast<ScalesDev *>(a(sizeof(ScalesDev), "quantizer scales"));
    c.red_f64 = static_cast<double *>(a(8 * (2 * (uint64_t)c.n_red_blocks + 2), "reduction scratch"));
    c.red_i64 = static_cast<int64_t *>(a(8 * (2 * (uint64_t)c.n_red_blocks + 2), "reduction scratch"));
    // The per-tree tables (tiles, tile features, split features) share one
    // buffer so that a tree's plan goes to the device in one copy.
    c.off_tilefeats = al256(sizeof(TileDev) * c.tiles.size());
    c.off_sfeats = c.off_tilefeats + al256(sizeof(TileFeatDev) * c.n_features);
    c.off_order = c.off_sfeats + al256(sizeof(SplitFeatDev) * c.n_features);
    c.off_pack = c.off_order + al256(4 * (uint64_t)c.n_features);
    // at most ceil(features / 16) packed tiles of each width
    c.off_root = c.off_pack + al256(sizeof(PackTileDev) * ((uint64_t)c.n_features / 16 + 2));
    c.tables_bytes = c.off_root + sizeof(TileDev) * c.tiles.size();
    uint8_t *tt = static_cast<uint8_t *>(a(c.tables_bytes, "tree tables"));
    c.d_tiles = reinterpret_cast<TileDev *>(tt);
    c.d_tilefeats = reinterpret_cast<TileFeatDev *>(tt ? tt + c.off_tilefeats : nullptr);
    c.d_sfeats = reinterpret_cast<SplitFeatDev *>(tt ? tt + c.off_sfeats : nullptr);
    c.d_split_order = reinterpret_cast<uint32_t *>(tt ? tt + c.off_order : nullptr);
    c.d_pack = reinterpret_cast<PackTileDev *>(tt ? tt + c.off_pack : nullptr);
    c.d_root_tiles = reinterpret_cast<TileDev *>(tt ? tt + c.off_root : nullptr);
    const uint64_t cw = std::max(1u, c.max_cat_words);
    c.d_cands = static_cast<FeatCandDev *>(
        a(sizeof(FeatCandDev) * (uint64_t)c.n_slots * c.n_features, "split candidates"));
    c.d_cat_scratch = static_cast<uint64_t *>(a(8 * (uint64_t)c.n_slots * cw, "category sets"));
    // Split packets, then (256-aligned) the category sets of the call.
    c.d_packets = static_cast<SplitPacketDev *>(
        a(sizeof(SplitPacketDev) * MAX_NODES + 256 + 8 * (uint64_t)c.n_slots * cw, "split packets"));
    c.cat_in_words = (uint64_t)c.n_slots * cw;
    c.max_chunks = n / PART_CHUNK + MAX_NODES + 1;
    c.d_counts = static_cast<uint32_t *>(a(4 * c.max_chunks, "partition counts"));
    c.d_excl = static_cast<uint32_t *>(a(4 * (c.max_chunks + 1), "partition offsets"));
    c.d_totals = static_cast<uint32_t *>(a(4 * (uint64_t)MAX_NODES, "partition totals"));
    c.d_cursors = static_cast<unsigned long long *>(
        a(8 * (uint64_t)PART_CURSOR_STRIDE * MAX_NODES, "partition cursors"));
    // Leaf table followed by the leaf values of one call.
    c.d_leaves = static_cast<LeafDev *>(a((sizeof(LeafDev) + 4) * MAX_NODES, "leaf table"));
    // Device plan of a fused partition + evaluation step.
    c.d_lvl_hist = static_cast<HistNodeDev *>(a(sizeof(HistNodeDev) * MAX_NODES, "level plan"));
    c.d_lvl_split =
        static_cast<SplitNodeDev *>(a(sizeof(SplitNodeDev) * MAX_NODES, "level plan"));
    c.d_lvl_out = static_cast<uint32_t *>(a(20 * (uint64_t)MAX_NODES + 256, "level plan"));
    c.d_lvl_rows = c.d_lvl_out ? c.d_lvl_out + 5 * MAX_NODES : nullptr;
    // Staging of the launch tables of one blocking call (each table 256-aligned);
    // a fused step stages a partition's and an evaluation's tables together.
    const size_t eval_tables = sizeof(HistNodeDev) * MAX_NODES + 4 * MAX_NODES +
                               12 * MAX_NODES + sizeof(SplitNodeDev) * MAX_NODES +
                               (size_t)c.n_slots * c.n_features + 8 * 256;
    const size_t part_tables = 2 * sizeof(PartReqDev) * MAX_NODES + 8 * c.cat_in_words + 4 * 256;
    const size_t pair_tables = sizeof(PairDev) * MAX_NODES + 256;
    c.stage_bytes = std::max<size_t>({eval_tables + part_tables + pair_tables, c.tables_bytes});
    c.d_stage = static_cast<uint8_t *>(a(c.stage_bytes, "launch tables"));
}

// StreamingMemModel + fill_residency (src/training/gpu_mem_plan.rs:279-600,
// 855-880) for LDS tiles in HBM: everything resident when it fits; else the
// columns go first, the streaming windows are reserved and tiles stay
// resident in order while they fit (tiles of one too-wide feature always).
fbh_plan plan_memory(fbh_ctx &c, uint64_t budget);

// The plan with the row bundle when the bundle and the columns fit, else the
// plan of separate tile records and pairs (which may stream).
fbh_plan plan_layout(fbh_ctx &c, uint64_t budget) {
    c.bundled = layout_bundles(c);
    if (c.bundled) {
        try {
            const fbh_plan P = plan_memory(c, budget);
            if (P.resident_tiles == P.n_tiles && P.columns_resident) return P;
        } catch (const InputError &) {
        }
        c.bundled = false;
        c.bundles.clear();
        for (auto &t : c.tiles) {
            t.bundle = -1;
            t.bundle_off = 0;
        }
    }
    return plan_memory(c, budget);
}

fbh_plan plan_memory(fbh_ctx &c, uint64_t budget) {
    fbh_plan P{};
    P.budget = budget;
    P.n_tiles = (uint32_t)c.tiles.size();
    uint64_t fixed = 0;
    fixed_allocations(c, [&](uint64_t b, const char *) -> void * {
        fixed += std::max<uint64_t>(b, 256);
        return nullptr;
    });
    const uint64_t n = c.n_rows;
    fixed += OBJECTIVE_ROW_BYTES * n;
    // More margin columns and the softmax row statistics (multiclass).
    if (c.n_outputs > 1) fixed += (4ull * (c.n_outputs - 1) + 8) * n;
    P.fixed_bytes = fixed;
    if (fixed > budget)
        throw InputError("gpu_memory_budget of " + std::to_string(budget) +
                         " bytes cannot hold the per-row arrays and tables (" +
                         std::to_string(fixed) + " bytes)");
    const uint64_t avail = budget - fixed;
    uint64_t rec_all = 0, col_all = 0;
    for (const auto &b : c.bundles) rec_all += n * b.pitch;
    for (const auto &t : c.tiles)
        if (t.bundle < 0) rec_all += n * t.rec;
    for (uint32_t f = 0; f < c.n_features; f++) col_all += n * c.width[f];
    for (auto &t : c.tiles) t.resident = true;
    // resident_blocks: at most this many tiles stay resident (tiles of a
    // feature too wide for LDS always do and are not counted).
    uint32_t lds_tiles = 0;
    for (const auto &t : c.tiles) lds_tiles += t.global ? 0 : 1;
    const bool capped = c.resident_cap < lds_tiles;
    if (rec_all + col_all <= avail && !capped) {
        P.resident_record_bytes = rec_all;
        P.column_bytes = col_all;
        P.columns_resident = 1;
        P.resident_tiles = P.n_tiles;
    } else if (c.bundled) {
        throw InputError("the row bundles do not fit the budget");
    } else {
        uint32_t max_stride = 4, max_w = 1;
        for (const auto &t : c.tiles) max_stride = std::max(max_stride, t.stride);
        for (uint32_t f = 0; f < c.n_features; f++) max_w = std::max<uint32_t>(max_w, c.width[f]);
        // Column windows (uploads, partitions of streamed features) and
        // record windows (histograms of streamed tiles): two of each, so
        // uploads overlap the kernels, or one (hist_streams = 1).
        const uint64_t nw = c.n_windows;
        const uint64_t col_win = nw * n * max_w;
        uint64_t w = std::min<uint64_t>(MAX_WINDOW_BYTES, avail / 8) / (2 * max_stride);
        w = std::min<uint64_t>(n, std::max<uint64_t>(w, MIN_WINDOW_ROWS));
        const uint64_t rec_win = nw * w * max_stride;
        if (col_win + rec_win > avail)
            throw InputError("gpu_memory_budget of " + std::to_string(budget) +
                             " bytes leaves " + std::to_string(avail) +
                             " bytes after the per-row arrays; streaming needs " +
                             std::to_string(col_win + rec_win));
        uint64_t left = avail - col_win - rec_win;
        for (auto &t : c.tiles) {
            if (!t.global) continue;
            if (n * t.stride > left)
                throw InputError("gpu_memory_budget too small for the records of a feature "
                                 "too wide for LDS, which must stay resident");
            left -= n * t.stride;
            P.resident_record_bytes += n * t.stride;
            P.resident_tiles++;
        }
        bool any_streamed = false;
        uint32_t kept = 0;
        for (auto &t : c.tiles) {
            if (t.global) continue;
            if (n * t.stride <= left && kept < c.resident_cap) {
                kept++;
                left -= n * t.stride;
                P.resident_record_bytes += n * t.stride;
                P.resident_tiles++;
            } else {
                t.resident = false;
                any_streamed = true;
                P.streamed_record_bytes += n * t.stride;
            }
        }
        P.columns_resident = 0;
        P.window_rows = any_streamed ? (uint32_t)w : 0;
        P.staging_bytes = col_win + (any_streamed ? rec_win : 0);
    }
    P.peak_bytes = P.fixed_bytes + P.resident_record_bytes + P.column_bytes + P.staging_bytes;
    return P;
}

uint64_t budget_of(const fbh_config &conf, uint64_t free_bytes) {
    if (conf.memory_budget) return conf.memory_budget;
    const uint64_t reserve = std::max<uint64_t>(free_bytes / 100 * 15, 512ull << 20);
    return free_bytes > reserve ? free_bytes - reserve : 0;
}

void ensure_tree(const fbh_ctx *c) {
    if (!c->tree_begun) throw InputError("fbh_begin_tree must be called before this operation");
}

}  // namespace

namespace {

// Shape and configuration of a context (no device work): shared by
// fbh_ctx_create and fbh_plan_memory.
fbh_config configure(fbh_ctx &c, uint64_t n_rows, const fbh_shape *shape, const fbh_config *cfg) {
    if (!shape || shape->n_features == 0) throw InputError("shape has no features");
    if (!shape->width || !shape->n_bins) throw InputError("shape needs widths and bin counts");
    if (n_rows == 0) throw InputError("training data must have at least one row");
    if (n_rows > 0xFFFFFFFFull)
        throw InputError("training data has " + std::to_string(n_rows) +
                         " rows, above the supported limit 4294967295");
    c.n_rows = n_rows;
    c.n_features = shape->n_features;
    c.width.assign(shape->width, shape->width + shape->n_features);
    c.n_bins.assign(shape->n_bins, shape->n_bins + shape->n_features);
    c.cat.assign(shape->n_features, 0);
    if (shape->categorical)
        c.cat.assign(shape->categorical, shape->categorical + shape->n_features);
    for (uint32_t f = 0; f < c.n_features; f++) {
        if (c.width[f] != 1 && c.width[f] != 2)
            throw InputError("feature " + std::to_string(f) + " has bin width " +
                             std::to_string(c.width[f]) + "; only 1 and 2 are supported");
        // An 8-bit numeric feature may hold 256 bins when it has no missing
        // row (the caller's promise): every byte is then a bin.
        const uint32_t lim = c.width[f] == 1 ? (c.cat[f] ? 255u : 256u) : 65535u;
        if (c.n_bins[f] == 0 || c.n_bins[f] > lim)
            throw InputError("feature " + std::to_string(f) + " has " +
                             std::to_string(c.n_bins[f]) + " bins, not storable at width " +
                             std::to_string(c.width[f]));
        if (c.cat[f] && c.n_bins[f] > MAX_DEVICE_CATS)
            throw InputError("categorical feature " + std::to_string(f) + " has " +
                             std::to_string(c.n_bins[f]) +
                             " categories; the device split scan supports at most " +
                             std::to_string(MAX_DEVICE_CATS));
        c.width_max += c.n_bins[f];
        if (c.cat[f]) c.max_cat_words += (c.n_bins[f] + 63) / 64;
    }
    fbh_config conf{};
    if (cfg) conf = *cfg;
    c.tile_bytes = (uint32_t)env_u64("FB_HIP_TILE_BYTES",
                                      conf.tile_bytes ? conf.tile_bytes : DEFAULT_TILE_BYTES);
    c.planar_tile_bytes = conf.tile_bytes || std::getenv("FB_HIP_TILE_BYTES")
                              ? c.tile_bytes
                              : PLANAR_TILE_BYTES;
    c.fixed_chunk_rows = (uint32_t)env_u64("FB_HIP_CHUNK_ROWS", conf.rows_per_block);
    c.hist_tpb = (uint32_t)env_u64("FB_HIP_HIST_TPB", 0);
    c.shared_line_rows = (uint32_t)env_u64("FB_HIP_LINE_ROWS", SHARED_LINE_CHUNK_ROWS);
    c.planar_max_feats = (uint32_t)env_u64("FB_HIP_PLANAR_MAXF", 0);
    c.max_partial_bytes = env_u64("FB_HIP_PARTIAL_MB", MAX_PARTIAL_BYTES >> 20) << 20;
    c.one_pass_chunks = (uint32_t)env_u64("FB_HIP_ONE_PASS_CHUNKS", ONE_PASS_CHUNKS_PER_NODE);
    c.pair_pass = env_u64("FB_HIP_NO_PAIR_PASS", 0) == 0;
    c.sub_in_scan = env_u64("FB_HIP_NO_SUB_IN_SCAN", 0) == 0;
    c.stage_rows_cap = env_u64("FB_HIP_STAGE_ROWS", 0);
    c.hist_waves = (uint32_t)env_u64("FB_HIP_HIST_WAVES", 0);
    c.host_hist_waves =
        (uint32_t)std::max<uint64_t>(1, env_u64("FB_HIP_HOST_HIST_WAVES", HOST_HIST_WAVES));
    if (c.tile_bytes < 4096 || c.tile_bytes > 160 * 1024)
        throw InputError("tile_bytes must be in 4096..=163840");
    if (c.fixed_chunk_rows && (c.fixed_chunk_rows < 256 || c.fixed_chunk_rows % 256))
        throw InputError("rows_per_block must be a positive multiple of 256");
    if (c.hist_tpb != 0 && c.hist_tpb != 256 && c.hist_tpb != 512 && c.hist_tpb != 1024)
        throw InputError("histogram threads per workgroup must be 256, 512 or 1024");
    if (conf.stream_windows > 2)
        throw InputError("stream_windows (hist_streams) must be 1 or 2, got " +
                         std::to_string(conf.stream_windows));
    c.n_windows = conf.stream_windows ? conf.stream_windows : 2;
    c.n_outputs = conf.n_outputs ? conf.n_outputs : 1;
    c.resident_cap = conf.resident_limit ? conf.resident_limit - 1 : UINT32_MAX;
    c.n_slots = conf.hist_slots ? conf.hist_slots : 64;
    if (c.n_slots > MAX_NODES)
        throw InputError("hist_slots must be at most " + std::to_string(MAX_NODES));
    plan_tiles(c);
    return conf;
}

}  // namespace

// ====================================================================== API
extern "C" {

size_t fbh_last_error(char *buf, size_t len) {
    if (buf && len) {
        size_t n = std::min(len - 1, g_err.size());
        std::memcpy(buf, g_err.data(), n);
        buf[n] = 0;
    }
    return g_err.size();
}

int fbh_device_available(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
    return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int fbh_ctx_create(int device, uint64_t n_rows, const fbh_shape *shape, const fbh_config *cfg,
                   fbh_ctx **out) {
    return guard([&] {
        if (!out) throw InputError("out must not be null");
        *out = nullptr;
        auto c = std::make_unique<fbh_ctx>();
        c->device = -1;
        const fbh_config conf = configure(*c, n_rows, shape, cfg);
        int n_dev = 0;
        if (hipGetDeviceCount(&n_dev) != hipSuccess || n_dev == 0)
            throw RuntimeError("no HIP device is available");
        if (device < 0 || device >= n_dev)
            throw InputError("device " + std::to_string(device) + " does not exist");
        c->device = device;
        check(hipSetDevice(device), "hipSetDevice");
        check(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "stream creation");
        {
            hipDeviceProp_t prop;
            check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
            c->n_cus = (uint32_t)std::max(1, prop.multiProcessorCount);
        }
        size_t free_b = 0, total_b = 0;
        check(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
        c->plan = plan_layout(*c, budget_of(conf, free_b));
        const fbh_plan &P = c->plan;

        // ---- allocation, once, as planned ----
        for (auto &b : c->bundles) b.data = c->alloc<uint8_t>(n_rows * b.pitch, "row bundle");
        for (auto &t : c->tiles) {
            if (t.bundle >= 0) {
                t.data = c->bundles[t.bundle].data + t.bundle_off;
                t.stride = c->bundles[t.bundle].pitch;
            } else if (t.resident) {
                t.data = c->alloc<uint8_t>(n_rows * t.stride, "tile records");
            } else {
                t.data = nullptr;
                t.host = c->host_alloc(n_rows * t.stride, "streamed tile records");
                std::memset(t.host, 0, n_rows * t.stride);
            }
        }
        c->cols.assign(c->n_features, nullptr);
        c->host_cols.assign(c->n_features, nullptr);
        if (P.columns_resident) {
            uint64_t col_bytes = 0;
            for (uint32_t f = 0; f < c->n_features; f++) col_bytes += n_rows * c->width[f];
            uint8_t *base = c->alloc<uint8_t>(col_bytes, "bin columns");
            for (uint32_t f = 0; f < c->n_features; f++) {
                c->cols[f] = base;
                base += n_rows * c->width[f];
            }
        } else {
            uint32_t max_stride = 4, max_w = 1;
            for (const auto &t : c->tiles) max_stride = std::max(max_stride, t.stride);
            for (uint32_t f = 0; f < c->n_features; f++)
                max_w = std::max<uint32_t>(max_w, c->width[f]);
            for (uint32_t k = 0; k < c->n_windows; k++)
                c->win_col[k] = c->alloc<uint8_t>(n_rows * max_w, "column window");
            if (P.window_rows)
                for (uint32_t k = 0; k < c->n_windows; k++)
                    c->win_rec[k] =
                        c->alloc<uint8_t>((uint64_t)P.window_rows * max_stride, "record window");
            for (const auto &t : c->tiles)
                if (!t.resident)
                    for (uint32_t f : t.feats)
                        c->host_cols[f] = c->host_alloc(n_rows * c->width[f], "streamed column");
            check(hipStreamCreateWithFlags(&c->copy_stream, hipStreamNonBlocking), "stream creation");
            for (int k = 0; k < 4; k++) {
                check(hipEventCreateWithFlags(&c->win_ready[k], hipEventDisableTiming), "event");
                check(hipEventCreateWithFlags(&c->win_free[k], hipEventDisableTiming), "event");
                check(hipEventRecord(c->win_free[k], c->stream), "event");
            }
        }
        c->uploaded.assign(c->n_features, 0);
        fixed_allocations(*c, [&](uint64_t b, const char *what) -> void * {
            return c->alloc<uint8_t>(b, what);
        });
        for (int k = 0; k < fbh_ctx::STAGE_SLOTS; k++) {
            c->pinned_mapped(c->pin_stage[k], c->stage_bytes);
            check(hipEventCreateWithFlags(&c->stage_ev[k], hipEventDisableTiming), "event");
        }
        c->pinned(c->pin_leaves, (sizeof(LeafDev) + 4) * MAX_NODES);
        // Results: packets, category sets, then a fused step's spans and slots.
        c->pin_out_spans = al256(sizeof(SplitPacketDev) * MAX_NODES) +
                           al256(8 * (size_t)c->n_slots * std::max(1u, c->max_cat_words));
        c->pinned(c->pin_out, c->pin_out_spans + 20 * (size_t)MAX_NODES + 256);
        check(hipEventCreateWithFlags(&c->leaves_done, hipEventDisableTiming), "event");
        // Zero the record padding once.
        for (const auto &b : c->bundles)
            check(hipMemsetAsync(b.data, 0, n_rows * b.pitch, c->stream), "bundle clear");
        for (auto &t : c->tiles)
            if (t.resident && t.bundle < 0)
                check(hipMemsetAsync(t.data, 0, n_rows * t.stride, c->stream), "tile clear");
        c->sync();
        *out = c.release();
    });
}

int fbh_plan_memory(uint64_t n_rows, const fbh_shape *shape, const fbh_config *cfg,
                    uint64_t free_bytes, fbh_plan *out) {
    return guard([&] {
        if (!out) throw InputError("out must not be null");
        fbh_ctx c;
        c.device = -1;
        const fbh_config conf = configure(c, n_rows, shape, cfg);
        *out = plan_layout(c, budget_of(conf, free_bytes));
    });
}

int fbh_ctx_plan(const fbh_ctx *c, fbh_plan *out) {
    return guard([&] {
        if (!c || !out) throw InputError("null argument");
        *out = c->plan;
    });
}

int fbh_ctx_destroy(fbh_ctx *ctx) {
    return guard([&] { delete ctx; });
}

uint64_t fbh_ctx_device_bytes(const fbh_ctx *ctx) { return ctx ? ctx->device_bytes : 0; }

uint64_t fbh_ctx_streamed_bytes(const fbh_ctx *ctx) { return ctx ? ctx->streamed_bytes : 0; }

int fbh_upload_block(fbh_ctx *c, const uint32_t *feat_ids, uint32_t n_feats, uint32_t width,
                     const void *bins) {
    return guard([&] {
        if (!c || !feat_ids || !bins) throw InputError("null argument");
        check(hipSetDevice(c->device), "hipSetDevice");
        c->tm_stale = true;
        c->hot_ready = false;
        for (uint32_t l = 0; l < n_feats; l++) {
            const uint32_t f = feat_ids[l];
            if (f >= c->n_features) throw InputError("feature id out of range");
            if (c->width[f] != width)
                throw InputError("feature " + std::to_string(f) +
                                 " does not have the block's bin width");
        }
        const uint64_t n = c->n_rows;
        for (uint32_t l = 0; l < n_feats; l++) {
            const uint32_t f = feat_ids[l];
            const fbh_ctx::Tile &t = c->tiles[c->feat_tile[f]];
            const uint32_t off = (uint32_t)c->feat_pos[f] * width;
            const uint8_t *src = static_cast<const uint8_t *>(bins) + (uint64_t)l * n * width;
            if (t.resident) {
                // Through the resident column, or a column window, into the
                // feature's record position.
                uint8_t *col = c->plan.columns_resident ? c->cols[f] : c->win_col[0];
                check(hipMemcpyAsync(col, src, n * width, hipMemcpyHostToDevice, c->stream),
                      "block upload");
                check(launch_pack_feature(col, n, width, t.data, t.stride, off, c->stream),
                      "tile packing");
                if (!c->plan.columns_resident) c->sync();  // the window is reused
            } else {
                // A streamed tile: records packed into pinned host memory, and
                // the column kept for the partitions of this feature.
                std::memcpy(c->host_cols[f], src, n * width);
                uint8_t *rec = t.host + off;
                const uint32_t stride = t.stride;
                const unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
                std::vector<std::thread> pool;
                for (unsigned k = 0; k < nt; k++)
                    pool.emplace_back([&, k] {
                        const uint64_t lo = n * k / nt, hi = n * (k + 1) / nt;
                        for (uint64_t r = lo; r < hi; r++)
                            std::memcpy(rec + r * stride, src + r * width, width);
                    });
                for (auto &th : pool) th.join();
            }
            c->uploaded[f] = 1;
        }
        c->pack_sig.clear();  // packed records of these features are stale
        c->sync();
    });
}

int fbh_set_cuts(fbh_ctx *c, const float *cut_values, const uint32_t *cut_offsets,
                 const uint8_t *categorical) {
    return guard([&] {
        if (!c || !cut_offsets || (!cut_values && cut_offsets[c->n_features] != 0))
            throw InputError("null argument");
        check(hipSetDevice(c->device), "hipSetDevice");
        const uint32_t nf = c->n_features;
        const bool staged = !c->plan.columns_resident;
        if (cut_offsets[0] != 0) throw InputError("cut offsets must start at 0");
        for (uint32_t f = 0; f < nf; f++) {
            if (cut_offsets[f + 1] < cut_offsets[f])
                throw InputError("cut offsets must not decrease");
            const uint32_t nc = cut_offsets[f + 1] - cut_offsets[f];
            if ((uint64_t)nc + 1 != c->n_bins[f])
                throw InputError("feature " + std::to_string(f) + " has " + std::to_string(nc) +
                                 " cuts for " + std::to_string(c->n_bins[f]) + " bins");
            if ((categorical && categorical[f]) != (c->cat[f] != 0))
                throw InputError("feature " + std::to_string(f) +
                                 " is categorical in the cuts and not in the shape, or back");
            for (uint32_t i = cut_offsets[f] + 1; i < cut_offsets[f + 1]; i++)
                if (!(cut_values[i] > cut_values[i - 1]))
                    throw InputError("feature " + std::to_string(f) +
                                     " cuts must be strictly increasing");
        }
        const uint64_t n_vals = cut_offsets[nf];
        const uint64_t bytes = 4 * std::max<uint64_t>(n_vals, 1) + sizeof(BinFeatDev) * nf + 512 +
                               (staged ? c->bin_stage_bytes() : 0);
        if (c->device_bytes + bytes > c->plan.budget)
            throw InputError("the device cuts do not fit the budget's remaining room");
        if (!c->d_cut_values) {
            c->d_cut_values = c->alloc<float>(std::max<uint64_t>(n_vals, 1), "device cuts");
            c->d_binfeats = c->alloc<BinFeatDev>(nf, "device binning table");
        } else {
            throw InputError("the cuts of this context are already set");
        }
        if (staged) {
            uint64_t stride = 0, off = 0;
            for (const auto &t : c->tiles)
                if (!t.resident) stride = std::max<uint64_t>(stride, t.stride);
            c->bin_off.assign(nf, 0);
            for (uint32_t f = 0; f < nf; f++) {
                c->bin_off[f] = off;
                off += al256(c->stage_rows() * c->width[f]);
            }
            c->bin_stage = c->alloc<uint8_t>(off, "binning stage");
            if (stride)
                c->rec_stage = c->alloc<uint8_t>(c->stage_rows() * stride, "record stage");
        }
        std::vector<BinFeatDev> tab(nf);
        for (uint32_t f = 0; f < nf; f++) {
            tab[f].cuts = c->d_cut_values + cut_offsets[f];
            tab[f].col = staged ? c->bin_stage + c->bin_off[f] : c->cols[f];
            tab[f].n_cuts = cut_offsets[f + 1] - cut_offsets[f];
            tab[f].n_bins = c->n_bins[f];
            tab[f].width = c->width[f];
            tab[f].categorical = c->cat[f];
        }
        if (n_vals)
            check(hipMemcpyAsync(c->d_cut_values, cut_values, 4 * n_vals, hipMemcpyHostToDevice,
                                 c->stream),
                  "cuts upload");
        check(hipMemcpyAsync(c->d_binfeats, tab.data(), sizeof(BinFeatDev) * nf,
                             hipMemcpyHostToDevice, c->stream),
              "binning table upload");
        c->sync();
        c->cuts_set = true;
    });
}

uint64_t fbh_rows_staging_bytes(const fbh_ctx *c) {
    if (!c) return 0;
    return c->stage_rows() * 4ull * c->n_features +
           (c->plan.columns_resident ? 0 : c->bin_stage_bytes());
}

// Rows [row0, row0 + k) binned into the binning stage: resident tiles'
// records packed in place, streamed tiles' records packed in the record
// stage and copied to their pinned host memory, with the streamed features'
// columns (for their partitions). All in stream order, so the next chunk's
// binning waits for these copies.
static void pack_staged_rows(fbh_ctx *c, uint64_t row0, uint64_t k) {
    for (const auto &t : c->tiles) {
        if (t.resident) {
            for (uint32_t f : t.feats)
                check(launch_pack_feature(c->bin_stage + c->bin_off[f], k, c->width[f],
                                          t.data + row0 * t.stride, t.stride,
                                          (uint32_t)c->feat_pos[f] * c->width[f], c->stream),
                      "tile packing");
            continue;
        }
        check(hipMemsetAsync(c->rec_stage, 0, k * t.stride, c->stream), "record stage clear");
        for (uint32_t f : t.feats)
            check(launch_pack_feature(c->bin_stage + c->bin_off[f], k, c->width[f],
                                      c->rec_stage, t.stride,
                                      (uint32_t)c->feat_pos[f] * c->width[f], c->stream),
                  "record packing");
        check(hipMemcpyAsync(t.host + row0 * t.stride, c->rec_stage, k * t.stride,
                             hipMemcpyDeviceToHost, c->stream),
              "record download");
        for (uint32_t f : t.feats)
            check(hipMemcpyAsync(c->host_cols[f] + row0 * c->width[f],
                                 c->bin_stage + c->bin_off[f], k * c->width[f],
                                 hipMemcpyDeviceToHost, c->stream),
                  "column download");
    }
}

int fbh_upload_rows(fbh_ctx *c, const float *x, uint64_t row0, uint64_t n_rows) {
    return guard([&] {
        if (!c || (!x && n_rows)) throw InputError("null argument");
        if (!c->cuts_set) throw InputError("fbh_set_cuts must come before fbh_upload_rows");
        if (row0 > c->n_rows || n_rows > c->n_rows - row0)
            throw InputError("rows out of range");
        if (n_rows == 0) return;
        check(hipSetDevice(c->device), "hipSetDevice");
        const uint64_t cap = c->stage_rows(), nf = c->n_features;
        if (!c->rows_stage) {
            const uint64_t bytes = cap * 4 * nf;
            if (c->device_bytes + bytes + 256 > c->plan.budget)
                throw InputError("the row staging of device binning (" + std::to_string(bytes) +
                                 " bytes) does not fit the budget's remaining room");
            c->rows_stage = c->alloc<float>(cap * nf, "row staging");
        }
        const bool staged = !c->plan.columns_resident;
        for (uint64_t r = 0; r < n_rows; r += cap) {
            const uint64_t b = std::min(cap, n_rows - r);
            // Stream order: this copy waits for the previous chunk's binning.
            check(hipMemcpyAsync(c->rows_stage, x + r * nf, 4 * b * nf, hipMemcpyHostToDevice,
                                 c->stream),
                  "row upload");
            check(launch_bin_rows(c->rows_stage, b, (uint32_t)nf, staged ? 0 : row0 + r,
                                  c->d_binfeats, c->stream),
                  "row binning");
            if (staged) pack_staged_rows(c, row0 + r, b);
        }
        c->sync();  // the caller may reuse x
    });
}

int fbh_finish_rows(fbh_ctx *c) {
    return guard([&] {
        if (!c) throw InputError("null argument");
        if (!c->cuts_set) throw InputError("fbh_set_cuts must come before fbh_finish_rows");
        check(hipSetDevice(c->device), "hipSetDevice");
        c->tm_stale = true;
        c->hot_ready = false;
        for (uint32_t f = 0; f < c->n_features; f++) {
            const fbh_ctx::Tile &t = c->tiles[c->feat_tile[f]];
            if (!c->plan.columns_resident) {
                // packed chunk by chunk as the rows came (pack_staged_rows)
            } else if (t.resident) {
                const uint32_t off = (uint32_t)c->feat_pos[f] * c->width[f];
                check(launch_pack_feature(c->cols[f], c->n_rows, c->width[f], t.data, t.stride,
                                          off, c->stream),
                      "tile packing");
            } else {
                // A streamed tile's records live in pinned host memory: bring
                // the column back and lay it into them as fbh_upload_block does.
                throw InputError("device binning needs every tile resident");
            }
            c->uploaded[f] = 1;
        }
        c->pack_sig.clear();
        c->sync();
    });
}

namespace {

// Tile-major copies (Tile::tm) of the given tiles, packed from the resident
// bin columns; made once (again after an upload changed the records), and
// only while they fit the budget's remaining room (they are outside the
// memory plan). Returns whether every tile has one.
bool ensure_tile_major(fbh_ctx &c, const std::vector<const fbh_ctx::Tile *> &tiles) {
    if (c.tm_stale) {
        for (auto &t : c.tiles)
            if (t.tm) {
                c.release_alloc(t.tm);
                t.tm = nullptr;
            }
        c.tm_stale = false;
    }
    uint64_t need = 0;
    for (const fbh_ctx::Tile *t : tiles)
        if (!t->tm) need += std::max<uint64_t>((uint64_t)t->rec * c.n_rows, 256);
    if (need && c.device_bytes + need + 256 > c.plan.budget) return false;
    for (const fbh_ctx::Tile *tp : tiles) {
        fbh_ctx::Tile &t = c.tiles[tp - c.tiles.data()];
        if (t.tm) continue;
        t.tm = c.alloc<uint8_t>((uint64_t)t.rec * c.n_rows, "tile-major records");
        for (uint32_t f : t.feats)
            check(launch_pack_feature(c.cols[f], c.n_rows, t.width, t.tm, t.rec,
                                      (uint32_t)c.feat_pos[f] * t.width, c.stream),
                  "tile-major packing");
    }
    return true;
}

// The hot bins of every categorical feature of at most HOT_MAX_BINS codes:
// its one or two codes that each hold at least 1/16 of the rows (sampled),
// from which a wave of 64 random rows takes four or more lanes on one
// address. Needs the bin columns on the device; none otherwise.
void ensure_hot_bins(fbh_ctx &c) {
    if (c.hot_ready) return;
    c.hot_a.assign(c.n_features, HOT_NONE);
    c.hot_b.assign(c.n_features, HOT_NONE);
    c.hot_ready = true;
    if (!c.plan.columns_resident || env_u64("FB_HIP_NO_HOT", 0)) return;
    std::vector<CatColDev> cols;
    std::vector<uint32_t> feats;
    for (uint32_t f = 0; f < c.n_features; f++)
        if (c.cat[f] && c.n_bins[f] <= HOT_MAX_BINS && c.n_bins[f] >= 2 && c.cols[f]) {
            cols.push_back({c.cols[f], c.width[f], c.n_bins[f]});
            feats.push_back(f);
        }
    if (cols.empty()) return;
    const uint32_t sample = 1u << 20;
    const uint64_t tb = sizeof(CatColDev) * cols.size(), ob = 16 * cols.size();
    if (c.device_bytes + tb + ob + 1024 > c.plan.budget) return;
    uint8_t *buf = c.alloc<uint8_t>(((tb + 255) & ~uint64_t(255)) + ob, "hot-bin search");
    uint32_t *d_out = reinterpret_cast<uint32_t *>(buf + ((tb + 255) & ~uint64_t(255)));
    check(hipMemcpyAsync(buf, cols.data(), tb, hipMemcpyHostToDevice, c.stream), "hot-bin table");
    check(launch_cat_hot(reinterpret_cast<const CatColDev *>(buf), (uint32_t)cols.size(), c.n_rows,
                         sample, d_out, c.stream),
          "hot-bin search");
    std::vector<uint32_t> out(4 * cols.size());
    check(hipMemcpyAsync(out.data(), d_out, ob, hipMemcpyDeviceToHost, c.stream),
          "hot-bin download");
    c.sync();
    c.release_alloc(buf);
    const uint64_t m = std::min<uint64_t>(c.n_rows, sample);
    const uint32_t need = (uint32_t)std::max<uint64_t>(4, m / 16);
    for (size_t i = 0; i < feats.size(); i++) {
        const uint32_t f = feats[i];
        if (out[4 * i] != HOT_NONE && out[4 * i + 2] >= need) c.hot_a[f] = out[4 * i];
        if (c.hot_a[f] != HOT_NONE && out[4 * i + 1] != HOT_NONE && out[4 * i + 3] >= need)
            c.hot_b[f] = out[4 * i + 1];
    }
}

// This tree's packed tiles (fbh_ctx::pack_tiles) from its compact histogram
// layout (hist_off). Per width, the tree's features of interleaved tiles are
// packed when every such tile is resident, the bin columns are on the
// device, ceil(features / 16) tiles are at most 3/4 of the tiles holding
// them, and the pack fits the budget's remaining room (it is outside the
// memory plan). Packed tiles of one width share 128-byte row bundles.
// Returns the widths packed: bit 1 for 8-bit, bit 2 for 16-bit tiles.
uint32_t plan_pack(fbh_ctx &c) {
    c.pack_tiles.clear();
    if (!c.plan.columns_resident) return 0;
    struct Want {
        uint32_t w;
        std::vector<uint32_t> feats;
    };
    std::vector<Want> want;
    for (uint32_t w : {1u, 2u}) {
        uint32_t holding = 0;
        bool resident = true;
        std::vector<uint32_t> feats;
        for (const auto &t : c.tiles) {
            if (!t.rot || t.width != w) continue;
            resident = resident && t.resident;
            bool any = false;
            for (uint32_t f : t.feats)
                if (c.hist_off[f] >= 0) {
                    feats.push_back(f);
                    any = true;
                }
            holding += any ? 1 : 0;
        }
        const uint32_t nt = (uint32_t)(feats.size() + 15) / 16;
        if (!resident || feats.empty() || 4 * nt > 3 * holding) continue;
        std::sort(feats.begin(), feats.end());
        want.push_back({w, std::move(feats)});
    }
    if (want.empty()) return 0;
    // Bundle b of width w: tiles [b * per, (b + 1) * per), per = 128 / (16 w).
    auto pitch_of = [](uint32_t w, uint32_t k) {
        uint32_t p = 16;
        while (p < 16 * w * k) p *= 2;
        return p;
    };
    uint64_t need = 0;
    for (const auto &x : want) {
        const uint32_t nt = (uint32_t)(x.feats.size() + 15) / 16, per = 8 / x.w;
        for (uint32_t b = 0; b * per < nt; b++)
            need += c.n_rows * pitch_of(x.w, std::min(per, nt - b * per));
    }
    if (need > c.pack_bytes) {
        if (c.device_bytes - c.pack_bytes + need + 256 > c.plan.budget) return 0;
        c.release_alloc(c.pack);
        c.pack = nullptr;
        c.pack_bytes = 0;
        c.pack_sig.clear();
        c.pack = c.alloc<uint8_t>(need, "packed tiles");
        c.pack_bytes = need;
    }
    uint32_t mask = 0, pack_bundles = 0;
    uint8_t *base = c.pack;
    for (const auto &x : want) {
        const uint32_t per = 8 / x.w;
        const uint32_t first = (uint32_t)c.pack_tiles.size();
        rot_tiles(x.w, x.feats, [&](fbh_ctx::Tile t) { c.pack_tiles.push_back(std::move(t)); });
        const uint32_t nt = (uint32_t)c.pack_tiles.size() - first;
        for (uint32_t b = 0; b * per < nt; b++) {
            const uint32_t k = std::min(per, nt - b * per);
            const uint32_t pitch = pitch_of(x.w, k);
            for (uint32_t j = 0; j < k; j++) {
                fbh_ctx::Tile &t = c.pack_tiles[first + b * per + j];
                t.data = base + 16u * x.w * j;
                t.stride = pitch;
                // bundle ids past the context's own
                t.bundle = (int32_t)(c.bundles.size() + pack_bundles);
                t.bundle_off = 16u * x.w * j;
            }
            pack_bundles++;
            base += c.n_rows * pitch;
        }
        mask |= 1u << x.w;
    }
    return mask;
}

// GradQuantizer::try_from_bounds (src/types.rs:288-303): the power-of-two
// scale of one component from its bound, with the host's libm.
double host_scale(double m, uint64_t n_rows) {
    double s = 1.0;
    if (m > 0.0 && std::isfinite(m)) {
        const double budget = (double)(1ull << 62) / (double)std::max<uint64_t>(n_rows, 1);
        const double raw = budget / m;
        if (std::isfinite(raw) && raw > 0.0) {
            double l = std::floor(std::log2(raw));
            int e = std::isnan(l) ? 0 : (l > 1000.0 ? 1000 : (l < -1000.0 ? -1000 : (int)l));
            s = std::exp2((double)e);
        }
    }
    return s;
}

const char *const NONFINITE_GRADIENT =
    "non-finite gradient or Hessian (or invalid bounds); reduce extreme labels, "
    "weights, base_score or objective parameters";

// The device's scales against the host's from the same bounds: they agree
// unless log2 of the scale budget lies within an ulp of an integer and the
// host's libm rounds it differently; then nothing grown with them is used.
void check_device_scales(const ScalesDev &S, uint64_t n_rows) {
    if (S.from_host) return;
    if (S.status) throw InputError(NONFINITE_GRADIENT);
    for (int k = 0; k < 2; k++)
        if (host_scale(S.max_abs[k], n_rows) != S.scale[k])
            throw RuntimeError("device quantizer scale differs from the host's libm for bound " +
                               std::to_string(S.max_abs[k]));
}

// Bounds, power-of-two scales and fixed-point pairs of the f32 pairs in
// gpair_f32 (GradQuantizer::try_from_bounds, src/types.rs:288-303, 367-385;
// device passes src/backend/cuda/histogram.cu:1079-1177). The scales are
// computed on the device; with scales_out NULL they stay there (no host
// round trip) and are checked when the tree is collected. bounds_done: the
// gradient kernel already masked the subsample and wrote the block bounds.
void quantize_device_pairs(fbh_ctx *c, uint64_t th, uint64_t seed, uint64_t tree,
                           double scales_out[2], int64_t root_out[2], bool bounds_done) {
    if (!bounds_done)
        check(launch_gpair_maxabs(c->gpair_f32, c->n_rows, th, seed, tree, c->red_f64,
                                  c->n_red_blocks, c->stream),
              "gradient bounds");
    check(launch_reduce_bounds(c->red_f64, c->n_red_blocks, c->red_f64 + 2 * c->n_red_blocks,
                               c->n_rows, c->d_scales, c->stream),
          "quantizer scales");
    if (scales_out) {
        ScalesDev S;
        check(hipMemcpyAsync(c->pin_out.p, c->d_scales, sizeof(S), hipMemcpyDeviceToHost,
                             c->stream),
              "scales download");
        c->sync();
        std::memcpy(&S, c->pin_out.p, sizeof(S));
        check_device_scales(S, c->n_rows);
        c->scales[0] = S.scale[0];
        c->scales[1] = S.scale[1];
    }
    // The per-block sums stay in red_i64; only a host caller needs them summed
    // here (a device-grown tree sums them in its root kernel).
    check(launch_gpair_quantize(c->gpair_f32, c->n_rows, c->d_scales, c->gpair, c->red_i64,
                                c->n_red_blocks,
                                root_out ? c->red_i64 + 2 * c->n_red_blocks : nullptr, c->stream),
          "gradient quantisation");
    c->root_on_device = true;
    c->f32_pairs = c->f32_hist();
    if (scales_out) {
        scales_out[0] = c->scales[0];
        scales_out[1] = c->scales[1];
    }
    if (!root_out) return;  // the sum stays on the device for fbh_grow_depthwise
    check(hipMemcpyAsync(c->pin_out.p, c->red_i64 + 2 * c->n_red_blocks, 16,
                         hipMemcpyDeviceToHost, c->stream),
          "root sum download");
    c->sync();
    std::memcpy(root_out, c->pin_out.p, 16);
}

}  // namespace

int fbh_upload_quantize_gpair(fbh_ctx *c, const float *g2n, uint64_t th, uint64_t seed,
                              uint64_t tree, double scales_out[2], int64_t root_out[2]) {
    return guard([&] {
        if (!c || !g2n || !scales_out || !root_out) throw InputError("null argument");
        check(hipSetDevice(c->device), "hipSetDevice");
        check(hipMemcpyAsync(c->gpair_f32, g2n, c->n_rows * 8, hipMemcpyHostToDevice, c->stream),
              "gradient upload");
        quantize_device_pairs(c, th, seed, tree, scales_out, root_out, false);
    });
}

int fbh_set_objective(fbh_ctx *c, uint32_t objective, const float *labels,
                      const float *grad_weights, float base_margin) {
    return guard([&] {
        if (!c || !labels) throw InputError("null argument");
        if (objective > 1) throw InputError("objective must be 0 (squared error) or 1 (logistic)");
        if (c->n_outputs != 1)
            throw InputError("a context planned for several outputs takes fbh_set_multiclass "
                             "or fbh_set_quantile");
        if (c->objective > 1) throw InputError("the context already holds another objective");
        check(hipSetDevice(c->device), "hipSetDevice");
        if (c->objective < 0) {
            c->labels = c->alloc<float>(c->n_rows, "labels");
            c->margin = c->alloc<float>(c->n_rows, "margins");
            c->leaf_ids = c->alloc<uint16_t>(c->n_rows, "leaf ids");
        }
        if (grad_weights && !c->gweights) c->gweights = c->alloc<float>(c->n_rows, "row weights");
        if (objective == 1 && !c->pin_ids.p) {
            c->sig = c->alloc<float>(c->n_rows, "sigmoids");
            c->pinned(c->pin_ids, std::max<uint64_t>(2 * c->n_rows, 64));
            c->pinned(c->pin_src, std::max<uint64_t>(4 * c->n_rows, 64));
            check(hipStreamCreateWithFlags(&c->up_stream, hipStreamNonBlocking), "stream");
            check(hipEventCreateWithFlags(&c->up_done, hipEventDisableTiming), "event");
            for (int k = 0; k < EXCHANGE_CHUNKS; k++) {
                hipEvent_t e;
                check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "event");
                c->chunk_ev.push_back(e);
            }
        }
        c->sync();
        check(hipMemcpy(c->labels, labels, 4 * c->n_rows, hipMemcpyHostToDevice), "label upload");
        c->has_weights = grad_weights != nullptr;
        if (grad_weights)
            check(hipMemcpy(c->gweights, grad_weights, 4 * c->n_rows, hipMemcpyHostToDevice),
                  "weight upload");
        check(launch_fill_f32(c->margin, base_margin, c->n_rows, c->stream), "margin init");
        c->sync();
        c->objective = (int)objective;
        c->ids_fresh = false;
    });
}

int fbh_set_multiclass(fbh_ctx *c, uint32_t n_classes, const float *labels,
                       const float *weights, const float *class_margins) {
    return guard([&] {
        if (!c || !labels || !class_margins) throw InputError("null argument");
        if (n_classes < 2) throw InputError("multiclass objectives require num_class >= 2");
        if (n_classes != c->n_outputs)
            throw InputError("the context was planned for " + std::to_string(c->n_outputs) +
                             " outputs, not " + std::to_string(n_classes) + " classes");
        check(hipSetDevice(c->device), "hipSetDevice");
        if (c->objective < 0) {
            c->labels = c->alloc<float>(c->n_rows, "labels");
            c->margin = c->alloc<float>((uint64_t)n_classes * c->n_rows, "class margins");
            c->leaf_ids = c->alloc<uint16_t>(c->n_rows, "leaf ids");
            c->softmax_stats = c->alloc<float2>(c->n_rows, "softmax row statistics");
        } else if (c->objective != 2) {
            throw InputError("the context already holds a single-output objective");
        }
        if (weights && !c->gweights) c->gweights = c->alloc<float>(c->n_rows, "row weights");
        c->sync();
        check(hipMemcpy(c->labels, labels, 4 * c->n_rows, hipMemcpyHostToDevice), "label upload");
        c->has_weights = weights != nullptr;
        if (weights)
            check(hipMemcpy(c->gweights, weights, 4 * c->n_rows, hipMemcpyHostToDevice),
                  "weight upload");
        for (uint32_t k = 0; k < n_classes; k++)
            check(launch_fill_f32(c->margin + (uint64_t)k * c->n_rows, class_margins[k],
                                  c->n_rows, c->stream),
                  "margin init");
        c->sync();
        c->objective = 2;
        c->out_k = 0;
        c->ids_fresh = false;
    });
}

int fbh_set_quantile(fbh_ctx *c, uint32_t n_alphas, const float *alphas, const float *labels,
                     const float *weights, const float *intercepts) {
    return guard([&] {
        if (!c || !alphas || !labels || !intercepts) throw InputError("null argument");
        if (n_alphas == 0) throw InputError("reg:quantileerror needs at least one quantile_alpha");
        if (n_alphas != c->n_outputs)
            throw InputError("the context was planned for " + std::to_string(c->n_outputs) +
                             " outputs, not " + std::to_string(n_alphas) + " quantiles");
        for (uint32_t k = 0; k < n_alphas; k++) {
            if (!(alphas[k] >= 0.0f && alphas[k] <= 1.0f))
                throw InputError("quantile_alpha must be in [0, 1]");
            if (k && alphas[k - 1] > alphas[k])
                throw InputError("quantile_alpha must be in ascending order");
        }
        check(hipSetDevice(c->device), "hipSetDevice");
        if (c->objective < 0) {
            c->labels = c->alloc<float>(c->n_rows, "labels");
            c->margin = c->alloc<float>((uint64_t)n_alphas * c->n_rows, "quantile margins");
            c->leaf_ids = c->alloc<uint16_t>(c->n_rows, "leaf ids");
            c->quantile_slot = c->alloc<float2>(1, "quantile scale");
            c->q_sums.resize(n_alphas);
            c->q_have.assign(n_alphas, 0);
            c->pinned(c->pin_src, std::max<uint64_t>(4 * c->n_rows, 64));
            for (int k = 0; k < EXCHANGE_CHUNKS; k++) {
                hipEvent_t e;
                check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "event");
                c->chunk_ev.push_back(e);
            }
        } else if (c->objective != 3) {
            throw InputError("the context already holds another objective");
        }
        if (weights && !c->gweights) c->gweights = c->alloc<float>(c->n_rows, "row weights");
        c->sync();
        check(hipMemcpy(c->labels, labels, 4 * c->n_rows, hipMemcpyHostToDevice), "label upload");
        c->has_weights = weights != nullptr;
        // Objective::quantile_scale's denominator: n, or the weights summed
        // in row order in double.
        double sw = 0.0;
        if (weights) {
            check(hipMemcpy(c->gweights, weights, 4 * c->n_rows, hipMemcpyHostToDevice),
                  "weight upload");
            for (uint64_t i = 0; i < c->n_rows; i++) sw += (double)weights[i];
        } else {
            sw = (double)c->n_rows;
        }
        c->quantile_sum_w = sw;
        c->q_forget(-1);
        for (uint32_t k = 0; k < n_alphas; k++)
            check(launch_fill_f32(c->margin + (uint64_t)k * c->n_rows, intercepts[k], c->n_rows,
                                  c->stream),
                  "margin init");
        c->sync();
        c->alphas.assign(alphas, alphas + n_alphas);
        c->objective = 3;
        c->out_k = 0;
        c->ids_fresh = false;
    });
}

int fbh_quantile_last_scale(fbh_ctx *c, float *scale) {
    return guard([&] {
        if (!c || !scale) throw InputError("null argument");
        if (c->objective != 3) throw InputError("fbh_set_quantile has not been called");
        check(hipSetDevice(c->device), "hipSetDevice");
        float2 v;
        check(hipMemcpyAsync(&v, c->quantile_slot, sizeof(v), hipMemcpyDeviceToHost, c->stream),
              "scale download");
        c->sync();
        *scale = v.x;
    });
}

// The round's scale of the current output (Objective::quantile_scale,
// src/training/objective.rs:1115-1137) into the (scale, alpha) slot the
// gradient reads. Exact: each row's f32 term on the device, summed on the
// host in row order in double (the reference's serial sum, which no parallel
// order reproduces). Fast: a fixed-order reduction on the device.
static void quantile_finish(fbh_ctx *c, double stat, float alpha);

// Every output's terms at once, downloaded in chunks, each output summed in
// row order on a host thread of its own (the same serial double sum as a
// single output's).
static void quantile_sum_all(fbh_ctx *c, const float *w) {
    c->q_forget(-1);  // their buffers and events are reused below
    const uint32_t K = c->n_outputs;
    const uint64_t n = c->n_rows;
    if (!c->q_terms) {
        c->q_terms = c->alloc<float>((uint64_t)K * n, "quantile terms");
        c->pinned(c->pin_q, 4ull * K * n);
    }
    for (uint32_t j = 0; j < K; j++)
        check(launch_quantile_terms(c->margin + (uint64_t)j * n, c->labels, w, n,
                                    c->q_terms + (uint64_t)j * n, c->stream),
              "quantile terms");
    float *host = static_cast<float *>(c->pin_q.p);
    const uint64_t step = ((n + EXCHANGE_CHUNKS - 1) / EXCHANGE_CHUNKS + 255) & ~uint64_t(255);
    for (int k = 0; k < EXCHANGE_CHUNKS; k++) {
        const uint64_t b = std::min<uint64_t>(n, k * step), e = std::min<uint64_t>(n, b + step);
        for (uint32_t j = 0; e > b && j < K; j++)
            check(hipMemcpyAsync(host + (uint64_t)j * n + b, c->q_terms + (uint64_t)j * n + b,
                                 4 * (e - b), hipMemcpyDeviceToHost, c->stream),
                  "quantile terms download");
        check(hipEventRecord(c->chunk_ev[k], c->stream), "event");
    }
    for (uint32_t j = 0; j < K; j++) {
        const float *t = host + (uint64_t)j * n;
        c->q_sums[j] = std::async(std::launch::async, [c, t, n, step] {
            double stat = 0.0;
            for (int k = 0; k < EXCHANGE_CHUNKS; k++) {
                const uint64_t b = std::min<uint64_t>(n, k * step);
                const uint64_t e = std::min<uint64_t>(n, b + step);
                check(hipEventSynchronize(c->chunk_ev[k]), "quantile terms download");
                for (uint64_t i = b; i < e; i++) stat += (double)t[i];
            }
            return stat;
        });
        c->q_have[j] = 1;
    }
}

static void quantile_take_scale(fbh_ctx *c) {
    c->q_raise();
    const float *w = c->has_weights ? c->gweights : nullptr;
    const float alpha = c->alphas[c->out_k];
    const uint64_t n = c->n_rows;
    if (c->fast_math) {
        check(launch_quantile_scale_fast(c->cur_margin(), c->labels, w, n, alpha, c->red_f64,
                                         c->quantile_slot, c->stream),
              "quantile scale");
        return;
    }
    const uint32_t K = c->n_outputs, out = c->out_k;
    const uint64_t batch_bytes = 4ull * K * n;
    if (K > 1 && (c->q_terms || (batch_bytes <= (1ull << 30) &&
                                 c->device_bytes + batch_bytes + 256 <= c->plan.budget))) {
        if (!c->q_have[out]) quantile_sum_all(c, w);
        const double stat = c->q_sums[out].get();  // a worker's error is raised here
        c->q_sums[out] = std::future<double>();
        c->q_have[out] = 0;  // this output's tree follows
        quantile_finish(c, stat, alpha);
        return;
    }
    float *terms = c->gpair_f32;  // rewritten by the gradient pass that follows
    check(launch_quantile_terms(c->cur_margin(), c->labels, w, n, terms, c->stream),
          "quantile terms");
    // The terms come down in chunks, each signalling its own event, and the
    // host sums chunk k while later chunks are still in flight.
    float *host = static_cast<float *>(c->pin_src.p);
    const uint64_t step = ((n + EXCHANGE_CHUNKS - 1) / EXCHANGE_CHUNKS + 255) & ~uint64_t(255);
    for (int k = 0; k < EXCHANGE_CHUNKS; k++) {
        const uint64_t b = std::min<uint64_t>(n, k * step), e = std::min<uint64_t>(n, b + step);
        if (e > b)
            check(hipMemcpyAsync(host + b, terms + b, 4 * (e - b), hipMemcpyDeviceToHost,
                                 c->stream),
                  "quantile terms download");
        check(hipEventRecord(c->chunk_ev[k], c->stream), "event");
    }
    double stat = 0.0;
    for (int k = 0; k < EXCHANGE_CHUNKS; k++) {
        const uint64_t b = std::min<uint64_t>(n, k * step), e = std::min<uint64_t>(n, b + step);
        check(hipEventSynchronize(c->chunk_ev[k]), "quantile terms download");
        for (uint64_t i = b; i < e; i++) stat += (double)host[i];
    }
    quantile_finish(c, stat, alpha);
}

// The scale from a term sum into the slot the gradient reads.
static void quantile_finish(fbh_ctx *c, double stat, float alpha) {
    float scale = 0.0f;
    if (!(std::fabs(c->quantile_sum_w) < 1e-6)) {
        const double root_mean = stat / c->quantile_sum_w;
        scale = (float)(root_mean * root_mean);
    }
    c->quantile_scale = scale;
    check(launch_quantile_set(c->quantile_slot, scale, alpha, c->stream), "quantile scale");
}

int fbh_multiclass_begin_round(fbh_ctx *c) {
    return guard([&] {
        if (!c) throw InputError("null argument");
        if (c->objective != 2) throw InputError("fbh_set_multiclass has not been called");
        if (c->leaves_deferred)
            throw InputError("the last grown tree's leaf values were deferred and not applied "
                             "(fbh_apply_leaf_values): the margins are not up to date");
        check(hipSetDevice(c->device), "hipSetDevice");
        check(launch_softmax_stats(c->margin, c->n_outputs, c->n_rows, c->fast_math ? 1 : 0,
                                   c->softmax_stats, c->stream),
              "softmax row statistics");
    });
}

int fbh_set_output(fbh_ctx *c, uint32_t k) {
    return guard([&] {
        if (!c) throw InputError("null argument");
        if (k >= c->n_outputs)
            throw InputError("output " + std::to_string(k) + " of " +
                             std::to_string(c->n_outputs));
        if (c->leaves_deferred)
            throw InputError("the last grown tree's leaf values were deferred and not applied "
                             "(fbh_apply_leaf_values): the margins are not up to date");
        c->out_k = k;
        c->ids_fresh = false;
    });
}

int fbh_set_gpu_math(fbh_ctx *c, uint32_t gpu_math) {
    return guard([&] {
        if (!c) throw InputError("null argument");
        if (gpu_math > 1) throw InputError("gpu_math must be 0 (exact) or 1 (fast)");
        c->fast_math = gpu_math == 1;
    });
}

int fbh_gradient_pairs(int device, uint32_t objective, uint32_t gpu_math, const float *margin,
                       const float *labels, const float *weights, uint64_t n, float *out) {
    return guard([&] {
        if ((!margin || !labels || !out) && n) throw InputError("null argument");
        if (objective > 1) throw InputError("objective must be 0 (squared error) or 1 (logistic)");
        if (gpu_math > 1) throw InputError("gpu_math must be 0 (exact) or 1 (fast)");
        if (n == 0) return;
        check(hipSetDevice(device), "hipSetDevice");
        float *d = nullptr;
        const uint64_t words = n * (weights ? 5 : 4);
        check(hipMalloc(&d, 4 * words), "gradient buffers");
        std::unique_ptr<float, decltype(&hipFree)> own(d, hipFree);
        float *dm = d, *dy = d + n, *dg = d + 2 * n, *dw = weights ? d + 4 * n : nullptr;
        check(hipMemcpy(dm, margin, 4 * n, hipMemcpyHostToDevice), "margin upload");
        check(hipMemcpy(dy, labels, 4 * n, hipMemcpyHostToDevice), "label upload");
        if (weights) check(hipMemcpy(dw, weights, 4 * n, hipMemcpyHostToDevice), "weight upload");
        const int mode = objective == 0 ? 0 : (gpu_math ? 3 : 2);
        check(launch_gradient(dm, dy, dw, n, mode, dg, UINT64_MAX, 0, 0, nullptr, 0, nullptr),
              "gradient");
        check(hipMemcpy(out, dg, 8 * n, hipMemcpyDeviceToHost), "gradient download");
    });
}

int fbh_gradient_exchange(fbh_ctx *c, fbh_sigmoid_fn fn, void *user, uint64_t th, uint64_t seed,
                          uint64_t tree, double scales_out[2], int64_t root_out[2]) {
    return guard([&] {
        if (!c) throw InputError("null argument");
        if (c->leaves_deferred)
            throw InputError("the last grown tree's leaf values were deferred and not applied "
                             "(fbh_apply_leaf_values): the margins are not up to date");
        if (!scales_out && (root_out || fn))
            throw InputError("the scales stay on the device only with neither a root sum nor "
                             "a sigmoid callback");
        if (c->objective < 0) throw InputError("fbh_set_objective has not been called");
        if (fn && c->fast_math && c->objective == 1)
            throw InputError("gpu_math=\"fast\" computes the logistic sigmoid on the device; "
                             "a host sigmoid callback is not used with it");
        check(hipSetDevice(c->device), "hipSetDevice");
        if (c->leaves_pending) {
            check(hipEventSynchronize(c->leaves_done), "leaf table reuse");
            c->leaves_pending = false;
        }
        const float *w = c->has_weights ? c->gweights : nullptr;
        if (c->objective == 3) quantile_take_scale(c);
        // Mode 6 reads (scale, alpha) from the slot; softmax reads row statistics.
        const float2 *stats = c->objective == 3 ? c->quantile_slot : c->softmax_stats;
        if (!scales_out) {
            // Everything stays on the device: the pairs' quantisation under
            // the previous round's scales, with its block sums, redone only
            // if this round's bounds give other scales. With few tiles the
            // f32 pairs go out too, for the histograms of scattered rows.
            const bool f32 = c->f32_hist();
            check(launch_gradient_spec(c->cur_margin(), c->labels, w, c->n_rows,
                                       c->gradient_mode(), th, seed, tree, c->red_f64,
                                       c->n_red_blocks, c->d_scales, c->gpair, c->red_i64,
                                       f32 ? c->gpair_f32 : nullptr, c->stream, stats,
                                       c->out_k),
                  "device gradient");
            c->ids_fresh = false;
            c->root_on_device = true;
            c->f32_pairs = f32;
            return;
        }
        if (c->objective != 1 || !fn) {
            // Squared error, softmax, or logistic with the device sigmoid.
            check(launch_gradient(c->cur_margin(), c->labels, w, c->n_rows, c->gradient_mode(),
                                  c->gpair_f32, th, seed, tree, c->red_f64, c->n_red_blocks,
                                  c->stream, stats, c->out_k),
                  "device gradient");
        } else {
            const uint64_t n = c->n_rows;
            const int idb = c->ids_fresh ? c->leaf_id_bytes : 0;
            uint8_t *ids = static_cast<uint8_t *>(c->pin_ids.p);
            float *src = static_cast<float *>(c->pin_src.p);
            const uint64_t step = ((n + EXCHANGE_CHUNKS - 1) / EXCHANGE_CHUNKS + 255) & ~uint64_t(255);
            // Leaf ids of every chunk go down at once, each chunk signalling
            // its own event; the host works on chunk k while later chunks are
            // still in flight and chunk k's sigmoids go up on the copy stream.
            if (idb)
                for (int k = 0; k < EXCHANGE_CHUNKS; k++) {
                    const uint64_t b = std::min<uint64_t>(n, k * step), e = std::min<uint64_t>(n, b + step);
                    if (e > b)
                        check(hipMemcpyAsync(ids + b * idb,
                                             static_cast<uint8_t *>(c->leaf_ids) + b * idb,
                                             (e - b) * idb, hipMemcpyDeviceToHost, c->stream),
                              "leaf id download");
                    check(hipEventRecord(c->chunk_ev[k], c->stream), "event");
                }
            for (int k = 0; k < EXCHANGE_CHUNKS; k++) {
                const uint64_t b = std::min<uint64_t>(n, k * step), e = std::min<uint64_t>(n, b + step);
                if (idb) check(hipEventSynchronize(c->chunk_ev[k]), "leaf id download");
                if (e <= b) continue;
                fn(user, b, e - b, idb ? ids + b * idb : nullptr, (uint32_t)idb, src + b);
                check(hipMemcpyAsync(c->sig + b, src + b, 4 * (e - b),
                                     hipMemcpyHostToDevice, c->up_stream),
                      "sigmoid upload");
            }
            check(hipEventRecord(c->up_done, c->up_stream), "event");
            check(hipStreamWaitEvent(c->stream, c->up_done, 0), "stream wait");
            check(launch_gradient(c->sig, c->labels, w, n, 1, c->gpair_f32, th, seed, tree,
                                  c->red_f64, c->n_red_blocks, c->stream),
                  "device gradient");
        }
        c->ids_fresh = false;
        quantize_device_pairs(c, th, seed, tree, scales_out, root_out, true);
    });
}

int fbh_set_margins(fbh_ctx *c, const float *margins) {
    return guard([&] {
        if (!c || !margins) throw InputError("null argument");
        if (c->objective < 0) throw InputError("fbh_set_objective has not been called");
        check(hipSetDevice(c->device), "hipSetDevice");
        c->sync();
        check(hipMemcpy(c->margin, margins, (uint64_t)c->n_outputs * c->n_rows * 4,
                        hipMemcpyHostToDevice),
              "margin upload");
        if (c->objective == 3) c->q_forget(-1);  // every output's scale sum is stale
    });
}

int fbh_download_margin(fbh_ctx *c, float *out) {
    return guard([&] {
        if (!c || !out) throw InputError("null argument");
        if (c->objective < 0) throw InputError("fbh_set_objective has not been called");
        if (c->leaves_deferred)
            throw InputError("the last grown tree's leaf values were deferred and not applied "
                             "(fbh_apply_leaf_values): the margins are not up to date");
        check(hipSetDevice(c->device), "hipSetDevice");
        check(hipMemcpyAsync(out, c->margin, (uint64_t)c->n_outputs * c->n_rows * 4,
                             hipMemcpyDeviceToHost, c->stream),
              "margin download");
        c->sync();
    });
}

int fbh_upload_gpair_fixed(fbh_ctx *c, const int64_t *g2n, const double scales[2]) {
    return guard([&] {
        if (!c || !g2n || !scales) throw InputError("null argument");
        check(hipSetDevice(c->device), "hipSetDevice");
        check(hipMemcpyAsync(c->gpair, g2n, c->n_rows * 16, hipMemcpyHostToDevice, c->stream),
              "gradient upload");
        c->scales[0] = scales[0];
        c->scales[1] = scales[1];
        check(launch_set_scales(c->d_scales, scales[0], scales[1], c->stream), "scales");
        c->root_on_device = false;
        c->f32_pairs = false;
        c->sync();
    });
}

int fbh_begin_tree(fbh_ctx *c, const uint32_t *features, uint32_t n_sel, const int8_t *monotone,
                   uint32_t n_monotone, fbh_span *root) {
    return guard([&] {
        if (!c || !root) throw InputError("null argument");
        check(hipSetDevice(c->device), "hipSetDevice");
        c->tree_feats.clear();
        if (features) {
            for (uint32_t i = 0; i < n_sel; i++) {
                if (features[i] >= c->n_features) throw InputError("feature id out of range");
                if (i && features[i] <= features[i - 1])
                    throw InputError("tree features must be strictly ascending");
                c->tree_feats.push_back(features[i]);
            }
        } else {
            for (uint32_t f = 0; f < c->n_features; f++) c->tree_feats.push_back(f);
        }
        if (c->tree_feats.empty()) throw InputError("a tree needs at least one feature");
        for (uint32_t f : c->tree_feats)
            if (!c->uploaded[f])
                throw InputError("feature " + std::to_string(f) + " was never uploaded");
        c->monotone.assign(c->n_features, 0);
        if (monotone)
            for (uint32_t i = 0; i < std::min(n_monotone, c->n_features); i++)
                c->monotone[i] = monotone[i];
        // compact histogram layout of this tree
        c->hist_off.assign(c->n_features, -1);
        uint64_t off = 0;
        for (uint32_t f : c->tree_feats) {
            c->hist_off[f] = (int64_t)off;
            off += c->n_bins[f];
        }
        c->hist_width = off;
        // tiles with active features, grouped by (width, record dwords)
        ensure_hot_bins(*c);
        std::vector<TileDev> td;
        std::vector<const fbh_ctx::Tile *> td_src;  // the tile of each entry
        std::vector<TileFeatDev> tf;
        c->groups.clear();
        c->streamed.clear();
        c->has_global = false;
        // Appends tile t's entry (and its active features) when it has any;
        // returns the LDS slots and active cell bytes per row.
        auto add_tile = [&](const fbh_ctx::Tile &t, uint32_t &lds, uint32_t &active_bytes) {
            TileDev d{};
            d.data = t.data;
            d.stride = t.stride;
            d.width = t.width;
            d.n_feat = (uint32_t)t.feats.size();
            d.feat_base = (uint32_t)tf.size();
            d.rec_dwords = t.rec / 4;
            lds = 0;
            active_bytes = 0;
            const bool hot_ok = !t.rot && !t.global && t.resident;
            for (uint32_t f : t.feats) {
                TileFeatDev e{};
                e.hot[0] = e.hot[1] = HOT_NONE;
                if (c->hist_off[f] >= 0) {
                    e.n_bins = c->n_bins[f];
                    e.lds_off = lds;
                    e.hist_off = (uint32_t)c->hist_off[f];
                    lds += c->n_bins[f];
                    active_bytes += t.width;
                    if (hot_ok && c->hot_a[f] != HOT_NONE) {
                        e.hot[0] = c->hot_a[f];
                        e.hot[1] = c->hot_b[f];
                        e.hot_off = lds;
                        lds += HOT_SLOTS;
                    }
                }
                tf.push_back(e);
            }
            if (lds == 0) {
                tf.resize(d.feat_base);
                return false;
            }
            if (t.rot) {
                // Interleaved layout: feature k at slot bin * 16 + k.
                for (uint32_t k = 0; k < d.n_feat; k++) tf[d.feat_base + k].lds_off = k;
                lds = HIST_ROT_SLOTS;
            }
            d.lds_slots = t.global ? 0 : lds;
            td.push_back(d);
            td_src.push_back(&t);
            return true;
        };
        const uint32_t packed = plan_pack(*c);
        std::vector<const fbh_ctx::Tile *> built;  // resident tiles of this tree's histograms
        for (const auto &t : c->tiles)
            if (t.resident && !(t.rot && (packed >> t.width & 1u))) built.push_back(&t);
        for (const auto &t : c->pack_tiles) built.push_back(&t);
        // One launch per (global, width, interleaved): interleaved tiles all
        // have 16-cell records; planar tiles of one width share a launch at
        // the largest record size among them (a smaller record loads only
        // its own dwords), so a few odd tiles never run as a launch of
        // their own with too few workgroups to fill the device.
        for (int glob = 0; glob < 2; glob++)
        for (uint32_t w : {1u, 2u})
        for (int rot = 0; rot < 2; rot++) {
            fbh_ctx::Group g{(int)w, 0, (uint32_t)td.size(), 0, 0, 0, glob == 1, rot == 1};
            for (const fbh_ctx::Tile *t : built) {
                if (t->width != w || (int)t->global != glob || (int)t->rot != rot) continue;
                uint32_t lds, active_bytes;
                if (!add_tile(*t, lds, active_bytes)) continue;
                g.n_tiles++;
                g.rd = std::max(g.rd, (int)t->rec / 4);
                if (!t->global) g.lds_max = std::max(g.lds_max, lds);
                g.bytes_per_row += active_bytes;
            }
            if (g.n_tiles) {
                c->groups.push_back(g);
                c->has_global = c->has_global || g.global;
            }
        }
        // Streamed tiles: entries after the resident groups, launched one
        // window at a time.
        for (const auto &t : c->tiles) {
            if (t.resident) continue;
            uint32_t lds, active_bytes;
            const uint32_t k = (uint32_t)td.size();
            if (!add_tile(t, lds, active_bytes)) continue;
            c->streamed.push_back({(uint32_t)(&t - c->tiles.data()), k, lds, active_bytes});
        }
        // Tiles sharing one row bundle among those built.
        {
            std::map<int32_t, uint32_t> per_bundle;
            c->line_share = 1;
            for (const fbh_ctx::Tile *t : built)
                if (t->bundle >= 0)
                    c->line_share = std::max(c->line_share, ++per_bundle[t->bundle]);
        }
        // Tile-major copies for the root when the built tiles share bundle
        // lines: the root's rows are in order, so each workgroup then reads
        // its own tile's records contiguously and its chunks can be as long
        // as one wave of workgroups allows (fewer flushes of the LDS
        // histograms); deeper levels gather rows and keep the bundles.
        std::vector<TileDev> td_root;
        c->root_tm = false;
        if (c->line_share > 4 && c->streamed.empty() && !c->has_global &&
            c->plan.columns_resident && !c->groups.empty()) {
            bool ok = true;
            for (const auto &g : c->groups) ok = ok && !g.rot && !g.global;
            for (size_t i = 0; ok && i < td_src.size(); i++)
                ok = td_src[i] >= c->tiles.data() && td_src[i] < c->tiles.data() + c->tiles.size();
            if (ok) ok = ensure_tile_major(*c, td_src);
            if (ok) {
                td_root = td;
                for (size_t i = 0; i < td_root.size(); i++) {
                    td_root[i].data = td_src[i]->tm;
                    td_root[i].stride = td_src[i]->rec;
                }
                c->root_tm = true;
            }
        }
        c->hist_row_bytes = 0;
        c->hist_tiles = 0;
        for (const auto &g : c->groups) {
            c->hist_row_bytes += g.bytes_per_row;
            c->hist_tiles += g.n_tiles;
        }
        for (const auto &sd : c->streamed) c->hist_row_bytes += sd.bytes_per_row;
        c->bins_active = 0;
        for (uint32_t f : c->tree_feats) c->bins_active += c->n_bins[f];
        // split feature table
        std::vector<SplitFeatDev> sf;
        uint32_t cat_base = 0;
        for (uint32_t f : c->tree_feats) {
            SplitFeatDev s{};
            s.feat = f;
            s.hist_off = (uint32_t)c->hist_off[f];
            s.n_bins = c->n_bins[f];
            s.monotone = c->monotone[f];
            s.categorical = c->cat[f];
            if (c->cat[f]) {
                s.cat_words = (c->n_bins[f] + 63) / 64;
                s.cat_base = cat_base;
                cat_base += s.cat_words;
            }
            sf.push_back(s);
        }
        c->cat_words_per_node = cat_base;
        // The tables go up only when they differ from the last tree's (every
        // tree of a run without column sampling has the same).
        // Split-scan order: numeric features of at most 256 bins (one wave
        // each, four bins a lane), numeric ones of at most 1024 (one
        // workgroup each, four bins a thread), then the others (one
        // workgroup each).
        auto group = [&](uint32_t j) {
            if (sf[j].categorical || sf[j].n_bins > 1024) return 2;
            return sf[j].n_bins <= 256 ? 0 : 1;
        };
        std::vector<uint32_t> order;
        uint32_t counts[3] = {0, 0, 0};
        for (int k = 0; k < 3; k++)
            for (uint32_t j = 0; j < sf.size(); j++)
                if (group(j) == k) {
                    order.push_back(j);
                    counts[k]++;
                }
        c->n_split_num = counts[0];
        c->n_split_wide = counts[1];
        c->n_split_cat = counts[2];
        // Packed tiles' sources: 16 columns each (null for an empty cell).
        std::vector<PackTileDev> pk;
        for (const auto &t : c->pack_tiles) {
            PackTileDev d{};
            d.out = t.data;
            d.stride = t.stride;
            for (size_t k = 0; k < 16; k++) {
                const bool live = k < t.feats.size();
                d.col[k] = c->cols[t.feats[live ? k : 0]];
                d.live |= live ? 1u << k : 0u;
            }
            pk.push_back(d);
        }
        std::vector<uint8_t> tables(
            !td_root.empty() ? c->off_root + sizeof(TileDev) * td_root.size()
            : pk.empty()     ? c->off_order + 4 * order.size()
                             : c->off_pack + sizeof(PackTileDev) * pk.size(),
            0);
        std::memcpy(tables.data(), td.data(), sizeof(TileDev) * td.size());
        std::memcpy(tables.data() + c->off_tilefeats, tf.data(), sizeof(TileFeatDev) * tf.size());
        std::memcpy(tables.data() + c->off_sfeats, sf.data(), sizeof(SplitFeatDev) * sf.size());
        std::memcpy(tables.data() + c->off_order, order.data(), 4 * order.size());
        if (!pk.empty())
            std::memcpy(tables.data() + c->off_pack, pk.data(), sizeof(PackTileDev) * pk.size());
        if (!td_root.empty())
            std::memcpy(tables.data() + c->off_root, td_root.data(),
                        sizeof(TileDev) * td_root.size());
        const bool upload = tables != c->tree_tables;
        if (upload) {
            int slot;
            std::memcpy(c->stage_acquire(slot), tables.data(), tables.size());
            c->stage_send(slot, c->d_tiles, tables.size());
            c->tree_tables = std::move(tables);
        }
        // The packed records, unless the pack already holds these features.
        std::vector<uint32_t> sig;
        for (const auto &t : c->pack_tiles) {
            sig.push_back(0x80000000u | (t.width << 8) | (uint32_t)t.feats.size());
            sig.insert(sig.end(), t.feats.begin(), t.feats.end());
        }
        if (!sig.empty() && sig != c->pack_sig) {
            for (uint32_t w : {1u, 2u}) {
                uint32_t first = 0, n = 0;
                for (uint32_t i = 0; i < c->pack_tiles.size(); i++)
                    if (c->pack_tiles[i].width == w) {
                        if (n == 0) first = i;
                        n++;
                    }
                check(launch_pack_tiles(c->d_pack + first, n, w, c->n_rows, c->stream),
                      "tile packing");
            }
            c->pack_sig = std::move(sig);
        }
        // The delta is kept only for callers without a device objective.
        if (c->objective < 0 && !c->delta) c->delta = c->alloc<float>(c->n_rows, "prediction delta");
        // Callers without a device objective also clear their prediction delta.
        c->rows_identity = true;
        if (c->objective < 0) c->ensure_rows();
        c->tree_begun = true;
        root->offset = 0;
        root->len = (uint32_t)c->n_rows;
    });
}

}  // extern "C"

namespace {

// Launch tables of one blocking call, laid out in the pinned staging at
// 256-byte aligned offsets and sent to the device staging at the same
// offsets in one copy.
struct Stager {
    fbh_ctx *c;
    size_t o = 0;
    int slot = -1;
    uint8_t *host = nullptr;
    size_t put(const void *src, size_t bytes) {
        if (!host) host = c->stage_acquire(slot);
        const size_t at = o;
        const size_t next = at + ((bytes + 255) & ~size_t(255));
        if (next > c->stage_bytes) throw RuntimeError("launch tables exceed the staging buffer");
        if (bytes) std::memcpy(host + at, src, bytes);
        o = next;
        return at;
    }
    template <class T>
    T *dev(size_t off) const {
        return reinterpret_cast<T *>(c->d_stage + off);
    }
    void send() {
        if (o) c->stage_send(slot, c->d_stage, o);
    }
};

// Histograms, sibling subtraction and split scan of one batch of nodes. The
// accumulated-node table is planned on the host (exact chunks) or on the
// device (dev_chunk_rows set, grid_chunks an upper bound).
struct EvalPlan {
    const HistNodeDev *hn = nullptr;
    uint32_t n_hn = 0;
    uint32_t grid_chunks = 0;
    uint32_t chunk_rows = 0;
    const uint32_t *dev_chunk_rows = nullptr;
    const uint32_t *zero_slots = nullptr;  // host plan: slots to clear
    uint32_t n_zero = 0;
    const uint32_t *triples = nullptr;     // (dst, parent, sibling) slots
    uint32_t n_tri = 0;
    const SplitNodeDev *sn = nullptr;
    uint32_t n_nodes = 0;
    const uint8_t *enabled = nullptr;
    // Device-grown trees: counts read on the device (the host values above
    // are then upper bounds that size the grids).
    const uint32_t *dev_n_hn = nullptr, *dev_n_tri = nullptr, *dev_n_nodes = nullptr;
    bool download = true;  // copy the packets back (a device-grown tree reads them in place)
    // The level decision makes the packets from the candidates itself
    // (device-grown trees of few features): no argmax launch.
    bool fused_argmax = false;
    // hn[e], triples[3e..3e+2] and split nodes 2e, 2e + 1 describe evaluated
    // pair e (the accumulated child, the subtraction, the left and right
    // child): with every tree feature numeric of at most 256 bins, the chunk
    // reduction, subtraction and split scan then run as one pass
    // (split_pair_kernel). write_children: the children's histograms are
    // stored (they are parents of a later evaluation).
    bool pairs = false;
    bool write_children = true;
    const uint32_t *rows = nullptr;  // arena of the accumulated nodes (null: the row arena)
    bool cleared = false;            // the accumulated slots were cleared by the partition
    bool identity = false;           // the accumulated rows are in order (no arena read)
    // Per-chunk partial histograms (device-grown trees): multi-chunk nodes
    // store their chunks here and reduce_chunks_kernel sums them into the
    // slots; max_groups bounds the reduction groups of the launch.
    int64_t *partials = nullptr;
    uint32_t max_groups = 0;
    bool host_rule = false;  // planned with the host-driven chunk rule (HOST_HIST_WAVES)
    const TileDev *tiles = nullptr;  // the tile table (null: the tree's, d_tiles)
};

// Whether evaluated pairs of the current tree take split_pair_kernel: every
// tree feature numeric of at most 256 bins, and large slots. The one pass
// pays where slots are large (their reduction, subtraction and scan each move
// them); with small slots its few waves a pair (four features a workgroup)
// leave the device idler than three launches.
bool pair_pass_ok(const fbh_ctx *c) {
    return c->pair_pass && c->n_split_cat == 0 && c->n_split_wide == 0 && c->n_split_num > 0 &&
           c->hist_width * 16 >= PAIR_PASS_MIN_SLOT_BYTES;
}

void enqueue_eval(fbh_ctx *c, const EvalPlan &E, const fbh_split_params *sp) {
    const bool fuse_pairs = E.pairs && pair_pass_ok(c);
    if (!E.cleared) {
        if (E.dev_chunk_rows)
            check(launch_zero_nodes(c->hist, c->hist_width, E.hn, E.n_hn, E.dev_n_hn,
                                    c->has_global || !c->streamed.empty(),
                                    E.partials ? REDUCE_GROUP : 0u, c->stream),
                  "histogram clear");
        else
            check(launch_zero_slots(c->hist, c->hist_width, E.zero_slots, E.n_zero, c->stream),
                  "histogram clear");
    }
    if (E.n_hn && E.grid_chunks) {
        const size_t ev = c->ev_used;
        // Timing: the first resident launch takes the start event and the
        // last one the stop event on their dispatch; streamed windows (host
        // copies in between) are bracketed by event records instead.
        hipEvent_t ev_start = nullptr, ev_stop = nullptr;
        const bool marker = c->timing && (!c->streamed.empty() || c->groups.empty());
        if (c->timing) {
            if (c->ev_pool.size() <= ev) {
                hipEvent_t a, b;
                check(hipEventCreate(&a), "event");
                check(hipEventCreate(&b), "event");
                c->ev_pool.push_back({a, b});
            }
            if (marker) check(hipEventRecord(c->ev_pool[ev].first, c->stream), "event");
        }
        auto launch_base = [&]() {
            HistLaunch L{};
            L.feats = c->d_tilefeats;
            L.nodes = E.hn;
            L.n_nodes = E.n_hn;
            L.dev_n_nodes = E.dev_n_hn;
            L.n_chunks = E.grid_chunks;
            L.chunk_rows = E.chunk_rows;
            L.dev_chunk_rows = E.dev_chunk_rows;
            L.chunk_groups = div_up(E.grid_chunks, XCDS);
            // Chunk-major XCD locality needs at least one chunk per XCD.
            L.linear = c->chunk_rule(E.host_rule).want_chunks < XCDS ? 1u : 0u;
            L.rows = E.identity ? nullptr : (E.rows ? E.rows : c->rows);
            L.gpair = c->gpair;
            // Rows in order (the root) read the fixed-point pairs: there
            // the reads are contiguous and the LDS atomics bound the launch,
            // which quantizing in registers slowed (210 against 162 us).
            if (c->f32_pairs && !E.identity) {
                L.gpair_f32 = c->gpair_f32;
                L.scales = c->d_scales;
            }
            L.hist = c->hist;
            L.partials = E.partials;
            L.clear_above = fuse_pairs ? PAIR_MAX_CHUNKS : REDUCE_GROUP;
            L.hist_width = c->hist_width;
            return L;
        };
        for (size_t gi = 0; gi < c->groups.size(); gi++) {
            const auto &g = c->groups[gi];
            HistLaunch L = launch_base();
            L.tiles = (E.tiles ? E.tiles : c->d_tiles) + g.tile_begin;
            L.n_tiles = g.n_tiles;
            if (c->timing && !marker) {
                ev_start = gi == 0 ? c->ev_pool[ev].first : nullptr;
                ev_stop = gi + 1 == c->groups.size() ? c->ev_pool[ev].second : nullptr;
            }
            if (g.global)
                check(launch_hist_global(L, g.width, ev_start, ev_stop, c->stream),
                      "histogram launch");
            else
                check(launch_hist(L, g.width, g.rd, g.rot, c->hist_threads(g), false,
                                  (size_t)(g.lds_max + 64) * 16, ev_start, ev_stop, c->stream),
                      "histogram launch");
        }
        // Streamed tiles: row windows of their pinned host records go up
        // on the copy stream, alternating between two device windows;
        // each window's launch accumulates the rows it holds.
        for (const auto &sd : c->streamed) {
            const fbh_ctx::Tile &t = c->tiles[sd.tile];
            const uint64_t W = c->plan.window_rows;
            for (uint64_t lo = 0; lo < c->n_rows; lo += W) {
                const uint64_t hi = std::min<uint64_t>(c->n_rows, lo + W);
                const int b = (int)(c->win_flip++ % c->n_windows);
                check(hipStreamWaitEvent(c->copy_stream, c->win_free[b], 0), "stream wait");
                check(hipMemcpyAsync(c->win_rec[b], t.host + lo * t.stride, (hi - lo) * t.stride,
                                     hipMemcpyHostToDevice, c->copy_stream),
                      "record window upload");
                check(hipEventRecord(c->win_ready[b], c->copy_stream), "event");
                check(hipStreamWaitEvent(c->stream, c->win_ready[b], 0), "stream wait");
                HistLaunch L = launch_base();
                L.tiles = c->d_tiles + sd.entry;
                L.n_tiles = 1;
                L.stream_data = c->win_rec[b];
                L.row_lo = (uint32_t)lo;
                L.row_hi = (uint32_t)hi;
                check(launch_hist(L, (int)t.width, (int)(t.rec / 4), t.rot, 256, true,
                                  (size_t)(sd.lds_slots + 64) * 16, nullptr, nullptr, c->stream),
                      "streamed histogram launch");
                check(hipEventRecord(c->win_free[b], c->stream), "event");
            }
            c->streamed_bytes += c->n_rows * t.stride;
        }
        c->hist_launches++;
        if (c->timing) {
            if (marker) check(hipEventRecord(c->ev_pool[ev].second, c->stream), "event");
            c->ev_used++;
        }
    }
    if (E.partials)
        check(launch_reduce_chunks(c->hist, c->hist_width, E.partials, E.hn, E.n_hn, E.dev_n_hn,
                                   E.max_groups, fuse_pairs ? PAIR_MAX_CHUNKS + 1 : 0u,
                                   c->stream),
              "chunk reduction");
    // Device-grown pairs: the split scan subtracts (one launch less a level).
    const bool sub_in_scan = E.pairs && !fuse_pairs && c->sub_in_scan;
    if (!fuse_pairs && !sub_in_scan)
        check(launch_subtract(c->hist, c->hist_width, E.triples, E.n_tri, E.dev_n_tri, c->stream),
              "sibling subtraction");
    // ---- split scan ----
    SplitParamsDev P{};
    P.scales = c->d_scales;
    P.lambda_ = sp->lambda_;
    P.gamma = sp->gamma;
    P.mcw = sp->min_child_weight;
    P.alpha = sp->alpha;
    P.mds = sp->max_delta_step;
    P.max_cat_to_onehot = sp->max_cat_to_onehot;
    P.max_cat_threshold = sp->max_cat_threshold;
    P.n_feats = (uint32_t)c->tree_feats.size();
    P.cat_words_per_node = c->cat_words_per_node;
    if (fuse_pairs)
        check(launch_split_pairs(c->hist, c->hist_width, E.partials, E.hn, E.triples, E.n_hn,
                                 E.sn, c->d_sfeats, c->d_split_order, c->n_split_num, E.enabled,
                                 P, c->d_cands, E.dev_n_hn, E.write_children, c->stream),
              "pair reduction, subtraction and split scan");
    else
        check(launch_split_feats(c->hist, c->hist_width, E.sn, E.n_nodes, c->d_sfeats,
                                 c->d_split_order, c->n_split_num, c->n_split_wide,
                                 c->n_split_cat, E.enabled, P,
                                 c->d_cands, c->d_cat_scratch, E.dev_n_nodes,
                                 sub_in_scan ? E.triples : nullptr, E.write_children, c->stream),
              "split scan");
    const uint32_t cw = std::max(1u, c->cat_words_per_node);
    const size_t pk_bytes = sizeof(SplitPacketDev) * E.n_nodes;
    uint8_t *d_out = reinterpret_cast<uint8_t *>(c->d_packets);
    uint64_t *d_cats = reinterpret_cast<uint64_t *>(d_out + ((pk_bytes + 255) & ~size_t(255)));
    if (!E.fused_argmax)
        check(launch_split_nodes(c->d_cands, c->d_sfeats, E.n_nodes, P, E.sn, c->d_cat_scratch,
                                 c->d_packets, d_cats, cw, E.dev_n_nodes, c->stream),
              "split argmax");
    if (!E.download) return;
    // Packets and category sets land back to back: one download.
    const size_t out_bytes = c->cat_words_per_node > 0
                                 ? ((pk_bytes + 255) & ~size_t(255)) + 8 * (size_t)E.n_nodes * cw
                                 : pk_bytes;
    check(hipMemcpyAsync(c->pin_out.p, d_out, out_bytes, hipMemcpyDeviceToHost, c->stream),
          "packet download");
}

// Packets and category sets of n nodes out of the pinned results (after the
// stream synchronised).
void unpack_packets(fbh_ctx *c, uint32_t n, fbh_split *out, uint64_t *cat_words,
                    uint32_t cat_capacity) {
    static_assert(sizeof(SplitPacketDev) == sizeof(fbh_split), "packet layout");
    const uint8_t *po = static_cast<const uint8_t *>(c->pin_out.p);
    std::memcpy(out, po, sizeof(fbh_split) * n);
    if (c->cat_words_per_node == 0) return;
    const uint32_t cw = c->cat_words_per_node;
    const size_t pk_bytes = sizeof(SplitPacketDev) * n;
    const uint64_t *words = reinterpret_cast<const uint64_t *>(po + ((pk_bytes + 255) & ~size_t(255)));
    for (uint32_t i = 0; i < n; i++) {
        if (!out[i].found || !out[i].is_cat) continue;
        if (!cat_words || (uint64_t)out[i].cat_offset + out[i].n_cat_words > cat_capacity)
            throw InputError("cat_words capacity is too small for the category sets");
        std::memcpy(cat_words + out[i].cat_offset, words + (size_t)i * cw, 8 * out[i].n_cat_words);
    }
}

// Algorithmic bytes of one histogram launch: cells + gpair (16) + row id (4)
// per accumulated row, and the written histogram (2 x 16 per bin) per node.
// The pair counts as the algorithm's 16-byte fixed-point pair also where the
// kernel reads it as 8 bytes of f32 and quantizes it in registers.
void account_hist(fbh_ctx *c, uint64_t acc_rows, uint64_t nodes_with_rows) {
    if (nodes_with_rows == 0) return;
    c->hist_bytes += acc_rows * (c->hist_row_bytes + 20) + nodes_with_rows * 32 * c->bins_active;
}

}  // namespace

extern "C" {

}  // extern "C"

namespace {

// Validates a batch of nodes and stages the tables of its evaluation as
// planned on the host: exact chunks of the accumulated nodes, slots to
// clear, subtraction triples and split-scan nodes. Returns the accumulated
// rows and the accumulated nodes with rows (for the byte count).
std::pair<uint64_t, uint64_t> stage_host_eval(fbh_ctx *c, const fbh_node *nodes, uint32_t n,
                                              const uint8_t *enabled, Stager &S, EvalPlan &E) {
        for (uint32_t i = 0; i < n; i++) {
            const fbh_node &nd = nodes[i];
            if (nd.slot >= c->n_slots) throw InputError("histogram slot out of range");
            if ((uint64_t)nd.rows.offset + nd.rows.len > c->n_rows)
                throw InputError("row span out of range");
            if (nd.subtract_parent >= 0) {
                if ((uint32_t)nd.subtract_parent >= c->n_slots)
                    throw InputError("parent slot out of range");
                if (nd.subtract_sibling < 0 || (uint32_t)nd.subtract_sibling >= n ||
                    nodes[nd.subtract_sibling].subtract_parent >= 0)
                    throw InputError("subtract sibling must be an accumulated node of the call");
            }
        }
        // ---- histograms of accumulated nodes, planned here ----
        std::vector<HistNodeDev> hn;
        std::vector<uint32_t> zero_slots;
        uint32_t chunks = 0;
        uint64_t acc_rows = 0;
        std::vector<uint32_t> acc_lens;
        for (uint32_t i = 0; i < n; i++)
            if (nodes[i].subtract_parent < 0) {
                acc_rows += nodes[i].rows.len;
                acc_lens.push_back(nodes[i].rows.len);
            }
        const uint32_t chunk_rows = c->chunk_rows_for(acc_lens.data(), acc_lens.size(), true);
        E.host_rule = true;
        uint64_t all_chunks = 0;
        for (uint32_t i = 0; i < n; i++)
            if (nodes[i].subtract_parent < 0) all_chunks += div_up(nodes[i].rows.len, chunk_rows);
        // Multi-chunk nodes store per-chunk partials (summed by the chunk
        // reduction) when the buffer allows; only nodes of more than
        // REDUCE_GROUP chunks, or without rows, then need a zeroed slot.
        E.partials = c->partial_buffer(all_chunks * c->hist_width * 16);
        uint32_t groups = 0;
        for (uint32_t i = 0; i < n; i++) {
            const fbh_node &nd = nodes[i];
            if (nd.subtract_parent >= 0) continue;
            const uint32_t nc = div_up(nd.rows.len, chunk_rows);
            // Single-chunk nodes are written by plain stores, except that a
            // globally accumulated feature needs a zeroed slot.
            const bool atomic = E.partials ? (nc == 0 || nc > REDUCE_GROUP) : nc != 1;
            if (atomic || c->has_global || !c->streamed.empty()) zero_slots.push_back(nd.slot);
            if (nc == 0) continue;
            HistNodeDev h{};
            h.row_off = nd.rows.offset;
            h.row_len = nd.rows.len;
            h.chunk_begin = chunks;
            h.slot = nd.slot;
            h.n_chunks = nc;
            h.group_begin = groups;
            hn.push_back(h);
            chunks += nc;
            groups += reduce_groups(nc);
        }
        E.max_groups = groups;
        std::vector<uint32_t> triples;
        for (uint32_t i = 0; i < n; i++) {
            const fbh_node &nd = nodes[i];
            if (nd.subtract_parent < 0) continue;
            triples.push_back(nd.slot);
            triples.push_back((uint32_t)nd.subtract_parent);
            triples.push_back(nodes[nd.subtract_sibling].slot);
        }
        std::vector<SplitNodeDev> sn(n);
        for (uint32_t i = 0; i < n; i++) {
            sn[i].sum_g = nodes[i].sum[0];
            sn[i].sum_h = nodes[i].sum[1];
            sn[i].lower = nodes[i].lower;
            sn[i].upper = nodes[i].upper;
            sn[i].slot = nodes[i].slot;
        }
        E.hn = S.dev<HistNodeDev>(S.put(hn.data(), sizeof(HistNodeDev) * hn.size()));
        E.n_hn = (uint32_t)hn.size();
        E.grid_chunks = chunks;
        E.chunk_rows = chunk_rows;
        E.zero_slots = S.dev<uint32_t>(S.put(zero_slots.data(), 4 * zero_slots.size()));
        E.n_zero = (uint32_t)zero_slots.size();
        E.triples = S.dev<uint32_t>(S.put(triples.data(), 4 * triples.size()));
        E.n_tri = (uint32_t)(triples.size() / 3);
        E.sn = S.dev<SplitNodeDev>(S.put(sn.data(), sizeof(SplitNodeDev) * n));
        E.n_nodes = n;
        if (enabled)
            E.enabled = S.dev<uint8_t>(S.put(enabled, (size_t)n * c->tree_feats.size()));
        return {acc_rows, (uint64_t)hn.size()};
}

}  // namespace

extern "C" {

int fbh_eval_nodes(fbh_ctx *c, const fbh_node *nodes, uint32_t n, const fbh_split_params *sp,
                   const uint8_t *enabled, fbh_split *out, uint64_t *cat_words,
                   uint32_t cat_capacity) {
    return guard([&] {
        if (!c || (!nodes && n) || !sp || (!out && n)) throw InputError("null argument");
        ensure_tree(c);
        if (n == 0) return;
        if (n > c->n_slots) throw InputError("more nodes than histogram slots");
        check(hipSetDevice(c->device), "hipSetDevice");
        c->ensure_rows();
        Stager S{c};
        EvalPlan E;
        const auto acc = stage_host_eval(c, nodes, n, enabled, S, E);
        S.send();
        enqueue_eval(c, E, sp);
        c->sync();
        if (c->timing) c->collect_timing();
        account_hist(c, acc.first, acc.second);
        unpack_packets(c, n, out, cat_words, cat_capacity);
    });
}

int fbh_download_histogram(fbh_ctx *c, uint32_t slot, int64_t *out, uint64_t *width_out) {
    return guard([&] {
        if (!c) throw InputError("null argument");
        ensure_tree(c);
        if (width_out) *width_out = c->hist_width;
        if (!out) return;
        if (slot >= c->n_slots) throw InputError("histogram slot out of range");
        check(hipMemcpyAsync(out, c->hist + (uint64_t)slot * c->hist_width * 2,
                             c->hist_width * 16, hipMemcpyDeviceToHost, c->stream),
              "histogram download");
        c->sync();
    });
}

}  // extern "C"

namespace {

// Partition tables of one call: the requests with rows (in call order),
// their count groups (requests whose split cells are on the device, then one
// group per streamed feature) and their places in the staging.
struct PartStage {
    std::vector<PartReqDev> pr;
    std::vector<uint32_t> which;   // pr index -> request index
    std::vector<uint32_t> req_of;  // request index -> pr index, NO_SLOT without rows
    std::vector<PartReqDev> grp;
    std::vector<std::pair<uint32_t, uint32_t>> groups;  // (first, count) in grp
    std::vector<uint32_t> group_feat;                  // UINT32_MAX: on the device
    std::vector<int> group_win;                        // column window of a streamed group
    uint32_t chunks = 0;
    size_t o_pr = 0, o_cats = 0, o_grp = 0;
};

PartStage stage_partition(fbh_ctx *c, const fbh_part_req *reqs, uint32_t n,
                          const uint64_t *cat_words, uint32_t n_cat_words, Stager &S) {
    PartStage P;
    P.req_of.assign(n, NO_SLOT);
    for (uint32_t i = 0; i < n; i++) {
        const fbh_part_req &r = reqs[i];
        if ((uint64_t)r.rows.offset + r.rows.len > c->n_rows)
            throw InputError("row span out of range");
        if (r.feat >= c->n_features) throw InputError("feature id out of range");
        if (r.n_cat_words && (uint64_t)r.cat_offset + r.n_cat_words > n_cat_words)
            throw InputError("category set out of range");
        if (r.rows.len == 0) continue;
        const auto &t = c->tiles[c->feat_tile[r.feat]];
        PartReqDev d{};
        d.row_off = r.rows.offset;
        d.row_len = r.rows.len;
        d.chunk_begin = P.chunks;
        d.count_base = P.chunks;
        d.n_chunks = div_up(r.rows.len, PART_CHUNK);
        if (c->plan.columns_resident) {  // the resident column
            d.data = c->cols[r.feat];
            d.stride = t.width;
            d.byte_off = 0;
        } else if (t.resident) {  // the cell inside the resident records
            d.data = t.data;
            d.stride = t.stride;
            d.byte_off = (uint32_t)c->feat_pos[r.feat] * t.width;
        } else {  // a streamed column, set per feature group below
            d.data = nullptr;
            d.stride = t.width;
            d.byte_off = 0;
        }
        d.width = t.width;
        d.missing = c->missing_code(r.feat);
        d.bin = r.bin;
        d.missing_left = r.missing_left;
        d.cat_off = r.cat_offset;
        d.n_cat_words = r.n_cat_words;
        P.req_of[i] = (uint32_t)P.pr.size();
        P.pr.push_back(d);
        P.which.push_back(i);
        P.chunks += d.n_chunks;
    }
    if (P.pr.empty()) return P;
    if (P.chunks > c->max_chunks)
        throw InputError("partition spans overlap or exceed the row arena");
    if (n_cat_words > c->cat_in_words)
        throw InputError("too many category words for one partition call");
    // A group numbers its own chunks; counts land at each request's place in
    // the call's chunk arrays.
    std::vector<uint32_t> order(P.pr.size());
    for (uint32_t k = 0; k < P.pr.size(); k++) order[k] = k;
    auto feat_of = [&](uint32_t k) { return reqs[P.which[k]].feat; };
    auto key = [&](uint32_t k) -> uint64_t { return P.pr[k].data ? 0 : 1 + (uint64_t)feat_of(k); };
    std::stable_sort(order.begin(), order.end(),
                     [&](uint32_t a, uint32_t b) { return key(a) < key(b); });
    uint32_t local = 0;
    for (size_t j = 0; j < order.size(); j++) {
        const uint32_t k = order[j];
        if (j == 0 || key(k) != key(order[j - 1])) {
            P.groups.push_back({(uint32_t)P.grp.size(), 0});
            P.group_feat.push_back(P.pr[k].data ? UINT32_MAX : feat_of(k));
            local = 0;
        }
        PartReqDev g = P.pr[k];
        g.chunk_begin = local;
        local += g.n_chunks;
        P.grp.push_back(g);
        P.groups.back().second++;
    }
    // Streamed groups alternate between the column windows.
    P.group_win.assign(P.groups.size(), -1);
    for (size_t gi = 0; gi < P.groups.size(); gi++) {
        if (P.group_feat[gi] == UINT32_MAX) continue;
        P.group_win[gi] = (int)(c->col_flip++ % c->n_windows);
        for (uint32_t k = P.groups[gi].first; k < P.groups[gi].first + P.groups[gi].second; k++)
            P.grp[k].data = c->win_col[P.group_win[gi]];
    }
    P.o_pr = S.put(P.pr.data(), sizeof(PartReqDev) * P.pr.size());
    P.o_cats = S.put(cat_words, n_cat_words ? 8 * (size_t)n_cat_words : 0);
    P.o_grp = S.put(P.grp.data(), sizeof(PartReqDev) * P.grp.size());
    return P;
}

// Count passes (streamed features after their column's upload), then the
// scan, stable scatter and copy back; left totals land in d_totals by pr index.
void enqueue_partition(fbh_ctx *c, const PartStage &P, const Stager &S) {
    const uint64_t *d_cats = S.dev<const uint64_t>(P.o_cats);
    PartReqDev *d_grp = S.dev<PartReqDev>(P.o_grp);
    for (size_t gi = 0; gi < P.groups.size(); gi++) {
        const uint32_t first = P.groups[gi].first, cnt = P.groups[gi].second;
        uint32_t g_chunks = 0;
        for (uint32_t k = first; k < first + cnt; k++) g_chunks += P.grp[k].n_chunks;
        if (P.group_feat[gi] != UINT32_MAX) {
            // A streamed feature: its column goes up into the group's window.
            const uint32_t f = P.group_feat[gi];
            const int b = P.group_win[gi];
            const uint64_t bytes = c->n_rows * c->width[f];
            check(hipStreamWaitEvent(c->copy_stream, c->win_free[2 + b], 0), "stream wait");
            check(hipMemcpyAsync(c->win_col[b], c->host_cols[f], bytes, hipMemcpyHostToDevice,
                                 c->copy_stream),
                  "column window upload");
            check(hipEventRecord(c->win_ready[2 + b], c->copy_stream), "event");
            c->streamed_bytes += bytes;
            check(hipStreamWaitEvent(c->stream, c->win_ready[2 + b], 0), "stream wait");
            check(launch_partition_count(d_grp + first, cnt, g_chunks, c->rows, c->flags,
                                         c->d_counts, d_cats, c->stream),
                  "partition count");
            check(hipEventRecord(c->win_free[2 + b], c->stream), "event");
        } else {
            check(launch_partition_count(d_grp + first, cnt, g_chunks, c->rows, c->flags,
                                         c->d_counts, d_cats, c->stream),
                  "partition count");
        }
    }
    check(launch_partition_finish(S.dev<const PartReqDev>(P.o_pr), (uint32_t)P.pr.size(),
                                  P.chunks, c->rows, c->tmp, c->flags, c->d_counts, c->d_excl,
                                  c->d_totals, c->stream),
          "partition");
}

}  // namespace

extern "C" {

int fbh_partition(fbh_ctx *c, const fbh_part_req *reqs, uint32_t n, const uint64_t *cat_words,
                  uint32_t n_cat_words, fbh_span *children) {
    return guard([&] {
        if (!c || (!reqs && n) || (!children && n)) throw InputError("null argument");
        ensure_tree(c);
        if (n == 0) return;
        if (n > MAX_NODES) throw InputError("too many partition requests");
        check(hipSetDevice(c->device), "hipSetDevice");
        c->ensure_rows();
        Stager S{c};
        const PartStage P = stage_partition(c, reqs, n, cat_words, n_cat_words, S);
        for (uint32_t i = 0; i < n; i++) {
            children[2 * i] = {reqs[i].rows.offset, 0};
            children[2 * i + 1] = {reqs[i].rows.offset, 0};
        }
        if (P.pr.empty()) return;
        S.send();
        enqueue_partition(c, P, S);
        check(hipMemcpyAsync(c->pin_out.p, c->d_totals, 4 * P.pr.size(), hipMemcpyDeviceToHost,
                             c->stream),
              "partition totals");
        c->sync();
        const uint32_t *tot = static_cast<const uint32_t *>(c->pin_out.p);
        for (size_t k = 0; k < P.pr.size(); k++) {
            const uint32_t i = P.which[k];
            const uint32_t nl = tot[k];
            children[2 * i] = {reqs[i].rows.offset, nl};
            children[2 * i + 1] = {reqs[i].rows.offset + nl, reqs[i].rows.len - nl};
        }
    });
}

int fbh_partition_eval(fbh_ctx *c, const fbh_part_req *reqs, uint32_t n,
                       const uint64_t *cat_words, uint32_t n_cat_words,
                       const fbh_child_pair *pairs, const fbh_split_params *sp,
                       fbh_span *children, uint32_t *left_slot, fbh_split *out,
                       uint64_t *cat_out, uint32_t cat_capacity) {
    return fbh_partition_eval_masked(c, reqs, n, cat_words, n_cat_words, pairs, sp, nullptr,
                                     children, left_slot, out, cat_out, cat_capacity);
}

int fbh_partition_eval_masked(fbh_ctx *c, const fbh_part_req *reqs, uint32_t n,
                              const uint64_t *cat_words, uint32_t n_cat_words,
                              const fbh_child_pair *pairs, const fbh_split_params *sp,
                              const uint8_t *enabled, fbh_span *children, uint32_t *left_slot,
                              fbh_split *out, uint64_t *cat_out, uint32_t cat_capacity) {
    return guard([&] {
        if (!c || (n && (!reqs || !pairs || !children || !left_slot)) || !sp)
            throw InputError("null argument");
        ensure_tree(c);
        if (n == 0) return;
        if (n > MAX_NODES) throw InputError("too many partition requests");
        check(hipSetDevice(c->device), "hipSetDevice");
        c->ensure_rows();
        // Every slot of the evaluated pairs is used once: the larger child
        // takes over the parent's slot, the smaller one accumulates into its own.
        std::vector<uint8_t> used(c->n_slots, 0);
        uint32_t n_eval = 0;
        for (uint32_t i = 0; i < n; i++) {
            if (!pairs[i].evaluate) continue;
            const uint32_t a = pairs[i].parent_slot, b = pairs[i].new_slot;
            if (a >= c->n_slots || b >= c->n_slots) throw InputError("histogram slot out of range");
            if (a == b || used[a] || used[b])
                throw InputError("each slot of the evaluated pairs must be used once");
            used[a] = used[b] = 1;
            n_eval++;
        }
        if (n_eval && !out) throw InputError("null argument");
        Stager S{c};
        const PartStage P = stage_partition(c, reqs, n, cat_words, n_cat_words, S);
        std::vector<PairDev> pd(n);
        std::vector<uint32_t> triples;
        const ChunkRule rule = c->chunk_rule(true);
        uint64_t bound_rule = rule_chunk_bound(rule, c->n_rows, n_eval);
        uint64_t bound_min = 0;  // the smaller child holds at most half its parent's rows
        uint32_t e = 0;
        for (uint32_t i = 0; i < n; i++) {
            const fbh_child_pair &q = pairs[i];
            PairDev &d = pd[i];
            d.req = P.req_of[i];
            d.row_off = reqs[i].rows.offset;
            d.row_len = d.req == NO_SLOT ? 0 : reqs[i].rows.len;
            d.parent_slot = q.parent_slot;
            d.new_slot = q.new_slot;
            d.eval_index = q.evaluate ? e++ : NO_SLOT;
            for (int k = 0; k < 2; k++) {
                d.lower[k] = q.lower[k];
                d.upper[k] = q.upper[k];
                d.left_sum[k] = q.left_sum[k];
                d.right_sum[k] = q.right_sum[k];
            }
            if (!q.evaluate) continue;
            triples.push_back(q.parent_slot);
            triples.push_back(q.parent_slot);
            triples.push_back(q.new_slot);
            bound_min += div_up(d.row_len / 2, rule.fixed ? rule.fixed : rule.min_rows);
        }
        const size_t o_pairs = S.put(pd.data(), sizeof(PairDev) * n);
        const size_t o_tri = S.put(triples.data(), 4 * triples.size());
        // children's masks, (left, right) per evaluated pair: the split
        // nodes' order of the level plan
        const size_t o_en =
            enabled && n_eval ? S.put(enabled, (size_t)2 * n_eval * c->tree_feats.size()) : 0;
        S.send();
        if (!P.pr.empty()) enqueue_partition(c, P, S);
        check(launch_level_plan(S.dev<const PairDev>(o_pairs), n, c->d_totals, rule,
                                c->d_lvl_hist, c->d_lvl_split, c->d_lvl_out,
                                c->d_lvl_out + 4 * (size_t)n, c->d_lvl_rows, GrowDevOut{},
                                c->stream),
              "level plan");
        if (n_eval) {
            EvalPlan E;
            E.hn = c->d_lvl_hist;
            E.n_hn = n_eval;
            E.grid_chunks = (uint32_t)(rule.fixed ? bound_min : std::min(bound_rule, bound_min));
            E.dev_chunk_rows = c->d_lvl_rows;
            E.partials = c->partial_buffer((uint64_t)E.grid_chunks * c->hist_width * 16);
            E.max_groups = E.grid_chunks / REDUCE_GROUP + n_eval + 1;
            E.host_rule = true;
            E.triples = S.dev<const uint32_t>(o_tri);
            E.n_tri = n_eval;
            E.sn = c->d_lvl_split;
            E.n_nodes = 2 * n_eval;
            if (enabled) E.enabled = S.dev<const uint8_t>(o_en);
            enqueue_eval(c, E, sp);
        }
        uint8_t *po = static_cast<uint8_t *>(c->pin_out.p);
        check(hipMemcpyAsync(po + c->pin_out_spans, c->d_lvl_out, 20 * (size_t)n,
                             hipMemcpyDeviceToHost, c->stream),
              "children download");
        c->sync();
        if (c->timing) c->collect_timing();
        const uint32_t *sp4 = reinterpret_cast<const uint32_t *>(po + c->pin_out_spans);
        uint64_t acc = 0, with_rows = 0;
        for (uint32_t i = 0; i < n; i++) {
            children[2 * i] = {sp4[4 * i], sp4[4 * i + 1]};
            children[2 * i + 1] = {sp4[4 * i + 2], sp4[4 * i + 3]};
            left_slot[i] = sp4[4 * (size_t)n + i];
            if (pairs[i].evaluate) {
                const uint32_t small = std::min(sp4[4 * i + 1], sp4[4 * i + 3]);
                acc += small;
                with_rows += small ? 1 : 0;
            }
        }
        account_hist(c, acc, with_rows);
        if (n_eval) unpack_packets(c, 2 * n_eval, out, cat_out, cat_capacity);
    });
}

}  // extern "C"

namespace {

constexpr uint32_t MAX_GROW_DEPTH = 14;


// Every tile's records in one row bundle of at most 64 bytes (the leaf
// walk holds a row in 16 registers): a row's cells for every feature are in
// one record, so leaves can be found by walking the tree in row order.
bool single_bundle(const fbh_ctx &c) {
    if (c.bundles.size() != 1 || c.bundles[0].pitch > 64) return false;
    for (const auto &t : c.tiles)
        if (t.bundle != 0 || t.global) return false;
    return true;
}

// Buffers of device-grown trees up to depth D (grown, never shrunk).
void ensure_grow(fbh_ctx *c, uint32_t D) {
    auto &G = c->grow;
    const uint32_t cw = std::max(1u, c->max_cat_words);
    if (!G.cols) {
        G.st = c->alloc<GrowState>(1, "grown tree state");
        G.root_tables = c->alloc<uint8_t>(256 + c->n_features, "grown tree root tables");
        G.h_root_hn.n_chunks = ~0u;  // never a real plan: the first tree uploads
        G.cols = c->alloc<DevColumn>(c->n_features, "grown tree columns");
        std::vector<DevColumn> cols(c->n_features);
        for (uint32_t f = 0; f < c->n_features; f++)
            cols[f] = {c->cols[f], c->width[f], c->missing_code(f)};
        check(hipMemcpy(G.cols, cols.data(), sizeof(DevColumn) * cols.size(),
                        hipMemcpyHostToDevice),
              "column table");
        if (single_bundle(*c)) {
            std::vector<uint16_t> off(c->n_features);
            for (uint32_t f = 0; f < c->n_features; f++) {
                const auto &t = c->tiles[c->feat_tile[f]];
                off[f] = (uint16_t)((t.bundle_off + c->feat_pos[f] * t.width) |
                                    (t.width == 2 ? 0x8000u : 0u) |
                                    (c->missing_code(f) == 0x100u ? 0x4000u : 0u));
            }
            G.feat_off = c->alloc<uint16_t>(c->n_features, "grown tree feature offsets");
            check(hipMemcpy(G.feat_off, off.data(), 2 * off.size(), hipMemcpyHostToDevice),
                  "feature offsets");
        }
    }
    if (G.depth >= D) return;
    if (!G.pending.empty())
        throw InputError("a deeper tree cannot start while grown trees wait to be collected");
    G.depth = D;
    G.level_cap = (size_t)1 << (D - 1);
    G.tree_cap = ((size_t)2 << D) - 1;
    G.leaf_cap = (size_t)1 << D;
    G.cat_cap = G.leaf_cap * cw;
    G.level[0] = c->alloc<LNodeDev>(G.level_cap, "grown tree level");
    G.level[1] = c->alloc<LNodeDev>(G.level_cap, "grown tree level");
    G.tree = c->alloc<TreeNodeDev>(G.tree_cap, "grown tree nodes");
    G.tree_cats = c->alloc<uint64_t>(G.cat_cap, "grown tree categories");
    G.reqs = c->alloc<PartReqDev>(G.level_cap, "grown tree requests");
    G.pairs = c->alloc<PairDev>(G.level_cap, "grown tree pairs");
    G.triples = c->alloc<uint32_t>(3 * G.level_cap, "grown tree triples");
    G.leaves = c->alloc<LeafDev>(G.leaf_cap, "grown tree leaves");
    G.leaf_vals = c->alloc<float>(G.leaf_cap, "grown tree leaf values");
    for (int k = 0; k < 2; k++) {
        if (G.out[k].p) (void)hipHostFree(G.out[k].p);
        G.out[k].p = nullptr;
        // Coherent: the kernel's writes go to host memory, not the device caches.
        const size_t bytes = al256(sizeof(GrowState)) + al256(sizeof(TreeNodeDev) * G.tree_cap) +
                             al256(8 * G.cat_cap) + al256(4 * G.leaf_cap);
        check(hipHostMalloc(&G.out[k].p, bytes, hipHostMallocCoherent), "pinned host allocation");
        G.out[k].bytes = bytes;
        void *dv = nullptr;
        check(hipHostGetDevicePointer(&dv, G.out[k].p, 0), "device view of the tree buffer");
        G.out_dev[k] = static_cast<uint8_t *>(dv);
        if (!G.done[k])
            check(hipEventCreateWithFlags(&G.done[k], hipEventDisableTiming), "event");
    }
}

}  // namespace

extern "C" {

}  // extern "C"

namespace {

// Enqueues a whole depthwise tree (see fbh_grow_depthwise) and its download
// into the next of two pinned result slots; returns without waiting.
void grow_enqueue(fbh_ctx *c, const fbh_grow_params *gp, const fbh_split_params *sp,
                  const int64_t *root_sum) {
    if (!c || !gp || !sp) throw InputError("null argument");
    ensure_tree(c);
    const uint32_t D = gp->max_depth;
    if (D == 0 || D > MAX_GROW_DEPTH)
        throw InputError("a device-grown tree needs max_depth in 1..=" +
                         std::to_string(MAX_GROW_DEPTH));
    if (gp->max_leaves == 1) throw InputError("max_leaves 1 leaves nothing to grow");
    if (gp->flags & ~(uint32_t)FBH_GROW_DEFER_LEAVES) throw InputError("unknown grow flags");
    if ((gp->flags & FBH_GROW_DEFER_LEAVES) && c->objective < 0)
        throw InputError("deferred leaf values need a device objective (fbh_set_objective)");
    if (c->leaves_deferred)
        throw InputError("the last grown tree's leaf values were deferred and not applied "
                         "(fbh_apply_leaf_values)");
    if (!c->plan.columns_resident || !c->streamed.empty())
        throw InputError("a device-grown tree needs every tile and column resident");
    if (c->n_slots > MAX_GROW_SLOTS)
        throw InputError("a device-grown tree supports at most " + std::to_string(MAX_GROW_SLOTS) +
                         " histogram slots");
    if (!root_sum && !c->root_on_device)
        throw InputError("no root sum: pass it, or compute the gradients on the device first");
    auto &GB = c->grow;
    if (GB.pending.size() >= 2)
        throw InputError("two grown trees are waiting; collect one with fbh_grow_collect");
    check(hipSetDevice(c->device), "hipSetDevice");
    ensure_grow(c, D);
    const uint32_t n_rows = (uint32_t)c->n_rows;
    const uint32_t n_slots = c->n_slots;
    auto lvl_bound = [&](uint32_t d) { return std::min<uint32_t>(1u << d, n_slots); };

    // Leaves by a row-order walk of the finished tree (no last-level
    // partition, no scattered leaf ids) when one bundle holds every cell and
    // the tree fits the walk's LDS table. Without leaf spans to assign, the
    // root's rows need not be written out: its accumulation and partition
    // take the identity.
    const bool walk = GB.feat_off && ((2u << D) - 1) <= MAX_WALK_NODES;
    if (!walk) c->ensure_rows();
    const bool ident = c->rows_identity;

    // The root: one accumulated node over every row, planned here (the
    // table and the monotone constraints go up only when they change); its
    // split node (sums, bounds) is written by the prep kernel from the root
    // sum, which also clears the root's slot when it accumulates atomically.
    // With tile-major root records (the root's rows are 0..n in order,
    // through the arena or not) no chunk shares bundle lines with another
    // tile's workgroups: chunks as long as one wave allows.
    const bool root_tm = c->root_tm;
    const uint32_t cr = c->chunk_rows_for(n_rows, root_tm);
    HistNodeDev h{};
    h.row_off = 0;
    h.row_len = n_rows;
    h.chunk_begin = 0;
    h.slot = 0;
    h.n_chunks = div_up(n_rows, cr);
    const bool new_hn = std::memcmp(&h, &GB.h_root_hn, sizeof(h)) != 0;
    const bool new_mono = c->monotone != GB.h_mono;
    if (new_hn || new_mono) {
        int slot;
        uint8_t *hp = c->stage_acquire(slot);
        std::memcpy(hp, &h, sizeof(h));
        std::memcpy(hp + 256, c->monotone.data(), c->n_features);
        c->stage_send(slot, GB.root_tables, 256 + c->n_features);
        GB.h_root_hn = h;
        GB.h_mono = c->monotone;
    }
    EvalPlan E0;
    E0.hn = reinterpret_cast<const HistNodeDev *>(GB.root_tables);
    E0.n_hn = 1;
    E0.grid_chunks = h.n_chunks;
    E0.chunk_rows = cr;
    E0.identity = ident;
    if (root_tm) E0.tiles = c->d_root_tiles;
    // Per-chunk partials instead of global atomics for multi-chunk nodes when
    // every tile is an LDS tile and the buffer (grid chunks x histogram) is
    // modest; only nodes of more than REDUCE_GROUP chunks then need cleared
    // slots (their groups add atomically).
    ChunkRule rule = c->chunk_rule();
    // Levels below the root take the one-pass pair step where it applies
    // (their evaluations set EvalPlan::pairs): only nodes of more than
    // PAIR_MAX_CHUNKS chunks then need reduction groups.
    if (pair_pass_ok(c)) rule.group_min_chunks = PAIR_MAX_CHUNKS + 1;
    auto level_grid = [&](uint32_t nb) {
        return rule.fixed ? n_rows / rule.fixed + nb + 1 : rule_chunk_bound(rule, n_rows, nb);
    };
    uint64_t all_bins = 0;
    for (uint32_t b : c->n_bins) all_bins += b;
    const uint64_t max_grid = std::max<uint64_t>(h.n_chunks, level_grid(lvl_bound(D - 1)));
    int64_t *partials = c->partial_buffer(max_grid * all_bins * 16);
    E0.partials = partials;
    E0.max_groups = reduce_groups(h.n_chunks);
    // With partials a node of several reduction groups has its slot cleared
    // by the histogram launch itself (its first chunk's workgroups).
    const bool root_atomic = partials ? false : h.n_chunks != 1;
    const bool clear_root = root_atomic || c->has_global;
    E0.cleared = true;
    E0.sn = c->d_lvl_split;
    E0.n_nodes = 1;
    E0.download = false;
    // The level decision picks each node's split itself (from candidates it
    // stages in LDS, or one thread a node scanning them) when the tree has
    // few features, or up to FUSED_STAGED_FEATS when the level's candidates
    // fit the staging (one thread a node scanning more features from LDS is
    // slower than split_node_kernel's workgroup a node: 400k x 2000 at 1000
    // features a tree lost 2 %).
    const size_t n_tf = c->tree_feats.size();
    auto fuse_at = [&](uint32_t d) {
        return n_tf <= FUSED_ARGMAX_FEATS ||
               (n_tf <= FUSED_STAGED_FEATS && (uint64_t)lvl_bound(d) * n_tf <= DECIDE_CAND_LDS);
    };
    E0.fused_argmax = fuse_at(0);
    // A root sum from the host is staged; else the prep kernel sums the
    // quantisation's block sums.
    const int64_t *d_root = nullptr;
    if (root_sum) {
        Stager S{c};
        d_root = S.dev<const int64_t>(S.put(root_sum, 16));
        S.send();
    }
    const int8_t *d_mono = reinterpret_cast<const int8_t *>(GB.root_tables + 256);

    GrowParamsDev G{};
    G.sp.scales = c->d_scales;
    G.sp.lambda_ = sp->lambda_;
    G.sp.gamma = sp->gamma;
    G.sp.mcw = sp->min_child_weight;
    G.sp.alpha = sp->alpha;
    G.sp.mds = sp->max_delta_step;
    G.sp.max_cat_to_onehot = sp->max_cat_to_onehot;
    G.sp.max_cat_threshold = sp->max_cat_threshold;
    G.sp.n_feats = (uint32_t)c->tree_feats.size();
    G.sp.cat_words_per_node = c->cat_words_per_node;
    G.learning_rate = gp->learning_rate;
    G.max_depth = D;
    G.max_leaves = gp->max_leaves;
    G.n_slots = n_slots;
    G.cw = std::max(1u, c->cat_words_per_node);
    G.n_rows = n_rows;
    // One-pass partitions need partials (no slot is cleared before the next
    // level's histograms) and few chunks a node (one_pass_chunks); the level
    // decision then zeroes each split node's cursors. Partials never exist
    // with streamed tiles, whose windows find a node's rows by binary search
    // and so need the ascending row ids of the three-pass partition.
    auto one_pass_at = [&](uint32_t d) {
        return partials != nullptr && c->one_pass_chunks &&
               n_rows / PART_CHUNK <= ((uint64_t)c->one_pass_chunks << std::min(d, 40u));
    };
    check(launch_grow_prep(G, d_root, d_root ? nullptr : c->red_i64, c->n_red_blocks, 0,
                           GB.level[0], c->d_lvl_split, GB.tree, GB.st,
                           clear_root ? c->hist : nullptr, 2 * c->hist_width, c->stream),
          "tree root");
    enqueue_eval(c, E0, sp);
    account_hist(c, n_rows, 1);

    uint8_t *pk_base = reinterpret_cast<uint8_t *>(c->d_packets);
    const FusedArgmaxDev A_fused{c->d_cands, c->d_sfeats, c->d_lvl_split, c->d_cat_scratch};
    for (uint32_t d = 0; d < D; d++) {
        const FusedArgmaxDev A = fuse_at(d) ? A_fused : FusedArgmaxDev{};
        const uint32_t nb = lvl_bound(d);
        uint64_t *pk_cats =
            reinterpret_cast<uint64_t *>(pk_base + al256(sizeof(SplitPacketDev) * nb));
        const bool one_pass = one_pass_at(d) && !(walk && d + 1 == D);
        G.part_cur = one_pass ? c->d_cursors : nullptr;
        check(launch_grow_decide(G, d, c->d_packets, pk_cats, GB.level[d & 1], GB.tree,
                                 GB.tree_cats, d_mono, GB.cols, GB.reqs, GB.pairs, GB.triples,
                                 GB.leaves, GB.leaf_vals, GB.st, A, c->stream),
              "tree level decision");
        if (walk && d + 1 == D) break;  // the last level's children are found by the walk
        // Level d's rows are in arena d % 2; its children go to the other.
        uint32_t *arena_in = (d & 1) ? c->tmp : (ident && d == 0 ? nullptr : c->rows);
        uint32_t *arena_out = (d & 1) ? c->rows : c->tmp;
        if (arena_out == c->rows) c->rows_identity = false;
        const GrowDevOut out{GB.st, GB.level[(d + 1) & 1], GB.tree, GB.leaves, GB.leaf_vals,
                             (d + 1) & 1u};
        if (one_pass) {
            check(launch_partition_split(GB.reqs, &GB.st->n_split, n_rows / PART_CHUNK + nb + 1,
                                         arena_in, arena_out, c->d_cursors, c->d_totals, pk_cats,
                                         GB.pairs, rule, c->d_lvl_hist, c->d_lvl_split,
                                         c->d_lvl_out, c->d_lvl_out + 4 * MAX_NODES,
                                         c->d_lvl_rows, out, c->stream),
                  "partition and level plan");
        } else {
            // Without partials the scatter clears the next level's
            // accumulated slots of several chunks (none after the last
            // level); with them the histogram launch clears what it needs.
            ZeroNodesDev Z{};
            if (d + 1 < D && !partials)
                Z = {c->hist, c->hist_width, c->d_lvl_hist, &GB.st->n_eval,
                     (c->has_global || !c->streamed.empty()) ? 1u : 0u, 0u};
            check(launch_partition_level(GB.reqs, &GB.st->n_split, n_rows / PART_CHUNK + nb + 1,
                                         arena_in, arena_out, c->flags, c->d_counts, c->d_excl,
                                         c->d_totals, pk_cats, GB.pairs, rule, c->d_lvl_hist,
                                         c->d_lvl_split, c->d_lvl_out, c->d_lvl_out + 4 * MAX_NODES,
                                         c->d_lvl_rows, out, Z, c->stream),
                  "partition and level plan");
        }
        if (d + 1 == D) break;
        EvalPlan E;
        E.hn = c->d_lvl_hist;
        E.n_hn = nb;
        E.dev_n_hn = &GB.st->n_eval;
        E.grid_chunks = level_grid(nb);
        E.partials = partials;
        E.max_groups = E.grid_chunks / REDUCE_GROUP + nb + 1;
        E.dev_chunk_rows = c->d_lvl_rows;
        E.triples = GB.triples;
        E.n_tri = nb;
        E.dev_n_tri = &GB.st->n_eval;
        E.sn = c->d_lvl_split;
        E.n_nodes = lvl_bound(d + 1);
        E.dev_n_nodes = &GB.st->n_level;
        E.download = false;
        E.fused_argmax = fuse_at(d + 1);
        E.rows = arena_out;
        E.cleared = true;
        E.pairs = true;
        // These children are parents of the next evaluation only if there is one.
        E.write_children = d + 2 < D;
        enqueue_eval(c, E, sp);
    }
    uint64_t leaf_bound = (uint64_t)1 << D;
    if (gp->max_leaves) leaf_bound = std::min<uint64_t>(leaf_bound, gp->max_leaves);
    const int idb = c->objective >= 0 ? (leaf_bound <= 256 ? 1 : 2) : 0;
    // Deferred leaves: ids only; fbh_apply_leaf_values adds the values.
    const bool defer = (gp->flags & FBH_GROW_DEFER_LEAVES) != 0;
    c->q_forget((int)c->out_k);  // this output's margins change
    if (walk) {
        check(launch_tree_leaves(c->bundles[0].data, c->bundles[0].pitch, c->n_rows, GB.tree,
                                 GB.tree_cats, GB.feat_off, GB.st, c->leaf_ids, idb,
                                 defer ? nullptr : c->cur_margin(), c->delta, GB.leaf_vals, c->stream),
              "leaf walk");
    } else {
        check(launch_leaf_plan(GB.leaves, GB.st, c->stream), "leaf plan");
        check(launch_assign_leaves(GB.leaves, 0,
                                   (uint32_t)(n_rows / PART_CHUNK + leaf_bound + 1), c->rows,
                                   c->tmp, c->delta, c->leaf_ids, idb, &GB.st->n_leaves,
                                   c->stream),
              "leaf assignment");
        if (idb && !defer)
            check(launch_apply_leaves(c->leaf_ids, idb, GB.leaf_vals, c->n_rows, c->cur_margin(),
                                      c->stream),
                  "margin update");
    }
    c->leaf_id_bytes = idb;
    c->ids_fresh = idb != 0;
    c->leaves_deferred = defer;

    // Written into the next result slot by a kernel in the stream (no copy
    // engine); collected in order.
    const int k = (int)(GB.next_slot++ & 1);
    const size_t o_tree = al256(sizeof(GrowState));
    const size_t o_cats = o_tree + al256(sizeof(TreeNodeDev) * GB.tree_cap);
    const size_t o_vals = o_cats + al256(8 * GB.cat_cap);
    check(launch_tree_out(GB.st, GB.tree, (uint32_t)GB.tree_cap,
                          c->cat_words_per_node ? GB.tree_cats : nullptr, (uint32_t)GB.cat_cap,
                          GB.leaf_vals, (uint32_t)GB.leaf_cap, GB.out_dev[k], o_tree, o_cats,
                          o_vals, c->stream),
          "tree download");
    check(hipEventRecord(GB.done[k], c->stream), "event");
    GB.pending.push_back({k, c->cat_words_per_node});
}

// Waits for the oldest enqueued tree and copies it out.
void grow_collect(fbh_ctx *c, fbh_tree_node *nodes, uint32_t node_capacity, uint32_t *n_nodes,
                  uint64_t *cat_words, uint32_t cat_capacity, float *leaf_values,
                  uint32_t leaf_capacity, uint32_t *n_leaves) {
    if (!c || !nodes || !n_nodes || !leaf_values || !n_leaves) throw InputError("null argument");
    auto &GB = c->grow;
    if (GB.pending.empty()) throw InputError("no grown tree to collect");
    const auto job = GB.pending.front();
    GB.pending.pop_front();
    check(hipSetDevice(c->device), "hipSetDevice");
    check(hipEventSynchronize(GB.done[job.slot]), "tree download");
    if (c->timing) c->collect_timing();
    const uint8_t *po = static_cast<const uint8_t *>(GB.out[job.slot].p);
    const size_t o_tree = al256(sizeof(GrowState));
    const size_t o_cats = o_tree + al256(sizeof(TreeNodeDev) * GB.tree_cap);
    const size_t o_vals = o_cats + al256(8 * GB.cat_cap);
    GrowState st;
    std::memcpy(&st, po, sizeof(st));
    check_device_scales(st.scales, c->n_rows);
    if (st.error & 1u) throw RuntimeError("histogram slots exhausted; raise the slot budget");
    if (st.error & 4u) throw RuntimeError("partition cursors out of range");
    account_hist(c, st.hist_rows, st.hist_nodes);
    if (st.covered != c->n_rows)
        throw RuntimeError("leaves cover " + std::to_string(st.covered) + " of " +
                           std::to_string(c->n_rows) + " rows");
    if (st.tree_size > node_capacity || st.n_leaves > leaf_capacity ||
        (job.cat_words && st.tree_cat_words > cat_capacity))
        throw InputError("output capacity too small for the grown tree");
    static_assert(sizeof(TreeNodeDev) == sizeof(fbh_tree_node), "tree node layout");
    std::memcpy(nodes, po + o_tree, sizeof(fbh_tree_node) * st.tree_size);
    // Split nodes carry their value as a leaf from the decision kernel; a
    // leaf's is its value.
    for (uint32_t i = 0; i < st.tree_size; i++) {
        if (nodes[i].flags & 1u) nodes[i].value_as_leaf = nodes[i].leaf_value;
        else nodes[i].leaf_pos = 0xFFFFFFFFu;
    }
    if (job.cat_words && cat_words) std::memcpy(cat_words, po + o_cats, 8 * (size_t)st.tree_cat_words);
    std::memcpy(leaf_values, po + o_vals, 4 * (size_t)st.n_leaves);
    *n_nodes = st.tree_size;
    *n_leaves = st.n_leaves;
}

}  // namespace

extern "C" {

int fbh_grow_depthwise(fbh_ctx *c, const fbh_grow_params *gp, const fbh_split_params *sp,
                       const int64_t root_sum[2], fbh_tree_node *nodes, uint32_t node_capacity,
                       uint32_t *n_nodes, uint64_t *cat_words, uint32_t cat_capacity,
                       float *leaf_values, uint32_t leaf_capacity, uint32_t *n_leaves) {
    return guard([&] {
        if (c && !c->grow.pending.empty())
            throw InputError("grown trees are waiting; collect them with fbh_grow_collect");
        grow_enqueue(c, gp, sp, root_sum);
        grow_collect(c, nodes, node_capacity, n_nodes, cat_words, cat_capacity, leaf_values,
                     leaf_capacity, n_leaves);
    });
}

int fbh_grow_depthwise_async(fbh_ctx *c, const fbh_grow_params *gp, const fbh_split_params *sp,
                             const int64_t root_sum[2]) {
    return guard([&] { grow_enqueue(c, gp, sp, root_sum); });
}

int fbh_grow_collect(fbh_ctx *c, fbh_tree_node *nodes, uint32_t node_capacity, uint32_t *n_nodes,
                     uint64_t *cat_words, uint32_t cat_capacity, float *leaf_values,
                     uint32_t leaf_capacity, uint32_t *n_leaves) {
    return guard([&] {
        grow_collect(c, nodes, node_capacity, n_nodes, cat_words, cat_capacity, leaf_values,
                     leaf_capacity, n_leaves);
    });
}

int fbh_apply_leaf_values(fbh_ctx *c, const float *values, uint32_t n) {
    return guard([&] {
        if (!c || (n && !values)) throw InputError("null argument");
        if (!c->leaves_deferred)
            throw InputError("the last grown tree's leaf values are already applied "
                             "(grow it with FBH_GROW_DEFER_LEAVES)");
        if (!c->grow.pending.empty())
            throw InputError("collect the grown tree (fbh_grow_collect) before applying its leaves");
        const uint32_t cap = c->leaf_id_bytes == 1 ? 256u : MAX_NODES;
        if (n == 0 || n > cap) throw InputError("leaf value count out of range");
        check(hipSetDevice(c->device), "hipSetDevice");
        if (c->leaves_pending) {
            check(hipEventSynchronize(c->leaves_done), "leaf table reuse");
            c->leaves_pending = false;
        }
        // Every id of the tree indexes the table: pad it to the id range.
        float *pv = static_cast<float *>(c->pin_leaves.p);
        std::memcpy(pv, values, 4 * (size_t)n);
        for (uint32_t i = n; i < cap; i++) pv[i] = 0.0f;
        const size_t bytes = 4 * (size_t)cap;
        float *d_vals = reinterpret_cast<float *>(c->d_leaves);
        check(hipMemcpyAsync(d_vals, pv, bytes, hipMemcpyHostToDevice, c->stream), "leaf values");
        check(hipEventRecord(c->leaves_done, c->stream), "event");
        c->leaves_pending = true;
        c->q_forget((int)c->out_k);
        check(launch_apply_leaves(c->leaf_ids, c->leaf_id_bytes, d_vals, c->n_rows, c->cur_margin(),
                                  c->stream),
              "margin update");
        c->leaves_deferred = false;
    });
}

int fbh_assign_leaves(fbh_ctx *c, const fbh_span *spans, const float *values, uint32_t n) {
    return guard([&] {
        if (!c || (n && (!spans || !values))) throw InputError("null argument");
        ensure_tree(c);
        if (n == 0) return;
        if (n > MAX_NODES) throw InputError("too many leaves");
        check(hipSetDevice(c->device), "hipSetDevice");
        c->ensure_rows();
        if (c->leaves_pending) {
            check(hipEventSynchronize(c->leaves_done), "leaf table reuse");
            c->leaves_pending = false;
        }
        LeafDev *ld = static_cast<LeafDev *>(c->pin_leaves.p);
        uint32_t m = 0, chunks = 0;
        for (uint32_t i = 0; i < n; i++) {
            if ((uint64_t)spans[i].offset + spans[i].len > c->n_rows)
                throw InputError("row span out of range");
            if (spans[i].len == 0) continue;
            ld[m].row_off = spans[i].offset;
            ld[m].row_len = spans[i].len;
            ld[m].chunk_begin = chunks;
            ld[m].value = values[i];
            ld[m].id = i;
            ld[m].arena = 0;
            chunks += div_up(spans[i].len, PART_CHUNK);
            m++;
        }
        if (m == 0) return;
        const int idb = c->objective >= 0 ? (n <= 256 ? 1 : 2) : 0;
        // Leaf values by position follow the leaf table: one copy.
        float *pv = reinterpret_cast<float *>(ld + m);
        if (idb) std::memcpy(pv, values, 4 * (size_t)n);
        check(hipMemcpyAsync(c->d_leaves, ld, sizeof(LeafDev) * m + (idb ? 4 * (size_t)n : 0),
                             hipMemcpyHostToDevice, c->stream),
              "leaf table");
        const float *d_vals = reinterpret_cast<const float *>(c->d_leaves + m);
        check(hipEventRecord(c->leaves_done, c->stream), "event");
        c->leaves_pending = true;
        check(launch_assign_leaves(c->d_leaves, m, chunks, c->rows, c->rows, c->delta,
                                   c->leaf_ids, idb, nullptr, c->stream),
              "leaf assignment");
        c->q_forget((int)c->out_k);
        if (idb)
            check(launch_apply_leaves(c->leaf_ids, idb, d_vals, c->n_rows, c->cur_margin(), c->stream),
                  "margin update");
        c->leaf_id_bytes = idb;
        c->ids_fresh = idb != 0;
    });
}

int fbh_download_delta(fbh_ctx *c, float *out) {
    return guard([&] {
        if (!c || !out) throw InputError("null argument");
        if (c->objective >= 0)
            throw InputError("this context keeps the margins (fbh_set_objective); use "
                             "fbh_download_margin");
        check(hipSetDevice(c->device), "hipSetDevice");
        check(hipMemcpyAsync(out, c->delta, c->n_rows * 4, hipMemcpyDeviceToHost, c->stream),
              "delta download");
        c->sync();
    });
}

int fbh_host_alloc(size_t bytes, void **out) {
    return guard([&] {
        if (!out) throw InputError("null argument");
        *out = nullptr;
        check(hipHostMalloc(out, std::max<size_t>(bytes, 64), hipHostMallocDefault),
              "pinned host allocation");
    });
}

int fbh_host_free(void *p) {
    return guard([&] {
        if (p) check(hipHostFree(p), "pinned host free");
    });
}

int fbh_download_rows(fbh_ctx *c, uint32_t *out) {
    return guard([&] {
        if (!c || !out) throw InputError("null argument");
        check(hipSetDevice(c->device), "hipSetDevice");
        c->ensure_rows();
        check(hipMemcpyAsync(out, c->rows, c->n_rows * 4, hipMemcpyDeviceToHost, c->stream),
              "row download");
        c->sync();
    });
}

int fbh_set_timing(fbh_ctx *c, int enabled) {
    return guard([&] {
        if (!c) throw InputError("null argument");
        c->timing = enabled != 0;
    });
}

int fbh_hist_timing(fbh_ctx *c, double *ms, uint64_t *launches, uint64_t *bytes, int reset) {
    return guard([&] {
        if (!c) throw InputError("null argument");
        c->collect_timing();  // launches still running are counted by a later call
        if (ms) *ms = c->hist_ms;
        if (launches) *launches = c->hist_launches;
        if (bytes) *bytes = c->hist_bytes;
        if (reset) {
            c->hist_ms = 0.0;
            c->hist_launches = 0;
            c->hist_bytes = 0;
        }
    });
}

// ------------------------------------------------------------- standalone
int fbh_sigmoid_host(const float *in, uint64_t n, float *out) {
    return guard([&] {
        if ((!in || !out) && n) throw InputError("null argument");
        for (uint64_t i = 0; i < n; i++) out[i] = fb_sigmoid(in[i]);
    });
}

int fbh_sigmoid_device(int device, const float *in, uint64_t n, float *out) {
    return guard([&] {
        if ((!in || !out) && n) throw InputError("null argument");
        if (n == 0) return;
        check(hipSetDevice(device), "hipSetDevice");
        float *d = nullptr;
        check(hipMalloc(&d, 8 * n), "device allocation");
        std::unique_ptr<float, hipError_t (*)(void *)> own(d, hipFree);
        check(hipMemcpy(d, in, 4 * n, hipMemcpyHostToDevice), "input upload");
        check(launch_sigmoid(d, n, d + n, nullptr), "sigmoid");
        check(hipMemcpy(out, d + n, 4 * n, hipMemcpyDeviceToHost), "output download");
    });
}

static void function_checksum(int device, uint64_t begin, uint64_t end, uint64_t *out,
                              bool tanh) {
    if (!out) throw InputError("null argument");
    if (end > (1ull << 32) || begin > end) throw InputError("range must lie in [0, 2^32]");
    check(hipSetDevice(device), "hipSetDevice");
    unsigned long long *d = nullptr;
    check(hipMalloc(&d, 8), "device allocation");
    std::unique_ptr<unsigned long long, hipError_t (*)(void *)> own(d, hipFree);
    const unsigned long long zero = 0;
    check(hipMemcpy(d, &zero, 8, hipMemcpyHostToDevice), "clear");
    check(launch_sigmoid_checksum(begin, end, d, nullptr, tanh), "checksum");
    unsigned long long v = 0;
    check(hipMemcpy(&v, d, 8, hipMemcpyDeviceToHost), "checksum download");
    *out = v;
}

int fbh_tanh_checksum(int device, uint64_t begin, uint64_t end, uint64_t *out) {
    return guard([&] { function_checksum(device, begin, end, out, true); });
}

int fbh_sigmoid_checksum(int device, uint64_t begin, uint64_t end, uint64_t *out) {
    return guard([&] { function_checksum(device, begin, end, out, false); });
}

int fbh_build_histogram(int device, const void *bins, uint32_t width, uint64_t n_rows,
                        uint32_t n_feats, const uint32_t *offsets, const int64_t *gpair2n,
                        const uint32_t *rows, uint64_t n_sel, int64_t *out) {
    return guard([&] {
        if (!bins || !offsets || !gpair2n || !out) throw InputError("null argument");
        if (width != 1 && width != 2) throw InputError("width must be 1 or 2");
        std::vector<uint8_t> wv(n_feats, (uint8_t)width);
        std::vector<uint32_t> nb(n_feats);
        for (uint32_t f = 0; f < n_feats; f++) {
            if (offsets[f + 1] < offsets[f]) throw InputError("offsets must be non-decreasing");
            nb[f] = offsets[f + 1] - offsets[f];
            if (nb[f] == 0) throw InputError("every feature needs at least one bin");
        }
        fbh_shape sh{n_feats, wv.data(), nb.data(), nullptr};
        fbh_config cf{};
        cf.hist_slots = 1;
        fbh_ctx *c = nullptr;
        int rc = fbh_ctx_create(device, n_rows, &sh, &cf, &c);
        if (rc) throw RuntimeError(g_err);
        std::unique_ptr<fbh_ctx> own(c);
        std::vector<uint32_t> ids(n_feats);
        for (uint32_t f = 0; f < n_feats; f++) ids[f] = f;
        if (fbh_upload_block(c, ids.data(), n_feats, width, bins)) throw RuntimeError(g_err);
        const double one[2] = {1.0, 1.0};
        if (fbh_upload_gpair_fixed(c, gpair2n, one)) throw RuntimeError(g_err);
        fbh_span root;
        if (fbh_begin_tree(c, nullptr, 0, nullptr, 0, &root)) throw RuntimeError(g_err);
        uint64_t n_use = rows ? n_sel : n_rows;
        if (rows) {
            for (uint64_t i = 0; i < n_sel; i++)
                if (rows[i] >= n_rows) throw InputError("row index out of range");
            if (n_sel > n_rows) throw InputError("more selected rows than rows");
            check(hipMemcpyAsync(c->rows, rows, 4 * n_sel, hipMemcpyHostToDevice, c->stream),
                  "row upload");
        }
        fbh_node nd{};
        nd.rows = {0, (uint32_t)n_use};
        nd.slot = 0;
        nd.subtract_parent = -1;
        nd.subtract_sibling = -1;
        nd.lower = -3.4028234663852886e38f;
        nd.upper = 3.4028234663852886e38f;
        fbh_split_params sp{};
        sp.lambda_ = 1.0f;
        sp.max_cat_to_onehot = 4;
        sp.max_cat_threshold = 64;
        fbh_split pk;
        if (fbh_eval_nodes(c, &nd, 1, &sp, nullptr, &pk, nullptr, 0)) throw RuntimeError(g_err);
        if (fbh_download_histogram(c, 0, out, nullptr)) throw RuntimeError(g_err);
    });
}

int fbh_partition_rows(int device, const void *col, uint32_t width, uint64_t n_rows,
                       const uint32_t *rows, uint64_t n, uint32_t split_bin, uint32_t missing_left,
                       const uint64_t *cat_words, uint32_t n_cat_words, uint32_t *out,
                       uint64_t *n_left) {
    return guard([&] {
        if (!col || !rows || !out || !n_left) throw InputError("null argument");
        if (width != 1 && width != 2) throw InputError("width must be 1 or 2");
        if (n > n_rows) throw InputError("more rows than the column holds");
        for (uint64_t i = 0; i < n; i++)
            if (rows[i] >= n_rows) throw InputError("row index out of range");
        uint8_t w8 = (uint8_t)width;
        // Only the bin width matters to a partition; a categorical column
        // needs category-set capacity for n_cat_words words.
        uint32_t nb = 1;
        uint8_t catf = n_cat_words ? 1 : 0;
        if (catf) {
            if ((uint64_t)n_cat_words * 64 > MAX_DEVICE_CATS)
                throw InputError("category sets wider than " + std::to_string(MAX_DEVICE_CATS) +
                                 " codes are not supported on the device");
            nb = std::min<uint32_t>(n_cat_words * 64, width == 1 ? 254u : MAX_DEVICE_CATS);
        }
        fbh_shape sh{1, &w8, &nb, &catf};
        fbh_config cf{};
        cf.hist_slots = 1;
        fbh_ctx *c = nullptr;
        if (fbh_ctx_create(device, n_rows, &sh, &cf, &c)) throw RuntimeError(g_err);
        std::unique_ptr<fbh_ctx> own(c);
        const uint32_t f0 = 0;
        if (fbh_upload_block(c, &f0, 1, width, col)) throw RuntimeError(g_err);
        fbh_span root;
        if (fbh_begin_tree(c, nullptr, 0, nullptr, 0, &root)) throw RuntimeError(g_err);
        check(hipMemcpyAsync(c->rows, rows, 4 * n, hipMemcpyHostToDevice, c->stream), "row upload");
        fbh_part_req r{};
        r.rows = {0, (uint32_t)n};
        r.feat = 0;
        r.bin = split_bin;
        r.missing_left = missing_left;
        r.cat_offset = 0;
        r.n_cat_words = n_cat_words;
        fbh_span ch[2];
        if (fbh_partition(c, &r, 1, cat_words, n_cat_words, ch)) throw RuntimeError(g_err);
        check(hipMemcpyAsync(out, c->rows, 4 * n, hipMemcpyDeviceToHost, c->stream), "download");
        c->sync();
        *n_left = ch[0].len;
    });
}

}  // extern "C"
