// fbt_train.cpp -- the round driver of the device path.
//
// Restates train_with_backend (src/training/mod.rs:1299-2376) for the
// single-output logistic and squared-error objectives, gpu_math "exact" or
// "fast".
// The device keeps labels, weights and margins; squared-error gradients are
// computed there. For logistic, every round downloads the previous tree's
// per-row leaf id (one byte at depth <= 8), the host applies the leaf value
// to its margins and computes the sigmoid with its libm (so exp() rounds like
// the CPU engine), in chunks overlapped with the copies, and uploads it; the
// device forms the f32 gradient pairs with the host's operations and
// quantises them to i64 fixed point. Trees are grown depthwise
// (build_tree, src/training/mod.rs:3357-4565) or loss-guided
// (src/training/lossguide.rs:494-700); histograms, split scans, partitions
// and leaf scatters all run through the fbh_* backend.

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <limits>
#include <map>
#include <memory>
#include <mutex>
#include <queue>
#include <thread>

#include "fbhip.h"
#include "fbt_internal.h"

namespace fbt {
namespace {

using Clock = std::chrono::steady_clock;

std::string backend_error() {
    char buf[1024];
    fbh_last_error(buf, sizeof(buf));
    return buf;
}

void call(int rc) {
    if (rc == FBH_INPUT_ERROR) throw InputError(backend_error());
    if (rc != FBH_OK) throw RuntimeError(backend_error());
}

// A fixed pool of host threads for the per-row passes.
class Pool {
  public:
    explicit Pool(unsigned n) : n_(std::max(1u, n)) {
        for (unsigned t = 1; t < n_; t++) workers_.emplace_back([this, t] { loop(t); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(m_);
            stop_ = true;
            gen_++;
        }
        cv_.notify_all();
        for (auto &w : workers_) w.join();
    }
    unsigned size() const { return n_; }
    // Runs f(t) on every thread t in [0, n) and waits.
    void run(const std::function<void(unsigned)> &f) {
        if (n_ == 1) {
            f(0);
            return;
        }
        {
            std::lock_guard<std::mutex> g(m_);
            job_ = &f;
            pending_ = n_ - 1;
            gen_++;
        }
        cv_.notify_all();
        f(0);
        std::unique_lock<std::mutex> lk(m_);
        done_.wait(lk, [this] { return pending_ == 0; });
        job_ = nullptr;
    }

  private:
    void loop(unsigned t) {
        uint64_t seen = 0;
        for (;;) {
            const std::function<void(unsigned)> *job;
            {
                std::unique_lock<std::mutex> lk(m_);
                cv_.wait(lk, [&] { return gen_ != seen; });
                seen = gen_;
                if (stop_) return;
                job = job_;
            }
            (*job)(t);
            {
                std::lock_guard<std::mutex> g(m_);
                if (--pending_ == 0) done_.notify_one();
            }
        }
    }
    unsigned n_;
    std::vector<std::thread> workers_;
    std::mutex m_;
    std::condition_variable cv_, done_;
    const std::function<void(unsigned)> *job_ = nullptr;
    unsigned pending_ = 0;
    uint64_t gen_ = 0;
    bool stop_ = false;
};

// Host half of the exact logistic gradient, one chunk of rows at a time:
// pred += the previous tree's leaf value, then s = 1 / (1 + expf(-pred))
// (Objective::gradient, src/training/objective.rs:37-39, 499-530).
struct SigmoidJob {
    Pool *pool;
    float *pred;
    const std::vector<float> *values;  // leaf values of the previous tree
};

void sigmoid_chunk(void *user, uint64_t begin, uint64_t n, const void *ids, uint32_t id_bytes,
                   float *out) {
    SigmoidJob &J = *static_cast<SigmoidJob *>(user);
    const float *vals = J.values->data();
    const uint32_t n_vals = (uint32_t)J.values->size();
    std::atomic<bool> bad{false};
    J.pool->run([&](unsigned t) {
        const uint64_t lo = n * t / J.pool->size(), hi = n * (t + 1) / J.pool->size();
        float *pred = J.pred + begin;
        for (uint64_t i = lo; i < hi; i++) {
            if (ids) {
                const uint32_t id = id_bytes == 1 ? static_cast<const uint8_t *>(ids)[i]
                                                  : static_cast<const uint16_t *>(ids)[i];
                if (id >= n_vals) {
                    bad = true;
                    continue;
                }
                pred[i] += vals[id];
            }
            out[i] = 1.0f / (1.0f + std::exp(-pred[i]));
        }
    });
    // The callback cannot throw across the C ABI; a bad id poisons the
    // sigmoids so the device bounds check rejects the round.
    if (bad)
        for (uint64_t i = 0; i < n; i++) out[i] = std::numeric_limits<float>::quiet_NaN();
}

// True when the device sigmoid equals the host libm's 1 / (1 + expf(-x)) on
// probe inputs: a prime-stride sweep of all float bit patterns plus a dense
// sweep of the margins training meets. A host whose libm rounds differently
// keeps the host sigmoid, so exactness never rests on the device restatement.
bool device_sigmoid_matches_host(int device) {
    std::vector<float> in;
    in.reserve(300000);
    for (uint64_t u = 0; u < (1ull << 32); u += 65521) {
        uint32_t b = (uint32_t)u;
        float x;
        std::memcpy(&x, &b, 4);
        in.push_back(x);
    }
    for (float x = -104.0f; x <= 104.0f; x += 0.001953125f) in.push_back(x);
    std::vector<float> dev(in.size());
    if (fbh_sigmoid_device(device, in.data(), in.size(), dev.data()) != FBH_OK) return false;
    for (size_t i = 0; i < in.size(); i++) {
        const float h = 1.0f / (1.0f + std::exp(-in[i]));
        uint32_t a, b;
        std::memcpy(&a, &h, 4);
        std::memcpy(&b, &dev[i], 4);
        if (a != b && !(h != h && dev[i] != dev[i])) return false;
    }
    return true;
}

// ---------------------------------------------------------------- host math
// The leaf-value arithmetic of split.rs:113-218, in f64 then f32.
struct LeafMath {
    float lambda_, alpha, mds, lr;
    double inv_g, inv_h;
    void to_f64(const int64_t s[2], double &g, double &h) const {
        g = (double)s[0] * inv_g;
        h = (double)s[1] * inv_h;
    }
    float weight(double g, double h) const {  // xgb_weight
        if (h <= 0.0) return 0.0f;
        const double a = (double)alpha;
        const double t = g > a ? g - a : (g < -a ? g + a : 0.0);
        double dw = -t / (h + (double)lambda_);
        if (mds != 0.0f && std::fabs(dw) > (double)mds) dw = std::copysign((double)mds, dw);
        return (float)dw;
    }
    float hess(const int64_t s[2]) const {
        double g, h;
        to_f64(s, g, h);
        return (float)h;
    }
};

struct Bounds {  // NodeBounds (split.rs:120-160)
    float lo = -std::numeric_limits<float>::max();
    float hi = std::numeric_limits<float>::max();
    float apply(float w) const { return w < lo ? lo : (w > hi ? hi : w); }
};

// The column samplers (src/data/colsample.rs). SplitMix64 with unbiased
// bounded draws (rejection above the last whole multiple of n).
struct Mix64 {
    uint64_t state;
    uint64_t next() {
        state += 0x9E3779B97F4A7C15ull;
        uint64_t z = state;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    uint64_t below(uint64_t n) {
        const uint64_t zone = UINT64_MAX - (UINT64_MAX % n) - 1;
        uint64_t v;
        do v = next();
        while (v > zone);
        return v % n;
    }
};

// sampled_count: max(1, floor(rate * n)), at most n (colsample.rs:57-68).
size_t sample_size(size_t n, float rate) {
    if (n == 0) return 0;
    const double c = std::floor((double)rate * (double)n);
    const size_t take = (std::isfinite(c) && c >= 1.0) ? (size_t)c : 1;
    return std::max<size_t>(std::min(take, n), 1);
}

// The first `take` ids after a backward Fisher-Yates shuffle under `key`,
// ascending (sample_features / sample_subset, colsample.rs:74-116).
std::vector<uint32_t> shuffle_take(std::vector<uint32_t> ids, size_t take, uint64_t key) {
    if (take >= ids.size()) return ids;
    Mix64 rng{key};
    for (size_t i = ids.size() - 1; i >= 1; i--) std::swap(ids[i], ids[rng.below(i + 1)]);
    ids.resize(take);
    std::sort(ids.begin(), ids.end());
    return ids;
}

uint64_t tree_key(uint64_t seed, uint64_t round) {
    const uint64_t r = round * 0x9E3779B97F4A7C15ull;
    return seed ^ ((r << 17) | (r >> 47));
}

// Weighted draws without replacement (sample_weighted, colsample.rs:
// 146-172): every positive-weight id of `base` gets the exponential clock
// -ln(U) / w with U = (52 random bits + 1) / (2^52 + 1); the `take` earliest
// clocks win, ties to the lower id. rate >= 1 keeps the whole base.
std::vector<uint32_t> weighted_take(const std::vector<uint32_t> &base, size_t n, float rate,
                                    uint64_t key, const float *w) {
    if (rate >= 1.0f) return base;
    std::vector<uint32_t> pos;
    for (uint32_t id : base)
        if (w[id] > 0.0f) pos.push_back(id);
    const size_t take = std::min(sample_size(n, rate), pos.size());
    if (take == pos.size()) return pos;
    Mix64 rng{key};
    std::vector<std::pair<double, uint32_t>> clock(pos.size());
    for (size_t i = 0; i < pos.size(); i++) {
        const double u = (double)((rng.next() >> 12) + 1) / 4503599627370497.0;
        clock[i] = {-std::log(u) / (double)w[pos[i]], pos[i]};
    }
    std::nth_element(clock.begin(), clock.begin() + take, clock.end());
    std::vector<uint32_t> out(take);
    for (size_t i = 0; i < take; i++) out[i] = clock[i].second;
    std::sort(out.begin(), out.end());
    return out;
}

// colsample_bytree's set of a tree (sample_features_weighted, colsample.rs:
// 174-195); w is NULL for the uniform sampler.
std::vector<uint32_t> sample_columns(uint32_t nf, float rate, uint64_t seed, uint64_t round,
                                     const float *w = nullptr) {
    std::vector<uint32_t> ids(nf);
    for (uint32_t i = 0; i < nf; i++) ids[i] = i;
    if (w) return weighted_take(ids, nf, rate, tree_key(seed, round), w);
    return shuffle_take(std::move(ids), sample_size(nf, rate), tree_key(seed, round));
}

// validated_weights (colsample.rs:119-141): NULL when absent or all equal.
const float *checked_weights(const float *w, uint32_t nf) {
    if (!w) return nullptr;
    bool positive = false;
    for (uint32_t f = 0; f < nf; f++) {
        if (!(std::isfinite(w[f]) && w[f] >= 0.0f))
            throw InputError("feature_weights must be finite and nonnegative");
        positive = positive || w[f] > 0.0f;
    }
    if (!positive) throw InputError("feature_weights must contain at least one positive weight");
    for (uint32_t f = 1; f < nf; f++)
        if (w[f] != w[0]) return w;
    return nullptr;
}

float rate_or_one(float r) { return r == 0.0f ? 1.0f : r; }

// NestedSampler (colsample.rs:203-286): the level set of a depth from the
// tree's set, the node set of a tree node id from its level's set, keyed
// by (seed, tree, tag, depth or node) through three SplitMix64 steps.
struct NestedSets {
    float bylevel = 1.0f, bynode = 1.0f;
    const float *w = nullptr;
    uint64_t seed = 0, tree = 0;
    bool active() const { return bylevel < 1.0f || bynode < 1.0f; }
    uint64_t key(uint64_t tag, uint64_t idx) const {
        auto step = [](uint64_t x) { return Mix64{x}.next(); };
        return step(step(step(seed ^ (tag * 0xD6E8FEB86659FD93ull)) ^ tree) ^ idx);
    }
    std::vector<uint32_t> pick(const std::vector<uint32_t> &base, float rate, uint64_t k) const {
        if (w) return weighted_take(base, base.size(), rate, k, w);
        return shuffle_take(base, sample_size(base.size(), rate), k);
    }
    std::vector<uint32_t> level(const std::vector<uint32_t> &tree_set, uint32_t depth) const {
        return pick(tree_set, bylevel, key(1, depth));
    }
    std::vector<uint32_t> node(const std::vector<uint32_t> &level_set, uint64_t id) const {
        return bynode < 1.0f ? pick(level_set, bynode, key(2, id)) : level_set;
    }
};

uint64_t sample_threshold(float rate) {  // subsample::threshold_for
    if (rate >= 1.0f || !(rate > 0.0f)) return UINT64_MAX;
    return (uint64_t)((double)rate * (double)(1ull << 53));
}

// ---------------------------------------------------------------- growers
class Grower {
  public:
    Grower(fbh_ctx *ctx, const fbt_params &p, const Cuts &cuts, const std::vector<int8_t> &mono,
           uint32_t n_slots, const NestedSets &nested)
        : ctx_(ctx), p_(p), cuts_(cuts), mono_(mono), nested_(nested) {
        sp_.lambda_ = p.lambda_;
        sp_.gamma = p.gamma;
        sp_.min_child_weight = p.min_child_weight;
        sp_.alpha = p.alpha;
        sp_.max_delta_step = p.max_delta_step;
        sp_.max_cat_to_onehot = p.max_cat_to_onehot;
        sp_.max_cat_threshold = p.max_cat_threshold;
        for (uint32_t s = n_slots; s-- > 0;) free_.push_back(s);
        // Category words of one node: every categorical feature's set.
        uint32_t words = 0;
        for (uint32_t f = 0; f < cuts.n_features(); f++)
            if (cuts.is_cat(f)) words += (cuts.n_bins(f) + 63) / 64;
        cat_cap_ = words;
    }

    // The next tree's features (ascending: its bytree set, or every
    // feature) and the key of its nested sets (the tree index).
    void begin_tree(std::vector<uint32_t> features, uint64_t tree) {
        tree_feats_ = std::move(features);
        nested_.tree = tree;
        levels_.clear();
    }
    // colsample_bylevel / bynode restrict each node's split scan to its own
    // feature set (mod.rs:3575-3638): such trees grow level by level from
    // the host, which draws the sets of the nodes it numbers.
    bool masked() const { return nested_.active(); }

    void lm_scales(const double scales[2]) {
        lm_ = {p_.lambda_, p_.alpha, p_.max_delta_step, p_.learning_rate, 1.0 / scales[0],
               1.0 / scales[1]};
    }

    Tree grow(const double scales[2], const int64_t root_sum[2]) {
        lm_scales(scales);
        leaves_spans_.clear();
        leaves_values_.clear();
        if (device_growth()) {
            grow_async(root_sum);
            return collect();
        }
        Tree t;
        double g, h;
        lm_.to_f64(root_sum, g, h);
        t.push_leaf(lm_.weight(g, h) * p_.learning_rate, (float)h);
        fbh_span root;
        root.offset = 0;
        root.len = n_rows_;
        if (p_.grow_policy == 1) lossguide(t, root, root_sum);
        else depthwise(t, root, root_sum);
        uint64_t covered = 0;
        for (const auto &sp : leaves_spans_) covered += sp.len;
        if (covered != n_rows_)
            throw RuntimeError("leaf spans cover " + std::to_string(covered) + " of " +
                               std::to_string(n_rows_) + " rows");
        if (!leaves_spans_.empty())
            call(fbh_assign_leaves(ctx_, leaves_spans_.data(), leaves_values_.data(),
                                   (uint32_t)leaves_spans_.size()));
        return t;
    }
    // Leaf values of the last grown tree, by leaf position.
    const std::vector<float> &leaf_values() const { return leaves_values_; }
    uint32_t n_rows_ = 0;
    bool device_trees_ = false;  // depthwise trees grow whole on the device
    uint32_t device_trees = 0;   // trees grown that way

    // Lossguide whose leaf cap cannot bind (max_leaves 0, or at least
    // 2^max_depth): best-first expansion then splits every node with a split
    // above depth max_depth, the same set of splits as depthwise growth
    // without a cap; only the node numbering (expansion order) differs.
    bool lossguide_uncapped() const {
        return p_.grow_policy == 1 && p_.max_depth <= 14 &&
               (p_.max_leaves == 0 || p_.max_leaves >= (1u << p_.max_depth));
    }

    // Lossguide under a binding leaf cap, grown speculatively on the device:
    // every split down to max_depth, of which the host keeps the ones the
    // best-first expansion takes before the cap (the rows' leaf values wait
    // for that choice). Used while the whole tree is at most 8 times the
    // cap's leaves; a deeper tree is grown expansion by expansion instead.
    bool lossguide_capped() const {
        return p_.grow_policy == 1 && !lossguide_uncapped() && p_.max_leaves >= 2 &&
               p_.max_depth >= 1 && p_.max_depth <= 14 &&
               (1ull << p_.max_depth) <= 8ull * p_.max_leaves;
    }

    bool device_growth() const {
        return device_trees_ && !masked() &&
               (p_.grow_policy == 0 || lossguide_uncapped() || lossguide_capped()) &&
               p_.max_depth >= 1 && p_.max_depth <= 14 && p_.max_leaves != 1;
    }
    // The device leaves the leaf values to collect() (FBH_GROW_DEFER_LEAVES):
    // such a tree is collected before the next round's gradients.
    bool deferred_leaves() const { return device_growth() && lossguide_capped(); }

    // Enqueues a depthwise tree on the device (root_sum NULL: the one the
    // gradient call left there); collect() waits for it and rebuilds it.
    void grow_async(const int64_t *root_sum) {
        fbh_grow_params gp{p_.max_depth, p_.grow_policy == 1 ? 0u : p_.max_leaves,
                           p_.learning_rate, deferred_leaves() ? (uint32_t)FBH_GROW_DEFER_LEAVES : 0u};
        call(fbh_grow_depthwise_async(ctx_, &gp, &sp_, root_sum));
    }

    // The oldest enqueued device tree, rebuilt with Tree::split_leaf in
    // node-id order (the order the device numbered it), or, for lossguide,
    // in best-first order.
    Tree collect() {
        const uint32_t cap_nodes = (2u << p_.max_depth) - 1, cap_leaves = 1u << p_.max_depth;
        std::vector<fbh_tree_node> tn(cap_nodes);
        std::vector<uint64_t> cats((size_t)std::max<uint32_t>(1, cat_cap_) * cap_leaves);
        leaves_values_.assign(cap_leaves, 0.0f);
        uint32_t nn = 0, nl = 0;
        call(fbh_grow_collect(ctx_, tn.data(), cap_nodes, &nn, cats.data(), (uint32_t)cats.size(),
                              leaves_values_.data(), cap_leaves, &nl));
        leaves_values_.resize(nl);
        device_trees++;
        if (p_.grow_policy == 1) return best_first(tn.data(), nn, cats.data());
        Tree t;
        t.push_leaf(tn[0].leaf_value, tn[0].sum_hess);
        for (uint32_t id = 0; id < nn; id++) {
            const fbh_tree_node &a = tn[id];
            if (a.flags & 1u) continue;
            const fbh_tree_node &l = tn[a.left], &r = tn[a.right];
            const bool is_cat = (a.flags & 4u) != 0;
            const auto lr = t.split_leaf(id, a.feat, is_cat ? 0.0f : cond_of(a.feat, a.bin),
                                         (a.flags & 2u) != 0, a.gain, l.leaf_value, l.sum_hess,
                                         r.leaf_value, r.sum_hess);
            if (lr.first != (uint32_t)a.left || lr.second != (uint32_t)a.right)
                throw RuntimeError("device tree nodes out of order");
            if (is_cat) t.set_categories(id, cats.data() + a.cat_offset, a.n_cat_words);
        }
        if (t.nodes.size() != nn) throw RuntimeError("device tree node count mismatch");
        return t;
    }

    // The lossguide tree of a device-grown one: the expansion loop of
    // src/training/lossguide.rs:571-690 replayed over the device's splits,
    // popping the highest gain first and, on equal gains, the lower node id
    // (PendingSplit's order, lossguide.rs:46-52); each expansion numbers the
    // two children next, as Tree::split_leaf does, and the loop stops at the
    // leaf cap. Uncapped (lossguide_uncapped) every split is taken; under a
    // cap the device's deeper splits are dropped, and each of its leaves
    // takes the value of the kept leaf above it, which collect() adds to the
    // margins (fbh_apply_leaf_values).
    Tree best_first(const fbh_tree_node *tn, uint32_t nn, const uint64_t *cats) {
        struct Open {
            float gain;
            uint32_t id;   // node id in the lossguide tree
            uint32_t dev;  // node id in the device tree
        };
        auto less = [](const Open &a, const Open &b) {
            if (a.gain != b.gain) return a.gain < b.gain;
            return a.id > b.id;
        };
        std::priority_queue<Open, std::vector<Open>, decltype(less)> heap(less);
        const bool capped = deferred_leaves();
        std::vector<uint32_t> kept(nn, UINT32_MAX);  // device node -> lossguide node
        std::vector<uint32_t> parent(nn, UINT32_MAX);
        Tree t;
        t.push_leaf(tn[0].value_as_leaf, tn[0].sum_hess);
        kept[0] = 0;
        if (!(tn[0].flags & 1u)) heap.push({tn[0].gain, 0, 0});
        uint32_t expanded = 0, leaf_count = 1;
        while (!heap.empty() && (p_.max_leaves == 0 || leaf_count < p_.max_leaves)) {
            const Open o = heap.top();
            heap.pop();
            const fbh_tree_node &a = tn[o.dev];
            if ((uint32_t)a.left >= nn || (uint32_t)a.right >= nn)
                throw RuntimeError("device tree child out of range");
            const fbh_tree_node &l = tn[a.left], &r = tn[a.right];
            const bool is_cat = (a.flags & 4u) != 0;
            const auto lr = t.split_leaf(o.id, a.feat, is_cat ? 0.0f : cond_of(a.feat, a.bin),
                                         (a.flags & 2u) != 0, a.gain, l.value_as_leaf,
                                         l.sum_hess, r.value_as_leaf, r.sum_hess);
            if (is_cat) t.set_categories(o.id, cats + a.cat_offset, a.n_cat_words);
            kept[a.left] = lr.first;
            kept[a.right] = lr.second;
            leaf_count++;
            expanded++;
            // lossguide.rs:677-690: at the cap the children stay leaves
            if (p_.max_leaves != 0 && leaf_count == p_.max_leaves) break;
            if (!(l.flags & 1u)) heap.push({l.gain, lr.first, (uint32_t)a.left});
            if (!(r.flags & 1u)) heap.push({r.gain, lr.second, (uint32_t)a.right});
        }
        if (!capped) {
            if (t.nodes.size() != nn || 2 * expanded + 1 != nn)
                throw RuntimeError("device tree node count mismatch");
            return t;
        }
        // Leaf values by the device's leaf positions: each device leaf takes
        // the value of its nearest kept ancestor (itself when kept).
        for (uint32_t i = 0; i < nn; i++)
            if (!(tn[i].flags & 1u)) {
                parent[(uint32_t)tn[i].left] = i;
                parent[(uint32_t)tn[i].right] = i;
            }
        std::vector<float> table(leaves_values_.size(), 0.0f);
        std::vector<uint8_t> seen(table.size(), 0);
        for (uint32_t i = 0; i < nn; i++) {
            if (!(tn[i].flags & 1u) || tn[i].leaf_pos == UINT32_MAX) continue;
            if (tn[i].leaf_pos >= table.size()) throw RuntimeError("device leaf position out of range");
            if (leaves_values_[tn[i].leaf_pos] != tn[i].leaf_value)
                throw RuntimeError("device leaf positions disagree with the leaf values");
            uint32_t k = i;
            while (kept[k] == UINT32_MAX) {
                k = parent[k];
                if (k == UINT32_MAX) throw RuntimeError("device tree node without a kept ancestor");
            }
            const auto &node = t.nodes[kept[k]];
            if (!node.is_leaf) throw RuntimeError("kept ancestor of a device leaf is not a leaf");
            table[tn[i].leaf_pos] = node.leaf_value;
            seen[tn[i].leaf_pos] = 1;
        }
        for (uint8_t v : seen)
            if (!v) throw RuntimeError("a device leaf position has no leaf");
        if (!table.empty())
            call(fbh_apply_leaf_values(ctx_, table.data(), (uint32_t)table.size()));
        leaves_values_ = std::move(table);
        return t;
    }

  private:
    struct Pending {
        uint32_t node;
        fbh_span rows;
        int64_t sum[2];
        Bounds b;
        uint32_t slot;
        int32_t parent_slot;  // -1: accumulate
        int32_t sibling;      // index of the accumulated sibling in the batch
        uint32_t depth;
    };

    uint32_t take_slot() {
        if (free_.empty())
            throw RuntimeError("histogram slots exhausted; raise the slot budget");
        const uint32_t s = free_.back();
        free_.pop_back();
        return s;
    }
    void give_slot(uint32_t s) { free_.push_back(s); }

    void finish_leaf(const Tree &t, uint32_t node, fbh_span rows) {
        if (rows.len == 0) return;
        leaves_spans_.push_back(rows);
        leaves_values_.push_back(t.nodes[node].leaf_value);
    }

    // The level set of a depth, drawn once per tree.
    const std::vector<uint32_t> &level_set(uint32_t depth) {
        auto it = levels_.find(depth);
        if (it == levels_.end()) it = levels_.emplace(depth, nested_.level(tree_feats_, depth)).first;
        return it->second;
    }

    // enabled bytes of the given nodes (tree node ids at one depth) over the
    // tree's features, node after node; empty when nothing is masked.
    std::vector<uint8_t> masks(uint32_t depth, const std::vector<uint32_t> &ids) {
        std::vector<uint8_t> out;
        if (!masked()) return out;
        const size_t F = tree_feats_.size();
        out.assign(ids.size() * F, 0);
        const std::vector<uint32_t> &level = level_set(depth);
        for (size_t i = 0; i < ids.size(); i++) {
            const std::vector<uint32_t> set = nested_.node(level, ids[i]);
            size_t k = 0;
            for (size_t j = 0; j < F && k < set.size(); j++)
                if (tree_feats_[j] == set[k]) {
                    out[i * F + j] = 1;
                    k++;
                }
            if (k != set.size()) throw RuntimeError("a node's feature set is not in the tree's");
        }
        return out;
    }

    // Split scans of a batch of nodes; returns packets.
    std::vector<fbh_split> eval(const std::vector<Pending> &batch,
                                const std::vector<uint8_t> &enabled = {}) {
        std::vector<fbh_node> nodes(batch.size());
        for (size_t i = 0; i < batch.size(); i++) {
            const Pending &b = batch[i];
            fbh_node &n = nodes[i];
            n.rows = b.rows;
            n.sum[0] = b.sum[0];
            n.sum[1] = b.sum[1];
            n.lower = b.b.lo;
            n.upper = b.b.hi;
            n.slot = b.slot;
            n.subtract_parent = b.parent_slot;
            n.subtract_sibling = b.sibling;
            n.reserved = 0;
        }
        std::vector<fbh_split> out(batch.size());
        cat_words_.assign((size_t)std::max<uint32_t>(1, cat_cap_) * batch.size(), 0);
        call(fbh_eval_nodes(ctx_, nodes.data(), (uint32_t)nodes.size(), &sp_,
                            enabled.empty() ? nullptr : enabled.data(), out.data(),
                            cat_words_.data(), (uint32_t)cat_words_.size()));
        return out;
    }

    // split_threshold (tree.rs:991-1001): the cut below the split bin.
    float cond_of(uint32_t feat, uint32_t bin) const {
        const uint32_t nc = cuts_.n_cuts(feat);
        if (bin == 0) return -std::numeric_limits<float>::max();
        if (bin > nc) return std::numeric_limits<float>::max();
        return cuts_.values[cuts_.offsets[feat] + bin - 1];
    }

    // Tree::split_leaf with child_leaves (src/training/mod.rs:5069-5094).
    void apply(Tree &t, uint32_t node, const fbh_split &s, const uint64_t *cats, Bounds parent,
               uint32_t &l, uint32_t &r, Bounds &lb, Bounds &rb) {
        double g, h;
        lm_.to_f64(s.left, g, h);
        const float wl = parent.apply(lm_.weight(g, h));
        lm_.to_f64(s.right, g, h);
        const float wr = parent.apply(lm_.weight(g, h));
        const int8_t c = s.feat < mono_.size() ? mono_[s.feat] : 0;
        const float mid = (wl + wr) / 2.0f;
        lb = parent;
        rb = parent;
        if (c < 0) {
            lb.lo = mid;
            rb.hi = mid;
        } else if (c > 0) {
            lb.hi = mid;
            rb.lo = mid;
        }
        const float cond = s.is_cat ? 0.0f : cond_of(s.feat, s.bin);
        auto lr = t.split_leaf(node, s.feat, cond, s.missing_left != 0, s.gain,
                               wl * p_.learning_rate, lm_.hess(s.left), wr * p_.learning_rate,
                               lm_.hess(s.right));
        if (s.is_cat) t.set_categories(node, cats, s.n_cat_words);
        l = lr.first;
        r = lr.second;
    }

    fbh_part_req part_req(const Pending &nd, const fbh_split &s, uint32_t cat_off) {
        fbh_part_req q{};
        q.rows = nd.rows;
        q.feat = s.feat;
        q.bin = s.bin;
        q.missing_left = s.missing_left;
        q.cat_offset = cat_off;
        q.n_cat_words = s.is_cat ? s.n_cat_words : 0;
        return q;
    }

    // One fused backend step: partition the split nodes and, when the
    // children are evaluated, build and scan their histograms. pairs carries
    // each node's slot, a new slot for one child, the children's bounds and
    // sums; on return next[2k], next[2k+1] hold the children's rows and
    // slots and the packets are (left, right) per pair.
    std::vector<fbh_split> step(const std::vector<fbh_part_req> &reqs,
                                const std::vector<fbh_child_pair> &pairs,
                                const std::vector<uint64_t> &cats, std::vector<Pending> &next) {
        const size_t n = reqs.size();
        std::vector<fbh_span> children(2 * n);
        std::vector<uint32_t> left_slot(n);
        std::vector<fbh_split> packets(2 * n);
        cat_words_.assign((size_t)std::max<uint32_t>(1, cat_cap_) * 2 * n, 0);
        // the children's sets, (left, right) per pair (every pair of a step
        // is evaluated, and its children share one depth)
        std::vector<uint32_t> ids;
        for (const Pending &c : next) ids.push_back(c.node);
        const std::vector<uint8_t> en = masks(next.empty() ? 0 : next[0].depth, ids);
        call(fbh_partition_eval_masked(ctx_, reqs.data(), (uint32_t)n, cats.data(),
                                       (uint32_t)cats.size(), pairs.data(), &sp_,
                                       en.empty() ? nullptr : en.data(), children.data(),
                                       left_slot.data(), packets.data(), cat_words_.data(),
                                       (uint32_t)cat_words_.size()));
        for (size_t k = 0; k < n; k++) {
            next[2 * k].rows = children[2 * k];
            next[2 * k + 1].rows = children[2 * k + 1];
            next[2 * k].slot = left_slot[k];
            next[2 * k + 1].slot =
                left_slot[k] == pairs[k].parent_slot ? pairs[k].new_slot : pairs[k].parent_slot;
        }
        return packets;
    }

    fbh_child_pair pair_of(const Pending &nd, const fbh_split &s, const Bounds &lb,
                           const Bounds &rb, bool evaluate) {
        fbh_child_pair q{};
        q.parent_slot = nd.slot;
        q.new_slot = evaluate ? take_slot() : UINT32_MAX;
        q.evaluate = evaluate ? 1u : 0u;
        q.lower[0] = lb.lo;
        q.lower[1] = rb.lo;
        q.upper[0] = lb.hi;
        q.upper[1] = rb.hi;
        for (int k = 0; k < 2; k++) {
            q.left_sum[k] = s.left[k];
            q.right_sum[k] = s.right[k];
        }
        return q;
    }

    // Depthwise growth (build_tree, src/training/mod.rs:3357-4565): the root
    // is evaluated alone, then each level is one fused step (partition of the
    // split nodes, histograms and split scans of their children).
    void depthwise(Tree &t, fbh_span root_rows, const int64_t root_sum[2]) {
        std::vector<Pending> level(1);
        level[0] = {0, root_rows, {root_sum[0], root_sum[1]}, Bounds(), take_slot(), -1, -1, 0};
        uint32_t leaf_count = 1;
        if (p_.max_depth == 0 || (p_.max_leaves != 0 && leaf_count >= p_.max_leaves)) {
            finish_leaf(t, 0, root_rows);
            give_slot(level[0].slot);
            return;
        }
        std::vector<fbh_split> chosen = eval(level, masks(0, {0}));
        std::vector<uint64_t> cats = cat_words_;
        for (uint32_t depth = 0;; depth++) {
            if (p_.max_leaves != 0) {
                uint32_t remaining = p_.max_leaves > leaf_count ? p_.max_leaves - leaf_count : 0;
                for (auto &c : chosen)
                    if (c.found) {
                        if (remaining == 0) c.found = 0;
                        else remaining--;
                    }
            }
            // Nodes without a split become leaves and hand back their slots
            // before the children take new ones.
            std::vector<uint32_t> split_idx;
            for (size_t i = 0; i < level.size(); i++) {
                if (chosen[i].found) {
                    split_idx.push_back((uint32_t)i);
                    leaf_count++;
                } else {
                    finish_leaf(t, level[i].node, level[i].rows);
                    give_slot(level[i].slot);
                }
            }
            if (split_idx.empty()) return;
            const bool evaluated = depth + 1 < p_.max_depth &&
                                   !(p_.max_leaves != 0 && leaf_count >= p_.max_leaves);
            std::vector<fbh_part_req> reqs;
            std::vector<fbh_child_pair> pairs;
            std::vector<Pending> next;
            for (uint32_t i : split_idx) {
                const Pending &ln = level[i];
                uint32_t l, r;
                Bounds lb, rb;
                apply(t, ln.node, chosen[i], cats.data() + chosen[i].cat_offset, ln.b, l, r, lb,
                      rb);
                reqs.push_back(part_req(ln, chosen[i], chosen[i].cat_offset));
                pairs.push_back(pair_of(ln, chosen[i], lb, rb, evaluated));
                next.push_back(
                    {l, {}, {chosen[i].left[0], chosen[i].left[1]}, lb, 0, -1, -1, depth + 1});
                next.push_back(
                    {r, {}, {chosen[i].right[0], chosen[i].right[1]}, rb, 0, -1, -1, depth + 1});
            }
            if (!evaluated) {  // the children are leaves
                std::vector<fbh_span> children(2 * reqs.size());
                call(fbh_partition(ctx_, reqs.data(), (uint32_t)reqs.size(), cats.data(),
                                   (uint32_t)cats.size(), children.data()));
                for (size_t k = 0; k < reqs.size(); k++) {
                    finish_leaf(t, next[2 * k].node, children[2 * k]);
                    finish_leaf(t, next[2 * k + 1].node, children[2 * k + 1]);
                    give_slot(pairs[k].parent_slot);
                }
                return;
            }
            chosen = step(reqs, pairs, cats, next);
            cats = cat_words_;
            level = std::move(next);
        }
    }

    // Lossguide growth (src/training/lossguide.rs): best-first expansion from
    // a priority queue by gain (ties: the lower node id); each expansion is
    // one fused step.
    void lossguide(Tree &t, fbh_span root_rows, const int64_t root_sum[2]) {
        struct Cand {
            Pending leaf;
            fbh_split split;
            std::vector<uint64_t> cats;
        };
        auto less = [](const Cand &a, const Cand &b) {
            if (a.split.gain != b.split.gain) return a.split.gain < b.split.gain;
            return a.leaf.node > b.leaf.node;
        };
        std::priority_queue<Cand, std::vector<Cand>, decltype(less)> heap(less);
        // Candidates or leaves from evaluated nodes (packets in batch order).
        auto take = [&](const std::vector<Pending> &batch, const std::vector<fbh_split> &res,
                        const std::vector<uint64_t> &words) {
            for (size_t i = 0; i < batch.size(); i++) {
                if (res[i].found) {
                    Cand c{batch[i], res[i], {}};
                    if (res[i].is_cat)
                        c.cats.assign(words.begin() + res[i].cat_offset,
                                      words.begin() + res[i].cat_offset + res[i].n_cat_words);
                    c.leaf.parent_slot = -1;
                    c.leaf.sibling = -1;
                    heap.push(std::move(c));
                } else {
                    finish_leaf(t, batch[i].node, batch[i].rows);
                    give_slot(batch[i].slot);
                }
            }
        };
        Pending root{0, root_rows, {root_sum[0], root_sum[1]}, Bounds(), 0, -1, -1, 0};
        if (p_.max_depth == 0 || p_.max_leaves == 1) {
            finish_leaf(t, 0, root_rows);
        } else {
            root.slot = take_slot();
            const std::vector<Pending> batch{root};
            take(batch, eval(batch, masks(0, {0})), cat_words_);
        }
        uint32_t leaf_count = 1;
        while (p_.max_leaves == 0 || leaf_count < p_.max_leaves) {
            if (heap.empty()) break;
            Cand c = heap.top();
            heap.pop();
            uint32_t l, r;
            Bounds lb, rb;
            apply(t, c.leaf.node, c.split, c.cats.data(), c.leaf.b, l, r, lb, rb);
            leaf_count++;
            const uint32_t depth = c.leaf.depth + 1;
            const std::vector<fbh_part_req> reqs{part_req(c.leaf, c.split, 0)};
            std::vector<Pending> next{
                {l, {}, {c.split.left[0], c.split.left[1]}, lb, 0, -1, -1, depth},
                {r, {}, {c.split.right[0], c.split.right[1]}, rb, 0, -1, -1, depth}};
            if (depth == p_.max_depth || leaf_count == p_.max_leaves) {
                fbh_span ch[2];
                call(fbh_partition(ctx_, reqs.data(), 1, c.cats.data(), (uint32_t)c.cats.size(),
                                   ch));
                finish_leaf(t, l, ch[0]);
                finish_leaf(t, r, ch[1]);
                give_slot(c.leaf.slot);
                continue;
            }
            const std::vector<fbh_child_pair> pairs{pair_of(c.leaf, c.split, lb, rb, true)};
            const std::vector<fbh_split> res = step(reqs, pairs, c.cats, next);
            // lossguide.rs evaluate: the smaller child (left on ties) first.
            const bool left_small = !(next[0].rows.len > next[1].rows.len);
            if (left_small)
                take(next, res, cat_words_);
            else
                take({next[1], next[0]}, {res[1], res[0]}, cat_words_);
        }
        while (!heap.empty()) {
            finish_leaf(t, heap.top().leaf.node, heap.top().leaf.rows);
            give_slot(heap.top().leaf.slot);
            heap.pop();
        }
    }

    fbh_ctx *ctx_;
    const fbt_params &p_;
    const Cuts &cuts_;
    const std::vector<int8_t> &mono_;
    NestedSets nested_;
    std::vector<uint32_t> tree_feats_;
    std::map<uint32_t, std::vector<uint32_t>> levels_;
    fbh_split_params sp_{};
    LeafMath lm_{};
    std::vector<uint32_t> free_;
    std::vector<fbh_span> leaves_spans_;
    std::vector<float> leaves_values_;
    std::vector<uint64_t> cat_words_;
    uint32_t cat_cap_ = 0;
};

void validate(const fbt_params &p, uint64_t n, uint32_t nf, const float *y) {
    if (n == 0) throw InputError("training data must have at least one row");
    if (n > 0xFFFFFFFFull)
        throw InputError("training data has " + std::to_string(n) +
                         " rows, above the supported limit 4294967295");
    if (nf == 0) throw InputError("training data must have at least one feature");
    if (p.objective > 4)
        throw InputError("objective must be reg:squarederror, binary:logistic, multi:softprob, "
                         "multi:softmax or reg:quantileerror");
    const bool multi = p.objective == 2 || p.objective == 3;
    if (p.objective == 4) {
        // QuantileAlphas::new and Objective::validate_params
        // (src/types.rs:700-712, src/training/objective.rs:317-330).
        if (p.n_quantile_alpha == 0 || !p.quantile_alpha)
            throw InputError("reg:quantileerror requires quantile_alpha (one or more ascending "
                             "quantiles in [0, 1])");
        if (p.n_quantile_alpha > 64)
            throw InputError("quantile_alpha accepts at most 64 quantiles, got " +
                             std::to_string(p.n_quantile_alpha));
        for (uint32_t k = 0; k < p.n_quantile_alpha; k++) {
            const float a = p.quantile_alpha[k];
            if (!(a >= 0.0f && a <= 1.0f))
                throw InputError("quantile_alpha must be in [0, 1], got " + std::to_string(a));
            if (k && p.quantile_alpha[k - 1] > a)
                throw InputError("quantile_alpha must be in ascending order (as XGBoost requires)");
        }
    }
    if (multi && p.num_class < 2)
        throw InputError(std::string(p.objective == 2 ? "multi:softprob" : "multi:softmax") +
                         " requires num_class >= 2, got " + std::to_string(p.num_class));
    if (p.grow_policy > 1) throw InputError("grow_policy must be depthwise or lossguide");
    if (p.gpu_math > 1) throw InputError("gpu_math must be 0 (exact) or 1 (fast)");
    if (p.gpu_math == 1 && p.host_sigmoid)
        throw InputError("gpu_math=\"fast\" computes the sigmoid on the device; it cannot be "
                         "combined with a host sigmoid");
    if (p.max_bin < 1 || p.max_bin > 65535)
        throw InputError("max_bin must be in 1..=65535, got " + std::to_string(p.max_bin));
    if (p.max_depth > 14)
        throw InputError("max_depth must be in 0..=14, got " + std::to_string(p.max_depth) +
                         "; 0 means a root-only tree");
    auto nonneg = [](float v, const char *name) {
        if (!(std::isfinite(v) && v >= 0.0f))
            throw InputError(std::string(name) + " must be finite and non-negative");
    };
    nonneg(p.learning_rate, "learning_rate");
    nonneg(p.lambda_, "lambda");
    nonneg(p.gamma, "gamma");
    nonneg(p.min_child_weight, "min_child_weight");
    nonneg(p.alpha, "alpha");
    nonneg(p.max_delta_step, "max_delta_step");
    nonneg(p.scale_pos_weight, "scale_pos_weight");
    if (!(p.subsample > 0.0f && p.subsample <= 1.0f))
        throw InputError("subsample must be in (0, 1]");
    if (!(p.colsample_bytree > 0.0f && p.colsample_bytree <= 1.0f))
        throw InputError("colsample_bytree must be in (0, 1]");
    // src/training/mod.rs:1550-1565 (0 in the struct reads as 1).
    if (!(rate_or_one(p.colsample_bylevel) > 0.0f && rate_or_one(p.colsample_bylevel) <= 1.0f))
        throw InputError("colsample_bylevel must be in (0, 1]");
    if (!(rate_or_one(p.colsample_bynode) > 0.0f && rate_or_one(p.colsample_bynode) <= 1.0f))
        throw InputError("colsample_bynode must be in (0, 1]");
    checked_weights(p.feature_weights, nf);
    // validate_start_margins (src/training/mod.rs:1109-1130).
    if (p.base_margin) {
        const uint64_t k = multi ? p.num_class : p.objective == 4 ? p.n_quantile_alpha : 1;
        for (uint64_t i = 0; i < k * n; i++)
            if (!std::isfinite(p.base_margin[i]))
                throw InputError("training set: base_margin values must all be finite");
    }
    if (p.cols_per_block == 0) throw InputError("cols_per_block must be > 0");
    for (uint64_t i = 0; i < n; i++) {
        if (!std::isfinite(y[i])) throw InputError("labels must all be finite");
        if (p.objective == 1 && !(y[i] >= 0.0f && y[i] <= 1.0f))
            throw InputError("training set: binary:logistic labels must be in [0, 1]");
        // Objective::validate_labels (src/training/objective.rs:681-687).
        if (multi && !(y[i] >= 0.0f && y[i] < (float)p.num_class && y[i] == std::trunc(y[i])))
            throw InputError(std::string("training set: ") +
                             (p.objective == 2 ? "multi:softprob" : "multi:softmax") +
                             " labels must be integers in [0, num_class=" +
                             std::to_string(p.num_class) + ")");
    }
}

// quantile_intercepts (src/training/objective.rs:1039-1087), XGBoost's
// common::Quantile / WeightedQuantile: the labels stably sorted once in
// f32::total_cmp order; without weights the order statistic at
// alpha (n + 1), linearly interpolated in double from the f32 difference;
// with weights the first label whose f32 running weight reaches
// alpha * total.
std::vector<float> quantile_intercepts(const float *alphas, uint32_t k, const float *y,
                                       const float *w, uint64_t n) {
    if (n == 0) return std::vector<float>(k, 0.5f);
    auto key = [](float v) {
        int32_t b;
        std::memcpy(&b, &v, 4);
        return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
    };
    auto lt = [&](float a, float b) { return key(a) < key(b); };
    std::vector<float> out(k);
    if (!w) {
        // Only order statistics are read, and labels of equal keys are equal
        // bits, so selection gives the stable sort's values in O(n).
        std::vector<float> v(y, y + n);
        const double nf = (double)n;
        for (uint32_t j = 0; j < k; j++) {
            const double alpha = (double)alphas[j];
            if (alpha <= 1.0 / (nf + 1.0)) {
                out[j] = *std::min_element(v.begin(), v.end(), lt);
            } else if (alpha >= nf / (nf + 1.0)) {
                out[j] = *std::max_element(v.begin(), v.end(), lt);
            } else {
                const double x = alpha * (nf + 1.0);
                const double lo = std::floor(x) - 1.0;
                const double d = (x - 1.0) - lo;
                const uint64_t i = (uint64_t)lo;
                std::nth_element(v.begin(), v.begin() + i, v.end(), lt);
                const float v0 = v[i];
                const float v1 = *std::min_element(v.begin() + i + 1, v.end(), lt);
                out[j] = (float)((double)v0 + d * (double)(v1 - v0));
            }
        }
        return out;
    }
    std::vector<uint32_t> idx(n);
    for (uint64_t i = 0; i < n; i++) idx[i] = (uint32_t)i;
    std::stable_sort(idx.begin(), idx.end(), [&](uint32_t a, uint32_t b) { return lt(y[a], y[b]); });
    std::vector<float> cdf(n);
    cdf[0] = w[idx[0]];
    for (uint64_t i = 1; i < n; i++) cdf[i] = cdf[i - 1] + w[idx[i]];
    for (uint32_t j = 0; j < k; j++) {
        const float thresh = (float)((double)cdf[n - 1] * (double)alphas[j]);
        const uint64_t at =
            (uint64_t)(std::lower_bound(cdf.begin(), cdf.end(), thresh) - cdf.begin());
        out[j] = y[idx[std::min<uint64_t>(at, n - 1)]];
    }
    return out;
}

// Objective::initial_class_margins (src/training/objective.rs:1225-1248):
// the centred logs of the class frequencies, in the reference's f32/f64
// steps with the host libm.
std::vector<float> initial_class_margins(const float *y, const float *w, uint64_t n, uint32_t k) {
    std::vector<float> bins(k, 0.0f);
    for (uint64_t i = 0; i < n; i++) bins[(uint32_t)y[i]] += w ? w[i] : 1.0f;
    double sum_w = 0.0;
    if (!w) {
        sum_w = (double)n;
    } else {
        for (uint64_t i = 0; i < n; i++) sum_w += (double)w[i];
    }
    const float eps = 1e-6f;
    if (sum_w < (double)eps) return std::vector<float>(k, 0.0f);
    const double inv = 1.0 / sum_w;
    std::vector<float> logs(k);
    for (uint32_t c = 0; c < k; c++) logs[c] = std::log((float)((double)bins[c] * inv) + eps);
    const float nk = (float)k;
    float mean = 0.0f;
    for (float v : logs) mean = mean + v / nk;
    for (float &v : logs) v = v - mean;
    return logs;
}

fbt_stats g_stats{};
std::vector<double> g_round_wall, g_round_hist_ms;
std::vector<uint64_t> g_round_hist_bytes, g_round_hist_launches;

}  // namespace

fbt_stats last_stats() { return g_stats; }

uint32_t last_round_stats(double *wall, double *ms, uint64_t *bytes, uint32_t cap) {
    const uint32_t n = (uint32_t)g_round_wall.size();
    for (uint32_t i = 0; i < std::min(n, cap); i++) {
        if (wall) wall[i] = g_round_wall[i];
        if (ms) ms[i] = g_round_hist_ms[i];
        if (bytes) bytes[i] = g_round_hist_bytes[i];
    }
    return n;
}

uint32_t last_round_launches(uint64_t *launches, uint32_t cap) {
    const uint32_t n = (uint32_t)g_round_hist_launches.size();
    for (uint32_t i = 0; i < std::min(n, cap); i++)
        if (launches) launches[i] = g_round_hist_launches[i];
    return n;
}

// Cuts::full from the rows: which 256-bin numeric features hold no NaN.
// One pass over the row-major matrix, rows split among threads.
void mark_full_features(Cuts &c, const float *x, uint64_t n, uint32_t nf, unsigned threads) {
    std::vector<uint32_t> cand;
    for (uint32_t f = 0; f < nf; f++)
        if (!c.is_cat(f) && c.n_bins(f) == 256) cand.push_back(f);
    c.full.assign(nf, 0);
    if (cand.empty() || n == 0) return;
    const unsigned nt = std::max(1u, std::min<unsigned>(threads, (unsigned)std::min<uint64_t>(n, 64)));
    std::vector<std::vector<uint8_t>> nan_seen(nt, std::vector<uint8_t>(cand.size(), 0));
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < nt; t++)
        pool.emplace_back([&, t] {
            std::vector<uint8_t> &seen = nan_seen[t];
            const uint64_t lo = n * t / nt, hi = n * (t + 1) / nt;
            for (uint64_t r = lo; r < hi; r++) {
                const float *row = x + r * nf;
                for (size_t k = 0; k < cand.size(); k++) seen[k] |= row[cand[k]] != row[cand[k]];
            }
        });
    for (auto &th : pool) th.join();
    for (size_t k = 0; k < cand.size(); k++) {
        uint8_t any = 0;
        for (unsigned t = 0; t < nt; t++) any |= nan_seen[t][k];
        c.full[cand[k]] = any ? 0 : 1;
    }
}

Model train(const RowSource &src, uint64_t n, uint32_t nf, const float *y, const float *w,
            const uint8_t *cat, const int8_t *mono_in, uint32_t n_mono, const fbt_params &p,
            const Cuts *given) {
    const auto t_setup = Clock::now();
    // A reader's rows are held in host memory only where a host pass needs
    // the whole matrix (the host sketch of weighted rows, host binning).
    const float *x = src.x;
    std::vector<float> held;
    auto materialise = [&]() {
        if (x) return;
        held.resize(n * nf);
        src.each_chunk(n, nf, [&](uint64_t r0, uint64_t k, const float *rows) {
            std::memcpy(held.data() + r0 * nf, rows, 4 * k * nf);
        });
        x = held.data();
    };
    validate(p, n, nf, y);
    if (n_mono > nf) throw InputError("monotone_constraints has more entries than features");
    std::vector<int8_t> mono(nf, 0);
    for (uint32_t i = 0; i < n_mono; i++) {
        if (mono_in[i] < -1 || mono_in[i] > 1)
            throw InputError("monotone_constraints accepts only -1 / 0 / 1");
        mono[i] = mono_in[i];
    }
    if (w)
        for (uint64_t i = 0; i < n; i++)
            if (!(std::isfinite(w[i]) && w[i] >= 0.0f))
                throw InputError("sample weights must be finite and non-negative");
    if (!fbh_device_available(p.device))
        throw RuntimeError("device cuda:" + std::to_string(p.device) +
                           " is not an available gfx950 GPU; the device path has no CPU fallback");
    const unsigned threads = p.nthread ? p.nthread : std::min(16u, std::max(1u, std::thread::hardware_concurrency()));
    Pool pool(threads);

    Model m;
    m.objective = p.objective;
    m.n_features = nf;
    m.scale_pos_weight = p.scale_pos_weight;
    const auto t_sketch = Clock::now();
    // The device sketch gives the host sketch's cuts for unit row weights.
    const bool device_sketch =
        !given && !w && !p.host_sketch &&
        fbh_sketch_fits(p.device, n, nf, p.max_bin, cat, p.gpu_memory_budget);
    if (given) {
        check_cuts(*given, nf, p.max_bin, cat);
        m.cuts = *given;
    } else if (device_sketch) {
        m.cuts = sketch_matrix_device(p.device, src, n, nf, p.max_bin, cat, p.gpu_memory_budget,
                                      threads);
    } else {
        materialise();
        m.cuts = sketch_matrix(x, n, nf, p.max_bin, w, cat, threads);
    }
    const double sketch_s = std::chrono::duration<double>(Clock::now() - t_sketch).count();
    // 256-bin numeric features without a missing row take 8-bit cells
    // (Cuts::full): known from the device sketch, else checked over the rows
    // when they are in host memory.
    if (m.cuts.full.empty() && x) mark_full_features(m.cuts, x, n, nf, threads);
    // Base score: explicit, else the label mean weighted by the sample weights
    // only (Objective::estimate_base_score, src/training/objective.rs:42-60,
    // 452-470; scale_pos_weight enters the gradient weights alone,
    // src/training/mod.rs:1450-1468). A multiclass model keeps one intercept
    // per class: base_score copied, else initial_class_margins
    // (src/training/mod.rs:1430-1449).
    // reg:quantileerror takes the labels' alpha quantiles (one intercept per
    // alpha, src/training/objective.rs:452-456, src/training/mod.rs:1442-1444).
    const bool multi = p.objective == 2 || p.objective == 3;
    const bool quantile = p.objective == 4;
    const uint32_t K = multi ? p.num_class : quantile ? p.n_quantile_alpha : 1;
    std::vector<float> intercepts;
    if (quantile) {
        m.quantile_alpha.assign(p.quantile_alpha, p.quantile_alpha + K);
        intercepts = p.has_base_score ? std::vector<float>(K, p.base_score)
                                      : quantile_intercepts(p.quantile_alpha, K, y, w, n);
        if (K > 1) m.class_margins = intercepts;
        m.base_score = intercepts[0];
    } else if (multi) {
        m.class_margins = p.has_base_score ? std::vector<float>(K, p.base_score)
                                           : initial_class_margins(y, w, n, K);
        m.base_score = m.class_margins[0];
    } else if (p.has_base_score) {
        m.base_score = p.base_score;
    } else {
        double acc = 0.0;
        if (!w) {
            const double nn = (double)n;
            for (uint64_t i = 0; i < n; i++) acc = acc + (double)y[i] / nn;
            m.base_score = (float)acc;
        } else {
            double sw = 0.0;
            for (uint64_t i = 0; i < n; i++) sw = sw + (double)w[i];
            if (sw <= 0.0) {
                m.base_score = 0.5f;
            } else {
                for (uint64_t i = 0; i < n; i++) acc = acc + (double)y[i] / sw * (double)w[i];
                m.base_score = (float)acc;
            }
        }
    }
    if (p.objective == 1 && !(m.base_score >= 0.0f && m.base_score <= 1.0f))
        throw InputError("logistic base_score is a probability and must be in [0, 1]");
    const float margin = m.base_margin();

    // scale_pos_weight folded into the gradient weights (mod.rs:5470-5496).
    std::vector<float> gw;
    const float *grad_w = w;
    if (p.scale_pos_weight != 1.0f && (p.objective == 0 || p.objective == 1)) {
        gw.resize(n);
        for (uint64_t i = 0; i < n; i++) {
            const float wi = w ? w[i] : 1.0f;
            gw[i] = y[i] == 1.0f ? wi * p.scale_pos_weight : wi;
        }
        grad_w = gw.data();
    }

    // ---- device context (allocates everything once) ----
    std::vector<uint8_t> widths(nf);
    std::vector<uint32_t> nbins(nf);
    for (uint32_t f = 0; f < nf; f++) {
        widths[f] = (uint8_t)m.cuts.width(f);
        nbins[f] = m.cuts.n_bins(f);
    }
    fbh_shape shape{nf, widths.data(), nbins.data(), m.cuts.categorical.data()};
    fbh_config cfg{};
    cfg.memory_budget = p.gpu_memory_budget;
    cfg.tile_bytes = p.tile_bytes;
    cfg.rows_per_block = p.rows_per_block;
    cfg.stream_windows = p.hist_streams;
    cfg.resident_limit = p.resident_limit;
    cfg.n_outputs = K;
    uint32_t slots;
    if (p.grow_policy == 1) {
        const uint64_t leaves = p.max_leaves ? p.max_leaves : (1ull << std::min(p.max_depth, 14u));
        slots = (uint32_t)std::min<uint64_t>(leaves + 2, 16384);
        // A capped tree grown speculatively on the device (Grower::
        // lossguide_capped) needs a depthwise level's slots.
        if (p.max_leaves >= 2 && p.max_depth >= 1 && p.max_depth <= 14 &&
            (1ull << p.max_depth) <= 8ull * p.max_leaves)
            slots = std::max<uint32_t>(slots, 1u << (p.max_depth - 1));
    } else {
        slots = 1u << (p.max_depth > 0 ? p.max_depth - 1 : 0);
        if (p.max_leaves) slots = std::min(slots, p.max_leaves + 1);
        slots = std::max(slots, 2u);
    }
    cfg.hist_slots = slots;
    fbh_ctx *raw = nullptr;
    call(fbh_ctx_create(p.device, n, &shape, &cfg, &raw));
    std::unique_ptr<fbh_ctx, int (*)(fbh_ctx *)> ctx(raw, fbh_ctx_destroy);
    call(fbh_set_timing(ctx.get(), p.profile ? 1 : 0));
    // Binning: on the device when the budget's room holds the row staging
    // (and, when the plan streams, the binning stages), else column blocks
    // binned on the host (the same bins either way).
    const auto t_bin = Clock::now();
    bool device_binning = false;
    {
        fbh_plan plan{};
        call(fbh_ctx_plan(ctx.get(), &plan));
        const uint64_t held = fbh_ctx_device_bytes(ctx.get());
        const uint64_t need = fbh_rows_staging_bytes(ctx.get()) +
                              4 * (uint64_t)m.cuts.values.size() + 64 * (uint64_t)nf + (1u << 16);
        device_binning = !p.host_binning && held + need <= plan.budget;
    }
    if (device_binning) {
        call(fbh_set_cuts(ctx.get(), m.cuts.values.data(), m.cuts.offsets.data(),
                          m.cuts.categorical.data()));
        RowSource rows = src;
        rows.x = x;
        rows.each_chunk(n, nf, [&](uint64_t r0, uint64_t k, const float *chunk) {
            const uint64_t step = 1u << 20;
            for (uint64_t b = 0; b < k; b += step)
                call(fbh_upload_rows(ctx.get(), chunk + b * nf, r0 + b, std::min(step, k - b)));
        });
        call(fbh_finish_rows(ctx.get()));
    } else {
        materialise();
        for (const auto &feats : blocks_by_width(m.cuts, p.cols_per_block)) {
            const uint32_t wdt = m.cuts.width(feats[0]);
            std::vector<uint8_t> buf((size_t)feats.size() * n * wdt);
            bin_columns(x, n, nf, m.cuts, feats, wdt, buf.data(), threads);
            call(fbh_upload_block(ctx.get(), feats.data(), (uint32_t)feats.size(), wdt, buf.data()));
        }
    }
    const double bin_s = std::chrono::duration<double>(Clock::now() - t_bin).count();
    g_stats = fbt_stats{};
    g_stats.device_binning = device_binning ? 1 : 0;
    g_stats.device_sketch = device_sketch ? 1 : 0;
    g_stats.sketch_seconds = sketch_s;
    g_stats.bin_seconds = bin_s;
    g_stats.device_bytes = (double)fbh_ctx_device_bytes(ctx.get());
    g_stats.setup_seconds = std::chrono::duration<double>(Clock::now() - t_setup).count();

    // ---- round loop ----
    const auto t_train = Clock::now();
    // Host margins feed the logistic sigmoid; the device keeps its own copy
    // (the same f32 additions), which squared error uses directly.
    std::vector<float> pred((uint64_t)K * n, margin);
    // base_margin: every row starts at its own margin (class-major), the
    // intercepts stay as estimated (src/training/mod.rs:1831-1852, 2605-2616).
    if (p.base_margin) std::copy(p.base_margin, p.base_margin + (uint64_t)K * n, pred.begin());
    const float *fw = checked_weights(p.feature_weights, nf);
    NestedSets nested;
    nested.bylevel = rate_or_one(p.colsample_bylevel);
    nested.bynode = rate_or_one(p.colsample_bynode);
    nested.w = fw;
    nested.seed = p.seed;
    Grower grower(ctx.get(), p, m.cuts, mono, slots, nested);
    grower.n_rows_ = (uint32_t)n;
    {
        fbh_plan plan{};
        call(fbh_ctx_plan(ctx.get(), &plan));
        grower.device_trees_ = !p.host_levels && plan.columns_resident &&
                               plan.resident_tiles == plan.n_tiles && slots <= 16384;
    }
    const uint32_t obj = p.objective;
    // train_multiclass_rounds takes the sample weights (scale_pos_weight is
    // a binary objective's).
    if (multi) call(fbh_set_multiclass(ctx.get(), K, y, w, m.class_margins.data()));
    else if (quantile)
        call(fbh_set_quantile(ctx.get(), K, p.quantile_alpha, y, w, intercepts.data()));
    else call(fbh_set_objective(ctx.get(), obj, y, grad_w, margin));
    if (p.base_margin) call(fbh_set_margins(ctx.get(), pred.data()));
    // gpu_math="fast" (fast_gradient_and_quantize, src/backend/cuda/train_ctx.rs:2404-2512):
    // the logistic gradient takes the hardware exponential on the device.
    call(fbh_set_gpu_math(ctx.get(), p.gpu_math));
    SigmoidJob job{&pool, pred.data(), &grower.leaf_values()};
    const bool dev_sigmoid =
        obj == 1 && !p.host_sigmoid && (p.gpu_math == 1 || device_sigmoid_matches_host(p.device));
    double grad_s = 0.0;
    g_round_wall.assign(p.n_rounds, 0.0);
    g_round_hist_ms.assign(p.n_rounds, 0.0);
    g_round_hist_bytes.assign(p.n_rounds, 0);
    g_round_hist_launches.assign(p.n_rounds, 0);
    auto t_round = Clock::now();
    const auto t_first = t_round;
    double ms_seen = 0.0;
    uint64_t bytes_seen = 0, launches_seen = 0;
    // FB_LOG_ROUNDS=k: a progress line on stderr every k rounds.
    const char *log_env = std::getenv("FB_LOG_ROUNDS");
    const unsigned long log_every = log_env ? std::strtoul(log_env, nullptr, 10) : 0ul;
    auto close_round = [&](uint32_t r) {
        const auto now = Clock::now();
        g_round_wall[r] = std::chrono::duration<double>(now - t_round).count();
        t_round = now;
        if (log_every && ((r + 1) % log_every == 0 || r + 1 == p.n_rounds)) {
            std::fprintf(stderr, "[ferrisboost_amd] round %u of %u done, %.1f s\n", r + 1,
                         p.n_rounds, std::chrono::duration<double>(now - t_first).count());
            std::fflush(stderr);
        }
        if (p.profile) {
            double ms = 0.0;
            uint64_t launches = 0, bytes = 0;
            call(fbh_hist_timing(ctx.get(), &ms, &launches, &bytes, 0));
            g_round_hist_ms[r] = ms - ms_seen;
            g_round_hist_bytes[r] = bytes - bytes_seen;
            g_round_hist_launches[r] = launches - launches_seen;
            ms_seen = ms;
            bytes_seen = bytes;
            launches_seen = launches;
        }
    };
    // Device-grown trees are collected one round late: round r + 1's
    // gradients and tree are enqueued before tree r is collected, with the
    // quantizer scales left on the device, so the host rebuilds tree r while
    // the device works on round r + 1 and no round waits for the host. A
    // host sigmoid needs tree r's leaf values first, so it collects before
    // its gradients (and takes the scales back to the host).
    const bool overlap = grower.device_growth() && !grower.deferred_leaves();
    const bool host_sig = obj == 1 && !dev_sigmoid;
    const bool device_scales = overlap && !host_sig;
    uint32_t pending = 0;
    auto collect_all = [&]() {
        for (; pending; pending--) m.trees.push_back(grower.collect());
    };
    // A multiclass round (train_multiclass_rounds, src/training/mod.rs:
    // 2578-2850) takes every class's statistics from the round's starting
    // margins, then grows one tree per class in class order: row and column
    // sampling key on the tree index round * K + class, and each tree's
    // leaves go to its own class's margins.
    for (uint32_t round = 0; round < p.n_rounds; round++) {
        if (pending && round == p.sync_round) collect_all();  // the device is idle when this round starts
        if (round > 0) close_round(round - 1);
        if (pending && host_sig) collect_all();
        if (multi) call(fbh_multiclass_begin_round(ctx.get()));
        for (uint32_t cls = 0; cls < K; cls++) {
            const uint64_t tree = (uint64_t)round * K + cls;
            if (K > 1) call(fbh_set_output(ctx.get(), cls));
            const auto tg = Clock::now();
            double scales[2];
            int64_t root_sum[2];
            call(fbh_gradient_exchange(ctx.get(), host_sig ? sigmoid_chunk : nullptr, &job,
                                       sample_threshold(p.subsample), p.seed, tree,
                                       device_scales ? nullptr : scales,
                                       overlap ? nullptr : root_sum));
            grad_s += std::chrono::duration<double>(Clock::now() - tg).count();
            if (pending && !device_scales) collect_all();
            std::vector<uint32_t> feats;
            if (p.colsample_bytree < 1.0f)
                feats = sample_columns(nf, p.colsample_bytree, p.seed, tree, fw);
            if (grower.masked()) {
                std::vector<uint32_t> all;
                if (feats.empty())
                    for (uint32_t f = 0; f < nf; f++) all.push_back(f);
                grower.begin_tree(feats.empty() ? std::move(all) : feats, tree);
            }
            fbh_span root;
            call(fbh_begin_tree(ctx.get(), feats.empty() ? nullptr : feats.data(),
                                (uint32_t)feats.size(), mono.data(), nf, &root));
            if (overlap) {
                if (!device_scales) grower.lm_scales(scales);
                grower.grow_async(nullptr);
                if (++pending == 2) {
                    m.trees.push_back(grower.collect());
                    pending--;
                }
            } else {
                m.trees.push_back(grower.grow(scales, root_sum));
            }
        }
    }
    collect_all();
    // The last round ends when its tree is collected (the device is then
    // idle); the one download of the training margins comes after it.
    if (overlap && p.n_rounds > 0) close_round(p.n_rounds - 1);
    call(fbh_download_margin(ctx.get(), pred.data()));
    if (!overlap && p.n_rounds > 0) close_round(p.n_rounds - 1);
    g_stats.train_seconds = std::chrono::duration<double>(Clock::now() - t_train).count();
    g_stats.host_gradient_seconds = grad_s;
    g_stats.device_trees = grower.device_trees;
    g_stats.rounds = p.n_rounds;
    g_stats.device_sigmoid = dev_sigmoid ? 1 : 0;
    {
        fbh_plan plan{};
        call(fbh_ctx_plan(ctx.get(), &plan));
        g_stats.n_tiles = plan.n_tiles;
        g_stats.resident_tiles = plan.resident_tiles;
        g_stats.planned_bytes = plan.peak_bytes;
        g_stats.budget_bytes = plan.budget;
        g_stats.streamed_bytes = fbh_ctx_streamed_bytes(ctx.get());
        g_stats.device_bytes = (double)fbh_ctx_device_bytes(ctx.get());
    }
    double ms = 0.0;
    uint64_t launches = 0, bytes = 0;
    call(fbh_hist_timing(ctx.get(), &ms, &launches, &bytes, 0));
    g_stats.hist_kernel_ms = ms;
    g_stats.hist_launches = launches;
    g_stats.hist_bytes = bytes;
    m.train_margins = std::move(pred);
    return m;
}

}  // namespace fbt
