// oracle.cpp -- CPU restatement of the FerrisBoost CPU engine.
//
// TEST INFRASTRUCTURE ONLY. The test suite, the smoke check and the
// benchmark's CPU-baseline leg load this library to check or time against
// it; the shipped package never links, loads or calls it.
//
// Each function names the reference file:line it restates (reference crate
// `ferrisboost` 0.1.1, Rust). The reference cannot be compiled here (no Rust
// toolchain), so parity is pinned instead by:
//   * end to end (quantizer + sketch + histogram + split + partition + leaf
//     values + logistic / squared-error gradients + base margin + predict):
//     the reference's XGBoost-3.4.1 golden margins, bit-exact, all 44 cases
//     of tests/fixtures/{index,weighted_index,monotone_index}.json
//     (unweighted, weighted and monotone-constrained);
//   * histogram: brute-force per-row accumulation, order independence, the
//     sibling identity parent = left + right, the 16-bit / 8-bit equivalence;
//   * split: brute-force enumeration over every (bin, missing direction)
//     partition of the rows (src/training/split.rs:806-898 restated in the
//     Python tests), missing-direction closed forms;
//   * partition: the stable-order closed form;
//   * TreeSHAP: additivity (sum of contributions = margin), exact Shapley
//     values by subset enumeration on small trees, the quadrature rule
//     integrating polynomials of degree <= 15 exactly;
//   * colsample: the reference's count, sortedness, nested and weighted
//     sampler tests (src/data/colsample.rs:313-465), the laws of the
//     weighted draws (first draw in proportion to weight, pairs by
//     successive draws) and of uniform subsets (tests/test_oracle_colsample.py);
//   * growth policies and categorical splits: the reference's lossguide and
//     max_leaves tests (tests/lossguide.rs, tests/max_leaves.rs) and its
//     categorical split tests (src/training/split.rs:1371-1590), restated in
//     tests/test_oracle_growth.py;
//   * sketch (tests/test_sketch_pins.py): in the exact-summary regime
//     (max_bin < distinct values <= 16 * max_bin) the cuts equal the cuts of
//     numpy's exact unique counts in any batch order; in the lossy regime
//     (C2's and C4's columns) estimated ranks never exceed true ranks and
//     every cut's true midrank lies in [target, target + B(N, limit)).
//     Planted in a copy of this file, a swapped pass_a / pass_b in
//     merge_entries, a dedup that keeps the last rmin, a cut walk with <=,
//     and ranks kept in f64 each fail those tests. Three choices are left
//     open because either way gives a valid summary: the operand order of
//     the level merge, the tie rule of merge_entries (<= vs <) and the tie
//     rule of compress's target walk; they move lossy-regime cuts by less
//     than the bound, and only the reference's own cut values on
//     high-cardinality data could pin them (parity unpinned there).
// Floating point: compiled with -ffp-contract=off and without fast-math so
// every f32 / f64 operation rounds like the reference's (Rust does not
// contract a*b+c). expf / logf come from the same glibc the reference links.

#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <memory>
#include <queue>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

using u8 = uint8_t;
using u16 = uint16_t;
using u32 = uint32_t;
using u64 = uint64_t;
using i64 = int64_t;

constexpr float MIN_GAIN_EPS = 1e-6f;      // src/training/split.rs:15
constexpr float K_RT_EPS = 1e-6f;          // src/training/objective.rs:18
constexpr u32 SKETCH_RATIO = 16;           // src/data/sketch.rs:28

// ------------------------------------------------------------ fixed point
// GradPairFixed (src/types.rs:151-227): wrapping i64 pair.
struct Fixed {
    i64 g = 0, h = 0;
};
inline Fixed add(Fixed a, Fixed b) {
    return {(i64)((u64)a.g + (u64)b.g), (i64)((u64)a.h + (u64)b.h)};
}
inline Fixed sub(Fixed a, Fixed b) {
    return {(i64)((u64)a.g - (u64)b.g), (i64)((u64)a.h - (u64)b.h)};
}
inline bool eq(Fixed a, Fixed b) { return a.g == b.g && a.h == b.h; }

// pow2_scale (src/types.rs:367-385).
double pow2_scale(double max_abs, u64 n_rows) {
    if (!(max_abs > 0.0) || !std::isfinite(max_abs)) return 1.0;
    double budget = (double)(1ull << 62) / (double)std::max<u64>(n_rows, 1);
    double raw = budget / max_abs;
    if (!std::isfinite(raw) || raw <= 0.0) return 1.0;
    double l = std::floor(std::log2(raw));
    int e;
    if (std::isnan(l)) e = 0;
    else if (l > 2147483647.0) e = 2147483647;
    else if (l < -2147483648.0) e = (int)-2147483648LL;
    else e = (int)l;
    e = std::max(-1000, std::min(1000, e));
    return std::exp2((double)e);
}

// `as i64` in Rust saturates (NaN -> 0).
inline i64 sat_i64(double x) {
    if (std::isnan(x)) return 0;
    if (x >= 9223372036854775808.0) return std::numeric_limits<i64>::max();
    if (x < -9223372036854775808.0) return std::numeric_limits<i64>::min();
    return (i64)x;
}

// GradQuantizer (src/types.rs:239-341).
struct Quantizer {
    double gs = 1, hs = 1, gi = 1, hi = 1;
    static Quantizer from_bounds(double mg, double mh, u64 n) {
        if (!(std::isfinite(mg) && std::isfinite(mh) && mg >= 0.0 && mh >= 0.0))
            throw std::runtime_error(
                "non-finite gradient or Hessian (or invalid bounds); reduce extreme labels, "
                "weights, base_score or objective parameters");
        Quantizer q;
        q.gs = pow2_scale(mg, n);
        q.hs = pow2_scale(mh, n);
        q.gi = 1.0 / q.gs;
        q.hi = 1.0 / q.hs;
        return q;
    }
    Fixed to_fixed(float g, float h) const {
        // quantize (src/types.rs:352-355): round half away from zero.
        return {sat_i64(std::round((double)g * gs)), sat_i64(std::round((double)h * hs))};
    }
    void to_f64(Fixed f, double &g, double &h) const {
        g = (double)f.g * gi;
        h = (double)f.h * hi;
    }
};

inline double finite_abs(float v) {  // src/types.rs:343-350
    return std::isfinite(v) ? std::fabs((double)v) : INFINITY;
}

// ------------------------------------------------------------ sketch
// src/data/sketch.rs:28-435.
struct Entry {
    float value, weight, rmin, rmax;
    float rmid() const { return 0.5f * (rmin + rmax); }
};

std::vector<Entry> build_summary(std::vector<std::pair<float, float>> &pairs) {
    std::sort(pairs.begin(), pairs.end(),
              [](const std::pair<float, float> &a, const std::pair<float, float> &b) {
                  return a.first < b.first;
              });
    std::vector<Entry> out;
    out.reserve(pairs.size());
    float acc = 0.0f;
    size_t i = 0;
    while (i < pairs.size()) {
        float v = pairs[i].first;
        float w = 0.0f;
        while (i < pairs.size() && pairs[i].first == v) {
            w += pairs[i].second;
            i++;
        }
        out.push_back({v, w, acc, acc + w});
        acc += w;
    }
    return out;
}

std::vector<Entry> dedup_same_value(const std::vector<Entry> &entries) {
    std::vector<Entry> out;
    out.reserve(entries.size());
    for (const Entry &e : entries) {
        if (!out.empty() && out.back().value == e.value) {
            Entry &last = out.back();
            last.weight += e.weight;
            last.rmin = std::min(last.rmin, e.rmin);
            last.rmax = std::max(last.rmax, e.rmax);
        } else {
            out.push_back(e);
        }
    }
    return out;
}

std::vector<Entry> merge_entries(const std::vector<Entry> &a, const std::vector<Entry> &b) {
    if (a.empty()) return b;
    if (b.empty()) return a;
    std::vector<Entry> out;
    out.reserve(a.size() + b.size());
    size_t i = 0, j = 0;
    float pass_a = 0.0f, pass_b = 0.0f;
    while (i < a.size() || j < b.size()) {
        bool take_a;
        if (i < a.size() && j < b.size()) take_a = a[i].value <= b[j].value;
        else take_a = i < a.size();
        if (take_a) {
            Entry e = a[i];
            out.push_back({e.value, e.weight, e.rmin + pass_b, e.rmax + pass_b});
            pass_a = e.rmax;
            i++;
        } else {
            Entry e = b[j];
            out.push_back({e.value, e.weight, e.rmin + pass_a, e.rmax + pass_a});
            pass_b = e.rmax;
            j++;
        }
    }
    return dedup_same_value(out);
}

// Test instrumentation: how often compress's ceiling moved a pick below the
// entry its target walk reached (read by the sketch-bound tests).
std::atomic<uint64_t> g_compress_clamps{0};

std::vector<Entry> compress(const std::vector<Entry> &entries, size_t max_size) {
    size_t n = entries.size();
    if (n <= max_size) return entries;
    float total = entries[n - 1].rmax;
    size_t slots = max_size - 1;
    std::vector<Entry> out;
    out.reserve(max_size);
    out.push_back(entries[0]);
    size_t taken = 0;
    for (size_t k = 1; k < slots; k++) {
        float target = total * (float)k / (float)slots;
        size_t j = taken + 1;
        while (j < n - 1 && entries[j].rmid() < target) j++;
        size_t ceiling = n - 1 - (slots - 1 - k);
        if (std::max(j, taken + 1) > ceiling) g_compress_clamps++;
        j = std::min(std::max(j, taken + 1), ceiling);
        if (j > taken) {
            out.push_back(entries[j]);
            taken = j;
        }
    }
    if (taken < n - 1) out.push_back(entries[n - 1]);
    return out;
}

float midpoint(float a, float b) {  // src/data/sketch.rs:290-302
    float d = b - a;
    float m = std::isfinite(d) ? a + d * 0.5f : a * 0.5f + b * 0.5f;
    return m <= a ? b : m;
}

struct FeatureSketch {
    std::vector<std::pair<float, float>> buffer;
    std::vector<std::vector<Entry>> levels;
    std::vector<bool> occupied;
    size_t limit;
    float total_weight = 0.0f;
    bool cat = false;
    int max_code = -1;
    bool bad = false;
    float bad_value = 0.0f;

    explicit FeatureSketch(size_t max_bins, bool categorical) {
        cat = categorical;
        limit = categorical ? 0 : std::max<size_t>(max_bins * SKETCH_RATIO, 32);
        if (!cat) buffer.reserve(limit);
    }

    void push(float value, float weight) {  // src/data/sketch.rs:128-149
        if (cat) {
            if (!std::isnan(value)) {
                bool invalid = value < 0.0f || value > 65533.0f || value != std::trunc(value);
                if (invalid) {
                    if (!bad) {
                        bad = true;
                        bad_value = value;
                    }
                } else {
                    max_code = std::max(max_code, (int)value);
                }
            }
            return;
        }
        if (std::isnan(value) || weight <= 0.0f) return;
        total_weight += weight;
        buffer.push_back({value, weight});
        if (buffer.size() >= limit) drain_buffer();
    }

    void drain_buffer() {
        if (buffer.empty()) return;
        std::vector<Entry> summary = compress(build_summary(buffer), limit);
        buffer.clear();
        insert_level(std::move(summary));
    }

    void insert_level(std::vector<Entry> cur) {
        size_t lvl = 0;
        for (;;) {
            if (lvl == levels.size()) {
                levels.push_back(std::move(cur));
                occupied.push_back(true);
                return;
            }
            if (!occupied[lvl]) {
                levels[lvl] = std::move(cur);
                occupied[lvl] = true;
                return;
            }
            std::vector<Entry> existing = std::move(levels[lvl]);
            occupied[lvl] = false;
            levels[lvl].clear();
            cur = compress(merge_entries(existing, cur), limit);
            lvl++;
        }
    }

    std::vector<Entry> collapse() {
        drain_buffer();
        std::vector<Entry> acc;
        for (size_t i = 0; i < levels.size(); i++) {
            if (!occupied[i]) continue;
            acc = acc.empty() ? levels[i] : merge_entries(acc, levels[i]);
        }
        levels.clear();
        occupied.clear();
        if (!acc.empty()) {
            levels.push_back(compress(acc, limit));
            occupied.push_back(true);
            return levels[0];
        }
        return {};
    }

    std::vector<float> cuts(size_t max_bins) {  // src/data/sketch.rs:236-275
        std::vector<float> out;
        if (cat) {
            u32 mc = (u32)std::max(max_code, 0);
            for (u32 c = 1; c <= mc; c++) out.push_back((float)c);
            return out;
        }
        size_t n_cuts = max_bins > 0 ? max_bins - 1 : 0;
        if (n_cuts == 0) return out;
        std::vector<Entry> entries = collapse();
        if (entries.empty()) return out;
        if (entries.size() <= n_cuts) {
            for (size_t i = 0; i + 1 < entries.size(); i++)
                out.push_back(midpoint(entries[i].value, entries[i + 1].value));
            return out;
        }
        float total = entries.back().rmax;
        for (size_t k = 1; k <= n_cuts; k++) {
            float target = total * (float)k / (float)max_bins;
            size_t idx = 0;
            {
                size_t lo = 0, hi = entries.size();
                while (lo < hi) {
                    size_t mid = (lo + hi) / 2;
                    if (entries[mid].rmid() < target) lo = mid + 1;
                    else hi = mid;
                }
                idx = std::min(lo, entries.size() - 1);
            }
            float v = entries[idx].value;
            if (out.empty() || v > out.back()) out.push_back(v);
        }
        return out;
    }
};

// ------------------------------------------------------------ cuts / bins
// BinWidth (src/data/bins.rs:17-76), BinCuts (src/data/columns.rs:50-360).
struct Cuts {
    std::vector<float> values;
    std::vector<u32> offsets;
    std::vector<u8> cat;
    u32 n_feats() const { return (u32)offsets.size() - 1; }
    u32 n_bins(u32 f) const { return offsets[f + 1] - offsets[f] + 1; }
    bool is_cat(u32 f) const { return f < cat.size() && cat[f]; }
    int width(u32 f) const {
        u32 n = n_bins(f);
        if (is_cat(f)) return n <= 254 ? 1 : 2;
        return n <= 255 ? 1 : 2;
    }
    const float *cuts_for(u32 f) const { return values.data() + offsets[f]; }
    u32 n_cuts(u32 f) const { return offsets[f + 1] - offsets[f]; }
    u32 find_bin(u32 f, float v) const {  // columns.rs:335-341, categorical.rs code_to_bin
        if (is_cat(f)) {
            u32 nb = n_bins(f);
            if (v >= 0.0f && v < (float)nb) return (u32)v;
            return (nb <= 254 ? 255u : 65535u) - 1;
        }
        const float *c = cuts_for(f);
        return (u32)(std::upper_bound(c, c + n_cuts(f), v, [](float a, float b) { return a < b; }) -
                     c);
    }
};

u32 missing_of(int width) { return width == 1 ? 0xFFu : 0xFFFFu; }

struct Block {
    std::vector<u32> feats;
    int width;
    u64 n_rows;
    std::vector<u8> d8;
    std::vector<u16> d16;
    u32 bin(u32 local, u64 row) const {
        return width == 1 ? d8[local * n_rows + row] : d16[local * n_rows + row];
    }
};

// partition_features_by_width (src/data/columns.rs:446-463).
std::vector<std::vector<u32>> partition_by_width(const std::vector<int> &widths, u32 cols) {
    std::vector<std::vector<u32>> blocks;
    for (int w : {1, 2}) {
        std::vector<u32> feats;
        for (u32 f = 0; f < widths.size(); f++)
            if (widths[f] == w) feats.push_back(f);
        u32 per = (cols + (u32)w - 1) / (u32)w;
        for (size_t i = 0; i < feats.size(); i += per)
            blocks.emplace_back(feats.begin() + i,
                                feats.begin() + std::min(feats.size(), i + per));
    }
    std::sort(blocks.begin(), blocks.end(),
              [](const std::vector<u32> &a, const std::vector<u32> &b) { return a[0] < b[0]; });
    return blocks;
}

// DenseSource binning pass (src/source/dense.rs:145-190): one sketch per
// feature, built start to finish by one thread, never merged across threads,
// so the cuts do not depend on the thread count.
Cuts sketch_cuts(const float *x, u64 n, u32 nf, u32 max_bin, const float *w, const u8 *cat,
                 unsigned threads = 0) {
    if (threads == 0) threads = std::min(16u, std::max(1u, std::thread::hardware_concurrency()));
    std::vector<std::vector<float>> per(nf);
    std::vector<int> bad(nf, 0);
    auto one = [&](u32 f) {
        FeatureSketch sk(max_bin, cat && cat[f]);
        for (u64 r = 0; r < n; r++) sk.push(x[r * nf + f], w ? w[r] : 1.0f);
        bad[f] = sk.bad;
        per[f] = sk.cuts(max_bin);
    };
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < std::min<unsigned>(threads, nf); t++)
        pool.emplace_back([&, t] {
            for (u32 f = t; f < nf; f += std::min<unsigned>(threads, nf)) one(f);
        });
    for (auto &th : pool) th.join();
    Cuts c;
    c.offsets.push_back(0);
    for (u32 f = 0; f < nf; f++) {
        if (bad[f]) throw std::runtime_error("categorical feature contains an invalid code");
        c.values.insert(c.values.end(), per[f].begin(), per[f].end());
        c.offsets.push_back((u32)c.values.size());
        c.cat.push_back(cat && cat[f] ? 1 : 0);
    }
    return c;
}

std::vector<Block> bin_blocks(const float *x, u64 n, u32 nf, const Cuts &c, u32 cols) {
    std::vector<int> widths(nf);
    for (u32 f = 0; f < nf; f++) widths[f] = c.width(f);
    std::vector<Block> blocks;
    for (auto &feats : partition_by_width(widths, cols)) {
        Block b;
        b.feats = feats;
        b.width = widths[feats[0]];
        b.n_rows = n;
        if (b.width == 1) b.d8.assign(feats.size() * n, 0);
        else b.d16.assign(feats.size() * n, 0);
        for (size_t l = 0; l < feats.size(); l++) {
            u32 f = feats[l];
            for (u64 r = 0; r < n; r++) {
                float v = x[r * nf + f];
                u32 bin = std::isnan(v) ? missing_of(b.width) : c.find_bin(f, v);
                if (b.width == 1) b.d8[l * n + r] = (u8)bin;
                else b.d16[l * n + r] = (u16)bin;
            }
        }
        blocks.push_back(std::move(b));
    }
    return blocks;
}

// ------------------------------------------------------------ params
struct Params {
    orc_params p;
    std::vector<int8_t> monotone;
    int8_t monotone_of(u32 f) const { return f < monotone.size() ? monotone[f] : 0; }
};

// ------------------------------------------------------------ split math
// src/training/split.rs:113-270.
struct Bounds {
    float lo = -std::numeric_limits<float>::max();
    float hi = std::numeric_limits<float>::max();
    float apply(float w) const {
        if (w < lo) return lo;
        if (w > hi) return hi;
        return w;
    }
    void children(int8_t c, float wl, float wr, Bounds &l, Bounds &r) const {
        float mid = (wl + wr) / 2.0f;
        l = *this;
        r = *this;
        if (c < 0) {
            l.lo = mid;
            r.hi = mid;
        } else if (c > 0) {
            l.hi = mid;
            r.lo = mid;
        }
    }
};

double threshold_l1(double g, float alpha) {
    double a = (double)alpha;
    if (g > a) return g - a;
    if (g < -a) return g + a;
    return 0.0;
}

float xgb_weight(double g, double h, const orc_params &p) {
    if (h <= 0.0) return 0.0f;
    double dw = -threshold_l1(g, p.alpha) / (h + (double)p.lambda_);
    float mds = p.max_delta_step;
    if (mds != 0.0f && std::fabs(dw) > (double)mds) dw = std::copysign((double)mds, dw);
    return (float)dw;
}

float gain_given_weight(double g, double h, float w, const orc_params &p) {
    if (h <= 0.0) return 0.0f;
    double square = (double)(w * w);
    double l1 = 2.0 * (double)p.alpha * (double)std::fabs(w);
    return (float)(-((2.0 * g * (double)w + (h + (double)p.lambda_) * square) + l1));
}

float bounded_node_gain(double g, double h, const orc_params &p, Bounds b) {
    float w = b.apply(xgb_weight(g, h, p));
    return gain_given_weight(g, h, w, p);
}

bool bounded_split_gain(float parent, double lg, double lh, double rg, double rh, int8_t c,
                        Bounds b, const orc_params &p, float &out) {
    double mcw = (double)p.min_child_weight;
    if (!(lh > 0.0 && rh > 0.0 && lh >= mcw && rh >= mcw)) return false;
    float wl = b.apply(xgb_weight(lg, lh, p));
    float wr = b.apply(xgb_weight(rg, rh, p));
    if ((c > 0 && wl > wr) || (c < 0 && wl < wr)) return false;
    float gain = gain_given_weight(lg, lh, wl, p) + gain_given_weight(rg, rh, wr, p);
    float loss = gain - parent;
    out = (float)((double)loss - (double)p.gamma);
    return true;
}

double plain_gain(double g, double h, const orc_params &p) { return g * g / (h + (double)p.lambda_); }

struct Cand {
    bool found = false;
    u32 feat = 0, bin = 0;
    float gain = 0;
    Fixed left, right;
    bool missing_left = false;
    std::vector<u64> cats;  // right-going set; empty = numeric
    bool is_cat = false;
};

// update_best (src/training/split.rs:260-270).
void update_best(Cand &best, const Cand &c) {
    if (!(c.gain > MIN_GAIN_EPS)) return;
    if (!best.found || c.gain > best.gain) best = c;
}

// reduce_best (src/training/split.rs:631-642).
void reduce_into(Cand &best, const Cand &c) {
    if (!c.found) return;
    if (best.found && c.gain == best.gain && c.feat < best.feat && c.gain > MIN_GAIN_EPS) {
        best = c;
        return;
    }
    update_best(best, c);
}

struct SplitCtx {
    const Quantizer *q;
    const orc_params *p;
    bool given_weight;
    Bounds bounds;
    const Params *params;  // monotone lookup (may be null)
    const std::vector<int8_t> *mono;
    float bounded_parent;
    double parent_gain;
    int8_t mono_of(u32 f) const { return (mono && f < mono->size()) ? (*mono)[f] : 0; }
    bool gain(u32 feat, Fixed l, Fixed r, float &out) const {
        double lg, lh, rg, rh;
        q->to_f64(l, lg, lh);
        q->to_f64(r, rg, rh);
        if (given_weight)
            return bounded_split_gain(bounded_parent, lg, lh, rg, rh, mono_of(feat), bounds, *p,
                                      out);
        double mcw = (double)p->min_child_weight;
        if (lh < mcw || rh < mcw) return false;
        double g = plain_gain(lg, lh, *p) + plain_gain(rg, rh, *p) - parent_gain - (double)p->gamma;
        out = (float)g;
        return true;
    }
};

// enumerate_categorical (src/training/split.rs:484-617).
void enumerate_categorical(u32 feat, const Fixed *bins, u32 n, Fixed node_sum, const SplitCtx &sc,
                           Cand &best) {
    struct Local {
        bool found = false;
        float gain = 0.0f;
        Fixed l, r;
        bool ml = false;
        size_t at = 0;
    };
    Local local;
    auto consider = [&](Local &loc, Fixed l, Fixed r, bool ml, size_t at) {
        float g;
        if (sc.gain(feat, l, r, g)) {
            if (g > MIN_GAIN_EPS && (!loc.found || g > loc.gain)) {
                loc.found = true;
                loc.gain = g;
                loc.l = l;
                loc.r = r;
                loc.ml = ml;
                loc.at = at;
            }
        }
    };
    size_t nwords = n <= 256 ? 4 : (n + 63) / 64;
    auto finish = [&](const Local &loc, const std::vector<u32> &set_members) {
        if (!loc.found) return;
        Cand c;
        c.found = true;
        c.feat = feat;
        c.bin = 0;
        c.gain = loc.gain;
        c.left = loc.l;
        c.right = loc.r;
        c.missing_left = loc.ml;
        c.is_cat = true;
        c.cats.assign(nwords, 0);
        for (u32 cat : set_members) c.cats[cat >> 6] |= 1ull << (cat & 63);
        update_best(best, c);
    };
    if ((u64)n < (u64)sc.p->max_cat_to_onehot) {
        Fixed fs;
        for (u32 i = 0; i < n; i++) fs = add(fs, bins[i]);
        Fixed missing = sub(node_sum, fs);
        for (u32 i = 0; i < n; i++) {
            consider(local, sub(node_sum, bins[i]), bins[i], true, i);
            Fixed right = add(bins[i], missing);
            consider(local, sub(node_sum, right), right, false, i);
        }
        if (local.found) finish(local, {(u32)local.at});
        return;
    }
    std::vector<float> weights(n);
    for (u32 i = 0; i < n; i++) {
        double g, h;
        sc.q->to_f64(bins[i], g, h);
        weights[i] = xgb_weight(g, h, *sc.p);
    }
    std::vector<u32> order(n);
    for (u32 i = 0; i < n; i++) order[i] = i;
    std::stable_sort(order.begin(), order.end(),
                     [&](u32 a, u32 b) { return weights[a] < weights[b]; });
    size_t n_scan = std::min<size_t>(sc.p->max_cat_threshold, n);
    if (n_scan < 2) return;
    auto prefix = [&](size_t k) { return std::vector<u32>(order.begin(), order.begin() + k); };
    Fixed right;
    for (size_t k = 0; k + 1 < n_scan; k++) {
        right = add(right, bins[order[k]]);
        consider(local, sub(node_sum, right), right, true, k + 1);
    }
    if (local.found) finish(local, prefix(local.at));
    local = Local();
    Fixed left;
    for (size_t j = n; j-- > n - (n_scan - 1);) {
        left = add(left, bins[order[j]]);
        consider(local, left, sub(node_sum, left), false, j);
    }
    if (local.found) finish(local, prefix(local.at));
}

// best_split_in_block_typed (src/training/split.rs:331-461).
Cand best_split_in_block(const Fixed *hist, const std::vector<u32> &feat_ids,
                         const std::vector<u32> &offsets, Fixed node_sum, const SplitCtx &sc0,
                         const std::vector<u32> *sampled, const std::vector<u8> *categorical) {
    SplitCtx sc = sc0;
    double ng, nh;
    sc.q->to_f64(node_sum, ng, nh);
    sc.parent_gain = plain_gain(ng, nh, *sc.p);
    sc.bounded_parent = sc.given_weight ? bounded_node_gain(ng, nh, *sc.p, sc.bounds) : 0.0f;
    Cand best;
    for (size_t local = 0; local < feat_ids.size(); local++) {
        u32 feat = feat_ids[local];
        if (sampled && !std::binary_search(sampled->begin(), sampled->end(), feat)) continue;
        u32 lo = offsets[local], hi = offsets[local + 1];
        const Fixed *bins = hist + lo;
        u32 n = hi - lo;
        if (categorical && feat < categorical->size() && (*categorical)[feat]) {
            enumerate_categorical(feat, bins, n, node_sum, sc, best);
            continue;
        }
        Fixed left;
        for (u32 i = 0; i < n; i++) {
            left = add(left, bins[i]);
            Fixed right = sub(node_sum, left);
            float g;
            if (!sc.gain(feat, left, right, g)) continue;
            Cand c;
            c.found = true;
            c.feat = feat;
            c.bin = i + 1;
            c.gain = g;
            c.left = left;
            c.right = right;
            c.missing_left = false;
            update_best(best, c);
        }
        if (eq(left, node_sum)) continue;
        Fixed right;
        for (u32 i = n; i-- > 0;) {
            right = add(right, bins[i]);
            Fixed l2 = sub(node_sum, right);
            float g;
            if (!sc.gain(feat, l2, right, g)) continue;
            Cand c;
            c.found = true;
            c.feat = feat;
            c.bin = i;
            c.gain = g;
            c.left = l2;
            c.right = right;
            c.missing_left = true;
            update_best(best, c);
        }
    }
    return best;
}

// ------------------------------------------------------------ histogram
// hist::build_rows (src/training/hist.rs:148-176), column-sliced form.
void hist_rows(const Block &b, const std::vector<u32> &locals, const std::vector<u32> &offsets,
               const std::vector<Fixed> &gpair, const u32 *rows, size_t n_sel, Fixed *out) {
    const u32 missing = missing_of(b.width);
    const size_t tile = 4096;
    for (size_t c0 = 0; c0 < n_sel; c0 += tile) {
        size_t c1 = std::min(n_sel, c0 + tile);
        for (size_t f = 0; f < locals.size(); f++) {
            Fixed *h = out + offsets[f];
            u32 l = locals[f];
            if (b.width == 1) {
                const u8 *col = b.d8.data() + (size_t)l * b.n_rows;
                for (size_t i = c0; i < c1; i++) {
                    u32 r = rows[i];
                    u32 bin = col[r];
                    if (bin == missing) continue;
                    h[bin] = add(h[bin], gpair[r]);
                }
            } else {
                const u16 *col = b.d16.data() + (size_t)l * b.n_rows;
                for (size_t i = c0; i < c1; i++) {
                    u32 r = rows[i];
                    u32 bin = col[r];
                    if (bin == missing) continue;
                    h[bin] = add(h[bin], gpair[r]);
                }
            }
        }
    }
}

// ------------------------------------------------------------ colsample
// src/data/colsample.rs:3-73.
struct SplitMix64 {
    u64 s;
    u64 next() {
        s += 0x9E3779B97F4A7C15ull;
        u64 z = s;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    u64 below(u64 n) {
        u64 zone = UINT64_MAX - (UINT64_MAX % n) - 1;
        for (;;) {
            u64 v = next();
            if (v <= zone) return v % n;
        }
    }
};

inline u64 rotl(u64 x, int r) { return (x << r) | (x >> (64 - r)); }

size_t sampled_count(size_t nf, float rate) {
    if (nf == 0) return 0;
    double n = std::floor((double)rate * (double)nf);
    size_t k = (std::isfinite(n) && n >= 1.0) ? (size_t)n : 1;
    return std::max<size_t>(std::min(k, nf), 1);
}

std::vector<u32> sample_features(u32 nf, float rate, u64 seed, u64 round) {
    size_t take = sampled_count(nf, rate);
    std::vector<u32> ids(nf);
    for (u32 i = 0; i < nf; i++) ids[i] = i;
    if (take >= nf) return ids;
    SplitMix64 rng{seed ^ rotl(round * 0x9E3779B97F4A7C15ull, 17)};
    for (size_t i = ids.size() - 1; i >= 1; i--) {
        size_t j = (size_t)rng.below(i + 1);
        std::swap(ids[i], ids[j]);
    }
    ids.resize(take);
    std::sort(ids.begin(), ids.end());
    return ids;
}

// validated_weights (src/data/colsample.rs:119-141): NULL when absent or
// when every weight is equal (the uniform sampler then runs unchanged).
const float *validated_weights(const float *w, u32 nf) {
    if (!w) return nullptr;
    bool positive = false;
    for (u32 f = 0; f < nf; f++) {
        if (!std::isfinite(w[f]) || w[f] < 0.0f)
            throw std::runtime_error("feature_weights must be finite and nonnegative");
        positive = positive || w[f] > 0.0f;
    }
    if (!positive)
        throw std::runtime_error("feature_weights must contain at least one positive weight");
    for (u32 f = 1; f < nf; f++)
        if (w[f] != w[0]) return w;
    return nullptr;
}

// sample_subset (src/data/colsample.rs:101-116): max(1, floor(rate * |base|))
// of an ascending set by Fisher-Yates under `key`, ascending.
std::vector<u32> sample_subset(const std::vector<u32> &base, float rate, u64 key) {
    const size_t take = sampled_count(base.size(), rate);
    if (take >= base.size()) return base;
    std::vector<u32> ids = base;
    SplitMix64 rng{key};
    for (size_t i = ids.size() - 1; i >= 1; i--) {
        const size_t j = (size_t)rng.below(i + 1);
        std::swap(ids[i], ids[j]);
    }
    ids.resize(take);
    std::sort(ids.begin(), ids.end());
    return ids;
}

// sample_weighted (src/data/colsample.rs:146-172): weighted draws without
// replacement by exponential clocks, key -ln(U) / w with U from 52 random
// bits, the `take` smallest keys (ties to the lower id); zero weights are
// never drawn, except that rate >= 1 keeps the whole base.
std::vector<u32> sample_weighted(const std::vector<u32> &base, size_t n, float rate, u64 key,
                                 const float *w) {
    if (rate >= 1.0f) return base;
    std::vector<u32> positive;
    for (u32 id : base)
        if (w[id] > 0.0f) positive.push_back(id);
    const size_t take = std::min(sampled_count(n, rate), positive.size());
    if (take == positive.size()) return positive;
    SplitMix64 rng{key};
    std::vector<std::pair<double, u32>> keys;
    keys.reserve(positive.size());
    for (u32 id : positive) {
        const double u = (double)((rng.next() >> 12) + 1) / 4503599627370497.0;
        keys.push_back({-std::log(u) / (double)w[id], id});
    }
    std::sort(keys.begin(), keys.end());
    std::vector<u32> out;
    for (size_t i = 0; i < take; i++) out.push_back(keys[i].second);
    std::sort(out.begin(), out.end());
    return out;
}

// sample_features_weighted (src/data/colsample.rs:174-195).
std::vector<u32> sample_features_weighted(u32 nf, float rate, u64 seed, u64 round,
                                          const float *w) {
    if (!w) return sample_features(nf, rate, seed, round);
    std::vector<u32> all(nf);
    for (u32 i = 0; i < nf; i++) all[i] = i;
    return sample_weighted(all, nf, rate, seed ^ rotl(round * 0x9E3779B97F4A7C15ull, 17), w);
}

// subset_key (src/data/colsample.rs:197-201): (seed, tree, tag, idx) through
// one SplitMix64 step each.
u64 subset_key(u64 seed, u64 tree, u64 tag, u64 idx) {
    auto mix = [](u64 x) { return SplitMix64{x}.next(); };
    return mix(mix(mix(seed ^ (tag * 0xD6E8FEB86659FD93ull)) ^ tree) ^ idx);
}

// NestedSampler (src/data/colsample.rs:203-286): bytree -> bylevel ->
// bynode; the level set once per depth, the node set per tree node id; they
// restrict the split enumeration only.
struct Nested {
    const float *weights = nullptr;
    float bylevel = 1.0f, bynode = 1.0f;
    u64 seed = 0, tree = 0;
    std::vector<u32> level_set(const std::vector<u32> &tree_set, u32 depth) const {
        const u64 key = subset_key(seed, tree, 1, depth);
        return weights ? sample_weighted(tree_set, tree_set.size(), bylevel, key, weights)
                       : sample_subset(tree_set, bylevel, key);
    }
    bool samples_nodes() const { return bynode < 1.0f; }
    std::vector<u32> node_set(const std::vector<u32> &level, u64 node) const {
        const u64 key = subset_key(seed, tree, 2, node);
        return weights ? sample_weighted(level, level.size(), bynode, key, weights)
                       : sample_subset(level, bynode, key);
    }
};

// subsample (src/data/subsample.rs).
inline u64 mix64(u64 z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
u64 threshold_for(float rate) {
    if (rate >= 1.0f) return UINT64_MAX;
    if (!(rate > 0.0f)) return UINT64_MAX;
    return (u64)((double)rate * (double)(1ull << 53));
}
bool row_selected(u64 row, u64 th, u64 seed, u64 tree) {
    if (th == UINT64_MAX) return true;
    u64 h = mix64(seed ^ rotl(tree * 0x9E3779B97F4A7C15ull, 23) ^ (row * 0xD6E8FEB86659FD93ull));
    return (h >> 11) < th;
}

// ------------------------------------------------------------ objective
float sigmoidf(float m) { return 1.0f / (1.0f + std::exp(-m)); }

void gradient(u32 obj, float pred, float label, float &g, float &h) {
    if (obj == 1) {  // binary:logistic (objective.rs:511-517)
        float s = sigmoidf(pred);
        g = s - label;
        h = std::fmax(s * (1.0f - s), 1e-16f);
    } else {  // reg:squarederror
        g = pred - label;
        h = 1.0f;
    }
}

// Objective::softmax_gradients (src/training/objective.rs:1175-1219): from
// every class's margin of row i, the pair of class k. wmax starts at the
// smallest normal float (as XGBoost's gradient does), the sum of expf runs
// in double in class order, and the Hessian takes the sample weight before
// its floor.
void softmax_pair(const std::vector<std::vector<float>> &preds, u64 i, float label, float wt,
                  u32 k, float &g, float &h) {
    float wmax = std::numeric_limits<float>::min();
    for (const auto &col : preds) wmax = std::fmax(col[i], wmax);
    double wsum = 0.0;
    for (const auto &col : preds) wsum += (double)std::exp(col[i] - wmax);
    float p = std::exp(preds[k][i] - wmax) / (float)wsum;
    h = std::fmax(2.0f * p * (1.0f - p) * wt, 1e-16f);
    if (label == (float)k) p -= 1.0f;
    g = p * wt;
}

// Objective::initial_class_margins (src/training/objective.rs:1225-1248):
// centred logs of the class frequencies.
std::vector<float> initial_class_margins(const float *y, const float *w, u64 n, u32 k_count) {
    std::vector<float> bins(k_count, 0.0f);
    for (u64 i = 0; i < n; i++) bins[(u32)y[i]] += w ? w[i] : 1.0f;
    double sum_w = 0.0;
    if (!w) {
        sum_w = (double)n;
    } else {
        for (u64 i = 0; i < n; i++) sum_w += (double)w[i];
    }
    if (sum_w < (double)K_RT_EPS) return std::vector<float>(k_count, 0.0f);
    const double inv = 1.0 / sum_w;
    std::vector<float> logs(k_count);
    for (u32 c = 0; c < k_count; c++) logs[c] = std::log((float)((double)bins[c] * inv) + K_RT_EPS);
    const float nk = (float)k_count;
    float mean = 0.0f;
    for (float v : logs) mean = mean + v / nk;
    for (float &v : logs) v = v - mean;
    return logs;
}

// reg:quantileerror (src/training/objective.rs:1002-1160, XGBoost 3.4.1's
// QuantileRegression): a smoothed pinball loss with a majorise-minimise
// curvature. Each round takes one scale from every row's margin,
//   S = (sum w sqrtf|p - y| / sum w)^2
// (f32 terms, a serial double sum), then per row
//   x = (p - y) / (0.04 S), g = S/2 (tanh x + 1 - 2 alpha),
//   h = 0.5 / 0.04 max(tanh x / x, 3e-4) (1 at x = 0),
// both times the sample weight; S <= 0 gives (0, 0). tanh is the host libm's.
constexpr float QUANTILE_SMOOTHING_SCALE = 0.04f;     // objective.rs:31
constexpr float QUANTILE_MIN_SURROGATE_RATIO = 3.0e-4f;  // objective.rs:32

// Objective::quantile_scale (objective.rs:1115-1137).
float quantile_scale(const float *pred, const float *y, const float *w, u64 n) {
    double stat = 0.0, sum_w = 0.0;
    if (!w) {
        for (u64 i = 0; i < n; i++) stat += (double)std::sqrt(std::fabs(pred[i] - y[i]));
        sum_w = (double)n;
    } else {
        for (u64 i = 0; i < n; i++) {
            stat += (double)(w[i] * std::sqrt(std::fabs(pred[i] - y[i])));
            sum_w += (double)w[i];
        }
    }
    if (std::fabs(sum_w) < 1e-6) return 0.0f;
    const double root_mean = stat / sum_w;
    return (float)(root_mean * root_mean);
}

// Objective::quantile_gradient (objective.rs:1142-1160), unweighted.
void quantile_pair(float alpha, float scale, float pred, float label, float &g, float &h) {
    if (!(scale > 0.0f)) {
        g = h = 0.0f;
        return;
    }
    const float r = pred - label;
    const float x = r / (QUANTILE_SMOOTHING_SCALE * scale);
    const float t = std::tanh(x);
    float ratio = x == 0.0f ? 1.0f : t / x;
    ratio = std::fmax(ratio, QUANTILE_MIN_SURROGATE_RATIO);
    g = 0.5f * scale * (t + 1.0f - 2.0f * alpha);
    h = 0.5f / QUANTILE_SMOOTHING_SCALE * ratio;
}

// f32::total_cmp's order as an integer key.
int32_t total_key(float v) {
    int32_t b;
    std::memcpy(&b, &v, 4);
    return b ^ (int32_t)((uint32_t)(b >> 31) >> 1);
}

// quantile_intercepts (objective.rs:1039-1087), XGBoost's common::Quantile /
// WeightedQuantile: labels stably sorted once; unweighted, linear
// interpolation between order statistics at alpha (n + 1); weighted, the
// first label whose f32 running weight reaches alpha times the total.
std::vector<float> quantile_intercepts(const float *alphas, u32 k, const float *y, const float *w,
                                       u64 n) {
    if (n == 0) return std::vector<float>(k, 0.5f);
    std::vector<u64> idx(n);
    for (u64 i = 0; i < n; i++) idx[i] = i;
    std::stable_sort(idx.begin(), idx.end(),
                     [&](u64 a, u64 b) { return total_key(y[a]) < total_key(y[b]); });
    auto val = [&](u64 i) { return y[idx[i]]; };
    std::vector<float> cdf;
    if (w) {
        cdf.resize(n);
        cdf[0] = w[idx[0]];
        for (u64 i = 1; i < n; i++) cdf[i] = cdf[i - 1] + w[idx[i]];
    }
    std::vector<float> out(k);
    for (u32 j = 0; j < k; j++) {
        const double alpha = (double)alphas[j];
        if (!w) {
            const double nf = (double)n;
            if (alpha <= 1.0 / (nf + 1.0)) {
                out[j] = val(0);
                continue;
            }
            if (alpha >= nf / (nf + 1.0)) {
                out[j] = val(n - 1);
                continue;
            }
            const double x = alpha * (nf + 1.0);
            const double kk = std::floor(x) - 1.0;
            const double d = (x - 1.0) - kk;
            const float v0 = val((u64)kk), v1 = val((u64)kk + 1);
            out[j] = (float)((double)v0 + d * (double)(v1 - v0));
        } else {
            const float thresh = (float)((double)cdf[n - 1] * alpha);
            u64 at = (u64)(std::lower_bound(cdf.begin(), cdf.end(), thresh,
                                            [](float c, float t) { return c < t; }) -
                           cdf.begin());
            out[j] = val(std::min<u64>(at, n - 1));
        }
    }
    return out;
}

float base_margin_of(u32 obj, float bs) {  // objective.rs:363-398
    if (obj == 1) {
        float x = std::min(std::max(bs, K_RT_EPS), 1.0f - K_RT_EPS);
        return -std::log(1.0f / x - 1.0f);
    }
    return bs;
}

float estimate_base_score(const float *y, const float *w, u64 n) {  // objective.rs:42-60
    if (!w) {
        double nn = (double)n, acc = 0.0;
        for (u64 i = 0; i < n; i++) acc = acc + (double)y[i] / nn;
        return (float)acc;
    }
    double sw = 0.0;
    for (u64 i = 0; i < n; i++) sw = sw + (double)w[i];
    if (sw <= 0.0) return 0.5f;
    double acc = 0.0;
    for (u64 i = 0; i < n; i++) acc = acc + (double)y[i] / sw * (double)w[i];
    return (float)acc;
}

// ------------------------------------------------------------ tree
struct Node {
    u32 feat = 0;
    float split_cond = 0;
    int32_t left = -1, right = -1;
    bool default_left = false;
    float leaf_value = 0;
    bool is_leaf = true;
    float gain = 0;
    float sum_hess = 0;
    std::vector<u32> cats;  // u32 words, trailing zeros trimmed
    bool is_cat = false;
};

struct Tree {
    std::vector<Node> nodes;
    size_t push_leaf(float v, float h) {
        Node n;
        n.leaf_value = v;
        n.sum_hess = h;
        nodes.push_back(n);
        return nodes.size() - 1;
    }
    std::pair<size_t, size_t> split_leaf(size_t node, u32 feat, float cond, bool dl, float gain,
                                         float lv, float lh, float rv, float rh) {
        size_t l = push_leaf(lv, lh), r = push_leaf(rv, rh);
        Node &n = nodes[node];
        n.feat = feat;
        n.split_cond = cond;
        n.left = (int32_t)l;
        n.right = (int32_t)r;
        n.default_left = dl;
        n.leaf_value = 0.0f;
        n.is_leaf = false;
        n.gain = gain;
        return {l, r};
    }
    void set_categories(size_t node, const std::vector<u64> &bits) {
        std::vector<u32> words;
        for (size_t i = 0; i < 2 * bits.size(); i++) words.push_back((u32)(bits[i / 2] >> (32 * (i % 2))));
        while (!words.empty() && words.back() == 0) words.pop_back();
        nodes[node].cats = words;
        nodes[node].is_cat = true;
        float one;
        u32 bitsone = 1;
        std::memcpy(&one, &bitsone, 4);
        nodes[node].split_cond = one;
    }
    // Node::goes_left (tree.rs:90-101) + categorical::goes_left
    // (src/data/categorical.rs goes_left).
    static bool goes_left(const Node &n, float v) {
        if (std::isnan(v)) return n.default_left;
        if (n.is_cat) {
            if (v < 0.0f || v >= 16777216.0f) return true;
            u32 cat = (u32)v;
            u32 word = cat / 32;
            if (word >= n.cats.size()) return true;
            return ((n.cats[word] >> (cat % 32)) & 1) == 0;
        }
        return v < n.split_cond;
    }
    float leaf_value(const float *x) const {
        if (nodes.empty()) return 0.0f;
        size_t i = 0;
        for (;;) {
            const Node &n = nodes[i];
            if (n.is_leaf) return n.leaf_value;
            i = goes_left(n, x[n.feat]) ? (size_t)n.left : (size_t)n.right;
        }
    }
};

float split_threshold(const Cuts &c, u32 f, u32 bin) {  // tree.rs:991-1001
    if (bin == 0) return -std::numeric_limits<float>::max();
    if (bin > c.n_cuts(f)) return std::numeric_limits<float>::max();
    return c.cuts_for(f)[bin - 1];
}

}  // namespace

// ------------------------------------------------------------ model
struct orc_model {
    std::vector<Tree> trees;
    float base_score = 0.5f;
    u32 objective = 1;
    std::vector<float> class_margins;  // a multiclass model's intercepts (K)
    std::vector<float> quantile_alpha;  // reg:quantileerror's quantiles
    std::vector<float> train_margins;
    double train_seconds = 0.0;
};

namespace {

// ------------------------------------------------------------ training
struct Plan {
    u32 block;                 // physical block
    std::vector<u32> feats;    // sampled global features of the block (ascending)
    std::vector<u32> locals;   // their local column index in the block
    std::vector<u32> offsets;  // compact histogram offsets
};

struct Trainer {
    const Cuts &cuts;
    const std::vector<Block> &blocks;
    const Params &P;
    const orc_params &p;
    const Quantizer &q;
    const std::vector<Fixed> &gpair;
    std::vector<float> &pred;
    std::vector<Plan> plans;
    std::vector<u32> rows_cur, rows_next;
    const std::vector<u32> *sampled;
    unsigned nthread;
    // bylevel / bynode (mod.rs:3524-3528, 3582-3638): the sets start from
    // the tree's bytree set (every feature when it is not sampled).
    const Nested *nested = nullptr;
    std::vector<u32> tree_features;

    Trainer(const Cuts &c, const std::vector<Block> &b, const Params &P_, const Quantizer &q_,
            const std::vector<Fixed> &g, std::vector<float> &pr, const std::vector<u32> *smp,
            const Nested *nst = nullptr)
        : cuts(c), blocks(b), P(P_), p(P_.p), q(q_), gpair(g), pred(pr), sampled(smp),
          nested(nst) {
        nthread = std::max(1u, p.nthread);
        if (nested) {
            if (sampled) tree_features = *sampled;
            else
                for (u32 f = 0; f < cuts.n_feats(); f++) tree_features.push_back(f);
        }
        for (u32 bi = 0; bi < blocks.size(); bi++) {
            Plan pl;
            pl.block = bi;
            for (u32 l = 0; l < blocks[bi].feats.size(); l++) {
                u32 f = blocks[bi].feats[l];
                if (sampled && !std::binary_search(sampled->begin(), sampled->end(), f)) continue;
                pl.feats.push_back(f);
                pl.locals.push_back(l);
            }
            if (pl.feats.empty()) continue;
            pl.offsets.push_back(0);
            for (u32 f : pl.feats) pl.offsets.push_back(pl.offsets.back() + cuts.n_bins(f));
            plans.push_back(std::move(pl));
        }
    }

    SplitCtx ctx(Bounds b) const {
        SplitCtx sc;
        sc.q = &q;
        sc.p = &p;
        sc.given_weight = true;  // uses_given_weight() is always true (types.rs:637-639)
        sc.bounds = b;
        sc.params = &P;
        sc.mono = &P.monotone;
        return sc;
    }

    // Histogram of one node for every plan; hists[plan] sized offsets.back().
    void build_hists(const u32 *rows, size_t n, std::vector<std::vector<Fixed>> &out) {
        out.resize(plans.size());
        auto work = [&](size_t pi) {
            out[pi].assign(plans[pi].offsets.back(), Fixed());
            hist_rows(blocks[plans[pi].block], plans[pi].locals, plans[pi].offsets, gpair, rows, n,
                      out[pi].data());
        };
        if (nthread <= 1 || plans.size() <= 1) {
            for (size_t pi = 0; pi < plans.size(); pi++) work(pi);
        } else {
            std::vector<std::thread> th;
            for (unsigned t = 0; t < nthread; t++)
                th.emplace_back([&, t] {
                    for (size_t pi = t; pi < plans.size(); pi += nthread) work(pi);
                });
            for (auto &x : th) x.join();
        }
    }

    // The enumeration sets of a batch of nodes at one depth (node ids as in
    // the tree): the node set, else the level set, else the bytree set
    // (enum_features, mod.rs:3626-3638; lossguide.rs:85-101).
    std::vector<std::vector<u32>> enum_sets(u32 depth, const std::vector<size_t> &ids) const {
        std::vector<std::vector<u32>> out;
        if (!nested) return out;
        const std::vector<u32> level = nested->level_set(tree_features, depth);
        for (size_t id : ids)
            out.push_back(nested->samples_nodes() ? nested->node_set(level, id) : level);
        return out;
    }

    Cand best_of(const std::vector<std::vector<Fixed>> &h, Fixed sum, Bounds b,
                 const std::vector<u32> *enum_set = nullptr) {
        SplitCtx sc = ctx(b);
        Cand best;
        for (size_t pi = 0; pi < plans.size(); pi++) {
            Cand c = best_split_in_block(h[pi].data(), plans[pi].feats, plans[pi].offsets, sum, sc,
                                         enum_set ? enum_set : sampled, &cuts.cat);
            reduce_into(best, c);
        }
        return best;
    }

    // Stable partition of rows[start, start+len) into out (same span).
    size_t partition(const u32 *rows, size_t len, const Cand &c, u32 *out) {
        int width = cuts.width(c.feat);
        const Block *blk = nullptr;
        u32 local = 0;
        for (const Block &b : blocks)
            for (u32 l = 0; l < b.feats.size(); l++)
                if (b.feats[l] == c.feat) {
                    blk = &b;
                    local = l;
                }
        u32 missing = missing_of(width);
        size_t nl = 0;
        std::vector<u32> right;
        right.reserve(len);
        for (size_t i = 0; i < len; i++) {
            u32 r = rows[i];
            u32 bin = blk->bin(local, r);
            bool gl;
            if (bin == missing) gl = c.missing_left;
            else if (c.is_cat) {
                u32 w = bin >> 6;
                bool in = w < c.cats.size() && ((c.cats[w] >> (bin & 63)) & 1);
                gl = !in;
            } else gl = bin < c.bin;
            if (gl) out[nl++] = r;
            else right.push_back(r);
        }
        std::copy(right.begin(), right.end(), out + nl);
        return nl;
    }

    void child_leaves(const Cand &c, Bounds parent, float &lv, float &rv, Bounds &lb, Bounds &rb) {
        double g, h;
        q.to_f64(c.left, g, h);
        float wl = parent.apply(xgb_weight(g, h, p));
        q.to_f64(c.right, g, h);
        float wr = parent.apply(xgb_weight(g, h, p));
        parent.children(P.monotone_of(c.feat), wl, wr, lb, rb);
        lv = wl * p.learning_rate;
        rv = wr * p.learning_rate;
    }

    float hess_of(Fixed s) const {
        double g, h;
        q.to_f64(s, g, h);
        return (float)h;
    }

    void apply_split(Tree &t, size_t node, const Cand &c, Bounds parent, size_t &l, size_t &r,
                     Bounds &lb, Bounds &rb) {
        float lv, rv;
        child_leaves(c, parent, lv, rv, lb, rb);
        float thr = c.is_cat ? 0.0f : split_threshold(cuts, c.feat, c.bin);
        auto lr = t.split_leaf(node, c.feat, thr, c.missing_left, c.gain, lv, hess_of(c.left), rv,
                               hess_of(c.right));
        if (c.is_cat) t.set_categories(node, c.cats);
        l = lr.first;
        r = lr.second;
    }

    // Depthwise build_tree (src/training/mod.rs:3357-4565), CPU branch.
    Tree depthwise(Fixed root_sum) {
        Tree t;
        double g, h;
        q.to_f64(root_sum, g, h);
        size_t root = t.push_leaf(xgb_weight(g, h, p) * p.learning_rate, (float)h);
        u64 n = pred.size();
        rows_cur.resize(n);
        for (u64 i = 0; i < n; i++) rows_cur[i] = (u32)i;
        rows_next.assign(n, 0);
        struct LN {
            size_t node, start, len;
            Fixed sum;
            int parent = -1, sibling = -1;  // Subtract source
            Bounds bounds;
        };
        std::vector<LN> level{{root, 0, (size_t)n, root_sum, -1, -1, Bounds()}};
        std::vector<std::vector<std::vector<Fixed>>> parent_hists;
        u32 leaf_count = 1;
        for (u32 depth = 0; depth < p.max_depth; depth++) {
            if (level.empty() || (p.max_leaves != 0 && leaf_count >= p.max_leaves)) break;
            std::vector<std::vector<std::vector<Fixed>>> hists(level.size());
            for (size_t i = 0; i < level.size(); i++)
                if (level[i].parent < 0)
                    build_hists(rows_cur.data() + level[i].start, level[i].len, hists[i]);
            for (size_t i = 0; i < level.size(); i++) {
                if (level[i].parent < 0) continue;
                auto &ph = parent_hists[level[i].parent];
                hists[i] = ph;
                for (size_t pi = 0; pi < plans.size(); pi++)
                    for (size_t k = 0; k < hists[i][pi].size(); k++)
                        hists[i][pi][k] = sub(ph[pi][k], hists[level[i].sibling][pi][k]);
            }
            std::vector<size_t> ids;
            for (const LN &ln : level) ids.push_back(ln.node);
            const std::vector<std::vector<u32>> sets = enum_sets(depth, ids);
            std::vector<Cand> chosen(level.size());
            for (size_t i = 0; i < level.size(); i++)
                chosen[i] = best_of(hists[i], level[i].sum, level[i].bounds,
                                    sets.empty() ? nullptr : &sets[i]);
            if (p.max_leaves != 0) {
                u32 remaining = p.max_leaves > leaf_count ? p.max_leaves - leaf_count : 0;
                for (Cand &c : chosen)
                    if (c.found) {
                        if (remaining == 0) c.found = false;
                        else remaining--;
                    }
            }
            std::vector<LN> next;
            for (size_t i = 0; i < level.size(); i++) {
                const LN &ln = level[i];
                if (!chosen[i].found) {
                    float v = t.nodes[ln.node].leaf_value;
                    for (size_t k = 0; k < ln.len; k++) pred[rows_cur[ln.start + k]] += v;
                    continue;
                }
                size_t nl = partition(rows_cur.data() + ln.start, ln.len, chosen[i],
                                      rows_next.data() + ln.start);
                leaf_count++;
                size_t lnode, rnode;
                Bounds lb, rb;
                apply_split(t, ln.node, chosen[i], ln.bounds, lnode, rnode, lb, rb);
                size_t slot = next.size();
                LN L{lnode, ln.start, nl, chosen[i].left, -1, -1, lb};
                LN R{rnode, ln.start + nl, ln.len - nl, chosen[i].right, -1, -1, rb};
                bool left_small = L.len <= R.len;
                if (left_small) {
                    R.parent = (int)i;
                    R.sibling = (int)slot;
                } else {
                    L.parent = (int)i;
                    L.sibling = (int)slot + 1;
                }
                next.push_back(L);
                next.push_back(R);
            }
            parent_hists = std::move(hists);
            // Rows of nodes that did not split stay where they are; copy them.
            for (size_t i = 0; i < level.size(); i++)
                if (!chosen[i].found)
                    std::copy(rows_cur.begin() + level[i].start,
                              rows_cur.begin() + level[i].start + level[i].len,
                              rows_next.begin() + level[i].start);
            std::swap(rows_cur, rows_next);
            level = std::move(next);
        }
        for (const LN &ln : level) {
            float v = t.nodes[ln.node].leaf_value;
            for (size_t k = 0; k < ln.len; k++) pred[rows_cur[ln.start + k]] += v;
        }
        return t;
    }

    // Lossguide grow (src/training/lossguide.rs:494-700), CPU branch.
    Tree lossguide(Fixed root_sum) {
        Tree t;
        double g, h;
        q.to_f64(root_sum, g, h);
        size_t root = t.push_leaf(xgb_weight(g, h, p) * p.learning_rate, (float)h);
        u64 n = pred.size();
        rows_cur.resize(n);
        for (u64 i = 0; i < n; i++) rows_cur[i] = (u32)i;
        struct Leaf {
            size_t id, start, len;
            u32 depth;
            Fixed sum;
            Bounds bounds;
        };
        struct Pending {
            Leaf leaf;
            Cand split;
            std::shared_ptr<std::vector<std::vector<Fixed>>> hist;
        };
        auto less = [](const Pending &a, const Pending &b) {
            // BinaryHeap max by (gain, then lower leaf id first).
            if (a.split.gain != b.split.gain) return a.split.gain < b.split.gain;
            return a.leaf.id > b.leaf.id;
        };
        std::priority_queue<Pending, std::vector<Pending>, decltype(less)> heap(less);
        auto finish_leaf = [&](const Leaf &l) {
            float v = t.nodes[l.id].leaf_value;
            for (size_t k = 0; k < l.len; k++) pred[rows_cur[l.start + k]] += v;
        };
        auto evaluate = [&](std::vector<Leaf> leaves,
                            std::shared_ptr<std::vector<std::vector<Fixed>>> parent_hist) {
            std::vector<std::shared_ptr<std::vector<std::vector<Fixed>>>> hs(leaves.size());
            if (parent_hist && leaves.size() == 2) {
                size_t small = leaves[0].len > leaves[1].len ? 1 : 0;
                hs[small] = std::make_shared<std::vector<std::vector<Fixed>>>();
                build_hists(rows_cur.data() + leaves[small].start, leaves[small].len, *hs[small]);
                hs[1 - small] = std::make_shared<std::vector<std::vector<Fixed>>>(*parent_hist);
                auto &big = *hs[1 - small];
                for (size_t pi = 0; pi < plans.size(); pi++)
                    for (size_t k = 0; k < big[pi].size(); k++)
                        big[pi][k] = sub(big[pi][k], (*hs[small])[pi][k]);
            } else {
                for (size_t i = 0; i < leaves.size(); i++) {
                    hs[i] = std::make_shared<std::vector<std::vector<Fixed>>>();
                    build_hists(rows_cur.data() + leaves[i].start, leaves[i].len, *hs[i]);
                }
            }
            std::vector<size_t> ids;
            for (const Leaf &l : leaves) ids.push_back(l.id);
            const std::vector<std::vector<u32>> sets = enum_sets(leaves[0].depth, ids);
            for (size_t i = 0; i < leaves.size(); i++) {
                Cand c = best_of(*hs[i], leaves[i].sum, leaves[i].bounds,
                                 sets.empty() ? nullptr : &sets[i]);
                if (c.found) heap.push(Pending{leaves[i], c, hs[i]});
                else finish_leaf(leaves[i]);
            }
        };
        Leaf rootl{root, 0, (size_t)n, 0, root_sum, Bounds()};
        if (p.max_depth == 0 || p.max_leaves == 1) finish_leaf(rootl);
        else evaluate({rootl}, nullptr);
        u32 leaf_count = 1;
        std::vector<u32> buf;
        while (p.max_leaves == 0 || leaf_count < p.max_leaves) {
            if (heap.empty()) break;
            Pending ps = heap.top();
            heap.pop();
            buf.resize(ps.leaf.len);
            size_t nl = partition(rows_cur.data() + ps.leaf.start, ps.leaf.len, ps.split, buf.data());
            std::copy(buf.begin(), buf.end(), rows_cur.begin() + ps.leaf.start);
            size_t lnode, rnode;
            Bounds lb, rb;
            apply_split(t, ps.leaf.id, ps.split, ps.leaf.bounds, lnode, rnode, lb, rb);
            leaf_count++;
            u32 depth = ps.leaf.depth + 1;
            std::vector<Leaf> children{
                {lnode, ps.leaf.start, nl, depth, ps.split.left, lb},
                {rnode, ps.leaf.start + nl, ps.leaf.len - nl, depth, ps.split.right, rb}};
            if (depth == p.max_depth || leaf_count == p.max_leaves) {
                for (auto &c : children) finish_leaf(c);
            } else {
                evaluate(children, ps.hist);
            }
        }
        while (!heap.empty()) {
            finish_leaf(heap.top().leaf);
            heap.pop();
        }
        return t;
    }
};

// QuadratureTreeSHAP (src/model/explain.rs:116-401).
constexpr int POINTS = 8;
constexpr float UNSEEN = -999.0f;
struct Rule {
    float nodes[POINTS], weights[POINTS];
};

double legendre(int n, double x) {
    if (n == 0) return 1.0;
    double p0 = 1.0, p1 = x;
    for (int k = 2; k <= n; k++) {
        double kf = (double)k;
        double pk = ((2.0 * kf - 1.0) * x * p1 - (kf - 1.0) * p0) / kf;
        p0 = p1;
        p1 = pk;
    }
    return p1;
}

Rule make_rule() {
    Rule r;
    const int n = POINTS;
    for (int i = 0; i < n; i++) {
        double theta = M_PI * ((double)i + 0.75) / ((double)n + 0.5);
        double x = std::cos(theta);
        for (int it = 0; it < 64; it++) {
            double pn = legendre(n, x);
            double dpn = (double)n * (x * pn - legendre(n - 1, x)) / (x * x - 1.0);
            double dx = pn / dpn;
            x -= dx;
            if (std::fabs(dx) < 1e-15) break;
        }
        double pn = legendre(n, x);
        double dpn = (double)n * (x * pn - legendre(n - 1, x)) / (x * x - 1.0);
        double w = 2.0 / ((1.0 - x * x) * dpn * dpn);
        double s = 0.5 * (x + 1.0);
        double ws = 0.5 * w;
        int out = n - 1 - i;
        r.nodes[out] = (float)(s * s);
        r.weights[out] = (float)(2.0 * s * ws);
    }
    return r;
}

float branch_weight(float cover, float parent) {
    if (parent <= 0.0f) return 0.5f;
    float w = cover / parent;
    return w < 1e-12f ? 1e-12f : w;
}

float extract_delta(const Rule &r, const float *h, float pe, float px) {
    float acc = 0.0f;
    if (pe != 1.0f) {
        float a = pe - 1.0f;
        for (int i = 0; i < POINTS; i++) acc += a * h[i] / (1.0f + a * r.nodes[i]);
    }
    if (px != 1.0f) {
        float a = px - 1.0f;
        for (int i = 0; i < POINTS; i++) acc -= a * h[i] / (1.0f + a * r.nodes[i]);
    }
    return acc;
}

// extract_interaction_delta (src/model/explain.rs:219-247).
float extract_interaction_delta(const Rule &r, const float *h, float pe, float px, float q) {
    if (q == 1.0f) return 0.0f;
    const float ap = q - 1.0f, ae = pe - 1.0f;
    float acc = 0.0f;
    if (px == 1.0f) {
        for (int i = 0; i < POINTS; i++) {
            const float edge = ae / (1.0f + ae * r.nodes[i]);
            acc += ap * h[i] * edge / (1.0f + ap * r.nodes[i]);
        }
    } else {
        const float ax = px - 1.0f;
        for (int i = 0; i < POINTS; i++) {
            const float edge = ae / (1.0f + ae * r.nodes[i]) - ax / (1.0f + ax * r.nodes[i]);
            acc += ap * h[i] * edge / (1.0f + ap * r.nodes[i]);
        }
    }
    return acc;
}

// Runner (src/model/explain.rs:303-401) with the Additive formulation
// (matrix == nullptr: phi[feat] += delta) or the Interaction formulation
// (:267-301: diag[feat] += delta, partners on the live path into matrix).
struct ShapRunner {
    const std::vector<Node> &nodes;
    const float *feats;
    const Rule &rule;
    std::vector<float> &path_prob;
    std::vector<float> &phi;  // Additive: per-tree contributions; Interaction: diag
    float *matrix = nullptr;  // Interaction: [nc][nc]
    size_t ncols = 0;
    std::vector<std::pair<u32, float>> path;

    void on_return(u32 feat, const float *h, float pe, float px) {
        phi[feat] += extract_delta(rule, h, pe, px);
        if (!matrix) return;
        const size_t len = path.size();
        bool skipped_current = false;
        for (size_t i = len; i-- > 0;) {
            const u32 split = path[i].first;
            bool shadowed = false;
            for (size_t j = i + 1; j < len; j++)
                if (path[j].first == split) shadowed = true;
            if (shadowed) continue;
            if (!skipped_current && split == feat) {
                skipped_current = true;
                continue;
            }
            matrix[feat * ncols + split] +=
                extract_interaction_delta(rule, h, pe, px, path[i].second);
        }
    }
    void visit(size_t split, size_t child, float cw, bool sat, const float *c, float wprod,
               float *out_h) {
        u32 feat = nodes[split].feat;
        float p_old = path_prob[feat];
        float pe = sat ? (p_old == UNSEEN ? 1.0f / cw : p_old / cw) : 0.0f;
        float cc[POINTS];
        std::memcpy(cc, c, sizeof(cc));
        float ae = pe - 1.0f;
        for (int i = 0; i < POINTS; i++) cc[i] *= 1.0f + ae * rule.nodes[i];
        if (p_old != UNSEEN) {
            float ao = p_old - 1.0f;
            if (ao != 0.0f)
                for (int i = 0; i < POINTS; i++) cc[i] /= 1.0f + ao * rule.nodes[i];
        }
        path_prob[feat] = pe;
        path.emplace_back(feat, pe);
        run(child, cc, wprod * cw, out_h);
        float px = p_old == UNSEEN ? 1.0f : p_old;
        on_return(feat, out_h, pe, px);
        path.pop_back();
        path_prob[feat] = p_old;
    }
    void run(size_t idx, const float *c, float wprod, float *out_h) {
        const Node &n = nodes[idx];
        if (n.is_leaf) {
            float ls = wprod * n.leaf_value;
            for (int i = 0; i < POINTS; i++) out_h[i] = c[i] * ls * rule.weights[i];
            return;
        }
        size_t l = (size_t)n.left, r = (size_t)n.right;
        float lw = branch_weight(nodes[l].sum_hess, n.sum_hess);
        float rw = branch_weight(nodes[r].sum_hess, n.sum_hess);
        bool gl = Tree::goes_left(n, feats[n.feat]);
        float rh[POINTS] = {0};
        visit(idx, l, lw, gl, c, wprod, out_h);
        visit(idx, r, rw, !gl, c, wprod, rh);
        for (int i = 0; i < POINTS; i++) out_h[i] += rh[i];
    }
};

// fill_node_means (src/model/explain.rs:409-422): f32 cover-weighted means.
float fill_node_means(const std::vector<Node> &nodes, size_t idx, std::vector<float> &means) {
    const Node &n = nodes[idx];
    float value;
    if (n.is_leaf) {
        value = n.leaf_value;
    } else {
        const size_t l = (size_t)n.left, r = (size_t)n.right;
        float result = fill_node_means(nodes, l, means) * nodes[l].sum_hess;
        result += fill_node_means(nodes, r, means) * nodes[r].sum_hess;
        value = result / n.sum_hess;
    }
    means[idx] = value;
    return value;
}

double root_mean(const std::vector<Node> &nodes, size_t idx) {
    const Node &n = nodes[idx];
    if (n.is_leaf) return (double)n.leaf_value;
    size_t l = (size_t)n.left, r = (size_t)n.right;
    double lm = root_mean(nodes, l), rm = root_mean(nodes, r);
    if (n.sum_hess == 0.0f) return 0.5 * (lm + rm);
    return (lm * (double)nodes[l].sum_hess + rm * (double)nodes[r].sum_hess) / (double)n.sum_hess;
}

thread_local std::string g_error;

}  // namespace

// ======================================================================== C ABI
extern "C" {

int orc_quantizer_from_bounds(double mg, double mh, uint64_t n, double out[2]) {
    try {
        Quantizer q = Quantizer::from_bounds(mg, mh, n);
        out[0] = q.gs;
        out[1] = q.hs;
        return 0;
    } catch (std::exception &e) {
        g_error = e.what();
        return 1;
    }
}

void orc_quantize(const float *gp, uint64_t n, const double scale[2], int64_t *out,
                  int64_t sum[2]) {
    Quantizer q;
    q.gs = scale[0];
    q.hs = scale[1];
    Fixed s;
    for (u64 i = 0; i < n; i++) {
        Fixed f = q.to_fixed(gp[2 * i], gp[2 * i + 1]);
        out[2 * i] = f.g;
        out[2 * i + 1] = f.h;
        s = add(s, f);
    }
    sum[0] = s.g;
    sum[1] = s.h;
}

void orc_to_f64(const int64_t *fx, uint64_t n, const double scale[2], double *out) {
    Quantizer q;
    q.gi = 1.0 / scale[0];
    q.hi = 1.0 / scale[1];
    for (u64 i = 0; i < n; i++) q.to_f64({fx[2 * i], fx[2 * i + 1]}, out[2 * i], out[2 * i + 1]);
}

int orc_sketch_cuts(const float *x, uint64_t n, uint32_t nf, uint32_t max_bin, const float *w,
                    const uint8_t *cat, float *cv, uint32_t *co) {
    try {
        Cuts c = sketch_cuts(x, n, nf, max_bin, w, cat);
        std::copy(c.values.begin(), c.values.end(), cv);
        std::copy(c.offsets.begin(), c.offsets.end(), co);
        return 0;
    } catch (std::exception &e) {
        g_error = e.what();
        return 1;
    }
}

uint32_t orc_find_bin(const float *cv, const uint32_t *co, uint32_t f, uint8_t cat, float v) {
    Cuts c;
    c.values.assign(cv, cv + co[f + 1]);
    c.offsets.assign(co, co + f + 2);
    c.cat.assign(f + 1, 0);
    c.cat[f] = cat;
    int w = c.width(f);
    if (std::isnan(v)) return missing_of(w);
    return c.find_bin(f, v);
}

void orc_hist_build(const void *bins, uint32_t width, uint64_t n_rows, uint32_t n_feats,
                    const uint32_t *offsets, const int64_t *gp, const uint32_t *rows,
                    uint64_t n_sel, int64_t *out) {
    u32 missing = missing_of((int)width);
    Fixed *o = reinterpret_cast<Fixed *>(out);
    const Fixed *g = reinterpret_cast<const Fixed *>(gp);
    u64 n = rows ? n_sel : n_rows;
    for (u32 f = 0; f < n_feats; f++) {
        Fixed *h = o + offsets[f];
        for (u64 i = 0; i < n; i++) {
            u64 r = rows ? rows[i] : i;
            u32 b = width == 1 ? ((const u8 *)bins)[(u64)f * n_rows + r]
                               : ((const u16 *)bins)[(u64)f * n_rows + r];
            if (b == missing) continue;
            h[b] = add(h[b], g[r]);
        }
    }
}

void orc_node_sum(const int64_t *gp, const uint32_t *rows, uint64_t n_sel, uint64_t n_rows,
                  int64_t out[2]) {
    const Fixed *g = reinterpret_cast<const Fixed *>(gp);
    Fixed s;
    u64 n = rows ? n_sel : n_rows;
    for (u64 i = 0; i < n; i++) s = add(s, g[rows ? rows[i] : i]);
    out[0] = s.g;
    out[1] = s.h;
}

void orc_best_split(const int64_t *hist, uint32_t n_feats, const uint32_t *feat_ids,
                    const uint32_t *offsets, const int64_t node_sum[2], const double scale[2],
                    const orc_params *p, const uint32_t *sampled, uint32_t n_sampled,
                    uint32_t given_weight, float lo, float hi, const int8_t *monotone,
                    uint32_t n_monotone, const uint8_t *categorical, uint32_t n_categorical,
                    orc_split *out) {
    Quantizer q;
    q.gs = scale[0];
    q.hs = scale[1];
    q.gi = 1.0 / q.gs;
    q.hi = 1.0 / q.hs;
    std::vector<int8_t> mono(monotone, monotone + n_monotone);
    SplitCtx sc;
    sc.q = &q;
    sc.p = p;
    sc.given_weight = given_weight != 0;
    sc.bounds.lo = lo;
    sc.bounds.hi = hi;
    sc.params = nullptr;
    sc.mono = &mono;
    std::vector<u32> ids(feat_ids, feat_ids + n_feats);
    std::vector<u32> offs(offsets, offsets + n_feats + 1);
    std::vector<u32> smp;
    if (sampled) smp.assign(sampled, sampled + n_sampled);
    std::vector<u8> cat;
    if (categorical) cat.assign(categorical, categorical + n_categorical);
    Cand c = best_split_in_block(reinterpret_cast<const Fixed *>(hist), ids, offs,
                                 {node_sum[0], node_sum[1]}, sc, sampled ? &smp : nullptr,
                                 categorical ? &cat : nullptr);
    std::memset(out, 0, sizeof(*out));
    out->found = c.found;
    if (!c.found) return;
    out->feat = c.feat;
    out->bin = c.bin;
    out->gain = c.gain;
    out->left[0] = c.left.g;
    out->left[1] = c.left.h;
    out->right[0] = c.right.g;
    out->right[1] = c.right.h;
    out->missing_left = c.missing_left;
    out->n_cat_words = (u32)std::min<size_t>(c.cats.size(), 1024);
    for (u32 i = 0; i < out->n_cat_words; i++) out->cats[i] = c.cats[i];
}

uint64_t orc_partition(const uint32_t *rows, uint64_t n, const void *col, uint32_t width,
                       uint32_t split_bin, uint32_t missing_left, const uint64_t *cats,
                       uint32_t n_cat_words, uint32_t *out) {
    u32 missing = missing_of((int)width);
    u64 nl = 0;
    std::vector<u32> right;
    for (u64 i = 0; i < n; i++) {
        u32 r = rows[i];
        u32 b = width == 1 ? ((const u8 *)col)[r] : ((const u16 *)col)[r];
        bool gl;
        if (b == missing) gl = missing_left != 0;
        else if (cats) {
            u32 w = b >> 6;
            gl = !(w < n_cat_words && ((cats[w] >> (b & 63)) & 1));
        } else gl = b < split_bin;
        if (gl) out[nl++] = r;
        else right.push_back(r);
    }
    std::copy(right.begin(), right.end(), out + nl);
    return nl;
}

}  // extern "C"

namespace {

// train_multiclass_rounds (src/training/mod.rs:2578-2850): K margin columns
// from the class intercepts (base_score copied K times when given); each
// round takes every class's pairs from the round's starting margins
// (softmax_gradients), then grows one tree per class in class order, with
// row and column sampling keyed on the tree index round * K + class, each
// tree's leaves added to its own class's margins.
// Several quantile_alpha values (multi-target reg:quantileerror) run the same
// loop with one output per alpha: intercepts the labels' alpha quantiles
// (mod.rs:1442-1444), each target's pairs from its own column's scale
// (quantile_multi_gradients, mod.rs:2871-2890).
float rate_or_one(float r) { return r == 0.0f ? 1.0f : r; }
bool nested_active(const orc_params &p) {
    return rate_or_one(p.colsample_bylevel) < 1.0f || rate_or_one(p.colsample_bynode) < 1.0f;
}
Nested nested_of(const orc_params &p, u64 tree, const float *fw) {
    Nested n;
    n.weights = fw;
    n.bylevel = rate_or_one(p.colsample_bylevel);
    n.bynode = rate_or_one(p.colsample_bynode);
    n.seed = p.seed;
    n.tree = tree;
    return n;
}

// The checks of validate_params and validate_start_margins
// (src/training/mod.rs:1109-1130, 1550-1565) that the oracle meets.
void validate_inputs(const orc_params &p, u64 n, u32 k) {
    for (float r : {p.colsample_bylevel, p.colsample_bynode}) {
        const float v = rate_or_one(r);
        if (!(v > 0.0f && v <= 1.0f))
            throw std::runtime_error("colsample_bylevel / colsample_bynode must be in (0, 1]");
    }
    if (p.base_margin)
        for (u64 i = 0; i < n * k; i++)
            if (!std::isfinite(p.base_margin[i]))
                throw std::runtime_error("base_margin values must all be finite");
}

void train_multiclass(const float *x, u64 n, u32 nf, const float *labels, const float *weights,
                      const Params &P, const Cuts &cuts, const std::vector<Block> &blocks,
                      orc_model &m) {
    (void)x;
    const orc_params &p = P.p;
    const bool quantile = p.objective == 4;
    const u32 K = quantile ? p.n_quantile_alpha : p.num_class;
    if (!quantile) {
        if (K < 2) throw std::runtime_error("multiclass objectives require num_class >= 2");
        for (u64 i = 0; i < n; i++) {
            const float v = labels[i];
            if (!(v >= 0.0f && v < (float)K && v == std::trunc(v)))
                throw std::runtime_error("labels must be integers in [0, num_class)");
        }
    }
    m.class_margins = p.has_base_score ? std::vector<float>(K, p.base_score)
                      : quantile ? quantile_intercepts(p.quantile_alpha, K, labels, weights, n)
                                 : initial_class_margins(labels, weights, n, K);
    m.base_score = m.class_margins[0];
    std::vector<std::vector<float>> preds(K);
    for (u32 k = 0; k < K; k++) {
        // base_margin: class-major starting margins (mod.rs:2605-2616)
        if (p.base_margin) preds[k].assign(p.base_margin + (u64)k * n, p.base_margin + (u64)(k + 1) * n);
        else preds[k].assign(n, m.class_margins[k]);
    }
    const float *fw = validated_weights(p.feature_weights, nf);
    std::vector<std::vector<float>> gf(K, std::vector<float>(2 * n));
    std::vector<Fixed> gpair(n);
    auto t0 = std::chrono::steady_clock::now();
    const u64 th = threshold_for(p.subsample);
    for (u32 round = 0; round < p.n_rounds; round++) {
        if (quantile) {
            for (u32 k = 0; k < K; k++) {
                const float qs = quantile_scale(preds[k].data(), labels, weights, n);
                for (u64 i = 0; i < n; i++) {
                    float &g = gf[k][2 * i], &h = gf[k][2 * i + 1];
                    quantile_pair(p.quantile_alpha[k], qs, preds[k][i], labels[i], g, h);
                    if (weights) {
                        g = g * weights[i];
                        h = h * weights[i];
                    }
                }
            }
        } else {
            for (u64 i = 0; i < n; i++) {
                const float wt = weights ? weights[i] : 1.0f;
                for (u32 k = 0; k < K; k++)
                    softmax_pair(preds, i, labels[i], wt, k, gf[k][2 * i], gf[k][2 * i + 1]);
            }
        }
        for (u32 k = 0; k < K; k++) {
            const u64 tree = (u64)round * K + k;
            double mg = 0, mh = 0;
            for (u64 i = 0; i < n; i++) {
                float &g = gf[k][2 * i], &h = gf[k][2 * i + 1];
                if (!row_selected(i, th, p.seed, tree)) g = h = 0.0f;
                mg = std::fmax(mg, finite_abs(g));
                mh = std::fmax(mh, finite_abs(h));
            }
            Quantizer q = Quantizer::from_bounds(mg, mh, n);
            Fixed root;
            for (u64 i = 0; i < n; i++) {
                gpair[i] = q.to_fixed(gf[k][2 * i], gf[k][2 * i + 1]);
                root = add(root, gpair[i]);
            }
            std::vector<u32> smp;
            const bool use_smp = p.colsample_bytree < 1.0f;
            if (use_smp) smp = sample_features_weighted(nf, p.colsample_bytree, p.seed, tree, fw);
            const Nested nst = nested_of(p, tree, fw);
            Trainer tr(cuts, blocks, P, q, gpair, preds[k], use_smp ? &smp : nullptr,
                       nested_active(p) ? &nst : nullptr);
            m.trees.push_back(p.grow_policy == 1 ? tr.lossguide(root) : tr.depthwise(root));
        }
    }
    m.train_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    m.train_margins.clear();
    for (u32 k = 0; k < K; k++) m.train_margins.insert(m.train_margins.end(), preds[k].begin(), preds[k].end());
}

}  // namespace

extern "C" {

int orc_train(const float *x, uint64_t n, uint32_t nf, const float *labels, const float *weights,
              const uint8_t *categorical, const int8_t *monotone, uint32_t n_monotone,
              const orc_params *pp, orc_model **out) {
    try {
        Params P;
        P.p = *pp;
        if (monotone) P.monotone.assign(monotone, monotone + n_monotone);
        const orc_params &p = P.p;
        if (n == 0 || nf == 0) throw std::runtime_error("training data must be non-empty");
        if (p.max_depth > 14) throw std::runtime_error("max_depth must be in 0..=14");
        Cuts cuts = sketch_cuts(x, n, nf, p.max_bin, weights, categorical);
        std::vector<Block> blocks = bin_blocks(x, n, nf, cuts, p.cols_per_block);
        auto m = std::make_unique<orc_model>();
        m->objective = p.objective;
        const bool quantile = p.objective == 4;
        if (quantile) {
            // Objective::validate_params (objective.rs:317-330).
            if (p.n_quantile_alpha == 0 || !p.quantile_alpha)
                throw std::runtime_error("reg:quantileerror requires quantile_alpha");
            for (u32 k = 0; k < p.n_quantile_alpha; k++) {
                const float a = p.quantile_alpha[k];
                if (!(a >= 0.0f && a <= 1.0f))
                    throw std::runtime_error("quantile_alpha must be in [0, 1]");
                if (k && p.quantile_alpha[k - 1] > a)
                    throw std::runtime_error("quantile_alpha must be in ascending order");
            }
            m->quantile_alpha.assign(p.quantile_alpha, p.quantile_alpha + p.n_quantile_alpha);
        }
        validate_inputs(p, n,
                        p.objective == 2 || p.objective == 3 ? p.num_class
                        : quantile                           ? std::max(1u, p.n_quantile_alpha)
                                                             : 1u);
        validated_weights(p.feature_weights, nf);
        if (p.objective == 2 || p.objective == 3 || (quantile && p.n_quantile_alpha > 1)) {
            train_multiclass(x, n, nf, labels, weights, P, cuts, blocks, *m);
            *out = m.release();
            return 0;
        }
        m->base_score = p.has_base_score ? p.base_score
                        : quantile ? quantile_intercepts(p.quantile_alpha, 1, labels, weights, n)[0]
                                   : estimate_base_score(labels, weights, n);
        float margin = base_margin_of(p.objective, m->base_score);
        std::vector<float> pred(n, margin);
        if (p.base_margin) pred.assign(p.base_margin, p.base_margin + n);  // mod.rs:1831-1834
        const float *fw = validated_weights(p.feature_weights, nf);
        std::vector<Fixed> gpair(n);
        std::vector<float> gf(2 * n);
        // gradient_weights (src/training/mod.rs:5466-5490): scale_pos_weight
        // multiplies the sample weight (1 when absent) of rows labelled 1;
        // logistic and squared error both use it (objective.rs:346-356).
        std::vector<float> spw_w;
        const float *gw = weights;
        if (p.scale_pos_weight != 1.0f && !quantile) {
            spw_w.resize(n);
            for (u64 i = 0; i < n; i++) {
                const float w = weights ? weights[i] : 1.0f;
                spw_w[i] = labels[i] == 1.0f ? w * p.scale_pos_weight : w;
            }
            gw = spw_w.data();
        }
        auto t0 = std::chrono::steady_clock::now();
        for (u32 round = 0; round < p.n_rounds; round++) {
            double mg = 0, mh = 0;
            u64 th = threshold_for(p.subsample);
            const float qs = quantile ? quantile_scale(pred.data(), labels, weights, n) : 0.0f;
            for (u64 i = 0; i < n; i++) {
                float g, h;
                if (quantile)
                    quantile_pair(p.quantile_alpha[0], qs, pred[i], labels[i], g, h);
                else
                    gradient(p.objective, pred[i], labels[i], g, h);
                if (gw) {
                    g = g * gw[i];
                    h = h * gw[i];
                }
                if (!row_selected(i, th, p.seed, round)) g = h = 0.0f;
                gf[2 * i] = g;
                gf[2 * i + 1] = h;
                mg = std::fmax(mg, finite_abs(g));
                mh = std::fmax(mh, finite_abs(h));
            }
            Quantizer q = Quantizer::from_bounds(mg, mh, n);
            Fixed root;
            for (u64 i = 0; i < n; i++) {
                gpair[i] = q.to_fixed(gf[2 * i], gf[2 * i + 1]);
                root = add(root, gpair[i]);
            }
            std::vector<u32> smp;
            bool use_smp = p.colsample_bytree < 1.0f;
            if (use_smp) smp = sample_features_weighted(nf, p.colsample_bytree, p.seed, round, fw);
            const Nested nst = nested_of(p, round, fw);
            Trainer tr(cuts, blocks, P, q, gpair, pred, use_smp ? &smp : nullptr,
                       nested_active(p) ? &nst : nullptr);
            m->trees.push_back(p.grow_policy == 1 ? tr.lossguide(root) : tr.depthwise(root));
        }
        m->train_seconds =
            std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        m->train_margins = std::move(pred);
        *out = m.release();
        return 0;
    } catch (std::exception &e) {
        g_error = e.what();
        return 1;
    }
}

void orc_model_free(orc_model *m) { delete m; }
uint32_t orc_model_n_trees(const orc_model *m) { return (u32)m->trees.size(); }
uint32_t orc_model_tree_len(const orc_model *m, uint32_t t) { return (u32)m->trees[t].nodes.size(); }

void orc_model_tree_nodes(const orc_model *m, uint32_t t, orc_node *out) {
    u32 cat_base = 0;
    for (u32 k = 0; k < t; k++)
        for (const Node &n : m->trees[k].nodes) cat_base += (u32)n.cats.size();
    for (size_t i = 0; i < m->trees[t].nodes.size(); i++) {
        const Node &n = m->trees[t].nodes[i];
        orc_node o;
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
        o.cat_begin = cat_base;
        o.cat_len = (u32)n.cats.size();
        cat_base += o.cat_len;
        out[i] = o;
    }
}

uint32_t orc_model_n_cat_words(const orc_model *m) {
    u32 s = 0;
    for (const Tree &t : m->trees)
        for (const Node &n : t.nodes) s += (u32)n.cats.size();
    return s;
}

void orc_model_cat_words(const orc_model *m, uint32_t *out) {
    for (const Tree &t : m->trees)
        for (const Node &n : t.nodes)
            for (u32 w : n.cats) *out++ = w;
}

float orc_model_base_score(const orc_model *m) { return m->base_score; }
float orc_model_base_margin(const orc_model *m) { return base_margin_of(m->objective, m->base_score); }
double orc_model_train_seconds(const orc_model *m) { return m->train_seconds; }

uint32_t orc_model_num_outputs(const orc_model *m) {
    return m->class_margins.empty() ? 1u : (u32)m->class_margins.size();
}

void orc_model_class_margins(const orc_model *m, float *out) {
    std::copy(m->class_margins.begin(), m->class_margins.end(), out);
}

void orc_predict_margin(const orc_model *m, const float *x, uint64_t n, uint32_t nf, float *out) {
    if (!m->class_margins.empty()) {  // Model::predict_margins_upto (src/model/tree.rs:470-480)
        const u32 K = (u32)m->class_margins.size();
        for (u64 r = 0; r < n; r++) {
            float *o = out + r * K;
            for (u32 k = 0; k < K; k++) o[k] = m->class_margins[k];
            for (size_t t = 0; t < m->trees.size(); t++) o[t % K] += m->trees[t].leaf_value(x + r * nf);
        }
        return;
    }
    float bm = base_margin_of(m->objective, m->base_score);
    for (u64 r = 0; r < n; r++) {
        float acc = bm;
        for (const Tree &t : m->trees) acc += t.leaf_value(x + r * nf);
        out[r] = acc;
    }
}

void orc_model_train_margins(const orc_model *m, float *out) {
    std::copy(m->train_margins.begin(), m->train_margins.end(), out);
}

void orc_quadrature_rule(float nodes[8], float weights[8]) {
    Rule r = make_rule();
    std::memcpy(nodes, r.nodes, sizeof(r.nodes));
    std::memcpy(weights, r.weights, sizeof(r.weights));
}

// Explainer::shap_row (src/model/explain.rs:704-728), single output group.
int orc_model_from_nodes(const orc_node *nodes, const uint32_t *offs, uint32_t n_trees,
                         const uint32_t *cat_words, uint32_t n_cat_words, uint32_t objective,
                         float base_score, orc_model **out) {
    try {
        auto m = std::make_unique<orc_model>();
        m->objective = objective;
        m->base_score = base_score;
        for (u32 t = 0; t < n_trees; t++) {
            Tree tr;
            for (u32 i = offs[t]; i < offs[t + 1]; i++) {
                const orc_node &o = nodes[i];
                Node n;
                n.feat = o.feat;
                n.split_cond = o.split_cond;
                n.left = o.left;
                n.right = o.right;
                n.default_left = o.default_left != 0;
                n.is_leaf = o.is_leaf != 0;
                n.leaf_value = o.leaf_value;
                n.gain = o.gain;
                n.sum_hess = o.sum_hess;
                if (o.cat_len) {
                    if ((u64)o.cat_begin + o.cat_len > n_cat_words)
                        throw std::runtime_error("category words out of range");
                    n.cats.assign(cat_words + o.cat_begin, cat_words + o.cat_begin + o.cat_len);
                    n.is_cat = true;
                }
                tr.nodes.push_back(n);
            }
            m->trees.push_back(std::move(tr));
        }
        *out = m.release();
        return 0;
    } catch (std::exception &e) {
        g_error = e.what();
        return 1;
    }
}

int orc_shap(const orc_model *m, const float *x, uint64_t n, uint32_t nf, float *out) {
    return orc_explain(m, 0, x, n, nf, nullptr, out);
}

// Explainer::compute_with_margin (src/model/explain.rs:612-811) for one
// output group: kind 0 shap_row, 1 saabas_row, 2 interaction_row, 3 leaf_row.
int orc_explain(const orc_model *m, uint32_t kind, const float *x, uint64_t n, uint32_t nf,
                const float *margin, float *out) {
    Rule rule = make_rule();
    double sum = 0.0;
    std::vector<std::vector<float>> means;
    for (const Tree &t : m->trees) {
        if (t.nodes.empty()) {
            g_error = "tree has no nodes";
            return 1;
        }
        if (kind == 1) {
            means.emplace_back(t.nodes.size(), 0.0f);
            fill_node_means(t.nodes, 0, means.back());
        }
        sum += root_mean(t.nodes, 0);
    }
    const float root_mean_f = (float)sum;
    const float base = base_margin_of(m->objective, m->base_score);
    const size_t nc = (size_t)nf + 1;
    std::vector<float> path_prob(nf, UNSEEN), contribs(nc), diag(nc);
    for (u64 r = 0; r < n; r++) {
        const float *feats = x + r * nf;
        const float bias = margin ? margin[r] : base;
        if (kind == 3) {  // leaf_row
            float *o = out + r * m->trees.size();
            for (size_t t = 0; t < m->trees.size(); t++) {
                const auto &nodes = m->trees[t].nodes;
                size_t i = 0;
                while (!nodes[i].is_leaf)
                    i = (size_t)(Tree::goes_left(nodes[i], feats[nodes[i].feat]) ? nodes[i].left
                                                                                 : nodes[i].right);
                o[t] = (float)i;
            }
            continue;
        }
        if (kind == 2) {  // interaction_row
            float *mat = out + r * nc * nc;
            std::fill(mat, mat + nc * nc, 0.0f);
            std::fill(diag.begin(), diag.end(), 0.0f);
            for (const Tree &t : m->trees) {
                if (t.nodes[0].is_leaf) continue;
                ShapRunner runner{t.nodes, feats, rule, path_prob, diag, mat, nc, {}};
                float ones[POINTS], h[POINTS] = {0};
                for (int i = 0; i < POINTS; i++) ones[i] = 1.0f;
                runner.run(0, ones, 1.0f, h);
            }
            diag[nc - 1] += root_mean_f;
            diag[nc - 1] += bias;
            for (size_t a = 0; a < nc; a++)
                for (size_t b = a + 1; b < nc; b++) {
                    const float sym = 0.5f * (mat[a * nc + b] + mat[b * nc + a]);
                    mat[a * nc + b] = sym;
                    mat[b * nc + a] = sym;
                }
            for (size_t a = 0; a < nc; a++) {
                float value = diag[a];
                for (size_t b = 0; b < nc; b++)
                    if (b != a) value -= mat[a * nc + b];
                mat[a * nc + a] = value;
            }
            continue;
        }
        float *p = out + r * nc;
        std::fill(p, p + nc, 0.0f);
        for (size_t ti = 0; ti < m->trees.size(); ti++) {
            const Tree &t = m->trees[ti];
            std::fill(contribs.begin(), contribs.end(), 0.0f);
            if (kind == 1) {  // saabas_row
                const auto &nodes = t.nodes;
                const auto &mn = means[ti];
                float node_value = mn[0];
                contribs[nc - 1] += node_value;
                if (!nodes[0].is_leaf) {
                    size_t idx = 0, split = 0;
                    while (!nodes[idx].is_leaf) {
                        split = nodes[idx].feat;
                        idx = (size_t)(Tree::goes_left(nodes[idx], feats[split]) ? nodes[idx].left
                                                                                 : nodes[idx].right);
                        const float nv = mn[idx];
                        contribs[split] += nv - node_value;
                        node_value = nv;
                    }
                    contribs[split] += nodes[idx].leaf_value - node_value;
                }
                for (size_t c = 0; c < nc; c++) p[c] += contribs[c];
                continue;
            }
            if (!t.nodes[0].is_leaf) {
                ShapRunner runner{t.nodes, feats, rule, path_prob, contribs, nullptr, 0, {}};
                float ones[POINTS], h[POINTS] = {0};
                for (int i = 0; i < POINTS; i++) ones[i] = 1.0f;
                runner.run(0, ones, 1.0f, h);
            }
            for (u32 c = 0; c < nf; c++) p[c] += contribs[c];
        }
        if (kind == 0) p[nf] += root_mean_f;
        p[nf] += bias;
    }
    return 0;
}

uint32_t orc_sample_features(uint32_t nf, float rate, uint64_t seed, uint64_t round,
                             uint32_t *out) {
    std::vector<u32> s = sample_features(nf, rate, seed, round);
    std::copy(s.begin(), s.end(), out);
    return (u32)s.size();
}

uint64_t orc_compress_clamps() { return g_compress_clamps.load(); }

uint64_t orc_sketch_summary(const float *col, uint64_t n, const float *w, uint32_t max_bin,
                            float *out, uint64_t capacity) {
    FeatureSketch sk(max_bin, false);
    for (uint64_t i = 0; i < n; i++) sk.push(col[i], w ? w[i] : 1.0f);
    const std::vector<Entry> e = sk.collapse();
    for (uint64_t i = 0; i < std::min<uint64_t>(e.size(), capacity); i++) {
        out[4 * i] = e[i].value;
        out[4 * i + 1] = e[i].weight;
        out[4 * i + 2] = e[i].rmin;
        out[4 * i + 3] = e[i].rmax;
    }
    return e.size();
}

int orc_validated_weights(const float *w, uint32_t nf) {
    try {
        return validated_weights(w, nf) ? 1 : 0;
    } catch (std::exception &e) {
        g_error = e.what();
        return -1;
    }
}

uint32_t orc_sample_features_weighted(uint32_t nf, float rate, uint64_t seed, uint64_t round,
                                      const float *w, uint32_t *out) {
    std::vector<u32> s = sample_features_weighted(nf, rate, seed, round, w);
    std::copy(s.begin(), s.end(), out);
    return (u32)s.size();
}

uint32_t orc_nested_set(const uint32_t *base, uint32_t n, float bylevel, float bynode,
                        uint64_t seed, uint64_t tree, uint32_t tag, uint64_t idx,
                        const float *w, uint32_t *out) {
    Nested ns;
    ns.weights = w;
    ns.bylevel = bylevel;
    ns.bynode = bynode;
    ns.seed = seed;
    ns.tree = tree;
    const std::vector<u32> b(base, base + n);
    const std::vector<u32> s = tag == 1 ? ns.level_set(b, (u32)idx) : ns.node_set(b, idx);
    std::copy(s.begin(), s.end(), out);
    return (u32)s.size();
}

uint64_t orc_subset_key(uint64_t seed, uint64_t tree, uint64_t tag, uint64_t idx) {
    return subset_key(seed, tree, tag, idx);
}

void orc_sigmoid(const float *in, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; i++) out[i] = sigmoidf(in[i]);
}

}  // extern "C"

namespace {

template <class F>
uint64_t function_checksum(uint64_t begin, uint64_t end, uint32_t threads, F fn) {
    if (threads == 0) threads = 1;
    std::vector<u64> part(threads, 0);
    std::vector<std::thread> pool;
    for (u32 t = 0; t < threads; t++)
        pool.emplace_back([&, t] {
            u64 acc = 0;
            for (u64 u = begin + t; u < end; u += threads) {
                const u32 b = (u32)u;
                float x;
                std::memcpy(&x, &b, 4);
                const float s = fn(x);
                u32 sb;
                std::memcpy(&sb, &s, 4);
                if (s != s) sb = 0x7fc00000u;
                acc += mix64(u ^ ((u64)sb << 32));
            }
            part[t] = acc;
        });
    for (auto &th : pool) th.join();
    u64 acc = 0;
    for (u64 v : part) acc += v;
    return acc;
}

}  // namespace

extern "C" {

uint64_t orc_tanh_checksum(uint64_t begin, uint64_t end, uint32_t threads) {
    return function_checksum(begin, end, threads, [](float x) { return std::tanh(x); });
}

uint64_t orc_sigmoid_checksum(uint64_t begin, uint64_t end, uint32_t threads) {
    if (threads == 0) threads = 1;
    std::vector<u64> part(threads, 0);
    std::vector<std::thread> pool;
    for (u32 t = 0; t < threads; t++)
        pool.emplace_back([&, t] {
            u64 acc = 0;
            for (u64 u = begin + t; u < end; u += threads) {
                const u32 b = (u32)u;
                float x;
                std::memcpy(&x, &b, 4);
                const float s = sigmoidf(x);
                u32 sb;
                std::memcpy(&sb, &s, 4);
                if (s != s) sb = 0x7fc00000u;
                acc += mix64(u ^ ((u64)sb << 32));
            }
            part[t] = acc;
        });
    for (auto &th : pool) th.join();
    u64 acc = 0;
    for (u64 v : part) acc += v;
    return acc;
}

void orc_splitmix64(uint64_t seed, uint64_t n, uint64_t *out) {
    SplitMix64 r{seed};
    for (uint64_t i = 0; i < n; i++) out[i] = r.next();
}

uint64_t orc_mix64(uint64_t z) { return mix64(z); }

uint64_t orc_row_hash(uint64_t row, uint64_t seed, uint64_t tree) {
    return mix64(seed ^ rotl(tree * 0x9E3779B97F4A7C15ull, 23) ^ (row * 0xD6E8FEB86659FD93ull));
}

uint64_t orc_threshold_for(float rate) { return threshold_for(rate); }

int orc_row_selected(uint64_t row, uint64_t th, uint64_t seed, uint64_t tree) {
    return row_selected(row, th, seed, tree) ? 1 : 0;
}

void orc_gradients(const float *pred, const float *labels, const float *w, uint64_t n, uint32_t obj,
                   float *out) {
    for (u64 i = 0; i < n; i++) {
        float g, h;
        gradient(obj, pred[i], labels[i], g, h);
        if (w) {
            g *= w[i];
            h *= w[i];
        }
        out[2 * i] = g;
        out[2 * i + 1] = h;
    }
}

void orc_softmax_pairs(const float *margins, const float *labels, const float *w, uint64_t n,
                       uint32_t k_count, uint32_t k, float *out) {
    std::vector<std::vector<float>> preds(k_count);
    for (u32 c = 0; c < k_count; c++) preds[c].assign(margins + (u64)c * n, margins + (u64)(c + 1) * n);
    for (u64 i = 0; i < n; i++)
        softmax_pair(preds, i, labels[i], w ? w[i] : 1.0f, k, out[2 * i], out[2 * i + 1]);
}

float orc_base_margin(uint32_t obj, float bs) { return base_margin_of(obj, bs); }

float orc_quantile_scale(const float *pred, const float *labels, const float *w, uint64_t n) {
    return quantile_scale(pred, labels, w, n);
}

void orc_quantile_pairs(const float *pred, const float *labels, const float *w, uint64_t n,
                        float alpha, float scale, float *out) {
    for (u64 i = 0; i < n; i++) {
        float g, h;
        quantile_pair(alpha, scale, pred[i], labels[i], g, h);
        if (w) {
            g *= w[i];
            h *= w[i];
        }
        out[2 * i] = g;
        out[2 * i + 1] = h;
    }
}

void orc_quantile_intercepts(const float *labels, const float *w, uint64_t n, const float *alphas,
                             uint32_t k, float *out) {
    const std::vector<float> v = quantile_intercepts(alphas, k, labels, w, n);
    std::copy(v.begin(), v.end(), out);
}
float orc_estimate_base_score(const float *y, const float *w, uint64_t n) {
    return estimate_base_score(y, w, n);
}

const char *orc_last_error() { return g_error.c_str(); }

}  // extern "C"
