// fbt_data.cpp -- data preparation of the device path: the weighted quantile
// sketch and cuts (src/data/sketch.rs), binning (src/data/columns.rs:335-356,
// src/data/categorical.rs code_to_bin) and the width-homogeneous column
// blocks (src/data/columns.rs:446-463), as DenseSource builds them
// (src/source/dense.rs:99-290): one sketch per feature, fed row by row, no
// merging across threads, so the cuts never depend on the thread count.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <thread>

#include "../../include/fbhip.h"

#include "fbt_internal.h"

namespace fbt {
namespace {

// A summary entry: value with the rank interval [rmin, rmax] of its weight.
struct Rank {
    float value, weight, rmin, rmax;
    float mid() const { return 0.5f * (rmin + rmax); }
};
using Summary = std::vector<Rank>;

// Sorted summary of a batch; equal values merge (build_summary).
Summary summarize(std::vector<std::pair<float, float>> &batch) {
    std::sort(batch.begin(), batch.end(),
              [](const std::pair<float, float> &a, const std::pair<float, float> &b) {
                  return a.first < b.first;
              });
    Summary s;
    s.reserve(batch.size());
    float run = 0.0f;
    for (size_t i = 0; i < batch.size();) {
        const float v = batch[i].first;
        float w = 0.0f;
        for (; i < batch.size() && batch[i].first == v; i++) w += batch[i].second;
        s.push_back({v, w, run, run + w});
        run += w;
    }
    return s;
}

// Merge two summaries; a value's rank bounds grow by the weight of the other
// summary already passed (merge_entries + dedup_same_value).
Summary merge(const Summary &a, const Summary &b) {
    if (a.empty()) return b;
    if (b.empty()) return a;
    Summary m;
    m.reserve(a.size() + b.size());
    size_t i = 0, j = 0;
    float passed_a = 0.0f, passed_b = 0.0f;
    while (i < a.size() || j < b.size()) {
        const bool from_a = j >= b.size() || (i < a.size() && a[i].value <= b[j].value);
        if (from_a) {
            const Rank &e = a[i++];
            m.push_back({e.value, e.weight, e.rmin + passed_b, e.rmax + passed_b});
            passed_a = e.rmax;
        } else {
            const Rank &e = b[j++];
            m.push_back({e.value, e.weight, e.rmin + passed_a, e.rmax + passed_a});
            passed_b = e.rmax;
        }
    }
    Summary out;
    out.reserve(m.size());
    for (const Rank &e : m) {
        if (!out.empty() && out.back().value == e.value) {
            Rank &l = out.back();
            l.weight += e.weight;
            l.rmin = std::min(l.rmin, e.rmin);
            l.rmax = std::max(l.rmax, e.rmax);
        } else {
            out.push_back(e);
        }
    }
    return out;
}

// Keep `cap` entries at evenly spaced target ranks, first and last kept
// (compress).
Summary prune(const Summary &s, size_t cap) {
    const size_t n = s.size();
    if (n <= cap) return s;
    const float total = s[n - 1].rmax;
    const size_t slots = cap - 1;
    Summary out;
    out.reserve(cap);
    out.push_back(s[0]);
    size_t last = 0;
    for (size_t k = 1; k < slots; k++) {
        const float target = total * (float)k / (float)slots;
        size_t j = last + 1;
        while (j < n - 1 && s[j].mid() < target) j++;
        const size_t ceiling = n - 1 - (slots - 1 - k);
        j = std::min(std::max(j, last + 1), ceiling);
        if (j > last) {
            out.push_back(s[j]);
            last = j;
        }
    }
    if (last < n - 1) out.push_back(s[n - 1]);
    return out;
}

float cut_between(float a, float b) {  // midpoint (sketch.rs:290-302)
    const float d = b - a;
    const float m = std::isfinite(d) ? a + d * 0.5f : a * 0.5f + b * 0.5f;
    return m <= a ? b : m;
}

// Log-structured sketch of one numeric feature: summaries are compressed only
// when two of the same level merge (FeatureSketch).
class FeatureQuantiles {
  public:
    explicit FeatureQuantiles(size_t max_bins)
        : cap_(std::max<size_t>(max_bins * 16, 32)) {
        pending_.reserve(cap_);
    }
    void add(float v, float w) {
        if (std::isnan(v) || w <= 0.0f) return;
        pending_.push_back({v, w});
        if (pending_.size() >= cap_) flush();
    }
    std::vector<float> cuts(size_t max_bins) {
        std::vector<float> out;
        const size_t n_cuts = max_bins > 0 ? max_bins - 1 : 0;
        if (n_cuts == 0) return out;
        flush();
        Summary all;
        for (size_t l = 0; l < levels_.size(); l++)
            if (used_[l]) all = all.empty() ? levels_[l] : merge(all, levels_[l]);
        if (all.empty()) return out;
        all = prune(all, cap_);
        if (all.size() <= n_cuts) {
            for (size_t i = 0; i + 1 < all.size(); i++)
                out.push_back(cut_between(all[i].value, all[i + 1].value));
            return out;
        }
        const float total = all.back().rmax;
        for (size_t k = 1; k <= n_cuts; k++) {
            const float target = total * (float)k / (float)max_bins;
            const auto it = std::lower_bound(all.begin(), all.end(), target,
                                             [](const Rank &e, float t) { return e.mid() < t; });
            const size_t idx = std::min<size_t>(it - all.begin(), all.size() - 1);
            const float v = all[idx].value;
            if (out.empty() || v > out.back()) out.push_back(v);
        }
        return out;
    }

  private:
    void flush() {
        if (pending_.empty()) return;
        Summary s = prune(summarize(pending_), cap_);
        pending_.clear();
        for (size_t l = 0;; l++) {
            if (l == levels_.size()) {
                levels_.push_back(std::move(s));
                used_.push_back(1);
                return;
            }
            if (!used_[l]) {
                levels_[l] = std::move(s);
                used_[l] = 1;
                return;
            }
            s = prune(merge(levels_[l], s), cap_);
            levels_[l].clear();
            used_[l] = 0;
        }
    }
    size_t cap_;
    std::vector<std::pair<float, float>> pending_;
    std::vector<Summary> levels_;
    std::vector<uint8_t> used_;
};

unsigned clamp_threads(unsigned t) {
    if (t == 0) t = std::max(1u, std::thread::hardware_concurrency());
    return std::min(t, 64u);
}

template <class F>
void parallel_for(uint32_t n, unsigned threads, F &&f) {
    threads = std::min<unsigned>(clamp_threads(threads), std::max<uint32_t>(n, 1));
    if (threads <= 1) {
        for (uint32_t i = 0; i < n; i++) f(i);
        return;
    }
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; t++)
        pool.emplace_back([&, t] {
            for (uint32_t i = t; i < n; i += threads) f(i);
        });
    for (auto &th : pool) th.join();
}

}  // namespace

uint32_t Cuts::bin_of(uint32_t f, float v) const {
    if (is_cat(f)) {  // categorical::code_to_bin
        const uint32_t nb = n_bins(f);
        if (v >= 0.0f && v < (float)nb) return (uint32_t)v;
        return (width(f) == 1 ? 255u : 65535u) - 1;
    }
    const float *c = values.data() + offsets[f];
    return (uint32_t)(std::upper_bound(c, c + n_cuts(f), v) - c);
}

static std::vector<float> sketch_numeric(const float *x, uint64_t n, uint32_t nf, uint32_t f,
                                  uint32_t max_bin, const float *w) {
    FeatureQuantiles q(max_bin);
    for (uint64_t r = 0; r < n; r++) q.add(x[r * nf + f], w ? w[r] : 1.0f);
    return q.cuts(max_bin);
}

static Cuts assemble_cuts(std::vector<std::vector<float>> &per, uint32_t nf, const uint8_t *cat) {
    Cuts c;
    c.offsets.push_back(0);
    for (uint32_t f = 0; f < nf; f++) {
        c.values.insert(c.values.end(), per[f].begin(), per[f].end());
        c.offsets.push_back((uint32_t)c.values.size());
        c.categorical.push_back(cat && cat[f] ? 1 : 0);
    }
    for (uint32_t f = 0; f < nf; f++)
        if (c.n_bins(f) > (c.is_cat(f) ? 65534u : 65535u))
            throw InputError("feature " + std::to_string(f) + " has too many bins");
    return c;
}

Cuts sketch_matrix(const float *x, uint64_t n, uint32_t nf, uint32_t max_bin, const float *w,
                   const uint8_t *cat, unsigned threads) {
    std::vector<std::vector<float>> per(nf);
    std::vector<int> bad(nf, 0);
    parallel_for(nf, threads, [&](uint32_t f) {
        if (cat && cat[f]) {
            int max_code = -1;
            for (uint64_t r = 0; r < n; r++) {
                const float v = x[r * nf + f];
                if (std::isnan(v)) continue;
                if (v < 0.0f || v > 65533.0f || v != std::trunc(v)) {
                    bad[f] = 1;
                    continue;
                }
                max_code = std::max(max_code, (int)v);
            }
            for (int c = 1; c <= std::max(max_code, 0); c++) per[f].push_back((float)c);
            return;
        }
        per[f] = sketch_numeric(x, n, nf, f, max_bin, w);
    });
    for (uint32_t f = 0; f < nf; f++)
        if (bad[f])
            throw InputError("categorical feature #" + std::to_string(f) +
                             " contains a value that is not an integer code in 0..=65533");
    return assemble_cuts(per, nf, cat);
}

Cuts sketch_matrix_device(int device, const RowSource &src, uint64_t n, uint32_t nf,
                          uint32_t max_bin, const uint8_t *cat, uint64_t memory_budget,
                          unsigned threads) {
    fbh_sketch *raw = nullptr;
    auto call = [](int rc) {
        if (rc == FBH_OK) return;
        char buf[1024];
        fbh_last_error(buf, sizeof buf);
        if (rc == FBH_INPUT_ERROR) throw InputError(buf);
        throw RuntimeError(buf);
    };
    call(fbh_sketch_create(device, n, nf, max_bin, cat, memory_budget, &raw));
    std::unique_ptr<fbh_sketch, int (*)(fbh_sketch *)> s(raw, fbh_sketch_destroy);
    src.each_chunk(n, nf, [&](uint64_t, uint64_t k, const float *rows) {
        call(fbh_sketch_push_rows(s.get(), rows, k));
    });
    uint64_t cap = 0;
    for (uint32_t f = 0; f < nf; f++) cap += (cat && cat[f]) ? 65533u : (max_bin ? max_bin - 1 : 0);
    std::vector<float> values(std::max<uint64_t>(cap, 1));
    std::vector<uint32_t> offsets(nf + 1);
    std::vector<uint8_t> host(nf);
    call(fbh_sketch_cuts(s.get(), values.data(), cap, offsets.data(), host.data()));
    std::vector<uint64_t> missing(nf);
    call(fbh_sketch_missing(s.get(), missing.data()));
    s.reset();
    std::vector<std::vector<float>> per(nf);
    std::vector<uint32_t> on_host;
    for (uint32_t f = 0; f < nf; f++) {
        if (host[f]) on_host.push_back(f);
        else per[f].assign(values.begin() + offsets[f], values.begin() + offsets[f + 1]);
    }
    // Features holding both zero signs with a zero among their cuts: the
    // host sketch decides the zero's sign (a reader's rows are read again for
    // just those columns).
    if (!on_host.empty()) {
        const uint32_t k = (uint32_t)on_host.size();
        std::vector<float> cols;
        const float *mat = src.x;
        uint32_t stride = nf;
        if (!mat) {
            cols.resize(n * k);
            src.each_chunk(n, nf, [&](uint64_t r0, uint64_t c, const float *rows) {
                for (uint64_t r = 0; r < c; r++)
                    for (uint32_t j = 0; j < k; j++) cols[(r0 + r) * k + j] = rows[r * nf + on_host[j]];
            });
            mat = cols.data();
            stride = k;
        }
        parallel_for(k, threads, [&](uint32_t i) {
            per[on_host[i]] = sketch_numeric(mat, n, stride, src.x ? on_host[i] : i, max_bin, nullptr);
        });
    }
    Cuts c = assemble_cuts(per, nf, cat);
    // 256-bin numeric features without a missing row take 8-bit cells.
    c.full.assign(nf, 0);
    for (uint32_t f = 0; f < nf; f++)
        if (!c.is_cat(f) && c.n_bins(f) == 256 && missing[f] == 0) c.full[f] = 1;
    return c;
}

void check_cuts(const Cuts &c, uint32_t nf, uint32_t max_bin, const uint8_t *cat) {
    if (c.offsets.size() != (size_t)nf + 1 || c.offsets[0] != 0 ||
        c.offsets.back() != c.values.size())
        throw InputError("cuts: offsets must hold n_features + 1 entries from 0 to the value count");
    for (uint32_t f = 0; f < nf; f++) {
        if (c.offsets[f + 1] < c.offsets[f]) throw InputError("cuts: offsets must not decrease");
        const bool is_cat = cat && cat[f];
        if ((c.categorical[f] != 0) != is_cat)
            throw InputError("cuts: feature " + std::to_string(f) +
                             " is categorical in one place and numeric in the other");
        const uint32_t nc = c.n_cuts(f);
        if (!is_cat && nc + 1 > std::max(max_bin, 1u))
            throw InputError("cuts: feature " + std::to_string(f) + " has " + std::to_string(nc) +
                             " cuts, more than max_bin - 1 = " + std::to_string(max_bin - 1));
        if (c.n_bins(f) > (is_cat ? 65534u : 65535u))
            throw InputError("cuts: feature " + std::to_string(f) + " has too many bins");
        const float *v = c.values.data() + c.offsets[f];
        for (uint32_t i = 0; i < nc; i++) {
            if (!std::isfinite(v[i]))
                throw InputError("cuts: feature " + std::to_string(f) + " has a non-finite cut");
            if (i && !(v[i] > v[i - 1]))
                throw InputError("cuts: feature " + std::to_string(f) +
                                 " cuts must be strictly increasing");
        }
    }
}

void bin_columns(const float *x, uint64_t n, uint32_t nf, const Cuts &cuts,
                 const std::vector<uint32_t> &feats, uint32_t width, void *out, unsigned threads) {
    parallel_for((uint32_t)feats.size(), threads, [&](uint32_t l) {
        const uint32_t f = feats[l];
        const uint32_t missing = width == 1 ? 0xFFu : 0xFFFFu;
        if (width == 1) {
            uint8_t *col = static_cast<uint8_t *>(out) + (uint64_t)l * n;
            for (uint64_t r = 0; r < n; r++) {
                const float v = x[r * nf + f];
                col[r] = (uint8_t)(std::isnan(v) ? missing : cuts.bin_of(f, v));
            }
        } else {
            uint16_t *col = static_cast<uint16_t *>(out) + (uint64_t)l * n;
            for (uint64_t r = 0; r < n; r++) {
                const float v = x[r * nf + f];
                col[r] = (uint16_t)(std::isnan(v) ? missing : cuts.bin_of(f, v));
            }
        }
    });
}

std::vector<std::vector<uint32_t>> blocks_by_width(const Cuts &cuts, uint32_t cols) {
    if (cols == 0) throw InputError("cols_per_block must be > 0");
    std::vector<std::vector<uint32_t>> blocks;
    for (uint32_t w : {1u, 2u}) {
        std::vector<uint32_t> feats;
        for (uint32_t f = 0; f < cuts.n_features(); f++)
            if (cuts.width(f) == w) feats.push_back(f);
        const uint32_t per = (cols + w - 1) / w;
        for (size_t i = 0; i < feats.size(); i += per)
            blocks.emplace_back(feats.begin() + i, feats.begin() + std::min(feats.size(), i + per));
    }
    std::sort(blocks.begin(), blocks.end(),
              [](const std::vector<uint32_t> &a, const std::vector<uint32_t> &b) {
                  return a[0] < b[0];
              });
    return blocks;
}

}  // namespace fbt
