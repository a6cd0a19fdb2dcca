// fbhip_shap.hip -- GPU QuadratureTreeSHAP model (fbh_shap_* of include/fbhip.h).
//
// The ensemble is flattened once into structure-of-nodes arrays with global
// child ids (GpuExplainModel::flatten, src/backend/cuda/explain.rs:186-345):
// each internal node carries the branch weights of its children
// (branch_weight, src/model/explain.rs:186-196) and the slot of its feature
// in its tree's list of distinct split features, so the kernel accumulates a
// tree's contributions in a short per-thread array before adding them to the
// row, in the host engine's order.

#include "fbhip_internal.h"
#include "../../include/fbhip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

using namespace fbh;

namespace {

struct ShapError : std::runtime_error {
    int code;
    ShapError(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

void chk(hipError_t e, const char *what) {
    if (e != hipSuccess) throw ShapError(FBH_RUNTIME_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}

// Gauss-Legendre nodes by Newton iteration on P_8, mapped to [0, 1] and
// squared (the endpoint rule of XGBoost's MakeEndpointQuadrature, restated
// in src/model/explain.rs:141-169).
void quadrature_rule(float nodes[8], float weights[8]) {
    const int n = 8;
    auto legendre = [](int m, double x) {
        if (m == 0) return 1.0;
        double p0 = 1.0, p1 = x;
        for (int k = 2; k <= m; k++) {
            const double kf = (double)k;
            const double pk = ((2.0 * kf - 1.0) * x * p1 - (kf - 1.0) * p0) / kf;
            p0 = p1;
            p1 = pk;
        }
        return p1;
    };
    for (int i = 0; i < n; i++) {
        double x = std::cos(M_PI * ((double)i + 0.75) / ((double)n + 0.5));
        for (int it = 0; it < 64; it++) {
            const double pn = legendre(n, x);
            const double dpn = (double)n * (x * pn - legendre(n - 1, x)) / (x * x - 1.0);
            const double dx = pn / dpn;
            x -= dx;
            if (std::fabs(dx) < 1e-15) break;
        }
        const double pn = legendre(n, x);
        const double dpn = (double)n * (x * pn - legendre(n - 1, x)) / (x * x - 1.0);
        const double w = 2.0 / ((1.0 - x * x) * dpn * dpn);
        const double s = 0.5 * (x + 1.0);
        const int o = n - 1 - i;
        nodes[o] = (float)(s * s);
        weights[o] = (float)(2.0 * s * (0.5 * w));
    }
}

float branch_weight(float cover, float parent) {
    if (parent <= 0.0f) return 0.5f;
    const float w = cover / parent;
    return w < 1e-12f ? 1e-12f : w;
}

}  // namespace

struct fbh_shap_model {
    int device = 0;
    hipStream_t stream = nullptr;
    uint32_t n_trees = 0, n_features = 0, max_unique = 1, max_depth = 1;
    float bias = 0.0f, root_mean = 0.0f;
    ShapNodeDev *d_nodes = nullptr;
    uint32_t *d_roots = nullptr, *d_uoff = nullptr, *d_ufeats = nullptr, *d_cats = nullptr;
    float *d_rule = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    double last_ms = 0.0;
    std::vector<void *> allocs;

    ~fbh_shap_model() {
        if (device >= 0) (void)hipSetDevice(device);
        if (stream) (void)hipStreamSynchronize(stream);
        for (void *p : allocs) (void)hipFree(p);
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
        if (stream) (void)hipStreamDestroy(stream);
    }
    template <class T>
    T *upload(const std::vector<T> &v, const char *what) {
        void *p = nullptr;
        const size_t bytes = std::max<size_t>(sizeof(T) * v.size(), 64);
        chk(hipMalloc(&p, bytes), what);
        allocs.push_back(p);
        if (!v.empty()) chk(hipMemcpy(p, v.data(), sizeof(T) * v.size(), hipMemcpyHostToDevice), what);
        return static_cast<T *>(p);
    }
};

namespace {

template <class F>
int shap_guard(F &&f) {
    try {
        f();
        return FBH_OK;
    } catch (const ShapError &e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::exception &e) {
        set_last_error(e.what());
        return FBH_RUNTIME_ERROR;
    }
}

// Cover-weighted mean leaf value in f64 (root_mean, src/model/explain.rs:409-423).
double root_mean(const std::vector<int32_t> &left, const std::vector<int32_t> &right,
                 const std::vector<float> &leaf, const std::vector<float> &hess,
                 const std::vector<uint8_t> &is_leaf, uint32_t base, uint32_t idx) {
    const uint32_t g = base + idx;
    if (is_leaf[g]) return (double)leaf[g];
    const uint32_t l = (uint32_t)left[g], r = (uint32_t)right[g];
    const double lm = root_mean(left, right, leaf, hess, is_leaf, base, l);
    const double rm = root_mean(left, right, leaf, hess, is_leaf, base, r);
    if (hess[g] == 0.0f) return 0.5 * (lm + rm);
    return (lm * (double)hess[base + l] + rm * (double)hess[base + r]) / (double)hess[g];
}

}  // namespace

extern "C" {

int fbh_shap_model_create(int device, uint32_t n_trees, const uint32_t *tree_offsets,
                          const uint32_t *feat, const float *split_cond, const int32_t *left,
                          const int32_t *right, const uint8_t *default_left,
                          const uint8_t *is_leaf, const float *leaf_value, const float *sum_hess,
                          const uint32_t *cat_offset, const uint32_t *cat_len,
                          const uint32_t *cat_words, uint32_t n_cat_words, uint32_t n_features,
                          float bias, fbh_shap_model **out) {
    return shap_guard([&] {
        if (!out || !tree_offsets) throw ShapError(FBH_INPUT_ERROR, "null argument");
        *out = nullptr;
        if (n_features == 0) throw ShapError(FBH_INPUT_ERROR, "model has no features");
        auto m = std::make_unique<fbh_shap_model>();
        m->device = device;
        chk(hipSetDevice(device), "hipSetDevice");
        chk(hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking), "stream");
        chk(hipEventCreate(&m->e0), "event");
        chk(hipEventCreate(&m->e1), "event");
        const uint32_t total = tree_offsets[n_trees];
        std::vector<int32_t> L(left, left + total), R(right, right + total);
        std::vector<float> lv(leaf_value, leaf_value + total), hs(sum_hess, sum_hess + total);
        std::vector<uint8_t> lf(is_leaf, is_leaf + total);
        std::vector<ShapNodeDev> nodes(total);
        std::vector<uint32_t> roots(n_trees), uoff(n_trees + 1, 0), ufeats;
        double rm_sum = 0.0;
        for (uint32_t t = 0; t < n_trees; t++) {
            const uint32_t b = tree_offsets[t], e = tree_offsets[t + 1];
            if (e <= b) throw ShapError(FBH_INPUT_ERROR, "tree " + std::to_string(t) + " has no nodes");
            roots[t] = b;
            std::vector<int32_t> slot_of(n_features, -1);
            uoff[t] = (uint32_t)ufeats.size();
            // depth of the tree (internal nodes on the longest path)
            std::vector<uint32_t> depth(e - b, 0);
            for (uint32_t i = b; i < e; i++) {
                ShapNodeDev d{};
                d.feat = feat[i];
                d.split_cond = split_cond[i];
                d.leaf_value = leaf_value[i];
                d.flags = (is_leaf[i] ? 1u : 0u) | (default_left[i] ? 2u : 0u) |
                          (cat_len && cat_len[i] ? 4u : 0u);
                d.cat_offset = cat_offset ? cat_offset[i] : 0;
                d.cat_len = cat_len ? cat_len[i] : 0;
                if (d.cat_len && (!cat_words || (uint64_t)d.cat_offset + d.cat_len > n_cat_words))
                    throw ShapError(FBH_INPUT_ERROR, "category set out of range");
                d.left = d.right = -1;
                if (!is_leaf[i]) {
                    if (feat[i] >= n_features)
                        throw ShapError(FBH_INPUT_ERROR, "split feature out of range");
                    const int32_t l = left[i], r = right[i];
                    if (l <= 0 || r <= 0 || (uint32_t)l >= e - b || (uint32_t)r >= e - b ||
                        (uint32_t)l <= i - b || (uint32_t)r <= i - b)
                        throw ShapError(FBH_INPUT_ERROR, "child ids must follow their parent");
                    if (hs[i] < 0.0f || hs[b + l] < 0.0f || hs[b + r] < 0.0f)
                        throw ShapError(FBH_INPUT_ERROR, "tree " + std::to_string(t) +
                                                             " has a negative cover (sum_hessian) at a split: SHAP is undefined");
                    if (std::isnan(hs[i]) || std::isnan(hs[b + l]) || std::isnan(hs[b + r]))
                        throw ShapError(FBH_INPUT_ERROR, "tree " + std::to_string(t) +
                                                             " has a NaN cover (sum_hessian): SHAP is undefined");
                    d.left = (int32_t)(b + l);
                    d.right = (int32_t)(b + r);
                    d.left_weight = branch_weight(hs[b + l], hs[i]);
                    d.right_weight = branch_weight(hs[b + r], hs[i]);
                    if (slot_of[feat[i]] < 0) {
                        slot_of[feat[i]] = (int32_t)(ufeats.size() - uoff[t]);
                        ufeats.push_back(feat[i]);
                    }
                    d.uslot = (uint32_t)slot_of[feat[i]];
                    depth[l] = depth[i - b] + 1;
                    depth[r] = depth[i - b] + 1;
                    m->max_depth = std::max(m->max_depth, depth[i - b] + 1);
                }
                nodes[i] = d;
            }
            m->max_unique = std::max<uint32_t>(m->max_unique, (uint32_t)ufeats.size() - uoff[t]);
            if (m->max_unique > MAX_SHAP_UNIQUE)
                throw ShapError(FBH_INPUT_ERROR, "a tree splits on more than " +
                                                     std::to_string(MAX_SHAP_UNIQUE) +
                                                     " distinct features");
            rm_sum += root_mean(L, R, lv, hs, lf, b, 0);
        }
        uoff[n_trees] = (uint32_t)ufeats.size();
        if (m->max_depth > 16)
            throw ShapError(FBH_INPUT_ERROR, "trees deeper than 16 splits are not supported on the device");
        float rule[16];
        quadrature_rule(rule, rule + 8);
        std::vector<float> rv(rule, rule + 16);
        std::vector<uint32_t> cw(cat_words ? cat_words : nullptr,
                                 cat_words ? cat_words + n_cat_words : nullptr);
        m->n_trees = n_trees;
        m->n_features = n_features;
        m->bias = bias;
        m->root_mean = (float)rm_sum;
        m->d_nodes = m->upload(nodes, "shap nodes");
        m->d_roots = m->upload(roots, "shap roots");
        m->d_uoff = m->upload(uoff, "shap features");
        m->d_ufeats = m->upload(ufeats, "shap features");
        m->d_cats = m->upload(cw, "shap categories");
        m->d_rule = m->upload(rv, "shap rule");
        *out = m.release();
    });
}

int fbh_shap_model_destroy(fbh_shap_model *m) {
    return shap_guard([&] { delete m; });
}

int fbh_shap_contribs_device(fbh_shap_model *m, const float *d_rows, uint64_t n_rows,
                             const float *d_margin, float *d_out, int sync) {
    return shap_guard([&] {
        if (!m || (!d_rows && n_rows) || (!d_out && n_rows))
            throw ShapError(FBH_INPUT_ERROR, "null argument");
        chk(hipSetDevice(m->device), "hipSetDevice");
        chk(hipEventRecord(m->e0, m->stream), "event");
        chk(launch_shap(m->d_nodes, m->d_roots, m->n_trees, m->d_uoff, m->d_ufeats, m->d_cats,
                        m->d_rule, d_rows, n_rows, m->n_features, d_margin, m->bias, m->root_mean,
                        d_out, m->max_unique, m->max_depth, m->stream),
            "shap launch");
        chk(hipEventRecord(m->e1, m->stream), "event");
        if (sync) {
            chk(hipStreamSynchronize(m->stream), "shap");
            float ms = 0.0f;
            chk(hipEventElapsedTime(&ms, m->e0, m->e1), "event");
            m->last_ms = ms;
        }
    });
}

double fbh_shap_last_ms(const fbh_shap_model *m) { return m ? m->last_ms : 0.0; }

int fbh_shap_contribs(fbh_shap_model *m, const float *rows, uint64_t n_rows, const float *margin,
                      float *out) {
    return shap_guard([&] {
        if (!m || (!rows && n_rows) || (!out && n_rows))
            throw ShapError(FBH_INPUT_ERROR, "null argument");
        if (n_rows == 0) return;
        chk(hipSetDevice(m->device), "hipSetDevice");
        // Batches of at most 512 MiB of inputs and outputs on the device
        // (GpuExplainModel::compute batching, src/backend/cuda/explain.rs:491-560).
        const uint64_t per_row = 4ull * (2 * m->n_features + 2);
        const uint64_t batch = std::max<uint64_t>(1, (512ull << 20) / per_row);
        float *d_rows = nullptr, *d_out = nullptr, *d_margin = nullptr;
        const uint64_t nb = std::min(batch, n_rows);
        chk(hipMalloc(&d_rows, 4 * nb * m->n_features), "shap rows");
        std::unique_ptr<float, decltype(&hipFree)> f1(d_rows, hipFree);
        chk(hipMalloc(&d_out, 4 * nb * (m->n_features + 1)), "shap out");
        std::unique_ptr<float, decltype(&hipFree)> f2(d_out, hipFree);
        if (margin) chk(hipMalloc(&d_margin, 4 * nb), "shap margin");
        std::unique_ptr<float, decltype(&hipFree)> f3(d_margin, hipFree);
        double kernel_ms = 0.0;
        for (uint64_t r0 = 0; r0 < n_rows; r0 += nb) {
            const uint64_t k = std::min(nb, n_rows - r0);
            chk(hipMemcpyAsync(d_rows, rows + r0 * m->n_features, 4 * k * m->n_features,
                               hipMemcpyHostToDevice, m->stream),
                "shap rows");
            if (margin)
                chk(hipMemcpyAsync(d_margin, margin + r0, 4 * k, hipMemcpyHostToDevice, m->stream),
                    "shap margin");
            if (fbh_shap_contribs_device(m, d_rows, k, margin ? d_margin : nullptr, d_out, 0))
                throw ShapError(FBH_RUNTIME_ERROR, last_error());
            chk(hipMemcpyAsync(out + r0 * (m->n_features + 1), d_out, 4 * k * (m->n_features + 1),
                               hipMemcpyDeviceToHost, m->stream),
                "shap out");
            chk(hipStreamSynchronize(m->stream), "shap");
            float ms = 0.0f;
            chk(hipEventElapsedTime(&ms, m->e0, m->e1), "event");
            kernel_ms += ms;
        }
        m->last_ms = kernel_ms;
    });
}

}  // extern "C"
