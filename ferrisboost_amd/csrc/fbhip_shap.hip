// fbhip_shap.hip -- the device explanation and prediction model (fbh_shap_*,
// fbh_predict*, fbh_saabas_contribs, fbh_shap_interactions of include/fbhip.h).
//
// The ensemble is flattened once into node arrays with global child ids
// (GpuExplainModel::flatten, src/backend/cuda/explain.rs:186-345):
//   * ShapNodeDev: every field an explanation needs -- the branch weights of
//     the children (branch_weight, src/model/explain.rs:186-196) and the slot
//     of the node's feature in its tree's list of distinct split features, so
//     TreeSHAP accumulates a tree's contributions in a short per-thread array
//     before adding them to the row, in the host engine's order;
//   * PredNodeDev: a 16-byte copy of what a root-to-leaf walk reads (feature
//     and flags in one word, threshold or leaf value, children), so the walks
//     of prediction, leaf indices and Saabas touch one cache line per node
//     pair;
//   * the cover-weighted mean of every node in f32 (fill_node_means,
//     src/model/explain.rs:409-422) for Saabas.
// Every kernel gives one thread one row and walks the trees in model order,
// with the host engine's float32 operations in the host engine's order, so
// results equal the CPU's bit for bit.

#include "fbhip_internal.h"
#include "fb_expf.h"
#include "../../include/fbhip.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

using namespace fbh;

// File-scope device array for fbh_shap_contribs_noalloc: every device holds
// its own copy at its own address, found once per device with
// hipGetSymbolAddress (scratch_of below); host code uses that address, never
// the array's name, which on the host is only a stand-in. Calls on one device
// share it.
static __device__ __align__(256) unsigned char scratch[FBH_NOALLOC_SCRATCH_BYTES];

namespace {

// ====================================================================== device

constexpr int QP = 8;          // quadrature points
constexpr float UNSEEN = -999.0f;
constexpr int SHAP_MAXD = 16;  // path frames (max_depth <= 14 in training; loaded models <= 16)
constexpr int SHAP_TPB = 128;
constexpr int PRED_TPB = 256;

// Walk node: feature and flags in one word.
struct PredNodeDev {
    uint32_t ff;     // feature | PN_LEAF | PN_DEFAULT_LEFT | PN_CAT
    float value;     // split condition, or the leaf value of a leaf
    int32_t left, right;
};
constexpr uint32_t PN_LEAF = 1u << 31;
constexpr uint32_t PN_DEFAULT_LEFT = 1u << 30;
constexpr uint32_t PN_CAT = 1u << 29;
constexpr uint32_t PN_FEAT = PN_CAT - 1;

// Output kinds of predict_kernel.
constexpr uint32_t PRED_MARGIN = 0, PRED_SIGMOID = 1, PRED_LEAF = 2;

// categorical::goes_left (src/data/categorical.rs:334-370): a category in the
// node's right-going set goes right; negative, non-integral-range and
// unlisted codes go left.
__device__ __forceinline__ bool cat_goes_left(float v, const uint32_t *words, uint32_t off,
                                              uint32_t len) {
    if (v < 0.0f || v >= 16777216.0f) return true;
    const uint32_t cat = (uint32_t)v;
    const uint32_t word = cat / 32;
    if (word >= len) return true;
    return ((words[off + word] >> (cat % 32)) & 1u) == 0;
}

// Node::goes_left (src/model/tree.rs:85-95).
__device__ __forceinline__ bool shap_goes_left(const ShapNodeDev &n, float v,
                                               const uint32_t *cat_words) {
    if (isnan(v)) return (n.flags & 2u) != 0;
    if (n.flags & 4u) return cat_goes_left(v, cat_words, n.cat_offset, n.cat_len);
    return v < n.split_cond;
}

// One step of a walk from node `id`.
__device__ __forceinline__ uint32_t walk_step(const PredNodeDev &n, uint32_t id, const float *x,
                                              const ShapNodeDev *full, const uint32_t *cats) {
    const float v = x[n.ff & PN_FEAT];
    bool left;
    if (v != v) left = (n.ff & PN_DEFAULT_LEFT) != 0;
    else if (n.ff & PN_CAT) left = cat_goes_left(v, cats, full[id].cat_offset, full[id].cat_len);
    else left = v < n.value;
    return (uint32_t)(left ? n.left : n.right);
}

// predict_margin_soa[_cat] (src/backend/cuda/histogram.cu:2459-2494,
// 3600-3642) and leaf_row (src/model/explain.rs:689-702): the row's margin
// starts from its own base margin (or the model's) and adds each tree's leaf
// in tree order (Model::predict_margin, src/model/tree.rs:486-510); the
// logistic link is the sigmoid of objective.rs:37-39 with glibc's expf
// method, bit-identical to the host's. PRED_LEAF writes each tree's
// tree-local leaf id as a float.
// One row's walk over every tree (x: the row's cells, in global memory or
// LDS): margins and values write out[row], leaf ids out[row * n_trees + t].
__device__ __forceinline__ void predict_row(const PredNodeDev *__restrict__ nodes,
                                            const ShapNodeDev *__restrict__ full,
                                            const uint32_t *__restrict__ cats,
                                            const uint32_t *__restrict__ roots, uint32_t n_trees,
                                            const float *x, uint64_t row,
                                            const float *__restrict__ init, float base,
                                            uint32_t mode, float *__restrict__ out) {
    if (mode == PRED_LEAF) {
        float *o = out + row * n_trees;
        for (uint32_t t = 0; t < n_trees; t++) {
            const uint32_t root = roots[t];
            uint32_t id = root;
            PredNodeDev n = nodes[id];
            while (!(n.ff & PN_LEAF)) {
                id = walk_step(n, id, x, full, cats);
                n = nodes[id];
            }
            o[t] = (float)(id - root);
        }
        return;
    }
    float m = init ? init[row] : base;
    for (uint32_t t = 0; t < n_trees; t++) {
        uint32_t id = roots[t];
        PredNodeDev n = nodes[id];
        while (!(n.ff & PN_LEAF)) {
            id = walk_step(n, id, x, full, cats);
            n = nodes[id];
        }
        m += n.value;
    }
    out[row] = mode == PRED_SIGMOID ? fb_sigmoid(m) : m;
}

__global__ __launch_bounds__(PRED_TPB) void predict_kernel(
    const PredNodeDev *__restrict__ nodes, const ShapNodeDev *__restrict__ full,
    const uint32_t *__restrict__ cats, const uint32_t *__restrict__ roots, uint32_t n_trees,
    const float *__restrict__ rows, uint64_t n_rows, uint32_t nf, const float *__restrict__ init,
    float base, uint32_t mode, float *__restrict__ out) {
    const uint64_t row = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= n_rows) return;
    predict_row(nodes, full, cats, roots, n_trees, rows + row * nf, row, init, base, mode, out);
}

// The same walk with a wave's 64 rows first copied into LDS (coalesced
// loads; row stride nf | 1, odd, so the 64 lanes' cells of one feature fall
// in distinct banks): a node's cell is then an LDS read instead of a
// gather of one cache line a lane from the row-major matrix.
constexpr uint32_t PRED_LDS_ROWS = 64;
constexpr uint32_t PRED_LDS_MAX_F = 255;  // 64 rows x 256 floats: 64 KiB of LDS

__global__ __launch_bounds__(PRED_LDS_ROWS) void predict_lds_kernel(
    const PredNodeDev *__restrict__ nodes, const ShapNodeDev *__restrict__ full,
    const uint32_t *__restrict__ cats, const uint32_t *__restrict__ roots, uint32_t n_trees,
    const float *__restrict__ rows, uint64_t n_rows, uint32_t nf, const float *__restrict__ init,
    float base, uint32_t mode, float *__restrict__ out) {
    extern __shared__ float xs[];
    const uint32_t S = nf | 1u;
    const uint64_t r0 = (uint64_t)blockIdx.x * PRED_LDS_ROWS;
    const uint32_t nr = (uint32_t)min<uint64_t>(PRED_LDS_ROWS, n_rows - r0);
    const float *src = rows + r0 * nf;
    for (uint32_t r = 0; r < nr; r++)
        for (uint32_t f = threadIdx.x; f < nf; f += PRED_LDS_ROWS) xs[r * S + f] = src[r * nf + f];
    __syncthreads();
    if (threadIdx.x >= nr) return;
    predict_row(nodes, full, cats, roots, n_trees, xs + threadIdx.x * S, r0 + threadIdx.x, init,
                base, mode, out);
}

// The LDS rows shared by four waves, which take every fourth tree of a run
// of PRED_RUN trees and put each row's leaf value in LDS; wave 0 then adds
// the run's values to the row's margin in tree order (the host's f32
// additions, so the margins stay bit-identical), and the waves go on to the
// next run. Four times the waves of predict_lds_kernel on the same rows.
constexpr uint32_t PRED_WAVES = 4;
constexpr uint32_t PRED_RUN = 32;
constexpr uint32_t PRED_LDS4_MAX_F = 223;  // 64 x 224 + 64 x 32 floats: 64 KiB of LDS

__global__ __launch_bounds__(PRED_LDS_ROWS * PRED_WAVES) void predict_lds4_kernel(
    const PredNodeDev *__restrict__ nodes, const ShapNodeDev *__restrict__ full,
    const uint32_t *__restrict__ cats, const uint32_t *__restrict__ roots, uint32_t n_trees,
    const float *__restrict__ rows, uint64_t n_rows, uint32_t nf, const float *__restrict__ init,
    float base, uint32_t mode, float *__restrict__ out) {
    extern __shared__ float xs[];
    const uint32_t S = nf | 1u;
    float *leafv = xs + PRED_LDS_ROWS * S;  // [PRED_RUN][64]
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint64_t r0 = (uint64_t)blockIdx.x * PRED_LDS_ROWS;
    const uint32_t nr = (uint32_t)min<uint64_t>(PRED_LDS_ROWS, n_rows - r0);
    const float *src = rows + r0 * nf;
    for (uint32_t r = wave; r < nr; r += PRED_WAVES)
        for (uint32_t f = lane; f < nf; f += 64) xs[r * S + f] = src[r * nf + f];
    __syncthreads();
    const bool live = lane < nr;
    const uint64_t row = r0 + lane;
    const float *x = xs + lane * S;
    float m = 0.0f;
    if (wave == 0 && live) m = init ? init[row] : base;
    for (uint32_t t0 = 0; t0 < n_trees; t0 += PRED_RUN) {
        const uint32_t t1 = min(t0 + PRED_RUN, n_trees);
        if (live)
            for (uint32_t t = t0 + wave; t < t1; t += PRED_WAVES) {
                const uint32_t root = roots[t];
                uint32_t id = root;
                PredNodeDev n = nodes[id];
                while (!(n.ff & PN_LEAF)) {
                    id = walk_step(n, id, x, full, cats);
                    n = nodes[id];
                }
                if (mode == PRED_LEAF) out[row * n_trees + t] = (float)(id - root);
                else leafv[(t - t0) * 64 + lane] = n.value;
            }
        if (mode == PRED_LEAF) continue;
        __syncthreads();
        if (wave == 0 && live)
            for (uint32_t t = t0; t < t1; t++) m += leafv[(t - t0) * 64 + lane];
        __syncthreads();
    }
    if (mode != PRED_LEAF && wave == 0 && live)
        out[row] = mode == PRED_SIGMOID ? fb_sigmoid(m) : m;
}

// saabas_row (src/model/explain.rs:730-760): along the row's path, each split
// feature receives the change of the cover-weighted node mean; the bias
// column the root mean. A tree's contributions are summed per feature first
// (the host's tree_contribs), then added to the row.
__global__ __launch_bounds__(PRED_TPB) void saabas_kernel(
    const PredNodeDev *__restrict__ nodes, const ShapNodeDev *__restrict__ full,
    const uint32_t *__restrict__ cats, const float *__restrict__ means,
    const uint32_t *__restrict__ roots, uint32_t n_trees, const float *__restrict__ rows,
    uint64_t n_rows, uint32_t nf, const float *__restrict__ init, float base,
    float *__restrict__ out) {
    const uint64_t row = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= n_rows) return;
    const float *x = rows + row * nf;
    float *p = out + row * (uint64_t)(nf + 1);
    for (uint32_t f = 0; f <= nf; f++) p[f] = 0.0f;
    uint32_t tf[SHAP_MAXD + 1];
    float tv[SHAP_MAXD + 1];
    for (uint32_t t = 0; t < n_trees; t++) {
        const uint32_t root = roots[t];
        float node_value = means[root];
        const float tb = 0.0f + node_value;
        uint32_t nu = 0;
        auto add = [&](uint32_t f, float d) {
            for (uint32_t u = 0; u < nu; u++)
                if (tf[u] == f) {
                    tv[u] += d;
                    return;
                }
            tf[nu] = f;
            tv[nu] = 0.0f + d;
            nu++;
        };
        uint32_t id = root;
        PredNodeDev n = nodes[id];
        if (!(n.ff & PN_LEAF)) {
            uint32_t split = 0;
            while (!(n.ff & PN_LEAF)) {
                split = n.ff & PN_FEAT;
                id = walk_step(n, id, x, full, cats);
                n = nodes[id];
                const float nv = means[id];
                add(split, nv - node_value);
                node_value = nv;
            }
            add(split, n.value - node_value);
        }
        for (uint32_t u = 0; u < nu; u++) p[tf[u]] += tv[u];
        p[nf] += tb;
    }
    p[nf] += init ? init[row] : base;
}

// QuadratureTreeSHAP: every tree's Runner::run_node / visit_child recursion
// (src/model/explain.rs:303-401) unrolled onto an explicit path stack, in the
// host's exact float32 operation order.
//   INTER == false: pred_contribs (Additive, shap_row :704-728): each visit's
//     extract_delta goes into the tree's per-feature sums.
//   INTER == true: pred_interactions (Interaction, interaction_row :762-811):
//     extract_delta goes into the row's diagonal accumulator (the matrix
//     diagonal, which no visit writes otherwise) and extract_interaction_delta
//     of every partner on the live path into the matrix row of the feature;
//     the matrix is symmetrised and its diagonal completed at the end.
template <int MAXU, bool INTER>
__global__ __launch_bounds__(SHAP_TPB) void shap_kernel(
    const ShapNodeDev *nodes, const uint32_t *tree_roots, uint32_t n_trees,
    const uint32_t *tree_ufeat_off, const uint32_t *ufeats, const uint32_t *cat_words,
    const float *rule, const float *rows, uint64_t n_rows, uint32_t n_features,
    const float *margin, float bias, float root_mean, float *out) {
    const uint64_t row = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= n_rows) return;
    float rn[QP], rw[QP];
#pragma unroll
    for (int i = 0; i < QP; i++) {
        rn[i] = rule[i];
        rw[i] = rule[QP + i];
    }
    const uint32_t nc = n_features + 1;
    const float *x = rows + row * n_features;
    // INTER: the caller zeroed the row's nc x nc matrix.
    float *p = INTER ? out + row * (uint64_t)nc * nc : out + row * (uint64_t)nc;
    if (!INTER)
        for (uint32_t f = 0; f <= n_features; f++) p[f] = 0.0f;

    float tc[MAXU];
    float c[SHAP_MAXD][QP];
    float hl[SHAP_MAXD][QP];
    float wprod[SHAP_MAXD];
    float pe[SHAP_MAXD], pold[SHAP_MAXD];
    uint32_t nid[SHAP_MAXD], pfeat[SHAP_MAXD];
    uint8_t stage[SHAP_MAXD], gl[SHAP_MAXD];

    for (uint32_t t = 0; t < n_trees; t++) {
        const uint32_t root = tree_roots[t];
        const uint32_t u0 = tree_ufeat_off[t], nu = tree_ufeat_off[t + 1] - u0;
        if (nodes[root].flags & 1u) continue;  // a leaf-only tree contributes nothing
        if (!INTER)
            for (uint32_t u = 0; u < nu; u++) tc[u] = 0.0f;
        int d = 0;
        nid[0] = root;
        wprod[0] = 1.0f;
#pragma unroll
        for (int i = 0; i < QP; i++) c[0][i] = 1.0f;
        stage[0] = 0;
        {
            const ShapNodeDev &n0 = nodes[root];
            gl[0] = shap_goes_left(n0, x[n0.feat], cat_words);
        }
        float ret[QP];
        for (;;) {
            const ShapNodeDev &n = nodes[nid[d]];
            // Begin the visit of the next child of frame d.
            const bool right = stage[d] != 0;
            const uint32_t child = (uint32_t)(right ? n.right : n.left);
            const float cw = right ? n.right_weight : n.left_weight;
            const bool sat = right ? !gl[d] : (gl[d] != 0);
            const uint32_t feat = n.feat;
            float p_old = UNSEEN;
            for (int k = d - 1; k >= 0; k--)
                if (pfeat[k] == feat) {
                    p_old = pe[k];
                    break;
                }
            const float p_e = sat ? (p_old == UNSEEN ? 1.0f / cw : p_old / cw) : 0.0f;
            float cc[QP];
            const float ae = p_e - 1.0f;
#pragma unroll
            for (int i = 0; i < QP; i++) {
                const float m = 1.0f + ae * rn[i];
                cc[i] = c[d][i] * m;
            }
            if (p_old != UNSEEN) {
                const float ao = p_old - 1.0f;
                if (ao != 0.0f) {
#pragma unroll
                    for (int i = 0; i < QP; i++) cc[i] /= 1.0f + ao * rn[i];
                }
            }
            pfeat[d] = feat;
            pe[d] = p_e;
            pold[d] = p_old;
            const float wchild = wprod[d] * cw;
            const ShapNodeDev &cn = nodes[child];
            if (!(cn.flags & 1u)) {
                // descend
                d++;
                nid[d] = child;
                wprod[d] = wchild;
#pragma unroll
                for (int i = 0; i < QP; i++) c[d][i] = cc[i];
                stage[d] = 0;
                gl[d] = shap_goes_left(cn, x[cn.feat], cat_words);
                continue;
            }
            const float ls = wchild * cn.leaf_value;
#pragma unroll
            for (int i = 0; i < QP; i++) {
                const float a = cc[i] * ls;
                ret[i] = a * rw[i];
            }
            // Finish visits upward while frames complete.
            for (;;) {
                // extract_delta (explain.rs:202-217) for the visit of frame d.
                const float pen = pe[d];
                const float px = pold[d] == UNSEEN ? 1.0f : pold[d];
                float acc = 0.0f;
                if (pen != 1.0f) {
                    const float a = pen - 1.0f;
#pragma unroll
                    for (int i = 0; i < QP; i++) {
                        const float num = a * ret[i];
                        const float den = 1.0f + a * rn[i];
                        acc += num / den;
                    }
                }
                if (px != 1.0f) {
                    const float a = px - 1.0f;
#pragma unroll
                    for (int i = 0; i < QP; i++) {
                        const float num = a * ret[i];
                        const float den = 1.0f + a * rn[i];
                        acc -= num / den;
                    }
                }
                if (!INTER) {
                    const uint32_t us = nodes[nid[d]].uslot;
                    tc[us] += acc;
                } else {
                    // Interaction::on_return (explain.rs:281-300): partners are
                    // the newest occurrence of every other feature on the live
                    // path, newest first; the current split is skipped once.
                    const uint32_t f = pfeat[d];
                    float *mrow = p + (uint64_t)f * nc;
                    mrow[f] += acc;
                    bool skipped = false;
                    for (int i = d; i >= 0; i--) {
                        const uint32_t s = pfeat[i];
                        bool shadowed = false;
                        for (int j = i + 1; j <= d; j++)
                            if (pfeat[j] == s) {
                                shadowed = true;
                                break;
                            }
                        if (shadowed) continue;
                        if (!skipped && s == f) {
                            skipped = true;
                            continue;
                        }
                        const float q = pe[i];
                        if (q == 1.0f) continue;  // extract_interaction_delta is 0
                        // extract_interaction_delta (explain.rs:219-247).
                        const float ap = q - 1.0f;
                        const float aen = pen - 1.0f;
                        float ia = 0.0f;
                        if (px == 1.0f) {
#pragma unroll
                            for (int k = 0; k < QP; k++) {
                                const float edge = aen / (1.0f + aen * rn[k]);
                                const float num = ap * ret[k] * edge;
                                ia += num / (1.0f + ap * rn[k]);
                            }
                        } else {
                            const float ax = px - 1.0f;
#pragma unroll
                            for (int k = 0; k < QP; k++) {
                                const float e1 = aen / (1.0f + aen * rn[k]);
                                const float e2 = ax / (1.0f + ax * rn[k]);
                                const float edge = e1 - e2;
                                const float num = ap * ret[k] * edge;
                                ia += num / (1.0f + ap * rn[k]);
                            }
                        }
                        mrow[s] += ia;
                    }
                }
                if (stage[d] == 0) {
#pragma unroll
                    for (int i = 0; i < QP; i++) hl[d][i] = ret[i];
                    stage[d] = 1;
                    break;  // begin the right visit of frame d
                }
#pragma unroll
                for (int i = 0; i < QP; i++) ret[i] = hl[d][i] + ret[i];
                if (d == 0) goto tree_done;
                d--;
            }
        }
    tree_done:
        if (!INTER)
            for (uint32_t u = 0; u < nu; u++) p[ufeats[u0 + u]] += tc[u];
    }
    if (!INTER) {
        p[n_features] += root_mean;
        p[n_features] += margin ? margin[row] : bias;
        return;
    }
    // interaction_row (explain.rs:790-810): bias, symmetrise, then each
    // diagonal entry = its accumulated SHAP value minus the row's interactions.
    const uint64_t b = (uint64_t)n_features * nc + n_features;
    p[b] += root_mean;
    p[b] += margin ? margin[row] : bias;
    for (uint32_t r = 0; r < nc; r++)
        for (uint32_t cidx = r + 1; cidx < nc; cidx++) {
            const float sym = 0.5f * (p[(uint64_t)r * nc + cidx] + p[(uint64_t)cidx * nc + r]);
            p[(uint64_t)r * nc + cidx] = sym;
            p[(uint64_t)cidx * nc + r] = sym;
        }
    for (uint32_t r = 0; r < nc; r++) {
        float value = p[(uint64_t)r * nc + r];
        for (uint32_t cidx = 0; cidx < nc; cidx++)
            if (cidx != r) value -= p[(uint64_t)r * nc + cidx];
        p[(uint64_t)r * nc + r] = value;
    }
}

// The same QuadratureTreeSHAP contributions for trees of at most SHAP_REC_D
// split levels, with the path stack in registers. Every row of a wave visits
// the same nodes in the same order (both children of every split, in
// order), so the recursion below unrolls into straight code over the frames
// (frame D's coefficients, left-subtree return and path entry are locals of
// shap_visit<D>), node loads are uniform across the wave, and only the
// tree's per-feature sums (tc, indexed by the node's unique slot) stay in
// memory. The float operations and their order are shap_kernel's, so the
// results are identical.
constexpr int SHAP_REC_D = 8;

struct ShapPath {
    uint32_t feat[SHAP_REC_D];
    float pe[SHAP_REC_D];
};

// A tree of at most SHAP_REC_D split levels has at most 2^(SHAP_REC_D + 1) - 1
// nodes: one go-left bit each, in words of 32 per lane.
constexpr int SHAP_REC_NODES = 1 << (SHAP_REC_D + 1);
constexpr int SHAP_GL_WORDS = SHAP_REC_NODES / 32;

// What the recursion reads of a node, 16 bytes, staged in LDS per tree:
// meta = left (9 bits) | right << 9 (9 bits) | unique slot << 18 (10 bits) |
// leaf << 31, children as tree-local ids; w0 the left branch weight (a
// leaf: its value), w1 the right branch weight.
struct RecNodeDev {
    uint32_t feat;
    uint32_t meta;
    float w0, w1;
};
constexpr uint32_t REC_LEAF = 1u << 31;

struct ShapRowCtx {
    float rn[QP], rw[QP];
    const RecNodeDev *tn;            // LDS: the tree's nodes, tree-local ids
    const uint32_t (*gl)[SHAP_TPB];  // LDS: go-left bit of node i in word i / 32
};

// A wave-uniform value in a scalar register (every active lane holds it).
__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uni(float v) {
    return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(v)));
}

// Visits internal node `li` (tree-local) at frame D whose incoming
// coefficients are c and path weight wprod; writes the frame's return (left
// + right subtree) to ret.
template <int D>
__device__ __forceinline__ void shap_visit(const ShapRowCtx &R, uint32_t li,
                                           const float (&c)[QP], float wprod, ShapPath &P,
                                           float *tc, float (&ret)[QP]) {
    const RecNodeDev n = R.tn[li];
    const uint32_t feat = uni(n.feat), meta = uni(n.meta);
    const bool gl = (R.gl[li >> 5][threadIdx.x] >> (li & 31)) & 1u;
    float p_old = UNSEEN;  // the newest occurrence of feat on the path above
#pragma unroll
    for (int k = 0; k < D; k++)
        if (P.feat[k] == feat) p_old = P.pe[k];
    const uint32_t uslot = (meta >> 18) & 1023u;
    for (int side = 0; side < 2; side++) {
        const bool right = side != 0;
        const uint32_t child = right ? (meta >> 9) & 511u : meta & 511u;
        const float cw = uni(right ? n.w1 : n.w0);
        const bool sat = right ? !gl : gl;
        const float p_e = sat ? (p_old == UNSEEN ? 1.0f / cw : p_old / cw) : 0.0f;
        float cc[QP];
        const float ae = p_e - 1.0f;
#pragma unroll
        for (int i = 0; i < QP; i++) {
            const float m = 1.0f + ae * R.rn[i];
            cc[i] = c[i] * m;
        }
        if (p_old != UNSEEN) {
            const float ao = p_old - 1.0f;
            if (ao != 0.0f) {
#pragma unroll
                for (int i = 0; i < QP; i++) cc[i] /= 1.0f + ao * R.rn[i];
            }
        }
        P.feat[D] = feat;
        P.pe[D] = p_e;
        const float wchild = wprod * cw;
        const RecNodeDev cn = R.tn[child];
        float r[QP];
        if (!(uni(cn.meta) & REC_LEAF)) {
#pragma unroll
            for (int i = 0; i < QP; i++) r[i] = 0.0f;
            if constexpr (D + 1 < SHAP_REC_D)
                shap_visit<D + 1>(R, child, cc, wchild, P, tc, r);
        } else {
            const float ls = wchild * uni(cn.w0);
#pragma unroll
            for (int i = 0; i < QP; i++) {
                const float a = cc[i] * ls;
                r[i] = a * R.rw[i];
            }
        }
        // extract_delta (explain.rs:202-217) for this visit of frame D. The
        // empty asm keeps the denominators (functions of p_e and p_old alone)
        // from being computed before the subtree and held across it.
        float pe_x = p_e, po_x = p_old;
        asm volatile("" : "+v"(pe_x), "+v"(po_x));
        const float px = po_x == UNSEEN ? 1.0f : po_x;
        float acc = 0.0f;
        if (pe_x != 1.0f) {
            const float a = pe_x - 1.0f;
#pragma unroll
            for (int i = 0; i < QP; i++) {
                const float num = a * r[i];
                const float den = 1.0f + a * R.rn[i];
                acc += num / den;
            }
        }
        if (px != 1.0f) {
            const float a = px - 1.0f;
#pragma unroll
            for (int i = 0; i < QP; i++) {
                const float num = a * r[i];
                const float den = 1.0f + a * R.rn[i];
                acc -= num / den;
            }
        }
        tc[uslot] += acc;
        // The frame's return: the left subtree's, then + the right subtree's
        // (0 + x == x for every x but -0, and a subtree return is never the
        // left operand of anything else).
#pragma unroll
        for (int i = 0; i < QP; i++) ret[i] = right ? ret[i] + r[i] : r[i];
    }
}

// The row's go-left bits of every node of the tree in [root, end) (leaves
// 0), 32 nodes at a time with their loads issued together, so the recursion
// reads no row data. Node fields are wave-uniform.
__device__ __forceinline__ void shap_gl_bits(const ShapNodeDev *__restrict__ nodes,
                                             const uint32_t *__restrict__ cat_words,
                                             const float *x, uint32_t root, uint32_t end,
                                             uint32_t (*gl)[SHAP_TPB]) {
    for (uint32_t w = 0; root + 32 * w < end; w++) {
        const uint32_t b = root + 32 * w;
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const uint32_t id = min(b + j, end - 1);
            const uint32_t fl = uni(nodes[id].flags);
            const uint32_t f = (fl & 1u) ? 0u : uni(nodes[id].feat);
            v[j] = x[f];
        }
        uint32_t bits = 0;
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const uint32_t id = min(b + j, end - 1);
            const ShapNodeDev &n = nodes[id];
            if (b + j < end && !(uni(n.flags) & 1u) && shap_goes_left(n, v[j], cat_words))
                bits |= 1u << j;
        }
        gl[w][threadIdx.x] = bits;
    }
}

template <int MAXU>
__global__ __launch_bounds__(SHAP_TPB) void shap_rec_kernel(
    const ShapNodeDev *__restrict__ nodes, const RecNodeDev *__restrict__ rec,
    const uint32_t *__restrict__ tree_roots,
    uint32_t n_trees, uint32_t n_nodes, const uint32_t *__restrict__ tree_ufeat_off,
    const uint32_t *__restrict__ ufeats, const uint32_t *__restrict__ cat_words,
    const float *__restrict__ rule, const float *__restrict__ rows, uint64_t n_rows,
    uint32_t n_features, const float *__restrict__ margin, float bias, float root_mean,
    float *__restrict__ out) {
    __shared__ uint32_t glw[SHAP_GL_WORDS][SHAP_TPB];
    __shared__ RecNodeDev tn[SHAP_REC_NODES];
    // Every thread takes part in the per-tree staging (barriers); a thread
    // past the last row computes on the last row and writes nothing.
    const uint64_t row0 = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool active = row0 < n_rows;
    const uint64_t row = active ? row0 : n_rows - 1;
    const float *x = rows + row * n_features;
    ShapRowCtx R;
    R.tn = tn;
    R.gl = glw;
#pragma unroll
    for (int i = 0; i < QP; i++) {
        R.rn[i] = rule[i];
        R.rw[i] = rule[QP + i];
    }
    const uint32_t nc = n_features + 1;
    float *p = out + row * (uint64_t)nc;
    if (active)
        for (uint32_t f = 0; f <= n_features; f++) p[f] = 0.0f;
    float tc[MAXU];
    ShapPath P;
    for (uint32_t t = 0; t < n_trees; t++) {
        const uint32_t root = uni(tree_roots[t]);
        const uint32_t end = t + 1 < n_trees ? tree_roots[t + 1] : n_nodes;
        if (nodes[root].flags & 1u) continue;  // a leaf-only tree contributes nothing
        const uint32_t u0 = tree_ufeat_off[t], nu = tree_ufeat_off[t + 1] - u0;
        __syncthreads();  // every wave is done with the previous tree's nodes
        for (uint32_t i = threadIdx.x; i < end - root; i += SHAP_TPB) tn[i] = rec[root + i];
        for (uint32_t u = 0; u < nu; u++) tc[u] = 0.0f;
        shap_gl_bits(nodes, cat_words, x, root, end, glw);
        __syncthreads();
        float c0[QP], ret[QP];
#pragma unroll
        for (int i = 0; i < QP; i++) c0[i] = 1.0f;
        shap_visit<0>(R, 0u, c0, 1.0f, P, tc, ret);
        if (active)
            for (uint32_t u = 0; u < nu; u++) p[ufeats[u0 + u]] += tc[u];
    }
    if (!active) return;
    p[n_features] += root_mean;
    p[n_features] += margin ? margin[row] : bias;
}

// ====================================================================== host

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
    uint32_t n_trees = 0, n_features = 0, max_unique = 1, max_depth = 1, n_nodes = 0;
    uint32_t max_tree_nodes = 0;
    float bias = 0.0f, root_mean = 0.0f;
    std::string cover_error;  // non-empty: TreeSHAP is undefined for this model
    ShapNodeDev *d_nodes = nullptr;
    RecNodeDev *d_rec = nullptr;
    PredNodeDev *d_pred = nullptr;
    float *d_means = nullptr;
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

// Cover-weighted mean leaf value in f64 (root_mean, src/model/explain.rs:424-438).
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

// Cover-weighted mean of every node in f32 (fill_node_means,
// src/model/explain.rs:409-422).
float node_means(const std::vector<int32_t> &left, const std::vector<int32_t> &right,
                 const std::vector<float> &leaf, const std::vector<float> &hess,
                 const std::vector<uint8_t> &is_leaf, uint32_t base, uint32_t idx,
                 std::vector<float> &means) {
    const uint32_t g = base + idx;
    float value;
    if (is_leaf[g]) {
        value = leaf[g];
    } else {
        const uint32_t l = (uint32_t)left[g], r = (uint32_t)right[g];
        float result = node_means(left, right, leaf, hess, is_leaf, base, l, means) * hess[base + l];
        result += node_means(left, right, leaf, hess, is_leaf, base, r, means) * hess[base + r];
        value = result / hess[g];
    }
    means[g] = value;
    return value;
}

hipError_t launch_shap(const fbh_shap_model *m, bool inter, const float *rows, uint64_t n_rows,
                       const float *margin, float *out) {
    if (n_rows == 0) return hipSuccess;
    if (m->max_depth > SHAP_MAXD) return hipErrorInvalidValue;
    const uint32_t blocks = (uint32_t)((n_rows + SHAP_TPB - 1) / SHAP_TPB);
    if (inter) {
        hipLaunchKernelGGL((shap_kernel<1, true>), dim3(blocks), dim3(SHAP_TPB), 0, m->stream,
                           m->d_nodes, m->d_roots, m->n_trees, m->d_uoff, m->d_ufeats, m->d_cats,
                           m->d_rule, rows, n_rows, m->n_features, margin, m->bias, m->root_mean,
                           out);
        return hipGetLastError();
    }
#define FBH_SHAP_REC_CASE(U)                                                                     \
    if (m->max_unique <= U) {                                                                    \
        hipLaunchKernelGGL((shap_rec_kernel<U>), dim3(blocks), dim3(SHAP_TPB), 0, m->stream,      \
                           m->d_nodes, m->d_rec, m->d_roots, m->n_trees, m->n_nodes, m->d_uoff, \
                           m->d_ufeats,                                                          \
                           m->d_cats, m->d_rule, rows, n_rows, m->n_features, margin, m->bias,  \
                           m->root_mean, out);                                                   \
        return hipGetLastError();                                                               \
    }
    if (m->max_depth <= SHAP_REC_D && m->max_tree_nodes <= (uint32_t)SHAP_REC_NODES) {
        FBH_SHAP_REC_CASE(32) FBH_SHAP_REC_CASE(64) FBH_SHAP_REC_CASE(128) FBH_SHAP_REC_CASE(256)
        FBH_SHAP_REC_CASE(1024)
    }
#undef FBH_SHAP_REC_CASE
#define FBH_SHAP_CASE(U)                                                                         \
    if (m->max_unique <= U) {                                                                    \
        hipLaunchKernelGGL((shap_kernel<U, false>), dim3(blocks), dim3(SHAP_TPB), 0, m->stream,   \
                           m->d_nodes, m->d_roots, m->n_trees, m->d_uoff, m->d_ufeats,          \
                           m->d_cats, m->d_rule, rows, n_rows, m->n_features, margin, m->bias,  \
                           m->root_mean, out);                                                   \
        return hipGetLastError();                                                               \
    }
    FBH_SHAP_CASE(32) FBH_SHAP_CASE(64) FBH_SHAP_CASE(128) FBH_SHAP_CASE(256)
    FBH_SHAP_CASE(1024)
#undef FBH_SHAP_CASE
    return hipErrorInvalidValue;
}

// What one explanation or prediction call computes.
enum class Kind { Contribs, Interactions, Saabas, Margin, Value, Leaf };

uint64_t out_width(const fbh_shap_model *m, Kind k) {
    const uint64_t nc = (uint64_t)m->n_features + 1;
    switch (k) {
        case Kind::Contribs:
        case Kind::Saabas: return nc;
        case Kind::Interactions: return nc * nc;
        case Kind::Leaf: return m->n_trees;
        default: return 1;
    }
}

void check_kind(const fbh_shap_model *m, Kind k) {
    if (k == Kind::Contribs || k == Kind::Interactions) {
        if (!m->cover_error.empty()) throw ShapError(FBH_INPUT_ERROR, m->cover_error);
    }
    if (k == Kind::Contribs || k == Kind::Interactions || k == Kind::Saabas) {
        if (m->max_depth > SHAP_MAXD)
            throw ShapError(FBH_INPUT_ERROR,
                            "trees deeper than 16 splits cannot be explained on the device");
    }
}

// Enqueues one kind over device-resident rows on the model's stream.
void enqueue(fbh_shap_model *m, Kind k, const float *d_rows, uint64_t n, const float *d_margin,
             float *d_out) {
    if (n == 0) return;
    const uint32_t blocks = (uint32_t)((n + PRED_TPB - 1) / PRED_TPB);
    switch (k) {
        case Kind::Contribs:
            chk(launch_shap(m, false, d_rows, n, d_margin, d_out), "shap launch");
            return;
        case Kind::Interactions:
            chk(launch_fill_f32(d_out, 0.0f, n * out_width(m, k), m->stream), "interaction clear");
            chk(launch_shap(m, true, d_rows, n, d_margin, d_out), "interaction launch");
            return;
        case Kind::Saabas:
            hipLaunchKernelGGL(saabas_kernel, dim3(blocks), dim3(PRED_TPB), 0, m->stream, m->d_pred,
                               m->d_nodes, m->d_cats, m->d_means, m->d_roots, m->n_trees, d_rows,
                               n, m->n_features, d_margin, m->bias, d_out);
            chk(hipGetLastError(), "saabas launch");
            return;
        default: {
            const uint32_t mode = k == Kind::Leaf ? PRED_LEAF
                                  : k == Kind::Value ? PRED_SIGMOID : PRED_MARGIN;
            const uint32_t nf = m->n_features;
            const char *kind_env = std::getenv("FB_HIP_PREDICT_KERNEL");
            const int pk = kind_env ? std::atoi(kind_env) : 4;
            if (pk == 4 && nf >= 1 && nf <= PRED_LDS4_MAX_F) {
                const uint32_t lb = (uint32_t)((n + PRED_LDS_ROWS - 1) / PRED_LDS_ROWS);
                hipLaunchKernelGGL(predict_lds4_kernel, dim3(lb), dim3(PRED_LDS_ROWS * PRED_WAVES),
                                   (size_t)PRED_LDS_ROWS * ((nf | 1u) + PRED_RUN) * 4, m->stream,
                                   m->d_pred, m->d_nodes, m->d_cats, m->d_roots, m->n_trees,
                                   d_rows, n, nf, d_margin, m->bias, mode, d_out);
            } else if (pk >= 1 && nf >= 1 && nf <= PRED_LDS_MAX_F) {
                const uint32_t lb = (uint32_t)((n + PRED_LDS_ROWS - 1) / PRED_LDS_ROWS);
                hipLaunchKernelGGL(predict_lds_kernel, dim3(lb), dim3(PRED_LDS_ROWS),
                                   (size_t)PRED_LDS_ROWS * (nf | 1u) * 4, m->stream, m->d_pred,
                                   m->d_nodes, m->d_cats, m->d_roots, m->n_trees, d_rows, n, nf,
                                   d_margin, m->bias, mode, d_out);
            } else {
                hipLaunchKernelGGL(predict_kernel, dim3(blocks), dim3(PRED_TPB), 0, m->stream,
                                   m->d_pred, m->d_nodes, m->d_cats, m->d_roots, m->n_trees, d_rows,
                                   n, nf, d_margin, m->bias, mode, d_out);
            }
            chk(hipGetLastError(), "predict launch");
            return;
        }
    }
}

// Device staging of one host call: rows, base margins and outputs of up to
// cap_rows rows.
struct Staging {
    float *rows = nullptr, *margin = nullptr, *out = nullptr;
    uint64_t cap_rows = 0;
};

// Runs one kind over host rows through `st`, batch after batch, and times the
// kernels with the model's events.
void run_host(fbh_shap_model *m, Kind k, const Staging &st, const float *rows, uint64_t n_rows,
              const float *margin, float *out) {
    const uint64_t w = out_width(m, k), nf = m->n_features;
    double kernel_ms = 0.0;
    for (uint64_t r0 = 0; r0 < n_rows; r0 += st.cap_rows) {
        const uint64_t b = std::min(st.cap_rows, n_rows - r0);
        chk(hipMemcpyAsync(st.rows, rows + r0 * nf, 4 * b * nf, hipMemcpyHostToDevice, m->stream),
            "rows upload");
        if (margin)
            chk(hipMemcpyAsync(st.margin, margin + r0, 4 * b, hipMemcpyHostToDevice, m->stream),
                "margin upload");
        chk(hipEventRecord(m->e0, m->stream), "event");
        enqueue(m, k, st.rows, b, margin ? st.margin : nullptr, st.out);
        chk(hipEventRecord(m->e1, m->stream), "event");
        chk(hipMemcpyAsync(out + r0 * w, st.out, 4 * b * w, hipMemcpyDeviceToHost, m->stream),
            "output download");
        chk(hipStreamSynchronize(m->stream), "explain");
        float ms = 0.0f;
        chk(hipEventElapsedTime(&ms, m->e0, m->e1), "event");
        kernel_ms += ms;
    }
    m->last_ms = kernel_ms;
}

// Host call with staging buffers allocated for the call: batches of at most
// 512 MiB of inputs and outputs (GpuExplainModel::compute batching,
// src/backend/cuda/explain.rs:491-560).
void run_host_alloc(fbh_shap_model *m, Kind k, const float *rows, uint64_t n_rows,
                    const float *margin, float *out) {
    if (!m || (!rows && n_rows) || (!out && n_rows)) throw ShapError(FBH_INPUT_ERROR, "null argument");
    check_kind(m, k);
    if (n_rows == 0) return;
    chk(hipSetDevice(m->device), "hipSetDevice");
    const uint64_t w = out_width(m, k);
    const uint64_t per_row = 4ull * (m->n_features + 1 + w);
    Staging st;
    st.cap_rows = std::min<uint64_t>(n_rows, std::max<uint64_t>(1, (512ull << 20) / per_row));
    chk(hipMalloc(&st.rows, 4 * st.cap_rows * m->n_features + 4), "staging rows");
    std::unique_ptr<float, decltype(&hipFree)> f1(st.rows, hipFree);
    chk(hipMalloc(&st.out, 4 * st.cap_rows * w + 4), "staging output");
    std::unique_ptr<float, decltype(&hipFree)> f2(st.out, hipFree);
    if (margin) chk(hipMalloc(&st.margin, 4 * st.cap_rows), "staging margin");
    std::unique_ptr<float, decltype(&hipFree)> f3(st.margin, hipFree);
    run_host(m, k, st, rows, n_rows, margin, out);
}

// ------------------------------------------------ the no-allocation scratch
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)FBH_NOALLOC_SCRATCH_BYTES;
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[MAX_DEVICES] = {};

// The device's scratch address; the device must be current.
void *scratch_of(int device) {
    if (device < 0 || device >= MAX_DEVICES) throw ShapError(FBH_INPUT_ERROR, "device index out of range");
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *p = nullptr;
        chk(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!p) throw ShapError(FBH_RUNTIME_ERROR, "hipGetSymbolAddress(scratch) returned null");
        g_scratch_ptr[device] = p;
    }
    return g_scratch_ptr[device];
}

uint64_t round256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

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
        if (n_features > PN_FEAT)
            throw ShapError(FBH_INPUT_ERROR, "models with more than 2^29 - 1 features are not supported");
        if (n_trees && (!feat || !split_cond || !left || !right || !default_left || !is_leaf ||
                        !leaf_value || !sum_hess))
            throw ShapError(FBH_INPUT_ERROR, "null argument");
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
        std::vector<RecNodeDev> rec(total);
        std::vector<PredNodeDev> pred(total);
        std::vector<float> means(total, 0.0f);
        std::vector<uint32_t> roots(n_trees), uoff(n_trees + 1, 0), ufeats;
        double rm_sum = 0.0;
        for (uint32_t t = 0; t < n_trees; t++) {
            const uint32_t b = tree_offsets[t], e = tree_offsets[t + 1];
            if (e <= b) throw ShapError(FBH_INPUT_ERROR, "tree " + std::to_string(t) + " has no nodes");
            m->max_tree_nodes = std::max(m->max_tree_nodes, e - b);
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
                PredNodeDev &pn = pred[i];
                pn.ff = is_leaf[i] ? PN_LEAF : (feat[i] | (default_left[i] ? PN_DEFAULT_LEFT : 0u) |
                                                (d.cat_len ? PN_CAT : 0u));
                pn.value = is_leaf[i] ? leaf_value[i] : split_cond[i];
                pn.left = pn.right = -1;
                if (!is_leaf[i]) {
                    if (feat[i] >= n_features)
                        throw ShapError(FBH_INPUT_ERROR, "split feature out of range");
                    const int32_t l = left[i], r = right[i];
                    if (l <= 0 || r <= 0 || (uint32_t)l >= e - b || (uint32_t)r >= e - b ||
                        (uint32_t)l <= i - b || (uint32_t)r <= i - b)
                        throw ShapError(FBH_INPUT_ERROR, "child ids must follow their parent");
                    // check_covers (src/model/explain.rs:440-457): TreeSHAP only.
                    if (m->cover_error.empty()) {
                        if (hs[i] < 0.0f || hs[b + l] < 0.0f || hs[b + r] < 0.0f)
                            m->cover_error = "tree " + std::to_string(t) +
                                             " has a negative cover (sum_hessian) at a split: SHAP is undefined";
                        else if (std::isnan(hs[i]) || std::isnan(hs[b + l]) || std::isnan(hs[b + r]))
                            m->cover_error = "tree " + std::to_string(t) +
                                             " has a NaN cover (sum_hessian): SHAP is undefined";
                    }
                    d.left = (int32_t)(b + l);
                    d.right = (int32_t)(b + r);
                    pn.left = d.left;
                    pn.right = d.right;
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
                RecNodeDev &q = rec[i];
                q.feat = d.feat;
                if (is_leaf[i]) {
                    q.meta = REC_LEAF;
                    q.w0 = d.leaf_value;
                } else {  // packed only where the tree fits (max_tree_nodes)
                    q.meta = ((uint32_t)(d.left - (int32_t)b) & 511u) |
                             (((uint32_t)(d.right - (int32_t)b) & 511u) << 9) |
                             ((d.uslot & 1023u) << 18);
                    q.w0 = d.left_weight;
                    q.w1 = d.right_weight;
                }
            }
            m->max_unique = std::max<uint32_t>(m->max_unique, (uint32_t)ufeats.size() - uoff[t]);
            if (m->max_unique > MAX_SHAP_UNIQUE)
                throw ShapError(FBH_INPUT_ERROR, "a tree splits on more than " +
                                                     std::to_string(MAX_SHAP_UNIQUE) +
                                                     " distinct features");
            rm_sum += root_mean(L, R, lv, hs, lf, b, 0);
            node_means(L, R, lv, hs, lf, b, 0, means);
        }
        uoff[n_trees] = (uint32_t)ufeats.size();
        float rule[16];
        quadrature_rule(rule, rule + 8);
        std::vector<float> rv(rule, rule + 16);
        std::vector<uint32_t> cw(cat_words ? cat_words : nullptr,
                                 cat_words ? cat_words + n_cat_words : nullptr);
        m->n_trees = n_trees;
        m->n_features = n_features;
        m->n_nodes = total;
        m->bias = bias;
        m->root_mean = (float)rm_sum;
        m->d_nodes = m->upload(nodes, "shap nodes");
        m->d_rec = m->upload(rec, "shap node records");
        m->d_pred = m->upload(pred, "walk nodes");
        m->d_means = m->upload(means, "node means");
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
        check_kind(m, Kind::Contribs);
        chk(hipSetDevice(m->device), "hipSetDevice");
        chk(hipEventRecord(m->e0, m->stream), "event");
        enqueue(m, Kind::Contribs, d_rows, n_rows, d_margin, d_out);
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
    return shap_guard([&] { run_host_alloc(m, Kind::Contribs, rows, n_rows, margin, out); });
}

int fbh_shap_interactions(fbh_shap_model *m, const float *rows, uint64_t n_rows,
                          const float *margin, float *out) {
    return shap_guard([&] { run_host_alloc(m, Kind::Interactions, rows, n_rows, margin, out); });
}

int fbh_saabas_contribs(fbh_shap_model *m, const float *rows, uint64_t n_rows,
                        const float *margin, float *out) {
    return shap_guard([&] { run_host_alloc(m, Kind::Saabas, rows, n_rows, margin, out); });
}

int fbh_predict(fbh_shap_model *m, const float *rows, uint64_t n_rows, const float *margin,
                uint32_t output, float *out) {
    return shap_guard([&] {
        if (output > FBH_PREDICT_LEAF) throw ShapError(FBH_INPUT_ERROR, "unknown prediction output");
        const Kind k = output == FBH_PREDICT_LEAF ? Kind::Leaf
                       : output == FBH_PREDICT_SIGMOID ? Kind::Value : Kind::Margin;
        run_host_alloc(m, k, rows, n_rows, k == Kind::Leaf ? nullptr : margin, out);
    });
}

int fbh_predict_device(fbh_shap_model *m, const float *d_rows, uint64_t n_rows,
                       const float *d_margin, uint32_t output, float *d_out, int sync) {
    return shap_guard([&] {
        if (!m || (!d_rows && n_rows) || (!d_out && n_rows))
            throw ShapError(FBH_INPUT_ERROR, "null argument");
        if (output > FBH_PREDICT_LEAF) throw ShapError(FBH_INPUT_ERROR, "unknown prediction output");
        const Kind k = output == FBH_PREDICT_LEAF ? Kind::Leaf
                       : output == FBH_PREDICT_SIGMOID ? Kind::Value : Kind::Margin;
        chk(hipSetDevice(m->device), "hipSetDevice");
        chk(hipEventRecord(m->e0, m->stream), "event");
        enqueue(m, k, d_rows, n_rows, k == Kind::Leaf ? nullptr : d_margin, d_out);
        chk(hipEventRecord(m->e1, m->stream), "event");
        if (sync) {
            chk(hipStreamSynchronize(m->stream), "predict");
            float ms = 0.0f;
            chk(hipEventElapsedTime(&ms, m->e0, m->e1), "event");
            m->last_ms = ms;
        }
    });
}

int fbh_shap_contribs_noalloc(fbh_shap_model *m, const float *rows, uint64_t n_rows,
                              const float *margin, float *out) {
    return shap_guard([&] {
        if (!m || (!rows && n_rows) || (!out && n_rows))
            throw ShapError(FBH_INPUT_ERROR, "null argument");
        check_kind(m, Kind::Contribs);
        const uint64_t nf = m->n_features, w = nf + 1;
        // Layout of one batch in the scratch: rows [b][nf], margins [b],
        // contributions [b][nf + 1], each region 256-byte aligned.
        const uint64_t per_row = 4 * (nf + 1 + w);
        const uint64_t room = NOALLOC_SCRATCH_BYTES - 3 * 256;
        const uint64_t cap = room / per_row;
        if (cap == 0)
            throw ShapError(FBH_INPUT_ERROR,
                            "fbh_shap_contribs_noalloc: one row of " + std::to_string(nf) +
                                " features needs " + std::to_string(per_row) +
                                " bytes of device scratch, above its " +
                                std::to_string(NOALLOC_SCRATCH_BYTES) + " bytes");
        if (n_rows == 0) return;
        chk(hipSetDevice(m->device), "hipSetDevice");
        unsigned char *base = static_cast<unsigned char *>(scratch_of(m->device));
        Staging st;
        st.cap_rows = std::min<uint64_t>(cap, n_rows);
        st.rows = reinterpret_cast<float *>(base);
        st.margin = reinterpret_cast<float *>(base + round256(4 * st.cap_rows * nf));
        st.out = reinterpret_cast<float *>(reinterpret_cast<unsigned char *>(st.margin) +
                                           round256(4 * st.cap_rows));
        if ((reinterpret_cast<unsigned char *>(st.out) - base) + 4 * st.cap_rows * w >
            NOALLOC_SCRATCH_BYTES)
            throw ShapError(FBH_RUNTIME_ERROR, "fbh_shap_contribs_noalloc: scratch layout overflow");
        run_host(m, Kind::Contribs, st, rows, n_rows, margin, out);
    });
}

}  // extern "C"
