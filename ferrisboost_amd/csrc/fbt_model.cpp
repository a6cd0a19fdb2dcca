// fbt_model.cpp -- trees, margins and the XGBoost-schema model JSON
// (src/model/tree.rs:52-290, 486-510, 600-760, 1093-1290).

#include <charconv>
#include <cmath>
#include <cstring>
#include <string>

#include "fbt_internal.h"

namespace fbt {

uint32_t Tree::push_leaf(float value, float hess) {
    Node n;
    n.leaf_value = value;
    n.sum_hess = hess;
    nodes.push_back(n);
    return (uint32_t)nodes.size() - 1;
}

std::pair<uint32_t, uint32_t> Tree::split_leaf(uint32_t node, uint32_t feat, float cond,
                                               bool default_left, float gain, float lv, float lh,
                                               float rv, float rh) {
    const uint32_t l = push_leaf(lv, lh);
    const uint32_t r = push_leaf(rv, rh);
    Node &n = nodes[node];
    n.feat = feat;
    n.split_cond = cond;
    n.left = (int32_t)l;
    n.right = (int32_t)r;
    n.default_left = default_left;
    n.leaf_value = 0.0f;
    n.is_leaf = false;
    n.gain = gain;
    return {l, r};
}

void Tree::set_categories(uint32_t node, const uint64_t *w64, uint32_t n64) {
    std::vector<uint32_t> words;
    for (uint32_t i = 0; i < 2 * n64; i++) words.push_back((uint32_t)(w64[i / 2] >> (32 * (i % 2))));
    while (!words.empty() && words.back() == 0) words.pop_back();
    nodes[node].cats = std::move(words);
    // XGBoost's placeholder condition of a categorical split: f32::from_bits(1).
    const uint32_t one = 1;
    std::memcpy(&nodes[node].split_cond, &one, 4);
}

// Node::goes_left + categorical::goes_left (src/data/categorical.rs).
static bool goes_left(const Node &n, float v) {
    if (std::isnan(v)) return n.default_left;
    if (!n.cats.empty()) {
        if (v < 0.0f || v >= 16777216.0f) return true;
        const uint32_t cat = (uint32_t)v;
        const uint32_t word = cat / 32;
        if (word >= n.cats.size()) return true;
        return ((n.cats[word] >> (cat % 32)) & 1u) == 0;
    }
    return v < n.split_cond;
}

float Tree::leaf_value(const float *x) const {
    if (nodes.empty()) return 0.0f;
    uint32_t i = 0;
    for (;;) {
        const Node &n = nodes[i];
        if (n.is_leaf) return n.leaf_value;
        i = goes_left(n, x[n.feat]) ? (uint32_t)n.left : (uint32_t)n.right;
    }
}

// Objective::base_margin (src/training/objective.rs:363-398).
float base_margin_of(uint32_t objective, float bs) {
    if (objective == 1) {
        const float eps = 1e-6f;
        const float x = std::min(std::max(bs, eps), 1.0f - eps);
        return -std::log(1.0f / x - 1.0f);
    }
    return bs;
}

float Model::base_margin() const { return base_margin_of(objective, base_score); }

namespace {

// serde_json's f32 formatting (the shortest round-trip digits, rendered the
// way the ryu crate's `format_finite` renders them).
std::string json_f32(float v) {
    if (!std::isfinite(v)) return "null";
    char sci[64];
    auto res = std::to_chars(sci, sci + sizeof(sci), v, std::chars_format::scientific);
    std::string s(sci, res.ptr);
    bool neg = false;
    if (!s.empty() && s[0] == '-') {
        neg = true;
        s.erase(0, 1);
    }
    const size_t epos = s.find('e');
    std::string mant = s.substr(0, epos);
    const int e10 = std::stoi(s.substr(epos + 1));
    std::string digits;
    for (char ch : mant)
        if (ch != '.') digits.push_back(ch);
    while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
    const int length = (int)digits.size();
    const int kk = e10 + 1;        // 10^(kk-1) <= v < 10^kk
    const int k = kk - length;     // v = digits * 10^k
    std::string out = neg ? "-" : "";
    if (digits == "0") return out + "0.0";
    if (0 <= k && kk <= 16) {
        out += digits + std::string(k, '0') + ".0";
    } else if (0 < kk && kk <= 16) {
        out += digits.substr(0, kk) + "." + digits.substr(kk);
    } else if (-5 < kk && kk <= 0) {
        out += "0." + std::string(-kk, '0') + digits;
    } else if (length == 1) {
        out += digits + "e" + std::to_string(kk - 1);
    } else {
        out += digits.substr(0, 1) + "." + digits.substr(1) + "e" + std::to_string(kk - 1);
    }
    return out;
}

// Rust's Display of f32 (`to_string`): shortest digits, never an exponent.
std::string display_f32(float v) {
    if (std::isnan(v)) return "NaN";
    if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
    char sci[64];
    auto res = std::to_chars(sci, sci + sizeof(sci), v, std::chars_format::scientific);
    std::string s(sci, res.ptr);
    bool neg = false;
    if (!s.empty() && s[0] == '-') {
        neg = true;
        s.erase(0, 1);
    }
    const size_t epos = s.find('e');
    std::string mant = s.substr(0, epos);
    const int e10 = std::stoi(s.substr(epos + 1));
    std::string digits;
    for (char ch : mant)
        if (ch != '.') digits.push_back(ch);
    while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
    std::string out = neg ? "-" : "";
    if (digits == "0") return out + "0";
    const int point = e10 + 1;  // digits before the decimal point
    if (point <= 0) return out + "0." + std::string(-point, '0') + digits;
    if (point >= (int)digits.size()) return out + digits + std::string(point - digits.size(), '0');
    return out + digits.substr(0, point) + "." + digits.substr(point);
}

template <class T, class F>
void json_array(std::string &o, const std::vector<T> &v, F fmt) {
    o += '[';
    for (size_t i = 0; i < v.size(); i++) {
        if (i) o += ',';
        o += fmt(v[i]);
    }
    o += ']';
}

}  // namespace

std::string model_to_json(const Model &m) {
    std::string o;
    o.reserve(1024 + m.trees.size() * 4096);
    const bool any_cat = [&] {
        for (uint8_t c : m.cuts.categorical)
            if (c) return true;
        return false;
    }();
    o += "{\"version\":[2,0,0],\"learner\":{\"attributes\":{},\"feature_names\":[],";
    o += "\"feature_types\":[";
    if (any_cat)
        for (uint32_t f = 0; f < m.n_features; f++) {
            if (f) o += ',';
            o += m.cuts.categorical[f] ? "\"c\"" : "\"q\"";
        }
    o += "],\"gradient_booster\":{\"name\":\"gbtree\",\"model\":{";
    const size_t nt = m.trees.size();
    // K trees a round (multiclass): indptr steps by K, the last round may be
    // short; tree i belongs to output i % K (src/model/tree.rs:689-699).
    const size_t K = m.n_outputs();
    o += "\"gbtree_model_param\":{\"num_trees\":\"" + std::to_string(nt) +
         "\",\"num_parallel_tree\":\"1\"},\"iteration_indptr\":[";
    for (size_t i = 0; i < nt; i += K) {
        if (i) o += ',';
        o += std::to_string(i);
    }
    if (nt) o += ',';
    o += std::to_string(nt);
    o += "],\"tree_info\":[";
    for (size_t i = 0; i < nt; i++) {
        if (i) o += ',';
        o += std::to_string(i % K);
    }
    o += "],\"trees\":[";
    auto i32s = [](int32_t v) { return std::to_string(v); };
    for (size_t t = 0; t < nt; t++) {
        const Tree &tr = m.trees[t];
        const size_t n = tr.nodes.size();
        std::vector<float> base(n), loss(n), cond(n), hess(n);
        std::vector<int32_t> left(n), right(n), parents(n, 2147483647), cats, cnodes, csegs, csizes;
        std::vector<uint32_t> idx(n);
        std::vector<int32_t> dl(n), stype(n, 0);
        for (size_t i = 0; i < n; i++) {
            const Node &nd = tr.nodes[i];
            left[i] = nd.left;
            right[i] = nd.right;
            dl[i] = nd.default_left ? 1 : 0;
            loss[i] = nd.gain;
            hess[i] = nd.sum_hess;
            if (nd.is_leaf) {
                cond[i] = nd.leaf_value;
                idx[i] = 0;
                base[i] = nd.leaf_value;
            } else {
                cond[i] = nd.split_cond;
                idx[i] = nd.feat;
                base[i] = 0.0f;
                parents[(size_t)nd.left] = (int32_t)i;
                parents[(size_t)nd.right] = (int32_t)i;
                if (!nd.cats.empty()) {
                    stype[i] = 1;
                    cnodes.push_back((int32_t)i);
                    csegs.push_back((int32_t)cats.size());
                    int32_t count = 0;
                    for (size_t w = 0; w < nd.cats.size(); w++)
                        for (uint32_t b = 0; b < 32; b++)
                            if ((nd.cats[w] >> b) & 1u) {
                                cats.push_back((int32_t)(w * 32 + b));
                                count++;
                            }
                    csizes.push_back(count);
                }
            }
        }
        if (t) o += ',';
        o += "{\"base_weights\":";
        json_array(o, base, json_f32);
        o += ",\"categories\":";
        json_array(o, cats, i32s);
        o += ",\"categories_nodes\":";
        json_array(o, cnodes, i32s);
        o += ",\"categories_segments\":";
        json_array(o, csegs, i32s);
        o += ",\"categories_sizes\":";
        json_array(o, csizes, i32s);
        o += ",\"default_left\":";
        json_array(o, dl, i32s);
        o += ",\"id\":" + std::to_string(t) + ",\"left_children\":";
        json_array(o, left, i32s);
        o += ",\"loss_changes\":";
        json_array(o, loss, json_f32);
        o += ",\"parents\":";
        json_array(o, parents, i32s);
        o += ",\"right_children\":";
        json_array(o, right, i32s);
        o += ",\"split_conditions\":";
        json_array(o, cond, json_f32);
        o += ",\"split_indices\":";
        json_array(o, idx, [](uint32_t v) { return std::to_string(v); });
        o += ",\"split_type\":";
        json_array(o, stype, i32s);
        o += ",\"sum_hessian\":";
        json_array(o, hess, json_f32);
        o += ",\"tree_param\":{\"num_deleted\":\"0\",\"num_feature\":\"" +
             std::to_string(m.n_features) + "\",\"num_nodes\":\"" + std::to_string(n) +
             "\",\"size_leaf_vector\":\"1\"}}";
    }
    // base_score: the scalar before the link, or a multiclass model's
    // intercepts as XGBoost's vector "[a,b,c]" (src/model/tree.rs:700-733).
    std::string bs;
    if (m.class_margins.empty()) {
        bs = display_f32(m.base_score);
    } else {
        bs = "[";
        for (size_t k = 0; k < m.class_margins.size(); k++) {
            if (k) bs += ',';
            bs += display_f32(m.class_margins[k]);
        }
        bs += "]";
    }
    // A multiclass model writes num_class; several quantiles are targets:
    // num_class 0, num_target K (src/model/tree.rs:720-732).
    const bool multi = m.objective == 2 || m.objective == 3;
    const bool quantile = m.objective == 4;
    o += "]}},\"learner_model_param\":{\"base_score\":\"" + bs +
         "\",\"boost_from_average\":\"1\",\"num_class\":\"" +
         (multi ? std::to_string(K) : std::string("0")) + "\",\"num_feature\":\"" +
         std::to_string(m.n_features) + "\",\"num_target\":\"" +
         (quantile ? std::to_string(K) : std::string("1")) + "\"},";
    o += "\"objective\":{\"name\":\"";
    static const char *const names[] = {"reg:squarederror", "binary:logistic", "multi:softprob",
                                        "multi:softmax", "reg:quantileerror"};
    o += names[m.objective <= 4 ? m.objective : 0];
    // Objective::json_params (src/training/objective.rs:772-822): the
    // quantiles as XGBoost's ParamArray string "[a,b,c]".
    if (quantile) {
        std::string qa = "[";
        for (size_t k = 0; k < m.quantile_alpha.size(); k++) {
            if (k) qa += ',';
            qa += display_f32(m.quantile_alpha[k]);
        }
        o += "\",\"quantile_loss_param\":{\"quantile_alpha\":\"" + qa + "]\"}}}}";
    } else if (multi)
        o += "\",\"softmax_multiclass_param\":{\"num_class\":\"" + std::to_string(K) + "\"}}}}";
    else
        o += "\",\"reg_loss_param\":{\"scale_pos_weight\":\"" +
             display_f32(m.scale_pos_weight) + "\"}}}}";
    return o;
}

}  // namespace fbt
