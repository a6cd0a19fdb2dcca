// fbt_json.cpp -- model load from XGBoost-schema JSON
// (Model::from_xgboost_json, src/model/tree.rs:754-990, 1259-1470).
//
// A small recursive-descent JSON reader builds a document tree; the model is
// then read field by field with the reference's checks and messages: gbtree
// only, one output, scalar leaves, no forests, trees whose children,
// parents, categories and features are consistent. Numbers of float arrays
// are read as doubles and rounded to f32 (as serde_json deserialises an f32:
// f64 first, then `as f32`); the string parameters XGBoost writes
// ("base_score": "5E-1") are parsed straight to f32, as Rust's str::parse.

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <map>
#include <memory>
#include <string>

#include "fbt_internal.h"

namespace fbt {
namespace {

struct JVal {
    enum Type { Null, Bool, Num, Str, Arr, Obj } t = Null;
    bool b = false;
    std::string s;  // string value, or the number's text
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;

    const JVal *get(const char *key) const {
        if (t != Obj) return nullptr;
        for (const auto &kv : o)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

InputError bad(const std::string &m) { return InputError("invalid model JSON: " + m); }

class Parser {
  public:
    Parser(const char *p, size_t n) : p_(p), e_(p + n) {}
    JVal document() {
        JVal v = value(0);
        ws();
        if (p_ != e_) throw bad("trailing characters after the document");
        return v;
    }

  private:
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    char peek() {
        ws();
        if (p_ >= e_) throw bad("unexpected end of input");
        return *p_;
    }
    void expect(char c) {
        if (peek() != c) throw bad(std::string("expected '") + c + "' at offset " + offset());
        p_++;
    }
    std::string offset() const { return std::to_string(p_ - b_); }

    JVal value(int depth) {
        if (depth > 64) throw bad("nesting deeper than 64 levels");
        const char c = peek();
        JVal v;
        if (c == '{') {
            v.t = JVal::Obj;
            p_++;
            if (peek() == '}') {
                p_++;
                return v;
            }
            for (;;) {
                if (peek() != '"') throw bad("expected a key at offset " + offset());
                std::string k = string();
                expect(':');
                v.o.emplace_back(std::move(k), value(depth + 1));
                const char d = peek();
                p_++;
                if (d == '}') break;
                if (d != ',') throw bad("expected ',' or '}' at offset " + offset());
            }
        } else if (c == '[') {
            v.t = JVal::Arr;
            p_++;
            if (peek() == ']') {
                p_++;
                return v;
            }
            for (;;) {
                v.a.push_back(value(depth + 1));
                const char d = peek();
                p_++;
                if (d == ']') break;
                if (d != ',') throw bad("expected ',' or ']' at offset " + offset());
            }
        } else if (c == '"') {
            v.t = JVal::Str;
            v.s = string();
        } else if (c == 't' || c == 'f' || c == 'n') {
            const char *w = c == 't' ? "true" : c == 'f' ? "false" : "null";
            const size_t n = std::strlen(w);
            if ((size_t)(e_ - p_) < n || std::strncmp(p_, w, n) != 0)
                throw bad("invalid literal at offset " + offset());
            p_ += n;
            v.t = c == 'n' ? JVal::Null : JVal::Bool;
            v.b = c == 't';
        } else {
            v.t = JVal::Num;
            const char *s = p_;
            if (p_ < e_ && *p_ == '-') p_++;
            while (p_ < e_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' ||
                               *p_ == 'E' || *p_ == '+' || *p_ == '-'))
                p_++;
            if (p_ == s) throw bad("unexpected character at offset " + offset());
            v.s.assign(s, p_);
        }
        return v;
    }

    std::string string() {
        expect('"');
        std::string out;
        while (true) {
            if (p_ >= e_) throw bad("unterminated string");
            const char c = *p_++;
            if (c == '"') break;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p_ >= e_) throw bad("unterminated escape");
            const char x = *p_++;
            switch (x) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    if (e_ - p_ < 4) throw bad("short \\u escape");
                    const unsigned cp = (unsigned)std::strtoul(std::string(p_, 4).c_str(), nullptr, 16);
                    p_ += 4;
                    // Names are kept as UTF-8; surrogate pairs are not combined.
                    if (cp < 0x80) out.push_back((char)cp);
                    else if (cp < 0x800) {
                        out.push_back((char)(0xC0 | (cp >> 6)));
                        out.push_back((char)(0x80 | (cp & 0x3F)));
                    } else {
                        out.push_back((char)(0xE0 | (cp >> 12)));
                        out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
                        out.push_back((char)(0x80 | (cp & 0x3F)));
                    }
                    break;
                }
                default: throw bad("invalid escape");
            }
        }
        return out;
    }

    const char *p_;
    const char *e_;
    const char *b_ = p_;
};

const JVal &req(const JVal &v, const char *key, const char *where) {
    const JVal *r = v.get(key);
    if (!r) throw bad(std::string("missing field `") + key + "` in " + where);
    return *r;
}

const std::string &str(const JVal &v, const char *what) {
    if (v.t != JVal::Str) throw bad(std::string(what) + " must be a string");
    return v.s;
}

// An integer JSON number of the type T (serde rejects fractions and overflow).
template <class T>
T int_of(const JVal &v, const char *what) {
    if (v.t != JVal::Num) throw bad(std::string(what) + " must hold integers");
    errno = 0;
    char *end = nullptr;
    const long long x = std::strtoll(v.s.c_str(), &end, 10);
    if (errno || *end != 0 || x < (long long)std::numeric_limits<T>::min() ||
        x > (long long)std::numeric_limits<T>::max())
        throw bad(std::string(what) + ": invalid integer " + v.s);
    return (T)x;
}

// An f32 JSON number (serde: parsed as f64, then rounded to f32).
float f32_of(const JVal &v, const char *what) {
    if (v.t != JVal::Num) throw bad(std::string(what) + " must hold numbers");
    char *end = nullptr;
    const double d = std::strtod(v.s.c_str(), &end);
    if (*end != 0) throw bad(std::string(what) + ": invalid number " + v.s);
    return (float)d;
}

template <class T, class F>
std::vector<T> array_of(const JVal *v, const char *what, F conv, bool optional) {
    std::vector<T> out;
    if (!v) {
        if (optional) return out;
        throw bad(std::string("missing field `") + what + "`");
    }
    if (v->t != JVal::Arr) throw bad(std::string(what) + " must be an array");
    out.reserve(v->a.size());
    for (const JVal &x : v->a) out.push_back(conv(x, what));
    return out;
}

std::string trim(const std::string &s) {
    size_t b = 0, e = s.size();
    while (b < e && std::isspace((unsigned char)s[b])) b++;
    while (e > b && std::isspace((unsigned char)s[e - 1])) e--;
    return s.substr(b, e - b);
}

// parse_param (src/model/tree.rs:1081-1088): Rust's str::parse of a trimmed
// string parameter.
long long param_int(const std::string &name, const std::string &raw) {
    const std::string t = trim(raw);
    errno = 0;
    char *end = nullptr;
    const long long x = std::strtoll(t.c_str(), &end, 10);
    if (t.empty() || errno || *end != 0)
        throw bad("cannot parse value \"" + raw + "\" of parameter " + name);
    return x;
}

float param_f32(const std::string &name, const std::string &raw) {
    const std::string t = trim(raw);
    char *end = nullptr;
    const float x = std::strtof(t.c_str(), &end);
    const bool hex = t.find('x') != std::string::npos || t.find('X') != std::string::npos;
    if (t.empty() || *end != 0 || hex)
        throw bad("cannot parse value \"" + raw + "\" of parameter " + name);
    return x;
}

// The comma-separated parts of "a", "[a]" or "[a,b,c]".
std::vector<std::string> base_score_parts(const std::string &raw) {
    std::string t = trim(raw);
    if (t.size() >= 2 && t.front() == '[' && t.back() == ']') t = t.substr(1, t.size() - 2);
    std::vector<std::string> parts;
    size_t s = 0;
    while (s <= t.size()) {
        size_t c = t.find(',', s);
        if (c == std::string::npos) c = t.size();
        const std::string p = trim(t.substr(s, c - s));
        if (!p.empty()) parts.push_back(p);
        s = c + 1;
    }
    if (parts.empty()) throw bad("base_score is empty: \"" + raw + "\"");
    return parts;
}

// parse_base_score (src/model/tree.rs:1060-1079): "5E-1" or "[5E-1]".
float parse_base_score(const std::string &raw) {
    const std::vector<std::string> parts = base_score_parts(raw);
    if (parts.size() > 1)
        throw bad("base_score is a vector (\"" + raw + "\"); multi-target models are not supported");
    return param_f32("base_score", parts[0]);
}

// parse_base_score_vector (src/model/tree.rs:1033-1050): a multiclass
// model's intercepts "[a,b,c]" (or a scalar).
std::vector<float> parse_base_score_vector(const std::string &raw) {
    std::vector<float> v;
    for (const std::string &p : base_score_parts(raw)) v.push_back(param_f32("base_score", p));
    return v;
}

// quantile_alphas_from_json (src/training/objective.rs:1015-1036):
// quantile_loss_param.quantile_alpha as XGBoost's string "[0.1,0.5]" (also
// "0.9", "(0.9)", "[1E-1,5E-1]"), a number, or an array of numbers; 1 to 64
// values (QuantileAlphas::new, src/types.rs:700-712). Empty when absent or
// unreadable.
std::vector<float> quantile_alphas_from_json(const JVal &obj) {
    const JVal *blk = obj.get("quantile_loss_param");
    const JVal *raw = blk ? blk->get("quantile_alpha") : nullptr;
    if (!raw) return {};
    std::vector<float> v;
    auto number = [](const std::string &text, float &out) {
        const std::string t = trim(text);
        char *end = nullptr;
        out = std::strtof(t.c_str(), &end);
        const bool hex = t.find('x') != std::string::npos || t.find('X') != std::string::npos;
        return !t.empty() && *end == 0 && !hex;
    };
    if (raw->t == JVal::Str) {
        std::string t = trim(raw->s);
        size_t b = 0, e = t.size();
        while (b < e && (t[b] == '[' || t[b] == '(')) b++;
        while (e > b && (t[e - 1] == ']' || t[e - 1] == ')')) e--;
        t = t.substr(b, e - b);
        size_t s0 = 0;
        while (true) {
            const size_t c = t.find(',', s0);
            float x;
            if (!number(t.substr(s0, c == std::string::npos ? std::string::npos : c - s0), x))
                return {};
            v.push_back(x);
            if (c == std::string::npos) break;
            s0 = c + 1;
        }
    } else if (raw->t == JVal::Num) {
        v.push_back((float)std::strtod(raw->s.c_str(), nullptr));
    } else if (raw->t == JVal::Arr) {
        for (const JVal &x : raw->a) {
            if (x.t != JVal::Num) return {};
            v.push_back((float)std::strtod(x.s.c_str(), nullptr));
        }
    } else {
        return {};
    }
    if (v.size() > 64) return {};
    return v;
}

constexpr int32_t NO_CHILD = -1;

// xgb::Tree::to_tree (src/model/tree.rs:1259-1470).
Tree read_tree(const JVal &t) {
    const JVal *idv = t.get("id");
    const std::string id = idv && idv->t == JVal::Num ? idv->s : "?";
    const JVal &tp = req(t, "tree_param", "tree");
    const size_t n_features = (size_t)param_int(
        "tree_param.num_feature", str(req(tp, "num_feature", "tree_param"), "num_feature"));
    auto left = array_of<int32_t>(t.get("left_children"), "left_children", int_of<int32_t>, false);
    auto right = array_of<int32_t>(t.get("right_children"), "right_children", int_of<int32_t>, false);
    auto cond = array_of<float>(t.get("split_conditions"), "split_conditions", f32_of, false);
    auto idx = array_of<uint32_t>(t.get("split_indices"), "split_indices", int_of<uint32_t>, false);
    auto dl = array_of<uint8_t>(t.get("default_left"), "default_left", int_of<uint8_t>, false);
    auto stype = array_of<uint8_t>(t.get("split_type"), "split_type", int_of<uint8_t>, true);
    auto loss = array_of<float>(t.get("loss_changes"), "loss_changes", f32_of, false);
    auto hess = array_of<float>(t.get("sum_hessian"), "sum_hessian", f32_of, false);
    (void)array_of<float>(t.get("base_weights"), "base_weights", f32_of, false);
    (void)array_of<int32_t>(t.get("parents"), "parents", int_of<int32_t>, false);
    auto cats = array_of<int32_t>(t.get("categories"), "categories", int_of<int32_t>, true);
    auto cnodes = array_of<int32_t>(t.get("categories_nodes"), "categories_nodes", int_of<int32_t>, true);
    auto csegs = array_of<int32_t>(t.get("categories_segments"), "categories_segments", int_of<int32_t>, true);
    auto csizes = array_of<int32_t>(t.get("categories_sizes"), "categories_sizes", int_of<int32_t>, true);
    const size_t n = left.size();
    const std::string tn = "tree " + id;
    if (n == 0) throw bad(tn + " has no root node");
    const std::pair<const char *, size_t> lens[] = {{"right_children", right.size()},
                                                    {"split_conditions", cond.size()},
                                                    {"split_indices", idx.size()},
                                                    {"default_left", dl.size()}};
    for (const auto &l : lens)
        if (l.second != n)
            throw bad(tn + ": " + l.first + " length " + std::to_string(l.second) +
                      " does not match node count " + std::to_string(n));
    if (!stype.empty() && stype.size() != n)
        throw bad(tn + ": split_type length " + std::to_string(stype.size()) +
                  " does not match node count " + std::to_string(n));
    for (uint8_t s : stype)
        if (s > 1)
            throw bad(tn + ": unknown split_type = " + std::to_string(s) +
                      " (0 = numerical, 1 = categorical)");
    if (csegs.size() != cnodes.size() || csizes.size() != cnodes.size())
        throw bad(tn + ": categories_nodes / segments / sizes have different lengths");
    std::map<size_t, std::vector<uint32_t>> cat_of;
    for (size_t k = 0; k < cnodes.size(); k++) {
        const int32_t node = cnodes[k];
        const int64_t b = csegs[k], sz = csizes[k];
        if (b < 0 || sz < 0 || (uint64_t)(b + sz) > cats.size())
            throw bad(tn + ": category segment [" + std::to_string(b) + ", +" + std::to_string(sz) +
                      ") is out of bounds, categories has " + std::to_string(cats.size()) +
                      " entries");
        if (node < 0 || (size_t)node >= n || (size_t)node >= stype.size() || stype[node] != 1)
            throw bad(tn + ": categories_nodes contains " + std::to_string(node) +
                      ", which is not a categorical split node");
        uint32_t mx = 0;
        for (int64_t i = b; i < b + sz; i++) {
            if (cats[i] < 0)
                throw bad(tn + ": node " + std::to_string(node) + " contains a negative category value");
            if (cats[i] >= (1 << 24))
                throw bad(tn + ": node " + std::to_string(node) +
                          " contains a category value above 2^24");
            mx = std::max(mx, (uint32_t)cats[i]);
        }
        // words_from_categories (src/data/categorical.rs:193-200).
        std::vector<uint32_t> words(mx / 32 + 1, 0u);
        for (int64_t i = b; i < b + sz; i++) words[(uint32_t)cats[i] / 32] |= 1u << ((uint32_t)cats[i] % 32);
        if (!cat_of.emplace((size_t)node, std::move(words)).second)
            throw bad(tn + ": node " + std::to_string(node) +
                      " appears more than once in categories_nodes");
    }
    for (size_t i = 0; i < stype.size(); i++)
        if (stype[i] == 1 && !cat_of.count(i))
            throw bad(tn + ": node " + std::to_string(i) +
                      " is a categorical split but has no category segment");
    Tree tree;
    tree.nodes.resize(n);
    std::vector<uint8_t> parents(n, 0);
    for (size_t i = 0; i < n; i++) {
        Node &nd = tree.nodes[i];
        const int32_t l = left[i], r = right[i];
        if (l == NO_CHILD) {
            if (r != NO_CHILD)
                throw bad(tn + ": node " + std::to_string(i) + " has only one child: " +
                          std::to_string(l) + " / " + std::to_string(r));
            nd.is_leaf = true;
            nd.leaf_value = cond[i];
            nd.sum_hess = i < hess.size() ? hess[i] : 0.0f;
            continue;
        }
        if (l < 0 || r < 0 || (size_t)l >= n || (size_t)r >= n || l == r)
            throw bad(tn + ": node " + std::to_string(i) + " has invalid child indices: " +
                      std::to_string(l) + " / " + std::to_string(r));
        for (int32_t ch : {l, r})
            if (++parents[(size_t)ch] > 1)
                throw bad(tn + ": node " + std::to_string(ch) + " has multiple parents");
        if (idx[i] >= n_features)
            throw bad(tn + ": node " + std::to_string(i) + " feature " + std::to_string(idx[i]) +
                      " is out of range for " + std::to_string(n_features) + " features");
        nd.is_leaf = false;
        nd.feat = idx[i];
        nd.split_cond = cond[i];
        nd.left = l;
        nd.right = r;
        nd.default_left = dl[i] != 0;
        nd.leaf_value = 0.0f;
        nd.gain = i < loss.size() ? loss[i] : 0.0f;
        nd.sum_hess = i < hess.size() ? hess[i] : 0.0f;
        auto it = cat_of.find(i);
        if (it != cat_of.end()) nd.cats = std::move(it->second);
    }
    if (parents[0] != 0) throw bad(tn + ": the root node is referenced by another node");
    std::vector<uint8_t> seen(n, 0);
    std::vector<size_t> stack{0};
    while (!stack.empty()) {
        const size_t i = stack.back();
        stack.pop_back();
        if (seen[i]) throw bad(tn + " contains a cycle");
        seen[i] = 1;
        if (!tree.nodes[i].is_leaf) {
            stack.push_back((size_t)tree.nodes[i].left);
            stack.push_back((size_t)tree.nodes[i].right);
        }
    }
    for (size_t i = 0; i < n; i++)
        if (!seen[i]) throw bad(tn + ": node " + std::to_string(i) + " is unreachable from the root");
    return tree;
}

}  // namespace

Model model_from_json(const char *text, size_t len) {
    Parser ps(text, len);
    const JVal doc = ps.document();
    if (doc.t != JVal::Obj) throw bad("the document is not an object");
    const JVal &learner = req(doc, "learner", "document");
    const JVal &booster = req(learner, "gradient_booster", "learner");
    const std::string &bname = str(req(booster, "name", "gradient_booster"), "gradient_booster.name");
    if (bname != "gbtree") throw bad("only gbtree is supported, this model is " + bname);
    const JVal &mp = req(learner, "learner_model_param", "learner");
    const JVal &obj = req(learner, "objective", "learner");
    const std::string &oname = str(req(obj, "name", "objective"), "objective.name");
    Model m;
    if (oname == "binary:logistic") m.objective = 1;
    else if (oname == "reg:squarederror") m.objective = 0;
    else if (oname == "multi:softprob") m.objective = 2;
    else if (oname == "multi:softmax") m.objective = 3;
    else if (oname == "reg:quantileerror") m.objective = 4;
    else
        throw bad("objective " + oname +
                  " is not supported; supported: binary:logistic, reg:squarederror, "
                  "multi:softprob, multi:softmax, reg:quantileerror");
    if (m.objective == 4) {
        m.quantile_alpha = quantile_alphas_from_json(obj);
        if (m.quantile_alpha.empty())
            throw bad("objective reg:quantileerror has no readable "
                      "quantile_loss_param.quantile_alpha");
    }
    const long long ncp = param_int("num_class", str(req(mp, "num_class", "learner_model_param"), "num_class"));
    const size_t num_class_param = (size_t)std::max(ncp, 1ll);
    size_t num_target = 1;
    if (const JVal *nt = mp.get("num_target")) {
        const std::string &s = str(*nt, "num_target");
        if (!trim(s).empty()) num_target = (size_t)std::max(param_int("num_target", s), 1ll);
    }
    // Several targets only as a multi-quantile model, one target per alpha
    // (src/model/tree.rs:793-802).
    if (num_target > 1 && !(m.objective == 4 && m.quantile_alpha.size() > 1 &&
                            num_target == m.quantile_alpha.size()))
        throw bad("multi-target models are not supported (num_target = " +
                  std::to_string(num_target) +
                  "); only reg:quantileerror with multiple quantile_alpha is supported");
    const size_t num_class = std::max(num_class_param, num_target);
    const JVal &model = req(booster, "model", "gradient_booster");
    auto tree_info = array_of<int32_t>(model.get("tree_info"), "tree_info", int_of<int32_t>, false);
    for (size_t i = 0; i < tree_info.size(); i++)
        if ((size_t)tree_info[i] != i % num_class)
            throw bad("tree " + std::to_string(i) + " has tree_info = " +
                      std::to_string(tree_info[i]) + ", not " + std::to_string(i) +
                      " % num_class (" + std::to_string(num_class) +
                      "); this output group layout is not supported");
    const JVal &trees = req(model, "trees", "model");
    if (trees.t != JVal::Arr) throw bad("trees must be an array");
    for (const JVal &t : trees.a) {
        const JVal &tp = req(t, "tree_param", "tree");
        const std::string leaf = trim(str(req(tp, "size_leaf_vector", "tree_param"), "size_leaf_vector"));
        if (!leaf.empty() && param_int("size_leaf_vector", leaf) > 1) {
            const JVal *idv = t.get("id");
            throw bad("tree " + (idv ? idv->s : std::string("?")) +
                      " has vector leaves (size_leaf_vector = " + leaf +
                      "); only scalar leaves are supported");
        }
    }
    const JVal &gp = req(model, "gbtree_model_param", "model");
    const std::string &npt = str(req(gp, "num_parallel_tree", "gbtree_model_param"), "num_parallel_tree");
    if (param_int("num_parallel_tree", npt) != 1)
        throw bad("num_parallel_tree = " + npt + " (random forest mode) is not supported");
    // num_class must match the objective's outputs (src/model/tree.rs:838-845).
    const size_t outputs = m.objective == 4 ? m.quantile_alpha.size() : 0;
    const bool multi = m.objective == 2 || m.objective == 3 || outputs > 1;
    if (m.objective == 4 ? num_class != outputs : multi ? num_class < 2 : num_class != 1)
        throw bad("num_class = " + std::to_string(num_class) + " is inconsistent with objective " + oname);
    const long long nf = param_int("num_feature", str(req(mp, "num_feature", "learner_model_param"), "num_feature"));
    if (nf < 0 || nf > 0xFFFFFFFFll) throw bad("num_feature out of range");
    m.n_features = (uint32_t)nf;
    const std::string &bs_raw = str(req(mp, "base_score", "learner_model_param"), "base_score");
    if (multi) {
        // The intercepts: a vector of num_class values, or a scalar copied
        // to every class (parse_base_score_vector, src/model/tree.rs:846-862).
        std::vector<float> v = parse_base_score_vector(bs_raw);
        if (v.size() == 1) v.assign(num_class, v[0]);
        if (v.size() != num_class)
            throw bad("base_score has " + std::to_string(v.size()) + " values, but num_class = " +
                      std::to_string(num_class));
        m.class_margins = v;
        m.base_score = v[0];
    } else {
        m.base_score = parse_base_score(bs_raw);
    }
    for (const JVal &t : trees.a) m.trees.push_back(read_tree(t));
    // A split feature past the model's feature count would read past a row
    // (CpuInferenceTree::new, src/model/inference.rs:50-62, refuses it).
    for (size_t t = 0; t < m.trees.size(); t++)
        for (const Node &nd : m.trees[t].nodes)
            if (!nd.is_leaf && nd.feat >= m.n_features)
                throw bad("tree " + std::to_string(t) + " contains out-of-range feature " +
                          std::to_string(nd.feat) + " (the model has " +
                          std::to_string(m.n_features) + " features)");
    // feature_types: "c" marks a categorical feature.
    m.cuts.categorical.assign(m.n_features, 0);
    m.cuts.offsets.assign((size_t)m.n_features + 1, 0);
    if (const JVal *ft = learner.get("feature_types")) {
        if (ft->t != JVal::Arr) throw bad("feature_types must be an array");
        bool any = false;
        for (const JVal &x : ft->a)
            if (x.t == JVal::Str && x.s == "c") any = true;
        if (any) {
            if (ft->a.size() != m.n_features)
                throw bad("feature_types has " + std::to_string(ft->a.size()) +
                          " entries, but the model has " + std::to_string(m.n_features) +
                          " features");
            for (size_t f = 0; f < ft->a.size(); f++)
                m.cuts.categorical[f] = ft->a[f].t == JVal::Str && ft->a[f].s == "c";
        }
    }
    // scale_pos_weight_from_json (src/training/objective.rs:851-853).
    m.scale_pos_weight = 1.0f;
    if (const JVal *blk = obj.get("reg_loss_param"))
        if (const JVal *v = blk->get("scale_pos_weight")) {
            if (v->t == JVal::Str) {
                char *end = nullptr;
                const std::string t = trim(v->s);
                const float x = std::strtof(t.c_str(), &end);
                if (!t.empty() && *end == 0) m.scale_pos_weight = x;
            } else if (v->t == JVal::Num) {
                m.scale_pos_weight = (float)std::strtod(v->s.c_str(), nullptr);
            }
        }
    return m;
}

}  // namespace fbt
