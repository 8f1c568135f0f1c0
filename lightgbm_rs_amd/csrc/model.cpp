// model.cpp — LightGBM v4 model text -> host trees -> flattened device arrays.
//
// Parsing follows the reference loader: header keys up to the first `Tree=` line
// (model_text.rs:48-160: num_class, num_tree_per_iteration (defaults to num_class),
// max_feature_idx, objective), then one key=value block per tree, ended by a blank
// line (Tree::parse, tree.rs:846-1060: num_leaves, num_cat, leaf_value; for more
// than one leaf split_feature, threshold, left_child, right_child, decision_type
// (default 0); cat_boundaries / cat_threshold when num_cat > 0), until `end of
// trees`.  Objective names and parameters as objective.rs:125-225.  Every index the
// device follows is checked here: children in range and forming one tree reachable
// from node 0, split features within max_feature_idx, categorical bitset indices
// within the tree's bitsets; linear trees are rejected.
#include "model.h"

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <map>

bool check_tree(const HostTree& t, int32_t max_feature_idx, std::string* err);

namespace {

std::atomic<uint64_t> g_model_uid{1};

bool fail(std::string* err, const std::string& m) {
  *err = m;
  return false;
}

bool parse_f64s(const std::string& v, std::vector<double>* out, const char* name, std::string* err) {
  out->clear();
  const char* p = v.c_str();
  while (*p) {
    while (*p == ' ') ++p;
    if (!*p) break;
    char* end = nullptr;
    errno = 0;
    const double x = std::strtod(p, &end);
    if (end == p) return fail(err, std::string("bad float in ") + name);
    out->push_back(x);
    p = end;
  }
  return true;
}

template <typename T>
bool parse_ints(const std::string& v, std::vector<T>* out, const char* name, std::string* err) {
  out->clear();
  const char* p = v.c_str();
  while (*p) {
    while (*p == ' ') ++p;
    if (!*p) break;
    char* end = nullptr;
    errno = 0;
    const long long x = std::strtoll(p, &end, 10);
    if (end == p || errno == ERANGE) return fail(err, std::string("bad integer in ") + name);
    out->push_back((T)x);
    p = end;
  }
  return true;
}

bool parse_int(const std::string& v, int32_t* out, const char* name, std::string* err) {
  std::vector<long long> xs;
  if (!parse_ints(v, &xs, name, err)) return false;
  if (xs.size() != 1 || xs[0] < INT32_MIN || xs[0] > INT32_MAX)
    return fail(err, std::string("bad scalar ") + name);
  *out = (int32_t)xs[0];
  return true;
}

bool parse_objective(const std::string& line, lgbm_hip_model* m, std::string* err) {
  std::vector<std::string> tok;
  size_t i = 0;
  while (i < line.size()) {
    while (i < line.size() && line[i] == ' ') ++i;
    size_t j = i;
    while (j < line.size() && line[j] != ' ') ++j;
    if (j > i) tok.push_back(line.substr(i, j - i));
    i = j;
  }
  if (tok.empty()) return fail(err, "empty objective= line");
  m->objective_outputs = 1;
  bool sqrt_ = false, have_nc = false;
  int32_t nc = 0;
  for (size_t k = 1; k < tok.size(); ++k) {
    if (tok[k] == "sqrt") {
      sqrt_ = true;
      continue;
    }
    const size_t c = tok[k].find(':');
    if (c == std::string::npos) continue;
    const std::string key = tok[k].substr(0, c), val = tok[k].substr(c + 1);
    if (key == "sigmoid") {
      char* end = nullptr;
      m->sigmoid = std::strtod(val.c_str(), &end);
      if (end == val.c_str() || *end) return fail(err, "objective sigmoid: not a float");
    } else if (key == "num_class") {
      if (!parse_int(val, &nc, "num_class", err)) return false;
      have_nc = true;
    }
  }
  const std::string& n = tok[0];
  if (n == "regression" || n == "regression_l2" || n == "regression_l1" ||
      n == "mean_squared_error" || n == "mse" || n == "l2" || n == "mean_absolute_error" ||
      n == "mae" || n == "l1") {
    m->objective = sqrt_ ? OBJ_REGRESSION_SQRT : OBJ_REGRESSION;
  } else if (n == "binary") {
    if (!(m->sigmoid > 0.0)) return fail(err, "binary sigmoid must be > 0");
    m->objective = OBJ_BINARY;
  } else if (n == "multiclass" || n == "softmax") {
    if (!have_nc || nc < 1) return fail(err, "multiclass objective must contain num_class >= 1");
    m->objective = OBJ_MULTICLASS;
    m->objective_outputs = nc;
  } else if (n == "multiclassova" || n == "multiclass_ova" || n == "ova" || n == "ovr") {
    if (!have_nc || nc < 1) return fail(err, "multiclassova objective must contain num_class >= 1");
    if (!(m->sigmoid > 0.0)) return fail(err, "multiclassova sigmoid must be > 0");
    m->objective = OBJ_MULTICLASS_OVA;
    m->objective_outputs = nc;
  } else if (n == "poisson" || n == "gamma" || n == "tweedie") {
    m->objective = OBJ_EXP;
  } else if (n == "cross_entropy" || n == "xentropy") {
    m->objective = OBJ_XENTROPY;
  } else if (n == "cross_entropy_lambda" || n == "xentlambda") {
    m->objective = OBJ_XENTLAMBDA;
  } else {
    return fail(err, "objective '" + n + "' is not supported");
  }
  return true;
}

bool parse_tree(const std::map<std::string, std::string>& kv, int32_t max_feature_idx,
                HostTree* t, std::string* err) {
  auto get = [&](const char* k) -> const std::string* {
    auto it = kv.find(k);
    return it == kv.end() ? nullptr : &it->second;
  };
  const std::string* s;
  if (!(s = get("num_leaves"))) return fail(err, "tree without num_leaves");
  if (!parse_int(*s, &t->num_leaves, "num_leaves", err)) return false;
  if (!(s = get("num_cat"))) return fail(err, "tree without num_cat");
  if (!parse_int(*s, &t->num_cat, "num_cat", err)) return false;
  if (t->num_leaves < 1) return fail(err, "num_leaves must be >= 1");
  if (t->num_cat < 0) return fail(err, "num_cat must be >= 0");
  if ((s = get("is_linear"))) {
    int32_t lin = 0;
    if (!parse_int(*s, &lin, "is_linear", err)) return false;
    t->is_linear = lin != 0;
  }
  if (t->is_linear) {  // parse_linear_model (tree.rs:1341-1412), also for one-leaf trees
    if (!(s = get("leaf_const"))) return fail(err, "linear tree model should contain leaf_const field");
    if (!parse_f64s(*s, &t->leaf_const, "leaf_const", err)) return false;
    if (!(s = get("num_features"))) return fail(err, "linear tree model should contain num_features field");
    if (!parse_ints(*s, &t->leaf_nfeat, "num_features", err)) return false;
    if ((s = get("leaf_features")) && !parse_ints(*s, &t->leaf_features, "leaf_features", err))
      return false;
    if ((s = get("leaf_coeff")) && !parse_f64s(*s, &t->leaf_coeff, "leaf_coeff", err)) return false;
  }
  if (!(s = get("leaf_value"))) return fail(err, "tree model should contain leaf_value field");
  if (!parse_f64s(*s, &t->leaf_value, "leaf_value", err)) return false;
  if ((int64_t)t->leaf_value.size() != t->num_leaves) return fail(err, "leaf_value length");
  const int32_t ni = t->num_leaves - 1;
  // metadata (optional; the reference's defaults)
  auto meta_f64 = [&](const char* k, std::vector<double>* v, int32_t n) -> bool {
    if ((s = get(k))) {
      if (!parse_f64s(*s, v, k, err)) return false;
      if ((int32_t)v->size() != n) return fail(err, std::string(k) + " length");
    } else {
      v->assign(n, 0.0);
    }
    return true;
  };
  auto meta_i32 = [&](const char* k, std::vector<int32_t>* v, int32_t n) -> bool {
    if ((s = get(k))) {
      if (!parse_ints(*s, v, k, err)) return false;
      if ((int32_t)v->size() != n) return fail(err, std::string(k) + " length");
    } else {
      v->assign(n, 0);
    }
    return true;
  };
  // A constant tree's leaf_weight line is empty in the C++ writer's output; kept so.
  const std::string* lw = get("leaf_weight");
  if (t->num_leaves == 1 && lw && lw->find_first_not_of(' ') == std::string::npos) {
    t->leaf_weight.clear();
  } else if (!meta_f64("leaf_weight", &t->leaf_weight, t->num_leaves)) {
    return false;
  }
  if (!meta_i32("leaf_count", &t->leaf_count, t->num_leaves)) return false;
  if ((s = get("shrinkage"))) {
    std::vector<double> v;
    if (!parse_f64s(*s, &v, "shrinkage", err)) return false;
    if (v.size() != 1) return fail(err, "bad scalar shrinkage");
    t->shrinkage = v[0];
  }
  if (t->num_leaves == 1) return true;
  if (!meta_f64("internal_value", &t->internal_value, ni)) return false;
  if (!meta_f64("internal_weight", &t->internal_weight, ni)) return false;
  if (!meta_i32("internal_count", &t->internal_count, ni)) return false;
  {
    std::vector<double> g;
    if (!meta_f64("split_gain", &g, ni)) return false;
    t->split_gain.assign(g.begin(), g.end());
  }
  if (!(s = get("split_feature"))) return fail(err, "tree without split_feature");
  if (!parse_ints(*s, &t->split_feature, "split_feature", err)) return false;
  if (!(s = get("threshold"))) return fail(err, "tree model should contain threshold field");
  if (!parse_f64s(*s, &t->threshold, "threshold", err)) return false;
  if (!(s = get("left_child"))) return fail(err, "tree without left_child");
  if (!parse_ints(*s, &t->left_child, "left_child", err)) return false;
  if (!(s = get("right_child"))) return fail(err, "tree without right_child");
  if (!parse_ints(*s, &t->right_child, "right_child", err)) return false;
  if ((s = get("decision_type"))) {
    if (!parse_ints(*s, &t->decision_type, "decision_type", err)) return false;
  } else {
    t->decision_type.assign(ni, 0);
  }
  if ((int32_t)t->split_feature.size() != ni || (int32_t)t->threshold.size() != ni ||
      (int32_t)t->left_child.size() != ni || (int32_t)t->right_child.size() != ni ||
      (int32_t)t->decision_type.size() != ni)
    return fail(err, "internal node array length != num_leaves - 1");
  if (t->num_cat > 0) {
    if (!(s = get("cat_boundaries"))) return fail(err, "tree model should contain cat_boundaries field");
    if (!parse_ints(*s, &t->cat_boundaries, "cat_boundaries", err)) return false;
    if ((int32_t)t->cat_boundaries.size() != t->num_cat + 1) return fail(err, "cat_boundaries length");
    if (!(s = get("cat_threshold"))) return fail(err, "tree model should contain cat_threshold field");
    if (!parse_ints(*s, &t->cat_threshold, "cat_threshold", err)) return false;
    if ((int64_t)t->cat_threshold.size() != (int64_t)t->cat_boundaries.back())
      return fail(err, "cat_threshold length");
    for (int32_t i = 0; i < t->num_cat; ++i)
      if (t->cat_boundaries[i] < 0 || t->cat_boundaries[i] > t->cat_boundaries[i + 1])
        return fail(err, "cat_boundaries not ascending");
  }
  return check_tree(*t, max_feature_idx, err);
}

void flatten_tree(lgbm_hip_model* m, const HostTree& t) {
  PredTree pt;
  pt.node0 = (int32_t)m->nodes.size();
  pt.leaf0 = (int32_t)m->leaf_values.size();
  pt.cat0 = (int32_t)m->cat_bounds.size();
  pt.num_leaves = t.num_leaves;
  pt.lin0 = -1;
  if (t.is_linear) {
    pt.lin0 = (int32_t)m->lin_leaves.size();
    int32_t off = (int32_t)m->lin_features.size();
    for (int32_t l = 0; l < t.num_leaves; ++l) {
      m->lin_leaves.push_back(PredLinLeaf{t.leaf_const[l], off, t.leaf_nfeat[l]});
      off += t.leaf_nfeat[l];
    }
    m->lin_features.insert(m->lin_features.end(), t.leaf_features.begin(), t.leaf_features.end());
    m->lin_coeffs.insert(m->lin_coeffs.end(), t.leaf_coeff.begin(), t.leaf_coeff.end());
  }
  m->tree_index.push_back(pt);
  m->any_linear = m->any_linear || t.is_linear;
  // Tree::expected_value (tree.rs:351-361) and the depth of Tree::max_depth (tree.rs:367-386)
  double ev = t.leaf_value[0];
  int32_t depth = 0;
  if (t.num_leaves > 1) {
    const double total = (double)t.internal_count[0];
    ev = 0.0;
    for (int32_t i = 0; i < t.num_leaves; ++i)
      ev += ((double)t.leaf_count[i] / total) * t.leaf_value[i];
    std::vector<std::pair<int32_t, int32_t>> stack{{0, 0}};
    while (!stack.empty()) {
      const auto [n, d] = stack.back();
      stack.pop_back();
      if (n < 0) {
        depth = std::max(depth, d);
      } else {
        stack.push_back({t.left_child[n], d + 1});
        stack.push_back({t.right_child[n], d + 1});
      }
    }
    for (int32_t i = 0; i + 1 < t.num_leaves; ++i) m->node_cover.push_back((double)t.internal_count[i]);
  }
  for (int32_t i = 0; i < t.num_leaves; ++i) m->leaf_cover.push_back((double)t.leaf_count[i]);
  m->tree_expected.push_back(ev);
  m->tree_depth.push_back(depth);
  const int32_t word0 = (int32_t)m->cat_words.size();
  for (int32_t i = 0; i + 1 < t.num_leaves; ++i) {
    PredNode n;
    n.threshold = t.threshold[i];
    n.feature = t.split_feature[i];
    n.left = t.left_child[i];
    n.right = t.right_child[i];
    n.dtype = t.decision_type[i];
    m->nodes.push_back(n);
  }
  for (double v : t.leaf_value) m->leaf_values.push_back(v);
  for (int32_t b : t.cat_boundaries) m->cat_bounds.push_back(word0 + b);
  for (uint32_t w : t.cat_threshold) m->cat_words.push_back(w);
}

// ---- model text writer ---------------------------------------------------------
// `%.17g` for threshold / leaf_value / leaf_weight, `%g` for split_gain /
// internal_value / internal_weight / shrinkage (the C printf forms the reference
// reproduces, format.rs:1-60).
void put_g(std::string* s, double v, int prec) {
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.*g", prec, v);
  *s += buf;
}
template <typename T, typename F>
void put_list(std::string* s, const char* key, const std::vector<T>& v, F put) {
  *s += key;
  *s += '=';
  for (size_t i = 0; i < v.size(); ++i) {
    if (i) *s += ' ';
    put(v[i]);
  }
  *s += '\n';
}

// Tree::to_string (tree.rs:800-836).
std::string tree_to_text(const HostTree& t) {
  std::string s;
  auto ints = [&](const char* k, const std::vector<int32_t>& v) {
    put_list(&s, k, v, [&](int32_t x) { s += std::to_string(x); });
  };
  auto g17 = [&](const char* k, const std::vector<double>& v) {
    put_list(&s, k, v, [&](double x) { put_g(&s, x, 17); });
  };
  auto g6 = [&](const char* k, const std::vector<double>& v) {
    put_list(&s, k, v, [&](double x) { put_g(&s, x, 6); });
  };
  s += "num_leaves=" + std::to_string(t.num_leaves) + "\n";
  s += "num_cat=" + std::to_string(t.num_cat) + "\n";
  ints("split_feature", t.split_feature);
  put_list(&s, "split_gain", t.split_gain, [&](float x) { put_g(&s, (double)x, 6); });
  g17("threshold", t.threshold);
  ints("decision_type", t.decision_type);
  ints("left_child", t.left_child);
  ints("right_child", t.right_child);
  g17("leaf_value", t.leaf_value);
  g17("leaf_weight", t.leaf_weight);
  ints("leaf_count", t.leaf_count);
  g6("internal_value", t.internal_value);
  g6("internal_weight", t.internal_weight);
  ints("internal_count", t.internal_count);
  if (t.num_cat > 0) {
    ints("cat_boundaries", t.cat_boundaries);
    put_list(&s, "cat_threshold", t.cat_threshold, [&](uint32_t x) { s += std::to_string(x); });
  }
  s += t.is_linear ? "is_linear=1\n" : "is_linear=0\n";
  if (t.is_linear) {
    // one "<value> " per term and one more space after each leaf's group (tree.rs:820-834)
    g17("leaf_const", t.leaf_const);
    ints("num_features", t.leaf_nfeat);
    std::string lf = "leaf_features=", lc = "leaf_coeff=";
    size_t k = 0;
    for (const int32_t c : t.leaf_nfeat) {
      for (int32_t j = 0; j < c; ++j, ++k) {
        lf += std::to_string(t.leaf_features[k]) + ' ';
        put_g(&lc, t.leaf_coeff[k], 17);
        lc += ' ';
      }
      lf += ' ';
      lc += ' ';
    }
    s += lf + "\n" + lc + "\n";
  }
  s += "shrinkage=";
  put_g(&s, t.shrinkage, 6);
  s += "\n\n";
  return s;
}

}  // namespace

bool check_tree(const HostTree& t_, int32_t max_feature_idx, std::string* err) {
  const HostTree* t = &t_;
  const int32_t ni = t->num_leaves - 1;
  if (t->num_leaves < 1) return fail(err, "num_leaves must be >= 1");
  if ((int32_t)t->leaf_value.size() != t->num_leaves) return fail(err, "leaf_value length");
  if (t->num_cat < 0) return fail(err, "num_cat must be >= 0");
  const bool lw_ok = (int32_t)t->leaf_weight.size() == t->num_leaves ||
                     (t->num_leaves == 1 && t->leaf_weight.empty());
  if (!lw_ok || (int32_t)t->leaf_count.size() != t->num_leaves)
    return fail(err, "leaf_weight / leaf_count length");
  if (t->num_cat > 0) {
    if ((int32_t)t->cat_boundaries.size() != t->num_cat + 1) return fail(err, "cat_boundaries length");
    for (int32_t i = 0; i < t->num_cat; ++i)
      if (t->cat_boundaries[i] < 0 || t->cat_boundaries[i] > t->cat_boundaries[i + 1])
        return fail(err, "cat_boundaries not ascending");
    if ((int64_t)t->cat_threshold.size() != (int64_t)t->cat_boundaries.back())
      return fail(err, "cat_threshold length");
  } else if (!t->cat_boundaries.empty() || !t->cat_threshold.empty()) {
    return fail(err, "categorical bitsets in a tree with num_cat=0");
  }
  if (t->is_linear) {
    if ((int32_t)t->leaf_const.size() != t->num_leaves) return fail(err, "leaf_const length");
    if ((int32_t)t->leaf_nfeat.size() != t->num_leaves) return fail(err, "num_features length");
    int64_t total = 0;
    for (const int32_t c : t->leaf_nfeat) {
      if (c < 0) return fail(err, "num_features entry is negative");
      total += c;
    }
    if ((int64_t)t->leaf_features.size() != total) return fail(err, "leaf_features length");
    if ((int64_t)t->leaf_coeff.size() != total) return fail(err, "leaf_coeff length");
    for (const int32_t f : t->leaf_features)
      if (f < 0 || f > max_feature_idx) return fail(err, "leaf_features entry out of range");
  } else if (!t->leaf_const.empty() || !t->leaf_nfeat.empty() || !t->leaf_features.empty() ||
             !t->leaf_coeff.empty()) {
    return fail(err, "linear leaves in a tree with is_linear=0");
  }
  if (ni == 0) return true;
  if ((int32_t)t->split_feature.size() != ni || (int32_t)t->threshold.size() != ni ||
      (int32_t)t->left_child.size() != ni || (int32_t)t->right_child.size() != ni ||
      (int32_t)t->decision_type.size() != ni || (int32_t)t->split_gain.size() != ni ||
      (int32_t)t->internal_value.size() != ni || (int32_t)t->internal_weight.size() != ni ||
      (int32_t)t->internal_count.size() != ni)
    return fail(err, "internal node array length != num_leaves - 1");
  // every index the traversal follows
  std::vector<int32_t> seen_node(ni, 0), seen_leaf(t->num_leaves, 0);
  for (int32_t i = 0; i < ni; ++i) {
    if (t->split_feature[i] < 0 || t->split_feature[i] > max_feature_idx)
      return fail(err, "split_feature out of range");
    const int32_t dt = t->decision_type[i];
    if (dt & 1) {
      const double c = t->threshold[i];
      if (!(c >= 0.0) || c >= (double)t->num_cat) return fail(err, "categorical split without its bitset");
    }
    for (const int32_t ch : {t->left_child[i], t->right_child[i]}) {
      if (ch >= 0) {
        if (ch >= ni || ch == 0) return fail(err, "child node index out of range");
        if (seen_node[ch]++) return fail(err, "node referenced twice");
      } else {
        const int32_t l = ~ch;
        if (l >= t->num_leaves) return fail(err, "child leaf index out of range");
        if (seen_leaf[l]++) return fail(err, "leaf referenced twice");
      }
    }
  }
  // one tree: every leaf reached from node 0 (then no node is on a cycle)
  std::vector<int32_t> stack{0};
  int32_t leaves = 0, visits = 0;
  while (!stack.empty()) {
    const int32_t n = stack.back();
    stack.pop_back();
    if (++visits > ni) return fail(err, "tree structure is not a tree");
    for (const int32_t ch : {t->left_child[n], t->right_child[n]}) {
      if (ch >= 0)
        stack.push_back(ch);
      else
        ++leaves;
    }
  }
  if (leaves != t->num_leaves) return fail(err, "tree structure is not a tree");
  return true;
}

bool model_set_objective(lgbm_hip_model* m, const std::string& line, std::string* err) {
  if (!parse_objective(line, m, err)) return false;
  m->objective_line = line;
  m->have_objective = true;
  return true;
}

bool model_add_tree(lgbm_hip_model* m, HostTree&& t, std::string* err) {
  if (!check_tree(t, m->max_feature_idx, err)) return false;
  flatten_tree(m, t);
  m->trees.push_back(std::move(t));
  m->uid = g_model_uid.fetch_add(1);  // a changed model is a new device copy
  return true;
}

// GBDT::SaveModelToString (model_text.rs:231-320).
std::string model_to_text(const lgbm_hip_model& m) {
  std::string s = "tree\nversion=v4\n";
  s += "num_class=" + std::to_string(m.num_class) + "\n";
  s += "num_tree_per_iteration=" + std::to_string(m.num_tree_per_iteration) + "\n";
  s += "label_index=" + std::to_string(m.label_index) + "\n";
  s += "max_feature_idx=" + std::to_string(m.max_feature_idx) + "\n";
  if (m.have_objective) s += "objective=" + m.objective_line + "\n";
  if (m.average_output) s += "average_output\n";
  s += "feature_names=" + m.feature_names + "\n";
  if (m.have_monotone) s += "monotone_constraints=" + m.monotone_constraints + "\n";
  s += "feature_infos=" + m.feature_infos + "\n";
  std::vector<std::string> blocks;
  for (size_t i = 0; i < m.trees.size(); ++i)
    blocks.push_back("Tree=" + std::to_string(i) + "\n" + tree_to_text(m.trees[i]) + "\n");
  s += "tree_sizes=";
  for (size_t i = 0; i < blocks.size(); ++i) {
    if (i) s += ' ';
    s += std::to_string(blocks[i].size());
  }
  s += "\n\n";
  for (const std::string& b : blocks) s += b;
  s += "end of trees\n";
  // split-count importances of splits with gain > 0, by count descending (stable)
  const int32_t nf = m.max_feature_idx + 1;
  std::vector<uint64_t> cnt((size_t)std::max(nf, 0), 0);
  for (const HostTree& t : m.trees)
    for (size_t i = 0; i < t.split_feature.size(); ++i)
      if (i < t.split_gain.size() && t.split_gain[i] > 0.0f && t.split_feature[i] < nf)
        ++cnt[(size_t)t.split_feature[i]];
  std::vector<std::string> names;
  {
    size_t p = 0;
    while (true) {
      const size_t e = m.feature_names.find(' ', p);
      names.push_back(m.feature_names.substr(p, e == std::string::npos ? std::string::npos : e - p));
      if (e == std::string::npos) break;
      p = e + 1;
    }
  }
  std::vector<std::pair<uint64_t, size_t>> pairs;
  for (size_t f = 0; f < cnt.size(); ++f)
    if (cnt[f] > 0) pairs.push_back({cnt[f], f});
  std::stable_sort(pairs.begin(), pairs.end(),
                   [](const std::pair<uint64_t, size_t>& a, const std::pair<uint64_t, size_t>& b) {
                     return a.first > b.first;
                   });
  s += "\nfeature_importances:\n";
  for (const auto& pr : pairs)
    s += (pr.second < names.size() ? names[pr.second] : std::string()) + "=" +
         std::to_string(pr.first) + "\n";
  if (m.have_trailer) {
    s += "\n";
    s += m.trailer;
  }
  return s;
}

bool parse_model_text(const char* text, size_t len, lgbm_hip_model* m, std::string* err) {
  std::string all(text, len);
  std::vector<std::string> lines;
  size_t p = 0;
  while (p <= all.size()) {
    size_t e = all.find('\n', p);
    if (e == std::string::npos) e = all.size();
    std::string line = all.substr(p, e - p);
    if (!line.empty() && line.back() == '\r') line.pop_back();
    lines.push_back(line);
    p = e + 1;
  }
  size_t i = 0;
  bool have_nc = false, have_ntpi = false, have_mfi = false;
  for (; i < lines.size() && lines[i].compare(0, 5, "Tree=") != 0; ++i) {
    const std::string& l = lines[i];
    if (l == "average_output") m->average_output = true;
    const size_t eq = l.find('=');
    if (eq == std::string::npos) continue;
    const std::string k = l.substr(0, eq), v = l.substr(eq + 1);
    if (k == "num_class") {
      if (!parse_int(v, &m->num_class, "num_class", err)) return false;
      have_nc = true;
    } else if (k == "num_tree_per_iteration") {
      if (!parse_int(v, &m->num_tree_per_iteration, "num_tree_per_iteration", err)) return false;
      have_ntpi = true;
    } else if (k == "max_feature_idx") {
      if (!parse_int(v, &m->max_feature_idx, "max_feature_idx", err)) return false;
      have_mfi = true;
    } else if (k == "objective") {
      if (!model_set_objective(m, v, err)) return false;
    } else if (k == "label_index") {
      if (!parse_int(v, &m->label_index, "label_index", err)) return false;
    } else if (k == "feature_names") {
      m->feature_names = v;
    } else if (k == "feature_infos") {
      m->feature_infos = v;
    } else if (k == "monotone_constraints") {
      m->monotone_constraints = v;
      m->have_monotone = true;
    }
  }
  if (!have_nc) return fail(err, "model without num_class");
  if (!have_mfi) return fail(err, "model without max_feature_idx");
  if (!have_ntpi) m->num_tree_per_iteration = m->num_class;
  if (m->num_class < 1 || m->num_tree_per_iteration < 1 || m->max_feature_idx < 0)
    return fail(err, "bad num_class / num_tree_per_iteration / max_feature_idx");
  while (i < lines.size()) {
    if (lines[i].compare(0, 5, "Tree=") == 0) {
      std::map<std::string, std::string> kv;
      size_t j = i + 1;
      for (; j < lines.size() && !lines[j].empty(); ++j) {
        const size_t eq = lines[j].find('=');
        if (eq == std::string::npos) return fail(err, "tree block line without '='");
        kv[lines[j].substr(0, eq)] = lines[j].substr(eq + 1);
      }
      HostTree t;
      if (!parse_tree(kv, m->max_feature_idx, &t, err)) return false;
      m->trees.push_back(std::move(t));
      i = j;
    } else if (lines[i] == "end of trees") {
      break;
    } else {
      ++i;
    }
  }
  // the `parameters:`..EOF tail, kept verbatim (model_text.rs:190-206)
  const size_t eot = all.find("end of trees");
  if (eot != std::string::npos) {
    size_t q = eot;
    while ((q = all.find("parameters:", q)) != std::string::npos) {
      const bool line_start = q == 0 || all[q - 1] == '\n';
      const size_t after = q + 11;
      const bool line_end = after == all.size() || all[after] == '\n' ||
                            (all[after] == '\r' && after + 1 < all.size() && all[after + 1] == '\n');
      if (line_start && line_end) {
        m->trailer = all.substr(q);
        m->have_trailer = true;
        break;
      }
      q = after;
    }
  }
  if (m->trees.size() % (size_t)m->num_tree_per_iteration != 0)
    return fail(err, "tree count is not a multiple of num_tree_per_iteration");
  for (const HostTree& t : m->trees) flatten_tree(m, t);
  m->uid = g_model_uid.fetch_add(1);
  return true;
}
