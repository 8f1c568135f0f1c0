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

#include <atomic>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>

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
  } else if (n == "multiclassova" || n == "multiclass_ova" || n == "ova" || n == "ovr") {
    if (!have_nc || nc < 1) return fail(err, "multiclassova objective must contain num_class >= 1");
    if (!(m->sigmoid > 0.0)) return fail(err, "multiclassova sigmoid must be > 0");
    m->objective = OBJ_MULTICLASS_OVA;
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
    if (lin) return fail(err, "linear trees are not supported");
  }
  if (!(s = get("leaf_value"))) return fail(err, "tree model should contain leaf_value field");
  if (!parse_f64s(*s, &t->leaf_value, "leaf_value", err)) return false;
  if ((int64_t)t->leaf_value.size() != t->num_leaves) return fail(err, "leaf_value length");
  if (t->num_leaves == 1) return true;
  const int32_t ni = t->num_leaves - 1;
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

void flatten(lgbm_hip_model* m) {
  for (const HostTree& t : m->trees) {
    PredTree pt;
    pt.node0 = (int32_t)m->nodes.size();
    pt.leaf0 = (int32_t)m->leaf_values.size();
    pt.cat0 = (int32_t)m->cat_bounds.size();
    pt.num_leaves = t.num_leaves;
    m->tree_index.push_back(pt);
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
}

}  // namespace

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
  bool have_nc = false, have_ntpi = false, have_mfi = false, have_obj = false;
  for (; i < lines.size() && lines[i].compare(0, 5, "Tree=") != 0; ++i) {
    const std::string& l = lines[i];
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
      if (!parse_objective(v, m, err)) return false;
      have_obj = true;
    }
  }
  if (!have_nc) return fail(err, "model without num_class");
  if (!have_mfi) return fail(err, "model without max_feature_idx");
  if (!have_ntpi) m->num_tree_per_iteration = m->num_class;
  if (!have_obj) m->objective = OBJ_REGRESSION;
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
  if (m->trees.size() % (size_t)m->num_tree_per_iteration != 0)
    return fail(err, "tree count is not a multiple of num_tree_per_iteration");
  flatten(m);
  m->uid = g_model_uid.fetch_add(1);
  return true;
}
