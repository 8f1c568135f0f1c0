// model.h — LightGBM v4 model text on the host and its flattened device form.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

// Objective ConvertOutput kinds (crates/lgbm-model/src/objective.rs:48-88).
enum PredObjective : int32_t {
  OBJ_REGRESSION = 0,       // identity
  OBJ_REGRESSION_SQRT = 1,  // sign(x) * x * x
  OBJ_BINARY = 2,           // 1 / (1 + exp(-sigmoid * x))
  OBJ_MULTICLASS = 3,       // softmax with max subtraction
  OBJ_MULTICLASS_OVA = 4,   // per-class sigmoid
  OBJ_EXP = 5,              // poisson / gamma / tweedie: exp(x)
  OBJ_XENTROPY = 6,         // 1 / (1 + exp(-x))
  OBJ_XENTLAMBDA = 7,       // log1p(exp(x))
};

// One internal node as the device reads it (24 bytes).  For a categorical split,
// `threshold` is the index of its bitset (Tree::cat_boundaries), as in the model text.
struct PredNode {
  double threshold;
  int32_t feature;
  int32_t left, right;  // >= 0: internal node of the same tree; < 0: ~leaf
  int32_t dtype;        // decision_type bits (1 categorical, 2 default left, missing << 2)
};

// Per tree: where its nodes, leaf values and categorical bitset bounds start.
struct PredTree {
  int32_t node0, leaf0, cat0, num_leaves;
  int32_t lin0;  // first PredLinLeaf of a linear tree; -1 for constant leaves
};

// A linear tree's leaf (Tree::linear_leaf_output, tree.rs:301-316): the output is
// `c + sum_j coeff[start + j] * x[feature[start + j]]` over `count` terms.
struct PredLinLeaf {
  double c;
  int32_t start, count;
};

struct HostTree {
  int32_t num_leaves = 0, num_cat = 0;
  std::vector<int32_t> split_feature, left_child, right_child, decision_type, cat_boundaries;
  std::vector<double> threshold, leaf_value;
  std::vector<uint32_t> cat_threshold;
  // metadata kept for the model text (Tree::to_string, tree.rs:800-836)
  std::vector<float> split_gain;
  std::vector<double> leaf_weight, internal_value, internal_weight;
  std::vector<int32_t> leaf_count, internal_count;
  double shrinkage = 1.0;
  // linear leaves (tree.rs:69-90): leaf_const, num_features, flat leaf_features / leaf_coeff
  bool is_linear = false;
  std::vector<double> leaf_const, leaf_coeff;
  std::vector<int32_t> leaf_nfeat, leaf_features;
};

struct lgbm_hip_model {
  int32_t num_class = 1, num_tree_per_iteration = 1, max_feature_idx = -1;
  int32_t objective = OBJ_REGRESSION;
  double sigmoid = 1.0;
  int32_t objective_outputs = 1;  // ObjectiveKind::num_output: num_class for the multiclass kinds
  // envelope kept verbatim for the model text (model_text.rs:216-320)
  int32_t label_index = 0;
  bool average_output = false;
  bool have_objective = false, have_monotone = false, have_trailer = false;
  std::string objective_line, feature_names, feature_infos, monotone_constraints, trailer;
  std::vector<HostTree> trees;
  uint64_t uid = 0;  // distinguishes models in the per-context device cache
  // flattened form
  std::vector<PredNode> nodes;
  std::vector<PredTree> tree_index;
  std::vector<double> leaf_values;
  std::vector<int32_t> cat_bounds;  // absolute offsets into cat_words
  std::vector<uint32_t> cat_words;
  // TreeSHAP inputs (tree.rs:336-400): covers per node and leaf (data counts as f64),
  // each tree's cover-weighted leaf average and maximum leaf depth
  std::vector<double> node_cover, leaf_cover, tree_expected;
  std::vector<int32_t> tree_depth;
  bool any_linear = false;
  std::vector<PredLinLeaf> lin_leaves;
  std::vector<int32_t> lin_features;
  std::vector<double> lin_coeffs;
};

// Parses `text`; on failure returns false with `err` set (nothing is allocated).
bool parse_model_text(const char* text, size_t len, lgbm_hip_model* m, std::string* err);
// The model text of `m` (GBDT::SaveModelToString with split-count importances).
std::string model_to_text(const lgbm_hip_model& m);
// Checks a tree built in memory and appends it (flattened form included).
bool model_add_tree(lgbm_hip_model* m, HostTree&& t, std::string* err);
// Parses the objective line into m->objective / m->sigmoid.
bool model_set_objective(lgbm_hip_model* m, const std::string& line, std::string* err);
