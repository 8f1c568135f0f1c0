/*
 * lgbm_hip.h — C-ABI of the MI355X (gfx950) GBDT tree-learner hot path.
 *
 * The library replaces the device half of the reference's compute seam,
 * `trait Backend` (crates/lgbm-compute/src/lib.rs:1092-2782), for the numeric
 * leaf-wise learner spine: the quantized gradient discretizer, the resident bin
 * layout, ConstructHistogram, FixHistogram + compaction, the subtraction trick,
 * FindBestThreshold, the cross-leaf ArgMax and DataPartition.  Every entry point
 * below names the reference interface it replaces.
 *
 * Conventions
 *  - All functions return an int status: LGBM_HIP_OK (0) or a negative code that
 *    mirrors `ComputeError` (crates/lgbm-compute/src/error.rs).  A message with the
 *    details is available from lgbm_hip_last_error().  Nothing aborts across the ABI.
 *  - Host pointers are borrowed for the duration of the call only.  Outputs are
 *    caller-allocated; capacities are implied by the documented sizes.
 *  - A context owns every device allocation (bins, gradients, quantized gradients,
 *    row permutation buffers, histogram slots, tree buffers).  A context is not
 *    thread-safe (the reference backend is `!Sync`, lib.rs:3840-3846); all calls
 *    on one context are synchronous at the API boundary.
 *  - Histogram cells use the reference layout: feature f occupies
 *    [slot_off[f], slot_off[f] + 2*num_bin[f]) of a leaf slot, grad at 2*bin,
 *    hess at 2*bin+1 (crates/lgbm-compute/src/kernels/histogram.rs:64-68,
 *    crates/lgbm-treelearner/src/learner.rs:4438-4446).
 */
#ifndef LGBM_HIP_H
#define LGBM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (crates/lgbm-compute/src/error.rs) ---------------------- */
#define LGBM_HIP_OK 0
#define LGBM_HIP_ERR_LENGTH_MISMATCH (-1)       /* ComputeError::LengthMismatch      */
#define LGBM_HIP_ERR_BIN_OUT_OF_RANGE (-2)      /* ComputeError::BinIndexOutOfRange  */
#define LGBM_HIP_ERR_CAPABILITY (-3)            /* ComputeError::CapabilityUnavailable */
#define LGBM_HIP_ERR_RUNTIME (-4)               /* ComputeError::Runtime             */
#define LGBM_HIP_ERR_HIP (-5)                   /* a HIP runtime call failed          */
#define LGBM_HIP_ERR_INVALID_ARGUMENT (-6)      /* null pointer / bad size            */
#define LGBM_HIP_ERR_INVALID_LEAF_HESSIAN (-7)  /* TreeLearnerError::InvalidLeafHessian */

/* MissingType (crates/lgbm-dataset/src/bin_mapper.rs; Tree decision_type bits 2-3) */
#define LGBM_MISSING_NONE 0
#define LGBM_MISSING_ZERO 1
#define LGBM_MISSING_NAN 2

/* `GainConfig` (crates/lgbm-compute/src/gain.rs:904-960), field for field. */
typedef struct lgbm_gain_config {
  int32_t min_data_in_leaf;
  int32_t _pad0;
  double min_sum_hessian_in_leaf;
  double max_delta_step;
  double lambda_l1;
  double lambda_l2;
  double min_gain_to_split;
  double path_smooth;
  double parent_output;
  int32_t min_data_per_group;
  int32_t max_cat_threshold;
  double cat_l2;
  double cat_smooth;
  int32_t max_cat_to_onehot;
  int32_t _pad1;
} lgbm_gain_config;

/* `SplitInfo` (crates/lgbm-compute/src/gain.rs:1019-1053).  gain == -inf is the
 * "no split" sentinel (`SplitInfo::none`, gain.rs:1068-1084). */
typedef struct lgbm_split_info {
  uint32_t threshold;
  int32_t left_count;
  int32_t right_count;
  int32_t default_left; /* bool */
  double gain;
  double left_sum_gradient;
  double left_sum_hessian;
  double right_sum_gradient;
  double right_sum_hessian;
  double left_output;
  double right_output;
} lgbm_split_info;

/* `BatchedSplitFeature` (crates/lgbm-compute/src/kernels/split.rs:77-95). */
typedef struct lgbm_batched_feature {
  uint64_t slot_off;
  uint32_t num_bin;
  int32_t offset;
  uint32_t default_bin;
  uint32_t most_freq_bin;
  int32_t skip_default_bin; /* bool */
  int32_t na_as_missing;    /* bool */
  int32_t run_forward;      /* bool */
  int32_t _pad;
} lgbm_batched_feature;

#define LGBM_BIN_NUMERICAL 0
#define LGBM_BIN_CATEGORICAL 1

/* The `FeatureColumn` descriptors (crates/lgbm-treelearner/src/learner.rs:87-204)
 * minus the bins themselves; `bin_upper_bound` values are passed as one
 * concatenated array (feature f at sum_{f'<f} num_bin[f']): a numerical feature's
 * upper bounds, a categorical feature's `bin_to_category` (bin -> category value,
 * -1 for bin 0, the NaN / unseen-category bin). */
typedef struct lgbm_feature_meta {
  uint32_t num_bin;
  int32_t offset; /* offset_for_most_freq_bin(most_freq_bin) (lgbm-treelearner/src/lib.rs:89-95) */
  uint32_t min_bin;
  uint32_t max_bin;
  uint32_t default_bin;
  uint32_t most_freq_bin;
  int32_t missing_type; /* LGBM_MISSING_* */
  int32_t real_feature_index;
  int32_t bin_type; /* LGBM_BIN_*: categorical features split by category sets */
} lgbm_feature_meta;

/* A grown tree (crates/lgbm-model/src/tree.rs: Tree fields written by
 * `Tree::split`, tree.rs:614-700).  Caller-allocated arrays; capacities:
 * node arrays num_leaves_cap-1, leaf arrays num_leaves_cap. */
typedef struct lgbm_tree_out {
  int32_t num_leaves; /* out */
  int32_t _pad;
  int32_t* split_feature;      /* real feature index per internal node */
  uint32_t* threshold_in_bin;
  double* threshold;           /* bin_upper_bound[threshold_in_bin] */
  float* split_gain;           /* f32(gain + min_gain_to_split), learner.rs:3985 */
  int8_t* decision_type;
  int32_t* left_child;
  int32_t* right_child;
  double* internal_value;
  int32_t* internal_count;
  double* leaf_value;
  double* leaf_weight;
  int32_t* leaf_count;
  int32_t* leaf_depth;
  int32_t* leaf_parent;
  double* internal_weight;     /* left + right sum_hessian of the split (the C++
                                  Tree::Split rule; tree.rs:655 stores 0) */
  /* Categorical splits (Tree::split_categorical, tree.rs:710-790): such a node's
   * threshold / threshold_in_bin hold its index among the categorical nodes and
   * decision_type has bit 0 set; its category set (left: in the set) is the bitset
   * cat_threshold[cat_boundaries[i] .. cat_boundaries[i + 1]) over category values. */
  int32_t num_cat;             /* out */
  int32_t cat_threshold_cap;   /* in: capacity of cat_threshold in 32-bit words */
  int32_t* cat_boundaries;     /* num_leaves_cap entries (num_cat + 1 used; NULL: none) */
  uint32_t* cat_threshold;
} lgbm_tree_out;

/* `LeafPartitionLayout` (crates/lgbm-dataset/src/dataset.rs:88-97): the data
 * partition a tree was grown over.  indices has num_data entries, leaf arrays
 * num_leaves_cap entries. */
typedef struct lgbm_layout_out {
  uint32_t* indices;
  int32_t* leaf_begin;
  int32_t* leaf_count;
} lgbm_layout_out;

/* Leaf totals handed to a per-leaf op (`LeafSplits`, lgbm-treelearner/src/
 * leaf_splits.rs:36-52). */
typedef struct lgbm_leaf_sums {
  double sum_gradient;
  double sum_hessian;
  int32_t num_data;
  int32_t _pad;
  double weight; /* parent_output for path smoothing */
} lgbm_leaf_sums;

typedef struct lgbm_hip_ctx lgbm_hip_ctx;

/* ---- context ---------------------------------------------------------------- */

/* Create a context on HIP device `device`.  Replaces constructing `GpuBackend`
 * with its resident caches (lib.rs:3848-3934; dispatch arm
 * crates/lgbm/src/booster.rs:1922-1932). */
int lgbm_hip_ctx_create(int device, lgbm_hip_ctx** out);
int lgbm_hip_ctx_destroy(lgbm_hip_ctx* ctx);
/* Copy the last error message of `ctx` (or of the last failed create when ctx is
 * NULL) into buf; always NUL-terminates when size > 0. */
int lgbm_hip_last_error(const lgbm_hip_ctx* ctx, char* buf, size_t size);

/* ---- resident data (lgbm-compute/src/lib.rs:1564-1620) ---------------------- */

/* Upload the binned columns once per train.  Replaces
 * `Backend::upload_resident_bins(&[&BinColumn])` (lib.rs:1564; GPU impl
 * lib.rs:4368-4433) and `resident_bin_width` (lib.rs:3752).  `bins` is
 * feature-major u8 ([f*num_data + row]); every bin must be < num_bin[f] (the
 * once-per-train bin-range gate, learner.rs:1161-1187): a violation returns
 * LGBM_HIP_ERR_BIN_OUT_OF_RANGE.  `bin_upper_bound` holds sum(num_bin) doubles
 * (may be NULL: thresholds then record the bin index). */
int lgbm_hip_upload_bins(lgbm_hip_ctx* ctx, const uint8_t* bins, int32_t num_features,
                         int64_t num_data, const lgbm_feature_meta* meta,
                         const double* bin_upper_bound);

/* Upload per-row f32 gradients/hessians (`Backend::upload_resident_grad_hess`,
 * lib.rs:1607).  n must equal the uploaded num_data. */
int lgbm_hip_set_gradients(lgbm_hip_ctx* ctx, const float* grad, const float* hess, int64_t n);

/* Quantize the resident gradients in place for `use_quantized_grad`:
 * `GradientDiscretizer::discretize_dequantize_in_place` + the call site
 * `quantize_grad_hess_in_place` (lgbm-treelearner/src/gradient_discretizer.rs:
 * 126-188, lgbm-boosting/src/gbdt.rs:43-62).  `stochastic` selects xorshift64
 * stochastic rounding seeded with `seed` (gbdt.rs:950 derives it per (iter,class)).
 * Writes the packed int8 (grad, hess) pairs the histogram kernels consume and,
 * when the out pointers are non-NULL, the dequantized f32 values and the scales
 * {grad_scale, hess_scale}. */
int lgbm_hip_quantize(lgbm_hip_ctx* ctx, int32_t num_grad_quant_bins, int32_t stochastic,
                      uint64_t seed, float* dequant_grad_out, float* dequant_hess_out,
                      double* scales_out);

/* Read back the packed discretized buffer in the reference `discretize` layout:
 * out[2*i] = hessian, out[2*i+1] = gradient (gradient_discretizer.rs:25-26,104-118). */
int lgbm_hip_get_discretized(lgbm_hip_ctx* ctx, int8_t* out, int64_t n);

/* Quantized gradients from their dequantized values, for the drop-in wiring at the
 * quantizer call site (quantize_grad_hess_in_place, gbdt.rs:43-62,945-960): the
 * reference replaces g/h in place by f32(q * scale) and the learner then uploads
 * those arrays.  Quantizing them again is not idempotent (the recomputed scales
 * round differently, stochastic draws differ), so this entry recovers q instead:
 * q = round(v / scale) per row, exact for every v = f32(q * scale), verified by
 * f32(q * scale) == v.  grad_scale / hess_scale are the discretizer's scales
 * (GradientDiscretizer grad_scale / hess_scale, gradient_discretizer.rs:145-165);
 * both <= 0 take those of this context's last lgbm_hip_quantize.  A row that is not
 * f32(q * scale) with |q_grad| <= num_grad_quant_bins / 2 and 0 <= q_hess <=
 * num_grad_quant_bins returns LGBM_HIP_ERR_INVALID_ARGUMENT naming the row, and the
 * context then holds no quantized gradients. */
int lgbm_hip_set_dequantized_gradients(lgbm_hip_ctx* ctx, const float* grad, const float* hess,
                                       int64_t n, int32_t num_grad_quant_bins,
                                       double grad_scale, double hess_scale);

/* config.feature_contri: per-feature split-gain multipliers indexed by REAL feature
 * index (n entries; features whose real index is >= n keep 1), applied to each
 * feature's scan result after its splittability is recorded and before the
 * cross-feature ArgMax (learner.rs:3235-3252, 3701-3709).  Affects the trees grown
 * after the call; a bins upload resets every multiplier to 1, as does n == 0. */
int lgbm_hip_set_feature_contri(lgbm_hip_ctx* ctx, const double* contri, int32_t n);

/* ---- per-op seam (parity tests / fine-grained driver) ----------------------- */

/* Exact integer histogram of the quantized gradients over `leaf_rows` (or all rows
 * when leaf_rows is NULL): out[slot cell] as int64, [g0,h0,g1,h1,...] per feature.
 * Replaces `construct_int_histogram` (gradient_discretizer.rs:235-250) per feature. */
int lgbm_hip_build_int_histogram(lgbm_hip_ctx* ctx, const uint32_t* leaf_rows, int64_t n_rows,
                                 int64_t* out);

/* Build one leaf's f64 histogram, then FixHistogram on the RAW leaf sums and
 * compaction: the device analog of `build_leaf_histogram_into`
 * (learner.rs:2464-2566) = `Backend::build_resident_leaf` (lib.rs:1953-1972).  out
 * has slot_len doubles.  Uses the quantized gradients after lgbm_hip_quantize
 * (bit-exact with the f64 fold of the dequantized values), otherwise the f32
 * gradients of lgbm_hip_set_gradients (64-bit fixed-point build, within ~1e-10
 * relative of the f64 fold). */
int lgbm_hip_build_leaf_histogram(lgbm_hip_ctx* ctx, const uint32_t* leaf_rows, int64_t n_rows,
                                  double sum_gradient, double sum_hessian, double* out);

/* FindBestThreshold over a batch of features of one leaf histogram:
 * `Backend::find_best_splits_batched` (lib.rs:1500-1548) whose per-feature body is
 * `find_best_split_cpu_native` (kernels/split.rs:8970-9329).  `hist` is host
 * memory of `hist_len` doubles; out has n_feats entries. */
int lgbm_hip_find_best_splits(lgbm_hip_ctx* ctx, const double* hist, int64_t hist_len,
                              const lgbm_batched_feature* feats, int32_t n_feats,
                              const lgbm_gain_config* cfg, double sum_gradient,
                              double sum_hessian, int32_t num_data, lgbm_split_info* out);

/* The same scans over device-resident inputs with no allocation at all: hist
 * (hist_len doubles), feats (n_feats lgbm_batched_feature) and out (n_feats
 * lgbm_split_info) are device memory of the context's device; cfg is a host struct.
 * No counterpart in the reference: this is for callers that cannot allocate device
 * memory (serving loops, harnesses that forbid hipMalloc).  It is not capturable in a
 * HIP graph: it copies its status word to the host and waits for the context stream.
 * Its working memory is one fixed library-owned device array per GPU
 * (LGBM_HIP_NOALLOC_MAX_FEATURES feature descriptors), held until the process ends
 * and shared by every context on that GPU: calls that overlap on one GPU race.
 * n_feats above the maximum returns LGBM_HIP_ERR_CAPABILITY before any work; a
 * feature the host entry would refuse returns the same status (first such feature
 * in order) after the scans, with out undefined for it. */
#define LGBM_HIP_NOALLOC_MAX_FEATURES 8192
int lgbm_hip_find_best_splits_noalloc(lgbm_hip_ctx* ctx, const double* d_hist, int64_t hist_len,
                                      const lgbm_batched_feature* d_feats, int32_t n_feats,
                                      const lgbm_gain_config* cfg, double sum_gradient,
                                      double sum_hessian, int32_t num_data,
                                      lgbm_split_info* d_out);

/* Elementwise larger = parent - smaller (`Backend::subtract_histograms`,
 * lib.rs:1314; kernels/subtract.rs:204-215). */
int lgbm_hip_subtract_histograms(lgbm_hip_ctx* ctx, const double* parent, const double* child,
                                 int64_t len, double* out);

/* Stable DataPartition of `n` rows: returns the reordered local positions
 * [left ascending | right ascending] and the left count.  Router of
 * `DataPartition::split` / `split_fused_host_impl`
 * (lgbm-treelearner/src/data_partition.rs:192-288,360-463) and
 * `data_partition_cpu_native` (kernels/partition.rs:115). */
int lgbm_hip_data_partition(lgbm_hip_ctx* ctx, const uint32_t* bins, int64_t n, uint32_t num_bin,
                            uint32_t min_bin, uint32_t max_bin, uint32_t threshold,
                            uint32_t most_freq_bin, int32_t na_as_missing, int32_t default_left,
                            uint32_t* order_out, int64_t* left_count_out);

/* `quant_train_renew_leaf` (Gbdt::with_quant_renew_leaf, gbdt.rs:472-477; applied at
 * gbdt.rs:1194-1212 through renew_tree_output, learner.rs:4411-4429): with quantized
 * gradients, every tree the train_iter entries grow gets its leaf outputs recomputed
 * from the original f32 gradients, -ThresholdL1(sum_g, lambda_l1) / (sum_h +
 * lambda_l2) of the cfg, the sums an ordered f64 fold over each leaf's rows in
 * partition order; before shrinkage and the score update.  No effect on f32-gradient
 * training.  Set after the bins upload (an upload of another row count needs it set
 * again). */
int lgbm_hip_set_quant_renew_leaf(lgbm_hip_ctx* ctx, int32_t enable);

/* ---- device-resident histogram slots ----------------------------------------- */
/* The reference's resident pool (lib.rs:1940-2058): each leaf's f64 histogram
 * (slot_len doubles, the concatenated stride-2 layout of the resident features)
 * stays in a device slot owned by the context; only SplitInfos come back.  Every
 * entry runs on the context stream and returns after it completes.  Slots are
 * invalidated by a new bins upload (reset again). */

/* `Backend::reset_resident_pool(num_slots, slot_len)` (lib.rs:1940): size the pool;
 * slot_len must equal the resident layout's (2 x the features' bin counts). */
int lgbm_hip_resident_reset(lgbm_hip_ctx* ctx, int32_t num_slots, int64_t slot_len);

/* `Backend::build_resident_leaf` (lib.rs:1953-1972): build the leaf's histogram from
 * the resident bins and the current gradients (quantized after lgbm_hip_quantize,
 * else f32), FixHistogram on its RAW sums, compaction, into `slot`.  leaf_rows (host,
 * n_rows entries) NULL = every row. */
int lgbm_hip_resident_build(lgbm_hip_ctx* ctx, int32_t slot, const uint32_t* leaf_rows,
                            int64_t n_rows, double sum_gradient, double sum_hessian);

/* `Backend::move_resident(src, dst)` (lib.rs:1978): dst receives src's histogram. */
int lgbm_hip_resident_move(lgbm_hip_ctx* ctx, int32_t src_slot, int32_t dst_slot);

/* `Backend::subtract_resident` (lib.rs:1988-2000): larger = parent - smaller in f64
 * (histogram_pool.rs:249; not re-fixed).  larger_slot may be parent_slot. */
int lgbm_hip_resident_subtract(lgbm_hip_ctx* ctx, int32_t parent_slot, int32_t smaller_slot,
                               int32_t larger_slot);

/* `Backend::scan_resident_leaf` (lib.rs:2012-2027): FindBestThreshold of every
 * `feats` entry over slot's histogram (cfg->parent_output as given); out has n_feats
 * entries, in input order. */
int lgbm_hip_resident_scan(lgbm_hip_ctx* ctx, int32_t slot, const lgbm_batched_feature* feats,
                           int32_t n_feats, const lgbm_gain_config* cfg, double sum_gradient,
                           double sum_hessian, int32_t num_data, lgbm_split_info* out);

/* `Backend::scan_resident_siblings` (lib.rs:2043-2058): both siblings of a split with
 * one wait and readback; each side's totals carry its own parent_output (`weight`),
 * which replaces cfg->parent_output for that side. */
int lgbm_hip_resident_scan_siblings(lgbm_hip_ctx* ctx, int32_t smaller_slot, int32_t larger_slot,
                                    const lgbm_batched_feature* feats, int32_t n_feats,
                                    const lgbm_gain_config* cfg, const lgbm_leaf_sums* smaller,
                                    const lgbm_leaf_sums* larger, lgbm_split_info* out_smaller,
                                    lgbm_split_info* out_larger);

/* Copy a slot's histogram to host memory (slot_len doubles); no counterpart in the
 * reference (its handles are read only by its own scans), for checks. */
int lgbm_hip_resident_read(lgbm_hip_ctx* ctx, int32_t slot, double* out);

/* ---- coarse seam: one whole tree per call ----------------------------------- */

/* Grow one tree on device from the resident bins and the CURRENT gradients:
 * `Backend::grow_tree_on_device_with_cfg` (lib.rs:2688,2771;
 * kernels/grow_driver.rs:1219), following the CPU learner `train_inner`
 * (learner.rs:980-1562) decision for decision.  After lgbm_hip_quantize the
 * quantized gradients are used (use_quantized_grad: trees bit-exact with the CPU
 * learner); otherwise the f32 gradients of lgbm_hip_set_gradients
 * (use_quantized_grad = false).  `tree` arrays need num_leaves capacity (<= 256);
 * `layout` may be NULL (else indices has num_data entries). */
int lgbm_hip_grow_tree(lgbm_hip_ctx* ctx, const lgbm_gain_config* cfg, int32_t num_leaves,
                       int32_t max_depth, lgbm_tree_out* tree, lgbm_layout_out* layout);

/* Capacity (32-bit words) a tree output's cat_threshold needs for a tree of
 * num_leaves leaves over the resident bins: (num_leaves - 1) x (largest category
 * value / 32 + 1) when some feature is categorical, else 0.  No counterpart in the
 * reference (its Tree grows its Vec); lgbm_hip_grow_tree and the train_iter entries
 * return LGBM_HIP_ERR_LENGTH_MISMATCH before any work when a non-NULL tree output
 * holds less. */
int lgbm_hip_cat_threshold_words(lgbm_hip_ctx* ctx, int32_t num_leaves, int64_t* out);

/* ---- boosting loop on device (binary objective) ----------------------------- */

/* Upload f32 labels and reset the resident f64 score to `init_score`
 * (`ScoreUpdater::new` + `add_constant`, lgbm-boosting/src/score_updater.rs:63-99). */
int lgbm_hip_set_labels(lgbm_hip_ctx* ctx, const float* labels, int64_t n, double init_score);

/* One binary-logloss boosting iteration, all resident:
 * `BinaryLogloss::get_gradients` (lgbm-objective/src/binary.rs:134-172) ->
 * quantize (gbdt.rs:945-960, seed ((iter<<20) ^ 0x51702010)) -> grow tree ->
 * `Tree::shrinkage` (tree.rs:1074) -> score update (score_updater.rs:133).
 * num_grad_quant_bins 2 or 4: use_quantized_grad; 0: f32 gradients
 * (use_quantized_grad = false, no quantization step).
 * `tree` (may be NULL) receives the shrunk tree. */
int lgbm_hip_train_iter_binary(lgbm_hip_ctx* ctx, int32_t iter, const lgbm_gain_config* cfg,
                               int32_t num_leaves, int32_t max_depth, double learning_rate,
                               int32_t num_grad_quant_bins, int32_t stochastic,
                               lgbm_tree_out* tree);

/* BinaryLogloss::boost_from_score (crates/lgbm-objective/src/binary.rs:178-192):
 * log(pavg / (1 - pavg)) / sigmoid for the positive fraction pavg (label > 0)
 * clamped to [kEpsilon, 1 - kEpsilon]; 0 for n == 0.  Host only. */
int lgbm_hip_binary_boost_from_score(const float* label, int64_t n, double sigmoid, double* out);

/* ---- other one-tree-per-iteration objectives, column sampling ---------------- */

/* Objectives of lgbm_hip_train_iter. */
#define LGBM_HIP_OBJECTIVE_BINARY 0     /* BinaryLogloss (binary.rs:134-172) */
#define LGBM_HIP_OBJECTIVE_REGRESSION 1 /* L2: Objective::Regression (regression.rs:427-431) */
#define LGBM_HIP_OBJECTIVE_LAMBDARANK 2 /* Lambdarank (rank.rs:100-365) */

/* The objective lgbm_hip_train_iter evaluates (binary by default); a reference
 * `Objective` / `BoostObjective` value (lgbm-boosting/src/objective.rs). */
int lgbm_hip_set_objective(lgbm_hip_ctx* ctx, int32_t objective);

/* LambdaRank over the resident labels (set with lgbm_hip_set_labels, init score 0:
 * ranking has no BoostFromAverage, lgbm-boosting/src/objective.rs:112-116):
 * `Lambdarank::new` (rank.rs:131-198) with the query boundaries (num_queries + 1
 * prefix sums from 0 to num_data), sigmoid > 0, lambdarank_norm and the truncation
 * level; the default label gains 2^i - 1 (labels must be integers in 0..=30).  Also
 * selects the objective.  Queries of more than 2048 rows are refused. */
int lgbm_hip_set_lambdarank(lgbm_hip_ctx* ctx, const int32_t* query_boundaries,
                            int32_t num_queries, double sigmoid, int32_t norm,
                            int32_t truncation_level);

/* One boosting iteration of the objective set by lgbm_hip_set_objective /
 * lgbm_hip_set_lambdarank, as lgbm_hip_train_iter_binary does for the binary one
 * (gbdt.rs:691-1300 with `objective.get_gradients`). */
int lgbm_hip_train_iter(lgbm_hip_ctx* ctx, int32_t iter, const lgbm_gain_config* cfg,
                        int32_t num_leaves, int32_t max_depth, double learning_rate,
                        int32_t num_grad_quant_bins, int32_t stochastic, lgbm_tree_out* tree);

/* Per-tree column sampling: `ColSampler` with feature_fraction and
 * feature_fraction_seed (lgbm-treelearner/src/col_sampler.rs:68-140; the draw at
 * creation, then one before every tree grown on this context, learner.rs:1190-1240;
 * features outside a tree's sample are never scanned).  feature_fraction >= 1 turns
 * it off; feature_fraction_bynode must be 1 (per-node sampling is not built).  A
 * new bins upload turns it off. */
int lgbm_hip_set_col_sampler(lgbm_hip_ctx* ctx, double feature_fraction,
                             double feature_fraction_bynode, int32_t seed);

/* The objective's BoostFromScore on host labels: binary log-odds (sigmoid 1), the
 * L2 label mean (regression.rs:563-575), 0 for lambdarank.  Host only. */
int lgbm_hip_boost_from_score(int32_t objective, const float* label, int64_t n, double* out);

/* The f32 gradients / hessians of the last objective evaluation on the device
 * (BinaryLogloss::get_gradients, binary.rs:134-172; either pointer may be NULL).
 * No reference counterpart at the boundary: the reference's are host arrays. */
int lgbm_hip_get_gradients(lgbm_hip_ctx* ctx, float* grad, float* hess, int64_t n);

/* Lookahead for lgbm_hip_train_iter_binary (off by default; no reference
 * counterpart): after enqueueing iteration i's tree copy, the call also enqueues
 * iteration i + 1's gradients and quantization (same num_grad_quant_bins and
 * stochastic) and returns once the copy is done, so the device works while the host
 * handles the tree.  The next call with iter == i + 1 and the same settings uses
 * them; any other call that changes the device inputs drops them.  Results are
 * identical either way.  While it is on, lgbm_hip_get_gradients and the quantized
 * values describe the iteration enqueued ahead.  Ignored while timing is enabled. */
int lgbm_hip_set_lookahead(lgbm_hip_ctx* ctx, int32_t enable);

/* Copy the resident f64 training score back to the host: n = num_data, or
 * num_class * num_data (class-major) after lgbm_hip_set_labels_multiclass. */
int lgbm_hip_get_scores(lgbm_hip_ctx* ctx, double* out, int64_t n);

/* ---- boosting loop on device (multiclass softmax) --------------------------- */

/* Upload f32 class labels (truncated toward zero to class ids in [0, num_class),
 * MulticlassSoftmax::new, lgbm-objective/src/multiclass.rs:76-101) and reset the
 * resident class-major f64 score [num_class][num_data] to init_scores[k] per class
 * (NULL: 0; the reference's BoostFromAverage adds log(max(kEpsilon, prior_k)),
 * gbdt.rs:614-640, multiclass.rs:184-187).  num_class in 2..=256. */
int lgbm_hip_set_labels_multiclass(lgbm_hip_ctx* ctx, const float* labels, int64_t n,
                                   int32_t num_class, const double* init_scores);

/* One softmax boosting iteration, all resident (gbdt.rs:691-1373, no bagging):
 * `MulticlassSoftmax::get_gradients` (multiclass.rs:138-180) for every class from
 * the current scores, then per class k: quantize (seed (iter << 20) ^ k ^
 * 0x51702010, gbdt.rs:946-958; num_grad_quant_bins 0: f32 gradients) -> grow tree
 * -> `Tree::shrinkage` -> score update of class k.  class_need_train (may be NULL:
 * all) skips a class (gbdt.rs:1003-1018): its tree gets num_leaves = 0.  `trees`
 * (may be NULL) is an array of num_class trees receiving the shrunk trees; the
 * caller pushes the reference's constant tree for a tree with num_leaves <= 1 and
 * adds the first iteration's init score (Tree::add_bias). */
int lgbm_hip_train_iter_multiclass(lgbm_hip_ctx* ctx, int32_t iter, const lgbm_gain_config* cfg,
                                   int32_t num_leaves, int32_t max_depth, double learning_rate,
                                   int32_t num_grad_quant_bins, int32_t stochastic,
                                   const int32_t* class_need_train, lgbm_tree_out* trees);

/* The class-major f32 gradients / hessians of the last softmax evaluation
 * (n = num_class * num_data; either pointer may be NULL).  No reference counterpart
 * at the boundary: the reference's are host arrays. */
int lgbm_hip_get_multiclass_gradients(lgbm_hip_ctx* ctx, float* grad, float* hess, int64_t n);

/* Per-kernel device time (ms, HIP events on the context stream) accumulated since
 * the last reset, by kernel family: [0] histogram, [1] partition, [2] split scan,
 * [3] quantize, [4] objective+score.  Also returns the algorithmic histogram bytes
 * and launch count.  Enabling timing adds event records per launch. */
int lgbm_hip_set_timing(lgbm_hip_ctx* ctx, int32_t enable);
int lgbm_hip_get_timing(lgbm_hip_ctx* ctx, double* ms_out5, double* hist_bytes_out,
                        int64_t* hist_launches_out);

/* Counters since the last lgbm_hip_set_timing (no reference counterpart; the
 * reference's equivalent is its env-gated phase profiler, lgbm-treelearner/src/
 * phase_prof.rs:1-60).  out[0..4]: ms per kernel family as above; [5] root
 * ConstructHistogram rows; [6] root ConstructHistogram launches; [7] rows moved by
 * partition passes (which also build one child's histogram per split); [8]
 * partition kernels launched while timing (rounds after a tree is complete
 * included); [9] bytes a partition pass reads per quantized row: the row record
 * plus its separately stored quantized pair (none when the record holds it);
 * [10] features; [11] histogram
 * cells; [12] leaf splits partitioned (including splits made ahead of their turn
 * that the tree never used); [13] partition rounds over all trees; [14] trees;
 * [15] rounds launched after the captured per-tree sequence; [16] ms in the binning
 * kernel (lgbm_hip_upload_raw*), [17] its launches, [18] values binned; [19] ms in
 * the prediction kernel, [20] its launches, [21] rows x trees walked; [22] rows
 * whose histogram the partition passes built (the child each split builds). */
int lgbm_hip_get_stats(lgbm_hip_ctx* ctx, double* out23);

/* ---- binning ------------------------------------------------------------------ */

/* BinMapper construction parameters (crates/lgbm/src/builder.rs config fields;
 * LightGBM defaults in brackets). */
typedef struct lgbm_bin_params {
  int32_t max_bin;                  /* [255] */
  int32_t min_data_in_bin;          /* [3] */
  int32_t min_data_in_leaf;         /* [20] scaled into the pre-filter threshold */
  int32_t pre_filter;               /* [0] feature_pre_filter (the facade passes false) */
  int32_t use_missing;              /* [1] */
  int32_t zero_as_missing;          /* [0] */
  int32_t bin_construct_sample_cnt; /* [200000] */
  int32_t data_random_seed;         /* [1] */
} lgbm_bin_params;

typedef struct lgbm_bin_mapper_info {
  int32_t num_bin;
  int32_t missing_type; /* LGBM_MISSING_* */
  int32_t bin_type;     /* LGBM_BIN_* */
  int32_t is_trivial;
  uint32_t default_bin; /* ValueToBin(0) */
  uint32_t most_freq_bin;
  double sparse_rate;
  double min_val;
  double max_val;
} lgbm_bin_mapper_info;

/* One feature's value -> bin mapper, built on the host. */
typedef struct lgbm_hip_bin_mapper lgbm_hip_bin_mapper;
/* BinMapper::find_bin_from_column (crates/lgbm-dataset/src/bin_mapper.rs:613-651):
 * Random(data_random_seed).Sample(num_rows, min(num_rows, bin_construct_sample_cnt))
 * rows of the column, the pre-filter threshold min_data_in_leaf * sampled / num_rows,
 * then the numeric FindBin (bin_mapper.rs:191-365) with optional forced bounds. */
int lgbm_hip_bin_mapper_from_column(const double* column, int64_t num_rows,
                                    const lgbm_bin_params* params,
                                    const double* forced_upper_bounds, int32_t num_forced,
                                    lgbm_hip_bin_mapper** out);
/* FindBin on given sample values: find_bin_numeric (bin_mapper.rs:191-365) or, with
 * categorical set, find_bin_categorical (bin_mapper.rs:409-560; the booster bins
 * categorical columns whole, booster.rs:466-476).  total_sample_cnt - num_values
 * zeros are implied; min_split_data is the pre-filter threshold as is. */
int lgbm_hip_bin_mapper_from_sample(const double* values, int64_t num_values,
                                    int64_t total_sample_cnt, int32_t categorical,
                                    const lgbm_bin_params* params, int32_t min_split_data,
                                    const double* forced_upper_bounds, int32_t num_forced,
                                    lgbm_hip_bin_mapper** out);
int lgbm_hip_bin_mapper_free(lgbm_hip_bin_mapper* mapper);
/* Message of the last failed lgbm_hip_bin_mapper_from_* (process-wide). */
int lgbm_hip_bin_last_error(char* buf, size_t size);
int lgbm_hip_bin_mapper_info(const lgbm_hip_bin_mapper* mapper, lgbm_bin_mapper_info* out);
/* num_bin entries each (either may be NULL): numerical upper bounds
 * (bin_upper_bound_, NaN for the NaN bin), categorical bin -> category
 * (bin_2_categorical_, -1 for bin 0). */
int lgbm_hip_bin_mapper_bounds(const lgbm_hip_bin_mapper* mapper, double* upper,
                               int32_t* categories);
/* ValueToBin (bin_mapper.rs:148-189) on the host. */
int lgbm_hip_bin_mapper_value_to_bin(const lgbm_hip_bin_mapper* mapper, const double* values,
                                     int64_t n, uint32_t* out);
/* Random::sample (crates/lgbm-core/src/random.rs) of min(num_rows, sample_cnt) rows:
 * out (capacity min(num_rows, sample_cnt), may be NULL) gets the ascending indices. */
int lgbm_hip_sample_indices(int32_t num_rows, int32_t sample_cnt, int32_t seed, int32_t* out,
                            int32_t* out_len);

#define LGBM_HIP_DTYPE_F32 0
#define LGBM_HIP_DTYPE_F64 1
/* Bins a dense raw matrix on the device into the resident bin layout: the feature
 * columns of the booster's ingestion (crates/lgbm/src/booster.rs:449-520: value_to_bin
 * per row, one single-feature group per mapper, offset_for_most_freq_bin), replacing
 * lgbm_hip_upload_bins' host-binned input.  values: num_rows x num_cols of
 * LGBM_HIP_DTYPE_*, column-major ([col][row]) when col_major is set, else row-major;
 * mappers[num_cols] numerical (categorical: LGBM_HIP_ERR_CAPABILITY).  _device takes
 * device memory of the context's device; the other copies a host matrix over. */
int lgbm_hip_upload_raw_device(lgbm_hip_ctx* ctx, const void* d_values, int32_t dtype,
                               int32_t col_major, int64_t num_rows, int32_t num_cols,
                               const lgbm_hip_bin_mapper* const* mappers);
int lgbm_hip_upload_raw(lgbm_hip_ctx* ctx, const void* values, int32_t dtype, int32_t col_major,
                        int64_t num_rows, int32_t num_cols,
                        const lgbm_hip_bin_mapper* const* mappers);
/* The resident bins, feature-major [num_features][num_data] (no reference
 * counterpart: the reference's FeatureColumn.bins are host data); refused when a
 * feature holds more than 256 bins (lgbm_hip_get_bins16). */
int lgbm_hip_get_bins(lgbm_hip_ctx* ctx, uint8_t* out, int64_t num_data);
/* The same as 2-byte bins (any resident layout). */
int lgbm_hip_get_bins16(lgbm_hip_ctx* ctx, uint16_t* out, int64_t num_data);

/* 2-byte bin columns (`BinColumn::U16`, lgbm-compute/src/lib.rs:75-211;
 * `resident_bin_width`, :3752): like lgbm_hip_upload_bins for features of up to 4096
 * bins (categorical ones at most 256).  A feature of more than 256 bins selects the
 * wide row layout with 2-byte bins; otherwise the columns are stored as 1-byte bins.
 * lgbm_hip_upload_raw[_device] take mappers of up to 4096 bins the same way. */
int lgbm_hip_upload_bins16(lgbm_hip_ctx* ctx, const uint16_t* bins, int32_t num_features,
                           int64_t num_data, const lgbm_feature_meta* meta,
                           const double* bin_upper_bound);

/* ---- models and batch prediction ------------------------------------------ */

/* A LightGBM v4 model text, parsed on the host (no device needed): replaces
 * `lgbm_model::model_text::load` (crates/lgbm-model/src/model_text.rs:48-160) with
 * `Tree::parse` (tree.rs:846-1060) and the objective line (objective.rs:125-225).
 * Numerical and categorical splits; linear trees and objectives outside
 * objective.rs's list are rejected (LGBM_HIP_ERR_INVALID_ARGUMENT, like the
 * reference's MalformedModel).  The text is borrowed for the call only. */
typedef struct lgbm_hip_model lgbm_hip_model;
int lgbm_hip_model_load(const char* text, int64_t len, lgbm_hip_model** out);
int lgbm_hip_model_free(lgbm_hip_model* model);
/* Message of the last failed lgbm_hip_model_load / _create / _add_tree (process-wide). */
int lgbm_hip_model_last_error(char* buf, size_t size);
/* out[0] trees, [1] num_class, [2] num_tree_per_iteration, [3] max_feature_idx,
 * [4] iterations (trees / num_tree_per_iteration), [5] objective (PredObjective:
 * 0 regression, 1 regression sqrt, 2 binary, 3 multiclass, 4 multiclassova,
 * 5 poisson/gamma/tweedie, 6 cross_entropy, 7 cross_entropy_lambda). */
int lgbm_hip_model_info(const lgbm_hip_model* model, int64_t* out6);

/* A model built in memory, for trees grown by this library: the `GbdtModel` the
 * reference's boosting loop fills (crates/lgbm-boosting/src/gbdt.rs:1094-1140).
 * objective: the model text's objective= value (e.g. "binary sigmoid:1"), or NULL
 * for none; feature_names / feature_infos: the space-separated lines, or NULL for
 * `Column_<i>` / `none` per feature. */
int lgbm_hip_model_create(int32_t num_class, int32_t num_tree_per_iteration,
                          int32_t max_feature_idx, const char* objective,
                          const char* feature_names, const char* feature_infos,
                          lgbm_hip_model** out);
/* Appends a grown tree (lgbm_tree_out as lgbm_hip_train_iter_binary or
 * lgbm_hip_grow_tree_on_device fill it; leaf and internal values already shrunk)
 * recording `shrinkage` as Tree::shrinkage does (tree.rs:1074-1096), then adds
 * `bias` to every leaf and internal value (Tree::add_bias, tree.rs:1161-1168: the
 * boost-from-average init score folded into the first iteration's trees,
 * gbdt.rs:1130-1140; 0 for none).  internal_weight is written as 0 like Tree::split
 * (tree.rs:655).  The tree is checked like a loaded one. */
int lgbm_hip_model_add_tree(lgbm_hip_model* model, const lgbm_tree_out* tree, double shrinkage,
                            double bias);
/* The model text (`model_text::save`, crates/lgbm-model/src/model_text.rs:216-320:
 * envelope, Tree::to_string blocks (tree.rs:800-836), tree_sizes, split-count
 * feature_importances, the verbatim `parameters:` tail of a loaded model).  Writes
 * at most size bytes including a terminating NUL and sets *needed to the full size
 * with the NUL; LGBM_HIP_ERR_LENGTH_MISMATCH when buf was too small (truncated). */
int lgbm_hip_model_to_text(const lgbm_hip_model* model, char* buf, size_t size, size_t* needed);

#define LGBM_HIP_PREDICT_RAW 0
#define LGBM_HIP_PREDICT_TRANSFORMED 1
#define LGBM_HIP_PREDICT_LEAF 2
#define LGBM_HIP_PREDICT_CONTRIB 3
/* Batch prediction of a dense row-major f32 matrix [num_rows][num_cols]
 * (num_cols >= max_feature_idx + 1), over iterations [start_iteration,
 * start_iteration + num_iteration) clamped as GbdtModel::init_predict
 * (ensemble.rs:75-84; num_iteration <= 0: all).  Replaces predict_raw_mat_range,
 * predict_mat and predict_leaf_index_mat (crates/lgbm-model/src/predict.rs:75-131,
 * 378-485).  kind RAW / TRANSFORMED: out is double[num_rows * num_tree_per_iteration]
 * (the f64 scores the reference casts to f32 at its own boundary); LEAF: out is
 * int32[num_rows * trees in range], row-major, trees in model order; CONTRIB
 * (predict_contrib_mat, predict.rs:607-697, TreeSHAP of tree.rs:336-583): out is
 * double[num_rows * num_tree_per_iteration * (max_feature_idx + 2)], per row and
 * class the feature contributions then the expected-value base (refused for
 * linear-tree models, as predict.rs:626-635).  data and out are host pointers
 * (copied through the context's device buffers). */
int lgbm_hip_predict(lgbm_hip_ctx* ctx, const lgbm_hip_model* model, const float* data,
                     int64_t num_rows, int32_t num_cols, int32_t start_iteration,
                     int32_t num_iteration, int32_t kind, void* out);
/* The same with data and out in device memory of the context's device (no copies;
 * the call returns when the results are written). */
int lgbm_hip_predict_device(lgbm_hip_ctx* ctx, const lgbm_hip_model* model, const float* d_data,
                            int64_t num_rows, int32_t num_cols, int32_t start_iteration,
                            int32_t num_iteration, int32_t kind, void* d_out);

/* The same kinds over a CSR matrix (predict_raw_csr_range / predict_csr /
 * predict_leaf_index_csr / predict_contrib_csr, crates/lgbm-model/src/predict.rs:132-160,
 * 405-500, 699-722): indptr int64[num_rows + 1], indices int32[nnz], values
 * float[nnz], host pointers.  Each row is all 0.0 but its entries (a repeated column
 * keeps its last value; columns past max_feature_idx are ignored), as scatter_csr_row
 * (predict.rs:841-870).  LGBM_HIP_ERR_INVALID_ARGUMENT for an indptr pair outside
 * [0, nnz] or decreasing, LGBM_HIP_ERR_LENGTH_MISMATCH for a column outside
 * [0, num_cols). */
int lgbm_hip_predict_csr(lgbm_hip_ctx* ctx, const lgbm_hip_model* model, const int64_t* indptr,
                         const int32_t* indices, const float* values, int64_t nnz,
                         int64_t num_rows, int32_t num_cols, int32_t start_iteration,
                         int32_t num_iteration, int32_t kind, void* out);

/* The same over a CSC matrix (predict_raw_csc_range / predict_csc /
 * predict_leaf_index_csc / predict_contrib_csc): indptr int64[num_cols + 1], indices
 * (row numbers) int32[nnz], values float[nnz]; scatter_csc_dense (predict.rs:868-894):
 * a repeated row of a column keeps its last value.  LGBM_HIP_ERR_LENGTH_MISMATCH for a
 * row outside [0, num_rows). */
int lgbm_hip_predict_csc(lgbm_hip_ctx* ctx, const lgbm_hip_model* model, const int64_t* indptr,
                         const int32_t* indices, const float* values, int64_t nnz,
                         int64_t num_rows, int32_t num_cols, int32_t start_iteration,
                         int32_t num_iteration, int32_t kind, void* out);

/* Prediction early stopping: predict_raw_early_stop_mat (crates/lgbm-model/src/
 * predict.rs:557-605) over GbdtModel::predict_raw_early_stop (ensemble.rs:120-151).
 * Every `freq` iterations a row whose margin exceeds `margin` (binary: 2|score|;
 * multiclass: top score minus the second) stops; objectives that need accurate
 * prediction (all but binary / multiclass / multiclassova) evaluate the whole range.
 * out: double[num_rows * num_tree_per_iteration] raw scores; iterations (may be
 * NULL): int32[num_rows] iterations evaluated per row.  Host buffers. */
int lgbm_hip_predict_early_stop(lgbm_hip_ctx* ctx, const lgbm_hip_model* model, const float* data,
                                int64_t num_rows, int32_t num_cols, int32_t start_iteration,
                                int32_t num_iteration, int32_t freq, double margin, double* out,
                                int32_t* iterations);

/* ---- measurement ------------------------------------------------------------ */

/* LDS-atomic throughput probe (no counterpart in the reference: the ceiling that
 * ConstructHistogram's packed-cell adds run against).  2 x CUs blocks of 512 threads;
 * each thread holds one row's num_features (<= 32) bins and adds `reps` times one cell
 * per feature to an LDS histogram of num_features x 64 cells.  mode bits 0-1: the
 * bin of each add (0: the lane's index, 64 distinct cells; 1: the row's bin from
 * bins, host u8 feature-major [num_features][n]; 2: bin 0 for every lane), bit
 * 2: u64 cells (else u32), bit 3: one histogram per wave (u32 only; else one per
 * block).  out[5]: ms of the timed launch, lane adds, lane adds per CU-cycle at the
 * device's reported peak clock, that clock in MHz, CUs.  Allocates its own stream,
 * events and an 8-byte sink. */
int lgbm_hip_probe_lds_atomics(int device, const uint8_t* bins, int64_t n,
                               int32_t num_features, int32_t mode, int32_t reps, double* out);

#ifdef __cplusplus
}
#endif

#endif /* LGBM_HIP_H */
