// lgbm_oracle.cpp — CPU restatement of the reference learner spine.
//
// TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP path
// and the timed CPU baseline in bench.py.  Only tests/, __graft_entry__.smoke()
// and bench.py's cpu_baseline leg may load it; the product (lightgbm_rs_amd/)
// never does.
//
// It restates, function by function, the reference CPU path of
// BectorVoom/lightgbm_rs (paths relative to crates/):
//   histogram fold      lgbm-compute/src/kernels/histogram.rs:207-233,
//                       lgbm-compute/src/lib.rs:223-246,262-390,1422-1469
//   discretizer         lgbm-treelearner/src/gradient_discretizer.rs:55-263
//   quantize call site  lgbm-boosting/src/gbdt.rs:43-62,945-960
//   FixHistogram        lgbm-treelearner/src/fix_histogram.rs:50-80
//   compaction          lgbm-treelearner/src/learner.rs:4460-4492
//   subtract            lgbm-compute/src/kernels/subtract.rs:204-215
//   gain math           lgbm-compute/src/gain.rs:107-655
//   FindBestThreshold   lgbm-compute/src/kernels/split.rs:8970-9329
//   split_gt / arg_max  lgbm-treelearner/src/split_info.rs:28-35, learner.rs:4537
//   DataPartition       lgbm-treelearner/src/data_partition.rs:99-288,360-463
//   LeafSplits          lgbm-treelearner/src/leaf_splits.rs:75-173
//   learner loop        lgbm-treelearner/src/learner.rs:980-2453,2708-3355,3895-4092
//   Tree::split         lgbm-model/src/tree.rs:614-700, shrinkage :1074, add_bias :1161
//   binary objective    lgbm-objective/src/binary.rs:134-220
//   L2 regression       lgbm-objective/src/regression.rs:398-431,563-575
//   lambdarank          lgbm-objective/src/rank.rs:100-390,
//                       lgbm-metric/src/dcg_calculator.rs:40-170
//   softmax multiclass  lgbm-objective/src/multiclass.rs:48-200
//   Random / ColSampler lgbm-core/src/random.rs:37-123,
//                       lgbm-treelearner/src/col_sampler.rs:68-203, learner.rs:1190-1240
//   boosting loop       lgbm-boosting/src/gbdt.rs:612-640,691-1300,
//                       lgbm-boosting/src/objective.rs:100-140 (ranking: no init score)
//
// Numeric conventions follow the Rust source: no FP contraction anywhere (build
// with -ffp-contract=off) except the explicit fma in GetLeafGainGivenOutput
// (gain.rs:204-220); `as i8` / `as i32` casts saturate with NaN -> 0; f64::max is
// NaN-ignoring (fmax).
//
// Parallelism (OpenMP) mirrors the reference CpuBackend's structure and is
// bit-identical to the serial order: feature-group parallel histogram folds
// (lib.rs:681-704), feature-parallel scans (lib.rs:728-748) and a block-parallel
// two-buffer partition (data_partition.rs:489-615).

#include "../include/lgbm_hip.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>
#include <algorithm>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

const double kEps = (double)1e-15f;  // K_EPSILON (lgbm-core/src/types.rs:31) widened
const double kMinScore = -std::numeric_limits<double>::infinity();
const double kZeroThreshold = (double)1e-35f;  // tree.rs MaybeRoundToZero

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

// Rust `f64 as i8` (saturating, NaN -> 0).
inline int8_t sat_i8(double x) {
  if (std::isnan(x)) return 0;
  if (x >= 127.0) return 127;
  if (x <= -128.0) return -128;
  return (int8_t)(int)std::trunc(x);
}
// Rust `f64 as i32` (saturating, NaN -> 0).
inline int32_t sat_i32(double x) {
  if (std::isnan(x)) return 0;
  if (x >= 2147483647.0) return 2147483647;
  if (x <= -2147483648.0) return (int32_t)(-2147483647 - 1);
  return (int32_t)std::trunc(x);
}
// `Common::RoundInt` as the reference writes it (split.rs:9069).
inline int32_t round_int(double x) { return sat_i32(x + (double)0.5f); }

inline double maybe_round_to_zero(double v) {
  return (v >= -kZeroThreshold && v <= kZeroThreshold) ? 0.0 : v;
}

// ---------------------------------------------------------------------------
// gain.rs
// ---------------------------------------------------------------------------
// threshold_l1 (gain.rs:107-116): Sign(s) * max(0, |s| - l1), Sign(0) == 0.
inline double threshold_l1(double s, double l1) {
  double reg = std::fmax(0.0, std::fabs(s) - l1);
  double pos = s > 0.0 ? 1.0 : 0.0;
  double neg = s < 0.0 ? 1.0 : 0.0;
  return (pos - neg) * reg;
}
// get_leaf_gain (gain.rs:132-139)
inline double get_leaf_gain(bool use_l1, double g, double h, double l1, double l2) {
  if (use_l1) {
    double s = threshold_l1(g, l1);
    return (s * s) / (h + l2);
  }
  return (g * g) / (h + l2);
}
// get_split_gains (gain.rs:149-161)
inline double get_split_gains(bool use_l1, double lg, double lh, double rg, double rh, double l1,
                              double l2) {
  return get_leaf_gain(use_l1, lg, lh, l1, l2) + get_leaf_gain(use_l1, rg, rh, l1, l2);
}
// get_leaf_gain_given_output (gain.rs:204-220): the fused multiply-add is part of the
// reference arithmetic.
inline double get_leaf_gain_given_output(bool use_l1, double g, double h, double l1, double l2,
                                         double out) {
  double gg = use_l1 ? threshold_l1(g, l1) : g;
  return -std::fma(2.0 * gg, out, (h + l2) * out * out);
}
// calculate_splitted_leaf_output (gain.rs:232-249)
inline double calc_leaf_output(bool use_l1, double g, double h, double l1, double l2) {
  if (use_l1) return -threshold_l1(g, l1) / (h + l2);
  return -g / (h + l2);
}
// calculate_splitted_leaf_output_full (gain.rs:494-535)
inline double calc_leaf_output_full(bool use_l1, double g, double h, double l1, double l2,
                                    double max_delta_step, bool use_smoothing, double path_smooth,
                                    int32_t num_data, double parent_output) {
  double base = calc_leaf_output(use_l1, g, h, l1, l2);
  bool clamp = max_delta_step > 0.0 && std::fabs(base) > max_delta_step;
  double pos = base > 0.0 ? 1.0 : 0.0;
  double neg = base < 0.0 ? 1.0 : 0.0;
  double clamped = clamp ? (pos - neg) * max_delta_step : base;
  if (use_smoothing) {
    double n_over_ps = (double)num_data / path_smooth;
    return clamped * n_over_ps / (n_over_ps + 1.0) + parent_output / (n_over_ps + 1.0);
  }
  return clamped;
}
// get_leaf_gain_full (gain.rs:556-593)
inline double get_leaf_gain_full(bool use_l1, double g, double h, double l1, double l2,
                                 double max_delta_step, bool use_smoothing, double path_smooth,
                                 int32_t num_data, double parent_output) {
  if (max_delta_step > 0.0 || use_smoothing) {
    double out = calc_leaf_output_full(use_l1, g, h, l1, l2, max_delta_step, use_smoothing,
                                       path_smooth, num_data, parent_output);
    return get_leaf_gain_given_output(use_l1, g, h, l1, l2, out);
  }
  return get_leaf_gain(use_l1, g, h, l1, l2);
}
// get_split_gains_full (gain.rs:604-655)
inline double get_split_gains_full(bool use_l1, double lg, double lh, double rg, double rh,
                                   double l1, double l2, double mds, bool sm, double ps,
                                   int32_t lc, int32_t rc, double po) {
  return get_leaf_gain_full(use_l1, lg, lh, l1, l2, mds, sm, ps, lc, po) +
         get_leaf_gain_full(use_l1, rg, rh, l1, l2, mds, sm, ps, rc, po);
}

inline bool cfg_use_l1(const lgbm_gain_config& c) { return c.lambda_l1 > 0.0; }
inline bool cfg_use_smoothing(const lgbm_gain_config& c) { return c.path_smooth > kEps; }

lgbm_split_info split_none() {
  lgbm_split_info s;
  std::memset(&s, 0, sizeof(s));
  s.gain = kMinScore;
  s.default_left = 1;
  return s;
}

// ---------------------------------------------------------------------------
// find_best_split_cpu_native (kernels/split.rs:8970-9329)
// ---------------------------------------------------------------------------
// Candidate record (optional): every REVERSE / FORWARD candidate the scan visits, in
// scan order, as the gain it compares against min_gain_shift, or NaN where the
// candidate is gated out (default-bin skip, continue gate, the break candidate, or a
// gain not above min_gain_shift).  The scan stops after a break candidate.  This is
// the encoding of the reference's SCAND_REV / SCAND_FWD goldens (kernel_parity.rs:
// 369-466).
struct ScanCandidates {
  std::vector<double> rev, fwd;
};

int find_best_split(const double* hist, size_t hist_len, const lgbm_gain_config& cfg,
                    uint32_t num_bin, int32_t offset, uint32_t default_bin,
                    bool skip_default_bin, bool na_as_missing, bool run_forward,
                    double sum_gradient, double sum_hessian, int32_t num_data,
                    lgbm_split_info* out, ScanCandidates* cand = nullptr) {
  const double kNaN = std::numeric_limits<double>::quiet_NaN();
  if (num_bin == 0) return fail(LGBM_HIP_ERR_RUNTIME, "find_best_split: num_bin must be > 0");
  if (hist_len != 2ull * num_bin) return fail(LGBM_HIP_ERR_LENGTH_MISMATCH, "hist length");
  if (!(sum_hessian > 0.0))
    return fail(LGBM_HIP_ERR_RUNTIME, "find_best_split: sum_hessian must be > 0");
  const double two_eps = 2.0 * kEps;
  const double sum_hessian_bumped = sum_hessian + two_eps;
  const bool use_l1 = cfg_use_l1(cfg);
  const bool use_smoothing = cfg_use_smoothing(cfg);
  const double mds = cfg.max_delta_step;
  const double po = cfg.parent_output;
  const bool use_full = use_smoothing || mds > 0.0;
  const double gain_shift =
      get_leaf_gain_full(use_l1, sum_gradient, sum_hessian_bumped, cfg.lambda_l1, cfg.lambda_l2,
                         mds, use_smoothing, cfg.path_smooth, num_data, po);
  const double min_gain_shift = gain_shift + cfg.min_gain_to_split;
  const int32_t nb = (int32_t)num_bin;
  const int32_t rev_count = std::max(nb - 1 - (na_as_missing ? 1 : 0), 0);
  const bool na_preamble = na_as_missing && offset == 1;
  int32_t fwd_count = 0;
  if (run_forward) {
    int32_t base = std::max(nb - 1 - offset, 0);
    fwd_count = na_preamble ? base + 1 : base;
  }
  const double l1 = cfg.lambda_l1, l2 = cfg.lambda_l2;
  const double cnt_factor = (double)num_data / sum_hessian_bumped;
  const double min_h = cfg.min_sum_hessian_in_leaf;
  const int32_t min_d = cfg.min_data_in_leaf;

  double best_lg = 0.0, best_lh = 0.0, best_gain = kMinScore;
  int32_t best_lc = 0, best_thr = 0;
  bool is_splittable = false, best_dl = true;

  auto gain_of = [&](double lg, double lh, double rg, double rh, int32_t lc, int32_t rc) {
    if (use_full)
      return get_split_gains_full(use_l1, lg, lh, rg, rh, l1, l2, mds, use_smoothing,
                                  cfg.path_smooth, lc, rc, po);
    return get_split_gains(use_l1, lg, lh, rg, rh, l1, l2);
  };

  {  // REVERSE
    double srg = 0.0, srh = kEps;
    int32_t rc = 0;
    const int32_t t_start = nb - 1 - offset - (na_as_missing ? 1 : 0);
    bool done = false;
    for (int32_t k = 0; k < rev_count; ++k) {
      if (done) break;
      const int32_t t = t_start - k;
      const bool in_range = t >= (1 - offset);
      const bool skip = skip_default_bin && (t + offset) == (int32_t)default_bin;
      const bool active = in_range && !skip && !done;
      if (active) {
        double hg = hist[(size_t)t * 2], hh = hist[(size_t)t * 2 + 1];
        srg += hg;
        srh += hh;
        rc += round_int(hh * cnt_factor);
      }
      const int32_t lc = num_data - rc;
      const double slh = sum_hessian_bumped - srh;
      const double slg = sum_gradient - srg;
      const bool cont = rc < min_d || srh < min_h;
      const bool brk = lc < min_d || slh < min_h;
      done = done || (active && !cont && brk);
      double rec = kNaN;
      if (active && !cont && !done) {
        double g = gain_of(slg, slh, srg, srh, lc, rc);
        if (g > min_gain_shift) {
          rec = g;
          is_splittable = true;
          if (g > best_gain) {
            best_lc = lc;
            best_lg = slg;
            best_lh = slh;
            best_thr = t - 1 + offset;
            best_gain = g;
            best_dl = true;
          }
        }
      }
      if (cand) cand->rev.push_back(rec);
    }
  }
  {  // FORWARD
    double slg = 0.0, slh = kEps;
    int32_t lc = 0;
    int32_t fwd_start = 0;
    if (na_preamble) {
      slg = sum_gradient;
      slh = sum_hessian_bumped - kEps;
      lc = num_data;
      for (int32_t i = 0; i < nb - offset; ++i) {
        slg -= hist[(size_t)i * 2];
        slh -= hist[(size_t)i * 2 + 1];
        lc -= round_int(hist[(size_t)i * 2 + 1] * cnt_factor);
      }
      fwd_start = -1;
    }
    bool done = false;
    for (int32_t k = 0; k < fwd_count; ++k) {
      if (done) break;
      const int32_t t = fwd_start + k;
      const bool skip = skip_default_bin && (t + offset) == (int32_t)default_bin;
      const bool active = !skip && !done;
      if (active && t >= 0) {
        double hg = hist[(size_t)t * 2], hh = hist[(size_t)t * 2 + 1];
        slg += hg;
        slh += hh;
        lc += round_int(hh * cnt_factor);
      }
      const int32_t rc = num_data - lc;
      const double srh = sum_hessian_bumped - slh;
      const double srg = sum_gradient - slg;
      const bool cont = lc < min_d || slh < min_h;
      const bool brk = rc < min_d || srh < min_h;
      done = done || (active && !cont && brk);
      double rec = kNaN;
      if (active && !cont && !done) {
        double g = gain_of(slg, slh, srg, srh, lc, rc);
        if (g > min_gain_shift) {
          rec = g;
          is_splittable = true;
          if (g > best_gain) {
            best_lc = lc;
            best_lg = slg;
            best_lh = slh;
            best_thr = t + offset;
            best_gain = g;
            best_dl = false;
          }
        }
      }
      if (cand) cand->fwd.push_back(rec);
    }
  }
  const int32_t best_rc = num_data - best_lc;
  const double lo = calc_leaf_output_full(use_l1, best_lg, best_lh, l1, l2, mds, use_smoothing,
                                          cfg.path_smooth, best_lc, po);
  const double rsg = sum_gradient - best_lg;
  const double rsh = sum_hessian_bumped - best_lh;
  const double ro = calc_leaf_output_full(use_l1, rsg, rsh, l1, l2, mds, use_smoothing,
                                          cfg.path_smooth, best_rc, po);
  if (is_splittable && best_gain > kMinScore) {
    out->threshold = (uint32_t)best_thr;
    out->gain = best_gain - min_gain_shift;
    out->left_count = best_lc;
    out->right_count = num_data - best_lc;
    out->left_sum_gradient = best_lg;
    out->left_sum_hessian = best_lh - kEps;
    out->right_sum_gradient = rsg;
    out->right_sum_hessian = rsh - kEps;
    out->left_output = lo;
    out->right_output = ro;
    out->default_left = best_dl ? 1 : 0;
  } else {
    *out = split_none();
  }
  return LGBM_HIP_OK;
}

// split_gt (split_info.rs:28-35)
inline bool split_gt(const lgbm_split_info& a, int32_t af, const lgbm_split_info& b, int32_t bf) {
  if (a.gain != b.gain) return a.gain > b.gain;
  int32_t x = af == -1 ? std::numeric_limits<int32_t>::max() : af;
  int32_t y = bf == -1 ? std::numeric_limits<int32_t>::max() : bf;
  return x < y;
}

// fix_histogram (fix_histogram.rs:50-80)
void fix_histogram(double* hist, uint32_t num_bin, uint32_t mfb, double sum_g, double sum_h) {
  if (mfb == 0 || mfb >= num_bin) return;
  double g = sum_g, h = sum_h;
  for (uint32_t i = 0; i < num_bin; ++i) {
    if (i != mfb) {
      g -= hist[(size_t)i * 2];
      h -= hist[(size_t)i * 2 + 1];
    }
  }
  hist[(size_t)mfb * 2] = g;
  hist[(size_t)mfb * 2 + 1] = h;
}

// compact_histogram (learner.rs:4460-4492)
void compact_histogram(double* hist, uint32_t num_bin, int32_t offset) {
  if (offset <= 0) return;
  uint32_t off = (uint32_t)offset;
  if (off >= num_bin) {
    for (size_t i = 0; i < 2ull * num_bin; ++i) hist[i] = 0.0;
    return;
  }
  for (uint32_t c = 0; c < num_bin - off; ++c) {
    hist[(size_t)c * 2] = hist[(size_t)(c + off) * 2];
    hist[(size_t)c * 2 + 1] = hist[(size_t)(c + off) * 2 + 1];
  }
  for (size_t i = (size_t)(num_bin - off) * 2; i < 2ull * num_bin; ++i) hist[i] = 0.0;
}

// ---------------------------------------------------------------------------
// Categorical split finding: find_best_threshold_categorical
// (lgbm-treelearner/src/feature_histogram_categorical.rs:96-495), the one-hot scan
// for num_bin <= max_cat_to_onehot, else many-vs-many over the bins sorted by
// grad / (hess + cat_smooth).  sum_hessian arrives bumped by 2 kEpsilon (the caller,
// learner.rs:3104-3118).  out->threshold is 0, default_left false; cat_bins
// receives the winning REAL bins (cat_threshold of the reference).
// ---------------------------------------------------------------------------
void find_best_threshold_categorical(const double* hist, const lgbm_gain_config& cfg,
                                     int32_t num_bin, int32_t offset, double sum_gradient,
                                     double sum_hessian, int32_t num_data, lgbm_split_info* out,
                                     std::vector<uint32_t>* cat_bins) {
  const bool use_l1 = cfg_use_l1(cfg);
  const double l1 = cfg.lambda_l1, eps = kEps;
  const double mds = cfg.max_delta_step, ps = cfg.path_smooth, parent = cfg.parent_output;
  const bool smoothing = cfg_use_smoothing(cfg);
  auto G = [&](int32_t t) { return hist[(size_t)t * 2]; };
  auto Hs = [&](int32_t t) { return hist[(size_t)t * 2 + 1]; };
  bool is_splittable = false;
  double best_gain = kMinScore, best_lg = 0.0, best_lh = 0.0;
  int32_t best_lc = 0;
  // gain_shift with the ORIGINAL l2 (the deliberate asymmetry, :123-157)
  const double gain_shift =
      smoothing ? get_leaf_gain_given_output(use_l1, sum_gradient, sum_hessian, l1, cfg.lambda_l2,
                                             parent)
                : get_leaf_gain_full(use_l1, sum_gradient, sum_hessian, l1, cfg.lambda_l2, mds,
                                     false, 0.0, num_data, 0.0);
  const double min_gain_shift = gain_shift + cfg.min_gain_to_split;
  const int32_t bin_start = 1 - offset, bin_end = num_bin - offset;
  const double cnt_factor = (double)num_data / sum_hessian;
  const bool use_onehot = num_bin <= cfg.max_cat_to_onehot;
  std::vector<int32_t> sorted_idx;
  int32_t used_bin = -1, best_threshold = -1, best_dir = 1;
  double l2 = cfg.lambda_l2;
  if (use_onehot) {
    for (int32_t t = bin_start; t < bin_end; ++t) {
      const double grad = G(t), hess = Hs(t);
      const int32_t cnt = round_int(hess * cnt_factor);
      if (cnt < cfg.min_data_in_leaf || hess < cfg.min_sum_hessian_in_leaf) continue;
      const int32_t other_count = num_data - cnt;
      if (other_count < cfg.min_data_in_leaf) continue;
      const double sum_other_hessian = sum_hessian - hess - eps;
      if (sum_other_hessian < cfg.min_sum_hessian_in_leaf) continue;
      const double sum_other_gradient = sum_gradient - grad;
      const double g = get_split_gains_full(use_l1, sum_other_gradient, sum_other_hessian, grad,
                                            hess + eps, l1, l2, mds, smoothing, ps, other_count,
                                            cnt, parent);
      if (g <= min_gain_shift) continue;
      is_splittable = true;
      if (g > best_gain) {
        best_threshold = t;
        best_lg = grad;
        best_lh = hess + eps;
        best_lc = cnt;
        best_gain = g;
      }
    }
  } else {
    for (int32_t i = bin_start; i < bin_end; ++i)
      if ((double)round_int(Hs(i) * cnt_factor) >= cfg.cat_smooth) sorted_idx.push_back(i);
    used_bin = (int32_t)sorted_idx.size();
    l2 += cfg.cat_l2;
    const double cat_smooth = cfg.cat_smooth;
    auto ctr = [&](int32_t t) { return G(t) / (Hs(t) + cat_smooth); };
    std::stable_sort(sorted_idx.begin(), sorted_idx.end(),
                     [&](int32_t a, int32_t b) { return ctr(a) < ctr(b); });
    const int32_t dirs[2] = {1, -1}, starts[2] = {0, used_bin - 1};
    const int32_t max_num_cat = std::min(cfg.max_cat_threshold, (used_bin + 1) / 2);
    is_splittable = false;
    for (int o = 0; o < 2; ++o) {
      const int32_t dir = dirs[o];
      int32_t start_pos = starts[o], cnt_cur_group = 0, left_count = 0;
      double slg = 0.0, slh = eps;
      for (int32_t i = 0; i < used_bin && i < max_num_cat; ++i) {
        const int32_t t = sorted_idx[(size_t)start_pos];
        start_pos += dir;
        const double grad = G(t), hess = Hs(t);
        const int32_t cnt = round_int(hess * cnt_factor);
        slg += grad;
        slh += hess;
        left_count += cnt;
        cnt_cur_group += cnt;
        if (left_count < cfg.min_data_in_leaf || slh < cfg.min_sum_hessian_in_leaf) continue;
        const int32_t right_count = num_data - left_count;
        if (right_count < cfg.min_data_in_leaf || right_count < cfg.min_data_per_group) break;
        const double srh = sum_hessian - slh;
        if (srh < cfg.min_sum_hessian_in_leaf) break;
        if (cnt_cur_group < cfg.min_data_per_group) continue;
        cnt_cur_group = 0;
        const double srg = sum_gradient - slg;
        const double g = get_split_gains_full(use_l1, slg, slh, srg, srh, l1, l2, mds, smoothing, ps,
                                              left_count, right_count, parent);
        if (g <= min_gain_shift) continue;
        is_splittable = true;
        if (g > best_gain) {
          best_lc = left_count;
          best_lg = slg;
          best_lh = slh;
          best_threshold = i;
          best_gain = g;
          best_dir = dir;
        }
      }
    }
  }
  cat_bins->clear();
  if (!is_splittable) {
    *out = split_none();
    out->default_left = 0;
    return;
  }
  // finalize (:395-495): outputs with this scan's l2, counts, sums, net gain, bins
  const int32_t rc_out = num_data - best_lc;
  out->left_output = calc_leaf_output_full(use_l1, best_lg, best_lh, l1, l2, mds, smoothing, ps,
                                           best_lc, parent);
  out->left_count = best_lc;
  out->left_sum_gradient = best_lg;
  out->left_sum_hessian = best_lh - eps;
  out->right_output = calc_leaf_output_full(use_l1, sum_gradient - best_lg, sum_hessian - best_lh,
                                            l1, l2, mds, smoothing, ps, rc_out, parent);
  out->right_count = rc_out;
  out->right_sum_gradient = sum_gradient - best_lg;
  out->right_sum_hessian = sum_hessian - best_lh - eps;
  out->gain = best_gain - min_gain_shift;
  out->default_left = 0;
  out->threshold = 0;
  if (use_onehot) {
    cat_bins->push_back((uint32_t)(best_threshold + offset));
  } else {
    for (int32_t i = 0; i < best_threshold + 1; ++i) {
      const int32_t t = best_dir == 1 ? sorted_idx[(size_t)i] : sorted_idx[(size_t)(used_bin - 1 - i)];
      cat_bins->push_back((uint32_t)(t + offset));
    }
  }
}

// Common::ConstructBitset (feature_histogram_categorical.rs:499-510): 32-bit blocks,
// max(vals) / 32 + 1 of them.
std::vector<uint32_t> construct_bitset(const std::vector<uint32_t>& vals) {
  std::vector<uint32_t> bits;
  if (vals.empty()) return bits;
  const uint32_t mx = *std::max_element(vals.begin(), vals.end());
  bits.assign(mx / 32 + 1, 0u);
  for (uint32_t v : vals) bits[v / 32] |= 1u << (v % 32);
  return bits;
}

// ---------------------------------------------------------------------------
// GradientDiscretizer (gradient_discretizer.rs)
// ---------------------------------------------------------------------------
struct Discretizer {
  int32_t bins;
  bool const_hess;
  bool stochastic;
  uint64_t rng;
  double gs = 0, hs = 0, igs = 0, ihs = 0;

  // next_u01 (gradient_discretizer.rs:255-263)
  double next_u01() {
    uint64_t x = rng;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    rng = x;
    return (double)(x >> 11) / (double)(1ull << 53);
  }
  // compute_scales (:145-165)
  void compute_scales(const float* g, const float* h, int64_t n) {
    double mg = std::fabs((double)g[0]), mh = std::fabs((double)h[0]);
    for (int64_t i = 0; i < n; ++i) {
      mg = std::fmax(mg, std::fabs((double)g[i]));
      mh = std::fmax(mh, std::fabs((double)h[i]));
    }
    double half = (double)(bins / 2);
    gs = mg / half;
    hs = const_hess ? mh : mh / (double)bins;
    igs = 1.0 / gs;
    ihs = 1.0 / hs;
  }
  // quantize_pair (:173-188)
  void quantize_pair(float g, float h, int8_t* qg, int8_t* qh) {
    double bg = 0.5, bh = 0.5;
    if (stochastic) {
      bg = next_u01();
      bh = next_u01();
    }
    double x = (double)g * igs;
    *qg = sat_i8(g >= 0.0f ? x + bg : x - bg);
    *qh = const_hess ? (int8_t)1 : sat_i8((double)h * ihs + bh);
  }
};

Discretizer make_discretizer(int32_t bins, bool const_hess, bool stochastic, uint64_t seed) {
  Discretizer d;
  d.bins = bins;
  d.const_hess = const_hess;
  d.stochastic = stochastic;
  d.rng = stochastic ? (seed ^ 0x9E3779B97F4A7C15ull) : 0;  // new_stochastic (:78-84)
  return d;
}

bool is_constant_hessian(const float* h, int64_t n) {  // gbdt.rs:54
  for (int64_t i = 0; i < n; ++i)
    if (!(h[i] == h[0])) return false;
  return true;
}

// quantize_grad_hess_in_place (gbdt.rs:43-62) -> discretize_dequantize_in_place (:126-139)
void quantize_in_place(float* g, float* h, int64_t n, int32_t bins, bool stochastic, uint64_t seed,
                       int8_t* disc_out, double* scales) {
  if (n == 0) return;
  bool ch = is_constant_hessian(h, n);
  Discretizer d = make_discretizer(bins, ch, stochastic, seed);
  d.compute_scales(g, h, n);
  for (int64_t i = 0; i < n; ++i) {
    int8_t qg, qh;
    d.quantize_pair(g[i], h[i], &qg, &qh);
    if (disc_out) {
      disc_out[2 * i] = qh;
      disc_out[2 * i + 1] = qg;
    }
    g[i] = (float)((double)qg * d.gs);
    h[i] = (float)((double)qh * d.hs);
  }
  if (scales) {
    scales[0] = d.gs;
    scales[1] = d.hs;
  }
}

// ---------------------------------------------------------------------------
// Bin columns (BinColumn, lib.rs:75-211): u8 / u16 / u32 feature-major storage.
// ---------------------------------------------------------------------------
struct Bins {
  const void* data;
  int width;  // 1, 2 or 4 bytes
  int64_t n;
  inline uint32_t at(int f, int64_t row) const {
    size_t i = (size_t)f * (size_t)n + (size_t)row;
    if (width == 1) return ((const uint8_t*)data)[i];
    if (width == 2) return ((const uint16_t*)data)[i];
    return ((const uint32_t*)data)[i];
  }
};

// fold_one_feature (lib.rs:223-246): ascending leaf rows, f32 read -> f64 accumulate.
template <typename T>
void fold_feature_t(const T* col, const uint32_t* rows, int64_t nr, const float* og,
                    const float* oh, double* h) {
  for (int64_t k = 0; k < nr; ++k) {
    size_t b = (size_t)col[rows[k]] * 2;
    h[b] += (double)og[k];
    h[b + 1] += (double)oh[k];
  }
}
// fold_u8_x4 (lib.rs:484-519): four independent per-feature chains in one walk.
void fold_u8_x4(const uint8_t* c0, const uint8_t* c1, const uint8_t* c2, const uint8_t* c3,
                const uint32_t* rows, int64_t nr, const float* og, const float* oh, double* h0,
                double* h1, double* h2, double* h3) {
  for (int64_t k = 0; k < nr; ++k) {
    uint32_t r = rows[k];
    double g = (double)og[k], hh = (double)oh[k];
    size_t b0 = (size_t)c0[r] * 2, b1 = (size_t)c1[r] * 2, b2 = (size_t)c2[r] * 2,
           b3 = (size_t)c3[r] * 2;
    h0[b0] += g;
    h0[b0 + 1] += hh;
    h1[b1] += g;
    h1[b1 + 1] += hh;
    h2[b2] += g;
    h2[b2 + 1] += hh;
    h3[b3] += g;
    h3[b3 + 1] += hh;
  }
}

void fold_feature(const Bins& bins, int f, const uint32_t* rows, int64_t nr, const float* og,
                  const float* oh, double* h) {
  size_t base = (size_t)f * (size_t)bins.n;
  if (bins.width == 1)
    fold_feature_t((const uint8_t*)bins.data + base, rows, nr, og, oh, h);
  else if (bins.width == 2)
    fold_feature_t((const uint16_t*)bins.data + base, rows, nr, og, oh, h);
  else
    fold_feature_t((const uint32_t*)bins.data + base, rows, nr, og, oh, h);
}

// build_histograms_into (lib.rs:262-390): zero, then fold every used feature;
// features are grouped by 4 and the groups run in parallel for large leaves
// (par_build_threshold, lib.rs:681-704).  Order within a feature is ascending rows
// in every arm, so the result is thread-count independent.
void build_histograms_into(const Bins& bins, const std::vector<uint32_t>& num_bin,
                           const std::vector<size_t>& slot_off, const uint32_t* rows, int64_t nr,
                           const float* og, const float* oh, const std::vector<char>* used,
                           double* out, size_t slot_len) {
  std::fill(out, out + slot_len, 0.0);
  const int F = (int)num_bin.size();
  std::vector<int> act;
  for (int f = 0; f < F; ++f)
    if (!used || (*used)[f]) act.push_back(f);
  const int ng = ((int)act.size() + 3) / 4;
  auto run_group = [&](int gi) {
    int a = gi * 4;
    int cnt = std::min(4, (int)act.size() - a);
    if (cnt == 4 && bins.width == 1) {
      const uint8_t* b = (const uint8_t*)bins.data;
      size_t n = (size_t)bins.n;
      fold_u8_x4(b + act[a] * n, b + act[a + 1] * n, b + act[a + 2] * n, b + act[a + 3] * n, rows,
                 nr, og, oh, out + slot_off[act[a]], out + slot_off[act[a + 1]],
                 out + slot_off[act[a + 2]], out + slot_off[act[a + 3]]);
    } else {
      for (int j = 0; j < cnt; ++j) fold_feature(bins, act[a + j], rows, nr, og, oh, out + slot_off[act[a + j]]);
    }
  };
  const bool parallel = nr >= 64;  // par_build_threshold default (lib.rs:681-704)
#pragma omp parallel for schedule(dynamic, 1) if (parallel && ng > 1)
  for (int gi = 0; gi < ng; ++gi) run_group(gi);
}

// ---------------------------------------------------------------------------
// Tree (lgbm-model/src/tree.rs)
// ---------------------------------------------------------------------------
struct Tree {
  int32_t num_leaves = 1;
  std::vector<int32_t> split_feature, left_child, right_child, internal_count, leaf_count,
      leaf_depth, leaf_parent;
  std::vector<uint32_t> threshold_in_bin;
  std::vector<double> threshold, internal_value, internal_weight, leaf_value, leaf_weight;
  std::vector<float> split_gain;
  std::vector<int8_t> decision_type;
  int32_t num_cat = 0;
  std::vector<int32_t> cat_boundaries;  // {0, ...} once a categorical node exists
  std::vector<uint32_t> cat_threshold;   // real-category bitsets, concatenated

  // root_tree (learner.rs:5398-5424)
  static Tree root(double out, int32_t n) {
    Tree t;
    t.leaf_value = {out};
    t.leaf_weight = {0.0};
    t.leaf_count = {n};
    t.leaf_depth = {0};
    t.leaf_parent = {-1};
    return t;
  }
  // Tree::split (tree.rs:614-700)
  void split(int32_t leaf, int32_t real_feature, uint32_t thr_bin, double thr, double lv, double rv,
             int32_t lc, int32_t rc, double lw, double rw, float gain, int8_t missing_type,
             bool default_left) {
    int32_t node = num_leaves - 1;
    int32_t new_leaf = num_leaves;
    int32_t parent = leaf_parent[leaf];
    if (parent >= 0) {
      if (right_child[parent] == ~leaf)
        right_child[parent] = node;
      else
        left_child[parent] = node;
    }
    split_feature.push_back(real_feature);
    split_gain.push_back(gain);
    threshold_in_bin.push_back(thr_bin);
    threshold.push_back(thr);
    internal_value.push_back(leaf_value[leaf]);
    internal_count.push_back(lc + rc);
    internal_weight.push_back(lw + rw);  // C++ Tree::Split (tree.rs:655 keeps 0)
    left_child.push_back(~leaf);
    right_child.push_back(~new_leaf);
    int8_t dt = 0;
    if (default_left) dt |= 2;  // kDefaultLeftMask
    dt |= (int8_t)((missing_type & 3) << 2);
    decision_type.push_back(dt);
    leaf_value[leaf] = lv;
    leaf_weight[leaf] = lw;
    leaf_count[leaf] = lc;
    leaf_value.push_back(rv);
    leaf_weight.push_back(rw);
    leaf_count.push_back(rc);
    leaf_depth.push_back(leaf_depth[leaf] + 1);
    leaf_depth[leaf] += 1;
    leaf_parent[leaf] = node;
    leaf_parent.push_back(node);
    num_leaves += 1;
  }
  // Tree::split_categorical (tree.rs:710-790): threshold / threshold_in_bin hold the
  // node's categorical index, decision_type the categorical bit and the missing type;
  // the category bitset (over category VALUES) is appended to cat_threshold.
  void split_categorical(int32_t leaf, int32_t real_feature, const std::vector<uint32_t>& bits,
                         double lv, double rv, int32_t lc, int32_t rc, double lw, double rw,
                         float gain, int8_t missing_type) {
    const int32_t node = num_leaves - 1, new_leaf = num_leaves;
    const int32_t parent = leaf_parent[leaf];
    if (parent >= 0) {
      if (right_child[parent] == ~leaf)
        right_child[parent] = node;
      else
        left_child[parent] = node;
    }
    split_feature.push_back(real_feature);
    split_gain.push_back(gain);
    threshold_in_bin.push_back((uint32_t)num_cat);
    threshold.push_back((double)num_cat);
    internal_value.push_back(leaf_value[leaf]);
    internal_count.push_back(lc + rc);
    internal_weight.push_back(lw + rw);  // C++ Tree::SplitCategorical
    left_child.push_back(~leaf);
    right_child.push_back(~new_leaf);
    decision_type.push_back((int8_t)(1 | ((missing_type & 3) << 2)));  // kCategoricalMask
    if (cat_boundaries.empty()) cat_boundaries.push_back(0);
    cat_boundaries.push_back(cat_boundaries.back() + (int32_t)bits.size());
    cat_threshold.insert(cat_threshold.end(), bits.begin(), bits.end());
    num_cat += 1;
    leaf_value[leaf] = lv;
    leaf_weight[leaf] = lw;
    leaf_count[leaf] = lc;
    leaf_value.push_back(rv);
    leaf_weight.push_back(rw);
    leaf_count.push_back(rc);
    leaf_depth.push_back(leaf_depth[leaf] + 1);
    leaf_depth[leaf] += 1;
    leaf_parent[leaf] = node;
    leaf_parent.push_back(node);
    num_leaves += 1;
  }
  void shrinkage(double rate) {  // tree.rs:1074
    for (auto& v : leaf_value) v = maybe_round_to_zero(v * rate);
    for (auto& v : internal_value) v = maybe_round_to_zero(v * rate);
  }
  void add_bias(double val) {  // tree.rs:1161
    for (auto& v : leaf_value) v = maybe_round_to_zero(v + val);
    for (auto& v : internal_value) v = maybe_round_to_zero(v + val);
  }
  void to_out(lgbm_tree_out* o) const {
    o->num_leaves = num_leaves;
    for (int i = 0; i < num_leaves - 1; ++i) {
      if (o->split_feature) o->split_feature[i] = split_feature[i];
      if (o->threshold_in_bin) o->threshold_in_bin[i] = threshold_in_bin[i];
      if (o->threshold) o->threshold[i] = threshold[i];
      if (o->split_gain) o->split_gain[i] = split_gain[i];
      if (o->decision_type) o->decision_type[i] = decision_type[i];
      if (o->left_child) o->left_child[i] = left_child[i];
      if (o->right_child) o->right_child[i] = right_child[i];
      if (o->internal_value) o->internal_value[i] = internal_value[i];
      if (o->internal_count) o->internal_count[i] = internal_count[i];
      if (o->internal_weight) o->internal_weight[i] = internal_weight[i];
    }
    for (int i = 0; i < num_leaves; ++i) {
      if (o->leaf_value) o->leaf_value[i] = leaf_value[i];
      if (o->leaf_weight) o->leaf_weight[i] = leaf_weight[i];
      if (o->leaf_count) o->leaf_count[i] = leaf_count[i];
      if (o->leaf_depth) o->leaf_depth[i] = leaf_depth[i];
      if (o->leaf_parent) o->leaf_parent[i] = leaf_parent[i];
    }
    o->num_cat = num_cat;
    if (num_cat > 0) {
      if (o->cat_boundaries)
        for (size_t i = 0; i < cat_boundaries.size(); ++i) o->cat_boundaries[i] = cat_boundaries[i];
      if (o->cat_threshold && (int64_t)cat_threshold.size() <= (int64_t)o->cat_threshold_cap)
        for (size_t i = 0; i < cat_threshold.size(); ++i) o->cat_threshold[i] = cat_threshold[i];
    }
  }
};

// ---------------------------------------------------------------------------
// DataPartition (data_partition.rs)
// ---------------------------------------------------------------------------
struct Router {  // split_fused_host_impl router (data_partition.rs:387-417)
  int32_t min_b, max_b, th, na_bin;
  bool default_to_right, na, default_left;
  Router(uint32_t num_bin, uint32_t min_bin, uint32_t max_bin, uint32_t threshold, uint32_t mfb,
         bool na_as_missing, bool dl) {
    min_b = (int32_t)min_bin;
    max_b = (int32_t)max_bin;
    th = (int32_t)threshold + min_b;
    if (mfb == 0) th -= 1;
    default_to_right = (int32_t)mfb > (int32_t)threshold;
    na_bin = (int32_t)num_bin - 1;
    na = na_as_missing;
    default_left = dl;
  }
  inline bool go_right(uint32_t b) const {
    int32_t bin = (int32_t)b;
    if (na && bin == na_bin) return !default_left;
    if (bin < min_b || bin > max_b) return default_to_right;
    return bin > th;
  }
};

struct DataPartition {
  // split_categorical (data_partition.rs:636-686): rows whose bin is in `left_bins`
  // go left, the others (bin 0, the NaN / unseen category, included) right; stable.
  int split_categorical(int32_t leaf, int32_t right_leaf, const Bins& bins, int f,
                        const std::vector<char>& left_bin) {
    const int64_t begin = leaf_begin[leaf], count = leaf_count[leaf];
    uint32_t* idx = indices.data() + begin;
    int64_t lc = 0, rc = 0;
    for (int64_t i = 0; i < count; ++i) {
      const uint32_t row = idx[i];
      const uint32_t b = bins.at(f, row);
      const bool left = b < left_bin.size() && left_bin[b];
      part_left[lc] = row;
      part_right[rc] = row;
      lc += left ? 1 : 0;
      rc += left ? 0 : 1;
    }
    std::memcpy(idx, part_left.data(), (size_t)lc * 4);
    std::memcpy(idx + lc, part_right.data(), (size_t)rc * 4);
    leaf_count[leaf] = (int32_t)lc;
    leaf_begin[right_leaf] = (int32_t)(begin + lc);
    leaf_count[right_leaf] = (int32_t)rc;
    return LGBM_HIP_OK;
  }
  int64_t n;
  std::vector<uint32_t> indices, part_left, part_right;
  std::vector<int32_t> leaf_begin, leaf_count;
  DataPartition(int64_t num_data, int32_t num_leaves)
      : n(num_data), indices(num_data), part_left(num_data), part_right(num_data),
        leaf_begin(std::max(num_leaves, 1), 0), leaf_count(std::max(num_leaves, 1), 0) {
    for (int64_t i = 0; i < num_data; ++i) indices[i] = (uint32_t)i;
    leaf_count[0] = (int32_t)num_data;
  }
  // split (:192-288) with the two-buffer serial body (:418-463) or the block-parallel
  // body (:489-615); both produce [left ascending | right ascending].
  int split(int32_t leaf, int32_t right_leaf, const Bins& bins, int f, uint32_t num_bin,
            uint32_t min_bin, uint32_t max_bin, uint32_t threshold, uint32_t mfb, bool na,
            bool default_left) {
    if (num_bin == 0) return fail(LGBM_HIP_ERR_RUNTIME, "data_partition: num_bin must be > 0");
    if (threshold >= num_bin)
      return fail(LGBM_HIP_ERR_RUNTIME, "data_partition: threshold >= num_bin");
    Router r(num_bin, min_bin, max_bin, threshold, mfb, na, default_left);
    const int64_t begin = leaf_begin[leaf], count = leaf_count[leaf];
    uint32_t* idx = indices.data() + begin;
    int64_t lc = 0, rc = 0;
    const int64_t par_min = 65536;  // LGBM_PAR_PARTITION_MIN default
#ifdef _OPENMP
    const int nt = omp_get_max_threads();
#else
    const int nt = 1;
#endif
    if (count >= par_min && nt > 1) {
      const int B = nt;
      std::vector<int64_t> bl(B + 1, 0), br(B + 1, 0);
      const int64_t blk = (count + B - 1) / B;
#pragma omp parallel for schedule(static, 1)
      for (int b = 0; b < B; ++b) {
        int64_t s = b * blk, e = std::min(count, s + blk);
        int64_t l = 0, rr = 0;
        for (int64_t i = s; i < e; ++i) {
          uint32_t row = idx[i];
          bool gr = r.go_right(bins.at(f, row));
          part_left[s + l] = row;
          part_right[s + rr] = row;
          l += gr ? 0 : 1;
          rr += gr ? 1 : 0;
        }
        bl[b + 1] = l;
        br[b + 1] = rr;
      }
      for (int b = 0; b < B; ++b) {
        bl[b + 1] += bl[b];
        br[b + 1] += br[b];
      }
      lc = bl[B];
      rc = br[B];
#pragma omp parallel for schedule(static, 1)
      for (int b = 0; b < B; ++b) {
        int64_t s = b * blk;
        std::memcpy(idx + bl[b], part_left.data() + s, (size_t)(bl[b + 1] - bl[b]) * 4);
        std::memcpy(idx + lc + br[b], part_right.data() + s, (size_t)(br[b + 1] - br[b]) * 4);
      }
    } else {
      for (int64_t i = 0; i < count; ++i) {
        uint32_t row = idx[i];
        bool gr = r.go_right(bins.at(f, row));
        part_right[rc] = row;
        part_left[lc] = row;
        rc += gr ? 1 : 0;
        lc += gr ? 0 : 1;
      }
      std::memcpy(idx, part_left.data(), (size_t)lc * 4);
      std::memcpy(idx + lc, part_right.data(), (size_t)rc * 4);
    }
    leaf_count[leaf] = (int32_t)lc;
    leaf_begin[right_leaf] = (int32_t)(begin + lc);
    leaf_count[right_leaf] = (int32_t)rc;
    return LGBM_HIP_OK;
  }
};

// ---------------------------------------------------------------------------
// LeafSplits (leaf_splits.rs)
// ---------------------------------------------------------------------------
struct LeafSplits {
  int32_t n = 0;
  double sg = 0, sh = 0, weight = 0;
};
double self_output(double sg, double sh, const lgbm_gain_config& c) {  // leaf_splits.rs:113-127
  return calc_leaf_output_full(cfg_use_l1(c), sg, sh, c.lambda_l1, c.lambda_l2, c.max_delta_step,
                               false, c.path_smooth, 0, 0.0);
}

// ---------------------------------------------------------------------------
// SerialTreeLearner spine (learner.rs:980-1562)
// ---------------------------------------------------------------------------
struct Learner {
  Bins bins;
  int F;
  std::vector<lgbm_feature_meta> meta;
  std::vector<uint32_t> num_bin;
  std::vector<size_t> slot_off;
  std::vector<size_t> ub_off;
  const double* ub = nullptr;
  size_t slot_len = 0;
  lgbm_gain_config cfg;
  int32_t num_leaves, max_depth;
  // config.feature_contri: per-feature split-gain multiplier by REAL feature index
  // (learner.rs:456-459, 3701-3709); empty = no multiply.
  std::vector<double> contri;

  // winning categorical bins per leaf (empty: the winner is numerical)
  std::vector<std::vector<uint32_t>> best_cat;
  // the tree's ColSampler selection by feature position (is_feature_used_bytree,
  // learner.rs:1932-1990): unselected features are never scanned; empty = all
  std::vector<char> tree_used;

  bool is_cat(int f) const { return meta[f].bin_type == LGBM_BIN_CATEGORICAL; }
  bool skip_default_bin(int f) const {
    return meta[f].num_bin > 2 && meta[f].missing_type == LGBM_MISSING_ZERO;
  }
  bool na_as_missing(int f) const {
    return meta[f].num_bin > 2 && meta[f].missing_type == LGBM_MISSING_NAN;
  }
  bool run_forward(int f) const {
    return meta[f].num_bin > 2 && meta[f].missing_type != LGBM_MISSING_NONE;
  }

  // scan_leaf_histogram (learner.rs:2708-3355), spine features only.
  void scan_leaf(int32_t leaf, const LeafSplits& ls, const double* buf,
                 const std::vector<char>* parent_split, std::vector<lgbm_split_info>& best,
                 std::vector<int32_t>& best_feat, std::vector<std::vector<char>>& splittable) {
    best_cat[leaf].clear();
    if (!(ls.sh > 0.0) || ls.n <= 0) {
      best[leaf] = split_none();
      best_feat[leaf] = -1;
      return;
    }
    lgbm_gain_config lc = cfg;
    lc.parent_output = ls.weight;
    std::vector<lgbm_split_info> res(F);
    std::vector<std::vector<uint32_t>> cats(F);
    std::vector<char> scanned(F, 0);
#pragma omp parallel for schedule(dynamic, 1) if (F >= 16)
    for (int f = 0; f < F; ++f) {
      if (!tree_used.empty() && !tree_used[f]) continue;
      if (parent_split && !(*parent_split)[f]) continue;
      if (is_cat(f))  // bin_type dispatch (learner.rs:3103-3118): the bumped sum_hessian
        find_best_threshold_categorical(buf + slot_off[f], lc, (int32_t)num_bin[f], meta[f].offset,
                                        ls.sg, ls.sh + 2.0 * kEps, ls.n, &res[f], &cats[f]);
      else
        find_best_split(buf + slot_off[f], 2ull * num_bin[f], lc, num_bin[f], meta[f].offset,
                        meta[f].default_bin, skip_default_bin(f), na_as_missing(f),
                        run_forward(f), ls.sg, ls.sh, ls.n, &res[f]);
      scanned[f] = 1;
    }
    std::vector<char> this_split(F, 0);
    lgbm_split_info lb = split_none();
    int32_t lbf = -1;
    for (int f = 0; f < F; ++f) {
      if (!scanned[f]) continue;
      lgbm_split_info& s = res[f];
      // splittability is recorded from the raw scan result, then feature_contri
      // multiplies the gain before the cross-feature ArgMax (learner.rs:3235-3252)
      this_split[f] = s.gain > kMinScore;
      const int32_t ri = meta[f].real_feature_index;
      if (ri >= 0 && (size_t)ri < contri.size()) s.gain *= contri[(size_t)ri];
      if (s.gain > kMinScore && split_gt(s, meta[f].real_feature_index, lb, lbf)) {
        lb = s;
        lbf = meta[f].real_feature_index;
        best_cat[leaf] = cats[f];
      }
    }
    best[leaf] = lb;
    best_feat[leaf] = lbf;
    splittable[leaf] = this_split;
  }

  // build_leaf_histogram_into (learner.rs:2464-2566)
  void build_leaf(const DataPartition& dp, int32_t leaf, const LeafSplits& ls, const float* g,
                  const float* h, const std::vector<char>* used, double* buf,
                  std::vector<float>& og, std::vector<float>& oh) {
    if (!(ls.sh > 0.0) || ls.n <= 0) {
      std::fill(buf, buf + slot_len, 0.0);
      return;
    }
    const uint32_t* rows = dp.indices.data() + dp.leaf_begin[leaf];
    const int64_t nr = dp.leaf_count[leaf];
    for (int64_t k = 0; k < nr; ++k) {
      og[k] = g[rows[k]];
      oh[k] = h[rows[k]];
    }
    build_histograms_into(bins, num_bin, slot_off, rows, nr, og.data(), oh.data(), used, buf,
                          slot_len);
    for (int f = 0; f < F; ++f) {
      if (used && !(*used)[f]) continue;
      fix_histogram(buf + slot_off[f], num_bin[f], meta[f].most_freq_bin, ls.sg, ls.sh);
      compact_histogram(buf + slot_off[f], num_bin[f], meta[f].offset);
    }
  }

  int train(const float* g, const float* h, Tree& tree, DataPartition& dp) {
    const int64_t N = bins.n;
    // bin-range gate (learner.rs:1161-1187)
    for (int f = 0; f < F; ++f)
      for (int64_t r = 0; r < N; ++r)
        if (bins.at(f, r) >= num_bin[f])
          return fail(LGBM_HIP_ERR_BIN_OUT_OF_RANGE, "bin index out of range");
    if (num_leaves < 1) return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "num_leaves < 1");
    std::vector<std::vector<double>> slot(num_leaves);
    std::vector<float> og(N), oh(N);
    // root LeafSplits::init (leaf_splits.rs:75-89): sequential ordered f64 fold.
    LeafSplits smaller, larger;
    {
      double sg = 0.0, sh = 0.0;
      for (int64_t i = 0; i < N; ++i) {
        sg += (double)g[i];
        sh += (double)h[i];
      }
      smaller.n = (int32_t)N;
      smaller.sg = sg;
      smaller.sh = sh;
      smaller.weight = self_output(sg, sh, cfg);
    }
    if (!(smaller.sh > 0.0)) return fail(LGBM_HIP_ERR_INVALID_LEAF_HESSIAN, "root sum_hessian <= 0");
    tree = Tree::root(smaller.weight, (int32_t)N);
    std::vector<lgbm_split_info> best(num_leaves, split_none());
    std::vector<int32_t> best_feat(num_leaves, -1);
    std::vector<std::vector<char>> splittable(num_leaves, std::vector<char>(F, 1));
    best_cat.assign(num_leaves, {});
    int32_t left_leaf = 0, right_leaf = -1;
    for (int32_t it = 0; it < num_leaves - 1; ++it) {
      // before_find_best_split (learner.rs:1808-1839)
      bool did = true;
      {
        int32_t nl = dp.leaf_count[left_leaf];
        if (max_depth > 0 && tree.leaf_depth[left_leaf] >= max_depth) {
          best[left_leaf].gain = kMinScore;
          if (right_leaf >= 0) best[right_leaf].gain = kMinScore;
          did = false;
        } else {
          int32_t min2 = cfg.min_data_in_leaf * 2;
          if (right_leaf >= 0) {
            int32_t nr = dp.leaf_count[right_leaf];
            if (nr < min2 && nl < min2) {
              best[left_leaf].gain = kMinScore;
              best[right_leaf].gain = kMinScore;
              did = false;
            }
          } else if (nl < min2) {
            best[left_leaf].gain = kMinScore;
            did = false;
          }
        }
      }
      if (did) {
        // find_best_splits (learner.rs:1851-2453)
        int32_t sm, lg;
        if (right_leaf < 0) {
          sm = left_leaf;
          lg = -1;
        } else if (dp.leaf_count[left_leaf] < dp.leaf_count[right_leaf]) {
          sm = left_leaf;
          lg = right_leaf;
        } else {
          sm = right_leaf;
          lg = left_leaf;
        }
        const bool use_subtract = right_leaf >= 0 && !slot[left_leaf].empty();
        std::vector<char> parent_split;
        if (use_subtract) parent_split = splittable[left_leaf];
        std::vector<double> parent;
        if (use_subtract) parent.swap(slot[left_leaf]);
        const LeafSplits& s_ls = smaller;
        const LeafSplits& l_ls = right_leaf < 0 ? smaller : larger;
        std::vector<double> sbuf(slot_len, 0.0);
        build_leaf(dp, sm, s_ls, g, h, use_subtract ? &parent_split : nullptr, sbuf.data(), og, oh);
        std::vector<double> lbuf;
        if (lg >= 0) {
          lbuf.resize(slot_len);
          if (use_subtract) {
            for (size_t i = 0; i < slot_len; ++i) lbuf[i] = parent[i] - sbuf[i];
          } else {
            build_leaf(dp, lg, l_ls, g, h, nullptr, lbuf.data(), og, oh);
          }
        }
        slot[sm].swap(sbuf);
        if (lg >= 0) slot[lg].swap(lbuf);
        const std::vector<char>* ps = use_subtract ? &parent_split : nullptr;
        scan_leaf(sm, s_ls, slot[sm].data(), ps, best, best_feat, splittable);
        if (lg >= 0) scan_leaf(lg, l_ls, slot[lg].data(), ps, best, best_feat, splittable);
      }
      // arg_max (learner.rs:4537)
      int32_t bl = 0;
      for (int32_t i = 1; i < num_leaves; ++i)
        if (split_gt(best[i], best_feat[i], best[bl], best_feat[bl])) bl = i;
      const lgbm_split_info b = best[bl];
      if (b.gain <= 0.0) break;
      // split_inner (learner.rs:3895-4092)
      const int32_t fr = best_feat[bl];
      int f = -1;
      for (int j = 0; j < F; ++j)
        if (meta[j].real_feature_index == fr) {
          f = j;
          break;
        }
      const int32_t new_left = bl, new_right = tree.num_leaves;
      const lgbm_feature_meta& m = meta[f];
      const float gain_field = (float)(b.gain + cfg.min_gain_to_split);
      int32_t pl = 0, pr = 0;
      if (is_cat(f)) {
        // split_inner_categorical (learner.rs:4104-4186): partition by the winning
        // bins, record the bitset over their category values (bin_to_category)
        std::vector<char> left_bin(m.num_bin, 0);
        std::vector<uint32_t> vals;
        for (uint32_t bb : best_cat[bl]) {
          if (bb < m.num_bin) left_bin[bb] = 1;
          const double cv = ub ? ub[ub_off[f] + bb] : (double)bb;
          vals.push_back((uint32_t)(int32_t)cv);
        }
        int rc = dp.split_categorical(bl, new_right, bins, f, left_bin);
        if (rc != LGBM_HIP_OK) return rc;
        pl = dp.leaf_count[new_left];
        pr = dp.leaf_count[new_right];
        tree.split_categorical(bl, fr, construct_bitset(vals), b.left_output, b.right_output, pl,
                               pr, b.left_sum_hessian, b.right_sum_hessian, gain_field,
                               (int8_t)m.missing_type);
      } else {
      const uint32_t pmin = m.min_bin + (uint32_t)std::max(m.offset, 0);
      int rc = dp.split(bl, new_right, bins, f, m.num_bin, pmin, m.max_bin, b.threshold,
                        m.most_freq_bin, na_as_missing(f), b.default_left != 0);
      if (rc != LGBM_HIP_OK) return rc;
      const double thr_real =
          ub ? ub[ub_off[f] + b.threshold] : (double)b.threshold;  // real_threshold (learner.rs:198-203)
      pl = dp.leaf_count[new_left];
      pr = dp.leaf_count[new_right];
      tree.split(bl, fr, b.threshold, thr_real, b.left_output, b.right_output, pl, pr,
                 b.left_sum_hessian, b.right_sum_hessian, gain_field, (int8_t)m.missing_type,
                 b.default_left != 0);
      }
      // Child seeding: the numerical path orders the children by partition counts
      // (learner.rs:4061), the categorical one by the SplitInfo counts
      // (seed_child_leaf_splits, learner.rs:4202); the histogram of the next pass goes
      // to the partition-smaller leaf either way.
      if (is_cat(f) ? b.left_count < b.right_count : pl < pr) {
        smaller = {pl, b.left_sum_gradient, b.left_sum_hessian, b.left_output};
        larger = {pr, b.right_sum_gradient, b.right_sum_hessian, b.right_output};
      } else {
        smaller = {pr, b.right_sum_gradient, b.right_sum_hessian, b.right_output};
        larger = {pl, b.left_sum_gradient, b.left_sum_hessian, b.left_output};
      }
      best[bl] = split_none();
      best_feat[bl] = -1;
      best_cat[bl].clear();
      best[new_left] = split_none();
      best_feat[new_left] = -1;
      best[new_right] = split_none();
      best_feat[new_right] = -1;
      left_leaf = new_left;
      right_leaf = new_right;
    }
    return LGBM_HIP_OK;
  }
};

int make_learner(Learner& L, const void* bins, int width, int32_t F, int64_t N,
                 const lgbm_feature_meta* meta, const double* ub, const lgbm_gain_config* cfg,
                 int32_t num_leaves, int32_t max_depth) {
  if (!bins || !meta || !cfg || F <= 0 || N <= 0)
    return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "null input or empty shape");
  if (width != 1 && width != 2 && width != 4)
    return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "bin width must be 1, 2 or 4");
  L.bins = {bins, width, N};
  L.F = F;
  L.meta.assign(meta, meta + F);
  L.num_bin.resize(F);
  L.slot_off.resize(F);
  L.ub_off.resize(F);
  size_t acc = 0, uacc = 0;
  for (int f = 0; f < F; ++f) {
    L.num_bin[f] = meta[f].num_bin;
    L.slot_off[f] = acc;
    L.ub_off[f] = uacc;
    acc += 2ull * meta[f].num_bin;
    uacc += meta[f].num_bin;
  }
  L.slot_len = acc;
  L.ub = ub;
  L.cfg = *cfg;
  L.num_leaves = num_leaves;
  L.max_depth = max_depth;
  return LGBM_HIP_OK;
}

// BinaryLogloss::get_gradients (lgbm-objective/src/binary.rs:134-172), sigmoid = 1,
// balanced label weights.
void binary_gradients(const double* score, const float* label, float* g, float* h, int64_t n,
                      double sigmoid) {
#pragma omp parallel for schedule(static) if (n > 65536)
  for (int64_t i = 0; i < n; ++i) {
    bool pos = label[i] > 0.0f;
    double lv = pos ? 1.0 : -1.0;
    double resp = -lv * sigmoid / (1.0 + std::exp(lv * sigmoid * score[i]));
    double ar = std::fabs(resp);
    g[i] = (float)(resp * 1.0);
    h[i] = (float)(ar * (sigmoid - ar) * 1.0);
  }
}
// BinaryLogloss::boost_from_score (binary.rs:178-192)
double binary_boost_from_score(const float* label, int64_t n, double sigmoid) {
  if (n == 0) return 0.0;
  double suml = 0.0;
  for (int64_t i = 0; i < n; ++i) suml += label[i] > 0.0f ? 1.0 : 0.0;
  double pavg = suml / (double)n;
  pavg = std::fmin(pavg, 1.0 - kEps);
  pavg = std::fmax(pavg, kEps);
  return std::log(pavg / (1.0 - pavg)) / sigmoid;
}

// MulticlassSoftmax (lgbm-objective/src/multiclass.rs:48-200).  Labels truncate to
// int class ids in [0, K) (:76-101); factor = K / (K - 1) (:84).
struct Multiclass {
  int32_t K = 0;
  double factor = 0.0;
  std::vector<int32_t> label;
  std::vector<double> init_probs;  // class_init_probs (:81-101)
  int init(const float* labels, int64_t n, int32_t k) {
    if (k < 2) return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "multiclass needs num_class >= 2");
    K = k;
    factor = (double)k / ((double)k - 1.0);
    label.resize(n);
    init_probs.assign(k, 0.0);
    for (int64_t i = 0; i < n; ++i) {
      // `l as i32`: truncation toward zero, NaN to 0 (saturating cast)
      const double l = labels[i];
      if (l == l && (l <= -1.0 || l >= (double)k))
        return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "multiclass label out of [0, num_class)");
      const int32_t li = l == l ? (int32_t)l : 0;
      init_probs[li] += 1.0;
      label[i] = li;
    }
    if (n > 0)
      for (double& p : init_probs) p /= (double)n;
    return LGBM_HIP_OK;
  }
  // get_gradients (:138-180) with Common::Softmax (lgbm-model/src/objective.rs:307-322):
  // max by fold from rec[0], exp(v - max), sum in class order, divide.
  void gradients(const double* score, int64_t n, float* g, float* h) const {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; ++i) {
      double rec[256];
      double wmax = score[i];
      for (int32_t k = 1; k < K; ++k) wmax = std::fmax(score[(size_t)k * n + i], wmax);
      double wsum = 0.0;
      for (int32_t k = 0; k < K; ++k) {
        rec[k] = std::exp(score[(size_t)k * n + i] - wmax);
        wsum += rec[k];
      }
      for (int32_t k = 0; k < K; ++k) {
        const double p = rec[k] / wsum;
        const size_t idx = (size_t)k * n + i;
        g[idx] = label[i] == k ? (float)(p - 1.0) : (float)p;
        h[idx] = (float)(factor * p * (1.0 - p));
      }
    }
  }
  // boost_from_score (:184-187): log(max(p, kEpsilon))
  double boost_from_score(int32_t k) const { return std::log(std::fmax(init_probs[k], kEps)); }
  // class_need_train (:193-197)
  bool need_train(int32_t k) const {
    const double p = std::fabs(init_probs[k]);
    return !(p <= kEps || p >= 1.0 - kEps);
  }
};

// ---------------------------------------------------------------------------
// Random (lgbm-core/src/random.rs:37-123): LightGBM's LCG, x = 214013 x + 2531011.
// ---------------------------------------------------------------------------
struct LcgRandom {
  uint32_t x;
  explicit LcgRandom(int32_t seed) : x((uint32_t)seed) {}
  int32_t rand_int16() {
    x = x * 214013u + 2531011u;
    return (int32_t)((x >> 16) & 0x7FFFu);
  }
  int32_t rand_int32() {
    x = x * 214013u + 2531011u;
    return (int32_t)(x & 0x7FFFFFFFu);
  }
  int32_t next_int(int32_t lo, int32_t hi) { return rand_int32() % (hi - lo) + lo; }
  float next_float() { return (float)rand_int16() / 32768.0f; }
  // Sample(N, K) (:87-123): K ordered values of 0..N-1; the streaming branch when
  // K > N / log2(K) (f64), else the ordered-set branch.
  std::vector<int32_t> sample(int32_t n, int32_t k) {
    std::vector<int32_t> ret;
    if (k > n || k <= 0) return ret;
    if (k == n) {
      for (int32_t i = 0; i < n; ++i) ret.push_back(i);
    } else if (k > 1 && (double)k > ((double)n / std::log2((double)k))) {
      for (int32_t i = 0; i < n; ++i) {
        const double prob = (double)(k - (int32_t)ret.size()) / (double)(n - i);
        if ((double)next_float() < prob) ret.push_back(i);
      }
    } else {
      std::vector<char> in(n, 0);
      for (int32_t r = n - k; r < n; ++r) {
        const int32_t v = next_int(0, r + 1);
        if (in[v])
          in[r] = 1;
        else
          in[v] = 1;
      }
      for (int32_t i = 0; i < n; ++i)
        if (in[i]) ret.push_back(i);
    }
    return ret;
  }
};

// ColSampler (lgbm-treelearner/src/col_sampler.rs:68-203), no interaction
// constraints: the Init draw at construction, then reset_by_tree once per tree
// (learner.rs:1190-1225: tree t uses draw t + 2), get_by_node per node.
struct ColSampler {
  double frac_tree = 1.0, frac_node = 1.0;
  LcgRandom rnd{0};
  bool need_reset = false;
  int32_t used_cnt = 0;
  std::vector<int32_t> valid, used_idx;
  std::vector<char> is_used;  // by real feature index
  static int32_t get_cnt(size_t total, double fraction) {  // GetCnt (:80-84)
    const int32_t mn = std::min<int32_t>(1, (int32_t)total);
    const int32_t c = (int32_t)((double)total * fraction + (double)0.5f);
    return std::max(c, mn);
  }
  void init(double ff, double ffn, int32_t seed, std::vector<int32_t> v, size_t nf) {
    frac_tree = ff;
    frac_node = ffn;
    rnd = LcgRandom(seed);
    need_reset = !(ff >= 1.0);
    valid = std::move(v);
    used_cnt = need_reset ? get_cnt(valid.size(), ff) : (int32_t)valid.size();
    is_used.assign(nf, 1);
    reset_by_tree();
  }
  void reset_by_tree() {  // (:119-135)
    if (!need_reset) return;
    std::fill(is_used.begin(), is_used.end(), 0);
    used_idx = rnd.sample((int32_t)valid.size(), used_cnt);
    for (int32_t pos : used_idx) is_used[(size_t)valid[(size_t)pos]] = 1;
  }
  std::vector<char> get_by_node() {  // (:150-185)
    const size_t nf = is_used.size();
    if (frac_node >= 1.0) return std::vector<char>(nf, 1);
    std::vector<char> ret(nf, 0);
    if (need_reset) {
      const int32_t cnt = get_cnt(used_idx.size(), frac_node);
      for (int32_t i : rnd.sample((int32_t)used_idx.size(), cnt))
        ret[(size_t)valid[(size_t)used_idx[(size_t)i]]] = 1;
    } else {
      const int32_t cnt = get_cnt(valid.size(), frac_node);
      for (int32_t i : rnd.sample((int32_t)valid.size(), cnt)) ret[(size_t)valid[(size_t)i]] = 1;
    }
    return ret;
  }
};

// Objective::Regression (L2) get_gradients (lgbm-objective/src/regression.rs:427-431):
// grad = f32(score - f64(label)), hess = 1.
void l2_gradients(const double* score, const float* label, float* g, float* h, int64_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
  for (int64_t i = 0; i < n; ++i) {
    g[i] = (float)(score[i] - (double)label[i]);
    h[i] = 1.0f;
  }
}
// boost_from_score (regression.rs:563-575): the ordered f64 label mean.
double l2_boost_from_score(const float* label, int64_t n) {
  if (n == 0) return 0.0;
  double suml = 0.0;
  for (int64_t i = 0; i < n; ++i) suml += (double)label[i];
  return suml / (double)n;
}

// LambdaRank with NDCG (lgbm-objective/src/rank.rs:100-390) and its DCG tables
// (lgbm-metric/src/dcg_calculator.rs:40-170): default label gain 2^i - 1 (31
// entries), discount 1 / log2(2 + i) for i < 10000, per-query inverse max DCG at
// the truncation level, the 2^20-bin sigmoid table.
struct Lambdarank {
  static constexpr int32_t kMaxPosition = 10000;
  static constexpr int32_t kSigmoidBins = 1024 * 1024;
  double sigmoid = 1.0;
  bool norm = true;
  int32_t trunc = 30;
  std::vector<int32_t> qb;
  std::vector<float> label;
  std::vector<double> gain, discount, inv_max_dcg, table;
  double min_in = 0, max_in = 0, idx_factor = 0;
  int init(const float* labels, int64_t n, const int32_t* bounds, int32_t nq, double sig,
           bool nrm, int32_t truncation) {
    if (!(sig > 0.0)) return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "lambdarank sigmoid must be > 0");
    if (!bounds || nq < 1 || bounds[0] != 0 || bounds[nq] != n)
      return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "query boundaries must run from 0 to num_data");
    for (int32_t q = 0; q < nq; ++q) {
      if (bounds[q + 1] < bounds[q])
        return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "query boundaries must be non-decreasing");
      if (bounds[q + 1] - bounds[q] > kMaxPosition)
        return fail(LGBM_HIP_ERR_CAPABILITY, "a query holds more than 10000 rows");
    }
    sigmoid = sig;
    norm = nrm;
    trunc = truncation;
    qb.assign(bounds, bounds + nq + 1);
    label.assign(labels, labels + n);
    gain.assign(1, 0.0);
    for (int i = 1; i < 31; ++i) gain.push_back((double)((1ll << i) - 1));
    for (int64_t i = 0; i < n; ++i) {  // DCGCalculator::check_labels order
      const float l = labels[i];
      if (std::fabs(l - (float)as_i32(l)) > (float)1e-15f)
        return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "ranking labels must be integers");
      if (l < 0.0f || as_usize(l) >= gain.size())
        return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "ranking label out of the label gain table");
    }
    discount.resize(kMaxPosition);
    for (int32_t i = 0; i < kMaxPosition; ++i) discount[i] = 1.0 / std::log2(2.0 + (double)i);
    inv_max_dcg.resize(nq);
    for (int32_t q = 0; q < nq; ++q) {
      double m = cal_max_dcg_at_k(trunc, labels + bounds[q], bounds[q + 1] - bounds[q]);
      if (m > 0.0) m = 1.0 / m;
      inv_max_dcg[q] = m;
    }
    min_in = -50.0;
    min_in = min_in / sigmoid / 2.0;
    max_in = -min_in;
    idx_factor = (double)kSigmoidBins / (max_in - min_in);
    table.resize(kSigmoidBins);
    for (int32_t i = 0; i < kSigmoidBins; ++i) {
      const double sc = (double)i / idx_factor + min_in;
      table[i] = 1.0 / (1.0 + std::exp(sc * sigmoid));
    }
    return LGBM_HIP_OK;
  }
  // Rust's saturating `l as i32` / `l as usize` (dcg_calculator.rs:118,128; rank.rs:329,
  // 334): NaN -> 0, truncation toward zero, clamped to the type's range.  A NaN label
  // passes check_labels (its comparisons are all false) and indexes gain 0, while the
  // pair loop still compares the f32 labels themselves.
  static int32_t as_i32(float l) {
    if (!(l == l)) return 0;
    if (l <= -2147483648.0f) return INT32_MIN;
    if (l >= 2147483648.0f) return INT32_MAX;
    return (int32_t)l;
  }
  static size_t as_usize(float l) { return l == l && l > 0.0f ? (size_t)as_i32(l) : 0; }
  double cal_max_dcg_at_k(int32_t k, const float* labels, int32_t cnt) const {
    std::vector<int64_t> lc(gain.size(), 0);
    for (int32_t i = 0; i < cnt; ++i) lc[as_usize(labels[i])] += 1;
    int64_t top = (int64_t)gain.size() - 1;
    double ret = 0.0;
    const int32_t kk = std::min(k, cnt);
    for (int32_t j = 0; j < kk; ++j) {
      while (top > 0 && lc[(size_t)top] <= 0) top -= 1;
      if (top < 0) break;
      ret += discount[j] * gain[(size_t)top];
      lc[(size_t)top] -= 1;
    }
    return ret;
  }
  double get_sigmoid(double s) const {
    if (s <= min_in) return table[0];
    if (s >= max_in) return table[kSigmoidBins - 1];
    return table[(size_t)((s - min_in) * idx_factor)];
  }
  // get_gradients -> gradients_for_one_query (rank.rs:260-365)
  void gradients(const double* score, float* g, float* h) const {
    const int32_t nq = (int32_t)qb.size() - 1;
    const double kMin = -std::numeric_limits<double>::infinity();
#pragma omp parallel for schedule(dynamic, 64) if (nq > 256)
    for (int32_t q = 0; q < nq; ++q) {
      const int32_t st = qb[q], cnt = qb[q + 1] - qb[q];
      const double* s = score + st;
      const float* ql = label.data() + st;
      float* lam = g + st;
      float* hes = h + st;
      for (int32_t i = 0; i < cnt; ++i) {
        lam[i] = 0.0f;
        hes[i] = 0.0f;
      }
      if (cnt == 0) continue;
      std::vector<int32_t> si(cnt);
      for (int32_t i = 0; i < cnt; ++i) si[i] = i;
      std::stable_sort(si.begin(), si.end(), [&](int32_t a, int32_t b) { return s[a] > s[b]; });
      const double best = s[si[0]];
      int32_t wi = cnt - 1;
      if (wi > 0 && s[si[wi]] == kMin) wi -= 1;
      const double worst = s[si[wi]];
      const double imd = inv_max_dcg[q];
      double sum_lambdas = 0.0;
      for (int32_t i = 0; i + 1 < cnt && i < trunc; ++i) {
        if (s[si[i]] == kMin) continue;
        for (int32_t j = i + 1; j < cnt; ++j) {
          if (s[si[j]] == kMin) continue;
          if (ql[si[i]] == ql[si[j]]) continue;
          const bool ihigh = ql[si[i]] > ql[si[j]];
          const int32_t hr = ihigh ? i : j, lr = ihigh ? j : i;
          const int32_t hi = si[hr], lo = si[lr];
          const double delta_score = s[hi] - s[lo];
          const double dcg_gap = gain[as_usize(ql[hi])] - gain[as_usize(ql[lo])];
          const double paired = std::fabs(discount[hr] - discount[lr]);
          double dpn = dcg_gap * paired * imd;
          if (norm && best != worst) dpn /= (double)0.01f + std::fabs(delta_score);
          double pl = get_sigmoid(delta_score);
          double ph = pl * (1.0 - pl);
          pl *= -sigmoid * dpn;
          ph *= sigmoid * sigmoid * dpn;
          lam[lo] -= (float)pl;
          hes[lo] += (float)ph;
          lam[hi] += (float)pl;
          hes[hi] += (float)ph;
          sum_lambdas -= 2.0 * pl;
        }
      }
      if (norm && sum_lambdas > 0.0) {
        const double nf = std::log2(1.0 + sum_lambdas) / sum_lambdas;
        for (int32_t i = 0; i < cnt; ++i) {
          lam[i] = (float)((double)lam[i] * nf);
          hes[i] = (float)((double)hes[i] * nf);
        }
      }
    }
  }
};

}  // namespace

// ===========================================================================
// C API (test infrastructure)
// ===========================================================================
extern "C" {

int oracle_last_error(char* buf, size_t size) {
  if (size == 0) return 0;
  std::snprintf(buf, size, "%s", g_err.c_str());
  return 0;
}

int oracle_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
  return omp_get_max_threads();
#else
  (void)n;
  return 1;
#endif
}

// construct_histograms_cpu_native (kernels/histogram.rs:207-233): rows in order.
int oracle_construct_histogram(const uint32_t* bins, const float* g, const float* h, int64_t n,
                               uint32_t num_bin, double* out) {
  for (int64_t i = 0; i < n; ++i)
    if (bins[i] >= num_bin) return fail(LGBM_HIP_ERR_BIN_OUT_OF_RANGE, "bin >= num_bin");
  std::fill(out, out + 2ull * num_bin, 0.0);
  for (int64_t i = 0; i < n; ++i) {
    size_t t = (size_t)bins[i] * 2;
    out[t] += (double)g[i];
    out[t + 1] += (double)h[i];
  }
  return LGBM_HIP_OK;
}

// construct_int_histogram (gradient_discretizer.rs:235-250)
int oracle_construct_int_histogram(const uint32_t* binned, const int8_t* disc,
                                   const uint32_t* rows, int64_t nr, uint32_t num_bin,
                                   int64_t* out) {
  std::fill(out, out + 2ull * num_bin, 0);
  for (int64_t k = 0; k < nr; ++k) {
    uint32_t r = rows[k];
    size_t t = (size_t)binned[r] * 2;
    out[t] += disc[2 * (size_t)r + 1];
    out[t + 1] += disc[2 * (size_t)r];
  }
  return LGBM_HIP_OK;
}

// Discretizer entry: discretize (:104-118) when disc_out != NULL, and the in-place
// dequantize write-back (:126-139).  constant-hessian inference per gbdt.rs:54 when
// const_hess < 0, else forced.
int oracle_quantize(float* g, float* h, int64_t n, int32_t bins, int32_t stochastic,
                    uint64_t seed, int32_t const_hess, int8_t* disc_out, double* scales) {
  if (n == 0) return LGBM_HIP_OK;
  bool ch = const_hess < 0 ? is_constant_hessian(h, n) : const_hess != 0;
  Discretizer d = make_discretizer(bins, ch, stochastic != 0, seed);
  d.compute_scales(g, h, n);
  for (int64_t i = 0; i < n; ++i) {
    int8_t qg, qh;
    d.quantize_pair(g[i], h[i], &qg, &qh);
    if (disc_out) {
      disc_out[2 * i] = qh;
      disc_out[2 * i + 1] = qg;
    }
    g[i] = (float)((double)qg * d.gs);
    h[i] = (float)((double)qh * d.hs);
  }
  if (scales) {
    scales[0] = d.gs;
    scales[1] = d.hs;
  }
  return LGBM_HIP_OK;
}

// xorshift64 stream (gradient_discretizer.rs:255-263) for RNG tests.
int oracle_xorshift_u01(uint64_t state, int64_t n, double* out) {
  Discretizer d;
  d.rng = state;
  for (int64_t i = 0; i < n; ++i) out[i] = d.next_u01();
  return LGBM_HIP_OK;
}

// Raw xorshift64 states (the transition next_u01 applies, gradient_discretizer.rs:
// 255-263): out[i] = the state after i + 1 steps.
int oracle_xorshift_states(uint64_t state, int64_t n, uint64_t* out) {
  Discretizer d;
  d.rng = state;
  for (int64_t i = 0; i < n; ++i) {
    (void)d.next_u01();
    out[i] = d.rng;
  }
  return LGBM_HIP_OK;
}

int oracle_fix_histogram(double* hist, uint32_t num_bin, uint32_t mfb, double sg, double sh) {
  fix_histogram(hist, num_bin, mfb, sg, sh);
  return LGBM_HIP_OK;
}
int oracle_compact_histogram(double* hist, uint32_t num_bin, int32_t offset) {
  compact_histogram(hist, num_bin, offset);
  return LGBM_HIP_OK;
}
int oracle_subtract(const double* parent, const double* child, int64_t n, double* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = parent[i] - child[i];
  return LGBM_HIP_OK;
}

int oracle_find_best_split(const double* hist, int64_t hist_len, const lgbm_gain_config* cfg,
                           uint32_t num_bin, int32_t offset, uint32_t default_bin,
                           int32_t skip_default_bin, int32_t na_as_missing, int32_t run_forward,
                           double sum_gradient, double sum_hessian, int32_t num_data,
                           lgbm_split_info* out) {
  return find_best_split(hist, (size_t)hist_len, *cfg, num_bin, offset, default_bin,
                         skip_default_bin != 0, na_as_missing != 0, run_forward != 0,
                         sum_gradient, sum_hessian, num_data, out);
}

// The per-candidate record of one FindBestThreshold scan (ScanCandidates): rev / fwd
// receive up to cap values each; *n_rev / *n_fwd the number the scan produced.
int oracle_split_candidates(const double* hist, int64_t hist_len, const lgbm_gain_config* cfg,
                            uint32_t num_bin, int32_t offset, uint32_t default_bin,
                            int32_t skip_default_bin, int32_t na_as_missing, int32_t run_forward,
                            double sum_gradient, double sum_hessian, int32_t num_data,
                            double* rev, int32_t* n_rev, double* fwd, int32_t* n_fwd,
                            int32_t cap) {
  lgbm_split_info out;
  ScanCandidates c;
  int rc = find_best_split(hist, (size_t)hist_len, *cfg, num_bin, offset, default_bin,
                           skip_default_bin != 0, na_as_missing != 0, run_forward != 0,
                           sum_gradient, sum_hessian, num_data, &out, &c);
  if (rc) return rc;
  if ((int64_t)c.rev.size() > cap || (int64_t)c.fwd.size() > cap)
    return fail(LGBM_HIP_ERR_LENGTH_MISMATCH, "candidate capacity");
  std::copy(c.rev.begin(), c.rev.end(), rev);
  std::copy(c.fwd.begin(), c.fwd.end(), fwd);
  *n_rev = (int32_t)c.rev.size();
  *n_fwd = (int32_t)c.fwd.size();
  return LGBM_HIP_OK;
}

// The learner router over a row set: stable [left | right] order of local positions.
int oracle_data_partition(const uint32_t* bins, int64_t n, uint32_t num_bin, uint32_t min_bin,
                          uint32_t max_bin, uint32_t threshold, uint32_t mfb,
                          int32_t na_as_missing, int32_t default_left, uint32_t* order,
                          int64_t* left_count) {
  if (num_bin == 0) return fail(LGBM_HIP_ERR_RUNTIME, "data_partition: num_bin must be > 0");
  if (threshold >= num_bin) return fail(LGBM_HIP_ERR_RUNTIME, "threshold >= num_bin");
  for (int64_t i = 0; i < n; ++i)
    if (bins[i] >= num_bin) return fail(LGBM_HIP_ERR_BIN_OUT_OF_RANGE, "bin >= num_bin");
  Router r(num_bin, min_bin, max_bin, threshold, mfb, na_as_missing != 0, default_left != 0);
  int64_t k = 0;
  for (int64_t i = 0; i < n; ++i)
    if (!r.go_right(bins[i])) order[k++] = (uint32_t)i;
  *left_count = k;
  for (int64_t i = 0; i < n; ++i)
    if (r.go_right(bins[i])) order[k++] = (uint32_t)i;
  return LGBM_HIP_OK;
}

// One tree of the SerialTreeLearner spine over feature-major bins of `width` bytes.
// feature_contri (n_contri entries by real feature index) may be NULL.
int oracle_train_tree(const void* bins, int32_t width, int32_t F, int64_t N,
                      const lgbm_feature_meta* meta, const double* ub, const float* g,
                      const float* h, const lgbm_gain_config* cfg, int32_t num_leaves,
                      int32_t max_depth, const double* feature_contri, int32_t n_contri,
                      lgbm_tree_out* tree_out, lgbm_layout_out* layout) {
  Learner L;
  int rc = make_learner(L, bins, width, F, N, meta, ub, cfg, num_leaves, max_depth);
  if (rc) return rc;
  if (feature_contri && n_contri > 0) L.contri.assign(feature_contri, feature_contri + n_contri);
  Tree t;
  DataPartition dp(N, num_leaves);
  rc = L.train(g, h, t, dp);
  if (rc) return rc;
  if (tree_out) t.to_out(tree_out);
  if (layout) {
    if (layout->indices) std::memcpy(layout->indices, dp.indices.data(), (size_t)N * 4);
    for (int i = 0; i < t.num_leaves; ++i) {
      if (layout->leaf_begin) layout->leaf_begin[i] = dp.leaf_begin[i];
      if (layout->leaf_count) layout->leaf_count[i] = dp.leaf_count[i];
    }
  }
  return LGBM_HIP_OK;
}

int oracle_binary_gradients(const double* score, const float* label, float* g, float* h,
                            int64_t n) {
  binary_gradients(score, label, g, h, n, 1.0);
  return LGBM_HIP_OK;
}
double oracle_binary_boost_from_score(const float* label, int64_t n) {
  return binary_boost_from_score(label, n, 1.0);
}

int oracle_multiclass_gradients(const double* score, const float* label, int64_t n,
                                int32_t num_class, float* g, float* h) {
  if (num_class > 256) return fail(LGBM_HIP_ERR_CAPABILITY, "num_class must be <= 256");
  Multiclass M;
  int rc = M.init(label, n, num_class);
  if (rc) return rc;
  M.gradients(score, n, g, h);
  return LGBM_HIP_OK;
}

// The multiclass (softmax) boosting loop (gbdt.rs:691-1373, no bagging): per
// iteration the class-major gradients of all K classes from the current scores,
// optional quantization per class (seed (iter << 20) ^ class ^ 0x51702010,
// gbdt.rs:946-958), then per class: class_need_train gate (a constant tree),
// grow, shrinkage, score update of that class, add_bias(init) on the first
// iteration; a class that does not split gets a constant tree (init on the first
// iteration, else 0).  A round in which no class splits ends training (after the
// first iteration its trees are dropped: gbdt.rs:1330-1349).  `scores` (K * n,
// class-major) receives the final scores; trees_out (optional) holds iters * K trees.
// RenewIntGradTreeOutput through renew_tree_output (learner.rs:4411-4429;
// gbdt.rs:1194-1212): every leaf's output from the ordered f64 fold of the original
// gradients og, oh over its rows in partition order, -ThresholdL1(sum_g, l1) /
// (sum_h + l2), before shrinkage.
void renew_leaf_outputs(Tree& t, const DataPartition& dp, const float* og, const float* oh,
                        const lgbm_gain_config& cfg) {
  if (t.num_leaves <= 1) return;
  for (int32_t leaf = 0; leaf < t.num_leaves; ++leaf) {
    const uint32_t* rows = dp.indices.data() + dp.leaf_begin[leaf];
    const int32_t c = dp.leaf_count[leaf];
    double sg = 0.0, sh = 0.0;
    for (int32_t k = 0; k < c; ++k) {
      sg += (double)og[rows[k]];
      sh += (double)oh[rows[k]];
    }
    t.leaf_value[leaf] = -threshold_l1(sg, cfg.lambda_l1) / (sh + cfg.lambda_l2);
  }
}

int oracle_train_multiclass(const void* bins, int32_t width, int32_t F, int64_t N,
                            const lgbm_feature_meta* meta, const double* ub, const float* label,
                            int32_t num_class, const lgbm_gain_config* cfg, int32_t num_leaves,
                            int32_t max_depth, int32_t iters, double lr,
                            int32_t boost_from_average, int32_t quantized, int32_t quant_bins,
                            int32_t stochastic, double* scores, lgbm_tree_out* trees_out,
                            int32_t* n_trees, int32_t quant_renew_leaf) {
  if (num_class > 256) return fail(LGBM_HIP_ERR_CAPABILITY, "num_class must be <= 256");
  Learner L;
  int rc = make_learner(L, bins, width, F, N, meta, ub, cfg, num_leaves, max_depth);
  if (rc) return rc;
  Multiclass M;
  if ((rc = M.init(label, N, num_class))) return rc;
  const int32_t K = num_class;
  std::vector<double> score((size_t)K * N, 0.0), init(K, 0.0);
  if (boost_from_average)
    for (int32_t k = 0; k < K; ++k) {
      init[k] = M.boost_from_score(k);
      if (std::fabs(init[k]) > kEps)
        for (int64_t i = 0; i < N; ++i) score[(size_t)k * N + i] += init[k];
    }
  std::vector<float> g((size_t)K * N), h((size_t)K * N);
  const bool renew = quantized && quant_renew_leaf;
  std::vector<float> og, oh;  // the original gradients of the iteration (renew)
  int32_t nt = 0;
  for (int32_t it = 0; it < iters; ++it) {
    M.gradients(score.data(), N, g.data(), h.data());
    if (renew) {
      og = g;
      oh = h;
    }
    if (quantized)
      for (int32_t k = 0; k < K; ++k) {
        const uint64_t seed = ((uint64_t)it << 20) ^ (uint64_t)k ^ 0x51702010ull;
        quantize_in_place(g.data() + (size_t)k * N, h.data() + (size_t)k * N, N, quant_bins,
                          stochastic != 0, seed, nullptr, nullptr);
      }
    const int32_t before = nt;
    bool any_split = false;
    for (int32_t k = 0; k < K; ++k) {
      Tree t;
      bool trained = false;
      if (M.need_train(k)) {
        DataPartition dp(N, num_leaves);
        rc = L.train(g.data() + (size_t)k * N, h.data() + (size_t)k * N, t, dp);
        if (rc) return rc;
        if (t.num_leaves > 1) {
          trained = true;
          any_split = true;
          if (renew)
            renew_leaf_outputs(t, dp, og.data() + (size_t)k * N, oh.data() + (size_t)k * N, *cfg);
          t.shrinkage(lr);
          double* sk = score.data() + (size_t)k * N;
          for (int32_t leaf = 0; leaf < t.num_leaves; ++leaf) {
            const double v = t.leaf_value[leaf];
            const uint32_t* rows = dp.indices.data() + dp.leaf_begin[leaf];
            const int32_t c = dp.leaf_count[leaf];
            for (int32_t r = 0; r < c; ++r) sk[rows[r]] += v;
          }
          if (it == 0 && std::fabs(init[k]) > kEps) t.add_bias(init[k]);
        }
      }
      if (!trained) t = Tree::root(it == 0 ? init[k] : 0.0, (int32_t)N);
      if (trees_out) t.to_out(&trees_out[nt]);
      nt++;
    }
    if (!any_split) {
      if (it > 0) nt = before;
      break;
    }
  }
  if (scores) std::memcpy(scores, score.data(), (size_t)K * N * 8);
  if (n_trees) *n_trees = nt;
  return LGBM_HIP_OK;
}

// The binary boosting loop (gbdt.rs:691-1300 for K = 1, no bagging): gradients ->
// optional quantization (seed per gbdt.rs:950) -> grow -> shrinkage -> score update
// through the partition (learner.rs:4380-4395) -> add_bias on the first tree.
// `scores` (n) receives the final training scores; trees_out (optional) is an array of
// `iters` tree descriptors.  Returns the number of trees in *n_trees.
// The boosting loop (gbdt.rs:612-640,691-1300) for one tree per iteration: the
// objective's BoostFromAverage init (added when |init| > kEpsilon; the first tree
// carries it as add_bias), gradients, the optional quantizer, the column sampler's
// per-tree draw, the tree, score updates, and the stop when a tree cannot split.
typedef struct {
  int32_t objective;  // 0 binary logloss, 1 L2 regression, 2 lambdarank
  int32_t num_leaves, max_depth, iters;
  double learning_rate;
  int32_t boost_from_average, quantized, quant_bins, stochastic;
  double feature_fraction;  // < 1: ColSampler by tree (feature_fraction_bynode = 1)
  int32_t feature_fraction_seed, lambdarank_norm;
  double sigmoid;
  int32_t truncation_level, num_queries;
  const int32_t* query_boundaries;  // num_queries + 1 (lambdarank)
  // quant_train_renew_leaf (gbdt.rs:936-943,1194-1212): with quantized gradients, each
  // tree's leaf outputs are recomputed from the original gradients
  int32_t quant_renew_leaf, _pad;
} oracle_train_params;

int oracle_train(const void* bins, int32_t width, int32_t F, int64_t N,
                 const lgbm_feature_meta* meta, const double* ub, const float* label,
                 const lgbm_gain_config* cfg, const oracle_train_params* p, double* scores,
                 lgbm_tree_out* trees_out, int32_t* n_trees) {
  if (!p || !label) return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "null params or labels");
  Learner L;
  int rc = make_learner(L, bins, width, F, N, meta, ub, cfg, p->num_leaves, p->max_depth);
  if (rc) return rc;
  Lambdarank rank;
  if (p->objective == 2) {
    rc = rank.init(label, N, p->query_boundaries, p->num_queries, p->sigmoid,
                   p->lambdarank_norm != 0, p->truncation_level);
    if (rc) return rc;
  } else if (p->objective != 0 && p->objective != 1) {
    return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "objective must be 0, 1 or 2");
  }
  ColSampler cs;
  const bool sampling = p->feature_fraction < 1.0;
  if (sampling) {
    std::vector<int32_t> valid(F);
    int32_t max_real = -1;
    for (int f = 0; f < F; ++f) {
      valid[f] = meta[f].real_feature_index;
      max_real = std::max(max_real, valid[f]);
    }
    cs.init(p->feature_fraction, 1.0, p->feature_fraction_seed, valid,
            (size_t)std::max<int32_t>(max_real + 1, F));
  }
  std::vector<double> score(N, 0.0);
  double init = 0.0;
  if (p->boost_from_average) {
    // ranking objectives have no init score (boosting/src/objective.rs:112-116)
    if (p->objective == 0) init = binary_boost_from_score(label, N, 1.0);
    if (p->objective == 1) init = l2_boost_from_score(label, N);
    if (std::fabs(init) > kEps)
      for (int64_t i = 0; i < N; ++i) score[i] += init;
  }
  std::vector<float> g(N), h(N);
  const bool renew = p->quantized && p->quant_renew_leaf;
  std::vector<float> og, oh;  // the original gradients of the iteration (renew)
  int32_t nt = 0;
  for (int32_t it = 0; it < p->iters; ++it) {
    if (p->objective == 0) binary_gradients(score.data(), label, g.data(), h.data(), N, 1.0);
    if (p->objective == 1) l2_gradients(score.data(), label, g.data(), h.data(), N);
    if (p->objective == 2) rank.gradients(score.data(), g.data(), h.data());
    if (renew) {
      og = g;
      oh = h;
    }
    if (p->quantized) {
      uint64_t seed = ((uint64_t)it << 20) ^ 0ull ^ 0x51702010ull;
      quantize_in_place(g.data(), h.data(), N, p->quant_bins, p->stochastic != 0, seed, nullptr,
                        nullptr);
    }
    if (sampling) {
      cs.reset_by_tree();
      L.tree_used.assign(F, 0);
      for (int f = 0; f < F; ++f) L.tree_used[f] = cs.is_used[(size_t)meta[f].real_feature_index];
    }
    Tree t;
    DataPartition dp(N, p->num_leaves);
    rc = L.train(g.data(), h.data(), t, dp);
    if (rc) return rc;
    if (t.num_leaves <= 1) {
      // No split anywhere this round: GBDT::TrainOneIter keeps the first iteration's
      // constant tree (init score) and stops training (gbdt.rs:981-992, the C++
      // should_continue / pop at gbdt.cpp:440-446).
      if (it == 0) {
        t = Tree::root(init, (int32_t)N);
        if (trees_out) t.to_out(&trees_out[it]);
        nt++;
      }
      break;
    }
    if (renew) renew_leaf_outputs(t, dp, og.data(), oh.data(), *cfg);
    {
      t.shrinkage(p->learning_rate);
      for (int32_t leaf = 0; leaf < t.num_leaves; ++leaf) {
        const double v = t.leaf_value[leaf];
        const uint32_t* rows = dp.indices.data() + dp.leaf_begin[leaf];
        const int32_t c = dp.leaf_count[leaf];
        for (int32_t k = 0; k < c; ++k) score[rows[k]] += v;
      }
      if (it == 0 && std::fabs(init) > kEps) t.add_bias(init);
    }
    if (trees_out) t.to_out(&trees_out[it]);
    nt++;
  }
  if (scores) std::memcpy(scores, score.data(), (size_t)N * 8);
  if (n_trees) *n_trees = nt;
  return LGBM_HIP_OK;
}

int oracle_train_binary(const void* bins, int32_t width, int32_t F, int64_t N,
                        const lgbm_feature_meta* meta, const double* ub, const float* label,
                        const lgbm_gain_config* cfg, int32_t num_leaves, int32_t max_depth,
                        int32_t iters, double lr, int32_t boost_from_average, int32_t quantized,
                        int32_t quant_bins, int32_t stochastic, double* scores,
                        lgbm_tree_out* trees_out, int32_t* n_trees) {
  oracle_train_params p{};
  p.objective = 0;
  p.num_leaves = num_leaves;
  p.max_depth = max_depth;
  p.iters = iters;
  p.learning_rate = lr;
  p.boost_from_average = boost_from_average;
  p.quantized = quantized;
  p.quant_bins = quant_bins;
  p.stochastic = stochastic;
  p.feature_fraction = 1.0;
  return oracle_train(bins, width, F, N, meta, ub, label, cfg, &p, scores, trees_out, n_trees);
}

int oracle_regression_gradients(const double* score, const float* label, int64_t n, float* g,
                                float* h) {
  l2_gradients(score, label, g, h, n);
  return LGBM_HIP_OK;
}
double oracle_regression_boost_from_score(const float* label, int64_t n) {
  return l2_boost_from_score(label, n);
}

int oracle_lambdarank_gradients(const double* score, const float* label, int64_t n,
                                const int32_t* query_boundaries, int32_t num_queries,
                                double sigmoid, int32_t norm, int32_t truncation_level, float* g,
                                float* h) {
  Lambdarank r;
  int rc = r.init(label, n, query_boundaries, num_queries, sigmoid, norm != 0, truncation_level);
  if (rc) return rc;
  r.gradients(score, g, h);
  return LGBM_HIP_OK;
}

// The column sampler's draws as the learner makes them: construction (the Init
// draw), one reset_by_tree, then n_nodes get_by_node calls.  Writes the tree's
// selection (nf flags) and each node's (n_nodes x nf flags).
int oracle_col_sampler_trace(double feature_fraction, double feature_fraction_bynode, int32_t seed,
                             int32_t nf, int32_t n_nodes, int8_t* bytree, int8_t* nodes) {
  if (nf <= 0 || !bytree || (n_nodes > 0 && !nodes))
    return fail(LGBM_HIP_ERR_INVALID_ARGUMENT, "bad trace arguments");
  ColSampler cs;
  std::vector<int32_t> valid(nf);
  for (int32_t f = 0; f < nf; ++f) valid[f] = f;
  cs.init(feature_fraction, feature_fraction_bynode, seed, valid, (size_t)nf);
  cs.reset_by_tree();
  for (int32_t f = 0; f < nf; ++f) bytree[f] = cs.is_used[(size_t)f];
  for (int32_t k = 0; k < n_nodes; ++k) {
    const std::vector<char> m = cs.get_by_node();
    for (int32_t f = 0; f < nf; ++f) nodes[(size_t)k * nf + f] = m[(size_t)f];
  }
  return LGBM_HIP_OK;
}

int oracle_random_sample(int32_t seed, int32_t n, int32_t k, int32_t* out, int32_t* out_len) {
  LcgRandom r(seed);
  const std::vector<int32_t> v = r.sample(n, k);
  for (size_t i = 0; i < v.size(); ++i) out[i] = v[i];
  *out_len = (int32_t)v.size();
  return LGBM_HIP_OK;
}

}  // extern "C"
