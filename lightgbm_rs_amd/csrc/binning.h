// binning.h — feature value -> bin mapping on the host (bin boundaries) and the
// per-feature tables the device binning kernel reads.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

// Missing and bin types as the model text and the learner encode them.
enum : int32_t { BIN_MISSING_NONE = 0, BIN_MISSING_ZERO = 1, BIN_MISSING_NAN = 2 };
enum : int32_t { BIN_NUMERICAL = 0, BIN_CATEGORICAL = 1 };

struct BinParams {
  int32_t max_bin = 255;
  int32_t min_data_in_bin = 3;
  int32_t min_split_data = 0;  // pre-filter threshold (already scaled)
  bool pre_filter = false;
  bool use_missing = true;
  bool zero_as_missing = false;
};

// One feature's mapper (BinMapper, crates/lgbm-dataset/src/bin_mapper.rs:94-135).
struct lgbm_hip_bin_mapper {
  int32_t num_bin = 1;
  int32_t missing_type = BIN_MISSING_NONE;
  int32_t bin_type = BIN_NUMERICAL;
  uint32_t default_bin = 0, most_freq_bin = 0;
  bool is_trivial = true;
  double sparse_rate = 1.0, min_val = 0.0, max_val = 0.0;
  std::vector<double> upper;         // numerical: inclusive upper bound per bin
  std::vector<int32_t> bin_to_cat;   // categorical: bin -> category (-1: the NaN bin 0)
  std::unordered_map<int32_t, uint32_t> cat_to_bin;

  uint32_t value_to_bin(double v) const;
};

// `values`: the sampled column (NaNs allowed), total_sample_cnt >= values.size()
// (the difference is the count of zeros not in `values`).
lgbm_hip_bin_mapper find_bin_numeric(std::vector<double> values, const BinParams& p,
                                     int64_t total_sample_cnt, const std::vector<double>& forced);
lgbm_hip_bin_mapper find_bin_categorical(std::vector<double> values, const BinParams& p,
                                         int64_t total_sample_cnt);
// Random(seed).Sample(n, min(n, sample_cnt)) (crates/lgbm-core/src/random.rs).
std::vector<int32_t> bin_sample_indices(int32_t n, int32_t sample_cnt, int32_t seed);
// `min_data_in_leaf * sample / rows` (bin_mapper.rs:654-683).
int32_t bin_scaled_filter_cnt(int32_t min_data_in_leaf, int32_t total_sample_cnt, int32_t num_rows);
