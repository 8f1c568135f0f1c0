// binning.cpp — bin boundaries of one feature from its sampled values (host side).
//
// The reference's BinMapper construction (crates/lgbm-dataset/src/bin_mapper.rs):
// NaN strip and missing-type choice (:205-230), sorted distinct values with the
// zero pseudo-value and the `b <= nextafter(a, +inf)` de-dup (:236-272), the three
// boundary builders — greedy (:736-835), zero-as-one-bin (:940-1005), forced bounds
// (:838-938) — the bin counts, pre-filter, default / most-frequent bin and sparse
// rate (:300-365), the categorical fold (:409-560) and ValueToBin (:148-189).  The
// steps and their floating-point order are the reference's, since the boundaries
// decide every bin index downstream; the code is this library's own.
#include "binning.h"

#include <algorithm>
#include <cmath>
#include <limits>
#include <set>

namespace {

constexpr double kZero = 1e-35;  // kZeroThreshold (lgbm-core/src/types.rs:35)
constexpr double kInf = std::numeric_limits<double>::infinity();

inline double next_up(double a) { return std::nextafter(a, kInf); }
// CheckDoubleEqualOrdered: b lies within one ulp above a
inline bool within_ulp(double a, double b) { return b <= next_up(a); }

// f64 -> i32 the way the reference's `as i32` does it (saturating, NaN -> 0)
inline int32_t sat_i32(double x) {
  if (!(x == x)) return 0;
  if (x >= 2147483647.0) return std::numeric_limits<int32_t>::max();
  if (x <= -2147483648.0) return std::numeric_limits<int32_t>::min();
  return (int32_t)x;
}

// LightGBM's linear congruential generator (lgbm-core/src/random.rs)
struct Lcg {
  uint32_t x;
  int32_t draw15() {
    x = x * 214013u + 2531011u;
    return (int32_t)((x >> 16) & 0x7FFFu);
  }
  int32_t draw31() {
    x = x * 214013u + 2531011u;
    return (int32_t)(x & 0x7FFFFFFFu);
  }
  float unit() { return (float)draw15() / 32768.0f; }
  int32_t in_range(int32_t lo, int32_t hi) { return draw31() % (hi - lo) + lo; }
};

// Bounds appended only when more than one ulp above the previous one.
struct Bounds {
  std::vector<double> b;
  bool add(double v) {
    if (!b.empty() && within_ulp(b.back(), v)) return false;
    b.push_back(v);
    return true;
  }
};

// GreedyFindBin over the distinct values v[0..nd) with counts c.
std::vector<double> greedy_bounds(const double* v, const int32_t* c, int32_t nd, int32_t max_bin,
                                  int64_t total, int32_t min_data_in_bin) {
  Bounds out;
  if (nd <= max_bin) {
    // few distinct values: a boundary midway between neighbours once a bin holds
    // min_data_in_bin samples
    int32_t in_bin = 0;
    for (int32_t i = 0; i + 1 < nd; ++i) {
      in_bin += c[i];
      if (in_bin >= min_data_in_bin && out.add(next_up((v[i] + v[i + 1]) / 2.0))) in_bin = 0;
    }
    out.b.push_back(kInf);
    return out.b;
  }
  if (min_data_in_bin > 0) max_bin = std::max(1, std::min(max_bin, (int32_t)(total / min_data_in_bin)));
  // values holding at least a mean bin's worth of samples get a bin of their own
  double mean = (double)total / (double)max_bin;
  int32_t bins_left = max_bin, samples_left = (int32_t)total;
  std::vector<char> big((size_t)nd, 0);
  for (int32_t i = 0; i < nd; ++i)
    if ((double)c[i] >= mean) {
      big[(size_t)i] = 1;
      --bins_left;
      samples_left -= c[i];
    }
  mean = (double)samples_left / (double)bins_left;
  std::vector<double> hi((size_t)max_bin + 1, kInf), lo((size_t)max_bin + 1, kInf);
  int32_t nb = 0, in_bin = 0;
  lo[0] = v[0];
  for (int32_t i = 0; i + 1 < nd; ++i) {
    if (!big[(size_t)i]) samples_left -= c[i];
    in_bin += c[i];
    const bool close = big[(size_t)i] || (double)in_bin >= mean ||
                       (big[(size_t)i + 1] && (double)in_bin >= std::max(1.0, mean * 0.5));
    if (!close) continue;
    hi[(size_t)nb] = v[i];
    ++nb;
    lo[(size_t)nb] = v[i + 1];
    if (nb >= max_bin - 1) break;
    in_bin = 0;
    if (!big[(size_t)i]) {
      --bins_left;
      mean = (double)samples_left / (double)bins_left;
    }
  }
  ++nb;
  for (int32_t i = 0; i + 1 < nb; ++i) out.add(next_up((hi[(size_t)i] + lo[(size_t)i + 1]) / 2.0));
  out.b.push_back(kInf);
  return out.b;
}

int32_t first_above(const std::vector<double>& v, int32_t from, double t) {
  for (int32_t i = from; i < (int32_t)v.size(); ++i)
    if (v[(size_t)i] > t) return i;
  return -1;
}

// FindBinWithZeroAsOneBin: negatives, the zero bin (-kZero, kZero], positives.
std::vector<double> zero_bin_bounds(const std::vector<double>& v, const std::vector<int32_t>& c,
                                    int32_t max_bin, int64_t total, int32_t min_data_in_bin) {
  const int32_t nd = (int32_t)v.size();
  int32_t neg = 0, zeros = 0, pos = 0;
  for (int32_t i = 0; i < nd; ++i) {
    if (v[(size_t)i] <= -kZero)
      neg += c[(size_t)i];
    else if (v[(size_t)i] > kZero)
      pos += c[(size_t)i];
    else
      zeros += c[(size_t)i];
  }
  int32_t n_neg = first_above(v, 0, -kZero);
  if (n_neg < 0) n_neg = nd;
  std::vector<double> out;
  if (n_neg > 0 && max_bin > 1) {
    const int32_t neg_bins =
        std::max(1, sat_i32((double)neg / (double)((int32_t)total - zeros) * (double)(max_bin - 1)));
    out = greedy_bounds(v.data(), c.data(), n_neg, neg_bins, neg, min_data_in_bin);
    if (!out.empty()) out.back() = -kZero;
  }
  const int32_t p0 = first_above(v, n_neg, kZero);
  const int32_t pos_bins = max_bin - 1 - (int32_t)out.size();
  if (p0 >= 0 && pos_bins > 0) {
    const std::vector<double> r =
        greedy_bounds(v.data() + p0, c.data() + p0, nd - p0, pos_bins, pos, min_data_in_bin);
    out.push_back(kZero);
    out.insert(out.end(), r.begin(), r.end());
  } else {
    out.push_back(kInf);
  }
  return out;
}

// FindBinWithPredefinedBin: the zero bin, the forced bounds, then greedy bounds
// inside each of those ranges in proportion to its sample count.
std::vector<double> forced_bounds(const std::vector<double>& v, const std::vector<int32_t>& c,
                                  int32_t max_bin, int64_t total, int32_t min_data_in_bin,
                                  const std::vector<double>& forced) {
  const int32_t nd = (int32_t)v.size();
  int32_t n_neg = first_above(v, 0, -kZero);
  if (n_neg < 0) n_neg = nd;
  const int32_t p0 = first_above(v, n_neg, kZero);
  std::vector<double> ub;
  if (max_bin == 2) {
    ub.push_back(n_neg == 0 ? kZero : -kZero);
  } else if (max_bin >= 3) {
    if (n_neg > 0) ub.push_back(-kZero);
    if (p0 >= 0) ub.push_back(kZero);
  }
  ub.push_back(kInf);
  const int32_t room = max_bin - (int32_t)ub.size();
  int32_t taken = 0;
  for (const double f : forced) {
    if (taken >= room) break;
    if (std::fabs(f) > kZero) {
      ub.push_back(f);
      ++taken;
    }
  }
  std::sort(ub.begin(), ub.end());
  const int32_t free_bins = max_bin - (int32_t)ub.size();
  std::vector<double> extra;
  size_t vi = 0;
  const size_t nr = ub.size();
  for (size_t i = 0; i < nr; ++i) {
    int32_t cnt = 0, dcnt = 0;
    const size_t start = vi;
    while (vi < (size_t)nd && v[vi] < ub[i]) {
      cnt += c[vi];
      ++dcnt;
      ++vi;
    }
    const int32_t left = max_bin - (int32_t)ub.size() - (int32_t)extra.size();
    int32_t sub = sat_i32(std::round((double)cnt * (double)free_bins / (double)total));
    sub = std::min(sub, left) + 1;
    if (i == nr - 1) sub = left + 1;
    const std::vector<double> r =
        greedy_bounds(v.data() + start, c.data() + start, dcnt, sub, cnt, min_data_in_bin);
    extra.insert(extra.end(), r.begin(), r.end() - 1);
  }
  ub.insert(ub.end(), extra.begin(), extra.end());
  std::sort(ub.begin(), ub.end());
  return ub;
}

struct Prepared {
  std::vector<double> dv;  // distinct values, ascending, with the zero pseudo-value
  std::vector<int32_t> dc;
  int32_t na = 0;
  int32_t missing = BIN_MISSING_NONE;
};

// NaN strip, missing type, and the distinct values of the sorted sample.
Prepared prepare(std::vector<double>& vals, const BinParams& p, int64_t total) {
  Prepared r;
  const int32_t n_in = (int32_t)vals.size();
  size_t k = 0;
  for (const double x : vals)
    if (!std::isnan(x)) vals[k++] = x;
  if (!p.use_missing) {
    r.missing = BIN_MISSING_NONE;
  } else if (p.zero_as_missing) {
    r.missing = BIN_MISSING_ZERO;
  } else if ((int32_t)k == n_in) {
    r.missing = BIN_MISSING_NONE;
  } else {
    r.na = n_in - (int32_t)k;
    r.missing = BIN_MISSING_NAN;
  }
  vals.resize(k);
  const int32_t zeros = (int32_t)(total - (int64_t)k - r.na);
  std::stable_sort(vals.begin(), vals.end());
  if (k == 0 || (vals[0] > 0.0 && zeros > 0)) {
    r.dv.push_back(0.0);
    r.dc.push_back(zeros);
  }
  if (k > 0) {
    r.dv.push_back(vals[0]);
    r.dc.push_back(1);
  }
  for (size_t i = 1; i < k; ++i) {
    if (within_ulp(vals[i - 1], vals[i])) {
      r.dv.back() = vals[i];  // keep the larger of the merged values
      ++r.dc.back();
      continue;
    }
    if (vals[i - 1] < 0.0 && vals[i] > 0.0) {
      r.dv.push_back(0.0);
      r.dc.push_back(zeros);
    }
    r.dv.push_back(vals[i]);
    r.dc.push_back(1);
  }
  if (k > 0 && vals[k - 1] < 0.0 && zeros > 0) {
    r.dv.push_back(0.0);
    r.dc.push_back(zeros);
  }
  return r;
}

// NeedFilter: no split of the bin counts leaves filter_cnt samples on both sides.
bool need_filter(const std::vector<int32_t>& cnt, int32_t total, int32_t filter, int32_t bin_type) {
  if (bin_type == BIN_NUMERICAL) {
    int32_t left = 0;
    for (size_t i = 0; i + 1 < cnt.size(); ++i) {
      left += cnt[i];
      if (left >= filter && total - left >= filter) return false;
    }
    return true;
  }
  if (cnt.size() <= 2) {
    for (size_t i = 0; i + 1 < cnt.size(); ++i)
      if (cnt[i] >= filter && total - cnt[i] >= filter) return false;
    return true;
  }
  return false;
}

// trivial flag, default bin, most frequent bin and sparse rate from the bin counts
void finish(lgbm_hip_bin_mapper* m, const std::vector<int32_t>& cnt, const BinParams& p,
            int64_t total) {
  m->is_trivial = m->num_bin <= 1 ||
                  (p.pre_filter && need_filter(cnt, (int32_t)total, p.min_split_data, m->bin_type));
  if (m->is_trivial) {
    m->sparse_rate = 1.0;
    return;
  }
  m->default_bin = m->value_to_bin(0.0);
  uint32_t best = 0;
  for (size_t i = 1; i < cnt.size(); ++i)
    if (cnt[i] > cnt[best]) best = (uint32_t)i;
  if (best != m->default_bin && (double)cnt[best] / (double)total < 0.7) best = m->default_bin;
  m->most_freq_bin = best;
  m->sparse_rate = (double)cnt[best] / (double)total;
}

}  // namespace

uint32_t lgbm_hip_bin_mapper::value_to_bin(double v) const {
  if (std::isnan(v)) {
    if (bin_type == BIN_CATEGORICAL) return 0;
    if (missing_type == BIN_MISSING_NAN) return (uint32_t)(num_bin - 1);
    v = 0.0;
  }
  if (bin_type == BIN_NUMERICAL) {
    // first bin whose upper bound is >= v (the NaN bin excluded)
    int32_t l = 0, r = num_bin - 1 - (missing_type == BIN_MISSING_NAN ? 1 : 0);
    while (l < r) {
      const int32_t m = (r + l - 1) / 2;
      if (v <= upper[(size_t)m])
        r = m;
      else
        l = m + 1;
    }
    return (uint32_t)l;
  }
  const int32_t iv = sat_i32(v);
  if (iv < 0) return 0;
  const auto it = cat_to_bin.find(iv);
  return it == cat_to_bin.end() ? 0u : it->second;
}

lgbm_hip_bin_mapper find_bin_numeric(std::vector<double> vals, const BinParams& p,
                                     int64_t total, const std::vector<double>& forced) {
  lgbm_hip_bin_mapper m;
  Prepared d = prepare(vals, p, total);
  m.bin_type = BIN_NUMERICAL;
  m.missing_type = d.missing;
  m.min_val = d.dv.empty() ? 0.0 : d.dv.front();
  m.max_val = d.dv.empty() ? 0.0 : d.dv.back();
  auto bounds = [&](int32_t max_bin, int64_t cnt) {
    return forced.empty() ? zero_bin_bounds(d.dv, d.dc, max_bin, cnt, p.min_data_in_bin)
                          : forced_bounds(d.dv, d.dc, max_bin, cnt, p.min_data_in_bin, forced);
  };
  if (d.missing == BIN_MISSING_NAN) {
    m.upper = bounds(p.max_bin - 1, total - d.na);
    m.upper.push_back(std::numeric_limits<double>::quiet_NaN());
  } else {
    m.upper = bounds(p.max_bin, total);
    if (d.missing == BIN_MISSING_ZERO && m.upper.size() == 2) m.missing_type = BIN_MISSING_NONE;
  }
  m.num_bin = (int32_t)m.upper.size();
  std::vector<int32_t> cnt((size_t)m.num_bin, 0);
  size_t b = 0;
  for (size_t i = 0; i < d.dv.size(); ++i) {
    while (d.dv[i] > m.upper[b] && b + 1 < (size_t)m.num_bin) ++b;
    cnt[b] += d.dc[i];
  }
  if (m.missing_type == BIN_MISSING_NAN) cnt[(size_t)m.num_bin - 1] = d.na;
  finish(&m, cnt, p, total);
  return m;
}

lgbm_hip_bin_mapper find_bin_categorical(std::vector<double> vals, const BinParams& p,
                                         int64_t total) {
  lgbm_hip_bin_mapper m;
  Prepared d = prepare(vals, p, total);
  m.bin_type = BIN_CATEGORICAL;
  m.missing_type = d.missing;
  m.min_val = d.dv.empty() ? 0.0 : d.dv.front();
  m.max_val = d.dv.empty() ? 0.0 : d.dv.back();
  // integer categories (negatives count as missing), adjacent equal ints merged
  std::vector<std::pair<int32_t, int32_t>> cats;  // (count, category)
  int32_t na = d.na;
  for (size_t i = 0; i < d.dv.size(); ++i) {
    const int32_t iv = sat_i32(d.dv[i]);
    if (iv < 0)
      na += d.dc[i];
    else if (cats.empty() || cats.back().second != iv)
      cats.push_back({d.dc[i], iv});
    else
      cats.back().first += d.dc[i];
  }
  std::vector<int32_t> cnt;
  m.num_bin = 1;
  const int32_t rest = (int32_t)(total - na);
  if (rest > 0) {
    std::stable_sort(cats.begin(), cats.end(),
                     [](const std::pair<int32_t, int32_t>& a, const std::pair<int32_t, int32_t>& b) {
                       return a.first > b.first;
                     });
    // the most frequent categories up to 99% of the samples (float arithmetic)
    const float scaled = (float)rest * 0.99f;
    const int32_t cut = (int32_t)((double)scaled + 0.5);
    const int32_t max_bin = std::min(p.max_bin, (int32_t)cats.size() + (na > 0 ? 1 : 0));
    m.bin_to_cat.push_back(-1);  // bin 0: NaN and unseen categories
    m.cat_to_bin[-1] = 0;
    cnt.push_back(0);
    int32_t used = 0;
    size_t i = 0;
    while (i < cats.size() && (used < cut || m.num_bin < max_bin)) {
      if (cats[i].first < p.min_data_in_bin && i > 1) break;
      m.bin_to_cat.push_back(cats[i].second);
      m.cat_to_bin[cats[i].second] = (uint32_t)m.num_bin;
      used += cats[i].first;
      cnt.push_back(cats[i].first);
      ++m.num_bin;
      ++i;
    }
    m.missing_type = (i == cats.size() && na == 0) ? BIN_MISSING_NONE : BIN_MISSING_NAN;
    cnt[0] = (int32_t)(total - used);
  }
  finish(&m, cnt, p, total);
  return m;
}

std::vector<int32_t> bin_sample_indices(int32_t n, int32_t sample_cnt, int32_t seed) {
  const int32_t k = n < sample_cnt ? n : sample_cnt;
  std::vector<int32_t> out;
  if (k > n || k <= 0) return out;
  if (k == n) {
    out.resize((size_t)n);
    for (int32_t i = 0; i < n; ++i) out[(size_t)i] = i;
    return out;
  }
  Lcg g{(uint32_t)seed};
  if (k > 1 && (double)k > (double)n / std::log2((double)k)) {
    // dense: one Bernoulli draw per row
    for (int32_t i = 0; i < n; ++i) {
      const double prob = (double)(k - (int32_t)out.size()) / (double)(n - i);
      if ((double)g.unit() < prob) out.push_back(i);
    }
  } else {
    // sparse: Floyd's algorithm over an ordered set
    std::set<int32_t> s;
    for (int32_t r = n - k; r < n; ++r) {
      const int32_t v = g.in_range(0, r + 1);
      if (!s.insert(v).second) s.insert(r);
    }
    out.assign(s.begin(), s.end());
  }
  return out;
}

int32_t bin_scaled_filter_cnt(int32_t min_data_in_leaf, int32_t total_sample_cnt, int32_t num_rows) {
  if (num_rows == 0) return min_data_in_leaf;
  return (int32_t)((int64_t)min_data_in_leaf * total_sample_cnt / num_rows);
}
