// lgbm_device.h — device-side structures and arithmetic shared by the gfx950 kernels.
//
// The f64 arithmetic here restates the reference's CPU path operation for operation
// (no contraction: the library is compiled with -ffp-contract=off; the only fused
// multiply-add is the explicit one of GetLeafGainGivenOutput, gain.rs:204-220).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lgbm_hip.h"

#define LGBM_WAVE 64
#define LGBM_MAX_W 8                    // record words (16 B): features <= 16*W - 4
#define HIST_THREADS 512                // ConstructHistogram block
#define HIST_WAVES (HIST_THREADS / LGBM_WAVE)
#define HIST_GRID 256                   // f32 builds: chunks over all jobs of a launch (at most)
#define HIST_GRID_Q 512                 // quantized builds: two 512-thread blocks per CU
#define HIST_SLOTS (HIST_GRID_Q + SPEC_MAX)  // partial slots >= blocks launched
#define HIST_MIN_ROWS 4096              // rows per chunk (at least)
#define HIST_WAVE_CELLS 1792            // wave-private scheme: 28 cells per lane
#define HIST_FOLD_STEPS 7               // 7 x 64 rows <= 511 per 11-bit field
#ifndef HIST_ROWS_PER_LANE
#define HIST_ROWS_PER_LANE 1            // rows per lane in flight per step (1: 114 us root
                                        // build, 2: 117, 3: 138, 4: 156; 16 waves a CU
                                        // hide the loads, fewer folds pay)
#endif
#define HIST_BLOCK_MAX_ROWS ((1 << 19) - 1)  // block-shared scheme field limit
#define HIST_FP_CELLS 3584              // f32 gradients: cells per feature group (16 B each)
#define MAX_FGROUPS 32
// wide layout (REC_FMT_WIDE): ConstructHistogram per (row chunk, feature group); a
// group is WIDE_GF_Q (quantized, 8-byte LDS cells) or WIDE_GF_F (f32, two 8-byte
// cells) consecutive features, at most 256 bins each: 128 KiB of LDS either way
#ifndef WIDE_GF_Q
#define WIDE_GF_Q 64
#endif
#ifndef WIDE_GF_F
#define WIDE_GF_F 32
#endif
#ifndef WIDE_THREADS
#define WIDE_THREADS 1024
#endif
// row-chunk blocks over all groups (at least), per gradient mode: more chunks spread
// the large builds over more blocks, fewer leave the scans fewer partial slots to sum
#ifndef WIDE_GRID_Q
#define WIDE_GRID_Q 512                 // quantized: 64-feature groups, 8-byte cells
#endif
#ifndef WIDE_GRID_F
#define WIDE_GRID_F 1024                // f32: 32-feature groups, 16-byte cells
#endif
#ifndef WIDE_MIN_ROWS
#define WIDE_MIN_ROWS 4096              // rows per chunk (at least): a flush costs a group
#endif
#ifndef WIDE_MIN_ROWS_SMALL_Q
#define WIDE_MIN_ROWS_SMALL_Q 2048      // ... and in rounds too small to fill the chip
#endif                                  //     (quantized; f32 keeps WIDE_MIN_ROWS)
#ifndef WIDE_MIN_ROWS_SMALL_F
#define WIDE_MIN_ROWS_SMALL_F 4096
#endif
#ifndef WIDE_FILL
#define WIDE_FILL 256                   // blocks a small round aims at
#endif
#define WIDE_MAX_ROWS ((1 << 19) - 1)   // packed LDS cell field limit (quantized)
#define WIDE_MAX_F 4096
#define WIDE_MAX_BIN 4096               // 2-byte bins (a feature of more than 256 bins)
#define WIDE16_GROUP_CELLS 8192         // 2-byte bins: cells of a feature group (LDS)
#define WIDE16_GROUP_F 64               // 2-byte bins: features of a group (at most)
#ifndef PART_THREADS
#define PART_THREADS 512                // partition block (two per CU)
#endif
#ifndef PART_ROWS_PER_THREAD
#define PART_ROWS_PER_THREAD 4          // records of <= 32 B; fewer for wider records
#endif
#ifndef PART_BLOCKS_PER_CU
#define PART_BLOCKS_PER_CU 2
#endif
#define PART_WAVES (PART_THREADS / LGBM_WAVE)
#define PART_SLOT_MAX 8                 // blocks per job whose cells go to per-block slots
#define PACKED_ACC_MAX_ROWS ((1 << 19) - 1)  // jobs whose accumulator takes packed 64-bit adds
#define QUANT_MAX_ROWS (1ll << 29)      // int32 cells: sum of q_h <= 4 N < 2^31
#define QUANT_LDS_CELLS 8192            // quantized builds: every cell in LDS (8 B, 64 KiB)
#define PART_MIN_TILE 1024                // smallest tile of any partition launch shape
#define SCAN_THREADS 128                // two waves: smaller leaf, larger leaf
#define PLAN_THREADS 1024
#define MAX_LEAVES 256                  // tree leaves per context (u8 leaf ids in the plan)
#define SLOT_CAP(leaves) (6 * (leaves) + 4)  // node slots: root + two per (speculated) split
#define QUANT_ROWS_PER_LANE 8          // consecutive rows per lane (power of 2)
#define QUANT_WAVE_MATS 27              // wave index bits (N <= 2^27 * 64 * C)
#define STAT_BLOCKS 1024                // partial-statistics blocks of the g/h reduction

// Buffer ids of the row stores.
#define BUF_ORIG 0
#define BUF_A 1
#define BUF_B 2
#define BUF_S0 3   // scratch (per-op entry points)
#define BUF_S1 4
#define NBUF 5

// ctl->error bits
#define ERR_ROOT_HESSIAN 2
#define ERR_FEATURE 4
#define ERR_SLOTS 8
#define ERR_NEG_HESSIAN 16  // quantized histograms: a hessian below zero

// Row record formats, one code per resident layout (`fmt`):
//   1..8   (W): W 16-byte words = 4W u32; four 8-bit bins per u32 (features 0..F-1 in
//          order), the row's original index in the last u32;
//   16 + U (U even, 2..8): U u32 = 4U bytes; five 6-bit bins per u32 (bits 0-29;
//          every num_bin <= 64), the quantized pair in bits 24-29 of the last u32
//          (which holds at most four bins: F <= 5U - 1); no row index.
//   32     (wide): the record is the row's original index (one u32); the bins stay
//          in a row-major matrix binmat[N][Fp] (u8, Fp = F rounded up to WIDE_GF_Q)
//          that is never moved.  For many features, where moving every bin at every
//          split would cost 2 F bytes per row.
#define REC_FMT_PACKED 16
#define REC_FMT_WIDE 32
__host__ __device__ constexpr bool rec_wide(int fmt) { return fmt == REC_FMT_WIDE; }
__host__ __device__ constexpr bool rec_packed(int fmt) {
  return fmt > REC_FMT_PACKED && fmt < REC_FMT_WIDE;
}
__host__ __device__ constexpr int rec_words(int fmt) {  // u32 per record
  return rec_wide(fmt) ? 1 : rec_packed(fmt) ? fmt - REC_FMT_PACKED : 4 * fmt;
}
__host__ __device__ constexpr int rec_bytes(int fmt) { return 4 * rec_words(fmt); }
__host__ __device__ constexpr int rec_bpw(int fmt) { return rec_packed(fmt) ? 5 : 4; }
__host__ __device__ constexpr int rec_bits(int fmt) { return rec_packed(fmt) ? 6 : 8; }
// bin slots of a record (the histogram's cell-base table covers them all; slots past
// the last feature read zero bins into a trash cell): legacy 4 per u32 but none in
// the row-index u32; packed 5 per u32 but 4 in the last (its top bits hold the pair)
__host__ __device__ constexpr int rec_slots(int fmt) {
  return rec_wide(fmt) ? 0 : rec_packed(fmt) ? 5 * rec_words(fmt) - 1 : 4 * (rec_words(fmt) - 1);
}
// word and bit offset of feature f's bin in a record
__host__ __device__ inline void rec_field_pos(int fmt, int f, int* wi, int* sh) {
  const int bpw = rec_bpw(fmt);
  *wi = f / bpw;
  *sh = (f - *wi * bpw) * rec_bits(fmt);
}
// packed quantized pair <-> the u16 form (q_g as u8) | (q_h as u8) << 8 used elsewhere:
// 6 bits (q_g + 2) | q_h << 3 for q_g in [-2, 2], q_h in [0, 4]
__host__ __device__ inline uint32_t gh_pack6(uint32_t q16) {
  const int32_t qg = (int32_t)(int8_t)(q16 & 0xffu);
  const uint32_t qh = (q16 >> 8) & 0xffu;
  return (uint32_t)(qg + 2) | (qh << 3);
}
__host__ __device__ inline uint32_t gh_unpack6(uint32_t e) {
  const int32_t qg = (int32_t)(e & 7u) - 2;
  return (uint32_t)(uint8_t)(int8_t)qg | ((e >> 3) << 8);
}

// Partition rows per thread: two tiles of records stay in registers (the next tile's
// loads overlap this tile's work) within 128 VGPRs.
__host__ __device__ constexpr int part_rows(int fmt) {
  return rec_bytes(fmt) <= 32 ? PART_ROWS_PER_THREAD : (rec_bytes(fmt) <= 64 ? 2 : 1);
}
__host__ __device__ constexpr int64_t part_tile(int fmt) {
  return (int64_t)PART_THREADS * part_rows(fmt);
}
// Block b of a G-block partition launch over T tiles takes tiles [b*T/G, (b+1)*T/G);
// the block that takes tile t:
__host__ __device__ inline int64_t part_owner(int64_t t, int64_t T, int64_t G) {
  return ((t + 1) * G - 1) / T;
}
// Blocks holding at least one of the tiles [t0, t0 + n) (n >= 1): one per tile when
// there are fewer tiles than blocks, else every block from the first owner to the
// last.
__host__ __device__ inline int64_t part_span_blocks(int64_t t0, int64_t n, int64_t T, int64_t G) {
  return T < G ? n : part_owner(t0 + n - 1, T, G) - part_owner(t0, T, G) + 1;
}

struct DevFeature {
  uint32_t num_bin;
  int32_t offset;
  uint32_t min_bin;
  uint32_t max_bin;
  uint32_t default_bin;
  uint32_t mfb;
  int32_t missing_type;
  int32_t real_index;
  uint32_t slot_off;   // first f64 cell of the feature in a leaf slot
  uint32_t cell_base;  // first bin cell in the integer histogram (= slot_off / 2)
  uint32_t ub_off;     // first bin_upper_bound entry
  int32_t skip_default_bin;
  int32_t na_as_missing;
  int32_t run_forward;
  double penalty;      // config.feature_contri of the feature's real index (1: none)
  int32_t categorical; // 1: split by category sets (FindBestThresholdCategorical)
  int32_t _pad2;
};

struct LeafSums {
  double sg, sh, weight;
  int32_t n;
  int32_t _pad;
};

// Node routing parameters recorded at split time (the SplitInner router inputs,
// data_partition.rs:387-417), used by the score-update traversal.
struct NodeRoute {
  int32_t f;          // feature position (record byte)
  int32_t pmin;       // min_bin + offset
  int32_t max_bin;
  int32_t th;         // threshold + pmin (- 1 if mfb == 0)
  int32_t na_bin;     // num_bin - 1
  int32_t flags;      // 1: default_to_right, 2: na_as_missing, 4: default_left,
                      // ROUTE_CAT: categorical (the bins going left are a bit set)
  int32_t left, right;
};
#define ROUTE_CAT 8

// One leaf split of a partition round.  The tree driver splits up to SPEC_MAX
// leaves per round (the best-ranked leaves not yet split; each is committed to
// the tree later in the reference's own ArgMax order), the per-op entry point
// exactly one.  parent/cl/cr are node slots (-1 in per-op mode).
struct PartJob {
  int32_t parent, cl, cr;
  int32_t src_buf, dst_buf, rev;  // rev: source range stored reversed
  int64_t begin, count;
  int32_t fbyte, pmin, max_bin, th, na_bin, flags;  // router
  int32_t acc_right;  // histogram side built in the pass: 0 left, 1 right, -1 none
  int32_t ntiles;
  int64_t tile0;      // first tile of the job in the round's tile space
  uint32_t cat[8];    // flags & ROUTE_CAT: bins going left (bit b of word w: bin 32w + b)
};

#define SPEC_MAX 32        // partition jobs per round
#define SPEC_DEFAULT 8
#define SPEC_SCAN_HEAVY 4  // speculation width where one job's scans are costly (PLAN_CAP_WORK)

// A histogram job: a physical row range of one row buffer.  nblk partial slots from
// a0 hold its histogram after k_hist_jobs.
struct HistJob {
  int32_t buf, _pad;
  int64_t begin, count;
  int32_t a0, nblk;
};

struct Ctl {
  // ---- quantizer (per iteration) ----
  double gs, hs, igs, ihs;
  float vg1, vh1, vh3;
  float hmin;                        // smallest hessian of the iteration
  int32_t quant_bins;
  int32_t const_hess;
  // ---- tree state ----
  int32_t done, error, num_leaves, max_leaves;
  int32_t max_depth, n_slots, slot_cap, spec_max;
  int32_t n_jobs, n_reduce, rounds, root_skip;
  int32_t fp_mode;                   // 1: f32 gradients (64-bit fixed-point histograms)
  int32_t g_shift, h_shift;          // fixed-point exponents: cell = sum * 2^-shift
  int32_t _i4;
  int64_t tile_total;
  // ---- histogram jobs of the current launch ----
  int32_t n_hjobs, _i1;
  HistJob hjobs[SPEC_MAX];
  LeafSums sm;                       // per-op build: the leaf's raw sums
  // ---- partition round ----
  int32_t part_left_count, _i6;
  unsigned long long part_cur[SPEC_MAX];  // per job: (left rows, right rows) reserved
  int32_t acc_used[SPEC_MAX];        // per job: a partition flush used its accumulator
  PartJob jobs[SPEC_MAX];
  int32_t reduce_list[2 * SPEC_MAX + 2];
  // ---- gain config ----
  lgbm_gain_config cfg;
};

// ---------------------------------------------------------------------------
// arithmetic helpers (restating crates/lgbm-compute/src/gain.rs)
// ---------------------------------------------------------------------------
__device__ __forceinline__ double k_eps() { return (double)1e-15f; }

__device__ __forceinline__ int32_t sat_i32(double x) {
  if (x != x) return 0;
  if (x >= 2147483647.0) return 2147483647;
  if (x <= -2147483648.0) return (int32_t)(-2147483647 - 1);
  return (int32_t)x;
}
__device__ __forceinline__ int8_t sat_i8(double x) {
  if (x != x) return 0;
  if (x >= 127.0) return 127;
  if (x <= -128.0) return -128;
  return (int8_t)(int32_t)x;
}
__device__ __forceinline__ int32_t round_int(double x) { return sat_i32(x + (double)0.5f); }

__device__ __forceinline__ double threshold_l1(double s, double l1) {
  double reg = fmax(0.0, fabs(s) - l1);
  double pos = s > 0.0 ? 1.0 : 0.0;
  double neg = s < 0.0 ? 1.0 : 0.0;
  return (pos - neg) * reg;
}
__device__ __forceinline__ double leaf_gain(bool use_l1, double g, double h, double l1, double l2) {
  if (use_l1) {
    double s = threshold_l1(g, l1);
    return (s * s) / (h + l2);
  }
  return (g * g) / (h + l2);
}
__device__ __forceinline__ double leaf_output(bool use_l1, double g, double h, double l1, double l2) {
  if (use_l1) return -threshold_l1(g, l1) / (h + l2);
  return -g / (h + l2);
}
__device__ __forceinline__ double leaf_output_full(bool use_l1, double g, double h, double l1,
                                                   double l2, double mds, bool sm, double ps,
                                                   int32_t n, double po) {
  double base = leaf_output(use_l1, g, h, l1, l2);
  bool clamp = mds > 0.0 && fabs(base) > mds;
  double pos = base > 0.0 ? 1.0 : 0.0;
  double neg = base < 0.0 ? 1.0 : 0.0;
  double c = clamp ? (pos - neg) * mds : base;
  if (sm) {
    double nps = (double)n / ps;
    return c * nps / (nps + 1.0) + po / (nps + 1.0);
  }
  return c;
}
__device__ __forceinline__ double leaf_gain_full(bool use_l1, double g, double h, double l1,
                                                 double l2, double mds, bool sm, double ps,
                                                 int32_t n, double po) {
  if (mds > 0.0 || sm) {
    double out = leaf_output_full(use_l1, g, h, l1, l2, mds, sm, ps, n, po);
    double gg = use_l1 ? threshold_l1(g, l1) : g;
    return -__builtin_fma(2.0 * gg, out, (h + l2) * out * out);
  }
  return leaf_gain(use_l1, g, h, l1, l2);
}

struct ScanCfg {
  bool use_l1, use_smoothing, use_full;
  double l1, l2, mds, ps, min_h, min_gain;
  int32_t min_d;
};

__device__ __forceinline__ ScanCfg make_scan_cfg(const lgbm_gain_config& c) {
  ScanCfg s;
  s.use_l1 = c.lambda_l1 > 0.0;
  s.use_smoothing = c.path_smooth > k_eps();
  s.use_full = s.use_smoothing || c.max_delta_step > 0.0;
  s.l1 = c.lambda_l1;
  s.l2 = c.lambda_l2;
  s.mds = c.max_delta_step;
  s.ps = c.path_smooth;
  s.min_h = c.min_sum_hessian_in_leaf;
  s.min_gain = c.min_gain_to_split;
  s.min_d = c.min_data_in_leaf;
  return s;
}

__device__ __forceinline__ double split_gain_of(const ScanCfg& c, double lg, double lh, double rg,
                                                double rh, int32_t lc, int32_t rc, double po) {
  if (c.use_full)
    return leaf_gain_full(c.use_l1, lg, lh, c.l1, c.l2, c.mds, c.use_smoothing, c.ps, lc, po) +
           leaf_gain_full(c.use_l1, rg, rh, c.l1, c.l2, c.mds, c.use_smoothing, c.ps, rc, po);
  return leaf_gain(c.use_l1, lg, lh, c.l1, c.l2) + leaf_gain(c.use_l1, rg, rh, c.l1, c.l2);
}

__device__ __forceinline__ void split_set_none(lgbm_split_info* s) {
  s->threshold = 0;
  s->left_count = 0;
  s->right_count = 0;
  s->default_left = 1;
  s->gain = -__builtin_inf();
  s->left_sum_gradient = 0.0;
  s->left_sum_hessian = 0.0;
  s->right_sum_gradient = 0.0;
  s->right_sum_hessian = 0.0;
  s->left_output = 0.0;
  s->right_output = 0.0;
}

// split_gt (crates/lgbm-treelearner/src/split_info.rs:28-35)
__device__ __forceinline__ bool split_gt(double ag, int32_t af, double bg, int32_t bf) {
  if (ag != bg) return ag > bg;
  int32_t x = af == -1 ? 0x7fffffff : af;
  int32_t y = bf == -1 ? 0x7fffffff : bf;
  return x < y;
}

__device__ __forceinline__ double maybe_round_to_zero(double v) {
  const double z = (double)1e-35f;
  return (v >= -z && v <= z) ? 0.0 : v;
}

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & (LGBM_WAVE - 1); }

// Broadcast lane `lane` (wave-uniform) of a register to the whole wave.
__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ int32_t readlane_i32(int32_t v, int lane) {
  return __builtin_amdgcn_readlane(v, lane);
}

// A DPP move of an f64 register (GFX9 data-parallel primitives, both halves moved
// alike); lanes outside ROW_MASK, or whose source lane is invalid, keep their own value.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const int lo = (int)(uint32_t)b, hi = (int)(uint32_t)(b >> 32);
  const uint32_t nlo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROW_MASK, 0xf, false);
  const uint32_t nhi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROW_MASK, 0xf, false);
  return __longlong_as_double((long long)(((unsigned long long)nhi << 32) | nlo));
}

// Inclusive prefix sum of an int32 over the wave's lanes (lane k: lanes 0..k):
// row_shr 1, 2, 4, 8 within each 16-lane row (invalid sources add 0), then the row
// broadcasts 15 and 31 carry the earlier rows' totals.
__device__ __forceinline__ int32_t wave_incl_sum_i32(int32_t v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// The maximum of the wave's f64 values (no NaN), in every lane: quad butterflies, the
// half-row and row mirrors, then the row broadcasts 15 and 31 carry rows 0-2 into row
// 3, whose lane 63 is read out.  max is exact and order-free.
__device__ __forceinline__ double wave_max_f64(double v) {
  v = fmax(v, dpp_f64<0xB1, 0xf>(v));   // quad_perm [1,0,3,2]
  v = fmax(v, dpp_f64<0x4E, 0xf>(v));   // quad_perm [2,3,0,1]
  v = fmax(v, dpp_f64<0x141, 0xf>(v));  // row_half_mirror
  v = fmax(v, dpp_f64<0x140, 0xf>(v));  // row_mirror
  v = fmax(v, dpp_f64<0x142, 0xa>(v));  // row_bcast:15 into rows 1, 3
  v = fmax(v, dpp_f64<0x143, 0xc>(v));  // row_bcast:31 into rows 2, 3
  return readlane_f64(v, LGBM_WAVE - 1);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  uint32_t l = lane_id();
  return l == 0 ? 0ull : ((1ull << l) - 1ull);
}

// SplitInner router (data_partition.rs:387-417).
__host__ __device__ __forceinline__ bool route_right(int32_t bin, int32_t pmin, int32_t max_bin,
                                                     int32_t th, int32_t na_bin, int32_t flags) {
  if ((flags & 2) && bin == na_bin) return !(flags & 4);
  if (bin < pmin || bin > max_bin) return (flags & 1) != 0;
  return bin > th;
}

// Bits of the bins in [a, b] that fall in word w (bins 32w .. 32w + 31).
__host__ __device__ __forceinline__ uint32_t bin_range_bits(int32_t w, int32_t a, int32_t b) {
  const int32_t lo = 32 * w, hi = lo + 31;
  if (a < lo) a = lo;
  if (b > hi) b = hi;
  if (a > b) return 0u;
  const uint32_t upto_b = (b - lo) == 31 ? 0xffffffffu : ((1u << (b - lo + 1)) - 1u);
  return upto_b & ~((1u << (a - lo)) - 1u);
}
// route_right over all 256 u8 bins as a bit set: word w, bit b <=> bin 32w + b goes
// right.
__host__ __device__ __forceinline__ uint32_t route_right_word(int32_t w, int32_t pmin,
                                                            int32_t max_bin, int32_t th,
                                                            int32_t na_bin, int32_t flags) {
  const int32_t first_right = th + 1 > pmin ? th + 1 : pmin;
  uint32_t m = bin_range_bits(w, first_right, max_bin);
  if (flags & 1) m |= ~bin_range_bits(w, pmin, max_bin);  // out of range: default right
  if ((flags & 2) && na_bin >= 32 * w && na_bin < 32 * w + 32) {
    const uint32_t bit = 1u << (na_bin - 32 * w);
    m = (flags & 4) ? (m & ~bit) : (m | bit);
  }
  return m;
}
