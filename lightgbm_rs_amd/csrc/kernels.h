// lgbm_kernels.h — gfx950 kernels of the tree-learner hot path.
//
// Row store.  Every row is one record (formats in lgbm_device.h): its bins, and either
// the original row index (8-bit bins, W x 16 bytes) or, with every num_bin <= 64, 6-bit
// bins and the row's quantized pair (4U bytes: 24 at 28 features).  A separate array
// holds the packed quantized (grad, hess) pairs in the original order (the quantizer's
// output).  Records are *physically* repartitioned at every split into ping-pong
// buffers, so a leaf's rows are always one contiguous range: ConstructHistogram streams
// them, and the partition is a single pass.  The right child of a split is stored in
// reverse order (its logical order is the reference's ascending order; see
// k_partition), which lets the partition place both children without knowing the left
// count in advance.
//
// Histograms are exact integers: per (feature, bin) cell the kernel counts
// sum(q_g), sum(q_h) and #(q_h == 3).  With num_grad_quant_bins = 4 every
// dequantized f32 value the reference folds is v(q) = f32(q * scale); v(+-1),
// v(+-2), v(4) are exact multiples of v(1) and v(3) is the only other value, so
// the reference's sequential f64 fold of those values equals
//   grad = sum(q_g) * v_g(1),  hess = (sum(q_h) - 3 n3) * v_h(1) + n3 * v_h(3)
// exactly (all partial sums are integer multiples of one ulp unit below 2^53).
#pragma once

#include "lgbm_device.h"

#include <hip/hip_ext.h>

struct RowBufs {
  uint4* rec[NBUF];
  uint16_t* gh[NBUF];   // packed quantized (q_g, q_h) per row
  float2* g32[NBUF];    // f32 (g, h) per row (non-quantized training)
};

// Buffer i of a row store, selected without indexing the kernel-argument array (the
// pointers stay in scalar registers; i is wave-uniform).
template <typename T>
__device__ __forceinline__ T* buf_sel(T* const (&a)[NBUF], int i) {
  T* p = a[0];
#pragma unroll
  for (int k = 1; k < NBUF; ++k) p = i == k ? a[k] : p;
  return p;
}
__device__ __forceinline__ uint4* rec_buf(const RowBufs& b, int i) { return buf_sel(b.rec, i); }
template <typename T>
__device__ __forceinline__ T* gh_buf(const RowBufs& b, int i);
template <>
__device__ __forceinline__ uint16_t* gh_buf<uint16_t>(const RowBufs& b, int i) {
  return buf_sel(b.gh, i);
}
template <>
__device__ __forceinline__ float2* gh_buf<float2>(const RowBufs& b, int i) {
  return buf_sel(b.g32, i);
}
__device__ __forceinline__ uint32_t gh_bits(uint16_t q) { return q; }
__device__ __forceinline__ uint32_t gh_bits(float2) { return 0u; }

// Per-leaf-id partition ranges, filled by k_tree_finalize for the layout export.
struct DevLeaves {
  int32_t* begin;
  int32_t* count;
  int32_t* buf;
  int32_t* rev;
};

// Node slots.  Every node the driver creates (the root, and both children of every
// split it performs, including speculative ones) owns one slot; a committed leaf id
// maps onto the slot of its current node (leaf_slot).  Slot state: the node's row
// range in a row buffer, depth, LeafSums, its speculated children (child[2s],
// child[2s+1], -1 if not split yet), and its best split (key_gain / key_feat, best,
// best_fpos) with the per-feature results and histograms it came from.
struct DevNodes {
  int32_t* begin;
  int32_t* count;
  int32_t* buf;
  int32_t* rev;
  int32_t* depth;
  int32_t* child;       // [2 * slot_cap]
  LeafSums* sums;
  double* key_gain;     // best split gain (-inf: none)
  int32_t* key_feat;    // real feature index of the best split (-1: none)
};

struct DevTree {
  int32_t* header;            // [0] num_leaves, [1] error (written by k_tree_finalize)
  int32_t* split_feature;
  uint32_t* threshold_in_bin;
  double* threshold;
  float* split_gain;
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
  double* internal_weight;  // left + right sum_hessian at the split (Tree::split)
  NodeRoute* nodes;
  uint32_t* route_mask;       // [MAX_LEAVES - 1][8]: bins a node routes right (bit set)
  uint32_t* route_node;       // [MAX_LEAVES - 1]: record byte | left << 8 | right << 20
  uint32_t* cat_left;         // [MAX_LEAVES - 1][8]: categorical node: bins going left
};

struct DevLearner {
  Ctl* ctl;
  const DevFeature* feats;
  const double* ub;
  int32_t F;
  int32_t total_cells;
  int32_t max_bins;           // the widest feature's num_bin (scan LDS rows)
  int32_t has_cat;            // some feature is categorical (the scans' categorical path)
  int32_t bin16;              // wide layout: 2-byte bins (a feature has more than 256)
  int32_t n_wgroups;          // 2-byte bins: feature groups of k_hist_wide
  const int32_t* wgroups;     // [n_wgroups + 1] their first features
  int32_t fmt;                // row record format (rec_words / rec_packed)
  int64_t N;
  uint64_t slot_len;
  int32_t* hist_part;         // [HIST_SLOTS][total_cells][3] root / per-op partials
  int32_t* hist_sum;          // [total_cells][3] job 0's partials summed (k_hist_reduce)
  int32_t* hist_acc;          // [SPEC_MAX][acc_cells][3] per-job accumulators
  unsigned long long* hist_accp;  // [SPEC_MAX][acc_cells] packed accumulators (small jobs)
  int64_t* hist_acc64;        // wide layout, f32 gradients: [SPEC_MAX][acc_cells][2]
  unsigned long long* wide_part;  // wide layout: per-chunk partial cells [chunks][cells][1 or 2]
  int32_t acc_cells;          // cells per accumulator: total_cells, + 1 (row totals) when wide
  const uint8_t* binmat;      // wide layout: row-major bins [N][row_stride]
  const uint8_t* bincol;      // wide layout: the same bins feature-major [F][N] (1 or 2
                              // bytes each; NULL if it did not fit), the partition's router
  int64_t row_stride;
  const uint8_t* feat_used;   // per feature position: the tree's column sample (NULL: all)
  unsigned long long* part_slots;  // [part blocks + SPEC_MAX][total_cells] packed (block, job) cells
  // f32-gradient training: 64-bit fixed-point (g, h) cells
  int64_t* hist_part64;       // [HIST_SLOTS][total_cells][2]
  int64_t* int_slots64;       // [slot_cap][total_cells][2]
  int32_t n_fgroups;          // feature groups of k_hist_f32 (cells of a group fit LDS)
  int32_t fgroup_first[MAX_FGROUPS + 1];
  int32_t* int_slots;         // [slot_cap][total_cells][3] per-node integer histograms
  double* slots;              // [slot_cap][slot_len] per-node f64 histograms (nodes with
                              // fmat set, and the root)
  // A node's f64 cells are its integer cells converted (int_cell_to_f64, or the
  // fixed-point scale), except the cell FixHistogram writes (its f64 pair in mfbv); a
  // node whose cells cannot be derived that way (fmat = 1) holds them in `slots`.
  double2* mfbv;              // [slot_cap][F] the fixed most-frequent-bin cell
  int32_t* fmat;              // [slot_cap] 1: the node's f64 cells are in `slots`
  lgbm_split_info* feat_split;  // [slot_cap][F]
  double* gain_dense;           // [slot_cap][F] the same gains, contiguous (the plan's ArgMax)
  lgbm_split_info* best;        // [slot_cap]
  int32_t* best_fpos;           // [slot_cap] feature position of best
  uint8_t* splittable;          // [slot_cap][F]
  uint32_t* cat_bits;           // [slot_cap][F][8] categorical features: best split's left bins
  int32_t* plan_state;          // [5][MAX_LEAVES] leaf / node linkage owned by k_plan
  uint64_t* tile_state;         // stable per-op partition: left-row prefix per tile
  double* stats;                // [0] rows partitioned, [1] partition launches, [2] root
                                // rows, [3] root launches, [4] partition jobs, [5] rows
                                // histogrammed by partition passes
  DevNodes nodes;
  DevLeaves leaves;
  DevTree tree;
  RowBufs bufs;
};

// LambdaRank on the device (objective.hip): one LAMBDARANK_THREADS block per query of at
// most RANK_MAX_QUERY rows; the tables are built on the host.
#define LAMBDARANK_THREADS 128
#define RANK_SIGMOID_BINS (1024 * 1024)
#define RANK_MAX_QUERY 2048
#ifndef PLAN_CAP_WORK
#define PLAN_CAP_WORK 2048             // features x (2 for f32 cells) from which k_plan caps speculation
#endif
#ifndef RANK_BATCH
#define RANK_BATCH 4                   // rows of the lambdarank loop per batch (2-5 measured alike, 8 and 16 slower)
#endif
#define RANK_LDS_BUDGET (150 * 1024)   // the lambdarank block's LDS at most
#define RANK_DISCOUNTS 10000
struct RankParams {
  double sigmoid, min_in, max_in, idx_factor;
  int32_t norm, trunc;
};
struct RankTables {
  const int32_t* qb;           // [num_queries + 1] query boundaries
  const double* inv_max_dcg;   // [num_queries]
  const double* table;         // [RANK_SIGMOID_BINS] 1 / (1 + exp(score * sigmoid))
  const double* discount;      // [RANK_DISCOUNTS] 1 / log2(2 + i)
  const double* gain;          // label gains (31)
  RankParams p;
  int32_t num_queries, max_query;
};

namespace lgbm {
// Per-launch timing: when either event is set, the launch goes through
// hipExtLaunchKernel, which binds `start` / `stop` to that kernel's begin / end.
struct KernelEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};

// Launch `kern` plainly, or with the kernel-stamped events of `ev` when timing.
#define KLAUNCH(ev, kern, grid, block, lds, s, ...)                                        \
  do {                                                                                   \
    if ((ev) && ((ev)->start || (ev)->stop))                                             \
      hipExtLaunchKernelGGL(kern, grid, block, (uint32_t)(lds), s, (ev)->start, (ev)->stop, \
                            0u, __VA_ARGS__);                                            \
    else                                                                                 \
      kern<<<grid, block, lds, s>>>(__VA_ARGS__);                                        \
  } while (0)

void launch_pack_records(const uint8_t* bins, int64_t n, int32_t F, int32_t fmt, uint4* rec,
                         hipStream_t s);

// One feature's mapper as the binning kernel reads it (ValueToBin,
// lgbm-dataset/src/bin_mapper.rs:148-189).
struct DevBinFeature {
  int32_t categorical;  // 0 numerical (search ub), 1 categorical (search cats)
  int32_t last;         // numerical: last searchable bin (num_bin-1, -1 more with a NaN bin)
  int32_t nan_bin;      // numerical: the NaN bin (num_bin-1) when missing_type is NaN, else -1
  int32_t off;          // offset into ub (numerical) or cats (categorical)
  int32_t ncat;         // categorical: number of (category, bin) pairs, sorted by category
  int32_t ub_pos;       // first of the feature's entries in the bounds array (any type)
  int32_t _pad[2];
};
// Bins a dense raw matrix (f32 or f64; row-major [n][F] or column-major [F][n]) into
// the resident records; `ub_count` upper bounds are staged in LDS.
void launch_bin_records(const void* x, int32_t f64, int32_t col_major, int64_t n, int32_t F,
                        int32_t fmt, const DevBinFeature* feats, const double* ub, int32_t ub_count,
                        const int2* cats, uint4* rec, hipStream_t s, const KernelEvents* ev);
void launch_absmax(const float* g, const float* h, int64_t n, uint4* partials, hipStream_t s);
void launch_grad_binary(const double* score, const float* label, float* g, float* h, int64_t n,
                        uint4* partials, hipStream_t s);
void launch_grad_l2(const double* score, const float* label, float* g, float* h, int64_t n,
                    hipStream_t s);
void launch_grad_lambdarank(const double* score, const float* label, const RankTables& t,
                            float* g, float* h, hipStream_t s);
// Opts the lambdarank kernel into the LDS of a query of max_query rows; 0 = ok.
int lambdarank_prepare(int32_t max_query);
void launch_grad_softmax(const double* score, const float* label, float* g, float* h, int64_t n,
                         int32_t K, double factor, hipStream_t s);
void launch_quant_scales(Ctl* ctl, const uint4* partials, int64_t n, int32_t bins,
                         int32_t force_const, hipStream_t s);
void launch_quantize(const float* g, const float* h, int64_t n, const Ctl* ctl,
                     const uint64_t* wave_mats, const uint64_t* lane_mats, uint64_t s0,
                     int32_t stochastic, uint16_t* gh, float* dg, float* dh, hipStream_t s);
void launch_requant(const float* g, const float* h, int64_t n, const Ctl* ctl, int32_t bins,
                    uint16_t* gh, unsigned long long* bad, hipStream_t s);
void launch_hist(const DevLearner& L, hipStream_t s, const KernelEvents* ev = nullptr);
void launch_fixscan(const DevLearner& L, int32_t mode, double* explicit_out, hipStream_t s,
                    const KernelEvents* ev = nullptr);
void launch_plan(const DevLearner& L, int32_t slot_cap, hipStream_t s,
                 const KernelEvents* ev = nullptr);
void launch_pair_scan(const DevLearner& L, int fp, int32_t spec_max, int32_t part_grid,
                      hipStream_t s, const KernelEvents* ev = nullptr);
void launch_scan_explicit(const double* hist, const DevFeature* feats, int32_t n_feats,
                          const lgbm_gain_config& cfg, double sg, double sh, int32_t n,
                          lgbm_split_info* out, hipStream_t s);
void launch_partition(const DevLearner& L, int fp, int64_t blocks, hipStream_t s,
                      const KernelEvents* ev = nullptr);
// Stable variant for the per-op entry point (job 0, W = 1): tile counts, their
// prefix, then the partition in DataPartition::split order.
void launch_partition_stable(const DevLearner& L, int64_t ntiles, int64_t blocks, hipStream_t s);
void launch_hist_f32(const DevLearner& L, hipStream_t s, const KernelEvents* ev = nullptr);
void launch_fp_prep(const DevLearner& L, const float* g, const float* h, int64_t n,
                    const uint4* partials, hipStream_t s);
// quantized gradients of a bin count other than 2 or 4: the dequantized values dg, dh
// through the fixed-point path with the exact scales of the quantizer's header
void launch_exact_prep(const DevLearner& L, const float* dg, const float* dh, int64_t n,
                       hipStream_t s);
// timing pass: a device-side wait of `ticks` wall-clock ticks ahead of a kernel sequence
void launch_hold(uint64_t ticks, hipStream_t s);
void launch_tree_init(const DevLearner& L, int32_t max_leaves, int32_t max_depth,
                      int32_t slot_cap, int32_t spec_max, int32_t fp_mode, hipStream_t s,
                      const KernelEvents* ev = nullptr);
void launch_score_update(const DevLearner& L, double lr, double* score, hipStream_t s,
                         const KernelEvents* ev = nullptr);
// leaf id (num_leaves <= 256) of every row by walking the tree from its original record
void launch_leaf_of(const DevLearner& L, uint8_t* leaf_of, hipStream_t s);
void launch_tree_finalize(const DevLearner& L, hipStream_t s, const KernelEvents* ev = nullptr);
size_t export_layout_scratch_bytes(int64_t n, int32_t num_leaves);
// quant_train_renew_leaf: the grown tree's leaf outputs from the original gradients
// over the exported layout (indices as launch_export_layout leaves them)
void launch_renew_leaves(const DevLearner& L, const uint32_t* indices, const float* g,
                         const float* h, double l1, double l2, hipStream_t s);
void launch_export_layout(const DevLearner& L, int32_t num_leaves, uint32_t* indices,
                          void* scratch, hipStream_t s);
void launch_gather_rows(int fmt, const uint32_t* rows, int64_t n, const uint4* rec,
                        const uint16_t* gh, const float2* g32, uint4* rec_out, uint16_t* gh_out,
                        float2* g32_out, hipStream_t s);
void launch_subtract(const double* a, const double* b, int64_t n, double* out, hipStream_t s);
// wide layout (REC_FMT_WIDE): feature-major u8 bins [F][n] -> the row-major matrix
// [n][stride] (padding bytes zero) and the identity row-index records
void launch_pack_wide(const uint8_t* bins, int64_t n, int32_t F, int64_t stride, uint8_t* binmat,
                      uint4* rec, hipStream_t s);
// Opts the wide histogram kernels into their LDS size (outside graph capture); 0 = ok.
int wide_prepare();
// The same for the scans' LDS rows of features wider than 256 bins.
int scan_prepare();
int fixscan_prepare();
// u64 words of the wide layout's per-chunk partial histogram slots
size_t wide_part_words(int32_t F, int64_t N, int32_t cells, int32_t n_groups16);
// feature-major 2-byte bins -> the row-major matrix (2-byte bins)
void launch_wide_cols(const uint8_t* binmat, int64_t n, int32_t F, int64_t stride, int bin16,
                      uint8_t* bincol, hipStream_t s);
void launch_pack_wide16(const uint16_t* bins, int64_t n, int32_t F, int64_t stride,
                        uint8_t* binmat, uint4* rec, hipStream_t s);
// ConstructHistogram of the launch's histogram jobs into the per-job accumulators
void launch_hist_wide(const DevLearner& L, int fp, hipStream_t s, const KernelEvents* ev = nullptr);
// raw values -> the row-major matrix (ValueToBin per feature group, bounds in LDS)
void launch_bin_wide(const void* x, int32_t f64, int32_t col_major, int64_t n, int32_t F,
                     int64_t stride, const DevBinFeature* feats, const double* ub,
                     const int2* cats, uint8_t* binmat, uint4* rec, int32_t bin16, hipStream_t s,
                     const KernelEvents* ev);
void launch_pack_partition(const uint32_t* bins, int64_t n, uint4* rec, hipStream_t s);
}  // namespace lgbm
