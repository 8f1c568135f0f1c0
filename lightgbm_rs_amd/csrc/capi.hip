// capi.hip — the C-ABI (include/lgbm_hip.h) over the gfx950 kernels.
//
// A context owns every device allocation.  Each call is synchronous at the API
// boundary (the reference backend's calls are blocking, lib.rs:3840-3846); inside a
// call everything is queued on the context's own HIP stream.
#include <algorithm>
#include <cmath>
#include <array>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "kernels.h"
#include "binning.h"
#include "model.h"

using namespace lgbm;

namespace lgbm {
void launch_predict(const PredNode* nodes, const PredTree* trees, const double* leaves,
                    const int32_t* cat_bounds, const uint32_t* cat_words,
                    const PredLinLeaf* lin_leaves, const int32_t* lin_features,
                    const double* lin_coeffs, const float* X, int64_t rows, int32_t cols, int32_t it0, int32_t it1, int32_t ntpi, int32_t kind,
                    int32_t objective, double sigmoid, int32_t average_output, int32_t es_freq,
                    double es_margin, int32_t* es_iters, double* out, int32_t* leaf_out,
                    hipStream_t s, const KernelEvents* ev);
int64_t shap_bytes_per_row(int32_t depth);
void launch_csr_dense(const int64_t* indptr, const int32_t* indices, const float* values,
                      int64_t nnz, int64_t rows, int32_t cols, int32_t width, float* dense,
                      uint32_t* err, hipStream_t s);
void launch_csc_dense(const int64_t* indptr, const int32_t* indices, const float* values,
                      int64_t nnz, int64_t rows, int32_t cols, int32_t width, float* dense,
                      uint32_t* err, hipStream_t s);
void launch_contrib(const PredNode* nodes, const PredTree* trees, const double* leaves,
                    const int32_t* cat_bounds, const uint32_t* cat_words, const double* node_cover,
                    const double* leaf_cover, const double* expected, const float* X, int64_t r0,
                    int64_t n, int64_t rows, int32_t cols, int32_t nf, int32_t it0, int32_t it1,
                    int32_t ntpi, int32_t depth, void* ws, double* out, hipStream_t s,
                    const KernelEvents* ev);
}

// Working memory of lgbm_hip_find_best_splits_noalloc: a 256-byte header (word 0:
// the first invalid feature's error code) and the converted feature table.  Host
// code never uses this name for memory: each device's address comes from
// hipGetSymbolAddress at context creation (noalloc_scratch_ptr).
#define NOALLOC_HEADER 256
static __device__ __align__(256) unsigned char
    scratch[NOALLOC_HEADER + (size_t)LGBM_HIP_NOALLOC_MAX_FEATURES * sizeof(DevFeature)];

namespace {

thread_local std::string g_create_err;
std::string g_bin_err;    // last failed lgbm_hip_bin_mapper_*
std::string g_model_err;  // last failed lgbm_hip_model_load

struct EventPair {
  hipEvent_t a, b;
  int family;
};

// LightGBM's LCG (lgbm-core/src/random.rs:37-123: x = 214013 x + 2531011) and its
// Sample(n, k).
struct Lcg32 {
  uint32_t state = 0;
  int32_t step16() {
    state = state * 214013u + 2531011u;
    return (int32_t)((state >> 16) & 0x7fffu);
  }
  int32_t step31() {
    state = state * 214013u + 2531011u;
    return (int32_t)(state & 0x7fffffffu);
  }
  // k sorted distinct values of [0, n): all of them when k == n; a streaming pass
  // when k > n / log2(k); else k draws into a set, a repeated draw v taking r instead
  std::vector<int32_t> sample(int32_t n, int32_t k) {
    std::vector<int32_t> out;
    if (k > n || k <= 0) return out;
    if (k == n) {
      for (int32_t i = 0; i < n; ++i) out.push_back(i);
      return out;
    }
    if (k > 1 && (double)k > (double)n / std::log2((double)k)) {
      for (int32_t i = 0; i < n; ++i) {
        const float u = (float)step16() / 32768.0f;
        if ((double)u < (double)(k - (int32_t)out.size()) / (double)(n - i)) out.push_back(i);
      }
      return out;
    }
    std::vector<uint8_t> taken((size_t)n, 0);
    for (int32_t r = n - k; r < n; ++r) {
      const int32_t v = step31() % (r + 1);
      taken[(size_t)(taken[(size_t)v] ? r : v)] = 1;
    }
    for (int32_t i = 0; i < n; ++i)
      if (taken[(size_t)i]) out.push_back(i);
    return out;
  }
};

// The per-tree column sample of feature_fraction (ColSampler, lgbm-treelearner/src/
// col_sampler.rs:68-140): the sampler draws once when it is created and once before
// every tree (learner.rs:1190-1240), round(F * fraction) (at least one) features.
struct FeatureSampler {
  Lcg32 rng;
  int32_t count = 0, F = 0;
  std::vector<uint8_t> used;  // by feature position
  void start(double fraction, int32_t seed, int32_t num_features) {
    rng.state = (uint32_t)seed;
    F = num_features;
    const int32_t c = (int32_t)((double)F * fraction + (double)0.5f);
    count = std::max(c, std::min(1, F));
    next_tree();
  }
  void next_tree() {
    used.assign((size_t)F, 0);
    for (int32_t pos : rng.sample(F, count)) used[(size_t)pos] = 1;
  }
};

}  // namespace

struct lgbm_hip_ctx {
  // device copy of the last model predicted with (keyed by the model's uid)
  uint64_t pm_uid = 0;
  PredNode* pm_nodes = nullptr;
  PredTree* pm_trees = nullptr;
  double* pm_leaves = nullptr;
  int32_t* pm_catb = nullptr;
  uint32_t* pm_catw = nullptr;
  PredLinLeaf* pm_linl = nullptr;
  int32_t* pm_linf = nullptr;
  double* pm_linc = nullptr;
  double* pm_ncov = nullptr;  // TreeSHAP covers and expected values
  double* pm_lcov = nullptr;
  double* pm_expv = nullptr;
  char* pm_csr = nullptr;  // sparse-input staging: error word, indptr, indices, values
  size_t pm_csr_cap = 0;
  char* pm_shap = nullptr;  // TreeSHAP path workspace
  size_t pm_shap_cap = 0;
  float* pm_x = nullptr;  // host-input staging
  size_t pm_x_cap = 0;
  void* pm_out = nullptr;
  size_t pm_out_cap = 0;
  int device = 0;
  hipStream_t stream = nullptr;
  std::string err;
  unsigned char* noalloc = nullptr;  // this device's `scratch` (hipGetSymbolAddress)
  // shape
  int64_t N = 0;
  int32_t F = 0, fmt = 1, total_cells = 0;  // fmt: row record format (lgbm_device.h)
  int32_t records_env = 0;  // LGBM_HIP_RECORDS: 0 automatic, 1 legacy (8-bit records), 2 wide
  bool no_bincol = false;   // LGBM_HIP_BINCOL=0: the wide layout without its feature-major copy
  int32_t max_bins = 0;     // the widest feature's num_bin
  int32_t has_cat = 0;      // some feature is categorical
  bool bin16 = false;       // wide layout with 2-byte bins
  int32_t n_wgroups = 0;    // 2-byte bins: feature groups of the histogram kernel
  int32_t* d_wgroups = nullptr;  // [n_wgroups + 1] first feature of each group
  uint8_t* binmat = nullptr;  // wide layout: row-major bins [N][row_stride]
  uint8_t* bincol = nullptr;  // wide layout: feature-major copy [F][N] (optional)
  int64_t row_stride = 0;
  uint64_t slot_len = 0;
  std::vector<DevFeature> feats;
  std::vector<double> ub_host;  // per-bin values (numerical: upper bounds, categorical: categories)
  // words of one categorical node's bitset at most (largest category value / 32 + 1);
  // 0 without categorical features
  int64_t cat_words_node = 0;
  bool have_bins = false, have_grad = false, quant_ready = false, have_labels = false;
  int32_t quant_bins = 0;
  // lookahead (lgbm_hip_set_lookahead): the next iteration's objective + quantizer
  // enqueued by train_iter_binary before it waits for its tree copy
  bool lookahead = false, ahead = false;
  int32_t ahead_iter = 0, ahead_qbins = 0, ahead_stoch = 0, ahead_obj = 0;
  // objective of lgbm_hip_train_iter (LGBM_HIP_OBJECTIVE_*)
  int32_t objective = LGBM_HIP_OBJECTIVE_BINARY;
  // lambdarank tables (lgbm_hip_set_lambdarank)
  int32_t* rk_qb = nullptr;
  double *rk_imd = nullptr, *rk_table = nullptr, *rk_disc = nullptr, *rk_gain = nullptr;
  RankTables rank{};
  bool have_rank = false;
  // feature_fraction (lgbm_hip_set_col_sampler): a new column sample before every tree
  FeatureSampler colsamp;
  bool colsamp_on = false;
  uint8_t* d_feat_used = nullptr;
  uint8_t* feat_used_host = nullptr;  // pinned
  hipEvent_t tree_ev = nullptr;
  // device memory
  Ctl* ctl = nullptr;
  DevFeature* d_feats = nullptr;
  double* d_ub = nullptr;
  uint4* rec[NBUF] = {};
  uint16_t* gh[NBUF] = {};
  float2* g32[NBUF] = {};  // f32 (g, h) pairs, allocated on first f32-gradient use
  int64_t g32_rows[NBUF] = {};
  int64_t buf_rows[NBUF] = {};
  float *g = nullptr, *h = nullptr, *label = nullptr;
  double* score = nullptr;     // [num_class][N] class-major
  int32_t num_class = 1;       // classes of the resident score (lgbm_hip_set_labels*)
  float *gk = nullptr, *hk = nullptr;  // multiclass: [num_class][N] gradients
  int32_t* hist_part = nullptr;  // [HIST_SLOTS][cells][3]
  int32_t* hist_sum = nullptr;   // [cells][3]
  int32_t* hist_acc = nullptr;   // [SPEC_MAX][acc_cells][3]
  unsigned long long* hist_accp = nullptr;  // [SPEC_MAX][acc_cells] packed (small jobs)
  int64_t* hist_acc64 = nullptr;  // wide layout: [SPEC_MAX][acc_cells][2]
  unsigned long long* wide_part = nullptr;  // wide layout: per-chunk partial cells
  int32_t acc_cells = 0;          // total_cells (+ 1 totals cell in the wide layout)
  unsigned long long* part_slots = nullptr;  // [part_blocks + SPEC_MAX][cells] packed
  int64_t* hist_part64 = nullptr;  // [HIST_SLOTS][cells][2]
  int64_t* int_slots64 = nullptr;  // [SLOT_CAP][cells][2]
  int32_t n_fgroups = 0;
  int32_t fgroup_first[MAX_FGROUPS + 1] = {};
  uint64_t* tile_state = nullptr;
  int64_t tile_cap = 0;
  uint64_t *wave_mats = nullptr, *lane_mats = nullptr;
  double* stats = nullptr;
  uint4* partials = nullptr;  // per-block g/h statistics
  unsigned long long* d_flags = nullptr;  // [2]: check kernels' (count, first row)
  // tree-sized: node slots (SLOT_CAP(lcap)) and per-leaf arrays
  int32_t lcap = 0;
  double* slots = nullptr;
  lgbm_split_info *feat_split = nullptr, *best = nullptr;
  double* gain_dense = nullptr;  // [slot_cap][F] feat_split's gains, contiguous
  double2* mfbv = nullptr;       // [slot_cap][F] quantized: the fixed cell's f64 pair
  int32_t* fmat = nullptr;       // [slot_cap] quantized: f64 cells held in `slots`
  int32_t* best_fpos = nullptr;
  int32_t* int_slots = nullptr;
  uint8_t* splittable = nullptr;
  uint32_t* cat_bits = nullptr;   // [SLOT_CAP][F][8]
  int32_t* plan_state = nullptr;  // [5][MAX_LEAVES]
  DevNodes nodes{};
  DevLeaves leaves{};
  DevTree tree{};
  void* tree_blob = nullptr;   // device tree arrays, one allocation
  void* tree_host = nullptr;   // pinned staging for the one-copy readback
  size_t tree_blob_bytes = 0;
  size_t tree_off[17] = {};
  // scratch
  void* scratch = nullptr;
  size_t scratch_cap = 0;
  double* slot_tmp = nullptr;
  // quant_train_renew_leaf (lgbm_hip_set_quant_renew_leaf): the exported layout and
  // its scratch, sized for num_data rows and MAX_LEAVES leaves
  bool renew_leaf = false;
  int64_t renew_rows = 0;
  // dequantized gradients of a bin count other than 2 or 4 ([2][N] f32), fed to the
  // fixed-point learner path with exact scales
  float* dq = nullptr;
  int64_t dq_rows = 0;
  uint32_t* renew_idx = nullptr;
  void* renew_scratch = nullptr;
  // device-resident histogram slots (lgbm_hip_resident_*)
  double* res_slots = nullptr;
  int32_t res_num = 0;
  int64_t res_len = 0, res_cap = 0;
  uint32_t* d_indices = nullptr;
  int64_t indices_cap = 0;
  // Captured per-tree launch sequences (all parameters live in device memory): one per
  // round count in use (the round count follows the trees, a re-instantiation costs
  // more than a tree's round), and a tail of TAIL_ROUNDS rounds launched when a tree
  // needs more rounds than its sequence holds.  Keyed together by the tree shape.
  static constexpr int GRAPH_CACHE = 8, TAIL_ROUNDS = 4, ROUND_HIST = 16;
  hipGraphExec_t graph_exec[GRAPH_CACHE] = {};
  int32_t graph_rounds[GRAPH_CACHE] = {};
  uint64_t graph_used[GRAPH_CACHE] = {};  // last use (LRU eviction)
  uint64_t graph_clock = 0;
  hipGraphExec_t tail_exec = nullptr;
  int32_t graph_nl = -1, graph_md = 0, graph_spec = 0, graph_fp = -1;
  int32_t round_cap = 24;     // partition rounds in the captured sequence
  bool round_fixed = false;   // LGBM_HIP_ROUNDS: a fixed round count
  int32_t round_hist[ROUND_HIST] = {};  // rounds the last trees used (ring)
  int32_t round_hist_n = 0;
  int32_t spec_max = SPEC_DEFAULT;
  bool spec_env = false;  // LGBM_HIP_SPEC fixes spec_max
  int32_t part_blocks = 256 * PART_BLOCKS_PER_CU;  // partition grid (set from the CU count)
  int32_t* done_host = nullptr;  // pinned: ctl->done after the captured rounds
  double tree_rounds = 0.0, trees = 0.0, extra_rounds = 0.0;
  double part_launches = 0.0;  // partition kernels enqueued while timing (empty rounds too)
  // binning and prediction launches while timing: launches, values binned, row-trees walked
  double bin_launches = 0.0, bin_values = 0.0, pred_launches = 0.0, pred_walks = 0.0;
  uint64_t graph_gen = 0, buf_gen = 1;
  bool use_graphs = true;
  // timing
  bool timing = false;
  uint64_t hold_ticks = 0;  // the timing pass's device wait ahead of each kernel sequence
  std::vector<EventPair> ev_pool;
  size_t ev_used = 0;
  // Per-tree event list: every timed kernel gets a (start, stop) pair bound to its own
  // begin / end by the launch, so chain[i] - chain[i-1] for a stop event i is that
  // kernel's duration alone (dispatch gaps excluded).
  std::vector<hipEvent_t> chain;
  std::vector<int> chain_family;
  size_t chain_used = 0;
  double ms[7] = {0, 0, 0, 0, 0, 0, 0};
};

namespace {

// Per-device address of `scratch`, resolved once per device with that device current.
std::mutex g_noalloc_mu;
std::vector<unsigned char*> g_noalloc_ptr;

int noalloc_scratch_ptr(int device, unsigned char** out) {
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if ((int)g_noalloc_ptr.size() <= device) g_noalloc_ptr.resize((size_t)device + 1, nullptr);
  if (!g_noalloc_ptr[(size_t)device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return (int)e ? (int)e : -1;
    g_noalloc_ptr[(size_t)device] = (unsigned char*)p;
  }
  *out = g_noalloc_ptr[(size_t)device];
  return 0;
}

int set_err(lgbm_hip_ctx* c, int code, const std::string& m) {
  if (c)
    c->err = m;
  else
    g_create_err = m;
  return code;
}

#define HIPCHK(c, expr)                                                                   \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess)                                                                 \
      return set_err(c, LGBM_HIP_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(_e)); \
  } while (0)

template <typename T>
int dalloc(lgbm_hip_ctx* c, T** p, size_t count) {
  if (*p) {
    (void)hipFree(*p);
    *p = nullptr;
  }
  if (count == 0) count = 1;
  HIPCHK(c, hipMalloc((void**)p, count * sizeof(T)));
  return LGBM_HIP_OK;
}

// ---- xorshift64 jump matrices (GF(2)); column i = image of basis vector e_i ----
using Mat = std::array<uint64_t, 64>;
uint64_t xs_step(uint64_t x) {
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  return x;
}
uint64_t mat_apply(const Mat& m, uint64_t v) {
  uint64_t y = 0;
  for (int i = 0; i < 64; ++i)
    if ((v >> i) & 1ull) y ^= m[i];
  return y;
}
Mat mat_mul(const Mat& a, const Mat& b) {
  Mat c;
  for (int i = 0; i < 64; ++i) c[i] = mat_apply(a, b[i]);
  return c;
}

int init_jump_tables(lgbm_hip_ctx* c) {
  Mat m;
  for (int i = 0; i < 64; ++i) m[i] = xs_step(1ull << i);
  // T = M^(2*C): two draws per row, C rows per lane
  Mat t = m;
  static_assert((QUANT_ROWS_PER_LANE & (QUANT_ROWS_PER_LANE - 1)) == 0, "C must be a power of 2");
  for (int k = 1; k < 2 * QUANT_ROWS_PER_LANE; k *= 2) t = mat_mul(t, t);
  // lane table: T^l for l = 0..63, stored column-major across lanes
  // (entry [i][l] = column i of T^l) so a wave reads one column of every lane's
  // matrix in one coalesced load
  std::vector<uint64_t> lane(64 * 64), wave(QUANT_WAVE_MATS * 64);
  Mat r;
  for (int i = 0; i < 64; ++i) r[i] = 1ull << i;  // T^0
  for (int l = 0; l < 64; ++l) {
    for (int i = 0; i < 64; ++i) lane[(size_t)i * 64 + l] = r[i];
    r = mat_mul(r, t);
  }
  Mat p = r;  // T^64 = M^(2*C*64): one wave's rows
  for (int k = 0; k < QUANT_WAVE_MATS; ++k) {
    std::copy(p.begin(), p.end(), wave.begin() + k * 64);
    p = mat_mul(p, p);
  }
  int rc = dalloc(c, &c->lane_mats, lane.size());
  if (rc) return rc;
  rc = dalloc(c, &c->wave_mats, wave.size());
  if (rc) return rc;
  HIPCHK(c, hipMemcpy(c->lane_mats, lane.data(), lane.size() * 8, hipMemcpyHostToDevice));
  HIPCHK(c, hipMemcpy(c->wave_mats, wave.data(), wave.size() * 8, hipMemcpyHostToDevice));
  return LGBM_HIP_OK;
}

DevLearner make_learner(lgbm_hip_ctx* c) {
  DevLearner L{};
  L.ctl = c->ctl;
  L.feats = c->d_feats;
  L.ub = c->d_ub;
  L.F = c->F;
  L.fmt = c->fmt;
  L.total_cells = c->total_cells;
  L.N = c->N;
  L.slot_len = c->slot_len;
  L.hist_part = c->hist_part;
  L.hist_sum = c->hist_sum;
  L.hist_acc = c->hist_acc;
  L.hist_acc64 = c->hist_acc64;
  L.hist_accp = c->hist_accp;
  L.wide_part = c->wide_part;
  L.acc_cells = c->acc_cells;
  L.binmat = c->binmat;
  L.bincol = c->bincol;
  L.row_stride = c->row_stride;
  L.max_bins = c->max_bins;
  L.has_cat = c->has_cat;
  L.bin16 = c->bin16 ? 1 : 0;
  L.n_wgroups = c->n_wgroups;
  L.wgroups = c->d_wgroups;
  L.feat_used = c->colsamp_on ? c->d_feat_used : nullptr;
  L.part_slots = c->part_slots;
  L.hist_part64 = c->hist_part64;
  L.int_slots64 = c->int_slots64;
  L.n_fgroups = c->n_fgroups;
  for (int i = 0; i <= MAX_FGROUPS; ++i) L.fgroup_first[i] = c->fgroup_first[i];
  L.slots = c->slots;
  L.feat_split = c->feat_split;
  L.gain_dense = c->gain_dense;
  L.mfbv = c->mfbv;
  L.fmat = c->fmat;
  L.best = c->best;
  L.best_fpos = c->best_fpos;
  L.int_slots = c->int_slots;
  L.splittable = c->splittable;
  L.cat_bits = c->cat_bits;
  L.plan_state = c->plan_state;
  L.nodes = c->nodes;
  L.tile_state = c->tile_state;
  L.stats = c->stats;
  L.leaves = c->leaves;
  L.tree = c->tree;
  for (int i = 0; i < NBUF; ++i) {
    L.bufs.rec[i] = c->rec[i];
    L.bufs.gh[i] = c->gh[i];
    L.bufs.g32[i] = c->g32[i];
  }
  return L;
}

template <typename T>
int ctl_write(lgbm_hip_ctx* c, size_t off, const T& v) {
  HIPCHK(c, hipMemcpyAsync((char*)c->ctl + off, &v, sizeof(T), hipMemcpyHostToDevice, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return LGBM_HIP_OK;
}
template <typename T>
int ctl_read(lgbm_hip_ctx* c, size_t off, T* v) {
  HIPCHK(c, hipMemcpyAsync(v, (char*)c->ctl + off, sizeof(T), hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return LGBM_HIP_OK;
}
#define CTL_OFF(field) offsetof(Ctl, field)

// Records of n rows in a given format, in 16-byte units.
size_t rec_units(int fmt, int64_t n) {
  return ((size_t)std::max<int64_t>(n, 1) * (size_t)rec_bytes(fmt) + 15) / 16;
}

int ensure_scratch_rows(lgbm_hip_ctx* c, int64_t n) {
  for (int b : {BUF_S0, BUF_S1}) {
    if (c->buf_rows[b] >= n && c->rec[b]) continue;
    int rc = dalloc(c, &c->rec[b], rec_units(c->fmt, n));
    if (rc) return rc;
    rc = dalloc(c, &c->gh[b], (size_t)std::max<int64_t>(n, 1));
    if (rc) return rc;
    rc = dalloc(c, &c->g32[b], (size_t)std::max<int64_t>(n, 1));
    if (rc) return rc;
    c->g32_rows[b] = n;
    c->buf_rows[b] = n;
    c->buf_gen++;
  }
  return LGBM_HIP_OK;
}

int ensure_scratch_bytes(lgbm_hip_ctx* c, size_t bytes) {
  if (c->scratch_cap >= bytes && c->scratch) return LGBM_HIP_OK;
  if (c->scratch) (void)hipFree(c->scratch);
  c->scratch = nullptr;
  HIPCHK(c, hipMalloc(&c->scratch, std::max<size_t>(bytes, 256)));
  c->scratch_cap = std::max<size_t>(bytes, 256);
  return LGBM_HIP_OK;
}

// Per-tile left-row prefix of the stable per-op partition (one job: at most
// rows / tile + 1 tiles); sized for the smallest tile of any launch shape.
int ensure_tile_state(lgbm_hip_ctx* c, int64_t rows) {
  const int64_t tiles = (rows + PART_MIN_TILE - 1) / PART_MIN_TILE + SPEC_MAX + 1;
  if (c->tile_cap >= tiles) return LGBM_HIP_OK;
  c->buf_gen++;
  int rc = dalloc(c, &c->tile_state, (size_t)tiles);
  if (rc) return rc;
  HIPCHK(c, hipMemset(c->tile_state, 0, (size_t)tiles * 8));
  c->tile_cap = tiles;
  return LGBM_HIP_OK;
}

int ensure_leaves(lgbm_hip_ctx* c, int32_t L) {
  if (c->lcap >= L) return LGBM_HIP_OK;
  int rc = 0;
  const size_t F = (size_t)c->F;
  const size_t P = (size_t)SLOT_CAP(L);  // node slots
  if ((rc = dalloc(c, &c->slots, P * c->slot_len))) return rc;
  if ((rc = dalloc(c, &c->feat_split, P * F))) return rc;
  if ((rc = dalloc(c, &c->gain_dense, P * F))) return rc;
  if ((rc = dalloc(c, &c->mfbv, P * F))) return rc;
  if ((rc = dalloc(c, &c->fmat, P))) return rc;
  if ((rc = dalloc(c, &c->best, P))) return rc;
  if ((rc = dalloc(c, &c->splittable, P * F))) return rc;
  if ((rc = dalloc(c, &c->cat_bits, P * F * 8))) return rc;
  if ((rc = dalloc(c, &c->best_fpos, P))) return rc;
  if ((rc = dalloc(c, &c->int_slots, P * c->total_cells * 3))) return rc;
  if ((rc = dalloc(c, &c->int_slots64, P * c->total_cells * 2))) return rc;
  DevNodes& nd = c->nodes;
  if ((rc = dalloc(c, &nd.begin, P))) return rc;
  if ((rc = dalloc(c, &nd.count, P))) return rc;
  if ((rc = dalloc(c, &nd.buf, P))) return rc;
  if ((rc = dalloc(c, &nd.rev, P))) return rc;
  if ((rc = dalloc(c, &nd.depth, P))) return rc;
  if ((rc = dalloc(c, &nd.child, 2 * P))) return rc;
  if ((rc = dalloc(c, &nd.sums, P))) return rc;
  if ((rc = dalloc(c, &nd.key_gain, P))) return rc;
  if ((rc = dalloc(c, &nd.key_feat, P))) return rc;
  if ((rc = dalloc(c, &c->plan_state, (size_t)5 * MAX_LEAVES))) return rc;
  if ((rc = dalloc(c, &c->leaves.begin, (size_t)L))) return rc;
  if ((rc = dalloc(c, &c->leaves.count, (size_t)L))) return rc;
  if ((rc = dalloc(c, &c->leaves.buf, (size_t)L))) return rc;
  if ((rc = dalloc(c, &c->leaves.rev, (size_t)L))) return rc;
  if ((rc = dalloc(c, &c->tree.nodes, (size_t)L))) return rc;
  if ((rc = dalloc(c, &c->tree.route_mask, (size_t)L * 8))) return rc;
  if ((rc = dalloc(c, &c->tree.route_node, (size_t)L))) return rc;
  // tree arrays: one device blob (one readback per tree) + pinned host staging
  const size_t sizes[17] = {64, 4, 4, 8, 4, 1, 4, 4, 8, 4, 8, 8, 4, 4, 4, 8, 32};
  size_t off = 0;
  for (int i = 0; i < 17; ++i) {
    c->tree_off[i] = off;
    off += ((i == 0 ? 64 : sizes[i] * (size_t)L) + 15) / 16 * 16;
  }
  c->tree_blob_bytes = off;
  if (c->tree_blob) (void)hipFree(c->tree_blob);
  if (c->tree_host) (void)hipHostFree(c->tree_host);
  c->tree_blob = nullptr;
  c->tree_host = nullptr;
  HIPCHK(c, hipMalloc(&c->tree_blob, off));
  HIPCHK(c, hipHostMalloc(&c->tree_host, off, hipHostMallocDefault));
  char* base = (char*)c->tree_blob;
  DevTree& T = c->tree;
  T.header = (int32_t*)(base + c->tree_off[0]);
  T.split_feature = (int32_t*)(base + c->tree_off[1]);
  T.threshold_in_bin = (uint32_t*)(base + c->tree_off[2]);
  T.threshold = (double*)(base + c->tree_off[3]);
  T.split_gain = (float*)(base + c->tree_off[4]);
  T.decision_type = (int8_t*)(base + c->tree_off[5]);
  T.left_child = (int32_t*)(base + c->tree_off[6]);
  T.right_child = (int32_t*)(base + c->tree_off[7]);
  T.internal_value = (double*)(base + c->tree_off[8]);
  T.internal_count = (int32_t*)(base + c->tree_off[9]);
  T.leaf_value = (double*)(base + c->tree_off[10]);
  T.leaf_weight = (double*)(base + c->tree_off[11]);
  T.leaf_count = (int32_t*)(base + c->tree_off[12]);
  T.leaf_depth = (int32_t*)(base + c->tree_off[13]);
  T.leaf_parent = (int32_t*)(base + c->tree_off[14]);
  T.internal_weight = (double*)(base + c->tree_off[15]);
  T.cat_left = (uint32_t*)(base + c->tree_off[16]);
  c->lcap = L;
  c->buf_gen++;
  return LGBM_HIP_OK;
}

// f32-gradient training: the (g, h) pair buffers that move with the rows.
// num_grad_quant_bins other than 2 and 4: the dequantized values go through the
// fixed-point path (its scales set from the quantizer's, exact); 2 and 4 take the
// packed integer cells.
bool gen_bins(int32_t bins) { return bins > 0 && bins != 2 && bins != 4; }
int ensure_dq(lgbm_hip_ctx* c) {
  if (c->dq && c->dq_rows >= c->N) return LGBM_HIP_OK;
  int rc = dalloc(c, &c->dq, 2 * (size_t)c->N);
  if (rc) return rc;
  c->dq_rows = c->N;
  return LGBM_HIP_OK;
}

int ensure_fp(lgbm_hip_ctx* c) {
  for (int b : {BUF_ORIG, BUF_A, BUF_B}) {
    if (c->g32[b] && c->g32_rows[b] >= c->N) continue;
    int rc = dalloc(c, &c->g32[b], (size_t)c->N);
    if (rc) return rc;
    c->g32_rows[b] = c->N;
    c->buf_gen++;
  }
  return LGBM_HIP_OK;
}

// ---- timing ---------------------------------------------------------------
hipEvent_t ev_begin(lgbm_hip_ctx* c, int family) {
  if (!c->timing) return nullptr;
  if (c->ev_used == c->ev_pool.size()) {
    EventPair p{};
    (void)hipEventCreateWithFlags(&p.a, hipEventDisableSystemFence);
    (void)hipEventCreateWithFlags(&p.b, hipEventDisableSystemFence);
    c->ev_pool.push_back(p);
  }
  EventPair& p = c->ev_pool[c->ev_used];
  p.family = family;
  (void)hipEventRecord(p.a, c->stream);
  return p.a;
}
hipEvent_t chain_next(lgbm_hip_ctx* c, int family) {
  if (c->chain_used == c->chain.size()) {
    hipEvent_t e = nullptr;
    (void)hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
    c->chain.push_back(e);
    c->chain_family.push_back(-1);
  }
  c->chain_family[c->chain_used] = family;
  return c->chain[c->chain_used++];
}
// The (start, stop) events of one kernel launch (family -1: not counted).  The launch
// binds them to the kernel's own begin and end (hipExtLaunchKernel), so no marker
// packet sits between consecutive kernels.
const KernelEvents* ev_kernel(lgbm_hip_ctx* c, int family, KernelEvents* slot) {
  if (!c->timing) return nullptr;
  slot->start = chain_next(c, -1);
  slot->stop = chain_next(c, family);
  return slot;
}
void ev_end(lgbm_hip_ctx* c) {
  if (!c->timing) return;
  (void)hipEventRecord(c->ev_pool[c->ev_used].b, c->stream);
  c->ev_used++;
}
void ev_collect(lgbm_hip_ctx* c) {
  if (!c->timing) return;
  for (size_t i = 0; i < c->ev_used; ++i) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, c->ev_pool[i].a, c->ev_pool[i].b) == hipSuccess)
      c->ms[c->ev_pool[i].family] += ms;
  }
  c->ev_used = 0;
  for (size_t i = 1; i < c->chain_used; ++i) {
    float ms = 0.f;
    if (c->chain_family[i] >= 0 &&
        hipEventElapsedTime(&ms, c->chain[i - 1], c->chain[i]) == hipSuccess)
      c->ms[c->chain_family[i]] += ms;
  }
  c->chain_used = 0;
}
// Timing pass: the host launches a timed kernel (and its two events) more slowly than
// a small round runs, so a device that has caught up with the host would stamp a start
// event while the kernel is not yet submitted.  A bounded device-side wait ahead of each
// kernel sequence lets the host enqueue the whole sequence first; the events then span
// each kernel's own execution.
void timing_hold(lgbm_hip_ctx* c) {
  if (c->timing) launch_hold(c->hold_ticks, c->stream);
}
enum { FAM_HIST = 0, FAM_PART = 1, FAM_SCAN = 2, FAM_QUANT = 3, FAM_OBJ = 4, FAM_BIN = 5,
       FAM_PRED = 6 };

void drop_graphs(lgbm_hip_ctx* c) {
  for (int i = 0; i < lgbm_hip_ctx::GRAPH_CACHE; ++i) {
    if (c->graph_exec[i]) (void)hipGraphExecDestroy(c->graph_exec[i]);
    c->graph_exec[i] = nullptr;
    c->graph_rounds[i] = 0;
  }
  if (c->tail_exec) (void)hipGraphExecDestroy(c->tail_exec);
  c->tail_exec = nullptr;
}

int check_ctx(lgbm_hip_ctx* c) {
  if (!c) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  HIPCHK(c, hipSetDevice(c->device));
  return LGBM_HIP_OK;
}

int do_quantize(lgbm_hip_ctx* c, int32_t bins, int32_t stochastic, uint64_t seed, float* dg,
                float* dh) {
  ev_begin(c, FAM_QUANT);
  launch_absmax(c->g, c->h, c->N, c->partials, c->stream);
  launch_quant_scales(c->ctl, c->partials, c->N, bins, -1, c->stream);
  launch_quantize(c->g, c->h, c->N, c->ctl, c->wave_mats, c->lane_mats,
                  seed ^ 0x9E3779B97F4A7C15ull, stochastic, c->gh[BUF_ORIG], dg, dh, c->stream);
  ev_end(c);
  HIPCHK(c, hipGetLastError());
  c->quant_ready = true;
  c->quant_bins = bins;
  return LGBM_HIP_OK;
}

// One partition round: plan (commit finished splits, pick the next leaves), the
// partition pass of every picked leaf (which also builds one child's histogram), and
// the children's scans.  Rounds after the tree is complete return at once.
void enqueue_rounds(lgbm_hip_ctx* c, int32_t rounds, int32_t fp) {
  DevLearner L = make_learner(c);
  KernelEvents ke;
  if (c->timing) c->part_launches += rounds;
  for (int32_t r = 0; r < rounds; ++r) {
    launch_plan(L, SLOT_CAP(c->lcap), c->stream, ev_kernel(c, FAM_SCAN, &ke));
    launch_partition(L, fp, c->part_blocks, c->stream, ev_kernel(c, FAM_PART, &ke));
    if (rec_wide(c->fmt))
      launch_hist_wide(L, fp, c->stream, ev_kernel(c, FAM_HIST, &ke));
    else if (fp)
      launch_hist_f32(L, c->stream, ev_kernel(c, FAM_HIST, &ke));
    launch_pair_scan(L, fp, c->spec_max, c->part_blocks, c->stream, ev_kernel(c, FAM_SCAN, &ke));
  }
}

// The per-tree kernel sequence: reset, root histogram + root scan, then rounds.
void enqueue_tree(lgbm_hip_ctx* c, int32_t num_leaves, int32_t max_depth, int32_t rounds,
                  int32_t fp) {
  DevLearner L = make_learner(c);
  KernelEvents ke;
  launch_tree_init(L, num_leaves, max_depth, SLOT_CAP(num_leaves), c->spec_max, fp, c->stream,
                   ev_kernel(c, -1, &ke));
  if (rec_wide(c->fmt))
    launch_hist_wide(L, fp, c->stream, ev_kernel(c, FAM_HIST, &ke));
  else if (fp)
    launch_hist_f32(L, c->stream, ev_kernel(c, FAM_HIST, &ke));
  else
    launch_hist(L, c->stream, ev_kernel(c, FAM_HIST, &ke));
  launch_fixscan(L, 1, nullptr, c->stream, ev_kernel(c, FAM_SCAN, &ke));
  enqueue_rounds(c, rounds, fp);
}

// The round count of the next trees' captured sequence, from the rounds the last trees
// used (ROUND_HIST of them).  The rounds a tree needs follow the training (more in
// later iterations) and vary from tree to tree (widely across the classes of a
// softmax iteration).  A round past the tree's end costs a near-empty plan /
// partition / scan; a tree that needs more runs a tail sequence of TAIL_ROUNDS after
// one host check, which costs about as much.  The count is the multiple of
// ROUND_QUANT that minimises (empty rounds + ROUND_W_TAIL x tail checks) over the
// history; the multiples bound the distinct captured sequences (each a graph
// instantiation).  (The 75th percentile of the history carried too many empty rounds
// where the trees' round counts spread.)
#ifndef ROUND_QUANT
#define ROUND_QUANT 8
#endif
#ifndef ROUND_W_TAIL
#define ROUND_W_TAIL 1
#endif
void update_round_cap(lgbm_hip_ctx* c, int32_t used, int32_t num_leaves) {
  constexpr int H = lgbm_hip_ctx::ROUND_HIST;
  c->round_hist[c->round_hist_n % H] = used;
  c->round_hist_n += 1;
  if (c->round_fixed) return;
  const int n = std::min(c->round_hist_n, H);
  const int32_t top = num_leaves + 1;  // no tree needs more rounds than this
  constexpr int32_t T = lgbm_hip_ctx::TAIL_ROUNDS;
  int32_t best = top;
  int64_t best_cost = INT64_MAX;
  for (int32_t q = ROUND_QUANT; q < top + ROUND_QUANT; q += ROUND_QUANT) {
    const int32_t cap = std::min(q, top);
    int64_t cost = 0;
    for (int i = 0; i < n; ++i) {
      const int32_t r = c->round_hist[i];
      if (r <= cap) {
        cost += cap - r;
      } else {
        const int32_t tails = (r - cap + T - 1) / T;
        cost += (int64_t)tails * T - (r - cap) + (int64_t)ROUND_W_TAIL * tails;
      }
    }
    if (cost < best_cost) {
      best_cost = cost;
      best = cap;
    }
  }
  c->round_cap = std::max(1, best);
}

// The tail sequence: TAIL_ROUNDS more rounds (captured once per tree shape), else the
// same rounds launched one by one.
int launch_tail(lgbm_hip_ctx* c, int32_t fp) {
  constexpr int32_t T = lgbm_hip_ctx::TAIL_ROUNDS;
  if (c->timing || !c->use_graphs) {
    timing_hold(c);
    enqueue_rounds(c, T, fp);
    HIPCHK(c, hipGetLastError());
    return LGBM_HIP_OK;
  }
  if (!c->tail_exec) {
    hipGraph_t g = nullptr;
    HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    enqueue_rounds(c, T, fp);
    HIPCHK(c, hipStreamEndCapture(c->stream, &g));
    hipError_t e = hipGraphInstantiate(&c->tail_exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
      c->tail_exec = nullptr;
      return set_err(c, LGBM_HIP_ERR_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    }
  }
  HIPCHK(c, hipGraphLaunch(c->tail_exec, c->stream));
  return LGBM_HIP_OK;
}

// After the enqueued rounds: rounds commit at least one split each once the first
// leaf is picked, so a tree needs at most num_leaves + 1 plans.  Runs the tail
// (checked after each) until the plan reports the tree complete, then the finalize
// kernel.
int finish_rounds(lgbm_hip_ctx* c, int32_t num_leaves, int32_t rounds, int32_t fp) {
  static_assert(offsetof(Ctl, rounds) - offsetof(Ctl, done) < 64, "ctl readback window");
  const size_t r_off = (offsetof(Ctl, rounds) - offsetof(Ctl, done)) / 4;
  int32_t done_rounds = rounds;
  while (true) {
    HIPCHK(c, hipMemcpyAsync(c->done_host, (char*)c->ctl + CTL_OFF(done), r_off * 4 + 4,
                             hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (c->done_host[0]) {
      update_round_cap(c, c->done_host[r_off], num_leaves);
      break;
    }
    if (done_rounds > num_leaves + 2)
      return set_err(c, LGBM_HIP_ERR_RUNTIME, "tree driver did not complete");
    int rc = launch_tail(c, fp);
    if (rc) return rc;
    done_rounds += lgbm_hip_ctx::TAIL_ROUNDS;
    c->extra_rounds += lgbm_hip_ctx::TAIL_ROUNDS;
  }
  DevLearner L = make_learner(c);
  KernelEvents ke;
  launch_tree_finalize(L, c->stream, ev_kernel(c, -1, &ke));
  HIPCHK(c, hipGetLastError());
  return LGBM_HIP_OK;
}

// One tree from the current gradients: fp = 0 quantized (lgbm_hip_quantize ran), 1 f32
// (the packed pairs and fixed-point scales were prepared by launch_fp_prep).
int grow_tree_async(lgbm_hip_ctx* c, const lgbm_gain_config* cfg, int32_t num_leaves,
                    int32_t max_depth, int32_t fp) {
  int rc = ensure_leaves(c, num_leaves);
  if (rc) return rc;
  // Speculation width.  Where one job's scans are costly (features x cell width at
  // least PLAN_CAP_WORK) the speculative jobs a wider round adds cost more than the
  // rounds they save, and their node slots run out sooner: 2000 features with f32
  // cells measured 8.20 ms an iteration at 8 against 7.20 at 4 (7.19 at 3, 7.59 at 5),
  // while 700 quantized features are fastest at 8.
  if (!c->spec_env)
    c->spec_max = c->F * (fp ? 2 : 1) >= PLAN_CAP_WORK ? SPEC_SCAN_HEAVY : SPEC_DEFAULT;
  if (c->colsamp_on) {
    // this tree's column sample (BeforeTrain's ResetByTree); the pinned copy is not
    // rewritten before this tree completes (every tree ends with a stream wait)
    c->colsamp.next_tree();
    std::memcpy(c->feat_used_host, c->colsamp.used.data(), (size_t)c->F);
    HIPCHK(c, hipMemcpyAsync(c->d_feat_used, c->feat_used_host, (size_t)c->F,
                             hipMemcpyHostToDevice, c->stream));
  }
  HIPCHK(c, hipMemcpyAsync((char*)c->ctl + CTL_OFF(cfg), cfg, sizeof(*cfg), hipMemcpyHostToDevice,
                           c->stream));
  const int32_t rounds = std::max(1, std::min(c->round_cap, num_leaves + 1));
  if (c->timing || !c->use_graphs) {
    enqueue_tree(c, num_leaves, max_depth, rounds, fp);
    HIPCHK(c, hipGetLastError());
    return finish_rounds(c, num_leaves, rounds, fp);
  }
  if (!(c->graph_nl == num_leaves && c->graph_md == max_depth && c->graph_gen == c->buf_gen &&
        c->graph_spec == c->spec_max && c->graph_fp == fp)) {
    drop_graphs(c);  // another tree shape: every cached sequence is stale
    c->graph_nl = num_leaves;
    c->graph_md = max_depth;
    c->graph_gen = c->buf_gen;
    c->graph_spec = c->spec_max;
    c->graph_fp = fp;
  }
  constexpr int GC = lgbm_hip_ctx::GRAPH_CACHE;
  int slot = -1;
  for (int i = 0; i < GC; ++i)
    if (c->graph_exec[i] && c->graph_rounds[i] == rounds) slot = i;
  if (slot < 0) {
    slot = 0;  // a free entry, else the least recently used
    for (int i = 0; i < GC; ++i) {
      if (!c->graph_exec[i]) {
        slot = i;
        break;
      }
      if (c->graph_used[i] < c->graph_used[slot]) slot = i;
    }
    if (c->graph_exec[slot]) (void)hipGraphExecDestroy(c->graph_exec[slot]);
    c->graph_exec[slot] = nullptr;
    hipGraph_t g = nullptr;
    HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    enqueue_tree(c, num_leaves, max_depth, rounds, fp);
    HIPCHK(c, hipStreamEndCapture(c->stream, &g));
    hipError_t e = hipGraphInstantiate(&c->graph_exec[slot], g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
      c->graph_exec[slot] = nullptr;
      return set_err(c, LGBM_HIP_ERR_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
    }
    c->graph_rounds[slot] = rounds;
  }
  c->graph_used[slot] = ++c->graph_clock;
  HIPCHK(c, hipGraphLaunch(c->graph_exec[slot], c->stream));
  return finish_rounds(c, num_leaves, rounds, fp);
}

// cat_threshold words a tree of num_leaves leaves may need: every internal node
// categorical with the widest bitset.
int64_t cat_words_needed(const lgbm_hip_ctx* c, int32_t num_leaves) {
  return c->cat_words_node * (int64_t)std::max(num_leaves - 1, 0);
}
// Refuses, before any work is enqueued, a tree output whose categorical arrays could
// not hold the tree (a later refusal would come after the score update).
int check_cat_capacity(lgbm_hip_ctx* c, const lgbm_tree_out* out, int32_t num_leaves) {
  if (!out || c->cat_words_node == 0) return LGBM_HIP_OK;
  const int64_t need = cat_words_needed(c, num_leaves);
  if (!out->cat_boundaries || !out->cat_threshold || (int64_t)out->cat_threshold_cap < need)
    return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH,
                   "categorical features: cat_threshold needs capacity for " + std::to_string(need) +
                       " words (lgbm_hip_cat_threshold_words), got " +
                       std::to_string(out->cat_threshold_cap));
  return LGBM_HIP_OK;
}

// `copied`: the caller has enqueued the blob copy and waited for it (the stream may
// still be busy with later work).
int finish_tree(lgbm_hip_ctx* c, lgbm_tree_out* out, lgbm_layout_out* layout, double shrink,
                bool copied = false) {
  if (!copied) {
    HIPCHK(c, hipMemcpyAsync(c->tree_host, c->tree_blob, out ? c->tree_blob_bytes : 64,
                             hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    ev_collect(c);
  }
  const char* hb = (const char*)c->tree_host;
  const int32_t nl = ((const int32_t*)hb)[0], err = ((const int32_t*)hb)[1];
  c->tree_rounds += ((const int32_t*)hb)[2];
  c->trees += 1.0;
  int rc = 0;
  if (err & ERR_ROOT_HESSIAN)
    return set_err(c, LGBM_HIP_ERR_INVALID_LEAF_HESSIAN, "root sum_hessian <= 0");
  if (err & ERR_NEG_HESSIAN)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT,
                   "quantized gradients need non-negative hessians");
  if (err & ERR_SLOTS) return set_err(c, LGBM_HIP_ERR_RUNTIME, "node slot budget exhausted");
  if (err) return set_err(c, LGBM_HIP_ERR_RUNTIME, "device learner error");
  if (out) {
    out->num_leaves = nl;
    const size_t ni = (size_t)std::max(nl - 1, 0), nl_ = (size_t)nl;
    auto cp = [&](void* dst, int idx, size_t bytes) {
      if (dst && bytes) std::memcpy(dst, hb + c->tree_off[idx], bytes);
    };
    cp(out->split_feature, 1, ni * 4);
    cp(out->threshold_in_bin, 2, ni * 4);
    cp(out->threshold, 3, ni * 8);
    cp(out->split_gain, 4, ni * 4);
    cp(out->decision_type, 5, ni);
    cp(out->left_child, 6, ni * 4);
    cp(out->right_child, 7, ni * 4);
    cp(out->internal_value, 8, ni * 8);
    cp(out->internal_count, 9, ni * 4);
    cp(out->leaf_value, 10, nl_ * 8);
    cp(out->leaf_weight, 11, nl_ * 8);
    cp(out->leaf_count, 12, nl_ * 4);
    cp(out->leaf_depth, 13, nl_ * 4);
    cp(out->leaf_parent, 14, nl_ * 4);
    cp(out->internal_weight, 15, ni * 8);
    // Categorical nodes (Tree::split_categorical, learner.rs:4104-4186): in node order
    // the k-th gets bitset index k as its threshold; its bitset is ConstructBitset over
    // the category values of the bins that went left.
    std::vector<int32_t> bounds{0};
    std::vector<uint32_t> words;
    const int8_t* dt = (const int8_t*)(hb + c->tree_off[5]);
    const int32_t* sf = (const int32_t*)(hb + c->tree_off[1]);
    const uint32_t* cl = (const uint32_t*)(hb + c->tree_off[16]);
    for (size_t n = 0; n < ni; ++n) {
      if (!(dt[n] & 1)) continue;
      const int32_t k = (int32_t)bounds.size() - 1;
      if (out->threshold_in_bin) out->threshold_in_bin[n] = (uint32_t)k;
      if (out->threshold) out->threshold[n] = (double)k;
      int32_t fpos = -1;
      for (int32_t f = 0; f < c->F; ++f)
        if (c->feats[(size_t)f].real_index == sf[n]) {
          fpos = f;
          break;
        }
      std::vector<uint32_t> bits;
      for (int32_t b = 0; b < 256; ++b) {
        if (!((cl[n * 8 + (size_t)(b >> 5)] >> (b & 31)) & 1u)) continue;
        const DevFeature& ft = c->feats[(size_t)std::max(fpos, 0)];
        const double v = fpos >= 0 && ft.ub_off + (size_t)b < c->ub_host.size()
                             ? c->ub_host[ft.ub_off + (size_t)b]
                             : (double)b;
        if (!(v >= 0.0 && v < 2147483648.0))  // the NaN dummy bin never wins a set
          return set_err(c, LGBM_HIP_ERR_RUNTIME, "a categorical split sent a negative category left");
        const uint32_t cat = (uint32_t)(int32_t)v;
        if (bits.size() <= cat / 32) bits.resize(cat / 32 + 1, 0u);
        bits[cat / 32] |= 1u << (cat % 32);
      }
      words.insert(words.end(), bits.begin(), bits.end());
      bounds.push_back((int32_t)words.size());
    }
    out->num_cat = (int32_t)bounds.size() - 1;
    if (out->num_cat > 0) {
      if (!out->cat_boundaries || !out->cat_threshold ||
          (int64_t)words.size() > (int64_t)out->cat_threshold_cap)
        return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH,
                       "categorical tree: cat_threshold needs " + std::to_string(words.size()) +
                           " words (cat_threshold_cap " + std::to_string(out->cat_threshold_cap) + ")");
      std::memcpy(out->cat_boundaries, bounds.data(), bounds.size() * 4);
      std::memcpy(out->cat_threshold, words.data(), words.size() * 4);
    }
    if (shrink != 1.0) {
      // Tree::shrinkage (tree.rs:1074): MaybeRoundToZero(v * rate)
      const double z = (double)1e-35f;
      auto mrz = [z](double v) { return (v >= -z && v <= z) ? 0.0 : v; };
      if (out->leaf_value)
        for (size_t i = 0; i < nl_; ++i) out->leaf_value[i] = mrz(out->leaf_value[i] * shrink);
      if (out->internal_value)
        for (size_t i = 0; i < ni; ++i) out->internal_value[i] = mrz(out->internal_value[i] * shrink);
    }
  }
  if (layout) {
    if (layout->indices) {
      if (c->indices_cap < c->N) {
        if ((rc = dalloc(c, &c->d_indices, (size_t)c->N))) return rc;
        c->indices_cap = c->N;
      }
      if ((rc = ensure_scratch_bytes(c, export_layout_scratch_bytes(c->N, nl)))) return rc;
      DevLearner L = make_learner(c);
      launch_export_layout(L, nl, c->d_indices, c->scratch, c->stream);
      HIPCHK(c, hipGetLastError());
      HIPCHK(c, hipStreamSynchronize(c->stream));
      HIPCHK(c, hipMemcpy(layout->indices, c->d_indices, (size_t)c->N * 4, hipMemcpyDeviceToHost));
    }
    if (layout->leaf_begin)
      HIPCHK(c, hipMemcpy(layout->leaf_begin, c->leaves.begin, (size_t)nl * 4,
                          hipMemcpyDeviceToHost));
    if (layout->leaf_count)
      HIPCHK(c, hipMemcpy(layout->leaf_count, c->leaves.count, (size_t)nl * 4,
                          hipMemcpyDeviceToHost));
  }
  return LGBM_HIP_OK;
}

DevFeature feature_from_batched(const lgbm_batched_feature& b) {
  DevFeature f{};
  f.num_bin = b.num_bin;
  f.offset = b.offset;
  f.default_bin = b.default_bin;
  f.mfb = b.most_freq_bin;
  f.slot_off = (uint32_t)b.slot_off;
  f.cell_base = (uint32_t)(b.slot_off / 2);
  f.skip_default_bin = b.skip_default_bin;
  f.na_as_missing = b.na_as_missing;
  f.run_forward = b.run_forward;
  f.penalty = 1.0;
  f.real_index = -1;
  return f;
}

}  // namespace

// Shared by the bin uploads: feature table, record and histogram buffers for a
// resident matrix of F features x N rows (the records themselves are written by the
// caller).
int resident_setup(lgbm_hip_ctx* c, int32_t F_in, int64_t num_data, const lgbm_feature_meta* meta,
                   const double* bin_upper_bound) {
  int rc = 0;
  const int32_t F = F_in;
  // Until the new layout is complete the context holds no usable resident state: a
  // failed allocation or copy below must not leave flags (or a captured graph)
  // pointing at buffers this call frees.
  c->have_bins = c->have_grad = c->quant_ready = c->have_labels = false;
  c->ahead = false;
  c->colsamp_on = false;
  c->have_rank = false;
  c->buf_gen++;
  drop_graphs(c);
  if (F > WIDE_MAX_F)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "more than " + std::to_string(WIDE_MAX_F) + " features");
  if (num_data >= (1ll << 31) - 1)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_data must fit data_size_t (i32)");
  std::vector<DevFeature> feats(F);
  uint32_t acc = 0, uacc = 0;
  for (int f = 0; f < F; ++f) {
    const lgbm_feature_meta& m = meta[f];
    if (m.num_bin == 0 || m.num_bin > WIDE_MAX_BIN)
      return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                     "num_bin must be in 1..=" + std::to_string(WIDE_MAX_BIN));
    if (m.bin_type == LGBM_BIN_CATEGORICAL && m.num_bin > 256)
      return set_err(c, LGBM_HIP_ERR_CAPABILITY, "categorical features hold at most 256 bins");
    DevFeature& d = feats[f];
    d.num_bin = m.num_bin;
    d.offset = m.offset;
    d.min_bin = m.min_bin;
    d.max_bin = m.max_bin;
    d.default_bin = m.default_bin;
    d.mfb = m.most_freq_bin;
    d.missing_type = m.missing_type;
    d.real_index = m.real_feature_index;
    d.slot_off = 2 * acc;
    d.cell_base = acc;
    d.ub_off = uacc;
    d.skip_default_bin = (m.num_bin > 2 && m.missing_type == LGBM_MISSING_ZERO) ? 1 : 0;
    d.na_as_missing = (m.num_bin > 2 && m.missing_type == LGBM_MISSING_NAN) ? 1 : 0;
    d.run_forward = (m.num_bin > 2 && m.missing_type != LGBM_MISSING_NONE) ? 1 : 0;
    d.penalty = 1.0;
    d.categorical = m.bin_type == LGBM_BIN_CATEGORICAL ? 1 : 0;
    if (d.categorical && !bin_upper_bound)
      return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT,
                     "categorical features need their bin -> category values in bin_upper_bound");
    acc += m.num_bin;
    uacc += m.num_bin;
  }
  // row layout: the wide one (row indices moved, bins in a fixed row-major matrix)
  // when the records cannot hold the features or the quantized builds' LDS cannot
  // hold the cells; else 6-bit bins with the quantized pair inside when every feature
  // has at most 64 bins and fits (F <= 39), else 8-bit bins and the row index
  uint32_t max_nb = 0;
  for (int f = 0; f < F; ++f) max_nb = std::max(max_nb, meta[f].num_bin);
  const bool bin16 = max_nb > 256;  // 2-byte bins: the wide layout only
  const bool wide =
      bin16 || c->records_env == 2 || F > 16 * LGBM_MAX_W - 4 || acc > QUANT_LDS_CELLS;
  if (!wide && acc > HIST_WAVE_CELLS && num_data > (int64_t)HIST_GRID_Q * HIST_BLOCK_MAX_ROWS)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "rows per histogram block exceed the packed LDS cell fields");
  if (wide && wide_prepare())
    return set_err(c, LGBM_HIP_ERR_HIP, "the wide histogram kernels' LDS size was refused");
  if (bin16 && (scan_prepare() || fixscan_prepare()))
    return set_err(c, LGBM_HIP_ERR_HIP, "the scans' LDS size was refused");
  c->F = F;
  c->N = num_data;
  c->max_bins = (int32_t)max_nb;
  c->has_cat = 0;
  for (int f = 0; f < F; ++f)
    if (meta[f].bin_type == LGBM_BIN_CATEGORICAL) c->has_cat = 1;
  c->bin16 = bin16;
  c->fmt = (F + 4 + 15) / 16;
  if (wide) {
    c->fmt = REC_FMT_WIDE;
  } else if (c->records_env != 1 && max_nb <= 64 && F <= 39) {
    int U = (F + 5) / 5;
    U = std::max(U + (U & 1), 2);
    c->fmt = REC_FMT_PACKED + U;
  }
  c->total_cells = (int32_t)acc;
  c->acc_cells = (int32_t)acc + (wide ? 1 : 0);
  c->slot_len = 2ull * acc;
  c->feats = feats;
  c->lcap = 0;  // slots depend on slot_len
  if ((rc = dalloc(c, &c->d_feats, (size_t)F))) return rc;
  HIPCHK(c, hipMemcpy(c->d_feats, feats.data(), F * sizeof(DevFeature), hipMemcpyHostToDevice));
  c->ub_host.assign(bin_upper_bound ? bin_upper_bound : nullptr,
                    bin_upper_bound ? bin_upper_bound + uacc : nullptr);
  // the widest bitset finish_tree can write for one categorical node (its category
  // values converted as there); a bin of negative category (the NaN dummy bin 0) is
  // never in a winning set (learner.rs:4120-4124)
  c->cat_words_node = 0;
  for (const DevFeature& d : c->feats) {
    if (!d.categorical) continue;
    for (uint32_t b = 0; b < d.num_bin; ++b) {
      const size_t k = d.ub_off + (size_t)b;
      const double v = k < c->ub_host.size() ? c->ub_host[k] : (double)b;
      if (!(v >= 0.0 && v < 2147483648.0)) continue;
      c->cat_words_node = std::max<int64_t>(c->cat_words_node, (int64_t)((uint32_t)(int32_t)v / 32) + 1);
    }
  }
  if (bin_upper_bound) {
    if ((rc = dalloc(c, &c->d_ub, (size_t)uacc))) return rc;
    HIPCHK(c, hipMemcpy(c->d_ub, bin_upper_bound, uacc * 8, hipMemcpyHostToDevice));
  } else if (c->d_ub) {
    (void)hipFree(c->d_ub);
    c->d_ub = nullptr;
  }
  const size_t words = rec_units(c->fmt, num_data);
  for (int b : {BUF_ORIG, BUF_A, BUF_B}) {
    if ((rc = dalloc(c, &c->rec[b], words))) return rc;
    if ((rc = dalloc(c, &c->gh[b], (size_t)num_data))) return rc;
    c->buf_rows[b] = num_data;
  }
  c->buf_rows[BUF_S0] = c->buf_rows[BUF_S1] = 0;
  if ((rc = dalloc(c, &c->g, (size_t)num_data))) return rc;
  if ((rc = dalloc(c, &c->h, (size_t)num_data))) return rc;
  // the record layouts' partial slots (the wide layout builds into the accumulators)
  const size_t pc = wide ? 1 : acc;
  if ((rc = dalloc(c, &c->hist_part, (size_t)HIST_SLOTS * pc * 3))) return rc;
  if ((rc = dalloc(c, &c->hist_sum, (size_t)acc * 3))) return rc;
  if ((rc = dalloc(c, &c->hist_part64, (size_t)HIST_SLOTS * pc * 2))) return rc;
  if (wide) {
    // row stride in bytes: F rounded up to a 64-feature group, times the bin width
    c->row_stride = ((int64_t)F + WIDE_GF_Q - 1) / WIDE_GF_Q * WIDE_GF_Q * (bin16 ? 2 : 1);
    if ((rc = dalloc(c, &c->binmat, (size_t)num_data * (size_t)c->row_stride))) return rc;
    // the feature-major copy is optional: without it the router reads binmat rows
    if (c->bincol) (void)hipFree(c->bincol);
    c->bincol = nullptr;
    if (c->no_bincol ||
        hipMalloc((void**)&c->bincol, (size_t)num_data * (size_t)F * (bin16 ? 2 : 1)) !=
            hipSuccess) {
      c->bincol = nullptr;
      (void)hipGetLastError();
    }
    // 2-byte bins: feature groups of at most WIDE16_GROUP_F consecutive features whose
    // cells fit WIDE16_GROUP_CELLS
    std::vector<int32_t> groups(1, 0);
    uint32_t gc = 0;
    for (int f = 0; f < F; ++f) {
      const int32_t nf = f - groups.back();
      if (nf > 0 && (nf >= WIDE16_GROUP_F || gc + meta[f].num_bin > WIDE16_GROUP_CELLS)) {
        groups.push_back(f);
        gc = 0;
      }
      gc += meta[f].num_bin;
    }
    groups.push_back(F);
    c->n_wgroups = (int32_t)groups.size() - 1;
    if ((rc = dalloc(c, &c->d_wgroups, groups.size()))) return rc;
    HIPCHK(c, hipMemcpy(c->d_wgroups, groups.data(), groups.size() * 4, hipMemcpyHostToDevice));
    if ((rc = dalloc(c, &c->hist_acc64, (size_t)SPEC_MAX * c->acc_cells * 2))) return rc;
    HIPCHK(c, hipMemset(c->hist_acc64, 0, (size_t)SPEC_MAX * c->acc_cells * 2 * 8));
    if ((rc = dalloc(c, &c->wide_part,
                     wide_part_words(F, num_data, (int32_t)acc, bin16 ? c->n_wgroups : 0))))
      return rc;
  } else {
    c->row_stride = 0;
    if (c->binmat) (void)hipFree(c->binmat);
    if (c->bincol) (void)hipFree(c->bincol);
    if (c->hist_acc64) (void)hipFree(c->hist_acc64);
    if (c->wide_part) (void)hipFree(c->wide_part);
    c->binmat = nullptr;
    c->bincol = nullptr;
    c->hist_acc64 = nullptr;
    c->wide_part = nullptr;
    if (acc > (uint32_t)(MAX_FGROUPS - 1) * (HIST_FP_CELLS - 256))
      return set_err(c, LGBM_HIP_ERR_CAPABILITY, "too many histogram cells for the f32 feature groups");
  }
  // feature groups of the record layouts' f32 histogram kernel: consecutive features
  // whose cells fit one block's LDS (at most MAX_FGROUPS: the cell check above)
  c->n_fgroups = 0;
  if (!wide) {
    int32_t ng = 0;
    uint32_t gcells = 0;
    c->fgroup_first[0] = 0;
    for (int f = 0; f < F; ++f) {
      if (f > 0 && gcells + feats[f].num_bin > HIST_FP_CELLS) {
        if (ng + 1 >= MAX_FGROUPS)
          return set_err(c, LGBM_HIP_ERR_CAPABILITY, "too many f32 feature groups");
        c->fgroup_first[++ng] = f;
        gcells = 0;
      }
      gcells += feats[f].num_bin;
    }
    c->fgroup_first[++ng] = F;
    c->n_fgroups = ng;
  }
  if ((rc = dalloc(c, &c->hist_acc, (size_t)SPEC_MAX * c->acc_cells * 3))) return rc;
  HIPCHK(c, hipMemset(c->hist_acc, 0, (size_t)SPEC_MAX * c->acc_cells * 3 * 4));
  if ((rc = dalloc(c, &c->hist_accp, (size_t)SPEC_MAX * c->acc_cells))) return rc;
  HIPCHK(c, hipMemset(c->hist_accp, 0, (size_t)SPEC_MAX * c->acc_cells * 8));
  if ((rc = dalloc(c, &c->part_slots, ((size_t)c->part_blocks + SPEC_MAX) * pc))) return rc;
  if ((rc = ensure_tile_state(c, num_data))) return rc;
  return LGBM_HIP_OK;
}

// BinaryLogloss::get_gradients on the resident score, then the f32 pair prep or the
// quantizer with iteration `iter`'s seed (gbdt.rs:945-960).
void enqueue_objective(lgbm_hip_ctx* c, int32_t objective, int32_t iter, int32_t qbins,
                       int32_t stochastic) {
  ev_begin(c, FAM_OBJ);
  if (objective == LGBM_HIP_OBJECTIVE_BINARY) {
    launch_grad_binary(c->score, c->label, c->g, c->h, c->N, c->partials, c->stream);
  } else {
    if (objective == LGBM_HIP_OBJECTIVE_REGRESSION)
      launch_grad_l2(c->score, c->label, c->g, c->h, c->N, c->stream);
    else
      launch_grad_lambdarank(c->score, c->label, c->rank, c->g, c->h, c->stream);
    if (qbins) launch_absmax(c->g, c->h, c->N, c->partials, c->stream);  // quantizer statistics
  }
  ev_end(c);
  c->have_grad = true;
  if (qbins == 0) {
    ev_begin(c, FAM_QUANT);
    DevLearner L0 = make_learner(c);
    launch_fp_prep(L0, c->g, c->h, c->N, c->partials, c->stream);
    ev_end(c);
    c->quant_ready = false;
  } else {
    const uint64_t seed = ((uint64_t)(uint32_t)iter << 20) ^ 0ull ^ 0x51702010ull;  // gbdt.rs:950
    const bool gen = gen_bins(qbins);  // the caller allocated c->dq
    ev_begin(c, FAM_QUANT);
    launch_quant_scales(c->ctl, c->partials, c->N, qbins, -1, c->stream);
    launch_quantize(c->g, c->h, c->N, c->ctl, c->wave_mats, c->lane_mats,
                    seed ^ 0x9E3779B97F4A7C15ull, stochastic, c->gh[BUF_ORIG],
                    gen ? c->dq : nullptr, gen ? c->dq + c->N : nullptr, c->stream);
    if (gen) {
      DevLearner L0 = make_learner(c);
      launch_exact_prep(L0, c->dq, c->dq + c->N, c->N, c->stream);
    }
    ev_end(c);
    c->quant_ready = true;
    c->quant_bins = qbins;
  }
}

BinParams bin_params_of(const lgbm_bin_params& p) {
  BinParams b;
  b.max_bin = p.max_bin;
  b.min_data_in_bin = p.min_data_in_bin;
  b.pre_filter = p.pre_filter != 0;
  b.use_missing = p.use_missing != 0;
  b.zero_as_missing = p.zero_as_missing != 0;
  return b;
}

int resident_done(lgbm_hip_ctx* c) {
  c->have_bins = true;
  c->have_grad = c->quant_ready = c->have_labels = false;
  c->buf_gen++;
  return LGBM_HIP_OK;
}

extern "C" {

int lgbm_hip_ctx_create(int device, lgbm_hip_ctx** out) {
  if (!out) return set_err(nullptr, LGBM_HIP_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return set_err(nullptr, LGBM_HIP_ERR_CAPABILITY, "no HIP device available");
  if (device < 0 || device >= n)
    return set_err(nullptr, LGBM_HIP_ERR_INVALID_ARGUMENT, "device index out of range");
  lgbm_hip_ctx* c = new lgbm_hip_ctx();
  c->device = device;
  auto fail = [&](int rc) {
    g_create_err = c->err;
    lgbm_hip_ctx_destroy(c);
    return rc;
  };
  if (hipSetDevice(device) != hipSuccess) return fail(set_err(c, LGBM_HIP_ERR_HIP, "hipSetDevice"));
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess)
    return fail(set_err(c, LGBM_HIP_ERR_HIP, "hipStreamCreate"));
  if (hipEventCreateWithFlags(&c->tree_ev, hipEventDisableTiming) != hipSuccess)
    return fail(set_err(c, LGBM_HIP_ERR_HIP, "hipEventCreate"));
  int rc = dalloc(c, &c->ctl, 1);
  if (rc) return fail(rc);
  Ctl init;
  std::memset(&init, 0, sizeof(init));
  if (hipMemcpy(c->ctl, &init, sizeof(init), hipMemcpyHostToDevice) != hipSuccess)
    return fail(set_err(c, LGBM_HIP_ERR_HIP, "ctl init"));
  if ((rc = dalloc(c, &c->stats, 8))) return fail(rc);
  if (hipMemset(c->stats, 0, 64) != hipSuccess) return fail(set_err(c, LGBM_HIP_ERR_HIP, "stats"));
  if (hipHostMalloc((void**)&c->done_host, 64, hipHostMallocDefault) != hipSuccess)
    return fail(set_err(c, LGBM_HIP_ERR_HIP, "hipHostMalloc"));
  if ((rc = init_jump_tables(c))) return fail(rc);
  if (noalloc_scratch_ptr(device, &c->noalloc) != 0)
    return fail(set_err(c, LGBM_HIP_ERR_HIP, "hipGetSymbolAddress(scratch) failed"));
  if ((rc = dalloc(c, &c->partials, STAT_BLOCKS))) return fail(rc);
  if ((rc = dalloc(c, &c->d_flags, 2))) return fail(rc);
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess &&
      cus > 0)
    c->part_blocks = cus * PART_BLOCKS_PER_CU;
  if (const char* e = std::getenv("LGBM_HIP_PART_BLOCKS"))
    c->part_blocks = std::max(1, std::min(65535, std::atoi(e)));
  if (const char* e = std::getenv("LGBM_HIP_GRAPHS")) c->use_graphs = std::strcmp(e, "0") != 0;
  if (const char* e = std::getenv("LGBM_HIP_RECORDS"))
    c->records_env = std::strcmp(e, "legacy") == 0 ? 1 : std::strcmp(e, "wide") == 0 ? 2 : 0;
  if (const char* e = std::getenv("LGBM_HIP_ROUNDS")) {
    c->round_cap = std::max(1, std::atoi(e));
    c->round_fixed = true;
  }
  if (const char* e = std::getenv("LGBM_HIP_SPEC")) {
    c->spec_max = std::max(1, std::min(SPEC_MAX, std::atoi(e)));
    c->spec_env = true;
  }
  if (const char* e = std::getenv("LGBM_HIP_BINCOL")) c->no_bincol = std::strcmp(e, "0") == 0;
  *out = c;
  return LGBM_HIP_OK;
}

int lgbm_hip_ctx_destroy(lgbm_hip_ctx* c) {
  if (!c) return LGBM_HIP_OK;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  drop_graphs(c);
  auto F = [](void* p) {
    if (p) (void)hipFree(p);
  };
  F(c->ctl);
  F(c->d_feats);
  F(c->d_ub);
  for (int i = 0; i < NBUF; ++i) {
    F(c->rec[i]);
    F(c->gh[i]);
    F(c->g32[i]);
  }
  F(c->g);
  F(c->h);
  F(c->label);
  F(c->score);
  F(c->gk);
  F(c->hk);
  F(c->hist_part);
  F(c->hist_sum);
  F(c->hist_acc);
  F(c->hist_accp);
  F(c->hist_acc64);
  F(c->wide_part);
  F(c->d_wgroups);
  F(c->binmat);
  F(c->bincol);
  F(c->rk_qb);
  F(c->rk_imd);
  F(c->rk_table);
  F(c->rk_disc);
  F(c->rk_gain);
  F(c->d_feat_used);
  if (c->feat_used_host) (void)hipHostFree(c->feat_used_host);
  F(c->cat_bits);
  F(c->part_slots);
  F(c->hist_part64);
  F(c->int_slots64);
  F(c->tile_state);
  F(c->wave_mats);
  F(c->lane_mats);
  F(c->stats);
  F(c->partials);
  F(c->d_flags);
  F(c->best_fpos);
  F(c->int_slots);
  F(c->tree_blob);
  if (c->tree_host) (void)hipHostFree(c->tree_host);
  F(c->slots);
  F(c->feat_split);
  F(c->gain_dense);
  F(c->mfbv);
  F(c->fmat);
  F(c->best);
  F(c->splittable);
  F(c->plan_state);
  F(c->nodes.begin);
  F(c->nodes.count);
  F(c->nodes.buf);
  F(c->nodes.rev);
  F(c->nodes.depth);
  F(c->nodes.child);
  F(c->nodes.sums);
  F(c->nodes.key_gain);
  F(c->nodes.key_feat);
  if (c->done_host) (void)hipHostFree(c->done_host);
  F(c->leaves.begin);
  F(c->leaves.count);
  F(c->leaves.buf);
  F(c->leaves.rev);
  F(c->pm_nodes);
  F(c->pm_trees);
  F(c->pm_leaves);
  F(c->pm_catb);
  F(c->pm_catw);
  F(c->pm_linl);
  F(c->pm_linf);
  F(c->pm_linc);
  F(c->pm_ncov);
  F(c->pm_lcov);
  F(c->pm_expv);
  F(c->pm_shap);
  F(c->pm_csr);
  F(c->pm_x);
  F(c->pm_out);
  DevTree& T = c->tree;
  F(T.nodes);
  F(T.route_mask);
  F(T.route_node);
  F(c->scratch);
  F(c->slot_tmp);
  F(c->res_slots);
  F(c->renew_idx);
  F(c->renew_scratch);
  F(c->dq);
  F(c->d_indices);
  for (auto& p : c->ev_pool) {
    (void)hipEventDestroy(p.a);
    (void)hipEventDestroy(p.b);
  }
  for (hipEvent_t e : c->chain) (void)hipEventDestroy(e);
  if (c->tree_ev) (void)hipEventDestroy(c->tree_ev);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  delete c;
  return LGBM_HIP_OK;
}

int lgbm_hip_last_error(const lgbm_hip_ctx* c, char* buf, size_t size) {
  if (!buf || size == 0) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  const std::string& s = c ? c->err : g_create_err;
  std::snprintf(buf, size, "%s", s.c_str());
  return LGBM_HIP_OK;
}

int lgbm_hip_upload_bins(lgbm_hip_ctx* c, const uint8_t* bins, int32_t num_features,
                         int64_t num_data, const lgbm_feature_meta* meta,
                         const double* bin_upper_bound) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!bins || !meta || num_features <= 0 || num_data <= 0)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null bins/meta or empty shape");
  const int32_t F = num_features;
  for (int f = 0; f < F; ++f)
    if (meta[f].num_bin == 0 || meta[f].num_bin > 256)
      return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_bin must be in 1..=256 (u8 bin storage)");
  // bin-range gate (learner.rs:1161-1187): first offending bin, feature order
  for (int f = 0; f < F; ++f) {
    const uint8_t* col = bins + (size_t)f * (size_t)num_data;
    const uint32_t nb = meta[f].num_bin;
    if (nb >= 256) continue;
    for (int64_t r = 0; r < num_data; ++r)
      if (col[r] >= nb)
        return set_err(c, LGBM_HIP_ERR_BIN_OUT_OF_RANGE,
                       "bin " + std::to_string(col[r]) + " >= num_bin " + std::to_string(nb) +
                           " (feature " + std::to_string(f) + ", row " + std::to_string(r) + ")");
  }
  if ((rc = resident_setup(c, F, num_data, meta, bin_upper_bound))) return rc;
  // transpose the feature-major upload into records
  uint8_t* tmp = nullptr;
  HIPCHK(c, hipMalloc((void**)&tmp, (size_t)F * num_data));
  hipError_t e = hipMemcpy(tmp, bins, (size_t)F * num_data, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    if (rec_wide(c->fmt)) {
      launch_pack_wide(tmp, num_data, F, c->row_stride, c->binmat, c->rec[BUF_ORIG], c->stream);
      launch_wide_cols(c->binmat, num_data, F, c->row_stride, 0, c->bincol, c->stream);
    } else {
      launch_pack_records(tmp, num_data, F, c->fmt, c->rec[BUF_ORIG], c->stream);
    }
    e = hipStreamSynchronize(c->stream);
  }
  (void)hipFree(tmp);
  if (e != hipSuccess) return set_err(c, LGBM_HIP_ERR_HIP, hipGetErrorString(e));
  return resident_done(c);
}

// ---- binning ------------------------------------------------------------------

int lgbm_hip_bin_mapper_from_column(const double* column, int64_t num_rows,
                                    const lgbm_bin_params* p, const double* forced_upper_bounds,
                                    int32_t num_forced, lgbm_hip_bin_mapper** out) {
  if (!out || !p || (num_rows > 0 && !column) || num_rows < 0 || num_rows >= (1ll << 31) ||
      num_forced < 0 || (num_forced > 0 && !forced_upper_bounds)) {
    g_bin_err = "null argument, negative size or more than 2^31-1 rows";
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  if (p->max_bin < 2 || p->bin_construct_sample_cnt < 1) {
    g_bin_err = "max_bin must be >= 2 and bin_construct_sample_cnt >= 1";
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  // BinMapper::find_bin_from_column (bin_mapper.rs:613-651): sample, scale the
  // pre-filter threshold, then the numeric FindBin
  const int32_t n = (int32_t)num_rows;
  const std::vector<int32_t> idx = bin_sample_indices(n, p->bin_construct_sample_cnt,
                                                      p->data_random_seed);
  std::vector<double> sample(idx.size());
  for (size_t i = 0; i < idx.size(); ++i) sample[i] = column[idx[i]];
  BinParams bp = bin_params_of(*p);
  bp.min_split_data = bin_scaled_filter_cnt(p->min_data_in_leaf, (int32_t)sample.size(), n);
  const int64_t total = (int64_t)sample.size();
  *out = new lgbm_hip_bin_mapper(find_bin_numeric(
      std::move(sample), bp, total,
      std::vector<double>(forced_upper_bounds, forced_upper_bounds + num_forced)));
  return LGBM_HIP_OK;
}

int lgbm_hip_bin_mapper_from_sample(const double* values, int64_t num_values,
                                    int64_t total_sample_cnt, int32_t categorical,
                                    const lgbm_bin_params* p, int32_t min_split_data,
                                    const double* forced_upper_bounds, int32_t num_forced,
                                    lgbm_hip_bin_mapper** out) {
  if (!out || !p || (num_values > 0 && !values) || num_values < 0 ||
      total_sample_cnt < num_values || total_sample_cnt >= (1ll << 31) || num_forced < 0 ||
      (num_forced > 0 && !forced_upper_bounds)) {
    g_bin_err = "null argument, or total_sample_cnt outside [num_values, 2^31)";
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  if (p->max_bin < 2) {
    g_bin_err = "max_bin must be >= 2";
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  BinParams bp = bin_params_of(*p);
  bp.min_split_data = min_split_data;
  std::vector<double> v(values, values + num_values);
  if (categorical)
    *out = new lgbm_hip_bin_mapper(find_bin_categorical(std::move(v), bp, total_sample_cnt));
  else
    *out = new lgbm_hip_bin_mapper(find_bin_numeric(
        std::move(v), bp, total_sample_cnt,
        std::vector<double>(forced_upper_bounds, forced_upper_bounds + num_forced)));
  return LGBM_HIP_OK;
}

int lgbm_hip_bin_mapper_free(lgbm_hip_bin_mapper* m) {
  delete m;
  return LGBM_HIP_OK;
}

int lgbm_hip_bin_last_error(char* buf, size_t size) {
  if (buf && size > 0) std::snprintf(buf, size, "%s", g_bin_err.c_str());
  return LGBM_HIP_OK;
}

int lgbm_hip_bin_mapper_info(const lgbm_hip_bin_mapper* m, lgbm_bin_mapper_info* out) {
  if (!m || !out) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  out->num_bin = m->num_bin;
  out->missing_type = m->missing_type;
  out->bin_type = m->bin_type;
  out->is_trivial = m->is_trivial ? 1 : 0;
  out->default_bin = m->default_bin;
  out->most_freq_bin = m->most_freq_bin;
  out->sparse_rate = m->sparse_rate;
  out->min_val = m->min_val;
  out->max_val = m->max_val;
  return LGBM_HIP_OK;
}

int lgbm_hip_bin_mapper_bounds(const lgbm_hip_bin_mapper* m, double* upper, int32_t* categories) {
  if (!m) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  for (int32_t b = 0; b < m->num_bin; ++b) {
    if (upper) upper[b] = m->bin_type == LGBM_BIN_NUMERICAL ? m->upper[(size_t)b] : 0.0;
    if (categories)
      categories[b] = m->bin_type == LGBM_BIN_CATEGORICAL && (size_t)b < m->bin_to_cat.size()
                          ? m->bin_to_cat[(size_t)b]
                          : 0;
  }
  return LGBM_HIP_OK;
}

int lgbm_hip_bin_mapper_value_to_bin(const lgbm_hip_bin_mapper* m, const double* values,
                                     int64_t n, uint32_t* out) {
  if (!m || n < 0 || (n > 0 && (!values || !out))) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  for (int64_t i = 0; i < n; ++i) out[i] = m->value_to_bin(values[i]);
  return LGBM_HIP_OK;
}

int lgbm_hip_sample_indices(int32_t num_rows, int32_t sample_cnt, int32_t seed, int32_t* out,
                            int32_t* out_len) {
  if (!out_len || num_rows < 0) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  const std::vector<int32_t> idx = bin_sample_indices(num_rows, sample_cnt, seed);
  *out_len = (int32_t)idx.size();
  if (out && !idx.empty()) std::memcpy(out, idx.data(), idx.size() * 4);
  return LGBM_HIP_OK;
}

int lgbm_hip_upload_raw_device(lgbm_hip_ctx* c, const void* d_values, int32_t dtype,
                               int32_t col_major, int64_t num_rows, int32_t num_cols,
                               const lgbm_hip_bin_mapper* const* mappers) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!d_values || !mappers || num_rows <= 0 || num_cols <= 0)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null values/mappers or empty shape");
  if (dtype != LGBM_HIP_DTYPE_F32 && dtype != LGBM_HIP_DTYPE_F64)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "dtype must be F32 or F64");
  const int32_t F = num_cols;
  // feature columns (booster.rs:449-520): one single-feature group per mapper
  std::vector<lgbm_feature_meta> meta((size_t)F);
  std::vector<DevBinFeature> bf((size_t)F);
  std::vector<double> ub;
  std::vector<int2> cats;
  for (int32_t f = 0; f < F; ++f) {
    const lgbm_hip_bin_mapper* m = mappers[f];
    if (!m) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null mapper");
    if (m->num_bin < 1 || m->num_bin > WIDE_MAX_BIN)
      return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                     "num_bin must be in 1..=" + std::to_string(WIDE_MAX_BIN));
    const bool cat = m->bin_type == LGBM_BIN_CATEGORICAL;
    lgbm_feature_meta& d = meta[(size_t)f];
    d.num_bin = (uint32_t)m->num_bin;
    d.offset = m->most_freq_bin == 0 ? 1 : 0;  // offset_for_most_freq_bin (lib.rs:89-95)
    d.min_bin = 0;
    d.max_bin = (uint32_t)m->num_bin - 1;
    d.default_bin = m->default_bin;
    d.most_freq_bin = m->most_freq_bin;
    d.missing_type = m->missing_type;
    d.real_feature_index = f;
    d.bin_type = cat ? LGBM_BIN_CATEGORICAL : LGBM_BIN_NUMERICAL;
    DevBinFeature& b = bf[(size_t)f];
    b = DevBinFeature{};
    b.ub_pos = (int32_t)ub.size();
    if (cat) {
      // ValueToBin of a categorical mapper: the (category, bin) pairs sorted by
      // category; the feature's per-bin values are its categories (bin 0: -1)
      b.categorical = 1;
      b.off = (int32_t)cats.size();
      std::vector<std::pair<int32_t, uint32_t>> pairs(m->cat_to_bin.begin(), m->cat_to_bin.end());
      std::sort(pairs.begin(), pairs.end());
      for (const auto& pr : pairs) cats.push_back(make_int2(pr.first, (int32_t)pr.second));
      b.ncat = (int32_t)pairs.size();
      for (int32_t k = 0; k < m->num_bin; ++k)
        ub.push_back((size_t)k < m->bin_to_cat.size() ? (double)m->bin_to_cat[(size_t)k] : -1.0);
      continue;
    }
    b.categorical = 0;
    b.nan_bin = m->missing_type == BIN_MISSING_NAN ? m->num_bin - 1 : -1;
    b.last = m->num_bin - 1 - (b.nan_bin >= 0 ? 1 : 0);
    b.off = (int32_t)ub.size();
    ub.insert(ub.end(), m->upper.begin(), m->upper.end());
  }
  cats.push_back(make_int2(0, 0));  // keeps the table non-empty
  if ((rc = resident_setup(c, F, num_rows, meta.data(), ub.data()))) return rc;
  DevBinFeature* d_bf = nullptr;
  int2* d_cats = nullptr;
  hipError_t e = hipMalloc((void**)&d_bf, bf.size() * sizeof(DevBinFeature));
  if (e == hipSuccess) e = hipMalloc((void**)&d_cats, cats.size() * sizeof(int2));
  if (e == hipSuccess)
    e = hipMemcpy(d_bf, bf.data(), bf.size() * sizeof(DevBinFeature), hipMemcpyHostToDevice);
  if (e == hipSuccess)
    e = hipMemcpy(d_cats, cats.data(), cats.size() * sizeof(int2), hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    // c->d_ub holds the same bounds, concatenated in feature order
    KernelEvents ke;
    if (rec_wide(c->fmt)) {
      launch_bin_wide(d_values, dtype == LGBM_HIP_DTYPE_F64, col_major, num_rows, F, c->row_stride,
                      d_bf, c->d_ub, d_cats, c->binmat, c->rec[BUF_ORIG], c->bin16 ? 1 : 0,
                      c->stream, ev_kernel(c, FAM_BIN, &ke));
      launch_wide_cols(c->binmat, num_rows, F, c->row_stride, c->bin16 ? 1 : 0, c->bincol,
                       c->stream);
    } else
      launch_bin_records(d_values, dtype == LGBM_HIP_DTYPE_F64, col_major, num_rows, F, c->fmt,
                         d_bf, c->d_ub, (int32_t)ub.size(), d_cats, c->rec[BUF_ORIG], c->stream,
                         ev_kernel(c, FAM_BIN, &ke));
    if (c->timing) {
      c->bin_launches += 1.0;
      c->bin_values += (double)num_rows * F;
    }
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  }
  (void)hipFree(d_bf);
  (void)hipFree(d_cats);
  if (e != hipSuccess) return set_err(c, LGBM_HIP_ERR_HIP, hipGetErrorString(e));
  return resident_done(c);
}

int lgbm_hip_upload_raw(lgbm_hip_ctx* c, const void* values, int32_t dtype, int32_t col_major,
                        int64_t num_rows, int32_t num_cols,
                        const lgbm_hip_bin_mapper* const* mappers) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!values || num_rows <= 0 || num_cols <= 0)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null values or empty shape");
  const size_t bytes = (size_t)num_rows * (size_t)num_cols * (dtype == LGBM_HIP_DTYPE_F64 ? 8 : 4);
  void* tmp = nullptr;
  HIPCHK(c, hipMalloc(&tmp, bytes));
  hipError_t e = hipMemcpy(tmp, values, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(tmp);
    return set_err(c, LGBM_HIP_ERR_HIP, hipGetErrorString(e));
  }
  rc = lgbm_hip_upload_raw_device(c, tmp, dtype, col_major, num_rows, num_cols, mappers);
  (void)hipFree(tmp);
  return rc;
}

int lgbm_hip_get_bins(lgbm_hip_ctx* c, uint8_t* out, int64_t n) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "no resident bins");
  if (!out || n != c->N) return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "n != num_data");
  if (c->bin16)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "the resident bins are 2-byte: lgbm_hip_get_bins16");
  if (rec_wide(c->fmt)) {
    const size_t st = (size_t)c->row_stride;
    std::vector<uint8_t> m((size_t)c->N * st);
    HIPCHK(c, hipMemcpy(m.data(), c->binmat, m.size(), hipMemcpyDeviceToHost));
    for (int32_t f = 0; f < c->F; ++f)
      for (int64_t r = 0; r < c->N; ++r) out[(size_t)f * c->N + r] = m[(size_t)r * st + f];
    return LGBM_HIP_OK;
  }
  // the original (unpartitioned) records, feature-major
  const int U = rec_words(c->fmt);
  const uint32_t mask = (1u << rec_bits(c->fmt)) - 1u;
  std::vector<uint32_t> rec((size_t)c->N * U);
  HIPCHK(c, hipMemcpy(rec.data(), c->rec[BUF_ORIG], rec.size() * 4, hipMemcpyDeviceToHost));
  for (int32_t f = 0; f < c->F; ++f) {
    int wi, sh;
    rec_field_pos(c->fmt, f, &wi, &sh);
    for (int64_t r = 0; r < c->N; ++r)
      out[(size_t)f * c->N + r] = (uint8_t)((rec[(size_t)r * U + wi] >> sh) & mask);
  }
  return LGBM_HIP_OK;
}

int lgbm_hip_get_bins16(lgbm_hip_ctx* c, uint16_t* out, int64_t n) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "no resident bins");
  if (!out || n != c->N) return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "n != num_data");
  if (!c->bin16) {
    std::vector<uint8_t> b8((size_t)c->F * (size_t)c->N);
    if ((rc = lgbm_hip_get_bins(c, b8.data(), n))) return rc;
    for (size_t i = 0; i < b8.size(); ++i) out[i] = b8[i];
    return LGBM_HIP_OK;
  }
  const size_t st = (size_t)c->row_stride;
  std::vector<uint8_t> m((size_t)c->N * st);
  HIPCHK(c, hipMemcpy(m.data(), c->binmat, m.size(), hipMemcpyDeviceToHost));
  for (int32_t f = 0; f < c->F; ++f)
    for (int64_t r = 0; r < c->N; ++r) {
      uint16_t v;
      std::memcpy(&v, m.data() + (size_t)r * st + 2 * (size_t)f, 2);
      out[(size_t)f * c->N + r] = v;
    }
  return LGBM_HIP_OK;
}

int lgbm_hip_upload_bins16(lgbm_hip_ctx* c, const uint16_t* bins, int32_t num_features,
                           int64_t num_data, const lgbm_feature_meta* meta,
                           const double* bin_upper_bound) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!bins || !meta || num_features <= 0 || num_data <= 0)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null bins/meta or empty shape");
  const int32_t F = num_features;
  for (int f = 0; f < F; ++f)
    if (meta[f].num_bin == 0 || meta[f].num_bin > WIDE_MAX_BIN)
      return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                     "num_bin must be in 1..=" + std::to_string(WIDE_MAX_BIN));
  // bin-range gate (learner.rs:1161-1187): first offending bin, feature order
  for (int f = 0; f < F; ++f) {
    const uint16_t* col = bins + (size_t)f * (size_t)num_data;
    const uint32_t nb = meta[f].num_bin;
    for (int64_t r = 0; r < num_data; ++r)
      if (col[r] >= nb)
        return set_err(c, LGBM_HIP_ERR_BIN_OUT_OF_RANGE,
                       "bin " + std::to_string(col[r]) + " >= num_bin " + std::to_string(nb) +
                           " (feature " + std::to_string(f) + ", row " + std::to_string(r) + ")");
  }
  if ((rc = resident_setup(c, F, num_data, meta, bin_upper_bound))) return rc;
  hipError_t e = hipSuccess;
  if (c->bin16) {
    uint16_t* tmp = nullptr;
    HIPCHK(c, hipMalloc((void**)&tmp, (size_t)F * num_data * 2));
    e = hipMemcpy(tmp, bins, (size_t)F * num_data * 2, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
      launch_pack_wide16(tmp, num_data, F, c->row_stride, c->binmat, c->rec[BUF_ORIG], c->stream);
      launch_wide_cols(c->binmat, num_data, F, c->row_stride, 1, c->bincol, c->stream);
      e = hipStreamSynchronize(c->stream);
    }
    (void)hipFree(tmp);
  } else {
    // every feature fits a byte: the 1-byte layouts
    std::vector<uint8_t> b8((size_t)F * (size_t)num_data);
    for (size_t i = 0; i < b8.size(); ++i) b8[i] = (uint8_t)bins[i];
    uint8_t* tmp = nullptr;
    HIPCHK(c, hipMalloc((void**)&tmp, b8.size()));
    e = hipMemcpy(tmp, b8.data(), b8.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess) {
      if (rec_wide(c->fmt)) {
        launch_pack_wide(tmp, num_data, F, c->row_stride, c->binmat, c->rec[BUF_ORIG], c->stream);
        launch_wide_cols(c->binmat, num_data, F, c->row_stride, 0, c->bincol, c->stream);
      } else {
        launch_pack_records(tmp, num_data, F, c->fmt, c->rec[BUF_ORIG], c->stream);
      }
      e = hipStreamSynchronize(c->stream);
    }
    (void)hipFree(tmp);
  }
  if (e != hipSuccess) return set_err(c, LGBM_HIP_ERR_HIP, hipGetErrorString(e));
  return resident_done(c);
}

int lgbm_hip_set_gradients(lgbm_hip_ctx* c, const float* grad, const float* hess, int64_t n) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_RUNTIME, "upload bins first");
  if (!grad || !hess) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null gradients");
  if (n != c->N) return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "gradient length != num_data");
  // the context stream does not wait on the null stream's copies: a lookahead left
  // queued by train_iter (the next objective and quantizer) writes these buffers
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(c->g, grad, (size_t)n * 4, hipMemcpyHostToDevice));
  HIPCHK(c, hipMemcpy(c->h, hess, (size_t)n * 4, hipMemcpyHostToDevice));
  c->have_grad = true;
  c->quant_ready = false;
  return LGBM_HIP_OK;
}

int lgbm_hip_quantize(lgbm_hip_ctx* c, int32_t bins, int32_t stochastic, uint64_t seed,
                      float* dg_out, float* dh_out, double* scales_out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!c->have_grad) return set_err(c, LGBM_HIP_ERR_RUNTIME, "set gradients first");
  if (bins < 1 || bins > 254)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "num_grad_quant_bins must be in 1..=254");
  float *dg = nullptr, *dh = nullptr;
  if (gen_bins(bins)) {
    // the learner reads these dequantized values (the fixed-point path)
    if ((rc = ensure_dq(c))) return rc;
    dg = c->dq;
    dh = c->dq + c->N;
  } else if (dg_out || dh_out) {
    if ((rc = ensure_scratch_bytes(c, (size_t)c->N * 8))) return rc;
    dg = (float*)c->scratch;
    dh = dg + c->N;
  }
  if ((rc = do_quantize(c, bins, stochastic, seed, dg, dh))) return rc;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  ev_collect(c);
  if (dg_out) HIPCHK(c, hipMemcpy(dg_out, dg, (size_t)c->N * 4, hipMemcpyDeviceToHost));
  if (dh_out) HIPCHK(c, hipMemcpy(dh_out, dh, (size_t)c->N * 4, hipMemcpyDeviceToHost));
  if (scales_out) {
    double s[2];
    if ((rc = ctl_read(c, CTL_OFF(gs), &s[0]))) return rc;
    if ((rc = ctl_read(c, CTL_OFF(hs), &s[1]))) return rc;
    scales_out[0] = s[0];
    scales_out[1] = s[1];
  }
  return LGBM_HIP_OK;
}

int lgbm_hip_get_discretized(lgbm_hip_ctx* c, int8_t* out, int64_t n) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!c->quant_ready) return set_err(c, LGBM_HIP_ERR_RUNTIME, "quantize first");
  if (!out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null out");
  if (n != c->N) return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "n != num_data");
  std::vector<uint16_t> q((size_t)n);
  HIPCHK(c, hipMemcpy(q.data(), c->gh[BUF_ORIG], (size_t)n * 2, hipMemcpyDeviceToHost));
  for (int64_t i = 0; i < n; ++i) {
    out[2 * i] = (int8_t)(uint8_t)(q[i] >> 8);        // hess
    out[2 * i + 1] = (int8_t)(uint8_t)(q[i] & 0xff);  // grad
  }
  return LGBM_HIP_OK;
}

int lgbm_hip_set_dequantized_gradients(lgbm_hip_ctx* c, const float* grad, const float* hess,
                                       int64_t n, int32_t bins, double grad_scale,
                                       double hess_scale) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_RUNTIME, "upload bins first");
  if (!grad || !hess) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null gradients");
  if (n != c->N) return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "gradient length != num_data");
  if (bins < 1 || bins > 254)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "num_grad_quant_bins must be in 1..=254");
  const bool given = grad_scale > 0.0 && hess_scale > 0.0;
  if (!given) {
    if (!c->quant_ready || c->quant_bins != bins)
      return set_err(c, LGBM_HIP_ERR_RUNTIME,
                     "no scales given and no lgbm_hip_quantize with these bins to take them from");
  }
  c->quant_ready = false;
  // as in lgbm_hip_set_gradients: a queued lookahead writes g, h and the scales
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(c->g, grad, (size_t)n * 4, hipMemcpyHostToDevice));
  HIPCHK(c, hipMemcpy(c->h, hess, (size_t)n * 4, hipMemcpyHostToDevice));
  c->have_grad = true;
  if (gen_bins(bins)) {
    // the learner's input for these bin counts: the dequantized values themselves
    if ((rc = ensure_dq(c))) return rc;
    HIPCHK(c, hipMemcpy(c->dq, grad, (size_t)n * 4, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(c->dq + n, hess, (size_t)n * 4, hipMemcpyHostToDevice));
  }
  if (given) {
    // the quantizer header of the control block, as compute_scales leaves it
    // (gradient_discretizer.rs:145-165); the packed cells need q_h >= 0 (hmin 0)
    const double v[4] = {grad_scale, hess_scale, 1.0 / grad_scale, 1.0 / hess_scale};
    const float f[4] = {(float)(1.0 * grad_scale), (float)(1.0 * hess_scale),
                        (float)(3.0 * hess_scale), 0.0f};
    HIPCHK(c, hipMemcpy((char*)c->ctl + CTL_OFF(gs), v, sizeof(v), hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy((char*)c->ctl + CTL_OFF(vg1), f, sizeof(f), hipMemcpyHostToDevice));
    const int32_t qb[2] = {bins, 0};
    HIPCHK(c, hipMemcpy((char*)c->ctl + CTL_OFF(quant_bins), qb, sizeof(qb), hipMemcpyHostToDevice));
  }
  const unsigned long long init[2] = {0ull, ~0ull};
  HIPCHK(c, hipMemcpyAsync(c->d_flags, init, sizeof(init), hipMemcpyHostToDevice, c->stream));
  launch_requant(c->g, c->h, n, c->ctl, bins, c->gh[BUF_ORIG], c->d_flags, c->stream);
  HIPCHK(c, hipGetLastError());
  unsigned long long bad[2] = {0ull, 0ull};
  HIPCHK(c, hipMemcpyAsync(bad, c->d_flags, sizeof(bad), hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (bad[0]) {
    c->have_grad = false;  // nothing consistent to grow from
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT,
                   std::to_string(bad[0]) + " rows are not f32(q * scale) for an in-range q "
                   "(first row " + std::to_string(bad[1]) + ")");
  }
  c->quant_ready = true;
  c->quant_bins = bins;
  return LGBM_HIP_OK;
}

int lgbm_hip_set_feature_contri(lgbm_hip_ctx* c, const double* contri, int32_t n) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_RUNTIME, "upload bins first");
  if (n < 0 || (n > 0 && !contri))
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null contri or negative length");
  for (DevFeature& d : c->feats) {
    const int32_t ri = d.real_index;
    d.penalty = (ri >= 0 && ri < n) ? contri[ri] : 1.0;
  }
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(c->d_feats, c->feats.data(), c->feats.size() * sizeof(DevFeature),
                      hipMemcpyHostToDevice));
  return LGBM_HIP_OK;
}

static int set_hist_job(lgbm_hip_ctx* c, const uint32_t* rows, int64_t n_rows) {
  int rc;
  int32_t buf = BUF_ORIG;
  int64_t count = c->N;
  if (rows) {
    for (int64_t i = 0; i < n_rows; ++i)
      if (rows[i] >= (uint64_t)c->N)
        return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "leaf row index out of range");
    if ((rc = ensure_scratch_rows(c, n_rows))) return rc;
    if ((rc = ensure_scratch_bytes(c, (size_t)std::max<int64_t>(n_rows, 1) * 4))) return rc;
    HIPCHK(c, hipMemcpy(c->scratch, rows, (size_t)n_rows * 4, hipMemcpyHostToDevice));
    launch_gather_rows(c->fmt, (const uint32_t*)c->scratch, n_rows, c->rec[BUF_ORIG],
                       c->gh[BUF_ORIG], c->g32[BUF_ORIG], c->rec[BUF_S0], c->gh[BUF_S0],
                       c->g32[BUF_S0], c->stream);
    buf = BUF_S0;
    count = n_rows;
  }
  const HistJob hj{buf, 0, 0, count, 0, 0};
  if ((rc = ctl_write(c, CTL_OFF(hjobs), hj))) return rc;
  const int32_t one = 1;
  if ((rc = ctl_write(c, CTL_OFF(n_hjobs), one))) return rc;
  return LGBM_HIP_OK;
}

int lgbm_hip_build_int_histogram(lgbm_hip_ctx* c, const uint32_t* leaf_rows, int64_t n_rows,
                                 int64_t* out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!c->quant_ready) return set_err(c, LGBM_HIP_ERR_RUNTIME, "quantize first");
  if (!out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null out");
  if (gen_bins(c->quant_bins))
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "integer (sum q) histograms need num_grad_quant_bins 2 or 4 (the packed cells)");
  if (rec_wide(c->fmt))
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "per-op histogram builds need the record layouts (F <= 124, cells <= 8192)");
  if (c->total_cells > QUANT_LDS_CELLS)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "quantized histograms hold every cell in LDS: at most 8192 (feature, bin) cells");
  if ((rc = set_hist_job(c, leaf_rows, n_rows))) return rc;
  DevLearner L = make_learner(c);
  launch_hist(L, c->stream);
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HistJob hj{};
  if ((rc = ctl_read(c, CTL_OFF(hjobs), &hj))) return rc;
  const size_t stride = (size_t)c->total_cells * 3;
  std::vector<int32_t> part((size_t)std::max(hj.nblk, 1) * stride, 0);
  if (hj.nblk > 0)
    HIPCHK(c, hipMemcpy(part.data(), c->hist_part + (size_t)hj.a0 * stride,
                        (size_t)hj.nblk * stride * 4, hipMemcpyDeviceToHost));
  for (int32_t i = 0; i < c->total_cells; ++i) {
    int64_t g = 0, h = 0;
    for (int32_t k = 0; k < hj.nblk; ++k) {
      g += part[k * stride + 3 * (size_t)i];
      h += part[k * stride + 3 * (size_t)i + 1];
    }
    out[2 * i] = g;
    out[2 * i + 1] = h;
  }
  return LGBM_HIP_OK;
}

}  // extern "C"

// build_resident_leaf's body (lib.rs:1953-1972): gather the leaf's rows, build its
// histogram (quantized or f32 gradients), FixHistogram + compaction on the leaf's RAW
// sums, into the device slot d_out (slot_len doubles); enqueued on the context stream.
static int build_leaf_into(lgbm_hip_ctx* c, const uint32_t* leaf_rows, int64_t n_rows,
                           double sum_gradient, double sum_hessian, double* d_out) {
  int rc;
  if (rec_wide(c->fmt))
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "per-op histogram builds need the record layouts (F <= 124, cells <= 8192)");
  // quantized gradients (after lgbm_hip_quantize; bin counts other than 2 and 4 as their
  // dequantized values through the exact fixed-point path) or the f32 gradients
  const bool gen = c->quant_ready && gen_bins(c->quant_bins);
  const int32_t fp = c->quant_ready && !gen ? 0 : 1;
  if (fp && !gen && !c->have_grad) return set_err(c, LGBM_HIP_ERR_RUNTIME, "set gradients first");
  if (gen && !c->dq) return set_err(c, LGBM_HIP_ERR_RUNTIME, "quantize again");
  if (!fp && c->N >= QUANT_MAX_ROWS)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "quantized int32 histogram cells need N < 2^29");
  if (!fp && !rec_wide(c->fmt) && c->total_cells > QUANT_LDS_CELLS)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "quantized histograms hold every cell in LDS: at most 8192 (feature, bin) cells");
  DevLearner L0 = make_learner(c);
  if (fp) {
    if ((rc = ensure_fp(c))) return rc;
    L0 = make_learner(c);
    if (gen)
      launch_exact_prep(L0, c->dq, c->dq + c->N, c->N, c->stream);
    else
      launch_fp_prep(L0, c->g, c->h, c->N, c->partials, c->stream);
  }
  if ((rc = set_hist_job(c, leaf_rows, n_rows))) return rc;
  LeafSums s{sum_gradient, sum_hessian, 0.0, (int32_t)(leaf_rows ? n_rows : c->N), 0};
  if ((rc = ctl_write(c, CTL_OFF(sm), s))) return rc;
  if ((rc = ctl_write(c, CTL_OFF(fp_mode), fp))) return rc;
  DevLearner L = make_learner(c);
  if (fp)
    launch_hist_f32(L, c->stream);
  else
    launch_hist(L, c->stream);
  launch_fixscan(L, 2, d_out, c->stream);
  HIPCHK(c, hipGetLastError());
  return LGBM_HIP_OK;
}

extern "C" {

int lgbm_hip_build_leaf_histogram(lgbm_hip_ctx* c, const uint32_t* leaf_rows, int64_t n_rows,
                                  double sum_gradient, double sum_hessian, double* out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null out");
  if ((rc = dalloc(c, &c->slot_tmp, (size_t)c->slot_len))) return rc;
  if ((rc = build_leaf_into(c, leaf_rows, n_rows, sum_gradient, sum_hessian, c->slot_tmp)))
    return rc;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(out, c->slot_tmp, (size_t)c->slot_len * 8, hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

int lgbm_hip_find_best_splits(lgbm_hip_ctx* c, const double* hist, int64_t hist_len,
                              const lgbm_batched_feature* feats, int32_t n_feats,
                              const lgbm_gain_config* cfg, double sum_gradient,
                              double sum_hessian, int32_t num_data, lgbm_split_info* out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!hist || !feats || !cfg || !out || n_feats < 0)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null argument");
  if (n_feats == 0) return LGBM_HIP_OK;
  std::vector<DevFeature> df(n_feats);
  for (int i = 0; i < n_feats; ++i) {
    if (feats[i].num_bin == 0) return set_err(c, LGBM_HIP_ERR_RUNTIME, "num_bin must be > 0");
    if (feats[i].num_bin > 256)
      return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_bin must be <= 256");
    if (feats[i].slot_off + 2ull * feats[i].num_bin > (uint64_t)hist_len)
      return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "feature region beyond the histogram");
    df[i] = feature_from_batched(feats[i]);
  }
  if (!(sum_hessian > 0.0))
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "find_best_split: sum_hessian must be > 0");
  const size_t bytes = (size_t)hist_len * 8 + (size_t)n_feats * (sizeof(DevFeature) + sizeof(lgbm_split_info)) + 64;
  if ((rc = ensure_scratch_bytes(c, bytes))) return rc;
  char* base = (char*)c->scratch;
  double* d_hist = (double*)base;
  DevFeature* d_f = (DevFeature*)(base + ((size_t)hist_len * 8 + 15) / 16 * 16);
  lgbm_split_info* d_out = (lgbm_split_info*)((char*)d_f + (size_t)n_feats * sizeof(DevFeature));
  HIPCHK(c, hipMemcpy(d_hist, hist, (size_t)hist_len * 8, hipMemcpyHostToDevice));
  HIPCHK(c, hipMemcpy(d_f, df.data(), df.size() * sizeof(DevFeature), hipMemcpyHostToDevice));
  launch_scan_explicit(d_hist, d_f, n_feats, *cfg, sum_gradient, sum_hessian, num_data, d_out,
                       c->stream);
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(out, d_out, (size_t)n_feats * sizeof(lgbm_split_info), hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

}  // extern "C"

// lgbm_hip_find_best_splits_noalloc's feature table: the host entry's checks and
// feature_from_batched on the device.  One block; word 0 of the header receives the
// smallest (feature * 4 + check) that fails (0 num_bin == 0, 1 num_bin > 256,
// 2 region past hist_len), ~0 for none.  A failing feature gets num_bin 0, which the
// scan reads as an empty feature.
__global__ __launch_bounds__(256) void k_noalloc_feats(const lgbm_batched_feature* __restrict__ in,
                                                       int32_t n, int64_t hist_len,
                                                       unsigned char* __restrict__ ws) {
  uint32_t* err = (uint32_t*)ws;
  DevFeature* out = (DevFeature*)(ws + NOALLOC_HEADER);
  if (threadIdx.x == 0) *err = ~0u;
  __syncthreads();
  for (int32_t i = threadIdx.x; i < n; i += blockDim.x) {
    const lgbm_batched_feature b = in[i];
    int32_t bad = -1;
    if (b.num_bin == 0) bad = 0;
    else if (b.num_bin > 256) bad = 1;
    else if (b.slot_off + 2ull * b.num_bin > (uint64_t)hist_len) bad = 2;
    DevFeature f{};
    f.num_bin = bad < 0 ? b.num_bin : 0u;
    f.offset = b.offset;
    f.default_bin = b.default_bin;
    f.mfb = b.most_freq_bin;
    f.slot_off = bad < 0 ? (uint32_t)b.slot_off : 0u;
    f.cell_base = f.slot_off / 2;
    f.skip_default_bin = b.skip_default_bin;
    f.na_as_missing = b.na_as_missing;
    f.run_forward = b.run_forward;
    f.real_index = -1;
    f.penalty = 1.0;
    out[i] = f;
    if (bad >= 0) atomicMin(err, (uint32_t)i * 4u + (uint32_t)bad);
  }
}

extern "C" {

int lgbm_hip_find_best_splits_noalloc(lgbm_hip_ctx* c, const double* d_hist, int64_t hist_len,
                                      const lgbm_batched_feature* d_feats, int32_t n_feats,
                                      const lgbm_gain_config* cfg, double sum_gradient,
                                      double sum_hessian, int32_t num_data,
                                      lgbm_split_info* d_out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!d_hist || !d_feats || !cfg || !d_out || n_feats < 0 || hist_len < 0)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null argument or negative size");
  if (n_feats > LGBM_HIP_NOALLOC_MAX_FEATURES)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "n_feats " + std::to_string(n_feats) + " exceeds the no-allocation maximum " +
                       std::to_string(LGBM_HIP_NOALLOC_MAX_FEATURES));
  if (n_feats == 0) return LGBM_HIP_OK;
  if (!c->noalloc) return set_err(c, LGBM_HIP_ERR_HIP, "no-allocation working memory unresolved");
  if (!(sum_hessian > 0.0))
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "find_best_split: sum_hessian must be > 0");
  k_noalloc_feats<<<dim3(1), dim3(256), 0, c->stream>>>(d_feats, n_feats, hist_len, c->noalloc);
  launch_scan_explicit(d_hist, (const DevFeature*)(c->noalloc + NOALLOC_HEADER), n_feats, *cfg,
                       sum_gradient, sum_hessian, num_data, d_out, c->stream);
  HIPCHK(c, hipGetLastError());
  uint32_t err = 0;
  HIPCHK(c, hipMemcpyAsync(&err, c->noalloc, sizeof(err), hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (err != ~0u) {
    const uint32_t f = err / 4u, k = err % 4u;
    if (k == 0) return set_err(c, LGBM_HIP_ERR_RUNTIME, "num_bin must be > 0 (feature " + std::to_string(f) + ")");
    if (k == 1) return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_bin must be <= 256 (feature " + std::to_string(f) + ")");
    return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH,
                   "feature region beyond the histogram (feature " + std::to_string(f) + ")");
  }
  return LGBM_HIP_OK;
}

int lgbm_hip_subtract_histograms(lgbm_hip_ctx* c, const double* parent, const double* child,
                                 int64_t len, double* out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!parent || !child || !out || len < 0)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null argument");
  if (len == 0) return LGBM_HIP_OK;
  if ((rc = ensure_scratch_bytes(c, (size_t)len * 24))) return rc;
  double* a = (double*)c->scratch;
  double* b = a + len;
  double* o = b + len;
  HIPCHK(c, hipMemcpy(a, parent, (size_t)len * 8, hipMemcpyHostToDevice));
  HIPCHK(c, hipMemcpy(b, child, (size_t)len * 8, hipMemcpyHostToDevice));
  launch_subtract(a, b, len, o, c->stream);
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(out, o, (size_t)len * 8, hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

int lgbm_hip_data_partition(lgbm_hip_ctx* c, const uint32_t* bins, int64_t n, uint32_t num_bin,
                            uint32_t min_bin, uint32_t max_bin, uint32_t threshold,
                            uint32_t most_freq_bin, int32_t na_as_missing, int32_t default_left,
                            uint32_t* order_out, int64_t* left_count_out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if ((!bins && n > 0) || (!order_out && n > 0) || !left_count_out || n < 0)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null argument");
  if (num_bin == 0) return set_err(c, LGBM_HIP_ERR_RUNTIME, "data_partition: num_bin must be > 0");
  if (threshold >= num_bin)
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "data_partition: threshold >= num_bin");
  for (int64_t i = 0; i < n; ++i)
    if (bins[i] >= num_bin)
      return set_err(c, LGBM_HIP_ERR_BIN_OUT_OF_RANGE,
                     "bin " + std::to_string(bins[i]) + " >= num_bin at row " + std::to_string(i));
  if (num_bin > 256) return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_bin must be <= 256");
  if (n == 0) {
    *left_count_out = 0;
    return LGBM_HIP_OK;
  }
  const int saved_fmt = c->fmt;
  c->fmt = 1;  // the per-op partition's own one-word records (k_pack_partition)
  rc = ensure_scratch_rows(c, n);
  c->fmt = saved_fmt;
  if (rc) return rc;
  if ((rc = ensure_tile_state(c, n))) return rc;
  if ((rc = ensure_scratch_bytes(c, (size_t)n * 4))) return rc;
  HIPCHK(c, hipMemcpy(c->scratch, bins, (size_t)n * 4, hipMemcpyHostToDevice));
  launch_pack_partition((const uint32_t*)c->scratch, n, c->rec[BUF_S0], c->stream);
  HIPCHK(c, hipMemsetAsync(c->gh[BUF_S0], 0, (size_t)n * 2, c->stream));
  PartJob J{};
  J.acc_right = -1;
  J.parent = -1;
  J.cl = -1;
  J.cr = -1;
  J.ntiles = (int32_t)((n + part_tile(1) - 1) / part_tile(1));
  J.tile0 = 0;
  J.src_buf = BUF_S0;
  J.dst_buf = BUF_S1;
  J.begin = 0;
  J.count = n;
  J.rev = 0;
  J.fbyte = 0;
  J.pmin = (int32_t)min_bin;
  J.max_bin = (int32_t)max_bin;
  J.th = (int32_t)threshold + (int32_t)min_bin - (most_freq_bin == 0 ? 1 : 0);
  J.na_bin = (int32_t)num_bin - 1;
  J.flags = ((int32_t)most_freq_bin > (int32_t)threshold ? 1 : 0) | (na_as_missing ? 2 : 0) |
            (default_left ? 4 : 0);
  if ((rc = ctl_write(c, CTL_OFF(jobs), J))) return rc;
  const int32_t one = 1;
  if ((rc = ctl_write(c, CTL_OFF(n_jobs), one))) return rc;
  const int64_t tiles = J.ntiles;
  if ((rc = ctl_write(c, CTL_OFF(tile_total), tiles))) return rc;
  DevLearner L = make_learner(c);
  L.fmt = 1;
  L.total_cells = 0;  // partition only: no histogram cells in LDS
  launch_partition_stable(L, tiles, std::min<int64_t>(c->part_blocks, tiles), c->stream);
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipStreamSynchronize(c->stream));
  int32_t lc = 0;
  if ((rc = ctl_read(c, CTL_OFF(part_left_count), &lc))) return rc;
  std::vector<uint4> recs((size_t)n);
  HIPCHK(c, hipMemcpy(recs.data(), c->rec[BUF_S1], (size_t)n * 16, hipMemcpyDeviceToHost));
  for (int64_t i = 0; i < lc; ++i) order_out[i] = recs[i].w;
  for (int64_t i = lc; i < n; ++i) order_out[i] = recs[n - 1 - (i - lc)].w;  // stored reversed
  *left_count_out = lc;
  // the scratch rows were sized for W=1 here; force a re-size for the next gather
  c->buf_rows[BUF_S0] = c->buf_rows[BUF_S1] = 0;
  return LGBM_HIP_OK;
}

// ---- device-resident histogram slots ----------------------------------------------
// The reference's resident arm keeps each leaf's f64 histogram in a device slot that
// never crosses to the host (Backend::reset_resident_pool, build_resident_leaf,
// move_resident, subtract_resident, scan_resident_leaf, scan_resident_siblings;
// lib.rs:1940-2058).  Here the slots are one context-owned array of num_slots x
// slot_len doubles; every entry runs on the context stream and returns after it.

}  // extern "C"

static int res_slot_ok(lgbm_hip_ctx* c, int32_t s) {
  if (!c->res_slots || c->res_num == 0)
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "reset the resident pool first");
  if (c->res_len != (int64_t)c->slot_len)
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "the resident pool predates the current bins: reset it");
  if (s < 0 || s >= c->res_num)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT,
                   "resident slot " + std::to_string(s) + " outside [0, " +
                       std::to_string(c->res_num) + ")");
  return LGBM_HIP_OK;
}

// The host entry's feature checks and table (find_best_splits), the table staged in
// the scratch buffer after `reserve` bytes; returns the device table in *d_f.
static int res_feature_table(lgbm_hip_ctx* c, const lgbm_batched_feature* feats, int32_t n_feats,
                             size_t reserve, DevFeature** d_f) {
  std::vector<DevFeature> df((size_t)n_feats);
  for (int i = 0; i < n_feats; ++i) {
    if (feats[i].num_bin == 0) return set_err(c, LGBM_HIP_ERR_RUNTIME, "num_bin must be > 0");
    if (feats[i].num_bin > 256) return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_bin must be <= 256");
    if (feats[i].slot_off + 2ull * feats[i].num_bin > (uint64_t)c->res_len)
      return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "feature region beyond the slot");
    df[(size_t)i] = feature_from_batched(feats[i]);
  }
  const size_t tab = (size_t)n_feats * sizeof(DevFeature);
  int rc = ensure_scratch_bytes(c, reserve + tab);
  if (rc) return rc;
  *d_f = (DevFeature*)((char*)c->scratch + reserve);
  HIPCHK(c, hipMemcpy(*d_f, df.data(), tab, hipMemcpyHostToDevice));
  return LGBM_HIP_OK;
}

extern "C" {

int lgbm_hip_resident_reset(lgbm_hip_ctx* c, int32_t num_slots, int64_t slot_len) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_RUNTIME, "upload bins first");
  if (num_slots < 1) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "num_slots must be >= 1");
  if (slot_len != (int64_t)c->slot_len)
    return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH,
                   "slot_len " + std::to_string(slot_len) + " != the resident layout's " +
                       std::to_string(c->slot_len));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (!c->res_slots || (int64_t)num_slots * slot_len > c->res_cap) {
    c->res_num = 0;
    if ((rc = dalloc(c, &c->res_slots, (size_t)num_slots * (size_t)slot_len))) {
      c->res_cap = 0;
      return rc;
    }
    c->res_cap = (int64_t)num_slots * slot_len;
  }
  c->res_num = num_slots;
  c->res_len = slot_len;
  return LGBM_HIP_OK;
}

int lgbm_hip_resident_build(lgbm_hip_ctx* c, int32_t slot, const uint32_t* leaf_rows,
                            int64_t n_rows, double sum_gradient, double sum_hessian) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;
  if ((rc = res_slot_ok(c, slot))) return rc;
  if (leaf_rows && n_rows < 0) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "negative n_rows");
  if ((rc = build_leaf_into(c, leaf_rows, n_rows, sum_gradient, sum_hessian,
                            c->res_slots + (size_t)slot * (size_t)c->res_len)))
    return rc;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return LGBM_HIP_OK;
}

int lgbm_hip_resident_move(lgbm_hip_ctx* c, int32_t src_slot, int32_t dst_slot) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if ((rc = res_slot_ok(c, src_slot)) || (rc = res_slot_ok(c, dst_slot))) return rc;
  if (src_slot == dst_slot) return LGBM_HIP_OK;
  const size_t L = (size_t)c->res_len;
  HIPCHK(c, hipMemcpyAsync(c->res_slots + (size_t)dst_slot * L, c->res_slots + (size_t)src_slot * L,
                           L * 8, hipMemcpyDeviceToDevice, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return LGBM_HIP_OK;
}

int lgbm_hip_resident_subtract(lgbm_hip_ctx* c, int32_t parent_slot, int32_t smaller_slot,
                               int32_t larger_slot) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if ((rc = res_slot_ok(c, parent_slot)) || (rc = res_slot_ok(c, smaller_slot)) ||
      (rc = res_slot_ok(c, larger_slot)))
    return rc;
  if (smaller_slot == larger_slot)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "smaller and larger slots coincide");
  const size_t L = (size_t)c->res_len;
  // elementwise: larger may be the parent's slot (each cell is read, then written)
  launch_subtract(c->res_slots + (size_t)parent_slot * L, c->res_slots + (size_t)smaller_slot * L,
                  (int64_t)L, c->res_slots + (size_t)larger_slot * L, c->stream);
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return LGBM_HIP_OK;
}

int lgbm_hip_resident_read(lgbm_hip_ctx* c, int32_t slot, double* out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if ((rc = res_slot_ok(c, slot))) return rc;
  if (!out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null out");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(out, c->res_slots + (size_t)slot * (size_t)c->res_len,
                      (size_t)c->res_len * 8, hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

int lgbm_hip_resident_scan(lgbm_hip_ctx* c, int32_t slot, const lgbm_batched_feature* feats,
                           int32_t n_feats, const lgbm_gain_config* cfg, double sum_gradient,
                           double sum_hessian, int32_t num_data, lgbm_split_info* out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;
  if ((rc = res_slot_ok(c, slot))) return rc;
  if (!feats || !cfg || !out || n_feats < 0)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null argument");
  if (n_feats == 0) return LGBM_HIP_OK;
  if (!(sum_hessian > 0.0))
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "find_best_split: sum_hessian must be > 0");
  const size_t outb = ((size_t)n_feats * sizeof(lgbm_split_info) + 255) / 256 * 256;
  DevFeature* d_f = nullptr;
  if ((rc = res_feature_table(c, feats, n_feats, outb, &d_f))) return rc;
  lgbm_split_info* d_out = (lgbm_split_info*)c->scratch;
  launch_scan_explicit(c->res_slots + (size_t)slot * (size_t)c->res_len, d_f, n_feats, *cfg,
                       sum_gradient, sum_hessian, num_data, d_out, c->stream);
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(out, d_out, (size_t)n_feats * sizeof(lgbm_split_info), hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

int lgbm_hip_resident_scan_siblings(lgbm_hip_ctx* c, int32_t smaller_slot, int32_t larger_slot,
                                    const lgbm_batched_feature* feats, int32_t n_feats,
                                    const lgbm_gain_config* cfg, const lgbm_leaf_sums* smaller,
                                    const lgbm_leaf_sums* larger, lgbm_split_info* out_smaller,
                                    lgbm_split_info* out_larger) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;
  if ((rc = res_slot_ok(c, smaller_slot)) || (rc = res_slot_ok(c, larger_slot))) return rc;
  if (!feats || !cfg || !smaller || !larger || !out_smaller || !out_larger || n_feats < 0)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null argument");
  if (n_feats == 0) return LGBM_HIP_OK;
  if (!(smaller->sum_hessian > 0.0) || !(larger->sum_hessian > 0.0))
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "find_best_split: sum_hessian must be > 0");
  const size_t one = ((size_t)n_feats * sizeof(lgbm_split_info) + 255) / 256 * 256;
  DevFeature* d_f = nullptr;
  if ((rc = res_feature_table(c, feats, n_feats, 2 * one, &d_f))) return rc;
  lgbm_split_info* d_out = (lgbm_split_info*)c->scratch;
  lgbm_split_info* d_out2 = (lgbm_split_info*)((char*)c->scratch + one);
  // each sibling's own parent_output (LeafSplits::weight) rides in its totals
  lgbm_gain_config cs = *cfg, cl = *cfg;
  cs.parent_output = smaller->weight;
  cl.parent_output = larger->weight;
  const size_t L = (size_t)c->res_len;
  launch_scan_explicit(c->res_slots + (size_t)smaller_slot * L, d_f, n_feats, cs,
                       smaller->sum_gradient, smaller->sum_hessian, smaller->num_data, d_out,
                       c->stream);
  launch_scan_explicit(c->res_slots + (size_t)larger_slot * L, d_f, n_feats, cl,
                       larger->sum_gradient, larger->sum_hessian, larger->num_data, d_out2,
                       c->stream);
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(out_smaller, d_out, (size_t)n_feats * sizeof(lgbm_split_info),
                      hipMemcpyDeviceToHost));
  HIPCHK(c, hipMemcpy(out_larger, d_out2, (size_t)n_feats * sizeof(lgbm_split_info),
                      hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

int lgbm_hip_grow_tree(lgbm_hip_ctx* c, const lgbm_gain_config* cfg, int32_t num_leaves,
                       int32_t max_depth, lgbm_tree_out* tree, lgbm_layout_out* layout) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!cfg) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null cfg");
  if (num_leaves < 1) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "num_leaves must be >= 1");
  if (num_leaves > 256) return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_leaves must be <= 256");
  // quantized gradients (after lgbm_hip_quantize; bin counts other than 2 and 4 as their
  // dequantized values through the exact fixed-point path) or the f32 gradients
  const bool gen = c->quant_ready && gen_bins(c->quant_bins);
  const int32_t fp = c->quant_ready && !gen ? 0 : 1;
  if (fp && !gen && !c->have_grad) return set_err(c, LGBM_HIP_ERR_RUNTIME, "set gradients first");
  if (gen && !c->dq) return set_err(c, LGBM_HIP_ERR_RUNTIME, "quantize again");
  if (gen && c->quant_bins == 1)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_grad_quant_bins 1 gives no gradient scale");
  if (!fp && c->N >= QUANT_MAX_ROWS)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "quantized int32 histogram cells need N < 2^29");
  if (!fp && !rec_wide(c->fmt) && c->total_cells > QUANT_LDS_CELLS)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "quantized histograms hold every cell in LDS: at most 8192 (feature, bin) cells");
  if ((rc = check_cat_capacity(c, tree, num_leaves))) return rc;
  if (fp) {
    if ((rc = ensure_fp(c))) return rc;
    if ((rc = ensure_leaves(c, num_leaves))) return rc;
    DevLearner L = make_learner(c);
    if (gen)
      launch_exact_prep(L, c->dq, c->dq + c->N, c->N, c->stream);
    else
      launch_fp_prep(L, c->g, c->h, c->N, c->partials, c->stream);
  }
  if ((rc = grow_tree_async(c, cfg, num_leaves, max_depth, fp))) return rc;
  return finish_tree(c, tree, layout, 1.0);
}

int lgbm_hip_cat_threshold_words(lgbm_hip_ctx* c, int32_t num_leaves, int64_t* out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null out");
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_RUNTIME, "upload bins first");
  *out = cat_words_needed(c, num_leaves);
  return LGBM_HIP_OK;
}

int lgbm_hip_set_labels(lgbm_hip_ctx* c, const float* labels, int64_t n, double init_score) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_RUNTIME, "upload bins first");
  if (!labels) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null labels");
  if (n != c->N) return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "labels length != num_data");
  if ((rc = dalloc(c, &c->label, (size_t)n))) return rc;
  if ((rc = dalloc(c, &c->score, (size_t)n))) return rc;
  HIPCHK(c, hipMemcpy(c->label, labels, (size_t)n * 4, hipMemcpyHostToDevice));
  std::vector<double> s((size_t)n, init_score);
  HIPCHK(c, hipMemcpy(c->score, s.data(), (size_t)n * 8, hipMemcpyHostToDevice));
  c->num_class = 1;
  c->have_labels = true;
  c->have_rank = false;  // the lambdarank tables were built from the old labels
  return LGBM_HIP_OK;
}

}  // extern "C"

namespace {
// quant_train_renew_leaf after a quantized tree (gbdt.rs:1194-1212): the tree's layout
// exported on the device, then every leaf's output from the original gradients g, h
// (the tree blob's leaf values, read by the score update and the host copy).
int renew_leaves(lgbm_hip_ctx* c, int32_t num_leaves, const float* g, const float* h,
                 const lgbm_gain_config* cfg) {
  if (!c->renew_idx || !c->renew_scratch || c->renew_rows != c->N)
    return set_err(c, LGBM_HIP_ERR_RUNTIME,
                   "quant_train_renew_leaf was set for other bins: set it again after the upload");
  DevLearner L = make_learner(c);
  launch_export_layout(L, num_leaves, c->renew_idx, c->renew_scratch, c->stream);
  launch_renew_leaves(L, c->renew_idx, g, h, cfg->lambda_l1, cfg->lambda_l2, c->stream);
  HIPCHK(c, hipGetLastError());
  return LGBM_HIP_OK;
}

// One resident boosting iteration of a one-tree-per-iteration objective.
int train_iter_single(lgbm_hip_ctx* c, int32_t objective, int32_t iter, const lgbm_gain_config* cfg,
                      int32_t num_leaves, int32_t max_depth, double learning_rate,
                      int32_t num_grad_quant_bins, int32_t stochastic, lgbm_tree_out* tree) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!c->have_labels) return set_err(c, LGBM_HIP_ERR_RUNTIME, "set labels first");
  if (objective == LGBM_HIP_OBJECTIVE_LAMBDARANK && !c->have_rank)
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "lambdarank needs lgbm_hip_set_lambdarank");
  if (c->num_class != 1)
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "the resident labels are multiclass");
  if (!cfg) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null cfg");
  if (num_leaves < 1 || num_leaves > 256)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_leaves must be in 1..=256");
  // num_grad_quant_bins = 0: use_quantized_grad = false (f32 gradients); 2 and 4: packed
  // integer cells; other counts: the dequantized values through the exact fixed-point path
  if (num_grad_quant_bins < 0 || num_grad_quant_bins > 254)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "num_grad_quant_bins must be in 0..=254");
  if (num_grad_quant_bins == 1)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_grad_quant_bins 1 gives no gradient scale");
  const bool gen = gen_bins(num_grad_quant_bins);
  const int32_t fp = num_grad_quant_bins == 0 || gen ? 1 : 0;
  if (!fp && c->N >= QUANT_MAX_ROWS)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "quantized int32 histogram cells need N < 2^29");
  if (!fp && !rec_wide(c->fmt) && c->total_cells > QUANT_LDS_CELLS)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "quantized histograms hold every cell in LDS: at most 8192 (feature, bin) cells");
  if ((rc = check_cat_capacity(c, tree, num_leaves))) return rc;
  if (fp) {
    if ((rc = ensure_fp(c))) return rc;
    if ((rc = ensure_leaves(c, num_leaves))) return rc;
  }
  if (gen && (rc = ensure_dq(c))) return rc;
  const bool pro = c->ahead && c->ahead_iter == iter && c->ahead_qbins == num_grad_quant_bins &&
                   c->ahead_stoch == stochastic && c->ahead_obj == objective;
  c->ahead = false;
  timing_hold(c);
  if (!pro) enqueue_objective(c, objective, iter, num_grad_quant_bins, stochastic);
  if ((rc = grow_tree_async(c, cfg, num_leaves, max_depth, fp))) return rc;
  if (num_grad_quant_bins > 0 && c->renew_leaf &&
      (rc = renew_leaves(c, num_leaves, c->g, c->h, cfg)))
    return rc;
  DevLearner L = make_learner(c);
  KernelEvents ke;
  launch_score_update(L, learning_rate, c->score, c->stream, ev_kernel(c, FAM_OBJ, &ke));
  HIPCHK(c, hipGetLastError());
  if (c->lookahead && !c->timing) {
    // the tree copy is enqueued first, then iteration iter + 1's gradients and
    // quantization (they read the score this tree just updated): the host waits for
    // the copy alone while the device goes on
    HIPCHK(c, hipMemcpyAsync(c->tree_host, c->tree_blob, tree ? c->tree_blob_bytes : 64,
                             hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipEventRecord(c->tree_ev, c->stream));
    enqueue_objective(c, objective, iter + 1, num_grad_quant_bins, stochastic);
    HIPCHK(c, hipGetLastError());
    c->ahead = true;
    c->ahead_iter = iter + 1;
    c->ahead_qbins = num_grad_quant_bins;
    c->ahead_stoch = stochastic;
    c->ahead_obj = objective;
    HIPCHK(c, hipEventSynchronize(c->tree_ev));
    return finish_tree(c, tree, nullptr, learning_rate, true);
  }
  return finish_tree(c, tree, nullptr, learning_rate);
}

// Rust's saturating float -> integer casts (`l as i32`, `l as usize`): truncation
// toward zero, NaN -> 0, values past the type's range clamped.  A NaN ranking label
// passes DCGCalculator::check_labels (dcg_calculator.rs:112-137, every comparison with
// NaN is false) and then indexes the label gains as 0.
int32_t rust_as_i32(float l) {
  if (!(l == l)) return 0;
  if (l <= -2147483648.0f) return INT32_MIN;
  if (l >= 2147483648.0f) return INT32_MAX;
  return (int32_t)l;
}
size_t rust_as_usize(float l) { return l == l && l > 0.0f ? (size_t)rust_as_i32(l) : 0; }

// DCGCalculator::cal_max_dcg_at_k (lgbm-metric/src/dcg_calculator.rs:142-165); labels
// already checked to be NaN or integers in [0, gain.size())
double max_dcg_at_k(const std::vector<double>& gain, const std::vector<double>& disc, int32_t k,
                    const float* labels, int32_t cnt) {
  std::vector<int64_t> n_of((size_t)gain.size(), 0);
  for (int32_t i = 0; i < cnt; ++i) n_of[rust_as_usize(labels[i])] += 1;
  int64_t top = (int64_t)gain.size() - 1;
  double sum = 0.0;
  for (int32_t j = 0; j < std::min(k, cnt); ++j) {
    while (top > 0 && n_of[(size_t)top] <= 0) --top;
    if (top < 0) break;
    sum += disc[(size_t)j] * gain[(size_t)top];
    n_of[(size_t)top] -= 1;
  }
  return sum;
}
}  // namespace

extern "C" {

int lgbm_hip_train_iter_binary(lgbm_hip_ctx* c, int32_t iter, const lgbm_gain_config* cfg,
                               int32_t num_leaves, int32_t max_depth, double learning_rate,
                               int32_t num_grad_quant_bins, int32_t stochastic,
                               lgbm_tree_out* tree) {
  return train_iter_single(c, LGBM_HIP_OBJECTIVE_BINARY, iter, cfg, num_leaves, max_depth,
                           learning_rate, num_grad_quant_bins, stochastic, tree);
}

int lgbm_hip_train_iter(lgbm_hip_ctx* c, int32_t iter, const lgbm_gain_config* cfg,
                        int32_t num_leaves, int32_t max_depth, double learning_rate,
                        int32_t num_grad_quant_bins, int32_t stochastic, lgbm_tree_out* tree) {
  int rc = check_ctx(c);
  if (rc) return rc;
  return train_iter_single(c, c->objective, iter, cfg, num_leaves, max_depth, learning_rate,
                           num_grad_quant_bins, stochastic, tree);
}

int lgbm_hip_set_objective(lgbm_hip_ctx* c, int32_t objective) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (objective != LGBM_HIP_OBJECTIVE_BINARY && objective != LGBM_HIP_OBJECTIVE_REGRESSION &&
      objective != LGBM_HIP_OBJECTIVE_LAMBDARANK)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "unknown objective");
  c->ahead = false;
  c->objective = objective;
  return LGBM_HIP_OK;
}

int lgbm_hip_set_lambdarank(lgbm_hip_ctx* c, const int32_t* query_boundaries, int32_t num_queries,
                            double sigmoid, int32_t norm, int32_t truncation_level) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;
  c->have_rank = false;
  if (!c->have_labels || c->num_class != 1)
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "set the (single-score) labels first");
  if (!query_boundaries || num_queries < 1)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "no query boundaries");
  if (!(sigmoid > 0.0))
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "lambdarank sigmoid must be > 0");
  // validate_query_boundaries (rank.rs:62-86)
  if (query_boundaries[0] != 0 || query_boundaries[num_queries] != c->N)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "query boundaries must run from 0 to num_data");
  int32_t max_q = 0;
  for (int32_t q = 0; q < num_queries; ++q) {
    const int32_t cnt = query_boundaries[q + 1] - query_boundaries[q];
    if (cnt < 0)
      return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "query boundaries must be non-decreasing");
    max_q = std::max(max_q, cnt);
  }
  if (max_q > RANK_MAX_QUERY)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "a query holds more than " + std::to_string(RANK_MAX_QUERY) + " rows");
  if (lambdarank_prepare(std::max(max_q, 1)))
    return set_err(c, LGBM_HIP_ERR_HIP, "the lambdarank kernel's LDS size was refused");
  std::vector<float> lab((size_t)c->N);
  HIPCHK(c, hipMemcpy(lab.data(), c->label, lab.size() * 4, hipMemcpyDeviceToHost));
  // DefaultLabelGain and the discounts (dcg_calculator.rs:48-90); labels checked as
  // DCGCalculator::check_labels does (integer, then in range)
  std::vector<double> gain(31, 0.0), disc(RANK_DISCOUNTS);
  for (int i = 1; i < 31; ++i) gain[(size_t)i] = (double)((1ll << i) - 1);
  for (int i = 0; i < RANK_DISCOUNTS; ++i) disc[(size_t)i] = 1.0 / std::log2(2.0 + (double)i);
  for (int64_t i = 0; i < c->N; ++i) {
    const float l = lab[(size_t)i];
    if (std::fabs(l - (float)rust_as_i32(l)) > 1e-15f)
      return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "ranking labels must be integers");
    if (l < 0.0f || rust_as_usize(l) >= gain.size())
      return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "ranking label outside the label gains");
  }
  std::vector<double> imd((size_t)num_queries);
  for (int32_t q = 0; q < num_queries; ++q) {
    const int32_t a = query_boundaries[q], cnt = query_boundaries[q + 1] - a;
    double m = max_dcg_at_k(gain, disc, truncation_level, lab.data() + a, cnt);
    imd[(size_t)q] = m > 0.0 ? 1.0 / m : m;
  }
  // ConstructSigmoidTable (rank.rs:170-182)
  RankParams rp{};
  rp.sigmoid = sigmoid;
  rp.min_in = -50.0 / sigmoid / 2.0;
  rp.max_in = -rp.min_in;
  rp.idx_factor = (double)RANK_SIGMOID_BINS / (rp.max_in - rp.min_in);
  rp.norm = norm ? 1 : 0;
  rp.trunc = truncation_level;
  std::vector<double> table(RANK_SIGMOID_BINS);
  for (int32_t i = 0; i < RANK_SIGMOID_BINS; ++i) {
    const double sc = (double)i / rp.idx_factor + rp.min_in;
    table[(size_t)i] = 1.0 / (1.0 + std::exp(sc * sigmoid));
  }
  if ((rc = dalloc(c, &c->rk_qb, (size_t)num_queries + 1))) return rc;
  if ((rc = dalloc(c, &c->rk_imd, (size_t)num_queries))) return rc;
  if ((rc = dalloc(c, &c->rk_table, (size_t)RANK_SIGMOID_BINS))) return rc;
  if ((rc = dalloc(c, &c->rk_disc, (size_t)RANK_DISCOUNTS))) return rc;
  if ((rc = dalloc(c, &c->rk_gain, gain.size()))) return rc;
  HIPCHK(c, hipMemcpy(c->rk_qb, query_boundaries, ((size_t)num_queries + 1) * 4, hipMemcpyHostToDevice));
  HIPCHK(c, hipMemcpy(c->rk_imd, imd.data(), imd.size() * 8, hipMemcpyHostToDevice));
  HIPCHK(c, hipMemcpy(c->rk_table, table.data(), table.size() * 8, hipMemcpyHostToDevice));
  HIPCHK(c, hipMemcpy(c->rk_disc, disc.data(), disc.size() * 8, hipMemcpyHostToDevice));
  HIPCHK(c, hipMemcpy(c->rk_gain, gain.data(), gain.size() * 8, hipMemcpyHostToDevice));
  RankTables& t = c->rank;
  t.qb = c->rk_qb;
  t.inv_max_dcg = c->rk_imd;
  t.table = c->rk_table;
  t.discount = c->rk_disc;
  t.gain = c->rk_gain;
  t.p = rp;
  t.num_queries = num_queries;
  t.max_query = std::max(max_q, 1);
  c->have_rank = true;
  c->objective = LGBM_HIP_OBJECTIVE_LAMBDARANK;
  return LGBM_HIP_OK;
}

int lgbm_hip_set_col_sampler(lgbm_hip_ctx* c, double feature_fraction,
                             double feature_fraction_bynode, int32_t seed) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_RUNTIME, "upload bins first");
  if (!(feature_fraction_bynode >= 1.0))
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "feature_fraction_bynode < 1 is not supported");
  if (!(feature_fraction > 0.0))
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "feature_fraction must be > 0");
  c->ahead = false;
  c->buf_gen++;  // the captured tree reads the mask pointer (or none)
  if (!(feature_fraction < 1.0)) {  // no sampling: no draws (col_sampler.rs:98-103)
    c->colsamp_on = false;
    return LGBM_HIP_OK;
  }
  if ((rc = dalloc(c, &c->d_feat_used, (size_t)c->F))) return rc;
  if (c->feat_used_host) (void)hipHostFree(c->feat_used_host);
  c->feat_used_host = nullptr;
  HIPCHK(c, hipHostMalloc((void**)&c->feat_used_host, (size_t)c->F, hipHostMallocDefault));
  c->colsamp.start(feature_fraction, seed, c->F);  // the construction draw
  c->colsamp_on = true;
  return LGBM_HIP_OK;
}

int lgbm_hip_boost_from_score(int32_t objective, const float* label, int64_t n, double* out) {
  if (!out || n < 0 || (n > 0 && !label)) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  if (objective == LGBM_HIP_OBJECTIVE_BINARY)
    return lgbm_hip_binary_boost_from_score(label, n, 1.0, out);
  if (objective == LGBM_HIP_OBJECTIVE_LAMBDARANK) {  // no init score (boosting objective.rs:112-116)
    *out = 0.0;
    return LGBM_HIP_OK;
  }
  if (objective != LGBM_HIP_OBJECTIVE_REGRESSION) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  // Objective::Regression::boost_from_score (regression.rs:563-575): the ordered
  // f64 label mean
  double sum = 0.0;
  for (int64_t i = 0; i < n; ++i) sum += (double)label[i];
  *out = n > 0 ? sum / (double)n : 0.0;
  return LGBM_HIP_OK;
}

int lgbm_hip_set_labels_multiclass(lgbm_hip_ctx* c, const float* labels, int64_t n,
                                   int32_t num_class, const double* init_scores) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;  // device inputs change: a pending lookahead is stale
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_RUNTIME, "upload bins first");
  if (!labels) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null labels");
  if (n != c->N) return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "labels length != num_data");
  if (num_class < 2 || num_class > 256)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_class must be in 2..=256");
  // MulticlassSoftmax::new (multiclass.rs:76-101): labels truncate toward zero (a
  // NaN to 0, the saturating cast) to class ids in [0, num_class)
  for (int64_t i = 0; i < n; ++i) {
    const double l = labels[i];
    if (l == l && (l <= -1.0 || l >= (double)num_class))
      return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT,
                     "label " + std::to_string(l) + " at row " + std::to_string(i) +
                         " is not a class in [0, num_class)");
  }
  c->have_labels = false;
  const size_t kn = (size_t)num_class * (size_t)n;
  if ((rc = dalloc(c, &c->label, (size_t)n))) return rc;
  if ((rc = dalloc(c, &c->score, kn))) return rc;
  if ((rc = dalloc(c, &c->gk, kn))) return rc;
  if ((rc = dalloc(c, &c->hk, kn))) return rc;
  HIPCHK(c, hipMemcpy(c->label, labels, (size_t)n * 4, hipMemcpyHostToDevice));
  std::vector<double> s(kn, 0.0);
  if (init_scores)
    for (int32_t k = 0; k < num_class; ++k)
      std::fill(s.begin() + (size_t)k * n, s.begin() + (size_t)(k + 1) * n, init_scores[k]);
  HIPCHK(c, hipMemcpy(c->score, s.data(), kn * 8, hipMemcpyHostToDevice));
  c->num_class = num_class;
  c->have_labels = true;
  c->have_rank = false;
  return LGBM_HIP_OK;
}

int lgbm_hip_train_iter_multiclass(lgbm_hip_ctx* c, int32_t iter, const lgbm_gain_config* cfg,
                                   int32_t num_leaves, int32_t max_depth, double learning_rate,
                                   int32_t num_grad_quant_bins, int32_t stochastic,
                                   const int32_t* class_need_train, lgbm_tree_out* trees) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;
  if (!c->have_labels || c->num_class < 2)
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "set multiclass labels first");
  if (!cfg) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null cfg");
  if (num_leaves < 1 || num_leaves > 256)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_leaves must be in 1..=256");
  if (num_grad_quant_bins < 0 || num_grad_quant_bins > 254)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "num_grad_quant_bins must be in 0..=254");
  if (num_grad_quant_bins == 1)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "num_grad_quant_bins 1 gives no gradient scale");
  const bool gen = gen_bins(num_grad_quant_bins);
  const int32_t fp = num_grad_quant_bins == 0 || gen ? 1 : 0;
  if (!fp && c->N >= QUANT_MAX_ROWS)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY, "quantized int32 histogram cells need N < 2^29");
  if (!fp && !rec_wide(c->fmt) && c->total_cells > QUANT_LDS_CELLS)
    return set_err(c, LGBM_HIP_ERR_CAPABILITY,
                   "quantized histograms hold every cell in LDS: at most 8192 (feature, bin) cells");
  if (trees)
    for (int32_t k = 0; k < c->num_class; ++k)
      if (!(class_need_train && !class_need_train[k]) &&
          (rc = check_cat_capacity(c, &trees[k], num_leaves)))
        return rc;
  if ((rc = ensure_leaves(c, num_leaves))) return rc;
  if (fp && (rc = ensure_fp(c))) return rc;
  if (gen && (rc = ensure_dq(c))) return rc;
  const int32_t K = c->num_class;
  const int64_t N = c->N;
  // factor = K / (K - 1) (multiclass.rs:84)
  const double factor = (double)K / ((double)K - 1.0);
  timing_hold(c);
  ev_begin(c, FAM_OBJ);
  launch_grad_softmax(c->score, c->label, c->gk, c->hk, N, K, factor, c->stream);
  ev_end(c);
  HIPCHK(c, hipGetLastError());
  for (int32_t k = 0; k < K; ++k) {
    lgbm_tree_out* out = trees ? &trees[k] : nullptr;
    if (class_need_train && !class_need_train[k]) {
      // class_need_train gate (gbdt.rs:1003-1018): no tree for this class
      if (out) out->num_leaves = 0;
      continue;
    }
    const float* gk = c->gk + (size_t)k * N;
    const float* hk = c->hk + (size_t)k * N;
    if (k > 0) timing_hold(c);
    DevLearner L0 = make_learner(c);
    if (num_grad_quant_bins == 0) {
      ev_begin(c, FAM_QUANT);
      launch_fp_prep(L0, gk, hk, N, c->partials, c->stream);
      ev_end(c);
      c->quant_ready = false;
    } else {
      // per-(iteration, class) seed (gbdt.rs:946-958)
      const uint64_t seed = ((uint64_t)(uint32_t)iter << 20) ^ (uint64_t)(uint32_t)k ^ 0x51702010ull;
      ev_begin(c, FAM_QUANT);
      launch_absmax(gk, hk, N, c->partials, c->stream);
      launch_quant_scales(c->ctl, c->partials, N, num_grad_quant_bins, -1, c->stream);
      launch_quantize(gk, hk, N, c->ctl, c->wave_mats, c->lane_mats, seed ^ 0x9E3779B97F4A7C15ull,
                      stochastic, c->gh[BUF_ORIG], gen ? c->dq : nullptr,
                      gen ? c->dq + N : nullptr, c->stream);
      if (gen) launch_exact_prep(L0, c->dq, c->dq + N, N, c->stream);
      ev_end(c);
      c->quant_ready = true;
      c->quant_bins = num_grad_quant_bins;
    }
    HIPCHK(c, hipGetLastError());
    c->have_grad = false;  // c->g / c->h do not hold this class's gradients
    if ((rc = grow_tree_async(c, cfg, num_leaves, max_depth, fp))) return rc;
    if (num_grad_quant_bins > 0 && c->renew_leaf &&
        (rc = renew_leaves(c, num_leaves, gk, hk, cfg)))
      return rc;
    DevLearner L = make_learner(c);
    KernelEvents ke;
    launch_score_update(L, learning_rate, c->score + (size_t)k * N, c->stream,
                        ev_kernel(c, FAM_OBJ, &ke));
    HIPCHK(c, hipGetLastError());
    if ((rc = finish_tree(c, out, nullptr, learning_rate))) return rc;
  }
  return LGBM_HIP_OK;
}

int lgbm_hip_get_multiclass_gradients(lgbm_hip_ctx* c, float* grad, float* hess, int64_t n) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!c->have_labels || c->num_class < 2 || !c->gk)
    return set_err(c, LGBM_HIP_ERR_RUNTIME, "no multiclass gradients yet");
  if (n != (int64_t)c->num_class * c->N)
    return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "n != num_class * num_data");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (grad) HIPCHK(c, hipMemcpy(grad, c->gk, (size_t)n * 4, hipMemcpyDeviceToHost));
  if (hess) HIPCHK(c, hipMemcpy(hess, c->hk, (size_t)n * 4, hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

int lgbm_hip_set_quant_renew_leaf(lgbm_hip_ctx* c, int32_t enable) {
  int rc = check_ctx(c);
  if (rc) return rc;
  c->ahead = false;
  if (!enable) {
    c->renew_leaf = false;
    return LGBM_HIP_OK;
  }
  if (!c->have_bins) return set_err(c, LGBM_HIP_ERR_RUNTIME, "upload bins first");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  c->renew_leaf = false;
  if ((rc = dalloc(c, &c->renew_idx, (size_t)c->N))) return rc;
  if ((rc = dalloc(c, (char**)&c->renew_scratch, export_layout_scratch_bytes(c->N, MAX_LEAVES))))
    return rc;
  c->renew_rows = c->N;
  c->renew_leaf = true;
  return LGBM_HIP_OK;
}

int lgbm_hip_set_lookahead(lgbm_hip_ctx* c, int32_t enable) {
  int rc = check_ctx(c);
  if (rc) return rc;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  c->lookahead = enable != 0;
  c->ahead = false;
  return LGBM_HIP_OK;
}

int lgbm_hip_binary_boost_from_score(const float* label, int64_t n, double sigmoid, double* out) {
  if (!out || n < 0 || (n > 0 && !label) || !(sigmoid > 0.0)) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  // BinaryLogloss::boost_from_score (binary.rs:178-192): log-odds of the positive
  // fraction, clamped to [kEpsilon, 1 - kEpsilon]
  if (n == 0) {
    *out = 0.0;
    return LGBM_HIP_OK;
  }
  double pos = 0.0;
  for (int64_t i = 0; i < n; ++i) pos += label[i] > 0.0f ? 1.0 : 0.0;
  const double eps = (double)1e-15f;
  const double pavg = std::max(std::min(pos / (double)n, 1.0 - eps), eps);
  *out = std::log(pavg / (1.0 - pavg)) / sigmoid;
  return LGBM_HIP_OK;
}

int lgbm_hip_get_gradients(lgbm_hip_ctx* c, float* grad, float* hess, int64_t n) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!c->have_grad) return set_err(c, LGBM_HIP_ERR_RUNTIME, "no gradients yet");
  if (n != c->N) return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "n != num_data");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (grad) HIPCHK(c, hipMemcpy(grad, c->g, (size_t)n * 4, hipMemcpyDeviceToHost));
  if (hess) HIPCHK(c, hipMemcpy(hess, c->h, (size_t)n * 4, hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

int lgbm_hip_get_scores(lgbm_hip_ctx* c, double* out, int64_t n) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!c->have_labels) return set_err(c, LGBM_HIP_ERR_RUNTIME, "set labels first");
  if (!out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null out");
  if (n != (int64_t)c->num_class * c->N)
    return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH, "n != num_class * num_data");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  HIPCHK(c, hipMemcpy(out, c->score, (size_t)n * 8, hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

int lgbm_hip_set_timing(lgbm_hip_ctx* c, int32_t enable) {
  int rc = check_ctx(c);
  if (rc) return rc;
  HIPCHK(c, hipStreamSynchronize(c->stream));
  ev_collect(c);
  c->timing = enable != 0;
  if (c->timing && !c->hold_ticks) {
    int khz = 0;
    HIPCHK(c, hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, c->device));
    c->hold_ticks = (uint64_t)std::max(khz, 1) * 10;  // 10 ms
  }
  for (double& m : c->ms) m = 0.0;
  HIPCHK(c, hipMemset(c->stats, 0, 64));
  c->tree_rounds = c->trees = c->extra_rounds = c->part_launches = 0.0;
  c->bin_launches = c->bin_values = c->pred_launches = c->pred_walks = 0.0;
  return LGBM_HIP_OK;
}

int lgbm_hip_get_timing(lgbm_hip_ctx* c, double* ms_out5, double* hist_bytes_out,
                        int64_t* hist_launches_out) {
  double st[23];
  int rc = lgbm_hip_get_stats(c, st);
  if (rc) return rc;
  if (ms_out5)
    for (int i = 0; i < 5; ++i) ms_out5[i] = st[i];
  // root ConstructHistogram algorithmic bytes: rows x (F bins + 2 B packed g/h)
  // + the histogram write (cells x 2 x 4 B) per launch
  if (hist_bytes_out) *hist_bytes_out = st[5] * (st[10] + 2.0) + st[6] * st[11] * 8.0;
  if (hist_launches_out) *hist_launches_out = (int64_t)(st[6] + 0.5);
  return LGBM_HIP_OK;
}

int lgbm_hip_get_stats(lgbm_hip_ctx* c, double* out) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null out");
  HIPCHK(c, hipStreamSynchronize(c->stream));
  ev_collect(c);
  double st[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  HIPCHK(c, hipMemcpy(st, c->stats, 64, hipMemcpyDeviceToHost));
  for (int i = 0; i < 5; ++i) out[i] = c->ms[i];
  out[5] = st[2];
  out[6] = st[3];
  out[7] = st[0];
  out[8] = c->part_launches;
  out[9] = (double)(rec_bytes(c->fmt) + (rec_packed(c->fmt) ? 0 : 2));
  out[10] = c->F;
  out[11] = c->total_cells;
  out[12] = st[4];
  out[13] = c->tree_rounds;
  out[14] = c->trees;
  out[15] = c->extra_rounds;
  out[16] = c->ms[FAM_BIN];
  out[17] = c->bin_launches;
  out[18] = c->bin_values;
  out[19] = c->ms[FAM_PRED];
  out[20] = c->pred_launches;
  out[21] = c->pred_walks;
  out[22] = st[5];
  return LGBM_HIP_OK;
}

// ---- models and batch prediction ---------------------------------------------

int lgbm_hip_model_load(const char* text, int64_t len, lgbm_hip_model** out) {
  if (!text || !out || len < 0) {
    g_model_err = "null text/out or negative length";
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  *out = nullptr;
  lgbm_hip_model* m = new lgbm_hip_model();
  std::string err;
  if (!parse_model_text(text, (size_t)len, m, &err)) {
    delete m;
    g_model_err = err;
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  *out = m;
  return LGBM_HIP_OK;
}

int lgbm_hip_model_free(lgbm_hip_model* model) {
  delete model;
  return LGBM_HIP_OK;
}

int lgbm_hip_model_last_error(char* buf, size_t size) {
  if (buf && size > 0) {
    std::snprintf(buf, size, "%s", g_model_err.c_str());
  }
  return LGBM_HIP_OK;
}

int lgbm_hip_model_create(int32_t num_class, int32_t num_tree_per_iteration,
                          int32_t max_feature_idx, const char* objective,
                          const char* feature_names, const char* feature_infos,
                          lgbm_hip_model** out) {
  if (!out || num_class < 1 || num_tree_per_iteration < 1 || max_feature_idx < 0) {
    g_model_err = "null out, or num_class / num_tree_per_iteration < 1, or max_feature_idx < 0";
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  *out = nullptr;
  lgbm_hip_model* m = new lgbm_hip_model();
  m->num_class = num_class;
  m->num_tree_per_iteration = num_tree_per_iteration;
  m->max_feature_idx = max_feature_idx;
  std::string err;
  if (objective && !model_set_objective(m, objective, &err)) {
    delete m;
    g_model_err = err;
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  // Dataset defaults (`Column_<i>` names, `none` infos) for the columns not named.
  auto fill = [&](const char* given, std::string* dst, bool names) {
    if (given) {
      *dst = given;
      return;
    }
    for (int32_t f = 0; f <= max_feature_idx; ++f) {
      if (f) *dst += ' ';
      *dst += names ? "Column_" + std::to_string(f) : std::string("none");
    }
  };
  fill(feature_names, &m->feature_names, true);
  fill(feature_infos, &m->feature_infos, false);
  *out = m;
  return LGBM_HIP_OK;
}

int lgbm_hip_model_add_tree(lgbm_hip_model* m, const lgbm_tree_out* t, double shrinkage,
                            double bias) {
  if (!m || !t || t->num_leaves < 1) {
    g_model_err = "null model/tree or num_leaves < 1";
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  const int32_t nl = t->num_leaves, ni = nl - 1;
  if (!t->leaf_value || (ni > 0 && (!t->split_feature || !t->threshold || !t->decision_type ||
                                    !t->left_child || !t->right_child))) {
    g_model_err = "tree without leaf_value or a structural array";
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  HostTree h;
  h.num_leaves = nl;
  h.num_cat = 0;
  h.shrinkage = shrinkage;
  auto take = [](auto* dst, const auto* src, int32_t n) {
    using T = typename std::remove_reference<decltype(*dst)>::type::value_type;
    dst->resize((size_t)n);
    for (int32_t i = 0; i < n; ++i) (*dst)[(size_t)i] = src ? (T)src[i] : T(0);
  };
  take(&h.split_feature, t->split_feature, ni);
  take(&h.threshold, t->threshold, ni);
  take(&h.decision_type, t->decision_type, ni);
  take(&h.left_child, t->left_child, ni);
  take(&h.right_child, t->right_child, ni);
  take(&h.split_gain, t->split_gain, ni);
  take(&h.internal_value, t->internal_value, ni);
  take(&h.internal_count, t->internal_count, ni);
  take(&h.internal_weight, t->internal_weight, ni);  // NULL: 0, as tree.rs:655 stores
  take(&h.leaf_value, t->leaf_value, nl);
  if (nl > 1) take(&h.leaf_weight, t->leaf_weight, nl);  // constant tree: empty, as C++ writes it
  take(&h.leaf_count, t->leaf_count, nl);
  if (bias != 0.0) {
    // Tree::add_bias (tree.rs:1161): MaybeRoundToZero(v + bias)
    const double z = (double)1e-35f;
    auto mrz = [z](double v) { return (v >= -z && v <= z) ? 0.0 : v; };
    for (double& v : h.leaf_value) v = mrz(v + bias);
    for (double& v : h.internal_value) v = mrz(v + bias);
    h.shrinkage = 1.0;  // AddBias forces shrinkage_ to 1 (the model texts' first trees)
  }
  std::string err;
  if (!model_add_tree(m, std::move(h), &err)) {
    g_model_err = err;
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  }
  return LGBM_HIP_OK;
}

int lgbm_hip_model_to_text(const lgbm_hip_model* m, char* buf, size_t size, size_t* needed) {
  if (!m) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  const std::string s = model_to_text(*m);
  if (needed) *needed = s.size() + 1;
  if (buf && size > 0) {
    const size_t n = std::min(size - 1, s.size());
    std::memcpy(buf, s.data(), n);
    buf[n] = '\0';
  }
  return buf && size < s.size() + 1 ? LGBM_HIP_ERR_LENGTH_MISMATCH : LGBM_HIP_OK;
}

int lgbm_hip_model_info(const lgbm_hip_model* m, int64_t* out) {
  if (!m || !out) return LGBM_HIP_ERR_INVALID_ARGUMENT;
  out[0] = (int64_t)m->trees.size();
  out[1] = m->num_class;
  out[2] = m->num_tree_per_iteration;
  out[3] = m->max_feature_idx;
  out[4] = (int64_t)m->trees.size() / m->num_tree_per_iteration;
  out[5] = m->objective;
  return LGBM_HIP_OK;
}

}  // extern "C"

namespace {

template <typename T>
int upload_vec(lgbm_hip_ctx* c, T** dst, const std::vector<T>& v) {
  int rc = dalloc(c, dst, v.size());
  if (rc) return rc;
  if (!v.empty()) HIPCHK(c, hipMemcpy(*dst, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
  return LGBM_HIP_OK;
}

// Validates the call, uploads the model when it is not the cached one, and returns
// the clamped iteration range and output width.
int predict_prepare(lgbm_hip_ctx* c, const lgbm_hip_model* m, int64_t rows, int32_t cols,
                    int32_t start_iteration, int32_t num_iteration, int32_t kind, int32_t* it0,
                    int32_t* it1, int64_t* width) {
  int rc = check_ctx(c);
  if (rc) return rc;
  if (!m) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null model");
  if (rows < 0 || cols < 0) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "negative shape");
  if (cols < m->max_feature_idx + 1)
    return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH,
                   "input has " + std::to_string(cols) + " columns, model needs max_feature_idx+1 = " +
                       std::to_string(m->max_feature_idx + 1));
  if (kind < LGBM_HIP_PREDICT_RAW || kind > LGBM_HIP_PREDICT_CONTRIB)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "unknown prediction kind");
  if (kind == LGBM_HIP_PREDICT_CONTRIB && m->any_linear)  // check_no_linear_trees (predict.rs:626-635)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT,
                   "feature contributions are not supported for linear_tree models");
  if (kind == LGBM_HIP_PREDICT_TRANSFORMED) {
    // resolve_objective (predict.rs:305-322)
    if (!m->have_objective)
      return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT,
                     "model has no objective= line; cannot apply ConvertOutput");
    if (m->objective_outputs != m->num_tree_per_iteration)
      return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT,
                     "objective output width " + std::to_string(m->objective_outputs) +
                         " != num_tree_per_iteration " + std::to_string(m->num_tree_per_iteration));
  }
  // GbdtModel::init_predict (ensemble.rs:75-84)
  const int32_t total = (int32_t)(m->trees.size() / m->num_tree_per_iteration);
  const int32_t start = std::min(std::max(start_iteration, 0), total);
  const int32_t num = num_iteration > 0 ? std::min(num_iteration, total - start) : total - start;
  *it0 = start;
  *it1 = start + num;
  *width = kind == LGBM_HIP_PREDICT_LEAF ? (int64_t)num * m->num_tree_per_iteration
           : kind == LGBM_HIP_PREDICT_CONTRIB
               ? (int64_t)m->num_tree_per_iteration * (m->max_feature_idx + 2)
               : (int64_t)m->num_tree_per_iteration;
  if (c->pm_uid != m->uid) {
    c->pm_uid = 0;  // a partial upload must not pass for the cached model
    if ((rc = upload_vec(c, &c->pm_nodes, m->nodes))) return rc;
    if ((rc = upload_vec(c, &c->pm_trees, m->tree_index))) return rc;
    if ((rc = upload_vec(c, &c->pm_leaves, m->leaf_values))) return rc;
    if ((rc = upload_vec(c, &c->pm_catb, m->cat_bounds))) return rc;
    if ((rc = upload_vec(c, &c->pm_catw, m->cat_words))) return rc;
    if ((rc = upload_vec(c, &c->pm_linl, m->lin_leaves))) return rc;
    if ((rc = upload_vec(c, &c->pm_linf, m->lin_features))) return rc;
    if ((rc = upload_vec(c, &c->pm_linc, m->lin_coeffs))) return rc;
    if ((rc = upload_vec(c, &c->pm_ncov, m->node_cover))) return rc;
    if ((rc = upload_vec(c, &c->pm_lcov, m->leaf_cover))) return rc;
    if ((rc = upload_vec(c, &c->pm_expv, m->tree_expected))) return rc;
    c->pm_uid = m->uid;
  }
  return LGBM_HIP_OK;
}

int predict_run(lgbm_hip_ctx* c, const lgbm_hip_model* m, const float* d_x, int64_t rows,
                int32_t cols, int32_t it0, int32_t it1, int32_t kind, void* d_out,
                int32_t es_freq = 0, double es_margin = 0.0, int32_t* d_iters = nullptr) {
  if (kind == LGBM_HIP_PREDICT_CONTRIB) {
    // the deepest tree of the range sizes each row's path buffer; rows go in chunks
    // whose workspace stays within 256 MiB
    int32_t depth = 0;
    for (int64_t t = (int64_t)it0 * m->num_tree_per_iteration;
         t < (int64_t)it1 * m->num_tree_per_iteration; ++t)
      depth = std::max(depth, m->tree_depth[t]);
    const int64_t per_row = shap_bytes_per_row(depth);
    int64_t chunk = std::max<int64_t>(256, ((int64_t)256 << 20) / per_row / 256 * 256);
    chunk = std::min(chunk, rows);
    const size_t need = (size_t)(per_row * chunk);
    if (c->pm_shap_cap < need) {
      c->pm_shap_cap = 0;  // dalloc frees the old workspace first
      int rc = dalloc(c, &c->pm_shap, need);
      if (rc) return rc;
      c->pm_shap_cap = need;
    }
    for (int64_t r0 = 0; r0 < rows; r0 += chunk)
      launch_contrib(c->pm_nodes, c->pm_trees, c->pm_leaves, c->pm_catb, c->pm_catw, c->pm_ncov,
                     c->pm_lcov, c->pm_expv, d_x, r0, std::min(chunk, rows - r0), rows, cols,
                     m->max_feature_idx + 1, it0, it1, m->num_tree_per_iteration, depth,
                     c->pm_shap, (double*)d_out, c->stream, nullptr);
    HIPCHK(c, hipGetLastError());
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return LGBM_HIP_OK;
  }
  KernelEvents ke;
  launch_predict(c->pm_nodes, c->pm_trees, c->pm_leaves, c->pm_catb, c->pm_catw, c->pm_linl,
                 c->pm_linf, c->pm_linc, d_x, rows, cols,
                 it0, it1, m->num_tree_per_iteration, kind, m->objective, m->sigmoid,
                 m->average_output ? 1 : 0, es_freq, es_margin, d_iters,
                 kind == LGBM_HIP_PREDICT_LEAF ? nullptr : (double*)d_out,
                 kind == LGBM_HIP_PREDICT_LEAF ? (int32_t*)d_out : nullptr, c->stream,
                 ev_kernel(c, FAM_PRED, &ke));
  if (c->timing) {
    c->pred_launches += 1.0;
    c->pred_walks += (double)rows * (double)(it1 - it0) * m->num_tree_per_iteration;
  }
  HIPCHK(c, hipGetLastError());
  HIPCHK(c, hipStreamSynchronize(c->stream));
  return LGBM_HIP_OK;
}

}  // namespace

extern "C" {

int lgbm_hip_predict(lgbm_hip_ctx* c, const lgbm_hip_model* m, const float* data, int64_t rows,
                     int32_t cols, int32_t start_iteration, int32_t num_iteration, int32_t kind,
                     void* out) {
  int32_t it0 = 0, it1 = 0;
  int64_t width = 0;
  int rc = predict_prepare(c, m, rows, cols, start_iteration, num_iteration, kind, &it0, &it1, &width);
  if (rc) return rc;
  if (rows == 0 || width == 0) return LGBM_HIP_OK;
  if (!data || !out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null data/out");
  const size_t xb = (size_t)rows * (size_t)cols * 4;
  const size_t ob = (size_t)rows * (size_t)width * (kind == LGBM_HIP_PREDICT_LEAF ? 4 : 8);
  if (c->pm_x_cap < xb) {
    c->pm_x_cap = 0;  // dalloc frees the old staging first
    if ((rc = dalloc(c, &c->pm_x, (size_t)rows * (size_t)cols))) return rc;
    c->pm_x_cap = xb;
  }
  if (c->pm_out_cap < ob) {
    char* p = nullptr;
    if ((rc = dalloc(c, &p, ob))) return rc;
    if (c->pm_out) (void)hipFree(c->pm_out);
    c->pm_out = p;
    c->pm_out_cap = ob;
  }
  HIPCHK(c, hipMemcpy(c->pm_x, data, xb, hipMemcpyHostToDevice));
  if ((rc = predict_run(c, m, c->pm_x, rows, cols, it0, it1, kind, c->pm_out))) return rc;
  HIPCHK(c, hipMemcpy(out, c->pm_out, ob, hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

int lgbm_hip_predict_device(lgbm_hip_ctx* c, const lgbm_hip_model* m, const float* d_data,
                            int64_t rows, int32_t cols, int32_t start_iteration,
                            int32_t num_iteration, int32_t kind, void* d_out) {
  int32_t it0 = 0, it1 = 0;
  int64_t width = 0;
  int rc = predict_prepare(c, m, rows, cols, start_iteration, num_iteration, kind, &it0, &it1, &width);
  if (rc) return rc;
  if (rows == 0 || width == 0) return LGBM_HIP_OK;
  if (!d_data || !d_out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null data/out");
  return predict_run(c, m, d_data, rows, cols, it0, it1, kind, d_out);
}

}  // extern "C"

namespace {
// CSR (csc = false) or CSC rows made dense on the device, then predicted.
int predict_sparse(lgbm_hip_ctx* c, const lgbm_hip_model* m, const int64_t* indptr,
                   const int32_t* indices, const float* values, int64_t nnz, int64_t num_rows,
                   int32_t num_cols, int32_t start_iteration, int32_t num_iteration, int32_t kind,
                   void* out, bool csc) {
  int32_t it0 = 0, it1 = 0;
  int64_t width = 0;
  int rc = predict_prepare(c, m, num_rows, num_cols, start_iteration, num_iteration, kind, &it0,
                           &it1, &width);
  if (rc) return rc;
  if (nnz < 0) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "negative nnz");
  if (csc && nnz >= (int64_t)UINT32_MAX)  // the densify claims cells with k + 1 in 32 bits
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "csc input of 2^32 - 1 entries or more");
  if (!indptr || (nnz > 0 && (!indices || !values)))
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null indptr/indices/values");
  if (num_rows == 0 || width == 0) return LGBM_HIP_OK;
  if (!out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null out");
  const int32_t fw = m->max_feature_idx + 1;  // the dense rows the model reads
  const size_t pb = (size_t)((csc ? (int64_t)num_cols : num_rows) + 1) * 8, ib = (size_t)nnz * 4;
  const size_t need = 256 + pb + 2 * ib;
  if (c->pm_csr_cap < need) {
    c->pm_csr_cap = 0;  // dalloc frees the old staging first
    if ((rc = dalloc(c, &c->pm_csr, need))) return rc;
    c->pm_csr_cap = need;
  }
  uint32_t* d_err = (uint32_t*)c->pm_csr;
  int64_t* d_ptr = (int64_t*)(c->pm_csr + 256);
  int32_t* d_idx = (int32_t*)(c->pm_csr + 256 + pb);
  float* d_val = (float*)(c->pm_csr + 256 + pb + ib);
  const size_t xb = (size_t)num_rows * (size_t)std::max(fw, 1) * 4;
  const size_t ob = (size_t)num_rows * (size_t)width * (kind == LGBM_HIP_PREDICT_LEAF ? 4 : 8);
  if (c->pm_x_cap < xb) {
    c->pm_x_cap = 0;  // dalloc frees the old staging first
    if ((rc = dalloc(c, &c->pm_x, xb / 4))) return rc;
    c->pm_x_cap = xb;
  }
  if (c->pm_out_cap < ob) {
    char* p = nullptr;
    if ((rc = dalloc(c, &p, ob))) return rc;
    if (c->pm_out) (void)hipFree(c->pm_out);
    c->pm_out = p;
    c->pm_out_cap = ob;
  }
  const uint32_t zero = 0;
  HIPCHK(c, hipMemcpy(d_err, &zero, 4, hipMemcpyHostToDevice));
  HIPCHK(c, hipMemcpy(d_ptr, indptr, pb, hipMemcpyHostToDevice));
  if (nnz > 0) {
    HIPCHK(c, hipMemcpy(d_idx, indices, ib, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(d_val, values, ib, hipMemcpyHostToDevice));
  }
  HIPCHK(c, hipMemsetAsync(c->pm_x, 0, (size_t)num_rows * (size_t)fw * 4, c->stream));
  if (csc) {
    launch_csc_dense(d_ptr, d_idx, d_val, nnz, num_rows, num_cols, fw, c->pm_x, d_err, c->stream);
  } else {
    launch_csr_dense(d_ptr, d_idx, d_val, nnz, num_rows, num_cols, fw, c->pm_x, d_err, c->stream);
  }
  HIPCHK(c, hipGetLastError());
  uint32_t bad = 0;
  HIPCHK(c, hipMemcpyAsync(&bad, d_err, 4, hipMemcpyDeviceToHost, c->stream));
  HIPCHK(c, hipStreamSynchronize(c->stream));
  if (bad & 1u) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "malformed indptr");
  if (bad & 2u)
    return set_err(c, LGBM_HIP_ERR_LENGTH_MISMATCH,
                   csc ? "csc row index out of range" : "csr column index out of range");
  if ((rc = predict_run(c, m, c->pm_x, num_rows, fw, it0, it1, kind, c->pm_out))) return rc;
  HIPCHK(c, hipMemcpy(out, c->pm_out, ob, hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}
}  // namespace

extern "C" {

int lgbm_hip_predict_csr(lgbm_hip_ctx* c, const lgbm_hip_model* m, const int64_t* indptr,
                         const int32_t* indices, const float* values, int64_t nnz,
                         int64_t num_rows, int32_t num_cols, int32_t start_iteration,
                         int32_t num_iteration, int32_t kind, void* out) {
  return predict_sparse(c, m, indptr, indices, values, nnz, num_rows, num_cols, start_iteration,
                        num_iteration, kind, out, false);
}

int lgbm_hip_predict_csc(lgbm_hip_ctx* c, const lgbm_hip_model* m, const int64_t* indptr,
                         const int32_t* indices, const float* values, int64_t nnz,
                         int64_t num_rows, int32_t num_cols, int32_t start_iteration,
                         int32_t num_iteration, int32_t kind, void* out) {
  return predict_sparse(c, m, indptr, indices, values, nnz, num_rows, num_cols, start_iteration,
                        num_iteration, kind, out, true);
}

int lgbm_hip_predict_early_stop(lgbm_hip_ctx* c, const lgbm_hip_model* m, const float* data,
                                int64_t rows, int32_t cols, int32_t start_iteration,
                                int32_t num_iteration, int32_t freq, double margin, double* out,
                                int32_t* iterations) {
  int32_t it0 = 0, it1 = 0;
  int64_t width = 0;
  int rc = predict_prepare(c, m, rows, cols, start_iteration, num_iteration, LGBM_HIP_PREDICT_RAW,
                           &it0, &it1, &width);
  if (rc) return rc;
  if (rows == 0) return LGBM_HIP_OK;
  if (!data || !out) return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT, "null data/out");
  // resolve_objective + the C++ Predictor gate (predict.rs:557-605): objectives that
  // need accurate prediction evaluate the whole range
  if (!m->have_objective)
    return set_err(c, LGBM_HIP_ERR_INVALID_ARGUMENT,
                   "model has no objective= line; cannot apply ConvertOutput");
  const bool accurate = !(m->objective == OBJ_BINARY || m->objective == OBJ_MULTICLASS ||
                          m->objective == OBJ_MULTICLASS_OVA);
  const int32_t f = accurate ? 0 : freq;
  const size_t xb = (size_t)rows * (size_t)cols * 4, ob = (size_t)rows * (size_t)width * 8;
  if (c->pm_x_cap < xb) {
    c->pm_x_cap = 0;  // dalloc frees the old staging first
    if ((rc = dalloc(c, &c->pm_x, (size_t)rows * (size_t)cols))) return rc;
    c->pm_x_cap = xb;
  }
  const size_t need = ob + (size_t)rows * 4;
  if (c->pm_out_cap < need) {
    char* p = nullptr;
    if ((rc = dalloc(c, &p, need))) return rc;
    if (c->pm_out) (void)hipFree(c->pm_out);
    c->pm_out = p;
    c->pm_out_cap = need;
  }
  int32_t* d_iters = (int32_t*)((char*)c->pm_out + ob);
  HIPCHK(c, hipMemcpy(c->pm_x, data, xb, hipMemcpyHostToDevice));
  if (f <= 0) {
    // the whole range: raw scores, every row evaluating every iteration
    if ((rc = predict_run(c, m, c->pm_x, rows, cols, it0, it1, LGBM_HIP_PREDICT_RAW, c->pm_out)))
      return rc;
    HIPCHK(c, hipMemcpy(out, c->pm_out, ob, hipMemcpyDeviceToHost));
    if (iterations)
      for (int64_t r = 0; r < rows; ++r) iterations[r] = it1 - it0;
    return LGBM_HIP_OK;
  }
  if ((rc = predict_run(c, m, c->pm_x, rows, cols, it0, it1, LGBM_HIP_PREDICT_RAW, c->pm_out, f,
                        margin, d_iters)))
    return rc;
  HIPCHK(c, hipMemcpy(out, c->pm_out, ob, hipMemcpyDeviceToHost));
  if (iterations) HIPCHK(c, hipMemcpy(iterations, d_iters, (size_t)rows * 4, hipMemcpyDeviceToHost));
  return LGBM_HIP_OK;
}

}  // extern "C"
