// grow.hip — the leaf-wise tree driver on device, in rounds of partition jobs.
//
// The reference grows a tree best-first (SerialTreeLearner::train_inner,
// crates/lgbm-treelearner/src/learner.rs:980-1562): split the leaf of highest gain
// (ArgMax, learner.rs:4537), build the smaller child's histogram, derive the larger
// one by subtraction, scan both, repeat.  Everything a split computes for its two
// children depends only on the split leaf itself (its rows, histogram, sums, depth
// and feature mask), never on the rest of the tree.  So each round here splits up to
// SPEC_MAX leaves at once — the best-ranked leaves that are not split yet — and the
// plan kernel then commits finished splits to the tree strictly in the reference's
// ArgMax order, assigning leaf ids and node numbers exactly as Tree::split does.
// A leaf split ahead of its turn that the reference never splits costs only the
// wasted pass; the tree is the reference's tree either way.
//
//   k_tree_init    per-tree reset (DataPartition::new, root LeafSplits; learner.rs:
//                  1242-1376)
//   k_plan         per-leaf feature ArgMax of the children scanned last round
//                  (learner.rs:3290-3330), commit loop (ArgMax + stop test,
//                  learner.rs:1503, 4537; Tree::split bookkeeping, tree.rs:614-700),
//                  selection of the next round's leaves and their partition jobs
//                  (split_inner router, learner.rs:3895-4011)
//   k_partition    DataPartition::split of every job of the round
//                  (data_partition.rs:192-288,360-463) + the ConstructHistogram of
//                  one child per job, accumulated while its rows are in registers
//   k_pair_scan    per (feature, job): integer other-child = parent - built child,
//                  exact f64 cells of the smaller child, FixHistogram, compaction,
//                  larger = parent - smaller (histogram_pool.rs:249), and
//                  FindBestThreshold of both children (kernels/split.rs:8970-9329)
//   k_tree_finalize  leaf arrays of the Tree and the LeafPartitionLayout ranges
#include "scan.h"

#include <hip/hip_ext.h>

#include <algorithm>

namespace lgbm {

#define PLAN_WAVES (PLAN_THREADS / LGBM_WAVE)
#define INT_MAX32 0x7fffffff
// plan_state rows (MAX_LEAVES entries each): the tree's leaf -> node-slot map and
// linkage, owned by k_plan and copied into the Tree by k_tree_finalize.
#define PS_LEAF_SLOT 0    // committed leaf id -> node slot
#define PS_LEAF_SIDE 1    // 1: the leaf is its parent node's right child
#define PS_LEAF_PARENT 2  // Tree::leaf_parent
#define PS_NODE_LEFT 3    // Tree::left_child
#define PS_NODE_RIGHT 4   // Tree::right_child


// SplitInner router inputs (split_inner, learner.rs:3957; data_partition.rs:387-417).
__device__ __forceinline__ void router_of(const DevFeature& ft, const lgbm_split_info& b,
                                          int32_t* pmin, int32_t* th, int32_t* flags) {
  const int32_t pm = (int32_t)ft.min_bin + max(ft.offset, 0);
  int32_t thr = (int32_t)b.threshold + pm;
  if (ft.mfb == 0) thr -= 1;
  int32_t fl = 0;
  if ((int32_t)ft.mfb > (int32_t)b.threshold) fl |= 1;
  if (ft.na_as_missing) fl |= 2;
  if (b.default_left) fl |= 4;
  *pmin = pm;
  *th = thr;
  *flags = fl;
}

// ===========================================================================
// per-tree reset
// ===========================================================================
__global__ void k_tree_init(DevLearner L, int32_t max_leaves, int32_t max_depth, int32_t slot_cap,
                            int32_t spec_max, int32_t fp_mode) {
  Ctl* ctl = L.ctl;
  const int tid = blockIdx.x * blockDim.x + threadIdx.x;
  const int nthr = gridDim.x * blockDim.x;
  for (int i = tid; i < L.F; i += nthr) L.splittable[i] = 1;  // node slot 0
  if (rec_wide(L.fmt)) {
    // the histogram cells go to per-chunk slots that every launch overwrites; the
    // totals cells gather atomic adds of the root build (job 0)
    for (int j = tid; j < SPEC_MAX; j += nthr) {
      const size_t t = (size_t)j * L.acc_cells + L.total_cells;
      if (fp_mode) {
        L.hist_acc64[2 * t] = 0;
        L.hist_acc64[2 * t + 1] = 0;
      } else {
        L.hist_acc[3 * t] = 0;
        L.hist_acc[3 * t + 1] = 0;
        L.hist_acc[3 * t + 2] = 0;
      }
    }
  } else {
    for (int i = tid; i < SPEC_MAX * L.acc_cells * 3; i += nthr) L.hist_acc[i] = 0;
    for (int i = tid; i < SPEC_MAX * L.acc_cells; i += nthr) L.hist_accp[i] = 0ull;
  }
  if (tid == 0) {
    const int32_t N = (int32_t)L.N;
    ctl->done = 0;
    ctl->error = 0;
    ctl->num_leaves = 1;
    ctl->max_leaves = max_leaves;
    ctl->max_depth = max_depth;
    ctl->n_slots = 1;
    ctl->slot_cap = slot_cap;
    ctl->spec_max = spec_max;
    ctl->fp_mode = fp_mode;
    ctl->n_jobs = 0;
    ctl->rounds = 0;
    ctl->tile_total = 0;
    // root gate (before_find_best_split, learner.rs:1830-1836): a single leaf with
    // fewer than 2 * min_data_in_leaf rows is never scanned
    const bool did = N >= ctl->cfg.min_data_in_leaf * 2;
    ctl->root_skip = did ? 0 : 1;
    ctl->n_reduce = did ? 1 : 0;
    ctl->reduce_list[0] = 0;
    // the root ConstructHistogram: all rows
    ctl->n_hjobs = 1;
    ctl->hjobs[0] = HistJob{BUF_ORIG, 1, 0, N, 0, 0};  // _pad bit 0: the root build
    DevNodes& nd = L.nodes;
    nd.begin[0] = 0;
    nd.count[0] = N;
    nd.buf[0] = BUF_ORIG;
    nd.rev[0] = 0;
    nd.depth[0] = 0;
    nd.child[0] = -1;
    nd.child[1] = -1;
    nd.sums[0] = LeafSums{0.0, 0.0, 0.0, N, 0};
    nd.key_gain[0] = -__builtin_inf();
    nd.key_feat[0] = -1;
    L.fmat[0] = 0;
    split_set_none(&L.best[0]);
    L.best_fpos[0] = -1;
    L.plan_state[PS_LEAF_SLOT * MAX_LEAVES] = 0;
    L.plan_state[PS_LEAF_SIDE * MAX_LEAVES] = 0;
    L.plan_state[PS_LEAF_PARENT * MAX_LEAVES] = -1;
    L.stats[2] += (double)N;
    L.stats[3] += 1.0;
  }
}

// Leaf keys in the reference's ArgMax order (split_gt, split_info.rs:28-35: higher
// gain, then lower real feature index with -1 last; then the lower leaf id, the
// first-max-wins scan of learner.rs:4537) packed into 128 bits that compare as
// unsigned integers.  Only positive gains qualify (smaller ones stop the tree): any
// other leaf gets 0, below every qualifying key.  The bit pattern of a positive
// double orders like the double.
struct LKey {
  uint64_t hi, lo;
};
__device__ __forceinline__ LKey lkey(double gain, int32_t feat, int32_t leaf) {
  if (!(gain > 0.0)) return LKey{0ull, 0ull};
  const uint32_t f = feat == -1 ? 0x7fffffffu : (uint32_t)feat;
  return LKey{(uint64_t)__double_as_longlong(gain),
              ((uint64_t)(0x7fffffffu - f) << 32) | (uint64_t)(0xffffffffu - (uint32_t)leaf)};
}
__device__ __forceinline__ bool lk_gt(const LKey& a, const LKey& b) {
  return a.hi > b.hi || (a.hi == b.hi && a.lo > b.lo);
}
__device__ __forceinline__ LKey lk_max(const LKey& a, const LKey& b) { return lk_gt(a, b) ? a : b; }
// A DPP move of a key (the four dwords alike); lanes outside ROW_MASK / BANK_MASK, or
// whose source lane is invalid, keep their own key.
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ LKey lk_dpp(const LKey& k) {
  auto mv = [](uint64_t v) {
    const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
    const uint32_t nlo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROW_MASK, BANK_MASK, false);
    const uint32_t nhi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROW_MASK, BANK_MASK, false);
    return ((uint64_t)nhi << 32) | nlo;
  };
  return LKey{mv(k.hi), mv(k.lo)};
}
// Inclusive prefix maximum of the wave's keys in lane order: row_shr 1, 2, 4, 8 within
// each 16-lane row, then the row broadcasts 15 and 31 (max is idempotent, so lanes
// that keep their own key change nothing).
__device__ __forceinline__ LKey lk_prefix_max(LKey v) {
  v = lk_max(v, lk_dpp<0x111, 0xf, 0xf>(v));  // row_shr:1
  v = lk_max(v, lk_dpp<0x112, 0xf, 0xf>(v));  // row_shr:2
  v = lk_max(v, lk_dpp<0x114, 0xf, 0xf>(v));  // row_shr:4
  v = lk_max(v, lk_dpp<0x118, 0xf, 0xf>(v));  // row_shr:8
  v = lk_max(v, lk_dpp<0x142, 0xa, 0xf>(v));  // row_bcast:15 into rows 1, 3
  v = lk_max(v, lk_dpp<0x143, 0xc, 0xf>(v));  // row_bcast:31 into rows 2, 3
  return v;
}
__device__ __forceinline__ LKey lk_readlane(const LKey& k, int lane) {
  auto rl = [&](uint64_t v) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane) << 32) |
           (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  };
  return LKey{rl(k.hi), rl(k.lo)};
}

// ===========================================================================
// k_plan: one block.
//   0. one prefetch of everything it reads (control block, features, node-slot keys,
//      leaf / node linkage) into LDS;
//   1. per-leaf feature ArgMax for the node slots scanned since the last plan
//      (the argmax of scan_leaf_histogram, learner.rs:3290-3330), one wave per slot;
//   2. commits: the reference's repeated ArgMax over the committed leaves
//      (learner.rs:4537, split_gt order, first leaf id wins) and its stop test
//      (gain <= 0, learner.rs:1503; num_leaves - 1 splits at most); while the chosen
//      leaf has already been split, commit that split: node = num_leaves - 1, the
//      left child keeps the leaf id, the right child gets id num_leaves
//      (tree.rs:614-700).  Computed as a rank of the split leaves and one pass;
//   3. selection: the chosen leaf, then the next best-ranked unsplit leaves with
//      gain > 0, up to spec_max, while two node slots per split the tree may still
//      need stay in reserve (ranks counted in parallel);
//   4. (all threads) the Tree::split fields of the committed splits, the partition
//      jobs (with zeroed output cursors) and child node slots of the selected leaves.
// A slot's best split is feat_split[slot * F + best_fpos[slot]].
// ===========================================================================
__global__ __launch_bounds__(PLAN_THREADS) void k_plan(DevLearner L, int32_t slot_cap) {
  __shared__ double s_gain[SLOT_CAP(MAX_LEAVES)];
  __shared__ int32_t s_feat[SLOT_CAP(MAX_LEAVES)];
  __shared__ int32_t s_fpos[SLOT_CAP(MAX_LEAVES)];
  __shared__ int2 s_child[SLOT_CAP(MAX_LEAVES)];
  __shared__ int32_t s_ps[5][MAX_LEAVES];  // PS_* linkage
  __shared__ DevFeature s_ft[16 * LGBM_MAX_W];  // the record layouts' features (wide: global)
  __shared__ int32_t s_ri[WIDE_MAX_F];     // per feature position: its real index (ArgMax ties)
  __shared__ int4 s_commit[MAX_LEAVES];    // (leaf, node slot, node, new right leaf)
  __shared__ int2 s_lc[MAX_LEAVES];        // per leaf: speculated children slots
  __shared__ double2 s_lcg[MAX_LEAVES];    //   and their keys
  __shared__ int2 s_lcf[MAX_LEAVES];
  __shared__ int4 s_pick[SPEC_MAX];        // (leaf, node slot, left slot, right slot)
  __shared__ int32_t s_red[2 * SPEC_MAX + 2];
  __shared__ int32_t s_nc, s_nj, s_nl, s_done, s_nslots, s_nS, s_ncand, s_nsurv;
  __shared__ int32_t s_surv[MAX_LEAVES];   //   the candidates that survive pass A
  __shared__ unsigned long long s_uhi, s_ulo;  // best unsplit leaf key at the start
  __shared__ LKey s_key[MAX_LEAVES];       // per leaf: its ArgMax key
  __shared__ LKey s_ck[MAX_LEAVES];        //   the same for selection candidates, else 0
  __shared__ int32_t s_S[MAX_LEAVES];      // split, uncommitted leaves
  __shared__ LKey s_SK[MAX_LEAVES];        //   and their keys
  __shared__ int32_t s_sorted[MAX_LEAVES]; //   in key order
  Ctl* ctl = L.ctl;
  const int tid = threadIdx.x;
  const int lane = (int)lane_id();
  const int wave = tid >> 6;
  const int F = L.F;
  const double ninf = -__builtin_inf();
  const DevNodes& nd = L.nodes;
  DevTree& T = L.tree;
  // ---- 0. prefetch --------------------------------------------------------------
  const int32_t cdone = ctl->done;
  const int32_t nl0 = ctl->num_leaves, ns0 = ctl->n_slots, maxl = ctl->max_leaves;
  const int32_t nred = ctl->n_reduce, spec = ctl->spec_max, cerr = ctl->error;
  const bool fp = ctl->fp_mode != 0;
  if (tid < 2 * SPEC_MAX + 2) s_red[tid] = ctl->reduce_list[tid];
  // this wave's first slot of phase 1 and its first chunk of feature gains, loaded
  // with the prefetch
  static_assert(PLAN_WAVES <= 2 * SPEC_MAX + 2, "reduce_list covers a slot per wave");
  const bool red0 = wave < nred;
  const int32_t s_w = ctl->reduce_list[wave];
  const double g_w = (red0 && lane < F) ? L.gain_dense[(size_t)s_w * F + lane] : ninf;
  if (tid == 0) {
    s_nS = 0;
    s_ncand = 0;
    s_nsurv = 0;
    s_uhi = 0ull;
    s_ulo = 0ull;
  }
  const bool ft_lds = F <= 16 * LGBM_MAX_W;
  const DevFeature* __restrict__ fts = ft_lds ? s_ft : L.feats;
  if (ft_lds)
    for (int f = tid; f < F; f += PLAN_THREADS) s_ft[f] = L.feats[f];
  // wide layouts: the tie-break indices of every feature, once; the per-slot ArgMax
  // below reads them for every slot, which from global memory is a cache line per
  // feature and slot
  if (!ft_lds)
    for (int f = tid; f < F; f += PLAN_THREADS) s_ri[f] = L.feats[f].real_index;
  for (int s = tid; s < slot_cap; s += PLAN_THREADS) {
    s_gain[s] = nd.key_gain[s];
    s_feat[s] = nd.key_feat[s];
    s_fpos[s] = L.best_fpos[s];
    s_child[s] = make_int2(nd.child[2 * s], nd.child[2 * s + 1]);
  }
  for (int i = tid; i < 5 * MAX_LEAVES; i += PLAN_THREADS) (&s_ps[0][0])[i] = L.plan_state[i];
  if (cdone) return;
  __syncthreads();

  // ---- 1. per-slot feature ArgMax -------------------------------------------
  if (nred > 0 && nred * 2 <= PLAN_WAVES) {
    // few slots (the late rounds): W waves a slot, each over every W-th 64-feature
    // chunk, then the slot's first wave combines their keys (one load round trip per
    // wave instead of F / 512)
    __shared__ double s_bkg[PLAN_WAVES];
    __shared__ int32_t s_bkf[PLAN_WAVES], s_bki[PLAN_WAVES];
    int W = 2;
    while (W * 2 * nred <= PLAN_WAVES) W *= 2;
    const int i = wave / W, part = wave - i * W;
    BestKey k{ninf, -1, INT_MAX32};
    if (i < nred) {
      const int32_t s = s_red[i];
      constexpr int KU = 4;
      for (int f0 = part * LGBM_WAVE + lane; f0 < F; f0 += KU * W * LGBM_WAVE) {
        double gv[KU];
        int32_t rv[KU];
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          const int f = f0 + u * W * LGBM_WAVE;
          gv[u] = f < F ? L.gain_dense[(size_t)s * F + f] : ninf;
          rv[u] = f < F ? (ft_lds ? fts[f].real_index : s_ri[f]) : -1;
        }
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          const BestKey c{gv[u], rv[u], f0 + u * W * LGBM_WAVE};
          if (gv[u] > ninf && key_better(c, k)) k = c;
        }
      }
      k = wave_best_fast(k);
    }
    if (lane == 0) {
      s_bkg[wave] = k.gain;
      s_bkf[wave] = k.feat;
      s_bki[wave] = k.idx;
    }
    __syncthreads();
    if (i < nred && part == 0) {
      BestKey c{ninf, -1, INT_MAX32};
      if (lane < W) c = BestKey{s_bkg[wave + lane], s_bkf[wave + lane], s_bki[wave + lane]};
      c = wave_best_fast(c);
      const int32_t s = s_red[i];
      const bool have = c.idx != INT_MAX32 && c.gain > ninf;
      if (lane == 0) {
        const double kg = have ? c.gain : ninf;
        const int32_t kf = have ? c.feat : -1, kp = have ? c.idx : -1;
        nd.key_gain[s] = kg;
        nd.key_feat[s] = kf;
        L.best_fpos[s] = kp;
        s_gain[s] = kg;
        s_feat[s] = kf;
        s_fpos[s] = kp;
      }
    }
  } else
  for (int i = wave; i < nred; i += PLAN_WAVES) {
    const int32_t s = s_red[i];
    BestKey k{ninf, -1, INT_MAX32};
    // eight features a lane in flight: with thousands of features one load round
    // trip per 64 features would set the phase's time
    constexpr int KU = 8;
    for (int f0 = lane; f0 < F; f0 += KU * LGBM_WAVE) {
      double gv[KU];
      int32_t rv[KU];
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const int f = f0 + u * LGBM_WAVE;
        gv[u] = f < F ? ((i == wave && f == lane) ? g_w : L.gain_dense[(size_t)s * F + f]) : ninf;
        rv[u] = f < F ? (ft_lds ? fts[f].real_index : s_ri[f]) : -1;
      }
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const BestKey c{gv[u], rv[u], f0 + u * LGBM_WAVE};
        if (gv[u] > ninf && key_better(c, k)) k = c;
      }
    }
    k = wave_best_fast(k);
    const bool have = k.idx != INT_MAX32 && k.gain > ninf;
    if (lane == 0) {
      const double kg = have ? k.gain : ninf;
      const int32_t kf = have ? k.feat : -1, kp = have ? k.idx : -1;
      nd.key_gain[s] = kg;
      nd.key_feat[s] = kf;
      L.best_fpos[s] = kp;
      s_gain[s] = kg;
      s_feat[s] = kf;
      s_fpos[s] = kp;
    }
  }
  __syncthreads();

  // ---- 2. commits ------------------------------------------------------------
  // Leaves split in earlier rounds but not committed yet (S) keep their keys, and a
  // commit only adds its two fresh, unsplit children.  So the reference's repeated
  // ArgMax commits S in key order for as long as the next S key beats the best
  // unsplit key so far (the best unsplit leaf at the start, raised by the children
  // of each commit); the right child of the i-th commit gets leaf id nl0 + i.  With S
  // ranked, that is one exclusive prefix maximum over the ranks and a ballot.
  static_assert(MAX_LEAVES <= PLAN_THREADS, "one thread per leaf");
  if (tid < MAX_LEAVES) {  // whole waves: the wave reductions below see every lane
    const int l = tid;
    const bool live = l < nl0;
    const int32_t s = live ? s_ps[PS_LEAF_SLOT][l] : 0;
    const int2 ch = live ? s_child[s] : make_int2(-1, -1);
    const LKey k = live ? lkey(s_gain[s], s_feat[s], l) : LKey{0ull, 0ull};
    if (live) {
      s_lc[l] = ch;
      s_key[l] = k;
    }
    if (live && ch.x >= 0) {
      s_lcg[l] = make_double2(s_gain[ch.x], s_gain[ch.y]);
      s_lcf[l] = make_int2(s_feat[ch.x], s_feat[ch.y]);
    }
    // S: one LDS atomic per wave reserves the wave's entries
    const bool in_s = live && ch.x >= 0 && k.hi != 0ull;
    const unsigned long long sm = __ballot(in_s);
    int32_t base = 0;
    if (lane == 0 && sm) base = atomicAdd(&s_nS, (int32_t)__popcll(sm));
    base = __builtin_amdgcn_readfirstlane(base);
    if (in_s) {
      const int32_t pos = base + (int32_t)__popcll(sm & lanemask_lt());
      s_S[pos] = l;
      s_SK[pos] = k;
    }
    // the best unsplit key's high word: a wave maximum (the bits of a positive double,
    // or 0, order like the double), one LDS atomic per wave
    const unsigned long long u = (unsigned long long)__double_as_longlong(wave_max_f64(
        __longlong_as_double((long long)((live && ch.x < 0) ? k.hi : 0ull))));
    if (lane == 0 && u != 0ull) atomicMax(&s_uhi, u);
  }
  __syncthreads();
  for (int l = tid; l < nl0; l += PLAN_THREADS) {
    const LKey k = s_key[l];
    if (s_lc[l].x < 0 && k.hi != 0ull && k.hi == s_uhi) atomicMax(&s_ulo, (unsigned long long)k.lo);
  }
  const int32_t nS = s_nS;
  {
    // rank of each S leaf within S (the leaves split ahead of their turn can number
    // well over a hundred): T consecutive threads per leaf (at most a DPP row), each
    // counting the better keys among every T-th entry, summed across the group
    int T = 1;
    while (T < 16 && nS * T * 2 <= PLAN_THREADS) T *= 2;
    for (int i0 = 0; i0 < nS * T; i0 += PLAN_THREADS) {
      const int idx = i0 + tid, i = idx / T, sub = idx - i * T;
      const bool valid = i < nS;
      int32_t r = 0;
      if (valid) {
        const LKey c = s_SK[i];
#pragma unroll 4
        for (int k = sub; k < nS; k += T) r += lk_gt(s_SK[k], c) ? 1 : 0;
      }
      if (T >= 2) r += __builtin_amdgcn_update_dpp(0, r, 0xB1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
      if (T >= 4) r += __builtin_amdgcn_update_dpp(0, r, 0x4E, 0xf, 0xf, false);   // quad_perm [2,3,0,1]
      if (T >= 8) r += __builtin_amdgcn_update_dpp(0, r, 0x141, 0xf, 0xf, false);  // row_half_mirror
      if (T >= 16) r += __builtin_amdgcn_update_dpp(0, r, 0x140, 0xf, 0xf, false); // row_mirror
      if (valid && sub == 0) s_sorted[r] = s_S[i];
    }
  }
  __syncthreads();
  if (wave == 0) {
    LKey P{s_uhi, s_ulo};  // best unsplit key so far (0: none)
    int32_t nc = 0;
    bool stop = cerr != 0;
    for (int base = 0; base < nS && !stop; base += LGBM_WAVE) {
      const int i = base + lane;
      const bool in = i < nS;
      LKey e{0ull, 0ull}, M{0ull, 0ull};
      if (in) {
        const int32_t l = s_sorted[i];
        const double2 cg = s_lcg[l];
        const int2 cf = s_lcf[l];
        e = s_key[l];
        M = lk_max(lkey(cg.x, cf.x, l), lkey(cg.y, cf.y, nl0 + i));  // Tree::split ids
      }
      const LKey inc = lk_prefix_max(M);  // inclusive prefix maximum of the children keys
      LKey ex = lk_dpp<0x138, 0xf, 0xf>(inc);  // wave_shr:1: lane i - 1's
      if (lane == 0) ex = LKey{0ull, 0ull};
      ex = lk_max(ex, P);
      const bool ok = in && i < maxl - nl0 && lk_gt(e, ex);
      const unsigned long long okm = __ballot(ok);
      const int run = okm == ~0ull ? LGBM_WAVE : (int)__builtin_ctzll(~okm);
      if (run > 0) P = lk_max(P, lk_readlane(inc, run - 1));
      nc = base + run;
      stop = run < LGBM_WAVE;
    }
    if (lane == 0) {
      const int32_t nl = nl0 + nc;
      // the stop test of the next ArgMax: no positive gain left, or all leaves used
      const bool done = cerr != 0 || nl >= maxl || (nc == nS && P.hi == 0ull);
      s_nc = nc;
      s_nl = nl;
      s_done = done ? 1 : 0;
    }
  }
  __syncthreads();
  const int32_t nc_ = s_nc, nl_ = s_nl;
  for (int c = tid; c < nc_; c += PLAN_THREADS) {
    // commit c: node nl0 - 1 + c, left child keeps the leaf id, right child nl0 + c.
    // Committed leaves are distinct leaves of earlier rounds, so these writes are
    // disjoint.
    const int32_t bl = s_sorted[c], node = nl0 - 1 + c, nr = nl0 + c;
    const int2 ch = s_lc[bl];
    const double2 cg = s_lcg[bl];
    const int2 cf = s_lcf[bl];
    const int32_t p = s_ps[PS_LEAF_SLOT][bl];
    const int32_t pn = s_ps[PS_LEAF_PARENT][bl], side = s_ps[PS_LEAF_SIDE][bl];
    if (pn >= 0) s_ps[side ? PS_NODE_RIGHT : PS_NODE_LEFT][pn] = node;
    s_ps[PS_NODE_LEFT][node] = ~bl;
    s_ps[PS_NODE_RIGHT][node] = ~nr;
    s_ps[PS_LEAF_SLOT][bl] = ch.x;
    s_ps[PS_LEAF_SLOT][nr] = ch.y;
    s_ps[PS_LEAF_PARENT][bl] = node;
    s_ps[PS_LEAF_PARENT][nr] = node;
    s_ps[PS_LEAF_SIDE][bl] = 0;
    s_ps[PS_LEAF_SIDE][nr] = 1;
    s_lc[bl] = make_int2(-1, -1);  // fresh leaves: not split yet
    s_lc[nr] = make_int2(-1, -1);
    s_key[bl] = lkey(cg.x, cf.x, bl);
    s_key[nr] = lkey(cg.y, cf.y, nr);
    s_commit[c] = make_int4(bl, p, node, nr);
  }
  __syncthreads();

  // ---- 3. selection ------------------------------------------------------------
  // The ArgMax leaf, then the next best-ranked unsplit leaves with gain > 0, up to
  // spec_max; beyond the first, two node slots stay in reserve for every split the
  // tree may still need, so the ArgMax leaf of every later round can be split.  A
  // candidate's rank is the number of better candidates (keys of non-candidates are
  // 0, below every candidate), found in two passes.
  static_assert(PLAN_THREADS == 4 * MAX_LEAVES && MAX_LEAVES % 32 == 0,
                "selection: four threads per leaf, groups of 32 leaves");
  if (!s_done) {
    const int32_t nl = nl_;
    if (tid < MAX_LEAVES) {  // whole waves, one LDS atomic per wave
      const int l = tid;
      bool cand = false;
      if (l < nl) {
        const LKey k = s_key[l];
        cand = s_lc[l].x < 0 && k.hi != 0ull;
        s_ck[l] = cand ? k : LKey{0ull, 0ull};
      } else {
        s_ck[l] = LKey{0ull, 0ull};
      }
      const unsigned long long cm = __ballot(cand);
      if (lane == 0 && cm) atomicAdd(&s_ncand, (int32_t)__popcll(cm));
    }
    __syncthreads();
    int32_t allowed = 0;
    if (ns0 + 2 <= slot_cap) {
      const int32_t extra = (slot_cap - ns0 - 2 - 2 * (maxl - nl)) / 2;
      allowed = min(spec, 1 + max(extra, 0));
      // Where a job's scans are costly next to a round's fixed latency (many features,
      // f32 cells twice the work), speculate beyond the ArgMax leaf only while the
      // leaves already split ahead of their turn are fewer than the splits the tree
      // can still take; with fewer features the rounds the cap adds cost more than
      // the jobs it saves
      if (F * (fp ? 2 : 1) >= PLAN_CAP_WORK)
        allowed = min(allowed, max(1, (maxl - nl) - (s_nS - s_nc)));
    }
    // pass A: a candidate's rank within its group of 32 leaves (4 threads, 8 keys
    // each); the group's best `allowed` survive.  Every candidate of the overall best
    // `allowed` survives (all better ones are better in their groups too), so pass B,
    // which ranks the survivors among themselves, gives the exact ranks of those.
    {
      const int l = tid >> 2, q = tid & 3, gb = l & ~31;
      const LKey c = s_ck[l];
      int32_t ra = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) ra += lk_gt(s_ck[gb + q + 4 * i], c) ? 1 : 0;
      ra += __builtin_amdgcn_update_dpp(0, ra, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
      ra += __builtin_amdgcn_update_dpp(0, ra, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
      const bool surv = q == 0 && c.hi != 0ull && ra < allowed;
      const unsigned long long sm = __ballot(surv);
      int32_t base = 0;
      if (lane == 0 && sm) base = atomicAdd(&s_nsurv, (int32_t)__popcll(sm));
      base = __builtin_amdgcn_readfirstlane(base);
      if (surv) s_surv[base + (int32_t)__popcll(sm & lanemask_lt())] = l;
    }
    __syncthreads();
    // pass B: 16 threads per survivor (one DPP row), 64 survivors per step
    const int32_t nsv = s_nsurv;
    for (int32_t u0 = 0; u0 < nsv; u0 += PLAN_THREADS / 16) {
      const int32_t u = u0 + (tid >> 4), sub = tid & 15;
      const int32_t l = u < nsv ? s_surv[u] : 0;
      const LKey c = u < nsv ? s_ck[l] : LKey{0ull, 0ull};
      int32_t rb = 0;
      for (int32_t v = sub; v < nsv; v += 16) rb += lk_gt(s_ck[s_surv[v]], c) ? 1 : 0;
      rb += __builtin_amdgcn_update_dpp(0, rb, 0xB1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
      rb += __builtin_amdgcn_update_dpp(0, rb, 0x4E, 0xf, 0xf, false);   // quad_perm [2,3,0,1]
      rb += __builtin_amdgcn_update_dpp(0, rb, 0x141, 0xf, 0xf, false);  // row_half_mirror
      rb += __builtin_amdgcn_update_dpp(0, rb, 0x140, 0xf, 0xf, false);  // row_mirror
      if (sub == 0 && c.hi != 0ull && rb < allowed)
        s_pick[rb] = make_int4(l, s_ps[PS_LEAF_SLOT][l], ns0 + 2 * rb, ns0 + 2 * rb + 1);
    }
    if (tid == 0) {
      const int32_t nj = min(s_ncand, allowed);
      s_nj = nj;
      s_nslots = ns0 + 2 * nj;
      if (nj == 0) {  // the slot reserve makes this unreachable
        s_done = 1;
        atomicOr(&ctl->error, ERR_SLOTS);
      }
    }
  } else if (tid == 0) {
    s_nj = 0;
    s_nslots = ns0;
  }
  __syncthreads();

  // ---- 4. tree fields of the committed splits; jobs of the selected leaves ------
  const int32_t nc = s_nc, nj = s_nj, nl = s_nl;
  for (int c = tid; c < nc; c += PLAN_THREADS) {
    const int4 cm = s_commit[c];
    const int32_t p = cm.y, node = cm.z, fpos = s_fpos[p];
    const lgbm_split_info& b = L.feat_split[(size_t)p * F + fpos];
    const uint32_t thr = b.threshold;
    const double gain = b.gain;
    const int32_t dl = b.default_left;
    const double iv = nd.sums[p].weight;
    const int32_t ic = nd.count[p];
    const DevFeature ft = fts[fpos];
    T.split_feature[node] = ft.real_index;
    T.split_gain[node] = (float)(gain + ctl->cfg.min_gain_to_split);  // learner.rs:3985
    T.threshold_in_bin[node] = thr;
    int8_t dt = 0;
    if (ft.categorical)
      dt |= 1;  // Tree::split_categorical: no default-left bit
    else if (dl)
      dt |= 2;
    dt |= (int8_t)((ft.missing_type & 3) << 2);
    T.decision_type[node] = dt;
    T.internal_value[node] = iv;  // the split leaf's output
    T.internal_count[node] = ic;  // partition counts (learner.rs:3994-4011)
    // Tree::Split: internal_weight = left_weight + right_weight (the children's
    // sum_hessians, which become their leaf_weight)
    T.internal_weight[node] = nd.sums[s_ps[PS_LEAF_SLOT][cm.x]].sh + nd.sums[s_ps[PS_LEAF_SLOT][cm.w]].sh;
    lgbm_split_info bb;
    bb.threshold = thr;
    bb.default_left = dl;
    NodeRoute r;
    r.f = fpos;
    router_of(ft, bb, &r.pmin, &r.th, &r.flags);
    r.max_bin = (int32_t)ft.max_bin;
    r.na_bin = (int32_t)ft.num_bin - 1;
    r.left = ~cm.x;
    r.right = ~cm.w;
    if (ft.categorical) {
      r.flags = ROUTE_CAT;
      const uint32_t* cb = L.cat_bits + ((size_t)p * F + fpos) * 8;
#pragma unroll
      for (int w = 0; w < 8; ++w) T.cat_left[node * 8 + w] = cb[w];
    }
    T.nodes[node] = r;
  }
  for (int l = tid; l < nl; l += PLAN_THREADS) {
    L.plan_state[PS_LEAF_SLOT * MAX_LEAVES + l] = s_ps[PS_LEAF_SLOT][l];
    L.plan_state[PS_LEAF_SIDE * MAX_LEAVES + l] = s_ps[PS_LEAF_SIDE][l];
    L.plan_state[PS_LEAF_PARENT * MAX_LEAVES + l] = s_ps[PS_LEAF_PARENT][l];
  }
  for (int n = tid; n < nl - 1; n += PLAN_THREADS) {
    L.plan_state[PS_NODE_LEFT * MAX_LEAVES + n] = s_ps[PS_NODE_LEFT][n];
    L.plan_state[PS_NODE_RIGHT * MAX_LEAVES + n] = s_ps[PS_NODE_RIGHT][n];
  }
  // the picks on wave PICK_WAVE, one lane each, beside the commits (waves 0-3): their
  // loads overlap, and the wave's prefix sum places each job's tiles
  constexpr int PICK_WAVE = PLAN_WAVES / 2;
  static_assert(SPEC_MAX <= LGBM_WAVE && PICK_WAVE * LGBM_WAVE >= MAX_LEAVES,
                "picks: one lane each on a wave of their own");
  if (wave == PICK_WAVE) {
    const int j = lane;
    const bool pick = j < nj;
    PartJob J;
    lgbm_split_info b;
    int32_t d = 0;
    if (pick) {
      const int4 pk = s_pick[j];
      const int32_t p = pk.y, fpos = s_fpos[p];
      b = L.feat_split[(size_t)p * F + fpos];
      const DevFeature ft = fts[fpos];
      J.parent = p;
      J.cl = pk.z;
      J.cr = pk.w;
      J.src_buf = nd.buf[p];
      J.rev = nd.rev[p];
      J.begin = nd.begin[p];
      J.count = nd.count[p];
      d = nd.depth[p] + 1;
      J.dst_buf = J.src_buf == BUF_A ? BUF_B : BUF_A;
      J.fbyte = fpos;
      router_of(ft, b, &J.pmin, &J.th, &J.flags);
      J.max_bin = (int32_t)ft.max_bin;
      J.na_bin = (int32_t)ft.num_bin - 1;
      if (ft.categorical) {
        // bit 8: the SplitInfo counts make the left child the smaller one
        J.flags = ROUTE_CAT | (b.left_count < b.right_count ? 1 << 8 : 0);
        const uint32_t* cb = L.cat_bits + ((size_t)p * F + fpos) * 8;
#pragma unroll
        for (int w = 0; w < 8; ++w) J.cat[w] = cb[w];
      }
      // quantized gradients: build the histogram of the side the scan expects to be
      // smaller inside the partition pass (f32: k_hist_f32 builds the smaller child)
      J.acc_right = fp ? -1 : (b.right_count < b.left_count ? 1 : 0);
      J.ntiles = (int32_t)((J.count + part_tile(L.fmt) - 1) / part_tile(L.fmt));
    }
    // each job's first tile: the exclusive prefix of the tile counts (all lanes)
    const int32_t nt = pick ? J.ntiles : 0;
    const int32_t incl = wave_incl_sum_i32(nt);
    if (pick) {
      const int32_t p = J.parent, cl = J.cl, cr = J.cr;
      J.tile0 = incl - nt;
      ctl->jobs[j] = J;
      ctl->part_cur[j] = 0ull;
      ctl->acc_used[j] = 0;
      nd.child[2 * p] = cl;
      nd.child[2 * p + 1] = cr;
      nd.child[2 * cl] = -1;
      nd.child[2 * cl + 1] = -1;
      nd.child[2 * cr] = -1;
      nd.child[2 * cr + 1] = -1;
      nd.depth[cl] = d;
      nd.depth[cr] = d;
      // LeafSplits::init_from_split (leaf_splits.rs:162-173): sums and outputs of the
      // SplitInfo; counts come from the partition.
      nd.sums[cl] = LeafSums{b.left_sum_gradient, b.left_sum_hessian, b.left_output, 0, 0};
      nd.sums[cr] = LeafSums{b.right_sum_gradient, b.right_sum_hessian, b.right_output, 0, 0};
      nd.key_gain[cl] = ninf;
      nd.key_gain[cr] = ninf;
      nd.key_feat[cl] = -1;
      nd.key_feat[cr] = -1;
      L.best_fpos[cl] = -1;
      L.best_fpos[cr] = -1;
      ctl->reduce_list[2 * j] = cl;
      ctl->reduce_list[2 * j + 1] = cr;
    }
    const int32_t total = readlane_i32(incl, LGBM_WAVE - 1);
    if (lane == 0) {
      ctl->tile_total = total;
      ctl->n_jobs = nj;
      if (fp || rec_wide(L.fmt)) ctl->n_hjobs = nj;  // k_partition fills in each job's side
      ctl->n_reduce = 2 * nj;
      ctl->num_leaves = nl;
      ctl->n_slots = s_nslots;
      ctl->rounds += 1;
      if (nj > 0) L.stats[1] += 1.0;
      if (s_done) ctl->done = 1;
    }
  }
}

// ===========================================================================
// k_partition: DataPartition::split of every job of the round in one pass.  The
// tiles of all jobs (job j owns tiles [tile0, tile0 + ntiles), part_tile(fmt) rows each,
// in the parent's logical row order) are dealt to the blocks in contiguous runs, so a
// block meets few job boundaries.  A tile ranks its rows with wave ballots, then
// takes its output ranges:
//   tree driver (STABLE = false): one 64-bit atomic add on the job's cursor reserves
//     (left rows, right rows) at once, so no tile waits for another; the order of
//     rows inside a child is then unspecified (every consumer is order-free: integer
//     histogram cells, per-row score update; the layout export sorts each leaf);
//   per-op entry point (STABLE = true): the exclusive left prefix of the tile within
//     its job, precomputed by k_tile_count + k_tile_scan, keeps DataPartition::split's
//     stable order.
// Left rows go to [begin, begin + L) ascending, right rows to [begin + L, begin +
// count) filled from the end (stored reversed: logical order = reverse storage
// order).  The block that completes a job (last cursor reservation, or the job's last
// tile when stable) records the children's ranges and counts.
// Quantized gradients (FP = 0): in the tree driver the pass also builds one child's
// integer histogram per job (the side the scan predicts to be smaller) from the rows
// while they are in registers, flushed per (block, job) into the job's accumulator;
// the other child's is parent - built in integers (k_pair_scan).  f32 gradients
// (FP = 1) move as (g, h) pairs; the smaller child's histogram is built afterwards by
// k_hist_f32.
// ===========================================================================
template <int FMT, int FP, bool STABLE>
__global__ __launch_bounds__(PART_THREADS) void k_partition(DevLearner L) {
  constexpr int PT = PART_THREADS, PR = part_rows(FMT);
  constexpr int U = rec_words(FMT), BPW = rec_bpw(FMT);
  constexpr int NS = rec_slots(FMT) > 0 ? rec_slots(FMT) : 1;
  // wide records are row indices: the pass routes by one byte of the row's binmat row
  // and builds no histogram (k_hist_wide builds the job's histogram side afterwards)
  constexpr bool WIDE = rec_wide(FMT);
  constexpr bool HIST = FP == 0 && !WIDE;
  // packed records carry the quantized pair in their last word (the original order's
  // pairs come from the quantizer's array)
  constexpr bool EMBED = rec_packed(FMT) && FP == 0;
  constexpr int kWaves = PT / LGBM_WAVE;
  constexpr int kTile = PT * PR;
  constexpr int kSlots = PR * kWaves;  // (row k, wave) left counts, k-major = row order
  static_assert(kSlots <= LGBM_WAVE, "wave 0 scans the per-(row, wave) left counts");
  // An LDS cell holds sums of q_h <= 4 below 2^21 (and |q_g| <= 2 below 2^21): a
  // block flushes its histogram after this many tiles of one job.
  constexpr int kFlushTiles = ((1 << 19) - 1) / kTile;
  static_assert(kFlushTiles >= 1, "tile larger than an LDS cell's row capacity");
  using GhT = typename std::conditional<FP != 0, float2, uint16_t>::type;
  extern __shared__ unsigned long long lds_hist[];
  __shared__ int32_t cb[NS];
  __shared__ PartJob s_jobs[SPEC_MAX];
  __shared__ int32_t s_cnt[kSlots];
  __shared__ int32_t s_pref[kSlots];
  __shared__ int32_t s_lbase, s_rbase, s_total, s_last;
  // packed records: each wave stages its rows of the built side densely (a ring of 128
  // records + pairs) so that the histogram adds run on full waves
  constexpr bool STAGE = HIST && EMBED;
  constexpr int kRing = 128;
  __shared__ uint32_t s_stage[STAGE ? kWaves * kRing * (U + 1) : 1];
  Ctl* ctl = L.ctl;
  const int tid = threadIdx.x, wave = tid >> 6, lane = (int)lane_id();
  const int32_t nj = ctl->n_jobs;
  const int64_t total = ctl->tile_total;
  const int64_t G = gridDim.x;
  const int64_t t_lo = (int64_t)blockIdx.x * total / G;
  const int64_t t_hi = ((int64_t)blockIdx.x + 1) * total / G;
  if (tid < SPEC_MAX) s_jobs[tid] = ctl->jobs[tid];
  if (nj <= 0 || t_lo >= t_hi) return;
  const int F = L.F, cells = L.total_cells, nw = (F + BPW - 1) / BPW;
  // the bin slots' cell bases, loaded before the first tile so that waiting for them
  // does not wait for the tile's loads (the load counter drains in issue order)
  static_assert(NS <= PT, "a slot per thread");
  const int32_t cb_v = tid < NS ? (tid < F ? (int32_t)L.feats[tid].cell_base : cells) : 0;
  struct TileBuf {
    uint32_t w[PR][U];
    GhT q[PR];
    bool valid[PR];
    bool q_in_rec;  // q still sits in the records (taken out when the tile is processed)
  };
  // Issues every load of tile t of a job (first tile tile0, `count` rows from `begin`,
  // stored reversed when rev) at once: positions past the job's end re-read its last
  // row (a job that owns a tile has count >= 1).
  auto load_job = [&](int64_t t, TileBuf& B, int64_t tile0, int64_t count, int64_t begin,
                      int32_t rev, int32_t src_buf) {
    const int64_t base = (t - tile0) * kTile;
    const uint4* __restrict__ src = rec_buf(L.bufs, src_buf);
    const GhT* __restrict__ sgh = gh_buf<GhT>(L.bufs, src_buf);
    const bool from_rec = EMBED && src_buf != BUF_ORIG;
#pragma unroll
    for (int k = 0; k < PR; ++k) {
      const int64_t p = base + (int64_t)k * PT + tid;
      B.valid[k] = p < count;
      const int64_t pc = B.valid[k] ? p : count - 1;
      const int64_t phys = rev ? begin + count - 1 - pc : begin + pc;
      rec_load<FMT>(src, phys, B.w[k]);
      if constexpr (EMBED) {
        if (!from_rec) B.q[k] = sgh[phys];
      } else {
        B.q[k] = sgh[phys];
      }
    }
    // the pairs embedded in the records are taken out in process(): reading them here
    // would wait for the loads and void the overlap with the current tile
    B.q_in_rec = from_rec;
  };
  int32_t jl = 0;  // job of the last tile loaded
  // tile t's job from the LDS job records; returns it
  auto load = [&](int64_t t, TileBuf& B) -> int32_t {
    while (jl + 1 < nj && s_jobs[jl + 1].tile0 <= t) ++jl;
    const PartJob& J = s_jobs[jl];
    load_job(t, B, J.tile0, J.count, J.begin, J.rev, J.src_buf);
    return jl;
  };
  // The first tile's job from the job records in registers (lane k: job k; jobs are in
  // tile order, an empty job shares the next one's first tile), so its loads are in
  // flight while the block sets up its LDS.
  TileBuf cur_b, next_b;
  int32_t jc = 0, jn = 0;
  {
    const bool lj = lane < nj;
    const PartJob& gj = ctl->jobs[lj ? lane : 0];
    const int64_t t0k = lj ? gj.tile0 : INT64_MAX;
    const int64_t cntk = gj.count, begk = gj.begin;
    const int32_t revk = gj.rev, srck = gj.src_buf;
    jc = (int32_t)__popcll(__ballot(t0k <= t_lo)) - 1;  // job 0 starts at tile 0
    jl = jc;
    auto rl64 = [&](int64_t v) {
      return (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), jc) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)v, jc));
    };
    load_job(t_lo, cur_b, rl64(t0k), rl64(cntk), rl64(begk), __builtin_amdgcn_readlane(revk, jc),
             __builtin_amdgcn_readlane(srck, jc));
  }
  if constexpr (HIST)
    for (int c = tid; c < cells + LDS_TRASH_CELLS; c += PT) lds_hist[c] = 0ull;
  if (tid < NS) cb[tid] = cb_v;
  __syncthreads();
  // bin-slot cell bases in scalar registers (slots beyond F map to the trash cell)
  int32_t cbr[NS];
#pragma unroll
  for (int f = 0; f < NS; ++f) cbr[f] = __builtin_amdgcn_readfirstlane(cb[f]);
  int32_t cur = -1;       // job whose rows the LDS histogram holds
  int32_t held = 0;       // tiles of that job in the LDS histogram
  bool flushed = false;   // this block already flushed part of that job
  // Where this block's cells of job `cur` go: a job spread over at most PART_SLOT_MAX
  // blocks gets one packed slot per block (slot block + job: unique, since blocks and
  // jobs both advance along the tile order), which k_pair_scan sums; a wider job, and
  // a block's second and later flush of one job, atomic adds into the job's
  // accumulator and marks it used (k_pair_scan then reads and clears it): one 64-bit
  // add of the packed cell when the job has fewer than 2^19 rows (its sums fit the
  // packed fields as a block's do), else three 32-bit adds.
  auto flush = [&]() {
    const PartJob& C = s_jobs[cur];
    if (!flushed && part_span_blocks(C.tile0, C.ntiles, total, G) <= PART_SLOT_MAX) {
      lds_hist_flush_clear(lds_hist, cells, L.part_slots + ((size_t)blockIdx.x + cur) * cells,
                           FLUSH_STORE);
    } else {
      if (tid == 0) ctl->acc_used[cur] = 1;
      if (C.count <= PACKED_ACC_MAX_ROWS)
        lds_hist_flush_clear(lds_hist, cells, L.hist_accp + (size_t)cur * L.acc_cells,
                             FLUSH_ATOMIC64);
      else
        lds_hist_flush_clear(lds_hist, cells, L.hist_acc + (size_t)cur * L.acc_cells * 3,
                             FLUSH_ATOMIC);
    }
  };
  // Shared-state hand-off per tile: s_cnt is written after the loads and read by
  // wave 0 before barrier B; s_pref / s_lbase / s_rbase / s_total / s_last are
  // written by wave 0 between barriers A and B and read after B; the next tile's
  // writes of each come after a barrier every reader has passed.  Histogram adds end
  // before B, so a flush at the top of the next tile sees them all.
  auto process = [&](int64_t t, int32_t j, TileBuf& B) {
    if (HIST && (j != cur || held == kFlushTiles)) {
      if (cur >= 0 && s_jobs[cur].acc_right >= 0 && held > 0) {
        flush();
        flushed = j == cur;
        __syncthreads();
      } else {
        flushed = false;
      }
      cur = j;
      held = 0;
    }
    if constexpr (EMBED) {
      if (B.q_in_rec) {
#pragma unroll
        for (int k = 0; k < PR; ++k) B.q[k] = (GhT)rec_gh<FMT>(B.w[k]);
      }
    }
    const PartJob& J = s_jobs[j];
    const int64_t count = J.count, begin = J.begin;
    const int64_t lt = t - J.tile0;
    const int64_t base = lt * kTile;
    uint4* __restrict__ dst = rec_buf(L.bufs, J.dst_buf);
    GhT* __restrict__ dgh = gh_buf<GhT>(L.bufs, J.dst_buf);
    auto& w = B.w;
    auto& q = B.q;
    auto& valid = B.valid;
    bool isleft[PR];
    int32_t rank[PR];
    int fwi, fsh;
    rec_field_pos(FMT, J.fbyte, &fwi, &fsh);
    int32_t wbin[PR];
    if constexpr (WIDE) {
      const int64_t stride = L.row_stride;
      if (L.bincol) {
        // the feature-major copy: the job's rows share the feature's column
        if (L.bin16) {
          const uint16_t* __restrict__ col = (const uint16_t*)L.bincol + (int64_t)J.fbyte * L.N;
#pragma unroll
          for (int k = 0; k < PR; ++k) wbin[k] = col[w[k][0]];
        } else {
          const uint8_t* __restrict__ col = L.bincol + (int64_t)J.fbyte * L.N;
#pragma unroll
          for (int k = 0; k < PR; ++k) wbin[k] = col[w[k][0]];
        }
      } else if (L.bin16) {
        const uint8_t* __restrict__ col = L.binmat + 2 * (int64_t)J.fbyte;
#pragma unroll
        for (int k = 0; k < PR; ++k)
          wbin[k] = *(const uint16_t*)(col + (int64_t)w[k][0] * stride);
      } else {
        const uint8_t* __restrict__ col = L.binmat + J.fbyte;
#pragma unroll
        for (int k = 0; k < PR; ++k) wbin[k] = col[(int64_t)w[k][0] * stride];
      }
    }
#pragma unroll
    for (int k = 0; k < PR; ++k) {
      const int32_t bin = WIDE ? wbin[k] : (int32_t)rec_field<FMT>(w[k], fwi, fsh);
      const bool left = (J.flags & ROUTE_CAT)
                            ? ((J.cat[bin >> 5] >> (bin & 31)) & 1u) != 0u
                            : !route_right(bin, J.pmin, J.max_bin, J.th, J.na_bin, J.flags);
      isleft[k] = valid[k] && left;
      const unsigned long long m = __ballot(isleft[k]);
      rank[k] = (int32_t)__popcll(m & lanemask_lt());
      if (lane == 0) s_cnt[k * kWaves + wave] = (int32_t)__popcll(m);
    }
    __syncthreads();  // A
    int32_t acc = 0, trows = 0;
    unsigned long long old = 0ull;
    if (wave == 0) {
      // exclusive prefix of the (row, wave) counts
      const int32_t c = lane < kSlots ? s_cnt[lane] : 0;
      const int32_t incl = wave_incl_sum_i32(c);
      if (lane < kSlots) s_pref[lane] = incl - c;
      acc = readlane_i32(incl, kSlots - 1);
      trows = (int32_t)min((int64_t)kTile, count - base);
      // the reservation is issued here and its result used after this wave's
      // histogram adds, so the atomic's round trip overlaps them
      if constexpr (!STABLE)
        if (lane == 0)
          old = atomicAdd(&ctl->part_cur[j], (unsigned long long)(uint32_t)acc |
                                                 ((unsigned long long)(uint32_t)(trows - acc) << 32));
    }
    // histogram adds (every wave, wave 0 while its reservation is in flight)
    if constexpr (STAGE) {
      if (J.acc_right >= 0) {
        // LDS atomics cost per instruction more than per active lane: the rows to add
        // (a fraction of the tile) go through the wave's ring and are added 64 at a
        // time, then the remainder
        const bool want_left = J.acc_right == 0;
        uint32_t* ring = s_stage + (size_t)wave * kRing * (U + 1);
        int staged = 0, consumed = 0;  // wave-uniform
        auto add_batch = [&](int n) {
          __builtin_amdgcn_wave_barrier();
          if (lane < n) {
            const uint32_t* e = ring + ((consumed + lane) & (kRing - 1)) * (U + 1);
            uint32_t rw[U];
#pragma unroll
            for (int u = 0; u < U; ++u) rw[u] = e[u];
            lds_hist_add<FMT>(lds_hist, cbr, nw, F, cells + 4 + lane, rw, e[U]);
          }
          __builtin_amdgcn_wave_barrier();
          consumed += n;
          staged -= n;
        };
#pragma unroll
        for (int k = 0; k < PR; ++k) {
          const bool act = valid[k] && isleft[k] == want_left && gh_bits(q[k]) != 0u;
          const unsigned long long am = __ballot(act);
          if (act) {
            uint32_t* e = ring + ((consumed + staged + (int)__popcll(am & lanemask_lt())) &
                                  (kRing - 1)) * (U + 1);
#pragma unroll
            for (int u = 0; u < U; ++u) e[u] = w[k][u];
            e[U] = gh_bits(q[k]);
          }
          staged += (int)__popcll(am);
          if (staged >= LGBM_WAVE) add_batch(LGBM_WAVE);
        }
        if (staged > 0) add_batch(staged);
        ++held;
      }
    } else if constexpr (HIST) {
      if (J.acc_right >= 0) {
        const bool want_left = J.acc_right == 0;
#pragma unroll
        for (int k = 0; k < PR; ++k)
          if (valid[k] && isleft[k] == want_left && gh_bits(q[k]) != 0u)
            lds_hist_add<FMT>(lds_hist, cbr, nw, F, cells + 4 + lane, w[k], gh_bits(q[k]));
        ++held;
      }
    }
    if (wave == 0 && lane == 0) {
      int64_t lb, rb;
      bool last;
      if constexpr (STABLE) {
        lb = (int64_t)L.tile_state[t];
        rb = base - lb;
        last = lt == J.ntiles - 1;
      } else {
        lb = (int64_t)(uint32_t)old;
        rb = (int64_t)(old >> 32);
        last = lb + rb + trows == count;
      }
      s_lbase = (int32_t)lb;
      s_rbase = (int32_t)rb;
      s_total = acc;
      s_last = last ? 1 : 0;
    }
    __syncthreads();  // B
    const int64_t lbase = s_lbase, rbase = s_rbase;
#pragma unroll
    for (int k = 0; k < PR; ++k) {
      if (!valid[k]) continue;
      const int64_t pos = (int64_t)k * PT + tid;
      const int64_t lrank = s_pref[k * kWaves + wave] + rank[k];
      int64_t d;
      if (isleft[k]) {
        d = begin + lbase + lrank;
      } else {
        const int64_t r = rbase + (pos - lrank);  // right rows before this one
        d = begin + count - 1 - r;
      }
      if constexpr (EMBED) {
        rec_set_gh<FMT>(w[k], gh_bits(q[k]));
        rec_store<FMT>(dst, d, w[k]);
      } else {
        rec_store<FMT>(dst, d, w[k]);
        dgh[d] = q[k];
      }
    }
    if (tid == 0 && s_last) {
      const int32_t lc = (int32_t)(lbase + s_total);
      const int32_t rc = (int32_t)(count - lc);
      if (J.parent >= 0) {
        DevNodes& nd = L.nodes;
        nd.begin[J.cl] = (int32_t)begin;
        nd.count[J.cl] = lc;
        nd.buf[J.cl] = J.dst_buf;
        nd.rev[J.cl] = 0;
        nd.begin[J.cr] = (int32_t)(begin + lc);
        nd.count[J.cr] = rc;
        nd.buf[J.cr] = J.dst_buf;
        nd.rev[J.cr] = 1;
        nd.sums[J.cl].n = lc;
        nd.sums[J.cr].n = rc;
        // categorical: the children's scan seeds follow the SplitInfo counts (pending
        // order in the job flags), the histogram the partition counts
        const int32_t sw = (J.flags & ROUTE_CAT) && (((J.flags >> 8) & 1) != (lc < rc ? 1 : 0));
        nd.sums[J.cl]._pad = sw;
        nd.sums[J.cr]._pad = sw;
        if (FP || WIDE) {
          // the round's ConstructHistogram job (k_hist_f32 / k_hist_wide run next):
          // f32, the smaller child (partition counts; a tie makes the right child the
          // smaller one, learner.rs:4061-4089); quantized, the side the scan predicted
          // smaller (the other is parent - built in integers); none for a gated pair
          // (before_find_best_split, learner.rs:1808-1839)
          const int32_t md = ctl->max_depth, min2 = ctl->cfg.min_data_in_leaf * 2;
          const bool gated = (md > 0 && nd.depth[J.cl] >= md) || (lc < min2 && rc < min2);
          const bool right = FP ? !(lc < rc) : J.acc_right == 1;
          HistJob hj;
          hj.buf = J.dst_buf;
          hj._pad = 0;
          hj.begin = right ? begin + lc : begin;
          hj.count = gated ? 0 : (right ? rc : lc);
          hj.a0 = 0;
          hj.nblk = 0;
          ctl->hjobs[j] = hj;
          atomicAdd(&L.stats[5], (double)hj.count);  // rows of the child builds
        }
        atomicAdd(&L.stats[0], (double)count);
        atomicAdd(&L.stats[4], 1.0);
        // rows whose histogram this pass built (the side predicted smaller; the f32 and
        // wide paths count their separate child builds above)
        if (HIST && J.acc_right >= 0) atomicAdd(&L.stats[5], (double)(J.acc_right ? rc : lc));
      } else {
        ctl->part_left_count = lc;
      }
    }
  };
  // Two register buffers: the next tile's loads are in flight while this tile is
  // ranked, histogrammed and scattered (its stores queue behind those loads).  One
  // copy of the per-tile code (the buffers swap by register moves) keeps the kernel
  // small enough to stay in the instruction cache next to the round's other kernels.
  for (int64_t t = t_lo; t < t_hi; ++t) {
    const bool more = t + 1 < t_hi;
    if (more) jn = load(t + 1, next_b);
    process(t, jc, cur_b);
    if (more) {
      cur_b = next_b;
      jc = jn;
    }
  }
  if (HIST && cur >= 0 && s_jobs[cur].acc_right >= 0 && held > 0) flush();
}

// Stable per-op partition, step 1: the left-row count of every tile of job 0.
template <int FMT>
__global__ __launch_bounds__(PART_THREADS) void k_tile_count(DevLearner L) {
  constexpr int PT = PART_THREADS, PR = part_rows(FMT), kTile = PT * PR;
  constexpr int U = rec_words(FMT);
  __shared__ int32_t s_w[PT / LGBM_WAVE];
  const PartJob J = L.ctl->jobs[0];
  const int64_t t = blockIdx.x;
  if (t >= J.ntiles) return;
  const uint4* __restrict__ src = rec_buf(L.bufs, J.src_buf);
  int32_t n = 0;
  for (int k = 0; k < PR; ++k) {
    const int64_t p = t * kTile + (int64_t)k * PT + threadIdx.x;
    if (p >= J.count) continue;
    const int64_t phys = J.rev ? J.begin + J.count - 1 - p : J.begin + p;
    uint32_t w[U];
    rec_load<FMT>(src, phys, w);
    int fwi, fsh;
    rec_field_pos(FMT, J.fbyte, &fwi, &fsh);
    const int32_t bin = (int32_t)rec_field<FMT>(w, fwi, fsh);
    n += route_right(bin, J.pmin, J.max_bin, J.th, J.na_bin, J.flags) ? 0 : 1;
  }
  for (int off = 32; off >= 1; off >>= 1) n += __shfl_xor(n, off);
  if (lane_id() == 0) s_w[threadIdx.x >> 6] = n;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t s = 0;
    for (int i = 0; i < PT / LGBM_WAVE; ++i) s += s_w[i];
    L.tile_state[t] = (uint64_t)s;
  }
}

// Stable per-op partition, step 2: tile counts -> exclusive prefix (one block).
__global__ __launch_bounds__(1024) void k_tile_scan(DevLearner L) {
  __shared__ int64_t s_part[1024 / LGBM_WAVE];
  __shared__ int64_t s_carry;
  const int64_t n = L.ctl->jobs[0].ntiles;
  const int tid = threadIdx.x, lane = (int)lane_id(), wave = tid >> 6;
  if (tid == 0) s_carry = 0;
  __syncthreads();
  for (int64_t b0 = 0; b0 < n; b0 += 1024) {
    const int64_t i = b0 + tid;
    const int64_t v = i < n ? (int64_t)L.tile_state[i] : 0;
    int64_t incl = v;
    for (int off = 1; off < LGBM_WAVE; off <<= 1) {
      const int64_t u = __shfl_up(incl, off);
      if (lane >= off) incl += u;
    }
    if (lane == LGBM_WAVE - 1) s_part[wave] = incl;
    __syncthreads();
    int64_t before = s_carry;
    for (int k = 0; k < wave; ++k) before += s_part[k];
    if (i < n) L.tile_state[i] = (uint64_t)(before + incl - v);
    __syncthreads();
    if (tid == 1023) s_carry = before + incl;
    __syncthreads();
  }
}

// ===========================================================================
// k_pair_scan: block (feature f, job j), two waves.  The children of job j:
//   integer cells: the side built in the partition pass from the job's accumulator
//   (cleared after reading), the other side = parent - built (exact); both stored in
//   the children's integer slots;
//   smaller child (partition counts, a tie makes the right child the smaller one:
//   learner.rs:4061-4089): exact f64 cells -> FixHistogram on its RAW sums ->
//   compaction; larger = parent - smaller in f64 (histogram_pool.rs:249, not re-fixed);
//   wave 0 scans the smaller, wave 1 the larger.  Children of a gated pair
//   (before_find_best_split, learner.rs:1808-1839: max_depth reached, or both below
//   2 * min_data_in_leaf rows) are not built or scanned.
// ===========================================================================
// CAT: the dataset has categorical features (the categorical scan's LDS rows are
// allocated only then: without them more blocks fit a CU).  A round of the wide layout
// runs F x jobs blocks of ~15-20 us each, more than the chip holds at once, so blocks a
// CU can hold set its time: six waves a SIMD (at most 80 VGPRs) and 12.5 KB of LDS at
// 256 bins give 12 blocks a CU where 89 VGPRs and the categorical rows gave 8.
// FP: f32 gradients (64-bit fixed-point integer cells).
// GRID: quantized cells below 2^53 units, scanned with prefix_grid.
template <bool CAT, bool FP, bool GRID>
__global__ __launch_bounds__(SCAN_THREADS, 6) void k_pair_scan(DevLearner L, int32_t part_grid) {
  static_assert(SCAN_THREADS == 128, "two bins and four f64 cells per thread cover 256 bins");
  // the smaller child's and the larger child's f64 cells, sized for the widest feature
  extern __shared__ __align__(16) double scan_lds[];
  double* cs = scan_lds;
  double* cp = scan_lds + 2 * L.max_bins;
  Ctl* ctl = L.ctl;
  const int f = blockIdx.x, j = blockIdx.y;
  const int tid = threadIdx.x, F = L.F, cells = L.total_cells;
  // The loads are grouped so the block waits for three memory round trips — the job
  // record (with the feature and the round's uniforms), then everything the job
  // names, then the parent's cells — instead of one per dependent step.
  const int32_t n_jobs = ctl->n_jobs;
  const PartJob& J = ctl->jobs[j];  // slot j always exists; its fields are used below
  const int32_t p = J.parent, cl = J.cl, cr = J.cr, acc_right = J.acc_right;
  const int32_t acc_used = ctl->acc_used[j];
  const int32_t jnt = J.ntiles;
  const int64_t jt0 = J.tile0;
  const DevFeature ft = L.feats[f];
  const int64_t T = ctl->tile_total;
  const int32_t md = ctl->max_depth, min2 = ctl->cfg.min_data_in_leaf * 2;
  constexpr bool fp_mode = FP;
  const ScanCfg sc = make_scan_cfg(ctl->cfg);
  if (j >= n_jobs) return;  // only after the job's fields are known to be live
  const DevNodes& nd = L.nodes;
  const int32_t lcnt = nd.count[cl], rcnt = nd.count[cr], dcl = nd.depth[cl];
  LeafSums scl = nd.sums[cl], scr = nd.sums[cr];
  if (scl._pad) {
    // a categorical split whose SplitInfo counts order the children unlike the
    // partition: the reference seeds each child's scan with the other's sums and count
    // (seed_child_leaf_splits, learner.rs:4191-4229)
    const LeafSums t = scl;
    scl = scr;
    scr = t;
  }
  const bool pgate = L.splittable[(size_t)p * F + f] == 0;
  const int nb = (int)ft.num_bin;
  const size_t sl = L.slot_len;
  const double* s_par = L.slots + (size_t)p * sl + ft.slot_off;
  // Both children's f64 cells come from their integer cells (fix_compact_pair); only
  // a parent whose cells are materialised (pmat) is read.
  const bool pmat = L.fmat[p] != 0;
  const double2 pm = L.mfbv[(size_t)p * F + f];
  const bool gated = (md > 0 && dcl >= md) || (lcnt < min2 && rcnt < min2);
  const bool right_small = !(lcnt < rcnt);
  const int32_t sm = right_small ? cr : cl, lg = right_small ? cl : cr;
  const LeafSums ss = right_small ? scr : scl, gs = right_small ? scl : scr;
  // A smaller child without rows or hessian has its cells cleared, so the reference's
  // larger child is the parent's cells (not its own integers): it is materialised, as
  // is every larger child of a materialised parent.
  const bool sm_zero = !(ss.sh > 0.0 && ss.n > 0);
  const bool lg_mat = pmat || sm_zero;
  if (f == 0 && tid == 0) {
    L.fmat[sm] = 0;
    L.fmat[lg] = lg_mat ? 1 : 0;
  }
  const double vg1 = (double)ctl->vg1, vh1 = (double)ctl->vh1, vh3 = (double)ctl->vh3;
  const bool wide = rec_wide(L.fmt);
  if (pgate && !gated && (fp_mode || wide)) {
    // The parent cannot split on this feature (outside the column sample, or no
    // valid threshold), so neither child scans it and no descendant reads its cells;
    // these layouts hold no accumulator to clear (their partial slots are rewritten
    // every round).  The children get what the scan below would give them.
    if (tid == 0 || tid == LGBM_WAVE) {
      const int32_t leaf = tid == 0 ? sm : lg;
      const LeafSums ls = (tid == 0) == right_small ? scr : scl;
      split_set_none(&L.feat_split[(size_t)leaf * F + f]);
      L.gain_dense[(size_t)leaf * F + f] = -__builtin_inf();
      if (ls.sh > 0.0 && ls.n > 0) L.splittable[(size_t)leaf * F + f] = 0;
    }
    return;
  }
  if constexpr (fp_mode) {
    // f32 gradients: the smaller child from its partial slots (k_hist_f32's, or the
    // wide layout's per-chunk ones); the larger = parent - smaller, exact in 64-bit
    // fixed point
    const int32_t a0 = ctl->hjobs[j].a0, na = ctl->hjobs[j].nblk;
    const double gu = ldexp(1.0, -ctl->g_shift), hu = ldexp(1.0, -ctl->h_shift);
    if (!gated) {
      for (int b = tid; b < nb; b += SCAN_THREADS) {
        const size_t ci = (size_t)(ft.cell_base + b);
        long long SG = 0, SH = 0;
        if (wide) {
          // the job's chunks, four loads in flight at a time (integer sums: any order)
          const ulonglong2* wp = (const ulonglong2*)L.wide_part + (size_t)a0 * cells + ci;
          int k = 0;
          for (; k + 4 <= na; k += 4) {
            ulonglong2 x[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) x[u] = wp[(size_t)(k + u) * cells];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              SG += (long long)x[u].x;
              SH += (long long)x[u].y;
            }
          }
          for (; k < na; ++k) {
            const ulonglong2 x = wp[(size_t)k * cells];
            SG += (long long)x.x;
            SH += (long long)x.y;
          }
        } else {
          hist_part_sum64(L, a0, na, ci, &SG, &SH);
        }
        const int64_t* ps = L.int_slots64 + ((size_t)p * cells + ci) * 2;
        int64_t* sp_ = L.int_slots64 + ((size_t)sm * cells + ci) * 2;
        int64_t* gp_ = L.int_slots64 + ((size_t)lg * cells + ci) * 2;
        const int64_t PG = ps[0], PH = ps[1];
        sp_[0] = SG;
        sp_[1] = SH;
        gp_[0] = PG - SG;
        gp_[1] = PH - SH;
        cs[2 * b] = (double)SG * gu;
        cs[2 * b + 1] = (double)SH * hu;
        // the larger child's cells from its exact integers (or the parent's, when the
        // larger is materialised): one rounding instead of one per subtraction level
        cp[2 * b] = (double)(lg_mat ? PG : PG - SG) * gu;
        cp[2 * b + 1] = (double)(lg_mat ? PH : PH - SH) * hu;
      }
    }
  } else {
    // the side built in the partition pass: for a job spread over few blocks its
    // per-block slots (the blocks of the partition launch from the one holding its
    // first tile to the one holding its last, slot = block + j; blocks without tiles
    // wrote nothing), plus the job's accumulator when a flush used it (read and
    // cleared even when the children are gated)
    // (wide: k_hist_wide's per-chunk slots)
    const int64_t s0 = jnt > 0 ? part_owner(jt0, T, part_grid) : 0;
    const int64_t s1 = jnt > 0 ? part_owner(jt0 + jnt - 1, T, part_grid) : -1;
    const bool use_slots =
        !wide && (jnt > 0 ? part_span_blocks(jt0, jnt, T, part_grid) <= PART_SLOT_MAX : true);
    const bool read_acc = !wide && (!use_slots || acc_used != 0);
    const bool acc_packed = J.count <= PACKED_ACC_MAX_ROWS;
    unsigned long long* accp = L.hist_accp + (size_t)j * L.acc_cells;
    const int32_t wa0 = ctl->hjobs[j].a0, wna = wide ? ctl->hjobs[j].nblk : 0;
    int32_t* acc = L.hist_acc + (size_t)j * L.acc_cells * 3;
    const unsigned long long* slots = L.part_slots;
    for (int b0 = 0; b0 < nb; b0 += 2 * SCAN_THREADS)  // one pass below 257 bins
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int b = b0 + tid + SCAN_THREADS * q;
      if (b >= nb) continue;
      const size_t ci = (size_t)(ft.cell_base + b);
      int32_t AG = 0, AH = 0, AT = 0;
      if (read_acc && acc_packed) {
        unpack_cell(accp[ci], &AG, &AH, &AT);
        accp[ci] = 0ull;
      } else if (read_acc) {
        int32_t* a = acc + ci * 3;
        AG = a[0];
        AH = a[1];
        AT = a[2];
        a[0] = 0;
        a[1] = 0;
        a[2] = 0;
      }
      {
        // the job's chunks (wide layout), four loads in flight at a time
        const unsigned long long* wp = L.wide_part + (size_t)wa0 * cells + ci;
        int k = 0;
        for (; k + 4 <= wna; k += 4) {
          unsigned long long x[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) x[u] = wp[(size_t)(k + u) * cells];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            int32_t g_, h_, t_;
            unpack_cell(x[u], &g_, &h_, &t_);
            AG += g_;
            AH += h_;
            AT += t_;
          }
        }
        for (; k < wna; ++k) {
          int32_t g_, h_, t_;
          unpack_cell(wp[(size_t)k * cells], &g_, &h_, &t_);
          AG += g_;
          AH += h_;
          AT += t_;
        }
      }
      if (use_slots) {
        // at most PART_SLOT_MAX blocks, enumerated without a dependent chain so all
        // their loads are issued before the sums: with fewer tiles than blocks each
        // tile has a block of its own, otherwise every block from s0 to s1 has tiles
#pragma unroll
        for (int u = 0; u < PART_SLOT_MAX; ++u) {
          int64_t k;
          if (T < part_grid) {
            if (u >= jnt) continue;
            k = part_owner(jt0 + u, T, part_grid);
          } else {
            k = s0 + u;
            if (k > s1) continue;
          }
          int32_t sg_, sh_, st_;
          unpack_cell(slots[(size_t)(k + j) * cells + ci], &sg_, &sh_, &st_);
          AG += sg_;
          AH += sh_;
          AT += st_;
        }
      }
      if (gated) continue;
      const int32_t* ps = L.int_slots + ((size_t)p * cells + ci) * 3;
      const int32_t PG = ps[0], PH = ps[1], PT = ps[2];
      const int32_t OG = PG - AG, OH = PH - AH, OT = PT - AT;  // exact
      int32_t* ls = L.int_slots + ((size_t)cl * cells + ci) * 3;
      int32_t* rs = L.int_slots + ((size_t)cr * cells + ci) * 3;
      const int32_t LG_ = acc_right ? OG : AG, LH = acc_right ? OH : AH, LT = acc_right ? OT : AT;
      const int32_t RG = acc_right ? AG : OG, RH = acc_right ? AH : OH, RT = acc_right ? AT : OT;
      ls[0] = LG_;
      ls[1] = LH;
      ls[2] = LT;
      rs[0] = RG;
      rs[1] = RH;
      rs[2] = RT;
      if (right_small)
        int_cell_to_f64(RG, RH, RT, vg1, vh1, vh3, &cs[2 * b], &cs[2 * b + 1]);
      else
        int_cell_to_f64(LG_, LH, LT, vg1, vh1, vh3, &cs[2 * b], &cs[2 * b + 1]);
      {
        // the larger child's cells, or the parent's when the larger is materialised
        if (lg_mat)
          int_cell_to_f64(PG, PH, PT, vg1, vh1, vh3, &cp[2 * b], &cp[2 * b + 1]);
        else if (right_small)
          int_cell_to_f64(LG_, LH, LT, vg1, vh1, vh3, &cp[2 * b], &cp[2 * b + 1]);
        else
          int_cell_to_f64(RG, RH, RT, vg1, vh1, vh3, &cp[2 * b], &cp[2 * b + 1]);
      }
    }
  }
  if (gated) {
    if (tid == 0) {
      split_set_none(&L.feat_split[(size_t)cl * F + f]);
      split_set_none(&L.feat_split[(size_t)cr * F + f]);
      L.gain_dense[(size_t)cl * F + f] = -__builtin_inf();
      L.gain_dense[(size_t)cr * F + f] = -__builtin_inf();
    }
    return;
  }
  double* s_lg = L.slots + (size_t)lg * sl + ft.slot_off;
  fix_compact_pair(ft, cs, cp, ss.sg, ss.sh, pgate || sm_zero, pm, !lg_mat);
  if (lg_mat) {
    // larger = parent - smaller cell by cell, kept in the node's f64 slot
    for (int i = tid; i < 2 * nb; i += SCAN_THREADS) {
      const double d = (pmat ? s_par[i] : cp[i]) - cs[i];
      cp[i] = d;
      s_lg[i] = d;
    }
  }
  __syncthreads();
  const int mfb = (int)ft.mfb, tm = mfb - ft.offset;
  if (tid == 0 && mfb > 0 && mfb < nb && tm >= 0) {
    L.mfbv[(size_t)sm * F + f] = make_double2(cs[2 * tm], cs[2 * tm + 1]);
    L.mfbv[(size_t)lg * F + f] = make_double2(cp[2 * tm], cp[2 * tm + 1]);
  }
  const int wv = tid >> 6;
  const int32_t leaf = wv == 0 ? sm : lg;
  const LeafSums ls = wv == 0 ? ss : gs;
  lgbm_split_info* out = L.feat_split + (size_t)leaf * F + f;
  double* out_gain = L.gain_dense + (size_t)leaf * F + f;
  if (!(ls.sh > 0.0 && ls.n > 0)) {
    if (lane_id() == 0) {
      split_set_none(out);
      *out_gain = -__builtin_inf();
    }
  } else if (pgate) {
    if (lane_id() == 0) {
      split_set_none(out);
      *out_gain = -__builtin_inf();
      L.splittable[(size_t)leaf * F + f] = 0;
    }
  } else {
    double gain;
    if constexpr (CAT)
      gain = ft.categorical  // bin_type dispatch (learner.rs:3103-3118)
                 ? wave_scan_cat(wv == 0 ? cs : cp, ft, sc, ctl->cfg, ls.sg, ls.sh, ls.n,
                                 ls.weight, out, L.cat_bits + ((size_t)leaf * F + f) * 8)
                 : wave_scan<GRID>(wv == 0 ? cs : cp, ft, sc, ls.sg, ls.sh, ls.n, ls.weight, out);
    else
      gain = wave_scan<GRID>(wv == 0 ? cs : cp, ft, sc, ls.sg, ls.sh, ls.n, ls.weight, out);
    if (lane_id() == 0) {
      // splittability from the raw scan, then feature_contri scales the gain the
      // ArgMax compares (learner.rs:3235-3252)
      L.splittable[(size_t)leaf * F + f] = gain > -__builtin_inf() ? 1 : 0;
      out->gain = gain * ft.penalty;
      *out_gain = gain * ft.penalty;
    }
  }
}

// ===========================================================================
// k_tree_finalize: the Tree's leaf arrays from the committed leaves' node slots
// (leaf_value = the leaf's output, leaf_weight = its sum_hessian, 0 for an unsplit
// root: Tree::root, learner.rs:5398-5424), its linkage and real thresholds, the
// score-update routes, and the per-leaf ranges of the LeafPartitionLayout.
// ===========================================================================
__global__ void k_tree_finalize(DevLearner L) {
  const Ctl* ctl = L.ctl;
  const int32_t nl = ctl->num_leaves;
  DevTree& T = L.tree;
  const DevNodes& nd = L.nodes;
  const int32_t* ps = L.plan_state;
  for (int l = threadIdx.x; l < nl; l += blockDim.x) {
    const int32_t s = ps[PS_LEAF_SLOT * MAX_LEAVES + l];
    T.leaf_parent[l] = ps[PS_LEAF_PARENT * MAX_LEAVES + l];
    T.leaf_value[l] = nd.sums[s].weight;
    T.leaf_weight[l] = s == 0 ? 0.0 : nd.sums[s].sh;
    T.leaf_count[l] = nd.count[s];
    T.leaf_depth[l] = nd.depth[s];
    L.leaves.begin[l] = nd.begin[s];
    L.leaves.count[l] = nd.count[s];
    L.leaves.buf[l] = nd.buf[s];
    L.leaves.rev[l] = nd.rev[s];
  }
  for (int n = threadIdx.x; n < nl - 1; n += blockDim.x) {
    const int32_t lc = ps[PS_NODE_LEFT * MAX_LEAVES + n], rc = ps[PS_NODE_RIGHT * MAX_LEAVES + n];
    T.left_child[n] = lc;
    T.right_child[n] = rc;
    T.nodes[n].left = lc;
    T.nodes[n].right = rc;
    // real_threshold (learner.rs:198-203): the bin's upper bound
    const uint32_t tb = T.threshold_in_bin[n];
    T.threshold[n] = L.ub ? L.ub[L.feats[T.nodes[n].f].ub_off + tb] : (double)tb;
    // the score update's routes: the bins going right as a 256-bit set, and the
    // record byte and children packed in one word (children fit 12 signed bits)
    const NodeRoute r = T.nodes[n];
#pragma unroll
    for (int w = 0; w < 8; ++w)
      T.route_mask[n * 8 + w] = (r.flags & ROUTE_CAT)
                                    ? ~T.cat_left[n * 8 + w]
                                    : route_right_word(w, r.pmin, r.max_bin, r.th, r.na_bin, r.flags);
    T.route_node[n] = ((uint32_t)r.f & 0xffu) | (((uint32_t)lc & 0xfffu) << 8) |
                      (((uint32_t)rc & 0xfffu) << 20);
  }
  if (threadIdx.x == 0) {
    T.header[0] = nl;
    T.header[1] = ctl->error;
    T.header[2] = ctl->rounds;
    T.header[3] = ctl->done;
  }
}

// Exports the partition layout the way DataPartition::split leaves it: each leaf's
// rows in ascending row order at the leaf's begin offset (the leaf of every row by a
// walk of the tree over its original record, k_walk; then a stable rank of every row
// within its leaf), whatever the storage order inside the leaf.

// Stable rank of every row among the rows of its leaf, RANK_ROWS rows per block in
// row order: wave peers by eight key-bit ballots, waves in order through LDS, and a
// running per-leaf count.  COUNT pass: per (leaf, block) row counts.  Scatter pass:
// indices[offset of (leaf, block) + rank in block] = row.
#define RANK_THREADS 256
#define RANK_ROWS 1024
template <bool SCATTER>
__global__ __launch_bounds__(RANK_THREADS) void k_leaf_rank(const uint8_t* __restrict__ leaf_of,
                                                          int64_t n, int32_t nl, int64_t nblk,
                                                          uint32_t* __restrict__ tab,
                                                          uint32_t* __restrict__ indices) {
  constexpr int kWaves = RANK_THREADS / LGBM_WAVE;
  __shared__ uint32_t run[256];
  __shared__ uint32_t wc[kWaves][256];
  const int tid = threadIdx.x, wave = tid >> 6;
  const int64_t blk = blockIdx.x;
  for (int i = tid; i < 256; i += RANK_THREADS) {
    run[i] = 0u;
    for (int w = 0; w < kWaves; ++w) wc[w][i] = 0u;
  }
  __syncthreads();
  for (int k = 0; k < RANK_ROWS / RANK_THREADS; ++k) {
    const int64_t r = blk * RANK_ROWS + (int64_t)k * RANK_THREADS + tid;
    const bool valid = r < n;
    const uint32_t key = valid ? (uint32_t)leaf_of[r] : 0u;
    unsigned long long peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const bool set = (key >> bit) & 1u;
      const unsigned long long bb = __ballot(set);
      peers &= set ? bb : ~bb;
    }
    const unsigned long long before = peers & lanemask_lt();
    if (valid && before == 0ull) wc[wave][key] = (uint32_t)__popcll(peers);
    __syncthreads();
    if (SCATTER && valid) {
      uint32_t off = run[key] + (uint32_t)__popcll(before);
      for (int w = 0; w < wave; ++w) off += wc[w][key];
      indices[tab[(size_t)key * nblk + blk] + off] = (uint32_t)r;
    }
    __syncthreads();
    for (int i = tid; i < 256; i += RANK_THREADS) {
      uint32_t add = 0u;
      for (int w = 0; w < kWaves; ++w) {
        add += wc[w][i];
        wc[w][i] = 0u;
      }
      run[i] += add;
    }
    __syncthreads();
  }
  if (!SCATTER)
    for (int i = tid; i < nl; i += RANK_THREADS) tab[(size_t)i * nblk + blk] = run[i];
}

// Per leaf (one block each): (leaf, block) counts -> output offsets, starting at the
// leaf's begin.
__global__ __launch_bounds__(1024) void k_leaf_rank_offsets(DevLearner L, int64_t nblk,
                                                            uint32_t* __restrict__ tab) {
  __shared__ int64_t s_part[1024 / LGBM_WAVE];
  __shared__ int64_t s_carry;
  const int32_t l = blockIdx.x;
  const int tid = threadIdx.x, lane = (int)lane_id(), wave = tid >> 6;
  uint32_t* row = tab + (size_t)l * nblk;
  if (tid == 0) s_carry = L.leaves.begin[l];
  __syncthreads();
  for (int64_t b0 = 0; b0 < nblk; b0 += 1024) {
    const int64_t i = b0 + tid;
    const int64_t v = i < nblk ? (int64_t)row[i] : 0;
    int64_t incl = v;
    for (int off = 1; off < LGBM_WAVE; off <<= 1) {
      const int64_t u = __shfl_up(incl, off);
      if (lane >= off) incl += u;
    }
    if (lane == LGBM_WAVE - 1) s_part[wave] = incl;
    __syncthreads();
    int64_t before = s_carry;
    for (int k = 0; k < wave; ++k) before += s_part[k];
    if (i < nblk) row[i] = (uint32_t)(before + incl - v);
    __syncthreads();
    if (tid == 1023) s_carry = before + incl;
    __syncthreads();
  }
}

// ===========================================================================
// quant_train_renew_leaf (gbdt.rs:936-943,1194-1212; renew_tree_output,
// learner.rs:4411-4429): after a quantized tree, every leaf's output from the ORIGINAL
// f32 gradients, -ThresholdL1(sum_g, l1) / (sum_h + l2), the sums an ordered f64 fold
// over the leaf's rows in partition order (the exported layout: each leaf's rows
// ascending, DataPartition::split's order).  One thread per leaf walks its rows
// sequentially (the fold's order is its value); the loads run eight rows ahead.
// ===========================================================================
__global__ __launch_bounds__(256) void k_renew_leaves(DevLearner L, const uint32_t* __restrict__ indices,
                                                      const float* __restrict__ g,
                                                      const float* __restrict__ h, double l1,
                                                      double l2) {
  const int32_t nl = L.ctl->num_leaves;
  const int l = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (nl <= 1 || l >= nl) return;  // renew_tree_output skips a single-leaf tree
  const int32_t c = L.leaves.count[l];
  const uint32_t* __restrict__ rows = indices + L.leaves.begin[l];
  double sg = 0.0, sh = 0.0;
  int32_t k = 0;
  for (; k + 8 <= c; k += 8) {
    uint32_t r[8];
    float gv[8], hv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) r[u] = rows[k + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      gv[u] = g[r[u]];
      hv[u] = h[r[u]];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      sg += (double)gv[u];
      sh += (double)hv[u];
    }
  }
  for (; k < c; ++k) {
    const uint32_t r = rows[k];
    sg += (double)g[r];
    sh += (double)h[r];
  }
  L.tree.leaf_value[l] = -threshold_l1(sg, l1) / (sh + l2);
}

// ===========================================================================
// launchers
// ===========================================================================
void launch_tree_init(const DevLearner& L, int32_t max_leaves, int32_t max_depth, int32_t slot_cap,
                      int32_t spec_max, int32_t fp_mode, hipStream_t s, const KernelEvents* ev) {
  KLAUNCH(ev, k_tree_init, dim3(16), dim3(256), 0, s, L, max_leaves, max_depth, slot_cap, spec_max,
          fp_mode);
}
void launch_plan(const DevLearner& L, int32_t slot_cap, hipStream_t s, const KernelEvents* ev) {
  KLAUNCH(ev, k_plan, dim3(1), dim3(PLAN_THREADS), 0, s, L, slot_cap);
}
void launch_partition(const DevLearner& L, int fp, int64_t blocks, hipStream_t s,
                      const KernelEvents* ev) {
  if (blocks < 1) blocks = 1;
  const dim3 g((unsigned)blocks), b(PART_THREADS);
  if (rec_wide(L.fmt)) {
    if (fp)
      KLAUNCH(ev, (k_partition<REC_FMT_WIDE, 1, false>), g, b, 0, s, L);
    else
      KLAUNCH(ev, (k_partition<REC_FMT_WIDE, 0, false>), g, b, 0, s, L);
  } else if (fp) {
    DISPATCH_FMT(L.fmt, KLAUNCH(ev, (k_partition<kF, 1, false>), g, b, 0, s, L));
  } else {
    const size_t lds = (size_t)(std::max(L.total_cells, 1) + LDS_TRASH_CELLS) * sizeof(unsigned long long);
    DISPATCH_FMT(L.fmt, KLAUNCH(ev, (k_partition<kF, 0, false>), g, b, lds, s, L));
  }
}
void launch_partition_stable(const DevLearner& L, int64_t ntiles, int64_t blocks, hipStream_t s) {
  if (blocks < 1) blocks = 1;
  k_tile_count<1><<<dim3((unsigned)ntiles), dim3(PART_THREADS), 0, s>>>(L);
  k_tile_scan<<<dim3(1), dim3(1024), 0, s>>>(L);
  const size_t lds = (size_t)(std::max(L.total_cells, 1) + LDS_TRASH_CELLS) * sizeof(unsigned long long);
  k_partition<1, 0, true><<<dim3((unsigned)blocks), dim3(PART_THREADS), lds, s>>>(L);
}
// Lets the scans take LDS rows for the widest feature (2-byte bins: 4096 bins, 128 KiB
// for k_pair_scan's two children); called outside graph capture.
int scan_prepare() {
  const void* k[6] = {(const void*)k_pair_scan<false, false, false>,
                      (const void*)k_pair_scan<true, false, false>,
                      (const void*)k_pair_scan<false, true, false>,
                      (const void*)k_pair_scan<true, true, false>,
                      (const void*)k_pair_scan<false, false, true>,
                      (const void*)k_pair_scan<true, false, true>};
  for (int i = 0; i < 6; ++i)
    if (hipFuncSetAttribute(k[i], hipFuncAttributeMaxDynamicSharedMemorySize,
                            4 * WIDE_MAX_BIN * (int)sizeof(double)) != hipSuccess)
      return 1;
  return 0;
}

void launch_pair_scan(const DevLearner& L, int fp, int32_t spec_max, int32_t part_grid,
                      hipStream_t s, const KernelEvents* ev) {
  const size_t lds = (size_t)4 * std::max(L.max_bins, 1) * sizeof(double);
  const dim3 g((unsigned)L.F, (unsigned)spec_max), b(SCAN_THREADS);
  // quantized cells are exact unit multiples while every sum stays below 2^53 units
  // (fewer than 2^24 rows); the grid prefix pays where a scan spans several 64-candidate
  // batches (at most 64 candidates: one batch, as cheap in order)
  const bool grid = !fp && L.N < (int64_t(1) << 24) && L.max_bins > LGBM_WAVE + 1;
  if (L.has_cat) {
    if (fp)
      KLAUNCH(ev, (k_pair_scan<true, true, false>), g, b, lds, s, L, part_grid);
    else if (grid)
      KLAUNCH(ev, (k_pair_scan<true, false, true>), g, b, lds, s, L, part_grid);
    else
      KLAUNCH(ev, (k_pair_scan<true, false, false>), g, b, lds, s, L, part_grid);
  } else if (fp) {
    KLAUNCH(ev, (k_pair_scan<false, true, false>), g, b, lds, s, L, part_grid);
  } else if (grid) {
    KLAUNCH(ev, (k_pair_scan<false, false, true>), g, b, lds, s, L, part_grid);
  } else {
    KLAUNCH(ev, (k_pair_scan<false, false, false>), g, b, lds, s, L, part_grid);
  }
}
void launch_tree_finalize(const DevLearner& L, hipStream_t s, const KernelEvents* ev) {
  KLAUNCH(ev, k_tree_finalize, dim3(1), dim3(256), 0, s, L);
}
void launch_renew_leaves(const DevLearner& L, const uint32_t* indices, const float* g,
                         const float* h, double l1, double l2, hipStream_t s) {
  k_renew_leaves<<<dim3(1), dim3(256), 0, s>>>(L, indices, g, h, l1, l2);
}
size_t export_layout_scratch_bytes(int64_t n, int32_t num_leaves) {
  const int64_t nblk = (n + RANK_ROWS - 1) / RANK_ROWS;
  return (((size_t)n + 255) & ~(size_t)255) + (size_t)num_leaves * (size_t)nblk * 4;
}
void launch_export_layout(const DevLearner& L, int32_t num_leaves, uint32_t* indices,
                          void* scratch, hipStream_t s) {
  const int64_t n = L.N, nblk = (n + RANK_ROWS - 1) / RANK_ROWS;
  uint8_t* leaf_of = (uint8_t*)scratch;
  uint32_t* tab = (uint32_t*)((char*)scratch + (((size_t)n + 255) & ~(size_t)255));
  launch_leaf_of(L, leaf_of, s);
  k_leaf_rank<false><<<dim3((unsigned)nblk), dim3(RANK_THREADS), 0, s>>>(leaf_of, n, num_leaves,
                                                                        nblk, tab, nullptr);
  k_leaf_rank_offsets<<<dim3((unsigned)num_leaves), dim3(1024), 0, s>>>(L, nblk, tab);
  k_leaf_rank<true><<<dim3((unsigned)nblk), dim3(RANK_THREADS), 0, s>>>(leaf_of, n, num_leaves,
                                                                       nblk, tab, indices);
}

}  // namespace lgbm
