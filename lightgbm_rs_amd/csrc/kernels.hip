// kernels.hip — gfx950 kernels of the tree-learner hot path and their launchers.
//
//   k_pack_records   resident bin layout (upload_resident_bins, lib.rs:4368-4433)
//   k_grad_binary    BinaryLogloss::get_gradients (lgbm-objective/src/binary.rs:134-172)
//   k_absmax         compute_scales max-abs pass (gradient_discretizer.rs:145-165)
//   k_quant_scales   compute_scales scale math
//   k_quantize       discretize (+ dequantized write-back), xorshift64 with jump-ahead
//   k_hist           ConstructHistogram (integer, exact) (lib.rs:262-390 is the f64 fold)
//   k_fixscan        f64 cells + FixHistogram + compaction + subtraction trick +
//                    FindBestThreshold (fix_histogram.rs:50-80, learner.rs:4460-4492,
//                    histogram_pool.rs:249, kernels/split.rs:8970-9329)
//   split_step       (last block of k_fixscan) per-leaf argmax (learner.rs:3290-3330),
//                    cross-leaf ArgMax (learner.rs:4537), Tree::split (tree.rs:614-700)
//   k_partition      DataPartition::split (data_partition.rs:192-288,360-463)
//   k_score_update   score update through the grown tree (score_updater.rs:133;
//                    learner.rs:4380-4395)
#include "scan.h"

#include <hip/hip_ext.h>

#include <algorithm>

namespace lgbm {

// ===========================================================================
// upload: feature-major u8 -> records
// ===========================================================================
__global__ void k_pack_records(const uint8_t* __restrict__ bins, int64_t n, int32_t F, int32_t W,
                               uint4* __restrict__ rec) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n) return;
  uint32_t words[4 * LGBM_MAX_W];
  for (int i = 0; i < 4 * W; ++i) words[i] = 0u;
  for (int f = 0; f < F; ++f) words[f >> 2] |= (uint32_t)bins[(size_t)f * n + r] << (8 * (f & 3));
  words[4 * W - 1] = (uint32_t)r;
  for (int w = 0; w < W; ++w)
    rec[r * W + w] = make_uint4(words[4 * w], words[4 * w + 1], words[4 * w + 2], words[4 * w + 3]);
}

// ===========================================================================
// max-abs / constant-hessian reduction
// ===========================================================================
__device__ __forceinline__ uint32_t f32_order_key(float x) {
  uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float f32_from_key(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(b);
}

// Per-block partial statistics of (g, h): max |g|, max |h| (f64::max ignores NaN, so a
// NaN contributes nothing) and min/max of h for the all-equal test of
// quantize_grad_hess_in_place (gbdt.rs:54).  No atomics: each block writes one
// partial and k_quant_scales reduces them.
struct GhStat {
  uint32_t ag, ah, hmin, hmax;
};
__device__ __forceinline__ void stat_add(GhStat& s, float gv, float hv) {
  if (gv == gv) s.ag = max(s.ag, __float_as_uint(fabsf(gv)));
  if (hv == hv) {
    s.ah = max(s.ah, __float_as_uint(fabsf(hv)));
    const uint32_t k = f32_order_key(hv);
    s.hmin = min(s.hmin, k);
    s.hmax = max(s.hmax, k);
  }
}
__device__ __forceinline__ void stat_merge(GhStat& a, const GhStat& b) {
  a.ag = max(a.ag, b.ag);
  a.ah = max(a.ah, b.ah);
  a.hmin = min(a.hmin, b.hmin);
  a.hmax = max(a.hmax, b.hmax);
}
__device__ void block_stat_write(GhStat s, uint4* __restrict__ partials) {
  __shared__ GhStat sh[16];
  for (int off = 32; off >= 1; off >>= 1) {
    GhStat o;
    o.ag = (uint32_t)__shfl_xor((int)s.ag, off);
    o.ah = (uint32_t)__shfl_xor((int)s.ah, off);
    o.hmin = (uint32_t)__shfl_xor((int)s.hmin, off);
    o.hmax = (uint32_t)__shfl_xor((int)s.hmax, off);
    stat_merge(s, o);
  }
  if (lane_id() == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    GhStat r = sh[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) stat_merge(r, sh[w]);
    partials[blockIdx.x] = make_uint4(r.ag, r.ah, r.hmin, r.hmax);
  }
}

__global__ __launch_bounds__(256) void k_absmax(const float* __restrict__ g,
                                                const float* __restrict__ h, int64_t n,
                                                uint4* __restrict__ partials) {
  GhStat s{0u, 0u, 0xffffffffu, 0u};
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride)
    stat_add(s, g[r], h[r]);
  block_stat_write(s, partials);
}

// BinaryLogloss::get_gradients (binary.rs:134-172), sigmoid = 1, balanced weights.
__global__ __launch_bounds__(256) void k_grad_binary(const double* __restrict__ score,
                                                     const float* __restrict__ label,
                                                     float* __restrict__ g, float* __restrict__ h,
                                                     int64_t n, uint4* __restrict__ partials) {
  GhStat s{0u, 0u, 0xffffffffu, 0u};
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const double sigmoid = 1.0;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride) {
    const bool pos = label[r] > 0.0f;
    const double lv = pos ? 1.0 : -1.0;
    const double resp = -lv * sigmoid / (1.0 + exp(lv * sigmoid * score[r]));
    const double ar = fabs(resp);
    const float gv = (float)(resp * 1.0);
    const float hv = (float)(ar * (sigmoid - ar) * 1.0);
    g[r] = gv;
    h[r] = hv;
    stat_add(s, gv, hv);
  }
  block_stat_write(s, partials);
}

// compute_scales (gradient_discretizer.rs:145-165) from the reduced statistics.
__global__ __launch_bounds__(256) void k_quant_scales(Ctl* ctl, const uint4* __restrict__ partials,
                                                      int32_t nparts, int32_t bins,
                                                      int32_t force_const) {
  GhStat s{0u, 0u, 0xffffffffu, 0u};
  for (int i = threadIdx.x; i < nparts; i += blockDim.x) {
    const uint4 p = partials[i];
    stat_merge(s, GhStat{p.x, p.y, p.z, p.w});
  }
  __shared__ GhStat sh[4];
  for (int off = 32; off >= 1; off >>= 1) {
    GhStat o;
    o.ag = (uint32_t)__shfl_xor((int)s.ag, off);
    o.ah = (uint32_t)__shfl_xor((int)s.ah, off);
    o.hmin = (uint32_t)__shfl_xor((int)s.hmin, off);
    o.hmax = (uint32_t)__shfl_xor((int)s.hmax, off);
    stat_merge(s, o);
  }
  if (lane_id() == 0) sh[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) stat_merge(s, sh[w]);
  const double mg = (double)__uint_as_float(s.ag);
  const double mh = (double)__uint_as_float(s.ah);
  bool ch;
  if (force_const >= 0) {
    ch = force_const != 0;
  } else {
    ch = f32_from_key(s.hmin) == f32_from_key(s.hmax);
  }
  const double half = (double)(bins / 2);
  ctl->gs = mg / half;
  ctl->hs = ch ? mh : mh / (double)bins;
  ctl->igs = 1.0 / ctl->gs;
  ctl->ihs = 1.0 / ctl->hs;
  ctl->vg1 = (float)(1.0 * ctl->gs);
  ctl->vh1 = (float)(1.0 * ctl->hs);
  ctl->vh3 = (float)(3.0 * ctl->hs);
  ctl->const_hess = ch ? 1 : 0;
  ctl->quant_bins = bins;
}

// ===========================================================================
// quantize: discretize_dequantize_in_place (gradient_discretizer.rs:126-139,
// quantize_pair :173-188, next_u01 :255-263).  Row r consumes xorshift draws
// 2r+1 (grad) and 2r+2 (hess) of the sequential stream; a lane starts at row
// wave_row0 + lane*C with state M^(2*(row)) s0, M being the GF(2) matrix of one
// xorshift step: the wave applies the precomputed powers P_k = M^(2*64*C*2^k)
// cooperatively (lane i owns column i, xor-reduce), then each lane applies
// R_k = M^(2*C*2^k) for the bits of its lane id.
// ===========================================================================
__device__ __forceinline__ double next_u01(uint64_t& s) {
  uint64_t x = s;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  s = x;
  return (double)(x >> 11) / (double)(1ull << 53);
}

// Rows per block: 4 waves x 64 lanes x QUANT_ROWS_PER_LANE.  g/h are staged through
// LDS so global loads and stores are coalesced while each lane walks its own run of
// consecutive rows (padded index: one spare slot per 16 rows avoids bank conflicts).
#define QUANT_BLOCK_ROWS (4 * LGBM_WAVE * QUANT_ROWS_PER_LANE)
__device__ __forceinline__ int qidx(int r) { return r + (r >> 4); }

__global__ __launch_bounds__(256) void k_quantize(const float* __restrict__ g,
                                                  const float* __restrict__ h, int64_t n,
                                                  const Ctl* __restrict__ ctl,
                                                  const uint64_t* __restrict__ wave_mats,
                                                  const uint64_t* __restrict__ lane_mats,
                                                  uint64_t s0, int32_t stochastic,
                                                  uint16_t* __restrict__ gh,
                                                  float* __restrict__ dg, float* __restrict__ dh) {
  __shared__ float sg_[QUANT_BLOCK_ROWS + QUANT_BLOCK_ROWS / 16];
  __shared__ float sh_[QUANT_BLOCK_ROWS + QUANT_BLOCK_ROWS / 16];
  __shared__ uint16_t sq_[QUANT_BLOCK_ROWS + QUANT_BLOCK_ROWS / 16];
  const int64_t brow0 = (int64_t)blockIdx.x * QUANT_BLOCK_ROWS;
  if (brow0 >= n) return;
  const int tid = threadIdx.x;
  const int64_t nblk = min((int64_t)QUANT_BLOCK_ROWS, n - brow0);
  for (int r = tid; r < QUANT_BLOCK_ROWS; r += 256) {
    const bool v = r < nblk;
    sg_[qidx(r)] = v ? g[brow0 + r] : 0.f;
    sh_[qidx(r)] = v ? h[brow0 + r] : 0.f;
  }
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + tid) >> 6;
  const int lane = (int)lane_id();
  const double igs = ctl->igs, ihs = ctl->ihs, gs = ctl->gs, hs = ctl->hs;
  const bool ch = ctl->const_hess != 0;
  uint64_t st = 0;
  if (stochastic) {
    uint64_t sw = s0;
    for (int k = 0; k < QUANT_WAVE_MATS; ++k) {
      if ((wave >> k) & 1) {
        uint64_t term = ((sw >> lane) & 1ull) ? wave_mats[k * 64 + lane] : 0ull;
        for (int off = 32; off >= 1; off >>= 1) term ^= __shfl_xor(term, off);
        sw = term;
      }
    }
    uint64_t sl = sw;
    for (int k = 0; k < QUANT_LANE_MATS; ++k) {
      uint64_t y = 0ull;
      for (int i = 0; i < 64; ++i) {
        const uint64_t col = lane_mats[k * 64 + i];
        y ^= ((sl >> i) & 1ull) ? col : 0ull;
      }
      if ((lane >> k) & 1) sl = y;
    }
    st = sl;
  }
  __syncthreads();
  const int lrow = (tid >> 6) * (LGBM_WAVE * QUANT_ROWS_PER_LANE) + lane * QUANT_ROWS_PER_LANE;
  for (int j = 0; j < QUANT_ROWS_PER_LANE; ++j) {
    const int r = lrow + j;
    if (r >= nblk) break;
    const float gv = sg_[qidx(r)], hv = sh_[qidx(r)];
    double bg = 0.5, bh = 0.5;
    if (stochastic) {
      bg = next_u01(st);
      bh = next_u01(st);
    }
    const double x = (double)gv * igs;
    const int8_t qg = sat_i8(gv >= 0.0f ? x + bg : x - bg);
    const int8_t qh = ch ? (int8_t)1 : sat_i8((double)hv * ihs + bh);
    sq_[qidx(r)] = (uint16_t)((uint16_t)(uint8_t)qg | ((uint16_t)(uint8_t)qh << 8));
    if (dg) {
      dg[brow0 + r] = (float)((double)qg * gs);
      dh[brow0 + r] = (float)((double)qh * hs);
    }
  }
  __syncthreads();
  for (int r = tid; r < nblk; r += 256) gh[brow0 + r] = sq_[qidx(r)];
}

// ===========================================================================
// ConstructHistogram (integer).  A block owns a contiguous run of the leaf's rows
// and a private LDS histogram of packed 64-bit cells
//   cell += q_g + (q_h << 22) + ([q_h == 3] << 43)
// (fields: 22-bit signed, 21-bit, 21-bit; exact for < 2^19 rows per block), then
// flushes the three fields with integer atomics into the global [cells][3] array.
// Integer addition is associative, so the result is independent of scheduling.
// ===========================================================================
template <int W>
__global__ __launch_bounds__(HIST_THREADS) void k_hist(DevLearner L, int32_t driver) {
  extern __shared__ unsigned long long lds_hist[];
  __shared__ int32_t cb[16 * LGBM_MAX_W];
  const Ctl* ctl = L.ctl;
  // driver 2: the root build of the tree driver, which the reference performs
  // unconditionally (LeafSplits::init, learner.rs:1323-1328); 0: per-op build.
  if (driver == 2 && ctl->done) return;
  const int32_t buf = ctl->h_buf;
  const int64_t begin = ctl->h_begin, count = ctl->h_count;
  if (count <= 0) return;
  int64_t nblk = (count + HIST_MIN_ROWS_PER_BLOCK - 1) / HIST_MIN_ROWS_PER_BLOCK;
  if (nblk > gridDim.x) nblk = gridDim.x;
  if ((int64_t)blockIdx.x >= nblk) return;
  const int64_t per = (count + nblk - 1) / nblk;
  const int64_t lo = (int64_t)blockIdx.x * per;
  const int64_t hi = min(count, lo + per);
  if (lo >= hi) return;
  const int F = L.F, cells = L.total_cells;
  for (int c = threadIdx.x; c < cells; c += HIST_THREADS) lds_hist[c] = 0ull;
  for (int f = threadIdx.x; f < F; f += HIST_THREADS) cb[f] = (int32_t)L.feats[f].cell_base;
  __syncthreads();
  const uint4* __restrict__ rec = L.bufs.rec[buf] + begin * W;
  const uint16_t* __restrict__ gh = L.bufs.gh[buf] + begin;
  for (int64_t r = lo + threadIdx.x; r < hi; r += HIST_THREADS) {
    uint4 w[W];
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = rec[r * W + i];
    const uint32_t q = gh[r];
    const int32_t qg = (int32_t)(int8_t)(q & 0xffu);
    const int32_t qh = (int32_t)(int8_t)(q >> 8);
    const unsigned long long v = (unsigned long long)(long long)qg +
                                 ((unsigned long long)(uint32_t)qh << 22) +
                                 ((unsigned long long)(qh == 3 ? 1u : 0u) << 43);
#pragma unroll
    for (int wi = 0; wi < W; ++wi) {
      const uint32_t ww[4] = {w[wi].x, w[wi].y, w[wi].z, w[wi].w};
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int f = wi * 16 + j;
        if (f < F) {
          const uint32_t bin = (ww[j >> 2] >> (8 * (j & 3))) & 0xffu;
          __hip_atomic_fetch_add(&lds_hist[cb[f] + bin], v, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
        }
      }
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < cells; c += HIST_THREADS) {
    const unsigned long long p = lds_hist[c];
    if (p == 0ull) continue;
    const int64_t lo22 = (int64_t)(p & ((1ull << 22) - 1));
    const int64_t gsum = lo22 >= (1ll << 21) ? lo22 - (1ll << 22) : lo22;
    const unsigned long long rest = (p - (unsigned long long)gsum) >> 22;
    const int32_t hsum = (int32_t)(rest & ((1ull << 21) - 1));
    const int32_t n3 = (int32_t)(rest >> 21);
    int32_t* dst = L.hist_int + (size_t)c * 3;
    if (gsum) __hip_atomic_fetch_add(dst, (int32_t)gsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (hsum) __hip_atomic_fetch_add(dst + 1, hsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (n3) __hip_atomic_fetch_add(dst + 2, n3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ===========================================================================
// k_fixscan: one block (two waves) per feature.
//   mode 1 (root):  node slot 0 from the histogram of all rows: root LeafSplits sums
//                   (exact, from the integer totals), FixHistogram, compaction, and
//                   the root's FindBestThreshold (wave 0).
//   mode 2 (build): per-op build into `explicit_out` (no scan).
// The integer accumulator cells are cleared after reading.
// ===========================================================================
__global__ __launch_bounds__(SCAN_THREADS) void k_fixscan(DevLearner L, int32_t mode,
                                                          double* __restrict__ explicit_out) {
  __shared__ double cs[2 * 256];
  __shared__ long long tot[3][SCAN_THREADS / LGBM_WAVE];
  Ctl* ctl = L.ctl;
  const int f = blockIdx.x;
  if (mode == 1 && ctl->done) return;
  const int tid = threadIdx.x;
  const DevFeature ft = L.feats[f];
  const int nb = (int)ft.num_bin;
  const double vg1 = (double)ctl->vg1, vh1 = (double)ctl->vh1, vh3 = (double)ctl->vh3;
  long long tg = 0, th = 0, t3 = 0;
  for (int b = tid; b < nb; b += SCAN_THREADS) {
    const size_t ci = (size_t)(ft.cell_base + b);
    int32_t* acc = L.hist_int + ci * 3;
    const int32_t G = acc[0], H = acc[1], T = acc[2];
    acc[0] = 0;
    acc[1] = 0;
    acc[2] = 0;
    if (mode == 1) {
      int32_t* ps = L.int_slots + ci * 3;  // node slot 0
      ps[0] = G;
      ps[1] = H;
      ps[2] = T;
    }
    int_cell_to_f64(G, H, T, vg1, vh1, vh3, &cs[2 * b], &cs[2 * b + 1]);
    tg += G;
    th += H;
    t3 += T;
  }
  double sg, sh, weight = 0.0;
  int32_t nrows;
  if (mode == 1) {
    // Every row adds to exactly one bin of every feature, so each block holds the
    // root totals.  LeafSplits::init (leaf_splits.rs:75-89): the ordered f64 fold of
    // the dequantized values equals these exact integer-weighted sums.
    for (int off = 32; off >= 1; off >>= 1) {
      tg += __shfl_xor(tg, off);
      th += __shfl_xor(th, off);
      t3 += __shfl_xor(t3, off);
    }
    if (lane_id() == 0) {
      tot[0][tid >> 6] = tg;
      tot[1][tid >> 6] = th;
      tot[2][tid >> 6] = t3;
    }
    __syncthreads();
    long long G = 0, H = 0, T = 0;
    for (int w = 0; w < SCAN_THREADS / LGBM_WAVE; ++w) {
      G += tot[0][w];
      H += tot[1][w];
      T += tot[2][w];
    }
    sg = (double)G * vg1;
    sh = (double)(H - 3ll * T) * vh1 + (double)T * vh3;
    nrows = (int32_t)L.N;
    const lgbm_gain_config& cfg = ctl->cfg;
    weight = leaf_output_full(cfg.lambda_l1 > 0.0, sg, sh, cfg.lambda_l1, cfg.lambda_l2,
                              cfg.max_delta_step, false, cfg.path_smooth, 0, 0.0);
    if (f == 0 && tid == 0) {
      L.nodes.sums[0] = LeafSums{sg, sh, weight, nrows, 0};
      if (!(sh > 0.0)) {
        ctl->error |= ERR_ROOT_HESSIAN;
        ctl->done = 1;
      }
    }
  } else {
    sg = ctl->sm.sg;
    sh = ctl->sm.sh;
    nrows = ctl->sm.n;
  }
  __syncthreads();
  fix_compact_block(ft, cs, sg, sh, !(sh > 0.0 && nrows > 0));
  if (mode == 2) {
    for (int i = tid; i < 2 * nb; i += SCAN_THREADS) explicit_out[ft.slot_off + i] = cs[i];
    return;
  }
  for (int i = tid; i < 2 * nb; i += SCAN_THREADS) L.slots[ft.slot_off + i] = cs[i];
  if (tid >= LGBM_WAVE) return;
  lgbm_split_info* out = L.feat_split + f;
  if (ctl->root_skip || !(sh > 0.0 && nrows > 0)) {
    if (lane_id() == 0) {
      split_set_none(out);
      L.splittable[f] = 0;
    }
    return;
  }
  const ScanCfg sc = make_scan_cfg(ctl->cfg);
  wave_scan(cs, ft, sc, sg, sh, nrows, weight, out);
  if (lane_id() == 0) L.splittable[f] = out->gain > -__builtin_inf() ? 1 : 0;
}

// Per-op FindBestThreshold over explicit features (find_best_splits_batched,
// lib.rs:1500-1548): one wave per feature, host-provided histogram.
__global__ __launch_bounds__(LGBM_WAVE) void k_scan_explicit(const double* __restrict__ hist,
                                                             const DevFeature* __restrict__ feats,
                                                             int32_t n_feats,
                                                             lgbm_gain_config cfg, double sg,
                                                             double sh, int32_t n,
                                                             lgbm_split_info* out) {
  __shared__ double cs[2 * 256];
  const int f = blockIdx.x;
  if (f >= n_feats) return;
  const DevFeature ft = feats[f];
  for (int i = threadIdx.x; i < 2 * (int)ft.num_bin; i += LGBM_WAVE) cs[i] = hist[ft.slot_off + i];
  __syncthreads();
  const ScanCfg sc = make_scan_cfg(cfg);
  wave_scan(cs, ft, sc, sg, sh, n, cfg.parent_output, out + f);
}

// ===========================================================================
// score update: traverse the tree per row with the split routers
// (equivalent to AddPredictionToScore over the partition, learner.rs:4380-4395),
// adding the shrunk leaf value (Tree::shrinkage, tree.rs:1074).
// ===========================================================================
template <int W>
__global__ __launch_bounds__(256) void k_score_update(DevLearner L, double lr,
                                                      double* __restrict__ score) {
  __shared__ NodeRoute nodes[256];
  __shared__ double vals[256];
  const int32_t nl = L.ctl->num_leaves;
  if (nl <= 1) return;
  for (int i = threadIdx.x; i < nl - 1; i += blockDim.x) nodes[i] = L.tree.nodes[i];
  for (int i = threadIdx.x; i < nl; i += blockDim.x)
    vals[i] = maybe_round_to_zero(L.tree.leaf_value[i] * lr);
  __syncthreads();
  const uint4* __restrict__ rec = L.bufs.rec[BUF_ORIG];
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < L.N; r += stride) {
    uint4 w[W];
#pragma unroll
    for (int i = 0; i < W; ++i) w[i] = rec[r * W + i];
    int32_t node = 0;
    for (int depth = 0; depth < nl && node >= 0; ++depth) {  // a path has < nl nodes
      const NodeRoute& n = nodes[node];
      const int32_t bin = (int32_t)rec_byte(w, n.f);
      node = route_right(bin, n.pmin, n.max_bin, n.th, n.na_bin, n.flags) ? n.right : n.left;
    }
    if (node < 0 && ~node < nl) score[r] += vals[~node];
  }
}

template <int W>
__global__ void k_gather_rows(const uint32_t* __restrict__ rows, int64_t n, const uint4* __restrict__ rec,
                              const uint16_t* __restrict__ gh, uint4* __restrict__ rec_out,
                              uint16_t* __restrict__ gh_out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t r = rows[i];
#pragma unroll
  for (int k = 0; k < W; ++k) rec_out[i * W + k] = rec[r * W + k];
  gh_out[i] = gh[r];
}

__global__ void k_subtract(const double* __restrict__ a, const double* __restrict__ b, int64_t n,
                           double* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = a[i] - b[i];
}

// per-op partition input: one-word records with the bin in byte 0
__global__ void k_pack_partition(const uint32_t* __restrict__ bins, int64_t n,
                                 uint4* __restrict__ rec) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) rec[i] = make_uint4(bins[i] & 0xffu, 0u, 0u, (uint32_t)i);
}

// ===========================================================================
// launchers
// ===========================================================================
void launch_pack_records(const uint8_t* bins, int64_t n, int32_t F, int32_t W, uint4* rec,
                         hipStream_t s) {
  const int64_t blocks = (n + 255) / 256;
  k_pack_records<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(bins, n, F, W, rec);
}
int32_t stat_blocks(int64_t n) {
  return (int32_t)std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, STAT_BLOCKS));
}
void launch_absmax(const float* g, const float* h, int64_t n, uint4* partials, hipStream_t s) {
  k_absmax<<<dim3((unsigned)stat_blocks(n)), dim3(256), 0, s>>>(g, h, n, partials);
}
void launch_grad_binary(const double* score, const float* label, float* g, float* h, int64_t n,
                        uint4* partials, hipStream_t s) {
  k_grad_binary<<<dim3((unsigned)stat_blocks(n)), dim3(256), 0, s>>>(score, label, g, h, n,
                                                                     partials);
}
void launch_quant_scales(Ctl* ctl, const uint4* partials, int64_t n, int32_t bins,
                         int32_t force_const, hipStream_t s) {
  k_quant_scales<<<1, 256, 0, s>>>(ctl, partials, stat_blocks(n), bins, force_const);
}
void launch_quantize(const float* g, const float* h, int64_t n, const Ctl* ctl,
                     const uint64_t* wave_mats, const uint64_t* lane_mats, uint64_t s0,
                     int32_t stochastic, uint16_t* gh, float* dg, float* dh, hipStream_t s) {
  const int64_t blocks = (n + QUANT_BLOCK_ROWS - 1) / QUANT_BLOCK_ROWS;
  k_quantize<<<dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256), 0, s>>>(
      g, h, n, ctl, wave_mats, lane_mats, s0, stochastic, gh, dg, dh);
}
void launch_hist(const DevLearner& L, int32_t driver, int64_t count_hint, hipStream_t s,
                 const KernelEvents* ev) {
  int64_t blocks = HIST_MAX_BLOCKS;
  if (count_hint > 0)
    blocks = std::min<int64_t>(HIST_MAX_BLOCKS,
                               (count_hint + HIST_MIN_ROWS_PER_BLOCK - 1) / HIST_MIN_ROWS_PER_BLOCK);
  if (blocks < 1) blocks = 1;
  const size_t lds = (size_t)L.total_cells * sizeof(unsigned long long);
  DISPATCH_W(L.W, KLAUNCH(ev, k_hist<kW>, dim3((unsigned)blocks), dim3(HIST_THREADS), lds, s, L,
                          driver));
}
void launch_fixscan(const DevLearner& L, int32_t mode, double* explicit_out, hipStream_t s,
                    const KernelEvents* ev) {
  KLAUNCH(ev, k_fixscan, dim3((unsigned)L.F), dim3(SCAN_THREADS), 0, s, L, mode, explicit_out);
}
void launch_scan_explicit(const double* hist, const DevFeature* feats, int32_t n_feats,
                          const lgbm_gain_config& cfg, double sg, double sh, int32_t n,
                          lgbm_split_info* out, hipStream_t s) {
  k_scan_explicit<<<dim3((unsigned)n_feats), dim3(LGBM_WAVE), 0, s>>>(hist, feats, n_feats, cfg, sg,
                                                                       sh, n, out);
}
void launch_score_update(const DevLearner& L, double lr, double* score, hipStream_t s,
                         const KernelEvents* ev) {
  int64_t blocks = std::min<int64_t>((L.N + 255) / 256, 4096);
  if (blocks < 1) blocks = 1;
  DISPATCH_W(L.W, KLAUNCH(ev, k_score_update<kW>, dim3((unsigned)blocks), dim3(256), 0, s, L, lr,
                          score));
}
void launch_gather_rows(int W, const uint32_t* rows, int64_t n, const uint4* rec, const uint16_t* gh,
                        uint4* rec_out, uint16_t* gh_out, hipStream_t s) {
  const int64_t blocks = (n + 255) / 256;
  if (blocks < 1) return;
  DISPATCH_W(W, (k_gather_rows<kW><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(rows, n, rec, gh,
                                                                                 rec_out, gh_out)));
}
void launch_subtract(const double* a, const double* b, int64_t n, double* out, hipStream_t s) {
  const int64_t blocks = (n + 255) / 256;
  if (blocks < 1) return;
  k_subtract<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(a, b, n, out);
}
void launch_pack_partition(const uint32_t* bins, int64_t n, uint4* rec, hipStream_t s) {
  const int64_t blocks = (n + 255) / 256;
  if (blocks < 1) return;
  k_pack_partition<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(bins, n, rec);
}

}  // namespace lgbm
