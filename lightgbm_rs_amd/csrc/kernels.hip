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
#include "kernels.h"

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
// Byte f of a record held in registers.  Selects with compile-time indices only, so
// the record never leaves the register file.
template <int W>
__device__ __forceinline__ uint32_t rec_byte(const uint4 (&w)[W], int f) {
  const int wi = f >> 4;
  const int j = (f >> 2) & 3;
  uint32_t word = 0u;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const uint4 q = w[i];
    const uint32_t x = j == 0 ? q.x : (j == 1 ? q.y : (j == 2 ? q.z : q.w));
    word = i == wi ? x : word;
  }
  return (word >> (8 * (f & 3))) & 0xffu;
}

template <int W>
__global__ __launch_bounds__(HIST_THREADS) void k_hist(DevLearner L, int32_t driver) {
  extern __shared__ unsigned long long lds_hist[];
  __shared__ int32_t cb[16 * LGBM_MAX_W];
  const Ctl* ctl = L.ctl;
  // driver 1: per-split build (gated by done/skip); driver 2: the root build, which
  // the reference performs unconditionally (LeafSplits::init, learner.rs:1323-1328).
  if (driver == 1 && (ctl->done || ctl->skip)) return;
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
// FindBestThreshold for one (leaf, feature) by one wave: find_best_split_cpu_native
// (kernels/split.rs:8970-9329).  The reference accumulates the candidate sums in a
// fixed sequential f64 order starting at kEpsilon; here lane k of a 64-candidate
// chunk recomputes the prefix over candidates 0..k in that same order (uniform LDS
// broadcast reads), so every lane holds bit-identical sums.  The sticky `done`
// break becomes "first candidate with active && !cont && brk" (ballot), and the
// sequential strict-> best becomes a max-gain, lowest-index wave reduction.
// ===========================================================================
__device__ void wave_scan(const double* hist, const DevFeature& ft, const ScanCfg& c,
                          double sum_gradient, double sum_hessian, int32_t num_data, double po,
                          lgbm_split_info* out) {
  const int lane = (int)lane_id();
  const double eps = k_eps();
  const double ninf = -__builtin_inf();
  const double shb = sum_hessian + 2.0 * eps;
  const double gain_shift =
      c.use_full ? leaf_gain_full(c.use_l1, sum_gradient, shb, c.l1, c.l2, c.mds, c.use_smoothing,
                                  c.ps, num_data, po)
                 : leaf_gain(c.use_l1, sum_gradient, shb, c.l1, c.l2);
  const double mgs = gain_shift + c.min_gain;
  const int32_t nb = (int32_t)ft.num_bin;
  const int32_t offset = ft.offset;
  const bool skip_def = ft.skip_default_bin != 0;
  const bool na_m = ft.na_as_missing != 0;
  const int32_t na = na_m ? 1 : 0;
  const int32_t defb = (int32_t)ft.default_bin;
  const int32_t rev_count = max(nb - 1 - na, 0);
  const bool na_pre = na_m && offset == 1;
  int32_t fwd_count = 0;
  if (ft.run_forward) {
    const int32_t base = max(nb - 1 - offset, 0);
    fwd_count = na_pre ? base + 1 : base;
  }
  const double cf = (double)num_data / shb;

  bool any_split = false;
  double best_gain = ninf, best_lg = 0.0, best_lh = 0.0;
  int32_t best_lc = 0, best_thr = 0;
  bool best_dl = true;

  {  // REVERSE (split.rs:9078-9176)
    double cg = 0.0, ch = eps;
    int32_t cc = 0;
    const int32_t t_start = nb - 1 - offset - na;
    for (int32_t base = 0; base < rev_count; base += LGBM_WAVE) {
      const int32_t cnt = min(LGBM_WAVE, rev_count - base);
      const bool valid = lane < cnt;
      const int32_t t = t_start - (base + lane);
      const bool act = valid && (t >= 1 - offset) && !(skip_def && t + offset == defb);
      const double mg = act ? hist[2 * t] : 0.0, mh = act ? hist[2 * t + 1] : 0.0;
      const int32_t mc = act ? round_int(mh * cf) : 0;
      double sg = cg, sh = ch;
      int32_t rc = cc;
      for (int32_t i = 0; i < cnt; ++i) {
        const int32_t ti = t_start - (base + i);
        if ((ti >= 1 - offset) && !(skip_def && ti + offset == defb)) {  // wave-uniform
          const double xg = readlane_f64(mg, i), xh = readlane_f64(mh, i);
          const int32_t xc = readlane_i32(mc, i);
          if (i <= lane) {
            sg += xg;
            sh += xh;
            rc += xc;
          }
        }
      }
      const int32_t lc = num_data - rc;
      const double slh = shb - sh, slg = sum_gradient - sg;
      const bool cont = rc < c.min_d || sh < c.min_h;
      const bool brk = lc < c.min_d || slh < c.min_h;
      const unsigned long long bm = __ballot(act && !cont && brk);
      const int first_brk = bm ? (__ffsll((unsigned long long)bm) - 1) : LGBM_WAVE;
      const bool consider = act && !cont && lane < first_brk;
      double gain = ninf;
      if (consider) gain = split_gain_of(c, slg, slh, sg, sh, lc, rc, po);
      const bool cand = consider && gain > mgs;
      if (__ballot(cand)) any_split = true;
      double rg = cand ? gain : ninf;
      int32_t rl = cand ? lane : LGBM_WAVE;
      for (int off = 32; off >= 1; off >>= 1) {
        const double og = __shfl_xor(rg, off);
        const int32_t ol = __shfl_xor(rl, off);
        if (og > rg || (og == rg && ol < rl)) {
          rg = og;
          rl = ol;
        }
      }
      if (rl < LGBM_WAVE && rg > best_gain) {
        best_gain = rg;
        best_lc = __shfl(lc, rl);
        best_lg = __shfl(slg, rl);
        best_lh = __shfl(slh, rl);
        best_thr = __shfl(t, rl) - 1 + offset;
        best_dl = true;
      }
      if (bm) break;
      cg = __shfl(sg, cnt - 1);
      ch = __shfl(sh, cnt - 1);
      cc = __shfl(rc, cnt - 1);
    }
  }
  {  // FORWARD (split.rs:9178-9277)
    double cg = 0.0, ch = eps;
    int32_t cc = 0, fwd_start = 0;
    if (na_pre) {
      cg = sum_gradient;
      ch = shb - eps;
      cc = num_data;
      const int32_t m = nb - offset;
      for (int32_t c0 = 0; c0 < m; c0 += LGBM_WAVE) {
        const int32_t bb = c0 + lane;
        const double vg = bb < m ? hist[2 * bb] : 0.0, vh = bb < m ? hist[2 * bb + 1] : 0.0;
        const int32_t vc = bb < m ? round_int(vh * cf) : 0;
        const int32_t lim = min(LGBM_WAVE, m - c0);
        for (int32_t i = 0; i < lim; ++i) {
          cg -= readlane_f64(vg, i);
          ch -= readlane_f64(vh, i);
          cc -= readlane_i32(vc, i);
        }
      }
      fwd_start = -1;
    }
    for (int32_t base = 0; base < fwd_count; base += LGBM_WAVE) {
      const int32_t cnt = min(LGBM_WAVE, fwd_count - base);
      const bool valid = lane < cnt;
      const int32_t t = fwd_start + base + lane;
      const bool act = valid && !(skip_def && t + offset == defb);
      const bool addl = act && t >= 0;
      const double mg = addl ? hist[2 * t] : 0.0, mh = addl ? hist[2 * t + 1] : 0.0;
      const int32_t mc = addl ? round_int(mh * cf) : 0;
      double sg = cg, sh = ch;
      int32_t lcn = cc;
      for (int32_t i = 0; i < cnt; ++i) {
        const int32_t ti = fwd_start + base + i;
        if (!(skip_def && ti + offset == defb) && ti >= 0) {  // wave-uniform
          const double xg = readlane_f64(mg, i), xh = readlane_f64(mh, i);
          const int32_t xc = readlane_i32(mc, i);
          if (i <= lane) {
            sg += xg;
            sh += xh;
            lcn += xc;
          }
        }
      }
      const int32_t rc = num_data - lcn;
      const double srh = shb - sh, srg = sum_gradient - sg;
      const bool cont = lcn < c.min_d || sh < c.min_h;
      const bool brk = rc < c.min_d || srh < c.min_h;
      const unsigned long long bm = __ballot(act && !cont && brk);
      const int first_brk = bm ? (__ffsll((unsigned long long)bm) - 1) : LGBM_WAVE;
      const bool consider = act && !cont && lane < first_brk;
      double gain = ninf;
      if (consider) gain = split_gain_of(c, sg, sh, srg, srh, lcn, rc, po);
      const bool cand = consider && gain > mgs;
      if (__ballot(cand)) any_split = true;
      double rg = cand ? gain : ninf;
      int32_t rl = cand ? lane : LGBM_WAVE;
      for (int off = 32; off >= 1; off >>= 1) {
        const double og = __shfl_xor(rg, off);
        const int32_t ol = __shfl_xor(rl, off);
        if (og > rg || (og == rg && ol < rl)) {
          rg = og;
          rl = ol;
        }
      }
      if (rl < LGBM_WAVE && rg > best_gain) {
        best_gain = rg;
        best_lc = __shfl(lcn, rl);
        best_lg = __shfl(sg, rl);
        best_lh = __shfl(sh, rl);
        best_thr = __shfl(t, rl) + offset;
        best_dl = false;
      }
      if (bm) break;
      cg = __shfl(sg, cnt - 1);
      ch = __shfl(sh, cnt - 1);
      cc = __shfl(lcn, cnt - 1);
    }
  }
  if (lane == 0) {
    if (any_split && best_gain > ninf) {
      const int32_t best_rc = num_data - best_lc;
      const double lo = leaf_output_full(c.use_l1, best_lg, best_lh, c.l1, c.l2, c.mds,
                                         c.use_smoothing, c.ps, best_lc, po);
      const double rsg = sum_gradient - best_lg;
      const double rsh = shb - best_lh;
      const double ro = leaf_output_full(c.use_l1, rsg, rsh, c.l1, c.l2, c.mds, c.use_smoothing,
                                         c.ps, best_rc, po);
      out->threshold = (uint32_t)best_thr;
      out->gain = best_gain - mgs;
      out->left_count = best_lc;
      out->right_count = num_data - best_lc;
      out->left_sum_gradient = best_lg;
      out->left_sum_hessian = best_lh - eps;
      out->right_sum_gradient = rsg;
      out->right_sum_hessian = rsh - eps;
      out->left_output = lo;
      out->right_output = ro;
      out->default_left = best_dl ? 1 : 0;
    } else {
      split_set_none(out);
    }
  }
}

// ===========================================================================
// Split step: per-leaf feature argmax for the leaves scanned last (the argmax of
// scan_leaf_histogram, learner.rs:3290-3330), the cross-leaf ArgMax
// (learner.rs:4537), the stop test (learner.rs:1503) and the Tree::split bookkeeping
// of the chosen split (tree.rs:614-700), plus the router and partition job of the
// split (split_inner, learner.rs:3895-4011).  Run by one whole block.
// ===========================================================================
struct BestKey {
  double gain;
  int32_t feat;  // real feature index (-1 none)
  int32_t idx;   // feature position / leaf id
};

__device__ __forceinline__ bool key_better(const BestKey& a, const BestKey& b) {
  if (split_gt(a.gain, a.feat, b.gain, b.feat)) return true;
  if (split_gt(b.gain, b.feat, a.gain, a.feat)) return false;
  return a.idx < b.idx;
}

__device__ BestKey block_best(BestKey k, BestKey* sh) {
  for (int off = 32; off >= 1; off >>= 1) {
    BestKey o;
    o.gain = __shfl_xor(k.gain, off);
    o.feat = __shfl_xor(k.feat, off);
    o.idx = __shfl_xor(k.idx, off);
    if (key_better(o, k)) k = o;
  }
  const int w = threadIdx.x >> 6;
  if (lane_id() == 0) sh[w] = k;
  __syncthreads();
  BestKey r = sh[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i)
    if (key_better(sh[i], r)) r = sh[i];
  __syncthreads();
  return r;
}

__device__ void split_step(DevLearner& L) {
  __shared__ BestKey sh[16];
  Ctl* ctl = L.ctl;
  const int F = L.F;
  const int tid = threadIdx.x;
  const double ninf = -__builtin_inf();
  if (ctl->pending_reduce) {
    const int32_t leaves[2] = {ctl->smaller, ctl->larger};
    for (int li = 0; li < 2; ++li) {
      const int32_t leaf = leaves[li];
      if (leaf < 0) continue;
      BestKey k{ninf, -1, 0x7fffffff};
      for (int f = tid; f < F; f += blockDim.x) {
        const double g = L.feat_split[(size_t)leaf * F + f].gain;
        BestKey c{g, L.feats[f].real_index, f};
        if (g > ninf && key_better(c, k)) k = c;
      }
      const BestKey r = block_best(k, sh);
      if (tid == 0) {
        if (r.idx != 0x7fffffff && r.gain > ninf) {
          L.best[leaf] = L.feat_split[(size_t)leaf * F + r.idx];
          L.best_feat[leaf] = r.feat;
          L.best_fpos[leaf] = r.idx;
        } else {
          split_set_none(&L.best[leaf]);
          L.best_feat[leaf] = -1;
          L.best_fpos[leaf] = -1;
        }
      }
      __syncthreads();
    }
    if (tid == 0) ctl->pending_reduce = 0;
    __threadfence_block();
  }
  const int32_t nl = ctl->num_leaves;
  BestKey k{ninf, -1, 0x7fffffff};
  for (int l = tid; l < nl; l += blockDim.x) {
    BestKey c{L.best[l].gain, L.best_feat[l], l};
    if (key_better(c, k)) k = c;
  }
  const BestKey r = block_best(k, sh);
  if (tid != 0) return;
  const int32_t bl = r.idx == 0x7fffffff ? 0 : r.idx;
  // independent loads first
  const lgbm_split_info b = L.best[bl];
  const int32_t fr = L.best_feat[bl];
  const int32_t f = L.best_fpos[bl];
  DevTree& T = L.tree;
  const int32_t parent = T.leaf_parent[bl];
  const double lv_old = T.leaf_value[bl];
  const int32_t depth = T.leaf_depth[bl];
  const int32_t src_buf = L.leaves.buf[bl];
  const int32_t lbegin = L.leaves.begin[bl];
  const int32_t lcount = L.leaves.count[bl];
  const int32_t lrev = L.leaves.rev[bl];
  if (!(b.gain > 0.0)) {  // learner.rs:1503: stop when gain <= 0
    ctl->done = 1;
    return;
  }
  if (f < 0 || f >= F) {
    ctl->error |= ERR_FEATURE;
    ctl->done = 1;
    return;
  }
  const DevFeature ft = L.feats[f];
  const int32_t node = nl - 1, nr = nl;
  const double thr_real = L.ub ? L.ub[ft.ub_off + b.threshold] : (double)b.threshold;
  // Tree::split (tree.rs:614-700); counts are written by k_partition.
  if (parent >= 0) {
    if (T.right_child[parent] == ~bl) {
      T.right_child[parent] = node;
      T.nodes[parent].right = node;
    } else {
      T.left_child[parent] = node;
      T.nodes[parent].left = node;
    }
  }
  T.split_feature[node] = fr;
  T.split_gain[node] = (float)(b.gain + ctl->cfg.min_gain_to_split);
  T.threshold_in_bin[node] = b.threshold;
  T.threshold[node] = thr_real;
  T.internal_value[node] = lv_old;
  T.left_child[node] = ~bl;
  T.right_child[node] = ~nr;
  int8_t dt = 0;
  if (b.default_left) dt |= 2;
  dt |= (int8_t)((ft.missing_type & 3) << 2);
  T.decision_type[node] = dt;
  T.leaf_value[bl] = b.left_output;
  T.leaf_weight[bl] = b.left_sum_hessian;
  T.leaf_value[nr] = b.right_output;
  T.leaf_weight[nr] = b.right_sum_hessian;
  T.leaf_depth[nr] = depth + 1;
  T.leaf_depth[bl] = depth + 1;
  T.leaf_parent[bl] = node;
  T.leaf_parent[nr] = node;
  // router (split_inner, learner.rs:3957; data_partition.rs:387-417)
  const int32_t pmin = (int32_t)ft.min_bin + max(ft.offset, 0);
  int32_t thr = (int32_t)b.threshold + pmin;
  if (ft.mfb == 0) thr -= 1;
  int32_t flags = 0;
  if ((int32_t)ft.mfb > (int32_t)b.threshold) flags |= 1;
  if (ft.na_as_missing) flags |= 2;
  if (b.default_left) flags |= 4;
  NodeRoute nrt;
  nrt.f = f;
  nrt.pmin = pmin;
  nrt.max_bin = (int32_t)ft.max_bin;
  nrt.th = thr;
  nrt.na_bin = (int32_t)ft.num_bin - 1;
  nrt.flags = flags;
  nrt.left = ~bl;
  nrt.right = ~nr;
  T.nodes[node] = nrt;
  PartJob J;
  J.src_buf = src_buf;
  J.dst_buf = src_buf == BUF_A ? BUF_B : BUF_A;
  J.begin = lbegin;
  J.count = lcount;
  J.rev = lrev;
  J.fbyte = f;
  J.pmin = pmin;
  J.max_bin = (int32_t)ft.max_bin;
  J.th = thr;
  J.na_bin = (int32_t)ft.num_bin - 1;
  J.flags = flags;
  J.driver = 1;
  ctl->part = J;
  ctl->split = b;
  ctl->split_leaf = bl;
  ctl->split_f = f;
  ctl->new_right = nr;
  ctl->node = node;
  split_set_none(&L.best[bl]);
  L.best_feat[bl] = -1;
  L.best_fpos[bl] = -1;
  split_set_none(&L.best[nr]);
  L.best_feat[nr] = -1;
  L.best_fpos[nr] = -1;
  ctl->num_leaves = nl + 1;
  ctl->left_leaf = bl;
  ctl->right_leaf = nr;
}

// ===========================================================================
// k_fixscan: one block (two waves) per feature, then the split step in the block
// that finishes last.
//   mode 0 (pair):  smaller child cells from the integer histogram -> FixHistogram on
//                   the smaller's RAW sums -> compaction -> slot[smaller];
//                   slot[larger] = slot[parent] - slot[smaller]; scan both leaves.
//   mode 1 (root):  leaf 0 from all rows; root LeafSplits sums from the histogram.
//   mode 2 (build): per-op build into `explicit_out` (no scan, no split step).
// The integer cells are cleared after reading so the next build starts from zero.
// With ctl->skip set (a gated pair), only the split step runs.
// ===========================================================================
__global__ __launch_bounds__(SCAN_THREADS) void k_fixscan(DevLearner L, int32_t mode,
                                                          double* __restrict__ explicit_out) {
  __shared__ double cs[2 * 256];
  __shared__ double cp[2 * 256];
  __shared__ long long tot[3][SCAN_THREADS / LGBM_WAVE];
  __shared__ int32_t s_last;
  Ctl* ctl = L.ctl;
  const int f = blockIdx.x;
  if (mode == 0 && ctl->done) return;
  const bool skip = mode == 2 ? false : (ctl->skip != 0);
  const int tid = threadIdx.x;
  const int F = L.F;

  const DevFeature ft = L.feats[f];
  const int nb = (int)ft.num_bin;
  const int cells = L.total_cells;
  long long tg = 0, th = 0, t3 = 0;
  {
    // Integer cells.  mode 0: the accumulator holds the LEFT child's histogram (built in
    // the partition pass); right = parent - left; the per-leaf integer slots keep both
    // for later splits.  mode 1: the root.  mode 2: a per-op build.
    const double vg1 = (double)ctl->vg1, vh1 = (double)ctl->vh1, vh3 = (double)ctl->vh3;
    const int32_t bl = ctl->left_leaf, nr = ctl->right_leaf, sml = ctl->smaller;
    for (int b = tid; b < nb; b += SCAN_THREADS) {
      const size_t ci = (size_t)(ft.cell_base + b);
      int32_t* acc = L.hist_int + ci * 3;
      int32_t G = acc[0], H = acc[1], T = acc[2];
      acc[0] = 0;
      acc[1] = 0;
      acc[2] = 0;
      if (mode == 0) {
        int32_t* ps = L.int_slots + ((size_t)bl * cells + ci) * 3;
        int32_t* rs = L.int_slots + ((size_t)nr * cells + ci) * 3;
        const int32_t RG = ps[0] - G, RH = ps[1] - H, RT = ps[2] - T;
        ps[0] = G;
        ps[1] = H;
        ps[2] = T;
        rs[0] = RG;
        rs[1] = RH;
        rs[2] = RT;
        if (sml == nr) {
          G = RG;
          H = RH;
          T = RT;
        }
      } else if (mode == 1) {
        int32_t* ps = L.int_slots + ci * 3;
        ps[0] = G;
        ps[1] = H;
        ps[2] = T;
      }
      cs[2 * b] = (double)G * vg1;
      cs[2 * b + 1] = (double)((long long)H - 3ll * T) * vh1 + (double)T * vh3;
      tg += G;
      th += H;
      t3 += T;
    }
  }

  if (!(mode == 0 && skip)) {
    const double vg1 = (double)ctl->vg1, vh1 = (double)ctl->vh1, vh3 = (double)ctl->vh3;
    double sg, sh, weight;
    int32_t nrows;
    if (mode == 1) {
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
      // LeafSplits::init (leaf_splits.rs:75-89): the ordered f64 fold of the
      // dequantized values equals these exact integer-weighted sums.
      sg = (double)G * vg1;
      sh = (double)(H - 3ll * T) * vh1 + (double)T * vh3;
      nrows = (int32_t)L.N;
      const lgbm_gain_config& cfg = ctl->cfg;
      weight = leaf_output_full(cfg.lambda_l1 > 0.0, sg, sh, cfg.lambda_l1, cfg.lambda_l2,
                                cfg.max_delta_step, false, cfg.path_smooth, 0, 0.0);
      if (f == 0 && tid == 0) {
        ctl->sm.sg = sg;
        ctl->sm.sh = sh;
        ctl->sm.weight = weight;
        ctl->sm.n = nrows;
        L.tree.leaf_value[0] = weight;
        if (!(sh > 0.0)) {
          ctl->error |= ERR_ROOT_HESSIAN;
          ctl->done = 1;
        }
      }
    } else {
      sg = ctl->sm.sg;
      sh = ctl->sm.sh;
      weight = ctl->sm.weight;
      nrows = ctl->sm.n;
    }
    __syncthreads();

    const int32_t left_leaf = ctl->left_leaf;
    const int32_t smaller = mode == 1 ? 0 : ctl->smaller;
    const int32_t larger = mode == 0 ? ctl->larger : -1;
    const bool pgate = mode == 0 && L.splittable[(size_t)left_leaf * F + f] == 0;
    const bool buildable = sh > 0.0 && nrows > 0;

    if (!buildable || pgate) {
      for (int i = tid; i < 2 * nb; i += SCAN_THREADS) cs[i] = 0.0;
    } else {
      // FixHistogram (fix_histogram.rs:50-80): sequential f64 subtraction in ascending
      // bin order, each wave-0 lane holding one bin and broadcasting it in turn.
      const int mfb = (int)ft.mfb;
      __syncthreads();
      if (tid < LGBM_WAVE && mfb > 0 && mfb < nb) {
        double g = sg, h = sh;
        for (int c0 = 0; c0 < nb; c0 += LGBM_WAVE) {
          const int bb = c0 + tid;
          const double vg = bb < nb ? cs[2 * bb] : 0.0;
          const double vh = bb < nb ? cs[2 * bb + 1] : 0.0;
          const int lim = min(LGBM_WAVE, nb - c0);
          for (int i = 0; i < lim; ++i) {
            if (c0 + i != mfb) {
              g -= readlane_f64(vg, i);
              h -= readlane_f64(vh, i);
            }
          }
        }
        if (tid == 0) {
          cs[2 * mfb] = g;
          cs[2 * mfb + 1] = h;
        }
      }
      __syncthreads();
      // compact_histogram (learner.rs:4460-4492)
      if (ft.offset > 0) {
        const int off = ft.offset;
        double a[4], b2[4];
        int k = 0;
        for (int c = tid; c < nb; c += SCAN_THREADS, ++k) {
          const int src = c + off;
          a[k] = src < nb ? cs[2 * src] : 0.0;
          b2[k] = src < nb ? cs[2 * src + 1] : 0.0;
        }
        __syncthreads();
        k = 0;
        for (int c = tid; c < nb; c += SCAN_THREADS, ++k) {
          cs[2 * c] = a[k];
          cs[2 * c + 1] = b2[k];
        }
      }
    }
    __syncthreads();

    if (mode == 2) {
      for (int i = tid; i < 2 * nb; i += SCAN_THREADS) explicit_out[ft.slot_off + i] = cs[i];
      return;
    }
    const size_t sl = L.slot_len;
    double* s_small = L.slots + (size_t)smaller * sl + ft.slot_off;
    if (larger >= 0) {
      // parent region lives in the slot of left_leaf (the split leaf keeps its id)
      const double* s_par = L.slots + (size_t)left_leaf * sl + ft.slot_off;
      for (int i = tid; i < 2 * nb; i += SCAN_THREADS) cp[i] = s_par[i];
      __syncthreads();
      double* s_large = L.slots + (size_t)larger * sl + ft.slot_off;
      for (int i = tid; i < 2 * nb; i += SCAN_THREADS) {
        const double d = cp[i] - cs[i];
        cp[i] = d;
        s_small[i] = cs[i];
        s_large[i] = d;
      }
    } else {
      for (int i = tid; i < 2 * nb; i += SCAN_THREADS) s_small[i] = cs[i];
    }
    __syncthreads();

    // ---- scans: wave 0 -> smaller (or root), wave 1 -> larger ----
    if (!skip) {
      const int wave = tid >> 6;
      const bool have = wave == 0 || larger >= 0;
      if (have) {
        const int32_t leaf = wave == 0 ? smaller : larger;
        const double* hist = wave == 0 ? cs : cp;
        const double lsg = wave == 0 ? sg : ctl->lg.sg;
        const double lsh = wave == 0 ? sh : ctl->lg.sh;
        const double lpo = wave == 0 ? weight : ctl->lg.weight;
        const int32_t ln = wave == 0 ? nrows : ctl->lg.n;
        lgbm_split_info* out = L.feat_split + (size_t)leaf * F + f;
        const bool scannable = lsh > 0.0 && ln > 0;
        if (!scannable) {
          if (lane_id() == 0) split_set_none(out);
        } else if (pgate) {
          if (lane_id() == 0) {
            split_set_none(out);
            L.splittable[(size_t)leaf * F + f] = 0;
          }
        } else {
          const lgbm_gain_config cfg = ctl->cfg;
          const ScanCfg sc = make_scan_cfg(cfg);
          wave_scan(hist, ft, sc, lsg, lsh, ln, lpo, out);
          if (lane_id() == 0)
            L.splittable[(size_t)leaf * F + f] = out->gain > -__builtin_inf() ? 1 : 0;
        }
      }
    }
  }
  // ---- the last block to finish runs the split step ----
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int32_t prev =
        __hip_atomic_fetch_add(&ctl->fs_count, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (int32_t)gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (tid == 0) __hip_atomic_store(&ctl->fs_count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (ctl->done) return;
  split_step(L);
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
// k_partition: stable single-pass split of one leaf's rows.  Tiles of PART_TILE
// logical positions are taken in ticket order; each tile ranks its rows with
// wave ballots, publishes its left count and derives its exclusive left prefix by
// decoupled look-back over predecessor tiles.  Left rows go to
// [begin, begin + L) ascending; right rows to [begin + L, begin + count) in
// descending position (logical order = ascending, stored reversed), so no total is
// needed in advance.  Look-back words: epoch(30) | flag(2) | value(32).
// ===========================================================================
#define TS_AGG 1ull
#define TS_INC 2ull
#define SPIN_LIMIT (1 << 20)

// Accumulate one row (packed quantized pair q) into the LDS histogram of all features.
template <int W>
__device__ __forceinline__ void lds_hist_add(unsigned long long* lds, const int32_t* cb, int F,
                                             const uint4 (&w)[W], uint32_t q) {
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
        __hip_atomic_fetch_add(&lds[cb[f] + bin], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
  }
}

// Flush a block's packed LDS histogram into the global [cells][3] integer cells.
__device__ __forceinline__ void lds_hist_flush(const unsigned long long* lds, int cells,
                                               int32_t* __restrict__ out) {
  for (int c = threadIdx.x; c < cells; c += blockDim.x) {
    const unsigned long long p = lds[c];
    if (p == 0ull) continue;
    const int64_t lo22 = (int64_t)(p & ((1ull << 22) - 1));
    const int64_t gsum = lo22 >= (1ll << 21) ? lo22 - (1ll << 22) : lo22;
    const unsigned long long rest = (p - (unsigned long long)gsum) >> 22;
    const int32_t hsum = (int32_t)(rest & ((1ull << 21) - 1));
    const int32_t n3 = (int32_t)(rest >> 21);
    int32_t* dst = out + (size_t)c * 3;
    if (gsum) __hip_atomic_fetch_add(dst, (int32_t)gsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (hsum) __hip_atomic_fetch_add(dst + 1, hsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (n3) __hip_atomic_fetch_add(dst + 2, n3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// In the tree driver, the partition pass also builds the LEFT child's integer
// histogram (ConstructHistogram over the rows routed left, accumulated while they are
// in registers); the right child's is parent - left in integers (k_fixscan).  The
// last split of a tree has no scan after it and skips the accumulation.
template <int W>
__global__ __launch_bounds__(PART_THREADS) void k_partition(DevLearner L) {
  extern __shared__ unsigned long long lds_hist[];
  __shared__ int32_t cb[16 * LGBM_MAX_W];
  __shared__ int32_t s_tile;
  __shared__ int32_t s_cnt[PART_ROWS_PER_THREAD][PART_WAVES];
  __shared__ int32_t s_pref[PART_ROWS_PER_THREAD][PART_WAVES];
  __shared__ int32_t s_total;
  __shared__ int32_t s_excl;
  Ctl* ctl = L.ctl;
  const PartJob J = ctl->part;
  if (J.driver && ctl->done) return;
  const int64_t count = J.count;
  const int64_t num_tiles = (count + PART_TILE - 1) / PART_TILE;
  const int64_t nblk = min((int64_t)gridDim.x, num_tiles);
  if ((int64_t)blockIdx.x >= nblk) return;
  const bool accum = J.driver && ctl->num_leaves < ctl->max_leaves;
  const uint32_t epoch = ctl->epoch & 0x3fffffffu;
  const int tid = threadIdx.x, wave = tid >> 6;
  const int F = L.F, cells = L.total_cells;
  if (accum) {
    for (int c = tid; c < cells; c += PART_THREADS) lds_hist[c] = 0ull;
    for (int f = tid; f < F; f += PART_THREADS) cb[f] = (int32_t)L.feats[f].cell_base;
  }
  const uint4* __restrict__ src = L.bufs.rec[J.src_buf];
  const uint16_t* __restrict__ sgh = L.bufs.gh[J.src_buf];
  uint4* __restrict__ dst = L.bufs.rec[J.dst_buf];
  uint16_t* __restrict__ dgh = L.bufs.gh[J.dst_buf];
  const int64_t begin = J.begin;
  while (true) {
    if (tid == 0)
      s_tile = __hip_atomic_fetch_add(&ctl->part_ticket, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int64_t t = s_tile;
    __syncthreads();
    if (t >= num_tiles) break;
    const int64_t base = t * PART_TILE;
    uint4 w[PART_ROWS_PER_THREAD][W];
    uint16_t q[PART_ROWS_PER_THREAD];
    bool isleft[PART_ROWS_PER_THREAD];
    int32_t rank[PART_ROWS_PER_THREAD];
#pragma unroll
    for (int k = 0; k < PART_ROWS_PER_THREAD; ++k) {
      const int64_t p = base + (int64_t)k * PART_THREADS + tid;
      const bool valid = p < count;
      bool right = false;
      if (valid) {
        const int64_t phys = J.rev ? begin + count - 1 - p : begin + p;
#pragma unroll
        for (int i = 0; i < W; ++i) w[k][i] = src[phys * W + i];
        q[k] = sgh[phys];
        const int32_t bin = (int32_t)rec_byte(w[k], J.fbyte);
        right = route_right(bin, J.pmin, J.max_bin, J.th, J.na_bin, J.flags);
      }
      isleft[k] = valid && !right;
      const unsigned long long m = __ballot(isleft[k]);
      rank[k] = (int32_t)__popcll(m & lanemask_lt());
      if (lane_id() == 0) s_cnt[k][wave] = (int32_t)__popcll(m);
    }
    __syncthreads();
    if (tid == 0) {
      int32_t acc = 0;
      for (int k = 0; k < PART_ROWS_PER_THREAD; ++k)
        for (int wv = 0; wv < PART_WAVES; ++wv) {
          s_pref[k][wv] = acc;
          acc += s_cnt[k][wv];
        }
      s_total = acc;
      // publish + look-back
      uint64_t* ts = L.tile_state;
      const uint64_t ep = (uint64_t)epoch << 34;
      int64_t excl = 0;
      if (t == 0) {
        __hip_atomic_store(&ts[0], ep | (TS_INC << 32) | (uint32_t)acc, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      } else {
        __hip_atomic_store(&ts[t], ep | (TS_AGG << 32) | (uint32_t)acc, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        int64_t p = t - 1;
        int spins = 0;
        while (p >= 0) {
          const uint64_t st = __hip_atomic_load(&ts[p], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const bool fresh = (st >> 34) == (uint64_t)epoch;
          const uint64_t flag = (st >> 32) & 3ull;
          if (!fresh || flag == 0ull) {
            ++spins;
            const bool give_up =
                spins > SPIN_LIMIT ||
                ((spins & 1023) == 0 &&
                 (__hip_atomic_load(&ctl->error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &
                  ERR_SPIN));
            if (give_up) {
              atomicOr(&ctl->error, ERR_SPIN);
              break;
            }
            __builtin_amdgcn_s_sleep(1);
            continue;
          }
          excl += (int64_t)(uint32_t)st;
          if (flag == TS_INC) break;
          --p;
        }
        __hip_atomic_store(&ts[t], ep | (TS_INC << 32) | (uint32_t)(excl + acc), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      s_excl = (int32_t)excl;
    }
    __syncthreads();
    const int64_t excl = s_excl;
    const int64_t rbase = base - excl;  // right rows before this tile
#pragma unroll
    for (int k = 0; k < PART_ROWS_PER_THREAD; ++k) {
      const int64_t pos = (int64_t)k * PART_THREADS + tid;
      if (base + pos >= count) continue;
      const int64_t lrank = s_pref[k][wave] + rank[k];
      int64_t d;
      if (isleft[k]) {
        d = begin + excl + lrank;
      } else {
        const int64_t r = rbase + (pos - lrank);
        d = begin + count - 1 - r;
      }
#pragma unroll
      for (int i = 0; i < W; ++i) dst[d * W + i] = w[k][i];
      dgh[d] = q[k];
    }
    if (accum) {
#pragma unroll
      for (int k = 0; k < PART_ROWS_PER_THREAD; ++k)
        if (isleft[k]) lds_hist_add<W>(lds_hist, cb, F, w[k], q[k]);
    }
    if (t == num_tiles - 1 && tid == 0) {
      const int32_t lc = (int32_t)(excl + s_total);
      const int32_t rc = (int32_t)(count - lc);
      if (J.driver) {
        const int32_t bl = ctl->split_leaf, nr = ctl->new_right, node = ctl->node;
        L.leaves.count[bl] = lc;
        L.leaves.begin[nr] = (int32_t)(begin + lc);
        L.leaves.count[nr] = rc;
        L.leaves.buf[bl] = J.dst_buf;
        L.leaves.buf[nr] = J.dst_buf;
        L.leaves.rev[bl] = 0;
        L.leaves.rev[nr] = 1;
        L.tree.leaf_count[bl] = lc;
        L.tree.leaf_count[nr] = rc;
        L.tree.internal_count[node] = lc + rc;
        const lgbm_split_info& b = ctl->split;
        LeafSums ls{b.left_sum_gradient, b.left_sum_hessian, b.left_output, lc, 0};
        LeafSums rs{b.right_sum_gradient, b.right_sum_hessian, b.right_output, rc, 0};
        // split_inner seeding (learner.rs:4061-4089): smaller by partition counts,
        // a tie makes the right child the smaller one.
        if (lc < rc) {
          ctl->smaller = bl;
          ctl->larger = nr;
          ctl->sm = ls;
          ctl->lg = rs;
        } else {
          ctl->smaller = nr;
          ctl->larger = bl;
          ctl->sm = rs;
          ctl->lg = ls;
        }
        // before_find_best_split gates (learner.rs:1808-1839)
        const int32_t md = ctl->max_depth;
        const int32_t min2 = ctl->cfg.min_data_in_leaf * 2;
        bool did = true;
        if (md > 0 && L.tree.leaf_depth[bl] >= md) did = false;
        if (rc < min2 && lc < min2) did = false;
        if (ctl->num_leaves >= ctl->max_leaves) did = false;  // last split: no scan follows
        ctl->skip = did ? 0 : 1;
        ctl->pending_reduce = did ? 1 : 0;
        L.stats[0] += (double)count;
        L.stats[1] += 1.0;
      } else {
        ctl->part_left_count = lc;
      }
    }
  }
  if (accum) {
    __syncthreads();
    lds_hist_flush(lds_hist, cells, L.hist_int);
  }
  if (tid == 0) {
    const int32_t prev =
        __hip_atomic_fetch_add(&ctl->part_exit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == (int32_t)nblk - 1) {
      __hip_atomic_store(&ctl->part_ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&ctl->part_exit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ctl->epoch = (ctl->epoch + 1u) & 0x3fffffffu;
      if (ctl->epoch == 0u) ctl->epoch = 1u;
    }
  }
}

// ===========================================================================
// per-tree reset (learner.rs:1242-1376: DataPartition::new, root LeafSplits,
// best_split_per_leaf, feature_splittable).
// ===========================================================================
__global__ void k_tree_init(DevLearner L, int32_t max_leaves, int32_t max_depth) {
  Ctl* ctl = L.ctl;
  const int tid = blockIdx.x * blockDim.x + threadIdx.x;
  const int nthr = gridDim.x * blockDim.x;
  const int F = L.F;
  for (int i = tid; i < max_leaves; i += nthr) {
    split_set_none(&L.best[i]);
    L.best_feat[i] = -1;
    L.best_fpos[i] = -1;
  }
  for (int i = tid; i < max_leaves * F; i += nthr) L.splittable[i] = 1;
  for (int i = tid; i < L.total_cells * 3; i += nthr) L.hist_int[i] = 0;
  if (tid == 0) {
    const int32_t N = (int32_t)L.N;
    ctl->done = 0;
    ctl->error = 0;
    ctl->num_leaves = 1;
    ctl->max_leaves = max_leaves;
    ctl->max_depth = max_depth;
    ctl->left_leaf = 0;
    ctl->right_leaf = -1;
    ctl->smaller = 0;
    ctl->larger = -1;
    // root gate (learner.rs:1830-1836): a single leaf with < 2*min_data rows
    const bool did = N >= ctl->cfg.min_data_in_leaf * 2;
    ctl->skip = did ? 0 : 1;
    ctl->pending_reduce = did ? 1 : 0;
    ctl->h_buf = BUF_ORIG;
    ctl->h_begin = 0;
    ctl->h_count = N;
    L.leaves.begin[0] = 0;
    L.leaves.count[0] = N;
    L.leaves.buf[0] = BUF_ORIG;
    L.leaves.rev[0] = 0;
    L.tree.leaf_count[0] = N;
    L.tree.leaf_depth[0] = 0;
    L.tree.leaf_parent[0] = -1;
    L.tree.leaf_weight[0] = 0.0;
    L.tree.leaf_value[0] = 0.0;
    L.stats[2] += (double)N;
    L.stats[3] += 1.0;
  }
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

__global__ void k_tree_finalize(DevLearner L) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    L.tree.header[0] = L.ctl->num_leaves;
    L.tree.header[1] = L.ctl->error;
  }
}

// Exports the partition layout: indices[leaf_begin[l] + p] = row of logical position p.
template <int W>
__global__ void k_export_layout(DevLearner L, uint32_t* __restrict__ indices) {
  const int32_t l = blockIdx.y;
  if (l >= L.ctl->num_leaves) return;
  const int64_t b = L.leaves.begin[l], c = L.leaves.count[l];
  const int32_t rev = L.leaves.rev[l];
  const uint4* __restrict__ rec = L.bufs.rec[L.leaves.buf[l]];
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < c;
       p += (int64_t)gridDim.x * blockDim.x) {
    const int64_t phys = rev ? b + c - 1 - p : b + p;
    indices[b + p] = rec[phys * W + (W - 1)].w;
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
#define DISPATCH_W(W, ...)                                                 \
  switch (W) {                                                              \
    case 1: { constexpr int kW = 1; __VA_ARGS__; } break;                  \
    case 2: { constexpr int kW = 2; __VA_ARGS__; } break;                  \
    case 3: { constexpr int kW = 3; __VA_ARGS__; } break;                  \
    case 4: { constexpr int kW = 4; __VA_ARGS__; } break;                  \
    case 5: { constexpr int kW = 5; __VA_ARGS__; } break;                  \
    case 6: { constexpr int kW = 6; __VA_ARGS__; } break;                  \
    case 7: { constexpr int kW = 7; __VA_ARGS__; } break;                  \
    case 8: { constexpr int kW = 8; __VA_ARGS__; } break;                  \
    default: break;                                                         \
  }

// Launch `kern` plainly, or with the kernel-stamped events of `ev` when timing.
#define KLAUNCH(ev, kern, grid, block, lds, s, ...)                                        \
  do {                                                                                   \
    if ((ev) && ((ev)->start || (ev)->stop))                                             \
      hipExtLaunchKernelGGL(kern, grid, block, (uint32_t)(lds), s, (ev)->start, (ev)->stop, \
                            0u, __VA_ARGS__);                                            \
    else                                                                                 \
      kern<<<grid, block, lds, s>>>(__VA_ARGS__);                                        \
  } while (0)

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
void launch_partition(const DevLearner& L, int W, int64_t count_hint, hipStream_t s,
                      const KernelEvents* ev) {
  int64_t blocks = PART_MAX_BLOCKS;
  if (count_hint > 0) blocks = std::min<int64_t>(blocks, (count_hint + PART_TILE - 1) / PART_TILE);
  if (blocks < 1) blocks = 1;
  const size_t lds = (size_t)std::max(L.total_cells, 1) * sizeof(unsigned long long);
  DISPATCH_W(W, KLAUNCH(ev, k_partition<kW>, dim3((unsigned)blocks), dim3(PART_THREADS), lds, s, L));
}
void launch_tree_init(const DevLearner& L, int32_t max_leaves, int32_t max_depth, hipStream_t s,
                      const KernelEvents* ev) {
  KLAUNCH(ev, k_tree_init, dim3(16), dim3(256), 0, s, L, max_leaves, max_depth);
}
void launch_score_update(const DevLearner& L, double lr, double* score, hipStream_t s,
                         const KernelEvents* ev) {
  int64_t blocks = std::min<int64_t>((L.N + 255) / 256, 4096);
  if (blocks < 1) blocks = 1;
  DISPATCH_W(L.W, KLAUNCH(ev, k_score_update<kW>, dim3((unsigned)blocks), dim3(256), 0, s, L, lr,
                          score));
}
void launch_tree_finalize(const DevLearner& L, hipStream_t s) { k_tree_finalize<<<1, 64, 0, s>>>(L); }
void launch_export_layout(const DevLearner& L, int32_t num_leaves, uint32_t* indices,
                          hipStream_t s) {
  DISPATCH_W(L.W, (k_export_layout<kW><<<dim3(64, (unsigned)num_leaves), dim3(256), 0, s>>>(
                      L, indices)));
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
