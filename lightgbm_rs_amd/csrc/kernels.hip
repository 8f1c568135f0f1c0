// kernels.hip — gfx950 kernels of the tree-learner hot path and their launchers.
//
//   k_pack_records   resident bin layout (upload_resident_bins, lib.rs:4368-4433)
//   k_grad_binary    BinaryLogloss::get_gradients (lgbm-objective/src/binary.rs:134-172)
//   k_grad_softmax   MulticlassSoftmax::get_gradients (lgbm-objective/src/multiclass.rs:138-180)
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
//   k_walk           score update through the grown tree (and the layout's leaf ids) (score_updater.rs:133;
//                    learner.rs:4380-4395)
#include "scan.h"

#include <hip/hip_ext.h>

#include <algorithm>

namespace lgbm {

// ===========================================================================
// upload: feature-major u8 -> records
// ===========================================================================
__global__ void k_pack_records(const uint8_t* __restrict__ bins, int64_t n, int32_t F, int32_t fmt,
                               uint4* __restrict__ rec) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n) return;
  const int U = rec_words(fmt);
  uint32_t words[4 * LGBM_MAX_W];
  for (int i = 0; i < U; ++i) words[i] = 0u;
  for (int f = 0; f < F; ++f) {
    int wi, sh;
    rec_field_pos(fmt, f, &wi, &sh);
    words[wi] |= (uint32_t)bins[(size_t)f * n + r] << sh;
  }
  if (!rec_packed(fmt)) words[U - 1] = (uint32_t)r;
  uint2* out = (uint2*)rec;
  for (int i = 0; i < U / 2; ++i) out[r * (U / 2) + i] = make_uint2(words[2 * i], words[2 * i + 1]);
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

// MulticlassSoftmax::get_gradients (lgbm-objective/src/multiclass.rs:138-180) with
// Common::Softmax (lgbm-model/src/objective.rs:307-322), per row over the class-major
// scores: the max by a fold from class 0, e_k = exp(s_k - max), their sum in class
// order, p_k = e_k / sum; grad = p - 1 for the row's class, else p; hess =
// factor p (1 - p); f32 on store.  KR > 0: the K exponentials stay in registers; KR =
// 0 (any K): they are recomputed (the same operations, so the same values).
template <int KR>
__global__ __launch_bounds__(256) void k_grad_softmax(const double* __restrict__ score,
                                                      const float* __restrict__ label,
                                                      float* __restrict__ g, float* __restrict__ h,
                                                      int64_t n, int32_t K, double factor) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride) {
    const float lf = label[r];
    const int32_t li = lf == lf ? (int32_t)lf : 0;  // labels were checked to lie in (-1, K)
    if constexpr (KR > 0) {
      double e[KR];
#pragma unroll
      for (int k = 0; k < KR; ++k) e[k] = score[(size_t)k * n + r];
      double wmax = e[0];
#pragma unroll
      for (int k = 1; k < KR; ++k) wmax = fmax(e[k], wmax);
      double wsum = 0.0;
#pragma unroll
      for (int k = 0; k < KR; ++k) {
        e[k] = exp(e[k] - wmax);
        wsum += e[k];
      }
#pragma unroll
      for (int k = 0; k < KR; ++k) {
        const double p = e[k] / wsum;
        g[(size_t)k * n + r] = li == k ? (float)(p - 1.0) : (float)p;
        h[(size_t)k * n + r] = (float)(factor * p * (1.0 - p));
      }
    } else {
      double wmax = score[r];
      for (int32_t k = 1; k < K; ++k) wmax = fmax(score[(size_t)k * n + r], wmax);
      double wsum = 0.0;
      for (int32_t k = 0; k < K; ++k) wsum += exp(score[(size_t)k * n + r] - wmax);
      for (int32_t k = 0; k < K; ++k) {
        const double p = exp(score[(size_t)k * n + r] - wmax) / wsum;
        g[(size_t)k * n + r] = li == k ? (float)(p - 1.0) : (float)p;
        h[(size_t)k * n + r] = (float)(factor * p * (1.0 - p));
      }
    }
  }
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
  ctl->hmin = s.hmin == 0xffffffffu ? 0.f : f32_from_key(s.hmin);
}

// ===========================================================================
// f32 gradients (use_quantized_grad = false): 64-bit fixed-point histogram scales.
// A row's g becomes the integer round(g * 2^g_shift) (h likewise).  With |g| <= 2^e
// and fewer than 2^b rows, g_shift = 62 - b - e keeps every partial sum below 2^62,
// so cells, leaf totals and parent - child differences are exact integers, and the
// f64 cell (double)sum * 2^-g_shift is within one rounding of the exact sum of the
// f32 values — far inside the 1e-5 relative parity bound of the f64 fold.
// ===========================================================================
__device__ __forceinline__ int32_t fp_shift(float amax, int64_t n) {
  int b = 1;
  while ((1ll << b) <= n) ++b;
  if (!(amax > 0.0f) || !(amax < __builtin_inff())) return 62 - b;
  int e = 0;
  (void)frexpf(amax, &e);  // amax < 2^e
  return 62 - b - e;
}

__global__ __launch_bounds__(256) void k_fp_scales(Ctl* ctl, const uint4* __restrict__ partials,
                                                   int32_t nparts, int64_t n) {
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
  ctl->g_shift = fp_shift(__uint_as_float(s.ag), n);
  ctl->h_shift = fp_shift(__uint_as_float(s.ah), n);
}

// Quantized gradients of any bin count (num_grad_quant_bins other than 2 and 4) go
// through the fixed-point path above with exact scales.  Every dequantized value
// f32(q * scale) with |q| >= 1 has at least f32(1 * scale)'s magnitude, so its ulp is a
// multiple of u = ulp(f32(1 * scale)) and the value an integer multiple of u: with
// shift = -log2(u) each row's fixed-point value is that integer exactly (below 2^32),
// cells, leaf totals and parent - child are exact, and (double)sum * u equals the
// reference's f64 fold of the dequantized values whenever that fold is exact (every
// partial sum below 2^53 u).
__device__ __forceinline__ int32_t exact_shift(float v1) {
  if (!(v1 > 0.0f) || !(v1 < __builtin_inff())) return 0;  // no nonzero value
  if (v1 < 1.17549435e-38f) return 149;                      // subnormal: u = 2^-149
  int e = 0;
  (void)frexpf(v1, &e);  // v1 = f * 2^e, f in [0.5, 1): ulp = 2^(e - 24)
  return 24 - e;
}
__global__ void k_exact_shifts(Ctl* ctl) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  ctl->g_shift = exact_shift(ctl->vg1);
  ctl->h_shift = exact_shift(ctl->vh1);
}

__global__ void k_pack_g32(const float* __restrict__ g, const float* __restrict__ h, int64_t n,
                           float2* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = make_float2(g[i], h[i]);
}

// ===========================================================================
// quantize: discretize_dequantize_in_place (gradient_discretizer.rs:126-139,
// quantize_pair :173-188, next_u01 :255-263).  Row r consumes xorshift draws
// 2r+1 (grad) and 2r+2 (hess) of the sequential stream; a lane starts at row
// wave_row0 + lane*C with state M^(2*(row)) s0, M being the GF(2) matrix of one
// xorshift step: the wave applies the precomputed powers P_k = M^(2*64*C*2^k) for the
// bits of its wave index cooperatively (lane i owns column i, xor-reduce), then
// lane l applies T^l, T = M^(2*C), from a table of all 64 lane offsets.
// ===========================================================================
// One DPP row rotation of a 64-bit value (all 64 lanes active).
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_ror_u64(uint64_t v) {
  const uint32_t lo =
      (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xf, 0xf, false);
  const uint32_t hi =
      (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
  return ((uint64_t)hi << 32) | lo;
}
// XOR of a 64-bit value over the wave, uniform result: row rotations by 1, 2, 4, 8
// leave every lane of a 16-lane row with the row's XOR; rows combine from lanes
// 0, 16, 32, 48.  Requires all 64 lanes active.
__device__ __forceinline__ uint64_t wave_xor_u64(uint64_t v) {
  v ^= dpp_ror_u64<0x121>(v);
  v ^= dpp_ror_u64<0x122>(v);
  v ^= dpp_ror_u64<0x124>(v);
  v ^= dpp_ror_u64<0x128>(v);
  uint64_t r = 0ull;
#pragma unroll
  for (int row = 0; row < 4; ++row) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 16 * row);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 16 * row);
    r ^= ((uint64_t)hi << 32) | lo;
  }
  return r;
}
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
// consecutive rows (padded index: one spare slot per run makes the lane stride odd,
// so the lanes of a wave hit different banks).
#define QUANT_BLOCK_ROWS (4 * LGBM_WAVE * QUANT_ROWS_PER_LANE)
#define QUANT_LDS_ROWS (QUANT_BLOCK_ROWS + QUANT_BLOCK_ROWS / QUANT_ROWS_PER_LANE)
__device__ __forceinline__ int qidx(int r) { return r + r / QUANT_ROWS_PER_LANE; }

__global__ __launch_bounds__(256) void k_quantize(const float* __restrict__ g,
                                                  const float* __restrict__ h, int64_t n,
                                                  const Ctl* __restrict__ ctl,
                                                  const uint64_t* __restrict__ wave_mats,
                                                  const uint64_t* __restrict__ lane_mats,
                                                  uint64_t s0, int32_t stochastic,
                                                  uint16_t* __restrict__ gh,
                                                  float* __restrict__ dg, float* __restrict__ dh) {
  __shared__ float sg_[QUANT_LDS_ROWS];
  __shared__ float sh_[QUANT_LDS_ROWS];
  __shared__ uint16_t sq_[QUANT_LDS_ROWS];
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
        const uint64_t term = ((sw >> lane) & 1ull) ? wave_mats[k * 64 + lane] : 0ull;
        sw = wave_xor_u64(term);
      }
    }
    // lane l: T^l applied to the wave's state (sw is wave-uniform)
    uint64_t y = 0ull;
    for (int i = 0; i < 64; ++i)
      if ((sw >> i) & 1ull) y ^= lane_mats[i * 64 + lane];
    st = y;
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

// Recovery of the quantized pairs from dequantized values f32(q * scale)
// (lgbm_hip_set_dequantized_gradients): q = round(v / scale), checked by the product.
// bad[0] counts rows that fail, bad[1] is the first such row.
__global__ __launch_bounds__(256) void k_requant(const float* __restrict__ g,
                                                 const float* __restrict__ h, int64_t n,
                                                 const Ctl* __restrict__ ctl, int32_t bins,
                                                 uint16_t* __restrict__ gh,
                                                 unsigned long long* __restrict__ bad) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n) return;
  const double gs = ctl->gs, hs = ctl->hs;
  const float gv = g[r], hv = h[r];
  const double qgd = rint((double)gv / gs), qhd = rint((double)hv / hs);
  const double gmax = (double)(bins / 2);
  bool ok = qgd >= -gmax && qgd <= gmax && qhd >= 0.0 && qhd <= (double)bins;
  const int32_t qg = ok ? (int32_t)qgd : 0, qh = ok ? (int32_t)qhd : 0;
  ok = ok && (float)((double)qg * gs) == gv && (float)((double)qh * hs) == hv;
  if (!ok) {
    atomicAdd(&bad[0], 1ull);
    atomicMin(&bad[1], (unsigned long long)r);
    return;
  }
  gh[r] = (uint16_t)((uint16_t)(uint8_t)(int8_t)qg | ((uint16_t)(uint8_t)qh << 8));
}

// ===========================================================================
// ConstructHistogram (integer), batched over the histogram jobs of a round (the
// smaller child of every split; the root; a per-op build).  A job is a physical row
// range of one row buffer; row order is irrelevant because integer addition is
// associative.  The rows of all jobs are cut into chunks of R rows (at least
// HIST_MIN_ROWS, at most HIST_GRID chunks over all jobs); chunk a is one block, which
// stores its histogram with plain stores into partial slot a.  Consumers add the
// partial slots [a0, a0 + nblk) of a job (recorded in its HistJob by block 0).
//
// Two accumulation schemes:
//  - wave-private (cells <= HIST_WAVE_CELLS): each wave owns a u32 LDS histogram of
//    packed cells  q_g + (q_h << 11) + ([q_h == 3] << 22)  (fields 11-bit signed,
//    11-bit, 10-bit: exact for <= 511 rows), folds it at least every
//    HIST_FOLD_STEPS x 64 rows into one 64-bit register per lane cell (lane l owns
//    cells l, l + 64, ...) packed the same way with 22 / 21 / 21-bit fields (exact
//    for < 2^19 rows per wave: N < 2^29 over 512 blocks of 8 waves), and the waves
//    are combined at the end.  One 32-bit LDS atomic per (row, feature); rows whose
//    quantized pair is (0, 0) add nothing and are skipped.
//  - block-shared: one u64 LDS histogram per block, cells
//    q_g + (q_h << 22) + ([q_h == 3] << 43) (exact for < 2^19 rows per block).
// ===========================================================================
__device__ __forceinline__ void hist_assign(const Ctl* ctl, int32_t nj, int32_t* s_a0,
                                            int32_t* s_nb, int64_t* s_R, int64_t grid) {
  int64_t S = 0;
  for (int j = 0; j < nj; ++j) S += max(ctl->hjobs[j].count, (int64_t)0);
  int64_t R = (S + grid - 1) / grid;
  if (R < HIST_MIN_ROWS) R = HIST_MIN_ROWS;
  int32_t acc = 0;
  for (int j = 0; j < nj; ++j) {
    const int64_t c = ctl->hjobs[j].count;
    const int32_t nb = c > 0 ? (int32_t)((c + R - 1) / R) : 0;
    s_a0[j] = acc;
    s_nb[j] = nb;
    acc += nb;
  }
  *s_R = R;
}

template <int FMT, bool WAVE_PRIVATE>
__global__ __launch_bounds__(HIST_THREADS, 2) void k_hist_jobs(DevLearner L) {
  constexpr int U = rec_words(FMT), BPW = rec_bpw(FMT), BB = rec_bits(FMT), NS = rec_slots(FMT);
  constexpr uint32_t BM = (1u << BB) - 1u;
  extern __shared__ uint32_t lds_u32[];
  __shared__ int32_t cb[NS];
  __shared__ int32_t s_a0[SPEC_MAX], s_nb[SPEC_MAX];
  __shared__ int64_t s_R;
  Ctl* ctl = L.ctl;
  const int32_t nj = ctl->n_hjobs;
  if (nj <= 0) return;
  const int tid = threadIdx.x, lane = (int)lane_id(), wave = tid >> 6;
  const int F = L.F, cells = L.total_cells;
  // Record words 0 .. nw-1 hold the bins; slots of the last word beyond F are zero
  // and land in a trash cell at index `cells`.
  const int nw = (F + BPW - 1) / BPW;
  if (tid == 0) {
    hist_assign(ctl, nj, s_a0, s_nb, &s_R, HIST_GRID_Q);
    if (blockIdx.x == 0)
      for (int j = 0; j < nj; ++j) {
        ctl->hjobs[j].a0 = s_a0[j];
        ctl->hjobs[j].nblk = s_nb[j];
      }
  }
  for (int f = tid; f < NS; f += HIST_THREADS)
    cb[f] = f < F ? (int32_t)L.feats[f].cell_base : cells;
  __syncthreads();
  const int32_t a = (int32_t)blockIdx.x;
  int32_t j = -1;
  for (int k = 0; k < nj; ++k)
    if (a >= s_a0[k] && a < s_a0[k] + s_nb[k]) j = k;
  if (j < 0) return;
  const HistJob& J = ctl->hjobs[j];
  const int64_t R = s_R;
  const int64_t lo = (int64_t)(a - s_a0[j]) * R;
  const int64_t hi = min(J.count, lo + R);
  // the jobs read the original order (root) or a gathered scratch buffer: pairs from
  // the gh array
  const uint4* __restrict__ rec = rec_buf(L.bufs, J.buf);  // rows J.begin + r
  const uint16_t* __restrict__ gh = L.bufs.gh[J.buf] + J.begin;
  const int64_t rb = J.begin;
  int32_t* __restrict__ out = L.hist_part + (size_t)a * cells * 3;
  // bin-slot cell bases in scalar registers (wave-uniform)
  int32_t cbr[NS];
#pragma unroll
  for (int f = 0; f < NS; ++f) cbr[f] = __builtin_amdgcn_readfirstlane(cb[f]);

  if constexpr (WAVE_PRIVATE) {
    constexpr int NPL = HIST_WAVE_CELLS / LGBM_WAVE;  // cells per lane
    const int stride = cells + LDS_TRASH_CELLS;       // + trash cells
    uint32_t* my = lds_u32 + (size_t)wave * stride;
    for (int c = lane; c < stride; c += LGBM_WAVE) my[c] = 0u;
    unsigned long long acc64[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) acc64[i] = 0ull;
    // the wave's contiguous share of the block's rows, HIST_ROWS_PER_LANE per lane
    // per step (loads first, then the atomics)
    const int64_t n = hi - lo;
    const int64_t wper = (n + HIST_WAVES - 1) / HIST_WAVES;
    const int64_t wlo = lo + min(n, (int64_t)wave * wper);
    const int64_t whi = lo + min(n, (int64_t)(wave + 1) * wper);
    int step = 0;
    auto fold = [&]() {
#pragma unroll
      for (int i = 0; i < NPL; ++i) {
        const int c = i * LGBM_WAVE + lane;
        if (c < cells) {
          const uint32_t p = my[c];
          my[c] = 0u;
          const int32_t g = ((int32_t)(p << 21)) >> 21;
          const uint32_t rest = (p - (uint32_t)g) >> 11;
          acc64[i] += (unsigned long long)(long long)g +
                      ((unsigned long long)(rest & 0x7ffu) << 22) +
                      ((unsigned long long)(rest >> 11) << 43);
        }
      }
    };
    constexpr int RU = HIST_ROWS_PER_LANE;
    for (int64_t r0 = wlo; r0 < whi; r0 += LGBM_WAVE * RU) {
      uint32_t w[RU][U];
      uint32_t q[RU];
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const int64_t r = r0 + u * LGBM_WAVE + lane;
        q[u] = 0u;
        if (r < whi) {
          rec_load<FMT>(rec, rb + r, w[u]);
          q[u] = (uint32_t)gh[r];  // 0: no row, or a (0, 0) pair
        }
      }
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        if (q[u] == 0u) continue;
        const int32_t qg = (int32_t)(int8_t)(q[u] & 0xffu);
        const int32_t qh = (int32_t)(int8_t)((q[u] >> 8) & 0xffu);
        const uint32_t v = (uint32_t)qg + ((uint32_t)qh << 11) + ((qh == 3 ? 1u : 0u) << 22);
        // slots past F hold no feature: skipped by a uniform branch
#pragma unroll
        for (int k = 0; k < (NS + BPW - 1) / BPW; ++k) {
          if (k < nw) {
            const uint32_t word = w[u][k];
#pragma unroll
            for (int bb = 0; bb < BPW; ++bb)
              if (BPW * k + bb < NS && BPW * k + bb < F) {
                const int ad = cbr[BPW * k + bb] + (int)((word >> (BB * bb)) & BM);
                __hip_atomic_fetch_add(&my[ad], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
              }
          }
        }
      }
      step += RU;
      if (step + RU > HIST_FOLD_STEPS) {
        step = 0;
        fold();
      }
    }
    fold();
    // combine the waves: int32 [cells][3] in the (now free) LDS
    __syncthreads();
    int32_t* acc = (int32_t*)lds_u32;
    for (int c = tid; c < cells * 3; c += HIST_THREADS) acc[c] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int c = i * LGBM_WAVE + lane;
      if (c < cells && acc64[i] != 0ull) {
        const unsigned long long p = acc64[i];
        const int64_t lo22 = (int64_t)(p & ((1ull << 22) - 1));
        const int64_t g = lo22 >= (1ll << 21) ? lo22 - (1ll << 22) : lo22;
        const unsigned long long rest = (p - (unsigned long long)g) >> 22;
        const int32_t h = (int32_t)(rest & ((1ull << 21) - 1)), t = (int32_t)(rest >> 21);
        if (g) atomicAdd(&acc[c * 3], (int32_t)g);
        if (h) atomicAdd(&acc[c * 3 + 1], h);
        if (t) atomicAdd(&acc[c * 3 + 2], t);
      }
    }
    __syncthreads();
    for (int c = tid; c < cells * 3; c += HIST_THREADS) out[c] = acc[c];
  } else {
    unsigned long long* h64 = (unsigned long long*)lds_u32;
    for (int c = tid; c < cells + LDS_TRASH_CELLS; c += HIST_THREADS) h64[c] = 0ull;
    __syncthreads();
    for (int64_t r = lo + tid; r < hi; r += HIST_THREADS) {
      uint32_t w[U];
      rec_load<FMT>(rec, rb + r, w);
      const uint16_t q = gh[r];
      if (q) lds_hist_add<FMT>(h64, cbr, nw, F, cells + 4 + lane, w, q);  // (0, 0) adds nothing
    }
    __syncthreads();
    for (int c = tid; c < cells; c += HIST_THREADS) {
      const unsigned long long p = h64[c];
      const int64_t lo22 = (int64_t)(p & ((1ull << 22) - 1));
      const int64_t gsum = lo22 >= (1ll << 21) ? lo22 - (1ll << 22) : lo22;
      const unsigned long long rest = (p - (unsigned long long)gsum) >> 22;
      out[c * 3] = (int32_t)gsum;
      out[c * 3 + 1] = (int32_t)(rest & ((1ull << 21) - 1));
      out[c * 3 + 2] = (int32_t)(rest >> 21);
    }
  }
}

// Sum of histogram job 0's partial slots into L.hist_sum ([cells][3] int32): one
// thread per (column, slot group), 16 columns x 16 groups per block, the groups
// combined through LDS.  Consumers then read one slot instead of one per block.
__global__ __launch_bounds__(256) void k_hist_reduce(DevLearner L) {
  __shared__ int32_t part[16][17];
  const Ctl* ctl = L.ctl;
  const int32_t a0 = ctl->hjobs[0].a0, na = ctl->n_hjobs > 0 ? ctl->hjobs[0].nblk : 0;
  const int64_t ncol = (int64_t)L.total_cells * 3;
  const int cl = threadIdx.x & 15, g = threadIdx.x >> 4;
  const int64_t col = (int64_t)blockIdx.x * 16 + cl;
  int32_t s = 0;
  if (col < ncol) {
    const int32_t* p = L.hist_part + (size_t)a0 * ncol + col;
    int32_t x[4] = {0, 0, 0, 0};
    int k = g;
    for (; k + 48 < na; k += 64) {
#pragma unroll
      for (int u = 0; u < 4; ++u) x[u] += p[(size_t)(k + 16 * u) * ncol];
    }
    for (; k < na; k += 16) x[0] += p[(size_t)k * ncol];
    s = (x[0] + x[1]) + (x[2] + x[3]);
  }
  part[g][cl] = s;
  __syncthreads();
  if (g == 0 && col < ncol) {
    int32_t t = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) t += part[k][cl];
    L.hist_sum[col] = t;
  }
}

// f32 gradients: ConstructHistogram of the histogram jobs into 64-bit fixed-point
// (g, h) cells with 64-bit LDS atomics (exact, order-independent).  Block (chunk a,
// feature group y): the rows of chunk a (hist_assign) and the features of group y,
// whose cells fit LDS; partial slot a receives the group's cells.
template <int FMT>
__global__ __launch_bounds__(HIST_THREADS) void k_hist_f32(DevLearner L) {
  constexpr int U = rec_words(FMT);
  extern __shared__ unsigned long long lds64[];
  __shared__ int32_t cb[16 * LGBM_MAX_W];
  __shared__ int32_t s_pos[16 * LGBM_MAX_W];  // feature f's field: word << 8 | shift
  __shared__ int32_t s_a0[SPEC_MAX], s_nb[SPEC_MAX];
  __shared__ int64_t s_R;
  Ctl* ctl = L.ctl;
  const int32_t nj = ctl->n_hjobs;
  const int grp = blockIdx.y;
  if (nj <= 0 || grp >= L.n_fgroups) return;
  const int tid = threadIdx.x;
  const int cells = L.total_cells;
  const int f0 = L.fgroup_first[grp], f1 = L.fgroup_first[grp + 1];
  if (tid == 0) {
    hist_assign(ctl, nj, s_a0, s_nb, &s_R, HIST_GRID);
    if (blockIdx.x == 0 && grp == 0)
      for (int j = 0; j < nj; ++j) {
        ctl->hjobs[j].a0 = s_a0[j];
        ctl->hjobs[j].nblk = s_nb[j];
      }
  }
  for (int f = f0 + tid; f < f1; f += HIST_THREADS) {
    cb[f] = (int32_t)L.feats[f].cell_base;
    int wi, sh;
    rec_field_pos(FMT, f, &wi, &sh);
    s_pos[f] = (wi << 8) | sh;
  }
  __syncthreads();
  const int32_t a = (int32_t)blockIdx.x;
  int32_t j = -1;
  for (int k = 0; k < nj; ++k)
    if (a >= s_a0[k] && a < s_a0[k] + s_nb[k]) j = k;
  if (j < 0) return;
  const int cbase = cb[f0];
  const int gcells = (f1 < L.F ? (int)L.feats[f1].cell_base : cells) - cbase;
  for (int c = tid; c < 2 * gcells; c += HIST_THREADS) lds64[c] = 0ull;
  __syncthreads();
  const HistJob& J = ctl->hjobs[j];
  const int64_t R = s_R;
  const int64_t lo = (int64_t)(a - s_a0[j]) * R;
  const int64_t hi = min(J.count, lo + R);
  const uint4* __restrict__ rec = rec_buf(L.bufs, J.buf);  // rows J.begin + r
  const float2* __restrict__ gh = L.bufs.g32[J.buf] + J.begin;
  const int64_t rb = J.begin;
  const double gm = ldexp(1.0, ctl->g_shift), hm = ldexp(1.0, ctl->h_shift);
  for (int64_t r = lo + tid; r < hi; r += HIST_THREADS) {
    uint32_t w[U];
    rec_load<FMT>(rec, rb + r, w);
    const float2 v = gh[r];
    const unsigned long long gi = (unsigned long long)(long long)rint((double)v.x * gm);
    const unsigned long long hi_ = (unsigned long long)(long long)rint((double)v.y * hm);
    for (int f = f0; f < f1; ++f) {
      const int pos = s_pos[f];
      const int c = cb[f] - cbase + (int)rec_field<FMT>(w, pos >> 8, pos & 0xff);
      __hip_atomic_fetch_add(&lds64[2 * c], gi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_fetch_add(&lds64[2 * c + 1], hi_, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
  __syncthreads();
  int64_t* out = L.hist_part64 + ((size_t)a * cells + cbase) * 2;
  for (int c = tid; c < 2 * gcells; c += HIST_THREADS) out[c] = (int64_t)lds64[c];
}

// ===========================================================================
// k_fixscan: one block (two waves) per feature.
//   mode 1 (root):  node slot 0 from the histogram of all rows: root LeafSplits sums
//                   (exact, from the integer totals), FixHistogram, compaction, and
//                   the root's FindBestThreshold (wave 0).
//   mode 2 (build): per-op build into `explicit_out` (no scan).
// The integer cells are the sum of histogram job 0's partial slots (the wide layout's
// per-chunk slots); the wide layout's root sums come from its totals cell (its
// most-frequent-bin cells are not accumulated).
// ===========================================================================
__global__ __launch_bounds__(SCAN_THREADS) void k_fixscan(DevLearner L, int32_t mode,
                                                          double* __restrict__ explicit_out) {
  extern __shared__ __align__(16) double cs[];  // [2 * max_bins] f64 cells of the feature
  __shared__ long long tot[3][SCAN_THREADS / LGBM_WAVE];
  Ctl* ctl = L.ctl;
  const int f = blockIdx.x;
  if (mode == 1 && ctl->done) return;
  const int tid = threadIdx.x;
  const DevFeature ft = L.feats[f];
  const int nb = (int)ft.num_bin;
  const double vg1 = (double)ctl->vg1, vh1 = (double)ctl->vh1, vh3 = (double)ctl->vh3;
  long long tg = 0, th = 0, t3 = 0;
  const int32_t a0 = ctl->hjobs[0].a0, na = ctl->hjobs[0].nblk;
  const bool fp = ctl->fp_mode != 0;
  const bool wide = rec_wide(L.fmt);
  const double gu = ldexp(1.0, -ctl->g_shift), hu = ldexp(1.0, -ctl->h_shift);
  for (int b = tid; b < nb; b += SCAN_THREADS) {
    const size_t ci = (size_t)(ft.cell_base + b);
    if (fp) {
      long long G = 0, H = 0;
      if (wide) {
        for (int k = 0; k < na; ++k) {
          const unsigned long long* wp = L.wide_part + ((size_t)(a0 + k) * L.total_cells + ci) * 2;
          G += (long long)wp[0];
          H += (long long)wp[1];
        }
      } else {
        hist_part_sum64(L, a0, na, ci, &G, &H);
      }
      if (mode == 1) {
        int64_t* ps = L.int_slots64 + ci * 2;  // node slot 0
        ps[0] = G;
        ps[1] = H;
      }
      cs[2 * b] = (double)G * gu;
      cs[2 * b + 1] = (double)H * hu;
      tg += G;
      th += H;
      continue;
    }
    int32_t G = 0, H = 0, T = 0;
    if (wide) {
      for (int k = 0; k < na; ++k) {
        int32_t g_, h_, t_;
        unpack_cell(L.wide_part[(size_t)(a0 + k) * L.total_cells + ci], &g_, &h_, &t_);
        G += g_;
        H += h_;
        T += t_;
      }
    } else {
      G = L.hist_sum[ci * 3];
      H = L.hist_sum[ci * 3 + 1];
      T = L.hist_sum[ci * 3 + 2];
    }
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
    if (wide) {  // the totals cell (job 0, cell total_cells)
      const size_t t = (size_t)L.total_cells;
      if (fp) {
        G = L.hist_acc64[2 * t];
        H = L.hist_acc64[2 * t + 1];
      } else {
        G = L.hist_acc[3 * t];
        H = L.hist_acc[3 * t + 1];
        T = L.hist_acc[3 * t + 2];
      }
    }
    if (fp) {
      sg = (double)G * gu;
      sh = (double)H * hu;
    } else {
      sg = (double)G * vg1;
      sh = (double)(H - 3ll * T) * vh1 + (double)T * vh3;
    }
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
      // the packed integer cells hold q_h in [0, bins]
      if (!fp && ctl->hmin < 0.f) {
        ctl->error |= ERR_NEG_HESSIAN;
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
  if (tid == 0) {
    // the root's fixed cell (its other f64 cells are its integer cells)
    const int mfb = (int)ft.mfb, tm = mfb - ft.offset;
    if (mfb > 0 && mfb < nb && tm >= 0) L.mfbv[f] = make_double2(cs[2 * tm], cs[2 * tm + 1]);
  }
  if (tid >= LGBM_WAVE) return;
  lgbm_split_info* out = L.feat_split + f;
  // a feature outside the tree's column sample is never scanned (learner.rs:1932-1990)
  const bool sampled_out = L.feat_used && !L.feat_used[f];
  if (ctl->root_skip || !(sh > 0.0 && nrows > 0) || sampled_out) {
    if (lane_id() == 0) {
      split_set_none(out);
      L.gain_dense[f] = -__builtin_inf();
      L.splittable[f] = 0;
    }
    return;
  }
  const ScanCfg sc = make_scan_cfg(ctl->cfg);
  const double gain =
      ft.categorical  // bin_type dispatch (learner.rs:3103-3118)
          ? wave_scan_cat(cs, ft, sc, ctl->cfg, sg, sh, nrows, weight, out,
                          L.cat_bits + (size_t)f * 8)
          : wave_scan(cs, ft, sc, sg, sh, nrows, weight, out);
  if (lane_id() == 0) {
    L.splittable[f] = gain > -__builtin_inf() ? 1 : 0;
    out->gain = gain * ft.penalty;  // feature_contri (learner.rs:3235-3252)
    L.gain_dense[f] = gain * ft.penalty;
  }
}

// Per-op FindBestThreshold over explicit features (find_best_splits_batched,
// lib.rs:1500-1548): one wave per feature, host-provided histogram.
__global__ __launch_bounds__(LGBM_WAVE) void k_scan_explicit(const double* __restrict__ hist,
                                                             const DevFeature* __restrict__ feats,
                                                             int32_t n_feats,
                                                             lgbm_gain_config cfg, double sg,
                                                             double sh, int32_t n,
                                                             lgbm_split_info* out) {
  __shared__ __align__(16) double cs[2 * 256];
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
// adding the shrunk leaf value (Tree::shrinkage, tree.rs:1074).  A thread stages its
// record in LDS and walks the tree with one byte read and one route-mask word per
// level (k_tree_finalize precomputes, per node, the set of bins routed right).  The
// wide layout reads each level's byte from the row's binmat row instead.
// ===========================================================================
template <int FMT, bool LEAF_OF>
__global__ __launch_bounds__(256) void k_walk(DevLearner L, double lr, double* __restrict__ score,
                                              uint8_t* __restrict__ leaf_of) {
  constexpr int U = rec_words(FMT), BPW = rec_bpw(FMT), BB = rec_bits(FMT);
  constexpr uint32_t BM = (1u << BB) - 1u;
  constexpr int kStride = U + 1;  // words per staged record: odd (U is even), so word
                                  // reads of different lanes hit different banks
  constexpr bool WIDE = rec_wide(FMT);
  __shared__ uint32_t s_mask[(MAX_LEAVES - 1) * 8];
  __shared__ uint32_t s_node[MAX_LEAVES - 1];
  __shared__ int32_t s_wf[WIDE ? MAX_LEAVES - 1 : 1];  // wide: node -> feature position
  __shared__ double vals[MAX_LEAVES];
  __shared__ uint32_t s_rec[256 * kStride];
  const int32_t nl = L.ctl->num_leaves;
  if (!LEAF_OF && nl <= 1) return;
  const int tid = threadIdx.x;
  for (int i = tid; i < (nl - 1) * 8; i += blockDim.x) s_mask[i] = L.tree.route_mask[i];
  for (int i = tid; i < nl - 1; i += blockDim.x) s_node[i] = L.tree.route_node[i];
  if constexpr (WIDE)
    for (int i = tid; i < nl - 1; i += blockDim.x) s_wf[i] = L.tree.nodes[i].f;
  if (!LEAF_OF)
    for (int i = tid; i < nl; i += blockDim.x)
      vals[i] = maybe_round_to_zero(L.tree.leaf_value[i] * lr);
  __syncthreads();
  const uint4* __restrict__ rec = L.bufs.rec[BUF_ORIG];
  uint32_t* mine = s_rec + tid * kStride;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const uint8_t* __restrict__ bm = L.binmat;
  const int64_t rstride = L.row_stride;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + tid; r < L.N; r += stride) {
    if constexpr (!WIDE) {
      uint32_t w[U];
      rec_load<FMT>(rec, r, w);
#pragma unroll
      for (int i = 0; i < U; ++i) mine[i] = w[i];
    }
    int32_t node = 0;
    for (int depth = 0; depth < nl && node >= 0; ++depth) {  // a path has < nl nodes
      const uint32_t u = s_node[node];
      uint32_t bin;
      if constexpr (WIDE) {
        if (L.bin16) {
          // 2-byte bins: the node's router, not the 256-bin route set (categorical
          // features keep at most 256 bins)
          bin = *(const uint16_t*)(bm + r * rstride + 2 * s_wf[node]);
          const NodeRoute nr = L.tree.nodes[node];
          if (!(nr.flags & ROUTE_CAT)) {
            const bool right =
                route_right((int32_t)bin, nr.pmin, nr.max_bin, nr.th, nr.na_bin, nr.flags);
            node = right ? ((int32_t)u >> 20) : ((int32_t)(u << 12) >> 20);
            continue;
          }
        } else {
          bin = bm[r * rstride + s_wf[node]];
        }
      } else {
        const uint32_t f = u & 0xffu;
        const uint32_t wi = f / BPW;
        bin = (mine[wi] >> (BB * (f - wi * BPW))) & BM;
      }
      const uint32_t right = (s_mask[node * 8 + (bin >> 5)] >> (bin & 31u)) & 1u;
      node = right ? ((int32_t)u >> 20) : ((int32_t)(u << 12) >> 20);
    }
    if (LEAF_OF) {
      leaf_of[r] = (uint8_t)(nl <= 1 ? 0 : ~node);
    } else if (node < 0 && ~node < nl) {
      score[r] += vals[~node];
    }
  }
}

__global__ void k_gather_rows(const uint32_t* __restrict__ rows, int64_t n, int32_t U,
                              const uint4* __restrict__ rec, const uint16_t* __restrict__ gh,
                              const float2* __restrict__ g32, uint4* __restrict__ rec_out,
                              uint16_t* __restrict__ gh_out, float2* __restrict__ g32_out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t r = rows[i];
  const uint2* src = (const uint2*)rec;
  uint2* dst = (uint2*)rec_out;
  for (int k = 0; k < U / 2; ++k) dst[i * (U / 2) + k] = src[r * (U / 2) + k];
  if (gh) gh_out[i] = gh[r];
  if (g32) g32_out[i] = g32[r];
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

// Timing pass only: one wave that waits `ticks` of the constant-rate wall clock (a
// second bound, 2^20 sleeps of ~3 us, ends it whatever the clock reads), so that the
// host has enqueued the whole kernel sequence behind it before the device starts it.
__global__ void k_hold(uint64_t ticks) {
  const uint64_t t0 = wall_clock64();
  for (uint32_t i = 0; i < (1u << 20) && wall_clock64() - t0 < ticks; ++i)
    __builtin_amdgcn_s_sleep(127);
}

// ===========================================================================
// launchers
// ===========================================================================
void launch_pack_records(const uint8_t* bins, int64_t n, int32_t F, int32_t fmt, uint4* rec,
                         hipStream_t s) {
  const int64_t blocks = (n + 255) / 256;
  k_pack_records<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(bins, n, F, fmt, rec);
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
void launch_grad_softmax(const double* score, const float* label, float* g, float* h, int64_t n,
                         int32_t K, double factor, hipStream_t s) {
  const int64_t blocks = std::min<int64_t>(std::max<int64_t>((n + 255) / 256, 1), 4096);
  const dim3 gr((unsigned)blocks), b(256);
  switch (K) {
#define SOFTMAX_K(k) \
  case k:            \
    k_grad_softmax<k><<<gr, b, 0, s>>>(score, label, g, h, n, K, factor); \
    break;
    SOFTMAX_K(2) SOFTMAX_K(3) SOFTMAX_K(4) SOFTMAX_K(5) SOFTMAX_K(6) SOFTMAX_K(7) SOFTMAX_K(8)
    SOFTMAX_K(9) SOFTMAX_K(10) SOFTMAX_K(11) SOFTMAX_K(12) SOFTMAX_K(13) SOFTMAX_K(14)
    SOFTMAX_K(15) SOFTMAX_K(16)
#undef SOFTMAX_K
    default:
      k_grad_softmax<0><<<gr, b, 0, s>>>(score, label, g, h, n, K, factor);
  }
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
void launch_requant(const float* g, const float* h, int64_t n, const Ctl* ctl, int32_t bins,
                    uint16_t* gh, unsigned long long* bad, hipStream_t s) {
  const int64_t blocks = (n + 255) / 256;
  if (blocks < 1) return;
  k_requant<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(g, h, n, ctl, bins, gh, bad);
}
void launch_hist(const DevLearner& L, hipStream_t s, const KernelEvents* ev) {
  const dim3 g(HIST_GRID_Q + SPEC_MAX), blk(HIST_THREADS);
  if (L.total_cells <= HIST_WAVE_CELLS) {
    const size_t lds = (size_t)HIST_WAVES * (L.total_cells + LDS_TRASH_CELLS) * sizeof(uint32_t);
    DISPATCH_FMT(L.fmt, KLAUNCH(ev, (k_hist_jobs<kF, true>), g, blk, lds, s, L));
  } else {
    const size_t lds = (size_t)(L.total_cells + LDS_TRASH_CELLS) * sizeof(unsigned long long);
    DISPATCH_FMT(L.fmt, KLAUNCH(ev, (k_hist_jobs<kF, false>), g, blk, lds, s, L));
  }
}
void launch_hist_f32(const DevLearner& L, hipStream_t s, const KernelEvents* ev) {
  const dim3 g(HIST_GRID + SPEC_MAX, (unsigned)std::max(L.n_fgroups, 1)), blk(HIST_THREADS);
  const size_t lds = (size_t)2 * HIST_FP_CELLS * sizeof(unsigned long long);
  DISPATCH_FMT(L.fmt, KLAUNCH(ev, (k_hist_f32<kF>), g, blk, lds, s, L));
}
void launch_exact_prep(const DevLearner& L, const float* dg, const float* dh, int64_t n,
                       hipStream_t s) {
  k_exact_shifts<<<1, 1, 0, s>>>(L.ctl);
  k_pack_g32<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(dg, dh, n, L.bufs.g32[BUF_ORIG]);
}
void launch_fp_prep(const DevLearner& L, const float* g, const float* h, int64_t n,
                    const uint4* partials, hipStream_t s) {
  k_absmax<<<dim3((unsigned)stat_blocks(n)), dim3(256), 0, s>>>(g, h, n, (uint4*)partials);
  k_fp_scales<<<1, 256, 0, s>>>(L.ctl, partials, stat_blocks(n), n);
  k_pack_g32<<<dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s>>>(g, h, n, L.bufs.g32[BUF_ORIG]);
}
int fixscan_prepare() {
  return hipFuncSetAttribute((const void*)k_fixscan, hipFuncAttributeMaxDynamicSharedMemorySize,
                             2 * WIDE_MAX_BIN * (int)sizeof(double)) != hipSuccess;
}
void launch_fixscan(const DevLearner& L, int32_t mode, double* explicit_out, hipStream_t s,
                    const KernelEvents* ev) {
  // quantized: the partial slots summed into hist_sum first (f32 cells are summed by
  // k_fixscan itself); f32 mode never reads hist_sum, so the launch is harmless
  const int64_t cols = (int64_t)L.total_cells * 3;
  if (!rec_wide(L.fmt))
    k_hist_reduce<<<dim3((unsigned)((cols + 15) / 16)), dim3(256), 0, s>>>(L);
  KLAUNCH(ev, k_fixscan, dim3((unsigned)L.F), dim3(SCAN_THREADS),
          (size_t)2 * std::max(L.max_bins, 1) * sizeof(double), s, L, mode, explicit_out);
}
// The wide layout's score update (ScoreUpdater::add_score over the partition,
// score_updater.rs:133-209): its records are row indices, and every committed leaf's
// rows are its range of the row buffer its partition wrote (the leaf ranges
// k_tree_finalize records), so each row gets its leaf's shrunk value from that range
// without walking the tree through the row's binmat bytes.  Block b takes
// LEAF_SCORE_ROWS positions of one leaf, found from the prefix of the leaves' block
// counts; every row belongs to exactly one leaf range, so the adds do not overlap.
#define LEAF_SCORE_ROWS 2048
__global__ __launch_bounds__(256) void k_leaf_score(DevLearner L, double lr,
                                                    double* __restrict__ score) {
  __shared__ int32_t s_leaf, s_blk0;
  const int32_t nl = L.ctl->num_leaves;
  if (nl <= 1) return;
  const int tid = threadIdx.x;
  const int32_t b = (int32_t)blockIdx.x;
  if (tid < LGBM_WAVE) {
    if (tid == 0) s_leaf = -1;
    int32_t run = 0;
    for (int32_t l0 = 0; l0 < nl; l0 += LGBM_WAVE) {
      const int32_t l = l0 + tid;
      const int32_t c = l < nl ? L.leaves.count[l] : 0;
      const int32_t nbk = (c + LEAF_SCORE_ROWS - 1) / LEAF_SCORE_ROWS;
      const int32_t incl = wave_incl_sum_i32(nbk);
      const int32_t ex = run + incl - nbk;
      if (l < nl && b >= ex && b < ex + nbk) {
        s_leaf = l;
        s_blk0 = ex;
      }
      run += readlane_i32(incl, LGBM_WAVE - 1);
    }
  }
  __syncthreads();
  const int32_t l = s_leaf;
  if (l < 0) return;
  const int64_t off = (int64_t)(b - s_blk0) * LEAF_SCORE_ROWS;
  const int64_t cnt = L.leaves.count[l], beg = L.leaves.begin[l];
  const int32_t buf = L.leaves.buf[l];
  const double v = maybe_round_to_zero(L.tree.leaf_value[l] * lr);
  const uint32_t* __restrict__ idx = (const uint32_t*)rec_buf(L.bufs, buf) + beg;
  constexpr int K = LEAF_SCORE_ROWS / 256;
  int64_t row[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int64_t p = off + k * 256 + tid;
    row[k] = p < cnt ? (buf == BUF_ORIG ? beg + p : (int64_t)idx[p]) : -1;
  }
#pragma unroll
  for (int k = 0; k < K; ++k)
    if (row[k] >= 0) score[row[k]] += v;
}

void launch_scan_explicit(const double* hist, const DevFeature* feats, int32_t n_feats,
                          const lgbm_gain_config& cfg, double sg, double sh, int32_t n,
                          lgbm_split_info* out, hipStream_t s) {
  k_scan_explicit<<<dim3((unsigned)n_feats), dim3(LGBM_WAVE), 0, s>>>(hist, feats, n_feats, cfg, sg,
                                                                       sh, n, out);
}
void launch_score_update(const DevLearner& L, double lr, double* score, hipStream_t s,
                         const KernelEvents* ev) {
  int64_t blocks = std::min<int64_t>((L.N + 255) / 256, 2048);
  if (blocks < 1) blocks = 1;
  if (rec_wide(L.fmt)) {
    // leaves' blocks: at most N / LEAF_SCORE_ROWS rounded up, plus one per leaf
    const int64_t lb = (L.N + LEAF_SCORE_ROWS - 1) / LEAF_SCORE_ROWS + MAX_LEAVES;
    KLAUNCH(ev, k_leaf_score, dim3((unsigned)lb), dim3(256), 0, s, L, lr, score);
  } else
    DISPATCH_FMT(L.fmt, KLAUNCH(ev, (k_walk<kF, false>), dim3((unsigned)blocks), dim3(256), 0, s, L,
                                lr, score, (uint8_t*)nullptr));
}
void launch_leaf_of(const DevLearner& L, uint8_t* leaf_of, hipStream_t s) {
  int64_t blocks = std::min<int64_t>((L.N + 255) / 256, 2048);
  if (blocks < 1) blocks = 1;
  if (rec_wide(L.fmt))
    k_walk<REC_FMT_WIDE, true><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(L, 0.0, (double*)nullptr,
                                                                           leaf_of);
  else
    DISPATCH_FMT(L.fmt, (k_walk<kF, true><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
                            L, 0.0, (double*)nullptr, leaf_of)));
}
void launch_gather_rows(int fmt, const uint32_t* rows, int64_t n, const uint4* rec, const uint16_t* gh,
                        const float2* g32, uint4* rec_out, uint16_t* gh_out, float2* g32_out,
                        hipStream_t s) {
  const int64_t blocks = (n + 255) / 256;
  if (blocks < 1) return;
  k_gather_rows<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(rows, n, rec_words(fmt), rec, gh, g32,
                                                              rec_out, gh_out, g32_out);
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

void launch_hold(uint64_t ticks, hipStream_t s) {
  k_hold<<<dim3(1), dim3(64), 0, s>>>(ticks);
}

}  // namespace lgbm
