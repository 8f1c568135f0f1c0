// objective.hip — the L2 regression and LambdaRank objectives on the device.
//
//   k_grad_l2          Objective::Regression::get_gradients (lgbm-objective/src/
//                      regression.rs:427-431): grad = f32(score - f64(label)), hess = 1
//                      (the quantizer's statistics come from k_absmax afterwards)
//   k_grad_lambdarank  Lambdarank::get_gradients -> gradients_for_one_query
//                      (lgbm-objective/src/rank.rs:260-365): one block per query
//
// LambdaRank is order-sensitive twice over: every row's f32 lambda and hessian are
// sums of f32-rounded pair terms, and the normalisation uses the f64 sum of all pair
// terms, both in the reference's loop order (pairs (i, j) of sorted positions,
// i ascending, then j ascending).  The block walks the rows i of that loop in order:
// for row i its threads evaluate the pairs (i, j) in parallel and add each term to
// the j side (row j's document gets one term per row i, so per document the terms
// still arrive in loop order); then one thread adds row i's terms to the i side and
// to the f64 sum in j order.  So every f32 and f64 sum is the reference's sequence
// of operations, and the gradients are bit-identical.  The gain, discount and
// sigmoid tables and the per-query inverse max DCG are built on the host with the
// reference's formulas (host libm exp / log2, as the reference's own tables).
#include "kernels.h"

namespace lgbm {

namespace {

__global__ __launch_bounds__(256) void k_grad_l2(const double* __restrict__ score,
                                                 const float* __restrict__ label,
                                                 float* __restrict__ g, float* __restrict__ h,
                                                 int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride) {
    g[r] = (float)(score[r] - (double)label[r]);
    h[r] = 1.0f;
  }
}

__device__ __forceinline__ double rank_sigmoid(const RankParams& p, const double* __restrict__ tab,
                                               double s) {
  if (s <= p.min_in) return tab[0];
  if (s >= p.max_in) return tab[RANK_SIGMOID_BINS - 1];
  // a NaN score indexes bin 0 (Rust's saturating `as usize`); the index stays inside
  // the table whatever the rounding
  const double x = (s - p.min_in) * p.idx_factor;
  const size_t i = x == x ? (size_t)x : 0;
  return tab[i < (size_t)RANK_SIGMOID_BINS ? i : (size_t)RANK_SIGMOID_BINS - 1];
}

// Rows i of the reference's loop are taken RANK_BATCH (`nbat`) at a time.  A batch's
// pair terms are evaluated in parallel over the columns j: the thread of column j
// walks the batch's rows in order, so row j's document still gets its j-side terms
// in loop order, and stores each pair's i-side terms.  Then lane k of wave 0 folds
// row i0 + k's i side in j order (its document holds exactly the j-side terms of
// the earlier rows by then: later rows never reach back to it), while wave 1 lane
// 0 continues the f64 normalisation sum over the batch's pairs in loop order.  Every
// f32 and f64 sequence is the reference's; the one-lane folds run B at a time.
__global__ __launch_bounds__(LAMBDARANK_THREADS) void k_grad_lambdarank(
    const double* __restrict__ score, const float* __restrict__ label,
    const int32_t* __restrict__ qb, const double* __restrict__ inv_max_dcg,
    const double* __restrict__ tab, const double* __restrict__ discount,
    const double* __restrict__ gain, RankParams p, int32_t nbat, float* __restrict__ g,
    float* __restrict__ h) {
  extern __shared__ double lds[];
  __shared__ double s_best, s_worst, s_nf;
  const int q = (int)blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t st = qb[q], cnt = qb[q + 1] - qb[q];
  if (cnt <= 0) return;
  // LDS: score per position and the batch's pairs' normalisation terms (f64), then
  // label, sorted document, lambda, hessian per position and the batch's pairs'
  // i-side lambda and hessian terms (32-bit); batch rows k at k * cnt
  double* s_sc = lds;
  double* t_nt = s_sc + cnt;
  float* s_lab = (float*)(t_nt + (size_t)nbat * cnt);
  int32_t* s_ord = (int32_t*)(s_lab + cnt);
  float* s_lam = (float*)(s_ord + cnt);
  float* s_hes = s_lam + cnt;
  float* t_lt = s_hes + cnt;
  float* t_ht = t_lt + (size_t)nbat * cnt;
  const double kmin = -__builtin_inf();
  for (int i = tid; i < cnt; i += LAMBDARANK_THREADS) {
    s_sc[i] = score[st + i];
    s_lab[i] = label[st + i];
    s_lam[i] = 0.0f;
    s_hes[i] = 0.0f;
  }
  __syncthreads();
  // stable sort by descending score: the rank of document i among the query's (a
  // NaN score, which the reference's comparison leaves unordered, sorts last so the
  // ranks stay a permutation)
  for (int i = tid; i < cnt; i += LAMBDARANK_THREADS) {
    const double si = s_sc[i];
    const bool ni = si != si;
    int32_t r = 0;
    if (!ni) {
      // before i: higher or equal scores (a NaN compares false); after i: higher
#pragma unroll 4
      for (int j = 0; j < i; ++j) r += s_sc[j] >= si ? 1 : 0;
#pragma unroll 4
      for (int j = i + 1; j < cnt; ++j) r += s_sc[j] > si ? 1 : 0;
    } else {
      for (int j = 0; j < cnt; ++j) {
        const bool nj = s_sc[j] != s_sc[j];
        r += (!nj || j < i) ? 1 : 0;
      }
    }
    s_ord[r] = i;
  }
  __syncthreads();
  if (tid == 0) {
    s_best = s_sc[s_ord[0]];
    int32_t wi = cnt - 1;
    if (wi > 0 && s_sc[s_ord[wi]] == kmin) wi -= 1;
    s_worst = s_sc[s_ord[wi]];
  }
  __syncthreads();
  const double best = s_best, worst = s_worst;
  const double imd = inv_max_dcg[q];
  const bool scale = p.norm && best != worst;
  const int32_t rows = min(cnt - 1, p.trunc);  // rows i < rows (i + 1 < cnt, i < trunc)
  double sum_lambdas = 0.0;  // wave 1 lane 0
  for (int32_t i0 = 0; i0 < rows; i0 += nbat) {
    const int32_t nb = min(nbat, rows - i0);
    for (int32_t j = i0 + 1 + tid; j < cnt; j += LAMBDARANK_THREADS) {
      const int32_t dj = s_ord[j];
      const double sj = s_sc[dj];
      const float lj = s_lab[dj];
      for (int32_t k = 0; k < nb && i0 + k < j; ++k) {
        const int32_t i = i0 + k;
        const int32_t di = s_ord[i];
        const double si = s_sc[di];
        if (si == kmin) continue;  // the reference skips the row (uniform per row)
        const float li = s_lab[di];
        // row i's side of the pair as addends: a pair without a term adds -0.0f to
        // the f32 sums and subtracts +0.0 from the f64 one, which leaves every value
        // (signed zeros included) as skipping it does; x - y is x + (-y) exactly
        float lt = -0.0f, ht = -0.0f;
        double nt = 0.0;
        if (sj != kmin && li != lj) {
          double pl, ph;
          const bool ihigh = li > lj;
          const int32_t hr = ihigh ? i : j, lr = ihigh ? j : i;
          const int32_t hd = ihigh ? di : dj, ld = ihigh ? dj : di;
          const double delta = s_sc[hd] - s_sc[ld];
          // a NaN label indexes gain 0 (Rust's saturating `as usize`); the host checked
          // every other label to be an integer in [0, 31)
          const float lh = s_lab[hd], ll = s_lab[ld];
          const double gap = gain[lh == lh ? (int32_t)lh : 0] - gain[ll == ll ? (int32_t)ll : 0];
          const double paired = fabs(discount[hr] - discount[lr]);
          double dpn = gap * paired * imd;
          if (scale) dpn /= (double)0.01f + fabs(delta);
          pl = rank_sigmoid(p, tab, delta);
          ph = pl * (1.0 - pl);
          pl *= -p.sigmoid * dpn;
          ph *= p.sigmoid * p.sigmoid * dpn;
          // the j side now: row j's document gets one term per row, rows in order
          if (ihigh)
            s_lam[dj] -= (float)pl;
          else
            s_lam[dj] += (float)pl;
          s_hes[dj] += (float)ph;
          lt = ihigh ? (float)pl : -(float)pl;
          ht = (float)ph;
          nt = 2.0 * pl;
        }
        t_lt[(size_t)k * cnt + j] = lt;
        t_ht[(size_t)k * cnt + j] = ht;
        t_nt[(size_t)k * cnt + j] = nt;
      }
    }
    __syncthreads();
    if (tid < nb) {
      // the i side of row i0 + tid, in j order, over branch-free addends
      const int32_t i = i0 + tid;
      const int32_t di = s_ord[i];
      if (s_sc[di] != kmin) {
        const float* lt = t_lt + (size_t)tid * cnt;
        const float* ht = t_ht + (size_t)tid * cnt;
        float lam = s_lam[di], hes = s_hes[di];
#pragma unroll 8
        for (int32_t j = i + 1; j < cnt; ++j) {
          lam += lt[j];
          hes += ht[j];
        }
        s_lam[di] = lam;
        s_hes[di] = hes;
      }
    } else if (tid == LGBM_WAVE) {
      // the normalisation sum over the batch's pairs in loop order
      double sl = sum_lambdas;
      for (int32_t k = 0; k < nb; ++k) {
        const int32_t i = i0 + k;
        if (s_sc[s_ord[i]] == kmin) continue;
        const double* nt = t_nt + (size_t)k * cnt;
#pragma unroll 8
        for (int32_t j = i + 1; j < cnt; ++j) sl -= nt[j];
      }
      sum_lambdas = sl;
    }
    __syncthreads();
  }
  if (tid == LGBM_WAVE) s_nf = (p.norm && sum_lambdas > 0.0) ? log2(1.0 + sum_lambdas) / sum_lambdas : 0.0;
  __syncthreads();
  const double nf = s_nf;
  for (int i = tid; i < cnt; i += LAMBDARANK_THREADS) {
    float lam = s_lam[i], hes = s_hes[i];
    if (nf != 0.0) {
      lam = (float)((double)lam * nf);
      hes = (float)((double)hes * nf);
    }
    g[st + i] = lam;
    h[st + i] = hes;
  }
}

}  // namespace

// Rows of a batch: RANK_BATCH, fewer when the longest query's pair terms would not fit
// the LDS budget (at least one row, whose layout fits RANK_MAX_QUERY).
int32_t rank_batch(int32_t max_query) {
  const size_t per_pos = sizeof(double) + 4 * sizeof(float);  // score, label, order, lambda, hessian
  const size_t per_row = sizeof(double) + 2 * sizeof(float);  // a batch row's pair terms
  const size_t q = (size_t)std::max(max_query, 1);
  int32_t b = RANK_BATCH;
  while (b > 1 && q * (per_pos + per_row * (size_t)b) + 16 > RANK_LDS_BUDGET) --b;
  return b;
}
size_t rank_lds_bytes(int32_t max_query) {
  const size_t q = (size_t)std::max(max_query, 1);
  return q * (24 + 16 * (size_t)rank_batch(max_query)) + 16;
}

// Opts the lambdarank kernel into the LDS of its longest query (above 64 KiB from
// 1639 rows on); outside any graph capture.  0 = ok.
int lambdarank_prepare(int32_t max_query) {
  return hipFuncSetAttribute((const void*)k_grad_lambdarank,
                             hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)rank_lds_bytes(max_query)) == hipSuccess
             ? 0
             : 1;
}

void launch_grad_l2(const double* score, const float* label, float* g, float* h, int64_t n,
                    hipStream_t s) {
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  if (blocks < 1) return;
  k_grad_l2<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(score, label, g, h, n);
}

void launch_grad_lambdarank(const double* score, const float* label, const RankTables& t,
                            float* g, float* h, hipStream_t s) {
  if (t.num_queries <= 0) return;
  k_grad_lambdarank<<<dim3((unsigned)t.num_queries), dim3(LAMBDARANK_THREADS),
                      rank_lds_bytes(t.max_query), s>>>(score, label, t.qb, t.inv_max_dcg, t.table,
                                                        t.discount, t.gain, t.p,
                                                        rank_batch(t.max_query), g, h);
}

}  // namespace lgbm
