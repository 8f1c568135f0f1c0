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
  return tab[(size_t)((s - p.min_in) * p.idx_factor)];
}

__global__ __launch_bounds__(LAMBDARANK_THREADS) void k_grad_lambdarank(
    const double* __restrict__ score, const float* __restrict__ label,
    const int32_t* __restrict__ qb, const double* __restrict__ inv_max_dcg,
    const double* __restrict__ tab, const double* __restrict__ discount,
    const double* __restrict__ gain, RankParams p, float* __restrict__ g, float* __restrict__ h) {
  extern __shared__ double lds[];
  __shared__ double s_best, s_worst;
  const int q = (int)blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t st = qb[q], cnt = qb[q + 1] - qb[q];
  if (cnt <= 0) return;
  // LDS: score and row i's pair j's normalisation term (f64) per position; label,
  // sorted document, lambda, hessian, row i's pair j's lambda and hessian terms
  // (32-bit) per position
  double* s_sc = lds;
  double* s_nt = s_sc + cnt;
  float* s_lab = (float*)(s_nt + cnt);
  int32_t* s_ord = (int32_t*)(s_lab + cnt);
  float* s_lam = (float*)(s_ord + cnt);
  float* s_hes = s_lam + cnt;
  float* s_lt = s_hes + cnt;
  float* s_ht = s_lt + cnt;
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
    for (int j = 0; j < cnt; ++j) {
      const double sj = s_sc[j];
      const bool nj = sj != sj;
      const bool before = (ni || nj) ? (ni && (!nj || j < i)) : (sj > si || (sj == si && j < i));
      r += before ? 1 : 0;
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
  double sum_lambdas = 0.0;  // thread 0
  for (int32_t i = 0; i + 1 < cnt && i < p.trunc; ++i) {
    const int32_t di = s_ord[i];
    const double si = s_sc[di];
    if (si == kmin) continue;  // block-uniform
    const float li = s_lab[di];
    for (int32_t j = i + 1 + tid; j < cnt; j += LAMBDARANK_THREADS) {
      const int32_t dj = s_ord[j];
      const double sj = s_sc[dj];
      const float lj = s_lab[dj];
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
        // the j side now: row j's document gets one term per row
        if (ihigh)
          s_lam[dj] -= (float)pl;
        else
          s_lam[dj] += (float)pl;
        s_hes[dj] += (float)ph;
        lt = ihigh ? (float)pl : -(float)pl;
        ht = (float)ph;
        nt = 2.0 * pl;
      }
      s_lt[j] = lt;
      s_ht[j] = ht;
      s_nt[j] = nt;
    }
    __syncthreads();
    if (tid == 0) {
      // the i side and the normalisation sum, in j order: three independent chains
      // over branch-free addends, so the LDS reads run ahead of the adds
      float lam = s_lam[di], hes = s_hes[di];
      double sl = sum_lambdas;
#pragma unroll 8
      for (int32_t j = i + 1; j < cnt; ++j) {
        lam += s_lt[j];
        hes += s_ht[j];
        sl -= s_nt[j];
      }
      sum_lambdas = sl;
      s_lam[di] = lam;
      s_hes[di] = hes;
    }
    __syncthreads();
  }
  __shared__ double s_nf;
  if (tid == 0) s_nf = (p.norm && sum_lambdas > 0.0) ? log2(1.0 + sum_lambdas) / sum_lambdas : 0.0;
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

size_t rank_lds_bytes(int32_t max_query) {
  return (size_t)max_query * (2 * sizeof(double) + 6 * 4) + 16;
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
                                                        t.discount, t.gain, t.p, g, h);
}

}  // namespace lgbm
