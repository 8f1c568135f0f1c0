// predict.hip — batch prediction of a LightGBM model over dense f32 rows.
//
// One thread per row walks every tree of the requested iteration range on the raw
// feature values (no binning), as the reference predictor does:
//   Tree::get_leaf / numerical_decision / categorical_decision (tree.rs:160-340),
//   GbdtModel::predict_raw (ensemble.rs:75-102): per class an f64 sum over the
//   iterations in order, starting from 0.0 — here class by class, which adds each
//   class's trees in the same order,
//   ConvertOutput (objective.rs:241-340) for the transformed kind.
#include <hip/hip_runtime.h>

#include "kernels.h"
#include "model.h"

namespace lgbm {

struct PredModelDev {
  const PredNode* nodes;
  const PredTree* trees;
  const double* leaves;
  const int32_t* cat_bounds;
  const uint32_t* cat_words;
  const PredLinLeaf* lin_leaves;
  const int32_t* lin_features;
  const double* lin_coeffs;
};

// The node's fields arrive as values: selecting between members of a struct held by
// reference makes the compiler keep the struct in scratch memory.
__device__ __forceinline__ int32_t pred_next(double thr, int32_t dtype, int32_t left,
                                             int32_t right, double fval, const PredModelDev& M,
                                             int32_t cat0) {
  bool go_left;
  if (dtype & 1) {  // CategoricalDecision (tree.rs:212-237)
    go_left = false;
    if (!isnan(fval)) {
      const int32_t iv = fval >= 2147483647.0 ? 2147483647
                         : fval <= -2147483648.0 ? (int32_t)(-2147483647 - 1)
                                                 : (int32_t)fval;  // saturating `as i32`
      if (iv >= 0) {
        const int32_t ci = (int32_t)thr;  // checked at load: 0 <= ci < num_cat
        const int32_t lo = M.cat_bounds[cat0 + ci], hi = M.cat_bounds[cat0 + ci + 1];
        const int32_t w = iv >> 5;
        go_left = w < hi - lo && ((M.cat_words[lo + w] >> (iv & 31)) & 1u) != 0u;
      }
    }
  } else {  // NumericalDecision (tree.rs:193-210)
    const int32_t mt = (dtype >> 2) & 3;
    if (isnan(fval) && mt != 2) fval = 0.0;
    if ((mt == 1 && fval >= -1e-35 && fval <= 1e-35) || (mt == 2 && isnan(fval)))
      go_left = (dtype & 2) != 0;
    else
      go_left = fval <= thr;
  }
  return go_left ? left : right;
}

// Leaf of tree t for the row at x (a path visits fewer than num_leaves nodes: the
// structure was checked at load).
__device__ __forceinline__ int32_t pred_leaf(const PredModelDev& M, int32_t t, const float* x) {
  const PredTree T = M.trees[t];
  if (T.num_leaves <= 1) return 0;
  int32_t node = 0;
  for (int32_t d = 0; d < T.num_leaves && node >= 0; ++d) {
    const PredNode* nd = M.nodes + T.node0 + node;
    const double thr = nd->threshold;
    const int32_t feat = nd->feature, left = nd->left, right = nd->right, dtype = nd->dtype;
    node = pred_next(thr, dtype, left, right, (double)x[feat], M, T.cat0);
  }
  return node < 0 ? ~node : 0;
}

// Tree::predict (tree.rs:279-316): the leaf's value, or for a linear tree the leaf's
// `leaf_const + sum coeff * x[feature]` in term order (f64, no fused multiply-add),
// falling back to the leaf's value when any of its features is NaN.
__device__ __forceinline__ double pred_tree(const PredModelDev& M, int32_t t, const float* x) {
  const int32_t leaf = pred_leaf(M, t, x);
  const PredTree T = M.trees[t];
  const double lv = M.leaves[T.leaf0 + leaf];
  if (T.lin0 < 0) return lv;
  const PredLinLeaf L = M.lin_leaves[T.lin0 + leaf];
  double v = L.c;
  for (int32_t j = 0; j < L.count; ++j) {
    const double xv = (double)x[M.lin_features[L.start + j]];
    if (isnan(xv)) return lv;
    v += M.lin_coeffs[L.start + j] * xv;
  }
  return v;
}

__device__ __forceinline__ double pred_sigmoid(double x, double s) { return 1.0 / (1.0 + exp(-s * x)); }

// Rows of up to this many columns are staged in LDS (256 rows x an odd stride of at
// most 63 floats = 63 KiB): one coalesced load of the block's rows, then every tree
// walk reads its feature values from LDS instead of one cache line per node visit.
constexpr int32_t PRED_STAGE_COLS = 63;

template <bool STAGE>
__global__ __launch_bounds__(256) void k_predict(PredModelDev M, const float* __restrict__ X,
                                                 int64_t rows, int32_t cols, int32_t it0,
                                                 int32_t it1, int32_t ntpi, int32_t kind,
                                                 int32_t objective, double sigmoid,
                                                 int32_t average_output, int32_t es_freq,
                                                 double es_margin, int32_t* __restrict__ es_iters,
                                                 double* __restrict__ out,
                                                 int32_t* __restrict__ leaf_out) {
  extern __shared__ float s_x[];
  const int64_t r0 = (int64_t)blockIdx.x * blockDim.x;
  const int64_t r = r0 + threadIdx.x;
  const float* x;
  if (STAGE) {
    const int32_t stride = cols | 1;  // odd: lanes' rows fall in different banks
    const int32_t total = (int32_t)(min((int64_t)blockDim.x, rows - r0) * cols);
    const float* src = X + r0 * cols;
    for (int32_t i = threadIdx.x; i < total; i += blockDim.x) {
      const int32_t rr = i / cols;
      s_x[rr * stride + (i - rr * cols)] = src[i];
    }
    __syncthreads();
    if (r >= rows) return;
    x = s_x + threadIdx.x * stride;
  } else {
    if (r >= rows) return;
    x = X + r * cols;
  }
  if (kind == 2) {
    const int64_t nt = (int64_t)(it1 - it0) * ntpi;
    for (int32_t i = it0; i < it1; ++i)
      for (int32_t k = 0; k < ntpi; ++k)
        leaf_out[r * nt + (int64_t)(i - it0) * ntpi + k] = pred_leaf(M, i * ntpi + k, x);
    return;
  }
  double* o = out + r * ntpi;
  if (es_freq > 0) {
    // GbdtModel::predict_raw_early_stop (ensemble.rs:120-151): iterations in order,
    // each adding its trees class by class; every es_freq iterations the margin
    // test of pred_early_stop_should_stop (ensemble.rs:337-356) may end the row
    for (int32_t k = 0; k < ntpi; ++k) o[k] = 0.0;
    int32_t counter = 0, evaluated = 0;
    for (int32_t i = it0; i < it1; ++i) {
      for (int32_t k = 0; k < ntpi; ++k) {
        const int32_t t = i * ntpi + k;
        o[k] += pred_tree(M, t, x);
      }
      ++evaluated;
      if (++counter == es_freq) {
        bool stop;
        if (ntpi == 1) {
          stop = 2.0 * fabs(o[0]) > es_margin;
        } else {
          double top1 = -__builtin_inf(), top2 = -__builtin_inf();
          for (int32_t k = 0; k < ntpi; ++k) {
            const double v = o[k];
            if (v > top1) {
              top2 = top1;
              top1 = v;
            } else if (v > top2) {
              top2 = v;
            }
          }
          stop = (top1 - top2) > es_margin;
        }
        if (stop) break;
        counter = 0;
      }
    }
    es_iters[r] = evaluated;
    return;
  }
  for (int32_t k = 0; k < ntpi; ++k) {
    double acc = 0.0;
    for (int32_t i = it0; i < it1; ++i) {
      const int32_t t = i * ntpi + k;
      acc += pred_tree(M, t, x);
    }
    o[k] = acc;
  }
  if (kind != 1) return;
  if (average_output && it1 > it0)  // RF: raw sum / iterations before ConvertOutput
    for (int32_t k = 0; k < ntpi; ++k) o[k] /= (double)(it1 - it0);
  switch (objective) {
    case OBJ_REGRESSION_SQRT: {
      const double v = o[0];
      o[0] = (v > 0.0 ? 1.0 : (v < 0.0 ? -1.0 : 0.0)) * v * v;
      break;
    }
    case OBJ_BINARY:
      o[0] = pred_sigmoid(o[0], sigmoid);
      break;
    case OBJ_XENTROPY:
      o[0] = pred_sigmoid(o[0], 1.0);
      break;
    case OBJ_XENTLAMBDA:
      o[0] = log1p(exp(o[0]));
      break;
    case OBJ_EXP:
      o[0] = exp(o[0]);
      break;
    case OBJ_MULTICLASS: {  // Common::Softmax: max subtraction, sum in class order
      double wmax = o[0];
      for (int32_t k = 1; k < ntpi; ++k) wmax = o[k] > wmax ? o[k] : wmax;
      double wsum = 0.0;
      for (int32_t k = 0; k < ntpi; ++k) {
        o[k] = exp(o[k] - wmax);
        wsum += o[k];
      }
      for (int32_t k = 0; k < ntpi; ++k) o[k] /= wsum;
      break;
    }
    case OBJ_MULTICLASS_OVA:
      for (int32_t k = 0; k < ntpi; ++k) o[k] = pred_sigmoid(o[k], sigmoid);
      break;
    default:
      break;
  }
}

void launch_predict(const PredNode* nodes, const PredTree* trees, const double* leaves,
                    const int32_t* cat_bounds, const uint32_t* cat_words,
                    const PredLinLeaf* lin_leaves, const int32_t* lin_features,
                    const double* lin_coeffs, const float* X, int64_t rows, int32_t cols, int32_t it0, int32_t it1, int32_t ntpi, int32_t kind,
                    int32_t objective, double sigmoid, int32_t average_output, int32_t es_freq,
                    double es_margin, int32_t* es_iters, double* out, int32_t* leaf_out,
                    hipStream_t s, const KernelEvents* ev) {
  if (rows <= 0) return;
  const PredModelDev M{nodes,      trees,        leaves,    cat_bounds,
                       cat_words,  lin_leaves,   lin_features, lin_coeffs};
  const int64_t blocks = (rows + 255) / 256;
  if (cols <= PRED_STAGE_COLS)
    KLAUNCH(ev, k_predict<true>, dim3((unsigned)blocks), dim3(256),
            (size_t)256 * (cols | 1) * sizeof(float), s, M, X, rows, cols, it0, it1, ntpi, kind,
            objective, sigmoid, average_output, es_freq, es_margin, es_iters, out, leaf_out);
  else
    KLAUNCH(ev, k_predict<false>, dim3((unsigned)blocks), dim3(256), 0, s, M, X, rows, cols, it0,
            it1, ntpi, kind, objective, sigmoid, average_output, es_freq, es_margin, es_iters, out,
            leaf_out);
}

}  // namespace lgbm
