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

// ---- feature contributions (TreeSHAP) ------------------------------------------------
// Lundberg et al., arXiv:1706.06060, Algorithm 2, as the reference computes it
// (Tree::predict_contrib / extend_path / unwind_path / unwound_path_sum / tree_shap,
// tree.rs:400-583): one thread per row, the recursion turned into a loop over the hot
// child with a stack of pending cold calls (popped in the recursion's order, so every
// f64 update happens in the same sequence), and every product and quotient in the
// reference's association (this file is built without fused multiply-add).
//
// Each thread's unique paths live in one flat buffer of (D+1)(D+2)/2 elements for the
// deepest tree D, as in the reference: a call's frame starts `d` elements after its
// parent's and copies the parent's first `d` elements; the cold call reads its parent's
// frame after the hot subtree returns, which wrote only past it.  The buffers are
// workspace memory laid out element-major (element k of thread i at k * stride + i), so
// a wave's accesses to one element are contiguous.
struct ShapWork {
  int32_t* feat;
  double* zero;
  double* one;
  double* pw;
  int32_t* s_node;  // pending cold calls: node, parent frame base, depth, split feature
  int32_t* s_base;
  int32_t* s_depth;
  int32_t* s_feat;
  double* s_zero;
  int64_t stride;  // threads of the launch
};

struct ShapModelDev {
  const double* node_cover;
  const double* leaf_cover;
  const double* expected;
};

__device__ __forceinline__ void shap_extend(const ShapWork& W, int64_t i0, int32_t b, int32_t d,
                                            double zf, double of, int32_t feat) {
  const int64_t e = (int64_t)(b + d) * W.stride + i0;
  W.feat[e] = feat;
  W.zero[e] = zf;
  W.one[e] = of;
  W.pw[e] = d == 0 ? 1.0 : 0.0;
  const double dd = (double)d;
  for (int32_t i = d - 1; i >= 0; --i) {
    const int64_t ei = (int64_t)(b + i) * W.stride + i0;
    const double prev = W.pw[ei];
    W.pw[ei + W.stride] += of * prev * ((double)i + 1.0) / (dd + 1.0);
    W.pw[ei] = zf * prev * (dd - (double)i) / (dd + 1.0);
  }
}

__device__ __forceinline__ void shap_unwind(const ShapWork& W, int64_t i0, int32_t b, int32_t d,
                                            int32_t k) {
  const int64_t ek = (int64_t)(b + k) * W.stride + i0;
  const double of = W.one[ek], zf = W.zero[ek];
  double next = W.pw[(int64_t)(b + d) * W.stride + i0];
  const double dd = (double)d;
  for (int32_t i = d - 1; i >= 0; --i) {
    const int64_t ei = (int64_t)(b + i) * W.stride + i0;
    if (of != 0.0) {
      const double tmp = W.pw[ei];
      W.pw[ei] = next * (dd + 1.0) / (((double)i + 1.0) * of);
      next = tmp - W.pw[ei] * zf * (dd - (double)i) / (dd + 1.0);
    } else {
      W.pw[ei] = (W.pw[ei] * (dd + 1.0)) / (zf * (dd - (double)i));
    }
  }
  for (int32_t i = k; i < d; ++i) {
    const int64_t ei = (int64_t)(b + i) * W.stride + i0;
    W.feat[ei] = W.feat[ei + W.stride];
    W.zero[ei] = W.zero[ei + W.stride];
    W.one[ei] = W.one[ei + W.stride];
  }
}

__device__ __forceinline__ double shap_unwound_sum(const ShapWork& W, int64_t i0, int32_t b,
                                                   int32_t d, int32_t k) {
  const int64_t ek = (int64_t)(b + k) * W.stride + i0;
  const double of = W.one[ek], zf = W.zero[ek];
  double next = W.pw[(int64_t)(b + d) * W.stride + i0];
  double total = 0.0;
  const double dd = (double)d;
  for (int32_t i = d - 1; i >= 0; --i) {
    const double pwi = W.pw[(int64_t)(b + i) * W.stride + i0];
    if (of != 0.0) {
      const double tmp = next * (dd + 1.0) / (((double)i + 1.0) * of);
      total += tmp;
      next = pwi - tmp * zf * ((dd - (double)i) / (dd + 1.0));
    } else {
      total += (pwi / zf) / ((dd - (double)i) / (dd + 1.0));
    }
  }
  return total;
}

__global__ __launch_bounds__(256) void k_contrib(PredModelDev M, ShapModelDev S, ShapWork W,
                                                 const float* __restrict__ X, int64_t r0,
                                                 int64_t rows, int32_t cols, int32_t nf,
                                                 int32_t it0, int32_t it1, int32_t ntpi,
                                                 double* __restrict__ out) {
  const int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t r = r0 + i0;
  if (i0 >= W.stride || r >= rows) return;
  const float* x = X + r * cols;
  const int32_t block = nf + 1;
  double* o = out + r * (int64_t)ntpi * block;
  for (int32_t j = 0; j < ntpi * block; ++j) o[j] = 0.0;
  for (int32_t it = it0; it < it1; ++it) {
    for (int32_t k = 0; k < ntpi; ++k) {
      const int32_t t = it * ntpi + k;
      double* phi = o + k * block;
      phi[nf] += S.expected[t];
      const PredTree T = M.trees[t];
      if (T.num_leaves <= 1) continue;
      int32_t node = 0, pb = 0, d = 0, pf = -1, sp = 0;
      double pz = 1.0, po = 1.0;
      for (;;) {
        const int32_t b = pb + d;
        for (int32_t i = 0; i < d; ++i) {
          const int64_t src = (int64_t)(pb + i) * W.stride + i0, dst = (int64_t)(b + i) * W.stride + i0;
          W.feat[dst] = W.feat[src];
          W.zero[dst] = W.zero[src];
          W.one[dst] = W.one[src];
          W.pw[dst] = W.pw[src];
        }
        shap_extend(W, i0, b, d, pz, po, pf);
        if (node < 0) {
          const double lv = M.leaves[T.leaf0 + ~node];
          for (int32_t i = 1; i <= d; ++i) {
            const double w = shap_unwound_sum(W, i0, b, d, i);
            const int64_t ei = (int64_t)(b + i) * W.stride + i0;
            phi[W.feat[ei]] += w * (W.one[ei] - W.zero[ei]) * lv;
          }
          if (sp == 0) break;
          --sp;
          const int64_t es = (int64_t)sp * W.stride + i0;
          node = W.s_node[es];
          pb = W.s_base[es];
          d = W.s_depth[es];
          pf = W.s_feat[es];
          pz = W.s_zero[es];
          po = 0.0;
          continue;
        }
        const PredNode* nd = M.nodes + T.node0 + node;
        const double thr = nd->threshold;
        const int32_t f = nd->feature, left = nd->left, right = nd->right, dtype = nd->dtype;
        const int32_t hot = pred_next(thr, dtype, left, right, (double)x[f], M, T.cat0);
        const int32_t cold = hot == left ? right : left;
        const double w = S.node_cover[T.node0 + node];
        const double hc = hot >= 0 ? S.node_cover[T.node0 + hot] : S.leaf_cover[T.leaf0 + ~hot];
        const double cc = cold >= 0 ? S.node_cover[T.node0 + cold] : S.leaf_cover[T.leaf0 + ~cold];
        const double hz = hc / w, cz = cc / w;
        double iz = 1.0, io = 1.0;
        int32_t pi = 0;
        while (pi <= d && W.feat[(int64_t)(b + pi) * W.stride + i0] != f) ++pi;
        int32_t nd1 = d;
        if (pi != d + 1) {
          const int64_t ep = (int64_t)(b + pi) * W.stride + i0;
          iz = W.zero[ep];
          io = W.one[ep];
          shap_unwind(W, i0, b, d, pi);
          nd1 -= 1;
        }
        const int64_t es = (int64_t)sp * W.stride + i0;
        W.s_node[es] = cold;
        W.s_base[es] = b;
        W.s_depth[es] = nd1 + 1;
        W.s_feat[es] = f;
        W.s_zero[es] = cz * iz;
        ++sp;
        node = hot;
        pb = b;
        d = nd1 + 1;
        pz = hz * iz;
        po = io;
        pf = f;
      }
    }
  }
}

// Path elements and stack entries one thread needs for trees of depth at most `depth`.
int64_t shap_path_elems(int32_t depth) { return (int64_t)(depth + 1) * (depth + 2) / 2; }
int64_t shap_bytes_per_row(int32_t depth) {
  return shap_path_elems(depth) * (4 + 8 + 8 + 8) + (int64_t)(depth + 1) * (4 * 4 + 8);
}

// Runs TreeSHAP for rows [r0, r0 + n) with `ws` holding shap_bytes_per_row(depth) * n
// bytes (n a multiple of 256 or the tail of the rows).
void launch_contrib(const PredNode* nodes, const PredTree* trees, const double* leaves,
                    const int32_t* cat_bounds, const uint32_t* cat_words, const double* node_cover,
                    const double* leaf_cover, const double* expected, const float* X, int64_t r0,
                    int64_t n, int64_t rows, int32_t cols, int32_t nf, int32_t it0, int32_t it1,
                    int32_t ntpi, int32_t depth, void* ws, double* out, hipStream_t s,
                    const KernelEvents* ev) {
  if (n <= 0) return;
  const PredModelDev M{nodes, trees, leaves, cat_bounds, cat_words, nullptr, nullptr, nullptr};
  const ShapModelDev S{node_cover, leaf_cover, expected};
  const int64_t pe = shap_path_elems(depth), se = depth + 1;
  char* p = (char*)ws;
  ShapWork W;
  W.stride = n;
  W.pw = (double*)p;
  p += pe * n * 8;
  W.zero = (double*)p;
  p += pe * n * 8;
  W.one = (double*)p;
  p += pe * n * 8;
  W.s_zero = (double*)p;
  p += se * n * 8;
  W.feat = (int32_t*)p;
  p += pe * n * 4;
  W.s_node = (int32_t*)p;
  p += se * n * 4;
  W.s_base = (int32_t*)p;
  p += se * n * 4;
  W.s_depth = (int32_t*)p;
  p += se * n * 4;
  W.s_feat = (int32_t*)p;
  KLAUNCH(ev, k_contrib, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, M, S, W, X, r0, rows,
          cols, nf, it0, it1, ntpi, out);
}

// ---- sparse rows ------------------------------------------------------------------
// scatter_csr_row + validate_indptr_pair (predict.rs:772-870): one thread per row
// writes its entries in order into its zeroed dense row of `width` (=
// max_feature_idx + 1) floats (a repeated column keeps the last value; columns in
// [width, cols) are dropped).  A row whose indptr pair leaves [0, nnz] or runs backwards sets bit 0
// of *err, a column outside [0, cols) bit 1; the host refuses the call on either.
__global__ __launch_bounds__(256) void k_csr_dense(const int64_t* __restrict__ indptr,
                                                   const int32_t* __restrict__ indices,
                                                   const float* __restrict__ values, int64_t nnz,
                                                   int64_t rows, int32_t cols, int32_t width,
                                                   float* __restrict__ dense,
                                                   uint32_t* __restrict__ err) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float* row = dense + r * width;
  const int64_t lo = indptr[r], hi = indptr[r + 1];
  if (lo < 0 || hi < lo || hi > nnz) {
    atomicOr(err, 1u);
    return;
  }
  for (int64_t k = lo; k < hi; ++k) {
    const int32_t c = indices[k];
    if (c < 0 || c >= cols) {
      atomicOr(err, 2u);
      return;
    }
    if (c < width) row[c] = values[k];
  }
}

// scatter_csc_dense (predict.rs:868-894) over the entries in parallel.  The dense
// rows are zeroed; a repeated row of a column keeps the column's last value; columns
// past `width` are only checked.  Bit 0 of *err: a column's indptr pair leaves
// [0, nnz] or runs backwards; bit 1: a row index outside [0, rows) (the host refuses
// the call on either, so the dense rows are then never read).
//   k_csc_check: one thread per column checks its indptr pair;
//   k_csc_claim: one thread per entry finds its column (the last c with indptr[c] <=
//     k; entries outside every column's range are skipped), checks its row and takes
//     its dense cell with a 32-bit atomic maximum of k + 1, so the last entry wins;
//     the claims live in the dense buffer itself (zeroed first);
//   k_csc_fill: one thread per cell replaces its claim by the claimed value (0: none).
__global__ __launch_bounds__(256) void k_csc_check(const int64_t* __restrict__ indptr,
                                                   int64_t nnz, int32_t cols,
                                                   uint32_t* __restrict__ err) {
  const int32_t c = (int32_t)(blockIdx.x * blockDim.x + threadIdx.x);
  if (c >= cols) return;
  const int64_t lo = indptr[c], hi = indptr[c + 1];
  if (lo < 0 || hi < lo || hi > nnz) atomicOr(err, 1u);
}
__global__ __launch_bounds__(256) void k_csc_claim(const int64_t* __restrict__ indptr,
                                                   const int32_t* __restrict__ indices,
                                                   int64_t nnz, int64_t rows, int32_t cols,
                                                   int32_t width, uint32_t* __restrict__ claim,
                                                   uint32_t* __restrict__ err) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= nnz) return;
  int32_t lo = 0, hi = cols + 1;  // first position in [0, cols] with indptr > k
  while (lo < hi) {
    const int32_t mid = lo + (hi - lo) / 2;
    if (indptr[mid] > k)
      hi = mid;
    else
      lo = mid + 1;
  }
  const int32_t c = lo - 1;
  if (c < 0 || c >= cols || k < indptr[c] || k >= indptr[c + 1]) return;
  const int32_t r = indices[k];
  if (r < 0 || (int64_t)r >= rows) {
    atomicOr(err, 2u);
    return;
  }
  if (c < width) atomicMax(&claim[(int64_t)r * width + c], (uint32_t)(k + 1));
}
__global__ __launch_bounds__(256) void k_csc_fill(const float* __restrict__ values, int64_t cells,
                                                  float* dense) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= cells) return;
  const uint32_t u = ((const uint32_t*)dense)[i];
  dense[i] = u ? values[u - 1] : 0.0f;
}

void launch_csc_dense(const int64_t* indptr, const int32_t* indices, const float* values,
                      int64_t nnz, int64_t rows, int32_t cols, int32_t width, float* dense,
                      uint32_t* err, hipStream_t s) {
  if (cols <= 0) return;
  k_csc_check<<<dim3((unsigned)((cols + 255) / 256)), dim3(256), 0, s>>>(indptr, nnz, cols, err);
  if (nnz > 0)
    k_csc_claim<<<dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, s>>>(
        indptr, indices, nnz, rows, cols, width, (uint32_t*)dense, err);
  const int64_t cells = rows * (int64_t)width;
  if (cells > 0)
    k_csc_fill<<<dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, s>>>(values, cells, dense);
}

void launch_csr_dense(const int64_t* indptr, const int32_t* indices, const float* values,
                      int64_t nnz, int64_t rows, int32_t cols, int32_t width, float* dense,
                      uint32_t* err, hipStream_t s) {
  if (rows <= 0) return;
  k_csr_dense<<<dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s>>>(
      indptr, indices, values, nnz, rows, cols, width, dense, err);
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
