// bin.hip — raw feature values -> resident bin records on the device.
//
// ValueToBin (crates/lgbm-dataset/src/bin_mapper.rs:148-189) for every value of a
// dense matrix, fused with the record packing of k_pack_records: one thread per
// row, the row's bins packed into its 16W-byte record with the row index in the
// last word.  Numerical features search their upper bounds (staged in LDS) for the
// reference's bisection result (the first bin whose bound is >= v); categorical
// features look their integer category up in a sorted (category, bin) table.
// HBM-bound: 4 or 8 bytes read and one byte written per value, plus the 4-byte row
// index per record.
#include "kernels.h"

namespace lgbm {

namespace {

constexpr int32_t BIN_LDS_BOUNDS = 7168;  // 56 KiB of staged upper bounds

__device__ __forceinline__ int32_t sat_i32(double x) {
  if (!(x == x)) return 0;
  if (x >= 2147483647.0) return 2147483647;
  if (x <= -2147483648.0) return (-2147483647 - 1);
  return (int32_t)x;
}

template <int TOP = 128>  // the largest binary-lifting step: num_bin <= 2 * TOP
__device__ __forceinline__ uint32_t bin_of(const DevBinFeature& f, const double* ub,
                                           const int2* __restrict__ cats, double v) {
  if (v != v) {
    if (f.categorical) return 0u;
    if (f.nan_bin >= 0) return (uint32_t)f.nan_bin;
    v = 0.0;
  }
  if (!f.categorical) {
    // The reference's bisection returns the first b in [0, last] with v <= ub[b]
    // (or last); over non-decreasing bounds that is the number of ub[0..last-1]
    // below v.  Counted here by binary lifting with eight fixed steps: every lane
    // of every feature runs the same trip count, the first probe is one broadcast
    // LDS address, and the unrolled searches of neighbouring features overlap.
    const double* u = ub + f.off;
    int32_t pos = 0;
#pragma unroll
    for (int32_t step = TOP; step > 0; step >>= 1)
      if (pos + step <= f.last && u[pos + step - 1] < v) pos += step;
    return (uint32_t)pos;
  }
  const int32_t key = sat_i32(v);
  if (key < 0) return 0u;
  const int2* c = cats + f.off;
  int32_t lo = 0, hi = f.ncat;
  while (lo < hi) {
    const int32_t m = (lo + hi) >> 1;
    if (c[m].x < key)
      lo = m + 1;
    else
      hi = m;
  }
  return (lo < f.ncat && c[lo].x == key) ? (uint32_t)c[lo].y : 0u;
}

template <typename T, bool COL_MAJOR>
__global__ __launch_bounds__(256) void k_bin_records(const T* __restrict__ x, int64_t n, int32_t F,
                                                     int32_t fmt, const DevBinFeature* __restrict__ feats,
                                                     const double* __restrict__ ub, int32_t ub_count,
                                                     const int2* __restrict__ cats,
                                                     uint4* __restrict__ rec) {
  extern __shared__ double s_ub[];
  __shared__ DevBinFeature s_f[16 * LGBM_MAX_W];
  // bounds beyond the LDS budget are read through the caches instead
  const bool staged = ub_count <= BIN_LDS_BOUNDS;
  if (staged)
    for (int i = threadIdx.x; i < ub_count; i += blockDim.x) s_ub[i] = ub[i];
  const double* bounds = staged ? s_ub : ub;
  for (int i = threadIdx.x; i < F; i += blockDim.x) s_f[i] = feats[i];
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  // record format (lgbm_device.h): bins per u32 and their width; the legacy format's
  // last u32 holds the row index, the packed one's stays clear (its quantized pair
  // is written by the partition)
  const int U = rec_words(fmt), bpw = rec_bpw(fmt), bb = rec_bits(fmt);
  const bool packed = rec_packed(fmt);
  uint2* out = (uint2*)rec;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride) {
    // two record words at a time, built in registers
    for (int w2 = 0; w2 < U / 2; ++w2) {
      uint32_t q[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int wi = 2 * w2 + k;
        uint32_t word = 0u;
        for (int j = 0; j < bpw; ++j) {
          const int f = bpw * wi + j;
          if (f < F) {
            const double v = (double)(COL_MAJOR ? x[(int64_t)f * n + r] : x[r * F + f]);
            word |= bin_of(s_f[f], bounds, cats, v) << (bb * j);
          }
        }
        q[k] = word;
      }
      if (!packed && w2 == U / 2 - 1) q[1] = (uint32_t)r;
      out[r * (U / 2) + w2] = make_uint2(q[0], q[1]);
    }
  }
}

// The wide layout: block (row chunk, 16-feature word); the word's bounds staged in
// LDS (16 features x at most 256 bins), one thread per row writes the word's 16 bytes
// of the row's binmat row (padding features 0).  Feature group 0 also writes the
// identity row-index records.
constexpr int32_t BIN_WIDE_F = 16;
template <typename T, bool COL_MAJOR>
__global__ __launch_bounds__(256) void k_bin_wide(const T* __restrict__ x, int64_t n, int32_t F,
                                                  int64_t stride,
                                                  const DevBinFeature* __restrict__ feats,
                                                  const double* __restrict__ ub,
                                                  const int2* __restrict__ cats,
                                                  uint8_t* __restrict__ binmat,
                                                  uint32_t* __restrict__ rec) {
  __shared__ double s_ub[BIN_WIDE_F * 256];
  __shared__ DevBinFeature s_f[BIN_WIDE_F];
  __shared__ int32_t s_lo, s_hi;
  const int f0 = (int)blockIdx.y * BIN_WIDE_F;
  const int nf = min(BIN_WIDE_F, F - f0);
  if (threadIdx.x < (unsigned)nf) s_f[threadIdx.x] = feats[f0 + threadIdx.x];
  __syncthreads();
  if (threadIdx.x == 0) {
    // the word's entries of the bounds array: from its first feature's to the next
    // word's first feature's (every feature holds num_bin entries)
    int32_t lo = nf > 0 ? s_f[0].ub_pos : 0, hi = lo;
    for (int k = 0; k < nf; ++k) {
      const DevBinFeature& f = s_f[k];
      const int32_t end = f.categorical ? f.ub_pos : f.off + f.last + 1;
      hi = max(hi, end);
    }
    s_lo = lo;
    s_hi = hi;
  }
  __syncthreads();
  const int32_t lo = s_lo, cnt = s_hi - s_lo;
  for (int i = threadIdx.x; i < cnt; i += blockDim.x) s_ub[i] = ub[lo + i];
  if (threadIdx.x < (unsigned)nf && !s_f[threadIdx.x].categorical) s_f[threadIdx.x].off -= lo;
  __syncthreads();
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += step) {
    uint32_t v[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < BIN_WIDE_F; ++k) {
      if (k < nf) {
        const int f = f0 + k;
        const double val = (double)(COL_MAJOR ? x[(int64_t)f * n + r] : x[r * F + f]);
        v[k >> 2] |= bin_of(s_f[k], s_ub, cats, val) << (8 * (k & 3));
      }
    }
    *(uint4*)(binmat + r * stride + f0) = make_uint4(v[0], v[1], v[2], v[3]);
    if (blockIdx.y == 0) rec[r] = (uint32_t)r;
  }
}

// 2-byte bins (a feature of more than 256 bins): block (row chunk, 8-feature word),
// bounds read through the caches (a word's can exceed LDS), 12 lifting steps.
template <typename T, bool COL_MAJOR>
__global__ __launch_bounds__(256) void k_bin_wide16(const T* __restrict__ x, int64_t n, int32_t F,
                                                    int64_t stride,
                                                    const DevBinFeature* __restrict__ feats,
                                                    const double* __restrict__ ub,
                                                    const int2* __restrict__ cats,
                                                    uint8_t* __restrict__ binmat,
                                                    uint32_t* __restrict__ rec) {
  __shared__ DevBinFeature s_f[8];
  const int f0 = (int)blockIdx.y * 8;
  const int nf = min(8, F - f0);
  if (threadIdx.x < (unsigned)max(nf, 0)) s_f[threadIdx.x] = feats[f0 + threadIdx.x];
  __syncthreads();
  const int64_t step = (int64_t)gridDim.x * blockDim.x;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += step) {
    uint32_t v[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k < nf) {
        const int f = f0 + k;
        const double val = (double)(COL_MAJOR ? x[(int64_t)f * n + r] : x[r * F + f]);
        v[k >> 1] |= bin_of<WIDE_MAX_BIN / 2>(s_f[k], ub, cats, val) << (16 * (k & 1));
      }
    }
    *(uint4*)(binmat + r * stride + 2 * f0) = make_uint4(v[0], v[1], v[2], v[3]);
    if (blockIdx.y == 0) rec[r] = (uint32_t)r;
  }
}

template <typename T, bool CM>
void launch_wide_typed(const void* x, int64_t n, int32_t F, int64_t stride, const DevBinFeature* feats,
                       const double* ub, const int2* cats, uint8_t* binmat, uint4* rec, int bin16,
                       hipStream_t s, const KernelEvents* ev) {
  const int64_t want = (n + 255) / 256;
  const unsigned blocks = (unsigned)std::min<int64_t>(std::max<int64_t>(want, 1), 1024);
  // every 16-byte word of a row, the padding words too (zeros)
  const unsigned words = (unsigned)(stride / 16);  // 16-byte words of a row
  if (bin16)
    KLAUNCH(ev, (k_bin_wide16<T, CM>), dim3(blocks, words), dim3(256), 0, s, (const T*)x, n, F,
            stride, feats, ub, cats, binmat, (uint32_t*)rec);
  else
    KLAUNCH(ev, (k_bin_wide<T, CM>), dim3(blocks, words), dim3(256), 0, s, (const T*)x, n, F,
            stride, feats, ub, cats, binmat, (uint32_t*)rec);
}

template <typename T, bool CM>
void launch_typed(const void* x, int64_t n, int32_t F, int32_t fmt, const DevBinFeature* feats,
                  const double* ub, int32_t ub_count, const int2* cats, uint4* rec, hipStream_t s,
                  const KernelEvents* ev) {
  const int64_t want = (n + 255) / 256;
  const unsigned blocks = (unsigned)std::min<int64_t>(std::max<int64_t>(want, 1), 4096);
  const size_t lds = ub_count <= BIN_LDS_BOUNDS ? (size_t)ub_count * sizeof(double) : 0;
  KLAUNCH(ev, (k_bin_records<T, CM>), dim3(blocks), dim3(256), lds, s, (const T*)x, n, F, fmt,
          feats, ub, ub_count, cats, rec);
}

}  // namespace

void launch_bin_wide(const void* x, int32_t f64, int32_t col_major, int64_t n, int32_t F,
                     int64_t stride, const DevBinFeature* feats, const double* ub,
                     const int2* cats, uint8_t* binmat, uint4* rec, int32_t bin16, hipStream_t s,
                     const KernelEvents* ev) {
  if (n <= 0) return;
  if (f64) {
    if (col_major)
      launch_wide_typed<double, true>(x, n, F, stride, feats, ub, cats, binmat, rec, bin16, s, ev);
    else
      launch_wide_typed<double, false>(x, n, F, stride, feats, ub, cats, binmat, rec, bin16, s, ev);
  } else {
    if (col_major)
      launch_wide_typed<float, true>(x, n, F, stride, feats, ub, cats, binmat, rec, bin16, s, ev);
    else
      launch_wide_typed<float, false>(x, n, F, stride, feats, ub, cats, binmat, rec, bin16, s, ev);
  }
}

void launch_bin_records(const void* x, int32_t f64, int32_t col_major, int64_t n, int32_t F,
                        int32_t fmt, const DevBinFeature* feats, const double* ub, int32_t ub_count,
                        const int2* cats, uint4* rec, hipStream_t s, const KernelEvents* ev) {
  if (n <= 0) return;
  if (f64) {
    if (col_major)
      launch_typed<double, true>(x, n, F, fmt, feats, ub, ub_count, cats, rec, s, ev);
    else
      launch_typed<double, false>(x, n, F, fmt, feats, ub, ub_count, cats, rec, s, ev);
  } else {
    if (col_major)
      launch_typed<float, true>(x, n, F, fmt, feats, ub, ub_count, cats, rec, s, ev);
    else
      launch_typed<float, false>(x, n, F, fmt, feats, ub, ub_count, cats, rec, s, ev);
  }
}

}  // namespace lgbm
