// probe.hip — LDS-atomic throughput probe (measurement only, no reference counterpart).
//
// ConstructHistogram's quantized builds add one packed integer cell per (row,
// feature) to an LDS histogram.  This kernel issues the same adds with nothing else
// in the loop, so the time it takes is the LDS-atomic ceiling of a build: blocks of
// 512 threads, two per CU, each thread one row whose F bins sit in registers, F x 64
// cells per histogram (config 1: 28 x 64 = 1792).  Modes vary one thing at a time:
//   pattern  0: lane l adds to bin l of every feature (64 consecutive cells, no two
//               lanes on one address; the u32 form touches 64 distinct banks)
//            1: the row's real bins (the device bins passed in)
//            2: every lane to bin 0 (all 64 lanes on one address)
//   width    u32 cells (the wave-private root scheme) or u64 cells (the partition's
//            and the block-shared scheme's packed cells)
//   scope    one histogram per block, or one per wave
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/lgbm_hip.h"

namespace {

constexpr int kThreads = 512;
constexpr int kMaxF = 32;
constexpr int kBins = 64;

template <bool U64, bool PRIV, int PAT>
__global__ __launch_bounds__(kThreads, 2) void k_probe_lds(const uint8_t* __restrict__ bins,
                                                            int64_t n, int32_t F, int32_t reps,
                                                            unsigned long long* __restrict__ sink) {
  using T = typename std::conditional<U64, unsigned long long, uint32_t>::type;
  extern __shared__ __align__(16) unsigned char probe_lds[];
  T* h = (T*)probe_lds;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cells = F * kBins;
  const int copies = PRIV ? kThreads / 64 : 1;
  for (int c = tid; c < cells * copies; c += kThreads) h[c] = 0;
  T* my = PRIV ? h + (size_t)wave * cells : h;
  const int64_t r = ((int64_t)blockIdx.x * kThreads + tid) % n;
  uint32_t b[kMaxF];
#pragma unroll
  for (int f = 0; f < kMaxF; ++f) {
    uint32_t v = 0;
    if (f < F) {
      if (PAT == 0) v = (uint32_t)lane;
      else if (PAT == 1) v = bins[(int64_t)f * n + r] & (kBins - 1);
      else v = 0;
    }
    b[f] = (uint32_t)(f * kBins) + v;
  }
  __syncthreads();
  // a packed cell value of a (q_g, q_h) pair; the sums are never read back as cells
  const T val = (T)(1u + (2u << 11));
  for (int i = 0; i < reps; ++i) {
#pragma unroll
    for (int f = 0; f < kMaxF; ++f)
      if (f < F) __hip_atomic_fetch_add(&my[b[f]], val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  __syncthreads();
  unsigned long long s = 0;
  for (int c = tid; c < cells * copies; c += kThreads) s += (unsigned long long)h[c];
  if (s) atomicAdd(sink, s);
}

template <bool U64, bool PRIV, int PAT>
hipError_t run(const uint8_t* bins, int64_t n, int32_t F, int32_t reps, int32_t blocks,
               unsigned long long* sink, hipStream_t s) {
  const size_t lds = (size_t)F * kBins * (U64 ? 8 : 4) * (PRIV ? kThreads / 64 : 1);
  hipError_t e = hipFuncSetAttribute((const void*)k_probe_lds<U64, PRIV, PAT>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  k_probe_lds<U64, PRIV, PAT><<<dim3(blocks), dim3(kThreads), lds, s>>>(bins, n, F, reps, sink);
  return hipGetLastError();
}

template <bool U64, bool PRIV>
hipError_t run_pat(int pat, const uint8_t* bins, int64_t n, int32_t F, int32_t reps,
                   int32_t blocks, unsigned long long* sink, hipStream_t s) {
  if (pat == 0) return run<U64, PRIV, 0>(bins, n, F, reps, blocks, sink, s);
  if (pat == 1) return run<U64, PRIV, 1>(bins, n, F, reps, blocks, sink, s);
  return run<U64, PRIV, 2>(bins, n, F, reps, blocks, sink, s);
}

}  // namespace

extern "C" int lgbm_hip_probe_lds_atomics(int device, const uint8_t* bins, int64_t n,
                                          int32_t num_features, int32_t mode, int32_t reps,
                                          double* out) {
  const int pat = mode & 3;
  const bool u64 = (mode & 4) != 0, priv = (mode & 8) != 0;
  if (!out || pat > 2 || num_features < 1 || num_features > kMaxF || reps < 1 ||
      (pat == 1 && (!bins || n < 1)))
    return LGBM_HIP_ERR_INVALID_ARGUMENT;
  if (u64 && priv) return LGBM_HIP_ERR_CAPABILITY;  // 8 x 14 KiB per block: one block per CU
  if (n < 1) n = 1;
  if (hipSetDevice(device) != hipSuccess) return LGBM_HIP_ERR_HIP;
  int cus = 0, clock_khz = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeClockRate, device) != hipSuccess)
    return LGBM_HIP_ERR_HIP;
  const int32_t blocks = 2 * cus;
  unsigned long long* sink = nullptr;
  uint8_t* d_bins = nullptr;
  hipStream_t s = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = LGBM_HIP_OK;
  if (hipMalloc(&sink, 8) != hipSuccess) return LGBM_HIP_ERR_HIP;
  if (pat == 1 && (hipMalloc(&d_bins, (size_t)n * num_features) != hipSuccess ||
                   hipMemcpy(d_bins, bins, (size_t)n * num_features, hipMemcpyHostToDevice) !=
                       hipSuccess)) {
    rc = LGBM_HIP_ERR_HIP;
  } else if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    rc = LGBM_HIP_ERR_HIP;
  } else {
    auto launch = [&](int32_t r) {
      return u64 ? run_pat<true, false>(pat, d_bins, n, num_features, r, blocks, sink, s)
                 : (priv ? run_pat<false, true>(pat, d_bins, n, num_features, r, blocks, sink, s)
                         : run_pat<false, false>(pat, d_bins, n, num_features, r, blocks, sink, s));
    };
    // warm-up, then the timed launch
    if (launch(1) != hipSuccess || hipEventRecord(e0, s) != hipSuccess ||
        launch(reps) != hipSuccess || hipEventRecord(e1, s) != hipSuccess ||
        hipEventSynchronize(e1) != hipSuccess) {
      rc = LGBM_HIP_ERR_HIP;
    } else {
      float ms = 0.0f;
      (void)hipEventElapsedTime(&ms, e0, e1);
      const double adds = (double)blocks * kThreads * (double)reps * num_features;
      out[0] = ms;
      out[1] = adds;
      out[2] = adds / ((double)ms * 1e-3 * (double)clock_khz * 1e3 * (double)cus);
      out[3] = clock_khz * 1e-3;
      out[4] = cus;
    }
  }
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (s) (void)hipStreamDestroy(s);
  if (d_bins) (void)hipFree(d_bins);
  (void)hipFree(sink);
  return rc;
}
