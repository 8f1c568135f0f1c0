// wide.hip — the wide row layout (REC_FMT_WIDE) for hundreds to thousands of features.
//
// The record layouts move every row's bins at every split, 2 F bytes per row and
// level; at F = 700 or 2000 that traffic dwarfs the histogram reads.  Here the bins
// stay in one row-major matrix binmat[N][Fp] (u8, Fp = F rounded up to WIDE_GF_Q,
// padding bytes 0) that is never moved; the partition moves the 4-byte row index and
// the row's gradient pair, and routes by one byte gathered from binmat.
//
// ConstructHistogram (build_histograms_into, crates/lgbm-compute/src/lib.rs:262-390:
// per feature, the leaf's rows folded into their bins) cannot hold a leaf's cells in
// LDS at this width (F x num_bin, up to 512k cells), so a block owns one group of
// consecutive features (WIDE_GF_Q = 64 with quantized pairs in packed 8-byte cells,
// WIDE_GF_F = 32 with 64-bit fixed-point (g, h) cells: 128 KiB of LDS either way)
// and a contiguous chunk of one job's rows.  Each thread takes a row at a time: its
// index, its pair, and the group's bytes of its binmat row in 16-byte loads; then one
// LDS atomic per (row, feature).  The block stores its group's cells, as they are in
// LDS, into its chunk's partial slot (plain stores; the launch's chunk a owns slot a);
// the reader (k_fixscan for the root, k_pair_scan for the children) sums the job's
// chunks (HistJob a0 / nblk).
//
// The most frequent bin of a feature is never accumulated.  The scans never read
// that cell's own sum: FixHistogram (fix_histogram.rs:50-80) overwrites it with the
// leaf sum minus the other bins when most_freq_bin > 0, and compaction drops bin 0
// when most_freq_bin == 0 (offset 1, lgbm-treelearner/src/lib.rs:89-95).  Every
// node's integer cell at that bin is then 0 (0 - 0 in the subtraction), and the f64
// cells the scans see are the reference's.  Sparse columns (most rows in one bin)
// thus cost one byte read per row but almost no atomics.  The root's sums, which
// the record layouts take from any feature's cells, come from a totals cell (index
// total_cells of the accumulator) that feature group 0's blocks fill for the root job.
#include "scan.h"

namespace lgbm {

namespace {

// Rows per chunk R and the first chunk of every job: jobs get ceil(count / R) chunks,
// R = the launch's rows / `chunks` (at least WIDE_MIN_ROWS); the host sizes `chunks`
// so that R <= WIDE_MAX_ROWS, and launches chunks + SPEC_MAX blocks per group.
// Wave 0, lane j = job j (nj <= SPEC_MAX): the counts load in parallel.
__device__ __forceinline__ void wide_assign(const Ctl* ctl, int32_t nj, int32_t* s_a0,
                                            int32_t* s_nb, int64_t* s_R, int64_t chunks,
                                            int64_t groups, int64_t min_small, int lane) {
  const int64_t c = lane < nj ? max(ctl->hjobs[lane].count, (int64_t)0) : 0;
  int64_t S = c;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) S += __shfl_xor(S, off);
  int64_t R = (S + chunks - 1) / chunks;
  // at least WIDE_MIN_ROWS rows a chunk (a chunk's flush costs its group's cells),
  // fewer down to `min_small` when the round is too small to give every CU a block
  // (about WIDE_FILL blocks over the groups)
  const int64_t rmin = min((int64_t)WIDE_MIN_ROWS, max(min_small, S * groups / WIDE_FILL));
  if (R < rmin) R = rmin;
  const int32_t nb = c > 0 ? (int32_t)((c + R - 1) / R) : 0;
  const int32_t incl = wave_incl_sum_i32(nb);
  if (lane < nj) {
    s_a0[lane] = incl - nb;
    s_nb[lane] = nb;
  }
  if (lane == 0) *s_R = R;
}

template <int FP, bool B16>
__global__ __launch_bounds__(WIDE_THREADS) void k_hist_wide(DevLearner L) {
  // B16: 2-byte bins, feature groups from the host's table (cells <= WIDE16_GROUP_CELLS)
  constexpr int GF = B16 ? WIDE16_GROUP_F : FP ? WIDE_GF_F : WIDE_GF_Q;
  constexpr int NV = GF / 16;      // 16-byte words of a row's group bytes
  constexpr int RU = FP ? 4 : 2;   // rows per thread in flight
  constexpr int NW = WIDE_THREADS / LGBM_WAVE;
  extern __shared__ unsigned long long lds[];
  __shared__ uint32_t s_fd[GF];    // per feature: (first cell - group base) << 8 | mfb
                                   // (2-byte bins: << 16)
  __shared__ int32_t s_a0[SPEC_MAX], s_nb[SPEC_MAX];
  __shared__ int64_t s_R;
  __shared__ long long s_tot[3][NW];
  Ctl* ctl = L.ctl;
  const int32_t nj = ctl->n_hjobs;
  if (nj <= 0) return;
  const int tid = threadIdx.x, wave = tid >> 6;
  const int F = L.F, cells = L.total_cells;
  // grid (feature group, row chunk): chunk-major launch order, so the chunks a round
  // uses (the first ones of every group) start before the idle tail
  const int grp = (int)blockIdx.x;
  const int f0 = B16 ? L.wgroups[grp] : grp * GF;
  if (f0 >= F) return;
  if (wave == 0) wide_assign(ctl, nj, s_a0, s_nb, &s_R, (int64_t)gridDim.y - SPEC_MAX,
                              (int64_t)gridDim.x,
                              (int64_t)(FP ? WIDE_MIN_ROWS_SMALL_F : WIDE_MIN_ROWS_SMALL_Q),
                              (int)lane_id());
  __syncthreads();
  const int32_t a = (int32_t)blockIdx.y;
  int32_t j = -1;
  for (int k = 0; k < nj; ++k)
    if (a >= s_a0[k] && a < s_a0[k] + s_nb[k]) j = k;
  if (tid == 0 && blockIdx.x == 0 && blockIdx.y == 0)
    for (int k = 0; k < nj; ++k) {  // the readers' chunk ranges
      ctl->hjobs[k].a0 = s_a0[k];
      ctl->hjobs[k].nblk = s_nb[k];
    }
  if (j < 0) return;
  const int f1 = B16 ? L.wgroups[grp + 1] : min(f0 + GF, F);
  const int gbase = (int)L.feats[f0].cell_base;
  const int gcells = (f1 < F ? (int)L.feats[f1].cell_base : cells) - gbase;
  for (int k = tid; k < GF; k += WIDE_THREADS) {
    uint32_t d = 0u;  // padding bytes: bin 0 == "mfb" 0, never added
    if (f0 + k < f1) {
      const DevFeature& ft = L.feats[f0 + k];
      d = B16 ? ((ft.cell_base - (uint32_t)gbase) << 16) | (ft.mfb & 0xffffu)
              : ((ft.cell_base - (uint32_t)gbase) << 8) | (ft.mfb & 0xffu);
    }
    s_fd[k] = d;
  }
  for (int c = tid; c < gcells * (FP ? 2 : 1); c += WIDE_THREADS) lds[c] = 0ull;
  __syncthreads();

  const HistJob& J = ctl->hjobs[j];
  const int64_t R = s_R;
  const int64_t lo = (int64_t)(a - s_a0[j]) * R;
  const int64_t hi = min(J.count, lo + R);
  const int64_t jb = J.begin;
  const bool orig = J.buf == BUF_ORIG;
  const uint32_t* __restrict__ rows = (const uint32_t*)rec_buf(L.bufs, J.buf) + jb;
  const uint8_t* __restrict__ bm = L.binmat + (B16 ? 2 : 1) * f0;
  const int nfeat = f1 - f0;
  const int64_t stride = L.row_stride;
  const bool totals = (J._pad & 1) != 0 && grp == 0;
  const uint16_t* __restrict__ ghq = L.bufs.gh[0];
  const float2* __restrict__ gh32 = L.bufs.g32[0];
  if constexpr (FP)
    gh32 = buf_sel(L.bufs.g32, J.buf) + jb;
  else
    ghq = buf_sel(L.bufs.gh, J.buf) + jb;
  const double gm = FP ? ldexp(1.0, ctl->g_shift) : 0.0, hm = FP ? ldexp(1.0, ctl->h_shift) : 0.0;
  long long tg = 0, th = 0, t3 = 0;
  if (FP && !B16 && orig && L.bincol) {
    // f32 root build: rows in their original order, so each feature's bytes of a
    // wave's rows are 64 consecutive bytes of the feature-major copy; a group of 32
    // features is half of each row's 64-byte sector of binmat, which every group
    // would fetch whole
    const uint8_t* __restrict__ colbase = L.bincol + (size_t)f0 * (size_t)L.N;
    const size_t cstride = (size_t)L.N;
    for (int64_t b0 = lo; b0 < hi; b0 += (int64_t)WIDE_THREADS) {
      const int64_t r = b0 + tid;
      if (r >= hi) continue;
      const int64_t src_row = jb + r;
      const float2 v = gh32[r];
      const long long gi = (long long)rint((double)v.x * gm);
      const long long hi_ = (long long)rint((double)v.y * hm);
      tg += gi;
      th += hi_;
      for (int k0 = 0; k0 < GF; k0 += 8) {  // eight features' bytes in flight
        uint32_t bins[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
          bins[k] = k0 + k < nfeat ? colbase[(size_t)(k0 + k) * cstride + src_row] : 0u;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t fd = __builtin_amdgcn_readfirstlane(s_fd[k0 + k]);
          if (bins[k] != (fd & 0xffu)) {
            const int c = (int)(fd >> 8) + (int)bins[k];
            __hip_atomic_fetch_add(&lds[2 * c], (unsigned long long)gi, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_fetch_add(&lds[2 * c + 1], (unsigned long long)hi_, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
          }
        }
      }
    }
  } else if constexpr (!FP && !B16) {
    // Quantized 1-byte bins: a row whose pair quantized to (0, 0) adds nothing (there
    // is no count field), and with 4 quantization bins that is most rows of a ranking
    // objective.  Each wave queues its live rows (source row, pair) in an LDS ring and
    // adds them 64 at a time, so the atomics and the row's binmat bytes are spent on
    // live rows only: LDS atomics cost per instruction more than per active lane.
    constexpr int kRing = 2 * LGBM_WAVE;
    __shared__ uint32_t s_rrow[NW * kRing], s_rq[NW * kRing];
    uint32_t* rrow = s_rrow + wave * kRing;
    uint32_t* rq = s_rq + wave * kRing;
    const int lane = (int)lane_id();
    int staged = 0, consumed = 0;  // wave-uniform
    auto add_batch = [&](int n) {
      __builtin_amdgcn_wave_barrier();  // the ring's stores come first (in-order LDS)
      if (lane < n) {
        const int e = (consumed + lane) & (kRing - 1);
        const uint32_t q = rq[e];
        const int64_t src_row = (int64_t)rrow[e];
        const int32_t qg = (int32_t)(int8_t)(q & 0xffu);
        const int32_t qh = (int32_t)(int8_t)(q >> 8);
        const unsigned long long v = (unsigned long long)(long long)qg +
                                     ((unsigned long long)(uint32_t)qh << 22) +
                                     ((unsigned long long)(qh == 3 ? 1u : 0u) << 43);
        const uint4* src = (const uint4*)(bm + src_row * stride);
        uint4 w4[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) w4[i] = src[i];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const uint32_t word[4] = {w4[i].x, w4[i].y, w4[i].z, w4[i].w};
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            const uint32_t fd = __builtin_amdgcn_readfirstlane(s_fd[16 * i + k]);
            const uint32_t bin = (word[k >> 2] >> (8 * (k & 3))) & 0xffu;
            if (bin != (fd & 0xffu))
              __hip_atomic_fetch_add(&lds[(int)(fd >> 8) + (int)bin], v, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_WORKGROUP);
          }
        }
      }
      __builtin_amdgcn_wave_barrier();  // the ring's loads complete before it is refilled
      consumed += n;
    };
    for (int64_t b0 = lo; b0 < hi; b0 += (int64_t)WIDE_THREADS * RU) {
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const int64_t r = b0 + (int64_t)u * WIDE_THREADS + tid;
        const bool ok = r < hi;
        const uint32_t q = ok ? (uint32_t)ghq[r] : 0u;
        const uint32_t srow = ok ? (orig ? (uint32_t)(jb + r) : rows[r]) : 0u;
        const int32_t qg = (int32_t)(int8_t)(q & 0xffu);
        const int32_t qh = (int32_t)(int8_t)(q >> 8);
        tg += qg;
        th += qh;
        t3 += qh == 3 ? 1 : 0;
        const bool live = q != 0u;
        const unsigned long long m = __ballot(live);
        if (live) {
          const int e = (staged + (int)__popcll(m & lanemask_lt())) & (kRing - 1);
          rrow[e] = srow;
          rq[e] = q;
        }
        staged += (int)__popcll(m);
        if (staged - consumed >= LGBM_WAVE) add_batch(LGBM_WAVE);
      }
    }
    if (staged > consumed) add_batch(staged - consumed);
  } else
  for (int64_t b0 = lo; b0 < hi; b0 += (int64_t)WIDE_THREADS * RU) {
    int64_t row[RU];
    bool ok[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int64_t r = b0 + (int64_t)u * WIDE_THREADS + tid;
      ok[u] = r < hi;
      const int64_t rr = ok[u] ? r : lo;  // in-range stand-in, adds nothing
      row[u] = rr;
    }
    uint4 w[RU][NV];
    const uint16_t* src16[RU];
    unsigned long long va[RU], vb[RU];  // quantized: packed cell add; f32: g, h fixed point
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int64_t src_row = orig ? jb + row[u] : (int64_t)rows[row[u]];
      if constexpr (B16) {
        src16[u] = (const uint16_t*)(bm + src_row * stride);
      } else {
        const uint4* src = (const uint4*)(bm + src_row * stride);
#pragma unroll
        for (int i = 0; i < NV; ++i) w[u][i] = src[i];
      }
      if constexpr (FP) {
        const float2 v = gh32[row[u]];
        const long long gi = (long long)rint((double)v.x * gm);
        const long long hi_ = (long long)rint((double)v.y * hm);
        va[u] = ok[u] ? (unsigned long long)gi : 0ull;
        vb[u] = ok[u] ? (unsigned long long)hi_ : 0ull;
        tg += (long long)va[u];
        th += (long long)vb[u];
      } else {
        const uint32_t q = ok[u] ? (uint32_t)ghq[row[u]] : 0u;
        const int32_t qg = (int32_t)(int8_t)(q & 0xffu);
        const int32_t qh = (int32_t)(int8_t)(q >> 8);
        va[u] = q == 0u ? 0ull
                        : (unsigned long long)(long long)qg + ((unsigned long long)(uint32_t)qh << 22) +
                              ((unsigned long long)(qh == 3 ? 1u : 0u) << 43);
        tg += qg;
        th += qh;
        t3 += qh == 3 ? 1 : 0;
      }
    }
    if constexpr (B16) {
      // one 2-byte load per (row, feature) of the group
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const bool live = FP ? ok[u] : va[u] != 0ull;
        if (!live) continue;
        for (int k = 0; k < nfeat; ++k) {
          const uint32_t d = s_fd[k];
          const uint32_t bin = src16[u][k];
          if (bin != (d & 0xffffu)) {
            const int c = (int)(d >> 16) + (int)bin;
            if constexpr (FP) {
              __hip_atomic_fetch_add(&lds[2 * c], va[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
              __hip_atomic_fetch_add(&lds[2 * c + 1], vb[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            } else {
              __hip_atomic_fetch_add(&lds[c], va[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
          }
        }
      }
    }
    if constexpr (!B16) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        uint32_t fd[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) fd[k] = __builtin_amdgcn_readfirstlane(s_fd[16 * i + k]);
#pragma unroll
        for (int u = 0; u < RU; ++u) {
          const bool live = FP ? ok[u] : va[u] != 0ull;
          if (!live) continue;
          const uint32_t word[4] = {w[u][i].x, w[u][i].y, w[u][i].z, w[u][i].w};
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            const uint32_t bin = (word[k >> 2] >> (8 * (k & 3))) & 0xffu;
            if (bin != (fd[k] & 0xffu)) {
              const int c = (int)(fd[k] >> 8) + (int)bin;
              if constexpr (FP) {
                __hip_atomic_fetch_add(&lds[2 * c], va[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                __hip_atomic_fetch_add(&lds[2 * c + 1], vb[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
              } else {
                __hip_atomic_fetch_add(&lds[c], va[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
              }
            }
          }
        }
      }
    }
  }
  __syncthreads();
  const size_t ac = (size_t)L.acc_cells;
  {
    constexpr int CW = FP ? 2 : 1;  // u64 words per cell
    unsigned long long* dst = L.wide_part + ((size_t)a * cells + gbase) * CW;
    for (int c = tid; c < gcells * CW; c += WIDE_THREADS) dst[c] = lds[c];
  }
  if (totals) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      tg += __shfl_xor(tg, off);
      th += __shfl_xor(th, off);
      t3 += __shfl_xor(t3, off);
    }
    if (lane_id() == 0) {
      s_tot[0][wave] = tg;
      s_tot[1][wave] = th;
      s_tot[2][wave] = t3;
    }
    __syncthreads();
    if (tid == 0) {
      long long G = 0, H = 0, T = 0;
      for (int w = 0; w < NW; ++w) {
        G += s_tot[0][w];
        H += s_tot[1][w];
        T += s_tot[2][w];
      }
      if constexpr (FP) {
        unsigned long long* tc = (unsigned long long*)L.hist_acc64 + ((size_t)j * ac + cells) * 2;
        atomicAdd(&tc[0], (unsigned long long)G);
        atomicAdd(&tc[1], (unsigned long long)H);
      } else {
        int32_t* tc = L.hist_acc + ((size_t)j * ac + cells) * 3;
        atomicAdd(&tc[0], (int32_t)G);
        atomicAdd(&tc[1], (int32_t)H);
        atomicAdd(&tc[2], (int32_t)T);
      }
    }
  }
}

// Feature-major bins -> row-major matrix: thread = (16-feature word, row), rows
// fastest (the byte reads of a wave are contiguous).
__global__ void k_pack_wide(const uint8_t* __restrict__ bins, int64_t n, int32_t F, int64_t stride,
                            uint8_t* __restrict__ binmat, uint32_t* __restrict__ rec) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t words = stride / 16;
  if (i >= n * words) return;
  const int64_t wd = i / n, r = i - wd * n;
  uint32_t v[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int64_t f = wd * 16 + k;
    if (f < F) v[k >> 2] |= (uint32_t)bins[f * n + r] << (8 * (k & 3));
  }
  ((uint4*)(binmat + r * stride))[wd] = make_uint4(v[0], v[1], v[2], v[3]);
  if (wd == 0) rec[r] = (uint32_t)r;
}

// Feature-major 2-byte bins -> the row-major matrix: thread = (8-feature word, row).
__global__ void k_pack_wide16(const uint16_t* __restrict__ bins, int64_t n, int32_t F,
                              int64_t stride, uint8_t* __restrict__ binmat,
                              uint32_t* __restrict__ rec) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t words = stride / 16;
  if (i >= n * words) return;
  const int64_t wd = i / n, r = i - wd * n;
  uint32_t v[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t f = wd * 8 + k;
    if (f < F) v[k >> 1] |= (uint32_t)bins[f * n + r] << (16 * (k & 1));
  }
  ((uint4*)(binmat + r * stride))[wd] = make_uint4(v[0], v[1], v[2], v[3]);
  if (wd == 0) rec[r] = (uint32_t)r;
}

// Row-major matrix -> feature-major copy (the partition's router reads one feature of
// many rows): thread = (16-byte word, row), rows fastest, so each feature's stores
// of a wave are 64 consecutive rows.
__global__ void k_wide_cols(const uint8_t* __restrict__ binmat, int64_t n, int32_t F,
                            int64_t stride, int32_t bin16, uint8_t* __restrict__ bincol) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t words = stride / 16;
  if (i >= n * words) return;
  const int64_t wd = i / n, r = i - wd * n;
  const uint4 v = ((const uint4*)(binmat + r * stride))[wd];
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
  if (bin16) {
    uint16_t* col = (uint16_t*)bincol;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int64_t f = wd * 8 + k;
      if (f < F) col[f * n + r] = (uint16_t)(u[k >> 1] >> (16 * (k & 1)));
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int64_t f = wd * 16 + k;
      if (f < F) bincol[f * n + r] = (uint8_t)(u[k >> 2] >> (8 * (k & 3)));
    }
  }
}

}  // namespace

void launch_wide_cols(const uint8_t* binmat, int64_t n, int32_t F, int64_t stride, int bin16,
                      uint8_t* bincol, hipStream_t s) {
  const int64_t total = n * (stride / 16);
  const int64_t blocks = (total + 255) / 256;
  if (blocks < 1 || !bincol) return;
  k_wide_cols<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(binmat, n, F, stride, bin16, bincol);
}

void launch_pack_wide16(const uint16_t* bins, int64_t n, int32_t F, int64_t stride,
                        uint8_t* binmat, uint4* rec, hipStream_t s) {
  const int64_t total = n * (stride / 16);
  const int64_t blocks = (total + 255) / 256;
  if (blocks < 1) return;
  k_pack_wide16<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(bins, n, F, stride, binmat,
                                                            (uint32_t*)rec);
}

// LDS of a block: its group's cells, 8 bytes each (quantized) or 16 (f32 gradients)
size_t wide_lds_bytes(int fp, bool b16) {
  const size_t cells = b16 ? (size_t)WIDE16_GROUP_CELLS : (size_t)(fp ? WIDE_GF_F : WIDE_GF_Q) * 256;
  return cells * (fp ? 16 : 8);
}

// Feature groups of a launch: fixed 1-byte groups, or the host's 2-byte-bin table.
int wide_groups(int32_t F, int fp, int32_t n_groups16) {
  if (n_groups16 > 0) return n_groups16;
  const int GF = fp ? WIDE_GF_F : WIDE_GF_Q;
  return (F + GF - 1) / GF;
}

// Blocks per feature group of a launch (row chunks + one per job at most): rows per
// chunk stay <= WIDE_MAX_ROWS, and the grid fills the chip.
int64_t wide_grid_x(int ng, int64_t N, int fp) {
  int64_t chunks = std::max<int64_t>((fp ? WIDE_GRID_F : WIDE_GRID_Q) / ng,
                                     (N + WIDE_MAX_ROWS - 1) / WIDE_MAX_ROWS);
  return std::max<int64_t>(chunks, 1) + SPEC_MAX;
}

// u64 words of the partial slots: every chunk of either gradient mode's launch
size_t wide_part_words(int32_t F, int64_t N, int32_t cells, int32_t n_groups16) {
  const int64_t gf = wide_grid_x(wide_groups(F, 1, n_groups16), N, 1);
  const int64_t gq = wide_grid_x(wide_groups(F, 0, n_groups16), N, 0);
  return std::max((size_t)gf * 2, (size_t)gq) * (size_t)cells;
}

// Opt the histogram kernels into their LDS size (outside any graph capture).
int wide_prepare() {
  const void* k[4] = {(const void*)k_hist_wide<0, false>, (const void*)k_hist_wide<1, false>,
                      (const void*)k_hist_wide<0, true>, (const void*)k_hist_wide<1, true>};
  for (int i = 0; i < 4; ++i)
    if (hipFuncSetAttribute(k[i], hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)wide_lds_bytes(i & 1, i >= 2)) != hipSuccess)
      return 1;
  return 0;
}

void launch_hist_wide(const DevLearner& L, int fp, hipStream_t s, const KernelEvents* ev) {
  const int ng = wide_groups(L.F, fp, L.bin16 ? L.n_wgroups : 0);
  const dim3 g((unsigned)ng, (unsigned)wide_grid_x(ng, L.N, fp)), blk(WIDE_THREADS);
  if (L.bin16) {
    if (fp)
      KLAUNCH(ev, (k_hist_wide<1, true>), g, blk, wide_lds_bytes(1, true), s, L);
    else
      KLAUNCH(ev, (k_hist_wide<0, true>), g, blk, wide_lds_bytes(0, true), s, L);
  } else if (fp) {
    KLAUNCH(ev, (k_hist_wide<1, false>), g, blk, wide_lds_bytes(1, false), s, L);
  } else {
    KLAUNCH(ev, (k_hist_wide<0, false>), g, blk, wide_lds_bytes(0, false), s, L);
  }
}

void launch_pack_wide(const uint8_t* bins, int64_t n, int32_t F, int64_t stride, uint8_t* binmat,
                      uint4* rec, hipStream_t s) {
  const int64_t total = n * (stride / 16);
  const int64_t blocks = (total + 255) / 256;
  if (blocks < 1) return;
  k_pack_wide<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(bins, n, F, stride, binmat,
                                                          (uint32_t*)rec);
}

}  // namespace lgbm
