// scan.h — device code shared by the tree-growth kernels: record byte access, the
// packed LDS histogram of quantized pairs, FindBestThreshold for one (leaf, feature)
// by one wave, and the split ordering.
#pragma once

#include "kernels.h"

#include <hip/hip_ext.h>

namespace lgbm {

// One case per record format (lgbm_device.h): kF is the format as a constant.
#define DISPATCH_FMT(FMT, ...)                                              \
  switch (FMT) {                                                            \
    case 1: { constexpr int kF = 1; __VA_ARGS__; } break;                   \
    case 2: { constexpr int kF = 2; __VA_ARGS__; } break;                   \
    case 3: { constexpr int kF = 3; __VA_ARGS__; } break;                   \
    case 4: { constexpr int kF = 4; __VA_ARGS__; } break;                   \
    case 5: { constexpr int kF = 5; __VA_ARGS__; } break;                   \
    case 6: { constexpr int kF = 6; __VA_ARGS__; } break;                   \
    case 7: { constexpr int kF = 7; __VA_ARGS__; } break;                   \
    case 8: { constexpr int kF = 8; __VA_ARGS__; } break;                   \
    case REC_FMT_PACKED + 2: { constexpr int kF = REC_FMT_PACKED + 2; __VA_ARGS__; } break; \
    case REC_FMT_PACKED + 4: { constexpr int kF = REC_FMT_PACKED + 4; __VA_ARGS__; } break; \
    case REC_FMT_PACKED + 6: { constexpr int kF = REC_FMT_PACKED + 6; __VA_ARGS__; } break; \
    case REC_FMT_PACKED + 8: { constexpr int kF = REC_FMT_PACKED + 8; __VA_ARGS__; } break; \
    default: break;                                                         \
  }

// Record r of a buffer into registers / out of registers: u32 words, moved as 16-byte
// words when the record size allows, else 8-byte words.
template <int FMT>
__device__ __forceinline__ void rec_load(const uint4* __restrict__ base, int64_t r,
                                         uint32_t (&w)[rec_words(FMT)]) {
  constexpr int U = rec_words(FMT);
  if constexpr (U == 1) {
    w[0] = ((const uint32_t*)base)[r];
  } else if constexpr (U % 4 == 0) {
#pragma unroll
    for (int i = 0; i < U / 4; ++i) {
      const uint4 q = base[r * (U / 4) + i];
      w[4 * i] = q.x;
      w[4 * i + 1] = q.y;
      w[4 * i + 2] = q.z;
      w[4 * i + 3] = q.w;
    }
  } else {
    const uint2* b2 = (const uint2*)base;
#pragma unroll
    for (int i = 0; i < U / 2; ++i) {
      const uint2 q = b2[r * (U / 2) + i];
      w[2 * i] = q.x;
      w[2 * i + 1] = q.y;
    }
  }
}
// The partition's record stores are non-temporal: the next reader is the next round's
// pass, long after they would have left the L2, and stores that stay dirty in the L2
// are written back at the end of the kernel, on the round's critical path.
template <int FMT>
__device__ __forceinline__ void rec_store(uint4* __restrict__ base, int64_t r,
                                          const uint32_t (&w)[rec_words(FMT)]) {
  constexpr int U = rec_words(FMT);
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  if constexpr (U == 1) {
    __builtin_nontemporal_store(w[0], (uint32_t*)base + r);
  } else if constexpr (U % 4 == 0) {
#pragma unroll
    for (int i = 0; i < U / 4; ++i) {
      u32x4 v;
      v.x = w[4 * i];
      v.y = w[4 * i + 1];
      v.z = w[4 * i + 2];
      v.w = w[4 * i + 3];
      __builtin_nontemporal_store(v, (u32x4*)(base + r * (U / 4) + i));
    }
  } else {
#pragma unroll
    for (int i = 0; i < U / 2; ++i) {
      u32x2 v;
      v.x = w[2 * i];
      v.y = w[2 * i + 1];
      __builtin_nontemporal_store(v, (u32x2*)base + r * (U / 2) + i);
    }
  }
}

// Word wi of a record held in registers: an OR of masked words with compile-time
// indices (a select chain would be turned into an indexed load, which moves the record
// to scratch memory); wi is wave-uniform where it is used.
template <int FMT>
__device__ __forceinline__ uint32_t rec_word(const uint32_t (&w)[rec_words(FMT)], int wi) {
  uint32_t x = 0u;
#pragma unroll
  for (int i = 0; i < rec_words(FMT); ++i)
    x |= w[i] & (uint32_t)__builtin_amdgcn_readfirstlane(-(int32_t)(i == wi));
  return x;
}
// The bin of a feature whose field is word wi, bit sh (rec_field_pos).
template <int FMT>
__device__ __forceinline__ uint32_t rec_field(const uint32_t (&w)[rec_words(FMT)], int wi, int sh) {
  return (rec_word<FMT>(w, wi) >> sh) & ((1u << rec_bits(FMT)) - 1u);
}
// The quantized pair of a packed record, in the u16 form.
template <int FMT>
__device__ __forceinline__ uint32_t rec_gh(const uint32_t (&w)[rec_words(FMT)]) {
  return gh_unpack6((w[rec_words(FMT) - 1] >> 24) & 63u);
}
template <int FMT>
__device__ __forceinline__ void rec_set_gh(uint32_t (&w)[rec_words(FMT)], uint32_t q16) {
  constexpr int U = rec_words(FMT);
  w[U - 1] = (w[U - 1] & 0x00ffffffu) | (gh_pack6(q16) << 24);
}

// Accumulate one row (quantized pair q in the u16 form) into the packed u64 LDS
// histogram of all features: every bin slot of the record words 0 .. nw-1; cbr[s] is
// slot s's first cell.  Slots at or past F hold no feature and are skipped by a
// uniform branch (an LDS atomic costs far more than the branch).  Callers skip a
// (0, 0) pair: it adds nothing.
#define LDS_TRASH_CELLS (4 + LGBM_WAVE)
template <int FMT>
__device__ __forceinline__ void lds_hist_add(unsigned long long* lds, const int32_t* cbr, int nw,
                                             int F, int tl, const uint32_t (&w)[rec_words(FMT)],
                                             uint32_t q) {
  constexpr int BPW = rec_bpw(FMT), BB = rec_bits(FMT), NS = rec_slots(FMT);
  constexpr uint32_t M = (1u << BB) - 1u;
  (void)tl;  // the trash cell: unused since the slots past F are skipped
  const int32_t qg = (int32_t)(int8_t)(q & 0xffu);
  const int32_t qh = (int32_t)(int8_t)(q >> 8);
  const unsigned long long v = (unsigned long long)(long long)qg +
                               ((unsigned long long)(uint32_t)qh << 22) +
                               ((unsigned long long)(qh == 3 ? 1u : 0u) << 43);
#pragma unroll
  for (int k = 0; k < (NS + BPW - 1) / BPW; ++k) {
    if (k < nw) {
      const uint32_t word = w[k];
#pragma unroll
      for (int bb = 0; bb < BPW; ++bb)
        if (BPW * k + bb < NS && BPW * k + bb < F) {  // F: a uniform branch
          const int a = cbr[BPW * k + bb] + (int)((word >> (BB * bb)) & M);
          __hip_atomic_fetch_add(&lds[a], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
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
// Per lane k < cnt: (sg, sh) += the lanes' (g, h) of lanes 0..k, added one at a time in
// lane order — the reference's sequential f64 accumulation, so every prefix rounds
// exactly as its loop does; sc += the integer counts of lanes 0..k (exact in any
// order: a DPP inclusive scan).  The f64 values go through a per-wave LDS row behind
// 64 cells of -0.0 (x + (-0.0) == x for every x, signed zeros included).  The loop
// runs n8 = cnt rounded up to 8 steps and lane k reads cell 65 + j + k - n8 at step j,
// so it adds only padding until step n8 - 1 - k and then its values 0..k in order:
// per-lane consecutive addresses, no masking; each batch of eight cells is loaded
// while the previous one is added.
__device__ __forceinline__ void prefix_in_order(double g, double h, int32_t c, int32_t cnt,
                                                int lane, double* sg, double* sh, int32_t* sc) {
  constexpr int kRow = 2 * LGBM_WAVE + 8;  // padding, values, one batch of overrun
  __shared__ double2 pf_gh[SCAN_THREADS / LGBM_WAVE][kRow];
  const int w = (int)(threadIdx.x / LGBM_WAVE);
  const bool in = lane < cnt;
  const double nz = -0.0;
  pf_gh[w][lane] = make_double2(nz, nz);
  pf_gh[w][LGBM_WAVE + lane] = in ? make_double2(g, h) : make_double2(nz, nz);
  if (lane < 8) pf_gh[w][2 * LGBM_WAVE + lane] = make_double2(nz, nz);
  __builtin_amdgcn_wave_barrier();
  *sc += wave_incl_sum_i32(in ? c : 0);
  double ag = *sg, ah = *sh;
  const int32_t n8 = (cnt + 7) & ~7;
  const double2* r = &pf_gh[w][LGBM_WAVE + 1 + lane - n8];
  double2 cur[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) cur[u] = r[u];
  for (int32_t j0 = 0; j0 < n8; j0 += 8) {
    double2 nxt[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) nxt[u] = r[j0 + 8 + u];  // <= cell 135 of the row
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      ag += cur[u].x;
      ah += cur[u].y;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
  }
  __builtin_amdgcn_wave_barrier();  // the row is rewritten by the next call
  *sg = ag;
  *sh = ah;
}

// A DPP move of an f64 (both halves alike); lanes without a source lane get +0.0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_f64(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const int lo = (int)(uint32_t)b, hi = (int)(uint32_t)(b >> 32);
  const uint32_t nlo = (uint32_t)__builtin_amdgcn_update_dpp(0, lo, CTRL, ROW_MASK, 0xf, false);
  const uint32_t nhi = (uint32_t)__builtin_amdgcn_update_dpp(0, hi, CTRL, ROW_MASK, 0xf, false);
  return __longlong_as_double((long long)(((unsigned long long)nhi << 32) | nlo));
}
// Inclusive prefix sum of the wave's values in lane order, as a DPP tree (row_shr 1, 2,
// 4, 8, then the row broadcasts 15 and 31): exact only when every partial sum is a
// double, as for multiples of one unit well below 2^53 units.
__device__ __forceinline__ double wave_incl_sum_f64_exact(double v) {
  v += dpp_f64<0x111, 0xf>(v);  // row_shr:1
  v += dpp_f64<0x112, 0xf>(v);  // row_shr:2
  v += dpp_f64<0x114, 0xf>(v);  // row_shr:4
  v += dpp_f64<0x118, 0xf>(v);  // row_shr:8
  v += dpp_f64<0x142, 0xa>(v);  // row_bcast:15 into rows 1, 3
  v += dpp_f64<0x143, 0xc>(v);  // row_bcast:31 into rows 2, 3
  return v;
}
// s == fl(a + b): true when the sum is exact (TwoSum's error term is zero).
__device__ __forceinline__ bool sum_is_exact(double a, double b, double s) {
  const double bv = s - a, av = s - bv;
  return ((a - av) + (b - bv)) == 0.0;
}

// prefix_in_order's result for cells that are exact multiples of one unit (quantized
// gradients: integer cells through int_cell_to_f64), except the lane `odd` (the
// FixHistogram cell; out of range: none).  The reference's sums S_k = fl(S_{k-1} +
// v_k) start from the carry (any double).  The unit cells' prefix P is exact in any
// order, so from the last step t that rounded, S_{k-1} = S_t + (P_{k-1} - P_t) exactly
// as long as no step in between rounds; every lane forms its own step from that and
// tests it with TwoSum, and the first lane whose step rounds (or holds the odd cell)
// takes the rounded sum, which is the reference's, as the next t.  The loop runs once
// per rounding step, plus once: a step rounds only where the sum changes binade or
// carries bits below the unit (the kEpsilon start, absorbed within a few binades).
__device__ __forceinline__ void prefix_grid(double g, double h, int32_t c, int32_t cnt, int lane,
                                            int odd, double* sg, double* sh, int32_t* sc) {
  const bool in = lane < cnt;
  *sc += wave_incl_sum_i32(in ? c : 0);
  const bool unit = in && lane != odd;
  const double pg = wave_incl_sum_f64_exact(unit ? g : 0.0);
  const double ph = wave_incl_sum_f64_exact(unit ? h : 0.0);
  const double qg = dpp_f64<0x138, 0xf>(pg), qh = dpp_f64<0x138, 0xf>(ph);  // wave_shr:1
  const double vg = in ? g : 0.0, vh = in ? h : 0.0;
  double tg = *sg, th = *sh, ptg = 0.0, pth = 0.0;
  double og = 0.0, oh = 0.0;
  int t = -1;
  for (;;) {
    // this lane's S_{k-1}, unchanged (signed zeros included) while P has not moved
    const double ag = qg == ptg ? tg : tg + (qg - ptg);
    const double ah = qh == pth ? th : th + (qh - pth);
    const double ng = ag + vg, nh = ah + vh;
    const bool live = in && lane > t;
    const bool bad = live && (lane == odd || !sum_is_exact(ag, vg, ng) || !sum_is_exact(ah, vh, nh));
    const unsigned long long m = __ballot(bad);
    const int j = m ? (int)__builtin_ctzll(m) : LGBM_WAVE;
    if (live && lane <= j) {
      og = ng;
      oh = nh;
    }
    if (!m) break;
    tg = readlane_f64(ng, j);
    th = readlane_f64(nh, j);
    ptg = readlane_f64(pg, j);
    pth = readlane_f64(ph, j);
    t = j;
  }
  *sg = og;
  *sh = oh;
}

// The best candidate of one batch of a threshold scan: the highest gain, the lowest
// lane among equal gains (the reference's strict-> scan in candidate order); -1 when
// no lane is a candidate.  `best` receives the gain.
__device__ __forceinline__ int wave_best_lane(bool cand, double gain, double* best) {
  const double g = wave_max_f64(cand ? gain : -__builtin_inf());
  const unsigned long long m = __ballot(cand && gain == g);
  *best = g;
  return m ? (int)__builtin_ctzll(m) : -1;
}

// FindBestThresholdNumerical for one (leaf, feature) by one wave over the compacted
// histogram; returns the gain written to `out` (-inf for none), in every lane.
// GRID: the cells are unit multiples but for the FixHistogram cell (prefix_grid).
template <bool GRID = false>
__device__ __attribute__((unused)) double wave_scan(const double* hist, const DevFeature& ft, const ScanCfg& c,
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
  // the FixHistogram cell's compacted index (-1: none)
  const int32_t tm = (ft.mfb > 0 && (int32_t)ft.mfb < nb && (int32_t)ft.mfb >= offset)
                         ? (int32_t)ft.mfb - offset
                         : -1;

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
      const double2 m2 = act ? ((const double2*)hist)[t] : make_double2(0.0, 0.0);
      const double mg = m2.x, mh = m2.y;
      const int32_t mc = act ? round_int(mh * cf) : 0;
      double sg = cg, sh = ch;
      int32_t rc = cc;
      if constexpr (GRID)
        prefix_grid(mg, mh, mc, cnt, lane, tm >= 0 ? t_start - base - tm : -1, &sg, &sh, &rc);
      else
        prefix_in_order(mg, mh, mc, cnt, lane, &sg, &sh, &rc);
      const int32_t lc = num_data - rc;
      const double slh = shb - sh, slg = sum_gradient - sg;
      const bool cont = rc < c.min_d || sh < c.min_h;
      const bool brk = lc < c.min_d || slh < c.min_h;
      const unsigned long long bm = __ballot(act && !cont && brk);
      const int first_brk = bm ? (__ffsll((unsigned long long)bm) - 1) : LGBM_WAVE;
      const bool consider = act && !cont && lane < first_brk;
      double gain = ninf;
      if (consider) gain = split_gain_of(c, slg, slh, sg, sh, lc, rc, po);
      double bg;
      const int rl = wave_best_lane(consider && gain > mgs, gain, &bg);
      if (rl >= 0) {
        any_split = true;
        if (bg > best_gain) {
          best_gain = bg;
          best_lc = readlane_i32(lc, rl);
          best_lg = readlane_f64(slg, rl);
          best_lh = readlane_f64(slh, rl);
          best_thr = readlane_i32(t, rl) - 1 + offset;
          best_dl = true;
        }
      }
      if (bm) break;
      cg = readlane_f64(sg, cnt - 1);
      ch = readlane_f64(sh, cnt - 1);
      cc = readlane_i32(rc, cnt - 1);
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
      const double2 m2 = addl ? ((const double2*)hist)[t] : make_double2(0.0, 0.0);
      const double mg = m2.x, mh = m2.y;
      const int32_t mc = addl ? round_int(mh * cf) : 0;
      double sg = cg, sh = ch;
      int32_t lcn = cc;
      if constexpr (GRID)
        prefix_grid(mg, mh, mc, cnt, lane, tm >= 0 ? tm - fwd_start - base : -1, &sg, &sh, &lcn);
      else
        prefix_in_order(mg, mh, mc, cnt, lane, &sg, &sh, &lcn);
      const int32_t rc = num_data - lcn;
      const double srh = shb - sh, srg = sum_gradient - sg;
      const bool cont = lcn < c.min_d || sh < c.min_h;
      const bool brk = rc < c.min_d || srh < c.min_h;
      const unsigned long long bm = __ballot(act && !cont && brk);
      const int first_brk = bm ? (__ffsll((unsigned long long)bm) - 1) : LGBM_WAVE;
      const bool consider = act && !cont && lane < first_brk;
      double gain = ninf;
      if (consider) gain = split_gain_of(c, sg, sh, srg, srh, lcn, rc, po);
      double bg;
      const int rl = wave_best_lane(consider && gain > mgs, gain, &bg);
      if (rl >= 0) {
        any_split = true;
        if (bg > best_gain) {
          best_gain = bg;
          best_lc = readlane_i32(lcn, rl);
          best_lg = readlane_f64(sg, rl);
          best_lh = readlane_f64(sh, rl);
          best_thr = readlane_i32(t, rl) + offset;
          best_dl = false;
        }
      }
      if (bm) break;
      cg = readlane_f64(sg, cnt - 1);
      ch = readlane_f64(sh, cnt - 1);
      cc = readlane_i32(lcn, cnt - 1);
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
  return any_split && best_gain > ninf ? best_gain - mgs : ninf;
}

// ===========================================================================
// FindBestThresholdCategorical for one (leaf, feature) by one wave
// (feature_histogram_categorical.rs:96-495) over the compacted histogram (index t =
// bin - offset, categories t in [1 - offset, num_bin - offset)).
//   one-hot (num_bin <= max_cat_to_onehot): lane t tries "category t left, the rest
//   right"; the strict-> best keeps the lowest t on ties;
//   many-vs-many: the categories whose round_int(hess * cnt_factor) >= cat_smooth,
//   ranked by grad / (hess + cat_smooth) with ties in bin order (the stable sort),
//   then lane 0 walks the ranked list from its low end and lane 1 from its high end
//   with the reference's sequential sums, gates and group counter; the low-end walk
//   wins ties (it runs first in the reference).
// sum_hessian is the leaf's raw sum; the scan bumps it by 2 kEpsilon as the
// categorical dispatch does (learner.rs:3103-3118).  `bits` (8 words) receives the
// bins that go left; the return value is the gain written to `out` (-inf for none).
// A NaN sort key (cat_smooth <= 0 and an empty category) ranks as 0.0: the
// reference's order for it depends on its sort algorithm.
// ===========================================================================
__device__ __forceinline__ double leaf_gain_given_output(bool use_l1, double g, double h,
                                                         double l1, double l2, double out) {
  const double gg = use_l1 ? threshold_l1(g, l1) : g;
  return -__builtin_fma(2.0 * gg, out, (h + l2) * out * out);
}

static __device__ __attribute__((unused)) double wave_scan_cat(const double* hist, const DevFeature& ft, const ScanCfg& c,
                                     const lgbm_gain_config& cfg, double sum_gradient,
                                     double sum_hessian, int32_t num_data, double po,
                                     lgbm_split_info* out, uint32_t* bits) {
  __shared__ double s_key[SCAN_THREADS / LGBM_WAVE][256];
  __shared__ int32_t s_sorted[SCAN_THREADS / LGBM_WAVE][256];
  __shared__ uint32_t s_bits[SCAN_THREADS / LGBM_WAVE][8];
  const int w = (int)(threadIdx.x / LGBM_WAVE);
  const int lane = (int)lane_id();
  const double eps = k_eps();
  const double ninf = -__builtin_inf();
  const double sh = sum_hessian + 2.0 * eps;
  const double gain_shift =
      c.use_smoothing
          ? leaf_gain_given_output(c.use_l1, sum_gradient, sh, c.l1, c.l2, po)
          : leaf_gain_full(c.use_l1, sum_gradient, sh, c.l1, c.l2, c.mds, false, 0.0, num_data, 0.0);
  const double mgs = gain_shift + c.min_gain;
  const int32_t nb = (int32_t)ft.num_bin, offset = ft.offset;
  const int32_t t0 = 1 - offset, t1 = nb - offset;  // categories t in [t0, t1)
  const double cf = (double)num_data / sh;
  const bool onehot = nb <= cfg.max_cat_to_onehot;
  ScanCfg cc = c;  // many-vs-many: l2 + cat_l2 for the gains and outputs
  if (!onehot) cc.l2 = c.l2 + cfg.cat_l2;
  bool any = false;
  double best_gain = ninf, best_lg = 0.0, best_lh = 0.0;
  int32_t best_lc = 0, best_t = -1, best_dir = 1, used = 0;
  if (lane < 8) s_bits[w][lane] = 0u;
  if (onehot) {
    for (int32_t base = t0; base < t1; base += LGBM_WAVE) {
      const int32_t t = base + lane;
      double gain = ninf, grad = 0.0, hess = 0.0;
      int32_t cnt = 0;
      bool cand = false;
      if (t < t1) {
        grad = hist[2 * t];
        hess = hist[2 * t + 1];
        cnt = round_int(hess * cf);
        const int32_t other = num_data - cnt;
        const double soh = sh - hess - eps;
        if (!(cnt < c.min_d || hess < c.min_h) && !(other < c.min_d) && !(soh < c.min_h)) {
          gain = split_gain_of(c, sum_gradient - grad, soh, grad, hess + eps, other, cnt, po);
          cand = gain > mgs;
        }
      }
      if (__ballot(cand)) any = true;
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
        best_t = __shfl(t, rl);
        best_lg = __shfl(grad, rl);
        best_lh = __shfl(hess, rl) + eps;
        best_lc = __shfl(cnt, rl);
      }
    }
  } else {
    // ranks of the kept categories by (key, bin); n kept in total
    const int32_t m = t1 - t0;
    unsigned long long keep[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int32_t i = lane + LGBM_WAVE * k;
      const int32_t t = t0 + i;
      bool kp = false;
      double key = 0.0;
      if (i < m) {
        const double hess = hist[2 * t + 1];
        kp = (double)round_int(hess * cf) >= cfg.cat_smooth;
        key = hist[2 * t] / (hess + cfg.cat_smooth);
        if (key != key) key = 0.0;
      }
      keep[k] = __ballot(kp);
      s_key[w][i] = key;
    }
    used = __popcll(keep[0]) + __popcll(keep[1]) + __popcll(keep[2]) + __popcll(keep[3]);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int32_t i = lane + LGBM_WAVE * k;
      if (!((keep[k] >> lane) & 1ull)) continue;
      const double key = s_key[w][i];
      int32_t r = 0;
      for (int32_t j = 0; j < m; ++j) {
        if (!((keep[j >> 6] >> (j & 63)) & 1ull)) continue;
        const double o = s_key[w][j];
        r += (o < key || (!(key < o) && j < i)) ? 1 : 0;
      }
      s_sorted[w][r] = t0 + i;
    }
    __builtin_amdgcn_wave_barrier();
    const int32_t max_num_cat = min(cfg.max_cat_threshold, (used + 1) / 2);
    bool split = false;
    double g_best = ninf, g_lg = 0.0, g_lh = 0.0;
    int32_t g_lc = 0, g_i = -1;
    if (lane < 2) {
      const int32_t dir = lane == 0 ? 1 : -1;
      int32_t pos = lane == 0 ? 0 : used - 1;
      int32_t group = 0, lcnt = 0;
      double slg = 0.0, slh = eps;
      for (int32_t i = 0; i < used && i < max_num_cat; ++i) {
        const int32_t t = s_sorted[w][pos];
        pos += dir;
        const double grad = hist[2 * t], hess = hist[2 * t + 1];
        const int32_t cnt = round_int(hess * cf);
        slg += grad;
        slh += hess;
        lcnt += cnt;
        group += cnt;
        if (lcnt < c.min_d || slh < c.min_h) continue;
        const int32_t rcnt = num_data - lcnt;
        if (rcnt < c.min_d || rcnt < cfg.min_data_per_group) break;
        const double srh = sh - slh;
        if (srh < c.min_h) break;
        if (group < cfg.min_data_per_group) continue;
        group = 0;
        const double gain = split_gain_of(cc, slg, slh, sum_gradient - slg, srh, lcnt, rcnt, po);
        if (gain <= mgs) continue;
        split = true;
        if (gain > g_best) {
          g_best = gain;
          g_lc = lcnt;
          g_lg = slg;
          g_lh = slh;
          g_i = i;
        }
      }
    }
    // lane 0: the low-end walk; lane 1 replaces it only with a strictly larger gain
    const bool s1 = __shfl(split, 1) != 0;
    const double gb1 = __shfl(g_best, 1);
    any = (__shfl(split, 0) != 0) || s1;
    const int src = gb1 > __shfl(g_best, 0) ? 1 : 0;
    best_gain = __shfl(g_best, src);
    best_lg = __shfl(g_lg, src);
    best_lh = __shfl(g_lh, src);
    best_lc = __shfl(g_lc, src);
    best_t = __shfl(g_i, src);
    best_dir = src == 0 ? 1 : -1;
  }
  __builtin_amdgcn_wave_barrier();
  if (any) {
    if (onehot) {
      if (lane == 0) {
        const int32_t b = best_t + offset;
        s_bits[w][b >> 5] |= 1u << (b & 31);
      }
    } else {
      for (int32_t p = lane; p < used; p += LGBM_WAVE) {
        const bool sel = best_dir == 1 ? p <= best_t : p >= used - 1 - best_t;
        if (!sel) continue;
        const int32_t b = s_sorted[w][p] + offset;
        atomicOr(&s_bits[w][b >> 5], 1u << (b & 31));
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  if (lane < 8) bits[lane] = s_bits[w][lane];
  if (lane == 0) {
    if (!any) {
      split_set_none(out);
      out->default_left = 0;
    } else {
      // the finalization (:395-495): outputs with the scan's l2, sums without kEpsilon
      const int32_t rc = num_data - best_lc;
      out->left_output = leaf_output_full(cc.use_l1, best_lg, best_lh, cc.l1, cc.l2, cc.mds,
                                          cc.use_smoothing, cc.ps, best_lc, po);
      out->left_count = best_lc;
      out->left_sum_gradient = best_lg;
      out->left_sum_hessian = best_lh - eps;
      out->right_output = leaf_output_full(cc.use_l1, sum_gradient - best_lg, sh - best_lh, cc.l1,
                                           cc.l2, cc.mds, cc.use_smoothing, cc.ps, rc, po);
      out->right_count = rc;
      out->right_sum_gradient = sum_gradient - best_lg;
      out->right_sum_hessian = sh - best_lh - eps;
      out->gain = best_gain - mgs;
      out->default_left = 0;
      out->threshold = 0;
    }
  }
  return any ? best_gain - mgs : ninf;
}

struct BestKey {
  double gain;
  int32_t feat;  // real feature index (-1 none)
  int32_t idx;   // feature position / leaf id
};

// split_gt order (split_info.rs:28-35), ties to the lower position / leaf id (the
// reference's sequential strict-> scans).
__device__ __forceinline__ bool key_better(const BestKey& a, const BestKey& b) {
  if (split_gt(a.gain, a.feat, b.gain, b.feat)) return true;
  if (split_gt(b.gain, b.feat, a.gain, a.feat)) return false;
  return a.idx < b.idx;
}

__device__ __forceinline__ BestKey wave_best(BestKey k) {
  for (int off = 32; off >= 1; off >>= 1) {
    BestKey o;
    o.gain = __shfl_xor(k.gain, off);
    o.feat = __shfl_xor(k.feat, off);
    o.idx = __shfl_xor(k.idx, off);
    if (key_better(o, k)) k = o;
  }
  return k;
}

// wave_best with the common case fast: the highest gain by a DPP maximum, and when
// one lane alone holds it, that lane's key; ties (or no key) take the exact order.
__device__ __forceinline__ BestKey wave_best_fast(BestKey k) {
  const double ninf = -__builtin_inf();
  const bool valid = k.idx != 0x7fffffff;  // no key
  const double gm = wave_max_f64(valid ? k.gain : ninf);
  if (!(gm > ninf)) return BestKey{ninf, -1, 0x7fffffff};
  const unsigned long long m = __ballot(valid && k.gain == gm);
  if (__popcll(m) == 1) {
    const int r = (int)__builtin_ctzll(m);
    return BestKey{gm, readlane_i32(k.feat, r), readlane_i32(k.idx, r)};
  }
  return wave_best(k);
}

// FixHistogram (fix_histogram.rs:50-80) on the RAW leaf sums: the most frequent bin's
// cell = leaf sum minus the other bins in ascending order (the sequential f64 chain),
// every lane of wave 0 the same chain over broadcast LDS reads, eight bins per batch.
// The skipped bin is parked at +0.0 first (x - (+0.0) == x for every x) and
// overwritten with the result, which every lane of wave 0 also returns in (g, h).
// Called by wave 0 when 0 < mfb < num_bin.
__device__ __forceinline__ void fix_mfb_wave(double* cs, int nb, int mfb, double sg, double sh,
                                             double* fg, double* fh) {
  const int tid = threadIdx.x;
  if (tid == 0) {
    cs[2 * mfb] = 0.0;
    cs[2 * mfb + 1] = 0.0;
  }
  __builtin_amdgcn_wave_barrier();
  const double2* c2 = (const double2*)cs;
  double g = sg, h = sh;
  int i = 0;
  for (; i + 8 <= nb; i += 8) {
    double2 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = c2[i + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      g -= v[u].x;
      h -= v[u].y;
    }
  }
  for (; i < nb; ++i) {
    const double2 v = c2[i];
    g -= v.x;
    h -= v.y;
  }
  __builtin_amdgcn_wave_barrier();
  if (tid == 0) {
    cs[2 * mfb] = g;
    cs[2 * mfb + 1] = h;
  }
  *fg = g;
  *fh = h;
}

// Compaction (compact_histogram, learner.rs:4460-4492): the cells shift down by the
// feature's offset, zeros enter at the top.  Every thread of a SCAN_THREADS block;
// the caller has synchronised the cells.
__device__ __forceinline__ void compact_shift(const DevFeature& ft, double* cs) {
  const int tid = threadIdx.x;
  const int nb = (int)ft.num_bin;
  const int off = ft.offset;
  if (off <= 0) return;
  if (nb <= 256) {
    double a[256 / SCAN_THREADS], b2[256 / SCAN_THREADS];
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
  } else {
    // wider features shift down chunk by chunk: a chunk reads only cells the
    // earlier chunks did not write
    for (int c0 = 0; c0 < nb; c0 += SCAN_THREADS) {
      const int c = c0 + tid, src = c + off;
      const double a = (c < nb && src < nb) ? cs[2 * src] : 0.0;
      const double b2 = (c < nb && src < nb) ? cs[2 * src + 1] : 0.0;
      __syncthreads();
      if (c < nb) {
        cs[2 * c] = a;
        cs[2 * c + 1] = b2;
      }
      __syncthreads();
    }
  }
}

// FixHistogram, then compaction, on one feature's cells in LDS.  `zero` (a leaf with
// no rows or no hessian, or a feature masked out by the parent) clears the cells
// instead.  Called by every thread of a SCAN_THREADS block.
__device__ __forceinline__ void fix_compact_block(const DevFeature& ft, double* cs, double sg,
                                                  double sh, bool zero) {
  const int tid = threadIdx.x;
  const int nb = (int)ft.num_bin;
  __syncthreads();
  if (zero) {
    for (int i = tid; i < 2 * nb; i += SCAN_THREADS) cs[i] = 0.0;
    __syncthreads();
    return;
  }
  const int mfb = (int)ft.mfb;
  if (tid < LGBM_WAVE && mfb > 0 && mfb < nb) {
    double fg, fh;
    fix_mfb_wave(cs, nb, mfb, sg, sh, &fg, &fh);
  }
  __syncthreads();
  compact_shift(ft, cs);
  __syncthreads();
}

// The same for both children of a split.  `cs` holds the smaller child's cells
// (fixed with its sums as above, or cleared by `zero`), `cp` the larger child's (or
// the parent's) cells from integers.  The reference's larger child is parent - smaller
// cell by cell, never re-fixed: quantized integer-derived cells subtract exactly (f32
// fixed-point ones within one rounding), so only its most-frequent-bin cell differs
// from its integers: the parent's fixed pair `pm` minus the smaller's fixed cell
// (`sub`), or `pm` itself (`cp` then holds the parent, from which the caller
// subtracts).  Both arrays are compacted.
__device__ __forceinline__ void fix_compact_pair(const DevFeature& ft, double* cs, double* cp,
                                                 double sg, double sh, bool zero, double2 pm,
                                                 bool sub) {
  const int tid = threadIdx.x;
  const int nb = (int)ft.num_bin;
  const int mfb = (int)ft.mfb;
  const bool has_fix = mfb > 0 && mfb < nb;
  __syncthreads();
  if (zero) {
    for (int i = tid; i < 2 * nb; i += SCAN_THREADS) cs[i] = 0.0;
    if (tid == 0 && has_fix) {
      cp[2 * mfb] = sub ? pm.x - 0.0 : pm.x;
      cp[2 * mfb + 1] = sub ? pm.y - 0.0 : pm.y;
    }
  } else if (tid < LGBM_WAVE && has_fix) {
    double fg, fh;
    fix_mfb_wave(cs, nb, mfb, sg, sh, &fg, &fh);
    if (tid == 0) {
      cp[2 * mfb] = sub ? pm.x - fg : pm.x;
      cp[2 * mfb + 1] = sub ? pm.y - fh : pm.y;
    }
  }
  __syncthreads();
  compact_shift(ft, cs);
  __syncthreads();
  compact_shift(ft, cp);
  __syncthreads();
}

// Packed cell (fields: q_g sum signed 22 bits, q_h sum 21 bits, count of q_h == 3
// 21 bits) -> its integer counters.
__device__ __forceinline__ void unpack_cell(unsigned long long p, int32_t* g, int32_t* h,
                                            int32_t* t) {
  const int64_t lo22 = (int64_t)(p & ((1ull << 22) - 1));
  const int64_t gsum = lo22 >= (1ll << 21) ? lo22 - (1ll << 22) : lo22;
  const unsigned long long rest = (p - (unsigned long long)gsum) >> 22;
  *g = (int32_t)gsum;
  *h = (int32_t)(rest & ((1ull << 21) - 1));
  *t = (int32_t)(rest >> 21);
}

// Moves a block's packed LDS histogram into integer cells (G, H, T) and clears it (the
// trash cells too).  mode FLUSH_ATOMIC: atomic adds into a shared int32 [cells][3]
// accumulator (zero cells skipped); FLUSH_ATOMIC64: 64-bit atomic adds of the packed
// cells into a u64 [cells] accumulator (the caller bounds the summed rows below 2^19,
// so no field carries); FLUSH_STORE: the packed cells as they are into
// the block's own u64 [cells] slot (one flush per slot: a slot holds fewer than 2^19
// rows per cell, as the LDS histogram does).  The caller has synchronised the block
// after the last accumulation.
#define FLUSH_ATOMIC 0
#define FLUSH_STORE 1
#define FLUSH_ATOMIC64 2
__device__ __forceinline__ void lds_hist_flush_clear(unsigned long long* lds, int cells,
                                                     void* __restrict__ out, int mode) {
  for (int c = threadIdx.x; c < cells + 4; c += blockDim.x) {
    const unsigned long long p = lds[c];
    lds[c] = 0ull;
    if (c >= cells) continue;  // trash cells
    if (mode == FLUSH_STORE) {
      ((unsigned long long*)out)[c] = p;
      continue;
    }
    if (mode == FLUSH_ATOMIC64) {
      if (p != 0ull)
        __hip_atomic_fetch_add((unsigned long long*)out + c, p, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      continue;
    }
    int32_t gsum, hsum, n3;
    unpack_cell(p, &gsum, &hsum, &n3);
    if (p != 0ull) {
      int32_t* dst = (int32_t*)out + (size_t)c * 3;
      if (gsum) __hip_atomic_fetch_add(dst, (int32_t)gsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (hsum) __hip_atomic_fetch_add(dst + 1, hsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (n3) __hip_atomic_fetch_add(dst + 2, n3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Integer cells (sum q_g, sum q_h, #q_h==3) of cell ci of a histogram job: the sum
// of its partial slots [a0, a0 + na), four slots per step with independent loads.
__device__ __forceinline__ void hist_part_sum(const DevLearner& L, int32_t a0, int32_t na, size_t ci,
                                              int32_t* G, int32_t* H, int32_t* T) {
  const size_t stride = (size_t)L.total_cells * 3;
  const int32_t* p = L.hist_part + (size_t)a0 * stride + ci * 3;
  int32_t g = 0, h = 0, t = 0;
  int32_t k = 0;
  for (; k + 4 <= na; k += 4, p += 4 * stride) {
    int32_t x[12];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      x[3 * u] = p[u * stride];
      x[3 * u + 1] = p[u * stride + 1];
      x[3 * u + 2] = p[u * stride + 2];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      g += x[3 * u];
      h += x[3 * u + 1];
      t += x[3 * u + 2];
    }
  }
  for (; k < na; ++k, p += stride) {
    g += p[0];
    h += p[1];
    t += p[2];
  }
  *G = g;
  *H = h;
  *T = t;
}

// The 64-bit fixed-point (g, h) cells of a histogram job (f32 gradients).
__device__ __forceinline__ void hist_part_sum64(const DevLearner& L, int32_t a0, int32_t na,
                                                size_t ci, long long* G, long long* H) {
  const size_t stride = (size_t)L.total_cells * 2;
  const int64_t* p = L.hist_part64 + (size_t)a0 * stride + ci * 2;
  long long g = 0, h = 0;
  for (int32_t k = 0; k < na; ++k, p += stride) {
    g += p[0];
    h += p[1];
  }
  *G = g;
  *H = h;
}

// Exact f64 histogram cells from the integer counters (sum q_g, sum q_h, #q_h==3).
__device__ __forceinline__ void int_cell_to_f64(int32_t G, int32_t H, int32_t T, double vg1,
                                                double vh1, double vh3, double* g, double* h) {
  *g = (double)G * vg1;
  *h = (double)((long long)H - 3ll * T) * vh1 + (double)T * vh3;
}

}  // namespace lgbm
