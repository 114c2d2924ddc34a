// The smooth-L0 imp-min inside the fused steps (pd/core/losses.py:316-394,
// pd/core/objective.py:101-131): per-value penalty psi(v) = s v^2 / (v^2 + gamma^2)
// (s = 1 + gamma^2 when normalized at one, else 1) on the upper CI, component frequencies
// f_c = sum psi / n over the batch's n tokens, loss coeff * sum f_c + freq_coeff *
// sum f_c log2(1 + a f_c) (a = the reference datapoint count; no frequency term when
// a = 0). A selected-emitting (expert) site's values add into their expert's block of
// the [E * c] components (pd/core/losses.py:316-330).
//
// In a fused step the mask forward writes, per 64-row job tile and group (expert) g
// present in it, the tile's column sums of psi to colpart[(tile + g) * c + col] (rows
// sorted by group, so tile + g is unique over the pairs that exist and stays below
// n_tiles + G); k_sl0_finalize adds each group's tiles in order (deterministic), forms
// f_c, the loss partials and the slope (coeff + freq_coeff Phi'(f_c)) / n that the mask
// backward multiplies into psi'(upper). With the EMA estimator (ImpSpec::ema) the
// frequency term reads f_hat, the debiased running estimate after this batch, in both its
// value Phi(f_hat) and its slope Phi'(f_hat) (the reference's first-order surrogate
// Phi'(f_hat) df_batch, pd/core/losses.py:449-456); the batch value Phi(f_c) is kept as a
// diagnostic (EmaFrequencyPenalty.batch_value, :501-503).
#pragma once

#include <type_traits>

#include "pd_tiles.hpp"

namespace pd {

// Imp-min mode of the mask kernels beside the L_p exponent modes (2, 1, 0 of pow_mode).
static constexpr int PM_SL0 = 3;

struct ImpSpec {
  int kind;  // PD_IMPMIN_PNORM or PD_IMPMIN_SMOOTH_L0
  float p, gamma;
  int normalize_at_one;
  float coeff, freq_coeff, ref_count;
  FreqEma ema;  // the frequency term's running estimate (off: the single-batch estimate)
  float g2() const { return gamma * gamma; }
  float psi_scale() const { return normalize_at_one ? 1.f + gamma * gamma : 1.f; }
};

inline int imp_mode(const ImpSpec& q) { return q.kind == PD_IMPMIN_SMOOTH_L0 ? PM_SL0 : pow_mode(q.p); }

inline int check_imp_spec(const ImpSpec& q, const char* what) {
  if (q.kind != PD_IMPMIN_PNORM && q.kind != PD_IMPMIN_SMOOTH_L0)
    return fail(PD_EINVAL, std::string(what) + ": unknown imp-min kind");
  if (q.kind == PD_IMPMIN_SMOOTH_L0 && !(q.gamma > 0.f)) return fail(PD_EINVAL, std::string(what) + ": gamma > 0");
  if (q.kind == PD_IMPMIN_SMOOTH_L0 && !(q.ref_count >= 0.f))
    return fail(PD_EINVAL, std::string(what) + ": reference datapoint count >= 0");
  if (q.ema.on() && !(q.kind == PD_IMPMIN_SMOOTH_L0 && q.ref_count > 0.f))
    return fail(PD_EINVAL, std::string(what) + ": the EMA estimate needs the smooth-L0 frequency term (ref_count > 0)");
  return PD_OK;
}

// The imp-min spec of a fused step from its C-ABI arguments (the EMA estimator's checks
// included).
inline int make_imp_spec(const char* what, int kind, float p, float gamma, int normalize_at_one, float coeff,
                         float freq_coeff, float ref_count, const float* ema_in, float* ema_out, float ema_count,
                         float ema_halflife, ImpSpec& q) {
  q = ImpSpec{kind, p, gamma, normalize_at_one, coeff, freq_coeff, ref_count, FreqEma{}};
  if (int rc = make_freq_ema(what, ema_in, ema_out, ema_count, ema_halflife, q.ema)) return rc;
  return check_imp_spec(q, what);
}

__device__ inline float sl0_psi(float v, float g2, float s) { return s * v * v / (v * v + g2); }
__device__ inline float sl0_dpsi(float v, float g2, float s) {
  const float den = v * v + g2;
  return s * 2.f * v * g2 / (den * den);
}

// The group g of sorted row j: off[g] <= j < off[g + 1] (off[G] = the row count > j).
__device__ inline int row_group(const int32_t* __restrict__ off, int G, int64_t j) {
  int lo = 1, hi = G;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (off[mid] > j) hi = mid;
    else lo = mid + 1;
  }
  return lo - 1;
}

// LDS of the in-tile column sums: psi of the 64x64 tile and each row's group (-1 = no row).
struct Sl0Tile {
  float ps[64][65];
  int grp[64];
};

struct NoSl0Tile {};  // the LDS slot of the other imp-min modes

// Rows j0 + tid (tid < 64) learn their group: group_of(j) from the offsets, or 0 for
// every row below n_rows when off is NULL (one group: a dense site).
__device__ inline void sl0_tile_groups(Sl0Tile& L, const int32_t* off, int G, int64_t j0, int64_t n_rows, int tid) {
  if (tid < 64) {
    const int64_t j = j0 + tid;
    L.grp[tid] = j < n_rows ? (off ? row_group(off, G, j) : 0) : -1;
  }
}

// After a barrier that made L.ps / L.grp visible: thread col (< 64) walks the tile's rows
// in order and writes each group's column sum (rows grouped consecutively).
__device__ inline void sl0_tile_colsums(const Sl0Tile& L, int64_t tile, int q0, int C, float* __restrict__ colpart,
                                        int tid) {
  if (tid >= 64 || q0 + tid >= C) return;
  float acc = 0.f;
  for (int r = 0; r < 64; ++r) {
    const int g = L.grp[r];
    if (g < 0) break;
    acc += L.ps[r][tid];
    if (r == 63 || L.grp[r + 1] != g) {
      colpart[(tile + g) * C + q0 + tid] = acc;
      acc = 0.f;
    }
  }
}

// One thread per (group g, column): f = (sum of g's tile partials, in tile order) / n;
// slope[g * C + col] = (coeff + freq_coeff Phi'(fe)) / n; per-block partials of sum f,
// sum Phi(fe) and, with the EMA estimator (fb_part non-NULL), sum Phi(f) (double, fixed
// order). fe is f, or f_hat with the EMA estimator, which also stores the site's new
// estimate (ema already offset to the site's components). off NULL: one group of rows
// [0, n_rows).
static __global__ __launch_bounds__(256) void k_sl0_finalize(const float* __restrict__ colpart,
                                                      const int32_t* __restrict__ off, int G, int64_t n_rows, int C,
                                                      float inv_n, float coeff, float freq_coeff, float ref_count,
                                                      FreqEma ema, float* __restrict__ slope,
                                                      float* __restrict__ act_part, float* __restrict__ freq_part,
                                                      float* __restrict__ fb_part) {
  __shared__ double sa[4], sf[4], sb[4];
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  double a = 0.0, fq = 0.0, fb = 0.0;
  if (i < (int64_t)G * C) {
    const int g = (int)(i / C), col = (int)(i % C);
    const int64_t lo = off ? off[g] : 0, hi = off ? off[g + 1] : n_rows;
    float F = 0.f;
    if (hi > lo)
      for (int64_t t = lo / 64; t <= (hi - 1) / 64; ++t) F += colpart[(t + g) * C + col];
    const float f = F * inv_n;
    float sl = coeff;
    if (ref_count > 0.f) {
      const float fe = ema.on() ? ema_frequency(ema, i, f, true) : f;
      const float af = ref_count * fe;
      fq = (double)fe * log2((double)(1.f + af));
      fb = (double)f * log2((double)(1.f + ref_count * f));
      sl += freq_coeff * (log2f(1.f + af) + af / ((1.f + af) * 0.69314718055994531f));
    }
    slope[i] = sl * inv_n;
    a = f;
  }
  a = wave_sum_d(a);
  fq = wave_sum_d(fq);
  fb = wave_sum_d(fb);
  if ((threadIdx.x & 63) == 0) {
    sa[threadIdx.x >> 6] = a;
    sf[threadIdx.x >> 6] = fq;
    sb[threadIdx.x >> 6] = fb;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    act_part[blockIdx.x] = (float)((sa[0] + sa[1]) + (sa[2] + sa[3]));
    freq_part[blockIdx.x] = (float)((sf[0] + sf[1]) + (sf[2] + sf[3]));
    if (fb_part) fb_part[blockIdx.x] = (float)((sb[0] + sb[1]) + (sb[2] + sb[3]));
  }
}

inline unsigned sl0_blocks(int G, int C) { return (unsigned)cdiv((int64_t)G * C, 256); }

}  // namespace pd
