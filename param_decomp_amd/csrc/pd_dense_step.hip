// The fused single-site stochastic-recon step (gfx950): one fwd+bwd of one decomposed
// linear with the paper-form gate, mask draw, MSE recon and L_p imp-min
// (pd/core/train.py:1126-1352 restricted to one site; pd/core/masking.py:148-167 draws;
// pd/core/decomposed_linear.py:142-175; spd_paper.md appendix gate).
//
// Every operand is consumed in the layout it is stored in: the bf16 GEMM reads an
// MN-contiguous operand through the transposing LDS read (ds_read_b64_tr_b16), so no
// transposed copy of x, V, U, acts, dy or dh is ever written. Every tensor of the step
// is token-major.
//
//   yt  = x @ W^T          A=x [T,d_in] (K-contig)     B=W [d_out,d_in] (K-contig)
//   h   = x @ V            A=x                         B=V [d_in,C] (N-contig)
//   fwd elementwise: gate, squash, u, acts = h*(m-d)  -> acts [T,C]
//   y   = acts @ U         A=acts [T,C]                B=U [C,d_out] (N-contig)
//   recon: e = y + d*yt - yt, dy = scale*e            -> dy [T,d_out]
//   dU  = acts^T @ dy      A=acts [T,C] (M-contig)     B=dy [T,d_out] (N-contig)
//   da  = dy @ U^T         A=dy [T,d_out]              B=U [C,d_out] (K-contig)
//   bwd elementwise: dh = da*(m-d) + gate pullback     -> dh [T,C]
//   dV  = x^T @ dh         A=x [T,d_in] (M-contig)     B=dh [T,C] (N-contig)
#include <algorithm>

#include "pd_impmin.hpp"

namespace pd {

static constexpr int SITE_COLS = 64;  // components per block in the column-mapped kernels
static constexpr int SITE_ROWS = 64;  // tokens per block chunk
static constexpr int TP = 64;         // recon tile

struct StepParams {
  int64_t T, C;
  uint32_t mk0, mk1;
  int draw_dtype, layout;
  float p, imp_scale;     // imp_scale = imp_coeff / T
  const float* delta;     // [T] per-token delta draw, or NULL (d = 0)
  uint8_t* ubits;         // [T, C] bf16-draw uniforms as 7-bit integers (bf16 draws only)
  // smooth-L0 imp-min (sl0 != 0): psi = psis * v^2 / (v^2 + g2); the forward writes each
  // 64-token chunk's column sums of psi to colpart [chunk][C], the backward reads the
  // per-component slope [C]
  int sl0;
  float g2, psis;
  float* colpart;
  const float* slope;
};


__device__ inline float step_delta(const StepParams& s, int64_t t) { return s.delta ? s.delta[t] : 0.f; }

__global__ void k_delta_fill(uint32_t k0, uint32_t k1, int64_t T, int draw_dtype, int layout, float* __restrict__ d) {
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < T; t += (int64_t)gridDim.x * blockDim.x)
    d[t] = draw_uniform(k0, k1, t, T, draw_dtype, layout);
}

__device__ inline float pow_p(float b, float p) { return p == 2.f ? b * b : (p == 1.f ? b : powf(b, p)); }
__device__ inline float dpow_p(float b, float p) {
  return p == 2.f ? 2.f * b : (p == 1.f ? 1.f : p * powf(b, p - 1.f));
}

// The per-element imp-min value (psi or upper^p) and its derivative's factor.
__device__ inline float step_imp(const StepParams& s, float up) {
  return s.sl0 ? sl0_psi(up, s.g2, s.psis) : pow_p(up, s.p);
}
__device__ inline float step_dimp(const StepParams& s, int64_t c, float up) {
  return s.sl0 ? s.slope[c] * sl0_dpsi(up, s.g2, s.psis) : s.imp_scale * dpow_p(up, s.p);
}

// The uniform of element i: bf16 draws are stored by the forward as the 7-bit integer
// k (u = k/128) and re-read by the backward; fp32 draws are regenerated from the key.
__device__ inline float step_uniform_fwd(const StepParams& s, int64_t i, int64_t n) {
  if (s.draw_dtype == PD_DTYPE_BF16) {
    const uint32_t k = (draw_bits(s.mk0, s.mk1, i, n, 8, s.layout) & 0xFFu) >> 1;
    s.ubits[i] = (uint8_t)k;
    return (float)k * (1.f / 128.f);
  }
  return draw_uniform(s.mk0, s.mk1, i, n, s.draw_dtype, s.layout);
}
__device__ inline float step_uniform_bwd(const StepParams& s, int64_t i, int64_t n) {
  if (s.draw_dtype == PD_DTYPE_BF16) return (float)s.ubits[i] * (1.f / 128.f);
  return draw_uniform(s.mk0, s.mk1, i, n, s.draw_dtype, s.layout);
}

// Forward, one component per lane over a 64-token chunk: gate MLP on h, squash, draw u,
// acts = h*(m-d), imp-min partial of upper^p. Writes g_raw (fp32) and acts.
template <typename T, bool PRECISE>
__global__ __launch_bounds__(SITE_COLS) void k_step_fwd(const T* __restrict__ h, const float* __restrict__ w_in,
                                                        const float* __restrict__ b_in,
                                                        const float* __restrict__ w_out,
                                                        const float* __restrict__ b_out, StepParams s,
                                                        float* __restrict__ g_raw, T* __restrict__ acts,
                                                        float* __restrict__ imp_partial) {
  const int64_t c = (int64_t)blockIdx.x * SITE_COLS + threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * SITE_ROWS;
  const int64_t r1 = r0 + SITE_ROWS < s.T ? r0 + SITE_ROWS : s.T;
  float imp = 0.f, col = 0.f;
  if (c < s.C) {
    float wi[16], bi[16], wo[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      wi[j] = w_in[c * 16 + j];
      bi[j] = b_in[c * 16 + j];
      wo[j] = w_out[c * 16 + j];
    }
    const float bo = b_out[c];
    const int64_t n = s.T * s.C;
    for (int64_t t = r0; t < r1; ++t) {
      const int64_t i = t * s.C + c;
      const float hv = load_f<T>(h, i);
      float g = bo;
#pragma unroll
      for (int j = 0; j < 16; ++j) g = fmaf(wo[j], gelu_only<PRECISE>(fmaf(wi[j], hv, bi[j])), g);
      g_raw[i] = g;
      const float lo = lower_fwd(g);
      const float iv = step_imp(s, upper_fwd(g));
      imp += iv;
      col += iv;
      const float u = step_uniform_fwd(s, i, n);
      const float m = lo + (1.f - lo) * u;
      store_f<T>(acts, i, hv * (m - step_delta(s, t)));
    }
    if (s.sl0) s.colpart[(int64_t)blockIdx.y * s.C + c] = col;
  }
  imp = wave_sum(imp);
  if (threadIdx.x == 0) imp_partial[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = imp;
}

// ---------------------------------------------------------------- binned gate (bf16 step)
// For one component c the gate preactivation g_c(h) = b_out + sum_j w_out_j GELU(w_in_j h +
// b_in_j) is a smooth function of the scalar h, and the step has all of its h values
// (from x @ V) before either elementwise pass. The bf16 step splits the component's
// observed [min h, max h] into GATE_TBINS equal bins and represents g_c on each by its
// degree-7 Chebyshev interpolant (exact g at the bin's 8 Chebyshev nodes), stored as
// power-series coefficients in the bin coordinate tau in [-1, 1]. The forward and the
// backward evaluate g and dg/dh from this one table with the same code, so the
// backward's squashing branches see the forward's g bit for bit without it being stored.
//
// The gate-parameter gradients are token sums of dg_t f(h_t) for 48 functions f of h
// (w_out_j GELU'(z_j) h, w_out_j GELU'(z_j), GELU(z_j), z_j = w_in_j h + b_in_j). The
// backward accumulates, per component and moment bin (a pair of table bins), the
// Chebyshev moments M_m = sum_t dg_t T_m(tau_t), m < 8. If p is the degree-7 Chebyshev
// interpolant of f on the bin, sum_t dg_t p(tau_t) = sum_k w_k f(node_k) with node
// weights w_k = (2/8) (M_0 / 2 + sum_{m>=1} cos(m theta_k) M_m), theta_k = (2k+1) pi / 16
// (discrete orthogonality of T_m on the nodes). So each component's T-token pullback
// becomes the exact pullback of 128 weighted virtual tokens (8 nodes per moment bin),
// evaluated once per step; sum_k w_k = M_0 keeps the b_out gradient exact.
//
// Error: with dz = |w_in_j| * (moment-bin width) <= GATE_DZ_MAX = 3 for every hidden
// unit, the moment interpolant of GELU, GELU' and h GELU' errs by at most 1.6e-4, 4.0e-4
// and 7.5e-4 of their scale (worst bin position; sums over tokens average it further),
// and the table (half as wide in z) by 8.3e-7 for GELU (so |g error| <= 8.3e-7 sum_j
// |w_out_j|) and 6.9e-5 for its derivative. A component with a wider unit is flagged by
// the table pass, and both passes evaluate its gate exactly, element by element, as the
// fp32 step does.
static constexpr int GATE_TBINS = 32;    // table bins over [min h, max h]
static constexpr int GATE_MBINS = 16;    // moment bins (pairs of table bins)
static constexpr int GATE_NC = 8;        // degree-7 table polynomials, 8 Chebyshev moments
static constexpr int GATE_MOM = GATE_MBINS * GATE_NC;  // moment slots per component (>= 49)
static constexpr float GATE_DZ_MAX = 3.f;
static constexpr int RANGE_ROWS = 256;   // tokens per block of the range pass
static constexpr int FWD_WAVES = 8;      // waves per binned-forward block (each 64 tokens)
static constexpr int BWD_COLS = 32;      // components per binned-backward block
static constexpr int BWD_WAVES = 4;      // waves per binned-backward block
static constexpr int BWD_ROWS = 256;     // tokens per half-wave stream of the backward
static constexpr int BWD_BLOCK_ROWS = 2 * BWD_WAVES * BWD_ROWS;  // tokens per backward block
static_assert(GATE_MOM >= 49, "the exact-gate sums share the moment slots");

// The Chebyshev nodes x_k = cos((2k+1) pi / 16), k < 8 (T_m(x_k) = cos(m (2k+1) pi / 16)
// follows by the recurrence T_{m+1} = 2 x T_m - T_{m-1}).
__constant__ float kChebNode[GATE_NC] = {0.980785280f,  0.831469612f,  0.555570233f,  0.195090322f,
                                         -0.195090322f, -0.555570233f, -0.831469612f, -0.980785280f};

// Partial per-component min/max of h over RANGE_ROWS tokens: rng_part[chunk][c] = (min, max).
__global__ __launch_bounds__(256) void k_gate_range(const bf16_t* __restrict__ h, int64_t T, int64_t C,
                                                    float2* __restrict__ rng_part) {
  __shared__ float2 red[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  const int64_t t0 = (int64_t)blockIdx.y * RANGE_ROWS;
  float lo = INFINITY, hi = -INFINITY;
  if (c < C)
    for (int64_t tb = t0 + w * 8; tb < t0 + RANGE_ROWS && tb < T; tb += 32) {  // 8 rows' loads at a time
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = tb + e < T ? bf16_to_f32(h[(tb + e) * C + c]) : v[0];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        lo = fminf(lo, v[e]);
        hi = fmaxf(hi, v[e]);
      }
    }
  red[w][lane] = make_float2(lo, hi);
  __syncthreads();
  if (w == 0 && c < C) {
    for (int k = 1; k < 4; ++k) {
      lo = fminf(lo, red[k][lane].x);
      hi = fmaxf(hi, red[k][lane].y);
    }
    rng_part[(int64_t)blockIdx.y * C + c] = make_float2(lo, hi);
  }
}

// One thread per (component, table bin): the bin's degree-7 Chebyshev interpolant of g in
// power form, tab[c][b][0..7] (tau = 2 (h - lo) / bw - 2b - 1, bw the table-bin width),
// from exact g (device erff/expf) at the nodes tau_k = cos((2k+1) pi / 16); and
// rng[c] = (lo, 1 / bw, bw, flag), flag = 1 when some |w_in_j| * 2 bw > GATE_DZ_MAX.
__global__ __launch_bounds__(256) void k_gate_table(const float2* __restrict__ rng_part, int nchunk, int64_t C,
                                                    const float* __restrict__ w_in, const float* __restrict__ b_in,
                                                    const float* __restrict__ w_out, const float* __restrict__ b_out,
                                                    float* __restrict__ tab, float4* __restrict__ rng) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= C * GATE_TBINS) return;
  const int64_t c = idx / GATE_TBINS;
  const int b = (int)(idx % GATE_TBINS);
  float lo = INFINITY, hi = -INFINITY;
  for (int i = 0; i < nchunk; ++i) {
    const float2 r = rng_part[(int64_t)i * C + c];
    lo = fminf(lo, r.x);
    hi = fmaxf(hi, r.y);
  }
  const float bw = fmaxf((hi - lo) / GATE_TBINS, 4e-6f * fmaxf(fabsf(lo), 1.f));
  float wi[16], bi[16], wo[16], wmax = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    wi[j] = w_in[c * 16 + j];
    bi[j] = b_in[c * 16 + j];
    wo[j] = w_out[c * 16 + j];
    wmax = fmaxf(wmax, fabsf(wi[j]));
  }
  // Chebyshev coefficients cm[m] = (2/8) sum_k g(x_k) T_m(x_k), cm[0] halved
  double cm[GATE_NC] = {};
  for (int k = 0; k < GATE_NC; ++k) {
    const float xk = kChebNode[k];
    const float hk = lo + bw * ((float)b + 0.5f + 0.5f * xk);
    float g = b_out[c];
#pragma unroll
    for (int j = 0; j < 16; ++j) g = fmaf(wo[j], gelu_and_grad<true>(fmaf(wi[j], hk, bi[j])).gelu, g);
    double t0 = 1.0, t1 = xk;
    cm[0] += g;
    cm[1] += (double)g * t1;
    for (int m = 2; m < GATE_NC; ++m) {
      const double t2 = 2.0 * xk * t1 - t0;
      cm[m] += (double)g * t2;
      t0 = t1;
      t1 = t2;
    }
  }
  // power form: sum_m cm[m] T_m(tau), T_m's coefficients by T_{m+1} = 2 tau T_m - T_{m-1}
  double a[GATE_NC] = {}, t0[GATE_NC] = {1.0}, t1[GATE_NC] = {0.0, 1.0};
  for (int m = 0; m < GATE_NC; ++m) {
    const double cmm = cm[m] * (m == 0 ? 0.125 : 0.25);
    const double* tm = m == 0 ? t0 : t1;
    for (int i = 0; i < GATE_NC; ++i) a[i] += cmm * tm[i];
    if (m >= 1) {
      double t2[GATE_NC];
      for (int i = 0; i < GATE_NC; ++i) t2[i] = (i > 0 ? 2.0 * t1[i - 1] : 0.0) - t0[i];
      for (int i = 0; i < GATE_NC; ++i) {
        t0[i] = t1[i];
        t1[i] = t2[i];
      }
    }
  }
  for (int i = 0; i < GATE_NC; ++i) tab[idx * GATE_NC + i] = (float)a[i];
  if (b == 0) rng[c] = make_float4(lo, 1.f / bw, bw, wmax * 2.f * bw > GATE_DZ_MAX ? 1.f : 0.f);
}

// Table bin and coordinate of h: s = (h - lo) / bw in [0, GATE_TBINS], b = floor(s)
// clamped, tau = 2 (s - b) - 1.
struct GateCoord {
  float s, tau;
  int b;
};
__device__ inline GateCoord gate_coord(float hv, float4 rg) {
  const float s = (hv - rg.x) * rg.y;
  const int b = min(max((int)s, 0), GATE_TBINS - 1);
  return {s, fmaf(2.f, s - (float)b, -1.f), b};
}

// g and dg/dtau from a table bin's power-form coefficients a0 = (a_0..a_3), a1 = (a_4..a_7)
// (Horner; the forward uses only g, which this one code path gives bit for bit in both
// passes).
__device__ inline float2 gate_poly(float4 a0, float4 a1, float tau) {
  // Horner for p, with the derivative carried along (d <- d tau + p before each step)
  float g = a1.w, d = a1.w;
  g = fmaf(g, tau, a1.z);
  d = fmaf(d, tau, g);
  g = fmaf(g, tau, a1.y);
  d = fmaf(d, tau, g);
  g = fmaf(g, tau, a1.x);
  d = fmaf(d, tau, g);
  g = fmaf(g, tau, a0.w);
  d = fmaf(d, tau, g);
  g = fmaf(g, tau, a0.z);
  d = fmaf(d, tau, g);
  g = fmaf(g, tau, a0.y);
  d = fmaf(d, tau, g);
  g = fmaf(g, tau, a0.x);
  return make_float2(g, d);
}

// A component's 49 gate weights at stride `st` (w_in[16], b_in[16], w_out[16], b_out).
__device__ inline void gate_weights_load(int64_t c, const float* __restrict__ w_in, const float* __restrict__ b_in,
                                         const float* __restrict__ w_out, const float* __restrict__ b_out, float* w,
                                         int st) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    w[j * st] = w_in[c * 16 + j];
    w[(16 + j) * st] = b_in[c * 16 + j];
    w[(32 + j) * st] = w_out[c * 16 + j];
  }
  w[48 * st] = b_out[c];
}

// The exact gate of a flagged component (device erff/expf GELU) from its weights at stride
// st, shared by both binned passes: returns g, sets gp = dg/dh and go[j] = (GELU,
// GELU')(z_j).
__device__ inline float gate_exact(const float* w, int st, float hv, GeluOut* go, float& gp) {
  float g = w[48 * st];
  gp = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float wi = w[j * st], wo = w[(32 + j) * st];
    go[j] = gelu_and_grad<true>(fmaf(wi, hv, w[(16 + j) * st]));
    g = fmaf(wo, go[j].gelu, g);
    gp = fmaf(wo * wi, go[j].grad, gp);
  }
  return g;
}

// Moment slot q = 8 mb + m of lane l in a wave's region: float4 (2 mb + m / 4) of lane l,
// component m % 4 (lane-contiguous 16-byte slots, so a wave's accesses are conflict-free
// whatever the lanes' bins).
__device__ inline int mom_index(int q, int lane) { return (((q >> 3) * 2 + ((q >> 2) & 1)) * 64 + lane) * 4 + (q & 3); }

// The bf16 forward with the binned gate: block = 64 components x (FWD_WAVES * 64) tokens;
// the 64 components' tables sit in LDS as lt[2b + half][lane] (16-byte slots, so a wave's
// reads are conflict-free whatever the lanes' bins); each wave walks 64 consecutive
// tokens, one component per lane. Otherwise as k_step_fwd; g is not stored (the backward
// recomputes it from the same table).
__global__ __launch_bounds__(64 * FWD_WAVES) void k_step_fwd_tab(
    const bf16_t* __restrict__ h, const float4* __restrict__ tab, const float4* __restrict__ rng,
    const float* __restrict__ w_in, const float* __restrict__ b_in, const float* __restrict__ w_out,
    const float* __restrict__ b_out, StepParams s, bf16_t* __restrict__ acts, float* __restrict__ imp_partial) {
  __shared__ float4 lt[GATE_TBINS * 2 * 64];
  __shared__ float wl[49 * 64];  // the components' gate weights, for flagged ones
  __shared__ float red[FWD_WAVES];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * 64;
  const int nc = (int)(s.C - c0 < 64 ? s.C - c0 : 64);
  for (int i = threadIdx.x; i < 64 * GATE_TBINS * 2; i += blockDim.x)
    if ((i & 63) < nc) lt[i] = tab[(c0 + (i & 63)) * GATE_TBINS * 2 + (i >> 6)];
  if (w == 0 && lane < nc) gate_weights_load(c0 + lane, w_in, b_in, w_out, b_out, wl + lane, 64);
  __syncthreads();
  const int64_t c = c0 + lane;
  const int64_t r0 = ((int64_t)blockIdx.y * FWD_WAVES + w) * 64;
  const int64_t r1 = r0 + 64 < s.T ? r0 + 64 : s.T;
  float imp = 0.f, col = 0.f;
  if (c < s.C && r0 < s.T) {
    const float4 rg = rng[c];
    const bool exact = rg.w != 0.f;
    const int64_t n = s.T * s.C;
    // 8 tokens per step: their h loads go out together, then the 8 elements are computed
    for (int64_t t8 = r0; t8 < r1; t8 += 8) {
      float hv8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) hv8[e] = bf16_to_f32(h[(t8 + e) * s.C + c]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t t = t8 + e, i = t * s.C + c;
        const float hv = hv8[e];
        const GateCoord q = gate_coord(hv, rg);
        float g = gate_poly(lt[(2 * q.b) * 64 + lane], lt[(2 * q.b + 1) * 64 + lane], q.tau).x;
        if (exact) {
          GeluOut go[16];
          float gp;
          g = gate_exact(wl + lane, 64, hv, go, gp);
        }
        const float lo = lower_fwd(g);
        const float iv = step_imp(s, upper_fwd(g));
        imp += iv;
        col += iv;
        const float u = step_uniform_fwd(s, i, n);
        const float m = lo + (1.f - lo) * u;
        acts[i] = f32_to_bf16(hv * (m - step_delta(s, t)));
      }
    }
    if (s.sl0) s.colpart[(r0 / 64) * s.C + c] = col;
  }
  imp = wave_sum(imp);
  if (lane == 0) red[w] = imp;
  __syncthreads();
  if (threadIdx.x == 0) {
    float sum = 0.f;
    for (int k = 0; k < FWD_WAVES; ++k) sum += red[k];
    imp_partial[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = sum;
  }
}

// Recon residual on a 64x64 tile: e = y + d*yt - yt; partial of e^2; dy = gscale*e.
template <typename T>
__global__ __launch_bounds__(256) void k_step_recon(const T* __restrict__ y, const T* __restrict__ yt, StepParams s,
                                                    int64_t D, float gscale, T* __restrict__ dy,
                                                    float* __restrict__ partial) {
  __shared__ float sw[4];
  const int64_t r0 = (int64_t)blockIdx.y * TP, c0 = (int64_t)blockIdx.x * TP;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  float acc = 0.f;
  for (int i = ty; i < TP; i += 4) {
    int64_t t = r0 + i, c = c0 + tx;
    if (t < s.T && c < D) {
      const int64_t idx = t * D + c;
      const float tv = load_f<T>(yt, idx);
      const float e = load_f<T>(y, idx) + step_delta(s, t) * tv - tv;
      acc = fmaf(e, e, acc);
      store_f<T>(dy, idx, gscale * e);
    }
  }
  acc = wave_sum(acc);
  if (tx == 0) sw[ty] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partial[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = sw[0] + sw[1] + sw[2] + sw[3];
}

// Backward, one component per lane: from da = dy@U^T, h, g_raw and the regenerated u:
// dh = da*(m-d) + gate pullback of dg_raw, where dg_raw = lower_vjp(g, da*h*(1-u))
// + upper_vjp(g, imp_scale * d upper^p). Writes dh [T, C]; gate parameter grads go to
// per-chunk partials [chunk][49][C].
template <typename T, bool PRECISE>
__global__ __launch_bounds__(SITE_COLS) void k_step_bwd(const T* __restrict__ da, const T* __restrict__ h,
                                                        const float* __restrict__ g_raw,
                                                        const float* __restrict__ w_in,
                                                        const float* __restrict__ b_in,
                                                        const float* __restrict__ w_out, StepParams s,
                                                        T* __restrict__ dh, float* __restrict__ partial) {
  const int64_t c = (int64_t)blockIdx.x * SITE_COLS + threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * SITE_ROWS;
  const int64_t r1 = r0 + SITE_ROWS < s.T ? r0 + SITE_ROWS : s.T;
  if (c < s.C) {
    float wi[16], bi[16], wo[16], a_wi[16], a_bi[16], a_wo[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      wi[j] = w_in[c * 16 + j];
      bi[j] = b_in[c * 16 + j];
      wo[j] = w_out[c * 16 + j];
      a_wi[j] = a_bi[j] = a_wo[j] = 0.f;
    }
    float a_bo = 0.f;
    const int64_t n = s.T * s.C;
    for (int64_t t = r0; t < r1; ++t) {
      const int64_t i = t * s.C + c;
      const float hv = load_f<T>(h, i), g = g_raw[i], dav = load_f<T>(da, i);
      const float lo = lower_fwd(g);
      const float u = step_uniform_bwd(s, i, n);
      const float m = lo + (1.f - lo) * u;
      float dhv = dav * (m - step_delta(s, t));
      const float dg = lower_vjp(g, dav * hv * (1.f - u)) + upper_vjp(g, step_dimp(s, c, upper_fwd(g)));
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        GeluOut go = gelu_and_grad<PRECISE>(fmaf(wi[j], hv, bi[j]));
        const float dz = dg * wo[j] * go.grad;
        dhv = fmaf(dz, wi[j], dhv);
        a_wi[j] = fmaf(dz, hv, a_wi[j]);
        a_bi[j] += dz;
        a_wo[j] = fmaf(dg, go.gelu, a_wo[j]);
      }
      a_bo += dg;
      store_f<T>(dh, i, dhv);
    }
    float* pp = partial + (int64_t)blockIdx.y * 49 * s.C;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      pp[(int64_t)j * s.C + c] = a_wi[j];
      pp[(int64_t)(16 + j) * s.C + c] = a_bi[j];
      pp[(int64_t)(32 + j) * s.C + c] = a_wo[j];
    }
    pp[(int64_t)48 * s.C + c] = a_bo;
  }
}

// The bf16 backward with the binned gate. Block = BWD_COLS components x BWD_BLOCK_ROWS
// tokens in BWD_WAVES waves; lane l of wave w takes component l % 32 and token stream
// 2w + l / 32 (BWD_ROWS consecutive tokens). Per element: g and dg/dh from the table
// (exactly, for a flagged component), the squashing pullback dg, dh = da (m - d) + dg g'
// written token-major, and dg T_m(tau_m), m < 8, added into the lane's own LDS slots of its
// moment bin mb (two 16-byte read-add-writes; one writer per slot and LDS operations of a
// wave run in order, so the sums are deterministic). A flagged component's lanes keep the
// 49 exact gate-parameter sums in registers and store them into their first 49 slots at
// the end. The block then adds its 8 streams per slot in a fixed order: partial[row
// block][q][c], q < GATE_MOM. LDS: the 32 components' tables (32 KB) and the 4 waves'
// slots (128 KB).
__global__ __launch_bounds__(64 * BWD_WAVES) void k_step_bwd_tab(
    const bf16_t* __restrict__ da, const bf16_t* __restrict__ h, const float4* __restrict__ tab,
    const float4* __restrict__ rng, const float* __restrict__ w_in, const float* __restrict__ b_in,
    const float* __restrict__ w_out, const float* __restrict__ b_out, StepParams s, bf16_t* __restrict__ dh,
    float* __restrict__ partial) {
  __shared__ float4 lt[GATE_TBINS * 2 * BWD_COLS];
  __shared__ float4 mom[BWD_WAVES * GATE_MOM / 4 * 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, cl = lane & (BWD_COLS - 1);
  // XCD-aware block order: workgroups go to the 8 XCDs round-robin by linear id, so the
  // 4 component groups that share 128-byte lines of h, da (2 groups) and the u bytes (4)
  // are given 4 consecutive workgroups of one XCD, which then reads each line into its L2
  // once.
  const unsigned nbx = gridDim.x, nb = gridDim.x * gridDim.y, p = blockIdx.y * nbx + blockIdx.x;
  const unsigned lb = (nb % 32 == 0 && nbx % 4 == 0) ? (p / 8 / 4) * 32 + (p % 8) * 4 + (p / 8) % 4 : p;
  const unsigned bx = lb % nbx, by = lb / nbx;
  const int64_t c0 = (int64_t)bx * BWD_COLS, c = c0 + cl;
  const int nc = (int)(s.C - c0 < BWD_COLS ? s.C - c0 : BWD_COLS);
  for (int i = threadIdx.x; i < BWD_COLS * GATE_TBINS * 2; i += blockDim.x)
    if ((i & (BWD_COLS - 1)) < nc) lt[i] = tab[(c0 + (i & (BWD_COLS - 1))) * GATE_TBINS * 2 + i / BWD_COLS];
  float4* my = mom + w * (GATE_MOM / 4) * 64 + lane;
  for (int q = 0; q < GATE_MOM / 4; ++q) my[q * 64] = make_float4(0.f, 0.f, 0.f, 0.f);
  __syncthreads();
  const int64_t r0 = (int64_t)by * BWD_BLOCK_ROWS + (2 * w + (lane >> 5)) * BWD_ROWS;
  const int64_t r1 = r0 + BWD_ROWS < s.T ? r0 + BWD_ROWS : s.T;
  if (c < s.C && r0 < s.T) {
    const float4 rg = rng[c];
    const bool exact = rg.w != 0.f;
    const float dtau_dh = 2.f * rg.y;
    const bool ubyte = s.draw_dtype == PD_DTYPE_BF16;
    const int64_t n = s.T * s.C;
    // Loads of 8 tokens; the next 8 tokens' loads are issued before this step's
    // arithmetic (the last step reloads its own rows).
    float hv8[8], da8[8], d8[8];
    uint32_t ub8[8];
    auto load8 = [&](int64_t t8, float* hv, float* dv, float* dl, uint32_t* ub) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t i = (t8 + e) * s.C + c;
        hv[e] = bf16_to_f32(h[i]);
        dv[e] = bf16_to_f32(da[i]);
        dl[e] = step_delta(s, t8 + e);
        ub[e] = ubyte ? (uint32_t)s.ubits[i] : 0u;
      }
    };
    load8(r0, hv8, da8, d8, ub8);
    for (int64_t t8 = r0; t8 < r1; t8 += 8) {
      float hn[8], dn[8], dln[8];
      uint32_t ubn[8];
      load8(t8 + 8 < r1 ? t8 + 8 : t8, hn, dn, dln, ubn);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int64_t t = t8 + e, i = t * s.C + c;
        const float hv = hv8[e], dav = da8[e];
        const GateCoord q = gate_coord(hv, rg);
        const float2 gd = gate_poly(lt[(2 * q.b) * BWD_COLS + cl], lt[(2 * q.b + 1) * BWD_COLS + cl], q.tau);
        const float g = gd.x, gp = gd.y * dtau_dh;
        const float lo = lower_fwd(g);
        float u;
        if (ubyte)
          u = (float)ub8[e] * (1.f / 128.f);
        else
          u = draw_uniform(s.mk0, s.mk1, i, n, s.draw_dtype, s.layout);
        const float m = lo + (1.f - lo) * u;
        const float dg = lower_vjp(g, dav * hv * (1.f - u)) + upper_vjp(g, step_dimp(s, c, upper_fwd(g)));
        dh[i] = f32_to_bf16(fmaf(dg, gp, dav * (m - d8[e])));  // a flagged lane rewrites it below
        if (!exact) {
          // moment bin mb = b / 2 and its coordinate tau_m = s - 2 mb - 1 in [-1, 1]
          const int mb = q.b >> 1;
          const float tm = q.s - (float)(2 * mb) - 1.f, t2 = tm + tm;
          float p[GATE_NC];
          p[0] = dg;
          p[1] = dg * tm;
#pragma unroll
          for (int k = 2; k < GATE_NC; ++k) p[k] = fmaf(t2, p[k - 1], -p[k - 2]);
          float4* slot = my + (2 * mb) * 64;
          float4 a = slot[0], b = slot[64];
          a.x += p[0];
          a.y += p[1];
          a.z += p[2];
          a.w += p[3];
          b.x += p[4];
          b.y += p[5];
          b.z += p[6];
          b.w += p[7];
          slot[0] = a;
          slot[64] = b;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        hv8[e] = hn[e];
        da8[e] = dn[e];
        d8[e] = dln[e];
        ub8[e] = ubn[e];
      }
    }
    if (exact) {
      // flagged component: the exact gate, element by element, rewriting dh, with the 49
      // gate-parameter sums in registers, stored into the lane's first 49 slots
      float wv[49], acc[49];
      gate_weights_load(c, w_in, b_in, w_out, b_out, wv, 1);
#pragma unroll
      for (int k = 0; k < 49; ++k) acc[k] = 0.f;
      for (int64_t t = r0; t < r1; ++t) {
        const int64_t i = t * s.C + c;
        const float hv = bf16_to_f32(h[i]), dav = bf16_to_f32(da[i]);
        GeluOut go[16];
        float gp;
        const float g = gate_exact(wv, 1, hv, go, gp);
        const float lo = lower_fwd(g);
        const float u = step_uniform_bwd(s, i, n);
        const float m = lo + (1.f - lo) * u;
        const float dg = lower_vjp(g, dav * hv * (1.f - u)) + upper_vjp(g, step_dimp(s, c, upper_fwd(g)));
        dh[i] = f32_to_bf16(fmaf(dg, gp, dav * (m - step_delta(s, t))));
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float dz = dg * wv[32 + j] * go[j].grad;
          acc[j] = fmaf(dz, hv, acc[j]);
          acc[16 + j] += dz;
          acc[32 + j] = fmaf(dg, go[j].gelu, acc[32 + j]);
        }
        acc[48] += dg;
      }
      float* mf = (float*)(mom + w * (GATE_MOM / 4) * 64);
#pragma unroll
      for (int k = 0; k < 49; ++k) mf[mom_index(k, lane)] = acc[k];
    }
  }
  __syncthreads();
  // float4 f of a lane's region holds slots 4f .. 4f+3
  for (int i = threadIdx.x; i < GATE_MOM / 4 * BWD_COLS; i += blockDim.x) {
    const int f = i / BWD_COLS, cc = i % BWD_COLS;
    if (cc < nc) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int ww = 0; ww < BWD_WAVES; ++ww) {
        const float4* r = mom + (ww * (GATE_MOM / 4) + f) * 64;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const float4 a = r[cc + 32 * half];
          v.x += a.x;
          v.y += a.y;
          v.z += a.z;
          v.w += a.w;
        }
      }
      float* dst = partial + ((int64_t)by * GATE_MOM + 4 * f) * s.C + c0 + cc;
      dst[0] = v.x;
      dst[s.C] = v.y;
      dst[2 * s.C] = v.z;
      dst[3 * s.C] = v.w;
    }
  }
}

// Gate-parameter gradients from the binned backward's slots. Block = FIN_COLS components;
// thread = (component, hidden unit j, node quarter). Slots are summed over the row blocks
// in order. A flagged component's slots hold its exact sums. Otherwise slot (mb, m) holds
// the Chebyshev moment M_m of moment bin mb; its node weights w_k make 128 virtual tokens
// (h_v, w_v), and each thread takes the exact pullback (GELU with the A&S 7.1.26 erf,
// |error| <= 1.5e-7) of the 32 in its quarter; the quarters are added in order. db_out =
// sum over bins of M_0 = sum_t dg_t.
static constexpr int FIN_COLS = 4;
__global__ __launch_bounds__(256) void k_gate_finalize(const float* __restrict__ partial, int64_t nchunk, int64_t C,
                                                       const float4* __restrict__ rng, const float* __restrict__ w_in,
                                                       const float* __restrict__ b_in, const float* __restrict__ w_out,
                                                       float* __restrict__ dw_in, float* __restrict__ db_in,
                                                       float* __restrict__ dw_out, float* __restrict__ db_out) {
  __shared__ float M[FIN_COLS][GATE_MOM];
  __shared__ float Wt[FIN_COLS][GATE_MOM];
  __shared__ float red[FIN_COLS][16][4][3];
  // XCD-aware block order: the 8 blocks whose components share 128-byte lines of the
  // slots are 8 consecutive workgroups of one XCD (workgroups go to XCDs round-robin)
  const unsigned nb = gridDim.x, p = blockIdx.x;
  const unsigned lb = nb % 64 == 0 ? (p / 8 / 8) * 64 + (p % 8) * 8 + (p / 8) % 8 : p;
  const int64_t c0 = (int64_t)lb * FIN_COLS;
  for (int i = threadIdx.x; i < FIN_COLS * GATE_MOM; i += blockDim.x) {
    const int cc = i % FIN_COLS, q = i / FIN_COLS;
    M[cc][q] = c0 + cc < C ? pd_ordered_sum(partial + (int64_t)q * C + c0 + cc, nchunk, (int64_t)GATE_MOM * C) : 0.f;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < FIN_COLS * GATE_MOM; i += blockDim.x) {
    const int cc = i / GATE_MOM, v = i % GATE_MOM, mb = v / GATE_NC, k = v % GATE_NC;
    const float* mm = &M[cc][mb * GATE_NC];
    const float xk = kChebNode[k];
    float t0 = 1.f, t1 = xk, acc = fmaf(xk, mm[1], 0.5f * mm[0]);
#pragma unroll
    for (int m = 2; m < GATE_NC; ++m) {
      const float t2 = fmaf(2.f * xk, t1, -t0);
      acc = fmaf(t2, mm[m], acc);
      t0 = t1;
      t1 = t2;
    }
    Wt[cc][v] = 0.25f * acc;
  }
  __syncthreads();
  const int cc = threadIdx.x >> 6, j = (threadIdx.x >> 2) & 15, qq = threadIdx.x & 3;
  const int64_t c = c0 + cc;
  const bool live = c < C;
  const float4 rg = live ? rng[c] : make_float4(0.f, 0.f, 0.f, 0.f);
  float a_wi = 0.f, a_bi = 0.f, a_wo = 0.f;
  if (live && rg.w == 0.f) {
    const float wi = w_in[c * 16 + j], bi = b_in[c * 16 + j], wo = w_out[c * 16 + j];
    const float lo = rg.x, bwm = 2.f * rg.z;
    for (int v = qq * (GATE_MOM / 4); v < (qq + 1) * (GATE_MOM / 4); ++v) {
      const int mb = v / GATE_NC, k = v % GATE_NC;
      const float hv = lo + bwm * ((float)mb + 0.5f + 0.5f * kChebNode[k]);
      const float wt = Wt[cc][v];
      const GeluOut go = gelu_and_grad<false>(fmaf(wi, hv, bi));
      const float dz = wt * wo * go.grad;
      a_wi = fmaf(dz, hv, a_wi);
      a_bi += dz;
      a_wo = fmaf(wt, go.gelu, a_wo);
    }
  }
  red[cc][j][qq][0] = a_wi;
  red[cc][j][qq][1] = a_bi;
  red[cc][j][qq][2] = a_wo;
  __syncthreads();
  if (!live || qq != 0) return;
  if (rg.w != 0.f) {
    a_wi = M[cc][j];
    a_bi = M[cc][16 + j];
    a_wo = M[cc][32 + j];
  } else {
    a_wi = ((red[cc][j][0][0] + red[cc][j][1][0]) + red[cc][j][2][0]) + red[cc][j][3][0];
    a_bi = ((red[cc][j][0][1] + red[cc][j][1][1]) + red[cc][j][2][1]) + red[cc][j][3][1];
    a_wo = ((red[cc][j][0][2] + red[cc][j][1][2]) + red[cc][j][2][2]) + red[cc][j][3][2];
  }
  dw_in[c * 16 + j] = a_wi;
  db_in[c * 16 + j] = a_bi;
  dw_out[c * 16 + j] = a_wo;
  if (j == 0) {
    float a_bo = 0.f;
    if (rg.w != 0.f)
      a_bo = M[cc][48];
    else
      for (int mb = 0; mb < GATE_MBINS; ++mb) a_bo += M[cc][mb * GATE_NC];
    db_out[c] = a_bo;
  }
}

__global__ void k_step_gate_reduce(const float* __restrict__ partial, int64_t chunks, int64_t C,
                                   float* __restrict__ dw_in, float* __restrict__ db_in, float* __restrict__ dw_out,
                                   float* __restrict__ db_out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= 49 * C) return;
  const int64_t q = idx / C, c = idx % C;
  const float acc = pd_ordered_sum(partial + idx, chunks, 49 * C);
  if (q < 16)
    dw_in[c * 16 + q] = acc;
  else if (q < 32)
    db_in[c * 16 + q - 16] = acc;
  else if (q < 48)
    dw_out[c * 16 + q - 32] = acc;
  else
    db_out[c] = acc;
}

// losses[0..3] = {loss, recon, activity, frequency} from the partial arrays (one block,
// fixed order): activity = imp_scale * sum(imp_part), frequency = sum(freq_part); with
// fb_part (the EMA estimator's batch penalty) losses[4] = sum(fb_part) over n_freq.
__global__ void k_step_losses(const float* __restrict__ rec_part, int64_t n_rec, const float* __restrict__ imp_part,
                              int64_t n_imp, const float* __restrict__ freq_part, int64_t n_freq,
                              const float* __restrict__ fb_part, double rec_scale, double imp_scale,
                              float recon_coeff, float imp_coeff, float freq_coeff, float* __restrict__ losses) {
  __shared__ double sr[16], si[16], sq[16], sb[16];
  double r = 0.0, m = 0.0, fq = 0.0, fb = 0.0;
  for (int64_t i = threadIdx.x; i < n_rec; i += blockDim.x) r += rec_part[i];
  for (int64_t i = threadIdx.x; i < n_imp; i += blockDim.x) m += imp_part[i];
  for (int64_t i = threadIdx.x; i < n_freq; i += blockDim.x) fq += freq_part[i];
  if (fb_part)
    for (int64_t i = threadIdx.x; i < n_freq; i += blockDim.x) fb += fb_part[i];
  r = wave_sum_d(r);
  m = wave_sum_d(m);
  fq = wave_sum_d(fq);
  fb = wave_sum_d(fb);
  if (threadIdx.x % 64 == 0) {
    sr[threadIdx.x / 64] = r;
    si[threadIdx.x / 64] = m;
    sq[threadIdx.x / 64] = fq;
    sb[threadIdx.x / 64] = fb;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double a = 0, b = 0, q = 0, qb = 0;
    for (int i = 0; i < (int)(blockDim.x / 64); ++i) {
      a += sr[i];
      b += si[i];
      q += sq[i];
      qb += sb[i];
    }
    if (fb_part) losses[4] = (float)qb;
    a *= rec_scale;
    b *= imp_scale;
    losses[0] = (float)(recon_coeff * a + imp_coeff * b + freq_coeff * q);
    losses[1] = (float)a;
    losses[2] = (float)b;
    losses[3] = (float)q;
  }
}

struct StepWorkspace {
  size_t yt, h, graw, acts, y, dy, da, dh, imp, rec, gate, delta, ubits, rng_part, rng, tab, sl0_col, sl0_slope,
      sl0_act, sl0_freq, sl0_fb, total;
};

static StepWorkspace step_layout(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C) {
  const bool bf = dtype == PD_DTYPE_BF16;
  const size_t es = bf ? 2 : 4;
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  StepWorkspace w{};
  size_t o = 0;
  auto take = [&](size_t& field, size_t bytes) {
    field = o;
    o += al(bytes);
  };
  (void)d_in;
  take(w.yt, es * T * d_out);
  take(w.h, es * T * C);
  take(w.graw, bf ? 0 : 4 * T * C);  // the bf16 step recomputes g from the gate table
  take(w.acts, es * T * C);
  take(w.y, es * T * d_out);
  take(w.dy, es * T * d_out);
  take(w.da, es * T * C);
  take(w.dh, es * T * C);
  take(w.imp, 4 * cdiv(T, SITE_ROWS) * cdiv(C, SITE_COLS));
  take(w.rec, 4 * cdiv(T, TP) * cdiv(d_out, TP));
  take(w.gate, bf ? 4 * cdiv(T, BWD_BLOCK_ROWS) * GATE_MOM * C : 4 * cdiv(T, SITE_ROWS) * 49 * C);
  take(w.delta, 4 * T);
  take(w.ubits, (size_t)T * C);
  take(w.rng_part, 8 * cdiv(T, RANGE_ROWS) * C);
  take(w.rng, 16 * C);
  take(w.tab, 4 * C * GATE_TBINS * GATE_NC);
  take(w.sl0_col, 4 * (size_t)(cdiv(T, 64) + 1) * C);
  take(w.sl0_slope, 4 * (size_t)C);
  take(w.sl0_act, 4 * (size_t)sl0_blocks(1, (int)C));
  take(w.sl0_freq, 4 * (size_t)sl0_blocks(1, (int)C));
  take(w.sl0_fb, 4 * (size_t)sl0_blocks(1, (int)C));
  w.total = o;
  return w;
}

// Phase boundaries recorded into caller events (events may be NULL); the phase order
// is documented at pd_dense_step_timed in the header.
static int dense_step_impl(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H, const void* x,
                           const void* W, const void* V, const void* U, const float* w_in, const float* b_in,
                           const float* w_out, const float* b_out, uint32_t mk0, uint32_t mk1, uint32_t dk0,
                           uint32_t dk1, int use_delta, int draw_dtype, int layout, const ImpSpec& imp,
                           float recon_coeff, float* losses, float* dV, float* dU, float* dw_in, float* db_in,
                           float* dw_out, float* db_out, void* workspace, size_t workspace_bytes, void* stream,
                           void** events) {
#define PD_MARK(i) \
  if (events) hipEventRecord((hipEvent_t)events[i], (hipStream_t)stream)
  if (H != 16) return fail(PD_EUNSUPPORTED, "pd_dense_step: gate hidden width must be 16");
  if (T <= 0 || d_in <= 0 || d_out <= 0 || C <= 0 || !x || !W || !V || !U || !w_in || !b_in || !w_out || !b_out ||
      !losses || !dV || !dU || !dw_in || !db_in || !dw_out || !db_out)
    return fail(PD_EINVAL, "pd_dense_step: bad args");
  if (dtype != PD_DTYPE_F32 && dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, "pd_dense_step: dtype");
  if (draw_dtype != PD_DTYPE_F32 && draw_dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, "pd_dense_step: draw dtype");
  if (int e = check_imp_spec(imp, "pd_dense_step")) return e;
  StepWorkspace L = step_layout(dtype, T, d_in, d_out, C);
  if (!workspace || workspace_bytes < L.total) return fail(PD_EWORKSPACE, "pd_dense_step: workspace too small");
  if (cdiv(T, SITE_ROWS) > 65535 || cdiv(d_in, TP) > 65535 || cdiv(C, TP) > 65535)
    return fail(PD_EUNSUPPORTED, "pd_dense_step: shape too large");
  if (T % 8 != 0) return fail(PD_EUNSUPPORTED, "pd_dense_step: T must be a multiple of 8");
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  void *yt = ws + L.yt, *h = ws + L.h, *acts = ws + L.acts, *y = ws + L.y, *dy = ws + L.dy, *da = ws + L.da,
       *dh = ws + L.dh;
  float* graw = (float*)(ws + L.graw);
  float* imp_part = (float*)(ws + L.imp);
  float* rec_part = (float*)(ws + L.rec);
  float* gate_part = (float*)(ws + L.gate);
  const bool bf = dtype == PD_DTYPE_BF16;
  float* delta = use_delta ? (float*)(ws + L.delta) : nullptr;
  const bool sl0 = imp.kind == PD_IMPMIN_SMOOTH_L0;
  float* sl0_slope = (float*)(ws + L.sl0_slope);
  float* sl0_act = (float*)(ws + L.sl0_act);
  float* sl0_freq = (float*)(ws + L.sl0_freq);
  float* sl0_fb = imp.ema.on() ? (float*)(ws + L.sl0_fb) : nullptr;
  StepParams sp{T, C, mk0, mk1, draw_dtype, layout, imp.p, imp.coeff / (float)T, delta, (uint8_t*)(ws + L.ubits),
                sl0 ? 1 : 0, imp.g2(), imp.psi_scale(), (float*)(ws + L.sl0_col), sl0_slope};
  const dim3 cgrid((unsigned)cdiv(C, SITE_COLS), (unsigned)cdiv(T, SITE_ROWS));
  const dim3 rgrid((unsigned)cdiv(d_out, TP), (unsigned)cdiv(T, TP));
  int rc;
  float4* rng = (float4*)(ws + L.rng);
  float4* tab = (float4*)(ws + L.tab);
  PD_MARK(0);
  if (delta)
    hipLaunchKernelGGL(k_delta_fill, dim3((unsigned)std::min<int64_t>(cdiv(T, 256), 1024)), dim3(256), 0, s, dk0, dk1,
                       T, draw_dtype, layout, delta);
  if ((rc = check_launch("pd_dense_step delta"))) return rc;
  PD_MARK(1);
  if ((rc = pd_gemm(dtype, T, d_out, d_in, x, d_in, 0, W, d_in, 1, yt, d_out, dtype, 1.f, 0.f, stream))) return rc;
  PD_MARK(2);
  if ((rc = pd_gemm(dtype, T, C, d_in, x, d_in, 0, V, C, 0, h, C, dtype, 1.f, 0.f, stream))) return rc;
  PD_MARK(3);
  const dim3 fgrid((unsigned)cdiv(C, 64), (unsigned)cdiv(T, 64 * FWD_WAVES));
  if (bf) {
    float2* rng_part = (float2*)(ws + L.rng_part);
    const int nchunk = (int)cdiv(T, RANGE_ROWS);
    hipLaunchKernelGGL(k_gate_range, dim3((unsigned)cdiv(C, 64), (unsigned)nchunk), dim3(256), 0, s, (const bf16_t*)h,
                       T, C, rng_part);
    hipLaunchKernelGGL(k_gate_table, dim3((unsigned)cdiv(C * GATE_TBINS, 256)), dim3(256), 0, s, rng_part, nchunk, C,
                       w_in, b_in, w_out, b_out, (float*)tab, rng);
    hipLaunchKernelGGL(k_step_fwd_tab, fgrid, dim3(64 * FWD_WAVES), 0, s, (const bf16_t*)h, (const float4*)tab,
                       (const float4*)rng, w_in, b_in, w_out, b_out, sp, (bf16_t*)acts, imp_part);
  } else
    hipLaunchKernelGGL((k_step_fwd<float, true>), cgrid, dim3(SITE_COLS), 0, s, (const float*)h, w_in, b_in, w_out,
                       b_out, sp, graw, (float*)acts, imp_part);
  if (sl0)  // per-component frequencies, loss partials and backward slopes
    hipLaunchKernelGGL(k_sl0_finalize, dim3(sl0_blocks(1, (int)C)), dim3(256), 0, s, sp.colpart,
                       (const int32_t*)nullptr, 1, T, (int)C, 1.f / (float)T, imp.coeff, imp.freq_coeff, imp.ref_count,
                       imp.ema, sl0_slope, sl0_act, sl0_freq, sl0_fb);
  if ((rc = check_launch("pd_dense_step fwd"))) return rc;
  PD_MARK(4);
  if ((rc = pd_gemm(dtype, T, d_out, C, acts, C, 0, U, d_out, 0, y, d_out, dtype, 1.f, 0.f, stream))) return rc;
  PD_MARK(5);
  const float gscale = recon_coeff * 2.f / (float)(T * d_out);
  if (bf)
    hipLaunchKernelGGL(k_step_recon<bf16_t>, rgrid, dim3(256), 0, s, (const bf16_t*)y, (const bf16_t*)yt, sp, d_out,
                       gscale, (bf16_t*)dy, rec_part);
  else
    hipLaunchKernelGGL(k_step_recon<float>, rgrid, dim3(256), 0, s, (const float*)y, (const float*)yt, sp, d_out,
                       gscale, (float*)dy, rec_part);
  if ((rc = check_launch("pd_dense_step recon"))) return rc;
  PD_MARK(6);
  const int64_t n_imp = bf ? (int64_t)fgrid.x * fgrid.y : (int64_t)cgrid.x * cgrid.y;
  const int64_t n_sl0 = sl0_blocks(1, (int)C);
  if (sl0)
    hipLaunchKernelGGL(k_step_losses, dim3(1), dim3(1024), 0, s, rec_part, (int64_t)(rgrid.x * rgrid.y), sl0_act,
                       n_sl0, sl0_freq, imp.ref_count > 0.f ? n_sl0 : (int64_t)0, sl0_fb, 1.0 / (double)(T * d_out), 1.0,
                       recon_coeff, imp.coeff, imp.freq_coeff, losses);
  else
    hipLaunchKernelGGL(k_step_losses, dim3(1), dim3(1024), 0, s, rec_part, (int64_t)(rgrid.x * rgrid.y), imp_part,
                       n_imp, (const float*)nullptr, (int64_t)0, (const float*)nullptr, 1.0 / (double)(T * d_out),
                       1.0 / (double)T,
                       recon_coeff, imp.coeff, 0.f, losses);
  PD_MARK(7);
  if ((rc = pd_gemm(dtype, C, d_out, T, acts, C, 1, dy, d_out, 0, dU, d_out, PD_DTYPE_F32, 1.f, 0.f, stream)))
    return rc;
  PD_MARK(8);
  if ((rc = pd_gemm(dtype, T, C, d_out, dy, d_out, 0, U, d_out, 1, da, C, dtype, 1.f, 0.f, stream))) return rc;
  PD_MARK(9);
  const dim3 bgrid((unsigned)cdiv(C, BWD_COLS), (unsigned)cdiv(T, BWD_BLOCK_ROWS));
  if (bf)
    hipLaunchKernelGGL(k_step_bwd_tab, bgrid, dim3(64 * BWD_WAVES), 0, s, (const bf16_t*)da, (const bf16_t*)h,
                       (const float4*)tab, (const float4*)rng, w_in, b_in, w_out, b_out, sp, (bf16_t*)dh, gate_part);
  else
    hipLaunchKernelGGL((k_step_bwd<float, true>), cgrid, dim3(SITE_COLS), 0, s, (const float*)da, (const float*)h,
                       graw, w_in, b_in, w_out, sp, (float*)dh, gate_part);
  if ((rc = check_launch("pd_dense_step bwd"))) return rc;
  PD_MARK(10);
  if (bf)
    hipLaunchKernelGGL(k_gate_finalize, dim3((unsigned)cdiv(C, FIN_COLS)), dim3(256), 0, s, gate_part, (int64_t)bgrid.y, C,
                       (const float4*)rng, w_in, b_in, w_out, dw_in, db_in, dw_out, db_out);
  else
    hipLaunchKernelGGL(k_step_gate_reduce, dim3((unsigned)cdiv(49 * C, 256)), dim3(256), 0, s, gate_part,
                       (int64_t)cgrid.y, C, dw_in, db_in, dw_out, db_out);
  if ((rc = check_launch("pd_dense_step gate reduce"))) return rc;
  PD_MARK(11);
  if ((rc = pd_gemm(dtype, d_in, C, T, x, d_in, 1, dh, C, 0, dV, C, PD_DTYPE_F32, 1.f, 0.f, stream))) return rc;
  PD_MARK(12);
  return PD_OK;
#undef PD_MARK
}

}  // namespace pd

using namespace pd;

extern "C" {

size_t pd_dense_step_workspace_size(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H) {
  (void)H;
  return step_layout(dtype, T, d_in, d_out, C).total;
}

int pd_dense_step(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H, const void* x, const void* W,
                  const void* V, const void* U, const float* w_in, const float* b_in, const float* w_out,
                  const float* b_out, uint32_t mk0, uint32_t mk1, uint32_t dk0, uint32_t dk1, int use_delta,
                  int draw_dtype, int layout, int imp_kind, float p, float gamma, int normalize_at_one,
                  float imp_coeff, float freq_coeff, float ref_count, const float* freq_ema_in,
                  float* freq_ema_out, float ema_count, float ema_halflife, float recon_coeff, float* losses,
                  float* dV, float* dU, float* dw_in, float* db_in, float* dw_out, float* db_out, void* workspace,
                  size_t workspace_bytes, void* stream) {
  ImpSpec imp;
  if (int e = make_imp_spec("pd_dense_step", imp_kind, p, gamma, normalize_at_one, imp_coeff, freq_coeff, ref_count,
                            freq_ema_in, freq_ema_out, ema_count, ema_halflife, imp))
    return e;
  return dense_step_impl(dtype, T, d_in, d_out, C, H, x, W, V, U, w_in, b_in, w_out, b_out, mk0, mk1, dk0, dk1,
                         use_delta, draw_dtype, layout, imp, recon_coeff, losses, dV, dU, dw_in, db_in, dw_out, db_out,
                         workspace, workspace_bytes, stream, nullptr);
}

int pd_dense_step_timed(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H, const void* x,
                        const void* W, const void* V, const void* U, const float* w_in, const float* b_in,
                        const float* w_out, const float* b_out, uint32_t mk0, uint32_t mk1, uint32_t dk0,
                        uint32_t dk1, int use_delta, int draw_dtype, int layout, int imp_kind, float p, float gamma,
                        int normalize_at_one, float imp_coeff, float freq_coeff, float ref_count,
                        const float* freq_ema_in, float* freq_ema_out, float ema_count, float ema_halflife,
                        float recon_coeff, float* losses, float* dV, float* dU, float* dw_in, float* db_in,
                        float* dw_out, float* db_out, void* workspace, size_t workspace_bytes, void* stream,
                        void** events) {
  if (!events) return fail(PD_EINVAL, "pd_dense_step_timed: events required");
  ImpSpec imp;
  if (int e = make_imp_spec("pd_dense_step_timed", imp_kind, p, gamma, normalize_at_one, imp_coeff, freq_coeff,
                            ref_count, freq_ema_in, freq_ema_out, ema_count, ema_halflife, imp))
    return e;
  return dense_step_impl(dtype, T, d_in, d_out, C, H, x, W, V, U, w_in, b_in, w_out, b_out, mk0, mk1, dk0, dk1,
                         use_delta, draw_dtype, layout, imp, recon_coeff, losses, dV, dU, dw_in, db_in, dw_out, db_out,
                         workspace, workspace_bytes, stream, events);
}

}  // extern "C"
