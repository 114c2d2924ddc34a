// The decomposed MoE stack step (gfx950): L layers of
//   h2 = rms_norm_zero_centered(r)        target_ports/qwen3_5_moe.py:33-41
//   router softmax, top-k, mixing weights pd/targets/qwen36_moe.py:473-514, 2923-2965
//   jobs = stable bucketing by expert     pd/routed/experts.py:115-123
//   decomposed expert sites in job space  pd/targets/qwen36_moe.py:2752-2837
//   r += sum_jobs(down)                   pd/routed/experts.py:202-206
// with the clean forward on the frozen expert weights pinning every masked layer's
// expert indices, stochastic masks drawn per (kind, layer) over the selected-CI values
// (pd/targets/qwen36_moe.py:3374-3401), MSE between masked and clean final residuals,
// L_p imp-min over the selected upper CI, and the full backward (V/U of every site, the
// CI preactivations, through routing weights, router softmax and the norm).
//
// Grouped GEMM operand layouts:
//   forward  out = in @ W[e]      rhs = W^T copies [E, N, K] made once per step (K-contiguous:
//                                  an MN-major rhs measured 6-13% slower per product)
//   d_input  d_in = d_out @ W[e]^T rhs = W in its own layout [E, K_in, N_out]
//   d_weight dW[e] = in^T @ d_out  both operands straight from the row-major job-space
//                                  tensors [J, width], MN-major for the contraction over
//                                  jobs (about 0.13 ms per step slower than K-major copies,
//                                  which would cost ~2.4 GB of extra writes per step)
#include <algorithm>
#include <vector>

#include "pd_common.hpp"
#include "pd_gemm_dtl.hpp"
#include "pd_impmin.hpp"

namespace pd {

static constexpr int MOE_KIND_GATE = 11, MOE_KIND_UP = 12, MOE_KIND_DOWN = 13;  // KIND_ORDER indices
// dst[b] = src[b]^T for B matrices of [R, Cc] (R, Cc multiples of 8).
__global__ __launch_bounds__(256) void k_batched_transpose(const bf16_t* __restrict__ src, int64_t R, int64_t Cc,
                                                           bf16_t* __restrict__ dst) {
  __shared__ TTile T;
  const int64_t b = blockIdx.z;
  const bf16_t* s = src + b * R * Cc;
  const int64_t r0 = (int64_t)blockIdx.y * TILE, c0 = (int64_t)blockIdx.x * TILE;
  const int tid = threadIdx.x, c8 = (tid & 7) * 8;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int r = (tid >> 3) + 32 * pass;
    uint4 v = {0, 0, 0, 0};
    if (r0 + r < R && c0 + c8 < Cc) v = *(const uint4*)(s + (r0 + r) * Cc + c0 + c8);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      T.v[c8 + 2 * e][r] = (bf16_t)(w[e] & 0xFFFFu);
      T.v[c8 + 2 * e + 1][r] = (bf16_t)(w[e] >> 16);
    }
  }
  __syncthreads();
  ttile_store(T, dst + b * R * Cc, R, r0, R, c0, Cc, tid);
}

// Job-space gather: out[j][:] = src[idx[j] / div][:] and/or its job-contiguous copy
// outT[:][j] (w % 8 == 0, J % 8 == 0).
__global__ __launch_bounds__(256) void k_gather_tile(const bf16_t* __restrict__ src, const int32_t* __restrict__ idx,
                                                     int div, int64_t J, int w, bf16_t* __restrict__ out,
                                                     bf16_t* __restrict__ outT) {
  __shared__ TTile T;
  const int64_t j0 = (int64_t)blockIdx.y * TILE;
  const int c0 = blockIdx.x * TILE;
  const int tid = threadIdx.x, c8 = (tid & 7) * 8;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int r = (tid >> 3) + 32 * pass;
    const int64_t j = j0 + r;
    uint4 v = {0, 0, 0, 0};
    if (j < J && c0 + c8 < w) {
      v = *(const uint4*)(src + (int64_t)(idx[j] / div) * w + c0 + c8);
      if (out) *(uint4*)(out + j * w + c0 + c8) = v;
    }
    if (outT) {
      const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        T.v[c8 + 2 * e][r] = (bf16_t)(u[e] & 0xFFFFu);
        T.v[c8 + 2 * e + 1][r] = (bf16_t)(u[e] >> 16);
      }
    }
  }
  if (!outT) return;
  __syncthreads();
  ttile_store(T, outT, J, j0, J, c0, w, tid);
}

// ---------------------------------------------------------------- token-space kernels
// Rows of width d (d % 8 == 0), lane l owning columns 8l..8l+7 of each 512-column chunk.
// y = x * rsqrt(mean x^2 + eps) * (1 + w), fp32 math, bf16 out; rinv saved for the
// backward.
__global__ __launch_bounds__(256) void k_rmsnorm_fwd(const bf16_t* __restrict__ x, int64_t T, int d,
                                                     const float* __restrict__ w, float eps, bf16_t* __restrict__ y,
                                                     float* __restrict__ rinv) {
  const int64_t t = (int64_t)blockIdx.x * 4 + wave_id();
  if (t >= T) return;
  const int lane = threadIdx.x & 63;
  const bf16_t* xr = x + t * d;
  float ss = 0.f;
  for (int i = lane * 8; i < d; i += 512) {
    float v[8];
    load8(xr + i, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(v[j], v[j], ss);
  }
  const float r = rsqrtf(wave_sum(ss) / (float)d + eps);
  if (lane == 0 && rinv) rinv[t] = r;
  for (int i = lane * 8; i < d; i += 512) {
    float v[8], g[8];
    load8(xr + i, v);
    load8f(w + i, g);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = v[j] * r * (1.f + g[j]);
    store8(y + t * d + i, v);
  }
}

// The value v[e >> 6] of lane e & 63 (an expert-e quantity of the lane-strided layout
// lane l <-> experts l + 64 i) for every lane; every lane takes part in the shuffles.
template <int EPL>
__device__ inline float expert_value(const float (&v)[EPL], int e) {
  float out = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const float x = __shfl(v[i], e & 63, 64);
    if ((e >> 6) == i) out = x;
  }
  return out;
}

// Masked-layer routing weights at pinned indices: probs = softmax(bf16(logits))
// (saved), w[t,s] = probs[idx[t,s]] / sum_s probs[idx[t,s]]. The fp32 product is
// rounded to bf16 first: the reference's router product runs in the bf16 matmul dtype
// (pd/targets/qwen36_moe.py:473-475). One wave per token; lane l holds experts
// l + 64 i (E <= 64 EPL).
template <int EPL>
__global__ __launch_bounds__(256) void k_router_pinned(const float* __restrict__ logits, int64_t T, int E, int k,
                                                       const int32_t* __restrict__ idx, float* __restrict__ probs,
                                                       float* __restrict__ w) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  float x[EPL];
  float mxl = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    x[i] = e < E ? bf16_to_f32(f32_to_bf16(logits[t * E + e])) : -INFINITY;
    mxl = fmaxf(mxl, x[i]);
  }
  const float mx = wave_max(mxl);
  float zl = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    x[i] = lane + 64 * i < E ? expf(x[i] - mx) : 0.f;
    zl += x[i];
  }
  const float z = wave_sum(zl);
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    x[i] = x[i] / z;
    if (e < E) probs[t * E + e] = x[i];
  }
  int e = lane < k ? idx[t * k + lane] : 0;
  e = e < 0 ? 0 : (e >= E ? E - 1 : e);
  const float sel = expert_value<EPL>(x, e);
  float s = wave_sum(lane < k ? sel : 0.f);
  if (lane < k) w[t * k + lane] = sel / s;
}

static void launch_router_pinned(const float* logits, int64_t T, int E, int k, const int32_t* idx, float* probs,
                                 float* w, hipStream_t s) {
  const dim3 grid((unsigned)cdiv(T, 4));
  if (E <= 64) hipLaunchKernelGGL(k_router_pinned<1>, grid, dim3(256), 0, s, logits, T, E, k, idx, probs, w);
  else if (E <= 128) hipLaunchKernelGGL(k_router_pinned<2>, grid, dim3(256), 0, s, logits, T, E, k, idx, probs, w);
  else if (E <= 256) hipLaunchKernelGGL(k_router_pinned<4>, grid, dim3(256), 0, s, logits, T, E, k, idx, probs, w);
  else hipLaunchKernelGGL(k_router_pinned<8>, grid, dim3(256), 0, s, logits, T, E, k, idx, probs, w);
}

// r_out[t,:] = bf16(r[t,:] + bf16(sum_s wt[t,s] * y[inv[t*k+s],:])) with fp32
// accumulation in slot order; wt NULL = the unweighted sum_jobs. With the frozen channel
// (yd, delta non-NULL) the routed sum also takes delta[t] * sum_s yd[inv[t*k+s],:]: a
// token's k jobs share its delta draw, so the slot sum of the frozen outputs is scaled
// once (pd/core/decomposed_linear.py:72-85). One wave per token.
__global__ __launch_bounds__(256) void k_combine_residual(const bf16_t* __restrict__ r, const bf16_t* __restrict__ y,
                                                          const int32_t* __restrict__ inv,
                                                          const float* __restrict__ wt, int64_t T, int k, int d,
                                                          const bf16_t* __restrict__ yd,
                                                          const float* __restrict__ delta,
                                                          bf16_t* __restrict__ r_out) {
  const int64_t t = (int64_t)blockIdx.x * 4 + wave_id();
  if (t >= T) return;
  for (int i = (threadIdx.x & 63) * 8; i < d; i += 512) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, v[8];
    for (int s = 0; s < k; ++s) {
      load8(y + (int64_t)inv[t * k + s] * d + i, v);
      if (wt) {
        const float ws = wt[t * k + s];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = fmaf(ws, v[j], acc[j]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += v[j];
      }
    }
    if (yd) {
      float fr[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int s = 0; s < k; ++s) {
        load8(yd + (int64_t)inv[t * k + s] * d + i, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) fr[j] += v[j];
      }
      const float dt = delta[t];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = fmaf(dt, fr[j], acc[j]);
    }
    load8(r + t * d + i, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = v[j] + bf16_to_f32(f32_to_bf16(acc[j]));
    store8(r_out + t * d + i, acc);
  }
}

// MSE between the masked and clean final residuals: partial sums of e^2 and
// dr = bf16(scale * e).
__global__ __launch_bounds__(256) void k_moe_recon(const bf16_t* __restrict__ r, const bf16_t* __restrict__ rc,
                                                   int64_t n, float scale, bf16_t* __restrict__ dr,
                                                   float* __restrict__ partial) {
  float acc = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    float e = bf16_to_f32(r[i]) - bf16_to_f32(rc[i]);
    acc = fmaf(e, e, acc);
    dr[i] = f32_to_bf16(scale * e);
  }
  __shared__ float red[4];
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

// ---------------------------------------------------------------- job-space kernels (64x64 tiles)
struct SiteMaskArgs {
  const bf16_t* ci_pre;  // [T, k, c] token-major (slot m = the token's m-th expert)
  const int32_t* sort_idx;
  int64_t J;
  int c;
  uint32_t k0, k1;
  int layout;
  float p;
  const float* delta;    // [T] the site's per-token delta draw, or NULL (d = 0)
  const uint8_t* route;  // [T] the site's per-token route, or NULL (every token routed)
  int k;                 // experts per token: job j belongs to token sort_idx[j] / k
  float uconst;        // MASK_CONST: the constant source value standing in for u
  // smooth-L0 imp-min (PM_SL0): psi = psis * v^2 / (v^2 + g2); the forward writes the
  // per-(tile, expert) column sums of psi to colpart, the backward reads the per-(expert,
  // component) slope; offsets [E + 1] locate each job's expert
  const int32_t* offsets;
  int E;
  float g2, psis;
  float* colpart;
  const float* slope;
  // persistent source tables (MASK_SRC): src [S, E, c] of this (layer, site), S = T / rps
  // rows of rps consecutive tokens; the backward writes the tables' gradient as
  // per-(tile, group) column sums colsrc (group = expert * S + row, rps > 1) or straight
  // into dsrc [T, E, c] (rps = 1), and each job's per-tile row sums of dm into rowdm
  const void* src;
  int src_dtype;
  int64_t rps, S;
  float* colsrc;
  float* dsrc;
  float* rowdm;
};

// (MASK_CONST: every source value is SiteMaskArgs::uconst. MASK_SRC: a selected value
// reads its expert's row of the table, u = src[(t / rps) E c + e c + q], the reference's
// SourceMaskIngredients, pd/core/masking.py:43-68.)

__device__ inline float job_delta(const SiteMaskArgs& a, int32_t slot) { return a.delta ? a.delta[slot / a.k] : 0.f; }
// An unrouted token's jobs take the frozen output (pd/core/decomposed_linear.py:72-85):
// their component coefficients are 0, so their masks get no recon gradient.
__device__ inline bool job_routed(const SiteMaskArgs& a, int32_t slot) { return !a.route || a.route[slot / a.k]; }

// One row of a 64-row mask tile, looked up once per block by the first wave (instead of
// in every pass of every lane): the job's token-major slot, its token's delta and routed
// flag and, with GROUP, its expert group ej and source-table row (t / rps) E + ej.
struct MaskRow {
  int32_t slot;
  float dt;
  int32_t routed;
  int32_t ej;
  int64_t srow;
};
template <bool GROUP>
__device__ inline void fill_mask_rows(MaskRow* rows, const SiteMaskArgs& a, int64_t j0, int tid) {
  if (tid >= TILE) return;
  const int64_t j = j0 + tid;
  MaskRow v{0, 0.f, 0, 0, 0};
  if (j < a.J) {
    const int32_t slot = a.sort_idx[j], tok = slot / a.k;
    v.slot = slot;
    v.dt = a.delta ? a.delta[tok] : 0.f;
    v.routed = !a.route || a.route[tok] ? 1 : 0;
    if constexpr (GROUP) {
      v.ej = row_group(a.offsets, a.E, j);
      v.srow = ((int64_t)tok / a.rps) * a.E + v.ej;
    }
  }
  rows[tid] = v;
}


// Thread -> (row (tid >> 4) + 16 * pass, columns q4 .. q4 + 3) of a 64x64 job-space tile.
#define PD_TILE4_ROW(pass) ((threadIdx.x >> 4) + 16 * (pass))
#define PD_TILE4_COL ((threadIdx.x & 15) * 4)

// Forward mask: m = lower(ci) + (1 - lower(ci)) u with ci and u taken at the job's
// token-major position sort_idx[j]*c + q (u drawn over [T, k*c] in bf16); acts =
// bf16(h * (m - delta)) (the component coefficients m - d, pd/core/decomposed_linear.py:65-69;
// d = 0 without the frozen channel; 0 on unrouted tokens) written as acts [J,c]; u stored
// as its 7-bit integer; per-block partial of upper(ci)^p. c % 8 == 0, J % 8 == 0.
template <int LAYOUT, int PM>
__global__ __launch_bounds__(256) void k_mask_fwd_tile(SiteMaskArgs a, const bf16_t* __restrict__ h,
                                                       bf16_t* __restrict__ acts, uint8_t* __restrict__ ubits,
                                                       float* __restrict__ imp_partial) {
  __shared__ float red[4];
  __shared__ typename std::conditional<PM == PM_SL0, Sl0Tile, NoSl0Tile>::type SLv;
  __shared__ MaskRow rows[TILE];
  const int tid = threadIdx.x;
  const int64_t j0 = (int64_t)blockIdx.y * TILE;
  const int q0 = blockIdx.x * TILE, q4 = PD_TILE4_COL;
  const int64_t n = a.J * a.c;
  const bool qok = q0 + q4 < a.c;
  if constexpr (PM == PM_SL0) sl0_tile_groups(SLv, a.offsets, a.E, j0, a.J, tid);
  fill_mask_rows<LAYOUT == MASK_SRC>(rows, a, j0, tid);
  __syncthreads();
  float imp = 0.f;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int r = PD_TILE4_ROW(pass);
    const int64_t j = j0 + r;
    bf16_t o[4] = {0, 0, 0, 0};
    if (j < a.J && qok) {
      const int64_t idx = j * a.c + q0 + q4;
      const MaskRow row = rows[r];
      const int32_t slot = row.slot;
      const int64_t src = (int64_t)slot * a.c + q0 + q4;
      const float dt = row.dt;
      const bool routed = row.routed != 0;
      const uint2 pw = *(const uint2*)(a.ci_pre + src);
      const uint2 hw = *(const uint2*)(h + idx);
      const float pre[4] = {bf_lo(pw.x), bf_hi(pw.x), bf_lo(pw.y), bf_hi(pw.y)};
      const float hv[4] = {bf_lo(hw.x), bf_hi(hw.x), bf_lo(hw.y), bf_hi(hw.y)};
      uint32_t ub = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = lower_fwd(pre[e]);
        if constexpr (PM == PM_SL0) SLv.ps[r][q4 + e] = sl0_psi(upper_fwd(pre[e]), a.g2, a.psis);
        else imp += powp<PM>(upper_fwd(pre[e]), a.p);
        float u;
        if constexpr (LAYOUT == MASK_CONST) {
          u = a.uconst;
        } else if constexpr (LAYOUT == MASK_SRC) {
          u = src_value(a.src, a.src_dtype, row.srow * a.c + q0 + q4 + e);
        } else {
          const uint32_t kb = (draw_bits(a.k0, a.k1, src + e, n, 8, LAYOUT) & 0xFFu) >> 1;
          ub |= kb << (8 * e);
          u = (float)kb * (1.f / 128.f);
        }
        o[e] = routed ? f32_to_bf16(hv[e] * (lo + (1.f - lo) * u - dt)) : (bf16_t)0;
      }
      if constexpr (LAYOUT != MASK_CONST && LAYOUT != MASK_SRC) *(uint32_t*)(ubits + idx) = ub;
      *(uint2*)(acts + idx) = make_uint2(bf_pack(o[0], o[1]), bf_pack(o[2], o[3]));
    } else if constexpr (PM == PM_SL0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) SLv.ps[r][q4 + e] = 0.f;
    }
  }
  if constexpr (PM == PM_SL0) {
    __syncthreads();
    sl0_tile_colsums(SLv, blockIdx.y, q0, a.c, a.colpart, tid);
  } else {
    imp = wave_sum(imp);
    if ((tid & 63) == 0) red[tid >> 6] = imp;
    __syncthreads();
    if (tid == 0) imp_partial[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = red[0] + red[1] + red[2] + red[3];
  }
}

// Backward mask: d_h = bf16(d_acts * (m - delta)) (in place over d_acts) and the
// CI pullback d_pre[sort_idx[j]*c + q] = lower_vjp(pre, d_acts*h*(1-u)) +
// upper_vjp(pre, imp_scale * d upper^p), written token-major; d_acts counts as 0 on an
// unrouted token's jobs.
// SRC: the sources are tables (MASK_SRC): u is read back from the table, and the tables'
// gradient dm (1 - lower) (dm = d_acts h) and each job's row sums of dm are written.
template <int PM, bool SRC>
__global__ __launch_bounds__(256) void k_mask_bwd_tile(SiteMaskArgs a, const bf16_t* __restrict__ h,
                                                       const uint8_t* __restrict__ ubits, float imp_scale,
                                                       bf16_t* __restrict__ d_acts, bf16_t* __restrict__ d_pre) {
  __shared__ typename std::conditional<SRC, Sl0Tile, NoSl0Tile>::type SG;
  __shared__ MaskRow rows[TILE];
  const int tid = threadIdx.x;
  const int64_t j0 = (int64_t)blockIdx.y * TILE;
  const int q0 = blockIdx.x * TILE, q4 = PD_TILE4_COL;
  const bool qok = q0 + q4 < a.c;
  if constexpr (SRC) {
    if (tid < 64) {  // each row's (expert, source row) group; rows are sorted by it
      const int64_t j = j0 + tid;
      SG.grp[tid] = j < a.J ? row_group(a.offsets, a.E, j) * (int)a.S + (int)((a.sort_idx[j] / a.k) / a.rps) : -1;
    }
  }
  fill_mask_rows<SRC || PM == PM_SL0>(rows, a, j0, tid);
  __syncthreads();
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int r = PD_TILE4_ROW(pass);
    const int64_t j = j0 + r;
    bf16_t o[4] = {0, 0, 0, 0};
    float dmsum = 0.f;
    if (j < a.J && qok) {
      const int64_t idx = j * a.c + q0 + q4;
      const MaskRow row = rows[r];
      const int32_t slot = row.slot;
      const int64_t src = (int64_t)slot * a.c + q0 + q4;
      const float dt = row.dt;
      const uint2 pw = *(const uint2*)(a.ci_pre + src);
      const uint2 hw = *(const uint2*)(h + idx);
      const uint2 dw = row.routed ? *(const uint2*)(d_acts + idx) : make_uint2(0u, 0u);
      const uint32_t ub = !SRC && a.uconst < 0.f ? *(const uint32_t*)(ubits + idx) : 0u;
      const float pre[4] = {bf_lo(pw.x), bf_hi(pw.x), bf_lo(pw.y), bf_hi(pw.y)};
      const float hv[4] = {bf_lo(hw.x), bf_hi(hw.x), bf_lo(hw.y), bf_hi(hw.y)};
      const float da[4] = {bf_lo(dw.x), bf_hi(dw.x), bf_lo(dw.y), bf_hi(dw.y)};
      bf16_t dp[4];
      float slope4[4] = {imp_scale, imp_scale, imp_scale, imp_scale};
      if constexpr (PM == PM_SL0) {
        const float4 sl = *(const float4*)(a.slope + (int64_t)row.ej * a.c + q0 + q4);
        slope4[0] = sl.x;
        slope4[1] = sl.y;
        slope4[2] = sl.z;
        slope4[3] = sl.w;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = lower_fwd(pre[e]), up = upper_fwd(pre[e]);
        float u;
        if constexpr (SRC) u = src_value(a.src, a.src_dtype, row.srow * a.c + q0 + q4 + e);
        else u = a.uconst < 0.f ? (float)((ub >> (8 * e)) & 0xFFu) * (1.f / 128.f) : a.uconst;
        const float m = lo + (1.f - lo) * u - dt;
        float dimp;
        if constexpr (PM == PM_SL0) dimp = slope4[e] * sl0_dpsi(up, a.g2, a.psis);
        else dimp = imp_scale * dpowp<PM>(up, a.p);
        const float dm = da[e] * hv[e];
        dp[e] = f32_to_bf16(lower_vjp(pre[e], dm * (1.f - u)) + upper_vjp(pre[e], dimp));
        o[e] = f32_to_bf16(da[e] * m);
        if constexpr (SRC) {
          dmsum += dm;
          const float gs = dm * (1.f - lo);
          if (a.rps == 1) a.dsrc[row.srow * a.c + q0 + q4 + e] = gs;
          else SG.ps[r][q4 + e] = gs;
        }
      }
      *(uint2*)(d_pre + src) = make_uint2(bf_pack(dp[0], dp[1]), bf_pack(dp[2], dp[3]));
      *(uint2*)(d_acts + idx) = make_uint2(bf_pack(o[0], o[1]), bf_pack(o[2], o[3]));
    } else if constexpr (SRC) {
#pragma unroll
      for (int e = 0; e < 4; ++e) SG.ps[r][q4 + e] = 0.f;
    }
    if constexpr (SRC) {  // the 16 lanes of a row add their columns in a fixed tree (all lanes)
      dmsum += __shfl_xor(dmsum, 1, 64);
      dmsum += __shfl_xor(dmsum, 2, 64);
      dmsum += __shfl_xor(dmsum, 4, 64);
      dmsum += __shfl_xor(dmsum, 8, 64);
      if (j < a.J && (tid & 15) == 0) a.rowdm[j * gridDim.x + blockIdx.x] = dmsum;
    }
  }
  if constexpr (SRC) {
    __syncthreads();
    if (a.rps > 1) sl0_tile_colsums(SG, blockIdx.y, q0, a.c, a.colsrc, tid);
  }
}

// The same backward mask for drawn or constant sources (no tables) as a streaming pass:
// each lane takes 8 consecutive components of one job (16-byte accesses of ci, h, d_acts,
// d_pre, 8 u bytes), the grid walks the jobs' rows in order, so every row of every operand
// is read and written whole. c % 8 == 0; ci_pre / d_pre 16-byte aligned.
// One 8-component chunk of the backward mask for drawn or constant sources: job j (of
// token slot / k, expert e), components q .. q + 7, da the chunk of d_acts (bf16 values;
// counted as 0 on an unrouted job). Writes d_pre (token-major) and d_h = d_acts (m - d).
// The values of one chunk: ci preactivations pre, h, the u bytes ub, the SL0 slopes (or
// imp_scale), the job's delta dt and d_acts da (0 on an unrouted job) -> d_pre, d_h.
// (uconst, g2, psis, p: the site's SiteMaskArgs fields of those names.)
template <int PM>
__device__ inline void mask_bwd_values(float uconst, float g2, float psis, float pexp, float imp_scale,
                                       const float (&pre)[8], const float (&hv)[8], uint2 ub,
                                       const float (&slope8)[8], float dt, const float (&da)[8], float (&dp)[8],
                                       float (&o)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float lo = lower_fwd(pre[e]), up = upper_fwd(pre[e]);
    const uint32_t w = e < 4 ? ub.x : ub.y;
    const float u = uconst < 0.f ? (float)((w >> (8 * (e & 3))) & 0xFFu) * (1.f / 128.f) : uconst;
    const float m = lo + (1.f - lo) * u - dt;
    float dimp;
    if constexpr (PM == PM_SL0) dimp = slope8[e] * sl0_dpsi(up, g2, psis);
    else dimp = imp_scale * dpowp<PM>(up, pexp);
    dp[e] = lower_vjp(pre[e], da[e] * hv[e] * (1.f - u)) + upper_vjp(pre[e], dimp);
    o[e] = da[e] * m;
  }
}

template <int PM>
__device__ inline void slope_chunk(const SiteMaskArgs& a, float imp_scale, int e_row, int q, float (&slope8)[8]) {
  if constexpr (PM == PM_SL0) {
    load8f(a.slope + (int64_t)e_row * a.c + q, slope8);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) slope8[e] = imp_scale;
  }
}

template <int PM>
__device__ inline void mask_bwd_chunk(const SiteMaskArgs& a, const bf16_t* __restrict__ h,
                                      const uint8_t* __restrict__ ubits, float imp_scale, int64_t j, int32_t slot,
                                      int e_row, int q, float (&da)[8], bf16_t* __restrict__ d_h,
                                      bf16_t* __restrict__ d_pre) {
  const int64_t idx = j * a.c + q, src = (int64_t)slot * a.c + q;
  const float dt = job_delta(a, slot);
  if (!job_routed(a, slot)) {
#pragma unroll
    for (int e = 0; e < 8; ++e) da[e] = 0.f;
  }
  float pre[8], hv[8];
  load8(a.ci_pre + src, pre);
  load8(h + idx, hv);
  const uint2 ub = a.uconst < 0.f ? *(const uint2*)(ubits + idx) : make_uint2(0u, 0u);
  float slope8[8];
  slope_chunk<PM>(a, imp_scale, e_row, q, slope8);
  float dp[8], o[8];
  mask_bwd_values<PM>(a.uconst, a.g2, a.psis, a.p, imp_scale, pre, hv, ub, slope8, dt, da, dp, o);
  store8(d_pre + src, dp);
  store8(d_h + idx, o);
}

template <int PM>
__global__ __launch_bounds__(256) void k_mask_bwd_vec(SiteMaskArgs a, const bf16_t* __restrict__ h,
                                                      const uint8_t* __restrict__ ubits, float imp_scale,
                                                      bf16_t* __restrict__ d_acts, bf16_t* __restrict__ d_pre) {
  const uint32_t cpr = (uint32_t)a.c >> 3;  // 8-component chunks per row
  const uint32_t nch = (uint32_t)a.J * cpr;
  for (uint32_t ch = blockIdx.x * 256u + threadIdx.x; ch < nch; ch += gridDim.x * 256u) {
    const uint32_t j = ch / cpr;
    const int q = (int)(ch - j * cpr) * 8;
    const int32_t slot = a.sort_idx[j];
    float da[8];
    load8(d_acts + (int64_t)j * a.c + q, da);
    mask_bwd_chunk<PM>(a, h, ubits, imp_scale, j, slot, PM == PM_SL0 ? row_group(a.offsets, a.E, j) : 0, q, da,
                       d_acts, d_pre);
  }
}

// The backward mask as the epilogue of the grouped d_acts = d_out @ U[e]^T product (one
// problem, or a pair of sites): the tile goes through the staged LDS image rounded to
// bf16, exactly as the product's store would write d_acts, then every lane takes an
// 8-component chunk of an image row through mask_bwd_chunk, writing d_h over the
// product's output (C) and d_pre token-major. The tile's rows all belong to its expert.
template <int PM>
struct EpiMaskBwd {
  static constexpr int LDS_BYTES = 0;
  struct Args {
    SiteMaskArgs a0, a1;  // the sites of problem 0 and (paired) problem 1
    const bf16_t* h0;
    const bf16_t* h1;
    const uint8_t* ub0;
    const uint8_t* ub1;
    bf16_t* dp0;
    bf16_t* dp1;
    float imp_scale;
  };
  template <class CFG, typename TC>
  __device__ static void run(const GemmArgs& p, const Args& ea, const TileJob& t, int wm, int wn, int tid,
                             f32x16 (&acc)[CFG::TM][CFG::TN], char* smem) {
    static_assert(sizeof(TC) == 2, "d_h is bf16");
    typedef StagedStore<CFG, 2> SS;
    static_assert(SS::OK, "the tile's image fits the stage ring");
    constexpr int CPR = CFG::BN / 8, RPP = CFG::NT / CPR;
    static_assert(CFG::NT % CPR == 0 && SS::ROWS % RPP == 0, "image passes");
    const int lane = tid & 63, rr = tid / CPR, cc = tid % CPR;
    // the tile's site: each field read as a value and selected (selecting between the
    // argument structs, or copies of them, takes their addresses and puts them in scratch)
    const bool p1 = t.prob != 0;
    const SiteMaskArgs& A0 = ea.a0;
    const SiteMaskArgs& A1 = ea.a1;
    const bf16_t *ci0 = A0.ci_pre, *ci1 = A1.ci_pre, *h0 = ea.h0, *h1 = ea.h1;
    const uint8_t *ub0 = ea.ub0, *ub1 = ea.ub1, *rt0 = A0.route, *rt1 = A1.route;
    const float *dl0 = A0.delta, *dl1 = A1.delta, *sl0 = A0.slope, *sl1 = A1.slope;
    bf16_t *dp0 = ea.dp0, *dp1 = ea.dp1;
    const bf16_t* ci = p1 ? ci1 : ci0;
    const bf16_t* h = p1 ? h1 : h0;
    const uint8_t* ub = p1 ? ub1 : ub0;
    const uint8_t* route = p1 ? rt1 : rt0;
    const float* delta = p1 ? dl1 : dl0;
    const float* slope = p1 ? sl1 : sl0;
    bf16_t* dp = p1 ? dp1 : dp0;
    const int32_t* sort_idx = A0.sort_idx;  // shared by the pair
    const int c = A0.c, kk = A0.k;
    const float uconst = A0.uconst, g2 = A0.g2, psis = A0.psis, pexp = A0.p;
    const int col = (int)t.n0 + cc * 8;
    const bool cok = col < p.N;
    bf16_t* dh = (bf16_t*)t.C;
    // the tile's rows: slot, the token's delta and routed flag, looked up once per row
    // (visible after the barrier that opens the first image pass)
    __shared__ int4 jrow[CFG::BM];
    for (int r = tid; r < CFG::BM; r += CFG::NT) {
      const int64_t row = t.m0 + r;
      int4 v = make_int4(0, 0, 0, 0);
      if (row < t.M) {
        const int32_t sl = sort_idx[row], tok = sl / kk;
        v = make_int4(sl, __float_as_int(delta ? delta[tok] : 0.f), !route || route[tok] ? 1 : 0, 0);
      }
      jrow[r] = v;
    }
    // every row of the tile has the tile's expert: one slope chunk per lane
    float slope8[8];
    if constexpr (PM == PM_SL0) {
      if (cok) load8f(slope + (int64_t)t.e * c + col, slope8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) slope8[e] = ea.imp_scale;
    }
    // a lane's chunks of one pass, one at a time (issuing several chunks' loads ahead of
    // their math measured slower)
    constexpr int IT = SS::ROWS / RPP, G = 1;
    static_assert(IT % G == 0, "chunk groups");
#pragma unroll
    for (int q = 0; q < SS::PASSES; ++q) {
      staged_image_pass<CFG, 2>(1.f, q, wm, wn, lane, acc, smem);
#pragma unroll
      for (int g0 = 0; g0 < IT; g0 += G) {
        int64_t row[G];
        int32_t slot[G];
        bool ok[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
          row[i] = t.m0 + q * SS::ROWS + rr + (g0 + i) * RPP;
          ok[i] = cok && row[i] < t.M;
        }
        uint4 pw[G], hw[G];
        uint2 uw[G];
        float dt[G];
        bool routed[G];
#pragma unroll
        for (int i = 0; i < G; ++i) {
          if (!ok[i]) continue;
          const int4 jr = jrow[q * SS::ROWS + rr + (g0 + i) * RPP];
          slot[i] = jr.x;
          dt[i] = __int_as_float(jr.y);
          routed[i] = jr.z != 0;
          pw[i] = *(const uint4*)(ci + (int64_t)slot[i] * c + col);
          hw[i] = *(const uint4*)(h + row[i] * c + col);
          uw[i] = uconst < 0.f ? *(const uint2*)(ub + row[i] * c + col) : make_uint2(0u, 0u);
        }
#pragma unroll
        for (int i = 0; i < G; ++i) {
          if (!ok[i]) continue;
          const int r = rr + (g0 + i) * RPP;
          const uint4 v = *(const uint4*)(smem + r * SS::RSB + cc * 16);
          float da[8], pre[8], hv[8], dpv[8], o[8];
          da[0] = bf_lo(v.x), da[1] = bf_hi(v.x), da[2] = bf_lo(v.y), da[3] = bf_hi(v.y);
          da[4] = bf_lo(v.z), da[5] = bf_hi(v.z), da[6] = bf_lo(v.w), da[7] = bf_hi(v.w);
          if (!routed[i]) {
#pragma unroll
            for (int e = 0; e < 8; ++e) da[e] = 0.f;
          }
          pre[0] = bf_lo(pw[i].x), pre[1] = bf_hi(pw[i].x), pre[2] = bf_lo(pw[i].y), pre[3] = bf_hi(pw[i].y);
          pre[4] = bf_lo(pw[i].z), pre[5] = bf_hi(pw[i].z), pre[6] = bf_lo(pw[i].w), pre[7] = bf_hi(pw[i].w);
          hv[0] = bf_lo(hw[i].x), hv[1] = bf_hi(hw[i].x), hv[2] = bf_lo(hw[i].y), hv[3] = bf_hi(hw[i].y);
          hv[4] = bf_lo(hw[i].z), hv[5] = bf_hi(hw[i].z), hv[6] = bf_lo(hw[i].w), hv[7] = bf_hi(hw[i].w);
          mask_bwd_values<PM>(uconst, g2, psis, pexp, ea.imp_scale, pre, hv, uw[i], slope8, dt[i], da, dpv, o);
          store8(dp + (int64_t)slot[i] * c + col, dpv);
          store8(dh + row[i] * c + col, o);
        }
      }
    }
  }
};

__device__ inline float sigm(float x) { return 1.f / (1.f + __expf(-x)); }

// din[j,:] = bf16(silu(g) * u * w[sort_idx[j]]) (fp32 math); wt NULL = the frozen arm (no
// weight). With the frozen channel (fg, fu
// non-NULL) the site outputs first take their delta share, g = bf16(g + dg[t] * fg) and
// u = bf16(u + du[t] * fu) for the job's token t = sort_idx[j] / k
// (pd/targets/qwen36_moe.py:2810-2815), written back over g and u for the backward.
// f % 8 == 0.
__global__ __launch_bounds__(256) void k_swiglu_fwd_tile(bf16_t* __restrict__ g, bf16_t* __restrict__ u,
                                                         const float* __restrict__ wt,
                                                         const int32_t* __restrict__ sort_idx, int64_t J, int f,
                                                         const bf16_t* __restrict__ fg, const bf16_t* __restrict__ fu,
                                                         const float* __restrict__ dg, const float* __restrict__ du,
                                                         int k, bf16_t* __restrict__ din) {
  const int tid = threadIdx.x;
  const int64_t j0 = (int64_t)blockIdx.y * TILE;
  const int q0 = blockIdx.x * TILE, q4 = PD_TILE4_COL;
  const bool qok = q0 + q4 < f;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int r = PD_TILE4_ROW(pass);
    const int64_t j = j0 + r;
    bf16_t o[4] = {0, 0, 0, 0};
    if (j < J && qok) {
      const int64_t idx = j * f + q0 + q4;
      const uint2 gw = *(const uint2*)(g + idx);
      const uint2 uw = *(const uint2*)(u + idx);
      float gv[4] = {bf_lo(gw.x), bf_hi(gw.x), bf_lo(gw.y), bf_hi(gw.y)};
      float uv[4] = {bf_lo(uw.x), bf_hi(uw.x), bf_lo(uw.y), bf_hi(uw.y)};
      const int32_t slot = sort_idx[j];
      if (fg) {
        const float dgt = dg[slot / k], dut = du[slot / k];
        const uint2 fgw = *(const uint2*)(fg + idx);
        const uint2 fuw = *(const uint2*)(fu + idx);
        const float fgv[4] = {bf_lo(fgw.x), bf_hi(fgw.x), bf_lo(fgw.y), bf_hi(fgw.y)};
        const float fuv[4] = {bf_lo(fuw.x), bf_hi(fuw.x), bf_lo(fuw.y), bf_hi(fuw.y)};
        bf16_t gb[4], ub[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gb[e] = f32_to_bf16(fmaf(dgt, fgv[e], gv[e]));
          ub[e] = f32_to_bf16(fmaf(dut, fuv[e], uv[e]));
          gv[e] = bf16_to_f32(gb[e]);
          uv[e] = bf16_to_f32(ub[e]);
        }
        *(uint2*)(g + idx) = make_uint2(bf_pack(gb[0], gb[1]), bf_pack(gb[2], gb[3]));
        *(uint2*)(u + idx) = make_uint2(bf_pack(ub[0], ub[1]), bf_pack(ub[2], ub[3]));
      }
      const float w = wt ? wt[slot] : 1.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = f32_to_bf16(gv[e] * sigm(gv[e]) * uv[e] * w);
      *(uint2*)(din + idx) = make_uint2(bf_pack(o[0], o[1]), bf_pack(o[2], o[3]));
    }
  }
}

// SwiGLU-fold backward on 64x64 tiles: d_g = bf16(d*u*w*silu'(g)), d_u = bf16(d*silu(g)*w)
// and the per-(job, tile) partial of
// d_w[j] = sum_f d*silu(g)*u into d_w_part [J, tiles]. With the down site's frozen channel
// (gd non-NULL) the cotangent of the down input is d = d_din + dd[t] * gd, gd = d_out @
// W_down[e]^T of the job, t = sort_idx[j] / k.
__global__ __launch_bounds__(256) void k_swiglu_bwd_tile(const bf16_t* __restrict__ d_din,
                                                         const bf16_t* __restrict__ g, const bf16_t* __restrict__ u,
                                                         const float* __restrict__ wt,
                                                         const int32_t* __restrict__ sort_idx, int64_t J, int f,
                                                         const bf16_t* __restrict__ gd, const float* __restrict__ dd,
                                                         int k, bf16_t* __restrict__ d_g, bf16_t* __restrict__ d_u,
                                                         float* __restrict__ d_w_part) {
  const int tid = threadIdx.x;
  const int64_t j0 = (int64_t)blockIdx.y * TILE;
  const int q0 = blockIdx.x * TILE, q4 = PD_TILE4_COL;
  const bool qok = q0 + q4 < f;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int r = PD_TILE4_ROW(pass);
    const int64_t j = j0 + r;
    bf16_t og[4] = {0, 0, 0, 0}, ou[4] = {0, 0, 0, 0};
    float part = 0.f;
    if (j < J && qok) {
      const int64_t idx = j * f + q0 + q4;
      const int32_t slot = sort_idx[j];
      const float w = wt[slot];
      const uint2 dw = *(const uint2*)(d_din + idx);
      const uint2 gw = *(const uint2*)(g + idx);
      const uint2 uw = *(const uint2*)(u + idx);
      float dv[4] = {bf_lo(dw.x), bf_hi(dw.x), bf_lo(dw.y), bf_hi(dw.y)};
      if (gd) {
        const float ddt = dd[slot / k];
        const uint2 fw = *(const uint2*)(gd + idx);
        const float fv[4] = {bf_lo(fw.x), bf_hi(fw.x), bf_lo(fw.y), bf_hi(fw.y)};
#pragma unroll
        for (int e = 0; e < 4; ++e) dv[e] = fmaf(ddt, fv[e], dv[e]);
      }
      const float gv[4] = {bf_lo(gw.x), bf_hi(gw.x), bf_lo(gw.y), bf_hi(gw.y)};
      const float uv[4] = {bf_lo(uw.x), bf_hi(uw.x), bf_lo(uw.y), bf_hi(uw.y)};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float sg = sigm(gv[e]);
        const float s = gv[e] * sg;
        og[e] = f32_to_bf16(dv[e] * uv[e] * w * sg * (1.f + gv[e] * (1.f - sg)));
        ou[e] = f32_to_bf16(dv[e] * s * w);
        part += dv[e] * s * uv[e];
      }
      *(uint2*)(d_g + idx) = make_uint2(bf_pack(og[0], og[1]), bf_pack(og[2], og[3]));
      *(uint2*)(d_u + idx) = make_uint2(bf_pack(ou[0], ou[1]), bf_pack(ou[2], ou[3]));
    }
    // the 16 lanes of one row sum their partials
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) part += __shfl_xor(part, o, 64);
    if ((tid & 15) == 0 && j < J) d_w_part[j * gridDim.x + blockIdx.x] = part;
  }
}

// d_logits of one token in the lane-strided layout (dl[i] = expert lane + 64 i, 0 past
// E), all 64 lanes active: d_w[s] = sum of the d_w_part tiles of job inv[t*k+s], through
// w = p_sel / sum p_sel and the router softmax, rounded to bf16.
template <int EPL>
__device__ inline void router_logit_vjp(const float* __restrict__ d_w_part, int n_part,
                                        const int32_t* __restrict__ inv, const int32_t* __restrict__ idx,
                                        const float* __restrict__ probs, const float* __restrict__ w, int64_t t,
                                        int E, int k, int lane, float (&dl)[EPL]) {
  float dw = 0.f;
  if (lane < k) {
    const int64_t jj = inv[t * k + lane];
    for (int pp = 0; pp < n_part; ++pp) dw += d_w_part[jj * n_part + pp];
  }
  const float wv = lane < k ? w[t * k + lane] : 0.f;
  const float dot = wave_sum(dw * wv);
  int e_of_slot = lane < k ? idx[t * k + lane] : 0;
  e_of_slot = e_of_slot < 0 ? 0 : (e_of_slot >= E ? E - 1 : e_of_slot);
  float pe[EPL], dpe[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    pe[i] = lane + 64 * i < E ? probs[t * E + lane + 64 * i] : 0.f;
    dpe[i] = 0.f;
  }
  const float psel = expert_value<EPL>(pe, e_of_slot);
  const float S = wave_sum(lane < k ? psel : 0.f);
  const float dps = lane < k ? (dw - dot) / S : 0.f;
  for (int s = 0; s < k; ++s) {
    const int es = __shfl(e_of_slot, s, 64);
    const float v = __shfl(dps, s, 64);
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (lane + 64 * i == es) dpe[i] += v;
  }
  float sl = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) sl += lane + 64 * i < E ? pe[i] * dpe[i] : 0.f;
  const float sdot = wave_sum(sl);
  // the logits were widened from the bf16 router product: their cotangent narrows to
  // bf16 on its way back into that product
#pragma unroll
  for (int i = 0; i < EPL; ++i)
    dl[i] = lane + 64 * i < E ? bf16_to_f32(f32_to_bf16(pe[i] * (dpe[i] - sdot))) : 0.f;
}

// Token backward, one wave per TPW consecutive tokens, lane l owning columns 8l..8l+7 of
// each of the NCH 512-column chunks (d <= 512 * NCH, d % 8 == 0):
//   d_h2 = sum_s (dxa + dxb)[inv[t*k+s]] + d_logits @ router (slot sums first, then the
//   experts in order, fp32); d_r_out = bf16(d_r + rms_norm_vjp(d_h2)). The TPW tokens of
//   a wave share each 16-byte router load. With the frozen channel (fxa non-NULL) each
//   slot also adds da[t] * fxa + db[t] * fxb, the gate and up frozen products' input
//   cotangents scaled by the token's delta draws.
template <int TPW, int NCH, int EPL>
__global__ __launch_bounds__(256) void k_token_bwd(const float* __restrict__ d_w_part, int n_part,
                                                   const int32_t* __restrict__ inv, const int32_t* __restrict__ idx,
                                                   const float* __restrict__ probs, const float* __restrict__ w,
                                                   const bf16_t* __restrict__ router, const bf16_t* __restrict__ dxa,
                                                   const bf16_t* __restrict__ dxb, const bf16_t* __restrict__ r,
                                                   const float* __restrict__ rinv, const float* __restrict__ ln,
                                                   const bf16_t* __restrict__ d_r, int64_t T, int E, int k, int d,
                                                   const bf16_t* __restrict__ fxa, const bf16_t* __restrict__ fxb,
                                                   const float* __restrict__ da, const float* __restrict__ db,
                                                   bf16_t* __restrict__ d_r_out) {
  const int64_t t0 = ((int64_t)blockIdx.x * 4 + wave_id()) * TPW;
  if (t0 >= T) return;
  const int lane = threadIdx.x & 63;
  float dl[TPW][EPL], a[TPW][NCH][8];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int64_t t = t0 + u;
    if (t < T) {
      router_logit_vjp<EPL>(d_w_part, n_part, inv, idx, probs, w, t, E, k, lane, dl[u]);
    } else {
#pragma unroll
      for (int i = 0; i < EPL; ++i) dl[u][i] = 0.f;
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) a[u][c][j] = 0.f;
    if (t >= T) continue;
    const float dat = fxa ? da[t] : 0.f, dbt = fxa ? db[t] : 0.f;
    for (int s = 0; s < k; ++s) {
      const int64_t row = (int64_t)inv[t * k + s] * d;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int i = c * 512 + lane * 8;
        if (i < d) {
          float va[8], vb[8];
          load8(dxa + row + i, va);
          load8(dxb + row + i, vb);
#pragma unroll
          for (int j = 0; j < 8; ++j) a[u][c][j] += va[j] + vb[j];
          if (fxa) {
            load8(fxa + row + i, va);
            load8(fxb + row + i, vb);
#pragma unroll
            for (int j = 0; j < 8; ++j) a[u][c][j] = fmaf(dat, va[j], fmaf(dbt, vb[j], a[u][c][j]));
          }
        }
      }
    }
  }
#pragma unroll
  for (int blk = 0; blk < EPL; ++blk) {
    for (int el = 0; el < 64 && blk * 64 + el < E; ++el) {
      const int e = blk * 64 + el;
      float de[TPW];
#pragma unroll
      for (int u = 0; u < TPW; ++u)
        de[u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dl[u][blk]), el));
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int i = c * 512 + lane * 8;
        if (i < d) {
          float rv[8];
          load8(router + (int64_t)e * d + i, rv);
#pragma unroll
          for (int u = 0; u < TPW; ++u)
#pragma unroll
            for (int j = 0; j < 8; ++j) a[u][c][j] = fmaf(de[u], rv[j], a[u][c][j]);
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int64_t t = t0 + u;
    if (t >= T) break;
    const bf16_t* xr = r + t * d;
    float part = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int i = c * 512 + lane * 8;
      if (i < d) {
        float g[8], xv[8];
        load8f(ln + i, g);
        load8(xr + i, xv);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          a[u][c][j] = (1.f + g[j]) * a[u][c][j];
          part = fmaf(a[u][c][j], xv[j], part);
        }
      }
    }
    const float ax = wave_sum(part);
    const float rv = rinv[t];
    const float c3 = rv * rv * rv * ax / (float)d;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int i = c * 512 + lane * 8;
      if (i < d) {
        float xv[8], dv[8];
        load8(xr + i, xv);
        load8(d_r + t * d + i, dv);
#pragma unroll
        for (int j = 0; j < 8; ++j) dv[j] = dv[j] + (rv * a[u][c][j] - xv[j] * c3);
        store8(d_r_out + t * d + i, dv);
      }
    }
  }
}

template <int TPW, int NCH>
static void launch_token_bwd_t(const float* d_w_part, int n_part, const int32_t* inv, const int32_t* idx,
                               const float* probs, const float* w, const bf16_t* router, const bf16_t* dxa,
                               const bf16_t* dxb, const bf16_t* r, const float* rinv, const float* ln,
                               const bf16_t* d_r, int64_t T, int E, int k, int d, const bf16_t* fxa,
                               const bf16_t* fxb, const float* da, const float* db, bf16_t* d_r_out, hipStream_t s) {
  const dim3 grid((unsigned)cdiv(T, 4 * TPW));
#define PD_TB(EPL)                                                                                                \
  hipLaunchKernelGGL((k_token_bwd<TPW, NCH, EPL>), grid, dim3(256), 0, s, d_w_part, n_part, inv, idx, probs, w, \
                     router, dxa, dxb, r, rinv, ln, d_r, T, E, k, d, fxa, fxb, da, db, d_r_out)
  if (E <= 64) PD_TB(1);
  else if (E <= 128) PD_TB(2);
  else if (E <= 256) PD_TB(4);
  else PD_TB(8);
#undef PD_TB
}

// d <= 4096 (checked by the step): the column chunks per lane set the register tile.
static void launch_token_bwd(const float* d_w_part, int n_part, const int32_t* inv, const int32_t* idx,
                             const float* probs, const float* w, const bf16_t* router, const bf16_t* dxa,
                             const bf16_t* dxb, const bf16_t* r, const float* rinv, const float* ln, const bf16_t* d_r,
                             int64_t T, int E, int k, int d, const bf16_t* fxa, const bf16_t* fxb, const float* da,
                             const float* db, bf16_t* d_r_out, hipStream_t s) {
  if (d <= 512)
    launch_token_bwd_t<2, 1>(d_w_part, n_part, inv, idx, probs, w, router, dxa, dxb, r, rinv, ln, d_r, T, E, k, d,
                             fxa, fxb, da, db, d_r_out, s);
  else if (d <= 1024)
    launch_token_bwd_t<2, 2>(d_w_part, n_part, inv, idx, probs, w, router, dxa, dxb, r, rinv, ln, d_r, T, E, k, d,
                             fxa, fxb, da, db, d_r_out, s);
  else if (d <= 2048)
    launch_token_bwd_t<1, 4>(d_w_part, n_part, inv, idx, probs, w, router, dxa, dxb, r, rinv, ln, d_r, T, E, k, d,
                             fxa, fxb, da, db, d_r_out, s);
  else
    launch_token_bwd_t<1, 8>(d_w_part, n_part, inv, idx, probs, w, router, dxa, dxb, r, rinv, ln, d_r, T, E, k, d,
                             fxa, fxb, da, db, d_r_out, s);
}

// losses[0..3] = {loss, recon, activity, frequency}: recon = rec_scale * sum(rec_part),
// activity = imp_scale * sum(imp_part), frequency = sum(freq_part) (n_freq = 0: none),
// loss = recon_coeff recon + imp_coeff activity + freq_coeff frequency; with fb_part (the
// EMA estimator's batch penalty) losses[4] = sum(fb_part) over n_freq; every sum in a
// fixed order in double.
__global__ void k_moe_losses(const float* __restrict__ rec_part, int n_rec, const float* __restrict__ imp_part,
                             int64_t n_imp, const float* __restrict__ freq_part, int64_t n_freq,
                             const float* __restrict__ fb_part, double rec_scale, double imp_scale, float recon_coeff,
                             float imp_coeff, float freq_coeff, float* __restrict__ losses) {
  __shared__ double sr[16], si[16], sq[16], sb[16];
  double r = 0.0, m = 0.0, fq = 0.0, fb = 0.0;
  for (int i = threadIdx.x; i < n_rec; i += blockDim.x) r += rec_part[i];
  for (int64_t i = threadIdx.x; i < n_freq; i += blockDim.x) fq += freq_part[i];
  if (fb_part)
    for (int64_t i = threadIdx.x; i < n_freq; i += blockDim.x) fb += fb_part[i];
  // four independent chains keep four loads in flight per lane; combined in a fixed order
  double m4[4] = {0.0, 0.0, 0.0, 0.0};
  const int64_t step = blockDim.x;
  int64_t i = threadIdx.x;
  for (; i + 3 * step < n_imp; i += 4 * step) {
#pragma unroll
    for (int q = 0; q < 4; ++q) m4[q] += imp_part[i + q * step];
  }
  for (; i < n_imp; i += step) m4[0] += imp_part[i];
  m = (m4[0] + m4[1]) + (m4[2] + m4[3]);
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

// Per-token delta draws of every (layer, site): delta[(l*3 + s)*T + t] =
// uniform_bf16(fold_in(fold_in(delta_base, kind_s), l), [T])[t], the frozen channel's
// sample_delta_mask (pd/core/masking.py:139-140) under the per-(kind, layer) keys of
// pd/targets/qwen36_moe.py:3380-3398. Grid (cdiv(T, 256), 3L).
__global__ __launch_bounds__(256) void k_delta_sites(uint32_t b0, uint32_t b1, int64_t T, int layout,
                                                     float* __restrict__ delta) {
  const int site = blockIdx.y;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= T) return;
  uint32_t x0 = 0, x1 = (uint32_t)(MOE_KIND_GATE + site % 3);
  threefry2x32(b0, b1, x0, x1);
  uint32_t k0 = 0, k1 = (uint32_t)(site / 3);
  threefry2x32(x0, x1, k0, k1);
  delta[(int64_t)site * T + t] = draw_uniform(k0, k1, t, T, PD_DTYPE_BF16, layout);
}

// ---------------------------------------------------------------- persistent sources

// goff[g] for g = e * S + row: the first job of expert e whose token lies in source row
// `row` or later (jobs of an expert are in token order), goff[E * S] = J.
__global__ __launch_bounds__(256) void k_src_group_offsets(const int32_t* __restrict__ off,
                                                           const int32_t* __restrict__ sort_idx, int E, int k,
                                                           int64_t S, int64_t rps, int64_t J,
                                                           int32_t* __restrict__ goff) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t G = (int64_t)E * S;
  if (g > G) return;
  if (g == G) {
    goff[G] = (int32_t)J;
    return;
  }
  const int e = (int)(g / S);
  const int64_t row = g % S;
  int64_t lo = off[e], hi = off[e + 1];
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)(sort_idx[mid] / k) / rps >= row) hi = mid;
    else lo = mid + 1;
  }
  goff[g] = (int32_t)lo;
}

// d_src[(row * E + e) * c + q] = the sum, in tile order, of the column partials of group
// g = e * S + row over the tiles its jobs [goff[g], goff[g+1]) touch (0 when it has none).
__global__ __launch_bounds__(256) void k_src_finalize(const float* __restrict__ colsrc,
                                                      const int32_t* __restrict__ goff, int E, int64_t S, int c,
                                                      float* __restrict__ d_src) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)E * S * c) return;
  const int64_t g = i / c;
  const int q = (int)(i % c);
  const int64_t lo = goff[g], hi = goff[g + 1];
  float F = 0.f;
  if (hi > lo)
    for (int64_t t = lo / 64; t <= (hi - 1) / 64; ++t) F += colsrc[(t + g) * c + q];
  const int e = (int)(g / S);
  const int64_t row = g % S;
  d_src[(row * E + e) * c + q] = F;
}

// q[j] = sum_o gout[j,o] frozen[j,o] - sum_p rowdm[j, p]: the delta cotangent of job j's
// site (d enters the site as acts = h (m - d) and as + d frozen). One wave per job, fp32.
__global__ __launch_bounds__(256) void k_job_delta_cot(const bf16_t* __restrict__ gout,
                                                       const bf16_t* __restrict__ frozen,
                                                       const float* __restrict__ rowdm, int n_parts, int64_t J,
                                                       int w, float* __restrict__ q) {
  const int64_t j = (int64_t)blockIdx.x * 4 + wave_id();
  if (j >= J) return;
  const int lane = threadIdx.x & 63;
  float acc = 0.f;
  for (int i = lane * 8; i < w; i += 512) {
    float a[8], b[8];
    load8(gout + j * w + i, a);
    load8(frozen + j * w + i, b);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf(a[e], b[e], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    float dm = 0.f;
    for (int p = 0; p < n_parts; ++p) dm += rowdm[j * n_parts + p];
    q[j] = acc - dm;
  }
}

// d_src_delta[row] = sum over the row's tokens t of sum_s q[inv[t*k + s]]. One wave per
// source row, a fixed order (lane-strided tokens, then the wave tree).
__global__ __launch_bounds__(256) void k_src_delta_grad(const float* __restrict__ q, const int32_t* __restrict__ inv,
                                                        int64_t S, int64_t rps, int k,
                                                        float* __restrict__ d_src_delta) {
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= S) return;
  const int lane = threadIdx.x & 63;
  float acc = 0.f;
  for (int64_t t = row * rps + lane; t < (row + 1) * rps; t += 64)
    for (int s = 0; s < k; ++s) acc += q[inv[t * k + s]];
  acc = wave_sum(acc);
  if (lane == 0) d_src_delta[row] = acc;
}

// out[0, n) = 0.
__global__ __launch_bounds__(256) void k_zero_f32(float* __restrict__ out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) out[i] = 0.f;
}

static void launch_mask_fwd(const SiteMaskArgs& ma, int pm, dim3 grid, hipStream_t s, const bf16_t* h, bf16_t* acts,
                            uint8_t* ub, float* part) {
#define PD_MF(LY, PMV) \
  hipLaunchKernelGGL((k_mask_fwd_tile<LY, PMV>), grid, dim3(256), 0, s, ma, h, acts, ub, part)
  if (ma.src) {
    if (pm == PM_SL0) PD_MF(MASK_SRC, PM_SL0);
    else if (pm == 2) PD_MF(MASK_SRC, 2);
    else if (pm == 1) PD_MF(MASK_SRC, 1);
    else PD_MF(MASK_SRC, 0);
  } else if (ma.uconst >= 0.f) {
    if (pm == PM_SL0) PD_MF(MASK_CONST, PM_SL0);
    else if (pm == 2) PD_MF(MASK_CONST, 2);
    else if (pm == 1) PD_MF(MASK_CONST, 1);
    else PD_MF(MASK_CONST, 0);
  } else if (ma.layout == PD_LAYOUT_PARTITIONABLE) {
    if (pm == PM_SL0) PD_MF(PD_LAYOUT_PARTITIONABLE, PM_SL0);
    else if (pm == 2) PD_MF(PD_LAYOUT_PARTITIONABLE, 2);
    else if (pm == 1) PD_MF(PD_LAYOUT_PARTITIONABLE, 1);
    else PD_MF(PD_LAYOUT_PARTITIONABLE, 0);
  } else {
    if (pm == PM_SL0) PD_MF(PD_LAYOUT_ORIGINAL, PM_SL0);
    else if (pm == 2) PD_MF(PD_LAYOUT_ORIGINAL, 2);
    else if (pm == 1) PD_MF(PD_LAYOUT_ORIGINAL, 1);
    else PD_MF(PD_LAYOUT_ORIGINAL, 0);
  }
#undef PD_MF
}

static void launch_mask_bwd(const SiteMaskArgs& ma, int pm, dim3 grid, hipStream_t s, const bf16_t* h,
                            const uint8_t* ub, float imp_scale, bf16_t* d_acts, bf16_t* d_pre) {
#define PD_MB(PMV, SRC) \
  hipLaunchKernelGGL((k_mask_bwd_tile<PMV, SRC>), grid, dim3(256), 0, s, ma, h, ub, imp_scale, d_acts, d_pre)
  if (ma.src) {
    if (pm == PM_SL0) PD_MB(PM_SL0, true);
    else if (pm == 2) PD_MB(2, true);
    else if (pm == 1) PD_MB(1, true);
    else PD_MB(0, true);
  } else if (((uintptr_t)ma.ci_pre & 15) == 0 && ((uintptr_t)d_pre & 15) == 0 && ma.J * (int64_t)ma.c < (1ll << 34)) {
    // the streaming pass: about 8 chunks of 8 components per lane in flight over the grid
    const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(ma.J * (int64_t)(ma.c / 8), 256), 8192);
#define PD_MBV(PMV) \
  hipLaunchKernelGGL((k_mask_bwd_vec<PMV>), dim3(blocks), dim3(256), 0, s, ma, h, ub, imp_scale, d_acts, d_pre)
    if (pm == PM_SL0) PD_MBV(PM_SL0);
    else if (pm == 2) PD_MBV(2);
    else if (pm == 1) PD_MBV(1);
    else PD_MBV(0);
#undef PD_MBV
  } else {
    if (pm == PM_SL0) PD_MB(PM_SL0, false);
    else if (pm == 2) PD_MB(2, false);
    else if (pm == 1) PD_MB(1, false);
    else PD_MB(0, false);
  }
#undef PD_MB
}

// The backward mask fused into the d_acts product's epilogue applies to drawn or constant
// sources (no tables) with K a multiple of 64 and 16-byte aligned rows.
static bool mask_bwd_fusable(const SiteMaskArgs& ma, const bf16_t* h, const uint8_t* ub, const bf16_t* d_pre,
                             const bf16_t* out, int64_t K) {
  auto al = [](const void* q, uintptr_t m) { return ((uintptr_t)q & m) == 0; };
  return !ma.src && K % 64 == 0 && ma.c % 8 == 0 && al(ma.ci_pre, 15) && al(h, 15) && al(d_pre, 15) && al(out, 15) &&
         (ma.uconst >= 0.f || al(ub, 7)) && ma.J * (int64_t)ma.c < (1ll << 31);
}

// d_acts = lhs [J, K] @ rhs[e]^T (rhs stored [E, N, K]) per expert group with the backward
// mask of site m0 as the epilogue (d_h over out, d_pre0 token-major); with lhs2 non-NULL
// a second site's product in the same launch. N = c.
static int grouped_gemm_mask_bwd(const bf16_t* lhs, const bf16_t* rhs, bf16_t* out, const SiteMaskArgs& m0,
                                 const bf16_t* h0, const uint8_t* ub0, bf16_t* d_pre0, const bf16_t* lhs2,
                                 const bf16_t* rhs2, bf16_t* out2, const SiteMaskArgs* m1, const bf16_t* h1,
                                 const uint8_t* ub1, bf16_t* d_pre1, const int32_t* offsets, int64_t J, int E,
                                 int64_t K, int64_t N, int pm, float imp_scale, hipStream_t s) {
  const bool pair = lhs2 != nullptr;
  if (J == 0) return PD_OK;
  if (!dtl_fits(J, K, N, K) || cdiv(J, CfgDtlRA::BM) + E > 65535)
    return fail(PD_EUNSUPPORTED, "pd_moe_stack_step: d_acts product too large");
  GemmArgs a{J, N, K, lhs, K, rhs, K, out, N, 1.f, 0.f, offsets, E, K * N, 0, 0, lhs2, rhs2, out2};
  // 128x128 tiles for pairs too (unlike the plain paired N=512 products): two blocks per
  // CU keep twice the waves to cover the epilogue's gathered loads (measured faster)
  const dim3 grid((unsigned)cdiv(N, CfgDtlRA::BN), (unsigned)(cdiv(J, CfgDtlRA::BM) + E), pair ? 2u : 1u);
#define PD_FM(PMV)                                                                                                    \
  {                                                                                                                   \
    typename EpiMaskBwd<PMV>::Args ea{m0, pair ? *m1 : m0, h0, pair ? h1 : h0, ub0, pair ? ub1 : ub0, d_pre0,         \
                                      pair ? d_pre1 : d_pre0, imp_scale};                                             \
    hipLaunchKernelGGL((k_gemm_dtl<CfgDtlRA, bf16_t, MODE_GROUPED, false, EpiMaskBwd<PMV>>), grid,                   \
                       dim3(CfgDtlRA::NT), 0, s, a, ea);                                                              \
  }
  if (pm == PM_SL0) PD_FM(PM_SL0)
  else if (pm == 2) PD_FM(2)
  else if (pm == 1) PD_FM(1)
  else PD_FM(0)
#undef PD_FM
  return check_launch("pd_moe_stack_step d_acts + mask backward");
}

// delta[0, n) = v (the constant sources' delta mask).
// blend[i] = route[i] ? delta[i] : 1 (delta NULL: 0), over every (layer, site, token): the
// frozen output's share of a job's site output, where(route, decomposed + d frozen, frozen).
__global__ __launch_bounds__(256) void k_route_blend(const float* __restrict__ delta,
                                                     const uint8_t* __restrict__ route, int64_t n,
                                                     float* __restrict__ blend) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    blend[i] = route[i] ? (delta ? delta[i] : 0.f) : 1.f;
}

__global__ __launch_bounds__(256) void k_fill_f32(float* __restrict__ out, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) out[i] = v;
}

// ---------------------------------------------------------------- workspace plan
static constexpr int REC_BLOCKS = 1024;

struct MoEDims {
  int64_t T, J;
  int d, f, E, k, c, L;
  int64_t S;  // persistent-source rows (0: no source tables)
};

struct Arena {
  char* base;
  size_t off;
  bool dry;
  template <typename X>
  X* take(size_t n) {
    size_t bytes = (n * sizeof(X) + 255) & ~(size_t)255;
    X* p = dry ? nullptr : (X*)(base + off);
    off += bytes;
    return p;
  }
};

struct LayerSave {
  bf16_t *r, *h2, *xj, *gout, *uout, *din;  // xj, din: the layer's job-space inputs of its products
  bf16_t *fg, *fu, *fd;  // the frozen channel's products x_jobs @ Wg/Wu[e], din @ Wd[e]
  float *rinv, *probs, *w;
  int32_t *idx, *sort_idx, *inv, *sizes, *offsets;
  bf16_t* h[3];
  bf16_t* acts[3];
  uint8_t* ub[3];
};

struct MoEPlan {
  std::vector<LayerSave> layers;
  // weight copies [L, E, N, K] for the forward products
  bf16_t *WgT, *WuT, *WdT, *VgT, *UgT, *VuT, *UuT, *VdT, *UdT;
  bf16_t *rc_a, *rc_b, *r_final, *h2c, *xjc, *gc, *uc, *din, *downc, *down, *dr_a, *dr_b;
  float *colsrc, *rowdm, *qjob;  // persistent sources: group column sums, job row sums, job delta cotangents
  int32_t* goff;
  float *logits, *logitsc, *probsc, *wc, *rec_part, *imp_part, *d_w_part, *delta, *blend;
  float *sl0_col, *sl0_slope, *sl0_act, *sl0_freq, *sl0_fb;  // smooth-L0: per site-layer regions
  size_t sl0_col_per_site, sl0_slope_per_site, sl0_blocks_per_site;
  int32_t* sort_ws;
  bf16_t *d_dout, *d_acts[3], *d_din, *d_g, *d_u, *dxa, *dxb;  // d_acts[si]: site si
  size_t imp_per_site, total;
};

static MoEPlan plan(const MoEDims& D, char* base, bool dry) {
  Arena A{base, 0, dry};
  MoEPlan P;
  const int64_t T = D.T, J = D.J;
  const size_t E = D.E, L = D.L;
  P.layers.resize(D.L);
  for (int l = 0; l < D.L; ++l) {
    LayerSave& S = P.layers[l];
    S.r = A.take<bf16_t>(T * D.d);
    S.h2 = A.take<bf16_t>(T * D.d);
    S.rinv = A.take<float>(T);
    S.probs = A.take<float>(T * D.E);
    S.w = A.take<float>(T * D.k);
    S.idx = A.take<int32_t>(T * D.k);
    S.sort_idx = A.take<int32_t>(J);
    S.inv = A.take<int32_t>(J);
    S.sizes = A.take<int32_t>(D.E);
    S.offsets = A.take<int32_t>(D.E + 1);
    S.xj = A.take<bf16_t>(J * D.d);
    S.gout = A.take<bf16_t>(J * D.f);
    S.uout = A.take<bf16_t>(J * D.f);
    S.din = A.take<bf16_t>(J * D.f);
    S.fg = A.take<bf16_t>(J * D.f);
    S.fu = A.take<bf16_t>(J * D.f);
    S.fd = A.take<bf16_t>(J * D.d);
    for (int s = 0; s < 3; ++s) {
      S.h[s] = A.take<bf16_t>(J * D.c);
      S.acts[s] = A.take<bf16_t>(J * D.c);
      S.ub[s] = A.take<uint8_t>(J * D.c);
    }
  }
  P.WgT = A.take<bf16_t>(L * E * D.d * D.f);
  P.WuT = A.take<bf16_t>(L * E * D.d * D.f);
  P.WdT = A.take<bf16_t>(L * E * D.d * D.f);
  P.VgT = A.take<bf16_t>(L * E * D.d * D.c);
  P.UgT = A.take<bf16_t>(L * E * D.c * D.f);
  P.VuT = A.take<bf16_t>(L * E * D.d * D.c);
  P.UuT = A.take<bf16_t>(L * E * D.c * D.f);
  P.VdT = A.take<bf16_t>(L * E * D.f * D.c);
  P.UdT = A.take<bf16_t>(L * E * D.c * D.d);
  P.rc_a = A.take<bf16_t>(T * D.d);
  P.rc_b = A.take<bf16_t>(T * D.d);
  P.r_final = A.take<bf16_t>(T * D.d);
  P.h2c = A.take<bf16_t>(T * D.d);
  P.xjc = A.take<bf16_t>(J * D.d);
  P.gc = A.take<bf16_t>(J * D.f);
  P.uc = A.take<bf16_t>(J * D.f);
  P.din = A.take<bf16_t>(J * D.f);
  P.downc = A.take<bf16_t>(J * D.d);
  P.down = A.take<bf16_t>(J * D.d);
  P.dr_a = A.take<bf16_t>(T * D.d);
  P.dr_b = A.take<bf16_t>(T * D.d);
  P.logits = A.take<float>(T * D.E);
  P.logitsc = A.take<float>(T * D.E);
  P.probsc = A.take<float>(T * D.E);
  P.wc = A.take<float>(T * D.k);
  P.rec_part = A.take<float>(REC_BLOCKS);
  P.imp_per_site = (size_t)cdiv(D.c, TILE) * cdiv(J, TILE);
  P.imp_part = A.take<float>(P.imp_per_site * 3 * D.L);
  P.sl0_col_per_site = (size_t)(cdiv(J, TILE) + D.E) * D.c;
  P.sl0_slope_per_site = (size_t)D.E * D.c;
  P.sl0_blocks_per_site = sl0_blocks(D.E, D.c);
  P.sl0_col = A.take<float>(P.sl0_col_per_site * 3 * L);
  P.sl0_slope = A.take<float>(P.sl0_slope_per_site * 3 * L);
  P.sl0_act = A.take<float>(P.sl0_blocks_per_site * 3 * L);
  P.sl0_freq = A.take<float>(P.sl0_blocks_per_site * 3 * L);
  P.sl0_fb = A.take<float>(P.sl0_blocks_per_site * 3 * L);
  P.colsrc = A.take<float>(D.S && D.S < T ? (size_t)(cdiv(J, TILE) + (int64_t)D.E * D.S) * D.c : 1);
  P.rowdm = A.take<float>(D.S ? (size_t)J * cdiv(D.c, TILE) : 1);
  P.qjob = A.take<float>(D.S ? (size_t)J : 1);
  P.goff = A.take<int32_t>(D.S ? (size_t)D.E * D.S + 1 : 1);
  P.d_w_part = A.take<float>(J * cdiv(D.f, TILE));
  P.delta = A.take<float>((size_t)T * 3 * L);
  P.blend = A.take<float>((size_t)T * 3 * L);
  P.sort_ws = A.take<int32_t>(pd_routed_jobs_workspace_size(J, D.E) / 4 + 1);
  P.d_dout = A.take<bf16_t>(J * D.d);
  for (int i = 0; i < 3; ++i) P.d_acts[i] = A.take<bf16_t>(J * D.c);
  P.d_din = A.take<bf16_t>(J * D.f);
  P.d_g = A.take<bf16_t>(J * D.f);
  P.d_u = A.take<bf16_t>(J * D.f);
  P.dxa = A.take<bf16_t>(J * D.d);
  P.dxb = A.take<bf16_t>(J * D.d);
  P.total = A.off;
  return P;
}

struct Recorder {
  void** ev;
  int32_t* cat;
  int cap, n;
  hipStream_t s;
  void mark(int category) {
    if (!ev || n >= cap) return;
    hipEventRecord((hipEvent_t)ev[n], s);
    if (cat) cat[n] = category;
    ++n;
  }
};

static void launch_batched_T(const void* src, int64_t B, int64_t R, int64_t Cc, bf16_t* dst, hipStream_t s) {
  hipLaunchKernelGGL(k_batched_transpose, dim3((unsigned)cdiv(Cc, TILE), (unsigned)cdiv(R, TILE), (unsigned)B),
                     dim3(256), 0, s, (const bf16_t*)src, R, Cc, dst);
}

static dim3 tile_grid(int64_t J, int w) { return dim3((unsigned)cdiv(w, TILE), (unsigned)cdiv(J, TILE)); }

}  // namespace pd

using namespace pd;

extern "C" {

size_t pd_moe_stack_workspace_size(int64_t T, int d, int f, int E, int k, int c, int L) {
  MoEDims D{T, T * k, d, f, E, k, c, L, 0};
  return plan(D, nullptr, true).total;
}

size_t pd_moe_stack_sources_workspace_size(int64_t T, int d, int f, int E, int k, int c, int L,
                                           int64_t rows_per_source) {
  if (rows_per_source <= 0 || T % rows_per_source) return 0;
  MoEDims D{T, T * k, d, f, E, k, c, L, T / rows_per_source};
  return plan(D, nullptr, true).total;
}

// Phase categories recorded by pd_moe_stack_step_timed (one event before each launch
// group and one at the end; cat[i] labels the interval [i, i+1)).
enum {
  MOE_CAT_CLEAN = 0,       // weight copies + clean forward (norm, router, bucketing, frozen GEMMs, combine)
  MOE_CAT_NORM_ROUTE = 1,  // masked-pass norm, router GEMM, pinned weights, gather
  MOE_CAT_GEMM_FWD = 2,    // grouped GEMMs of the decomposed sites, forward
  MOE_CAT_MASK_FWD = 3,    // job-space mask passes, forward
  MOE_CAT_SWIGLU = 4,      // SwiGLU fold fwd/bwd
  MOE_CAT_COMBINE = 5,     // sum_jobs + residual, loss, gathers
  MOE_CAT_GEMM_DX = 6,     // grouped GEMMs d_input
  MOE_CAT_GEMM_DW = 7,     // grouped GEMMs d_weight (ragged contraction)
  MOE_CAT_MASK_BWD = 8,    // job-space mask passes, backward
  MOE_CAT_TOKEN_BWD = 9,   // router/norm token backward
  MOE_CAT_WAIT = 10,       // waiting for the helper stream (clean layers, weight gradients)
  MOE_CAT_GEMM_MASK = 11,  // grouped GEMMs d_acts with the backward mask as their epilogue
  MOE_CAT_END = 12
};

// Persistent (adversarial) source tables for pd_moe_stack_step_sources.
struct SrcArgs {
  const void* src;    // [L, 3, S, E, c]
  int src_dtype;
  const void* delta;  // [L, 3, S] or NULL (no delta channel)
  int delta_dtype;
  int64_t rps;        // tokens per source row (S = T / rps)
  int want_wgrads;    // 0: only the source gradients (warmup ascents)
  float* d_src;       // fp32 [L, 3, S, E, c]
  float* d_src_delta; // fp32 [L, 3, S]
};

static int moe_step_impl(int64_t T, int d, int f, int E, int k, int c, int L, const void* x0, const float* ln,
                         const void* router, const void* Wg, const void* Wu, const void* Wd, const void* Vg,
                         const void* Ug, const void* Vu, const void* Uu, const void* Vd, const void* Ud,
                         const void* ci_pre, uint32_t draw_k0, uint32_t draw_k1, int use_delta,
                         const uint8_t* routes, float source_value,
                         int layout, const ImpSpec& imp, float recon_coeff, float* losses, float* dVg, float* dUg,
                         float* dVu, float* dUu, float* dVd, float* dUd, void* d_ci_pre, int32_t* top_idx_out,
                         void* workspace, size_t workspace_bytes, void* stream, Recorder& rec,
                         const SrcArgs* srcs = nullptr, bool reuse_clean = false) {
  int rc0;
  if (T <= 0 || d <= 0 || f <= 0 || E <= 0 || E > 512 || k <= 0 || k > E || k > 64 || c <= 0 || L <= 0)
    return fail(PD_EINVAL, "pd_moe_stack_step: bad dims (E <= 512, k <= 64)");
  if (d % 8 || f % 8 || c % 8 || (T * k) % 8)
    return fail(PD_EUNSUPPORTED, "pd_moe_stack_step: d, f, c and T*k must be multiples of 8");
  if (d > 4096 || T * k > 0x7FFFFFFF || cdiv(T * k, TILE) > 65535)
    return fail(PD_EUNSUPPORTED, "pd_moe_stack_step: shape too large");
  if (!x0 || !ln || !router || !Wg || !Wu || !Wd || !Vg || !Ug || !Vu || !Uu || !Vd || !Ud || !ci_pre || !losses ||
      !d_ci_pre)
    return fail(PD_EINVAL, "pd_moe_stack_step: null pointer");
  if ((!srcs || srcs->want_wgrads) && (!dVg || !dUg || !dVu || !dUu || !dVd || !dUd))
    return fail(PD_EINVAL, "pd_moe_stack_step: null weight-gradient output");
  if (layout != PD_LAYOUT_PARTITIONABLE && layout != PD_LAYOUT_ORIGINAL)
    return fail(PD_EINVAL, "pd_moe_stack_step: unknown counter layout");
  if (!(source_value <= 1.f)) return fail(PD_EINVAL, "pd_moe_stack_step: source_value must be < 0 (drawn) or in [0, 1]");
  if ((rc0 = check_imp_spec(imp, "pd_moe_stack_step"))) return rc0;
  const float uconst = source_value >= 0.f ? source_value : -1.f;
  if (srcs) {
    if (!srcs->src || srcs->rps <= 0 || T % srcs->rps || !srcs->d_src || (srcs->delta && !srcs->d_src_delta))
      return fail(PD_EINVAL, "pd_moe_stack_step_sources: source tables, rows_per_source | T and outputs required");
    for (int dt : {srcs->src_dtype, srcs->delta ? srcs->delta_dtype : PD_DTYPE_F32})
      if (dt != PD_DTYPE_F32 && dt != PD_DTYPE_BF16 && dt != PD_DTYPE_U16)
        return fail(PD_EINVAL, "pd_moe_stack_step_sources: source dtype");
    use_delta = srcs->delta ? 1 : 0;
    if (routes) return fail(PD_EINVAL, "pd_moe_stack_step_sources: no per-token routes with source tables");
  }
  // the frozen channel (x_jobs @ W[e] beside every site) runs with the delta draws, and
  // with routes, whose unrouted tokens take the frozen output alone
  const bool use_frozen = use_delta || routes;
  // Without source tables the frozen products join their site's second product as a first
  // contraction segment, scaled per token (one launch, one rounding): gate / up from layer
  // 1 on (layer 0's come from the clean pass), down, and the backward's d_input products.
  // The source-table path keeps them apart, since its delta gradient reads them.
  const bool kc = use_frozen && !srcs;
  const bool want_wgrads = !srcs || srcs->want_wgrads;
  const MoEDims D{T, T * k, d, f, E, k, c, L, srcs ? T / srcs->rps : 0};
  if (!workspace || workspace_bytes < plan(D, nullptr, true).total)
    return fail(PD_EWORKSPACE, "pd_moe_stack_step: workspace too small");
  MoEPlan P = plan(D, (char*)workspace, false);
  hipStream_t s = (hipStream_t)stream;
  rec.s = s;
  const int64_t J = D.J;
  const size_t szW = (size_t)E * d * f, szVg = (size_t)E * d * c, szUg = (size_t)E * c * f, szVd = (size_t)E * f * c,
               szUd = (size_t)E * c * d;
  const size_t szCI = (size_t)T * k * c;
  auto bf = [](const void* base, size_t off) { return (const bf16_t*)base + off; };
  int rc;
  // ---- site keys: src_base, delta_base = split(draw_key);
  //      key(kind, layer) = fold_in(fold_in(base, kind), layer)
  uint32_t halves[4];
  split2(draw_k0, draw_k1, layout, halves);
  const uint32_t sb0 = halves[0], sb1 = halves[1];
  const float* dlt[3] = {nullptr, nullptr, nullptr};  // the current layer's per-token delta draws
  const float* bl[3] = {nullptr, nullptr, nullptr};   // ... the frozen outputs' shares (d, or route ? d : 1)
  const uint8_t* rt[3] = {nullptr, nullptr, nullptr}; // ... per-token routes
  auto site_key = [&](int kind, int layer, uint32_t& o0, uint32_t& o1) {
    uint32_t x0_ = 0, x1_ = (uint32_t)kind;
    threefry2x32(sb0, sb1, x0_, x1_);
    uint32_t y0 = 0, y1 = (uint32_t)layer;
    threefry2x32(x0_, x1_, y0, y1);
    o0 = y0;
    o1 = y1;
  };
  const int kinds[3] = {MOE_KIND_GATE, MOE_KIND_UP, MOE_KIND_DOWN};
  const int pm = imp_mode(imp);
  const bool sl0 = pm == PM_SL0;
  auto sl0_fill = [&](SiteMaskArgs& ma, const LayerSave& S, int l, int si) {
    const size_t sl = (size_t)l * 3 + si;
    ma.offsets = S.offsets;
    ma.E = E;
    ma.g2 = imp.g2();
    ma.psis = imp.psi_scale();
    ma.colpart = P.sl0_col + sl * P.sl0_col_per_site;
    ma.slope = P.sl0_slope + sl * P.sl0_slope_per_site;
  };
  // the (layer, site)'s source table, or none
  const size_t src_site = (size_t)D.S * E * c;
  auto src_fill = [&](SiteMaskArgs& ma, int l, int si) {
    ma.src = nullptr;
    ma.src_dtype = PD_DTYPE_F32;
    ma.rps = 1;
    ma.S = 0;
    ma.colsrc = ma.dsrc = ma.rowdm = nullptr;
    if (!srcs) return;
    const size_t es = srcs->src_dtype == PD_DTYPE_F32 ? 4 : 2;
    ma.src = (const char*)srcs->src + ((size_t)l * 3 + si) * src_site * es;
    ma.src_dtype = srcs->src_dtype;
    ma.rps = srcs->rps;
    ma.S = D.S;
    ma.colsrc = P.colsrc;
    ma.dsrc = srcs->d_src + ((size_t)l * 3 + si) * src_site;
    ma.rowdm = P.rowdm;
  };

  // ================= K-contiguous weight copies for the forward products (once per step)
  rec.mark(MOE_CAT_CLEAN);
  const int64_t LE = (int64_t)L * E;
  // With L > 1 a helper stream takes every weight copy and the clean pass after layer 0's
  // routing: this stream forms layer 0's routing (the masked pass runs under it), then
  // starts the masked forward while the helper finishes clean layer 0 and runs clean
  // layers 1.. beside it. The two chains are independent until masked layer l reads clean
  // layer l's routing (and masked layer 0 the clean gate / up products of the frozen
  // channel), and the matrix-core phases of one overlap the VALU-bound mask passes of the
  // other. In the backward the helper stream runs the weight-gradient products. Its
  // events: start, the copies of Vg / Vu (masked layer 0's first product) and of the rest,
  // weight-gradient inputs ready [4] and done [4], layer 0's routing formed, clean layer
  // 0's gate / up products formed, clean layer l done (layer l % 64: a wait on a shared
  // event waits for the last layer recorded on it, later than needed).
  constexpr int LAYER_EVENTS = 64;
  struct {
    hipStream_t st = nullptr;
    hipEvent_t start, vcopies, copies, *wg_in, *wg_out, route0, clean0, *layer_ev;
    hipEvent_t layer(int l) const { return layer_ev[l % LAYER_EVENTS]; }
  } cs;
  const bool side = !reuse_clean && L > 1;
  AuxStream ax;  // its lease is held until this call has enqueued all of its work
  if (side || want_wgrads) {
    if ((rc0 = aux_stream(0, 14 + std::min(L, LAYER_EVENTS), ax))) return rc0;
    cs.st = ax.st;
    cs.start = ax.ev[0];
    cs.vcopies = ax.ev[1];
    cs.copies = ax.ev[2];
    cs.wg_in = ax.ev + 3;
    cs.wg_out = ax.ev + 7;
    cs.route0 = ax.ev[11];
    cs.clean0 = ax.ev[12];
    cs.layer_ev = ax.ev + 14;
  }
  if (side) {
    hipEventRecord(cs.start, s);
    hipStreamWaitEvent(cs.st, cs.start, 0);
  }
  // the frozen weights' copies (else as the previous call left them): on this stream
  // ahead of everything without the helper, after the components' copies with it
  auto frozen_copies = [&](hipStream_t st) {
    launch_batched_T(Wg, LE, d, f, P.WgT, st);
    launch_batched_T(Wu, LE, d, f, P.WuT, st);
    launch_batched_T(Wd, LE, f, d, P.WdT, st);
  };
  if (!reuse_clean && !side) frozen_copies(s);
  const hipStream_t scp = side ? cs.st : s;
  launch_batched_T(Vg, LE, d, c, P.VgT, scp);
  launch_batched_T(Vu, LE, d, c, P.VuT, scp);
  if (side) hipEventRecord(cs.vcopies, cs.st);
  launch_batched_T(Ug, LE, c, f, P.UgT, scp);
  launch_batched_T(Uu, LE, c, f, P.UuT, scp);
  launch_batched_T(Vd, LE, f, c, P.VdT, scp);
  launch_batched_T(Ud, LE, c, d, P.UdT, scp);
  if (side) {
    frozen_copies(cs.st);
    hipEventRecord(cs.copies, cs.st);
  }
  const bf16_t* VT[3] = {P.VgT, P.VuT, P.VdT};
  const bf16_t* UT[3] = {P.UgT, P.UuT, P.UdT};
  const size_t szV[3] = {szVg, szVg, szVd};
  const size_t szU[3] = {szUg, szUg, szUd};

  if (srcs && use_delta)  // persistent sources: each token's delta is its source row's
    hipLaunchKernelGGL(k_src_delta_fill, dim3((unsigned)std::min<int64_t>(cdiv(3 * L * T, 256), 4096)), dim3(256), 0,
                       s, srcs->delta, srcs->delta_dtype, D.S, srcs->rps, T, 3 * L, P.delta);
  else if (use_delta && uconst >= 0.f)  // constant sources: the delta mask is the constant too
    hipLaunchKernelGGL(k_fill_f32, dim3((unsigned)std::min<int64_t>(cdiv(3 * L * T, 256), 4096)), dim3(256), 0, s,
                       P.delta, (int64_t)3 * L * T, uconst);
  else if (use_delta)
    hipLaunchKernelGGL(k_delta_sites, dim3((unsigned)cdiv(T, 256), (unsigned)(3 * L)), dim3(256), 0, s, halves[2],
                       halves[3], T, layout, P.delta);
  if (routes)
    hipLaunchKernelGGL(k_route_blend, dim3((unsigned)std::min<int64_t>(cdiv(3 * L * T, 256), 4096)), dim3(256), 0, s,
                       use_delta ? (const float*)P.delta : nullptr, routes, (int64_t)3 * L * T, P.blend);
  auto set_delta = [&](int l) {
    for (int si = 0; si < 3; ++si) {
      const size_t o = ((size_t)l * 3 + si) * T;
      dlt[si] = use_delta ? P.delta + o : nullptr;
      bl[si] = routes ? P.blend + o : dlt[si];
      rt[si] = routes ? routes + o : nullptr;
    }
  };

  // ================= clean forward (frozen weights): pins the expert indices. Layer 0 sees
  // the masked pass's own input under the same routing, so its norm (h2, rinv), routing
  // weights, gathered x_jobs (and copy) and the gate/up products of the frozen channel
  // are written straight into the masked pass's buffers; later clean layers gather into
  // a buffer the masked pass only uses afterwards. Layer 0's routing runs on this stream,
  // the rest of the clean pass on the helper stream (when there is one). With reuse_clean the workspace still
  // holds all of it from the previous call (nothing after the clean pass writes these
  // buffers), and the clean final residual is the ping-pong buffer L layers end in.
  bf16_t* rcur = P.rc_a;
  bf16_t* rnext = P.rc_b;
  if (!reuse_clean) hipMemcpyAsync(P.rc_a, x0, (size_t)T * d * 2, hipMemcpyDeviceToDevice, s);
  for (int l = 0; l < L && reuse_clean; ++l) {
    std::swap(rcur, rnext);
    if (top_idx_out)
      hipMemcpyAsync(top_idx_out + (size_t)l * T * k, P.layers[l].idx, (size_t)T * k * 4, hipMemcpyDeviceToDevice, s);
  }
  for (int l = 0; l < L && !reuse_clean; ++l) {
    LayerSave& S = P.layers[l];
    hipStream_t sc = l == 0 ? s : cs.st;  // the routing part
    bf16_t* h2l = l == 0 ? S.h2 : P.h2c;
    hipLaunchKernelGGL(k_rmsnorm_fwd, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, sc, rcur, T, d, ln + (size_t)l * d, 1e-6f,
                       h2l, l == 0 ? S.rinv : (float*)nullptr);
    if ((rc = pd_gemm(PD_DTYPE_BF16, T, E, d, h2l, d, 0, bf(router, (size_t)l * E * d), d, 1, P.logitsc, E,
                      PD_DTYPE_F32, 1.f, 0.f, sc)))
      return rc;
    if ((rc = router_topk(P.logitsc, T, E, k, true, P.probsc, S.idx, P.wc, sc))) return rc;
    if (l == 0)
      launch_router_pinned(P.logitsc, T, E, k, S.idx, S.probs, S.w, sc);
    if ((rc = pd_routed_jobs(S.idx, T, k, E, S.sort_idx, S.inv, S.sizes, S.offsets, P.sort_ws,
                             pd_routed_jobs_workspace_size(J, E), sc)))
      return rc;
    bf16_t* xjl = l == 0 ? S.xj : P.xjc;
    hipLaunchKernelGGL(k_gather_tile, tile_grid(J, d), dim3(256), 0, sc, h2l, S.sort_idx, k, J, d, xjl,
                       (bf16_t*)nullptr);
    if (top_idx_out)
      hipMemcpyAsync(top_idx_out + (size_t)l * T * k, S.idx, (size_t)T * k * 4, hipMemcpyDeviceToDevice, sc);
    const hipStream_t sr = side ? cs.st : s;  // the rest of the layer
    if (l == 0 && side) {
      hipEventRecord(cs.route0, s);
      hipStreamWaitEvent(cs.st, cs.route0, 0);
    }
    bf16_t* gcl = l == 0 ? S.fg : P.gc;
    bf16_t* ucl = l == 0 ? S.fu : P.uc;
    if ((rc = grouped_gemm_pair(xjl, P.WgT + l * szW, gcl, xjl, P.WuT + l * szW, ucl, S.offsets, J, E, d, f,
                                PD_DTYPE_BF16, sr)))
      return rc;
    if (l == 0 && side) hipEventRecord(cs.clean0, cs.st);
    hipLaunchKernelGGL(k_swiglu_fwd_tile, tile_grid(J, f), dim3(256), 0, sr, gcl, ucl, (const float*)nullptr,
                       S.sort_idx, J, f, (const bf16_t*)nullptr, (const bf16_t*)nullptr, (const float*)nullptr,
                       (const float*)nullptr, k, P.din);
    if ((rc = grouped_gemm(P.din, P.WdT + l * szW, S.offsets, J, E, f, d, 1, P.downc, PD_DTYPE_BF16, sr, false)))
      return rc;
    hipLaunchKernelGGL(k_combine_residual, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, sr, rcur, P.downc, S.inv, P.wc, T, k, d,
                       (const bf16_t*)nullptr, (const float*)nullptr, rnext);
    std::swap(rcur, rnext);
    if (l > 0) hipEventRecord(cs.layer(l), sr);
  }
  bf16_t* rc_final = rcur;
  if ((rc = check_launch("pd_moe_stack_step clean"))) return rc;

  // ================= masked forward
  if (side) {
    rec.mark(MOE_CAT_WAIT);
    hipStreamWaitEvent(s, cs.vcopies, 0);
  }
  const bf16_t* r_in = (const bf16_t*)x0;
  for (int l = 0; l < L; ++l) {
    LayerSave& S = P.layers[l];
    if (side && l > 0) {
      rec.mark(MOE_CAT_WAIT);
      hipStreamWaitEvent(s, cs.layer(l), 0);  // clean layer l's routing
    }
    rec.mark(MOE_CAT_NORM_ROUTE);
    if (S.r != r_in) hipMemcpyAsync(S.r, r_in, (size_t)T * d * 2, hipMemcpyDeviceToDevice, s);
    if (l > 0) {  // layer 0's were formed by the clean pass
      hipLaunchKernelGGL(k_rmsnorm_fwd, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, s, S.r, T, d, ln + (size_t)l * d, 1e-6f,
                         S.h2, S.rinv);
      if ((rc = pd_gemm(PD_DTYPE_BF16, T, E, d, S.h2, d, 0, bf(router, (size_t)l * E * d), d, 1, P.logits, E,
                        PD_DTYPE_F32, 1.f, 0.f, stream)))
        return rc;
      launch_router_pinned(P.logits, T, E, k, S.idx, S.probs, S.w, s);
      hipLaunchKernelGGL(k_gather_tile, tile_grid(J, d), dim3(256), 0, s, S.h2, S.sort_idx, k, J, d, S.xj,
                         (bf16_t*)nullptr);
    }
    set_delta(l);
    auto mask_fwd = [&](int si) {
      SiteMaskArgs ma;
      ma.ci_pre = bf(ci_pre, ((size_t)l * 3 + si) * szCI);
      ma.sort_idx = S.sort_idx;
      ma.J = J;
      ma.c = c;
      site_key(kinds[si], l, ma.k0, ma.k1);
      ma.layout = layout;
      ma.p = imp.p;
      ma.delta = dlt[si];
      ma.route = rt[si];
      ma.k = k;
      ma.uconst = uconst;
      sl0_fill(ma, S, l, si);
      src_fill(ma, l, si);
      float* part = P.imp_part + ((size_t)l * 3 + si) * P.imp_per_site;
      launch_mask_fwd(ma, pm, tile_grid(J, c), s, S.h[si], S.acts[si], S.ub[si], part);
      if (sl0) {  // this site's frequencies, loss partials and backward slopes
        const size_t sl = (size_t)l * 3 + si;
        hipLaunchKernelGGL(k_sl0_finalize, dim3(sl0_blocks(E, c)), dim3(256), 0, s, ma.colpart, S.offsets, E, J, c,
                           1.f / (float)T, imp.coeff, imp.freq_coeff, imp.ref_count,
                           imp.ema.at((int64_t)sl * P.sl0_slope_per_site), P.sl0_slope + sl * P.sl0_slope_per_site,
                           P.sl0_act + sl * P.sl0_blocks_per_site, P.sl0_freq + sl * P.sl0_blocks_per_site,
                           imp.ema.on() ? P.sl0_fb + sl * P.sl0_blocks_per_site : nullptr);
      }
    };
    // ---- gate and up sites: both products of each stage in one paired launch
    rec.mark(MOE_CAT_GEMM_FWD);
    if ((rc = grouped_gemm_pair(S.xj, VT[0] + l * szV[0], S.h[0], S.xj, VT[1] + l * szV[1], S.h[1], S.offsets, J, E,
                                d, c, PD_DTYPE_BF16, stream)))
      return rc;
    // frozen channel of gate and up: x_jobs @ W[e] (layer 0: the clean pass's products)
    const bf16_t* fg = nullptr;
    const bf16_t* fu = nullptr;
    if (use_frozen) {
      fg = S.fg;
      fu = S.fu;
      if (l > 0 && !kc &&
          (rc = grouped_gemm_pair(S.xj, P.WgT + l * szW, S.fg, S.xj, P.WuT + l * szW, S.fu, S.offsets, J, E, d, f,
                                  PD_DTYPE_BF16, stream)))
        return rc;
    }
    rec.mark(MOE_CAT_MASK_FWD);
    mask_fwd(0);
    mask_fwd(1);
    if (side && l == 0) {  // every other weight copy; the clean gate / up products
      rec.mark(MOE_CAT_WAIT);
      hipStreamWaitEvent(s, cs.copies, 0);
      hipStreamWaitEvent(s, cs.clean0, 0);
    }
    rec.mark(MOE_CAT_GEMM_FWD);
    if (kc && l > 0) {  // g = bl_g (x_jobs @ Wg[e]) + acts_g @ Ug[e], u likewise: blended here
      if ((rc = grouped_gemm_kcat(S.xj, P.WgT + l * szW, d, S.acts[0], UT[0] + l * szU[0], c, S.gout, bl[0], S.xj,
                                  P.WuT + l * szW, S.acts[1], UT[1] + l * szU[1], S.uout, bl[1], S.sort_idx, k,
                                  S.offsets, J, E, f, stream)))
        return rc;
      fg = fu = nullptr;
    } else if ((rc = grouped_gemm_pair(S.acts[0], UT[0] + l * szU[0], S.gout, S.acts[1], UT[1] + l * szU[1], S.uout,
                                       S.offsets, J, E, c, f, PD_DTYPE_BF16, stream))) {
      return rc;
    }
    // ---- down site
    rec.mark(MOE_CAT_SWIGLU);
    hipLaunchKernelGGL(k_swiglu_fwd_tile, tile_grid(J, f), dim3(256), 0, s, S.gout, S.uout, S.w, S.sort_idx, J, f,
                       fg, fu, bl[0], bl[1], k, S.din);
    rec.mark(MOE_CAT_GEMM_FWD);
    if ((rc = grouped_gemm(S.din, VT[2] + l * szV[2], S.offsets, J, E, f, c, 1, S.h[2], PD_DTYPE_BF16, stream, false)))
      return rc;
    if (use_frozen && !kc &&
        (rc = grouped_gemm(S.din, P.WdT + l * szW, S.offsets, J, E, f, d, 1, S.fd, PD_DTYPE_BF16, stream, false)))
      return rc;
    rec.mark(MOE_CAT_MASK_FWD);
    mask_fwd(2);
    rec.mark(MOE_CAT_GEMM_FWD);
    if (kc) {  // down = bl_d (din @ Wd[e]) + acts_d @ Ud[e]
      if ((rc = grouped_gemm_kcat(S.din, P.WdT + l * szW, f, S.acts[2], UT[2] + l * szU[2], c, P.down, bl[2], nullptr,
                                  nullptr, nullptr, nullptr, nullptr, nullptr, S.sort_idx, k, S.offsets, J, E, d,
                                  stream)))
        return rc;
    } else if ((rc = grouped_gemm(S.acts[2], UT[2] + l * szU[2], S.offsets, J, E, c, d, 1, P.down, PD_DTYPE_BF16,
                                  stream, false))) {
      return rc;
    }
    rec.mark(MOE_CAT_COMBINE);
    bf16_t* r_out = (l + 1 < L) ? P.layers[l + 1].r : P.r_final;
    hipLaunchKernelGGL(k_combine_residual, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, s, S.r, P.down, S.inv,
                       (const float*)nullptr, T, k, d, use_frozen && !kc ? S.fd : (const bf16_t*)nullptr, bl[2],
                       r_out);
    r_in = r_out;
    if ((rc = check_launch("pd_moe_stack_step masked fwd"))) return rc;
  }
  // ================= loss (and everything after it) after the whole clean pass
  if (side) {
    rec.mark(MOE_CAT_WAIT);
    hipStreamWaitEvent(s, cs.layer(L - 1), 0);
  }
  rec.mark(MOE_CAT_COMBINE);
  const int64_t nres = T * d;
  hipLaunchKernelGGL(k_moe_recon, dim3(REC_BLOCKS), dim3(256), 0, s, P.r_final, rc_final, nres,
                     recon_coeff * 2.f / (float)nres, P.dr_a, P.rec_part);
  if (sl0)
    hipLaunchKernelGGL(k_moe_losses, dim3(1), dim3(1024), 0, s, P.rec_part, REC_BLOCKS, P.sl0_act,
                       (int64_t)(P.sl0_blocks_per_site * 3 * L), P.sl0_freq,
                       imp.ref_count > 0.f ? (int64_t)(P.sl0_blocks_per_site * 3 * L) : (int64_t)0,
                       imp.ema.on() ? (const float*)P.sl0_fb : nullptr, 1.0 / (double)nres, 1.0, recon_coeff,
                       imp.coeff, imp.freq_coeff, losses);
  else
    hipLaunchKernelGGL(k_moe_losses, dim3(1), dim3(1024), 0, s, P.rec_part, REC_BLOCKS, P.imp_part,
                       (int64_t)(P.imp_per_site * 3 * L), (const float*)nullptr, (int64_t)0, (const float*)nullptr,
                       1.0 / (double)nres, 1.0 / (double)T, recon_coeff, imp.coeff, 0.f, losses);
  // ================= backward
  bf16_t* dr = P.dr_a;
  bf16_t* dr_next = P.dr_b;
  const float imp_scale = imp.coeff / (float)T;
  const int n_wpart = (int)cdiv(f, TILE);
  // Weight gradients run on the second stream: each product starts once its inputs are
  // ready on this stream (event wg_in[i]), and this stream waits for it (wg_out[i]) before
  // it next overwrites one of those inputs, and before it returns. Nothing on this stream
  // reads a weight gradient.
  bool wpend[4] = {false, false, false, false};
  auto wgrad = [&](int i, auto&& product, bool on_caller = false) -> int {
    if (!cs.st || on_caller) return product((void*)s);
    hipEventRecord(cs.wg_in[i], s);
    hipStreamWaitEvent(cs.st, cs.wg_in[i], 0);
    const int r = product((void*)cs.st);
    hipEventRecord(cs.wg_out[i], cs.st);
    wpend[i] = true;
    return r;
  };
  auto wjoin = [&](int i) {
    if (wpend[i]) hipStreamWaitEvent(s, cs.wg_out[i], 0);
    wpend[i] = false;
  };
  for (int l = L - 1; l >= 0; --l) {
    LayerSave& S = P.layers[l];
    rec.mark(MOE_CAT_WAIT);
    wjoin(0);  // the down site's dU reads d_dout, its dV d_acts[2]
    wjoin(1);
    rec.mark(MOE_CAT_COMBINE);
    hipLaunchKernelGGL(k_gather_tile, tile_grid(J, d), dim3(256), 0, s, dr, S.sort_idx, k, J, d, P.d_dout,
                       (bf16_t*)nullptr);
    SiteMaskArgs ma;
    ma.sort_idx = S.sort_idx;
    ma.J = J;
    ma.c = c;
    ma.layout = layout;
    ma.p = imp.p;
    ma.k = k;
    ma.uconst = uconst;
    set_delta(l);
    if (srcs && srcs->rps > 1)  // each (expert, source row) group's job range, for the tables' gradient
      hipLaunchKernelGGL(k_src_group_offsets, dim3((unsigned)cdiv((int64_t)E * D.S + 1, 256)), dim3(256), 0, s,
                         S.offsets, S.sort_idx, E, k, D.S, srcs->rps, J, P.goff);
    // the source tables' gradient of site si, after its mask backward: the group sums in
    // tile order (or, one token per row, the entries the mask pass wrote), then the delta
    // table's gradient from each job's delta cotangent
    auto src_grads = [&](int si, const bf16_t* gout, const bf16_t* frozen, int width) {
      if (!srcs) return;
      float* dsrc = srcs->d_src + ((size_t)l * 3 + si) * src_site;
      if (srcs->rps > 1)
        hipLaunchKernelGGL(k_src_finalize, dim3((unsigned)cdiv((int64_t)src_site, 256)), dim3(256), 0, s, P.colsrc,
                           P.goff, E, D.S, c, dsrc);
      if (use_delta) {
        hipLaunchKernelGGL(k_job_delta_cot, dim3((unsigned)cdiv(J, 4)), dim3(256), 0, s, gout, frozen, P.rowdm,
                           (int)cdiv(c, TILE), J, width, P.qjob);
        hipLaunchKernelGGL(k_src_delta_grad, dim3((unsigned)cdiv(D.S, 4)), dim3(256), 0, s, P.qjob, S.inv, D.S,
                           srcs->rps, k, srcs->d_src_delta + ((size_t)l * 3 + si) * D.S);
      }
    };
    auto src_zero = [&](int si) {  // one token per row: the mask pass writes only the selected entries
      if (srcs && srcs->rps == 1)
        hipLaunchKernelGGL(k_zero_f32, dim3((unsigned)std::min<int64_t>(cdiv((int64_t)src_site, 256), 8192)),
                           dim3(256), 0, s, srcs->d_src + ((size_t)l * 3 + si) * src_site, (int64_t)src_site);
    };
    // ---- down site: d_acts, with the backward mask as its epilogue where it applies
    SiteMaskArgs mg[3];
    for (int si = 0; si < 3; ++si) {
      mg[si] = ma;
      mg[si].ci_pre = bf(ci_pre, ((size_t)l * 3 + si) * szCI);
      site_key(kinds[si], l, mg[si].k0, mg[si].k1);
      mg[si].delta = dlt[si];
      mg[si].route = rt[si];
      sl0_fill(mg[si], S, l, si);
      src_fill(mg[si], l, si);
    }
    bf16_t* dpre[3];
    for (int si = 0; si < 3; ++si) dpre[si] = (bf16_t*)d_ci_pre + ((size_t)l * 3 + si) * szCI;
    const bool fuse_d = mask_bwd_fusable(mg[2], S.h[2], S.ub[2], dpre[2], P.d_acts[2], d);
    rec.mark(fuse_d ? MOE_CAT_GEMM_MASK : MOE_CAT_GEMM_DX);
    if (fuse_d)
      rc = grouped_gemm_mask_bwd(P.d_dout, bf(Ud, l * szUd), P.d_acts[2], mg[2], S.h[2], S.ub[2], dpre[2], nullptr,
                                 nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, S.offsets, J, E, d, c, pm,
                                 imp_scale, s);
    else
      rc = grouped_gemm(P.d_dout, bf(Ud, l * szUd), S.offsets, J, E, d, c, 1, P.d_acts[2], PD_DTYPE_BF16, stream,
                        false);
    if (rc) return rc;
    rec.mark(MOE_CAT_GEMM_DW);
    if (want_wgrads && (rc = wgrad(0, [&](void* st) {
                          return pd_grouped_gemm_dw(S.acts[2], P.d_dout, S.offsets, J, E, c, d, dUd + l * szUd,
                                                    PD_DTYPE_F32, st);
                        })))
      return rc;
    rec.mark(MOE_CAT_MASK_BWD);
    src_zero(2);
    if (!fuse_d) launch_mask_bwd(mg[2], pm, tile_grid(J, c), s, S.h[2], S.ub[2], imp_scale, P.d_acts[2], dpre[2]);
    src_grads(2, P.d_dout, S.fd, d);
    rec.mark(MOE_CAT_GEMM_DW);
    if (want_wgrads && (rc = wgrad(1, [&](void* st) {
                          return pd_grouped_gemm_dw(S.din, P.d_acts[2], S.offsets, J, E, f, c, dVd + l * szVd,
                                                    PD_DTYPE_F32, st);
                        })))
      return rc;
    rec.mark(MOE_CAT_GEMM_DX);
    if (kc) {  // d_din = bl_d (d_out @ Wd[e]^T) + d_h @ Vd[e]^T
      if ((rc = grouped_gemm_kcat(P.d_dout, bf(Wd, l * szW), d, P.d_acts[2], bf(Vd, l * szVd), c, P.d_din, bl[2],
                                  nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, S.sort_idx, k, S.offsets, J, E,
                                  f, stream)))
        return rc;
    } else if ((rc = grouped_gemm(P.d_acts[2], bf(Vd, l * szVd), S.offsets, J, E, c, f, 1, P.d_din, PD_DTYPE_BF16,
                                  stream, false))) {
      return rc;
    }
    // frozen channel of down: d_out @ W_down[e]^T, scaled by the token's delta in the fold
    if (use_frozen && !kc &&
        (rc = grouped_gemm(P.d_dout, bf(Wd, l * szW), S.offsets, J, E, d, f, 1, P.gc, PD_DTYPE_BF16, stream, false)))
      return rc;
    rec.mark(MOE_CAT_WAIT);
    wjoin(2);  // dU of gate / up reads d_g, d_u
    rec.mark(MOE_CAT_SWIGLU);
    hipLaunchKernelGGL(k_swiglu_bwd_tile, tile_grid(J, f), dim3(256), 0, s, P.d_din, S.gout, S.uout, S.w, S.sort_idx,
                       J, f, use_frozen && !kc ? P.gc : (const bf16_t*)nullptr, bl[2], k, P.d_g, P.d_u,
                       P.d_w_part);
    // ---- gate and up sites: paired launches
    rec.mark(MOE_CAT_WAIT);
    wjoin(3);  // the previous layer's gate / up dV read d_acts[0], d_acts[1]
    const bool fuse_gu = mask_bwd_fusable(mg[0], S.h[0], S.ub[0], dpre[0], P.d_acts[0], f) &&
                         mask_bwd_fusable(mg[1], S.h[1], S.ub[1], dpre[1], P.d_acts[1], f);
    rec.mark(fuse_gu ? MOE_CAT_GEMM_MASK : MOE_CAT_GEMM_DX);
    if (fuse_gu)
      rc = grouped_gemm_mask_bwd(P.d_g, bf(Ug, l * szUg), P.d_acts[0], mg[0], S.h[0], S.ub[0], dpre[0], P.d_u,
                                 bf(Uu, l * szUg), P.d_acts[1], &mg[1], S.h[1], S.ub[1], dpre[1], S.offsets, J, E, f, c,
                                 pm, imp_scale, s);
    else
      rc = grouped_gemm_pair(P.d_g, bf(Ug, l * szUg), P.d_acts[0], P.d_u, bf(Uu, l * szUg), P.d_acts[1], S.offsets, J,
                             E, f, c, PD_DTYPE_BF16, stream);
    if (rc) return rc;
    rec.mark(MOE_CAT_GEMM_DW);
    if (want_wgrads && (rc = wgrad(2, [&](void* st) {
                          return grouped_gemm_dw_pair(S.acts[0], P.d_g, dUg + l * szUg, S.acts[1], P.d_u,
                                                      dUu + l * szUg, S.offsets, J, E, c, f, PD_DTYPE_F32, st);
                        })))
      return rc;
    rec.mark(MOE_CAT_MASK_BWD);
    for (int si = 0; si < 2; ++si) {
      src_zero(si);
      if (!fuse_gu) launch_mask_bwd(mg[si], pm, tile_grid(J, c), s, S.h[si], S.ub[si], imp_scale, P.d_acts[si], dpre[si]);
      src_grads(si, si == 0 ? P.d_g : P.d_u, si == 0 ? S.fg : S.fu, f);
    }
    // layer 0's gate / up dV products are the step's last work: this stream has nothing
    // else left, so they run here, beside the helper's dU products, instead of after them
    rec.mark(MOE_CAT_GEMM_DW);
    if (want_wgrads && (rc = wgrad(
                            3,
                            [&](void* st) {
                              return grouped_gemm_dw_pair(S.xj, P.d_acts[0], dVg + l * szVg, S.xj, P.d_acts[1],
                                                          dVu + l * szVg, S.offsets, J, E, d, c, PD_DTYPE_F32, st);
                            },
                            l == 0)))
      return rc;
    // The stack input carries no parameter gradient: layer 0 stops at its weight
    // gradients (its gate/up input products and the token backward feed only d x0).
    if (l > 0) {
      rec.mark(MOE_CAT_GEMM_DX);
      if (kc) {  // dx_g = bl_g (d_g @ Wg[e]^T) + d_h_g @ Vg[e]^T, dx_u likewise
        if ((rc = grouped_gemm_kcat(P.d_g, bf(Wg, l * szW), f, P.d_acts[0], bf(Vg, l * szVg), c, P.dxa, bl[0], P.d_u,
                                    bf(Wu, l * szW), P.d_acts[1], bf(Vu, l * szVg), P.dxb, bl[1], S.sort_idx, k,
                                    S.offsets, J, E, d, stream)))
          return rc;
      } else if ((rc = grouped_gemm_pair(P.d_acts[0], bf(Vg, l * szVg), P.dxa, P.d_acts[1], bf(Vu, l * szVg), P.dxb,
                                         S.offsets, J, E, c, d, PD_DTYPE_BF16, stream))) {
        return rc;
      }
      // frozen channel of gate and up: d_g @ Wg[e]^T, d_u @ Wu[e]^T
      if (use_frozen && !kc &&
          (rc = grouped_gemm_pair(P.d_g, bf(Wg, l * szW), P.downc, P.d_u, bf(Wu, l * szW), P.down, S.offsets, J, E, f,
                                  d, PD_DTYPE_BF16, stream)))
        return rc;
      // ---- routing weights, router, gather VJP and the norm
      rec.mark(MOE_CAT_TOKEN_BWD);
      launch_token_bwd(P.d_w_part, n_wpart, S.inv, S.idx, S.probs, S.w, bf(router, (size_t)l * E * d), P.dxa, P.dxb,
                       S.r, S.rinv, ln + (size_t)l * d, dr, T, E, k, d,
                       use_frozen && !kc ? P.downc : (const bf16_t*)nullptr,
                       P.down, bl[0], bl[1], dr_next, s);
      std::swap(dr, dr_next);
    }
    if ((rc = check_launch("pd_moe_stack_step bwd"))) return rc;
  }
  rec.mark(MOE_CAT_WAIT);
  for (int i = 0; i < 4; ++i) wjoin(i);
  rec.mark(MOE_CAT_END);
  return PD_OK;
}

int pd_moe_stack_step(int64_t T, int d, int f, int E, int k, int c, int L, const void* x0, const float* ln,
                      const void* router, const void* Wg, const void* Wu, const void* Wd, const void* Vg,
                      const void* Ug, const void* Vu, const void* Uu, const void* Vd, const void* Ud, const void* ci_pre,
                      uint32_t draw_k0, uint32_t draw_k1, int use_delta, const uint8_t* routes, float source_value,
                      int layout, int imp_kind, float p, float gamma, int normalize_at_one, float imp_coeff,
                      float freq_coeff, float ref_count, const float* freq_ema_in, float* freq_ema_out,
                      float ema_count, float ema_halflife, float recon_coeff, float* losses, float* dVg, float* dUg,
                      float* dVu, float* dUu, float* dVd, float* dUd, void* d_ci_pre, int32_t* top_idx_out,
                      void* workspace, size_t workspace_bytes, void* stream) {
  Recorder rec{nullptr, nullptr, 0, 0, nullptr};
  ImpSpec imp;
  if (int e = make_imp_spec("pd_moe_stack_step", imp_kind, p, gamma, normalize_at_one, imp_coeff, freq_coeff,
                            ref_count, freq_ema_in, freq_ema_out, ema_count, ema_halflife, imp))
    return e;
  return moe_step_impl(T, d, f, E, k, c, L, x0, ln, router, Wg, Wu, Wd, Vg, Ug, Vu, Uu, Vd, Ud, ci_pre, draw_k0,
                       draw_k1, use_delta, routes, source_value, layout, imp, recon_coeff, losses, dVg, dUg, dVu, dUu,
                       dVd, dUd, d_ci_pre, top_idx_out, workspace, workspace_bytes, stream, rec);
}

int pd_moe_stack_step_sources(int64_t T, int d, int f, int E, int k, int c, int L, const void* x0, const float* ln,
                              const void* router, const void* Wg, const void* Wu, const void* Wd, const void* Vg,
                              const void* Ug, const void* Vu, const void* Uu, const void* Vd, const void* Ud,
                              const void* ci_pre, const void* src, int src_dtype, const void* src_delta,
                              int delta_dtype, int64_t rows_per_source, int imp_kind, float p, float gamma,
                              int normalize_at_one, float imp_coeff, float freq_coeff, float ref_count,
                              const float* freq_ema_in, float* freq_ema_out, float ema_count, float ema_halflife,
                              float recon_coeff, int want_weight_grads, int reuse_clean, float* losses, float* dVg,
                              float* dUg, float* dVu, float* dUu, float* dVd, float* dUd, void* d_ci_pre,
                              float* d_src, float* d_src_delta, int32_t* top_idx_out, void* workspace,
                              size_t workspace_bytes, void* stream) {
  Recorder rec{nullptr, nullptr, 0, 0, nullptr};
  ImpSpec imp;
  if (int e = make_imp_spec("pd_moe_stack_step_sources", imp_kind, p, gamma, normalize_at_one, imp_coeff,
                            freq_coeff, ref_count, freq_ema_in, freq_ema_out, ema_count, ema_halflife, imp))
    return e;
  const SrcArgs sa{src, src_dtype, src_delta, delta_dtype, rows_per_source, want_weight_grads, d_src, d_src_delta};
  if (rows_per_source <= 0 || T % rows_per_source)
    return fail(PD_EINVAL, "pd_moe_stack_step_sources: rows_per_source must divide T");
  const MoEDims D{T, T * k, d, f, E, k, c, L, T / rows_per_source};
  if (!workspace || workspace_bytes < plan(D, nullptr, true).total)
    return fail(PD_EWORKSPACE, "pd_moe_stack_step_sources: workspace too small");
  return moe_step_impl(T, d, f, E, k, c, L, x0, ln, router, Wg, Wu, Wd, Vg, Ug, Vu, Uu, Vd, Ud, ci_pre, 0, 0,
                       src_delta != nullptr, nullptr, -1.f, PD_LAYOUT_PARTITIONABLE, imp, recon_coeff, losses, dVg,
                       dUg, dVu, dUu, dVd, dUd, d_ci_pre, top_idx_out, workspace, workspace_bytes, stream, rec, &sa,
                       reuse_clean != 0);
}

int pd_moe_stack_step_timed(int64_t T, int d, int f, int E, int k, int c, int L, const void* x0, const float* ln,
                            const void* router, const void* Wg, const void* Wu, const void* Wd, const void* Vg,
                            const void* Ug, const void* Vu, const void* Uu, const void* Vd, const void* Ud,
                            const void* ci_pre, uint32_t draw_k0, uint32_t draw_k1, int use_delta,
                            const uint8_t* routes, float source_value, int layout, int imp_kind, float p, float gamma,
                            int normalize_at_one, float imp_coeff, float freq_coeff, float ref_count,
                            const float* freq_ema_in, float* freq_ema_out, float ema_count, float ema_halflife,
                            float recon_coeff, float* losses, float* dVg, float* dUg, float* dVu, float* dUu,
                            float* dVd, float* dUd, void* d_ci_pre, int32_t* top_idx_out, void* workspace,
                            size_t workspace_bytes, void* stream, void** events, int32_t* categories, int capacity,
                            int* n_recorded) {
  if (!events || !categories || capacity <= 0 || !n_recorded)
    return fail(PD_EINVAL, "pd_moe_stack_step_timed: events/categories required");
  Recorder rec{events, categories, capacity, 0, nullptr};
  ImpSpec imp;
  if (int e = make_imp_spec("pd_moe_stack_step_timed", imp_kind, p, gamma, normalize_at_one, imp_coeff, freq_coeff,
                            ref_count, freq_ema_in, freq_ema_out, ema_count, ema_halflife, imp))
    return e;
  int rc = moe_step_impl(T, d, f, E, k, c, L, x0, ln, router, Wg, Wu, Wd, Vg, Ug, Vu, Uu, Vd, Ud, ci_pre, draw_k0,
                         draw_k1, use_delta, routes, source_value, layout, imp, recon_coeff, losses, dVg, dUg, dVu,
                         dUu, dVd, dUd, d_ci_pre, top_idx_out, workspace, workspace_bytes, stream, rec);
  *n_recorded = rec.n;
  if (rc == PD_OK && rec.n >= capacity) return fail(PD_EINVAL, "pd_moe_stack_step_timed: event capacity too small");
  return rc;
}

}  // extern "C"
