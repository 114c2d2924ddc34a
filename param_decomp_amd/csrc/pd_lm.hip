// The decomposed Llama-style LM step (gfx950): L pre-RMSNorm transformer blocks
//   h = rms_norm(r, ln1)                        pd/target_ports/llama.py:90-97
//   q, k, v = site(h); a = causal_attention(rope(q), rope(k), v)
//                                               pd/targets/transformer.py:701-747, 1085-1100
//   r1 = r + site_o(a); h2 = rms_norm(r1, ln2)
//   r2 = r1 + site_down(gelu_tanh(site_fc(h2))) pd/targets/transformer.py:1101-1140, 802-805
// with every q/k/v/o/c_fc/down matrix decomposed (site = ((x@V) * (m - d)) @ U + d * (x @ W^T),
// pd/core/decomposed_linear.py:142-175), stochastic masks drawn in-block per (kind, layer)
// (pd/targets/transformer.py:1048-1058, 1424-1451), the final norm and the tied head, the
// streamed per-position KL against the frozen forward (pd/targets/losses.py:102-163), the
// L_p imp-min over the upper CI, and the full backward to every site's V/U and CI
// preactivations (the attention is frozen: gradients flow through it).
//
// Layouts: activations row-major [N = B*T, width] bf16. Every product runs on the
// buffer-fed MFMA kernel. The weights are read K-contiguous (an MN-contiguous operand
// costs the product 6-20% here), from per-step transposed copies made by one batched
// launch per (kind, matrix) for all layers; activations are read as stored, MN-contiguous
// where the contraction runs over tokens:
//   x @ V            B = V^T [C, d_in] (copy)
//   out              s (.) (x @ W^T) + acts @ U in one two-segment product (W as stored,
//                    U^T [d_out, C] copy), s = d on routed rows and 1 on the rest
//   d_acts           g @ U^T: U as stored
//   dU = acts^T g    A = acts [N, C] (MN-major), B = g^T [d_out, N] (a per-call copy the
//                    helper stream reads while this stream moves on)
//   dV = x^T dxV     A = x [N, d_in], B = dxV [N, C] (both MN-major)
//   d_input          s (.) (g @ W) + dxV @ V^T in one two-segment product (W^T [d_in,
//                    d_out] copy, V as stored)
// Attention (hd = 64) is fused per (batch, head) with nothing T x T stored: the forward
// forms each query row's softmax max and sum, then O = P V with P = bf16(softmax(Q K^T /
// sqrt(hd))) over 32-key blocks in registers, keeping the row stats and the fp32 O; the
// backward recomputes P from the stats and forms dS = bf16(P (dP - D) / sqrt(hd)) (dP =
// dO V^T, D = rowsum(P dP) = rowsum(dO O)), dQ = dS K per query tile and dK = dS^T Q,
// dV = P^T dO per key tile.
#include <algorithm>
#include <vector>

#include "pd_common.hpp"
#include "pd_gemm_dtl.hpp"
#include "pd_impmin.hpp"

namespace pd {

enum { LK_Q = 0, LK_K = 1, LK_V = 2, LK_O = 3, LK_FC = 4, LK_DOWN = 5, LM_NK = 6 };  // KIND_ORDER indices
static constexpr int LM_HD = 64;

// ---------------------------------------------------------------- token-space kernels
// r[n, :] = wte[tok[n], :] (ids clamped into [0, V)); one wave per token, d % 8 == 0.
__global__ __launch_bounds__(256) void k_lm_embed(const int32_t* __restrict__ tok, const bf16_t* __restrict__ wte,
                                                  int64_t N, int d, int64_t V, bf16_t* __restrict__ r) {
  const int64_t n = (int64_t)blockIdx.x * 4 + wave_id();
  if (n >= N) return;
  int64_t t = tok[n];
  t = t < 0 ? 0 : (t >= V ? V - 1 : t);
  for (int i = (threadIdx.x & 63) * 8; i < d; i += 512) *(uint4*)(r + n * d + i) = *(const uint4*)(wte + t * d + i);
}

// y = bf16(w * bf16(x * rinv)), rinv = rsqrt(mean x^2 + eps) kept for the backward
// (the reference rounds the normalized value to the activation dtype before the weight
// multiply). One wave per token.
__global__ __launch_bounds__(256) void k_lm_rms_fwd(const bf16_t* __restrict__ x, int64_t N, int d,
                                                    const float* __restrict__ w, float eps, bf16_t* __restrict__ y,
                                                    float* __restrict__ rinv) {
  const int64_t n = (int64_t)blockIdx.x * 4 + wave_id();
  if (n >= N) return;
  const int lane = threadIdx.x & 63;
  const bf16_t* xr = x + n * d;
  float ss = 0.f, v[8];
  for (int i = lane * 8; i < d; i += 512) {
    load8(xr + i, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(v[j], v[j], ss);
  }
  const float r = rsqrtf(wave_sum(ss) / (float)d + eps);
  if (rinv && lane == 0) rinv[n] = r;
  for (int i = lane * 8; i < d; i += 512) {
    float g[8];
    load8(xr + i, v);
    load8f(w + i, g);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = g[j] * bf16_to_f32(f32_to_bf16(v[j] * r));
    store8(y + n * d + i, v);
  }
}

// RMSNorm pullback added into the residual cotangent:
//   d_out[n,:] = bf16(d_in[n,:] + rinv * (w dy) - x * rinv^3 * mean((w dy) x))
// with dy fp32 (the straight-through derivative of the bf16 rounding of x * rinv).
// d_in NULL = 0. One wave per token.
__global__ __launch_bounds__(256) void k_lm_rms_bwd(const float* __restrict__ dy, const bf16_t* __restrict__ x,
                                                    const float* __restrict__ rinv, const float* __restrict__ w,
                                                    int64_t N, int d, const bf16_t* __restrict__ d_in,
                                                    bf16_t* __restrict__ d_out) {
  const int64_t n = (int64_t)blockIdx.x * 4 + wave_id();
  if (n >= N) return;
  const int lane = threadIdx.x & 63;
  const float r = rinv[n];
  float dot = 0.f, xv[8], gv[8], wv[8];
  for (int i = lane * 8; i < d; i += 512) {
    load8(x + n * d + i, xv);
    load8f(dy + n * d + i, gv);
    load8f(w + i, wv);
#pragma unroll
    for (int j = 0; j < 8; ++j) dot = fmaf(wv[j] * gv[j], xv[j], dot);
  }
  const float c = wave_sum(dot) / (float)d * r * r * r;
  for (int i = lane * 8; i < d; i += 512) {
    float o[8], di[8];
    load8(x + n * d + i, xv);
    load8f(dy + n * d + i, gv);
    load8f(w + i, wv);
    if (d_in) load8(d_in + n * d + i, di);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = (d_in ? di[j] : 0.f) + r * wv[j] * gv[j] - xv[j] * c;
    store8(d_out + n * d + i, o);
  }
}

// out = bf16(a + b), 8 elements per thread (n % 8 == 0).
__global__ __launch_bounds__(256) void k_lm_add(const bf16_t* __restrict__ a, const bf16_t* __restrict__ b, int64_t n,
                                                bf16_t* __restrict__ out) {
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += (int64_t)gridDim.x * 256 * 8) {
    float x[8], y[8];
    load8(a + i, x);
    load8(b + i, y);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] += y[j];
    store8(out + i, x);
  }
}

// dst[c * ld + r] = src[r * Cc + c] (src [R, Cc]; R, Cc, ld multiples of 8, dst 16-byte
// aligned): 64x64 tiles through a transposed LDS tile.
__global__ __launch_bounds__(256) void k_lm_transpose(const bf16_t* __restrict__ src, int64_t R, int64_t Cc,
                                                      bf16_t* __restrict__ dst, int64_t ld) {
  __shared__ TTile Tt;
  const int64_t r0 = (int64_t)blockIdx.y * TILE, c0 = (int64_t)blockIdx.x * TILE;
  const int tid = threadIdx.x, c8 = (tid & 7) * 8;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int r = (tid >> 3) + 32 * pass;
    uint4 v = {0, 0, 0, 0};
    if (r0 + r < R && c0 + c8 < Cc) v = *(const uint4*)(src + (r0 + r) * Cc + c0 + c8);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      Tt.v[c8 + 2 * e][r] = (bf16_t)(w[e] & 0xFFFFu);
      Tt.v[c8 + 2 * e + 1][r] = (bf16_t)(w[e] >> 16);
    }
  }
  __syncthreads();
  ttile_store(Tt, dst, ld, r0, R, c0, Cc, tid);
}

// dst[b] = src[b]^T, b = blockIdx.z, for [R, Cc] matrices (R, Cc multiples of 8).
__global__ __launch_bounds__(256) void k_lm_transpose_b(const bf16_t* __restrict__ src, int64_t R, int64_t Cc,
                                                        bf16_t* __restrict__ dst) {
  __shared__ TTile Tt;
  const int64_t b = blockIdx.z;
  const bf16_t* sb = src + b * R * Cc;
  const int64_t r0 = (int64_t)blockIdx.y * TILE, c0 = (int64_t)blockIdx.x * TILE;
  const int tid = threadIdx.x, c8 = (tid & 7) * 8;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int r = (tid >> 3) + 32 * pass;
    uint4 v = {0, 0, 0, 0};
    if (r0 + r < R && c0 + c8 < Cc) v = *(const uint4*)(sb + (r0 + r) * Cc + c0 + c8);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      Tt.v[c8 + 2 * e][r] = (bf16_t)(w[e] & 0xFFFFu);
      Tt.v[c8 + 2 * e + 1][r] = (bf16_t)(w[e] >> 16);
    }
  }
  __syncthreads();
  ttile_store(Tt, dst + b * R * Cc, R, r0, R, c0, Cc, tid);
}

// Per-token delta draws of every (layer, kind): delta[(l * 6 + k) * N + n] =
// uniform_bf16(fold_in(fold_in(delta_base, k), l), [N])[n] (pd/core/masking.py:139-140
// under the keys of pd/targets/transformer.py:1424-1451). Grid (cdiv(N, 256), 6L).
__global__ __launch_bounds__(256) void k_lm_deltas(uint32_t b0, uint32_t b1, int64_t N, int layout,
                                                   float* __restrict__ delta) {
  const int site = blockIdx.y;
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  uint32_t x0 = 0, x1 = (uint32_t)(site % LM_NK);
  threefry2x32(b0, b1, x0, x1);
  uint32_t k0 = 0, k1 = (uint32_t)(site / LM_NK);
  threefry2x32(x0, x1, k0, k1);
  delta[(int64_t)site * N + n] = draw_uniform(k0, k1, n, N, PD_DTYPE_BF16, layout);
}

// ---------------------------------------------------------------- site mask passes (64x64 tiles)
struct LMMaskArgs {
  const bf16_t* ci_pre;  // [N, C] bf16
  int64_t N;
  int C;
  uint32_t k0, k1;
  float p;
  const float* delta;    // [N] or NULL (d = 0)
  const uint8_t* route;  // [N] or NULL (every token routed); unrouted tokens take the target
  int64_t ld;            // row stride of acts / d_xV (the concatenated operand)
  // smooth-L0 imp-min (PM_SL0): psi = psis * v^2 / (v^2 + g2); per-tile column sums of
  // psi out (colpart), per-component slopes in (slope)
  float g2, psis;
  float* colpart;
  const float* slope;
  // persistent source tables (MASK_SRC): src [S, C] of this (layer, kind), S = N / rps; the
  // backward writes the table's gradient dm (1 - lower) as per-(64-token tile, source row)
  // column sums colsrc (rps > 1; tiles and rows both run in token order, so tile + row is
  // unique) or straight into dsrc [N, C] (rps = 1), and each token's per-tile sums of dm
  // into rowdm [N, tiles of C] (for the delta table's gradient)
  const void* src = nullptr;
  int src_dtype = PD_DTYPE_F32;
  int64_t rps = 1;
  float* colsrc = nullptr;
  float* dsrc = nullptr;
  float* rowdm = nullptr;
};

#define PD_LM_ROW(pass) ((threadIdx.x >> 4) + 16 * (pass))
#define PD_LM_COL ((threadIdx.x & 15) * 4)

// m = lower(ci) + (1 - lower(ci)) u (u drawn in bf16 over [N, C], counter n*C + c);
// acts = bf16(xV * (m - d)) into acts[n * ld + c] (0 on unrouted tokens,
// whose output is the target's x @ W^T, pd/core/decomposed_linear.py:72-85); u kept as its
// 7-bit integer; per-block partial of upper(ci)^p. C % 8 == 0, N % 8 == 0. LAYOUT ==
// MASK_SRC reads u from the source table instead (u = bf16(src[n / rps, c])), no u bytes.
template <int LAYOUT, int PM>
__global__ __launch_bounds__(256) void k_lm_mask_fwd(LMMaskArgs a, const bf16_t* __restrict__ xV,
                                                     bf16_t* __restrict__ acts, uint8_t* __restrict__ ubits,
                                                     float* __restrict__ imp_part) {
  __shared__ float red[4];
  __shared__ typename std::conditional<PM == PM_SL0, Sl0Tile, NoSl0Tile>::type SLv;
  const int tid = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.y * TILE;
  const int q0 = blockIdx.x * TILE, q4 = PD_LM_COL;
  const int64_t total = a.N * a.C;
  const bool qok = q0 + q4 < a.C;
  if constexpr (PM == PM_SL0) sl0_tile_groups(SLv, nullptr, 1, n0, a.N, tid);
  // source tables: each row's table row n / rps, divided once per row instead of per pass
  __shared__ int srow[LAYOUT == MASK_SRC ? TILE : 1];
  if constexpr (LAYOUT == MASK_SRC) {
    if (tid < TILE) srow[tid] = n0 + tid < a.N ? (int)((n0 + tid) / a.rps) : 0;
    __syncthreads();
  }
  float imp = 0.f;
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int r = PD_LM_ROW(pass);
    const int64_t n = n0 + r;
    bf16_t o[4] = {0, 0, 0, 0};
    if (n < a.N && qok) {
      const int64_t idx = n * a.C + q0 + q4;
      const float dt = a.delta ? a.delta[n] : 0.f;
      const bool routed = !a.route || a.route[n];
      const uint2 pw = *(const uint2*)(a.ci_pre + idx);
      const uint2 hw = *(const uint2*)(xV + idx);
      const float pre[4] = {bf_lo(pw.x), bf_hi(pw.x), bf_lo(pw.y), bf_hi(pw.y)};
      const float hv[4] = {bf_lo(hw.x), bf_hi(hw.x), bf_lo(hw.y), bf_hi(hw.y)};
      uint32_t ub = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = lower_fwd(pre[e]);
        if constexpr (PM == PM_SL0) SLv.ps[r][q4 + e] = sl0_psi(upper_fwd(pre[e]), a.g2, a.psis);
        else imp += powp<PM>(upper_fwd(pre[e]), a.p);
        float u;
        if constexpr (LAYOUT == MASK_SRC) {
          u = src_value(a.src, a.src_dtype, (int64_t)srow[r] * a.C + q0 + q4 + e);
        } else {
          const uint32_t kb = (draw_bits(a.k0, a.k1, idx + e, total, 8, LAYOUT) & 0xFFu) >> 1;
          ub |= kb << (8 * e);
          u = (float)kb * (1.f / 128.f);
        }
        o[e] = routed ? f32_to_bf16(hv[e] * (lo + (1.f - lo) * u - dt)) : (bf16_t)0;
      }
      if constexpr (LAYOUT != MASK_SRC) *(uint32_t*)(ubits + idx) = ub;
      *(uint2*)(acts + n * a.ld + q0 + q4) = make_uint2(bf_pack(o[0], o[1]), bf_pack(o[2], o[3]));
    } else if constexpr (PM == PM_SL0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) SLv.ps[r][q4 + e] = 0.f;
    }
  }
  if constexpr (PM == PM_SL0) {
    __syncthreads();
    sl0_tile_colsums(SLv, blockIdx.y, q0, a.C, a.colpart, tid);
  } else {
    imp = wave_sum(imp);
    if ((tid & 63) == 0) red[tid >> 6] = imp;
    __syncthreads();
    if (tid == 0) imp_part[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = red[0] + red[1] + red[2] + red[3];
  }
}

// d_xV = bf16(d_acts * (m - d)) into d_xV[n * ld + c]; the CI pullback
// d_pre = lower_vjp(pre, d_acts * xV * (1 - u)) + upper_vjp(pre, imp_scale * d upper^p).
// An unrouted token's masked product does not reach the output: d_acts counts as 0 there.
// SRC: u is read back from the source table, whose gradient dm (1 - lower) (dm = d_acts xV)
// goes to dsrc (rps = 1) or the tile's column sums per source row (colsrc), and each
// token's row sum of dm over the tile to rowdm.
template <int PM, bool SRC>
__global__ __launch_bounds__(256) void k_lm_mask_bwd(LMMaskArgs a, const bf16_t* __restrict__ xV,
                                                     const uint8_t* __restrict__ ubits, float imp_scale,
                                                     const bf16_t* __restrict__ d_acts, bf16_t* __restrict__ d_xV,
                                                     bf16_t* __restrict__ d_pre) {
  __shared__ typename std::conditional<SRC, Sl0Tile, NoSl0Tile>::type SG;
  const int tid = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.y * TILE;
  const int q0 = blockIdx.x * TILE, q4 = PD_LM_COL;
  const bool qok = q0 + q4 < a.C;
  if constexpr (SRC) {
    if (tid < 64) SG.grp[tid] = n0 + tid < a.N ? (int)((n0 + tid) / a.rps) : -1;  // each row's source row
    __syncthreads();
  }
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int r = PD_LM_ROW(pass);
    const int64_t n = n0 + r;
    bf16_t o[4] = {0, 0, 0, 0};
    float dmsum = 0.f;
    if (n < a.N && qok) {
      const int64_t idx = n * a.C + q0 + q4;
      const float dt = a.delta ? a.delta[n] : 0.f;
      const uint2 pw = *(const uint2*)(a.ci_pre + idx);
      const uint2 hw = *(const uint2*)(xV + idx);
      const uint2 dw = (!a.route || a.route[n]) ? *(const uint2*)(d_acts + idx) : make_uint2(0u, 0u);
      const uint32_t ub = SRC ? 0u : *(const uint32_t*)(ubits + idx);
      const float pre[4] = {bf_lo(pw.x), bf_hi(pw.x), bf_lo(pw.y), bf_hi(pw.y)};
      const float hv[4] = {bf_lo(hw.x), bf_hi(hw.x), bf_lo(hw.y), bf_hi(hw.y)};
      const float da[4] = {bf_lo(dw.x), bf_hi(dw.x), bf_lo(dw.y), bf_hi(dw.y)};
      bf16_t dp[4];
      float slope4[4] = {imp_scale, imp_scale, imp_scale, imp_scale};
      if constexpr (PM == PM_SL0) {
        const float4 sl = *(const float4*)(a.slope + q0 + q4);
        slope4[0] = sl.x;
        slope4[1] = sl.y;
        slope4[2] = sl.z;
        slope4[3] = sl.w;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = lower_fwd(pre[e]), up = upper_fwd(pre[e]);
        float u;
        if constexpr (SRC) u = src_value(a.src, a.src_dtype, (int64_t)SG.grp[r] * a.C + q0 + q4 + e);
        else u = (float)((ub >> (8 * e)) & 0xFFu) * (1.f / 128.f);
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
          if (a.rps == 1) a.dsrc[idx + e] = gs;
          else SG.ps[r][q4 + e] = gs;
        }
      }
      *(uint2*)(d_pre + idx) = make_uint2(bf_pack(dp[0], dp[1]), bf_pack(dp[2], dp[3]));
      *(uint2*)(d_xV + n * a.ld + q0 + q4) = make_uint2(bf_pack(o[0], o[1]), bf_pack(o[2], o[3]));
    } else if constexpr (SRC) {
#pragma unroll
      for (int e = 0; e < 4; ++e) SG.ps[r][q4 + e] = 0.f;
    }
    if constexpr (SRC) {  // the 16 lanes of a row add their columns in a fixed tree (all lanes)
      dmsum += __shfl_xor(dmsum, 1, 64);
      dmsum += __shfl_xor(dmsum, 2, 64);
      dmsum += __shfl_xor(dmsum, 4, 64);
      dmsum += __shfl_xor(dmsum, 8, 64);
      if (n < a.N && (tid & 15) == 0 && a.rowdm) a.rowdm[n * gridDim.x + blockIdx.x] = dmsum;
    }
  }
  if constexpr (SRC) {
    __syncthreads();
    if (a.rps > 1) sl0_tile_colsums(SG, blockIdx.y, q0, a.C, a.colsrc, tid);
  }
}

// The source table's gradient from the tiles' column sums (rps > 1): d_src[g C + q] = the
// sum over the 64-token tiles covering source row g (tokens [g rps, (g + 1) rps)) of
// colsrc[(tile + g) C + q], tiles in order.
__global__ __launch_bounds__(256) void k_lm_src_finalize(const float* __restrict__ colsrc, int64_t N, int64_t rps,
                                                         int64_t S, int C, float* __restrict__ dsrc) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= S * C) return;
  const int64_t g = i / C, q = i % C;
  const int64_t lo = g * rps, hi = lo + rps < N ? lo + rps : N;
  float F = 0.f;
  for (int64_t t = lo / TILE; t <= (hi - 1) / TILE; ++t) F += colsrc[(t + g) * C + q];
  dsrc[i] = F;
}

// The delta cotangent of each token: qtok[n] = sum_o g[n, o] frozen[n, o] - sum_b
// rowdm[n, b] (d enters as acts = xV (m - d) and as + d x @ W^T). One wave per token,
// lanes striding o, then a fixed-order wave sum.
__global__ __launch_bounds__(256) void k_lm_delta_cot(const bf16_t* __restrict__ g, const bf16_t* __restrict__ frozen,
                                                      int64_t N, int dout, const float* __restrict__ rowdm, int nb,
                                                      float* __restrict__ qtok) {
  const int64_t n = (int64_t)blockIdx.x * 4 + wave_id();
  if (n >= N) return;
  const int lane = threadIdx.x & 63;
  float acc = 0.f;
  for (int o = lane; o < dout; o += 64)
    acc = fmaf(bf16_to_f32(g[n * dout + o]), bf16_to_f32(frozen[n * dout + o]), acc);
  acc = wave_sum(acc);
  if (lane == 0) {
    float dm = 0.f;
    for (int b = 0; b < nb; ++b) dm += rowdm[n * nb + b];
    qtok[n] = acc - dm;
  }
}

// The delta table's gradient: dsd[gi] = the sum of qtok over the tokens of source row gi.
// One block per row: each thread adds a strided share in order, then a fixed tree.
__global__ __launch_bounds__(256) void k_lm_src_delta_sum(const float* __restrict__ qtok, int64_t N, int64_t rps,
                                                          float* __restrict__ dsd) {
  __shared__ float red[256];
  const int64_t lo = (int64_t)blockIdx.x * rps, hi = lo + rps < N ? lo + rps : N;
  float acc = 0.f;
  for (int64_t n = lo + threadIdx.x; n < hi; n += 256) acc += qtok[n];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) dsd[blockIdx.x] = red[0];
}

// ---------------------------------------------------------------- attention (hd = 64)
// RoPE angle table value for position t and pair c: cos/sin of t * base^(-2c/64), computed
// in fp32 and rounded to bf16 as the reference's tables are (pd/target_ports/llama.py:100-105).
__device__ inline void rope_cs(int64_t t, int c, float log2_base, float& cs, float& sn) {
  const float inv = exp2f(-(float)(2 * c) / (float)LM_HD * log2_base);
  float sv, cv;
  sincosf((float)t * inv, &sv, &cv);
  cs = bf16_to_f32(f32_to_bf16(cv));
  sn = bf16_to_f32(f32_to_bf16(sv));
}

// Head-major copies of one (batch, head, 64-token) tile: Qh, Kh, Vh [B*H, T, 64] (q and k
// rotated; a kv head serves H/KV query heads, so its k and v are repeated).
// Grid (T/64, H, B); thread = (token tid / 4, pairs 8 (tid % 4) .. +8).
__global__ __launch_bounds__(256) void k_lm_attn_in(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                    const bf16_t* __restrict__ v, int64_t T, int H, int KV,
                                                    float log2_base, bf16_t* __restrict__ Qh, bf16_t* __restrict__ Kh,
                                                    bf16_t* __restrict__ Vh) {
  const int tid = threadIdx.x;
  const int h = blockIdx.y, g = h / (H / KV);
  const int64_t b = blockIdx.z, t0 = (int64_t)blockIdx.x * TILE;
  const int r = tid >> 2, cp = (tid & 3) * 8;
  const int64_t t = t0 + r, n = b * T + t;
  const int64_t bh = b * H + h;
  float q1[8], q2[8], k1[8], k2[8];
  load8(q + n * (int64_t)H * LM_HD + h * LM_HD + cp, q1);
  load8(q + n * (int64_t)H * LM_HD + h * LM_HD + cp + 32, q2);
  load8(k + n * (int64_t)KV * LM_HD + g * LM_HD + cp, k1);
  load8(k + n * (int64_t)KV * LM_HD + g * LM_HD + cp + 32, k2);
  const uint4 v1 = *(const uint4*)(v + n * (int64_t)KV * LM_HD + g * LM_HD + cp);
  const uint4 v2 = *(const uint4*)(v + n * (int64_t)KV * LM_HD + g * LM_HD + cp + 32);
  float qa[8], qb[8], ka[8], kb[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float cs, sn;
    rope_cs(t, cp + j, log2_base, cs, sn);
    qa[j] = q1[j] * cs - q2[j] * sn;
    qb[j] = q2[j] * cs + q1[j] * sn;
    ka[j] = k1[j] * cs - k2[j] * sn;
    kb[j] = k2[j] * cs + k1[j] * sn;
  }
  const int64_t row = (bh * T + t) * LM_HD;
  store8(Qh + row + cp, qa);
  store8(Qh + row + cp + 32, qb);
  store8(Kh + row + cp, ka);
  store8(Kh + row + cp + 32, kb);
  *(uint4*)(Vh + row + cp) = v1;
  *(uint4*)(Vh + row + cp + 32) = v2;
}

// ---------------------------------------------------------------- fused causal attention
// Nothing T x T is stored. A workgroup of 8 waves owns a span of up to 512 rows of one
// (batch, head); wave w takes the span's 32-row tiles w and nt - 1 - w (nt tiles in the
// span), so with causal masking every wave walks the same number of blocks. The other
// side's rows are staged through LDS 512 rows at a time (one stage when T <= 512) and read
// from there by every wave.
//
// MFMA operands: written mfma(X, Y) (X the first source of the 32x32x16 bf16 MFMA), lane
// l = 32 hh + r supplies row r of X and of Y over k = 8 hh .. +8 of a 16-wide slice and
// receives out[Y row r][X row 8 g + 4 hh + e] = sum_k X[.][k] Y[r][k] in accumulator
// register 4 g + e. An accumulator tile reused as an operand (P or dS) therefore carries,
// in slice kk, the positions 16 kk + 4 hh + 0..3 and 16 kk + 8 + 4 hh + 0..3; its partner
// (V^T, K^T, Q^T or dO^T: channels as rows, positions as k) is read in that order straight
// from the row-major LDS image by ds_read_b64_tr_b16. Within each 16-lane group that read
// gives output lane 4 a + b element b of the 8 bytes source lanes a, a + 4, a + 8, a + 12
// read; source lane 16 G + 4 e + a reads position row 16 kk + 8 h + 4 (G >> 1) + e (h = 0,
// 1: the two halves of the slice), channels 32 cb + 16 (G & 1) + 4 a .. + 3, so output lane
// l receives channel 32 cb + (l & 31) at the positions its own accumulator slice holds.
//
// LDS image of a row-major [rows, 64] bf16 block: 128-byte rows, the 16-byte chunk c of row
// R at physical chunk c ^ fa_swz(R). Each half wave's reads are conflict-free: 16
// consecutive rows at one chunk (row fragments: fa_swz is a permutation of 0..7 over the
// even rows and over the odd rows of any 16) and 4 consecutive rows at 4 consecutive
// chunks (transposing reads: rows 4q and 4q + 2 differ in bit 2 of fa_swz).
constexpr int FA_SPAN = 512;
constexpr int FA_THREADS = 512;
constexpr float FA_SCALE = 0.125f;                        // 1 / sqrt(64)
constexpr float FA_C2 = 0.125f * 1.4426950408889634f;     // scale * log2(e): P = 2^(s C2 - m)

typedef __attribute__((__vector_size__(4 * sizeof(unsigned)))) unsigned att_u32x4;

__device__ inline int fa_swz(int R) { return (((R >> 1) & 1) << 2) | ((R >> 2) & 3); }
__device__ inline int fa_off(int R, int c) { return R * 128 + ((c ^ fa_swz(R)) << 4); }

// Rows [0, n) of src (row stride ld elements) into the image at dst; n <= 512.
__device__ inline void fa_stage(char* dst, const bf16_t* __restrict__ src, int64_t ld, int n, int tid) {
  uint4 v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int i = tid + k * FA_THREADS;
    if (i < n * 8) v[k] = *(const uint4*)(src + (int64_t)(i >> 3) * ld + (i & 7) * 8);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int i = tid + k * FA_THREADS;
    if (i < n * 8) *(uint4*)(dst + fa_off(i >> 3, i & 7)) = v[k];
  }
}
// Row fragments (row R, the four 16-wide slices) from an image.
__device__ inline void fa_rows(const char* img, int R, int hh, bf16x8 (&f)[4]) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) f[kk] = *(const bf16x8*)(img + fa_off(R, 2 * kk + hh));
}
// The transposed partner of accumulator slice kk over image rows R0 .. R0 + 31, channels
// 32 cb + (lane & 31).
__device__ inline bf16x8 fa_tr(const char* img, int R0, int kk, int cb, int lane) {
  const int G = lane >> 4, e = (lane >> 2) & 3, a = lane & 3;
  const int c = 4 * cb + 2 * (G & 1) + (a >> 1);
  const int R = R0 + 16 * kk + 4 * (G >> 1) + e;
  const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(img + fa_off(R, c) + 8 * (a & 1)));
  const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(img + fa_off(R + 8, c) + 8 * (a & 1)));
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
// Row fragments from global memory (row-major, stride ld elements).
__device__ inline void att_rows(const bf16_t* base, int64_t ld, int row, int hh, bf16x8 (&f)[4]) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) f[kk] = *(const bf16x8*)(base + (int64_t)row * ld + 16 * kk + 8 * hh);
}
// Accumulator registers v[0..7] as a bf16 operand slice (round to nearest even).
__device__ inline bf16x8 att_pack(const float* v) {
  return (bf16x8)(att_u32x4){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                             pack_bf16x2(v[6], v[7])};
}
__device__ inline float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }
__device__ inline f32x16 att_mm(const bf16x8 (&x)[4], const bf16x8 (&y)[4]) {
  f32x16 acc = {};
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x[kk], y[kk], acc, 0, 0, 0);
  return acc;
}
// Causal test inside a diagonal block: accumulator register i of lane (hh, r) pairs row r
// of the Y side with row 8 (i >> 2) + 4 hh + (i & 3) of the X side.
__device__ inline int att_xrow(int i, int hh) { return 8 * (i >> 2) + 4 * hh + (i & 3); }
__device__ inline float att_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Scores of one 32-row block of the image against the wave's Y fragments:
// out[lane: Y row r][reg: image row R0 + 8 g + 4 hh + e].
__device__ inline f32x16 fa_scores(const char* img, int R0, int r, int hh, const bf16x8 (&yf)[4]) {
  bf16x8 xf[4];
  fa_rows(img, R0 + r, hh, xf);
  return att_mm(xf, yf);
}
// Forward pass 1 on one key block: the row's running max m (in 2^x units, taken over the
// scaled scores, whose products are canonical) and this lane's partial sum l.
template <bool DIAG>
__device__ inline void fa_rowstats(const f32x16& sc, int r, int hh, float& m, float& l) {
  float t[16], bm = -INFINITY;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    t[i] = sc[i] * FA_C2;
    if (!DIAG || att_xrow(i, hh) <= r) bm = fmaxf(bm, t[i]);
  }
  const float mn = fmaxf(m, fmaxf(bm, __shfl_xor(bm, 32, 64)));
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (!DIAG || att_xrow(i, hh) <= r) acc += att_exp2(t[i] - mn);
  l = l * att_exp2(m - mn) + acc;  // the first block: m = -inf, l = 0
  m = mn;
}
// P = 2^(s C2 - m) / l on one block (0 above the diagonal).
template <bool DIAG>
__device__ inline void fa_probs(const f32x16& sc, int r, int hh, float m, float il, float (&p)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) p[i] = (!DIAG || att_xrow(i, hh) <= r) ? att_exp2(fmaf(sc[i], FA_C2, -m)) * il : 0.f;
}
// dS = (dP - D) bf16(P) / 8 on one block of a query-major tile.
template <bool DIAG>
__device__ inline void fa_dscores(const f32x16& sc, const f32x16& dp, int r, int hh, float m, float il, float D,
                                  float (&ds)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float p = (!DIAG || att_xrow(i, hh) <= r) ? bf16r(att_exp2(fmaf(sc[i], FA_C2, -m)) * il) : 0.f;
    ds[i] = (dp[i] - D) * (p * FA_SCALE);
  }
}

// Forward: a = softmax(Q K^T / 8, causal) V written row-major into a [B*T, H*64] (bf16; P
// rounded to bf16 before the product, as a materialized P is stored). Per tile, pass 1
// forms each query row's max and sum of exp over its keys (both halves of a wave carry
// the row's running max, each its own partial sum); pass 2 forms P = 2^(s C2 - m) / l and
// accumulates P V. Each block's scores are formed one block ahead of its softmax math, and
// the diagonal block (the tile's last) runs the masked variant. With SAVE the row's m and
// 1/l (stats [2][B*H*T]) and the fp32 output (Of [B*H, T, 64]) are kept for the backward.
// Grid (query spans, B*H), the spans with the most keys first.
template <bool SAVE>
__global__ __launch_bounds__(FA_THREADS) void k_lm_flash_fwd(const bf16_t* __restrict__ Qh,
                                                             const bf16_t* __restrict__ Kh,
                                                             const bf16_t* __restrict__ Vh, int T, int H,
                                                             bf16_t* __restrict__ a, float* __restrict__ stats,
                                                             float* __restrict__ Of) {
  __shared__ __attribute__((aligned(1024))) char lds[2 * FA_SPAN * 128];
  char* Kl = lds;
  char* Vl = lds + FA_SPAN * 128;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 31, hh = lane >> 5;
  const int s = (int)gridDim.x - 1 - (int)blockIdx.x;
  const int64_t bh = blockIdx.y, BHT = (int64_t)gridDim.y * T;
  const int64_t b = bh / H, hd = bh % H;
  const int q0 = s * FA_SPAN, nt = min(FA_SPAN, T - q0) / 32;
  const bool act = w < nt / 2;
  const int tl[2] = {w, nt - 1 - w};
  const bf16_t* K = Kh + bh * T * LM_HD;
  const bf16_t* V = Vh + bh * T * LM_HD;
  const bool one = s == 0;  // a single stage of keys: K and V stay resident throughout
  if (one) {
    fa_stage(Kl, K, LM_HD, min(FA_SPAN, T), tid);
    fa_stage(Vl, V, LM_HD, min(FA_SPAN, T), tid);
    __syncthreads();
  }
#pragma unroll 1
  for (int X = 0; X < 2; ++X) {
    const int t = tl[X], qi = q0 + 32 * t + r;
    bf16x8 qf[4];
    if (act) att_rows(Qh + bh * T * LM_HD, LM_HD, qi, hh, qf);
    float m = -INFINITY, l = 0.f;
    for (int c = 0; c <= s; ++c) {
      if (!one) {
        __syncthreads();
        fa_stage(Kl, K + (int64_t)c * FA_SPAN * LM_HD, LM_HD, min(FA_SPAN, T - c * FA_SPAN), tid);
        __syncthreads();
      }
      if (!act) continue;
      const int nb = c < s ? 16 : t + 1;
      f32x16 sc = fa_scores(Kl, 0, r, hh, qf);
      for (int j = 0; j < nb; ++j) {
        const f32x16 cur = sc;
        sc = fa_scores(Kl, 32 * min(j + 1, nb - 1), r, hh, qf);
        if (c == s && j == nb - 1) fa_rowstats<true>(cur, r, hh, m, l);
        else fa_rowstats<false>(cur, r, hh, m, l);
      }
    }
    const float il = 1.f / (l + __shfl_xor(l, 32, 64));
    f32x16 o[2] = {};
    for (int c = 0; c <= s; ++c) {
      if (!one) {
        __syncthreads();
        fa_stage(Kl, K + (int64_t)c * FA_SPAN * LM_HD, LM_HD, min(FA_SPAN, T - c * FA_SPAN), tid);
        fa_stage(Vl, V + (int64_t)c * FA_SPAN * LM_HD, LM_HD, min(FA_SPAN, T - c * FA_SPAN), tid);
        __syncthreads();
      }
      if (!act) continue;
      const int nb = c < s ? 16 : t + 1;
      f32x16 sc = fa_scores(Kl, 0, r, hh, qf);
      for (int j = 0; j < nb; ++j) {
        const f32x16 cur = sc;
        sc = fa_scores(Kl, 32 * min(j + 1, nb - 1), r, hh, qf);
        float p[16];
        if (c == s && j == nb - 1) fa_probs<true>(cur, r, hh, m, il, p);
        else fa_probs<false>(cur, r, hh, m, il, p);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf16x8 pf = att_pack(p + 8 * kk);
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
            o[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa_tr(Vl, 32 * j, kk, cb, lane), pf, o[cb], 0, 0, 0);
        }
      }
    }
    if (!act) continue;
    bf16_t* arow = a + ((b * T + qi) * H + hd) * LM_HD;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int ch = cb * 32 + 8 * g + 4 * hh;
        *(uint2*)(arow + ch) =
            make_uint2(pack_bf16x2(o[cb][4 * g], o[cb][4 * g + 1]), pack_bf16x2(o[cb][4 * g + 2], o[cb][4 * g + 3]));
        if (SAVE)
          *(float4*)(Of + (bh * T + qi) * LM_HD + ch) =
              make_float4(o[cb][4 * g], o[cb][4 * g + 1], o[cb][4 * g + 2], o[cb][4 * g + 3]);
      }
    if (SAVE && hh == 0) {
      stats[bh * T + qi] = m;
      stats[BHT + bh * T + qi] = il;
    }
  }
}

// dQ = dS K per query row, dS = bf16(P (dP - D) / 8), dP = dO V^T, P = bf16(2^(s C2 - m) / l)
// from the forward's row stats, D = sum_c dO O over the forward's fp32 output (equal to
// sum_j P dP for the same P; written to Dq for the key-side kernel). dO is read from the
// cotangent da [B*T, H*64]. Spans and waves as the forward's (one tile after the other, K
// and V staged through LDS, scores and dP one block ahead). dQh [B*H, T, 64] bf16.
__global__ __launch_bounds__(FA_THREADS) void k_lm_flash_dq(const bf16_t* __restrict__ Qh,
                                                            const bf16_t* __restrict__ Kh,
                                                            const bf16_t* __restrict__ Vh,
                                                            const bf16_t* __restrict__ da,
                                                            const float* __restrict__ Of,
                                                            const float* __restrict__ stats, int T, int H,
                                                            bf16_t* __restrict__ dQh, float* __restrict__ Dq) {
  __shared__ __attribute__((aligned(1024))) char lds[2 * FA_SPAN * 128];
  char* Kl = lds;
  char* Vl = lds + FA_SPAN * 128;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 31, hh = lane >> 5;
  const int s = (int)gridDim.x - 1 - (int)blockIdx.x;
  const int64_t bh = blockIdx.y, BHT = (int64_t)gridDim.y * T;
  const int64_t b = bh / H, hd = bh % H;
  const int q0 = s * FA_SPAN, nt = min(FA_SPAN, T - q0) / 32;
  const bool act = w < nt / 2;
  const int tl[2] = {w, nt - 1 - w};
  const bf16_t* K = Kh + bh * T * LM_HD;
  const bf16_t* V = Vh + bh * T * LM_HD;
  const bf16_t* dO = da + (b * T * H + hd) * LM_HD;
  const bool one = s == 0;
  if (one) {
    fa_stage(Kl, K, LM_HD, min(FA_SPAN, T), tid);
    fa_stage(Vl, V, LM_HD, min(FA_SPAN, T), tid);
    __syncthreads();
  }
#pragma unroll 1
  for (int X = 0; X < 2; ++X) {
    const int t = tl[X], qi = q0 + 32 * t + r;
    bf16x8 qf[4], df[4];
    float m = 0.f, il = 0.f, Dv = 0.f;
    if (act) {
      att_rows(Qh + bh * T * LM_HD, LM_HD, qi, hh, qf);
      att_rows(dO, (int64_t)H * LM_HD, qi, hh, df);
      m = stats[bh * T + qi];
      il = stats[BHT + bh * T + qi];
      // D over the channels this lane's dO fragments hold: 16 kk + 8 hh + 0..7
      const float* orow = Of + (bh * T + qi) * LM_HD;
      float dot = 0.f;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const float4 o0 = *(const float4*)(orow + 16 * kk + 8 * hh);
        const float4 o1 = *(const float4*)(orow + 16 * kk + 8 * hh + 4);
        const att_u32x4 dw = (att_u32x4)df[kk];
        dot = fmaf(bf_lo(dw[0]), o0.x, dot);
        dot = fmaf(bf_hi(dw[0]), o0.y, dot);
        dot = fmaf(bf_lo(dw[1]), o0.z, dot);
        dot = fmaf(bf_hi(dw[1]), o0.w, dot);
        dot = fmaf(bf_lo(dw[2]), o1.x, dot);
        dot = fmaf(bf_hi(dw[2]), o1.y, dot);
        dot = fmaf(bf_lo(dw[3]), o1.z, dot);
        dot = fmaf(bf_hi(dw[3]), o1.w, dot);
      }
      Dv = dot + __shfl_xor(dot, 32, 64);
      if (hh == 0) Dq[bh * T + qi] = Dv;
    }
    f32x16 dq[2] = {};
    for (int c = 0; c <= s; ++c) {
      if (!one) {
        __syncthreads();
        fa_stage(Kl, K + (int64_t)c * FA_SPAN * LM_HD, LM_HD, min(FA_SPAN, T - c * FA_SPAN), tid);
        fa_stage(Vl, V + (int64_t)c * FA_SPAN * LM_HD, LM_HD, min(FA_SPAN, T - c * FA_SPAN), tid);
        __syncthreads();
      }
      if (!act) continue;
      const int nb = c < s ? 16 : t + 1;
      f32x16 sc = fa_scores(Kl, 0, r, hh, qf), dp = fa_scores(Vl, 0, r, hh, df);
      for (int j = 0; j < nb; ++j) {
        const f32x16 cs = sc, cp = dp;
        const int jn = 32 * min(j + 1, nb - 1);
        sc = fa_scores(Kl, jn, r, hh, qf);
        dp = fa_scores(Vl, jn, r, hh, df);
        float ds[16];
        if (c == s && j == nb - 1) fa_dscores<true>(cs, cp, r, hh, m, il, Dv, ds);
        else fa_dscores<false>(cs, cp, r, hh, m, il, Dv, ds);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf16x8 sf = att_pack(ds + 8 * kk);
#pragma unroll
          for (int cb = 0; cb < 2; ++cb)
            dq[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa_tr(Kl, 32 * j, kk, cb, lane), sf, dq[cb], 0, 0, 0);
        }
      }
    }
    if (!act) continue;
    bf16_t* out = dQh + (bh * T + qi) * LM_HD;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(uint2*)(out + cb * 32 + 8 * g + 4 * hh) =
            make_uint2(pack_bf16x2(dq[cb][4 * g], dq[cb][4 * g + 1]), pack_bf16x2(dq[cb][4 * g + 2], dq[cb][4 * g + 3]));
  }
}

// Half kk of one key-major block of the key-side backward: P^T and dS^T for the lane's
// key row against the 8 queries registers 8 kk .. 8 kk + 7 hold (row stats and D from
// LDS), as bf16 operand slices.
template <bool DIAG>
__device__ inline void fa_kblock(const f32x16& st, const f32x16& dpt, const float (*qs)[FA_SPAN], int i0, int kk,
                                 int r, int hh, bf16x8& pf, bf16x8& sf) {
  float p[8], ds[8];
#pragma unroll
  for (int gg = 0; gg < 2; ++gg) {
    const int g = 2 * kk + gg, qq = i0 + 8 * g + 4 * hh;
    const float4 mq = *(const float4*)&qs[0][qq];
    const float4 lq = *(const float4*)&qs[1][qq];
    const float4 dq4 = *(const float4*)&qs[2][qq];
    const float mv[4] = {mq.x, mq.y, mq.z, mq.w}, lv[4] = {lq.x, lq.y, lq.z, lq.w};
    const float dv4[4] = {dq4.x, dq4.y, dq4.z, dq4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ii = 4 * g + e;
      const float pv = (!DIAG || att_xrow(ii, hh) >= r) ? bf16r(att_exp2(fmaf(st[ii], FA_C2, -mv[e])) * lv[e]) : 0.f;
      p[4 * gg + e] = pv;
      ds[4 * gg + e] = (dpt[ii] - dv4[e]) * (pv * FA_SCALE);
    }
  }
  pf = att_pack(p);
  sf = att_pack(ds);
}

// dK = dS^T Q and dV = P^T dO per key row: the workgroup owns a span of up to 512 keys
// (waves pair key tiles as the forward pairs query tiles, one tile after the other) and
// stages the queries from the span on, 512 at a time, through LDS (Q and dO rows, each
// query's m, 1/l and D). S^T = K Q^T and dP^T = V dO^T are formed key-major (each lane one
// key row, its registers 16 queries); the diagonal block is the tile's first. dKh, dVh [B*H, T, 64] bf16. Grid (key spans, B*H), the spans with the
// most queries first.
__global__ __launch_bounds__(FA_THREADS) void k_lm_flash_dkv(const bf16_t* __restrict__ Qh,
                                                             const bf16_t* __restrict__ Kh,
                                                             const bf16_t* __restrict__ Vh,
                                                             const bf16_t* __restrict__ da,
                                                             const float* __restrict__ stats,
                                                             const float* __restrict__ Dq, int T, int H,
                                                             bf16_t* __restrict__ dKh, bf16_t* __restrict__ dVh) {
  __shared__ __attribute__((aligned(1024))) char lds[2 * FA_SPAN * 128];
  __shared__ __attribute__((aligned(16))) float qs[3][FA_SPAN];  // m, 1/l, D of the staged queries
  char* Ql = lds;
  char* Ol = lds + FA_SPAN * 128;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, r = lane & 31, hh = lane >> 5;
  const int s = blockIdx.x, ns = (T + FA_SPAN - 1) / FA_SPAN;
  const int64_t bh = blockIdx.y, BHT = (int64_t)gridDim.y * T;
  const int64_t b = bh / H, hd = bh % H;
  const int k0 = s * FA_SPAN, nt = min(FA_SPAN, T - k0) / 32;
  const bool act = w < nt / 2;
  const int tl[2] = {w, nt - 1 - w};
  const bf16_t* Q = Qh + bh * T * LM_HD;
  const bf16_t* dO = da + (b * T * H + hd) * LM_HD;
  auto stage = [&](int c) {
    const int c0 = c * FA_SPAN, n = min(FA_SPAN, T - c0);
    fa_stage(Ql, Q + (int64_t)c0 * LM_HD, LM_HD, n, tid);
    fa_stage(Ol, dO + (int64_t)c0 * H * LM_HD, (int64_t)H * LM_HD, n, tid);
    if (tid < n) {
      qs[0][tid] = stats[bh * T + c0 + tid];
      qs[1][tid] = stats[BHT + bh * T + c0 + tid];
      qs[2][tid] = Dq[bh * T + c0 + tid];
    }
  };
  const bool one = ns - s == 1;  // one stage holds every query the span's keys meet
  if (one) {
    stage(s);
    __syncthreads();
  }
#pragma unroll 1
  for (int X = 0; X < 2; ++X) {
    f32x16 dk[2] = {}, dv[2] = {};
    bf16x8 kf[4], vf[4];
    const int kj = k0 + 32 * tl[X] + r;
    if (act) {
      att_rows(Kh + bh * T * LM_HD, LM_HD, kj, hh, kf);
      att_rows(Vh + bh * T * LM_HD, LM_HD, kj, hh, vf);
    }
    for (int c = s; c < ns; ++c) {
      if (!one) {
        __syncthreads();
        stage(c);
        __syncthreads();
      }
      if (!act) continue;
      auto block = [&](int i, auto diag) {
        const f32x16 cs = fa_scores(Ql, 32 * i, r, hh, kf), cp = fa_scores(Ol, 32 * i, r, hh, vf);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          bf16x8 pf, sf;
          fa_kblock<decltype(diag)::value>(cs, cp, qs, 32 * i, kk, r, hh, pf, sf);
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) {
            dv[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa_tr(Ol, 32 * i, kk, cb, lane), pf, dv[cb], 0, 0, 0);
            dk[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa_tr(Ql, 32 * i, kk, cb, lane), sf, dk[cb], 0, 0, 0);
          }
        }
      };
      int i = 0;
      if (c == s) block(i = tl[X], std::true_type{});
      const int nb = min(FA_SPAN, T - c * FA_SPAN) / 32;
      for (i = c == s ? tl[X] + 1 : 0; i < nb; ++i) block(i, std::false_type{});
    }
    if (!act) continue;
    const int64_t row = (bh * T + kj) * LM_HD;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int ch = cb * 32 + 8 * g + 4 * hh;
        *(uint2*)(dKh + row + ch) =
            make_uint2(pack_bf16x2(dk[cb][4 * g], dk[cb][4 * g + 1]), pack_bf16x2(dk[cb][4 * g + 2], dk[cb][4 * g + 3]));
        *(uint2*)(dVh + row + ch) =
            make_uint2(pack_bf16x2(dv[cb][4 * g], dv[cb][4 * g + 1]), pack_bf16x2(dv[cb][4 * g + 2], dv[cb][4 * g + 3]));
      }
  }
}

// Cotangents of q, k, v from the head-major dQh, dKh, dVh [B*H, T, 64]: the inverse RoPE
// rotation on dq and dk (rope is orthogonal per pair: dx = dy cos - rot(dy) sin, the
// transpose of the forward rotation) and, for k and v, the sum over the H/KV query heads
// sharing a kv head. Grid (T/64, KV, B); thread = (token tid / 4, pairs 8 (tid % 4) .. +8).
__global__ __launch_bounds__(256) void k_lm_attn_out_grads(const bf16_t* __restrict__ dQh,
                                                           const bf16_t* __restrict__ dKh,
                                                           const bf16_t* __restrict__ dVh, int64_t T, int H, int KV,
                                                           float log2_base, bf16_t* __restrict__ dq,
                                                           bf16_t* __restrict__ dk, bf16_t* __restrict__ dv) {
  const int tid = threadIdx.x;
  const int g = blockIdx.y, rep = H / KV;
  const int64_t b = blockIdx.z, t0 = (int64_t)blockIdx.x * TILE;
  const int r = tid >> 2, cp = (tid & 3) * 8;
  const int64_t t = t0 + r, n = b * T + t;
  float cs[8], sn[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) rope_cs(t, cp + j, log2_base, cs[j], sn[j]);
  float ka[8] = {0, 0, 0, 0, 0, 0, 0, 0}, kb[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float va[8] = {0, 0, 0, 0, 0, 0, 0, 0}, vb[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int i = 0; i < rep; ++i) {
    const int h = g * rep + i;
    const int64_t row = ((b * H + h) * T + t) * LM_HD;
    float y1[8], y2[8], o1[8], o2[8];
    load8(dQh + row + cp, y1);
    load8(dQh + row + cp + 32, y2);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o1[j] = y1[j] * cs[j] + y2[j] * sn[j];
      o2[j] = y2[j] * cs[j] - y1[j] * sn[j];
    }
    store8(dq + n * (int64_t)H * LM_HD + h * LM_HD + cp, o1);
    store8(dq + n * (int64_t)H * LM_HD + h * LM_HD + cp + 32, o2);
    load8(dKh + row + cp, y1);
    load8(dKh + row + cp + 32, y2);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ka[j] += y1[j] * cs[j] + y2[j] * sn[j];
      kb[j] += y2[j] * cs[j] - y1[j] * sn[j];
    }
    load8(dVh + row + cp, y1);
    load8(dVh + row + cp + 32, y2);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      va[j] += y1[j];
      vb[j] += y2[j];
    }
  }
  store8(dk + n * (int64_t)KV * LM_HD + g * LM_HD + cp, ka);
  store8(dk + n * (int64_t)KV * LM_HD + g * LM_HD + cp + 32, kb);
  store8(dv + n * (int64_t)KV * LM_HD + g * LM_HD + cp, va);
  store8(dv + n * (int64_t)KV * LM_HD + g * LM_HD + cp + 32, vb);
}

// ---------------------------------------------------------------- GELU (tanh form)
__device__ inline void gelu_tanh_fg(float x, float& f, float& g) {
  const float k0 = 0.7978845608028654f, k1 = 0.044715f;
  const float u = k0 * (x + k1 * x * x * x);
  const float th = tanhf(u);
  f = 0.5f * x * (1.f + th);
  g = 0.5f * (1.f + th) + 0.5f * x * (1.f - th * th) * k0 * (1.f + 3.f * k1 * x * x);
}

// y = bf16(gelu_tanh(x)), 8 elements per thread.
__global__ __launch_bounds__(256) void k_lm_gelu_fwd(const bf16_t* __restrict__ x, int64_t n, bf16_t* __restrict__ y) {
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += (int64_t)gridDim.x * 256 * 8) {
    float v[8];
    load8(x + i, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float f, g;
      gelu_tanh_fg(v[j], f, g);
      v[j] = f;
    }
    store8(y + i, v);
  }
}

// dx = bf16(dy * gelu_tanh'(x)).
__global__ __launch_bounds__(256) void k_lm_gelu_bwd(const bf16_t* __restrict__ x, const bf16_t* __restrict__ dy,
                                                     int64_t n, bf16_t* __restrict__ dx) {
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += (int64_t)gridDim.x * 256 * 8) {
    float v[8], d[8];
    load8(x + i, v);
    load8(dy + i, d);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float f, g;
      gelu_tanh_fg(v[j], f, g);
      v[j] = d[j] * g;
    }
    store8(dx + i, v);
  }
}

// losses[0..3] = (recon_coeff kl + imp_coeff act + freq_coeff freq, kl, act, freq) with
// kl = mean of the position KLs, act = imp_scale * sum of the imp partials, freq = sum
// of the frequency partials (none when n_freq = 0); with fb_part (the EMA estimator's
// batch penalty) losses[4] = sum(fb_part) over n_freq; each added in a fixed order in
// double.
__global__ void k_lm_losses(const float* __restrict__ pos_kl, int64_t N, const float* __restrict__ imp_part,
                            int64_t n_imp, const float* __restrict__ freq_part, int64_t n_freq,
                            const float* __restrict__ fb_part, double imp_scale, float recon_coeff, float imp_coeff,
                            float freq_coeff, float* __restrict__ losses) {
  __shared__ double sr[16], si[16], sq[16], sb[16];
  double r = 0.0, m = 0.0, fq = 0.0, fb = 0.0;
  for (int64_t i = threadIdx.x; i < N; i += blockDim.x) r += pos_kl[i];
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
    double a = 0, c = 0, q = 0, qb = 0;
    for (int i = 0; i < (int)(blockDim.x / 64); ++i) {
      a += sr[i];
      c += si[i];
      q += sq[i];
      qb += sb[i];
    }
    if (fb_part) losses[4] = (float)qb;
    a /= (double)N;
    c *= imp_scale;
    losses[0] = (float)(recon_coeff * a + imp_coeff * c + freq_coeff * q);
    losses[1] = (float)a;
    losses[2] = (float)c;
    losses[3] = (float)q;
  }
}

// g[n] = v (the per-position cotangent of the mean KL).
__global__ __launch_bounds__(256) void k_lm_fill(float* __restrict__ g, int64_t n, float v) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) g[i] = v;
}

// ---------------------------------------------------------------- workspace plan
struct LMDims {
  int64_t B, T, N, V;
  int d, H, KV, f, L, n_chunks;
  int C[LM_NK], din[LM_NK], dout[LM_NK];
  bool use_delta;
  bool routed = false;  // per-token routes: the target segment is needed without a delta too
  int64_t S = 0, rps = 0;  // persistent source tables: S rows of rps tokens (rps = 0: none)
  bool srcs() const { return rps > 0; }
  int64_t BH() const { return B * H; }
  // the site products add a target segment, s (.) (x @ W^T) (s = d on routed rows, 1 on the
  // rest), and its cotangent s (.) (g @ W) to the d_input
  bool cat() const { return use_delta || routed; }
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

struct LMSiteSave {
  bf16_t *xV, *acts;
  uint8_t* ub;
  bf16_t* frozen;  // source tables with the delta channel: the site's x @ W^T [N, d_out]
  // smooth-L0: tile column sums of psi, per-component slopes, loss partials (act, freq,
  // the EMA estimator's batch penalty), and the site's offset in the EMA estimate
  float *sl0_col, *sl0_slope, *sl0_act, *sl0_freq, *sl0_fb;
  size_t ema_off;
};

struct LMLayerSave {
  bf16_t *r, *h, *r1, *h2, *a, *fc, *g;
  float *rinv1, *rinv2;
  bf16_t *Qh, *Kh, *Vh;   // the attention's head-major operands [B*H, T, 64]
  float *att_stats, *Of;  // row max and 1/sum [2][B*H*T]; fp32 output [B*H, T, 64]
  LMSiteSave site[LM_NK];
};

struct LMPlan {
  std::vector<LMLayerSave> layers;
  bf16_t *VT[LM_NK], *UT[LM_NK], *WT[LM_NK];  // per-step transposed weights, [L, ...] per kind
  bf16_t *rc_a, *rc_b, *rL, *act_m, *act_c, *hc, *qc, *kc, *vc, *ac, *Oh, *fcc, *gc;
  bf16_t *cQh, *cKh, *cVh;  // the clean pass's own attention operands
  bf16_t *q, *k, *v;
  float *rinvF, *att_D, *delta, *imp_part, *pos_kl, *stats, *gpos, *d_act, *dhf;
  bf16_t *dr_a, *dr_b, *drT[2], *dacts, *dxV[2], *dqkv[3], *da, *dQh, *dKh, *dVh, *dg, *dfc;
  char *kl_ws, *sk_ws;
  size_t kl_ws_bytes, sk_ws_bytes, imp_per_site[LM_NK], imp_total, total;
  float *sl0_act, *sl0_freq, *sl0_fb;  // every site's smooth-L0 loss partials, contiguous
  size_t sl0_blocks_total;
  float *colsrc, *rowdm, *qtok;  // source tables: tile column sums, token row sums, delta cotangents
};

static size_t site_imp_blocks(const LMDims& D, int k) { return (size_t)cdiv(D.C[k], TILE) * cdiv(D.N, TILE); }

static LMPlan lm_plan(const LMDims& D, char* base, bool dry) {
  Arena A{base, 0, dry};
  LMPlan P;
  const int64_t N = D.N, d = D.d, f = D.f, BH = D.BH(), T = D.T;
  const int64_t qd = (int64_t)D.H * LM_HD;
  P.layers.resize(D.L);
  for (int l = 0; l < D.L; ++l) {
    LMLayerSave& S = P.layers[l];
    S.r = A.take<bf16_t>(N * d);
    S.h = A.take<bf16_t>(N * d);
    S.r1 = A.take<bf16_t>(N * d);
    S.h2 = A.take<bf16_t>(N * d);
    S.a = A.take<bf16_t>(N * qd);
    S.fc = A.take<bf16_t>(N * f);
    S.g = A.take<bf16_t>(N * f);
    S.rinv1 = A.take<float>(N);
    S.rinv2 = A.take<float>(N);
    S.Qh = A.take<bf16_t>(BH * T * LM_HD);
    S.Kh = A.take<bf16_t>(BH * T * LM_HD);
    S.Vh = A.take<bf16_t>(BH * T * LM_HD);
    S.att_stats = A.take<float>(2 * BH * T);
    S.Of = A.take<float>(BH * T * LM_HD);
    for (int k = 0; k < LM_NK; ++k) {
      S.site[k].xV = A.take<bf16_t>(N * D.C[k]);
      S.site[k].acts = A.take<bf16_t>(N * D.C[k]);
      S.site[k].ub = A.take<uint8_t>(N * D.C[k]);
      S.site[k].frozen = D.srcs() && D.use_delta ? A.take<bf16_t>(N * D.dout[k]) : nullptr;
    }
  }
  for (int k = 0; k < LM_NK; ++k) {
    P.VT[k] = A.take<bf16_t>((size_t)D.L * D.C[k] * D.din[k]);
    P.UT[k] = A.take<bf16_t>((size_t)D.L * D.dout[k] * D.C[k]);
    P.WT[k] = D.cat() ? A.take<bf16_t>((size_t)D.L * D.din[k] * D.dout[k]) : nullptr;
  }
  int64_t maxw = std::max<int64_t>(d, f), maxC = 0;
  for (int k = 0; k < LM_NK; ++k) maxC = std::max<int64_t>(maxC, D.C[k]);
  P.rc_a = A.take<bf16_t>(N * d);
  P.rc_b = A.take<bf16_t>(N * d);
  P.rL = A.take<bf16_t>(N * d);
  P.act_m = A.take<bf16_t>(N * d);
  P.act_c = A.take<bf16_t>(N * d);
  P.hc = A.take<bf16_t>(N * d);
  P.qc = A.take<bf16_t>(N * qd);
  P.kc = A.take<bf16_t>(N * qd);
  P.vc = A.take<bf16_t>(N * qd);
  P.ac = A.take<bf16_t>(N * qd);
  P.fcc = A.take<bf16_t>(N * f);
  P.gc = A.take<bf16_t>(N * f);
  P.q = A.take<bf16_t>(N * qd);
  P.k = A.take<bf16_t>(N * qd);
  P.v = A.take<bf16_t>(N * qd);
  P.rinvF = A.take<float>(N);
  P.att_D = A.take<float>(BH * T);
  P.cQh = A.take<bf16_t>(BH * T * LM_HD);
  P.cKh = A.take<bf16_t>(BH * T * LM_HD);
  P.cVh = A.take<bf16_t>(BH * T * LM_HD);
  P.delta = A.take<float>((size_t)D.L * LM_NK * N);
  P.imp_total = 0;
  for (int k = 0; k < LM_NK; ++k) {
    P.imp_per_site[k] = site_imp_blocks(D, k);
    P.imp_total += P.imp_per_site[k] * D.L;
  }
  P.imp_part = A.take<float>(P.imp_total);
  size_t nblk = 0;
  for (int l = 0; l < D.L; ++l)
    for (int k = 0; k < LM_NK; ++k) nblk += sl0_blocks(1, D.C[k]);
  P.sl0_blocks_total = nblk;
  P.sl0_act = A.take<float>(nblk);
  P.sl0_freq = A.take<float>(nblk);
  P.sl0_fb = A.take<float>(nblk);
  nblk = 0;
  size_t ema_off = 0;  // the EMA estimate is [L][kind][C_kind], layer-major
  for (int l = 0; l < D.L; ++l)
    for (int k = 0; k < LM_NK; ++k) {
      LMSiteSave& S = P.layers[l].site[k];
      S.sl0_col = A.take<float>((size_t)(cdiv(N, TILE) + 1) * D.C[k]);
      S.sl0_slope = A.take<float>(D.C[k]);
      S.sl0_act = P.sl0_act ? P.sl0_act + nblk : nullptr;
      S.sl0_freq = P.sl0_freq ? P.sl0_freq + nblk : nullptr;
      S.sl0_fb = P.sl0_fb ? P.sl0_fb + nblk : nullptr;
      S.ema_off = ema_off;
      nblk += sl0_blocks(1, D.C[k]);
      ema_off += (size_t)D.C[k];
    }
  P.pos_kl = A.take<float>(N);
  P.stats = A.take<float>(N * 5);
  P.gpos = A.take<float>(N);
  P.d_act = A.take<float>(N * d);
  P.dhf = A.take<float>(N * maxw);
  P.dr_a = A.take<bf16_t>(N * d);
  P.dr_b = A.take<bf16_t>(N * d);
  for (int b = 0; b < 2; ++b) P.drT[b] = A.take<bf16_t>(N * maxw);
  P.dacts = A.take<bf16_t>(N * maxC);
  for (int b = 0; b < 2; ++b) P.dxV[b] = A.take<bf16_t>(N * maxC);
  for (int i = 0; i < 3; ++i) P.dqkv[i] = A.take<bf16_t>(N * qd);
  P.da = A.take<bf16_t>(N * qd);
  P.dQh = A.take<bf16_t>(BH * T * LM_HD);
  P.dKh = A.take<bf16_t>(BH * T * LM_HD);
  P.dVh = A.take<bf16_t>(BH * T * LM_HD);
  P.dg = A.take<bf16_t>(N * f);
  P.dfc = A.take<bf16_t>(N * f);
  P.kl_ws_bytes = pd_streamed_kl_workspace_size(PD_DTYPE_BF16, N, d, D.V, D.n_chunks);
  P.kl_ws = A.take<char>(P.kl_ws_bytes);
  P.sk_ws_bytes = 0;  // split-contraction partials of the weight-gradient products
  for (int k = 0; k < LM_NK; ++k)
    P.sk_ws_bytes = std::max({P.sk_ws_bytes, gemm_splitk_ws_bytes(D.C[k], D.dout[k], N),
                              gemm_splitk_ws_bytes(D.din[k], D.C[k], N)});
  P.sk_ws = A.take<char>(P.sk_ws_bytes);
  P.colsrc = D.srcs() && D.rps > 1 ? A.take<float>((size_t)(cdiv(N, TILE) + D.S) * maxC) : nullptr;
  P.rowdm = D.srcs() && D.use_delta ? A.take<float>((size_t)N * cdiv(maxC, TILE)) : nullptr;
  P.qtok = D.srcs() && D.use_delta ? A.take<float>(N) : nullptr;
  P.total = A.off;
  return P;
}

// Persistent source tables of a pd_lm_stack_step_sources call.
struct LMSources {
  const void* const* src;  // [6] kinds: [L, S, C_k]
  int src_dtype;
  const void* delta;       // [L, 6, S] or NULL (no delta channel)
  int delta_dtype;
  int64_t rps;
  float* const* d_src;     // [6] kinds: [L, S, C_k] fp32
  float* d_src_delta;      // [L, 6, S] fp32
  bool want_wgrads, reuse_clean;
};

struct LMRecorder {
  void** ev;
  int32_t* cat;
  int cap, n;
  hipStream_t s;
  void mark(int category) {
    if (!ev || n >= cap) return;
    (void)hipEventRecord((hipEvent_t)ev[n], s);
    if (cat) cat[n] = category;
    ++n;
  }
};

static unsigned ew_blocks(int64_t n8) { return (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(n8, 256), 8192)); }

static void transpose(const bf16_t* src, int64_t R, int64_t Cc, bf16_t* dst, int64_t ld, hipStream_t s) {
  hipLaunchKernelGGL(k_lm_transpose, dim3((unsigned)cdiv(Cc, TILE), (unsigned)cdiv(R, TILE)), dim3(256), 0, s, src,
                     R, Cc, dst, ld);
}

// A site's output s (.) (x @ W^T) + acts @ U (s: d on routed rows, 0 without a delta,
// 1 on unrouted rows), every operand K-contiguous: x [N, d_in], W [d_out, d_in] as
// stored, acts [N, C], UT = U^T [d_out, C]. Without the target segment, acts @ U alone.
static int site_out(int64_t N, int64_t dout, int64_t di, int64_t C, const bf16_t* x, const bf16_t* W,
                    const bf16_t* acts, const bf16_t* UT, const float* delta, const uint8_t* route, bool cat,
                    bf16_t* out, hipStream_t s) {
  if (!cat) return pd_gemm(PD_DTYPE_BF16, N, dout, C, acts, C, 0, UT, C, 1, out, dout, PD_DTYPE_BF16, 1.f, 0.f, s);
  GemmArgs g{N, dout, C, acts, C, UT, C, out, dout, 1.f, 0.f, nullptr, 0, 0, 0};
  KcatArgs q{x, di, W, di, di, nullptr, route};
  q.delta_f = delta;
  return launch_kcat_epi<EpiStore, bf16_t, false, false>(g, q, EpiStore::Args{}, s, "pd_lm_stack_step site out");
}

// A site's input cotangent s (.) (g @ W) + dxV @ V^T, every operand K-contiguous: g [N,
// d_out], WT = W^T [d_in, d_out], dxV [N, C], V [d_in, C] as stored; fp32 (beta
// accumulates into out) or bf16 out.
static int site_din(int64_t N, int64_t dout, int64_t di, int64_t C, const bf16_t* g, const bf16_t* WT,
                    const bf16_t* dxV, const bf16_t* V, const float* delta, const uint8_t* route, bool cat, void* out,
                    bool f32, float beta, hipStream_t s) {
  if (!cat)
    return pd_gemm(PD_DTYPE_BF16, N, di, C, dxV, C, 0, V, C, 1, out, di, f32 ? PD_DTYPE_F32 : PD_DTYPE_BF16, 1.f,
                   beta, s);
  GemmArgs a{N, di, C, dxV, C, V, C, out, di, 1.f, beta, nullptr, 0, 0, 0};
  KcatArgs q{g, dout, WT, dout, dout, nullptr, route};
  q.delta_f = delta;
  if (f32) return launch_kcat_epi<EpiStore, float, false, false>(a, q, EpiStore::Args{}, s, "pd_lm_stack_step site din");
  return launch_kcat_epi<EpiStore, bf16_t, false, false>(a, q, EpiStore::Args{}, s, "pd_lm_stack_step site din");
}

// dst[b] = src[b]^T for B matrices [R, Cc] (R, Cc multiples of 8): every layer's copy of
// one weight in one launch.
static void transpose_layers(const void* src, int64_t B, int64_t R, int64_t Cc, bf16_t* dst, hipStream_t s) {
  hipLaunchKernelGGL(k_lm_transpose_b, dim3((unsigned)cdiv(Cc, TILE), (unsigned)cdiv(R, TILE), (unsigned)B), dim3(256),
                     0, s, (const bf16_t*)src, R, Cc, dst);
}

// C = A @ B^T with both operands K-contiguous (the buffer-fed kernel).
static int gemm_nt(int64_t M, int64_t Nn, int64_t K, const bf16_t* A, int64_t lda, const bf16_t* Bt, int64_t ldb,
                   void* C, int64_t ldc, int c_dtype, float beta, hipStream_t s) {
  return pd_gemm(PD_DTYPE_BF16, M, Nn, K, A, lda, 0, Bt, ldb, 1, C, ldc, c_dtype, 1.f, beta, s);
}

}  // namespace pd

using namespace pd;

extern "C" {

size_t pd_lm_stack_workspace_size(int64_t B, int64_t T, int d, int n_head, int n_kv_head, int d_mlp, int64_t vocab,
                                  int L, const int32_t* C, int use_delta, int n_kl_chunks) {
  if (B <= 0 || T <= 0 || d <= 0 || n_head <= 0 || n_kv_head <= 0 || d_mlp <= 0 || vocab <= 0 || L <= 0 || !C ||
      n_kl_chunks <= 0)
    return 0;
  LMDims D{B, T, B * T, vocab, d, n_head, n_kv_head, d_mlp, L, n_kl_chunks, {}, {}, {}, use_delta != 0};
  const int qd = n_head * LM_HD, kvd = n_kv_head * LM_HD;
  const int din[LM_NK] = {d, d, d, qd, d, d_mlp}, dout[LM_NK] = {qd, kvd, kvd, d, d_mlp, d};
  for (int k = 0; k < LM_NK; ++k) {
    D.C[k] = C[k];
    D.din[k] = din[k];
    D.dout[k] = dout[k];
  }
  return lm_plan(D, nullptr, true).total;
}

enum {
  LM_CAT_PREP = 0,     // delta draws
  LM_CAT_CLEAN = 1,    // frozen forward
  LM_CAT_GEMM_FWD = 2, // masked-forward site products
  LM_CAT_MASK_FWD = 3, // mask passes (forward)
  LM_CAT_ATTN = 4,     // attention forward and backward
  LM_CAT_ELEM = 5,     // norms, residual adds, GELU, the cotangent copies g^T
  LM_CAT_KL = 6,       // streamed KL forward and backward
  LM_CAT_GEMM_DX = 7,  // d_acts and d_input products
  LM_CAT_GEMM_DW = 8,  // dU and dV products
  LM_CAT_MASK_BWD = 9, // mask passes (backward)
  LM_CAT_WAIT = 10,    // waiting for the helper stream (the clean pass)
  LM_CAT_END = 11
};

static int lm_step_impl(int64_t B, int64_t T, int d, int H, int KV, int f, int64_t V, int L, const int32_t* Cs,
                        const int32_t* tokens, const void* wte, const float* ln1, const float* ln2, const float* norm,
                        float eps, float rope_base, const void* const* W, const void* const* Vf, const void* const* Uf,
                        const void* const* ci_pre, uint32_t draw_k0, uint32_t draw_k1, int use_delta,
                        const uint8_t* routes, int layout, const ImpSpec& imp, float recon_coeff, int n_chunks,
                        float* losses, float* const* dV,
                        float* const* dU, void* const* d_ci_pre, void* workspace, size_t workspace_bytes, void* stream,
                        LMRecorder& rec, const LMSources* srcs = nullptr) {
  const char* what = srcs ? "pd_lm_stack_step_sources" : "pd_lm_stack_step";
  const bool want_wgrads = !srcs || srcs->want_wgrads;
  if (int e = check_imp_spec(imp, what)) return e;
  if (B <= 0 || T <= 0 || d <= 0 || H <= 0 || KV <= 0 || f <= 0 || V <= 0 || L <= 0 || n_chunks <= 0 || !Cs)
    return fail(PD_EINVAL, std::string(what) + ": bad dims");
  if (H % KV) return fail(PD_EINVAL, std::string(what) + ": n_head must be a multiple of n_kv_head");
  if (d != H * LM_HD) return fail(PD_EUNSUPPORTED, std::string(what) + ": head_dim must be 64 (d = 64 * n_head)");
  if (T % TILE || d % 64 || f % 64 || V % n_chunks || T > 8192 || d > 4096 || f > 65536)
    return fail(PD_EUNSUPPORTED, std::string(what) + ": need T % 64 == 0 (T <= 8192), d and d_mlp multiples of 64, "
                                                     "vocab % n_chunks == 0");
  for (int k = 0; k < LM_NK; ++k)
    if (Cs[k] <= 0 || Cs[k] % 8) return fail(PD_EUNSUPPORTED, std::string(what) + ": every C must be a positive multiple of 8");
  if (!tokens || !wte || !ln1 || !ln2 || !norm || !W || !Vf || !Uf || !ci_pre || !losses || !d_ci_pre ||
      (want_wgrads && (!dV || !dU)))
    return fail(PD_EINVAL, std::string(what) + ": null pointer");
  for (int k = 0; k < LM_NK; ++k)
    if (!W[k] || !Vf[k] || !Uf[k] || !ci_pre[k] || !d_ci_pre[k] || (want_wgrads && (!dV[k] || !dU[k])))
      return fail(PD_EINVAL, std::string(what) + ": null per-kind pointer");
  if (srcs) {
    if (routes) return fail(PD_EINVAL, std::string(what) + ": no per-token routes with source tables");
    if (!srcs->src || !srcs->d_src || srcs->rps <= 0 || (B * T) % srcs->rps || (srcs->delta && !srcs->d_src_delta))
      return fail(PD_EINVAL, std::string(what) + ": source tables, rows_per_source | B*T and outputs required");
    for (int k = 0; k < LM_NK; ++k)
      if (!srcs->src[k] || !srcs->d_src[k]) return fail(PD_EINVAL, std::string(what) + ": null source table");
    for (int dt : {srcs->src_dtype, srcs->delta ? srcs->delta_dtype : PD_DTYPE_F32})
      if (dt != PD_DTYPE_F32 && dt != PD_DTYPE_BF16 && dt != PD_DTYPE_U16)
        return fail(PD_EINVAL, std::string(what) + ": source dtype");
    use_delta = srcs->delta ? 1 : 0;
  }
  if (layout != PD_LAYOUT_PARTITIONABLE && layout != PD_LAYOUT_ORIGINAL)
    return fail(PD_EINVAL, std::string(what) + ": unknown counter layout");
  LMDims D{B, T, B * T, V, d, H, KV, f, L, n_chunks, {}, {}, {}, use_delta != 0};
  D.routed = routes != nullptr;
  if (srcs) {
    D.rps = srcs->rps;
    D.S = D.N / srcs->rps;
  }
  const int qd = H * LM_HD, kvd = KV * LM_HD;
  {
    const int din[LM_NK] = {d, d, d, qd, d, f}, dout[LM_NK] = {qd, kvd, kvd, d, f, d};
    for (int k = 0; k < LM_NK; ++k) {
      D.C[k] = Cs[k];
      D.din[k] = din[k];
      D.dout[k] = dout[k];
    }
  }
  if (!workspace || workspace_bytes < lm_plan(D, nullptr, true).total)
    return fail(PD_EWORKSPACE, std::string(what) + ": workspace too small (size routed calls with use_delta = 1)");
  if (D.N * (int64_t)std::max<int64_t>(f, 4096) > ((int64_t)1 << 31) / 2 || D.BH() * T * T > ((int64_t)1 << 31))
    return fail(PD_EUNSUPPORTED, std::string(what) + ": activations of 2 GiB or more");
  LMPlan P = lm_plan(D, (char*)workspace, false);
  hipStream_t s = (hipStream_t)stream;
  rec.s = s;
  const int64_t N = D.N, BH = D.BH();
  const float log2b = log2f(rope_base);
  const int pm = imp_mode(imp);
  const bool sl0 = pm == PM_SL0;
  int rc;
  auto bfp = [](const void* base, size_t off) { return (const bf16_t*)base + off; };
  auto rows4 = [](int64_t n) { return dim3((unsigned)cdiv(n, 4)); };
  auto tgrid = [](int64_t rows, int64_t cols) { return dim3((unsigned)cdiv(cols, TILE), (unsigned)cdiv(rows, TILE)); };

  // ---- keys: src_base, delta_base = split(draw_key); key(kind, layer) = fold_in(fold_in(base, kind), layer)
  uint32_t halves[4];
  split2(draw_k0, draw_k1, layout, halves);
  auto site_key = [&](int kind, int layer, uint32_t& o0, uint32_t& o1) {
    uint32_t x0 = 0, x1 = (uint32_t)kind;
    threefry2x32(halves[0], halves[1], x0, x1);
    uint32_t y0 = 0, y1 = (uint32_t)layer;
    threefry2x32(x0, x1, y0, y1);
    o0 = y0;
    o1 = y1;
  };

  // the clean pass's helper stream starts once the inputs are ready
  AuxStream ax;
  if ((rc = aux_stream(0, 5, ax))) return rc;  // inputs ready, act_c ready, dW fork, dW done [2]
  const hipStream_t sc = ax.st;
  hipEventRecord(ax.ev[0], s);
  hipStreamWaitEvent(sc, ax.ev[0], 0);

  // ================= per-step transposed weights (one launch per kind and matrix) and the
  // per-token deltas
  rec.mark(LM_CAT_PREP);
  for (int k = 0; k < LM_NK; ++k) {
    transpose_layers(Vf[k], L, D.din[k], D.C[k], P.VT[k], s);    // V^T [C, d_in]
    transpose_layers(Uf[k], L, D.C[k], D.dout[k], P.UT[k], s);   // U^T [d_out, C]
    if (D.cat()) transpose_layers(W[k], L, D.dout[k], D.din[k], P.WT[k], s);  // W^T [d_in, d_out]
  }
  if (srcs && D.use_delta)  // each token's delta is its source row's
    hipLaunchKernelGGL(k_src_delta_fill, dim3((unsigned)std::min<int64_t>(cdiv((int64_t)LM_NK * L * N, 256), 4096)),
                       dim3(256), 0, s, srcs->delta, srcs->delta_dtype, D.S, D.rps, N, LM_NK * L, P.delta);
  else if (D.use_delta)
    hipLaunchKernelGGL(k_lm_deltas, dim3((unsigned)cdiv(N, 256), (unsigned)(LM_NK * L)), dim3(256), 0, s, halves[2],
                       halves[3], N, layout, P.delta);
  if ((rc = check_launch("pd_lm_stack_step prep"))) return rc;

  // ================= fused causal attention on head-major copies, output a row-major;
  // Ls (a layer's saves) also receives the row stats and fp32 output the backward reads
  const dim3 fa_grid((unsigned)cdiv(T, FA_SPAN), (unsigned)BH);
  auto attn_fwd = [&](const bf16_t* q, const bf16_t* k, const bf16_t* v, bf16_t* Qh, bf16_t* Kh, bf16_t* Vh,
                      LMLayerSave* Ls, bf16_t* a, hipStream_t st) -> int {
    hipLaunchKernelGGL(k_lm_attn_in, dim3((unsigned)(T / TILE), (unsigned)H, (unsigned)B), dim3(256), 0, st, q, k, v,
                       T, H, KV, log2b, Qh, Kh, Vh);
    if (Ls)
      hipLaunchKernelGGL(k_lm_flash_fwd<true>, fa_grid, dim3(FA_THREADS), 0, st, Qh, Kh, Vh, (int)T, H, a,
                         Ls->att_stats, Ls->Of);
    else
      hipLaunchKernelGGL(k_lm_flash_fwd<false>, fa_grid, dim3(FA_THREADS), 0, st, Qh, Kh, Vh, (int)T, H, a,
                         (float*)nullptr, (float*)nullptr);
    return check_launch("pd_lm_stack_step attention");
  };

  // ================= clean forward (frozen target): act_c. It is independent of the masked
  // forward until the KL reads act_c, so it runs on a helper stream beside the per-step
  // weight copies and the masked forward, with attention buffers of its own.
  // With reuse_clean (source tables) act_c is the one the previous call left in the workspace.
  rec.mark(LM_CAT_CLEAN);
  const bool clean = !(srcs && srcs->reuse_clean);
  if (clean) hipLaunchKernelGGL(k_lm_embed, rows4(N), dim3(256), 0, sc, tokens, (const bf16_t*)wte, N, d, V, P.rc_a);
  if (clean) {
    bf16_t* rcur = P.rc_a;
    bf16_t* rnext = P.rc_b;
    for (int l = 0; l < L; ++l) {
      auto Wk = [&](int k) { return bfp(W[k], (size_t)l * D.dout[k] * D.din[k]); };
      hipLaunchKernelGGL(k_lm_rms_fwd, rows4(N), dim3(256), 0, sc, rcur, N, d, ln1 + (size_t)l * d, eps, P.hc,
                         (float*)nullptr);
      if ((rc = gemm_nt(N, qd, d, P.hc, d, Wk(LK_Q), d, P.qc, qd, PD_DTYPE_BF16, 0.f, sc))) return rc;
      if ((rc = gemm_nt(N, kvd, d, P.hc, d, Wk(LK_K), d, P.kc, kvd, PD_DTYPE_BF16, 0.f, sc))) return rc;
      if ((rc = gemm_nt(N, kvd, d, P.hc, d, Wk(LK_V), d, P.vc, kvd, PD_DTYPE_BF16, 0.f, sc))) return rc;
      if ((rc = attn_fwd(P.qc, P.kc, P.vc, P.cQh, P.cKh, P.cVh, nullptr, P.ac, sc)))
        return rc;
      if ((rc = gemm_nt(N, d, qd, P.ac, qd, Wk(LK_O), qd, P.hc, d, PD_DTYPE_BF16, 0.f, sc))) return rc;
      hipLaunchKernelGGL(k_lm_add, dim3(ew_blocks(N * d / 8)), dim3(256), 0, sc, rcur, P.hc, N * d, rnext);
      std::swap(rcur, rnext);
      hipLaunchKernelGGL(k_lm_rms_fwd, rows4(N), dim3(256), 0, sc, rcur, N, d, ln2 + (size_t)l * d, eps, P.hc,
                         (float*)nullptr);
      if ((rc = gemm_nt(N, f, d, P.hc, d, Wk(LK_FC), d, P.fcc, f, PD_DTYPE_BF16, 0.f, sc))) return rc;
      hipLaunchKernelGGL(k_lm_gelu_fwd, dim3(ew_blocks(N * f / 8)), dim3(256), 0, sc, P.fcc, N * f, P.gc);
      if ((rc = gemm_nt(N, d, f, P.gc, f, Wk(LK_DOWN), f, P.hc, d, PD_DTYPE_BF16, 0.f, sc))) return rc;
      hipLaunchKernelGGL(k_lm_add, dim3(ew_blocks(N * d / 8)), dim3(256), 0, sc, rcur, P.hc, N * d, rnext);
      std::swap(rcur, rnext);
    }
    hipLaunchKernelGGL(k_lm_rms_fwd, rows4(N), dim3(256), 0, sc, rcur, N, d, norm, eps, P.act_c, (float*)nullptr);
  }
  if (clean) hipEventRecord(ax.ev[1], sc);  // act_c is ready
  if ((rc = check_launch("pd_lm_stack_step clean"))) return rc;

  // ================= masked forward
  auto mask_args = [&](int k, int l) {
    LMMaskArgs ma;
    ma.ci_pre = bfp(ci_pre[k], (size_t)l * N * D.C[k]);
    ma.N = N;
    ma.C = D.C[k];
    site_key(k, l, ma.k0, ma.k1);
    ma.p = imp.p;
    ma.delta = D.use_delta ? P.delta + ((size_t)l * LM_NK + k) * N : nullptr;
    ma.route = routes ? routes + ((size_t)l * LM_NK + k) * N : nullptr;
    ma.ld = D.C[k];
    ma.g2 = imp.g2();
    ma.psis = imp.psi_scale();
    ma.colpart = P.layers[l].site[k].sl0_col;
    ma.slope = P.layers[l].site[k].sl0_slope;
    if (srcs) {
      const size_t es = srcs->src_dtype == PD_DTYPE_F32 ? 4 : 2;
      ma.src = (const char*)srcs->src[k] + (size_t)l * D.S * D.C[k] * es;
      ma.src_dtype = srcs->src_dtype;
      ma.rps = D.rps;
      ma.colsrc = P.colsrc;
      ma.dsrc = srcs->d_src[k] + (size_t)l * D.S * D.C[k];
      ma.rowdm = P.rowdm;
    }
    return ma;
  };
  // site forward: x [N, d_in] (and the site's saves) -> out [N, d_out]
  auto site_fwd = [&](int k, int l, const bf16_t* x, bf16_t* out) -> int {
    LMSiteSave& S = P.layers[l].site[k];
    const int64_t C = D.C[k], di = D.din[k], dout = D.dout[k];
    rec.mark(LM_CAT_GEMM_FWD);
    int r = gemm_nt(N, C, di, x, di, P.VT[k] + (size_t)l * C * di, di, S.xV, C, PD_DTYPE_BF16, 0.f, s);
    if (r) return r;
    rec.mark(LM_CAT_MASK_FWD);
    const LMMaskArgs ma = mask_args(k, l);
    float* part = P.imp_part + [&] {
      size_t o = 0;
      for (int ll = 0; ll < l; ++ll)
        for (int kk = 0; kk < LM_NK; ++kk) o += P.imp_per_site[kk];
      for (int kk = 0; kk < k; ++kk) o += P.imp_per_site[kk];
      return o;
    }();
#define PD_LMF(LY, PMV) \
  hipLaunchKernelGGL((k_lm_mask_fwd<LY, PMV>), tgrid(N, C), dim3(256), 0, s, ma, S.xV, S.acts, S.ub, part)
    if (srcs) {
      if (pm == PM_SL0) PD_LMF(MASK_SRC, PM_SL0);
      else if (pm == 2) PD_LMF(MASK_SRC, 2);
      else if (pm == 1) PD_LMF(MASK_SRC, 1);
      else PD_LMF(MASK_SRC, 0);
    } else if (layout == PD_LAYOUT_PARTITIONABLE) {
      if (pm == PM_SL0) PD_LMF(PD_LAYOUT_PARTITIONABLE, PM_SL0);
      else if (pm == 2) PD_LMF(PD_LAYOUT_PARTITIONABLE, 2);
      else if (pm == 1) PD_LMF(PD_LAYOUT_PARTITIONABLE, 1);
      else PD_LMF(PD_LAYOUT_PARTITIONABLE, 0);
    } else {
      if (pm == PM_SL0) PD_LMF(PD_LAYOUT_ORIGINAL, PM_SL0);
      else if (pm == 2) PD_LMF(PD_LAYOUT_ORIGINAL, 2);
      else if (pm == 1) PD_LMF(PD_LAYOUT_ORIGINAL, 1);
      else PD_LMF(PD_LAYOUT_ORIGINAL, 0);
    }
#undef PD_LMF
    if (sl0)  // the site's frequencies, loss partials and backward slopes
      hipLaunchKernelGGL(k_sl0_finalize, dim3(sl0_blocks(1, (int)C)), dim3(256), 0, s, S.sl0_col,
                         (const int32_t*)nullptr, 1, N, (int)C, 1.f / (float)N, imp.coeff, imp.freq_coeff,
                         imp.ref_count, imp.ema.at((int64_t)S.ema_off), S.sl0_slope, S.sl0_act, S.sl0_freq,
                         imp.ema.on() ? S.sl0_fb : nullptr);
    rec.mark(LM_CAT_GEMM_FWD);
    const bf16_t* Wl = bfp(W[k], (size_t)l * dout * di);
    if (S.frozen &&  // the target output the delta table's gradient reads
        (r = gemm_nt(N, dout, di, x, di, Wl, di, S.frozen, dout, PD_DTYPE_BF16, 0.f, s)))
      return r;
    return site_out(N, dout, di, C, x, Wl, S.acts, P.UT[k] + (size_t)l * dout * C, ma.delta, ma.route, D.cat(), out,
                    s);
  };

  hipLaunchKernelGGL(k_lm_embed, rows4(N), dim3(256), 0, s, tokens, (const bf16_t*)wte, N, d, V, P.layers[0].r);
  for (int l = 0; l < L; ++l) {
    LMLayerSave& S = P.layers[l];
    rec.mark(LM_CAT_ELEM);
    hipLaunchKernelGGL(k_lm_rms_fwd, rows4(N), dim3(256), 0, s, S.r, N, d, ln1 + (size_t)l * d, eps, S.h, S.rinv1);
    if ((rc = site_fwd(LK_Q, l, S.h, P.q))) return rc;
    if ((rc = site_fwd(LK_K, l, S.h, P.k))) return rc;
    if ((rc = site_fwd(LK_V, l, S.h, P.v))) return rc;
    rec.mark(LM_CAT_ATTN);
    if ((rc = attn_fwd(P.q, P.k, P.v, S.Qh, S.Kh, S.Vh, &S, S.a, s))) return rc;
    rec.mark(LM_CAT_ELEM);
    if ((rc = site_fwd(LK_O, l, S.a, P.q))) return rc;  // o output into the q scratch
    rec.mark(LM_CAT_ELEM);
    hipLaunchKernelGGL(k_lm_add, dim3(ew_blocks(N * d / 8)), dim3(256), 0, s, S.r, P.q, N * d, S.r1);
    hipLaunchKernelGGL(k_lm_rms_fwd, rows4(N), dim3(256), 0, s, S.r1, N, d, ln2 + (size_t)l * d, eps, S.h2, S.rinv2);
    if ((rc = site_fwd(LK_FC, l, S.h2, S.fc))) return rc;
    rec.mark(LM_CAT_ELEM);
    hipLaunchKernelGGL(k_lm_gelu_fwd, dim3(ew_blocks(N * f / 8)), dim3(256), 0, s, S.fc, N * f, S.g);
    if ((rc = site_fwd(LK_DOWN, l, S.g, P.q))) return rc;
    rec.mark(LM_CAT_ELEM);
    bf16_t* rnext = l + 1 < L ? P.layers[l + 1].r : P.rL;
    hipLaunchKernelGGL(k_lm_add, dim3(ew_blocks(N * d / 8)), dim3(256), 0, s, S.r1, P.q, N * d, rnext);
  }
  hipLaunchKernelGGL(k_lm_rms_fwd, rows4(N), dim3(256), 0, s, P.rL, N, d, norm, eps, P.act_m, P.rinvF);
  if ((rc = check_launch("pd_lm_stack_step masked forward"))) return rc;

  // ================= streamed KL (clean || masked) over the tied head, and its cotangent
  rec.mark(LM_CAT_WAIT);
  if (clean) hipStreamWaitEvent(s, ax.ev[1], 0);  // the clean pass's act_c
  rec.mark(LM_CAT_KL);
  if ((rc = pd_streamed_kl_fwd(PD_DTYPE_BF16, N, d, V, n_chunks, P.act_m, wte, P.act_c, wte, P.pos_kl, P.stats,
                               P.kl_ws, P.kl_ws_bytes, s)))
    return rc;
  if (sl0)
    hipLaunchKernelGGL(k_lm_losses, dim3(1), dim3(1024), 0, s, P.pos_kl, N, P.sl0_act, (int64_t)P.sl0_blocks_total,
                       P.sl0_freq, imp.ref_count > 0.f ? (int64_t)P.sl0_blocks_total : (int64_t)0,
                       imp.ema.on() ? (const float*)P.sl0_fb : nullptr, 1.0, recon_coeff, imp.coeff, imp.freq_coeff,
                       losses);
  else
    hipLaunchKernelGGL(k_lm_losses, dim3(1), dim3(1024), 0, s, P.pos_kl, N, P.imp_part, (int64_t)P.imp_total,
                       (const float*)nullptr, (int64_t)0, (const float*)nullptr, 1.0 / (double)N, recon_coeff,
                       imp.coeff, 0.f, losses);
  hipLaunchKernelGGL(k_lm_fill, dim3(ew_blocks(N)), dim3(256), 0, s, P.gpos, N, recon_coeff / (float)N);
  if ((rc = pd_streamed_kl_bwd(PD_DTYPE_BF16, N, d, V, n_chunks, P.act_m, wte, P.act_c, wte, P.stats, P.gpos,
                               P.d_act, P.kl_ws, P.kl_ws_bytes, s)))
    return rc;
  rec.mark(LM_CAT_ELEM);
  hipLaunchKernelGGL(k_lm_rms_bwd, rows4(N), dim3(256), 0, s, P.d_act, P.rL, P.rinvF, norm, N, d,
                     (const bf16_t*)nullptr, P.dr_a);
  if ((rc = check_launch("pd_lm_stack_step loss"))) return rc;

  // ================= backward
  const float imp_scale = imp.coeff / (float)N;
  // site backward: g [N, d_out] (the output cotangent), the site input x [N, d_in] -> dU,
  // dV, d_ci_pre, and d_input (+)= into din_out (fp32 accumulate when din_f32, else bf16
  // written).
  // The weight gradients (split-contraction products) run on the helper stream: site call
  // n writes g^T and d(xV) into buffer set n % 2, forks the helper stream once both are
  // written, and call n + 2 waits for that call's products before it rewrites the set.
  // Nothing on this stream reads a weight gradient; the step joins them all at its end.
  int wg_call = 0;
  bool wg_pend[2] = {false, false};
  auto wg_join = [&](int b) {
    if (wg_pend[b]) hipStreamWaitEvent(s, ax.ev[3 + b], 0);
    wg_pend[b] = false;
  };
  auto site_bwd = [&](int k, int l, const bf16_t* g, const bf16_t* x, void* din_out, bool din_f32,
                      float din_beta) -> int {
    // din_out NULL: the site's input carries no gradient (layer 0's q/k/v read the
    // embedding), so its d_input product is not formed (nor counted by the reference's
    // FLOP rule, pd/core/flops/target.py:53-93)
    LMSiteSave& S = P.layers[l].site[k];
    const int64_t C = D.C[k], di = D.din[k], dout = D.dout[k];
    const LMMaskArgs ma = mask_args(k, l);
    const int wb = wg_call++ & 1;
    bf16_t* const drT = P.drT[wb];
    bf16_t* const dxV = P.dxV[wb];
    rec.mark(LM_CAT_WAIT);
    wg_join(wb);
    rec.mark(LM_CAT_ELEM);
    if (want_wgrads) transpose(g, N, dout, drT, N, s);  // g^T [d_out, N]
    rec.mark(LM_CAT_GEMM_DX);
    int r = gemm_nt(N, C, dout, g, dout, bfp(Uf[k], (size_t)l * C * dout), dout, P.dacts, C, PD_DTYPE_BF16, 0.f, s);
    if (r) return r;
    rec.mark(LM_CAT_MASK_BWD);
    bf16_t* dpre = (bf16_t*)d_ci_pre[k] + (size_t)l * N * C;
#define PD_LMB(PMV, SRC)                                                                                          \
  hipLaunchKernelGGL((k_lm_mask_bwd<PMV, SRC>), tgrid(N, C), dim3(256), 0, s, ma, S.xV, S.ub, imp_scale, P.dacts, \
                     dxV, dpre)
    if (srcs) {
      if (pm == PM_SL0) PD_LMB(PM_SL0, true);
      else if (pm == 2) PD_LMB(2, true);
      else if (pm == 1) PD_LMB(1, true);
      else PD_LMB(0, true);
      // the table's gradient (rows of several tokens: from the tiles' column sums), and the
      // delta table's from each token's delta cotangent
      if (D.rps > 1)
        hipLaunchKernelGGL(k_lm_src_finalize, dim3((unsigned)cdiv(D.S * C, 256)), dim3(256), 0, s, P.colsrc, N, D.rps,
                           D.S, (int)C, ma.dsrc);
      if (D.use_delta) {
        hipLaunchKernelGGL(k_lm_delta_cot, rows4(N), dim3(256), 0, s, g, S.frozen, N, (int)dout, P.rowdm,
                           (int)cdiv(C, TILE), P.qtok);
        hipLaunchKernelGGL(k_lm_src_delta_sum, dim3((unsigned)D.S), dim3(256), 0, s, P.qtok, N, D.rps,
                           srcs->d_src_delta + ((size_t)l * LM_NK + k) * D.S);
      }
    } else {
      if (pm == PM_SL0) PD_LMB(PM_SL0, false);
      else if (pm == 2) PD_LMB(2, false);
      else if (pm == 1) PD_LMB(1, false);
      else PD_LMB(0, false);
    }
#undef PD_LMB
    if (want_wgrads) {
      rec.mark(LM_CAT_GEMM_DW);
      hipEventRecord(ax.ev[2], s);  // g^T and d(xV) of this call are written
      hipStreamWaitEvent(ax.st, ax.ev[2], 0);
      // dU = acts^T @ g (acts MN-major, g^T K-contiguous), dV = x^T @ d(xV) (both MN-major)
      if ((r = gemm_splitk(C, dout, N, S.acts, C, 1, drT, N, 1, dU[k] + (size_t)l * C * dout, dout, PD_DTYPE_F32, 0.f,
                           P.sk_ws, P.sk_ws_bytes, ax.st)))
        return r;
      if ((r = gemm_splitk(di, C, N, x, di, 1, dxV, C, 0, dV[k] + (size_t)l * di * C, C, PD_DTYPE_F32, 0.f, P.sk_ws,
                           P.sk_ws_bytes, ax.st)))
        return r;
      hipEventRecord(ax.ev[3 + wb], ax.st);
      wg_pend[wb] = true;
    }
    if (!din_out) return PD_OK;
    rec.mark(LM_CAT_GEMM_DX);
    return site_din(N, dout, di, C, g, D.cat() ? P.WT[k] + (size_t)l * di * dout : nullptr, dxV,
                    bfp(Vf[k], (size_t)l * di * C), ma.delta, ma.route, D.cat(), din_out, din_f32, din_beta, s);
  };

  bf16_t* dr = P.dr_a;     // cotangent of the residual leaving layer l
  bf16_t* dr_o = P.dr_b;
  for (int l = L - 1; l >= 0; --l) {
    LMLayerSave& S = P.layers[l];
    // down site: input g, output cotangent dr
    if ((rc = site_bwd(LK_DOWN, l, dr, S.g, P.dg, false, 0.f))) return rc;
    rec.mark(LM_CAT_ELEM);
    hipLaunchKernelGGL(k_lm_gelu_bwd, dim3(ew_blocks(N * f / 8)), dim3(256), 0, s, S.fc, P.dg, N * f, P.dfc);
    // fc site: input h2 -> d_h2 (fp32) -> norm pullback added to dr
    if ((rc = site_bwd(LK_FC, l, P.dfc, S.h2, P.dhf, true, 0.f))) return rc;
    rec.mark(LM_CAT_ELEM);
    hipLaunchKernelGGL(k_lm_rms_bwd, rows4(N), dim3(256), 0, s, P.dhf, S.r1, S.rinv2, ln2 + (size_t)l * d, N, d, dr,
                       dr_o);
    std::swap(dr, dr_o);  // dr: cotangent of r1
    // o site: input a, output cotangent dr -> d_a
    if ((rc = site_bwd(LK_O, l, dr, S.a, P.da, false, 0.f))) return rc;
    // attention backward
    rec.mark(LM_CAT_ATTN);
    // dQ (query spans; also the softmax row sums D), then dK, dV (key spans)
    hipLaunchKernelGGL(k_lm_flash_dq, fa_grid, dim3(FA_THREADS), 0, s, S.Qh, S.Kh, S.Vh, P.da, S.Of, S.att_stats,
                       (int)T, H, P.dQh, P.att_D);
    hipLaunchKernelGGL(k_lm_flash_dkv, fa_grid, dim3(FA_THREADS), 0, s, S.Qh, S.Kh, S.Vh, P.da, S.att_stats, P.att_D,
                       (int)T, H, P.dKh, P.dVh);
    hipLaunchKernelGGL(k_lm_attn_out_grads, dim3((unsigned)(T / TILE), (unsigned)KV, (unsigned)B), dim3(256), 0, s,
                       P.dQh, P.dKh, P.dVh, T, H, KV, log2b, P.dqkv[0], P.dqkv[1], P.dqkv[2]);
    if ((rc = check_launch("pd_lm_stack_step attention backward"))) return rc;
    // q, k, v sites: input h, d_h accumulated in fp32 (none for layer 0: the embedding)
    float* dh = l > 0 ? P.dhf : nullptr;
    if ((rc = site_bwd(LK_Q, l, P.dqkv[0], S.h, dh, true, 0.f))) return rc;
    if ((rc = site_bwd(LK_K, l, P.dqkv[1], S.h, dh, true, 1.f))) return rc;
    if ((rc = site_bwd(LK_V, l, P.dqkv[2], S.h, dh, true, 1.f))) return rc;
    if (l > 0) {
      rec.mark(LM_CAT_ELEM);
      hipLaunchKernelGGL(k_lm_rms_bwd, rows4(N), dim3(256), 0, s, P.dhf, S.r, S.rinv1, ln1 + (size_t)l * d, N, d, dr,
                         dr_o);
      std::swap(dr, dr_o);  // dr: cotangent of layer l's input
    }
  }
  rec.mark(LM_CAT_WAIT);
  wg_join(0);
  wg_join(1);
  rec.mark(LM_CAT_END);
  return check_launch("pd_lm_stack_step backward");
}

int pd_lm_stack_step(int64_t B, int64_t T, int d, int n_head, int n_kv_head, int d_mlp, int64_t vocab, int L,
                     const int32_t* C, const int32_t* tokens, const void* wte, const float* ln1, const float* ln2,
                     const float* norm, float eps, float rope_base, const void* const* W, const void* const* V,
                     const void* const* U, const void* const* ci_pre, uint32_t draw_k0, uint32_t draw_k1,
                     int use_delta, const uint8_t* routes, int layout, int imp_kind, float p, float gamma,
                     int normalize_at_one, float imp_coeff, float freq_coeff, float ref_count,
                     const float* freq_ema_in, float* freq_ema_out, float ema_count, float ema_halflife,
                     float recon_coeff, int n_kl_chunks, float* losses, float* const* dV, float* const* dU,
                     void* const* d_ci_pre, void* workspace, size_t workspace_bytes, void* stream) {
  LMRecorder rec{nullptr, nullptr, 0, 0, nullptr};
  ImpSpec imp;
  if (int e = make_imp_spec("pd_lm_stack_step", imp_kind, p, gamma, normalize_at_one, imp_coeff, freq_coeff,
                            ref_count, freq_ema_in, freq_ema_out, ema_count, ema_halflife, imp))
    return e;
  return lm_step_impl(B, T, d, n_head, n_kv_head, d_mlp, vocab, L, C, tokens, wte, ln1, ln2, norm, eps, rope_base, W,
                      V, U, ci_pre, draw_k0, draw_k1, use_delta, routes, layout, imp, recon_coeff, n_kl_chunks, losses,
                      dV, dU, d_ci_pre, workspace, workspace_bytes, stream, rec);
}

int pd_lm_stack_step_timed(int64_t B, int64_t T, int d, int n_head, int n_kv_head, int d_mlp, int64_t vocab, int L,
                           const int32_t* C, const int32_t* tokens, const void* wte, const float* ln1,
                           const float* ln2, const float* norm, float eps, float rope_base, const void* const* W,
                           const void* const* V, const void* const* U, const void* const* ci_pre, uint32_t draw_k0,
                           uint32_t draw_k1, int use_delta, const uint8_t* routes, int layout, int imp_kind, float p,
                           float gamma, int normalize_at_one, float imp_coeff, float freq_coeff, float ref_count,
                           const float* freq_ema_in, float* freq_ema_out, float ema_count, float ema_halflife,
                           float recon_coeff, int n_kl_chunks, float* losses, float* const* dV, float* const* dU,
                           void* const* d_ci_pre, void* workspace, size_t workspace_bytes, void* stream,
                           void** events, int32_t* categories, int capacity, int* n_recorded) {
  LMRecorder rec{events, categories, capacity, 0, nullptr};
  ImpSpec imp;
  if (int e = make_imp_spec("pd_lm_stack_step_timed", imp_kind, p, gamma, normalize_at_one, imp_coeff, freq_coeff,
                            ref_count, freq_ema_in, freq_ema_out, ema_count, ema_halflife, imp))
    return e;
  int rc = lm_step_impl(B, T, d, n_head, n_kv_head, d_mlp, vocab, L, C, tokens, wte, ln1, ln2, norm, eps, rope_base,
                        W, V, U, ci_pre, draw_k0, draw_k1, use_delta, routes, layout, imp, recon_coeff, n_kl_chunks,
                        losses, dV, dU, d_ci_pre, workspace, workspace_bytes, stream, rec);
  if (n_recorded) *n_recorded = rec.n;
  return rc;
}

size_t pd_lm_stack_sources_workspace_size(int64_t B, int64_t T, int d, int n_head, int n_kv_head, int d_mlp,
                                          int64_t vocab, int L, const int32_t* C, int use_delta, int n_kl_chunks,
                                          int64_t rows_per_source) {
  if (B <= 0 || T <= 0 || d <= 0 || n_head <= 0 || n_kv_head <= 0 || d_mlp <= 0 || vocab <= 0 || L <= 0 || !C ||
      n_kl_chunks <= 0 || rows_per_source <= 0 || (B * T) % rows_per_source)
    return 0;
  LMDims D{B, T, B * T, vocab, d, n_head, n_kv_head, d_mlp, L, n_kl_chunks, {}, {}, {}, use_delta != 0};
  D.rps = rows_per_source;
  D.S = B * T / rows_per_source;
  const int qd = n_head * LM_HD, kvd = n_kv_head * LM_HD;
  const int din[LM_NK] = {d, d, d, qd, d, d_mlp}, dout[LM_NK] = {qd, kvd, kvd, d, d_mlp, d};
  for (int k = 0; k < LM_NK; ++k) {
    D.C[k] = C[k];
    D.din[k] = din[k];
    D.dout[k] = dout[k];
  }
  return lm_plan(D, nullptr, true).total;
}

int pd_lm_stack_step_sources(int64_t B, int64_t T, int d, int n_head, int n_kv_head, int d_mlp, int64_t vocab, int L,
                             const int32_t* C, const int32_t* tokens, const void* wte, const float* ln1,
                             const float* ln2, const float* norm, float eps, float rope_base, const void* const* W,
                             const void* const* V, const void* const* U, const void* const* ci_pre,
                             const void* const* src, int src_dtype, const void* src_delta, int delta_dtype,
                             int64_t rows_per_source, int imp_kind, float p, float gamma, int normalize_at_one,
                             float imp_coeff, float freq_coeff, float ref_count, const float* freq_ema_in,
                             float* freq_ema_out, float ema_count, float ema_halflife, float recon_coeff,
                             int n_kl_chunks, int want_weight_grads, int reuse_clean, float* losses, float* const* dV,
                             float* const* dU, void* const* d_ci_pre, float* const* d_src, float* d_src_delta,
                             void* workspace, size_t workspace_bytes, void* stream) {
  LMRecorder rec{nullptr, nullptr, 0, 0, nullptr};
  ImpSpec imp;
  if (int e = make_imp_spec("pd_lm_stack_step_sources", imp_kind, p, gamma, normalize_at_one, imp_coeff, freq_coeff,
                            ref_count, freq_ema_in, freq_ema_out, ema_count, ema_halflife, imp))
    return e;
  const LMSources srcs{src, src_dtype, src_delta, delta_dtype, rows_per_source, d_src, d_src_delta,
                       want_weight_grads != 0, reuse_clean != 0};
  return lm_step_impl(B, T, d, n_head, n_kv_head, d_mlp, vocab, L, C, tokens, wte, ln1, ln2, norm, eps, rope_base, W,
                      V, U, ci_pre, 0u, 0u, src_delta ? 1 : 0, nullptr, PD_LAYOUT_PARTITIONABLE, imp, recon_coeff,
                      n_kl_chunks, losses, dV, dU, d_ci_pre, workspace, workspace_bytes, stream, rec, &srcs);
}

}  // extern "C"
