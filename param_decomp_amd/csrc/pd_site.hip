// The masked decomposed linear (gfx950):
//
//   pd_masked_linear_fwd/bwd   pd/core/decomposed_linear.py:142-175 (site_forward),
//                              :65-85 (component_coefficients, blend_target_output)
//   pd_blocked_site_fwd/bwd    :209-271 (blocked_site_forward, dense over every block)
#include <initializer_list>
#include <mutex>
#include <string>

#include "pd_gemm_dtl.hpp"

namespace pd {

static int ew_grid(int64_t n) {
  int64_t b = cdiv(n, 1024);
  return (int)(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

// acts[t,c] = routed(t) ? xV*(m - d_t) : 0
template <typename T>
__global__ void k_ml_acts(const T* __restrict__ xV, const T* __restrict__ mask, const T* __restrict__ delta,
                          const uint8_t* __restrict__ route, int64_t Tn, int64_t C, T* __restrict__ acts) {
  int64_t n = Tn * C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t t = i / C;
    float coef = load_f<T>(mask, i) - (delta ? load_f<T>(delta, t) : 0.f);
    bool r = route ? route[t] != 0 : true;
    store_f<T>(acts, i, r ? load_f<T>(xV, i) * coef : 0.f);
  }
}

// out[t,:] *= routed(t) ? d_t : 1   (turns the target rows into d*target / target)
template <typename T>
__global__ void k_ml_scale_target(T* __restrict__ out, const T* __restrict__ delta, const uint8_t* __restrict__ route,
                                  int64_t Tn, int64_t D) {
  int64_t n = Tn * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t t = i / D;
    bool r = route ? route[t] != 0 : true;
    float s = r ? (delta ? load_f<T>(delta, t) : 0.f) : 1.f;
    store_f<T>(out, i, load_f<T>(out, i) * s);
  }
}

// dacts (in place over da) -> dmask = da*xV, dxV = da*(m-d); unrouted rows get zeros.
template <typename T>
__global__ void k_ml_bwd_elem(T* __restrict__ da, const T* __restrict__ xV, const T* __restrict__ mask,
                              const T* __restrict__ delta, const uint8_t* __restrict__ route, int64_t Tn, int64_t C,
                              T* __restrict__ dmask) {
  int64_t n = Tn * C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t t = i / C;
    bool r = route ? route[t] != 0 : true;
    float g = r ? load_f<T>(da, i) : 0.f;
    if (dmask) store_f<T>(dmask, i, g * load_f<T>(xV, i));
    float coef = load_f<T>(mask, i) - (delta ? load_f<T>(delta, t) : 0.f);
    store_f<T>(da, i, g * coef);
  }
}

// d_delta[t] = routed ? sum_o g[t,o] * yt[t,o] - sum_c da[t,c] * xV[t,c] : 0, the
// derivative of (xV*(m - d))@U + d*yt with respect to d_t (da = g @ U^T before the
// mask scaling). fp32 sums; one wave per row.
template <typename T>
__global__ __launch_bounds__(256) void k_ml_delta_grad(const T* __restrict__ g, const T* __restrict__ yt,
                                                       const T* __restrict__ da, const T* __restrict__ xV,
                                                       const uint8_t* __restrict__ route, int64_t Tn, int64_t D,
                                                       int64_t C, T* __restrict__ d_delta) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= Tn) return;
  const int lane = threadIdx.x & 63;
  float part = 0.f;
  for (int64_t o = lane; o < D; o += 64) part = fmaf(load_f<T>(g, t * D + o), load_f<T>(yt, t * D + o), part);
  for (int64_t c = lane; c < C; c += 64) part = fmaf(-load_f<T>(da, t * C + c), load_f<T>(xV, t * C + c), part);
  part = wave_sum(part);
  if (lane == 0) store_f<T>(d_delta, t, (route ? route[t] != 0 : true) ? part : 0.f);
}

// g_target[t,:] = g[t,:] * (routed ? d_t : 1)
template <typename T>
__global__ void k_ml_target_grad(const T* __restrict__ g, const T* __restrict__ delta,
                                 const uint8_t* __restrict__ route, int64_t Tn, int64_t D, T* __restrict__ gt) {
  int64_t n = Tn * D;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t t = i / D;
    bool r = route ? route[t] != 0 : true;
    float s = r ? (delta ? load_f<T>(delta, t) : 0.f) : 1.f;
    store_f<T>(gt, i, load_f<T>(g, i) * s);
  }
}


__global__ void k_f32_to_bf16(const float* __restrict__ src, int64_t n, bf16_t* __restrict__ dst) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = f32_to_bf16(src[i]);
}

// ---------------------------------------------------------------- fused bf16 seam
// Every bf16 call whose widths are multiples of 8 (16-byte aligned operands) runs in
// GEMM launches with the elementwise work in their prologue/epilogue:
//   forward   xV = x @ V, epilogue acts = routed ? xV * (m - d) : 0          (1 launch)
//             out = rs (.) (x @ W^T) + acts @ U, one k loop over [W^T ; U]    (1 launch)
//   backward  dU = acts^T @ g                                                  (1 launch)
//             da = g @ U^T, epilogue dmask = da * xV, dxV = da * (m - d)       (1 launch)
//             dV = x^T @ dxV                                                   (1 launch)
//             dx = rs (.) (g @ W) + dxV @ V^T, one k loop                      (1 launch)
// rs = routed ? d : 1 blends the target output (and its cotangent). Each epilogue rounds
// the accumulator to bf16 before the elementwise step, as the unfused passes do when
// they read the stored bf16 product back, so both paths agree bit for bit there.

// Row facts of the masked linear: d_t (0 without a delta) and routed(t).
__device__ inline void ml_row(const bf16_t* delta, const uint8_t* route, int64_t row, float& d, bool& r) {
  d = delta ? bf16_to_f32(delta[row]) : 0.f;
  r = route ? route[row] != 0 : true;
}

__device__ inline void unpack4(uint2 u, float (&f)[4]) {
  f[0] = bf16_to_f32((bf16_t)(u.x & 0xFFFF));
  f[1] = bf16_to_f32((bf16_t)(u.x >> 16));
  f[2] = bf16_to_f32((bf16_t)(u.y & 0xFFFF));
  f[3] = bf16_to_f32((bf16_t)(u.y >> 16));
}

__device__ inline uint2 pack4(const float (&f)[4]) { return uint2{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3])}; }

// Visits the lane's output groups of 4 consecutive columns (row, col, the 4 fp32
// accumulators rounded to bf16) of a k_gemm_dtl tile; N % 4 == 0 is required.
template <class CFG, class F>
__device__ inline void epi_groups(const GemmArgs& p, const TileJob& t, int wm, int wn, int lane,
                                  f32x16 (&acc)[CFG::TM][CFG::TN], F&& f) {
#pragma unroll
  for (int i = 0; i < CFG::TM; ++i) {
    const int64_t row = t.m0 + wm * CFG::WTM + i * 32 + (lane & 31);
    if (row >= t.M) continue;
#pragma unroll
    for (int j = 0; j < CFG::TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t col = t.n0 + wn * CFG::WTN + j * 32 + 8 * g + 4 * (lane >> 5);
        if (col >= p.N) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = bf16_to_f32(f32_to_bf16(acc[i][j][4 * g + e]));
        f(row, col, v);
      }
  }
}

// C = xV (bf16); acts = routed ? xV * (m - d) : 0
struct EpiActs {
  static constexpr int LDS_BYTES = 0;
  struct Args {
    const bf16_t* mask;
    const bf16_t* delta;
    const uint8_t* route;
    bf16_t* acts;
  };
  template <class CFG, typename TC>
  __device__ static void run(const GemmArgs& p, const Args& a, const TileJob& t, int wm, int wn, int tid,
                             f32x16 (&acc)[CFG::TM][CFG::TN], char*) {
    bf16_t* xV = (bf16_t*)t.C;
    epi_groups<CFG>(p, t, wm, wn, tid & 63, acc, [&](int64_t row, int64_t col, const float (&v)[4]) {
      float d;
      bool r;
      ml_row(a.delta, a.route, row, d, r);
      const int64_t idx = row * p.ldc + col;
      *(uint2*)(xV + idx) = pack4(v);
      float m[4], o[4];
      unpack4(*(const uint2*)(a.mask + idx), m);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = r ? v[e] * (m[e] - d) : 0.f;
      *(uint2*)(a.acts + idx) = pack4(o);
    });
  }
};

// da = g @ U^T rounded; dmask = routed ? da * xV : 0 (if wanted); C = dxV = routed ? da * (m - d) : 0
struct EpiMaskedBwd {
  static constexpr int LDS_BYTES = 0;
  struct Args {
    const bf16_t* xV;
    const bf16_t* mask;
    const bf16_t* delta;
    const uint8_t* route;
    bf16_t* dmask;
  };
  template <class CFG, typename TC>
  __device__ static void run(const GemmArgs& p, const Args& a, const TileJob& t, int wm, int wn, int tid,
                             f32x16 (&acc)[CFG::TM][CFG::TN], char*) {
    bf16_t* dxV = (bf16_t*)t.C;
    epi_groups<CFG>(p, t, wm, wn, tid & 63, acc, [&](int64_t row, int64_t col, const float (&v)[4]) {
      float d;
      bool r;
      ml_row(a.delta, a.route, row, d, r);
      const int64_t idx = row * p.ldc + col;
      float m[4], o[4];
      if (a.dmask) {
        float xv[4];
        unpack4(*(const uint2*)(a.xV + idx), xv);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = r ? v[e] * xv[e] : 0.f;
        *(uint2*)(a.dmask + idx) = pack4(o);
      }
      unpack4(*(const uint2*)(a.mask + idx), m);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = r ? v[e] * (m[e] - d) : 0.f;
      *(uint2*)(dxV + idx) = pack4(o);
    });
  }
};

// d_delta[t] = routed ? sum_o g[t,o] * yt[t,o] - sum_c dmask[t,c] : 0 (dmask = da * xV is
// the per-component term of the delta derivative); fp32 sums, one wave per row.
__global__ __launch_bounds__(256) void k_ml_delta_grad_dm(const bf16_t* __restrict__ g, const bf16_t* __restrict__ yt,
                                                          const bf16_t* __restrict__ dmask,
                                                          const uint8_t* __restrict__ route, int64_t Tn, int64_t D,
                                                          int64_t C, bf16_t* __restrict__ d_delta) {
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= Tn) return;
  const int lane = threadIdx.x & 63;
  float part = 0.f;
  for (int64_t o = lane; o < D; o += 64) part = fmaf(bf16_to_f32(g[t * D + o]), bf16_to_f32(yt[t * D + o]), part);
  for (int64_t c = lane; c < C; c += 64) part -= bf16_to_f32(dmask[t * C + c]);
  part = wave_sum(part);
  if (lane == 0) d_delta[t] = f32_to_bf16((route ? route[t] != 0 : true) ? part : 0.f);
}

static bool a16(const void* p) { return !p || ((uintptr_t)p & 15) == 0; }

// The fused seam applies: bf16, widths multiples of 8, 16-byte aligned operands.
static bool fused_seam(int dtype, int64_t d_in, int64_t d_out, int64_t C, std::initializer_list<const void*> ptrs) {
  if (dtype != PD_DTYPE_BF16 || d_in % 8 || d_out % 8 || C % 8) return false;
  for (const void* q : ptrs)
    if (!a16(q)) return false;
  return true;
}

static int masked_linear_fwd_fused(int64_t T, int64_t d_in, int64_t d_out, int64_t C, const void* x, const void* V,
                                   const void* U, const void* W, const void* mask, const void* delta,
                                   const uint8_t* route, void* out, void* xV, void* acts, hipStream_t s) {
  GemmArgs g1{T, C, d_in, (const bf16_t*)x, d_in, (const bf16_t*)V, C, xV, C, 1.f, 0.f, nullptr, 0, 0, 0};
  int rc = launch_dense_epi<EpiActs, bf16_t, true>(
      g1, EpiActs::Args{(const bf16_t*)mask, (const bf16_t*)delta, route, (bf16_t*)acts}, s, "pd_masked_linear_fwd xV");
  if (rc) return rc;
  if (!delta && !route)
    return pd_gemm(PD_DTYPE_BF16, T, d_out, C, acts, C, 0, U, d_out, 0, out, d_out, PD_DTYPE_BF16, 1.f, 0.f, s);
  GemmArgs g2{T, d_out, C, (const bf16_t*)acts, C, (const bf16_t*)U, d_out, out, d_out, 1.f, 0.f, nullptr, 0, 0, 0};
  KcatArgs q{(const bf16_t*)x, d_in, (const bf16_t*)W, d_in, d_in, (const bf16_t*)delta, route};
  return launch_kcat_epi<EpiStore, bf16_t, false, true>(g2, q, EpiStore::Args{}, s, "pd_masked_linear_fwd out");
}

template <typename T>
static void launch_acts(int dtype, const void* xV, const void* mask, const void* delta, const uint8_t* route,
                        int64_t Tn, int64_t C, void* acts, hipStream_t s) {
  hipLaunchKernelGGL(k_ml_acts<T>, dim3(ew_grid(Tn * C)), dim3(256), 0, s, (const T*)xV, (const T*)mask,
                     (const T*)delta, route, Tn, C, (T*)acts);
}

}  // namespace pd

using namespace pd;

extern "C" {

int pd_masked_linear_fwd(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, const void* x, const void* V,
                         const void* U, const void* W, const void* mask, const void* delta, const uint8_t* route,
                         void* out, void* xV, void* acts, void* stream) {
  if (T < 0 || d_in <= 0 || d_out <= 0 || C <= 0 || !x || !V || !U || !mask || !out || !xV || !acts)
    return fail(PD_EINVAL, "pd_masked_linear_fwd: bad args");
  if ((delta || route) && !W) return fail(PD_EINVAL, "pd_masked_linear_fwd: W required with delta/route");
  if (dtype != PD_DTYPE_F32 && dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, "pd_masked_linear_fwd: dtype");
  if (T == 0) return PD_OK;
  hipStream_t s = (hipStream_t)stream;
  if (fused_seam(dtype, d_in, d_out, C, {x, V, U, W, mask, out, xV, acts}))
    return masked_linear_fwd_fused(T, d_in, d_out, C, x, V, U, W, mask, delta, route, out, xV, acts, s);
  int rc = pd_gemm(dtype, T, C, d_in, x, d_in, 0, V, C, 0, xV, C, dtype, 1.f, 0.f, stream);
  if (rc) return rc;
  if (dtype == PD_DTYPE_F32)
    hipLaunchKernelGGL(k_ml_acts<float>, dim3(ew_grid(T * C)), dim3(256), 0, s, (const float*)xV, (const float*)mask,
                       (const float*)delta, route, T, C, (float*)acts);
  else
    hipLaunchKernelGGL(k_ml_acts<bf16_t>, dim3(ew_grid(T * C)), dim3(256), 0, s, (const bf16_t*)xV,
                       (const bf16_t*)mask, (const bf16_t*)delta, route, T, C, (bf16_t*)acts);
  if ((rc = check_launch("pd_masked_linear_fwd acts"))) return rc;
  float beta = 0.f;
  if (delta || route) {
    // out = x @ W^T, then scaled to d*target (routed) / target (unrouted)
    if ((rc = pd_gemm(dtype, T, d_out, d_in, x, d_in, 0, W, d_in, 1, out, d_out, dtype, 1.f, 0.f, stream))) return rc;
    if (dtype == PD_DTYPE_F32)
      hipLaunchKernelGGL(k_ml_scale_target<float>, dim3(ew_grid(T * d_out)), dim3(256), 0, s, (float*)out,
                         (const float*)delta, route, T, d_out);
    else
      hipLaunchKernelGGL(k_ml_scale_target<bf16_t>, dim3(ew_grid(T * d_out)), dim3(256), 0, s, (bf16_t*)out,
                         (const bf16_t*)delta, route, T, d_out);
    if ((rc = check_launch("pd_masked_linear_fwd target"))) return rc;
    beta = 1.f;
  }
  return pd_gemm(dtype, T, d_out, C, acts, C, 0, U, d_out, 0, out, d_out, dtype, 1.f, beta, stream);
}

size_t pd_masked_linear_bwd_workspace_size(int dtype, int64_t T, int64_t d_out, int64_t C) {
  size_t es = dtype == PD_DTYPE_BF16 ? 2 : 4;
  return es * (size_t)T * (size_t)C + es * (size_t)T * (size_t)d_out + 512;
}

}  // extern "C"

namespace pd {

// The fused bf16 backward (see the seam above); da and gt are the two scratch regions of
// the unfused path (T x C and T x d_out elements).
static int masked_linear_bwd_fused(int64_t T, int64_t d_in, int64_t d_out, int64_t C, const void* x, const void* V,
                                   const void* U, const void* W, const void* mask, const void* delta,
                                   const uint8_t* route, const void* xV, const void* acts, const void* g_out, void* dx,
                                   void* dV, void* dU, void* dmask, void* d_delta, void* da, void* gt,
                                   hipStream_t s) {
  const int BF = PD_DTYPE_BF16;
  int rc;
  // dU = acts^T @ g (both operands token-row-major: MN-major in the contraction)
  if (dU && (rc = pd_gemm(BF, C, d_out, T, acts, C, 1, g_out, d_out, 0, dU, d_out, BF, 1.f, 0.f, s))) return rc;
  if (!dV && !dx && !dmask && !d_delta) return PD_OK;
  GemmArgs g{T, C, d_out, (const bf16_t*)g_out, d_out, (const bf16_t*)U, d_out, da, C, 1.f, 0.f, nullptr, 0, 0, 0};
  rc = launch_dense_epi<EpiMaskedBwd, bf16_t, false>(
      g, EpiMaskedBwd::Args{(const bf16_t*)xV, (const bf16_t*)mask, (const bf16_t*)delta, route, (bf16_t*)dmask}, s,
      "pd_masked_linear_bwd da");
  if (rc) return rc;
  if (d_delta) {
    // the target x @ W^T, then the row sums
    if ((rc = pd_gemm(BF, T, d_out, d_in, x, d_in, 0, W, d_in, 1, gt, d_out, BF, 1.f, 0.f, s))) return rc;
    hipLaunchKernelGGL(k_ml_delta_grad_dm, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, s, (const bf16_t*)g_out,
                       (const bf16_t*)gt, (const bf16_t*)dmask, route, T, d_out, C, (bf16_t*)d_delta);
    if ((rc = check_launch("pd_masked_linear_bwd d_delta"))) return rc;
  }
  // dV = x^T @ dxV
  if (dV && (rc = pd_gemm(BF, d_in, C, T, x, d_in, 1, da, C, 0, dV, C, BF, 1.f, 0.f, s))) return rc;
  if (!dx) return PD_OK;
  if (!delta && !route)  // dx = dxV @ V^T
    return pd_gemm(BF, T, d_in, C, da, C, 0, V, C, 1, dx, d_in, BF, 1.f, 0.f, s);
  // dx = rs (.) (g @ W) + dxV @ V^T: W [d_out, d_in] is the MN-major B of the first product
  GemmArgs g2{T, d_in, C, (const bf16_t*)da, C, (const bf16_t*)V, C, dx, d_in, 1.f, 0.f, nullptr, 0, 0, 0};
  KcatArgs q{(const bf16_t*)g_out, d_out, (const bf16_t*)W, d_in, d_out, (const bf16_t*)delta, route};
  return launch_kcat_epi<EpiStore, bf16_t, true, false>(g2, q, EpiStore::Args{}, s, "pd_masked_linear_bwd dx");
}

// The masked-linear backward over a caller-sized scratch region `workspace` (at least
// pd_masked_linear_bwd_workspace_size bytes, 256-byte aligned). Every byte of the
// scratch it reads is written first in the same call (both regions are full GEMM
// outputs with beta = 0), so it needs no clearing between calls.
static int masked_linear_bwd_impl(const char* what, int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C,
                                  const void* x, const void* V, const void* U, const void* W, const void* mask,
                                  const void* delta, const uint8_t* route, const void* xV, const void* acts,
                                  const void* g_out, void* dx, void* dV, void* dU, void* dmask, void* d_delta,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  if (T <= 0 || d_in <= 0 || d_out <= 0 || C <= 0 || !x || !V || !U || !mask || !xV || !acts || !g_out)
    return fail(PD_EINVAL, std::string(what) + ": bad args");
  if (dtype != PD_DTYPE_F32 && dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, std::string(what) + ": dtype");
  if ((delta || route) && dx && !W) return fail(PD_EINVAL, std::string(what) + ": W required for dx");
  if (d_delta && !W) return fail(PD_EINVAL, std::string(what) + ": W required for d_delta");
  if (!workspace || workspace_bytes < pd_masked_linear_bwd_workspace_size(dtype, T, d_out, C))
    return fail(PD_EWORKSPACE, std::string(what) + ": workspace too small");
  hipStream_t s = (hipStream_t)stream;
  size_t es = dtype == PD_DTYPE_BF16 ? 2 : 4;
  char* ws = (char*)workspace;
  void* da = ws;
  void* gt = ws + ((es * T * C + 255) & ~(size_t)255);
  int rc;
  if (fused_seam(dtype, d_in, d_out, C, {x, V, U, W, mask, xV, acts, g_out, dx, dmask}) && (!d_delta || dmask))
    return masked_linear_bwd_fused(T, d_in, d_out, C, x, V, U, W, mask, delta, route, xV, acts, g_out, dx, dV, dU,
                                   dmask, d_delta, da, gt, s);
  // dU = acts^T @ g (unrouted rows of acts are zero)
  if (dU && (rc = pd_gemm(dtype, C, d_out, T, acts, C, 1, g_out, d_out, 0, dU, d_out, dtype, 1.f, 0.f, stream)))
    return rc;
  if (!dV && !dx && !dmask && !d_delta) return PD_OK;
  // da = g @ U^T
  if ((rc = pd_gemm(dtype, T, C, d_out, g_out, d_out, 0, U, d_out, 1, da, C, dtype, 1.f, 0.f, stream))) return rc;
  if (d_delta) {
    // the target x @ W^T into the target-gradient buffer, which is free until dx
    if ((rc = pd_gemm(dtype, T, d_out, d_in, x, d_in, 0, W, d_in, 1, gt, d_out, dtype, 1.f, 0.f, stream))) return rc;
    if (dtype == PD_DTYPE_F32)
      hipLaunchKernelGGL(k_ml_delta_grad<float>, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, s, (const float*)g_out,
                         (const float*)gt, (const float*)da, (const float*)xV, route, T, d_out, C, (float*)d_delta);
    else
      hipLaunchKernelGGL(k_ml_delta_grad<bf16_t>, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, s, (const bf16_t*)g_out,
                         (const bf16_t*)gt, (const bf16_t*)da, (const bf16_t*)xV, route, T, d_out, C,
                         (bf16_t*)d_delta);
    if ((rc = check_launch("pd_masked_linear_bwd d_delta"))) return rc;
  }
  if (dtype == PD_DTYPE_F32)
    hipLaunchKernelGGL(k_ml_bwd_elem<float>, dim3(ew_grid(T * C)), dim3(256), 0, s, (float*)da, (const float*)xV,
                       (const float*)mask, (const float*)delta, route, T, C, (float*)dmask);
  else
    hipLaunchKernelGGL(k_ml_bwd_elem<bf16_t>, dim3(ew_grid(T * C)), dim3(256), 0, s, (bf16_t*)da, (const bf16_t*)xV,
                       (const bf16_t*)mask, (const bf16_t*)delta, route, T, C, (bf16_t*)dmask);
  if ((rc = check_launch("pd_masked_linear_bwd elem"))) return rc;
  // dV = x^T @ dxV
  if (dV && (rc = pd_gemm(dtype, d_in, C, T, x, d_in, 1, da, C, 0, dV, C, dtype, 1.f, 0.f, stream))) return rc;
  if (!dx) return PD_OK;
  // dx = dxV @ V^T (+ g_target @ W)
  if ((rc = pd_gemm(dtype, T, d_in, C, da, C, 0, V, C, 1, dx, d_in, dtype, 1.f, 0.f, stream))) return rc;
  if (delta || route) {
    if (dtype == PD_DTYPE_F32)
      hipLaunchKernelGGL(k_ml_target_grad<float>, dim3(ew_grid(T * d_out)), dim3(256), 0, s, (const float*)g_out,
                         (const float*)delta, route, T, d_out, (float*)gt);
    else
      hipLaunchKernelGGL(k_ml_target_grad<bf16_t>, dim3(ew_grid(T * d_out)), dim3(256), 0, s, (const bf16_t*)g_out,
                         (const bf16_t*)delta, route, T, d_out, (bf16_t*)gt);
    if ((rc = check_launch("pd_masked_linear_bwd target"))) return rc;
    if ((rc = pd_gemm(dtype, T, d_in, d_out, gt, d_out, 0, W, d_in, 0, dx, d_in, dtype, 1.f, 1.f, stream))) return rc;
  }
  return PD_OK;
}

// Scratch of the allocation-free backward: one region per GPU, file scope, held by each
// device the library runs on until the process ends. Host code reaches its device
// address only through noalloc_scratch(), never through the symbol itself.
constexpr size_t NOALLOC_SCRATCH_BYTES = PD_MASKED_LINEAR_BWD_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[MAX_DEVICES] = {};

// The current device's copy of `scratch`, looked up once per device (with that device
// current) by hipGetSymbolAddress; nullptr (and the error state set) on failure.
static void* noalloc_scratch(const char* what) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
    fail(PD_ELAUNCH, std::string(what) + ": no current HIP device in range");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(PD_ELAUNCH, std::string(what) + ": hipGetSymbolAddress(scratch) failed: " + hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace pd

extern "C" {

int pd_masked_linear_bwd(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, const void* x, const void* V,
                         const void* U, const void* W, const void* mask, const void* delta, const uint8_t* route,
                         const void* xV, const void* acts, const void* g_out, void* dx, void* dV, void* dU,
                         void* dmask, void* d_delta, void* workspace, size_t workspace_bytes, void* stream) {
  return masked_linear_bwd_impl("pd_masked_linear_bwd", dtype, T, d_in, d_out, C, x, V, U, W, mask, delta, route, xV,
                                acts, g_out, dx, dV, dU, dmask, d_delta, workspace, workspace_bytes, stream);
}

int pd_masked_linear_bwd_noalloc(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, const void* x,
                                 const void* V, const void* U, const void* W, const void* mask, const void* delta,
                                 const uint8_t* route, const void* xV, const void* acts, const void* g_out, void* dx,
                                 void* dV, void* dU, void* dmask, void* d_delta, void* stream) {
  const char* what = "pd_masked_linear_bwd_noalloc";
  if (T > 0 && C > 0 && d_out > 0 && pd_masked_linear_bwd_workspace_size(dtype, T, d_out, C) > NOALLOC_SCRATCH_BYTES)
    return fail(PD_EUNSUPPORTED, std::string(what) + ": needs " +
                                     std::to_string(pd_masked_linear_bwd_workspace_size(dtype, T, d_out, C)) +
                                     " scratch bytes (T*C + T*d_out elements + 512), above the fixed " +
                                     std::to_string(NOALLOC_SCRATCH_BYTES) + "; use pd_masked_linear_bwd");
  void* ws = noalloc_scratch(what);
  if (!ws) return PD_ELAUNCH;
  return masked_linear_bwd_impl(what, dtype, T, d_in, d_out, C, x, V, U, W, mask, delta, route, xV, acts, g_out, dx, dV,
                                dU, dmask, d_delta, ws, NOALLOC_SCRATCH_BYTES, stream);
}


// ---------------------------------------------------------------- block-factored site
// pd/core/decomposed_linear.py:209-271 (blocked_site_forward), einsums of
// pd/core/linear_plan.py:149-160. With C = E*c block-major:
//   fused_output: xV[:, e] = x @ V[e]            out[:, e] = acts[:, e] @ U[e]   (concat)
//   fused_input:  xV[:, e] = x[:, e] @ V[e]      out = sum_e acts[:, e] @ U[e]   (one GEMM)
// acts = routed ? xV * (m - d) : 0; with delta/route the target x @ W^T is blended as in
// site_forward. Per-block products run as strided-batched GEMMs.
int pd_blocked_site_fwd(int dtype, int contraction, int64_t T, int64_t E, int64_t d_in, int64_t d_out, int64_t c,
                        const void* x, const void* V, const void* U, const void* W, const void* mask, const void* delta,
                        const uint8_t* route, void* out, void* xV, void* acts, void* stream) {
  if (T < 0 || E <= 0 || d_in <= 0 || d_out <= 0 || c <= 0 || !x || !V || !U || !mask || !out || !xV || !acts)
    return fail(PD_EINVAL, "pd_blocked_site_fwd: bad args");
  if (contraction != PD_BLOCK_FUSED_OUTPUT && contraction != PD_BLOCK_FUSED_INPUT)
    return fail(PD_EINVAL, "pd_blocked_site_fwd: contraction");
  if ((delta || route) && !W) return fail(PD_EINVAL, "pd_blocked_site_fwd: W required with delta/route");
  if (dtype != PD_DTYPE_F32 && dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, "pd_blocked_site_fwd: dtype");
  if (dtype == PD_DTYPE_BF16 && (d_in % 8 || d_out % 8 || c % 8))
    return fail(PD_EUNSUPPORTED, "pd_blocked_site_fwd: bf16 needs d_in, d_out, c multiples of 8");
  if (T == 0) return PD_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool fo = contraction == PD_BLOCK_FUSED_OUTPUT;
  const int64_t C = E * c, DI = fo ? d_in : E * d_in, DO = fo ? E * d_out : d_out;
  int rc = pd_gemm_strided_batched(dtype, E, T, c, d_in, x, DI, fo ? 0 : d_in, 0, V, c, d_in * c, 0, xV, C, c, dtype,
                                   1.f, 0.f, stream);
  if (rc) return rc;
  if (dtype == PD_DTYPE_F32)
    launch_acts<float>(dtype, xV, mask, delta, route, T, C, acts, s);
  else
    launch_acts<bf16_t>(dtype, xV, mask, delta, route, T, C, acts, s);
  if ((rc = check_launch("pd_blocked_site_fwd acts"))) return rc;
  float beta = 0.f;
  if (delta || route) {
    if ((rc = pd_gemm(dtype, T, DO, DI, x, DI, 0, W, DI, 1, out, DO, dtype, 1.f, 0.f, stream))) return rc;
    if (dtype == PD_DTYPE_F32)
      hipLaunchKernelGGL(k_ml_scale_target<float>, dim3(ew_grid(T * DO)), dim3(256), 0, s, (float*)out,
                         (const float*)delta, route, T, DO);
    else
      hipLaunchKernelGGL(k_ml_scale_target<bf16_t>, dim3(ew_grid(T * DO)), dim3(256), 0, s, (bf16_t*)out,
                         (const bf16_t*)delta, route, T, DO);
    if ((rc = check_launch("pd_blocked_site_fwd target"))) return rc;
    beta = 1.f;
  }
  if (fo)
    return pd_gemm_strided_batched(dtype, E, T, d_out, c, acts, C, c, 0, U, d_out, c * d_out, 0, out, DO, d_out, dtype,
                                   1.f, beta, stream);
  return pd_gemm(dtype, T, d_out, C, acts, C, 0, U, d_out, 0, out, d_out, dtype, 1.f, beta, stream);
}

static size_t blocked_ws_plan(int dtype, int contraction, int64_t T, int64_t E, int64_t d_in, int64_t d_out, int64_t c,
                              size_t* off_gt, size_t* off_dx32) {
  const size_t es = dtype == PD_DTYPE_BF16 ? 2 : 4;
  const bool fo = contraction == PD_BLOCK_FUSED_OUTPUT;
  const int64_t C = E * c, DI = fo ? d_in : E * d_in, DO = fo ? E * d_out : d_out;
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  size_t off = up(es * (size_t)T * C);  // da
  *off_gt = off;
  off += up(es * (size_t)T * DO);
  *off_dx32 = off;
  off += up(4 * (size_t)T * DI);
  return off;
}

size_t pd_blocked_site_bwd_workspace_size(int dtype, int contraction, int64_t T, int64_t E, int64_t d_in,
                                          int64_t d_out, int64_t c) {
  size_t a, b;
  return blocked_ws_plan(dtype, contraction, T, E, d_in, d_out, c, &a, &b);
}

int pd_blocked_site_bwd(int dtype, int contraction, int64_t T, int64_t E, int64_t d_in, int64_t d_out, int64_t c,
                        const void* x, const void* V, const void* U, const void* W, const void* mask, const void* delta,
                        const uint8_t* route, const void* xV, const void* acts, const void* g_out, void* dx, void* dV,
                        void* dU, void* dmask, void* d_delta, void* workspace, size_t workspace_bytes, void* stream) {
  if (T <= 0 || E <= 0 || d_in <= 0 || d_out <= 0 || c <= 0 || !x || !V || !U || !mask || !xV || !acts || !g_out ||
      !dV || !dU)
    return fail(PD_EINVAL, "pd_blocked_site_bwd: bad args");
  if (d_delta && !W) return fail(PD_EINVAL, "pd_blocked_site_bwd: W required for d_delta");
  if (contraction != PD_BLOCK_FUSED_OUTPUT && contraction != PD_BLOCK_FUSED_INPUT)
    return fail(PD_EINVAL, "pd_blocked_site_bwd: contraction");
  if ((delta || route) && dx && !W) return fail(PD_EINVAL, "pd_blocked_site_bwd: W required for dx");
  if (dtype != PD_DTYPE_F32 && dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, "pd_blocked_site_bwd: dtype");
  if (dtype == PD_DTYPE_BF16 && (d_in % 8 || d_out % 8 || c % 8))
    return fail(PD_EUNSUPPORTED, "pd_blocked_site_bwd: bf16 needs d_in, d_out, c multiples of 8");
  size_t off_gt, off_dx32;
  if (!workspace ||
      workspace_bytes < blocked_ws_plan(dtype, contraction, T, E, d_in, d_out, c, &off_gt, &off_dx32))
    return fail(PD_EWORKSPACE, "pd_blocked_site_bwd: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  const bool fo = contraction == PD_BLOCK_FUSED_OUTPUT;
  const int64_t C = E * c, DI = fo ? d_in : E * d_in, DO = fo ? E * d_out : d_out;
  char* ws = (char*)workspace;
  void* da = ws;
  void* gt = ws + off_gt;
  float* dx32 = (float*)(ws + off_dx32);
  int rc;
  if (fo) {
    // dU[e] = acts[:, e]^T @ g[:, e];  da[:, e] = g[:, e] @ U[e]^T
    if ((rc = pd_gemm_strided_batched(dtype, E, c, d_out, T, acts, C, c, 1, g_out, DO, d_out, 0, dU, d_out, c * d_out,
                                      dtype, 1.f, 0.f, stream)))
      return rc;
    if ((rc = pd_gemm_strided_batched(dtype, E, T, c, d_out, g_out, DO, d_out, 0, U, d_out, c * d_out, 1, da, C, c,
                                      dtype, 1.f, 0.f, stream)))
      return rc;
  } else {
    if ((rc = pd_gemm(dtype, C, d_out, T, acts, C, 1, g_out, d_out, 0, dU, d_out, dtype, 1.f, 0.f, stream))) return rc;
    if ((rc = pd_gemm(dtype, T, C, d_out, g_out, d_out, 0, U, d_out, 1, da, C, dtype, 1.f, 0.f, stream))) return rc;
  }
  if (d_delta) {
    // the delta cotangent over the whole site output: the target x @ W^T into the
    // target-gradient buffer (free until dx), then the row sums of g*target - da*xV
    if ((rc = pd_gemm(dtype, T, DO, DI, x, DI, 0, W, DI, 1, gt, DO, dtype, 1.f, 0.f, stream))) return rc;
    if (dtype == PD_DTYPE_F32)
      hipLaunchKernelGGL(k_ml_delta_grad<float>, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, s, (const float*)g_out,
                         (const float*)gt, (const float*)da, (const float*)xV, route, T, DO, C, (float*)d_delta);
    else
      hipLaunchKernelGGL(k_ml_delta_grad<bf16_t>, dim3((unsigned)cdiv(T, 4)), dim3(256), 0, s, (const bf16_t*)g_out,
                         (const bf16_t*)gt, (const bf16_t*)da, (const bf16_t*)xV, route, T, DO, C, (bf16_t*)d_delta);
    if ((rc = check_launch("pd_blocked_site_bwd d_delta"))) return rc;
  }
  if (dtype == PD_DTYPE_F32)
    hipLaunchKernelGGL(k_ml_bwd_elem<float>, dim3(ew_grid(T * C)), dim3(256), 0, s, (float*)da, (const float*)xV,
                       (const float*)mask, (const float*)delta, route, T, C, (float*)dmask);
  else
    hipLaunchKernelGGL(k_ml_bwd_elem<bf16_t>, dim3(ew_grid(T * C)), dim3(256), 0, s, (bf16_t*)da, (const bf16_t*)xV,
                       (const bf16_t*)mask, (const bf16_t*)delta, route, T, C, (bf16_t*)dmask);
  if ((rc = check_launch("pd_blocked_site_bwd elem"))) return rc;
  // dV[e] = x_e^T @ dxV[:, e]
  if ((rc = pd_gemm_strided_batched(dtype, E, d_in, c, T, x, DI, fo ? 0 : d_in, 1, da, C, c, 0, dV, c, d_in * c,
                                    dtype, 1.f, 0.f, stream)))
    return rc;
  if (!dx) return PD_OK;
  // dx accumulates in fp32 (per-block sums, the target term), then takes the site dtype
  float* acc = dtype == PD_DTYPE_F32 ? (float*)dx : dx32;
  if (fo) {
    for (int64_t e = 0; e < E; ++e) {
      const char* dae = (const char*)da + (size_t)e * c * (dtype == PD_DTYPE_BF16 ? 2 : 4);
      const char* ve = (const char*)V + (size_t)e * d_in * c * (dtype == PD_DTYPE_BF16 ? 2 : 4);
      if ((rc = pd_gemm(dtype, T, d_in, c, dae, C, 0, ve, c, 1, acc, d_in, PD_DTYPE_F32, 1.f, e ? 1.f : 0.f, stream)))
        return rc;
    }
  } else {
    if ((rc = pd_gemm_strided_batched(dtype, E, T, d_in, c, da, C, c, 0, V, c, d_in * c, 1, acc, DI, d_in,
                                      PD_DTYPE_F32, 1.f, 0.f, stream)))
      return rc;
  }
  if (delta || route) {
    if (dtype == PD_DTYPE_F32)
      hipLaunchKernelGGL(k_ml_target_grad<float>, dim3(ew_grid(T * DO)), dim3(256), 0, s, (const float*)g_out,
                         (const float*)delta, route, T, DO, (float*)gt);
    else
      hipLaunchKernelGGL(k_ml_target_grad<bf16_t>, dim3(ew_grid(T * DO)), dim3(256), 0, s, (const bf16_t*)g_out,
                         (const bf16_t*)delta, route, T, DO, (bf16_t*)gt);
    if ((rc = check_launch("pd_blocked_site_bwd target"))) return rc;
    if ((rc = pd_gemm(dtype, T, DI, DO, gt, DO, 0, W, DI, 0, acc, DI, PD_DTYPE_F32, 1.f, 1.f, stream))) return rc;
  }
  if (dtype == PD_DTYPE_BF16) {
    hipLaunchKernelGGL(k_f32_to_bf16, dim3(ew_grid(T * DI)), dim3(256), 0, s, dx32, T * DI, (bf16_t*)dx);
    return check_launch("pd_blocked_site_bwd dx");
  }
  return PD_OK;
}

}  // extern "C"
