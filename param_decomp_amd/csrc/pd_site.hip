// Site-level entry points (gfx950): the masked decomposed linear and the fused
// single-site stochastic-recon step.
//
//   pd_masked_linear_fwd/bwd   pd/core/decomposed_linear.py:142-175 (site_forward),
//                              :65-85 (component_coefficients, blend_target_output)
//   pd_dense_step              one stochastic-recon + imp-min fwd+bwd of a single site
//                              (pd/core/train.py:1126-1352 restricted to one site, the
//                              paper-form gate, pd/core/masking.py:148-167 draws)
#include "pd_common.hpp"

namespace pd {

static constexpr int SITE_COLS = 64;  // columns (components) per block in column-mapped kernels
static constexpr int SITE_ROWS = 64;  // rows per block chunk

static int ew_grid(int64_t n) {
  int64_t b = cdiv(n, 1024);
  return (int)(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

// ---------------------------------------------------------------- masked linear helpers
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

// ---------------------------------------------------------------- dense step kernels
struct StepParams {
  int64_t T, C;
  uint32_t mk0, mk1, dk0, dk1;
  int use_delta, draw_dtype, layout;
  float p, imp_scale;  // imp_scale = imp_coeff / T
};

__device__ inline float step_delta(const StepParams& s, int64_t t) {
  return s.use_delta ? draw_uniform(s.dk0, s.dk1, t, s.T, s.draw_dtype, s.layout) : 0.f;
}

__device__ inline float pow_p(float b, float p) { return p == 2.f ? b * b : (p == 1.f ? b : powf(b, p)); }
__device__ inline float dpow_p(float b, float p) {
  return p == 2.f ? 2.f * b : (p == 1.f ? 1.f : p * powf(b, p - 1.f));
}

// Forward, one component per lane: gate MLP on h, squash, draw u, acts = h*(m-d),
// imp-min partial sum of upper^p. Writes g_raw (fp32) for the backward.
template <typename T, bool PRECISE>
__global__ __launch_bounds__(SITE_COLS) void k_step_fwd(const T* __restrict__ h, const float* __restrict__ w_in,
                                                        const float* __restrict__ b_in,
                                                        const float* __restrict__ w_out,
                                                        const float* __restrict__ b_out, StepParams s,
                                                        float* __restrict__ g_raw, T* __restrict__ acts,
                                                        float* __restrict__ imp_partial) {
  const int64_t c = (int64_t)blockIdx.x * SITE_COLS + threadIdx.x;
  float imp = 0.f;
  if (c < s.C) {
    float wi[16], bi[16], wo[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      wi[j] = w_in[c * 16 + j];
      bi[j] = b_in[c * 16 + j];
      wo[j] = w_out[c * 16 + j];
    }
    const float bo = b_out[c];
    const int64_t r0 = (int64_t)blockIdx.y * SITE_ROWS;
    const int64_t r1 = r0 + SITE_ROWS < s.T ? r0 + SITE_ROWS : s.T;
    const int64_t n = s.T * s.C;
    for (int64_t t = r0; t < r1; ++t) {
      const int64_t i = t * s.C + c;
      const float hv = load_f<T>(h, i);
      float g = bo;
#pragma unroll
      for (int j = 0; j < 16; ++j) g = fmaf(wo[j], gelu_only<PRECISE>(fmaf(wi[j], hv, bi[j])), g);
      g_raw[i] = g;
      const float lo = lower_fwd(g);
      imp += pow_p(upper_fwd(g), s.p);
      const float u = draw_uniform(s.mk0, s.mk1, i, n, s.draw_dtype, s.layout);
      const float m = lo + (1.f - lo) * u;
      store_f<T>(acts, i, hv * (m - step_delta(s, t)));
    }
  }
  imp = wave_sum(imp);
  if (threadIdx.x == 0) imp_partial[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = imp;
}

// Recon residual: e = y + d*yt - yt; accumulates e^2; writes dy = gscale*e over y.
template <typename T>
__global__ void k_step_recon(T* __restrict__ y, const T* __restrict__ yt, StepParams s, int64_t D, float gscale,
                             float* __restrict__ partial) {
  const int64_t n = s.T * D;
  float acc = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / D;
    const float tv = load_f<T>(yt, i);
    const float e = load_f<T>(y, i) + step_delta(s, t) * tv - tv;
    acc = fmaf(e, e, acc);
    store_f<T>(y, i, gscale * e);
  }
  __shared__ float sw[4];
  acc = wave_sum(acc);
  if (threadIdx.x % 64 == 0) sw[threadIdx.x / 64] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = sw[0] + sw[1] + sw[2] + sw[3];
}

// Backward, one component per lane: from da = dy@U^T, h, g_raw and the regenerated u:
// dh = da*(m-d) + gate pullback of dg_raw, where dg_raw = lower_vjp(g, da*h*(1-u))
// + upper_vjp(g, imp_scale * d upper^p). Gate parameter grads go to per-chunk partials.
template <typename T, bool PRECISE>
__global__ __launch_bounds__(SITE_COLS) void k_step_bwd(const T* __restrict__ da, const T* __restrict__ h,
                                                        const float* __restrict__ g_raw,
                                                        const float* __restrict__ w_in,
                                                        const float* __restrict__ b_in,
                                                        const float* __restrict__ w_out, StepParams s,
                                                        T* __restrict__ dh, float* __restrict__ partial) {
  const int64_t c = (int64_t)blockIdx.x * SITE_COLS + threadIdx.x;
  if (c >= s.C) return;
  float wi[16], bi[16], wo[16], a_wi[16], a_bi[16], a_wo[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    wi[j] = w_in[c * 16 + j];
    bi[j] = b_in[c * 16 + j];
    wo[j] = w_out[c * 16 + j];
    a_wi[j] = a_bi[j] = a_wo[j] = 0.f;
  }
  float a_bo = 0.f;
  const int64_t r0 = (int64_t)blockIdx.y * SITE_ROWS;
  const int64_t r1 = r0 + SITE_ROWS < s.T ? r0 + SITE_ROWS : s.T;
  const int64_t n = s.T * s.C;
  for (int64_t t = r0; t < r1; ++t) {
    const int64_t i = t * s.C + c;
    const float hv = load_f<T>(h, i), g = g_raw[i], dav = load_f<T>(da, i);
    const float lo = lower_fwd(g);
    const float u = draw_uniform(s.mk0, s.mk1, i, n, s.draw_dtype, s.layout);
    const float m = lo + (1.f - lo) * u;
    float dhv = dav * (m - step_delta(s, t));
    float dg = lower_vjp(g, dav * hv * (1.f - u)) + upper_vjp(g, s.imp_scale * dpow_p(upper_fwd(g), s.p));
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

__global__ void k_step_gate_reduce(const float* __restrict__ partial, int64_t chunks, int64_t C,
                                   float* __restrict__ dw_in, float* __restrict__ db_in, float* __restrict__ dw_out,
                                   float* __restrict__ db_out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= 49 * C) return;
  const int64_t q = idx / C, c = idx % C;
  float acc = 0.f;
  for (int64_t k = 0; k < chunks; ++k) acc += partial[k * 49 * C + idx];
  if (q < 16)
    dw_in[c * 16 + q] = acc;
  else if (q < 32)
    db_in[c * 16 + q - 16] = acc;
  else if (q < 48)
    dw_out[c * 16 + q - 32] = acc;
  else
    db_out[c] = acc;
}

// losses[0..2] = {loss, recon, imp} from the two partial arrays (one block, fixed order)
__global__ void k_step_losses(const float* __restrict__ rec_part, int64_t n_rec, const float* __restrict__ imp_part,
                              int64_t n_imp, double rec_scale, double imp_scale, float recon_coeff, float imp_coeff,
                              float* __restrict__ losses) {
  __shared__ double sr[16], si[16];
  double r = 0.0, m = 0.0;
  for (int64_t i = threadIdx.x; i < n_rec; i += blockDim.x) r += rec_part[i];
  for (int64_t i = threadIdx.x; i < n_imp; i += blockDim.x) m += imp_part[i];
  r = wave_sum_d(r);
  m = wave_sum_d(m);
  if (threadIdx.x % 64 == 0) {
    sr[threadIdx.x / 64] = r;
    si[threadIdx.x / 64] = m;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double a = 0, b = 0;
    for (int i = 0; i < (int)(blockDim.x / 64); ++i) {
      a += sr[i];
      b += si[i];
    }
    a *= rec_scale;
    b *= imp_scale;
    losses[0] = (float)(recon_coeff * a + imp_coeff * b);
    losses[1] = (float)a;
    losses[2] = (float)b;
  }
}

static constexpr int RECON_BLOCKS = 1024;

struct StepWorkspace {
  size_t yt, h, acts, y, da, dh, graw, imp, rec, gate, total;
};

static StepWorkspace step_layout(int dtype, int64_t T, int64_t C, int64_t d_out) {
  size_t es = dtype == PD_DTYPE_BF16 ? 2 : 4;
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  StepWorkspace w{};
  size_t o = 0;
  w.yt = o;
  o += al(es * T * d_out);
  w.h = o;
  o += al(es * T * C);
  w.acts = o;
  o += al(es * T * C);
  w.y = o;
  o += al(es * T * d_out);
  w.da = o;
  o += al(es * T * C);
  w.dh = o;
  o += al(es * T * C);
  w.graw = o;
  o += al(4 * T * C);
  w.imp = o;
  o += al(4 * cdiv(T, SITE_ROWS) * cdiv(C, SITE_COLS));
  w.rec = o;
  o += al(4 * RECON_BLOCKS);
  w.gate = o;
  o += al(4 * cdiv(T, SITE_ROWS) * 49 * C);
  w.total = o;
  return w;
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

int pd_masked_linear_bwd(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, const void* x, const void* V,
                         const void* U, const void* W, const void* mask, const void* delta, const uint8_t* route,
                         const void* xV, const void* acts, const void* g_out, void* dx, void* dV, void* dU,
                         void* dmask, void* workspace, size_t workspace_bytes, void* stream) {
  if (T <= 0 || d_in <= 0 || d_out <= 0 || C <= 0 || !x || !V || !U || !mask || !xV || !acts || !g_out || !dV || !dU)
    return fail(PD_EINVAL, "pd_masked_linear_bwd: bad args");
  if ((delta || route) && dx && !W) return fail(PD_EINVAL, "pd_masked_linear_bwd: W required for dx");
  if (!workspace || workspace_bytes < pd_masked_linear_bwd_workspace_size(dtype, T, d_out, C))
    return fail(PD_EWORKSPACE, "pd_masked_linear_bwd: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  size_t es = dtype == PD_DTYPE_BF16 ? 2 : 4;
  char* ws = (char*)workspace;
  void* da = ws;
  void* gt = ws + ((es * T * C + 255) & ~(size_t)255);
  int rc;
  // dU = acts^T @ g (unrouted rows of acts are zero)
  if ((rc = pd_gemm(dtype, C, d_out, T, acts, C, 1, g_out, d_out, 0, dU, d_out, dtype, 1.f, 0.f, stream))) return rc;
  // da = g @ U^T
  if ((rc = pd_gemm(dtype, T, C, d_out, g_out, d_out, 0, U, d_out, 1, da, C, dtype, 1.f, 0.f, stream))) return rc;
  if (dtype == PD_DTYPE_F32)
    hipLaunchKernelGGL(k_ml_bwd_elem<float>, dim3(ew_grid(T * C)), dim3(256), 0, s, (float*)da, (const float*)xV,
                       (const float*)mask, (const float*)delta, route, T, C, (float*)dmask);
  else
    hipLaunchKernelGGL(k_ml_bwd_elem<bf16_t>, dim3(ew_grid(T * C)), dim3(256), 0, s, (bf16_t*)da, (const bf16_t*)xV,
                       (const bf16_t*)mask, (const bf16_t*)delta, route, T, C, (bf16_t*)dmask);
  if ((rc = check_launch("pd_masked_linear_bwd elem"))) return rc;
  // dV = x^T @ dxV
  if ((rc = pd_gemm(dtype, d_in, C, T, x, d_in, 1, da, C, 0, dV, C, dtype, 1.f, 0.f, stream))) return rc;
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

size_t pd_dense_step_workspace_size(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H) {
  (void)d_in;
  (void)H;
  return step_layout(dtype, T, C, d_out).total;
}

}  // extern "C"

// Phase boundaries recorded into caller events (events may be NULL): see
// pd_dense_step_timed in the header for the phase order.
static int dense_step_impl(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H, const void* x,
                           const void* W, const void* V, const void* U, const float* w_in, const float* b_in,
                           const float* w_out, const float* b_out, uint32_t mk0, uint32_t mk1, uint32_t dk0,
                           uint32_t dk1, int use_delta, int draw_dtype, int layout, float p, float imp_coeff,
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
  StepWorkspace L = step_layout(dtype, T, C, d_out);
  if (!workspace || workspace_bytes < L.total) return fail(PD_EWORKSPACE, "pd_dense_step: workspace too small");
  if (cdiv(T, SITE_ROWS) > 65535) return fail(PD_EUNSUPPORTED, "pd_dense_step: T too large");
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  void *yt = ws + L.yt, *h = ws + L.h, *acts = ws + L.acts, *y = ws + L.y, *da = ws + L.da, *dh = ws + L.dh;
  float* graw = (float*)(ws + L.graw);
  float* imp_part = (float*)(ws + L.imp);
  float* rec_part = (float*)(ws + L.rec);
  float* gate_part = (float*)(ws + L.gate);
  const bool precise = dtype == PD_DTYPE_F32;
  StepParams sp{T, C, mk0, mk1, dk0, dk1, use_delta, draw_dtype, layout, p, imp_coeff / (float)T};
  dim3 cgrid((unsigned)cdiv(C, SITE_COLS), (unsigned)cdiv(T, SITE_ROWS));
  int rc;
  // clean target and inner activations
  PD_MARK(0);
  if ((rc = pd_gemm(dtype, T, d_out, d_in, x, d_in, 0, W, d_in, 1, yt, d_out, dtype, 1.f, 0.f, stream))) return rc;
  PD_MARK(1);
  if ((rc = pd_gemm(dtype, T, C, d_in, x, d_in, 0, V, C, 0, h, C, dtype, 1.f, 0.f, stream))) return rc;
  PD_MARK(2);
#define PD_STEP_FWD(TT, PR)                                                                                    \
  hipLaunchKernelGGL((k_step_fwd<TT, PR>), cgrid, dim3(SITE_COLS), 0, s, (const TT*)h, w_in, b_in, w_out, b_out, \
                     sp, graw, (TT*)acts, imp_part)
  if (dtype == PD_DTYPE_F32)
    PD_STEP_FWD(float, true);
  else
    PD_STEP_FWD(bf16_t, false);
#undef PD_STEP_FWD
  if ((rc = check_launch("pd_dense_step fwd"))) return rc;
  PD_MARK(3);
  if ((rc = pd_gemm(dtype, T, d_out, C, acts, C, 0, U, d_out, 0, y, d_out, dtype, 1.f, 0.f, stream))) return rc;
  PD_MARK(4);
  const float gscale = recon_coeff * 2.f / (float)(T * d_out);
  if (dtype == PD_DTYPE_F32)
    hipLaunchKernelGGL(k_step_recon<float>, dim3(RECON_BLOCKS), dim3(256), 0, s, (float*)y, (const float*)yt, sp,
                       d_out, gscale, rec_part);
  else
    hipLaunchKernelGGL(k_step_recon<bf16_t>, dim3(RECON_BLOCKS), dim3(256), 0, s, (bf16_t*)y, (const bf16_t*)yt, sp,
                       d_out, gscale, rec_part);
  if ((rc = check_launch("pd_dense_step recon"))) return rc;
  PD_MARK(5);
  hipLaunchKernelGGL(k_step_losses, dim3(1), dim3(1024), 0, s, rec_part, (int64_t)RECON_BLOCKS, imp_part,
                     (int64_t)(cgrid.x * cgrid.y), 1.0 / (double)(T * d_out), 1.0 / (double)T, recon_coeff, imp_coeff,
                     losses);
  PD_MARK(6);
  // backward: y now holds dy
  if ((rc = pd_gemm(dtype, C, d_out, T, acts, C, 1, y, d_out, 0, dU, d_out, PD_DTYPE_F32, 1.f, 0.f, stream)))
    return rc;
  PD_MARK(7);
  if ((rc = pd_gemm(dtype, T, C, d_out, y, d_out, 0, U, d_out, 1, da, C, dtype, 1.f, 0.f, stream))) return rc;
  PD_MARK(8);
#define PD_STEP_BWD(TT, PR)                                                                                  \
  hipLaunchKernelGGL((k_step_bwd<TT, PR>), cgrid, dim3(SITE_COLS), 0, s, (const TT*)da, (const TT*)h, graw, w_in, \
                     b_in, w_out, sp, (TT*)dh, gate_part)
  if (dtype == PD_DTYPE_F32)
    PD_STEP_BWD(float, true);
  else
    PD_STEP_BWD(bf16_t, false);
#undef PD_STEP_BWD
  if ((rc = check_launch("pd_dense_step bwd"))) return rc;
  PD_MARK(9);
  hipLaunchKernelGGL(k_step_gate_reduce, dim3((unsigned)cdiv(49 * C, 256)), dim3(256), 0, s, gate_part,
                     (int64_t)cgrid.y, C, dw_in, db_in, dw_out, db_out);
  if ((rc = check_launch("pd_dense_step gate reduce"))) return rc;
  PD_MARK(10);
  if ((rc = pd_gemm(dtype, d_in, C, T, x, d_in, 1, dh, C, 0, dV, C, PD_DTYPE_F32, 1.f, 0.f, stream))) return rc;
  PD_MARK(11);
  return PD_OK;
#undef PD_MARK
}

extern "C" {

int pd_dense_step(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H, const void* x, const void* W,
                  const void* V, const void* U, const float* w_in, const float* b_in, const float* w_out,
                  const float* b_out, uint32_t mk0, uint32_t mk1, uint32_t dk0, uint32_t dk1, int use_delta,
                  int draw_dtype, int layout, float p, float imp_coeff, float recon_coeff, float* losses, float* dV,
                  float* dU, float* dw_in, float* db_in, float* dw_out, float* db_out, void* workspace,
                  size_t workspace_bytes, void* stream) {
  return dense_step_impl(dtype, T, d_in, d_out, C, H, x, W, V, U, w_in, b_in, w_out, b_out, mk0, mk1, dk0, dk1,
                         use_delta, draw_dtype, layout, p, imp_coeff, recon_coeff, losses, dV, dU, dw_in, db_in,
                         dw_out, db_out, workspace, workspace_bytes, stream, nullptr);
}

int pd_dense_step_timed(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H, const void* x,
                        const void* W, const void* V, const void* U, const float* w_in, const float* b_in,
                        const float* w_out, const float* b_out, uint32_t mk0, uint32_t mk1, uint32_t dk0,
                        uint32_t dk1, int use_delta, int draw_dtype, int layout, float p, float imp_coeff,
                        float recon_coeff, float* losses, float* dV, float* dU, float* dw_in, float* db_in,
                        float* dw_out, float* db_out, void* workspace, size_t workspace_bytes, void* stream,
                        void** events) {
  if (!events) return fail(PD_EINVAL, "pd_dense_step_timed: events required");
  return dense_step_impl(dtype, T, d_in, d_out, C, H, x, W, V, U, w_in, b_in, w_out, b_out, mk0, mk1, dk0, dk1,
                         use_delta, draw_dtype, layout, p, imp_coeff, recon_coeff, losses, dV, dU, dw_in, db_in,
                         dw_out, db_out, workspace, workspace_bytes, stream, events);
}

}  // extern "C"
