// Elementwise and reduction kernels of the masked-component path (gfx950).
//
//   pd_uniform            jax.random.uniform           pd/core/linear_plan.py:80-106
//   pd_squash_fwd/bwd     leaky hard sigmoids          pd/core/ci_fn/squashing.py:8-45
//   pd_component_mask_*   m = g + (1-g) u              pd/core/masking.py:135-136
//   pd_gate_fwd/bwd       per-component gate MLP       spd_paper.md appendix (CI MLPs)
//   pd_impmin             L_p / smooth-L0 imp-min      pd/core/losses.py:357-485
//   pd_mse, pd_kl         recon losses                 pd/targets/tms.py:380, pd/core/losses.py:80-92
//
// Every reduction is two-phase with a fixed grid (per-block partials, then one block
// summing them in index order), so results are bit-reproducible run to run.
#include <math.h>

#include <mutex>
#include <string>

#include "pd_common.hpp"

namespace pd {

static thread_local std::string g_last_error;
void set_error(const std::string& msg) { g_last_error = msg; }
int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}
int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PD_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return PD_OK;
}

static constexpr int EW_THREADS = 256;
static constexpr int RED_BLOCKS = 1024;  // fixed partial count for scalar reductions

static int ew_blocks(int64_t n) {
  int64_t b = cdiv(n, (int64_t)EW_THREADS * 4);
  if (b < 1) b = 1;
  if (b > 8192) b = 8192;
  return (int)b;
}

// ---------------------------------------------------------------- uniform
template <typename TO>
__global__ void k_uniform(uint32_t k0, uint32_t k1, int64_t n, int draw_dtype, int layout, TO* out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    store_f<TO>(out, i, draw_uniform(k0, k1, i, n, draw_dtype, layout));
}

// ---------------------------------------------------------------- squashing
template <typename T>
__global__ void k_squash_fwd(const T* pre, int64_t n, T* lower, T* upper) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float x = load_f<T>(pre, i);
    if (lower) store_f<T>(lower, i, lower_fwd(x));
    if (upper) store_f<T>(upper, i, upper_fwd(x));
  }
}

template <typename T>
__global__ void k_squash_bwd(const T* pre, const T* gl, const T* gu, int64_t n, T* d) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float x = load_f<T>(pre, i);
    float v = 0.f;
    if (gl) v += lower_vjp(x, load_f<T>(gl, i));
    if (gu) v += upper_vjp(x, load_f<T>(gu, i));
    store_f<T>(d, i, v);
  }
}

// ---------------------------------------------------------------- component mask
// kd (device key, optional): the key read from device memory at launch time instead of
// (k0, k1), so a captured graph draws fresh masks on each replay once the key is rewritten.
template <typename T>
__global__ void k_mask_fwd(const T* ci, int64_t n, uint32_t k0, uint32_t k1, const uint32_t* kd, int draw_dtype,
                           int layout, T* mask) {
  if (kd) k0 = kd[0], k1 = kd[1];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float g = load_f<T>(ci, i);
    float u = draw_uniform(k0, k1, i, n, draw_dtype, layout);
    store_f<T>(mask, i, g + (1.f - g) * u);
  }
}

template <typename T>
__global__ void k_mask_bwd(const T* gm, int64_t n, uint32_t k0, uint32_t k1, const uint32_t* kd, int draw_dtype,
                           int layout, T* dci) {
  if (kd) k0 = kd[0], k1 = kd[1];
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float u = draw_uniform(k0, k1, i, n, draw_dtype, layout);
    store_f<T>(dci, i, load_f<T>(gm, i) * (1.f - u));
  }
}

// ---------------------------------------------------------------- gate MLP
// Thread mapping: one column (component) per lane, a chunk of rows per block, so the
// lane keeps its component's 49 gate parameters in registers and the row loop reads
// h coalesced across lanes.
static constexpr int GATE_COLS = 64;
// Rows per block chunk (also the bwd partial granularity): 64, or fewer (down to 4) when
// there are few components, so the grid has about 2048 blocks (C = 100 components over
// 2048 rows: 4-row chunks instead of 64 one-wave blocks each walking 64 rows).
static int64_t gate_rows(int64_t rows, int64_t C) {
  const int64_t r = cdiv(rows * cdiv(C, GATE_COLS), 2048);
  return r < 4 ? 4 : (r > 64 ? 64 : r);
}

template <typename T, bool PRECISE>
__global__ __launch_bounds__(GATE_COLS) void k_gate_fwd(const T* __restrict__ h, int64_t rows, int64_t C,
                                                        const float* __restrict__ w_in, const float* __restrict__ b_in,
                                                        const float* __restrict__ w_out,
                                                        const float* __restrict__ b_out, float* __restrict__ g_raw,
                                                        int64_t chunk_rows) {
  int64_t c = (int64_t)blockIdx.x * GATE_COLS + threadIdx.x;
  if (c >= C) return;
  float wi[16], bi[16], wo[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    wi[j] = w_in[c * 16 + j];
    bi[j] = b_in[c * 16 + j];
    wo[j] = w_out[c * 16 + j];
  }
  float bo = b_out[c];
  int64_t r0 = (int64_t)blockIdx.y * chunk_rows;
  int64_t r1 = r0 + chunk_rows < rows ? r0 + chunk_rows : rows;
  for (int64_t r = r0; r < r1; ++r) {
    float hv = load_f<T>(h, r * C + c);
    float g = bo;
#pragma unroll
    for (int j = 0; j < 16; ++j) g = fmaf(wo[j], gelu_only<PRECISE>(fmaf(wi[j], hv, bi[j])), g);
    g_raw[r * C + c] = g;
  }
}

template <typename T, bool PRECISE>
__global__ __launch_bounds__(GATE_COLS) void k_gate_bwd(const T* __restrict__ h, int64_t rows, int64_t C,
                                                        const float* __restrict__ w_in, const float* __restrict__ b_in,
                                                        const float* __restrict__ w_out,
                                                        const float* __restrict__ dg_raw, T* __restrict__ dh,
                                                        float* __restrict__ partial, int64_t chunk_rows) {
  int64_t c = (int64_t)blockIdx.x * GATE_COLS + threadIdx.x;
  if (c >= C) return;
  float wi[16], bi[16], wo[16], a_wi[16], a_bi[16], a_wo[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    wi[j] = w_in[c * 16 + j];
    bi[j] = b_in[c * 16 + j];
    wo[j] = w_out[c * 16 + j];
    a_wi[j] = a_bi[j] = a_wo[j] = 0.f;
  }
  float a_bo = 0.f;
  int64_t r0 = (int64_t)blockIdx.y * chunk_rows;
  int64_t r1 = r0 + chunk_rows < rows ? r0 + chunk_rows : rows;
  for (int64_t r = r0; r < r1; ++r) {
    float hv = load_f<T>(h, r * C + c);
    float dg = dg_raw[r * C + c];
    float dhv = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      GeluOut go = gelu_and_grad<PRECISE>(fmaf(wi[j], hv, bi[j]));
      float dz = dg * wo[j] * go.grad;
      dhv = fmaf(dz, wi[j], dhv);
      a_wi[j] = fmaf(dz, hv, a_wi[j]);
      a_bi[j] += dz;
      a_wo[j] = fmaf(dg, go.gelu, a_wo[j]);
    }
    a_bo += dg;
    store_f<T>(dh, r * C + c, dhv);
  }
  // partial layout: [chunk][49][C] (column-contiguous for a coalesced final reduce)
  float* p = partial + (int64_t)blockIdx.y * 49 * C;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    p[(int64_t)j * C + c] = a_wi[j];
    p[(int64_t)(16 + j) * C + c] = a_bi[j];
    p[(int64_t)(32 + j) * C + c] = a_wo[j];
  }
  p[(int64_t)48 * C + c] = a_bo;
}

// sum_{k < n} p[k * stride] added in k order; loads go out 16 at a time so a long chunk
// list is not one serial chain of load latencies.
__global__ void k_gate_bwd_reduce(const float* __restrict__ partial, int64_t chunks, int64_t C,
                                  float* __restrict__ dw_in, float* __restrict__ db_in, float* __restrict__ dw_out,
                                  float* __restrict__ db_out) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // over 49*C
  if (idx >= 49 * C) return;
  int64_t q = idx / C, c = idx % C;
  const float s = pd_ordered_sum(partial + idx, chunks, 49 * C);
  if (q < 16)
    dw_in[c * 16 + q] = s;
  else if (q < 32)
    db_in[c * 16 + (q - 16)] = s;
  else if (q < 48)
    dw_out[c * 16 + (q - 32)] = s;
  else
    db_out[c] = s;
}

// ---------------------------------------------------------------- imp-min
struct ImpParams {
  int kind;
  float p, eps, beta, world_size, gamma;
  int normalize_at_one;
  float ref_count, coeff_act, coeff_freq;
  FreqEma ema;  // the frequency term's running estimate (off: the batch estimate)
};

// The frequency the smooth-L0 penalty reads for column c with column sum s: the batch
// f = s / rows, or the debiased EMA estimate after this batch (stored when write).
__device__ inline float imp_penalty_frequency(float s, int64_t rows, int64_t c, const ImpParams& q, bool write) {
  const float f = s / (float)rows;
  return q.ema.on() ? ema_frequency(q.ema, c, f, write) : f;
}

__device__ inline float imp_psi(float v, const ImpParams& q) {
  if (q.kind == PD_IMPMIN_PNORM) {
    float b = v + q.eps;
    return q.p == 2.f ? b * b : (q.p == 1.f ? b : powf(b, q.p));
  }
  float g2 = q.gamma * q.gamma;
  float base = v * v / (v * v + g2);
  return q.normalize_at_one ? (1.f + g2) * base : base;
}

__device__ inline float imp_dpsi(float v, const ImpParams& q) {
  if (q.kind == PD_IMPMIN_PNORM) {
    float b = v + q.eps;
    return q.p == 2.f ? 2.f * b : (q.p == 1.f ? 1.f : q.p * powf(b, q.p - 1.f));
  }
  float g2 = q.gamma * q.gamma;
  float den = v * v + g2;
  float d = 2.f * v * g2 / (den * den);
  return q.normalize_at_one ? (1.f + g2) * d : d;
}

// Rows per partial chunk in column reductions: rows / 128 within [8, 256], so short
// batches still spread over ~128 row chunks (a thread's rows are a serial chain of loads).
static int64_t col_rows(int64_t rows) {
  const int64_t r = cdiv(rows, 128);
  return r < 8 ? 8 : (r > 256 ? 256 : r);
}

template <typename T>
__global__ void k_imp_colsum_partial(const T* __restrict__ ci, int64_t rows, int64_t C, ImpParams q,
                                     float* __restrict__ partial, int64_t chunk_rows) {
  int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  int64_t r0 = (int64_t)blockIdx.y * chunk_rows;
  int64_t r1 = r0 + chunk_rows < rows ? r0 + chunk_rows : rows;
  float s = 0.f;
  for (int64_t r = r0; r < r1; ++r) s += imp_psi(load_f<T>(ci, r * C + c), q);
  partial[(int64_t)blockIdx.y * C + c] = s;
}

__global__ void k_colsum_final(const float* __restrict__ partial, int64_t chunks, int64_t C, float* __restrict__ colsum) {
  int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  colsum[c] = pd_ordered_sum(partial + c, chunks, C);
}

// per-column slope dL/ds_c of the imp-min objective in terms of the column sum s_c (the
// frequency term's slope at the penalty's frequency: Phi'(f_hat) under the EMA estimate,
// pd/core/losses.py:449-456)
__device__ inline float imp_col_slope(float s, int64_t rows, int64_t c, const ImpParams& q) {
  float n = (float)rows;
  if (q.kind == PD_IMPMIN_PNORM) {
    float a = s * q.world_size;
    return q.coeff_act * (1.f / n * (1.f + q.beta * log2f(1.f + a)) +
                          q.beta * (s / n) * q.world_size / ((1.f + a) * 0.69314718055994531f));
  }
  float slope = q.coeff_act;
  if (q.ref_count > 0.f) {
    float af = q.ref_count * imp_penalty_frequency(s, rows, c, q, false);
    slope += q.coeff_freq * (log2f(1.f + af) + af / ((1.f + af) * 0.69314718055994531f));
  }
  return slope / n;
}

// out[0] = activity, out[1] = frequency penalty (at f_hat under the EMA estimate, which
// this kernel also stores), out[2] = the batch penalty when the EMA estimate is on.
__global__ void k_imp_scalar(const float* __restrict__ colsum, int64_t rows, int64_t C, ImpParams q,
                             float* __restrict__ out) {
  __shared__ double sa[16], sf[16], sb[16];
  double act = 0.0, freq = 0.0, fbat = 0.0;
  double n = (double)rows;
  for (int64_t c = threadIdx.x; c < C; c += blockDim.x) {
    double s = colsum[c], f = s / n;
    if (q.kind == PD_IMPMIN_PNORM) {
      act += f + q.beta * f * log2(1.0 + s * q.world_size);
    } else {
      act += f;
      if (q.ref_count > 0.f) {
        const double fe = q.ema.on() ? (double)imp_penalty_frequency(colsum[c], rows, c, q, true) : f;
        freq += fe * log2(1.0 + q.ref_count * fe);
        fbat += f * log2(1.0 + q.ref_count * f);
      }
    }
  }
  act = wave_sum_d(act);
  freq = wave_sum_d(freq);
  fbat = wave_sum_d(fbat);
  int w = threadIdx.x / 64, l = threadIdx.x % 64;
  if (l == 0) {
    sa[w] = act;
    sf[w] = freq;
    sb[w] = fbat;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double a = 0, f = 0, b = 0;
    for (int i = 0; i < (int)(blockDim.x / 64); ++i) {
      a += sa[i];
      f += sf[i];
      b += sb[i];
    }
    out[0] = (float)a;
    out[1] = (float)f;
    if (q.ema.on()) out[2] = (float)b;
  }
}

template <typename T>
__global__ void k_imp_grad(const T* __restrict__ ci, const float* __restrict__ colsum, int64_t rows, int64_t C,
                           ImpParams q, T* __restrict__ grad) {
  int64_t n = rows * C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t c = i % C;
    float v = load_f<T>(ci, i);
    store_f<T>(grad, i, imp_col_slope(colsum[c], rows, c, q) * imp_dpsi(v, q));
  }
}

// ---------------------------------------------------------------- MSE
template <typename T>
__global__ void k_mse_partial(const T* __restrict__ a, const T* __restrict__ b, int64_t n, float gscale,
                              T* __restrict__ grad, float* __restrict__ partial) {
  float s = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    float e = load_f<T>(a, i) - load_f<T>(b, i);
    s = fmaf(e, e, s);
    if (grad) store_f<T>(grad, i, gscale * e);
  }
  __shared__ float sw[EW_THREADS / 64];
  s = wave_sum(s);
  if (threadIdx.x % 64 == 0) sw[threadIdx.x / 64] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int i = 0; i < EW_THREADS / 64; ++i) t += sw[i];
    partial[blockIdx.x] = t;
  }
}

// One block: out[0] = scale * sum(partial[0..n)) accumulated in double, in index order.
__global__ void k_final_sum(const float* __restrict__ partial, int64_t n, double scale, float* __restrict__ out) {
  __shared__ double sw[16];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) s += partial[i];
  s = wave_sum_d(s);
  if (threadIdx.x % 64 == 0) sw[threadIdx.x / 64] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int i = 0; i < (int)(blockDim.x / 64); ++i) t += sw[i];
    out[0] = (float)(t * scale);
  }
}

// ---------------------------------------------------------------- KL
template <typename T>
__global__ __launch_bounds__(256) void k_kl_rows(const T* __restrict__ masked, const T* __restrict__ clean,
                                                 int64_t vocab, float gscale, T* __restrict__ grad,
                                                 float* __restrict__ row_kl) {
  const int64_t r = blockIdx.x;
  const T* m = masked + r * vocab;
  const T* c = clean + r * vocab;
  __shared__ float sm[8], sc[8];
  float mm = -INFINITY, mc = -INFINITY;
  for (int64_t i = threadIdx.x; i < vocab; i += blockDim.x) {
    mm = fmaxf(mm, load_f<T>(m, i));
    mc = fmaxf(mc, load_f<T>(c, i));
  }
  mm = wave_max(mm);
  mc = wave_max(mc);
  int w = threadIdx.x / 64;
  if (threadIdx.x % 64 == 0) {
    sm[w] = mm;
    sc[w] = mc;
  }
  __syncthreads();
  mm = sm[0];
  mc = sc[0];
  for (int i = 1; i < (int)(blockDim.x / 64); ++i) {
    mm = fmaxf(mm, sm[i]);
    mc = fmaxf(mc, sc[i]);
  }
  __syncthreads();
  float zm = 0.f, zc = 0.f;
  for (int64_t i = threadIdx.x; i < vocab; i += blockDim.x) {
    zm += __expf(load_f<T>(m, i) - mm);
    zc += __expf(load_f<T>(c, i) - mc);
  }
  zm = wave_sum(zm);
  zc = wave_sum(zc);
  if (threadIdx.x % 64 == 0) {
    sm[w] = zm;
    sc[w] = zc;
  }
  __syncthreads();
  zm = 0.f;
  zc = 0.f;
  for (int i = 0; i < (int)(blockDim.x / 64); ++i) {
    zm += sm[i];
    zc += sc[i];
  }
  __syncthreads();
  float lzm = mm + logf(zm), lzc = mc + logf(zc);
  float kl = 0.f;
  for (int64_t i = threadIdx.x; i < vocab; i += blockDim.x) {
    float lp = load_f<T>(c, i) - lzc;
    float lq = load_f<T>(m, i) - lzm;
    float p = __expf(lp);
    kl = fmaf(p, lp - lq, kl);
    if (grad) store_f<T>(grad + r * vocab, i, gscale * (__expf(lq) - p));
  }
  kl = wave_sum(kl);
  if (threadIdx.x % 64 == 0) sm[w] = kl;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x / 64); ++i) t += sm[i];
    row_kl[r] = t;
  }
}

}  // namespace pd

using namespace pd;

#define PD_DISPATCH_DTYPE(dtype, T, ...)                  \
  do {                                                    \
    if ((dtype) == PD_DTYPE_F32) {                        \
      typedef float T;                                    \
      __VA_ARGS__;                                        \
    } else if ((dtype) == PD_DTYPE_BF16) {                \
      typedef bf16_t T;                                   \
      __VA_ARGS__;                                        \
    } else {                                              \
      return fail(PD_EINVAL, "unsupported dtype");        \
    }                                                     \
  } while (0)

extern "C" {

const char* pd_last_error(void) { return g_last_error.c_str(); }
int pd_abi_version(void) { return 1; }

int pd_uniform(uint32_t k0, uint32_t k1, int64_t n, int draw_dtype, int layout, void* out, int out_dtype,
               void* stream) {
  if (n < 0 || !out) return fail(PD_EINVAL, "pd_uniform: bad n/out");
  if (draw_dtype != PD_DTYPE_F32 && draw_dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, "pd_uniform: draw dtype");
  if (layout == PD_LAYOUT_ORIGINAL && n > (int64_t)0xFFFFFFF0LL) return fail(PD_EUNSUPPORTED, "pd_uniform: size");
  if (n == 0) return PD_OK;
  hipStream_t s = (hipStream_t)stream;
  PD_DISPATCH_DTYPE(out_dtype, TO,
                    hipLaunchKernelGGL(k_uniform<TO>, dim3(ew_blocks(n)), dim3(EW_THREADS), 0, s, k0, k1, n,
                                       draw_dtype, layout, (TO*)out));
  return check_launch("pd_uniform");
}

int pd_squash_fwd(const void* pre, int dtype, int64_t n, void* lower, void* upper, void* stream) {
  if (n < 0 || !pre) return fail(PD_EINVAL, "pd_squash_fwd: bad args");
  if (n == 0) return PD_OK;
  PD_DISPATCH_DTYPE(dtype, T,
                    hipLaunchKernelGGL(k_squash_fwd<T>, dim3(ew_blocks(n)), dim3(EW_THREADS), 0,
                                       (hipStream_t)stream, (const T*)pre, n, (T*)lower, (T*)upper));
  return check_launch("pd_squash_fwd");
}

int pd_squash_bwd(const void* pre, const void* gl, const void* gu, int dtype, int64_t n, void* d, void* stream) {
  if (n < 0 || !pre || !d) return fail(PD_EINVAL, "pd_squash_bwd: bad args");
  if (n == 0) return PD_OK;
  PD_DISPATCH_DTYPE(dtype, T,
                    hipLaunchKernelGGL(k_squash_bwd<T>, dim3(ew_blocks(n)), dim3(EW_THREADS), 0,
                                       (hipStream_t)stream, (const T*)pre, (const T*)gl, (const T*)gu, n, (T*)d));
  return check_launch("pd_squash_bwd");
}

static int mask_fwd(const void* ci, int dtype, int64_t n, uint32_t k0, uint32_t k1, const uint32_t* kd,
                    int draw_dtype, int layout, void* mask, void* stream, const char* who) {
  if (n < 0 || !ci || !mask) return fail(PD_EINVAL, std::string(who) + ": bad args");
  if (n == 0) return PD_OK;
  PD_DISPATCH_DTYPE(dtype, T,
                    hipLaunchKernelGGL(k_mask_fwd<T>, dim3(ew_blocks(n)), dim3(EW_THREADS), 0, (hipStream_t)stream,
                                       (const T*)ci, n, k0, k1, kd, draw_dtype, layout, (T*)mask));
  return check_launch(who);
}

static int mask_bwd(const void* gm, int dtype, int64_t n, uint32_t k0, uint32_t k1, const uint32_t* kd,
                    int draw_dtype, int layout, void* dci, void* stream, const char* who) {
  if (n < 0 || !gm || !dci) return fail(PD_EINVAL, std::string(who) + ": bad args");
  if (n == 0) return PD_OK;
  PD_DISPATCH_DTYPE(dtype, T,
                    hipLaunchKernelGGL(k_mask_bwd<T>, dim3(ew_blocks(n)), dim3(EW_THREADS), 0, (hipStream_t)stream,
                                       (const T*)gm, n, k0, k1, kd, draw_dtype, layout, (T*)dci));
  return check_launch(who);
}

int pd_component_mask_fwd(const void* ci, int dtype, int64_t n, uint32_t k0, uint32_t k1, int draw_dtype, int layout,
                          void* mask, void* stream) {
  return mask_fwd(ci, dtype, n, k0, k1, nullptr, draw_dtype, layout, mask, stream, "pd_component_mask_fwd");
}

int pd_component_mask_bwd(const void* gm, int dtype, int64_t n, uint32_t k0, uint32_t k1, int draw_dtype, int layout,
                          void* dci, void* stream) {
  return mask_bwd(gm, dtype, n, k0, k1, nullptr, draw_dtype, layout, dci, stream, "pd_component_mask_bwd");
}

int pd_component_mask_fwd_dkey(const void* ci, int dtype, int64_t n, const uint32_t* key, int draw_dtype, int layout,
                               void* mask, void* stream) {
  if (!key) return fail(PD_EINVAL, "pd_component_mask_fwd_dkey: null key");
  return mask_fwd(ci, dtype, n, 0, 0, key, draw_dtype, layout, mask, stream, "pd_component_mask_fwd_dkey");
}

int pd_component_mask_bwd_dkey(const void* gm, int dtype, int64_t n, const uint32_t* key, int draw_dtype, int layout,
                               void* dci, void* stream) {
  if (!key) return fail(PD_EINVAL, "pd_component_mask_bwd_dkey: null key");
  return mask_bwd(gm, dtype, n, 0, 0, key, draw_dtype, layout, dci, stream, "pd_component_mask_bwd_dkey");
}

int pd_gate_fwd(const void* h, int dtype, int64_t rows, int64_t C, int H, const float* w_in, const float* b_in,
                const float* w_out, const float* b_out, int precise, float* g_raw, void* stream) {
  if (H != 16) return fail(PD_EUNSUPPORTED, "pd_gate_fwd: gate hidden width must be 16");
  if (rows < 0 || C < 0 || !h || !g_raw) return fail(PD_EINVAL, "pd_gate_fwd: bad args");
  if (rows == 0 || C == 0) return PD_OK;
  const int64_t cr = gate_rows(rows, C);
  if (cdiv(rows, cr) > 65535) return fail(PD_EUNSUPPORTED, "pd_gate_fwd: too many rows");
  dim3 grid((unsigned)cdiv(C, GATE_COLS), (unsigned)cdiv(rows, cr));
  hipStream_t s = (hipStream_t)stream;
  PD_DISPATCH_DTYPE(dtype, T, {
    if (precise)
      hipLaunchKernelGGL((k_gate_fwd<T, true>), grid, dim3(GATE_COLS), 0, s, (const T*)h, rows, C, w_in, b_in, w_out,
                         b_out, g_raw, cr);
    else
      hipLaunchKernelGGL((k_gate_fwd<T, false>), grid, dim3(GATE_COLS), 0, s, (const T*)h, rows, C, w_in, b_in,
                         w_out, b_out, g_raw, cr);
  });
  return check_launch("pd_gate_fwd");
}

size_t pd_gate_bwd_workspace_size(int64_t rows, int64_t C, int H) {
  (void)H;
  return rows > 0 && C > 0 ? (size_t)cdiv(rows, gate_rows(rows, C)) * 49 * (size_t)C * sizeof(float) : 0;
}

int pd_gate_bwd(const void* h, int dtype, int64_t rows, int64_t C, int H, const float* w_in, const float* b_in,
                const float* w_out, const float* b_out, const float* dg_raw, int precise, void* dh, float* dw_in,
                float* db_in, float* dw_out, float* db_out, void* workspace, size_t workspace_bytes, void* stream) {
  (void)b_out;
  if (H != 16) return fail(PD_EUNSUPPORTED, "pd_gate_bwd: gate hidden width must be 16");
  if (rows <= 0 || C <= 0 || !h || !dg_raw || !dh) return fail(PD_EINVAL, "pd_gate_bwd: bad args");
  if (workspace_bytes < pd_gate_bwd_workspace_size(rows, C, H) || !workspace)
    return fail(PD_EWORKSPACE, "pd_gate_bwd: workspace too small");
  const int64_t cr = gate_rows(rows, C), chunks = cdiv(rows, cr);
  if (chunks > 65535) return fail(PD_EUNSUPPORTED, "pd_gate_bwd: too many rows");
  dim3 grid((unsigned)cdiv(C, GATE_COLS), (unsigned)chunks);
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)workspace;
  PD_DISPATCH_DTYPE(dtype, T, {
    if (precise)
      hipLaunchKernelGGL((k_gate_bwd<T, true>), grid, dim3(GATE_COLS), 0, s, (const T*)h, rows, C, w_in, b_in, w_out,
                         dg_raw, (T*)dh, part, cr);
    else
      hipLaunchKernelGGL((k_gate_bwd<T, false>), grid, dim3(GATE_COLS), 0, s, (const T*)h, rows, C, w_in, b_in,
                         w_out, dg_raw, (T*)dh, part, cr);
  });
  int rc = check_launch("pd_gate_bwd");
  if (rc) return rc;
  hipLaunchKernelGGL(k_gate_bwd_reduce, dim3((unsigned)cdiv(49 * C, 256)), dim3(256), 0, s, part, chunks, C, dw_in,
                     db_in, dw_out, db_out);
  return check_launch("pd_gate_bwd reduce");
}

size_t pd_impmin_workspace_size(int64_t rows, int64_t C) {
  return rows > 0 && C > 0 ? ((size_t)cdiv(rows, col_rows(rows)) + 1) * (size_t)C * sizeof(float) : 0;
}

int pd_impmin(const void* ci, int dtype, int64_t rows, int64_t C, int kind, float p, float eps, float beta,
              float world_size, float gamma, int normalize_at_one, float ref_count, const float* freq_ema_in,
              float* freq_ema_out, float ema_count, float ema_halflife, float coeff_act, float coeff_freq,
              float* out, void* grad, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows <= 0 || C <= 0 || !ci || !out) return fail(PD_EINVAL, "pd_impmin: bad args");
  if (kind != PD_IMPMIN_PNORM && kind != PD_IMPMIN_SMOOTH_L0) return fail(PD_EINVAL, "pd_impmin: kind");
  if (!workspace || workspace_bytes < pd_impmin_workspace_size(rows, C))
    return fail(PD_EWORKSPACE, "pd_impmin: workspace too small");
  ImpParams q{kind, p, eps, beta, world_size, gamma, normalize_at_one, ref_count, coeff_act, coeff_freq, FreqEma{}};
  if (int e = make_freq_ema("pd_impmin", freq_ema_in, freq_ema_out, ema_count, ema_halflife, q.ema)) return e;
  if (q.ema.on() && !(kind == PD_IMPMIN_SMOOTH_L0 && ref_count > 0.f))
    return fail(PD_EINVAL, "pd_impmin: the EMA estimate needs the smooth-L0 frequency term (ref_count > 0)");
  const int64_t cr = col_rows(rows), chunks = cdiv(rows, cr);
  if (chunks > 65535) return fail(PD_EUNSUPPORTED, "pd_impmin: too many rows");
  float* part = (float*)workspace;
  float* colsum = part + chunks * C;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)cdiv(C, 256), (unsigned)chunks);
  PD_DISPATCH_DTYPE(dtype, T,
                    hipLaunchKernelGGL(k_imp_colsum_partial<T>, grid, dim3(256), 0, s, (const T*)ci, rows, C, q, part, cr));
  hipLaunchKernelGGL(k_colsum_final, dim3((unsigned)cdiv(C, 256)), dim3(256), 0, s, part, chunks, C, colsum);
  if (grad) {  // before the scalar pass, which stores the new estimate (possibly over the old)
    PD_DISPATCH_DTYPE(dtype, T,
                      hipLaunchKernelGGL(k_imp_grad<T>, dim3(ew_blocks(rows * C)), dim3(EW_THREADS), 0, s,
                                         (const T*)ci, colsum, rows, C, q, (T*)grad));
  }
  hipLaunchKernelGGL(k_imp_scalar, dim3(1), dim3(1024), 0, s, colsum, rows, C, q, out);
  return check_launch("pd_impmin");
}

size_t pd_mse_workspace_size(int64_t n) {
  (void)n;
  return RED_BLOCKS * sizeof(float);
}

int pd_mse(const void* a, const void* b, int dtype, int64_t n, float coeff, float* out, void* grad_a, void* workspace,
           size_t workspace_bytes, void* stream) {
  if (n <= 0 || !a || !b || !out) return fail(PD_EINVAL, "pd_mse: bad args");
  if (!workspace || workspace_bytes < pd_mse_workspace_size(n)) return fail(PD_EWORKSPACE, "pd_mse: workspace");
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)workspace;
  int blocks = (int)std::min<int64_t>(RED_BLOCKS, cdiv(n, EW_THREADS));
  float gscale = coeff * 2.f / (float)n;
  PD_DISPATCH_DTYPE(dtype, T,
                    hipLaunchKernelGGL(k_mse_partial<T>, dim3(blocks), dim3(EW_THREADS), 0, s, (const T*)a,
                                       (const T*)b, n, gscale, (T*)grad_a, part));
  hipLaunchKernelGGL(k_final_sum, dim3(1), dim3(1024), 0, s, part, (int64_t)blocks, 1.0 / (double)n, out);
  return check_launch("pd_mse");
}

size_t pd_kl_workspace_size(int64_t rows) { return (size_t)rows * sizeof(float); }

int pd_kl(const void* masked, const void* clean, int dtype, int64_t rows, int64_t vocab, float coeff, float* out,
          void* grad, void* workspace, size_t workspace_bytes, void* stream) {
  if (rows <= 0 || vocab <= 0 || !masked || !clean || !out) return fail(PD_EINVAL, "pd_kl: bad args");
  if (!workspace || workspace_bytes < pd_kl_workspace_size(rows)) return fail(PD_EWORKSPACE, "pd_kl: workspace");
  if (rows > 0x7FFFFFFF) return fail(PD_EUNSUPPORTED, "pd_kl: rows");
  hipStream_t s = (hipStream_t)stream;
  float* row_kl = (float*)workspace;
  float gscale = coeff / (float)rows;
  PD_DISPATCH_DTYPE(dtype, T,
                    hipLaunchKernelGGL(k_kl_rows<T>, dim3((unsigned)rows), dim3(256), 0, s, (const T*)masked,
                                       (const T*)clean, vocab, gscale, (T*)grad, row_kl));
  hipLaunchKernelGGL(k_final_sum, dim3(1), dim3(1024), 0, s, row_kl, rows, 1.0 / (double)rows, out);
  return check_launch("pd_kl");
}

}  // extern "C"
