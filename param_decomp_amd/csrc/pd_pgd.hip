// Adversarial (PGD) sources on gfx950: source masks, their pullback onto the sources,
// and the projected source ascents.
//
//   pd_source_mask_fwd   m = ci + (1 - ci) s           pd/core/source_mask.py:56-63,
//                                                       pd/core/masking.py:260-272
//   pd_source_mask_bwd   d_s = sum over the rows a source covers of g (1 - ci),
//                        d_ci = g (1 - s)
//   pd_source_ascend     SGD / momentum SGD / Adam projected ascents and the fresh-PGD
//                        sign ascent, clipped to [0, 1]   pd/core/adversary.py:392-470,
//                                                         pd/core/train.py:788-800
//                        uint16 fixed-point storage u / 65535 with unbiased stochastic
//                        rounding on store                pd/core/adversary.py:150-214
//
// A source row covers `rows_per_source` consecutive rows of the [rows, C] CI: the
// reference's source shapes over (batch, positions) are `bsc` (1 row each), `bc` (the
// positions of a sample) and `c` (every row).
#include <algorithm>

#include "pd_common.hpp"

namespace pd {

static constexpr int SRC_ROWS = 64;  // rows per block of the mask passes

__device__ inline float bfr16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

template <int SD>
__device__ inline float source_view(const void* src, int64_t i) {
  if (SD == PD_DTYPE_F32) return ((const float*)src)[i];
  if (SD == PD_DTYPE_BF16) return bf16_to_f32(((const bf16_t*)src)[i]);
  return (float)((const uint16_t*)src)[i] / 65535.0f;  // pd/core/adversary.py:171-184
}

template <typename T>
__device__ inline float as_compute(float v);
template <>
__device__ inline float as_compute<float>(float v) {
  return v;
}
template <>
__device__ inline float as_compute<bf16_t>(float v) {
  return bf16_to_f32(f32_to_bf16(v));
}

// One lane per column, SRC_ROWS rows per block; the source value is re-read only when a
// row enters a new source.
template <typename T, int SD>
__global__ __launch_bounds__(256) void k_source_mask_fwd(const T* __restrict__ ci, int64_t rows, int64_t C,
                                                         const void* __restrict__ src, int64_t rows_per_source,
                                                         T* __restrict__ mask) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  const int64_t r0 = (int64_t)blockIdx.y * SRC_ROWS, r1 = std::min<int64_t>(r0 + SRC_ROWS, rows);
  int64_t cur = -1;
  float s = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t sr = r / rows_per_source;
    if (sr != cur) {
      cur = sr;
      s = as_compute<T>(source_view<SD>(src, sr * C + c));
    }
    const float g = load_f<T>(ci, r * C + c);
    store_f<T>(mask, r * C + c, g + (1.f - g) * s);
  }
}

// Partial pullback: block (column chunk, p) covers rows [p_lo, p_hi) of one source, p =
// source * chunks + chunk; part[p][c] = sum of g (1 - ci) over those rows in row order.
// With one row per source the partial is the gradient itself (chunks == 1).
template <typename T, int SD>
__global__ __launch_bounds__(256) void k_source_mask_bwd(const T* __restrict__ gm, const T* __restrict__ ci,
                                                         int64_t rows, int64_t C, const void* __restrict__ src,
                                                         int64_t rows_per_source, int64_t chunks,
                                                         float* __restrict__ part, T* __restrict__ d_ci) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  const int64_t p = blockIdx.y, sr = p / chunks, ch = p % chunks;
  const int64_t s_lo = sr * rows_per_source;
  const int64_t r0 = s_lo + ch * SRC_ROWS;
  const int64_t r1 = std::min<int64_t>(std::min<int64_t>(r0 + SRC_ROWS, s_lo + rows_per_source), rows);
  const float s = d_ci ? as_compute<T>(source_view<SD>(src, sr * C + c)) : 0.f;
  float acc = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const float g = load_f<T>(gm, r * C + c);
    const float v = load_f<T>(ci, r * C + c);
    acc += g * (1.f - v);
    if (d_ci) store_f<T>(d_ci, r * C + c, g * (1.f - s));
  }
  part[p * C + c] = acc;
}

// d_src[sr][c] = sum over chunks of part[sr * chunks + k][c], k in order.
__global__ void k_source_grad_reduce(const float* __restrict__ part, int64_t n_src, int64_t chunks, int64_t C,
                                     float* __restrict__ d_src) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_src * C) return;
  const int64_t sr = i / C, c = i % C;
  d_src[i] = pd_ordered_sum(part + sr * chunks * C + c, chunks, C);
}

// ---- vector forms (C % 8 == 0, 16-byte aligned operands): 8 columns per lane.
template <typename T>
struct Vec8;
template <>
struct Vec8<float> {
  __device__ static void load(const float* p, float (&v)[8]) {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
  }
  __device__ static void store(float* p, const float (&v)[8]) {
    *(float4*)p = make_float4(v[0], v[1], v[2], v[3]);
    *(float4*)(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
};
template <>
struct Vec8<bf16_t> {
  __device__ static void load(const bf16_t* p, float (&v)[8]) {
    const uint4 q = *(const uint4*)p;
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_to_f32((bf16_t)(u[i] & 0xFFFF));
      v[2 * i + 1] = bf16_to_f32((bf16_t)(u[i] >> 16));
    }
  }
  __device__ static void store(bf16_t* p, const float (&v)[8]) {
    *(uint4*)p = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                            pack_bf16x2(v[6], v[7]));
  }
};

template <int SD>
__device__ inline void source_view8(const void* src, int64_t i, float (&v)[8]) {
  if (SD == PD_DTYPE_F32) {
    Vec8<float>::load((const float*)src + i, v);
  } else if (SD == PD_DTYPE_BF16) {
    Vec8<bf16_t>::load((const bf16_t*)src + i, v);
  } else {
    const uint4 q = *(const uint4*)((const uint16_t*)src + i);
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = (float)(u[k] & 0xFFFF) / 65535.0f;
      v[2 * k + 1] = (float)(u[k] >> 16) / 65535.0f;
    }
  }
}

// Rows per block `rpb` (<= SRC_ROWS) is chosen by the host so the grid has enough blocks.
template <typename T, int SD>
__global__ __launch_bounds__(256) void k_source_mask_fwd8(const T* __restrict__ ci, int64_t rows, int64_t C,
                                                          const void* __restrict__ src, int64_t rows_per_source,
                                                          int64_t rpb, T* __restrict__ mask) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= C) return;
  const int64_t r0 = (int64_t)blockIdx.y * rpb, r1 = std::min<int64_t>(r0 + rpb, rows);
  int64_t cur = -1;
  float s[8];
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t sr = rows_per_source == 1 ? r : r / rows_per_source;
    if (sr != cur) {
      cur = sr;
      source_view8<SD>(src, sr * C + c, s);
#pragma unroll
      for (int e = 0; e < 8; ++e) s[e] = as_compute<T>(s[e]);
    }
    float g[8], m[8];
    Vec8<T>::load(ci + r * C + c, g);
#pragma unroll
    for (int e = 0; e < 8; ++e) m[e] = g[e] + (1.f - g[e]) * s[e];
    Vec8<T>::store(mask + r * C + c, m);
  }
}

template <typename T, int SD>
__global__ __launch_bounds__(256) void k_source_mask_bwd8(const T* __restrict__ gm, const T* __restrict__ ci,
                                                          int64_t rows, int64_t C, const void* __restrict__ src,
                                                          int64_t rows_per_source, int64_t chunks,
                                                          float* __restrict__ part, T* __restrict__ d_ci) {
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= C) return;
  const int64_t p = blockIdx.y, sr = p / chunks, ch = p % chunks;
  const int64_t s_lo = sr * rows_per_source;
  const int64_t r0 = s_lo + ch * SRC_ROWS;
  const int64_t r1 = std::min<int64_t>(std::min<int64_t>(r0 + SRC_ROWS, s_lo + rows_per_source), rows);
  float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (d_ci) {
    source_view8<SD>(src, sr * C + c, s);
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = as_compute<T>(s[e]);
  }
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t r = r0; r < r1; ++r) {
    float g[8], v[8];
    Vec8<T>::load(gm + r * C + c, g);
    Vec8<T>::load(ci + r * C + c, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += g[e] * (1.f - v[e]);
    if (d_ci) {
      float d[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] = g[e] * (1.f - s[e]);
      Vec8<T>::store(d_ci + r * C + c, d);
    }
  }
  Vec8<float>::store(part + p * C + c, acc);
}

static bool al16p(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ---------------------------------------------------------------- ascents
struct AscendArgs {
  int opt;
  int64_t n;
  void* src;
  const float* grad;
  void* sa;  // adam m (storage dtype) or momentum velocity (fp32 for fp32 storage, else bf16)
  void* sb;  // adam v (storage dtype)
  // beta and its complement as the reference's arithmetic sees them: rounded to the
  // moment dtype (fp32, or bf16 for bf16 moments), (1 - beta) formed in double first;
  // the bias corrections 1 - beta^step are fp32 arithmetic on fp32(beta)
  float lr, beta1, omb1, beta2, omb2, eps, momentum, bc1, bc2;
  uint32_t k0, k1;
  int layout;
};

__device__ inline float clip01(float v) { return fminf(fmaxf(v, 0.f), 1.f); }
__device__ inline float sgnf(float g) { return g > 0.f ? 1.f : (g < 0.f ? -1.f : 0.f); }

// One element: the float view of the source, the optimizer's update, the projection, and
// the store back into the storage representation.
template <int SD>
__global__ void k_source_ascend(AscendArgs a) {
  constexpr bool B16 = SD == PD_DTYPE_BF16;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n; i += (int64_t)gridDim.x * blockDim.x) {
    const float val = source_view<SD>(a.src, i);
    // the gradient is taken w.r.t. the float view: bf16 for bf16 storage
    const float g = B16 ? bfr16(a.grad[i]) : a.grad[i];
    float upd;
    if (a.opt == PD_PGD_SGD) {
      upd = a.lr * g;
    } else if (a.opt == PD_PGD_MOMENTUM) {
      // v = momentum v + g in fp32, rounded once to the velocity dtype
      float v;
      if (SD == PD_DTYPE_F32) {
        v = a.momentum * ((float*)a.sa)[i] + g;
        ((float*)a.sa)[i] = v;
      } else {
        v = bfr16(a.momentum * bf16_to_f32(((bf16_t*)a.sa)[i]) + g);
        ((bf16_t*)a.sa)[i] = f32_to_bf16(v);
      }
      upd = a.lr * v;
    } else if (a.opt == PD_PGD_ADAM) {
      // moments at the storage dtype; every bf16 operation rounds
      float m, v;
      if (B16) {
        m = bfr16(bfr16(a.beta1 * bf16_to_f32(((bf16_t*)a.sa)[i])) + bfr16(a.omb1 * g));
        v = bfr16(bfr16(a.beta2 * bf16_to_f32(((bf16_t*)a.sb)[i])) + bfr16(bfr16(a.omb2 * g) * g));
        ((bf16_t*)a.sa)[i] = f32_to_bf16(m);
        ((bf16_t*)a.sb)[i] = f32_to_bf16(v);
      } else {
        m = a.beta1 * ((float*)a.sa)[i] + a.omb1 * g;
        v = a.beta2 * ((float*)a.sb)[i] + a.omb2 * g * g;
        ((float*)a.sa)[i] = m;
        ((float*)a.sb)[i] = v;
      }
      upd = a.lr * (m / a.bc1) / (sqrtf(v / a.bc2) + a.eps);
    } else {  // PD_PGD_SIGN
      upd = a.lr * sgnf(g);
    }
    if (SD == PD_DTYPE_U16) {
      // pd/core/adversary.py:186-194: floor plus a Bernoulli(frac) carry, one uniform per
      // element of the leaf under the caller's key
      const float scaled = clip01(val + upd) * 65535.0f;
      const float low = floorf(scaled);
      const float u = draw_uniform(a.k0, a.k1, i, a.n, PD_DTYPE_F32, a.layout);
      const float q = fminf(fmaxf(low + (u < scaled - low ? 1.f : 0.f), 0.f), 65535.0f);
      ((uint16_t*)a.src)[i] = (uint16_t)q;
    } else if (B16) {
      ((bf16_t*)a.src)[i] = f32_to_bf16(clip01(bfr16(val + bfr16(upd))));
    } else {
      ((float*)a.src)[i] = clip01(val + upd);
    }
  }
}

}  // namespace pd

using namespace pd;

#define PD_SRC_DISPATCH(SD_VAR, ...)                                   \
  do {                                                                 \
    if ((SD_VAR) == PD_DTYPE_F32) {                                    \
      constexpr int SDC = PD_DTYPE_F32;                                \
      __VA_ARGS__;                                                     \
    } else if ((SD_VAR) == PD_DTYPE_BF16) {                            \
      constexpr int SDC = PD_DTYPE_BF16;                               \
      __VA_ARGS__;                                                     \
    } else {                                                           \
      constexpr int SDC = PD_DTYPE_U16;                                \
      __VA_ARGS__;                                                     \
    }                                                                  \
  } while (0)

extern "C" {

static int src_args_ok(const char* what, int dtype, int src_dtype, int64_t rows, int64_t C, int64_t rows_per_source) {
  if (dtype != PD_DTYPE_F32 && dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, std::string(what) + ": ci dtype");
  if (src_dtype != PD_DTYPE_F32 && src_dtype != PD_DTYPE_BF16 && src_dtype != PD_DTYPE_U16)
    return fail(PD_EINVAL, std::string(what) + ": source dtype");
  if (rows <= 0 || C <= 0 || rows_per_source <= 0 || rows % rows_per_source)
    return fail(PD_EINVAL, std::string(what) + ": rows must be a positive multiple of rows_per_source");
  if (cdiv(rows, SRC_ROWS) > 65535 || cdiv(C, 256) > 65535) return fail(PD_EUNSUPPORTED, std::string(what) + ": too large");
  return PD_OK;
}

int pd_source_mask_fwd(const void* ci, int dtype, int64_t rows, int64_t C, const void* sources, int src_dtype,
                       int64_t rows_per_source, void* mask, void* stream) {
  int rc;
  if ((rc = src_args_ok("pd_source_mask_fwd", dtype, src_dtype, rows, C, rows_per_source))) return rc;
  if (!ci || !sources || !mask) return fail(PD_EINVAL, "pd_source_mask_fwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (C % 8 == 0 && al16p(ci) && al16p(sources) && al16p(mask)) {
    // about 4096 blocks: fewer rows per block for narrow C, up to SRC_ROWS
    const int64_t col_blocks = cdiv(C / 8, 256);
    const int64_t rpb = std::max<int64_t>(std::min<int64_t>(rows * col_blocks / 4096, SRC_ROWS), 1);
    if (cdiv(rows, rpb) > 65535) return fail(PD_EUNSUPPORTED, "pd_source_mask_fwd: too many rows");
    const dim3 grid((unsigned)col_blocks, (unsigned)cdiv(rows, rpb));
    PD_SRC_DISPATCH(src_dtype, {
      if (dtype == PD_DTYPE_F32)
        hipLaunchKernelGGL((k_source_mask_fwd8<float, SDC>), grid, dim3(256), 0, s, (const float*)ci, rows, C,
                           sources, rows_per_source, rpb, (float*)mask);
      else
        hipLaunchKernelGGL((k_source_mask_fwd8<bf16_t, SDC>), grid, dim3(256), 0, s, (const bf16_t*)ci, rows, C,
                           sources, rows_per_source, rpb, (bf16_t*)mask);
    });
    return check_launch("pd_source_mask_fwd");
  }
  const dim3 grid((unsigned)cdiv(C, 256), (unsigned)cdiv(rows, SRC_ROWS));
  PD_SRC_DISPATCH(src_dtype, {
    if (dtype == PD_DTYPE_F32)
      hipLaunchKernelGGL((k_source_mask_fwd<float, SDC>), grid, dim3(256), 0, s, (const float*)ci, rows, C, sources,
                         rows_per_source, (float*)mask);
    else
      hipLaunchKernelGGL((k_source_mask_fwd<bf16_t, SDC>), grid, dim3(256), 0, s, (const bf16_t*)ci, rows, C,
                         sources, rows_per_source, (bf16_t*)mask);
  });
  return check_launch("pd_source_mask_fwd");
}

size_t pd_source_mask_bwd_workspace_size(int64_t rows, int64_t C, int64_t rows_per_source) {
  if (rows <= 0 || C <= 0 || rows_per_source <= 0) return 0;
  return 4 * (size_t)(rows / rows_per_source) * cdiv(rows_per_source, SRC_ROWS) * C;
}

int pd_source_mask_bwd(const void* g_mask, const void* ci, int dtype, int64_t rows, int64_t C, const void* sources,
                       int src_dtype, int64_t rows_per_source, float* d_sources, void* d_ci, void* workspace,
                       size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = src_args_ok("pd_source_mask_bwd", dtype, src_dtype, rows, C, rows_per_source))) return rc;
  if (!g_mask || !ci || !sources || !d_sources) return fail(PD_EINVAL, "pd_source_mask_bwd: null pointer");
  const int64_t n_src = rows / rows_per_source, chunks = cdiv(rows_per_source, SRC_ROWS);
  if (n_src * chunks > 65535) return fail(PD_EUNSUPPORTED, "pd_source_mask_bwd: too many rows");
  float* part = chunks == 1 ? d_sources : (float*)workspace;
  if (chunks > 1 && (!workspace || workspace_bytes < pd_source_mask_bwd_workspace_size(rows, C, rows_per_source)))
    return fail(PD_EWORKSPACE, "pd_source_mask_bwd: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  if (C % 8 == 0 && al16p(g_mask) && al16p(ci) && al16p(sources) && al16p(part) && al16p(d_ci)) {
    const dim3 grid((unsigned)cdiv(C / 8, 256), (unsigned)(n_src * chunks));
    PD_SRC_DISPATCH(src_dtype, {
      if (dtype == PD_DTYPE_F32)
        hipLaunchKernelGGL((k_source_mask_bwd8<float, SDC>), grid, dim3(256), 0, s, (const float*)g_mask,
                           (const float*)ci, rows, C, sources, rows_per_source, chunks, part, (float*)d_ci);
      else
        hipLaunchKernelGGL((k_source_mask_bwd8<bf16_t, SDC>), grid, dim3(256), 0, s, (const bf16_t*)g_mask,
                           (const bf16_t*)ci, rows, C, sources, rows_per_source, chunks, part, (bf16_t*)d_ci);
    });
  } else {
    const dim3 grid((unsigned)cdiv(C, 256), (unsigned)(n_src * chunks));
    PD_SRC_DISPATCH(src_dtype, {
      if (dtype == PD_DTYPE_F32)
        hipLaunchKernelGGL((k_source_mask_bwd<float, SDC>), grid, dim3(256), 0, s, (const float*)g_mask,
                           (const float*)ci, rows, C, sources, rows_per_source, chunks, part, (float*)d_ci);
      else
        hipLaunchKernelGGL((k_source_mask_bwd<bf16_t, SDC>), grid, dim3(256), 0, s, (const bf16_t*)g_mask,
                           (const bf16_t*)ci, rows, C, sources, rows_per_source, chunks, part, (bf16_t*)d_ci);
    });
  }
  if (chunks > 1)
    hipLaunchKernelGGL(k_source_grad_reduce, dim3((unsigned)cdiv(n_src * C, 256)), dim3(256), 0, s, part, n_src, chunks,
                       C, d_sources);
  return check_launch("pd_source_mask_bwd");
}

int pd_source_ascend(int opt, int src_dtype, int64_t n, void* sources, const float* grad, void* state_a,
                     void* state_b, float step_count, float lr, double beta1, double beta2, float eps, float momentum,
                     uint32_t k0, uint32_t k1, int layout, void* stream) {
  if (n <= 0 || !sources || !grad) return fail(PD_EINVAL, "pd_source_ascend: bad args");
  if (src_dtype != PD_DTYPE_F32 && src_dtype != PD_DTYPE_BF16 && src_dtype != PD_DTYPE_U16)
    return fail(PD_EINVAL, "pd_source_ascend: source dtype");
  if (opt == PD_PGD_ADAM && src_dtype == PD_DTYPE_U16)
    return fail(PD_EINVAL, "pd_source_ascend: adam keeps its moments at the source dtype; uint16 storage pairs with "
                           "sgd or momentum_sgd");
  if (opt == PD_PGD_SIGN && src_dtype != PD_DTYPE_F32)
    return fail(PD_EINVAL, "pd_source_ascend: fresh-PGD sign ascents run on fp32 sources");
  if (opt == PD_PGD_MOMENTUM && !state_a) return fail(PD_EINVAL, "pd_source_ascend: momentum needs a velocity");
  if (opt == PD_PGD_ADAM && (!state_a || !state_b || step_count < 1.f))
    return fail(PD_EINVAL, "pd_source_ascend: adam needs m, v and a step count >= 1");
  if (opt < PD_PGD_SGD || opt > PD_PGD_SIGN) return fail(PD_EINVAL, "pd_source_ascend: optimizer");
  const float b1 = (float)beta1, b2 = (float)beta2;
  // beta * moment and (1 - beta) * g take the Python-float coefficients at the moment
  // dtype (JAX's weak typing, pd/core/adversary.py:475-480): fp32 for fp32 moments,
  // bf16-rounded for bf16 moments (bf16(0.999) = 1, so v does not decay there). The bias
  // corrections 1 - beta^step are fp32 on fp32(beta) in both.
  const bool b16m = src_dtype == PD_DTYPE_BF16;
  auto coef = [&](double c) { return b16m ? bf16_to_f32(f32_to_bf16((float)c)) : (float)c; };
  AscendArgs a{opt,      n,        sources,  grad,     state_a,
               state_b,  lr,       coef(beta1),        coef(1.0 - beta1),
               coef(beta2),        coef(1.0 - beta2),  eps,    momentum,
               1.f - powf(b1, step_count),     1.f - powf(b2, step_count),
               k0,       k1,       layout};
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(n, 256), 16384);
  hipStream_t s = (hipStream_t)stream;
  PD_SRC_DISPATCH(src_dtype, hipLaunchKernelGGL((k_source_ascend<SDC>), dim3(blocks), dim3(256), 0, s, a));
  return check_launch("pd_source_ascend");
}

}  // extern "C"
