// Shared device helpers for the gfx950 masked-component kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <mutex>
#include <string>

#include "../../include/pd_mi355x.h"

namespace pd {

// ---------------------------------------------------------------- error state
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// A helper stream of the current device for running an independent chain of work beside
// the caller's stream inside one entry point, with a pool of timing-free events for the
// fork / join points. Default priority (like every stream here); created on first use with
// the device current and kept until the process ends. `which` (0 or 1) selects one of two
// such streams; at least n_events events are returned. The lease holds the (device, which)
// slot's lock until the AuxStream is destroyed: an entry point keeps it for its whole
// fork / join enqueue sequence, so calls from several host threads on one device enqueue
// one after another and no call re-records an event before another call's wait on it has
// been enqueued (a wait binds to the record that precedes it on the host). The helper
// stream's work of such calls runs in enqueue order; each call's dependencies are its own.
struct AuxStream {
  hipStream_t st = nullptr;
  hipEvent_t* ev = nullptr;
  std::unique_lock<std::mutex> lease;
};
int aux_stream(int which, int n_events, AuxStream& out);
// pd_grouped_gemm without the launch that zeroes rows past the last group offset (for
// callers whose groups cover every row).
int grouped_gemm(const void* lhs, const void* rhs, const int32_t* offsets, int64_t J, int E, int64_t K, int64_t N,
                 int trans_rhs, void* out, int out_dtype, void* stream, bool zero_tail);
// Two grouped products of one shape and one set of group offsets in a single launch:
// out_i = lhs_i [J,K] @ rhs_i[e] with rhs_i stored [E,N,K] (K-contiguous); no tail zeroing.
int grouped_gemm_pair(const void* lhs1, const void* rhsT1, void* out1, const void* lhs2, const void* rhsT2, void* out2,
                      const int32_t* offsets, int64_t J, int E, int64_t K, int64_t N, int out_dtype, void* stream);
// Grouped two-segment products in job space, one launch for a pair (lhs1b NULL: one):
// out[j] = rs[sort_idx[j] / k] * (lhs1[j] @ rhs1[e]) + lhs2[j] @ rhs2[e] for job j of
// expert e, every rhs stored [E, N, K_seg] (K-contiguous), fp32 accumulation through both
// segments and one bf16 rounding; the second problem uses lhs1b / rhs1b / lhs2b / rhs2b /
// outb and the same row scale rs2 (NULL: rs).
int grouped_gemm_kcat(const void* lhs1, const void* rhs1, int64_t K1, const void* lhs2, const void* rhs2, int64_t K2,
                      void* out, const float* rs, const void* lhs1b, const void* rhs1b, const void* lhs2b,
                      const void* rhs2b, void* outb, const float* rs2, const int32_t* sort_idx, int k,
                      const int32_t* offsets, int64_t J, int E, int64_t N, void* stream);
// Two ragged-contraction weight gradients in one launch: out_i[e] = lhs_i[rows_e]^T @
// dout_i[rows_e] from the row-major job-space operands lhs_i [J,K] and dout_i [J,N].
int grouped_gemm_dw_pair(const void* lhs1, const void* dout1, void* out1, const void* lhs2, const void* dout2,
                         void* out2, const int32_t* offsets, int64_t J, int E, int64_t K, int64_t N, int out_dtype,
                         void* stream);

// pd_router_topk with the logits first rounded to bf16 when round_bf16 is set (the
// reference's router product runs in the target's bf16 matmul dtype and is widened to
// fp32 afterwards, pd/targets/qwen36_moe.py:473-475).
int router_topk(const float* logits, int64_t T, int E, int k, bool round_bf16, float* probs, int32_t* top_idx,
                float* weights, void* stream);

// C = A @ Bt^T (bf16, both operands K-contiguous: A [M, K] ld lda, Bt [N, K] ld ldb) with
// the contraction split into slices when the output alone has too few tiles to occupy
// the GPU: each slice's fp32 partial goes to `ws` and a second pass adds the slices in
// order (deterministic), writing C (+ beta * C) in c_dtype. gemm_splitk_ws_bytes gives the
// scratch the same call needs (0: no split; the call then needs no scratch). `splits` > 0
// asks for that many slices (each a multiple of 64 deep) instead of the tile-count rule.
size_t gemm_splitk_ws_bytes(int64_t M, int64_t N, int64_t K, int splits = 0);
// The same for any operand layouts (trans_a / trans_b as pd_gemm's).
int gemm_splitk(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, int trans_a, const void* B, int64_t ldb,
                int trans_b, void* C, int64_t ldc, int c_dtype, float beta, void* ws, size_t ws_bytes, void* stream,
                int splits = 0);
int gemm_nt_splitk(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* Bt, int64_t ldb, void* C,
                   int64_t ldc, int c_dtype, float beta, void* ws, size_t ws_bytes, void* stream);

// ---------------------------------------------------------------- bf16
typedef uint16_t bf16_t;

__host__ __device__ inline float bf16_to_f32(bf16_t v) {
  union {
    uint32_t u;
    float f;
  } c;
  c.u = (uint32_t)v << 16;
  return c.f;
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays NaN). On the device this is gfx950's
// v_cvt_pk_bf16_f32; the host keeps the bit-level rounding.
__host__ __device__ inline bf16_t f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(bf16_t, (__bf16)f);
#else
  union {
    uint32_t u;
    float f;
  } c;
  c.f = f;
  uint32_t u = c.u;
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (bf16_t)((u >> 16) | 0x40);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
#endif
}

// Two fp32 values -> packed bf16 pair (a in the low half) with one v_cvt_pk_bf16_f32.
__device__ inline uint32_t pack_bf16x2(float a, float b) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

template <typename T>
__device__ inline float load_f(const T* p, int64_t i);
template <>
__device__ inline float load_f<float>(const float* p, int64_t i) {
  return p[i];
}
template <>
__device__ inline float load_f<bf16_t>(const bf16_t* p, int64_t i) {
  return bf16_to_f32(p[i]);
}
template <typename T>
__device__ inline void store_f(T* p, int64_t i, float v);
template <>
__device__ inline void store_f<float>(float* p, int64_t i, float v) {
  p[i] = v;
}
template <>
__device__ inline void store_f<bf16_t>(bf16_t* p, int64_t i, float v) {
  p[i] = f32_to_bf16(v);
}

// ---------------------------------------------------------------- Threefry-2x32-20
// Salmon et al., SC'11; rotation constants (13,15,26,6,17,29,16,24), parity 0x1BD11BDA.
__host__ __device__ inline uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

__host__ __device__ inline void threefry2x32(uint32_t k0, uint32_t k1, uint32_t& x0, uint32_t& x1) {
  const uint32_t k2 = k0 ^ k1 ^ 0x1BD11BDAu;
  x0 += k0;
  x1 += k1;
#define PD_TF_ROUND(r) \
  x0 += x1;            \
  x1 = rotl32(x1, r);  \
  x1 ^= x0;
  PD_TF_ROUND(13) PD_TF_ROUND(15) PD_TF_ROUND(26) PD_TF_ROUND(6)
  x0 += k1; x1 += k2 + 1u;
  PD_TF_ROUND(17) PD_TF_ROUND(29) PD_TF_ROUND(16) PD_TF_ROUND(24)
  x0 += k2; x1 += k0 + 2u;
  PD_TF_ROUND(13) PD_TF_ROUND(15) PD_TF_ROUND(26) PD_TF_ROUND(6)
  x0 += k0; x1 += k1 + 3u;
  PD_TF_ROUND(17) PD_TF_ROUND(29) PD_TF_ROUND(16) PD_TF_ROUND(24)
  x0 += k1; x1 += k2 + 4u;
  PD_TF_ROUND(13) PD_TF_ROUND(15) PD_TF_ROUND(26) PD_TF_ROUND(6)
  x0 += k2; x1 += k0 + 5u;
#undef PD_TF_ROUND
}

// Raw random bits of element `i` of an `n`-element jax.random draw of `nbits` (8 or
// 32) under JAX's partitionable (PD_LAYOUT_PARTITIONABLE) or original counter layout.
__device__ inline uint32_t draw_bits(uint32_t k0, uint32_t k1, int64_t i, int64_t n, int nbits, int layout) {
  if (layout == PD_LAYOUT_PARTITIONABLE) {
    uint32_t x0 = (uint32_t)((uint64_t)i >> 32), x1 = (uint32_t)i;
    threefry2x32(k0, k1, x0, x1);
    return x0 ^ x1;  // 8-bit draws keep the low byte
  }
  // original layout: the stream is threefry_2x32(key, iota(max_count))
  int64_t max_count = (nbits == 32) ? n : (n + 3) / 4;
  int64_t word = (nbits == 32) ? i : i / 4;
  int64_t half = (max_count + 1) / 2;
  uint32_t x0, x1;
  bool first;
  if (word < half) {
    x0 = (uint32_t)word;
    x1 = (half + word < max_count) ? (uint32_t)(half + word) : 0u;
    first = true;
  } else {
    x0 = (uint32_t)(word - half);
    x1 = (uint32_t)word;
    first = false;
  }
  threefry2x32(k0, k1, x0, x1);
  uint32_t w = first ? x0 : x1;
  return (nbits == 32) ? w : (w >> (8 * (int)(i & 3)));
}

// jax.random.uniform's mantissa trick: fp32 keeps bits[31:9]; bf16 draws 8 bits and
// keeps the top 7 of that byte.
__device__ inline float bits_to_uniform(uint32_t b, int draw_dtype) {
  return draw_dtype == PD_DTYPE_BF16 ? (float)((b & 0xFFu) >> 1) * (1.0f / 128.0f)
                                     : (float)(b >> 9) * (1.0f / 8388608.0f);
}

__device__ inline float draw_uniform(uint32_t k0, uint32_t k1, int64_t i, int64_t n, int draw_dtype, int layout) {
  return bits_to_uniform(draw_bits(k0, k1, i, n, draw_dtype == PD_DTYPE_BF16 ? 8 : 32, layout), draw_dtype);
}

// ---------------------------------------------------------------- mask sources
// Mask-source variants of the mask kernels beside the two Threefry counter layouts
// (PD_LAYOUT_*): MASK_CONST, every source value one constant (the reference's
// ConstantSources; 0 is the CI-masked reconstruction); MASK_SRC, persistent (adversarial)
// source tables, each row covering rps consecutive tokens (pd/core/masking.py:43-68,
// 260-272). Neither draws nor keeps u bytes.
static constexpr int MASK_CONST = 2;
static constexpr int MASK_SRC = 3;

// Source value i of a table stored as src_dtype (F32, BF16, or U16 = u / 65535), cast to
// bf16 as the reference casts the table to the CI dtype before use.
__device__ inline float src_value(const void* src, int dtype, int64_t i) {
  float v;
  if (dtype == PD_DTYPE_F32) v = ((const float*)src)[i];
  else if (dtype == PD_DTYPE_BF16) v = bf16_to_f32(((const bf16_t*)src)[i]);
  else v = (float)((const uint16_t*)src)[i] * (1.f / 65535.f);
  return bf16_to_f32(f32_to_bf16(v));
}

// delta[site * T + t] = bf16(src_delta[site * S + t / rps]) over n_sites sites: each
// token's delta is its source row's value, cast to the CI dtype as the reference casts the
// delta table.
static __global__ __launch_bounds__(256) void k_src_delta_fill(const void* __restrict__ src_delta, int dtype,
                                                               int64_t S, int64_t rps, int64_t T, int n_sites,
                                                               float* __restrict__ delta) {
  const int64_t n = (int64_t)n_sites * T;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t site = i / T, t = i % T;
    delta[i] = src_value(src_delta, dtype, site * S + t / rps);
  }
}

// ---------------------------------------------------------------- squashing
// lower: forward clip(x,0,1); VJP leaks 0.01*g below zero only for g<0.
__device__ inline float lower_fwd(float x) { return fminf(fmaxf(x, 0.f), 1.f); }
__device__ inline float lower_vjp(float x, float g) {
  return x <= 0.f ? (g < 0.f ? 0.01f * g : 0.f) : (x <= 1.f ? g : 0.f);
}
// upper: x>1 ? 1+0.01(x-1) : clip(x,0,1); VJP of that expression under JAX autodiff
// (clip's max/min split the cotangent evenly at exact ties x==0, x==1).
__device__ inline float upper_fwd(float x) { return x > 1.f ? 1.f + 0.01f * (x - 1.f) : fminf(fmaxf(x, 0.f), 1.f); }
__device__ inline float upper_vjp(float x, float g) {
  float s = x > 1.f ? 0.01f : ((x > 0.f && x < 1.f) ? 1.f : ((x == 0.f || x == 1.f) ? 0.5f : 0.f));
  return s * g;
}

// ---------------------------------------------------------------- GELU
// Exact-erf GELU. PRECISE uses the device library's erff/expf. The fast form uses the
// Abramowitz & Stegun 7.1.26 rational approximation of erf (|error| <= 1.5e-7), whose
// exp(-z^2/2) factor is shared with the Gaussian density needed by the derivative.
struct GeluOut {
  float gelu, grad;
};

template <bool PRECISE>
__device__ inline GeluOut gelu_and_grad(float z) {
  if (PRECISE) {
    float phi_cdf = 0.5f * (1.f + erff(z * 0.70710678118654752f));
    float pdf = 0.39894228040143268f * expf(-0.5f * z * z);
    return {z * phi_cdf, phi_cdf + z * pdf};
  } else {
    float az = fabsf(z) * 0.70710678118654752f;
    float t = __frcp_rn(fmaf(0.3275911f, az, 1.f));
    float poly = t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, 1.061405429f, -1.453152027f), 1.421413741f), -0.284496736f),
                          0.254829592f);
    float e = __expf(-0.5f * z * z);
    float q = 0.5f * poly * e;  // = 1 - Phi(|z|)
    float phi_cdf = z >= 0.f ? 1.f - q : q;
    return {z * phi_cdf, phi_cdf + z * (0.39894228040143268f * e)};
  }
}

template <bool PRECISE>
__device__ inline float gelu_only(float z) {
  if (PRECISE) return 0.5f * z * (1.f + erff(z * 0.70710678118654752f));
  float az = fabsf(z) * 0.70710678118654752f;
  float t = __frcp_rn(fmaf(0.3275911f, az, 1.f));
  float poly =
      t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, 1.061405429f, -1.453152027f), 1.421413741f), -0.284496736f), 0.254829592f);
  float q = 0.5f * poly * __expf(-0.5f * z * z);
  return z * (z >= 0.f ? 1.f - q : q);
}

// ---------------------------------------------------------------- reductions
__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ inline double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ inline float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// sum_{k < n} p[k * stride] added in k order (a deterministic reduction of per-chunk
// partials). The loads of 64 chunks are issued before their adds: with one dependent load
// per chunk such a pass is bound by n round trips to L2.
__device__ inline float pd_ordered_sum(const float* __restrict__ p, int64_t n, int64_t stride) {
  constexpr int Q = 64;
  float s = 0.f;
  int64_t k = 0;
  for (; k + Q <= n; k += Q) {
    float v[Q];
#pragma unroll
    for (int i = 0; i < Q; ++i) v[i] = p[(k + i) * stride];
#pragma unroll
    for (int i = 0; i < Q; ++i) s += v[i];
  }
  for (; k < n; ++k) s += p[k * stride];
  return s;
}

// jax.random.split(key, 2) on the host: out = {key0.x0, key0.x1, key1.x0, key1.x1}.
// partitionable: key i = block(key, (0, i)); original: the block outputs of the counter
// pairs (0, 2) and (1, 3), concatenated word-wise and read as [2, 2].
inline void split2(uint32_t k0, uint32_t k1, int layout, uint32_t out[4]) {
  if (layout == PD_LAYOUT_PARTITIONABLE) {
    uint32_t a0 = 0, a1 = 0, b0 = 0, b1 = 1;
    threefry2x32(k0, k1, a0, a1);
    threefry2x32(k0, k1, b0, b1);
    out[0] = a0, out[1] = a1, out[2] = b0, out[3] = b1;
  } else {
    uint32_t a0 = 0, a1 = 2, b0 = 1, b1 = 3;
    threefry2x32(k0, k1, a0, a1);
    threefry2x32(k0, k1, b0, b1);
    out[0] = a0, out[1] = b0, out[2] = a1, out[3] = b1;
  }
}

// ---------------------------------------------------------------- EMA frequency estimate
// The frequency penalty's running estimate of f_c (pd/core/losses.py:425-458 and
// EmaFrequency :522-543): new = ema + alpha (f - ema), f_hat = new / debias, with
// alpha = 1 - 2^(-1/h) = -expm1(-ln 2 / h) and debias = 1 - 2^(-(count + 1)/h) =
// -expm1(-ln 2 / h * (count + 1)), both in the expm1 form that stays finite up to the
// configuration's 1e6 half-life cap. alpha is the double-precision value rounded to fp32
// and debias is formed in fp32, as the reference's fp32 array arithmetic forms them; the
// update and the division run in fp32. `count` is the number of earlier observations.
struct FreqEma {
  const float* in = nullptr;  // [components] the estimate before this step; NULL = batch estimate
  float* out = nullptr;       // [components] the estimate after it (may alias in; NULL = not written)
  float alpha = 0.f, debias = 1.f;
  __host__ __device__ bool on() const { return in != nullptr; }
  // the same estimator over components [off, ...)
  __host__ __device__ FreqEma at(int64_t off) const {
    FreqEma e = *this;
    if (e.in) e.in += off;
    if (e.out) e.out += off;
    return e;
  }
};

inline int make_freq_ema(const char* what, const float* in, float* out, float count, float halflife, FreqEma& e) {
  e = FreqEma{};
  if (!in) {
    if (out) return fail(PD_EINVAL, std::string(what) + ": freq_ema_out needs freq_ema_in");
    return PD_OK;
  }
  if (!(halflife > 0.f) || !(halflife <= 1e6f))
    return fail(PD_EINVAL, std::string(what) + ": EMA half-life must be in (0, 1e6]");
  if (!(count >= 0.f) || !std::isfinite(count))
    return fail(PD_EINVAL, std::string(what) + ": EMA observation count must be >= 0");
  const double log_decay = -std::log(2.0) / (double)halflife;
  e.in = in;
  e.out = out;
  e.alpha = (float)(-std::expm1(log_decay));
  e.debias = -std::expm1((float)log_decay * (count + 1.f));
  return PD_OK;
}

// f_hat of component i from this batch's frequency f; the thread that owns component i
// passes write = true to store the new estimate.
__device__ inline float ema_frequency(const FreqEma& e, int64_t i, float f, bool write) {
  const float prev = e.in[i];
  const float next = prev + e.alpha * (f - prev);
  if (write && e.out) e.out[i] = next;
  return next / e.debias;
}

}  // namespace pd
