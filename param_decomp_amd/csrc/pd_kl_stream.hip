// Streamed-vocab KL (param_decomp/param_decomp/targets/losses.py:101-170): per-position
// KL(softmax(clean) || softmax(masked)) with z = act @ head^T produced one vocab chunk at
// a time, so the [N, V] logits never exist. Each chunk's two logit blocks come from the
// bf16 MFMA GEMM (fp32 accumulate, as the reference's `_chunk_logits`), then one block per
// row advances the paired online-softmax accumulators
//   m' = max(m, max z);  s' = s e^{m-m'} + sum e^{z-m'};  a' = a e^{m_p-m_p'} + sum e^{z_p-m_p'}(z_p - z_q)
// and KL = a/s_p - (m_p + log s_p) + (m_q + log s_q). The backward re-derives each chunk's
// logits and pushes the exact softmax cotangent (q - p) * g through the masked head.
#include <algorithm>
#include <cmath>

#include "pd_common.hpp"

namespace pd {

static constexpr int KL_THREADS = 256;

__device__ inline float block_max256(float v, float* red) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return r;
}

__device__ inline float block_sum256(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float r = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return r;
}

// stats[n] = (m_p, s_p, a, m_q, s_q); `first` starts from m = -inf, s = a = 0.
__global__ __launch_bounds__(KL_THREADS) void k_kl_chunk(const float* __restrict__ zp, const float* __restrict__ zq,
                                                         int64_t ch, int64_t ld, float* __restrict__ stats, int first) {
  __shared__ float red[4];
  const int64_t n = blockIdx.x;
  const float* p = zp + n * ld;
  const float* q = zq + n * ld;
  float mp = -INFINITY, mq = -INFINITY;
  for (int64_t v = threadIdx.x; v < ch; v += KL_THREADS) {
    mp = fmaxf(mp, p[v]);
    mq = fmaxf(mq, q[v]);
  }
  mp = block_max256(mp, red);
  mq = block_max256(mq, red);
  float* st = stats + n * 5;
  const float mp_old = first ? -INFINITY : st[0], mq_old = first ? -INFINITY : st[3];
  const float mp2 = fmaxf(mp_old, mp), mq2 = fmaxf(mq_old, mq);
  float sp = 0.f, sa = 0.f, sq = 0.f;
  for (int64_t v = threadIdx.x; v < ch; v += KL_THREADS) {
    const float a = p[v], b = q[v];
    const float e = expf(a - mp2);
    sp += e;
    sa = fmaf(e, a - b, sa);
    sq += expf(b - mq2);
  }
  sp = block_sum256(sp, red);
  sa = block_sum256(sa, red);
  sq = block_sum256(sq, red);
  if (threadIdx.x == 0) {
    if (first) {
      st[0] = mp2, st[1] = sp, st[2] = sa, st[3] = mq2, st[4] = sq;
    } else {
      const float rp = expf(mp_old - mp2);
      st[0] = mp2;
      st[1] = st[1] * rp + sp;
      st[2] = st[2] * rp + sa;
      st[3] = mq2;
      st[4] = st[4] * expf(mq_old - mq2) + sq;
    }
  }
}

__global__ void k_kl_final(const float* __restrict__ stats, int64_t N, float* __restrict__ kl) {
  for (int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; n < N; n += (int64_t)gridDim.x * blockDim.x) {
    const float* st = stats + n * 5;
    kl[n] = st[2] / st[1] - (st[0] + logf(st[1])) + (st[3] + logf(st[4]));
  }
}

// G[n, v] = (e^{z_q - logZ_q} - e^{z_p - logZ_p}) * g[n] for v < ch, stored in the GEMM
// operand type with row pitch ld; columns [ch, kpad) are zeroed (the contraction of the
// input-gradient product is padded to a multiple of 8).
template <typename T>
__global__ __launch_bounds__(KL_THREADS) void k_kl_grad(const float* __restrict__ zp, const float* __restrict__ zq,
                                                        int64_t ch, int64_t ld, int64_t kpad,
                                                        const float* __restrict__ stats, const float* __restrict__ g,
                                                        T* __restrict__ G) {
  const int64_t n = blockIdx.x;
  const float* st = stats + n * 5;
  const float lzp = st[0] + logf(st[1]), lzq = st[3] + logf(st[4]);
  const float gn = g[n];
  for (int64_t v = threadIdx.x; v < kpad; v += KL_THREADS)
    store_f<T>(G, n * ld + v, v < ch ? (expf(zq[n * ld + v] - lzq) - expf(zp[n * ld + v] - lzp)) * gn : 0.f);
}

// Copies rows [0, rows) of a [rows, d] head chunk into a [kpad, d] buffer, zero rows after.
template <typename T>
__global__ void k_pad_rows(const T* __restrict__ src, int64_t rows, int64_t kpad, int64_t d, T* __restrict__ dst) {
  const int64_t n = kpad * d;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = i / d < rows ? src[i] : (T)0;
}

// The kernels stream the vocab in chunks of cw columns (the reference chunk V / n_chunks,
// rounded up to a multiple of 8 for bf16 so every product's operands stay 16-byte rows);
// the last chunk may be narrower. The KL does not depend on the chunking.
struct KLChunks {
  int64_t cw, nc;
  int64_t width(int64_t c, int64_t V) const { return std::min(cw, V - c * cw); }
};
static KLChunks kl_chunks(int dtype, int64_t V, int n_chunks) {
  const int64_t ch = V / n_chunks;
  const int64_t cw = dtype == PD_DTYPE_BF16 ? (ch + 7) & ~(int64_t)7 : ch;
  return {cw, cdiv(V, cw)};
}

struct KLPlan {
  float *zp, *zq;
  void* G;
  void* head_pad;  // [cw, d]: the last chunk's head rows, zero-padded (bf16, ragged last chunk only)
  size_t total;
};

static KLPlan kl_plan(int dtype, int64_t N, int64_t d, int64_t V, int n_chunks, char* base) {
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const KLChunks K = kl_chunks(dtype, V, n_chunks);
  const size_t esz = dtype == PD_DTYPE_BF16 ? 2 : 4;
  KLPlan P;
  size_t off = 0;
  P.zp = (float*)(base + off);
  off += up((size_t)N * K.cw * 4);
  P.zq = (float*)(base + off);
  off += up((size_t)N * K.cw * 4);
  P.G = base + off;
  off += up((size_t)N * K.cw * esz);
  P.head_pad = base + off;
  if (dtype == PD_DTYPE_BF16 && K.width(K.nc - 1, V) % 8) off += up((size_t)K.cw * d * esz);
  P.total = off;
  return P;
}

static int kl_check(int dtype, int64_t N, int64_t d, int64_t V, int n_chunks, const void* am, const void* hm,
                    const void* ac, const void* hc, const char* who) {
  if (N <= 0 || d <= 0 || V <= 0 || n_chunks <= 0 || V % n_chunks || !am || !hm || !ac || !hc)
    return fail(PD_EINVAL, std::string(who) + ": need N, d, V > 0 and n_chunks dividing V");
  if (dtype != PD_DTYPE_F32 && dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, std::string(who) + ": dtype");
  if (dtype == PD_DTYPE_BF16 && d % 8)
    return fail(PD_EUNSUPPORTED, std::string(who) + ": bf16 needs d to be a multiple of 8");
  if (N > 0x7FFFFFFF) return fail(PD_EUNSUPPORTED, std::string(who) + ": too many positions");
  return PD_OK;
}

}  // namespace pd

using namespace pd;

extern "C" {

size_t pd_streamed_kl_workspace_size(int dtype, int64_t N, int64_t d, int64_t V, int n_chunks) {
  if (N <= 0 || d <= 0 || V <= 0 || n_chunks <= 0 || V % n_chunks) return 0;
  return kl_plan(dtype, N, d, V, n_chunks, nullptr).total;
}

int pd_streamed_kl_fwd(int dtype, int64_t N, int64_t d, int64_t V, int n_chunks, const void* act_masked,
                       const void* head_masked, const void* act_clean, const void* head_clean, float* position_kl,
                       float* stats, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = kl_check(dtype, N, d, V, n_chunks, act_masked, head_masked, act_clean, head_clean, "pd_streamed_kl_fwd");
  if (rc) return rc;
  if (!position_kl || !stats) return fail(PD_EINVAL, "pd_streamed_kl_fwd: outputs required");
  if (!workspace || workspace_bytes < kl_plan(dtype, N, d, V, n_chunks, nullptr).total)
    return fail(PD_EWORKSPACE, "pd_streamed_kl_fwd: workspace too small");
  const KLChunks K = kl_chunks(dtype, V, n_chunks);
  KLPlan P = kl_plan(dtype, N, d, V, n_chunks, (char*)workspace);
  hipStream_t s = (hipStream_t)stream;
  const size_t esz = dtype == PD_DTYPE_BF16 ? 2 : 4;
  for (int64_t c = 0; c < K.nc; ++c) {
    const int64_t w = K.width(c, V);
    const char* hcc = (const char*)head_clean + (size_t)c * K.cw * d * esz;
    const char* hmc = (const char*)head_masked + (size_t)c * K.cw * d * esz;
    if ((rc = pd_gemm(dtype, N, w, d, act_clean, d, 0, hcc, d, 1, P.zp, K.cw, PD_DTYPE_F32, 1.f, 0.f, stream)))
      return rc;
    if ((rc = pd_gemm(dtype, N, w, d, act_masked, d, 0, hmc, d, 1, P.zq, K.cw, PD_DTYPE_F32, 1.f, 0.f, stream)))
      return rc;
    hipLaunchKernelGGL(k_kl_chunk, dim3((unsigned)N), dim3(KL_THREADS), 0, s, P.zp, P.zq, w, K.cw, stats, c == 0);
  }
  hipLaunchKernelGGL(k_kl_final, dim3((unsigned)std::min<int64_t>(cdiv(N, 256), 4096)), dim3(256), 0, s, stats, N,
                     position_kl);
  return check_launch("pd_streamed_kl_fwd");
}

int pd_streamed_kl_bwd(int dtype, int64_t N, int64_t d, int64_t V, int n_chunks, const void* act_masked,
                       const void* head_masked, const void* act_clean, const void* head_clean, const float* stats,
                       const float* g_position, float* d_act_masked, void* workspace, size_t workspace_bytes,
                       void* stream) {
  int rc = kl_check(dtype, N, d, V, n_chunks, act_masked, head_masked, act_clean, head_clean, "pd_streamed_kl_bwd");
  if (rc) return rc;
  if (!stats || !g_position || !d_act_masked) return fail(PD_EINVAL, "pd_streamed_kl_bwd: stats, g and output required");
  if (!workspace || workspace_bytes < kl_plan(dtype, N, d, V, n_chunks, nullptr).total)
    return fail(PD_EWORKSPACE, "pd_streamed_kl_bwd: workspace too small");
  const KLChunks K = kl_chunks(dtype, V, n_chunks);
  KLPlan P = kl_plan(dtype, N, d, V, n_chunks, (char*)workspace);
  hipStream_t s = (hipStream_t)stream;
  const size_t esz = dtype == PD_DTYPE_BF16 ? 2 : 4;
  for (int64_t c = 0; c < K.nc; ++c) {
    const int64_t w = K.width(c, V);
    const int64_t kpad = dtype == PD_DTYPE_BF16 ? (w + 7) & ~(int64_t)7 : w;
    const char* hcc = (const char*)head_clean + (size_t)c * K.cw * d * esz;
    const char* hmc = (const char*)head_masked + (size_t)c * K.cw * d * esz;
    if ((rc = pd_gemm(dtype, N, w, d, act_clean, d, 0, hcc, d, 1, P.zp, K.cw, PD_DTYPE_F32, 1.f, 0.f, stream)))
      return rc;
    if ((rc = pd_gemm(dtype, N, w, d, act_masked, d, 0, hmc, d, 1, P.zq, K.cw, PD_DTYPE_F32, 1.f, 0.f, stream)))
      return rc;
    if (dtype == PD_DTYPE_BF16)
      hipLaunchKernelGGL(k_kl_grad<bf16_t>, dim3((unsigned)N), dim3(KL_THREADS), 0, s, P.zp, P.zq, w, K.cw, kpad,
                         stats, g_position, (bf16_t*)P.G);
    else
      hipLaunchKernelGGL(k_kl_grad<float>, dim3((unsigned)N), dim3(KL_THREADS), 0, s, P.zp, P.zq, w, K.cw, kpad,
                         stats, g_position, (float*)P.G);
    // d_act += G [N, kpad] @ head_chunk [kpad, d]; a ragged bf16 chunk reads a zero-padded
    // copy of its head rows so the contraction stays whole 16-byte rows
    const void* hk = hmc;
    if (kpad != w) {
      hipLaunchKernelGGL(k_pad_rows<bf16_t>, dim3((unsigned)std::min<int64_t>(cdiv(kpad * d, 256), 4096)), dim3(256),
                         0, s, (const bf16_t*)hmc, w, kpad, d, (bf16_t*)P.head_pad);
      hk = P.head_pad;
    }
    if ((rc = pd_gemm(dtype, N, d, kpad, P.G, K.cw, 0, hk, d, 0, d_act_masked, d, PD_DTYPE_F32, 1.f,
                      c == 0 ? 0.f : 1.f, stream)))
      return rc;
  }
  return check_launch("pd_streamed_kl_bwd");
}

}  // extern "C"
