// MoE routing, deterministic bucketing and job-space gathers (gfx950).
//
//   pd_router_topk      softmax + select_experts + expert_mixing_weights
//                       (pd/targets/qwen36_moe.py:473-514)
//   pd_routed_jobs      stable argsort by expert, inverse, bincount
//                       (pd/routed/experts.py:115-123) as a three-phase counting sort
//   pd_gather_rows(_vjp), pd_combine_jobs   (pd/routed/experts.py:127-206, 351-359)
#include <algorithm>

#include "pd_common.hpp"

namespace pd {

// One wave per token; lane l holds experts l + 64 i (i < EPL, E <= 64 EPL). Top-k by k
// rounds of a wave argmax that prefers the larger probability and, on equal
// probabilities, the lower index: the order of a stable descending sort. ROUND: the
// logits are rounded to bf16 first. k <= 64.
template <bool ROUND, int EPL>
__global__ __launch_bounds__(256) void k_router_topk(const float* __restrict__ logits, int64_t T, int E, int k,
                                                     float* __restrict__ probs, int32_t* __restrict__ top_idx,
                                                     float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  if (t >= T) return;
  float x[EPL], cand[EPL];
  float mxl = -INFINITY;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + 64 * i;
    x[i] = e < E ? logits[t * E + e] : -INFINITY;
    if (ROUND && e < E) x[i] = bf16_to_f32(f32_to_bf16(x[i]));
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
    const float p = x[i] / z;
    if (probs && e < E) probs[t * E + e] = p;
    cand[i] = e < E ? p : -INFINITY;
  }
  float sel_sum = 0.f, my_w = 0.f;
  for (int s = 0; s < k; ++s) {
    float bv = cand[0];
    int bi = lane;
#pragma unroll
    for (int i = 1; i < EPL; ++i)
      if (cand[i] > bv) {  // strict: the lower index keeps a tie
        bv = cand[i];
        bi = lane + 64 * i;
      }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      float ov = __shfl_xor(bv, off, 64);
      int oi = __shfl_xor(bi, off, 64);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi >= E) bi = E - 1;  // only reachable with NaN probabilities
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (lane + 64 * i == bi) cand[i] = -INFINITY;
    if (lane == s) my_w = bv;
    sel_sum += bv;
    if (lane == 0) top_idx[t * k + s] = bi;
  }
  if (lane < k) weights[t * k + lane] = my_w / sel_sum;
}

// ---- counting sort. Phase 1: per-chunk histograms.
constexpr int SORT_CHUNK = 256;
constexpr int SORT_MAX_E = 1024;

// Expert ids outside [0, E) (only possible from corrupt routing input) are clamped
// into range identically in every phase, so positions stay a permutation of [0, n).
__device__ inline int clamp_key(int k, int E) { return k < 0 ? 0 : (k >= E ? E - 1 : k); }

__global__ __launch_bounds__(256) void k_sort_hist(const int32_t* __restrict__ keys, int64_t n, int E,
                                                   int32_t* __restrict__ counts) {
  __shared__ int32_t h[SORT_MAX_E];
  for (int e = threadIdx.x; e < E; e += blockDim.x) h[e] = 0;
  __syncthreads();
  int64_t j0 = (int64_t)blockIdx.x * SORT_CHUNK;
  for (int64_t j = j0 + threadIdx.x; j < n && j < j0 + SORT_CHUNK; j += blockDim.x)
    atomicAdd(&h[clamp_key(keys[j], E)], 1);
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) counts[(int64_t)blockIdx.x * E + e] = h[e];
}

// Phase 2 (one block): group sizes, exclusive group offsets, and each chunk's base
// position per expert (in place over counts). One wave per expert scans the chunk
// counts 64 at a time.
__global__ __launch_bounds__(1024) void k_sort_scan(int32_t* __restrict__ counts, int64_t nchunks, int E,
                                                    int32_t* __restrict__ group_sizes,
                                                    int32_t* __restrict__ group_offsets) {
  __shared__ int32_t tot[SORT_MAX_E + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  for (int e = wave; e < E; e += nwaves) {
    int32_t carry = 0;
    for (int64_t b0 = 0; b0 < nchunks; b0 += 64) {
      const int64_t b = b0 + lane;
      const int32_t c = b < nchunks ? counts[b * E + e] : 0;
      int32_t incl = c;
      for (int o = 1; o < 64; o <<= 1) {
        const int32_t v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
      }
      if (b < nchunks) counts[b * E + e] = carry + incl - c;  // exclusive prefix over chunks
      carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) {
      tot[e] = carry;
      group_sizes[e] = carry;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t acc = 0;
    for (int e = 0; e < E; ++e) {
      int32_t c = tot[e];
      tot[e] = acc;
      group_offsets[e] = acc;
      acc += c;
    }
    group_offsets[E] = acc;
    tot[E] = acc;
  }
  __syncthreads();
  for (int64_t i = threadIdx.x; i < nchunks * E; i += blockDim.x) counts[i] += tot[i % E];
}

// Phase 3: one wave per chunk walks it in 64-job steps. Lanes holding the same expert
// find each other with one ballot per key bit; a lane's position is its chunk base +
// the running count of its expert + the number of earlier lanes with that expert.
// Stable by construction.
__global__ __launch_bounds__(64) void k_sort_scatter(const int32_t* __restrict__ keys, int64_t n, int E,
                                                     const int32_t* __restrict__ base, int32_t* __restrict__ sort_idx,
                                                     int32_t* __restrict__ inv_sort_idx) {
  __shared__ int32_t run[SORT_MAX_E];
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) run[e] = base[(int64_t)blockIdx.x * E + e];
  __syncthreads();
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
  int64_t j0 = (int64_t)blockIdx.x * SORT_CHUNK;
  int64_t j1 = j0 + SORT_CHUNK < n ? j0 + SORT_CHUNK : n;
  for (int64_t s0 = j0; s0 < j1; s0 += 64) {
    const int64_t j = s0 + lane;
    const bool valid = j < j1;
    const int key = valid ? clamp_key(keys[j], E) : 0;
    uint64_t same = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const uint64_t ones = __ballot((key >> b) & 1);
      same &= ((key >> b) & 1) ? ones : ~ones;
    }
    const int before = __popcll(same & lt);
    const int32_t start = run[key];
    if (valid) {
      const int32_t pos = start + before;
      sort_idx[pos] = (int32_t)j;
      inv_sort_idx[j] = pos;
    }
    __syncthreads();  // every lane has read run[] before any lane advances it
    if (valid && (same >> lane) == 1ull) run[key] = start + before + 1;  // last lane of its expert
    __syncthreads();
  }
}

// ---- gathers (16-byte vectors when rows allow it)
template <typename T>
__global__ void k_gather_rows(const T* __restrict__ src, int64_t width, const int32_t* __restrict__ idx, int div,
                              int64_t n_out, T* __restrict__ out) {
  for (int64_t r = blockIdx.x; r < n_out; r += gridDim.x) {
    int64_t srow = idx[r] / div;
    const T* s = src + srow * width;
    T* d = out + r * width;
    if ((width * (int64_t)sizeof(T)) % 16 == 0 && ((uintptr_t)src % 16 == 0) && ((uintptr_t)out % 16 == 0)) {
      int64_t nv = width * (int64_t)sizeof(T) / 16;
      for (int64_t i = threadIdx.x; i < nv; i += blockDim.x) ((uint4*)d)[i] = ((const uint4*)s)[i];
    } else {
      for (int64_t i = threadIdx.x; i < width; i += blockDim.x) d[i] = s[i];
    }
  }
}

template <typename T>
__global__ void k_combine(const T* __restrict__ y, int64_t width, const int32_t* __restrict__ inv,
                          const float* __restrict__ w, int64_t T_, int k, T* __restrict__ out) {
  for (int64_t t = blockIdx.x; t < T_; t += gridDim.x) {
    for (int64_t i = threadIdx.x; i < width; i += blockDim.x) {
      float acc = 0.f;
      for (int s = 0; s < k; ++s) {
        float v = load_f<T>(y, (int64_t)inv[t * k + s] * width + i);
        acc = w ? fmaf(w[t * k + s], v, acc) : acc + v;
      }
      store_f<T>(out, t * width + i, acc);
    }
  }
}

// ---- routing samplers (which sites take the decomposed output at each position)
constexpr int ROUTE_MAX_SITES = 64, ROUTE_BLOCK = 128;

// Uniform-k subset: k = 1 + randint offset from 32 high bits (key hk) and 32 low bits
// (key lk), the 64-bit value reduced mod n_sites in 32-bit steps; u[j] = fp32 uniform of
// element j*N + pos of an [S, N] draw (key pk); routes[rank(j)][pos] = (j < k), with
// rank(j) = j's place in the stable ascending order of u[:, pos].
template <int LAYOUT>
__global__ __launch_bounds__(ROUTE_BLOCK) void k_route_uniform_k(uint32_t hk0, uint32_t hk1, uint32_t lk0,
                                                                 uint32_t lk1, uint32_t pk0, uint32_t pk1, int64_t N,
                                                                 int S, uint8_t* __restrict__ routes) {
  __shared__ float u[ROUTE_MAX_SITES][ROUTE_BLOCK];
  const int64_t pos = (int64_t)blockIdx.x * ROUTE_BLOCK + threadIdx.x;
  if (pos >= N) return;  // each thread only touches its own LDS column
  const uint32_t span = (uint32_t)S;
  const uint32_t hb = draw_bits(hk0, hk1, pos, N, 32, LAYOUT);
  const uint32_t lb = draw_bits(lk0, lk1, pos, N, 32, LAYOUT);
  const uint32_t m = ((65536u % span) * (65536u % span)) % span;
  const uint32_t k = 1u + ((hb % span) * m + lb % span) % span;
  for (int j = 0; j < S; ++j)
    u[j][threadIdx.x] =
        bits_to_uniform(draw_bits(pk0, pk1, (int64_t)j * N + pos, (int64_t)S * N, 32, LAYOUT), PD_DTYPE_F32);
  for (int j = 0; j < S; ++j) {
    const float uj = u[j][threadIdx.x];
    int rank = 0;
    for (int t = 0; t < S; ++t) {
      const float ut = u[t][threadIdx.x];
      rank += (ut < uj) || (ut == uj && t < j);
    }
    routes[(int64_t)rank * N + pos] = (uint8_t)((uint32_t)j < k);
  }
}

// Static probability: routes[j][pos] = (fp32 uniform of fold_in(key, j) at pos) < p.
template <int LAYOUT>
__global__ __launch_bounds__(256) void k_route_static_p(uint32_t k0, uint32_t k1, int64_t N, float p,
                                                        uint8_t* __restrict__ routes) {
  const int j = blockIdx.y;
  uint32_t f0 = 0, f1 = (uint32_t)j;
  threefry2x32(k0, k1, f0, f1);
  for (int64_t pos = (int64_t)blockIdx.x * 256 + threadIdx.x; pos < N; pos += (int64_t)gridDim.x * 256)
    routes[(int64_t)j * N + pos] =
        (uint8_t)(bits_to_uniform(draw_bits(f0, f1, pos, N, 32, LAYOUT), PD_DTYPE_F32) < p);
}

int router_topk(const float* logits, int64_t T, int E, int k, bool round_bf16, float* probs, int32_t* top_idx,
                float* weights, void* stream) {
  if (T < 0 || E <= 0 || E > 512 || k <= 0 || k > E || k > 64 || !logits || !top_idx || !weights)
    return fail(PD_EINVAL, "pd_router_topk: need 0 < k <= min(E, 64), E <= 512");
  if (T == 0) return PD_OK;
  const dim3 grid((unsigned)cdiv(T, 4));
  hipStream_t s = (hipStream_t)stream;
#define PD_RT(EPL)                                                                                           \
  do {                                                                                                       \
    if (round_bf16)                                                                                          \
      hipLaunchKernelGGL((k_router_topk<true, EPL>), grid, dim3(256), 0, s, logits, T, E, k, probs, top_idx, \
                         weights);                                                                           \
    else                                                                                                     \
      hipLaunchKernelGGL((k_router_topk<false, EPL>), grid, dim3(256), 0, s, logits, T, E, k, probs,        \
                         top_idx, weights);                                                                  \
  } while (0)
  if (E <= 64) PD_RT(1);
  else if (E <= 128) PD_RT(2);
  else if (E <= 256) PD_RT(4);
  else PD_RT(8);
#undef PD_RT
  return check_launch("pd_router_topk");
}

}  // namespace pd

using namespace pd;

extern "C" {

int pd_router_topk(const float* logits, int64_t T, int E, int k, float* probs, int32_t* top_idx, float* weights,
                   void* stream) {
  return router_topk(logits, T, E, k, false, probs, top_idx, weights, stream);
}

size_t pd_routed_jobs_workspace_size(int64_t n_jobs, int E) {
  return (size_t)cdiv(n_jobs, SORT_CHUNK) * (size_t)E * sizeof(int32_t);
}

int pd_routed_jobs(const int32_t* top_idx, int64_t T, int k, int E, int32_t* sort_idx, int32_t* inv_sort_idx,
                   int32_t* group_sizes, int32_t* group_offsets, void* workspace, size_t workspace_bytes,
                   void* stream) {
  if (T < 0 || k <= 0 || E <= 0 || E > SORT_MAX_E || !top_idx || !sort_idx || !inv_sort_idx || !group_sizes ||
      !group_offsets)
    return fail(PD_EINVAL, "pd_routed_jobs: bad args (E <= 1024)");
  int64_t n = T * k;
  if (n > 0x7FFFFFFF) return fail(PD_EUNSUPPORTED, "pd_routed_jobs: too many jobs");
  if (!workspace || workspace_bytes < pd_routed_jobs_workspace_size(n, E))
    return fail(PD_EWORKSPACE, "pd_routed_jobs: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  int64_t nchunks = cdiv(n, SORT_CHUNK);
  int32_t* counts = (int32_t*)workspace;
  if (nchunks > 0) hipLaunchKernelGGL(k_sort_hist, dim3((unsigned)nchunks), dim3(256), 0, s, top_idx, n, E, counts);
  hipLaunchKernelGGL(k_sort_scan, dim3(1), dim3(1024), 0, s, counts, nchunks, E, group_sizes, group_offsets);
  if (nchunks > 0)
    hipLaunchKernelGGL(k_sort_scatter, dim3((unsigned)nchunks), dim3(64), 0, s, top_idx, n, E, counts, sort_idx,
                       inv_sort_idx);
  return check_launch("pd_routed_jobs");
}

int pd_gather_rows(const void* src, int dtype, int64_t width, const int32_t* idx, int div, int64_t n_out, void* out,
                   void* stream) {
  if (width <= 0 || n_out < 0 || div <= 0 || !src || !idx || !out) return fail(PD_EINVAL, "pd_gather_rows: bad args");
  if (n_out == 0) return PD_OK;
  unsigned blocks = (unsigned)std::min<int64_t>(n_out, 65535);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PD_DTYPE_F32)
    hipLaunchKernelGGL(k_gather_rows<float>, dim3(blocks), dim3(128), 0, s, (const float*)src, width, idx, div, n_out,
                       (float*)out);
  else if (dtype == PD_DTYPE_BF16)
    hipLaunchKernelGGL(k_gather_rows<bf16_t>, dim3(blocks), dim3(128), 0, s, (const bf16_t*)src, width, idx, div,
                       n_out, (bf16_t*)out);
  else
    return fail(PD_EINVAL, "pd_gather_rows: dtype");
  return check_launch("pd_gather_rows");
}

int pd_combine_jobs(const void* y, int dtype, int64_t width, const int32_t* inv, const float* weights, int64_t T,
                    int k, void* out, void* stream) {
  if (width <= 0 || T < 0 || k <= 0 || !y || !inv || !out) return fail(PD_EINVAL, "pd_combine_jobs: bad args");
  if (T == 0) return PD_OK;
  unsigned blocks = (unsigned)std::min<int64_t>(T, 65535);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == PD_DTYPE_F32)
    hipLaunchKernelGGL(k_combine<float>, dim3(blocks), dim3(256), 0, s, (const float*)y, width, inv, weights, T, k,
                       (float*)out);
  else if (dtype == PD_DTYPE_BF16)
    hipLaunchKernelGGL(k_combine<bf16_t>, dim3(blocks), dim3(256), 0, s, (const bf16_t*)y, width, inv, weights, T, k,
                       (bf16_t*)out);
  else
    return fail(PD_EINVAL, "pd_combine_jobs: dtype");
  return check_launch("pd_combine_jobs");
}

int pd_gather_rows_vjp(const void* grad, int dtype, int64_t width, const int32_t* inv, int64_t T, int k, void* out,
                       void* stream) {
  return pd_combine_jobs(grad, dtype, width, inv, nullptr, T, k, out, stream);
}


int pd_route_uniform_k(uint32_t key0, uint32_t key1, int64_t n_positions, int n_sites, int layout, uint8_t* routes,
                       void* stream) {
  if (n_positions < 0 || n_sites < 1 || n_sites > ROUTE_MAX_SITES || !routes)
    return fail(PD_EINVAL, "pd_route_uniform_k: need 1 <= n_sites <= 64 and an output");
  if (layout != PD_LAYOUT_PARTITIONABLE && layout != PD_LAYOUT_ORIGINAL)
    return fail(PD_EINVAL, "pd_route_uniform_k: unknown counter layout");
  if (n_positions == 0) return PD_OK;
  if (cdiv(n_positions, ROUTE_BLOCK) > 0x7FFFFFFF) return fail(PD_EUNSUPPORTED, "pd_route_uniform_k: too large");
  uint32_t kp[4], hl[4];
  split2(key0, key1, layout, kp);     // (k_key, perm_key)
  split2(kp[0], kp[1], layout, hl);   // randint's (high-bits key, low-bits key)
  const dim3 grid((unsigned)cdiv(n_positions, ROUTE_BLOCK));
  if (layout == PD_LAYOUT_PARTITIONABLE)
    hipLaunchKernelGGL(k_route_uniform_k<PD_LAYOUT_PARTITIONABLE>, grid, dim3(ROUTE_BLOCK), 0, (hipStream_t)stream,
                       hl[0], hl[1], hl[2], hl[3], kp[2], kp[3], n_positions, n_sites, routes);
  else
    hipLaunchKernelGGL(k_route_uniform_k<PD_LAYOUT_ORIGINAL>, grid, dim3(ROUTE_BLOCK), 0, (hipStream_t)stream, hl[0],
                       hl[1], hl[2], hl[3], kp[2], kp[3], n_positions, n_sites, routes);
  return check_launch("pd_route_uniform_k");
}

int pd_route_static_p(uint32_t key0, uint32_t key1, int64_t n_positions, int n_sites, float p, int layout,
                      uint8_t* routes, void* stream) {
  if (n_positions < 0 || n_sites < 1 || n_sites > 65535 || !routes)
    return fail(PD_EINVAL, "pd_route_static_p: need 1 <= n_sites <= 65535 and an output");
  if (layout != PD_LAYOUT_PARTITIONABLE && layout != PD_LAYOUT_ORIGINAL)
    return fail(PD_EINVAL, "pd_route_static_p: unknown counter layout");
  if (n_positions == 0) return PD_OK;
  const dim3 grid((unsigned)std::min<int64_t>(cdiv(n_positions, 256), 4096), (unsigned)n_sites);
  if (layout == PD_LAYOUT_PARTITIONABLE)
    hipLaunchKernelGGL(k_route_static_p<PD_LAYOUT_PARTITIONABLE>, grid, dim3(256), 0, (hipStream_t)stream, key0,
                       key1, n_positions, p, routes);
  else
    hipLaunchKernelGGL(k_route_static_p<PD_LAYOUT_ORIGINAL>, grid, dim3(256), 0, (hipStream_t)stream, key0, key1,
                       n_positions, p, routes);
  return check_launch("pd_route_static_p");
}

}  // extern "C"
