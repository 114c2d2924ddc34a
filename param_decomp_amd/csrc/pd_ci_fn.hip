// The engine's CI functions on gfx950: the per-site vector MLP and the
// component-activation readout.
//
// SiteMLP (pd/core/ci_fn/implementations/mlp.py:57-78; layerwise_mlp.py:127-140): the
// preactivations of a site are L_n(GELU(... GELU(L_1(x)))), L_i(a) = a @ W_i + b_i with
// W_i stored [d_i, d_i+1] and exact-erf GELU, in bf16 compute with fp32 accumulation:
// every product is rounded to bf16, the bias is added to that bf16 value and rounded,
// and GELU's output is rounded. The forward GEMMs run on W_i^T copies (both operands
// K-contiguous) with the bias and GELU in the epilogue, saving z_i (pre-GELU) and
// a_i = GELU(z_i) in the workspace. The backward runs d_a = d_z @ W_i^T with
// d_z_prev = bf16(d_a * GELU'(z_prev)) in the epilogue, dW_i = a_i-1^T @ d_z_i on
// K-contiguous copies, and db_i as a two-phase fixed-order column sum.
//
// Component-activation readout (pd/core/ci_fn/implementations/transformer/
// component_conditioning.py:215-245): per component, s+ sig(a+ h + b+) + s- sig(a- (-h) +
// b-) + bias with sig the symmetric leaky hard sigmoid (pd/core/ci_fn/squashing.py:25-38),
// added to a base preactivation when one is given.
#include <algorithm>
#include <vector>

#include "pd_gemm_dtl.hpp"

namespace pd {

static constexpr int CT = 64;            // transpose tile
static constexpr int COLSUM_ROWS = 256;  // rows per block of a column-sum pass
static constexpr int MLP_MAX_LAYERS = 16;

__device__ inline float bfr(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// dst[c][r] = src[r][c] for bf16 [R, Cc] into rows of ldd >= R elements, the columns
// r in [R, ldd) zeroed (a contraction padded to a multiple of 8). 64x64 tiles through
// LDS with 16-byte global loads and stores: Cc % 8 == 0, ldd % 8 == 0, 16-byte aligned.
__global__ __launch_bounds__(256) void k_ci_transpose(const bf16_t* __restrict__ src, int64_t R, int64_t Cc,
                                                      bf16_t* __restrict__ dst, int64_t ldd) {
  constexpr int LDT = CT + 8;  // row pitch keeps 16-byte LDS stores aligned
  __shared__ __attribute__((aligned(16))) bf16_t tile[CT][LDT];
  const int64_t r0 = (int64_t)blockIdx.y * CT, c0 = (int64_t)blockIdx.x * CT;
  const int t = threadIdx.x, ch = t & 7;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int row = (t >> 3) + 32 * pass;
    const int64_t r = r0 + row, c = c0 + ch * 8;
    const uint4 v = (r < R && c < Cc) ? *(const uint4*)(src + r * Cc + c) : make_uint4(0, 0, 0, 0);
    *(uint4*)&tile[row][ch * 8] = v;
  }
  __syncthreads();
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int col = (t >> 3) + 32 * pass;
    const int64_t c = c0 + col, r = r0 + ch * 8;
    if (c < Cc && r < ldd) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = (uint32_t)tile[ch * 8 + 2 * j][col] | ((uint32_t)tile[ch * 8 + 2 * j + 1][col] << 16);
      *(uint4*)(dst + c * ldd + r) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

static void ci_transpose(const bf16_t* src, int64_t R, int64_t Cc, bf16_t* dst, int64_t ldd, hipStream_t s) {
  hipLaunchKernelGGL(k_ci_transpose, dim3((unsigned)cdiv(Cc, CT), (unsigned)cdiv(ldd, CT)), dim3(256), 0, s, src, R,
                     Cc, dst, ldd);
}

// Epilogue of L_i: z = bf16(bf16(acc) + b); a hidden layer stores z to zsave and
// bf16(GELU(z)) to C, the head stores z to C. N % 4 == 0.
struct EpiBiasGelu {
  static constexpr int LDS_BYTES = 0;
  struct Args {
    const bf16_t* bias;
    bf16_t* zsave;  // NULL for the head
  };
  template <class CFG, typename TC>
  __device__ static void run(const GemmArgs& p, const Args& a, const TileJob& t, int wm, int wn, int tid,
                             f32x16 (&acc)[CFG::TM][CFG::TN], char*) {
    const int lane = tid & 63;
    bf16_t* C = (bf16_t*)t.C;
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
          const uint2 bw = *(const uint2*)(a.bias + col);
          const float b[4] = {bf16_to_f32((bf16_t)(bw.x & 0xFFFF)), bf16_to_f32((bf16_t)(bw.x >> 16)),
                              bf16_to_f32((bf16_t)(bw.y & 0xFFFF)), bf16_to_f32((bf16_t)(bw.y >> 16))};
          float z[4], o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            z[e] = bfr(bfr(acc[i][j][4 * g + e]) + b[e]);
            o[e] = a.zsave ? gelu_and_grad<true>(z[e]).gelu : z[e];
          }
          const int64_t idx = row * p.ldc + col;
          if (a.zsave) *(uint2*)(a.zsave + idx) = make_uint2(pack_bf16x2(z[0], z[1]), pack_bf16x2(z[2], z[3]));
          *(uint2*)(C + idx) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
        }
    }
  }
};

// Epilogue of d_a = d_z @ W^T: d_a = bf16(acc); with z given, C = bf16(d_a * GELU'(z)),
// else C = d_a. N % 4 == 0.
struct EpiGeluGrad {
  static constexpr int LDS_BYTES = 0;
  struct Args {
    const bf16_t* z;  // saved pre-activations [M, N] (ld = ldc), or NULL
  };
  template <class CFG, typename TC>
  __device__ static void run(const GemmArgs& p, const Args& a, const TileJob& t, int wm, int wn, int tid,
                             f32x16 (&acc)[CFG::TM][CFG::TN], char*) {
    const int lane = tid & 63;
    bf16_t* C = (bf16_t*)t.C;
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
          const int64_t idx = row * p.ldc + col;
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = bfr(acc[i][j][4 * g + e]);
          if (a.z) {
            const uint2 zw = *(const uint2*)(a.z + idx);
            const float z[4] = {bf16_to_f32((bf16_t)(zw.x & 0xFFFF)), bf16_to_f32((bf16_t)(zw.x >> 16)),
                                bf16_to_f32((bf16_t)(zw.y & 0xFFFF)), bf16_to_f32((bf16_t)(zw.y >> 16))};
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] *= gelu_and_grad<true>(z[e]).grad;
          }
          *(uint2*)(C + idx) = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
        }
    }
  }
};

// part[chunk][c] = sum over the chunk's MLP_SUM_ROWS rows of x[row][c]: a lane sums 8
// columns (16-byte loads), the 4 waves a quarter of the rows each, added in wave order.
// Cc % 8 == 0, 16-byte aligned.
static constexpr int MLP_SUM_ROWS = 64;
__global__ __launch_bounds__(256) void k_colsum_part(const bf16_t* __restrict__ x, int64_t R, int64_t Cc,
                                                     float* __restrict__ part) {
  constexpr int WROWS = MLP_SUM_ROWS / 4;
  __shared__ float red[3][8][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = ((int64_t)blockIdx.x * 64 + lane) * 8;
  const bool live = c < Cc;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (live) {
    const int64_t r0 = (int64_t)blockIdx.y * MLP_SUM_ROWS + w * WROWS, r1 = r0 + WROWS < R ? r0 + WROWS : R;
    for (int64_t r = r0; r < r1; r += 4) {
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (r + u < r1) v[u] = *(const uint4*)(x + (r + u) * Cc + c);
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (r + u < r1) {
          const uint32_t q[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[2 * i] += bf16_to_f32((bf16_t)(q[i] & 0xFFFF));
            acc[2 * i + 1] += bf16_to_f32((bf16_t)(q[i] >> 16));
          }
        }
    }
  }
  if (w > 0)
#pragma unroll
    for (int e = 0; e < 8; ++e) red[w - 1][e][lane] = acc[e];
  __syncthreads();
  if (w == 0 && live) {
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = ((acc[e] + red[0][e][lane]) + red[1][e][lane]) + red[2][e][lane];
    float* dst = part + (int64_t)blockIdx.y * Cc + c;
    *(float4*)dst = make_float4(o[0], o[1], o[2], o[3]);
    *(float4*)(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
  }
}

// out[j] = sum over the n_part rows of part[.][j] (rows of width n): the 4 waves of a
// block take the rows k = w mod 4 in order and are added in wave order, so the result
// depends on n_part alone. Grid cdiv(n, 64).
__global__ __launch_bounds__(256) void k_sum_parts(const float* __restrict__ part, int64_t n_part, int64_t n,
                                                   float* __restrict__ out) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t j = (int64_t)blockIdx.x * 64 + lane;
  float acc = 0.f;
  if (j < n) {
#pragma unroll 4
    for (int64_t k = w; k < n_part; k += 4) acc += part[k * n + j];
  }
  red[w][lane] = acc;
  __syncthreads();
  if (w == 0 && j < n) out[j] = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
}

// ---------------------------------------------------------------- MLP workspace
struct MlpPlan {
  bf16_t* WT[MLP_MAX_LAYERS];  // W_i^T [d_i+1, d_i]
  bf16_t* Z[MLP_MAX_LAYERS];   // hidden pre-activations [N, d_i+1]
  bf16_t* A[MLP_MAX_LAYERS];   // hidden activations [N, d_i+1]
  bf16_t *dz_a, *dz_b;         // backward ping-pong [N, max d]
  bf16_t *aT, *dzT;            // K-contiguous copies [max d, Np], Np = N rounded up to 8
  float* part;                 // column-sum partials [N / MLP_SUM_ROWS, max d]
  size_t total;
};

static MlpPlan mlp_plan(int L, const int64_t* dims, int64_t N, char* base) {
  MlpPlan P{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? base + off : nullptr;
    off += (bytes + 255) & ~(size_t)255;
    return p;
  };
  int64_t mx = 0;
  for (int i = 0; i <= L; ++i) mx = std::max(mx, dims[i]);
  for (int i = 0; i < L; ++i) P.WT[i] = (bf16_t*)take(2 * (size_t)dims[i] * dims[i + 1]);
  for (int i = 0; i + 1 < L; ++i) {
    P.Z[i] = (bf16_t*)take(2 * (size_t)N * dims[i + 1]);
    P.A[i] = (bf16_t*)take(2 * (size_t)N * dims[i + 1]);
  }
  P.dz_a = (bf16_t*)take(2 * (size_t)N * mx);
  P.dz_b = (bf16_t*)take(2 * (size_t)N * mx);
  const int64_t Np = (N + 7) & ~(int64_t)7;
  P.aT = (bf16_t*)take(2 * (size_t)Np * mx);
  P.dzT = (bf16_t*)take(2 * (size_t)Np * mx);
  P.part = (float*)take(4 * (size_t)cdiv(N, MLP_SUM_ROWS) * mx);
  P.total = off;
  return P;
}

static int mlp_check(const char* what, int L, const int64_t* dims, int64_t N) {
  if (L < 1 || L > MLP_MAX_LAYERS || !dims || N <= 0)
    return fail(PD_EINVAL, std::string(what) + ": 1 <= n_layers <= 16, dims and n_tokens required");
  for (int i = 0; i <= L; ++i)
    if (dims[i] <= 0 || dims[i] % 8)
      return fail(PD_EUNSUPPORTED, std::string(what) + ": every width must be a positive multiple of 8");
  if (cdiv(N + 7, CT) > 65535) return fail(PD_EUNSUPPORTED, std::string(what) + ": more than 4194240 tokens");
  for (int i = 0; i <= L; ++i)
    if (cdiv(dims[i], CT) > 65535) return fail(PD_EUNSUPPORTED, std::string(what) + ": width too large");
  return PD_OK;
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ---------------------------------------------------------------- readout
struct ReadoutParams {  // fp32 masters, used as bf16 (the engine's compute cast)
  float ap, bp, sp, an, bn, sn, bias;
};
__device__ inline ReadoutParams readout_params(const float* __restrict__ prm, int64_t C, int64_t c) {
  return {bfr(prm[c]),         bfr(prm[C + c]),     bfr(prm[2 * C + c]), bfr(prm[3 * C + c]),
          bfr(prm[4 * C + c]), bfr(prm[5 * C + c]), bfr(prm[6 * C + c])};
}
__device__ inline float clamp01(float x) { return fminf(fmaxf(x, 0.f), 1.f); }
// VJP of the symmetric leaky hard sigmoid: inside (0, 1) pass g; at or below 0 leak 0.01 g
// only for g < 0; at or above 1 leak 0.01 g only for g > 0 (pd/core/ci_fn/squashing.py:32-35).
__device__ inline float sym_vjp(float x, float g) {
  return x <= 0.f ? (g < 0.f ? 0.01f * g : 0.f) : (x >= 1.f ? (g > 0.f ? 0.01f * g : 0.f) : g);
}

// out = base + s+ clamp(a+ h + b+) + s- clamp(a- (-h) + b-) + bias; prm [7, C] = a+, b+, s+,
// a-, b-, s-, bias.
__global__ __launch_bounds__(256) void k_readout_fwd(const bf16_t* __restrict__ h, const float* __restrict__ prm,
                                                     const bf16_t* __restrict__ base, int64_t N, int64_t C,
                                                     bf16_t* __restrict__ out) {
  const int64_t n = N * C;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t c = i % C;
    const ReadoutParams q = readout_params(prm, C, c);
    const float hv = bf16_to_f32(h[i]);
    float v = q.sp * clamp01(q.ap * hv + q.bp) + q.sn * clamp01(q.an * -hv + q.bn) + q.bias;
    if (base) v += bf16_to_f32(base[i]);
    out[i] = f32_to_bf16(v);
  }
}

// d_h = a+ dx+ - a- dx- with dx± = sym_vjp(x±, g s±); per-chunk partials of the 7
// parameter gradients: part[chunk][k][c] (lane = component, 4 waves of rows).
__global__ __launch_bounds__(256) void k_readout_bwd(const bf16_t* __restrict__ h, const float* __restrict__ prm,
                                                     const bf16_t* __restrict__ g_out, int64_t N, int64_t C,
                                                     bf16_t* __restrict__ d_h, float* __restrict__ part) {
  __shared__ float red[4][7][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane, r0 = (int64_t)blockIdx.y * COLSUM_ROWS;
  float acc[7] = {0, 0, 0, 0, 0, 0, 0};
  if (c < C) {
    const ReadoutParams q = readout_params(prm, C, c);
    for (int64_t r = r0 + w; r < r0 + COLSUM_ROWS && r < N; r += 4) {
      const int64_t i = r * C + c;
      const float hv = bf16_to_f32(h[i]), g = bf16_to_f32(g_out[i]);
      const float xp = q.ap * hv + q.bp, xn = q.an * -hv + q.bn;
      const float dxp = sym_vjp(xp, g * q.sp), dxn = sym_vjp(xn, g * q.sn);
      if (d_h) d_h[i] = f32_to_bf16(q.ap * dxp - q.an * dxn);
      acc[0] = fmaf(hv, dxp, acc[0]);
      acc[1] += dxp;
      acc[2] = fmaf(g, clamp01(xp), acc[2]);
      acc[3] = fmaf(-hv, dxn, acc[3]);
      acc[4] += dxn;
      acc[5] = fmaf(g, clamp01(xn), acc[5]);
      acc[6] += g;
    }
  }
#pragma unroll
  for (int k = 0; k < 7; ++k) red[w][k][lane] = acc[k];
  __syncthreads();
  if (w == 0 && c < C)
#pragma unroll
    for (int k = 0; k < 7; ++k)
      part[((int64_t)blockIdx.y * 7 + k) * C + c] = red[0][k][lane] + red[1][k][lane] + red[2][k][lane] + red[3][k][lane];
}

// ---- vector forms: VEC consecutive components per lane (8- or 16-byte I/O), parameters
// held in registers, rows looped with RO_UNROLL loads in flight. C % VEC == 0, bf16
// tensors aligned to 2 * VEC bytes, params and partials 16-byte aligned.
static constexpr int RO_ROWS_FWD = 64;
static constexpr int RO_UNROLL = 4;
static constexpr int RO_UNROLL_BWD = 2;  // the backward's 7 accumulators leave room for 2
static constexpr int RO_VEC = 4;

template <int VEC>
struct BfVec;
template <>
struct BfVec<4> {
  typedef uint2 T;
  __device__ static void unpack(T w, float (&v)[4]) {
    v[0] = bf16_to_f32((bf16_t)(w.x & 0xFFFF));
    v[1] = bf16_to_f32((bf16_t)(w.x >> 16));
    v[2] = bf16_to_f32((bf16_t)(w.y & 0xFFFF));
    v[3] = bf16_to_f32((bf16_t)(w.y >> 16));
  }
  __device__ static T pack(const float (&v)[4]) { return make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])); }
  __device__ static T zero() { return make_uint2(0, 0); }
};
template <>
struct BfVec<8> {
  typedef uint4 T;
  __device__ static void unpack(T w, float (&v)[8]) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_to_f32((bf16_t)(u[i] & 0xFFFF));
      v[2 * i + 1] = bf16_to_f32((bf16_t)(u[i] >> 16));
    }
  }
  __device__ static T pack(const float (&v)[8]) {
    return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                      pack_bf16x2(v[6], v[7]));
  }
  __device__ static T zero() { return make_uint4(0, 0, 0, 0); }
};

template <int VEC>
__device__ inline void load_params_v(const float* __restrict__ prm, int64_t C, int64_t c, float (&q)[7][VEC]) {
#pragma unroll
  for (int k = 0; k < 7; ++k)
#pragma unroll
    for (int e4 = 0; e4 < VEC; e4 += 4) {
      const float4 a = *(const float4*)(prm + k * C + c + e4);
      q[k][e4] = bfr(a.x);
      q[k][e4 + 1] = bfr(a.y);
      q[k][e4 + 2] = bfr(a.z);
      q[k][e4 + 3] = bfr(a.w);
    }
}

template <int VEC>
__global__ __launch_bounds__(256) void k_readout_fwd_v(const bf16_t* __restrict__ h, const float* __restrict__ prm,
                                                       const bf16_t* __restrict__ base, int64_t N, int64_t C,
                                                       bf16_t* __restrict__ out) {
  typedef BfVec<VEC> BV;
  typedef typename BV::T VT;
  const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VEC;
  if (c >= C) return;
  float q[7][VEC];
  load_params_v<VEC>(prm, C, c, q);
  const int64_t r0 = (int64_t)blockIdx.y * RO_ROWS_FWD, r1 = r0 + RO_ROWS_FWD < N ? r0 + RO_ROWS_FWD : N;
  for (int64_t r = r0; r < r1; r += RO_UNROLL) {
    VT hw[RO_UNROLL], bw[RO_UNROLL];
#pragma unroll
    for (int u = 0; u < RO_UNROLL; ++u)
      if (r + u < r1) {
        hw[u] = *(const VT*)(h + (r + u) * C + c);
        bw[u] = base ? *(const VT*)(base + (r + u) * C + c) : BV::zero();
      }
#pragma unroll
    for (int u = 0; u < RO_UNROLL; ++u)
      if (r + u < r1) {
        float hv[VEC], bv[VEC], o[VEC];
        BV::unpack(hw[u], hv);
        BV::unpack(bw[u], bv);
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          o[e] = bv[e] + (q[2][e] * clamp01(q[0][e] * hv[e] + q[1][e]) +
                          q[5][e] * clamp01(q[3][e] * -hv[e] + q[4][e]) + q[6][e]);
        *(VT*)(out + (r + u) * C + c) = BV::pack(o);
      }
  }
}

// One block = 64 lanes x VEC components over COLSUM_ROWS rows, the 4 waves taking a
// quarter of the rows each and summed through LDS in wave order; partials
// part[chunk][k][c] as in k_readout_bwd.
template <int VEC, int UNR = RO_UNROLL_BWD>
__global__ __launch_bounds__(256) void k_readout_bwd_v(const bf16_t* __restrict__ h, const float* __restrict__ prm,
                                                       const bf16_t* __restrict__ g_out, int64_t N, int64_t C,
                                                       bf16_t* __restrict__ d_h, float* __restrict__ part) {
  typedef BfVec<VEC> BV;
  typedef typename BV::T VT;
  constexpr int WROWS = COLSUM_ROWS / 4;
  __shared__ float red[3][7][VEC][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = ((int64_t)blockIdx.x * 64 + lane) * VEC;
  const bool live = c < C;
  float acc[7][VEC];
#pragma unroll
  for (int k = 0; k < 7; ++k)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[k][e] = 0.f;
  if (live) {
    float q[7][VEC];
    load_params_v<VEC>(prm, C, c, q);
    const int64_t r0 = (int64_t)blockIdx.y * COLSUM_ROWS + w * WROWS;
    const int64_t r1 = r0 + WROWS < N ? r0 + WROWS : N;
    for (int64_t r = r0; r < r1; r += UNR) {
      VT hw[UNR], gw[UNR];
#pragma unroll
      for (int u = 0; u < UNR; ++u)
        if (r + u < r1) {
          hw[u] = *(const VT*)(h + (r + u) * C + c);
          gw[u] = *(const VT*)(g_out + (r + u) * C + c);
        }
#pragma unroll
      for (int u = 0; u < UNR; ++u)
        if (r + u < r1) {
          float hv[VEC], gv[VEC], dh[VEC];
          BV::unpack(hw[u], hv);
          BV::unpack(gw[u], gv);
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const float xp = q[0][e] * hv[e] + q[1][e], xn = q[3][e] * -hv[e] + q[4][e];
            const float dxp = sym_vjp(xp, gv[e] * q[2][e]), dxn = sym_vjp(xn, gv[e] * q[5][e]);
            dh[e] = q[0][e] * dxp - q[3][e] * dxn;
            acc[0][e] = fmaf(hv[e], dxp, acc[0][e]);
            acc[1][e] += dxp;
            acc[2][e] = fmaf(gv[e], clamp01(xp), acc[2][e]);
            acc[3][e] = fmaf(-hv[e], dxn, acc[3][e]);
            acc[4][e] += dxn;
            acc[5][e] = fmaf(gv[e], clamp01(xn), acc[5][e]);
            acc[6][e] += gv[e];
          }
          if (d_h) *(VT*)(d_h + (r + u) * C + c) = BV::pack(dh);
        }
    }
  }
  if (w > 0)
#pragma unroll
    for (int k = 0; k < 7; ++k)
#pragma unroll
      for (int e = 0; e < VEC; ++e) red[w - 1][k][e][lane] = acc[k][e];
  __syncthreads();
  if (w == 0 && live)
#pragma unroll
    for (int k = 0; k < 7; ++k) {
      float v[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[e] = ((acc[k][e] + red[0][k][e][lane]) + red[1][k][e][lane]) + red[2][k][e][lane];
      float* dst = part + ((int64_t)blockIdx.y * 7 + k) * C + c;
#pragma unroll
      for (int e4 = 0; e4 < VEC; e4 += 4) *(float4*)(dst + e4) = make_float4(v[e4], v[e4 + 1], v[e4 + 2], v[e4 + 3]);
    }
}

static bool readout_vec_ok(int64_t C, const void* a, const void* b, const void* c, const void* d, const float* prm) {
  auto al = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  return C % RO_VEC == 0 && C % 4 == 0 && al(a) && al(b) && al(c) && al(d) && al(prm);
}

}  // namespace pd

using namespace pd;

extern "C" {

size_t pd_ci_mlp_workspace_size(int n_layers, const int64_t* dims, int64_t n_tokens) {
  if (n_layers < 1 || n_layers > MLP_MAX_LAYERS || !dims || n_tokens <= 0) return 0;
  return mlp_plan(n_layers, dims, n_tokens, nullptr).total;
}

int pd_ci_mlp_fwd(int n_layers, const int64_t* dims, int64_t n_tokens, const void* x, const void* const* weights,
                  const void* const* biases, void* preact, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = mlp_check("pd_ci_mlp_fwd", n_layers, dims, n_tokens))) return rc;
  if (!x || !weights || !biases || !preact) return fail(PD_EINVAL, "pd_ci_mlp_fwd: null pointer");
  for (int i = 0; i < n_layers; ++i)
    if (!weights[i] || !biases[i]) return fail(PD_EINVAL, "pd_ci_mlp_fwd: null weight or bias");
  bool ok = al16(x) && al16(preact);
  for (int i = 0; i < n_layers; ++i) ok = ok && al16(weights[i]) && al16(biases[i]);
  if (!ok) return fail(PD_EUNSUPPORTED, "pd_ci_mlp_fwd: every tensor must be 16-byte aligned");
  if (!workspace || workspace_bytes < mlp_plan(n_layers, dims, n_tokens, nullptr).total)
    return fail(PD_EWORKSPACE, "pd_ci_mlp_fwd: workspace too small");
  const MlpPlan P = mlp_plan(n_layers, dims, n_tokens, (char*)workspace);
  hipStream_t s = (hipStream_t)stream;
  const bf16_t* a = (const bf16_t*)x;
  for (int i = 0; i < n_layers; ++i) {
    const int64_t din = dims[i], dout = dims[i + 1];
    ci_transpose((const bf16_t*)weights[i], din, dout, P.WT[i], din, s);
    const bool head = i + 1 == n_layers;
    bf16_t* out = head ? (bf16_t*)preact : P.A[i];
    GemmArgs g{n_tokens, dout, din, a, din, P.WT[i], din, out, dout, 1.f, 0.f, nullptr, 0, 0, 0, 0,
               nullptr, nullptr, nullptr};
    EpiBiasGelu::Args ea{(const bf16_t*)biases[i], head ? nullptr : P.Z[i]};
    if ((rc = launch_dense_epi<EpiBiasGelu, bf16_t>(g, ea, s, "pd_ci_mlp_fwd"))) return rc;
    a = out;
  }
  return PD_OK;
}

int pd_ci_mlp_bwd(int n_layers, const int64_t* dims, int64_t n_tokens, const void* x, const void* const* weights,
                  const void* d_preact, float* const* d_weights, float* const* d_biases, void* d_x, void* workspace,
                  size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = mlp_check("pd_ci_mlp_bwd", n_layers, dims, n_tokens))) return rc;
  if (!x || !weights || !d_preact || !d_weights || !d_biases) return fail(PD_EINVAL, "pd_ci_mlp_bwd: null pointer");
  for (int i = 0; i < n_layers; ++i)
    if (!weights[i] || !d_weights[i] || !d_biases[i]) return fail(PD_EINVAL, "pd_ci_mlp_bwd: null weight or gradient");
  bool ok = al16(x) && al16(d_preact) && al16(d_x);
  for (int i = 0; i < n_layers; ++i) ok = ok && al16(weights[i]) && al16(d_weights[i]);
  if (!ok) return fail(PD_EUNSUPPORTED, "pd_ci_mlp_bwd: every tensor must be 16-byte aligned");
  if (!workspace || workspace_bytes < mlp_plan(n_layers, dims, n_tokens, nullptr).total)
    return fail(PD_EWORKSPACE, "pd_ci_mlp_bwd: workspace too small");
  const MlpPlan P = mlp_plan(n_layers, dims, n_tokens, (char*)workspace);
  hipStream_t s = (hipStream_t)stream;
  const int64_t N = n_tokens, Np = (N + 7) & ~(int64_t)7, nchunk = cdiv(N, MLP_SUM_ROWS);
  const bf16_t* dz = (const bf16_t*)d_preact;
  for (int i = n_layers - 1; i >= 0; --i) {
    const int64_t din = dims[i], dout = dims[i + 1];
    const bf16_t* ain = i == 0 ? (const bf16_t*)x : P.A[i - 1];
    // db_i = column sums of d_z_i
    hipLaunchKernelGGL(k_colsum_part, dim3((unsigned)cdiv(dout / 8, 64), (unsigned)nchunk), dim3(256), 0, s, dz, N, dout,
                       P.part);
    hipLaunchKernelGGL(k_sum_parts, dim3((unsigned)cdiv(dout, 64)), dim3(256), 0, s, P.part, nchunk, dout,
                       d_biases[i]);
    // dW_i [din, dout] = a^T [din, N] @ (d_z^T [dout, N])^T
    ci_transpose(ain, N, din, P.aT, Np, s);
    ci_transpose(dz, N, dout, P.dzT, Np, s);
    if ((rc = pd_gemm(PD_DTYPE_BF16, din, dout, Np, P.aT, Np, 0, P.dzT, Np, 1, d_weights[i], dout, PD_DTYPE_F32, 1.f,
                      0.f, stream)))
      return rc;
    // d_a = d_z @ W_i^T (B = W_i stored [din, dout]: [N, K] K-contiguous), then the GELU
    // pullback of layer i-1, or the input gradient
    if (i > 0 || d_x) {
      bf16_t* dst = i > 0 ? (dz == P.dz_a ? P.dz_b : P.dz_a) : (bf16_t*)d_x;
      GemmArgs g{N, din, dout, dz, dout, (const bf16_t*)weights[i], dout, dst, din, 1.f, 0.f, nullptr, 0, 0, 0, 0,
                 nullptr, nullptr, nullptr};
      EpiGeluGrad::Args ea{i > 0 ? P.Z[i - 1] : nullptr};
      if ((rc = launch_dense_epi<EpiGeluGrad, bf16_t>(g, ea, s, "pd_ci_mlp_bwd"))) return rc;
      dz = dst;
    }
  }
  return check_launch("pd_ci_mlp_bwd");
}

size_t pd_ci_readout_workspace_size(int64_t n_tokens, int64_t C) {
  if (n_tokens <= 0 || C <= 0) return 0;
  return (size_t)cdiv(n_tokens, COLSUM_ROWS) * 7 * C * 4;
}

int pd_ci_readout_fwd(int64_t n_tokens, int64_t C, const void* h, const float* params, const void* base, void* out,
                      void* stream) {
  if (n_tokens <= 0 || C <= 0 || !h || !params || !out) return fail(PD_EINVAL, "pd_ci_readout_fwd: bad args");
  const int64_t n = n_tokens * C;
  if (readout_vec_ok(C, h, base, out, nullptr, params) && cdiv(n_tokens, RO_ROWS_FWD) <= 65535)
    hipLaunchKernelGGL(k_readout_fwd_v<RO_VEC>, dim3((unsigned)cdiv(C / RO_VEC, 256), (unsigned)cdiv(n_tokens, RO_ROWS_FWD)),
                       dim3(256), 0, (hipStream_t)stream, (const bf16_t*)h, params, (const bf16_t*)base, n_tokens, C,
                       (bf16_t*)out);
  else
    hipLaunchKernelGGL(k_readout_fwd, dim3((unsigned)std::min<int64_t>(cdiv(n, 256), 8192)), dim3(256), 0,
                       (hipStream_t)stream, (const bf16_t*)h, params, (const bf16_t*)base, n_tokens, C, (bf16_t*)out);
  return check_launch("pd_ci_readout_fwd");
}

int pd_ci_readout_bwd(int64_t n_tokens, int64_t C, const void* h, const float* params, const void* d_out, void* d_h,
                      float* d_params, void* workspace, size_t workspace_bytes, void* stream) {
  if (n_tokens <= 0 || C <= 0 || !h || !params || !d_out || !d_params)
    return fail(PD_EINVAL, "pd_ci_readout_bwd: bad args");
  const int64_t nchunk = cdiv(n_tokens, COLSUM_ROWS);
  if (nchunk > 65535) return fail(PD_EUNSUPPORTED, "pd_ci_readout_bwd: too many tokens");
  if (!workspace || workspace_bytes < pd_ci_readout_workspace_size(n_tokens, C))
    return fail(PD_EWORKSPACE, "pd_ci_readout_bwd: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)workspace;
  if (readout_vec_ok(C, h, d_out, d_h, part, params))
    hipLaunchKernelGGL(k_readout_bwd_v<RO_VEC>, dim3((unsigned)cdiv(C / RO_VEC, 64), (unsigned)nchunk), dim3(256), 0, s,
                       (const bf16_t*)h, params, (const bf16_t*)d_out, n_tokens, C, (bf16_t*)d_h, part);
  else
    hipLaunchKernelGGL(k_readout_bwd, dim3((unsigned)cdiv(C, 64), (unsigned)nchunk), dim3(256), 0, s,
                       (const bf16_t*)h, params, (const bf16_t*)d_out, n_tokens, C, (bf16_t*)d_h, part);
  hipLaunchKernelGGL(k_sum_parts, dim3((unsigned)cdiv(7 * C, 64)), dim3(256), 0, s, part, nchunk, 7 * C, d_params);
  return check_launch("pd_ci_readout_bwd");
}

}  // extern "C"
