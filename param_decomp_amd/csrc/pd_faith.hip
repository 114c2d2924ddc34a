// Faithfulness on gfx950: the relative squared weight error of every decomposed matrix
// and its gradients onto the fp32 V/U masters.
//
// The reference forms fp32 deltas Delta = W - (V U)^T per stack
// (pd/targets/transformer.py:2134-2184: `Ws.astype(f32) - einsum("gic,gco->goi", V, U)`;
// the protocol is pd/core/model.py:430-449) and reduces them to the mean over sites of
// ||Delta_s||^2 / ||W_s||^2 (pd/core/faithfulness.py:16-75). A block-factored site (an
// expert group, `[g, expert, d_out, d_in]`) sums its blocks before the division.
//
// Kernels, all fp32 on v_mfma_f32_32x32x2f32 (the deltas cancel, W ~ (VU)^T near a
// faithful decomposition, so a bf16 product would swamp them):
//   forward   Delta tile = W - U^T V^T as a GEMM whose epilogue reads W, writes Delta
//             (when the caller keeps it for the backward) and a per-block partial of
//             sum Delta^2;
//   reduce    fixed-order partial sums -> per-site errors and the loss (double);
//   backward  dV = alpha Delta^T U^T and dU = alpha V^T Delta^T with
//             alpha = -2 scale d_loss / ||W_site||^2, one GEMM each.
// Every product here has its A operand stored [K][M] (M-contiguous) and its B operand
// stored [N][K] (K-contiguous), so one GEMM layout serves all three.
#include <algorithm>

#include "pd_common.hpp"

namespace pd {

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

// Block tile 128x128, 4 waves of 64x64 (2x2 MFMA tiles of 32x32), k in stages of 16.
static constexpr int FBM = 128, FBN = 128, FBK = 16;
static constexpr int FBPAD = FBK + 1;  // B is staged [n][k]; the odd pitch spreads the banks

struct FaithArgs {
  int64_t M, N, K;
  const float* A;  // [K][M] per matrix, row pitch lda
  int64_t lda, sA;
  const float* B;  // [N][K] per matrix, row pitch ldb
  int64_t ldb, sB;
  float* C;  // [M][N] per matrix, row pitch ldc
  int64_t ldc, sC;
  int splits;   // blockIdx.z = matrix * splits + split; a split covers k in [split*kc, +kc)
  int64_t kc;   // a multiple of FBK
};

// The forward epilogue: Delta = W - acc (W [M][N] per matrix, bf16 or fp32), stored to
// C, and this block's sum of Delta^2 to part[z][tile].
struct EpiDelta {
  const void* W;
  int w_bf16;
  int64_t ldw, sW;
  float* part;
};
// The backward epilogue: C = alpha_site * acc with
// alpha_site = coef * (*gscale, when given) / norms[z / per_site].
struct EpiScale {
  const float* norms;
  int64_t per_site;
  float coef;
  const float* gscale;
};

template <bool VEC>
__device__ inline void stage_load(const FaithArgs& p, const float* A, const float* B, int64_t m0, int64_t n0,
                                  int64_t k0, int64_t kend, int tid, float (&ra)[8], float (&rb)[8]) {
  // A: FBK rows (k) x FBM floats (m); 2 float4 per thread. B: FBN rows (n) x FBK floats.
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int e = tid + 256 * q;
    const int ak = e >> 5, am = (e & 31) * 4;  // 32 float4 per A row
    const int bn = e >> 2, bk = (e & 3) * 4;   // 4 float4 per B row
    const int64_t gk = k0 + ak, gm = m0 + am;
    const int64_t gn = n0 + bn, gkb = k0 + bk;
    if (VEC) {
      float4 va = make_float4(0.f, 0.f, 0.f, 0.f), vb = va;
      if (gk < kend && gm < p.M) va = *(const float4*)(A + gk * p.lda + gm);
      if (gn < p.N && gkb < kend) vb = *(const float4*)(B + gn * p.ldb + gkb);
      ra[4 * q] = va.x, ra[4 * q + 1] = va.y, ra[4 * q + 2] = va.z, ra[4 * q + 3] = va.w;
      rb[4 * q] = vb.x, rb[4 * q + 1] = vb.y, rb[4 * q + 2] = vb.z, rb[4 * q + 3] = vb.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ra[4 * q + i] = (gk < kend && gm + i < p.M) ? A[gk * p.lda + gm + i] : 0.f;
        rb[4 * q + i] = (gn < p.N && gkb + i < kend) ? B[gn * p.ldb + gkb + i] : 0.f;
      }
    }
  }
}

__device__ inline void stage_store(float* As, float* Bs, int tid, const float (&ra)[8], const float (&rb)[8]) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int e = tid + 256 * q;
    const int ak = e >> 5, am = (e & 31) * 4;
    const int bn = e >> 2, bk = (e & 3) * 4;
    *(float4*)(As + ak * FBM + am) = make_float4(ra[4 * q], ra[4 * q + 1], ra[4 * q + 2], ra[4 * q + 3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) Bs[bn * FBPAD + bk + i] = rb[4 * q + i];
  }
}

// C[z] = op over the k loop; EPI selects the epilogue (0: delta + partial, 1: scaled store,
// 2: raw store of one k split's partial product).
// Grid (cdiv(N, 128), cdiv(M, 128), n_mats). VEC: M, K % 4 == 0 for the float4 staging
// (rows of A hold m, rows of B hold k) and 16-byte aligned bases.
template <bool VEC, int EPI>
__global__ __launch_bounds__(256) void k_faith_gemm(FaithArgs p, EpiDelta ed, EpiScale es) {
  __shared__ __attribute__((aligned(16))) float As[2][FBK * FBM];
  __shared__ float Bs[2][FBN * FBPAD];
  __shared__ float red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t zz = blockIdx.z, z = zz / p.splits;
  const int64_t kbeg = (zz % p.splits) * p.kc, kend = kbeg + p.kc < p.K ? kbeg + p.kc : p.K;
  const float* A = p.A + z * p.sA;
  const float* B = p.B + z * p.sB;
  const int64_t m0 = (int64_t)blockIdx.y * FBM, n0 = (int64_t)blockIdx.x * FBN;
  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  const int nk = (int)((kend - kbeg + FBK - 1) / FBK);
  float ra[8], rb[8];
  stage_load<VEC>(p, A, B, m0, n0, kbeg, kend, tid, ra, rb);
  stage_store(As[0], Bs[0], tid, ra, rb);
  __syncthreads();
  const int lm = lane & 31, lk = lane >> 5;
  for (int s = 0; s < nk; ++s) {
    const int cur = s & 1;
    if (s + 1 < nk) stage_load<VEC>(p, A, B, m0, n0, kbeg + (int64_t)(s + 1) * FBK, kend, tid, ra, rb);
    const float* as = As[cur];
    const float* bs = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < FBK; kk += 2) {
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = as[(kk + lk) * FBM + wm * 64 + i * 32 + lm];
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = bs[(wn * 64 + j * 32 + lm) * FBPAD + kk + lk];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < nk) {
      stage_store(As[cur ^ 1], Bs[cur ^ 1], tid, ra, rb);
      __syncthreads();
    }
  }
  // D[i][j] of a 32x32 tile: j = lane % 32 (n), i = 8 (v / 4) + 4 (lane / 32) + v % 4 (m)
  float* C = p.C ? p.C + (EPI == 2 ? zz : z) * p.sC : nullptr;
  float sq = 0.f;
  float alpha = 0.f;
  if (EPI == 1) alpha = es.coef * (es.gscale ? es.gscale[0] : 1.f) / es.norms[z / es.per_site];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = n0 + wn * 64 + j * 32 + lm;
      if (col >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t row = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * lk + (v & 3);
        if (row >= p.M) continue;
        if (EPI == 0) {
          const int64_t wi = z * ed.sW + row * ed.ldw + col;
          const float w = ed.w_bf16 ? bf16_to_f32(((const bf16_t*)ed.W)[wi]) : ((const float*)ed.W)[wi];
          const float d = w - acc[i][j][v];
          if (C) C[row * p.ldc + col] = d;
          sq = fmaf(d, d, sq);
        } else if (EPI == 1) {
          C[row * p.ldc + col] = alpha * acc[i][j][v];
        } else {
          C[row * p.ldc + col] = acc[i][j][v];
        }
      }
    }
  if (EPI == 0) {
    sq = wave_sum(sq);
    if (lane == 0) red[wave] = sq;
    __syncthreads();
    if (tid == 0)
      ed.part[(z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x] = ((red[0] + red[1]) + red[2]) + red[3];
  }
}

// Split-k forward: Delta = W - sum over splits of the partial products (added in split
// order), 8 consecutive elements of a matrix per lane, 2048 per block; part[z][block]
// takes the block's sum of Delta^2. Grid (cdiv(MN, 2048), n_mats). VEC: MN % 8 == 0 and
// 16-byte aligned W and delta.
static constexpr int DELTA_PER_BLOCK = 2048;
template <bool VEC>
__global__ __launch_bounds__(256) void k_faith_delta(const float* __restrict__ prod, int splits, int64_t MN,
                                                     EpiDelta ed, float* __restrict__ delta) {
  __shared__ float red[4];
  const int64_t z = blockIdx.y;
  const int64_t base = (int64_t)blockIdx.x * DELTA_PER_BLOCK + threadIdx.x * 8;
  float sq = 0.f;
  if (VEC && base < MN) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int sp = 0; sp < splits; ++sp) {
      const float* src = prod + (z * splits + sp) * MN + base;
      const float4 a = *(const float4*)src, b = *(const float4*)(src + 4);
      acc[0] += a.x, acc[1] += a.y, acc[2] += a.z, acc[3] += a.w;
      acc[4] += b.x, acc[5] += b.y, acc[6] += b.z, acc[7] += b.w;
    }
    float w[8];
    if (ed.w_bf16) {
      const uint4 q = *(const uint4*)((const bf16_t*)ed.W + z * MN + base);
      const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[2 * i] = bf16_to_f32((bf16_t)(u[i] & 0xFFFF));
        w[2 * i + 1] = bf16_to_f32((bf16_t)(u[i] >> 16));
      }
    } else {
      const float* wp = (const float*)ed.W + z * MN + base;
      const float4 a = *(const float4*)wp, b = *(const float4*)(wp + 4);
      w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
    }
    float d[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      d[i] = w[i] - acc[i];
      sq = fmaf(d[i], d[i], sq);
    }
    if (delta) {
      float* dp = delta + z * MN + base;
      *(float4*)dp = make_float4(d[0], d[1], d[2], d[3]);
      *(float4*)(dp + 4) = make_float4(d[4], d[5], d[6], d[7]);
    }
  } else if (!VEC) {
    for (int i = 0; i < 8; ++i) {
      const int64_t e = base + i;
      if (e >= MN) break;
      float acc = 0.f;
      for (int sp = 0; sp < splits; ++sp) acc += prod[(z * splits + sp) * MN + e];
      const float w = ed.w_bf16 ? bf16_to_f32(((const bf16_t*)ed.W)[z * MN + e]) : ((const float*)ed.W)[z * MN + e];
      const float dd = w - acc;
      if (delta) delta[z * MN + e] = dd;
      sq = fmaf(dd, dd, sq);
    }
  }
  sq = wave_sum(sq);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
  __syncthreads();
  if (threadIdx.x == 0) ed.part[z * gridDim.x + blockIdx.x] = ((red[0] + red[1]) + red[2]) + red[3];
}

// site_err[s] = sum over the site's matrices and tiles of part (fixed order, double) /
// norms[s]; loss = scale * sum_s site_err[s]. One block of 256 threads.
__global__ __launch_bounds__(256) void k_faith_reduce(const float* __restrict__ part, int64_t tiles_per_mat,
                                                      int64_t n_sites, int64_t per_site, const float* __restrict__ norms,
                                                      float scale, float* __restrict__ loss,
                                                      float* __restrict__ site_err) {
  __shared__ double red[4];
  double total = 0.0;
  const int64_t per = tiles_per_mat * per_site;
  for (int64_t s = 0; s < n_sites; ++s) {
    double acc = 0.0;
    for (int64_t t = threadIdx.x; t < per; t += 256) acc += (double)part[s * per + t];
    acc = wave_sum_d(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    const double e = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
    const double rel = e / (double)norms[s];
    if (threadIdx.x == 0 && site_err) site_err[s] = (float)rel;
    total += rel;
  }
  if (threadIdx.x == 0) loss[0] = (float)(scale * total);
}

template <int EPI>
static void launch_faith(const FaithArgs& a, const EpiDelta& ed, const EpiScale& es, int64_t n_mats, hipStream_t s) {
  const bool vec = a.M % 4 == 0 && a.K % 4 == 0 && a.lda % 4 == 0 && a.ldb % 4 == 0 && a.sA % 4 == 0 &&
                   a.sB % 4 == 0 && ((uintptr_t)a.A & 15) == 0 && ((uintptr_t)a.B & 15) == 0;
  const dim3 grid((unsigned)cdiv(a.N, FBN), (unsigned)cdiv(a.M, FBM), (unsigned)(n_mats * a.splits));
  if (vec)
    hipLaunchKernelGGL((k_faith_gemm<true, EPI>), grid, dim3(256), 0, s, a, ed, es);
  else
    hipLaunchKernelGGL((k_faith_gemm<false, EPI>), grid, dim3(256), 0, s, a, ed, es);
}

// k splits for the forward product: enough blocks for two per CU when the matrices alone
// give fewer, with every split at least 512 deep.
static int faith_splits(int64_t n_mats, int64_t d_in, int64_t d_out, int64_t C) {
  const int64_t blocks = n_mats * cdiv(d_in, FBN) * cdiv(d_out, FBM);
  int sp = 1;
  while (blocks * sp < 512 && C / (2 * sp) >= 512 && sp < 8 && n_mats * 2 * sp <= 65535) sp *= 2;
  return sp;
}

}  // namespace pd

using namespace pd;

extern "C" {

static size_t faith_part_bytes(int64_t n_mats, int64_t d_in, int64_t d_out) {
  const int64_t per = std::max(cdiv(d_in, FBN) * cdiv(d_out, FBM), cdiv(d_in * d_out, DELTA_PER_BLOCK));
  return ((4 * (size_t)n_mats * per) + 255) & ~(size_t)255;
}

size_t pd_faithfulness_workspace_size(int64_t n_mats, int64_t d_in, int64_t d_out, int64_t C) {
  if (n_mats <= 0 || d_in <= 0 || d_out <= 0 || C <= 0) return 0;
  const int sp = faith_splits(n_mats, d_in, d_out, C);
  return faith_part_bytes(n_mats, d_in, d_out) + (sp > 1 ? 4 * (size_t)sp * n_mats * d_in * d_out : 0);
}

static int faith_check(const char* what, int64_t n_mats, int64_t mats_per_site, int64_t d_in, int64_t d_out,
                       int64_t C) {
  if (n_mats <= 0 || mats_per_site <= 0 || n_mats % mats_per_site || d_in <= 0 || d_out <= 0 || C <= 0)
    return fail(PD_EINVAL, std::string(what) + ": positive sizes with n_mats a multiple of mats_per_site required");
  if (n_mats > 65535 || cdiv(std::max(d_out, C), FBM) > 65535 || cdiv(std::max(d_in, C), FBN) > 65535)
    return fail(PD_EUNSUPPORTED, std::string(what) + ": too large");
  return PD_OK;
}

int pd_faithfulness_fwd(int64_t n_mats, int64_t mats_per_site, int64_t d_in, int64_t d_out, int64_t C, const void* W,
                        int w_dtype, const float* V, const float* U, const float* w_sq_norms, float scale, float* loss,
                        float* site_errors, float* delta, void* workspace, size_t workspace_bytes, void* stream) {
  int rc;
  if ((rc = faith_check("pd_faithfulness_fwd", n_mats, mats_per_site, d_in, d_out, C))) return rc;
  if (!W || !V || !U || !w_sq_norms || !loss) return fail(PD_EINVAL, "pd_faithfulness_fwd: null pointer");
  if (w_dtype != PD_DTYPE_F32 && w_dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, "pd_faithfulness_fwd: bad W dtype");
  if (!workspace || workspace_bytes < pd_faithfulness_workspace_size(n_mats, d_in, d_out, C))
    return fail(PD_EWORKSPACE, "pd_faithfulness_fwd: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)workspace;
  const int sp = faith_splits(n_mats, d_in, d_out, C);
  const EpiDelta ed{W, w_dtype == PD_DTYPE_BF16, d_in, d_out * d_in, part};
  if (sp == 1) {
    // Delta [d_out, d_in] = W - U^T (A: U stored [C][d_out]) x V^T (B: V stored [d_in][C])
    const FaithArgs f{d_out, d_in, C, U, d_out, C * d_out, V, C, d_in * C, delta, d_in, d_out * d_in, 1, C};
    launch_faith<0>(f, ed, EpiScale{}, n_mats, s);
  } else {
    float* prod = (float*)((char*)workspace + faith_part_bytes(n_mats, d_in, d_out));
    const int64_t kc = cdiv(cdiv(C, sp), FBK) * FBK;
    const FaithArgs f{d_out, d_in, C, U, d_out, C * d_out, V, C, d_in * C, prod, d_in, d_out * d_in, sp, kc};
    launch_faith<2>(f, ed, EpiScale{}, n_mats, s);
    const int64_t MN = d_out * d_in;
    const dim3 grid((unsigned)cdiv(MN, DELTA_PER_BLOCK), (unsigned)n_mats);
    const bool vec = MN % 8 == 0 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)delta & 15) == 0;
    if (vec)
      hipLaunchKernelGGL(k_faith_delta<true>, grid, dim3(256), 0, s, prod, sp, MN, ed, delta);
    else
      hipLaunchKernelGGL(k_faith_delta<false>, grid, dim3(256), 0, s, prod, sp, MN, ed, delta);
  }
  const int64_t tiles = sp == 1 ? cdiv(d_in, FBN) * cdiv(d_out, FBM) : cdiv(d_out * d_in, DELTA_PER_BLOCK);
  hipLaunchKernelGGL(k_faith_reduce, dim3(1), dim3(256), 0, s, part, tiles, n_mats / mats_per_site, mats_per_site,
                     w_sq_norms, scale, loss, site_errors);
  return check_launch("pd_faithfulness_fwd");
}

int pd_faithfulness_bwd(int64_t n_mats, int64_t mats_per_site, int64_t d_in, int64_t d_out, int64_t C,
                        const float* delta, const float* V, const float* U, const float* w_sq_norms, float scale,
                        const float* d_loss, float* dV, float* dU, void* stream) {
  int rc;
  if ((rc = faith_check("pd_faithfulness_bwd", n_mats, mats_per_site, d_in, d_out, C))) return rc;
  if (!delta || !V || !U || !w_sq_norms || !dV || !dU) return fail(PD_EINVAL, "pd_faithfulness_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const EpiScale es{w_sq_norms, mats_per_site, -2.f * scale, d_loss};
  // dV [d_in, C] = Delta^T (A: Delta stored [d_out][d_in]) x U^T (B: U stored [C][d_out])
  const FaithArgs gv{d_in, C, d_out, delta, d_in, d_out * d_in, U, d_out, C * d_out, dV, C, d_in * C, 1, d_out};
  launch_faith<1>(gv, EpiDelta{}, es, n_mats, s);
  // dU [C, d_out] = V^T (A: V stored [d_in][C]) x Delta^T (B: Delta stored [d_out][d_in])
  const FaithArgs gu{C, d_out, d_in, V, C, d_in * C, delta, d_in, d_out * d_in, dU, d_out, C * d_out, 1, d_in};
  launch_faith<1>(gu, EpiDelta{}, es, n_mats, s);
  return check_launch("pd_faithfulness_bwd");
}

}  // extern "C"
