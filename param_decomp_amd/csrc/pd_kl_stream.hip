// Streamed-vocab KL (param_decomp/param_decomp/targets/losses.py:101-170): per-position
// KL(softmax(clean) || softmax(masked)) with z = act @ head^T produced one vocab chunk at
// a time, so the [N, V] logits never exist. Each chunk's two logit blocks come from the
// bf16 MFMA GEMM (fp32 accumulate, as the reference's `_chunk_logits`), then one block per
// row advances the paired online-softmax accumulators
//   m' = max(m, max z);  s' = s e^{m-m'} + sum e^{z-m'};  a' = a e^{m_p-m_p'} + sum e^{z_p-m_p'}(z_p - z_q)
// and KL = a/s_p - (m_p + log s_p) + (m_q + log s_q). The backward re-derives each chunk's
// logits and pushes the exact softmax cotangent (q - p) * g through the masked head.
//
// bf16 runs fused: one block computes the clean and the masked logit tile of the same
// (positions, vocab) block together (`k_gemm_dtl_dual`), so the logits never reach HBM.
// The forward epilogue reduces its tile to per-position partial accumulators, and a
// fixed-order merge combines the tiles. The backward epilogue writes (q - p) g in bf16
// straight into the input-gradient product's operand; that product runs on a
// K-contiguous copy of the masked head. fp32 runs the unfused chunk passes.
#include <algorithm>
#include <cmath>

#include "pd_gemm_dtl.hpp"

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

// ---------------------------------------------------------------- fused bf16 path
__device__ inline void kl_merge(float& mp, float& sp, float& sa, float& mq, float& sq, float mp2, float sp2, float sa2,
                                float mq2, float sq2) {
  if (mp2 == -INFINITY) return;  // an empty partial
  if (mp == -INFINITY) {
    mp = mp2, sp = sp2, sa = sa2, mq = mq2, sq = sq2;
    return;
  }
  const float m = fmaxf(mp, mp2), r1 = expf(mp - m), r2 = expf(mp2 - m);
  sp = sp * r1 + sp2 * r2;
  sa = sa * r1 + sa2 * r2;
  mp = m;
  const float n = fmaxf(mq, mq2), q1 = expf(mq - n), q2 = expf(mq2 - n);
  sq = sq * q1 + sq2 * q2;
  mq = n;
}

// e^x for the epilogues' per-logit exponentials, x <= 0 up to rounding: one v_exp_f32 of
// x log2(e) (relative error ~1e-6 for |x| <= 30, the fused passes' logits being bf16
// products) instead of the library expf's range-reduced sequence, a third of the fused
// epilogues' VALU work.
__device__ inline float kl_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// Forward epilogue: the tile's partial (m_p, s_p, a, m_q, s_q) of each position over the
// tile's vocab columns, to part[(row * n_tiles + tile) * 5]. Rows are summed across the
// lane pair (lane, lane ^ 32) and the two waves of a row in a fixed order.
struct EpiKLStats {
  static constexpr int LDS_BYTES = 0;
  struct Args {
    float* part;
    int64_t n_tiles, tile_base;
  };
  template <class CFG>
  __device__ static void run(const GemmArgs& p, const Args& a, const TileJob& t, int wm, int wn, int tid,
                             f32x16 (&zp)[CFG::TM][CFG::TN], f32x16 (&zq)[CFG::TM][CFG::TN], char* smem) {
    static_assert(CFG::TM == 1 && CFG::WN == 2 && CFG::WTM == 32, "one 32-row MFMA tile per wave, two waves across N");
    const int lane = tid & 63;
    float mp = -INFINITY, mq = -INFINITY;
#pragma unroll
    for (int j = 0; j < CFG::TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t col = t.n0 + wn * CFG::WTN + j * 32 + 8 * g + 4 * (lane >> 5) + e;
          if (col < p.N) {
            mp = fmaxf(mp, zp[0][j][4 * g + e]);
            mq = fmaxf(mq, zq[0][j][4 * g + e]);
          }
        }
    mp = fmaxf(mp, __shfl_xor(mp, 32, 64));
    mq = fmaxf(mq, __shfl_xor(mq, 32, 64));
    float* red = (float*)smem;  // [WM][2][32][3]
    lds_write_barrier();        // the k loop's stage buffers are free
    if (lane < 32) {
      red[((wm * 2 + wn) * 32 + lane) * 3 + 0] = mp;
      red[((wm * 2 + wn) * 32 + lane) * 3 + 1] = mq;
    }
    lds_write_barrier();
    const int rl = lane & 31;
    mp = fmaxf(red[((wm * 2) * 32 + rl) * 3 + 0], red[((wm * 2 + 1) * 32 + rl) * 3 + 0]);
    mq = fmaxf(red[((wm * 2) * 32 + rl) * 3 + 1], red[((wm * 2 + 1) * 32 + rl) * 3 + 1]);
    float sp = 0.f, sa = 0.f, sq = 0.f;
#pragma unroll
    for (int j = 0; j < CFG::TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t col = t.n0 + wn * CFG::WTN + j * 32 + 8 * g + 4 * (lane >> 5) + e;
          if (col < p.N) {
            const float x = zp[0][j][4 * g + e], y = zq[0][j][4 * g + e];
            const float ex = kl_exp(x - mp);
            sp += ex;
            sa = fmaf(ex, x - y, sa);
            sq += kl_exp(y - mq);
          }
        }
    sp += __shfl_xor(sp, 32, 64);
    sa += __shfl_xor(sa, 32, 64);
    sq += __shfl_xor(sq, 32, 64);
    lds_write_barrier();
    if (lane < 32) {
      red[((wm * 2 + wn) * 32 + lane) * 3 + 0] = sp;
      red[((wm * 2 + wn) * 32 + lane) * 3 + 1] = sa;
      red[((wm * 2 + wn) * 32 + lane) * 3 + 2] = sq;
    }
    lds_write_barrier();
    const int64_t row = t.m0 + wm * 32 + rl;
    if (wn == 0 && lane < 32 && row < t.M) {
      const float* r0 = red + ((wm * 2) * 32 + rl) * 3;
      const float* r1 = red + ((wm * 2 + 1) * 32 + rl) * 3;
      float* dst = a.part + (row * a.n_tiles + a.tile_base + t.n0 / CFG::BN) * 5;
      dst[0] = mp;
      dst[1] = r0[0] + r1[0];
      dst[2] = r0[1] + r1[1];
      dst[3] = mq;
      dst[4] = r0[2] + r1[2];
    }
  }
};

// Backward epilogue: G[row, col] = (e^{z_q - logZ_q} - e^{z_p - logZ_p}) g[row] in bf16 for
// col < width, zero for width <= col < kpad (the contraction padding).
struct EpiKLGrad {
  static constexpr int LDS_BYTES = 0;
  struct Args {
    const float* stats;
    const float* g;
    bf16_t* G;
    int64_t ldg, width, kpad;
  };
  template <class CFG>
  __device__ static void run(const GemmArgs& p, const Args& a, const TileJob& t, int wm, int wn, int tid,
                             f32x16 (&zp)[CFG::TM][CFG::TN], f32x16 (&zq)[CFG::TM][CFG::TN], char*) {
    static_assert(CFG::TM == 1 && CFG::WTM == 32, "one 32-row MFMA tile per wave");
    const int lane = tid & 63;
    const int64_t row = t.m0 + wm * 32 + (lane & 31);
    if (row >= t.M) return;
    const float* st = a.stats + row * 5;
    const float lzp = st[0] + logf(st[1]), lzq = st[3] + logf(st[4]);
    const float gn = a.g[row];
#pragma unroll
    for (int j = 0; j < CFG::TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t col = t.n0 + wn * CFG::WTN + j * 32 + 8 * g + 4 * (lane >> 5);
        if (col >= a.kpad) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = col + e < a.width ? (kl_exp(zq[0][j][4 * g + e] - lzq) - kl_exp(zp[0][j][4 * g + e] - lzp)) * gn : 0.f;
        *(uint2*)(a.G + row * a.ldg + col) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      }
  }
};

// stats[n] and kl[n] from the n_tiles partials of row n: one wave per row, lanes merge
// tiles lane, lane + 64, ... in order, then an xor tree (the merge is symmetric, so every
// lane holds the same result). Grid cdiv(N, 4) x 256.
__global__ __launch_bounds__(256) void k_kl_merge(const float* __restrict__ part, int64_t N, int64_t n_tiles,
                                                  float* __restrict__ stats, float* __restrict__ kl) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;
  float mp = -INFINITY, sp = 0.f, sa = 0.f, mq = -INFINITY, sq = 0.f;
  for (int64_t t = lane; t < n_tiles; t += 64) {
    const float* q = part + (row * n_tiles + t) * 5;
    kl_merge(mp, sp, sa, mq, sq, q[0], q[1], q[2], q[3], q[4]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    kl_merge(mp, sp, sa, mq, sq, __shfl_xor(mp, off, 64), __shfl_xor(sp, off, 64), __shfl_xor(sa, off, 64),
             __shfl_xor(mq, off, 64), __shfl_xor(sq, off, 64));
  if (lane == 0) {
    float* st = stats + row * 5;
    st[0] = mp, st[1] = sp, st[2] = sa, st[3] = mq, st[4] = sq;
    kl[row] = sa / sp - (mp + logf(sp)) + (mq + logf(sq));
  }
}

// dst[c][r] = src[r][c] for bf16 src [R, Cc] into rows of ldd >= R, zeroing r in [R, ldd).
__global__ __launch_bounds__(256) void k_kl_transpose(const bf16_t* __restrict__ src, int64_t R, int64_t Cc,
                                                      bf16_t* __restrict__ dst, int64_t ldd) {
  __shared__ bf16_t tile[64][66];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int64_t r = r0 + i, c = c0 + tx;
    tile[i][tx] = (r < R && c < Cc) ? src[r * Cc + c] : (bf16_t)0;
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (c < Cc && r < ldd) dst[c * ldd + r] = tile[tx][i];
  }
}

struct KLFused {
  float* part;  // [N, n_tiles, 5]
  bf16_t* G;    // [N, cw]
  bf16_t* hT;   // [d, Vp], Vp = V rounded up to 8
  float* sk;    // the input-gradient product's contraction slices
  int64_t n_tiles, Vp;
  int splits;
  size_t sk_bytes, total;
};

// Contraction slices of the input-gradient product d_act += G @ head: its N x d output has
// few 128 x 128 tiles (384 at 8192 x 768: three quarters of one round of two blocks per
// CU), so it is split into the fewest slices (at most 8, each at least 1024 deep) that
// fill whole rounds to 90%.
static int kl_dact_splits(int64_t N, int64_t d, int64_t kw) {
  const int64_t tiles = cdiv(N, 128) * cdiv(d, 128);
  int best = 1;
  double best_eff = 0.0;
  for (int sp = 1; sp <= 8 && (sp == 1 || kw / sp >= 1024); ++sp) {
    const int64_t work = tiles * sp;
    const double eff = (double)work / (double)(cdiv(work, 512) * 512);
    if (eff > best_eff + 1e-9) {
      best = sp;
      best_eff = eff;
    }
    if (eff >= 0.9) break;
  }
  return best;
}

static KLFused kl_fused_plan(int64_t N, int64_t d, int64_t V, int n_chunks, char* base) {
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const KLChunks K = kl_chunks(PD_DTYPE_BF16, V, n_chunks);
  KLFused P;
  P.n_tiles = 0;
  for (int64_t c = 0; c < K.nc; ++c) P.n_tiles += cdiv(K.width(c, V), CfgDtl::BN);
  P.Vp = (V + 7) & ~(int64_t)7;
  size_t off = 0;
  P.part = (float*)(base + off);
  off += up((size_t)N * P.n_tiles * 5 * 4);
  P.G = (bf16_t*)(base + off);
  off += up((size_t)N * K.cw * 2);
  P.hT = (bf16_t*)(base + off);
  // + 64 columns: the input-gradient product reads each chunk's k range in 64-wide
  // stages from a column offset, so its last row may read up to 63 elements past hT
  off += up((size_t)d * P.Vp * 2 + 64 * 2);
  P.splits = kl_dact_splits(N, d, (K.cw + 7) & ~(int64_t)7);
  P.sk_bytes = P.splits > 1 ? gemm_splitk_ws_bytes(N, d, (K.cw + 7) & ~(int64_t)7, P.splits) : 0;
  P.sk = (float*)(base + off);
  off += up(P.sk_bytes);
  P.total = off;
  return P;
}

// Tiles of the fused passes: with one head for both sides (a tied head, as in the LM
// step) 128 positions x 256 vocab columns, whose stage (A | B | A2, 64 KB) carries half
// the operand bytes per MFMA of the 128 x 128 tile; with two heads 128 x 128.
typedef DtlCfg<128, 256, 4, 2, 2> CfgKLWide;
static int64_t kl_tiles(const KLChunks& K, int64_t V, int bn) {
  int64_t n = 0;
  for (int64_t c = 0; c < K.nc; ++c) n += cdiv(K.width(c, V), bn);
  return n;
}
template <class CFG, bool SHARED, class EPI>
static void kl_dual_launch(const GemmArgs& a, const typename EPI::Args& ea, int64_t d, hipStream_t s) {
  const dim3 grid((unsigned)cdiv(a.N, CFG::BN), (unsigned)cdiv(a.M, CFG::BM));
  if (d % CFG::BK) hipLaunchKernelGGL((k_gemm_dtl_dual<CFG, true, EPI, SHARED>), grid, dim3(CFG::NT), 0, s, a, ea);
  else hipLaunchKernelGGL((k_gemm_dtl_dual<CFG, false, EPI, SHARED>), grid, dim3(CFG::NT), 0, s, a, ea);
}

static int kl_fused_fits(int64_t N, int64_t d, int64_t V) {
  return cdiv(N, CfgDtl::BM) <= 65535 && dtl_fits(N, d, V, d) && cdiv(d, 64) <= 65535 && cdiv(V, 64) <= 65535;
}

}  // namespace pd

using namespace pd;

extern "C" {

size_t pd_streamed_kl_workspace_size(int dtype, int64_t N, int64_t d, int64_t V, int n_chunks) {
  if (N <= 0 || d <= 0 || V <= 0 || n_chunks <= 0 || V % n_chunks) return 0;
  if (dtype == PD_DTYPE_BF16) return kl_fused_plan(N, d, V, n_chunks, nullptr).total;
  return kl_plan(dtype, N, d, V, n_chunks, nullptr).total;
}

int pd_streamed_kl_fwd(int dtype, int64_t N, int64_t d, int64_t V, int n_chunks, const void* act_masked,
                       const void* head_masked, const void* act_clean, const void* head_clean, float* position_kl,
                       float* stats, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = kl_check(dtype, N, d, V, n_chunks, act_masked, head_masked, act_clean, head_clean, "pd_streamed_kl_fwd");
  if (rc) return rc;
  if (!position_kl || !stats) return fail(PD_EINVAL, "pd_streamed_kl_fwd: outputs required");
  hipStream_t s = (hipStream_t)stream;
  const KLChunks K = kl_chunks(dtype, V, n_chunks);
  if (dtype == PD_DTYPE_BF16) {
    if (!kl_fused_fits(N, d, V)) return fail(PD_EUNSUPPORTED, "pd_streamed_kl_fwd: too large");
    if (!workspace || workspace_bytes < kl_fused_plan(N, d, V, n_chunks, nullptr).total)
      return fail(PD_EWORKSPACE, "pd_streamed_kl_fwd: workspace too small");
    const KLFused F = kl_fused_plan(N, d, V, n_chunks, (char*)workspace);
    const bool shared = head_masked == head_clean;
    const int bn = shared ? CfgKLWide::BN : CfgDtl::BN;
    const int64_t n_tiles = kl_tiles(K, V, bn);  // <= F.n_tiles (the plan counts 128-wide tiles)
    int64_t tile_base = 0;
    for (int64_t c = 0; c < K.nc; ++c) {
      const int64_t w = K.width(c, V);
      const bf16_t* hc = (const bf16_t*)head_clean + c * K.cw * d;
      const bf16_t* hm = (const bf16_t*)head_masked + c * K.cw * d;
      GemmArgs a{N, w, d, (const bf16_t*)act_clean, d, hc, d, nullptr, 0, 1.f, 0.f, nullptr, 0, 0, 0, 0,
                 (const bf16_t*)act_masked, hm, nullptr};
      const EpiKLStats::Args ea{F.part, n_tiles, tile_base};
      if (shared) kl_dual_launch<CfgKLWide, true, EpiKLStats>(a, ea, d, s);
      else kl_dual_launch<CfgDtl, false, EpiKLStats>(a, ea, d, s);
      tile_base += cdiv(w, bn);
    }
    hipLaunchKernelGGL(k_kl_merge, dim3((unsigned)cdiv(N, 4)), dim3(256), 0, s, F.part, N, n_tiles, stats,
                       position_kl);
    return check_launch("pd_streamed_kl_fwd");
  }
  if (!workspace || workspace_bytes < kl_plan(dtype, N, d, V, n_chunks, nullptr).total)
    return fail(PD_EWORKSPACE, "pd_streamed_kl_fwd: workspace too small");
  KLPlan P = kl_plan(dtype, N, d, V, n_chunks, (char*)workspace);
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
  hipStream_t s = (hipStream_t)stream;
  const KLChunks K = kl_chunks(dtype, V, n_chunks);
  if (dtype == PD_DTYPE_BF16) {
    if (!kl_fused_fits(N, d, V)) return fail(PD_EUNSUPPORTED, "pd_streamed_kl_bwd: too large");
    if (!workspace || workspace_bytes < kl_fused_plan(N, d, V, n_chunks, nullptr).total)
      return fail(PD_EWORKSPACE, "pd_streamed_kl_bwd: workspace too small");
    const KLFused F = kl_fused_plan(N, d, V, n_chunks, (char*)workspace);
    // masked head^T [d, Vp] (columns past V zero): the input-gradient product's K-contiguous operand
    hipLaunchKernelGGL(k_kl_transpose, dim3((unsigned)cdiv(d, 64), (unsigned)cdiv(F.Vp, 64)), dim3(256), 0, s,
                       (const bf16_t*)head_masked, V, d, F.hT, F.Vp);
    for (int64_t c = 0; c < K.nc; ++c) {
      const int64_t w = K.width(c, V), kpad = (w + 7) & ~(int64_t)7;
      const bf16_t* hc = (const bf16_t*)head_clean + c * K.cw * d;
      const bf16_t* hm = (const bf16_t*)head_masked + c * K.cw * d;
      GemmArgs a{N, w, d, (const bf16_t*)act_clean, d, hc, d, nullptr, 0, 1.f, 0.f, nullptr, 0, 0, 0, 0,
                 (const bf16_t*)act_masked, hm, nullptr};
      const EpiKLGrad::Args ea{stats, g_position, F.G, K.cw, w, kpad};
      if (head_masked == head_clean) kl_dual_launch<CfgKLWide, true, EpiKLGrad>(a, ea, d, s);
      else kl_dual_launch<CfgDtl, false, EpiKLGrad>(a, ea, d, s);
      // d_act (+)= G [N, kpad] @ (head^T [d, c cw + kpad))^T
      if ((rc = gemm_splitk(N, d, kpad, F.G, K.cw, 0, F.hT + c * K.cw, F.Vp, 1, d_act_masked, d, PD_DTYPE_F32,
                            c == 0 ? 0.f : 1.f, F.sk, F.sk_bytes, stream, F.splits)))
        return rc;
    }
    return check_launch("pd_streamed_kl_bwd");
  }
  if (!workspace || workspace_bytes < kl_plan(dtype, N, d, V, n_chunks, nullptr).total)
    return fail(PD_EWORKSPACE, "pd_streamed_kl_bwd: workspace too small");
  KLPlan P = kl_plan(dtype, N, d, V, n_chunks, (char*)workspace);
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
