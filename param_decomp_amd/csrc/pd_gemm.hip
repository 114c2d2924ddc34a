// GEMM kernels for the masked-component path (gfx950), v_mfma_f32_32x32x16_bf16.
//
// bf16 products run on the buffer-fed kernel of pd_gemm_dtl.hpp in every operand layout
// (an MN-contiguous operand is transposed on its way out of LDS): 128x128x64 tiles, 8
// waves of 32x64, two stages, two blocks per CU; 256x256 tiles (one block per CU) once the
// grid has at least 256 of them.
//
// Operands beyond the buffer kernel's 31-bit addressing: the register-staged kernel
// below. LDS holds both operands
// K-contiguous ([rows][BK+8]; the 144-byte row stride makes a wave's 16-byte fragment
// reads of 16 consecutive rows hit 16 distinct 4-bank groups); an operand whose global
// layout is MN-contiguous is transposed in registers (4 k-rows x 8 elements per thread)
// on its way into LDS. Two tile configurations:
//   BIG   256x256x64, 8 waves (2x4), 128x64 per wave (4x2 MFMA tiles), 144 KB LDS
//   SMALL 128x128x64, 4 waves (2x2), 64x64 per wave, for grids the big tile leaves
//         under-occupied (fewer than ~200 tiles on 256 CUs).
//
// Dense launches use an XCD-aware tile order: workgroups are dispatched round-robin
// over the 8 XCDs, so the linear id is remapped so each XCD's share is a compact
// 8-row-grouped region (fewer distinct A/B panels per XCD-local L2).
//
// Four problem mappings share the kernels:
//   DENSE     C = alpha*op(A)@op(B) + beta*C                  (x@V, acts@U, transposes)
//   GROUPED   out[rows_e] = lhs[rows_e] @ rhs[e], ragged rows  (pd/routed/experts.py:326-348)
//   GROUPED_K out[e] = lhs[rows_e]^T @ dout[rows_e]            (pd/routed/experts.py:209-280)
//   BATCHED   C[z] = op(A[z]) @ op(B[z]), per-operand strides  (per-block einsums,
//                                                              pd/core/linear_plan.py:149-160)
// Group offsets live on the device; blocks locate their group by scanning them, so no
// host synchronization is needed.
#include <algorithm>

#include "pd_gemm_dtl.hpp"

namespace pd {

typedef __attribute__((__vector_size__(4 * sizeof(short)))) short bf16x4;

constexpr int BK = 64, LDS_PAD = 8, LDS_STRIDE = BK + LDS_PAD;

template <int BM_, int BN_, int WM_, int WN_>
struct TileCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr int NT = WM_ * WN_ * 64;
  static constexpr int TM = BM_ / WM_ / 32, TN = BN_ / WN_ / 32;
  static constexpr int LDS_ELEMS = (BM_ + BN_) * LDS_STRIDE;
};
typedef TileCfg<256, 256, 2, 4> CfgBig;
typedef TileCfg<128, 128, 2, 2> CfgSmall;

// Loads one operand tile (ROWS x BK, rows = M or N index) into registers.
// KMAJ: global is [rows][K] (K contiguous): 16-byte chunks, 8 per row.
// !KMAJ: global is [K][rows] (rows contiguous): groups of 4 k-rows x 8 rows.
template <bool KMAJ, int ROWS, int NT>
struct TileLoader {
  static constexpr int NCH = KMAJ ? ROWS * BK / 8 / NT : (BK / 4) * (ROWS / 8) / NT;
  static constexpr int NV = KMAJ ? NCH : 4 * NCH;
  static_assert(NCH >= 1, "tile too small for the thread count");
  bf16x8 v[NV];
  // kmin: elements with k < kmin are zeroed (ragged-K groups whose tiles start at an
  // 8-aligned k below the group's first row); chunks are 8-aligned so loads stay 16 B.
  __device__ inline void load(const bf16_t* __restrict__ g, int64_t ld, int64_t row0, int64_t nrows, int64_t k0,
                              int64_t kmax, int tid, int64_t kmin = 0) {
    if (KMAJ) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        int id = tid + NT * i;
        int r = id >> 3, kc = id & 7;
        int64_t gr = row0 + r, gk = k0 + kc * 8;
        if (gr < nrows && gk < kmax) {
          v[i] = *(const bf16x8*)(g + gr * ld + gk);
          if (gk < kmin || gk + 8 > kmax) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (gk + e < kmin || gk + e >= kmax) v[i][e] = 0;
          }
        } else {
          v[i] = bf16x8{0, 0, 0, 0, 0, 0, 0, 0};
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        int id = tid + NT * i;
        int rc = id % (ROWS / 8), kg = id / (ROWS / 8);
        int64_t gr = row0 + rc * 8;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          int64_t gk = k0 + kg * 4 + q;
          if (gr < nrows && gk < kmax && gk >= kmin)
            v[4 * i + q] = *(const bf16x8*)(g + gk * ld + gr);
          else
            v[4 * i + q] = bf16x8{0, 0, 0, 0, 0, 0, 0, 0};
        }
      }
    }
  }
  __device__ inline void store(bf16_t* __restrict__ lds, int tid) {
    if (KMAJ) {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        int id = tid + NT * i;
        int r = id >> 3, kc = id & 7;
        *(bf16x8*)(lds + r * LDS_STRIDE + kc * 8) = v[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        int id = tid + NT * i;
        int rc = id % (ROWS / 8), kg = id / (ROWS / 8);
        // v[4i+q][e]: k-row q, element e (row rc*8+e). Write row rc*8+e with its 4 k values.
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          bf16x4 w = {v[4 * i][e], v[4 * i + 1][e], v[4 * i + 2][e], v[4 * i + 3][e]};
          *(bf16x4*)(lds + (rc * 8 + e) * LDS_STRIDE + kg * 4) = w;
        }
      }
    }
  }
};

template <class CFG, bool A_KMAJ, bool B_KMAJ, typename TC, int MODE>
__global__ __launch_bounds__(CFG::NT) void k_gemm_bf16(GemmArgs p) {
  constexpr int BM = CFG::BM, BN = CFG::BN, NT = CFG::NT, TM = CFG::TM, TN = CFG::TN;
  constexpr int WTM = BM / CFG::WM, WTN = BN / CFG::WN;  // wave tile
  __shared__ __attribute__((aligned(16))) bf16_t lds[2][CFG::LDS_ELEMS];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / CFG::WN, wn = wave % CFG::WN;

  TileJob t;
  if (!map_tile<BM, BN, MODE, TC>(p, lane, t)) return;
  const int64_t M = t.M, N = p.N, m0 = t.m0, n0 = t.n0, kend = t.kend;
  int64_t kbeg = t.kbeg;
  const bf16_t* A = t.A;
  const bf16_t* B = t.B;
  TC* C = (TC*)t.C;

  TileLoader<A_KMAJ, BM, NT> la;
  TileLoader<B_KMAJ, BN, NT> lb;
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // K-major operands read 16-byte chunks, so a ragged group's K walk starts at the
  // 8-aligned k below its first row and the loaders zero k < kmin.
  const int64_t kmin = kbeg;
  if (MODE == MODE_GROUPED_K && (A_KMAJ || B_KMAJ)) kbeg &= ~(int64_t)7;
  const int64_t nk = (kend - kbeg + BK - 1) / BK;
  if (nk > 0) {
    la.load(A, p.lda, m0, M, kbeg, kend, tid, kmin);
    lb.load(B, p.ldb, n0, N, kbeg, kend, tid, kmin);
    la.store(lds[0], tid);
    lb.store(lds[0] + BM * LDS_STRIDE, tid);
    __syncthreads();
  }
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int s = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      int64_t k0 = kbeg + (kt + 1) * BK;
      la.load(A, p.lda, m0, M, k0, kend, tid, kmin);
      lb.load(B, p.ldb, n0, N, k0, kend, tid, kmin);
    }
    const bf16_t* As = lds[s] + (wm * WTM + (lane & 31)) * LDS_STRIDE + (lane >> 5) * 8;
    const bf16_t* Bs = lds[s] + (BM + wn * WTN + (lane & 31)) * LDS_STRIDE + (lane >> 5) * 8;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *(const bf16x8*)(As + i * 32 * LDS_STRIDE + kk * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[j] = *(const bf16x8*)(Bs + j * 32 * LDS_STRIDE + kk * 16);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      la.store(lds[s ^ 1], tid);
      lb.store(lds[s ^ 1] + BM * LDS_STRIDE, tid);
    }
    __syncthreads();
  }

  // epilogue: lane holds column (lane&31) and rows 8*(v/4) + 4*(lane>>5) + (v&3)
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      int64_t col = n0 + wn * WTN + j * 32 + (lane & 31);
      if (col >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        int64_t row = m0 + wm * WTM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row < M) store1<TC>(C, row * p.ldc + col, p.alpha * acc[i][j][v], p.beta);
      }
    }
}

// fp32 GEMM on the fp32 matrix cores (v_mfma_f32_32x32x2_f32), any operand layout;
// blockIdx.z = batch, each operand advancing by its own stride (0 = shared).
//
// Every wave computes a 32x32 output tile from 32x16 A and 16x32 B chunks it streams
// through a private LDS slice: coalesced loads along whichever dimension is contiguous,
// stored k-major so each MFMA operand read is one conflict-free float per lane; the next
// chunk's loads are in flight (registers) while the current chunk's MFMAs run. Two block
// forms of 4 waves:
//   KW > 1  one 32x32 tile per block of KW waves, the contraction cut into KW consecutive
//           k ranges (multiples of 16), the waves' partial tiles added in wave order
//           through LDS: for small outputs over long contractions (the toy targets' weight
//           gradients, e.g. 1000x100 over 2048 rows), which would otherwise leave most
//           CUs idle (KW = 8 from K = 1024 on, else 4);
//   KW = 1  a 64x64 tile per block of 4 waves, each one 32x32 quarter over the whole
//           contraction.
// Either way the summation order is fixed: results are deterministic, no workspace.
constexpr int FT = 32, FK = 16;
template <int KW, bool TA, bool TB>
__global__ __launch_bounds__(KW > 1 ? 64 * KW : 256) void k_gemm_f32(int64_t M, int64_t N, int64_t K, const float* __restrict__ A,
                                                  int64_t lda, const float* __restrict__ B, int64_t ldb,
                                                  float* __restrict__ C, int64_t ldc, float alpha, float beta,
                                                  int64_t sA, int64_t sB, int64_t sC) {
  constexpr bool SPLIT = KW > 1;
  constexpr int NWV = SPLIT ? KW : 4, NT = 64 * NWV;
  __shared__ float As[NWV][FK][FT], Bs[NWV][FK][FT];  // [wave][k][m or n]
  __shared__ float red[SPLIT ? KW : 1][SPLIT ? FT * FT : 1];
  A += (int64_t)blockIdx.z * sA;
  B += (int64_t)blockIdx.z * sB;
  C += (int64_t)blockIdx.z * sC;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t bt = SPLIT ? FT : 2 * FT;
  const int64_t m0 = (int64_t)blockIdx.y * bt + (SPLIT ? 0 : (w >> 1) * FT);
  const int64_t n0 = (int64_t)blockIdx.x * bt + (SPLIT ? 0 : (w & 1) * FT);
  int64_t kb = 0, ke = K;
  if (SPLIT) {
    const int64_t kq = (K + KW * FK - 1) / (KW * FK) * FK;  // each wave's k range, a multiple of FK
    kb = (int64_t)w * kq;
    ke = kb + kq < K ? kb + kq : K;
  }
  f32x16 acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.f;
  // a lane's 8 loads of a chunk: along k (K-contiguous rows: row l/2, k (l%2)*8 + e) or
  // along m / n (MN-contiguous k-rows: k l/4, column (l%4)*8 + e)
  const int r_k = lane >> 1, c_k = (lane & 1) * 8, r_mn = lane >> 2, c_mn = (lane & 3) * 8;
  float ra[8], rb[8];
  uint32_t okm = 0;  // bit e: ra[e] in range; bit 8 + e: rb[e]
  // out-of-range elements load the operand's first element (always valid) and are zeroed
  // when stored to LDS: no branches, and nothing waits for the loads until the next
  // chunk's stores, so all 16 loads are in flight during this chunk's MFMAs
  auto load = [&](int64_t k0) {
    okm = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      int64_t off;
      bool ok;
      if constexpr (!TA) {  // A [M, K]
        const int64_t m = m0 + r_k, k = k0 + c_k + e;
        ok = m < M && k < ke;
        off = m * lda + k;
      } else {  // A [K, M]
        const int64_t k = k0 + r_mn, m = m0 + c_mn + e;
        ok = m < M && k < ke;
        off = k * lda + m;
      }
      ra[e] = A[ok ? off : 0];
      okm |= (uint32_t)ok << e;
      if constexpr (TB) {  // B [N, K]
        const int64_t n = n0 + r_k, k = k0 + c_k + e;
        ok = n < N && k < ke;
        off = n * ldb + k;
      } else {  // B [K, N]
        const int64_t k = k0 + r_mn, n = n0 + c_mn + e;
        ok = n < N && k < ke;
        off = k * ldb + n;
      }
      rb[e] = B[ok ? off : 0];
      okm |= (uint32_t)ok << (8 + e);
    }
  };
  if (kb < ke) load(kb);
  for (int64_t k0 = kb; k0 < ke; k0 += FK) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float av = (okm >> e) & 1u ? ra[e] : 0.f, bv = (okm >> (8 + e)) & 1u ? rb[e] : 0.f;
      if constexpr (!TA) As[w][c_k + e][r_k] = av;
      else As[w][r_mn][c_mn + e] = av;
      if constexpr (TB) Bs[w][c_k + e][r_k] = bv;
      else Bs[w][r_mn][c_mn + e] = bv;
    }
    if (k0 + FK < ke) load(k0 + FK);  // in flight during this chunk's MFMAs
    // the slice is this wave's alone: its LDS writes and reads stay in program order
    asm volatile("" ::: "memory");
#pragma unroll
    for (int kk = 0; kk < FK; kk += 2)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(As[w][kk + (lane >> 5)][lane & 31], Bs[w][kk + (lane >> 5)][lane & 31],
                                                 acc, 0, 0, 0);
    asm volatile("" ::: "memory");
  }
  // lane holds column lane & 31, rows 8 (v / 4) + 4 (lane / 32) + v % 4 of its tile
  if constexpr (SPLIT) {
#pragma unroll
    for (int v = 0; v < 16; ++v) red[w][(8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)) * FT + (lane & 31)] = acc[v];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < FT * FT / NT; ++q) {
      const int i = q * NT + tid, r = i / FT, c = i % FT;
      float sum = red[0][i];
#pragma unroll
      for (int x = 1; x < KW; ++x) sum += red[x][i];
      const int64_t gr = m0 + r, gc = n0 + c;
      if (gr < M && gc < N) C[gr * ldc + gc] = alpha * sum + (beta != 0.f ? beta * C[gr * ldc + gc] : 0.f);
    }
  } else {
    const int64_t gc = n0 + (lane & 31);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t gr = m0 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      if (gr < M && gc < N) C[gr * ldc + gc] = alpha * acc[v] + (beta != 0.f ? beta * C[gr * ldc + gc] : 0.f);
    }
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// fp32 GEMM, direct form: the MFMA operands go from memory straight into registers, no
// LDS stage. Within each 16-k batch the two lane halves take different k: half h supplies
// k = kc + 8h + s on MFMA step s (the two k slots of v_mfma_f32_32x32x2_f32), so
//   an MN-contiguous operand is one coalesced dword per lane and step (32 consecutive
//     floats per half), loaded through a buffer descriptor: an element outside the matrix
//     or the wave's k range gets an offset past the descriptor's end, which the hardware
//     returns as 0, so no value select follows a load and nothing waits for one until the
//     MFMA that reads it;
//   a K-contiguous operand is 8 consecutive floats per lane: two 16-byte loads when
//     `vec` says rows are 16-byte aligned and K % 4 == 0 (each 4-run then lies wholly
//     inside or outside the k range), else 8 dwords through the descriptor.
// The next batch's loads are in flight during this batch's 8 MFMAs. Block forms as in
// k_gemm_f32 (KW waves splitting the contraction of a 32x32 tile, or 4 waves of a 64x64
// tile); the summation order is fixed. Measured at the residual-MLP target's products
// (2048 rows, d 1000 / 100 / 50) it takes 0.35-0.6x the time of the LDS-staged form: those
// launches hold one or two waves per SIMD, and the LDS round trip per 16-k chunk was
// exposed latency there. Each operand must span fewer than 2^31 bytes (checked on the host).
template <int KW, bool TA, bool TB>
__global__ __launch_bounds__(KW > 1 ? 64 * KW : 256) void k_gemm_f32_direct(
    int64_t M, int64_t N, int64_t K, const float* __restrict__ A, int64_t lda, const float* __restrict__ B,
    int64_t ldb, float* __restrict__ C, int64_t ldc, float alpha, float beta, int64_t sA, int64_t sB, int64_t sC,
    int32_t bytes_a, int32_t bytes_b, int vec) {
  constexpr bool SPLIT = KW > 1;
  constexpr int NWV = SPLIT ? KW : 4, NT = 64 * NWV, S = 8;
  __shared__ float red[SPLIT ? KW : 1][SPLIT ? FT * FT : 1];
  A += (int64_t)blockIdx.z * sA;
  B += (int64_t)blockIdx.z * sB;
  C += (int64_t)blockIdx.z * sC;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5;
  const int64_t bt = SPLIT ? FT : 2 * FT;
  const int64_t m0 = (int64_t)blockIdx.y * bt + (SPLIT ? 0 : (w >> 1) * FT);
  const int64_t n0 = (int64_t)blockIdx.x * bt + (SPLIT ? 0 : (w & 1) * FT);
  int kb = 0, ke = (int)K;
  if (SPLIT) {
    const int kq = (int)((K + KW * FK - 1) / (KW * FK) * FK);
    kb = w * kq;
    ke = kb + kq < ke ? kb + kq : ke;
  }
  const uint32_t m = (uint32_t)(m0 + (lane & 31)), n = (uint32_t)(n0 + (lane & 31));
  const bool mok = m < M, nok = n < N;
  const uint32_t la = (uint32_t)lda, lb = (uint32_t)ldb;
  const auto rsa = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(A), (short)0, bytes_a, 0x00020000);
  const auto rsb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(B), (short)0, bytes_b, 0x00020000);
  // bit 31 set for an element outside the operand: offsets of in-range elements are < 2^31
  auto oob = [](bool ok) { return (uint32_t)(!ok) << 31; };
  auto load = [&](float (&a)[S], float (&b)[S], int kc) {
    const int k0 = kc + h * S;
    if (!TA && (vec & 1)) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float4 v = {0.f, 0.f, 0.f, 0.f};
        if (mok && k0 + 4 * q < ke) v = *(const float4*)(A + (int64_t)m * lda + k0 + 4 * q);
        a[4 * q] = v.x, a[4 * q + 1] = v.y, a[4 * q + 2] = v.z, a[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const uint32_t k = (uint32_t)(k0 + s), e = TA ? k * la + m : m * la + k;
        a[s] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsa, (e * 4u) | oob(mok & (k0 + s < ke)),
                                                                              0, 0));
      }
    }
    if (TB && (vec & 2)) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float4 v = {0.f, 0.f, 0.f, 0.f};
        if (nok && k0 + 4 * q < ke) v = *(const float4*)(B + (int64_t)n * ldb + k0 + 4 * q);
        b[4 * q] = v.x, b[4 * q + 1] = v.y, b[4 * q + 2] = v.z, b[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const uint32_t k = (uint32_t)(k0 + s), e = TB ? n * lb + k : k * lb + n;
        b[s] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsb, (e * 4u) | oob(nok & (k0 + s < ke)),
                                                                              0, 0));
      }
    }
  };
  f32x16 acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.f;
  auto mma = [&](const float (&a)[S], const float (&b)[S]) {
#pragma unroll
    for (int s = 0; s < S; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], acc, 0, 0, 0);
  };
  float a0[S], b0[S], a1[S], b1[S];
  if (kb < ke) load(a0, b0, kb);
  for (int kc = kb; kc < ke; kc += 2 * FK) {
    if (kc + FK < ke) load(a1, b1, kc + FK);
    mma(a0, b0);
    if (kc + FK >= ke) break;
    if (kc + 2 * FK < ke) load(a0, b0, kc + 2 * FK);
    mma(a1, b1);
  }
  // lane holds column lane & 31, rows 8 (v / 4) + 4 (lane / 32) + v % 4 of its tile
  if constexpr (SPLIT) {
#pragma unroll
    for (int v = 0; v < 16; ++v) red[w][(8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)) * FT + (lane & 31)] = acc[v];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < FT * FT / NT; ++q) {
      const int i = q * NT + tid, r = i / FT, c = i % FT;
      float sum = red[0][i];
#pragma unroll
      for (int x = 1; x < KW; ++x) sum += red[x][i];
      const int64_t gr = m0 + r, gc = n0 + c;
      if (gr < M && gc < N) C[gr * ldc + gc] = alpha * sum + (beta != 0.f ? beta * C[gr * ldc + gc] : 0.f);
    }
  } else {
    const int64_t gc = n0 + (lane & 31);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t gr = m0 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      if (gr < M && gc < N) C[gr * ldc + gc] = alpha * acc[v] + (beta != 0.f ? beta * C[gr * ldc + gc] : 0.f);
    }
  }
}

// The fp32 block form. Whole-contraction 64x64 tiles once they alone give >= 512 blocks
// (direct form up to K = 256, the LDS-staged one beyond), else 32x32 tiles with the
// contraction split over waves: the direct form with 16 waves from K = 512 on, else 8.
// The LDS-staged form also serves operands of 2^31 bytes or more.
template <bool TA, bool TB>
static void launch_gemm_f32_l(int64_t batch, int64_t M, int64_t N, int64_t K, const float* A, int64_t lda,
                              const float* B, int64_t ldb, float* C, int64_t ldc, float alpha, float beta, int64_t sA,
                              int64_t sB, int64_t sC, hipStream_t s) {
  const dim3 g32((unsigned)cdiv(N, FT), (unsigned)cdiv(M, FT), (unsigned)batch);
  const dim3 g64((unsigned)cdiv(N, 2 * FT), (unsigned)cdiv(M, 2 * FT), (unsigned)batch);
  const int64_t ea = 4 * (TA ? (K - 1) * lda + M : (M - 1) * lda + K);  // bytes one operand spans
  const int64_t eb = 4 * (TB ? (N - 1) * ldb + K : (K - 1) * ldb + N);
  const bool direct = ea < (int64_t(1) << 31) && eb < (int64_t(1) << 31);
  const bool big = cdiv(M, 2 * FT) * cdiv(N, 2 * FT) * batch >= 512;
  if (direct && (!big || K <= 256)) {
    const bool v4 = K % 4 == 0;
    const int vec = (!TA && v4 && lda % 4 == 0 && sA % 4 == 0 && aligned16(A) ? 1 : 0) |
                    (TB && v4 && ldb % 4 == 0 && sB % 4 == 0 && aligned16(B) ? 2 : 0);
#define PD_FD(KW_, G_)                                                                                               \
  hipLaunchKernelGGL((k_gemm_f32_direct<KW_, TA, TB>), G_, dim3(KW_ > 1 ? 64 * KW_ : 256), 0, s, M, N, K, A, lda, B, \
                     ldb, C, ldc, alpha, beta, sA, sB, sC, (int32_t)ea, (int32_t)eb, vec)
    if (big) PD_FD(1, g64);
    else if (K >= 512) PD_FD(16, g32);
    else PD_FD(8, g32);
#undef PD_FD
  } else if (big)
    hipLaunchKernelGGL((k_gemm_f32<1, TA, TB>), g64, dim3(256), 0, s, M, N, K, A, lda, B, ldb, C, ldc, alpha, beta, sA,
                       sB, sC);
  else if (K >= 1024)
    hipLaunchKernelGGL((k_gemm_f32<8, TA, TB>), g32, dim3(512), 0, s, M, N, K, A, lda, B, ldb, C, ldc, alpha, beta, sA,
                       sB, sC);
  else
    hipLaunchKernelGGL((k_gemm_f32<4, TA, TB>), g32, dim3(256), 0, s, M, N, K, A, lda, B, ldb, C, ldc, alpha, beta, sA,
                       sB, sC);
}

static void launch_gemm_f32(int64_t batch, int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, int ta,
                            const float* B, int64_t ldb, int tb, float* C, int64_t ldc, float alpha, float beta,
                            int64_t sA, int64_t sB, int64_t sC, hipStream_t s) {
  if (ta && tb) launch_gemm_f32_l<true, true>(batch, M, N, K, A, lda, B, ldb, C, ldc, alpha, beta, sA, sB, sC, s);
  else if (ta) launch_gemm_f32_l<true, false>(batch, M, N, K, A, lda, B, ldb, C, ldc, alpha, beta, sA, sB, sC, s);
  else if (tb) launch_gemm_f32_l<false, true>(batch, M, N, K, A, lda, B, ldb, C, ldc, alpha, beta, sA, sB, sC, s);
  else launch_gemm_f32_l<false, false>(batch, M, N, K, A, lda, B, ldb, C, ldc, alpha, beta, sA, sB, sC, s);
}

__global__ void k_zero_tail_rows(const int32_t* __restrict__ offsets, int E, int64_t J, int64_t width, int out_bytes,
                                 void* __restrict__ out) {
  int64_t start = offsets[E];
  if (start < 0) start = 0;
  int64_t n = (J - start) * width;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    if (out_bytes == 4)
      ((float*)out)[start * width + i] = 0.f;
    else
      ((bf16_t*)out)[start * width + i] = 0;
  }
}

template <class CFG, int MODE>
static int launch_bf16(const GemmArgs& a, bool a_kmaj, bool b_kmaj, int c_dtype, dim3 grid, hipStream_t s) {
#define PD_L(AK, BKM, TC) \
  hipLaunchKernelGGL((k_gemm_bf16<CFG, AK, BKM, TC, MODE>), grid, dim3(CFG::NT), 0, s, a)
  if (c_dtype == PD_DTYPE_F32) {
    if (a_kmaj && b_kmaj) PD_L(true, true, float);
    else if (a_kmaj) PD_L(true, false, float);
    else if (b_kmaj) PD_L(false, true, float);
    else PD_L(false, false, float);
  } else {
    if (a_kmaj && b_kmaj) PD_L(true, true, bf16_t);
    else if (a_kmaj) PD_L(true, false, bf16_t);
    else if (b_kmaj) PD_L(false, true, bf16_t);
    else PD_L(false, false, bf16_t);
  }
#undef PD_L
  return check_launch("pd_gemm bf16");
}

// host-side validation of a bf16 operand: contiguous dim a multiple of 8 elements,
// leading dim a multiple of 8, 16-byte aligned base.
static bool bf16_operand_ok(const void* ptr, int64_t ld, int64_t contig_extent) {
  return aligned16(ptr) && ld % 8 == 0 && contig_extent % 8 == 0;
}

// The big tile needs enough tiles to occupy the 256 CUs; otherwise use the small one.
static bool use_big_tile(int64_t M, int64_t N) { return cdiv(M, 256) * cdiv(N, 256) >= 192; }

template <class CFG, int MODE, bool AMN = false, bool BMN = false>
static int launch_dtl(const GemmArgs& a, int c_dtype, bool kedge, dim3 grid, hipStream_t s) {
#define PD_L(TC, KE) \
  hipLaunchKernelGGL((k_gemm_dtl<CFG, TC, MODE, KE, EpiStore, AMN, BMN>), grid, dim3(CFG::NT), 0, s, a, EpiStore::Args{})
  if (c_dtype == PD_DTYPE_F32) {
    if (kedge) PD_L(float, true);
    else PD_L(float, false);
  } else {
    if (kedge) PD_L(bf16_t, true);
    else PD_L(bf16_t, false);
  }
#undef PD_L
  return check_launch("pd_gemm bf16 (buffer-fed)");
}

// Any operand layout through the buffer-fed kernel (a_kmaj / b_kmaj: K-contiguous).
template <class CFG, int MODE>
static int launch_dtl_any(const GemmArgs& a, bool a_kmaj, bool b_kmaj, int c_dtype, bool kedge, dim3 grid,
                          hipStream_t s) {
  if (a_kmaj && b_kmaj) return launch_dtl<CFG, MODE, false, false>(a, c_dtype, kedge, grid, s);
  if (a_kmaj) return launch_dtl<CFG, MODE, false, true>(a, c_dtype, kedge, grid, s);
  if (b_kmaj) return launch_dtl<CFG, MODE, true, false>(a, c_dtype, kedge, grid, s);
  return launch_dtl<CFG, MODE, true, true>(a, c_dtype, kedge, grid, s);
}

// Every operand of the buffer-fed kernel within its 31-bit addressing range.
static bool dtl_fits_any(int64_t M, int64_t N, int64_t K, int64_t lda, bool a_kmaj, int64_t ldb, bool b_kmaj) {
  return (a_kmaj ? M * lda * 2 <= 0x7FFFFFFF : dtl_fits_mn(K, lda)) &&
         (b_kmaj ? N * ldb * 2 <= 0x7FFFFFFF : dtl_fits_mn(K, ldb));
}

}  // namespace pd

using namespace pd;

extern "C" {

int pd_gemm(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, int trans_a, const void* B,
            int64_t ldb, int trans_b, void* C, int64_t ldc, int c_dtype, float alpha, float beta, void* stream) {
  if (M < 0 || N < 0 || K < 0 || !A || !B || !C) return fail(PD_EINVAL, "pd_gemm: bad args");
  if (M == 0 || N == 0) return PD_OK;
  hipStream_t s = (hipStream_t)stream;
  if (cdiv(M, FT) > 65535 || cdiv(N, FT) > 65535) return fail(PD_EUNSUPPORTED, "pd_gemm: too large");
  if (dtype == PD_DTYPE_F32) {
    if (c_dtype != PD_DTYPE_F32) return fail(PD_EINVAL, "pd_gemm: fp32 path writes fp32");
    launch_gemm_f32(1, M, N, K, (const float*)A, lda, trans_a, (const float*)B, ldb, trans_b, (float*)C, ldc, alpha,
                    beta, 0, 0, 0, s);
    return check_launch("pd_gemm f32");
  }
  if (dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, "pd_gemm: dtype");
  bool a_kmaj = !trans_a, b_kmaj = trans_b;
  if (!bf16_operand_ok(A, lda, a_kmaj ? K : M) || !bf16_operand_ok(B, ldb, b_kmaj ? K : N))
    return fail(PD_EUNSUPPORTED, "pd_gemm: bf16 operands need 16B alignment and contiguous dims / ld % 8 == 0");
  GemmArgs a{M, N, K, (const bf16_t*)A, lda, (const bf16_t*)B, ldb, C, ldc, alpha, beta, nullptr, 0, 0, 0};
  if (dtl_fits_any(M, N, K, lda, a_kmaj, ldb, b_kmaj)) {
    // 256x256 tiles once they fill every CU at least once: they read each operand panel
    // half as often. Measured in the LM step (21.8 -> 21.1 ms) and the dense step (0.83 ->
    // 0.81 ms); only whole rounds of big tiles (no 1.5-round shapes) was 21.5 ms.
    if (cdiv(M, CfgDtlBig::BM) * cdiv(N, CfgDtlBig::BN) >= 256)
      return launch_dtl_any<CfgDtlBig, MODE_DENSE>(
          a, a_kmaj, b_kmaj, c_dtype, K % CfgDtlBig::BK != 0,
          dim3((unsigned)cdiv(N, CfgDtlBig::BN), (unsigned)cdiv(M, CfgDtlBig::BM)), s);
    return launch_dtl_any<CfgDtlRA, MODE_DENSE>(a, a_kmaj, b_kmaj, c_dtype, K % CfgDtlRA::BK != 0,
                                                dim3((unsigned)cdiv(N, CfgDtlRA::BN), (unsigned)cdiv(M, CfgDtlRA::BM)),
                                                s);
  }
  if (use_big_tile(M, N))
    return launch_bf16<CfgBig, MODE_DENSE>(a, a_kmaj, b_kmaj, c_dtype,
                                           dim3((unsigned)cdiv(N, 256), (unsigned)cdiv(M, 256)), s);
  return launch_bf16<CfgSmall, MODE_DENSE>(a, a_kmaj, b_kmaj, c_dtype,
                                           dim3((unsigned)cdiv(N, 128), (unsigned)cdiv(M, 128)), s);
}

int pd_gemm_strided_batched(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                            int64_t stride_a, int trans_a, const void* B, int64_t ldb, int64_t stride_b, int trans_b,
                            void* C, int64_t ldc, int64_t stride_c, int c_dtype, float alpha, float beta,
                            void* stream) {
  if (batch < 0 || M < 0 || N < 0 || K < 0 || stride_a < 0 || stride_b < 0 || stride_c < 0 || !A || !B || !C)
    return fail(PD_EINVAL, "pd_gemm_strided_batched: bad args");
  if (batch == 0 || M == 0 || N == 0) return PD_OK;
  hipStream_t s = (hipStream_t)stream;
  if (batch > 65535 || cdiv(M, FT) > 65535 || cdiv(N, FT) > 65535)
    return fail(PD_EUNSUPPORTED, "pd_gemm_strided_batched: too large");
  if (dtype == PD_DTYPE_F32) {
    if (c_dtype != PD_DTYPE_F32) return fail(PD_EINVAL, "pd_gemm_strided_batched: fp32 path writes fp32");
    launch_gemm_f32(batch, M, N, K, (const float*)A, lda, trans_a, (const float*)B, ldb, trans_b, (float*)C, ldc,
                    alpha, beta, stride_a, stride_b, stride_c, s);
    return check_launch("pd_gemm_strided_batched f32");
  }
  if (dtype != PD_DTYPE_BF16) return fail(PD_EINVAL, "pd_gemm_strided_batched: dtype");
  bool a_kmaj = !trans_a, b_kmaj = trans_b;
  if (!bf16_operand_ok(A, lda, a_kmaj ? K : M) || !bf16_operand_ok(B, ldb, b_kmaj ? K : N) || stride_a % 8 ||
      stride_b % 8)
    return fail(PD_EUNSUPPORTED,
                "pd_gemm_strided_batched: bf16 operands need 16B alignment, ld and batch strides % 8 == 0");
  GemmArgs a{M, N, K, (const bf16_t*)A, lda, (const bf16_t*)B, ldb, C, ldc, alpha, beta, nullptr, 0, stride_b,
             stride_c, stride_a};
  if (dtl_fits_any(M, N, K, lda, a_kmaj, ldb, b_kmaj))
    return launch_dtl_any<CfgDtlRA, MODE_BATCHED>(
        a, a_kmaj, b_kmaj, c_dtype, K % CfgDtlRA::BK != 0,
        dim3((unsigned)cdiv(N, CfgDtlRA::BN), (unsigned)cdiv(M, CfgDtlRA::BM), (unsigned)batch), s);
  return launch_bf16<CfgSmall, MODE_BATCHED>(
      a, a_kmaj, b_kmaj, c_dtype, dim3((unsigned)cdiv(N, 128), (unsigned)cdiv(M, 128), (unsigned)batch), s);
}

int pd_grouped_gemm(const void* lhs, const void* rhs, const int32_t* offsets, int64_t J, int E, int64_t K, int64_t N,
                    int trans_rhs, void* out, int out_dtype, void* stream) {
  return pd::grouped_gemm(lhs, rhs, offsets, J, E, K, N, trans_rhs, out, out_dtype, stream, true);
}

}  // extern "C"

namespace pd {

int grouped_gemm(const void* lhs, const void* rhs, const int32_t* offsets, int64_t J, int E, int64_t K, int64_t N,
                 int trans_rhs, void* out, int out_dtype, void* stream, bool zero_tail) {
  if (J < 0 || E <= 0 || K <= 0 || N <= 0 || !lhs || !rhs || !offsets || !out)
    return fail(PD_EINVAL, "pd_grouped_gemm: bad args");
  if (J == 0) return PD_OK;
  bool b_kmaj = trans_rhs != 0;
  if (!bf16_operand_ok(lhs, K, K) || !bf16_operand_ok(rhs, b_kmaj ? K : N, b_kmaj ? K : N))
    return fail(PD_EUNSUPPORTED, "pd_grouped_gemm: K and N must be multiples of 8 with 16B-aligned bases");
  hipStream_t s = (hipStream_t)stream;
  // zero rows past sum(group_sizes) (ragged_dot leaves them 0)
  if (zero_tail)
    hipLaunchKernelGGL(k_zero_tail_rows, dim3(256), dim3(256), 0, s, offsets, E, J, N,
                       out_dtype == PD_DTYPE_F32 ? 4 : 2, out);
  GemmArgs a{J, N, K, (const bf16_t*)lhs, K, (const bf16_t*)rhs, b_kmaj ? K : N, out, N, 1.f, 0.f, offsets, E,
             K * N, 0};
  static_assert(CfgDtl::BM == CfgSmall::BM && CfgDtl::BN == CfgSmall::BN, "one grid shape for both kernels");
  int64_t max_tiles = cdiv(J, CfgSmall::BM) + E;
  if (max_tiles > 65535) return fail(PD_EUNSUPPORTED, "pd_grouped_gemm: too many rows");
  dim3 grid((unsigned)cdiv(N, CfgSmall::BN), (unsigned)max_tiles);
  static_assert(CfgDtlRA::BM == CfgSmall::BM && CfgDtlRA::BN == CfgSmall::BN, "one grid shape for both kernels");
  if (b_kmaj && dtl_fits(J, K, N, K))
    return launch_dtl<CfgDtlRA, MODE_GROUPED>(a, out_dtype, K % CfgDtlRA::BK != 0, grid, s);
  if (!b_kmaj && dtl_fits(J, K, 0, 0) && dtl_fits_mn(K, N))  // each expert's rhs stored [K][N]
    return launch_dtl<CfgDtlRA, MODE_GROUPED, false, true>(a, out_dtype, K % CfgDtlRA::BK != 0, grid, s);
  return launch_bf16<CfgSmall, MODE_GROUPED>(a, true, b_kmaj, out_dtype, grid, s);
}

// ---------------------------------------------------------------- split contraction
// Slices: enough (tiles x slices >= 512, two blocks per CU) when the output has fewer than
// 384 128x128 tiles, each slice at least 512 deep, at most 16 slices; or the caller's
// count (`splits` > 0).
static int64_t splitk_slice(int64_t M, int64_t N, int64_t K, int splits_req = 0) {
  if (splits_req > 0) return splits_req < 2 || K < 2 * 64 ? 0 : cdiv(cdiv(K, splits_req), 64) * 64;
  const int64_t tiles = cdiv(M, CfgDtlRA::BM) * cdiv(N, CfgDtlRA::BN);
  if (tiles >= 384 || K < 1024) return 0;
  int64_t splits = std::min<int64_t>(std::min<int64_t>(cdiv(512, tiles), K / 512), 16);
  if (splits < 2) return 0;
  return cdiv(cdiv(K, splits), 64) * 64;
}

size_t gemm_splitk_ws_bytes(int64_t M, int64_t N, int64_t K, int splits) {
  const int64_t kc = splitk_slice(M, N, K, splits);
  return kc ? (size_t)cdiv(K, kc) * M * N * sizeof(float) : 0;
}

// C[m, n] = sum_z part[z][m, n] (+ beta * C), slices added in order; 4 columns per thread.
template <typename TC>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ part, int64_t M, int64_t N,
                                                       int splits, TC* __restrict__ C, int64_t ldc, float beta) {
  const int64_t n4 = N / 4, total = M * n4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / n4, c = (i % n4) * 4;
    float4 acc = *(const float4*)(part + m * N + c);
    for (int z = 1; z < splits; ++z) {
      const float4 v = *(const float4*)(part + ((int64_t)z * M + m) * N + c);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    const float o[4] = {acc.x, acc.y, acc.z, acc.w};
    store4<TC>(C, m * ldc + c, o, 1.f, beta);
  }
}

int gemm_splitk(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, int trans_a, const void* B, int64_t ldb,
                int trans_b, void* C, int64_t ldc, int c_dtype, float beta, void* ws, size_t ws_bytes, void* stream,
                int splits_req) {
  const int64_t kc = splitk_slice(M, N, K, splits_req);
  if (!kc || N % 4 || ldc % 4 || !aligned16(C))
    return pd_gemm(PD_DTYPE_BF16, M, N, K, A, lda, trans_a, B, ldb, trans_b, C, ldc, c_dtype, 1.f, beta, stream);
  const bool a_kmaj = !trans_a, b_kmaj = trans_b;
  if (!bf16_operand_ok(A, lda, a_kmaj ? K : M) || !bf16_operand_ok(B, ldb, b_kmaj ? K : N) ||
      !dtl_fits_any(M, N, K, lda, a_kmaj, ldb, b_kmaj))
    return fail(PD_EUNSUPPORTED, "gemm_splitk: operands");
  const int splits = (int)cdiv(K, kc);
  if (!ws || ws_bytes < (size_t)splits * M * N * sizeof(float)) return fail(PD_EWORKSPACE, "gemm_splitk: scratch");
  hipStream_t s = (hipStream_t)stream;
  GemmArgs a{M, N, K, (const bf16_t*)A, lda, (const bf16_t*)B, ldb, ws, N, 1.f, 0.f, nullptr, 0, 0, M * N, kc};
  const dim3 grid((unsigned)cdiv(N, CfgDtlRA::BN), (unsigned)cdiv(M, CfgDtlRA::BM), (unsigned)splits);
  int rc = launch_dtl_any<CfgDtlRA, MODE_SPLITK>(a, a_kmaj, b_kmaj, PD_DTYPE_F32, K % CfgDtlRA::BK != 0, grid, s);
  if (rc) return rc;
  const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(cdiv(M * N / 4, 256), 8192));
  if (c_dtype == PD_DTYPE_F32)
    hipLaunchKernelGGL(k_splitk_reduce<float>, dim3(blocks), dim3(256), 0, s, (const float*)ws, M, N, splits,
                       (float*)C, ldc, beta);
  else
    hipLaunchKernelGGL(k_splitk_reduce<bf16_t>, dim3(blocks), dim3(256), 0, s, (const float*)ws, M, N, splits,
                       (bf16_t*)C, ldc, beta);
  return check_launch("gemm_splitk reduce");
}

int gemm_nt_splitk(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* Bt, int64_t ldb, void* C,
                   int64_t ldc, int c_dtype, float beta, void* ws, size_t ws_bytes, void* stream) {
  return gemm_splitk(M, N, K, A, lda, 0, Bt, ldb, 1, C, ldc, c_dtype, beta, ws, ws_bytes, stream);
}

int grouped_gemm_pair(const void* lhs1, const void* rhsT1, void* out1, const void* lhs2, const void* rhsT2, void* out2,
                      const int32_t* offsets, int64_t J, int E, int64_t K, int64_t N, int out_dtype, void* stream) {
  if (J < 0 || E <= 0 || K <= 0 || N <= 0 || !lhs1 || !rhsT1 || !out1 || !lhs2 || !rhsT2 || !out2 || !offsets)
    return fail(PD_EINVAL, "grouped_gemm_pair: bad args");
  if (J == 0) return PD_OK;
  if (!bf16_operand_ok(lhs1, K, K) || !bf16_operand_ok(rhsT1, K, K) || !bf16_operand_ok(lhs2, K, K) ||
      !bf16_operand_ok(rhsT2, K, K))
    return fail(PD_EUNSUPPORTED, "grouped_gemm_pair: K must be a multiple of 8 with 16B-aligned bases");
  GemmArgs a{J, N, K, (const bf16_t*)lhs1, K, (const bf16_t*)rhsT1, K, out1, N, 1.f, 0.f, offsets, E, K * N, 0, 0,
             (const bf16_t*)lhs2, (const bf16_t*)rhsT2, out2};
  if (cdiv(J, CfgDtlRA::BM) + E > 65535) return fail(PD_EUNSUPPORTED, "grouped_gemm_pair: too many rows");
  if (!dtl_fits(J, K, N, K)) return fail(PD_EUNSUPPORTED, "grouped_gemm_pair: operands of 2 GiB or more");
  if (N >= 512)  // 256x256 tiles: measured faster for the paired N=512 products
    return launch_dtl<CfgDtlBig, MODE_GROUPED>(
        a, out_dtype, K % CfgDtlBig::BK != 0,
        dim3((unsigned)cdiv(N, CfgDtlBig::BN), (unsigned)(cdiv(J, CfgDtlBig::BM) + E), 2), (hipStream_t)stream);
  return launch_dtl<CfgDtlRA, MODE_GROUPED>(
      a, out_dtype, K % CfgDtlRA::BK != 0,
      dim3((unsigned)cdiv(N, CfgDtlRA::BN), (unsigned)(cdiv(J, CfgDtlRA::BM) + E), 2), (hipStream_t)stream);
}

int grouped_gemm_kcat(const void* lhs1, const void* rhs1, int64_t K1, const void* lhs2, const void* rhs2, int64_t K2,
                      void* out, const float* rs, const void* lhs1b, const void* rhs1b, const void* lhs2b,
                      const void* rhs2b, void* outb, const float* rs2, const int32_t* sort_idx, int k,
                      const int32_t* offsets, int64_t J, int E, int64_t N, void* stream) {
  const bool pair = lhs1b != nullptr;
  if (J < 0 || E <= 0 || E > 65535 || K1 <= 0 || K2 <= 0 || N <= 0 || k <= 0 || !lhs1 || !rhs1 || !lhs2 || !rhs2 ||
      !out || !rs || !sort_idx || !offsets || (pair && (!rhs1b || !lhs2b || !rhs2b || !outb)))
    return fail(PD_EINVAL, "grouped_gemm_kcat: bad args");
  if (J == 0) return PD_OK;
  const void* ops[8] = {lhs1, rhs1, lhs2, rhs2, pair ? lhs1b : lhs1, pair ? rhs1b : rhs1, pair ? lhs2b : lhs2,
                        pair ? rhs2b : rhs2};
  for (int i = 0; i < 8; ++i)
    if (!bf16_operand_ok(ops[i], (i & 2) ? K2 : K1, (i & 2) ? K2 : K1))
      return fail(PD_EUNSUPPORTED, "grouped_gemm_kcat: K1, K2 must be multiples of 8 with 16B-aligned bases");
  if (!aligned16(out) || (pair && !aligned16(outb)) || N % 8)
    return fail(PD_EUNSUPPORTED, "grouped_gemm_kcat: N % 8 and 16B-aligned outputs");
  if (!dtl_fits(J, K1, N, K1) || !dtl_fits(J, K2, N, K2))
    return fail(PD_EUNSUPPORTED, "grouped_gemm_kcat: operands of 2 GiB or more");
  if (cdiv(J, CfgDtlRA::BM) + E > 65535) return fail(PD_EUNSUPPORTED, "grouped_gemm_kcat: too many rows");
  GemmArgs a{J, N, K2, (const bf16_t*)lhs2, K2, (const bf16_t*)rhs2, K2, out, N, 1.f, 0.f, offsets, E, K2 * N, 0, 0,
             pair ? (const bf16_t*)lhs2b : nullptr, pair ? (const bf16_t*)rhs2b : nullptr, pair ? outb : nullptr};
  KcatArgs q{(const bf16_t*)lhs1, K1, (const bf16_t*)rhs1, K1, K1, nullptr, nullptr};
  q.A1b = pair ? (const bf16_t*)lhs1b : nullptr;
  q.B1b = pair ? (const bf16_t*)rhs1b : nullptr;
  q.strideB1 = K1 * N;
  q.rs_tok = rs;
  q.rs_tok2 = rs2 ? rs2 : rs;
  q.sort_idx = sort_idx;
  q.k = k;
  if (N >= 512) {  // 256x256 tiles, as for the paired N=512 products
    const dim3 grid((unsigned)cdiv(N, CfgDtlBig::BN), (unsigned)(cdiv(J, CfgDtlBig::BM) + E), pair ? 2u : 1u);
    hipLaunchKernelGGL((k_gemm_dtl_kcat<CfgDtlBig, bf16_t, false, false, EpiStore, MODE_GROUPED>), grid,
                       dim3(CfgDtlBig::NT), 0, (hipStream_t)stream, a, q, EpiStore::Args{});
  } else {
    const dim3 grid((unsigned)cdiv(N, CfgDtlRA::BN), (unsigned)(cdiv(J, CfgDtlRA::BM) + E), pair ? 2u : 1u);
    hipLaunchKernelGGL((k_gemm_dtl_kcat<CfgDtlRA, bf16_t, false, false, EpiStore, MODE_GROUPED>), grid,
                       dim3(CfgDtlRA::NT), 0, (hipStream_t)stream, a, q, EpiStore::Args{});
  }
  return check_launch("grouped_gemm_kcat");
}

int grouped_gemm_dw_pair(const void* lhs1, const void* dout1, void* out1, const void* lhs2, const void* dout2,
                         void* out2, const int32_t* offsets, int64_t J, int E, int64_t K, int64_t N, int out_dtype,
                         void* stream) {
  if (J < 0 || E <= 0 || K <= 0 || N <= 0 || !lhs1 || !dout1 || !out1 || !lhs2 || !dout2 || !out2 || !offsets)
    return fail(PD_EINVAL, "grouped_gemm_dw_pair: bad args");
  if (!bf16_operand_ok(lhs1, K, K) || !bf16_operand_ok(dout1, N, N) || !bf16_operand_ok(lhs2, K, K) ||
      !bf16_operand_ok(dout2, N, N))
    return fail(PD_EUNSUPPORTED, "grouped_gemm_dw_pair: K and N must be multiples of 8 with 16B-aligned bases");
  if (2 * (int64_t)E > 65535 || cdiv(K, CfgDtlRA::BM) > 65535) return fail(PD_EUNSUPPORTED, "grouped_gemm_dw_pair: size");
  if (!dtl_fits_mn(J, K) || !dtl_fits_mn(J, N))
    return fail(PD_EUNSUPPORTED, "grouped_gemm_dw_pair: operands of 2 GiB or more");
  // both operands MN-major (their rows are the contraction's jobs), 128x128 tiles
  GemmArgs a{K, N, J, (const bf16_t*)lhs1, K, (const bf16_t*)dout1, N, out1, N, 1.f, 0.f, offsets, E, 0, K * N, 0,
             (const bf16_t*)lhs2, (const bf16_t*)dout2, out2};
  dim3 grid((unsigned)cdiv(N, CfgDtlRA::BN), (unsigned)cdiv(K, CfgDtlRA::BM), (unsigned)(2 * E));
  return launch_dtl<CfgDtlRA, MODE_GROUPED_K, true, true>(a, out_dtype, true, grid, (hipStream_t)stream);
}

}  // namespace pd

extern "C" {

int pd_grouped_gemm_dw(const void* lhs, const void* dout, const int32_t* offsets, int64_t J, int E, int64_t K,
                       int64_t N, void* out, int out_dtype, void* stream) {
  if (J < 0 || E <= 0 || K <= 0 || N <= 0 || !lhs || !dout || !offsets || !out)
    return fail(PD_EINVAL, "pd_grouped_gemm_dw: bad args");
  if (!bf16_operand_ok(lhs, K, K) || !bf16_operand_ok(dout, N, N))
    return fail(PD_EUNSUPPORTED, "pd_grouped_gemm_dw: K and N must be multiples of 8 with 16B-aligned bases");
  if (E > 65535 || cdiv(K, CfgSmall::BM) > 65535) return fail(PD_EUNSUPPORTED, "pd_grouped_gemm_dw: E or K too large");
  // out[e] (M=K_in x N) = lhs[rows_e]^T (A stored [J,K]: M-contiguous) @ dout[rows_e] ([J,N])
  GemmArgs a{K, N, J, (const bf16_t*)lhs, K, (const bf16_t*)dout, N, out, N, 1.f, 0.f, offsets, E, 0, K * N};
  dim3 grid((unsigned)cdiv(N, CfgSmall::BN), (unsigned)cdiv(K, CfgSmall::BM), (unsigned)E);
  static_assert(CfgDtlRA::BM == CfgSmall::BM && CfgDtlRA::BN == CfgSmall::BN, "one grid shape for both kernels");
  if (dtl_fits_mn(J, K) && dtl_fits_mn(J, N))  // both operands MN-major: rows of lhs / dout are k
    return launch_dtl<CfgDtlRA, MODE_GROUPED_K, true, true>(a, out_dtype, true, grid, (hipStream_t)stream);
  return launch_bf16<CfgSmall, MODE_GROUPED_K>(a, false, false, out_dtype, grid, (hipStream_t)stream);
}

int pd_grouped_gemm_dw_kmajor(const void* lhsT, const void* doutT, const int32_t* offsets, int64_t J, int E,
                              int64_t K, int64_t N, void* out, int out_dtype, void* stream) {
  if (J < 0 || E <= 0 || K <= 0 || N <= 0 || !lhsT || !doutT || !offsets || !out)
    return fail(PD_EINVAL, "pd_grouped_gemm_dw_kmajor: bad args");
  if (!bf16_operand_ok(lhsT, J, J) || !bf16_operand_ok(doutT, J, J))
    return fail(PD_EUNSUPPORTED, "pd_grouped_gemm_dw_kmajor: J must be a multiple of 8 with 16B-aligned bases");
  if (E > 65535 || cdiv(K, CfgDtl::BM) > 65535) return fail(PD_EUNSUPPORTED, "pd_grouped_gemm_dw_kmajor: size");
  // (J == 0: every group has an empty k range, no loads are issued, out = 0)
  // out[e] (M=K x N) = lhsT[:, rows_e] (A stored [K, J]: K-major) @ doutT[:, rows_e]^T (B stored [N, J])
  GemmArgs a{K, N, J, (const bf16_t*)lhsT, J, (const bf16_t*)doutT, J, out, N, 1.f, 0.f, offsets, E, 0, K * N};
  if (!dtl_fits(K, J, N, J)) return fail(PD_EUNSUPPORTED, "pd_grouped_gemm_dw_kmajor: operands of 2 GiB or more");
  dim3 grid((unsigned)cdiv(N, CfgDtlRA::BN), (unsigned)cdiv(K, CfgDtlRA::BM), (unsigned)E);
  return launch_dtl<CfgDtlRA, MODE_GROUPED_K>(a, out_dtype, true, grid, (hipStream_t)stream);
}

}  // extern "C"
