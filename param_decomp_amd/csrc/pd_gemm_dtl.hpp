// bf16 GEMM with both operands K-contiguous, fed by direct global->LDS loads (gfx950).
//
// Operand tiles (rows x BK k, BK = 64 or 32) live in LDS as 2*BK-byte rows without
// padding. The 16-byte chunk c of row R sits at physical chunk c ^ swz(R), with
// swz(R) = (R & 7) ^ ((R >> 3) & 1) for 128-byte rows and (R >> 2) & 3 for 64-byte rows,
// so the 16 consecutive rows a quarter-wave fragment read touches cover all 64 banks.
// Each global_load_lds_dwordx4 moves one 1 KB block of whole rows: lane l writes physical
// chunk l % (BK/8) of row l / (BK/8), so it fetches the logical chunk the swizzle puts
// there.
//
// NS LDS stages form a ring with NS-1 k-tiles in flight: iteration kt waits (vmcnt) until
// its own tile has landed, one s_barrier makes it visible and frees the stage of tile
// kt-1, the loads of tile kt+NS-1 go out, then tile kt is consumed. The barrier is a bare
// s_barrier with compiler-only memory clobbers: a fenced __syncthreads would wait for
// every load in flight.
//
// The MFMA runs with the operands swapped (B rows as the 32-row "A" input), so each lane
// ends with 4 consecutive output columns of one row per 4 accumulators; the epilogue
// writes them as one 8-byte (bf16) or 16-byte (fp32) store.
//
// Rows past the operand extent are clamped to the last row (their outputs are never
// stored); k chunks past the row end are clamped in-bounds and, with k < kmin (ragged
// contraction groups start at an 8-aligned k), zeroed in the fragments of the edge tiles.
#pragma once

#include "pd_common.hpp"

namespace pd {

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((address_space(3))) void lds_void_t;

enum GemmMode { MODE_DENSE = 0, MODE_GROUPED = 1, MODE_GROUPED_K = 2, MODE_BATCHED = 3 };

struct GemmArgs {
  int64_t M, N, K;
  const bf16_t* A;
  int64_t lda;
  const bf16_t* B;
  int64_t ldb;
  void* C;
  int64_t ldc;
  float alpha, beta;
  const int32_t* offsets;  // [E+1] group offsets (grouped modes)
  int E;
  int64_t strideB;  // elements between consecutive groups' B (GROUPED, BATCHED)
  int64_t strideC;  // elements between consecutive groups' C (GROUPED_K, BATCHED)
  int64_t strideA;  // elements between consecutive batches' A (BATCHED; 0 = shared)
  // Grouped modes: a second problem of identical shape and group offsets in the same
  // launch (gridDim.z doubles; the upper half uses A2/B2/C2). NULL = one problem.
  const bf16_t* A2;
  const bf16_t* B2;
  void* C2;
};

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2): give
// XCD x a contiguous range [x*q + min(x, r), ...) of the linear tile order (q, r =
// total / 8, total % 8) so tiles that share operand panels share an L2.
__device__ inline int64_t xcd_contiguous(int64_t L, int64_t total) {
  const int64_t x = L & 7, q = total >> 3, r = total & 7;
  return x * q + (x < r ? x : r) + (L >> 3);
}

// Number of BM-row tiles of group g (0 past the last group or for empty groups).
__device__ inline int group_tiles(const int32_t* __restrict__ off, int g, int E, int BMv) {
  if (g >= E) return 0;
  const int sz = off[g + 1] - off[g];
  return sz > 0 ? (sz + BMv - 1) / BMv : 0;
}

__device__ inline int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}

// XCD-aware order for dense launches: XCD-contiguous ranges, then groups of 8 row
// tiles walked column by column.
__device__ inline void dense_tile(int& my, int& nx) {
  const int gx = gridDim.x, gy = gridDim.y;
  const int total = gx * gy;
  int L = blockIdx.y * gx + blockIdx.x;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
  const int GROUP = 8;
  const int g = L / (GROUP * gx);
  const int first = g * GROUP;
  const int gm = gy - first < GROUP ? gy - first : GROUP;
  const int within = L - g * GROUP * gx;
  my = first + within % gm;
  nx = within / gm;
}

// One block's output tile: rows [m0, M) of the block's problem (M is an absolute bound),
// columns from n0, contraction [kbeg, kend), and the operand/output bases.
struct TileJob {
  int64_t m0, n0, M, kbeg, kend;
  const bf16_t* A;
  const bf16_t* B;
  void* C;
};

// Maps this block to its tile (the four problem mappings); false = no work.
template <int BM, int BN, int MODE, typename TC>
__device__ inline bool map_tile(const GemmArgs& p, int lane, TileJob& t) {
  t.M = p.M;
  t.A = p.A;
  t.B = p.B;
  t.C = p.C;
  t.kbeg = 0;
  t.kend = p.K;
  if (MODE == MODE_DENSE) {
    int my, nx;
    dense_tile(my, nx);
    t.m0 = (int64_t)my * BM;
    t.n0 = (int64_t)nx * BN;
  } else if (MODE == MODE_GROUPED) {
    // Row tiles are enumerated over all groups in order. Every wave scans the groups'
    // tile counts 64 at a time (lane = group); the grid has a few spare rows of blocks,
    // so the XCD remap runs over the tiles that exist. With E <= 64 one load of the
    // offsets serves the count, the lookup and the group's row range.
    const int64_t gx = gridDim.x;
    const int64_t lin = ((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * gx + blockIdx.x;
    int e = -1, before = 0, tile = 0;
    int64_t off = 0, end = 0;
    auto pick = [&](int64_t per) -> bool {  // this block's (problem, column, row tile)
      if (lin >= per * gridDim.z) return false;
      int64_t lr = xcd_contiguous(lin, per * gridDim.z);
      if (lr >= per) {  // second problem of a paired launch
        lr -= per;
        t.A = p.A2;
        t.B = p.B2;
        t.C = p.C2;
      }
      t.n0 = (lr % gx) * BN;
      tile = (int)(lr / gx);
      return true;
    };
    if (p.E <= 64) {
      const bool in = lane < p.E;
      const int lo = in ? p.offsets[lane] : 0, hi = in ? p.offsets[lane + 1] : 0;
      const int nt = in && hi > lo ? (hi - lo + BM - 1) / BM : 0;
      const int incl = wave_incl_scan(nt, lane);
      if (!pick((int64_t)__shfl(incl, 63, 64) * gx)) return false;
      const unsigned long long hit = __ballot(incl > tile);
      if (!hit) return false;
      const int ln = __ffsll(hit) - 1;
      e = ln;
      before = __shfl(incl - nt, ln, 64);
      off = __shfl(lo, ln, 64);
      end = __shfl(hi, ln, 64);
    } else {
      int real = 0;
      for (int g0 = 0; g0 < p.E; g0 += 64)
        real += __shfl(wave_incl_scan(group_tiles(p.offsets, g0 + lane, p.E, BM), lane), 63, 64);
      if (!pick((int64_t)real * gx)) return false;
      for (int g0 = 0, base = 0; g0 < p.E; g0 += 64) {
        const int nt = group_tiles(p.offsets, g0 + lane, p.E, BM);
        const int incl = wave_incl_scan(nt, lane);
        const unsigned long long hit = __ballot(base + incl > tile);
        if (hit) {
          const int ln = __ffsll(hit) - 1;
          e = g0 + ln;
          before = base + __shfl(incl - nt, ln, 64);
          break;
        }
        base += __shfl(incl, 63, 64);
      }
      if (e < 0) return false;
      off = p.offsets[e];
      end = p.offsets[e + 1];
    }
    t.M = end < p.M ? end : p.M;  // absolute row bound, clamped to J
    t.m0 = off + (int64_t)(tile - before) * BM;
    if (t.m0 < 0) return false;
    t.B += (int64_t)e * p.strideB;
  } else if (MODE == MODE_BATCHED) {
    // blockIdx.z = batch; each operand advances by its own stride (0 = shared)
    const int64_t z = blockIdx.z;
    t.m0 = (int64_t)blockIdx.y * BM;
    t.n0 = (int64_t)blockIdx.x * BN;
    t.A = p.A + z * p.strideA;
    t.B = p.B + z * p.strideB;
    t.C = (TC*)p.C + z * p.strideC;
  } else {
    const int64_t gx = gridDim.x, gxy = gx * gridDim.y;
    const int64_t lin = ((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * gx + blockIdx.x;
    const int64_t lr = xcd_contiguous(lin, gxy * gridDim.z);
    int e = (int)(lr / gxy);
    if (e >= p.E) {  // second problem of a paired launch (gridDim.z = 2E)
      e -= p.E;
      t.A = p.A2;
      t.B = p.B2;
      t.C = p.C2;
    }
    t.m0 = (lr % gxy) / gx * BM;
    t.n0 = (lr % gx) * BN;
    t.kbeg = p.offsets[e] < 0 ? 0 : p.offsets[e];
    t.kend = p.offsets[e + 1] < p.K ? p.offsets[e + 1] : p.K;  // clamped to J
    if (t.kend < t.kbeg) t.kend = t.kbeg;
    t.C = (TC*)t.C + (int64_t)e * p.strideC;
  }
  return t.m0 < t.M && t.n0 < p.N;
}

template <int BM_, int BN_, int WM_, int WN_, int NS_, int RD_ = 0, int BK_ = 64>
struct DtlCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, NS = NS_, RD = RD_, BK = BK_;
  static constexpr int NW = WM_ * WN_, NT = NW * 64;
  static constexpr int WTM = BM_ / WM_, WTN = BN_ / WN_;  // wave tile
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int ROWB = 2 * BK_, RPI = 1024 / ROWB;  // LDS row bytes, rows per 1 KB load
  static constexpr int KK = BK_ / 16;                      // k16 MFMA steps per stage
  static constexpr int STAGE_BYTES = (BM_ + BN_) * ROWB;
  static constexpr int A_INSTS = BM_ / (RPI * NW), B_INSTS = BN_ / (RPI * NW);  // 1 KB loads per wave per stage
  static constexpr int INSTS = A_INSTS + B_INSTS;
  static_assert(BK_ == 64 || BK_ == 32, "stage depth");
  static_assert(BM_ % (RPI * NW) == 0 && BN_ % (RPI * NW) == 0, "every wave moves whole 1 KB row blocks");
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile is a multiple of 32x32");
  static_assert(NS_ >= 2 && INSTS * (NS_ - 2) < 64, "vmcnt range");
  static_assert(NS_ * STAGE_BYTES <= 160 * 1024, "LDS");
};

// s_waitcnt on the vector-memory counter only (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt_hi[15:14]; expcnt and lgkmcnt at their maxima = no wait).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Waits until at most `ahead` (<= A) stages of this wave's loads are still in flight.
template <int INSTS, int A>
__device__ inline void wait_stages(int ahead) {
  if constexpr (A > 0) {
    if (ahead >= A) {
      wait_vmcnt<A * INSTS>();
      return;
    }
    wait_stages<INSTS, A - 1>(ahead);
  } else {
    wait_vmcnt<0>();
  }
}

__device__ inline void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Physical-chunk swizzle of LDS row R (see the top of this file).
template <int BK>
__device__ inline int dtl_swz(int R) {
  return BK == 64 ? (R & 7) ^ ((R >> 3) & 1) : (R >> 2) & 3;
}

// Issues this wave's share of one operand tile (ROWS x BK k) into `dst`.
template <int ROWS, int NW, int BK>
__device__ inline void dtl_issue(char* dst, const bf16_t* __restrict__ g, int64_t ld, int64_t row0, int64_t rows,
                                 int64_t k0, int64_t kcap, int wave, int lane) {
  constexpr int CH = BK / 8, RPI = 64 / CH;
  const int rsub = lane / CH;
#pragma unroll
  for (int q = 0; q < ROWS / (RPI * NW); ++q) {
    const int R0 = (q * NW + wave) * RPI;
    const int c = (lane % CH) ^ dtl_swz<BK>(R0 + rsub);
    int64_t gr = row0 + R0 + rsub;
    gr = gr < rows ? gr : rows - 1;
    int64_t gk = k0 + c * 8;
    gk = gk < kcap ? gk : kcap;
    __builtin_amdgcn_global_load_lds((const void*)(g + gr * ld + gk), (lds_void_t*)(dst + R0 * 2 * BK), 16, 0, 0);
  }
}

__device__ inline void mask_frag(bf16x8& v, int64_t k, int64_t kmin, int64_t kend) {
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (k + e < kmin || k + e >= kend) v[e] = 0;
}

template <typename TC>
__device__ inline void store4(TC* C, int64_t idx, const float* v, float alpha, float beta);
template <>
__device__ inline void store4<float>(float* C, int64_t idx, const float* v, float alpha, float beta) {
  float4 o = {alpha * v[0], alpha * v[1], alpha * v[2], alpha * v[3]};
  if (beta != 0.f) {
    const float4 c = *(const float4*)(C + idx);
    o.x += beta * c.x;
    o.y += beta * c.y;
    o.z += beta * c.z;
    o.w += beta * c.w;
  }
  *(float4*)(C + idx) = o;
}
template <>
__device__ inline void store4<bf16_t>(bf16_t* C, int64_t idx, const float* v, float alpha, float beta) {
  float o[4] = {alpha * v[0], alpha * v[1], alpha * v[2], alpha * v[3]};
  if (beta != 0.f) {
    const uint2 c = *(const uint2*)(C + idx);
    o[0] += beta * bf16_to_f32((bf16_t)(c.x & 0xFFFF));
    o[1] += beta * bf16_to_f32((bf16_t)(c.x >> 16));
    o[2] += beta * bf16_to_f32((bf16_t)(c.y & 0xFFFF));
    o[3] += beta * bf16_to_f32((bf16_t)(c.y >> 16));
  }
  uint2 w;
  w.x = pack_bf16x2(o[0], o[1]);
  w.y = pack_bf16x2(o[2], o[3]);
  *(uint2*)(C + idx) = w;
}

template <typename TC>
__device__ inline void store1(TC* C, int64_t idx, float v, float beta);
template <>
__device__ inline void store1<float>(float* C, int64_t idx, float v, float beta) {
  C[idx] = beta != 0.f ? v + beta * C[idx] : v;
}
template <>
__device__ inline void store1<bf16_t>(bf16_t* C, int64_t idx, float v, float beta) {
  C[idx] = f32_to_bf16(beta != 0.f ? v + beta * bf16_to_f32(C[idx]) : v);
}

// Consumes one BK-k stage (BK/16 k16 steps). CFG::RD picks the LDS read schedule:
//   0  each step reads its fragments, then runs its MFMAs
//   1  all fragments of the stage are read before the first MFMA
//   2  software pipeline: step kk+1's reads are issued ahead of step kk's MFMAs
// EDGE zeroes k outside [kmin, kend).
template <class CFG, bool EDGE>
__device__ inline void dtl_read(const char* st, int a_off, int b_off, int sw, int lane, int kk, int64_t k0,
                                int64_t kmin, int64_t kend, bf16x8 (&af)[CFG::TM], bf16x8 (&bfr)[CFG::TN]) {
  const int coff = ((2 * kk + (lane >> 5)) ^ sw) << 4;
#pragma unroll
  for (int i = 0; i < CFG::TM; ++i) af[i] = *(const bf16x8*)(st + a_off + i * 32 * CFG::ROWB + coff);
#pragma unroll
  for (int j = 0; j < CFG::TN; ++j) bfr[j] = *(const bf16x8*)(st + b_off + j * 32 * CFG::ROWB + coff);
  if (EDGE) {
    const int64_t kf = k0 + kk * 16 + (lane >> 5) * 8;
#pragma unroll
    for (int i = 0; i < CFG::TM; ++i) mask_frag(af[i], kf, kmin, kend);
#pragma unroll
    for (int j = 0; j < CFG::TN; ++j) mask_frag(bfr[j], kf, kmin, kend);
  }
}

template <class CFG>
__device__ inline void dtl_mfma(const bf16x8 (&af)[CFG::TM], const bf16x8 (&bfr)[CFG::TN],
                                f32x16 (&acc)[CFG::TM][CFG::TN]) {
#pragma unroll
  for (int i = 0; i < CFG::TM; ++i)
#pragma unroll
    for (int j = 0; j < CFG::TN; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
}

template <class CFG, bool EDGE>
__device__ inline void dtl_stage(const char* st, int a_off, int b_off, int sw, int lane, int64_t k0, int64_t kmin,
                                 int64_t kend, f32x16 (&acc)[CFG::TM][CFG::TN]) {
  constexpr int TM = CFG::TM, TN = CFG::TN, KK = CFG::KK;
  if constexpr (CFG::RD == 1) {
    bf16x8 af[KK][TM], bfr[KK][TN];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) dtl_read<CFG, EDGE>(st, a_off, b_off, sw, lane, kk, k0, kmin, kend, af[kk], bfr[kk]);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) dtl_mfma<CFG>(af[kk], bfr[kk], acc);
  } else if constexpr (CFG::RD == 2) {
    bf16x8 af[2][TM], bfr[2][TN];
    dtl_read<CFG, EDGE>(st, a_off, b_off, sw, lane, 0, k0, kmin, kend, af[0], bfr[0]);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (kk + 1 < KK)
        dtl_read<CFG, EDGE>(st, a_off, b_off, sw, lane, kk + 1, k0, kmin, kend, af[(kk + 1) & 1], bfr[(kk + 1) & 1]);
      dtl_mfma<CFG>(af[kk & 1], bfr[kk & 1], acc);
    }
  } else {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      bf16x8 af[TM], bfr[TN];
      dtl_read<CFG, EDGE>(st, a_off, b_off, sw, lane, kk, k0, kmin, kend, af, bfr);
      dtl_mfma<CFG>(af, bfr, acc);
    }
  }
}

template <class CFG, typename TC, int MODE>
__global__ __launch_bounds__(CFG::NT) void k_gemm_dtl(GemmArgs p) {
  constexpr int BM = CFG::BM, TM = CFG::TM, TN = CFG::TN, NS = CFG::NS, NW = CFG::NW;
  __shared__ __attribute__((aligned(1024))) char smem[NS * CFG::STAGE_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / CFG::WN, wn = wave % CFG::WN;

  TileJob t;
  if (!map_tile<BM, CFG::BN, MODE, TC>(p, lane, t)) return;
  const int64_t kmin = t.kbeg;
  const int64_t kbeg = t.kbeg & ~(int64_t)7;  // 16-byte chunks start 8-aligned
  const int64_t kend = t.kend;
  const int64_t kcap = p.K - 8;  // last in-bounds chunk of a row
  constexpr int BK = CFG::BK, ROWB = CFG::ROWB;
  const int64_t nk = (kend - kbeg + BK - 1) / BK;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  auto issue = [&](int64_t kt) {
    char* st = smem + (int)(kt % NS) * CFG::STAGE_BYTES;
    const int64_t k0 = kbeg + kt * BK;
    dtl_issue<BM, NW, BK>(st, t.A, p.lda, t.m0, p.M, k0, kcap, wave, lane);
    dtl_issue<CFG::BN, NW, BK>(st + BM * ROWB, t.B, p.ldb, t.n0, p.N, k0, kcap, wave, lane);
  };

#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue(s);

  const int sw = dtl_swz<BK>(lane & 31);  // fragment rows sit at multiples of 32 plus lane & 31
  const int a_off = (wm * CFG::WTM + (lane & 31)) * ROWB;
  const int b_off = BM * ROWB + (wn * CFG::WTN + (lane & 31)) * ROWB;
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int64_t left = nk - 1 - kt;
    wait_stages<CFG::INSTS, NS - 2>((int)(left < NS - 2 ? left : NS - 2));
    lds_barrier();
    if (kt + NS - 1 < nk) issue(kt + NS - 1);
    const char* st = smem + (int)(kt % NS) * CFG::STAGE_BYTES;
    const int64_t k0 = kbeg + kt * BK;
    if (k0 < kmin || k0 + BK > kend)
      dtl_stage<CFG, true>(st, a_off, b_off, sw, lane, k0, kmin, kend, acc);
    else
      dtl_stage<CFG, false>(st, a_off, b_off, sw, lane, k0, kmin, kend, acc);
  }

  // lane holds row (lane & 31) of each 32x32 block and columns 8g + 4(lane >> 5) + 0..3
  TC* C = (TC*)t.C;
  const bool vec = (p.ldc & 3) == 0 && ((uintptr_t)C & (4 * sizeof(TC) - 1)) == 0;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t row = t.m0 + wm * CFG::WTM + i * 32 + (lane & 31);
    if (row >= t.M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t col = t.n0 + wn * CFG::WTN + j * 32 + 8 * g + 4 * (lane >> 5);
        const float v[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
        if (vec && col + 3 < p.N) {
          store4<TC>(C, row * p.ldc + col, v, p.alpha, p.beta);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (col + e < p.N) store1<TC>(C, row * p.ldc + col + e, p.alpha * v[e], p.beta);
        }
      }
    }
  }
}

}  // namespace pd
