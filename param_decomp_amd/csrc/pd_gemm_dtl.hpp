// bf16 GEMM with both operands K-contiguous, fed into LDS by buffer loads
// (buffer_load_dwordx4 ... lds, gfx950).
//
// Operand tiles (rows x 64 k) live in LDS as 128-byte rows without padding. The 16-byte
// chunk c of row R sits at physical chunk c ^ swz(R), swz(R) = (R & 7) ^ ((R >> 3) & 1),
// so the 16 consecutive rows a quarter-wave fragment read touches cover all 64 banks.
// Each load instruction moves one 1 KB block of whole rows: lane l writes physical chunk
// l % 8 of row l / 8, so it fetches the logical chunk the swizzle puts there.
//
// Operand addressing: a tile's rows start at a per-tile buffer descriptor base (scalar
// registers); each load's per-lane byte offset (row within the tile, swizzled chunk) is
// computed once per kernel and the stage's k position is added to it. The descriptor's
// record count ends at the operand's last row, so rows past the operand extent, and
// chunks past the end of its last row, load as zeros; their outputs are never stored.
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
// Ragged contraction groups start at the 64-aligned k below the group's first row, so
// every 128-byte piece of a K-major row a stage loads is one whole cache line (from an
// 8-aligned start each piece straddled two lines: 20-25% slower weight gradients); k
// outside [kmin, kend) is zeroed in the fragments of a tile's first and last stage.
//
// MN-major operands (stored [K][rows], rows contiguous: the B of x @ V and acts @ U, both
// operands of a weight gradient x^T @ g). A stage of such an operand holds its 64 k-rows
// of R = BM (or BN) elements, 2R bytes each; the 16-byte chunk c of k-row r sits at
// physical chunk c ^ (4 * (r & 3)). One 1 KB load moves 1024 / 2R whole k-rows (lane l
// writes physical chunk l % (R / 8) of k-row l / (R / 8)). Fragments come out of LDS
// already transposed by ds_read_b64_tr_b16: within each 16-lane group, output lane
// 4a + b receives element b of the 8 bytes read by source lanes a, a + 4, a + 8, a + 12.
// Source lane 16g + 4e + a reads k-row 8 (g >> 1) + 4h + e (h = 0, 1: the fragment's two
// halves), elements 16 (g & 1) + 4a .. + 3 of the fragment's 32 rows, so output lane l
// holds rows l & 31 at k 8 (l >> 5) + 4h .. + 3: the same fragment the K-major path reads
// with one ds_read_b128. The four k-rows one 16-lane group reads (r & 3 = e = 0..3) sit in
// four distinct 64-byte bank groups, so a half-wave's 256 bytes are conflict-free.
#pragma once

#include <type_traits>

#include "pd_common.hpp"

namespace pd {

typedef __attribute__((__vector_size__(8 * sizeof(short)))) short bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((address_space(3))) void lds_void_t;

enum GemmMode { MODE_DENSE = 0, MODE_GROUPED = 1, MODE_GROUPED_K = 2, MODE_BATCHED = 3, MODE_SPLITK = 4 };

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
  int prob;    // 0, or 1 for the second problem of a paired launch
  int64_t lin;  // GROUPED: the tile's index within its problem, < (J / BM + E) * ceil(N / BN)
  int e;        // GROUPED / GROUPED_K: the tile's group (expert); 0 otherwise
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
  t.prob = 0;
  t.lin = 0;
  t.e = 0;
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
        t.prob = 1;
      }
      t.n0 = (lr % gx) * BN;
      t.lin = lr;
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
    t.e = e;
  } else if (MODE == MODE_SPLITK) {
    // a dense tile, over the contraction slice blockIdx.z of gridDim.z equal slices of
    // p.strideA k each (a multiple of 64); slice z writes its partial sum to
    // C + z * strideC (the caller adds the slices in order)
    int my, nx;
    dense_tile(my, nx);
    t.m0 = (int64_t)my * BM;
    t.n0 = (int64_t)nx * BN;
    t.kbeg = (int64_t)blockIdx.z * p.strideA;
    t.kend = t.kbeg + p.strideA < p.K ? t.kbeg + p.strideA : p.K;
    t.C = (TC*)p.C + (int64_t)blockIdx.z * p.strideC;
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
      t.prob = 1;
    }
    t.m0 = (lr % gxy) / gx * BM;
    t.n0 = (lr % gx) * BN;
    t.kbeg = p.offsets[e] < 0 ? 0 : p.offsets[e];
    t.kend = p.offsets[e + 1] < p.K ? p.offsets[e + 1] : p.K;  // clamped to J
    if (t.kend < t.kbeg) t.kend = t.kbeg;
    t.C = (TC*)t.C + (int64_t)e * p.strideC;
    t.e = e;
  }
  return t.m0 < t.M && t.n0 < p.N;
}

// RA_: read every fragment of a stage from LDS before its first MFMA (false: one k16
// step ahead of the MFMAs).
template <int BM_, int BN_, int WM_, int WN_, int NS_, bool RA_ = false>
struct DtlCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, NS = NS_, BK = 64;
  static constexpr bool READ_ALL = RA_;
  static constexpr int NW = WM_ * WN_, NT = NW * 64;
  static constexpr int WTM = BM_ / WM_, WTN = BN_ / WN_;  // wave tile
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int ROWB = 128, RPI = 8;  // LDS row bytes, rows per 1 KB load
  static constexpr int KK = BK / 16;         // k16 MFMA steps per stage
  static constexpr int STAGE_BYTES = (BM_ + BN_) * ROWB;
  static constexpr int A_INSTS = BM_ / (RPI * NW), B_INSTS = BN_ / (RPI * NW);  // 1 KB loads per wave per stage
  static constexpr int INSTS = A_INSTS + B_INSTS;
  static_assert(NW % 2 == 0, "the swizzle parity of a wave's rows must not depend on the load index");
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

// A bare s_barrier: it orders the waves but waits for none of this wave's memory
// operations (gfx950 inserts no wait before s_barrier). It suffices where the LDS data
// the barrier publishes arrived by buffer-to-LDS loads already waited for (vmcnt), or
// where it only frees LDS whose reads this wave has consumed.
__device__ inline void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// A barrier after which every LDS access (ds_read / ds_write) any wave made before it has
// completed: LDS written before it is visible to all, LDS read before it is free to
// overwrite. This wave's LDS operations complete first (lgkmcnt = 0; the gfx9 s_waitcnt
// fields vmcnt [3:0] + [15:14] and expcnt [6:4] stay at their maxima), then the s_barrier.
__device__ inline void lds_write_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Physical-chunk swizzle of LDS row R (see the top of this file).
__device__ inline int dtl_swz(int R) { return (R & 7) ^ ((R >> 3) & 1); }

__device__ inline int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ inline int64_t uni64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// 128x128x64 tiles, 8 waves (4x2, 32x64 per wave), 2 LDS stages (64 KB, two blocks per CU).
typedef DtlCfg<128, 128, 4, 2, 2> CfgDtl;
// The same tile reading a whole stage's fragments before its MFMAs: never slower, and
// 10-19% faster on the K=512 MoE shapes (measured per shape).
typedef DtlCfg<128, 128, 4, 2, 2, true> CfgDtlRA;
// 256x256x64 tiles, 8 waves of 64x128 (128 KB of LDS, one block per CU): fewer LDS
// bytes per MFMA; faster for the paired N=512 products and the paired weight gradients.
typedef DtlCfg<256, 256, 4, 2, 2> CfgDtlBig;

// The kernel addresses each operand through a 31-bit buffer record count (rows = M or N
// for a K-major operand; for an MN-major one, K plus the 128 k-rows a last stage may
// reach past it).
inline bool dtl_fits(int64_t rows_a, int64_t lda, int64_t rows_b, int64_t ldb) {
  return rows_a * lda * 2 <= 0x7FFFFFFF && rows_b * ldb * 2 <= 0x7FFFFFFF;
}
inline bool dtl_fits_mn(int64_t K, int64_t ld) { return (K + 128) * ld * 2 <= 0x7FFFFFFF; }

// Record count (bytes) of a raw buffer descriptor, clamped to the 31-bit range (the
// launchers keep every operand below 2 GiB).
__device__ inline int32_t buf_bytes(int64_t bytes) {
  return bytes > 0x7FFFFFFF ? 0x7FFFFFFF : (bytes < 0 ? 0 : (int32_t)bytes);
}

// Per-lane byte offsets of a wave's 1 KB row-block loads of one operand tile (relative
// to the tile's first row, k = 0): lane l fills physical chunk l % 8 of row l / 8 of the
// block, i.e. logical chunk (l % 8) ^ swz(row); the block of load q starts at row
// (q * NW + wave) * 8, so swz's parity bit is wave & 1 for every q.
template <int ROWS, int NW>
__device__ inline void dtl_offsets(uint32_t (&off)[ROWS / (8 * NW)], int64_t ld, int wave, int lane) {
  const int rsub = lane >> 3;
  const int c = (lane & 7) ^ rsub ^ (wave & 1);
#pragma unroll
  for (int q = 0; q < ROWS / (8 * NW); ++q) {
    const int64_t row = (int64_t)(q * NW + wave) * 8 + rsub;
    off[q] = (uint32_t)((row * ld + c * 8) * 2);
  }
}

// Per-lane byte offsets of a wave's 1 KB loads of an MN-major operand tile (R elements
// per k-row, relative to the tile's first column, k = 0): load q covers k-rows
// (q * NW + wave) * RPL .. + RPL - 1; lane l fills physical chunk l % CPR of k-row l / CPR.
template <int R, int NW>
__device__ inline void dtl_offsets_mn(uint32_t (&off)[R / (8 * NW)], int64_t ld, int wave, int lane) {
  static_assert(R >= 128 && R <= 512, "an MN-major tile row is 256..1024 bytes");
  constexpr int CPR = R / 8, RPL = 1024 / (2 * R);
  const int rsub = lane / CPR, pc = lane % CPR;
#pragma unroll
  for (int q = 0; q < R / (8 * NW); ++q) {
    const int64_t row = (int64_t)(q * NW + wave) * RPL + rsub;
    const int c = pc ^ (4 * (int)(row & 3));
    off[q] = (uint32_t)((row * ld + c * 8) * 2);
  }
}

// LDS byte offset (within the operand's stage region, kk = 0, first half) of the
// transposing reads of fragment i of an MN-major tile of R elements per k-row; wave_r =
// the wave tile's first element within the block tile (a multiple of 32).
template <int R>
__device__ inline int mn_frag_off(int wave_r, int i, int lane) {
  constexpr int RB = 2 * R;
  const int g = lane >> 4, e = (lane >> 2) & 3, a = lane & 3;
  const int c = ((wave_r >> 3) + 4 * i) ^ (4 * e);
  return (8 * (g >> 1) + e) * RB + (c + 2 * (g & 1) + (a >> 1)) * 16 + (a & 1) * 8;
}

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t* lds_v4i16_ptr;

// One fragment (rows lane & 31, k 8 (lane >> 5) .. + 7 of k16 step kk): MN: two transposing
// 8-byte reads; K-major: one 16-byte read at the lane's swizzled chunk coff.
template <bool MN, int R>
__device__ inline bf16x8 frag_load(const char* st, int off, int kk, int coff) {
  if constexpr (MN) {
    constexpr int RB = 2 * R;
    const char* q = st + off + kk * 16 * RB;
    const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(q));
    const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(q + 4 * RB));
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  } else {
    return *(const bf16x8*)(st + off + coff);
  }
}

// A wave's fragment offsets within a stage (A region first, then B), per operand layout.
template <class CFG, bool AMN, bool BMN>
struct FragOffs {
  int a[CFG::TM], b[CFG::TN];
  int sw;
  __device__ inline FragOffs(int wm, int wn, int lane) {
    sw = dtl_swz(lane & 31);  // K-major fragment rows sit at multiples of 32 plus lane & 31
#pragma unroll
    for (int i = 0; i < CFG::TM; ++i)
      a[i] = AMN ? mn_frag_off<CFG::BM>(wm * CFG::WTM, i, lane) : (wm * CFG::WTM + i * 32 + (lane & 31)) * CFG::ROWB;
#pragma unroll
    for (int j = 0; j < CFG::TN; ++j)
      b[j] = CFG::BM * CFG::ROWB +
             (BMN ? mn_frag_off<CFG::BN>(wn * CFG::WTN, j, lane) : (wn * CFG::WTN + j * 32 + (lane & 31)) * CFG::ROWB);
  }
};

// One stage of one operand at byte offset koff (the stage's k position) within each
// row. The descriptor spans [base, base + bytes) (stride 0); the whole offset goes in the
// per-lane register so the record-count check covers it.
template <int ROWS, int NW>
__device__ inline void dtl_issue(char* dst, const bf16_t* base, int32_t bytes, const uint32_t* off, uint32_t koff,
                                 int wave) {
  const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), (short)0, bytes, 0x00020000);
#pragma unroll
  for (int q = 0; q < ROWS / (8 * NW); ++q)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(dst + (q * NW + wave) * 8 * 128), 16, off[q] + koff,
                                             0, 0, 0);
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

// Fragment reads of k16 step kk of a stage; EDGE zeroes k outside [kmin, kend).
template <class CFG, bool EDGE, bool AMN, bool BMN>
__device__ inline void dtl_read(const char* st, const FragOffs<CFG, AMN, BMN>& fo, int lane, int kk, int64_t k0,
                                int64_t kmin, int64_t kend, bf16x8 (&af)[CFG::TM], bf16x8 (&bfr)[CFG::TN]) {
  const int coff = ((2 * kk + (lane >> 5)) ^ fo.sw) << 4;
#pragma unroll
  for (int i = 0; i < CFG::TM; ++i) af[i] = frag_load<AMN, CFG::BM>(st, fo.a[i], kk, coff);
#pragma unroll
  for (int j = 0; j < CFG::TN; ++j) bfr[j] = frag_load<BMN, CFG::BN>(st, fo.b[j], kk, coff);
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

// Consumes one 64-k stage (4 k16 steps), reading step kk+1's fragments ahead of step
// kk's MFMAs.
template <class CFG, bool EDGE, bool AMN, bool BMN>
__device__ inline void dtl_stage(const char* st, const FragOffs<CFG, AMN, BMN>& fo, int lane, int64_t k0,
                                 int64_t kmin, int64_t kend, f32x16 (&acc)[CFG::TM][CFG::TN]) {
  constexpr int TM = CFG::TM, TN = CFG::TN, KK = CFG::KK;
  if constexpr (CFG::READ_ALL) {
    // every fragment of the stage in flight at once; each MFMA then waits only for its
    // own reads, so the LDS latency of later steps hides behind earlier MFMAs
    bf16x8 af[KK][TM], bfr[KK][TN];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) dtl_read<CFG, EDGE>(st, fo, lane, kk, k0, kmin, kend, af[kk], bfr[kk]);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) dtl_mfma<CFG>(af[kk], bfr[kk], acc);
    return;
  }
  bf16x8 af[2][TM], bfr[2][TN];
  dtl_read<CFG, EDGE>(st, fo, lane, 0, k0, kmin, kend, af[0], bfr[0]);
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    if (kk + 1 < KK)
      dtl_read<CFG, EDGE>(st, fo, lane, kk + 1, k0, kmin, kend, af[(kk + 1) & 1], bfr[(kk + 1) & 1]);
    dtl_mfma<CFG>(af[kk & 1], bfr[kk & 1], acc);
  }
}

template <class CFG, typename TC>
__device__ inline void dtl_epilogue(const GemmArgs& p, const TileJob& t, int wm, int wn, int lane,
                                    f32x16 (&acc)[CFG::TM][CFG::TN]) {
  TC* C = (TC*)t.C;
  const bool vec = (p.ldc & 3) == 0 && ((uintptr_t)C & (4 * sizeof(TC) - 1)) == 0;
#pragma unroll
  for (int i = 0; i < CFG::TM; ++i) {
    const int64_t row = t.m0 + wm * CFG::WTM + i * 32 + (lane & 31);
    if (row >= t.M) continue;
#pragma unroll
    for (int j = 0; j < CFG::TN; ++j) {
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

// A tile written through LDS: the accumulators go to a row-major LDS image (rows padded
// by 16 bytes, so the 32 rows one write instruction touches spread over the banks), then
// every lane stores 16 contiguous bytes and each instruction covers whole output rows.
// Straight from the MFMA layout a store instruction writes 16 (bf16) or 32 (fp32) bytes
// into each of 32 rows; through LDS the tile's 128-byte lines are written whole, which
// measured 13-25% faster on the grouped products with bf16 outputs. The image holds
// BM / PASSES rows at a time (the stage ring is the space); in pass q the waves whose
// rows fall in it write. Values are rounded as the register path rounds them: the bf16
// image holds round(alpha * acc) (so beta must be 0), the fp32 image alpha * acc, to
// which the store pass adds beta * C.
template <class CFG, int ES>
struct StagedStore {
  static constexpr int RSB = CFG::BN * ES + 16;  // LDS bytes per image row
  static constexpr int RING = CFG::NS * CFG::STAGE_BYTES;
  static constexpr int PASSES = CFG::BM * RSB <= RING           ? 1
                                : CFG::BM / 2 * RSB <= RING     ? 2
                                : CFG::BM / 4 * RSB <= RING     ? 4
                                                                : 0;
  static constexpr int ROWS = PASSES ? CFG::BM / PASSES : 0;
  static constexpr bool OK = PASSES > 0 && ROWS % CFG::WTM == 0;  // a wave's rows fall in one pass
};

// Pass q of the staged image: the waves whose rows fall in it write alpha * acc (bf16
// rounded for ES == 2) into the row-major LDS image; a barrier before (the k loop's last
// reads, or the previous pass's reads of the image, are done) and after (the image is
// complete).
template <class CFG, int ES>
__device__ inline void staged_image_pass(float alpha, int q, int wm, int wn, int lane,
                                         f32x16 (&acc)[CFG::TM][CFG::TN], char* smem) {
  typedef StagedStore<CFG, ES> SS;
  lds_write_barrier();
  const int r0 = wm * CFG::WTM - q * SS::ROWS;
  if (r0 >= 0 && r0 < SS::ROWS) {
#pragma unroll
    for (int i = 0; i < CFG::TM; ++i) {
      char* rowp = smem + (r0 + i * 32 + (lane & 31)) * SS::RSB;
#pragma unroll
      for (int j = 0; j < CFG::TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int c = wn * CFG::WTN + j * 32 + 8 * g + 4 * (lane >> 5);
          const float v0 = alpha * acc[i][j][4 * g], v1 = alpha * acc[i][j][4 * g + 1];
          const float v2 = alpha * acc[i][j][4 * g + 2], v3 = alpha * acc[i][j][4 * g + 3];
          if constexpr (ES == 2) {
            *(uint2*)(rowp + c * 2) = uint2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
          } else {
            *(float4*)(rowp + c * 4) = float4{v0, v1, v2, v3};
          }
        }
    }
  }
  lds_write_barrier();
}

template <class CFG, typename TC>
__device__ inline void dtl_epilogue_staged(const GemmArgs& p, const TileJob& t, int wm, int wn, int tid,
                                           f32x16 (&acc)[CFG::TM][CFG::TN], char* smem) {
  constexpr int ES = sizeof(TC);
  typedef StagedStore<CFG, ES> SS;
  constexpr int EPC = 16 / ES;              // elements per 16-byte chunk
  constexpr int CPR = CFG::BN / EPC;        // chunks per output row
  constexpr int RPP = CFG::NT / CPR;        // rows one pass of the block's stores covers
  static_assert(CFG::NT % CPR == 0 && SS::ROWS % RPP == 0, "store passes");
  const int lane = tid & 63, rr = tid / CPR, cc = tid % CPR;
  TC* C = (TC*)t.C;
  const int64_t col = t.n0 + cc * EPC;
#pragma unroll
  for (int q = 0; q < SS::PASSES; ++q) {
    staged_image_pass<CFG, ES>(p.alpha, q, wm, wn, lane, acc, smem);
#pragma unroll
    for (int r = rr; r < SS::ROWS; r += RPP) {
      const int64_t row = t.m0 + q * SS::ROWS + r;
      if (row >= t.M || col >= p.N) continue;
      if constexpr (ES == 2) {
        *(uint4*)(C + row * p.ldc + col) = *(const uint4*)(smem + r * SS::RSB + cc * 16);
      } else {
        float4 o = *(const float4*)(smem + r * SS::RSB + cc * 16);
        if (p.beta != 0.f) {
          const float4 c = *(const float4*)(C + row * p.ldc + col);
          o.x += p.beta * c.x;
          o.y += p.beta * c.y;
          o.z += p.beta * c.z;
          o.w += p.beta * c.w;
        }
        *(float4*)(C + row * p.ldc + col) = o;
      }
    }
  }
}

// The epilogue is a policy: EPI::run(p, args, tile, wm, wn, tid, acc, smem) runs after the
// k loop with the LDS stage buffers still owned by the k loop (a policy that reuses
// them starts with a barrier); the block's LDS is max(stages, EPI::LDS_BYTES). EpiStore
// writes C = alpha * acc + beta * C: with 16-byte aligned rows and N a whole number of
// 16-byte chunks (and beta == 0 for a bf16 C) through the staged store, otherwise
// straight from the registers.
struct EpiStore {
  static constexpr int LDS_BYTES = 0;
  struct Args {};
  template <class CFG, typename TC>
  __device__ static void run(const GemmArgs& p, const Args&, const TileJob& t, int wm, int wn, int tid,
                             f32x16 (&acc)[CFG::TM][CFG::TN], char* smem) {
    constexpr int EPC = 16 / sizeof(TC);
    if constexpr (StagedStore<CFG, sizeof(TC)>::OK) {
      if ((sizeof(TC) == 4 || p.beta == 0.f) && p.ldc % EPC == 0 && p.N % EPC == 0 && ((uintptr_t)t.C & 15) == 0) {
        dtl_epilogue_staged<CFG, TC>(p, t, wm, wn, tid, acc, smem);
        return;
      }
    }
    dtl_epilogue<CFG, TC>(p, t, wm, wn, tid & 63, acc);
  }
};

// KEDGE: some stages cover k outside [kmin, kend) and are masked (ragged contraction
// groups, or K % 64 != 0). Only a tile's first and last stage can be such stages, so they
// are peeled off the main loop, which then has a single body: a branch between a masked
// and a plain stage inside the loop makes the compiler shuttle the accumulators between
// AGPRs and VGPRs on every iteration.
//
// AMN / BMN: A (or B) is MN-major, stored [K][M] (or [K][N]) with leading dimension lda
// (ldb) between k-rows.
template <class CFG, typename TC, int MODE, bool KEDGE, class EPI = EpiStore, bool AMN = false, bool BMN = false>
__global__ __launch_bounds__(CFG::NT) void k_gemm_dtl(GemmArgs p, typename EPI::Args ea) {
  constexpr int BM = CFG::BM, BN = CFG::BN, TM = CFG::TM, TN = CFG::TN, NS = CFG::NS, NW = CFG::NW;
  constexpr int BK = CFG::BK, ROWB = CFG::ROWB;
  constexpr int LDS = NS * CFG::STAGE_BYTES > EPI::LDS_BYTES ? NS * CFG::STAGE_BYTES : EPI::LDS_BYTES;
  __shared__ __attribute__((aligned(1024))) char smem[LDS];
  const int tid = threadIdx.x, lane = tid & 63, wave = uni(tid >> 6);
  const int wm = wave / CFG::WN, wn = wave % CFG::WN;

  TileJob t;
  if (!map_tile<BM, BN, MODE, TC>(p, lane, t)) return;
  // every tile field is wave-uniform; say so, so the descriptors stay in scalar registers
  const int64_t m0 = uni64(t.m0), n0 = uni64(t.n0);
  const int64_t kmin = uni64(t.kbeg), kend = uni64(t.kend);
  const int64_t kbeg = kmin & ~(int64_t)63;
  const int64_t nk = kend > kmin ? (kend - kbeg + BK - 1) / BK : 0;
  // a K-major tile starts at its first row, an MN-major one at its first column; either
  // descriptor ends at the operand's end (rows past M / N, or k-rows past K, load zeros;
  // an MN-major tile's columns past M / N only feed outputs that are never stored)
  const bf16_t* abase = (const bf16_t*)uni64((int64_t)(AMN ? t.A + m0 : t.A + m0 * p.lda));
  const bf16_t* bbase = (const bf16_t*)uni64((int64_t)(BMN ? t.B + n0 : t.B + n0 * p.ldb));
  const int32_t abytes = buf_bytes(AMN ? (p.K * p.lda - m0) * 2 : (p.M - m0) * p.lda * 2);
  const int32_t bbytes = buf_bytes(BMN ? (p.K * p.ldb - n0) * 2 : (p.N - n0) * p.ldb * 2);
  uint32_t offa[CFG::A_INSTS], offb[CFG::B_INSTS];
  if constexpr (AMN) dtl_offsets_mn<BM, NW>(offa, p.lda, wave, lane);
  else dtl_offsets<BM, NW>(offa, p.lda, wave, lane);
  if constexpr (BMN) dtl_offsets_mn<BN, NW>(offb, p.ldb, wave, lane);
  else dtl_offsets<BN, NW>(offb, p.ldb, wave, lane);
  // a stage's k position as a byte offset: along the row (K-major) or down k-rows (MN)
  const uint32_t kstep_a = AMN ? (uint32_t)(p.lda * 2) : 2u, kstep_b = BMN ? (uint32_t)(p.ldb * 2) : 2u;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  auto issue = [&](int64_t kt) {
    char* st = smem + (int)(kt % NS) * CFG::STAGE_BYTES;
    const uint32_t kpos = (uint32_t)(kbeg + kt * BK);
    dtl_issue<BM, NW>(st, abase, abytes, offa, kpos * kstep_a, wave);
    dtl_issue<BN, NW>(st + BM * ROWB, bbase, bbytes, offb, kpos * kstep_b, wave);
  };

#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue(s);

  const FragOffs<CFG, AMN, BMN> fo(wm, wn, lane);
  auto sync = [&](int64_t kt) {  // stage kt has landed and is visible; stage kt+NS-1 goes out
    const int64_t left = nk - 1 - kt;
    wait_stages<CFG::INSTS, NS - 2>((int)(left < NS - 2 ? left : NS - 2));
    lds_barrier();
    if (kt + NS - 1 < nk) issue(kt + NS - 1);
  };
  auto st_of = [&](int64_t kt) { return smem + (int)(kt % NS) * CFG::STAGE_BYTES; };
  if constexpr (KEDGE) {
    if (nk > 0) {
      sync(0);
      dtl_stage<CFG, true>(st_of(0), fo, lane, kbeg, kmin, kend, acc);
    }
    for (int64_t kt = 1; kt < nk - 1; ++kt) {
      sync(kt);
      dtl_stage<CFG, false>(st_of(kt), fo, lane, kbeg + kt * BK, kmin, kend, acc);
    }
    if (nk > 1) {
      sync(nk - 1);
      dtl_stage<CFG, true>(st_of(nk - 1), fo, lane, kbeg + (nk - 1) * BK, kmin, kend, acc);
    }
  } else {
    for (int64_t kt = 0; kt < nk; ++kt) {
      sync(kt);
      dtl_stage<CFG, false>(st_of(kt), fo, lane, kbeg + kt * BK, kmin, kend, acc);
    }
  }
  EPI::template run<CFG, TC>(p, ea, t, wm, wn, tid, acc, smem);
}

// Two products of one shape in one block, P1 = A @ B^T and P2 = A2 @ B2^T (dense, every
// operand K-contiguous with the same lda / ldb), for epilogues that need both tiles of the
// same (row, column) block at once. A stage holds A | B | A2 | B2 (B2 == B shares B's
// rows and skips their loads; with SHARED_B the caller guarantees B2 == B and a stage
// has no B2 region). EPI::run(p, ea, tile, wm, wn, tid, acc1, acc2, smem).
template <class CFG, bool KEDGE, class EPI, bool SHARED_B = false>
__global__ __launch_bounds__(CFG::NT) void k_gemm_dtl_dual(GemmArgs p, typename EPI::Args ea) {
  static_assert(CFG::NS == 2, "two LDS stages");
  constexpr int BM = CFG::BM, BN = CFG::BN, TM = CFG::TM, TN = CFG::TN, NW = CFG::NW;
  constexpr int BK = CFG::BK, ROWB = CFG::ROWB;
  constexpr int SB = (SHARED_B ? 2 * BM + BN : 2 * (BM + BN)) * ROWB;
  constexpr int LDS = 2 * SB > EPI::LDS_BYTES ? 2 * SB : EPI::LDS_BYTES;
  static_assert(2 * SB <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) char smem[LDS];
  const int tid = threadIdx.x, lane = tid & 63, wave = uni(tid >> 6);
  const int wm = wave / CFG::WN, wn = wave % CFG::WN;

  TileJob t;
  if (!map_tile<BM, BN, MODE_DENSE, float>(p, lane, t)) return;
  const int64_t m0 = uni64(t.m0), n0 = uni64(t.n0);
  const int64_t kmin = uni64(t.kbeg), kend = uni64(t.kend);
  const int64_t kbeg = kmin & ~(int64_t)63;
  const int64_t nk = kend > kmin ? (kend - kbeg + BK - 1) / BK : 0;
  const bool share_b = SHARED_B || p.B2 == p.B;
  const bf16_t* abase = (const bf16_t*)uni64((int64_t)(p.A + m0 * p.lda));
  const bf16_t* a2base = (const bf16_t*)uni64((int64_t)(p.A2 + m0 * p.lda));
  const bf16_t* bbase = (const bf16_t*)uni64((int64_t)(p.B + n0 * p.ldb));
  const bf16_t* b2base = (const bf16_t*)uni64((int64_t)(p.B2 + n0 * p.ldb));
  const int32_t abytes = buf_bytes((p.M - m0) * p.lda * 2), bbytes = buf_bytes((p.N - n0) * p.ldb * 2);
  uint32_t offa[CFG::A_INSTS], offb[CFG::B_INSTS];
  dtl_offsets<BM, NW>(offa, p.lda, wave, lane);
  dtl_offsets<BN, NW>(offb, p.ldb, wave, lane);

  f32x16 acc[TM][TN], acc2[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = acc2[i][j][v] = 0.f;

  auto issue = [&](int64_t kt) {
    char* st = smem + (int)(kt & 1) * SB;
    const uint32_t koff = (uint32_t)((kbeg + kt * BK) * 2);
    dtl_issue<BM, NW>(st, abase, abytes, offa, koff, wave);
    dtl_issue<BN, NW>(st + BM * ROWB, bbase, bbytes, offb, koff, wave);
    dtl_issue<BM, NW>(st + (BM + BN) * ROWB, a2base, abytes, offa, koff, wave);
    if (!share_b) dtl_issue<BN, NW>(st + (2 * BM + BN) * ROWB, b2base, bbytes, offb, koff, wave);
  };
  if (nk > 0) issue(0);

  const FragOffs<CFG, false, false> fo(wm, wn, lane);
  FragOffs<CFG, false, false> fo2 = fo;  // the second problem's A (and B) sit after the first's
#pragma unroll
  for (int i = 0; i < TM; ++i) fo2.a[i] += (BM + BN) * ROWB;
#pragma unroll
  for (int j = 0; j < TN; ++j) fo2.b[j] += share_b ? 0 : (BM + BN) * ROWB;
  auto sync = [&](int64_t kt) {
    wait_vmcnt<0>();
    lds_barrier();
    if (kt + 1 < nk) issue(kt + 1);
  };
  auto stage = [&](int64_t kt, auto edge) {
    constexpr bool E = decltype(edge)::value;
    const char* st = smem + (int)(kt & 1) * SB;
    dtl_stage<CFG, E>(st, fo, lane, kbeg + kt * BK, kmin, kend, acc);
    dtl_stage<CFG, E>(st, fo2, lane, kbeg + kt * BK, kmin, kend, acc2);
  };
  if constexpr (KEDGE) {
    if (nk > 0) {
      sync(0);
      stage(0, std::true_type{});
    }
    for (int64_t kt = 1; kt < nk - 1; ++kt) {
      sync(kt);
      stage(kt, std::false_type{});
    }
    if (nk > 1) {
      sync(nk - 1);
      stage(nk - 1, std::true_type{});
    }
  } else {
    for (int64_t kt = 0; kt < nk; ++kt) {
      sync(kt);
      stage(kt, std::false_type{});
    }
  }
  EPI::template run<CFG>(p, ea, t, wm, wn, tid, acc, acc2, smem);
}

// Two contractions into one accumulator, C = rs (.) (A1 @ op(B1)) + A2 @ op(B2): the
// k loop runs over A1's K1 columns, then A2's K2 (p.K), with rs, the per-row scale of
// the first product, applied to the accumulators in between. Every lane's 16 accumulators
// of a 32x32 MFMA tile sit in one output row, so the scale is one multiply per register.
// rs(t) = routed(t) ? (delta ? delta[t] : 0) : 1, routed(t) = !route || route[t] (delta
// bf16, or fp32 through delta_f): the
// blend weight of the target output x @ W^T in the masked linear (and of its cotangent).
// A1 and A2 are K-contiguous; B1MN / B2MN: the B operand is MN-major. The LDS stage ring
// runs straight through the segment boundary, so the second product's first stages
// load while the first product's last stage is consumed.
// MODE_GROUPED (job space of routed experts): rows are jobs sorted by expert, each B is an
// expert-major [E, N, K] stack (B1 advances by strideB1 per expert, B2 by p.strideB), an
// optional second problem of the same shape runs in the same launch (A1b, B1b with p.A2,
// p.B2, p.C2), and the row scale is per token, rs(row) = rs_tok[sort_idx[row] / k] (the
// second problem's from rs_tok2).
struct KcatArgs {
  const bf16_t* A1;
  int64_t lda1;
  const bf16_t* B1;
  int64_t ldb1;
  int64_t K1;
  const bf16_t* delta;
  const uint8_t* route;
  const bf16_t* A1b = nullptr;
  const bf16_t* B1b = nullptr;
  int64_t strideB1 = 0;
  const float* rs_tok = nullptr;
  const float* rs_tok2 = nullptr;
  const int32_t* sort_idx = nullptr;
  int k = 1;
  const float* delta_f = nullptr;  // fp32 per-row delta (dense mode; preferred over `delta`)
};

template <class CFG, typename TC, bool B1MN, bool B2MN, class EPI = EpiStore, int MODE = MODE_DENSE>
__global__ __launch_bounds__(CFG::NT) void k_gemm_dtl_kcat(GemmArgs p, KcatArgs q, typename EPI::Args ea) {
  constexpr int BM = CFG::BM, BN = CFG::BN, TM = CFG::TM, TN = CFG::TN, NS = CFG::NS, NW = CFG::NW;
  constexpr int BK = CFG::BK, ROWB = CFG::ROWB;
  constexpr int LDS = NS * CFG::STAGE_BYTES > EPI::LDS_BYTES ? NS * CFG::STAGE_BYTES : EPI::LDS_BYTES;
  __shared__ __attribute__((aligned(1024))) char smem[LDS];
  const int tid = threadIdx.x, lane = tid & 63, wave = uni(tid >> 6);
  const int wm = wave / CFG::WN, wn = wave % CFG::WN;

  TileJob t;
  if (!map_tile<BM, BN, MODE, TC>(p, lane, t)) return;
  const int64_t m0 = uni64(t.m0), n0 = uni64(t.n0);
  const int64_t K1 = q.K1, K2 = p.K;
  const int64_t nk1 = (K1 + BK - 1) / BK, nk = nk1 + (K2 + BK - 1) / BK;
  // the tile's segment-1 operands (its problem's, its expert's) and segment-2 operands
  // (map_tile placed t.A / t.B / t.C); selected by assignment, since a conditional over
  // the argument fields would take their address and move the arguments to scratch
  const bf16_t* A1 = q.A1;
  const bf16_t* B1 = q.B1;
  const float* rs_tok = q.rs_tok;
  if (t.prob) {
    A1 = q.A1b;
    B1 = q.B1b;
    rs_tok = q.rs_tok2;
  }
  B1 += (int64_t)t.e * q.strideB1;
  const bf16_t* a1 = (const bf16_t*)uni64((int64_t)(A1 + m0 * q.lda1));
  const bf16_t* b1 = (const bf16_t*)uni64((int64_t)(B1MN ? B1 + n0 : B1 + n0 * q.ldb1));
  const bf16_t* a2 = (const bf16_t*)uni64((int64_t)(t.A + m0 * p.lda));
  const bf16_t* b2 = (const bf16_t*)uni64((int64_t)(B2MN ? t.B + n0 : t.B + n0 * p.ldb));
  const int32_t a1bytes = buf_bytes((p.M - m0) * q.lda1 * 2), a2bytes = buf_bytes((p.M - m0) * p.lda * 2);
  const int32_t b1bytes = buf_bytes(B1MN ? (K1 * q.ldb1 - n0) * 2 : (p.N - n0) * q.ldb1 * 2);
  const int32_t b2bytes = buf_bytes(B2MN ? (K2 * p.ldb - n0) * 2 : (p.N - n0) * p.ldb * 2);
  uint32_t oa1[CFG::A_INSTS], ob1[CFG::B_INSTS], oa2[CFG::A_INSTS], ob2[CFG::B_INSTS];
  dtl_offsets<BM, NW>(oa1, q.lda1, wave, lane);
  dtl_offsets<BM, NW>(oa2, p.lda, wave, lane);
  if constexpr (B1MN) dtl_offsets_mn<BN, NW>(ob1, q.ldb1, wave, lane);
  else dtl_offsets<BN, NW>(ob1, q.ldb1, wave, lane);
  if constexpr (B2MN) dtl_offsets_mn<BN, NW>(ob2, p.ldb, wave, lane);
  else dtl_offsets<BN, NW>(ob2, p.ldb, wave, lane);
  const uint32_t ks1 = B1MN ? (uint32_t)(q.ldb1 * 2) : 2u, ks2 = B2MN ? (uint32_t)(p.ldb * 2) : 2u;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // One issue path whose operands are selected value by value: two calls under an
  // if / else get merged into one call over selected array addresses, which moves the
  // offset arrays to scratch and the descriptors into vector registers.
  auto issue = [&](int64_t kt) {
    char* st = smem + (int)(kt % NS) * CFG::STAGE_BYTES;
    const bool s1 = kt < nk1;
    const uint32_t kpos = (uint32_t)((s1 ? kt : kt - nk1) * BK);
    uint32_t oa[CFG::A_INSTS], ob[CFG::B_INSTS];
#pragma unroll
    for (int i = 0; i < CFG::A_INSTS; ++i) oa[i] = s1 ? oa1[i] : oa2[i];
#pragma unroll
    for (int i = 0; i < CFG::B_INSTS; ++i) ob[i] = s1 ? ob1[i] : ob2[i];
    dtl_issue<BM, NW>(st, s1 ? a1 : a2, s1 ? a1bytes : a2bytes, oa, kpos * 2, wave);
    dtl_issue<BN, NW>(st + BM * ROWB, s1 ? b1 : b2, s1 ? b1bytes : b2bytes, ob, kpos * (s1 ? ks1 : ks2), wave);
  };
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nk) issue(s);

  const FragOffs<CFG, false, B1MN> fo1(wm, wn, lane);
  const FragOffs<CFG, false, B2MN> fo2(wm, wn, lane);
  auto sync = [&](int64_t kt) {
    const int64_t left = nk - 1 - kt;
    wait_stages<CFG::INSTS, NS - 2>((int)(left < NS - 2 ? left : NS - 2));
    lds_barrier();
    if (kt + NS - 1 < nk) issue(kt + NS - 1);
  };
  auto st_of = [&](int64_t kt) { return smem + (int)(kt % NS) * CFG::STAGE_BYTES; };
  // segment 1 (k tail masked in its last stage)
  const bool tail1 = (K1 % BK) != 0;
  for (int64_t kt = 0; kt < nk1 - (tail1 ? 1 : 0); ++kt) {
    sync(kt);
    dtl_stage<CFG, false>(st_of(kt), fo1, lane, kt * BK, 0, K1, acc);
  }
  if (tail1) {
    sync(nk1 - 1);
    dtl_stage<CFG, true>(st_of(nk1 - 1), fo1, lane, (nk1 - 1) * BK, 0, K1, acc);
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t row = m0 + wm * CFG::WTM + i * 32 + (lane & 31);
    float rs = 1.f;
    if (rs_tok) rs = row < t.M ? rs_tok[q.sort_idx[row] / q.k] : 0.f;
    else if (row < p.M && (!q.route || q.route[row]))
      rs = q.delta_f ? q.delta_f[row] : (q.delta ? bf16_to_f32(q.delta[row]) : 0.f);
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] *= rs;
  }
  // segment 2
  const bool tail2 = (K2 % BK) != 0;
  for (int64_t kt = nk1; kt < nk - (tail2 ? 1 : 0); ++kt) {
    sync(kt);
    dtl_stage<CFG, false>(st_of(kt), fo2, lane, (kt - nk1) * BK, 0, K2, acc);
  }
  if (tail2) {
    sync(nk - 1);
    dtl_stage<CFG, true>(st_of(nk - 1), fo2, lane, (nk - 1 - nk1) * BK, 0, K2, acc);
  }
  EPI::template run<CFG, TC>(p, ea, t, wm, wn, tid, acc, smem);
}

// Dense C = A [M, K] @ B^T (B stored [N, K], both K-contiguous, lda/ldb % 8 == 0, 16-byte
// aligned) with the epilogue policy EPI (its Args carry everything beyond C's tile).
template <class EPI, typename TC, bool BMN = false>
inline int launch_dense_epi(const GemmArgs& a, const typename EPI::Args& ea, hipStream_t s, const char* what) {
  if (a.M * a.lda * 2 > 0x7FFFFFFF || !(BMN ? dtl_fits_mn(a.K, a.ldb) : a.N * a.ldb * 2 <= 0x7FFFFFFF))
    return fail(PD_EUNSUPPORTED, std::string(what) + ": operands of 2 GiB or more");
  if ((a.M + CfgDtlRA::BM - 1) / CfgDtlRA::BM > 65535 || (a.N + CfgDtlRA::BN - 1) / CfgDtlRA::BN > 65535)
    return fail(PD_EUNSUPPORTED, std::string(what) + ": too large");
  const dim3 grid((unsigned)((a.N + CfgDtlRA::BN - 1) / CfgDtlRA::BN), (unsigned)((a.M + CfgDtlRA::BM - 1) / CfgDtlRA::BM));
  if (a.K % CfgDtlRA::BK)
    hipLaunchKernelGGL((k_gemm_dtl<CfgDtlRA, TC, MODE_DENSE, true, EPI, false, BMN>), grid, dim3(CfgDtlRA::NT), 0, s,
                       a, ea);
  else
    hipLaunchKernelGGL((k_gemm_dtl<CfgDtlRA, TC, MODE_DENSE, false, EPI, false, BMN>), grid, dim3(CfgDtlRA::NT), 0, s,
                       a, ea);
  return check_launch(what);
}

// C = rs (.) (A1 @ op(B1)) + A2 @ op(B2) (k_gemm_dtl_kcat) with the epilogue policy EPI.
template <class EPI, typename TC, bool B1MN, bool B2MN>
inline int launch_kcat_epi(const GemmArgs& a, const KcatArgs& q, const typename EPI::Args& ea, hipStream_t s,
                           const char* what) {
  if (a.M * a.lda * 2 > 0x7FFFFFFF || a.M * q.lda1 * 2 > 0x7FFFFFFF ||
      !(B1MN ? dtl_fits_mn(q.K1, q.ldb1) : a.N * q.ldb1 * 2 <= 0x7FFFFFFF) ||
      !(B2MN ? dtl_fits_mn(a.K, a.ldb) : a.N * a.ldb * 2 <= 0x7FFFFFFF))
    return fail(PD_EUNSUPPORTED, std::string(what) + ": operands of 2 GiB or more");
  if ((a.M + CfgDtlRA::BM - 1) / CfgDtlRA::BM > 65535 || (a.N + CfgDtlRA::BN - 1) / CfgDtlRA::BN > 65535)
    return fail(PD_EUNSUPPORTED, std::string(what) + ": too large");
  // 256x256 tiles once the grid has at least 256 of them (pd_gemm's rule)
  const int64_t gbx = (a.N + CfgDtlBig::BN - 1) / CfgDtlBig::BN, gby = (a.M + CfgDtlBig::BM - 1) / CfgDtlBig::BM;
  if (EPI::LDS_BYTES <= 2 * CfgDtlBig::STAGE_BYTES && gbx * gby >= 256)
    hipLaunchKernelGGL((k_gemm_dtl_kcat<CfgDtlBig, TC, B1MN, B2MN, EPI>), dim3((unsigned)gbx, (unsigned)gby),
                       dim3(CfgDtlBig::NT), 0, s, a, q, ea);
  else
    hipLaunchKernelGGL((k_gemm_dtl_kcat<CfgDtlRA, TC, B1MN, B2MN, EPI>),
                       dim3((unsigned)((a.N + CfgDtlRA::BN - 1) / CfgDtlRA::BN),
                            (unsigned)((a.M + CfgDtlRA::BM - 1) / CfgDtlRA::BM)),
                       dim3(CfgDtlRA::NT), 0, s, a, q, ea);
  return check_launch(what);
}

}  // namespace pd
