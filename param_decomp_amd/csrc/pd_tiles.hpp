// Shared device helpers for the token- and tile-space kernels of the fused steps (gfx950).
#pragma once
#include "pd_common.hpp"

namespace pd {

static constexpr int TILE = 64;

// ---------------------------------------------------------------- layout kernels
// All job-space producers work on 64 (rows) x 64 (columns) tiles with 256 threads. A
// thread moves 4 or 8 consecutive columns of a row with one 8- or 16-byte access; the
// transposed copy goes through an LDS tile held transposed (tT[col][row], 144-byte rows)
// so it leaves as 16-byte stores of 8 consecutive rows.
struct TTile {
  bf16_t v[TILE][TILE + 8];
};

// dst[(c0 + cc) * ld + r0 + rr ...] = tT[cc][rr ...]: rows r < nrows (nrows % 8 == 0),
// columns c0 + cc < ncols.
__device__ inline void ttile_store(const TTile& T, bf16_t* __restrict__ dst, int64_t ld, int64_t r0, int64_t nrows,
                                   int64_t c0, int64_t ncols, int tid) {
  const int cc = tid >> 2, rr = (tid & 3) * 16;
  if (c0 + cc >= ncols) return;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t r = r0 + rr + 8 * h;
    if (r < nrows) *(uint4*)(dst + (c0 + cc) * ld + r) = *(const uint4*)&T.v[cc][rr + 8 * h];
  }
}

__device__ inline float bf_lo(uint32_t w) { return bf16_to_f32((bf16_t)(w & 0xFFFFu)); }
__device__ inline float bf_hi(uint32_t w) { return bf16_to_f32((bf16_t)(w >> 16)); }
__device__ inline uint32_t bf_pack(bf16_t a, bf16_t b) { return (uint32_t)a | ((uint32_t)b << 16); }

// 8 consecutive bf16 values <-> fp32 through one 16-byte access (p 16-byte aligned).
__device__ inline void load8(const bf16_t* p, float f[8]) {
  const uint4 v = *(const uint4*)p;
  f[0] = bf_lo(v.x), f[1] = bf_hi(v.x), f[2] = bf_lo(v.y), f[3] = bf_hi(v.y);
  f[4] = bf_lo(v.z), f[5] = bf_hi(v.z), f[6] = bf_lo(v.w), f[7] = bf_hi(v.w);
}
__device__ inline void store8(bf16_t* p, const float f[8]) {
  *(uint4*)p = make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                          pack_bf16x2(f[6], f[7]));
}
__device__ inline void load8f(const float* p, float f[8]) {
  const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
  f[0] = a.x, f[1] = a.y, f[2] = a.z, f[3] = a.w, f[4] = b.x, f[5] = b.y, f[6] = b.z, f[7] = b.w;
}
// Token-space kernels run one wave per token row, 4 waves per block; the wave index is
// read into a scalar register so per-token indices and weights come in as scalar loads.
__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// b^p and d(b^p)/db with the exponent's common cases fixed at compile time (PM = 2: p = 2,
// PM = 1: p = 1, PM = 0: any p), so no pow code sits beside the fast paths.
template <int PM>
__device__ inline float powp(float b, float p) {
  if constexpr (PM == 2) return b * b;
  else if constexpr (PM == 1) return b;
  else return powf(b, p);
}
template <int PM>
__device__ inline float dpowp(float b, float p) {
  if constexpr (PM == 2) return 2.f * b;
  else if constexpr (PM == 1) return 1.f;
  else return p * powf(b, p - 1.f);
}
inline int pow_mode(float p) { return p == 2.f ? 2 : (p == 1.f ? 1 : 0); }

}  // namespace pd
