// The TMS decomposition step as one fused kernel plus one reduction (gfx950, fp32).
//
//   target   hid = x W1^T, out = relu(hid W1 + b2)        pd/targets/tms.py:254-271
//   masked   linear1 -> linear2 + b2 -> relu, both sites  pd/targets/tms.py:311-359
//            decomposed (site_forward, pd/core/decomposed_linear.py:142-175)
//   CI       paper-form gate per component on the clean input's x @ V, lower / upper
//            leaky hard sigmoids, m = lower + (1 - lower) u with fp32 Threefry draws
//            per site (pd/core/masking.py:148-167), optional delta and routes
//   loss     recon_coeff mse(out, clean) + imp_coeff sum_sites sum_c mean_b upper^p
//            (pd/targets/tms.py:380-388; the paper's L_p)
//
// At B = 4096 rows, 5 features, 2 hidden and 20 components per site, the step is tens of
// small products and elementwise passes; as separate launches it is bound by launch
// latency. Here one thread owns one (row, component) end to end: its component's CI
// gates (the bulk of the arithmetic: 16 GELUs forward and backward per site), its mask
// draws, its share of the masked products and its parameter gradients, in registers; the
// parameters sit in LDS. The three sums over components a row needs (the masked hidden,
// the output pre-activation, the hidden's cotangent) go through LDS in component order.
// A block is 16 rows x 20 components (5 waves, 256 blocks at B = 4096); each gradient slot
// is summed over the block's rows in row order into a per-block partial, and
// k_tms_reduce adds the blocks' partials in a fixed order, so the result is deterministic.
#include <algorithm>
#include <type_traits>

#include "pd_common.hpp"

namespace pd {

static constexpr int TOY_GATE_H = 16;

struct TmsArgs {
  int64_t B;
  const float *x, *W1, *b2, *V1, *U1, *V2, *U2;
  const float* gate[2][4];  // per site: w_in [C,16], b_in [C,16], w_out [C,16], b_out [C]
  uint32_t mk[2][2], dk[2][2];
  int use_delta, layout;
  const uint8_t* route;  // [2, B] or NULL (every row routed)
  float p, imp_coeff, recon_coeff;
  float* partial;  // [gridDim.x, P]
};

// The flat gradient layout (the partial rows and the reduced output):
// V1 [F,C] | U1 [C,H] | V2 [H,C] | U2 [C,F] | gate 1 | gate 2 | recon sum | imp sum,
// a gate being w_in [C,16] | b_in [C,16] | w_out [C,16] | b_out [C].
template <int F, int H, int C>
struct TmsLayout {
  static constexpr int V1 = 0, U1 = V1 + F * C, V2 = U1 + C * H, U2 = V2 + H * C, G1 = U2 + C * F;
  static constexpr int GSZ = 3 * C * TOY_GATE_H + C, G2 = G1 + GSZ, REC = G2 + GSZ, IMP = REC + 1, P = IMP + 1;
  static constexpr int PARAMS = F * H + F + F * C + C * H + H * C + C * F + 2 * GSZ;  // LDS floats
};

// Rows per block pass: a block is TMS_RS rows x C components, one thread per (row,
// component), so a row's threads are C consecutive lanes.
static constexpr int TMS_RS = 16;

// Per-thread gradient slots of one component: V1[:, c] (F) | U1[c, :] (H) | V2[:, c] (H) |
// U2[c, :] (F) | gate 1 of c (w_in 16, b_in 16, w_out 16, b_out) | gate 2 of c.
template <int F, int H, int C>
struct TmsSlots {
  static constexpr int G = TOY_GATE_H, GS = 3 * G + 1;
  static constexpr int V1 = 0, U1 = F, V2 = F + H, U2 = F + 2 * H, G1 = 2 * F + 2 * H, G2 = G1 + GS, N = G2 + GS;
  // the flat gradient index of slot k of component c
  __device__ static int flat(int k, int c) {
    typedef TmsLayout<F, H, C> LY;
    if (k < U1) return LY::V1 + k * C + c;
    if (k < V2) return LY::U1 + c * H + (k - U1);
    if (k < U2) return LY::V2 + (k - V2) * C + c;
    if (k < G1) return LY::U2 + c * F + (k - U2);
    const int base = k < G2 ? LY::G1 : LY::G2;
    const int q = k < G2 ? k - G1 : k - G2;  // 0..GS-1
    return q < 3 * G ? base + (q / G) * C * G + c * G + q % G : base + 3 * C * G + c;
  }
};

template <int F, int H, int C>
__global__ __launch_bounds__(TMS_RS * C) void k_tms_step(TmsArgs a, int iters) {
  typedef TmsLayout<F, H, C> LY;
  typedef TmsSlots<F, H, C> SL;
  constexpr int G = TOY_GATE_H, NT = TMS_RS * C, NS = SL::N, CH = TMS_RS, NCH = (NS + CH - 1) / CH;
  static_assert(NT % 64 == 0 && C * CH == NT, "a block is whole waves; one reduction column per thread");
  __shared__ float sW1[H * F], sb2[F], sV1[F * C], sU1[C * H], sV2[H * C], sU2[C * F];
  __shared__ float sG[2][SL::GS][C];  // [site][w_in j | b_in j | w_out j | b_out][component]
  __shared__ float xa[TMS_RS][C][H], xp[TMS_RS][C][F], xd[TMS_RS][C][H];  // cross-component sums
  __shared__ float red[TMS_RS][NT];
  __shared__ float bacc[LY::P - 2];  // the block's gradient sums, flat layout
  __shared__ float bred[NT / 64][2];
  const int tid = threadIdx.x, c = tid % C, rs = tid / C;
  for (int i = tid; i < H * F; i += NT) sW1[i] = a.W1[i];
  for (int i = tid; i < F; i += NT) sb2[i] = a.b2[i];
  for (int i = tid; i < F * C; i += NT) sV1[i] = a.V1[i];
  for (int i = tid; i < C * H; i += NT) sU1[i] = a.U1[i];
  for (int i = tid; i < H * C; i += NT) sV2[i] = a.V2[i];
  for (int i = tid; i < C * F; i += NT) sU2[i] = a.U2[i];
  for (int i = tid; i < 2 * 3 * C * G; i += NT) {  // w_in, b_in, w_out [C, G] -> [q * G + j][c]
    const int st = i / (3 * C * G), r = i % (3 * C * G), q = r / (C * G), cj = r % (C * G);
    sG[st][q * G + cj % G][cj / G] = a.gate[st][q][cj];
  }
  for (int i = tid; i < 2 * C; i += NT) sG[i / C][3 * G][i % C] = a.gate[i / C][3][i % C];
  for (int i = tid; i < LY::P - 2; i += NT) bacc[i] = 0.f;
  __syncthreads();

  const float inv_b = 1.f / (float)a.B, gs = a.recon_coeff * 2.f / (float)(a.B * F);
  const int64_t n = a.B * C;
  float rec = 0.f, imp = 0.f;
  // Adds slots K0 .. K0 + NK - 1 of every thread (vals) into bacc, summed over the block's
  // rows in row order: 16 slots per round through red, thread t owning slot t % 16 of
  // component t / 16. Every thread of the block calls it (it holds barriers).
  auto flush = [&](auto K0, auto NK, const float* vals) __attribute__((always_inline)) {
    constexpr int k0 = decltype(K0)::value, nk = decltype(NK)::value;
#pragma unroll
    for (int ch = 0; ch < (nk + CH - 1) / CH; ++ch) {
#pragma unroll
      for (int k = 0; k < CH; ++k) red[rs][c * CH + k] = ch * CH + k < nk ? vals[ch * CH + k] : 0.f;
      __syncthreads();
      const int k = ch * CH + tid % CH;
      if (k < nk) {
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < TMS_RS; ++r) sum += red[r][tid];
        bacc[SL::flat(k0 + k, tid / CH)] += sum;
      }
      __syncthreads();
    }
  };
  auto gate_fwd = [&](auto ST, float h) __attribute__((always_inline)) {
    constexpr int st = decltype(ST)::value;
    float g = sG[st][3 * G][c];
#pragma unroll
    for (int j = 0; j < G; ++j) g = fmaf(sG[st][2 * G + j][c], gelu_only<true>(fmaf(sG[st][j][c], h, sG[st][G + j][c])), g);
    return g;
  };
  // the gate's pullback of dg at h: returns dh, writes the gate's parameter gradients (gsl:
  // w_in j | b_in j | w_out j | b_out)
  auto gate_bwd = [&](auto ST, float h, float dg, float (&gsl)[SL::GS]) __attribute__((always_inline)) {
    constexpr int st = decltype(ST)::value;
    float dh = 0.f;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float wi = sG[st][j][c], wo = sG[st][2 * G + j][c];
      const GeluOut go = gelu_and_grad<true>(fmaf(wi, h, sG[st][G + j][c]));
      const float dz = dg * wo * go.grad;
      dh = fmaf(dz, wi, dh);
      gsl[j] = dz * h;
      gsl[G + j] = dz;
      gsl[2 * G + j] = dg * go.gelu;
    }
    gsl[3 * G] = dg;
    return dh;
  };
  auto dimp = [&](bool valid, float up) {
    if (!valid) return 0.f;
    return a.imp_coeff * inv_b * (a.p == 1.f ? 1.f : a.p * powf(up, a.p - 1.f));
  };

  for (int it = 0; it < iters; ++it) {
    const int64_t row = ((int64_t)blockIdx.x * iters + it) * TMS_RS + rs;
    const bool valid = row < a.B;
    float x[F];
#pragma unroll
    for (int f = 0; f < F; ++f) x[f] = valid ? a.x[row * F + f] : 0.f;
    // ---- target (every thread of the row computes it)
    float hid[H], outc[F];
#pragma unroll
    for (int h = 0; h < H; ++h) {
      float s = 0.f;
#pragma unroll
      for (int f = 0; f < F; ++f) s = fmaf(x[f], sW1[h * F + f], s);
      hid[h] = s;
    }
#pragma unroll
    for (int f = 0; f < F; ++f) {
      float s = sb2[f];
#pragma unroll
      for (int h = 0; h < H; ++h) s = fmaf(hid[h], sW1[h * F + f], s);
      outc[f] = fmaxf(s, 0.f);
    }
    float d[2], sc[2];
    bool routed[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      routed[st] = a.route ? (valid && a.route[(int64_t)st * a.B + row] != 0) : true;
      d[st] = a.use_delta && valid ? draw_uniform(a.dk[st][0], a.dk[st][1], row, a.B, PD_DTYPE_F32, a.layout) : 0.f;
      sc[st] = routed[st] ? d[st] : 1.f;  // the target output's blend weight
    }
    // ---- site 1, component c (CI and product on x)
    float h1 = 0.f;
#pragma unroll
    for (int f = 0; f < F; ++f) h1 = fmaf(x[f], sV1[f * C + c], h1);
    const float g1 = gate_fwd(std::integral_constant<int, 0>{}, h1);
    const float u1 = valid ? draw_uniform(a.mk[0][0], a.mk[0][1], row * C + c, n, PD_DTYPE_F32, a.layout) : 0.f;
    const float lo1 = lower_fwd(g1);
    const float coef1 = routed[0] ? lo1 + (1.f - lo1) * u1 - d[0] : 0.f;
    if (valid) imp += a.p == 1.f ? upper_fwd(g1) : powf(upper_fwd(g1), a.p);
    const float act1 = h1 * coef1;
#pragma unroll
    for (int h = 0; h < H; ++h) xa[rs][c][h] = act1 * sU1[c * H + h];
    __syncthreads();
    float a1[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
      float s = sc[0] * hid[h];
      for (int q = 0; q < C; ++q) s += xa[rs][q][h];
      a1[h] = s;
    }
    // ---- site 2 (CI from the clean hidden, the product on the masked one)
    float h2c = 0.f, h2m = 0.f;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      h2c = fmaf(hid[h], sV2[h * C + c], h2c);
      h2m = fmaf(a1[h], sV2[h * C + c], h2m);
    }
    const float g2 = gate_fwd(std::integral_constant<int, 1>{}, h2c);
    const float u2 = valid ? draw_uniform(a.mk[1][0], a.mk[1][1], row * C + c, n, PD_DTYPE_F32, a.layout) : 0.f;
    const float lo2 = lower_fwd(g2);
    const float coef2 = routed[1] ? lo2 + (1.f - lo2) * u2 - d[1] : 0.f;
    if (valid) imp += a.p == 1.f ? upper_fwd(g2) : powf(upper_fwd(g2), a.p);
    const float act2 = h2m * coef2;
#pragma unroll
    for (int f = 0; f < F; ++f) xp[rs][c][f] = act2 * sU2[c * F + f];
    __syncthreads();
    float dpre[F];
#pragma unroll
    for (int f = 0; f < F; ++f) {
      float t = 0.f;
#pragma unroll
      for (int h = 0; h < H; ++h) t = fmaf(a1[h], sW1[h * F + f], t);
      float s = fmaf(sc[1], t, sb2[f]);
      for (int q = 0; q < C; ++q) s += xp[rs][q][f];
      const float e = fmaxf(s, 0.f) - outc[f];
      if (valid && c == 0) rec = fmaf(e, e, rec);
      dpre[f] = valid && s > 0.f ? gs * e : 0.f;
    }
    // ---- backward, site 2
    float uv[SL::G1];  // this row's V1 | U1 | V2 | U2 slots
    float dacts2 = 0.f;
#pragma unroll
    for (int f = 0; f < F; ++f) {
      uv[SL::U2 + f] = act2 * dpre[f];
      dacts2 = fmaf(dpre[f], sU2[c * F + f], dacts2);
    }
    const float dm2 = routed[1] ? dacts2 * h2m : 0.f;
    const float dhm = dacts2 * coef2;
#pragma unroll
    for (int h = 0; h < H; ++h) xd[rs][c][h] = dhm * sV2[h * C + c];
    const float dg2 = lower_vjp(g2, dm2 * (1.f - u2)) + upper_vjp(g2, dimp(valid, upper_fwd(g2)));
    float gsl[SL::GS];
    const float dhc2 = gate_bwd(std::integral_constant<int, 1>{}, h2c, dg2, gsl);
#pragma unroll
    for (int h = 0; h < H; ++h) uv[SL::V2 + h] = fmaf(a1[h], dhm, hid[h] * dhc2);
    flush(std::integral_constant<int, SL::G2>{}, std::integral_constant<int, SL::GS>{}, gsl);  // (its barriers publish xd)
    float da1[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
      float t = 0.f;
#pragma unroll
      for (int f = 0; f < F; ++f) t = fmaf(dpre[f], sW1[h * F + f], t);
      float s = sc[1] * t;
      for (int q = 0; q < C; ++q) s += xd[rs][q][h];
      da1[h] = s;
    }
    // ---- site 1
    float dacts1 = 0.f;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      uv[SL::U1 + h] = act1 * da1[h];
      dacts1 = fmaf(da1[h], sU1[c * H + h], dacts1);
    }
    const float dm1 = routed[0] ? dacts1 * h1 : 0.f;
    const float dh1 = dacts1 * coef1;
    const float dg1 = lower_vjp(g1, dm1 * (1.f - u1)) + upper_vjp(g1, dimp(valid, upper_fwd(g1)));
    const float dhc1 = gate_bwd(std::integral_constant<int, 0>{}, h1, dg1, gsl);
#pragma unroll
    for (int f = 0; f < F; ++f) uv[SL::V1 + f] = x[f] * (dh1 + dhc1);
    flush(std::integral_constant<int, SL::G1>{}, std::integral_constant<int, SL::GS>{}, gsl);
    flush(std::integral_constant<int, 0>{}, std::integral_constant<int, SL::G1>{}, uv);
  }

  // ---- block partial: the gradient sums (complete after the last flush's barrier), then
  // the recon and imp sums over the whole block
  float* part = a.partial + (int64_t)blockIdx.x * LY::P;
  for (int i = tid; i < LY::P - 2; i += NT) part[i] = bacc[i];
  rec = wave_sum(rec);
  imp = wave_sum(imp);
  if ((tid & 63) == 0) {
    bred[tid >> 6][0] = rec;
    bred[tid >> 6][1] = imp;
  }
  __syncthreads();
  if (tid == 0) {
    float r = 0.f, m = 0.f;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
      r += bred[w][0];
      m += bred[w][1];
    }
    part[LY::REC] = r;
    part[LY::IMP] = m;
  }
}

// Column i of partials [b0, b1) of the [nblk, P] partials, in block order (double), the
// loads of 64 blocks issued before their adds.
__device__ inline double tms_colsum(const float* __restrict__ partial, int b0, int b1, int P, int i) {
  constexpr int Q = 64;
  double acc = 0.0;
  int b = b0;
  for (; b + Q <= b1; b += Q) {
    float v[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) v[q] = partial[(int64_t)(b + q) * P + i];
#pragma unroll
    for (int q = 0; q < Q; ++q) acc += v[q];
  }
  for (; b < b1; ++b) acc += partial[(int64_t)b * P + i];
  return acc;
}

// grads[i] = sum over blocks of partial[b][i]; losses = {loss, recon, imp}. Four
// consecutive lanes take one slot, each summing a quarter of the blocks in block order,
// and the quarters are added in order ((q0 + q1) + q2) + q3 (double): a fixed order, so
// the result is deterministic, with a quarter of the dependent round trips of one lane
// per slot (one lane per slot, one dependent load per block: 79 us at 256 blocks).
__global__ __launch_bounds__(256) void k_tms_reduce(const float* __restrict__ partial, int nblk, int P, int64_t B,
                                                    int F, float imp_coeff, float recon_coeff,
                                                    float* __restrict__ grads, float* __restrict__ losses) {
  const int i = blockIdx.x * 64 + (threadIdx.x >> 2), part = threadIdx.x & 3, lead = threadIdx.x & ~3;
  const int per = (nblk + 3) / 4, b0 = min(nblk, part * per), b1 = min(nblk, b0 + per);
  const bool last = i == P - 1;  // the imp sum: the last entry; the recon sum precedes it
  const double acc = i < P ? tms_colsum(partial, b0, b1, P, i) : 0.0;
  const double rec = last ? tms_colsum(partial, b0, b1, P, P - 2) : 0.0;
  const double a1 = __shfl(acc, lead + 1), a2 = __shfl(acc, lead + 2), a3 = __shfl(acc, lead + 3);
  const double r1 = __shfl(rec, lead + 1), r2 = __shfl(rec, lead + 2), r3 = __shfl(rec, lead + 3);
  if (part != 0 || i >= P) return;
  const double total = ((acc + a1) + a2) + a3;
  if (i < P - 2) {
    grads[i] = (float)total;
  } else if (last) {
    const double recon = (((rec + r1) + r2) + r3) / (double)(B * F), impv = total / (double)B;
    losses[0] = (float)(recon_coeff * recon + imp_coeff * impv);
    losses[1] = (float)recon;
    losses[2] = (float)impv;
  }
}

// Row passes per block: enough blocks for the chip (about 256) before a block takes more
// rows.
static int tms_iters(int64_t B) { return (int)std::max<int64_t>(1, cdiv(B, (int64_t)TMS_RS * 256)); }
static int64_t tms_blocks(int64_t B) { return cdiv(B, (int64_t)TMS_RS * tms_iters(B)); }

template <int F, int H, int C>
static int launch_tms(const TmsArgs& a, float* grads, float* losses, size_t ws_bytes, hipStream_t s) {
  typedef TmsLayout<F, H, C> LY;
  const int nblk = (int)tms_blocks(a.B);
  if (ws_bytes < (size_t)nblk * LY::P * sizeof(float)) return fail(PD_EWORKSPACE, "pd_tms_step: workspace too small");
  hipLaunchKernelGGL((k_tms_step<F, H, C>), dim3((unsigned)nblk), dim3(TMS_RS * C), 0, s, a, tms_iters(a.B));
  hipLaunchKernelGGL(k_tms_reduce, dim3((unsigned)cdiv(LY::P, 64)), dim3(256), 0, s, a.partial, nblk, LY::P, a.B, F,
                     a.imp_coeff, a.recon_coeff, grads, losses);
  return check_launch("pd_tms_step");
}

}  // namespace pd

using namespace pd;

extern "C" {

size_t pd_tms_step_workspace_size(int64_t B, int F, int H, int C) {
  if (B > 0 && F == 5 && H == 2 && C == 20) return (size_t)tms_blocks(B) * TmsLayout<5, 2, 20>::P * sizeof(float);
  return 0;
}

int pd_tms_step_grads_size(int F, int H, int C) {
  if (F == 5 && H == 2 && C == 20) return TmsLayout<5, 2, 20>::P - 2;
  return 0;
}

int pd_tms_step(int64_t B, int F, int H, int C, const float* x, const float* W1, const float* b2, const float* V1,
                const float* U1, const float* V2, const float* U2, const float* const* gates, uint32_t draw_k0,
                uint32_t draw_k1, int use_delta, int layout, const uint8_t* routes, float p, float imp_coeff,
                float recon_coeff, float* grads, float* losses, void* workspace, size_t workspace_bytes,
                void* stream) {
  if (B <= 0 || !x || !W1 || !b2 || !V1 || !U1 || !V2 || !U2 || !gates || !grads || !losses || !workspace)
    return fail(PD_EINVAL, "pd_tms_step: bad args");
  if (layout != PD_LAYOUT_PARTITIONABLE && layout != PD_LAYOUT_ORIGINAL)
    return fail(PD_EINVAL, "pd_tms_step: unknown counter layout");
  if (!(p > 0.f)) return fail(PD_EINVAL, "pd_tms_step: p > 0");
  TmsArgs a{};
  a.B = B;
  a.x = x;
  a.W1 = W1;
  a.b2 = b2;
  a.V1 = V1;
  a.U1 = U1;
  a.V2 = V2;
  a.U2 = U2;
  // the sites' keys: mask_key, delta_key = split(draw_key); site key = fold_in(key, site)
  uint32_t halves[4];
  split2(draw_k0, draw_k1, layout, halves);
  for (int s = 0; s < 2; ++s) {
    for (int q = 0; q < 4; ++q) {
      a.gate[s][q] = gates[s * 4 + q];
      if (!a.gate[s][q]) return fail(PD_EINVAL, "pd_tms_step: null gate parameter");
    }
    for (int h = 0; h < 2; ++h) {
      uint32_t k0 = 0, k1 = (uint32_t)s;
      threefry2x32(halves[2 * h], halves[2 * h + 1], k0, k1);
      (h == 0 ? a.mk : a.dk)[s][0] = k0;
      (h == 0 ? a.mk : a.dk)[s][1] = k1;
    }
  }
  a.use_delta = use_delta;
  a.layout = layout;
  a.route = routes;
  a.p = p;
  a.imp_coeff = imp_coeff;
  a.recon_coeff = recon_coeff;
  a.partial = (float*)workspace;
  if (F == 5 && H == 2 && C == 20) return launch_tms<5, 2, 20>(a, grads, losses, workspace_bytes, (hipStream_t)stream);
  return fail(PD_EUNSUPPORTED, "pd_tms_step: compiled for the 5-2 target with 20 components per site");
}

}  // extern "C"
