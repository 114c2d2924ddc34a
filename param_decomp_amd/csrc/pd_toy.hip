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
// latency. Here one wave owns 64 rows end to end: the target, both sites' gates, masks,
// the masked forward, the loss and the whole backward live in registers, the parameters
// in LDS. Each parameter's gradient is summed over the wave's rows (a fixed shuffle
// tree) into a per-block partial; k_tms_reduce adds the blocks' partials in order, so
// the result is deterministic.
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

template <int F, int H, int C>
__global__ __launch_bounds__(64) void k_tms_step(TmsArgs a) {
  typedef TmsLayout<F, H, C> LY;
  constexpr int G = TOY_GATE_H;
  __shared__ float prm[LY::PARAMS];
  float* sW1 = prm;                 // [H][F]
  float* sb2 = sW1 + F * H;         // [F]
  float* sV1 = sb2 + F;             // [F][C]
  float* sU1 = sV1 + F * C;         // [C][H]
  float* sV2 = sU1 + C * H;         // [H][C]
  float* sU2 = sV2 + H * C;         // [C][F]
  float* sG = sU2 + C * F;          // 2 x (w_in, b_in, w_out, b_out)
  const int lane = threadIdx.x;
  auto load = [&](float* dst, const float* src, int n) {
    for (int i = lane; i < n; i += 64) dst[i] = src[i];
  };
  load(sW1, a.W1, F * H);
  load(sb2, a.b2, F);
  load(sV1, a.V1, F * C);
  load(sU1, a.U1, C * H);
  load(sV2, a.V2, H * C);
  load(sU2, a.U2, C * F);
  for (int s = 0; s < 2; ++s) {
    float* g = sG + s * LY::GSZ;
    load(g, a.gate[s][0], C * G);
    load(g + C * G, a.gate[s][1], C * G);
    load(g + 2 * C * G, a.gate[s][2], C * G);
    load(g + 3 * C * G, a.gate[s][3], C);
  }
  __syncthreads();

  const int64_t row = (int64_t)blockIdx.x * 64 + lane;
  const bool valid = row < a.B;
  float* part = a.partial + (int64_t)blockIdx.x * LY::P;
  auto emit = [&](int idx, float v) {
    v = wave_sum(v);
    if (lane == 0) part[idx] = v;
  };
  const float inv_b = 1.f / (float)a.B;

  float x[F];
#pragma unroll
  for (int f = 0; f < F; ++f) x[f] = valid ? a.x[row * F + f] : 0.f;
  // ---- target
  float hid[H], outc[F];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    float acc = 0.f;
#pragma unroll
    for (int f = 0; f < F; ++f) acc = fmaf(x[f], sW1[h * F + f], acc);
    hid[h] = acc;
  }
#pragma unroll
  for (int f = 0; f < F; ++f) {
    float acc = sb2[f];
#pragma unroll
    for (int h = 0; h < H; ++h) acc = fmaf(hid[h], sW1[h * F + f], acc);
    outc[f] = fmaxf(acc, 0.f);
  }

  // ---- a site's CI and mask: g_raw from the gate on h, u, the coefficient
  auto gate_fwd = [&](int s, float h, int c) {
    const float* g = sG + s * LY::GSZ;
    float acc = g[3 * C * G + c];
#pragma unroll
    for (int j = 0; j < G; ++j) acc = fmaf(g[2 * C * G + c * G + j], gelu_only<true>(fmaf(g[c * G + j], h, g[C * G + c * G + j])), acc);
    return acc;
  };
  const int64_t n = a.B * C;
  float d[2], sc[2];
  bool routed[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    routed[s] = a.route ? (valid && a.route[(int64_t)s * a.B + row] != 0) : true;
    d[s] = a.use_delta && valid ? draw_uniform(a.dk[s][0], a.dk[s][1], row, a.B, PD_DTYPE_F32, a.layout) : 0.f;
    sc[s] = routed[s] ? d[s] : 1.f;  // the target output's blend weight
  }
  // site 1 (input x for both the CI and the masked product)
  float h1[C], g1[C], u1[C], coef1[C];
  float imp = 0.f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    float acc = 0.f;
#pragma unroll
    for (int f = 0; f < F; ++f) acc = fmaf(x[f], sV1[f * C + c], acc);
    h1[c] = acc;
    g1[c] = gate_fwd(0, acc, c);
    u1[c] = valid ? draw_uniform(a.mk[0][0], a.mk[0][1], row * C + c, n, PD_DTYPE_F32, a.layout) : 0.f;
    const float lo = lower_fwd(g1[c]);
    coef1[c] = routed[0] ? lo + (1.f - lo) * u1[c] - d[0] : 0.f;
    if (valid) imp += a.p == 1.f ? upper_fwd(g1[c]) : powf(upper_fwd(g1[c]), a.p);
  }
  float a1[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    float acc = sc[0] * hid[h];
#pragma unroll
    for (int c = 0; c < C; ++c) acc = fmaf(h1[c] * coef1[c], sU1[c * H + h], acc);
    a1[h] = acc;
  }
  // site 2 (CI from the clean hidden, the product on the masked one)
  float h2c[C], g2[C], u2[C], coef2[C], h2m[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    float acc = 0.f, accm = 0.f;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      acc = fmaf(hid[h], sV2[h * C + c], acc);
      accm = fmaf(a1[h], sV2[h * C + c], accm);
    }
    h2c[c] = acc;
    h2m[c] = accm;
    g2[c] = gate_fwd(1, acc, c);
    u2[c] = valid ? draw_uniform(a.mk[1][0], a.mk[1][1], row * C + c, n, PD_DTYPE_F32, a.layout) : 0.f;
    const float lo = lower_fwd(g2[c]);
    coef2[c] = routed[1] ? lo + (1.f - lo) * u2[c] - d[1] : 0.f;
    if (valid) imp += a.p == 1.f ? upper_fwd(g2[c]) : powf(upper_fwd(g2[c]), a.p);
  }
  float pre[F], dpre[F];
  float rec = 0.f;
  const float gs = a.recon_coeff * 2.f / (float)(a.B * F);
#pragma unroll
  for (int f = 0; f < F; ++f) {
    float t = 0.f;
#pragma unroll
    for (int h = 0; h < H; ++h) t = fmaf(a1[h], sW1[h * F + f], t);
    float acc = fmaf(sc[1], t, sb2[f]);
#pragma unroll
    for (int c = 0; c < C; ++c) acc = fmaf(h2m[c] * coef2[c], sU2[c * F + f], acc);
    pre[f] = acc;
    const float e = fmaxf(acc, 0.f) - outc[f];
    if (valid) rec = fmaf(e, e, rec);
    dpre[f] = valid && acc > 0.f ? gs * e : 0.f;
  }

  // ---- backward: site 2
  auto dimp = [&](float up) {
    if (!valid) return 0.f;
    return a.imp_coeff * inv_b * (a.p == 1.f ? 1.f : a.p * powf(up, a.p - 1.f));
  };
  // the gate's pullback of dg at h: returns dh, emits the gate parameters' gradients
  auto gate_bwd = [&](int s, float h, int c, float dg) {
    const float* g = sG + s * LY::GSZ;
    const int base = s == 0 ? LY::G1 : LY::G2;
    float dh = 0.f;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float wi = g[c * G + j], wo = g[2 * C * G + c * G + j];
      const GeluOut go = gelu_and_grad<true>(fmaf(wi, h, g[C * G + c * G + j]));
      const float dz = dg * wo * go.grad;
      dh = fmaf(dz, wi, dh);
      emit(base + c * G + j, dz * h);
      emit(base + C * G + c * G + j, dz);
      emit(base + 2 * C * G + c * G + j, dg * go.gelu);
    }
    emit(base + 3 * C * G + c, dg);
    return dh;
  };
  float da1[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    float acc = 0.f;
#pragma unroll
    for (int f = 0; f < F; ++f) acc = fmaf(dpre[f], sW1[h * F + f], acc);
    da1[h] = sc[1] * acc;
  }
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const float acts = h2m[c] * coef2[c];
    float dacts = 0.f;
#pragma unroll
    for (int f = 0; f < F; ++f) {
      emit(LY::U2 + c * F + f, acts * dpre[f]);
      dacts = fmaf(dpre[f], sU2[c * F + f], dacts);
    }
    const float dm = routed[1] ? dacts * h2m[c] : 0.f;
    const float dhm = dacts * coef2[c];
#pragma unroll
    for (int h = 0; h < H; ++h) da1[h] = fmaf(dhm, sV2[h * C + c], da1[h]);
    const float dg = lower_vjp(g2[c], dm * (1.f - u2[c])) + upper_vjp(g2[c], dimp(upper_fwd(g2[c])));
    const float dhc = gate_bwd(1, h2c[c], c, dg);
#pragma unroll
    for (int h = 0; h < H; ++h) emit(LY::V2 + h * C + c, fmaf(a1[h], dhm, hid[h] * dhc));
  }
  // ---- site 1
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const float acts = h1[c] * coef1[c];
    float dacts = 0.f;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      emit(LY::U1 + c * H + h, acts * da1[h]);
      dacts = fmaf(da1[h], sU1[c * H + h], dacts);
    }
    const float dm = routed[0] ? dacts * h1[c] : 0.f;
    const float dh = dacts * coef1[c];
    const float dg = lower_vjp(g1[c], dm * (1.f - u1[c])) + upper_vjp(g1[c], dimp(upper_fwd(g1[c])));
    const float dhc = gate_bwd(0, h1[c], c, dg);
#pragma unroll
    for (int f = 0; f < F; ++f) emit(LY::V1 + f * C + c, x[f] * (dh + dhc));
  }
  emit(LY::REC, rec);
  emit(LY::IMP, imp);
}

// grads[i] = sum over blocks of partial[b][i] in block order; losses = {loss, recon, imp}.
__global__ __launch_bounds__(256) void k_tms_reduce(const float* __restrict__ partial, int nblk, int P, int64_t B,
                                                    int F, float imp_coeff, float recon_coeff,
                                                    float* __restrict__ grads, float* __restrict__ losses) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= P) return;
  double acc = 0.0;
  for (int b = 0; b < nblk; ++b) acc += partial[(int64_t)b * P + i];
  if (i < P - 2) {
    grads[i] = (float)acc;
  } else if (i == P - 1) {  // the imp sum: the last entry; the recon sum precedes it
    double rec = 0.0;
    for (int b = 0; b < nblk; ++b) rec += partial[(int64_t)b * P + P - 2];
    const double recon = rec / (double)(B * F), impv = acc / (double)B;
    losses[0] = (float)(recon_coeff * recon + imp_coeff * impv);
    losses[1] = (float)recon;
    losses[2] = (float)impv;
  }
}

template <int F, int H, int C>
static int launch_tms(const TmsArgs& a, float* grads, float* losses, size_t ws_bytes, hipStream_t s) {
  typedef TmsLayout<F, H, C> LY;
  const int nblk = (int)cdiv(a.B, 64);
  if (ws_bytes < (size_t)nblk * LY::P * sizeof(float)) return fail(PD_EWORKSPACE, "pd_tms_step: workspace too small");
  hipLaunchKernelGGL((k_tms_step<F, H, C>), dim3((unsigned)nblk), dim3(64), 0, s, a);
  hipLaunchKernelGGL(k_tms_reduce, dim3((unsigned)cdiv(LY::P, 256)), dim3(256), 0, s, a.partial, nblk, LY::P, a.B, F,
                     a.imp_coeff, a.recon_coeff, grads, losses);
  return check_launch("pd_tms_step");
}

}  // namespace pd

using namespace pd;

extern "C" {

size_t pd_tms_step_workspace_size(int64_t B, int F, int H, int C) {
  if (F == 5 && H == 2 && C == 20) return (size_t)cdiv(B, 64) * TmsLayout<5, 2, 20>::P * sizeof(float);
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
