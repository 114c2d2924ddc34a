// The ResidMLP toy decomposition step as one native call (gfx950, fp32).
//
//   target   r_0 = x W_E; per layer hid = relu(r W_in^T), r += hid W_out^T; out = r W_U
//                                                     pd/targets/resid_mlp.py:266-333
//   masked   the same with every mlp_in / mlp_out decomposed, site output
//            ((a V) (.) m) U (site_forward, pd/core/decomposed_linear.py:142-175;
//            the masked forward pd/targets/resid_mlp.py:336-390)
//   CI       paper-form gate per component on the clean input's a V, lower / upper leaky
//            hard sigmoids, m = lower + (1 - lower) u with fp32 Threefry draws per site
//            (pd/core/masking.py:148-167)
//   loss     recon_coeff mse(out, clean) + imp_coeff sum_sites sum_c mean_b upper^p
//            (pd/targets/resid_mlp.py:411-418; the paper's L_p), fwd + bwd
//
// The products run on the library's fp32 MFMA GEMM. Each site's CI gate, squashing, mask
// draw, masked activations and imp-min term form one column-mapped pass (one lane per
// component over RM_ROWS rows), and its backward (mask pullback into both a V operands,
// squashing and gate pullbacks, gate-parameter partials) another; the partials are added
// over row chunks in a fixed order. At the 1-layer benchmark shape that is 31 launches
// per step, against about 90 for the same step composed from the library's primitives.
#include <algorithm>
#include <vector>

#include "pd_common.hpp"

namespace pd {

static constexpr int RM_COLS = 64;   // components per block of the site passes
static constexpr int RM_WAVES = 4;   // waves per block, each RM_ROWS / RM_WAVES of its rows
static constexpr int RM_ROWS = 8;    // rows per block of the site passes
static constexpr int RM_GATE = 49;  // gate-parameter gradient slots per component

struct RmGate {
  const float *w_in, *b_in, *w_out, *b_out;  // [C,16], [C,16], [C,16], [C]
  uint32_t k0, k1;                           // the site's mask key
};

__device__ inline float rm_pow(float b, float p) { return p == 2.f ? b * b : (p == 1.f ? b : powf(b, p)); }
__device__ inline float rm_dpow(float b, float p) {
  return p == 2.f ? 2.f * b : (p == 1.f ? 1.f : p * powf(b, p - 1.f));
}

// Forward of one site: g = gate(hg) (kept in g_raw for the backward), lower / upper, the
// fp32 uniform u of element (t, c) of the site's [B, C] draw, acts = ha (lower + (1 -
// lower) u), and the block's sum of upper^p. Block = 64 components x RM_ROWS rows, wave w
// taking rows RM_ROWS / RM_WAVES w .. (sums added in wave order). hg is the clean input's a V (the gate
// input); ha the masked input's (the same array at the first mlp_in).
__global__ __launch_bounds__(RM_COLS * RM_WAVES) void k_rm_site_fwd(const float* __restrict__ hg,
                                                                    const float* __restrict__ ha, int64_t B, int C,
                                                                    RmGate gt, int layout, float p,
                                                                    float* __restrict__ g_raw,
                                                                    float* __restrict__ acts,
                                                                    float* __restrict__ imp_part) {
  __shared__ float red[RM_WAVES];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c = blockIdx.x * RM_COLS + lane;
  constexpr int WR = RM_ROWS / RM_WAVES;
  const int64_t r0 = (int64_t)blockIdx.y * RM_ROWS + wv * WR, r1 = r0 + WR < B ? r0 + WR : B;
  float imp = 0.f;
  if (c < C) {
    float wi[16], bi[16], wo[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      wi[j] = gt.w_in[c * 16 + j];
      bi[j] = gt.b_in[c * 16 + j];
      wo[j] = gt.w_out[c * 16 + j];
    }
    const float bo = gt.b_out[c];
    const int64_t n = B * C;
    for (int64_t t = r0; t < r1; ++t) {
      const int64_t i = t * C + c;
      const float hv = hg[i];
      float g = bo;
#pragma unroll
      for (int j = 0; j < 16; ++j) g = fmaf(wo[j], gelu_only<true>(fmaf(wi[j], hv, bi[j])), g);
      g_raw[i] = g;
      const float lo = lower_fwd(g);
      imp += rm_pow(upper_fwd(g), p);
      const float u = draw_uniform(gt.k0, gt.k1, i, n, PD_DTYPE_F32, layout);
      acts[i] = ha[i] * (lo + (1.f - lo) * u);
    }
  }
  imp = wave_sum(imp);
  if (lane == 0) red[wv] = imp;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = red[0];
#pragma unroll
    for (int k = 1; k < RM_WAVES; ++k) t += red[k];
    imp_part[(int64_t)blockIdx.y * gridDim.x + blockIdx.x] = t;
  }
}

// Backward of one site from d_acts: the mask pullback d_ha = d_acts m (onto the masked
// input's a V), and dg = lower_vjp(g, d_acts ha (1 - u)) + upper_vjp(g, imp_scale d upper^p)
// pulled back through the gate onto hg (d_hg) and into the lane's gate-parameter sums,
// written per row chunk to partial [chunk][49][C] (the block's waves added in row order).
// With d_hg == d_ha (the gate and the mask read the same a V) the two pullbacks are
// written summed.
__global__ __launch_bounds__(RM_COLS * RM_WAVES) void k_rm_site_bwd(
    const float* __restrict__ d_acts, const float* __restrict__ hg, const float* __restrict__ ha,
    const float* __restrict__ g_raw, int64_t B, int C, RmGate gt, int layout, float p, float imp_scale, float* d_ha,
    float* d_hg, float* __restrict__ partial) {
  __shared__ float red[RM_WAVES - 1][RM_GATE][RM_COLS];  // waves 1.. hand their sums to wave 0
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, c = blockIdx.x * RM_COLS + lane;
  constexpr int WR = RM_ROWS / RM_WAVES;
  const int64_t r0 = (int64_t)blockIdx.y * RM_ROWS + wv * WR, r1 = r0 + WR < B ? r0 + WR : B;
  const bool ok = c < C, same = d_ha == d_hg;
  float wi[16], bi[16], wo[16], a_wi[16], a_bi[16], a_wo[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    wi[j] = ok ? gt.w_in[c * 16 + j] : 0.f;
    bi[j] = ok ? gt.b_in[c * 16 + j] : 0.f;
    wo[j] = ok ? gt.w_out[c * 16 + j] : 0.f;
    a_wi[j] = a_bi[j] = a_wo[j] = 0.f;
  }
  float a_bo = 0.f;
  const int64_t n = B * C;
  for (int64_t t = r0; t < r1 && ok; ++t) {
    const int64_t i = t * C + c;
    const float hv = hg[i], av = ha[i], g = g_raw[i], da = d_acts[i];
    const float lo = lower_fwd(g);
    const float u = draw_uniform(gt.k0, gt.k1, i, n, PD_DTYPE_F32, layout);
    const float dmask = da * (lo + (1.f - lo) * u);
    const float dg = lower_vjp(g, da * av * (1.f - u)) + upper_vjp(g, imp_scale * rm_dpow(upper_fwd(g), p));
    float dh = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const GeluOut go = gelu_and_grad<true>(fmaf(wi[j], hv, bi[j]));
      const float dz = dg * wo[j] * go.grad;
      dh = fmaf(dz, wi[j], dh);
      a_wi[j] = fmaf(dz, hv, a_wi[j]);
      a_bi[j] += dz;
      a_wo[j] = fmaf(dg, go.gelu, a_wo[j]);
    }
    a_bo += dg;
    if (same) {
      d_ha[i] = dmask + dh;
    } else {
      d_ha[i] = dmask;
      d_hg[i] = dh;
    }
  }
  // the block's sum in wave order (the rows' order), by wave 0
  if (wv > 0) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      red[wv - 1][j][lane] = a_wi[j];
      red[wv - 1][16 + j][lane] = a_bi[j];
      red[wv - 1][32 + j][lane] = a_wo[j];
    }
    red[wv - 1][48][lane] = a_bo;
  }
  __syncthreads();
  if (wv > 0 || !ok) return;
#pragma unroll
  for (int k = 0; k < RM_WAVES - 1; ++k) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      a_wi[j] += red[k][j][lane];
      a_bi[j] += red[k][16 + j][lane];
      a_wo[j] += red[k][32 + j][lane];
    }
    a_bo += red[k][48][lane];
  }
  float* pp = partial + (int64_t)blockIdx.y * RM_GATE * C;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    pp[(int64_t)j * C + c] = a_wi[j];
    pp[(int64_t)(16 + j) * C + c] = a_bi[j];
    pp[(int64_t)(32 + j) * C + c] = a_wo[j];
  }
  pp[(int64_t)48 * C + c] = a_bo;
}

// Every site's gate-parameter gradients: the row-chunk partials of slot q of component c
// added in chunk order into the flat gradient buffer (w_in [C,16] | b_in | w_out | b_out
// after the site's dV and dU; every site spans (D + M + 49) C floats).
__global__ void k_rm_gate_reduce(const float* __restrict__ partial, int64_t chunks, int C, int D, int M, int nsites,
                                 float* __restrict__ grads) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per = (int64_t)RM_GATE * C;
  if (idx >= per * nsites) return;
  const int s = (int)(idx / per);
  const int64_t rem = idx % per, q = rem / C, c = rem % C;
  const float acc = pd_ordered_sum(partial + (int64_t)s * chunks * per + rem, chunks, per);
  float* g = grads + ((int64_t)s * (D + M + RM_GATE) + D + M) * C;
  if (q < 48) g[(q / 16) * C * 16 + c * 16 + q % 16] = acc;
  else g[48 * C + c] = acc;
}

// relu in place; and the relu pullback d *= (y > 0) in place.
__global__ void k_rm_relu(float* __restrict__ a, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    a[i] = fmaxf(a[i], 0.f);
}
__global__ void k_rm_relu_bwd(float* __restrict__ d, const float* __restrict__ y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    d[i] = y[i] > 0.f ? d[i] : 0.f;
}

// d_out = scale (out - clean) (scale = recon_coeff 2 / n) and each block's sum of squares.
static constexpr int RM_REC_BLOCKS = 256;
__global__ __launch_bounds__(256) void k_rm_recon(const float* __restrict__ out, const float* __restrict__ clean,
                                                  int64_t n, float scale, float* __restrict__ d_out,
                                                  float* __restrict__ rec_part) {
  __shared__ float red[4];
  float acc = 0.f;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float e = out[i] - clean[i];
    d_out[i] = scale * e;
    acc = fmaf(e, e, acc);
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) rec_part[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

// losses = {recon_coeff recon + imp_coeff imp, recon, imp}: recon = sum(rec_part) / n,
// imp = sum(imp_part) / B (one block, partials added in order per thread, then in
// thread order).
__global__ void k_rm_losses(const float* __restrict__ rec_part, int n_rec, const float* __restrict__ imp_part,
                            int64_t n_imp, double inv_n, double inv_b, float recon_coeff, float imp_coeff,
                            float* __restrict__ losses) {
  __shared__ double sr[256], si[256];
  double r = 0.0, m = 0.0;
  for (int64_t i = threadIdx.x; i < n_rec; i += blockDim.x) r += rec_part[i];
  for (int64_t i = threadIdx.x; i < n_imp; i += blockDim.x) m += imp_part[i];
  sr[threadIdx.x] = r;
  si[threadIdx.x] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    double R = 0.0, I = 0.0;
    for (int k = 0; k < (int)blockDim.x; ++k) {
      R += sr[k];
      I += si[k];
    }
    const double recon = R * inv_n, imp = I * inv_b;
    losses[0] = (float)(recon_coeff * recon + imp_coeff * imp);
    losses[1] = (float)recon;
    losses[2] = (float)imp;
  }
}

struct RmDims {
  int64_t B;
  int F, D, M, C, L;
  int nsites() const { return 2 * L; }
  int din(int s) const { return s % 2 ? M : D; }
  int dout(int s) const { return s % 2 ? D : M; }
  int64_t chunks() const { return cdiv(B, RM_ROWS); }
  int64_t cblocks() const { return cdiv(C, RM_COLS); }
};

// The flat gradient buffer: per site dV [din, C] | dU [C, dout] | gate (w_in | b_in |
// w_out | b_out), sites in order (layers.l.mlp_in, layers.l.mlp_out).
struct RmGradLayout {
  std::vector<int64_t> dV, dU, gate;
  int64_t total = 0;
  explicit RmGradLayout(const RmDims& D) {
    for (int s = 0; s < D.nsites(); ++s) {
      dV.push_back(total);
      total += (int64_t)D.din(s) * D.C;
      dU.push_back(total);
      total += (int64_t)D.C * D.dout(s);
      gate.push_back(total);
      total += (int64_t)RM_GATE * D.C;
    }
  }
};

struct RmArena {
  char* base;
  size_t off = 0;
  float* take(int64_t n) {
    float* p = base ? (float*)(base + off) : nullptr;
    off += ((size_t)n * sizeof(float) + 255) & ~(size_t)255;
    return p;
  }
};

struct RmWork {
  std::vector<float*> r, rm, hidc, hid, hg, ha, graw, acts;  // per layer (r, rm: L + 1) / per site
  float *clean, *out, *d_out, *d_r, *d_r2, *d_acts, *d_ha, *d_hg, *d_hid, *rec_part, *imp_part, *gpart;
  size_t bytes;
};

static RmWork rm_layout(const RmDims& D, char* base) {
  RmArena A{base};
  RmWork W;
  const int64_t B = D.B;
  for (int l = 0; l <= D.L; ++l) {
    W.r.push_back(A.take(B * D.D));
    W.rm.push_back(l == 0 ? W.r[0] : A.take(B * D.D));  // the masked pass starts from the same r_0
  }
  for (int l = 0; l < D.L; ++l) {
    W.hidc.push_back(A.take(B * D.M));
    W.hid.push_back(A.take(B * D.M));
  }
  for (int s = 0; s < D.nsites(); ++s) {
    W.hg.push_back(A.take(B * D.C));
    W.ha.push_back(s == 0 ? W.hg[0] : A.take(B * D.C));  // mlp_in of layer 0 reads r_0 in both passes
    W.graw.push_back(A.take(B * D.C));
    W.acts.push_back(A.take(B * D.C));
  }
  W.clean = A.take(B * D.F);
  W.out = A.take(B * D.F);
  W.d_out = A.take(B * D.F);
  W.d_r = A.take(B * D.D);
  W.d_r2 = A.take(B * D.D);
  W.d_acts = A.take(B * D.C);
  W.d_ha = A.take(B * D.C);
  W.d_hg = A.take(B * D.C);
  W.d_hid = A.take(B * D.M);
  W.rec_part = A.take(RM_REC_BLOCKS);
  W.imp_part = A.take((int64_t)D.nsites() * D.chunks() * D.cblocks());
  W.gpart = A.take((int64_t)D.nsites() * D.chunks() * RM_GATE * D.C);
  W.bytes = A.off;
  return W;
}

static unsigned rm_ew_blocks(int64_t n) { return (unsigned)std::min<int64_t>(cdiv(n, 256), 4096); }

}  // namespace pd

using namespace pd;

extern "C" {

size_t pd_resid_mlp_step_workspace_size(int64_t B, int F, int D, int M, int C, int L) {
  if (B <= 0 || F <= 0 || D <= 0 || M <= 0 || C <= 0 || L <= 0) return 0;
  return rm_layout(RmDims{B, F, D, M, C, L}, nullptr).bytes;
}

int64_t pd_resid_mlp_step_grads_size(int D, int M, int C, int L) {
  if (D <= 0 || M <= 0 || C <= 0 || L <= 0) return 0;
  return RmGradLayout(RmDims{1, 1, D, M, C, L}).total;
}

int pd_resid_mlp_step(int64_t B, int F, int D, int M, int C, int L, const float* x, const float* W_E,
                      const float* W_U, const float* const* W_in, const float* const* W_out, const float* const* V,
                      const float* const* U, const float* const* gates, uint32_t draw_k0, uint32_t draw_k1,
                      int layout, float p, float imp_coeff, float recon_coeff, float* grads, float* losses,
                      float* out, void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "pd_resid_mlp_step";
  if (B <= 0 || F <= 0 || D <= 0 || M <= 0 || C <= 0 || L <= 0 || !x || !W_E || !W_U || !W_in || !W_out || !V ||
      !U || !gates || !grads || !losses || !workspace)
    return fail(PD_EINVAL, std::string(what) + ": bad args");
  if (layout != PD_LAYOUT_PARTITIONABLE && layout != PD_LAYOUT_ORIGINAL)
    return fail(PD_EINVAL, std::string(what) + ": unknown counter layout");
  if (!(p > 0.f)) return fail(PD_EINVAL, std::string(what) + ": p > 0");
  if (B * (int64_t)std::max({F, D, M, C}) >= (int64_t(1) << 31))
    return fail(PD_EUNSUPPORTED, std::string(what) + ": B * width must stay below 2^31");
  const RmDims Dm{B, F, D, M, C, L};
  const int ns = Dm.nsites();
  for (int l = 0; l < L; ++l)
    if (!W_in[l] || !W_out[l]) return fail(PD_EINVAL, std::string(what) + ": null target weight");
  for (int s = 0; s < ns; ++s) {
    if (!V[s] || !U[s]) return fail(PD_EINVAL, std::string(what) + ": null component weight");
    for (int q = 0; q < 4; ++q)
      if (!gates[4 * s + q]) return fail(PD_EINVAL, std::string(what) + ": null gate parameter");
  }
  if (workspace_bytes < rm_layout(Dm, nullptr).bytes) return fail(PD_EWORKSPACE, std::string(what) + ": workspace too small");
  RmWork W = rm_layout(Dm, (char*)workspace);
  if (out) W.out = out;
  hipStream_t s = (hipStream_t)stream;
  const RmGradLayout G(Dm);

  // the sites' mask keys: mask_key = split(draw_key)[0], site key = fold_in(mask_key, site)
  uint32_t halves[4];
  split2(draw_k0, draw_k1, layout, halves);
  std::vector<RmGate> gt(ns);
  for (int i = 0; i < ns; ++i) {
    gt[i] = RmGate{gates[4 * i], gates[4 * i + 1], gates[4 * i + 2], gates[4 * i + 3], 0u, (uint32_t)i};
    threefry2x32(halves[0], halves[1], gt[i].k0, gt[i].k1);
  }

  int rc;
  auto gemm = [&](int64_t m, int64_t nn, int64_t k, const float* a, int64_t lda, int ta, const float* b, int64_t ldb,
                  int tb, float* c, int64_t ldc, float beta) {
    return pd_gemm(PD_DTYPE_F32, m, nn, k, a, lda, ta, b, ldb, tb, c, ldc, PD_DTYPE_F32, 1.f, beta, s);
  };
  const dim3 sgrid((unsigned)Dm.cblocks(), (unsigned)Dm.chunks());
  const int64_t nsite_blocks = Dm.chunks() * Dm.cblocks();

  // ---- clean pass: r_{l+1} = r_l + relu(r_l W_in^T) W_out^T; the gate inputs a V
  if ((rc = gemm(B, D, F, x, F, 0, W_E, D, 0, W.r[0], D, 0.f))) return rc;
  for (int l = 0; l < L; ++l) {
    if ((rc = gemm(B, M, D, W.r[l], D, 0, W_in[l], D, 1, W.hidc[l], M, 0.f))) return rc;
    hipLaunchKernelGGL(k_rm_relu, dim3(rm_ew_blocks(B * M)), dim3(256), 0, s, W.hidc[l], B * M);
    hipMemcpyAsync(W.r[l + 1], W.r[l], (size_t)B * D * sizeof(float), hipMemcpyDeviceToDevice, s);
    if ((rc = gemm(B, D, M, W.hidc[l], M, 0, W_out[l], M, 1, W.r[l + 1], D, 1.f))) return rc;
    if ((rc = gemm(B, C, D, W.r[l], D, 0, V[2 * l], C, 0, W.hg[2 * l], C, 0.f))) return rc;
    if ((rc = gemm(B, C, M, W.hidc[l], M, 0, V[2 * l + 1], C, 0, W.hg[2 * l + 1], C, 0.f))) return rc;
  }
  if ((rc = gemm(B, F, D, W.r[L], D, 0, W_U, F, 0, W.clean, F, 0.f))) return rc;

  // ---- masked pass
  auto site_fwd = [&](int si) {
    hipLaunchKernelGGL(k_rm_site_fwd, sgrid, dim3(RM_COLS * RM_WAVES), 0, s, W.hg[si], W.ha[si], B, C, gt[si], layout, p,
                       W.graw[si], W.acts[si], W.imp_part + si * nsite_blocks);
  };
  for (int l = 0; l < L; ++l) {
    const int si = 2 * l, so = 2 * l + 1;
    if (l > 0 && (rc = gemm(B, C, D, W.rm[l], D, 0, V[si], C, 0, W.ha[si], C, 0.f))) return rc;
    site_fwd(si);
    if ((rc = gemm(B, M, C, W.acts[si], C, 0, U[si], M, 0, W.hid[l], M, 0.f))) return rc;
    hipLaunchKernelGGL(k_rm_relu, dim3(rm_ew_blocks(B * M)), dim3(256), 0, s, W.hid[l], B * M);
    if ((rc = gemm(B, C, M, W.hid[l], M, 0, V[so], C, 0, W.ha[so], C, 0.f))) return rc;
    site_fwd(so);
    hipMemcpyAsync(W.rm[l + 1], W.rm[l], (size_t)B * D * sizeof(float), hipMemcpyDeviceToDevice, s);
    if ((rc = gemm(B, D, C, W.acts[so], C, 0, U[so], D, 0, W.rm[l + 1], D, 1.f))) return rc;
  }
  if ((rc = gemm(B, F, D, W.rm[L], D, 0, W_U, F, 0, W.out, F, 0.f))) return rc;
  const int64_t nout = B * F;
  hipLaunchKernelGGL(k_rm_recon, dim3(RM_REC_BLOCKS), dim3(256), 0, s, W.out, W.clean, nout,
                     recon_coeff * 2.f / (float)nout, W.d_out, W.rec_part);
  if ((rc = check_launch(what))) return rc;

  // ---- backward: d_r is the masked residual's cotangent
  if ((rc = gemm(B, D, F, W.d_out, F, 0, W_U, F, 1, W.d_r, D, 0.f))) return rc;
  const float imp_scale = imp_coeff / (float)B;
  auto site_bwd = [&](int si, float* d_hg) {
    hipLaunchKernelGGL(k_rm_site_bwd, sgrid, dim3(RM_COLS * RM_WAVES), 0, s, W.d_acts, W.hg[si], W.ha[si], W.graw[si], B, C,
                       gt[si], layout, p, imp_scale, W.d_ha, d_hg, W.gpart + (int64_t)si * Dm.chunks() * RM_GATE * C);
  };
  for (int l = L - 1; l >= 0; --l) {
    const int si = 2 * l, so = 2 * l + 1;
    // mlp_out: its output adds into the residual
    if ((rc = gemm(C, D, B, W.acts[so], C, 1, W.d_r, D, 0, grads + G.dU[so], D, 0.f))) return rc;
    if ((rc = gemm(B, C, D, W.d_r, D, 0, U[so], D, 1, W.d_acts, C, 0.f))) return rc;
    site_bwd(so, W.d_hg);
    if ((rc = gemm(M, C, B, W.hid[l], M, 1, W.d_ha, C, 0, grads + G.dV[so], C, 0.f))) return rc;
    if ((rc = gemm(M, C, B, W.hidc[l], M, 1, W.d_hg, C, 0, grads + G.dV[so], C, 1.f))) return rc;
    if ((rc = gemm(B, M, C, W.d_ha, C, 0, V[so], C, 1, W.d_hid, M, 0.f))) return rc;
    hipLaunchKernelGGL(k_rm_relu_bwd, dim3(rm_ew_blocks(B * M)), dim3(256), 0, s, W.d_hid, W.hid[l], B * M);
    // mlp_in
    if ((rc = gemm(C, M, B, W.acts[si], C, 1, W.d_hid, M, 0, grads + G.dU[si], M, 0.f))) return rc;
    if ((rc = gemm(B, C, M, W.d_hid, M, 0, U[si], M, 1, W.d_acts, C, 0.f))) return rc;
    const bool shared = W.ha[si] == W.hg[si];
    site_bwd(si, shared ? W.d_ha : W.d_hg);
    if ((rc = gemm(D, C, B, W.rm[l], D, 1, W.d_ha, C, 0, grads + G.dV[si], C, 0.f))) return rc;
    if (!shared && (rc = gemm(D, C, B, W.r[l], D, 1, W.d_hg, C, 0, grads + G.dV[si], C, 1.f))) return rc;
    if (l > 0) {  // the residual cotangent below this layer
      hipMemcpyAsync(W.d_r2, W.d_r, (size_t)B * D * sizeof(float), hipMemcpyDeviceToDevice, s);
      if ((rc = gemm(B, D, C, W.d_ha, C, 0, V[si], C, 1, W.d_r2, D, 1.f))) return rc;
      std::swap(W.d_r, W.d_r2);
    }
  }
  const int64_t gslots = (int64_t)ns * RM_GATE * C;
  hipLaunchKernelGGL(k_rm_gate_reduce, dim3((unsigned)cdiv(gslots, 256)), dim3(256), 0, s, W.gpart, Dm.chunks(), C,
                     D, M, ns, grads);
  hipLaunchKernelGGL(k_rm_losses, dim3(1), dim3(256), 0, s, W.rec_part, RM_REC_BLOCKS, W.imp_part,
                     (int64_t)ns * nsite_blocks, 1.0 / (double)nout, 1.0 / (double)B, recon_coeff, imp_coeff, losses);
  return check_launch(what);
}

}  // extern "C"
