/*
 * C restatement of the masked-component step — TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ as a fast checker for large Threefry draws, and by bench.py as the
 * timed CPU baseline (fp32, OpenMP). It restates the same arithmetic as
 * oracle/pd_oracle.py (which carries the reference citations):
 *   - Threefry-2x32-20 block and JAX's counter layouts / uniform conversion
 *     (param_decomp/param_decomp/core/linear_plan.py:80-106 draws with jax.random.uniform)
 *   - the per-component gate MLP (spd_paper.md appendix), lower/upper leaky squashing
 *     (param_decomp/param_decomp/core/ci_fn/squashing.py:8-45)
 *   - m = g + (1-g) u (core/masking.py:135-136), site_forward
 *     (core/decomposed_linear.py:142-175), MSE recon and the L_p imp-min, and the
 *     backward of all of it.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

void or_threefry2x32(uint32_t k0, uint32_t k1, uint32_t x0, uint32_t x1, uint32_t *y0, uint32_t *y1) {
  static const int R[8] = {13, 15, 26, 6, 17, 29, 16, 24};
  uint32_t ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
  x0 += ks[0];
  x1 += ks[1];
  for (int b = 0; b < 5; ++b) {
    for (int i = 0; i < 4; ++i) {
      x0 += x1;
      x1 = rotl32(x1, R[(b & 1) * 4 + i]);
      x1 ^= x0;
    }
    x0 += ks[(b + 1) % 3];
    x1 += ks[(b + 2) % 3] + (uint32_t)(b + 1);
  }
  *y0 = x0;
  *y1 = x1;
}

/* Uniform [0,1) draw of n elements in JAX's partitionable layout. bf16 != 0 gives the
 * bfloat16 draw (8 random bits, top 7 kept) as exact float values. */
void or_uniform(uint32_t k0, uint32_t k1, int64_t n, int bf16, float *out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    uint32_t y0, y1;
    or_threefry2x32(k0, k1, (uint32_t)((uint64_t)i >> 32), (uint32_t)i, &y0, &y1);
    uint32_t b = y0 ^ y1;
    out[i] = bf16 ? (float)((b & 0xFFu) >> 1) * (1.0f / 128.0f) : (float)(b >> 9) * (1.0f / 8388608.0f);
  }
}

/* C[M,N] (+)= op(A) @ op(B), row-major, fp32, cache-blocked, OpenMP over row blocks.
 * ta: A is stored [K,M]; tb: B is stored [N,K]. */
static void gemm(int M, int N, int K, const float *A, int ta, const float *B, int tb, float *Cm, int accumulate) {
  float *At = NULL, *Bt = NULL;
  const float *a = A, *bm = B;
  if (ta) {
    At = (float *)malloc(sizeof(float) * (size_t)M * K);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i)
      for (int k = 0; k < K; ++k) At[(size_t)i * K + k] = A[(size_t)k * M + i];
    a = At;
  }
  if (tb) {
    Bt = (float *)malloc(sizeof(float) * (size_t)K * N);
#pragma omp parallel for schedule(static)
    for (int k = 0; k < K; ++k)
      for (int j = 0; j < N; ++j) Bt[(size_t)k * N + j] = B[(size_t)j * K + k];
    bm = Bt;
  }
  if (!accumulate) memset(Cm, 0, sizeof(float) * (size_t)M * N);
  const int KB = 128, NB = 512, MB = 16;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
  for (int i0 = 0; i0 < M; i0 += MB)
    for (int j0 = 0; j0 < N; j0 += NB) {
      int i1 = i0 + MB < M ? i0 + MB : M;
      int j1 = j0 + NB < N ? j0 + NB : N;
      for (int k0 = 0; k0 < K; k0 += KB) {
        int k1 = k0 + KB < K ? k0 + KB : K;
        for (int i = i0; i < i1; ++i) {
          float *crow = Cm + (size_t)i * N;
          for (int k = k0; k < k1; ++k) {
            float av = a[(size_t)i * K + k];
            const float *brow = bm + (size_t)k * N;
            for (int j = j0; j < j1; ++j) crow[j] += av * brow[j];
          }
        }
      }
    }
  free(At);
  free(Bt);
}

static inline float gelu_f(float z) { return 0.5f * z * (1.0f + erff(z * 0.70710678118654752f)); }
static inline float gelu_grad_f(float z) {
  return 0.5f * (1.0f + erff(z * 0.70710678118654752f)) + z * 0.39894228040143268f * expf(-0.5f * z * z);
}

/*
 * One dense-site stochastic-recon + L_p imp-min step (fp32), the same composition as
 * oracle.pd_oracle.dense_site_step. Shapes: x[T,din], W[dout,din], V[din,C], U[C,dout],
 * gate w_in/b_in/w_out [C,H], b_out[C]. mask_key / delta_key are the per-site keys
 * (already folded). use_delta selects the weight-delta channel. Outputs: losses[3] =
 * {loss, recon, imp}; dV[din,C], dU[C,dout], dgate = {dw_in[C,H], db_in[C,H],
 * dw_out[C,H], db_out[C]} packed contiguously. Returns 0 on success.
 */
int or_dense_step(int T, int din, int dout, int C, int H, const float *x, const float *W, const float *V,
                  const float *U, const float *w_in, const float *b_in, const float *w_out, const float *b_out,
                  const uint32_t *mask_key, const uint32_t *delta_key, int use_delta, int bf16_mask, float p,
                  float imp_coeff, float recon_coeff, float *losses, float *dV, float *dU, float *dgate) {
  size_t TC = (size_t)T * C, TO = (size_t)T * dout;
  float *yt = malloc(sizeof(float) * TO), *y = malloc(sizeof(float) * TO);
  float *h = malloc(sizeof(float) * TC), *graw = malloc(sizeof(float) * TC);
  float *u = malloc(sizeof(float) * TC), *acts = malloc(sizeof(float) * TC);
  float *d = malloc(sizeof(float) * (size_t)T);
  if (!yt || !y || !h || !graw || !u || !acts || !d) return 1;
  gemm(T, dout, din, x, 0, W, 1, yt, 0);
  gemm(T, C, din, x, 0, V, 0, h, 0);
  or_uniform(mask_key[0], mask_key[1], (int64_t)TC, bf16_mask, u);
  if (use_delta)
    or_uniform(delta_key[0], delta_key[1], T, bf16_mask, d);
  else
    memset(d, 0, sizeof(float) * (size_t)T);
  double imp = 0.0;
#pragma omp parallel for schedule(static) reduction(+ : imp)
  for (int t = 0; t < T; ++t)
    for (int c = 0; c < C; ++c) {
      size_t i = (size_t)t * C + c;
      float hv = h[i], g = b_out[c];
      for (int j = 0; j < H; ++j) g += w_out[c * H + j] * gelu_f(w_in[c * H + j] * hv + b_in[c * H + j]);
      graw[i] = g;
      float lo = g < 0.f ? 0.f : (g > 1.f ? 1.f : g);
      float up = g > 1.f ? 1.f + 0.01f * (g - 1.f) : lo;
      imp += powf(up, p);
      float m = lo + (1.f - lo) * u[i];
      acts[i] = hv * (m - d[t]);
    }
  imp /= (double)T;
  gemm(T, dout, C, acts, 0, U, 0, y, 0);
  double rec = 0.0;
  float scale = recon_coeff * 2.0f / (float)TO;
#pragma omp parallel for schedule(static) reduction(+ : rec)
  for (size_t i = 0; i < TO; ++i) {
    float yv = y[i] + d[i / dout] * yt[i];
    float e = yv - yt[i];
    rec += (double)e * e;
    y[i] = scale * e; /* y now holds dy */
  }
  rec /= (double)TO;
  losses[0] = (float)(recon_coeff * rec + imp_coeff * imp);
  losses[1] = (float)rec;
  losses[2] = (float)imp;
  gemm(C, dout, T, acts, 1, y, 0, dU, 0);
  float *da = acts; /* acts no longer needed after dU */
  gemm(T, C, dout, y, 0, U, 1, da, 0);
  float *dwi = dgate, *dbi = dgate + (size_t)C * H, *dwo = dgate + 2 * (size_t)C * H, *dbo = dgate + 3 * (size_t)C * H;
  memset(dgate, 0, sizeof(float) * (3 * (size_t)C * H + C));
  int nth = 1;
#ifdef _OPENMP
  nth = omp_get_max_threads();
#endif
  size_t per = 3 * (size_t)C * H + C;
  float *part = calloc((size_t)nth * per, sizeof(float));
  if (!part) return 1;
  float imp_scale = imp_coeff / (float)T;
#pragma omp parallel
  {
    int tid = 0;
#ifdef _OPENMP
    tid = omp_get_thread_num();
#endif
    float *pw = part + (size_t)tid * per;
#pragma omp for schedule(static)
    for (int t = 0; t < T; ++t)
      for (int c = 0; c < C; ++c) {
        size_t i = (size_t)t * C + c;
        float hv = h[i], g = graw[i], dav = da[i];
        float lo = g < 0.f ? 0.f : (g > 1.f ? 1.f : g);
        float m = lo + (1.f - lo) * u[i];
        float dh = dav * (m - d[t]);
        float dlo = dav * hv * (1.f - u[i]);
        float dg = g <= 0.f ? (dlo < 0.f ? 0.01f * dlo : 0.f) : (g <= 1.f ? dlo : 0.f);
        float up = g > 1.f ? 1.f + 0.01f * (g - 1.f) : lo;
        float dup = imp_scale * p * powf(up, p - 1.f);
        float cg = g > 1.f ? 0.01f : ((g > 0.f && g < 1.f) ? 1.f : ((g == 0.f || g == 1.f) ? 0.5f : 0.f));
        dg += cg * dup;
        for (int j = 0; j < H; ++j) {
          int q = c * H + j;
          float z = w_in[q] * hv + b_in[q];
          float dz = dg * w_out[q] * gelu_grad_f(z);
          dh += dz * w_in[q];
          pw[q] += dz * hv;
          pw[(size_t)C * H + q] += dz;
          pw[2 * (size_t)C * H + q] += dg * gelu_f(z);
        }
        pw[3 * (size_t)C * H + c] += dg;
        h[i] = dh; /* h now holds dh */
      }
  }
  for (int tid = 0; tid < nth; ++tid)
    for (size_t q = 0; q < per; ++q) dgate[q] += part[(size_t)tid * per + q];
  (void)dwi; (void)dbi; (void)dwo; (void)dbo;
  gemm(din, C, T, x, 1, h, 0, dV, 0);
  free(part);
  free(yt); free(y); free(h); free(graw); free(u); free(acts); free(d);
  return 0;
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
