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
 *     backward of all of it;
 *   - the decomposed MoE stack step of oracle/moe_oracle.py (routing, stable bucketing,
 *     grouped expert products, the masked expert sites and their backward).
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

/* C[M,N] (+)= op(A) @ op(B), row-major, fp32, OpenMP over (row, column) blocks.
 * ta: A is stored [K,M]; tb: B is stored [N,K]. Transposed operands are copied to
 * row-major first; the inner kernel keeps a 4 x 16 block of C in eight 8-wide vector
 * registers over a 256-deep slice of k. */
typedef float v8f __attribute__((vector_size(32)));

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
  const int MB = 64, NB = 256, KB = 256;
#pragma omp parallel for schedule(dynamic, 1) collapse(2)
  for (int i0 = 0; i0 < M; i0 += MB)
    for (int j0 = 0; j0 < N; j0 += NB) {
      const int i1 = i0 + MB < M ? i0 + MB : M, j1 = j0 + NB < N ? j0 + NB : N;
      for (int k0 = 0; k0 < K; k0 += KB) {
        const int k1 = k0 + KB < K ? k0 + KB : K;
        int i = i0;
        for (; i + 4 <= i1; i += 4) {
          int j = j0;
          for (; j + 16 <= j1; j += 16) {
            v8f c[4][2];
            for (int r = 0; r < 4; ++r) {
              memcpy(&c[r][0], Cm + (size_t)(i + r) * N + j, 32);
              memcpy(&c[r][1], Cm + (size_t)(i + r) * N + j + 8, 32);
            }
            for (int k = k0; k < k1; ++k) {
              v8f b0, b1;
              memcpy(&b0, bm + (size_t)k * N + j, 32);
              memcpy(&b1, bm + (size_t)k * N + j + 8, 32);
              for (int r = 0; r < 4; ++r) {
                const float av = a[(size_t)(i + r) * K + k];
                c[r][0] += av * b0;
                c[r][1] += av * b1;
              }
            }
            for (int r = 0; r < 4; ++r) {
              memcpy(Cm + (size_t)(i + r) * N + j, &c[r][0], 32);
              memcpy(Cm + (size_t)(i + r) * N + j + 8, &c[r][1], 32);
            }
          }
          for (int r = 0; r < 4; ++r)
            for (int k = k0; k < k1; ++k) {
              const float av = a[(size_t)(i + r) * K + k];
              for (int jj = j; jj < j1; ++jj) Cm[(size_t)(i + r) * N + jj] += av * bm[(size_t)k * N + jj];
            }
        }
        for (; i < i1; ++i)
          for (int k = k0; k < k1; ++k) {
            const float av = a[(size_t)i * K + k];
            for (int jj = j0; jj < j1; ++jj) Cm[(size_t)i * N + jj] += av * bm[(size_t)k * N + jj];
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

/* ------------------------------------------------------------------------------------
 * The decomposed MoE stack step (fp32), the composition of oracle.moe_oracle.moe_stack_step
 * without its bf16 storage model: clean forward pinning each layer's top-k experts, the
 * masked forward with every routed expert's gate/up/down matrix decomposed (job space,
 * stable bucketing by expert, coefficients m - d with the weight-delta channel), MSE of the
 * final residuals + L_p imp-min over the selected upper CI, and the backward to every V/U
 * and the CI preactivations (through routing weights, the router softmax and the norm).
 * Shapes (row-major fp32): x0[T,d]; ln[L,d]; router[L,E,d]; Wg,Wu[L,E,d,f]; Wd[L,E,f,d];
 * Vg,Vu[L,E,d,c]; Ug,Uu[L,E,c,f]; Vd[L,E,f,c]; Ud[L,E,c,d]; ci_pre[L,3,T,k,c];
 * mkeys/dkeys[L,3,2] the per-(layer, site) mask and delta keys. Outputs: losses[3];
 * dVg..dUd in the V/U layouts; d_ci_pre like ci_pre; top_idx[L,T,k]. Returns 0.
 * ---------------------------------------------------------------------------------- */
static float silu_f(float x) { return x / (1.f + expf(-x)); }
static float silu_grad_f(float x) {
  float s = 1.f / (1.f + expf(-x));
  return s * (1.f + x * (1.f - s));
}
static float lower_vjp_f(float x, float g) { return x <= 0.f ? (g < 0.f ? 0.01f * g : 0.f) : (x <= 1.f ? g : 0.f); }
static float upper_f(float x) { return x > 1.f ? 1.f + 0.01f * (x - 1.f) : (x < 0.f ? 0.f : x); }
static float upper_vjp_f(float x, float g) {
  if (x > 1.f) return 0.01f * g;
  return (x > 0.f && x < 1.f) ? g : ((x == 0.f || x == 1.f) ? 0.5f * g : 0.f);
}

/* out[rows of group e] = lhs[rows] @ rhs[e] (rhs[e] [K,N]); trans: @ rhs[e]^T (rhs[e] [N,K]) */
static void gmm(const float *lhs, const float *rhs, const int *off, int E, int K, int N, int trans, float *out) {
  for (int e = 0; e < E; ++e) {
    int n = off[e + 1] - off[e];
    if (n > 0) gemm(n, N, K, lhs + (size_t)off[e] * K, 0, rhs + (size_t)e * K * N, trans, out + (size_t)off[e] * N, 0);
  }
}
/* out[e] = lhs[rows_e]^T @ dout[rows_e] ([K,N]); zero for empty groups */
static void gmm_dw(const float *lhs, const float *dout, const int *off, int E, int K, int N, float *out) {
  for (int e = 0; e < E; ++e) {
    int n = off[e + 1] - off[e];
    if (n > 0) gemm(K, N, n, lhs + (size_t)off[e] * K, 1, dout + (size_t)off[e] * N, 0, out + (size_t)e * K * N, 0);
    else memset(out + (size_t)e * K * N, 0, sizeof(float) * (size_t)K * N);
  }
}
static void rms_fwd(const float *x, const float *w, int T, int d, float eps, float *y, float *rinv) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    const float *xr = x + (size_t)t * d;
    double ss = 0.0;
    for (int i = 0; i < d; ++i) ss += (double)xr[i] * xr[i];
    float r = 1.f / sqrtf((float)(ss / d) + eps);
    if (rinv) rinv[t] = r;
    for (int i = 0; i < d; ++i) y[(size_t)t * d + i] = xr[i] * r * (1.f + w[i]);
  }
}
/* routing of one layer: probs [T,E] from logits; idx [T,k] (stable descending, lowest index
 * on ties) unless pinned; w [T,k] renormalized; jobs sorted stably by expert. */
static void route(const float *logits, int T, int E, int k, int pinned, int *idx, float *probs, float *w, int *sort_idx,
                  int *inv, int *off) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; ++t) {
    const float *l = logits + (size_t)t * E;
    float mx = l[0];
    for (int e = 1; e < E; ++e) mx = l[e] > mx ? l[e] : mx;
    double z = 0.0;
    for (int e = 0; e < E; ++e) z += exp((double)l[e] - mx);
    float *p = probs + (size_t)t * E;
    for (int e = 0; e < E; ++e) p[e] = (float)(exp((double)l[e] - mx) / z);
    int *id = idx + (size_t)t * k;
    if (!pinned)
      for (int s = 0; s < k; ++s) {
        int best = -1;
        for (int e = 0; e < E; ++e) {
          int taken = 0;
          for (int q = 0; q < s; ++q) taken |= id[q] == e;
          if (!taken && (best < 0 || p[e] > p[best])) best = e;
        }
        id[s] = best;
      }
    float sum = 0.f;
    for (int s = 0; s < k; ++s) sum += p[id[s]];
    for (int s = 0; s < k; ++s) w[(size_t)t * k + s] = p[id[s]] / sum;
  }
  int J = T * k;
  memset(off, 0, sizeof(int) * (E + 1));
  for (int j = 0; j < J; ++j) off[idx[j] + 1]++;
  for (int e = 0; e < E; ++e) off[e + 1] += off[e];
  int *pos = (int *)malloc(sizeof(int) * E);
  memcpy(pos, off, sizeof(int) * E);
  for (int j = 0; j < J; ++j) {
    int p = pos[idx[j]]++;
    sort_idx[p] = j;
    inv[j] = p;
  }
  free(pos);
}

/* A grow-only bump arena for the MoE restatement's buffers, kept across calls so that a
 * timed call does not pay first-touch page faults (test infrastructure: one caller at a
 * time). */
static char *g_arena = NULL;
static size_t g_arena_cap = 0, g_arena_off = 0, g_arena_need = 0;
static void *g_heap[4096];
static int g_nheap = 0;
static void arena_reset(void) {
  for (int i = 0; i < g_nheap; ++i) free(g_heap[i]);
  g_nheap = 0;
  if (g_arena_need > g_arena_cap) {
    free(g_arena);
    g_arena = (char *)malloc(g_arena_need);
    g_arena_cap = g_arena ? g_arena_need : 0;
  }
  g_arena_off = 0;
  g_arena_need = 0;
}
static void *arena_take(size_t bytes) {
  bytes = (bytes + 63) & ~(size_t)63;
  g_arena_need += bytes;
  if (g_arena_off + bytes <= g_arena_cap) {
    void *p = g_arena + g_arena_off;
    g_arena_off += bytes;
    return p;
  }
  /* past the arena (the first call at a size): the heap, released at the next reset,
   * when the arena grows to this call's total */
  void *p = malloc(bytes);
  if (p && g_nheap < 4096) g_heap[g_nheap++] = p;
  return p;
}

typedef struct {
  float *r, *h2, *rinv, *probs, *w, *xj, *din, *gq, *uq, *wj, *dj;
  int *idx, *sort_idx, *inv, *off;
  float *h[3], *coef[3], *u[3], *pre_lo[3];
} MoELayer;

int or_moe_step(int T, int d, int f, int E, int k, int c, int L, const float *x0, const float *ln, const float *router,
                const float *Wg, const float *Wu, const float *Wd, const float *Vg, const float *Ug, const float *Vu,
                const float *Uu, const float *Vd, const float *Ud, const float *ci_pre, const uint32_t *mkeys,
                const uint32_t *dkeys, int use_delta, float p, float imp_coeff, float recon_coeff, float *losses,
                float *dVg, float *dUg, float *dVu, float *dUu, float *dVd, float *dUd, float *d_ci_pre,
                int32_t *top_idx) {
  const int J = T * k;
  const float eps = 1e-6f;
  const size_t szW = (size_t)E * d * f, szVd = (size_t)E * f * c, szVg = (size_t)E * d * c;
  const size_t szUg = (size_t)E * c * f, szUd = (size_t)E * c * d, szCI = (size_t)J * c;
  const float *Vs[3] = {Vg, Vu, Vd}, *Us[3] = {Ug, Uu, Ud}, *Ws[3] = {Wg, Wu, Wd};
  const size_t szV[3] = {szVg, szVg, szVd}, szU[3] = {szUg, szUg, szUd};
  float *dVs[3] = {dVg, dVu, dVd}, *dUs[3] = {dUg, dUu, dUd};
  arena_reset();
  MoELayer *S = (MoELayer *)arena_take(sizeof(MoELayer) * L);
  memset(S, 0, sizeof(MoELayer) * L);
  float *rc = (float *)arena_take(sizeof(float) * T * d), *logits = (float *)arena_take(sizeof(float) * T * E);
  float *tmpJ = (float *)arena_take(sizeof(float) * (size_t)J * (f > d ? f : d));
  float *tmpJ2 = (float *)arena_take(sizeof(float) * (size_t)J * (f > d ? f : d));
  float *h2c = (float *)arena_take(sizeof(float) * T * d);
  if (!S || !rc || !logits || !tmpJ || !tmpJ2 || !h2c) return 1;
  /* ---------------- clean forward */
  memcpy(rc, x0, sizeof(float) * T * d);
  for (int l = 0; l < L; ++l) {
    MoELayer *Z = &S[l];
    Z->idx = (int *)arena_take(sizeof(int) * J);
    Z->sort_idx = (int *)arena_take(sizeof(int) * J);
    Z->inv = (int *)arena_take(sizeof(int) * J);
    Z->off = (int *)arena_take(sizeof(int) * (E + 1));
    Z->probs = (float *)arena_take(sizeof(float) * T * E);
    Z->w = (float *)arena_take(sizeof(float) * T * k);
    rms_fwd(rc, ln + (size_t)l * d, T, d, eps, h2c, NULL);
    gemm(T, E, d, h2c, 0, router + (size_t)l * E * d, 1, logits, 0);
    route(logits, T, E, k, 0, Z->idx, Z->probs, Z->w, Z->sort_idx, Z->inv, Z->off);
    float *xj = (float *)arena_take(sizeof(float) * (size_t)J * d);
#pragma omp parallel for schedule(static)
    for (int j = 0; j < J; ++j) memcpy(xj + (size_t)j * d, h2c + (size_t)(Z->sort_idx[j] / k) * d, sizeof(float) * d);
    gmm(xj, Wg + l * szW, Z->off, E, d, f, 0, tmpJ);
    gmm(xj, Wu + l * szW, Z->off, E, d, f, 0, tmpJ2);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < (size_t)J * f; ++i) tmpJ[i] = silu_f(tmpJ[i]) * tmpJ2[i];
    gmm(tmpJ, Wd + l * szW, Z->off, E, f, d, 0, tmpJ2);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t)
      for (int s = 0; s < k; ++s) {
        float wv = Z->w[(size_t)t * k + s];
        const float *row = tmpJ2 + (size_t)Z->inv[t * k + s] * d;
        for (int i = 0; i < d; ++i) rc[(size_t)t * d + i] += wv * row[i];
      }
    for (int j = 0; j < J; ++j) top_idx[(size_t)l * J + j] = Z->idx[j];
  }
  /* ---------------- masked forward */
  float *r = (float *)arena_take(sizeof(float) * T * d);
  memcpy(r, x0, sizeof(float) * T * d);
  double imp = 0.0;
  for (int l = 0; l < L; ++l) {
    MoELayer *Z = &S[l];
    Z->r = (float *)arena_take(sizeof(float) * T * d);
    memcpy(Z->r, r, sizeof(float) * T * d);
    Z->h2 = (float *)arena_take(sizeof(float) * T * d);
    Z->rinv = (float *)arena_take(sizeof(float) * T);
    rms_fwd(r, ln + (size_t)l * d, T, d, eps, Z->h2, Z->rinv);
    gemm(T, E, d, Z->h2, 0, router + (size_t)l * E * d, 1, logits, 0);
    route(logits, T, E, k, 1, Z->idx, Z->probs, Z->w, Z->sort_idx, Z->inv, Z->off);
    Z->xj = (float *)arena_take(sizeof(float) * (size_t)J * d);
    Z->wj = (float *)arena_take(sizeof(float) * J);
    Z->dj = (float *)arena_take(sizeof(float) * 3 * J);
#pragma omp parallel for schedule(static)
    for (int j = 0; j < J; ++j) {
      memcpy(Z->xj + (size_t)j * d, Z->h2 + (size_t)(Z->sort_idx[j] / k) * d, sizeof(float) * d);
      Z->wj[j] = Z->w[Z->sort_idx[j]];
    }
    float *dtok = (float *)arena_take(sizeof(float) * T);
    for (int si = 0; si < 3; ++si) {
      const float *pre = ci_pre + ((size_t)l * 3 + si) * szCI;
      Z->u[si] = (float *)arena_take(sizeof(float) * szCI);
      or_uniform(mkeys[(l * 3 + si) * 2], mkeys[(l * 3 + si) * 2 + 1], (int64_t)szCI, 1, Z->u[si]);
      if (use_delta) or_uniform(dkeys[(l * 3 + si) * 2], dkeys[(l * 3 + si) * 2 + 1], T, 1, dtok);
      else memset(dtok, 0, sizeof(float) * T);
      Z->coef[si] = (float *)arena_take(sizeof(float) * szCI);
      double ims = 0.0;
#pragma omp parallel for schedule(static) reduction(+ : ims)
      for (size_t i = 0; i < szCI; ++i) ims += powf(upper_f(pre[i]), p);
      imp += ims / T;
#pragma omp parallel for schedule(static)
      for (int j = 0; j < J; ++j) {
        int slot = Z->sort_idx[j];
        float dv = dtok[slot / k];
        Z->dj[(size_t)si * J + j] = dv;
        for (int q = 0; q < c; ++q) {
          size_t src = (size_t)slot * c + q;
          float lo = pre[src] < 0.f ? 0.f : (pre[src] > 1.f ? 1.f : pre[src]);
          Z->coef[si][(size_t)j * c + q] = lo + (1.f - lo) * Z->u[si][src] - dv;
        }
      }
    }
    /* gate, up */
    float *outs[2];
    for (int si = 0; si < 2; ++si) {
      Z->h[si] = (float *)arena_take(sizeof(float) * (size_t)J * c);
      gmm(Z->xj, Vs[si] + l * szV[si], Z->off, E, d, c, 0, Z->h[si]);
      float *acts = (float *)arena_take(sizeof(float) * (size_t)J * c);
#pragma omp parallel for schedule(static)
      for (size_t i = 0; i < (size_t)J * c; ++i) acts[i] = Z->h[si][i] * Z->coef[si][i];
      outs[si] = (float *)arena_take(sizeof(float) * (size_t)J * f);
      gmm(acts, Us[si] + l * szU[si], Z->off, E, c, f, 0, outs[si]);
      gmm(Z->xj, Ws[si] + l * szW, Z->off, E, d, f, 0, tmpJ);
#pragma omp parallel for schedule(static)
      for (int j = 0; j < J; ++j)
        for (int q = 0; q < f; ++q) outs[si][(size_t)j * f + q] += Z->dj[(size_t)si * J + j] * tmpJ[(size_t)j * f + q];
    }
    Z->gq = outs[0];
    Z->uq = outs[1];
    Z->din = (float *)arena_take(sizeof(float) * (size_t)J * f);
#pragma omp parallel for schedule(static)
    for (int j = 0; j < J; ++j)
      for (int q = 0; q < f; ++q) {
        size_t i = (size_t)j * f + q;
        Z->din[i] = silu_f(Z->gq[i]) * Z->uq[i] * Z->wj[j];
      }
    Z->h[2] = (float *)arena_take(sizeof(float) * (size_t)J * c);
    gmm(Z->din, Vd + l * szVd, Z->off, E, f, c, 0, Z->h[2]);
    float *acts = (float *)arena_take(sizeof(float) * (size_t)J * c);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < (size_t)J * c; ++i) acts[i] = Z->h[2][i] * Z->coef[2][i];
    gmm(acts, Ud + l * szUd, Z->off, E, c, d, 0, tmpJ2);
    gmm(Z->din, Wd + l * szW, Z->off, E, f, d, 0, tmpJ);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t)
      for (int s = 0; s < k; ++s) {
        int j = Z->inv[t * k + s];
        float dv = Z->dj[2 * (size_t)J + j];
        for (int i = 0; i < d; ++i) r[(size_t)t * d + i] += tmpJ2[(size_t)j * d + i] + dv * tmpJ[(size_t)j * d + i];
      }
  }
  /* ---------------- losses */
  const size_t n = (size_t)T * d;
  double rec = 0.0;
#pragma omp parallel for schedule(static) reduction(+ : rec)
  for (size_t i = 0; i < n; ++i) rec += (double)(r[i] - rc[i]) * (r[i] - rc[i]);
  rec /= (double)n;
  losses[0] = (float)(recon_coeff * rec + imp_coeff * imp);
  losses[1] = (float)rec;
  losses[2] = (float)imp;
  /* ---------------- backward */
  float *dr = (float *)arena_take(sizeof(float) * n);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) dr[i] = recon_coeff * 2.f * (r[i] - rc[i]) / (float)n;
  float *d_dout = (float *)arena_take(sizeof(float) * (size_t)J * d);
  float *d_acts = (float *)arena_take(sizeof(float) * (size_t)J * c);
  float *d_h = (float *)arena_take(sizeof(float) * (size_t)J * c);
  float *d_din = (float *)arena_take(sizeof(float) * (size_t)J * f);
  float *d_go[2] = {(float *)arena_take(sizeof(float) * (size_t)J * f), (float *)arena_take(sizeof(float) * (size_t)J * f)};
  float *d_xj = (float *)arena_take(sizeof(float) * (size_t)J * d);
  float *dm[3];
  float *d_wj = (float *)arena_take(sizeof(float) * J);
  float *dh2 = (float *)arena_take(sizeof(float) * n);
  float *d_logits = (float *)arena_take(sizeof(float) * T * E);
  const float imp_scale = imp_coeff / (float)T;
  for (int l = L - 1; l >= 0; --l) {
    MoELayer *Z = &S[l];
    for (int si = 0; si < 3; ++si) dm[si] = (float *)arena_take(sizeof(float) * (size_t)J * c);
#pragma omp parallel for schedule(static)
    for (int j = 0; j < J; ++j) memcpy(d_dout + (size_t)j * d, dr + (size_t)(Z->sort_idx[j] / k) * d, sizeof(float) * d);
    /* down */
    gmm(d_dout, Ud + l * szUd, Z->off, E, d, c, 1, d_acts);
    float *acts = (float *)arena_take(sizeof(float) * (size_t)J * c);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < (size_t)J * c; ++i) {
      acts[i] = Z->h[2][i] * Z->coef[2][i];
      dm[2][i] = d_acts[i] * Z->h[2][i];
      d_h[i] = d_acts[i] * Z->coef[2][i];
    }
    gmm_dw(acts, d_dout, Z->off, E, c, d, dUd + l * szUd);
    gmm_dw(Z->din, d_h, Z->off, E, f, c, dVd + l * szVd);
    gmm(d_h, Vd + l * szVd, Z->off, E, c, f, 1, d_din);
    gmm(d_dout, Wd + l * szW, Z->off, E, d, f, 1, tmpJ);
#pragma omp parallel for schedule(static)
    for (int j = 0; j < J; ++j) {
      float dv = Z->dj[2 * (size_t)J + j], dw = 0.f;
      for (int q = 0; q < f; ++q) {
        size_t i = (size_t)j * f + q;
        float dd = d_din[i] + dv * tmpJ[i];
        float g = Z->gq[i], u = Z->uq[i], sg = silu_f(g);
        d_go[0][i] = dd * u * Z->wj[j] * silu_grad_f(g);
        d_go[1][i] = dd * sg * Z->wj[j];
        dw += dd * sg * u;
      }
      d_wj[j] = dw;
    }
    memset(d_xj, 0, sizeof(float) * (size_t)J * d);
    for (int si = 0; si < 2; ++si) {
      gmm(d_go[si], Us[si] + l * szU[si], Z->off, E, f, c, 1, d_acts);
#pragma omp parallel for schedule(static)
      for (size_t i = 0; i < (size_t)J * c; ++i) {
        acts[i] = Z->h[si][i] * Z->coef[si][i];
        dm[si][i] = d_acts[i] * Z->h[si][i];
        d_h[i] = d_acts[i] * Z->coef[si][i];
      }
      gmm_dw(acts, d_go[si], Z->off, E, c, f, dUs[si] + l * szU[si]);
      gmm_dw(Z->xj, d_h, Z->off, E, d, c, dVs[si] + l * szV[si]);
      gmm(d_h, Vs[si] + l * szV[si], Z->off, E, c, d, 1, tmpJ);
      gmm(d_go[si], Ws[si] + l * szW, Z->off, E, f, d, 1, tmpJ2);
#pragma omp parallel for schedule(static)
      for (int j = 0; j < J; ++j) {
        float dv = Z->dj[(size_t)si * J + j];
        for (int q = 0; q < d; ++q) d_xj[(size_t)j * d + q] += tmpJ[(size_t)j * d + q] + dv * tmpJ2[(size_t)j * d + q];
      }
    }
    /* mask pullback to the CI preactivations (token-major) */
    for (int si = 0; si < 3; ++si) {
      const float *pre = ci_pre + ((size_t)l * 3 + si) * szCI;
      float *dp = d_ci_pre + ((size_t)l * 3 + si) * szCI;
#pragma omp parallel for schedule(static)
      for (int j = 0; j < J; ++j) {
        int slot = Z->sort_idx[j];
        for (int q = 0; q < c; ++q) {
          size_t src = (size_t)slot * c + q;
          float x = pre[src];
          float up = upper_f(x);
          float dup = imp_scale * p * powf(up, p - 1.f);
          dp[src] = lower_vjp_f(x, dm[si][(size_t)j * c + q] * (1.f - Z->u[si][src])) + upper_vjp_f(x, dup);
        }
      }
    }
    /* routing weights -> probs -> logits; gather VJP; router; norm */
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
      const float *pr = Z->probs + (size_t)t * E;
      const int *id = Z->idx + (size_t)t * k;
      float dwv[64], ssum = 0.f, dot = 0.f;
      for (int s = 0; s < k; ++s) {
        dwv[s] = d_wj[Z->inv[t * k + s]];
        ssum += pr[id[s]];
        dot += dwv[s] * Z->w[(size_t)t * k + s];
      }
      float *dl = d_logits + (size_t)t * E;
      for (int e = 0; e < E; ++e) dl[e] = 0.f;
      for (int s = 0; s < k; ++s) dl[id[s]] += (dwv[s] - dot) / ssum;
      float sdot = 0.f;
      for (int e = 0; e < E; ++e) sdot += pr[e] * dl[e];
      for (int e = 0; e < E; ++e) dl[e] = pr[e] * (dl[e] - sdot);
      for (int i = 0; i < d; ++i) {
        float acc = 0.f;
        for (int s = 0; s < k; ++s) acc += d_xj[(size_t)Z->inv[t * k + s] * d + i];
        dh2[(size_t)t * d + i] = acc;
      }
    }
    gemm(T, d, E, d_logits, 0, router + (size_t)l * E * d, 0, dh2, 1);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
      const float *x = Z->r + (size_t)t * d, *w = ln + (size_t)l * d;
      float rr = Z->rinv[t];
      double dot = 0.0;
      for (int i = 0; i < d; ++i) dot += (double)(1.f + w[i]) * dh2[(size_t)t * d + i] * x[i];
      float cc = (float)(dot / d) * rr * rr * rr;
      for (int i = 0; i < d; ++i) dr[(size_t)t * d + i] += rr * (1.f + w[i]) * dh2[(size_t)t * d + i] - x[i] * cc;
    }
  }
  return 0;
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
