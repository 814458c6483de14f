/*
 * dspark_oracle.c — C (OpenMP) restatement of the verify hot path. TEST INFRASTRUCTURE ONLY:
 * used by tests/ to check large shapes and by bench.py as the timed CPU baseline.
 * Never linked into the product library.
 *
 *  orc_qmm        factored affine qmm (skinny_qmm.py:86-158; A.1): per group g,
 *                 acc = fma(bias, sum x, fma(scale, sum q*x, acc)) in fp32, like the kernel.
 *  orc_attention  causal-in-block GQA attention (multirow_attn.py:52-178; A.2) with an fp32
 *                 online softmax per row (exp, not the kernel's bf16 P: the exact definition).
 *  orc_route      softmax top-k with (logit desc, id asc) order and bf16 renormalisation
 *                 (mlx-lm SparseMoeBlock; see oracle/moe_ref.py).
 * Inputs are bf16 bit patterns (uint16) laid out as the GPU receives them.
 *
 * Build: oracle/Makefile -> oracle/_build/liboracle.so.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf(uint16_t h) {
  union { uint32_t u; float f; } c;
  c.u = (uint32_t)h << 16;
  return c.f;
}

static inline float bf16r(float f) {
  union { uint32_t u; float f; } c;
  c.f = f;
  if ((c.u & 0x7F800000u) == 0x7F800000u) return f; /* inf / nan */
  c.u = (c.u + 0x7FFFu + ((c.u >> 16) & 1u)) & 0xFFFF0000u;
  return c.f;
}

int orc_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

void orc_unpack(const uint32_t* w, int64_t words, int bits, int32_t* q) {
  const int f = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t i = 0; i < words; ++i)
    for (int s = 0; s < f; ++s) q[i * f + s] = (int32_t)((w[i] >> (bits * s)) & mask);
}

/* y[m, n] (fp32, before the bf16 store) */
void orc_qmm(const uint16_t* x, int64_t M, int64_t K, const uint32_t* w, const uint16_t* scales,
             const uint16_t* biases, int64_t N, int bits, float* y) {
  const int64_t G = K / 64;
  const int64_t wpr = K * bits / 32;
  float* xf = (float*)malloc(sizeof(float) * M * K);
  float* xs = (float*)malloc(sizeof(float) * M * G);
  for (int64_t i = 0; i < M * K; ++i) xf[i] = bf(x[i]);
  for (int64_t m = 0; m < M; ++m)
    for (int64_t g = 0; g < G; ++g) {
      float s = 0.f;
      for (int j = 0; j < 64; ++j) s += xf[m * K + g * 64 + j];
      xs[m * G + g] = s;
    }
#pragma omp parallel
  {
    float* q = (float*)malloc(sizeof(float) * K);
    int32_t* qi = (int32_t*)malloc(sizeof(int32_t) * K);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      orc_unpack(w + n * wpr, wpr, bits, qi);
      for (int64_t j = 0; j < K; ++j) q[j] = (float)qi[j];
      for (int64_t m = 0; m < M; ++m) {
        const float* xr = xf + m * K;
        float acc = 0.f;
        for (int64_t g = 0; g < G; ++g) {
          float p = 0.f;
          const float* qg = q + g * 64;
          const float* xg = xr + g * 64;
          for (int j = 0; j < 64; ++j) p += qg[j] * xg[j];
          acc = fmaf(bf(biases[n * G + g]), xs[m * G + g], fmaf(bf(scales[n * G + g]), p, acc));
        }
        y[m * N + n] = acc;
      }
    }
    free(q);
    free(qi);
  }
  free(xf);
  free(xs);
}

/* out fp32 [B, Hq, Mq, D]; k/v strides {batch, head, seq} in elements, last dim contiguous */
void orc_attention(const uint16_t* q, int64_t B, int64_t Hq, int64_t Mq, int64_t D, const uint16_t* k,
                   const uint16_t* v, const int64_t* ks, const int64_t* vs, int64_t Hk, int64_t L, float scale,
                   int causal, const uint32_t* anc, float* out) {
  const int64_t gqa = Hq / Hk;
  const int64_t tail0 = L - Mq;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < Hq; ++h) {
      const int64_t hk = h / gqa;
      float* qf = (float*)malloc(sizeof(float) * D);
      float* acc = (float*)malloc(sizeof(float) * D);
      for (int64_t i = 0; i < Mq; ++i) {
        const uint16_t* qr = q + ((b * Hq + h) * Mq + i) * D;
        for (int64_t d = 0; d < D; ++d) qf[d] = bf(qr[d]);
        float m = -INFINITY, l = 0.f;
        for (int64_t d = 0; d < D; ++d) acc[d] = 0.f;
        const int64_t kmax = causal ? tail0 + i : L - 1;
        for (int64_t j = 0; j < L; ++j) {
          int vis;
          if (anc) vis = (j < tail0) || ((anc[i] >> (j - tail0)) & 1u);
          else vis = j <= kmax;
          if (!vis) continue;
          const uint16_t* kr = k + b * ks[0] + hk * ks[1] + j * ks[2];
          float s = 0.f;
          for (int64_t d = 0; d < D; ++d) s += qf[d] * bf(kr[d]);
          s *= scale;
          const float mn = s > m ? s : m;
          const float a = expf(m - mn), p = expf(s - mn);
          l = l * a + p;
          const uint16_t* vr = v + b * vs[0] + hk * vs[1] + j * vs[2];
          for (int64_t d = 0; d < D; ++d) acc[d] = acc[d] * a + p * bf(vr[d]);
          m = mn;
        }
        float* o = out + ((b * Hq + h) * Mq + i) * D;
        for (int64_t d = 0; d < D; ++d) o[d] = acc[d] / l;
      }
      free(qf);
      free(acc);
    }
}

/* inds int32 [M, k], scores fp32 holding bf16 values [M, k] */
void orc_route(const uint16_t* logits, int64_t M, int64_t E, int64_t k, int renorm, int32_t* inds, float* scores) {
  for (int64_t t = 0; t < M; ++t) {
    const uint16_t* x = logits + t * E;
    double mx = -INFINITY, sum = 0.0;
    for (int64_t e = 0; e < E; ++e) mx = fmax(mx, (double)bf(x[e]));
    for (int64_t e = 0; e < E; ++e) sum += exp((double)bf(x[e]) - mx);
    unsigned char* taken = (unsigned char*)calloc((size_t)E, 1);
    float gs = 0.f;
    for (int64_t j = 0; j < k; ++j) {
      int64_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        if (taken[e]) continue;
        if (best < 0 || bf(x[e]) > bf(x[best])) best = e;
      }
      taken[best] = 1;
      inds[t * k + j] = (int32_t)best;
      const float g = bf16r((float)(exp((double)bf(x[best]) - mx) / sum));
      scores[t * k + j] = g;
      gs += g;
    }
    if (renorm) {
      const float den = bf16r(gs);
      for (int64_t j = 0; j < k; ++j) scores[t * k + j] = bf16r(scores[t * k + j] / den);
    }
    free(taken);
  }
}
