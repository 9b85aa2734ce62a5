/*
 * moe_oracle.c -- CPU restatement of com.microsoft MoE / QMoE (ORT 1.26 CPU EP
 * semantics).  TEST INFRASTRUCTURE ONLY: the product library never links it.
 * See moe_oracle.h for the algorithm and its provenance.
 *
 * Build: oracle/Makefile  (gcc -O2 -fopenmp -shared).
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* Scalar conversions.  fp16 per IEEE 754 binary16, round-to-nearest-even.
 * bf16 per the reference's test helper float32_to_bfloat16_bits
 * (test/ops/op_test_utils.py:235-245): add 0x7FFF + lsb, keep the top half. */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
  if (exp == 0) {
    float v = ldexpf((float)mant, -24); /* subnormal or zero, exact */
    return sign ? -v : v;
  }
  if (exp == 31) return u2f(sign | 0x7F800000u | (mant << 13));
  return u2f(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

uint16_t orc_f32_to_f16(float f) {
  uint32_t x = f2u(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u);
  if (ax >= 0x477FF000u) return sign | 0x7C00u; /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {                       /* below 2^-14: fp16 subnormal */
    float v = u2f(ax) * 16777216.0f;            /* exact scale by 2^24 */
    return sign | (uint16_t)nearbyintf(v);      /* RNE (default rounding mode) */
  }
  uint32_t mant = ax & 0x7FFFFFu;
  uint32_t h = ((((ax >> 23) - 127 + 15)) << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return sign | (uint16_t)h;
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_f32_to_bf16(float f) {
  uint32_t x = f2u(f);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7FFFu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

static float load_f(const void *p, int32_t dt, int64_t i) {
  switch (dt) {
    case ORC_F32: return ((const float *)p)[i];
    case ORC_F16: return orc_f16_to_f32(((const uint16_t *)p)[i]);
    case ORC_BF16: return orc_bf16_to_f32(((const uint16_t *)p)[i]);
    default: return NAN;
  }
}

static void store_f(void *p, int32_t dt, int64_t i, float v) {
  switch (dt) {
    case ORC_F32: ((float *)p)[i] = v; break;
    case ORC_F16: ((uint16_t *)p)[i] = orc_f32_to_f16(v); break;
    case ORC_BF16: ((uint16_t *)p)[i] = orc_f32_to_bf16(v); break;
    default: break;
  }
}

/* ------------------------------------------------------------------ */
/* Router.  Softmax follows the reference's max-subtracted fp32 softmax
 * (musa/ep/src/kernels/math/softmax_impl.mu:61-82); selection is a top-k on
 * the logits ordered by (value desc, id asc), the reference TopK tie rule
 * (musa/ep/src/kernels/math/topk_impl.mu:46-65). */

static int before(float va, int32_t ia, float vb, int32_t ib) {
  if (va > vb) return 1;
  if (vb > va) return 0;
  return ia < ib;
}

int orc_route(const float *logits, int64_t T, int64_t E, int64_t k, int32_t normalize,
              int32_t sigmoid, int32_t *ids, float *w) {
  if (T < 0 || E <= 0 || k <= 0 || k > E) return 1;
  float *p = (float *)malloc(sizeof(float) * (size_t)E);
  if (!p) return 2;
  float *l = (float *)malloc(sizeof(float) * (size_t)E);
  if (!l) { free(p); return 2; }
  for (int64_t t = 0; t < T; ++t) {
    /* NaN logits rank below every number (as -inf) */
    for (int64_t e = 0; e < E; ++e) {
      const float v = logits[t * E + e];
      l[e] = v != v ? -INFINITY : v;
    }
    if (sigmoid) {
      for (int64_t e = 0; e < E; ++e) p[e] = 1.0f / (1.0f + expf(-l[e]));
    } else {
      float m = l[0];
      for (int64_t e = 1; e < E; ++e) m = l[e] > m ? l[e] : m;
      float s = 0.0f;
      for (int64_t e = 0; e < E; ++e) { p[e] = expf(l[e] - m); s += p[e]; }
      for (int64_t e = 0; e < E; ++e) p[e] = p[e] / s;
    }
    /* k rounds of arg-max over the not-yet-chosen experts */
    int32_t *id = ids + t * k;
    for (int64_t j = 0; j < k; ++j) {
      int32_t best = -1;
      for (int64_t e = 0; e < E; ++e) {
        int taken = 0;
        for (int64_t q = 0; q < j; ++q) taken |= (id[q] == (int32_t)e);
        if (taken) continue;
        if (best < 0 || before(l[e], (int32_t)e, l[best], best)) best = (int32_t)e;
      }
      id[j] = best;
    }
    float sum = 0.0f;
    for (int64_t j = 0; j < k; ++j) { w[t * k + j] = p[id[j]]; sum += p[id[j]]; }
    if (normalize)
      for (int64_t j = 0; j < k; ++j) w[t * k + j] = w[t * k + j] / sum;
  }
  free(l);
  free(p);
  return 0;
}

/* ------------------------------------------------------------------ */
/* Dispatch: counting sort of the flat (t*k + j) entries by expert id, stable
 * in the flat index, i.e. expert-major with ascending token id inside an
 * expert (a token never picks one expert twice). */
int orc_dispatch(const int32_t *ids, int64_t T, int64_t k, int64_t E, int32_t *offsets,
                 int32_t *perm) {
  if (E <= 0 || T < 0 || k <= 0) return 1;
  int64_t n = T * k;
  for (int64_t e = 0; e <= E; ++e) offsets[e] = 0;
  for (int64_t f = 0; f < n; ++f) {
    if (ids[f] < 0 || ids[f] >= E) return 1;
    offsets[ids[f] + 1]++;
  }
  for (int64_t e = 0; e < E; ++e) offsets[e + 1] += offsets[e];
  int32_t *fill = (int32_t *)calloc((size_t)E, sizeof(int32_t));
  if (!fill) return 2;
  for (int64_t f = 0; f < n; ++f) {
    int32_t e = ids[f];
    perm[offsets[e] + fill[e]++] = (int32_t)f;
  }
  free(fill);
  return 0;
}

/* ------------------------------------------------------------------ */
/* Dequantization of one row (symmetric, zero point 128 for int8 and 8 for
 * int4, even-k element in the low nibble). */
static void dequant_row(const uint8_t *q, const void *scales, int32_t sdt, int32_t bits,
                        int64_t block_size, int64_t n, int64_t K, float *out) {
  int64_t row_bytes = bits == 8 ? K : K / 2;
  const uint8_t *r = q + n * row_bytes;
  int64_t nblk = block_size > 0 ? K / block_size : 1;
  for (int64_t kk = 0; kk < K; ++kk) {
    float s = load_f(scales, sdt, n * nblk + (block_size > 0 ? kk / block_size : 0));
    int v;
    if (bits == 8) v = (int)r[kk] - 128;
    else v = (int)((kk & 1) ? (r[kk >> 1] >> 4) : (r[kk >> 1] & 0x0F)) - 8;
    out[kk] = (float)v * s;
  }
}

int orc_dequant(const uint8_t *q, const void *scales, int32_t scale_dtype, int32_t bits,
                int64_t block_size, int64_t N, int64_t K, float *out) {
  if (bits != 4 && bits != 8) return 1;
  for (int64_t n = 0; n < N; ++n)
    dequant_row(q, scales, scale_dtype, bits, block_size, n, K, out + n * K);
  return 0;
}

/* MXFP4 per the OCP Microscaling Formats (MX) v1.0 specification: an FP4
 * E2M1 element (sign, 2 exponent bits with bias 1, 1 mantissa bit; exponent
 * 0 is subnormal: 0 or 0.5) times the block's E8M0 scale (2^(e - 127), the
 * byte 0xFF encoding NaN).  Public format (openai/gpt-oss ships its expert
 * weights in it); no reference file restates it. */
float orc_e2m1_to_f32(uint32_t nib) {
  const uint32_t e = (nib >> 1) & 3u, m = nib & 1u;
  const float mag = e == 0 ? 0.5f * (float)m : ldexpf(1.0f + 0.5f * (float)m, (int)e - 1);
  return (nib & 8u) ? -mag : mag;
}

float orc_e8m0_to_f32(uint32_t e) { return e == 255u ? NAN : ldexpf(1.0f, (int)e - 127); }

static void dequant_row_mxfp4(const uint8_t *q, const uint8_t *scales, int64_t n, int64_t K, float *out) {
  const uint8_t *r = q + n * (K / 2);
  const uint8_t *s = scales + n * (K / 32);
  for (int64_t kk = 0; kk < K; ++kk) {
    const uint32_t nib = (kk & 1) ? (r[kk >> 1] >> 4) : (r[kk >> 1] & 0x0F);
    out[kk] = orc_e2m1_to_f32(nib) * orc_e8m0_to_f32(s[kk / 32]);
  }
}

int orc_dequant_mxfp4(const uint8_t *q, const uint8_t *scales, int64_t N, int64_t K, float *out) {
  if (K % 32) return 1;
  for (int64_t n = 0; n < N; ++n) dequant_row_mxfp4(q, scales, n, K, out + n * K);
  return 0;
}

/* Weight row n of one expert matrix [N, K] as fp32. */
static void weight_row(const orc_moe_args *a, const void *w, const void *s, int64_t e,
                       int64_t N, int64_t K, int64_t n, float *out) {
  if (a->quant_bits == 0) {
    const int64_t base = (e * N + n) * K;
    for (int64_t kk = 0; kk < K; ++kk) out[kk] = load_f(w, a->act_dtype, base + kk);
    return;
  }
  const int64_t row_bytes = a->quant_bits == 8 ? K : K / 2;
  if (a->weight_format == 1) {
    dequant_row_mxfp4((const uint8_t *)w + e * N * row_bytes, (const uint8_t *)s + e * N * (K / 32), n, K, out);
    return;
  }
  const int64_t nblk = a->block_size > 0 ? K / a->block_size : 1;
  const uint8_t *qe = (const uint8_t *)w + e * N * row_bytes;
  const int64_t soff = e * N * nblk;
  /* scales pointer offset by expert: element offset soff */
  const size_t esz = a->scale_dtype == ORC_F32 ? 4 : 2;
  dequant_row(qe, (const uint8_t *)s + soff * esz, a->scale_dtype, a->quant_bits,
              a->block_size, n, K, out);
}

/* fp32 dot product with a fixed 8-way blocked summation order. */
static float dot8(const float *x, const float *w, int64_t K) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t kk = 0;
  for (; kk + 8 <= K; kk += 8)
    for (int l = 0; l < 8; ++l) acc[l] += x[kk + l] * w[kk + l];
  for (int l = 0; kk < K; ++kk, ++l) acc[l] += x[kk] * w[kk];
  return ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
}

static float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

static float act1(float x, int32_t act) {
  switch (act) {
    case ORC_ACT_RELU: return x > 0.0f ? x : 0.0f;
    case ORC_ACT_GELU: return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f));
    case ORC_ACT_SILU: return x * sigm(x);
    default: return x;
  }
}

static float swiglu1(float g, float l, float alpha, float beta, float limit) {
  g = fminf(g, limit);
  l = fminf(fmaxf(l, -limit), limit);
  return g * sigm(alpha * g) * (l + beta);
}

void orc_activation(const float *h1, const float *h3, int64_t I, int32_t activation,
                    int32_t fusion, float alpha, float beta, float limit, float *a) {
  for (int64_t i = 0; i < I; ++i) {
    if (activation == ORC_ACT_SWIGLU) {
      float g, l;
      if (h3) { g = h1[i]; l = h3[i]; }
      else if (fusion == 1) { g = h1[2 * i]; l = h1[2 * i + 1]; }
      else { g = h1[i]; l = h1[I + i]; }
      a[i] = swiglu1(g, l, alpha, beta, limit);
    } else if (h3) {
      a[i] = act1(h1[i], activation) * h3[i];
    } else {
      a[i] = act1(h1[i], activation);
    }
  }
}

/* ------------------------------------------------------------------ */
int orc_moe_forward(const orc_moe_args *a) {
  const int64_t T = a->num_tokens, H = a->hidden, I = a->inter, E = a->num_experts,
                k = a->k;
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0 || k > E) return 1;
  if (a->quant_bits != 0 && a->quant_bits != 4 && a->quant_bits != 8) return 1;
  if (a->quant_bits == 4 && ((H & 1) || (I & 1))) return 1;
  if (a->block_size > 0 && (H % a->block_size || I % a->block_size)) return 1;
  if (a->weight_format == 1 && (a->quant_bits != 4 || a->block_size != 32)) return 1;
  const int gated3 = a->w3 != NULL;
  const int fused = (a->activation == ORC_ACT_SWIGLU && !gated3);
  if (fused && a->swiglu_fusion != 1 && a->swiglu_fusion != 2) return 1;
  const int64_t N1 = fused ? 2 * I : I;
#ifdef _OPENMP
  if (a->num_threads > 0) omp_set_num_threads(a->num_threads);
#endif

  /* 1. router */
  float *logits = (float *)malloc(sizeof(float) * (size_t)(T * E + 1));
  int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * (size_t)(T * k + 1));
  float *rw = (float *)malloc(sizeof(float) * (size_t)(T * k + 1));
  int32_t *offs = (int32_t *)malloc(sizeof(int32_t) * (size_t)(E + 1));
  int32_t *perm = (int32_t *)malloc(sizeof(int32_t) * (size_t)(T * k + 1));
  float *acc = (float *)calloc((size_t)(T * H + 1), sizeof(float));
  if (!logits || !ids || !rw || !offs || !perm || !acc) return 2;
  for (int64_t i = 0; i < T * E; ++i) logits[i] = load_f(a->logits, a->act_dtype, i);
  orc_route(logits, T, E, k, a->normalize, a->router_sigmoid, ids, rw);
  /* 2. dispatch */
  orc_dispatch(ids, T, k, E, offs, perm);
  if (a->topk_ids) memcpy(a->topk_ids, ids, sizeof(int32_t) * (size_t)(T * k));
  if (a->topk_w) memcpy(a->topk_w, rw, sizeof(float) * (size_t)(T * k));
  if (a->expert_offsets) memcpy(a->expert_offsets, offs, sizeof(int32_t) * (size_t)(E + 1));
  if (a->perm) memcpy(a->perm, perm, sizeof(int32_t) * (size_t)(T * k));

  /* 3. experts, one at a time, tokens ascending (the CPU EP's batching) */
  int64_t *rows = (int64_t *)malloc(sizeof(int64_t) * (size_t)(T * k + 1));
  for (int64_t e = 0; e < E; ++e) {
    int64_t ne = 0;
    for (int64_t r = offs[e]; r < offs[e + 1]; ++r) {
      int64_t t = perm[r] / k;
      if (a->token_mask && !a->token_mask[t]) continue;
      rows[ne++] = perm[r];
    }
    if (ne == 0) continue;
    float *X = (float *)malloc(sizeof(float) * (size_t)(ne * H));
    float *h1 = (float *)malloc(sizeof(float) * (size_t)(ne * N1));
    float *h3 = gated3 ? (float *)malloc(sizeof(float) * (size_t)(ne * I)) : NULL;
    float *A = (float *)malloc(sizeof(float) * (size_t)(ne * I));
    float *Y = (float *)malloc(sizeof(float) * (size_t)(ne * H));
    for (int64_t r = 0; r < ne; ++r)
      for (int64_t c = 0; c < H; ++c) X[r * H + c] = load_f(a->x, a->act_dtype, (rows[r] / k) * H + c);

#pragma omp parallel
    {
      float *wrow = (float *)malloc(sizeof(float) * (size_t)(H > I ? H : I));
#pragma omp for schedule(static)
      for (int64_t n = 0; n < N1; ++n) {
        weight_row(a, a->w1, a->s1, e, N1, H, n, wrow);
        float b = a->b1 ? load_f(a->b1, a->act_dtype, e * N1 + n) : 0.0f;
        for (int64_t r = 0; r < ne; ++r) h1[r * N1 + n] = dot8(X + r * H, wrow, H) + b;
      }
      if (gated3) {
#pragma omp for schedule(static)
        for (int64_t n = 0; n < I; ++n) {
          weight_row(a, a->w3, a->s3, e, I, H, n, wrow);
          float b = a->b3 ? load_f(a->b3, a->act_dtype, e * I + n) : 0.0f;
          for (int64_t r = 0; r < ne; ++r) h3[r * I + n] = dot8(X + r * H, wrow, H) + b;
        }
      }
#pragma omp for schedule(static)
      for (int64_t r = 0; r < ne; ++r)
        orc_activation(h1 + r * N1, gated3 ? h3 + r * I : NULL, I, a->activation,
                       a->swiglu_fusion, a->alpha, a->beta, a->swiglu_limit, A + r * I);
#pragma omp for schedule(static)
      for (int64_t n = 0; n < H; ++n) {
        weight_row(a, a->w2, a->s2, e, H, I, n, wrow);
        float b = a->b2 ? load_f(a->b2, a->act_dtype, e * H + n) : 0.0f;
        for (int64_t r = 0; r < ne; ++r) Y[r * H + n] = dot8(A + r * I, wrow, I) + b;
      }
      free(wrow);
    }
    /* 4. finalize contribution of this expert */
    for (int64_t r = 0; r < ne; ++r) {
      int64_t t = rows[r] / k;
      float wt = rw[rows[r]];
      for (int64_t c = 0; c < H; ++c) acc[t * H + c] += wt * Y[r * H + c];
    }
    free(X); free(h1); free(h3); free(A); free(Y);
  }
  for (int64_t t = 0; t < T; ++t) {
    if (a->token_mask && !a->token_mask[t]) continue;
    for (int64_t c = 0; c < H; ++c) {
      if (a->out) store_f(a->out, a->act_dtype, t * H + c, acc[t * H + c]);
      if (a->out_f32) a->out_f32[t * H + c] = acc[t * H + c];
    }
  }
  free(rows); free(logits); free(ids); free(rw); free(offs); free(perm); free(acc);
  return 0;
}
