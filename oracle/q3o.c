/* q3o.c - CPU restatement of the Qwen3-TTS frame step (the oracle).
 *
 * TEST INFRASTRUCTURE ONLY: what the tests compare libq3h against, never part
 * of the product path. See q3o.h for what each function restates (reference file:line) and
 * how it is pinned.
 *
 * Arithmetic conventions. The mathematics is the reference's; the order of
 * the fp32 operations is fixed explicitly (fused multiply-adds written out)
 * so that a device implementation can follow it to the bit:
 *  - dot products of the linear layers: fp32 fused multiply-adds per 32-element
 *    block in 8 partial lanes, block results accumulated in fp32 in column
 *    order;
 *  - Q8_0 weights with f32 activations: sum_b d_b * (sum_j q_j x_j);
 *  - Q8_0 weights with Q8_0 activations (ggml vec_dot_q8_0_q8_0): per block
 *    the exact int32 dot, times (dw_b * dx_b) (both scales via fp16), fused
 *    into a chain over the 16 blocks of each 512-column chunk; the chunk sums
 *    added in chunk order;
 *  - attention scores: q . k as 16 partial chains (dims 8l .. 8l + 7) joined
 *    by a balanced pairwise tree; weighted values: 8 chains over the
 *    positions p = j mod 8, joined as ((c0 + c1) + (c2 + c3)) +
 *    ((c4 + c5) + (c6 + c7));
 *  - e^x: q3o_expf (Cody-Waite reduction, Taylor series), in the softmax and
 *    in SiLU;
 *  - RMSNorm, softmax sums: double accumulation, results rounded to fp32 (the
 *    order of a double sum does not reach the fp32 result in practice);
 *  - RoPE: inv_freq_i = (float)(1 / theta^(2i/d)), angle = (float)pos *
 *    inv_freq_i in fp32, cos/sin of that angle in double rounded to fp32
 *    (the HIP library builds its table the same way on the host);
 *    a' = fma(a, c, -(b s)), b' = fma(b, c, a s).
 */
#include "q3o.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* threads                                                             */

void q3o_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int q3o_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------ */
/* IEEE half floats, round to nearest even                             */

uint16_t q3o_fp32_to_fp16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t a = x & 0x7fffffffu;
  if (a >= 0x7f800000u) /* inf, nan */
    return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0u));
  if (a >= 0x477ff000u) /* >= 65520: rounds to inf */
    return (uint16_t)(sign | 0x7c00u);
  if (a < 0x38800000u) { /* below 2^-14: half subnormal or zero */
    if (a < 0x33000000u) return (uint16_t)sign; /* below 2^-25 */
    uint32_t e = a >> 23;
    uint32_t m = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e; /* value / 2^-24 = m * 2^(e-126) */
    uint32_t r = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (r & 1u))) r++;
    return (uint16_t)(sign | r);
  }
  uint32_t r = (a - 0x38000000u) >> 13; /* rebias 127 -> 15 */
  uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
  return (uint16_t)(sign | r);
}

float q3o_fp16_to_fp32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t x;
  if (e == 0) {
    if (m == 0) {
      x = sign;
    } else { /* subnormal: m * 2^-24 */
      float v = (float)m * 5.9604644775390625e-8f;
      memcpy(&x, &v, 4);
      x |= sign;
    }
  } else if (e == 31) {
    x = sign | 0x7f800000u | (m << 13);
  } else {
    x = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

void q3o_fp32_to_fp16_row(const float *x, uint16_t *y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = q3o_fp32_to_fp16(x[i]);
}

void q3o_fp16_to_fp32_row(const uint16_t *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = q3o_fp16_to_fp32(x[i]);
}

/* ------------------------------------------------------------------ */
/* e^x in fp32 from IEEE operations only                                */

/* Cody & Waite (1980) argument reduction x = k ln2 + r, k = rint(x log2 e),
 * with ln 2 split in a 16-bit head and its tail; e^r by its Taylor series to
 * r^7 (|r| <= 0.35: truncation < 6e-9 relative), Horner form with fused
 * multiply-adds; times 2^k from the exponent bits. Each step is one
 * correctly rounded IEEE operation, so any IEEE machine gives the same bits.
 * Error < 2 ulp; 0 below -86 (no subnormal results), +inf above 88. */
float q3o_expf(float x) {
  if (x != x) return x;
  if (x < -86.0f) return 0.0f;
  if (x > 88.0f) return INFINITY;
  const float k = rintf(x * 0x1.715476p+0f);
  float r = fmaf(k, -0x1.62e4p-1f, x);
  r = fmaf(k, -0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;       /* 1/7! */
  p = fmaf(p, r, 0x1.6c16c2p-10f); /* 1/6! */
  p = fmaf(p, r, 0x1.111112p-7f);  /* 1/5! */
  p = fmaf(p, r, 0x1.555556p-5f);  /* 1/4! */
  p = fmaf(p, r, 0x1.555556p-3f);  /* 1/3! */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const uint32_t bits = (uint32_t)((int)k + 127) << 23;
  float scale;
  memcpy(&scale, &bits, 4);
  return p * scale;
}

/* ------------------------------------------------------------------ */
/* Q8_0: ggml quantize_row_q8_0_ref semantics                          */

void q3o_quantize_row_q8_0(const float *x, void *vy, int64_t k) {
  q3o_block_q8_0 *y = (q3o_block_q8_0 *)vy;
  const int64_t nb = k / 32;
  for (int64_t i = 0; i < nb; i++) {
    const float *b = x + i * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) {
      const float v = fabsf(b[j]);
      amax = amax > v ? amax : v;
    }
    const float d = amax / 127;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    y[i].d = q3o_fp32_to_fp16(d);
    for (int j = 0; j < 32; j++) y[i].qs[j] = (int8_t)roundf(b[j] * id);
  }
}

void q3o_dequantize_row_q8_0(const void *vx, float *y, int64_t k) {
  const q3o_block_q8_0 *x = (const q3o_block_q8_0 *)vx;
  const int64_t nb = k / 32;
  for (int64_t i = 0; i < nb; i++) {
    const float d = q3o_fp16_to_fp32(x[i].d);
    for (int j = 0; j < 32; j++) y[i * 32 + j] = x[i].qs[j] * d;
  }
}

void q3o_quantize_matrix_q8_0(const float *x, void *vy, int64_t rows, int64_t cols) {
  q3o_block_q8_0 *y = (q3o_block_q8_0 *)vy;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++)
    q3o_quantize_row_q8_0(x + r * cols, y + r * (cols / 32), cols);
}

/* ------------------------------------------------------------------ */
/* dot products and the linear layer                                   */

static inline float dot32(const float *w, const float *x) {
  float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int j = 0; j < 32; j += 8)
    for (int t = 0; t < 8; t++) s[t] = fmaf(w[j + t], x[j + t], s[t]);
  return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

/* q . k over one head of D = 16 * n dims: 16 partial chains (partial l over
 * dims l*n .. l*n + n - 1), then a balanced pairwise tree over l */
static inline float head_dot(const float *q, const float *k, int D) {
  const int n = D / 16;
  float t[16];
  for (int l = 0; l < 16; l++) {
    float a = 0.0f;
    for (int e = 0; e < n; e++) a = fmaf(q[l * n + e], k[l * n + e], a);
    t[l] = a;
  }
  for (int w = 8; w >= 1; w /= 2)
    for (int l = 0; l < w; l++) t[l] = t[2 * l] + t[2 * l + 1];
  return t[0];
}

static inline int32_t idot32(const int8_t *a, const int8_t *b) {
  int32_t s = 0;
  for (int j = 0; j < 32; j++) s += (int32_t)a[j] * (int32_t)b[j];
  return s;
}

/* Y[m][n] (+)= W[n] . X[m]; W [N][K] f32 or Q8_0 blocks; X [M][K]; the
 * quantized activations (act_q8) also to xq_out [M][K / 32] when non-null */
static void linear_q(const void *W, int dtype, int act_q8, int N, int K,
                     const float *X, int M, float *Y, int ldy, int add, void *xq_out) {
  const int nb = K / 32;
  q3o_block_q8_0 *xq = NULL;
  if (dtype == Q3O_Q8_0 && act_q8) {
    xq = (q3o_block_q8_0 *)malloc(sizeof(q3o_block_q8_0) * (size_t)nb * M);
    for (int m = 0; m < M; m++) q3o_quantize_row_q8_0(X + (size_t)m * K, xq + (size_t)m * nb, K);
    if (xq_out) memcpy(xq_out, xq, sizeof(q3o_block_q8_0) * (size_t)nb * M);
  }
#pragma omp parallel
  {
    float *wrow = (float *)malloc(sizeof(float) * K);
    float *scale = (float *)malloc(sizeof(float) * nb);
#pragma omp for schedule(static)
    for (int n = 0; n < N; n++) {
      if (dtype == Q3O_F32) {
        const float *w = (const float *)W + (size_t)n * K;
        for (int m = 0; m < M; m++) {
          const float *x = X + (size_t)m * K;
          float acc = 0.0f;
          for (int b = 0; b < nb; b++) acc += dot32(w + b * 32, x + b * 32);
          if (add)
            Y[(size_t)m * ldy + n] += acc;
          else
            Y[(size_t)m * ldy + n] = acc;
        }
      } else {
        const q3o_block_q8_0 *w = (const q3o_block_q8_0 *)W + (size_t)n * nb;
        if (!act_q8) {
          for (int b = 0; b < nb; b++) {
            scale[b] = q3o_fp16_to_fp32(w[b].d);
            for (int j = 0; j < 32; j++) wrow[b * 32 + j] = (float)w[b].qs[j];
          }
        }
        for (int m = 0; m < M; m++) {
          float acc = 0.0f;
          if (act_q8) {
            const q3o_block_q8_0 *x = xq + (size_t)m * nb;
            for (int b0 = 0; b0 < nb; b0 += 16) {
              float part = 0.0f;
              for (int b = b0; b < b0 + 16 && b < nb; b++) {
                const int32_t s = idot32(w[b].qs, x[b].qs);
                part = fmaf((float)s, q3o_fp16_to_fp32(w[b].d) * q3o_fp16_to_fp32(x[b].d),
                            part);
              }
              acc += part;
            }
          } else {
            const float *x = X + (size_t)m * K;
            for (int b = 0; b < nb; b++) acc += scale[b] * dot32(wrow + b * 32, x + b * 32);
          }
          if (add)
            Y[(size_t)m * ldy + n] += acc;
          else
            Y[(size_t)m * ldy + n] = acc;
        }
      }
    }
    free(wrow);
    free(scale);
  }
  free(xq);
}

static void linear(const void *W, int dtype, int act_q8, int N, int K,
                   const float *X, int M, float *Y, int ldy, int add) {
  linear_q(W, dtype, act_q8, N, K, X, M, Y, ldy, add, NULL);
}

/* ------------------------------------------------------------------ */
/* norms, RoPE                                                         */

static void rmsnorm(const float *x, const float *w, int n, float eps, float *y) {
  double ss = 0.0;
  for (int i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
  const float inv = (float)(1.0 / sqrt(ss / n + (double)eps));
  for (int i = 0; i < n; i++) y[i] = w[i] * (x[i] * inv);
}

void q3o_rmsnorm_rows(const float *x, int rows, int n, const float *w, float eps, float *y) {
  for (int r = 0; r < rows; r++) rmsnorm(x + (size_t)r * n, w, n, eps, y + (size_t)r * n);
}

static void rope(float *x, int d, int pos, float theta) {
  const int half = d / 2;
  for (int i = 0; i < half; i++) {
    const float inv_freq = (float)(1.0 / pow((double)theta, (double)(2 * i) / (double)d));
    const float angle = (float)pos * inv_freq;
    const float c = (float)cos((double)angle);
    const float s = (float)sin((double)angle);
    const float a = x[i], b = x[i + half];
    x[i] = fmaf(a, c, -(b * s));
    x[i + half] = fmaf(b, c, a * s);
  }
}

/* ------------------------------------------------------------------ */
/* stack and context                                                   */

struct q3o_stack {
  q3o_config cfg;
  q3o_layer *layers;
  const float *final_norm;
};

struct q3o_ctx {
  q3o_stack *s;
  int len, max_pos;
  float *k, *v; /* [layers][kv_heads][max_pos][head_dim] */
};

q3o_stack *q3o_stack_create(const q3o_config *cfg, const q3o_layer *layers,
                            const float *final_norm) {
  if (cfg->hidden % 32 || cfg->intermediate % 32 || (cfg->heads * cfg->head_dim) % 32 ||
      cfg->heads % cfg->kv_heads || cfg->head_dim % 16)
    return NULL;
  q3o_stack *s = (q3o_stack *)calloc(1, sizeof(*s));
  s->cfg = *cfg;
  s->layers = (q3o_layer *)malloc(sizeof(q3o_layer) * cfg->layers);
  memcpy(s->layers, layers, sizeof(q3o_layer) * cfg->layers);
  s->final_norm = final_norm;
  return s;
}

void q3o_stack_destroy(q3o_stack *s) {
  if (!s) return;
  free(s->layers);
  free(s);
}

q3o_ctx *q3o_ctx_create(q3o_stack *s, int max_positions) {
  q3o_ctx *c = (q3o_ctx *)calloc(1, sizeof(*c));
  c->s = s;
  c->max_pos = max_positions;
  size_t n = (size_t)s->cfg.layers * s->cfg.kv_heads * max_positions * s->cfg.head_dim;
  c->k = (float *)calloc(n, sizeof(float));
  c->v = (float *)calloc(n, sizeof(float));
  return c;
}

void q3o_ctx_destroy(q3o_ctx *c) {
  if (!c) return;
  free(c->k);
  free(c->v);
  free(c);
}

void q3o_ctx_reset(q3o_ctx *c) { c->len = 0; }

int q3o_ctx_length(const q3o_ctx *c) { return c->len; }

static size_t kv_off(const q3o_ctx *c, int layer, int g, int pos) {
  const q3o_config *q = &c->s->cfg;
  return (((size_t)layer * q->kv_heads + g) * c->max_pos + pos) * q->head_dim;
}

const float *q3o_ctx_k(const q3o_ctx *c, int layer) { return c->k + kv_off(c, layer, 0, 0); }
const float *q3o_ctx_v(const q3o_ctx *c, int layer) { return c->v + kv_off(c, layer, 0, 0); }

static inline float kv_round(const q3o_config *q, float v) {
  return q->kv_f16 ? q3o_fp16_to_fp32(q3o_fp32_to_fp16(v)) : v;
}

int q3o_ctx_fill(q3o_ctx *c, const float *k, const float *v, int len) {
  const q3o_config *q = &c->s->cfg;
  if (len > c->max_pos || len < 0) return -1;
  for (int l = 0; l < q->layers; l++)
    for (int g = 0; g < q->kv_heads; g++)
      for (int p = 0; p < len; p++)
        for (int d = 0; d < q->head_dim; d++) {
          size_t src = (((size_t)l * q->kv_heads + g) * len + p) * q->head_dim + d;
          c->k[kv_off(c, l, g, p) + d] = kv_round(q, k[src]);
          c->v[kv_off(c, l, g, p) + d] = kv_round(q, v[src]);
        }
  c->len = len;
  return 0;
}

int q3o_forward_embeds(q3o_ctx *c, const float *x, int rows, float *normed_last,
                       float *layer_out) {
  return q3o_forward_embeds_traced(c, x, rows, normed_last, layer_out, NULL);
}

/* the trace slot of layer l for a tensor of n values (or blocks) per row */
#define TRACE_F(ptr, l, n) ((ptr) ? (ptr) + ((size_t)(l) * rows) * (size_t)(n) : NULL)
#define TRACE_B(ptr, l, n) \
  ((ptr) ? (void *)((q3o_block_q8_0 *)(ptr) + ((size_t)(l) * rows) * (size_t)(n)) : NULL)

static void trace_copy(float *dst, const float *src, size_t n) {
  if (dst) memcpy(dst, src, sizeof(float) * n);
}

int q3o_forward_embeds_traced(q3o_ctx *c, const float *x, int rows, float *normed_last,
                              float *layer_out, const q3o_trace *t) {
  const q3o_config *q = &c->s->cfg;
  const q3o_trace none = {0};
  if (!t) t = &none;
  if (rows <= 0) return 0;
  if (c->len + rows > c->max_pos) return -1;
  const int H = q->hidden, D = q->head_dim, NQ = q->heads * D, NKV = q->kv_heads * D;
  const int I = q->intermediate, grp = q->heads / q->kv_heads;
  const float scale = (float)(1.0 / sqrt((double)D));
  float *h = (float *)malloc(sizeof(float) * rows * H);
  float *xn = (float *)malloc(sizeof(float) * rows * H);
  float *qb = (float *)malloc(sizeof(float) * rows * NQ);
  float *kb = (float *)malloc(sizeof(float) * rows * NKV);
  float *vb = (float *)malloc(sizeof(float) * rows * NKV);
  float *att = (float *)malloc(sizeof(float) * rows * NQ);
  float *gb = (float *)malloc(sizeof(float) * rows * I);
  float *ub = (float *)malloc(sizeof(float) * rows * I);
  float *pb = (float *)malloc(sizeof(float) * rows * H);
  const int NQKV = NQ + 2 * NKV;
  memcpy(h, x, sizeof(float) * rows * H);
  for (int l = 0; l < q->layers; l++) {
    const q3o_layer *L = &c->s->layers[l];
    for (int r = 0; r < rows; r++) rmsnorm(h + r * H, L->input_norm, H, q->rms_eps, xn + r * H);
    trace_copy(TRACE_F(t->x_qkv, l, H), xn, (size_t)rows * H);
    linear_q(L->wq, q->dtype, q->act_q8, NQ, H, xn, rows, qb, NQ, 0, TRACE_B(t->b_qkv, l, H / 32));
    linear(L->wk, q->dtype, q->act_q8, NKV, H, xn, rows, kb, NKV, 0);
    linear(L->wv, q->dtype, q->act_q8, NKV, H, xn, rows, vb, NKV, 0);
    if (t->y_qkv)
      for (int r = 0; r < rows; r++) {
        float *y = TRACE_F(t->y_qkv, l, NQKV) + (size_t)r * NQKV;
        memcpy(y, qb + r * NQ, sizeof(float) * NQ);
        memcpy(y + NQ, kb + r * NKV, sizeof(float) * NKV);
        memcpy(y + NQ + NKV, vb + r * NKV, sizeof(float) * NKV);
      }
    for (int r = 0; r < rows; r++) {
      const int pos = c->len + r;
      for (int hh = 0; hh < q->heads; hh++) {
        float *qh = qb + r * NQ + hh * D;
        rmsnorm(qh, L->q_norm, D, q->rms_eps, qh);
        rope(qh, D, pos, q->rope_theta);
      }
      for (int g = 0; g < q->kv_heads; g++) {
        float *kh = kb + r * NKV + g * D;
        const float *vh = vb + r * NKV + g * D;
        rmsnorm(kh, L->k_norm, D, q->rms_eps, kh);
        rope(kh, D, pos, q->rope_theta);
        float *kc = c->k + kv_off(c, l, g, pos), *vc = c->v + kv_off(c, l, g, pos);
        for (int d = 0; d < D; d++) {
          kc[d] = kv_round(q, kh[d]);
          vc[d] = kv_round(q, vh[d]);
        }
      }
    }
#pragma omp parallel for collapse(2) schedule(static)
    for (int r = 0; r < rows; r++) {
      for (int hh = 0; hh < q->heads; hh++) {
        const int n = c->len + r + 1, g = hh / grp;
        const float *qh = qb + r * NQ + hh * D;
        float *sc = (float *)malloc(sizeof(float) * n);
        float mx = -INFINITY;
        for (int p = 0; p < n; p++) {
          sc[p] = head_dot(qh, c->k + kv_off(c, l, g, p), D) * scale;
          mx = sc[p] > mx ? sc[p] : mx;
        }
        double sum = 0.0;
        for (int p = 0; p < n; p++) {
          sc[p] = q3o_expf(sc[p] - mx);
          sum += sc[p];
        }
        const float inv = (float)(1.0 / sum);
        float *o = att + r * NQ + hh * D;
        /* 8 chains over the positions p mod 8, joined as a balanced tree */
        float *ch = (float *)calloc((size_t)8 * D, sizeof(float));
        for (int p = 0; p < n; p++) {
          const float *vc = c->v + kv_off(c, l, g, p);
          const float w = sc[p] * inv;
          float *cj = ch + (size_t)(p & 7) * D;
          for (int d = 0; d < D; d++) cj[d] = fmaf(w, vc[d], cj[d]);
        }
        for (int d = 0; d < D; d++)
          o[d] = ((ch[d] + ch[D + d]) + (ch[2 * D + d] + ch[3 * D + d])) +
                 ((ch[4 * D + d] + ch[5 * D + d]) + (ch[6 * D + d] + ch[7 * D + d]));
        free(ch);
        free(sc);
      }
    }
    /* o_proj, then the residual: h + (W_o . att), one rounding of the sum */
    trace_copy(TRACE_F(t->x_o, l, NQ), att, (size_t)rows * NQ);
    linear_q(L->wo, q->dtype, q->act_q8, H, NQ, att, rows, pb, H, 0, TRACE_B(t->b_o, l, NQ / 32));
    trace_copy(TRACE_F(t->y_o, l, H), pb, (size_t)rows * H);
    for (int i = 0; i < rows * H; i++) h[i] += pb[i];
    for (int r = 0; r < rows; r++) rmsnorm(h + r * H, L->post_norm, H, q->rms_eps, xn + r * H);
    trace_copy(TRACE_F(t->x_gu, l, H), xn, (size_t)rows * H);
    linear_q(L->wgate, q->dtype, q->act_q8, I, H, xn, rows, gb, I, 0, TRACE_B(t->b_gu, l, H / 32));
    linear(L->wup, q->dtype, q->act_q8, I, H, xn, rows, ub, I, 0);
    trace_copy(TRACE_F(t->y_gate, l, I), gb, (size_t)rows * I);
    trace_copy(TRACE_F(t->y_up, l, I), ub, (size_t)rows * I);
    for (int i = 0; i < rows * I; i++) {
      const float g = gb[i];
      gb[i] = g / (1.0f + q3o_expf(-g)) * ub[i];
    }
    trace_copy(TRACE_F(t->x_down, l, I), gb, (size_t)rows * I);
    linear_q(L->wdown, q->dtype, q->act_q8, H, I, gb, rows, pb, H, 0,
             TRACE_B(t->b_down, l, I / 32));
    trace_copy(TRACE_F(t->y_down, l, H), pb, (size_t)rows * H);
    for (int i = 0; i < rows * H; i++) h[i] += pb[i];
    if (layer_out) memcpy(layer_out + (size_t)l * rows * H, h, sizeof(float) * rows * H);
  }
  if (normed_last) rmsnorm(h + (size_t)(rows - 1) * H, c->s->final_norm, H, q->rms_eps, normed_last);
  c->len += rows;
  free(h);
  free(xn);
  free(qb);
  free(kb);
  free(vb);
  free(att);
  free(gb);
  free(ub);
  free(pb);
  return 0;
}

void q3o_head(const void *w, int dtype, int act_q8, int rows_out, int hidden,
              const float *state, float *logits) {
  linear(w, dtype, act_q8, rows_out, hidden, state, 1, logits, rows_out, 0);
}

/* ------------------------------------------------------------------ */
/* text projection                                                     */

/* InferRowToF32 of one text-embedding row: f32 as is, BF16 = the high half
 * of an f32 (exact) */
static void text_row(const void *emb, int emb_dtype, int id, int cols, float *out) {
  if (emb_dtype == Q3O_BF16) {
    const uint16_t *r = (const uint16_t *)emb + (size_t)id * cols;
    for (int c = 0; c < cols; c++) {
      const uint32_t u = (uint32_t)r[c] << 16;
      memcpy(out + c, &u, 4);
    }
  } else {
    memcpy(out, (const float *)emb + (size_t)id * cols, sizeof(float) * cols);
  }
}

/* TQwenTalker.TextProject (talker.pas:390-421): e = embedding rows of ids,
 * h = fc1 . e + b1, SiLU(h) (0 below -80, else v / (1 + Exp(-v)) with the
 * exponential and the quotient in double, as Pascal's Exp on x86-64 returns
 * a double), y = fc2 . h + b2. Each bias is the start of its row's sum. */
int q3o_text_project(const void *emb, int emb_dtype, int vocab, int text_hidden, int hidden,
                     const float *fc1_w, const float *fc1_b, const float *fc2_w,
                     const float *fc2_b, const int32_t *ids, int n, float *y) {
  if (n <= 0) return 0;
  for (int r = 0; r < n; r++)
    if (ids[r] < 0 || ids[r] >= vocab) return -1;
  const int TH = text_hidden;
  float *e = (float *)malloc(sizeof(float) * (size_t)n * TH);
  float *h = (float *)malloc(sizeof(float) * (size_t)n * TH);
  for (int r = 0; r < n; r++) {
    text_row(emb, emb_dtype, ids[r], TH, e + (size_t)r * TH);
    memcpy(h + (size_t)r * TH, fc1_b, sizeof(float) * TH);
    memcpy(y + (size_t)r * hidden, fc2_b, sizeof(float) * hidden);
  }
  linear(fc1_w, Q3O_F32, 0, TH, TH, e, n, h, TH, 1);
  for (size_t i = 0; i < (size_t)n * TH; i++) {
    const float v = h[i];
    h[i] = v < -80.0f ? 0.0f : (float)((double)v / (1.0 + exp(-(double)v)));
  }
  linear(fc2_w, Q3O_F32, 0, hidden, TH, h, n, y, hidden, 1);
  free(e);
  free(h);
  return 0;
}

/* ------------------------------------------------------------------ */
/* code choice (greedy)                                                */

/* tests/test.tts.qwen.lm.pas:109-117: result 0, moved to i only when p[i] >
 * p[result]; so a NaN never wins and a NaN p[0] keeps 0 */
int q3o_argmax(const float *p, int n) {
  int r = 0;
  for (int i = 1; i < n; i++)
    if (p[i] > p[r]) r = i;
  return r;
}

static void code0_scores(const float *logits, int vocab, int eos, const int *history,
                         int nhistory, float penalty, float *work);

int q3o_choose_code0(const float *logits, int vocab, int eos, const int *history,
                     int nhistory, float penalty) {
  float *work = (float *)malloc(sizeof(float) * vocab);
  code0_scores(logits, vocab, eos, history, nhistory, penalty, work);
  const int r = q3o_argmax(work, vocab);
  free(work);
  return r;
}

/* ------------------------------------------------------------------ */
/* sampling                                                            */

/* Philox4x64-10 (Salmon, Moraes, Dror, Shaw, SC 2011): 10 rounds of the
 * two 64 x 64 -> 128-bit products, the key bumped by the Weyl constants */
void q3o_philox4x64(const uint64_t ctr[4], const uint64_t key[2], uint64_t out[4]) {
  uint64_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; r++) {
    const unsigned __int128 p0 = (unsigned __int128)0xD2E7470EE14C6C93ull * c0;
    const unsigned __int128 p1 = (unsigned __int128)0xCA5A826395121157ull * c2;
    const uint64_t hi0 = (uint64_t)(p0 >> 64), lo0 = (uint64_t)p0;
    const uint64_t hi1 = (uint64_t)(p1 >> 64), lo1 = (uint64_t)p1;
    c0 = hi1 ^ c1 ^ k0;
    c1 = lo1;
    c2 = hi0 ^ c3 ^ k1;
    c3 = lo0;
    k0 += 0x9E3779B97F4A7C15ull;
    k1 += 0xBB67AE8584CAA73Bull;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

float q3o_draw_uniform(uint64_t seed, uint64_t frame, uint64_t group) {
  const uint64_t ctr[4] = {frame, group, 0, 0}, key[2] = {seed, 0};
  uint64_t out[4];
  q3o_philox4x64(ctr, key, out);
  return (float)(uint32_t)(out[0] >> 40) * 0x1p-24f;
}

static uint32_t order_key(float v) {
  uint32_t b;
  memcpy(&b, &v, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

typedef struct {
  uint32_t key;
  int idx;
  float v;
} cand_t;

/* descending key, then ascending index */
static int cand_cmp(const void *a, const void *b) {
  const cand_t *x = (const cand_t *)a, *y = (const cand_t *)b;
  if (x->key != y->key) return x->key > y->key ? -1 : 1;
  return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

static int u32_desc(const void *a, const void *b) {
  const uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
  return x > y ? -1 : (x < y);
}

static int last_positive(const float *W, int lo, int hi) {
  int best = -1;
  for (int i = lo; i < hi; i++)
    if (W[i] > 0.0f) best = i;
  return best;
}

/* The draw of the library's sampler (temperature, top-k, top-p, one uniform
 * through the inverse distribution), with its fixed evaluation order: the
 * values in 1024 threads of NPT = ceil(n / 1024) consecutive indices, sums by
 * thread, by 64 segments of 16 threads, then over the segments; top-p over
 * at most 64 values kept by a top-k of at most 64. */
int q3o_sample(const float *x, int n, float temperature, int top_k, float top_p, float u) {
  if (n <= 0 || n > 3 * 1024) return -1;
  const int NPT = (n + 1023) / 1024, N = 1024 * NPT;
  float *v = (float *)malloc(sizeof(float) * N);
  float *W = (float *)malloc(sizeof(float) * N);
  uint32_t *key = (uint32_t *)malloc(sizeof(uint32_t) * N);
  uint8_t *kept = (uint8_t *)malloc(N);
  for (int i = 0; i < N; i++) {
    const int in = i < n;
    const float a = in ? x[i] : -INFINITY;
    v[i] = temperature == 1.0f ? a : a / temperature;
    key[i] = order_key(v[i]);
    kept[i] = (uint8_t)in;
  }
  const int topk = top_k >= 1 && top_k < n;
  if (topk) {
    uint32_t *ks = (uint32_t *)malloc(sizeof(uint32_t) * n);
    memcpy(ks, key, sizeof(uint32_t) * n);
    qsort(ks, n, sizeof(uint32_t), u32_desc);
    const uint32_t tau = ks[top_k - 1];
    free(ks);
    for (int i = 0; i < n; i++) kept[i] = kept[i] && key[i] >= tau;
  }
  float M = -INFINITY;
  for (int i = 0; i < n; i++)
    if (kept[i] && v[i] > M) M = v[i];
  if (top_p < 1.0f && topk && top_k <= 64) {
    cand_t c[64];
    int cnt = 0;
    for (int i = 0; i < n; i++)
      if (kept[i]) {
        if (cnt < 64) {
          c[cnt].key = key[i];
          c[cnt].idx = i;
          c[cnt].v = v[i];
        }
        cnt++;
      }
    if (cnt <= 64) {
      qsort(c, cnt, sizeof(cand_t), cand_cmp);
      float w[64], S = 0.0f;
      for (int q = 0; q < cnt; q++) w[q] = q3o_expf(c[q].v - M);
      for (int q = cnt - 1; q >= 0; q--) S = S + w[q];
      const float lim = 1.0f - top_p;
      float cum = 0.0f;
      int last = 0;
      for (int q = cnt - 1; q >= 1; q--) {
        cum = cum + w[q] / S;
        if (cum > lim) {
          last = q;
          break;
        }
      }
      const uint32_t tk = c[last].key;
      const int ti = c[last].idx;
      for (int i = 0; i < n; i++)
        kept[i] = kept[i] && (key[i] > tk || (key[i] == tk && i <= ti));
    }
  }
  float A[1024], B[64];
  for (int i = 0; i < N; i++) W[i] = kept[i] ? q3o_expf(v[i] - M) : 0.0f;
  for (int t = 0; t < 1024; t++) {
    float a = 0.0f;
    for (int j = 0; j < NPT; j++) a = a + W[t * NPT + j];
    A[t] = a;
  }
  for (int s = 0; s < 64; s++) {
    float b = 0.0f;
    for (int q = 0; q < 16; q++) b = b + A[16 * s + q];
    B[s] = b;
  }
  float S = 0.0f;
  for (int s = 0; s < 64; s++) S = S + B[s];
  const float target = u * S;
  float r = 0.0f;
  int seg = -1, pick = -1;
  for (int s = 0; s < 64; s++) {
    if (r + B[s] > target) {
      seg = s;
      break;
    }
    r = r + B[s];
  }
  if (seg < 0) {
    pick = last_positive(W, 0, N);
  } else {
    int th = -1;
    for (int q = 0; q < 16; q++) {
      const float aq = A[16 * seg + q];
      if (r + aq > target) {
        th = 16 * seg + q;
        break;
      }
      r = r + aq;
    }
    if (th < 0) {
      pick = last_positive(W, 16 * seg * NPT, 16 * (seg + 1) * NPT);
    } else {
      for (int j = 0; j < NPT; j++) {
        const float wj = W[th * NPT + j];
        if (r + wj > target) {
          pick = th * NPT + j;
          break;
        }
        r = r + wj;
      }
      if (pick < 0) pick = last_positive(W, th * NPT, th * NPT + NPT);
    }
  }
  free(v);
  free(W);
  free(key);
  free(kept);
  /* no code drawn (every weight 0 or NaN: NaN or infinite scores): the greedy
   * code of x, so the result is always an index of the table */
  if (pick < 0) pick = q3o_argmax(x, n);
  return pick;
}

/* the scores ChooseCode0 hands to the argmax or the sampler (talker.pas:
 * 603-626) */
static void code0_scores(const float *logits, int vocab, int eos, const int *history,
                         int nhistory, float penalty, float *work) {
  memcpy(work, logits, sizeof(float) * vocab);
  for (int i = vocab - 1024; i < vocab; i++)
    if (i != eos) work[i] = -INFINITY;
  if (nhistory < 2 && eos >= 0 && eos < vocab) work[eos] = -INFINITY;
  if (penalty != 1.0f)
    for (int j = 0; j < nhistory; j++) {
      const int i = history[j];
      const float s = logits[i];
      if (work[i] != s) continue; /* already penalized (or forbidden) */
      work[i] = s > 0 ? s / penalty : s * penalty;
    }
}

/* ------------------------------------------------------------------ */
/* frame step                                                          */

struct q3o_frame {
  q3o_stack *talker, *cp;
  q3o_frame_tables t;
  q3o_ctx *tctx, *cctx;
  float *logits, *past, *x, *plogits, *trailing, *work;
  int *history;
  int nhist, cap_hist, trailing_rows, step;
  q3o_sampling sampling;
};

void q3o_frame_set_sampling(q3o_frame *f, const q3o_sampling *s) { f->sampling = *s; }

q3o_frame *q3o_frame_create(q3o_stack *talker, q3o_stack *cp,
                            const q3o_frame_tables *t, int max_positions) {
  q3o_frame *f = (q3o_frame *)calloc(1, sizeof(*f));
  const int H = talker->cfg.hidden;
  f->talker = talker;
  f->cp = cp;
  f->t = *t;
  f->tctx = q3o_ctx_create(talker, max_positions);
  f->cctx = q3o_ctx_create(cp, t->groups);
  f->logits = (float *)calloc(t->vocab, sizeof(float));
  f->plogits = (float *)calloc(t->cp_vocab, sizeof(float));
  f->work = (float *)calloc(t->vocab, sizeof(float));
  f->past = (float *)calloc(H, sizeof(float));
  f->x = (float *)calloc(2 * H, sizeof(float));
  f->cap_hist = 64;
  f->history = (int *)malloc(sizeof(int) * f->cap_hist);
  return f;
}

void q3o_frame_destroy(q3o_frame *f) {
  if (!f) return;
  q3o_ctx_destroy(f->tctx);
  q3o_ctx_destroy(f->cctx);
  free(f->logits);
  free(f->plogits);
  free(f->work);
  free(f->past);
  free(f->x);
  free(f->history);
  free(f->trailing);
  free(f);
}

int q3o_frame_start(q3o_frame *f, const float *prefill, int rows,
                    const float *trailing, int trailing_rows) {
  const int H = f->talker->cfg.hidden;
  free(f->trailing);
  f->trailing = NULL;
  f->trailing_rows = trailing_rows > 0 ? trailing_rows : 0;
  if (f->trailing_rows) {
    f->trailing = (float *)malloc(sizeof(float) * f->trailing_rows * H);
    memcpy(f->trailing, trailing, sizeof(float) * f->trailing_rows * H);
  }
  q3o_ctx_reset(f->tctx);
  if (q3o_forward_embeds(f->tctx, prefill, rows, f->past, NULL)) return -1;
  q3o_head(f->t.talker_head, f->talker->cfg.dtype, f->talker->cfg.act_q8, f->t.vocab, H,
           f->past, f->logits);
  f->nhist = 0;
  f->step = 0;
  return 0;
}

static void add_row(const float *emb, int id, int H, float *y) {
  for (int c = 0; c < H; c++) y[c] = y[c] + emb[(size_t)id * H + c];
}

int q3o_frame_next(q3o_frame *f, int *codes) {
  const int H = f->talker->cfg.hidden;
  const q3o_frame_tables *t = &f->t;
  const q3o_sampling *sp = &f->sampling;
  const uint64_t frame = (uint64_t)f->nhist;
  code0_scores(f->logits, t->vocab, t->eos, f->history, f->nhist, t->penalty, f->work);
  const int code =
      sp->do_sample
          ? q3o_sample(f->work, t->vocab, sp->temperature, sp->top_k, sp->top_p,
                       q3o_draw_uniform(sp->seed, frame, 0))
          : q3o_argmax(f->work, t->vocab);
  if (code == t->eos) return 0;
  codes[0] = code;
  if (f->nhist == f->cap_hist) {
    f->cap_hist *= 2;
    f->history = (int *)realloc(f->history, sizeof(int) * f->cap_hist);
  }
  f->history[f->nhist++] = code;
  /* the code predictor: [talker state, embedding of code 0], then each code */
  memcpy(f->x, f->past, sizeof(float) * H);
  memcpy(f->x + H, t->codec_emb + (size_t)code * H, sizeof(float) * H);
  q3o_ctx_reset(f->cctx);
  float *normed = (float *)malloc(sizeof(float) * H);
  const int cdt = f->cp->cfg.dtype, caq = f->cp->cfg.act_q8;
  for (int g = 0; g < t->groups - 1; g++) {
    if (g == 0) {
      q3o_forward_embeds(f->cctx, f->x, 2, normed, NULL);
    } else {
      memcpy(f->x, t->pred_emb[g - 1] + (size_t)codes[g] * H, sizeof(float) * H);
      q3o_forward_embeds(f->cctx, f->x, 1, normed, NULL);
    }
    q3o_head(t->cp_heads[g], cdt, caq, t->cp_vocab, H, normed, f->plogits);
    codes[g + 1] =
        sp->sub_do_sample
            ? q3o_sample(f->plogits, t->cp_vocab, sp->sub_temperature, sp->sub_top_k,
                         sp->sub_top_p, q3o_draw_uniform(sp->seed ^ 0x5DEECE66Dull, frame, g + 1))
            : q3o_argmax(f->plogits, t->cp_vocab);
  }
  free(normed);
  /* the next talker input: the 16 embeddings, plus the text (or tts_pad) */
  memcpy(f->x, t->codec_emb + (size_t)code * H, sizeof(float) * H);
  for (int g = 1; g < t->groups; g++) add_row(t->pred_emb[g - 1], codes[g], H, f->x);
  if (f->step < f->trailing_rows)
    add_row(f->trailing, f->step, H, f->x);
  else
    add_row(t->tts_pad, 0, H, f->x);
  if (q3o_forward_embeds(f->tctx, f->x, 1, f->past, NULL)) return -1;
  q3o_head(t->talker_head, f->talker->cfg.dtype, f->talker->cfg.act_q8, t->vocab, H, f->past,
           f->logits);
  f->step++;
  return 1;
}

const float *q3o_frame_logits(const q3o_frame *f) { return f->logits; }
const float *q3o_frame_past_hidden(const q3o_frame *f) { return f->past; }
q3o_ctx *q3o_frame_talker_ctx(q3o_frame *f) { return f->tctx; }
