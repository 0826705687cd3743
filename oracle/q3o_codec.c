/* q3o_codec.c - CPU restatement of the back part of the Qwen3-TTS 12 Hz
 * decoder (the oracle of the HIP codec).
 *
 * TEST INFRASTRUCTURE ONLY (see q3o.h).
 *
 * What it restates (reference files, relative to the reference checkout):
 *  - TQwenCodec.Back (src/tts/mormot.ai.tts.qwen.codec.pas:1040-1083): two
 *    upsampling stages (transposed convolution, kernel 2 stride 2, then a
 *    ConvNeXt block), the input convolution (1024 -> 1536, kernel 7), four
 *    decoder blocks (SnakeBeta, transposed convolution of kernel 2 rate and
 *    stride rate, rates 8 / 5 / 4 / 3, then three residual units of
 *    dilations 1 / 3 / 9), SnakeBeta, the output convolution (96 -> 1,
 *    kernel 7) and the clamp to [-1, 1];
 *  - TQwenConv (codec.pas:296-357): causal convolution over [history ;
 *    input], history = the last (K - 1) dil input rows of the previous call
 *    (zeros after Reset);
 *  - TQwenTransConv (codec.pas:360-425): y[t stride + j] = b + sum over taps
 *    i < K / stride and channels c of w[c][o][j + i stride] x[t - i], the
 *    previous taps - 1 input rows kept;
 *  - TQwenSnake (codec.pas:429-478): x + 1 / (e^beta + 1e-9) sin(e^alpha x)^2,
 *    e^alpha and the reciprocal in float32 as PyTorch computes them;
 *  - TQwenConvNeXt (codec.pas:481-536): causal depthwise convolution of
 *    kernel 7, LayerNorm (eps 1e-6), pointwise 1024 -> 4096, GELU (erf),
 *    pointwise 4096 -> 1024, y = x + gamma * that;
 *  - TQwenResUnit (codec.pas:539-600): x + conv2(snake2(conv1(snake1(x)))).
 * Sums in double, rounded to float once per output.
 *
 * How it is pinned (tests/test_oracle_codec.py): the whole back part against
 * a float64 PyTorch composition of the same modules over the full sequence
 * (torch conv1d with causal left padding, conv_transpose1d truncated to
 * T stride samples, layer_norm, gelu, the SnakeBeta formula), decoded here
 * in chunks of 1, 2 and 3 frames (the history carried across calls).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "q3o.h"

#define LATENT 1024
#define DEC_DIM 1536
#define FRAME_SAMPLES 1920

static const int RATES[4] = {8, 5, 4, 3};
static const int DILS[3] = {1, 3, 9};

typedef struct {
  const float *w, *b; /* w [out][in][k] */
  int in, out, k, dil, past;
  float *hist; /* [past][in] */
} conv_t;

typedef struct {
  const float *w, *b; /* w [in][out][k] */
  int in, out, k, stride, taps;
  float *hist; /* [taps - 1][in] */
} tconv_t;

typedef struct {
  float *a, *ib; /* e^alpha, 1 / (e^beta + 1e-9) */
  int n;
} snake_t;

typedef struct {
  const float *dw_w, *dw_b, *nw, *nb, *pw1_w, *pw1_b, *pw2_w, *pw2_b, *gamma;
  float *hist; /* [6][1024] */
} next_t;

typedef struct {
  snake_t a1, a2;
  conv_t c1, c2;
} res_t;

typedef struct {
  snake_t act;
  tconv_t up;
  res_t res[3];
  int in, out, rate;
} block_t;

struct q3o_codec {
  tconv_t up[2];
  next_t next[2];
  conv_t conv0;
  block_t blocks[4];
  snake_t act_out;
  conv_t conv_out;
};

static void conv_init(conv_t *c, const float *w, const float *b, int in, int out, int k, int dil) {
  c->w = w;
  c->b = b;
  c->in = in;
  c->out = out;
  c->k = k;
  c->dil = dil;
  c->past = (k - 1) * dil;
  c->hist = (float *)calloc((size_t)(c->past ? c->past : 1) * in, sizeof(float));
}

static void snake_init(snake_t *s, const float *alpha, const float *beta, int n) {
  s->n = n;
  s->a = (float *)malloc(sizeof(float) * n);
  s->ib = (float *)malloc(sizeof(float) * n);
  for (int c = 0; c < n; c++) {
    s->a[c] = expf(alpha[c]);
    s->ib[c] = 1.0f / (expf(beta[c]) + 1e-9f);
  }
}

static void snake_apply(const snake_t *s, float *x, int rows) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < rows; t++)
    for (int c = 0; c < s->n; c++) {
      float *p = x + (size_t)t * s->n + c;
      const float v = *p * s->a[c];
      const float sn = (float)sin((double)v);
      *p = *p + s->ib[c] * (sn * sn);
    }
}

/* y [rows][out] = conv over [hist ; x] */
static void conv_forward(conv_t *c, const float *x, int rows, float *y) {
  const int in = c->in, past = c->past;
  float *buf = (float *)malloc(sizeof(float) * (size_t)(past + rows) * in);
  memcpy(buf, c->hist, sizeof(float) * (size_t)past * in);
  memcpy(buf + (size_t)past * in, x, sizeof(float) * (size_t)rows * in);
#pragma omp parallel for schedule(static)
  for (int t = 0; t < rows; t++)
    for (int o = 0; o < c->out; o++) {
      const float *w = c->w + (size_t)o * in * c->k;
      double acc = 0.0;
      for (int ch = 0; ch < in; ch++)
        for (int k = 0; k < c->k; k++)
          acc += (double)w[ch * c->k + k] * buf[(size_t)(t + k * c->dil) * in + ch];
      y[(size_t)t * c->out + o] = (float)(acc + c->b[o]);
    }
  memcpy(c->hist, buf + (size_t)rows * in, sizeof(float) * (size_t)past * in);
  free(buf);
}

/* y [rows * stride][out] */
static void tconv_forward(tconv_t *c, const float *x, int rows, float *y) {
  const int in = c->in, past = c->taps - 1;
  float *buf = (float *)malloc(sizeof(float) * (size_t)(past + rows) * in);
  memcpy(buf, c->hist, sizeof(float) * (size_t)past * in);
  memcpy(buf + (size_t)past * in, x, sizeof(float) * (size_t)rows * in);
#pragma omp parallel for schedule(static)
  for (int t = 0; t < rows; t++)
    for (int j = 0; j < c->stride; j++)
      for (int o = 0; o < c->out; o++) {
        double acc = 0.0;
        for (int i = 0; i < c->taps; i++) {
          const float *xr = buf + (size_t)(past + t - i) * in;
          for (int ch = 0; ch < in; ch++)
            acc += (double)c->w[((size_t)ch * c->out + o) * c->k + j + i * c->stride] * xr[ch];
        }
        y[((size_t)t * c->stride + j) * c->out + o] = (float)(acc + c->b[o]);
      }
  if (past) memcpy(c->hist, buf + (size_t)rows * in, sizeof(float) * (size_t)past * in);
  free(buf);
}

static void linear(const float *x, int rows, int in, const float *w, const float *b, int out,
                   float *y) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < rows; t++)
    for (int o = 0; o < out; o++) {
      double acc = 0.0;
      for (int i = 0; i < in; i++) acc += (double)w[(size_t)o * in + i] * x[(size_t)t * in + i];
      y[(size_t)t * out + o] = (float)(acc + b[o]);
    }
}

/* y = x + gamma * pw2(gelu(pw1(layernorm(dwconv(x))))) */
static void next_forward(next_t *n, const float *x, int rows, float *y) {
  const int C = LATENT;
  float *buf = (float *)malloc(sizeof(float) * (size_t)(6 + rows) * C);
  float *h = (float *)malloc(sizeof(float) * (size_t)rows * C);
  float *g = (float *)malloc(sizeof(float) * (size_t)rows * 4 * C);
  memcpy(buf, n->hist, sizeof(float) * 6 * C);
  memcpy(buf + (size_t)6 * C, x, sizeof(float) * (size_t)rows * C);
#pragma omp parallel for schedule(static)
  for (int t = 0; t < rows; t++) {
    float *hr = h + (size_t)t * C;
    for (int c = 0; c < C; c++) {
      double acc = 0.0;
      for (int k = 0; k < 7; k++) acc += (double)n->dw_w[c * 7 + k] * buf[(size_t)(t + k) * C + c];
      hr[c] = (float)(acc + n->dw_b[c]);
    }
    double mean = 0.0, var = 0.0;
    for (int c = 0; c < C; c++) mean += hr[c];
    mean /= C;
    for (int c = 0; c < C; c++) var += (hr[c] - mean) * (hr[c] - mean);
    var /= C;
    const double inv = 1.0 / sqrt(var + 1e-6);
    for (int c = 0; c < C; c++) hr[c] = (float)((hr[c] - mean) * inv * n->nw[c] + n->nb[c]);
  }
  memcpy(n->hist, buf + (size_t)rows * C, sizeof(float) * 6 * C);
  linear(h, rows, C, n->pw1_w, n->pw1_b, 4 * C, g);
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < (size_t)rows * 4 * C; i++) {
    const double v = g[i];
    g[i] = (float)(0.5 * v * (1.0 + erf(v / sqrt(2.0))));
  }
  linear(g, rows, 4 * C, n->pw2_w, n->pw2_b, C, h);
  for (size_t i = 0; i < (size_t)rows * C; i++) y[i] = x[i] + n->gamma[i % C] * h[i];
  free(buf);
  free(h);
  free(g);
}

static void res_forward(res_t *r, float *x, int rows, int dim) {
  float *c = (float *)malloc(sizeof(float) * (size_t)rows * dim);
  float *d = (float *)malloc(sizeof(float) * (size_t)rows * dim);
  memcpy(c, x, sizeof(float) * (size_t)rows * dim);
  snake_apply(&r->a1, c, rows);
  conv_forward(&r->c1, c, rows, d);
  snake_apply(&r->a2, d, rows);
  conv_forward(&r->c2, d, rows, c);
  for (size_t i = 0; i < (size_t)rows * dim; i++) x[i] = c[i] + x[i];
  free(c);
  free(d);
}

q3o_codec *q3o_codec_create(const q3o_codec_weights *w) {
  q3o_codec *c = (q3o_codec *)calloc(1, sizeof(*c));
  for (int i = 0; i < 2; i++) {
    tconv_t *u = &c->up[i];
    u->w = w->up_w[i];
    u->b = w->up_b[i];
    u->in = u->out = LATENT;
    u->k = u->stride = 2;
    u->taps = 1;
    u->hist = (float *)calloc(LATENT, sizeof(float));
    next_t *n = &c->next[i];
    n->dw_w = w->dw_w[i];
    n->dw_b = w->dw_b[i];
    n->nw = w->norm_w[i];
    n->nb = w->norm_b[i];
    n->pw1_w = w->pw1_w[i];
    n->pw1_b = w->pw1_b[i];
    n->pw2_w = w->pw2_w[i];
    n->pw2_b = w->pw2_b[i];
    n->gamma = w->gamma[i];
    n->hist = (float *)calloc(6 * LATENT, sizeof(float));
  }
  conv_init(&c->conv0, w->conv0_w, w->conv0_b, LATENT, DEC_DIM, 7, 1);
  for (int i = 0; i < 4; i++) {
    block_t *b = &c->blocks[i];
    const q3o_codec_block *bw = &w->block[i];
    b->in = DEC_DIM >> i;
    b->out = DEC_DIM >> (i + 1);
    b->rate = RATES[i];
    snake_init(&b->act, bw->act_alpha, bw->act_beta, b->in);
    b->up.w = bw->up_w;
    b->up.b = bw->up_b;
    b->up.in = b->in;
    b->up.out = b->out;
    b->up.k = 2 * b->rate;
    b->up.stride = b->rate;
    b->up.taps = 2;
    b->up.hist = (float *)calloc(b->in, sizeof(float));
    for (int r = 0; r < 3; r++) {
      const q3o_codec_res *rw = &bw->res[r];
      snake_init(&b->res[r].a1, rw->a1_alpha, rw->a1_beta, b->out);
      snake_init(&b->res[r].a2, rw->a2_alpha, rw->a2_beta, b->out);
      conv_init(&b->res[r].c1, rw->c1_w, rw->c1_b, b->out, b->out, 7, DILS[r]);
      conv_init(&b->res[r].c2, rw->c2_w, rw->c2_b, b->out, b->out, 1, 1);
    }
  }
  snake_init(&c->act_out, w->out_alpha, w->out_beta, DEC_DIM >> 4);
  conv_init(&c->conv_out, w->out_w, w->out_b, DEC_DIM >> 4, 1, 7, 1);
  return c;
}

static void conv_reset(conv_t *c) { memset(c->hist, 0, sizeof(float) * (size_t)c->past * c->in); }

void q3o_codec_reset(q3o_codec *c) {
  for (int i = 0; i < 2; i++) memset(c->next[i].hist, 0, sizeof(float) * 6 * LATENT);
  conv_reset(&c->conv0);
  for (int i = 0; i < 4; i++) {
    memset(c->blocks[i].up.hist, 0, sizeof(float) * c->blocks[i].in);
    for (int r = 0; r < 3; r++) {
      conv_reset(&c->blocks[i].res[r].c1);
      conv_reset(&c->blocks[i].res[r].c2);
    }
  }
  conv_reset(&c->conv_out);
}

void q3o_codec_back(q3o_codec *c, const float *x, int frames, float *pcm) {
  if (frames <= 0) return;
  const size_t big = (size_t)frames * FRAME_SAMPLES * 96 > (size_t)frames * 32 * DEC_DIM
                         ? (size_t)frames * FRAME_SAMPLES * 96
                         : (size_t)frames * 32 * DEC_DIM;
  float *a = (float *)malloc(sizeof(float) * big);
  float *b = (float *)malloc(sizeof(float) * big);
  memcpy(a, x, sizeof(float) * (size_t)frames * LATENT);
  int rows = frames;
  for (int i = 0; i < 2; i++) {
    tconv_forward(&c->up[i], a, rows, b);
    rows *= 2;
    next_forward(&c->next[i], b, rows, a);
  }
  conv_forward(&c->conv0, a, rows, b);
  for (int i = 0; i < 4; i++) {
    block_t *bl = &c->blocks[i];
    snake_apply(&bl->act, b, rows);
    tconv_forward(&bl->up, b, rows, a);
    rows *= bl->rate;
    for (int r = 0; r < 3; r++) res_forward(&bl->res[r], a, rows, bl->out);
    float *t = a;
    a = b;
    b = t;
  }
  snake_apply(&c->act_out, b, rows);
  conv_forward(&c->conv_out, b, rows, a);
  for (int i = 0; i < rows; i++) pcm[i] = a[i] > 1.0f ? 1.0f : (a[i] < -1.0f ? -1.0f : a[i]);
  free(a);
  free(b);
}

static void snake_free(snake_t *s) {
  free(s->a);
  free(s->ib);
}

void q3o_codec_destroy(q3o_codec *c) {
  if (!c) return;
  for (int i = 0; i < 2; i++) {
    free(c->up[i].hist);
    free(c->next[i].hist);
  }
  free(c->conv0.hist);
  for (int i = 0; i < 4; i++) {
    snake_free(&c->blocks[i].act);
    free(c->blocks[i].up.hist);
    for (int r = 0; r < 3; r++) {
      snake_free(&c->blocks[i].res[r].a1);
      snake_free(&c->blocks[i].res[r].a2);
      free(c->blocks[i].res[r].c1.hist);
      free(c->blocks[i].res[r].c2.hist);
    }
  }
  snake_free(&c->act_out);
  free(c->conv_out.hist);
  free(c);
}
