/* q3o.h - CPU restatement of the Qwen3-TTS frame step (the oracle).
 *
 * TEST INFRASTRUCTURE ONLY. The tests compare the HIP library (libq3h)
 * against this one: only tests/, __graft_entry__.smoke() and the cpu_baseline leg of
 * bench.py may load it. The product path never links or calls it.
 *
 * What it restates (reference files, relative to the reference checkout):
 *  - Q8_0 block format and quantizer: ggml block_q8_0 / quantize_row_q8_0_ref,
 *    named at src/tts/mormot.ai.tts.qwen.lm.pas:259-267 (TQwenLmHeads.MatrixRows)
 *    and sized at lm.pas:182-197 (StackBytes).
 *  - the Qwen3 stack fed with embedding rows (TDecoderModel.ForwardEmbeds,
 *    called at lm.pas:391-408; the layer math follows the model note of
 *    tests/data/infer-ref/qwen3-tts-lm/manifest.json: per-head q_norm/k_norm,
 *    SwiGLU, no bias, rotate_half RoPE theta 1e6, RMSNorm eps 1e-6).
 *  - TQwenLm.Forward (lm.pas:391-408): the normed last row and its head.
 *  - TQwenTalker.ChooseCode0 / ChooseCode / AddRow / NextFrame
 *    (src/tts/mormot.ai.tts.qwen.talker.pas:423-429, 595-681) in greedy mode.
 *  - InferArgMax with the first-max rule of tests/test.tts.qwen.lm.pas:109-117.
 *
 * How each part is pinned (tests/test_oracle_*.py):
 *  - fp16 conversion: against numpy float16 (round to nearest even) on every
 *    finite half value and random floats, subnormals and overflow included;
 *  - Q8_0 quantizer: closed forms (zeros, the amax element is +-127, halfway
 *    rounding away from zero), brute force against an independent numpy
 *    restatement, dequantization error <= d/2;
 *  - f32 stack: golden vectors from the third-party transformers Qwen3Model
 *    (tests/golden/make_qwen3_golden.py), incremental calls == one call
 *    (the causal property the reference fixture states for predictor.logits);
 *  - argmax / ChooseCode0: the reference fixture's logits rows and codes
 *    (tests/data/infer-ref/qwen3-tts-lm: predictor.codes = argmax of each row)
 *    plus brute-force checks of the logits processors on tiny vectors.
 *  - Q8_0 stack numerics (activation quantization or not) of the un-vendored
 *    mormot2-ai engine: parity unpinned (both modes are provided); the int8
 *    layer's composition (which inputs are quantized, the block products and
 *    their order) is checked op by op against numpy through
 *    q3o_forward_embeds_traced;
 *  - the frame step (q3o_frame_*): marker tables through zero-weight stacks
 *    (closed-form codes and decoded states) and a composition of NextFrame
 *    over transformers' Qwen3 decoder.
 */
#ifndef Q3O_H
#define Q3O_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q3O_F32 0
#define Q3O_Q8_0 1
#define Q3O_BF16 2 /* text embedding only */

/* ggml block_q8_0: fp16 scale then 32 int8 quants, 34 bytes */
typedef struct {
  uint16_t d;
  int8_t qs[32];
} q3o_block_q8_0;

typedef struct {
  int32_t layers, hidden, heads, kv_heads, head_dim, intermediate;
  float rms_eps, rope_theta;
  int32_t dtype;  /* Q3O_F32 or Q3O_Q8_0 (weights and heads) */
  int32_t kv_f16; /* K/V cache rounded to half floats */
  int32_t act_q8; /* Q8_0 only: 1 = activations quantized per 32-block
                     (int32 block dot, ggml vec_dot_q8_0_q8_0), 0 = f32
                     activations times dequantized weights */
} q3o_config;

/* one layer: matrices [out][in] row-major, f32 or ggml Q8_0 blocks */
typedef struct {
  const void *wq, *wk, *wv, *wo, *wgate, *wup, *wdown;
  const float *input_norm, *post_norm, *q_norm, *k_norm;
} q3o_layer;

typedef struct q3o_stack q3o_stack;
typedef struct q3o_ctx q3o_ctx;
typedef struct q3o_frame q3o_frame;

void q3o_set_threads(int n);
int q3o_get_threads(void);

uint16_t q3o_fp32_to_fp16(float f);
float q3o_fp16_to_fp32(uint16_t h);
void q3o_fp32_to_fp16_row(const float *x, uint16_t *y, int64_t n);
void q3o_fp16_to_fp32_row(const uint16_t *x, float *y, int64_t n);

/* k % 32 == 0 */
void q3o_quantize_row_q8_0(const float *x, void *y, int64_t k);
void q3o_dequantize_row_q8_0(const void *x, float *y, int64_t k);
/* rows x cols matrix, rows in parallel (the bytes do not depend on threads) */
void q3o_quantize_matrix_q8_0(const float *x, void *y, int64_t rows, int64_t cols);

/* the stack keeps the pointers (no copy): they must outlive it */
q3o_stack *q3o_stack_create(const q3o_config *cfg, const q3o_layer *layers,
                            const float *final_norm);
void q3o_stack_destroy(q3o_stack *s);

q3o_ctx *q3o_ctx_create(q3o_stack *s, int max_positions);
void q3o_ctx_destroy(q3o_ctx *c);
void q3o_ctx_reset(q3o_ctx *c);
int q3o_ctx_length(const q3o_ctx *c);
/* raw K/V rows of one layer: [kv_heads][max_positions][head_dim] f32 */
const float *q3o_ctx_k(const q3o_ctx *c, int layer);
const float *q3o_ctx_v(const q3o_ctx *c, int layer);
/* write K/V of positions [0, len) directly (long-context setups);
   k, v: [layers][kv_heads][len][head_dim]; sets the length */
int q3o_ctx_fill(q3o_ctx *c, const float *k, const float *v, int len);

/* x [rows][hidden] at positions length..length+rows-1; normed_last [hidden]
   (nullable); layer_out [layers][rows][hidden] raw layer outputs (nullable);
   returns 0, or -1 when the context would overflow */
/* the stack's RMSNorm (double sum of squares) of `rows` rows of n values:
   the final norm of every row that TQwenLm's probe receives as name.out
   (lm.pas:383-384) */
void q3o_rmsnorm_rows(const float *x, int rows, int n, const float *w, float eps, float *y);
int q3o_forward_embeds(q3o_ctx *c, const float *x, int rows, float *normed_last,
                       float *layer_out);

/* the operands of every product of a forward, per layer l (each pointer
   nullable; [layers][rows][n] row-major, blocks as ggml block_q8_0):
   x_*: the f32 input of the product (the normed row, the attention output,
   the post-attention normed row, SwiGLU's output); b_*: the Q8_0 blocks of
   that input the int8 products read (act_q8 stacks only); y_*: the product's
   output, before any residual add (q/k/v before QK-norm and RoPE) */
typedef struct {
  float *x_qkv, *y_qkv;   /* [H], [NQ + 2 NKV] (q, k, v side by side) */
  void *b_qkv;            /* [H / 32] */
  float *x_o, *y_o;       /* [NQ], [H] */
  void *b_o;              /* [NQ / 32] */
  float *x_gu, *y_gate, *y_up; /* [H], [I], [I] */
  void *b_gu;             /* [H / 32] */
  float *x_down, *y_down; /* [I], [H] */
  void *b_down;           /* [I / 32] */
} q3o_trace;

/* q3o_forward_embeds with the operands of its products written to *t */
int q3o_forward_embeds_traced(q3o_ctx *c, const float *x, int rows, float *normed_last,
                              float *layer_out, const q3o_trace *t);

/* logits[rows_out] = W[rows_out][hidden] . state, W f32 or Q8_0 */
void q3o_head(const void *w, int dtype, int act_q8, int rows_out, int hidden,
              const float *state, float *logits);

/* TQwenTalker.TextProject (talker.pas:390-421): y [n][hidden] =
   fc2 . SiLU(fc1 . emb[ids[r]] + b1) + b2, SiLU 0 below -80; emb
   [vocab][text_hidden] in Q3O_F32 or Q3O_BF16, fc1 [text_hidden][text_hidden],
   fc2 [hidden][text_hidden] f32. Returns 0, or -1 (nothing written) when an
   id is out of range. */
int q3o_text_project(const void *emb, int emb_dtype, int vocab, int text_hidden, int hidden,
                     const float *fc1_w, const float *fc1_b, const float *fc2_w,
                     const float *fc2_b, const int32_t *ids, int n, float *y);

/* first max wins */
int q3o_argmax(const float *p, int n);

/* e^x from IEEE operations only (Cody-Waite reduction, Taylor series to r^7),
   the exponential of the attention softmax and of SiLU; < 2 ulp, 0 below
   -86, +inf above 88 */
float q3o_expf(float x);

/* TQwenTalker.ChooseCode0, greedy: logits processors then argmax */
int q3o_choose_code0(const float *logits, int vocab, int eos, const int *history,
                     int nhistory, float penalty);

/* Philox4x64-10 (Salmon et al., SC 2011): out = the block of counter ctr
   under key */
void q3o_philox4x64(const uint64_t ctr[4], const uint64_t key[2], uint64_t out[4]);
/* the sampler's uniform of draw (frame, group) under seed: counter (frame,
   group, 0, 0), key (seed, 0), (first output >> 40) * 2^-24 */
float q3o_draw_uniform(uint64_t seed, uint64_t frame, uint64_t group);
/* the library's draw from x[n] (n <= 3072): temperature, top-k (0: off),
   top-p (1: off; applied when 1 <= top_k <= 64), then u through the inverse
   distribution in the library's evaluation order; returns the index */
int q3o_sample(const float *x, int n, float temperature, int top_k, float top_p, float u);

/* TQwenSampling (talker.pas:60-70) without the repetition penalty (a frame
   table); seed: the sentence seed (the sub-sampler uses seed xor 0x5DEECE66D,
   talker.pas:585) */
typedef struct {
  int32_t do_sample;
  float temperature;
  int32_t top_k;
  float top_p;
  int32_t sub_do_sample;
  float sub_temperature;
  int32_t sub_top_k;
  float sub_top_p;
  uint64_t seed;
} q3o_sampling;

/* frame step: the talker and code-predictor stacks, their heads, the tables */
typedef struct {
  const void *talker_head; /* [vocab][hidden] */
  const void *cp_heads[15]; /* [cp_vocab][hidden] */
  const float *codec_emb;  /* [vocab][hidden] */
  const float *pred_emb[15]; /* [cp_vocab][hidden] */
  int32_t vocab, cp_vocab, groups;
  int32_t eos; /* -1: none */
  float penalty;
  const float *tts_pad; /* [hidden] */
} q3o_frame_tables;

q3o_frame *q3o_frame_create(q3o_stack *talker, q3o_stack *cp,
                            const q3o_frame_tables *t, int max_positions);
void q3o_frame_destroy(q3o_frame *f);
/* TQwenTalker.Start's talker part: reset, prefill rows, logits + past state;
   trailing [trailing_rows][hidden] is copied */
int q3o_frame_start(q3o_frame *f, const float *prefill, int rows,
                    const float *trailing, int trailing_rows);
/* TQwenTalker.NextFrame: 1 and codes[groups], or 0 at eos */
int q3o_frame_next(q3o_frame *f, int *codes);
const float *q3o_frame_logits(const q3o_frame *f);
const float *q3o_frame_past_hidden(const q3o_frame *f);
q3o_ctx *q3o_frame_talker_ctx(q3o_frame *f);
/* the choosers of q3o_frame_next: argmax (the default) or the draws of
   q3o_sample with the uniforms of q3o_draw_uniform (code 0: seed, group 0;
   code g: seed ^ 0x5DEECE66D, group g; frame = frames emitted before) */
void q3o_frame_set_sampling(q3o_frame *f, const q3o_sampling *s);

/* ---- the 12 Hz decoder's back part (q3o_codec.c) ---- */

/* the tensors of TQwenCodec's back part (codec.pas:644-751), f32, in the
   safetensors layouts (decoder.* of the speech tokenizer) */
typedef struct {
  const float *a1_alpha, *a1_beta; /* block.{2+r}.act1 [dim] */
  const float *c1_w, *c1_b;        /* block.{2+r}.conv1.conv [dim][dim][7], [dim] */
  const float *a2_alpha, *a2_beta; /* act2 */
  const float *c2_w, *c2_b;        /* conv2.conv [dim][dim][1], [dim] */
} q3o_codec_res;

typedef struct {
  const float *act_alpha, *act_beta; /* decoder.{i+1}.block.0 [in] */
  const float *up_w, *up_b;          /* block.1.conv [in][out][2 rate], [out] */
  q3o_codec_res res[3];              /* dilations 1, 3, 9 */
} q3o_codec_block;

typedef struct {
  const float *up_w[2], *up_b[2];     /* upsample.i.0.conv [1024][1024][2], [1024] */
  const float *dw_w[2], *dw_b[2];     /* upsample.i.1.dwconv.conv [1024][1][7], [1024] */
  const float *norm_w[2], *norm_b[2]; /* upsample.i.1.norm [1024] */
  const float *pw1_w[2], *pw1_b[2];   /* upsample.i.1.pwconv1 [4096][1024], [4096] */
  const float *pw2_w[2], *pw2_b[2];   /* upsample.i.1.pwconv2 [1024][4096], [1024] */
  const float *gamma[2];              /* upsample.i.1.gamma [1024] */
  const float *conv0_w, *conv0_b;     /* decoder.0.conv [1536][1024][7], [1536] */
  q3o_codec_block block[4];           /* decoder.1 .. 4: 1536 -> 768 -> 384 -> 192 -> 96 */
  const float *out_alpha, *out_beta;  /* decoder.5 [96] */
  const float *out_w, *out_b;         /* decoder.6.conv [1][96][7], [1] */
} q3o_codec_weights;

typedef struct q3o_codec q3o_codec;

/* TQwenCodec's back part (codec.pas:1040-1083); the weights are referenced,
   not copied */
q3o_codec *q3o_codec_create(const q3o_codec_weights *w);
/* TQwenCodec.Reset: the histories back to zeros */
void q3o_codec_reset(q3o_codec *c);
/* x [frames][1024] (the transformer output) -> pcm [frames * 1920] */
void q3o_codec_back(q3o_codec *c, const float *x, int frames, float *pcm);
void q3o_codec_destroy(q3o_codec *c);

#ifdef __cplusplus
}
#endif
#endif
