/* q3h.h - C ABI of libq3h, the MI355X (gfx950) engine of the Qwen3-TTS frame
 * step: the talker (Qwen3, 28 layers) and the code predictor (Qwen3, 5 layers,
 * 15 forwards per frame), with device-resident weights and K/V caches.
 *
 * Every entry point is extern "C", cdecl, takes plain pointers and sizes, and
 * returns an int status: 0 on success, a negative Q3H_E* code on failure, with
 * the message in q3h_last_error() (thread-local, valid until the next call on
 * the same thread). Ownership follows mormot.ai.tts.qwen.lm.pas:364-368
 * (TQwenLm.Destroy): contexts and frames before their stacks, stacks before
 * their device. A stack may serve contexts used from several threads at once;
 * one context (or frame) is used by one thread at a time
 * (mormot.ai.tts.qwen.talker.pas:77). Each entry point makes its device
 * current, so calls may arrive on any thread (mormot.ai.tts.qwen.pas:281-291).
 *
 * Each declaration names the reference interface it replaces (paths relative
 * to the reference checkout). The mormot2-ai engine those Pascal call sites
 * reach (TQwen3Model, TQwen3Vulkan, TDecoderContext) is an un-vendored
 * submodule; only its call sites in the reference tree are cited.
 */
#ifndef Q3H_H
#define Q3H_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* weight formats: the host side of q3h_stack_create / q3h_stack_add_head,
   and the storage of a stack (TInferDType idtF32 / idtQ8_0) */
#define Q3H_F32 0
#define Q3H_Q8_0 1 /* ggml block_q8_0 on the host: fp16 scale + 32 int8, 34 B */
#define Q3H_BF16 2 /* bfloat16 (the text embedding table) */

/* status codes */
#define Q3H_OK 0
#define Q3H_E_ARG (-1)      /* invalid argument or shape */
#define Q3H_E_HIP (-2)      /* a HIP runtime call failed */
#define Q3H_E_CAPACITY (-3) /* a context would exceed its positions */
#define Q3H_E_STATE (-4)    /* call out of order (e.g. step before start) */
#define Q3H_E_NODEV (-5)    /* no usable gfx950 device */

typedef struct q3h_device q3h_device;
typedef struct q3h_stack q3h_stack;
typedef struct q3h_context q3h_context;
typedef struct q3h_frame q3h_frame;
typedef struct q3h_text_proj q3h_text_proj;
typedef struct q3h_codec q3h_codec;

/* TDecoderConfig (mormot.ai.tts.qwen.lm.pas:184-191) + TQwen3Vulkan.KvF16
   (lm.pas:353) + the numerics of the Q8_0 products */
typedef struct {
  int32_t layers, hidden, heads, kv_heads, head_dim, intermediate;
  float rms_eps, rope_theta;
  int32_t dtype;         /* storage: Q3H_F32 or Q3H_Q8_0 (weights and heads) */
  int32_t kv_f16;        /* K/V cache in half floats (lm.pas:128-130) */
  int32_t act_q8;        /* Q8_0 only: 1 = activations quantized per 32-block
                            (int8 products, ggml vec_dot_q8_0_q8_0); 0 = f32
                            activations times dequantized weights */
  int32_t max_positions; /* the largest context of this stack (RoPE table) */
} q3h_stack_config;

/* one layer, host memory, matrices [out][in] row-major in src_dtype */
typedef struct {
  const void *wq, *wk, *wv, *wo, *wgate, *wup, *wdown;
  const float *input_norm, *post_norm; /* [hidden] */
  const float *q_norm, *k_norm;        /* [head_dim] */
} q3h_layer_weights;

typedef struct {
  int32_t src_dtype;               /* Q3H_F32, Q3H_Q8_0 (ggml blocks) or Q3H_BF16 (the
                                      safetensors rows as stored: widened and, for a
                                      Q8_0 stack, quantized on the device, the
                                      conversion of lm.pas:244-308) */
  const q3h_layer_weights *layers; /* [layers] */
  const float *final_norm;         /* [hidden] */
} q3h_weights;

/* ---- device: replaces TQwenVulkan (lm.pas:44-62, 202-222) ---- */

/* 1 when a gfx950 device is present (TQwenVulkan.Available, lm.pas:202-205) */
int q3h_device_available(void);
/* TQwenVulkan.Create (lm.pas:207-211) */
int q3h_device_open(int ordinal, q3h_device **out);
/* TQwenVulkan.DeviceName (lm.pas:219-222); NULL on a NULL device */
const char *q3h_device_name(const q3h_device *dev);
/* TQwenVulkan.DeviceBytes (lm.pas:57-59): the weight bytes of its stacks */
int64_t q3h_device_bytes(const q3h_device *dev);
/* TQwenVulkan.Destroy (lm.pas:213-217) */
int q3h_device_close(q3h_device *dev);
/* the message of the last failure on this thread ("" if none) */
const char *q3h_last_error(void);

/* ---- stack: replaces TQwen3Model.CreateStack (lm.pas:174-179) followed by
   TQwen3Vulkan.Create(model, backend) (lm.pas:351); the library copies (and
   quantizes or repacks) the host weights, so they may be freed on return ---- */
int q3h_stack_create(q3h_device *dev, const q3h_stack_config *cfg,
                     const q3h_weights *w, q3h_stack **out);
/* TQwenLmHeads.Add (lm.pas:277-308): a head [rows][hidden] in src_dtype
   (Q3H_F32, Q3H_Q8_0 or Q3H_BF16), stored in the stack's dtype; *index
   receives its number (0, 1, ...) */
int q3h_stack_add_head(q3h_stack *s, const void *w, int rows, int src_dtype,
                       int *index);
/* StackBytes (lm.pas:182-197) of the layers on the device, heads excluded */
int64_t q3h_stack_bytes(const q3h_stack *s);
/* TQwen3Vulkan.Free (lm.pas:366) */
int q3h_stack_destroy(q3h_stack *s);

/* ---- context: replaces TQwen3Vulkan.NewContext / TDecoderContext ---- */

/* lm.pas:354 (NewContext); max_positions <= the stack's max_positions */
int q3h_context_create(q3h_stack *s, int max_positions, q3h_context **out);
/* TQwenLm.Reset (lm.pas:374-378): the next row is at position 0 */
int q3h_context_reset(q3h_context *c);
/* TQwenLm.Length (lm.pas:136-138); negative on error */
int q3h_context_length(const q3h_context *c);
/* lm.pas:365 (fCtx.Free) */
int q3h_context_destroy(q3h_context *c);
/* no reference counterpart (long-context setups and tests): write the K/V of
   positions [0, len) from host f32 [layers][kv_heads][len][head_dim] (rounded
   to half floats when kv_f16) and set the length to len */
int q3h_context_fill_kv(q3h_context *c, const float *k, const float *v, int len);
/* no reference counterpart (tests): read the K/V cache of one layer for
   positions [0, length) as f32 [kv_heads][length][head_dim] */
int q3h_context_read_kv(q3h_context *c, int layer, float *k, float *v);
/* no reference counterpart (measurement): the decode attention of every
   layer for one new row at position length (the attention kernels of
   q3h_forward_embeds with rows = 1, fused QK-norm / RoPE / K/V append),
   launched directly iters times over the layers on one stream.
   us_per_launch: the time between two events around those launches per
   layer (with the merge of the splits on long contexts: both kernels and the
   gaps between launches); bytes_per_launch: algorithmic bytes
   (the cache of length positions read, the new key and value written, the
   q / k / v row read, the outputs written). The row's q / k / v are zeros;
   the key and value written at position length are scratch (the length does
   not change). Stacks with f32 activations (act_q8 = 0). */
int q3h_context_time_attention(q3h_context *c, int iters, float *us_per_launch,
                               int64_t *bytes_per_launch);

/* ---- the forward: TQwenLm.Forward (lm.pas:391-408), i.e.
   TQwen3Vulkan.ForwardEmbeds(ctx, x, rows, nil, false, fLast) (lm.pas:397)
   followed by fCpu.Linear(fLast, 1, hidden, head, rows) (lm.pas:404-406),
   with the head on the device. x [rows][hidden] host f32 at positions
   length..length+rows-1; normed_last [hidden] (nullable) receives the
   final-normed state of the last row; head: an index of q3h_stack_add_head,
   or -1 for none; logits [head rows] (nullable). Blocks until the outputs
   are in host memory. rows <= 0 does nothing (lm.pas:394-395). One row
   replays a HIP graph the context captures per (head, position cover)
   (covers of 64 positions up to 256, of 256 beyond; at most 32 graphs per
   context, dropped when its work buffers grow) and copies its row, logits
   and state through a pinned host buffer of the context; the results are
   those of the same launches made directly (q3h_forward_embeds_noalloc). ---- */
int q3h_forward_embeds(q3h_context *c, const float *x, int rows, int head,
                       float *logits, float *normed_last);

/* No counterpart in the reference. For callers that cannot allocate device
   memory (tight serving loops, harnesses that forbid hipMalloc); it is called
   outside any stream capture, like q3h_forward_embeds: it launches on the
   context's own stream, copies pageable host memory and blocks until the
   outputs are in host memory. q3h_forward_embeds with the same arguments and results,
   but its work buffers are carved from one static device array of
   Q3H_NOALLOC_SCRATCH_BYTES per GPU (set up by q3h_device_open) instead of
   the context's own buffers, which q3h_forward_embeds grows with hipMalloc.
   Calls no allocating routine. rows <= Q3H_NOALLOC_MAX_ROWS, and the
   buffers of the call (they grow with rows and, for fewer than 16 rows of
   an f32-activation stack over more than 256 positions, with the decode
   attention's splits) must fit the array: otherwise
   Q3H_E_CAPACITY and nothing is computed. Every call on one GPU shares that
   GPU's array, which keeps the last call's contents (no kernel reads a
   buffer before writing it); calls on one device are serialized by a lock
   of the device, since overlapping calls would race on the array. */
#define Q3H_NOALLOC_MAX_ROWS 64
#define Q3H_NOALLOC_SCRATCH_BYTES (16 << 20)
int q3h_forward_embeds_noalloc(q3h_context *c, const float *x, int rows, int head,
                               float *logits, float *normed_last);

/* TQwenLm.Forward with TQwenLm.Probe set (lm.pas:139-142, 380-389: the
   probe receives the output of every layer, "name.layerN", then the normed
   state of every row, "name.out"): q3h_forward_embeds, plus layer_out
   [layers][rows][hidden] (host f32, nullable) receiving the raw output of
   each layer for every row (the residual stream after the layer's down
   projection), so that a difference against another implementation can be
   located at a layer, and normed_rows [rows][hidden] (host f32, nullable)
   receiving the final RMSNorm of every row (normed_last is its last row).
   The outputs are those of q3h_forward_embeds; the copies add one
   device-to-device copy per layer. */
int q3h_forward_embeds_probe(q3h_context *c, const float *x, int rows, int head,
                             float *logits, float *normed_last, float *layer_out,
                             float *normed_rows);

/* no reference counterpart (the reference is single-stream): one row per
   context, n contexts of the same stack at their own positions;
   x [n][hidden]; heads [n] (or NULL: no logits); logits [n][head rows of
   heads[0]] (all heads of one call must have the same rows); normed [n][hidden]
   (nullable). */
int q3h_forward_embeds_batch(q3h_context *const *ctxs, int n, const float *x,
                             const int *heads, float *logits, float *normed);

/* ---- the frame step: a device-resident, greedy restatement of
   TQwenTalker.NextFrame (talker.pas:640-681) with ChooseCode0 (talker.pas:
   595-630), ChooseCode (talker.pas:632-638) and AddRow (talker.pas:423-429),
   for n_streams independent sentences, replayed as one hipGraph per step ---- */
typedef struct {
  int32_t n_streams;          /* 1..64 */
  int32_t talker_head;        /* head index in the talker stack */
  int32_t cp_heads[15];       /* head indices in the code-predictor stack */
  int32_t vocab, cp_vocab;    /* 3072, 2048 */
  int32_t groups;             /* 16 */
  int32_t eos;                /* codec_eos_token_id, -1: none */
  float repetition_penalty;   /* 1.05 (talker.pas:215) */
  int32_t max_frames;         /* frames per sentence (history capacity) */
  int32_t max_positions;      /* talker positions per stream */
  int32_t use_graph;          /* 1: capture the step once, replay it */
} q3h_frame_config;

/* TQwenTalker.Create's tables (talker.pas:300-311): codec_emb [vocab][hidden],
   pred_emb[g] [cp_vocab][hidden] (g = 0..groups-2), tts_pad [hidden];
   copied to the device */
int q3h_frame_create(q3h_stack *talker, q3h_stack *cp, const q3h_frame_config *cfg,
                     const float *codec_emb, const float *const *pred_emb,
                     const float *tts_pad, q3h_frame **out);
/* the talker part of TQwenTalker.Start (talker.pas:586-593): reset stream s,
   prefill its rows, keep the logits and the last normed state; trailing
   [trailing_rows][hidden] (talker.pas:578-580) follows the frames */
int q3h_frame_start(q3h_frame *f, int stream, const float *prefill, int rows,
                    const float *trailing, int trailing_rows);
/* no reference counterpart (batched serving; the reference starts one
   sentence at a time): q3h_frame_start for n distinct streams at once, each
   prefill on its stream's own talker context and HIP stream so that the
   prefills overlap on the device; blocks until all are done. streams [n];
   prefill[i] [rows[i]][hidden]; trailing (nullable) and trailing_rows
   (nullable: none) as q3h_frame_start's per stream. The results equal n
   calls of q3h_frame_start. Every argument is checked before any prefill is
   enqueued (a bad or repeated stream: Q3H_E_ARG, nothing started). */
int q3h_frame_start_batch(q3h_frame *f, int n, const int *streams,
                          const float *const *prefill, const int *rows,
                          const float *const *trailing, const int *trailing_rows);
/* one NextFrame for every started stream: codes [n_streams][groups] (-1 for a
   stream that has ended); alive [n_streams] (nullable) 1 while a stream runs,
   0 once its code 0 was eos. */
int q3h_frame_step(q3h_frame *f, int32_t *codes, int32_t *alive);
/* the talker logits [vocab] and normed state [hidden] of stream s (nullable
   outputs), as fLogits / fPastHidden after the last Start or step */
int q3h_frame_state(q3h_frame *f, int stream, float *logits, float *past_hidden);
int q3h_frame_destroy(q3h_frame *f);

/* TQwenSampling (talker.pas:60-70) without the repetition penalty (a frame
   setting): the choosers of code 0 (talker) and of codes 1..15 (code
   predictor, the sub-sampler). do_sample 0: argmax, as QwenGreedy. Else the
   scores (code 0: after ChooseCode0's processors) / temperature, top-k (0:
   off; ties at the k-th value kept), top-p (1: off; < 1 needs 1 <= top_k <=
   64), then one uniform through the inverse distribution (the logits warpers
   of Hugging Face generate(), which NewSampler, talker.pas:455-469,
   configures). Uniforms: Philox4x64-10 of counter (frame, group, 0, 0) under
   key (seed, 0) for code 0 (group 0), (seed xor 0x5DEECE66D, 0) for code g
   (group g), frame = frames of the sentence before this one. seed: the
   sentence seed of every q3h_frame_start* (0: a fresh random one per start,
   as talker.pas:582-584). At most 3072 codes per chooser. */
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
} q3h_sampling;

/* property TQwenTalker.Sampling (talker.pas:150-151) for every stream of the
   frame; takes effect at the next step (its seed at the next start) */
int q3h_frame_set_sampling(q3h_frame *f, const q3h_sampling *s);

/* ---- the text projection and the device-side prefill ---- */
typedef struct {
  int32_t text_vocab;  /* rows of the text embedding (talker text_vocab_size, 151936) */
  int32_t text_hidden; /* text_hidden_size, 2048 (1024, 2048 or 3072) */
  int32_t hidden;      /* the talker's hidden_size, 1024 (a multiple of 16) */
  int32_t emb_dtype;   /* Q3H_BF16 (as in the safetensors file) or Q3H_F32 */
} q3h_text_config;

/* TQwenTalker's text projection weights (talker.pas:302-307): emb
   [text_vocab][text_hidden] (talker.model.text_embedding), fc1 [text_hidden]
   [text_hidden] + b1 [text_hidden], fc2 [hidden][text_hidden] + b2 [hidden]
   (talker.text_projection.linear_fc1 / fc2, widened to f32); copied to the
   device as given (the products stay in f32) */
int q3h_text_create(q3h_device *dev, const q3h_text_config *cfg, const void *emb,
                    const float *fc1_w, const float *fc1_b, const float *fc2_w,
                    const float *fc2_b, q3h_text_proj **out);
/* TQwenTalker.TextProject (talker.pas:390-421): y [n][hidden] =
   fc2 . SiLU(fc1 . emb[ids[r]] + b1) + b2, SiLU 0 below -80. n == 0 does
   nothing; an id outside [0, text_vocab) is Q3H_E_ARG ("text token out of
   range", nothing computed) */
int q3h_text_project(q3h_text_proj *t, const int32_t *ids, int n, float *y);
int q3h_text_destroy(q3h_text_proj *t);

/* the special ids TQwenTalker.Start uses (talker.pas:256-261): text ids
   tts_bos / tts_eos / tts_pad (config tts_*_token_id), codec ids codec_pad /
   codec_bos (talker_config codec_pad_id / codec_bos_id) */
typedef struct {
  int32_t tts_bos, tts_eos, tts_pad;
  int32_t codec_pad, codec_bos;
} q3h_start_ids;

/* TQwenTalker.Start (talker.pas:471-593) from its token ids, on the device:
   ids [n_ids] = PromptIds (im_start, assistant, \n, the text, im_end, \n,
   im_start, assistant, \n; n_ids >= 9), codec [n_codec] = the think /
   language / speaker ids then codec_pad, codec_bos (n_codec >= 2). The
   prefill rows (the role, tts_pad / tts_bos over the codec ids, then the text
   over codec_pad and tts_eos, tts_pad over codec_bos when non_streaming, else
   the first text token over codec_bos) and the trailing rows are built on the
   device from t's projection and the frame's codec_emb, then stream s starts
   as q3h_frame_start does with them. tts_bos / tts_eos / tts_pad are
   projected with the text. Errors: an id out of range (Q3H_E_ARG), more
   rows than max_positions (Q3H_E_CAPACITY) or trailing rows than max_frames
   (Q3H_E_ARG). */
int q3h_frame_start_text(q3h_frame *f, int stream, q3h_text_proj *t, const q3h_start_ids *sp,
                         const int32_t *ids, int n_ids, const int32_t *codec, int n_codec,
                         int non_streaming);

/* ---- the 12 Hz decoder's back part: replaces TQwenCodecVulkan's GPU pass
   (src/tts/mormot.ai.tts.qwen.codec.vulkan.pas:568-652) ---- */

/* the tensors of the back part (TQwenCodec.Create, codec.pas:644-751), f32,
   host memory, in their safetensors layouts (decoder.* of the speech
   tokenizer); the library repacks and copies them */
typedef struct {
  const float *a1_alpha, *a1_beta; /* block.{2+r}.act1.alpha / beta [dim] */
  const float *c1_w, *c1_b;        /* block.{2+r}.conv1.conv [dim][dim][7], [dim] */
  const float *a2_alpha, *a2_beta; /* block.{2+r}.act2 */
  const float *c2_w, *c2_b;        /* block.{2+r}.conv2.conv [dim][dim][1], [dim] */
} q3h_codec_res;

typedef struct {
  const float *act_alpha, *act_beta; /* decoder.{i+1}.block.0 [in] */
  const float *up_w, *up_b;          /* block.1.conv [in][out][2 rate], [out] */
  q3h_codec_res res[3];              /* dilations 1, 3, 9 */
} q3h_codec_block;

typedef struct {
  const float *up_w[2], *up_b[2];     /* upsample.i.0.conv [1024][1024][2], [1024] */
  const float *dw_w[2], *dw_b[2];     /* upsample.i.1.dwconv.conv [1024][1][7], [1024] */
  const float *norm_w[2], *norm_b[2]; /* upsample.i.1.norm [1024] */
  const float *pw1_w[2], *pw1_b[2];   /* upsample.i.1.pwconv1 [4096][1024], [4096] */
  const float *pw2_w[2], *pw2_b[2];   /* upsample.i.1.pwconv2 [1024][4096], [1024] */
  const float *gamma[2];              /* upsample.i.1.gamma [1024] */
  const float *conv0_w, *conv0_b;     /* decoder.0.conv [1536][1024][7], [1536] */
  q3h_codec_block block[4];           /* decoder.1 .. 4 (rates 8, 5, 4, 3) */
  const float *out_alpha, *out_beta;  /* decoder.5 [96] */
  const float *out_w, *out_b;         /* decoder.6.conv [1][96][7], [1] */
} q3h_codec_weights;

/* TQwenCodecVulkan.CreateVulkan's upload (codec.vulkan.pas:166-237):
   max_frames frames per device pass (1..64; longer inputs run in passes, as
   CHUNK_FRAMES does) */
int q3h_codec_create(q3h_device *dev, const q3h_codec_weights *w, int max_frames,
                     q3h_codec **out);
/* TQwenCodecVulkan.Reset (codec.vulkan.pas:455-488): every history to zeros */
int q3h_codec_reset(q3h_codec *c);
/* TQwenCodecVulkan.Back (codec.vulkan.pas:633-652): x [frames][1024] (the
   transformer output) -> pcm [frames * 1920] in [-1, 1]. Causal: each
   convolution keeps the last rows of its input for the next call, and every
   output sums its terms in one order whatever the frames per call, so
   decoding 1 + 3 frames or 4 at once gives the same samples. */
int q3h_codec_back(q3h_codec *c, const float *x, int frames, float *pcm);
int64_t q3h_codec_bytes(const q3h_codec *c);
int q3h_codec_destroy(q3h_codec *c);

/* ---- helpers ---- */

/* ggml quantize_row_q8_0_ref (InferQuantizeRowQ8_0Ref, lm.pas:265-267) on the
   host: k % 32 == 0, y receives k/32 blocks of 34 bytes */
int q3h_quantize_row_q8_0(const float *x, void *y, int64_t k);

/* no reference counterpart (measurement): the weight products of one
   single-row decode step of stack s - per layer the fused q/k/v, o, gate/up
   and down matrix-vector products, then head `head` (-1: none) - run iters
   times on one stream. mode 0: launched directly, us_per_launch = wall time
   between two hipEvents / launches; mode 1: captured in a hipGraph and
   replayed, same wall-time measure; mode 2: every launch carries its own
   start / end events (hipExtLaunchKernelGGL), us_per_launch = the average
   execution time of the kernels themselves (Q8_0 stacks). launches: products
   per step; bytes: algorithmic bytes per step (weights, norm vectors, input
   and output vectors). The activations are zeros; contexts are untouched. */
int q3h_stack_time_gemv(q3h_stack *s, int head, int iters, int mode, float *us_per_launch,
                        int *launches, int64_t *bytes);

#ifdef __cplusplus
}
#endif
#endif
