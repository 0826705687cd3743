// q3h_frame.hip - the frame step of q3h.h: a device-resident, greedy
// restatement of TQwenTalker.NextFrame (mormot.ai.tts.qwen.talker.pas:640-681)
// for n independent streams. Per step: code 0 from the talker logits with the
// logits processors of ChooseCode0 (talker.pas:595-630), 15 code-predictor
// forwards (2 rows, then 14 x 1 row) each with its head and argmax
// (ChooseCode, talker.pas:632-638), the sum of the 16 embeddings plus the
// trailing text row (AddRow, talker.pas:423-429, 668-675), one talker forward
// with its head. No host round trip inside a step; the step is captured once
// in a hipGraph and replayed (re-captured only when the talker attention
// needs more position splits).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <type_traits>
#include <vector>

#include "q3h.h"
#include "q3h_api_internal.h"
#include "q3h_quant.h"
#include "q3h_sample.h"

namespace q3h {

// the device view of a frame (kernel argument, by value)
struct FrameDev {
  int n, H, vocab, cp_vocab, groups, eos, max_trailing;
  float penalty;
  float *logits;          // [n][vocab] talker logits
  float *past;            // [n][H] normed talker state
  int *codes;             // [n][groups]
  // the host's pinned copy of the codes [n][groups] and alive flags [n]
  // (coherent host memory, written by k_frame_end)
  int32_t *host_codes, *host_alive;
  uint8_t *seen;          // [n][vocab]: codes already emitted (repetition penalty)
  int *nframes;           // [n]
  int *step;              // [n]
  int *alive;             // [n]
  float *trailing;        // [n][max_trailing][H]
  int *trailing_rows;     // [n]
  const float *codec_emb; // [vocab][H]
  const float *pred_emb;  // [groups - 1][cp_vocab][H]
  const float *tts_pad;   // [H]
  float *cp_h;            // code-predictor input rows [n][2][H] (then [n][H])
  float *t_h;             // talker input rows [n][H]
  const float *cp_logits; // [n][cp_vocab]
  CtxDev *const *cp_ctx;  // [n]
  // the int8 path over few rows (partial products): the row descriptors and
  // the layer-0 inputs (normed, quantized) of both stacks are written by the
  // kernels that build the rows, the talker length advanced at the frame end,
  // and the code-predictor head left as chunk partials (nullptr / 0: the
  // separate kernels do it)
  RowDesc *cp_rd;          // [2n] rows of the code-predictor step
  RowDesc *t_rd;           // [n]
  CtxDev *const *t_ctx;    // [n]
  int8_t *cp_xq, *t_xq;    // operand tiles of layer 0 of each stack
  int t_fold;              // k_cp_next builds the talker input (int8 both, H <= kArgBlock)
  const float *cp_norm0, *t_norm0;
  float cp_eps, t_eps;
  const float *cp_part;    // head partials [cp_hch][rows][cp_vocab]
  int cp_hch;
  // the choosers (argmax when do_sample == 0) and the sentence seed of each
  // stream (the code predictor's: seed ^ kSubSeedXor)
  SampleParams sp0, sp;
  const uint64_t *seeds;   // [n]
};

constexpr int kArgBlock = 1024;
constexpr int kArgUnroll = 4;  // argmax rounds whose loads are issued together (4096 codes)

// the block's (value, index) argmax; every thread merges the waves' results
// itself (in wave order), so one barrier. Called once per kernel: its LDS is
// not reused.
__device__ int block_argmax(float v, int i) {
  __shared__ float sv[kArgBlock / 64];
  __shared__ int si[kArgBlock / 64];
  for (int off = 32; off >= 1; off >>= 1) {
    const float v2 = __shfl_xor(v, off, 64);
    const int i2 = __shfl_xor(i, off, 64);
    argmax_merge(v, i, v2, i2);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = v;
    si[wave] = i;
  }
  __syncthreads();
  float bv = sv[0];
  int bi = si[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); w++) argmax_merge(bv, bi, sv[w], si[w]);
  return bi;
}

// the descriptor of a row at position pos of context c (pos < 0: inactive)
__device__ __forceinline__ RowDesc row_desc(const CtxDev *c, int pos) {
  c = global_ptr(c);
  RowDesc d;
  d.k = c->k;
  d.v = c->v;
  d.max_pos = c->max_pos;
  d.pos = pos < c->max_pos ? pos : -1;
  return d;
}

// ChooseCode0 + the code-predictor input [past state; codec_emb[code]] and
// the reset of the code-predictor context. One block per stream. The int8
// path: also the descriptors (positions 0, 1) and the quantized layer-0
// inputs of both rows (zeros for a stream that does not run).
template <bool SAMPLE>
__global__ __launch_bounds__(kArgBlock) void k_choose_code0(FrameDev f) {
  __shared__ double red[2][kArgBlock / 64];
  __shared__ std::conditional_t<SAMPLE, SampleShared, char> sh;
  const int s = blockIdx.x, tid = threadIdx.x;
  // the int8 path: this thread's chunks of the norm weights and of the past
  // state (which does not depend on the code) loaded first
  const bool q8 = f.cp_xq != nullptr;
  float w8[8], pv[8], ev[8];
  row_chunk8(q8 ? f.cp_norm0 : nullptr, f.H, w8);
  row_chunk8(q8 ? f.past + (size_t)s * f.H : nullptr, f.H, pv);
  row_chunk8(nullptr, f.H, ev);
  const float *lg = f.logits + (size_t)s * f.vocab;
  const uint8_t *seen = f.seen + (size_t)s * f.vocab;
  // the argmax's loads issued before the alive flag is known (every stream's
  // rows exist): every logit this thread scores and its seen flag, logit 0,
  // the frame count (kArgUnroll rounds unrolled, indices past the vocabulary
  // clamped and not merged; a larger vocabulary continues in a loop)
  float lv[SAMPLE ? 1 : kArgUnroll], l0 = 0.f;
  uint8_t sv[SAMPLE ? 1 : kArgUnroll], s0 = 0;
  if constexpr (!SAMPLE) {
#pragma unroll
    for (int k = 0; k < kArgUnroll; k++) {
      const int i = min(tid + k * kArgBlock, f.vocab - 1);
      lv[k] = lg[i];
      sv[k] = seen[i];
    }
    l0 = lg[0];
    s0 = seen[0];
  }
  const int nf = f.nframes[s];
  int code = -1;
  if (f.alive[s]) {
    // the scores of ChooseCode0's logits processors, of logit v of code i
    // (seen: code i already returned)
    auto score_v = [&](float v, bool sn, int i) {
      // 2048..3071 forbidden but eos; eos forbidden before 2 frames
      if (i >= f.vocab - 1024 && i != f.eos) v = -INFINITY;
      if (i == f.eos && nf < 2) v = -INFINITY;
      // repetition penalty, once per code already returned (not when forbidden)
      if (sn && v != -INFINITY && f.penalty != 1.0f)
        v = v > 0.f ? __fdiv_rn(v, f.penalty) : v * f.penalty;
      return v;
    };
    auto score = [&](int i) { return score_v(lg[i], seen[i] != 0, i); };
    if constexpr (SAMPLE) {
      float x[3];
#pragma unroll
      for (int j = 0; j < 3; j++) {
        const int i = 3 * tid + j;
        x[j] = i < f.vocab ? score(i) : -INFINITY;
      }
      code = block_sample<3>(x, f.vocab, f.sp0, draw_uniform(f.seeds[s], (uint64_t)nf, 0), sh);
    } else {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int k = 0; k < kArgUnroll; k++) {
        const int i = tid + k * kArgBlock;
        if (i < f.vocab) argmax_merge(bv, bi, score_v(lv[k], sv[k] != 0, i), i);
      }
      for (int i = tid + kArgUnroll * kArgBlock; i < f.vocab; i += kArgBlock)
        argmax_merge(bv, bi, score(i), i);
      code = first_max_code(block_argmax(bv, bi), score_v(l0, s0 != 0, 0));
    }
    int *codes = f.codes + (size_t)s * f.groups;
    if (code == f.eos) {
      if (tid < f.groups) codes[tid] = -1;
      __syncthreads();
      if (tid == 0) f.alive[s] = 0;
      code = -1;
    } else {
      if (tid == 0) {
        codes[0] = code;
        f.seen[(size_t)s * f.vocab + code] = 1;
        f.nframes[s] = nf + 1;
        global_ptr(f.cp_ctx[s])->len = 0;
      }
      float *x = f.cp_h + (size_t)s * 2 * f.H;
      const float *past = f.past + (size_t)s * f.H;
      const float *emb = f.codec_emb + (size_t)code * f.H;
      if (q8) {  // the rows from registers (the embedding loaded once)
        row_chunk8(emb, f.H, ev);
        if (tid < (f.H >> 3)) {
          float4 *xp = reinterpret_cast<float4 *>(x) + 2 * tid;
          float4 *xe = reinterpret_cast<float4 *>(x + f.H) + 2 * tid;
          xp[0] = make_float4(pv[0], pv[1], pv[2], pv[3]);
          xp[1] = make_float4(pv[4], pv[5], pv[6], pv[7]);
          xe[0] = make_float4(ev[0], ev[1], ev[2], ev[3]);
          xe[1] = make_float4(ev[4], ev[5], ev[6], ev[7]);
        }
      } else {
        for (int c = tid; c < f.H; c += kArgBlock) {
          x[c] = past[c];
          x[f.H + c] = emb[c];
        }
      }
    }
  }
  if (q8) {
    // both rows quantized (zeros for a stream that does not run), each with
    // its own reduction slots
    const bool live = code >= 0;
    if (tid < 2) f.cp_rd[2 * s + tid] = row_desc(f.cp_ctx[s], live ? tid : -1);
    if (!live)
#pragma unroll
      for (int e = 0; e < 8; e++) pv[e] = 0.f;
    quant_row_regs(pv, w8, live, f.cp_eps, f.H, 2 * s, 2 * f.n, f.cp_xq, red[0]);
    quant_row_regs(ev, w8, live, f.cp_eps, f.H, 2 * s + 1, 2 * f.n, f.cp_xq, red[1]);
  }
}

// the code predictor's draw for code g + 1 of stream s from its logits (a
// row that thread t reads at indices t NPT ..)
template <class Get>
__device__ int cp_draw(Get get, int cp_vocab, const SampleParams &sp, uint64_t seed,
                       int frame, int g, SampleShared &sh) {
  const float u = draw_uniform(seed ^ kSubSeedXor, (uint64_t)frame, (uint64_t)(g + 1));
  if (cp_vocab <= 2 * kArgBlock) {
    float x[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int i = 2 * threadIdx.x + j;
      x[j] = i < cp_vocab ? get(i) : -INFINITY;
    }
    return block_sample<2>(x, cp_vocab, sp, u, sh);
  }
  float x[3];
#pragma unroll
  for (int j = 0; j < 3; j++) {
    const int i = 3 * threadIdx.x + j;
    x[j] = i < cp_vocab ? get(i) : -INFINITY;
  }
  return block_sample<3>(x, cp_vocab, sp, u, sh);
}

// ChooseCode for group g + 1 (argmax of the head-g logits), then the input row
// of the next code-predictor forward: pred_emb[g][code]. One block per stream.
// Plain scalar arguments (preloaded into SGPRs).
__global__ __launch_bounds__(kArgBlock) void k_cp_argmax(const float *__restrict__ cp_logits,
                                                         const int *__restrict__ alive,
                                                         const float *__restrict__ pred_emb,
                                                         float *__restrict__ cp_h,
                                                         int *__restrict__ codes, int cp_vocab,
                                                         int groups, int H, int g) {
  const int s = blockIdx.x, tid = threadIdx.x;
  if (!alive[s]) return;
  const float *lg = cp_logits + (size_t)s * cp_vocab;
  // every logit this thread merges, and logit 0, loaded before the first merge
  float lv[kArgUnroll];
#pragma unroll
  for (int k = 0; k < kArgUnroll; k++) lv[k] = lg[min(tid + k * kArgBlock, cp_vocab - 1)];
  const float l0 = lg[0];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int k = 0; k < kArgUnroll; k++)
    if (tid + k * kArgBlock < cp_vocab) argmax_merge(bv, bi, lv[k], tid + k * kArgBlock);
  for (int i = tid + kArgUnroll * kArgBlock; i < cp_vocab; i += kArgBlock)
    argmax_merge(bv, bi, lg[i], i);
  const int code = first_max_code(block_argmax(bv, bi), l0);
  if (tid == 0) codes[(size_t)s * groups + g + 1] = code;
  if (g + 1 < groups - 1) {
    const float *emb = pred_emb + ((size_t)g * cp_vocab + code) * H;
    float *x = cp_h + (size_t)s * H;
    for (int c = tid; c < H; c += kArgBlock) x[c] = emb[c];
  }
}

// k_cp_argmax with the sub-sampler's draw (the code predictor's sampling)
__global__ __launch_bounds__(kArgBlock) void k_cp_sample(const float *__restrict__ cp_logits,
                                                         const int *__restrict__ alive,
                                                         const float *__restrict__ pred_emb,
                                                         float *__restrict__ cp_h,
                                                         int *__restrict__ codes, int cp_vocab,
                                                         int groups, int H, int g,
                                                         SampleParams sp,
                                                         const uint64_t *__restrict__ seeds,
                                                         const int *__restrict__ nframes) {
  __shared__ SampleShared sh;
  const int s = blockIdx.x, tid = threadIdx.x;
  if (!alive[s]) return;
  const float *lg = cp_logits + (size_t)s * cp_vocab;
  const int code =
      cp_draw([&](int i) { return lg[i]; }, cp_vocab, sp, seeds[s], nframes[s] - 1, g, sh);
  if (tid == 0) codes[(size_t)s * groups + g + 1] = code;
  if (g + 1 < groups - 1) {
    const float *emb = pred_emb + ((size_t)g * cp_vocab + code) * H;
    float *x = cp_h + (size_t)s * H;
    for (int c = tid; c < H; c += kArgBlock) x[c] = emb[c];
  }
}

// the end of a step for stream s (k_frame_end's work, by one workgroup): its
// codes (code `code` at index `last`, the others from f.codes) and alive flag
// into the host's pinned copy (system-scope stores: in host memory when the
// kernel ends); a running stream's frame count and talker context length
// advanced
__device__ __forceinline__ void frame_end_stream(const FrameDev &f, int s, bool alive, int last,
                                                 int code) {
  const int t = threadIdx.x;
  if (t < f.groups) {
    const size_t i = (size_t)s * f.groups + t;
    __hip_atomic_store(f.host_codes + i, t == last ? code : f.codes[i], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
  }
  if (t == 0) {
    __hip_atomic_store(f.host_alive + s, alive ? 1 : 0, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
    if (alive) {
      f.step[s] += 1;
      CtxDev *c = global_ptr(f.t_ctx[s]);  // the talker context took the step's row
      c->len = min(c->len + 1, c->max_pos);
    }
  }
}

// the last term of stream s's next talker input: its trailing text row for
// this step, or tts_pad past them
__device__ __forceinline__ const float *talker_tail(const FrameDev &f, int s) {
  const int st = f.step[s];
  return st < f.trailing_rows[s] ? f.trailing + ((size_t)s * f.max_trailing + st) * f.H
                                 : f.tts_pad;
}

// The int8 path's k_cp_argmax: the head-g logits as the sum of the head's
// chunk partials in chunk order (row R s + R - 1 of the step's R n rows),
// ChooseCode for group g + 1, then the next step's input row pred_emb[g][code]
// (to cp_h), its descriptor (position g + 2) and its quantized layer-0 input.
// FOLD (the last group's launch with t_fold: int8 talker, H <= kArgBlock; the
// argmax variant, the sampler's registers leaving no room) also
// builds the next talker input (k_talker_input_q's work): thread c loads
// element c of every row whose code is known (codes 0 .. g) and of the tail
// before the argmax, adds the new code's row after it, in talker_input_elem's
// order, and writes the row, its descriptor and its quantized layer-0 input;
// and it does the stream's part of k_frame_end (the talker layers read the
// row's descriptor, not the context length).
template <bool SAMPLE, bool FOLD>
__global__ __launch_bounds__(kArgBlock) void k_cp_next(FrameDev f, int g) {
  static_assert(!(SAMPLE && FOLD), "the talker input is folded into the argmax variant");
  __shared__ double red[kArgBlock / 64];
  __shared__ std::conditional_t<SAMPLE, SampleShared, char> sh_cp;
  const int s = blockIdx.x, tid = threadIdx.x;
  const bool next = g + 1 < f.groups - 1;
  const int R = g == 0 ? 2 : 1, rows = R * f.n, row = R * s + R - 1;
  // the head's logit i: the chunk partials (cp_hch <= kPartialSlots) loaded
  // together, added in chunk order
  constexpr int NPS = kPartialSlots;
  auto logit = [&](int i) {
    float p4[NPS];
#pragma unroll
    for (int c = 0; c < NPS; c++)
      p4[c] = f.cp_part[((size_t)min(c, f.cp_hch - 1) * rows + row) * f.cp_vocab + i];
    float v = 0.f;
#pragma unroll
    for (int c = 0; c < NPS; c++) v = c < f.cp_hch ? __fadd_rn(v, p4[c]) : v;
    return v;
  };
  auto chunk_sum = [&](const float(&p4)[NPS]) {
    float v = 0.f;
#pragma unroll
    for (int c = 0; c < NPS; c++) v = c < f.cp_hch ? __fadd_rn(v, p4[c]) : v;
    return v;
  };
  // issued before the stream's alive flag is known (the rows exist for every
  // stream): this thread's chunk of the next input's norm weights and, for
  // the argmax, every partial of the logits it merges and of logit 0
  float w8[8];
  row_chunk8(next ? f.cp_norm0 : nullptr, f.H, w8);
  // the last group with t_fold: the talker's norm weights, and element tid of
  // the tail and of the rows of codes 0 .. g (clamped codes: a stream that
  // does not run loads valid rows it does not use)
  __shared__ float xs[FOLD ? kArgBlock : 1];
  constexpr bool fold = FOLD;
  constexpr int G = FOLD ? 16 : 1;  // the most groups a frame takes
  float tw8[8], te[G], tl = 0.f;
  row_chunk8(fold ? f.t_norm0 : nullptr, f.H, tw8);
  if constexpr (FOLD) {
    const int *cd = f.codes + (size_t)s * f.groups;
    const int c = min(tid, f.H - 1);
#pragma unroll
    for (int j = 0; j < G; j++) {
      const int cj = j <= g ? max(cd[j], 0) : 0;
      te[j] = j == 0 ? f.codec_emb[(size_t)cj * f.H + c]
              : j <= g ? f.pred_emb[((size_t)(j - 1) * f.cp_vocab + cj) * f.H + c]
                       : 0.f;
    }
    tl = talker_tail(f, s)[c];
  }
  float pl[SAMPLE ? 1 : kArgUnroll][NPS], p0[NPS];
  if constexpr (!SAMPLE) {
#pragma unroll
    for (int k = 0; k < kArgUnroll; k++) {
      const int i = min(tid + k * kArgBlock, f.cp_vocab - 1);
#pragma unroll
      for (int c = 0; c < NPS; c++)
        pl[k][c] = f.cp_part[((size_t)min(c, f.cp_hch - 1) * rows + row) * f.cp_vocab + i];
    }
#pragma unroll
    for (int c = 0; c < NPS; c++)
      p0[c] = f.cp_part[((size_t)min(c, f.cp_hch - 1) * rows + row) * f.cp_vocab];
  }
  if (!f.alive[s]) {
    if (next) {
      if (tid == 0) f.cp_rd[s] = row_desc(f.cp_ctx[s], -1);
      quant_row_block(nullptr, nullptr, 0.f, f.H, s, f.n, f.cp_xq, red);
    }
    if constexpr (FOLD) {  // the talker row does not run: zero blocks
      if (tid == 0) f.t_rd[s] = row_desc(f.t_ctx[s], -1);
      quant_row_block(nullptr, nullptr, 0.f, f.H, s, f.n, f.t_xq, red);
      frame_end_stream(f, s, false, -1, 0);
    }
    return;
  }
  // the next rows' descriptors do not depend on the code (the talker row's
  // position: the context length)
  if (next && tid == 0) f.cp_rd[s] = row_desc(f.cp_ctx[s], g + 2);
  if (fold && tid == 0) f.t_rd[s] = row_desc(f.t_ctx[s], global_ptr(f.t_ctx[s])->len);
  int code;
  if constexpr (SAMPLE) {
    code = cp_draw(logit, f.cp_vocab, f.sp, f.seeds[s], f.nframes[s] - 1, g, sh_cp);
  } else {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int k = 0; k < kArgUnroll; k++) {
      const int i = tid + k * kArgBlock;
      if (i < f.cp_vocab) argmax_merge(bv, bi, chunk_sum(pl[k]), i);
    }
    for (int i = tid + kArgUnroll * kArgBlock; i < f.cp_vocab; i += kArgBlock)
      argmax_merge(bv, bi, logit(i), i);
    code = first_max_code(block_argmax(bv, bi), chunk_sum(p0));
  }
  if (tid == 0) f.codes[(size_t)s * f.groups + g + 1] = code;
  const float *emb = f.pred_emb + ((size_t)g * f.cp_vocab + code) * f.H;
  if (next) {
    // the input row pred_emb[g][code], loaded once: to cp_h and quantized
    float v[8];
    row_chunk8(emb, f.H, v);
    if (tid < (f.H >> 3)) {
      float4 *x = reinterpret_cast<float4 *>(f.cp_h + (size_t)s * f.H) + 2 * tid;
      x[0] = make_float4(v[0], v[1], v[2], v[3]);
      x[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
    quant_row_regs(v, w8, true, f.cp_eps, f.H, s, f.n, f.cp_xq, red);
  }
  if constexpr (FOLD) {
    // the next talker input: codec_emb[code 0] + pred_emb[j - 1][code j] for
    // j = 1 .. g + 1 + the tail, added in that order
    const int c = tid;
    if (c < f.H) {
      float x = te[0];
#pragma unroll
      for (int j = 1; j < G; j++)
        if (j <= g) x = x + te[j];
      x = x + emb[c];
      x = x + tl;
      f.t_h[(size_t)s * f.H + c] = x;
      xs[c] = x;
    }
    __syncthreads();
    float v[8];
    row_chunk8(xs, f.H, v);
    quant_row_regs(v, tw8, true, f.t_eps, f.H, s, f.n, f.t_xq, red);
    // after the barrier: every thread has read the frame count (the tail) and
    // thread 0 the context length (the descriptor)
    frame_end_stream(f, s, true, g + 1, code);
  }
}

// element c of stream s's next talker input: codec_emb[code 0] +
// pred_emb[g - 1][code g] for g = 1 .. groups - 1 + (trailing[step] or
// tts_pad), added in that order. The codes (at most 16) are read first and
// every row's element is loaded before the first add, so the sum waits for
// one round of loads instead of one per group.
__device__ __forceinline__ float talker_input_elem(const FrameDev &f, int s, int c) {
  constexpr int G = 16;  // the most groups a frame takes
  const int *codes = f.codes + (size_t)s * f.groups;
  const float *tail = talker_tail(f, s);
  int code[G];
#pragma unroll
  for (int g = 0; g < G; g++) code[g] = g < f.groups ? codes[g] : 0;
  float e[G];
#pragma unroll
  for (int g = 0; g < G; g++)
    e[g] = g == 0 ? f.codec_emb[(size_t)code[0] * f.H + c]
           : g < f.groups ? f.pred_emb[((size_t)(g - 1) * f.cp_vocab + code[g]) * f.H + c]
                          : 0.f;
  const float t = tail[c];
  float x = e[0];
#pragma unroll
  for (int g = 1; g < G; g++)
    if (g < f.groups) x = x + e[g];
  return x + t;
}

__global__ void k_talker_input(FrameDev f) {
  const int s = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  // the row's descriptor: position = the context length (inactive: -1)
  if (c == 0) f.t_rd[s] = row_desc(f.t_ctx[s], f.alive[s] ? global_ptr(f.t_ctx[s])->len : -1);
  if (c >= f.H || !f.alive[s]) return;
  const float x = talker_input_elem(f, s, c);
  f.t_h[(size_t)s * f.H + c] = x;
}

// k_cp_argmax of the last group (g + 1 == groups - 1) with k_talker_input's
// and k_frame_end's work (greedy, f32 activations, H <= kArgBlock; one block
// per stream): the argmax, then element tid of the next talker input (the
// rows of codes 0 .. g and the tail loaded before the argmax, the new code's
// row after it, added in talker_input_elem's order), the row's descriptor and
// the stream's end of the step. The talker layers read the descriptor, not
// the context length.
__global__ __launch_bounds__(kArgBlock) void k_cp_argmax_end(FrameDev f, int g) {
  const int s = blockIdx.x, tid = threadIdx.x;
  const float *lg = f.cp_logits + (size_t)s * f.cp_vocab;
  // the argmax's loads (every logit this thread merges, and logit 0), then
  // element tid of the rows of the codes already chosen and of the tail
  // (clamped codes: a stream that does not run loads valid rows it does not use)
  float lv[kArgUnroll];
#pragma unroll
  for (int k = 0; k < kArgUnroll; k++) lv[k] = lg[min(tid + k * kArgBlock, f.cp_vocab - 1)];
  const float l0 = lg[0];
  constexpr int G = 16;  // the most groups a frame takes
  const int *cd = f.codes + (size_t)s * f.groups;
  const int c = min(tid, f.H - 1);
  float te[G];
#pragma unroll
  for (int j = 0; j < G; j++) {
    const int cj = j <= g ? max(cd[j], 0) : 0;
    te[j] = j == 0 ? f.codec_emb[(size_t)cj * f.H + c]
            : j <= g ? f.pred_emb[((size_t)(j - 1) * f.cp_vocab + cj) * f.H + c]
                     : 0.f;
  }
  const float tl = talker_tail(f, s)[c];
  if (!f.alive[s]) {
    if (tid == 0) f.t_rd[s] = row_desc(f.t_ctx[s], -1);
    frame_end_stream(f, s, false, -1, 0);
    return;
  }
  if (tid == 0) f.t_rd[s] = row_desc(f.t_ctx[s], global_ptr(f.t_ctx[s])->len);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int k = 0; k < kArgUnroll; k++)
    if (tid + k * kArgBlock < f.cp_vocab) argmax_merge(bv, bi, lv[k], tid + k * kArgBlock);
  for (int i = tid + kArgUnroll * kArgBlock; i < f.cp_vocab; i += kArgBlock)
    argmax_merge(bv, bi, lg[i], i);
  const int code = first_max_code(block_argmax(bv, bi), l0);
  if (tid == 0) f.codes[(size_t)s * f.groups + g + 1] = code;
  if (tid < f.H) {
    float x = te[0];
#pragma unroll
    for (int j = 1; j < G; j++)
      if (j <= g) x = x + te[j];
    x = x + f.pred_emb[((size_t)g * f.cp_vocab + code) * f.H + tid];
    x = x + tl;
    f.t_h[(size_t)s * f.H + tid] = x;
  }
  // every thread has read the frame count (the tail), thread 0 the length
  __syncthreads();
  frame_end_stream(f, s, true, g + 1, code);
}

// The int8 path's k_talker_input: one block per stream, the row also kept in
// LDS for its descriptor (position = the context length) and its quantized
// layer-0 input (H <= 4096).
__global__ __launch_bounds__(kArgBlock) void k_talker_input_q(FrameDev f) {
  __shared__ double red[kArgBlock / 64];
  __shared__ float xs[4096];
  const int s = blockIdx.x, tid = threadIdx.x;
  float w8[8];  // this thread's chunk of the norm weights, loaded first
  row_chunk8(f.t_norm0, f.H, w8);
  if (!f.alive[s]) {
    if (tid == 0) f.t_rd[s] = row_desc(f.t_ctx[s], -1);
    quant_row_block(nullptr, nullptr, 0.f, f.H, s, f.n, f.t_xq, red);
    return;
  }
  for (int c = tid; c < f.H; c += kArgBlock) {
    const float x = talker_input_elem(f, s, c);
    f.t_h[(size_t)s * f.H + c] = x;
    xs[c] = x;
  }
  if (tid == 0) f.t_rd[s] = row_desc(f.t_ctx[s], global_ptr(f.t_ctx[s])->len);
  __syncthreads();
  float v[8];
  row_chunk8(xs, f.H, v);
  quant_row_regs(v, w8, true, f.t_eps, f.H, s, f.n, f.t_xq, red);
}

// The rows of a device-side Start (TQwenTalker.Start, talker.pas:536-573):
// row i = proj[plan[i].x] (+ codec_emb[plan[i].y] when plan[i].y >= 0, the
// AddRow of talker.pas:423-429, added in that order); rows 0 .. rows - 1 go
// to the prefill, the next ones to the stream's trailing rows.
__global__ __launch_bounds__(256) void k_start_rows(const int2 *__restrict__ plan, int rows,
                                                    const float *__restrict__ proj,
                                                    const float *__restrict__ codec_emb, int H,
                                                    float *__restrict__ prefill,
                                                    float *__restrict__ trailing) {
  const int i = blockIdx.x;
  const int2 p = plan[i];
  const float *src = proj + (size_t)p.x * H;
  const float *add = p.y >= 0 ? codec_emb + (size_t)p.y * H : nullptr;
  float *dst = i < rows ? prefill + (size_t)i * H : trailing + (size_t)(i - rows) * H;
  for (int c = threadIdx.x; c < H; c += 256) dst[c] = add ? src[c] + add[c] : src[c];
}

// the end of a step: the frame count and the talker context length of every
// running stream, and every stream's codes and alive flag into the host's
// pinned copy (system-scope stores: in host memory when the kernel ends)
__global__ void k_frame_end(FrameDev f) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < f.n) {  // stream i
    const int a = f.alive[i];
    if (a) {
      f.step[i] += 1;
      CtxDev *c = global_ptr(f.t_ctx[i]);  // the talker context took the step's row
      c->len = min(c->len + 1, c->max_pos);
    }
    __hip_atomic_store(f.host_alive + i, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  // code i of the slice's [n][groups] (consecutive threads, consecutive words)
  if (i < f.n * f.groups)
    __hip_atomic_store(f.host_codes + i, f.codes[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace q3h

using namespace q3h;

// A slice of a frame's streams (first .. first + n - 1) with its own work
// buffers, HIP stream and captured step. The slices of one frame run their
// steps concurrently: every kernel of the batched step is latency-bound, so
// two chains of them on two queues overlap where one chain waits. Each
// stream's arithmetic does not depend on the other rows of its products, so
// the codes do not depend on the slicing.
struct FrameSlice {
  int first = 0, n = 0;
  Work tw, cw;
  FrameDev fd{};  // the view of the slice's streams
  hipStream_t stream = nullptr;
  // the captured steps, by the attention positions each covers (ascending)
  std::vector<std::pair<int, hipGraphExec_t>> graphs;
};

struct q3h_frame {
  q3h_stack *talker = nullptr, *cp = nullptr;
  q3h_frame_config cfg{};
  int H = 0;
  std::vector<q3h_context *> tctx, cctx;
  CtxDev **t_arr = nullptr, **c_arr = nullptr;
  FrameDev fd{};  // every stream: the state arrays the slices view
  std::vector<FrameSlice> slices;
  float *codec_emb = nullptr, *pred_emb = nullptr, *tts_pad = nullptr;
  std::vector<int> started, host_len, max_trailing_rows;
  int32_t *pinned = nullptr;  // [n][groups] codes + [n] alive
  std::vector<void *> allocs;
  // the choosers (TQwenTalker.Sampling) and the source of sentence seeds when
  // its seed is 0 (a fresh one per Start, talker.pas:582-584)
  q3h_sampling sampling{};
  std::mt19937_64 seed_rng{std::random_device{}()};
  // device-side Start: the row plan and the projected rows
  int start_cap = 0;
  int2 *start_plan = nullptr;  // [start_cap]
  float *start_proj = nullptr; // [start_cap][H]
};

namespace {

void drop_graphs(q3h_frame *f) {
  for (FrameSlice &sl : f->slices) {
    for (auto &g : sl.graphs) (void)hipGraphExecDestroy(g.second);
    sl.graphs.clear();
  }
}

// every slice's work done (the frame's state may be read or changed)
void sync_slices(q3h_frame *f) {
  for (FrameSlice &sl : f->slices) check_hip(hipStreamSynchronize(sl.stream), "frame sync");
}

void frame_release(q3h_frame *f) {
  for (FrameSlice &sl : f->slices)
    if (sl.stream) (void)hipStreamSynchronize(sl.stream);
  drop_graphs(f);
  for (auto *c : f->tctx) {
    c->s->contexts--;
    free_context(c);
  }
  for (auto *c : f->cctx) {
    c->s->contexts--;
    free_context(c);
  }
  for (FrameSlice &sl : f->slices) {
    sl.tw.release();
    sl.cw.release();
    if (sl.stream) (void)hipStreamDestroy(sl.stream);
  }
  for (void *p : f->allocs) dev_free(p);
  dev_free(f->start_plan);
  dev_free(f->start_proj);
  if (f->pinned) (void)hipHostFree(f->pinned);
}

// The view of streams first .. first + n - 1 of the frame's state, with the
// slice's work buffers (the int8 path's folded inputs when `partial`).
FrameDev slice_view(const q3h_frame *f, FrameSlice &sl, bool cp_partial, bool t_partial) {
  const q3h_frame_config &c = f->cfg;
  const size_t first = sl.first, H = f->H;
  FrameDev d = f->fd;
  d.n = sl.n;
  d.logits += first * c.vocab;
  d.past += first * H;
  d.codes += first * c.groups;
  d.host_codes = f->pinned + first * c.groups;
  d.host_alive = f->pinned + (size_t)c.n_streams * c.groups + first;
  d.seen += first * c.vocab;
  d.nframes += first;
  d.step += first;
  d.alive += first;
  d.trailing += first * c.max_frames * H;
  d.trailing_rows += first;
  d.seeds += first;
  d.cp_h = sl.cw.h;
  d.t_h = sl.tw.h;
  d.cp_logits = sl.cw.logits;
  d.cp_ctx = f->c_arr + first;
  d.cp_rd = sl.cw.rd;
  d.t_rd = sl.tw.rd;
  d.t_ctx = f->t_arr + first;
  d.cp_xq = nullptr;
  d.cp_part = nullptr;
  d.cp_hch = 0;
  d.t_xq = nullptr;
  if (cp_partial) {
    d.cp_xq = sl.cw.xa.q;
    d.cp_norm0 = f->cp->layers[0].in_norm;
    d.cp_eps = f->cp->cfg.rms_eps;
    d.cp_part = sl.cw.gpart;
    d.cp_hch = gemm_i8_chunks(f->H);
  }
  if (t_partial) {
    d.t_xq = sl.tw.xa.q;
    d.t_norm0 = f->talker->layers[0].in_norm;
    d.t_eps = f->talker->cfg.rms_eps;
  }
  d.t_fold = cp_partial && t_partial && f->H <= kArgBlock;
  return d;
}

// the views of every slice, again after the frame-wide parameters changed
// (the captured steps hold them as kernel arguments: captured again)
void refresh_slices(q3h_frame *f) {
  const q3h_frame_config &c = f->cfg;
  int nmax = 0;
  for (const FrameSlice &sl : f->slices) nmax = std::max(nmax, sl.n);
  const bool cp_partial =
      partial_path(f->cp, 2 * nmax) && f->cp->heads[c.cp_heads[0]].N % 16 == 0;
  const bool t_partial = partial_path(f->talker, nmax) && f->H <= 4096;
  for (FrameSlice &sl : f->slices) sl.fd = slice_view(f, sl, cp_partial, t_partial);
  drop_graphs(f);
}

// The number of slices of a frame of n streams: on the int8 path one slice
// per 32 streams (its products take each 16-row tile as workgroups of their
// own, so a slice of 32 streams costs a 16-stream slice's launches; at 16,
// 24 and 32 streams one slice is 6 %, 1.5 % and 0.3 % faster than two, and the
// code predictor's first step keeps at most 64 rows per slice), one
// otherwise. Q3H_FRAME_SLICES (1..4) overrides it, for measurements.
int slice_count(const q3h_stack *talker, int n) {
  if (const char *e = std::getenv("Q3H_FRAME_SLICES")) {
    const int v = std::atoi(e);
    if (v >= 1 && v <= 4) return std::min(v, n);
  }
  return partial_path(talker, n) ? (n + 31) / 32 : 1;
}

template <class T>
T *falloc(q3h_frame *f, size_t n) {
  T *p = (T *)dev_alloc(sizeof(T) * (n ? n : 1));
  f->allocs.push_back(p);
  return p;
}

// The step's kernel sequence of slice sl on stream st (captured into the
// slice's graph).
void enqueue_step(q3h_frame *f, FrameSlice &sl, int positions, hipStream_t st) {
  const q3h_frame_config &c = f->cfg;
  const int n = sl.n, H = f->H;
  q3h_stack *cp = f->cp, *tk = f->talker;
  const FrameDev fd = sl.fd;
  Work &cw = sl.cw, &tw = sl.tw;
  CtxDev **c_arr = f->c_arr + sl.first;
  q3h_context *cctx0 = f->cctx[sl.first];
  const bool cq = fd.cp_xq != nullptr, tq = fd.t_xq != nullptr;  // the folded int8 paths
  // the last code-predictor argmax builds the talker input and ends the step
  // (int8: k_cp_next<false, true>; f32 activations: k_cp_argmax_end)
  const bool fold_tail = cq && fd.t_fold && !fd.sp.do_sample;
  const bool fold_end = !cq && !tq && !fd.sp.do_sample && H <= kArgBlock;
  if (fd.sp0.do_sample)
    hipLaunchKernelGGL(k_choose_code0<true>, dim3(n), dim3(kArgBlock), 0, st, fd);
  else
    hipLaunchKernelGGL(k_choose_code0<false>, dim3(n), dim3(kArgBlock), 0, st, fd);
  // code predictor: 2 rows per stream, then one row per group
  // one stream on the Qwen3-TTS shapes: step 0 runs the fused two-row path,
  // steps 1.. the fused single-row path (positions are fixed: step g adds
  // position g + 1)
  const bool fused = n == 1 && cp_fused_supported(cp->cfg) && cctx0->max_pos == 16;
  // greedy on that path: the argmax of head g and the next input row are taken
  // by the first product of forward g + 1 (one launch fewer per group)
  const bool code_in_product =
      fused && !fd.sp.do_sample && (c.cp_vocab == 2048 || c.cp_vocab == 3072);
  for (int g = 0; g < c.groups - 1; g++) {
    const int R = g == 0 ? 2 : 1;
    if (cq) {
      // inputs and descriptors written by k_choose_code0 / k_cp_next; the
      // last layer's residual kernel applies the final norm and quantizes the
      // head input; k_cp_next adds the head's chunk partials
      LayerIO io;
      io.input_quantized = true;
      io.final_norm = cp->final_norm;
      io.row_pairs = R == 2;  // rows 2s, 2s + 1: positions 0, 1 of stream s
      run_layers(cp, cw, n * R, c.groups, R == 1, st, io);
      launch_gemm_i8_partial(cp->heads[c.cp_heads[g]], cw.xa, n * R, cw.gpart, st);
      if (fd.sp.do_sample)
        hipLaunchKernelGGL((k_cp_next<true, false>), dim3(n), dim3(kArgBlock), 0, st, fd, g);
      else if (fold_tail && g + 1 == c.groups - 1)  // the last group: + the talker input
        hipLaunchKernelGGL((k_cp_next<false, true>), dim3(n), dim3(kArgBlock), 0, st, fd, g);
      else
        hipLaunchKernelGGL((k_cp_next<false, false>), dim3(n), dim3(kArgBlock), 0, st, fd, g);
      continue;
    }
    if (fused && g == 0) {
      run_cp_fused_first(cp, cw, cctx0, st);
    } else if (fused) {
      const CodeSrc src{fd.cp_logits, fd.cp_vocab,
                        fd.pred_emb + (size_t)(g - 1) * fd.cp_vocab * H, fd.codes + g, fd.alive};
      run_cp_fused(cp, cw, cctx0, g + 1, st, code_in_product ? &src : nullptr);
    } else {
      launch_prep(c_arr, fd.alive, n, R, cw.rd, st);
      run_layers(cp, cw, n * R, c.groups, R == 1, st);
      launch_advance(c_arr, fd.alive, n, R, st);
    }
    // final norm of each stream's last row + head g, one launch
    linear(cp, cw, cp->heads[c.cp_heads[g]], cw.h + (size_t)(R - 1) * H, R * H, n,
           cp->final_norm, cw.logits, c.cp_vocab, EPI_STORE, nullptr, st);
    if (fd.sp.do_sample)
      hipLaunchKernelGGL(k_cp_sample, dim3(n), dim3(kArgBlock), 0, st, fd.cp_logits, fd.alive,
                         fd.pred_emb, fd.cp_h, fd.codes, fd.cp_vocab, fd.groups, fd.H, g, fd.sp,
                         fd.seeds, (const int *)fd.nframes);
    else if (fold_end && g + 1 == c.groups - 1)
      hipLaunchKernelGGL(k_cp_argmax_end, dim3(n), dim3(kArgBlock), 0, st, fd, g);
    else if (!code_in_product || g + 1 == c.groups - 1)
      hipLaunchKernelGGL(k_cp_argmax, dim3(n), dim3(kArgBlock), 0, st, fd.cp_logits, fd.alive,
                         fd.pred_emb, fd.cp_h, fd.codes, fd.cp_vocab, fd.groups, fd.H, g);
  }
  // the talker
  const Mat &th = tk->heads[c.talker_head];
  if (tq) {
    // the last layer's residual kernel applies the final norm (the normed
    // state to past) and quantizes the head input
    // with t_fold the last (argmax) k_cp_next built the talker input
    if (!fold_tail) hipLaunchKernelGGL(k_talker_input_q, dim3(n), dim3(kArgBlock), 0, st, fd);
    LayerIO io;
    io.input_quantized = true;
    io.final_norm = tk->final_norm;
    io.final_normed = fd.past;
    run_layers(tk, tw, n, positions, true, st, io);
    launch_gemm_i8(th, tw.xa, n, EPI_STORE, fd.logits, c.vocab, st);
  } else {
    if (!fold_end)
      hipLaunchKernelGGL(k_talker_input, dim3((H + 255) / 256, n), dim3(256), 0, st, fd);
    run_layers(tk, tw, n, positions, true, st);
    if (n == 1) {  // final norm fused into the head, the normed state written alongside
      linear(tk, tw, th, tw.h, H, 1, tk->final_norm, fd.logits, c.vocab, EPI_STORE, fd.past,
             st);
    } else {
      launch_rmsnorm_rows(tw.h, H, n, H, tk->final_norm, tk->cfg.rms_eps, fd.past, H, st);
      linear(tk, tw, th, fd.past, H, n, nullptr, fd.logits, c.vocab, EPI_STORE, nullptr, st);
    }
  }
  if (!fold_tail && !fold_end)
    hipLaunchKernelGGL(k_frame_end, dim3((n * c.groups + 63) / 64), dim3(64), 0, st, fd);
}

}  // namespace

extern "C" int q3h_frame_create(q3h_stack *talker, q3h_stack *cp, const q3h_frame_config *cfg,
                                const float *codec_emb, const float *const *pred_emb,
                                const float *tts_pad, q3h_frame **out) {
  q3h_frame *f = nullptr;
  int rc = guard([&] {
    require(talker && cp && cfg && codec_emb && pred_emb && tts_pad && out, Q3H_E_ARG,
            "q3h_frame_create: NULL argument");
    *out = nullptr;
    const q3h_frame_config &c = *cfg;
    require(talker->dev == cp->dev, Q3H_E_ARG, "q3h_frame_create: stacks on different devices");
    require(talker->cfg.hidden == cp->cfg.hidden, Q3H_E_ARG,
            "q3h_frame_create: talker and code predictor widths differ");
    require(c.n_streams >= 1 && c.n_streams <= 64, Q3H_E_ARG,
            "q3h_frame_create: n_streams must be in [1, 64]");
    require(c.groups >= 2 && c.groups <= 16, Q3H_E_ARG, "q3h_frame_create: groups in [2, 16]");
    require(c.vocab > 1024 && c.cp_vocab > 0, Q3H_E_ARG, "q3h_frame_create: bad vocab sizes");
    require(c.eos < c.vocab, Q3H_E_ARG, "q3h_frame_create: eos beyond the vocab");
    require(c.max_frames > 0, Q3H_E_ARG, "q3h_frame_create: max_frames <= 0");
    require(c.talker_head >= 0 && c.talker_head < (int)talker->heads.size() &&
                talker->heads[c.talker_head].N == c.vocab,
            Q3H_E_ARG, "q3h_frame_create: bad talker head");
    for (int g = 0; g < c.groups - 1; g++) {
      require(pred_emb[g] != nullptr, Q3H_E_ARG, "q3h_frame_create: NULL pred_emb");
      require(c.cp_heads[g] >= 0 && c.cp_heads[g] < (int)cp->heads.size() &&
                  cp->heads[c.cp_heads[g]].N == c.cp_vocab,
              Q3H_E_ARG, "q3h_frame_create: bad code-predictor head");
    }
    require(c.max_positions > 0 && c.max_positions <= talker->cfg.max_positions, Q3H_E_ARG,
            "q3h_frame_create: max_positions beyond the talker stack");
    require(cp->cfg.max_positions >= c.groups, Q3H_E_ARG,
            "q3h_frame_create: the code predictor needs groups positions");
    check_hip(hipSetDevice(talker->dev->ordinal), "hipSetDevice");
    f = new q3h_frame();
    f->talker = talker;
    f->cp = cp;
    f->cfg = c;
    const int n = c.n_streams, H = talker->cfg.hidden;
    f->H = H;
    for (int s = 0; s < n; s++) {
      f->tctx.push_back(new_context(talker, c.max_positions));
      f->cctx.push_back(new_context(cp, c.groups));
    }
    f->t_arr = falloc<CtxDev *>(f, n);
    f->c_arr = falloc<CtxDev *>(f, n);
    std::vector<CtxDev *> ta(n), ca(n);
    for (int s = 0; s < n; s++) {
      ta[s] = f->tctx[s]->dev;
      ca[s] = f->cctx[s]->dev;
    }
    check_hip(hipMemcpy(f->t_arr, ta.data(), sizeof(CtxDev *) * n, hipMemcpyHostToDevice),
              "frame init");
    check_hip(hipMemcpy(f->c_arr, ca.data(), sizeof(CtxDev *) * n, hipMemcpyHostToDevice),
              "frame init");
    // the slices: consecutive runs of streams, the first ones one longer
    const int ns = slice_count(talker, n);
    f->slices.resize(ns);
    for (int k = 0, first = 0; k < ns; k++) {
      FrameSlice &sl = f->slices[k];
      sl.first = first;
      sl.n = n / ns + (k < n % ns ? 1 : 0);
      first += sl.n;
      check_hip(hipStreamCreateWithFlags(&sl.stream, hipStreamNonBlocking), "hipStreamCreate");
      sl.tw.ensure(talker, sl.n, attention_splits_upto(talker, c.max_positions), c.vocab);
      sl.cw.ensure(cp, 2 * sl.n, 1, c.cp_vocab);
    }
    f->codec_emb = falloc<float>(f, (size_t)c.vocab * H);
    check_hip(hipMemcpy(f->codec_emb, codec_emb, sizeof(float) * c.vocab * H,
                        hipMemcpyHostToDevice),
              "upload codec_emb");
    f->pred_emb = falloc<float>(f, (size_t)(c.groups - 1) * c.cp_vocab * H);
    for (int g = 0; g < c.groups - 1; g++)
      check_hip(hipMemcpy(f->pred_emb + (size_t)g * c.cp_vocab * H, pred_emb[g],
                          sizeof(float) * c.cp_vocab * H, hipMemcpyHostToDevice),
                "upload pred_emb");
    f->tts_pad = falloc<float>(f, H);
    check_hip(hipMemcpy(f->tts_pad, tts_pad, sizeof(float) * H, hipMemcpyHostToDevice),
              "upload tts_pad");
    FrameDev &d = f->fd;
    d.n = n;
    d.H = H;
    d.vocab = c.vocab;
    d.cp_vocab = c.cp_vocab;
    d.groups = c.groups;
    d.eos = c.eos;
    d.penalty = c.repetition_penalty;
    d.max_trailing = c.max_frames;
    d.logits = falloc<float>(f, (size_t)n * c.vocab);
    d.past = falloc<float>(f, (size_t)n * H);
    // codes [n][groups] then alive [n]: one download per step
    d.codes = falloc<int>(f, (size_t)n * (c.groups + 1));
    d.seen = falloc<uint8_t>(f, (size_t)n * c.vocab);
    d.seeds = falloc<uint64_t>(f, n);
    d.sp0 = d.sp = SampleParams{0, 1.0f, 0, 1.0f};  // greedy until q3h_frame_set_sampling
    f->sampling.temperature = f->sampling.sub_temperature = 1.0f;
    f->sampling.top_p = f->sampling.sub_top_p = 1.0f;
    d.nframes = falloc<int>(f, n);
    d.step = falloc<int>(f, n);
    d.alive = d.codes + (size_t)n * c.groups;
    d.trailing = falloc<float>(f, (size_t)n * c.max_frames * H);
    d.trailing_rows = falloc<int>(f, n);
    d.codec_emb = f->codec_emb;
    d.pred_emb = f->pred_emb;
    d.tts_pad = f->tts_pad;
    d.cp_ctx = f->c_arr;
    d.t_ctx = f->t_arr;
    // the host's copy of the codes and alive flags, written by the step's
    // last kernel (coherent: the kernel's stores reach it uncached)
    check_hip(hipHostMalloc((void **)&f->pinned, sizeof(int32_t) * n * (c.groups + 1),
                            hipHostMallocCoherent),
              "hipHostMalloc");
    refresh_slices(f);
    check_hip(hipMemset(d.alive, 0, sizeof(int) * n), "frame init");
    check_hip(hipMemset(const_cast<uint64_t *>(d.seeds), 0, sizeof(uint64_t) * n), "frame init");
    check_hip(hipMemset(d.codes, 0xff, sizeof(int) * n * c.groups), "frame init");
    f->started.assign(n, 0);
    f->host_len.assign(n, 0);
    *out = f;
  });
  if (rc != 0 && f) {
    frame_release(f);
    delete f;
  }
  return rc;
}

namespace {

// The host values a start copies to the device: kept until the start's
// stream has been synchronized.
struct StartVals {
  uint64_t seed = 0;
  int32_t zero = 0, one = 1, trailing_rows = 0;
};

// the checks of a start of stream `stream` with rows prefill rows
void start_checks(const q3h_frame *f, int stream, int rows, int trailing_rows) {
  const q3h_frame_config &c = f->cfg;
  require(stream >= 0 && stream < c.n_streams, Q3H_E_ARG, "q3h_frame_start: bad stream");
  require(rows > 0, Q3H_E_ARG, "q3h_frame_start: empty prefill");
  require(trailing_rows >= 0 && trailing_rows <= c.max_frames, Q3H_E_ARG,
          "q3h_frame_start: more trailing rows than max_frames");
  require(rows <= c.max_positions, Q3H_E_CAPACITY, "q3h_frame_start: prefill too long");
}

// The talker part of TQwenTalker.Start (talker.pas:586-593) for stream
// `stream`, enqueued on its talker context's own HIP stream (the device is
// current, the slices synchronized, the arguments checked): reset, fill
// (prefill, trailing, st) writes the rows prefill [rows][H] (the context's
// work buffer) and trailing [trailing_rows][H] (the stream's trailing rows)
// on stream st, then the prefill runs and the stream's state is reset from
// sv. start_finish completes it.
template <class Fill>
void start_enqueue(q3h_frame *f, int stream, int rows, int trailing_rows, StartVals &sv,
                   Fill &&fill) {
  const q3h_frame_config &c = f->cfg;
  q3h_context *tc = f->tctx[stream];
  set_len(tc, 0, tc->stream);
  // the prefill through the single-context path, outputs kept on the device
  const int H = f->H;
  q3h_stack *s = f->talker;
  Work &w = tc->w;
  w.ensure(s, rows, attention_splits(s, rows), c.vocab);
  hipStream_t st = tc->stream;
  FrameDev &d = f->fd;
  fill(w.h, d.trailing + (size_t)stream * c.max_frames * H, st);
  launch_prep(tc->dev_arr, nullptr, 1, rows, w.rd, st);
  LayerIO io;
  io.single_context = true;
  run_layers(s, w, rows, rows, rows == 1, st, io);
  float *past = d.past + (size_t)stream * H;
  linear(s, w, s->heads[c.talker_head], w.h + (size_t)(rows - 1) * H, H, 1, s->final_norm,
         d.logits + (size_t)stream * c.vocab, c.vocab, EPI_STORE, past, st);
  launch_advance(tc->dev_arr, nullptr, 1, rows, st);
  check_hip(hipGetLastError(), "prefill kernels");
  // the sentence seed: the one of the settings, or a fresh one (Random64 shr 1)
  sv.seed = f->sampling.seed ? f->sampling.seed : (f->seed_rng() >> 1);
  sv.trailing_rows = trailing_rows;
  check_hip(hipMemcpyAsync(const_cast<uint64_t *>(d.seeds) + stream, &sv.seed, 8,
                           hipMemcpyHostToDevice, st),
            "seed");
  check_hip(hipMemsetAsync(d.seen + (size_t)stream * c.vocab, 0, c.vocab, st), "reset seen");
  check_hip(hipMemcpyAsync(d.nframes + stream, &sv.zero, 4, hipMemcpyHostToDevice, st), "state");
  check_hip(hipMemcpyAsync(d.step + stream, &sv.zero, 4, hipMemcpyHostToDevice, st), "state");
  check_hip(hipMemcpyAsync(d.trailing_rows + stream, &sv.trailing_rows, 4,
                           hipMemcpyHostToDevice, st),
            "state");
  check_hip(hipMemcpyAsync(d.alive + stream, &sv.one, 4, hipMemcpyHostToDevice, st), "state");
}

// waits for a start_enqueue of stream `stream` and marks the stream started
void start_finish(q3h_frame *f, int stream, int rows) {
  q3h_context *tc = f->tctx[stream];
  check_hip(hipStreamSynchronize(tc->stream), "prefill sync");
  tc->len = rows;
  f->host_len[stream] = rows;
  f->started[stream] = 1;
}

template <class Fill>
void start_stream(q3h_frame *f, int stream, int rows, int trailing_rows, Fill &&fill) {
  start_checks(f, stream, rows, trailing_rows);
  check_hip(hipSetDevice(f->talker->dev->ordinal), "hipSetDevice");
  sync_slices(f);
  StartVals sv;
  start_enqueue(f, stream, rows, trailing_rows, sv, fill);
  start_finish(f, stream, rows);
}

}  // namespace

extern "C" int q3h_frame_set_sampling(q3h_frame *f, const q3h_sampling *sp) {
  return guard([&] {
    require(f != nullptr && sp != nullptr, Q3H_E_ARG, "q3h_frame_set_sampling: NULL argument");
    const q3h_frame_config &c = f->cfg;
    auto check = [&](int on, float t, int k, float p, int vocab, const char *who) {
      if (!on) return;
      const std::string w = std::string("q3h_frame_set_sampling: ") + who;
      require(t > 0.0f, Q3H_E_ARG, w + " temperature must be positive");
      require(k >= 0, Q3H_E_ARG, w + " top_k must be >= 0");
      require(p > 0.0f && p <= 1.0f, Q3H_E_ARG, w + " top_p must be in (0, 1]");
      require(p == 1.0f || (k >= 1 && k <= 64), Q3H_E_ARG,
              w + " top_p < 1 needs 1 <= top_k <= 64");
      require(vocab <= 3 * kSampleThreads, Q3H_E_ARG, w + " sampling takes at most 3072 codes");
    };
    check(sp->do_sample, sp->temperature, sp->top_k, sp->top_p, c.vocab, "talker");
    check(sp->sub_do_sample, sp->sub_temperature, sp->sub_top_k, sp->sub_top_p, c.cp_vocab,
          "code predictor");
    check_hip(hipSetDevice(f->talker->dev->ordinal), "hipSetDevice");
    sync_slices(f);
    f->sampling = *sp;
    auto params = [](int on, float t, int k, float p) {
      return on ? SampleParams{1, t, k, p} : SampleParams{0, 1.0f, 0, 1.0f};
    };
    f->fd.sp0 = params(sp->do_sample, sp->temperature, sp->top_k, sp->top_p);
    f->fd.sp = params(sp->sub_do_sample, sp->sub_temperature, sp->sub_top_k, sp->sub_top_p);
    // the parameters are kernel arguments of the captured steps: capture again
    refresh_slices(f);
  });
}

extern "C" int q3h_frame_start(q3h_frame *f, int stream, const float *prefill, int rows,
                               const float *trailing, int trailing_rows) {
  return guard([&] {
    require(f != nullptr, Q3H_E_ARG, "q3h_frame_start: NULL frame");
    require(prefill != nullptr && rows > 0, Q3H_E_ARG, "q3h_frame_start: empty prefill");
    require(trailing_rows == 0 || trailing != nullptr, Q3H_E_ARG,
            "q3h_frame_start: trailing is NULL");
    const size_t H = f->H;
    start_stream(f, stream, rows, trailing_rows, [&](float *pre, float *trail, hipStream_t st) {
      check_hip(hipMemcpyAsync(pre, prefill, sizeof(float) * rows * H, hipMemcpyHostToDevice, st),
                "upload prefill");
      if (trailing_rows > 0)
        check_hip(hipMemcpyAsync(trail, trailing, sizeof(float) * trailing_rows * H,
                                 hipMemcpyHostToDevice, st),
                  "upload trailing");
    });
  });
}

extern "C" int q3h_frame_start_batch(q3h_frame *f, int n, const int *streams,
                                     const float *const *prefill, const int *rows,
                                     const float *const *trailing, const int *trailing_rows) {
  return guard([&] {
    require(f != nullptr, Q3H_E_ARG, "q3h_frame_start_batch: NULL frame");
    require(n > 0 && streams && prefill && rows, Q3H_E_ARG,
            "q3h_frame_start_batch: invalid argument");
    // every start checked before any is enqueued
    std::vector<char> seen(f->cfg.n_streams, 0);
    for (int i = 0; i < n; i++) {
      const int tr = trailing_rows ? trailing_rows[i] : 0;
      start_checks(f, streams[i], rows[i], tr);
      require(!seen[streams[i]], Q3H_E_ARG, "q3h_frame_start_batch: repeated stream");
      seen[streams[i]] = 1;
      require(prefill[i] != nullptr, Q3H_E_ARG, "q3h_frame_start_batch: NULL prefill");
      require(tr == 0 || (trailing && trailing[i]), Q3H_E_ARG,
              "q3h_frame_start_batch: trailing is NULL");
    }
    check_hip(hipSetDevice(f->talker->dev->ordinal), "hipSetDevice");
    sync_slices(f);
    const size_t H = f->H;
    std::vector<StartVals> sv(n);
    int enqueued = 0;
    try {
      for (int i = 0; i < n; i++) {
        const int tr = trailing_rows ? trailing_rows[i] : 0;
        start_enqueue(f, streams[i], rows[i], tr, sv[i],
                      [&](float *pre, float *trail, hipStream_t st) {
                        check_hip(hipMemcpyAsync(pre, prefill[i], sizeof(float) * rows[i] * H,
                                                 hipMemcpyHostToDevice, st),
                                  "upload prefill");
                        if (tr > 0)
                          check_hip(hipMemcpyAsync(trail, trailing[i], sizeof(float) * tr * H,
                                                   hipMemcpyHostToDevice, st),
                                    "upload trailing");
                      });
        enqueued++;
      }
    } catch (...) {
      // the enqueued starts still read sv: let them end before it goes
      for (int i = 0; i < enqueued; i++) (void)hipStreamSynchronize(f->tctx[streams[i]]->stream);
      throw;
    }
    for (int i = 0; i < n; i++) start_finish(f, streams[i], rows[i]);
  });
}

extern "C" int q3h_frame_start_text(q3h_frame *f, int stream, q3h_text_proj *t,
                                    const q3h_start_ids *sp, const int32_t *ids, int n_ids,
                                    const int32_t *codec, int n_codec, int non_streaming) {
  return guard([&] {
    require(f != nullptr && t != nullptr && sp != nullptr, Q3H_E_ARG,
            "q3h_frame_start_text: NULL frame, projection or ids");
    require(t->dev == f->talker->dev, Q3H_E_ARG,
            "q3h_frame_start_text: the projection is on another device");
    require(t->cfg.hidden == f->H, Q3H_E_ARG,
            "q3h_frame_start_text: the projection's hidden size is not the talker's");
    // PromptIds: [im_start, assistant, \n] text [im_end, \n, im_start, assistant, \n]
    require(ids != nullptr && n_ids >= 9, Q3H_E_ARG, "q3h_frame_start_text: empty text");
    require(codec != nullptr && n_codec >= 2, Q3H_E_ARG,
            "q3h_frame_start_text: the codec ids end with codec_pad, codec_bos");
    const int TV = t->cfg.text_vocab, V = f->cfg.vocab;
    auto text_ok = [&](int id) { return id >= 0 && id < TV; };
    auto codec_ok = [&](int id) { return id >= 0 && id < V; };
    for (int i = 0; i < n_ids; i++)
      require(text_ok(ids[i]), Q3H_E_ARG,
              "q3h_frame_start_text: text token " + std::to_string(ids[i]) + " out of range");
    require(text_ok(sp->tts_bos) && text_ok(sp->tts_eos) && text_ok(sp->tts_pad), Q3H_E_ARG,
            "q3h_frame_start_text: tts_bos / tts_eos / tts_pad out of range");
    for (int i = 0; i < n_codec; i++)
      require(codec_ok(codec[i]), Q3H_E_ARG,
              "q3h_frame_start_text: codec id " + std::to_string(codec[i]) + " out of range");
    require(codec_ok(sp->codec_pad) && codec_ok(sp->codec_bos), Q3H_E_ARG,
            "q3h_frame_start_text: codec_pad / codec_bos out of range");
    const int nt = n_ids - 8, nc = n_codec;
    // the projected rows: the role (ids 0..2), tts_pad, tts_bos, tts_eos, the text
    std::vector<int32_t> proj_ids = {ids[0], ids[1], ids[2], sp->tts_pad, sp->tts_bos,
                                     sp->tts_eos};
    proj_ids.insert(proj_ids.end(), ids + 3, ids + 3 + nt);
    const int P_PAD = 3, P_BOS = 4, P_EOS = 5, P_TEXT = 6;
    // the rows: (projected row, codec id or -1)
    std::vector<int2> plan;
    for (int r = 0; r < 3; r++) plan.push_back(make_int2(r, -1));
    for (int i = 0; i < nc - 1; i++) plan.push_back(make_int2(i < nc - 2 ? P_PAD : P_BOS, codec[i]));
    if (non_streaming) {
      for (int i = 0; i < nt; i++) plan.push_back(make_int2(P_TEXT + i, sp->codec_pad));
      plan.push_back(make_int2(P_EOS, sp->codec_pad));
      plan.push_back(make_int2(P_PAD, sp->codec_bos));
    } else {
      plan.push_back(make_int2(P_TEXT, sp->codec_bos));
    }
    const int rows = (int)plan.size();
    if (non_streaming) {
      plan.push_back(make_int2(P_PAD, -1));
    } else {
      for (int i = 1; i < nt; i++) plan.push_back(make_int2(P_TEXT + i, -1));
      plan.push_back(make_int2(P_EOS, -1));
    }
    const int trailing_rows = (int)plan.size() - rows;
    const int np = (int)proj_ids.size();
    std::lock_guard<std::mutex> lk(t->mu);
    check_hip(hipSetDevice(f->talker->dev->ordinal), "hipSetDevice");
    text_ensure(t, np);
    const int need = std::max(np, (int)plan.size());
    if (need > f->start_cap) {
      sync_slices(f);
      dev_free(f->start_plan);
      dev_free(f->start_proj);
      f->start_plan = nullptr;
      f->start_proj = nullptr;
      f->start_cap = 0;
      const int cap = std::max(need, 64);
      f->start_plan = (int2 *)dev_alloc(sizeof(int2) * cap);
      f->start_proj = (float *)dev_alloc(sizeof(float) * cap * f->H);
      f->start_cap = cap;
    }
    start_stream(f, stream, rows, trailing_rows, [&](float *pre, float *trail, hipStream_t st) {
      check_hip(hipMemcpyAsync(t->ids, proj_ids.data(), sizeof(int32_t) * np,
                               hipMemcpyHostToDevice, st),
                "upload ids");
      check_hip(hipMemcpyAsync(f->start_plan, plan.data(), sizeof(int2) * plan.size(),
                               hipMemcpyHostToDevice, st),
                "upload plan");
      text_project_dev(t, t->ids, np, f->start_proj, f->H, st);
      hipLaunchKernelGGL(k_start_rows, dim3((unsigned)plan.size()), dim3(256), 0, st,
                         f->start_plan, rows, f->start_proj, f->codec_emb, f->H, pre, trail);
      check_hip(hipGetLastError(), "start rows");
    });
  });
}

extern "C" int q3h_frame_step(q3h_frame *f, int32_t *codes, int32_t *alive) {
  return guard([&] {
    require(f != nullptr, Q3H_E_ARG, "q3h_frame_step: NULL frame");
    const q3h_frame_config &c = f->cfg;
    const int n = c.n_streams;
    bool any = false;
    for (int s = 0; s < n; s++) {
      if (!f->started[s]) continue;
      any = true;
      require(f->host_len[s] + 1 <= c.max_positions, Q3H_E_CAPACITY,
              "q3h_frame_step: a stream reached max_positions");
    }
    require(any, Q3H_E_STATE, "q3h_frame_step: no stream was started");
    check_hip(hipSetDevice(f->talker->dev->ordinal), "hipSetDevice");
    for (FrameSlice &sl : f->slices) {
      // the longest context of the slice's running streams
      int slen = 0;
      for (int s = sl.first; s < sl.first + sl.n; s++)
        if (f->started[s]) slen = std::max(slen, f->host_len[s] + 1);
      if (slen == 0) continue;  // no stream of the slice runs (its codes read as -1)
      // the int8 talker's step does not depend on the cover (its attention
      // takes any context length): one graph, captured once for every length
      if (sl.fd.t_xq) slen = c.max_positions;
      if (c.use_graph) {
        // the captured step that covers slen; on the first capture every
        // cover up to 256 positions is captured too, so that growing
        // contexts switch graphs without capturing again
        auto find = [&]() -> hipGraphExec_t {
          for (auto &g : sl.graphs)
            if (g.first >= slen) return g.second;
          return nullptr;
        };
        hipGraphExec_t exec = find();
        if (!exec) {
          std::vector<int> covers = {graph_cover(slen, c.max_positions)};
          if (sl.graphs.empty())
            for (int p = 64; p <= 256; p += 64)
              if (p > slen) covers.push_back(graph_cover(p, c.max_positions));
          std::sort(covers.begin(), covers.end());
          covers.erase(std::unique(covers.begin(), covers.end()), covers.end());
          for (int cover : covers) {
            hipGraph_t graph =
                capture_graph(sl.stream, [&] { enqueue_step(f, sl, cover, sl.stream); });
            hipGraphExec_t e = nullptr;
            const hipError_t r = hipGraphInstantiate(&e, graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            check_hip(r, "hipGraphInstantiate");
            sl.graphs.emplace_back(cover, e);
          }
          std::sort(sl.graphs.begin(), sl.graphs.end());
          exec = find();
        }
        check_hip(hipGraphLaunch(exec, sl.stream), "hipGraphLaunch");
      } else {
        // the cover a captured step would use, so that both give the same sums
        // (beyond 256 positions the split attention's shape follows the cover)
        enqueue_step(f, sl, graph_cover(slen, c.max_positions), sl.stream);
        check_hip(hipGetLastError(), "frame kernels");
      }
      // the slice's codes and alive flags reach the pinned copy from the
      // step's last kernel (k_frame_end)
    }
    for (FrameSlice &sl : f->slices)
      check_hip(hipStreamSynchronize(sl.stream), "frame step sync");
    for (int s = 0; s < n; s++) {
      const bool live = f->started[s] && f->pinned[n * c.groups + s] != 0;
      if (codes)
        for (int g = 0; g < c.groups; g++)
          codes[s * c.groups + g] = live ? f->pinned[s * c.groups + g] : -1;
      if (alive) alive[s] = live ? 1 : 0;
      if (live) {
        f->host_len[s] += 1;
        f->tctx[s]->len += 1;
      } else {
        f->started[s] = 0;
      }
    }
  });
}

extern "C" int q3h_frame_state(q3h_frame *f, int stream, float *logits, float *past_hidden) {
  return guard([&] {
    require(f != nullptr, Q3H_E_ARG, "q3h_frame_state: NULL frame");
    require(stream >= 0 && stream < f->cfg.n_streams, Q3H_E_ARG, "q3h_frame_state: bad stream");
    check_hip(hipSetDevice(f->talker->dev->ordinal), "hipSetDevice");
    sync_slices(f);
    if (logits)
      check_hip(hipMemcpy(logits, f->fd.logits + (size_t)stream * f->cfg.vocab,
                          sizeof(float) * f->cfg.vocab, hipMemcpyDeviceToHost),
                "download logits");
    if (past_hidden)
      check_hip(hipMemcpy(past_hidden, f->fd.past + (size_t)stream * f->H, sizeof(float) * f->H,
                          hipMemcpyDeviceToHost),
                "download state");
  });
}

extern "C" int q3h_frame_destroy(q3h_frame *f) {
  return guard([&] {
    require(f != nullptr, Q3H_E_ARG, "q3h_frame_destroy: NULL frame");
    check_hip(hipSetDevice(f->talker->dev->ordinal), "hipSetDevice");
    sync_slices(f);
    frame_release(f);
    delete f;
  });
}
