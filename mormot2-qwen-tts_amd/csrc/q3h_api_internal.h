// q3h_api_internal.h - host-side objects behind the opaque handles of q3h.h.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "q3h.h"
#include "q3h_internal.h"

struct q3h_device {
  int ordinal = 0;
  int cus = 0;
  std::string name;
  std::atomic<int64_t> bytes{0};
  std::atomic<int> stacks{0};
  // the device address of this GPU's copy of the static scratch array of
  // q3h_forward_embeds_noalloc, and the lock its calls take
  void *scratch = nullptr;
  std::mutex scratch_mu;
};

namespace q3h {

constexpr int kAttnChunk = 256;  // positions per attention split (k_attention)
constexpr int kMaxGroup = 4;     // q heads per kv head (1, 2 or 4)

struct Error {
  int code;
  std::string msg;
};

extern thread_local std::string g_last_error;

void check_hip(hipError_t e, const char *what);
void require(bool cond, int code, const std::string &msg);
void *dev_alloc(size_t bytes);
void dev_free(void *p);

template <class F>
int guard(F &&f) {
  try {
    f();
    g_last_error.clear();
    return Q3H_OK;
  } catch (const Error &e) {
    g_last_error = e.msg;
    return e.code;
  } catch (const std::exception &e) {
    g_last_error = e.what();
    return Q3H_E_HIP;
  }
}

// The attention positions a captured step covers for contexts of up to len
// positions: up to 256 in steps of 64 (the single-workgroup attention loads
// what it covers), beyond that in steps of 256 with one step of headroom (the
// split attention leaves extra splits empty); at most max_positions. A launch
// sized for the cover gives the same sums at every length it covers up to 256
// (the extra positions add exact zeros); beyond, the split count follows the
// cover.
inline int graph_cover(int len, int max_positions) {
  const int cap = len <= 256 ? (len + 63) / 64 * 64 : ((len + 255) / 256 + 1) * 256;
  return std::min(max_positions, cap);
}

// Captures what enqueue() launches on stream st into a new graph. When
// enqueue throws, the capture is ended and its partial graph destroyed before
// the error goes on, so the stream leaves capture mode and later calls work.
template <class F>
hipGraph_t capture_graph(hipStream_t st, F &&enqueue) {
  check_hip(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  try {
    enqueue();
  } catch (...) {
    hipGraph_t partial = nullptr;
    (void)hipStreamEndCapture(st, &partial);
    if (partial) (void)hipGraphDestroy(partial);
    (void)hipGetLastError();
    throw;
  }
  hipGraph_t g = nullptr;
  check_hip(hipStreamEndCapture(st, &g), "hipStreamEndCapture");
  return g;
}

struct Layer {
  Mat qkv;   // [q; k; v] rows
  Mat o;     // [hidden][heads * head_dim]
  Mat gu;    // gate and up interleaved: row 2j = gate j, row 2j + 1 = up j
  Mat down;  // [hidden][intermediate]
  float *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

struct q3h_stack_fwd;

// device buffers of one forward over up to rows_cap rows
struct Work {
  int rows_cap = 0, splits_cap = 0, head_cap = 0;
  unsigned gen = 0;  // counts the (re)allocations: graphs that captured the buffers check it
  float *h = nullptr;       // residual stream [rows][hidden]
  float *qkv = nullptr;     // [rows][q + k + v]
  float *att = nullptr;     // [rows][heads * head_dim]
  float *act = nullptr;     // [rows][intermediate]
  float *normed = nullptr;  // [rows][hidden]
  float *logits = nullptr;  // [rows][head rows]
  RowDesc *rd = nullptr;    // [rows]
  float *part = nullptr;    // attention partials [rows][heads][splits][head_dim + 2]
  CtxDev **ctx_arr = nullptr;
  QAct xa, xb;              // quantized activations (act_q8 stacks)
  float *gpart = nullptr;   // chunk partials of the int8 products (act_q8)
  void ensure(const struct ::q3h_stack *s, int rows, int splits, int head_rows);
  void release();
};

// w's buffers for (rows, splits, head_rows) carved from [base, base + cap),
// each at a 256-byte boundary (w owns nothing: never release it); false when
// they do not fit
bool work_carve(const struct ::q3h_stack *s, int rows, int splits, int head_rows, void *base,
                size_t cap, Work &w);

// attention splits (the partial buffer) for contexts of up to `positions`
int attention_splits(const struct ::q3h_stack *s, int positions);
// the most splits of any context of up to `positions` positions
int attention_splits_upto(const struct ::q3h_stack *s, int positions);
// y [M][ldy] (+)= W . x (x RMS-normed with norm_w when non-null; epi: EPI_*):
// the f32-activation GEMV, or for act_q8 stacks the quantizer and the int8
// product; xn_out, when non-null, receives the (normed) row M - 1
void linear(const struct ::q3h_stack *s, Work &w, const Mat &W, const float *x, int ldx, int M,
            const float *norm_w, float *y, int ldy, int epi, float *xn_out, hipStream_t st);
GemvArgs make_gemv(const Mat &W, const float *x, int ldx, int M, const float *norm_w, float eps,
                   float *y, int ldy);
// the shapes the fused code-predictor kernel takes (Q8_0, hidden 1024,
// 16 / 8 heads of 128)
bool cp_fused_supported(const q3h_stack_config &c);

// one new row at position pos of a code-predictor context (16 positions)
// through the layers of stack s, attention fused into o_proj; the row is in
// w.h and stays there (cp_fused_supported(s->cfg), ctx->max_pos == 16)
// src (optional): the row is chosen on the device instead, by the first
// product (launch_gemv_q8_code: the argmax of src->logits, row of src->rows,
// code to src->code_out), and written to w.h by that product
struct CodeSrc {
  const float *logits;
  int vocab;
  const float *rows;
  int *code_out;
  const int *alive;
};
void run_cp_fused(const struct ::q3h_stack *s, Work &w, const struct ::q3h_context *ctx,
                  int pos, hipStream_t st, const CodeSrc *src = nullptr);

// the first step of a code-predictor context (its two rows, positions 0 and
// 1, in w.h) through the layers, attention fused into o_proj; the rows stay
// in w.h (cp_fused_supported(s->cfg), ctx->max_pos == 16)
void run_cp_fused_first(const struct ::q3h_stack *s, Work &w, const struct ::q3h_context *ctx,
                        hipStream_t st);

// options of run_layers (the first two: the int8 path over few rows, partial_path)
struct LayerIO {
  bool input_quantized = false;       // w.xa already holds layer 0's normed, quantized input
  const float *final_norm = nullptr;  // after the last layer: RMSNorm with it, quantized into w.xa
  float *final_normed = nullptr;      // [M][hidden] device: those normed rows (int8 path, few rows)
  bool single_context = false;        // the rows are consecutive positions of one context
  float *layer_out = nullptr;         // [layers][M][hidden] device: w.h after each layer
  // the rows come in pairs, row 2i + 1 at the position after row 2i's in the
  // same context (the int8 path over few rows then runs the fused attention)
  bool row_pairs = false;
};
// whether run_layers takes the int8 partial-product path for M rows of stack s
bool partial_path(const struct ::q3h_stack *s, int M);

// fused: every row is the single new position of its own context; positions:
// the most positions any row attends to (its own included), Work sized for
// attention_splits(s, positions)
void run_layers(const struct ::q3h_stack *s, Work &w, int M, int positions, bool fused,
                hipStream_t st, const LayerIO &io = LayerIO{});

}  // namespace q3h

struct q3h_stack {
  q3h_device *dev = nullptr;
  q3h_stack_config cfg{};
  std::vector<q3h::Layer> layers;
  float *final_norm = nullptr;
  float *rope_cs = nullptr;  // [max_positions][head_dim / 2] (cos, sin)
  std::vector<q3h::Mat> heads;
  int64_t bytes = 0, head_bytes = 0;
  int64_t aux_bytes = 0;  // the split-bf16 planes of f32 layers (not in StackBytes)
  std::atomic<int> contexts{0};
  std::mutex mu;
  hipStream_t stream = nullptr;  // uploads
};

struct q3h_context {
  q3h_stack *s = nullptr;
  int max_pos = 0;
  int len = 0;  // host mirror of dev->len
  void *k = nullptr, *v = nullptr;
  q3h::CtxDev *dev = nullptr;
  q3h::CtxDev **dev_arr = nullptr;  // {dev}
  hipStream_t stream = nullptr;
  q3h::Work w;
  float *probe = nullptr;  // the layer outputs of q3h_forward_embeds_probe
  size_t probe_bytes = 0;
  // the captured single-row forwards, keyed by (head + 1) << 32 | cover, valid
  // for the Work buffers of generation graphs_gen
  std::vector<std::pair<uint64_t, hipGraphExec_t>> graphs;
  unsigned graphs_gen = 0;
  // pinned host staging of a single-row forward: the input row, the logits,
  // the normed state (hipHostMalloc'ed on first use, pin_floats floats)
  float *pin = nullptr;
  size_t pin_floats = 0;
};

// the text projection (q3h_text.hip)
struct q3h_text_proj {
  q3h_device *dev = nullptr;
  q3h_text_config cfg{};
  void *emb = nullptr;  // [text_vocab][text_hidden], BF16 or f32
  q3h::Mat fc1, fc2;    // f32
  float *b1 = nullptr, *b2 = nullptr;
  int cap = 0;               // rows of the work buffers
  int32_t *ids = nullptr;    // [cap]
  float *e = nullptr;        // [cap][text_hidden] embedding rows
  float *h = nullptr;        // [cap][text_hidden] SiLU(fc1 . e + b1)
  float *y = nullptr;        // [cap][hidden]
  int64_t bytes = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
};

namespace q3h {
// the work buffers of t for n rows (grows, synchronizing t->stream first)
void text_ensure(q3h_text_proj *t, int n);
// y [n][ldy] = the projection of the n ids at ids_dev (device, each in
// [0, text_vocab): the caller checks), on stream st; uses t->e and t->h
// (text_ensure(t, n) first)
void text_project_dev(q3h_text_proj *t, const int32_t *ids_dev, int n, float *y, int ldy,
                      hipStream_t st);

q3h_context *new_context(q3h_stack *s, int max_positions);
void free_context(q3h_context *ctx);
void set_len(q3h_context *c, int len, hipStream_t st);
}  // namespace q3h
