// q3h_api.hip - the C ABI of libq3h (include/q3h.h): device, stacks, contexts,
// the forward and the batched forward. The frame step lives in q3h_frame.hip.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "q3h.h"
#include "q3h_api_internal.h"

using namespace q3h;

namespace q3h {

thread_local std::string g_last_error;

void check_hip(hipError_t e, const char *what) {
  if (e != hipSuccess)
    throw Error{Q3H_E_HIP, std::string(what) + ": " + hipGetErrorString(e)};
}

void require(bool cond, int code, const std::string &msg) {
  if (!cond) throw Error{code, msg};
}

void *dev_alloc(size_t bytes) {
  void *p = nullptr;
  if (bytes == 0) bytes = 256;
  check_hip(hipMalloc(&p, bytes), "hipMalloc");
  return p;
}

void dev_free(void *p) {
  if (p) (void)hipFree(p);
}

// ---------------------------------------------------------------------------
// work buffers of a forward over M rows

// Every buffer of a Work for R rows, `splits` attention splits per row and
// head_rows logits per row, in one order: each(slot, bytes) per buffer.
template <class Each>
void work_fields(const q3h_stack *s, size_t R, int splits, int head_rows, Work &w, Each &&each) {
  const q3h_stack_config &c = s->cfg;
  const size_t H = c.hidden, NQ = (size_t)c.heads * c.head_dim;
  const size_t NKV = (size_t)c.kv_heads * c.head_dim, I = c.intermediate;
  each((void **)&w.h, sizeof(float) * R * H);
  each((void **)&w.qkv, sizeof(float) * R * (NQ + 2 * NKV));
  each((void **)&w.att, sizeof(float) * R * NQ);
  each((void **)&w.act, sizeof(float) * R * I);
  each((void **)&w.normed, sizeof(float) * R * H);
  each((void **)&w.logits, sizeof(float) * R * (head_rows > 0 ? head_rows : 1));
  each((void **)&w.rd, sizeof(RowDesc) * R);
  // attention partials; at least the code predictor's four o_proj partials
  each((void **)&w.part,
       sizeof(float) * std::max(R * c.heads * splits * (c.head_dim + 2), 4 * H));
  each((void **)&w.ctx_arr, sizeof(CtxDev *) * R);
  if (c.act_q8) {
    const int maxK = std::max(std::max((int)H, (int)NQ), (int)I);
    each((void **)&w.xa.q, qact_bytes((int)R, maxK));
    each((void **)&w.xb.q, qact_bytes((int)R, maxK));
    // chunk partials of the products over up to kPartialRows rows
    const size_t pr = std::min<size_t>(R, kPartialRows);
    const size_t ldq = NQ + 2 * NKV;
    size_t pn = (size_t)gemm_i8_chunks((int)H) * pr * std::max(ldq, (size_t)2 * I);
    pn = std::max(pn, (size_t)gemm_i8_chunks((int)NQ) * pr * H);
    pn = std::max(pn, (size_t)gemm_i8_chunks((int)I) * pr * H);
    each((void **)&w.gpart, sizeof(float) * pn);
  } else {
    // K-slice sums of the products of o_proj and down (f32 activations); up
    // to kQ8SliceRows rows, the 256-column slices of Q8_0 q/k/v, o_proj and
    // down
    const size_t sr = std::min<size_t>(R, kQ8SliceRows), ldq = NQ + 2 * NKV;
    size_t pn = kF32Slices * R * H;
    pn = std::max(pn, sr * (H / 256) * ldq);
    pn = std::max(pn, sr * std::min<size_t>(kMaxPartSlices, std::max(NQ, I) / 256) * H);
    each((void **)&w.gpart, sizeof(float) * pn);
  }
}

void Work::ensure(const q3h_stack *s, int rows, int splits, int head_rows) {
  if (rows <= rows_cap && splits <= splits_cap && head_rows <= head_cap) return;
  release();
  rows_cap = rows > rows_cap ? rows : rows_cap;
  splits_cap = splits > splits_cap ? splits : splits_cap;
  head_cap = head_rows > head_cap ? head_rows : head_cap;
  work_fields(s, rows_cap, splits_cap, head_cap, *this,
              [](void **slot, size_t bytes) { *slot = dev_alloc(bytes); });
  gen++;
}

bool work_carve(const q3h_stack *s, int rows, int splits, int head_rows, void *base, size_t cap,
                Work &w) {
  size_t off = 0;
  bool fits = true;
  work_fields(s, rows, splits, head_rows, w, [&](void **slot, size_t bytes) {
    off = (off + 255) & ~(size_t)255;
    fits = fits && off + bytes <= cap;
    *slot = fits ? (char *)base + off : nullptr;
    off += bytes;
  });
  w.rows_cap = rows;
  w.splits_cap = splits;
  w.head_cap = head_rows;
  return fits;
}

void Work::release() {
  dev_free(h);
  dev_free(qkv);
  dev_free(att);
  dev_free(act);
  dev_free(normed);
  dev_free(logits);
  dev_free(rd);
  dev_free(part);
  dev_free(ctx_arr);
  dev_free(xa.q);
  dev_free(xb.q);
  dev_free(gpart);
  xa = QAct{};
  xb = QAct{};
  gpart = nullptr;
  h = qkv = att = act = normed = logits = part = nullptr;
  rd = nullptr;
  ctx_arr = nullptr;
}

int attention_splits(const q3h_stack *s, int positions) {
  return attn_splits(positions, s->cfg.kv_f16 != 0);
}

int attention_splits_upto(const q3h_stack *s, int positions) {
  return attn_splits_upto(positions, s->cfg.kv_f16 != 0);
}

void linear(const q3h_stack *s, Work &w, const Mat &W, const float *x, int ldx, int M,
            const float *norm_w, float *y, int ldy, int epi, float *xn_out, hipStream_t st) {
  const q3h_stack_config &c = s->cfg;
  if (c.act_q8) {
    launch_quantize_act(x, ldx, M, W.K, norm_w, c.rms_eps, w.xa, xn_out, st);
    launch_gemm_i8(W, w.xa, M, epi, y, ldy, st);
  } else if ((c.dtype == Q3H_F32 || M > kGemvRows) && gemm_f32_supported(W.N, W.K) &&
             (xn_out == nullptr || M == 1)) {
    // f32 weights (or Q8_0 weights over more rows than the matrix-vector
    // kernels take in one pass) on the matrix cores, with f32 activations; the
    // RMSNorm of the rows first (into the work buffer, or into xn_out, the one
    // row the caller wants back)
    if (norm_w) {
      float *xn = xn_out ? xn_out : w.normed;
      launch_rmsnorm_rows(x, ldx, M, W.K, norm_w, c.rms_eps, xn, W.K, st);
      x = xn;
      ldx = W.K;
    }
    launch_gemm_f32(W, x, ldx, M, epi, y, ldy, st);
  } else {
    GemvArgs a = make_gemv(W, x, ldx, M, norm_w, c.rms_eps, y, ldy);
    a.xn_out = xn_out;
    launch_gemv(a, epi, c.dtype == Q3H_Q8_0, st);
  }
}

// the residual stream after layer l into the probe buffer (when one is set)
static void probe_layer(const LayerIO &io, const Work &w, int l, int M, int H, hipStream_t st) {
  if (io.layer_out)
    check_hip(hipMemcpyAsync(io.layer_out + (size_t)l * M * H, w.h, sizeof(float) * M * H,
                             hipMemcpyDeviceToDevice, st),
              "probe copy");
}

// The int8 path over M <= kPartialRows rows: every product leaves its chunk
// partials (one wave per 16 rows and 512 columns over the whole chip), and
// the consumer adds them in chunk order: the attention prologue (q/k/v, decode
// rows), the residual add + RMSNorm + quantization of the next input (o_proj,
// down), SiLU(gate) * up + quantization (gate/up). Results equal the
// workgroup-reduced schedule of run_layers to the bit.
static void run_layers_partial(const q3h_stack *s, Work &w, int M, bool fused,
                               const LayerIO &io, hipStream_t st) {
  const q3h_stack_config &c = s->cfg;
  const int H = c.hidden, hd = c.head_dim, NQ = c.heads * hd, NKV = c.kv_heads * hd;
  const int I = c.intermediate, ldq = NQ + 2 * NKV;
  const bool kv16 = c.kv_f16 != 0;
  const float eps = c.rms_eps;
  // rows in pairs of consecutive positions take the fused attention too
  const bool pairs = io.row_pairs && M % 2 == 0 && attn_x_pairs_supported(c.max_positions);
  if (!io.input_quantized)
    launch_quantize_act(w.h, H, M, H, s->layers[0].in_norm, eps, w.xa, nullptr, st);
  for (int l = 0; l < c.layers; l++) {
    const Layer &L = s->layers[l];
    AttnArgs at{};
    at.ldq = ldq;
    at.rd = w.rd;
    at.layer = l;
    at.heads = c.heads;
    at.kvh = c.kv_heads;
    at.qkn = L.q_norm;
    at.rope_cs = reinterpret_cast<const float2 *>(s->rope_cs);
    if (fused || pairs) {
      launch_gemm_i8_partial(L.qkv, w.xa, M, w.gpart, st);
      at.qkv = w.gpart;
      launch_attn_x(at, M, true, kv16, gemm_i8_chunks(H), w.xa, c.max_positions, st,
                    !fused && pairs);
    } else {
      launch_gemm_i8(L.qkv, w.xa, M, EPI_STORE, w.qkv, ldq, st);
      launch_qk_rope_append(w.qkv, ldq, w.rd, M, l, c.heads, c.kv_heads, hd, L.q_norm,
                            L.k_norm, eps, s->rope_cs, kv16, st);
      at.qkv = w.qkv;
      launch_attn_x(at, M, false, kv16, 0, w.xa, c.max_positions, st);
    }
    launch_gemm_i8_partial(L.o, w.xa, M, w.gpart, st);
    launch_residual_quantize(w.h, w.gpart, gemm_i8_chunks(NQ), M, H, L.post_norm, eps, &w.xa,
                             st);
    const QAct *act = &w.xb;
    if (!launch_gemm_i8_swiglu_quantize(L.gu, w.xa, M, w.xb, st)) {
      launch_gemm_i8_partial(L.gu, w.xa, M, w.gpart, st);
      launch_swiglu_quantize(w.gpart, gemm_i8_chunks(H), M, I, w.xa, st);
      act = &w.xa;
    }
    launch_gemm_i8_partial(L.down, *act, M, w.gpart, st);
    const bool next = l + 1 < c.layers;
    const float *nw = next ? s->layers[l + 1].in_norm : io.final_norm;
    launch_residual_quantize(w.h, w.gpart, gemm_i8_chunks(I), M, H, nw, eps,
                             nw ? &w.xa : nullptr, st, next ? nullptr : io.final_normed);
    probe_layer(io, w, l, M, H, st);
  }
}

// f32 activations on the matrix cores (f32 weights at any row count, Q8_0
// weights over more rows than the matrix-vector kernels take): o_proj and
// down (N = hidden: too few weight-row tiles to fill the chip) are cut into K
// slices; each slice sum is added to the residual in slice order by the
// kernel that also applies the next RMSNorm, whose output feeds the next
// product directly.
bool f32_slice_path(const q3h_stack *s, int M) {
  const q3h_stack_config &c = s->cfg;
  const int NQ = c.heads * c.head_dim, I = c.intermediate, H = c.hidden;
  const int ldq = NQ + 2 * c.kv_heads * c.head_dim;
  return !c.act_q8 && (c.dtype == Q3H_F32 || M > kGemvRows) && gemm_f32_supported(ldq, H) &&
         gemm_f32_supported(2 * I, H) && gemm_f32_slices_supported(H, NQ) &&
         gemm_f32_slices_supported(H, I);
}

static void run_layers_f32(const q3h_stack *s, Work &w, int M, int positions, bool fused,
                           const LayerIO &io, hipStream_t st) {
  const bool single_context = io.single_context;
  const q3h_stack_config &c = s->cfg;
  const int H = c.hidden, hd = c.head_dim, NQ = c.heads * hd, NKV = c.kv_heads * hd;
  const int I = c.intermediate, ldq = NQ + 2 * NKV;
  const bool kv16 = c.kv_f16 != 0;
  const float eps = c.rms_eps;
  launch_rmsnorm_rows(w.h, H, M, H, s->layers[0].in_norm, eps, w.normed, H, st);
  for (int l = 0; l < c.layers; l++) {
    const Layer &L = s->layers[l];
    // q/k/v as K slices (Q8_0, 17-64 rows of a prefill) added by the append
    const int qs = fused ? 0 : q8x_slices(L.qkv, M);
    if (qs > 0 && qs <= kRopeMaxSlices) {
      launch_gemm_f32_part(L.qkv, w.normed, H, M, w.gpart, st);
      launch_qk_rope_append(w.qkv, ldq, w.rd, M, l, c.heads, c.kv_heads, hd, L.q_norm,
                            L.k_norm, eps, s->rope_cs, kv16, st, w.gpart, qs);
    } else {
      launch_gemm_f32(L.qkv, w.normed, H, M, EPI_STORE, w.qkv, ldq, st);
      if (!fused)
        launch_qk_rope_append(w.qkv, ldq, w.rd, M, l, c.heads, c.kv_heads, hd, L.q_norm,
                              L.k_norm, eps, s->rope_cs, kv16, st);
    }
    AttnArgs at{};
    at.qkv = w.qkv;
    at.ldq = ldq;
    at.rd = w.rd;
    at.layer = l;
    at.heads = c.heads;
    at.kvh = c.kv_heads;
    at.qkn = L.q_norm;
    at.rope_cs = reinterpret_cast<const float2 *>(s->rope_cs);
    at.out = w.att;
    at.part = w.part;
    if (!fused && single_context && M >= kPrefillRows)
      launch_attn_prefill(at, M, kv16, st);
    else
      launch_attn(at, M, positions, fused, kv16, st);
    const int so = launch_gemm_f32_part(L.o, w.att, NQ, M, w.gpart, st);
    launch_resid_norm(w.h, w.gpart, M, H, L.post_norm, eps, w.normed, so, st);
    launch_gemm_f32(L.gu, w.normed, H, M, EPI_SWIGLU, w.act, I, st);
    const int sd = launch_gemm_f32_part(L.down, w.act, I, M, w.gpart, st);
    const float *next = l + 1 < c.layers ? s->layers[l + 1].in_norm : nullptr;
    launch_resid_norm(w.h, w.gpart, M, H, next, eps, w.normed, sd, st);
    probe_layer(io, w, l, M, H, st);
  }
}

// The layers of a stack over M rows of w.h, n contexts of R rows each (M =
// n * R), their descriptors already in w.rd: the per-layer kernel sequence.
bool partial_path(const q3h_stack *s, int M) {
  return s->cfg.act_q8 && M <= kPartialRows && gemm_i8_chunks(s->cfg.hidden) <= kPartialSlots;
}

void run_layers(const q3h_stack *s, Work &w, int M, int positions, bool fused, hipStream_t st,
                const LayerIO &io) {
  const q3h_stack_config &c = s->cfg;
  const int H = c.hidden, hd = c.head_dim, NQ = c.heads * hd, NKV = c.kv_heads * hd;
  const int I = c.intermediate, ldq = NQ + 2 * NKV;
  const bool kv16 = c.kv_f16 != 0;
  if (partial_path(s, M)) {
    run_layers_partial(s, w, M, fused, io, st);
    return;
  }
  if (f32_slice_path(s, M)) {
    run_layers_f32(s, w, M, positions, fused, io, st);
    return;
  }
  for (int l = 0; l < c.layers; l++) {
    const Layer &L = s->layers[l];
    // RMSNorm + fused q/k/v projection
    linear(s, w, L.qkv, w.h, H, M, L.in_norm, w.qkv, ldq, EPI_STORE, nullptr, st);
    if (c.act_q8) {
      // the int8 path: attention in its fixed order, output quantized for o_proj
      if (!fused)
        launch_qk_rope_append(w.qkv, ldq, w.rd, M, l, c.heads, c.kv_heads, hd, L.q_norm,
                              L.k_norm, c.rms_eps, s->rope_cs, kv16, st);
      AttnArgs at{};
      at.qkv = w.qkv;
      at.ldq = ldq;
      at.rd = w.rd;
      at.layer = l;
      at.heads = c.heads;
      at.kvh = c.kv_heads;
      at.qkn = L.q_norm;
      at.rope_cs = reinterpret_cast<const float2 *>(s->rope_cs);
      launch_attn_x(at, M, fused, kv16, 0, w.xa, c.max_positions, st);
      launch_gemm_i8(L.o, w.xa, M, EPI_ADD, w.h, H, st);
      linear(s, w, L.gu, w.h, H, M, L.post_norm, w.act, I, EPI_SWIGLU, nullptr, st);
      linear(s, w, L.down, w.act, I, M, nullptr, w.h, H, EPI_ADD, nullptr, st);
      probe_layer(io, w, l, M, H, st);
      continue;
    }
    // QK-norm, RoPE, K/V append (in the attention prologue when fused)
    if (!fused)
      launch_qk_rope_append(w.qkv, ldq, w.rd, M, l, c.heads, c.kv_heads, hd, L.q_norm,
                            L.k_norm, c.rms_eps, s->rope_cs, kv16, st);
    // GQA attention
    AttnArgs at{};
    at.qkv = w.qkv;
    at.ldq = ldq;
    at.rd = w.rd;
    at.layer = l;
    at.heads = c.heads;
    at.kvh = c.kv_heads;
    at.qkn = L.q_norm;
    at.rope_cs = reinterpret_cast<const float2 *>(s->rope_cs);
    at.out = w.att;
    at.part = w.part;
    at.layers = c.layers;  // decode: the next layer's cache rows loaded one launch ahead
    if (!fused && io.single_context && M >= kPrefillRows) {
      launch_attn_prefill(at, M, kv16, st);
    } else if (attn_merge_o_supported(at, L.o, M, positions, kv16)) {
      // one decode row over a split context: the splits' merge in the o_proj
      // product (+ residual)
      launch_attn(at, M, positions, fused, kv16, st, false);
      launch_attn_merge_o(at, L.o, w.h, positions, fused, kv16, st);
      linear(s, w, L.gu, w.h, H, M, L.post_norm, w.act, I, EPI_SWIGLU, nullptr, st);
      linear(s, w, L.down, w.act, I, M, nullptr, w.h, H, EPI_ADD, nullptr, st);
      probe_layer(io, w, l, M, H, st);
      continue;
    } else {
      launch_attn(at, M, positions, fused, kv16, st);
    }
    // o_proj + residual
    linear(s, w, L.o, w.att, NQ, M, nullptr, w.h, H, EPI_ADD, nullptr, st);
    // RMSNorm + gate/up + SwiGLU
    linear(s, w, L.gu, w.h, H, M, L.post_norm, w.act, I, EPI_SWIGLU, nullptr, st);
    // down + residual
    linear(s, w, L.down, w.act, I, M, nullptr, w.h, H, EPI_ADD, nullptr, st);
    probe_layer(io, w, l, M, H, st);
  }
}

void run_cp_fused(const q3h_stack *s, Work &w, const q3h_context *ctx, int pos, hipStream_t st,
                  const CodeSrc *src) {
  const q3h_stack_config &c = s->cfg;
  const int H = c.hidden, hd = c.head_dim, NQ = c.heads * hd, NKV = c.kv_heads * hd;
  const int I = c.intermediate, ldq = NQ + 2 * NKV;
  const bool kv16 = c.kv_f16 != 0;
  const size_t per_layer = (size_t)c.kv_heads * ctx->max_pos * hd;  // K/V elements per layer
  const int v_off = (int)(per_layer * c.layers);
  const size_t esz = kv16 ? 2 : 4;
  const float *rope_row = s->rope_cs + (size_t)pos * hd;  // (cos, sin) x head_dim / 2
  for (int l = 0; l < c.layers; l++) {
    const Layer &L = s->layers[l];
    const GemvArgs qa = make_gemv(L.qkv, w.h, H, 1, L.in_norm, c.rms_eps, w.qkv, ldq);
    if (l == 0 && src)
      require(launch_gemv_q8_code(qa, src->logits, src->vocab, src->rows, src->code_out, w.h,
                                  src->alive, st),
              Q3H_E_ARG, "code-predictor input: shape not supported on the device");
    else
      launch_gemv(qa, EPI_STORE, true, st);
    void *kl = static_cast<char *>(ctx->k) + l * per_layer * esz;
    // o_proj as four partials (one per kv-head pair), added with the residual
    // in the gate/up product's prologue, which writes the new h
    launch_attn_o_cp(L.o, w.qkv, kl, v_off, w.h, w.part, L.q_norm, rope_row, pos, kv16, st);
    require(launch_gemv_q8_swiglu_parts(make_gemv(L.gu, w.part, H, 1, L.post_norm, c.rms_eps,
                                                  w.act, I),
                                        w.h, st),
            Q3H_E_ARG, "code-predictor gate/up: shape not supported on the device");
    launch_gemv(make_gemv(L.down, w.act, I, 1, nullptr, 0.f, w.h, H), EPI_ADD, true, st);
  }
}

void run_cp_fused_first(const q3h_stack *s, Work &w, const q3h_context *ctx, hipStream_t st) {
  const q3h_stack_config &c = s->cfg;
  const int H = c.hidden, hd = c.head_dim, NQ = c.heads * hd, NKV = c.kv_heads * hd;
  const int I = c.intermediate, ldq = NQ + 2 * NKV;
  const bool kv16 = c.kv_f16 != 0;
  const size_t per_layer = (size_t)c.kv_heads * ctx->max_pos * hd;
  const int v_off = (int)(per_layer * c.layers);
  const size_t esz = kv16 ? 2 : 4;
  for (int l = 0; l < c.layers; l++) {
    const Layer &L = s->layers[l];
    launch_gemv(make_gemv(L.qkv, w.h, H, 2, L.in_norm, c.rms_eps, w.qkv, ldq), EPI_STORE, true,
                st);
    void *kl = static_cast<char *>(ctx->k) + l * per_layer * esz;
    launch_attn2_o_cp(L.o, w.qkv, ldq, kl, v_off, w.h, L.q_norm, s->rope_cs, kv16, st);
    launch_gemv(make_gemv(L.gu, w.h, H, 2, L.post_norm, c.rms_eps, w.act, I), EPI_SWIGLU, true,
                st);
    launch_gemv(make_gemv(L.down, w.act, I, 2, nullptr, 0.f, w.h, H), EPI_ADD, true, st);
  }
}

GemvArgs make_gemv(const Mat &W, const float *x, int ldx, int M, const float *norm_w,
                   float eps, float *y, int ldy) {
  GemvArgs a{};
  a.wq = W.q;
  a.wd = W.d;
  a.wf = W.f;
  a.N = W.N;
  a.K = W.K;
  a.x = x;
  a.ldx = ldx;
  a.M = M;
  a.norm_w = norm_w;
  a.eps = eps;
  a.y = y;
  a.ldy = ldy;
  a.xn_out = nullptr;
  return a;
}

}  // namespace q3h

// ---------------------------------------------------------------------------
// host Q8_0 quantizer (ggml quantize_row_q8_0_ref semantics)

static uint16_t half_bits(float f) {
  const _Float16 h = (_Float16)f;  // round to nearest even
  uint16_t b;
  std::memcpy(&b, &h, 2);
  return b;
}

extern "C" int q3h_quantize_row_q8_0(const float *x, void *y, int64_t k) {
  return guard([&] {
    require(x && y && k >= 0 && k % 32 == 0, Q3H_E_ARG, "q3h_quantize_row_q8_0: k % 32 != 0");
    uint8_t *out = (uint8_t *)y;
    for (int64_t b = 0; b < k / 32; b++) {
      const float *v = x + b * 32;
      float amax = 0.f;
      for (int j = 0; j < 32; j++) {
        const float a = std::fabs(v[j]);
        amax = amax > a ? amax : a;
      }
      const float d = amax / 127;
      const float id = d != 0.f ? 1.0f / d : 0.f;
      const uint16_t db = half_bits(d);
      out[b * 34] = (uint8_t)(db & 0xff);
      out[b * 34 + 1] = (uint8_t)(db >> 8);
      for (int j = 0; j < 32; j++) out[b * 34 + 2 + j] = (uint8_t)(int8_t)std::round(v[j] * id);
    }
  });
}

// ---------------------------------------------------------------------------
// device

extern "C" const char *q3h_last_error(void) { return g_last_error.c_str(); }

static bool is_gfx950(int ordinal) {
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, ordinal) != hipSuccess) return false;
  return std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
}

extern "C" int q3h_device_available(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  for (int i = 0; i < n; i++)
    if (is_gfx950(i)) return 1;
  return 0;
}

// The work buffers of q3h_forward_embeds_noalloc: one static array, a copy
// per GPU. Host code never uses its name as an address: q3h_device_open
// takes each GPU's address of it (hipGetSymbolAddress) into dev->scratch.
static __device__ __align__(256) unsigned char scratch[Q3H_NOALLOC_SCRATCH_BYTES];

extern "C" int q3h_device_open(int ordinal, q3h_device **out) {
  return guard([&] {
    require(out != nullptr, Q3H_E_ARG, "q3h_device_open: out is NULL");
    *out = nullptr;
    int n = 0;
    require(hipGetDeviceCount(&n) == hipSuccess && n > 0, Q3H_E_NODEV, "no HIP device");
    require(ordinal >= 0 && ordinal < n, Q3H_E_NODEV, "q3h_device_open: no device " +
                                                          std::to_string(ordinal));
    require(is_gfx950(ordinal), Q3H_E_NODEV,
            "q3h_device_open: device " + std::to_string(ordinal) + " is not gfx950");
    check_hip(hipSetDevice(ordinal), "hipSetDevice");
    check_hip(hipFree(nullptr), "hipFree(0)");
    hipDeviceProp_t p;
    check_hip(hipGetDeviceProperties(&p, ordinal), "hipGetDeviceProperties");
    // this GPU's copy of the scratch array (the device is current)
    void *scratch_ptr = nullptr;
    check_hip(hipGetSymbolAddress(&scratch_ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress");
    q3h_device *d = new q3h_device();
    d->ordinal = ordinal;
    d->name = p.name;
    d->cus = p.multiProcessorCount;
    d->scratch = scratch_ptr;
    *out = d;
  });
}

extern "C" const char *q3h_device_name(const q3h_device *dev) {
  return dev ? dev->name.c_str() : nullptr;
}

extern "C" int64_t q3h_device_bytes(const q3h_device *dev) { return dev ? dev->bytes.load() : 0; }

extern "C" int q3h_device_close(q3h_device *dev) {
  return guard([&] {
    require(dev != nullptr, Q3H_E_ARG, "q3h_device_close: NULL device");
    require(dev->stacks.load() == 0, Q3H_E_STATE,
            "q3h_device_close: stacks are still alive on this device");
    delete dev;
  });
}

// ---------------------------------------------------------------------------
// stack

namespace {

size_t src_row_bytes(int src_dtype, int K) {
  return src_dtype == Q3H_Q8_0 ? (size_t)(K / 32) * 34
                               : (size_t)K * (src_dtype == Q3H_BF16 ? 2 : 4);
}

Mat alloc_mat(int N, int K, int dtype, int64_t &bytes) {
  Mat m;
  m.N = N;
  m.K = K;
  if (dtype == Q3H_Q8_0) {
    // one allocation: the quants, then the scales (kernels that take one
    // pointer find the scales at q + N * K)
    m.q = (int8_t *)dev_alloc((size_t)N * K + (size_t)N * (K / 32) * 2);
    m.d = reinterpret_cast<_Float16 *>(m.q + (size_t)N * K);
    bytes += (int64_t)N * (K / 32) * 34;
  } else {
    m.f = (float *)dev_alloc((size_t)N * K * 4);
    bytes += (int64_t)N * K * 4;
  }
  return m;
}

void free_mat(Mat &m) {
  dev_free(m.q);  // the scales share this allocation
  dev_free(m.f);
  dev_free(m.x3);
  m = Mat();
}

// the split-bf16 planes of an f32 layer matrix (the operands of the prefill
// products); their bytes go to aux
void make_x3(Mat &m, int64_t &aux, hipStream_t st) {
  m.x3 = (uint16_t *)dev_alloc((size_t)3 * m.N * m.K * 2);
  aux += (int64_t)3 * m.N * m.K * 2;
  launch_split3(m, st);
  check_hip(hipGetLastError(), "split3");
}

// Upload rows x K of host matrix src (src_dtype) into rows r*stride+off of m.
void upload_rows(Mat &m, int dtype, const void *src, int src_dtype, int rows, int K,
                 int stride, int off, void *staging, hipStream_t st) {
  require(src != nullptr, Q3H_E_ARG, "a weight matrix is NULL");
  const size_t bytes = src_row_bytes(src_dtype, K) * rows;
  check_hip(hipMemcpyAsync(staging, src, bytes, hipMemcpyHostToDevice, st), "upload");
  const bool bf16 = src_dtype == Q3H_BF16;
  if (dtype == Q3H_Q8_0) {
    if (src_dtype == Q3H_Q8_0)
      launch_repack_q8((const uint8_t *)staging, rows, K, m.q, m.d, stride, off, st);
    else
      launch_quantize_q8(staging, bf16, rows, K, m.q, m.d, stride, off, st);
  } else {
    require(src_dtype != Q3H_Q8_0, Q3H_E_ARG, "f32 stacks take f32 or BF16 weights");
    launch_copy_rows_f32(staging, bf16, rows, K, m.f, stride, off, st);
  }
  check_hip(hipGetLastError(), "conversion kernel");
  // the staging buffer is reused by the next matrix
  check_hip(hipStreamSynchronize(st), "upload sync");
}

float *upload_vec(const float *src, int n, const char *what) {
  require(src != nullptr, Q3H_E_ARG, std::string("a norm vector is NULL: ") + what);
  float *d = (float *)dev_alloc(sizeof(float) * n);
  check_hip(hipMemcpy(d, src, sizeof(float) * n, hipMemcpyHostToDevice), "upload norm");
  return d;
}

void destroy_stack(q3h_stack *s) {
  for (auto &L : s->layers) {
    free_mat(L.qkv);
    free_mat(L.o);
    free_mat(L.gu);
    free_mat(L.down);
    dev_free(L.in_norm);
    dev_free(L.post_norm);
    dev_free(L.q_norm);  // k_norm shares this allocation
  }
  for (auto &h : s->heads) free_mat(h);
  dev_free(s->final_norm);
  dev_free(s->rope_cs);
  if (s->stream) (void)hipStreamDestroy(s->stream);
}

}  // namespace

extern "C" int q3h_stack_create(q3h_device *dev, const q3h_stack_config *cfg,
                                const q3h_weights *w, q3h_stack **out) {
  q3h_stack *s = nullptr;
  int rc = guard([&] {
    require(dev && cfg && w && out, Q3H_E_ARG, "q3h_stack_create: NULL argument");
    *out = nullptr;
    const q3h_stack_config &c = *cfg;
    require(c.layers > 0 && c.hidden > 0 && c.heads > 0 && c.kv_heads > 0 && c.head_dim > 0 &&
                c.intermediate > 0,
            Q3H_E_ARG, "q3h_stack_create: non-positive dimension");
    require(c.hidden % 32 == 0 && c.intermediate % 32 == 0 &&
                (c.heads * c.head_dim) % 32 == 0,
            Q3H_E_ARG, "q3h_stack_create: widths must be multiples of 32");
    require(c.hidden % 16 == 0 && c.intermediate % 16 == 0, Q3H_E_ARG,
            "q3h_stack_create: widths must be multiples of 16");
    require(c.heads % c.kv_heads == 0 &&
                (c.heads / c.kv_heads == 1 || c.heads / c.kv_heads == 2 ||
                 c.heads / c.kv_heads == 4),
            Q3H_E_ARG, "q3h_stack_create: heads / kv_heads must be 1, 2 or 4");
    require(c.head_dim == 128, Q3H_E_ARG, "q3h_stack_create: head_dim must be 128");
    require(c.dtype == Q3H_F32 || c.dtype == Q3H_Q8_0, Q3H_E_ARG,
            "q3h_stack_create: dtype must be Q3H_F32 or Q3H_Q8_0");
    require(w->src_dtype == Q3H_F32 || w->src_dtype == Q3H_Q8_0 || w->src_dtype == Q3H_BF16,
            Q3H_E_ARG, "q3h_stack_create: src_dtype must be Q3H_F32, Q3H_Q8_0 or Q3H_BF16");
    require(c.dtype == Q3H_Q8_0 || w->src_dtype != Q3H_Q8_0, Q3H_E_ARG,
            "q3h_stack_create: an f32 stack takes f32 or BF16 weights");
    require(c.max_positions > 0, Q3H_E_ARG, "q3h_stack_create: max_positions <= 0");
    require(c.max_positions <= attn_max_positions(c.kv_f16 != 0), Q3H_E_ARG,
            "q3h_stack_create: max_positions above " +
                std::to_string(attn_max_positions(c.kv_f16 != 0)));
    require(c.act_q8 == 0 || c.dtype == Q3H_Q8_0, Q3H_E_ARG,
            "q3h_stack_create: act_q8 needs Q8_0 weights");
    require(c.act_q8 == 0 ||
                (gemm_i8_supported(c.heads * c.head_dim + 2 * c.kv_heads * c.head_dim, c.hidden) &&
                 gemm_i8_supported(c.hidden, c.heads * c.head_dim) &&
                 gemm_i8_supported(2 * c.intermediate, c.hidden) &&
                 gemm_i8_supported(c.hidden, c.intermediate)),
            Q3H_E_ARG, "q3h_stack_create: act_q8 takes widths up to 3072");
    require(c.act_q8 == 0 ||
                attn_x_supported(c.heads, c.kv_heads, c.head_dim, c.max_positions),
            Q3H_E_ARG,
            "q3h_stack_create: act_q8 takes up to " +
                std::to_string(kAttnXMaxPositions / std::max(1, c.heads / std::max(1, c.kv_heads))) +
                " positions");
    require(w->layers != nullptr && w->final_norm != nullptr, Q3H_E_ARG,
            "q3h_stack_create: NULL layers or final norm");
    check_hip(hipSetDevice(dev->ordinal), "hipSetDevice");
    s = new q3h_stack();
    s->dev = dev;
    s->cfg = c;
    check_hip(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreate");
    const int H = c.hidden, hd = c.head_dim, NQ = c.heads * hd, NKV = c.kv_heads * hd;
    const int I = c.intermediate;
    const int maxK = std::max(std::max(H, NQ), I), maxN = std::max(std::max(NQ, I), H);
    void *staging = dev_alloc(src_row_bytes(w->src_dtype, maxK) * maxN);
    try {
      s->layers.resize(c.layers);
      for (int l = 0; l < c.layers; l++) {
        const q3h_layer_weights &lw = w->layers[l];
        Layer &L = s->layers[l];
        L.qkv = alloc_mat(NQ + 2 * NKV, H, c.dtype, s->bytes);
        L.o = alloc_mat(H, NQ, c.dtype, s->bytes);
        L.gu = alloc_mat(2 * I, H, c.dtype, s->bytes);
        L.down = alloc_mat(H, I, c.dtype, s->bytes);
        upload_rows(L.qkv, c.dtype, lw.wq, w->src_dtype, NQ, H, 1, 0, staging, s->stream);
        upload_rows(L.qkv, c.dtype, lw.wk, w->src_dtype, NKV, H, 1, NQ, staging, s->stream);
        upload_rows(L.qkv, c.dtype, lw.wv, w->src_dtype, NKV, H, 1, NQ + NKV, staging,
                    s->stream);
        upload_rows(L.o, c.dtype, lw.wo, w->src_dtype, H, NQ, 1, 0, staging, s->stream);
        upload_rows(L.gu, c.dtype, lw.wgate, w->src_dtype, I, H, 2, 0, staging, s->stream);
        upload_rows(L.gu, c.dtype, lw.wup, w->src_dtype, I, H, 2, 1, staging, s->stream);
        upload_rows(L.down, c.dtype, lw.wdown, w->src_dtype, H, I, 1, 0, staging, s->stream);
        if (c.dtype == Q3H_F32 && c.max_positions > 64)
          for (Mat *m : {&L.qkv, &L.o, &L.gu, &L.down}) make_x3(*m, s->aux_bytes, s->stream);
        L.in_norm = upload_vec(lw.input_norm, H, "input_layernorm");
        L.post_norm = upload_vec(lw.post_norm, H, "post_attention_layernorm");
        // q_norm and k_norm side by side, then the RMSNorm epsilon:
        // [q_norm | k_norm | eps] (the attention kernels read all three from
        // one pointer)
        require(lw.q_norm != nullptr && lw.k_norm != nullptr, Q3H_E_ARG,
                "a norm vector is NULL: q_norm / k_norm");
        L.q_norm = (float *)dev_alloc(sizeof(float) * (2 * hd + 4));
        L.k_norm = L.q_norm + hd;
        check_hip(hipMemcpy(L.q_norm, lw.q_norm, sizeof(float) * hd, hipMemcpyHostToDevice),
                  "upload q_norm");
        check_hip(hipMemcpy(L.k_norm, lw.k_norm, sizeof(float) * hd, hipMemcpyHostToDevice),
                  "upload k_norm");
        const float eps4[4] = {c.rms_eps, 0.f, 0.f, 0.f};
        check_hip(hipMemcpy(L.q_norm + 2 * hd, eps4, sizeof(eps4), hipMemcpyHostToDevice),
                  "upload eps");
        s->bytes += (int64_t)(2 * H + 2 * hd) * 4;
      }
      s->final_norm = upload_vec(w->final_norm, H, "norm");
      s->bytes += (int64_t)H * 4;
      // RoPE table [max_positions][head_dim/2] of (cos, sin): the fp32 angle
      // pos * inv_freq, its cosine and sine in double rounded to fp32
      const int half = hd / 2;
      std::vector<float> cs((size_t)c.max_positions * half * 2);
      std::vector<float> inv_freq(half);
      for (int i = 0; i < half; i++)
        inv_freq[i] = (float)(1.0 / std::pow((double)c.rope_theta, (double)(2 * i) / (double)hd));
      for (int p = 0; p < c.max_positions; p++)
        for (int i = 0; i < half; i++) {
          const float angle = (float)p * inv_freq[i];
          cs[((size_t)p * half + i) * 2] = (float)std::cos((double)angle);
          cs[((size_t)p * half + i) * 2 + 1] = (float)std::sin((double)angle);
        }
      s->rope_cs = (float *)dev_alloc(sizeof(float) * cs.size());
      check_hip(hipMemcpy(s->rope_cs, cs.data(), sizeof(float) * cs.size(),
                          hipMemcpyHostToDevice),
                "upload rope");
    } catch (...) {
      dev_free(staging);
      throw;
    }
    dev_free(staging);
    dev->bytes += s->bytes + s->aux_bytes;
    dev->stacks++;
    *out = s;
  });
  if (rc != 0 && s) {
    destroy_stack(s);
    delete s;
  }
  return rc;
}

extern "C" int q3h_stack_add_head(q3h_stack *s, const void *w, int rows, int src_dtype,
                                  int *index) {
  return guard([&] {
    require(s && w && index && rows > 0, Q3H_E_ARG, "q3h_stack_add_head: invalid argument");
    require(src_dtype == Q3H_F32 || src_dtype == Q3H_Q8_0 || src_dtype == Q3H_BF16, Q3H_E_ARG,
            "q3h_stack_add_head: src_dtype must be Q3H_F32, Q3H_Q8_0 or Q3H_BF16");
    require(s->cfg.dtype == Q3H_Q8_0 || src_dtype != Q3H_Q8_0, Q3H_E_ARG,
            "q3h_stack_add_head: an f32 stack takes f32 or BF16 heads");
    require(!s->cfg.act_q8 || rows % 16 == 0, Q3H_E_ARG,
            "q3h_stack_add_head: an act_q8 stack takes heads of a multiple of 16 rows");
    check_hip(hipSetDevice(s->dev->ordinal), "hipSetDevice");
    std::lock_guard<std::mutex> lock(s->mu);
    const int H = s->cfg.hidden;
    int64_t bytes = 0;
    Mat m = alloc_mat(rows, H, s->cfg.dtype, bytes);
    void *staging = dev_alloc(src_row_bytes(src_dtype, H) * rows);
    try {
      upload_rows(m, s->cfg.dtype, w, src_dtype, rows, H, 1, 0, staging, s->stream);
    } catch (...) {
      dev_free(staging);
      free_mat(m);
      throw;
    }
    dev_free(staging);
    s->heads.push_back(m);
    s->head_bytes += bytes;
    s->dev->bytes += bytes;
    *index = (int)s->heads.size() - 1;
  });
}

extern "C" int64_t q3h_stack_bytes(const q3h_stack *s) { return s ? s->bytes : 0; }

extern "C" int q3h_stack_destroy(q3h_stack *s) {
  return guard([&] {
    require(s != nullptr, Q3H_E_ARG, "q3h_stack_destroy: NULL stack");
    require(s->contexts.load() == 0, Q3H_E_STATE,
            "q3h_stack_destroy: contexts or frames still use this stack");
    check_hip(hipSetDevice(s->dev->ordinal), "hipSetDevice");
    s->dev->bytes -= s->bytes + s->head_bytes + s->aux_bytes;
    s->dev->stacks--;
    destroy_stack(s);
    delete s;
  });
}

// ---------------------------------------------------------------------------
// context

namespace q3h {

q3h_context *new_context(q3h_stack *s, int max_positions) {
  const q3h_stack_config &c = s->cfg;
  q3h_context *ctx = new q3h_context();
  ctx->s = s;
  ctx->max_pos = max_positions;
  try {
    check_hip(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking), "hipStreamCreate");
    const size_t n = (size_t)c.layers * c.kv_heads * max_positions * c.head_dim;
    const size_t esz = c.kv_f16 ? 2 : 4;
    // keys then values in one allocation: v = k + n elements
    ctx->k = dev_alloc(2 * n * esz);
    ctx->v = static_cast<char *>(ctx->k) + n * esz;
    // zeros: a position is finite before it is first written (the long-context
    // attention reads rows past the context with weight 0)
    check_hip(hipMemset(ctx->k, 0, 2 * n * esz), "zero K/V");
    ctx->dev = (CtxDev *)dev_alloc(sizeof(CtxDev));
    ctx->dev_arr = (CtxDev **)dev_alloc(sizeof(CtxDev *));
    CtxDev h{ctx->k, ctx->v, max_positions, 0};
    check_hip(hipMemcpy(ctx->dev, &h, sizeof(h), hipMemcpyHostToDevice), "ctx init");
    check_hip(hipMemcpy(ctx->dev_arr, &ctx->dev, sizeof(CtxDev *), hipMemcpyHostToDevice),
              "ctx init");
  } catch (...) {
    free_context(ctx);
    throw;
  }
  s->contexts++;
  return ctx;
}

void drop_graphs(q3h_context *ctx) {
  for (auto &g : ctx->graphs) (void)hipGraphExecDestroy(g.second);
  ctx->graphs.clear();
}

void free_context(q3h_context *ctx) {
  drop_graphs(ctx);
  ctx->w.release();
  if (ctx->pin) (void)hipHostFree(ctx->pin);
  dev_free(ctx->probe);
  dev_free(ctx->k);  // the values share this allocation
  dev_free(ctx->dev);
  dev_free(ctx->dev_arr);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

void set_len(q3h_context *c, int len, hipStream_t st) {
  check_hip(hipMemcpyAsync(&c->dev->len, &len, sizeof(int), hipMemcpyHostToDevice, st),
            "set length");
  check_hip(hipStreamSynchronize(st), "set length sync");
  c->len = len;
}

}  // namespace q3h

extern "C" int q3h_context_create(q3h_stack *s, int max_positions, q3h_context **out) {
  return guard([&] {
    require(s && out, Q3H_E_ARG, "q3h_context_create: NULL argument");
    *out = nullptr;
    require(max_positions > 0 && max_positions <= s->cfg.max_positions, Q3H_E_ARG,
            "q3h_context_create: max_positions must be in [1, " +
                std::to_string(s->cfg.max_positions) + "]");
    check_hip(hipSetDevice(s->dev->ordinal), "hipSetDevice");
    *out = new_context(s, max_positions);
  });
}

extern "C" int q3h_context_reset(q3h_context *c) {
  return guard([&] {
    require(c != nullptr, Q3H_E_ARG, "q3h_context_reset: NULL context");
    check_hip(hipSetDevice(c->s->dev->ordinal), "hipSetDevice");
    set_len(c, 0, c->stream);
  });
}

extern "C" int q3h_context_length(const q3h_context *c) {
  if (!c) {
    g_last_error = "q3h_context_length: NULL context";
    return Q3H_E_ARG;
  }
  return c->len;
}

extern "C" int q3h_context_destroy(q3h_context *c) {
  return guard([&] {
    require(c != nullptr, Q3H_E_ARG, "q3h_context_destroy: NULL context");
    check_hip(hipSetDevice(c->s->dev->ordinal), "hipSetDevice");
    check_hip(hipStreamSynchronize(c->stream), "context sync");
    c->s->contexts--;
    free_context(c);
  });
}

extern "C" int q3h_context_fill_kv(q3h_context *c, const float *k, const float *v, int len) {
  return guard([&] {
    require(c && k && v, Q3H_E_ARG, "q3h_context_fill_kv: NULL argument");
    require(len >= 0 && len <= c->max_pos, Q3H_E_CAPACITY,
            "q3h_context_fill_kv: length beyond the context");
    const q3h_stack_config &cf = c->s->cfg;
    check_hip(hipSetDevice(c->s->dev->ordinal), "hipSetDevice");
    const size_t n = (size_t)cf.layers * cf.kv_heads * len * cf.head_dim;
    if (n > 0) {
      float *st = (float *)dev_alloc(n * sizeof(float));
      try {
        for (int which = 0; which < 2; which++) {
          check_hip(hipMemcpyAsync(st, which ? v : k, n * sizeof(float), hipMemcpyHostToDevice,
                                   c->stream),
                    "fill kv upload");
          launch_kv_fill(st, cf.layers, cf.kv_heads, len, cf.head_dim, which ? c->v : c->k,
                         c->max_pos, cf.kv_f16 != 0, c->stream);
          check_hip(hipGetLastError(), "kv fill kernel");
          check_hip(hipStreamSynchronize(c->stream), "fill kv sync");
        }
      } catch (...) {
        dev_free(st);
        throw;
      }
      dev_free(st);
    }
    set_len(c, len, c->stream);
  });
}

extern "C" int q3h_context_read_kv(q3h_context *c, int layer, float *k, float *v) {
  return guard([&] {
    require(c && k && v, Q3H_E_ARG, "q3h_context_read_kv: NULL argument");
    const q3h_stack_config &cf = c->s->cfg;
    require(layer >= 0 && layer < cf.layers, Q3H_E_ARG, "q3h_context_read_kv: bad layer");
    check_hip(hipSetDevice(c->s->dev->ordinal), "hipSetDevice");
    const size_t n = (size_t)cf.kv_heads * c->len * cf.head_dim;
    if (n == 0) return;
    float *st = (float *)dev_alloc(n * sizeof(float));
    try {
      for (int which = 0; which < 2; which++) {
        launch_kv_read(which ? c->v : c->k, layer, cf.kv_heads, c->len, cf.head_dim, c->max_pos,
                       cf.kv_f16 != 0, st, c->stream);
        check_hip(hipGetLastError(), "kv read kernel");
        check_hip(hipMemcpyAsync(which ? v : k, st, n * sizeof(float), hipMemcpyDeviceToHost,
                                 c->stream),
                  "kv read download");
        check_hip(hipStreamSynchronize(c->stream), "kv read sync");
      }
    } catch (...) {
      dev_free(st);
      throw;
    }
    dev_free(st);
  });
}

extern "C" int q3h_context_time_attention(q3h_context *c, int iters, float *us_per_launch,
                                          int64_t *bytes_per_launch) {
  Work w;
  hipStream_t st = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;  // around the timed passes
  int rc = guard([&] {
    require(c && us_per_launch && bytes_per_launch && iters > 0, Q3H_E_ARG,
            "q3h_context_time_attention: invalid argument");
    q3h_stack *s = c->s;
    const q3h_stack_config &cf = s->cfg;
    require(!cf.act_q8, Q3H_E_ARG,
            "q3h_context_time_attention: a stack with f32 activations is required");
    require(c->len + 1 <= c->max_pos, Q3H_E_CAPACITY, "q3h_context_time_attention: context full");
    check_hip(hipSetDevice(s->dev->ordinal), "hipSetDevice");
    const int positions = c->len + 1;
    const int NQ = cf.heads * cf.head_dim, NKV = cf.kv_heads * cf.head_dim;
    const int ldq = NQ + 2 * NKV;
    const bool kv16 = cf.kv_f16 != 0;
    w.ensure(s, 1, attention_splits(s, positions), 0);
    check_hip(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
    check_hip(hipMemsetAsync(w.qkv, 0, sizeof(float) * ldq, st), "zero");
    launch_prep(c->dev_arr, nullptr, 1, 1, w.rd, st);
    AttnArgs at{};
    at.qkv = w.qkv;
    at.ldq = ldq;
    at.rd = w.rd;
    at.heads = cf.heads;
    at.kvh = cf.kv_heads;
    at.rope_cs = reinterpret_cast<const float2 *>(s->rope_cs);
    at.out = w.att;
    at.part = w.part;
    check_hip(hipEventCreate(&e0), "event");
    check_hip(hipEventCreate(&e1), "event");
    // the layers' attention launches, direct, on one stream: the time between
    // two events around iters passes counts the gaps between launches too
    auto pass = [&] {
      for (int l = 0; l < cf.layers; l++) {
        at.layer = l;
        at.qkn = s->layers[l].q_norm;
        launch_attn(at, 1, positions, true, kv16, st);
      }
    };
    pass();  // warm-up
    check_hip(hipStreamSynchronize(st), "warm-up sync");
    check_hip(hipEventRecord(e0, st), "event record");
    for (int it = 0; it < iters; it++) pass();
    check_hip(hipEventRecord(e1, st), "event record");
    check_hip(hipEventSynchronize(e1), "timed sync");
    float ms = 0.f;
    check_hip(hipEventElapsedTime(&ms, e0, e1), "elapsed");
    const double total = ms;
    check_hip(hipGetLastError(), "attention kernels");
    *us_per_launch = (float)(total * 1000.0 / ((double)iters * cf.layers));
    const int64_t es = kv16 ? 2 : 4;
    // the cache read for len positions, the new key and value written, the
    // q / k / v row read, the head outputs written
    *bytes_per_launch = 2 * es * (int64_t)NKV * c->len + 2 * es * NKV + 4 * (int64_t)ldq +
                        4 * (int64_t)NQ;
  });
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (st) {
    (void)hipStreamSynchronize(st);
    (void)hipStreamDestroy(st);
  }
  w.release();
  return rc;
}

// ---------------------------------------------------------------------------
// forward

namespace {

// the checks of q3h_forward_embeds (false: rows <= 0, nothing to do)
bool forward_args(const q3h_context *c, const float *x, int rows, int head, const char *who) {
  require(c != nullptr, Q3H_E_ARG, std::string(who) + ": NULL context");
  if (rows <= 0) return false;
  require(x != nullptr, Q3H_E_ARG, std::string(who) + ": x is NULL");
  const q3h_stack *s = c->s;
  require(head >= -1 && head < (int)s->heads.size(), Q3H_E_ARG,
          std::string(who) + ": no head " + std::to_string(head));
  require(c->len + rows <= c->max_pos, Q3H_E_CAPACITY,
          std::string(who) + ": " + std::to_string(c->len) + " + " + std::to_string(rows) +
              " positions exceed the context's " + std::to_string(c->max_pos));
  return true;
}

// the positions a forward of `rows` rows launches for: one row, the graph
// cover of its length (so the captured single-row forward and the direct one
// run the same launches); more rows, their exact count
int forward_positions(const q3h_context *c, int rows) {
  return rows == 1 ? graph_cover(c->len + 1, c->max_pos) : c->len + rows;
}

// the attention splits whose partials a forward of `rows` rows keeps: none on
// an int8 stack (its attention quantizes its output directly) or over
// kPrefillRows rows or more (the causal prefill attention), else those of the
// decode attention over forward_positions
int forward_splits(const q3h_context *c, int rows) {
  if (c->s->cfg.act_q8 || rows >= kPrefillRows) return 0;
  return attention_splits(c->s, forward_positions(c, rows));
}

// the kernels of a forward: descriptors, layers, head (or final norm), the
// device length
void enqueue_forward(q3h_context *c, Work &w, int rows, int positions, int head,
                     const LayerIO &io, hipStream_t st) {
  q3h_stack *s = c->s;
  const q3h_stack_config &cf = s->cfg;
  const int H = cf.hidden;
  const int head_rows = head >= 0 ? s->heads[head].N : 0;
  launch_prep(c->dev_arr, nullptr, 1, rows, w.rd, st);
  run_layers(s, w, rows, positions, rows == 1, st, io);
  // final norm of the last row, fused into the head product when there is one
  if (head >= 0) {
    linear(s, w, s->heads[head], w.h + (size_t)(rows - 1) * H, H, 1, s->final_norm, w.logits,
           head_rows, EPI_STORE, w.normed, st);
  } else {
    launch_rmsnorm_rows(w.h + (size_t)(rows - 1) * H, H, 1, H, s->final_norm, cf.rms_eps,
                        w.normed, H, st);
  }
  launch_advance(c->dev_arr, nullptr, 1, rows, st);
}

// the captured single-row forward of (head, cover) on c's Work buffers
hipGraphExec_t forward_graph(q3h_context *c, int head, int positions) {
  constexpr size_t kMaxGraphs = 32;  // per context: a code predictor's heads, a talker's covers
  if (c->graphs_gen != c->w.gen || c->graphs.size() >= kMaxGraphs) {
    drop_graphs(c);
    c->graphs_gen = c->w.gen;
  }
  const uint64_t key = ((uint64_t)(uint32_t)(head + 1) << 32) | (uint32_t)positions;
  for (auto &g : c->graphs)
    if (g.first == key) return g.second;
  LayerIO io;
  io.single_context = true;
  hipGraph_t graph =
      capture_graph(c->stream, [&] { enqueue_forward(c, c->w, 1, positions, head, io, c->stream); });
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  check_hip(e, "forward graph instantiate");
  c->graphs.push_back({key, exec});
  return exec;
}

// TQwenLm.Forward on the work buffers w (sized for rows, the attention splits
// of forward_positions and the head's rows), replayed from a captured graph
// when graph: blocks until the outputs are in host memory
void forward_rows(q3h_context *c, Work &w, const float *x, int rows, int head, float *logits,
                  float *normed_last, float *layer_out = nullptr, bool graph = false,
                  float *normed_rows = nullptr) {
  q3h_stack *s = c->s;
  const q3h_stack_config &cf = s->cfg;
  const int H = cf.hidden;
  const int head_rows = head >= 0 ? s->heads[head].N : 0;
  const int positions = forward_positions(c, rows);
  hipStream_t st = c->stream;
  // the replayed single-row forward copies through pinned host memory (a
  // pageable copy is staged by the runtime on every call)
  float *pin_x = nullptr, *pin_lg = nullptr, *pin_n = nullptr;
  if (graph) {
    const size_t need = (size_t)2 * H + head_rows;
    if (c->pin_floats < need) {
      if (c->pin) check_hip(hipHostFree(c->pin), "hipHostFree");
      c->pin = nullptr;
      c->pin_floats = 0;
      check_hip(hipHostMalloc((void **)&c->pin, sizeof(float) * need, hipHostMallocDefault),
                "hipHostMalloc");
      c->pin_floats = need;
    }
    pin_x = c->pin;
    pin_n = c->pin + H;
    pin_lg = c->pin + 2 * H;
    std::memcpy(pin_x, x, sizeof(float) * H);
    x = pin_x;
  }
  check_hip(hipMemcpyAsync(w.h, x, sizeof(float) * rows * H, hipMemcpyHostToDevice, st),
            "upload x");
  LayerIO io;
  io.single_context = true;
  // the probe's device buffer: the layer outputs [layers][rows][hidden], then
  // the final-normed rows [rows][hidden]
  const size_t layer_floats = (size_t)cf.layers * rows * H;
  const size_t probe_bytes = sizeof(float) * (layer_floats + (size_t)rows * H);
  if (layer_out || normed_rows) {
    if (c->probe_bytes < probe_bytes) {
      check_hip(hipStreamSynchronize(st), "probe sync");
      dev_free(c->probe);
      c->probe = nullptr;
      c->probe_bytes = 0;
      c->probe = (float *)dev_alloc(probe_bytes);
      c->probe_bytes = probe_bytes;
    }
    if (layer_out) io.layer_out = c->probe;
  }
  if (graph)
    check_hip(hipGraphLaunch(forward_graph(c, head, positions), st), "forward graph launch");
  else
    enqueue_forward(c, w, rows, positions, head, io, st);
  // the final RMSNorm of every row (the probe's "norm" state, lm.pas:383-384)
  if (normed_rows)
    launch_rmsnorm_rows(w.h, H, rows, H, s->final_norm, cf.rms_eps, c->probe + layer_floats, H,
                        st);
  check_hip(hipGetLastError(), "forward kernels");
  if (normed_last)
    check_hip(hipMemcpyAsync(graph ? pin_n : normed_last, w.normed, sizeof(float) * H,
                             hipMemcpyDeviceToHost, st),
              "download state");
  if (logits && head >= 0)
    check_hip(hipMemcpyAsync(graph ? pin_lg : logits, w.logits, sizeof(float) * head_rows,
                             hipMemcpyDeviceToHost, st),
              "download logits");
  if (layer_out)
    check_hip(hipMemcpyAsync(layer_out, c->probe, sizeof(float) * layer_floats,
                             hipMemcpyDeviceToHost, st),
              "download layer outputs");
  if (normed_rows)
    check_hip(hipMemcpyAsync(normed_rows, c->probe + layer_floats, sizeof(float) * rows * H,
                             hipMemcpyDeviceToHost, st),
              "download normed rows");
  check_hip(hipStreamSynchronize(st), "forward sync");
  if (graph) {
    if (normed_last) std::memcpy(normed_last, pin_n, sizeof(float) * H);
    if (logits && head >= 0) std::memcpy(logits, pin_lg, sizeof(float) * head_rows);
  }
  c->len += rows;
}

}  // namespace

extern "C" int q3h_forward_embeds(q3h_context *c, const float *x, int rows, int head,
                                  float *logits, float *normed_last) {
  return guard([&] {
    if (!forward_args(c, x, rows, head, "q3h_forward_embeds")) return;
    q3h_stack *s = c->s;
    check_hip(hipSetDevice(s->dev->ordinal), "hipSetDevice");
    const int head_rows = head >= 0 ? s->heads[head].N : 0;
    c->w.ensure(s, rows, forward_splits(c, rows), head_rows);
    // one row (a decode step): the forward replayed from a captured graph
    forward_rows(c, c->w, x, rows, head, logits, normed_last, nullptr, rows == 1);
  });
}

extern "C" int q3h_forward_embeds_probe(q3h_context *c, const float *x, int rows, int head,
                                        float *logits, float *normed_last, float *layer_out,
                                        float *normed_rows) {
  return guard([&] {
    if (!forward_args(c, x, rows, head, "q3h_forward_embeds_probe")) return;
    q3h_stack *s = c->s;
    check_hip(hipSetDevice(s->dev->ordinal), "hipSetDevice");
    const int head_rows = head >= 0 ? s->heads[head].N : 0;
    c->w.ensure(s, rows, forward_splits(c, rows), head_rows);
    forward_rows(c, c->w, x, rows, head, logits, normed_last, layer_out, false, normed_rows);
  });
}

extern "C" int q3h_forward_embeds_noalloc(q3h_context *c, const float *x, int rows, int head,
                                          float *logits, float *normed_last) {
  return guard([&] {
    if (!forward_args(c, x, rows, head, "q3h_forward_embeds_noalloc")) return;
    require(rows <= Q3H_NOALLOC_MAX_ROWS, Q3H_E_CAPACITY,
            "q3h_forward_embeds_noalloc: " + std::to_string(rows) + " rows exceed " +
                std::to_string(Q3H_NOALLOC_MAX_ROWS));
    q3h_stack *s = c->s;
    q3h_device *dev = s->dev;
    require(dev->scratch != nullptr, Q3H_E_STATE,
            "q3h_forward_embeds_noalloc: the device has no scratch array");
    const int head_rows = head >= 0 ? s->heads[head].N : 0;
    Work w;  // a view of the array: owns nothing
    require(work_carve(s, rows, forward_splits(c, rows), head_rows,
                       dev->scratch, Q3H_NOALLOC_SCRATCH_BYTES, w),
            Q3H_E_CAPACITY,
            "q3h_forward_embeds_noalloc: the work buffers of " + std::to_string(rows) +
                " rows at " + std::to_string(c->len + rows) + " positions exceed the " +
                std::to_string(Q3H_NOALLOC_SCRATCH_BYTES) + "-byte scratch array");
    std::lock_guard<std::mutex> lk(dev->scratch_mu);
    check_hip(hipSetDevice(dev->ordinal), "hipSetDevice");
    forward_rows(c, w, x, rows, head, logits, normed_last);
  });
}

extern "C" int q3h_forward_embeds_batch(q3h_context *const *ctxs, int n, const float *x,
                                        const int *heads, float *logits, float *normed) {
  return guard([&] {
    require(ctxs && n > 0 && x, Q3H_E_ARG, "q3h_forward_embeds_batch: invalid argument");
    q3h_context *c0 = ctxs[0];
    require(c0 != nullptr, Q3H_E_ARG, "q3h_forward_embeds_batch: NULL context");
    q3h_stack *s = c0->s;
    const q3h_stack_config &cf = s->cfg;
    int maxlen = 0;
    for (int i = 0; i < n; i++) {
      require(ctxs[i] && ctxs[i]->s == s, Q3H_E_ARG,
              "q3h_forward_embeds_batch: contexts of different stacks");
      for (int j = 0; j < i; j++)
        require(ctxs[j] != ctxs[i], Q3H_E_ARG, "q3h_forward_embeds_batch: repeated context");
      require(ctxs[i]->len + 1 <= ctxs[i]->max_pos, Q3H_E_CAPACITY,
              "q3h_forward_embeds_batch: a context is full");
      maxlen = std::max(maxlen, ctxs[i]->len + 1);
    }
    int head_rows = 0;
    if (heads) {
      for (int i = 0; i < n; i++)
        require(heads[i] >= 0 && heads[i] < (int)s->heads.size(), Q3H_E_ARG,
                "q3h_forward_embeds_batch: bad head index");
      head_rows = s->heads[heads[0]].N;
      for (int i = 0; i < n; i++)
        require(s->heads[heads[i]].N == head_rows, Q3H_E_ARG,
                "q3h_forward_embeds_batch: heads of different sizes");
    }
    check_hip(hipSetDevice(s->dev->ordinal), "hipSetDevice");
    for (int i = 1; i < n; i++) check_hip(hipStreamSynchronize(ctxs[i]->stream), "batch sync");
    const int H = cf.hidden;
    Work &w = c0->w;
    w.ensure(s, n, attention_splits(s, maxlen), head_rows);
    hipStream_t st = c0->stream;
    std::vector<CtxDev *> arr(n);
    for (int i = 0; i < n; i++) arr[i] = ctxs[i]->dev;
    check_hip(hipMemcpyAsync(w.ctx_arr, arr.data(), sizeof(CtxDev *) * n, hipMemcpyHostToDevice,
                             st),
              "upload contexts");
    check_hip(hipMemcpyAsync(w.h, x, sizeof(float) * n * H, hipMemcpyHostToDevice, st),
              "upload x");
    launch_prep(w.ctx_arr, nullptr, n, 1, w.rd, st);
    run_layers(s, w, n, maxlen, true, st);
    launch_rmsnorm_rows(w.h, H, n, H, s->final_norm, cf.rms_eps, w.normed, H, st);
    if (heads) {
      bool same = true;
      for (int i = 1; i < n; i++) same = same && heads[i] == heads[0];
      if (same) {
        linear(s, w, s->heads[heads[0]], w.normed, H, n, nullptr, w.logits, head_rows,
               EPI_STORE, nullptr, st);
      } else {
        for (int i = 0; i < n; i++)
          linear(s, w, s->heads[heads[i]], w.normed + (size_t)i * H, H, 1, nullptr,
                 w.logits + (size_t)i * head_rows, head_rows, EPI_STORE, nullptr, st);
      }
    }
    launch_advance(w.ctx_arr, nullptr, n, 1, st);
    check_hip(hipGetLastError(), "batch kernels");
    if (normed)
      check_hip(hipMemcpyAsync(normed, w.normed, sizeof(float) * n * H, hipMemcpyDeviceToHost,
                               st),
                "download states");
    if (logits && heads)
      check_hip(hipMemcpyAsync(logits, w.logits, sizeof(float) * n * head_rows,
                               hipMemcpyDeviceToHost, st),
                "download logits");
    check_hip(hipStreamSynchronize(st), "batch sync");
    for (int i = 0; i < n; i++) ctxs[i]->len += 1;
  });
}

// ---------------------------------------------------------------------------
// measurement: the weight products of one decode step, graph-replayed

extern "C" int q3h_stack_time_gemv(q3h_stack *s, int head, int iters, int mode,
                                   float *us_per_launch, int *launches, int64_t *bytes) {
  Work w;
  hipStream_t st = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  std::vector<hipEvent_t> kev;  // mode 2: a start and an end event per launch
  int rc = guard([&] {
    require(s && us_per_launch && launches && bytes && iters > 0, Q3H_E_ARG,
            "q3h_stack_time_gemv: invalid argument");
    require(mode >= 0 && mode <= 2, Q3H_E_ARG, "q3h_stack_time_gemv: mode must be 0, 1 or 2");
    require(head >= -1 && head < (int)s->heads.size(), Q3H_E_ARG,
            "q3h_stack_time_gemv: no head " + std::to_string(head));
    check_hip(hipSetDevice(s->dev->ordinal), "hipSetDevice");
    const q3h_stack_config &c = s->cfg;
    const int H = c.hidden, NQ = c.heads * c.head_dim, NKV = c.kv_heads * c.head_dim;
    const int I = c.intermediate, ldq = NQ + 2 * NKV;
    const bool q8 = c.dtype == Q3H_Q8_0;
    require(mode != 2 || q8, Q3H_E_ARG,
            "q3h_stack_time_gemv: kernel-attached timing needs a Q8_0 stack");
    const int head_rows = head >= 0 ? s->heads[head].N : 0;
    w.ensure(s, 1, 1, head_rows);
    check_hip(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
    check_hip(hipMemsetAsync(w.h, 0, sizeof(float) * H, st), "zero");
    check_hip(hipMemsetAsync(w.att, 0, sizeof(float) * NQ, st), "zero");
    check_hip(hipMemsetAsync(w.act, 0, sizeof(float) * I, st), "zero");
    check_hip(hipMemsetAsync(w.normed, 0, sizeof(float) * H, st), "zero");
    check_hip(hipStreamSynchronize(st), "zero sync");
    auto mat_bytes = [&](const Mat &m) {
      return q8 ? (int64_t)m.N * (m.K / 32) * 34 : (int64_t)m.N * m.K * 4;
    };
    // the products of one step, in order, with their algorithmic bytes
    struct Op {
      GemvArgs a;
      int epi;
    };
    std::vector<Op> ops;
    int64_t b = 0;
    for (int l = 0; l < c.layers; l++) {
      const Layer &L = s->layers[l];
      ops.push_back({make_gemv(L.qkv, w.h, H, 1, L.in_norm, c.rms_eps, w.qkv, ldq), EPI_STORE});
      ops.push_back({make_gemv(L.o, w.att, NQ, 1, nullptr, 0.f, w.h, H), EPI_ADD});
      ops.push_back({make_gemv(L.gu, w.h, H, 1, L.post_norm, c.rms_eps, w.act, I), EPI_SWIGLU});
      ops.push_back({make_gemv(L.down, w.act, I, 1, nullptr, 0.f, w.h, H), EPI_ADD});
      b += mat_bytes(L.qkv) + mat_bytes(L.o) + mat_bytes(L.gu) + mat_bytes(L.down);
      // norm vectors, inputs read, outputs written (the residual adds read y too)
      b += 4 * (int64_t)(2 * H) + 4 * (int64_t)(H + ldq) + 4 * (int64_t)(NQ + 2 * H) +
           4 * (int64_t)(H + I) + 4 * (int64_t)(I + 2 * H);
    }
    if (head >= 0) {
      ops.push_back(
          {make_gemv(s->heads[head], w.normed, H, 1, nullptr, 0.f, w.logits, head_rows), EPI_STORE});
      b += mat_bytes(s->heads[head]) + 4 * (int64_t)(H + head_rows);
    }
    const int n = (int)ops.size();
    auto enqueue = [&](bool timed) {
      for (int i = 0; i < n; i++) {
        if (timed)
          require(launch_gemv_q8_wide(ops[i].a, ops[i].epi, st, kev[2 * i], kev[2 * i + 1]),
                  Q3H_E_ARG, "q3h_stack_time_gemv: a product outside the single-row kernel");
        else
          launch_gemv(ops[i].a, ops[i].epi, q8, st);
      }
    };
    check_hip(hipEventCreate(&e0), "event");
    check_hip(hipEventCreate(&e1), "event");
    float ms = 0.f;
    if (mode == 2) {
      kev.assign(2 * n, nullptr);
      for (auto &e : kev) check_hip(hipEventCreate(&e), "event");
      enqueue(true);  // warm-up
      check_hip(hipStreamSynchronize(st), "warm-up sync");
      double total = 0.0;
      for (int it = 0; it < iters; it++) {
        enqueue(true);
        check_hip(hipStreamSynchronize(st), "timed sync");
        for (int i = 0; i < n; i++) {
          float t = 0.f;
          check_hip(hipEventElapsedTime(&t, kev[2 * i], kev[2 * i + 1]), "elapsed");
          total += t;
        }
      }
      ms = (float)total;
    } else {
      if (mode == 1) {
        graph = capture_graph(st, [&] { enqueue(false); });
        check_hip(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate");
      }
      auto once = [&] {
        if (mode == 1)
          check_hip(hipGraphLaunch(exec, st), "graph launch");
        else
          enqueue(false);
      };
      for (int i = 0; i < 2; i++) once();
      check_hip(hipEventRecord(e0, st), "event record");
      for (int i = 0; i < iters; i++) once();
      check_hip(hipEventRecord(e1, st), "event record");
      check_hip(hipEventSynchronize(e1), "event sync");
      check_hip(hipEventElapsedTime(&ms, e0, e1), "elapsed");
    }
    check_hip(hipGetLastError(), "gemv kernels");
    *us_per_launch = ms * 1000.f / ((float)iters * n);
    *launches = n;
    *bytes = b;
  });
  for (auto e : kev)
    if (e) (void)hipEventDestroy(e);
  if (e0) (void)hipEventDestroy(e0);
  if (e1) (void)hipEventDestroy(e1);
  if (exec) (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
  if (st) {
    (void)hipStreamSynchronize(st);
    (void)hipStreamDestroy(st);
  }
  w.release();
  return rc;
}
