// q3h_internal.h - device data structures and kernel launchers of libq3h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace q3h {

// A matrix [N][K] on the device: Q8_0 as int8 quants [N][K] followed, in the
// same allocation, by the fp16 scales [N][K/32] (d == q + N*K; structure of
// arrays, so a wave reads 1 KB of quants per instruction), or f32 [N][K].
struct Mat {
  int N = 0, K = 0;
  int8_t *q = nullptr;
  _Float16 *d = nullptr;
  float *f = nullptr;
  // f32 matrices of stacks that prefill many rows: the same values as three
  // bf16 planes [3][N][K] (w = hi + mid + lo exactly), the operands of the
  // split-bf16 matrix-core products (null: not made)
  uint16_t *x3 = nullptr;
};

// Per-row view of a K/V cache for the attention kernels. k, v: the cache of
// layer 0, [layers][kv_heads][max_pos][head_dim] in f32 or f16 (one
// allocation: v = k + layers*kv_heads*max_pos*head_dim elements); pos: the
// position of the row (it attends to [0, pos]); pos < 0: inactive row.
struct RowDesc {
  void *k;
  void *v;
  int max_pos;
  int pos;
};

// p as a pointer the compiler knows to be in device (global) memory. Pointers
// read from memory (row descriptors, frame state) otherwise stay generic and
// their accesses become flat loads / stores, which also count in lgkmcnt: a
// wait for an LDS or scalar access then waits for them as well.
template <typename T>
__device__ __forceinline__ T *global_ptr(T *p) {
  return (T *)(__attribute__((address_space(1))) T *)(uintptr_t)p;
}

// x stored at the K/V cache's precision: its fp32 value rounded to KV. For a
// half cache an empty asm keeps the compiler from folding the operation that
// produced x (a RoPE fused multiply-add, a sum) into a mixed-precision
// instruction that rounds once, straight to half, which can differ in the
// last place
template <typename KV>
__device__ __forceinline__ KV to_cache(float x) {
  if constexpr (sizeof(KV) == 2) asm volatile("" : "+v"(x));
  return (KV)x;
}

// Context state that kernels read and advance on the device.
struct CtxDev {
  void *k;
  void *v;
  int max_pos;
  int len;
};

// EPI_PART (f32 matrix-core products only): sums to a slice of a partial buffer
// EPI_ADD_SILU (f32 matrix-core products, f32 weights): y = SiLU(y + sum),
// 0 where y + sum < -80 (the text projection's fc1, its bias in y)
enum Epi { EPI_STORE = 0, EPI_ADD = 1, EPI_SWIGLU = 2, EPI_PART = 3, EPI_ADD_SILU = 4 };

struct GemvArgs {
  const int8_t *wq;
  const _Float16 *wd;
  const float *wf;
  int N, K;
  const float *x;  // [M][ldx]
  int ldx, M;
  const float *norm_w;  // RMSNorm prologue over each x row when non-null
  float eps;
  float *y;  // [M][ldy]
  int ldy;
  float *xn_out;  // optional: the (normed) last x row, [K], written by block 0
};

// Activations quantized per 32-block for the int8 products, M rows padded to
// Mp = M rounded up to 16, one buffer: the int8 values at q in MFMA operand
// order (qtile_offset), then the fp16-rounded block scales [Mp][K/32] as f32
// at q + Mp * K (qact_bytes(M, K) in all).
struct QAct {
  int8_t *q = nullptr;
};
// byte of element (m, k) (mt16 = Mp / 16): 16-row tiles per pair of 32-blocks
// b = k / 32 = 2p + h, each 64 lanes x 16 bytes; lane g * 16 + m % 16, g =
// (k % 32) / 8, holds elements 32b + 8g .. + 7 of row m at bytes 8h .. 8h + 7,
// so one 16-byte load per lane gives the B operands of two blocks
__host__ __device__ inline size_t qtile_offset(int m, int k, int mt16) {
  const int b = k >> 5, g = (k & 31) >> 3;
  return ((((size_t)(b >> 1) * mt16 + (m >> 4)) * 64 + g * 16 + (m & 15)) * 16) + (b & 1) * 8 +
         (k & 7);
}
size_t qact_bytes(int M, int K);

void launch_gemv(const GemvArgs &a, int epi, bool q8, hipStream_t st);
// the wide Q8_0 kernel (K in {1024, 2048, 3072}, N % 256 == 0, M <= 4);
// false when the shape is not one it takes (nothing launched)
bool launch_gemv_q8_wide(const GemvArgs &a, int epi, hipStream_t st, hipEvent_t ev0 = nullptr,
                         hipEvent_t ev1 = nullptr);
// the RMSNorm + gate/up + SwiGLU product of one row given as four partial
// rows [4][K] at a.x (the code predictor's o_proj partials per kv-head pair),
// added as (p0 + p1) + (p2 + p3); workgroup 0 writes the row to x_out. False
// when the shape is not one of these kernels' (gemv_q8_parts_supported).
bool gemv_q8_parts_supported(int N, int K);
bool launch_gemv_q8_swiglu_parts(const GemvArgs &a, float *x_out, hipStream_t st);
// the single-row product with an RMSNorm prologue (M == 1, K == 1024, N a
// multiple of 1024 up to 4096) over row `code` of rows [vocab][K], code = the
// argmax of logits [vocab] (vocab 2048 or 3072; the smallest index among
// equal maxima); when *alive, the code goes to *code_out and the raw row to
// h_out [K]. false when the shape is not one it takes (nothing launched)
bool launch_gemv_q8_code(const GemvArgs &a, const float *logits, int vocab, const float *rows,
                         int *code_out, float *h_out, const int *alive, hipStream_t st);
// the f32 matrix-core products (q3h_gemm_f32.hip): y[m][n] (+)= W[n] . x[m]
// for f32 W [N][K] (N % 16 == 0, K in {1024, 2048, 3072}); epi EPI_* (SwiGLU:
// interleaved gate / up rows, y [M][N / 2])
// (Q8_0 weights, f32 activations: the same products on the bf16 matrix cores,
// the quants exact in bf16 and the activations split exactly into three bf16
// parts; taken for more than kGemvRows rows)
bool gemm_f32_supported(int N, int K);
// the three bf16 planes of m.f into m.x3 (allocated by the caller)
void launch_split3(const Mat &m, hipStream_t st);
constexpr int kGemvRows = 4;
void launch_gemm_f32(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy,
                     hipStream_t st);
// the same with K cut into slices, one workgroup per (16 rows, slice): the
// slices' sums go to part [slices][M][N] (fills the chip when N / 16 is
// small). f32 weights: kF32Slices slices. Q8_0 weights over 17 to
// kQ8SliceRows rows: slices of 256 columns (K / 256 of them: 1-4, 6, 8 or
// 12; 32 weight rows per workgroup), each workgroup then splitting
// a quarter or less of the rows' activations (48 rows: q/k/v 11.1 -> 7.3 us,
// o_proj 7.9 -> 5.3 us, down 9.7 -> 7.2 us); kF32Slices slices otherwise.
// Returns the slice count.
constexpr int kF32Slices = 4;
constexpr int kQ8SliceRows = 64;
constexpr int kMaxPartSlices = 12;  // the most 256-column slices of a product
bool gemm_f32_slices_supported(int N, int K);
int launch_gemm_f32_part(const Mat &W, const float *x, int ldx, int M, float *part,
                         hipStream_t st);
// K / 256 when W takes the 256-column slices over M rows, else 0
int q8x_slices(const Mat &W, int M);
// h [M][K] += the `slices` slices of part (1-4, 6, 8 or 12), in slice order; then,
// when norm_w != nullptr, xn [M][K] = RMSNorm(h) with norm_w (double sum of
// squares)
void launch_resid_norm(float *h, const float *part, int M, int K, const float *norm_w,
                       float eps, float *xn, int slices, hipStream_t st);
// the int8 path (q3h_gemm.hip): shapes it takes (N % 16 == 0, K % 256 == 0,
// K <= 3072)
bool gemm_i8_supported(int N, int K);
// rows x [M][ldx] (RMS-normed with norm_w when non-null) quantized into out;
// xn_out, when non-null, receives the (normed) row M - 1
void launch_quantize_act(const float *x, int ldx, int M, int K, const float *norm_w, float eps,
                         QAct out, float *xn_out, hipStream_t st);
// y [M][ldy] (+)= W . x over the quantized rows xa (Q8_0 W)
void launch_gemm_i8(const Mat &W, const QAct &xa, int M, int epi, float *y, int ldy,
                    hipStream_t st);
// the same chains for M <= kPartialRows, one wave per (16 rows, chunk):
// part[gemm_i8_chunks(K)][M][N], to be added in chunk order by the consumer
constexpr int kPartialRows = 64;
// chunk partials a consumer of the batched products' partials reads (the
// attention prologue, the code predictor's argmax): the chunks of a K of
// at most 1024
constexpr int kPartialSlots = 2;
// rows from which a one-context forward takes the matrix-core prefill attention
constexpr int kPrefillRows = 16;
int gemm_i8_chunks(int K);
void launch_gemm_i8_partial(const Mat &W, const QAct &xa, int M, float *part, hipStream_t st);
// h [M][K] += the chunk partials of a product (in chunk order); then RMSNorm
// with norm_w (when non-null; every normed row also into normed [M][K] when
// that is non-null) and quantization into *out (when non-null)
void launch_residual_quantize(float *h, const float *part, int chunks, int M, int K,
                              const float *norm_w, float eps, const QAct *out, hipStream_t st,
                              float *normed = nullptr);
// the gate/up product, silu(gate) * up and its quantization into out in one
// launch (M <= 64, K == 1024, N % 64 == 0; out must not alias xa); false
// when the shape is not one it takes (nothing launched)
bool launch_gemm_i8_swiglu_quantize(const Mat &W, const QAct &xa, int M, QAct out,
                                    hipStream_t st);
// silu(gate) * up from the chunk partials (chunks <= 4) of the gate/up
// product (N = 2K), quantized into out
void launch_swiglu_quantize(const float *part, int chunks, int M, int K, QAct out,
                            hipStream_t st);

// rows of n contexts, R consecutive rows each (R > 1: one context's prefill)
void launch_prep(CtxDev *const *cs, const int *alive, int n, int R, RowDesc *rd,
                 hipStream_t st);
void launch_advance(CtxDev *const *cs, const int *alive, int n, int R, hipStream_t st);

// part != nullptr: the q/k/v rows are the sum of nsl <= kRopeMaxSlices K-slice
// partials part [nsl][M][ldq], added in slice order (the normed and rotated q
// heads still go to qkv)
constexpr int kRopeMaxSlices = 4;
void launch_qk_rope_append(float *qkv, int ldq, const RowDesc *rd, int M, int layer,
                           int heads, int kvh, int hd, const float *qn, const float *kn,
                           float eps, const float *rope_cs, bool kv16, hipStream_t st,
                           const float *part = nullptr, int nsl = 0);

// decode attention (q3h_attn.hip): rows m of qkv [M][ldq] with descriptors
// rd; fused: each row is the one new position of its own context (QK-norm,
// RoPE and the K/V append in the prologue); otherwise q is already normed and
// rotated in qkv and the cache holds every position (launch_qk_rope_append).
struct AttnArgs {
  const float *qkv;
  int ldq;
  const RowDesc *rd;
  int layer, heads, kvh;
  const float *qkn;  // [q_norm | k_norm | eps] of the layer
  const float2 *rope_cs;
  float *out;    // [M][heads * head_dim]
  float *part;   // [M][heads][attn_splits slots][head_dim + 2]
  int layers;    // > layer + 1: a decode launch also loads layer + 1's cache rows ahead
};
// how the decode attention cuts contexts of up to `positions` positions: len
// positions per split (a multiple of 16), threads per workgroup (0: one
// workgroup per query head over at most 256 positions, no split); fold: the
// splits are merged by the o_proj product (launch_attn_merge_o), which
// re-reads every split's partials in each of its workgroups, so it takes the
// longest splits while they number at most kMergeOMaxSplits
struct SplitShape {
  int len, threads;
};
SplitShape attn_split_shape(int positions, bool kv16, bool fold = false);
// partial-buffer slots per (row, query head): the splits and the query head
// (1 when one workgroup covers the context)
int attn_splits(int positions, bool kv16);
// the most slots any context of up to `positions` positions needs
int attn_splits_upto(int positions, bool kv16);
// prefill attention on the matrix cores: the M rows of one context at
// positions rd[0].pos + m, their K/V already appended, q normed and rotated
void launch_attn_prefill(const AttnArgs &a, int M, bool kv16, hipStream_t st);
// the most positions the split kernel merges (splits per kv head are bounded)
int attn_max_positions(bool kv16);
// positions: the most positions any of the M rows attends to (its own
// included). Returns the kernels launched (1, or 2 with the split merge).
// merge == false: the split kernel alone when the context is split (its
// partials left for launch_attn_merge_o; the fold shape)
int launch_attn(const AttnArgs &a, int M, int positions, bool fused, bool kv16, hipStream_t st,
                bool merge = true);
// one decode row's o_proj (Q8_0 W_o [N][16 x 128]) with the split attention's
// merge in its prologue: y [N] += W_o x, x merged from a.part (the split
// kernel of launch_attn(..., merge = false) launched before); for contexts
// cut into at most kMergeOMaxSplits splits (the caller checks
// attn_merge_o_supported). Every workgroup reads all the splits' partials, so
// the fold gains less as splits are added: 15 splits 5.2 us against 3.7 + 3.2
// us for the merge and the o_proj product, 29 splits 7.5 us against 3.6 + 3.2
constexpr int kMergeOMaxSplits = 24;
bool attn_merge_o_supported(const AttnArgs &a, const Mat &wo, int M, int positions, bool kv16);
void launch_attn_merge_o(const AttnArgs &a, const Mat &wo, float *y, int positions, bool fused,
                         bool kv16, hipStream_t st);

// attention of the int8 path (q3h_attnx.hip): the rows of a (fused: each the
// one new position of its own context, QK-norm / RoPE / K/V append in the
// prologue), outputs quantized into xa for the o_proj product; positions up
// to kAttnXMaxPositions / (heads / kv_heads) (the scores of a kv group held
// in LDS). qkv_chunks in 1..kPartialSlots (fused only):
// a.qkv holds the chunk partials [qkv_chunks][M][a.ldq] of the q/k/v product
// instead of its rows, added in chunk order in the prologue. pairs (fused,
// attn_x_pairs_supported): the rows come in pairs, row 2i + 1 at the position
// after row 2i's in the same context (the code predictor's first step).
constexpr int kAttnXMaxPositions = 8192;
bool attn_x_supported(int heads, int kvh, int head_dim, int max_positions);
bool attn_x_pairs_supported(int max_positions);
void launch_attn_x(const AttnArgs &a, int M, bool fused, bool kv16, int qkv_chunks,
                   const QAct &xa, int max_positions, hipStream_t st, bool pairs = false);

// the code predictor's fused attention + o_proj (q3h_cp.hip): one context
// of 16 positions, the new row at pos; k_layer: the layer's keys, values at
// k_layer + v_off elements; qkn: [q_norm | k_norm | eps]; rope_row: the
// (cos, sin) row of pos. Writes part [4][1024]: the o_proj partial of each
// kv-head pair, h added to the first (their sum, in the order
// launch_gemv_q8_swiglu_parts takes, is h + o_proj)
void launch_attn_o_cp(const Mat &wo, const float *qkv, void *k_layer, int v_off, const float *h,
                      float *part, const float *qkn, const float *rope_row, int pos, bool kv16,
                      hipStream_t st);

// the same for the first step of a code-predictor context: its two rows at
// positions 0 and 1 (qkv rows ldq apart, h rows [2][1024], rope_rows the
// (cos, sin) rows of positions 0 and 1), no cached positions read
void launch_attn2_o_cp(const Mat &wo, const float *qkv, int ldq, void *k_layer, int v_off,
                       float *h, const float *qkn, const float *rope_rows, bool kv16,
                       hipStream_t st);

// y [M][ldy] = RMSNorm of the rows x [M][ldx] with w (double sum of
// squares)
void launch_rmsnorm_rows(const float *x, int ldx, int M, int K, const float *w, float eps,
                         float *y, int ldy, hipStream_t st);

// weight conversion at load: src rows of K f32 (or BF16 when bf16) values
void launch_quantize_q8(const void *src, bool bf16, int rows, int K, int8_t *q, _Float16 *d,
                        int row_stride, int row_off, hipStream_t st);
void launch_repack_q8(const uint8_t *blocks, int rows, int K, int8_t *q, _Float16 *d,
                      int row_stride, int row_off, hipStream_t st);
void launch_copy_rows_f32(const void *src, bool bf16, int rows, int K, float *dst,
                          int row_stride, int row_off, hipStream_t st);
void launch_kv_fill(const float *src, int layers, int kvh, int len, int hd, void *dst,
                    int max_pos, bool kv16, hipStream_t st);
void launch_kv_read(const void *src, int layer, int kvh, int len, int hd, int max_pos,
                    bool kv16, float *dst, hipStream_t st);

// frame step kernels
struct FrameDev;
void launch_choose_code0(FrameDev *fd, int n, hipStream_t st);
void launch_cp_argmax(FrameDev *fd, int n, int g, hipStream_t st);
void launch_talker_input(FrameDev *fd, int n, hipStream_t st);
void launch_frame_end(FrameDev *fd, int n, hipStream_t st);

}  // namespace q3h
