// q3h_gemm.hip - the int8 path of the Q8_0 products (stacks created with
// act_q8 = 1): activations are quantized per 32-block with the weights' own
// quantizer (ggml quantize_row_q8_0_ref: d = amax / 127, q = round(x / d)
// half away from zero, d kept as fp16; the format of lm.pas:259-267), then
// every Q8_0 block of the product is one v_mfma_i32_16x16x32_i8 whose exact
// int32 dot is scaled by d_w * d_x into an fp32 sum (ggml
// vec_dot_q8_0_q8_0).
//
// Evaluation order (fixed, so that the products equal a CPU evaluation in the
// same order to the bit): per output, one fused multiply-add chain over the
// 16 blocks of each 512-column chunk, acc = fma((float)dot_b, d_w * d_x, acc)
// from 0 in block order, and the chunk sums added in chunk order.
//
// Operand layouts (v_mfma_i32_16x16x32_i8, wave64): lane l holds 8 int8 of
// row l % 16 of A and of column l % 16 of B, k = 8 * (l / 16) .. + 7; the
// result C[4 * (l / 16) + r][l % 16], r < 4, lands in lane l. A is 16 weight
// rows of the row-major Q8_0 matrix; B is 16 activation rows, which the
// quantizers write already in operand order (qtile_offset), so one coalesced
// 1 KB load gives the B operands of two blocks.
//
// Two schedules of the same chains:
//  - k_gemm_i8: a workgroup per 16 weight rows, its waves taking the chunks
//    and adding them through LDS; any number of rows (prefill);
//  - k_gemm_i8p (up to 64 rows, the batched decode step): one wave per (16
//    weight rows, chunk) over the whole chip, the chunk sums written out as
//    partials that the consumer adds in chunk order (k_quant_act with a
//    partial source, or the attention prologue).
#include "q3h_internal.h"
#include "q3h_math.h"
#include "q3h_wave.h"

namespace q3h {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kQuantThreads = 128;
constexpr int kQuantChunks = 3;  // 8-element chunks per thread: K <= 3072
constexpr int kChunkBlocks = 16;  // 32-blocks per chunk of a product (512 columns)
constexpr int kMaxChunks = 6;     // chunks of a product: K <= 3072

__device__ __forceinline__ float *scales_of(int8_t *xq, int M, int K) {
  return reinterpret_cast<float *>(xq + (size_t)((M + 15) & ~15) * K);
}

// The quantizer. One workgroup per activation row m < Mp and slice of its
// 8-element chunks (gridDim.x == Mp, M rounded up to 16; gridDim.y == nsl
// slices): a thread owns chunks j = blockIdx.y * 128 + t + i * 128 * nsl, and the
// four chunks of a lane quad make one 32-block. Rows M..Mp-1 are written as
// zeros. The row is
//  SRC_X:      x[m][0..K) (row stride ld);
//  SRC_ADD:    x[m] + sum_c part[c][m] (c < ld <= kMaxChunks chunk partials
//              of a product with N = K, added in chunk order), written back
//              to x (the residual stream, row stride K);
//  SRC_SWIGLU: silu(sum_c part[c][m][2k]) * sum_c part[c][m][2k + 1] (c < ld
//              <= 2 partials; gate / up interleaved, N = 2K).
// Then RMSNorm when norm_w != nullptr (one slice only): y = w * (x * inv),
// inv = 1/sqrt(mean(x^2) + eps) with the sum of squares in double; xn_out,
// when non-null, receives the (normed) rows M - xn_rows .. M - 1 (row
// M - xn_rows + r at xn_out + r K); and the Q8_0 blocks
// (skipped when xq == nullptr). Partial loads are all issued before the sums.
enum { SRC_X = 0, SRC_ADD = 1, SRC_SWIGLU = 2 };

// KC: chunks per thread (the row's chunks / (128 slices), rounded up); NC: the
// partial slots read (ld <= NC; SRC_ADD and SRC_SWIGLU). The arguments the
// loads depend on (the slice count among them, instead of gridDim) sit in the
// first 14 dwords, which arrive preloaded in SGPRs; xn_out, used only at the
// end, comes last.
template <int SRC, int KC, int NC>
__global__ __launch_bounds__(kQuantThreads) void k_quant_act(float *x, const float *part,
                                                              int8_t *xq, const float *norm_w,
                                                              int M, int K, int ld, float eps,
                                                              int nsl, float *xn_out,
                                                              int xn_rows) {
  const int m = blockIdx.x, t = threadIdx.x;
  const int mt16 = (M + 15) >> 4, nch = K >> 3, nb = K >> 5;
  const int j0 = blockIdx.y * kQuantThreads + t, js = kQuantThreads * nsl;
  float *dx = xq ? scales_of(xq, M, K) : nullptr;
  if (m >= M) {
    if (xq)
      for (int j = j0; j < nch; j += js) {
        *reinterpret_cast<long *>(xq + qtile_offset(m, 8 * j, mt16)) = 0;
        if ((j & 3) == 0) dx[(size_t)m * nb + (j >> 2)] = 0.f;
      }
    return;
  }
  // the norm weights of this thread's chunks, loaded first (they are read by
  // every row, so they come from L2 before the partials arrive)
  float4 wpre[KC][2];
  if (norm_w) {
    const float4 *wr = reinterpret_cast<const float4 *>(norm_w);
#pragma unroll
    for (int i = 0; i < KC; i++) {
      const int jc = min(j0 + i * js, nch - 1);
      wpre[i][0] = wr[2 * jc];
      wpre[i][1] = wr[2 * jc + 1];
    }
  }
  // loads from clamped chunk / partial indices (a guarded load would be waited
  // for on its own); chunks past the row and partials past ld contribute zeros
  float v[KC][8];
#pragma unroll
  for (int i = 0; i < KC; i++) {
    const int j = j0 + i * js, jc = min(j, nch - 1);
    const bool on = j < nch;
    if (SRC == SRC_X) {
      const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)m * ld);
      const float4 a = xr[2 * jc], b = xr[2 * jc + 1];
      const float x8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; e++) v[i][e] = on ? x8[e] : 0.f;
    } else if (SRC == SRC_ADD) {
      float4 pa[NC], pb[NC];
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const float4 *pr =
            reinterpret_cast<const float4 *>(part + ((size_t)min(c, ld - 1) * M + m) * K);
        pa[c] = pr[2 * jc];
        pb[c] = pr[2 * jc + 1];
      }
      float4 *xr = reinterpret_cast<float4 *>(x + (size_t)m * K);
      const float4 a = xr[2 * jc], b = xr[2 * jc + 1];
      float s[8];
#pragma unroll
      for (int e = 0; e < 8; e++) s[e] = 0.f;
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const float p8[8] = {pa[c].x, pa[c].y, pa[c].z, pa[c].w,
                             pb[c].x, pb[c].y, pb[c].z, pb[c].w};
#pragma unroll
        for (int e = 0; e < 8; e++) s[e] = c < ld ? __fadd_rn(s[e], p8[e]) : s[e];
      }
      const float h8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; e++) v[i][e] = on ? __fadd_rn(h8[e], s[e]) : 0.f;
      if (on) {
        xr[2 * j] = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
        xr[2 * j + 1] = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
      }
    } else {
      constexpr int MC = NC;
      float4 pr[MC][4];
#pragma unroll
      for (int c = 0; c < MC; c++) {
        const float4 *pp =
            reinterpret_cast<const float4 *>(part + ((size_t)min(c, ld - 1) * M + m) * (2 * K)) +
            4 * jc;
#pragma unroll
        for (int q = 0; q < 4; q++) pr[c][q] = pp[q];
      }
      float gs[8], us[8];
#pragma unroll
      for (int e = 0; e < 8; e++) gs[e] = us[e] = 0.f;
#pragma unroll
      for (int c = 0; c < MC; c++) {
        if (c >= ld) break;  // uniform
#pragma unroll
        for (int q = 0; q < 4; q++) {  // gate, up of outputs 8j + 2q, 8j + 2q + 1
          gs[2 * q] = __fadd_rn(gs[2 * q], pr[c][q].x);
          us[2 * q] = __fadd_rn(us[2 * q], pr[c][q].y);
          gs[2 * q + 1] = __fadd_rn(gs[2 * q + 1], pr[c][q].z);
          us[2 * q + 1] = __fadd_rn(us[2 * q + 1], pr[c][q].w);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; e++) v[i][e] = on ? silu_mul_ieee(gs[e], us[e]) : 0.f;
    }
  }
  if (norm_w) {
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < KC; i++)
#pragma unroll
      for (int e = 0; e < 8; e++) ss += (double)v[i][e] * (double)v[i][e];
    ss = wave_sum_dpp_d(ss);
    __shared__ double red[kQuantThreads / 64];
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    ss = red[0] + red[1];
    const float inv = (float)(1.0 / sqrt(ss / K + (double)eps));
#pragma unroll
    for (int i = 0; i < KC; i++) {
      const int j = j0 + i * js;
      if (j < nch) {
        const float4 a = wpre[i][0], b = wpre[i][1];
        const float w8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; e++) v[i][e] = w8[e] * (v[i][e] * inv);
      }
    }
  }
  if (xn_out && m >= M - xn_rows) {
    float4 *xo = reinterpret_cast<float4 *>(xn_out + (size_t)(m - (M - xn_rows)) * K);
#pragma unroll
    for (int i = 0; i < KC; i++) {
      const int j = j0 + i * js;
      if (j < nch) {
        xo[2 * j] = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
        xo[2 * j + 1] = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
      }
    }
  }
  if (!xq) return;
#pragma unroll
  for (int i = 0; i < KC; i++) {
    const int j = j0 + i * js;
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[i][e]));
    // nch and the slice starts are multiples of 4, so a quad is wholly inside
    // or outside the row
    amax = quad_max_dpp(amax);
    if (j >= nch) continue;
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.f ? __fdiv_rn(1.0f, d) : 0.f;
    unsigned long long packed = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int q = (int)roundf(__fmul_rn(v[i][e], id));
      packed |= (unsigned long long)(uint8_t)(int8_t)q << (8 * e);
    }
    *reinterpret_cast<long *>(xq + qtile_offset(m, 8 * j, mt16)) = (long)packed;
    if ((j & 3) == 0) dx[(size_t)m * nb + (j >> 2)] = (float)(_Float16)d;
  }
}

// The fused multiply-add chains over NB blocks from their operands, continuing
// acc: A av[i] (16 weight rows), B bv[t][i] (16 activation rows of tile t),
// the weight scales of the lane's 4 rows dwv[r][i] and the activation scales
// of its row dxv[t][i]: acc[t][r] = fma((float)dot, d_w * d_x, acc) in block
// order.
template <int TM, int NB>
__device__ __forceinline__ void chains(const long (&av)[NB], const long (&bv)[TM][NB],
                                       const float (&dwv)[4][NB], const float (&dxv)[TM][NB],
                                       float (&acc)[TM][4]) {
#pragma unroll
  for (int i = 0; i < NB; i++) {
#pragma unroll
    for (int t = 0; t < TM; t++) {
      const v4i ci =
          __builtin_amdgcn_mfma_i32_16x16x32_i8(av[i], bv[t][i], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; r++)
        acc[t][r] = fmaf((float)ci[r], __fmul_rn(dwv[r][i], dxv[t][i]), acc[t][r]);
    }
  }
}

// The chains of NB blocks (b0 .. b0 + NB - 1, K % 512 == 0), continuing acc,
// for 16 weight rows from n0 and the activation tiles mt0 .. mt0 + TM - 1:
// acc[t][r] = output (n0 + 4 (lane / 16) + r, 16 (mt0 + t) + lane % 16); a
// tile past the last (mt16) repeats the last one and its outputs are not
// stored. All loads are unconditional and issued before the first MFMA (a
// guarded load would make the compiler wait for each one). LDSA: the weight
// tile is read with 16-byte loads (4 rows x 256 bytes per instruction instead
// of 16 rows x 32 bytes) and rearranged through the wave's own 16 x (4 NB + 1)
// longs of LDS (at).
template <int TM, bool LDSA, int NB>
__device__ __forceinline__ void chunk_chains(const int8_t *wq, const int8_t *xq, const float *dx,
                                             int N, int K, int n0, int mt0, int mt16, int b0,
                                             long (*at)[4 * NB + 1], float (&acc)[TM][4]) {
  static_assert(NB % 8 == 0, "whole 8-block groups");
  constexpr int NH = NB / 8;  // 256-byte pieces of a weight row
  const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int nb = K >> 5;
  const _Float16 *wd = reinterpret_cast<const _Float16 *>(wq + (size_t)N * K);
  const int4 *xq16 = reinterpret_cast<const int4 *>(xq);
  long av[NB], bv[TM][NB];
  float dwv[4][NB], dxv[TM][NB];
  int4 araw[4 * NH];
  if (LDSA) {
#pragma unroll
    for (int i = 0; i < 4; i++)  // rows 4i + lane / 16, bytes 256 h + 16 (lane % 16) of the chunk
#pragma unroll
      for (int h = 0; h < NH; h++)
        araw[i * NH + h] = *reinterpret_cast<const int4 *>(
            wq + (size_t)(n0 + 4 * i + (lane >> 4)) * K + b0 * 32 + 256 * h + 16 * (lane & 15));
  } else {
    const int8_t *wr = wq + (size_t)(n0 + c) * K + 8 * g;
#pragma unroll
    for (int i = 0; i < NB; i++) av[i] = *reinterpret_cast<const long *>(wr + 32 * (b0 + i));
  }
#pragma unroll
  for (int t = 0; t < TM; t++) {
    const int tt = min(mt0 + t, mt16 - 1);
#pragma unroll
    for (int q = 0; q < NB / 2; q++) {  // blocks b0 + 2q, b0 + 2q + 1
      const int4 v = xq16[((size_t)((b0 >> 1) + q) * mt16 + tt) * 64 + lane];
      bv[t][2 * q] = ((long)(unsigned)v.y << 32) | (unsigned)v.x;
      bv[t][2 * q + 1] = ((long)(unsigned)v.w << 32) | (unsigned)v.z;
    }
  }
#pragma unroll
  for (int r = 0; r < 4; r++)
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const uint4 u =
          *reinterpret_cast<const uint4 *>(wd + (size_t)(n0 + 4 * g + r) * nb + b0 + 8 * h);
      const unsigned uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        dwv[r][8 * h + 2 * i] = (float)__builtin_bit_cast(_Float16, (unsigned short)(uw[i] & 0xffff));
        dwv[r][8 * h + 2 * i + 1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(uw[i] >> 16));
      }
    }
#pragma unroll
  for (int t = 0; t < TM; t++) {
    const int tt = min(mt0 + t, mt16 - 1);
    const float4 *dp = reinterpret_cast<const float4 *>(dx + (size_t)(tt * 16 + c) * nb + b0);
#pragma unroll
    for (int q = 0; q < NB / 4; q++) {
      const float4 p = dp[q];
      dxv[t][4 * q] = p.x, dxv[t][4 * q + 1] = p.y, dxv[t][4 * q + 2] = p.z, dxv[t][4 * q + 3] = p.w;
    }
  }
  if (LDSA) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int h = 0; h < NH; h++) {
        const int row = 4 * i + (lane >> 4), l2 = 32 * h + 2 * (lane & 15);
        at[row][l2] = ((long)(unsigned)araw[i * NH + h].y << 32) | (unsigned)araw[i * NH + h].x;
        at[row][l2 + 1] = ((long)(unsigned)araw[i * NH + h].w << 32) | (unsigned)araw[i * NH + h].z;
      }
    // the wave reads back only what it wrote itself (LDS keeps a wave's order)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < NB; i++) av[i] = at[c][4 * i + g];  // row c, bytes 32 i + 8 g
  }
  __builtin_amdgcn_sched_barrier(0);
  chains<TM, NB>(av, bv, dwv, dxv, acc);
}

// y[m][n] (+)= sum_b d_w[n][b] d_x[m][b] sum_{k in b} q_w[n][k] q_x[m][k].
// A workgroup owns 16 weight rows (blockIdx.x) and TM 16-column activation
// tiles (blockIdx.y); its KW waves take the chunks in turn, each chunk's
// chains land in their own LDS slot, and the slots are added in chunk order.
// EPI_SWIGLU: rows 2j / 2j + 1 are gate / up of output j.
template <int TM, int KW, int EPI>
__global__ __launch_bounds__(KW * 64) void k_gemm_i8(const int8_t *wq, const int8_t *xq,
                                                      float *y, int N, int K, int M, int ldy) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int nb = K >> 5, nch = nb / kChunkBlocks;
  const int mt16 = (M + 15) >> 4;
  const int n0 = blockIdx.x * 16, mt0 = blockIdx.y * TM;
  const float *dx = scales_of(const_cast<int8_t *>(xq), M, K);
  constexpr int LD = TM * 16 + 4;
  __shared__ float red[kMaxChunks][16][LD];
  for (int ch = w; ch < nch; ch += KW) {
    // a chunk's chain as two passes of 8 blocks (the second continues it):
    // TM tiles of 16 blocks would not fit the registers
    float acc[TM][4];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[t][r] = 0.f;
    chunk_chains<TM, false, 8>(wq, xq, dx, N, K, n0, mt0, mt16, ch * kChunkBlocks, nullptr, acc);
    chunk_chains<TM, false, 8>(wq, xq, dx, N, K, n0, mt0, mt16, ch * kChunkBlocks + 8, nullptr,
                               acc);
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) red[ch][4 * g + r][t * 16 + c] = acc[t][r];
  }
  __syncthreads();
  if (EPI == EPI_SWIGLU) {
    for (int idx = threadIdx.x; idx < TM * 16 * 8; idx += KW * 64) {
      const int ml = idx >> 3, p = idx & 7, m = mt0 * 16 + ml;
      float gs = 0.f, us = 0.f;
      for (int v = 0; v < nch; v++) {
        gs = __fadd_rn(gs, red[v][2 * p][ml]);
        us = __fadd_rn(us, red[v][2 * p + 1][ml]);
      }
      if (m < M) y[(size_t)m * ldy + (n0 >> 1) + p] = silu_mul_ieee(gs, us);
    }
  } else {
    for (int idx = threadIdx.x; idx < TM * 16 * 16; idx += KW * 64) {
      const int ml = idx >> 4, nl = idx & 15, m = mt0 * 16 + ml;
      float s = 0.f;
      for (int v = 0; v < nch; v++) s = __fadd_rn(s, red[v][nl][ml]);
      if (m < M) {
        float *yp = y + (size_t)m * ldy + n0 + nl;
        if (EPI == EPI_ADD)
          *yp = __fadd_rn(*yp, s);
        else
          *yp = s;
      }
    }
  }
}

// One wave per (16 weight rows, chunk, TM activation tiles from TM z):
// part[chunk][m][n] = the chunk's chains. The waves of one (weight rows,
// chunk) over the row tiles are gridDim.x * gridDim.y workgroups apart (a
// multiple of 8 for the Qwen3-TTS shapes), so they run on one XCD and share
// the weight tile through its L2.
template <int TM>
__global__ __launch_bounds__(64) void k_gemm_i8p(const int8_t *wq, const int8_t *xq,
                                                  float *part, int N, int K, int M) {
  const int lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int n0 = blockIdx.x * 16, ch = blockIdx.y, mt0 = blockIdx.z * TM;
  const int mt16 = (M + 15) >> 4;
  const float *dx = scales_of(const_cast<int8_t *>(xq), M, K);
  __shared__ long at[16][4 * kChunkBlocks + 1];
  float acc[TM][4];
#pragma unroll
  for (int t = 0; t < TM; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) acc[t][r] = 0.f;
  chunk_chains<TM, true, kChunkBlocks>(wq, xq, dx, N, K, n0, mt0, mt16, ch * kChunkBlocks, at,
                                       acc);
#pragma unroll
  for (int t = 0; t < TM; t++) {
    const int m = (mt0 + t) * 16 + c;
    if (m < M)
      *reinterpret_cast<float4 *>(part + ((size_t)ch * M + m) * N + n0 + 4 * g) =
          make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
  }
}

// The gate/up product with SiLU(gate) * up and the quantization of the result
// fused: a workgroup owns 64 gate/up rows, i.e. one 32-block of the output,
// its 2 chunks (a wave per (16 rows, chunk), K == 1024) and the TM 16-row
// activation tiles from TM blockIdx.y; the chunk chains meet in LDS and are
// added in chunk order, then each row's block is quantized into yq (yq must
// not alias xq). The same values as k_gemm_i8p followed by
// k_quant_act<SRC_SWIGLU>. The workgroups of one output block over the row
// tiles are gridDim.x apart (a multiple of 8 for the Qwen3-TTS shapes: one
// XCD, one L2 for the weights).
template <int TM>
__global__ __launch_bounds__(512) void k_gemm_i8_swq(const int8_t *wq, const int8_t *xq,
                                                     int8_t *yq, int N, int M) {
  constexpr int K = 1024, LD = TM * 16 + 4, NCH = K / (32 * kChunkBlocks);
  __shared__ float red[NCH][64][LD];
  __shared__ long at[4 * NCH][16][4 * kChunkBlocks + 1];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int mt16 = (M + 15) >> 4, mt0 = blockIdx.y * TM;
  const int tile = w & 3, ch = w >> 2;  // 16-row tile of the 64, chunk
  const int n0 = blockIdx.x * 64 + tile * 16;
  const float *dx = scales_of(const_cast<int8_t *>(xq), M, K);
  float acc[TM][4];
#pragma unroll
  for (int t = 0; t < TM; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) acc[t][r] = 0.f;
  chunk_chains<TM, true, kChunkBlocks>(wq, xq, dx, N, K, n0, mt0, mt16, ch * kChunkBlocks, at[w],
                                       acc);
#pragma unroll
  for (int t = 0; t < TM; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) red[ch][tile * 16 + 4 * g + r][t * 16 + c] = acc[t][r];
  __syncthreads();
  // output block b = blockIdx.x of this workgroup's rows, 32 lanes per row
  const int KO = N >> 1, nbo = KO >> 5, b = blockIdx.x;
  float *dy = scales_of(yq, M, KO);
  const int nrow = min(TM, mt16 - mt0) * 16;
  for (int idx = threadIdx.x; idx < nrow * 32; idx += 64 * 4 * NCH) {
    const int ml = idx >> 5, j = idx & 31, m = mt0 * 16 + ml;
    float o = 0.f;
    if (m < M) {
      float gs = 0.f, us = 0.f;
#pragma unroll
      for (int v = 0; v < NCH; v++) {
        gs = __fadd_rn(gs, red[v][2 * j][ml]);
        us = __fadd_rn(us, red[v][2 * j + 1][ml]);
      }
      o = silu_mul_ieee(gs, us);
    }
    float amax = fabsf(o);
    amax = half_max_dpp(amax);
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.f ? __fdiv_rn(1.0f, d) : 0.f;
    yq[qtile_offset(m, 32 * b + j, mt16)] = (int8_t)(int)roundf(__fmul_rn(o, id));
    if (j == 0) dy[(size_t)m * nbo + b] = (float)(_Float16)d;
  }
}

template <int TM, int KW>
void gemm_launch(const Mat &W, const QAct &xa, int M, int epi, float *y, int ldy,
                 hipStream_t st) {
  const int mt16 = (M + 15) >> 4;
  const dim3 grid(W.N / 16, (mt16 + TM - 1) / TM), block(KW * 64);
#define Q3H_GEMM(E)                                                                           \
  hipLaunchKernelGGL((k_gemm_i8<TM, KW, E>), grid, block, 0, st, W.q, xa.q, y, W.N, W.K, M, \
                     ldy)
  if (epi == EPI_STORE)
    Q3H_GEMM(EPI_STORE);
  else if (epi == EPI_ADD)
    Q3H_GEMM(EPI_ADD);
  else
    Q3H_GEMM(EPI_SWIGLU);
#undef Q3H_GEMM
}

template <int TM>
void gemm_by_k(const Mat &W, const QAct &xa, int M, int epi, float *y, int ldy, hipStream_t st) {
  // a wave per chunk
  const int nch = W.K / (32 * kChunkBlocks);
  if (nch >= 6)
    gemm_launch<TM, 6>(W, xa, M, epi, y, ldy, st);
  else if (nch >= 4)
    gemm_launch<TM, 4>(W, xa, M, epi, y, ldy, st);
  else
    gemm_launch<TM, 2>(W, xa, M, epi, y, ldy, st);
}

// slices > 1 only without a norm (each slice a whole number of 32-blocks)
template <int SRC, int NC>
void quant_launch_nc(float *x, const float *part, int ld, int M, int K, const float *norm_w,
                     float eps, const QAct &out, float *xn_out, int xn_rows, hipStream_t st,
                     int slices) {
  const int Mp = (M + 15) & ~15;
  const int kc = (K / 8 + kQuantThreads * slices - 1) / (kQuantThreads * slices);
  const dim3 grid(Mp, slices);
#define Q3H_QUANT(KC)                                                                          \
  hipLaunchKernelGGL((k_quant_act<SRC, KC, NC>), grid, dim3(kQuantThreads), 0, st, x, part,    \
                     out.q, norm_w, M, K, ld, eps, slices, xn_out, xn_rows)
  if (kc <= 1)
    Q3H_QUANT(1);
  else if (kc == 2)
    Q3H_QUANT(2);
  else
    Q3H_QUANT(3);
#undef Q3H_QUANT
}

template <int SRC>
void quant_launch(float *x, const float *part, int ld, int M, int K, const float *norm_w,
                  float eps, const QAct &out, float *xn_out, int xn_rows, hipStream_t st,
                  int slices = 1) {
  if (SRC == SRC_X || ld <= 2)
    quant_launch_nc<SRC, 2>(x, part, ld, M, K, norm_w, eps, out, xn_out, xn_rows, st, slices);
  else if (ld <= 4)
    quant_launch_nc<SRC, 4>(x, part, ld, M, K, norm_w, eps, out, xn_out, xn_rows, st, slices);
  else
    quant_launch_nc<SRC, 6>(x, part, ld, M, K, norm_w, eps, out, xn_out, xn_rows, st, slices);
}

}  // namespace

bool gemm_i8_supported(int N, int K) {
  return N > 0 && N % 16 == 0 && K > 0 && K % (32 * kChunkBlocks) == 0 &&
         K <= kQuantThreads * kQuantChunks * 8;
}

int gemm_i8_chunks(int K) { return K / (32 * kChunkBlocks); }

size_t qact_bytes(int M, int K) {
  const size_t Mp = (M + 15) & ~15;
  return Mp * K + sizeof(float) * Mp * (K / 32);
}

void launch_quantize_act(const float *x, int ldx, int M, int K, const float *norm_w, float eps,
                         QAct out, float *xn_out, hipStream_t st) {
  quant_launch<SRC_X>(const_cast<float *>(x), nullptr, ldx, M, K, norm_w, eps, out, xn_out, 1,
                      st);
}

void launch_residual_quantize(float *h, const float *part, int chunks, int M, int K,
                              const float *norm_w, float eps, const QAct *out, hipStream_t st,
                              float *normed) {
  quant_launch<SRC_ADD>(h, part, chunks, M, K, norm_w, eps, out ? *out : QAct{}, normed, M, st);
}

void launch_swiglu_quantize(const float *part, int chunks, int M, int K, QAct out,
                            hipStream_t st) {
  const int slices = (K / 8 + kQuantThreads - 1) / kQuantThreads;
  quant_launch<SRC_SWIGLU>(nullptr, part, chunks, M, K, nullptr, 0.f, out, nullptr, 0, st,
                           slices);
}

void launch_gemm_i8(const Mat &W, const QAct &xa, int M, int epi, float *y, int ldy,
                    hipStream_t st) {
  if (M <= 16)
    gemm_by_k<1>(W, xa, M, epi, y, ldy, st);
  else if (M <= 32)
    gemm_by_k<2>(W, xa, M, epi, y, ldy, st);
  else
    gemm_by_k<4>(W, xa, M, epi, y, ldy, st);
}

// Both products below take one 16-row activation tile per workgroup, the
// tiles on a grid dimension of their own: a tile's waves do the work of a
// 16-row product, and more rows add workgroups instead of lengthening each.
// Above 32 rows a wave takes two tiles (its weights loaded once for both):
// one tile per wave would put more workgroups than CUs on the gate/up product.
bool launch_gemm_i8_swiglu_quantize(const Mat &W, const QAct &xa, int M, QAct out,
                                    hipStream_t st) {
  if (M > 64 || W.K != 1024 || W.N % 64 != 0) return false;
  const int mt16 = (M + 15) >> 4;
  if (mt16 > 2)
    hipLaunchKernelGGL(k_gemm_i8_swq<2>, dim3(W.N / 64, (mt16 + 1) / 2), dim3(512), 0, st, W.q,
                       xa.q, out.q, W.N, M);
  else
    hipLaunchKernelGGL(k_gemm_i8_swq<1>, dim3(W.N / 64, mt16), dim3(512), 0, st, W.q, xa.q,
                       out.q, W.N, M);
  return true;
}

void launch_gemm_i8_partial(const Mat &W, const QAct &xa, int M, float *part, hipStream_t st) {
  const int mt16 = (M + 15) >> 4;
  if (mt16 > 2) {
    const dim3 grid(W.N / 16, gemm_i8_chunks(W.K), (mt16 + 1) / 2);
    hipLaunchKernelGGL(k_gemm_i8p<2>, grid, dim3(64), 0, st, W.q, xa.q, part, W.N, W.K, M);
  } else {
    const dim3 grid(W.N / 16, gemm_i8_chunks(W.K), mt16);
    hipLaunchKernelGGL(k_gemm_i8p<1>, grid, dim3(64), 0, st, W.q, xa.q, part, W.N, W.K, M);
  }
}

}  // namespace q3h
