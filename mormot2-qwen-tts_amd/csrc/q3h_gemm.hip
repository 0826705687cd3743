// q3h_gemm.hip - the int8 path of the Q8_0 products (stacks created with
// act_q8 = 1): activations are quantized per 32-block with the weights' own
// quantizer (ggml quantize_row_q8_0_ref: d = amax / 127, q = round(x / d)
// half away from zero, d kept as fp16; the format of lm.pas:259-267), then
// every Q8_0 block of the product is one v_mfma_i32_16x16x32_i8 whose exact
// int32 dot is scaled by d_w * d_x into an fp32 sum (ggml
// vec_dot_q8_0_q8_0).
//
// Evaluation order (fixed, so that the products equal a CPU evaluation in the
// same order to the bit): per output, one fused multiply-add chain over the 8
// blocks of each 256-column chunk, acc = fma((float)dot_b, d_w * d_x, acc)
// from 0 in block order, and the chunk sums added in chunk order.
//
// Operand layouts (v_mfma_i32_16x16x32_i8, wave64): lane l holds 8 int8 of
// row l % 16 of A and of column l % 16 of B, k = 8 * (l / 16) .. + 7; the
// result C[4 * (l / 16) + r][l % 16], r < 4, lands in lane l. A is 16 weight
// rows read straight from the row-major Q8_0 matrix; B is 16 activation rows,
// which the quantizer writes already in operand order, so each B operand is
// one coalesced 512-byte load.
#include "q3h_internal.h"
#include "q3h_math.h"
#include "q3h_wave.h"

namespace q3h {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kQuantThreads = 128;
constexpr int kQuantChunks = 3;  // 8-element chunks per thread: K <= 3072
constexpr int kMaxChunks = 12;   // 256-column chunks of a product: K <= 3072

// One workgroup per activation row m < Mp (gridDim.x == Mp, M rounded up to
// 16); a thread owns 8-element chunks j = t, t + 128, ... and the four chunks
// of a lane quad make one 32-block. Rows M..Mp-1 are written as zeros.
// RMSNorm first when norm_w != nullptr: y = w * (x * inv), inv =
// 1/sqrt(mean(x^2) + eps) with the sum of squares in double. xn_out, when
// non-null, receives the (normed) row M - 1.
__global__ __launch_bounds__(kQuantThreads) void k_quant_act(const float *x, int ldx, int M,
                                                              int K, const float *norm_w,
                                                              float eps, int8_t *xq, float *dx,
                                                              float *xn_out) {
  const int m = blockIdx.x, t = threadIdx.x;
  const int mt16 = gridDim.x >> 4, nch = K >> 3, nb = K >> 5;
  long *xq8 = reinterpret_cast<long *>(xq);
  const size_t slot = (size_t)(m >> 4) * 64 + (m & 15);  // + (b * mt16 * 64 + g * 16)
  if (m >= M) {
    for (int j = t; j < nch; j += kQuantThreads) {
      const int b = j >> 2, g = j & 3;
      xq8[(size_t)b * mt16 * 64 + slot + g * 16] = 0;
      if (g == 0) dx[(size_t)m * nb + b] = 0.f;
    }
    return;
  }
  const float4 *xr = reinterpret_cast<const float4 *>(x + (size_t)m * ldx);
  float v[kQuantChunks][8];
#pragma unroll
  for (int i = 0; i < kQuantChunks; i++) {
    const int j = t + i * kQuantThreads;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (j < nch) {
      a = xr[2 * j];
      b = xr[2 * j + 1];
    }
    v[i][0] = a.x, v[i][1] = a.y, v[i][2] = a.z, v[i][3] = a.w;
    v[i][4] = b.x, v[i][5] = b.y, v[i][6] = b.z, v[i][7] = b.w;
  }
  if (norm_w) {
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < kQuantChunks; i++)
#pragma unroll
      for (int e = 0; e < 8; e++) ss += (double)v[i][e] * (double)v[i][e];
    ss = wave_sum_dpp_d(ss);
    __shared__ double part[kQuantThreads / 64];
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    ss = part[0] + part[1];
    const float inv = (float)(1.0 / sqrt(ss / K + (double)eps));
    const float4 *wr = reinterpret_cast<const float4 *>(norm_w);
#pragma unroll
    for (int i = 0; i < kQuantChunks; i++) {
      const int j = t + i * kQuantThreads;
      if (j < nch) {
        const float4 a = wr[2 * j], b = wr[2 * j + 1];
        const float w8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; e++) v[i][e] = w8[e] * (v[i][e] * inv);
      }
    }
  }
  if (xn_out && m == M - 1) {
    float4 *xo = reinterpret_cast<float4 *>(xn_out);
#pragma unroll
    for (int i = 0; i < kQuantChunks; i++) {
      const int j = t + i * kQuantThreads;
      if (j < nch) {
        xo[2 * j] = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
        xo[2 * j + 1] = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kQuantChunks; i++) {
    const int j = t + i * kQuantThreads;
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[i][e]));
    // nch is a multiple of 4, so a quad is wholly inside or outside the row
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    if (j >= nch) continue;
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = d != 0.f ? __fdiv_rn(1.0f, d) : 0.f;
    unsigned long long packed = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int q = (int)roundf(__fmul_rn(v[i][e], id));
      packed |= (unsigned long long)(uint8_t)(int8_t)q << (8 * e);
    }
    const int b = j >> 2, g = j & 3;
    xq8[(size_t)b * mt16 * 64 + slot + g * 16] = (long)packed;
    if (g == 0) dx[(size_t)m * nb + b] = (float)(_Float16)d;
  }
}

// y[m][n] (+)= sum_b d_w[n][b] d_x[m][b] sum_{k in b} q_w[n][k] q_x[m][k].
// A workgroup owns 16 weight rows (blockIdx.x) and TM 16-column activation
// tiles (blockIdx.y); its KW waves take the chunks of 8 blocks (256 k) in
// turn, each chunk's chain lands in its own LDS slot, and the slots are
// added in chunk order. Each wave issues every load of a chunk before its
// first MFMA. EPI_SWIGLU: rows 2j / 2j + 1 are gate / up of output j.
template <int TM, int KW, int EPI>
__global__ __launch_bounds__(KW * 64) void k_gemm_i8(const int8_t *wq, const int8_t *xq,
                                                      const float *dx, float *y, int N, int K,
                                                      int M, int ldy) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int g = lane >> 4, c = lane & 15;
  const int nb = K >> 5, nch = (nb + 7) >> 3;
  const int mt16 = (M + 15) >> 4;
  const int n0 = blockIdx.x * 16, mt0 = blockIdx.y * TM;
  const _Float16 *wd = reinterpret_cast<const _Float16 *>(wq + (size_t)N * K);
  const long *xq8 = reinterpret_cast<const long *>(xq);
  const bool full = (nb & 7) == 0;
  constexpr int LD = TM * 16 + 4;
  __shared__ float red[kMaxChunks][16][LD];

  for (int ch = w; ch < nch; ch += KW) {
    float acc[TM][4];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) acc[t][r] = 0.f;
    const int b0 = ch * 8;
    long av[8], bv[TM][8];
    float dwv[4][8], dxv[TM][8];
    const int8_t *wr = wq + (size_t)(n0 + c) * K + 8 * g;
#pragma unroll
    for (int i = 0; i < 8; i++)
      av[i] = b0 + i < nb ? *reinterpret_cast<const long *>(wr + 32 * (b0 + i)) : 0;
#pragma unroll
    for (int t = 0; t < TM; t++) {
      const bool on = mt0 + t < mt16;
#pragma unroll
      for (int i = 0; i < 8; i++)
        bv[t][i] = on && b0 + i < nb ? xq8[((size_t)(b0 + i) * mt16 + mt0 + t) * 64 + lane] : 0;
    }
    if (full) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const uint4 u = *reinterpret_cast<const uint4 *>(wd + (size_t)(n0 + 4 * g + r) * nb + b0);
        const unsigned uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          dwv[r][2 * i] = (float)__builtin_bit_cast(_Float16, (unsigned short)(uw[i] & 0xffff));
          dwv[r][2 * i + 1] = (float)__builtin_bit_cast(_Float16, (unsigned short)(uw[i] >> 16));
        }
      }
#pragma unroll
      for (int t = 0; t < TM; t++) {
        float4 p = make_float4(0.f, 0.f, 0.f, 0.f), q = p;
        if (mt0 + t < mt16) {
          const float4 *dp =
              reinterpret_cast<const float4 *>(dx + (size_t)((mt0 + t) * 16 + c) * nb + b0);
          p = dp[0];
          q = dp[1];
        }
        dxv[t][0] = p.x, dxv[t][1] = p.y, dxv[t][2] = p.z, dxv[t][3] = p.w;
        dxv[t][4] = q.x, dxv[t][5] = q.y, dxv[t][6] = q.z, dxv[t][7] = q.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const bool on = b0 + i < nb;
#pragma unroll
        for (int r = 0; r < 4; r++)
          dwv[r][i] = on ? (float)wd[(size_t)(n0 + 4 * g + r) * nb + b0 + i] : 0.f;
#pragma unroll
        for (int t = 0; t < TM; t++)
          dxv[t][i] =
              on && mt0 + t < mt16 ? dx[(size_t)((mt0 + t) * 16 + c) * nb + b0 + i] : 0.f;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
      for (int t = 0; t < TM; t++) {
        const v4i ci = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[i], bv[t][i], v4i{0, 0, 0, 0},
                                                             0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; r++)
          acc[t][r] = fmaf((float)ci[r], __fmul_rn(dwv[r][i], dxv[t][i]), acc[t][r]);
      }
    }
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

template <int TM, int KW>
void gemm_launch(const Mat &W, const QAct &xa, int M, int epi, float *y, int ldy,
                 hipStream_t st) {
  const int mt16 = (M + 15) >> 4;
  const dim3 grid(W.N / 16, (mt16 + TM - 1) / TM), block(KW * 64);
#define Q3H_GEMM(E)                                                                        \
  hipLaunchKernelGGL((k_gemm_i8<TM, KW, E>), grid, block, 0, st, W.q, xa.q, xa.d, y, W.N, \
                     W.K, M, ldy)
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
  const int nch = (W.K / 32 + 7) / 8;
  if (TM <= 2 && nch >= 12)
    gemm_launch<TM, (TM <= 2 ? 12 : 8)>(W, xa, M, epi, y, ldy, st);
  else if (nch >= 8)
    gemm_launch<TM, 8>(W, xa, M, epi, y, ldy, st);
  else
    gemm_launch<TM, 4>(W, xa, M, epi, y, ldy, st);
}

}  // namespace

bool gemm_i8_supported(int N, int K) {
  return N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0 && K <= kQuantThreads * kQuantChunks * 8;
}

void launch_quantize_act(const float *x, int ldx, int M, int K, const float *norm_w, float eps,
                         QAct out, float *xn_out, hipStream_t st) {
  const int Mp = (M + 15) & ~15;
  hipLaunchKernelGGL(k_quant_act, dim3(Mp), dim3(kQuantThreads), 0, st, x, ldx, M, K, norm_w,
                     eps, out.q, out.d, xn_out);
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

}  // namespace q3h
