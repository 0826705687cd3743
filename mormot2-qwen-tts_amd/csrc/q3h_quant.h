// q3h_quant.h - one activation row RMS-normed and quantized per 32-block into
// the operand tiles of the int8 products by the threads of one workgroup, for
// kernels that build a row themselves (the frame step's input rows).
#pragma once

#include <hip/hip_runtime.h>

#include "q3h_internal.h"
#include "q3h_wave.h"

namespace q3h {

// this thread's 8-element chunk t of a K-element row (t < K / 8; zeros past
// the row, and for p == nullptr)
__device__ __forceinline__ void row_chunk8(const float *p, int K, float (&v)[8]) {
  const int t = threadIdx.x;
  const bool on = p != nullptr && t < (K >> 3);
  const int tc = on ? t : 0;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
  if (p) {
    a = reinterpret_cast<const float4 *>(p)[2 * tc];
    b = reinterpret_cast<const float4 *>(p)[2 * tc + 1];
  }
  const float x8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = on ? x8[e] : 0.f;
}

// The row held as each thread's chunk v (row_chunk8: threads t < K / 8 own
// the 8-element chunks t, K / 8 <= blockDim, K % 256 == 0), RMS-normed when
// norm (sum of squares in double, inv = (float)(1 / sqrt(ss / K + eps)),
// y = w * (x * inv), w8 the thread's chunk of the weights) and quantized
// (ggml quantize_row_q8_0_ref) into row m of the M-row tiles at xq, scales
// after the tiles. Every thread of the workgroup must call it. red: LDS for
// blockDim / 64 doubles.
__device__ inline void quant_row_regs(float (&v)[8], const float (&w8)[8], bool norm, float eps,
                                      int K, int m, int M, int8_t *xq, double *red) {
  const int t = threadIdx.x, nchk = K >> 3, nb = K >> 5, mt16 = (M + 15) >> 4;
  const bool on = t < nchk;
  if (norm) {
    double ss = 0.0;
#pragma unroll
    for (int e = 0; e < 8; e++) ss += (double)v[e] * (double)v[e];
    ss = wave_sum_dpp_d(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    double tot = 0.0;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) tot += red[i];
    const float inv = (float)(1.0 / sqrt(tot / K + (double)eps));
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = w8[e] * (v[e] * inv);
  }
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
  amax = quad_max_dpp(amax);
  if (!on) return;
  const float d = __fdiv_rn(amax, 127.0f);
  const float id = d != 0.f ? __fdiv_rn(1.0f, d) : 0.f;
  unsigned long long packed = 0;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const int q = (int)roundf(__fmul_rn(v[e], id));
    packed |= (unsigned long long)(uint8_t)(int8_t)q << (8 * e);
  }
  *reinterpret_cast<unsigned long long *>(xq + qtile_offset(m, 8 * t, mt16)) = packed;
  if ((t & 3) == 0)
    reinterpret_cast<float *>(xq + (size_t)mt16 * 16 * K)[(size_t)m * nb + (t >> 2)] =
        (float)(_Float16)d;
}

// Row x[0..K) (x == nullptr: zeros) RMS-normed with w when both are non-null
// and quantized, as quant_row_regs; the row and the weights are loaded
// together.
__device__ inline void quant_row_block(const float *x, const float *w, float eps, int K, int m,
                                       int M, int8_t *xq, double *red) {
  const bool norm = w && x;
  float w8[8], v[8];
  row_chunk8(norm ? w : nullptr, K, w8);
  row_chunk8(x, K, v);
  quant_row_regs(v, w8, norm, eps, K, m, M, xq, red);
}

}  // namespace q3h
