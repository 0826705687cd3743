// q3h_gemm_f32.hip - the products of f32 stacks (the reference's f32 mode,
// lm.pas:177-178 with idtF32) over several rows, on the matrix cores:
// y[m][n] (+)= sum_k W[n][k] x[m][k], W row-major [N][K] f32, x [M][ldx].
//
// v_mfma_f32_16x16x4_f32 (wave64): lane l holds A[l % 16][l / 16] and
// B[l / 16][l % 16] of a 16x4 and a 4x16 operand and receives
// D[4 (l / 16) + r][l % 16], r < 4. Here A is 16 activation rows and B 16
// weight rows (as columns), both read straight from memory: lane l loads 16
// bytes, columns 4 (l / 16) .. + 3 of its row, of each 16-column step, so one
// load instruction covers 64 contiguous bytes of 16 rows, and the four floats
// feed four MFMAs (MFMA i takes column 4 (l / 16) + i of the step in k slot
// l / 16, the same for A and B, so the products pair up as in the sum).
// fp32 inputs, fp32 products and accumulation: no rounding of the operands.
//
// A workgroup owns 16 weight rows (n) and TM tiles of 16 activation rows (m);
// its K / 256 waves take 256 columns each, with the loads of up to 16
// 16-column steps in flight ahead of the MFMAs, and their partial sums meet in LDS
// in wave order (a fixed order: results do not depend on scheduling). The
// epilogue stores, adds to y (the residual), or applies SwiGLU to the
// interleaved gate / up rows (row 2j gate j, 2j + 1 up j: out[m][j] =
// silu(gate) * up). The grid covers all M rows in tiles of 16 TM, so a prefill
// of 512 rows is one launch per product; every tile reads the weights, which
// the later tiles find in L2 / Infinity Cache.
#include <hip/hip_runtime.h>

#include "q3h_api_internal.h"
#include "q3h_math.h"

namespace q3h {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int KC = 256;  // columns per wave

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

__device__ __forceinline__ float silu_mul_f(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// SiLU of the text projection: 0 below -80 (where e^-v would overflow)
__device__ __forceinline__ float silu_clamp_f(float v) {
  return v < -80.0f ? 0.0f : v / (1.0f + expf(-v));
}

typedef __bf16 bf8v __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

// 8 Q8_0 quants (two dwords, little-endian bytes) as 8 bf16: the high halves
// of their f32 values, exact (at most 8 significant bits)
__device__ __forceinline__ bf8v q8_bf16x8(uint2 w) {
  const uint32_t w2[2] = {w.x, w.y};
  u32x4v o;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t word = w2[i >> 1], sh = 16 * (i & 1);
    const uint32_t f0 = __float_as_uint((float)(int8_t)(word >> sh));
    const uint32_t f1 = __float_as_uint((float)(int8_t)(word >> (sh + 8)));
    o[i] = (f0 >> 16) | (f1 & 0xffff0000u);
  }
  return __builtin_bit_cast(bf8v, o);
}

// the sums of a tile, met in LDS (red[wave][t][q][lane]: the MFMA result
// layout), added in wave order and stored / added / SwiGLU'd / kept as a slice
template <int TM, int KW, int EPI>
__device__ __forceinline__ void epilogue(const float (&red)[KW][TM][4][64], int m0, int n0, int M,
                                         float *__restrict__ y, int ldy) {
  // output (m, n) of this tile: t, lane' = 16 (m / 4 % 4) + n % 16, q = m % 4
  for (int o = threadIdx.x; o < TM * 256; o += 64 * KW) {
    const int t = o >> 8, q = (o >> 6) & 3, l = o & 63;
    const int m = m0 + 16 * t + 4 * (l >> 4) + q, n = n0 + (l & 15);
    if (m >= M) continue;
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < KW; i++) v += red[i][t][q][l];
    if (EPI == EPI_SWIGLU) {
      // gate in even rows, up in the odd row after it (the next lane)
      float u = 0.f;
#pragma unroll
      for (int i = 0; i < KW; i++) u += red[i][t][q][l ^ 1];
      if ((l & 1) == 0) y[(size_t)m * ldy + n / 2] = silu_mul_f(v, u);
    } else if (EPI == EPI_ADD) {
      y[(size_t)m * ldy + n] += v;
    } else if (EPI == EPI_ADD_SILU) {
      float *p = y + (size_t)m * ldy + n;
      *p = silu_clamp_f(*p + v);
    } else if (EPI == EPI_PART) {
      y[((size_t)blockIdx.z * M + m) * ldy + n] = v;
    } else {
      y[(size_t)m * ldy + n] = v;
    }
  }
}

// KK: the columns of one workgroup (K / gridDim.z; 256 per wave), K: the
// row stride of W. EPI_PART: the workgroup's sums go to slice blockIdx.z of
// y [gridDim.z][M][ldy] for a consumer that adds the slices in order.
template <int TM, int KK, int EPI>
__global__ __launch_bounds__(64 * (KK / KC)) void k_gemm_f32(const float *__restrict__ w,
                                                             const float *__restrict__ x,
                                                             int ldx, int M, int N, int K,
                                                             float *__restrict__ y, int ldy) {
  constexpr int KW = KK / KC;  // waves
  constexpr int ST = KC / 16;  // 16-column steps per wave
  __shared__ float red[KW][TM][4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * (TM * 16);
  const int r = lane & 15, g = lane >> 4;
  const int kb = blockIdx.z * KK + wave * KC + 4 * g;
  const float *wr = w + (size_t)min(n0 + r, N - 1) * K + kb;
  const float *xr[TM];
#pragma unroll
  for (int t = 0; t < TM; t++) xr[t] = x + (size_t)min(m0 + 16 * t + r, M - 1) * ldx + kb;

  v4f acc[TM];
#pragma unroll
  for (int t = 0; t < TM; t++) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
  // a ring of D steps in flight: the loads of step s + D are issued before
  // the MFMAs of step s (scheduling barriers keep the order, so each step
  // waits only for its own loads)
  constexpr int D = TM == 1 ? ST : (TM == 4 && KW > 8 ? 4 : 8);
  float4 wb[D], xb[D][TM];
#pragma unroll
  for (int s = 0; s < D; s++) {
    wb[s] = ld4(wr + 16 * s);
#pragma unroll
    for (int t = 0; t < TM; t++) xb[s][t] = ld4(xr[t] + 16 * s);
  }
#pragma unroll
  for (int s = 0; s < ST; s++) {
    const int c = s % D;
    const float4 wc = wb[c];
    float4 xc[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) xc[t] = xb[c][t];
    if (s + D < ST) {
      wb[c] = ld4(wr + 16 * (s + D));
#pragma unroll
      for (int t = 0; t < TM; t++) xb[c][t] = ld4(xr[t] + 16 * (s + D));
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < TM; t++) {
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xc[t].x, wc.x, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xc[t].y, wc.y, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xc[t].z, wc.z, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xc[t].w, wc.w, acc[t], 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int t = 0; t < TM; t++)
#pragma unroll
    for (int q = 0; q < 4; q++) red[wave][t][q][lane] = acc[t][q];
  __syncthreads();

  epilogue<TM, KW, EPI>(red, m0, n0, M, y, ldy);
}

// Many rows (prefill): a workgroup per 64 activation rows x 16 WN weight rows
// over the whole K, so that each activation chunk is read once per 16 WN
// weight rows instead of once per 16. Wave w owns weight rows n0 + 16 w ..
// + 15 and all 4 tiles of 16 activation rows. Per 32-column chunk: the
// activations (64 x 32) go through LDS (double buffered, one barrier per
// chunk), each wave's weights straight to registers; the loads of chunk c + 1
// are issued before the MFMAs of chunk c. Operands as in k_gemm_f32 (lane l:
// row l % 16, columns 4 (l / 16) .. + 3 of each 16-column step); the result
// tile of a wave is complete, so the epilogue needs no reduction.
//
// K-slices: workgroup z takes columns z kc .. z kc + kc - 1 (kc = K without a
// split); EPI_PART stores its sums to slice z of y [gridDim.z][M][ldy].
template <int WN, int EPI>
__global__ __launch_bounds__(64 * WN) void k_gemm_f32_m64(const float *__restrict__ w,
                                                          const float *__restrict__ x, int ldx,
                                                          int M, int N, int K, int kc,
                                                          float *__restrict__ y, int ldy) {
  constexpr int NT = 64 * WN, XS = 36;  // threads; LDS row stride (floats, padded)
  constexpr int XF4 = 64 * 32 / 4 / NT;  // float4 of an activation chunk per thread
  __shared__ float xs[2][64 * XS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * WN + 16 * wave, m0 = blockIdx.y * 64;
  const int kz = blockIdx.z * kc;
  const float *wr = w + (size_t)min(n0 + r, N - 1) * K + kz + 4 * g;
  // activation chunk loads: float4 f = t + NT i of the 64 x 8 float4 chunk
  const float *xr[XF4];
  int xo[XF4];
#pragma unroll
  for (int i = 0; i < XF4; i++) {
    const int f = t + NT * i, row = f >> 3, c4 = f & 7;
    xr[i] = x + (size_t)min(m0 + row, M - 1) * ldx + kz + 4 * c4;
    xo[i] = row * XS + 4 * c4;
  }
  float4 xn[XF4], wn[2], wc[2];
  auto load = [&](int kc) {
#pragma unroll
    for (int i = 0; i < XF4; i++) xn[i] = ld4(xr[i] + kc);
    wn[0] = ld4(wr + kc);
    wn[1] = ld4(wr + kc + 16);
  };
  v4f acc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
  load(0);
#pragma unroll
  for (int i = 0; i < XF4; i++) *reinterpret_cast<float4 *>(&xs[0][xo[i]]) = xn[i];
  wc[0] = wn[0];
  wc[1] = wn[1];
  __syncthreads();
  const int nc = kc / 32;
  for (int c = 0; c < nc; c++) {
    const int b = c & 1;
    if (c + 1 < nc) load(32 * (c + 1));
#pragma unroll
    for (int s = 0; s < 2; s++) {
#pragma unroll
      for (int tm = 0; tm < 4; tm++) {
        const float4 xa = *reinterpret_cast<const float4 *>(&xs[b][(16 * tm + r) * XS + 16 * s + 4 * g]);
        acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.x, wc[s].x, acc[tm], 0, 0, 0);
        acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.y, wc[s].y, acc[tm], 0, 0, 0);
        acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.z, wc[s].z, acc[tm], 0, 0, 0);
        acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.w, wc[s].w, acc[tm], 0, 0, 0);
      }
    }
    if (c + 1 < nc) {
#pragma unroll
      for (int i = 0; i < XF4; i++) *reinterpret_cast<float4 *>(&xs[b ^ 1][xo[i]]) = xn[i];
      wc[0] = wn[0];
      wc[1] = wn[1];
    }
    __syncthreads();
  }
  // lane l holds (m = m0 + 16 tm + 4 g + q, n = n0 + r)
  const int n = n0 + r;
#pragma unroll
  for (int tm = 0; tm < 4; tm++)
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int m = m0 + 16 * tm + 4 * g + q;
      const float v = acc[tm][q];
      if (EPI == EPI_SWIGLU) {
        const float u = __shfl_xor(v, 1);  // up: the odd row after its gate
        if (m < M && (r & 1) == 0) y[(size_t)m * ldy + n / 2] = silu_mul_f(v, u);
      } else if (m < M) {
        if (EPI == EPI_ADD)
          y[(size_t)m * ldy + n] += v;
        else if (EPI == EPI_ADD_SILU)
          y[(size_t)m * ldy + n] = silu_clamp_f(y[(size_t)m * ldy + n] + v);
        else if (EPI == EPI_PART)
          y[((size_t)blockIdx.z * M + m) * ldy + n] = v;
        else
          y[(size_t)m * ldy + n] = v;
      }
    }
}

// f32 x f32 products on the bf16 matrix cores, exact to the fp32 rounding of
// the sum: each operand split into three bf16 parts, x = x_hi + x_mid + x_lo
// (the top 8 significant bits, the next 8, the last 8: exact, as an f32
// significand has 24 bits), and the six part products whose weight is at
// least 2^-16 of x w accumulated in fp32 (hi hi, hi mid, mid hi, hi lo,
// lo hi, mid mid; each bf16 product is exact in fp32). The dropped three
// weigh below 2^-23 of the product, under its fp32 rounding.
//
// v_mfma_f32_16x16x32_bf16: lane l holds A[l % 16][8 (l / 16) .. + 7] and
// B[8 (l / 16) .. + 7][l % 16] (8 bf16 each) and receives
// D[4 (l / 16) + r][l % 16]. The tile and pipeline are those of
// k_gemm_f32_m64: 64 activation rows x 16 WN weight rows per workgroup, a 32-
// column chunk at a time; the activations are split as they go to LDS (three
// bf16 planes, double buffered), the weights come pre-split (Mat::x3) to
// registers one chunk ahead. 24 MFMAs per wave and chunk instead of 32 of
// the f32 kind, each a sixteenth of the cycles per flop.
template <int WN, int EPI>
__global__ __launch_bounds__(64 * WN) void k_gemm_x3_m64(const uint16_t *__restrict__ w3,
                                                         const float *__restrict__ x, int ldx,
                                                         int M, int N, int K, int kc,
                                                         float *__restrict__ y, int ldy) {
  constexpr int NT = 64 * WN;
  constexpr int NB = 1;                  // 16-column weight tiles per wave
  constexpr int XS = 40;                 // LDS row stride, bf16 (80 bytes)
  constexpr int XF4 = 64 * 32 / 4 / NT;  // float4 of an activation chunk per thread
  __shared__ uint16_t xs[2][3][64 * XS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NB * WN + 16 * NB * wave, m0 = blockIdx.y * 64;
  const int kz = blockIdx.z * kc;
  const size_t plane = (size_t)N * K;
  const uint16_t *wr[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) wr[j] = w3 + (size_t)min(n0 + 16 * j + r, N - 1) * K + kz + 8 * g;
  const float *xr[XF4];
  int xo[XF4];
#pragma unroll
  for (int i = 0; i < XF4; i++) {
    const int f = t + NT * i, row = f >> 3, c4 = f & 7;
    xr[i] = x + (size_t)min(m0 + row, M - 1) * ldx + kz + 4 * c4;
    xo[i] = row * XS + 4 * c4;
  }
  float4 xn[XF4];
  u32x4v wn[NB][3], wc[NB][3];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < XF4; i++) xn[i] = ld4(xr[i] + k0);
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int p = 0; p < 3; p++)
        wn[j][p] = *reinterpret_cast<const u32x4v *>(wr[j] + p * plane + k0);
  };
  // the chunk's activations into the three planes of LDS buffer b
  auto stage = [&](int b) {
#pragma unroll
    for (int i = 0; i < XF4; i++) {
      uint32_t h[4], m[4], l[4];
      split3(xn[i].x, h[0], m[0], l[0]);
      split3(xn[i].y, h[1], m[1], l[1]);
      split3(xn[i].z, h[2], m[2], l[2]);
      split3(xn[i].w, h[3], m[3], l[3]);
      *reinterpret_cast<uint2 *>(&xs[b][0][xo[i]]) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
      *reinterpret_cast<uint2 *>(&xs[b][1][xo[i]]) = make_uint2(m[0] | (m[1] << 16), m[2] | (m[3] << 16));
      *reinterpret_cast<uint2 *>(&xs[b][2][xo[i]]) = make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
    }
  };
  v4f acc[NB][4];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[j][i] = v4f{0.f, 0.f, 0.f, 0.f};
  load(0);
  stage(0);
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int p = 0; p < 3; p++) wc[j][p] = wn[j][p];
  __syncthreads();
  const int nc = kc / 32;
  for (int c = 0; c < nc; c++) {
    const int b = c & 1;
    if (c + 1 < nc) load(32 * (c + 1));
#pragma unroll
    for (int tm = 0; tm < 4; tm++) {
      const int o = (16 * tm + r) * XS + 8 * g;
      const bf8v ah = __builtin_bit_cast(bf8v, *reinterpret_cast<const u32x4v *>(&xs[b][0][o]));
      const bf8v am = __builtin_bit_cast(bf8v, *reinterpret_cast<const u32x4v *>(&xs[b][1][o]));
      const bf8v al = __builtin_bit_cast(bf8v, *reinterpret_cast<const u32x4v *>(&xs[b][2][o]));
#pragma unroll
      for (int j = 0; j < NB; j++) {
        const bf8v bh = __builtin_bit_cast(bf8v, wc[j][0]), bm = __builtin_bit_cast(bf8v, wc[j][1]),
                   bl = __builtin_bit_cast(bf8v, wc[j][2]);
        v4f a = acc[j][tm];
        a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bm, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bh, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bm, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, a, 0, 0, 0);
        acc[j][tm] = a;
      }
    }
    if (c + 1 < nc) {
      stage(b ^ 1);
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int p = 0; p < 3; p++) wc[j][p] = wn[j][p];
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int n = n0 + 16 * j + r;
#pragma unroll
    for (int tm = 0; tm < 4; tm++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int m = m0 + 16 * tm + 4 * g + q;
        const float v = acc[j][tm][q];
        if (EPI == EPI_SWIGLU) {
          const float u = __shfl_xor(v, 1);
          if (m < M && (r & 1) == 0) y[(size_t)m * ldy + n / 2] = silu_mul_f(v, u);
        } else if (m < M) {
          if (EPI == EPI_ADD)
            y[(size_t)m * ldy + n] += v;
          else if (EPI == EPI_PART)
            y[((size_t)blockIdx.z * M + m) * ldy + n] = v;
          else
            y[(size_t)m * ldy + n] = v;
        }
      }
  }
}

// the three bf16 planes of an f32 matrix
__global__ void k_split3(const float *__restrict__ f, size_t n, uint16_t *__restrict__ x3) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  uint32_t h, m, l;
  split3(f[i], h, m, l);
  x3[i] = (uint16_t)h;
  x3[n + i] = (uint16_t)m;
  x3[2 * n + i] = (uint16_t)l;
}

// The same products with Q8_0 weights (int8 quants [N][K], then fp16 scales
// [N][K/32]) and f32 activations, on the bf16 matrix cores. A quant is an
// integer of at most 8 significant bits, exact in bf16; an activation is
// split exactly into three bf16 parts (split3). One 32-block of 16 weight
// rows and 16 activation rows is three v_mfma_f32_16x16x32_bf16 (low, middle,
// high part, each adding exact products in fp32) into a block sum, which is
// scaled by the weight row's fp16 block scale and added to the row's fp32
// sum: y = sum over blocks of d * (sum over the block of x q).
//
// Lane l holds, per block, the 8 quants 8 (l / 16) .. + 7 of weight row
// n0 + l % 16 (one 8-byte load) and the same 8 columns of activation row
// m0 + 16 t + l % 16 of each tile t (two 16-byte loads), and receives
// D[4 (l / 16) + q][l % 16]: the output layout of k_gemm_f32, whose
// epilogues this kernel shares. A workgroup owns 16 NB weight rows and TM
// tiles of 16 activation rows (the activations split once for the NB weight
// tiles); its waves take NBW blocks each. A wave issues the
// loads of all its weights and scales first, then of its activations D
// blocks ahead of the arithmetic, so that it waits for few memory round
// trips. (Its time is the activation loads: every workgroup reads all M rows
// over its K range; k_gemm_q8x_m64 shares them over 64 weight rows.)
template <int KK>
constexpr int q8x_blocks_per_wave() {
  return KK <= 256 ? 2 : KK <= 1024 ? 4 : KK / 256;  // 4 to 8 waves
}

template <int TM, int KK, int EPI, int NB>
__global__ __launch_bounds__(64 * (KK / (32 * q8x_blocks_per_wave<KK>()))) void k_gemm_q8x(
    const int8_t *__restrict__ wq, const float *__restrict__ x, int ldx, int M, int N, int K,
    float *__restrict__ y, int ldy) {
  constexpr int NBW = q8x_blocks_per_wave<KK>();
  constexpr int KW = KK / (32 * NBW);     // waves
  constexpr int D = NBW < 4 ? NBW : 4;    // blocks in flight
  __shared__ float red[NB][KW][TM][4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16 * NB, m0 = blockIdx.y * (TM * 16);
  const int r = lane & 15, g = lane >> 4;
  const int kw = blockIdx.z * KK + wave * (32 * NBW);  // the wave's first column
  uint2 wv[NB][NBW];
  uint32_t dw[NB][NBW / 2];  // the block scales, 2 per dword
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int row = min(n0 + 16 * j + r, N - 1);
    const int8_t *wr = wq + (size_t)row * K + kw + 8 * g;
    const _Float16 *dr =
        reinterpret_cast<const _Float16 *>(wq + (size_t)N * K) + (size_t)row * (K / 32) + kw / 32;
#pragma unroll
    for (int b = 0; b < NBW; b++) wv[j][b] = *reinterpret_cast<const uint2 *>(wr + 32 * b);
    if constexpr (NBW == 2) {
      dw[j][0] = *reinterpret_cast<const uint32_t *>(dr);
    } else {
#pragma unroll
      for (int i = 0; i < NBW / 4; i++) {
        const uint2 t = *reinterpret_cast<const uint2 *>(dr + 4 * i);
        dw[j][2 * i] = t.x;
        dw[j][2 * i + 1] = t.y;
      }
    }
  }
  const float *xr[TM];
#pragma unroll
  for (int t = 0; t < TM; t++) xr[t] = x + (size_t)min(m0 + 16 * t + r, M - 1) * ldx + kw + 8 * g;

  u32x4v xb[D][TM][2];
  auto load = [&](int b, int c) {
#pragma unroll
    for (int t = 0; t < TM; t++) {
      xb[c][t][0] = *reinterpret_cast<const u32x4v *>(xr[t] + 32 * b);
      xb[c][t][1] = *reinterpret_cast<const u32x4v *>(xr[t] + 32 * b + 4);
    }
  };
#pragma unroll
  for (int s = 0; s < D; s++) load(s, s);
  v4f acc[NB][TM];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int t = 0; t < TM; t++) acc[j][t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < NBW; b++) {
    const int c = b % D;
    u32x4v xc[TM][2];
#pragma unroll
    for (int t = 0; t < TM; t++) {
      xc[t][0] = xb[c][t][0];
      xc[t][1] = xb[c][t][1];
    }
    if (b + D < NBW) load(b + D, c);
    __builtin_amdgcn_sched_barrier(0);
    bf8v bw[NB];
    float d[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) {
      bw[j] = q8_bf16x8(wv[j][b]);
      d[j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(dw[j][b >> 1] >> (16 * (b & 1))));
    }
#pragma unroll
    for (int t = 0; t < TM; t++) {
      u32x4v ph, pm, pl;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const u32x4v &src = xc[t][i >> 1];
        uint32_t h0, m0_, l0, h1, m1, l1;
        split3(__uint_as_float(src[2 * (i & 1)]), h0, m0_, l0);
        split3(__uint_as_float(src[2 * (i & 1) + 1]), h1, m1, l1);
        ph[i] = h0 | (h1 << 16);
        pm[i] = m0_ | (m1 << 16);
        pl[i] = l0 | (l1 << 16);
      }
#pragma unroll
      for (int j = 0; j < NB; j++) {
        v4f s = v4f{0.f, 0.f, 0.f, 0.f};
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8v, pl), bw[j], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8v, pm), bw[j], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8v, ph), bw[j], s, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; q++) acc[j][t][q] = fmaf(d[j], s[q], acc[j][t][q]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
      for (int q = 0; q < 4; q++) red[j][wave][t][q][lane] = acc[j][t][q];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NB; j++) epilogue<TM, KW, EPI>(red[j], m0, n0 + 16 * j, M, y, ldy);
}

// Q8_0 products over many rows with the activations staged in LDS: a
// workgroup of WN waves owns 64 activation rows and 16 WN weight rows (wave w:
// rows n0 + 16 w .. + 15) over the K range of its slice, so each activation
// chunk crosses the vector memory path once per 16 WN weight rows instead of
// once per 16 (k_gemm_q8x). Per 64-column chunk (two 32-blocks): the 64 x 64
// activations are split into three bf16 planes in LDS (double buffered, one
// barrier per chunk), each wave's quants and block scales go to registers one
// chunk ahead; per block and 16-row tile three v_mfma_f32_16x16x32_bf16 (low,
// middle, high part) into the block sum, scaled by the block scale into the
// fp32 sum, as in k_gemm_q8x. Lane l holds weight row n0 + 16 w + l % 16 and
// receives rows 4 (l / 16) + q of each tile: a wave's sums are complete, the
// epilogue stores them directly. Used above 64 rows: with fewer, its
// N / (16 WN) workgroups leave most CUs idle.
template <int WN, int EPI>
__global__ __launch_bounds__(64 * WN) void k_gemm_q8x_m64(const int8_t *__restrict__ wq,
                                                          const float *__restrict__ x, int ldx,
                                                          int M, int N, int K, int kc,
                                                          float *__restrict__ y, int ldy) {
  constexpr int NT = 64 * WN;
  constexpr int CW = 64;                  // chunk columns
  constexpr int XS = CW + 8;              // LDS row stride, bf16 (144 bytes)
  constexpr int SF = 64 * CW / 4 / NT;    // float4 of a chunk per thread
  __shared__ uint16_t xs[2][3][64 * XS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * WN + 16 * wave, m0 = blockIdx.y * 64;
  const int kz = blockIdx.z * kc;
  const int row = min(n0 + r, N - 1);
  const int8_t *wr = wq + (size_t)row * K + kz + 8 * g;
  const _Float16 *dr =
      reinterpret_cast<const _Float16 *>(wq + (size_t)N * K) + (size_t)row * (K / 32) + kz / 32;
  // this thread's float4 of a chunk: global and LDS offsets
  const float *xg[SF];
  int lo[SF];
#pragma unroll
  for (int i = 0; i < SF; i++) {
    const int f = t + NT * i, rw = f / (CW / 4), c4 = f % (CW / 4);
    xg[i] = x + (size_t)min(m0 + rw, M - 1) * ldx + kz + 4 * c4;
    lo[i] = rw * XS + 4 * c4;
  }
  float4 xn[SF];
  uint2 wn[2], wc[2];
  uint32_t dn, dc;  // the chunk's two block scales
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < SF; i++) xn[i] = ld4(xg[i] + k0);
    wn[0] = *reinterpret_cast<const uint2 *>(wr + k0);
    wn[1] = *reinterpret_cast<const uint2 *>(wr + k0 + 32);
    dn = *reinterpret_cast<const uint32_t *>(dr + k0 / 32);
  };
  auto stage = [&](int b) {
#pragma unroll
    for (int i = 0; i < SF; i++) {
      uint32_t h[4], md[4], l[4];
      split3(xn[i].x, h[0], md[0], l[0]);
      split3(xn[i].y, h[1], md[1], l[1]);
      split3(xn[i].z, h[2], md[2], l[2]);
      split3(xn[i].w, h[3], md[3], l[3]);
      *reinterpret_cast<uint2 *>(&xs[b][0][lo[i]]) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
      *reinterpret_cast<uint2 *>(&xs[b][1][lo[i]]) = make_uint2(md[0] | (md[1] << 16), md[2] | (md[3] << 16));
      *reinterpret_cast<uint2 *>(&xs[b][2][lo[i]]) = make_uint2(l[0] | (l[1] << 16), l[2] | (l[3] << 16));
    }
  };
  v4f acc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
  load(0);
  stage(0);
  wc[0] = wn[0];
  wc[1] = wn[1];
  dc = dn;
  __syncthreads();
  const int nc = kc / CW;
  for (int c = 0; c < nc; c++) {
    const int b = c & 1;
    if (c + 1 < nc) load(CW * (c + 1));
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
      const bf8v bw = q8_bf16x8(wc[kb]);
      const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(dc >> (16 * kb)));
#pragma unroll
      for (int tm = 0; tm < 4; tm++) {
        const int o = (16 * tm + r) * XS + 32 * kb + 8 * g;
        const bf8v ah = __builtin_bit_cast(bf8v, *reinterpret_cast<const u32x4v *>(&xs[b][0][o]));
        const bf8v am = __builtin_bit_cast(bf8v, *reinterpret_cast<const u32x4v *>(&xs[b][1][o]));
        const bf8v al = __builtin_bit_cast(bf8v, *reinterpret_cast<const u32x4v *>(&xs[b][2][o]));
        v4f sm = v4f{0.f, 0.f, 0.f, 0.f};
        sm = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bw, sm, 0, 0, 0);
        sm = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bw, sm, 0, 0, 0);
        sm = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bw, sm, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; q++) acc[tm][q] = fmaf(d, sm[q], acc[tm][q]);
      }
    }
    if (c + 1 < nc) {
      stage(b ^ 1);
      wc[0] = wn[0];
      wc[1] = wn[1];
      dc = dn;
    }
    __syncthreads();
  }
  const int n = n0 + r;
#pragma unroll
  for (int tm = 0; tm < 4; tm++)
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int m = m0 + 16 * tm + 4 * g + q;
      const float v = acc[tm][q];
      if (EPI == EPI_SWIGLU) {
        const float u = __shfl_xor(v, 1);  // up: the odd row after its gate
        if (m < M && (r & 1) == 0) y[(size_t)m * ldy + n / 2] = silu_mul_f(v, u);
      } else if (m < M) {
        if (EPI == EPI_ADD)
          y[(size_t)m * ldy + n] += v;
        else if (EPI == EPI_PART)
          y[((size_t)blockIdx.z * M + m) * ldy + n] = v;
        else
          y[(size_t)m * ldy + n] = v;
      }
    }
}

// h[m] += slices 0 .. S-1 of part [S][M][K], added in slice order; then, with
// a norm weight, xn[m] = w * (h[m] * inv), inv = 1 / sqrt(mean(h[m]^2) + eps)
// (sum of squares in double). One workgroup per row, K <= 4096: a thread
// holds columns t + 256 i of each 1024-column round in registers, and the norm
// weights are loaded before the partials, so the normalization needs no
// second trip to memory.
constexpr int kResidNormRounds = 4;

template <int S>
__global__ __launch_bounds__(256) void k_resid_norm(float *__restrict__ h,
                                                    const float *__restrict__ part, int M,
                                                    int K, const float *__restrict__ w,
                                                    float eps, float *__restrict__ xn) {
  constexpr int NR = kResidNormRounds;
  __shared__ double red[4];
  const int m = blockIdx.x, t = threadIdx.x;
  float *hr = h + (size_t)m * K;
  float wv[NR][4];
  if (w) {
#pragma unroll
    for (int r = 0; r < NR; r++)
      if (1024 * r < K)
#pragma unroll
        for (int i = 0; i < 4; i++) wv[r][i] = w[min(1024 * r + t + 256 * i, K - 1)];
  }
  float hv[NR][4];
  double ss = 0.0;
#pragma unroll
  for (int r = 0; r < NR; r++) {
    const int k0 = 1024 * r;
    if (k0 >= K) break;
    // four columns per thread, every load (clamped) issued before the sums
    float a[4][S];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int k = min(k0 + t + 256 * i, K - 1);
#pragma unroll
      for (int s = 0; s < S; s++) a[i][s] = part[((size_t)s * M + m) * K + k];
      hv[r][i] = hr[k];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int k = k0 + t + 256 * i;
      float v = hv[r][i];
#pragma unroll
      for (int s = 0; s < S; s++) v += a[i][s];
      hv[r][i] = v;
      if (k < K) {
        hr[k] = v;
        ss += (double)v * v;
      }
    }
  }
  if (w == nullptr) return;
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  const double tot = red[0] + red[1] + red[2] + red[3];
  const float inv = (float)(1.0 / sqrt(tot / K + (double)eps));
#pragma unroll
  for (int r = 0; r < NR; r++) {
    if (1024 * r >= K) break;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int k = 1024 * r + t + 256 * i;
      if (k < K) xn[(size_t)m * K + k] = wv[r][i] * (hv[r][i] * inv);
    }
  }
}

template <int TM, int KK>
void launch_tk(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy, int ks,
               hipStream_t st) {
  const dim3 grid(W.N / 16, (M + 16 * TM - 1) / (16 * TM), ks), block(64 * (KK / KC));
#define Q3H_G(E)                                                                            \
  hipLaunchKernelGGL((k_gemm_f32<TM, KK, E>), grid, block, 0, st, W.f, x, ldx, M, W.N, W.K, \
                     y, ldy)
  if (epi == EPI_STORE)
    Q3H_G(EPI_STORE);
  else if (epi == EPI_ADD)
    Q3H_G(EPI_ADD);
  else if (epi == EPI_SWIGLU)
    Q3H_G(EPI_SWIGLU);
  else if (epi == EPI_PART)
    Q3H_G(EPI_PART);
  else if constexpr (KK >= 1024)
    Q3H_G(EPI_ADD_SILU);
  else
    require(false, Q3H_E_ARG, "EPI_ADD_SILU takes the whole K");
#undef Q3H_G
}

template <int TM>
void launch_t(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy, int ks,
              hipStream_t st) {
  switch (W.K / ks) {
    case 256: launch_tk<TM, 256>(W, x, ldx, M, epi, y, ldy, ks, st); break;
    case 512: launch_tk<TM, 512>(W, x, ldx, M, epi, y, ldy, ks, st); break;
    case 768: launch_tk<TM, 768>(W, x, ldx, M, epi, y, ldy, ks, st); break;
    case 1024: launch_tk<TM, 1024>(W, x, ldx, M, epi, y, ldy, ks, st); break;
    case 2048: launch_tk<TM, 2048>(W, x, ldx, M, epi, y, ldy, ks, st); break;
    default: launch_tk<TM, 3072>(W, x, ldx, M, epi, y, ldy, ks, st); break;
  }
}

template <int WN>
void launch_m64(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy,
                hipStream_t st, int ks = 1) {
  const dim3 grid(W.N / (16 * WN), (M + 63) / 64, ks), block(64 * WN);
  const int kc = W.K / ks;
  if (W.x3 && epi != EPI_ADD_SILU) {
    const dim3 gx(W.N / (16 * WN), (M + 63) / 64, ks);  // one 16-column tile per wave
#define Q3H_X(E)                                                                              \
  hipLaunchKernelGGL((k_gemm_x3_m64<WN, E>), gx, block, 0, st, W.x3, x, ldx, M, W.N, W.K, kc, \
                     y, ldy)
    if (epi == EPI_STORE)
      Q3H_X(EPI_STORE);
    else if (epi == EPI_ADD)
      Q3H_X(EPI_ADD);
    else if (epi == EPI_PART)
      Q3H_X(EPI_PART);
    else
      Q3H_X(EPI_SWIGLU);
#undef Q3H_X
    return;
  }
#define Q3H_G(E)                                                                               \
  hipLaunchKernelGGL((k_gemm_f32_m64<WN, E>), grid, block, 0, st, W.f, x, ldx, M, W.N, W.K, kc, \
                     y, ldy)
  if (epi == EPI_STORE)
    Q3H_G(EPI_STORE);
  else if (epi == EPI_ADD)
    Q3H_G(EPI_ADD);
  else if (epi == EPI_ADD_SILU)
    Q3H_G(EPI_ADD_SILU);
  else if (epi == EPI_PART)
    Q3H_G(EPI_PART);
  else
    Q3H_G(EPI_SWIGLU);
#undef Q3H_G
}

// Q8_0 weights: k_gemm_q8x over the whole K (KK = K: every epilogue but
// EPI_ADD_SILU) or over K slices of KK <= 1024 columns (EPI_PART)
template <int TM, int KK, int NB>
void launch_q8x_k(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy,
                  int ks, hipStream_t st) {
  const dim3 grid(W.N / (16 * NB), (M + 16 * TM - 1) / (16 * TM), ks),
      block(64 * (KK / (32 * q8x_blocks_per_wave<KK>())));
#define Q3H_Q(E)                                                                                 \
  hipLaunchKernelGGL((k_gemm_q8x<TM, KK, E, NB>), grid, block, 0, st, W.q, x, ldx, M, W.N, W.K, \
                     y, ldy)
  if (epi == EPI_PART) {
    if constexpr (KK <= 1024)
      Q3H_Q(EPI_PART);
    else
      require(false, Q3H_E_ARG, "Q8_0 K slices take at most 1024 columns");
  } else if constexpr (KK >= 1024) {
    if (epi == EPI_STORE)
      Q3H_Q(EPI_STORE);
    else if (epi == EPI_ADD)
      Q3H_Q(EPI_ADD);
    else if (epi == EPI_SWIGLU)
      Q3H_Q(EPI_SWIGLU);
    else
      require(false, Q3H_E_ARG, "EPI_ADD_SILU takes f32 weights");
  } else {
    require(false, Q3H_E_ARG, "Q8_0 products over a K slice store partial sums only");
  }
#undef Q3H_Q
}

// NB 16-row weight tiles per wave: two over more than 16 rows (each
// activation load then feeds twice the matrix-core work: 48-row prefill
// 1.92 -> 1.85 ms), one below (8 rows: 1.03 against 1.07 ms with two)
template <int TM, int NB>
void launch_q8x_t(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy,
                  int ks, hipStream_t st) {
  switch (W.K / ks) {
    case 256: launch_q8x_k<TM, 256, NB>(W, x, ldx, M, epi, y, ldy, ks, st); break;
    case 512: launch_q8x_k<TM, 512, NB>(W, x, ldx, M, epi, y, ldy, ks, st); break;
    case 768: launch_q8x_k<TM, 768, NB>(W, x, ldx, M, epi, y, ldy, ks, st); break;
    case 1024: launch_q8x_k<TM, 1024, NB>(W, x, ldx, M, epi, y, ldy, ks, st); break;
    case 2048: launch_q8x_k<TM, 2048, 1>(W, x, ldx, M, epi, y, ldy, ks, st); break;
    default: launch_q8x_k<TM, 3072, 1>(W, x, ldx, M, epi, y, ldy, ks, st); break;
  }
}

constexpr int kQ8M64Waves = 4;  // 64 weight rows per workgroup

void launch_q8x_m64(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy,
                    int ks, hipStream_t st) {
  constexpr int WN = kQ8M64Waves;
  const dim3 grid(W.N / (16 * WN), (M + 63) / 64, ks), block(64 * WN);
  const int kc = W.K / ks;
#define Q3H_Q(E)                                                                           \
  hipLaunchKernelGGL((k_gemm_q8x_m64<WN, E>), grid, block, 0, st, W.q, x, ldx, M, W.N, W.K, \
                     kc, y, ldy)
  if (epi == EPI_STORE)
    Q3H_Q(EPI_STORE);
  else if (epi == EPI_ADD)
    Q3H_Q(EPI_ADD);
  else if (epi == EPI_SWIGLU)
    Q3H_Q(EPI_SWIGLU);
  else if (epi == EPI_PART)
    Q3H_Q(EPI_PART);
  else
    require(false, Q3H_E_ARG, "EPI_ADD_SILU takes f32 weights");
#undef Q3H_Q
}

// Q8_0 weights, f32 activations [M][ldx], over K slices of K / ks columns
void launch_q8x(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy, int ks,
                hipStream_t st) {
  if (M > 64 && W.N % (16 * kQ8M64Waves) == 0 && (W.K / ks) % 64 == 0) {
    launch_q8x_m64(W, x, ldx, M, epi, y, ldy, ks, st);
  } else if (M <= 16) {
    launch_q8x_t<1, 1>(W, x, ldx, M, epi, y, ldy, ks, st);
  } else if (W.N % 32 != 0) {
    if (M <= 32)
      launch_q8x_t<2, 1>(W, x, ldx, M, epi, y, ldy, ks, st);
    else
      launch_q8x_t<4, 1>(W, x, ldx, M, epi, y, ldy, ks, st);
  } else if (M <= 32) {
    launch_q8x_t<2, 2>(W, x, ldx, M, epi, y, ldy, ks, st);
  } else if (M <= 48) {
    launch_q8x_t<3, 2>(W, x, ldx, M, epi, y, ldy, ks, st);
  } else {
    launch_q8x_t<4, 2>(W, x, ldx, M, epi, y, ldy, ks, st);
  }
}

void launch_m(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy,
              hipStream_t st) {
  if (M > 32 && epi != EPI_PART && W.N % 64 == 0 && (W.N / 64) * ((M + 63) / 64) >= 256) {
    // many rows and wide products: 64-row tiles over the whole K (at least
    // 1024 waves; narrower products keep the K split over waves below, whose
    // waves each take a quarter to a twelfth of K)
    launch_m64<4>(W, x, ldx, M, epi, y, ldy, st);
    return;
  }
  if (M <= 16)
    launch_t<1>(W, x, ldx, M, epi, y, ldy, 1, st);
  else if (M <= 32)
    launch_t<2>(W, x, ldx, M, epi, y, ldy, 1, st);
  else
    launch_t<4>(W, x, ldx, M, epi, y, ldy, 1, st);
}

}  // namespace

void launch_split3(const Mat &m, hipStream_t st) {
  const size_t n = (size_t)m.N * m.K;
  hipLaunchKernelGGL(k_split3, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, m.f, n, m.x3);
}

bool gemm_f32_supported(int N, int K) {
  return N % 16 == 0 && (K == 1024 || K == 2048 || K == 3072);
}

void launch_gemm_f32(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy,
                     hipStream_t st) {
  if (W.f)
    launch_m(W, x, ldx, M, epi, y, ldy, st);
  else
    launch_q8x(W, x, ldx, M, epi, y, ldy, 1, st);
}

bool gemm_f32_slices_supported(int N, int K) {
  const int kk = K / kF32Slices;
  return N % 16 == 0 && K % kF32Slices == 0 && (kk == 256 || kk == 512 || kk == 768 || kk == 1024);
}

int q8x_slices(const Mat &W, int M) {
  if (W.f || !W.q || M <= 16 || M > kQ8SliceRows || W.N % 32 != 0 || W.K % 256 != 0) return 0;
  const int ks = W.K / 256;  // a slice count launch_resid_norm takes
  return ks <= 4 || ks == 6 || ks == 8 || ks == 12 ? ks : 0;
}

int launch_gemm_f32_part(const Mat &W, const float *x, int ldx, int M, float *part,
                         hipStream_t st) {
  if (!W.f) {
    const int ks = q8x_slices(W, M) ? W.K / 256 : kF32Slices;
    launch_q8x(W, x, ldx, M, EPI_PART, part, W.N, ks, st);
    return ks;
  }
  if (M > 64 && W.N % 64 == 0)
    launch_m64<4>(W, x, ldx, M, EPI_PART, part, W.N, st, kF32Slices);
  else if (M <= 16)
    launch_t<1>(W, x, ldx, M, EPI_PART, part, W.N, kF32Slices, st);
  else if (M <= 32)
    launch_t<2>(W, x, ldx, M, EPI_PART, part, W.N, kF32Slices, st);
  else
    launch_t<4>(W, x, ldx, M, EPI_PART, part, W.N, kF32Slices, st);
  return kF32Slices;
}

void launch_resid_norm(float *h, const float *part, int M, int K, const float *norm_w,
                       float eps, float *xn, int slices, hipStream_t st) {
  require(K <= 1024 * kResidNormRounds, Q3H_E_ARG, "launch_resid_norm: K above 4096");
#define Q3H_RN(S)                                                                              \
  hipLaunchKernelGGL(k_resid_norm<S>, dim3(M), dim3(256), 0, st, h, part, M, K, norm_w, eps, xn)
  switch (slices) {
    case 1: Q3H_RN(1); break;
    case 2: Q3H_RN(2); break;
    case 3: Q3H_RN(3); break;
    case 4: Q3H_RN(4); break;
    case 6: Q3H_RN(6); break;
    case 8: Q3H_RN(8); break;
    case 12: Q3H_RN(12); break;
    default: require(false, Q3H_E_ARG, "launch_resid_norm: 1-4, 6, 8 or 12 slices");
  }
#undef Q3H_RN
}

}  // namespace q3h
