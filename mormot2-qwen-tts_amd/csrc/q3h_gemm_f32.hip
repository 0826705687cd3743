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

#include "q3h_internal.h"

namespace q3h {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int KC = 256;  // columns per wave

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

__device__ __forceinline__ float silu_mul_f(float g, float u) { return g / (1.0f + expf(-g)) * u; }

template <int TM, int K, int EPI>
__global__ __launch_bounds__(64 * (K / KC)) void k_gemm_f32(const float *__restrict__ w,
                                                            const float *__restrict__ x, int ldx,
                                                            int M, int N, float *__restrict__ y,
                                                            int ldy) {
  constexpr int KW = K / KC;   // waves
  constexpr int ST = KC / 16;  // 16-column steps per wave
  __shared__ float red[KW][TM][4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16, m0 = blockIdx.y * (TM * 16);
  const int r = lane & 15, g = lane >> 4;
  const int kb = wave * KC + 4 * g;
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
    } else {
      y[(size_t)m * ldy + n] = v;
    }
  }
}

template <int TM, int K>
void launch_tk(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy,
               hipStream_t st) {
  const dim3 grid(W.N / 16, (M + 16 * TM - 1) / (16 * TM)), block(64 * (K / KC));
  if (epi == EPI_STORE)
    hipLaunchKernelGGL((k_gemm_f32<TM, K, EPI_STORE>), grid, block, 0, st, W.f, x, ldx, M, W.N,
                       y, ldy);
  else if (epi == EPI_ADD)
    hipLaunchKernelGGL((k_gemm_f32<TM, K, EPI_ADD>), grid, block, 0, st, W.f, x, ldx, M, W.N, y,
                       ldy);
  else
    hipLaunchKernelGGL((k_gemm_f32<TM, K, EPI_SWIGLU>), grid, block, 0, st, W.f, x, ldx, M, W.N,
                       y, ldy);
}

template <int TM>
void launch_t(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy,
              hipStream_t st) {
  switch (W.K) {
    case 1024: launch_tk<TM, 1024>(W, x, ldx, M, epi, y, ldy, st); break;
    case 2048: launch_tk<TM, 2048>(W, x, ldx, M, epi, y, ldy, st); break;
    default: launch_tk<TM, 3072>(W, x, ldx, M, epi, y, ldy, st); break;
  }
}

}  // namespace

bool gemm_f32_supported(int N, int K) {
  return N % 16 == 0 && (K == 1024 || K == 2048 || K == 3072);
}

void launch_gemm_f32(const Mat &W, const float *x, int ldx, int M, int epi, float *y, int ldy,
                     hipStream_t st) {
  if (M <= 16)
    launch_t<1>(W, x, ldx, M, epi, y, ldy, st);
  else if (M <= 32)
    launch_t<2>(W, x, ldx, M, epi, y, ldy, st);
  else
    launch_t<4>(W, x, ldx, M, epi, y, ldy, st);
}

}  // namespace q3h
