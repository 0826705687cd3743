// q3h_gemv.hip - the Q8_0 matrix-vector product of the decode step on gfx950,
// for the widths of the Qwen3-TTS stacks: K = 1024, 2048 or 3072 columns and
// N a multiple of 256 rows (q/k/v 4096 x 1024, o 1024 x 2048, gate/up
// 6144 x 1024, down 1024 x 3072, heads 3072 / 2048 x 1024).
//
// One launch is 256 workgroups, one per CU: workgroup b owns N/256 consecutive
// rows, spread over its waves (R rows per wave), for M <= 4 activation rows.
// The kernel is latency-bound at these sizes (2-7 MB per launch), so its
// order of work is chosen to keep a single memory round trip on the critical
// path:
//   1. every lane issues its share of the activation rows (and of the RMSNorm
//      weight) first, coalesced, then all its weight loads: for each of its
//      rows and each 1024-column chunk, 16 quants (one dwordx4: a wave reads
//      1 KB of a row per instruction) and the fp16 scale of their block;
//   2. while the weights are in flight, w * x is staged in LDS once per
//      workgroup and the sum of squares of x is reduced (per wave, then the
//      loader waves' sums in a fixed order);
//   3. one barrier, then the dot products from registers and LDS, a wave
//      reduction, and the epilogue (store, residual add, or SwiGLU of an
//      interleaved gate/up row pair). The RMSNorm factor multiplies the dot:
//      W (w * x * inv) = inv * (W (w * x)).
// Staging the rows once per workgroup matters: loaded by every wave, a row and
// its norm weight cost each CU's load path more bytes than the weights
// themselves (these loads hit L2, so HBM traffic does not show it).
// LDS layout of the staged rows: element c*1024 + l*16 + 4*i + j of a row sits
// in float4 slot (c*4 + i)*64 + l, so the 64 lanes of a wave read 64
// consecutive float4 (no bank conflict). The normed row can also be written
// out (xn_out, one row, by the first wave), so the final norm of a stack and
// its head are one launch.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "q3h_internal.h"
#include "q3h_wave.h"

namespace q3h {

namespace {

constexpr int kMaxWaves = 16;
constexpr int kMaxRowsX = 4;  // activation rows per launch

__device__ __forceinline__ float dot4_i8(int w, float4 x, float acc) {
  acc = fmaf((float)(int8_t)(w), x.x, acc);
  acc = fmaf((float)(int8_t)(w >> 8), x.y, acc);
  acc = fmaf((float)(int8_t)(w >> 16), x.z, acc);
  acc = fmaf((float)(int8_t)(w >> 24), x.w, acc);
  return acc;
}

// M <= MR activation rows (x rows ldx apart, y rows ldy apart; one row: the
// batch-1 decode step), each loaded once per workgroup. Plain scalar
// arguments: the first 14 dwords are preloaded in SGPRs (all the kernel reads
// before its loads; one row reads neither M nor ldx / ldy), so the loads issue
// without waiting on a scalar memory read; xn_out, read only at the end, comes
// last. The scales are found after the quants (wq + N*K). W (waves per workgroup) is an argument: blockDim is not read.
// LW = min(W, 4) loader waves: thread t of them loads float4 t + 64*LW*j of
// each row (and of the RMSNorm weight), coalesced; waves past LW repeat the
// loads of the first LW, and rows past M repeat row M - 1, so no branch sits
// before the weight loads. The residual of EPI_ADD is loaded with the weights,
// not at the end. Every row gets the same arithmetic in the same order as a
// single row does, so a row's result does not depend on M. xn_out (the normed
// row, by the first wave of workgroup 0) is taken with a single row only.
// NP = 4 (one row): x holds four partial rows K apart whose sum
// (p0 + p1) + (p2 + p3) is the row; the loader waves of workgroup 0 write that
// sum (not normed) to xn_out. The argument list stays at 64 bytes.
template <int R, int C, int EPI, int LW, int MR, int NP = 0>
__global__ __launch_bounds__(1024) void k_gemv_q8v(const int8_t *__restrict__ wq,
                                                   const float *__restrict__ x,
                                                   const float *__restrict__ norm_w,
                                                   float *__restrict__ y, int N, int W, float eps,
                                                   int ldx, int ldy, int M,
                                                   float *__restrict__ xn_out) {
  static_assert(NP == 0 || (NP == 4 && MR == 1), "partial rows: one row of four parts");
  constexpr int K = C * 1024, NB = K / 32;
  constexpr int T = 64 * LW, J = C * 256 / T;  // loader threads, float4 per loader thread
  __shared__ float4 xs[MR][C * 256];           // w * x, slot (c*4 + i)*64 + l
  __shared__ float ssw[MR][LW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = (blockIdx.x * W + wave) * R;
  const _Float16 *__restrict__ wd = reinterpret_cast<const _Float16 *>(wq + (size_t)N * K);
  const bool nrm = norm_w != nullptr;

  // 1. the rows (and the norm weight) first, then every weight load
  const int t = tid % T;
  float4 xv[MR][J], wn[J], xp[NP > 0 ? NP : 1][J];
#pragma unroll
  for (int m = 0; m < MR; m++) {
    const float4 *xm =
        reinterpret_cast<const float4 *>(MR == 1 ? x : x + (size_t)min(m, M - 1) * ldx);
    if (NP > 0) {
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int j = 0; j < J; j++) xp[p][j] = xm[p * (K / 4) + t + T * j];
    } else {
#pragma unroll
      for (int j = 0; j < J; j++) xv[m][j] = xm[t + T * j];
    }
  }
  if (nrm) {
#pragma unroll
    for (int j = 0; j < J; j++) wn[j] = reinterpret_cast<const float4 *>(norm_w)[t + T * j];
  }
  int4 wv[R][C];
  float sc[R][C];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = min(row0 + r, N - 1);
    const int8_t *q = wq + (size_t)row * K + lane * 16;
    const _Float16 *d = wd + (size_t)row * NB + (lane >> 1);
#pragma unroll
    for (int c = 0; c < C; c++) {
      wv[r][c] = *reinterpret_cast<const int4 *>(q + c * 1024);
      sc[r][c] = (float)d[c * 32];
    }
  }
  float yres[MR][R];
  if (EPI == EPI_ADD) {
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
      for (int r = 0; r < R; r++)
        yres[m][r] = y[(MR == 1 ? 0 : (size_t)min(m, M - 1) * ldy) + min(row0 + r, N - 1)];
  }
  // every load above is issued before any arithmetic
  __builtin_amdgcn_sched_barrier(0);
  if (NP > 0) {
#pragma unroll
    for (int j = 0; j < J; j++) {
      const float4 a = xp[0][j], b = xp[1 % NP][j], c = xp[2 % NP][j], d = xp[3 % NP][j];
      xv[0][j] = make_float4((a.x + b.x) + (c.x + d.x), (a.y + b.y) + (c.y + d.y),
                             (a.z + b.z) + (c.z + d.z), (a.w + b.w) + (c.w + d.w));
    }
    if (blockIdx.x == 0 && wave < LW) {
#pragma unroll
      for (int j = 0; j < J; j++) reinterpret_cast<float4 *>(xn_out)[t + T * j] = xv[0][j];
    }
  }

  // 2. while the weights are in flight: the loader waves stage w * x in LDS
  // and sum the squares of x (fp32, per thread then per wave, then the LW
  // wave sums in a fixed order)
#pragma unroll
  for (int m = 0; m < MR; m++) {
    float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
    for (int j = 0; j < J; j++) {
      const float4 v = xv[m][j];
      ss0 = fmaf(v.x, v.x, fmaf(v.y, v.y, ss0));
      ss1 = fmaf(v.z, v.z, fmaf(v.w, v.w, ss1));
    }
    if (wave < LW) {
#pragma unroll
      for (int j = 0; j < J; j++) {
        const int f = t + T * j;  // elements 4f .. 4f + 3
        const int li = (((f >> 8) * 4 + (f & 3)) << 6) + ((f & 255) >> 2);
        const float4 v = xv[m][j];
        xs[m][li] =
            nrm ? make_float4(wn[j].x * v.x, wn[j].y * v.y, wn[j].z * v.z, wn[j].w * v.w) : v;
      }
    }
    if (nrm) {
      const float sw = wave_sum_dpp(ss0 + ss1);
      if (wave < LW && lane == 0) ssw[m][wave] = sw;
    }
  }
  __syncthreads();
  float inv[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) {
    inv[m] = 1.f;
    if (nrm) {
      float ss = ssw[m][0];
      if (LW == 2) ss += ssw[m][1 % LW];
      if (LW == 4) ss = (ss + ssw[m][1 % LW]) + (ssw[m][2 % LW] + ssw[m][3 % LW]);
      inv[m] = 1.0f / sqrtf(ss * (1.0f / K) + eps);
    }
  }
  if (NP == 0 && xn_out != nullptr && blockIdx.x == 0 && wave == 0) {
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float4 v = xs[0][c * 256 + i * 64 + lane];
        reinterpret_cast<float4 *>(xn_out + c * 1024 + lane * 16)[i] =
            make_float4(v.x * inv[0], v.y * inv[0], v.z * inv[0], v.w * inv[0]);
      }
  }

  // 3. the dot products (this lane's 16 columns of each chunk, row by row),
  // a wave reduction, the epilogue
  float acc[MR][R];
#pragma unroll
  for (int m = 0; m < MR; m++) {
    float4 xl[C][4];
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
      for (int i = 0; i < 4; i++) xl[c][i] = xs[m][c * 256 + i * 64 + lane];
#pragma unroll
    for (int r = 0; r < R; r++) {
      acc[m][r] = 0.f;
#pragma unroll
      for (int c = 0; c < C; c++) {
        float p0 = dot4_i8(wv[r][c].x, xl[c][0], 0.f);
        float p1 = dot4_i8(wv[r][c].y, xl[c][1], 0.f);
        p0 = dot4_i8(wv[r][c].z, xl[c][2], p0);
        p1 = dot4_i8(wv[r][c].w, xl[c][3], p1);
        acc[m][r] = fmaf(sc[r][c], p0 + p1, acc[m][r]);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MR; m++)
#pragma unroll
    for (int r = 0; r < R; r++) acc[m][r] = wave_sum_dpp(acc[m][r]) * inv[m];
  if (lane != 0 || row0 >= N) return;
#pragma unroll
  for (int m = 0; m < MR; m++) {
    if (MR > 1 && m >= M) break;
    float *ym = MR == 1 ? y : y + (size_t)m * ldy;
    if (EPI == EPI_SWIGLU) {
#pragma unroll
      for (int p = 0; p < R / 2; p++) {
        const float g = acc[m][2 * p], u = acc[m][2 * p + 1];
        ym[row0 / 2 + p] = g / (1.0f + expf(-g)) * u;
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; r++) {
        if (row0 + r < N) {
          if (EPI == EPI_ADD)
            ym[row0 + r] = yres[m][r] + acc[m][r];
          else
            ym[row0 + r] = acc[m][r];
        }
      }
    }
  }
}

// The single-row product (EPI_STORE, RMSNorm prologue) whose activation row
// is chosen on the device: row `code` of rows [vocab][K], code the argmax of
// logits [vocab] (the smallest index among equal maxima: ChooseCode). Each of
// the 4 waves takes the argmax of a quarter of the L2-resident logits, the
// quarters meet in LDS (the merge keeps the largest value and, among equal
// ones, the smallest index, so its order does not matter), then the row is
// loaded once per workgroup and staged as in k_gemv_q8v. The logit and
// norm-weight loads go out before the weight loads, so the argmax waits only
// for them and the row's load overlaps the weight stream. Workgroup 0 also
// writes, when *alive, the code and the raw row (h_out): what k_cp_argmax
// writes for the next code-predictor forward. The product equals k_gemv_q8v
// on that row (the same sums in the same order). Arguments: the first 14
// dwords are preloaded into SGPRs; h_out and alive, used only at the end,
// come after.
template <int R, int C, int W, int V4>
__global__ __launch_bounds__(W * 64) void k_gemv_q8v_code(
    const int8_t *__restrict__ wq, const float *__restrict__ logits,
    const float *__restrict__ rows, const float *__restrict__ norm_w, float *__restrict__ y,
    int N, float eps, int *__restrict__ code_out, float *__restrict__ h_out,
    const int *__restrict__ alive) {
  static_assert(W == 4 && V4 % W == 0, "4 waves, each a quarter of the logits");
  constexpr int K = C * 1024, NB = K / 32, VW = V4 / W;
  __shared__ float4 xs[C * 256];  // w * x, slot (c*4 + i)*64 + l
  __shared__ float ssw[W], amv[W], ap0;
  __shared__ int ami[W];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = (blockIdx.x * W + wave) * R;
  const _Float16 *__restrict__ wd = reinterpret_cast<const _Float16 *>(wq + (size_t)N * K);
  // 1. this wave's quarter of the logits, the norm weight, then the weights
  float4 lg[VW];
#pragma unroll
  for (int i = 0; i < VW; i++)
    lg[i] = reinterpret_cast<const float4 *>(logits)[(wave * VW + i) * 64 + lane];
  float4 wn[C];
#pragma unroll
  for (int j = 0; j < C; j++) wn[j] = reinterpret_cast<const float4 *>(norm_w)[tid + 256 * j];
  __builtin_amdgcn_sched_barrier(0);
  int4 wv[R][C];
  float sc[R][C];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = min(row0 + r, N - 1);
    const int8_t *q = wq + (size_t)row * K + lane * 16;
    const _Float16 *d = wd + (size_t)row * NB + (lane >> 1);
#pragma unroll
    for (int c = 0; c < C; c++) {
      wv[r][c] = *reinterpret_cast<const int4 *>(q + c * 1024);
      sc[r][c] = (float)d[c * 32];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // 2. the argmax: element 4 ((wave VW + i) 64 + lane) + e of the logits
  float bv = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int i = 0; i < VW; i++) {
    const float e4[4] = {lg[i].x, lg[i].y, lg[i].z, lg[i].w};
#pragma unroll
    for (int e = 0; e < 4; e++) argmax_merge(bv, bi, e4[e], 4 * ((wave * VW + i) * 64 + lane) + e);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float v2 = __shfl_xor(bv, off, 64);
    const int i2 = __shfl_xor(bi, off, 64);
    argmax_merge(bv, bi, v2, i2);
  }
  if (lane == 0) {
    amv[wave] = bv;
    ami[wave] = bi;
    if (wave == 0) ap0 = lg[0].x;  // logits[0]
  }
  __syncthreads();
  bv = -INFINITY;
  bi = 0x7fffffff;
#pragma unroll
  for (int w = 0; w < W; w++) argmax_merge(bv, bi, amv[w], ami[w]);
  const int code = first_max_code(bi, ap0);
  // 3. the row, a quarter per wave (float4 tid + 256 j), staged as k_gemv_q8v
  const float *x = rows + (size_t)code * K;
  float4 xv[C];
#pragma unroll
  for (int j = 0; j < C; j++) xv[j] = reinterpret_cast<const float4 *>(x)[tid + 256 * j];
  float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
  for (int j = 0; j < C; j++) {
    const float4 v = xv[j];
    ss0 = fmaf(v.x, v.x, fmaf(v.y, v.y, ss0));
    ss1 = fmaf(v.z, v.z, fmaf(v.w, v.w, ss1));
    const int f = tid + 256 * j;
    const int li = (((f >> 8) * 4 + (f & 3)) << 6) + ((f & 255) >> 2);
    xs[li] = make_float4(wn[j].x * v.x, wn[j].y * v.y, wn[j].z * v.z, wn[j].w * v.w);
  }
  const float sw = wave_sum_dpp(ss0 + ss1);
  if (lane == 0) ssw[wave] = sw;
  __syncthreads();
  const float inv =
      1.0f / sqrtf(((ssw[0] + ssw[1]) + (ssw[2] + ssw[3])) * (1.0f / K) + eps);
  float4 xl[C][4];
#pragma unroll
  for (int c = 0; c < C; c++)
#pragma unroll
    for (int i = 0; i < 4; i++) xl[c][i] = xs[c * 256 + i * 64 + lane];
  // 4. the dot products
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    acc[r] = 0.f;
#pragma unroll
    for (int c = 0; c < C; c++) {
      float p0 = dot4_i8(wv[r][c].x, xl[c][0], 0.f);
      float p1 = dot4_i8(wv[r][c].y, xl[c][1], 0.f);
      p0 = dot4_i8(wv[r][c].z, xl[c][2], p0);
      p1 = dot4_i8(wv[r][c].w, xl[c][3], p1);
      acc[r] = fmaf(sc[r][c], p0 + p1, acc[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = wave_sum_dpp(acc[r]) * inv;
  // the code and the raw row, after every load of the product has been used
  if (blockIdx.x == 0 && *alive) {
    if (tid == 0) *code_out = code;
#pragma unroll
    for (int j = 0; j < C; j++) reinterpret_cast<float4 *>(h_out)[tid + 256 * j] = xv[j];
  }
  if (lane != 0 || row0 >= N) return;
#pragma unroll
  for (int r = 0; r < R; r++)
    if (row0 + r < N) y[row0 + r] = acc[r];
}

// ev0 / ev1 (optional): events recorded at the start and the end of the
// kernel's own execution (hipExtLaunchKernelGGL), for measurement
template <int R, int C, int LW, int MR>
void launch_vl(const GemvArgs &a, int epi, int waves, hipStream_t st, hipEvent_t ev0,
               hipEvent_t ev1) {
  const dim3 grid(a.N / (waves * R)), block(64 * waves);
#define Q3H_V(E)                                                                                 \
  do {                                                                                           \
    if (ev0)                                                                                     \
      hipExtLaunchKernelGGL((k_gemv_q8v<R, C, E, LW, MR>), grid, block, 0, st, ev0, ev1, 0, a.wq, \
                            a.x, a.norm_w, a.y, a.N, waves, a.eps, a.ldx, a.ldy, a.M, a.xn_out); \
    else                                                                                         \
      hipLaunchKernelGGL((k_gemv_q8v<R, C, E, LW, MR>), grid, block, 0, st, a.wq, a.x, a.norm_w, \
                         a.y, a.N, waves, a.eps, a.ldx, a.ldy, a.M, a.xn_out);                   \
  } while (0)
  if (epi == EPI_STORE)
    Q3H_V(EPI_STORE);
  else if (epi == EPI_ADD)
    Q3H_V(EPI_ADD);
  else if (R % 2 == 0)
    Q3H_V(EPI_SWIGLU);
#undef Q3H_V
}

template <int R, int C, int MR>
void launch_v(const GemvArgs &a, int epi, int waves, hipStream_t st, hipEvent_t ev0,
              hipEvent_t ev1) {
  if (waves >= 4)
    launch_vl<R, C, 4, MR>(a, epi, waves, st, ev0, ev1);
  else if (MR > 1)
    return;  // not reached: more rows take 4 waves or more
  else if (waves >= 2)
    launch_vl<R, C, 2, 1>(a, epi, waves, st, ev0, ev1);
  else
    launch_vl<R, C, 1, 1>(a, epi, waves, st, ev0, ev1);
}

// W waves of R rows, M <= MR activation rows
template <int R, int MR>
void launch_k(const GemvArgs &a, int epi, int W, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
  switch (a.K) {
    case 1024: launch_v<R, 1, MR>(a, epi, W, st, ev0, ev1); break;
    case 2048: launch_v<R, 2, MR>(a, epi, W, st, ev0, ev1); break;
    default: launch_v<R, 3, MR>(a, epi, W, st, ev0, ev1); break;
  }
}

// R1 rows per wave (1-4)
template <int MR>
bool launch_rows(const GemvArgs &a, int epi, int R1, int W, hipStream_t st, hipEvent_t ev0,
                 hipEvent_t ev1) {
  switch (R1) {
    case 1: launch_k<1, MR>(a, epi, W, st, ev0, ev1); return true;
    case 2: launch_k<2, MR>(a, epi, W, st, ev0, ev1); return true;
    case 3: launch_k<3, MR>(a, epi, W, st, ev0, ev1); return true;
    case 4: launch_k<4, MR>(a, epi, W, st, ev0, ev1); return true;
    default: return false;
  }
}

}  // namespace

bool launch_gemv_q8_code(const GemvArgs &a, const float *logits, int vocab, const float *rows,
                         int *code_out, float *h_out, const int *alive, hipStream_t st) {
  if (reinterpret_cast<const int8_t *>(a.wd) != a.wq + (size_t)a.N * a.K) return false;
  if (a.M != 1 || a.K != 1024 || a.norm_w == nullptr || a.N % 1024 != 0) return false;
  const int R = a.N / 1024;  // 256 workgroups of 4 waves
  const dim3 grid(256), block(256);
#define Q3H_C(RR, V4)                                                                             \
  hipLaunchKernelGGL((k_gemv_q8v_code<RR, 1, 4, V4>), grid, block, 0, st, a.wq, logits, rows,     \
                     a.norm_w, a.y, a.N, a.eps, code_out, h_out, alive)
#define Q3H_C_V(RR)          \
  if (vocab == 2048)         \
    Q3H_C(RR, 8);            \
  else if (vocab == 3072)    \
    Q3H_C(RR, 12);           \
  else                       \
    return false
  switch (R) {
    case 1: Q3H_C_V(1); break;
    case 2: Q3H_C_V(2); break;
    case 3: Q3H_C_V(3); break;
    case 4: Q3H_C_V(4); break;
    default: return false;
  }
#undef Q3H_C_V
#undef Q3H_C
  return true;
}

// gate/up (SwiGLU) shapes: R1 rows per wave, W waves per workgroup, 256 workgroups
static bool swiglu_shape(int N, int &R1, int &W) {
  if (N % 256 != 0) return false;
  const int rpb = N / 256;
  R1 = rpb % 4 == 0 ? 4 : 2;
  W = rpb / R1;
  return R1 * W == rpb && W >= 1 && W <= kMaxWaves;
}

// four waves, all of them loaders of the partial rows, of N / 1024 rows each
// (256 workgroups): at N = 6144 6-row waves took 1.470 ms per frame against
// 1.485 for the plain products' 6 waves of 4 rows, whose two extra waves
// repeat the loaders' 16 KB of partials
bool gemv_q8_parts_supported(int N, int K) {
  const int R1 = N / 1024;
  return K == 1024 && N % 1024 == 0 && (R1 == 2 || R1 == 4 || R1 == 6);
}

bool launch_gemv_q8_swiglu_parts(const GemvArgs &a, float *x_out, hipStream_t st) {
  if (reinterpret_cast<const int8_t *>(a.wd) != a.wq + (size_t)a.N * a.K) return false;
  if (a.M != 1 || a.norm_w == nullptr || a.xn_out != nullptr || x_out == nullptr) return false;
  if (!gemv_q8_parts_supported(a.N, a.K)) return false;
  const int R1 = a.N / 1024, W = 4;
  const dim3 grid(256), block(64 * W);
#define Q3H_P(RR)                                                                                 \
  hipLaunchKernelGGL((k_gemv_q8v<RR, 1, EPI_SWIGLU, 4, 1, 4>), grid, block, 0, st, a.wq, a.x,     \
                     a.norm_w, a.y, a.N, W, a.eps, a.ldx, a.ldy, a.M, x_out)
  if (R1 == 6)
    Q3H_P(6);
  else if (R1 == 4)
    Q3H_P(4);
  else
    Q3H_P(2);
#undef Q3H_P
  return true;
}

bool launch_gemv_q8_wide(const GemvArgs &a, int epi, hipStream_t st, hipEvent_t ev0,
                         hipEvent_t ev1) {
  // the kernels find the scales right after the quants
  if (reinterpret_cast<const int8_t *>(a.wd) != a.wq + (size_t)a.N * a.K) return false;
  if (ev0 != nullptr && a.M != 1) return false;  // events: single-row kernel only
  if (a.M < 1 || a.M > kMaxRowsX || (a.xn_out != nullptr && a.M != 1)) return false;
  if (a.K != 1024 && a.K != 2048 && a.K != 3072) return false;
  if (a.N % 256 != 0) return false;
  const int rpb = a.N / 256;  // rows per workgroup, 256 workgroups
  // measured on the Qwen3-TTS shapes, for one row and for two: one wave per
  // SIMD (R = rpb / 4 rows per wave) for the plain products; the gate/up
  // pairs (SwiGLU) as 4-row waves (6 per workgroup: 3.47 us per launch against
  // 3.78 for 2-row waves at one row, 4.45 against 4.54 at two)
  int R1 = rpb / 4, W = 4;
  if (epi == EPI_SWIGLU && !swiglu_shape(a.N, R1, W)) return false;
  if (R1 < 1 || R1 * W != rpb || W > kMaxWaves) return false;
  if (a.M == 1) return launch_rows<1>(a, epi, R1, W, st, ev0, ev1);
  if (W < 4) return false;  // more rows: 4 loader waves
  if (a.M == 2) return launch_rows<2>(a, epi, R1, W, st, ev0, ev1);
  return launch_rows<4>(a, epi, R1, W, st, ev0, ev1);
}

}  // namespace q3h
