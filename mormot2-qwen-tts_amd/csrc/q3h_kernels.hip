// q3h_kernels.hip - gfx950 kernels of the Qwen3 stack step (decode and small
// multi-row forwards): fused RMSNorm + GEMV over Q8_0 or f32 weights, QK-norm
// + RoPE + K/V append, load-time Q8_0 conversion.
//
// Layouts (HBM):
//  - Q8_0 matrix [N][K]: int8 quants row-major + fp16 scales [N][K/32]. A lane
//    owns 16 consecutive quants of a row per 1024-column chunk, so one
//    dwordx4 load instruction of a wave covers 1 KB of one row, coalesced.
//  - f32 matrix [N][K]: a lane owns 4 consecutive floats per 256-column chunk.
//  - K/V cache: [layers][kv_heads][max_pos][head_dim], f32 or f16: the keys
//    of one head are contiguous, so a split of positions is one linear read.
#include <hip/hip_runtime.h>

#include "q3h_api_internal.h"
#include "q3h_internal.h"
#include "q3h_math.h"

namespace q3h {

constexpr int kBlock = 256;
constexpr int kMaxRows = 4;  // activation rows held in LDS per GEMV pass

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + expf(-g)) * u;
}

// Stage M (<= kMaxRows) activation rows of K floats into LDS, RMS-normalized
// with weight w when w != nullptr: y = w * (x * inv), inv = 1/sqrt(mean(x^2)+eps)
// (sum of squares in double). Block 0 may also publish the last staged row.
__device__ void stage_rows(const float *__restrict__ x, int ldx, int M, int K,
                           const float *__restrict__ w, float eps, float *xs,
                           float *xn_out) {
  __shared__ double red[kBlock / 64][kMaxRows];
  __shared__ float inv[kMaxRows];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int m = 0; m < M; m++) {
    const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)m * ldx);
    float4 *dst = reinterpret_cast<float4 *>(xs + m * K);
    double ss = 0.0;
    for (int k = tid; k < (K >> 2); k += kBlock) {
      const float4 v = src[k];
      dst[k] = v;
      ss += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
    }
    if (w) {
      ss = wave_sum_d(ss);
      if (lane == 0) red[wave][m] = ss;
    }
  }
  if (!w) {
    __syncthreads();
    if (xn_out && blockIdx.x == 0)
      for (int k = tid; k < K; k += kBlock) xn_out[k] = xs[(M - 1) * K + k];
    return;
  }
  __syncthreads();
  if (tid < M) {
    double t = 0.0;
    for (int i = 0; i < kBlock / 64; i++) t += red[i][tid];
    inv[tid] = (float)(1.0 / sqrt(t / K + (double)eps));
  }
  __syncthreads();
  for (int m = 0; m < M; m++) {
    const float iv = inv[m];
    for (int k = tid; k < K; k += kBlock) xs[m * K + k] = w[k] * (xs[m * K + k] * iv);
  }
  __syncthreads();
  if (xn_out && blockIdx.x == 0)
    for (int k = tid; k < K; k += kBlock) xn_out[k] = xs[(M - 1) * K + k];
}

__device__ __forceinline__ float dot16_i8(const int4 w, const float *x) {
  const int ws[4] = {w.x, w.y, w.z, w.w};
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int v = ws[i];
    s0 = fmaf((float)(int8_t)(v), x[4 * i + 0], s0);
    s1 = fmaf((float)(int8_t)(v >> 8), x[4 * i + 1], s1);
    s0 = fmaf((float)(int8_t)(v >> 16), x[4 * i + 2], s0);
    s1 = fmaf((float)(int8_t)(v >> 24), x[4 * i + 3], s1);
  }
  return s0 + s1;
}

template <int RPW, int EPI>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs &a, float (&acc)[RPW][kMaxRows],
                                              int row0) {
  // every lane holds the reduced sums; lane 0 stores
  if ((threadIdx.x & 63) != 0) return;
#pragma unroll
  for (int m = 0; m < kMaxRows; m++) {
    if (m >= a.M) break;
    float *y = a.y + (size_t)m * a.ldy;
    if (EPI == EPI_SWIGLU) {
#pragma unroll
      for (int p = 0; p < RPW / 2; p++) {
        const int j = row0 / 2 + p;
        if (2 * j + 1 < a.N) y[j] = silu_mul(acc[2 * p][m], acc[2 * p + 1][m]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < RPW; r++) {
        const int row = row0 + r;
        if (row < a.N) {
          if (EPI == EPI_ADD)
            y[row] += acc[r][m];
          else
            y[row] = acc[r][m];
        }
      }
    }
  }
}

// y[m][n] (+)= sum_k W[n][k] xn[m][k]: Q8_0 weights, f32 activations.
// Each wave owns RPW consecutive rows; a lane owns 16-column segments.
template <int RPW, int EPI>
__global__ __launch_bounds__(kBlock) void k_gemv_q8(GemvArgs a) {
  extern __shared__ float xs[];
  stage_rows(a.x, a.ldx, a.M, a.K, a.norm_w, a.eps, xs, a.xn_out);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * (kBlock / 64) + wave) * RPW;
  if (row0 >= a.N) return;
  const int K = a.K, M = a.M, nseg = K >> 4, nb = K >> 5;
  float acc[RPW][kMaxRows];
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int m = 0; m < kMaxRows; m++) acc[r][m] = 0.f;
  const int8_t *wq[RPW];
  const _Float16 *wd[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const int row = min(row0 + r, a.N - 1);
    wq[r] = a.wq + (size_t)row * K;
    wd[r] = a.wd + (size_t)row * nb;
  }
  for (int seg = lane; seg < nseg; seg += 64) {
    int4 wv[RPW];
    float sc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      wv[r] = *reinterpret_cast<const int4 *>(wq[r] + seg * 16);
      sc[r] = (float)wd[r][seg >> 1];
    }
#pragma unroll
    for (int m = 0; m < kMaxRows; m++) {
      if (m < M) {
        float xv[16];
        const float4 *xp = reinterpret_cast<const float4 *>(xs + m * K + seg * 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float4 t = xp[i];
          xv[4 * i] = t.x;
          xv[4 * i + 1] = t.y;
          xv[4 * i + 2] = t.z;
          xv[4 * i + 3] = t.w;
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) acc[r][m] = fmaf(sc[r], dot16_i8(wv[r], xv), acc[r][m]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int m = 0; m < kMaxRows; m++)
      if (m < M) acc[r][m] = wave_sum(acc[r][m]);
  gemv_epilogue<RPW, EPI>(a, acc, row0);
}

// Same over f32 weights: a lane owns 4-column segments (coalesced 1 KB per
// wave instruction).
template <int RPW, int EPI>
__global__ __launch_bounds__(kBlock) void k_gemv_f32(GemvArgs a) {
  extern __shared__ float xs[];
  stage_rows(a.x, a.ldx, a.M, a.K, a.norm_w, a.eps, xs, a.xn_out);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * (kBlock / 64) + wave) * RPW;
  if (row0 >= a.N) return;
  const int K = a.K, M = a.M, nseg = K >> 2;
  float acc[RPW][kMaxRows];
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int m = 0; m < kMaxRows; m++) acc[r][m] = 0.f;
  const float *wf[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) wf[r] = a.wf + (size_t)min(row0 + r, a.N - 1) * K;
  for (int seg = lane; seg < nseg; seg += 64) {
    float4 wv[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) wv[r] = reinterpret_cast<const float4 *>(wf[r])[seg];
#pragma unroll
    for (int m = 0; m < kMaxRows; m++) {
      if (m < M) {
        const float4 xv = reinterpret_cast<const float4 *>(xs + m * K)[seg];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
          float s = acc[r][m];
          s = fmaf(wv[r].x, xv.x, s);
          s = fmaf(wv[r].y, xv.y, s);
          s = fmaf(wv[r].z, xv.z, s);
          s = fmaf(wv[r].w, xv.w, s);
          acc[r][m] = s;
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int m = 0; m < kMaxRows; m++)
      if (m < M) acc[r][m] = wave_sum(acc[r][m]);
  gemv_epilogue<RPW, EPI>(a, acc, row0);
}

template <int RPW>
static void gemv_dispatch(const GemvArgs &a, int epi, bool q8, hipStream_t st) {
  const int rows_per_block = (kBlock / 64) * RPW;
  const dim3 grid((a.N + rows_per_block - 1) / rows_per_block);
  const size_t lds = sizeof(float) * a.M * a.K;
#define Q3H_GEMV(KER, E) hipLaunchKernelGGL((KER<RPW, E>), grid, dim3(kBlock), lds, st, a)
  if (q8) {
    if (epi == EPI_STORE) Q3H_GEMV(k_gemv_q8, EPI_STORE);
    else if (epi == EPI_ADD) Q3H_GEMV(k_gemv_q8, EPI_ADD);
    else Q3H_GEMV(k_gemv_q8, EPI_SWIGLU);
  } else {
    if (epi == EPI_STORE) Q3H_GEMV(k_gemv_f32, EPI_STORE);
    else if (epi == EPI_ADD) Q3H_GEMV(k_gemv_f32, EPI_ADD);
    else Q3H_GEMV(k_gemv_f32, EPI_SWIGLU);
  }
#undef Q3H_GEMV
}

// Rows per wave: keep >= ~256 blocks on the 256 CUs when the matrix allows;
// SwiGLU needs gate/up pairs inside one wave.
void launch_gemv(const GemvArgs &a0, int epi, bool q8, hipStream_t st) {
  GemvArgs a = a0;
  for (int m0 = 0; m0 < a0.M; m0 += kMaxRows) {
    a.M = min(kMaxRows, a0.M - m0);
    a.x = a0.x + (size_t)m0 * a0.ldx;
    a.y = a0.y + (size_t)m0 * a0.ldy;
    a.xn_out = (m0 + a.M == a0.M) ? a0.xn_out : nullptr;
    // the Qwen3-TTS widths: one workgroup per CU, loads issued up front
    if (q8 && launch_gemv_q8_wide(a, epi, st)) continue;
    const int waves = a.N;  // with RPW = 1
    if (epi == EPI_SWIGLU || waves >= 8192)
      gemv_dispatch<4>(a, epi, q8, st);
    else if (waves >= 2048)
      gemv_dispatch<2>(a, epi, q8, st);
    else
      gemv_dispatch<1>(a, epi, q8, st);
  }
}

// ---------------------------------------------------------------------------
// row descriptors and context lengths

__global__ void k_prep(CtxDev *const *cs, const int *alive, int n, int R, RowDesc *rd) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * R) return;
  const int s = i / R, r = i % R;
  const CtxDev *c = global_ptr(cs[s]);
  RowDesc d;
  d.k = c->k;
  d.v = c->v;
  d.max_pos = c->max_pos;
  const int pos = c->len + r;
  d.pos = (alive && !alive[s]) || pos >= c->max_pos ? -1 : pos;
  rd[i] = d;
}

__global__ void k_advance(CtxDev *const *cs, const int *alive, int n, int R) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= n) return;
  if (alive && !alive[s]) return;
  CtxDev *c = global_ptr(cs[s]);
  c->len = min(c->len + R, c->max_pos);
}

void launch_prep(CtxDev *const *cs, const int *alive, int n, int R, RowDesc *rd,
                 hipStream_t st) {
  hipLaunchKernelGGL(k_prep, dim3((n * R + 63) / 64), dim3(64), 0, st, cs, alive, n, R, rd);
}

void launch_advance(CtxDev *const *cs, const int *alive, int n, int R, hipStream_t st) {
  hipLaunchKernelGGL(k_advance, dim3((n + 63) / 64), dim3(64), 0, st, cs, alive, n, R);
}

// ---------------------------------------------------------------------------
// QK-norm, RoPE, K/V append: one wave per head vector (q heads, k heads,
// v heads of each row); a lane holds elements i and i + head_dim/2, the pair
// that rotate_half mixes.

template <typename KV>
__global__ __launch_bounds__(kBlock) void k_qk_rope_append(
    float *qkv, int ldq, const RowDesc *rd, int layer, int heads, int kvh, int hd,
    const float *qn, const float *kn, float eps, const float2 *rope_cs, const float *part,
    int nsl) {
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  const int m = blockIdx.y;
  if (j >= heads + 2 * kvh) return;
  const RowDesc d = rd[m];
  if (d.pos < 0) return;
  const int half = hd >> 1;
  float *vec = qkv + (size_t)m * ldq + (size_t)j * hd;
  const bool on = lane < half;
  float x0 = 0.f, x1 = 0.f;
  if (nsl > 0) {
    // the slices' loads issued together (clamped), added in slice order
    const int M = gridDim.y;
    float a0[kRopeMaxSlices], a1[kRopeMaxSlices];
#pragma unroll
    for (int z = 0; z < kRopeMaxSlices; z++) {
      const float *p = part + ((size_t)min(z, nsl - 1) * M + m) * ldq + (size_t)j * hd;
      a0[z] = on ? p[lane] : 0.f;
      a1[z] = on ? p[lane + half] : 0.f;
    }
    x0 = a0[0];
    x1 = a1[0];
#pragma unroll
    for (int z = 1; z < kRopeMaxSlices; z++)
      if (z < nsl) x0 += a0[z], x1 += a1[z];
  } else if (on) {
    x0 = vec[lane];
    x1 = vec[lane + half];
  }
  if (j < heads + kvh) {
    const float *w = j < heads ? qn : kn;
    double ss = (double)x0 * x0 + (double)x1 * x1;
    ss = wave_sum_d(ss);
    const float inv = (float)(1.0 / sqrt(ss / hd + (double)eps));
    if (on) {
      x0 = w[lane] * (x0 * inv);
      x1 = w[lane + half] * (x1 * inv);
      const float2 cs = rope_cs[(size_t)d.pos * half + lane];
      rope_pair(x0, x1, cs.x, cs.y);
    }
  }
  if (!on) return;
  if (j < heads) {
    vec[lane] = x0;
    vec[lane + half] = x1;
    return;
  }
  const int g = j < heads + kvh ? j - heads : j - heads - kvh;
  void *base = j < heads + kvh ? d.k : d.v;
  KV *dst = global_ptr(reinterpret_cast<KV *>(base)) +
            (((size_t)layer * kvh + g) * d.max_pos + d.pos) * hd;
  dst[lane] = to_cache<KV>(x0);
  dst[lane + half] = to_cache<KV>(x1);
}

void launch_qk_rope_append(float *qkv, int ldq, const RowDesc *rd, int M, int layer,
                           int heads, int kvh, int hd, const float *qn, const float *kn,
                           float eps, const float *rope_cs, bool kv16, hipStream_t st,
                           const float *part, int nsl) {
  require(part == nullptr || (nsl >= 1 && nsl <= kRopeMaxSlices), Q3H_E_ARG,
          "launch_qk_rope_append: 1 to 4 slices");
  const int ns = part ? nsl : 0;
  const dim3 grid((heads + 2 * kvh + 3) / 4, M);
  const float2 *cs = reinterpret_cast<const float2 *>(rope_cs);
  if (kv16)
    hipLaunchKernelGGL(k_qk_rope_append<_Float16>, grid, dim3(kBlock), 0, st, qkv, ldq, rd,
                       layer, heads, kvh, hd, qn, kn, eps, cs, part, ns);
  else
    hipLaunchKernelGGL(k_qk_rope_append<float>, grid, dim3(kBlock), 0, st, qkv, ldq, rd,
                       layer, heads, kvh, hd, qn, kn, eps, cs, part, ns);
}

// ---------------------------------------------------------------------------
// plain row RMSNorm (the final norm of a stack)

__global__ __launch_bounds__(kBlock) void k_rmsnorm_rows(const float *x, int ldx, int K,
                                                         const float *w, float eps,
                                                         float *y, int ldy) {
  __shared__ double red[kBlock / 64];
  const int m = blockIdx.x, tid = threadIdx.x;
  const float *xr = x + (size_t)m * ldx;
  double ss = 0.0;
  for (int k = tid; k < K; k += kBlock) ss += (double)xr[k] * xr[k];
  ss = wave_sum_d(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < kBlock / 64; i++) t += red[i];
  const float inv = (float)(1.0 / sqrt(t / K + (double)eps));
  for (int k = tid; k < K; k += kBlock) y[(size_t)m * ldy + k] = w[k] * (xr[k] * inv);
}

void launch_rmsnorm_rows(const float *x, int ldx, int M, int K, const float *w, float eps,
                         float *y, int ldy, hipStream_t st) {
  hipLaunchKernelGGL(k_rmsnorm_rows, dim3(M), dim3(kBlock), 0, st, x, ldx, K, w, eps, y, ldy);
}

// ---------------------------------------------------------------------------
// load-time conversion: f32 rows -> Q8_0 (ggml quantize_row_q8_0_ref: d =
// amax/127 rounded to fp16, q = round(x * (1/d)) half away from zero, both
// divisions correctly rounded), ggml blocks -> structure of arrays, f32 row
// copies; dst row = src row * row_stride + row_off (fused QKV, interleaved
// gate/up).

// a source element widened to f32 (BF16: the high half of an f32, exact)
template <bool BF16>
__device__ __forceinline__ float src_elem(const void *src, size_t i) {
  if constexpr (BF16)
    return __uint_as_float((uint32_t) static_cast<const uint16_t *>(src)[i] << 16);
  else
    return static_cast<const float *>(src)[i];
}

template <bool BF16>
__global__ void k_quantize_q8(const void *src, int rows, int K, int8_t *q, _Float16 *d,
                              int row_stride, int row_off) {
  const int nb = K >> 5;
  const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= (size_t)rows * nb) return;
  const int r = (int)(b / nb), i = (int)(b % nb);
  const size_t x0 = (size_t)r * K + i * 32;
  float v[32];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 32; j++) {
    v[j] = src_elem<BF16>(src, x0 + j);
    const float a = fabsf(v[j]);
    amax = amax > a ? amax : a;
  }
  const float dd = __fdiv_rn(amax, 127.0f);
  const float id = dd != 0.f ? __fdiv_rn(1.0f, dd) : 0.f;
  const size_t orow = (size_t)r * row_stride + row_off;
  d[orow * nb + i] = (_Float16)dd;
  int8_t *qo = q + orow * K + i * 32;
#pragma unroll
  for (int j = 0; j < 32; j++) qo[j] = (int8_t)roundf(__fmul_rn(v[j], id));
}

__global__ void k_repack_q8(const uint8_t *blocks, int rows, int K, int8_t *q, _Float16 *d,
                            int row_stride, int row_off) {
  const int nb = K >> 5;
  const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= (size_t)rows * nb) return;
  const int r = (int)(b / nb), i = (int)(b % nb);
  const uint8_t *src = blocks + b * 34;
  const size_t orow = (size_t)r * row_stride + row_off;
  const uint16_t bits = (uint16_t)src[0] | ((uint16_t)src[1] << 8);
  d[orow * nb + i] = __builtin_bit_cast(_Float16, bits);
  int8_t *qo = q + orow * K + i * 32;
#pragma unroll
  for (int j = 0; j < 32; j++) qo[j] = (int8_t)src[2 + j];
}

template <bool BF16>
__global__ void k_copy_rows_f32(const void *src, int rows, int K, float *dst, int row_stride,
                                int row_off) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)rows * K) return;
  const int r = (int)(i / K), k = (int)(i % K);
  dst[((size_t)r * row_stride + row_off) * K + k] = src_elem<BF16>(src, i);
}

void launch_quantize_q8(const void *src, bool bf16, int rows, int K, int8_t *q, _Float16 *d,
                        int row_stride, int row_off, hipStream_t st) {
  const size_t n = (size_t)rows * (K >> 5);
  const dim3 grid((unsigned)((n + 255) / 256));
  if (bf16)
    hipLaunchKernelGGL(k_quantize_q8<true>, grid, dim3(256), 0, st, src, rows, K, q, d,
                       row_stride, row_off);
  else
    hipLaunchKernelGGL(k_quantize_q8<false>, grid, dim3(256), 0, st, src, rows, K, q, d,
                       row_stride, row_off);
}

void launch_repack_q8(const uint8_t *blocks, int rows, int K, int8_t *q, _Float16 *d,
                      int row_stride, int row_off, hipStream_t st) {
  const size_t n = (size_t)rows * (K >> 5);
  hipLaunchKernelGGL(k_repack_q8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, blocks,
                     rows, K, q, d, row_stride, row_off);
}

void launch_copy_rows_f32(const void *src, bool bf16, int rows, int K, float *dst,
                          int row_stride, int row_off, hipStream_t st) {
  const size_t n = (size_t)rows * K;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (bf16)
    hipLaunchKernelGGL(k_copy_rows_f32<true>, grid, dim3(256), 0, st, src, rows, K, dst,
                       row_stride, row_off);
  else
    hipLaunchKernelGGL(k_copy_rows_f32<false>, grid, dim3(256), 0, st, src, rows, K, dst,
                       row_stride, row_off);
}

// K/V fill / read (long-context setups, tests): src [layers][kvh][len][hd]
template <typename KV>
__global__ void k_kv_fill(const float *src, int layers, int kvh, int len, int hd, KV *dst,
                          int max_pos) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t n = (size_t)layers * kvh * len * hd;
  if (i >= n) return;
  const int dd = (int)(i % hd);
  const size_t t = i / hd;
  const int p = (int)(t % len);
  const size_t lg = t / len;  // layer * kvh + g
  dst[(lg * max_pos + p) * hd + dd] = (KV)src[i];
}

template <typename KV>
__global__ void k_kv_read(const KV *src, int layer, int kvh, int len, int hd, int max_pos,
                          float *dst) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t n = (size_t)kvh * len * hd;
  if (i >= n) return;
  const int dd = (int)(i % hd);
  const size_t t = i / hd;
  const int p = (int)(t % len), g = (int)(t / len);
  dst[i] = (float)src[(((size_t)layer * kvh + g) * max_pos + p) * hd + dd];
}

void launch_kv_fill(const float *src, int layers, int kvh, int len, int hd, void *dst,
                    int max_pos, bool kv16, hipStream_t st) {
  const size_t n = (size_t)layers * kvh * len * hd;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (kv16)
    hipLaunchKernelGGL(k_kv_fill<_Float16>, grid, dim3(256), 0, st, src, layers, kvh, len, hd,
                       (_Float16 *)dst, max_pos);
  else
    hipLaunchKernelGGL(k_kv_fill<float>, grid, dim3(256), 0, st, src, layers, kvh, len, hd,
                       (float *)dst, max_pos);
}

void launch_kv_read(const void *src, int layer, int kvh, int len, int hd, int max_pos,
                    bool kv16, float *dst, hipStream_t st) {
  const size_t n = (size_t)kvh * len * hd;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (kv16)
    hipLaunchKernelGGL(k_kv_read<_Float16>, grid, dim3(256), 0, st, (const _Float16 *)src,
                       layer, kvh, len, hd, max_pos, dst);
  else
    hipLaunchKernelGGL(k_kv_read<float>, grid, dim3(256), 0, st, (const float *)src, layer,
                       kvh, len, hd, max_pos, dst);
}

}  // namespace q3h
