// q3h_cp.hip - the code predictor's single-row step, attention fused into the
// output projection.
//
// A code-predictor context holds at most 16 positions (one frame's codes), so
// its attention is cheap enough to be recomputed by every workgroup of the
// o_proj product. One launch does, for the new row at position pos of one
// context:
//   QK-norm + RoPE of the 16 query heads and 8 keys (rows of the raw q/k/v
//   product), the K/V append at pos (workgroup 0 writes it; every workgroup
//   uses its own copy for that position), causal softmax attention over
//   positions 0..pos, then h[rows] += Wo[rows] . attention for the workgroup's
//   16 rows of Wo (Q8_0).
// That is one launch instead of two (attention, o_proj) and no attention
// output round trip through memory; every workgroup computes the same
// attention, so the result does not depend on scheduling.
//
// Shape (the Qwen3-TTS code predictor): hidden 1024, 16 query heads and 8 kv
// heads of 128, 16 positions. 128 workgroups of 8 waves; wave w serves kv
// head w for the attention, then one row of Wo.
//
// Layouts: K/V cache of the layer [8][16][128] (kl), values at kl + v_off;
// q_norm, k_norm, then the RMSNorm epsilon (qkn); the RoPE (cos, sin) row of pos (rope); Wo quants
// [1024][2048] followed by their fp16 scales [1024][64].
#include <hip/hip_runtime.h>

#include "q3h.h"
#include "q3h_internal.h"
#include "q3h_math.h"
#include "q3h_wave.h"

namespace q3h {

namespace {

constexpr int HD = 128, KVH = 8, GRP = 2, NQ = KVH * GRP * HD, HID = 1024;
constexpr int P = 16;     // positions of a code-predictor context
constexpr int ROWS = 8;   // o_proj rows per workgroup: one per wave
constexpr int NT = 512;   // 8 waves
constexpr int NBO = NQ / 32;

__device__ __forceinline__ void ld32(const float *p, float *o) {
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float4 t = reinterpret_cast<const float4 *>(p)[i];
    o[4 * i] = t.x;
    o[4 * i + 1] = t.y;
    o[4 * i + 2] = t.z;
    o[4 * i + 3] = t.w;
  }
}

__device__ __forceinline__ void ld32(const _Float16 *p, float *o) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const h8 t = reinterpret_cast<const h8 *>(p)[i];
#pragma unroll
    for (int j = 0; j < 8; j++) o[8 * i + j] = (float)t[j];
  }
}

__device__ __forceinline__ float2 ld2(const float *p) { return *reinterpret_cast<const float2 *>(p); }

__device__ __forceinline__ float2 ld2(const _Float16 *p) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 t = *reinterpret_cast<const h2 *>(p);
  return make_float2((float)t[0], (float)t[1]);
}

__device__ __forceinline__ float dot4(int w, float4 x, float acc) {
  acc = fmaf((float)(int8_t)(w), x.x, acc);
  acc = fmaf((float)(int8_t)(w >> 8), x.y, acc);
  acc = fmaf((float)(int8_t)(w >> 16), x.z, acc);
  acc = fmaf((float)(int8_t)(w >> 24), x.w, acc);
  return acc;
}

// RMSNorm over a head (lanes hold elements lane, lane + 64), weight (w0, w1),
// then rotate_half RoPE with (cos, sin) = cs; fp32 throughout
__device__ __forceinline__ void norm_rope(float &x0, float &x1, float w0, float w1, float2 cs,
                                          float eps) {
  const float ss = wave_sum_dpp(fmaf(x0, x0, x1 * x1));
  const float inv = 1.0f / sqrtf(ss * (1.0f / HD) + eps);
  const float a = w0 * (x0 * inv), b = w1 * (x1 * inv);
  x0 = a;
  x1 = b;
  rope_pair(x0, x1, cs.x, cs.y);
}

// LDS written by some lanes of a wave and read by others of the same wave
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename KV>
__global__ __launch_bounds__(NT) void k_attn_o_cp(const int8_t *__restrict__ wo,
                                                  const float *__restrict__ qkv,
                                                  KV *__restrict__ kl, float *__restrict__ h,
                                                  const float *__restrict__ qkn,
                                                  const float2 *__restrict__ rope, int pos,
                                                  int v_off) {
  __shared__ float att[NQ];
  __shared__ float qs[KVH][GRP][HD];
  __shared__ float kvs[KVH][2][HD];  // the new key and value of each kv head
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = blockIdx.x * ROWS + w;  // this wave's o_proj row
  const _Float16 *wd = reinterpret_cast<const _Float16 *>(wo + (size_t)HID * NQ);

  // 1. every load up front: the Wo row, the residual, the raw q/k/v of kv
  // head w, the norm weights, the RoPE row, the cached keys and values
  int4 wv[2];
  float sc[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    wv[c] = *reinterpret_cast<const int4 *>(wo + (size_t)row * NQ + c * 1024 + lane * 16);
    sc[c] = (float)wd[(size_t)row * NBO + c * 32 + (lane >> 1)];
  }
  const float hr = h[row];
  float xq[GRP][2], xk[2], xv[2];
#pragma unroll
  for (int j = 0; j < GRP; j++) {
    xq[j][0] = qkv[(w * GRP + j) * HD + lane];
    xq[j][1] = qkv[(w * GRP + j) * HD + lane + 64];
  }
  xk[0] = qkv[NQ + w * HD + lane];
  xk[1] = qkv[NQ + w * HD + lane + 64];
  xv[0] = qkv[NQ + KVH * HD + w * HD + lane];
  xv[1] = qkv[NQ + KVH * HD + w * HD + lane + 64];
  const float qn0 = qkn[lane], qn1 = qkn[lane + 64];
  const float kn0 = qkn[HD + lane], kn1 = qkn[HD + lane + 64];
  const float eps = qkn[2 * HD];
  const float2 cs = rope[lane];
  KV *kh = kl + (size_t)w * P * HD;
  KV *vh = kl + v_off + (size_t)w * P * HD;
  // keys: lane 4p + j holds dims 32j .. 32j + 31 of key p
  const int kp = lane >> 2, kj = lane & 3;
  float kk[32];
  if (kp < pos) ld32(kh + (size_t)kp * HD + kj * 32, kk);
  // values: lane holds dims 2 lane, 2 lane + 1 of every cached position
  float2 vv[P];
#pragma unroll
  for (int p = 0; p < P; p++)
    if (p < pos) vv[p] = ld2(vh + (size_t)p * HD + 2 * lane);
  __builtin_amdgcn_sched_barrier(0);

  // 2. QK-norm + RoPE; the new key and value rounded as the cache holds them
#pragma unroll
  for (int j = 0; j < GRP; j++) {
    float x0 = xq[j][0], x1 = xq[j][1];
    norm_rope(x0, x1, qn0, qn1, cs, eps);
    qs[w][j][lane] = x0;
    qs[w][j][lane + 64] = x1;
  }
  {
    float x0 = xk[0], x1 = xk[1];
    norm_rope(x0, x1, kn0, kn1, cs, eps);
    const KV k0 = (KV)x0, k1 = (KV)x1, v0 = (KV)xv[0], v1 = (KV)xv[1];
    kvs[w][0][lane] = (float)k0;
    kvs[w][0][lane + 64] = (float)k1;
    kvs[w][1][lane] = (float)v0;
    kvs[w][1][lane + 64] = (float)v1;
    if (blockIdx.x == 0) {
      kh[(size_t)pos * HD + lane] = k0;
      kh[(size_t)pos * HD + lane + 64] = k1;
      vh[(size_t)pos * HD + lane] = v0;
      vh[(size_t)pos * HD + lane + 64] = v1;
    }
  }
  wave_lds_sync();

  // 3. scores of key kp (the new key from LDS), softmax over 0..pos; the
  // probability of key p ends up in lanes 4p .. 4p + 3
  if (kp == pos) {
#pragma unroll
    for (int i = 0; i < 32; i++) kk[i] = kvs[w][0][kj * 32 + i];
  }
  const float scale = (float)(1.0 / sqrt((double)HD));
  const bool live = kp <= pos;
  float pr[GRP];
#pragma unroll
  for (int j = 0; j < GRP; j++) {
    const float *q = &qs[w][j][kj * 32];
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i += 2) {
      a0 = fmaf(q[i], kk[i], a0);
      a1 = fmaf(q[i + 1], kk[i + 1], a1);
    }
    float a = a0 + a1;
    a += dpp_f<kQuadXor1>(a);
    a += dpp_f<kQuadXor2>(a);
    const float sv = live ? a * scale : -INFINITY;
    const float mx = wave_max_dpp(sv);
    const float e = live ? expf(sv - mx) : 0.f;
    const float sum = wave_sum_dpp(kj == 0 ? e : 0.f);
    pr[j] = e * (1.0f / sum);
  }

  // 4. outputs (lane holds dims 2 lane, 2 lane + 1), probabilities read
  // from lane 4p
  float o[GRP][2];
#pragma unroll
  for (int j = 0; j < GRP; j++) o[j][0] = o[j][1] = 0.f;
#pragma unroll
  for (int p = 0; p < P; p++) {
    if (p < pos) {
#pragma unroll
      for (int j = 0; j < GRP; j++) {
        const float pw = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pr[j]), 4 * p));
        o[j][0] = fmaf(pw, vv[p].x, o[j][0]);
        o[j][1] = fmaf(pw, vv[p].y, o[j][1]);
      }
    }
  }
  {
    const float2 vn = make_float2(kvs[w][1][2 * lane], kvs[w][1][2 * lane + 1]);
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      const float pw = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pr[j]), 4 * pos));
      o[j][0] = fmaf(pw, vn.x, o[j][0]);
      o[j][1] = fmaf(pw, vn.y, o[j][1]);
      att[(w * GRP + j) * HD + 2 * lane] = o[j][0];
      att[(w * GRP + j) * HD + 2 * lane + 1] = o[j][1];
    }
  }
  __syncthreads();

  // 5. h[row] += Wo[row] . att
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const float4 *xp = reinterpret_cast<const float4 *>(att + c * 1024 + lane * 16);
    float p0 = dot4(wv[c].x, xp[0], 0.f);
    float p1 = dot4(wv[c].y, xp[1], 0.f);
    p0 = dot4(wv[c].z, xp[2], p0);
    p1 = dot4(wv[c].w, xp[3], p1);
    acc = fmaf(sc[c], p0 + p1, acc);
  }
  acc = wave_sum_dpp(acc);
  if (lane == 0) h[row] = hr + acc;
}

}  // namespace

bool cp_fused_supported(const q3h_stack_config &c) {
  return c.dtype == Q3H_Q8_0 && !c.act_q8 && c.hidden == HID && c.heads == KVH * GRP && c.kv_heads == KVH &&
         c.head_dim == HD;
}

void launch_attn_o_cp(const Mat &wo, const float *qkv, void *k_layer, int v_off, float *h,
                      const float *qkn, const float *rope_row, int pos, bool kv16,
                      hipStream_t st) {
  const dim3 grid(HID / ROWS), block(NT);
  const float2 *rope = reinterpret_cast<const float2 *>(rope_row);
  if (kv16)
    hipLaunchKernelGGL(k_attn_o_cp<_Float16>, grid, block, 0, st, wo.q, qkv,
                       static_cast<_Float16 *>(k_layer), h, qkn, rope, pos, v_off);
  else
    hipLaunchKernelGGL(k_attn_o_cp<float>, grid, block, 0, st, wo.q, qkv,
                       static_cast<float *>(k_layer), h, qkn, rope, pos, v_off);
}

}  // namespace q3h
