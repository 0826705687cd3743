// q3h_attnx.hip - GQA attention of the int8 path (stacks with act_q8 = 1):
// a fixed evaluation order, followed to the bit by the CPU restatement of the
// same layer, and the Q8_0 quantization of its output (the o_proj input)
// fused into the epilogue. The int8 products make the layer output a
// discontinuous function of the attention output (one element on the other
// side of a rounding boundary of its block moves it by d / 127 of the block
// maximum), so this path computes every fp32 value in one documented order
// instead of to a tolerance.
//
// One workgroup of 256 threads per (query head, row):
//  - prologue (a decode row, one new position of its own context): RMSNorm
//    of q and of the new k (double sum of squares), RoPE as rope_pair, v
//    copied; the first query head of the kv group appends k, v to the cache;
//    the others use their own copy for the new position;
//  - scores: 16 lanes per key, lane l a fused multiply-add chain over dims
//    8l .. 8l + 7, a balanced pairwise tree over the 16 lanes (DPP row
//    operations), times 1/sqrt(128);
//  - softmax: maximum, exp_ieee(s - max), double sum, inv = (float)(1/sum),
//    weights s * inv;
//  - values: 4 chains of fused multiply-adds over the positions p = j mod 4
//    (a thread per chain and pair of dims, 512 coalesced bytes per key and
//    wave), joined as (c0 + c1) + (c2 + c3);
//  - the head's 128 outputs quantized per 32-block (ggml quantize_row_q8_0_ref
//    semantics) into the operand tiles of the int8 product.
// The attention itself follows src/tts/mormot.ai.tts.qwen.lm.pas (TQwenLm.
// Forward, lm.pas:391-408) through the stack's ForwardEmbeds: causal softmax
// attention with head_dim 128, q head h reading kv head h / (heads / kv_heads).
#include <hip/hip_runtime.h>

#include "q3h_internal.h"
#include "q3h_math.h"
#include "q3h_wave.h"

namespace q3h {
namespace {

constexpr int HD = 128;
constexpr int NT = 256;

template <typename KV>
__device__ __forceinline__ void load8(const KV *p, float (&o)[8]) {
  if constexpr (sizeof(KV) == 4) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0];
    const float4 b = reinterpret_cast<const float4 *>(p)[1];
    o[0] = a.x, o[1] = a.y, o[2] = a.z, o[3] = a.w;
    o[4] = b.x, o[5] = b.y, o[6] = b.z, o[7] = b.w;
  } else {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const h8 v = *reinterpret_cast<const h8 *>(p);
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = (float)v[e];
  }
}

template <typename KV>
__device__ __forceinline__ float2 load2(const KV *p) {
  if constexpr (sizeof(KV) == 4) {
    return *reinterpret_cast<const float2 *>(p);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 v = *reinterpret_cast<const h2 *>(p);
    return make_float2((float)v[0], (float)v[1]);
  }
}

// sum over a 16-lane DPP row, the balanced pairwise tree in lane order
// ((l0 + l1) + (l2 + l3)) + ..., the same value in all 16 lanes
__device__ __forceinline__ float row16_tree(float v) {
  v = __fadd_rn(v, dpp_f<kQuadXor1>(v));
  v = __fadd_rn(v, dpp_f<kQuadXor2>(v));
  v = __fadd_rn(v, dpp_f<kHalfMirror>(v));
  v = __fadd_rn(v, dpp_f<kRowMirror>(v));
  return v;
}

template <typename KV, bool FUSED>
__global__ __launch_bounds__(NT) void k_attn_x(const RowDesc *rd, const float *qkv, int ldq,
                                               const float *qkn, const float2 *rope_cs,
                                               int layer, int heads, int kvh, int8_t *xq,
                                               float *dx, int M) {
  extern __shared__ float sc[];  // per position: score, then e^(score - max)
  __shared__ float qs[HD], kn[HD], vn[HD];
  __shared__ float cv[4][HD];
  __shared__ float redf[NT / 64];
  __shared__ double redd[NT / 64];
  const int h = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int grp = heads / kvh, g = h / grp;
  const int NQ = heads * HD, nbq = NQ >> 5, mt16 = (M + 15) >> 4;
  const RowDesc d = rd[m];
  // this head's 4 output blocks in the operand tiles: byte of element k of
  // row m at ((b * mt16 + m / 16) * 64 + (k % 32) / 8 * 16 + m % 16) * 8 + k % 8
  const int kk = t & 31, bg = h * 4 + (t >> 5);
  const size_t qoff =
      (((size_t)bg * mt16 + (m >> 4)) * 64 + (kk >> 3) * 16 + (m & 15)) * 8 + (kk & 7);
  if (d.pos < 0) {  // inactive row: zero blocks
    if (t < HD) {
      xq[qoff] = 0;
      if (kk == 0) dx[(size_t)m * nbq + bg] = 0.f;
    }
    return;
  }
  const int pos = d.pos, L = pos + 1;
  const float *row = qkv + (size_t)m * ldq;
  const size_t head_off = ((size_t)layer * kvh + g) * d.max_pos * HD;
  const KV *kc = reinterpret_cast<const KV *>(d.k) + head_off;
  const KV *vc = reinterpret_cast<const KV *>(d.v) + head_off;

  if (FUSED) {
    if (wave < 2) {  // wave 0: q, wave 1: the new k
      const float *src = wave == 0 ? row + (size_t)h * HD : row + NQ + (size_t)g * HD;
      const float *w = qkn + (wave == 0 ? 0 : HD);
      const float eps = qkn[2 * HD];
      float x0 = src[lane], x1 = src[lane + 64];
      double ss = (double)x0 * (double)x0 + (double)x1 * (double)x1;
      ss = wave_sum_dpp_d(ss);
      const float inv = (float)(1.0 / sqrt(ss / HD + (double)eps));
      x0 = w[lane] * (x0 * inv);
      x1 = w[lane + 64] * (x1 * inv);
      const float2 cs = rope_cs[(size_t)pos * (HD / 2) + lane];
      rope_pair(x0, x1, cs.x, cs.y);
      if (wave == 0) {
        qs[lane] = x0;
        qs[lane + 64] = x1;
      } else {
        const KV k0 = (KV)x0, k1 = (KV)x1;  // the cache's precision
        kn[lane] = (float)k0;
        kn[lane + 64] = (float)k1;
        if (h % grp == 0) {
          KV *dst = const_cast<KV *>(kc) + (size_t)pos * HD;
          dst[lane] = k0;
          dst[lane + 64] = k1;
        }
      }
    } else if (wave == 2) {  // the new v
      const float *src = row + NQ + (size_t)(kvh + g) * HD;
      const KV v0 = (KV)src[lane], v1 = (KV)src[lane + 64];
      vn[lane] = (float)v0;
      vn[lane + 64] = (float)v1;
      if (h % grp == 0) {
        KV *dst = const_cast<KV *>(vc) + (size_t)pos * HD;
        dst[lane] = v0;
        dst[lane + 64] = v1;
      }
    }
  } else if (t < HD) {
    qs[t] = row[(size_t)h * HD + t];  // normed and rotated by the append kernel
  }
  __syncthreads();

  // scores: key group kg = t / 16 takes positions kg, kg + 16, ...
  const float scale = (float)(1.0 / __builtin_sqrt((double)HD));
  {
    const int kg = t >> 4, li = t & 15;
    float qv[8];
#pragma unroll
    for (int e = 0; e < 8; e++) qv[e] = qs[8 * li + e];
    for (int p0 = 0; p0 < L; p0 += NT / 16) {
      const int p = p0 + kg;
      float a = 0.f;
      if (p < L) {
        float k8[8];
        if (FUSED && p == pos) {
#pragma unroll
          for (int e = 0; e < 8; e++) k8[e] = kn[8 * li + e];
        } else {
          load8(kc + (size_t)p * HD + 8 * li, k8);
        }
#pragma unroll
        for (int e = 0; e < 8; e++) a = fmaf(qv[e], k8[e], a);
      }
      a = row16_tree(a);
      if (p < L && li == 0) sc[p] = __fmul_rn(a, scale);
    }
  }
  __syncthreads();

  // softmax
  float mx = -INFINITY;
  for (int p = t; p < L; p += NT) mx = fmaxf(mx, sc[p]);
  mx = wave_max_dpp(mx);
  if (lane == 0) redf[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(redf[0], redf[1]), fmaxf(redf[2], redf[3]));
  double sum = 0.0;
  for (int p = t; p < L; p += NT) {
    const float e = exp_ieee(__fsub_rn(sc[p], mx));
    sc[p] = e;
    sum += (double)e;
  }
  sum = wave_sum_dpp_d(sum);
  if (lane == 0) redd[wave] = sum;
  __syncthreads();
  const float inv = (float)(1.0 / ((redd[0] + redd[1]) + (redd[2] + redd[3])));

  // values: chain j = wave over positions p = j mod 4, dims 2 lane, 2 lane + 1
  {
    float c0 = 0.f, c1 = 0.f;
    for (int p = wave; p < L; p += 4) {
      const float w = __fmul_rn(sc[p], inv);
      float2 v;
      if (FUSED && p == pos)
        v = make_float2(vn[2 * lane], vn[2 * lane + 1]);
      else
        v = load2(vc + (size_t)p * HD + 2 * lane);
      c0 = fmaf(w, v.x, c0);
      c1 = fmaf(w, v.y, c1);
    }
    cv[wave][2 * lane] = c0;
    cv[wave][2 * lane + 1] = c1;
  }
  __syncthreads();

  // quantize the head's 128 outputs per 32-block
  if (t < HD) {
    const float o = __fadd_rn(__fadd_rn(cv[0][t], cv[1][t]), __fadd_rn(cv[2][t], cv[3][t]));
    float amax = fabsf(o);
#pragma unroll
    for (int s = 16; s >= 1; s >>= 1) amax = fmaxf(amax, __shfl_xor(amax, s));
    const float dq = __fdiv_rn(amax, 127.0f);
    const float id = dq != 0.f ? __fdiv_rn(1.0f, dq) : 0.f;
    xq[qoff] = (int8_t)(int)roundf(__fmul_rn(o, id));
    if (kk == 0) dx[(size_t)m * nbq + bg] = (float)(_Float16)dq;
  }
}

}  // namespace

bool attn_x_supported(int heads, int kvh, int head_dim, int max_positions) {
  return head_dim == HD && kvh > 0 && heads % kvh == 0 && max_positions > 0 &&
         max_positions <= kAttnXMaxPositions;
}

void launch_attn_x(const AttnArgs &a, int M, bool fused, bool kv16, const QAct &xa,
                   int max_positions, hipStream_t st) {
  const dim3 grid(a.heads, M);
  const size_t lds = sizeof(float) * (size_t)max_positions;
#define Q3H_ATTNX(KV, F)                                                                    \
  hipLaunchKernelGGL((k_attn_x<KV, F>), grid, dim3(NT), lds, st, a.rd, a.qkv, a.ldq, a.qkn, \
                     a.rope_cs, a.layer, a.heads, a.kvh, xa.q, xa.d, M)
  if (kv16) {
    if (fused)
      Q3H_ATTNX(_Float16, true);
    else
      Q3H_ATTNX(_Float16, false);
  } else {
    if (fused)
      Q3H_ATTNX(float, true);
    else
      Q3H_ATTNX(float, false);
  }
#undef Q3H_ATTNX
}

}  // namespace q3h
