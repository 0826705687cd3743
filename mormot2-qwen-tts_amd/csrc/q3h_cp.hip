// q3h_cp.hip - the code predictor's attention fused into the output
// projection.
//
// A code-predictor context holds at most 16 positions (one frame's codes), so
// its attention is cheap enough to be recomputed by every workgroup of the
// o_proj product: one launch instead of two (attention, o_proj) and no
// attention output round trip through memory.
//
// The single-row step (k_attn_pair_cp) splits the product over the four
// kv-head pairs: workgroup b computes the causal attention of pair b % 4 only
// (QK-norm + RoPE of its 4 query heads and 2 keys, rows of the raw q/k/v
// product; the K/V append at pos by the pair's first workgroup) and the
// partial product of 16 Wo rows over the pair's 512 columns. The four
// partials go to part [4][1024] (h added to the first); the gate/up product
// that follows adds them in a fixed order, so the result does not depend on
// scheduling.
//
// The first step of a context (k_attn2_o_cp, positions 0 and 1 in one launch)
// keeps every kv head in each workgroup and adds its o_proj to h directly.
//
// Shape (the Qwen3-TTS code predictor): hidden 1024, 16 query heads and 8 kv
// heads of 128, 16 positions.
//
// Layouts: K/V cache of the layer [8][16][128] (kl), values at kl + v_off;
// q_norm, k_norm, then the RMSNorm epsilon (qkn); the RoPE (cos, sin) row of
// pos (rope); Wo quants [1024][2048] followed by their fp16 scales [1024][64].
#include <hip/hip_runtime.h>

#include <algorithm>

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

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 8 cache elements from one 16-byte load (f16) or two (f32), as f32
__device__ __forceinline__ void cvt8(const u32x4 (&r)[1], float (&o)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 v = __builtin_bit_cast(h8, r[0]);
#pragma unroll
  for (int e = 0; e < 8; e++) o[e] = (float)v[e];
}

__device__ __forceinline__ void cvt8(const u32x4 (&r)[2], float (&o)[8]) {
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) o[4 * i + e] = __uint_as_float(r[i][e]);
}

// The single-row step split over the four kv-head pairs, so that a workgroup
// computes the attention of one pair (4 query heads) instead of all 8 kv
// heads: workgroup b serves pair p = b % 4 (Wo columns 512 p .. 512 p + 511)
// and Wo rows 16 (b / 4) .. + 15; 256 workgroups of 4 waves, wave j = query
// head 4 p + j (kv head 2 p + j / 2). It writes the partial product
// part[p][row] = Wo[row][pair columns] . attention of the pair, with h[row]
// added in pair 0; the next product (RMSNorm + gate/up) adds the four
// partials in a fixed order, so the result does not depend on scheduling.
// Per wave: QK-norm + RoPE of its query head and of its kv head's new key, the
// K/V append at pos (the first workgroup of each pair, waves 0 and 2), the
// causal softmax over 0 .. pos as in k_attn_o_cp for one query head, then 4
// Wo rows of the pair's columns (two rows per 16-byte load, 32 lanes each).
constexpr int PAIRS = KVH / 2, PCOLS = NQ / PAIRS;  // 512 columns of Wo per pair
constexpr int PROWS = 16;                            // Wo rows per workgroup
constexpr int PNT = 256;                             // 4 waves

// NJ: cached positions per lane (4 NJ >= pos; slots past pos weigh exactly 0,
// so any such NJ gives the same sums)
template <typename KV, int NJ>
__global__ __launch_bounds__(PNT) void k_attn_pair_cp(const int8_t *__restrict__ wo,
                                                      const float *__restrict__ qkv,
                                                      KV *__restrict__ kl,
                                                      const float *__restrict__ qkn,
                                                      const float2 *__restrict__ rope, int pos,
                                                      int v_off, const float *__restrict__ h,
                                                      float *__restrict__ part) {
  constexpr int LW = sizeof(KV) / 2;
  static_assert(NJ >= 1 && 4 * NJ <= P, "positions per lane");
  __shared__ float att[4 * HD];         // the pair's 4 query heads
  __shared__ float qs[4][HD];
  __shared__ float kvs[4][2][HD];       // each wave's copy of its kv head's new key, value
  const int lane = threadIdx.x & 63, j = threadIdx.x >> 6;
  const int r16 = lane & 15, rg = lane >> 4;
  const int pair = blockIdx.x % PAIRS;
  const int kh = 2 * pair + (j >> 1), qh = 4 * pair + j;
  const _Float16 *wd = reinterpret_cast<const _Float16 *>(wo + (size_t)HID * NQ);

  // 1. every load up front, in the order of use (a wave's loads complete in
  // issue order): the raw q/k/v, the norm weights, the RoPE row, the cached
  // keys, the cached values, then the Wo rows and the residual
  const float xq0 = qkv[qh * HD + lane], xq1 = qkv[qh * HD + lane + 64];
  const float xk0 = qkv[NQ + kh * HD + lane], xk1 = qkv[NQ + kh * HD + lane + 64];
  const float xv0 = qkv[NQ + KVH * HD + kh * HD + lane];
  const float xv1 = qkv[NQ + KVH * HD + kh * HD + lane + 64];
  const float qn0 = qkn[lane], qn1 = qkn[lane + 64];
  const float kn0 = qkn[HD + lane], kn1 = qkn[HD + lane + 64];
  const float eps = qkn[2 * HD];
  const float2 cs = rope[lane];
  KV *kh_p = kl + (size_t)kh * P * HD;
  KV *vh_p = kl + v_off + (size_t)kh * P * HD;
  // cached keys and values of positions 0 .. pos - 1: lane holds dims
  // 8 (lane % 16) .. + 7 of positions lane / 16 + 4 i, so each load
  // instruction reads 4 whole rows; positions at or past pos are read at
  // pos - 1 (a context's cache starts as zeros: finite) and weighted 0
  const int last = max(pos - 1, 0);
  u32x4 kr[NJ][LW], vr[NJ][LW];
#pragma unroll
  for (int i = 0; i < NJ; i++) {
    const size_t off = (size_t)min(rg + 4 * i, last) * HD + 8 * r16;
#pragma unroll
    for (int e = 0; e < LW; e++) kr[i][e] = *reinterpret_cast<const u32x4 *>(kh_p + off + 4 * e);
  }
#pragma unroll
  for (int i = 0; i < NJ; i++) {
    const size_t off = (size_t)min(rg + 4 * i, last) * HD + 8 * r16;
#pragma unroll
    for (int e = 0; e < LW; e++) vr[i][e] = *reinterpret_cast<const u32x4 *>(vh_p + off + 4 * e);
  }
  __builtin_amdgcn_sched_barrier(0);
  // Wo rows rb + 2 i + lane / 32 (i = 0, 1), columns 16 (lane % 32) .. + 15 of the pair
  const int rb = (blockIdx.x / PAIRS) * PROWS + 4 * j;
  int4 wv[2];
  float sc[2], hr[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int row = rb + 2 * i + (lane >> 5);
    wv[i] = *reinterpret_cast<const int4 *>(wo + (size_t)row * NQ + pair * PCOLS +
                                            (lane & 31) * 16);
    sc[i] = (float)wd[(size_t)row * NBO + pair * (PCOLS / 32) + ((lane & 31) >> 1)];
    hr[i] = h[row];
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. QK-norm + RoPE; the new key and value rounded as the cache holds them
  {
    float x0 = xq0, x1 = xq1;
    norm_rope(x0, x1, qn0, qn1, cs, eps);
    qs[j][lane] = x0;
    qs[j][lane + 64] = x1;
  }
  {
    float x0 = xk0, x1 = xk1;
    norm_rope(x0, x1, kn0, kn1, cs, eps);
    const KV k0 = to_cache<KV>(x0), k1 = to_cache<KV>(x1), v0 = to_cache<KV>(xv0),
             v1 = to_cache<KV>(xv1);
    kvs[j][0][lane] = (float)k0;
    kvs[j][0][lane + 64] = (float)k1;
    kvs[j][1][lane] = (float)v0;
    kvs[j][1][lane + 64] = (float)v1;
    if (blockIdx.x < PAIRS && (j & 1) == 0) {
      kh_p[(size_t)pos * HD + lane] = k0;
      kh_p[(size_t)pos * HD + lane + 64] = k1;
      vh_p[(size_t)pos * HD + lane] = v0;
      vh_p[(size_t)pos * HD + lane + 64] = v1;
    }
  }
  wave_lds_sync();

  // 3. scores: an 8-term chain per lane summed over its 16-lane row
  const float scale = (float)(1.0 / sqrt((double)HD));
  float q[8], s[NJ], sn;
#pragma unroll
  for (int e = 0; e < 8; e++) q[e] = qs[j][8 * r16 + e];
#pragma unroll
  for (int i = 0; i < NJ; i++) {
    float k8[8];
    cvt8(kr[i], k8);
    float a = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) a = fmaf(q[e], k8[e], a);
    s[i] = a;
  }
  {
    float a = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) a = fmaf(q[e], kvs[j][0][8 * r16 + e], a);
    sn = a;
  }
#pragma unroll
  for (int i = 0; i < NJ; i++) s[i] += dpp_f<kQuadXor1>(s[i]);
  sn += dpp_f<kQuadXor1>(sn);
#pragma unroll
  for (int i = 0; i < NJ; i++) s[i] += dpp_f<kQuadXor2>(s[i]);
  sn += dpp_f<kQuadXor2>(sn);
#pragma unroll
  for (int i = 0; i < NJ; i++) s[i] += dpp_f<kHalfMirror>(s[i]);
  sn += dpp_f<kHalfMirror>(sn);
#pragma unroll
  for (int i = 0; i < NJ; i++) s[i] += dpp_f<kRowMirror>(s[i]);
  sn += dpp_f<kRowMirror>(sn);

  // 4. softmax over 0 .. pos; the outputs summed over the four rows and
  // scattered: after the two swap stages lane (rg, r16) holds dims
  // 8 r16 + rg and 8 r16 + 4 + rg
  sn *= scale;
  float mx = sn;
#pragma unroll
  for (int i = 0; i < NJ; i++) {
    s[i] = rg + 4 * i < pos ? s[i] * scale : -INFINITY;
    mx = fmaxf(mx, s[i]);
  }
  mx = rows4_max(mx);
  float ls = 0.f;
#pragma unroll
  for (int i = 0; i < NJ; i++) {
    s[i] = __expf(s[i] - mx);
    ls += s[i];
  }
  sn = __expf(sn - mx);
  const float den = rows4_sum(ls) + sn;
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; e++) o[e] = 0.f;
#pragma unroll
  for (int i = 0; i < NJ; i++) {
    float v8[8];
    cvt8(vr[i], v8);
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = fmaf(s[i], v8[e], o[e]);
  }
  float lo, hi;
  rows4_scatter8(o, lo, hi);
  {
    const float inv = 1.0f / den;
    const int d = 8 * r16 + rg;
    att[j * HD + d] = fmaf(sn, kvs[j][1][d], lo) * inv;
    att[j * HD + d + 4] = fmaf(sn, kvs[j][1][d + 4], hi) * inv;
  }
  __syncthreads();

  // 5. part[pair][row] = Wo[row][pair columns] . att (+ h[row] in pair 0)
  float acc[2];
  const float4 *xp = reinterpret_cast<const float4 *>(att + (lane & 31) * 16);
#pragma unroll
  for (int i = 0; i < 2; i++) {
    float p0 = dot4(wv[i].x, xp[0], 0.f);
    float p1 = dot4(wv[i].y, xp[1], 0.f);
    p0 = dot4(wv[i].z, xp[2], p0);
    p1 = dot4(wv[i].w, xp[3], p1);
    acc[i] = sc[i] * (p0 + p1);
  }
#pragma unroll
  for (int i = 0; i < 2; i++) acc[i] += dpp_f<kQuadXor1>(acc[i]);
#pragma unroll
  for (int i = 0; i < 2; i++) acc[i] += dpp_f<kQuadXor2>(acc[i]);
#pragma unroll
  for (int i = 0; i < 2; i++) acc[i] += dpp_f<kHalfMirror>(acc[i]);
#pragma unroll
  for (int i = 0; i < 2; i++) acc[i] += dpp_f<kRowMirror>(acc[i]);
  // rows 0 / 2: row i = 0 of lanes 0-31 / 32-63; rows 1 / 3: row i = 1
  const float tot = swap16_add(acc[0], acc[1]);
  if (r16 == 0) {
    const int i = rg & 1, row = rb + 2 * i + (rg >> 1);
    part[pair * HID + row] = pair == 0 ? hr[i] + tot : tot;
  }
}

// The first step of a code-predictor context: its two rows (positions 0 and
// 1: the talker's normed state and the embedding of code 0) in one launch,
// with no cached positions to read. Per workgroup, wave w = kv head w: QK-norm
// + RoPE of both rows' queries and keys, the K/V of both positions appended
// (workgroup 0), the causal attention (row 0 attends to itself: its output is
// v0; row 1 softmax over positions 0 and 1), then h[r][row] += Wo[row] .
// attention of row r for the wave's Wo row. qkv: the two q/k/v rows, ldq
// apart; rope: the (cos, sin) rows of positions 0 and 1.
template <typename KV>
__global__ __launch_bounds__(NT) void k_attn2_o_cp(const int8_t *__restrict__ wo,
                                                   const float *__restrict__ qkv, int ldq,
                                                   KV *__restrict__ kl, float *__restrict__ h,
                                                   const float *__restrict__ qkn,
                                                   const float2 *__restrict__ rope, int v_off) {
  __shared__ float att[2][NQ];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = blockIdx.x * ROWS + w;
  const _Float16 *wd = reinterpret_cast<const _Float16 *>(wo + (size_t)HID * NQ);
  // loads in the order of use (a wave's loads complete in issue order): the
  // two rows' q/k/v, the norm weights and RoPE rows, then the Wo row and the
  // residuals
  float xq[2][GRP][2], xk[2][2], xv[2][2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const float *x = qkv + (size_t)r * ldq;
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      xq[r][j][0] = x[(w * GRP + j) * HD + lane];
      xq[r][j][1] = x[(w * GRP + j) * HD + lane + 64];
    }
    xk[r][0] = x[NQ + w * HD + lane];
    xk[r][1] = x[NQ + w * HD + lane + 64];
    xv[r][0] = x[NQ + KVH * HD + w * HD + lane];
    xv[r][1] = x[NQ + KVH * HD + w * HD + lane + 64];
  }
  const float qn0 = qkn[lane], qn1 = qkn[lane + 64];
  const float kn0 = qkn[HD + lane], kn1 = qkn[HD + lane + 64];
  const float eps = qkn[2 * HD];
  const float2 cs0 = rope[lane], cs1 = rope[HD / 2 + lane];
  __builtin_amdgcn_sched_barrier(0);
  int4 wv[2];
  float sc[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    wv[c] = *reinterpret_cast<const int4 *>(wo + (size_t)row * NQ + c * 1024 + lane * 16);
    sc[c] = (float)wd[(size_t)row * NBO + c * 32 + (lane >> 1)];
  }
  const float hr0 = h[row], hr1 = h[HID + row];
  __builtin_amdgcn_sched_barrier(0);

  // keys and values as the cache holds them
  float k[2][2], v[2][2];
  KV *kh = kl + (size_t)w * P * HD;
  KV *vh = kl + v_off + (size_t)w * P * HD;
#pragma unroll
  for (int r = 0; r < 2; r++) {
    float x0 = xk[r][0], x1 = xk[r][1];
    norm_rope(x0, x1, kn0, kn1, r ? cs1 : cs0, eps);
    const KV k0 = to_cache<KV>(x0), k1 = to_cache<KV>(x1), v0 = to_cache<KV>(xv[r][0]),
             v1 = to_cache<KV>(xv[r][1]);
    k[r][0] = (float)k0;
    k[r][1] = (float)k1;
    v[r][0] = (float)v0;
    v[r][1] = (float)v1;
    if (blockIdx.x == 0) {
      kh[(size_t)r * HD + lane] = k0;
      kh[(size_t)r * HD + lane + 64] = k1;
      vh[(size_t)r * HD + lane] = v0;
      vh[(size_t)r * HD + lane + 64] = v1;
    }
  }
  const float scale = (float)(1.0 / sqrt((double)HD));
#pragma unroll
  for (int j = 0; j < GRP; j++) {
    const int o = (w * GRP + j) * HD;
    // row 0: softmax over its own position: the value itself
    att[0][o + lane] = v[0][0];
    att[0][o + lane + 64] = v[0][1];
    // row 1: positions 0 and 1
    float q0 = xq[1][j][0], q1 = xq[1][j][1];
    norm_rope(q0, q1, qn0, qn1, cs1, eps);
    const float s0 = wave_sum_dpp(fmaf(q0, k[0][0], q1 * k[0][1])) * scale;
    const float s1 = wave_sum_dpp(fmaf(q0, k[1][0], q1 * k[1][1])) * scale;
    const float mx = fmaxf(s0, s1);
    const float e0 = __expf(s0 - mx), e1 = __expf(s1 - mx);
    const float inv = 1.0f / (e0 + e1);
    att[1][o + lane] = fmaf(e0, v[0][0], e1 * v[1][0]) * inv;
    att[1][o + lane + 64] = fmaf(e0, v[0][1], e1 * v[1][1]) * inv;
  }
  __syncthreads();

  // h[r][row] += Wo[row] . att[r]
#pragma unroll
  for (int r = 0; r < 2; r++) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const float4 *xp = reinterpret_cast<const float4 *>(att[r] + c * 1024 + lane * 16);
      float p0 = dot4(wv[c].x, xp[0], 0.f);
      float p1 = dot4(wv[c].y, xp[1], 0.f);
      p0 = dot4(wv[c].z, xp[2], p0);
      p1 = dot4(wv[c].w, xp[3], p1);
      acc = fmaf(sc[c], p0 + p1, acc);
    }
    acc = wave_sum_dpp(acc);
    if (lane == 0) h[(size_t)r * HID + row] = (r ? hr1 : hr0) + acc;
  }
}

}  // namespace

bool cp_fused_supported(const q3h_stack_config &c) {
  return c.dtype == Q3H_Q8_0 && !c.act_q8 && c.hidden == HID && c.heads == KVH * GRP && c.kv_heads == KVH &&
         c.head_dim == HD && gemv_q8_parts_supported(2 * c.intermediate, c.hidden);
}

void launch_attn_o_cp(const Mat &wo, const float *qkv, void *k_layer, int v_off, const float *h,
                      float *part, const float *qkn, const float *rope_row, int pos, bool kv16,
                      hipStream_t st) {
  const dim3 grid(PAIRS * (HID / PROWS)), block(PNT);
  const float2 *rope = reinterpret_cast<const float2 *>(rope_row);
  // the cached positions 0 .. pos - 1 in 4 NJ lane slots (pos is fixed per
  // code-predictor step, so each step's launch reads only what it attends to)
  const int nj = std::min(std::max((pos + 3) / 4, 1), P / 4);
#define Q3H_AOC(KV, NJ)                                                                     \
  hipLaunchKernelGGL((k_attn_pair_cp<KV, NJ>), grid, block, 0, st, wo.q, qkv,               \
                     static_cast<KV *>(k_layer), qkn, rope, pos, v_off, h, part)
#define Q3H_AOC_NJ(KV) \
  switch (nj) {        \
    case 1: Q3H_AOC(KV, 1); break; \
    case 2: Q3H_AOC(KV, 2); break; \
    case 3: Q3H_AOC(KV, 3); break; \
    default: Q3H_AOC(KV, 4); break; \
  }
  if (kv16) {
    Q3H_AOC_NJ(_Float16)
  } else {
    Q3H_AOC_NJ(float)
  }
#undef Q3H_AOC_NJ
#undef Q3H_AOC
}

void launch_attn2_o_cp(const Mat &wo, const float *qkv, int ldq, void *k_layer, int v_off,
                       float *h, const float *qkn, const float *rope_rows, bool kv16,
                       hipStream_t st) {
  const dim3 grid(HID / ROWS), block(NT);
  const float2 *rope = reinterpret_cast<const float2 *>(rope_rows);
  if (kv16)
    hipLaunchKernelGGL(k_attn2_o_cp<_Float16>, grid, block, 0, st, wo.q, qkv, ldq,
                       static_cast<_Float16 *>(k_layer), h, qkn, rope, v_off);
  else
    hipLaunchKernelGGL(k_attn2_o_cp<float>, grid, block, 0, st, wo.q, qkv, ldq,
                       static_cast<float *>(k_layer), h, qkn, rope, v_off);
}

}  // namespace q3h
