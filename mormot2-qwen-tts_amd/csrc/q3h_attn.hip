// q3h_attn.hip - GQA decode attention of the Qwen3 stacks on gfx950.
//
// One workgroup of 512 threads per (query head h, row m, split s); a split is
// up to 256 consecutive positions (one split for the contexts of the frame
// step). Query head h reads the keys and values of kv head h / GRP. The
// kernel is short and latency-bound, so it is laid out to issue every load of
// the split at once and to keep the per-CU instruction count low:
//   - keys: 2 lanes per position (64 dims each), each lane loads its half
//     row; the score is a 64-term dot + one DPP add;
//   - values: lane (dg, kg) = (t % 32, t / 32) holds dims 4dg..4dg+3 of
//     positions p0 + kg + 16 i; its 16 float4 loads are issued with the keys;
//   - softmax in two passes over the block (max, then sum), no rescaling;
//   - outputs: 16 partial sums per dim merged in LDS.
// Fused prologue (FUSED: each row is the one new position of its own context):
// the q head and the key get their RMSNorm (q_norm / k_norm) and RoPE here,
// the new key and value are rounded as the cache stores them, the workgroup
// of the group's first query head appends them to the cache, and position
// pos is read from LDS (other positions from the cache, written by earlier
// launches). Rows that add several positions of one context at once
// (prefill) run the separate append kernel first and this kernel unfused.
// Splits (contexts beyond 256 positions): each workgroup leaves (max, sum,
// unnormalized output) in the partial buffer and takes a ticket; the last
// workgroup of (m, h) merges the splits in split order and clears the ticket.
#include <hip/hip_runtime.h>

#include "q3h_internal.h"
#include "q3h_math.h"
#include "q3h_wave.h"

namespace q3h {

namespace {

constexpr int HD = 128;  // head_dim (checked at stack creation)
constexpr int NT = 512;
constexpr int NW = NT / 64;
constexpr int kSplit = 256;  // positions per split
constexpr int KG = NT / 32;  // value key groups
constexpr int VK = kSplit / KG;  // value positions per lane

__device__ __forceinline__ void ld64(const float *p, float *o) {
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const float4 t = reinterpret_cast<const float4 *>(p)[i];
    o[4 * i] = t.x;
    o[4 * i + 1] = t.y;
    o[4 * i + 2] = t.z;
    o[4 * i + 3] = t.w;
  }
}

__device__ __forceinline__ void ld64(const _Float16 *p, float *o) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const h8 t = reinterpret_cast<const h8 *>(p)[i];
#pragma unroll
    for (int j = 0; j < 8; j++) o[8 * i + j] = (float)t[j];
  }
}

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

__device__ __forceinline__ float4 ld4(const _Float16 *p) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 t = *reinterpret_cast<const h4 *>(p);
  return make_float4((float)t[0], (float)t[1], (float)t[2], (float)t[3]);
}

// RMSNorm over a head held as (x0, x1) = elements (lane, lane + 64), weight
// (w0, w1), then rotate_half RoPE with (cos, sin) = cs
__device__ __forceinline__ void norm_rope(float &x0, float &x1, float w0, float w1, float2 cs,
                                          float eps) {
  const float ss = wave_sum_dpp(fmaf(x0, x0, x1 * x1));
  const float inv = 1.0f / sqrtf(ss * (1.0f / HD) + eps);
  const float a = w0 * (x0 * inv), b = w1 * (x1 * inv);
  x0 = a;
  x1 = b;
  rope_pair(x0, x1, cs.x, cs.y);
}

__device__ __forceinline__ float rescale(float m, float mn) {
  return m == -INFINITY ? 0.f : expf(m - mn);
}

// Plain scalar arguments, those of the prologue first (the first 14 argument
// dwords are preloaded into SGPRs); the split buffers come last. qkn holds
// [q_norm | k_norm | eps] of the layer.
template <typename KV, bool FUSED, int GRP>
__global__ __launch_bounds__(NT) void k_attn(const RowDesc *__restrict__ rd,
                                             const float *__restrict__ qkv,
                                             const float2 *__restrict__ rope_cs,
                                             const float *__restrict__ qkn,
                                             float *__restrict__ outp, int layer, int kvh, int S,
                                             float *__restrict__ part, int *__restrict__ tickets) {
  __shared__ float qs[HD];
  __shared__ float kvn[2][HD];  // the new key and value, as the cache holds them
  __shared__ float red[NW];
  __shared__ float pr[kSplit];
  __shared__ float po[KG][HD];
  __shared__ int last;
  const int heads = GRP * kvh, ldq = (heads + 2 * kvh) * HD;
  const int h = blockIdx.x, m = blockIdx.y, s = blockIdx.z, g = h / GRP;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float *row = qkv + (size_t)m * ldq;

  // raw q of head h (wave 0), key (wave 1), value (wave 2) of kv head g
  float x0 = 0.f, x1 = 0.f;
  if (FUSED && wave < 3) {
    const size_t off = wave == 0 ? (size_t)h * HD : (size_t)(heads + (wave - 1) * kvh + g) * HD;
    x0 = row[off + lane];
    x1 = row[off + lane + 64];
  }
  const RowDesc d = rd[m];
  float *out = outp + ((size_t)m * heads + h) * HD;
  if (d.pos < 0) {  // inactive row: zeros, no ticket
    if (s == 0 && t < HD) out[t] = 0.f;
    return;
  }
  const int n = d.pos + 1;
  const int p0 = s * kSplit, p1 = min(n, p0 + kSplit);
  const size_t head_off = ((size_t)layer * kvh + g) * d.max_pos * HD;
  KV *kc = reinterpret_cast<KV *>(d.k) + head_off;
  KV *vc = reinterpret_cast<KV *>(d.v) + head_off;

  // every key and value of the split, loaded before the prologue
  const int kp = p0 + (t >> 1), kh = (t & 1) * 64;
  const bool kown = kp < p1 && !(FUSED && kp == d.pos);
  float kk[64];
  if (kown) ld64(kc + (size_t)kp * HD + kh, kk);
  const int dg = t & 31, kg = t >> 5;
  float4 vv[VK];
#pragma unroll
  for (int i = 0; i < VK; i++) {
    const int p = p0 + kg + KG * i;
    if (p < p1 && !(FUSED && p == d.pos)) vv[i] = ld4(vc + (size_t)p * HD + 4 * dg);
  }
  float2 cs = make_float2(1.f, 0.f);
  float w0 = 1.f, w1 = 1.f, eps = 0.f;
  if (FUSED && wave < 2) {
    cs = rope_cs[(size_t)d.pos * (HD / 2) + lane];
    const float *w = qkn + wave * HD;
    w0 = w[lane];
    w1 = w[lane + 64];
    eps = qkn[2 * HD];
  }
  __builtin_amdgcn_sched_barrier(0);

  if (FUSED) {
    if (wave == 0) {
      norm_rope(x0, x1, w0, w1, cs, eps);
      qs[lane] = x0;
      qs[lane + 64] = x1;
    } else if (wave < 3) {
      if (wave == 1) norm_rope(x0, x1, w0, w1, cs, eps);
      const KV y0 = (KV)x0, y1 = (KV)x1;
      kvn[wave - 1][lane] = (float)y0;
      kvn[wave - 1][lane + 64] = (float)y1;
      // the group's first query head appends, in the split holding pos
      if (h % GRP == 0 && d.pos >= p0 && d.pos < p0 + kSplit) {
        KV *dst = (wave == 1 ? kc : vc) + (size_t)d.pos * HD;
        dst[lane] = y0;
        dst[lane + 64] = y1;
      }
    }
  } else if (t < HD) {
    qs[t] = row[(size_t)h * HD + t];
  }
  __syncthreads();

  // scores: 2 lanes per key
  const float scale = (float)(1.0 / sqrt((double)HD));
  const bool klive = kp < p1;
  if (FUSED && kp == d.pos) {
#pragma unroll
    for (int i = 0; i < 64; i++) kk[i] = kvn[0][kh + i];
  }
  float a0 = 0.f, a1 = 0.f;
  if (klive) {
#pragma unroll
    for (int i = 0; i < 64; i += 2) {
      a0 = fmaf(qs[kh + i], kk[i], a0);
      a1 = fmaf(qs[kh + i + 1], kk[i + 1], a1);
    }
  }
  float sc = a0 + a1;
  sc += dpp_f<kQuadXor1>(sc);
  sc = klive ? sc * scale : -INFINITY;
  // block max
  float mx = wave_max_dpp(sc);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int i = 1; i < NW; i++) mx = fmaxf(mx, red[i]);
  const float e = klive ? expf(sc - mx) : 0.f;
  if ((t & 1) == 0 && kp - p0 < kSplit) pr[kp - p0] = e;
  float sum = wave_sum_dpp((t & 1) == 0 ? e : 0.f);
  __syncthreads();
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  sum = 0.f;
#pragma unroll
  for (int i = 0; i < NW; i++) sum += red[i];

  // values: dims 4dg..4dg+3 over this lane's positions
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < VK; i++) {
    const int p = p0 + kg + KG * i;
    if (p < p1) {
      const float pw = pr[p - p0];
      float4 v;
      if (FUSED && p == d.pos)
        v = make_float4(kvn[1][4 * dg], kvn[1][4 * dg + 1], kvn[1][4 * dg + 2], kvn[1][4 * dg + 3]);
      else
        v = vv[i];
      o.x = fmaf(pw, v.x, o.x);
      o.y = fmaf(pw, v.y, o.y);
      o.z = fmaf(pw, v.z, o.z);
      o.w = fmaf(pw, v.w, o.w);
    }
  }
  po[kg][4 * dg] = o.x;
  po[kg][4 * dg + 1] = o.y;
  po[kg][4 * dg + 2] = o.z;
  po[kg][4 * dg + 3] = o.w;
  __syncthreads();
  if (t < HD) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < KG; i++) acc += po[i][t];
    if (S == 1) {
      out[t] = sum > 0.f ? acc / sum : 0.f;
    } else {
      float *pp = part + (((size_t)m * heads + h) * S + s) * (HD + 2);
      pp[t] = acc;
      if (t == 0) {
        pp[HD] = sum > 0.f ? mx : -INFINITY;
        pp[HD + 1] = sum;
      }
    }
  }
  if (S == 1) return;

  // splits: the last workgroup of (m, h) merges them
  __threadfence();
  __syncthreads();
  if (t == 0) {
    int *ticket = tickets + (size_t)m * heads + h;
    const int old = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    last = old == S - 1;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (t < HD) {
    const float *pp = part + ((size_t)m * heads + h) * S * (HD + 2);
    float mn = -INFINITY;
    for (int i = 0; i < S; i++) mn = fmaxf(mn, pp[i * (HD + 2) + HD]);
    float l = 0.f, acc = 0.f;
    for (int i = 0; i < S; i++) {
      const float c = rescale(pp[i * (HD + 2) + HD], mn);
      l += pp[i * (HD + 2) + HD + 1] * c;
      acc += pp[i * (HD + 2) + t] * c;
    }
    out[t] = l > 0.f ? acc / l : 0.f;
  }
  if (t == 0) tickets[(size_t)m * heads + h] = 0;
}

template <typename KV, bool FUSED>
void launch_grp(const AttnArgs &a, int grp, dim3 grid, hipStream_t st) {
#define Q3H_A(G)                                                                               \
  hipLaunchKernelGGL((k_attn<KV, FUSED, G>), grid, dim3(NT), 0, st, a.rd, a.qkv, a.rope_cs,     \
                     a.qkn, a.out, a.layer, a.kvh, (int)grid.z, a.part, a.tickets)
  if (grp == 1)
    Q3H_A(1);
  else if (grp == 2)
    Q3H_A(2);
  else
    Q3H_A(4);
#undef Q3H_A
}

}  // namespace

int attn_splits(int positions) {
  const int n = (positions + kSplit - 1) / kSplit;
  return n < 1 ? 1 : n;
}

void launch_attn(const AttnArgs &a, int M, int splits, bool fused, bool kv16, hipStream_t st) {
  const int grp = a.heads / a.kvh;
  const dim3 grid(a.heads, M, splits);
  if (kv16) {
    if (fused)
      launch_grp<_Float16, true>(a, grp, grid, st);
    else
      launch_grp<_Float16, false>(a, grp, grid, st);
  } else {
    if (fused)
      launch_grp<float, true>(a, grp, grid, st);
    else
      launch_grp<float, false>(a, grp, grid, st);
  }
}

}  // namespace q3h
