// q3h_attn.hip - GQA decode attention of the Qwen3 stacks on gfx950 (the
// f32-activation path; the int8 path has its own in q3h_attnx.hip).
//
//  - up to 256 positions (the frame step): k_attn_short, one workgroup per
//    query head and row, one launch;
//  - longer contexts: k_attn_split, one workgroup per (kv head, split) for
//    both query heads of the group, then k_attn_merge.
// Both read the cache with the same thread mapping: 16 lanes per cache row, 8
// dims per lane, so every load instruction of a wave covers 4 whole rows
// (a layout with 2 lanes per row, each walking its own half row, touched 64
// separate segments per instruction and took 1.5-3 us to issue the loads of
// a 256-position workgroup). Fused rows (each the one new position of its
// own context) get the QK-norm (q_norm / k_norm), RoPE and the K/V append in
// the prologue; rows that add several positions of one context at once
// (prefill) run the separate append kernel first and these kernels unfused.
#include <algorithm>
#include <type_traits>

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "q3h_internal.h"
#include "q3h_math.h"
#include "q3h_wave.h"

namespace q3h {

namespace {

constexpr int HD = 128;  // head_dim (checked at stack creation)
constexpr int kSplit = 256;  // positions of the single-launch kernel

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
  return m == -INFINITY ? 0.f : __expf(m - mn);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// a 16-byte load from device memory through a global-address-space pointer
// (global_load, not flat_load: the cache pointers come from row descriptors
// in memory, which the compiler cannot place in an address space itself)
__device__ __forceinline__ u32x4 gload16(const void *p) {
  return *reinterpret_cast<const __attribute__((address_space(1))) u32x4 *>(
      reinterpret_cast<uintptr_t>(p));
}

// 8 cache elements (one 16-byte load of f16, two of f32) as f32
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

// Contexts of up to 256 positions (the frame step's talker and code
// predictor at batch sizes that take the f32 path): one workgroup of NTS
// threads per (query head h, row m), kv head h / GRP, covering NJ NTS / 16
// positions (the launch sizes NJ to the positions it must cover, in steps of
// 64: the load instructions, issued for every covered position, are most of
// the kernel's time at these lengths). The thread mapping of
// the split kernel below: thread t owns dims 8 (t % 16) .. + 7 of positions
// t / 16 + (NTS / 16) j, so each load instruction of a wave reads 4 whole
// consecutive cache rows (coalesced), scores are 8-term chains summed over a
// 16-lane DPP row, and a position's key and value sit in the same lanes.
//   - loads first: the prologue's (q head, key, value of the row), then the
//     keys and values of positions [0, n) clamped into range (a context's
//     cache starts as zeros, so a row read past the context is finite, and
//     its weight is 0);
//   - FUSED (each row the one new position pos of its own context): waves 0,
//     1, 2 norm and rotate the q head and the key, round key and value as the
//     cache stores them; the group's first query head appends them; the new
//     position joins the softmax as one more score (its 128-dim dot from the
//     prologue's vectors) instead of through the cache, so the cache rows
//     read here are the positions before pos;
//   - softmax in two passes over the workgroup (maximum, then sum).
// Workgroups of k_attn_short past its query heads load, one launch ahead, the
// cache rows that the next layer's attention reads (positions [0, pos) of
// layer pf_layer, keys and values of kv head g = i % kvh, i the workgroup's
// index among them), on the XCD of that attention's workgroups (the
// dispatcher deals workgroup x to XCD x % 8; workgroup x of kv head g has
// x % kvh == g). The L2 does not keep them until then: in the batch-1 frame
// each launch fetches its own rows past L2 again (FETCH_SIZE per launch = its
// own rows + the next layer's), but those fetches complete sooner (3.95 against
// 5.44 us per layer at 126 positions), as from the memory-side Infinity Cache
// rather than HBM. kPrefetchParts workgroups share a kv head; each thread
// issues all of its 16-byte loads before using any, then folds them into one
// value that an empty asm statement consumes (no store).
constexpr int kPrefetchParts = 4;
template <typename KV, int NTS>
__device__ __forceinline__ void prefetch_next_layer(const RowDesc *__restrict__ rd, int pf_layer,
                                                    int kvh, int i) {
  const RowDesc d = rd[blockIdx.y];
  if (d.pos <= 0) return;
  const int g = i % kvh, part = i / kvh;
  const size_t head_off = ((size_t)pf_layer * kvh + g) * d.max_pos * HD * sizeof(KV);
  const char *kc = reinterpret_cast<const char *>(global_ptr(d.k)) + head_off;
  const char *vc = reinterpret_cast<const char *>(global_ptr(d.v)) + head_off;
  // 16-byte units of one tensor's rows [0, pos): at most 256 rows
  const int units = d.pos * (HD * (int)sizeof(KV) / 16);
  constexpr int PER = 2 * kSplit * (HD * (int)sizeof(KV) / 16) / (kPrefetchParts * NTS);
  u32x4 r[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int u = min(part * NTS + (int)threadIdx.x + j * kPrefetchParts * NTS, 2 * units - 1);
    r[j] = gload16(u < units ? kc + (size_t)u * 16 : vc + (size_t)(u - units) * 16);
  }
  unsigned f = 0;
#pragma unroll
  for (int j = 0; j < PER; j++) f ^= r[j].x ^ r[j].y ^ r[j].z ^ r[j].w;
  asm volatile("" ::"v"(f));
}

template <typename KV, bool FUSED, int GRP, int NTS, int NJ>
__global__ __launch_bounds__(NTS) void k_attn_short(const RowDesc *__restrict__ rd,
                                                    const float *__restrict__ qkv,
                                                    const float2 *__restrict__ rope_cs,
                                                    const float *__restrict__ qkn,
                                                    float *__restrict__ outp, int layer, int kvh,
                                                    int pf_layer) {
  constexpr int PG = NTS / 16;         // position groups (NJ positions per thread)
  static_assert(NJ * PG <= kSplit, "at most 256 positions");
  constexpr int LW = sizeof(KV) / 2;   // 16-byte loads per 8 elements
  constexpr int NWV = NTS / 64;
  static_assert(NWV >= 3, "prologue waves");
  if ((int)blockIdx.x >= GRP * kvh) {  // the next layer's cache rows (pf_layer >= 0)
    prefetch_next_layer<KV, NTS>(rd, pf_layer, kvh, blockIdx.x - GRP * kvh);
    return;
  }
  __shared__ float qs[HD], kvn[2][HD];
  __shared__ float red[2][NWV];
  __shared__ float po[NWV][HD];
  const int heads = GRP * kvh, ldq = (heads + 2 * kvh) * HD;
  // workgroup x takes query head GRP (x % kvh) + x / kvh: the GRP heads of kv
  // head g are workgroups g, g + kvh, ..., which the dispatcher deals to one
  // XCD when kvh is a multiple of 8, so the group's second read of the cache
  // is served by that XCD's L2
  const int g = blockIdx.x % kvh, h = g * GRP + blockIdx.x / kvh, m = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r16 = t & 15, pg = t >> 4;
  const float *row = qkv + (size_t)m * ldq;
  float *out = outp + ((size_t)m * heads + h) * HD;

  // raw q of head h (wave 0), key (wave 1), value (wave 2) of kv head g
  float x0 = 0.f, x1 = 0.f, w0 = 1.f, w1 = 1.f, eps = 0.f;
  if (FUSED && wave < 3) {
    const size_t off = wave == 0 ? (size_t)h * HD : (size_t)(heads + (wave - 1) * kvh + g) * HD;
    x0 = row[off + lane];
    x1 = row[off + lane + 64];
    const float *w = qkn + min(wave, 1) * HD;
    w0 = w[lane];
    w1 = w[lane + 64];
    eps = qkn[2 * HD];
  }
  const RowDesc d = rd[m];
  if (d.pos < 0) {  // inactive row: zeros
    if (t < HD) out[t] = 0.f;
    return;
  }
  const int pos = d.pos;
  const int n = FUSED ? pos : pos + 1;  // positions read from the cache
  const int last = max(n - 1, 0);
  const size_t head_off = ((size_t)layer * kvh + g) * d.max_pos * HD;
  KV *kc = global_ptr(reinterpret_cast<KV *>(d.k)) + head_off;
  KV *vc = global_ptr(reinterpret_cast<KV *>(d.v)) + head_off;
  const float2 cs =
      FUSED && wave < 2 ? rope_cs[(size_t)pos * (HD / 2) + lane] : make_float2(1.f, 0.f);
  u32x4 kr[NJ][LW], vr[NJ][LW];
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const KV *p = kc + (size_t)min(pg + PG * j, last) * HD + 8 * r16;
#pragma unroll
    for (int e = 0; e < LW; e++) kr[j][e] = gload16(p + e * 4);
  }
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const KV *p = vc + (size_t)min(pg + PG * j, last) * HD + 8 * r16;
#pragma unroll
    for (int e = 0; e < LW; e++) vr[j][e] = gload16(p + e * 4);
  }
  __builtin_amdgcn_sched_barrier(0);

  if (FUSED) {
    if (wave == 0) {
      norm_rope(x0, x1, w0, w1, cs, eps);
      qs[lane] = x0;
      qs[lane + 64] = x1;
    } else if (wave < 3) {
      if (wave == 1) norm_rope(x0, x1, w0, w1, cs, eps);
      const KV y0 = to_cache<KV>(x0), y1 = to_cache<KV>(x1);
      kvn[wave - 1][lane] = (float)y0;
      kvn[wave - 1][lane + 64] = (float)y1;
      if (h % GRP == 0) {  // the group's first query head appends
        KV *dst = (wave == 1 ? kc : vc) + (size_t)pos * HD;
        dst[lane] = y0;
        dst[lane + 64] = y1;
      }
    }
  } else if (t < HD) {
    qs[t] = row[(size_t)h * HD + t];
  }
  __syncthreads();

  const float scale = (float)(1.0 / sqrt((double)HD));
  float q[8];
#pragma unroll
  for (int e = 0; e < 8; e++) q[e] = qs[8 * r16 + e];
  float sc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    float k8[8];
    cvt8(kr[j], k8);
    float a = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) a = fmaf(q[e], k8[e], a);
    sc[j] = a;
  }
  float sn = -INFINITY;  // the new position's score (FUSED)
  if (FUSED) {
    float a = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) a = fmaf(q[e], kvn[0][8 * r16 + e], a);
    sn = group16_sum_dpp(a) * scale;
  }
#pragma unroll
  for (int j = 0; j < NJ; j++) sc[j] += dpp_f<kQuadXor1>(sc[j]);
#pragma unroll
  for (int j = 0; j < NJ; j++) sc[j] += dpp_f<kQuadXor2>(sc[j]);
#pragma unroll
  for (int j = 0; j < NJ; j++) sc[j] += dpp_f<kHalfMirror>(sc[j]);
#pragma unroll
  for (int j = 0; j < NJ; j++) sc[j] += dpp_f<kRowMirror>(sc[j]);
  float mx = sn;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    sc[j] = pg + PG * j < n ? sc[j] * scale : -INFINITY;
    mx = fmaxf(mx, sc[j]);
  }
  // the scores are alike across a 16-lane row (one position group): the
  // wave's maximum and sum are those over its four rows
  mx = rows4_max(mx);
  if (lane == 0) red[0][wave] = mx;
  __syncthreads();
  mx = red[0][0];
#pragma unroll
  for (int w = 1; w < NWV; w++) mx = fmaxf(mx, red[0][w]);
  float ls = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    sc[j] = __expf(sc[j] - mx);
    ls += sc[j];
  }
  ls = rows4_sum(ls);
  if (lane == 0) red[1][wave] = ls;
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; e++) o[e] = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    float v8[8];
    cvt8(vr[j], v8);
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = fmaf(sc[j], v8[e], o[e]);
  }
  // summed over the wave's four position groups, scattered over its lanes
  {
    float lo, hi;
    rows4_scatter8(o, lo, hi);
    po[wave][8 * r16 + (lane >> 4)] = lo;
    po[wave][8 * r16 + 4 + (lane >> 4)] = hi;
  }
  __syncthreads();
  if (t < HD) {
    float sum = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; w++) {
      sum += red[1][w];
      acc += po[w][t];
    }
    if (FUSED) {
      const float c = __expf(sn - mx);
      sum += c;
      acc = fmaf(c, kvn[1][t], acc);
    }
    out[t] = sum > 0.f ? acc / sum : 0.f;
  }
}

// The split kernel's workgroups past its S splits load, one launch ahead, the
// cache rows [0, pos) of layer pf_layer (keys and values of kv head
// blockIdx.x, row blockIdx.z) that the next layer's split workgroups read,
// n workgroups per (kv head, row), workgroup i taking every n-th 4 KB; 8
// loads in flight per thread, folded into one value that an empty asm
// statement consumes (no store). As with k_attn_short's, the next launch
// fetches the rows past its L2 again, sooner than from HBM.
template <typename KV, int NT>
__device__ __forceinline__ void prefetch_split(const RowDesc *__restrict__ rd, int pf_layer,
                                               int kvh, int i, int n) {
  const RowDesc d = rd[blockIdx.z];
  if (pf_layer < 0 || d.pos <= 0) return;
  const size_t head_off = ((size_t)pf_layer * kvh + blockIdx.x) * d.max_pos * HD * sizeof(KV);
  const char *kc = reinterpret_cast<const char *>(global_ptr(d.k)) + head_off;
  const char *vc = reinterpret_cast<const char *>(global_ptr(d.v)) + head_off;
  const int units = d.pos * (HD * (int)sizeof(KV) / 16);  // 16-byte units of one tensor
  const int stride = n * NT;
  for (int u0 = i * NT + (int)threadIdx.x; u0 < 2 * units; u0 += 8 * stride) {
    u32x4 r[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int u = min(u0 + k * stride, 2 * units - 1);
      r[k] = gload16(u < units ? kc + (size_t)u * 16 : vc + (size_t)(u - units) * 16);
    }
    unsigned f = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) f ^= r[k].x ^ r[k].y ^ r[k].z ^ r[k].w;
    asm volatile("" ::"v"(f));
  }
}

constexpr int kMaxSplitsLong = 256;
constexpr size_t kPrefetchSplitBytes = (size_t)12 << 20;

// Long contexts (more than 256 positions): k_attn_split, one workgroup of NT
// threads per (kv head g, split s, row m) for all GRP query heads of g, so
// that every key and value of the cache is read once per step, then
// k_attn_merge. A split is P positions, and P grows with the context so that
// a step launches a few hundred workgroups and the merge stays short.
// The context is cut into blocks of NT / 16 consecutive positions dealt out
// to the S splits in turn (block b to split b % S): at any moment the
// workgroups of a kv head read one contiguous stretch of the cache. Thread t
// owns dims 8 (t % 16) .. + 7 of position t / 16 of each of its blocks: one
// load instruction of a wave reads 4 whole consecutive rows, and a
// position's key and value sit in the same lanes, so its softmax weights
// never leave the registers.
// The waves of a workgroup meet once, at the end. Its loads are all in
// flight together and arrive over the whole time the cache streams, so a
// wave computes its scores and values as its own data arrives; the
// workgroup-wide maximum before the exponentials (two more block barriers)
// left that arithmetic waiting for the slowest wave, after the stream.
//   - the split covers the positions before pos (FUSED: the new position
//     pos is added by the merge) or up to pos (rows whose K/V were appended
//     beforehand); every key and value is loaded before the prologue, at
//     positions clamped into the covered range (a context's cache starts as
//     zeros, so a row read there is finite, and its weight is 0);
//   - prologue (FUSED): every wave norms and rotates the GRP query heads
//     itself (RMSNorm with q_norm, RoPE) and takes its 8 dims of each through
//     its own rows of LDS; in split 0, wave h leaves query head h in the
//     partial buffer for the merge, and the last two waves append the row's
//     key (k_norm, RoPE) and value to the cache;
//   - scores: an 8-term chain per lane, summed over the 16 lanes of a DPP
//     row, one DPP stage at a time over all of the thread's sums;
//   - softmax per query head over the wave's positions, online over the two
//     halves of the thread's positions (the loads are issued a half at a time,
//     so the first half's scores, softmax and values run while the second
//     half streams in): the running maximum, the sum and the output rescaled
//     when the maximum grows;
//   - values: 8 dims x GRP heads of partial outputs per lane, summed over the
//     position groups of a wave (lane shuffles);
//   - the waves' (maximum, sum, output) meet in LDS, rescaled to the split's
//     maximum, and go to the partial buffer [M][heads][S + 1][HD + 2] (slot
//     S: the query head).
// The kernel boundary makes the partials of every workgroup visible to the
// merge (a device-scope fence and ticket per workgroup, the alternative, was
// measured here at 10-30 us per launch on long contexts).
template <typename KV, bool FUSED, int GRP, int P, int NTL>
__global__ __launch_bounds__(NTL) void k_attn_split(const RowDesc *__restrict__ rd,
                                                    const float *__restrict__ qkv,
                                                    const float2 *__restrict__ rope_cs,
                                                    const float *__restrict__ qkn, int layer,
                                                    int kvh, int S, float *__restrict__ part,
                                                    int pf_layer) {
  constexpr int PG = NTL / 16;        // position groups
  constexpr int NJ = P / PG;          // positions per thread
  constexpr int LW = sizeof(KV) / 2;  // 16-byte loads per 8 elements
  constexpr int NWV = NTL / 64;
  static_assert(NJ * PG == P, "split size");
  static_assert(NWV >= 2 && GRP <= NWV, "a wave per query head, two for the append");
  __shared__ float qw[FUSED ? NWV : 1][GRP][HD];  // each wave's normed query heads
  __shared__ float wmx[NWV][GRP], wsum[NWV][GRP];  // each wave's maximum and sum
  __shared__ float po[NWV][GRP][HD];               // each wave's output
  if ((int)blockIdx.y >= S) {  // the next layer's cache rows, one launch ahead (above)
    prefetch_split<KV, NTL>(rd, pf_layer, kvh, blockIdx.y - S, gridDim.y - S);
    return;
  }
  const int g = blockIdx.x, s = blockIdx.y, m = blockIdx.z;
  const int heads = GRP * kvh, ldq = (heads + 2 * kvh) * HD;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r16 = t & 15, pg = t >> 4;
  const float *row = qkv + (size_t)m * ldq;
  // loads in the order of their use: the prologue's (the q / k / v row needs
  // no descriptor), the keys, the values
  float q[GRP][8];          // the thread's 8 dims of each query head
  float x0[GRP], x1[GRP];   // FUSED: query head h as (dim lane, dim lane + 64)
  float a0 = 0.f, a1 = 0.f;  // FUSED, split 0: the row's key or value
  float wq0 = 1.f, wq1 = 1.f, wk0 = 1.f, wk1 = 1.f, eps = 0.f;
  const bool app = FUSED && s == 0 && wave >= NWV - 2;  // appends the key (NWV - 2) / value
  if (FUSED) {
#pragma unroll
    for (int h = 0; h < GRP; h++) {
      x0[h] = row[(g * GRP + h) * HD + lane];
      x1[h] = row[(g * GRP + h) * HD + lane + 64];
    }
    if (app) {
      const int col = (heads + (wave - (NWV - 2)) * kvh + g) * HD;
      a0 = row[col + lane];
      a1 = row[col + lane + 64];
    }
    wq0 = qkn[lane];
    wq1 = qkn[lane + 64];
    wk0 = qkn[HD + lane];
    wk1 = qkn[HD + lane + 64];
    eps = qkn[2 * HD];
  } else {
#pragma unroll
    for (int h = 0; h < GRP; h++) {
      const float4 *p = reinterpret_cast<const float4 *>(row + (g * GRP + h) * HD + 8 * r16);
      const float4 u = p[0], v = p[1];
      q[h][0] = u.x, q[h][1] = u.y, q[h][2] = u.z, q[h][3] = u.w;
      q[h][4] = v.x, q[h][5] = v.y, q[h][6] = v.z, q[h][7] = v.w;
    }
  }
  const RowDesc d = rd[m];
  if (d.pos < 0) return;  // inactive row (the merge writes its zeros)
  const int pos = d.pos;
  const int n = FUSED ? pos : pos + 1;  // positions covered here
  const int last = max(n - 1, 0);
  const size_t head_off = ((size_t)layer * kvh + g) * d.max_pos * HD;
  KV *kc = global_ptr(reinterpret_cast<KV *>(d.k)) + head_off;
  KV *vc = global_ptr(reinterpret_cast<KV *>(d.v)) + head_off;
  // block j of this split: positions (j S + s) PG .. + PG - 1
  auto position = [&](int j) { return (j * S + s) * PG + pg; };
  const float2 cs = FUSED ? rope_cs[(size_t)pos * (HD / 2) + lane] : make_float2(1.f, 0.f);

  // the loads in two halves, each its keys then its values: loads return in
  // issue order, so the first half's arithmetic waits for the first half only
  // and runs while the second half streams in
  constexpr int J0 = (NJ + 1) / 2;
  u32x4 kr[NJ][LW], vr[NJ][LW];
#pragma unroll
  for (int half = 0; half < 2; half++) {
#pragma unroll
    for (int j = half ? J0 : 0; j < (half ? NJ : J0); j++) {
      const KV *p = kc + (size_t)min(position(j), last) * HD + 8 * r16;
#pragma unroll
      for (int e = 0; e < LW; e++) kr[j][e] = gload16(p + e * 4);
    }
#pragma unroll
    for (int j = half ? J0 : 0; j < (half ? NJ : J0); j++) {
      const KV *p = vc + (size_t)min(position(j), last) * HD + 8 * r16;
#pragma unroll
      for (int e = 0; e < LW; e++) vr[j][e] = gload16(p + e * 4);
    }
    __builtin_amdgcn_sched_barrier(0);  // the halves issued in this order
  }

  const size_t slot = (HD + 2);
  float *pm = part + ((size_t)m * heads + g * GRP) * (S + 1) * slot;  // head h at h (S + 1) slot
  if (FUSED) {
#pragma unroll
    for (int h = 0; h < GRP; h++) {
      norm_rope(x0[h], x1[h], wq0, wq1, cs, eps);
      qw[wave][h][lane] = x0[h];
      qw[wave][h][lane + 64] = x1[h];
      if (s == 0 && wave == h) {
        float *qo = pm + ((size_t)h * (S + 1) + S) * slot;
        qo[lane] = x0[h];
        qo[lane + 64] = x1[h];
      }
    }
    if (app) {
      if (wave == NWV - 2) norm_rope(a0, a1, wk0, wk1, cs, eps);
      KV *dst = (wave == NWV - 2 ? kc : vc) + (size_t)pos * HD;
      dst[lane] = to_cache<KV>(a0);
      dst[lane + 64] = to_cache<KV>(a1);
    }
    // the wave's own rows of LDS: ordered within the wave, no block barrier
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int h = 0; h < GRP; h++) {
      const float4 *p = reinterpret_cast<const float4 *>(&qw[wave][h][8 * r16]);
      const float4 u = p[0], v = p[1];
      q[h][0] = u.x, q[h][1] = u.y, q[h][2] = u.z, q[h][3] = u.w;
      q[h][4] = v.x, q[h][5] = v.y, q[h][6] = v.z, q[h][7] = v.w;
    }
  }

  // scores, softmax and values in two phases over the halves of the loads,
  // an online softmax per wave and query head: the running maximum mw
  // (alike across the wave), and lane partials of the sum (ls) and output (o)
  // rescaled when the maximum grows
  const float scale = (float)(1.0 / sqrt((double)HD));
  float mw[GRP], ls[GRP], o[GRP][8];
#pragma unroll
  for (int h = 0; h < GRP; h++) {
    mw[h] = -INFINITY;
    ls[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) o[h][e] = 0.f;
  }
  auto phase = [&](auto lo_c, auto hi_c) {
    constexpr int LO = decltype(lo_c)::value, HI = decltype(hi_c)::value;
    float sc[GRP][NJ];
#pragma unroll
    for (int j = LO; j < HI; j++) {
      float k8[8];
      cvt8(kr[j], k8);
#pragma unroll
      for (int h = 0; h < GRP; h++) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) a = fmaf(q[h][e], k8[e], a);
        sc[h][j] = a;
      }
    }
#pragma unroll
    for (int h = 0; h < GRP; h++)
#pragma unroll
      for (int j = LO; j < HI; j++) sc[h][j] += dpp_f<kQuadXor1>(sc[h][j]);
#pragma unroll
    for (int h = 0; h < GRP; h++)
#pragma unroll
      for (int j = LO; j < HI; j++) sc[h][j] += dpp_f<kQuadXor2>(sc[h][j]);
#pragma unroll
    for (int h = 0; h < GRP; h++)
#pragma unroll
      for (int j = LO; j < HI; j++) sc[h][j] += dpp_f<kHalfMirror>(sc[h][j]);
#pragma unroll
    for (int h = 0; h < GRP; h++)
#pragma unroll
      for (int j = LO; j < HI; j++) sc[h][j] += dpp_f<kRowMirror>(sc[h][j]);
#pragma unroll
    for (int h = 0; h < GRP; h++) {
      float v = -INFINITY;
#pragma unroll
      for (int j = LO; j < HI; j++) {
        sc[h][j] = position(j) < n ? sc[h][j] * scale : -INFINITY;
        v = fmaxf(v, sc[h][j]);
      }
      v = rows4_max(v);  // alike across a 16-lane row: the four rows' maximum
      const float m_new = fmaxf(mw[h], v);
      // no position so far: weights 0 whatever the reference
      const float ref = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = mw[h] == -INFINITY ? 0.f : __expf(mw[h] - ref);
      mw[h] = m_new;
      float l = ls[h] * alpha;
#pragma unroll
      for (int e = 0; e < 8; e++) o[h][e] *= alpha;
#pragma unroll
      for (int j = LO; j < HI; j++) {
        sc[h][j] = __expf(sc[h][j] - ref);
        l += sc[h][j];
      }
      ls[h] = l;
    }
#pragma unroll
    for (int j = LO; j < HI; j++) {
      float v8[8];
      cvt8(vr[j], v8);
#pragma unroll
      for (int h = 0; h < GRP; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[h][e] = fmaf(sc[h][j], v8[e], o[h][e]);
    }
  };
  phase(std::integral_constant<int, 0>{}, std::integral_constant<int, J0>{});
  phase(std::integral_constant<int, J0>{}, std::integral_constant<int, NJ>{});
  float lw[GRP];
#pragma unroll
  for (int h = 0; h < GRP; h++) lw[h] = rows4_sum(ls[h]);
  // the 4 position groups of a wave (lanes l, l + 16, l + 32, l + 48), then
  // the waves through LDS, each rescaled to the split's maximum
#pragma unroll
  for (int h = 0; h < GRP; h++) {
    float lo, hi;
    rows4_scatter8(o[h], lo, hi);
    po[wave][h][8 * r16 + (lane >> 4)] = lo;
    po[wave][h][8 * r16 + 4 + (lane >> 4)] = hi;
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < GRP; h++) {
      wmx[wave][h] = mw[h];
      wsum[wave][h] = lw[h];
    }
  }
  __syncthreads();
  for (int i = t; i < GRP * HD; i += NTL) {
    const int h = i / HD, dd = i % HD;
    float mx = wmx[0][h];
#pragma unroll
    for (int w = 1; w < NWV; w++) mx = fmaxf(mx, wmx[w][h]);
    float acc = 0.f, sum = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; w++) {
      const float c = rescale(wmx[w][h], mx);
      acc = fmaf(c, po[w][h][dd], acc);
      sum = fmaf(c, wsum[w][h], sum);
    }
    float *pp = pm + ((size_t)h * (S + 1) + s) * slot;
    pp[dd] = acc;
    if (dd == 0) {
      pp[HD] = sum > 0.f ? mx : -INFINITY;
      pp[HD + 1] = sum;
    }
  }
}

// The splits of (query head h, row m) merged, with the new position of a
// fused row: out = sum_s c_s acc_s / sum_s c_s sum_s, c_s = exp(max_s - max).
// 512 threads, thread (q, d) adding the splits q, q + 4, ... for dim d, 16
// loads at a time, all issued first with the splits' maxima and sums. Every
// wave finds the maximum and the c_s of all splits itself (a lane per split,
// wave reductions) into its own row of LDS, read back by that wave only, so
// the block meets twice: for the new position's score (fused: the 128-dim dot
// of the query head in slot S with the new key, the halves of waves 0 and 1)
// and for the four split groups' sums, added in group order.
template <typename KV, bool FUSED, int GRP>
__global__ __launch_bounds__(512) void k_attn_merge(const RowDesc *__restrict__ rd,
                                                    const float *__restrict__ part,
                                                    float *__restrict__ outp, int layer, int kvh,
                                                    int S) {
  constexpr int NQ = 4, U = 16, NW = 8, SPL = kMaxSplitsLong / 64;
  __shared__ float cw[NW][kMaxSplitsLong];
  __shared__ float red[NQ - 1][HD];
  __shared__ float qk[2];
  const int h = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
  const int q = t / HD, dd = t % HD;
  const int lane = t & 63, wave = t >> 6;
  const int heads = GRP * kvh, g = h / GRP;
  const size_t slot = HD + 2;
  const float *p0 = part + ((size_t)m * heads + h) * (S + 1) * slot;
  const float *ph = p0 + dd;
  float *out = outp + ((size_t)m * heads + h) * HD;
  float a[U];
#pragma unroll
  for (int u = 0; u < U; u++) a[u] = ph[(size_t)min(q + NQ * u, S - 1) * slot];
  float mv[SPL], lv[SPL];
#pragma unroll
  for (int j = 0; j < SPL; j++) {
    const int sp = min(lane + 64 * j, S - 1);
    mv[j] = p0[(size_t)sp * slot + HD];
    lv[j] = p0[(size_t)sp * slot + HD + 1];
  }
  float qv = 0.f;
  if (FUSED) qv = ph[(size_t)S * slot];
  const RowDesc d = rd[m];
  if (d.pos < 0) {  // inactive row (the same for the whole block): zeros
    if (q == 0) out[dd] = 0.f;
    return;
  }
  const float scale = (float)(1.0 / sqrt((double)HD));
  float score = -INFINITY, vn = 0.f;
  if (FUSED) {
    const size_t off = (((size_t)layer * kvh + g) * d.max_pos + d.pos) * HD + dd;
    const float kn = (float)global_ptr(reinterpret_cast<const KV *>(d.k))[off];
    vn = (float)global_ptr(reinterpret_cast<const KV *>(d.v))[off];
    if (q == 0) {  // waves 0 and 1: dims 0-63 and 64-127
      const float v = wave_sum_dpp(qv * kn);
      if (lane == 0) qk[wave] = v;
    }
    __syncthreads();
    score = (qk[0] + qk[1]) * scale;
  }
  // this wave: the maximum over the splits (and the new position), the c_s
  // into its own LDS row, the denominator
  float mx = score;
#pragma unroll
  for (int j = 0; j < SPL; j++)
    if (lane + 64 * j < S) mx = fmaxf(mx, mv[j]);
  mx = wave_max_dpp(mx);
  float den = 0.f;
#pragma unroll
  for (int j = 0; j < SPL; j++) {
    const int sp = lane + 64 * j;
    if (sp < S) {
      const float c = rescale(mv[j], mx);
      cw[wave][sp] = c;
      den = fmaf(lv[j], c, den);
    }
  }
  den = wave_sum_dpp(den);
  // the row is this wave's own: its LDS accesses are done in order
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float acc = 0.f;
  for (int k0 = 0;; k0 += U) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int sp = q + NQ * (k0 + u);
      acc = sp < S ? fmaf(a[u], cw[wave][min(sp, S - 1)], acc) : acc;
    }
    if (q + NQ * (k0 + U) >= S) break;
#pragma unroll
    for (int u = 0; u < U; u++) a[u] = ph[(size_t)min(q + NQ * (k0 + U + u), S - 1) * slot];
  }
  if (q > 0) red[q - 1][dd] = acc;
  __syncthreads();
  if (q == 0) {
#pragma unroll
    for (int i = 0; i < NQ - 1; i++) acc += red[i][dd];
    float l = den;
    if (FUSED) {
      const float c = __expf(score - mx);
      l += c;
      acc = fmaf(c, vn, acc);
    }
    out[dd] = l > 0.f ? acc / l : 0.f;
  }
}

// 4 quants (one dword) times 4 activations, added to acc
__device__ __forceinline__ float dot4_q8(int w, float4 x, float acc) {
  acc = fmaf((float)(int8_t)(w), x.x, acc);
  acc = fmaf((float)(int8_t)(w >> 8), x.y, acc);
  acc = fmaf((float)(int8_t)(w >> 16), x.z, acc);
  acc = fmaf((float)(int8_t)(w >> 24), x.w, acc);
  return acc;
}

// o_proj of one decode row with the split attention's merge in its prologue
// (up to 16 SR splits): every workgroup merges the splits of all 16 query
// heads into LDS, then computes its Q8_0 rows of y += W_o x as k_gemv_q8v
// does (a wave per row, 16 quants per lane and 1024-column chunk, its scales,
// a wave sum). Thread t merges head t / 16, dims 8 (t % 16) .. + 7: the 16
// threads of a head hold the splits' maxima and sums (split t % 16 + 16 r),
// meet in 16-lane DPP reductions for the maximum (with the new position's
// score when fused: the query head from slot S times the new key) and the
// denominator, and pass the weights c_s = exp(max_s - max) by lane shuffles;
// the first 16 splits' outputs are loaded with everything else, before the
// maximum is known (one memory round trip), the next 16 after. x goes to LDS in k_gemv_q8w's
// bank-conflict-free order (element c 1024 + l 16 + 4 i + e in float4 slot
// (c 4 + i) 64 + l). Replaces k_attn_merge + the o_proj product: one launch
// and one dependent round trip fewer per layer; each workgroup re-reads the
// partials (16 heads x S x 130 floats, from L2), which bounds S.
template <typename KV, bool FUSED, int GRP, int SR, int R>
__global__ __launch_bounds__(256) void k_attn_merge_o(const int8_t *__restrict__ wq,
                                                      const RowDesc *__restrict__ rd,
                                                      const float *__restrict__ part,
                                                      float *__restrict__ y, int N, int layer,
                                                      int kvh, int S) {
  constexpr int C = 2, K = C * 1024, NB = K / 32;  // 16 query heads of 128
  __shared__ float4 xs[K / 4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int h = t >> 4, j = t & 15, g = h / GRP;
  const size_t slot = HD + 2;
  // 1. this wave's R weight rows (4 R per workgroup)
  const int row0 = (blockIdx.x * 4 + wave) * R;
  const _Float16 *dsc = reinterpret_cast<const _Float16 *>(wq + (size_t)N * K);
  int4 wv[R][C];
  float sc[R][C], yres[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = min(row0 + r, N - 1);
    const int8_t *qw = wq + (size_t)row * K + lane * 16;
    const _Float16 *dw = dsc + (size_t)row * NB + (lane >> 1);
#pragma unroll
    for (int c = 0; c < C; c++) {
      wv[r][c] = *reinterpret_cast<const int4 *>(qw + c * 1024);
      sc[r][c] = (float)dw[c * 32];
    }
    yres[r] = y[row];
  }
  // 2. the merge's inputs: head h's split maxima and sums, the query head
  const float *p0 = part + (size_t)h * (S + 1) * slot;
  float mv[SR], lv[SR];
#pragma unroll
  for (int r = 0; r < SR; r++) {
    const int sp = min(j + 16 * r, S - 1);
    mv[r] = p0[(size_t)sp * slot + HD];
    lv[r] = p0[(size_t)sp * slot + HD + 1];
  }
  float qh[8];
  if (FUSED) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float2 v = *reinterpret_cast<const float2 *>(p0 + (size_t)S * slot + 8 * j + 2 * e);
      qh[2 * e] = v.x;
      qh[2 * e + 1] = v.y;
    }
  }
  // the first 16 splits' outputs (this thread's 8 dims), with the rest
  float2 a[16][4];
#pragma unroll
  for (int u = 0; u < 16; u++) {
    if (u < S) {  // (S is the same for the whole workgroup)
      const float *ps = p0 + (size_t)u * slot + 8 * j;
#pragma unroll
      for (int e = 0; e < 4; e++) a[u][e] = *reinterpret_cast<const float2 *>(ps + 2 * e);
    }
  }
  const RowDesc d = rd[0];
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; e++) x[e] = 0.f;
  if (d.pos >= 0) {  // (an inactive row adds nothing)
    const float scale = (float)(1.0 / sqrt((double)HD));
    float score = -INFINITY, vn[8];
    if (FUSED) {
      const size_t off = (((size_t)layer * kvh + g) * d.max_pos + d.pos) * HD + 8 * j;
      const KV *kr = global_ptr(reinterpret_cast<const KV *>(d.k)) + off;
      const KV *vr = global_ptr(reinterpret_cast<const KV *>(d.v)) + off;
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        dot = fmaf(qh[e], (float)kr[e], dot);
        vn[e] = (float)vr[e];
      }
      score = group16_sum_dpp(dot) * scale;
    }
    float mx = score;
#pragma unroll
    for (int r = 0; r < SR; r++)
      if (j + 16 * r < S) mx = fmaxf(mx, mv[r]);
    mx = fmaxf(mx, dpp_f_keep<kQuadXor1>(mx));
    mx = fmaxf(mx, dpp_f_keep<kQuadXor2>(mx));
    mx = fmaxf(mx, dpp_f_keep<kHalfMirror>(mx));
    mx = fmaxf(mx, dpp_f_keep<kRowMirror>(mx));
    float cw[SR], den = 0.f;
#pragma unroll
    for (int r = 0; r < SR; r++) {
      cw[r] = j + 16 * r < S ? rescale(mv[r], mx) : 0.f;
      den = fmaf(lv[r], cw[r], den);
    }
    den = group16_sum_dpp(den);
    const int base = lane & ~15;
#pragma unroll
    for (int r = 0; r < SR; r++) {
      if (r > 0) {  // splits 16 r .. min(16 r + 15, S - 1)
#pragma unroll
        for (int u = 0; u < 16; u++) {
          if (16 * r + u < S) {
            const float *ps = p0 + (size_t)(16 * r + u) * slot + 8 * j;
#pragma unroll
            for (int e = 0; e < 4; e++) a[u][e] = *reinterpret_cast<const float2 *>(ps + 2 * e);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 16; u++) {
        const int s = 16 * r + u;
        const float c = __shfl(cw[r], base | u);
        if (s < S) {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            x[2 * e] = fmaf(c, a[u][e].x, x[2 * e]);
            x[2 * e + 1] = fmaf(c, a[u][e].y, x[2 * e + 1]);
          }
        }
      }
    }
    float l = den;
    if (FUSED) {
      const float cn = __expf(score - mx);
      l += cn;
#pragma unroll
      for (int e = 0; e < 8; e++) x[e] = fmaf(cn, vn[e], x[e]);
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) x[e] = l > 0.f ? x[e] * inv : 0.f;
  }
  // x into LDS: elements k0 .. k0 + 7, k0 = 128 h + 8 j
  {
    const int k0 = 128 * h + 8 * j, c = k0 >> 10, l = (k0 & 1023) >> 4, i0 = (k0 & 15) >> 2;
    xs[(c * 4 + i0) * 64 + l] = make_float4(x[0], x[1], x[2], x[3]);
    xs[(c * 4 + i0 + 1) * 64 + l] = make_float4(x[4], x[5], x[6], x[7]);
  }
  __syncthreads();
  // 3. the rows' dot products
  float4 xl[C][4];
#pragma unroll
  for (int c = 0; c < C; c++)
#pragma unroll
    for (int i = 0; i < 4; i++) xl[c][i] = xs[(c * 4 + i) * 64 + lane];
#pragma unroll
  for (int r = 0; r < R; r++) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < C; c++) {
      float p0s = dot4_q8(wv[r][c].x, xl[c][0], 0.f);
      float p1s = dot4_q8(wv[r][c].y, xl[c][1], 0.f);
      p0s = dot4_q8(wv[r][c].z, xl[c][2], p0s);
      p1s = dot4_q8(wv[r][c].w, xl[c][3], p1s);
      acc = fmaf(sc[r][c], p0s + p1s, acc);
    }
    acc = wave_sum_dpp(acc);
    if (lane == 0 && row0 + r < N) y[row0 + r] = yres[r] + acc;
  }
}

typedef float v4f __attribute__((ext_vector_type(4)));

// 4 cache elements as f32 (16 bytes of f32, 8 of f16)
__device__ __forceinline__ float4 ld4kv(const float *p) {
  return *reinterpret_cast<const float4 *>(p);
}
__device__ __forceinline__ float4 ld4kv(const _Float16 *p) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 v = *reinterpret_cast<const h4 *>(p);
  return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}

typedef __bf16 bf8v __attribute__((ext_vector_type(8)));

// eight f32 values split into three bf16 parts each (x = hi + mid + lo
// exactly), each part packed as the 8 bf16 of one matrix-core operand
__device__ __forceinline__ void split8(const float (&x)[8], u32x4 &h, u32x4 &m, u32x4 &l) {
  uint32_t hh[8], mm[8], ll[8];
#pragma unroll
  for (int e = 0; e < 8; e++) split3(x[e], hh[e], mm[e], ll[e]);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    h[i] = hh[2 * i] | (hh[2 * i + 1] << 16);
    m[i] = mm[2 * i] | (mm[2 * i + 1] << 16);
    l[i] = ll[2 * i] | (ll[2 * i + 1] << 16);
  }
}

// acc += A B for f32 operands given as three bf16 parts each: the six part
// products of weight at least 2^-16 of the product (mid mid, lo hi, hi lo,
// mid hi, hi mid, hi hi, smallest first), each exact in fp32; the three
// dropped weigh below 2^-23 of the product, under its fp32 rounding
__device__ __forceinline__ v4f mfma_x3(const u32x4 (&a)[3], const u32x4 (&b)[3], v4f acc) {
  const bf8v ah = __builtin_bit_cast(bf8v, a[0]), am = __builtin_bit_cast(bf8v, a[1]),
             al = __builtin_bit_cast(bf8v, a[2]);
  const bf8v bh = __builtin_bit_cast(bf8v, b[0]), bm = __builtin_bit_cast(bf8v, b[1]),
             bl = __builtin_bit_cast(bf8v, b[2]);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bm, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bm, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
  return acc;
}

// Prefill attention (rows m = 0 .. M-1 of one context at positions pos0 + m,
// their keys and values already in the cache, q already normed and rotated):
// causal softmax(q K^T / sqrt(128)) V on the bf16 matrix cores
// (v_mfma_f32_16x16x32_bf16, lane l holding A[l % 16][8 (l / 16) .. + 7] and
// B[8 (l / 16) .. + 7][l % 16], receiving D[4 (l / 16) + r][l % 16]) with
// every f32 operand split exactly into three bf16 parts (mfma_x3): 6 bf16
// products per 32 dims or keys where f32 operands take 8 v_mfma_f32_16x16x4_f32
// of twice the cycles each. One workgroup of 4 waves per (query head h, tile of
// 16 query rows); wave w takes the 32-key blocks w, w + 4, ... up to the
// tile's last position and keeps its own running maximum, sum and output:
//   - scores S^T = K Q^T per 16-key half: A = 16 keys, B = the 16 queries, k =
//     32 dims at a time (4 steps); lane l receives S[query l % 16][key
//     16 half + 4 (l / 16) + r];
//   - online softmax per query over the 32 keys (lanes l, l ^ 16, l ^ 32,
//     l ^ 48 hold a query's keys); keys after the query's position masked;
//   - O += P V with k = the 32 keys in the order the scores left them in the
//     lanes: slot 8 (l / 16) + j is key 4 (l / 16) + j (j < 4) of the first
//     half, 16 + 4 (l / 16) + j - 4 of the second, so lane l's eight scores
//     are its A operand as they are, and its B operand the values of the same
//     eight keys in dims 16 t + l % 16;
//   - the 4 waves' (max, sum, output) merged in LDS; each output element
//     rescaled to the largest of the waves' maxima.
template <typename KV, int GRP>
__global__ __launch_bounds__(256) void k_attn_prefill_x3(const RowDesc *__restrict__ rd,
                                                         const float *__restrict__ qkv, int ldq,
                                                         int layer, int kvh, int M,
                                                         float *__restrict__ outp) {
  __shared__ float ms[4][16], ls[4][16];
  __shared__ float os[4][8][4][64];
  // the tiles with the most keys first; a kv head's query heads on one XCD
  const int g = blockIdx.x % kvh, h = g * GRP + blockIdx.x / kvh;
  const int q0 = (gridDim.y - 1 - blockIdx.y) * 16;
  const int heads = GRP * kvh;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r16 = lane & 15, gq = lane >> 4;
  const RowDesc d = rd[0];
  const int pos0 = d.pos;
  const int p_hi = pos0 + min(q0 + 15, M - 1);  // the tile's last position
  const int pq = pos0 + q0 + r16;              // this lane's query position
  const size_t head_off = ((size_t)layer * kvh + g) * d.max_pos * HD;
  const KV *kc = global_ptr(reinterpret_cast<const KV *>(d.k)) + head_off;
  const KV *vc = global_ptr(reinterpret_cast<const KV *>(d.v)) + head_off;
  // this lane's query: row min(q0 + r16, M - 1), dims 32 c + 8 gq .. + 7
  u32x4 qp[4][3];
  {
    const float *qr = qkv + (size_t)min(q0 + r16, M - 1) * ldq + h * HD + 8 * gq;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float4 a = *reinterpret_cast<const float4 *>(qr + 32 * c);
      const float4 b = *reinterpret_cast<const float4 *>(qr + 32 * c + 4);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      split8(x, qp[c][0], qp[c][1], qp[c][2]);
    }
  }
  const float scale = (float)(1.0 / sqrt((double)HD));
  float m_run = -INFINITY, l_run = 0.f;
  v4f o[8];
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = v4f{0.f, 0.f, 0.f, 0.f};
  const int nblk = p_hi / 32 + 1;
  for (int b = wave; b < nblk; b += 4) {
    const int kb = 32 * b;
    // keys kb + 16 hf + r16, dims 32 c + 8 gq .. + 7; values of the lane's
    // eight key slots, dims 16 i + r16
    float4 kf[2][4][2];
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      const KV *kr = kc + (size_t)min(kb + 16 * hf + r16, p_hi) * HD + 8 * gq;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        kf[hf][c][0] = ld4kv(kr + 32 * c);
        kf[hf][c][1] = ld4kv(kr + 32 * c + 4);
      }
    }
    v4f sa[2];
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      sa[hf] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float x[8] = {kf[hf][c][0].x, kf[hf][c][0].y, kf[hf][c][0].z, kf[hf][c][0].w,
                            kf[hf][c][1].x, kf[hf][c][1].y, kf[hf][c][1].z, kf[hf][c][1].w};
        u32x4 kp[3];
        split8(x, kp[0], kp[1], kp[2]);
        sa[hf] = mfma_x3(kp, qp[c], sa[hf]);
      }
    }
    // the values, loaded once the keys are consumed (both in flight together
    // would take the registers of a second wave per SIMD)
    float vv[8][8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int key = kb + (j < 4 ? 4 * gq + j : 16 + 4 * gq + j - 4);
      const KV *vr = vc + (size_t)min(key, p_hi) * HD + r16;
#pragma unroll
      for (int i = 0; i < 8; i++) vv[i][j] = (float)vr[16 * i];
    }
    float p[8], bm = -INFINITY;
#pragma unroll
    for (int hf = 0; hf < 2; hf++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float s = kb + 16 * hf + 4 * gq + r <= pq ? sa[hf][r] * scale : -INFINITY;
        p[4 * hf + r] = s;
        bm = fmaxf(bm, s);
      }
    bm = rows4_max(bm);
    const float m_new = fmaxf(m_run, bm);
    const float ref = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = m_run == -INFINITY ? 0.f : __expf(m_run - ref);
    float ps = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      p[j] = __expf(p[j] - ref);
      ps += p[j];
    }
    ps = rows4_sum(ps);
    l_run = fmaf(l_run, alpha, ps);
    m_run = m_new;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float ar = __shfl(alpha, 4 * gq + r);
#pragma unroll
      for (int i = 0; i < 8; i++) o[i][r] *= ar;
    }
    u32x4 pp[3];
    split8(p, pp[0], pp[1], pp[2]);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      u32x4 vp[3];
      split8(vv[i], vp[0], vp[1], vp[2]);
      o[i] = mfma_x3(pp, vp, o[i]);
    }
  }
  if (gq == 0) {
    ms[wave][r16] = m_run;
    ls[wave][r16] = l_run;
  }
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) os[wave][i][r][lane] = o[i][r];
  __syncthreads();
  // output (query q, dim k): tile i = k / 16, lane 16 (q / 4) + k % 16, r = q % 4
  for (int e = t; e < 16 * HD; e += 256) {
    const int q = e / HD, k = e % HD;
    if (q0 + q >= M) break;
    const int i = k >> 4, l = 16 * (q >> 2) + (k & 15), r = q & 3;
    float mx = ms[0][q];
#pragma unroll
    for (int w = 1; w < 4; w++) mx = fmaxf(mx, ms[w][q]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float c = ms[w][q] == -INFINITY ? 0.f : __expf(ms[w][q] - mx);
      num = fmaf(os[w][i][r][l], c, num);
      den = fmaf(ls[w][q], c, den);
    }
    outp[(size_t)(q0 + q) * (heads * HD) + h * HD + k] = den > 0.f ? num / den : 0.f;
  }
}

template <typename KV, bool FUSED, int G>
int launch_g(const AttnArgs &a, int M, int positions, hipStream_t st, bool merge) {
  const SplitShape sh = attn_split_shape(positions, sizeof(KV) == 2, !merge);
  const int S = (positions + sh.len - 1) / sh.len;
  // decode rows: as many workgroups again load the next layer's cache rows
  // ahead, while a layer's cache of the launch is at most kPrefetchSplitBytes
  // (measured: decode step at 2048 positions, f16, 598 -> 584 us; at 8192, where
  // the extra 34 MB per layer doubles this kernel's HBM stream, 676 -> 775 us)
  const bool pf_fits = (size_t)positions * M * a.kvh * HD * 2 * sizeof(KV) <= kPrefetchSplitBytes;
  const int pfl = FUSED && pf_fits && a.layer + 1 < a.layers ? a.layer + 1 : -1;
  const int gy = S + (pfl >= 0 ? S : 0);
#define Q3H_S(NJ)                                                                              \
  hipLaunchKernelGGL((k_attn_split<KV, FUSED, G, 16 * NJ, 256>), dim3(a.kvh, gy, M), dim3(256), 0, \
                     st, a.rd, a.qkv, a.rope_cs, a.qkn, a.layer, a.kvh, S, a.part, pfl)
  if (sh.len == kSplit && sh.threads == 0) {
    // decode rows: extra workgroups load the next layer's cache rows ahead (above)
    const int pf = FUSED && a.layer + 1 < a.layers ? a.layer + 1 : -1;
    const int gx = a.heads + (pf >= 0 ? a.kvh * kPrefetchParts : 0);
    // 32 position groups: 2 positions per thread for every 64 covered
#define Q3H_SH(NJ)                                                                          \
  hipLaunchKernelGGL((k_attn_short<KV, FUSED, G, 512, NJ>), dim3(gx, M), dim3(512), 0, st,    \
                     a.rd, a.qkv, a.rope_cs, a.qkn, a.out, a.layer, a.kvh, pf)
    switch ((std::max(positions, 1) + 63) / 64) {
      case 1: Q3H_SH(2); break;
      case 2: Q3H_SH(4); break;
      case 3: Q3H_SH(6); break;
      default: Q3H_SH(8); break;
    }
#undef Q3H_SH
  } else {
    switch (sh.len / 16) {
      case 2: Q3H_S(2); break;
      case 3: Q3H_S(3); break;
      case 4: Q3H_S(4); break;
      case 5: Q3H_S(5); break;
      case 6: Q3H_S(6); break;
      case 7: Q3H_S(7); break;
      default:
        if constexpr (sizeof(KV) == 2) {
          if (sh.len / 16 == 8)
            Q3H_S(8);
          else if (sh.len / 16 == 9)
            Q3H_S(9);
          else
            Q3H_S(16);
        } else {
          Q3H_S(8);
        }
        break;
    }
  }
#undef Q3H_S
  if (sh.threads == 0 || !merge) return 1;
  hipLaunchKernelGGL((k_attn_merge<KV, FUSED, G>), dim3(a.heads, M), dim3(512), 0, st, a.rd,
                     a.part, a.out, a.layer, a.kvh, S);
  return 2;
}

template <typename KV, bool FUSED>
int launch_kv(const AttnArgs &a, int M, int positions, hipStream_t st, bool merge) {
  const int grp = a.heads / a.kvh;
  if (grp == 1) return launch_g<KV, FUSED, 1>(a, M, positions, st, merge);
  if (grp == 2) return launch_g<KV, FUSED, 2>(a, M, positions, st, merge);
  return launch_g<KV, FUSED, 4>(a, M, positions, st, merge);
}

constexpr int kMergeORows = 1;  // weight rows per wave

template <typename KV, bool FUSED, int G>
void launch_mo(const AttnArgs &a, const Mat &wo, float *y, int S, hipStream_t st) {
  constexpr int R = kMergeORows;
  const dim3 grid((wo.N + 4 * R - 1) / (4 * R)), block(256);
  if (S <= 16)
    hipLaunchKernelGGL((k_attn_merge_o<KV, FUSED, G, 1, R>), grid, block, 0, st, wo.q, a.rd,
                       a.part, y, wo.N, a.layer, a.kvh, S);
  else
    hipLaunchKernelGGL((k_attn_merge_o<KV, FUSED, G, 2, R>), grid, block, 0, st, wo.q, a.rd,
                       a.part, y, wo.N, a.layer, a.kvh, S);
}

template <typename KV, bool FUSED>
void launch_mo_kv(const AttnArgs &a, const Mat &wo, float *y, int S, hipStream_t st) {
  const int grp = a.heads / a.kvh;
  if (grp == 1)
    launch_mo<KV, FUSED, 1>(a, wo, y, S, st);
  else if (grp == 2)
    launch_mo<KV, FUSED, 2>(a, wo, y, S, st);
  else
    launch_mo<KV, FUSED, 4>(a, wo, y, S, st);
}

}  // namespace

// The split length for contexts of `positions` positions: a multiple of the
// 16 positions of one block (nj blocks per split, 256 threads). The splits of
// kv head g are workgroups g, g + kvh, ...: with 8 kv heads they share one
// XCD's 32 CUs, so a launch takes ceil(S / 32) rounds of a split's time, and
// S = 33 or 65 left one CU per XCD with an extra split (measured here: 4096
// positions 7.8 -> 6.3 us, 8192 positions 10.6 -> 9.6 us with S = 29 / 57
// instead of 33 / 65). nj minimizes rounds x (nj + 2), the 2 standing for a
// workgroup's fixed work (descriptor, prologue, reductions, stores), ties to
// the fewer splits; nj <= 9 (f16) or 6 (f32) while the splits fit
// kMaxSplitsLong, longer contexts take 16 (f16) or 8 (f32) blocks per split.
SplitShape attn_split_shape(int positions, bool kv16, bool fold) {
  if (positions <= kSplit) return {kSplit, 0};  // one workgroup per query head
  const int blocks = (positions + 15) / 16;
  const int njmax = kv16 ? 9 : 6;
  // merged in o_proj: each of its workgroups reads all the splits' partials
  // (2048 positions: 15 splits of 144 instead of 27 of 80, 0.6 us per layer)
  if (fold && (blocks + njmax - 1) / njmax <= kMergeOMaxSplits) return {16 * njmax, 256};
  int best = 0, cost = 0;
  for (int nj = 2; nj <= njmax; nj++) {
    const int S = (blocks + nj - 1) / nj;
    if (S > kMaxSplitsLong) continue;
    const int c = (S + 31) / 32 * (nj + 2);
    if (best == 0 || c <= cost) best = nj, cost = c;
  }
  // more than kMaxSplitsLong splits of njmax blocks: 16 (f16) or 8 (f32)
  // blocks per split, up to attn_max_positions
  if (best == 0) best = kv16 ? 16 : 8;
  return {16 * best, 256};
}

int attn_splits(int positions, bool kv16) {
  if (positions < 1) return 1;
  // the split kernel's partial slots: one per split and one for the query
  // head, for either shape
  int n = 1;
  for (bool fold : {false, true}) {
    const SplitShape sh = attn_split_shape(positions, kv16, fold);
    if (sh.threads != 0) n = std::max(n, (positions + sh.len - 1) / sh.len + 1);
  }
  return n;
}

int attn_splits_upto(int positions, bool kv16) {
  // the split length changes with the context, so the count is not monotonic:
  // the most over every length up to positions (within a block of 16, the
  // count is largest at the block's last position)
  int n = attn_splits(positions, kv16);
  for (int p = 16; p < positions; p += 16) n = std::max(n, attn_splits(p, kv16));
  return n;
}

int attn_max_positions(bool kv16) { return kMaxSplitsLong * 16 * (kv16 ? 16 : 8); }

int launch_attn(const AttnArgs &a, int M, int positions, bool fused, bool kv16, hipStream_t st,
                bool merge) {
  if (kv16)
    return fused ? launch_kv<_Float16, true>(a, M, positions, st, merge)
                 : launch_kv<_Float16, false>(a, M, positions, st, merge);
  return fused ? launch_kv<float, true>(a, M, positions, st, merge)
               : launch_kv<float, false>(a, M, positions, st, merge);
}

bool attn_merge_o_supported(const AttnArgs &a, const Mat &wo, int M, int positions, bool kv16) {
  const SplitShape sh = attn_split_shape(positions, kv16, true);
  const int S = (positions + sh.len - 1) / sh.len;
  return M == 1 && wo.q != nullptr && wo.K == a.heads * HD && a.heads == 16 && wo.N % 4 == 0 &&
         sh.threads != 0 && S <= kMergeOMaxSplits;
}

void launch_attn_merge_o(const AttnArgs &a, const Mat &wo, float *y, int positions, bool fused,
                         bool kv16, hipStream_t st) {
  const SplitShape sh = attn_split_shape(positions, kv16, true);
  const int S = (positions + sh.len - 1) / sh.len;
  if (kv16)
    fused ? launch_mo_kv<_Float16, true>(a, wo, y, S, st)
          : launch_mo_kv<_Float16, false>(a, wo, y, S, st);
  else
    fused ? launch_mo_kv<float, true>(a, wo, y, S, st) : launch_mo_kv<float, false>(a, wo, y, S, st);
}

}  // namespace q3h

namespace q3h {
void launch_attn_prefill(const AttnArgs &a, int M, bool kv16, hipStream_t st) {
  const dim3 grid(a.heads, (M + 15) / 16), block(256);
  const int grp = a.heads / a.kvh;
#define Q3H_P(KV, G)                                                                         \
  hipLaunchKernelGGL((k_attn_prefill_x3<KV, G>), grid, block, 0, st, a.rd, a.qkv, a.ldq,      \
                     a.layer, a.kvh, M, a.out)
  if (kv16) {
    if (grp == 1) Q3H_P(_Float16, 1);
    else if (grp == 2) Q3H_P(_Float16, 2);
    else Q3H_P(_Float16, 4);
  } else {
    if (grp == 1) Q3H_P(float, 1);
    else if (grp == 2) Q3H_P(float, 2);
    else Q3H_P(float, 4);
  }
#undef Q3H_P
}
}  // namespace q3h
