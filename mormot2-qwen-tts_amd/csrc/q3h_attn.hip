// q3h_attn.hip - GQA decode attention of the Qwen3 stacks on gfx950.
//
// One workgroup per (kv head g, row m, split s); a split is up to 256
// consecutive positions. The GRP query heads of kv head g are served by one
// read of its keys and values. Workgroups of NT = 512 threads (64 groups of
// 8 lanes, at most 4 keys per group per split) serve long contexts; stacks of
// at most 64 positions (the code predictor) use NT = 256. The first two keys
// and values of each group are loaded before the prologue.
//
// Fused prologue (FUSED, rows of distinct contexts, one new position each):
// the workgroup applies the per-head RMSNorm (q_norm / k_norm) and RoPE to the
// raw q and k of its row (straight out of the q/k/v product), rounds the new
// key and value as the cache stores them, and the workgroup whose split holds
// the new position appends them to the cache. That position is then read from
// LDS, the others from the cache (written by earlier launches). Rows that add
// several positions of one context at once (prefill) run the separate append
// kernel first and this kernel unfused.
//
// Body: 8 lanes per key (16 dims each), NT/8 keys per pass, keys and values
// loaded together; each 8-lane group keeps a running max, sum and 16 output
// dims per query head (online softmax), merged across groups by shuffles and
// across waves in LDS.
//
// Splits: with more than one split, each workgroup leaves (max, sum, output)
// per head in the partial buffer and takes a ticket; the last workgroup of a
// (row, kv head) merges the splits in split order and writes the output, then
// clears the ticket for the next launch. No second kernel.
#include <hip/hip_runtime.h>

#include "q3h_internal.h"
#include "q3h_wave.h"

namespace q3h {

namespace {

constexpr int HD = 128;  // head_dim (checked at stack creation)
constexpr int kSplit = 256;  // positions per split (default)

__device__ __forceinline__ double wsum_d(double v) { return wave_sum_dpp_d(v); }

__device__ __forceinline__ void ld16(const float *p, float *o) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float4 t = reinterpret_cast<const float4 *>(p)[i];
    o[4 * i] = t.x;
    o[4 * i + 1] = t.y;
    o[4 * i + 2] = t.z;
    o[4 * i + 3] = t.w;
  }
}

__device__ __forceinline__ void ld16(const _Float16 *p, float *o) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const h8 t = reinterpret_cast<const h8 *>(p)[i];
#pragma unroll
    for (int j = 0; j < 8; j++) o[8 * i + j] = (float)t[j];
  }
}

// weight of a partial state (max m) relative to the merged max mn
__device__ __forceinline__ float rescale(float m, float mn) {
  return m == -INFINITY ? 0.f : expf(m - mn);
}

// Plain scalar arguments, those of the prologue first (the first 16 dwords
// are preloaded into SGPRs); the split buffers come last, read only when S > 1.
template <typename KV, bool FUSED, int GRP, int NT>
__global__ __launch_bounds__(NT) void k_attn(const RowDesc *__restrict__ rd,
                                             const float *__restrict__ qkv,
                                             const float2 *__restrict__ rope_cs,
                                             const float *__restrict__ qn,
                                             const float *__restrict__ kn, float *__restrict__ outp,
                                             int layer, int kvh, float eps, int S, int chunk,
                                             float *__restrict__ part, int *__restrict__ tickets) {
  constexpr int NW = NT / 64, NG = NT / 8;
  const int heads = GRP * kvh, ldq = (heads + 2 * kvh) * HD;
  __shared__ float qs[GRP][HD];
  __shared__ float kvn[2][HD];  // the new key and value, as the cache holds them
  __shared__ float wm[NW][GRP], wl[NW][GRP];
  __shared__ float wo[NW][GRP][HD];
  __shared__ int last;
  const int g = blockIdx.x, m = blockIdx.y, s = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float *row = qkv + (size_t)m * ldq;
  // raw q / k / v of this row (independent of the row descriptor): each wave
  // takes vectors wave and wave + NW of the GRP + 2 (q heads, key, value)
  float xr[2][2];
  if (FUSED) {
#pragma unroll
    for (int vi = 0; vi < 2; vi++) {
      const int vec = wave + vi * NW;
      if (vec < GRP + 2) {
        const size_t off = vec < GRP ? (size_t)(g * GRP + vec) * HD
                                     : (size_t)(heads + (vec - GRP) * kvh + g) * HD;
        xr[vi][0] = row[off + lane];
        xr[vi][1] = row[off + lane + 64];
      }
    }
  }
  const RowDesc d = rd[m];
  float *out = outp + (size_t)m * heads * HD + (size_t)g * GRP * HD;
  if (d.pos < 0) {  // inactive row: zeros, no ticket
    if (s == 0)
      for (int i = tid; i < GRP * HD; i += NT) out[i] = 0.f;
    return;
  }
  const int n = d.pos + 1;
  const int p0 = s * chunk, p1 = min(n, p0 + chunk);
  const size_t head_off = ((size_t)layer * kvh + g) * d.max_pos * HD;
  const KV *kc = reinterpret_cast<const KV *>(d.k) + head_off;
  const KV *vc = reinterpret_cast<const KV *>(d.v) + head_off;

  // the first two keys and values of this thread's group, loaded before the
  // prologue (they do not depend on q); the new position comes from LDS
  const int sub = tid & 7, pg = tid >> 3;
  const int pf0 = p0 + pg, pf1 = pf0 + NG;
  float kk0[16], vv0[16], kk1[16], vv1[16];
  if (pf0 < p1 && !(FUSED && pf0 == d.pos)) {
    ld16(kc + (size_t)pf0 * HD + sub * 16, kk0);
    ld16(vc + (size_t)pf0 * HD + sub * 16, vv0);
  }
  if (pf1 < p1 && !(FUSED && pf1 == d.pos)) {
    ld16(kc + (size_t)pf1 * HD + sub * 16, kk1);
    ld16(vc + (size_t)pf1 * HD + sub * 16, vv1);
  }
  const float2 cs = FUSED ? rope_cs[(size_t)d.pos * (HD / 2) + lane] : make_float2(1.f, 0.f);
  __builtin_amdgcn_sched_barrier(0);

  if (FUSED) {
#pragma unroll
    for (int vi = 0; vi < 2; vi++) {
      const int vec = wave + vi * NW;
      if (vec >= GRP + 2) continue;
      float x0 = xr[vi][0], x1 = xr[vi][1];
      if (vec <= GRP) {  // q heads and the key: RMSNorm over the head, RoPE
        const float *w = vec < GRP ? qn : kn;
        const double ss = wsum_d((double)x0 * x0 + (double)x1 * x1);
        const float inv = (float)(1.0 / sqrt(ss / HD + (double)eps));
        x0 = w[lane] * (x0 * inv);
        x1 = w[lane + 64] * (x1 * inv);
        const float y0 = x0 * cs.x - x1 * cs.y;
        const float y1 = x1 * cs.x + x0 * cs.y;
        x0 = y0;
        x1 = y1;
      }
      if (vec < GRP) {
        qs[vec][lane] = x0;
        qs[vec][lane + 64] = x1;
      } else {
        const KV k0 = (KV)x0, k1 = (KV)x1;
        kvn[vec - GRP][lane] = (float)k0;
        kvn[vec - GRP][lane + 64] = (float)k1;
        if (d.pos >= p0 && d.pos < p0 + chunk) {
          KV *dst = const_cast<KV *>(vec == GRP ? kc : vc) + (size_t)d.pos * HD;
          dst[lane] = k0;
          dst[lane + 64] = k1;
        }
      }
    }
  } else {
    for (int i = tid; i < GRP * HD; i += NT) qs[i / HD][i % HD] = row[(size_t)g * GRP * HD + i];
  }
  __syncthreads();

  // one pass over the keys and values of the split
  const float scale = (float)(1.0 / sqrt((double)HD));
  float qv[GRP][16];
#pragma unroll
  for (int j = 0; j < GRP; j++)
#pragma unroll
    for (int i = 0; i < 16; i++) qv[j][i] = qs[j][sub * 16 + i];
  float mx[GRP], sm[GRP], o[GRP][16];
#pragma unroll
  for (int j = 0; j < GRP; j++) {
    mx[j] = -INFINITY;
    sm[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) o[j][i] = 0.f;
  }
  for (int p = pf0; p < p1; p += NG) {
    float kk[16], vv[16];
    if (FUSED && p == d.pos) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        kk[i] = kvn[0][sub * 16 + i];
        vv[i] = kvn[1][sub * 16 + i];
      }
    } else if (p == pf0) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        kk[i] = kk0[i];
        vv[i] = vv0[i];
      }
    } else if (p == pf1) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        kk[i] = kk1[i];
        vv[i] = vv1[i];
      }
    } else {
      ld16(kc + (size_t)p * HD + sub * 16, kk);
      ld16(vc + (size_t)p * HD + sub * 16, vv);
    }
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 16; i++) acc = fmaf(qv[j][i], kk[i], acc);
      acc = group8_sum_dpp(acc);
      const float sc = acc * scale;
      const float mn = fmaxf(mx[j], sc);
      const float c0 = rescale(mx[j], mn), c1 = expf(sc - mn);
      sm[j] = sm[j] * c0 + c1;
#pragma unroll
      for (int i = 0; i < 16; i++) o[j][i] = fmaf(c1, vv[i], o[j][i] * c0);
      mx[j] = mn;
    }
  }
  // merge the 8 key groups of the wave (lanes differing in bits 3..5)
#pragma unroll
  for (int off = 8; off <= 32; off <<= 1) {
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      const float m2 = __shfl_xor(mx[j], off, 64), s2 = __shfl_xor(sm[j], off, 64);
      const float mn = fmaxf(mx[j], m2);
      const float c0 = rescale(mx[j], mn), c1 = rescale(m2, mn);
      sm[j] = sm[j] * c0 + s2 * c1;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float o2 = __shfl_xor(o[j][i], off, 64);
        o[j][i] = o[j][i] * c0 + o2 * c1;
      }
      mx[j] = mn;
    }
  }
  if (lane < 8) {
#pragma unroll
    for (int j = 0; j < GRP; j++) {
#pragma unroll
      for (int i = 0; i < 16; i++) wo[wave][j][lane * 16 + i] = o[j][i];
      if (lane == 0) {
        wm[wave][j] = mx[j];
        wl[wave][j] = sm[j];
      }
    }
  }
  __syncthreads();
  // merge the waves: thread (j, dd)
  for (int t = tid; t < GRP * HD; t += NT) {
    const int j = t / HD, dd = t % HD;
    float mn = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; w++) mn = fmaxf(mn, wm[w][j]);
    float l = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float c = rescale(wm[w][j], mn);
      l += wl[w][j] * c;
      acc += wo[w][j][dd] * c;
    }
    if (S == 1) {
      out[t] = l > 0.f ? acc / l : 0.f;
    } else {
      float *pp = part + (((size_t)m * heads + g * GRP + j) * S + s) * (HD + 2);
      pp[dd] = acc;
      if (dd == 0) {
        pp[HD] = mn;
        pp[HD + 1] = l;
      }
    }
  }
  if (S == 1) return;

  // splits: the last workgroup of (m, g) merges them
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    int *ticket = tickets + (size_t)m * kvh + g;
    const int old = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    last = old == S - 1;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  for (int t = tid; t < GRP * HD; t += NT) {
    const int j = t / HD, dd = t % HD;
    const float *pp = part + ((size_t)m * heads + g * GRP + j) * S * (HD + 2);
    float mn = -INFINITY;
    for (int i = 0; i < S; i++) mn = fmaxf(mn, pp[i * (HD + 2) + HD]);
    float l = 0.f, acc = 0.f;
    for (int i = 0; i < S; i++) {
      const float c = rescale(pp[i * (HD + 2) + HD], mn);
      l += pp[i * (HD + 2) + HD + 1] * c;
      acc += pp[i * (HD + 2) + dd] * c;
    }
    out[t] = l > 0.f ? acc / l : 0.f;
  }
  if (tid == 0) tickets[(size_t)m * kvh + g] = 0;
}

template <typename KV, bool FUSED, int NT>
void launch_grp(const AttnArgs &a, int grp, dim3 grid, hipStream_t st) {
#define Q3H_A(G)                                                                               \
  hipLaunchKernelGGL((k_attn<KV, FUSED, G, NT>), grid, dim3(NT), 0, st, a.rd, a.qkv, a.rope_cs, \
                     a.qn, a.kn, a.out, a.layer, a.kvh, a.eps, (int)grid.z,                    \
                     a.chunk > 0 ? a.chunk : kSplit, a.part, a.tickets)
  if (grp == 1)
    Q3H_A(1);
  else if (grp == 2)
    Q3H_A(2);
  else
    Q3H_A(4);
#undef Q3H_A
}

template <typename KV, int NT>
void launch_nt(const AttnArgs &a, int grp, dim3 grid, bool fused, hipStream_t st) {
  if (fused)
    launch_grp<KV, true, NT>(a, grp, grid, st);
  else
    launch_grp<KV, false, NT>(a, grp, grid, st);
}

}  // namespace

int attn_splits(int positions) {
  const int n = (positions + kSplit - 1) / kSplit;
  return n < 1 ? 1 : n;
}

void launch_attn(const AttnArgs &a, int M, int splits, int max_positions, bool fused, bool kv16,
                 hipStream_t st) {
  const int grp = a.heads / a.kvh;
  const dim3 grid(a.kvh, M, splits);
  const bool wide = max_positions > 64;
  if (kv16) {
    if (wide)
      launch_nt<_Float16, 512>(a, grp, grid, fused, st);
    else
      launch_nt<_Float16, 256>(a, grp, grid, fused, st);
  } else {
    if (wide)
      launch_nt<float, 512>(a, grp, grid, fused, st);
    else
      launch_nt<float, 256>(a, grp, grid, fused, st);
  }
}

}  // namespace q3h
