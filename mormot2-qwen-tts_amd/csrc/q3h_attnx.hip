// q3h_attnx.hip - GQA attention of the int8 path (stacks with act_q8 = 1):
// a fixed evaluation order, followed to the bit by the CPU restatement of the
// same layer, and the Q8_0 quantization of its output (the o_proj input)
// fused into the epilogue. The int8 products make the layer output a
// discontinuous function of the attention output (one element on the other
// side of a rounding boundary of its block moves it by d / 127 of the block
// maximum), so this path computes every fp32 value in one documented order
// instead of to a tolerance.
//
// One workgroup per (kv head, row) for the kv head's query heads:
//  - prologue (a decode row, one new position of its own context): q, k, v
//    of the row (from the product's chunk partials, added in chunk order,
//    when the product left them as partials); RMSNorm of q and of the new k
//    (double sum of squares), RoPE as rope_pair, v copied; the first query
//    head of the kv group appends k, v to the cache, the others use their
//    own copy for the new position;
//  - scores: 16 lanes per key, lane l a fused multiply-add chain over dims
//    8l .. 8l + 7, a balanced pairwise tree over the 16 lanes (DPP row
//    operations), times 1/sqrt(128);
//  - softmax: maximum, exp_ieee(s - max), double sum, inv = (float)(1/sum),
//    weights s * inv;
//  - values: 8 chains of fused multiply-adds over the positions p = j mod 8
//    (wave w runs chain w % 8 for 128 / (waves / 8) of the dims, 512
//    coalesced bytes per key and wave), joined as ((c0 + c1) + (c2 + c3)) +
//    ((c4 + c5) + (c6 + c7));
//  - the head's 128 outputs quantized per 32-block (ggml quantize_row_q8_0_ref
//    semantics) into the operand tiles of the int8 product.
// The attention itself follows src/tts/mormot.ai.tts.qwen.lm.pas (TQwenLm.
// Forward, lm.pas:391-408) through the stack's ForwardEmbeds: causal softmax
// attention with head_dim 128, q head h reading kv head h / (heads / kv_heads).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "q3h_api_internal.h"
#include "q3h_internal.h"
#include "q3h_math.h"
#include "q3h_wave.h"

namespace q3h {
namespace {

constexpr int HD = 128;
constexpr int NCH = 8;  // value chains

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

// elements col and col + 64 of row m: the product's output, or (nch > 0)
// its chunk partials [nch][M][ld] (nch <= kPartialSlots), loaded together
// (clamped chunk indices; qkv_sum adds the first nch in chunk order)
constexpr int NPS = kPartialSlots;
__device__ __forceinline__ void qkv_load(const float *qkv, int ld, int nch, int M, int m, int col,
                                         float (&a)[NPS], float (&b)[NPS]) {
  if (nch == 0) {
    a[0] = qkv[(size_t)m * ld + col];
    b[0] = qkv[(size_t)m * ld + col + 64];
    return;
  }
#pragma unroll
  for (int c = 0; c < NPS; c++) {
    const float *r = qkv + ((size_t)min(c, nch - 1) * M + m) * ld + col;
    a[c] = r[0];
    b[c] = r[64];
  }
}

__device__ __forceinline__ void qkv_sum(int nch, const float (&a)[NPS], const float (&b)[NPS],
                                        float &x0, float &x1) {
  if (nch == 0) {
    x0 = a[0];
    x1 = b[0];
    return;
  }
  x0 = x1 = 0.f;
#pragma unroll
  for (int c = 0; c < NPS; c++) {
    x0 = c < nch ? __fadd_rn(x0, a[c]) : x0;
    x1 = c < nch ? __fadd_rn(x1, b[c]) : x1;
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

// grid (kv heads, M): the GRP query heads of kv head g = blockIdx.x share one
// read of its K/V; nch > 0: the q/k/v come as nch chunk partials. SU / VU:
// the key rounds of the score loop / the positions of the value chains whose
// loads are issued together (deeper for long contexts). The first round of
// keys (and, with PV, of values) is loaded right after the q/k/v loads, so
// that it arrives during the prologue: the cache rows before the row's own
// position were written by earlier launches, and the own position's key and
// value are taken from the prologue in every round. PAIR (FUSED): rows come
// in pairs, row 2i + 1 at the position after row 2i's in the same context;
// the odd row's spare waves rebuild its pair row's key and value (the cache
// row that row 2i's workgroup writes in this launch) from row 2i's partials
// by the same code as that workgroup, so both rows run in one launch.
template <typename KV, bool FUSED, int GRP, int SU, int VU, int NT, bool PV, bool PAIR>
__global__ __launch_bounds__(NT) void k_attn_x(const RowDesc *rd, const float *qkv,
                                               const float *qkn, const float2 *rope_cs,
                                               int8_t *xq, int layer, int nch, int kvh,
                                               int M) {
  constexpr int NWV = NT / 64;
  constexpr int DPW = 16 / NWV;  // dims per lane in the value chains (2 or 1)
  // the launch shapes for contexts of several rounds take unmasked rounds
  // before the row's own position (the short-context shape keeps one code path)
  constexpr bool LONG = SU > 1;
  static_assert(NWV % NCH == 0 && DPW * 64 * (NWV / NCH) == HD, "8 chains over 128 dims");
  extern __shared__ float sc[];  // [GRP][L]: scores, then e^(score - max)
  __shared__ float qs[GRP][HD], kn[HD], vn[HD];
  __shared__ float kn2[PAIR ? HD : 1], vn2[PAIR ? HD : 1];  // the pair row's key, value
  __shared__ float cv[NCH][GRP][HD];
  __shared__ float redf[GRP][NWV];
  __shared__ double redd[GRP][NWV];
  const int g = blockIdx.x, m = blockIdx.y, t = threadIdx.x;
  const int heads = kvh * GRP, ldq = (heads + 2 * kvh) * HD;
  const int lane = t & 63, wave = t >> 6;
  const int NQ = heads * HD, nbq = NQ >> 5, mt16 = (M + 15) >> 4;
  float *dx = reinterpret_cast<float *>(xq + (size_t)mt16 * 16 * NQ);
  // output k of query head h, row m: element (m, h * 128 + k) of the operand tiles
  auto qoff = [&](int h, int k) { return qtile_offset(m, h * HD + k, mt16); };
  // vector j = wave: query head g GRP + j (j < GRP), the new k (j == GRP), v
  // (GRP + 1), and with PAIR the pair row's k and v (GRP + 2, GRP + 3, of
  // kind jv = j - 2); its loads depend on no descriptor, so they are issued
  // first, by every wave (the waves past the last vector load v again and do
  // not use it: no divergent branch before the descriptor's scalar load)
  static_assert(GRP + (PAIR ? 4 : 2) <= NWV, "one prologue vector per wave");
  const int j = wave;
  const bool pairv = PAIR && j >= GRP + 2;
  const int jv = pairv ? j - 2 : j;
  const bool odd = PAIR && (m & 1);
  const bool pj = FUSED && jv < GRP + 2;
  const int col = jv < GRP ? (g * GRP + jv) * HD : jv == GRP ? NQ + g * HD : NQ + (kvh + g) * HD;
  float pa[NPS], pb[NPS];
  if (FUSED) qkv_load(qkv, ldq, nch, M, pairv ? m & ~1 : m, col + lane, pa, pb);
  const RowDesc d = rd[m];
  if (d.pos < 0) {  // inactive row: zero blocks
    for (int i = t; i < GRP * HD; i += NT) {
      const int h = g * GRP + i / HD, k = i % HD;
      xq[qoff(h, k)] = 0;
      if ((k & 31) == 0) dx[(size_t)m * nbq + 4 * h + (k >> 5)] = 0.f;
    }
    return;
  }
  const int pos = d.pos, L = pos + 1;
  // positions below clean hold rows written by earlier launches (the new
  // position, and with PAIR the odd row's pair position, come from the prologue)
  const int clean = FUSED ? pos - (odd ? 1 : 0) : L;
  const size_t head_off = ((size_t)layer * kvh + g) * d.max_pos * HD;
  const KV *kc = global_ptr(reinterpret_cast<const KV *>(d.k)) + head_off;
  const KV *vc = global_ptr(reinterpret_cast<const KV *>(d.v)) + head_off;
  constexpr int KG = NT / 16;
  const int kg = t >> 4, li = t & 15;
  // value chain ch over positions ch, ch + 8, ...; dims dim0 + 64 e, e < DPW
  const int ch = wave % NCH, dim0 = (wave / NCH) * 64 + lane;

  // the first round of keys (positions u KG + kg) and values (ch + NCH u),
  // from clamped positions
  float k8p[SU][8], vp[PV ? VU : 1][DPW];
#pragma unroll
  for (int u = 0; u < SU; u++) load8(kc + (size_t)min(u * KG + kg, L - 1) * HD + 8 * li, k8p[u]);
  if constexpr (PV) {
#pragma unroll
    for (int u = 0; u < VU; u++)
#pragma unroll
      for (int e = 0; e < DPW; e++)
        vp[u][e] = (float)vc[(size_t)min(ch + NCH * u, L - 1) * HD + dim0 + 64 * e];
  }
  if (FUSED) {
    if (pj && (!pairv || odd)) {
      float x0, x1;
      qkv_sum(nch, pa, pb, x0, x1);
      if (jv <= GRP) {
        const float *w = qkn + (jv < GRP ? 0 : HD);
        const float eps = qkn[2 * HD];
        double ss = (double)x0 * (double)x0 + (double)x1 * (double)x1;
        ss = wave_sum_dpp_d(ss);
        const float inv = (float)(1.0 / sqrt(ss / HD + (double)eps));
        x0 = w[lane] * (x0 * inv);
        x1 = w[lane + 64] * (x1 * inv);
        const int rp = pairv ? max(pos - 1, 0) : pos;
        const float2 cs = rope_cs[(size_t)rp * (HD / 2) + lane];
        rope_pair(x0, x1, cs.x, cs.y);
      }
      if (jv < GRP) {
        qs[jv][lane] = x0;
        qs[jv][lane + 64] = x1;
      } else {
        const KV a0 = to_cache<KV>(x0), a1 = to_cache<KV>(x1);  // the cache's precision
        float *own = jv == GRP ? (pairv ? kn2 : kn) : (pairv ? vn2 : vn);
        own[lane] = (float)a0;
        own[lane + 64] = (float)a1;
        if (!pairv) {
          KV *dst = const_cast<KV *>(jv == GRP ? kc : vc) + (size_t)pos * HD;
          dst[lane] = a0;
          dst[lane + 64] = a1;
        }
      }
    }
  } else {
    for (int i = t; i < GRP * HD; i += NT)  // normed and rotated by the append kernel
      qs[i / HD][i % HD] = qkv[(size_t)m * ldq + (g * GRP + i / HD) * HD + i % HD];
  }
  __syncthreads();

  // scores: key group kg = t / 16 takes positions kg, kg + 32, ...; the loads
  // of SU positions are issued together
  const float scale = (float)(1.0 / __builtin_sqrt((double)HD));
  {
    float qv[GRP][8], kn8[8], kp8[8];
#pragma unroll
    for (int j = 0; j < GRP; j++)
#pragma unroll
      for (int e = 0; e < 8; e++) qv[j][e] = qs[j][8 * li + e];
#pragma unroll
    for (int e = 0; e < 8; e++) {
      kn8[e] = FUSED ? kn[8 * li + e] : 0.f;
      kp8[e] = PAIR ? kn2[8 * li + e] : 0.f;
    }
    for (int p0 = 0; p0 < L; p0 += KG * SU) {
      // unconditional loads from clamped positions (a guarded load would be
      // waited for on its own), then the new position's own k, zeros past L
      float k8[SU][8];
      if (p0 == 0) {
#pragma unroll
        for (int u = 0; u < SU; u++)
#pragma unroll
          for (int e = 0; e < 8; e++) k8[u][e] = k8p[u][e];
      } else {
#pragma unroll
        for (int u = 0; u < SU; u++)
          load8(kc + (size_t)min(p0 + u * KG + kg, L - 1) * HD + 8 * li, k8[u]);
      }
      // a round wholly before the row's own position needs no masks
      auto round = [&](auto masked) {
        constexpr bool MK = decltype(masked)::value;
        if constexpr (MK) {
#pragma unroll
          for (int u = 0; u < SU; u++) {
            const int p = p0 + u * KG + kg;
#pragma unroll
            for (int e = 0; e < 8; e++)
              k8[u][e] = p >= L               ? 0.f
                         : FUSED && p == pos   ? kn8[e]
                         : odd && p == pos - 1 ? kp8[e]
                                               : k8[u][e];
          }
        }
#pragma unroll
        for (int u = 0; u < SU; u++) {
          const int p = p0 + u * KG + kg;
#pragma unroll
          for (int j = 0; j < GRP; j++) {
            float a = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) a = fmaf(qv[j][e], k8[u][e], a);
            a = row16_tree(a);
            if ((!MK || p < L) && li == 0) sc[j * L + p] = __fmul_rn(a, scale);
          }
        }
      };
      if (LONG && p0 + KG * SU <= clean)
        round(std::false_type{});
      else
        round(std::true_type{});
    }
  }
  __syncthreads();

  // softmax per head
  float inv[GRP], ew[GRP];
  if constexpr (!LONG) {
    // the one-round shape (covers of at most 32 positions): one wave holds a
    // head's scores, one per lane, so every wave takes the maximum, the
    // exponentials and the double sum itself (no barrier, no LDS trip) and
    // keeps its lane's exponential for the value weights
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      const float sv = lane < L ? sc[j * L + lane] : -INFINITY;
      const float mx = wave_max_dpp(sv);
      ew[j] = lane < L ? exp_ieee(__fsub_rn(sv, mx)) : 0.f;
      inv[j] = (float)(1.0 / wave_sum_dpp_d((double)ew[j]));
    }
  } else {
#pragma unroll
    for (int j = 0; j < GRP; j++) ew[j] = 0.f;
    float mx[GRP];
#pragma unroll
    for (int j = 0; j < GRP; j++) mx[j] = -INFINITY;
    for (int p = t; p < L; p += NT)
#pragma unroll
      for (int j = 0; j < GRP; j++) mx[j] = fmaxf(mx[j], sc[j * L + p]);
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      mx[j] = wave_max_dpp(mx[j]);
      if (lane == 0) redf[j][wave] = mx[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      float v = redf[j][0];
#pragma unroll
      for (int w = 1; w < NWV; w++) v = fmaxf(v, redf[j][w]);
      mx[j] = v;
    }
    double sum[GRP];
#pragma unroll
    for (int j = 0; j < GRP; j++) sum[j] = 0.0;
    for (int p = t; p < L; p += NT)
#pragma unroll
      for (int j = 0; j < GRP; j++) {
        const float e = exp_ieee(__fsub_rn(sc[j * L + p], mx[j]));
        sc[j * L + p] = e;
        sum[j] += (double)e;
      }
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      sum[j] = wave_sum_dpp_d(sum[j]);
      if (lane == 0) redd[j][wave] = sum[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      double s2 = 0.0;
#pragma unroll
      for (int w = 0; w < NWV; w++) s2 += redd[j][w];
      inv[j] = (float)(1.0 / s2);
    }
  }

  // values: chain ch = wave % 8 over positions p = ch mod 8, dims dim0 + 64 e,
  // every head of the group; the loads of VU positions issued together
  {
    float c[DPW][GRP];
#pragma unroll
    for (int e = 0; e < DPW; e++)
#pragma unroll
      for (int j = 0; j < GRP; j++) c[e][j] = 0.f;
    float vnd[DPW], vpd[DPW];
#pragma unroll
    for (int e = 0; e < DPW; e++) {
      vnd[e] = FUSED ? vn[dim0 + 64 * e] : 0.f;
      vpd[e] = PAIR ? vn2[dim0 + 64 * e] : 0.f;
    }
    for (int p0 = ch; p0 < L; p0 += NCH * VU) {
      float v[VU][DPW];
      if (PV && p0 == ch) {
#pragma unroll
        for (int u = 0; u < VU; u++)
#pragma unroll
          for (int e = 0; e < DPW; e++) v[u][e] = vp[PV ? u : 0][e];
      } else {
#pragma unroll
        for (int u = 0; u < VU; u++)
#pragma unroll
          for (int e = 0; e < DPW; e++)
            v[u][e] = (float)vc[(size_t)min(p0 + NCH * u, L - 1) * HD + dim0 + 64 * e];
      }
      // the new position: its own v; past L: zero (the clamped load may have
      // read the new row before it was written); weights of the round read
      // together, past L a zero weight times a zero value adds an exact zero to
      // the chain. A round wholly before the row's own position needs no masks.
      auto round = [&](auto masked) {
        constexpr bool MK = decltype(masked)::value;
        if constexpr (MK) {
#pragma unroll
          for (int u = 0; u < VU; u++) {
            const int p = p0 + NCH * u;
#pragma unroll
            for (int e = 0; e < DPW; e++)
              v[u][e] = p >= L               ? 0.f
                        : FUSED && p == pos   ? vnd[e]
                        : odd && p == pos - 1 ? vpd[e]
                                              : v[u][e];
          }
        }
        float wgt[VU][GRP];
#pragma unroll
        for (int u = 0; u < VU; u++) {
          const int p = p0 + NCH * u;  // the same for the whole wave
#pragma unroll
          for (int j = 0; j < GRP; j++) {
            const float e = LONG ? sc[j * L + (MK ? min(p, L - 1) : p)] : lane_f(ew[j], min(p, L - 1));
            wgt[u][j] = !MK || p < L ? __fmul_rn(e, inv[j]) : 0.f;
          }
        }
#pragma unroll
        for (int u = 0; u < VU; u++)
#pragma unroll
          for (int j = 0; j < GRP; j++)
#pragma unroll
            for (int e = 0; e < DPW; e++) c[e][j] = fmaf(wgt[u][j], v[u][e], c[e][j]);
      };
      if (LONG && p0 + NCH * (VU - 1) < clean)
        round(std::false_type{});
      else
        round(std::true_type{});
    }
#pragma unroll
    for (int j = 0; j < GRP; j++)
#pragma unroll
      for (int e = 0; e < DPW; e++) cv[ch][j][dim0 + 64 * e] = c[e][j];
  }
  __syncthreads();

  // quantize each head's 128 outputs per 32-block (a 32-lane half-wave each)
  for (int i = t; i < GRP * HD; i += NT) {
    const int j = i / HD, k = i % HD, h = g * GRP + j;
    const float o = __fadd_rn(
        __fadd_rn(__fadd_rn(cv[0][j][k], cv[1][j][k]), __fadd_rn(cv[2][j][k], cv[3][j][k])),
        __fadd_rn(__fadd_rn(cv[4][j][k], cv[5][j][k]), __fadd_rn(cv[6][j][k], cv[7][j][k])));
    float amax = fabsf(o);
    amax = half_max_dpp(amax);
    const float dq = __fdiv_rn(amax, 127.0f);
    const float id = dq != 0.f ? __fdiv_rn(1.0f, dq) : 0.f;
    xq[qoff(h, k)] = (int8_t)(int)roundf(__fmul_rn(o, id));
    if ((k & 31) == 0) dx[(size_t)m * nbq + 4 * h + (k >> 5)] = (float)(_Float16)dq;
  }
}

}  // namespace

bool attn_x_supported(int heads, int kvh, int head_dim, int max_positions) {
  return head_dim == HD && kvh > 0 && heads % kvh == 0 &&
         (heads / kvh == 1 || heads / kvh == 2 || heads / kvh == 4) && max_positions > 0 &&
         (size_t)max_positions * (heads / kvh) <= (size_t)kAttnXMaxPositions;
}

template <typename KV, bool F, int SU, int VU, int NT, bool PV, bool PAIR = false>
void attn_x_grp(const AttnArgs &a, int M, int nch, const QAct &xa, int max_positions,
                hipStream_t st) {
  const dim3 grid(a.kvh, M);
  const int grp = a.heads / a.kvh;
  // the kernel takes the q/k/v row stride as (heads + 2 kv heads) * 128, so
  // that its arguments fit the 14 dwords preloaded in SGPRs (the grid size,
  // a hidden argument past them, would be a dependent load before the first)
  require(a.ldq == (a.heads + 2 * a.kvh) * HD, Q3H_E_ARG, "attention: q/k/v rows not packed");
  const size_t lds = sizeof(float) * (size_t)grp * max_positions;
#define Q3H_ATTNX(G)                                                                         \
  hipLaunchKernelGGL((k_attn_x<KV, F, G, SU, VU, NT, PV, PAIR>), grid, dim3(NT), lds, st, a.rd, \
                     a.qkv, a.qkn, a.rope_cs, xa.q, a.layer, nch, a.kvh, M)
  if (grp == 1)
    Q3H_ATTNX(1);
  else if (grp == 2)
    Q3H_ATTNX(2);
  else
    Q3H_ATTNX(4);
#undef Q3H_ATTNX
}

// short contexts (the code predictor's 16 positions): one round of each loop;
// decode rows over longer contexts: 128 keys and 64 values per round, the
// first values loaded with the keys (the loads of a round come from clamped
// positions, so deeper rounds cost a short context their full width: 1024
// threads with 512 keys and 128 values per round measured 2.5 us slower per
// talker layer over 32 ragged contexts); prefill rows 256 keys and 128 values
// per round. Results do not depend on the thread count or the round depths.
template <typename KV, bool F>
void attn_x_len(const AttnArgs &a, int M, int nch, const QAct &xa, int max_positions,
                bool pairs, hipStream_t st) {
  if (F && pairs)  // the short shape only (attn_x_pairs_supported)
    attn_x_grp<KV, F, 1, 4, 512, true, true>(a, M, nch, xa, max_positions, st);
  else if (max_positions <= 32)
    attn_x_grp<KV, F, 1, 4, 512, true>(a, M, nch, xa, max_positions, st);
  else if constexpr (F)
    attn_x_grp<KV, F, 4, 8, 512, true>(a, M, nch, xa, max_positions, st);
  else
    attn_x_grp<KV, F, 8, 16, 512, false>(a, M, nch, xa, max_positions, st);
}

bool attn_x_pairs_supported(int max_positions) { return max_positions <= 32; }

void launch_attn_x(const AttnArgs &a, int M, bool fused, bool kv16, int qkv_chunks,
                   const QAct &xa, int max_positions, hipStream_t st, bool pairs) {
  const int nch = fused ? qkv_chunks : 0;
  require(!pairs || (fused && M % 2 == 0 && attn_x_pairs_supported(max_positions)), Q3H_E_ARG,
          "attention: row pairs need the fused short-context shape and an even row count");
  if (kv16) {
    if (fused)
      attn_x_len<_Float16, true>(a, M, nch, xa, max_positions, pairs, st);
    else
      attn_x_len<_Float16, false>(a, M, nch, xa, max_positions, false, st);
  } else {
    if (fused)
      attn_x_len<float, true>(a, M, nch, xa, max_positions, pairs, st);
    else
      attn_x_len<float, false>(a, M, nch, xa, max_positions, false, st);
  }
}

}  // namespace q3h
