// q3h_sample.h - the draw of a code from logits on the device (temperature,
// top-k, top-p, then one uniform through the inverse distribution), as the
// logits warpers of Hugging Face generate() apply them in the order the
// reference names (talker.pas:599-601: "temperature, top-k, top-p and the
// draw"). Every floating-point step has a fixed order, so a CPU evaluation of
// the same definition (the oracle) picks the same code from the same logits
// and the same uniform.
//
// The uniform: Philox4x64-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC 2011) of a counter (frame, group, 0, 0)
// under a key (seed, 0); u = (first 64-bit output >> 40) * 2^-24, in [0, 1).
//
// The draw over n <= 1024 * NPT values, thread t of a 1024-thread block
// holding the NPT values of indices t NPT .. t NPT + NPT - 1:
//  1. v = x / T (fp32 division; x as is when T == 1);
//  2. top-k (1 <= k < n): keep v >= the k-th largest v (ties at it kept, as
//     TopKLogitsWarper does), found by a radix select on order-preserving
//     32-bit keys;
//  3. M = the largest kept v;
//  4. top-p (p < 1, with 1 <= k <= 64 and at most 64 values kept by top-k):
//     the kept values in ascending (key, descending index) order, w = e^(v - M)
//     (exp_ieee), S = their sum in that order, then from the smallest up
//     c += w / S; a value is removed while c <= 1 - p; the largest is always
//     kept (TopPLogitsWarper);
//  5. w_i = e^(v_i - M) for kept values, 0 otherwise; A_t = the sum of
//     thread t's w in index order; B_s = the sum of A_t over t = 16 s ..
//     16 s + 15 in order; S = the sum of B_0 .. B_63 in order; target = u S;
//     the walk: the first segment s with r + B_s > target (r the sum of the
//     segments before, accumulated in order), in it the first thread, in it
//     the first index; when a level finds none (rounding at the top end), the
//     last index with w > 0 in the range of that level;
//  6. when that finds no index either (every w is 0 or NaN, which only NaN or
//     infinite scores cause), the greedy code of x: its first maximum, NaN
//     never winning, 0 when x[0] is NaN or nothing is a maximum
//     (first_max_code), so the result is always an index of the table.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "q3h_math.h"
#include "q3h_wave.h"

namespace q3h {

// sampling parameters of one chooser (the talker's code 0 or the code
// predictor's codes), as TQwenSampling holds them (talker.pas:60-70)
struct SampleParams {
  int do_sample;      // 0: argmax (greedy)
  float temperature;  // > 0
  int top_k;          // 0: off
  float top_p;        // 1: off
};

constexpr uint64_t kSubSeedXor = 0x5DEECE66Dull;  // the sub-sampler's seed (talker.pas:585)

__device__ __forceinline__ void philox4x64_10(uint64_t c[4], uint64_t k0, uint64_t k1) {
#pragma unroll
  for (int r = 0; r < 10; r++) {
    const uint64_t lo0 = 0xD2E7470EE14C6C93ull * c[0], hi0 = __umul64hi(0xD2E7470EE14C6C93ull, c[0]);
    const uint64_t lo1 = 0xCA5A826395121157ull * c[2], hi1 = __umul64hi(0xCA5A826395121157ull, c[2]);
    const uint64_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
    k0 += 0x9E3779B97F4A7C15ull;
    k1 += 0xBB67AE8584CAA73Bull;
  }
}

// the uniform of draw (frame, group) under seed
__device__ __forceinline__ float draw_uniform(uint64_t seed, uint64_t frame, uint64_t group) {
  uint64_t c[4] = {frame, group, 0, 0};
  philox4x64_10(c, seed, 0);
  return (float)(uint32_t)(c[0] >> 40) * 0x1p-24f;
}

// order-preserving key of a float (larger float, larger key)
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

constexpr int kSampleThreads = 1024;
constexpr int kSampleMaxNPT = 3;  // up to 3072 values

struct SampleShared {
  alignas(16) int hist[2][512];  // the radix passes alternate between the two
  uint32_t prefix, remaining;
  int exact;  // the selected bucket holds exactly the values still wanted
  float fred[kSampleThreads / 64];
  int cnt;
  uint32_t ck[64];
  int ci[64];
  float cv[64];
  uint32_t th_key;
  int th_idx;
  alignas(16) float A[kSampleThreads];
  alignas(16) float B[64];
  alignas(16) float P[64];   // B_0 + .. + B_q, in order
  alignas(16) float P2[16];  // the same over one segment's A_t
  float W[kSampleThreads * kSampleMaxNPT];
  int pick;
  int fidx[kSampleThreads / 64];
};

// the last index in [lo, hi) with W > 0 (-1: none), over one wave
__device__ __forceinline__ int last_positive(const float *W, int lo, int hi) {
  const int lane = threadIdx.x & 63;
  int best = -1;
  for (int i = lo + lane; i < hi; i += 64)
    if (W[i] > 0.0f) best = i;
  for (int off = 32; off >= 1; off >>= 1) best = max(best, __shfl_xor(best, off, 64));
  return best;
}

// The code drawn from x (this thread's NPT values, indices t NPT + j; n
// values in all, the rest ignored) with parameters p and uniform u. A block
// of kSampleThreads threads; every thread returns the code.
template <int NPT>
__device__ int block_sample(const float (&x)[NPT], int n, const SampleParams &p, float u,
                            SampleShared &sh) {
  static_assert(NPT <= kSampleMaxNPT, "at most 3 values per thread");
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int base = t * NPT;
  float v[NPT];
  uint32_t key[NPT];
  bool kept[NPT];
#pragma unroll
  for (int j = 0; j < NPT; j++) {
    const bool in = base + j < n;
    const float a = in ? x[j] : -__builtin_inff();
    v[j] = p.temperature == 1.0f ? a : __fdiv_rn(a, p.temperature);
    key[j] = order_key(v[j]);
    kept[j] = in;
  }
  // 2. top-k: the k-th largest key by a radix select, 9 bits per pass (the
  // first pass buckets by sign and exponent), 5 in the last. A pass
  // whose selected bucket holds exactly the values still wanted ends the
  // select: every key of that bucket is kept, so the bucket's lowest key (the
  // prefix with zero low bits) keeps the same set as the exact k-th key.
  const bool topk = p.top_k >= 1 && p.top_k < n;
  if (topk) {
    if (t == 0) {
      sh.prefix = 0;
      sh.remaining = (uint32_t)p.top_k;
      sh.exact = 0;
    }
    for (int b = t; b < 1024; b += kSampleThreads) sh.hist[b >> 9][b & 511] = 0;
    __syncthreads();
    for (int pass = 0; pass < 4; pass++) {
      const int width = pass < 3 ? 9 : 5, shift = 32 - 9 * pass - width;
      const uint32_t hmask = pass == 0 ? 0u : (0xFFFFFFFFu << (shift + width));
      int *hist = sh.hist[pass & 1];
      const uint32_t prefix = sh.prefix;
#pragma unroll
      for (int j = 0; j < NPT; j++)
        if (kept[j] && (key[j] & hmask) == prefix)
          atomicAdd(&hist[(key[j] >> shift) & ((1u << width) - 1)], 1);
      __syncthreads();
      if (wave == 1) {  // the other buffer, for the next pass
        int *nxt = sh.hist[(pass + 1) & 1];
        for (int b = lane; b < 512; b += 64) nxt[b] = 0;
      }
      if (wave == 0) {
        // lane l: buckets 8 (63 - l) .. + 7 (larger buckets in smaller lanes)
        const int4 ha = reinterpret_cast<const int4 *>(hist)[2 * (63 - lane)];
        const int4 hb = reinterpret_cast<const int4 *>(hist)[2 * (63 - lane) + 1];
        const int h[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
        int mine = 0;
#pragma unroll
        for (int q = 0; q < 8; q++) mine += h[q];
        const int above = wave_prefix_sum_i(mine) - mine;
        const uint32_t rem = sh.remaining;
        if ((uint32_t)above < rem && rem <= (uint32_t)(above + mine)) {
          int acc = above, d = 8 * (63 - lane);
          int hd = 0;
          for (int q = 7; q >= 0; q--) {
            if ((uint32_t)(acc + h[q]) >= rem) {
              d = 8 * (63 - lane) + q;
              hd = h[q];
              break;
            }
            acc += h[q];
          }
          sh.prefix = prefix | ((uint32_t)d << shift);
          sh.remaining = rem - (uint32_t)acc;
          sh.exact = (uint32_t)hd == rem - (uint32_t)acc;
        }
      }
      __syncthreads();
      if (sh.exact) break;  // uniform
    }
    const uint32_t tau = sh.prefix;
#pragma unroll
    for (int j = 0; j < NPT; j++) kept[j] = kept[j] && key[j] >= tau;
  }
  // 3. M
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < NPT; j++)
    if (kept[j]) m = fmaxf(m, v[j]);
  m = wave_max_dpp(m);
  if (lane == 0) sh.fred[wave] = m;
  __syncthreads();
  m = sh.fred[0];
  for (int q = 1; q < kSampleThreads / 64; q++) m = fmaxf(m, sh.fred[q]);
  // 4. top-p over at most 64 values
  if (p.top_p < 1.0f && topk && p.top_k <= 64) {
    if (t == 0) sh.cnt = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NPT; j++)
      if (kept[j]) {
        const int slot = atomicAdd(&sh.cnt, 1);
        if (slot < 64) {
          sh.ck[slot] = key[j];
          sh.ci[slot] = base + j;
          sh.cv[slot] = v[j];
        }
      }
    __syncthreads();
    const int cnt = sh.cnt;
    if (cnt <= 64) {
      if (wave == 0) {
        // bitonic sort into descending (key, then ascending index); empty slots last
        uint32_t k = lane < cnt ? sh.ck[lane] : 0u;
        int ix = lane < cnt ? sh.ci[lane] : 0x7fffffff;
        float vv = lane < cnt ? sh.cv[lane] : -__builtin_inff();
        for (int size = 2; size <= 64; size <<= 1)
          for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint32_t ok = __shfl_xor(k, stride, 64);
            const int oi = __shfl_xor(ix, stride, 64);
            const float ov = __shfl_xor(vv, stride, 64);
            const bool lower = (lane & stride) == 0;
            const bool desc = (lane & size) == 0;
            const bool mine_first = k > ok || (k == ok && ix < oi);
            const bool keep_mine = (lower == desc) ? mine_first : !mine_first;
            if (!keep_mine) {
              k = ok;
              ix = oi;
              vv = ov;
            }
          }
        // lane 0 holds the largest; the ascending order is lanes cnt - 1 .. 0
        const float w = lane < cnt ? exp_ieee(__fsub_rn(vv, m)) : 0.0f;
        float S = 0.0f;
        for (int q = cnt - 1; q >= 0; q--) S = __fadd_rn(S, lane_f(w, q));
        const float lim = __fsub_rn(1.0f, p.top_p);
        float c = 0.0f;
        int last = 0;  // lanes 0 .. last stay
        for (int q = cnt - 1; q >= 1; q--) {
          c = __fadd_rn(c, __fdiv_rn(lane_f(w, q), S));
          if (c > lim) {
            last = q;
            break;
          }
        }
        if (lane == last) {
          sh.th_key = k;
          sh.th_idx = ix;
        }
      }
      __syncthreads();
      const uint32_t tk = sh.th_key;
      const int ti = sh.th_idx;
#pragma unroll
      for (int j = 0; j < NPT; j++)
        kept[j] = kept[j] && (key[j] > tk || (key[j] == tk && base + j <= ti));
    }
  }
  // 5. the draw. B_s is summed in lane 16 s of its row from the row's A_t
  // (DPP row shifts, in order); wave 0 runs the chain of the segment sums in
  // registers and writes the running sums once, lane q reading the sum
  // through segment q, so the first segment whose running sum passes the
  // target is a ballot (the same sums and comparisons as a walk over the
  // segments); the same over the threads of that segment
  float a = 0.0f;
#pragma unroll
  for (int j = 0; j < NPT; j++) {
    const float w = kept[j] ? exp_ieee(__fsub_rn(v[j], m)) : 0.0f;
    sh.W[base + j] = w;
    a = __fadd_rn(a, w);
  }
  sh.A[t] = a;
  float b = a;
  b = __fadd_rn(b, row_shl_f<1>(a));
  b = __fadd_rn(b, row_shl_f<2>(a));
  b = __fadd_rn(b, row_shl_f<3>(a));
  b = __fadd_rn(b, row_shl_f<4>(a));
  b = __fadd_rn(b, row_shl_f<5>(a));
  b = __fadd_rn(b, row_shl_f<6>(a));
  b = __fadd_rn(b, row_shl_f<7>(a));
  b = __fadd_rn(b, row_shl_f<8>(a));
  b = __fadd_rn(b, row_shl_f<9>(a));
  b = __fadd_rn(b, row_shl_f<10>(a));
  b = __fadd_rn(b, row_shl_f<11>(a));
  b = __fadd_rn(b, row_shl_f<12>(a));
  b = __fadd_rn(b, row_shl_f<13>(a));
  b = __fadd_rn(b, row_shl_f<14>(a));
  b = __fadd_rn(b, row_shl_f<15>(a));
  if ((lane & 15) == 0) sh.B[t >> 4] = b;
  __syncthreads();
  if (wave == 0) {
    float bq[64];
#pragma unroll
    for (int q = 0; q < 16; q++) {
      const float4 f = reinterpret_cast<const float4 *>(sh.B)[q];
      bq[4 * q] = f.x, bq[4 * q + 1] = f.y, bq[4 * q + 2] = f.z, bq[4 * q + 3] = f.w;
    }
    float r = 0.0f;
#pragma unroll
    for (int q = 0; q < 64; q++) {
      r = __fadd_rn(r, bq[q]);
      bq[q] = r;
    }
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < 16; q++)
        reinterpret_cast<float4 *>(sh.P)[q] = make_float4(bq[4 * q], bq[4 * q + 1], bq[4 * q + 2], bq[4 * q + 3]);
    }
    __builtin_amdgcn_wave_barrier();
    const float mine = sh.P[lane];
    const float target = __fmul_rn(u, r);
    const unsigned long long hit = __ballot(mine > target);
    int pick;
    if (hit == 0) {
      pick = last_positive(sh.W, 0, kSampleThreads * NPT);
    } else {
      const int seg = __ffsll((long long)hit) - 1;
      const float r0 = seg == 0 ? 0.0f : lane_f(mine, seg - 1);  // the sum before seg
      float aq[16];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 f = reinterpret_cast<const float4 *>(sh.A + 16 * seg)[q];
        aq[4 * q] = f.x, aq[4 * q + 1] = f.y, aq[4 * q + 2] = f.z, aq[4 * q + 3] = f.w;
      }
      float rr = r0;
#pragma unroll
      for (int q = 0; q < 16; q++) {
        rr = __fadd_rn(rr, aq[q]);
        aq[q] = rr;
      }
      if (lane == 0) {
#pragma unroll
        for (int q = 0; q < 4; q++)
          reinterpret_cast<float4 *>(sh.P2)[q] = make_float4(aq[4 * q], aq[4 * q + 1], aq[4 * q + 2], aq[4 * q + 3]);
      }
      __builtin_amdgcn_wave_barrier();
      const float mine2 = sh.P2[lane & 15];
      const unsigned long long hit2 = __ballot(lane < 16 && mine2 > target);
      if (hit2 == 0) {
        pick = last_positive(sh.W, 16 * seg * NPT, 16 * (seg + 1) * NPT);
      } else {
        const int tq = __ffsll((long long)hit2) - 1, th = 16 * seg + tq;
        float r1 = tq == 0 ? r0 : lane_f(mine2, tq - 1);
        pick = -1;
        for (int j = 0; j < NPT; j++) {
          const float wj = sh.W[th * NPT + j];
          if (__fadd_rn(r1, wj) > target) {
            pick = th * NPT + j;
            break;
          }
          r1 = __fadd_rn(r1, wj);
        }
        if (pick < 0) pick = last_positive(sh.W, th * NPT, th * NPT + NPT);
      }
    }
    if (lane == 0) sh.pick = pick;
  }
  __syncthreads();
  int code = sh.pick;
  if (code < 0) {
    // 6. no code drawn (every weight 0 or NaN: NaN or infinite scores): the
    // greedy choice over x, first_max_code's rule (uniform branch)
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < NPT; j++)
      if (base + j < n) argmax_merge(bv, bi, x[j], base + j);
    for (int off = 32; off >= 1; off >>= 1) {
      const float v2 = __shfl_xor(bv, off, 64);
      const int i2 = __shfl_xor(bi, off, 64);
      argmax_merge(bv, bi, v2, i2);
    }
    __syncthreads();
    if (lane == 0) {
      sh.fred[wave] = bv;
      sh.fidx[wave] = bi;
    }
    if (t == 0) sh.cv[0] = x[0];  // thread 0 holds index 0
    __syncthreads();
    bv = sh.fred[0];
    bi = sh.fidx[0];
    for (int q = 1; q < kSampleThreads / 64; q++) argmax_merge(bv, bi, sh.fred[q], sh.fidx[q]);
    code = first_max_code(bi, sh.cv[0]);
  }
  __syncthreads();  // the shared state is reused by the next call
  return code;
}

}  // namespace q3h
