// q3h_codec.hip - the back part of the Qwen3-TTS 12 Hz decoder on the device
// (TQwenCodec.Back, src/tts/mormot.ai.tts.qwen.codec.pas:1040-1083, the pass
// TQwenCodecVulkan records, codec.vulkan.pas:568-652): two upsampling stages
// (transposed convolution 2 / 2, ConvNeXt), the input convolution, four
// blocks (SnakeBeta, transposed convolution of rate 8 / 5 / 4 / 3, three
// residual units of dilations 1 / 3 / 9), SnakeBeta, the output convolution
// and the clamp: 1920 samples per frame, ~2.4 GMAC.
//
// Every convolution (transposed ones included, rewritten as causal
// convolutions of taps K / stride whose stride x out output columns are the
// stride output rows) is one f32 matrix-core product over an implicit
// im2col: output row t reads input rows t + k dil, k < taps, of a sequence
// buffer that holds the `past` history rows of the previous call on top of
// the new rows (TQwenVkSeq, codec.vulkan.pas:33-40). A workgroup owns 64
// output rows x 16 WN output columns and walks the whole K = taps x Cin in
// 32-column chunks (activations through double-buffered LDS, weights in
// registers one chunk ahead): the order of every sum depends only on the
// layer, not on the rows of the call, so decoding 1 + 3 frames or 4 at once
// gives the same samples (the reference's property, codec.vulkan.pas:12-13).
//
// The elementwise steps ride in the products' epilogues: bias, GELU (erf),
// the residual add, the ConvNeXt layer scale, and SnakeBeta of the output
// written as the input of the next convolution (at its history offset). The
// depthwise convolution + LayerNorm of ConvNeXt is one kernel per row; the
// output convolution (96 -> 1) + clamp one thread per sample. At the end of a
// pass one kernel moves every sequence's last rows to its history.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "q3h_api_internal.h"

namespace q3h {
namespace {

constexpr int kLatent = 1024, kDecDim = 1536, kFrameSamples = 1920;
constexpr int kRates[4] = {8, 5, 4, 3};
constexpr int kDils[3] = {1, 3, 9};

enum ConvEpi { CE_BIAS = 0, CE_GELU = 1, CE_RES = 2, CE_SCALED_RES = 3 };

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld4(const float *p) { return *reinterpret_cast<const float4 *>(p); }

struct ConvArgs {
  const float *x;  // sequence buffer [past + T][cin] (history rows first)
  const float *w;  // [n][taps cin], column k cin + c
  const float *b;  // [n]
  float *y;        // [T][n] or null
  const float *r;  // residual [T][n] (CE_RES, CE_SCALED_RES)
  const float *g;  // layer scale [n] (CE_SCALED_RES)
  float *z;        // SnakeBeta of the output [T][n] or null
  const float *sa, *sib;  // e^alpha, 1 / (e^beta + 1e-9), indexed by column % sc
  float *part;            // K-slice sums [gridDim.z][T][n] when the K walk is split
  int cin, taps, dil, T, n, sc;
};

// chunks of 32 K columns per K slice: a product whose K walk is longer runs
// as ceil(chunks / kSliceChunks) slices, summed in slice order by
// k_conv_reduce (a fixed split per layer: the sums do not depend on T)
constexpr int kSliceChunks = 16;
constexpr int kRingWorkgroups = 512;  // launches up to this size take k_conv_gemm_ring

// the epilogue of one output: bias, GELU / residual / layer scale, then the
// stores (y, and SnakeBeta of the value to z)
template <int EPI>
__device__ __forceinline__ void conv_out(const ConvArgs &a, int m, int n, float acc) {
  const size_t o = (size_t)m * a.n + n;
  float v = acc + a.b[n];
  if (EPI == CE_GELU) v = 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
  if (EPI == CE_RES) v = a.r[o] + v;
  if (EPI == CE_SCALED_RES) v = a.r[o] + a.g[n] * v;
  if (a.y) a.y[o] = v;
  if (a.z) {
    const int sc = n % a.sc;
    const float s = sinf(v * a.sa[sc]);
    a.z[o] = v + a.sib[sc] * (s * s);
  }
}

// one workgroup: output rows m0 .. m0 + 16 TM - 1, columns n0 .. n0 + 16 WN
// - 1 (the row tile follows T; every output's sum has the same order in any
// tile: a sum of the same MFMAs over the same chunks)
template <int WN, int TM, int EPI>
__global__ __launch_bounds__(64 * WN) void k_conv_gemm(ConvArgs a) {
  constexpr int NT = 64 * WN, XS = 36, MR = 16 * TM;
  constexpr int NF4 = MR * 32 / 4;                  // float4 of an activation chunk
  constexpr int XF4 = NF4 >= NT ? NF4 / NT : 1;     // per thread
  __shared__ float xs[2][MR * XS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * WN + 16 * wave, m0 = blockIdx.y * MR;
  const int K = a.taps * a.cin, cpk = a.cin / 32;
  const int q0 = blockIdx.z * kSliceChunks, q1 = min(a.taps * cpk, q0 + kSliceChunks);
  const float *wr = a.w + (size_t)min(n0 + r, a.n - 1) * K + 4 * g;
  int xrow[XF4], xcol[XF4], xo[XF4];
  const bool xact = NF4 >= NT || t < NF4;  // threads that move activations
#pragma unroll
  for (int i = 0; i < XF4; i++) {
    const int f = min(t + NT * i, NF4 - 1), row = f >> 3, c4 = f & 7;
    xrow[i] = min(m0 + row, a.T - 1);
    xcol[i] = 4 * c4;
    xo[i] = row * XS + 4 * c4;
  }
  float4 xn[XF4], wn[2], wc[2];
  auto load = [&](int q) {
    const int k = q / cpk, c0 = (q - k * cpk) * 32;
#pragma unroll
    for (int i = 0; i < XF4; i++)
      xn[i] = ld4(a.x + (size_t)(xrow[i] + k * a.dil) * a.cin + c0 + xcol[i]);
    wn[0] = ld4(wr + 32 * q);
    wn[1] = ld4(wr + 32 * q + 16);
  };
  v4f acc[TM];
#pragma unroll
  for (int i = 0; i < TM; i++) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
  load(q0);
  if (xact)
#pragma unroll
    for (int i = 0; i < XF4; i++) *reinterpret_cast<float4 *>(&xs[0][xo[i]]) = xn[i];
  wc[0] = wn[0];
  wc[1] = wn[1];
  __syncthreads();
  for (int q = q0; q < q1; q++) {
    const int b = (q - q0) & 1;
    if (q + 1 < q1) load(q + 1);
#pragma unroll
    for (int s = 0; s < 2; s++) {
#pragma unroll
      for (int tm = 0; tm < TM; tm++) {
        const float4 xa = *reinterpret_cast<const float4 *>(&xs[b][(16 * tm + r) * XS + 16 * s + 4 * g]);
        acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.x, wc[s].x, acc[tm], 0, 0, 0);
        acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.y, wc[s].y, acc[tm], 0, 0, 0);
        acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.z, wc[s].z, acc[tm], 0, 0, 0);
        acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.w, wc[s].w, acc[tm], 0, 0, 0);
      }
    }
    if (q + 1 < q1) {
      if (xact)
#pragma unroll
        for (int i = 0; i < XF4; i++) *reinterpret_cast<float4 *>(&xs[b ^ 1][xo[i]]) = xn[i];
      wc[0] = wn[0];
      wc[1] = wn[1];
    }
    __syncthreads();
  }
  // lane l holds (m = m0 + 16 tm + 4 g + q, n = n0 + r)
  const int n = n0 + r;
  if (n >= a.n) return;
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int m = m0 + 16 * tm + 4 * g + q;
      if (m >= a.T) continue;
      if (gridDim.z > 1)
        a.part[((size_t)blockIdx.z * a.T + m) * a.n + n] = acc[tm][q];
      else
        conv_out<EPI>(a, m, n, acc[tm][q]);
    }
}

// k_conv_gemm for launches of few workgroups (a frame per call), where the
// serial K walk is the time: the same tile and sums, the chunks of the slice
// walked with the loads of D chunks in flight (a register ring,
// the loop unrolled over the kSliceChunks chunks a slice can hold, loads at
// clamped chunk indices so that none sits behind a branch); chunk i's
// activations go through LDS buffer i & 1. The operands the loads need come
// as plain arguments (preloaded in SGPRs); the epilogue's in a.
template <int WN, int TM, int EPI>
__global__ __launch_bounds__(64 * WN) void k_conv_gemm_ring(const float *__restrict__ x,
                                                       const float *__restrict__ w, int cin,
                                                       int taps, int dil, int T, int n,
                                                       ConvArgs a) {
  constexpr int NT = 64 * WN, XS = 36, MR = 16 * TM, D = 4;
  constexpr int NF4 = MR * 32 / 4;                  // float4 of an activation chunk
  constexpr int XF4 = NF4 >= NT ? NF4 / NT : 1;     // per thread
  __shared__ float xs[2][MR * XS];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * WN + 16 * wave, m0 = blockIdx.y * MR;
  const int K = taps * cin, cpk = cin / 32;
  const int q0 = blockIdx.z * kSliceChunks, nq = min(taps * cpk - q0, kSliceChunks);
  const float *wr = w + (size_t)min(n0 + r, n - 1) * K + 4 * g;
  int xrow[XF4], xcol[XF4], xo[XF4];
  const bool xact = NF4 >= NT || t < NF4;  // threads that move activations
#pragma unroll
  for (int i = 0; i < XF4; i++) {
    const int f = min(t + NT * i, NF4 - 1), row = f >> 3, c4 = f & 7;
    xrow[i] = min(m0 + row, T - 1);
    xcol[i] = 4 * c4;
    xo[i] = row * XS + 4 * c4;
  }
  float4 xn[D][XF4], wn[D][2];
  // chunk q0 + i (clamped to the slice's last) into ring slot i % D
  auto load = [&](int i) {
    const int q = q0 + min(i, nq - 1), k = q / cpk, c0 = (q - k * cpk) * 32, sl = i % D;
#pragma unroll
    for (int j = 0; j < XF4; j++)
      xn[sl][j] = ld4(x + (size_t)(xrow[j] + k * dil) * cin + c0 + xcol[j]);
    wn[sl][0] = ld4(wr + 32 * q);
    wn[sl][1] = ld4(wr + 32 * q + 16);
  };
  v4f acc[TM];
#pragma unroll
  for (int i = 0; i < TM; i++) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < D; i++) load(i);
  if (xact)
#pragma unroll
    for (int j = 0; j < XF4; j++) *reinterpret_cast<float4 *>(&xs[0][xo[j]]) = xn[0][j];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSliceChunks; i++) {
    const int b = i & 1, sl = i % D, sn = (i + 1) % D;
    const float4 wc[2] = {wn[sl][0], wn[sl][1]};
    // chunk i + 1's activations to the other buffer, then chunk i + D's loads
    // into the slot chunk i leaves
    if (xact)
#pragma unroll
      for (int j = 0; j < XF4; j++) *reinterpret_cast<float4 *>(&xs[b ^ 1][xo[j]]) = xn[sn][j];
    load(i + D);
    if (i < nq) {
      // the chunk's activation operands read from LDS before the MFMAs
      float4 xa[2][TM];
#pragma unroll
      for (int s = 0; s < 2; s++)
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
          xa[s][tm] =
              *reinterpret_cast<const float4 *>(&xs[b][(16 * tm + r) * XS + 16 * s + 4 * g]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < 2; s++) {
#pragma unroll
        for (int tm = 0; tm < TM; tm++) {
          acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[s][tm].x, wc[s].x, acc[tm], 0, 0, 0);
          acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[s][tm].y, wc[s].y, acc[tm], 0, 0, 0);
          acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[s][tm].z, wc[s].z, acc[tm], 0, 0, 0);
          acc[tm] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[s][tm].w, wc[s].w, acc[tm], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }
  // lane l holds (m = m0 + 16 tm + 4 g + q, n = n0 + r)
  const int nc = n0 + r;
  if (nc >= n) return;
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int m = m0 + 16 * tm + 4 * g + q;
      if (m >= T) continue;
      if (gridDim.z > 1)
        a.part[((size_t)blockIdx.z * T + m) * n + nc] = acc[tm][q];
      else
        conv_out<EPI>(a, m, nc, acc[tm][q]);
    }
}

// the slices of a split product added in slice order, then the epilogue
template <int EPI>
__global__ __launch_bounds__(256) void k_conv_reduce(ConvArgs a, int S) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)a.T * a.n) return;
  const size_t plane = (size_t)a.T * a.n;
  float v = a.part[i];
  for (int s = 1; s < S; s++) v += a.part[s * plane + i];
  conv_out<EPI>(a, (int)(i / a.n), (int)(i % a.n), v);
}

// ConvNeXt's causal depthwise convolution (kernel 7) and LayerNorm (eps 1e-6)
// of row t: x [6 + T][1024] (history first) -> h [T][1024]. One workgroup of
// 256 threads per row, 4 channels per thread.
__global__ __launch_bounds__(256) void k_dw_ln(const float *__restrict__ x,
                                               const float *__restrict__ dw,
                                               const float *__restrict__ db,
                                               const float *__restrict__ nw,
                                               const float *__restrict__ nb,
                                               float *__restrict__ h) {
  __shared__ float red[2][4];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float v[4];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int c = tid + 256 * j;
    float acc = db[c];
#pragma unroll
    for (int k = 0; k < 7; k++) acc = fmaf(dw[c * 7 + k], x[(size_t)(t + k) * kLatent + c], acc);
    v[j] = acc;
    s += acc;
  }
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) red[0][wave] = s;
  __syncthreads();
  const float mean = ((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])) * (1.0f / kLatent);
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) q = fmaf(v[j] - mean, v[j] - mean, q);
  for (int off = 32; off >= 1; off >>= 1) q += __shfl_xor(q, off, 64);
  if (lane == 0) red[1][wave] = q;
  __syncthreads();
  const float var = ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])) * (1.0f / kLatent);
  const float inv = 1.0f / sqrtf(var + 1e-6f);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int c = tid + 256 * j;
    h[(size_t)t * kLatent + c] = fmaf((v[j] - mean) * inv, nw[c], nb[c]);
  }
}

// the output convolution (96 -> 1, kernel 7) and the clamp: x [6 + T][96].
// Four lanes per sample, lane j over channels 24 j .. 24 j + 23 of the 7
// rows, the four sums joined as (p0 + p1) + (p2 + p3).
__global__ __launch_bounds__(256) void k_conv_out(const float *__restrict__ x,
                                                  const float *__restrict__ w,
                                                  float b, int T, float *__restrict__ pcm) {
  const int t = blockIdx.x * 64 + (threadIdx.x >> 2), j = threadIdx.x & 3;
  const int tc = min(t, T - 1);
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < 7; k++) {
    const float *xr = x + (size_t)(tc + k) * 96 + 24 * j;
    const float *wk = w + k * 96 + 24 * j;
#pragma unroll
    for (int c = 0; c < 24; c += 4) {
      const float4 xv = *reinterpret_cast<const float4 *>(xr + c);
      const float4 wv = *reinterpret_cast<const float4 *>(wk + c);
      acc = fmaf(wv.x, xv.x, acc);
      acc = fmaf(wv.y, xv.y, acc);
      acc = fmaf(wv.z, xv.z, acc);
      acc = fmaf(wv.w, xv.w, acc);
    }
  }
  const float p1 = __shfl_xor(acc, 1, 64);
  const float s01 = (j & 1) ? p1 + acc : acc + p1;  // p0 + p1 (p2 + p3) in both lanes
  const float s23 = __shfl_xor(s01, 2, 64);
  const float v = ((j & 2) ? s23 + s01 : s01 + s23) + b;
  if (j == 0 && t < T) pcm[t] = fminf(1.0f, fmaxf(-1.0f, v));
}

// a sequence buffer whose last `past` rows become its history
struct HistEntry {
  float *buf;
  int past, cols, mult;  // rows of the pass = frames x mult
};

// One workgroup per sequence: rows T .. T + past - 1 move to 0 .. past - 1,
// in blocks of min(T, past) rows from the top (a block never reads what an
// earlier block wrote, nor what it writes itself).
// (the loads of a block are all issued before its stores: up to 32 values
// per thread, 8192 per block, more than any history holds)
__global__ __launch_bounds__(256) void k_save_hist(const HistEntry *__restrict__ e, int frames) {
  const HistEntry h = e[blockIdx.x];
  const int T = frames * h.mult;
  const int B = min(T, h.past);
  for (int d0 = 0; d0 < h.past; d0 += B) {
    const int rows = min(B, h.past - d0);
    const int n = rows * h.cols;
    float *dst = global_ptr(h.buf) + (size_t)d0 * h.cols;
    const float *src = global_ptr(h.buf) + (size_t)(d0 + T) * h.cols;
    for (int base = 0; base < n; base += 32 * 256) {
      float v[32];
#pragma unroll
      for (int j = 0; j < 32; j++) {
        const int i = base + j * 256 + threadIdx.x;
        v[j] = i < n ? src[i] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 32; j++) {
        const int i = base + j * 256 + threadIdx.x;
        if (i < n) dst[i] = v[j];
      }
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace q3h

using namespace q3h;

namespace {

// a convolution as the product kernels take it
struct DConv {
  float *w = nullptr, *b = nullptr;
  int cin = 0, n = 0, taps = 1, dil = 1;
};

struct DSnake {
  float *a = nullptr, *ib = nullptr;
};

struct DNext {
  float *dw = nullptr, *db = nullptr, *nw = nullptr, *nb = nullptr, *gamma = nullptr;
  DConv pw1, pw2;
};

struct DRes {
  DSnake a1, a2;
  DConv c1, c2;
};

struct DBlock {
  DSnake act;
  DConv up;
  DRes res[3];
  int cin = 0, cout = 0, rate = 0;
};

}  // namespace

struct q3h_codec {
  q3h_device *dev = nullptr;
  int max_frames = 0;
  hipStream_t stream = nullptr;
  std::vector<void *> allocs;
  int64_t bytes = 0;
  DConv up[2];
  DNext next[2];
  DConv conv0;
  DBlock blocks[4];
  DSnake act_out;
  float *out_w = nullptr;  // [7][96]
  float out_b = 0.f;
  // sequences (history rows first) and work buffers
  float *x_in = nullptr, *s_nx[2] = {nullptr, nullptr}, *x_mid = nullptr, *hn = nullptr,
        *gbuf = nullptr, *s_c0 = nullptr, *s_up[4] = {}, *xres[4] = {}, *s_r1[4][3] = {},
        *s_c2 = nullptr, *s_out = nullptr, *pcm = nullptr;
  float *part = nullptr;  // K-slice sums of the split products
  HistEntry *hist = nullptr;
  std::vector<HistEntry> hist_host;
  // the kernels of a pass of F frames, captured once per F and replayed
  std::vector<hipGraphExec_t> exec;  // [max_frames + 1]
  std::mutex mu;
};

namespace {

template <class T>
T *calloc_dev(q3h_codec *c, size_t n) {
  T *p = (T *)dev_alloc(sizeof(T) * (n ? n : 1));
  c->allocs.push_back(p);
  c->bytes += (int64_t)(sizeof(T) * n);
  check_hip(hipMemset(p, 0, sizeof(T) * (n ? n : 1)), "codec init");
  return p;
}

float *upload_f(q3h_codec *c, const std::vector<float> &v) {
  float *p = calloc_dev<float>(c, v.size());
  check_hip(hipMemcpy(p, v.data(), sizeof(float) * v.size(), hipMemcpyHostToDevice), "codec upload");
  return p;
}

const float *need(const float *p, const char *what) {
  require(p != nullptr, Q3H_E_ARG, std::string("q3h_codec_create: NULL ") + what);
  return p;
}

// torch Conv1d weight [out][in][k] -> [out][k in + c]
DConv make_conv(q3h_codec *c, const float *w, const float *b, int cin, int out, int k, int dil,
                const char *what) {
  need(w, what);
  need(b, what);
  std::vector<float> wp((size_t)out * k * cin), bp(b, b + out);
  for (int o = 0; o < out; o++)
    for (int ch = 0; ch < cin; ch++)
      for (int j = 0; j < k; j++)
        wp[(size_t)o * k * cin + (size_t)j * cin + ch] = w[((size_t)o * cin + ch) * k + j];
  DConv d;
  d.w = upload_f(c, wp);
  d.b = upload_f(c, bp);
  d.cin = cin;
  d.n = out;
  d.taps = k;
  d.dil = dil;
  return d;
}

// torch ConvTranspose1d weight [in][out][K], K = taps x stride, as a causal
// convolution of `taps` over [history ; x]: output column j out + o of row t
// (the sample t stride + j), tap k reading input row t - (taps - 1 - k)
DConv make_tconv(q3h_codec *c, const float *w, const float *b, int cin, int out, int K,
                 int stride, const char *what) {
  need(w, what);
  need(b, what);
  const int taps = K / stride, n = stride * out;
  std::vector<float> wp((size_t)n * taps * cin), bp(n);
  for (int j = 0; j < stride; j++)
    for (int o = 0; o < out; o++) {
      bp[(size_t)j * out + o] = b[o];
      for (int k = 0; k < taps; k++) {
        const int i = taps - 1 - k;
        for (int ch = 0; ch < cin; ch++)
          wp[((size_t)j * out + o) * taps * cin + (size_t)k * cin + ch] =
              w[((size_t)ch * out + o) * K + j + i * stride];
      }
    }
  DConv d;
  d.w = upload_f(c, wp);
  d.b = upload_f(c, bp);
  d.cin = cin;
  d.n = n;
  d.taps = taps;
  d.dil = 1;
  return d;
}

DConv make_linear(q3h_codec *c, const float *w, const float *b, int cin, int out,
                  const char *what) {
  return make_conv(c, w, b, cin, out, 1, 1, what);
}

DSnake make_snake(q3h_codec *c, const float *alpha, const float *beta, int n, const char *what) {
  need(alpha, what);
  need(beta, what);
  std::vector<float> a(n), ib(n);
  for (int i = 0; i < n; i++) {
    a[i] = expf(alpha[i]);
    ib[i] = 1.0f / (expf(beta[i]) + 1e-9f);
  }
  DSnake s;
  s.a = upload_f(c, a);
  s.ib = upload_f(c, ib);
  return s;
}

float *copy_vec(q3h_codec *c, const float *p, int n, const char *what) {
  need(p, what);
  return upload_f(c, std::vector<float>(p, p + n));
}

// the K slices of a layer's product (fixed per layer)
int slices(const DConv &d) {
  const int nch = d.taps * d.cin / 32;
  return (nch + kSliceChunks - 1) / kSliceChunks;
}

// y / z of a product over T output rows of sequence x
void conv(q3h_codec *c, const DConv &d, const float *x, int T, float *y, int epi,
          const float *r = nullptr, const float *g = nullptr, float *z = nullptr,
          const DSnake *sn = nullptr, int sc = 1) {
  ConvArgs a{};
  a.x = x;
  a.w = d.w;
  a.b = d.b;
  a.y = y;
  a.r = r;
  a.g = g;
  a.z = z;
  a.sa = sn ? sn->a : nullptr;
  a.sib = sn ? sn->ib : nullptr;
  a.cin = d.cin;
  a.taps = d.taps;
  a.dil = d.dil;
  a.T = T;
  a.n = d.n;
  a.sc = sc;
  a.part = c->part;
  const int S = slices(d);
  const int wn = d.n % 64 == 0 ? 4 : 2;
  const int tm = T <= 16 ? 1 : (T <= 32 ? 2 : 4);
  const dim3 grid(d.n / (16 * wn), (T + 16 * tm - 1) / (16 * tm), S);
  // few workgroups: the deep load ring (a frame per call: 0.77 -> 0.68 ms per
  // frame); the single-chunk lookahead otherwise (16-frame passes were 10-30 %
  // slower on the ring)
  const bool ring = (size_t)grid.x * grid.y * grid.z <= kRingWorkgroups;
#define Q3H_C(WN, TM, E)                                                                     \
  do {                                                                                       \
    if (ring)                                                                                \
      hipLaunchKernelGGL((k_conv_gemm_ring<WN, TM, E>), grid, dim3(64 * WN), 0, c->stream,   \
                         a.x, a.w, a.cin, a.taps, a.dil, a.T, a.n, a);                       \
    else                                                                                     \
      hipLaunchKernelGGL((k_conv_gemm<WN, TM, E>), grid, dim3(64 * WN), 0, c->stream, a);    \
  } while (0)
#define Q3H_E(WN, TM)                      \
  do {                                     \
    if (epi == CE_BIAS)                    \
      Q3H_C(WN, TM, CE_BIAS);              \
    else if (epi == CE_GELU)               \
      Q3H_C(WN, TM, CE_GELU);              \
    else if (epi == CE_RES)                \
      Q3H_C(WN, TM, CE_RES);               \
    else                                   \
      Q3H_C(WN, TM, CE_SCALED_RES);        \
  } while (0)
#define Q3H_T(WN)         \
  do {                    \
    if (tm == 1)          \
      Q3H_E(WN, 1);       \
    else if (tm == 2)     \
      Q3H_E(WN, 2);       \
    else                  \
      Q3H_E(WN, 4);       \
  } while (0)
  if (wn == 4)
    Q3H_T(4);
  else
    Q3H_T(2);
#undef Q3H_T
#undef Q3H_E
#undef Q3H_C
  if (S > 1) {
    const dim3 rg((unsigned)(((size_t)T * d.n + 255) / 256));
    if (epi == CE_BIAS)
      hipLaunchKernelGGL(k_conv_reduce<CE_BIAS>, rg, dim3(256), 0, c->stream, a, S);
    else if (epi == CE_GELU)
      hipLaunchKernelGGL(k_conv_reduce<CE_GELU>, rg, dim3(256), 0, c->stream, a, S);
    else if (epi == CE_RES)
      hipLaunchKernelGGL(k_conv_reduce<CE_RES>, rg, dim3(256), 0, c->stream, a, S);
    else
      hipLaunchKernelGGL(k_conv_reduce<CE_SCALED_RES>, rg, dim3(256), 0, c->stream, a, S);
  }
}

// one pass of F <= max_frames frames: x already in c->x_in, pcm to c->pcm
void pass(q3h_codec *c, int F) {
  hipStream_t st = c->stream;
  const int L = kLatent;
  // upsampling: transposed convolution 2 / 2 then ConvNeXt, twice
  const float *in = c->x_in;
  int rows = F;
  for (int i = 0; i < 2; i++) {
    float *seq = c->s_nx[i];  // 6 history rows, then 2 rows new rows
    conv(c, c->up[i], in, rows, seq + 6 * L, CE_BIAS);
    rows *= 2;
    hipLaunchKernelGGL(k_dw_ln, dim3(rows), dim3(256), 0, st, seq, c->next[i].dw, c->next[i].db,
                       c->next[i].nw, c->next[i].nb, c->hn);
    conv(c, c->next[i].pw1, c->hn, rows, c->gbuf, CE_GELU);
    float *out = i == 0 ? c->x_mid : c->s_c0 + 6 * L;
    conv(c, c->next[i].pw2, c->gbuf, rows, out, CE_SCALED_RES, seq + 6 * L, c->next[i].gamma);
    in = out;
  }
  // input convolution; its SnakeBeta (block 1's) written as block 1's input
  conv(c, c->conv0, c->s_c0, rows, nullptr, CE_BIAS, nullptr, nullptr,
       c->s_up[0] + kDecDim, &c->blocks[0].act, kDecDim);
  for (int b = 0; b < 4; b++) {
    DBlock &B = c->blocks[b];
    const int co = B.cout;
    // transposed convolution: the residual stream, and SnakeBeta of it as the
    // first unit's conv1 input
    conv(c, B.up, c->s_up[b], rows, c->xres[b], CE_BIAS, nullptr, nullptr,
         c->s_r1[b][0] + 6 * kDils[0] * co, &B.res[0].a1, co);
    rows *= B.rate;
    for (int u = 0; u < 3; u++) {
      DRes &R = B.res[u];
      // conv1 (dilated), SnakeBeta as conv2's input
      conv(c, R.c1, c->s_r1[b][u], rows, nullptr, CE_BIAS, nullptr, nullptr, c->s_c2, &R.a2, co);
      // conv2 + residual; SnakeBeta of the new stream for what comes next
      float *z;
      const DSnake *sn;
      if (u < 2) {
        z = c->s_r1[b][u + 1] + 6 * kDils[u + 1] * co;
        sn = &B.res[u + 1].a1;
      } else if (b < 3) {
        z = c->s_up[b + 1] + co;
        sn = &c->blocks[b + 1].act;
      } else {
        z = c->s_out + 6 * 96;
        sn = &c->act_out;
      }
      conv(c, R.c2, c->s_c2, rows, u < 2 ? c->xres[b] : nullptr, CE_RES, c->xres[b], nullptr, z,
           sn, co);
    }
  }
  hipLaunchKernelGGL(k_conv_out, dim3((rows + 63) / 64), dim3(256), 0, st, c->s_out, c->out_w,
                     c->out_b, rows, c->pcm);
  hipLaunchKernelGGL(k_save_hist, dim3((unsigned)c->hist_host.size()), dim3(256), 0, st, c->hist,
                     F);
  check_hip(hipGetLastError(), "codec kernels");
}

// the pass of F frames as one graph launch (captured at its first use)
void run_pass(q3h_codec *c, int F) {
  hipGraphExec_t &e = c->exec[F];
  if (!e) {
    hipGraph_t g = capture_graph(c->stream, [&] { pass(c, F); });
    const hipError_t r = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    check_hip(r, "instantiate");
  }
  check_hip(hipGraphLaunch(e, c->stream), "graph launch");
}

void codec_release(q3h_codec *c) {
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  for (hipGraphExec_t e : c->exec)
    if (e) (void)hipGraphExecDestroy(e);
  for (void *p : c->allocs) dev_free(p);
  if (c->stream) (void)hipStreamDestroy(c->stream);
}

}  // namespace

extern "C" int q3h_codec_create(q3h_device *dev, const q3h_codec_weights *w, int max_frames,
                                q3h_codec **out) {
  q3h_codec *c = nullptr;
  const int rc = guard([&] {
    require(dev && w && out, Q3H_E_ARG, "q3h_codec_create: NULL argument");
    require(max_frames >= 1 && max_frames <= 64, Q3H_E_ARG,
            "q3h_codec_create: max_frames must be in 1..64");
    check_hip(hipSetDevice(dev->ordinal), "hipSetDevice");
    c = new q3h_codec();
    c->dev = dev;
    c->max_frames = max_frames;
    c->exec.assign(max_frames + 1, nullptr);
    check_hip(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate");
    const int L = kLatent;
    for (int i = 0; i < 2; i++) {
      c->up[i] = make_tconv(c, w->up_w[i], w->up_b[i], L, L, 2, 2, "upsample conv");
      DNext &n = c->next[i];
      n.dw = copy_vec(c, w->dw_w[i], 7 * L, "dwconv weight");
      n.db = copy_vec(c, w->dw_b[i], L, "dwconv bias");
      n.nw = copy_vec(c, w->norm_w[i], L, "norm weight");
      n.nb = copy_vec(c, w->norm_b[i], L, "norm bias");
      n.gamma = copy_vec(c, w->gamma[i], L, "gamma");
      n.pw1 = make_linear(c, w->pw1_w[i], w->pw1_b[i], L, 4 * L, "pwconv1");
      n.pw2 = make_linear(c, w->pw2_w[i], w->pw2_b[i], 4 * L, L, "pwconv2");
    }
    c->conv0 = make_conv(c, w->conv0_w, w->conv0_b, L, kDecDim, 7, 1, "decoder.0.conv");
    for (int b = 0; b < 4; b++) {
      DBlock &B = c->blocks[b];
      const q3h_codec_block &bw = w->block[b];
      B.cin = kDecDim >> b;
      B.cout = kDecDim >> (b + 1);
      B.rate = kRates[b];
      B.act = make_snake(c, bw.act_alpha, bw.act_beta, B.cin, "block snake");
      B.up = make_tconv(c, bw.up_w, bw.up_b, B.cin, B.cout, 2 * B.rate, B.rate, "block conv");
      for (int u = 0; u < 3; u++) {
        const q3h_codec_res &rw = bw.res[u];
        B.res[u].a1 = make_snake(c, rw.a1_alpha, rw.a1_beta, B.cout, "act1");
        B.res[u].a2 = make_snake(c, rw.a2_alpha, rw.a2_beta, B.cout, "act2");
        B.res[u].c1 = make_conv(c, rw.c1_w, rw.c1_b, B.cout, B.cout, 7, kDils[u], "conv1");
        B.res[u].c2 = make_conv(c, rw.c2_w, rw.c2_b, B.cout, B.cout, 1, 1, "conv2");
      }
    }
    c->act_out = make_snake(c, w->out_alpha, w->out_beta, 96, "decoder.5");
    need(w->out_w, "decoder.6.conv weight");
    need(w->out_b, "decoder.6.conv bias");
    {
      std::vector<float> ow(7 * 96);
      for (int k = 0; k < 7; k++)
        for (int ch = 0; ch < 96; ch++) ow[k * 96 + ch] = w->out_w[ch * 7 + k];
      c->out_w = upload_f(c, ow);
      c->out_b = w->out_b[0];
    }
    // sequences and work buffers for max_frames frames
    const size_t F = max_frames;
    c->x_in = calloc_dev<float>(c, F * L);
    c->s_nx[0] = calloc_dev<float>(c, (6 + 2 * F) * L);
    c->x_mid = calloc_dev<float>(c, 2 * F * L);
    c->s_nx[1] = calloc_dev<float>(c, (6 + 4 * F) * L);
    c->hn = calloc_dev<float>(c, 4 * F * L);
    c->gbuf = calloc_dev<float>(c, 4 * F * 4 * L);
    c->s_c0 = calloc_dev<float>(c, (6 + 4 * F) * L);
    std::vector<HistEntry> &h = c->hist_host;
    h.push_back({c->s_nx[0], 6, L, 2});
    h.push_back({c->s_nx[1], 6, L, 4});
    h.push_back({c->s_c0, 6, L, 4});
    size_t rin = 4, c2max = 0;
    for (int b = 0; b < 4; b++) {
      const DBlock &B = c->blocks[b];
      const size_t rout = rin * B.rate;
      c->s_up[b] = calloc_dev<float>(c, (1 + rin * F) * B.cin);
      h.push_back({c->s_up[b], 1, B.cin, (int)rin});
      c->xres[b] = calloc_dev<float>(c, rout * F * B.cout);
      for (int u = 0; u < 3; u++) {
        const int past = 6 * kDils[u];
        c->s_r1[b][u] = calloc_dev<float>(c, (past + rout * F) * B.cout);
        h.push_back({c->s_r1[b][u], past, B.cout, (int)rout});
      }
      c2max = std::max(c2max, rout * F * B.cout);
      rin = rout;
    }
    c->s_c2 = calloc_dev<float>(c, c2max);
    c->s_out = calloc_dev<float>(c, (6 + rin * F) * 96);
    h.push_back({c->s_out, 6, 96, (int)rin});
    c->pcm = calloc_dev<float>(c, rin * F);
    // the split products' slices: the largest S x T x n of any layer
    size_t pmax = 0;
    auto need_part = [&](const DConv &d, size_t T) {
      const int S = slices(d);
      if (S > 1) pmax = std::max(pmax, (size_t)S * T * d.n);
    };
    for (int i = 0; i < 2; i++) {
      need_part(c->up[i], (i + 1) * F);
      need_part(c->next[i].pw1, 2 * (i + 1) * F);
      need_part(c->next[i].pw2, 2 * (i + 1) * F);
    }
    need_part(c->conv0, 4 * F);
    size_t rr = 4;
    for (int b = 0; b < 4; b++) {
      need_part(c->blocks[b].up, rr * F);
      rr *= c->blocks[b].rate;
      for (int u = 0; u < 3; u++) {
        need_part(c->blocks[b].res[u].c1, rr * F);
        need_part(c->blocks[b].res[u].c2, rr * F);
      }
    }
    c->part = calloc_dev<float>(c, pmax);
    c->hist = calloc_dev<HistEntry>(c, h.size());
    check_hip(hipMemcpy(c->hist, h.data(), sizeof(HistEntry) * h.size(), hipMemcpyHostToDevice),
              "codec init");
    dev->bytes += c->bytes;
    dev->stacks++;
    *out = c;
  });
  if (rc != 0 && c) {
    codec_release(c);
    delete c;
  }
  return rc;
}

extern "C" int q3h_codec_reset(q3h_codec *c) {
  return guard([&] {
    require(c != nullptr, Q3H_E_ARG, "q3h_codec_reset: NULL codec");
    std::lock_guard<std::mutex> lk(c->mu);
    check_hip(hipSetDevice(c->dev->ordinal), "hipSetDevice");
    for (const HistEntry &h : c->hist_host)
      check_hip(hipMemsetAsync(h.buf, 0, sizeof(float) * h.past * h.cols, c->stream), "reset");
    check_hip(hipStreamSynchronize(c->stream), "reset sync");
  });
}

extern "C" int q3h_codec_back(q3h_codec *c, const float *x, int frames, float *pcm) {
  return guard([&] {
    require(c != nullptr, Q3H_E_ARG, "q3h_codec_back: NULL codec");
    require(frames >= 0, Q3H_E_ARG, "q3h_codec_back: negative frame count");
    if (frames == 0) return;
    require(x != nullptr && pcm != nullptr, Q3H_E_ARG, "q3h_codec_back: NULL x or pcm");
    std::lock_guard<std::mutex> lk(c->mu);
    check_hip(hipSetDevice(c->dev->ordinal), "hipSetDevice");
    for (int f0 = 0; f0 < frames; f0 += c->max_frames) {
      const int F = std::min(c->max_frames, frames - f0);
      check_hip(hipMemcpyAsync(c->x_in, x + (size_t)f0 * kLatent, sizeof(float) * F * kLatent,
                               hipMemcpyHostToDevice, c->stream),
                "upload x");
      run_pass(c, F);
      check_hip(hipMemcpyAsync(pcm + (size_t)f0 * kFrameSamples, c->pcm,
                               sizeof(float) * F * kFrameSamples, hipMemcpyDeviceToHost, c->stream),
                "download pcm");
    }
    check_hip(hipStreamSynchronize(c->stream), "codec sync");
  });
}

extern "C" int64_t q3h_codec_bytes(const q3h_codec *c) { return c ? c->bytes : 0; }

extern "C" int q3h_codec_destroy(q3h_codec *c) {
  return guard([&] {
    if (!c) return;
    check_hip(hipSetDevice(c->dev->ordinal), "hipSetDevice");
    c->dev->bytes -= c->bytes;
    c->dev->stacks--;
    codec_release(c);
    delete c;
  });
}
