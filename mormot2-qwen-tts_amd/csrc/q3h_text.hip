// q3h_text.hip - the talker's text projection on the device
// (TQwenTalker.TextProject, src/tts/mormot.ai.tts.qwen.talker.pas:390-421):
// y[r] = fc2 . SiLU(fc1 . emb[ids[r]] + b1) + b2, SiLU(v) = 0 below -80.
//
// Three launches over all n rows at once:
//  1. k_text_rows: row r of the embedding widened to f32 (BF16 is the high
//     half of an f32: exact), and the biases written where the products add:
//     h[r] = b1, y[r] = b2;
//  2. fc1 on the f32 matrix cores, epilogue h = SiLU(h + sum) (EPI_ADD_SILU);
//  3. fc2 on the f32 matrix cores, epilogue y += sum (EPI_ADD).
// Weights and products stay in f32 (the reference's idtF32 products). The
// embedding table stays in the dtype it came in (BF16: 622 MB for 151936 x
// 2048), gathered one row per token.
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>

#include "q3h_api_internal.h"

namespace q3h {
namespace {

__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// one workgroup per row: e[r] = emb[ids[r]] in f32, h[r] = b1, y[r] = b2
// (TH % 8 == 0, H % 4 == 0; rows 16-byte aligned)
template <bool BF16>
__global__ __launch_bounds__(256) void k_text_rows(const void *__restrict__ emb,
                                                   const int32_t *__restrict__ ids, int TH,
                                                   int H, const float *__restrict__ b1,
                                                   const float *__restrict__ b2,
                                                   float *__restrict__ e, float *__restrict__ h,
                                                   float *__restrict__ y, int ldy) {
  const int r = blockIdx.x, t = threadIdx.x;
  const size_t id = (size_t)ids[r];
  float4 *er = reinterpret_cast<float4 *>(e + (size_t)r * TH);
  if (BF16) {
    const uint4 *src = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(emb) + id * TH);
    for (int i = t; i < TH / 8; i += 256) {
      const uint4 v = src[i];
      er[2 * i] = make_float4(bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y));
      er[2 * i + 1] = make_float4(bf_lo(v.z), bf_hi(v.z), bf_lo(v.w), bf_hi(v.w));
    }
  } else {
    const float4 *src = reinterpret_cast<const float4 *>(static_cast<const float *>(emb) + id * TH);
    for (int i = t; i < TH / 4; i += 256) er[i] = src[i];
  }
  float4 *hr = reinterpret_cast<float4 *>(h + (size_t)r * TH);
  const float4 *b1v = reinterpret_cast<const float4 *>(b1);
  for (int i = t; i < TH / 4; i += 256) hr[i] = b1v[i];
  float *yr = y + (size_t)r * ldy;
  for (int i = t; i < H; i += 256) yr[i] = b2[i];
}

void text_release(q3h_text_proj *t) {
  dev_free(t->emb);
  dev_free(t->fc1.f);
  dev_free(t->fc2.f);
  dev_free(t->b1);
  dev_free(t->b2);
  dev_free(t->ids);
  dev_free(t->e);
  dev_free(t->h);
  dev_free(t->y);
  if (t->stream) (void)hipStreamDestroy(t->stream);
}

template <class T>
T *upload(const T *src, size_t n, const char *what) {
  require(src != nullptr, Q3H_E_ARG, std::string("q3h_text_create: ") + what + " is NULL");
  T *d = (T *)dev_alloc(sizeof(T) * n);
  check_hip(hipMemcpy(d, src, sizeof(T) * n, hipMemcpyHostToDevice), what);
  return d;
}

}  // namespace

void text_ensure(q3h_text_proj *t, int n) {
  if (n <= t->cap) return;
  const int cap = std::max(n, std::max(64, 2 * t->cap));
  check_hip(hipStreamSynchronize(t->stream), "text sync");
  dev_free(t->ids);
  dev_free(t->e);
  dev_free(t->h);
  dev_free(t->y);
  t->ids = nullptr;
  t->e = t->h = t->y = nullptr;
  t->cap = 0;
  const size_t TH = t->cfg.text_hidden, H = t->cfg.hidden;
  t->ids = (int32_t *)dev_alloc(sizeof(int32_t) * cap);
  t->e = (float *)dev_alloc(sizeof(float) * cap * TH);
  t->h = (float *)dev_alloc(sizeof(float) * cap * TH);
  t->y = (float *)dev_alloc(sizeof(float) * cap * H);
  t->cap = cap;
}

void text_project_dev(q3h_text_proj *t, const int32_t *ids_dev, int n, float *y, int ldy,
                      hipStream_t st) {
  const q3h_text_config &c = t->cfg;
  const int TH = c.text_hidden, H = c.hidden;
  if (c.emb_dtype == Q3H_BF16)
    hipLaunchKernelGGL(k_text_rows<true>, dim3(n), dim3(256), 0, st, t->emb, ids_dev, TH, H,
                       t->b1, t->b2, t->e, t->h, y, ldy);
  else
    hipLaunchKernelGGL(k_text_rows<false>, dim3(n), dim3(256), 0, st, t->emb, ids_dev, TH, H,
                       t->b1, t->b2, t->e, t->h, y, ldy);
  launch_gemm_f32(t->fc1, t->e, TH, n, EPI_ADD_SILU, t->h, TH, st);
  launch_gemm_f32(t->fc2, t->h, TH, n, EPI_ADD, y, ldy, st);
  check_hip(hipGetLastError(), "text projection kernels");
}

}  // namespace q3h

using namespace q3h;

extern "C" int q3h_text_create(q3h_device *dev, const q3h_text_config *cfg, const void *emb,
                               const float *fc1_w, const float *fc1_b, const float *fc2_w,
                               const float *fc2_b, q3h_text_proj **out) {
  q3h_text_proj *t = nullptr;
  const int rc = guard([&] {
    require(dev && cfg && out, Q3H_E_ARG, "q3h_text_create: NULL argument");
    const q3h_text_config c = *cfg;
    require(c.text_vocab > 0, Q3H_E_ARG, "q3h_text_create: text_vocab must be positive");
    require(c.emb_dtype == Q3H_BF16 || c.emb_dtype == Q3H_F32, Q3H_E_ARG,
            "q3h_text_create: emb_dtype must be Q3H_BF16 or Q3H_F32");
    require(c.hidden > 0 && gemm_f32_supported(c.text_hidden, c.text_hidden) &&
                gemm_f32_supported(c.hidden, c.text_hidden),
            Q3H_E_ARG,
            "q3h_text_create: text_hidden must be 1024, 2048 or 3072 and hidden a multiple of 16");
    check_hip(hipSetDevice(dev->ordinal), "hipSetDevice");
    t = new q3h_text_proj();
    t->dev = dev;
    t->cfg = c;
    const size_t TH = c.text_hidden, H = c.hidden;
    const size_t es = c.emb_dtype == Q3H_BF16 ? 2 : 4;
    require(emb != nullptr, Q3H_E_ARG, "q3h_text_create: emb is NULL");
    t->emb = dev_alloc(es * c.text_vocab * TH);
    check_hip(hipMemcpy(t->emb, emb, es * c.text_vocab * TH, hipMemcpyHostToDevice),
              "upload text embedding");
    t->fc1.N = t->fc1.K = c.text_hidden;
    t->fc1.f = upload(fc1_w, TH * TH, "fc1_w");
    t->fc2.N = c.hidden;
    t->fc2.K = c.text_hidden;
    t->fc2.f = upload(fc2_w, H * TH, "fc2_w");
    t->b1 = upload(fc1_b, TH, "fc1_b");
    t->b2 = upload(fc2_b, H, "fc2_b");
    t->bytes = (int64_t)(es * c.text_vocab * TH + 4 * (TH * TH + H * TH + TH + H));
    check_hip(hipStreamCreateWithFlags(&t->stream, hipStreamNonBlocking), "hipStreamCreate");
    dev->bytes += t->bytes;
    dev->stacks++;
    *out = t;
  });
  if (rc != 0 && t) {
    text_release(t);
    delete t;
  }
  return rc;
}

extern "C" int q3h_text_project(q3h_text_proj *t, const int32_t *ids, int n, float *y) {
  return guard([&] {
    require(t != nullptr, Q3H_E_ARG, "q3h_text_project: NULL projection");
    require(n >= 0, Q3H_E_ARG, "q3h_text_project: negative row count");
    if (n == 0) return;
    require(ids != nullptr && y != nullptr, Q3H_E_ARG, "q3h_text_project: NULL ids or y");
    for (int r = 0; r < n; r++)
      require(ids[r] >= 0 && ids[r] < t->cfg.text_vocab, Q3H_E_ARG,
              "q3h_text_project: text token " + std::to_string(ids[r]) + " out of range");
    std::lock_guard<std::mutex> lk(t->mu);
    check_hip(hipSetDevice(t->dev->ordinal), "hipSetDevice");
    text_ensure(t, n);
    hipStream_t st = t->stream;
    check_hip(hipMemcpyAsync(t->ids, ids, sizeof(int32_t) * n, hipMemcpyHostToDevice, st),
              "upload ids");
    text_project_dev(t, t->ids, n, t->y, t->cfg.hidden, st);
    check_hip(hipMemcpyAsync(y, t->y, sizeof(float) * n * t->cfg.hidden, hipMemcpyDeviceToHost,
                             st),
              "download y");
    check_hip(hipStreamSynchronize(st), "text sync");
  });
}

extern "C" int q3h_text_destroy(q3h_text_proj *t) {
  return guard([&] {
    if (!t) return;
    check_hip(hipSetDevice(t->dev->ordinal), "hipSetDevice");
    if (t->stream) (void)hipStreamSynchronize(t->stream);
    t->dev->bytes -= t->bytes;
    t->dev->stacks--;
    text_release(t);
    delete t;
  });
}
