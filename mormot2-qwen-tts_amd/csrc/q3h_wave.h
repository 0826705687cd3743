// q3h_wave.h - wavefront (64-lane) reductions for gfx950 built on DPP row
// operations instead of LDS permutes: a sum is six DPP adds (quad swaps,
// half-row and row mirrors, row broadcasts 15 and 31) and a read of lane 63.
#pragma once

#include <hip/hip_runtime.h>

namespace q3h {

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false));
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_i(int v, int old) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xf, false);
}

// DPP controls (gfx9)
constexpr int kQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
constexpr int kBcast15 = 0x142;
constexpr int kBcast31 = 0x143;

// sum over the 64 lanes, returned in every lane (all lanes must be active)
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f<kQuadXor1>(v);
  v += dpp_f<kQuadXor2>(v);
  v += dpp_f<kHalfMirror>(v);
  v += dpp_f<kRowMirror>(v);
  v += dpp_f<kBcast15, 0xa>(v);
  v += dpp_f<kBcast31, 0xc>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ double dpp_d_step(double v, int which) {
  // one DPP step on both halves of a double; which selects the control
  const long long b = __builtin_bit_cast(long long, v);
  int lo = (int)b, hi = (int)(b >> 32);
  switch (which) {
    case 0: lo = dpp_i<kQuadXor1>(lo, 0); hi = dpp_i<kQuadXor1>(hi, 0); break;
    case 1: lo = dpp_i<kQuadXor2>(lo, 0); hi = dpp_i<kQuadXor2>(hi, 0); break;
    case 2: lo = dpp_i<kHalfMirror>(lo, 0); hi = dpp_i<kHalfMirror>(hi, 0); break;
    case 3: lo = dpp_i<kRowMirror>(lo, 0); hi = dpp_i<kRowMirror>(hi, 0); break;
    case 4: lo = dpp_i<kBcast15, 0xa>(lo, 0); hi = dpp_i<kBcast15, 0xa>(hi, 0); break;
    default: lo = dpp_i<kBcast31, 0xc>(lo, 0); hi = dpp_i<kBcast31, 0xc>(hi, 0); break;
  }
  return __builtin_bit_cast(double, ((long long)hi << 32) | (unsigned int)lo);
}

// double sum over the 64 lanes, returned in every lane
__device__ __forceinline__ double wave_sum_dpp_d(double v) {
#pragma unroll
  for (int i = 0; i < 6; i++) v += dpp_d_step(v, i);
  const long long b = __builtin_bit_cast(long long, v);
  const int lo = __builtin_amdgcn_readlane((int)b, 63);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), 63);
  return __builtin_bit_cast(double, ((long long)hi << 32) | (unsigned int)lo);
}

// lane q's value (q uniform across the wave): a register read, no LDS trip
__device__ __forceinline__ float lane_f(float v, int q) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), q));
}

// inclusive prefix sum over the 64 lanes (lane i: lanes 0 .. i), exact for
// integers: row scans by DPP row shifts, then the row totals broadcast by
// row_bcast15 / row_bcast31
__device__ __forceinline__ int wave_prefix_sum_i(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, true);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, kBcast15, 0xa, 0xf, false);
  v += __builtin_amdgcn_update_dpp(0, v, kBcast31, 0xc, 0xf, false);
  return v;
}

// the value of lane l + K of the same 16-lane row (DPP row_shl:K; 0 past the
// row's end)
template <int K>
__device__ __forceinline__ float row_shl_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + K, 0xf, 0xf, true));
}

// DPP move where lanes outside the row mask keep their own value (the
// identity of max)
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f_keep(float v) {
  const int b = __builtin_bit_cast(int, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b, b, CTRL, ROW_MASK, 0xf, false));
}

// maximum over the 64 lanes, returned in every lane
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_f_keep<kQuadXor1>(v));
  v = fmaxf(v, dpp_f_keep<kQuadXor2>(v));
  v = fmaxf(v, dpp_f_keep<kHalfMirror>(v));
  v = fmaxf(v, dpp_f_keep<kRowMirror>(v));
  v = fmaxf(v, dpp_f_keep<kBcast15, 0xa>(v));
  v = fmaxf(v, dpp_f_keep<kBcast31, 0xc>(v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// maximum over the lane's quad (lanes 4 (l / 4) .. + 3), in every lane of it
__device__ __forceinline__ float quad_max_dpp(float v) {
  v = fmaxf(v, dpp_f_keep<kQuadXor1>(v));
  return fmaxf(v, dpp_f_keep<kQuadXor2>(v));
}

// maximum over the lane's 32-lane half (rows 0-1 or 2-3): the row maximum by
// DPP, then the other row's through gfx950's row swap (v_permlane16_swap)
__device__ __forceinline__ float half_max_dpp(float v) {
  v = quad_max_dpp(v);
  v = fmaxf(v, dpp_f_keep<kHalfMirror>(v));
  v = fmaxf(v, dpp_f_keep<kRowMirror>(v));
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)a[0]), __builtin_bit_cast(float, (unsigned)a[1]));
}

// v summed over the wave's four 16-lane rows at one place in the row (lanes
// l, l ^ 16, l ^ 32, l ^ 48), in every lane: (v_l + v_l^16) + (v_l^32 +
// v_l^48), the pairs in the same order as two xor shuffles by 16 and 32 add
// them (an add commutes exactly), through gfx950's row swaps
// (v_permlane16_swap: odd rows of the first operand with even rows of the
// second; v_permlane32_swap: the upper half of the first with the lower half
// of the second) instead of LDS permutes
__device__ __forceinline__ float rows4_sum(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = __builtin_bit_cast(float, (unsigned)a[0]) + __builtin_bit_cast(float, (unsigned)a[1]);
  const unsigned w = __builtin_bit_cast(unsigned, v);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return __builtin_bit_cast(float, (unsigned)b[0]) + __builtin_bit_cast(float, (unsigned)b[1]);
}

// the maximum over the same four lanes, in every lane
__device__ __forceinline__ float rows4_max(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__builtin_bit_cast(float, (unsigned)a[0]), __builtin_bit_cast(float, (unsigned)a[1]));
  const unsigned w = __builtin_bit_cast(unsigned, v);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)b[0]), __builtin_bit_cast(float, (unsigned)b[1]));
}

// Eight values o[0..7] summed over the wave's four 16-lane rows with the
// pairs of rows4_sum, scattered: lane l of row r = l / 16 gets the sum of
// o[r] in lo and of o[4 + r] in hi. Each stage is one row swap and one add
// for two registers: permlane16_swap(x, y) added holds x's rows 0 + 1 in row
// 0, y's in row 1, x's rows 2 + 3 in row 2, y's in row 3; permlane32_swap(x,
// y) added holds x's rows 0 + 2 and 1 + 3 in rows 0 and 1, y's in rows 2, 3
// (12 instructions where eight rows4_sum take 32 and their copies)
__device__ __forceinline__ float swap16_add(float x, float y) {
  const auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, x),
                                                  __builtin_bit_cast(unsigned, y), false, false);
  return __builtin_bit_cast(float, (unsigned)a[0]) + __builtin_bit_cast(float, (unsigned)a[1]);
}
__device__ __forceinline__ float swap32_add(float x, float y) {
  const auto a = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x),
                                                  __builtin_bit_cast(unsigned, y), false, false);
  return __builtin_bit_cast(float, (unsigned)a[0]) + __builtin_bit_cast(float, (unsigned)a[1]);
}
__device__ __forceinline__ void rows4_scatter8(const float (&o)[8], float &lo, float &hi) {
  lo = swap32_add(swap16_add(o[0], o[1]), swap16_add(o[2], o[3]));
  hi = swap32_add(swap16_add(o[4], o[5]), swap16_add(o[6], o[7]));
}

// sum over aligned groups of 8 lanes (lanes 8k..8k+7), in every lane of the group
__device__ __forceinline__ float group8_sum_dpp(float v) {
  v += dpp_f<kQuadXor1>(v);
  v += dpp_f<kQuadXor2>(v);
  v += dpp_f<kHalfMirror>(v);
  return v;
}

// sum over the 16 lanes of a DPP row (lanes 16k..16k+15), in every lane of the row
__device__ __forceinline__ float group16_sum_dpp(float v) {
  v += dpp_f<kQuadXor1>(v);
  v += dpp_f<kQuadXor2>(v);
  v += dpp_f<kHalfMirror>(v);
  v += dpp_f<kRowMirror>(v);
  return v;
}

// (value, index) maximum with the first index winning ties
__device__ __forceinline__ void argmax_merge(float &v, int &i, float v2, int i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// The code of a first-max argmax as tests/test.tts.qwen.lm.pas:109-117 runs
// it (result 0, moved to i only when p[i] > p[result]), from the reduction of
// argmax_merge over every (p[i], i) starting at (-inf, 0x7fffffff): a NaN
// never wins, a NaN p[0] keeps 0 (nothing compares greater), and no maximum
// at all (every value NaN) is 0 as well. Always an index of the table.
__device__ __forceinline__ int first_max_code(int bi, float p0) {
  return (bi == 0x7fffffff || p0 != p0) ? 0 : bi;
}

}  // namespace q3h
