// One 128-dim (or 64/256-dim) head row's Qwen3 RMSNorm + rotate-half RoPE
// in 16-lane DPP rows, with HF's rounding points and the CPU reduction's
// order for mean(x^2). Shared by the norm/RoPE kernels and the single-launch
// decode step, so both round identically.
#pragma once

#include "tsa_common.h"

namespace tsa {

template <typename T>
__device__ __forceinline__ float round_t(float x) { return to_float(from_float<T>(x)); }

// Cross-lane moves inside the 16-lane rows of a wave (DPP, no LDS traffic):
// lane i gets lane i + N of its row (row_shl), or lane (i - N) mod 16
// (row_ror).
template <int N>
__device__ __forceinline__ float dpp_row_shl(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + N, 0xF, 0xF, true));
}
template <int N>
__device__ __forceinline__ float dpp_row_ror(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x120 + N, 0xF, 0xF, false));
}

// One (token, head) row's norm + RoPE on the values already in registers.
template <typename T, int D>
__device__ __forceinline__ void norm_rope_row(const float (&x)[8], const float (&wf)[8], const float (&cs)[8],
                                              const float (&sn)[8], float eps, int lane_in_row, float (&o)[8]) {
  constexpr int LANES = D / 8;  // lanes per (token, head) row
  // mean(x^2) in fp32, summed in the order of the CPU reduction the model's
  // RMSNorm runs through (four 8-wide accumulators over 32-element strides,
  // added in order, then the 8 lanes in order), so the rounded sum -- and the
  // bf16 results downstream of it -- match it bit for bit. Element 8c + e of
  // the row lives in lane c: accumulator k = c % 4 collects lanes k, k+4, ...
  // (The sums are meaningful in lanes 0..3 of the row.)
  float sq[8], acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = sq[e] = __fmul_rn(x[e], x[e]);
  float ss = 0.f;
  if constexpr (LANES == 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[e] = __fadd_rn(acc[e], dpp_row_shl<4>(sq[e]));
      acc[e] = __fadd_rn(acc[e], dpp_row_shl<8>(sq[e]));
      acc[e] = __fadd_rn(acc[e], dpp_row_shl<12>(sq[e]));
      float v = acc[e];
      v = __fadd_rn(v, dpp_row_shl<1>(acc[e]));
      v = __fadd_rn(v, dpp_row_shl<2>(acc[e]));
      v = __fadd_rn(v, dpp_row_shl<3>(acc[e]));
      ss = __fadd_rn(ss, v);
    }
  } else {
#pragma unroll
    for (int step = 4; step < LANES; step += 4)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = __fadd_rn(acc[e], __shfl_down(sq[e], step, LANES));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[e];
#pragma unroll
      for (int k = 1; k < 4; ++k) v = __fadd_rn(v, __shfl_down(acc[e], k, LANES));
      ss = __fadd_rn(ss, v);  // meaningful in lane 0 of the row
    }
  }
  ss = __shfl(ss, 0, LANES);
  const float var = __fdiv_rn(ss, static_cast<float>(D));
  const float rinv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));

  float z[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = round_t<T>(__fmul_rn(wf[i], round_t<T>(__fmul_rn(x[i], rinv))));

  // Partner half: lane c holds dims 8c..8c+7, dims +- D/2 are in lane c ^ (LANES/2).
  float zp[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) zp[i] = LANES == 16 ? dpp_row_ror<8>(z[i]) : __shfl_xor(z[i], LANES / 2, 64);
  const bool first_half = lane_in_row < LANES / 2;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float rot = first_half ? -zp[i] : zp[i];
    o[i] = round_t<T>(__fadd_rn(round_t<T>(__fmul_rn(z[i], cs[i])), round_t<T>(__fmul_rn(rot, sn[i]))));
  }
}

// Two values rounded to T (a pair shares one v_cvt_pk) and widened again.
template <typename T>
__device__ __forceinline__ void round2_t(float& a, float& b) {
  const uint32_t p = pack2<T>(a, b);
  a = lo_f<T>(p);
  b = hi_f<T>(p);
}

// The same row computation for head_dim 128 and a 16-bit T in another lane
// layout: 8 lanes per row, lane c holding dims 8c..8c+7 (chunk 0) and
// 64+8c..64+8c+7 (chunk 1) as packed pairs. A dim's RoPE partner (d +- 64)
// is then in the same lane, and one DPP instruction serves the 8 rows of a
// wave. The arithmetic, its rounding points and the order of the sum of
// squares are those of norm_rope_row, so the two agree bit for bit: the
// CPU order's accumulator k = c % 4 takes chunks k, k+4, k+8, k+12, which
// are lane k's chunk 0, lane k+4's chunk 0, lane k's chunk 1 and lane
// k+4's chunk 1. Every lane must run this (lanes 8r..8r+7 form a row).
template <typename T>
__device__ __forceinline__ void norm_rope_row_d128x8(const u32x4 (&xp)[2], const u32x4 (&wp)[2], const u32x4 (&cp)[2],
                                                     const u32x4 (&sp)[2], float eps, u32x4 (&op)[2]) {
  static_assert(sizeof(T) == 2, "16-bit element types only");
  float x[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[j][2 * i] = lo_f<T>(xp[j][i]);
      x[j][2 * i + 1] = hi_f<T>(xp[j][i]);
    }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float s0 = __fmul_rn(x[0][e], x[0][e]), s1 = __fmul_rn(x[1][e], x[1][e]);
    float acc = __fadd_rn(s0, dpp_row_shl<4>(s0));
    acc = __fadd_rn(acc, s1);
    acc = __fadd_rn(acc, dpp_row_shl<4>(s1));
    float v = acc;
    v = __fadd_rn(v, dpp_row_shl<1>(acc));
    v = __fadd_rn(v, dpp_row_shl<2>(acc));
    v = __fadd_rn(v, dpp_row_shl<3>(acc));
    ss = __fadd_rn(ss, v);  // meaningful in lane 0 of each 8-lane row
  }
  // Broadcast lane 0 of each 8-lane row: quad_perm(0,0,0,0) fills lanes
  // 0-3 (and 8-11) from lane 0 (8), then row_shr:4 restricted to banks 1
  // and 3 copies lanes 0-3 (8-11) into lanes 4-7 (12-15).
  int b = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, ss), 0x00, 0xF, 0xF, false);
  b = __builtin_amdgcn_update_dpp(b, b, 0x114, 0xF, 0xA, false);
  ss = __builtin_bit_cast(float, b);
  const float var = __fdiv_rn(ss, 128.0f);
  const float rinv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));

  float z[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float y0 = __fmul_rn(x[j][2 * i], rinv), y1 = __fmul_rn(x[j][2 * i + 1], rinv);
      round2_t<T>(y0, y1);
      float z0 = __fmul_rn(lo_f<T>(wp[j][i]), y0), z1 = __fmul_rn(hi_f<T>(wp[j][i]), y1);
      round2_t<T>(z0, z1);
      z[j][2 * i] = z0;
      z[j][2 * i + 1] = z1;
    }
  // rotate_half: dims < 64 (chunk 0) pair with -z[d + 64], dims >= 64 with z[d - 64].
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float c0 = lo_f<T>(cp[j][i]), c1 = hi_f<T>(cp[j][i]);
      const float s0 = lo_f<T>(sp[j][i]), s1 = hi_f<T>(sp[j][i]);
      const float r0 = j == 0 ? -z[1][2 * i] : z[0][2 * i];
      const float r1 = j == 0 ? -z[1][2 * i + 1] : z[0][2 * i + 1];
      float a0 = __fmul_rn(z[j][2 * i], c0), a1 = __fmul_rn(z[j][2 * i + 1], c1);
      round2_t<T>(a0, a1);
      float b0 = __fmul_rn(r0, s0), b1 = __fmul_rn(r1, s1);
      round2_t<T>(b0, b1);
      op[j][i] = pack2<T>(__fadd_rn(a0, b0), __fadd_rn(a1, b1));
    }
}

}  // namespace tsa
