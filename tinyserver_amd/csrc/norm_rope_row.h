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

}  // namespace tsa
