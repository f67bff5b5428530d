// Shared device/host helpers for the gfx950 attention-path kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "tsa_api.h"

namespace tsa {

// ---------------------------------------------------------------- errors --
// Per-thread last-error message (the library keeps no other host state).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
const char* last_error();

#define TSA_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      ::tsa::set_error(__VA_ARGS__);  \
      return TSA_ERR_INVALID;         \
    }                                 \
  } while (0)

#define TSA_UNSUPPORTED(cond, ...)    \
  do {                                \
    if (!(cond)) {                    \
      ::tsa::set_error(__VA_ARGS__);  \
      return TSA_ERR_UNSUPPORTED;     \
    }                                 \
  } while (0)

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return TSA_ERR_LAUNCH;
  }
  return TSA_OK;
}

// ----------------------------------------------------------------- views --
inline bool is_float_dtype(int dt) { return dt == TSA_BF16 || dt == TSA_F16 || dt == TSA_F32; }
inline bool is_index_dtype(int dt) { return dt == TSA_I32 || dt == TSA_I64; }
inline int dtype_bytes(int dt) { return dt == TSA_F32 || dt == TSA_I32 ? 4 : dt == TSA_I64 ? 8 : 2; }
inline const char* dtype_name(int dt) {
  switch (dt) {
    case TSA_BF16: return "bf16";
    case TSA_F16: return "f16";
    case TSA_F32: return "f32";
    case TSA_I32: return "i32";
    case TSA_I64: return "i64";
  }
  return "?";
}

// A view is usable when it is non-NULL, has the expected rank, a sane dtype
// and non-negative sizes. Data may be NULL only for an empty view.
inline bool view_ok(const tsa_view* v, int ndim) {
  if (!v || v->ndim != ndim) return false;
  if (v->dtype < TSA_BF16 || v->dtype > TSA_I64) return false;
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) {
    if (v->size[d] < 0) return false;
    n *= v->size[d];
  }
  return n == 0 || v->data != nullptr;
}
inline int64_t numel(const tsa_view* v) {
  int64_t n = 1;
  for (int d = 0; d < v->ndim; ++d) n *= v->size[d];
  return n;
}
// Innermost dimension is unit-stride and every row starts 16-byte aligned, so
// rows can be moved with 128-bit accesses.
inline bool rows_vec16(const tsa_view* v) {
  const int eb = dtype_bytes(v->dtype);
  const int nd = v->ndim;
  if (v->stride[nd - 1] != 1 && v->size[nd - 1] > 1) return false;
  if ((v->size[nd - 1] * eb) % 16 != 0) return false;
  if (reinterpret_cast<uintptr_t>(v->data) % 16 != 0) return false;
  for (int d = 0; d < nd - 1; ++d)
    if (v->size[d] > 1 && (v->stride[d] * eb) % 16 != 0) return false;
  return true;
}

// ------------------------------------------------------- element helpers --
struct bf16_t { uint16_t x; };
struct f16_t { uint16_t x; };

__device__ __forceinline__ float to_float(bf16_t v) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(v.x) << 16);
}
__device__ __forceinline__ float to_float(f16_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v.x));
}
__device__ __forceinline__ float to_float(float v) { return v; }

// Round-to-nearest-even conversions (gfx950 has a hardware bf16 convert).
template <typename T> __device__ __forceinline__ T from_float(float f);
template <> __device__ __forceinline__ bf16_t from_float<bf16_t>(float f) {
  return bf16_t{__builtin_bit_cast(uint16_t, static_cast<__bf16>(f))};
}
template <> __device__ __forceinline__ f16_t from_float<f16_t>(float f) {
  return f16_t{__builtin_bit_cast(uint16_t, static_cast<_Float16>(f))};
}
template <> __device__ __forceinline__ float from_float<float>(float f) { return f; }

// Low/high 16-bit element of a packed dword, as float.
template <typename T> __device__ __forceinline__ float lo_f(uint32_t w);
template <typename T> __device__ __forceinline__ float hi_f(uint32_t w);
template <> __device__ __forceinline__ float lo_f<bf16_t>(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
template <> __device__ __forceinline__ float hi_f<bf16_t>(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
template <> __device__ __forceinline__ float lo_f<f16_t>(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
}
template <> __device__ __forceinline__ float hi_f<f16_t>(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}
// Two floats rounded to nearest-even and packed (a in the low half): one
// v_cvt_pk_{bf16,f16}_f32.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b);
template <> __device__ __forceinline__ uint32_t pack2<bf16_t>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
template <> __device__ __forceinline__ uint32_t pack2<f16_t>(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
}

// ------------------------------------------------------------ MFMA types --
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// D(16x16 f32) += A(16x32) * B(32x16). Lane i supplies A[i%16][8(i/16)..+8]
// and B[8(i/16)..+8][i%16] as 8 packed 16-bit values; lane i receives
// D[4(i/16)+r][i%16] in element r.
template <typename T> __device__ __forceinline__ f32x4 mfma_k32(u32x4 a, u32x4 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mfma_k32<bf16_t>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma_k32<f16_t>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
// D(16x16 f32) += A(16x16) * B(16x16). Lane i supplies A[i%16][4(i/16)..+4]
// and B[4(i/16)..+4][i%16]; lane i receives D[4(i/16)+r][i%16].
template <typename T> __device__ __forceinline__ f32x4 mfma_k16(u32x2 a, u32x2 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mfma_k16<bf16_t>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ f32x4 mfma_k16<f16_t>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
}

// D(32x32 f32) += A(32x16) * B(16x32). Lane i supplies A[i%32][8(i/32)..+8]
// and B[8(i/32)..+8][i%32]; lane i receives D[8(e/4) + 4(i/32) + e%4][i%32]
// in element e. On gfx950 this form has about 1.6x the throughput of the
// 16x16x32 one.
typedef float f32x16 __attribute__((ext_vector_type(16)));
template <typename T> __device__ __forceinline__ f32x16 mfma_k16x32(u32x4 a, u32x4 b, f32x16 c);
template <> __device__ __forceinline__ f32x16 mfma_k16x32<bf16_t>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                 0);
}
template <> __device__ __forceinline__ f32x16 mfma_k16x32<f16_t>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Select 16-bit halves: result = (lo16 of a | lo16 of b << 16) or the high
// halves, via v_perm_b32.
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup barrier that orders LDS accesses only: unlike __syncthreads() it
// does not wait for outstanding global loads, so prefetches stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ------------------------------------------------- global->LDS DMA loads --
// global_load_lds_dwordx4: lane l's 16 bytes land at LDS byte address
// M0 + 16 l, with no register staging. The LDS address is an operand bound
// to M0 ("{m0}"), so the compiler sets M0 itself and knows the asm reads it;
// the s_nop is the one wait state the DMA needs after an M0 write.
//
// They are written as assembly, not __builtin_amdgcn_global_load_lds, on
// purpose. With the builtin, the compiler counts the loads as pending LDS
// writes: every workgroup-scope release fence (lds_barrier) then becomes
// s_waitcnt vmcnt(0), and it drains them before the first
// ds_read_b64_tr_b16 of a block -- both empty the prefetch pipeline that
// the staging exists for -- while it places no wait at all before an
// ordinary ds_read of the staged data. So the kernels wait for these loads
// themselves (wait_vmcnt), counting them in issue order; the compiler's own
// vmcnt waits, which do not count them, are then only ever stricter than
// needed, never too weak.
//
// dma16: a per-lane 64-bit address. dma16_sv: a wave-uniform base plus a
// 32-bit lane offset (half the address registers).
//
// Hazard: a VMEM instruction that reads an SGPR written by a VALU
// instruction (v_readfirstlane_b32, v_readlane_b32, v_cmp ...) needs 5 wait
// states in between. The compiler pads that for its own instructions, not
// for the SGPR inputs of an asm statement. dma16_sv takes its base as the
// compiler computed it, which must be SALU work in SGPRs (the kernels' bases
// derive from kernel arguments and readfirstlane'd indices);
// tests/test_dma_hazards.py checks every DMA site of the built kernels for
// this. dma16_su is for a wave-uniform base the compiler may hold in VGPRs:
// it moves it to SGPRs itself and waits the 5 states.
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma16_sv(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma16_su(const void* ubase, uint32_t voff, uint32_t lds) {
  // readfirstlane returns int: each half goes through uint32_t so that the
  // low half is zero-extended, not sign-extended, into the 64-bit address.
  const uint64_t p = reinterpret_cast<uint64_t>(ubase);
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(p >> 32))));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(p))));
  const uint64_t su = (static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(lo);
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(reinterpret_cast<const void*>(su)),
               "{m0}"(lds)
               : "memory");
}

// Wait until at most N of this wave's vector memory operations are in
// flight (they complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is a 6-bit field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Inclusive scan over a wave's 64 lanes on DPP moves (no LDS round trip):
// sums within rows of 16 lanes (row shifts by 1, 2, 4, 8; a lane whose
// source lies before its row's start reads 0), then lane 15's sum added to
// row 1 and lane 47's to row 3 (row_bcast:15), then lane 31's to rows 2
// and 3 (row_bcast:31). These lane mappings were checked on the GPU. Every
// lane of the wave must take part.
template <int CTRL, int ROWS, bool BC>
__device__ __forceinline__ uint32_t dpp32(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, ROWS, 0xf, BC));
}
template <int CTRL, int ROWS, bool BC>
__device__ __forceinline__ uint64_t dpp64(uint64_t x) {
  const uint32_t lo = dpp32<CTRL, ROWS, BC>(static_cast<uint32_t>(x));
  const uint32_t hi = dpp32<CTRL, ROWS, BC>(static_cast<uint32_t>(x >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x) {
  x += dpp32<0x111, 0xf, true>(x);
  x += dpp32<0x112, 0xf, true>(x);
  x += dpp32<0x114, 0xf, true>(x);
  x += dpp32<0x118, 0xf, true>(x);
  x += dpp32<0x142, 0xa, false>(x);
  x += dpp32<0x143, 0xc, false>(x);
  return x;
}
__device__ __forceinline__ uint64_t wave_scan_u64(uint64_t x) {
  x += dpp64<0x111, 0xf, true>(x);
  x += dpp64<0x112, 0xf, true>(x);
  x += dpp64<0x114, 0xf, true>(x);
  x += dpp64<0x118, 0xf, true>(x);
  x += dpp64<0x142, 0xa, false>(x);
  x += dpp64<0x143, 0xc, false>(x);
  return x;
}

// The value held by lane (lane ^ J), for J a power of two below 64, without
// an LDS round trip: quad permutes [1,0,3,2] and [2,3,0,1] for 1 and 2, a
// row rotation by 8 for 8, rotations by 4 and 12 with a per-lane choice for
// 4, and the half-row and half-wave swaps (v_permlane16_swap,
// v_permlane32_swap, whose second result is the partner's value in the
// lower half and whose first is it in the upper half) for 16 and 32. These
// lane mappings were checked on the GPU. Every lane of the wave must take
// part.
template <int J>
__device__ __forceinline__ uint32_t xor_lane32(uint32_t v, int lane) {
  if constexpr (J == 1) {
    return dpp32<0xB1, 0xf, false>(v);
  } else if constexpr (J == 2) {
    return dpp32<0x4E, 0xf, false>(v);
  } else if constexpr (J == 4) {
    // (row_ror:n: lane l reads lane (l - n) mod 16 of its row.)
    const uint32_t up = dpp32<0x12C, 0xf, false>(v), down = dpp32<0x124, 0xf, false>(v);
    return (lane & 4) ? down : up;
  } else if constexpr (J == 8) {
    return dpp32<0x128, 0xf, false>(v);
  } else if constexpr (J == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else {
    static_assert(J == 32, "xor_lane32: J in {1, 2, 4, 8, 16, 32}");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? r[0] : r[1];
  }
}
template <int J>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v, int lane) {
  const uint32_t lo = xor_lane32<J>(static_cast<uint32_t>(v), lane);
  const uint32_t hi = xor_lane32<J>(static_cast<uint32_t>(v >> 32), lane);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

}  // namespace tsa
