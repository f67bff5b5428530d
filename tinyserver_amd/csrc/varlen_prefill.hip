// Varlen (packed, cu_seqlens) causal prefill attention for gfx950.
//
// Reference: server/model/kernels/varlen_attention.py:8-142 -- one program per
// (32-row query block, sequence, q-head), online softmax over 32-key blocks,
// top-left causal mask q_idx >= k_idx within the sequence (:116-119),
// P cast to the V dtype before P.V (:126), l summing the fp32 P (:128-129).
//
// Three kernels, chosen per call:
//   varlen_prefill_gqa   bf16/f16, head_dim 64/128, GQA group 2, 4 or 8, up
//                        to 1024-2048 sequences: persistent workgroups, each
//                        computing (kv head, sequence, 32 queries) items with
//                        K/V staged in LDS once for the whole group, 32x32x16
//                        MFMA tiles (the main path);
//   varlen_prefill_mfma  other group sizes: 4 q-heads per workgroup, operands
//                        straight from global memory, 16x16x32 MFMA tiles;
//   varlen_prefill_generic  fp32, other head_dims or non-unit innermost
//                        strides: one wave per (query, q-head), fp32 VALU.
// Causal key blocks past a query block's last query are never visited, and
// the heaviest query blocks are computed first.
#include <cmath>
#include <type_traits>

#include "tsa_common.h"
#include "varlen_prefill_gqa.h"

namespace tsa {

template <typename T, int D>
__global__ __launch_bounds__(256) void varlen_prefill_mfma(PrefillArgs a) {
  constexpr int KJ = D / 32;
  const int qb = a.nqb - 1 - static_cast<int>(blockIdx.x);  // heaviest blocks first
  const int b = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, c = lane & 15;
  const int h = blockIdx.z * 4 + wave;
  int64_t q_start, q_len, k_start, k_len;
  seq_range(a.cu_q, a.cuq_s, b, a.total_q, q_start, q_len);
  seq_range(a.cu_k, a.cuk_s, b, a.total_k, k_start, k_len);
  const int64_t row0 = static_cast<int64_t>(qb) * 32;
  if (row0 >= q_len || h >= a.Hq) return;
  const int kvh = h / a.G;

  const T* qb_ptr = static_cast<const T*>(a.q) + q_start * a.q_st + h * a.q_sh;
  const T* kb_ptr = static_cast<const T*>(a.k) + k_start * a.k_st + kvh * a.k_sh;
  const T* vb_ptr = static_cast<const T*>(a.v) + k_start * a.v_st + kvh * a.v_sh;
  const bool v_lane = 8 * c < D;

  // Q^T operands of the two 16-row subtiles.
  u32x4 qop[2][KJ];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    const int64_t row = row0 + 16 * qs + c;
#pragma unroll
    for (int j = 0; j < KJ; ++j)
      qop[qs][j] = row < q_len ? *reinterpret_cast<const u32x4*>(qb_ptr + row * a.q_st + 8 * (g + 4 * j))
                               : u32x4{0, 0, 0, 0};
  }

  float m[2] = {kNegInfP, kNegInfP};  // running max of query (16 qs + c), log2 domain
  float l[2] = {0.f, 0.f};            // lane share of its denominator (fp32 p)
  f32x4 acc[2][8];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs)
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[qs][u] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t kend = a.causal ? (k_len < row0 + 32 ? k_len : row0 + 32) : k_len;
  for (int64_t kb0 = 0; kb0 < kend; kb0 += 32) {
    u32x4 kop[2][KJ];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int64_t key = kb0 + 16 * ks + c;
#pragma unroll
      for (int j = 0; j < KJ; ++j)
        kop[ks][j] = key < k_len ? *reinterpret_cast<const u32x4*>(kb_ptr + key * a.k_st + 8 * (g + 4 * j))
                                 : u32x4{0, 0, 0, 0};
    }
    u32x4 vrow[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t key = kb0 + (e < 4 ? 4 * g + e : 16 + 4 * g + e - 4);
      vrow[e] = (v_lane && key < k_len) ? *reinterpret_cast<const u32x4*>(vb_ptr + key * a.v_st + 8 * c)
                                        : u32x4{0, 0, 0, 0};
    }

#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      const int64_t qq = row0 + 16 * qs + c;
      float sv[2][4];
      float tmax = kNegInfP;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KJ; ++j) sc = mfma_k32<T>(kop[ks][j], qop[qs][j], sc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t kk = kb0 + 16 * ks + 4 * g + r;
          const bool ok = kk < k_len && (!a.causal || kk <= qq);
          sv[ks][r] = ok ? sc[r] * a.scale_log2 : kNegInfP;
          tmax = fmaxf(tmax, sv[ks][r]);
        }
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float m_new = fmaxf(m[qs], tmax);
      const bool fin = m_new != kNegInfP;
      if (__any(m_new > m[qs])) {
        const float alpha = fin ? fast_exp2(m[qs] - m_new) : 1.f;
        l[qs] *= alpha;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ar = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
          for (int u = 0; u < 8; ++u) acc[qs][u][r] *= ar;
        }
        m[qs] = m_new;
      }
      float p[2][4];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[ks][r] = fin ? fast_exp2(sv[ks][r] - m[qs]) : 0.f;
          l[qs] += p[ks][r];
        }
      const u32x4 pop = u32x4{pack2<T>(p[0][0], p[0][1]), pack2<T>(p[0][2], p[0][3]), pack2<T>(p[1][0], p[1][1]),
                              pack2<T>(p[1][2], p[1][3])};
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int w = u >> 1;
        u32x4 bop;
        if (u & 1) {
          bop[0] = pack_hi(vrow[0][w], vrow[1][w]);
          bop[1] = pack_hi(vrow[2][w], vrow[3][w]);
          bop[2] = pack_hi(vrow[4][w], vrow[5][w]);
          bop[3] = pack_hi(vrow[6][w], vrow[7][w]);
        } else {
          bop[0] = pack_lo(vrow[0][w], vrow[1][w]);
          bop[1] = pack_lo(vrow[2][w], vrow[3][w]);
          bop[2] = pack_lo(vrow[4][w], vrow[5][w]);
          bop[3] = pack_lo(vrow[6][w], vrow[7][w]);
        }
        acc[qs][u] = mfma_k32<T>(pop, bop, acc[qs][u]);  // O[query 16qs+4g+r][dim 8c+u]
      }
    }
  }

  T* ob_ptr = static_cast<T*>(a.out) + q_start * a.o_st + h * a.o_sh;
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    float lt = l[qs];
    lt += __shfl_xor(lt, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float lr = __shfl(lt, 4 * g + r, 64);
      const int64_t row = row0 + 16 * qs + 4 * g + r;
      if (row < q_len && v_lane) {
        T* op = ob_ptr + row * a.o_st + 8 * c;
        float vals[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) vals[u] = acc[qs][u][r] / lr;
        u32x4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = pack2<T>(vals[2 * i], vals[2 * i + 1]);
        *reinterpret_cast<u32x4*>(op) = w;
      }
    }
  }
}

// The standalone LDS-staged GQA kernel (prefill_gqa_body in
// varlen_prefill_gqa.h): the grid is as many workgroups as fit on the device.
template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void varlen_prefill_gqa(
    PrefillArgs a, const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k) {
  __shared__ __align__(16) char smem[gqa_smem_bytes<D, NW>()];
  prefill_gqa_body<T, D, NW>(a, cu_q, cu_k, smem, 0);
}

// Generic path: one wave per (query row, q-head), fp32 VALU.
template <typename T>
__global__ __launch_bounds__(64) void varlen_prefill_generic(PrefillArgs a, int64_t total_q) {
  const int64_t qi = blockIdx.x;
  const int h = blockIdx.y, lane = threadIdx.x;
  // Sequence of query token qi.
  int lo = 0, hi = a.nseq;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (a.cu_q[mid * a.cuq_s] <= qi) lo = mid; else hi = mid;
  }
  const int b = lo;
  int64_t q_start, q_len, k_start, k_len;
  seq_range(a.cu_q, a.cuq_s, b, a.total_q, q_start, q_len);
  seq_range(a.cu_k, a.cuk_s, b, a.total_k, k_start, k_len);
  if (qi < q_start || qi >= q_start + q_len) return;
  const int64_t qq = qi - q_start;
  const int kvh = h / a.G, D = a.D;
  const T* qrow = static_cast<const T*>(a.q) + qi * a.q_st + h * a.q_sh;
  const T* kb = static_cast<const T*>(a.k) + k_start * a.k_st + kvh * a.k_sh;
  const T* vb = static_cast<const T*>(a.v) + k_start * a.v_st + kvh * a.v_sh;
  const int64_t kend = a.causal ? (k_len < qq + 1 ? k_len : qq + 1) : k_len;
  constexpr int kMaxPerLane = 8;
  float acc[kMaxPerLane];
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) acc[i] = 0.f;
  float m = kNegInfP, l = 0.f;
  for (int64_t base = 0; base < kend; base += 64) {
    const int64_t key = base + lane;
    float sc = kNegInfP;
    if (key < kend) {
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot += to_float(qrow[d * a.q_sd]) * to_float(kb[key * a.k_st + d * a.k_sd]);
      sc = dot * a.scale_log2;
    }
    float cmax = sc;
    for (int off = 32; off >= 1; off >>= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, off, 64));
    const float m_new = fmaxf(m, cmax);
    const float alpha = fast_exp2(m - m_new);
    const float p = fast_exp2(sc - m_new);
    const float pr = to_float(from_float<T>(p));  // P.V in the V dtype, as the reference does
    float psum = p;
    for (int off = 32; off >= 1; off >>= 1) psum += __shfl_xor(psum, off, 64);
    l = l * alpha + psum;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) acc[i] *= alpha;
    const int n = static_cast<int>(kend - base < 64 ? kend - base : 64);
    for (int j = 0; j < n; ++j) {
      const float pj = __shfl(pr, j, 64);
      const T* vr = vb + (base + j) * a.v_st;
#pragma unroll
      for (int i = 0; i < kMaxPerLane; ++i) {
        const int d = lane + 64 * i;
        if (d < D) acc[i] += pj * to_float(vr[d * a.v_sd]);
      }
    }
    m = m_new;
  }
  T* orow = static_cast<T*>(a.out) + qi * a.o_st + h * a.o_sh;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int d = lane + 64 * i;
    if (d < D) orow[d * a.o_sd] = from_float<T>(acc[i] / l);
  }
}

// The persistent kernel runs as many workgroups as fit on the device at once
// (the occupancy the compiler's resources allow, times the CU count).
template <typename T, int D, int NW>
static int launch_persistent(const PrefillArgs& a, hipStream_t stream) {
  static int per_cu = 0;
  if (per_cu == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, varlen_prefill_gqa<T, D, NW>, 64 * NW, 0) != hipSuccess || n <= 0)
      n = 1;
    per_cu = n;
  }
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  varlen_prefill_gqa<T, D, NW><<<dim3(per_cu * cus), dim3(64 * NW), 0, stream>>>(a, a.cu_q, a.cu_k);
  return check_launch("tsa_varlen_prefill");
}

// The LDS-staged kernels keep 32 rows of K/V byte offsets in 32 bits, and
// per-sequence query-block counts in 16 bits (every sequence's length is at
// most total_q). Both need a positive scale (the masked-score sentinel).
constexpr int64_t kMaxStride = int64_t{1} << 24;
// varlen_prefill_w64 (varlen_prefill_w64.hip): head_dim 128, groups of a
// multiple of 4 q-heads, its per-sequence tile counts in LDS, 16-bit tile
// counts.
static bool takes_w64(const PrefillArgs& a) {
  return a.D == 128 && a.G % 4 == 0 && a.scale_log2 > 0.f && a.q_st < kMaxStride && a.k_st < kMaxStride &&
         a.v_st < kMaxStride &&
         a.nseq <= kW64MaxSeqsHost && a.total_q <= int64_t{65535} * 64 && a.Hkv * (a.G / 4) < 32768 &&
         prefill_w64_enabled();
}
static bool takes_gqa(const PrefillArgs& a) {
  return (a.G == 2 || a.G == 4 || a.G == 8) && a.scale_log2 > 0.f && a.k_st < kMaxStride && a.v_st < kMaxStride &&
         a.nseq <= max_persist_seqs(a.G) && a.total_q <= int64_t{65535} * 32;
}

template <typename T>
static int launch_prefill(PrefillArgs& a, bool mfma, int64_t total_q, int64_t max_seqlen_q, hipStream_t stream) {
  if (a.nseq == 0 || a.Hq == 0 || total_q == 0) return TSA_OK;
  if (!mfma) {
    varlen_prefill_generic<T><<<dim3(total_q, a.Hq), dim3(64), 0, stream>>>(a, total_q);
    return check_launch("tsa_varlen_prefill");
  }
  if constexpr (sizeof(T) == 2) {
    if (takes_w64(a)) return prefill_w64_launch(a, sizeof(T) == 2 && std::is_same<T, bf16_t>::value, stream);
    if (takes_gqa(a)) {
      if (a.D == 128) {
        if (a.G == 2) return launch_persistent<T, 128, 2>(a, stream);
        if (a.G == 4) return launch_persistent<T, 128, 4>(a, stream);
        return launch_persistent<T, 128, 8>(a, stream);
      }
      if (a.G == 2) return launch_persistent<T, 64, 2>(a, stream);
      if (a.G == 4) return launch_persistent<T, 64, 4>(a, stream);
      return launch_persistent<T, 64, 8>(a, stream);
    } else {
      a.nqb = static_cast<int32_t>((max_seqlen_q + 31) / 32);
      if (a.nqb == 0) return TSA_OK;
      const dim3 grid(a.nqb, a.nseq, (a.Hq + 3) / 4);
      if (a.D == 128) varlen_prefill_mfma<T, 128><<<grid, dim3(256), 0, stream>>>(a);
      else varlen_prefill_mfma<T, 64><<<grid, dim3(256), 0, stream>>>(a);
    }
  }
  return check_launch("tsa_varlen_prefill");
}

}  // namespace tsa

using namespace tsa;

namespace tsa {

int prefill_prepare(const tsa_view* out, const tsa_view* q, const tsa_view* k, const tsa_view* v,
                    const tsa_view* cu_seqlens_q, const tsa_view* cu_seqlens_k, int64_t max_seqlen_q,
                    int64_t max_seqlen_k, int32_t causal, double softmax_scale, PrefillArgs& a, bool& mfma) {
  TSA_REQUIRE(view_ok(q, 3) && view_ok(k, 3) && view_ok(v, 3), "q, k, v must be 3D tensors");
  TSA_REQUIRE(view_ok(out, 3), "out must be a 3D tensor shaped like q");
  TSA_REQUIRE(view_ok(cu_seqlens_q, 1) && view_ok(cu_seqlens_k, 1) && cu_seqlens_q->dtype == TSA_I32 &&
                  cu_seqlens_k->dtype == TSA_I32,
              "cu_seqlens_q and cu_seqlens_k must be 1D int32 tensors");
  TSA_REQUIRE(cu_seqlens_q->size[0] == cu_seqlens_k->size[0] && cu_seqlens_q->size[0] >= 1,
              "cu_seqlens_q and cu_seqlens_k must have batch + 1 entries each");
  const int dt = q->dtype;
  TSA_REQUIRE(is_float_dtype(dt) && k->dtype == dt && v->dtype == dt && out->dtype == dt,
              "q, k, v and out must share one floating dtype");
  for (int d = 0; d < 3; ++d) TSA_REQUIRE(out->size[d] == q->size[d], "out must have q's shape");
  for (int d = 0; d < 3; ++d) TSA_REQUIRE(v->size[d] == k->size[d], "k and v must have the same shape");
  const int64_t Hq = q->size[1], Hkv = k->size[1], D = q->size[2];
  TSA_REQUIRE(k->size[2] == D, "k head_dim %lld != q head_dim %lld", (long long)k->size[2], (long long)D);
  TSA_REQUIRE(Hkv > 0 && Hq % Hkv == 0, "num_heads_q must be divisible by num_heads_k for GQA");
  TSA_REQUIRE(max_seqlen_q >= 0 && max_seqlen_k >= 0, "max_seqlen must be non-negative");
  TSA_UNSUPPORTED(D <= 512, "head_dim %lld > 512 is not implemented", (long long)D);

  a = PrefillArgs{};
  a.out = out->data; a.q = q->data; a.k = k->data; a.v = v->data;
  a.cu_q = static_cast<const int32_t*>(cu_seqlens_q->data);
  a.cu_k = static_cast<const int32_t*>(cu_seqlens_k->data);
  a.cuq_s = cu_seqlens_q->stride[0]; a.cuk_s = cu_seqlens_k->stride[0];
  a.q_st = q->stride[0]; a.q_sh = q->stride[1]; a.q_sd = q->stride[2];
  a.k_st = k->stride[0]; a.k_sh = k->stride[1]; a.k_sd = k->stride[2];
  a.v_st = v->stride[0]; a.v_sh = v->stride[1]; a.v_sd = v->stride[2];
  a.o_st = out->stride[0]; a.o_sh = out->stride[1]; a.o_sd = out->stride[2];
  a.nseq = static_cast<int32_t>(cu_seqlens_q->size[0] - 1);
  a.Hq = static_cast<int32_t>(Hq); a.Hkv = static_cast<int32_t>(Hkv);
  a.G = static_cast<int32_t>(Hq / Hkv); a.D = static_cast<int32_t>(D);
  a.total_q = q->size[0]; a.total_k = k->size[0];
  a.causal = causal ? 1 : 0;
  a.scale_log2 = static_cast<float>(softmax_scale * 1.4426950408889634);
  mfma = (dt == TSA_BF16 || dt == TSA_F16) && (D == 64 || D == 128) && rows_vec16(q) && rows_vec16(k) &&
         rows_vec16(v) && rows_vec16(out);
  return TSA_OK;
}

int prefill_launch(PrefillArgs& a, bool mfma, int dtype, int64_t max_seqlen_q, hipStream_t stream) {
  switch (dtype) {
    case TSA_BF16: return launch_prefill<bf16_t>(a, mfma, a.total_q, max_seqlen_q, stream);
    case TSA_F16: return launch_prefill<f16_t>(a, mfma, a.total_q, max_seqlen_q, stream);
    case TSA_F32: return launch_prefill<float>(a, false, a.total_q, max_seqlen_q, stream);
  }
  set_error("unsupported dtype");
  return TSA_ERR_UNSUPPORTED;
}

bool prefill_takes_gqa4(const PrefillArgs& a, bool mfma) {
  return mfma && a.D == 128 && a.G == 4 && takes_gqa(a);
}

}  // namespace tsa

extern "C" int tsa_varlen_prefill(const tsa_view* out, const tsa_view* q, const tsa_view* k, const tsa_view* v,
                                  const tsa_view* cu_seqlens_q, const tsa_view* cu_seqlens_k, int64_t max_seqlen_q,
                                  int64_t max_seqlen_k, int32_t causal, double softmax_scale, void* stream) {
  PrefillArgs a;
  bool mfma = false;
  if (int rc = prefill_prepare(out, q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal,
                               softmax_scale, a, mfma))
    return rc;
  return prefill_launch(a, mfma, q->dtype, max_seqlen_q, static_cast<hipStream_t>(stream));
}
