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
#include <cstdlib>
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

// ---------------------------------------------------------------------------
// Wide persistent prefill: head_dim 128, bf16/f16, GQA groups of a multiple
// of 4 q-heads per kv head. A work item is (64 queries, sequence, kv head,
// group of 4 q-heads); the workgroup's 4 waves take its 4 q-heads, wave w
// the item's 64 queries of q-head w as two 32-query halves (tiles 0 and 1).
// One workgroup runs per CU and each wave has a SIMD to itself, so it can
// hold both halves' state in the whole register file: every K and V operand
// read from LDS feeds two MFMAs, and the two halves give each wave
// independent work to interleave. Per 32-key block j of an item, iteration j
// issues P.V of block j - 1 (16 MFMAs) and the scores of block j + 1 (16
// MFMAs) around the softmax of block j (VALU), so the matrix cores run while
// the exponentials do.
//   Scores: S^T(32 keys x 32 queries) = K Q^T over 8 16-dim steps, as in
//     varlen_prefill_gqa (lane (h, c): query c's scores of keys
//     8(e/4) + 4h + e%4).
//   Output: O^T(32 dims x 32 queries) += V^T P^T per 32-dim column tile u
//     and 16-key step s. The operands hold exactly the registers of
//     varlen_prefill_gqa's P V (an MFMA's A and B operands have the same
//     register layout, rows and columns swapped), so the V reads and the
//     P packing are unchanged; the accumulator is transposed: lane (h, c)
//     holds dims 32u + 8(e/4) + 4h + e%4 of query c. A query's rescale and
//     final 1/l are then lane-local (no cross-lane moves), and its output
//     leaves as 8-byte runs of 4 dims.
//   Staging: K/V blocks go to LDS by DMA kWidePF blocks ahead through
//     kWideNB slots (the slot ring runs on across items); each item's Q goes
//     by DMA to a per-wave LDS area when the load cursor enters the item,
//     and to registers at the item's start. Every vector load is therefore
//     an LDS DMA the compiler does not see, and the kernel counts exactly
//     how many were issued after the block it waits for.
constexpr int kWideNB = 5;            // K/V block slots (8 KB of K + 8 KB of V each)
constexpr int kWidePF = kWideNB - 2;  // DMA runs this many blocks ahead of the compute block
constexpr int kWideMaxSeqs = 2048;    // per-sequence 64-query tile counts kept in LDS

// Wait until at most n of this wave's vector memory operations are in flight
// (n wave-uniform, at most 63 is meaningful; larger n waits for 63).
__device__ __forceinline__ void wait_vmcnt_rt(int n) {
  if (n >= 32) {
    if (n >= 48) wait_vmcnt<48>();
    else if (n >= 40) wait_vmcnt<40>();
    else wait_vmcnt<32>();
  } else if (n >= 16) {
    if (n >= 24) wait_vmcnt<24>();
    else if (n >= 20) wait_vmcnt<20>();
    else wait_vmcnt<16>();
  } else if (n >= 8) {
    if (n >= 12) wait_vmcnt<12>();
    else wait_vmcnt<8>();
  } else if (n >= 4) {
    wait_vmcnt<4>();
  } else {
    wait_vmcnt<0>();
  }
}

template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void varlen_prefill_wide(
    PrefillArgs a, const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k) {
  // head_dim 128: KJ 16-dim K steps, NU 32-dim output column tiles, CPR
  // 16-byte chunks per K/V row of RB bytes.
  constexpr int KJ = 8, NU = 4, CPR = 16, RB = 256, BLKB = 32 * RB;
  constexpr int NB = kWideNB, PF = kWidePF;
  constexpr int VOFF = NB * BLKB;          // V slots after the K slots
  constexpr int QOFF = 2 * NB * BLKB;      // per-wave Q areas: 2 tiles x 8 steps x 1 KB
  constexpr int QWB = 16 * 1024;
  constexpr int COFF = QOFF + 4 * QWB;     // per-sequence 64-query tile counts
  constexpr int SMEM = COFF + kWideMaxSeqs * 2;
  constexpr float kRescale = 8.0f;
  __shared__ __align__(16) char smem[SMEM];
  uint16_t* const nqt_s = reinterpret_cast<uint16_t*>(smem + COFF);

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nseq = a.nseq;
  const int HG = a.G / 4;                  // q-head groups per kv head
  const int HH = a.Hkv * HG;               // items per (sequence, query tile)
  const float cs = a.scale_log2;

  // ---- Items, heaviest (latest) query tiles first: level Q holds tile Q of
  // every sequence that has one, in sequence order, (kv head, head group)
  // fastest. Workgroup w takes items w, w + grid, ...
  for (int b = tid; b < nseq; b += 256) {
    int64_t qs, ql;
    seq_range(cu_q, a.cuq_s, b, a.total_q, qs, ql);
    nqt_s[b] = static_cast<uint16_t>((ql + 63) / 64);
  }
  __syncthreads();
  auto items_above = [&](int Q) {
    int sum = 0;
    for (int b = lane; b < nseq; b += 64) sum += max(0, static_cast<int>(nqt_s[b]) - Q - 1);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
    return __builtin_amdgcn_readfirstlane(sum) * HH;
  };
  int qt_max = 0;
  for (int b = lane; b < nseq; b += 64) qt_max = max(qt_max, static_cast<int>(nqt_s[b]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) qt_max = max(qt_max, __shfl_xor(qt_max, off, 64));
  qt_max = __builtin_amdgcn_readfirstlane(qt_max);
  const int n_items = items_above(-1);

  struct Item {
    int q0, q_len, k_len, nblk;
    const T* qb;  // this wave's q-head column of the sequence's queries
    const T* kb;
    const T* vb;
    T* ob;
  };
  auto resolve = [&](int i, Item& it) {
    int lo = 0, hi = qt_max - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (items_above(mid) <= i) hi = mid; else lo = mid + 1;
    }
    const int Q = lo;
    const int r = i - items_above(Q);
    int rank = r / HH;
    const int hh = r - rank * HH;
    const int kvh = hh / HG, hg = hh - kvh * HG;
    int b = 0;
    for (int base = 0; base < nseq; base += 64) {
      const int bb = base + lane;
      const uint64_t msk = __ballot(bb < nseq && static_cast<int>(nqt_s[bb]) > Q);
      const int cnt = __builtin_popcountll(msk);
      if (rank < cnt) {
        uint64_t mm = msk;
        for (int k = 0; k < rank; ++k) mm &= mm - 1;
        b = base + __builtin_ctzll(mm);
        break;
      }
      rank -= cnt;
    }
    b = __builtin_amdgcn_readfirstlane(b);
    int64_t qs, ql, ks, kl;
    seq_range(cu_q, a.cuq_s, b, a.total_q, qs, ql);
    seq_range(cu_k, a.cuk_s, b, a.total_k, ks, kl);
    it.q_len = static_cast<int>(ql);
    it.k_len = static_cast<int>(kl);
    it.q0 = Q * 64;
    const int q_last = it.q0 + 64 < it.q_len ? it.q0 + 64 : it.q_len;
    const int kend = a.causal ? (it.k_len < q_last ? it.k_len : q_last) : it.k_len;
    it.nblk = (kend + 31) / 32;
    const int head = kvh * a.G + hg * 4 + wave;
    it.qb = static_cast<const T*>(a.q) + qs * a.q_st + head * a.q_sh;
    it.kb = static_cast<const T*>(a.k) + ks * a.k_st + kvh * a.k_sh;
    it.vb = static_cast<const T*>(a.v) + ks * a.v_st + kvh * a.v_sh;
    it.ob = static_cast<T*>(a.out) + qs * a.o_st + head * a.o_sh;
  };

  // ---- LDS layout of a K/V block: 32 rows of RB bytes, the 16-byte chunk
  // ch of row r at position ch ^ swz(r) (varlen_prefill_gqa's layout).
  auto swz = [](int r) { return ((r & 3) << 2) | ((r >> 2) & 3); };
  typedef __attribute__((address_space(3))) void lds_void;
  const uint32_t smem_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)smem));
  // DMA of a block: waves 0, 1 move K rows 0-15 / 16-31, waves 2, 3 the V
  // rows; 4 loads of 4 rows (1 KB) each. Lane l of load i fetches the chunk
  // that belongs at row R0 + l / 16, position l % 16.
  const bool k_wave = wave < 2;
  const int row0w = (wave & 1) * 16;
  const int64_t st_b = (k_wave ? a.k_st : a.v_st) * static_cast<int64_t>(sizeof(T));
  const int lrow = lane / CPR;
  auto lane_chunk = [&](int i) { return (lane % CPR) ^ swz(row0w + 4 * i + lrow); };
  uint32_t doff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) doff[i] = static_cast<uint32_t>(lrow * st_b) + 16u * lane_chunk(i);
  auto dma_block = [&](const Item& it, int blk, int slot) __attribute__((always_inline)) {
    const int key0 = blk * 32 + row0w;
    const uint32_t lds0 = smem_lds + (k_wave ? 0 : VOFF) + slot * BLKB + row0w * RB;
    const char* gbase = reinterpret_cast<const char*>(k_wave ? it.kb : it.vb);
    if (key0 + 16 <= it.k_len) {
      const char* src = gbase + key0 * st_b;
#pragma unroll
      for (int i = 0; i < 4; ++i) dma16_su(src + i * 4 * st_b, doff[i], lds0 + i * 1024);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = min(key0 + 4 * i + lrow, it.k_len - 1);
        dma16(gbase + key * st_b + 16 * lane_chunk(i), lds0 + i * 1024);
      }
    }
  };
  // DMA of this wave's Q for an item: 16 loads; load (t, jj) holds, in lane
  // (h, c), query q0 + 32t + c's dims 16jj + 8h..+8 (rows past q_len repeat
  // the last row; their outputs are never stored).
  const uint32_t q_lds = smem_lds + QOFF + wave * QWB;
  auto dma_q = [&](const Item& it) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int row = min(it.q0 + 32 * t + c, it.q_len - 1);
      const T* src = it.qb + static_cast<int64_t>(row) * a.q_st + 8 * h;
#pragma unroll
      for (int jj = 0; jj < KJ; ++jj) dma16(src + 16 * jj, q_lds + (t * KJ + jj) * 1024);
    }
  };
  u32x4 qop[2][KJ];
  auto read_q = [&]() {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int jj = 0; jj < KJ; ++jj)
        qop[t][jj] = *reinterpret_cast<const u32x4*>(smem + QOFF + wave * QWB + (t * KJ + jj) * 1024 + 16 * lane);
  };

  // K operands of the block in slot ks: lane (h, c) reads key c, dims
  // 16jj + 8h..+8 (chunk 2jj + h at position (2jj + h) ^ swz(c)).
  const int ka = c * RB + 16 * (h ^ swz(c));
  u32x4 kop[KJ];
  auto kread = [&](int ks) {
    const int kb = ks * BLKB + ka;
#pragma unroll
    for (int jj = 0; jj < KJ; ++jj) kop[jj] = *reinterpret_cast<const u32x4*>(smem + (kb ^ (32 * jj)));
  };
  // V operands (the same transposed reads as varlen_prefill_gqa's P.V).
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  int vofs[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int jl = c & 15, r = 4 * h + (jl >> 2), ch = 4 * u + 2 * (c >> 4) + ((jl & 3) >> 1);
    vofs[u] = r * RB + 16 * (ch ^ swz(r)) + 8 * (jl & 1);
  }
  u32x4 vop[2][NU];
  auto vread = [&](int vs) {
    const int vb = VOFF + vs * BLKB;
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int lo_b = vb + 16 * s2 * RB + vofs[u];
        const int hi_b = vb + 16 * s2 * RB + 8 * RB + (vofs[u] ^ 32);
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(smem + lo_b));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(smem + hi_b));
        const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
        vop[s2][u] = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
      }
  };

  // ---- Per-tile softmax state and the transposed output accumulators.
  float m[2], l[2];
  f32x16 acc[2][NU];
  u32x4 pop[2][2];
  auto reset = [&]() {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      m[t] = kNegInfP;
      l[t] = 0.f;
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[t][u][e] = 0.f;
    }
  };
  auto qk = [&](int t, f32x16& sc) {
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = 0.f;
#pragma unroll
    for (int jj = 0; jj < KJ; ++jj) sc = mfma_k16x32<T>(kop[jj], qop[t][jj], sc);
  };
  // Masking (only the blocks that reach a sequence's end or, causal, pass
  // the tile's first query), the running max and the rare rescale; then
  // p = 2^(s cs - m) in fp32 (summed into l), packed to the P operands.
  auto softmax = [&](const Item& it, int t, f32x16& sc, int blk) {
    const int kb0 = blk * 32, qt0 = it.q0 + 32 * t;
    if (kb0 + 32 > it.k_len || (a.causal && kb0 + 31 > qt0)) {
      const int qq = qt0 + c;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int kk = kb0 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (!(kk < it.k_len && (!a.causal || kk <= qq))) sc[e] = kNegInfP;
      }
    }
    float tmax = kNegInfP;
#pragma unroll
    for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, sc[e]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float mt = tmax * cs;
    if (__any(mt > m[t] + kRescale)) {
      const float m_new = fmaxf(m[t], mt);
      const float alpha = m_new == kNegInfP ? 1.f : fast_exp2(m[t] - m_new);
      l[t] *= alpha;
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[t][u][e] *= alpha;
      m[t] = m_new;
    }
    const float mm = m[t] == kNegInfP ? 0.f : m[t];
    float p[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      p[e] = fast_exp2(fmaf(sc[e], cs, -mm));
      l[t] += p[e];
    }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
      pop[t][s2] = u32x4{pack2<T>(p[8 * s2], p[8 * s2 + 1]), pack2<T>(p[8 * s2 + 2], p[8 * s2 + 3]),
                         pack2<T>(p[8 * s2 + 4], p[8 * s2 + 5]), pack2<T>(p[8 * s2 + 6], p[8 * s2 + 7])};
  };
  auto pv = [&]() {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[t][u] = mfma_k16x32<T>(vop[s2][u], pop[t][s2], acc[t][u]);
  };
  // The item's output: O^T / l, lane (h, c) storing query c's 4-dim runs.
  auto store_out = [&](const Item& it) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float rl = 1.f / (l[t] + __shfl_xor(l[t], 32, 64));
      const int row = it.q0 + 32 * t + c;
      if (row < it.q_len) {
        T* orow = it.ob + static_cast<int64_t>(row) * a.o_st + 4 * h;
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
          for (int e4 = 0; e4 < 4; ++e4) {
            const u32x2 w = u32x2{pack2<T>(acc[t][u][4 * e4] * rl, acc[t][u][4 * e4 + 1] * rl),
                                  pack2<T>(acc[t][u][4 * e4 + 2] * rl, acc[t][u][4 * e4 + 3] * rl)};
            *reinterpret_cast<u32x2*>(orow + 32 * u + 8 * e4) = w;
          }
      }
    }
  };

  // ---- The block stream. Compute runs over the workgroup's items in
  // order; the load cursor (item L, block lj; global block gl) issues each
  // block's DMA kWidePF blocks ahead. It may enter the next item (issuing
  // that item's Q first) but not the one after, and only once the current
  // item's Q has been read to registers: the Q area holds one item.
  // Loads per wave: a block is 4 DMA instructions, an item's Q 16.
  int idx = blockIdx.x;
  if (idx >= n_items) return;
  Item X, N;
  resolve(idx, X);
  int nidx = idx + static_cast<int>(gridDim.x);
  bool have_n = false;     // N resolved (the load cursor entered it)
  int gl = 0, lj = 0;      // next block to issue: global index, block of the load item
  bool l_in_n = false;     // the load cursor is in N (else in X)
  bool q_free = false;     // X's Q has left the Q area for registers: N's may be loaded
  int q_after = -1;        // global block index whose DMA directly follows the last Q group
  int gb = 0;              // global index of the compute block
  int slot_l = 0;          // slot of block gl
  // DMA issue for one block of the load cursor, if it may advance.
  auto issue = [&]() __attribute__((always_inline)) {
    if (!l_in_n && lj == X.nblk) {  // X fully issued: enter the next item
      if (!have_n || !q_free) return false;
      l_in_n = true;
      lj = 0;
      dma_q(N);
      q_after = gl;
      if (N.nblk == 0) return false;
    } else if (l_in_n && lj == N.nblk) {
      return false;  // would enter the item after N
    }
    if (l_in_n) dma_block(N, lj, slot_l);
    else dma_block(X, lj, slot_l);
    ++lj;
    ++gl;
    slot_l = slot_l + 1 == NB ? 0 : slot_l + 1;
    return true;
  };
  // Loads issued after block g's group: 4 per later block, 16 for a Q group
  // issued after it.
  auto wait_block = [&](int g) __attribute__((always_inline)) {
    int n = 4 * (gl - 1 - g);
    if (q_after > g && q_after <= gl) n += 16;
    wait_vmcnt_rt(n);
  };

  if (nidx < n_items) {
    resolve(nidx, N);
    have_n = true;
  }
  dma_q(X);
  q_after = 0;
  for (int i = 0; i < PF && issue(); ++i) {
  }
  while (true) {
    reset();
    const int nb = X.nblk;
    // X's Q is in its area (its group precedes block 0's); read it.
    if (nb > 0) wait_block(gb); else wait_vmcnt<0>();
    lds_barrier();
    read_q();
    q_free = true;
    f32x16 sc[2];
    int slot_c = gb % NB;
    if (nb > 0) {
      kread(slot_c);
      qk(0, sc[0]);
      qk(1, sc[1]);
    }
    // Block j: P.V of block j - 1, then each tile's softmax of block j
    // followed by that tile's scores of block j + 1 (into the same
    // registers, which the softmax has consumed): the matrix cores take P.V
    // during tile 0's softmax and tile 0's scores during tile 1's.
    for (int j = 0; j < nb; ++j) {
      const bool more = j + 1 < nb;
      if (more) wait_block(gb + 1);
      lds_barrier();
      issue();
      if (more) kread(slot_c + 1 == NB ? 0 : slot_c + 1);
      if (j > 0) {
        vread(slot_c == 0 ? NB - 1 : slot_c - 1);
        pv();
      }
      softmax(X, 0, sc[0], j);
      if (more) qk(0, sc[0]);
      softmax(X, 1, sc[1], j);
      if (more) qk(1, sc[1]);
      ++gb;
      slot_c = slot_c + 1 == NB ? 0 : slot_c + 1;
    }
    if (nb > 0) {  // P.V of the last block (its V is still in its slot)
      vread(slot_c == 0 ? NB - 1 : slot_c - 1);
      pv();
    }
    store_out(X);
    // Next item (resolved at X's start; its Q and first blocks are in flight
    // unless X's stream ended before the load cursor reached it).
    if (!have_n) break;
    if (!l_in_n) {
      dma_q(N);
      q_after = gl;
      lj = 0;
      l_in_n = true;
    }
    X = N;
    have_n = false;
    l_in_n = false;
    q_free = false;
    nidx += static_cast<int>(gridDim.x);
    if (nidx < n_items) {
      resolve(nidx, N);
      have_n = true;
    }
    // keep the load cursor kWidePF blocks ahead
    for (int i = 0; gl - gb < PF && i < PF && issue(); ++i) {
    }
  }
  wait_vmcnt<0>();
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

// TSA_PREFILL_WIDE=1 in the environment routes the calls it takes to
// varlen_prefill_wide (read once per process); otherwise they go to
// varlen_prefill_gqa.
static bool wide_enabled() {
  static const int on = [] {
    const char* e = getenv("TSA_PREFILL_WIDE");
    return (e && e[0] == '1') ? 1 : 0;
  }();
  return on != 0;
}

// The wide kernel: one workgroup per CU (its LDS allows no more).
template <typename T>
static int launch_wide(const PrefillArgs& a, hipStream_t stream) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  varlen_prefill_wide<T><<<dim3(cus), dim3(256), 0, stream>>>(a, a.cu_q, a.cu_k);
  return check_launch("tsa_varlen_prefill");
}

// The LDS-staged kernels keep 32 rows of K/V byte offsets in 32 bits, and
// per-sequence query-block counts in 16 bits (every sequence's length is at
// most total_q). Both need a positive scale (the masked-score sentinel).
constexpr int64_t kMaxStride = int64_t{1} << 24;
static bool takes_wide(const PrefillArgs& a) {
  return a.D == 128 && a.G % 4 == 0 && a.scale_log2 > 0.f && a.k_st < kMaxStride && a.v_st < kMaxStride &&
         a.nseq <= kWideMaxSeqs && a.total_q <= int64_t{65535} * 64 && wide_enabled();
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
    if (takes_wide(a)) return launch_wide<T>(a, stream);
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
  return mfma && a.D == 128 && a.G == 4 && !takes_wide(a) && takes_gqa(a);
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
