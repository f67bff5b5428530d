// Varlen causal prefill with 64 query rows per wave: varlen_prefill_w64.
//
// Reference: server/model/kernels/varlen_attention.py:8-142 (per query
// block, an fp32 online softmax over 32-key blocks, top-left causal mask
// :116-119, P cast to the V dtype before P.V :126, l summing the fp32 P
// :128-129). Here l sums the 16-bit P that P.V takes (in fp32, on the
// matrix cores), so numerator and denominator weigh the same P: the
// output moves by a relative ~2^-9 / sqrt(keys) at most against summing
// the fp32 P, well inside the attention tolerance.
//
// head_dim 128, bf16/f16, GQA groups of a multiple of 4 q-heads. A work item
// is (sequence, kv head, group of 4 q-heads, 64 queries); the workgroup's 4
// waves take the group's 4 q-heads, so all of them read the same K/V blocks,
// and wave w holds the item's 64 queries of its q-head as two 32-query
// tiles. One workgroup runs per CU, one wave per SIMD: the softmax state,
// both tiles' scores and their output accumulators (2 x 64 fp32 per lane,
// which the compiler keeps in AGPRs) fit the whole register file.
//
// Every K and V operand read from LDS, every DMA instruction, barrier and
// loop step serves both tiles. The tiles run half an iteration apart, so one
// tile's softmax (VALU) always has the other tile's MFMAs to overlap:
//   H0(j): softmax of tile 0, block j     | QK of tile 1, block j; P.V of tile 1, block j-1
//   H1(j): softmax of tile 1, block j     | QK of tile 0, block j+1; P.V of tile 0, block j
// A half's MFMAs depend only on the previous half's results. K(j + 1) and
// V(j) are read from LDS during H0(j), into the registers the half's MFMAs
// have just consumed, and used in H1(j) (K(j + 1) again in H0(j + 1), V(j)
// again in H0(j + 1)), so each K/V byte leaves LDS once per wave.
//
// Operand layouts are those of varlen_prefill_gqa (lane (h, c) = (lane / 32,
// lane % 32)):
//   S^T(32 keys x 32 queries) = K Q^T on v_mfma_f32_32x32x16 over 8 16-dim
//     steps; lane (h, c) gets query c's scores of keys 8(e/4) + 4h + e%4;
//   O^T(32 dims x 32 queries) += V^T P^T over two 16-key steps; the P
//     operand is the lane's own score accumulators, packed; V comes from
//     ds_read_b64_tr_b16. Lane (h, c) accumulates query c's outputs, so the
//     rescale and 1/l are lane-local.
// K/V blocks and each item's Q go from global memory straight into LDS
// (global_load_lds_dwordx4); the loads of block step s (K(s + 1), V(s)) run
// kW64A steps ahead through kW64Slots slots.
#pragma once

#include <type_traits>

#include "varlen_prefill_gqa.h"

namespace tsa {

constexpr int kW64Slots = 4;               // K/V block slots: 8 KB of K + 8 KB of V each
constexpr int kW64A = kW64Slots - 1;       // block steps the loads run ahead
constexpr int kW64QArea = 16 * 1024;       // per-wave Q area: 2 tiles x 8 dim steps x 1 KB
constexpr int kW64MaxSeqs = 2048;          // per-sequence 64-query tile counts kept in LDS
constexpr int kW64OutStage = 32 * 128;     // per-wave output staging: 32 rows of 128 bytes
constexpr int w64_smem_bytes() {
  return 2 * kW64Slots * 8192 + 4 * kW64QArea + 4 * kW64OutStage + kW64MaxSeqs * 2 + kPlanItems * 6 * 4 +
         kPlanLevels * 4;
}

// Register homes. The output accumulators (2 x 64 fp32 per lane) live in
// AGPRs, where the P.V MFMAs (builtins) accumulate them; Q lives in AGPRs
// too (the score MFMAs' B operand). The scores must land in VGPRs, where the
// softmax reads them, so the score MFMA is inline assembly with a VGPR
// destination; and the rare rescale of the accumulators is assembly that
// reads, scales and rewrites the AGPRs in place, so the compiler never
// needs them in VGPRs. The compiler's hazard recognizer does not look into
// assembly, so the wait states around it are placed here:
//   * the scores of an 8-pass XDL op need 11 wait states before a VALU
//     reads them: softmax_max begins with kXdlToValuNops;
//   * the rescale reads accumulators that P.V MFMAs wrote (11 wait states)
//     and its writes must precede the next P.V's read of them as SrcC by 2:
//     it is wrapped in the same waits;
//   * the score MFMA's A and B operands come from ds_read (waited for by
//     the compiler's counters); its SrcC chain is the exact register range
//     the previous score MFMA wrote, which needs no wait state.
template <typename V> __device__ __forceinline__ void in_agpr(V& x) { asm volatile("" : "+a"(x)); }
__device__ __forceinline__ void xdl_to_valu_nops() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }
template <typename T> __device__ __forceinline__ void mfma_qk_v(f32x16& d, u32x4 a, u32x4 b, bool first);
template <> __device__ __forceinline__ void mfma_qk_v<bf16_t>(f32x16& d, u32x4 a, u32x4 b, bool first) {
  if (first) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "a"(b));
  else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "a"(b));
}
template <> __device__ __forceinline__ void mfma_qk_v<f16_t>(f32x16& d, u32x4 a, u32x4 b, bool first) {
  if (first) asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "a"(b));
  else asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "a"(b));
}
// x (16 fp32 in AGPRs) *= alpha, in place: each element is read to a VGPR,
// scaled and written back inside the assembly, so the compiler never moves
// the accumulators out of their AGPRs (a C++ multiply makes it hoist the
// copies into the hot loop).
__device__ __forceinline__ void scale_agpr16(f32x16& x, float alpha) {
  float e[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) e[i] = x[i];
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    float tmp;
    asm volatile(
        "v_accvgpr_read_b32 %4, %0\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %0, %4\n\t"
        "v_accvgpr_read_b32 %4, %1\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %1, %4\n\t"
        "v_accvgpr_read_b32 %4, %2\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %2, %4\n\t"
        "v_accvgpr_read_b32 %4, %3\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %3, %4"
        : "+a"(e[i]), "+a"(e[i + 1]), "+a"(e[i + 2]), "+a"(e[i + 3]), "=&v"(tmp)
        : "v"(alpha));
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = e[i];
  in_agpr(x);
}

// Elements 0 and 1 of x (4 fp32 in AGPRs) *= a0 and a1, in place, as
// scale_agpr16 does. Elements 2 and 3 are left alone, but pass through the
// assembly as AGPR operands too: otherwise the compiler keeps copies of
// them in VGPRs across the branch that holds this.
__device__ __forceinline__ void scale_agpr2(f32x4& x, float a0, float a1) {
  float e[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) e[i] = x[i];
  float tmp;
  asm volatile(
      "v_accvgpr_read_b32 %4, %0\n\tv_mul_f32 %4, %4, %5\n\tv_accvgpr_write_b32 %0, %4\n\t"
      "v_accvgpr_read_b32 %4, %1\n\tv_mul_f32 %4, %4, %6\n\tv_accvgpr_write_b32 %1, %4"
      : "+a"(e[0]), "+a"(e[1]), "+a"(e[2]), "+a"(e[3]), "=&v"(tmp)
      : "v"(a0), "v"(a1));
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = e[i];
  in_agpr(x);
}

template <typename T>
__device__ __forceinline__ void prefill_w64_body(PrefillArgs a, const int32_t* __restrict__ cu_q,
                                                 const int32_t* __restrict__ cu_k, char* smem) {
  constexpr int KJ = 8, NU = 4, CPR = 16, RB = 256, BLKB = 32 * RB;
  constexpr int NB = kW64Slots, A = kW64A;
  constexpr int RPI = 4;                    // K/V rows per 1 KB load instruction
  constexpr int IPW = 4;                    // load instructions per wave per block step
  constexpr int VOFF = NB * BLKB;           // V slots after the K slots
  constexpr int QOFF = 2 * NB * BLKB;       // per-wave Q areas
  constexpr int OOFF = QOFF + 4 * kW64QArea;  // per-wave output staging
  constexpr int COFF = OOFF + 4 * kW64OutStage;  // per-sequence 64-query tile counts
  constexpr int PLOFF = COFF + kW64MaxSeqs * 2;
  constexpr int LVOFF = PLOFF + kPlanItems * 6 * 4;
  static_assert(LVOFF + kPlanLevels * 4 == w64_smem_bytes(), "LDS layout and its size agree");
  constexpr float kRescale = 8.0f;
  constexpr int kInFlight = (A - 1) * IPW;  // loads of the later steps, still in flight at a step's wait
  uint16_t* const nqt_s = reinterpret_cast<uint16_t*>(smem + COFF);
  int32_t* const plan_s = reinterpret_cast<int32_t*>(smem + PLOFF);
  int32_t* const lev_s = reinterpret_cast<int32_t*>(smem + LVOFF);

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nseq = a.nseq;
  const int HG = a.G / 4;      // q-head groups per kv head
  const int HH = a.Hkv * HG;   // items per (sequence, query tile)
  const float cs = a.scale_log2;  // > 0 on this path

  // ---- Work items (64-query tile, sequence, kv head, head group), heaviest
  // tiles first: level Q holds tile Q of every sequence that has one, in
  // sequence order, (kv head, head group) fastest. Workgroups take them in
  // rounds (item_of), as varlen_prefill_gqa does.
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
    int jm;     // first block that needs a mask
    int kfull;  // rows below min(k_len, 32 nblk) load without clamping
    const T* qb;  // this wave's q-head column of the sequence's queries
    const T* kb;
    const T* vb;
    T* ob;
  };
  auto fill_item = [&](Item& it, int b, int hh, int Q, int64_t qs, int64_t ql, int64_t ks, int64_t kl) {
    const int kvh = hh / HG, hg = hh - kvh * HG;
    it.q_len = static_cast<int>(ql);
    it.k_len = static_cast<int>(kl);
    it.q0 = Q * 64;
    const int q_last = it.q0 + 64 < it.q_len ? it.q0 + 64 : it.q_len;
    const int kend = a.causal ? (it.k_len < q_last ? it.k_len : q_last) : it.k_len;
    it.nblk = (kend + 31) / 32;
    it.jm = a.causal ? min(it.k_len / 32, 2 * Q) : it.k_len / 32;
    it.kfull = min(it.k_len, it.nblk * 32);
    const int head = kvh * a.G + hg * 4 + wave;
    it.qb = static_cast<const T*>(a.q) + qs * a.q_st + head * a.q_sh;
    it.kb = static_cast<const T*>(a.k) + ks * a.k_st + kvh * a.k_sh;
    it.vb = static_cast<const T*>(a.v) + ks * a.v_st + kvh * a.v_sh;
    it.ob = static_cast<T*>(a.out) + qs * a.o_st + head * a.o_sh;
    (void)b;
  };
  // Item i -> level Q (the smallest with items_above(Q) <= i), then the
  // sequence of rank (i - items_above(Q)) / HH among those with nqt > Q.
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
    fill_item(it, b, hh, Q, qs, ql, ks, kl);
  };
  // The item plan (as varlen_prefill_gqa's): for at most kPlanSeqs sequences
  // and kPlanLevels tile levels, wave 0 resolves kPlanItems rounds at a
  // time into LDS descriptors.
  const bool planned = nseq <= kPlanSeqs && qt_max <= kPlanLevels;
  if (planned) {
    for (int Q = tid; Q < qt_max; Q += 256) {
      int sum = 0;
      for (int b = 0; b < nseq; ++b) sum += max(0, static_cast<int>(nqt_s[b]) - Q - 1);
      lev_s[Q] = sum * HH;
    }
    __syncthreads();
  }
  const int P = static_cast<int>(gridDim.x), wr = static_cast<int>(blockIdx.x);
  auto item_of = [&](int k) { return k * P + ((k & 1) ? P - 1 - wr : wr); };
  auto make_plan = [&](int k0) {
    if (wave == 0) {
      const int i = item_of(k0 + lane);
      if (i < n_items) {
        int lo = 0, hi = qt_max - 1;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (lev_s[mid] <= i) hi = mid; else lo = mid + 1;
        }
        const int r = i - lev_s[lo];
        int rank = r / HH;
        const int hh = r - rank * HH;
        int b = 0;
        for (int bb = 0; bb < nseq; ++bb)
          if (static_cast<int>(nqt_s[bb]) > lo) {
            if (rank == 0) { b = bb; break; }
            --rank;
          }
        int64_t qs, ql, ks, kl;
        seq_range(cu_q, a.cuq_s, b, a.total_q, qs, ql);
        seq_range(cu_k, a.cuk_s, b, a.total_k, ks, kl);
        int32_t* const e = plan_s + 6 * lane;
        e[0] = b | (hh << 16);
        e[1] = lo;
        e[2] = static_cast<int32_t>(qs);
        e[3] = static_cast<int32_t>(ql);
        e[4] = static_cast<int32_t>(ks);
        e[5] = static_cast<int32_t>(kl);
      }
    }
    __syncthreads();
  };
  auto resolve_round = [&](int k, int i, Item& it) {
    if (planned) {
      if (k % kPlanItems == 0) make_plan(k);
      const int32_t* const e = plan_s + 6 * (k % kPlanItems);
      const int w0 = __builtin_amdgcn_readfirstlane(e[0]);
      const int Q = __builtin_amdgcn_readfirstlane(e[1]);
      const int64_t qs = __builtin_amdgcn_readfirstlane(e[2]), ks = __builtin_amdgcn_readfirstlane(e[4]);
      const int64_t ql = __builtin_amdgcn_readfirstlane(e[3]), kl = __builtin_amdgcn_readfirstlane(e[5]);
      fill_item(it, w0 & 0xFFFF, w0 >> 16, Q, qs, ql, ks, kl);
    } else {
      resolve(i, it);
    }
  };

  // ---- LDS layout of K/V blocks: 32 rows of RB bytes, the 16-byte chunk ch
  // of row r at position ch ^ swz(r) (varlen_prefill_gqa's layout: K operand
  // reads and transposed V reads are both free of bank conflicts).
  auto swz = [](int r) { return ((r & 3) << 2) | ((r >> 2) & 3); };
  typedef __attribute__((address_space(3))) void lds_void;
  const uint32_t smem_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)smem));
  // Block step s moves K(s + 1) and V(s): waves 0, 1 the K rows 0-15 / 16-31,
  // waves 2, 3 the V rows, IPW loads of RPI rows each. Lane l of a load whose
  // first row is R0 fetches the chunk that belongs at row R0 + l / CPR,
  // position l % CPR. Rows past the sequence re-read its last key (masked).
  const bool k_wave = wave < 2;
  const int row0w = (wave & 1) * 16;
  const int64_t st_b = (k_wave ? a.k_st : a.v_st) * static_cast<int64_t>(sizeof(T));
  const int lrow = lane / CPR;
  auto lane_chunk = [&](int i) { return (lane % CPR) ^ swz(row0w + i * RPI + lrow); };
  uint32_t doff[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) doff[i] = static_cast<uint32_t>(lrow * st_b) + 16u * lane_chunk(i);
  uint32_t doffs[IPW];  // doff[i] plus load i's row offset
#pragma unroll
  for (int i = 0; i < IPW; ++i) doffs[i] = doff[i] + static_cast<uint32_t>(i * RPI * st_b);
  auto load_block = [&](const Item& it, int blk, int slot) __attribute__((always_inline)) {
    const int key0 = min(blk, it.nblk - 1) * 32 + row0w;
    const int lds0 = (k_wave ? 0 : VOFF) + slot * BLKB + row0w * RB;
    const char* gbase = reinterpret_cast<const char*>(k_wave ? it.kb : it.vb);
    if (key0 + IPW * RPI <= it.k_len) {
      const char* src = gbase + key0 * st_b;
#pragma unroll
      for (int i = 0; i < IPW; ++i) dma16_sv(src + i * RPI * st_b, doff[i], smem_lds + lds0 + i * 1024);
    } else {
#pragma unroll
      for (int i = 0; i < IPW; ++i) {
        const int key = min(key0 + i * RPI + lrow, it.k_len - 1);
        dma16(gbase + key * st_b + 16 * lane_chunk(i), smem_lds + lds0 + i * 1024);
      }
    }
  };
  // An item's first loads: K(0) (K waves), then steps 0 .. A-1 that exist.
  auto load_head = [&](const Item& it) __attribute__((always_inline)) {
    if (it.nblk == 0) return;
    if (k_wave) load_block(it, 0, 0);
#pragma unroll
    for (int s0 = 0; s0 < A; ++s0)
      if (s0 < it.nblk) load_block(it, k_wave ? s0 + 1 : s0, k_wave ? (s0 + 1) % NB : s0);
  };
  // The loop's loads, step j + A issued in iteration j (slot phase S = j % NB
  // a compile-time constant): the wave's row pointer advances one block per
  // step, so a full block's loads take no address arithmetic beyond M0.
  const char* rp = nullptr;
  int rk = 0;
  auto loop_loads_start = [&](const Item& it) {
    rk = (A + (k_wave ? 1 : 0)) * 32 + row0w;
    rp = reinterpret_cast<const char*>(k_wave ? it.kb : it.vb) + rk * st_b;
  };
  auto load_step_c = [&](const Item& it, int j, auto S) __attribute__((always_inline)) {
    constexpr int s = decltype(S)::value;
    constexpr int kslot = (s + A + 1) % NB, vslot = (s + A) % NB;
    const int lds0 = (k_wave ? kslot * BLKB : VOFF + vslot * BLKB) + row0w * RB;
    if (rk + IPW * RPI <= it.kfull) {
#pragma unroll
      for (int i = 0; i < IPW; ++i) dma16_sv(rp, doffs[i], smem_lds + lds0 + i * 1024);
    } else {
      load_block(it, j + A + (k_wave ? 1 : 0), k_wave ? kslot : vslot);
    }
    rp += 32 * st_b;
    rk += 32;
  };
  // This wave's Q for an item into its Q area, each 32-query tile laid out
  // as a K block (tile t at t * 8 KB, row r = query q0 + 32t + r), whole
  // rows per load: load i of a tile fetches rows 4i .. 4i+3, lane l the chunk
  // (l % 16) ^ swz(4i + l / 16) of row 4i + l / 16 (swz(4i + l / 16) =
  // 4(l / 16) + i % 4). Rows past q_len repeat the last row; their outputs
  // are never stored. 16 loads, each of 8 whole 128-byte lines.
  const uint32_t q_lds = smem_lds + QOFF + wave * kW64QArea;
  const int64_t qst_b = a.q_st * static_cast<int64_t>(sizeof(T));
  const uint32_t q_rpart = static_cast<uint32_t>(lrow * qst_b);
  const uint32_t q_cpart = 16u * static_cast<uint32_t>((lane % CPR) ^ (lrow << 2));
  auto dma_q = [&](const Item& it) __attribute__((always_inline)) {
    const char* const qb = reinterpret_cast<const char*>(it.qb);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r0 = it.q0 + 32 * t;
      if (r0 + 32 <= it.q_len) {
        const char* const tb = qb + r0 * qst_b;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          dma16_sv(tb + 4 * i * qst_b, q_rpart + (q_cpart ^ (16u * (i & 3))), q_lds + t * BLKB + i * 1024);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int row = min(r0 + 4 * i + lrow, it.q_len - 1);
          dma16(qb + row * qst_b + (q_cpart ^ (16u * (i & 3))), q_lds + t * BLKB + i * 1024);
        }
      }
    }
  };
  constexpr int kQLoads = 2 * KJ;
  auto wait_loads = [&](auto n) { wait_vmcnt<decltype(n)::value>(); };

  // K operands of the block in slot ks: lane (h, c) reads key c, dims
  // 16jj + 8h..+8 (chunk 2jj + h at position (2jj + h) ^ swz(c)).
  int kaj[KJ];
#pragma unroll
  for (int jj = 0; jj < KJ; ++jj) kaj[jj] = (c * RB + 16 * (h ^ swz(c))) ^ (32 * jj);
  // Q stays in AGPRs for the whole item: the score MFMAs read their B
  // operand from there, which leaves the VGPRs to the softmax and the K/V
  // operands. Lane (h, c) takes query c's dims 16jj + 8h..+8, read as a K
  // operand is.
  u32x4 qop[2][KJ];
  auto read_q = [&]() {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int jj = 0; jj < KJ; ++jj) {
        qop[t][jj] = *reinterpret_cast<const u32x4*>(smem + QOFF + wave * kW64QArea + t * BLKB + kaj[jj]);
        in_agpr(qop[t][jj]);
      }
  };
  u32x4 kop[KJ];
  auto kread1 = [&](auto ks, int jj) __attribute__((always_inline)) {
    kop[jj] = *reinterpret_cast<const u32x4*>(smem + static_cast<int>(ks) * BLKB + kaj[jj]);
  };
  // V operands of the block in slot vs (varlen_prefill_gqa's transposed
  // reads): step s2, column tile u.
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  int vofs[NU], vofx[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int jl = c & 15, r = 4 * h + (jl >> 2), ch = 4 * u + 2 * (c >> 4) + ((jl & 3) >> 1);
    vofs[u] = r * RB + 16 * (ch ^ swz(r)) + 8 * (jl & 1);
    vofx[u] = vofs[u] ^ 32;
  }
  u32x4 vop[2][NU];
  auto vread1 = [&](auto vs, int s2, int u) __attribute__((always_inline)) {
    const int vb = VOFF + static_cast<int>(vs) * BLKB;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(smem + vb + 16 * s2 * RB + vofs[u]));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(smem + vb + 16 * s2 * RB + 8 * RB + vofx[u]));
    const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
    vop[s2][u] = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
  };

  // ---- Per-tile softmax state, scores and output accumulators. m: the
  // running max (log2 units); mt: the max of the tile's scores in sc, found
  // in the half that computed them; lacc: the denominators, summed on the
  // matrix cores from the P operands the P.V MFMAs take: a 16x16x32 MFMA
  // with A = ones where row m meets the k-groups g with g % 2 == m (lane l
  // supplies A[l % 16][8(l / 16)..+8]) and B = the P operand (lane (h, c)
  // supplies query c's 8 keys of the step, read as B[8(2h + c / 16)..+8][c %
  // 16]) gives D[0][n] = query n's 16 keys and D[1][n] = query 16 + n's, so
  // lane n < 16 holds l of query n in element 0 and of query 16 + n in
  // element 1 (the other elements stay zero). l sums the bf16 P the product
  // takes, in fp32.
  float m[2], mt[2];
  f32x4 lacc[2];
  uint32_t one2 = 0;  // the A operand: ones (two 16-bit 1.0) where lane % 16 == (lane / 16) % 2
  if ((lane & 15) == ((lane >> 4) & 1)) one2 = std::is_same<T, bf16_t>::value ? 0x3F803F80u : 0x3C003C00u;
  u32x4 lone = u32x4{one2, one2, one2, one2};
  in_agpr(lone);
  f32x16 sc[2];
  f32x16 acc[2][NU];
  u32x4 pop[2][2];
  auto qk1 = [&](int t, int jj) __attribute__((always_inline)) { mfma_qk_v<T>(sc[t], kop[jj], qop[t][jj], jj == 0); };
  auto pv1 = [&](int t, int s2, int u) __attribute__((always_inline)) {
    acc[t][u] = mfma_k16x32<T>(vop[s2][u], pop[t][s2], acc[t][u]);
  };
  auto lsum1 = [&](int t, int s2) __attribute__((always_inline)) {
    lacc[t] = mfma_k32<T>(lone, pop[t][s2], lacc[t]);
    in_agpr(lacc[t]);
  };
  // Scores e0 .. e1-1 of tile t in block blk set to -inf past k_len and,
  // causal, past the query (the key of accumulator e is 8(e/4) + 4h + e%4).
  // With base = 32 blk + 4h the key is base + ke(e), ke(e) = 8(e/4) + e%4 a
  // compile-time constant, so one per-lane bound serves all 16 scores: score
  // e is kept iff ke(e) < min(k_len - base, query - base + 1).
  auto mask_scores = [&](const Item& it, int t, int blk, int e0, int e1) __attribute__((always_inline)) {
    const int base = blk * 32 + 4 * h;
    int bound = it.k_len - base;
    if (a.causal) bound = min(bound, it.q0 + 32 * t + c - base + 1);
#pragma unroll
    for (int e = e0; e < e1; ++e)
      if (!(8 * (e >> 2) + (e & 3) < bound)) sc[t][e] = kNegInfP;
  };
  // The max of tile t's 16 scores (two chains of v_max3), then across the
  // lane halves (v_permlane32_swap), in log2 units.
  float mxa, mxb;
  auto max_part = [&](int t, int part) __attribute__((always_inline)) {
    if (part == 0) {
      mxa = fmaxf(fmaxf(sc[t][0], sc[t][1]), sc[t][2]);
      mxb = fmaxf(fmaxf(sc[t][3], sc[t][4]), sc[t][5]);
    } else if (part == 1) {
      mxa = fmaxf(fmaxf(mxa, sc[t][6]), sc[t][7]);
      mxb = fmaxf(fmaxf(mxb, sc[t][8]), sc[t][9]);
    } else if (part == 2) {
      mxa = fmaxf(fmaxf(mxa, sc[t][10]), sc[t][11]);
      mxb = fmaxf(fmaxf(mxb, sc[t][12]), sc[t][13]);
    } else {
      mxa = fmaxf(fmaxf(mxa, sc[t][14]), sc[t][15]);
    }
  };
  auto max_end = [&](int t) __attribute__((always_inline)) {
    const float mx = fmaxf(mxa, mxb);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mt[t] = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * cs;
  };
  // The rare rescale, before tile t's exponentials: when its block max
  // passes m by more than kRescale, m moves to it and l and the
  // accumulators are scaled by 2^(m_old - m_new). Until a tile's first key,
  // l and the accumulators are zero and only m moves.
  auto rescale_check = [&](int t) __attribute__((always_inline)) {
    if (__any(mt[t] > m[t] + kRescale)) {
      const float m_new = fmaxf(m[t], mt[t]);
      if (!__all(m[t] == kNegInfP)) {
        const float alpha = m_new == kNegInfP ? 1.f : fast_exp2(m[t] - m_new);
        const float alpha16 = __shfl_down(alpha, 16, 64);  // query lane + 16's (lacc element 1)
        xdl_to_valu_nops();
#pragma unroll
        for (int u = 0; u < NU; ++u) scale_agpr16(acc[t][u], alpha);
        scale_agpr2(lacc[t], alpha, alpha16);
        xdl_to_valu_nops();
      }
      m[t] = m_new;
    }
  };

  // ---- One half-iteration: the softmax of tile t (its scores are in sc[t],
  // their max in mt[t]) under 16 MFMA slots of tile o = 1 - t: slots 0-7 the
  // score MFMAs of o's next block (QK), slots 8-15 the P.V MFMAs of o's
  // previous block. Slot g issues its MFMA, operand reads (H0: K of the next
  // block after each QK; H1: the V operands of the block, pair g in QK slot
  // g, eight slots before the P.V MFMA that uses it, so each half reads half
  // of the wave's LDS bytes), the fma of score g, the exponential of score
  // g-1, the l term of score g-2 and, every other slot, the P operand of a
  // finished pair; slots 12-15 also take the max of o's new scores (its QK
  // MFMAs finished by then: >= 11 wait states after the last one), and slot
  // 10 masks them where needed. The fences hold this order, so every
  // instruction's inputs were produced at least one slot earlier.
  auto half = [&](const Item& it, int t, int mblk, auto kslot, auto vslot, bool do_qk)
                  __attribute__((always_inline)) {
    constexpr bool KREADS = decltype(kslot)::value >= 0, VREADS = decltype(vslot)::value >= 0;
    const int o = 1 - t;
    rescale_check(t);
    const float mm = m[t] == kNegInfP ? 0.f : m[t];
    float x[16], p[16];
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      if (g < 8) {
        if (do_qk) qk1(o, g);
        if constexpr (KREADS) kread1(kslot, g);
        if constexpr (VREADS) vread1(vslot, g / NU, g % NU);
      } else {
        pv1(o, (g - 8) / NU, (g - 8) % NU);
        in_agpr(acc[o][(g - 8) % NU]);  // keeps the MFMA in its slot
        if ((g - 8) % NU == NU - 1) lsum1(o, (g - 8) / NU);  // l of the step's P, after its last P.V
      }
      x[g] = fmaf(sc[t][g], cs, -mm);
      if (g >= 1) p[g - 1] = fast_exp2(x[g - 1]);
      if (g >= 3 && (g & 1)) {
        uint32_t pk = pack2<T>(p[g - 3], p[g - 2]);
        asm volatile("" : "+v"(pk));
        pop[t][(g - 3) >> 3][((g - 3) & 7) >> 1] = pk;
      }
      // Blocks from jm on may hold keys past k_len or (causal) past the
      // query: a uniform branch, rarely taken.
      if (g == 10 && do_qk && mblk >= it.jm) {
        xdl_to_valu_nops();
        mask_scores(it, o, mblk, 0, 16);
      }
      if (g >= 12 && do_qk) max_part(o, g - 12);
      // The slot's results, pinned here: nothing of it can sink into a later
      // slot or past the mask branch.
      asm volatile("" : "+v"(x[g]));
      if (g >= 1) asm volatile("" : "+v"(p[g - 1]));
      if (g >= 12 && do_qk) asm volatile("" : "+v"(mxa), "+v"(mxb));
      __builtin_amdgcn_sched_barrier(0);
    }
    p[15] = fast_exp2(x[15]);
    pop[t][1][3] = pack2<T>(p[14], p[15]);
    if (do_qk) max_end(o);
    // Everything of this half is computed here, under its MFMAs: without
    // this the compiler sinks it to the first use in the next half.
    float& mto = mt[o];
    asm volatile("" : "+v"(pop[t][0]), "+v"(pop[t][1]), "+v"(mto));
  };

  // ---- One iteration j: on entry S0(j) is in sc[0] with its max in mt[0],
  // P1(j-1) in pop[1], K(j) in kop and V(j-1) in vop (zeros before the
  // first block); step j's loads (K(j + 1), V(j)) were issued A iterations
  // ago. H0(j): softmax of tile 0, block j | QK1(j), PV1(j-1), reads K(j+1);
  // H1(j): softmax of tile 1, block j | QK0(j+1), reads V(j), PV0(j). In the
  // last iteration the K(j + 1) read and QK0(j+1) are not used (the slot
  // holds a clamped copy of the last block). S is the slot phase j % NB, a
  // compile-time constant.
  auto iter = [&](const Item& it, int j, auto S) __attribute__((always_inline)) {
    // Step j has landed for every wave: wait for this wave's loads of it,
    // meet the others, then issue step j + A (its slots were last read in
    // iteration j + A - NB < j, before this barrier).
    const bool issue = j + A < it.nblk;
    if (issue) wait_loads(std::integral_constant<int, kInFlight>{});
    else wait_loads(std::integral_constant<int, 0>{});
    lds_barrier();
    constexpr int s = decltype(S)::value;
    if (issue) load_step_c(it, j, S);
    half(it, 0, j, std::integral_constant<int, (s + 1) % NB>{}, std::integral_constant<int, -1>{}, true);
    half(it, 1, j + 1, std::integral_constant<int, -1>{}, S, true);
  };

  // The output of a finished item, in whole 128-byte lines: each tile goes
  // out through this wave's 4 KB staging area (32 rows x 128 bytes) in two
  // rounds, one half of the 128 dims per round. Every lane writes its
  // query's 4-dim runs of the round's two 32-dim column tiles (lane (h, c)
  // holds query c's dims 32u + 8g + 4h .. +3 in elements 4g .. 4g+3 of
  // acc[t][u]) as 8-byte pieces, the 16-byte chunk k = 4(u % 2) + g of row c
  // at position k ^ (c & 7); then lane l reads back chunk l % 8 of rows
  // l / 8 + 8i and the wave stores 8 half-rows of 128 bytes per
  // instruction. A wave's LDS operations run in order, so the next round may
  // overwrite the area once this one's reads are issued; each round's global
  // stores follow one round later. Rows past q_len are not stored. The stores
  // are non-temporal: the output is not read again here, and allocating it
  // in L2 evicts K/V lines that later items re-read (measured 4% slower).
  auto store_out = [&](const Item& it) {
    xdl_to_valu_nops();  // the last P.V MFMAs wrote the accumulators
    char* const ost = smem + OOFF + wave * kW64OutStage;
    const int rr = lane >> 3, ch = lane & 7;  // read-back: rows rr + 8i, chunk ch
    u32x4 pend[4];
    char* pend_p[4];
    bool pend_ok[4];
    bool pend_full = true, have = false;
    auto flush = [&]() __attribute__((always_inline)) {
      if (pend_full) {
#pragma unroll
        for (int i = 0; i < 4; ++i) __builtin_nontemporal_store(pend[i], reinterpret_cast<u32x4*>(pend_p[i]));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (pend_ok[i]) __builtin_nontemporal_store(pend[i], reinterpret_cast<u32x4*>(pend_p[i]));
      }
    };
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float l0 = __shfl(lacc[t][0], c & 15, 64), l1 = __shfl(lacc[t][1], c & 15, 64);
      const float rl = 1.f / (c < 16 ? l0 : l1);  // 1 / query c's denominator
      const int rbase = it.q0 + 32 * t;
      const bool full = rbase + 32 <= it.q_len;
      char* rowp[4];
      bool rok[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = rbase + rr + 8 * i;
        rok[i] = row < it.q_len;
        rowp[i] = reinterpret_cast<char*>(it.ob + static_cast<int64_t>(row) * a.o_st) + 16 * ch;
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int uu = 0; uu < 2; ++uu)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int u = 2 * half + uu;
            const u32x2 w = {pack2<T>(acc[t][u][4 * g] * rl, acc[t][u][4 * g + 1] * rl),
                             pack2<T>(acc[t][u][4 * g + 2] * rl, acc[t][u][4 * g + 3] * rl)};
            *reinterpret_cast<u32x2*>(ost + c * 128 + 16 * ((4 * uu + g) ^ (c & 7)) + 8 * h) = w;
          }
        u32x4 got[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = rr + 8 * i;
          got[i] = *reinterpret_cast<const u32x4*>(ost + r * 128 + 16 * (ch ^ (r & 7)));
        }
        if (have) flush();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pend[i] = got[i];
          pend_ok[i] = rok[i];
          pend_p[i] = rowp[i] + 128 * half;
        }
        pend_full = full;
        have = true;
      }
    }
    flush();
  };

  // ---- The item loop. At an item's end, after its last barrier, the next
  // item's Q and head blocks are issued (every slot and the Q area are free
  // then), and its last P.V and output store run while they load.
  int round = 0;
  int idx = item_of(0);
  Item X;
  if (idx < n_items) {
    resolve_round(0, idx, X);
    dma_q(X);
    load_head(X);
  }
  using std::integral_constant;
  while (idx < n_items) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      m[t] = kNegInfP;
      lacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
      in_agpr(lacc[t]);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[t][u][e] = 0.f;
        in_agpr(acc[t][u]);
      }
    }
    // X's Q and K(0) (steps 0 .. A-1 may still be in flight: IPW loads each).
    if (X.nblk >= A) wait_loads(integral_constant<int, A * IPW>{});
    else wait_loads(integral_constant<int, 0>{});
    lds_barrier();
    read_q();
    if (X.nblk > 0) {
#pragma unroll
      for (int jj = 0; jj < KJ; ++jj) kread1(integral_constant<int, 0>{}, jj);
#pragma unroll
      for (int jj = 0; jj < KJ; ++jj) qk1(0, jj);
      xdl_to_valu_nops();
      if (X.jm == 0) mask_scores(X, 0, 0, 0, 16);
#pragma unroll
      for (int part = 0; part < 4; ++part) max_part(0, part);
      max_end(0);
    }
    loop_loads_start(X);
    const int n = X.nblk;
    // P1(-1) V(-1) of the first iteration adds zeros.
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      pop[1][s2] = u32x4{0, 0, 0, 0};
#pragma unroll
      for (int u = 0; u < NU; ++u) vop[s2][u] = u32x4{0, 0, 0, 0};
    }
    // Iterations 0 .. n-1, unrolled by slot phase.
    for (int j = 0; j < n;) {
      iter(X, j, integral_constant<int, 0>{});
      if (++j == n) break;
      iter(X, j, integral_constant<int, 1>{});
      if (++j == n) break;
      iter(X, j, integral_constant<int, 2>{});
      if (++j == n) break;
      iter(X, j, integral_constant<int, 3>{});
      ++j;
    }
    // Every wave has read X's last K/V block (in H0 of the last iteration)
    // and its Q: the slots and the Q area are free for the next item.
    lds_barrier();
    ++round;
    const int nidx = item_of(round);
    Item Y;
    if (nidx < n_items) {
      resolve_round(round, nidx, Y);
      dma_q(Y);
      load_head(Y);
    }
    // X's last P.V of tile 1 (V(n-1) and P1(n-1) are in registers), then
    // its output. (An item without keys: 0/0, as the reference's.)
    if (n > 0) {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
        for (int u = 0; u < NU; ++u) pv1(1, s2, u);
        lsum1(1, s2);
      }
    }
    store_out(X);
    X = Y;
    idx = nidx;
  }
  wait_loads(integral_constant<int, 0>{});
  (void)kQLoads;
}

}  // namespace tsa
