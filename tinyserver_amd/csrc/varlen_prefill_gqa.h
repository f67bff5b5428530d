// The LDS-staged GQA prefill attention body, shared by varlen_prefill_gqa
// (varlen_prefill.hip) and the mixed prefill + decode kernel
// (paged_decode.hip), plus the argument block and host helpers of the
// prefill entry points.
//
// Reference: server/model/kernels/varlen_attention.py:8-142.
#pragma once

#include <cmath>

#include "tsa_common.h"

namespace tsa {

struct PrefillArgs {
  void* out;
  const void* q;
  const void* k;
  const void* v;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int64_t cuq_s, cuk_s;
  int64_t q_st, q_sh, q_sd, k_st, k_sh, k_sd, v_st, v_sh, v_sd, o_st, o_sh, o_sd;
  int64_t total_q, total_k;
  int32_t nseq, Hq, Hkv, G, D, nqb;
  int32_t causal;
  float scale_log2;
};

// Sequences per call the persistent kernel keeps counts of in LDS.
constexpr int max_persist_seqs(int nw) { return nw == 2 ? 1024 : 2048; }

constexpr float kNegInfP = -INFINITY;

// [start, end) of sequence b in a packed tensor of n tokens; out-of-range
// cu_seqlens entries are clamped so a malformed table cannot read past it.
__device__ __forceinline__ void seq_range(const int32_t* cu, int64_t stride, int b, int64_t n, int64_t& start,
                                          int64_t& len) {
  int64_t s0 = cu[b * stride], s1 = cu[(b + 1) * stride];
  s0 = s0 < 0 ? 0 : (s0 > n ? n : s0);
  s1 = s1 < s0 ? s0 : (s1 > n ? n : s1);
  start = s0;
  len = s1 - s0;
}

// The work-item plan: up to kPlanItems item descriptors of a workgroup (6
// int32 each), computed kPlanItems at a time, and the level table (items
// above each query-block level) they are found with, for calls of at most
// kPlanSeqs sequences and kPlanLevels query blocks per sequence.
constexpr int kPlanItems = 64, kPlanSeqs = 64, kPlanLevels = 256;

// LDS bytes of prefill_gqa_body<D, NW>: NB K and NB V block slots of 32 rows,
// the output staging (one 32-dim column tile of the 32 queries per wave),
// the per-sequence query-block counts and the work-item plan.
constexpr int kOutStage = 32 * 64;  // bytes of output staging per wave
template <int D, int NW>
constexpr int gqa_smem_bytes() {
  return 2 * (NW == 2 ? 2 : 4) * (32 * 2 * D) + NW * kOutStage + max_persist_seqs(NW) * 2 +
         kPlanItems * 6 * 4 + kPlanLevels * 4;
}

// LDS-staged GQA flash attention on 32x32 tiles, persistent. A work item is
// one kv head of one sequence and 32 queries; a workgroup of NW = G waves
// (G = q heads per kv head: 2, 4 or 8) computes it, wave w taking those
// queries of q-head w, so all NW tiles read the same K/V and need the same
// key blocks. The grid is as many workgroups as fit on the device at once,
// each walking its share of the items (the item loop below). 32-key K/V
// blocks go from global memory straight into LDS (global_load_lds_dwordx4,
// no registers), NB slots per tensor, the loads A = NB - 1 blocks ahead and
// K one block ahead of V. Rows are unpadded; the 16-byte chunk ch of row r
// sits at position ch ^ swz(r). Both products run on v_mfma_f32_32x32x16
// (the 16x16x32 form has about 60% of its throughput on gfx950). With lane
// (h, c) = (lane / 32, lane % 32) and accumulator element e holding row
// 8(e/4) + 4h + e%4, column c:
//   S^T(32 keys x 32 queries) = K Q^T over head_dim/16 steps: lane (h, c)
//     reads key c, dims 16jj + 8h..+8 (the swizzle puts the 16 rows of a
//     128-bit read in 16 distinct bank quads) and holds query c's Q slice in
//     registers; it gets query c's scores of keys 8(e/4) + 4h + e%4;
//   O^T(32 dims x 32 queries) += V^T P^T over two 16-key steps s: the P^T
//     operand's k-slots 8h..8h+7 are keys 16s+4h+0..3 and 16s+8+4h+0..3,
//     i.e. the score accumulators 8s..8s+7 of the same lane, so P goes to the
//     operand in registers; the V^T operand comes from two ds_read_b64_tr_b16,
//     in which a 16-lane group whose lane 4e+q reads dims 4q..4q+3 of key row
//     e gets, in lane j, element e = V[key e][dim j]. V stays row-major in
//     LDS, and the swizzle keeps these reads free of bank conflicts too.
//     Lane (h, c) accumulates query c's outputs, so the softmax's row scales
//     (the rescale and 1/l) are the lane's own.
// Scores, probabilities and the output accumulators all stay in VGPRs (at most
// 256 per wave, two waves per SIMD); the workgroups sharing a CU drift apart,
// so one workgroup's softmax overlaps another's MFMAs.
template <typename T, int D, int NW>
__device__ __forceinline__ void prefill_gqa_body(PrefillArgs a, const int32_t* __restrict__ cu_q,
                                                 const int32_t* __restrict__ cu_k, char* smem, int wg_base) {
  constexpr int KJ = D / 16;              // 16-dim steps of the QK reduction
  constexpr int NU = D / 32;              // 32-dim column tiles of the output
  constexpr int CPR = D / 8;              // 16-byte chunks per K/V row
  constexpr int RB = 2 * D;               // bytes per K/V row in LDS (unpadded)
  constexpr int BLKB = 32 * RB;           // bytes per 32-row K or V block
  // K/V block slots in LDS and the prefetch distance in blocks: the loads
  // of a block are issued A iterations before it is needed.
  constexpr int NB = NW == 2 ? 2 : 4, A = NB - 1;
  constexpr int RPI = 1024 / RB;          // rows per 1 KB load instruction
  constexpr int IPW = 2 * (32 / RPI) / NW;  // load instructions per wave per block step
  constexpr int VOFF = NB * BLKB;           // byte offset of the V slots
  constexpr int OOFF = 2 * NB * BLKB;       // byte offset of the output staging
  constexpr int QOFF = OOFF + NW * kOutStage;  // byte offset of the per-sequence query-block counts
  constexpr int PLOFF = QOFF + max_persist_seqs(NW) * 2;  // byte offset of the item plan
  constexpr int LVOFF = PLOFF + kPlanItems * 6 * 4;       // byte offset of the level table
  static_assert(LVOFF + kPlanLevels * 4 == gqa_smem_bytes<D, NW>(), "LDS layout and its size agree");
  static_assert(IPW >= 1 && IPW * NW == 2 * (32 / RPI), "a block step is a whole number of loads per wave");
  static_assert((A > 1 ? A - 1 : 0) * IPW <= 63, "outstanding loads fit the vmcnt field");
  // A row's running max only moves when it grows by more than this (log2
  // units): p = 2^(s - m) then stays below 2^8, and the accumulator is
  // rescaled rarely. l uses the same m, so the result is unchanged.
  constexpr float kRescale = 8.0f;
  uint16_t* const nqb_s = reinterpret_cast<uint16_t*>(smem + QOFF);  // query blocks of each sequence
  int32_t* const plan_s = reinterpret_cast<int32_t*>(smem + PLOFF);   // item descriptors, 6 words each
  int32_t* const lev_s = reinterpret_cast<int32_t*>(smem + LVOFF);    // items above each level

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nseq = a.nseq, Hkv = a.Hkv;
  const float cs = a.scale_log2;  // > 0 on this path

  // ---- Work items: (query block, sequence, kv head) with a non-empty query
  // block, heaviest (latest) query blocks first: level Q holds query block Q
  // of every sequence that has one, in sequence order, kv head fastest.
  // The workgroups take them in rounds (item_of below), heaviest first. (No
  // work-queue atomic: a returning atomic holds up every load the wave issues
  // after it until it completes, and under load that took longer than the
  // imbalance it would remove.) The per-sequence counts live in LDS.
  for (int b = tid; b < nseq; b += 64 * NW) {
    int64_t qs, ql;
    seq_range(cu_q, a.cuq_s, b, a.total_q, qs, ql);
    nqb_s[b] = static_cast<uint16_t>((ql + 31) / 32);
  }
  __syncthreads();
  // Items above level Q: Hkv * sum_b max(0, nqb_b - Q - 1) (wave reduction).
  auto items_above = [&](int Q) {
    int sum = 0;
    for (int b = lane; b < nseq; b += 64) sum += max(0, static_cast<int>(nqb_s[b]) - Q - 1);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
    return __builtin_amdgcn_readfirstlane(sum) * Hkv;
  };
  int qb_max = 0;
  for (int b = lane; b < nseq; b += 64) qb_max = max(qb_max, static_cast<int>(nqb_s[b]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) qb_max = max(qb_max, __shfl_xor(qb_max, off, 64));
  qb_max = __builtin_amdgcn_readfirstlane(qb_max);
  const int n_items = items_above(-1);

  struct Item {
    int b, kvh, q0, q_len, k_len, nblk;
    int jm;     // first block that needs a mask (keys past k_len, or causal keys after a query)
    int kfull;  // rows below min(k_len, 32 nblk) load without clamping
    int64_t q_start;
    const T* kb;
    const T* vb;
  };
  // Item i -> its level (the smallest Q with items_above(Q) <= i), then the
  // sequence of rank (i - items_above(Q)) / Hkv among those with nqb > Q.
  auto resolve = [&](int i, Item& it) {
    int lo = 0, hi = qb_max - 1;  // answer in [lo, hi]
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (items_above(mid) <= i) hi = mid; else lo = mid + 1;
    }
    const int Q = lo;
    const int r = i - items_above(Q);
    int rank = r / Hkv;
    it.kvh = r - rank * Hkv;
    int b = 0;
    for (int base = 0; base < nseq; base += 64) {
      const int bb = base + lane;
      const uint64_t m = __ballot(bb < nseq && static_cast<int>(nqb_s[bb]) > Q);
      const int cnt = __builtin_popcountll(m);
      if (rank < cnt) {
        // the rank-th set bit of m
        uint64_t mm = m;
        for (int k = 0; k < rank; ++k) mm &= mm - 1;
        b = base + __builtin_ctzll(mm);
        break;
      }
      rank -= cnt;
    }
    it.b = __builtin_amdgcn_readfirstlane(b);
    int64_t qs, ql, ks, kl;
    seq_range(cu_q, a.cuq_s, it.b, a.total_q, qs, ql);
    seq_range(cu_k, a.cuk_s, it.b, a.total_k, ks, kl);
    it.q_start = qs;
    it.q_len = static_cast<int>(ql);
    it.k_len = static_cast<int>(kl);
    it.q0 = Q * 32;
    const int q_last = it.q0 + 32 < it.q_len ? it.q0 + 32 : it.q_len;
    const int kend = a.causal ? (it.k_len < q_last ? it.k_len : q_last) : it.k_len;
    it.nblk = (kend + 31) / 32;
    it.jm = a.causal ? min(it.k_len / 32, Q) : it.k_len / 32;
    it.kfull = min(it.k_len, it.nblk * 32);
    it.kb = static_cast<const T*>(a.k) + ks * a.k_st + it.kvh * a.k_sh;
    it.vb = static_cast<const T*>(a.v) + ks * a.v_st + it.kvh * a.v_sh;
  };

  // ---- The item plan. For calls of at most kPlanSeqs sequences and
  // kPlanLevels query blocks per sequence, the level table lev_s[Q] =
  // items_above(Q) is built once, and wave 0 resolves kPlanItems items at a
  // time, one per lane (a binary search over the table, the rank-th
  // sequence by a scan, its ranges by a vector load), into plan_s: the item
  // loop then reads a descriptor from LDS instead of running the
  // wave-cooperative search above for every item.
  const bool planned = nseq <= kPlanSeqs && qb_max <= kPlanLevels;
  if (planned) {
    for (int Q = tid; Q < qb_max; Q += 64 * NW) {
      int sum = 0;
      for (int b = 0; b < nseq; ++b) sum += max(0, static_cast<int>(nqb_s[b]) - Q - 1);
      lev_s[Q] = sum * Hkv;
    }
    __syncthreads();
  }
  // Round k of the deal gives workgroup w item k P + w when k is even and
  // k P + P - 1 - w when it is odd (P workgroups, items heaviest first).
  const int P = static_cast<int>(gridDim.x) - wg_base, wr = static_cast<int>(blockIdx.x) - wg_base;
  auto item_of = [&](int k) { return k * P + ((k & 1) ? P - 1 - wr : wr); };
  // Items of rounds k0 .. k0 + kPlanItems - 1 into plan_s (every wave calls it).
  auto make_plan = [&](int k0) {
    if (wave == 0) {
      const int i = item_of(k0 + lane);
      if (i < n_items) {
        int lo = 0, hi = qb_max - 1;  // the smallest Q with lev_s[Q] <= i
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (lev_s[mid] <= i) hi = mid; else lo = mid + 1;
        }
        const int r = i - lev_s[lo];
        int rank = r / Hkv;
        const int kvh = r - rank * Hkv;
        int b = 0;
        for (int bb = 0; bb < nseq; ++bb)
          if (static_cast<int>(nqb_s[bb]) > lo) {
            if (rank == 0) { b = bb; break; }
            --rank;
          }
        int64_t qs, ql, ks, kl;
        seq_range(cu_q, a.cuq_s, b, a.total_q, qs, ql);
        seq_range(cu_k, a.cuk_s, b, a.total_k, ks, kl);
        int32_t* const e = plan_s + 6 * lane;
        e[0] = b | (kvh << 16);
        e[1] = lo;
        e[2] = static_cast<int32_t>(qs);
        e[3] = static_cast<int32_t>(ql);
        e[4] = static_cast<int32_t>(ks);
        e[5] = static_cast<int32_t>(kl);
      }
    }
    __syncthreads();
  };
  // Item of round k from the plan (its descriptor is in plan_s).
  auto resolve_planned = [&](int k, Item& it) {
    const int32_t* const e = plan_s + 6 * (k % kPlanItems);
    const int w0 = __builtin_amdgcn_readfirstlane(e[0]);
    it.b = w0 & 0xFFFF;
    it.kvh = w0 >> 16;
    const int Q = __builtin_amdgcn_readfirstlane(e[1]);
    const int64_t qs = __builtin_amdgcn_readfirstlane(e[2]), ks = __builtin_amdgcn_readfirstlane(e[4]);
    it.q_start = qs;
    it.q_len = __builtin_amdgcn_readfirstlane(e[3]);
    it.k_len = __builtin_amdgcn_readfirstlane(e[5]);
    it.q0 = Q * 32;
    const int q_last = it.q0 + 32 < it.q_len ? it.q0 + 32 : it.q_len;
    const int kend = a.causal ? (it.k_len < q_last ? it.k_len : q_last) : it.k_len;
    it.nblk = (kend + 31) / 32;
    it.jm = a.causal ? min(it.k_len / 32, Q) : it.k_len / 32;
    it.kfull = min(it.k_len, it.nblk * 32);
    it.kb = static_cast<const T*>(a.k) + ks * a.k_st + it.kvh * a.k_sh;
    it.vb = static_cast<const T*>(a.v) + ks * a.v_st + it.kvh * a.v_sh;
  };
  // The item of round k (k: this workgroup's round; i = item_of(k)).
  auto resolve_round = [&](int k, int i, Item& it) {
    if (planned) {
      if (k % kPlanItems == 0) make_plan(k);
      resolve_planned(k, it);
    } else {
      resolve(i, it);
    }
  };

  // ---- LDS layout of K/V: rows are stored unpadded, RB bytes each, with the
  // 16-byte chunk ch of row r at position ch ^ swz(r). swz is a bijection on
  // r % 16, so the 16 lanes of a K operand read (16 rows, one chunk) hit 16
  // distinct bank quads, and it maps r % 4 to the upper bits, so a
  // transposed V read (4 consecutive rows x 2 chunks per 16 lanes) is
  // conflict-free as well.
  auto swz = [](int r) {
    return D == 128 ? ((r & 3) << 2) | ((r >> 2) & 3) : (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  };

  // K and V go from global memory straight into LDS (global_load_lds_dwordx4:
  // each lane carries 16 bytes, the wave's 1 KB lands contiguously at a
  // wave-uniform LDS address), so no registers stage them and the loads run
  // A blocks ahead. Lane l of a load whose first row is R0 fetches the chunk
  // that belongs at row R0 + l / CPR, position l % CPR. Block step s moves K
  // block s + 1 and V block s, IPW loads per wave: waves 0 .. NW/2 - 1 the K
  // rows, the others the V rows; every wave issues the same number of loads
  // per step. Rows past the sequence's end re-read its last key, which the
  // mask or a zero probability then ignores; so does the last step's K block
  // (one past the end, a clamped copy of the last block). Block j of every
  // item goes to slot j % NB.
  typedef __attribute__((address_space(3))) void lds_void;
  const bool k_wave = wave < NW / 2;
  const int row0w = (wave % (NW / 2)) * IPW * RPI;  // first row this wave loads
  const int64_t st_b = (k_wave ? a.k_st : a.v_st) * static_cast<int64_t>(sizeof(T));
  const int lrow = lane / CPR;
  auto lane_chunk = [&](int i) { return (lane % CPR) ^ swz(row0w + i * RPI + lrow); };
  uint32_t doff[IPW];  // lane byte offsets from the first row of load i (< 2^32: strides checked on the host)
#pragma unroll
  for (int i = 0; i < IPW; ++i) doff[i] = static_cast<uint32_t>(lrow * st_b) + 16u * lane_chunk(i);
  // A full block's loads take a wave-uniform base plus a 32-bit lane offset
  // (dma16_sv), which reads half the address registers of the 64-bit
  // per-lane form.
  const uint32_t smem_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)smem));  // address-space cast
  auto dma = [&](const char* sbase, uint32_t voff, int lds_byte) __attribute__((always_inline)) {
    dma16_sv(sbase, voff, smem_lds + lds_byte);
  };
  auto dma64 = [&](const char* src, int lds_byte) __attribute__((always_inline)) {
    dma16(src, smem_lds + lds_byte);
  };
  // This wave's loads of block blk of item `it` (K if k_wave) into slot `slot`.
  auto load_block = [&](const Item& it, int blk, int slot) __attribute__((always_inline)) {
    const int key0 = min(blk, it.nblk - 1) * 32 + row0w;
    const int lds0 = (k_wave ? 0 : VOFF) + slot * BLKB + row0w * RB;
    const char* gbase = reinterpret_cast<const char*>(k_wave ? it.kb : it.vb);
    if (key0 + IPW * RPI <= it.k_len) {
      const char* src = gbase + key0 * st_b;
#pragma unroll
      for (int i = 0; i < IPW; ++i) dma(src + i * RPI * st_b, doff[i], lds0 + i * 1024);
    } else {
#pragma unroll
      for (int i = 0; i < IPW; ++i) {
        const int key = min(key0 + i * RPI + lrow, it.k_len - 1);
        dma64(gbase + key * st_b + 16 * lane_chunk(i), lds0 + i * 1024);
      }
    }
  };
  // K block 0 and block steps 0 .. A - 1 (those that exist) of an item;
  // nothing for an item without keys. Block b of every item goes to slot
  // b % NB.
  // The K waves' part (K blocks 0 .. A) and the V waves' part (V blocks
  // 0 .. A - 1) can be issued apart.
  auto load_head_k = [&](const Item& it) __attribute__((always_inline)) {
    if (it.nblk == 0 || !k_wave) return;
    load_block(it, 0, 0);
#pragma unroll
    for (int s0 = 0; s0 < A; ++s0)
      if (s0 < it.nblk) load_block(it, s0 + 1, s0 + 1);
  };
  auto load_head_v = [&](const Item& it) __attribute__((always_inline)) {
    if (it.nblk == 0 || k_wave) return;
#pragma unroll
    for (int s0 = 0; s0 < A; ++s0)
      if (s0 < it.nblk) load_block(it, s0, s0);
  };
  auto load_head = [&](const Item& it) __attribute__((always_inline)) {
    load_head_k(it);
    load_head_v(it);
  };
  // The block loop's loads: step j + A of the item, issued in iteration j,
  // whose slot phase S = j % NB is a compile-time constant there. The wave's
  // row pointer and first key advance by one block per step, so a full
  // block's loads take no address arithmetic beyond M0.
  uint32_t doffs[IPW];  // doff[i] plus load i's row offset (< 2^32: strides checked on the host)
#pragma unroll
  for (int i = 0; i < IPW; ++i) doffs[i] = doff[i] + static_cast<uint32_t>(i * RPI * st_b);
  const char* rp = nullptr;  // this wave's first row of its next step's block
  int rk = 0;                // that row's key index
  auto loop_loads_start = [&](const Item& it) {
    rk = (A + (k_wave ? 1 : 0)) * 32 + row0w;
    rp = reinterpret_cast<const char*>(k_wave ? it.kb : it.vb) + rk * st_b;
  };
  auto load_step_c = [&](const Item& it, int j, auto S) __attribute__((always_inline)) {
    constexpr int s = decltype(S)::value;
    const int lds0 = (k_wave ? s * BLKB : VOFF + ((s + NB - 1) % NB) * BLKB) + row0w * RB;
    if (rk + IPW * RPI <= it.kfull) {
#pragma unroll
      for (int i = 0; i < IPW; ++i) dma(rp, doffs[i], lds0 + i * 1024);
    } else {
      load_block(it, j + A + (k_wave ? 1 : 0), k_wave ? s : (s + NB - 1) % NB);
    }
    rp += 32 * st_b;
    rk += 32;
  };
  // Wait until at most n of this wave's loads are in flight (they complete
  // in issue order; other memory operations issued among them only make the
  // wait stricter). The compiler does not count the DMA loads, so the
  // kernel places these waits itself.
  auto wait_loads = [&](auto n) { wait_vmcnt<decltype(n)::value>(); };
  constexpr int kInFlight = (A - 1) * IPW;  // loads of the later steps, still in flight at a block's end

  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

  // Q operand of the item (lane (h, c): query q0 + c, dims 16jj + 8h..+8).
  u32x4 qop[KJ];
  auto load_q = [&](const Item& it) {
    const int row = it.q0 + c;
    const int head = it.kvh * NW + wave;
    const T* qp = static_cast<const T*>(a.q) + (it.q_start + row) * a.q_st + head * a.q_sh;
#pragma unroll
    for (int jj = 0; jj < KJ; ++jj)
      qop[jj] = row < it.q_len ? *reinterpret_cast<const u32x4*>(qp + 16 * jj + 8 * h) : u32x4{0, 0, 0, 0};
  };

  // K operands of the block in slot ks: lane (h, c) reads key c, dims
  // 16jj + 8h..+8, i.e. chunk 2jj + h at position (2jj + h) ^ swz(c): byte
  // c RB + ((32 jj) ^ 16 (h ^ swz(c))), the XOR staying inside the row.
  int kaj[KJ];
#pragma unroll
  for (int jj = 0; jj < KJ; ++jj) kaj[jj] = (c * RB + 16 * (h ^ swz(c))) ^ (32 * jj);
  u32x4 kop[KJ];
  auto kread = [&](auto ks) {
#pragma unroll
    for (int jj = 0; jj < KJ; ++jj) kop[jj] = *reinterpret_cast<const u32x4*>(smem + ks * BLKB + kaj[jj]);
  };
  // S^T(block) = K Q^T: lane (h, c) gets query c's scores of keys
  // 8(e/4) + 4h + e%4 of the block.
  auto qk = [&](f32x16& sc) {
#pragma unroll
    for (int e = 0; e < 16; ++e) sc[e] = 0.f;
#pragma unroll
    for (int jj = 0; jj < KJ; ++jj) sc = mfma_k16x32<T>(kop[jj], qop[jj], sc);
  };
  float m = kNegInfP, l = 0.f;  // query c's running max (log2 domain) and this lane's share of its sum
  f32x16 acc[NU];
  // Keys past k_len, and (causal) keys after the query, only occur in a
  // sequence's last block or on the diagonal: a wave-uniform branch.
  auto mask_block = [&](const Item& it, f32x16& sc, int blk) {
    const int kb0 = blk * 32;
    if (blk >= it.jm) {
      const int qq = it.q0 + c;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int kk = kb0 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (!(kk < it.k_len && (!a.causal || kk <= qq))) sc[e] = kNegInfP;
      }
    }
  };
  // Query c's max over the block (log2 units): the lane's 16 scores, then
  // the other lane half's through v_permlane32_swap (no LDS round trip).
  auto block_max = [&](const f32x16& sc) {
    float tmax = kNegInfP;
#pragma unroll
    for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, sc[e]);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(tmax), __float_as_uint(tmax), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * cs;
  };
  // The (rare) rescale when the max moves by more than kRescale; a lane's
  // accumulators are its own query's, so they take its own alpha.
  auto rescale = [&](float mt) {
    if (__any(mt > m + kRescale)) {
      const float m_new = fmaxf(m, mt);
      const float alpha = m_new == kNegInfP ? 1.f : fast_exp2(m - m_new);
      l *= alpha;
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[u][e] *= alpha;
      m = m_new;
    }
  };
  // p = 2^(s cs - m) in fp32 (summed into l), packed to the P operands of
  // the two 16-key steps: k-slots 8h..8h+7 of step s are keys 16s+4h+0..3
  // and 16s+8+4h+0..3, i.e. score accumulators 8s..8s+7 of the same lane.
  u32x4 pop[2];
  auto softmax_exp = [&](const f32x16& sc) {
    const float mm = m == kNegInfP ? 0.f : m;
    float p[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      p[e] = fast_exp2(fmaf(sc[e], cs, -mm));
      l += p[e];
    }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
      pop[s2] = u32x4{pack2<T>(p[8 * s2], p[8 * s2 + 1]), pack2<T>(p[8 * s2 + 2], p[8 * s2 + 3]),
                      pack2<T>(p[8 * s2 + 4], p[8 * s2 + 5]), pack2<T>(p[8 * s2 + 6], p[8 * s2 + 7])};
  };
  // V operands of the block in slot vs: the B operand of step s, column
  // tile u is V[keys 16s+4h+e, 16s+8+4h+e][dims 32u + c], read transposed.
  // Lane (h, c) with jl = c % 16 reads 8 bytes of row 4h + jl/4 (+8, +16s),
  // dims 32u + 16(c/16) + 4(jl%4): vofs[u] for the first row; the row 8
  // further has swz XORed by 2, i.e. the byte offset XORed by 32. They are
  // read into registers one block ahead of their P V.
  int vofs[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int jl = c & 15, r = 4 * h + (jl >> 2), ch = 4 * u + 2 * (c >> 4) + ((jl & 3) >> 1);
    vofs[u] = r * RB + 16 * (ch ^ swz(r)) + 8 * (jl & 1);
  }
  int vofx[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) vofx[u] = vofs[u] ^ 32;
  u32x4 vop[2][NU];
  auto vread = [&](auto vs) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int lo_b = VOFF + vs * BLKB + 16 * s2 * RB + vofs[u];
        const int hi_b = VOFF + vs * BLKB + 16 * s2 * RB + 8 * RB + vofx[u];
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(smem + lo_b));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(smem + hi_b));
        const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
        vop[s2][u] = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
      }
  };
  // O^T += V^T P^T of the pending block, operands in registers. The P and
  // V operand registers serve as B and A: lane (h, c) holds P[query c][k-slots
  // 8h..8h+7] and V[k-slots 8h..8h+7][dim 32u + c], which are the B operand
  // of P^T and the A operand of V^T. So lane (h, c) accumulates query c's
  // outputs, dims 32u + 8(e/4) + 4h + e%4: its row scales are its own.
  auto pv = [&]() {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int u = 0; u < NU; ++u) acc[u] = mfma_k16x32<T>(vop[s2][u], pop[s2], acc[u]);
  };

  // Software pipeline, one 32-key block per iteration j, whose slot phase
  // S = j % NB is a compile-time constant (the loop is unrolled NB times, so
  // every LDS address is a lane offset plus an immediate). On entry S(j) is
  // in registers, K block j + 1 and V block j are in their LDS slots, and
  // (PREV) block j - 1's P and V operands are in registers. The wave issues
  // block step j + A's loads (into the slots of K(j) and V(j - 1), both last
  // read before the previous barrier) and reads K(j + 1); then P(j - 1)
  // V(j - 1) runs on the matrix cores under S(j)'s max, and S(j + 1) under
  // S(j)'s exponentials and the reads of V(j). It then waits for step
  // j + 1's rows and meets the other waves at the barrier. Steps past the
  // last block are not issued; once they stop, fewer loads than kInFlight
  // are younger than the one a block needs, so those blocks wait for all of
  // them.
  f32x16 sca, scb;  // S of the even / odd blocks
  auto full = [&](const Item& it, int j, auto S, auto prev) {
    constexpr int s = decltype(S)::value;
    f32x16& cur = (s & 1) ? scb : sca;
    f32x16& nxt = (s & 1) ? sca : scb;
    const bool issue = j < it.nblk - A;
    if (issue) load_step_c(it, j, S);
    kread(std::integral_constant<int, (s + 1) % NB>{});
    mask_block(it, cur, j);
    if constexpr (decltype(prev)::value) pv();
    const float mt = block_max(cur);
    if constexpr (decltype(prev)::value) {
#pragma unroll
      for (int i = 0; i < 2 * NU; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      }
    }
    rescale(mt);
    qk(nxt);
    softmax_exp(cur);
    vread(S);
#pragma unroll
    for (int jj = 0; jj < KJ; ++jj) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 56 / KJ, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 4 * NU / KJ, 0);
    }
    // P(j) is computed here, under S(j + 1): without this the compiler sinks
    // the exponentials to their use after the barrier.
    asm volatile("" : "+v"(pop[0]), "+v"(pop[1]), "+v"(l));
    if (issue) wait_loads(std::integral_constant<int, kInFlight>{});
    else wait_loads(std::integral_constant<int, 0>{});
    lds_barrier();
  };
  // The output tile of a finished item, normalised and stored through this
  // wave's staging area (32 rows of 64 bytes) in NU rounds, one 32-dim
  // column tile per round: each lane writes its query's four 4-dim runs as
  // 8-byte pieces, then the wave stores whole 64-byte row segments as
  // 16-byte chunks. Chunk q of row r sits at position q ^ ((r >> 2) & 3),
  // which keeps a wave's writes within two-way bank conflicts.
  char* const ost = smem + OOFF + wave * kOutStage;
  auto store_out = [&](const Item& it) {
    const float rl = 1.f / (l + __shfl_xor(l, 32, 64));  // 1 / query c's denominator
    T* const obase = static_cast<T*>(a.out) + it.q_start * a.o_st + (it.kvh * NW + wave) * a.o_sh;
    const int wsw = (c >> 2) & 3;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      __builtin_amdgcn_sched_barrier(0);  // one round's addresses at a time
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const u32x2 w = {pack2<T>(acc[u][4 * g] * rl, acc[u][4 * g + 1] * rl),
                         pack2<T>(acc[u][4 * g + 2] * rl, acc[u][4 * g + 3] * rl)};
        *reinterpret_cast<u32x2*>(ost + c * 64 + 16 * (g ^ wsw) + 8 * h) = w;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int id = lane + 64 * i, r = id >> 2, q = id & 3;
        const int row = it.q0 + r;
        const u32x4 w = *reinterpret_cast<const u32x4*>(ost + r * 64 + 16 * (q ^ ((r >> 2) & 3)));
        if (row < it.q_len) *reinterpret_cast<u32x4*>(obase + row * a.o_st + 32 * u + 8 * q) = w;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    }
  };

  // ---- The item loop. The next item's K/V blocks and Q are fetched while
  // X's last block and its output are finished, so its first block is
  // usually in LDS when it starts.
  int round = 0;
  int idx = item_of(0);
  Item X;
  if (idx < n_items) {
    resolve_round(0, idx, X);
    load_q(X);
    load_head(X);
  }
  using std::integral_constant;
  while (idx < n_items) {
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[u][e] = 0.f;
    m = kNegInfP;
    l = 0.f;
    // X's K(0) and step 0 (steps 1 .. A-1 may still be in flight).
    if (X.nblk >= A) wait_loads(integral_constant<int, kInFlight>{});
    else wait_loads(integral_constant<int, 0>{});
    lds_barrier();
    // Unconditional, also for an item without keys (whose scores are never
    // used): every path into the block loop then consumes Q here, so the
    // compiler's wait for X's Q loads is placed here and not in the loop,
    // where it would also drain the K/V loads in flight.
    kread(integral_constant<int, 0>{});
    qk(sca);
    // Iteration 0's loads overwrite K(0)'s slot: every wave must have read it.
    lds_barrier();
    loop_loads_start(X);
    int j = 0;
    if (X.nblk > 1) {
      full(X, 0, integral_constant<int, 0>{}, std::false_type{});
      j = 1;
      // S(j) is in scb at the top of each round of NB blocks.
      for (; j + NB < X.nblk; j += NB) {
        full(X, j, integral_constant<int, 1 % NB>{}, std::true_type{});
        full(X, j + 1, integral_constant<int, 2 % NB>{}, std::true_type{});
        if constexpr (NB == 4) {
          full(X, j + 2, integral_constant<int, 3>{}, std::true_type{});
          full(X, j + 3, integral_constant<int, 0>{}, std::true_type{});
        }
      }
      // The remaining blocks but the last, then the last block's scores into sca.
      if (j + 1 < X.nblk) {
        full(X, j, integral_constant<int, 1 % NB>{}, std::true_type{});
        ++j;
        if constexpr (NB == 4) {
          if (j + 1 < X.nblk) {
            full(X, j, integral_constant<int, 2>{}, std::true_type{});
            ++j;
            if (j + 1 < X.nblk) {
              full(X, j, integral_constant<int, 3>{}, std::true_type{});
              ++j;
            } else {
              sca = scb;
            }
          }
        }
      } else {
        sca = scb;
      }
    }
    // X's last block j: its P V after the next item's loads are issued.
    ++round;
    const int nidx = item_of(round);
    Item Y;
    // The next item, its Q and its K blocks (the K slots are free: X's last
    // K read was before the loop's last barrier) are fetched first; its V
    // blocks wait until every wave has read X's last V block.
    if (nidx < n_items) {
      resolve_round(round, nidx, Y);
      load_q(Y);
      load_head_k(Y);
    }
    // (An item without keys has no block: its output is 0/0, as the
    // reference's.)
    if (X.nblk > 0) {
      mask_block(X, sca, j);
      if (X.nblk > 1) pv();
      rescale(block_max(sca));
      softmax_exp(sca);
      vread(j % NB);
    }
    // The next item's blocks go to slots 0 .. A: every wave must have read
    // X's last V block (whichever slot it is in) before they are issued.
    lds_barrier();
    if (nidx < n_items) load_head_v(Y);
    if (X.nblk > 0) pv();
    store_out(X);
    X = Y;
    idx = nidx;
  }
}


// Host side, in varlen_prefill.hip: the checks of tsa_varlen_prefill, filling
// a (mfma: the 16-bit MFMA kernels may serve the call); the launch of the
// kernel it selects; and whether that kernel is varlen_prefill_gqa<T, 128, 4>
// with these arguments (the one the mixed kernel embeds).
int prefill_prepare(const tsa_view* out, const tsa_view* q, const tsa_view* k, const tsa_view* v,
                    const tsa_view* cu_seqlens_q, const tsa_view* cu_seqlens_k, int64_t max_seqlen_q,
                    int64_t max_seqlen_k, int32_t causal, double softmax_scale, PrefillArgs& a, bool& mfma);
int prefill_launch(PrefillArgs& a, bool mfma, int dtype, int64_t max_seqlen_q, hipStream_t stream);
bool prefill_takes_gqa4(const PrefillArgs& a, bool mfma);
// varlen_prefill_w64.hip: its launch (bf16 or f16) and its sequence limit.
constexpr int kW64MaxSeqsHost = 2048;
int prefill_w64_launch(const PrefillArgs& a, bool bf16, hipStream_t stream);
bool prefill_w64_enabled();

}  // namespace tsa
