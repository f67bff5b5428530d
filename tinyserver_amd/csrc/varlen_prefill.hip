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
//   O(32 queries x 32 dims) += P V over two 16-key steps s: the P operand's
//     k-slots 8h..8h+7 are keys 16s+4h+0..3 and 16s+8+4h+0..3, i.e. the score
//     accumulators 8s..8s+7 of the same lane, so P goes to the operand in
//     registers; the V operand comes from two ds_read_b64_tr_b16, in which a
//     16-lane group whose lane 4e+q reads dims 4q..4q+3 of key row e gets, in
//     lane j, element e = V[key e][dim j]. V stays row-major in LDS, and the
//     swizzle keeps these reads free of bank conflicts too.
// Scores, probabilities and the output accumulators all stay in VGPRs (at most
// 256 per wave, two waves per SIMD); the workgroups sharing a CU drift apart,
// so one workgroup's softmax overlaps another's MFMAs.
template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void varlen_prefill_gqa(
    PrefillArgs a, const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k) {
  constexpr int KJ = D / 16;              // 16-dim steps of the QK reduction
  constexpr int NU = D / 32;              // 32-dim column tiles of the output
  constexpr int CPR = D / 8;              // 16-byte chunks per K/V row
  constexpr int RB = 2 * D;               // bytes per K/V row in LDS (unpadded)
  constexpr int ROWO = D + 8;             // output staging row stride, elements
  constexpr int BLKB = 32 * RB;           // bytes per 32-row K or V block
  // K/V block slots in LDS and the prefetch distance in blocks: the loads
  // of a block are issued A iterations before it is needed.
  constexpr int NB = NW == 2 ? 2 : 4, A = NB - 1;
  constexpr int RPI = 1024 / RB;          // rows per 1 KB load instruction
  constexpr int IPW = 2 * (32 / RPI) / NW;  // load instructions per wave per block step
  constexpr int VOFF = NB * BLKB;           // byte offset of the V slots
  constexpr int OOFF = 2 * NB * BLKB;       // byte offset of the output staging (8 rows per wave)
  constexpr int QOFF = OOFF + NW * 8 * ROWO * 2;  // byte offset of the per-sequence query-block counts
  constexpr int SMEM = QOFF + max_persist_seqs(NW) * 2;
  static_assert(IPW >= 1 && IPW * NW == 2 * (32 / RPI), "a block step is a whole number of loads per wave");
  static_assert((A > 1 ? A - 1 : 0) * IPW <= 63, "outstanding loads fit the vmcnt field");
  // A row's running max only moves when it grows by more than this (log2
  // units): p = 2^(s - m) then stays below 2^8, and the accumulator is
  // rescaled rarely. l uses the same m, so the result is unchanged.
  constexpr float kRescale = 8.0f;
  __shared__ __align__(16) char smem[SMEM];
  uint16_t* const nqb_s = reinterpret_cast<uint16_t*>(smem + QOFF);  // query blocks of each sequence

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nseq = a.nseq, Hkv = a.Hkv;
  const float cs = a.scale_log2;  // > 0 on this path

  // ---- Work items: (query block, sequence, kv head) with a non-empty query
  // block, heaviest (latest) query blocks first: level Q holds query block Q
  // of every sequence that has one, in sequence order, kv head fastest.
  // Workgroup w takes items w, w + grid, w + 2 grid, ...: with the heaviest
  // first, that deals the work out evenly. (No work-queue atomic: a returning
  // atomic holds up every load the wave issues after it until it completes,
  // and under load that took longer than the imbalance it would remove.) The
  // per-sequence counts live in LDS.
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
    it.kb = static_cast<const T*>(a.k) + ks * a.k_st + it.kvh * a.k_sh;
    it.vb = static_cast<const T*>(a.v) + ks * a.v_st + it.kvh * a.v_sh;
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
  // (one past the end, a clamped copy of the last block). Blocks take slots
  // in order across items: block j of an item whose first block is the
  // workgroup's g-th goes to slot (g + j) % NB.
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
  // Block step s of item `it` (first block: the workgroup's g-th).
  auto load_step = [&](const Item& it, int g, int s) __attribute__((always_inline)) {
    if (k_wave) load_block(it, s + 1, (g + s + 1) % NB);
    else load_block(it, s, (g + s) % NB);
  };
  // K block 0 and steps 0 .. A - 1 (those that exist) of an item; nothing
  // for an item without keys.
  auto load_head = [&](const Item& it, int g) __attribute__((always_inline)) {
    if (it.nblk == 0) return;
    if (k_wave) load_block(it, 0, g % NB);
#pragma unroll
    for (int s0 = 0; s0 < A; ++s0)
      if (s0 < it.nblk) load_step(it, g, s0);
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
  const int ka = c * RB + 16 * (h ^ swz(c));
  u32x4 kop[KJ];
  auto kread = [&](int ks) {
    const int kb = ks * BLKB + ka;
#pragma unroll
    for (int jj = 0; jj < KJ; ++jj) kop[jj] = *reinterpret_cast<const u32x4*>(smem + (kb ^ (32 * jj)));
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
  // Masking, the running max and the (rare) rescale for block blk's scores.
  auto softmax_max = [&](const Item& it, f32x16& sc, int blk) {
    const int kb0 = blk * 32;
    // Keys past k_len, and (causal) keys after the query, only occur in a
    // sequence's last block or on the diagonal: a wave-uniform branch.
    if (kb0 + 32 > it.k_len || (a.causal && kb0 + 31 > it.q0)) {
      const int qq = it.q0 + c;
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
    if (__any(mt > m + kRescale)) {
      const float m_new = fmaxf(m, mt);
      const float alpha = m_new == kNegInfP ? 1.f : fast_exp2(m - m_new);
      l *= alpha;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float ar = __shfl(alpha, 8 * (e >> 2) + 4 * h + (e & 3), 64);
#pragma unroll
        for (int u = 0; u < NU; ++u) acc[u][e] *= ar;
      }
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
  // O += P V from the V block in slot vs: the B operand of step s, column
  // tile u is V[keys 16s+4h+e, 16s+8+4h+e][dims 32u + c], read transposed.
  // Lane (h, c) with jl = c % 16 reads 8 bytes of row 4h + jl/4 (+8, +16s),
  // dims 32u + 16(c/16) + 4(jl%4): vofs[u] for the first row; the row 8
  // further has swz XORed by 2, i.e. the byte offset XORed by 32.
  int vofs[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int jl = c & 15, r = 4 * h + (jl >> 2), ch = 4 * u + 2 * (c >> 4) + ((jl & 3) >> 1);
    vofs[u] = r * RB + 16 * (ch ^ swz(r)) + 8 * (jl & 1);
  }
  auto pv = [&](int vs) {
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
        acc[u] = mfma_k16x32<T>(pop[s2], u32x4{lo2[0], lo2[1], hi2[0], hi2[1]}, acc[u]);
      }
  };

  // Software pipeline, one 32-key block per iteration j. On entry S(j) is in
  // registers, K block j + 1 and V block j are in their LDS slots. The wave
  // issues block step j + A's loads (into the slots of K(j) and V(j - 1),
  // both last read before the previous barrier), reads K(j + 1), does the
  // max/rescale of S(j), then issues the S(j + 1) MFMAs interleaved with the
  // exponentials of S(j), so the matrix pipe and the VALU work at once, and
  // finally P(j) V(j). It then waits for step j + 1's rows and meets the
  // other waves at the barrier. Steps past the last block are not issued;
  // once they stop, fewer loads than kInFlight are younger than the one a
  // block needs, so those blocks wait for all of them.
  auto full = [&](const Item& it, int g, int j, f32x16& cur, f32x16& nxt) {
    const bool issue = j + A < it.nblk;
    if (issue) load_step(it, g, j + A);
    kread((g + j + 1) % NB);
    softmax_max(it, cur, j);
    qk(nxt);
    softmax_exp(cur);
    // One score MFMA, then a slice of the exponentials, and so on.
#pragma unroll
    for (int jj = 0; jj < KJ; ++jj) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 64 / KJ, 0);
    }
    pv((g + j) % NB);
    if (issue) wait_loads(std::integral_constant<int, kInFlight>{});
    else wait_loads(std::integral_constant<int, 0>{});
    lds_barrier();
  };
  // The output tile of a finished item, normalised and stored through this
  // wave's 8-row staging area in four rounds of 8 rows, as 16-byte chunks.
  uint16_t* const ost = reinterpret_cast<uint16_t*>(smem + OOFF) + wave * 8 * ROWO;
  auto store_out = [&](const Item& it) {
    const float rl = 1.f / (l + __shfl_xor(l, 32, 64));  // 1 / query c's denominator
    T* const obase = static_cast<T*>(a.out) + it.q_start * a.o_st + (it.kvh * NW + wave) * a.o_sh;
#pragma unroll
    for (int R = 0; R < 4; ++R) {
      __builtin_amdgcn_sched_barrier(0);  // one round's addresses at a time
#pragma unroll
      for (int e = 4 * R; e < 4 * R + 4; ++e) {
        const int rr = 4 * h + (e & 3);  // row inside the round
        const float sc = __shfl(rl, 8 * R + rr, 64);
#pragma unroll
        for (int u = 0; u < NU; ++u) ost[rr * ROWO + 32 * u + c] = from_float<T>(acc[u][e] * sc).x;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
      for (int i = 0; i < 8 * CPR / 64; ++i) {
        const int chunk = lane + 64 * i;
        const int r = chunk / CPR, ch = chunk % CPR;
        const int row = it.q0 + 8 * R + r;
        const u32x4 w = *reinterpret_cast<const u32x4*>(ost + r * ROWO + 8 * ch);
        if (row < it.q_len) *reinterpret_cast<u32x4*>(obase + row * a.o_st + 8 * ch) = w;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    }
  };

  // ---- The item loop. The next item's K/V blocks and Q are fetched while
  // X's last block and its output are finished, so its first block is
  // usually in LDS when it starts.
  int idx = blockIdx.x;
  Item X;
  if (idx < n_items) {
    resolve(idx, X);
    load_q(X);
    load_head(X, 0);
  }
  int g = 0;  // slot counter: X's block 0 is the workgroup's g-th block
  while (idx < n_items) {
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[u][e] = 0.f;
    m = kNegInfP;
    l = 0.f;
    // X's K(0) and step 0 (steps 1 .. A-1 may still be in flight).
    if (X.nblk >= A) wait_loads(std::integral_constant<int, kInFlight>{});
    else wait_loads(std::integral_constant<int, 0>{});
    lds_barrier();
    f32x16 sca, scb;  // S of the even / odd blocks
    // Unconditional, also for an item without keys (whose scores are never
    // used): every path into the block loop then consumes Q here, so the
    // compiler's wait for X's Q loads is placed here and not in the loop,
    // where it would also drain the K/V loads in flight.
    kread(g % NB);
    qk(sca);
    // Iteration 0's loads overwrite K(0)'s slot: every wave must have read it.
    lds_barrier();
    int j = 0;
    for (; j + 2 < X.nblk; j += 2) {
      full(X, g, j, sca, scb);
      full(X, g, j + 1, scb, sca);
    }
    if (j + 1 < X.nblk) {
      full(X, g, j, sca, scb);
      sca = scb;  // the last block's scores, in one place
      ++j;
    }
    // X's last block j, after all of X's loads have landed: fetch the next
    // item's blocks and Q behind X's last block, then store X's output. (The
    // next item's loads go to slots no wave reads any more: X's last V slot is
    // not among them, and every other slot was last read before the block
    // loop's final barrier.)
    const int nidx = idx + static_cast<int>(gridDim.x);
    Item Y;
    if (nidx < n_items) resolve(nidx, Y);
    // (An item without keys has no block: its output is 0/0, as the
    // reference's.)
    if (X.nblk > 0) {
      softmax_max(X, sca, j);
      softmax_exp(sca);
    }
    if (nidx < n_items) {
      load_head(Y, g + X.nblk);
      load_q(Y);
    }
    if (X.nblk > 0) pv((g + j) % NB);
    store_out(X);
    g += X.nblk;
    X = Y;
    idx = nidx;
  }
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
  // that item's Q first) but not the one after: the Q area holds one item.
  // Loads per wave: a block is 4 DMA instructions, an item's Q 16.
  int idx = blockIdx.x;
  if (idx >= n_items) return;
  Item X, N;
  resolve(idx, X);
  int nidx = idx + static_cast<int>(gridDim.x);
  bool have_n = false;     // N resolved (the load cursor entered it)
  int gl = 0, lj = 0;      // next block to issue: global index, block of the load item
  bool l_in_n = false;     // the load cursor is in N (else in X)
  int q_after = -1;        // global block index whose DMA directly follows the last Q group
  int gb = 0;              // global index of the compute block
  int slot_l = 0;          // slot of block gl
  // DMA issue for one block of the load cursor, if it may advance.
  auto issue = [&]() __attribute__((always_inline)) {
    if (!l_in_n && lj == X.nblk) {  // X fully issued: enter the next item
      if (!have_n) return false;
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

template <typename T>
static int launch_prefill(PrefillArgs& a, bool mfma, int64_t total_q, int64_t max_seqlen_q, hipStream_t stream) {
  if (a.nseq == 0 || a.Hq == 0 || total_q == 0) return TSA_OK;
  if (!mfma) {
    varlen_prefill_generic<T><<<dim3(total_q, a.Hq), dim3(64), 0, stream>>>(a, total_q);
    return check_launch("tsa_varlen_prefill");
  }
  if constexpr (sizeof(T) == 2) {
    // The LDS-staged kernel keeps 32 rows of K/V byte offsets in 32 bits.
    const int64_t kMaxStride = int64_t{1} << 24;
    if (a.D == 128 && a.G % 4 == 0 && a.scale_log2 > 0.f && a.k_st < kMaxStride && a.v_st < kMaxStride &&
        a.nseq <= kWideMaxSeqs && total_q <= int64_t{65535} * 64 && wide_enabled())
      return launch_wide<T>(a, stream);
    // (Per-sequence query-block counts are 16-bit in LDS: every sequence's
    // length is at most total_q.)
    if ((a.G == 2 || a.G == 4 || a.G == 8) && a.scale_log2 > 0.f && a.k_st < kMaxStride && a.v_st < kMaxStride &&
        a.nseq <= max_persist_seqs(a.G) && total_q <= int64_t{65535} * 32) {
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

extern "C" int tsa_varlen_prefill(const tsa_view* out, const tsa_view* q, const tsa_view* k, const tsa_view* v,
                                  const tsa_view* cu_seqlens_q, const tsa_view* cu_seqlens_k, int64_t max_seqlen_q,
                                  int64_t max_seqlen_k, int32_t causal, double softmax_scale, void* stream) {
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

  PrefillArgs a{};
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
  const bool mfma = (dt == TSA_BF16 || dt == TSA_F16) && (D == 64 || D == 128) && rows_vec16(q) && rows_vec16(k) &&
                    rows_vec16(v) && rows_vec16(out);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t total_q = q->size[0];
  switch (dt) {
    case TSA_BF16: return launch_prefill<bf16_t>(a, mfma, total_q, max_seqlen_q, st);
    case TSA_F16: return launch_prefill<f16_t>(a, mfma, total_q, max_seqlen_q, st);
    case TSA_F32: return launch_prefill<float>(a, false, total_q, max_seqlen_q, st);
  }
  set_error("unsupported dtype");
  return TSA_ERR_UNSUPPORTED;
}
