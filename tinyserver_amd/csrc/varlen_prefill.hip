// Varlen (packed, cu_seqlens) causal prefill attention for gfx950.
//
// Reference: server/model/kernels/varlen_attention.py:8-142 -- one program per
// (32-row query block, sequence, q-head), online softmax over 32-key blocks,
// top-left causal mask q_idx >= k_idx within the sequence (:116-119),
// P cast to the V dtype before P.V (:126), l summing the fp32 P (:128-129).
//
// Three kernels, chosen per call:
//   varlen_prefill_gqa   bf16/f16, head_dim 64/128, GQA group a divisor of 8:
//                        one workgroup per (kv head, sequence, query block),
//                        K/V staged in LDS once for the whole group, 32x32x16
//                        MFMA tiles (the main path);
//   varlen_prefill_mfma  other group sizes: 4 q-heads per workgroup, operands
//                        straight from global memory, 16x16x32 MFMA tiles;
//   varlen_prefill_generic  fp32, other head_dims or non-unit innermost
//                        strides: one wave per (query, q-head), fp32 VALU.
// Causal key blocks past a workgroup's last query are never visited, and the
// heaviest query blocks are dispatched first.
#include <cmath>
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

// LDS-staged GQA flash attention on 32x32 tiles. A workgroup of NW waves (4
// or 8) owns one kv head of one sequence and 32 NW/G queries (G = q heads per
// kv head, a divisor of NW): wave w takes the 32 queries 32 (w / G).. of
// q-head w % G, so all NW tiles read the same K/V. 32-key K/V blocks are staged once per
// workgroup in double-buffered LDS, the global loads of block i+2 in flight
// while block i is computed. Both products run on v_mfma_f32_32x32x16 (the
// 16x16x32 form has about 60% of its throughput on gfx950). With lane
// (h, c) = (lane / 32, lane % 32) and accumulator element e holding row
// 8(e/4) + 4h + e%4, column c:
//   S^T(32 keys x 32 queries) = K Q^T over head_dim/16 steps: lane (h, c)
//     reads key c, dims 16jj + 8h..+8 (row-major K, row stride D+8 elements:
//     the 16 lanes of a 128-bit read hit 16 distinct bank quads) and holds
//     query c's Q slice in registers; it gets query c's scores of keys
//     8(e/4) + 4h + e%4;
//   O(32 queries x 32 dims) += P V over two 16-key steps s: the P operand's
//     k-slots 8h..8h+7 are keys 16s+4h+0..3 and 16s+8+4h+0..3, i.e. the score
//     accumulators 8s..8s+7 of the same lane, so P goes to the operand in
//     registers; the V operand comes from two ds_read_b64_tr_b16, in which a
//     16-lane group whose lane 4e+q reads dims 4q..4q+3 of key row e gets, in
//     lane j, element e = V[key e][dim j]. V stays row-major in LDS with row
//     stride D+32 elements, so the two groups of a half-wave hit disjoint
//     banks.
// Scores, probabilities and the output accumulators all stay in VGPRs (at most
// 256 per wave, two waves per SIMD). With NW = 4 two workgroups share a CU and
// drift apart, so one workgroup's softmax overlaps the other's MFMAs. A wave
// skips the blocks whose keys all lie after its last query. Workgroup ids put
// the kv head fastest (a kv head's query blocks share one XCD's L2) and the
// heaviest query blocks first.
template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void varlen_prefill_gqa(PrefillArgs a) {
  constexpr int NT = 64 * NW;             // threads per workgroup
  constexpr int KJ = D / 16;              // 16-dim steps of the QK reduction
  constexpr int NU = D / 32;              // 32-dim column tiles of the output
  constexpr int CPR = D / 8;              // 16-byte chunks per K/V row
  constexpr int ROWK = D + 8, ROWV = D + 32, ROWO = D + 8;  // LDS row strides, elements
  constexpr int KCH = 32 * CPR;           // chunks per tensor per block
  constexpr int NCH = 2 * KCH / NT;       // chunks per thread per block
  constexpr int KBUF = 32 * ROWK, VBUF = 32 * ROWV;
  static_assert(NCH >= 1 && 2 * KCH == NT * NCH, "one K/V block is an exact number of chunks per thread");
  constexpr int SMEM = 2 * (KBUF + VBUF) > NW * 32 * ROWO ? 2 * (KBUF + VBUF) : NW * 32 * ROWO;
  // A row's running max only moves when it grows by more than this (log2
  // units): p = 2^(s - m) then stays below 2^8, and the accumulator is
  // rescaled rarely. l uses the same m, so the result is unchanged.
  constexpr float kRescale = 8.0f;
  __shared__ __align__(16) uint16_t smem[SMEM];  // K/V blocks, then the output tiles
  uint16_t* const kl = smem;               // [2][32][ROWK]
  uint16_t* const vl = smem + 2 * KBUF;    // [2][32][ROWV]

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.G, QB = 32 * NW / G;
  const int id = blockIdx.x;
  const int kvh = id % a.Hkv;
  const int rest = id / a.Hkv;
  const int b = rest % a.nseq;
  const int qblk = a.nqb - 1 - rest / a.nseq;
  int64_t q_start64, q_len64, k_start64, k_len64;
  seq_range(a.cu_q, a.cuq_s, b, a.total_q, q_start64, q_len64);
  seq_range(a.cu_k, a.cuk_s, b, a.total_k, k_start64, k_len64);
  // Positions inside one sequence fit 32 bits (cu_seqlens are int32).
  const int q_len = static_cast<int>(q_len64), k_len = static_cast<int>(k_len64);
  const int row0 = qblk * QB;
  if (row0 >= q_len) return;

  const T* kb_ptr = static_cast<const T*>(a.k) + k_start64 * a.k_st + kvh * a.k_sh;
  const T* vb_ptr = static_cast<const T*>(a.v) + k_start64 * a.v_st + kvh * a.v_sh;
  const float cs = a.scale_log2;  // > 0 on this path

  // This wave's tile: queries q0..q0+31 of q-head `head`.
  const int q0 = row0 + 32 * (wave / G);
  const int head = kvh * G + wave % G;
  u32x4 qop[KJ];
  {
    const int row = q0 + c;
    const T* qp = static_cast<const T*>(a.q) + (q_start64 + row) * a.q_st + head * a.q_sh;
#pragma unroll
    for (int jj = 0; jj < KJ; ++jj)
      qop[jj] = row < q_len ? *reinterpret_cast<const u32x4*>(qp + 16 * jj + 8 * h) : u32x4{0, 0, 0, 0};
  }

  float m = kNegInfP, l = 0.f;  // query c's running max (log2 domain) and this lane's share of its sum
  f32x16 acc[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[u][e] = 0.f;

  const int q_last = row0 + QB < q_len ? row0 + QB : q_len;  // one past the block's last query
  const int kend = a.causal ? (k_len < q_last ? k_len : q_last) : k_len;
  const int nblk = (kend + 31) / 32;
  // Keys this wave needs (its tile is 32 queries from q0).
  const int wend = q0 >= q_len ? 0 : (a.causal ? (kend < q0 + 32 ? kend : q0 + 32) : kend);

  // Chunk i of this thread: K chunks first, then V; key-major, 16 bytes
  // each. A thread's chunks share the column chunk ch0 and lie whole rows
  // apart, so each address is a per-thread offset plus a uniform term. A
  // block wholly inside the sequence loads from a uniform block pointer plus
  // those offsets. In the sequence's last, partial block keys past k_len read
  // the last key instead (no exec-masked load has to wait for a stage still
  // in flight), and those rows are zeroed when the stage is written to LDS.
  constexpr bool kSplitUniform = KCH % NT == 0;  // chunk i is all K or all V
  const int r0 = tid / CPR, ch0 = tid % CPR;
  auto chunk_isk = [&](int i) { return kSplitUniform ? NT * i < KCH : tid + NT * i < KCH; };
  auto chunk_drow = [&](int i) { return (NT * i - (chunk_isk(i) ? 0 : KCH)) / CPR; };  // row - r0
  const int64_t kst_b = a.k_st * static_cast<int64_t>(sizeof(T)), vst_b = a.v_st * static_cast<int64_t>(sizeof(T));
  const uint32_t koff0 = static_cast<uint32_t>(r0 * kst_b) + 16u * ch0;  // < 2^32: strides checked on the host
  const uint32_t voff0 = static_cast<uint32_t>(r0 * vst_b) + 16u * ch0;
  u32x4 stg[2][NCH];
  auto gload = [&](int blk, int st) {
    const int kb = blk * 32;
    if (kb + 32 <= k_len) {
      const char* kbase = reinterpret_cast<const char*>(kb_ptr) + kb * kst_b;
      const char* vbase = reinterpret_cast<const char*>(vb_ptr) + kb * vst_b;
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int dr = chunk_drow(i);
        const char* src = chunk_isk(i) ? kbase + dr * kst_b + koff0 : vbase + dr * vst_b + voff0;
        stg[st][i] = *reinterpret_cast<const u32x4*>(src);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const bool isk = chunk_isk(i);
        const int kk = min(kb + r0 + chunk_drow(i), k_len - 1);
        const T* src = isk ? kb_ptr + static_cast<int64_t>(kk) * a.k_st : vb_ptr + static_cast<int64_t>(kk) * a.v_st;
        stg[st][i] = *reinterpret_cast<const u32x4*>(src + 8 * ch0);
      }
    }
  };
  auto swrite = [&](int buf, int st, int blk) {
    const bool full = blk * 32 + 32 <= k_len;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int dr = chunk_drow(i);
      uint16_t* dst = chunk_isk(i) ? kl + buf * KBUF + (r0 + dr) * ROWK + 8 * ch0 : vl + buf * VBUF + (r0 + dr) * ROWV + 8 * ch0;
      u32x4 w = stg[st][i];
      if (!full && blk * 32 + r0 + dr >= k_len) w = u32x4{0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(dst) = w;
    }
  };

  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  auto clampb = [&](int blk) { return blk < nblk ? blk : nblk - 1; };
  // Block blk computes from LDS buffer blk & 1 while block blk + 2's global
  // loads are in flight into register stage blk & 1 and block blk + 1 (stage
  // (blk + 1) & 1) is written to the other LDS buffer. The loop is unrolled by
  // two so the stages are compile-time registers.
  auto block_step = [&](int blk, auto stage) {
    constexpr int st = decltype(stage)::value;
    gload(clampb(blk + 2), st);
    __builtin_amdgcn_sched_barrier(0);
    const int kb0 = blk * 32;
    const uint16_t* kbuf = kl + st * KBUF;
    const uint16_t* vbuf = vl + st * VBUF;
    // A block whose keys all lie after this wave's last query (or a wave
    // with no queries) contributes nothing: p would be exactly 0.
    if (kb0 < wend) {
      // S^T: lane (h, c) gets query c's scores of keys 8(e/4) + 4h + e%4.
      // All K operand reads are issued before the first MFMA, so the LDS latency
      // is paid once per block rather than once per step. The reduction over
      // head_dim runs as two interleaved accumulator chains (even and odd
      // steps), so consecutive MFMAs never wait on each other's result.
      u32x4 kop[KJ];
#pragma unroll
      for (int jj = 0; jj < KJ; ++jj) kop[jj] = *reinterpret_cast<const u32x4*>(kbuf + c * ROWK + 16 * jj + 8 * h);
      f32x16 sc0, sc1;
#pragma unroll
      for (int e = 0; e < 16; ++e) sc0[e] = sc1[e] = 0.f;
#pragma unroll
      for (int jj = 0; jj < KJ; jj += 2) {
        sc0 = mfma_k16x32<T>(kop[jj], qop[jj], sc0);
        sc1 = mfma_k16x32<T>(kop[jj + 1], qop[jj + 1], sc1);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, KJ, 0);  // the K operand reads
      __builtin_amdgcn_sched_group_barrier(0x008, KJ, 0);  // then the score MFMAs
      f32x16 sc;
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] = sc0[e] + sc1[e];

      // Keys past k_len, and (causal) keys after the query, only occur in a
      // sequence's last block or on the diagonal: a wave-uniform branch.
      if (kb0 + 32 > k_len || (a.causal && kb0 + 31 > q0)) {
        const int qq = q0 + c;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kk = kb0 + 8 * (e >> 2) + 4 * h + (e & 3);
          if (!(kk < k_len && (!a.causal || kk <= qq))) sc[e] = kNegInfP;
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
      const float mm = m == kNegInfP ? 0.f : m;
      float p[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        p[e] = fast_exp2(fmaf(sc[e], cs, -mm));
        l += p[e];
      }
      u32x4 pop[2];
#pragma unroll
      for (int s = 0; s < 2; ++s)
        pop[s] = u32x4{pack2<T>(p[8 * s], p[8 * s + 1]), pack2<T>(p[8 * s + 2], p[8 * s + 3]),
                       pack2<T>(p[8 * s + 4], p[8 * s + 5]), pack2<T>(p[8 * s + 6], p[8 * s + 7])};

      // P.V: B operand of step s, column tile u: V[keys 16s+4h+e, 16s+8+4h+e]
      // [dims 32u + c], read transposed from the row-major LDS block.
      const int jl = c & 15;
      const uint16_t* vt = vbuf + (4 * h + (jl >> 2)) * ROWV + 16 * (c >> 4) + 4 * (jl & 3);
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int u = 0; u < NU; ++u) {
          const uint16_t* base = vt + 16 * s * ROWV + 32 * u;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)base);
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + 8 * ROWV));
          const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
          acc[u] = mfma_k16x32<T>(pop[s], u32x4{lo2[0], lo2[1], hi2[0], hi2[1]}, acc[u]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    swrite(st ^ 1, st ^ 1, clampb(blk + 1));
    lds_barrier();
  };
  if (nblk > 0) {
    gload(0, 0);
    gload(clampb(1), 1);
    swrite(0, 0, 0);
    lds_barrier();
    for (int blk = 0; blk < nblk; blk += 2) {
      block_step(blk, std::integral_constant<int, 0>{});
      if (blk + 1 < nblk) block_step(blk + 1, std::integral_constant<int, 1>{});
    }
  }

  // Output: each wave stages its 32 x D tile in its own slice of the (now
  // idle) K/V buffers and stores it as 16-byte row chunks. The loop ended on
  // a workgroup barrier after every wave's last read of the K/V buffers.
  if (q0 >= q_len) return;
  uint16_t* ost = smem + wave * 32 * ROWO;
  const float rl = 1.f / (l + __shfl_xor(l, 32, 64));  // 1 / query c's denominator
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int r = 8 * (e >> 2) + 4 * h + (e & 3);
    const float rr = __shfl(rl, r, 64);
#pragma unroll
    for (int u = 0; u < NU; ++u) ost[r * ROWO + 32 * u + c] = from_float<T>(acc[u][e] * rr).x;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
  for (int i = 0; i < 32 * CPR / 64; ++i) {
    const int chunk = lane + 64 * i;
    const int r = chunk / CPR, ch = chunk % CPR;
    const int row = q0 + r;
    const u32x4 w = *reinterpret_cast<const u32x4*>(ost + r * ROWO + 8 * ch);
    if (row < q_len) {
      T* op = static_cast<T*>(a.out) + (q_start64 + row) * a.o_st + head * a.o_sh + 8 * ch;
      *reinterpret_cast<u32x4*>(op) = w;
    }
  }
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
    if (a.G <= 8 && 8 % a.G == 0 && a.scale_log2 > 0.f && a.k_st < kMaxStride && a.v_st < kMaxStride) {
      // Four waves per workgroup when the group fits (two workgroups per CU),
      // else eight.
      const int nw = 4 % a.G == 0 ? 4 : 8;
      const int QB = 32 * nw / a.G;
      a.nqb = static_cast<int32_t>((max_seqlen_q + QB - 1) / QB);
      if (a.nqb == 0) return TSA_OK;
      const dim3 grid(static_cast<uint32_t>(a.nqb) * a.nseq * a.Hkv);
      if (nw == 4) {
        if (a.D == 128) varlen_prefill_gqa<T, 128, 4><<<grid, dim3(256), 0, stream>>>(a);
        else varlen_prefill_gqa<T, 64, 4><<<grid, dim3(256), 0, stream>>>(a);
      } else {
        if (a.D == 128) varlen_prefill_gqa<T, 128, 8><<<grid, dim3(512), 0, stream>>>(a);
        else varlen_prefill_gqa<T, 64, 8><<<grid, dim3(512), 0, stream>>>(a);
      }
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
