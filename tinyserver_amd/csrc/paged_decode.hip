// Paged GQA decode attention for gfx950.
//
// Reference: server/model/kernels/paged_attention.py:8-121. The reference runs
// one program per (sequence, q-head) and walks the block table serially, so
// each K/V page is re-read Hq/Hkv times and a 32k-token context is one long
// serial program. Here:
//
// * Work is the list of 16-token tiles of every (sequence, kv head) "unit",
//   unit-major. A fixed grid of workgroups (by default one 4-wave
//   workgroup per CU, all resident at once) gives each of its waves -- a
//   "wave worker" -- one equal, contiguous run of that list, so every wave
//   streams the same number of K/V bytes whatever the mix of context
//   lengths, and the whole call is a single wave of workgroups. Every K/V
//   byte is read once and shared by the G = Hq/Hkv query heads of its kv
//   head. Each wave derives the tile prefix over seq_lens itself (a
//   wave-shuffle scan into its own LDS copy), so nothing is precomputed on
//   the host.
// * A wave crosses unit boundaries without stopping: its ring keeps loading
//   the next unit's tiles (and that unit's Q) while the current unit
//   finishes, and at a unit's end it writes its partial (m, l, acc) and starts
//   afresh. No workgroup barrier follows the prefix scan.
// * Scores on the matrix cores: S^T(16 tok x 16 head) = K(16 tok x D) Q^T with
//   v_mfma_f32_16x16x32_{bf16,f16}. The K operand wants token = lane%16 and 8
//   consecutive dims per lane, which is a plain 128-bit global load (lane
//   (g, c) reads token c, dims 8(g+4j)..+8 for k-step j; the dot product is
//   order-free, so Q uses the same dim order). Each load instruction reads 16
//   contiguous 64-byte segments.
// * The accumulator of that MFMA leaves lane (g, c) holding head c for tokens
//   4g..4g+3 -- exactly the A operand of the 16x16x16 MFMA for O = P V with
//   tokens as the reduction index, so softmax weights go from the score
//   accumulator to the P.V product without any cross-lane move. V rows are
//   read row-major (16 lanes per 256-byte row, fully coalesced) and four
//   v_perm_b32 per MFMA regroup them into the token-major B operand.
// * fp32 online softmax in the log2 domain (scale pre-multiplied by log2 e,
//   v_exp_f32), the running max shared across the 4 lanes of a head by two
//   cross-lane exchanges; the accumulator is rescaled only when a head's max
//   grows, which a wave-uniform branch detects. The reference's P.V is fp32
//   (paged_attention.py:107-112): P goes to the MFMA as two cache-dtype
//   halves, hi + lo, so the weights keep 16 (bf16) or 22 (f16) significant
//   bits; l sums the fp32 p.
// * Each wave keeps a ring of RING tiles in registers: the loads of the next
//   RING-1 tiles are in flight while one is on the matrix cores. K/V loads
//   are unconditional (past its last tile a wave reloads that tile, which
//   hits the cache) so the compiler waits for exactly one tile. A unit's Q
//   operand is loaded once, with the unit's first tile (or the wave's first,
//   when its run starts inside the unit), and kept in registers.
// * A second kernel merges, per unit, the partials of the wave workers whose
//   runs cover it with a log-sum-exp reduce. The kernel boundary orders the
//   two, so no cache flushes or atomics are needed; no host sync, no memset.
// * Small batches (at most 64 units, tables of at most 512 tokens, no grid
//   asked for) run one workgroup per unit instead: its four waves split the
//   unit's tiles through the same ring, leave their partials in LDS, and
//   the workgroup merges them and writes the output. One launch.
//
// Tokens past seq_len are scored -inf and their V rows zeroed (the
// reference's masked loads, :88-105). seq_len is clamped to the block table's
// capacity, and a tile whose block id is outside [0, num_blocks) is masked
// (the reference would read out of bounds), so a malformed table cannot
// fault. seq_len == 0 yields NaN, as the reference's 0/0 does.
//
// A generic kernel (one wave per (sequence, q-head), fp32 VALU math) covers
// what the MFMA path does not: fp32 caches, head_dim other than 64/128, GQA
// groups over 16, non-unit innermost strides.
#include <atomic>
#include <cmath>
#include <mutex>
#include <type_traits>

#include "tsa_common.h"
#include "norm_rope_row.h"
#include "varlen_prefill_gqa.h"

namespace tsa {

struct DecodeArgs {
  void* out;
  const void* q;
  const void* kc;
  const void* vc;
  const int32_t* bt;
  const int32_t* seq_lens;
  int64_t o_ss, o_sh, o_sd;
  int64_t q_ss, q_sh, q_sd;
  int64_t kc_b, kc_h, kc_s, kc_d;
  int64_t vc_b, vc_h, vc_s, vc_d;
  int64_t bt_s0, bt_s1, sl_s;
  int64_t NB;
  int32_t B, Hq, Hkv, G, BS, max_blocks, D;
  int32_t W;        // workgroups of the stream kernel
  int32_t NW;       // wave workers sharing the tile list (kWaves * W)
  int32_t unit;     // 1: one workgroup per (sequence, kv head) unit, W = B * Hkv, no merge launch
  float scale_log2;
  float* part;      // [B * Hkv + NW][G * (D + 2)]: per (unit, worker) acc[G][D], m[G], l[G]
  int32_t* pref_out;  // [B + 1] tile prefix over the sequences, for the merge
  // The fused decode step only: query is the raw projection, and the new
  // token's raw k/v rows (B, Hkv, D), the norm weights (D) and the cos/sin
  // rows (B, D) come in here; eps is the RMSNorm epsilon.
  const void* kn; const void* vn; const void* qw; const void* kw; const void* cos; const void* sin;
  void* kc_out; void* vc_out;  // the caches, written (the new token's rows)
  int64_t kn_ss, kn_sh, vn_ss, vn_sh, cs_ss, sn_ss;
  float eps;
};

template <typename T>
__device__ __forceinline__ u32x4 pack8(const float (&v)[8]) {
  u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack2<T>(v[2 * i], v[2 * i + 1]);
  return w;
}

// An LDS byte address (of this wave's fused area) as a 16-byte pointer.
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
__device__ __forceinline__ lds_u32x4* lds16(uint32_t addr) { return (lds_u32x4*)(uintptr_t)addr; }

// In place, norm + RoPE of the 128-dim rows at LDS byte address rows (256 B
// apart): lane l takes row first + l / 16, 8-dim chunk l % 16 (a DPP row of
// 16 lanes per head row), with the weights at w and the cos/sin rows at cs
// (sin follows at cs + 256). The arithmetic is the norm/RoPE kernels' own
// norm_rope_row, so the rounding is identical to theirs. Rows past last are
// not written (their lanes redo row last).
template <typename T>
__device__ __forceinline__ void norm_rope_rows_lds(uint32_t rows, int first, int last, uint32_t w, uint32_t cs,
                                                   float eps) {
  const int lane = threadIdx.x & 63, r = first + (lane >> 4), ch = lane & 15;
  const int rr = min(r, last);
  float x[8], wf[8], csf[8], snf[8], o[8];
  auto get = [](uint32_t addr, float (&out)[8]) {
    const u32x4 v = *lds16(addr);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = lo_f<T>(v[i]);
      out[2 * i + 1] = hi_f<T>(v[i]);
    }
  };
  get(rows + 256 * rr + 16 * ch, x);
  get(w + 16 * ch, wf);
  get(cs + 16 * ch, csf);
  get(cs + 256 + 16 * ch, snf);
  norm_rope_row<T, 128>(x, wf, csf, snf, eps, ch, o);
  if (r <= last) *lds16(rows + 256 * r + 16 * ch) = pack8<T>(o);
  // Keep the wave's later LDS reads after these writes (LDS runs a wave's
  // accesses in order; this stops the compiler from moving them).
  asm volatile("" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

// Waves per stream-kernel workgroup, and workgroups per CU of the default
// grid (TSA_DECODE_WAVES * TSA_DECODE_WG_PER_CU waves per CU in all).
#ifndef TSA_DECODE_WAVES
#define TSA_DECODE_WAVES 4
#endif
#ifndef TSA_DECODE_WG_PER_CU
#define TSA_DECODE_WG_PER_CU 1
#endif
constexpr int kWaves = TSA_DECODE_WAVES;
constexpr int kThreads = 64 * kWaves;
constexpr float kNegInf = -INFINITY;

// Minimum waves per SIMD the stream kernel is compiled for (register budget:
// 512 / waves VGPRs per lane), and the number of tiles each wave keeps in
// registers (RING - 1 in flight while one computes).
#ifndef TSA_DECODE_WAVES_PER_EU
#define TSA_DECODE_WAVES_PER_EU 2
#endif
#ifndef TSA_DECODE_RING
#define TSA_DECODE_RING 3
#endif
constexpr int RING = TSA_DECODE_RING;

// Fused decode step: per wave, 1 KB of norm weights and RING unit buffers of
// kUnitBytes in LDS after the tile prefixes. A unit buffer holds the raw q
// rows of its G <= 8 heads (2 KB), then the cos, sin, raw k and raw v rows of
// the sequence's new token (256 B each at head_dim 128).
constexpr int kUnitBytes = 3072;
// The fused step's per-step values, kept in the wave's LDS area and read at
// the unit events: held in scalar registers through the tile loop they
// overflow them, and the spill reloads land in the loop.
struct FusedState {
  const void* q; const void* cos; const void* sin; const void* kn; const void* vn;
  void* kc_out; void* vc_out;
  int64_t q_ss, q_sh, cs_ss, sn_ss, kn_ss, kn_sh, vn_ss, vn_sh;
  float eps;
};
constexpr int kStateOff = 1024 + RING * kUnitBytes;
constexpr int kFusedWaveBytes = kStateOff + 128;
static_assert(sizeof(FusedState) <= 128, "fused state exceeds its LDS slot");

// K/V are read exactly once per call, with non-temporal loads (the
// streaming hint). A gather of the same 4 KB pages with the same static
// split and no arithmetic moves the Qwen3-8B batch-64 pool in about 97 us
// with them and 111 us without. They pay only because Q is not in the
// stream: loaded once per unit (not per tile, an ordinary-load L2 read of
// half the K/V bytes again), the non-temporal K/V stream takes this kernel
// from 127 to 114 us on the same box; with the per-tile Q reads it took 124.
// A wave whose run has fewer than kStreamNtMin tiles uses ordinary loads.
// The fused step keeps ordinary loads for runs below kFusedNtMin tiles: with
// non-temporal loads there, its Qwen3-8B batch-64 step measured 138 us
// against 130.
#ifndef TSA_DECODE_NT_MIN_TILES
#define TSA_DECODE_NT_MIN_TILES 0
#endif
constexpr int kStreamNtMin = TSA_DECODE_NT_MIN_TILES;
#ifndef TSA_FUSED_NT_MIN_TILES
#define TSA_FUSED_NT_MIN_TILES 128
#endif
constexpr int kFusedNtMin = TSA_FUSED_NT_MIN_TILES;
template <bool NT, typename T>
__device__ __forceinline__ u32x4 load_stream(const T* p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ int64_t clamp_len(const DecodeArgs& a, int s) {
  int64_t L = a.seq_lens[s * a.sl_s];
  const int64_t cap = static_cast<int64_t>(a.max_blocks) * a.BS;
  return L < 0 ? 0 : (L > cap ? cap : L);
}

__device__ __forceinline__ int tiles_of(const DecodeArgs& a, int s) {
  return static_cast<int>((clamp_len(a, s) + 15) >> 4);
}

// Exclusive prefix of tiles per sequence into pref[0..B] (pref[B] = total),
// computed by one wave alone into its own LDS copy: lane i sums sequences
// [i * per, (i + 1) * per), a DPP scan combines the lanes, and no
// workgroup barrier is needed. Only this wave reads pref afterwards.
__device__ void tile_prefix_wave(const DecodeArgs& a, int* pref) {
  const int lane = threadIdx.x & 63;
  const int per = (a.B + 63) / 64;
  int local = 0;
  for (int i = 0; i < per; ++i) {
    const int s = lane * per + i;
    if (s < a.B) local += tiles_of(a, s);
  }
  const int incl = static_cast<int>(wave_scan_u32(static_cast<uint32_t>(local)));
  int run = incl - local;  // exclusive prefix of this lane's first sequence
  for (int i = 0; i < per; ++i) {
    const int s = lane * per + i;
    if (s < a.B) {
      pref[s] = run;
      run += tiles_of(a, s);
    }
  }
  if (lane == 63) pref[a.B] = incl;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Position of one wave in the global tile list (unit-major): unit (s, kvh),
// tile t of the unit's n tiles. Wave-uniform; empty sequences are skipped.
// One workgroup per unit: the four waves' partials (acc[G][D], m[G], l[G],
// padded to 16 bytes) in LDS after the tile prefixes -- or, in the fused
// step, at the start of each wave's own area, which its stream no longer
// reads once the partial is written (no LDS DMA is in flight by then: the
// only one, the unit's, lands before the wave's first tile is computed).
__host__ __device__ inline int unit_slot_floats(int G, int D) { return (G * (D + 2) + 3) & ~3; }
__host__ __device__ inline int prefix_lds_bytes16(int B) { return (kWaves * (B + 1) * 4 + 15) & ~15; }
static_assert(kFusedWaveBytes >= 8 * (128 + 2) * 4, "a fused wave's area holds its partial (G <= 8, head_dim 128)");
template <bool FUSED>
__device__ __forceinline__ float* unit_slot(const DecodeArgs& a, int* lds_i, int w) {
  char* const base = reinterpret_cast<char*>(lds_i) + prefix_lds_bytes16(a.B);
  if constexpr (FUSED) return reinterpret_cast<float*>(base + w * kFusedWaveBytes);
  else return reinterpret_cast<float*>(base) + w * unit_slot_floats(a.G, a.D);
}

// Workgroup barrier over the LDS partials only. The fences order LDS and not
// global memory, so the barrier does not wait for the ring's last loads
// (repeats of the wave's last tile, whose registers nothing reads).
__device__ __forceinline__ void unit_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The merge of one unit's wave partials (after the workgroup barrier):
// output (head h, dim d) combines the waves that had tiles in wave order,
// with the running-max rescale of paged_decode_stream_merge. A unit with no
// tiles (seq_len 0) gives 0/0 = NaN, as the reference's does.
template <typename T, bool FUSED>
__device__ __forceinline__ void unit_merge(const DecodeArgs& a, int* lds_i) {
  const int Hkv = a.Hkv, G = a.G, D = a.D;
  const int s = blockIdx.x / Hkv, kvh = blockIdx.x - s * Hkv;
  const int n = lds_i[s + 1] - lds_i[s];  // wave 0's prefix copy
  const int q = (n + kWaves - 1) / kWaves;
  const int nw = n == 0 ? 0 : (n + q - 1) / q;
  T* orow = static_cast<T*>(a.out) + s * a.o_ss + (kvh * G) * a.o_sh;
  for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
    const int hd = idx / D;
    float M = kNegInf, den = 0.f, o = 0.f;
    for (int w = 0; w < nw; ++w) {
      const float* sl = unit_slot<FUSED>(a, lds_i, w);
      const float mb = sl[G * D + hd], lb = sl[G * D + G + hd], ab = sl[idx];
      const float mn = fmaxf(M, mb);
      if (mn == kNegInf) continue;
      const float c_old = fast_exp2(M - mn), c_new = fast_exp2(mb - mn);
      o = o * c_old + ab * c_new;
      den = den * c_old + lb * c_new;
      M = mn;
    }
    orow[hd * a.o_sh + (idx - hd * D) * a.o_sd] = from_float<T>(o / den);
  }
}

struct TileCursor {
  int s, kvh, n, t;
  // Values read from the LDS prefix go through readfirstlane, so the compiler
  // keeps the cursor (and the block-table addresses built from it) in SGPRs.
  __device__ __forceinline__ void next_unit(const int* pref, int B, int Hkv) {
    if (++kvh == Hkv) {
      kvh = 0;
      int nn = 0;
      while (nn == 0 && ++s < B) nn = __builtin_amdgcn_readfirstlane(pref[s + 1] - pref[s]);
      s = __builtin_amdgcn_readfirstlane(s);
    }
    n = s < B ? __builtin_amdgcn_readfirstlane(pref[s + 1] - pref[s]) : 0;
    t = 0;
  }
  __device__ __forceinline__ void advance(const int* pref, int B, int Hkv) {
    if (++t == n) next_unit(pref, B, Hkv);
  }
};

// Wave worker v = 4 * workgroup + wave streams the contiguous tiles
// [v * share, (v + 1) * share) of the global list, crossing unit boundaries
// without stopping: its ring of RING tiles (K operand and V rows, plus the
// unit's Q operand at a unit's first tile) keeps prefetching into the next
// unit while the current one finishes. At the end of each of its units the wave writes
// its partial (m, l, acc) to workspace slot unit + v (injective, since a
// worker's units form a range that starts where the previous worker's ended)
// and starts afresh; nothing waits for the other waves. The merge kernel
// combines every unit's partials.
// The block table, seq_lens and the partial buffer come in again as
// __restrict__ parameters: with the partial stores inside the loop, that is
// what lets the compiler read block-table entries and lengths with scalar
// loads.
// decode_stream_body runs workgroup blockIdx.x of that grid (the first
// workgroups of the launch); lds_i is the workgroup's LDS: kWaves tile prefixes of B + 1 ints, then (fused step)
// kWaves areas of kFusedWaveBytes at the next 16-byte boundary. With GPREF
// (batches whose prefixes would not fit in LDS) the waves read the tile
// prefix that decode_tile_prefix wrote to the workspace instead, and the
// workgroup takes no LDS.
template <typename T, int D, bool PAGE16, bool CONTIG, bool FUSED, bool GPREF = false, bool UNIT = false>
__device__ __forceinline__ void decode_stream_body(DecodeArgs a, const int32_t* __restrict__ bt,
                                                   const int32_t* __restrict__ sl, float* __restrict__ part,
                                                   int* lds_i) {
  static_assert(!(GPREF && FUSED), "the fused step keeps its tile prefixes in LDS");
  static_assert(!(GPREF && UNIT), "one workgroup per unit keeps its tile prefixes in LDS");
  constexpr int KJ = D / 32;  // k-steps of the score MFMA
  a.bt = bt;
  a.seq_lens = sl;
  a.part = part;
  const int G = a.G, Hkv = a.Hkv;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
  // Wave-uniform (scalar) so tile indices, block-table reads and page bases
  // stay in SGPRs and the table lookups are scalar loads.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // One workgroup per unit, 16-token pages: lane i holds the unit's block-table
  // entry i, loaded beside the sequence lengths, and each tile's page id is a
  // lane read rather than a dependent scalar load. (The plan takes this form
  // only for tables of at most kUnitMaxTiles = 32 tiles per unit, so 16-token
  // or larger pages give at most 32 entries, within the wave's 64 lanes.)
  int btv = 0;
  if constexpr (UNIT && PAGE16) {
    const int us = blockIdx.x / Hkv;
    if (lane < a.max_blocks) btv = bt[us * a.bt_s0 + lane * a.bt_s1];
  }
  const int* pref;
  if constexpr (GPREF) {
    pref = a.pref_out;  // [B + 1], written by decode_tile_prefix before this launch
  } else {
    int* const mine = lds_i + wave * (a.B + 1);  // this wave's copy, [B + 1]
    tile_prefix_wave(a, mine);
    if (blockIdx.x == 0 && wave == 0)
      for (int i = lane; i <= a.B; i += 64) a.pref_out[i] = mine[i];
    pref = mine;
  }

  // Fused step: this wave's LDS area (weights, then the unit ring). Data
  // arrives by LDS DMA (global_load_lds_dwordx4: lane l's 16 bytes land at
  // M0 + 16 l), issued before the tile loads that need it: loads complete in
  // issue order, so once a tile's K/V registers are waited for, the unit data
  // issued before them is in LDS.
  typedef __attribute__((address_space(3))) void lds_void;
  const int fused_off = ((kWaves * (a.B + 1) * 4 + 15) & ~15) + wave * kFusedWaveBytes;
  char* const fbuf = reinterpret_cast<char*>(lds_i) + fused_off;
  const uint32_t fbuf_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)fbuf));  // address-space cast
  auto dma64 = [&](const void* src, uint32_t lds_byte) __attribute__((always_inline)) {
    dma16(src, __builtin_amdgcn_readfirstlane(lds_byte));
  };

  const int v = blockIdx.x * kWaves + wave;
  int64_t lo, hi;
  if constexpr (UNIT) {
    // Workgroup u takes unit (u / Hkv, u % Hkv); wave w its w-th quarter
    // of the unit's n tiles (ceil(n / kWaves) each, the last waves fewer or
    // none). The wave's partial goes to LDS and the workgroup merges.
    const int us = blockIdx.x / Hkv, ukvh = blockIdx.x - us * Hkv;
    const int n = __builtin_amdgcn_readfirstlane(pref[us + 1] - pref[us]);
    const int q = (n + kWaves - 1) / kWaves;
    const int64_t u0 = static_cast<int64_t>(Hkv) * __builtin_amdgcn_readfirstlane(pref[us]) +
                       static_cast<int64_t>(ukvh) * n;
    lo = u0 + min(n, wave * q);
    hi = u0 + min(n, (wave + 1) * q);
  } else {
    const int64_t total = static_cast<int64_t>(Hkv) * pref[a.B];
    const int64_t share = (total + a.NW - 1) / a.NW;
    lo = static_cast<int64_t>(v) * share;
    hi = min(total, lo + share);
  }
  if (lo >= hi) return;  // no barrier follows (one workgroup per unit: the caller's barrier)
  const int n_tiles = static_cast<int>(hi - lo);
  if constexpr (FUSED) {  // weights: lanes 0-15 q_weight, 16-31 k_weight (32-63 repeat them)
    const T* wsrc = static_cast<const T*>((lane & 16) ? a.kw : a.qw) + 8 * (lane & 15);
    dma64(wsrc, fbuf_lds);
    if (lane == 0)
      *reinterpret_cast<FusedState*>(fbuf + kStateOff) =
          FusedState{a.q, a.cos, a.sin, a.kn, a.vn, a.kc_out, a.vc_out, a.q_ss, a.q_sh,
                     a.cs_ss, a.sn_ss, a.kn_ss, a.kn_sh, a.vn_ss, a.vn_sh, a.eps};
    asm volatile("" ::: "memory");
    __builtin_amdgcn_wave_barrier();
  }

  // Locate tile lo: the last sequence with Hkv * pref[s] <= lo (that skips
  // empty sequences), then the kv head and the tile inside it.
  TileCursor cur;
  {
    int l0 = 0, h0 = a.B;  // answer in [l0, h0): Hkv pref[l0] <= lo < Hkv pref[h0]
    if constexpr (GPREF) {
      // The prefix is in global memory: each step probes 64 evenly spaced
      // entries at once (one load per lane) and keeps the interval between
      // the last probe <= lo and the next, so a batch of B sequences takes
      // about log64(B) dependent loads instead of log2(B).
      while (h0 - l0 > 1) {
        const int step = (h0 - l0 + 63) / 64;
        const int idx = l0 + lane * step;
        const bool le = idx < h0 && static_cast<int64_t>(Hkv) * pref[idx] <= lo;
        const int cnt = __builtin_popcountll(__ballot(le));  // >= 1: the probe at l0
        l0 = __builtin_amdgcn_readfirstlane(l0 + (cnt - 1) * step);
        h0 = min(h0, l0 + step);
      }
    } else {
      while (h0 - l0 > 1) {
        const int mid = (l0 + h0) >> 1;
        if (static_cast<int64_t>(Hkv) * pref[mid] <= lo) l0 = mid; else h0 = mid;
      }
    }
    cur.s = __builtin_amdgcn_readfirstlane(l0);
    cur.n = __builtin_amdgcn_readfirstlane(pref[cur.s + 1] - pref[cur.s]);
    const int64_t off = lo - static_cast<int64_t>(Hkv) * __builtin_amdgcn_readfirstlane(pref[cur.s]);
    cur.kvh = __builtin_amdgcn_readfirstlane(static_cast<int>(off / cur.n));
    cur.t = __builtin_amdgcn_readfirstlane(static_cast<int>(off - static_cast<int64_t>(cur.kvh) * cur.n));
  }
  const bool v_lane = 8 * c < D;
  const int cq = c % G;  // lanes past the group load a real head; their rows are never stored
  // Slot strides: the contiguous pool layout makes them the compile-time D.
  const int64_t ks = CONTIG ? D : a.kc_s;
  const int64_t vs = CONTIG ? D : a.vc_s;

  auto page_of = [&](const int32_t* bt_row, int64_t tok, int64_t& phys, int64_t& slot) -> bool {
    const int64_t lb = tok / a.BS;
    phys = bt_row[lb * a.bt_s1];
    slot = tok - lb * a.BS;
    return phys >= 0 && phys < a.NB;
  };
  // The page of a tile's first token (tok wave-uniform).
  auto tile_page = [&](const int32_t* bt_row, int64_t tok, int64_t& phys, int64_t& slot) -> bool {
    if constexpr (UNIT && PAGE16) {
      const int lb = static_cast<int>(tok / a.BS);
      phys = __builtin_amdgcn_readlane(btv, lb);
      slot = tok - static_cast<int64_t>(lb) * a.BS;
      return phys >= 0 && phys < a.NB;
    } else {
      return page_of(bt_row, tok, phys, slot);
    }
  };

  // One tile's operands: Q^T (lane (g, c): head c, dims 8(g + 4j)..+8), the K
  // operand (token c of the tile, same dims) and V rows (tokens 4g..4g+3).
  // With 16-token pages the loads are unconditional (an invalid page id reads
  // page 0 and the tile is masked in compute), so nothing waits on the data
  // until it is consumed.
  auto load_tile = [&](const TileCursor& tc, u32x4 (&qo)[KJ], u32x4 (&ko)[KJ], u32x4 (&vo)[4], auto nt, bool first) {
    constexpr bool NT = decltype(nt)::value;
    const int32_t* bt_row = a.bt + tc.s * a.bt_s0;
    if constexpr (!FUSED) {  // (fused: Q is made once per unit, from LDS)
      // The unit's Q operand, once per unit: at its first tile, or at the
      // wave's first tile when its run starts inside the unit. Issued ahead
      // of the tile's K/V, so the wait for those covers it.
      if (tc.t == 0 || first) {
        const T* qrow = static_cast<const T*>(a.q) + tc.s * a.q_ss + (tc.kvh * G + cq) * a.q_sh + 8 * g;
#pragma unroll
        for (int j = 0; j < KJ; ++j) qo[j] = *reinterpret_cast<const u32x4*>(qrow + 32 * j);
      }
    }
    const T* kbase = static_cast<const T*>(a.kc) + tc.kvh * a.kc_h;
    const T* vbase = static_cast<const T*>(a.vc) + tc.kvh * a.vc_h;
    const int64_t tok0 = static_cast<int64_t>(tc.t) * 16;
    if constexpr (PAGE16) {
      int64_t phys, slot0;
      if (!tile_page(bt_row, tok0, phys, slot0)) phys = 0;
      const T* kp = kbase + phys * a.kc_b + (slot0 + c) * ks + 8 * g;
#pragma unroll
      for (int j = 0; j < KJ; ++j) ko[j] = load_stream<NT>(kp + 32 * j);
      const T* vp = vbase + phys * a.vc_b + (slot0 + 4 * g) * vs + (v_lane ? 8 * c : 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) vo[r] = load_stream<NT>(vp + r * vs);
    } else {
      const int64_t L = clamp_len(a, tc.s);
      int64_t phys, slot;
      const int64_t tk = tok0 + c;
      const bool okk = tk < L && page_of(bt_row, tk, phys, slot);
      const T* kp = kbase + (okk ? phys * a.kc_b + slot * ks : 0);
#pragma unroll
      for (int j = 0; j < KJ; ++j)
        ko[j] = okk ? load_stream<NT>(kp + 8 * (g + 4 * j)) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t tv = tok0 + 4 * g + r;
        const bool okv = v_lane && tv < L && page_of(bt_row, tv, phys, slot);
        vo[r] = okv ? load_stream<NT>(vbase + phys * a.vc_b + slot * vs + 8 * c)
                    : u32x4{0, 0, 0, 0};
      }
    }
  };

  float m = kNegInf;  // running max of head c (log2 domain), same in all 4 row-groups
  float l = 0.f;      // this lane's share of head c's softmax denominator
  f32x4 acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute_tile = [&](const TileCursor& tc, const u32x4 (&qo)[KJ], const u32x4 (&ko)[KJ], u32x4 (&vo)[4]) {
    const int64_t tok0 = static_cast<int64_t>(tc.t) * 16;
    // Tokens past seq_len, and (page-16 path) tiles whose block id is out of
    // range, are masked: score -inf and V rows zeroed so 0 * (inf/nan) cannot
    // leak into the accumulator. Only the last tile of a sequence (or a bad
    // page) takes this wave-uniform branch.
    int64_t lim = tc.t + 1 < tc.n ? tok0 + 16 : clamp_len(a, tc.s);
    if constexpr (PAGE16) {
      int64_t phys, slot0;
      if (!tile_page(a.bt + tc.s * a.bt_s0, tok0, phys, slot0)) lim = tok0;
    }
    if (tok0 + 16 > lim) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (tok0 + 4 * g + r >= lim) vo[r] = u32x4{0, 0, 0, 0};
    }
    f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KJ; ++j) sc = mfma_k32<T>(ko[j], qo[j], sc);
    // sc[r] = q_c . k_{tok0 + 4g + r}
    const int64_t tb = tok0 + 4 * g;
    float sv[4];
    float tmax = kNegInf;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sv[r] = tb + r < lim ? sc[r] * a.scale_log2 : kNegInf;
      tmax = fmaxf(tmax, sv[r]);
    }
    // (across the 4 row groups: lane swaps, no LDS round trip)
    tmax = fmaxf(tmax, __builtin_bit_cast(float, xor_lane32<16>(__builtin_bit_cast(uint32_t, tmax), lane)));
    tmax = fmaxf(tmax, __builtin_bit_cast(float, xor_lane32<32>(__builtin_bit_cast(uint32_t, tmax), lane)));
    const float m_new = fmaxf(m, tmax);
    if (__any(m_new > m)) {
      const float alpha = m_new == kNegInf ? 1.f : fast_exp2(m - m_new);  // 0 on the first tile
      l *= alpha;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float ar = __shfl(alpha, 4 * g + r, 64);  // alpha of head 4g + r
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[u][r] *= ar;
      }
      m = m_new;
    }
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = m == kNegInf ? 0.f : fast_exp2(sv[r] - m);
      l += p[r];
    }
    // P.V with fp32-grade P, as the reference's fp32 p times V: p = hi + lo
    // with hi = p rounded to the cache dtype and lo = (p - hi) rounded, two
    // MFMAs per output block (hi + lo carries 16 significant bits for bf16,
    // 22 for f16; V is exact in either). The matrix cores have the slack:
    // this kernel streams memory.
    const u32x2 phi = u32x2{pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3])};
    const u32x2 plo = u32x2{pack2<T>(p[0] - lo_f<T>(phi[0]), p[1] - hi_f<T>(phi[0])),
                            pack2<T>(p[2] - lo_f<T>(phi[1]), p[3] - hi_f<T>(phi[1]))};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int wd = u >> 1;
      u32x2 bop;
      if (u & 1) {
        bop[0] = pack_hi(vo[0][wd], vo[1][wd]);
        bop[1] = pack_hi(vo[2][wd], vo[3][wd]);
      } else {
        bop[0] = pack_lo(vo[0][wd], vo[1][wd]);
        bop[1] = pack_lo(vo[2][wd], vo[3][wd]);
      }
      acc[u] = mfma_k16<T>(phi, bop, acc[u]);  // acc[u][r] = O[head 4g + r][dim 8c + u]
      acc[u] = mfma_k16<T>(plo, bop, acc[u]);
    }
  };

  // This wave's partial of unit (s, kvh) to slot unit + v: acc[G][D], then
  // m[G], l[G]; then a fresh state for the next unit.
  const int64_t slot_floats = static_cast<int64_t>(G) * (D + 2);
  auto flush = [&](const TileCursor& tc) {
    float lt = l;
    lt += __shfl_xor(lt, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    float* slot;
    if constexpr (UNIT) slot = unit_slot<FUSED>(a, lds_i, wave);
    else slot = a.part + (static_cast<int64_t>(tc.s) * Hkv + tc.kvh + v) * slot_floats;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int hd = 4 * g + r;
      if (hd < G && v_lane) {
        float* dst = slot + hd * D + 8 * c;
        *reinterpret_cast<f32x4*>(dst) = f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
        *reinterpret_cast<f32x4*>(dst + 4) = f32x4{acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
      }
    }
    if (g == 0 && c < G) {
      slot[G * D + c] = m;
      slot[G * D + G + c] = lt;
    }
    m = kNegInf;
    l = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  };

  // Ring of RING tile buffers; the load cursor runs RING tiles ahead of the
  // compute cursor and stops on the wave's last tile (repeats hit the cache),
  // so every load is unconditional and each compute waits for its own tile.
  u32x4 qbuf[RING][KJ], kbuf[RING][KJ], vbuf[RING][4];

  // ---- Fused step. unit_dma: a unit's raw q rows, and the cos/sin/raw k/raw v
  // rows of its sequence's new token, into unit buffer ub (issued before the
  // unit's first tile loads). make_q: the unit's normalised, rotated Q
  // operand. new_token: in the unit's last tile, the new token's rotated K
  // and raw V replace the cache rows that do not hold them yet, and are
  // stored to the cache after the tile.
  u32x4 qn[KJ];  // the current unit's Q operand
  auto unit_dma = [&](const TileCursor& tc, int ub) __attribute__((always_inline)) {
    const FusedState fs = *reinterpret_cast<const FusedState*>(fbuf + kStateOff);
    const uint32_t base = fbuf_lds + 1024 + ub * kUnitBytes;
    for (int i = 0; 4 * i < G; ++i) {  // heads 4i .. 4i+3, 16 lanes each
      const int hh = min(4 * i + (lane >> 4), G - 1);
      dma64(static_cast<const T*>(fs.q) + tc.s * fs.q_ss + (tc.kvh * G + hh) * fs.q_sh + 8 * (lane & 15),
            base + 1024 * i);
    }
    const int part = lane >> 4, ch = 8 * (lane & 15);
    const T* src = part == 0   ? static_cast<const T*>(fs.cos) + tc.s * fs.cs_ss + ch
                   : part == 1 ? static_cast<const T*>(fs.sin) + tc.s * fs.sn_ss + ch
                   : part == 2 ? static_cast<const T*>(fs.kn) + tc.s * fs.kn_ss + tc.kvh * fs.kn_sh + ch
                               : static_cast<const T*>(fs.vn) + tc.s * fs.vn_ss + tc.kvh * fs.vn_sh + ch;
    dma64(src, base + 2048);
  };
  // The unit's G q rows normalised and rotated in place (four rows per
  // pass of the wave), then read back in the operand layout: lane (g, c)
  // takes chunks g + 4j of head c % G.
  auto make_q = [&](int ub) __attribute__((always_inline)) {
    const FusedState fs = *reinterpret_cast<const FusedState*>(fbuf + kStateOff);
    const uint32_t base = fbuf_lds + 1024 + ub * kUnitBytes;
    for (int first = 0; first < G; first += 4)
      norm_rope_rows_lds<T>(base, first, G - 1, fbuf_lds, base + 2048, fs.eps);
#pragma unroll
    for (int j = 0; j < KJ; ++j) qn[j] = *lds16(base + 256 * cq + 16 * (g + 4 * j));
  };
  // The new token (position L - 1) in the tile starting at tok0.
  auto new_token = [&](const TileCursor& tc, int ub, u32x4 (&ko)[KJ], u32x4 (&vo)[4], u32x4 (&kn)[KJ], u32x4& vnew,
                       int& cn) __attribute__((always_inline)) {
    const FusedState fs = *reinterpret_cast<const FusedState*>(fbuf + kStateOff);
    const int64_t L = clamp_len(a, tc.s);
    cn = static_cast<int>(L - 1 - static_cast<int64_t>(tc.t) * 16);  // 0..15
    const int ubo = 1024 + ub * kUnitBytes;
    const uint32_t ubase = fbuf_lds + ubo;
    norm_rope_rows_lds<T>(ubase + 2048 + 512, 0, 0, fbuf_lds + 256, ubase + 2048, fs.eps);  // the new k row
#pragma unroll
    for (int j = 0; j < KJ; ++j) kn[j] = *lds16(ubase + 2048 + 512 + 16 * (g + 4 * j));
    vnew = *reinterpret_cast<const u32x4*>(fbuf + ubo + 2048 + 768 + 16 * c);
#pragma unroll
    for (int j = 0; j < KJ; ++j)
      if (c == cn) ko[j] = kn[j];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (4 * g + r == cn) vo[r] = vnew;
  };
  auto store_new_token = [&](const TileCursor& tc, const u32x4 (&kn)[KJ], const u32x4& vnew, int cn) {
    const FusedState fs = *reinterpret_cast<const FusedState*>(fbuf + kStateOff);
    int64_t phys, slot;
    if (!page_of(a.bt + tc.s * a.bt_s0, clamp_len(a, tc.s) - 1, phys, slot)) return;  // (as the standalone store)
    T* kd = static_cast<T*>(fs.kc_out) + tc.kvh * a.kc_h + phys * a.kc_b + slot * ks;
    T* vd = static_cast<T*>(fs.vc_out) + tc.kvh * a.vc_h + phys * a.vc_b + slot * vs;
    if (c == cn) {
#pragma unroll
      for (int j = 0; j < KJ; ++j) *reinterpret_cast<u32x4*>(kd + 8 * (g + 4 * j)) = kn[j];
    }
    if (4 * g <= cn && cn < 4 * g + 4 && v_lane) *reinterpret_cast<u32x4*>(vd + 8 * c) = vnew;
  };

  auto stream = [&](auto nt) {
    TileCursor ld = cur;
    int ld_left = n_tiles - 1;  // advances the load cursor may still make
    int ld_unit = 0, cu_unit = 0;  // units entered by the load / compute cursor (fused)
    auto advance_load = [&]() {
      if (ld_left > 0) {
        ld.advance(pref, a.B, Hkv);
        --ld_left;
        if constexpr (FUSED) {
          if (ld.t == 0) unit_dma(ld, ++ld_unit % RING);
        }
      }
    };
    if constexpr (FUSED) unit_dma(ld, 0);
#pragma unroll
    for (int d = 0; d < RING; ++d) {
      load_tile(ld, qbuf[d], kbuf[d], vbuf[d], nt, d == 0);
      advance_load();
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int i = 0; i < n_tiles; i += RING) {
#pragma unroll
      for (int d = 0; d < RING; ++d) {
        if (i + d < n_tiles) {
          if constexpr (FUSED) {
            const bool ustart = cur.t == 0 && i + d > 0;
            if (ustart) ++cu_unit;
            const bool ulast = cur.t + 1 == cur.n;
            if (ustart || i + d == 0 || ulast) {
              // The tile's K/V have landed, so has this unit's LDS data.
              asm volatile("" ::"v"(kbuf[d][0]), "v"(vbuf[d][0]));
              if (ustart || i + d == 0) make_q(cu_unit % RING);
            }
            if (ulast) {
              u32x4 kn[KJ], vnew;
              int cn;
              new_token(cur, cu_unit % RING, kbuf[d], vbuf[d], kn, vnew, cn);
              compute_tile(cur, qn, kbuf[d], vbuf[d]);
              store_new_token(cur, kn, vnew, cn);
            } else {
              compute_tile(cur, qn, kbuf[d], vbuf[d]);
            }
          } else {
            if (cur.t == 0 || i + d == 0) {  // a unit starts: its Q arrived with this tile
#pragma unroll
              for (int j = 0; j < KJ; ++j) qn[j] = qbuf[d][j];
            }
            compute_tile(cur, qn, kbuf[d], vbuf[d]);
          }
          if (cur.t + 1 == cur.n || i + d + 1 == n_tiles) flush(cur);
          cur.advance(pref, a.B, Hkv);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_tile(ld, qbuf[d], kbuf[d], vbuf[d], nt, false);
        advance_load();
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // One workgroup per unit (small batches) streams with ordinary loads: the
  // ring's repeats of the wave's last tile then hit L2 rather than HBM, and
  // the merge's registers wait for them.
  if (!UNIT && n_tiles >= (FUSED ? kFusedNtMin : kStreamNtMin)) stream(std::true_type{});
  else stream(std::false_type{});
}

template <typename T, int D, bool PAGE16, bool CONTIG, bool FUSED, bool GPREF, bool UNIT = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(TSA_DECODE_WAVES_PER_EU)))
void paged_decode_stream(DecodeArgs a, const int32_t* __restrict__ bt, const int32_t* __restrict__ sl,
                         float* __restrict__ part) {
  extern __shared__ int lds_i[];
  decode_stream_body<T, D, PAGE16, CONTIG, FUSED, GPREF, UNIT>(a, bt, sl, part, lds_i);
  if constexpr (UNIT) {
    unit_barrier();
    unit_merge<T, FUSED>(a, lds_i);
  }
}

// The exclusive tile prefix over the sequences (pref_out[0..B], pref_out[B]
// = total) for batches whose per-wave LDS copies would not fit: one
// workgroup, thread t summing a contiguous run of ceil(B / 1024) sequences,
// a scan of the 1024 run totals in LDS, then each run written out.
constexpr int kPrefixThreads = 1024;
__global__ __launch_bounds__(kPrefixThreads) void decode_tile_prefix(DecodeArgs a) {
  __shared__ int tot[kPrefixThreads];
  const int t = threadIdx.x;
  const int per = (a.B + kPrefixThreads - 1) / kPrefixThreads;
  const int s0 = min(a.B, t * per), s1 = min(a.B, s0 + per);
  int local = 0;
  for (int s = s0; s < s1; ++s) local += tiles_of(a, s);
  tot[t] = local;
  __syncthreads();
  for (int off = 1; off < kPrefixThreads; off <<= 1) {  // inclusive Hillis-Steele scan
    const int add = t >= off ? tot[t - off] : 0;
    __syncthreads();
    tot[t] += add;
    __syncthreads();
  }
  int run = tot[t] - local;
  for (int s = s0; s < s1; ++s) {
    a.pref_out[s] = run;
    run += tiles_of(a, s);
  }
  if (t == kPrefixThreads - 1) a.pref_out[a.B] = tot[t];
}

// out[s, kvh * G + hd] = sum_v 2^(m_v - M) acc_v / sum_v 2^(m_v - M) l_v over
// the wave workers v whose tiles cover unit (s, kvh); an empty sequence gives
// 0/0 = NaN, as the reference's does. One workgroup per unit, one thread per
// (head, dim) output (head_dim * G <= 2048 outputs over 256 threads). The
// contributors are combined in order with an online log-sum-exp, in batches
// whose loads are all issued before any is used, so a unit costs a few
// memory round trips however many waves covered it. A batch past the last
// contributor repeats its loads and weighs them by exactly 0 (scale 2^0 on
// the sum, 2^-inf on the repeat), so the batch size leaves the result
// unchanged. Batches of 4 suit the usual 2 to 5 contributors (batches of 8
// measured 0.8 us slower per Qwen3-8B batch-64 call); a unit of more
// contributors takes batches of 16.
template <typename T, int kOut>  // kOut: outputs per thread, G * head_dim / 256 rounded up
__global__ __launch_bounds__(256) void paged_decode_stream_merge(DecodeArgs a) {
  const int u = blockIdx.x, tid = threadIdx.x;
  const int Hkv = a.Hkv, G = a.G, D = a.D;
  const int s = u / Hkv, kvh = u - s * Hkv;
  const int p0 = a.pref_out[s], n = a.pref_out[s + 1] - p0;
  const int64_t total = static_cast<int64_t>(Hkv) * a.pref_out[a.B];
  T* orow = static_cast<T*>(a.out) + s * a.o_ss + (kvh * G) * a.o_sh;
  const int nout = G * D;
  if (n == 0) {
    for (int idx = tid; idx < nout; idx += 256)
      orow[(idx / D) * a.o_sh + (idx % D) * a.o_sd] = from_float<T>(NAN);
    return;
  }
  const int64_t share = (total + a.NW - 1) / a.NW;
  const int64_t P = static_cast<int64_t>(Hkv) * p0 + static_cast<int64_t>(kvh) * n;
  const int v0 = static_cast<int>(P / share), v1 = static_cast<int>((P + n - 1) / share);
  const int64_t slot_floats = static_cast<int64_t>(G) * (D + 2);
  const float* base = a.part + static_cast<int64_t>(u) * slot_floats;  // slot u + v = base + v * slot_floats
  int hd[kOut];
  float M[kOut], den[kOut], o[kOut];
#pragma unroll
  for (int i = 0; i < kOut; ++i) {
    const int idx = min(tid + 256 * i, nout - 1);  // spare threads repeat the last output
    hd[i] = idx / D;
    M[i] = kNegInf;
    den[i] = 0.f;
    o[i] = 0.f;
  }
  auto combine = [&](auto batch) {
    constexpr int kBatch = decltype(batch)::value;  // contributors per batch
    for (int v = v0; v <= v1; v += kBatch) {
      float mb[kBatch][kOut], lb[kBatch][kOut], ab[kBatch][kOut];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const float* sl = base + static_cast<int64_t>(min(v + k, v1)) * slot_floats;
#pragma unroll
        for (int i = 0; i < kOut; ++i) {
          const int idx = min(tid + 256 * i, nout - 1);
          mb[k][i] = v + k <= v1 ? sl[G * D + hd[i]] : kNegInf;
          lb[k][i] = sl[G * D + G + hd[i]];
          ab[k][i] = sl[idx];
        }
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
#pragma unroll
        for (int i = 0; i < kOut; ++i) {
          const float mn = fmaxf(M[i], mb[k][i]);
          if (mn == kNegInf) continue;
          const float c_old = fast_exp2(M[i] - mn), c_new = fast_exp2(mb[k][i] - mn);
          o[i] = o[i] * c_old + ab[k][i] * c_new;
          den[i] = den[i] * c_old + lb[k][i] * c_new;
          M[i] = mn;
        }
    }
  };
  // Many contributors (small batches: a wave per tile or two) in batches of
  // 16, so a unit of up to 16 one-tile partials costs one round trip.
  if constexpr (kOut <= 2) {
    if (v1 - v0 >= 4) combine(std::integral_constant<int, 16>{});
    else combine(std::integral_constant<int, 4>{});
  } else {
    combine(std::integral_constant<int, 4>{});
  }
#pragma unroll
  for (int i = 0; i < kOut; ++i) {
    const int idx = tid + 256 * i;
    if (idx < nout) orow[hd[i] * a.o_sh + (idx % D) * a.o_sd] = from_float<T>(o[i] / den[i]);
  }
}

// Generic path: one wave per (sequence, q-head), fp32 VALU math, any strides,
// page size and head_dim <= 512. Lane j scores token base + j of a 64-token
// chunk; the chunk's weights then stream V with lanes over dims.
template <typename T>
__global__ __launch_bounds__(64) void paged_decode_generic(DecodeArgs a) {
  const int h = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
  const int kvh = h / a.G;
  const int D = a.D;
  const int64_t L = clamp_len(a, s);
  const T* qrow = static_cast<const T*>(a.q) + s * a.q_ss + h * a.q_sh;
  const T* kbase = static_cast<const T*>(a.kc) + kvh * a.kc_h;
  const T* vbase = static_cast<const T*>(a.vc) + kvh * a.vc_h;
  const int32_t* bt_row = a.bt + s * a.bt_s0;
  constexpr int kMaxPerLane = 8;  // D <= 512
  float acc[kMaxPerLane];
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) acc[i] = 0.f;
  float m = kNegInf, l = 0.f;
  for (int64_t base = 0; base < L; base += 64) {
    const int64_t tok = base + lane;
    float sc = kNegInf;
    int64_t phys = -1, slot = 0;
    if (tok < L) {
      const int64_t lb = tok / a.BS;
      phys = bt_row[lb * a.bt_s1];
      slot = tok - lb * a.BS;
      if (phys >= 0 && phys < a.NB) {
        float dot = 0.f;
        const T* kr = kbase + phys * a.kc_b + slot * a.kc_s;
        for (int d = 0; d < D; ++d) dot += to_float(qrow[d * a.q_sd]) * to_float(kr[d * a.kc_d]);
        sc = dot * a.scale_log2;
      }
    }
    float cmax = sc;
    for (int off = 32; off >= 1; off >>= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, off, 64));
    const float m_new = fmaxf(m, cmax);
    const float alpha = m_new == kNegInf ? 1.f : fast_exp2(m - m_new);
    const float p = m_new == kNegInf ? 0.f : fast_exp2(sc - m_new);
    float psum = p;
    for (int off = 32; off >= 1; off >>= 1) psum += __shfl_xor(psum, off, 64);
    l = l * alpha + psum;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) acc[i] *= alpha;
    const int n = static_cast<int>(L - base < 64 ? L - base : 64);
    for (int j = 0; j < n; ++j) {
      const float pj = __shfl(p, j, 64);
      const int64_t ph = __shfl(phys, j, 64);
      const int64_t sl = __shfl(slot, j, 64);
      if (ph < 0 || ph >= a.NB) continue;
      const T* vr = vbase + ph * a.vc_b + sl * a.vc_s;
#pragma unroll
      for (int i = 0; i < kMaxPerLane; ++i) {
        const int d = lane + 64 * i;
        if (d < D) acc[i] += pj * to_float(vr[d * a.vc_d]);
      }
    }
    m = m_new;
  }
  T* orow = static_cast<T*>(a.out) + s * a.o_ss + h * a.o_sh;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int d = lane + 64 * i;
    if (d < D) orow[d * a.o_sd] = from_float<T>(acc[i] / l);
  }
}

static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Workgroups of the stream kernel: TSA_DECODE_WG_PER_CU per CU (one by
// default: one 4-wave workgroup per CU streams as fast as two, and with one
// per CU no workgroup runs ahead of another on its CU), all resident at once.
static int default_workgroups() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return TSA_DECODE_WG_PER_CU * cus;
}

struct DecodePlan {
  int W;
  bool unit;
  size_t part_bytes, pref_bytes, total;
};

// Workspace: one partial slot per (unit, wave worker) pair that can occur --
// units * 1 + workers, since slot = unit + worker -- and the tile prefix.
// With no grid asked for, a batch whose block tables hold few tiles (at
// most 8 per workgroup of the default grid, Hkv * B * ceil(max_blocks *
// block_size / 16) -- a bound the host knows without reading seq_lens)
// takes a grid of about two tiles per wave worker, but at least kMinAutoWG
// workgroups: fewer workers leave fewer partials per unit for the merge
// (Qwen3-0.6B batch of 4, 1024-tile tables: 11.5 us replayed at 128
// workgroups against 12.6 at 256; a 56-tile batch 10.7 us at any grid).
constexpr int kMinAutoWG = 64;
// With no grid asked for, a batch of at most kUnitMaxUnits (sequence, kv
// head) units whose block tables hold at most kUnitMaxTiles tiles per unit
// takes one workgroup per unit instead: its four waves split the unit's
// tiles, merge in LDS and write the output, so the call is one launch with
// no merge launch after it. Its waves compute their tiles one after
// another (about 0.7 us of computation per tile, measured), so it pays only
// while the units are few and short: the Qwen3-0.6B batch of 4 (32 units,
// 32-tile tables) went from 11.7 to 10.3-10.5 us replayed.
constexpr int64_t kUnitMaxUnits = 64;
constexpr int64_t kUnitMaxTiles = 32;
static_assert(kUnitMaxTiles <= 64, "a unit's block-table row (16-token or larger pages) fits one wave's lanes");
static DecodePlan make_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_blocks, int64_t BS,
                            int32_t num_workgroups) {
  DecodePlan p{};
  p.W = num_workgroups > 0 ? num_workgroups : default_workgroups();
  constexpr int64_t k31 = int64_t(1) << 31;
  if (num_workgroups == 0 && max_blocks > 0 && BS > 0 && max_blocks < k31 && BS < k31 && max_blocks * BS < k31 &&
      B < k31 && Hkv < k31 && B * Hkv < k31) {
    const int64_t unit_tiles = (max_blocks * BS + 15) / 16;
    const int64_t cap_tiles = Hkv * B * unit_tiles;
    const int64_t want = (cap_tiles + 2 * kWaves - 1) / (2 * kWaves);
    if (want < p.W) p.W = static_cast<int>(want < kMinAutoWG ? kMinAutoWG : want);
    if (B > 0 && B * Hkv <= kUnitMaxUnits && unit_tiles <= kUnitMaxTiles) {
      p.unit = true;
      p.W = static_cast<int>(B * Hkv);
    }
  }
  const int64_t G = Hq / Hkv;
  // (one workgroup per unit keeps its partials in LDS: no slots)
  const int64_t slots = p.unit ? 0 : B * Hkv + static_cast<int64_t>(kWaves) * p.W;
  p.part_bytes = align256(static_cast<size_t>(slots) * G * (D + 2) * sizeof(float));
  p.pref_bytes = align256(static_cast<size_t>(B + 1) * sizeof(int32_t));
  p.total = p.part_bytes + p.pref_bytes;
  return p;
}

// The merge of the stream kernel's partials (after it, on the same stream).
template <typename T>
static int launch_merge(const DecodeArgs& a, hipStream_t stream) {
  const dim3 mgrid(a.B * a.Hkv);
  const int outs = (a.G * a.D + 255) / 256;
  if (outs <= 1) paged_decode_stream_merge<T, 1><<<mgrid, dim3(256), 0, stream>>>(a);
  else if (outs <= 2) paged_decode_stream_merge<T, 2><<<mgrid, dim3(256), 0, stream>>>(a);
  else if (outs <= 4) paged_decode_stream_merge<T, 4><<<mgrid, dim3(256), 0, stream>>>(a);
  else paged_decode_stream_merge<T, 8><<<mgrid, dim3(256), 0, stream>>>(a);
  return check_launch("tsa_paged_decode");
}

// The stream kernel keeps kWaves copies of the tile prefix (B + 1 ints
// each) in LDS up to this batch; larger batches read one copy from the
// workspace (decode_tile_prefix).
static bool prefix_in_lds(int64_t B) { return static_cast<int64_t>(kWaves) * (B + 1) * 4 <= 64 * 1024; }

// LDS bytes of the fused stream kernel: kWaves tile prefixes, then the
// per-wave fused areas at the next 16-byte boundary.
static size_t fused_lds_bytes(int64_t B) {
  return ((static_cast<size_t>(kWaves) * (B + 1) * 4 + 15) & ~size_t(15)) +
         static_cast<size_t>(kWaves) * kFusedWaveBytes;
}

template <typename T>
static int launch_decode(DecodeArgs& a, bool mfma, hipStream_t stream, bool fused = false) {
  if (a.B == 0 || a.Hq == 0) return TSA_OK;
  if (!mfma) {
    paged_decode_generic<T><<<dim3(a.Hq, a.B), dim3(64), 0, stream>>>(a);
    return check_launch("tsa_paged_decode");
  }
  if constexpr (sizeof(T) == 2) {
    const bool gpref = !prefix_in_lds(a.B);
    const size_t lds = gpref ? 0 : static_cast<size_t>(kWaves) * (a.B + 1) * sizeof(int);
    const bool page16 = a.BS % 16 == 0;
    const bool contig = a.kc_s == a.D && a.vc_s == a.D;
    const dim3 grid(a.W);
    if (a.unit) {  // one workgroup per unit (the plan keeps such batches' prefixes in LDS), no merge launch
      if (fused) {
        paged_decode_stream<T, 128, true, true, true, false, true><<<grid, dim3(kThreads), fused_lds_bytes(a.B),
                                                                    stream>>>(a, a.bt, a.seq_lens, a.part);
        return check_launch("tsa_paged_decode");
      }
      const size_t lds_u = prefix_lds_bytes16(a.B) + static_cast<size_t>(kWaves) * unit_slot_floats(a.G, a.D) * 4;
#define TSA_UNIT_LAUNCH(DD, P16, CT)                                                                       \
  paged_decode_stream<T, DD, P16, CT, false, false, true><<<grid, dim3(kThreads), lds_u, stream>>>(a, a.bt, \
                                                                                             a.seq_lens, a.part)
      if (a.D == 128) {
        if (page16 && contig) TSA_UNIT_LAUNCH(128, true, true);
        else if (page16) TSA_UNIT_LAUNCH(128, true, false);
        else TSA_UNIT_LAUNCH(128, false, false);
      } else {
        if (page16 && contig) TSA_UNIT_LAUNCH(64, true, true);
        else if (page16) TSA_UNIT_LAUNCH(64, true, false);
        else TSA_UNIT_LAUNCH(64, false, false);
      }
#undef TSA_UNIT_LAUNCH
      return check_launch("tsa_paged_decode");
    }
    if (gpref) {
      decode_tile_prefix<<<dim3(1), dim3(kPrefixThreads), 0, stream>>>(a);
      if (int rc = check_launch("tsa_paged_decode")) return rc;
    }
#define TSA_DECODE_LAUNCH(DD, P16, CT)                                                                              \
  do {                                                                                                              \
    if (gpref)                                                                                                      \
      paged_decode_stream<T, DD, P16, CT, false, true><<<grid, dim3(kThreads), 0, stream>>>(a, a.bt, a.seq_lens,  \
                                                                                              a.part);              \
    else                                                                                                            \
      paged_decode_stream<T, DD, P16, CT, false, false><<<grid, dim3(kThreads), lds, stream>>>(a, a.bt, a.seq_lens, \
                                                                                                 a.part);           \
  } while (0)
    if (fused) {  // checked by the caller: head_dim 128, 16-token pages, contiguous rows, prefixes in LDS
      const size_t lds_f = fused_lds_bytes(a.B);
      paged_decode_stream<T, 128, true, true, true, false><<<grid, dim3(kThreads), lds_f, stream>>>(
          a, a.bt, a.seq_lens, a.part);
    } else if (a.D == 128) {
      if (page16 && contig) TSA_DECODE_LAUNCH(128, true, true);
      else if (page16) TSA_DECODE_LAUNCH(128, true, false);
      else TSA_DECODE_LAUNCH(128, false, false);
    } else {
      if (page16 && contig) TSA_DECODE_LAUNCH(64, true, true);
      else if (page16) TSA_DECODE_LAUNCH(64, true, false);
      else TSA_DECODE_LAUNCH(64, false, false);
    }
#undef TSA_DECODE_LAUNCH
    if (int rc = check_launch("tsa_paged_decode")) return rc;
    return launch_merge<T>(a, stream);
  }
  return check_launch("tsa_paged_decode");
}

}  // namespace tsa

using namespace tsa;

extern "C" size_t tsa_paged_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads,
                                                   int64_t head_dim, int64_t max_blocks_per_seq, int64_t block_size,
                                                   int32_t num_workgroups) {
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || num_heads % num_kv_heads) return 0;
  return make_plan(num_seqs, num_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size, num_workgroups).total;
}

namespace tsa {
// Checks shared by the decode entry points; fills a (and mfma: whether the
// stream kernel serves the call, plan: its grid and workspace layout). No
// device work and no workspace yet.
static int check_decode(const tsa_view* out, const tsa_view* query, const tsa_view* k_cache, const tsa_view* v_cache,
                        const tsa_view* block_tables, const tsa_view* seq_lens, double softmax_scale,
                        int32_t num_workgroups, DecodeArgs& a, bool& mfma, DecodePlan& plan) {
  TSA_REQUIRE(view_ok(query, 3), "query must be a 3D tensor (num_seqs, num_heads, head_dim)");
  TSA_REQUIRE(view_ok(out, 3), "out must be a 3D tensor shaped like query");
  TSA_REQUIRE(view_ok(k_cache, 4) && view_ok(v_cache, 4),
              "k_cache and v_cache must be 4D tensors (num_blocks, num_kv_heads, block_size, head_dim)");
  TSA_REQUIRE(view_ok(block_tables, 2) && block_tables->dtype == TSA_I32,
              "block_tables must be a 2D int32 tensor (num_seqs, max_num_blocks_per_seq)");
  TSA_REQUIRE(view_ok(seq_lens, 1) && seq_lens->dtype == TSA_I32, "seq_lens must be a 1D int32 tensor");
  const int dt = query->dtype;
  TSA_REQUIRE(is_float_dtype(dt) && out->dtype == dt && k_cache->dtype == dt && v_cache->dtype == dt,
              "query, out, k_cache and v_cache must share one floating dtype");
  for (int d = 0; d < 3; ++d) TSA_REQUIRE(out->size[d] == query->size[d], "out must have query's shape");
  for (int d = 0; d < 4; ++d) TSA_REQUIRE(k_cache->size[d] == v_cache->size[d], "k_cache and v_cache must match");
  const int64_t B = query->size[0], Hq = query->size[1], D = query->size[2];
  const int64_t NB = k_cache->size[0], Hkv = k_cache->size[1], BS = k_cache->size[2];
  TSA_REQUIRE(k_cache->size[3] == D, "cache head_dim %lld != query head_dim %lld", (long long)k_cache->size[3],
              (long long)D);
  TSA_REQUIRE(Hkv > 0 && Hq % Hkv == 0, "num_heads (%lld) must be a multiple of num_kv_heads (%lld)",
              (long long)Hq, (long long)Hkv);
  TSA_REQUIRE(BS > 0, "block_size must be positive");
  TSA_REQUIRE(block_tables->size[0] == B && seq_lens->size[0] == B,
              "block_tables and seq_lens must have num_seqs (%lld) rows", (long long)B);
  TSA_REQUIRE(B < 65536 && Hq < 65536, "num_seqs and num_heads must be below 65536");
  TSA_REQUIRE(block_tables->size[1] * BS < (int64_t(1) << 31) / 16, "block table too long");
  TSA_REQUIRE(B * ((block_tables->size[1] * BS + 15) / 16) < (int64_t(1) << 31),
              "num_seqs x block-table capacity exceeds 2^31 16-token tiles");
  TSA_UNSUPPORTED(D <= 512, "head_dim %lld > 512 is not implemented", (long long)D);
  TSA_REQUIRE(num_workgroups >= 0, "num_workgroups must be non-negative");

  a = DecodeArgs{};
  a.out = out->data; a.q = query->data; a.kc = k_cache->data; a.vc = v_cache->data;
  a.bt = static_cast<const int32_t*>(block_tables->data);
  a.seq_lens = static_cast<const int32_t*>(seq_lens->data);
  a.o_ss = out->stride[0]; a.o_sh = out->stride[1]; a.o_sd = out->stride[2];
  a.q_ss = query->stride[0]; a.q_sh = query->stride[1]; a.q_sd = query->stride[2];
  a.kc_b = k_cache->stride[0]; a.kc_h = k_cache->stride[1]; a.kc_s = k_cache->stride[2]; a.kc_d = k_cache->stride[3];
  a.vc_b = v_cache->stride[0]; a.vc_h = v_cache->stride[1]; a.vc_s = v_cache->stride[2]; a.vc_d = v_cache->stride[3];
  a.bt_s0 = block_tables->stride[0]; a.bt_s1 = block_tables->stride[1]; a.sl_s = seq_lens->stride[0];
  a.NB = NB;
  a.B = static_cast<int32_t>(B); a.Hq = static_cast<int32_t>(Hq); a.Hkv = static_cast<int32_t>(Hkv);
  a.G = static_cast<int32_t>(Hq / Hkv); a.BS = static_cast<int32_t>(BS);
  a.max_blocks = static_cast<int32_t>(block_tables->size[1]); a.D = static_cast<int32_t>(D);
  a.scale_log2 = static_cast<float>(softmax_scale * 1.4426950408889634);

  mfma = (dt == TSA_BF16 || dt == TSA_F16) && (D == 64 || D == 128) && a.G <= 16 && rows_vec16(query) &&
         rows_vec16(k_cache) && rows_vec16(v_cache) && out->stride[2] == 1;
  plan = DecodePlan{};
  if (mfma) {
    plan = make_plan(B, Hq, Hkv, D, block_tables->size[1], BS, num_workgroups);
    a.W = plan.W;
    a.NW = kWaves * plan.W;
    a.unit = plan.unit ? 1 : 0;
  }
  return TSA_OK;
}

// The stream kernel's partials and tile prefix in the workspace (only the
// stream path takes one).
static int bind_workspace(DecodeArgs& a, bool mfma, const DecodePlan& plan, void* workspace, size_t workspace_bytes,
                          const char* workspace_name) {
  if (!mfma) return TSA_OK;
  TSA_REQUIRE(workspace != nullptr && workspace_bytes >= plan.total, "%s of %zu bytes is too small: %zu needed",
              workspace_name, workspace_bytes, plan.total);
  TSA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "%s must be 256-byte aligned", workspace_name);
  char* ws = static_cast<char*>(workspace);
  a.part = reinterpret_cast<float*>(ws);
  a.pref_out = reinterpret_cast<int32_t*>(ws + plan.part_bytes);
  return TSA_OK;
}

// check_decode, then the caller's workspace.
static int prepare_decode(const tsa_view* out, const tsa_view* query, const tsa_view* k_cache, const tsa_view* v_cache,
                          const tsa_view* block_tables, const tsa_view* seq_lens, double softmax_scale, void* workspace,
                          size_t workspace_bytes, int32_t num_workgroups, DecodeArgs& a, bool& mfma) {
  DecodePlan plan;
  if (int rc = check_decode(out, query, k_cache, v_cache, block_tables, seq_lens, softmax_scale, num_workgroups, a,
                            mfma, plan))
    return rc;
  return bind_workspace(a, mfma, plan, workspace, workspace_bytes, "workspace");
}
}  // namespace tsa

extern "C" int tsa_paged_decode(const tsa_view* out, const tsa_view* query, const tsa_view* k_cache,
                                const tsa_view* v_cache, const tsa_view* block_tables, const tsa_view* seq_lens,
                                double softmax_scale, void* workspace, size_t workspace_bytes,
                                int32_t num_workgroups, void* stream) {
  DecodeArgs a;
  bool mfma = false;
  if (int rc = prepare_decode(out, query, k_cache, v_cache, block_tables, seq_lens, softmax_scale, workspace,
                              workspace_bytes, num_workgroups, a, mfma))
    return rc;
  const int dt = query->dtype;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dt) {
    case TSA_BF16: return launch_decode<bf16_t>(a, mfma, st);
    case TSA_F16: return launch_decode<f16_t>(a, mfma, st);
    case TSA_F32: return launch_decode<float>(a, false, st);
  }
  set_error("unsupported dtype");
  return TSA_ERR_UNSUPPORTED;
}

namespace tsa {
// Checks of the fused decode step: prepare_decode's, then the new token's
// rows, the norm weights and the cos/sin rows, and the shapes the fused
// kernel covers (else TSA_ERR_UNSUPPORTED: such calls go through
// tsa_qk_norm_rope_store + tsa_paged_decode).
static int prepare_decode_step(const tsa_view* out, const tsa_view* query, const tsa_view* k_new,
                               const tsa_view* v_new, const tsa_view* q_weight, const tsa_view* k_weight,
                               const tsa_view* cos, const tsa_view* sin, double eps, const tsa_view* k_cache,
                               const tsa_view* v_cache, const tsa_view* block_tables, const tsa_view* seq_lens,
                               double softmax_scale, void* workspace, size_t workspace_bytes, int32_t num_workgroups,
                               DecodeArgs& a) {
  bool mfma = false;
  if (int rc = prepare_decode(out, query, k_cache, v_cache, block_tables, seq_lens, softmax_scale, workspace,
                              workspace_bytes, num_workgroups, a, mfma))
    return rc;
  const int dt = query->dtype;
  const int64_t B = a.B, Hkv = a.Hkv, D = a.D;
  TSA_REQUIRE(view_ok(k_new, 3) && view_ok(v_new, 3) && k_new->dtype == dt && v_new->dtype == dt,
              "k and v must be 3D tensors (num_seqs, num_kv_heads, head_dim) of query's dtype");
  TSA_REQUIRE(k_new->size[0] == B && k_new->size[1] == Hkv && k_new->size[2] == D && v_new->size[0] == B &&
                  v_new->size[1] == Hkv && v_new->size[2] == D,
              "k and v must be (num_seqs, num_kv_heads, head_dim)");
  TSA_REQUIRE(view_ok(q_weight, 1) && view_ok(k_weight, 1) && q_weight->size[0] == D && k_weight->size[0] == D &&
                  q_weight->dtype == dt && k_weight->dtype == dt,
              "q_weight and k_weight must be (head_dim,) of query's dtype");
  TSA_REQUIRE(view_ok(cos, 2) && view_ok(sin, 2) && cos->size[0] == B && cos->size[1] == D && sin->size[0] == B &&
                  sin->size[1] == D && cos->dtype == dt && sin->dtype == dt,
              "cos and sin must be (num_seqs, head_dim) of query's dtype");
  TSA_UNSUPPORTED(mfma && D == 128 && a.BS % 16 == 0 && a.kc_s == D && a.vc_s == D && a.G <= 8 &&
                      rows_vec16(k_new) && rows_vec16(v_new) && rows_vec16(q_weight) && rows_vec16(k_weight) &&
                      rows_vec16(cos) && rows_vec16(sin) && fused_lds_bytes(B) <= 64 * 1024,
                  "the fused decode step needs a 16-bit dtype, head_dim 128, 16-token-multiple pages, contiguous "
                  "cache rows, at most 8 q-heads per kv head and unit-stride 16-byte-aligned rows");
  a.kn = k_new->data; a.vn = v_new->data; a.qw = q_weight->data; a.kw = k_weight->data;
  a.cos = cos->data; a.sin = sin->data;
  a.kn_ss = k_new->stride[0]; a.kn_sh = k_new->stride[1];
  a.vn_ss = v_new->stride[0]; a.vn_sh = v_new->stride[1];
  a.cs_ss = cos->stride[0]; a.sn_ss = sin->stride[0];
  a.eps = static_cast<float>(eps);
  a.kc_out = k_cache->data; a.vc_out = v_cache->data;
  return TSA_OK;
}
}  // namespace tsa

extern "C" int tsa_paged_decode_step(const tsa_view* out, const tsa_view* query, const tsa_view* k_new,
                                     const tsa_view* v_new, const tsa_view* q_weight, const tsa_view* k_weight,
                                     const tsa_view* cos, const tsa_view* sin, double eps, const tsa_view* k_cache,
                                     const tsa_view* v_cache, const tsa_view* block_tables, const tsa_view* seq_lens,
                                     double softmax_scale, void* workspace, size_t workspace_bytes,
                                     int32_t num_workgroups, void* stream) {
  DecodeArgs a;
  if (int rc = prepare_decode_step(out, query, k_new, v_new, q_weight, k_weight, cos, sin, eps, k_cache, v_cache,
                                   block_tables, seq_lens, softmax_scale, workspace, workspace_bytes, num_workgroups,
                                   a))
    return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (query->dtype == TSA_BF16) return launch_decode<bf16_t>(a, true, st, true);
  return launch_decode<f16_t>(a, true, st, true);
}

// ---------------------------------------------------------------------------
// tsa_mixed_attention: a continuous-batching step's two attention calls in
// one launch (plus the decode merge). The first W workgroups run the decode
// stream (decode_stream_body: paged attention of each decode sequence over
// its pages); the others run the LDS-staged GQA prefill (prefill_gqa_body)
// over the prefill batch. Both take 4-wave workgroups with at most 256
// registers per lane, and the kernel's 78 KB of LDS lets two workgroups share
// a CU, so with the default split (W = one decode workgroup per CU, one
// prefill workgroup per CU) every workgroup is resident at once and each CU
// runs one of each (a per-workgroup trace of CU ids and start/end times
// showed exactly that). Both read only (the caches and q/k/v); each writes
// its own output and the decode its workspace, so they need no ordering;
// every output is bit-identical to tsa_varlen_prefill followed by
// tsa_paged_decode.
namespace tsa {

constexpr int kMixedLds = gqa_smem_bytes<128, 4>();
// Automatic choice (prefill_workgroups == 0): one kernel only for prefill
// batches of at most kMixedAutoMaxTokens tokens beside a decode batch whose
// block tables span at most kMixedAutoMaxDecodeTokens tokens (batch x table
// width x page size, a bound the host knows without reading seq_lens).
// Sharing a CU, the two roles slow each other down -- the LDS-staged
// prefill's loads wait behind the decode's HBM stream -- so one launch pays
// only when both halves are small. Measured on Qwen3-4B heads, one kernel vs
// the two launches, both replayed from a captured graph:
//   4 decode (ctx 128-512) + 322 prefill tokens        23.1 vs 26.7 us
//   16 decode (ctx 256-2048) + 365 prefill tokens      30.3 vs 35.4 us
//   32 decode (ctx 256-4096) + 402 prefill tokens      67.5 vs 70.7 us
//   64 decode (ctx 256-4096) + 402 prefill tokens     118.9 vs 117.9 us
//   120 decode (ctx 256-8192) + 402 prefill tokens    350.3 vs 339.6 us
//   120 decode (ctx 256-8192) + 5760 prefill tokens   436.1 vs 402.0 us
constexpr int64_t kMixedAutoMaxTokens = 512;
constexpr int64_t kMixedAutoMaxDecodeTokens = 131072;
static_assert(kMixedLds >= 64 * 1024, "the mixed kernel's LDS also holds the decode tile prefixes (at most 64 KB)");
static_assert(kMixedLds >= kWaves * (kUnitMaxUnits + 1) * 4 + 16 + kWaves * 16 * (128 + 2) * 4,
              "the mixed kernel's LDS holds a unit-mode decode workgroup's prefixes and wave partials");
static_assert(kThreads == 64 * 4 && TSA_DECODE_WAVES_PER_EU == 2,
              "the decode and prefill roles share a 4-wave workgroup compiled for two waves per SIMD");

template <typename T>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void mixed_attention_kernel(
    DecodeArgs d, const int32_t* __restrict__ bt, const int32_t* __restrict__ sl, float* __restrict__ part,
    PrefillArgs p, const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k) {
  __shared__ __align__(16) char lds_m[kMixedLds];
  if (static_cast<int>(blockIdx.x) < d.W) {
    if (d.unit) {  // one workgroup per decode unit, merged here (as tsa_paged_decode's plan takes it)
      decode_stream_body<T, 128, true, true, false, false, true>(d, bt, sl, part, reinterpret_cast<int*>(lds_m));
      unit_barrier();
      unit_merge<T, false>(d, reinterpret_cast<int*>(lds_m));
    } else {
      decode_stream_body<T, 128, true, true, false>(d, bt, sl, part, reinterpret_cast<int*>(lds_m));
    }
  } else {
    prefill_gqa_body<T, 128, 4>(p, cu_q, cu_k, lds_m, d.W);
  }
}

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}

}  // namespace tsa

extern "C" int tsa_mixed_attention(const tsa_view* prefill_out, const tsa_view* prefill_q, const tsa_view* prefill_k,
                                   const tsa_view* prefill_v, const tsa_view* cu_seqlens, int64_t max_seqlen,
                                   double prefill_scale, const tsa_view* out, const tsa_view* query,
                                   const tsa_view* k_cache, const tsa_view* v_cache, const tsa_view* block_tables,
                                   const tsa_view* seq_lens, double softmax_scale, void* workspace,
                                   size_t workspace_bytes, int32_t num_workgroups, int32_t prefill_workgroups,
                                   void* stream) {
  PrefillArgs pa;
  bool pmfma = false;
  if (int rc = prefill_prepare(prefill_out, prefill_q, prefill_k, prefill_v, cu_seqlens, cu_seqlens, max_seqlen,
                               max_seqlen, 1, prefill_scale, pa, pmfma))
    return rc;
  DecodeArgs a;
  bool dmfma = false;
  if (int rc = prepare_decode(out, query, k_cache, v_cache, block_tables, seq_lens, softmax_scale, workspace,
                              workspace_bytes, num_workgroups, a, dmfma))
    return rc;
  TSA_REQUIRE(prefill_workgroups >= 0, "prefill_workgroups must be non-negative");
  const int dt = query->dtype;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // One launch when the decode takes the head_dim-128, 16-token-page,
  // contiguous-row stream kernel, the prefill varlen_prefill_gqa<T, 128, 4>
  // in the same dtype, both halves have work, and the caller asks for it
  // (prefill_workgroups > 0) or both halves are small; else the two
  // launches.
  const bool small = pa.total_q <= kMixedAutoMaxTokens &&
                     int64_t{a.B} * a.max_blocks * a.BS <= kMixedAutoMaxDecodeTokens;
  const bool one = dmfma && a.D == 128 && a.BS % 16 == 0 && a.kc_s == a.D && a.vc_s == a.D && a.B > 0 &&
                   prefix_in_lds(a.B) &&
                   pa.nseq > 0 && pa.Hq > 0 && pa.total_q > 0 && prefill_q->dtype == dt &&
                   prefill_takes_gqa4(pa, pmfma) && (prefill_workgroups > 0 || small);
  if (!one) {
    if (int rc = prefill_launch(pa, pmfma, prefill_q->dtype, max_seqlen, st)) return rc;
    switch (dt) {
      case TSA_BF16: return launch_decode<bf16_t>(a, dmfma, st);
      case TSA_F16: return launch_decode<f16_t>(a, dmfma, st);
      case TSA_F32: return launch_decode<float>(a, false, st);
    }
    set_error("unsupported dtype");
    return TSA_ERR_UNSUPPORTED;
  }
  const int P = prefill_workgroups > 0 ? prefill_workgroups : device_cus();
  const dim3 grid(a.W + P);
  if (dt == TSA_BF16) {
    mixed_attention_kernel<bf16_t><<<grid, dim3(kThreads), 0, st>>>(a, a.bt, a.seq_lens, a.part, pa, pa.cu_q,
                                                                     pa.cu_k);
    if (int rc = check_launch("tsa_mixed_attention")) return rc;
    return a.unit ? TSA_OK : launch_merge<bf16_t>(a, st);
  }
  mixed_attention_kernel<f16_t><<<grid, dim3(kThreads), 0, st>>>(a, a.bt, a.seq_lens, a.part, pa, pa.cu_q, pa.cu_k);
  if (int rc = check_launch("tsa_mixed_attention")) return rc;
  return a.unit ? TSA_OK : launch_merge<f16_t>(a, st);
}

// ---------------------------------------------------------------------------
// tsa_paged_decode_noalloc: tsa_paged_decode for callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc). The same kernels take their partials and tile prefix from a
// file-scope device array instead of a caller workspace. Each GPU the
// library runs on holds its own copy of the array until the process ends;
// every call on a GPU shares it and leaves the last call's contents, which
// is harmless here -- every partial slot a merge reads is written by the
// stream launch of the same call, and the prefix too, so nothing needs
// clearing. Two calls that overlap on one GPU (on different streams, say)
// race on it; calls ordered on one stream do not.
namespace tsa {

constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;  // 16 MiB per GPU
// In host code this name is a host-side stand-in: kernels get the address
// from hipGetSymbolAddress (noalloc_scratch), never the name itself.
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
static std::atomic<void*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// This GPU's scratch address: looked up once per device, on the first call
// there, with that device current (each GPU holds its copy at its own
// address), then read from the per-device cache.
static int noalloc_scratch(hipStream_t stream, void** ptr) {
  int dev = 0;
  const hipError_t e0 = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e0 != hipSuccess) {
    set_error("tsa_paged_decode_noalloc: cannot find the stream's device: %s", hipGetErrorString(e0));
    return TSA_ERR_LAUNCH;
  }
  TSA_REQUIRE(dev >= 0 && dev < kMaxDevices, "tsa_paged_decode_noalloc: device %d beyond the %d supported", dev,
              kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      int cur = -1;
      hipError_t e = hipGetDevice(&cur);
      if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
      if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (cur >= 0 && cur != dev) {
        const hipError_t er = hipSetDevice(cur);
        if (e == hipSuccess) e = er;
      }
      if (e != hipSuccess || p == nullptr) {
        set_error("tsa_paged_decode_noalloc: hipGetSymbolAddress of the scratch array failed on device %d: %s", dev,
                  hipGetErrorString(e));
        return TSA_ERR_LAUNCH;
      }
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return TSA_OK;
}

}  // namespace tsa

extern "C" int tsa_paged_decode_noalloc(const tsa_view* out, const tsa_view* query, const tsa_view* k_cache,
                                        const tsa_view* v_cache, const tsa_view* block_tables,
                                        const tsa_view* seq_lens, double softmax_scale, int32_t num_workgroups,
                                        void* stream) {
  // Every argument check first, before any device work; the scratch limit
  // and the device's scratch address only where the stream kernel takes a
  // workspace (the generic kernel needs none).
  DecodeArgs a;
  bool mfma = false;
  DecodePlan plan;
  if (int rc = check_decode(out, query, k_cache, v_cache, block_tables, seq_lens, softmax_scale, num_workgroups, a,
                            mfma, plan))
    return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (mfma) {
    TSA_REQUIRE(plan.total <= kNoAllocScratchBytes,
                "tsa_paged_decode_noalloc: this call needs %zu bytes of scratch, beyond the %zu bytes the library "
                "holds per GPU; use tsa_paged_decode with a caller workspace",
                plan.total, kNoAllocScratchBytes);
    void* ws = nullptr;
    if (int rc = noalloc_scratch(st, &ws)) return rc;
    if (int rc = bind_workspace(a, mfma, plan, ws, kNoAllocScratchBytes, "the no-allocation scratch")) return rc;
  }
  switch (query->dtype) {
    case TSA_BF16: return launch_decode<bf16_t>(a, mfma, st);
    case TSA_F16: return launch_decode<f16_t>(a, mfma, st);
    case TSA_F32: return launch_decode<float>(a, false, st);
  }
  set_error("unsupported dtype");
  return TSA_ERR_UNSUPPORTED;
}
