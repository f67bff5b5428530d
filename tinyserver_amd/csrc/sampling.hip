// Batched token sampling for gfx950: tinyserver's sample_tokens
// (server/model/sampling.py:119-194), one workgroup per row, no sort of the
// row.
//
// The reference scales a row by its temperature, stably sorts it (x
// descending, index ascending), masks ranks >= top_k, softmaxes, drops the
// ranks whose preceding mass exceeds top_p, and picks the first rank whose
// cumulative mass reaches u * (kept mass). Each of those three decisions is
// the same question: which element, in rank order, is the first whose running
// weight (1 per element for top-k, its mass otherwise) reaches a target? The
// kernel answers it without sorting the row:
// * One pass histograms the candidates into 2048 buckets by
//   (hi - x) * scale, a function that never increases with x, so bucket order
//   is rank order; the scale spreads the candidates' value range over the
//   buckets, so a bucket holds a few hundred elements of a real logit row.
// * A scan over the buckets finds the one where the running weight reaches
//   the target. Only that bucket's elements are gathered into LDS and sorted
//   exactly (bitonic, on (x descending, index ascending)), and a prefix sum
//   over them finds the element.
// * A bucket too large for LDS is split again over its own value range (at
//   most 4 levels); one whose elements all hold the same x is resolved in
//   index order, which is the stable sort's order for ties.
// Masses are exp(x - max) in fp32, held as 2^-40 fixed point in 64-bit
// integers, so every sum is exact and order-free: the kernel is deterministic
// and its decisions differ from the reference's fp32 cumsum only where a
// target lies within fp32 rounding of a cumulative sum.
// The usual path builds one histogram (counts and masses of every element)
// and reads all three decisions from it, gathering only the buckets where a
// cut or the pick falls; a bucket too large for LDS sends the row to the
// per-decision path above.
// Greedy rows (temperature <= 0) take the first index of the row's maximum,
// which is the stable sort's rank 0, as the reference does.
//
// Top-k rows (top_k <= 512) and greedy rows of a 16-bit row of at most
// 155,648 logits first take a candidate pass: the row is read once into
// registers, a sample of it bounds its k-th largest value from below, and
// only the few elements above that bound are gathered, ranked and decided
// on. A row it cannot finish (too many candidates, NaN or inf) continues down
// the paths above.
#include <cmath>
#include <cstdlib>

#include "tsa_common.h"

namespace tsa {

constexpr int kSampThreads = 1024;
constexpr int kSampWaves = kSampThreads / 64;
constexpr int kBuckets = 2048;
constexpr int kCap = 8192;  // elements of one bucket sorted in LDS
constexpr int kPrefixMax = 1024;  // top ranks worth one gather + sort + scans instead of per-bucket gathers
constexpr int kMaxLevels = 4;
constexpr float kMassOne = 1099511627776.0f;  // 2^40: the row maximum's mass

struct SampleArgs {
  const void* logits;
  int64_t ls0, ls1;
  int64_t B, V;
  const float* temp; int64_t temp_s;
  const void* topk; int topk_dt; int64_t topk_s;
  const float* topp; int64_t topp_s;
  const float* unif; int64_t unif_s;
  int64_t* out; int64_t out_s;
  int cand;  // 1: top-k and greedy rows may take the register-resident candidate pass
  // Rows split over S workgroups (split_row; S = 0: none): per (row,
  // segment) the statistics record and the partial histogram, as the
  // exclusive prefix of its counts (plp) and its masses (pmass); with
  // bucket lists (pidx non-null) also its elements' indices, relative to
  // the segment's first element, in bucket order (segcap each).
  struct SplitStat* stat;
  struct SplitStat* mstat;  // per row: the merge of its S records (sample_split_hist, segment 0)
  uint32_t* plp;
  uint64_t* pmass;
  int S;
  uint16_t* pidx;
  int segcap;
};

// ---- Rows split over several workgroups. A histogram row (temperature >
// 0, not a candidate row) of 16-bit logits in 8-logit chunks has its two
// full passes -- the statistics, then the count and mass histogram -- run
// by S workgroups, each over a contiguous range of the row's chunks
// (sample_split_stats, sample_split_hist); sample_tokens_kernel then merges
// the S records and partial histograms instead of making those passes
// itself and decides as before. The statistics' tie rules (first index of
// the maximum, last of the minimum) and the exact fixed-point mass sums are
// order-free, so the merged values -- and the tokens -- are the one-
// workgroup path's.
constexpr int kSplitThreads = 256;
constexpr int kMaxSegments = 16;  // workgroups per split row, at most
// Elements of a segment whose bucket list sample_split_hist builds in LDS:
// 55 KB beside the 24 KB histogram, so two workgroups fit a CU's 160 KB.
constexpr int kSegListMax = 28160;
struct SplitStat {
  float mx, mn, fmn;
  int imx, imn, inan;
  int pad[2];
};

// f(w, ch) for chunks ch = first, first + step, ... < end of a row, in
// increasing order, kLoadBatch loads issued before any is used: a pass over
// a row is then bound by bandwidth rather than by one load's latency per
// chunk.
constexpr int kLoadBatch = 8;
template <typename F>
__device__ __forceinline__ void each_chunk(const u32x4* r4, int first, int end, int step, F f) {
  for (int base = first; base < end; base += kLoadBatch * step) {
    u32x4 w[kLoadBatch];
#pragma unroll
    for (int j = 0; j < kLoadBatch; ++j) {
      const int ch = base + j * step;
      w[j] = ch < end ? r4[ch] : u32x4{0, 0, 0, 0};
    }
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the first use
#pragma unroll
    for (int j = 0; j < kLoadBatch; ++j) {
      const int ch = base + j * step;
      if (ch < end) f(w[j], ch);
    }
  }
}

// Statistics of a thread's 8-logit chunks, visited in increasing order: the
// maximum and its first index (rank 0), the minimum and the last index of
// it (the last rank), the finite minimum and the first NaN. A strict >
// keeps the first index of a maximum and <= the last of a minimum.
struct ChunkStats {
  float mx, mn, fmn;
  int imx, imn, inan;
  __device__ __forceinline__ void init(int V) {
    mx = -INFINITY;
    mn = INFINITY;
    fmn = INFINITY;
    imx = V;
    imn = -1;
    inan = V;
  }
  template <typename T>
  __device__ __forceinline__ void add(const u32x4 w, int ch, int V) {
    float l[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      l[2 * e] = lo_f<T>(w[e]);
      l[2 * e + 1] = hi_f<T>(w[e]);
    }
    // cmax propagates NaN (v_maximum3_f32): a chunk holding a NaN never
    // passes cmax > mx, and records its first NaN instead.
    float cmax = l[0], cmin = l[0], cfin = l[0] != -INFINITY ? l[0] : INFINITY;
#pragma unroll
    for (int e = 1; e < 8; ++e) {
      cmax = __builtin_elementwise_maximum(cmax, l[e]);
      cmin = fminf(cmin, l[e]);
      cfin = fminf(cfin, l[e] != -INFINITY ? l[e] : INFINITY);
    }
    fmn = fminf(fmn, cfin);
    if (cmax != cmax && inan == V) {
      int first = 7;
#pragma unroll
      for (int e = 7; e >= 0; --e)
        if (l[e] != l[e]) first = e;
      inan = 8 * ch + first;
    }
    if (cmax > mx) {
      int first = 0;
#pragma unroll
      for (int e = 7; e >= 0; --e)
        if (l[e] == cmax) first = e;
      mx = cmax;
      imx = 8 * ch + first;
    }
    if (cmin <= mn) {
      int last = 7;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (l[e] == cmin) last = e;
      mn = cmin;
      imn = 8 * ch + last;
    }
  }
  // Combine with the statistics of other elements (in any order).
  __device__ __forceinline__ void merge(float omx, int oimx, float omn, int oimn, float ofm, int onan) {
    if (omx > mx || (omx == mx && oimx < imx)) {
      mx = omx;
      imx = oimx;
    }
    if (omn < mn || (omn == mn && oimn > imn)) {
      mn = omn;
      imn = oimn;
    }
    fmn = fminf(fmn, ofm);
    inan = min(inan, onan);
  }
  __device__ __forceinline__ void merge(const SplitStat& o) { merge(o.mx, o.imx, o.mn, o.imn, o.fmn, o.inan); }
  __device__ __forceinline__ void wave_reduce() {
    for (int o = 32; o > 0; o >>= 1)
      merge(__shfl_xor(mx, o, 64), __shfl_xor(imx, o, 64), __shfl_xor(mn, o, 64), __shfl_xor(imn, o, 64),
            __shfl_xor(fmn, o, 64), __shfl_xor(inan, o, 64));
  }
};

// One compare-exchange stage (K, J) of a bitonic sort of 64 keys held one
// per lane, ascending over the lanes when the network is done.
template <int K, int J>
__device__ __forceinline__ uint64_t bitonic_stage(uint64_t x, int lane) {
  const uint64_t y = xor_lane64<J>(x, lane);
  const bool keep_min = ((lane & J) == 0) == ((lane & K) == 0);
  return keep_min == (x < y) ? x : y;
}
template <int K>
__device__ __forceinline__ uint64_t bitonic_merge(uint64_t x, int lane) {
  if constexpr (K >= 64) x = bitonic_stage<K, 32>(x, lane);
  if constexpr (K >= 32) x = bitonic_stage<K, 16>(x, lane);
  if constexpr (K >= 16) x = bitonic_stage<K, 8>(x, lane);
  if constexpr (K >= 8) x = bitonic_stage<K, 4>(x, lane);
  if constexpr (K >= 4) x = bitonic_stage<K, 2>(x, lane);
  return bitonic_stage<K, 1>(x, lane);
}
__device__ __forceinline__ uint64_t wave_sort_u64(uint64_t x, int lane) {
  x = bitonic_merge<2>(x, lane);
  x = bitonic_merge<4>(x, lane);
  x = bitonic_merge<8>(x, lane);
  x = bitonic_merge<16>(x, lane);
  x = bitonic_merge<32>(x, lane);
  return bitonic_merge<64>(x, lane);
}

__device__ __forceinline__ int64_t load_int(const void* p, int dt, int64_t i) {
  return dt == TSA_I64 ? static_cast<const int64_t*>(p)[i] : static_cast<int64_t>(static_cast<const int32_t*>(p)[i]);
}

// Rank key: ascending order of (~orderable(x) << 32 | index) is the stable
// descending sort's order. -0 is folded into +0 first (they compare equal).
__device__ __forceinline__ uint64_t rank_key(float x, int64_t i) {
  uint32_t u = __builtin_bit_cast(uint32_t, x + 0.0f);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (static_cast<uint64_t>(~u) << 32) | static_cast<uint32_t>(i);
}

// The value a rank key was made from (-0 comes back as +0).
__device__ __forceinline__ float key_of_rank(uint64_t rk) {
  const uint32_t o = ~static_cast<uint32_t>(rk >> 32);
  return __builtin_bit_cast(float, (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// 2^40 exp2((kv - kmax) * kc) on v_exp_f32, truncated to an integer in two
// 32-bit halves (exact: the value has at most 24 significant bits). Both
// paths weigh keys with this one function, so their sums agree bit for bit.
__device__ __forceinline__ uint64_t mass_of(float kv, float kmax, float kc) {
  const float v = fast_exp2((kv - kmax) * kc) * kMassOne;
  const uint32_t hi = static_cast<uint32_t>(v * 2.3283064365386963e-10f);  // v / 2^32
  const uint32_t lo = static_cast<uint32_t>(v - static_cast<float>(hi) * 4294967296.0f);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// ---- The candidate pass (top-k and greedy rows of 16-bit logits).
constexpr int kRegChunks = 19;  // 8-logit chunks per thread: the row stays in registers
constexpr int64_t kRegMaxV = int64_t{kSampThreads} * kRegChunks * 8;  // 155,648 logits
constexpr int64_t kFastK = 512;                                        // the largest top_k it takes
constexpr int kWaveStage = 64;    // chunks holding a candidate one wave may stage
constexpr int kCandOff = 4608;    // the candidates: keys[kCandOff, kCap)
constexpr int kRunStride = 68;    // a sorted run of 64 keys with a slot after each 16 (sort_keys)
static_assert(kRunStride * (kSampWaves - 1) + kRunStride <= kCandOff, "sorted runs stay below the candidates");
constexpr int kGatherCap = kCap - kCandOff;
constexpr int kSelBins = 4096;        // 12-bit key prefixes

// The rows the candidate pass takes: greedy rows (rank 0) and rows whose
// top-k cut falls inside the row, with top_k <= kFastK.
__device__ __forceinline__ bool candidate_row(const SampleArgs& a, float temp, int64_t k) {
  return temp <= 0.f || (k > 0 && k <= kFastK && k < a.V);
}

// The rows whose statistics and histogram sample_split_stats and
// sample_split_hist make (a.S > 1: the launch split rows).
__device__ __forceinline__ bool split_row(const SampleArgs& a, float temp, int64_t k) {
  return a.S > 1 && temp > 0.f && !(a.cand && a.V <= kRegMaxV && candidate_row(a, temp, k));
}

// The chunks of segment seg of a split row: [seg * per, min((seg + 1) *
// per, V / 8)), per = ceil(V / 8 / S).
__device__ __forceinline__ void split_range(const SampleArgs& a, int seg, int& c0, int& c1) {
  const int n8 = static_cast<int>(a.V >> 3), per = (n8 + a.S - 1) / a.S;
  c0 = min(n8, seg * per);
  c1 = min(n8, c0 + per);
}

// Two 16-bit floats (one word) -> two order-preserving 16-bit keys, larger
// keys for larger values (v_pk_ashrrev_i16 + v_bitop3_b32). -0 (0x7FFF) sits
// just below +0 (0x8000); a positive NaN lies above +inf, a negative NaN below
// -inf.
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_key(uint32_t w) {
  const s16x2 m = __builtin_bit_cast(s16x2, w) >> (s16x2){15, 15};
  return w ^ (__builtin_bit_cast(uint32_t, m) | 0x80008000u);
}
__device__ __forceinline__ uint32_t pk_max(uint32_t x, uint32_t y) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_max(__builtin_bit_cast(u16x2, x), __builtin_bit_cast(u16x2, y)));
}
__device__ __forceinline__ uint32_t pk_min(uint32_t x, uint32_t y) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_min(__builtin_bit_cast(u16x2, x), __builtin_bit_cast(u16x2, y)));
}
__device__ __forceinline__ uint32_t pk_smax(uint32_t x, uint32_t y) {  // signed 16-bit halves
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_max(__builtin_bit_cast(s16x2, x), __builtin_bit_cast(s16x2, y)));
}
__device__ __forceinline__ uint32_t hmax(uint32_t w) { return max(w & 0xFFFFu, w >> 16); }
// A key's 16-bit float bits.
__device__ __forceinline__ uint32_t key_bits(uint32_t key) {
  return (key & 0x8000u) ? (key & 0x7FFFu) : (~key & 0xFFFFu);
}
template <typename T> struct Inf16;
template <> struct Inf16<bf16_t> {
  static constexpr uint32_t kPosKey = 0xFF80u, kNegKey = 0x007Fu, kNegBits = 0xFF80u;
};
template <> struct Inf16<f16_t> {
  static constexpr uint32_t kPosKey = 0xFC00u, kNegKey = 0x03FFu, kNegBits = 0xFC00u;
};

struct SampleLds {
  uint32_t cnt[kBuckets];
  uint64_t wsum[kBuckets];  // weight per bucket, then its exclusive prefix
  uint32_t pcnt[kBuckets];   // shared histogram: exclusive prefixes of cnt
  uint64_t pmass[kBuckets];  // and of the masses
  uint64_t keys[kCap];
  uint64_t wave_u64[kSampWaves];
  float wave_f[kSampWaves];
  int64_t wave_i[kSampWaves];
  uint32_t list_lo[2 * kMaxSegments];  // gather_lists: per (range, segment) its first list entry
  int list_n[2 * kMaxSegments];        // and its entries
  uint32_t n_gather;
  int found_bucket, found_bucket2;
  uint64_t found_cum;
  int64_t found_index;
  float found_x;
};

template <typename T, bool UNIT>  // UNIT: the row's elements are adjacent (stride 1)
struct RowSampler {
  const SampleArgs& a;
  SampleLds& s;
  const T* row;
  float t;     // clamped temperature
  float xmax;  // row maximum of x
  int tid, lane, wave;

  __device__ __forceinline__ float logit(int64_t i) const { return to_float(UNIT ? row[static_cast<int>(i)] : row[i * a.ls1]); }
  __device__ __forceinline__ float x_at(int64_t i) const { return __fdiv_rn(logit(i), t); }
  // The value the single-histogram path orders by. For 16-bit logits it is
  // the logit itself: distinct 16-bit values differ by at least 2^-8
  // relatively, so dividing them by one t keeps them distinct and in order,
  // and ties in x are exactly ties in the logit. fp32 logits order by x.
  static constexpr bool kByLogit = sizeof(T) == 2;
  __device__ __forceinline__ float key_at(int64_t i) const { return kByLogit ? logit(i) : x_at(i); }
  // f(i, key_at(i)) for every element of the row, each thread taking its
  // elements in an order of its own (every use is order-free). A 16-bit row
  // that is 16-byte aligned with a multiple of 8 elements is read 8 logits
  // per lane per load, so each load moves 1 KB per wave and several are in
  // flight; other rows one element at a time.
  __device__ __forceinline__ bool chunked() const {
    return UNIT && sizeof(T) == 2 && (reinterpret_cast<uintptr_t>(row) & 15) == 0 && (a.V & 7) == 0;
  }
  // f(i, key) for the elements whose key may lie in [lo, hi]: in a chunked
  // row an 8-logit chunk entirely outside the range is skipped after one
  // comparison (the callers' ranges carry a margin, and f still tests each
  // element exactly); otherwise every element.
  template <typename F>
  __device__ __forceinline__ void each_key_in(float lo, float hi, F f) const {
    if constexpr (UNIT && sizeof(T) == 2) {
      if (chunked()) {
        const u32x4* r4 = reinterpret_cast<const u32x4*>(row);
        each_chunk(r4, tid, static_cast<int>(a.V >> 3), kSampThreads, [&](const u32x4 w, int ch) {
          float l[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            l[2 * e] = lo_f<T>(w[e]);
            l[2 * e + 1] = hi_f<T>(w[e]);
          }
          float cmax = l[0], cmin = l[0];
#pragma unroll
          for (int e = 1; e < 8; ++e) {
            cmax = fmaxf(cmax, l[e]);
            cmin = fminf(cmin, l[e]);
          }
          if (cmax < lo || cmin > hi) return;  // (kByLogit: keys are the logits)
#pragma unroll
          for (int e = 0; e < 8; ++e) f(8 * ch + e, l[e]);
        });
        return;
      }
    }
    each_key(f);
  }
  // The key range that holds buckets [b0, b1] of the shared histogram, with
  // a bucket's width of margin on each side; unbounded where that cannot be
  // said (no spread, or the last bucket, which also takes -inf and NaN).
  __device__ __forceinline__ void bucket_range(int b0, int b1, float scale, float& lo, float& hi) const {
    lo = -INFINITY;
    hi = INFINITY;
    if (!(scale > 0.f) || b1 >= kBuckets - 1) return;
    lo = kmax - static_cast<float>(b1 + 2) / scale;
    lo -= fabsf(lo) * 1e-6f;  // and at least 16 ulps, for rows of tiny spread
    if (b0 > 0) {
      hi = kmax - static_cast<float>(b0 - 1) / scale;
      hi += fabsf(hi) * 1e-6f;
    }
  }

  template <typename F>
  __device__ __forceinline__ void each_key(F f) const {
    if constexpr (UNIT && sizeof(T) == 2) {
      if (chunked()) {
        const u32x4* r4 = reinterpret_cast<const u32x4*>(row);
        each_chunk(r4, tid, static_cast<int>(a.V >> 3), kSampThreads, [&](const u32x4 w, int ch) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float l = (e & 1) ? hi_f<T>(w[e >> 1]) : lo_f<T>(w[e >> 1]);
            f(8 * ch + e, kByLogit ? l : __fdiv_rn(l, t));
          }
        });
        return;
      }
    }
    for (int i = tid; i < static_cast<int>(a.V); i += kSampThreads) f(i, key_at(i));
  }
  __device__ __forceinline__ float key_to_x(float k) const { return kByLogit ? __fdiv_rn(k, t) : k; }
  float kmax;  // row maximum of key_at
  float kc;    // log2(e) / t for 16-bit logits, log2(e) for fp32 (keys are x)
  int64_t srow = -1;  // >= 0: the shared histogram is the sum of this row's split partials
  // 2^40 exp(x - xmax) from a key (mass_of): the single-histogram path's
  // mass; the row maximum weighs exactly 2^40.
  __device__ __forceinline__ uint64_t mass_key(float kv) const { return mass_of(kv, kmax, kc); }
  __device__ __forceinline__ uint64_t mass(float x) const {
    return static_cast<uint64_t>(rintf(expf(x - xmax) * kMassOne));
  }

  // Wave then block sum of a 64-bit value; every thread gets the total.
  __device__ __forceinline__ uint64_t block_sum(uint64_t v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    __syncthreads();
    if (lane == 0) s.wave_u64[wave] = v;
    __syncthreads();
    uint64_t tot = 0;
    for (int w = 0; w < kSampWaves; ++w) tot += s.wave_u64[w];
    return tot;
  }

  // Exclusive prefix of s.wsum over the buckets in place (two per thread),
  // in bucket order.
  __device__ __forceinline__ void scan_buckets() {
    const uint64_t w0 = s.wsum[2 * tid], w1 = s.wsum[2 * tid + 1];
    uint64_t incl = w0 + w1;
    incl = wave_scan_u64(incl);
    __syncthreads();
    if (lane == 63) s.wave_u64[wave] = incl;
    __syncthreads();
    uint64_t before = 0;
    for (int w = 0; w < wave; ++w) before += s.wave_u64[w];
    const uint64_t excl = before + incl - (w0 + w1);
    s.wsum[2 * tid] = excl;
    s.wsum[2 * tid + 1] = excl + w0;
    __syncthreads();
  }

  // s.keys[0, n) sorted ascending: up to one key per thread as below, more
  // by a bitonic network in LDS padded to a power of two.
  __device__ __forceinline__ void sort_keys(int n) {
    if (n <= kSampThreads) {
      // At most one key per thread: each wave sorts its 64 (a bitonic
      // network on cross-lane register moves; ~0, above every rank key,
      // pads the last run), the sorted runs go to LDS, and a key's place is
      // its lane plus the keys below it in every other run. The keys are
      // distinct (they hold the index).
      //
      // The count below x in a run is found by a 4-ary search in three
      // dependent rounds, four runs' searches side by side: keys 15, 31,
      // 47, 63 fix the block of 16, three keys in it the block of 4, three
      // keys in that the count. A run is stored with one empty slot after
      // each 16 keys (key e at kRunStride * run + e + e / 16), which puts
      // the addresses of each round's reads on distinct LDS banks.
      const int runs = (n + 63) >> 6;
      uint64_t x = tid < n ? s.keys[tid] : ~uint64_t{0};
      if (wave < runs) x = wave_sort_u64(x, lane);
      __syncthreads();
      if (wave < runs) s.keys[kRunStride * wave + lane + (lane >> 4)] = x;
      __syncthreads();
      int rank = lane;
      if (wave < runs) {
#pragma unroll 1
        for (int g = 0; g < runs; g += 4) {
          int below[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            below[i] = 0;
            if (g + i < runs && g + i != wave) {
              const uint64_t* r = &s.keys[kRunStride * (g + i)];
              below[i] = 16 * ((r[15] < x) + (r[32] < x) + (r[49] < x) + (r[66] < x));
            }
          }
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (g + i < runs && g + i != wave && below[i] < 64) {
              const uint64_t* r = &s.keys[kRunStride * (g + i) + below[i] + (below[i] >> 4)];
              below[i] += 4 * ((r[3] < x) + (r[7] < x) + (r[11] < x));
            }
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (g + i < runs && g + i != wave && below[i] < 64) {
              const uint64_t* r = &s.keys[kRunStride * (g + i) + below[i] + (below[i] >> 4)];
              below[i] += (r[0] < x) + (r[1] < x) + (r[2] < x);
            }
          rank += below[0] + below[1] + below[2] + below[3];
        }
      }
      __syncthreads();
      if (wave < runs && x != ~uint64_t{0}) s.keys[rank] = x;
      __syncthreads();
      return;
    }
    int p = 1;
    while (p < n) p <<= 1;
    for (int i = n + tid; i < p; i += kSampThreads) s.keys[i] = ~uint64_t{0};
    __syncthreads();
    for (int k = 2; k <= p; k <<= 1)
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < p; i += kSampThreads) {
          const int l = i ^ j;
          if (l > i) {
            const uint64_t x = s.keys[i], y = s.keys[l];
            if ((x > y) == ((i & k) == 0)) {
              s.keys[i] = y;
              s.keys[l] = x;
            }
          }
        }
        __syncthreads();
      }
  }

  __device__ __forceinline__ static int bucket0(float x, float h, float sc) {
    if (x == -INFINITY) return kBuckets - 1;
    const float f = (h - x) * sc;
    if (!(f < static_cast<float>(kBuckets - 1))) return kBuckets - 1;  // also NaN: never an index from it
    return f > 0.f ? static_cast<int>(f) : 0;
  }

  // Exclusive prefix over the buckets (two per thread) of in[] into out[].
  template <typename U>
  __device__ __forceinline__ void scan2(const U* in, U* out) {
    const U w0 = in[2 * tid], w1 = in[2 * tid + 1];
    uint64_t incl = static_cast<uint64_t>(w0) + w1;
    incl = wave_scan_u64(incl);
    __syncthreads();
    if (lane == 63) s.wave_u64[wave] = incl;
    __syncthreads();
    uint64_t before = 0;
    for (int w = 0; w < wave; ++w) before += s.wave_u64[w];
    const uint64_t excl = before + incl - (static_cast<uint64_t>(w0) + w1);
    out[2 * tid] = static_cast<U>(excl);
    out[2 * tid + 1] = static_cast<U>(excl + w0);
    __syncthreads();
  }

  // Both exclusive prefixes of the shared histogram, cnt into pcnt and wsum
  // into pmass, with one set of barriers (the sums of scan2, together).
  __device__ __forceinline__ void scan2_hist() {
    const uint32_t c0 = s.cnt[2 * tid], c1 = s.cnt[2 * tid + 1];
    const uint64_t m0 = s.wsum[2 * tid], m1 = s.wsum[2 * tid + 1];
    int64_t ic = static_cast<int64_t>(c0) + c1;
    uint64_t im = m0 + m1;
    ic = static_cast<int64_t>(wave_scan_u64(static_cast<uint64_t>(ic)));
    im = wave_scan_u64(im);
    __syncthreads();
    if (lane == 63) {
      s.wave_i[wave] = ic;
      s.wave_u64[wave] = im;
    }
    __syncthreads();
    int64_t bc = 0;
    uint64_t bm = 0;
    for (int w = 0; w < wave; ++w) {
      bc += s.wave_i[w];
      bm += s.wave_u64[w];
    }
    const int64_t ec = bc + ic - (static_cast<int64_t>(c0) + c1);
    const uint64_t em = bm + im - (m0 + m1);
    s.pcnt[2 * tid] = static_cast<uint32_t>(ec);
    s.pcnt[2 * tid + 1] = static_cast<uint32_t>(ec + c0);
    s.pmass[2 * tid] = em;
    s.pmass[2 * tid + 1] = em + m0;
    __syncthreads();
  }

  // atomicMin(at, b) for the wave's lowest lane with hit, where the wave's
  // lanes hold consecutive b (b = tid + j kSampThreads, the same j in every
  // lane): one LDS atomic per wave, not one per qualifying lane (on one
  // address those serialise).
  __device__ __forceinline__ void min_first_hit(int* at, bool hit, int b) {
    const uint64_t m = __ballot(hit);
    if (m != 0 && lane == __builtin_ctzll(m)) atomicMin(at, b);
  }

  // The smallest non-empty bucket b <= last whose running mass through b
  // (the full bucket, or last_incl for bucket `last`) reaches the target.
  __device__ __forceinline__ int first_bucket(int last, uint64_t last_incl, bool ge, double target) {
    if (tid == 0) s.found_bucket = kBuckets;
    __syncthreads();
    for (int b = tid; b < kBuckets; b += kSampThreads) {
      bool hit = false;
      if (b <= last && s.cnt[b] != 0) {
        const double incl = static_cast<double>(b == last ? last_incl : s.pmass[b] + s.wsum[b]);
        hit = ge ? incl >= target : incl > target;
      }
      min_first_hit(&s.found_bucket, hit, b);
    }
    __syncthreads();
    const int fb = s.found_bucket;
    __syncthreads();
    return fb;
  }

  // Gathers bucket b of the shared histogram into s.keys in rank order.
  // The first 16-bit key (pk_key order, between the -inf and +inf keys)
  // whose logit's bucket is at most b: bucket0 never increases along the
  // keys, so bisection finds it. No NaN reaches the histogram path.
  __device__ __forceinline__ uint32_t first_key_at_most(int b, float scale) const {
    uint32_t lo = Inf16<T>::kNegKey, hi = Inf16<T>::kPosKey + 1;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      if (bucket0(lo_f<T>(key_bits(mid)), kmax, scale) <= b) hi = mid;
      else lo = mid + 1;
    }
    return lo;
  }
  // Every element whose 16-bit key lies in [klo, khi] (or in [klo2, khi2]
  // too: TWO) into s.keys (as a rank key), for a chunked 16-bit row: per
  // 8-logit chunk, packed 16-bit keys, their offsets from klo and the
  // offsets' minimum tell in a few instructions whether any key of the
  // chunk is in range; only such chunks are looked into. (Reserving a
  // wave's matches with one atomic after a wave prefix of the lanes' counts
  // measured slower: the gather is bound by its instructions, not the
  // atomics' latency.)
  template <bool TWO = false>
  __device__ __forceinline__ void gather_key_range(uint32_t klo, uint32_t khi, uint32_t klo2 = 0, uint32_t khi2 = 0) {
    const uint32_t span = khi - klo, lo2 = klo | (klo << 16);
    const uint32_t span2 = khi2 - klo2, lo22 = klo2 | (klo2 << 16);
    each_chunk(reinterpret_cast<const u32x4*>(row), tid, static_cast<int>(a.V >> 3), kSampThreads,
               [&](const u32x4 w, int ch) {
                 uint32_t k[4], m = 0xFFFFFFFFu, m2 = 0xFFFFFFFFu;
#pragma unroll
                 for (int e = 0; e < 4; ++e) {
                   k[e] = pk_key(w[e]);
                   // key - klo in each half, mod 2^16: a key below klo wraps above span
                   m = pk_min(m, __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, k[e]) -
                                                                  __builtin_bit_cast(u16x2, lo2)));
                   if constexpr (TWO)
                     m2 = pk_min(m2, __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, k[e]) -
                                                                      __builtin_bit_cast(u16x2, lo22)));
                 }
                 const bool none = min(m & 0xFFFFu, m >> 16) > span;
                 if (TWO ? none && min(m2 & 0xFFFFu, m2 >> 16) > span2 : none) return;  // no key of the chunk in range
#pragma unroll
                 for (int e = 0; e < 8; ++e) {
                   const uint32_t key = (k[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
                   if (key - klo <= span || (TWO && key - klo2 <= span2)) {
                     const uint32_t at = atomicAdd(&s.n_gather, 1u);
                     if (at < kCap)
                       s.keys[at] = rank_key((e & 1) ? hi_f<T>(w[e >> 1]) : lo_f<T>(w[e >> 1]), 8 * ch + e);
                   }
                 }
               });
  }

  // A split row whose segments' bucket lists sample_split_hist wrote
  // (lists()): every element of buckets b0 .. b1 and, when b2 <= b3, of
  // buckets b2 .. b3, appended to s.keys (as a rank key) from the lists,
  // without a pass over the row: three dependent reads (the prefixes, the
  // list entries, the logits) for both ranges together. Segment g holds
  // [plp[g][b], plp[g][b' + 1]) of a range b .. b' (its element count past
  // the last bucket); an element's list entry is its index relative to
  // the segment.
  __device__ __forceinline__ bool lists() const { return srow >= 0 && a.pidx != nullptr; }
  __device__ __forceinline__ void gather_lists(int b0, int b1, int b2 = 1, int b3 = 0) {
    const int S = a.S;
    const size_t rs0 = static_cast<size_t>(srow) * S;
    if (tid < 2 * S) {  // thread g + S r: segment g, range r
      const int g = tid % S, rg = tid / S;
      const int lo_b = rg ? b2 : b0, hi_b = rg ? b3 : b1;
      int c0, c1;
      split_range(a, g, c0, c1);
      const uint32_t len = static_cast<uint32_t>(8 * (c1 - c0));  // the segment's elements
      uint32_t lo = 0, hi = 0;
      if (lo_b <= hi_b) {
        // (prefixes never exceed len: the clamps only bound every read below
        // to the segment's list, whatever the workspace held)
        lo = min(a.plp[(rs0 + g) * kBuckets + lo_b], len);
        hi = min(hi_b + 1 < kBuckets ? a.plp[(rs0 + g) * kBuckets + hi_b + 1] : len, len);
      }
      s.list_lo[tid] = lo;
      s.list_n[tid] = static_cast<int>(hi > lo ? hi - lo : 0);
    }
    __syncthreads();
    const uint32_t at0 = s.n_gather;
    int n = 0;
    for (int q = 0; q < 2 * S; ++q) n += s.list_n[q];
    for (int e = tid; e < n; e += kSampThreads) {
      int q = 0, first = 0;  // q: the (range, segment) pair holding element e
      while (q + 1 < 2 * S && e >= first + s.list_n[q]) first += s.list_n[q++];
      const int g = q % S;
      int c0, c1;
      split_range(a, g, c0, c1);
      const uint32_t li = a.pidx[(rs0 + g) * a.segcap + s.list_lo[q] + (e - first)];
      const int i = min(8 * c0 + static_cast<int>(li), 8 * c1 - 1);
      if (at0 + e < static_cast<uint32_t>(kCap)) s.keys[at0 + e] = rank_key(logit(i), i);
    }
    __syncthreads();
    if (tid == 0) s.n_gather = at0 + static_cast<uint32_t>(n);
    __syncthreads();
  }

  __device__ __forceinline__ bool gather_sorted(int b, float scale, int& cached) {
    if (cached == b) return true;
    if (tid == 0) s.n_gather = 0;
    __syncthreads();
    bool keyed = false;
    if (lists()) {
      gather_lists(b, b);
      keyed = true;
    }
    if constexpr (UNIT && sizeof(T) == 2) {
      if (!keyed && chunked()) {  // the bucket: keys [first_key_at_most(b), first_key_at_most(b - 1))
        const uint32_t klo = first_key_at_most(b, scale);
        const uint32_t khi = (b > 0 ? first_key_at_most(b - 1, scale) : Inf16<T>::kPosKey + 1) - 1;
        gather_key_range(klo, khi);
        keyed = true;
      }
    }
    // (a single bucket is a narrow range most chunks straddle: no skipping)
    if (!keyed)
      each_key([&](int i, float kv) {
        if (bucket0(kv, kmax, scale) == b) {
          const uint32_t at = atomicAdd(&s.n_gather, 1u);
          if (at < kCap) s.keys[at] = rank_key(kv, i);
        }
      });
    __syncthreads();
    if (s.n_gather != s.cnt[b]) return false;  // (the histogram's own count: never expected to differ)
    sort_keys(static_cast<int>(s.cnt[b]));
    cached = b;
    return true;
  }

  // Gathers every bucket up to nb (the top ranks of the row) into s.keys in
  // rank order: position e of the sorted list is rank e of the row.
  __device__ __forceinline__ bool gather_prefix(int nb, float scale) {
    if (tid == 0) s.n_gather = 0;
    __syncthreads();
    bool keyed = false;
    if (lists()) {
      gather_lists(0, nb);
      keyed = true;
    }
    if constexpr (UNIT && sizeof(T) == 2) {
      if (!keyed && chunked()) {  // buckets 0 .. nb: the keys from first_key_at_most(nb) up
        gather_key_range(first_key_at_most(nb, scale), Inf16<T>::kPosKey);
        keyed = true;
      }
    }
    if (!keyed) {
      float lo, hi;
      bucket_range(0, nb, scale, lo, hi);
      each_key_in(lo, hi, [&](int i, float kv) {
        if (bucket0(kv, kmax, scale) <= nb) {
          const uint32_t at = atomicAdd(&s.n_gather, 1u);
          if (at < kCap) s.keys[at] = rank_key(kv, i);
        }
      });
    }
    __syncthreads();
    if (s.n_gather != s.pcnt[nb] + s.cnt[nb]) return false;  // (never expected)
    sort_keys(static_cast<int>(s.pcnt[nb] + s.cnt[nb]));
    return true;
  }

  // Running masses of the sorted keys s.keys[0, n) (n <= kSampThreads),
  // into s.keys[kCumOff + e]: base0 plus the masses of [0, e] for e < n0,
  // base1 plus those of [n0, e] for e >= n0 (two runs of the rank order,
  // each starting from the mass of every bucket before it). One key per
  // thread, one scan; the decisions then read them (first_reaching).
  static constexpr int kCumOff = kCap - kSampThreads;
  __device__ __forceinline__ void running_mass(int n, int n0, uint64_t base0, uint64_t base1) {
    const uint64_t m = tid < n ? mass_key(key_of_rank(s.keys[tid])) : 0;
    uint64_t incl = m;
    incl = wave_scan_u64(incl);
    if (lane == 63) s.wave_u64[wave] = incl;
    __syncthreads();
    for (int w = 0; w < wave; ++w) incl += s.wave_u64[w];  // the masses of [0, tid]
    if (tid == n0 - 1) s.found_cum = incl;                  // the first run's
    __syncthreads();
    if (tid < n) s.keys[kCumOff + tid] = tid < n0 ? base0 + incl : base1 + incl - (n0 > 0 ? s.found_cum : 0);
    __syncthreads();
  }
  // The first position e in [lo, hi) (hi - lo <= kSampThreads) whose
  // running mass reaches the target (>= with ge, else >), or -1; the
  // running masses never decrease along [lo, hi).
  __device__ __forceinline__ int first_reaching(int lo, int hi, bool ge, double target) {
    if (tid == 0) s.found_index = -1;
    __syncthreads();
    auto reached = [&](int e) {
      const double c = static_cast<double>(s.keys[kCumOff + e]);
      return ge ? c >= target : c > target;
    };
    const int e = lo + tid;
    if (e < hi && reached(e) && (e == lo || !reached(e - 1))) s.found_index = e;
    __syncthreads();
    const int pos = static_cast<int>(s.found_index);
    __syncthreads();
    return pos;
  }

  // The decisions on the sorted top ranks [0, n): top-k keeps the first
  // lim_k, top-p the ranks through the first whose running mass exceeds
  // p * Z (z: the kept mass when known from the histogram, else summed
  // here), the pick is the first kept rank reaching u * (kept mass).
  __device__ __forceinline__ int64_t decide_on_prefix(int n, int lim_k, bool z_known, uint64_t z, double p, double u) {
    const int lk = lim_k >= 0 ? lim_k : n;
    running_mass(n, n, 0, 0);
    if (!z_known) z = lk > 0 ? s.keys[kCumOff + lk - 1] : 0;
    int lim = lk;
    uint64_t kept = z;
    const int pos_p = first_reaching(0, lk, false, p * static_cast<double>(z));
    if (pos_p >= 0) {
      lim = pos_p + 1;
      kept = s.keys[kCumOff + pos_p];
    }
    const int pos = first_reaching(0, lim, true, u * static_cast<double>(kept));
    if (pos < 0) return -1;
    const int64_t token = static_cast<uint32_t>(s.keys[pos]);
    __syncthreads();
    return token;
  }

  // Over the first `limit` sorted elements, with `base` before them: the
  // position of the one element that reaches the target (see select), its
  // running mass through it, and the mass of all `limit` elements.
  __device__ __forceinline__ int scan_sorted(int limit, uint64_t base, bool ge, double target, uint64_t& cum_at,
                                             uint64_t& total, int off = 0) {
    // (elements keys[off, off + limit); the position returned is relative to off)
    const int per = (limit + kSampThreads - 1) / kSampThreads;
    const int e0 = off + min(limit, tid * per), e1 = off + min(limit, tid * per + per);
    uint64_t mine = 0;
    for (int e = e0; e < e1; ++e) mine += mass_key(key_of_rank(s.keys[e]));  // no reload of the row
    uint64_t incl = mine;
    incl = wave_scan_u64(incl);
    __syncthreads();
    if (lane == 63) s.wave_u64[wave] = incl;
    if (tid == 0) s.found_index = -1;
    __syncthreads();
    uint64_t cum = base + incl - mine;
    for (int w = 0; w < wave; ++w) cum += s.wave_u64[w];
    uint64_t all = base;
    for (int w = 0; w < kSampWaves; ++w) all += s.wave_u64[w];
    for (int e = e0; e < e1; ++e) {
      const uint64_t excl = cum;
      cum += mass_key(key_of_rank(s.keys[e]));
      const bool r = ge ? static_cast<double>(cum) >= target : static_cast<double>(cum) > target;
      const bool rx = ge ? static_cast<double>(excl) >= target : static_cast<double>(excl) > target;
      if (r && (e == off || !rx)) {
        s.found_index = e - off;
        s.found_cum = cum;
        break;
      }
    }
    __syncthreads();
    const int pos = static_cast<int>(s.found_index);
    cum_at = s.found_cum;
    total = all;
    __syncthreads();
    return pos;
  }

  // The candidate pass for a top-k or greedy row of a 16-bit row of at most
  // kRegMaxV logits (chunked). load_row reads the row into registers (issued
  // before the row's parameters arrive); candidates then:
  //   1. takes each half-lane's largest logit as a sample (2048 distinct
  //      elements) and each chunk's largest key into LDS, from packed signed
  //      maxima of the raw patterns, and flags a NaN, a +inf or no sign of a
  //      value above -inf (those rows go on to the histogram paths);
  //   2. K = the k-th largest sample (12-bit prefix histogram, then the low 4
  //      bits of the samples in that prefix), so at least k elements have key
  //      >= K; +0's key is lowered to take -0 too; a cut at or below zero
  //      recomputes the chunk maxima from every key, and a row of negatives
  //      takes its samples from the keys too;
  //   3. finds the chunks holding a key >= K from each chunk's maximum (kept
  //      in LDS by step 1), skipping with a scalar test every chunk no lane
  //      of the wave holds one in, and stages those chunks in the wave's own
  //      LDS region (ballot offsets);
  //   4. wave 0 turns the staged chunks' keys >= K into candidates -- a
  //      prefix of the row in rank order that holds its first k ranks -- and,
  //      for at most 64, ranks them (a count: keys are distinct), moves each
  //      to its rank's lane (ds_permute) and decides there (decide_lanes);
  //   5. more candidates are ranked by the block, and decide_wave decides;
  //      a greedy row takes rank 0.
  // The token, or -1 to send the row on (more than kWaveStage chunks in a
  // wave or kGatherCap candidates, a non-finite row, or a pick past the
  // candidates).
  __device__ __forceinline__ void load_row(u32x4 (&ch)[kRegChunks]) const {
    // Chunk min(j * kSampThreads + tid, n8 - 1) of the row: a uniform base
    // (the first chunk of the block's j-th span, or the row's last chunk)
    // plus a clamped 32-bit lane offset.
    const int n8 = static_cast<int>(a.V >> 3);  // in [1, kSampThreads * kRegChunks]
    const char* base = reinterpret_cast<const char*>(row);
    const uint32_t toff = static_cast<uint32_t>(tid) << 4;
#pragma unroll
    for (int j = 0; j < kRegChunks; ++j) {
      const int cj = min(j * kSampThreads, n8 - 1);                      // (uniform)
      const uint32_t lim = static_cast<uint32_t>(n8 - 1 - cj) << 4;      // (uniform)
      ch[j] = *reinterpret_cast<const u32x4*>(base + (static_cast<int64_t>(cj) << 4) + min(toff, lim));
    }
  }

  __device__ __forceinline__ int64_t candidates(u32x4 (&ch)[kRegChunks], float temp, int64_t k, double p,
                                                double u) {
    constexpr uint32_t kNegKeys = Inf16<T>::kNegKey * 0x10001u;   // two -inf keys
    constexpr uint32_t kNegPair = Inf16<T>::kNegBits * 0x10001u;  // two -inf patterns
    constexpr int kMaxWords = (kRegChunks + 1) / 2;                // chunk maxima words per thread
    const int n8 = static_cast<int>(a.V >> 3);
    const uint32_t k_eff = temp <= 0.f ? 1u : static_cast<uint32_t>(k);  // in [1, kFastK]
    // LDS: red = s.cnt ([0, 16) wave maxima, [16, 32) unsigned maxima, [32, 48) bin
    // sums, [48] samples above the bin, [49] candidates, [64, 80) the
    // low-bits histogram, [80, 96) chunks staged per wave, [96, 112) wave
    // maxima of a negative row's exact samples); hist = s.wsum as kSelBins counts; cmx = each
    // thread's chunk maxima (two 16-bit keys a word, word w of thread t at
    // w * kSampThreads + t) from s.pcnt on; staged chunks after them; the
    // candidates in s.keys[kCandOff, kCap); ranked keys in s.keys[0, k)
    // once cmx is no longer read.
    static_assert(offsetof(SampleLds, pcnt) + sizeof(uint32_t) * kMaxWords * kSampThreads +
                          (sizeof(u32x4) + sizeof(uint32_t)) * kWaveStage * kSampWaves <=
                      offsetof(SampleLds, keys) + sizeof(uint64_t) * kCandOff,
                  "chunk maxima and staged chunks end before the candidates");
    uint32_t* red = s.cnt;
    uint32_t* hist = reinterpret_cast<uint32_t*>(s.wsum);
    uint32_t* cmx = s.pcnt;
    u32x4* stage = reinterpret_cast<u32x4*>(cmx + kMaxWords * kSampThreads);
    uint32_t* sid = reinterpret_cast<uint32_t*>(stage + kWaveStage * kSampWaves);
    uint64_t* cand = s.keys + kCandOff;
#pragma unroll
    for (int b = tid; b < kSelBins; b += kSampThreads) hist[b] = 0;
    if (tid < 16) red[64 + tid] = 0;
    __syncthreads();
    // 1. samples, chunk maxima and the row's flags from the raw 16-bit
    // patterns, two per packed op. A signed 16-bit maximum of the raw
    // patterns is the true maximum of any set holding a value >= +0 (sign-
    // magnitude order is integer order there, and every negative pattern is
    // below every non-negative one); in a set of negatives it is some element
    // of the set, which is all a sample needs. A positive NaN or +inf shows in
    // it; a negative NaN shows in the unsigned maximum (above -inf's pattern).
    // A chunk past the row's end (its load was clamped onto the row's last
    // chunk) counts as -inf, so it is never sampled or gathered.
    uint32_t t0 = 0x80008000u, um = 0, pend = 0;  // packed: each half-lane's signed and unsigned maxima
#pragma unroll
    for (int j = 0; j < kRegChunks; ++j) {
      const u32x4 w = ch[j];
      uint32_t sm = pk_smax(pk_smax(w[0], w[1]), pk_smax(w[2], w[3]));
      um = pk_max(um, pk_max(pk_max(w[0], w[1]), pk_max(w[2], w[3])));
      if (__builtin_expect((j + 1) * kSampThreads > n8, 0)) {  // (uniform: the row may end in this span)
        if (tid + j * kSampThreads >= n8) sm = kNegPair;
      }
      t0 = pk_smax(t0, sm);
      const uint32_t cm = hmax(pk_key(sm));  // the chunk's largest key if it holds a value >= +0
      if (j & 1) cmx[(j >> 1) * kSampThreads + tid] = pend | (cm << 16);
      else pend = cm;
    }
    if (kRegChunks & 1) cmx[(kMaxWords - 1) * kSampThreads + tid] = pend;
    const uint32_t tk = pk_key(t0);
    uint32_t wmx = hmax(tk), wum = hmax(um);
    for (int o = 32; o > 0; o >>= 1) {
      wmx = max(wmx, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wmx), o, 64)));
      wum = max(wum, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wum), o, 64)));
    }
    if (lane == 0) {
      red[wave] = wmx;
      red[16 + wave] = wum;
    }
    uint32_t s0 = tk & 0xFFFFu, s1 = tk >> 16;  // this thread's two samples (keys)
    atomicAdd(&hist[s0 >> 4], 1u);
    atomicAdd(&hist[s1 >> 4], 1u);
    __syncthreads();
    uint32_t kmx = 0, kum = 0;
#pragma unroll
    for (int w = 0; w < kSampWaves; ++w) {
      kmx = max(kmx, red[w]);
      kum = max(kum, red[16 + w]);
    }
    // A NaN or +inf, or no sign of anything above -inf (for a row of
    // negatives the signed maximum may not be the row's): the other paths.
    if (kmx >= Inf16<T>::kPosKey || kum > Inf16<T>::kNegBits) return -1;  // a NaN or +inf (uniform)
    bool exact_cmx = false;
    if (kmx < 0x8000u) {  // (uniform)
      // Every sample is negative, so the whole row is (a set holding a value
      // >= +0 has a sample >= +0): the signed maxima are then each set's
      // smallest element, which would put the cut far too low. Samples and
      // chunk maxima are taken again from the keys (one more pass over the
      // registers), and histogrammed instead.
#pragma unroll
      for (int b = tid; b < kSelBins; b += kSampThreads) hist[b] = 0;
      uint32_t tkk = 0;
#pragma unroll
      for (int j = 0; j < kRegChunks; ++j) {
        const u32x4 w = ch[j];
        uint32_t mj = pk_max(pk_max(pk_key(w[0]), pk_key(w[1])), pk_max(pk_key(w[2]), pk_key(w[3])));
        if (tid + j * kSampThreads >= n8) mj = kNegKeys;
        tkk = pk_max(tkk, mj);
        if (j & 1) cmx[(j >> 1) * kSampThreads + tid] = pend | (hmax(mj) << 16);
        else pend = hmax(mj);
      }
      if (kRegChunks & 1) cmx[(kMaxWords - 1) * kSampThreads + tid] = pend;
      exact_cmx = true;
      uint32_t wm = hmax(tkk);
      for (int o = 32; o > 0; o >>= 1) wm = max(wm, static_cast<uint32_t>(__shfl_xor(static_cast<int>(wm), o, 64)));
      if (lane == 0) red[96 + wave] = wm;
      __syncthreads();
      kmx = 0;
#pragma unroll
      for (int w = 0; w < kSampWaves; ++w) kmx = max(kmx, red[96 + w]);
      if (kmx <= Inf16<T>::kNegKey) return -1;  // every logit -inf (uniform)
      s0 = tkk & 0xFFFFu;
      s1 = tkk >> 16;
      atomicAdd(&hist[s0 >> 4], 1u);
      atomicAdd(&hist[s1 >> 4], 1u);
      __syncthreads();
    }
    // 2. thread t holds bins 4095 - 4t down to 4092 - 4t: a scan in descending order
    const int b0 = kSelBins - 1 - 4 * tid;
    const uint32_t h0 = hist[b0], h1 = hist[b0 - 1], h2 = hist[b0 - 2], h3 = hist[b0 - 3];
    const uint32_t mine = h0 + h1 + h2 + h3;
    uint32_t incl = mine;
    incl = wave_scan_u32(incl);
    if (lane == 63) red[32 + wave] = incl;
    __syncthreads();
    uint32_t excl = incl - mine;
    for (int w = 0; w < wave; ++w) excl += red[32 + w];
    if (excl < k_eff && excl + mine >= k_eff) {  // the one thread whose bins reach k_eff
      const uint32_t c0 = excl + h0, c1 = c0 + h1, c2 = c1 + h2;
      s.found_bucket = c0 >= k_eff ? b0 : c1 >= k_eff ? b0 - 1 : c2 >= k_eff ? b0 - 2 : b0 - 3;
      red[48] = c0 >= k_eff ? excl : c1 >= k_eff ? c0 : c2 >= k_eff ? c1 : c2;  // samples above that bin
    }
    __syncthreads();
    const uint32_t bin = static_cast<uint32_t>(s.found_bucket), need = k_eff - red[48];
    if ((s0 >> 4) == bin) atomicAdd(&red[64 + (s0 & 15u)], 1u);
    if ((s1 >> 4) == bin) atomicAdd(&red[64 + (s1 & 15u)], 1u);
    __syncthreads();
    uint32_t low = 0, c = 0;
#pragma unroll
    for (int b = 15; b >= 0; --b) {  // the low bits where the count from the top reaches `need`
      const uint32_t c2 = c + red[64 + b];
      if (c < need && c2 >= need) low = static_cast<uint32_t>(b);
      c = c2;
    }
    uint32_t K = (bin << 4) | low;  // >= the -inf key: the row holds no NaN
    if (K == 0x8000u) K = 0x7FFFu;   // +0: -0 has the same value
    if (K <= 0x8000u && !exact_cmx) {  // (uniform) a cut at or below zero: every chunk's exact largest key
#pragma unroll
      for (int j = 0; j < kRegChunks; ++j) {
        const u32x4 w = ch[j];
        uint32_t mj = pk_max(pk_max(pk_key(w[0]), pk_key(w[1])), pk_max(pk_key(w[2]), pk_key(w[3])));
        if (tid + j * kSampThreads >= n8) mj = kNegKeys;
        if (j & 1) cmx[(j >> 1) * kSampThreads + tid] = pend | (hmax(mj) << 16);
        else pend = hmax(mj);
      }
      if (kRegChunks & 1) cmx[(kMaxWords - 1) * kSampThreads + tid] = pend;
    }
    // 3. the chunks holding a key >= K (from the chunk maxima), staged in
    // the wave's own LDS region (ballot offsets)
    uint32_t mask = 0;
#pragma unroll
    for (int w2 = 0; w2 < kMaxWords; ++w2) {
      const uint32_t v = cmx[w2 * kSampThreads + tid];
      mask |= ((v & 0xFFFFu) >= K ? 1u : 0u) << (2 * w2);
      if (2 * w2 + 1 < kRegChunks) mask |= ((v >> 16) >= K ? 1u : 0u) << (2 * w2 + 1);
    }
    const int nv = n8 > tid ? (n8 - tid + kSampThreads - 1) / kSampThreads : 0;  // this lane's chunks in the row
    mask &= (1u << nv) - 1u;                                                      // (nv <= kRegChunks < 32)
    uint32_t wmask = mask;
    for (int o = 1; o < 64; o <<= 1) wmask |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(wmask), o, 64));
    wmask = __builtin_amdgcn_readfirstlane(wmask);  // (uniform: the wave's hot chunks)
    u32x4* my_stage = stage + wave * kWaveStage;
    uint32_t* my_sid = sid + wave * kWaveStage;
    uint32_t nst = 0;  // (uniform) chunks this wave staged
#pragma unroll
    for (int j = 0; j < kRegChunks; ++j) {
      if (!(wmask & (1u << j))) continue;  // (uniform)
      const bool hot = (mask >> j) & 1u;
      const uint64_t b = __ballot(hot);
      const uint32_t at = nst + lane_rank(b);
      if (hot && at < static_cast<uint32_t>(kWaveStage)) {
        my_stage[at] = ch[j];
        my_sid[at] = static_cast<uint32_t>(tid + j * kSampThreads);
      }
      nst += static_cast<uint32_t>(__popcll(b));
    }
    if (lane == 0) red[80 + wave] = nst;
    __syncthreads();
    uint32_t total = 0;
    bool over = false;
#pragma unroll
    for (int w = 0; w < kSampWaves; ++w) {
      total += red[80 + w];
      over = over || red[80 + w] > static_cast<uint32_t>(kWaveStage);
    }
    if (over) return -1;  // (uniform)
    const float kc0 = 1.4426950408889634f / t;  // (16-bit rows order by the logit)
    // 4. wave 0: the staged chunks' keys >= K become candidates; for at most
    // 64 it ranks and decides at once
    if (wave == 0) {
      uint32_t nc = 0;  // (uniform) candidates written
      for (uint32_t i0 = 0; i0 < total; i0 += 64) {
        const uint32_t i = i0 + lane;
        uint32_t base = 0, reg = 0;  // staged chunk i: region `reg`, whose chunks start at `base`
#pragma unroll
        for (int w = 1; w < kSampWaves; ++w) {
          uint32_t pre = 0;
#pragma unroll
          for (int w3 = 0; w3 < w; ++w3) pre += red[80 + w3];
          if (i >= pre) {
            base = pre;
            reg = static_cast<uint32_t>(w);
          }
        }
        u32x4 w = u32x4{0, 0, 0, 0};
        uint32_t id = 0;
        if (i < total) {
          const u32x4 raw = stage[reg * kWaveStage + (i - base)];
          w = u32x4{pk_key(raw[0]), pk_key(raw[1]), pk_key(raw[2]), pk_key(raw[3])};
          id = sid[reg * kWaveStage + (i - base)];
        }
        uint32_t take = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          take |= ((w[e] & 0xFFFFu) >= K ? 1u : 0u) << (2 * e) | ((w[e] >> 16) >= K ? 1u : 0u) << (2 * e + 1);
        if (i >= total) take = 0;
        const uint32_t cnt = __popc(take);
        uint32_t pre = 0, tot = 0;  // exclusive prefix of cnt (<= 8) over the wave, by bit planes
#pragma unroll
        for (int bp = 0; bp < 4; ++bp) {
          const uint64_t bb = __ballot((cnt >> bp) & 1u);
          pre += lane_rank(bb) << bp;
          tot += static_cast<uint32_t>(__popcll(bb)) << bp;
        }
        uint32_t at = nc + pre;
        while (take) {  // (usually once)
          const int e = __builtin_ctz(take);
          take &= take - 1;
          const uint32_t word = e >= 4 ? (e >= 6 ? w[3] : w[2]) : (e >= 2 ? w[1] : w[0]);
          const uint32_t key = (word >> ((e & 1) * 16)) & 0xFFFFu;
          if (at < static_cast<uint32_t>(kGatherCap)) cand[at] = cand_key(key, 8 * id + static_cast<uint32_t>(e));
          ++at;
        }
        nc += tot;
      }
      const uint32_t nc8 = (nc + 7) & ~7u;  // padded with keys that rank below every candidate
      if (nc + lane < min(nc8, static_cast<uint32_t>(kGatherCap))) cand[nc + lane] = ~uint64_t{0};
      int64_t token = -2;  // (more than 64 candidates: the block ranks them below)
      if (nc <= 64) {
        const int lk = static_cast<int>(min(k_eff, nc));  // (nc >= k_eff: at least k_eff samples are >= K)
        const uint64_t kv = lane < static_cast<int>(nc) ? cand[lane] : ~uint64_t{0};
        int rank = 0;
        for (uint32_t q = 0; q < nc8; q += 8) {
#pragma unroll
          for (int i = 0; i < 8; ++i) rank += cand[q + i] < kv ? 1 : 0;
        }
        if (lane >= static_cast<int>(nc)) rank = lane;  // (distinct from the ranks below nc)
        const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_ds_permute(rank * 4, static_cast<int>(kv)));
        const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_ds_permute(rank * 4, static_cast<int>(kv >> 32)));
        const uint64_t sorted = (static_cast<uint64_t>(hi) << 32) | lo;  // lane e: rank e
        const uint32_t top_lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(lo)));
        const uint32_t top_hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(hi)));
        token = temp <= 0.f ? static_cast<int64_t>(top_lo)  // greedy: rank 0
                            : decide_lanes(sorted, lk, cand_value((static_cast<uint64_t>(top_hi) << 32) | top_lo),
                                           kc0, p, u);
      }
      if (lane == 0) {
        s.found_index = token;
        red[49] = nc;
      }
    }
    __syncthreads();
    if (s.found_index != -2) return s.found_index;  // (uniform)
    // 5. more than 64 candidates: every thread ranks, wave 0 decides
    const uint32_t n = red[49];
    if (n > static_cast<uint32_t>(kGatherCap)) return -1;
    const int lk = static_cast<int>(min(k_eff, n));
    const int n8c = static_cast<int>(min((n + 7) & ~7u, static_cast<uint32_t>(kGatherCap)));
    for (int i = tid; i < static_cast<int>(n); i += kSampThreads) {  // each candidate's rank among them
      const uint64_t kv = cand[i];
      int rank = 0, q = 0;
      for (; q + 8 <= n8c; q += 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) rank += cand[q + e] < kv ? 1 : 0;
      }
      for (; q < static_cast<int>(n); ++q) rank += cand[q] < kv ? 1 : 0;
      if (rank < lk) s.keys[rank] = kv;
    }
    __syncthreads();
    if (temp <= 0.f) return static_cast<uint32_t>(s.keys[0]);  // greedy: the first index of the maximum
    kmax = cand_value(s.keys[0]);
    kc = kc0;
    if (wave == 0) {
      const int64_t token = decide_wave(lk, p, u);
      if (lane == 0) s.found_index = token;
    }
    __syncthreads();
    return s.found_index;
  }

  // Candidate keys: (0xFFFF - key) << 32 | index, with -0's key folded into
  // +0's. Ascending order is the stable descending sort's order (larger
  // values first, ties by index), as for rank_key; cand_value gives back the
  // logit (-0 as +0).
  __device__ __forceinline__ static uint64_t cand_key(uint32_t key, uint32_t index) {
    const uint32_t folded = key == 0x7FFFu ? 0x8000u : key;
    return (static_cast<uint64_t>(0xFFFFu - folded) << 32) | index;
  }
  __device__ __forceinline__ static float cand_value(uint64_t ck) {
    return lo_f<T>(key_bits(0xFFFFu - static_cast<uint32_t>(ck >> 32)));
  }
  // The lane's place among the lanes of a ballot below it.
  __device__ __forceinline__ static uint32_t lane_rank(uint64_t b) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(b >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(b), 0u));
  }

  // decide_on_prefix(lk, lk, ...) on ranks held one per lane (lane e: rank e,
  // lk <= 64), with the row's maximum km: the same masses and comparisons.
  __device__ __forceinline__ int64_t decide_lanes(uint64_t sorted, int lk, float km, float kcv, double p,
                                                  double u) const {
    const uint64_t m = lane < lk ? mass_of(cand_value(sorted), km, kcv) : 0;
    uint64_t incl = m;
    incl = wave_scan_u64(incl);
    const uint64_t excl = incl - m;
    const uint64_t z = __shfl(incl, 63, 64);
    const double tp = p * static_cast<double>(z);
    const uint64_t hp = __ballot(lane < lk && static_cast<double>(incl) > tp &&
                                 (lane == 0 || !(static_cast<double>(excl) > tp)));
    int lim = lk;
    uint64_t kept = z;
    if (hp != 0) {
      const int src = __builtin_ctzll(hp);
      lim = src + 1;
      kept = __shfl(incl, src, 64);
    }
    const double tu = u * static_cast<double>(kept);
    const uint64_t hu = __ballot(lane < lim && static_cast<double>(incl) >= tu &&
                                 (lane == 0 || !(static_cast<double>(excl) >= tu)));
    if (hu == 0) return -1;
    return static_cast<uint32_t>(__shfl(static_cast<int>(static_cast<uint32_t>(sorted)), __builtin_ctzll(hu), 64));
  }

  // decide_on_prefix(lk, lk, ...) in one wave, on s.keys[0, lk) (lk <= 512):
  // lane L holds ranks [8L, 8L + 8); the masses are exact integers, so the
  // running sums, and every comparison with the targets, are the same.
  __device__ __forceinline__ int64_t decide_wave(int lk, double p, double u) const {
    uint64_t m[8];
    uint64_t mine = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = 8 * lane + i;
      m[i] = e < lk ? mass_key(cand_value(s.keys[e])) : 0;
      mine += m[i];
    }
    uint64_t incl = mine;
    incl = wave_scan_u64(incl);
    const uint64_t z = __shfl(incl, 63, 64);
    // top-p: the first rank whose running mass exceeds p * z (exactly one lane holds it)
    const double tp = p * static_cast<double>(z);
    uint64_t cum = incl - mine;
    int pos_p = -1;
    uint64_t cum_p = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = 8 * lane + i;
      const uint64_t c2 = cum + m[i];
      if (e < lk && pos_p < 0 && static_cast<double>(c2) > tp && (e == 0 || !(static_cast<double>(cum) > tp))) {
        pos_p = e;
        cum_p = c2;
      }
      cum = c2;
    }
    const uint64_t hp = __ballot(pos_p >= 0);
    int lim = lk;
    uint64_t kept = z;
    if (hp != 0) {
      const int src = __builtin_ctzll(hp);
      lim = __shfl(pos_p, src, 64) + 1;
      kept = __shfl(cum_p, src, 64);
    }
    // the pick: the first kept rank whose running mass reaches u * kept
    const double tu = u * static_cast<double>(kept);
    cum = incl - mine;
    int pos = -1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = 8 * lane + i;
      const uint64_t c2 = cum + m[i];
      if (e < lim && pos < 0 && static_cast<double>(c2) >= tu && (e == 0 || !(static_cast<double>(cum) >= tu)))
        pos = e;
      cum = c2;
    }
    const uint64_t hu = __ballot(pos >= 0);
    if (hu == 0) return -1;
    const int at = __shfl(pos, __builtin_ctzll(hu), 64);
    return static_cast<int64_t>(static_cast<uint32_t>(s.keys[at]));
  }

  // All three decisions from one histogram of every element (count and
  // mass): each decision's kept set is a prefix in rank order -- full buckets,
  // then a known prefix of one sorted bucket -- so only the buckets where a
  // cut or the pick falls are gathered. False if such a bucket is larger
  // than LDS holds (the caller then runs the per-decision path).
  // A top-p cut in bucket bp (no top-k cut) and the pick from one gather of
  // the row. The kept mass lies in [pmass[bp], pmass[bp] + wsum[bp]]:
  // whole buckets before bp, then a prefix of bp. The pick bucket is the
  // first non-empty bucket whose running mass reaches u * (kept mass), bp's
  // own running mass being the kept mass (which u < 1 reaches), so it lies
  // between the buckets that u times either end reaches (blo and bhi; a
  // larger target never reaches an earlier bucket), or is bp. The buckets
  // blo .. min(bhi, bp - 1) and bp are gathered in one pass (two key
  // ranges) and sorted together (rank order: the earlier buckets first),
  // and the cut and the pick are the scans the two-gather path makes, on the
  // same sorted elements. False (nothing decided) when they exceed one key
  // per thread, or the gathered count is not the histogram's.
  __device__ __forceinline__ bool cut_and_pick(int bp, uint64_t z, double p, double u, float scale, int64_t& token) {
    const double tlo = u * static_cast<double>(s.pmass[bp]);
    const double thi = u * static_cast<double>(s.pmass[bp] + s.wsum[bp]);
    if (tid == 0) {
      s.found_bucket = bp;
      s.found_bucket2 = bp;
    }
    __syncthreads();
    for (int b = tid; b < kBuckets; b += kSampThreads) {
      bool hlo = false, hhi = false;
      if (b < bp && s.cnt[b] != 0) {
        const double incl = static_cast<double>(s.pmass[b] + s.wsum[b]);
        hlo = incl >= tlo;
        hhi = incl >= thi;
      }
      min_first_hit(&s.found_bucket, hlo, b);
      min_first_hit(&s.found_bucket2, hhi, b);
    }
    __syncthreads();
    const int blo = s.found_bucket, last = min(s.found_bucket2, bp - 1);
    __syncthreads();
    const uint32_t n_u = blo <= last ? s.pcnt[last] + s.cnt[last] - s.pcnt[blo] : 0u;  // elements of blo .. last
    const uint32_t n = n_u + s.cnt[bp];
    if (n > static_cast<uint32_t>(kSampThreads)) return false;
    // bucket b holds the keys [first_key_at_most(b), first_key_at_most(b - 1)), bucket 0 up to +inf
    auto key_end = [&](int b) { return b > 0 ? first_key_at_most(b - 1, scale) - 1 : Inf16<T>::kPosKey; };
    if (tid == 0) s.n_gather = 0;
    __syncthreads();
    if (lists()) {
      if (blo > last) gather_lists(bp, bp);
      else if (last + 1 == bp) gather_lists(blo, bp);
      else gather_lists(blo, last, bp, bp);
    } else {
      const uint32_t kb_lo = first_key_at_most(bp, scale), kb_hi = key_end(bp);
      if (blo > last) gather_key_range(kb_lo, kb_hi);
      else if (last + 1 == bp) gather_key_range(kb_lo, key_end(blo));  // adjacent: one range
      else gather_key_range<true>(kb_lo, kb_hi, first_key_at_most(last, scale), key_end(blo));
    }
    __syncthreads();
    if (s.n_gather != n) return false;  // (the histogram's own counts: never expected to differ)
    sort_keys(static_cast<int>(n));
    // Rank order: buckets blo .. last, then bp; the running mass of each
    // run starts from the mass of the buckets before it, and never
    // decreases along the list (the buckets between last and bp, if any,
    // come after the pick). The cut: the first of bp's keys past p * Z; the
    // pick: the first key through the cut reaching u * (the kept mass).
    running_mass(static_cast<int>(n), static_cast<int>(n_u), n_u > 0 ? s.pmass[blo] : 0, s.pmass[bp]);
    const int pos = first_reaching(static_cast<int>(n_u), static_cast<int>(n), false, p * static_cast<double>(z));
    if (pos < 0) return false;
    const uint64_t kept = s.keys[kCumOff + pos];
    const int pos2 = first_reaching(0, pos + 1, true, u * static_cast<double>(kept));
    if (pos2 < 0) return false;
    token = static_cast<uint32_t>(s.keys[pos2]);
    __syncthreads();
    return true;
  }

  // The shared histogram of split row srow: the sum of its S partials
  // (sample_split_hist: the same buckets and masses), into s.pcnt (the
  // count prefix) and s.wsum, then s.cnt. Made before the row's statistics
  // are used (it needs none of them), so its loads share a round trip with
  // the statistics record's.
  __device__ __forceinline__ void merge_partials() {
    // The segments' count prefixes add up to the row's (pcnt), and a
    // bucket's count is the step to the next bucket's prefix (the last
    // bucket's to V: every element is in one bucket).
    const size_t base = static_cast<size_t>(srow) * a.S * kBuckets;
    static_assert(kBuckets == 2 * kSampThreads, "two buckets per thread");
    // Thread t takes buckets 2t and 2t + 1: one 8-byte count load and one
    // 16-byte mass load per segment. Eight segments per step, every load (at
    // a clamped segment) issued before any is summed: one round trip for
    // the usual 8 segments.
    u32x2 c = {0u, 0u};
    uint64_t m0 = 0, m1 = 0;
    for (int w0 = 0; w0 < a.S; w0 += 8) {
      u32x2 cw[8];
      u32x4 mw[8];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const size_t at = base + static_cast<size_t>(min(w0 + w, a.S - 1)) * kBuckets + 2 * tid;
        cw[w] = *reinterpret_cast<const u32x2*>(a.plp + at);
        mw[w] = *reinterpret_cast<const u32x4*>(a.pmass + at);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        if (w0 + w < a.S) {
          c[0] += cw[w][0];
          c[1] += cw[w][1];
          m0 += (static_cast<uint64_t>(mw[w][1]) << 32) | mw[w][0];
          m1 += (static_cast<uint64_t>(mw[w][3]) << 32) | mw[w][2];
        }
      }
    }
    s.pcnt[2 * tid] = c[0];
    s.pcnt[2 * tid + 1] = c[1];
    s.wsum[2 * tid] = m0;
    s.wsum[2 * tid + 1] = m1;
    __syncthreads();
    for (int b = tid; b < kBuckets; b += kSampThreads)
      s.cnt[b] = (b + 1 < kBuckets ? s.pcnt[b + 1] : static_cast<uint32_t>(a.V)) - s.pcnt[b];
  }

  __device__ __forceinline__ bool fast(float lo, int64_t k, bool cut_k, double p, double u, int64_t& token) {
    // lo: the smallest finite key
    const float scale = kmax > lo ? static_cast<float>(kBuckets - 1) / (kmax - lo) : 0.f;
    if (srow < 0) {  // (a split row's partials were merged by merge_partials)
      for (int b = tid; b < kBuckets; b += kSampThreads) {
        s.cnt[b] = 0;
        s.wsum[b] = 0;
      }
      __syncthreads();
      each_key([&](int, float kv) {
        const int b = bucket0(kv, kmax, scale);
        atomicAdd(&s.cnt[b], 1u);
        atomicAdd(reinterpret_cast<unsigned long long*>(&s.wsum[b]), static_cast<unsigned long long>(mass_key(kv)));
      });
    }
    __syncthreads();
    // (for a split row this recomputes the count prefix the merge summed,
    // with the mass prefix: one scan, and the kernel stays in 124 VGPRs
    // where a mass-only scan here made it spill)
    scan2_hist();
    int cached = -1;
    uint64_t cum, tot;
    // top-k: bucket bk holds rank k - 1; its first need_k sorted elements stay.
    int bk = kBuckets - 1, lim_k = -1;
    uint64_t z = s.pmass[kBuckets - 1] + s.wsum[kBuckets - 1];
    if (cut_k) {
      if (tid == 0) s.found_bucket = kBuckets;
      __syncthreads();
      for (int b = tid; b < kBuckets; b += kSampThreads)
        min_first_hit(&s.found_bucket, s.cnt[b] > 0 && static_cast<int64_t>(s.pcnt[b]) + s.cnt[b] >= k, b);
      __syncthreads();
      bk = s.found_bucket;
      __syncthreads();
      if (s.pcnt[bk] + s.cnt[bk] <= kPrefixMax) {  // every decision lies in the few top ranks: one gather
        if (!gather_prefix(bk, scale)) return false;
        token = decide_on_prefix(static_cast<int>(s.pcnt[bk] + s.cnt[bk]), static_cast<int>(k), false, 0, p, u);
        return token >= 0;
      }
      if (s.cnt[bk] > kCap) return false;
      lim_k = static_cast<int>(k - s.pcnt[bk]);
      if (!gather_sorted(bk, scale, cached)) return false;
      scan_sorted(lim_k, s.pmass[bk], true, -1.0, cum, tot);
      z = tot;  // mass of every kept rank
    }
    // top-p: the first rank whose running mass exceeds p * Z is the last kept.
    int last = bk, lim_last = lim_k;
    uint64_t kept = z;
    const int bp = first_bucket(bk, z, false, p * static_cast<double>(z));
    if (!cut_k && bp < kBuckets && s.pcnt[bp] + s.cnt[bp] <= kPrefixMax) {  // few kept ranks: one gather
      if (!gather_prefix(bp, scale)) return false;
      token = decide_on_prefix(static_cast<int>(s.pcnt[bp] + s.cnt[bp]), -1, true, z, p, u);
      return token >= 0;
    }
    if constexpr (UNIT && sizeof(T) == 2) {
      if (!cut_k && bp < kBuckets && chunked() && cut_and_pick(bp, z, p, u, scale, token)) return true;
    }
    if (bp < kBuckets) {
      if (s.cnt[bp] > kCap) return false;
      if (!gather_sorted(bp, scale, cached)) return false;
      const int lim = bp == bk && lim_k >= 0 ? lim_k : static_cast<int>(s.cnt[bp]);
      const int pos = scan_sorted(lim, s.pmass[bp], false, p * static_cast<double>(z), cum, tot);
      if (pos < 0) return false;
      last = bp;
      lim_last = pos + 1;
      kept = cum;
    }
    // pick: the first kept rank whose running mass reaches u * (kept mass).
    const double tu = u * static_cast<double>(kept);
    const int bu = first_bucket(last, kept, true, tu);
    if (bu == kBuckets || s.cnt[bu] > kCap) return false;
    if (!gather_sorted(bu, scale, cached)) return false;
    const int lim = bu == last && lim_last >= 0 ? lim_last : static_cast<int>(s.cnt[bu]);
    const int pos = scan_sorted(lim, s.pmass[bu], true, tu, cum, tot);
    if (pos < 0) return false;
    token = static_cast<uint32_t>(s.keys[pos]);
    __syncthreads();
    return true;
  }

  // The first candidate (keep(i, x)) in rank order whose running weight
  // (1 or its mass) reaches the target: cum >= target (ge) or cum > target.
  // The target is target_abs, or frac * (total candidate weight) when
  // use_frac. Returns false when no candidate reaches it.
  template <typename Keep>
  __device__ __forceinline__ bool select(Keep keep, bool by_mass, bool ge, bool use_frac, double frac, double target_abs,
                         float lo, float hi, float& rx, int64_t& ri, uint64_t& rcum) {
    float lv_hi[kMaxLevels] = {}, lv_scale[kMaxLevels] = {};
    int lv_b[kMaxLevels] = {};
    int levels = 0;
    uint64_t base = 0;
    double target = target_abs;
    auto bucket_of = [](float x, float h, float sc) -> int {
      if (x == -INFINITY) return kBuckets - 1;
      const float f = (h - x) * sc;
      // NaN (a NaN logit, or +inf - +inf) fails the test and takes the last
      // bucket, so no index is ever formed from it.
      if (!(f < static_cast<float>(kBuckets - 1))) return kBuckets - 1;
      return f > 0.f ? static_cast<int>(f) : 0;
    };
    // (the level arrays are only ever indexed by unrolled constants, so they
    // stay in registers)
    auto in_levels = [&](float x) {
      bool in = true;
#pragma unroll
      for (int l = 0; l < kMaxLevels; ++l)
        if (l < levels && bucket_of(x, lv_hi[l], lv_scale[l]) != lv_b[l]) in = false;
      return in;
    };
    auto reached = [&](uint64_t cum) {
      const double c = static_cast<double>(cum);
      return ge ? c >= target : c > target;
    };
    for (;;) {
      const float scale = hi > lo ? static_cast<float>(kBuckets - 1) / (hi - lo) : 0.f;
      for (int b = tid; b < kBuckets; b += kSampThreads) {
        s.cnt[b] = 0;
        s.wsum[b] = 0;
      }
      __syncthreads();
      for (int i = tid; i < static_cast<int>(a.V); i += kSampThreads) {
        const float x = x_at(i);
        if (!keep(i, x) || !in_levels(x)) continue;
        const int b = bucket_of(x, hi, scale);
        atomicAdd(&s.cnt[b], 1u);
        atomicAdd(reinterpret_cast<unsigned long long*>(&s.wsum[b]),
                  static_cast<unsigned long long>(by_mass ? mass(x) : 1));
      }
      __syncthreads();
      if (levels == 0 && use_frac) {
        uint64_t part = s.wsum[2 * tid] + s.wsum[2 * tid + 1];
        target = frac * static_cast<double>(block_sum(part));
      }
      const uint64_t w_last = s.wsum[kBuckets - 1];
      scan_buckets();  // s.wsum[b] = weight of buckets before b
      // The first non-empty bucket whose inclusive running weight reaches the
      // target (the running weight never decreases along the buckets).
      if (tid == 0) s.found_bucket = kBuckets;
      __syncthreads();
      for (int b = tid; b < kBuckets; b += kSampThreads) {
        const uint64_t incl = b + 1 < kBuckets ? s.wsum[b + 1] : s.wsum[b] + w_last;
        min_first_hit(&s.found_bucket, s.cnt[b] > 0 && reached(base + incl), b);
      }
      __syncthreads();
      const int fb = s.found_bucket;
      if (fb == kBuckets) return false;
      base += s.wsum[fb];
      const uint32_t n = s.cnt[fb];
      __syncthreads();
      if (n <= kCap) {
        // Gather the bucket, sort it in rank order, prefix-sum its weights.
        if (tid == 0) s.n_gather = 0;
        __syncthreads();
        for (int i = tid; i < static_cast<int>(a.V); i += kSampThreads) {
          const float x = x_at(i);
          if (!keep(i, x) || !in_levels(x) || bucket_of(x, hi, scale) != fb) continue;
          const uint32_t at = atomicAdd(&s.n_gather, 1u);
          if (at < kCap) s.keys[at] = rank_key(x, i);
        }
        __syncthreads();
        sort_keys(static_cast<int>(n));
        // Each thread takes a contiguous run of the sorted elements.
        const int per = (static_cast<int>(n) + kSampThreads - 1) / kSampThreads;
        const int e0 = min(static_cast<int>(n), tid * per), e1 = min(static_cast<int>(n), e0 + per);
        uint64_t mine = 0;
        for (int e = e0; e < e1; ++e) mine += by_mass ? mass(x_at(static_cast<uint32_t>(s.keys[e]))) : 1;
        uint64_t incl = mine;
        incl = wave_scan_u64(incl);
        __syncthreads();
        if (lane == 63) s.wave_u64[wave] = incl;
        if (tid == 0) s.found_index = -1;
        __syncthreads();
        uint64_t cum = base + incl - mine;
        for (int w = 0; w < wave; ++w) cum += s.wave_u64[w];
        // The one element that reaches the target while the one before it
        // does not (or that is the bucket's first, when the running weight
        // before the bucket already reaches it).
        for (int e = e0; e < e1; ++e) {
          const int64_t i = static_cast<uint32_t>(s.keys[e]);
          const float x = x_at(i);
          const uint64_t excl = cum;
          cum += by_mass ? mass(x) : 1;
          if (reached(cum) && (e == 0 || !reached(excl))) {
            s.found_index = i;
            s.found_x = x;
            s.found_cum = cum;
            break;
          }
        }
        __syncthreads();
        ri = s.found_index;
        rx = s.found_x;
        rcum = s.found_cum;
        __syncthreads();
        return ri >= 0;
      }
      // Too many for LDS: the bucket's value range, then split it again or,
      // if all its elements hold one value, resolve in index order.
      float bmin = INFINITY, bmax = -INFINITY;
      for (int i = tid; i < static_cast<int>(a.V); i += kSampThreads) {
        const float x = x_at(i);
        if (!keep(i, x) || !in_levels(x) || bucket_of(x, hi, scale) != fb) continue;
        bmin = fminf(bmin, x);
        bmax = fmaxf(bmax, x);
      }
      for (int o = 32; o > 0; o >>= 1) {
        bmin = fminf(bmin, __shfl_xor(bmin, o, 64));
        bmax = fmaxf(bmax, __shfl_xor(bmax, o, 64));
      }
      __syncthreads();
      if (lane == 0) {
        s.wave_f[wave] = bmin;
        s.keys[wave] = __builtin_bit_cast(uint32_t, bmax);
      }
      __syncthreads();
      for (int w = 0; w < kSampWaves; ++w) {
        bmin = fminf(bmin, s.wave_f[w]);
        bmax = fmaxf(bmax, __builtin_bit_cast(float, static_cast<uint32_t>(s.keys[w])));
      }
      __syncthreads();
      if (bmin == bmax) {
        // Equal values: rank order is index order, and every element weighs
        // the same w0. Count, per contiguous index run, the bucket's elements.
        const uint64_t w0 = by_mass ? mass(bmax) : 1;
        const int64_t per = (a.V + kSampThreads - 1) / kSampThreads;
        const int64_t i0 = min(a.V, tid * per), i1 = min(a.V, i0 + per);
        auto member = [&](int64_t i, float x) {
          return x == bmax && keep(i, x) && in_levels(x) && bucket_of(x, hi, scale) == fb;
        };
        uint64_t mine = 0;  // members in this thread's run
        for (int64_t i = i0; i < i1; ++i) mine += member(i, x_at(i)) ? 1 : 0;
        uint64_t incl = mine;
        incl = wave_scan_u64(incl);
        __syncthreads();
        if (lane == 63) s.wave_u64[wave] = incl;
        if (tid == 0) s.found_index = -1;
        __syncthreads();
        uint64_t before = incl - mine;  // members before this run
        for (int w = 0; w < wave; ++w) before += s.wave_u64[w];
        uint64_t cum = base + before * w0;
        for (int64_t i = i0; i < i1; ++i) {
          const float x = x_at(i);
          if (!member(i, x)) continue;
          const uint64_t excl = cum;
          cum += w0;
          if (reached(cum) && (before == 0 || !reached(excl))) {
            s.found_index = i;
            s.found_cum = cum;
            break;
          }
          ++before;
        }
        __syncthreads();
        ri = s.found_index;
        rx = bmax;
        rcum = s.found_cum;
        __syncthreads();
        return ri >= 0;
      }
      if (levels == kMaxLevels) return false;  // distinct values closer than 4 splits resolve: not expected
#pragma unroll
      for (int l = 0; l < kMaxLevels; ++l) {
        if (l == levels) {
          lv_hi[l] = hi;
          lv_scale[l] = scale;
          lv_b[l] = fb;
        }
      }
      ++levels;
      lo = bmin;
      hi = bmax;
    }
  }
};

// The statistics record of segment blockIdx.x of split row blockIdx.y.
template <typename T>
__global__ __launch_bounds__(kSplitThreads) void sample_split_stats(SampleArgs a) {
  const int64_t r = blockIdx.y;
  const int seg = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (!split_row(a, a.temp[r * a.temp_s], load_int(a.topk, a.topk_dt, r * a.topk_s))) return;
  int c0, c1;
  split_range(a, seg, c0, c1);
  const u32x4* r4 = reinterpret_cast<const u32x4*>(static_cast<const T*>(a.logits) + r * a.ls0);
  const int V = static_cast<int>(a.V);
  ChunkStats st;
  st.init(V);
  each_chunk(r4, c0 + tid, c1, kSplitThreads, [&](const u32x4 w, int ch) { st.add<T>(w, ch, V); });
  st.wave_reduce();
  __shared__ SplitStat red[kSplitThreads / 64];
  if (lane == 0) red[wave] = SplitStat{st.mx, st.mn, st.fmn, st.imx, st.imn, st.inan, {0, 0}};
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kSplitThreads / 64; ++w) st.merge(red[w]);
    a.stat[r * a.S + seg] = SplitStat{st.mx, st.mn, st.fmn, st.imx, st.imn, st.inan, {0, 0}};
  }
}

// The merged statistics of split row r (its S records).
__device__ __forceinline__ ChunkStats split_stats(const SampleArgs& a, int64_t r) {
  // Eight records per step, every one loaded (at a clamped segment: merging
  // a record twice changes nothing) before the first merge.
  ChunkStats st;
  st.init(static_cast<int>(a.V));
  for (int w0 = 0; w0 < a.S; w0 += 8) {
    SplitStat rec[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) rec[w] = a.stat[r * a.S + min(w0 + w, a.S - 1)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int w = 0; w < 8; ++w) st.merge(rec[w]);
  }
  return st;
}

// The partial histogram (count and mass per bucket, the buckets and masses
// of RowSampler::fast) of segment blockIdx.x of split row blockIdx.y, for a
// row that reaches the histogram path: no NaN, a finite maximum of x; the
// counts as their exclusive prefix (a.plp). With bucket lists (a.pidx),
// also the segment's elements in bucket order: each element's index
// relative to the segment at its bucket's next place (a counting sort in
// LDS, order within a bucket free), written out whole. sample_tokens_kernel then
// gathers a bucket range from the lists instead of reading the row.
template <typename T>
__global__ __launch_bounds__(kSplitThreads) void sample_split_hist(SampleArgs a) {
  __shared__ uint32_t cnt[kBuckets];
  __shared__ uint64_t msum[kBuckets];
  __shared__ __align__(16) uint16_t list[kSegListMax];
  __shared__ uint32_t wtot[kSplitThreads / 64];
  const int64_t r = blockIdx.y;
  const int seg = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float temp = a.temp[r * a.temp_s];
  if (!split_row(a, temp, load_int(a.topk, a.topk_dt, r * a.topk_s))) return;
  int c0, c1;
  split_range(a, seg, c0, c1);
  const u32x4* r4 = reinterpret_cast<const u32x4*>(static_cast<const T*>(a.logits) + r * a.ls0);
  // With bucket lists the segment (at most kSegListMax elements) is
  // loaded at once, KEEP chunks per thread, before the row's statistics
  // records (which the loads do not need): both arrive in one round trip.
  constexpr int KEEP = (kSegListMax / 8 + kSplitThreads - 1) / kSplitThreads;
  const bool lists = a.pidx != nullptr;
  u32x4 seg_w[KEEP];
  if (lists) {
#pragma unroll
    for (int j = 0; j < KEEP; ++j) {
      const int ch = c0 + tid + j * kSplitThreads;
      seg_w[j] = ch < c1 ? r4[ch] : u32x4{0, 0, 0, 0};
    }
  }
  const ChunkStats st = split_stats(a, r);
  if (seg == 0 && tid == 0) a.mstat[r] = SplitStat{st.mx, st.mn, st.fmn, st.imx, st.imn, st.inan, {0, 0}};
  const float t = fmaxf(temp, 1e-5f);
  if (st.inan < static_cast<int>(a.V) || !(fabsf(__fdiv_rn(st.mx, t)) < INFINITY)) return;  // (uniform)
  const float kmax = st.mx, kc = 1.4426950408889634f / t, lo = fminf(st.fmn, st.mx);
  const float scale = kmax > lo ? static_cast<float>(kBuckets - 1) / (kmax - lo) : 0.f;
  for (int b = tid; b < kBuckets; b += kSplitThreads) {
    cnt[b] = 0;
    msum[b] = 0;
  }
  __syncthreads();
  auto add = [&](const u32x4 w) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float kv = (e & 1) ? hi_f<T>(w[e >> 1]) : lo_f<T>(w[e >> 1]);
      const int b = RowSampler<T, true>::bucket0(kv, kmax, scale);
      atomicAdd(&cnt[b], 1u);
      atomicAdd(reinterpret_cast<unsigned long long*>(&msum[b]),
                static_cast<unsigned long long>(mass_of(kv, kmax, kc)));
    }
  };
  // With bucket lists each element's count atomic returns its place among
  // its bucket's elements in the segment: the thread keeps (bucket << 16 |
  // place) for each of its elements, so the list pass needs neither the
  // logits nor another atomic.
  static_assert(kSegListMax <= 65536 && kBuckets <= 65536, "a bucket and a place share 32 bits");
  uint32_t bp_el[KEEP][8];
  if (lists) {
#pragma unroll
    for (int j = 0; j < KEEP; ++j) {
      if (c0 + tid + j * kSplitThreads >= c1) continue;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float kv = (e & 1) ? hi_f<T>(seg_w[j][e >> 1]) : lo_f<T>(seg_w[j][e >> 1]);
        const int b = RowSampler<T, true>::bucket0(kv, kmax, scale);
        bp_el[j][e] = (static_cast<uint32_t>(b) << 16) | atomicAdd(&cnt[b], 1u);
        atomicAdd(reinterpret_cast<unsigned long long*>(&msum[b]),
                  static_cast<unsigned long long>(mass_of(kv, kmax, kc)));
      }
    }
  } else {
    each_chunk(r4, c0 + tid, c1, kSplitThreads, [&](const u32x4 w, int) { add(w); });
  }
  __syncthreads();
  const size_t base = (static_cast<size_t>(r) * a.S + seg) * kBuckets;
  for (int b = tid; b < kBuckets; b += kSplitThreads) a.pmass[base + b] = msum[b];
  // The counts go out as their exclusive prefix (cnt -> prefix in place: 8
  // buckets per thread, a wave scan of the threads' sums, then the waves'
  // totals): the bucket lists' offsets, and the merge's row prefix without
  // a scan of the counts.
  constexpr int BPT = kBuckets / kSplitThreads;
  uint32_t v[BPT], run = 0;
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    v[i] = cnt[BPT * tid + i];
    run += v[i];
  }
  uint32_t incl = run;
  incl = wave_scan_u32(incl);
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  uint32_t before = incl - run;
  for (int w = 0; w < wave; ++w) before += wtot[w];
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    cnt[BPT * tid + i] = before;
    a.plp[base + BPT * tid + i] = before;
    before += v[i];
  }
  if (!lists) return;
  __syncthreads();
  // Each element's index at its bucket's first place plus its own.
#pragma unroll
  for (int j = 0; j < KEEP; ++j) {
    const int ch = c0 + tid + j * kSplitThreads;
    if (ch >= c1) continue;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      list[cnt[bp_el[j][e] >> 16] + (bp_el[j][e] & 0xFFFFu)] = static_cast<uint16_t>(8 * (ch - c0) + e);
  }
  __syncthreads();
  u32x4* const dst = reinterpret_cast<u32x4*>(a.pidx + (static_cast<size_t>(r) * a.S + seg) * a.segcap);
  const u32x4* const src = reinterpret_cast<const u32x4*>(list);
  for (int i = tid; i < c1 - c0; i += kSplitThreads) dst[i] = src[i];  // 8 indices per 16 bytes
}

template <typename T, bool UNIT>
__global__ __launch_bounds__(kSampThreads) void sample_tokens_kernel(SampleArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  SampleLds& s = *reinterpret_cast<SampleLds*>(lds_raw);
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // (uniform: an SGPR)
  const float temp = a.temp[r * a.temp_s];
  RowSampler<T, UNIT> rs{a, s, static_cast<const T*>(a.logits) + r * a.ls0, fmaxf(temp, 1e-5f), 0.f, tid, lane, wave, 0.f, 0.f};

  // Split rows: their statistics and histogram were made by
  // sample_split_stats and sample_split_hist.
  const bool split = split_row(a, temp, load_int(a.topk, a.topk_dt, r * a.topk_s));

  // Top-k and greedy rows of a 16-bit row that fits the registers: the
  // candidate pass decides from one read of the row, or sends it on.
  if constexpr (UNIT && sizeof(T) == 2) {
    if (!split && a.cand && rs.chunked() && a.V <= kRegMaxV) {
      // The row's parameters are loaded first: loads complete in order, so
      // the test below waits for them alone while the row is in flight.
      const int64_t k = load_int(a.topk, a.topk_dt, r * a.topk_s);
      const float pf = a.topp[r * a.topp_s], uf = a.unif[r * a.unif_s];
      u32x4 ch[kRegChunks];
      rs.load_row(ch);
      if (candidate_row(a, temp, k)) {
        const int64_t token = rs.candidates(ch, temp, k, pf, uf);
        if (token >= 0) {
          if (tid == 0) a.out[r * a.out_s] = token;
          return;
        }
      }
    }
  }

  // Row maximum and its first index (rank 0), the finite minimum, the last
  // index of the minimum (the last rank), and the first NaN.
  // A thread visits its elements in increasing index order, so a strict >
  // keeps the first index of its maximum and <= the last of its minimum.
  float mx = -INFINITY, mn = INFINITY, fmn = INFINITY;
  int imx = static_cast<int>(a.V), imn = -1, inan = static_cast<int>(a.V);
  if (split) {
    // The row's merged statistics record (sample_split_hist's segment 0
    // wrote it), then the partials' merge, which needs none of it: the
    // record's load and the partials' share one round trip.
    const SplitStat st = a.mstat[r];
    rs.srow = r;
    rs.merge_partials();
    mx = st.mx;
    mn = st.mn;
    fmn = st.fmn;
    imx = st.imx;
    imn = st.imn;
    inan = st.inan;
  } else {
    if constexpr (UNIT && sizeof(T) == 2) {
      if (rs.chunked()) {  // per 8-logit chunk: its max and min first, indices only when they win
        const u32x4* r4 = reinterpret_cast<const u32x4*>(rs.row);
        const int V = static_cast<int>(a.V);
        ChunkStats cs;
        cs.init(V);
        each_chunk(r4, tid, V >> 3, kSampThreads, [&](const u32x4 w, int ch) { cs.add<T>(w, ch, V); });
        mx = cs.mx;
        mn = cs.mn;
        fmn = cs.fmn;
        imx = cs.imx;
        imn = cs.imn;
        inan = cs.inan;
      } else {
        rs.each_key([&](int i, float x) {
          if (x > mx) { mx = x; imx = i; }
          if (x <= mn) { mn = x; imn = i; }
          if (x != -INFINITY) fmn = fminf(fmn, x);
          if (x != x) inan = min(inan, i);
        });
      }
    } else {
      rs.each_key([&](int i, float x) {  // x, or for 16-bit logits the logit (same order, same ties)
        if (x > mx) { mx = x; imx = i; }
        if (x <= mn) { mn = x; imn = i; }
        if (x != -INFINITY) fmn = fminf(fmn, x);
        if (x != x) inan = min(inan, i);
      });
    }
    for (int o = 32; o > 0; o >>= 1) {
      const float omx = __shfl_xor(mx, o, 64), omn = __shfl_xor(mn, o, 64), ofm = __shfl_xor(fmn, o, 64);
      const int oimx = __shfl_xor(imx, o, 64), oimn = __shfl_xor(imn, o, 64);
      if (omx > mx || (omx == mx && oimx < imx)) { mx = omx; imx = oimx; }
      if (omn < mn || (omn == mn && oimn > imn)) { mn = omn; imn = oimn; }
      fmn = fminf(fmn, ofm);
      inan = min(inan, __shfl_xor(inan, o, 64));
    }
    __shared__ float red_mx[kSampWaves], red_mn[kSampWaves], red_fm[kSampWaves];
    __shared__ int red_imx[kSampWaves], red_imn[kSampWaves], red_nan[kSampWaves];
    if (lane == 0) {
      red_mx[wave] = mx; red_imx[wave] = imx;
      red_mn[wave] = mn; red_imn[wave] = imn;
      red_fm[wave] = fmn;
      red_nan[wave] = inan;
    }
    __syncthreads();
    for (int w = 0; w < kSampWaves; ++w) {
      if (red_mx[w] > mx || (red_mx[w] == mx && red_imx[w] < imx)) { mx = red_mx[w]; imx = red_imx[w]; }
      if (red_mn[w] < mn || (red_mn[w] == mn && red_imn[w] > imn)) { mn = red_mn[w]; imn = red_imn[w]; }
      fmn = fminf(fmn, red_fm[w]);
      inan = min(inan, red_nan[w]);
    }
  }
  int64_t* out = a.out + r * a.out_s;
  // A row whose softmax is NaN: a NaN logit, a +inf maximum, or every logit
  // -inf. The reference's stable descending sort puts NaN first; its softmax
  // and cumsum are then NaN everywhere, searchsorted of the NaN target
  // returns vocab_size and the clamp makes that the last rank: the last
  // index of the minimum (NaN ignored), or vocab_size - 1 when every logit is
  // NaN. A greedy row still takes rank 0: the first NaN, else the first index
  // of the maximum (0 when every logit is -inf).
  const bool has_nan = inan < static_cast<int>(a.V);
  if (has_nan || !(fabsf(rs.key_to_x(mx)) < INFINITY)) {
    if (tid == 0) {
      if (temp <= 0.f) *out = has_nan ? inan : (imx < static_cast<int>(a.V) ? imx : 0);
      else *out = imn >= 0 ? imn : a.V - 1;
    }
    return;
  }
  if (temp <= 0.f) {  // greedy: rank 0
    if (tid == 0) *out = imx;
    return;
  }
  rs.kmax = mx;
  rs.kc = RowSampler<T, UNIT>::kByLogit ? 1.4426950408889634f / rs.t : 1.4426950408889634f;
  const float klo = fminf(fmn, mx);
  rs.xmax = rs.key_to_x(mx);  // division never decreases, so these are x's maximum and finite minimum
  const float lo0 = rs.key_to_x(klo);
  const int64_t k = load_int(a.topk, a.topk_dt, r * a.topk_s);
  const bool cut_k = k > 0 && k < a.V;
  const double p = a.topp[r * a.topp_s];
  const double u = a.unif[r * a.unif_s];
  int64_t token;
  if (rs.fast(klo, k, cut_k, p, u, token)) {
    if (tid == 0) *out = token;
    return;
  }

  // The per-decision path. top-k: the element at rank k - 1 bounds the kept set.
  float xk = -INFINITY;
  int64_t ik = a.V;
  uint64_t dummy;
  if (cut_k) {
    auto all = [](int64_t, float) { return true; };
    rs.select(all, false, true, false, 0.0, static_cast<double>(k), lo0, rs.xmax, xk, ik, dummy);
  }
  auto keep_k = [&](int64_t i, float x) { return !cut_k || x > xk || (x == xk && i <= ik); };

  // top-p: the first rank whose running mass exceeds top_p * Z is the last
  // kept one (every rank before it has at most top_p before it).
  float xp = -INFINITY;
  int64_t ip = a.V;
  uint64_t kept_mass = 0;
  const float lo1 = cut_k ? fmaxf(lo0, xk) : lo0;
  const bool cut_p = rs.select(keep_k, true, false, true, p, 0.0, lo1, rs.xmax, xp, ip, kept_mass);
  if (!cut_p) {
    uint64_t part = 0;
    for (int i = tid; i < static_cast<int>(a.V); i += kSampThreads) {
      const float x = rs.x_at(i);
      if (keep_k(i, x)) part += rs.mass(x);
    }
    kept_mass = rs.block_sum(part);
  }
  auto keep_kp = [&](int64_t i, float x) {
    return keep_k(i, x) && (!cut_p || x > xp || (x == xp && i <= ip));
  };

  // Inverse-CDF pick: the first kept rank whose running mass reaches u * S.
  float xs;
  int64_t is = -1;
  uint64_t cs;
  const float lo2 = cut_p ? fmaxf(lo1, xp) : lo1;
  const bool ok = rs.select(keep_kp, true, true, false, 0.0, u * static_cast<double>(kept_mass), lo2, rs.xmax, xs,
                            is, cs);
  if (tid == 0) *out = ok ? is : imn;  // past the end: the reference clamps to the last rank
}

}  // namespace tsa

using namespace tsa;

namespace {
// TSA_SAMPLE_CANDIDATES=0 turns the candidate pass off (every row then takes
// the histogram paths; the tokens are the same).
bool candidates_enabled() {
  const char* e = getenv("TSA_SAMPLE_CANDIDATES");
  return !(e && e[0] == '0');
}
}  // namespace

namespace {
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Segments per split row: for a batch too small to fill the device with one
// workgroup per row, about 512 workgroups per pass (0: no split).
int split_segments(int64_t B, int64_t V) {
  if (B <= 0 || B > 256 || V < 16384) return 0;
  const int64_t S = 512 / B;
  return S < 2 ? 0 : static_cast<int>(S > kMaxSegments ? kMaxSegments : S);
}

// Elements per segment of a split row (S segments of whole 8-logit chunks),
// and whether sample_split_hist builds the segments' bucket lists: when a
// segment's list fits its LDS (kSegListMax).
int64_t seg_elems(int64_t V, int S) { return 8 * (((V >> 3) + S - 1) / S); }
bool split_lists(int64_t V, int S) { return S > 1 && seg_elems(V, S) <= kSegListMax; }

// Workspace of a split launch, each region 256-byte aligned: the statistics
// records and each row's merged one, the partial count prefixes and masses,
// and the bucket lists.
struct SplitLayout {
  size_t mstat, plp, pmass, pidx, total;
};
SplitLayout split_layout(int64_t B, int64_t V, int S) {
  const size_t segs = static_cast<size_t>(B) * S;
  SplitLayout l{};
  l.mstat = align256(segs * sizeof(SplitStat));
  l.plp = l.mstat + align256(static_cast<size_t>(B) * sizeof(SplitStat));
  l.pmass = l.plp + align256(segs * kBuckets * sizeof(uint32_t));
  l.pidx = l.pmass + segs * kBuckets * sizeof(uint64_t);
  l.total = l.pidx;
  if (split_lists(V, S)) {
    l.pidx = align256(l.pidx);
    l.total = l.pidx + segs * static_cast<size_t>(seg_elems(V, S)) * sizeof(uint16_t);
  }
  return l;
}
size_t split_bytes(int64_t B, int64_t V, int S) { return S <= 1 ? 0 : split_layout(B, V, S).total; }

int sample_impl(const tsa_view* out, const tsa_view* logits, const tsa_view* temperature, const tsa_view* top_k,
                const tsa_view* top_p, const tsa_view* uniforms, void* workspace, size_t workspace_bytes,
                void* stream) {
  TSA_REQUIRE(view_ok(logits, 2), "Expected logits shape [B, vocab_size]");
  const int64_t B = logits->size[0], V = logits->size[1];
  TSA_REQUIRE(is_float_dtype(logits->dtype), "logits must be bf16, f16 or f32");
  auto vec_ok = [&](const tsa_view* v) { return view_ok(v, 1) && v->size[0] == B; };
  TSA_REQUIRE(vec_ok(temperature) && temperature->dtype == TSA_F32, "Expected temperature shape [%lld] (f32)",
              (long long)B);
  TSA_REQUIRE(vec_ok(top_k) && is_index_dtype(top_k->dtype), "Expected top_k shape [%lld] (i32 or i64)",
              (long long)B);
  TSA_REQUIRE(vec_ok(top_p) && top_p->dtype == TSA_F32, "Expected top_p shape [%lld] (f32)", (long long)B);
  TSA_REQUIRE(vec_ok(uniforms) && uniforms->dtype == TSA_F32, "Expected uniforms shape [%lld] (f32)",
              (long long)B);
  TSA_REQUIRE(vec_ok(out) && out->dtype == TSA_I64, "out must be an int64 tensor of shape [%lld]", (long long)B);
  TSA_REQUIRE(V > 0 && V < (int64_t(1) << 31), "vocab_size must be in [1, 2^31)");
  if (B == 0) return TSA_OK;
  SampleArgs a{};
  a.logits = logits->data; a.ls0 = logits->stride[0]; a.ls1 = logits->stride[1];
  a.B = B; a.V = V;
  a.temp = static_cast<const float*>(temperature->data); a.temp_s = temperature->stride[0];
  a.topk = top_k->data; a.topk_dt = top_k->dtype; a.topk_s = top_k->stride[0];
  a.topp = static_cast<const float*>(top_p->data); a.topp_s = top_p->stride[0];
  a.unif = static_cast<const float*>(uniforms->data); a.unif_s = uniforms->stride[0];
  a.out = static_cast<int64_t*>(out->data); a.out_s = out->stride[0];
  hipStream_t st = static_cast<hipStream_t>(stream);
  a.cand = candidates_enabled() ? 1 : 0;
  // Split rows: 16-bit logits, rows of 16-byte aligned 8-logit chunks, a
  // workspace, and a batch small enough (split_segments).
  const bool rows16 = (logits->dtype == TSA_BF16 || logits->dtype == TSA_F16) && a.ls1 == 1 && (V & 7) == 0 &&
                      (reinterpret_cast<uintptr_t>(logits->data) & 15) == 0 && ((a.ls0 * 2) & 15) == 0;
  const int S = workspace != nullptr && rows16 ? split_segments(B, V) : 0;
  if (S > 1) {
    const size_t need = split_bytes(B, V, S);
    TSA_REQUIRE(workspace_bytes >= need, "workspace too small: %zu bytes, need %zu (tsa_sample_tokens_workspace_bytes)",
                workspace_bytes, need);
    TSA_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "workspace must be 256-byte aligned");
    const SplitLayout l = split_layout(B, V, S);
    char* w = static_cast<char*>(workspace);
    a.stat = reinterpret_cast<SplitStat*>(w);
    a.mstat = reinterpret_cast<SplitStat*>(w + l.mstat);
    a.plp = reinterpret_cast<uint32_t*>(w + l.plp);
    a.pmass = reinterpret_cast<uint64_t*>(w + l.pmass);
    if (split_lists(V, S)) {
      a.pidx = reinterpret_cast<uint16_t*>(w + l.pidx);
      a.segcap = static_cast<int>(seg_elems(V, S));
    }
    a.S = S;
    const dim3 sgrid(S, B);
    if (logits->dtype == TSA_BF16) {
      sample_split_stats<bf16_t><<<sgrid, dim3(kSplitThreads), 0, st>>>(a);
      sample_split_hist<bf16_t><<<sgrid, dim3(kSplitThreads), 0, st>>>(a);
    } else {
      sample_split_stats<f16_t><<<sgrid, dim3(kSplitThreads), 0, st>>>(a);
      sample_split_hist<f16_t><<<sgrid, dim3(kSplitThreads), 0, st>>>(a);
    }
  }
  const size_t lds = sizeof(SampleLds);
  switch (logits->dtype) {
    case TSA_BF16:
      if (a.ls1 == 1) sample_tokens_kernel<bf16_t, true><<<dim3(B), dim3(kSampThreads), lds, st>>>(a);
      else sample_tokens_kernel<bf16_t, false><<<dim3(B), dim3(kSampThreads), lds, st>>>(a);
      break;
    case TSA_F16:
      if (a.ls1 == 1) sample_tokens_kernel<f16_t, true><<<dim3(B), dim3(kSampThreads), lds, st>>>(a);
      else sample_tokens_kernel<f16_t, false><<<dim3(B), dim3(kSampThreads), lds, st>>>(a);
      break;
    default:
      if (a.ls1 == 1) sample_tokens_kernel<float, true><<<dim3(B), dim3(kSampThreads), lds, st>>>(a);
      else sample_tokens_kernel<float, false><<<dim3(B), dim3(kSampThreads), lds, st>>>(a);
      break;
  }
  return check_launch("tsa_sample_tokens");
}
}  // namespace

extern "C" int tsa_sample_tokens(const tsa_view* out, const tsa_view* logits, const tsa_view* temperature,
                                 const tsa_view* top_k, const tsa_view* top_p, const tsa_view* uniforms,
                                 void* stream) {
  return sample_impl(out, logits, temperature, top_k, top_p, uniforms, nullptr, 0, stream);
}

extern "C" size_t tsa_sample_tokens_workspace_bytes(int64_t batch, int64_t vocab) {
  return split_bytes(batch, vocab, split_segments(batch, vocab));
}

extern "C" int tsa_sample_tokens_ws(const tsa_view* out, const tsa_view* logits, const tsa_view* temperature,
                                    const tsa_view* top_k, const tsa_view* top_p, const tsa_view* uniforms,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  return sample_impl(out, logits, temperature, top_k, top_p, uniforms, workspace, workspace_bytes, stream);
}
