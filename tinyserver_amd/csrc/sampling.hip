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
#include <cmath>

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
};

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

struct SampleLds {
  uint32_t cnt[kBuckets];
  uint64_t wsum[kBuckets];  // weight per bucket, then its exclusive prefix
  uint32_t pcnt[kBuckets];   // shared histogram: exclusive prefixes of cnt
  uint64_t pmass[kBuckets];  // and of the masses
  uint64_t keys[kCap];
  uint64_t wave_u64[kSampWaves];
  float wave_f[kSampWaves];
  int64_t wave_i[kSampWaves];
  uint32_t n_gather;
  int found_bucket;
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

  __device__ float logit(int64_t i) const { return to_float(UNIT ? row[static_cast<int>(i)] : row[i * a.ls1]); }
  __device__ float x_at(int64_t i) const { return __fdiv_rn(logit(i), t); }
  // The value the single-histogram path orders by. For 16-bit logits it is
  // the logit itself: distinct 16-bit values differ by at least 2^-8
  // relatively, so dividing them by one t keeps them distinct and in order,
  // and ties in x are exactly ties in the logit. fp32 logits order by x.
  static constexpr bool kByLogit = sizeof(T) == 2;
  __device__ float key_at(int64_t i) const { return kByLogit ? logit(i) : x_at(i); }
  // f(i, key_at(i)) for every element of the row, each thread taking its
  // elements in an order of its own (every use is order-free). A 16-bit row
  // that is 16-byte aligned with a multiple of 8 elements is read 8 logits
  // per lane per load, so each load moves 1 KB per wave and several are in
  // flight; other rows one element at a time.
  __device__ bool chunked() const {
    return UNIT && sizeof(T) == 2 && (reinterpret_cast<uintptr_t>(row) & 15) == 0 && (a.V & 7) == 0;
  }
  // f(i, key) for the elements whose key may lie in [lo, hi]: in a chunked
  // row an 8-logit chunk entirely outside the range is skipped after one
  // comparison (the callers' ranges carry a margin, and f still tests each
  // element exactly); otherwise every element.
  template <typename F>
  __device__ void each_key_in(float lo, float hi, F f) const {
    if constexpr (UNIT && sizeof(T) == 2) {
      if (chunked()) {
        const u32x4* r4 = reinterpret_cast<const u32x4*>(row);
        const int n8 = static_cast<int>(a.V >> 3);
#pragma unroll 8
        for (int ch = tid; ch < n8; ch += kSampThreads) {
          const u32x4 w = r4[ch];
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
          if (cmax < lo || cmin > hi) continue;  // (kByLogit: keys are the logits)
#pragma unroll
          for (int e = 0; e < 8; ++e) f(8 * ch + e, l[e]);
        }
        return;
      }
    }
    each_key(f);
  }
  // The key range that holds buckets [b0, b1] of the shared histogram, with
  // a bucket's width of margin on each side; unbounded where that cannot be
  // said (no spread, or the last bucket, which also takes -inf and NaN).
  __device__ void bucket_range(int b0, int b1, float scale, float& lo, float& hi) const {
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
  __device__ void each_key(F f) const {
    if constexpr (UNIT && sizeof(T) == 2) {
      if (chunked()) {
        const u32x4* r4 = reinterpret_cast<const u32x4*>(row);
        const int n8 = static_cast<int>(a.V >> 3);
#pragma unroll 8
        for (int ch = tid; ch < n8; ch += kSampThreads) {
          const u32x4 w = r4[ch];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float l = (e & 1) ? hi_f<T>(w[e >> 1]) : lo_f<T>(w[e >> 1]);
            f(8 * ch + e, kByLogit ? l : __fdiv_rn(l, t));
          }
        }
        return;
      }
    }
    for (int i = tid; i < static_cast<int>(a.V); i += kSampThreads) f(i, key_at(i));
  }
  __device__ float key_to_x(float k) const { return kByLogit ? __fdiv_rn(k, t) : k; }
  float kmax;  // row maximum of key_at
  float kc;    // log2(e) / t for 16-bit logits, log2(e) for fp32 (keys are x)
  // 2^40 exp(x - xmax) from a key, as exp2((key - kmax) * kc) on v_exp_f32,
  // truncated to an integer in two 32-bit halves (exact: the value has at
  // most 24 significant bits). The single-histogram path's mass; the row
  // maximum weighs exactly 2^40.
  __device__ uint64_t mass_key(float kv) const {
    const float v = fast_exp2((kv - kmax) * kc) * kMassOne;
    const uint32_t hi = static_cast<uint32_t>(v * 2.3283064365386963e-10f);  // v / 2^32
    const uint32_t lo = static_cast<uint32_t>(v - static_cast<float>(hi) * 4294967296.0f);
    return (static_cast<uint64_t>(hi) << 32) | lo;
  }
  __device__ uint64_t mass(float x) const {
    return static_cast<uint64_t>(rintf(expf(x - xmax) * kMassOne));
  }

  // Wave then block sum of a 64-bit value; every thread gets the total.
  __device__ uint64_t block_sum(uint64_t v) {
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
  __device__ void scan_buckets() {
    const uint64_t w0 = s.wsum[2 * tid], w1 = s.wsum[2 * tid + 1];
    uint64_t incl = w0 + w1;
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t up = __shfl_up(incl, o, 64);
      if (lane >= o) incl += up;
    }
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

  // Bitonic sort of s.keys[0, n) ascending, padded to a power of two.
  __device__ void sort_keys(int n) {
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

  __device__ static int bucket0(float x, float h, float sc) {
    if (x == -INFINITY) return kBuckets - 1;
    const float f = (h - x) * sc;
    if (!(f < static_cast<float>(kBuckets - 1))) return kBuckets - 1;  // also NaN: never an index from it
    return f > 0.f ? static_cast<int>(f) : 0;
  }

  // Exclusive prefix over the buckets (two per thread) of in[] into out[].
  template <typename U>
  __device__ void scan2(const U* in, U* out) {
    const U w0 = in[2 * tid], w1 = in[2 * tid + 1];
    uint64_t incl = static_cast<uint64_t>(w0) + w1;
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t up = __shfl_up(incl, o, 64);
      if (lane >= o) incl += up;
    }
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

  // The smallest non-empty bucket b <= last whose running mass through b
  // (the full bucket, or last_incl for bucket `last`) reaches the target.
  __device__ int first_bucket(int last, uint64_t last_incl, bool ge, double target) {
    if (tid == 0) s.found_bucket = kBuckets;
    __syncthreads();
    for (int b = tid; b < kBuckets; b += kSampThreads) {
      if (b > last || s.cnt[b] == 0) continue;
      const double incl = static_cast<double>(b == last ? last_incl : s.pmass[b] + s.wsum[b]);
      if (ge ? incl >= target : incl > target) atomicMin(&s.found_bucket, b);
    }
    __syncthreads();
    const int fb = s.found_bucket;
    __syncthreads();
    return fb;
  }

  // Gathers bucket b of the shared histogram into s.keys in rank order.
  __device__ bool gather_sorted(int b, float scale, int& cached) {
    if (cached == b) return true;
    if (tid == 0) s.n_gather = 0;
    __syncthreads();
    // (a single bucket is a narrow range most chunks straddle: no skipping)
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
  __device__ bool gather_prefix(int nb, float scale) {
    if (tid == 0) s.n_gather = 0;
    __syncthreads();
    float lo, hi;
    bucket_range(0, nb, scale, lo, hi);
    each_key_in(lo, hi, [&](int i, float kv) {
      if (bucket0(kv, kmax, scale) <= nb) {
        const uint32_t at = atomicAdd(&s.n_gather, 1u);
        if (at < kCap) s.keys[at] = rank_key(kv, i);
      }
    });
    __syncthreads();
    if (s.n_gather != s.pcnt[nb] + s.cnt[nb]) return false;  // (never expected)
    sort_keys(static_cast<int>(s.pcnt[nb] + s.cnt[nb]));
    return true;
  }

  // The decisions on the sorted top ranks [0, n): top-k keeps the first
  // lim_k, top-p the ranks through the first whose running mass exceeds
  // p * Z (z: the kept mass when known from the histogram, else summed
  // here), the pick is the first kept rank reaching u * (kept mass).
  __device__ int64_t decide_on_prefix(int n, int lim_k, bool z_known, uint64_t z, double p, double u) {
    uint64_t cum, tot;
    const int lk = lim_k >= 0 ? lim_k : n;
    if (!z_known) {
      scan_sorted(lk, 0, true, -1.0, cum, tot);
      z = tot;
    }
    int lim = lk;
    uint64_t kept = z;
    const int pos_p = scan_sorted(lk, 0, false, p * static_cast<double>(z), cum, tot);
    if (pos_p >= 0) {
      lim = pos_p + 1;
      kept = cum;
    }
    const int pos = scan_sorted(lim, 0, true, u * static_cast<double>(kept), cum, tot);
    if (pos < 0) return -1;
    const int64_t token = static_cast<uint32_t>(s.keys[pos]);
    __syncthreads();
    return token;
  }

  // Over the first `limit` sorted elements, with `base` before them: the
  // position of the one element that reaches the target (see select), its
  // running mass through it, and the mass of all `limit` elements.
  __device__ int scan_sorted(int limit, uint64_t base, bool ge, double target, uint64_t& cum_at, uint64_t& total) {
    const int per = (limit + kSampThreads - 1) / kSampThreads;
    const int e0 = min(limit, tid * per), e1 = min(limit, e0 + per);
    uint64_t mine = 0;
    for (int e = e0; e < e1; ++e) mine += mass_key(key_of_rank(s.keys[e]));  // no reload of the row
    uint64_t incl = mine;
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t up = __shfl_up(incl, o, 64);
      if (lane >= o) incl += up;
    }
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
      if (r && (e == 0 || !rx)) {
        s.found_index = e;
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

  // All three decisions from one histogram of every element (count and
  // mass): each decision's kept set is a prefix in rank order -- full buckets,
  // then a known prefix of one sorted bucket -- so only the buckets where a
  // cut or the pick falls are gathered. False if such a bucket is larger
  // than LDS holds (the caller then runs the per-decision path).
  __device__ bool fast(float lo, int64_t k, bool cut_k, double p, double u, int64_t& token) {
    // lo: the smallest finite key
    const float scale = kmax > lo ? static_cast<float>(kBuckets - 1) / (kmax - lo) : 0.f;
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
    __syncthreads();
    scan2(s.cnt, s.pcnt);
    scan2(s.wsum, s.pmass);
    int cached = -1;
    uint64_t cum, tot;
    // top-k: bucket bk holds rank k - 1; its first need_k sorted elements stay.
    int bk = kBuckets - 1, lim_k = -1;
    uint64_t z = s.pmass[kBuckets - 1] + s.wsum[kBuckets - 1];
    if (cut_k) {
      if (tid == 0) s.found_bucket = kBuckets;
      __syncthreads();
      for (int b = tid; b < kBuckets; b += kSampThreads)
        if (s.cnt[b] > 0 && static_cast<int64_t>(s.pcnt[b]) + s.cnt[b] >= k) atomicMin(&s.found_bucket, b);
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
  __device__ bool select(Keep keep, bool by_mass, bool ge, bool use_frac, double frac, double target_abs,
                         float lo, float hi, float& rx, int64_t& ri, uint64_t& rcum) {
    float lv_hi[kMaxLevels], lv_scale[kMaxLevels];
    int lv_b[kMaxLevels];
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
    auto in_levels = [&](float x) {
      for (int l = 0; l < levels; ++l)
        if (bucket_of(x, lv_hi[l], lv_scale[l]) != lv_b[l]) return false;
      return true;
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
        if (s.cnt[b] > 0 && reached(base + incl)) atomicMin(&s.found_bucket, b);
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
        for (int o = 1; o < 64; o <<= 1) {
          const uint64_t up = __shfl_up(incl, o, 64);
          if (lane >= o) incl += up;
        }
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
        for (int o = 1; o < 64; o <<= 1) {
          const uint64_t up = __shfl_up(incl, o, 64);
          if (lane >= o) incl += up;
        }
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
      lv_hi[levels] = hi;
      lv_scale[levels] = scale;
      lv_b[levels] = fb;
      ++levels;
      lo = bmin;
      hi = bmax;
    }
  }
};

template <typename T, bool UNIT>
__global__ __launch_bounds__(kSampThreads) void sample_tokens_kernel(SampleArgs a) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  SampleLds& s = *reinterpret_cast<SampleLds*>(lds_raw);
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float temp = a.temp[r * a.temp_s];
  RowSampler<T, UNIT> rs{a, s, static_cast<const T*>(a.logits) + r * a.ls0, fmaxf(temp, 1e-5f), 0.f, tid, lane, wave, 0.f, 0.f};

  // Row maximum and its first index (rank 0), the finite minimum, the last
  // index of the minimum (the last rank), and the first NaN.
  // A thread visits its elements in increasing index order, so a strict >
  // keeps the first index of its maximum and <= the last of its minimum.
  float mx = -INFINITY, mn = INFINITY, fmn = INFINITY;
  int imx = static_cast<int>(a.V), imn = -1, inan = static_cast<int>(a.V);
  if constexpr (UNIT && sizeof(T) == 2) {
    if (rs.chunked()) {  // per 8-logit chunk: its max and min first, indices only when they win
      const u32x4* r4 = reinterpret_cast<const u32x4*>(rs.row);
      const int n8 = static_cast<int>(a.V >> 3);
#pragma unroll 8
      for (int ch = tid; ch < n8; ch += kSampThreads) {
        const u32x4 w = r4[ch];
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
        if (cmax != cmax && inan == static_cast<int>(a.V)) {
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

extern "C" int tsa_sample_tokens(const tsa_view* out, const tsa_view* logits, const tsa_view* temperature,
                                 const tsa_view* top_k, const tsa_view* top_p, const tsa_view* uniforms,
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
