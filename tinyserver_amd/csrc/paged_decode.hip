// Paged GQA decode attention for gfx950.
//
// Reference: server/model/kernels/paged_attention.py:8-121. The reference runs
// one program per (sequence, q-head) and walks the block table serially, so
// each K/V page is re-read Hq/Hkv times and a 32k-token context is one long
// serial program. Here:
//
// * One workgroup (4 waves) per (sequence, kv head, context split). Every
//   K/V byte is read once and shared by the G = Hq/Hkv query heads of the
//   group. A split is `tiles_per_split` 16-token tiles; the waves of a
//   workgroup take its tiles round-robin.
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
//   grows, which a wave-uniform branch detects. P is rounded to the cache
//   dtype to feed the MFMA (the reference's P.V is fp32); l sums the fp32 p.
// * Each wave keeps two tiles in registers (ping-pong): the loads of tile
//   i+1 are in flight while tile i is on the matrix cores. Loads are issued
//   unconditionally (the tile index is clamped to the wave's last tile, whose
//   repeat hits the cache) so the compiler can wait for exactly one tile.
// * Split-K: each workgroup merges its waves in LDS; a sequence that fits one
//   split writes its output directly, otherwise each split writes (m, l, acc)
//   to the workspace and a small second kernel merges the splits with a
//   log-sum-exp reduce. The kernel boundary orders the two, so no cache
//   flushes or atomics are needed; no host sync, no memset.
//
// Tokens past seq_len are scored -inf and their V rows zeroed (the
// reference's masked loads, :88-105). seq_len is clamped to the block table's
// capacity and block ids outside [0, num_blocks) read as zeros, so a malformed
// table cannot fault. seq_len == 0 yields NaN, as the reference's 0/0 does.
//
// A generic kernel (one wave per (sequence, q-head), fp32 VALU math) covers
// what the MFMA path does not: fp32 caches, head_dim other than 64/128,
// non-unit innermost strides.
#include <cmath>

#include "tsa_common.h"

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
  int32_t tiles_per_split, max_splits;
  float scale_log2;
  float* ws_o;         // [B][Hq][max_splits][D]
  float* ws_ml;        // [B][Hq][max_splits][2]
};

constexpr int kWaves = 4;
constexpr float kNegInf = -INFINITY;

// Minimum waves per SIMD the split kernel is compiled for (register budget:
// 512 / waves VGPRs per lane), and the number of tiles each wave keeps in
// registers (RING - 1 in flight while one computes).
#ifndef TSA_DECODE_WAVES_PER_EU
#define TSA_DECODE_WAVES_PER_EU 2
#endif
#ifndef TSA_DECODE_RING
#define TSA_DECODE_RING 3
#endif
constexpr int RING = TSA_DECODE_RING;

__device__ __forceinline__ int64_t clamp_len(const DecodeArgs& a, int s) {
  int64_t L = a.seq_lens[s * a.sl_s];
  const int64_t cap = static_cast<int64_t>(a.max_blocks) * a.BS;
  return L < 0 ? 0 : (L > cap ? cap : L);
}

template <typename T, int D, bool PAGE16, bool CONTIG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TSA_DECODE_WAVES_PER_EU)))
void paged_decode_mfma(DecodeArgs a) {
  constexpr int KJ = D / 32;  // k-steps of the score MFMA
  extern __shared__ float lds[];
  // Workgroups are numbered kv-head fastest, then sequence, then split. The
  // hardware deals consecutive workgroup ids to the 8 XCDs round-robin, so
  // every XCD gets an even share of each split index (split-major order would
  // leave the XCDs that draw the late, mostly empty splits idle), and the
  // always-populated first splits are dispatched first.
  const int id = blockIdx.x;
  const int kvh = id % a.Hkv;
  const int s = (id / a.Hkv) % a.B;
  const int split = id / (a.Hkv * a.B);
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
  // Wave-uniform (scalar) so tile indices, block-table reads and page bases
  // stay in SGPRs and the table lookups are scalar loads.
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = a.G;
  const int64_t L = clamp_len(a, s);
  const int ntiles = static_cast<int>((L + 15) >> 4);
  const int nsplit = (ntiles + a.tiles_per_split - 1) / a.tiles_per_split;

  if (split >= nsplit) {
    if (L == 0 && split == 0) {  // empty sequence: 0/0 like the reference
      for (int idx = tid; idx < G * D; idx += 256) {
        T* o = static_cast<T*>(a.out) + s * a.o_ss + (kvh * G + idx / D) * a.o_sh + (idx % D);
        *o = from_float<T>(NAN);
      }
    }
    return;
  }
  const int t_begin = split * a.tiles_per_split;
  const int t_end = min(ntiles, t_begin + a.tiles_per_split);

  // Q^T operand: lane (g, c) holds head c, dims 8(g + 4j)..+8 for k-step j.
  u32x4 qop[KJ];
  {
    const T* qrow = static_cast<const T*>(a.q) + s * a.q_ss + (kvh * G + c) * a.q_sh;
#pragma unroll
    for (int j = 0; j < KJ; ++j)
      qop[j] = c < G ? *reinterpret_cast<const u32x4*>(qrow + 8 * (g + 4 * j)) : u32x4{0, 0, 0, 0};
  }

  const int32_t* bt_row = a.bt + s * a.bt_s0;
  const T* kbase = static_cast<const T*>(a.kc) + kvh * a.kc_h;
  const T* vbase = static_cast<const T*>(a.vc) + kvh * a.vc_h;
  const bool v_lane = 8 * c < D;

  auto page_of = [&](int64_t tok, int64_t& phys, int64_t& slot) -> bool {
    const int64_t lb = tok / a.BS;
    phys = bt_row[lb * a.bt_s1];
    slot = tok - lb * a.BS;
    return phys >= 0 && phys < a.NB;
  };

  // Slot strides: the contiguous pool layout makes them the compile-time D.
  const int64_t ks = CONTIG ? D : a.kc_s;
  const int64_t vs = CONTIG ? D : a.vc_s;

  // K operand (token c of the tile) and V rows (tokens 4g..4g+3) of one tile.
  // With 16-token pages the whole tile is one page: the loads are
  // unconditional (an invalid page id reads page 0 and the tile is masked in
  // compute_tile), so nothing waits on the data until it is consumed.
  auto load_tile = [&](int t, u32x4 (&ko)[KJ], u32x4 (&vo)[4]) {
    const int64_t tok0 = static_cast<int64_t>(t) * 16;
    if constexpr (PAGE16) {
      int64_t phys, slot0;
      if (!page_of(tok0, phys, slot0)) phys = 0;
      const T* kp = kbase + phys * a.kc_b + (slot0 + c) * ks + 8 * g;
#pragma unroll
      for (int j = 0; j < KJ; ++j) ko[j] = *reinterpret_cast<const u32x4*>(kp + 32 * j);
      const T* vp = vbase + phys * a.vc_b + (slot0 + 4 * g) * vs + (v_lane ? 8 * c : 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) vo[r] = *reinterpret_cast<const u32x4*>(vp + r * vs);
    } else {
      int64_t phys, slot;
      const int64_t tk = tok0 + c;
      const bool okk = tk < L && page_of(tk, phys, slot);
      const T* kp = kbase + (okk ? phys * a.kc_b + slot * ks : 0);
#pragma unroll
      for (int j = 0; j < KJ; ++j)
        ko[j] = okk ? *reinterpret_cast<const u32x4*>(kp + 8 * (g + 4 * j)) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t tv = tok0 + 4 * g + r;
        const bool okv = v_lane && tv < L && page_of(tv, phys, slot);
        vo[r] = okv ? *reinterpret_cast<const u32x4*>(vbase + phys * a.vc_b + slot * vs + 8 * c)
                    : u32x4{0, 0, 0, 0};
      }
    }
  };

  float m = kNegInf;  // running max of head c (log2 domain), same in all 4 row-groups
  float l = 0.f;      // this lane's share of head c's softmax denominator
  f32x4 acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute_tile = [&](int t, const u32x4 (&ko)[KJ], u32x4 (&vo)[4]) {
    const int64_t tok0 = static_cast<int64_t>(t) * 16;
    // Tokens past seq_len, and (page-16 path) tiles whose block id is out of
    // range, are masked: score -inf and V rows zeroed so 0 * (inf/nan) cannot
    // leak into the accumulator. Only the last tile of a sequence (or a bad
    // page) takes this wave-uniform branch.
    int64_t lim = L;
    if constexpr (PAGE16) {
      int64_t phys, slot0;
      if (!page_of(tok0, phys, slot0)) lim = tok0;
    }
    if (tok0 + 16 > lim) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (tok0 + 4 * g + r >= lim) vo[r] = u32x4{0, 0, 0, 0};
    }
    f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KJ; ++j) sc = mfma_k32<T>(ko[j], qop[j], sc);
    // sc[r] = q_c . k_{tok0 + 4g + r}
    const int64_t tb = tok0 + 4 * g;
    float sv[4];
    float tmax = kNegInf;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sv[r] = tb + r < lim ? sc[r] * a.scale_log2 : kNegInf;
      tmax = fmaxf(tmax, sv[r]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m, tmax);
    if (__any(m_new > m)) {
      const float alpha = fast_exp2(m - m_new);  // 0 on the first tile (m = -inf)
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
      p[r] = fast_exp2(sv[r] - m);
      l += p[r];
    }
    const u32x2 pop = u32x2{pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3])};
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int w = u >> 1;
      u32x2 bop;
      if (u & 1) {
        bop[0] = pack_hi(vo[0][w], vo[1][w]);
        bop[1] = pack_hi(vo[2][w], vo[3][w]);
      } else {
        bop[0] = pack_lo(vo[0][w], vo[1][w]);
        bop[1] = pack_lo(vo[2][w], vo[3][w]);
      }
      acc[u] = mfma_k16<T>(pop, bop, acc[u]);  // acc[u][r] = O[head 4g + r][dim 8c + u]
    }
  };

  // Ring of RING tile buffers over this wave's tiles t_begin + wave + 4i,
  // i < nw: while one tile is on the matrix cores the loads of the next
  // RING-1 are in flight. The scheduling barriers keep every buffer's loads in
  // ring order on all paths, so a compute waits for its own tile only.
  const int first = t_begin + wave;
  const int nw = first < t_end ? (t_end - first + kWaves - 1) / kWaves : 0;
  if (nw > 0) {
    auto tile = [&](int i) { return first + kWaves * min(i, nw - 1); };
    u32x4 kbuf[RING][KJ], vbuf[RING][4];
#pragma unroll
    for (int d = 0; d < RING; ++d) {
      load_tile(tile(d), kbuf[d], vbuf[d]);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int i = 0; i < nw; i += RING) {
#pragma unroll
      for (int d = 0; d < RING; ++d) {
        if (i + d < nw) compute_tile(tile(i + d), kbuf[d], vbuf[d]);
        __builtin_amdgcn_sched_barrier(0);
        load_tile(tile(i + d + RING), kbuf[d], vbuf[d]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // Head c's denominator: sum the four row-groups.
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);

  // Merge the waves through LDS: [wave][head][D] acc, then [wave][head] m and l.
  float* s_o = lds;
  float* s_m = lds + kWaves * G * D;
  float* s_l = s_m + kWaves * G;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int hd = 4 * g + r;
    if (hd < G && v_lane) {
#pragma unroll
      for (int u = 0; u < 8; ++u) s_o[(wave * G + hd) * D + 8 * c + u] = acc[u][r];
    }
  }
  if (g == 0 && c < G) {
    s_m[wave * G + c] = m;
    s_l[wave * G + c] = l;
  }
  __syncthreads();

  const int64_t head0 = static_cast<int64_t>(s) * a.Hq + kvh * G;  // row of (s, first head of the group)
  for (int idx = tid; idx < G * D; idx += 256) {
    const int hd = idx / D, d = idx - hd * D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w * G + hd]);
    float o = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float e = fast_exp2(s_m[w * G + hd] - M);
      o += e * s_o[(w * G + hd) * D + d];
      den += e * s_l[w * G + hd];
    }
    if (nsplit == 1) {
      T* op = static_cast<T*>(a.out) + s * a.o_ss + (kvh * G + hd) * a.o_sh + d * a.o_sd;
      *op = from_float<T>(o / den);
    } else {
      const int64_t slot = (head0 + hd) * a.max_splits + split;
      a.ws_o[slot * D + d] = o;
      if (d == 0) {
        a.ws_ml[slot * 2] = M;
        a.ws_ml[slot * 2 + 1] = den;
      }
    }
  }
}

// Merge the splits of one (sequence, kv head): out = sum_s 2^(m_s - M) acc_s /
// sum_s 2^(m_s - M) l_s. Sequences that fit one split were written directly.
template <typename T>
__global__ __launch_bounds__(256) void paged_decode_merge(DecodeArgs a) {
  const int kvh = blockIdx.x, s = blockIdx.y, tid = threadIdx.x;
  const int G = a.G, D = a.D;
  const int64_t L = clamp_len(a, s);
  const int ntiles = static_cast<int>((L + 15) >> 4);
  const int nsplit = (ntiles + a.tiles_per_split - 1) / a.tiles_per_split;
  if (nsplit <= 1) return;
  const int64_t head0 = static_cast<int64_t>(s) * a.Hq + kvh * G;
  for (int idx = tid; idx < G * D; idx += 256) {
    const int hd = idx / D, d = idx - hd * D;
    const int64_t base = (head0 + hd) * a.max_splits;
    float M = kNegInf;
    for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, a.ws_ml[(base + sp) * 2]);
    float o = 0.f, den = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) {
      const float e = fast_exp2(a.ws_ml[(base + sp) * 2] - M);
      o += e * a.ws_o[(base + sp) * D + d];
      den += e * a.ws_ml[(base + sp) * 2 + 1];
    }
    T* op = static_cast<T*>(a.out) + s * a.o_ss + (kvh * G + hd) * a.o_sh + d * a.o_sd;
    *op = from_float<T>(o / den);
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
      float dot = 0.f;
      if (phys >= 0 && phys < a.NB) {
        const T* kr = kbase + phys * a.kc_b + slot * a.kc_s;
        for (int d = 0; d < D; ++d) dot += to_float(qrow[d * a.q_sd]) * to_float(kr[d * a.kc_d]);
      }
      sc = dot * a.scale_log2;
    }
    float cmax = sc;
    for (int off = 32; off >= 1; off >>= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, off, 64));
    const float m_new = fmaxf(m, cmax);
    const float alpha = fast_exp2(m - m_new);
    const float p = fast_exp2(sc - m_new);
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

struct DecodePlan {
  int tiles_per_split;
  int max_splits;
  size_t ws_o_bytes, ws_ml_bytes, total;
};

static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

static DecodePlan make_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_blocks, int64_t BS,
                            int32_t tiles_per_split) {
  DecodePlan p{};
  const int64_t max_tiles = (max_blocks * BS + 15) / 16;
  int64_t tps = tiles_per_split;
  if (tps <= 0) {
    // Aim for ~4096 workgroup slots over the longest sequence's tiles.
    const int64_t units = B * Hkv;
    tps = (units * max_tiles + 4095) / 4096;
    if (tps < 8) tps = 8;
  }
  tps = (tps + kWaves - 1) / kWaves * kWaves;
  if (tps > 1 << 20) tps = 1 << 20;
  p.tiles_per_split = static_cast<int>(tps);
  p.max_splits = static_cast<int>(max_tiles > 0 ? (max_tiles + tps - 1) / tps : 1);
  if (p.max_splits < 1) p.max_splits = 1;
  if (p.max_splits > 1) {
    p.ws_o_bytes = align256(static_cast<size_t>(B * Hq) * p.max_splits * D * sizeof(float));
    p.ws_ml_bytes = align256(static_cast<size_t>(B * Hq) * p.max_splits * 2 * sizeof(float));
  }
  p.total = p.ws_o_bytes + p.ws_ml_bytes;
  return p;
}

template <typename T>
static int launch_decode(DecodeArgs& a, bool mfma, hipStream_t stream) {
  if (a.B == 0 || a.Hq == 0) return TSA_OK;
  if (!mfma) {
    paged_decode_generic<T><<<dim3(a.Hq, a.B), dim3(64), 0, stream>>>(a);
    return check_launch("tsa_paged_decode");
  }
  if constexpr (sizeof(T) == 2) {
    const dim3 grid(static_cast<uint32_t>(a.max_splits) * a.Hkv * a.B);
    const size_t lds = static_cast<size_t>(kWaves) * a.G * (a.D + 2) * sizeof(float);
    const bool page16 = a.BS % 16 == 0;
    const bool contig = a.kc_s == a.D && a.vc_s == a.D;
#define TSA_DECODE_LAUNCH(DD, P16, CT) \
  paged_decode_mfma<T, DD, P16, CT><<<grid, dim3(256), lds, stream>>>(a)
    if (a.D == 128) {
      if (page16 && contig) TSA_DECODE_LAUNCH(128, true, true);
      else if (page16) TSA_DECODE_LAUNCH(128, true, false);
      else TSA_DECODE_LAUNCH(128, false, false);
    } else {
      if (page16 && contig) TSA_DECODE_LAUNCH(64, true, true);
      else if (page16) TSA_DECODE_LAUNCH(64, true, false);
      else TSA_DECODE_LAUNCH(64, false, false);
    }
#undef TSA_DECODE_LAUNCH
    if (a.max_splits > 1) {
      if (int rc = check_launch("tsa_paged_decode")) return rc;
      paged_decode_merge<T><<<dim3(a.Hkv, a.B), dim3(256), 0, stream>>>(a);
    }
  }
  return check_launch("tsa_paged_decode");
}

}  // namespace tsa

using namespace tsa;

extern "C" size_t tsa_paged_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads,
                                                   int64_t head_dim, int64_t max_blocks_per_seq, int64_t block_size,
                                                   int32_t tiles_per_split) {
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0) return 0;
  return make_plan(num_seqs, num_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size, tiles_per_split).total;
}

extern "C" int tsa_paged_decode(const tsa_view* out, const tsa_view* query, const tsa_view* k_cache,
                                const tsa_view* v_cache, const tsa_view* block_tables, const tsa_view* seq_lens,
                                double softmax_scale, void* workspace, size_t workspace_bytes,
                                int32_t tiles_per_split, void* stream) {
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
  TSA_UNSUPPORTED(D <= 512, "head_dim %lld > 512 is not implemented", (long long)D);

  DecodeArgs a{};
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

  const bool mfma = (dt == TSA_BF16 || dt == TSA_F16) && (D == 64 || D == 128) && a.G <= 16 &&
                    rows_vec16(query) && rows_vec16(k_cache) && rows_vec16(v_cache) && out->stride[2] == 1;
  if (mfma) {
    const DecodePlan plan = make_plan(B, Hq, Hkv, D, a.max_blocks, BS, tiles_per_split);
    a.tiles_per_split = plan.tiles_per_split;
    a.max_splits = plan.max_splits;
    TSA_REQUIRE(plan.max_splits < 65536, "context too long for one launch (%d splits)", plan.max_splits);
    if (plan.total > 0) {
      TSA_REQUIRE(workspace != nullptr && workspace_bytes >= plan.total,
                  "workspace of %zu bytes is too small: %zu needed", workspace_bytes, plan.total);
      TSA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-byte aligned");
      char* w = static_cast<char*>(workspace);
      a.ws_o = reinterpret_cast<float*>(w);
      a.ws_ml = reinterpret_cast<float*>(w + plan.ws_o_bytes);
    }
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dt) {
    case TSA_BF16: return launch_decode<bf16_t>(a, mfma, st);
    case TSA_F16: return launch_decode<f16_t>(a, mfma, st);
    case TSA_F32: return launch_decode<float>(a, false, st);
  }
  set_error("unsupported dtype");
  return TSA_ERR_UNSUPPORTED;
}
