// Fused Qwen3 per-head QK RMSNorm + rotate-half RoPE (+ optional paged K/V
// store).
//
// Replaces the eager sequence at server/model/patches/qwen3.py:268-287:
// q_norm/k_norm (transformers models/qwen3/modeling_qwen3.py:59-64) followed by
// apply_rotary_pos_emb (modeling_qwen3.py:140-170), about 15 element-wise
// launches per tensor, with one pass over q and k. The rounding points are
// HF's, in the model dtype T:
//   y   = T(x * (1 / sqrt(mean(x^2) + eps)))      statistics in fp32
//   z   = T(w * y)
//   out = T( T(z * cos) + T(rotate_half(z) * sin) )
// where rotate_half(z)_i = -z_{i+D/2} for i < D/2 and z_{i-D/2} otherwise.
// Products of two 16-bit values are exact in fp32, so every T(.) above is a
// single rounding exactly as torch does it; fp32 arithmetic uses the _rn
// intrinsics so no multiply-add is contracted across a rounding point.
//
// Layout (the per-row and per-token kernels): one lane owns 8 consecutive
// elements of a (token, head) row, so a D=128 row is 16 lanes and the RoPE
// partner elements (i +- D/2) sit in lane c ^ (D/16), one cross-lane exchange
// away. The 16-bit head-dim-128 kernel (qk_norm_rope_rows8) gives a lane 16
// elements, dims d and d + 64, so a row is 8 lanes and the partner is local. Rows are ordered token-major
// (all Hq + Hkv heads of a token are adjacent) so a token's cos/sin and its
// block-table lookup are shared by neighbouring lanes.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "kv_store.h"
#include "norm_rope_row.h"

namespace tsa {

template <typename T>
struct NormRopeArgs {
  const T* q; const T* k;
  T* q_out; T* k_out;
  const T* qw; const T* kw;
  const T* cos; const T* sin;
  const T* v;                 // raw V rows, (T, Hkv, D); only when storing
  int64_t q_st, q_sh, q_sd, k_st, k_sh, k_sd;
  int64_t qo_st, qo_sh, qo_sd, ko_st, ko_sh, ko_sd;
  int64_t qw_s, kw_s, cos_st, cos_sd, sin_st, sin_sd;
  int64_t v_st, v_sh, v_sd;
  int64_t T_, Hq, Hkv;
  float eps;
  // Paged store target (k_cache == nullptr: no store).
  T* k_cache; T* v_cache;
  int64_t kc_b, kc_h, kc_s, kc_d, vc_b, vc_h, vc_s, vc_d, NB, BS;
  PagedAddr addr;
};

template <typename T, bool VEC>
__device__ __forceinline__ void load8(const T* p, int64_t stride, float (&out)[8]) {
  if constexpr (VEC && sizeof(T) == 2) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = lo_f<T>(w[i]);
      out[2 * i + 1] = hi_f<T>(w[i]);
    }
  } else if constexpr (VEC) {
    const f32x4 a = reinterpret_cast<const f32x4*>(p)[0];
    const f32x4 b = reinterpret_cast<const f32x4*>(p)[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) { out[i] = a[i]; out[4 + i] = b[i]; }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = to_float(p[i * stride]);
  }
}

// Values are already representable in T, so the conversion here is exact.
// Unit-stride 8-element row chunk with non-temporal loads / stores: for data
// read or written once whose lines are not wanted in the caches afterwards.
template <typename T>
__device__ __forceinline__ void load8_nt(const T* p, float (&out)[8]) {
  if constexpr (sizeof(T) == 2) {
    const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = lo_f<T>(w[i]);
      out[2 * i + 1] = hi_f<T>(w[i]);
    }
  } else {
    const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) { out[i] = a[i]; out[4 + i] = b[i]; }
  }
}
template <typename T>
__device__ __forceinline__ void store8_nt(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack2<T>(v[2 * i], v[2 * i + 1]);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
  } else {
    f32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) { a[i] = v[i]; b[i] = v[4 + i]; }
    __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(p));
    __builtin_nontemporal_store(b, reinterpret_cast<f32x4*>(p) + 1);
  }
}

// 8 elements copied as they are (16 bytes of a 16-bit type, 32 of fp32),
// non-temporal both ways.
template <typename T>
struct RawRow {
  u32x4 w[sizeof(T) / 2];
};
template <typename T>
__device__ __forceinline__ RawRow<T> load_raw_nt(const T* p) {
  RawRow<T> r;
#pragma unroll
  for (int i = 0; i < static_cast<int>(sizeof(T) / 2); ++i)
    r.w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + i);
  return r;
}
template <typename T>
__device__ __forceinline__ void store_raw_nt(T* p, const RawRow<T>& r) {
#pragma unroll
  for (int i = 0; i < static_cast<int>(sizeof(T) / 2); ++i)
    __builtin_nontemporal_store(r.w[i], reinterpret_cast<u32x4*>(p) + i);
}

template <typename T, bool VEC>
__device__ __forceinline__ void store8(T* p, int64_t stride, const float (&v)[8]) {
  if constexpr (VEC && sizeof(T) == 2) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack2<T>(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4*>(p) = w;
  } else if constexpr (VEC) {
    f32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) { a[i] = v[i]; b[i] = v[4 + i]; }
    reinterpret_cast<f32x4*>(p)[0] = a;
    reinterpret_cast<f32x4*>(p)[1] = b;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i * stride] = from_float<T>(v[i]);
  }
}


// One lane per 8 elements of a (token, head) row; rows are token-major. With
// IDX32 (the host has checked every offset fits) the index arithmetic is
// 32-bit, which is most of this kernel's integer work.
template <typename T, int D, bool VEC, bool IDX32>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(NormRopeArgs<T> a) {
  typedef typename std::conditional<IDX32, int32_t, int64_t>::type I;
  constexpr int LANES = D / 8;  // lanes per (token, head) row
  constexpr int ROWS = 256 / LANES;
  const int lane_in_row = threadIdx.x % LANES;
  const I heads = static_cast<I>(a.Hq + a.Hkv);
  const I row = static_cast<I>(blockIdx.x) * ROWS + static_cast<I>(threadIdx.x / LANES);
  const bool live = row < static_cast<I>(a.T_) * heads;
  // Dead lanes still join the cross-lane exchanges below (they read row 0).
  const I r = live ? row : 0;
  const I t = IDX32 ? static_cast<I>(static_cast<uint32_t>(r) / static_cast<uint32_t>(heads)) : r / heads;
  const I hh = r - t * heads;
  const bool is_k = hh >= static_cast<I>(a.Hq);
  const I h = is_k ? hh - static_cast<I>(a.Hq) : hh;
  const int d0 = lane_in_row * 8;

  const T* src = is_k ? a.k + (t * static_cast<I>(a.k_st) + h * static_cast<I>(a.k_sh) + d0 * static_cast<I>(a.k_sd))
                      : a.q + (t * static_cast<I>(a.q_st) + h * static_cast<I>(a.q_sh) + d0 * static_cast<I>(a.q_sd));
  const T* w = is_k ? a.kw + d0 * a.kw_s : a.qw + d0 * a.qw_s;
  float x[8], wf[8], cs[8], sn[8], vv[8];
  load8<T, VEC>(src, is_k ? a.k_sd : a.q_sd, x);
  load8<T, VEC>(w, is_k ? a.kw_s : a.qw_s, wf);
  load8<T, VEC>(a.cos + (t * static_cast<I>(a.cos_st) + d0 * static_cast<I>(a.cos_sd)), a.cos_sd, cs);
  load8<T, VEC>(a.sin + (t * static_cast<I>(a.sin_st) + d0 * static_cast<I>(a.sin_sd)), a.sin_sd, sn);
  // A stored k row: its V row and its cache slot are fetched before the math.
  const bool store = a.k_cache != nullptr && is_k && live;
  int64_t blk = 0, slot = 0;
  bool placed = false;
  if (store) {
    load8<T, VEC>(a.v + (t * static_cast<I>(a.v_st) + h * static_cast<I>(a.v_sh) + d0 * static_cast<I>(a.v_sd)), a.v_sd,
                  vv);
    placed = a.addr.locate(t, a.BS, a.NB, blk, slot);
  }

  float o[8];
  norm_rope_row<T, D>(x, wf, cs, sn, a.eps, lane_in_row, o);
  if (!live) return;

  if (!is_k) {
    store8<T, VEC>(a.q_out + (t * static_cast<I>(a.qo_st) + h * static_cast<I>(a.qo_sh) + d0 * static_cast<I>(a.qo_sd)),
                   a.qo_sd, o);
    return;
  }
  if (a.k_out)
    store8<T, VEC>(a.k_out + (t * static_cast<I>(a.ko_st) + h * static_cast<I>(a.ko_sh) + d0 * static_cast<I>(a.ko_sd)),
                   a.ko_sd, o);
  if (placed) {
    store8<T, VEC>(a.k_cache + blk * a.kc_b + h * a.kc_h + slot * a.kc_s + d0 * a.kc_d, a.kc_d, o);
    store8<T, VEC>(a.v_cache + blk * a.vc_b + h * a.vc_h + slot * a.vc_s + d0 * a.vc_d, a.vc_d, vv);
  }
}

static bool vec_ok(const tsa_view* v) { return v == nullptr || v->data == nullptr || rows_vec16(v); }

// Head-dim-128 path for fp32 (and for 16-bit types whose head strides do not
// fit the 8-lanes-per-row kernel's int offsets): one workgroup per token, 16
// groups of 16 lanes; group g takes the token's rows (heads, q first then k)
// g, g + 16, ..., at most R of them. The token is workgroup-uniform, so its cos/sin are loaded once per
// lane and its cache slot is found with scalar loads, and the rows of a lane
// differ only by a head stride. The q/k/v rows are read once and the cache
// rows are not read back here, so those go non-temporal; the rotated q and k
// stay ordinary stores (the attention reads them next). One short-lived
// workgroup per token keeps more loads in flight than resident workgroups
// walking the tokens with a prefetch (measured 109 vs 157 us at 17794 tokens).
template <typename T, int R>
__global__ __launch_bounds__(256) void qk_norm_rope_token(NormRopeArgs<T> a) {
  constexpr int D = 128;
  const int t = blockIdx.x;
  const int g = threadIdx.x >> 4, c = threadIdx.x & 15, d0 = 8 * c;
  const int Hq = static_cast<int>(a.Hq), H = static_cast<int>(a.Hq + a.Hkv);
  float qwf[8], kwf[8], cs[8], sn[8];
  load8<T, true>(a.qw + d0, 1, qwf);
  load8<T, true>(a.kw + d0, 1, kwf);
  load8<T, true>(a.cos + t * a.cos_st + d0, 1, cs);
  load8<T, true>(a.sin + t * a.sin_st + d0, 1, sn);
  const T* qrow = a.q + t * a.q_st + d0;
  const T* krow = a.k + t * a.k_st + d0;
  const T* vrow = a.v + t * a.v_st + d0;
  const bool store = a.k_cache != nullptr;

  // Every row load is issued before anything waits on one: q/k rows by an
  // address select, v rows (when storing) for each round that holds a k
  // head (a q lane of such a round reads v head 0's row and drops it). No
  // load sits in a divergent branch, whose join would wait for all of them.
  float x[R][8];
  RawRow<T> vv[R];  // (copied to the cache as read)
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int hh = min(g + 16 * j, H - 1);  // rows past the token's last head redo it (never stored)
    load8_nt<T>(hh < Hq ? qrow + hh * a.q_sh : krow + (hh - Hq) * a.k_sh, x[j]);
    if (store && 16 * j + 15 >= Hq) vv[j] = load_raw_nt<T>(vrow + max(hh - Hq, 0) * a.v_sh);  // (uniform test)
  }
  // The token's cache slot: scalar loads, while the rows are in flight.
  int64_t blk = 0, slot = 0;
  const bool placed = store && a.addr.locate(t, a.BS, a.NB, blk, slot);
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int hh = g + 16 * j;
    const bool is_k = hh >= Hq;
    float o[8];
    norm_rope_row<T, D>(x[j], is_k ? kwf : qwf, cs, sn, a.eps, c, o);
    if (hh >= H) continue;
    if (!is_k) {
      store8<T, true>(a.q_out + t * a.qo_st + hh * a.qo_sh + d0, 1, o);
      continue;
    }
    const int h = hh - Hq;
    if (a.k_out) store8<T, true>(a.k_out + t * a.ko_st + h * a.ko_sh + d0, 1, o);
    if (placed) {
      store8_nt<T>(a.k_cache + blk * a.kc_b + h * a.kc_h + slot * a.kc_s + d0, o);
      store_raw_nt<T>(a.v_cache + blk * a.vc_b + h * a.vc_h + slot * a.vc_s + d0, vv[j]);
    }
  }
}

// Head-dim-128 path for 16-bit types: one workgroup per token and 8 lanes
// per (token, head) row, 8*H lanes for a token's H = Hq + Hkv rows (q first,
// then k), rounded up to whole waves. Lane c of a row holds dims 8c..8c+7
// and 64+8c..64+8c+7 (norm_rope_row_d128x8), so no row needs a second pass
// and a wave's VALU work serves 8 rows. The token is workgroup-uniform: its
// cos/sin rows, its cache slot (scalar loads) and the scalar part of every
// address are shared, and the per-lane part is a head offset the host has
// checked fits 32 bits. Q/K/V rows are read once and the cache rows are not
// read back here, so those go non-temporal; the rotated q and k stay
// ordinary stores (the attention reads them next).
template <typename T>
__global__ __launch_bounds__(1024) void qk_norm_rope_rows8(NormRopeArgs<T> a) {
  const int t = blockIdx.x;
  const int Hq = static_cast<int>(a.Hq), H = static_cast<int>(a.Hq + a.Hkv);
  const int r = threadIdx.x >> 3, c = threadIdx.x & 7;
  const int hh = min(r, H - 1);  // lanes past the last row redo it (never stored)
  const bool is_k = hh >= Hq;
  const int h = is_k ? hh - Hq : hh;
  const int d0 = 8 * c;
  const bool store = a.k_cache != nullptr;

  const T* src = is_k ? a.k + t * a.k_st + (h * static_cast<int>(a.k_sh) + d0)
                      : a.q + t * a.q_st + (h * static_cast<int>(a.q_sh) + d0);
  const T* w = (is_k ? a.kw : a.qw) + d0;
  const T* cs = a.cos + t * a.cos_st + d0;
  const T* sn = a.sin + t * a.sin_st + d0;
  u32x4 xp[2], wp[2], cp[2], sp[2];
  RawRow<T> vv[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    xp[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + 64 * j));
    wp[j] = *reinterpret_cast<const u32x4*>(w + 64 * j);
    cp[j] = *reinterpret_cast<const u32x4*>(cs + 64 * j);
    sp[j] = *reinterpret_cast<const u32x4*>(sn + 64 * j);
  }
  const T* vrow = a.v + t * a.v_st + (max(hh - Hq, 0) * static_cast<int>(a.v_sh) + d0);
  if (store && is_k) {
#pragma unroll
    for (int j = 0; j < 2; ++j) vv[j] = load_raw_nt<T>(vrow + 64 * j);
  }
  // The token's cache slot (scalar loads, while the rows are in flight), in
  // the waves that hold a k row.
  int64_t blk = 0, slot = 0;
  const bool placed =
      store && __builtin_amdgcn_ballot_w64(is_k) != 0 && a.addr.locate(t, a.BS, a.NB, blk, slot);

  u32x4 op[2];
  norm_rope_row_d128x8<T>(xp, wp, cp, sp, a.eps, op);
  if (r >= H) return;
  if (!is_k) {
    T* dst = a.q_out + t * a.qo_st + (h * static_cast<int>(a.qo_sh) + d0);
#pragma unroll
    for (int j = 0; j < 2; ++j) *reinterpret_cast<u32x4*>(dst + 64 * j) = op[j];
    return;
  }
  if (a.k_out) {
    T* dst = a.k_out + t * a.ko_st + (h * static_cast<int>(a.ko_sh) + d0);
#pragma unroll
    for (int j = 0; j < 2; ++j) *reinterpret_cast<u32x4*>(dst + 64 * j) = op[j];
  }
  if (placed) {
    T* kd = a.k_cache + (blk * a.kc_b + slot * a.kc_s) + (h * static_cast<int>(a.kc_h) + d0);
    T* vd = a.v_cache + (blk * a.vc_b + slot * a.vc_s) + (h * static_cast<int>(a.vc_h) + d0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      __builtin_nontemporal_store(op[j], reinterpret_cast<u32x4*>(kd + 64 * j));
      store_raw_nt<T>(vd + 64 * j, vv[j]);
    }
  }
}

// Largest element offset a view reaches (0 for an absent view).
static int64_t max_offset(const tsa_view* v) {
  if (!v || !v->data) return 0;
  int64_t m = 0;
  for (int d = 0; d < v->ndim; ++d) m += (v->size[d] > 0 ? v->size[d] - 1 : 0) * (v->stride[d] < 0 ? -v->stride[d] : v->stride[d]);
  return m;
}

template <typename T, int D>
static int launch_norm_rope(const NormRopeArgs<T>& a, bool vec, bool idx32, hipStream_t stream) {
  constexpr int ROWS = 256 / (D / 8);
  const int64_t rows = a.T_ * (a.Hq + a.Hkv);
  if (rows == 0) return TSA_OK;
  // Unit innermost strides everywhere (vec) and at most 80 heads per token:
  // the token-per-workgroup kernel.
  const int64_t H = a.Hq + a.Hkv;
  if constexpr (D == 128 && sizeof(T) == 2) {
    // Every per-lane head offset (head index x head stride, plus the row's
    // 128 elements) must fit an int for the 8-lanes-per-row kernel.
    const int64_t hs = std::max({std::abs(a.q_sh) * a.Hq, std::abs(a.qo_sh) * a.Hq, std::abs(a.k_sh) * a.Hkv,
                                 std::abs(a.ko_sh) * a.Hkv, std::abs(a.v_sh) * a.Hkv, std::abs(a.kc_h) * a.Hkv,
                                 std::abs(a.vc_h) * a.Hkv});
    if (vec && a.T_ <= INT32_MAX && H <= 128 && hs + D < INT32_MAX) {
      const int threads = static_cast<int>((8 * H + 63) / 64 * 64);
      qk_norm_rope_rows8<T><<<dim3(static_cast<uint32_t>(a.T_)), dim3(threads), 0, stream>>>(a);
      return check_launch("tsa_qk_norm_rope");
    }
  }
  if constexpr (D == 128) {
    if (vec && a.T_ <= INT32_MAX && H <= 80) {
      const dim3 grid(static_cast<uint32_t>(a.T_));
      switch ((H + 15) / 16) {
        case 1: qk_norm_rope_token<T, 1><<<grid, dim3(256), 0, stream>>>(a); break;
        case 2: qk_norm_rope_token<T, 2><<<grid, dim3(256), 0, stream>>>(a); break;
        case 3: qk_norm_rope_token<T, 3><<<grid, dim3(256), 0, stream>>>(a); break;
        case 4: qk_norm_rope_token<T, 4><<<grid, dim3(256), 0, stream>>>(a); break;
        default: qk_norm_rope_token<T, 5><<<grid, dim3(256), 0, stream>>>(a); break;
      }
      return check_launch("tsa_qk_norm_rope");
    }
  }
  const dim3 grid((rows + ROWS - 1) / ROWS);
  if (vec && idx32) qk_norm_rope_kernel<T, D, true, true><<<grid, dim3(256), 0, stream>>>(a);
  else if (vec) qk_norm_rope_kernel<T, D, true, false><<<grid, dim3(256), 0, stream>>>(a);
  else qk_norm_rope_kernel<T, D, false, false><<<grid, dim3(256), 0, stream>>>(a);
  return check_launch("tsa_qk_norm_rope");
}

template <typename T>
static int run_norm_rope(NormRopeArgs<T>& a, int64_t D, bool vec, bool idx32, hipStream_t stream) {
  switch (D) {
    case 64: return launch_norm_rope<T, 64>(a, vec, idx32, stream);
    case 128: return launch_norm_rope<T, 128>(a, vec, idx32, stream);
    case 256: return launch_norm_rope<T, 256>(a, vec, idx32, stream);
  }
  set_error("tsa_qk_norm_rope: head_dim %lld is not implemented (64, 128, 256)", (long long)D);
  return TSA_ERR_UNSUPPORTED;
}

template <typename T>
static int norm_rope_entry(const tsa_view* q, const tsa_view* k, const tsa_view* v, const tsa_view* q_out,
                           const tsa_view* k_out, const tsa_view* qw, const tsa_view* kw, const tsa_view* cos,
                           const tsa_view* sin, double eps, const tsa_view* k_cache, const tsa_view* v_cache,
                           const PagedAddr* addr, hipStream_t stream) {
  NormRopeArgs<T> a{};
  a.q = static_cast<const T*>(q->data);
  a.k = static_cast<const T*>(k->data);
  a.q_out = static_cast<T*>(q_out->data);
  a.k_out = k_out ? static_cast<T*>(k_out->data) : nullptr;
  a.qw = static_cast<const T*>(qw->data);
  a.kw = static_cast<const T*>(kw->data);
  a.cos = static_cast<const T*>(cos->data);
  a.sin = static_cast<const T*>(sin->data);
  a.q_st = q->stride[0]; a.q_sh = q->stride[1]; a.q_sd = q->stride[2];
  a.k_st = k->stride[0]; a.k_sh = k->stride[1]; a.k_sd = k->stride[2];
  a.qo_st = q_out->stride[0]; a.qo_sh = q_out->stride[1]; a.qo_sd = q_out->stride[2];
  if (a.k_out) { a.ko_st = k_out->stride[0]; a.ko_sh = k_out->stride[1]; a.ko_sd = k_out->stride[2]; }
  a.qw_s = qw->stride[0]; a.kw_s = kw->stride[0];
  a.cos_st = cos->stride[0]; a.cos_sd = cos->stride[1];
  a.sin_st = sin->stride[0]; a.sin_sd = sin->stride[1];
  a.T_ = q->size[0]; a.Hq = q->size[1]; a.Hkv = k->size[1];
  a.eps = static_cast<float>(eps);
  bool vec = vec_ok(q) && vec_ok(k) && vec_ok(q_out) && vec_ok(k_out) && vec_ok(cos) && vec_ok(sin) &&
             (qw->stride[0] == 1 && reinterpret_cast<uintptr_t>(qw->data) % 16 == 0) &&
             (kw->stride[0] == 1 && reinterpret_cast<uintptr_t>(kw->data) % 16 == 0);
  if (k_cache) {
    a.v = static_cast<const T*>(v->data);
    a.v_st = v->stride[0]; a.v_sh = v->stride[1]; a.v_sd = v->stride[2];
    a.k_cache = static_cast<T*>(k_cache->data);
    a.v_cache = static_cast<T*>(v_cache->data);
    a.kc_b = k_cache->stride[0]; a.kc_h = k_cache->stride[1]; a.kc_s = k_cache->stride[2]; a.kc_d = k_cache->stride[3];
    a.vc_b = v_cache->stride[0]; a.vc_h = v_cache->stride[1]; a.vc_s = v_cache->stride[2]; a.vc_d = v_cache->stride[3];
    a.NB = k_cache->size[0];
    a.BS = k_cache->size[2];
    a.addr = *addr;
    vec = vec && vec_ok(v) && vec_ok(k_cache) && vec_ok(v_cache);
  }
  // 32-bit index arithmetic when every row index and every offset into the
  // token-major tensors fits (the cache offsets stay 64-bit).
  const int64_t lim = int64_t{1} << 31;
  const bool idx32 = a.T_ * (a.Hq + a.Hkv) < lim && max_offset(q) < lim && max_offset(k) < lim &&
                     max_offset(q_out) < lim && max_offset(k_out) < lim && max_offset(cos) < lim &&
                     max_offset(sin) < lim && max_offset(v) < lim;
  return run_norm_rope<T>(a, q->size[2], vec, idx32, stream);
}

static int check_norm_rope(const tsa_view* q, const tsa_view* k, const tsa_view* q_out, const tsa_view* k_out,
                           const tsa_view* qw, const tsa_view* kw, const tsa_view* cos, const tsa_view* sin) {
  TSA_REQUIRE(view_ok(q, 3) && view_ok(k, 3), "q and k must be 3D tensors (num_tokens, num_heads, head_dim)");
  TSA_REQUIRE(view_ok(q_out, 3), "q_out must be a 3D tensor shaped like q");
  TSA_REQUIRE(view_ok(qw, 1) && view_ok(kw, 1), "q_weight and k_weight must be 1D tensors (head_dim)");
  TSA_REQUIRE(view_ok(cos, 2) && view_ok(sin, 2), "cos and sin must be 2D tensors (num_tokens, head_dim)");
  const int dt = q->dtype;
  TSA_REQUIRE(is_float_dtype(dt), "q must be bf16, f16 or f32 (got %s)", dtype_name(dt));
  TSA_REQUIRE(k->dtype == dt && q_out->dtype == dt && qw->dtype == dt && kw->dtype == dt && cos->dtype == dt &&
                  sin->dtype == dt,
              "q, k, outputs, norm weights and cos/sin must share the model dtype %s", dtype_name(dt));
  const int64_t T = q->size[0], D = q->size[2];
  TSA_REQUIRE(k->size[0] == T && k->size[2] == D, "k must be (num_tokens=%lld, Hkv, head_dim=%lld)", (long long)T,
              (long long)D);
  for (int d = 0; d < 3; ++d) TSA_REQUIRE(q_out->size[d] == q->size[d], "q_out must have q's shape");
  if (k_out && k_out->data) {
    TSA_REQUIRE(view_ok(k_out, 3) && k_out->dtype == dt, "k_out must be a 3D tensor shaped like k");
    for (int d = 0; d < 3; ++d) TSA_REQUIRE(k_out->size[d] == k->size[d], "k_out must have k's shape");
  }
  TSA_REQUIRE(qw->size[0] == D && kw->size[0] == D, "norm weights must have head_dim (%lld) entries", (long long)D);
  TSA_REQUIRE(cos->size[0] == T && cos->size[1] == D && sin->size[0] == T && sin->size[1] == D,
              "cos and sin must be (num_tokens=%lld, head_dim=%lld)", (long long)T, (long long)D);
  TSA_REQUIRE(D % 16 == 0, "head_dim must be a multiple of 16 (got %lld)", (long long)D);
  return TSA_OK;
}

}  // namespace tsa

using namespace tsa;

template <typename... Args>
static int dispatch_dtype(int dt, Args&&... args) {
  switch (dt) {
    case TSA_BF16: return norm_rope_entry<bf16_t>(args...);
    case TSA_F16: return norm_rope_entry<f16_t>(args...);
    case TSA_F32: return norm_rope_entry<float>(args...);
  }
  set_error("unsupported dtype %d", dt);
  return TSA_ERR_UNSUPPORTED;
}

extern "C" int tsa_qk_norm_rope(const tsa_view* q, const tsa_view* k, const tsa_view* q_out, const tsa_view* k_out,
                                const tsa_view* q_weight, const tsa_view* k_weight, const tsa_view* cos,
                                const tsa_view* sin, double eps, void* stream) {
  if (int rc = check_norm_rope(q, k, q_out, k_out, q_weight, k_weight, cos, sin)) return rc;
  TSA_REQUIRE(k_out && k_out->data, "k_out is required when K is not stored into a cache");
  return dispatch_dtype(q->dtype, q, k, nullptr, q_out, k_out, q_weight, k_weight, cos, sin, eps, nullptr, nullptr,
                        nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int tsa_qk_norm_rope_store(const tsa_view* q, const tsa_view* k, const tsa_view* v,
                                      const tsa_view* q_out, const tsa_view* k_out, const tsa_view* q_weight,
                                      const tsa_view* k_weight, const tsa_view* cos, const tsa_view* sin, double eps,
                                      const tsa_view* k_cache, const tsa_view* v_cache,
                                      const tsa_view* block_tables, const tsa_view* cu_seqlens,
                                      const tsa_view* positions, void* stream) {
  if (int rc = check_norm_rope(q, k, q_out, k_out, q_weight, k_weight, cos, sin)) return rc;
  TSA_REQUIRE(view_ok(v, 3), "v must be a 3D tensor (num_tokens, Hkv, head_dim)");
  for (int d = 0; d < 3; ++d) TSA_REQUIRE(v->size[d] == k->size[d], "v must have k's shape");
  TSA_REQUIRE(view_ok(k_cache, 4) && view_ok(v_cache, 4),
              "k_cache and v_cache must be 4D tensors (num_blocks, num_kv_heads, block_size, head_dim)");
  for (int d = 0; d < 4; ++d) TSA_REQUIRE(k_cache->size[d] == v_cache->size[d], "k_cache and v_cache must match");
  TSA_REQUIRE(v->dtype == q->dtype && k_cache->dtype == q->dtype && v_cache->dtype == q->dtype,
              "v and the caches must share the model dtype %s", dtype_name(q->dtype));
  TSA_REQUIRE(k_cache->size[1] == k->size[1] && k_cache->size[3] == k->size[2],
              "cache (NB, %lld, BS, %lld) does not match k (T, %lld, %lld)", (long long)k_cache->size[1],
              (long long)k_cache->size[3], (long long)k->size[1], (long long)k->size[2]);
  TSA_REQUIRE(k_cache->size[2] > 0, "block_size must be positive");
  PagedAddr addr;
  if (int rc = make_paged_addr(block_tables, cu_seqlens, positions, k->size[0], addr)) return rc;
  const tsa_view* ko = (k_out && k_out->data) ? k_out : nullptr;
  return dispatch_dtype(q->dtype, q, k, v, q_out, ko, q_weight, k_weight, cos, sin, eps, k_cache, v_cache, &addr,
                        static_cast<hipStream_t>(stream));
}
