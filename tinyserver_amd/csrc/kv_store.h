// Internal interface of the paged K/V store, shared with the fused
// norm+RoPE+store kernel.
#pragma once

#include "tsa_common.h"

namespace tsa {

// Source rows (Hkv, T, D) and destination pool (NB, Hkv, BS, D); byte
// strides except the *_d element strides of the innermost dimension.
struct StoreGeom {
  const char* k_src;
  const char* v_src;
  char* k_dst;
  char* v_dst;
  int64_t T, H, D, NB, BS, chunks;
  int64_t ks_h, ks_t, ks_d, vs_h, vs_t, vs_d;
  int64_t kc_b, kc_h, kc_s, kc_d, vc_b, vc_h, vc_s, vc_d;
  int elem_bytes;
  bool vec16;
};

// Device-side (block, slot) lookup from per-sequence block tables,
// cu_seqlens and optional absolute positions.
struct PagedAddr {
  const int32_t* bt;
  int64_t bt_s0, bt_s1, max_blocks;
  const int32_t* cu;
  int64_t cu_stride, nseq;
  const void* pos;
  int64_t pos_stride;
  int pos_kind;  // 0: position = t - cu[s]; 1: int32 positions; 2: int64 positions
  __device__ __forceinline__ bool locate(int64_t t, int64_t BS, int64_t NB, int64_t& blk, int64_t& slot) const;
};

__device__ __forceinline__ bool PagedAddr::locate(int64_t t, int64_t BS, int64_t NB, int64_t& blk, int64_t& slot) const {
  // Sequence of token t: the last s with cu[s] <= t (binary search, cu sorted).
  int64_t lo = 0, hi = nseq;  // answer in [lo, hi)
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (cu[mid * cu_stride] <= t) lo = mid; else hi = mid;
  }
  const int64_t s = lo;
  const int64_t t0 = cu[s * cu_stride];
  if (t < t0 || t >= cu[(s + 1) * cu_stride]) return false;
  int64_t p;
  if (pos_kind == 2) p = static_cast<const int64_t*>(pos)[t * pos_stride];
  else if (pos_kind == 1) p = static_cast<const int32_t*>(pos)[t * pos_stride];
  else p = t - t0;
  if (p < 0) return false;
  const int64_t lb = p / BS;
  if (lb >= max_blocks) return false;
  blk = bt[s * bt_s0 + lb * bt_s1];
  slot = p % BS;
  return blk >= 0 && blk < NB;
}


int make_store_geom(const tsa_view* k_src, const tsa_view* v_src, const tsa_view* k_cache,
                    const tsa_view* v_cache, StoreGeom& g);
int make_paged_addr(const tsa_view* block_tables, const tsa_view* cu_seqlens, const tsa_view* positions,
                    int64_t num_tokens, PagedAddr& a);
int launch_store_paged(const StoreGeom& g, const PagedAddr& a, hipStream_t stream);

}  // namespace tsa
