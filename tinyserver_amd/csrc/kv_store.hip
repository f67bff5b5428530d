// Paged K/V store: copy new K/V rows (Hkv, T, D) into the paged pool
// (NB, Hkv, BS, D) at cache[block, h, slot, :].
//
// Reference: server/model/kernels/kv_cache.py:6-70 (_store_kv_kernel, one
// program per (token, kv head)) and :122-191 (_store_kv_cache_batched_kernel,
// 16-token tiles with int64 offsets). Here one thread moves one 16-byte chunk
// of a row, so a 256-byte bf16 D=128 row is 16 lanes and a wave writes four
// rows with fully coalesced 128-bit stores. The three addressing modes differ
// only in how (block, slot) is found for token t:
//   start   block_table[(p0 + t) / BS], (p0 + t) % BS        (kv_cache.py:41-53)
//   mapped  block_mapping[t], slot_mapping[t]                 (kv_cache.py:168-173)
//   paged   sequence s = the cu_seqlens bucket of t, p = positions[t] or
//           t - cu_seqlens[s]; block_tables[s, p / BS], p % BS (qwen3.py:296-303)
// Unlike the reference (no device-side checks, a bad id is undefined
// behaviour), a token whose logical block is past its table or whose block or
// slot is out of range is skipped instead of written out of bounds.
#include "kv_store.h"

namespace tsa {

struct AddrStart {
  const int32_t* bt;
  int64_t bt_stride, bt_len, start;
  __device__ bool locate(int64_t t, int64_t BS, int64_t NB, int64_t& blk, int64_t& slot) const {
    const int64_t p = start + t;
    if (p < 0) return false;
    const int64_t lb = p / BS;
    if (lb >= bt_len) return false;
    blk = bt[lb * bt_stride];
    slot = p % BS;
    return blk >= 0 && blk < NB;
  }
};

struct AddrMapped {
  const void* bm;
  const void* sm;
  int64_t bm_stride, sm_stride;
  int bm64, sm64;
  __device__ bool locate(int64_t t, int64_t BS, int64_t NB, int64_t& blk, int64_t& slot) const {
    blk = bm64 ? static_cast<const int64_t*>(bm)[t * bm_stride] : static_cast<const int32_t*>(bm)[t * bm_stride];
    slot = sm64 ? static_cast<const int64_t*>(sm)[t * sm_stride] : static_cast<const int32_t*>(sm)[t * sm_stride];
    return blk >= 0 && blk < NB && slot >= 0 && slot < BS;
  }
};

// One thread per 16-byte chunk of one (token, head) row; rows are ordered
// token-major so the heads of a token share its (block, slot) lookup.
template <class Addr>
__global__ __launch_bounds__(256) void store_rows_vec16(StoreGeom g, Addr addr) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = g.T * g.H * g.chunks;
  if (gid >= total) return;
  const int64_t row = gid / g.chunks;
  const int64_t chunk = gid - row * g.chunks;
  const int64_t t = row / g.H;
  const int64_t h = row - t * g.H;
  int64_t blk, slot;
  if (!addr.locate(t, g.BS, g.NB, blk, slot)) return;
  const int64_t off = chunk * 16;
  const u32x4 kv = *reinterpret_cast<const u32x4*>(g.k_src + h * g.ks_h + t * g.ks_t + off);
  const u32x4 vv = *reinterpret_cast<const u32x4*>(g.v_src + h * g.vs_h + t * g.vs_t + off);
  *reinterpret_cast<u32x4*>(g.k_dst + blk * g.kc_b + h * g.kc_h + slot * g.kc_s + off) = kv;
  *reinterpret_cast<u32x4*>(g.v_dst + blk * g.vc_b + h * g.vc_h + slot * g.vc_s + off) = vv;
}

// Any strides: one thread per element (element size 2 or 4 bytes).
template <class Addr, typename E>
__global__ __launch_bounds__(256) void store_elems(StoreGeom g, Addr addr) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = g.T * g.H * g.D;
  if (gid >= total) return;
  const int64_t row = gid / g.D;
  const int64_t d = gid - row * g.D;
  const int64_t t = row / g.H;
  const int64_t h = row - t * g.H;
  int64_t blk, slot;
  if (!addr.locate(t, g.BS, g.NB, blk, slot)) return;
  const int64_t e = sizeof(E);
  const E kv = *reinterpret_cast<const E*>(g.k_src + h * g.ks_h + t * g.ks_t + d * g.ks_d * e);
  const E vv = *reinterpret_cast<const E*>(g.v_src + h * g.vs_h + t * g.vs_t + d * g.vs_d * e);
  *reinterpret_cast<E*>(g.k_dst + blk * g.kc_b + h * g.kc_h + slot * g.kc_s + d * g.kc_d * e) = kv;
  *reinterpret_cast<E*>(g.v_dst + blk * g.vc_b + h * g.vc_h + slot * g.vc_s + d * g.vc_d * e) = vv;
}

template <class Addr>
static int launch_store(const StoreGeom& g, const Addr& addr, hipStream_t stream, const char* what) {
  if (g.T == 0 || g.H == 0 || g.D == 0) return TSA_OK;
  const int threads = 256;
  if (g.vec16) {
    const int64_t total = g.T * g.H * g.chunks;
    store_rows_vec16<Addr><<<dim3((total + threads - 1) / threads), dim3(threads), 0, stream>>>(g, addr);
  } else {
    const int64_t total = g.T * g.H * g.D;
    const dim3 grid((total + threads - 1) / threads);
    if (g.elem_bytes == 4) store_elems<Addr, uint32_t><<<grid, dim3(threads), 0, stream>>>(g, addr);
    else store_elems<Addr, uint16_t><<<grid, dim3(threads), 0, stream>>>(g, addr);
  }
  return check_launch(what);
}

// Validate src (Hkv, T, D) and cache (NB, Hkv, BS, D) views and fill a geometry.
int make_store_geom(const tsa_view* k_src, const tsa_view* v_src, const tsa_view* k_cache,
                    const tsa_view* v_cache, StoreGeom& g) {
  TSA_REQUIRE(view_ok(k_src, 3) && view_ok(v_src, 3),
              "k_src and v_src must be 3D tensors (num_kv_heads, num_tokens, head_dim)");
  TSA_REQUIRE(view_ok(k_cache, 4) && view_ok(v_cache, 4),
              "k_cache and v_cache must be 4D tensors (num_blocks, num_kv_heads, block_size, head_dim)");
  for (int d = 0; d < 3; ++d)
    TSA_REQUIRE(k_src->size[d] == v_src->size[d], "k_src and v_src must have the same shape");
  for (int d = 0; d < 4; ++d)
    TSA_REQUIRE(k_cache->size[d] == v_cache->size[d], "k_cache and v_cache must have the same shape");
  TSA_REQUIRE(is_float_dtype(k_src->dtype) && k_src->dtype == v_src->dtype && k_cache->dtype == k_src->dtype &&
                  v_cache->dtype == k_src->dtype,
              "k_src, v_src, k_cache and v_cache must share one floating dtype (got %s/%s/%s/%s)",
              dtype_name(k_src->dtype), dtype_name(v_src->dtype), dtype_name(k_cache->dtype),
              dtype_name(v_cache->dtype));
  TSA_REQUIRE(k_src->size[0] == k_cache->size[1], "k_src has %lld kv heads but the cache has %lld",
              (long long)k_src->size[0], (long long)k_cache->size[1]);
  TSA_REQUIRE(k_src->size[2] == k_cache->size[3], "k_src head_dim %lld != cache head_dim %lld",
              (long long)k_src->size[2], (long long)k_cache->size[3]);
  TSA_REQUIRE(k_cache->size[2] > 0, "block_size must be positive");
  const int64_t eb = dtype_bytes(k_src->dtype);
  g.H = k_src->size[0];
  g.T = k_src->size[1];
  g.D = k_src->size[2];
  g.NB = k_cache->size[0];
  g.BS = k_cache->size[2];
  g.elem_bytes = static_cast<int>(eb);
  g.k_src = static_cast<const char*>(k_src->data);
  g.v_src = static_cast<const char*>(v_src->data);
  g.k_dst = static_cast<char*>(k_cache->data);
  g.v_dst = static_cast<char*>(v_cache->data);
  g.ks_h = k_src->stride[0] * eb; g.ks_t = k_src->stride[1] * eb; g.ks_d = k_src->stride[2];
  g.vs_h = v_src->stride[0] * eb; g.vs_t = v_src->stride[1] * eb; g.vs_d = v_src->stride[2];
  g.kc_b = k_cache->stride[0] * eb; g.kc_h = k_cache->stride[1] * eb; g.kc_s = k_cache->stride[2] * eb;
  g.kc_d = k_cache->stride[3];
  g.vc_b = v_cache->stride[0] * eb; g.vc_h = v_cache->stride[1] * eb; g.vc_s = v_cache->stride[2] * eb;
  g.vc_d = v_cache->stride[3];
  g.vec16 = rows_vec16(k_src) && rows_vec16(v_src) && rows_vec16(k_cache) && rows_vec16(v_cache);
  g.chunks = g.D * eb / 16;
  return TSA_OK;
}

int make_paged_addr(const tsa_view* block_tables, const tsa_view* cu_seqlens, const tsa_view* positions,
                    int64_t num_tokens, PagedAddr& a) {
  TSA_REQUIRE(view_ok(block_tables, 2) && block_tables->dtype == TSA_I32,
              "block_tables must be a 2D int32 tensor (num_seqs, max_blocks)");
  TSA_REQUIRE(view_ok(cu_seqlens, 1) && cu_seqlens->dtype == TSA_I32 && cu_seqlens->size[0] >= 1,
              "cu_seqlens must be a 1D int32 tensor (num_seqs + 1)");
  TSA_REQUIRE(cu_seqlens->size[0] == block_tables->size[0] + 1,
              "cu_seqlens has %lld entries for %lld block-table rows", (long long)cu_seqlens->size[0],
              (long long)block_tables->size[0]);
  a.bt = static_cast<const int32_t*>(block_tables->data);
  a.bt_s0 = block_tables->stride[0];
  a.bt_s1 = block_tables->stride[1];
  a.max_blocks = block_tables->size[1];
  a.cu = static_cast<const int32_t*>(cu_seqlens->data);
  a.cu_stride = cu_seqlens->stride[0];
  a.nseq = block_tables->size[0];
  a.pos = nullptr;
  a.pos_stride = 0;
  a.pos_kind = 0;
  if (positions && positions->data) {
    TSA_REQUIRE(view_ok(positions, 1) && is_index_dtype(positions->dtype) && positions->size[0] == num_tokens,
                "positions must be a 1D int32/int64 tensor of num_tokens (%lld) entries", (long long)num_tokens);
    a.pos = positions->data;
    a.pos_stride = positions->stride[0];
    a.pos_kind = positions->dtype == TSA_I64 ? 2 : 1;
  }
  TSA_REQUIRE(a.nseq > 0 || num_tokens == 0, "no sequences for %lld tokens", (long long)num_tokens);
  return TSA_OK;
}

int launch_store_paged(const StoreGeom& g, const PagedAddr& a, hipStream_t stream) {
  return launch_store(g, a, stream, "tsa_store_kv_paged");
}

}  // namespace tsa

using namespace tsa;

extern "C" int tsa_store_kv(const tsa_view* k_src, const tsa_view* v_src, const tsa_view* k_cache,
                            const tsa_view* v_cache, const tsa_view* block_table, int64_t start_position,
                            void* stream) {
  StoreGeom g;
  if (int rc = make_store_geom(k_src, v_src, k_cache, v_cache, g)) return rc;
  TSA_REQUIRE(view_ok(block_table, 1) && block_table->dtype == TSA_I32, "block_table must be a 1D int32 tensor");
  AddrStart a{static_cast<const int32_t*>(block_table->data), block_table->stride[0], block_table->size[0],
              start_position};
  return launch_store(g, a, static_cast<hipStream_t>(stream), "tsa_store_kv");
}

extern "C" int tsa_store_kv_mapped(const tsa_view* k_src, const tsa_view* v_src, const tsa_view* k_cache,
                                   const tsa_view* v_cache, const tsa_view* block_mapping,
                                   const tsa_view* slot_mapping, void* stream) {
  StoreGeom g;
  if (int rc = make_store_geom(k_src, v_src, k_cache, v_cache, g)) return rc;
  TSA_REQUIRE(view_ok(block_mapping, 1) && view_ok(slot_mapping, 1) && is_index_dtype(block_mapping->dtype) &&
                  is_index_dtype(slot_mapping->dtype),
              "block_mapping and slot_mapping must be 1D int32/int64 tensors");
  TSA_REQUIRE(block_mapping->size[0] == g.T && slot_mapping->size[0] == g.T,
              "block_mapping and slot_mapping must have length num_tokens (%lld), but got %lld and %lld",
              (long long)g.T, (long long)block_mapping->size[0], (long long)slot_mapping->size[0]);
  AddrMapped a{block_mapping->data, slot_mapping->data, block_mapping->stride[0], slot_mapping->stride[0],
               block_mapping->dtype == TSA_I64, slot_mapping->dtype == TSA_I64};
  return launch_store(g, a, static_cast<hipStream_t>(stream), "tsa_store_kv_mapped");
}

extern "C" int tsa_store_kv_paged(const tsa_view* k_src, const tsa_view* v_src, const tsa_view* k_cache,
                                  const tsa_view* v_cache, const tsa_view* block_tables,
                                  const tsa_view* cu_seqlens, const tsa_view* positions, void* stream) {
  StoreGeom g;
  if (int rc = make_store_geom(k_src, v_src, k_cache, v_cache, g)) return rc;
  PagedAddr a;
  if (int rc = make_paged_addr(block_tables, cu_seqlens, positions, g.T, a)) return rc;
  return launch_store_paged(g, a, static_cast<hipStream_t>(stream));
}
