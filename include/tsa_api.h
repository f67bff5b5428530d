/*
 * tsa_api.h -- C ABI of the MI355X (gfx950) Qwen3 attention hot path.
 *
 * One shared library, libtsa.so, built with hipcc for gfx950. Every entry
 * point takes plain views of caller-owned device memory plus a HIP stream
 * (passed as void*, so no HIP header is needed to bind it) and returns an int
 * status. The library never allocates device memory: outputs and the decode
 * workspace are passed in by the caller (tsa_paged_decode_noalloc uses a
 * fixed array the library's code object holds instead). Launches are asynchronous on the
 * given stream; nothing synchronises.
 *
 * Status codes: TSA_OK (0); TSA_ERR_INVALID (-1) for an argument that the
 * reference would reject or that is malformed (message from tsa_last_error);
 * TSA_ERR_UNSUPPORTED (-2) for a well-formed call outside what the kernels
 * implement (for example head_dim 96); TSA_ERR_LAUNCH (-3) for a HIP error.
 * tsa_last_error() is per calling thread.
 *
 * Reference interfaces replaced (paths relative to the tinyserver repository):
 *   tsa_store_kv            server/model/kernels/kv_cache.py:73-119   (store_kv_cache)
 *   tsa_store_kv_mapped     server/model/kernels/kv_cache.py:194-251  (store_kv_cache_batched)
 *   tsa_store_kv_paged      server/model/patches/qwen3.py:296-318, 335-357
 *                           (the per-token mapping loop and per-sequence store
 *                           loop at the call site, done on the device)
 *   tsa_qk_norm_rope        server/model/patches/qwen3.py:268-287 (q_norm, k_norm,
 *                           apply_rotary_pos_emb; transformers
 *                           models/qwen3/modeling_qwen3.py:59-64, 140-170)
 *   tsa_qk_norm_rope_store  the same, fused with tsa_store_kv_paged
 *   tsa_paged_decode        server/model/kernels/paged_attention.py:124-192
 *                           (paged_attention_forward)
 *   tsa_paged_decode_noalloc  no counterpart: tsa_paged_decode with library-held
 *                           scratch, for callers that cannot allocate
 *   tsa_paged_decode_step   the decode call site (qwen3.py:268-287, 335-409):
 *                           norm/RoPE, store and paged attention, fused
 *   tsa_varlen_prefill      server/model/kernels/varlen_attention.py:145-218
 *                           (flash_attn_varlen_func)
 *   tsa_mixed_attention     no single counterpart: a prefill batch's attention
 *                           (flash_attn_varlen_func, qwen3.py:173-214) and a
 *                           decode batch's (paged_attention_forward,
 *                           qwen3.py:387-409) in one launch, for an engine
 *                           that batches them together (the reference's
 *                           scheduler issues them apart, scheduler.py:128-227)
 *   tsa_sample_tokens       server/model/sampling.py:119-194 (sample_tokens)
 *   tsa_sample_tokens_ws    the same, with a workspace that lets a small
 *                           batch spread each row over several workgroups
 *   tsa_sample_tokens_workspace_bytes  its size
 */
#ifndef TSA_API_H
#define TSA_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSA_ABI_VERSION 1

enum tsa_status {
  TSA_OK = 0,
  TSA_ERR_INVALID = -1,
  TSA_ERR_UNSUPPORTED = -2,
  TSA_ERR_LAUNCH = -3,
};

enum tsa_dtype {
  TSA_BF16 = 0,
  TSA_F16 = 1,
  TSA_F32 = 2,
  TSA_I32 = 3,
  TSA_I64 = 4,
};

/* A strided view of caller-owned device memory: element (i0, i1, ...) sits at
 * data + sum(i_d * stride[d]) elements. Sizes and strides are in elements,
 * outermost first; entries past ndim are ignored. */
typedef struct tsa_view {
  void* data;
  int64_t size[4];
  int64_t stride[4];
  int32_t ndim;
  int32_t dtype; /* enum tsa_dtype */
} tsa_view;

/* ABI version of the loaded library (TSA_ABI_VERSION). */
int tsa_abi_version(void);

/* Message for the last non-zero status returned on this thread. */
const char* tsa_last_error(void);

/* store_kv_cache (kv_cache.py:73-119): for one sequence, token i of
 * k_src/v_src (Hkv, n, D) goes to absolute position start_position + i:
 * cache[block_table[p / BS], h, p % BS, :] for k_cache/v_cache
 * (NB, Hkv, BS, D). block_table: (n_blocks,) int32. Positions whose logical
 * block is past the table, or whose block id is outside [0, NB), are not
 * written. */
int tsa_store_kv(const tsa_view* k_src, const tsa_view* v_src, const tsa_view* k_cache,
                 const tsa_view* v_cache, const tsa_view* block_table, int64_t start_position,
                 void* stream);

/* store_kv_cache_batched (kv_cache.py:194-251): token t of k_src/v_src
 * (Hkv, T, D) goes to cache[block_mapping[t], h, slot_mapping[t], :].
 * block_mapping/slot_mapping: (T,) int32 or int64. Out-of-range ids are
 * skipped. */
int tsa_store_kv_mapped(const tsa_view* k_src, const tsa_view* v_src, const tsa_view* k_cache,
                        const tsa_view* v_cache, const tsa_view* block_mapping,
                        const tsa_view* slot_mapping, void* stream);

/* Device-side addressing for a whole batch (replaces qwen3.py:296-318 and
 * :335-357). Tokens of sequence s are k_src[:, cu_seqlens[s]:cu_seqlens[s+1], :];
 * token t sits at position positions[t] when positions is non-NULL (int32 or
 * int64, (T,)), else at t - cu_seqlens[s] (prefill). It is written to
 * cache[block_tables[s, p / BS], h, p % BS, :]. block_tables: (nseq, max_blocks)
 * int32; cu_seqlens: (nseq + 1,) int32. */
int tsa_store_kv_paged(const tsa_view* k_src, const tsa_view* v_src, const tsa_view* k_cache,
                       const tsa_view* v_cache, const tsa_view* block_tables,
                       const tsa_view* cu_seqlens, const tsa_view* positions, void* stream);

/* Fused Qwen3 per-head RMSNorm + rotate-half RoPE with HF's rounding points:
 * y = w * round(x * rsqrt(mean(x^2) + eps)); out = round(round(y*cos) +
 * round(rotate_half(y)*sin)). q: (T, Hq, D), k: (T, Hkv, D) inputs;
 * q_out/k_out same shapes (may alias the inputs); q_weight/k_weight: (D,);
 * cos/sin: (T, D) in the model dtype. eps is rounded to fp32 as HF does. */
int tsa_qk_norm_rope(const tsa_view* q, const tsa_view* k, const tsa_view* q_out,
                     const tsa_view* k_out, const tsa_view* q_weight, const tsa_view* k_weight,
                     const tsa_view* cos, const tsa_view* sin, double eps, void* stream);

/* tsa_qk_norm_rope plus the paged store of the rotated K and of v (T, Hkv, D)
 * into k_cache/v_cache with tsa_store_kv_paged's addressing. k_out may have
 * data == NULL when the caller needs the rotated K only in the cache. */
int tsa_qk_norm_rope_store(const tsa_view* q, const tsa_view* k, const tsa_view* v,
                           const tsa_view* q_out, const tsa_view* k_out,
                           const tsa_view* q_weight, const tsa_view* k_weight,
                           const tsa_view* cos, const tsa_view* sin, double eps,
                           const tsa_view* k_cache, const tsa_view* v_cache,
                           const tsa_view* block_tables, const tsa_view* cu_seqlens,
                           const tsa_view* positions, void* stream);

/* Bytes of workspace tsa_paged_decode needs: one partial-result slot per
 * (sequence x kv head, wave) pair that can occur -- num_seqs * num_kv_heads
 * + 4 * num_workgroups slots of (G * head_dim + 2 * G) floats -- and the tile
 * prefix (num_workgroups 0 = the library's choice, one per CU). */
size_t tsa_paged_decode_workspace_bytes(int64_t num_seqs, int64_t num_heads, int64_t num_kv_heads,
                                        int64_t head_dim, int64_t max_blocks_per_seq,
                                        int64_t block_size, int32_t num_workgroups);

/* paged_attention_forward (paged_attention.py:124-192):
 * out[s, h] = softmax(query[s, h] . K_s^T * softmax_scale) V_s over the first
 * seq_lens[s] tokens gathered through block_tables[s], kv head h / (Hq/Hkv).
 * query/out: (B, Hq, D); caches (NB, Hkv, BS, D); block_tables (B, max_blocks)
 * int32; seq_lens (B,) int32. The 16-token tiles of all sequences are split
 * evenly over the 4 waves of num_workgroups workgroups (0 = the library's
 * choice: one per CU, fewer for small tables); a second launch merges each
 * sequence's per-wave partial results, which the workspace holds (no
 * initialisation needed; calls that share one must be ordered on one
 * stream). With num_workgroups 0, a batch of at most 64 (sequence, kv head)
 * units whose tables hold at most 512 tokens takes one launch instead: one
 * workgroup per unit, whose waves merge in LDS and write out. */
int tsa_paged_decode(const tsa_view* out, const tsa_view* query, const tsa_view* k_cache,
                     const tsa_view* v_cache, const tsa_view* block_tables,
                     const tsa_view* seq_lens, double softmax_scale, void* workspace,
                     size_t workspace_bytes, int32_t num_workgroups, void* stream);

/* tsa_paged_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). It has no counterpart in the reference.
 * Same arguments, kernels and results as tsa_paged_decode; the partials and
 * tile prefix live in a 16 MiB array the library holds on each GPU it runs on
 * until the process ends, so it allocates nothing. Every argument is checked
 * before any device work. A call served by the MFMA stream kernel whose
 * workspace (tsa_paged_decode_workspace_bytes) would exceed 16 MiB is then
 * rejected with TSA_ERR_INVALID; calls served by the generic kernel (fp32,
 * other head_dims, more than 16 q-heads per kv head, strided rows) take no
 * scratch and are accepted as tsa_paged_decode accepts them. All calls on one GPU share that
 * GPU's array: calls ordered on one stream are fine; calls that overlap on
 * one GPU (concurrent streams, threads) race and must not be issued. */
int tsa_paged_decode_noalloc(const tsa_view* out, const tsa_view* query, const tsa_view* k_cache,
                             const tsa_view* v_cache, const tsa_view* block_tables,
                             const tsa_view* seq_lens, double softmax_scale, int32_t num_workgroups,
                             void* stream);
/* The decode step of the Qwen3 call site, fused (qwen3.py:268-287 norm and
 * RoPE of q and of the new k, :335-357 the store of the new token's k and v,
 * :359-409 paged_attention_forward), in the two launches of tsa_paged_decode:
 * query (B, Hq, D) and k / v (B, Hkv, D) are the raw projections of each
 * sequence's new token, at position seq_lens[s] - 1; q_weight, k_weight (D);
 * cos / sin (B, D) for those positions. The rotated k and the raw v are
 * written to the token's cache slot; out is the attention over the first
 * seq_lens[s] tokens, the new one included. Same rounding as
 * tsa_qk_norm_rope_store followed by tsa_paged_decode. TSA_ERR_UNSUPPORTED
 * unless: bf16/f16, head_dim 128, pages a multiple of 16 tokens, contiguous
 * cache rows, at most 8 q-heads per kv head; callers then use those two. */
int tsa_paged_decode_step(const tsa_view* out, const tsa_view* query, const tsa_view* k_new,
                          const tsa_view* v_new, const tsa_view* q_weight, const tsa_view* k_weight,
                          const tsa_view* cos, const tsa_view* sin, double eps, const tsa_view* k_cache,
                          const tsa_view* v_cache, const tsa_view* block_tables, const tsa_view* seq_lens,
                          double softmax_scale, void* workspace, size_t workspace_bytes,
                          int32_t num_workgroups, void* stream);

/* flash_attn_varlen_func (varlen_attention.py:145-218): per sequence b and
 * q-head h, softmax(q k^T * softmax_scale) v over keys cu_seqlens_k[b] ..
 * cu_seqlens_k[b+1], kv head h / (Hq/Hkv); causal masks key j > query i
 * (positions within the sequence, top-left aligned). q/out: (Tq, Hq, D);
 * k/v: (Tk, Hkv, D); cu_seqlens_*: (b + 1,) int32. */
int tsa_varlen_prefill(const tsa_view* out, const tsa_view* q, const tsa_view* k,
                       const tsa_view* v, const tsa_view* cu_seqlens_q,
                       const tsa_view* cu_seqlens_k, int64_t max_seqlen_q, int64_t max_seqlen_k,
                       int32_t causal, double softmax_scale, void* stream);

/* A continuous-batching step's two attention calls in one launch (+ the
 * decode merge): the causal varlen prefill of a prefill batch --
 * prefill_out, prefill_q/k/v and cu_seqlens as tsa_varlen_prefill's out, q,
 * k, v and cu_seqlens_q = cu_seqlens_k, causal, scale prefill_scale -- and
 * the paged decode attention of a decode batch, with tsa_paged_decode's
 * arguments and rules (its K/V already stored). Same outputs, bit for bit,
 * as tsa_varlen_prefill then tsa_paged_decode on one stream. One kernel can
 * run both when the decode has head_dim 128, 16-token-multiple pages and
 * contiguous cache rows and the prefill takes the 4-head-group,
 * head_dim-128 LDS-staged kernel in the decode's dtype: num_workgroups
 * decode workgroups (0: one per CU) beside the prefill workgroups, so that
 * each CU runs one of each. prefill_workgroups > 0 asks for that kernel with
 * that many prefill workgroups; 0 takes it for prefill batches of at most 512
 * tokens beside decode block tables spanning at most 131072 tokens (batch x
 * table width x page size; the two roles slow each other down on a shared
 * CU, so it pays only when both are small) and issues the two calls
 * otherwise. */
int tsa_mixed_attention(const tsa_view* prefill_out, const tsa_view* prefill_q, const tsa_view* prefill_k,
                        const tsa_view* prefill_v, const tsa_view* cu_seqlens, int64_t max_seqlen,
                        double prefill_scale, const tsa_view* out, const tsa_view* query,
                        const tsa_view* k_cache, const tsa_view* v_cache, const tsa_view* block_tables,
                        const tsa_view* seq_lens, double softmax_scale, void* workspace,
                        size_t workspace_bytes, int32_t num_workgroups, int32_t prefill_workgroups,
                        void* stream);

/* sample_tokens (server/model/sampling.py:119-194): one token per row of
 * logits (B, V) (bf16, f16 or f32): x = logits / max(temperature, 1e-5), in
 * rank order (x descending, index ascending, the stable sort's order) keep
 * the first top_k ranks (0 or >= V: all), then the ranks whose preceding mass
 * is at most top_p (rank 0 always), and pick the first kept rank whose
 * cumulative mass reaches uniforms * (kept mass); rows with temperature <= 0
 * take the first index of the maximum. temperature, top_p, uniforms: (B,)
 * f32; top_k: (B,) int32 or int64; out: (B,) int64. One launch, no host
 * sync, no workspace. */
int tsa_sample_tokens(const tsa_view* out, const tsa_view* logits, const tsa_view* temperature,
                      const tsa_view* top_k, const tsa_view* top_p, const tsa_view* uniforms,
                      void* stream);

/* Bytes of the workspace tsa_sample_tokens_ws takes for `batch` rows of
 * `vocab` logits; 0 when such a batch never splits its rows. */
size_t tsa_sample_tokens_workspace_bytes(int64_t batch, int64_t vocab);

/* sample_tokens (server/model/sampling.py:119-194), as tsa_sample_tokens,
 * with a workspace (256-byte aligned, at least
 * tsa_sample_tokens_workspace_bytes(B, V) bytes, contents arbitrary; NULL:
 * tsa_sample_tokens). For a batch of at most 256 rows of at least 16384
 * bf16/f16 logits in 16-byte aligned rows, the rows that take the histogram
 * path (temperature > 0 and not top-k/greedy candidate rows: the server's
 * default top-p request among them) have their statistics and histogram
 * passes spread over several workgroups per row (two more launches on
 * `stream`); for batches of up to about 85 such rows the histogram pass
 * also leaves each segment's elements sorted by bucket in the workspace,
 * and the decision gathers from those lists (about 32 MB of workspace at
 * 64 x 151936). The tokens are those of tsa_sample_tokens. Calls that
 * share a workspace must be ordered on one stream. */
int tsa_sample_tokens_ws(const tsa_view* out, const tsa_view* logits, const tsa_view* temperature,
                         const tsa_view* top_k, const tsa_view* top_p, const tsa_view* uniforms,
                         void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TSA_API_H */
