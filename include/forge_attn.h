/*
 * forge_attn.h -- C ABI of the MI355X (gfx950) attention hot path of Sleuth FORGE.
 *
 * Every entry point takes plain device pointers, element strides and scalars, launches
 * on the HIP stream it is given (`stream` is a hipStream_t passed as void*), never
 * allocates, frees or synchronises, and is safe to record into a HIP graph: positions
 * may come from device memory (`row_pos`, `pos_dev`) instead of host integers.
 *
 * Status codes: 0 = launched; < 0 = the arguments were rejected before anything was
 * launched (forge_last_error() returns the reason, per calling thread); > 0 = the
 * hipError_t the launch reported.
 *
 * Tensor conventions (names as in the reference):
 *   B batch, H query heads, K key/value heads (H % K == 0, head h reads KV head h / (H/K)),
 *   T new tokens, D head dim, S keys visible.
 *   q   [B, H, T, D]  any strides, last dim contiguous (the transposed q_proj view)
 *   k,v [B, K, T, D]  new keys/values, same rules
 *   cache [B, K, max_len, D] (kv_cache.py:31-32), last dim contiguous
 *   out [B, T, H, D]  (the `y.transpose(1, 2)` layout that o_proj reads, attention.py:155-157)
 *   cos/sin: fp32 tables of rows of D values (rope.py:21-38), addressed per (b, t) with
 *   strides (s_cos_b may be 0 when every row shares the positions).
 *
 * Write positions: token t of batch row b sits at absolute position base_b + t, where
 *   base_b = row_pos[b] if row_pos != NULL (per-row lengths, ragged batches),
 *          else *pos_dev if pos_dev != NULL (StaticKVCache.pos_t, kv_cache.py:90),
 *          else pos0 (KVCache.pos, kv_cache.py:34).
 */
#ifndef FORGE_ATTN_H
#define FORGE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FORGE_ABI_VERSION 3

/* dtype codes */
#define FORGE_F32 0
#define FORGE_BF16 1
#define FORGE_F16 2

/* flags */
#define FORGE_NORM_QK 1 /* per-head RMSNorm of q and k (optional gain) */
#define FORGE_ROPE 2    /* NEOX rotate-half RoPE of q and k */
#define FORGE_NORM_V 4  /* per-head RMSNorm of v without gain (cfg.v_norm) */

/* Library version, for the host's compatibility check. */
int forge_abi_version(void);

/* Text of the last rejected call on this thread ("" if none). */
const char* forge_last_error(void);

/*
 * Per-row RMSNorm (optional gain) then NEOX RoPE, fp32 math, one rounding to the
 * tensor's dtype.  Replaces fused_ops.head_norm_rope (fused_ops.py:101-121; kernel
 * _head_kernel fused_ops.py:53-85): x [B,H,T,D] -> y with its own strides.
 * weight: fp32 [D] or NULL; norm: 0/1; cos/sin NULL = no RoPE.
 */
int forge_head_norm_rope(int dtype, const void* x, void* y, int B, int H, int T, int D,
                         int64_t sxb, int64_t sxh, int64_t sxt, int64_t syb, int64_t syh,
                         int64_t syt, const float* weight, float eps, int norm,
                         const float* cos, const float* sin, int64_t s_cos_b, int64_t s_cos_t,
                         void* stream);

/*
 * The K/V half of Attention.forward before SDPA (attention.py:109-130): k -> RMSNorm
 * (FORGE_NORM_QK, gain k_weight) -> RoPE (FORGE_ROPE); v -> RMSNorm without gain
 * (FORGE_NORM_V) -- and the cache write KVCache.update (kv_cache.py:52-60: slice-assign
 * at pos) / StaticKVCache.update (kv_cache.py:107-114: index_copy_ at pos_t + arange(T)).
 * k_dst/v_dst: cache tensors [B,K,dst_len,D] with strides (sdb, sdh, sds); token t of
 * row b goes to position base_b + t (see above); positions >= dst_len are not written.
 */
int forge_kv_append(int dtype, int B, int T, int K, int D, const void* k, int64_t skb,
                    int64_t skh, int64_t skt, const void* v, int64_t svb, int64_t svh,
                    int64_t svt, void* k_dst, void* v_dst, int64_t sdb, int64_t sdh,
                    int64_t sds, int64_t dst_len, const int32_t* row_pos,
                    const int64_t* pos_dev, int64_t pos0, const float* k_weight, float eps,
                    int flags, const float* cos, const float* sin, int64_t s_cos_b,
                    int64_t s_cos_t, void* stream);

/*
 * Split-K ("flash-decoding") attention of T new queries per row against the cache:
 * decode (T = 1, attention.py:189-191), the speculative verify step (T = k+1,
 * attention.py:192-193 with _mask 160-169), the CUDA-graph static step
 * (attention.py:134-141 with StaticKVCache.attn_mask, kv_cache.py:116-128), and any
 * other T (it is the general path: fp32, odd head sizes, device positions).
 * Query t of row b sits at position base_b + t and sees keys
 * [max(0, pos - window + 1), pos]  (window 0 = all), i.e. kv_len_b = base_b + T.
 * q is the RAW projection when flags has FORGE_NORM_QK / FORGE_ROPE (norm + RoPE are
 * fused into the q load, gain q_weight), else already normalised.
 * max_kv_len: host upper bound on kv_len_b (sizes the grid); chunk: keys per split
 * (0 = forge_attn_decode_chunk over the span a row can see: window + 16 when a window
 * is shorter than max_kv_len, else max_kv_len). Rows are computed independently and a
 * key's contribution does not depend on T, so a verify row equals the decode of that
 * token alone bit for bit when both use the same chunk (pass the chunk explicitly, or
 * the same max_kv_len, to guarantee that).
 * workspace: device memory of forge_attn_decode_workspace_bytes(...) bytes (fp32 split-K
 * partials, and a work counter that the call zeroes on its own stream before use); calls
 * that may run at the same time need separate workspaces.
 */
int forge_attn_decode(int dtype, int B, int T, int H, int K, int D, const void* q,
                      int64_t sqb, int64_t sqh, int64_t sqt, const float* q_weight, float eps,
                      int flags, const float* cos, const float* sin, int64_t s_cos_b,
                      int64_t s_cos_t, const void* k_cache, const void* v_cache, int64_t skb,
                      int64_t skh, int64_t sks, int64_t max_len, const int32_t* row_pos,
                      const int64_t* pos_dev, int64_t pos0, int64_t max_kv_len, int window,
                      float scale, int chunk, void* out, int64_t sob, int64_t sot, int64_t soh,
                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * forge_kv_append followed by forge_attn_decode, in one launch where the shape allows:
 * the new tokens' raw keys k and values v [B,K,T,D] (strides sknb.., svnb..) are
 * normalised/rotated (kv_flags: FORGE_NORM_QK with gain k_weight and FORGE_ROPE for the
 * keys, FORGE_NORM_V for the values; the same cos/sin rows as q), written into the caches
 * at base_b + t (KVCache.update, kv_cache.py:52-60; StaticKVCache.update 107-114), and
 * attended to: the split-K unit whose chunk holds a new position makes that key and value,
 * writes them and then streams its chunk. The keys, values and outputs are those of the two
 * calls, bit for bit. Where a KV head's G*T query rows need more than one row block (8 rows
 * on the split-K path, 32 on the wide-group MFMA path: G >= 4, bf16/fp16, D 128/256) or a
 * lane group would hold more than two new keys, it issues forge_kv_append's kernel first.
 * Other arguments and the workspace as forge_attn_decode. ws_flags = FORGE_WS_ZEROED
 * promises that the workspace's first 4 bytes (the persistent grid's work ticket) hold zero,
 * which saves the small kernel that otherwise zeroes them; every call leaves them zero, so a
 * workspace cleared once before its first use keeps the promise for the calls that follow it
 * on one stream.
 * With device-held positions (row_pos or pos_dev), max_kv_len must be at least base_b + T
 * for every row: the launch covers the keys below max_kv_len only, so a new key or value at
 * a position at or past max_kv_len is not written (forge_kv_append writes up to max_len).
 * With pos0 the call raises max_kv_len to pos0 + T itself.
 */
#define FORGE_WS_ZEROED 1 /* ws_flags: the workspace's first 4 bytes hold zero */
int forge_attn_decode_append(int dtype, int B, int T, int H, int K, int D, const void* q,
                             int64_t sqb, int64_t sqh, int64_t sqt, const float* q_weight,
                             float eps, int flags, const void* k, int64_t sknb, int64_t sknh,
                             int64_t sknt, const void* v, int64_t svnb, int64_t svnh,
                             int64_t svnt, const float* k_weight, int kv_flags,
                             const float* cos, const float* sin, int64_t s_cos_b,
                             int64_t s_cos_t, void* k_cache, void* v_cache, int64_t skb,
                             int64_t skh, int64_t sks, int64_t max_len, const int32_t* row_pos,
                             const int64_t* pos_dev, int64_t pos0, int64_t max_kv_len,
                             int window, float scale, int chunk, void* out, int64_t sob,
                             int64_t sot, int64_t soh, void* workspace, size_t workspace_bytes,
                             int ws_flags, void* stream);
/*
 * Allocation-free forge_attn_decode (no counterpart in the reference). For callers that
 * cannot allocate device memory: code under graph capture that may not call hipMalloc,
 * tight serving loops, harnesses that forbid allocation. Same arguments and results as
 * forge_attn_decode (bit for bit, same chunk) without the workspace: the split-K partials
 * and the work ticket live in a device array inside the library, FORGE_NOALLOC_SCRATCH_BYTES
 * per device, held from the library's load until the process ends. A call that needs more
 * (forge_attn_decode_workspace_bytes > FORGE_NOALLOC_SCRATCH_BYTES) is rejected (< 0) before
 * anything is launched. It calls no allocator. Every call on one device uses that device's
 * one array: calls that may overlap on a device (other streams, no ordering between them)
 * race; calls ordered on one stream do not.
 */
#define FORGE_NOALLOC_SCRATCH_BYTES (48 * 1024 * 1024)
int forge_attn_decode_noalloc(int dtype, int B, int T, int H, int K, int D, const void* q,
                              int64_t sqb, int64_t sqh, int64_t sqt, const float* q_weight,
                              float eps, int flags, const float* cos, const float* sin,
                              int64_t s_cos_b, int64_t s_cos_t, const void* k_cache,
                              const void* v_cache, int64_t skb, int64_t skh, int64_t sks,
                              int64_t max_len, const int32_t* row_pos, const int64_t* pos_dev,
                              int64_t pos0, int64_t max_kv_len, int window, float scale,
                              int chunk, void* out, int64_t sob, int64_t sot, int64_t soh,
                              void* stream);

/* Keys per split for a row span of max_kv_len keys (pure host function): the rule for
 * per-row positions (row_pos), whose ragged rows need chunks short enough to balance. The
 * cap is max(1024, 16 block iterations) keys: 1024 for most shapes, 2048 at D 32 in
 * bf16/fp16 (128 keys per block iteration); the MFMA path on more than 512 rows takes at
 * most 512. T is accepted for the signature but does not enter, so decode and verify steps
 * of one layer agree. Size buffers with forge_attn_decode_workspace_bytes, not the cap. */
int forge_attn_decode_chunk(int dtype, int B, int T, int H, int K, int D, int64_t max_kv_len);

/* Keys per split for calls whose rows all start at one position (pos0 or pos_dev, no
 * row_pos): every row has the same length, so the split only has to spread the work over
 * the CUs, and rows are not split at all when the (row, KV head) pairs already fill them.
 * Use it for such calls in place of forge_attn_decode_chunk (no counterpart in the
 * reference: a tuning query, like forge_attn_decode_chunk). T does not enter. */
int forge_attn_decode_chunk_uniform(int dtype, int B, int T, int H, int K, int D,
                                    int64_t max_kv_len);

/* Workspace bytes forge_attn_decode needs (pure host function). */
size_t forge_attn_decode_workspace_bytes(int dtype, int B, int T, int H, int K, int D,
                                         int64_t max_kv_len, int chunk);

/*
 * Causal prefill on bf16/fp16 MFMA (flash attention): SDPA with is_causal
 * (attention.py:187-188) or with the chunked-prefill mask at an offset
 * (attention.py:192-193, _mask 160-169), sliding window included.
 * Queries are at positions offset .. offset+T-1; k/v [B,K,offset+T,D] (normally the
 * cache, already normalised by forge_kv_append) with strides (skb, skh, sks).
 * q is raw when flags has FORGE_NORM_QK / FORGE_ROPE: norm + RoPE run in the Q tile load.
 * Supports D in {64, 128, 256}; returns < 0 for other shapes (use forge_attn_decode).
 */
int forge_attn_prefill(int dtype, int B, int T, int H, int K, int D, const void* q,
                       int64_t sqb, int64_t sqh, int64_t sqt, const float* q_weight,
                       float eps, int flags, const float* cos, const float* sin,
                       int64_t s_cos_t, const void* k, const void* v, int64_t skb,
                       int64_t skh, int64_t sks, int64_t offset, int window, float scale,
                       void* out, int64_t sob, int64_t sot, int64_t soh, void* stream);

/*
 * forge_attn_prefill with document masking: the reference's `same_doc` mask, causal and only
 * within a document (transformer.py:271-275 builds it from doc_ids, attention.py:184-186
 * applies it), for forward passes over packed windows such as scoring. doc_start[b * s_doc_b
 * + t] is the position of the first token of query t's document; the documents of a row are
 * contiguous runs, so doc_start is non-decreasing in t and doc_start <= offset + t (the
 * caller checks both). Query t then sees keys [max(doc_start, window bound), offset + t].
 */
int forge_attn_prefill_docs(int dtype, int B, int T, int H, int K, int D, const void* q,
                            int64_t sqb, int64_t sqh, int64_t sqt, const float* q_weight,
                            float eps, int flags, const float* cos, const float* sin,
                            int64_t s_cos_t, const void* k, const void* v, int64_t skb,
                            int64_t skh, int64_t sks, int64_t offset, int window, float scale,
                            const int32_t* doc_start, int64_t s_doc_b, void* out, int64_t sob,
                            int64_t sot, int64_t soh, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FORGE_ATTN_H */
