/*
 * mi355x_attn.h - C ABI of the MI355X (gfx950) paged-attention library
 * (libmi355x_attn.so, built from sglang_restomod_amd/csrc).
 *
 * Conventions for every entry point:
 *   - Device pointers, element strides (in elements of the tensor's own dtype,
 *     bytes for fp8), int sizes, float scales, and a hipStream_t passed as void*.
 *     No torch types cross this boundary.
 *   - The caller owns every buffer, outputs and workspaces included. Nothing
 *     here allocates, frees or synchronises the host; every launch is enqueued
 *     on `stream`, so the calls can be captured into a HIP graph.
 *   - Return 0 (MA_OK) or a negative status; ma_last_error() then holds a
 *     message for the calling thread. Stateless and thread-safe.
 *
 * KV addressing ("token table"): the KV caches are SGLang's flat token pools
 * [slots, num_kv_heads, head_dim] (any row/head stride, head_dim contiguous).
 * Token `pos` of sequence b lives in pool row
 *     table[r * table_stride + (pos >> log2(page_size))] * page_size + (pos & (page_size - 1)),
 *     r = row_index ? row_index[b] : b.
 * With page_size 1, table = req_to_token and row_index = req_pool_indices this
 * is SGLang's slot lookup; with a page table [B, max_pages] and row_index NULL it
 * is the paged layout [pages, page_size, Hkv, D] of the reference's kernels.
 * The table must cover every position below seq_lens[b]. A KV row (one slot's
 * num_kv_heads x head_dim) must stay below 4 GiB of stride: the kernels multiply
 * slots by it in 32 bits (MA_EUNSUPPORTED otherwise).
 *
 * Score scale is softmax_scale * k_scale; outputs are multiplied by v_scale
 * (sglang_restomod/attention/v100/tilelang/_paged_adapter.py:658,753-754).
 * Query head h reads kv head h / (num_q_heads / num_kv_heads).
 *
 * Head dims of the attention entry points: every multiple of 16 from 16 to 512, with
 * every KV dtype (the reference's paged kernels take any head dim: configurations for
 * 64, 128, 256 and 512 and a default for the rest, _kernels_paged.py:397-418). 64, 128
 * and 256 run on the split-KV and tiled extend kernels; the others on one kernel that
 * serves decode, verify and extend rows alike (16 rows per wave; a decode also splits each
 * sequence's keys over several workgroups when the batch alone would leave compute units
 * idle). Other head dims return MA_EUNSUPPORTED.
 */
#ifndef MI355X_ATTN_H
#define MI355X_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MA_ABI_VERSION 10

/* dtype codes */
#define MA_DT_F16 0
#define MA_DT_BF16 1
#define MA_DT_E4M3 2 /* OCP e4m3fn, stored as bytes */
#define MA_DT_E5M2 3 /* OCP e5m2, stored as bytes */
#define MA_DT_F32 4  /* output only: the attention result before its cast to 16 bits */

/* status codes */
#define MA_OK 0
#define MA_EINVAL (-1)
#define MA_ELAUNCH (-2)
#define MA_EUNSUPPORTED (-3)

/* Message for the last failing call on this thread ("" if none yet). */
const char* ma_last_error(void);

/* MA_ABI_VERSION of the loaded library. */
int ma_abi_version(void);

/* gcnArchName of the current device into buf (for load-time checks). */
int ma_device_arch(char* buf, int len);

/*
 * Number of compute units of the current device: the default persistent grid size
 * (`num_workgroups`) of the split-KV entry points.
 */
int ma_device_workgroups(void);

/*
 * Bytes of workspace the split-KV entry points need for a persistent grid of
 * `num_workgroups` workgroups (1..16384): one descriptor per wave, then the partial
 * results of segments shared by several waves. No initialisation is needed; calls
 * that overlap in time must use different workspaces. At the head dims other than 64,
 * 128 and 256 it holds only the key pieces of a split decode (2 * num_workgroups
 * pieces of 16 rows); there a decode given no workspace runs without the split, and
 * verify uses none.
 */
size_t ma_splitkv_workspace_bytes(int num_workgroups, int head_dim);

/*
 * Grouped split-KV decode: one query token per sequence.
 * Replaces grouped_decode_forward (sglang_restomod/attention/v100/tilelang/
 * _paged_adapter.py:402-486) with its partial and combine kernels
 * (_kernels_paged_decode.py:41-312), and serves the decode that the V100
 * backend hands to Triton at other shapes (flash_attn_v100_backend.py:1093-1115).
 *   q   [batch, num_q_heads, head_dim], q_dtype MA_DT_F16 / MA_DT_BF16
 *   k/v pools as above; kv_dtype = q_dtype, MA_DT_E4M3 or MA_DT_E5M2
 *   seq_lens [batch] int32: keys of each sequence (0 gives a zero output)
 *   sliding_window: -1 for none, else keys >= seq_len - 1 - window only
 *   max_seq_len: an upper bound of seq_lens the caller knows without reading the device
 *     (the engine's host copy of the lengths), or 0 for none. It only chooses the kernels:
 *     a batch whose split-KV work is small (a few thousand 32-key tiles at this bound)
 *     runs as one pass of the any-head-dim kernel over key pieces plus a merge, which
 *     has a shorter critical path; the result does not depend on it (each piece is a
 *     share of its sequence's own keys), so a wrong bound costs time, never correctness.
 *   num_workgroups: persistent grid size (ma_device_workgroups() fills the chip); the
 *     key axis of every (sequence, kv head) is cut into 32-token tiles and each wave
 *     takes an equal contiguous share of all tiles (stream-K, at least 2 tiles per
 *     wave), so ragged lengths balance; a second, short kernel merges the pieces of
 *     segments that several waves shared.
 *   workspace: ma_splitkv_workspace_bytes(num_workgroups, head_dim) bytes, 256-byte
 *     aligned
 *   out [batch, num_q_heads, head_dim] in out_dtype: q_dtype, or MA_DT_F32 for the result
 *     before its rounding to 16 bits (strides in elements of out_dtype)
 */
int ma_grouped_decode(const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype,
                      const void* k_cache, const void* v_cache, int64_t kv_stride_row,
                      int64_t kv_stride_head, int kv_dtype, const int32_t* table,
                      int64_t table_stride, const int64_t* row_index, int page_size,
                      const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads,
                      int head_dim, int num_workgroups, float softmax_scale, float k_scale,
                      float v_scale, int sliding_window, int max_seq_len, void* workspace,
                      size_t workspace_bytes, void* out, int out_dtype, int64_t out_stride_tok,
                      int64_t out_stride_head, void* stream);

/*
 * Allocation-free variant of ma_grouped_decode. No counterpart in the reference: it is for
 * callers that cannot allocate device memory, not even a workspace (code under HIP graph
 * capture that may not call hipMalloc, tight serving loops, harnesses that forbid it).
 * Same arguments and results as ma_grouped_decode minus the workspace: the split-KV
 * partials go to a static scratch array in the library's device code (one copy per GPU,
 * held from the library's first use on that GPU until the process ends) sized for
 * num_workgroups <= MA_NOALLOC_MAX_WORKGROUPS at head_dim <= 256: 67,403,776 bytes, which
 * also holds the key pieces of a split decode at every head dim up to 512.
 * Larger grids return MA_EINVAL. Nothing is allocated or freed; the scratch needs no
 * clearing (every call rewrites what it reads). Calls that overlap in time on one GPU
 * (two streams) share the scratch and race: serialise them.
 */
#define MA_NOALLOC_MAX_WORKGROUPS 256
int ma_grouped_decode_noalloc(const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype,
                              const void* k_cache, const void* v_cache, int64_t kv_stride_row,
                              int64_t kv_stride_head, int kv_dtype, const int32_t* table,
                              int64_t table_stride, const int64_t* row_index, int page_size,
                              const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads,
                              int head_dim, int num_workgroups, float softmax_scale, float k_scale,
                              float v_scale, int sliding_window, int max_seq_len, void* out,
                              int out_dtype, int64_t out_stride_tok, int64_t out_stride_head,
                              void* stream);

/*
 * Grouped split-KV verify: a few query tokens per sequence (linear speculative
 * chain), query row i of sequence b seeing keys j <= prefix_lens[b] + i when causal.
 * Replaces the linear_verify branch of paged_forward
 * (_paged_adapter.py:613-660) and its kernels (_kernels_paged_verify.py:52-433).
 *   q [num_tokens, num_q_heads, head_dim]; query_start_loc [batch+1];
 *   prefix_lens [batch] (NULL: seq_lens - query count); seq_lens [batch] total keys;
 *   max_q_per_seq: the longest chain expected (1..64); it picks the row-group shape
 *     (16 or 32 rows). A sequence with more query tokens is still computed in full.
 *   Query rows are clamped into [0, num_tokens): metadata pointing outside q / out
 *     shortens a sequence instead of addressing memory past the buffers.
 *   num_workgroups / workspace: as for ma_grouped_decode
 */
int ma_paged_verify(const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype,
                    int64_t num_tokens, const void* k_cache, const void* v_cache,
                    int64_t kv_stride_row, int64_t kv_stride_head, int kv_dtype,
                    const int32_t* table, int64_t table_stride, const int64_t* row_index,
                    int page_size, const int32_t* seq_lens, const int32_t* query_start_loc,
                    const int32_t* prefix_lens, int batch, int max_q_per_seq, int num_q_heads,
                    int num_kv_heads, int head_dim, int causal, int sliding_window,
                    int num_workgroups, float softmax_scale, float k_scale, float v_scale,
                    void* workspace, size_t workspace_bytes, void* out, int out_dtype,
                    int64_t out_stride_tok, int64_t out_stride_head, void* stream);

/*
 * Bytes of workspace ma_paged_extend needs for `num_tokens` query tokens in `batch`
 * sequences: the work list, one 8-byte entry per row tile. Row tiles have 256 rows at
 * head_dim 64 and 128 and 128 rows at 256; the size covers the smaller tile (at most
 * ceil(num_tokens * G / 128) + batch entries, G = num_q_heads / num_kv_heads), so one
 * workspace serves every head dim. 0 for bad arguments.
 */
size_t ma_extend_workspace_bytes(int64_t num_tokens, int num_q_heads, int num_kv_heads, int batch);

/*
 * Prefix-aware paged extend (chunked prefill), MFMA tiles.
 * Replaces the reference's paged extend kernel (_kernels_paged.py:55-393 via
 * get_paged_kernel, _kernels_paged.py:414-436, called from paged_forward,
 * _paged_adapter.py:567-759): query token i of sequence b (tokens
 * query_start_loc[b] .. query_start_loc[b+1], query_start_loc[batch] <= num_tokens)
 * sees key j < seq_lens[b] with j <= prefix_lens[b] + i when causal, and
 * j >= prefix_lens[b] + i - window when sliding_window >= 0 (a left bound, also for
 * non-causal layers).
 *   prefix_lens NULL: seq_lens - query count.
 *   Query rows are clamped into [0, num_tokens), as for ma_paged_verify.
 *   batch <= 16384. No host-side maximum of the query lengths is needed: a plan kernel
 *   lists the row tiles on the device (reference: max_seq_len from seq_lens.max().item(),
 *   _paged_adapter.py:605-606).
 *   workspace: ma_extend_workspace_bytes(num_tokens, ...) bytes, 256-byte aligned, no
 *   initialisation; calls that overlap in time must use different workspaces.
 *   The new tokens' K/V must already be in the pools.
 *   out [num_tokens, num_q_heads, head_dim] in out_dtype (q_dtype or MA_DT_F32).
 */
int ma_paged_extend(const void* q, int64_t q_stride_tok, int64_t q_stride_head, int q_dtype,
                    int64_t num_tokens, const void* k_cache, const void* v_cache,
                    int64_t kv_stride_row, int64_t kv_stride_head, int kv_dtype,
                    const int32_t* table, int64_t table_stride, const int64_t* row_index,
                    int page_size, const int32_t* seq_lens, const int32_t* query_start_loc,
                    const int32_t* prefix_lens, int batch, int num_q_heads, int num_kv_heads,
                    int head_dim, int causal, int sliding_window, float softmax_scale,
                    float k_scale, float v_scale, void* workspace, size_t workspace_bytes,
                    void* out, int out_dtype, int64_t out_stride_tok, int64_t out_stride_head,
                    void* stream);

/*
 * KV write into the token pools with quantisation on write.
 * Replaces the pool write before every attention call (set_kv_buffer, called at
 * flash_attn_v100_backend.py:1174-1182 and 1038-1046, draft_decode.py:132-139) with
 * SGLang's token-pool semantics: row t of k and v ([num_tokens, num_kv_heads, head_dim],
 * src_dtype MA_DT_F16 / MA_DT_BF16, any token/head stride, head_dim contiguous and a
 * multiple of 8 in 8..2048) is stored at pool slot loc[t] of k_cache / v_cache.
 *   cache_dtype = src_dtype: a copy (scales ignored).
 *   otherwise: if apply_scale, x / scale in fp32 rounded to src_dtype, then cast to the
 *     cache dtype (fp8: round to nearest even; past the largest finite value e4m3fn
 *     gives NaN, e5m2 infinity).
 * Slots outside [0, num_slots) are skipped. Slots must be distinct.
 */
int ma_set_kv_buffer(const void* k, const void* v, int64_t src_stride_tok, int64_t src_stride_head,
                     int src_dtype, const int64_t* loc, int64_t num_tokens, int num_kv_heads,
                     int head_dim, void* k_cache, void* v_cache, int64_t cache_stride_row,
                     int64_t cache_stride_head, int cache_dtype, int64_t num_slots, float k_scale,
                     float v_scale, int apply_scale, void* stream);

/*
 * Token-table rows translated through a slot mapping, on the device.
 * Replaces the sliding-window page-table build (flash_attn_v100_backend.py:460-503:
 * req_to_token rows up to the longest sequence, read with seq_lens.max().item(), then
 * the pool's translate_loc_from_full_to_swa):
 *   out[b * out_stride + j] = mapping[table[r * table_stride + j]] for
 *   j < min(seq_lens[b], width), r = row_index ? row_index[b] : b.
 * mapping is int64 [mapping_len] (the SWA pool's full_to_swa_index_mapping); a slot
 * outside [0, mapping_len) gives 0. Positions from seq_lens[b] on are not written.
 * batch <= 65535; out_stride >= width.
 */
int ma_translate_slots(const int32_t* table, int64_t table_stride, const int64_t* row_index,
                       const int32_t* seq_lens, int batch, const int64_t* mapping, int64_t mapping_len,
                       int32_t* out, int64_t out_stride, int width, void* stream);

/*
 * Key rows of a multi-step speculative draft, on the device.
 * Replaces the per-step draft KV-index build of the reference's draft container
 * (draft_decode.py:172-208, the engine container's common_template)
 * and its per-step page-table conversion (draft_decode_plan.py:42-78). Row
 * r = b * topk + k of out is branch k of request b:
 *   out[r * out_stride + j] = T(b, j)                      for j < seq_lens[b]
 *   out[r * out_stride + j] = T(b, j + k * num_steps)      for seq_lens[b] <= j < seq_lens[b] + num_steps
 *   T(b, p) = table[row * table_stride + p] (0 when p >= table_width), row = row_index ?
 *   row_index[b] : b, passed through mapping (int64 [mapping_len], a slot outside gives 0)
 *   when mapping is not NULL.
 * This is the engine's placement of draft tokens in req_to_token (branch k's num_steps
 * tokens follow the prefix at k * num_steps) for page size 1, or for any page size with
 * topk 1. Draft step i then attends over the first seq_lens[b] + i + 1 entries of each
 * row (ma_grouped_decode with table = out, row_index NULL). Entries from
 * min(seq_lens[b] + num_steps, width) on are not written.
 * batch * topk <= 65535; out_stride >= width; table_stride >= table_width.
 */
int ma_draft_table(const int32_t* table, int64_t table_stride, int table_width, const int64_t* row_index,
                   const int32_t* seq_lens, int batch, int topk, int num_steps, const int64_t* mapping,
                   int64_t mapping_len, int32_t* out, int64_t out_stride, int width, void* stream);

/*
 * fp8 paged KV decoded into fp16 logical pages.
 * Replaces gather_fp8_paged_kv (_paged_adapter.py:527-564, _kernels_fp8_bridge.py:20-70):
 * for logical page p < ceil(seq_lens[b] / page_size) of sequence b, physical page
 * page_table[b * table_stride + p] of k_cache / v_cache (fp8 bytes, [num_pages,
 * page_size, num_kv_heads, head_dim] with the given byte strides) is decoded into page
 * b * max_blocks + p of k_out / v_out (fp16, contiguous [batch * max_blocks, page_size,
 * num_kv_heads, head_dim]). kv_dtype MA_DT_E4M3 or MA_DT_E5M2; decoding is exact (e5m2:
 * the byte shifted into the high half, NaN payloads included). Other output pages and
 * physical pages outside [0, num_pages) are left untouched. head_dim a multiple of 16;
 * caches, outputs and strides 16-byte aligned.
 */
int ma_gather_fp8_paged_kv(const void* k_cache, const void* v_cache, int64_t stride_page, int64_t stride_tok,
                           int64_t stride_head, int kv_dtype, int64_t num_pages, const int32_t* page_table,
                           int64_t table_stride, const int32_t* seq_lens, int batch, int max_blocks,
                           int page_size, int num_kv_heads, int head_dim, void* k_out, void* v_out,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_ATTN_H */
