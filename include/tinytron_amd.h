/*
 * tinytron_amd.h -- C ABI of the MI355X (gfx950) decode-step library.
 *
 * One shared library, libtinytron_amd.so, replaces the per-layer decode path
 * of liangyuwang/Tinytron's Attention.forward
 * (tinytron/model/modules/attn.py:378-440) under the unchanged engine loop
 * (tinytron/inference/engine.py:195-225):
 *
 *   rope_impl(q, k, pos)                      attn.py:397 -> 13-63
 *   gqa_impl(k, v) + cache.append(k, v)       attn.py:308-312, 324-325 -> cache.py:34-45
 *   cache.get_kv() + build_cache_causal_mask  attn.py:326, 332-339 -> cache.py:47-51, attn.py:86-95
 *   F.scaled_dot_product_attention(...)       attn.py:420-423
 *
 * Conventions (every entry point):
 *   - All tensor pointers are device pointers owned by the caller; nothing is
 *     allocated, freed or synchronised inside the library. Work is enqueued
 *     on `stream` (a hipStream_t; NULL = the default stream).
 *   - Strides are in elements. The innermost (head_dim) stride is 1; the
 *     token-slot stride inside a cache page is head_dim.
 *   - Return value: 0 on success; < 0 for an invalid argument (nothing was
 *     launched; tt_last_error_string() says why); > 0 is the hipError_t of a
 *     failed launch.
 *   - The library keeps no mutable global state; calls on different streams
 *     from different threads are independent. tt_last_error_string() is
 *     per thread.
 *
 * KV-cache addressing (shared by append and attention). Token t of sequence
 * b, KV head h, element d lives at element offset
 *     base(b, t / P) + h * cache_strides[2] + (t % P) * head_dim + d
 * with base(b, j) = b * cache_strides[0] + j * cache_strides[1] when
 * page_table == NULL (the reference's contiguous [B, H, ceil(S/P), P, D]
 * store, cache.py:27-32, with H = num_kv_heads), and
 * base(b, j) = page_table[b * max_pages + j] * cache_strides[1] for a paged
 * pool [num_pages, H, P, D] (page_table int32 [B, max_pages]).
 * fp8 caches keep one fp32 scale per (token, KV head). With row r = (element
 * offset of d = 0) / head_dim, the K scale is k_scale[r + 16 * (r / 16)] and
 * the V scale v_scale[r + 16 * (r / 16)]: rows are grouped by 16, and one
 * array of 2 x rows entries (rows rounded up to 16) holds both with
 * v_scale = k_scale + 16, so that each group's 16 K scales and 16 V scales
 * share one 128-byte line. fp8 caches need every 16-token block of a
 * (sequence, head) to start a group: page and head strides (paged pool) or
 * sequence and head strides (contiguous store) multiples of 16 * head_dim.
 */
#ifndef TINYTRON_AMD_H
#define TINYTRON_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TT_ABI_VERSION 7

#define TT_OK 0
#define TT_ERR_INVALID_ARGUMENT (-1)
#define TT_ERR_UNSUPPORTED (-2)
#define TT_ERR_WORKSPACE_TOO_SMALL (-3)

/* split_tokens of the decode attention entry points: one workgroup per
 * (sequence, KV head), merged inside the launch. */
#define TT_SPLIT_PER_SEGMENT (-1)
/* split_tokens of the decode attention entry points: the sequences ranked by
 * length, one workgroup per (rank pair (p, batch - 1 - p), KV head), merged
 * inside the launch; batch <= 256. */
#define TT_SPLIT_PAIRED (-2)

/* A hipStream_t, kept opaque so that the header needs no HIP include. */
typedef void *tt_stream_t;

/* ABI version of the loaded library (TT_ABI_VERSION it was built with). */
int tt_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char *tt_last_error_string(void);

/*
 * Fused RoPE + KV-cache append, bf16 activations and bf16 cache.
 *
 * Replaces, for T new tokens per sequence:
 *   rope_impl(q, k, position_ids)         attn.py:13-63, called at attn.py:397
 *   LayerPagedKVCache.append(k, v)        cache.py:34-45 (called at attn.py:325)
 * with the cache holding num_kv_heads heads (K/V appended before the GQA
 * expansion of attn.py:308-312; the expansion is an index map in attention).
 *
 * q_in  [B, H_q,  T, D], strides q_in_strides  = {b, h, t}
 * k_in  [B, H_kv, T, D], strides k_in_strides  = {b, h, t}
 * v_in  [B, H_kv, T, D], strides v_in_strides  = {b, h, t}
 * q_out [B, H_q,  T, D], strides q_out_strides = {b, h, t} (rotated q)
 * rope_table [rope_table_len, D]: row p = [cos(p*f_0..p*f_{D/2-1}) |
 *   sin(p*f_0..)] in the activation dtype, f_i = 1/theta^(2i/D) (the values
 *   of attn.py:30-54; columns i and i+D/2 of the reference's cos are equal).
 * positions [B] int32: slot of token 0 of sequence b (its length before the
 *   append). Token t goes to slot positions[b] + t and is rotated by that
 *   position.
 * new_lens [B] int32 or NULL: sequence b writes only its first new_lens[b]
 *   tokens to the cache (ragged prefill; the rest are padding). q_out is
 *   rotated for all T tokens either way. NULL = all T.
 * lens_out [B] int32 or NULL: receives positions[b] + (tokens written for
 *   sequence b), i.e. the sequence's length after the append (the
 *   reference's current_length update, cache.py:43-44). It must not alias
 *   positions; callers alternate two length buffers between steps.
 * Each rounding point of the reference under bf16 autocast is reproduced:
 *   out = bf16(bf16(x*cos) + bf16(rotate_half(x)*sin)).
 * Tokens whose slot is >= capacity, >= rope_table_len, or whose page lies
 * outside the page table / pool are skipped (the caller checks overflow and
 * raises, as cache.py:37-40 does).
 */
int tt_rope_append_bf16(const void *q_in, const int64_t q_in_strides[3],
                        const void *k_in, const int64_t k_in_strides[3],
                        const void *v_in, const int64_t v_in_strides[3],
                        void *q_out, const int64_t q_out_strides[3],
                        const void *rope_table, int64_t rope_table_len,
                        const int32_t *positions, const int32_t *new_lens, int32_t *lens_out,
                        const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                        void *k_cache, void *v_cache, const int64_t cache_strides[3],
                        int64_t capacity, int64_t batch, int64_t num_new,
                        int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                        int64_t page_size, tt_stream_t stream);

/*
 * As tt_rope_append_bf16, fp32 activations, table and cache (the reference
 * without autocast, e.g. on its CPU path: engine.py:180-184). Each op rounds
 * to fp32; nothing is fused into an FMA.
 */
int tt_rope_append_f32(const void *q_in, const int64_t q_in_strides[3],
                       const void *k_in, const int64_t k_in_strides[3],
                       const void *v_in, const int64_t v_in_strides[3],
                       void *q_out, const int64_t q_out_strides[3],
                       const void *rope_table, int64_t rope_table_len,
                       const int32_t *positions, const int32_t *new_lens, int32_t *lens_out,
                       const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                       void *k_cache, void *v_cache, const int64_t cache_strides[3],
                       int64_t capacity, int64_t batch, int64_t num_new,
                       int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                       int64_t page_size, tt_stream_t stream);

/*
 * As tt_rope_append_bf16 with an fp8-e4m3fn cache (no counterpart in the
 * reference, whose cache is in the engine dtype, cache.py:19,29-30).
 * Per (token, KV head): absmax = max|x| over D of the rotated bf16 K (of the
 * raw V), scale = absmax / 448 (fp32), code = e4m3fn_rne(x / scale); an
 * all-zero row stores code 0 and scale 0. Scales are written to k_scale /
 * v_scale (fp32, grouped by 16 rows as described at the top).
 */
int tt_rope_append_fp8(const void *q_in, const int64_t q_in_strides[3],
                       const void *k_in, const int64_t k_in_strides[3],
                       const void *v_in, const int64_t v_in_strides[3],
                       void *q_out, const int64_t q_out_strides[3],
                       const void *rope_table, int64_t rope_table_len,
                       const int32_t *positions, const int32_t *new_lens, int32_t *lens_out,
                       const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                       void *k_cache, void *v_cache, float *k_scale, float *v_scale,
                       const int64_t cache_strides[3],
                       int64_t capacity, int64_t batch, int64_t num_new,
                       int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                       int64_t page_size, tt_stream_t stream);

/*
 * As tt_rope_append_bf16 (fp8_cache = 0) / tt_rope_append_fp8 (fp8_cache =
 * 1; k_scale, v_scale as there, NULL for bf16), for a prompt batch packed
 * without padding (the reference's prefill, attn.py:378-423, over ragged
 * prompts): q_in [num_rows, H_q, D], k_in / v_in [num_rows, H_kv, D] with
 * strides {row, head}; token t < new_lens[b] of sequence b is row
 * row_offsets[b] + t (int32 device arrays, both required). q_out keeps the
 * [B, H_q, num_new, D] grid of tt_rope_append_bf16 (strides {b, h, t}); rows
 * t >= new_lens[b] are not written. Input rows are clamped to [0, num_rows).
 * (Packing is this library's; the reference pads every prompt to T.)
 */
int tt_rope_append_rows_bf16(const void *q_in, const int64_t q_in_strides[2], const void *k_in,
                             const int64_t k_in_strides[2], const void *v_in, const int64_t v_in_strides[2],
                             const int32_t *row_offsets, int64_t num_rows, void *q_out, const int64_t q_out_strides[3],
                             const void *rope_table, int64_t rope_table_len, const int32_t *positions,
                             const int32_t *new_lens, int32_t *lens_out, const int32_t *page_table, int64_t max_pages,
                             int64_t num_pages, void *k_cache, void *v_cache, float *k_scale, float *v_scale,
                             const int64_t cache_strides[3], int64_t capacity, int64_t batch, int64_t num_new,
                             int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                             int fp8_cache, tt_stream_t stream);

/*
 * As tt_rope_append_bf16 / tt_rope_append_fp8, with q, k and v read from the
 * fp32 split-K partials of their projection (tt_linear_splitk*_bf16): each
 * input element is bf16(sum over s < splits of in[s * split_stride + i]),
 * added in order -- the projection's bf16 output, so the cache bytes equal
 * those of tt_splitk_reduce_bf16 followed by tt_rope_append_*. Strides are
 * in fp32 elements within one split. (Fuses the projection's reduction into
 * the append; no counterpart in the reference.)
 */
int tt_rope_append_partials_bf16(const float *q_in, const int64_t q_in_strides[3],
                                 const float *k_in, const int64_t k_in_strides[3],
                                 const float *v_in, const int64_t v_in_strides[3],
                                 int64_t splits, int64_t split_stride,
                                 void *q_out, const int64_t q_out_strides[3],
                                 const void *rope_table, int64_t rope_table_len,
                                 const int32_t *positions, const int32_t *new_lens, int32_t *lens_out,
                                 const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                                 void *k_cache, void *v_cache, const int64_t cache_strides[3],
                                 int64_t capacity, int64_t batch, int64_t num_new,
                                 int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                 int64_t page_size, tt_stream_t stream);

int tt_rope_append_partials_fp8(const float *q_in, const int64_t q_in_strides[3],
                                const float *k_in, const int64_t k_in_strides[3],
                                const float *v_in, const int64_t v_in_strides[3],
                                int64_t splits, int64_t split_stride,
                                void *q_out, const int64_t q_out_strides[3],
                                const void *rope_table, int64_t rope_table_len,
                                const int32_t *positions, const int32_t *new_lens, int32_t *lens_out,
                                const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                                void *k_cache, void *v_cache, float *k_scale, float *v_scale,
                                const int64_t cache_strides[3],
                                int64_t capacity, int64_t batch, int64_t num_new,
                                int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                int64_t page_size, tt_stream_t stream);

/*
 * GQA decode attention over a ragged batch, bf16 cache, split-K
 * (flash-decoding) with a merge pass.
 *
 * Replaces, for one new token per sequence (T = 1):
 *   cache.get_kv()                             cache.py:47-51
 *   gqa_impl expansion (q head h reads KV head h / (H_q/H_kv))  attn.py:66-83
 *   build_cache_causal_mask (all True for T=1) attn.py:86-95, 332-339
 *   F.scaled_dot_product_attention(q, K, V, attn_mask, dropout_p=0)  attn.py:420-423
 *
 * q   [B, H_q, D] bf16 (rotated), strides q_strides = {b, h}
 * seq_lens [B] int32: number of cached tokens sequence b attends to
 *   (including the token just appended); values are clamped to max_seq_len.
 * max_seq_len: host-side upper bound of seq_lens (sizes the launch grid).
 * out [B, H_q, D] bf16, strides out_strides = {b, h}. A sequence with
 *   seq_lens[b] <= 0 gets zeros.
 * sm_scale: softmax scale (1/sqrt(D) for the reference's SDPA default).
 * split_tokens: 0 = balanced partition: the 32-token tiles of all
 *   (sequence, KV head) pairs are dealt out in equal contiguous runs to the
 *   resident waves, whatever the length mix, and a second launch merges each
 *   pair's pieces (bf16 and fp8; fp32 uses the automatic fixed split);
 *   TT_SPLIT_PER_SEGMENT (-1) = one workgroup per (sequence, KV head) pair,
 *   its 4 waves taking equal quarters of the pair's tiles and merging in LDS:
 *   one launch, no workspace; correct for any lengths, balanced when every
 *   sequence has the same length and batch * num_kv_heads fills whole rounds
 *   of the GPU (tt_decode_pick_split says when);
 *   TT_SPLIT_PAIRED (-2) = the sequences ranked by length (longest first,
 *   ties by index), one workgroup per KV head and rank pair (p,
 *   batch - 1 - p) (the middle rank of an odd batch alone), its waves taking
 *   equal shares of the two segments' tiles and merging in LDS: one launch,
 *   no workspace, batch <= 256; correct for any lengths, balanced when the
 *   pairs' lengths add up to about the same total and (batch + 1) / 2 *
 *   num_kv_heads fills whole rounds of the GPU (tt_decode_pick_split says
 *   when); the VALU kernel (fp32 caches, head dims the MFMA tiles do not
 *   take) treats -1 and -2 as 0;
 *   128, 256, 512 or 1024 = fixed splits of that many tokens.
 * length_order: NULL, or with TT_SPLIT_PAIRED a device int32 [batch] array
 *   holding the batch's sequence indices ordered by seq_lens, longest first,
 *   ties by the smaller index (a permutation of 0 .. batch - 1; entries are
 *   clamped into that range). Workgroup p then takes the sequences
 *   length_order[p] and length_order[batch - 1 - p] instead of ranking the
 *   lengths itself (which costs each workgroup a few microseconds before its
 *   first tile). The order does not change when every length grows by the
 *   same count, so a decode loop uploads it once per change of its batch.
 *   Ignored by the other partitions.
 * workspace: device scratch of at least tt_decode_workspace_bytes(...) bytes
 *   for the same (batch, num_q_heads, num_kv_heads, head_dim, max_seq_len,
 *   split_tokens); its contents need no initialisation. May be NULL when the
 *   call needs none (TT_SPLIT_PER_SEGMENT and TT_SPLIT_PAIRED on the MFMA
 *   kernels).
 * Requirements: head_dim even and <= 128 (a multiple of 8 for a bf16 cache
 *   or 16 for an fp8 cache runs the MFMA kernels, other head dims and fp32
 *   caches the VALU kernel); H_q % H_kv == 0 and
 *   H_q / H_kv <= 16; a paged pool has a power-of-two page_size >= 16; the
 *   contiguous store has dense pages (cache_strides[1] == page_size *
 *   head_dim, as the reference's [B, H, pages, P, D] store), any page_size,
 *   and holds max_seq_len tokens per (sequence, head): cache_strides[2] >=
 *   max_seq_len * head_dim when num_kv_heads > 1 and cache_strides[0] >=
 *   max_seq_len * head_dim when batch > 1;
 *   q and cache 16-byte aligned, their strides multiples of 8 elements;
 *   batch <= 4096 (bf16 / fp8).
 * Physical page numbers read from page_table are clamped into
 *   [0, num_pages) so that a bad table cannot address outside the pool.
 */
int tt_gqa_decode_attn_bf16(const void *q, const int64_t q_strides[2],
                            const void *k_cache, const void *v_cache,
                            const int64_t cache_strides[3],
                            const int32_t *seq_lens, int64_t max_seq_len,
                            const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                            void *out, const int64_t out_strides[2],
                            int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                            int64_t head_dim, int64_t page_size, float sm_scale,
                            int64_t split_tokens, const int32_t *length_order,
                            void *workspace, size_t workspace_bytes, tt_stream_t stream);

/*
 * As tt_gqa_decode_attn_bf16 with an fp8-e4m3fn cache and per-(token, head)
 * fp32 scales (layout as in tt_rope_append_fp8). Dequantisation is
 * float(code) * scale inside the kernel with fp32 accumulation; q and out
 * stay bf16. (No counterpart in the reference.)
 */
int tt_gqa_decode_attn_fp8(const void *q, const int64_t q_strides[2],
                           const void *k_cache, const void *v_cache,
                           const float *k_scale, const float *v_scale,
                           const int64_t cache_strides[3],
                           const int32_t *seq_lens, int64_t max_seq_len,
                           const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                           void *out, const int64_t out_strides[2],
                           int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                           int64_t head_dim, int64_t page_size, float sm_scale,
                           int64_t split_tokens, const int32_t *length_order,
                           void *workspace, size_t workspace_bytes, tt_stream_t stream);

/*
 * As tt_gqa_decode_attn_bf16 with fp32 q, cache and out (the reference
 * without autocast), without length_order (the VALU kernel has no paired
 * partition). Requirements as above except that 4-byte alignment suffices.
 */
int tt_gqa_decode_attn_f32(const void *q, const int64_t q_strides[2],
                           const void *k_cache, const void *v_cache,
                           const int64_t cache_strides[3],
                           const int32_t *seq_lens, int64_t max_seq_len,
                           const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                           void *out, const int64_t out_strides[2],
                           int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                           int64_t head_dim, int64_t page_size, float sm_scale,
                           int64_t split_tokens, void *workspace, size_t workspace_bytes,
                           tt_stream_t stream);

/*
 * Prefill attention: causal GQA attention of T new tokens per sequence over
 * the sequence's cache, after tt_rope_append_* has appended them.
 *
 * Replaces the prefill branch of the reference's attention (attn.py:321-341:
 * cache append + get_kv, then F.scaled_dot_product_attention with
 * is_causal=True at past_len 0, or the mask key_pos <= past_len + query_pos,
 * attn.py:86-95) for a ragged batch.
 *
 * q   [B, H_q, T, D] bf16 (rotated), strides q_strides = {b, h, t}
 * positions [B] int32: tokens cached before the new ones (the new token t of
 *   sequence b is at position positions[b] + t and attends keys 0 .. that).
 * new_lens [B] int32 or NULL: new tokens of sequence b (<= T; NULL = T);
 *   output rows t >= new_lens[b] are left untouched.
 * max_seq_len: host-side bound of positions[b] + new_lens[b] (the keys read
 *   are clamped to it).
 * out [B, T, H_q, D] bf16, strides out_strides = {b, t, h}.
 * Requirements as tt_gqa_decode_attn_bf16 (G <= 16, ...), with head_dim a
 * multiple of 8 (bf16 cache) or 16 (fp8 cache), <= 128.
 */
int tt_prefill_attn_bf16(const void *q, const int64_t q_strides[3],
                         const void *k_cache, const void *v_cache, const int64_t cache_strides[3],
                         const int32_t *positions, const int32_t *new_lens, int64_t max_seq_len,
                         const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                         void *out, const int64_t out_strides[3],
                         int64_t batch, int64_t num_new, int64_t num_q_heads, int64_t num_kv_heads,
                         int64_t head_dim, int64_t page_size, float sm_scale, tt_stream_t stream);

/* As tt_prefill_attn_bf16 with an fp8-e4m3fn cache and per-(token, head) scales. */
int tt_prefill_attn_fp8(const void *q, const int64_t q_strides[3],
                        const void *k_cache, const void *v_cache,
                        const float *k_scale, const float *v_scale, const int64_t cache_strides[3],
                        const int32_t *positions, const int32_t *new_lens, int64_t max_seq_len,
                        const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                        void *out, const int64_t out_strides[3],
                        int64_t batch, int64_t num_new, int64_t num_q_heads, int64_t num_kv_heads,
                        int64_t head_dim, int64_t page_size, float sm_scale, tt_stream_t stream);

/*
 * One decode step of attention with this step's RoPE + KV append folded into
 * the attention launch: the result equals tt_rope_append_bf16 (one new token
 * per sequence at position positions[b], lens_out = positions + 1) followed
 * by tt_gqa_decode_attn_bf16 (split_tokens 0) over seq_lens = positions + 1,
 * without the rotated q being written out. Replaces attn.py:397 (rope_impl),
 * 308-312 + cache.py:41-44 (append) and attn.py:420-423 (SDPA) for T = 1.
 * q_in / k_in / v_in are [B, H, D] with element strides {batch, head}: bf16
 * activations (splits == 0), or with 1 <= splits <= 4 fp32 split-K partials
 * of the projection (split stride split_stride), each element the bf16 sum of
 * the splits in order. The wave that reads a segment's last tile writes that
 * segment's new k / v first, so no other launch is needed. max_seq_len must
 * bound positions[b] + 1 and the cache capacity. split_tokens: 0 (balanced
 * partition), TT_SPLIT_PER_SEGMENT or TT_SPLIT_PAIRED, and length_order
 * (ordered by positions), as for tt_gqa_decode_attn_bf16 (bf16 / fp8
 * caches); workspace as
 * tt_decode_workspace_bytes(..., split_tokens) (NULL for the two one-launch
 * partitions).
 */
int tt_decode_attn_append_bf16(const void *q_in, const int64_t q_in_strides[2], const void *k_in,
                               const int64_t k_in_strides[2], const void *v_in, const int64_t v_in_strides[2],
                               int64_t splits, int64_t split_stride, const void *rope_table, int64_t rope_table_len,
                               const int32_t *positions, int32_t *lens_out, int64_t max_seq_len,
                               const int32_t *page_table, int64_t max_pages, int64_t num_pages, void *k_cache,
                               void *v_cache, const int64_t cache_strides[3], int64_t capacity, void *out,
                               const int64_t out_strides[2], int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                               int64_t head_dim, int64_t page_size, float sm_scale, int64_t split_tokens,
                               const int32_t *length_order, void *workspace, size_t workspace_bytes,
                               tt_stream_t stream);

/* As tt_decode_attn_append_bf16 with an fp8-e4m3fn cache (per-(token, head) scales written by the append). */
int tt_decode_attn_append_fp8(const void *q_in, const int64_t q_in_strides[2], const void *k_in,
                              const int64_t k_in_strides[2], const void *v_in, const int64_t v_in_strides[2],
                              int64_t splits, int64_t split_stride, const void *rope_table, int64_t rope_table_len,
                              const int32_t *positions, int32_t *lens_out, int64_t max_seq_len,
                              const int32_t *page_table, int64_t max_pages, int64_t num_pages, void *k_cache,
                              void *v_cache, float *k_scale, float *v_scale, const int64_t cache_strides[3],
                              int64_t capacity, void *out, const int64_t out_strides[2], int64_t batch,
                              int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                              float sm_scale, int64_t split_tokens, const int32_t *length_order, void *workspace,
                              size_t workspace_bytes, tt_stream_t stream);

/*
 * One fused bf16 decode step of a layer, as the library's kernels run it
 * (gpt.py:98-109 with attn.py:378-440, mlp.py:24-26 + 44-45 and norm.py:6-19
 * per layer, the reference's Block.forward for T = 1 under bf16 autocast):
 *   P  = h . Wqkv^T                       split-K partials (kc_qkv-wide chunks)
 *   y  = attention step from P            tt_decode_attn_append_bf16 / _fp8
 *                                         (RoPE, append, attention; positions ->
 *                                         lens_out)
 *   P  = y . Wo^T                          split-K partials (kc_o)
 *   h  = RMSNorm_2(x += bf16(sum P))       tt_add_rmsnorm_bf16
 *   a  = SwiGLU(h . Wg^T, h . Wu^T)        one launch (kc_gu 0: tt_linear_swiglu_packed_bf16)
 *                                         or split-K partials (kc_gu) + tt_silu_mul_bf16
 *   P  = a . Wd^T                          split-K partials (kc_down)
 *   h  = RMSNorm_next(x += bf16(sum P))    the next layer's first norm (or the final one)
 * Every step is the entry point named beside it with these arguments, so the
 * results equal those calls made one by one, bit for bit; this entry point
 * issues them from the host in one call (a decode step's ~170 launches cost
 * the host ~0.5 ms instead of ~1.7 ms through per-call bindings), so an eager
 * decode loop keeps ahead of the GPU. No counterpart in the reference.
 * Weights are the packed fragment-order layouts (w_gu rows interleaved by 8
 * for the one-launch SwiGLU); h / attn_out / act are bf16 row-major
 * [batch, hidden] / [batch, num_q_heads * head_dim] / [batch, intermediate];
 * partials holds the largest split-K product of the layer.
 */
typedef struct tt_decode_layer {
  float *x;                 /* fp32 residual [batch, hidden], updated in place */
  void *h;                  /* bf16 [batch, hidden]: in: this layer's norm-1 output; out: the next norm's */
  float *partials;          /* fp32 split-K scratch */
  void *attn_out;           /* bf16 [batch, num_q_heads * head_dim] */
  void *act;                /* bf16 [batch, intermediate] */
  const void *w_qkv, *w_o, *w_gu, *w_down;
  const float *ln2_weight, *next_norm_weight;
  float eps;
  int64_t batch, hidden, intermediate, num_q_heads, num_kv_heads, head_dim;
  int64_t kc_qkv, kc_o, kc_gu, kc_down;
  int32_t fp8_cache;        /* 0: bf16 cache; 1: fp8-e4m3fn cache with k_scale / v_scale */
  const void *rope_table;
  int64_t rope_table_len;
  const int32_t *positions; /* tokens cached before the step, [batch] */
  int32_t *lens_out;        /* positions + 1 after the step, or NULL */
  const int32_t *page_table;
  int64_t max_pages, num_pages;
  void *k_cache, *v_cache;
  float *k_scale, *v_scale;
  int64_t cache_strides[3];
  int64_t capacity, page_size;
  float sm_scale;
  int64_t split_tokens;
  const int32_t *length_order;
  void *workspace;
  size_t workspace_bytes;
} tt_decode_layer_t;

/* layers[0 .. num_layers) in order on one stream, each with the attention
 * launch bound max_seq_len. Stops at the first failing step and returns its
 * status (tt_last_error_string names the layer and the step); the layers
 * before it have run, so their caches already hold the step's token. */
int tt_decode_layers_bf16(const tt_decode_layer_t *layers, int64_t num_layers, int64_t max_seq_len,
                          tt_stream_t stream);

/*
 * tt_decode_attn_append_bf16 without the workspace argument: the attention
 * workspace is a device array inside the library, TT_NOALLOC_SCRATCH_BYTES
 * per GPU, held by every GPU the entry point runs on until the process ends.
 * No counterpart in the reference: this is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, hosts
 * that forbid hipMalloc). The call itself allocates nothing; the caller
 * still passes every input and output. A call whose workspace (tile prefix
 * plus (B * H_kv + waves of the launched grid) * G * (D + 2) fp32 partials)
 * exceeds the scratch returns TT_ERR_WORKSPACE_TOO_SMALL before launching.
 * Every call on one GPU shares that GPU's scratch, which keeps the last
 * call's contents (nothing in it needs to start at zero): calls that overlap
 * on one GPU (different streams, or threads) race and must be serialised by
 * the caller. Results are those of tt_decode_attn_append_bf16, bit for bit.
 */
#define TT_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

int tt_decode_attn_append_bf16_noalloc(const void *q_in, const int64_t q_in_strides[2], const void *k_in,
                                       const int64_t k_in_strides[2], const void *v_in,
                                       const int64_t v_in_strides[2], int64_t splits, int64_t split_stride,
                                       const void *rope_table, int64_t rope_table_len, const int32_t *positions,
                                       int32_t *lens_out, int64_t max_seq_len, const int32_t *page_table,
                                       int64_t max_pages, int64_t num_pages, void *k_cache, void *v_cache,
                                       const int64_t cache_strides[3], int64_t capacity, void *out,
                                       const int64_t out_strides[2], int64_t batch, int64_t num_q_heads,
                                       int64_t num_kv_heads, int64_t head_dim, int64_t page_size, float sm_scale,
                                       tt_stream_t stream);

/*
 * Row attention: `rows` query rows, row r attending to the first
 * row_lens[r] cached tokens of sequence seq_of_row[r] (< num_seqs; the
 * cache holds num_seqs sequences, addressed as in tt_gqa_decode_attn_*).
 * With rows = the new tokens of a prefill chunk (row r = token t of
 * sequence b, row_lens[r] = tokens cached before the chunk + t + 1) this is
 * the prefill branch of the reference attention with its cache-causal mask
 * (attn.py:321-341: build_cache_causal_mask + F.scaled_dot_product_attention
 * after cache.append / get_kv, cache.py:34-51) for the cases the prefill
 * kernel does not take: fp32 caches and activations (the reference's fp32
 * path), and head dims whose rows are not whole 16-byte fragments. Runs the
 * VALU split kernel and its combine; q / out as in tt_gqa_decode_attn_*
 * (strides {row, head}); row_lens[r] <= 0 gives zeros; rows <= 65535;
 * workspace as tt_decode_workspace_bytes(rows, ..., max_row_len,
 * 0).
 */
int tt_rows_attn_bf16(const void *q, const int64_t q_strides[2], const void *k_cache, const void *v_cache,
                      const int64_t cache_strides[3], const int32_t *seq_of_row, const int32_t *row_lens,
                      int64_t max_row_len, const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                      int64_t num_seqs, void *out, const int64_t out_strides[2], int64_t rows, int64_t num_q_heads,
                      int64_t num_kv_heads, int64_t head_dim, int64_t page_size, float sm_scale, void *workspace,
                      size_t workspace_bytes, tt_stream_t stream);
int tt_rows_attn_fp8(const void *q, const int64_t q_strides[2], const void *k_cache, const void *v_cache,
                     const float *k_scale, const float *v_scale, const int64_t cache_strides[3],
                     const int32_t *seq_of_row, const int32_t *row_lens, int64_t max_row_len,
                     const int32_t *page_table, int64_t max_pages, int64_t num_pages, int64_t num_seqs, void *out,
                     const int64_t out_strides[2], int64_t rows, int64_t num_q_heads, int64_t num_kv_heads,
                     int64_t head_dim, int64_t page_size, float sm_scale, void *workspace, size_t workspace_bytes,
                     tt_stream_t stream);
int tt_rows_attn_f32(const void *q, const int64_t q_strides[2], const void *k_cache, const void *v_cache,
                     const int64_t cache_strides[3], const int32_t *seq_of_row, const int32_t *row_lens,
                     int64_t max_row_len, const int32_t *page_table, int64_t max_pages, int64_t num_pages,
                     int64_t num_seqs, void *out, const int64_t out_strides[2], int64_t rows, int64_t num_q_heads,
                     int64_t num_kv_heads, int64_t head_dim, int64_t page_size, float sm_scale, void *workspace,
                     size_t workspace_bytes, tt_stream_t stream);

/* Fixed split size the fp32 entry point uses when split_tokens == 0. */
int64_t tt_decode_split_tokens(int64_t batch, int64_t num_kv_heads, int64_t max_seq_len);

/* The split_tokens value for a decode attention call over a bf16 (fp8_cache
 * 0) or fp8 cache whose batch holds the host-side lengths seq_lens_host[0 ..
 * batch): TT_SPLIT_PER_SEGMENT when they are all equal, the MFMA kernels take
 * head_dim and batch * num_kv_heads is a multiple of the workgroups resident
 * in one round of the current GPU (its CUs, times 2 at tile widths <= 64);
 * TT_SPLIT_PAIRED when they differ, batch <= 256, (batch + 1) / 2 *
 * num_kv_heads is a multiple of the GPU's CUs and no rank pair's tiles (plus
 * 2 tiles' worth of start-up per segment) exceed 1.06 times the pairs' mean;
 * else 0. No counterpart in the reference (whose batches always have one
 * length). */
int64_t tt_decode_pick_split(const int32_t *seq_lens_host, int64_t batch, int64_t num_kv_heads, int64_t head_dim,
                             int32_t fp8_cache);

/* Workspace bytes the attention entry points need; for split_tokens 0 the
 * size covers every cache dtype; for TT_SPLIT_PER_SEGMENT and TT_SPLIT_PAIRED
 * it is what the VALU kernel's automatic split needs (the MFMA kernels need
 * none). */
size_t tt_decode_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                 int64_t head_dim, int64_t max_seq_len, int64_t split_tokens);

/*
 * Decode-step layer operations: the dense work of a decode step around the
 * attention path (projections, residual adds, RMSNorm, SwiGLU), for M rows
 * (one token per sequence). bf16 activations and weights, fp32 accumulation
 * and residual stream. Deterministic: split-K partials are summed in a fixed
 * order by the operation that consumes them.
 */

/*
 * partials[s][m][n] = sum over k in [s * k_chunk, (s + 1) * k_chunk) of
 * x[m][k] * weight[n][k], s < K / k_chunk (fp32, [K / k_chunk, M, N]).
 * Replaces nn.Linear(bias=False) under bf16 autocast for the projections
 * q/k/v/c_proj (attn.py:141-145, 420-430), gate/up/down (mlp.py:24-26,
 * 44-45); the rows of several projections of one input may be stacked into
 * one weight (q|k|v, gate|up). x bf16 [M, K] (row stride ldx), weight bf16
 * [N, K] (row stride ldw). Requirements: N % 64 == 0, K % k_chunk == 0,
 * k_chunk in {256, 512, 1024}, 16-byte aligned pointers, strides multiples
 * of 8.
 */
int tt_linear_splitk_bf16(const void *x, int64_t ldx, const void *weight, int64_t ldw, float *partials, int64_t m,
                          int64_t n, int64_t k, int64_t k_chunk, tt_stream_t stream);

/*
 * As tt_linear_splitk_bf16 with the weight in fragment order: element
 * W[n][k] at index ((n / 16) * (K / 32) + k / 32) * 512 + ((k % 32) / 8) * 128
 * + (n % 16) * 8 + k % 8, i.e. W.view(N/16, 16, K/32, 4, 8).permute(0, 2, 3,
 * 1, 4) made contiguous, so each 32-wide k step of a 16-row block is one
 * contiguous 1 KB read. (Layout of this library; no counterpart in the
 * reference.)
 */
int tt_linear_splitk_packed_bf16(const void *x, int64_t ldx, const void *weight_packed, float *partials, int64_t m,
                                 int64_t n, int64_t k, int64_t k_chunk, tt_stream_t stream);

/* y[m][n] = bf16(sum_s partials[s][m][n]) (the projection's bf16 output). */
int tt_splitk_reduce_bf16(const float *partials, int64_t splits, int64_t m, int64_t n, void *y, tt_stream_t stream);

/*
 * Residual add + RMSNorm (gpt.py:40-41 + norm.py:6-19, eps as given):
 * with partials (a projection's split-K output for this residual stream),
 * x[m] += bf16(sum_s partials[s][m]) first; then
 * y[m] = bf16(weight * (x[m] * rsqrt(mean(x[m]^2) + eps))), the normalised
 * row as the next projection's bf16 input. partials may be NULL (plain
 * RMSNorm). x, weight fp32; C a multiple of 4, 4 <= C <= 8192.
 */
int tt_add_rmsnorm_bf16(float *x, const float *partials, int64_t splits, const float *weight, float eps, void *y,
                        int64_t m, int64_t c, tt_stream_t stream);

/*
 * SwiGLU of a stacked gate|up projection (mlp.py:44-45): with g, u the bf16
 * sums of the partials of columns [0, I) and [I, 2I),
 * y[m][i] = bf16(bf16(silu(g)) * u). partials [splits, M, 2I] fp32.
 */
int tt_silu_mul_bf16(const float *partials, int64_t splits, int64_t m, int64_t inter, void *y, tt_stream_t stream);

/*
 * The gate and up projections and SwiGLU of one MLP (mlp.py:24-26, 44-45
 * under bf16 autocast) in one launch, with no split-K partials:
 * y[m][i] = bf16(bf16(silu(bf16 g)) * bf16 u), g = x[m] . Wg[i], u = x[m] . Wu[i]
 * summed in fp32 over the whole K. weight_packed is the fragment-ordered
 * (as tt_linear_splitk_packed_bf16) matrix of 2I rows interleaved by 8:
 * rows 16j .. 16j+7 are gate rows 8j .. 8j+7, rows 16j+8 .. 16j+15 up rows
 * 8j .. 8j+7. x bf16 [M, K] (row stride ldx), y bf16 [M, I] (row stride
 * ldy). Requirements: K 768, 1024 or 2048, I a multiple of 16 or 24 (tt_swiglu_gemm_supported),
 * ldx % 8 == 0, ldy % 4 == 0, 16-byte aligned x and weight, 8-byte aligned y.
 * (Replaces the gate|up tt_linear_splitk_packed_bf16 + tt_silu_mul_bf16 pair;
 * the interleaved layout is this library's, no counterpart in the reference.)
 */
int tt_linear_swiglu_packed_bf16(const void *x, int64_t ldx, const void *weight_packed, void *y, int64_t ldy,
                                 int64_t m, int64_t inter, int64_t k, tt_stream_t stream);

/* 1 when tt_linear_swiglu_packed_bf16 takes this K and I, else 0. */
int tt_swiglu_gemm_supported(int64_t k, int64_t inter);

/*
 * Prefill rows (gpt.py:40-41 + norm.py:6-19 over every prompt token): the
 * residual add of a projection's bf16 output a [M, C] (row stride lda) into
 * the fp32 stream x, x[m] += float(a[m]), then y[m] = bf16(weight * (x[m] *
 * rsqrt(mean(x[m]^2) + eps))). a may be NULL (plain RMSNorm). C as for
 * tt_add_rmsnorm_bf16; lda % 4 == 0.
 */
int tt_add_rmsnorm_rows_bf16(float *x, const void *a, int64_t lda, const float *weight, float eps, void *y, int64_t m,
                             int64_t c, tt_stream_t stream);

/*
 * SwiGLU over prompt rows, mlp.py:44-45 under autocast: g and u are the bf16
 * outputs of the gate and up projections [M, I] (row strides ldg, ldu; a
 * stacked gate|up output passes u = g + I), y[m][i] = bf16(bf16(silu(g)) * u),
 * y contiguous [M, I]. I, ldg, ldu multiples of 4.
 */
int tt_silu_mul_rows_bf16(const void *g, int64_t ldg, const void *u, int64_t ldu, int64_t m, int64_t inter, void *y,
                          tt_stream_t stream);

/*
 * Token sampling from logits [M, V] (row stride ld), replacing
 * filter_logits + sample_next_token / sample_next_token_with_log_prob
 * (tinytron/inference/sampler.py:6-62; called at engine.py:196-212):
 * fp32 cast, division by temperature (skipped at 1.0; temperature <= 0 is an
 * error), top-k when top_k > 0 (keeps values >= the k-th largest, ties
 * kept), top-p when 0 < top_p < 1 (keeps the shortest descending prefix
 * whose cumulative probability exceeds top_p, the first token always; equal
 * values are ordered by index), then one token per row:
 *   - top_k == 1: the first maximum (the reference draws among exactly tied
 *     maxima at random);
 *   - otherwise a draw from softmax(filtered) by inverse CDF in index order,
 *     driven by a 64-bit uniform from SplitMix64 over (seed, offset, row):
 *     the distribution of torch.multinomial, not its random stream. The
 *     same (seed, offset) gives the same tokens.
 * tokens int64 [M] (required). token_logprob [M] (optional): the chosen
 * token's log_softmax(filtered) value (sampler.py:56-61). logprobs [M, V]
 * with row stride ld_logprobs (optional): log_softmax of the filtered logits,
 * -inf where filtered. V <= 65536 (bf16 logits), 32768 (fp32 logits).
 * workspace (optional, 16-byte aligned, workspace_bytes >=
 * tt_sample_workspace_bytes(m, vocab, top_k)): with 2 <= top_k <= 64, V >
 * 8192 and no logprobs rows, every 8192-logit chunk of a row first reduces to
 * its top-k candidates on a workgroup of its own, and the row is decided from
 * those (the same tokens as the one-workgroup-per-row path, which runs when
 * workspace is NULL or a row's candidates cannot decide it; token
 * log-probabilities agree with that path's to within the rounding of the
 * exp-sum order: this path adds them in rank order, that one by a block
 * reduction). More than 65535 rows always take the one-workgroup-per-row path.
 * Calls that share a workspace must not overlap.
 */
int tt_sample_bf16(const void *logits, int64_t ld, int64_t m, int64_t vocab, float temperature, int64_t top_k,
                   float top_p, uint64_t seed, uint64_t offset, int64_t *tokens, float *token_logprob,
                   float *logprobs, int64_t ld_logprobs, void *workspace, size_t workspace_bytes,
                   tt_stream_t stream);

/* As tt_sample_bf16 with fp32 logits (fp32 models). */
int tt_sample_f32(const float *logits, int64_t ld, int64_t m, int64_t vocab, float temperature, int64_t top_k,
                  float top_p, uint64_t seed, uint64_t offset, int64_t *tokens, float *token_logprob,
                  float *logprobs, int64_t ld_logprobs, void *workspace, size_t workspace_bytes,
                  tt_stream_t stream);

/* Workspace bytes tt_sample_* uses for m rows of vocab logits at this top_k (0: none). */
size_t tt_sample_workspace_bytes(int64_t m, int64_t vocab, int64_t top_k);

#ifdef __cplusplus
}
#endif

#endif /* TINYTRON_AMD_H */
