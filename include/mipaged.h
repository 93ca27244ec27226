/*
 * mipaged.h — C ABI of the MI355X paged KV-cache kernels (gfx950).
 *
 * Operations behind this boundary:
 *   1. KV append          : scatter new K/V rows into the paged pool through a slot mapping
 *                           (optionally fused with the rotary embedding of q and k).
 *   2. Paged decode attn  : one query token per sequence, GQA, reading K/V pages in place
 *                           through per-sequence block tables (optionally fused with the
 *                           append, and driven by a per-step work plan).
 *   3. Block copy         : copy whole blocks (all layers, K and V) for copy-on-write of
 *                           shared prefix blocks (the (src, dst) pairs in device memory, or
 *                           in host memory, passed in the kernel arguments).
 *   4. Paged prefill attn : packed new tokens of several sequences over their cached
 *                           prefixes and themselves, causal, reading K/V pages in place.
 *
 * Pool layout (one layer; identical to the reference pool
 * engine/kv_cache.py:426-428, `k, v: [num_layers, num_blocks + 1, num_kv_heads,
 * block_size, head_dim]`, the extra block being the scratch block):
 *
 *     cache[block][kv_head][offset][d]     d contiguous, element type = dtype
 *
 * so the (block, kv_head) tile of block_size * head_dim elements is one contiguous run.
 * A slot is the flat token index  slot = block * block_size + offset.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers owned by the caller, except the pairs of
 *     mip_copy_blocks_host, which the call reads on the host before it returns. Nothing
 *     here allocates, frees or synchronises. Work is enqueued on `stream` (a hipStream_t;
 *     NULL = the null stream) and the call returns immediately.
 *   - Strides are in ELEMENTS, not bytes. The last (head_dim) dimension must be
 *     contiguous.
 *   - Return value: MIP_OK (0) on success, MIP_EINVAL (-22) for arguments that fail the
 *     host-side checks (nothing is launched), MIP_EUNSUPPORTED (-95) for a shape with no
 *     compiled kernel, or a positive hipError_t from the launch.
 *   - Calls are asynchronous and graph-capturable: the grid depends only on the integer
 *     arguments, never on device data.
 */
#ifndef MIPAGED_H_
#define MIPAGED_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum mip_dtype { MIP_F32 = 0, MIP_F16 = 1, MIP_BF16 = 2 };

enum mip_status { MIP_OK = 0, MIP_E2BIG = -7, MIP_EINVAL = -22, MIP_EUNSUPPORTED = -95 };

/* Library version, (major << 16) | minor. */
int mip_version(void);

/*
 * Decode attention algorithm (no reference counterpart: the reference has one path, SDPA).
 * MIP_ALGO_AUTO picks per shape: the stream-K MFMA kernel for 16-bit K/V at head_dim 64/128
 * (batch <= 4096), else the per-partition MFMA kernel, else the VALU kernel (fp32, other head
 * sizes; a query group of more than 8 heads is split over workgroups of at most 8, each of
 * which reads the kv head's keys and values). A forced algorithm applies only where its kernel
 * exists for the shape (the MFMA kernels: group <= 16). The setting is
 * process-wide, starts from the MIP_DECODE_ALGO environment variable (valu | mfma | stream,
 * read once), and is meant for kernel comparisons and tests; it must not change while decode
 * calls are being enqueued, since the workspace and plan sizes depend on it. Returns the
 * previous setting, or MIP_EINVAL for an unknown value.
 */
enum mip_decode_algo { MIP_ALGO_AUTO = 0, MIP_ALGO_VALU = 1, MIP_ALGO_MFMA = 2, MIP_ALGO_STREAM = 3 };
int mip_set_decode_algo(int32_t algo);

/* Human-readable text for a status code returned by any entry point. */
const char* mip_status_string(int status);

/*
 * KV append.
 *
 * Replaces the scatter in PagedDecodeContext.attend
 *   engine/kv_cache.py:613-614   k_layer[write_blocks, :, write_offsets] = k[:, :, 0]
 * and the packed-prefill scatter in PackedPrefillContext.attend
 *   engine/kv_cache.py:286-289   k_layer[where_0, :, where_2] = k[0].transpose(0, 1)
 * (and the same writes inside the graphed decode, engine/cuda_graphs.py:82-83).
 *
 * Token i (0 <= i < n_tokens), kv head h: the head_dim elements at
 *     k_src + i * k_stride_tok + h * k_stride_head
 * are copied bit for bit to row ((s / block_size) * num_kv_heads + h) * block_size
 * + s % block_size of k_cache, where s = slot_mapping[i]; likewise for V.
 * A slot outside [0, num_cache_blocks * block_size) is skipped (write nothing), so
 * negative slots can mark padding rows. Slots must be distinct (as for index_put_
 * without accumulate, duplicate targets leave an unspecified winner).
 */
int mip_kv_append(const void* k_src, const void* v_src,
                  int64_t k_stride_tok, int64_t k_stride_head,
                  int64_t v_stride_tok, int64_t v_stride_head,
                  void* k_cache, void* v_cache, int64_t num_cache_blocks,
                  const int64_t* slot_mapping, int32_t n_tokens,
                  int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                  int32_t dtype, void* stream);

/*
 * Rotary position embedding of q and k, fused with the KV append.
 *
 * Replaces, in one launch, the rotation of one decoder layer
 *   engine/model.py:249          q, k = apply_rope(q, k, cos, sin)
 *   engine/model.py:216-224      x * cos + _rotate_half(x) * sin,  _rotate_half(x) = cat(-x2, x1)
 * and the scatter that follows it in the cache context (engine/kv_cache.py:613-614 decode,
 * :286-289 packed prefill).
 *
 * Token i, element j of a head row x (d = head_dim / 2, c = cos row i, s = sin row i):
 *     x'[j]     = rnd(rnd(x[j] * c[j])         + rnd(-x[j + d] * s[j]))       j < d
 *     x'[j + d] = rnd(rnd(x[j + d] * c[j + d]) + rnd(x[j] * s[j + d]))
 * with products and sums in fp32 and rnd = round to nearest even into dtype (identity for
 * fp32): exactly the values torch's op-by-op evaluation stores, so the results are
 * bit-identical to apply_rope in dtype. The q rows (num_heads per token) and k rows
 * (num_kv_heads per token) are rotated IN PLACE. The rotated k rows and the v rows are
 * then written to the pool as mip_kv_append does: slot = slot_mapping[i], slots outside
 * [0, num_cache_blocks * block_size) are skipped (no pool write; q and k are still rotated).
 *
 * cos/sin: one row of head_dim elements of dtype per token, row i at cos + i * cs_stride_tok
 * (the [B, 1, T, D] tables of engine/model.py:211-213, token i = b * T + t). q may be NULL
 * when num_heads is 0. head_dim must be even.
 */
int mip_rope_kv_append(void* q, int64_t q_stride_tok, int64_t q_stride_head,
                       void* k, int64_t k_stride_tok, int64_t k_stride_head,
                       const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                       const void* cos, const void* sin, int64_t cs_stride_tok,
                       void* k_cache, void* v_cache, int64_t num_cache_blocks,
                       const int64_t* slot_mapping, int32_t n_tokens, int32_t num_heads,
                       int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                       int32_t dtype, void* stream);

/*
 * Paged decode attention (one new token per sequence, GQA).
 *
 * Replaces the gather + SDPA of PagedDecodeContext.attend
 *   engine/kv_cache.py:615-620   keys = k_layer[tables].permute(0, 2, 1, 3, 4).reshape(...)
 *                                 decode_attention(q, keys, values, attn_mask=mask)
 * and engine/model.py:126-147 (decode_attention: query head h reads kv head
 * h / (num_heads / num_kv_heads)), with the mask `arange(kv_len) <= positions`
 * (engine/kv_cache.py:609) expressed as context_lens[b] = positions[b] + 1.
 *
 *   out[b, h, :] = softmax_j( scale * q[b, h, :] . K_b[j, :] ) @ V_b[j, :],
 *                  j < context_lens[b],
 *   K_b[j] = k_cache row (block_tables[b * bt_stride + j / block_size], h / group, j % block_size)
 *
 * Arithmetic: products and sums in fp32, output rounded once to dtype.
 * Entries of a block table past ceil(context_lens[b] / block_size) are never read.
 * A sequence with context_lens[b] <= 0 gets a zero output row.
 * context_lens[b] must not exceed max_blocks_per_seq * block_size (larger values are
 * clamped to it).
 *
 * `workspace` is scratch device memory for split contexts (per-piece softmax state and
 * partial outputs, combined by a second kernel on the same stream; for a batch of at most
 * 16 sequence x kv-head segments, a third kernel folds the second's per-run states). It must hold
 * mip_paged_decode_workspace(...) bytes for the same shape, asked with the same device
 * current, and be 256-byte aligned. It needs no initialisation and its contents are
 * undefined afterwards; calls on one stream may reuse it, calls that can run
 * concurrently must not share it.
 *
 * `plan` (may be NULL) is a work plan made by mip_paged_decode_plan from the same
 * context_lens and block_tables contents and the same shape, earlier on the stream; the
 * kernel then streams from its tile descriptors instead of deriving its work split and
 * walking the block tables (every layer of a decode step shares one plan). `plan_bytes` is
 * the size of the plan buffer: below mip_paged_decode_plan_bytes for this shape it is
 * MIP_EINVAL. The plan is ignored where the stream kernel does not run and for
 * block_size < 16. A plan made for another batch size or kv-head count (its header does not
 * match the call) cannot be detected before launch, since it lives in device memory: the call
 * then writes NaN to every output row and, for mip_paged_decode_append, leaves the pool
 * unchanged.
 */
int mip_paged_decode(void* out, int64_t out_stride_b, int64_t out_stride_h,
                     const void* q, int64_t q_stride_b, int64_t q_stride_h,
                     const void* k_cache, const void* v_cache, int64_t num_cache_blocks,
                     const int32_t* block_tables, int64_t bt_stride,
                     const int32_t* context_lens,
                     int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                     float scale, void* workspace, size_t workspace_bytes,
                     const void* plan, size_t plan_bytes, int32_t dtype, void* stream);

/*
 * KV append + paged decode attention in one call: the whole of
 *   PagedDecodeContext.attend   engine/kv_cache.py:611-620
 * (scatter of the step's new K/V rows, then attention over every sequence's keys including
 * the new one). The result, pool and output, is exactly that of mip_kv_append(k_new, v_new,
 * ..., slot_mapping, n_tokens = batch, ...) followed by mip_paged_decode(...) with the same
 * arguments.
 *
 * Where the stream kernel runs (16-bit K/V, head_dim 64/128, group <= 16) and the new rows
 * and their strides are 16-byte aligned, no separate append kernel runs: the attention
 * kernel reads each sequence's newest key straight from k_new / v_new, and its merge kernel
 * (which follows it on the stream) copies the new rows into the pool. That needs
 * slot_mapping[b] to be the slot of key context_lens[b] - 1 of sequence b (as
 * PagedDecodeContext builds it) or outside the pool; a slot that some sequence reads as an
 * older key is a race. Otherwise the append kernel and the decode run one after the other.
 */
int mip_paged_decode_append(const void* k_new, const void* v_new,
                            int64_t k_stride_tok, int64_t k_stride_head,
                            int64_t v_stride_tok, int64_t v_stride_head,
                            const int64_t* slot_mapping,
                            void* out, int64_t out_stride_b, int64_t out_stride_h,
                            const void* q, int64_t q_stride_b, int64_t q_stride_h,
                            void* k_cache, void* v_cache, int64_t num_cache_blocks,
                            const int32_t* block_tables, int64_t bt_stride,
                            const int32_t* context_lens,
                            int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                            int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                            float scale, void* workspace, size_t workspace_bytes,
                            const void* plan, size_t plan_bytes, int32_t dtype, void* stream);

/*
 * mip_paged_decode_append without a workspace argument: the same call, the same kernels and the
 * same results, with the scratch memory taken from a static device array of the library
 * (MIP_NOALLOC_SCRATCH_BYTES on every device it runs on, held until the process ends).
 *
 * No reference counterpart: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It calls no
 * allocating routine. The array's device address is looked up on the first call on each device
 * (the current device, which must own `stream`). A shape whose workspace
 * (mip_paged_decode_workspace) exceeds MIP_NOALLOC_SCRATCH_BYTES returns MIP_E2BIG before
 * anything is launched. Every call on one device shares that device's array, so calls that can
 * run concurrently on one device (different streams, several host threads) race; calls ordered
 * on one stream do not.
 */
#define MIP_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int mip_paged_decode_append_noalloc(const void* k_new, const void* v_new,
                                    int64_t k_stride_tok, int64_t k_stride_head,
                                    int64_t v_stride_tok, int64_t v_stride_head,
                                    const int64_t* slot_mapping,
                                    void* out, int64_t out_stride_b, int64_t out_stride_h,
                                    const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                    void* k_cache, void* v_cache, int64_t num_cache_blocks,
                                    const int32_t* block_tables, int64_t bt_stride,
                                    const int32_t* context_lens,
                                    int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                    int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                                    float scale, const void* plan, size_t plan_bytes, int32_t dtype,
                                    void* stream);

/*
 * Work plan of the decode kernels for one decode step (no reference counterpart: the
 * reference derives nothing per step beyond PagedDecodeContext's tensors,
 * engine/kv_cache.py:592-609).
 *
 * Every layer of a step attends the same sequences, so the stream kernel's work split is
 * the same for all of them: each wavefront's range of 16-key tiles, which pieces the merge
 * combines, and one descriptor per tile (its pool row, sequence, kv head, valid keys and
 * segment edges, read through the block tables once). One launch writes it; pass the plan
 * to each layer's mip_paged_decode / mip_paged_decode_append, which then stream from the
 * descriptors instead of walking the block tables. Returns MIP_EUNSUPPORTED (nothing
 * launched) for shapes the stream kernel does not run and for block_size < 16 (a tile must
 * lie in one block); mip_paged_decode_plan_bytes returns 0 for those. The plan buffer must
 * be 8-byte aligned; it holds int32 data and stays valid while context_lens, block_tables
 * and the shape do not change. A decode call given a plan made for another batch size or
 * kv-head count writes NaN outputs and appends nothing (see mip_paged_decode).
 */
size_t mip_paged_decode_plan_bytes(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                   int32_t head_dim, int32_t block_size,
                                   int32_t max_blocks_per_seq, int32_t dtype);
int mip_paged_decode_plan(const int32_t* context_lens, const int32_t* block_tables,
                          int64_t bt_stride, int32_t batch, int32_t num_heads,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          int32_t max_blocks_per_seq, int32_t dtype, void* plan,
                          size_t plan_bytes, void* stream);

/*
 * Paged varlen prefill attention over a cached prefix.
 *
 * Replaces the read-back gather + dense-mask SDPA of PackedPrefillContext.attend
 *   engine/kv_cache.py:286-294   keys = k_layer[read_0, :, read_2] ...; sdpa_attention(q, keys,
 *                                 values, attn_mask=self.mask)
 * with its mask (engine/kv_cache.py:268-276) `key_seg == seg & key_pos <= position`, and, for
 * sequences with nothing cached, the packed block-diagonal causal SDPA of :290-294.
 *
 * Sequence s (0 <= s < num_seqs) owns packed rows r in [cu_q[s], cu_q[s + 1]); row r is its new
 * token i = r - cu_q[s], at position p = ctx_start[s] + i. For every query head h:
 *
 *   out[r, h, :] = softmax_j( scale * q[r, h, :] . K_s[j, :] ) @ V_s[j, :],   0 <= j <= p,
 *   K_s[j] = k_cache row (block_tables[s * bt_stride + j / block_size], h / group, j % block_size)
 *
 * (group = num_heads / num_kv_heads), i.e. each new token sees its sequence's cached prefix
 * and its own sequence's new tokens up to itself; every key it reads must already be in the
 * pool (append first). Scores, sums and products accumulate in fp32; on the MFMA kernel the
 * softmax weights enter the V product rounded to fp16 (2^-11 relative): bf16 V is staged as
 * fp16 (exact below 65536 in magnitude), and an item whose V holds a larger value, inf or NaN
 * uses bf16 V with each weight split into two bf16 parts. The output is rounded once to
 * dtype. Keys past
 * max_blocks_per_seq * block_size are never read (positions beyond are clamped to the last
 * one). max_q_len must be >= every cu_q[s + 1] - cu_q[s]; it only sizes the grid, which
 * depends on the integer arguments alone.
 *
 * Kernels: 16-bit dtypes at head_dim 64 or 128 with group <= 16 run the MFMA prefill kernel
 * (q rows 16-byte aligned, out rows 8-byte aligned). Every other shape with head_dim a power
 * of two in 8 .. 256 (fp32 included) runs the VALU decode kernel, one workgroup per (new
 * token, kv head, group of at most 8 of its query heads) over that token's keys (q rows
 * 4-byte aligned); the grid then has num_seqs * max_q_len workgroups per such group. Other
 * shapes: MIP_EUNSUPPORTED.
 */
int mip_paged_prefill(void* out, int64_t out_stride_tok, int64_t out_stride_head,
                      const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                      const void* k_cache, const void* v_cache, int64_t num_cache_blocks,
                      const int32_t* block_tables, int64_t bt_stride,
                      const int32_t* cu_q, const int32_t* ctx_start,
                      int32_t num_seqs, int32_t max_q_len, int32_t num_heads, int32_t num_kv_heads,
                      int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq, float scale,
                      int32_t dtype, void* stream);

/* Workspace bytes mip_paged_decode and mip_paged_decode_append need for this shape (0 when
 * they need none). */
size_t mip_paged_decode_workspace(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                  int32_t head_dim, int32_t block_size,
                                  int32_t max_blocks_per_seq, int32_t dtype);

/*
 * Block copy for copy-on-write of shared prefix blocks.
 *
 * No reference counterpart: the reference shares only full, never-rewritten prefix
 * blocks (engine/kv_cache.py:499-508, 527). The operation is the bitwise
 *     k[l, dst] = k[l, src];  v[l, dst] = v[l, src]     for every layer l
 * over a pool laid out [num_layers][num_cache_blocks][block_bytes].
 * `pairs` is int64 [n_pairs][2] = (src, dst). Pairs with an index outside
 * [0, num_cache_blocks) are skipped. Destinations must be distinct and must not be
 * the source of another pair in the same call. One launch copies up to 2^24 - 1
 * (pair, layer, K|V) units; a larger call is split into several launches in pair order.
 * num_layers must be below 2^23 (MIP_EINVAL otherwise).
 */
int mip_copy_blocks(void* k_cache, void* v_cache, const int64_t* pairs, int32_t n_pairs,
                    int32_t num_layers, int64_t num_cache_blocks, int64_t block_bytes,
                    void* stream);

/*
 * mip_copy_blocks with `pairs` in host memory: the same copy and the same rules. The pairs
 * travel in the kernel arguments, MIP_COPY_INLINE_PAIRS per launch (one launch per group), so
 * the copy needs no upload of the pairs and reads no pair list from device memory before its
 * data. `pairs` may be reused or freed as soon as the call returns. Like any kernel argument,
 * the pairs are fixed when a stream capture records the call.
 *
 * No reference counterpart (as mip_copy_blocks); PagedKVCache.copy_blocks uses it for the
 * copy-on-write pairs it builds on the host.
 */
#define MIP_COPY_INLINE_PAIRS 128
int mip_copy_blocks_host(void* k_cache, void* v_cache, const int64_t* pairs, int32_t n_pairs,
                         int32_t num_layers, int64_t num_cache_blocks, int64_t block_bytes,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MIPAGED_H_ */
