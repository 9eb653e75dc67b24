/*
 * pkv.h -- C ABI of libpkv, the MI355X (gfx950) paged KV-cache attention path.
 *
 * Drop-in for the attention step of phildrip/llm-mojo's
 * model_speculative_moe_batched.mojo: per-sequence block tables, token append into
 * partially filled blocks, LIFO block free/reuse under continuous batching, read-only
 * KV sharing with the MTP assistant layers, and rollback after rejected drafts.
 *
 * Conventions
 *   - Every pointer argument named *_pool, block_tables, table_lens, free_list,
 *     free_count, pos, tok_off, new_len, q, k_new, v_new, out, status and workspace is
 *     DEVICE memory owned by the caller. `stream` is a hipStream_t (NULL = the null
 *     stream). All calls are stream-ordered and asynchronous; the library keeps no
 *     device state between calls (all state lives in caller-owned buffers).
 *   - Return value: PKV_OK (0) or a negative PKV_ERR_* code. Nothing throws across
 *     the ABI; pkv_last_error() gives a message for the calling thread's last error.
 *   - Pool layout is the reference's (model_speculative_moe_batched.mojo:1427-1451):
 *     element (block b, slot i, kv head g, dim d) of a layer pool lives at
 *     ((b * block_size + i) * num_kv_heads + g) * head_dim + d.
 *   - Block tables: int32 [batch][table_stride]; table_lens: int32 [batch]. Row s of
 *     the tables is sequence slot s. The reference's List[Int] tables hold the same
 *     values in 64-bit.
 *   - Free list: int32 [num_blocks] used as a LIFO stack free_list[0 .. *free_count);
 *     allocation pops the back, freeing pushes to the back (BlockManager,
 *     model_speculative_moe_batched.mojo:789-807). Initialise it to 0..num_blocks-1
 *     and *free_count = num_blocks to start from the reference's fresh state.
 *   - Concurrent calls that touch the same tables / free list / workspace race; order
 *     them on one stream.
 *   - Ring pools (pkv_params.ring_size > 0; the engine's default for sliding layers,
 *     model_speculative_moe_batched.mojo:1301-1304, :1440-1442): a layer pool holds
 *     num_blocks rings of ring_size rows, and token t of a sequence whose ring slot is
 *     `slot` lives in row slot * ring_size + t % ring_size (ring_row,
 *     attention.mojo:144-148). In this mode block_tables[s * table_stride] is sequence
 *     s's ring slot (Sequence.kv_slot, :819) -- an int32 [batch] array with
 *     table_stride 1 -- and no block is allocated or freed.
 */
#ifndef PKV_H
#define PKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKV_OK 0
#define PKV_ERR_INVALID (-1)     /* bad argument (shape, dtype, null pointer)       */
#define PKV_ERR_UNSUPPORTED (-2) /* geometry or mode this build has no kernel for   */
#define PKV_ERR_WORKSPACE (-3)   /* workspace smaller than pkv_workspace_size()     */
#define PKV_ERR_HIP (-4)         /* a HIP runtime call failed (see pkv_last_error)  */

#define PKV_DTYPE_F32 0
#define PKV_DTYPE_BF16 1

/* Per-sequence status written by pkv_append / pkv_rollback. */
#define PKV_SEQ_OK 0
#define PKV_SEQ_OUT_OF_BLOCKS (-1) /* BlockManager.allocate() returned -1          */
#define PKV_SEQ_TABLE_FULL (-2)    /* position beyond table_stride blocks           */
#define PKV_SEQ_BAD_BLOCK (-3)     /* a table entry outside [0, num_blocks)         */
#define PKV_SEQ_FREE_OVERFLOW (-4) /* freeing would overflow the free list          */
#define PKV_SEQ_BAD_ARGS (-5)      /* token range outside [0, total_rows) or > max_new */
#define PKV_SEQ_BAD_INDEX (-6)     /* LSA index or bucket id out of range (skipped)   */

/* Layer geometry and numerics, shared by every entry point.
 * Mirrors paged_attention_layer's scalar arguments (attention.mojo:240-256). */
typedef struct pkv_params {
    int32_t num_heads;    /* query heads Hq                                            */
    int32_t num_kv_heads; /* KV heads Hkv; Hq % Hkv == 0                               */
    int32_t head_dim;     /* D: 64, 256 or 512                                         */
    int32_t block_size;   /* tokens per block, a power of two (the engine uses 16)     */
    int32_t num_blocks;   /* physical blocks in each pool (bounds every table entry)   */
    int32_t window;       /* > 0: keys t >= pos - window + 1 (attention.mojo:135-141);
                             <= 0: full causal                                          */
    float scale;          /* multiplies q.k before the softmax. 1.0f reproduces the
                             reference exactly (Gemma-4 has no softmax scale)          */
    int32_t kv_dtype;     /* PKV_DTYPE_F32 or PKV_DTYPE_BF16 (pool element type)       */
    int32_t ring_size;    /* 0: paged pools; > 0: ring pools of ring_size rows per slot
                             (num_blocks then counts ring slots)                      */
    int32_t reserved;     /* must be 0                                                 */
} pkv_params;

/* Bytes of workspace pkv_attend / pkv_decode need for `batch` sequences of `q_len`
 * queries whose last query position is at most max_pos (the split-K partials).
 * 0 on invalid params. */
size_t pkv_workspace_size(const pkv_params* p, int32_t batch, int32_t q_len, int32_t max_pos);

/* K1 -- fused block allocation + K/V scatter.
 * Replaces the engine's inline append sites: model_speculative_moe_batched.mojo
 * :1984-2001 (decode), :2513-2523 + :2621-2630 (chunked prefill), :2808-2825 (CPU
 * prefill), :3011-3023 + :3106-3116 (verify).
 * New tokens are ragged: sequence s appends n_s = tok_off[s+1] - tok_off[s] tokens whose
 * K / V rows are rows tok_off[s] .. tok_off[s+1]-1 of k_new / v_new
 * ([total_rows][num_kv_heads * head_dim] in kv_dtype). A decode step is tok_off = 0..B.
 * For each sequence s (in index order), the tokens at positions pos[s] .. pos[s]+n_s-1
 * grow the table while p / block_size >= table_lens[s], popping blocks from the back of
 * the free list, then their K and V rows are copied bit-exactly to row
 * table[p / bs] * bs + p % bs of k_pool / v_pool.
 * Out of blocks: blocks popped before the list ran dry stay in the table, none of the
 * sequence's rows is written and status[s] = PKV_SEQ_OUT_OF_BLOCKS.
 * pos[s] < 0 or n_s <= 0 skips sequence s. A token range outside [0, total_rows) or
 * longer than max_new (which sizes the grid) changes nothing for s and gives
 * PKV_SEQ_BAD_ARGS. A block the append touches whose table entry (held, or just popped
 * from the free list) lies outside [0, num_blocks) gives PKV_SEQ_BAD_BLOCK: the rows of
 * that block are skipped and the others written. A *free_count outside [0, num_blocks]
 * pops nothing and gives PKV_SEQ_BAD_BLOCK to every sequence that needs a block; such a
 * sequence writes only the rows of blocks it already holds. tok_off: int32 [batch + 1]
 * (device).
 * status: int32 [batch] (device), written for every sequence. batch <= 4096.
 * Two launches on `stream`: the allocation (one workgroup) and the row scatter.
 * Ring pools (ring_size > 0): one launch, the scatter; token p of sequence s goes to
 * row slot * ring_size + p % ring_size of its ring (the write sites :1996, :2625,
 * :3111); table_lens, free_list and free_count are not used and may be NULL. Of more
 * than ring_size new tokens only the last ring_size are written (the rows a serial
 * pass leaves). A slot outside [0, num_blocks) gives PKV_SEQ_BAD_BLOCK and writes
 * nothing. Two sequences sharing a slot in one call race. */
int32_t pkv_append(void* stream, const pkv_params* p, void* k_pool, void* v_pool,
                   int32_t* block_tables, int32_t table_stride, int32_t* table_lens,
                   int32_t* free_list, int32_t* free_count, const int32_t* pos,
                   const int32_t* tok_off, int32_t max_new, const void* k_new,
                   const void* v_new, int32_t total_rows, int32_t batch, int32_t* status);

/* K1' -- the producer step before the append, fused with it.
 * Replaces the engine's per-token sequence rms_norm(q) / rms_norm(k) / rms_norm_noscale(v)
 * per head + apply_rope_qk + KV write: model_speculative_moe_batched.mojo:1974-2001
 * (decode), :2612-2630 (chunked prefill), :3099-3116 (verify); rms_norm :857-867,
 * rms_norm_noscale :870-878, apply_rope_qk attention.mojo:69-132.
 * Inputs are the projections' fp32 rows, ragged as in pkv_append: row r of q
 * ([total_rows][num_heads][head_dim]), k and v ([total_rows][num_kv_heads][head_dim])
 * belongs to token b = r - tok_off[s] of sequence s at position pos[s] + b. Per head:
 * q = rms_norm(q, q_norm_weight), k = rms_norm(k, k_norm_weight), v = rms_norm_noscale(v)
 * (x / sqrt(mean(x^2) + 1e-6), times the weight [head_dim]); then Q and K are rotated at
 * the token's position with apply_rope_qk's constants (is_global != 0: the first
 * min(64, head_dim/2) pairs, base 1e6 over 512 dims; else all pairs, base 1e4 over 256).
 * v == NULL means V := K as read, before the norms (global layers, :1962-1964).
 * The processed Q goes to q_out ([total_rows][num_heads][head_dim] in q_out_dtype: fp32
 * for pkv_attend, bf16 for pkv_prefill; may alias q when fp32) for every sequence with a
 * usable token range. K / V rows (rounded to nearest even for bf16 pools) are appended
 * exactly as pkv_append appends k_new / v_new -- same block allocation, status codes and
 * ring mode. head_dim 256 or 512. Two launches (one in ring mode). */
int32_t pkv_append_qkv(void* stream, const pkv_params* p, int32_t is_global, void* k_pool,
                       void* v_pool, int32_t* block_tables, int32_t table_stride,
                       int32_t* table_lens, int32_t* free_list, int32_t* free_count,
                       const int32_t* pos, const int32_t* tok_off, int32_t max_new,
                       const float* q, const float* k, const float* v,
                       const float* q_norm_weight, const float* k_norm_weight, void* q_out,
                       int32_t q_out_dtype, int32_t total_rows, int32_t batch,
                       int32_t* status);

/* K2 -- split-K paged attention for decode and multi-token verify (fp32 or bf16 pools).
 * Replaces paged_attention_layer + _eval_head_range + _softmax (attention.mojo:151-294)
 * as called per query token by execute_attention_for_token
 * (model_speculative_moe_batched.mojo:601-657), the verify loop (:3090-3123) and
 * mtp_paged_attention (:577-599, read-only on the target's pool and table).
 * Query j of sequence s sits at position pos[s] + j and attends keys
 * [window_start(pos[s]+j), pos[s]+j] of its own table: softmax(scale * q.k) . V with
 * the reference's sum + 1e-10 denominator. pos[s] < 0 gives zeros (attention.mojo
 * :180-185).
 * q, out: fp32 [batch][q_len][num_heads][head_dim].
 * max_pos: an upper bound on pos[s] + q_len - 1 over the batch (sizes the grid); a
 * sequence that exceeds it, or whose table holds an entry outside [0, num_blocks),
 * gets NaN outputs. q_len * (num_heads / num_kv_heads) must be <= 16.
 * Ring pools (ring_size > 0): keys are read from sequence s's ring (execute_attention_
 * for_token's ring_base = ring_row(kv_slot, ring_size, 0), :648). Every key of the call,
 * [window_start(pos[s]), pos[s] + q_len - 1], must still be in the ring: a sequence
 * spanning more than ring_size keys, or whose slot lies outside [0, num_blocks), gets
 * NaN outputs (the reference aborts, attention.mojo:265-266). With the engine's
 * ring_size = window + 8 a verify of up to 9 queries fits. */
int32_t pkv_attend(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                   const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                   const int32_t* pos, int32_t q_len, int32_t batch, int32_t max_pos,
                   float* out, void* workspace, size_t workspace_bytes);

/* pkv_attend with q_len = 1: one decode token per sequence (the B=32 hot path). */
int32_t pkv_decode(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                   const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                   const int32_t* pos, int32_t batch, int32_t max_pos, float* out,
                   void* workspace, size_t workspace_bytes);

/* Fused decode/verify step of one layer: pkv_append, then pkv_attend over the same pos
 * (queries at positions pos[s] .. pos[s] + q_len - 1), as the engine's per-layer step
 * writes the new tokens' K/V into the paged cache and attends over it
 * (model_speculative_moe_batched.mojo:1996, :2625, :3111 write sites; :3090-3123 verify).
 * Block tables, table lengths, free list, status, every pool byte and out are those of the
 * two separate calls, with one exception: a sequence whose append fails (status
 * PKV_SEQ_OUT_OF_BLOCKS, PKV_SEQ_TABLE_FULL, PKV_SEQ_BAD_ARGS, or PKV_SEQ_BAD_BLOCK from a
 * free count out of range) is not attended -- the engine skips its attention
 * (model_speculative_moe_batched.mojo:1989-1992) -- and gets NaN rows where the separate
 * calls would attend positions the append did not write.
 * When one launch of the stream kernel covers the call (paged pools, head_dim 256 or 512,
 * G * q_len <= 8, batch <= 1024; on the vector kernel, fp32 pools with up to 4 rows per kv
 * head or bf16 pools, every kv head in one workgroup; fp32 pools with 5..8 rows per kv
 * head run the fp64 MFMA kernel), that launch also computes the block allocation from the
 * state as it stands before the call, copies the appended rows into the pool and reads
 * them from k_new / v_new; the merge launch after it writes the new table entries,
 * table_lens, free_count and status. No allocation or scatter launch is made, and no
 * state word is read and written in one launch. Otherwise the append runs whole first.
 * Arguments as in pkv_append and pkv_attend. Every check of the attention's arguments
 * (including an unsupported geometry) runs before the append launches anything, so a
 * call that returns an error has changed no table, free list or pool. No reference
 * counterpart as one call. */
int32_t pkv_append_attend(void* stream, const pkv_params* p, void* k_pool, void* v_pool,
                          int32_t* block_tables, int32_t table_stride, int32_t* table_lens,
                          int32_t* free_list, int32_t* free_count, const int32_t* pos,
                          const int32_t* tok_off, int32_t max_new, const void* k_new,
                          const void* v_new, int32_t total_rows, int32_t* status, const float* q,
                          int32_t q_len, int32_t batch, int32_t max_pos, float* out,
                          void* workspace, size_t workspace_bytes);

/* Bytes of the device scratch pkv_attend_noalloc uses on each GPU (held from its first
 * call on that GPU until the process ends). */
#define PKV_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* pkv_attend without a workspace argument. No counterpart in the reference: it is for
 * callers that cannot allocate device memory -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc. Same arguments, results and
 * contract as pkv_attend (decode, verify with q_len queries, MTP reads, ring pools),
 * for head_dim 256 or 512 with num_heads / num_kv_heads <= 8; other geometries give
 * PKV_ERR_UNSUPPORTED. The split-K partials live in a library-owned device array of
 * PKV_NOALLOC_SCRATCH_BYTES (64 MiB) per GPU, whose address is looked up on the first
 * call on each device; the call allocates nothing. A call whose partials cannot fit
 * (batch + 1 slots of num_heads * q_len rows of (head_dim + 2) doubles) gives
 * PKV_ERR_WORKSPACE. Every call on one GPU shares that array: calls that overlap on a
 * GPU (other streams, other host threads) race, so order them on one stream. Under HIP
 * graph capture (relaxed mode): make one call with the same shape on the device first
 * (the first call on a device looks up the array's address and the kernels' occupancy);
 * the captured graph then replays with whatever the inputs hold at each launch. */
int32_t pkv_attend_noalloc(void* stream, const pkv_params* p, const float* q,
                           const void* k_pool, const void* v_pool, const int32_t* block_tables,
                           int32_t table_stride, const int32_t* pos, int32_t q_len,
                           int32_t batch, int32_t max_pos, float* out);

/* K2'' -- verify attention with a query count per sequence. The engine verifies each
 * sequence's own draft: verify_b = drafts + 1 tokens (model_speculative_moe_batched.mojo
 * :3005), fewer when drafting stopped early at a terminal token (:2990-2993), so counts
 * differ across the batch. Replaces that loop (:3090-3123) for the whole batch at once:
 * sequence s has q_lens[s] in [0, max_q_len] queries, rows j < q_lens[s] of q / out (fp32
 * [batch][max_q_len][num_heads][head_dim], the pkv_attend layout for q_len = max_q_len) at
 * positions pos[s] + j, each attending [window_start(pos[s] + j), pos[s] + j]. Rows
 * j >= q_lens[s] of out are not written. A count outside [0, max_q_len] gives NaN rows;
 * the other contract violations behave as in pkv_attend. max_pos bounds pos[s] +
 * q_lens[s] - 1. Workspace: pkv_workspace_size(p, batch, max_q_len, max_pos). head_dim
 * 256 or 512 with num_heads / num_kv_heads <= 8 (every geometry of the engine); other
 * geometries give PKV_ERR_UNSUPPORTED. Two launches per group of up to 8 query rows per
 * kv head. */
int32_t pkv_verify(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                   const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                   const int32_t* pos, const int32_t* q_lens, int32_t max_q_len, int32_t batch,
                   int32_t max_pos, float* out, void* workspace, size_t workspace_bytes);

/* Bytes of workspace pkv_attend_sparse needs for `batch` key lists of at most max_keys
 * entries. 0 on invalid params. */
size_t pkv_sparse_workspace_size(const pkv_params* p, int32_t batch, int32_t max_keys);

/* K2' -- sparse paged attention over explicit key lists (LSA on global layers).
 * Replaces lsa_sparse_paged_attention (lsa_core.mojo:630-680) as called by
 * execute_attention_for_token's LSA branch (model_speculative_moe_batched.mojo:630-646)
 * with the key list from LSALayerIndex.expand_buckets (lsa_core.mojo:573-604).
 * Sequence s (one query: q, out fp32 [batch][num_heads][head_dim]) attends exactly the key
 * positions keys[key_off[s] .. key_off[s+1]) of its own table -- softmax(scale * q.k) . V
 * over that set, with the reference's sum + 1e-10 denominator; p->window is ignored. An
 * empty list gives zeros (lsa_core.mojo:651-655). A list longer than max_keys, or a key
 * whose block lies outside the table or the pool, gives NaN outputs. keys, key_off (int32,
 * [batch + 1]) are device memory. Paged pools only (ring_size 0). Two launches. */
int32_t pkv_attend_sparse(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                          const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                          const int32_t* keys, const int32_t* key_off, int32_t max_keys,
                          int32_t batch, float* out, void* workspace, size_t workspace_bytes);

/* LSA bucket cache in device memory. The reference keeps one LSALayerIndex per kv slot and
 * global-layer group (model_speculative_moe_batched.mojo:1885-1888, :632); its bucket
 * cache (lsa_core.mojo:222-233) lives here as index instance i = kv_slot * 5 + group:
 *   int32 sizes[num_indices][max_buckets]        member count per bucket (<= 32);
 *   int32 members[num_indices][max_buckets][32]  token positions, in append order;
 *   int32 closed_blocks[num_indices], total_tokens[num_indices];
 * max_buckets = ceil(max_capacity / 512) * 32. Filling a block's buckets when its 512
 * tokens close (Ward clustering, lsa_core.mojo:325-518) and picking buckets
 * (select_top_p, :520-566) stay with the index on the host, which copies a closed
 * block's 32 sizes and member rows in. */

/* Longest key list pkv_lsa_expand can build: max(top_k, 1) + window_size + sink_size
 * (-1 if that overflows int32). Use it for keys_capacity / batch and as
 * pkv_attend_sparse's max_keys. */
int32_t pkv_lsa_max_keys(int32_t top_k, int32_t sink_size, int32_t window_size);

/* Bytes of workspace pkv_lsa_expand needs (the lists at a fixed stride, then their
 * lengths); 0 on invalid sizes. */
size_t pkv_lsa_expand_workspace_size(int32_t batch, int32_t top_k, int32_t sink_size,
                                     int32_t window_size);

/* LSALayerIndex.expand_buckets (lsa_core.mojo:568-604) for a batch of queries, writing
 * the CSR key lists pkv_attend_sparse takes. Sequence s uses index instance
 * index_ids[s] and its picked buckets picked[s * picked_stride + j], j < n_picked[s], in
 * order. Its list is the members of those buckets that lie in [sink_size, window_start),
 * in order, up to top_k of them (the reference stops once the list holds top_k after an
 * append, so top_k <= 0 keeps one); then the window [window_start, pos[s]] with
 * window_start = max(0, pos[s] + 1 - window_size); then the sinks [0, min(sink_size,
 * window_start, pos[s] + 1)). keys[key_off[s] .. key_off[s+1]) receives it; key_off is
 * int32 [batch + 1]. keys_capacity (int32 entries) must be >= batch *
 * pkv_lsa_max_keys(). status[s] = PKV_SEQ_BAD_INDEX when the index id, n_picked or a
 * bucket id is out of range (the offending part is skipped), else PKV_SEQ_OK. All arrays
 * are device memory; batch <= 1024; sink_size, window_size >= 0. Two launches. */
int32_t pkv_lsa_expand(void* stream, const int32_t* index_ids, const int32_t* picked,
                       int32_t picked_stride, const int32_t* n_picked, const int32_t* pos,
                       int32_t top_k, int32_t sink_size, int32_t window_size, int32_t batch,
                       const int32_t* sizes, const int32_t* members, int32_t num_indices,
                       int32_t max_buckets, int32_t* keys, int32_t* key_off,
                       int64_t keys_capacity, int32_t* status, void* workspace,
                       size_t workspace_bytes);

/* LSALayerIndex.rollback_to (lsa_core.mojo:287-303) -- and reset (:281-285) for targets
 * <= 0 -- as the engine calls it after verify (model_speculative_moe_batched.mojo:3368,
 * rollback_to(seq.pos) for each of the sequence's groups) and on admission (:2415,
 * :2432). Entry k applies to instance index_ids[k] with target_tokens[k], entries in
 * order: total_tokens = min(target, max_capacity); every closed 512-token block past
 * total_tokens / 512 reopens and its 32 buckets get size 0 (members and centroids stay, as
 * in the reference). Out-of-range ids are skipped. Device arrays; one launch. */
int32_t pkv_lsa_rollback(void* stream, const int32_t* index_ids, const int32_t* target_tokens,
                         int32_t count, int32_t num_indices, int32_t max_capacity,
                         int32_t max_buckets, int32_t* closed_blocks, int32_t* total_tokens,
                         int32_t* sizes);

/* K3 -- chunked-prefill attention over bf16 pages with bf16 MFMA (fp32 accumulation).
 * Replaces the engine's per-token prefill loop (append one token, then one
 * paged_attention_layer call for it: model_speculative_moe_batched.mojo:2600-2637 for
 * the chunked path, :2767-2833 for the CPU path) once the chunk's K/V rows have been
 * appended with pkv_append. Queries are ragged: sequence s owns query rows
 * q_off[s] .. q_off[s+1]-1 of q (bf16 [rows][num_heads][head_dim]) at positions
 * pos[s], pos[s]+1, ...; query i attends keys [window_start(pos[s]+i), pos[s]+i] of its
 * own table (prefix plus the causal part of the chunk). out: fp32 [rows][num_heads]
 * [head_dim]. kv_dtype must be PKV_DTYPE_BF16, head_dim 256, num_heads / num_kv_heads in
 * {1, 2, 4}, block_size >= 8 (the engine uses 16). max_q bounds q_off[s+1]-q_off[s] (it
 * sizes the grid: batch * num_kv_heads * ceil(max_q * G / 128) workgroups, at most
 * 2^32 / 512, else PKV_ERR_UNSUPPORTED) and max_pos bounds
 * pos[s] + its query count - 1; a sequence violating either, or whose table holds an
 * entry outside [0, num_blocks), gets NaN outputs; pos[s] < 0 gives zeros. One launch,
 * no workspace. q_off: int32 [batch + 1] (device). Paged pools only: ring_size > 0
 * gives PKV_ERR_UNSUPPORTED (a whole chunk appended into a ring would overwrite keys its
 * own earlier queries attend; ring layers prefill through pkv_attend in chunks of at
 * most ring_size - window + 1 queries, as the engine's per-token loop does). */
int32_t pkv_prefill(void* stream, const pkv_params* p, const void* q, const void* k_pool,
                    const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                    const int32_t* pos, const int32_t* q_off, int32_t max_q, int32_t batch,
                    int32_t max_pos, float* out);

/* K5 -- rollback / retire. No reference counterpart for draft rollback (the engine
 * leaves rejected rows in place and only advances pos, :3295-3368); retire is
 * model_speculative_moe_batched.mojo:3626-3628 and chat reset :2424-2439.
 * For each sequence s in index order with new_len[s] >= 0: keep
 * ceil(new_len[s] / block_size) table entries (never more than it holds) and push the
 * rest onto the back of the free list in ascending logical order. new_len[s] = 0
 * retires the sequence; new_len[s] < 0 leaves it untouched. Pool rows are not
 * modified. status (optional, int32 [batch]) receives PKV_SEQ_* per sequence. If any
 * length or freed entry is out of range, or the pushes would overflow the free list,
 * the call changes nothing and the offending sequences get PKV_SEQ_BAD_BLOCK /
 * PKV_SEQ_FREE_OVERFLOW. batch <= 4096. Block tables only: ring params (ring_size > 0)
 * give PKV_ERR_INVALID -- a ring layer keeps rejected draft rows in place, as the
 * engine does, and they are overwritten by the next appends at those positions. */
int32_t pkv_rollback(void* stream, const pkv_params* p, int32_t* block_tables,
                     int32_t table_stride, int32_t* table_lens, int32_t* free_list,
                     int32_t* free_count, const int32_t* new_len, int32_t batch,
                     int32_t* status);

/* Single-sequence drop-in with paged_attention_layer's argument list
 * (attention.mojo:240-256): q, k_pool, v_pool, block_table (device int32, at least
 * pos / block_size + 1 entries), block_size, pos, num_heads, num_kv_heads, head_dim,
 * window, attn_out. The reference's `scores` / `rows` scratch is replaced by
 * `workspace` (pkv_workspace_size(p, 1, 1, pos) bytes); the pool size and element
 * type the GPU needs for bounds checks come in num_blocks / kv_dtype. ring_size > 0
 * reads the ring starting at row ring_base (block_table is not read and may be NULL;
 * num_blocks counts rings): ring_base < 0, a ring ending past num_blocks * ring_size,
 * or more attended keys than ring_size give PKV_ERR_INVALID (the reference aborts,
 * attention.mojo:265-266). Softmax scale 1 (the reference has none). */
int32_t pkv_paged_attention_layer(void* stream, const float* q, const void* k_pool,
                                  const void* v_pool, const int32_t* block_table,
                                  int32_t block_size, int32_t pos, int32_t num_heads,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t window,
                                  float* attn_out, int32_t ring_size, int32_t ring_base,
                                  int32_t num_blocks, int32_t kv_dtype, void* workspace,
                                  size_t workspace_bytes);

/* Bytes of workspace pkv_q4_matmul needs (split-K partials and per-row-group arrival
 * counts); 0 on invalid sizes. */
size_t pkv_q4_matmul_workspace_size(int32_t c_in, int32_t c_out, int32_t batch);

/* Wo projection after attention -- batched Q4_0 matrix-vector products.
 * Replaces q4_matmul_vec (moe_kernels.mojo:59-163) as called on attn_out
 * (model_speculative_moe_batched.mojo:2011-2051), for `batch` input vectors at once:
 * out[s][r] = sum_k W[r][k] * x[s][k], x fp32 [batch][c_in] (e.g. pkv_attend's output,
 * c_in = num_heads * head_dim), out fp32 [batch][c_out]. W is in the reference's Q4_0
 * block-32 form (moe_kernels.mojo:7-57): w_packed uint8 [c_out][c_in / 2] (byte j of a
 * block: element 2j in the low nibble, 2j + 1 in the high one; value nibble - 8) and
 * scales fp32 [c_out][c_in / 32]. c_in % 32 == 0, batch <= 64; w_packed and x 16-byte,
 * scales 4-byte aligned (the weights are read in 16-byte chunks). Products are exact (bf16
 * matrix cores on a three-way split of x) and sums are fp32, added in a fixed order. The
 * workspace (16-byte aligned) must be zero-filled before its first use; every call leaves
 * its counters at zero again, so one workspace serves any sequence of calls on a stream.
 * One launch. */
int32_t pkv_q4_matmul(void* stream, const uint8_t* w_packed, const float* scales, const float* x,
                      int32_t c_in, int32_t c_out, int32_t batch, float* out, void* workspace,
                      size_t workspace_bytes);

/* Message for the calling thread's most recent error ("" if none). */
const char* pkv_last_error(void);

/* ABI version: (major << 16) | minor. */
int32_t pkv_version(void);

#ifdef __cplusplus
}
#endif

#endif /* PKV_H */
