/*
 * pkv_oracle.c -- CPU restatement of the reference paged KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker and the timed CPU
 * baseline; it is never part of the product. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load the library built from it.
 *
 * The reference is Mojo (phildrip/llm-mojo, mojo 1.0.0b2). Mojo is not available
 * to build or run, so each function below restates the reference code it cites.
 *
 *   oracle function                  reference (file:line)
 *   -------------------------------  ------------------------------------------------
 *   pkvo_window_start                attention.mojo:135-141
 *   pkvo_ring_row                    attention.mojo:144-148
 *   softmax_ref (static)             attention.mojo:151-162
 *   eval_head_range (static)         attention.mojo:165-237
 *   pkvo_paged_attention_layer       attention.mojo:240-294
 *   pkvo_legacy_paged_attention      test_attention.mojo:62-117 (pre-refactor engine loop)
 *   pkvo_attention_f64               test_attention.mojo:123-163 (float64 naive oracle)
 *   pkvo_lcg_* / pkvo_fill_random    test_attention.mojo:27-42
 *   pkvo_bm_*                        model_speculative_moe_batched.mojo:789-807 (BlockManager)
 *   pkvo_append                      model_speculative_moe_batched.mojo:1984-2001 (decode),
 *                                    :2513-2523 + :2621-2630 (chunked prefill),
 *                                    :2808-2825 (CPU prefill), :3011-3023 + :3106-3116 (verify)
 *   pkvo_ring_append                 ring-pool write sites :1996 (decode), :2625 (chunked
 *                                    prefill), :3111 (verify): row ring_row(kv_slot, ring, p)
 *   pkvo_rms_norm / _noscale         model_speculative_moe_batched.mojo:857-867, :870-878
 *   pkvo_apply_rope                  attention.mojo:24-66
 *   pkvo_apply_rope_qk               attention.mojo:69-132
 *   pkvo_ref_apply_rope              test_rope_and_parallel_attn.mojo:9-29 (scalar per-element
 *                                    restatement the reference asserts bit-exact with the above)
 *   pkvo_append_qkv                  the producer step before each append site: per-head
 *                                    rms_norm of Q / K, rms_norm_noscale of V, apply_rope_qk
 *                                    (:1974-1982 decode, :2612-2619 chunked prefill, :3099-3106
 *                                    verify; V := K before the norms on global layers,
 *                                    :1962-1964), then pkvo_append / pkvo_ring_append
 *   pkvo_append_qkv_f64              the same producer step in float64 (the fp32 angle of the
 *                                    reference, then exact arithmetic): the exact values both
 *                                    fp32 evaluations approximate
 *   pkvo_lsa_sparse_paged_attention  lsa_core.mojo:630-680 (attention over an explicit key list)
 *   pkvo_lsa_expand_buckets          lsa_core.mojo:573-604 (bucket members, window, sinks)
 *   pkvo_attend_sparse / _f64        lsa_sparse_paged_attention per sequence of a batch
 *   pkvo_lsa_reset                   LSALayerIndex.reset, lsa_core.mojo:281-285
 *   pkvo_lsa_rollback_to             LSALayerIndex.rollback_to, lsa_core.mojo:287-303
 *   pkvo_quantize_q4_0               moe_kernels.mojo:7-57 (Q4_0 block-32 quantization)
 *   pkvo_q4_matmul_vec               moe_kernels.mojo:59-163 (the Wo projection after attention,
 *                                    model_speculative_moe_batched.mojo:2011-2051)
 *   pkvo_scalar_q4                   test_q4_4row_tiling.mojo:14-34 (scalar dequantizing oracle)
 *   pkvo_q4_matmul_f64               the same product in float64
 *   pkvo_rollback                    retire :3626-3628 / reset :2424-2439 (ascending free order);
 *                                    truncation after rejected drafts has no reference code and
 *                                    follows the build's definition (keep ceil(len/bs) blocks,
 *                                    free the tail in ascending logical order).
 *   pkvo_attend                      execute_attention_for_token :601-657 / mtp_paged_attention
 *                                    :577-599, one paged_attention_layer call per query token
 *                                    (ring pools: ring_base = ring_row(kv_slot, ring, 0), :648).
 *
 * Bit-level notes (parity of the fp32 attention output is a tolerance, not bits):
 *   - SIMD[f32, 8] accumulation is restated as 8 independent lane accumulators; the
 *     horizontal reduce_add is a halving tree. Mojo's exact reduce order and its exp()
 *     are not pinned (the Mojo stdlib is absent); compile with -ffp-contract=off so no
 *     FMA contraction is introduced here.
 *   - bf16 pools are read by exact upcast (bits << 16), i.e. the reference run on the
 *     bf16-rounded values.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define PKVO_F32 0
#define PKVO_BF16 1

/* ---------------------------------------------------------------- helpers */

static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = ((uint32_t)b) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even fp32 -> bf16 (NaN kept quiet). */
uint16_t pkvo_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

void pkvo_f32_to_bf16_array(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = pkvo_f32_to_bf16(src[i]);
}

/* Load 8 consecutive pool elements as fp32 (SIMD[f32, 8] load). */
static inline void load8(const void* pool, int dtype, int64_t off, float* out) {
    if (dtype == PKVO_BF16) {
        const uint16_t* p = (const uint16_t*)pool + off;
        for (int j = 0; j < 8; ++j) out[j] = bf16_to_f32(p[j]);
    } else {
        const float* p = (const float*)pool + off;
        for (int j = 0; j < 8; ++j) out[j] = p[j];
    }
}

static inline float load1(const void* pool, int dtype, int64_t off) {
    if (dtype == PKVO_BF16) return bf16_to_f32(((const uint16_t*)pool)[off]);
    return ((const float*)pool)[off];
}

/* SIMD[f32, 8].reduce_add restated as a halving tree. */
static inline float reduce_add8(const float* a) {
    float b0 = a[0] + a[4], b1 = a[1] + a[5], b2 = a[2] + a[6], b3 = a[3] + a[7];
    float c0 = b0 + b2, c1 = b1 + b3;
    return c0 + c1;
}

/* ------------------------------------------------- attention.mojo:135-148 */

int64_t pkvo_window_start(int64_t pos, int64_t window) {
    if (window <= 0) return 0;
    int64_t start = pos - window + 1;
    return start > 0 ? start : 0;
}

int64_t pkvo_ring_row(int64_t slot, int64_t ring_size, int64_t t) {
    return slot * ring_size + t % ring_size;
}

/* ------------------------------------------------- attention.mojo:151-162 */

static void softmax_ref(float* scores, int64_t size) {
    float max_val = scores[0];
    for (int64_t i = 1; i < size; ++i)
        if (scores[i] > max_val) max_val = scores[i];
    float sum_exp = 0.0f;
    for (int64_t i = 0; i < size; ++i) {
        scores[i] = expf(scores[i] - max_val);
        sum_exp += scores[i];
    }
    for (int64_t i = 0; i < size; ++i) scores[i] /= (sum_exp + 1e-10f);
}

/* ------------------------------------------------- attention.mojo:165-237 */

static void eval_head_range(const float* q, const void* k_pool, const void* v_pool, int dtype,
                            const int64_t* rows, float* scores, float* attn_out, int64_t n,
                            int64_t g_offset, int64_t h_start, int64_t h_end, int64_t head_dim) {
    if (n <= 0) {
        for (int64_t h = h_start; h < h_end; ++h)
            for (int64_t d = 0; d < head_dim; ++d) attn_out[h * head_dim + d] = 0.0f;
        return;
    }
    float kv[8];
    /* 1. scores: head pairs share each K row load */
    for (int64_t i = 0; i < n; ++i) {
        int64_t k_off = rows[i] + g_offset;
        int64_t h = h_start;
        while (h + 1 < h_end) {
            const float* q0 = q + h * head_dim;
            const float* q1 = q + (h + 1) * head_dim;
            float s0[8] = {0}, s1[8] = {0};
            for (int64_t d = 0; d < head_dim; d += 8) {
                load8(k_pool, dtype, k_off + d, kv);
                for (int j = 0; j < 8; ++j) {
                    s0[j] = s0[j] + q0[d + j] * kv[j];
                    s1[j] = s1[j] + q1[d + j] * kv[j];
                }
            }
            scores[h * n + i] = reduce_add8(s0);
            scores[(h + 1) * n + i] = reduce_add8(s1);
            h += 2;
        }
        while (h < h_end) {
            const float* q0 = q + h * head_dim;
            float s0[8] = {0};
            for (int64_t d = 0; d < head_dim; d += 8) {
                load8(k_pool, dtype, k_off + d, kv);
                for (int j = 0; j < 8; ++j) s0[j] = s0[j] + q0[d + j] * kv[j];
            }
            scores[h * n + i] = reduce_add8(s0);
            h += 1;
        }
    }
    /* 2. softmax and zero-init output per head */
    for (int64_t h = h_start; h < h_end; ++h) {
        softmax_ref(scores + h * n, n);
        for (int64_t d = 0; d < head_dim; ++d) attn_out[h * head_dim + d] = 0.0f;
    }
    /* 3. values: head pairs share each V row load */
    for (int64_t i = 0; i < n; ++i) {
        int64_t v_off = rows[i] + g_offset;
        int64_t h = h_start;
        while (h + 1 < h_end) {
            float* o0 = attn_out + h * head_dim;
            float* o1 = attn_out + (h + 1) * head_dim;
            float a0 = scores[h * n + i], a1 = scores[(h + 1) * n + i];
            for (int64_t d = 0; d < head_dim; d += 8) {
                load8(v_pool, dtype, v_off + d, kv);
                for (int j = 0; j < 8; ++j) {
                    o0[d + j] = o0[d + j] + a0 * kv[j];
                    o1[d + j] = o1[d + j] + a1 * kv[j];
                }
            }
            h += 2;
        }
        while (h < h_end) {
            float* o0 = attn_out + h * head_dim;
            float a0 = scores[h * n + i];
            for (int64_t d = 0; d < head_dim; d += 8) {
                load8(v_pool, dtype, v_off + d, kv);
                for (int j = 0; j < 8; ++j) o0[d + j] = o0[d + j] + a0 * kv[j];
            }
            h += 1;
        }
    }
}

/* ------------------------------------------------- attention.mojo:240-294
 * Returns 0, or -1 when the ring is smaller than the attended window (the
 * reference aborts there, :265-266), or -2 when pos lies beyond the table
 * (the reference's debug_assert, :271).
 * nthreads > 1 runs the head-pair tasks on OpenMP threads, mirroring the
 * reference's parallelize over num_heads // 2 tasks (:276-287).            */
/* Key rows of paged_attention_layer (attention.mojo:258-274): rows[i] = pool offset of
 * key start_t + i. Returns n, or -1 / -2 as pkvo_paged_attention_layer. */
static int64_t pal_rows(const int64_t* block_table, int64_t table_len, int64_t block_size,
                        int64_t pos, int64_t kv_stride, int64_t window, int64_t* rows,
                        int64_t ring_size, int64_t ring_base) {
    int64_t start_t = pkvo_window_start(pos, window);
    int64_t n = pos + 1 - start_t;
    if (ring_size > 0) {
        if (n > ring_size) return -1;
        for (int64_t i = 0; i < n; ++i) {
            int64_t t = start_t + i;
            rows[i] = (ring_base + t % ring_size) * kv_stride;
        }
    } else {
        if (pos >= 0 && pos / block_size >= table_len) return -2;
        for (int64_t i = 0; i < n; ++i) {
            int64_t t = start_t + i;
            rows[i] = (block_table[t / block_size] * block_size + t % block_size) * kv_stride;
        }
    }
    return n < 0 ? 0 : n;
}

/* The head-pair dispatch condition of attention.mojo:276. */
static int pal_pairs(int64_t n, int64_t num_heads, int64_t ratio) {
    return n >= 64 && num_heads >= 4 && (num_heads % 2 == 0) && (ratio % 2 == 0);
}

int pkvo_paged_attention_layer(const float* q, const void* k_pool, const void* v_pool, int dtype,
                               const int64_t* block_table, int64_t table_len, int64_t block_size,
                               int64_t pos, int64_t num_heads, int64_t num_kv_heads,
                               int64_t head_dim, int64_t window, float* scores, int64_t* rows,
                               float* attn_out, int64_t ring_size, int64_t ring_base, int nthreads) {
    int64_t kv_stride = num_kv_heads * head_dim;
    int64_t ratio = num_heads / num_kv_heads;
    int64_t n = pal_rows(block_table, table_len, block_size, pos, kv_stride, window, rows,
                         ring_size, ring_base);
    if (n < 0) return (int)n;

    if (pal_pairs(n, num_heads, ratio)) {
        int64_t num_pairs = num_heads / 2;
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static, 1) if (nthreads > 1)
        for (int64_t t = 0; t < num_pairs; ++t) {
            int64_t h_start = t * 2;
            int64_t g = h_start / ratio;
            eval_head_range(q, k_pool, v_pool, dtype, rows, scores, attn_out, n, g * head_dim,
                            h_start, h_start + 2, head_dim);
        }
    } else {
        for (int64_t g = 0; g < num_kv_heads; ++g) {
            int64_t h_first = g * ratio;
            eval_head_range(q, k_pool, v_pool, dtype, rows, scores, attn_out, n, g * head_dim,
                            h_first, h_first + ratio, head_dim);
        }
    }
    return 0;
}

/* ------------------------------------------- test_attention.mojo:62-117
 * The engine's pre-refactor loop (full causal, one head at a time). The
 * reference asserts paged_attention_layer is bit-exact with it.           */
void pkvo_legacy_paged_attention(const float* q, const void* k_pool, const void* v_pool, int dtype,
                                 const int64_t* block_table, int64_t block_size, int64_t pos,
                                 int64_t layer_heads, int64_t layer_kv_heads,
                                 int64_t layer_head_dim, float* attn_scores, float* attn_out) {
    int64_t kv_stride = layer_kv_heads * layer_head_dim;
    int64_t ratio = layer_heads / layer_kv_heads;
    float kv[8];
    for (int64_t h = 0; h < layer_heads; ++h) {
        int64_t h_offset = h * layer_head_dim;
        int64_t g_offset = (h / ratio) * layer_head_dim;
        for (int64_t t = 0; t <= pos; ++t) {
            int64_t off = (block_table[t / block_size] * block_size + t % block_size) * kv_stride +
                          g_offset;
            float sv[8] = {0};
            for (int64_t d = 0; d < layer_head_dim; d += 8) {
                load8(k_pool, dtype, off + d, kv);
                for (int j = 0; j < 8; ++j) sv[j] = sv[j] + q[h_offset + d + j] * kv[j];
            }
            attn_scores[t] = reduce_add8(sv);
        }
        softmax_ref(attn_scores, pos + 1);
        for (int64_t d = 0; d < layer_head_dim; ++d) attn_out[h_offset + d] = 0.0f;
        for (int64_t t = 0; t <= pos; ++t) {
            int64_t off = (block_table[t / block_size] * block_size + t % block_size) * kv_stride +
                          g_offset;
            float a = attn_scores[t];
            for (int64_t d = 0; d < layer_head_dim; d += 8) {
                load8(v_pool, dtype, off + d, kv);
                for (int j = 0; j < 8; ++j)
                    attn_out[h_offset + d + j] = attn_out[h_offset + d + j] + a * kv[j];
            }
        }
    }
}

/* ------------------------------------------ test_attention.mojo:123-163
 * Naive float64 attention over keys [start_t, pos].                         */
void pkvo_attention_f64(const float* q, const void* k_pool, const void* v_pool, int dtype,
                        const int64_t* block_table, int64_t block_size, int64_t pos,
                        int64_t start_t, int64_t heads, int64_t kv_heads, int64_t head_dim,
                        double* out_ref) {
    int64_t kv_stride = kv_heads * head_dim;
    int64_t ratio = heads / kv_heads;
    int64_t n = pos + 1 - start_t;
    double* s = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
    for (int64_t h = 0; h < heads; ++h) {
        int64_t g = h / ratio;
        double mx = -1e300;
        for (int64_t i = 0; i < n; ++i) {
            int64_t t = start_t + i;
            int64_t row = (block_table[t / block_size] * block_size + t % block_size) * kv_stride +
                          g * head_dim;
            double acc = 0.0;
            for (int64_t d = 0; d < head_dim; ++d)
                acc += (double)q[h * head_dim + d] * (double)load1(k_pool, dtype, row + d);
            s[i] = acc;
            if (acc > mx) mx = acc;
        }
        double tot = 0.0;
        for (int64_t i = 0; i < n; ++i) {
            s[i] = exp(s[i] - mx);
            tot += s[i];
        }
        for (int64_t d = 0; d < head_dim; ++d) out_ref[h * head_dim + d] = 0.0;
        for (int64_t i = 0; i < n; ++i) {
            int64_t t = start_t + i;
            int64_t row = (block_table[t / block_size] * block_size + t % block_size) * kv_stride +
                          g * head_dim;
            double w = s[i] / tot;
            for (int64_t d = 0; d < head_dim; ++d)
                out_ref[h * head_dim + d] += w * (double)load1(v_pool, dtype, row + d);
        }
    }
    free(s);
}

/* -------------------------------------------- test_attention.mojo:27-42 */

uint64_t pkvo_lcg_init(uint64_t seed) {
    return seed * 6364136223846793005ULL + 1442695040888963407ULL;
}

/* Fills p[0..n) with uniform [-1, 1) * scale; returns the advanced state. */
uint64_t pkvo_fill_random(float* p, int64_t n, float scale, uint64_t state) {
    for (int64_t i = 0; i < n; ++i) {
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        uint64_t bits = (state >> 40) & 0xFFFFFFULL;
        float x = (float)bits / (float)0x800000 - 1.0f;
        p[i] = x * scale;
    }
    return state;
}

/* ------------------------- model_speculative_moe_batched.mojo:789-807
 * BlockManager: the free list is initialised [0..max-1]; allocate() pops the
 * back (-1 when empty); free() pushes to the back.                          */
void pkvo_bm_init(int32_t* free_list, int32_t* free_count, int32_t max_blocks) {
    for (int32_t i = 0; i < max_blocks; ++i) free_list[i] = i;
    *free_count = max_blocks;
}

int32_t pkvo_bm_allocate(int32_t* free_list, int32_t* free_count) {
    if (*free_count == 0) return -1;
    *free_count -= 1;
    return free_list[*free_count];
}

void pkvo_bm_free(int32_t* free_list, int32_t* free_count, int32_t block_id) {
    free_list[*free_count] = block_id;
    *free_count += 1;
}

/* ------------------------------------------------------------- KV append
 * Sequence s appends n_s = tok_off[s+1] - tok_off[s] tokens whose K / V rows are rows
 * tok_off[s] .. tok_off[s+1]-1 of k_new / v_new ([total_rows][kv_stride], pool dtype).
 * For each sequence s in index order (the engine serves sequences one after
 * another): for each new token b in order, position p = pos[s] + b grows the
 * table while p // bs >= len(table) (allocate() pops the LIFO back). If a pop
 * fails the sequence is marked out of blocks (status -1): blocks popped before
 * the failure stay in its table and none of its K/V rows is written (decode
 * returns before the copy, :1989-1992; verify sets oom_abort before any write,
 * :3017-3026; chunked prefill breaks before the layer pass, :2516-2530).
 * Otherwise the rows row = table[p // bs] * bs + p % bs receive exact copies
 * of the new rows (:1994-2001).
 * pos[s] < 0 or n_s <= 0 skips the sequence (status 0). A token range outside
 * [0, total_rows) or longer than max_new is rejected with status -5 (the C ABI's
 * PKV_SEQ_BAD_ARGS); a table that would exceed table_stride entries gives status -2
 * (PKV_SEQ_TABLE_FULL). Neither changes anything.                              */
void pkvo_append(int dtype, int32_t kv_stride, int32_t block_size, void* k_pool, void* v_pool,
                 int32_t* tables, int32_t table_stride, int32_t* table_lens, int32_t* free_list,
                 int32_t* free_count, const int32_t* pos, const int32_t* tok_off, int32_t max_new,
                 const void* k_new, const void* v_new, int32_t total_rows, int32_t batch,
                 int32_t* status) {
    size_t elt = dtype == PKVO_BF16 ? 2 : 4;
    for (int32_t s = 0; s < batch; ++s) {
        status[s] = 0;
        int32_t r0 = tok_off[s], n = tok_off[s + 1] - tok_off[s];
        if (pos[s] < 0 || n <= 0) continue;
        if (n > max_new || r0 < 0 || tok_off[s + 1] > total_rows) {
            status[s] = -5;
            continue;
        }
        int64_t last = (int64_t)pos[s] + n - 1;
        if (last / block_size >= table_stride) {
            status[s] = -2;
            continue;
        }
        int32_t* table = tables + (int64_t)s * table_stride;
        int oom = 0;
        for (int32_t b = 0; b < n && !oom; ++b) {
            int64_t p = (int64_t)pos[s] + b;
            while (p / block_size >= table_lens[s]) {
                int32_t blk = pkvo_bm_allocate(free_list, free_count);
                if (blk < 0) {
                    oom = 1;
                    break;
                }
                table[table_lens[s]] = blk;
                table_lens[s] += 1;
            }
        }
        if (oom) {
            status[s] = -1;
            continue;
        }
        for (int32_t b = 0; b < n; ++b) {
            int64_t p = (int64_t)pos[s] + b;
            int64_t row = (int64_t)table[p / block_size] * block_size + p % block_size;
            size_t src = ((size_t)r0 + b) * kv_stride * elt;
            memcpy((char*)k_pool + row * kv_stride * elt, (const char*)k_new + src, kv_stride * elt);
            memcpy((char*)v_pool + row * kv_stride * elt, (const char*)v_new + src, kv_stride * elt);
        }
    }
}

/* ------------------------------------------------------------ ring append
 * Ring pools (the engine's default for sliding layers, …batched.mojo:1301-1304,
 * :1440-1442): sequence s owns ring slot slots[s * slot_stride] of num_slots, and each
 * new token at position p is copied to row ring_row(slot, ring_size, p)
 * (attention.mojo:144-148) as at the write sites :1996, :2625, :3111. No block is
 * allocated. Tokens are written in order, so of more than ring_size new tokens the last
 * ring_size remain. Status as pkvo_append: -5 for a bad token range, -3 (the C ABI's
 * PKV_SEQ_BAD_BLOCK) for a slot outside [0, num_slots); neither writes anything. */
void pkvo_ring_append(int dtype, int32_t kv_stride, int32_t ring_size, int32_t num_slots,
                      void* k_pool, void* v_pool, const int32_t* slots, int32_t slot_stride,
                      const int32_t* pos, const int32_t* tok_off, int32_t max_new,
                      const void* k_new, const void* v_new, int32_t total_rows, int32_t batch,
                      int32_t* status) {
    size_t elt = dtype == PKVO_BF16 ? 2 : 4;
    for (int32_t s = 0; s < batch; ++s) {
        status[s] = 0;
        int32_t r0 = tok_off[s], n = tok_off[s + 1] - tok_off[s];
        if (pos[s] < 0 || n <= 0) continue;
        if (n > max_new || r0 < 0 || tok_off[s + 1] > total_rows) {
            status[s] = -5;
            continue;
        }
        int32_t slot = slots[(int64_t)s * slot_stride];
        if (slot < 0 || slot >= num_slots) {
            status[s] = -3;
            continue;
        }
        for (int32_t b = 0; b < n; ++b) {
            int64_t row = pkvo_ring_row(slot, ring_size, (int64_t)pos[s] + b);
            size_t src = ((size_t)r0 + b) * kv_stride * elt;
            memcpy((char*)k_pool + row * kv_stride * elt, (const char*)k_new + src, kv_stride * elt);
            memcpy((char*)v_pool + row * kv_stride * elt, (const char*)v_new + src, kv_stride * elt);
        }
    }
}

/* ----------------------------------------- model_speculative_moe_batched.mojo:857-878
 * rms_norm: SIMD[f32, 8] sum of squares, reduce_add, 1 / sqrt(ss / size + 1e-6), then
 * v * inv_rms * weight. rms_norm_noscale omits the weight. size % 8 == 0.           */
static float sum_squares8(const float* x, int64_t size) {
    float acc[8] = {0};
    for (int64_t i = 0; i < size; i += 8)
        for (int j = 0; j < 8; ++j) acc[j] = acc[j] + x[i + j] * x[i + j];
    return reduce_add8(acc);
}

void pkvo_rms_norm(const float* x, const float* w, float* out, int64_t size) {
    float inv_rms = 1.0f / sqrtf(sum_squares8(x, size) / (float)size + 1e-6f);
    for (int64_t i = 0; i < size; ++i) out[i] = x[i] * inv_rms * w[i];
}

void pkvo_rms_norm_noscale(const float* x, float* out, int64_t size) {
    float inv_rms = 1.0f / sqrtf(sum_squares8(x, size) / (float)size + 1e-6f);
    for (int64_t i = 0; i < size; ++i) out[i] = x[i] * inv_rms;
}

/* ------------------------------------------------- attention.mojo:24-132
 * Rotary embedding of every head of `vec` at position pos. Sliding layers rotate all
 * head_dim / 2 pairs (i, i + head_dim / 2) with base 1e4 over rope_dim 256; global
 * layers rotate only the first min(64, head_dim / 2) pairs, base 1e6 over rope_dim 512.
 * theta_i = pos / base^(2i / rope_dim) in fp32; cos / sin computed once per call.   */
static int rope_tables(int64_t head_dim, int64_t pos, int is_global, float* cos_arr,
                       float* sin_arr) {
    int64_t half_dim = head_dim / 2;
    int64_t rotary_half = is_global ? (half_dim < 64 ? half_dim : 64) : half_dim;
    float base = is_global ? 1000000.0f : 10000.0f;
    float rope_dim = is_global ? 512.0f : 256.0f;
    float pos_f = (float)pos;
    for (int64_t i = 0; i < rotary_half; ++i) {
        float theta = pos_f / powf(base, (float)(2 * i) / rope_dim);
        cos_arr[i] = cosf(theta);
        sin_arr[i] = sinf(theta);
    }
    return (int)rotary_half;
}

static void rope_heads(float* vec, int64_t num_heads, int64_t head_dim, int rotary_half,
                       const float* c, const float* sn) {
    int64_t half_dim = head_dim / 2;
    for (int64_t h = 0; h < num_heads; ++h) {
        float* v1 = vec + h * head_dim;
        float* v2 = v1 + half_dim;
        for (int i = 0; i < rotary_half; ++i) {
            float a = v1[i], b = v2[i];
            v1[i] = a * c[i] - b * sn[i];
            v2[i] = b * c[i] + a * sn[i];
        }
    }
}

void pkvo_apply_rope(float* vec, int64_t num_heads, int64_t head_dim, int64_t pos,
                     int is_global) {
    float c[256], sn[256];
    int rh = rope_tables(head_dim, pos, is_global, c, sn);
    rope_heads(vec, num_heads, head_dim, rh, c, sn);
}

void pkvo_apply_rope_qk(float* q, float* k, int64_t num_q_heads, int64_t num_kv_heads,
                        int64_t head_dim, int64_t pos, int is_global) {
    float c[256], sn[256];
    int rh = rope_tables(head_dim, pos, is_global, c, sn);
    rope_heads(q, num_q_heads, head_dim, rh, c, sn);
    rope_heads(k, num_kv_heads, head_dim, rh, c, sn);
}

/* ------------------------------ test_rope_and_parallel_attn.mojo:9-29
 * The reference's scalar RoPE: theta per element (0 for global pairs >= 64).       */
void pkvo_ref_apply_rope(float* vec, int64_t num_heads, int64_t head_dim, int64_t pos,
                         int is_global) {
    int64_t half_dim = head_dim / 2;
    float base = is_global ? 1000000.0f : 10000.0f;
    int64_t rope_dim = is_global ? 512 : 256;
    for (int64_t h = 0; h < num_heads; ++h) {
        int64_t off = h * head_dim;
        for (int64_t i = 0; i < half_dim; ++i) {
            float theta = 0.0f;
            if (!is_global || i < 64)
                theta = (float)pos / powf(base, (float)(2 * i) / (float)rope_dim);
            float ct = cosf(theta), st = sinf(theta);
            float v1 = vec[off + i], v2 = vec[off + half_dim + i];
            vec[off + i] = v1 * ct - v2 * st;
            vec[off + half_dim + i] = v2 * ct + v1 * st;
        }
    }
}

/* --------------------------------------------------- fused producer + append
 * The engine's per-token producer step before each KV write (decode :1974-1982,
 * chunked prefill :2612-2619, verify :3099-3106): per head, q = rms_norm(q, q_norm_w),
 * k = rms_norm(k, k_norm_w), v = rms_norm_noscale(v); then apply_rope_qk(q, k) at the
 * token's position. v == NULL gives V := K as read, before any norm (global layers,
 * attention_k_eq_v, :1962-1964). Rows are ragged as in pkvo_append: sequence s owns
 * input rows tok_off[s] .. tok_off[s+1]-1 at positions pos[s], pos[s] + 1, ...
 * q_out (fp32 [total_rows][Hq][D]) receives the processed Q of every sequence with a
 * valid token range (pos >= 0, 0 < n <= max_new, rows inside total_rows); rows of other
 * sequences are not written. The processed K / V rows (rounded to bf16 for bf16 pools)
 * then go through pkvo_append (ring_size == 0) or pkvo_ring_append (ring_size > 0, where
 * tables[s * table_stride] is the ring slot and num_blocks counts ring slots).     */
void pkvo_append_qkv(int dtype, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                     int32_t block_size, int32_t ring_size, int32_t num_blocks, int is_global,
                     void* k_pool, void* v_pool, int32_t* tables, int32_t table_stride,
                     int32_t* table_lens, int32_t* free_list, int32_t* free_count,
                     const int32_t* pos, const int32_t* tok_off, int32_t max_new, const float* q,
                     const float* k, const float* v, const float* q_norm_w,
                     const float* k_norm_w, float* q_out, int32_t total_rows, int32_t batch,
                     int32_t* status) {
    int64_t D = head_dim, qs = (int64_t)num_heads * D, ks = (int64_t)num_kv_heads * D;
    size_t elt = dtype == PKVO_BF16 ? 2 : 4;
    float* kn = (float*)calloc((size_t)(total_rows > 0 ? total_rows : 1) * ks, sizeof(float));
    float* vn = (float*)calloc((size_t)(total_rows > 0 ? total_rows : 1) * ks, sizeof(float));
    void* kc = calloc((size_t)(total_rows > 0 ? total_rows : 1) * ks, elt);
    void* vc = calloc((size_t)(total_rows > 0 ? total_rows : 1) * ks, elt);
    for (int32_t s = 0; s < batch; ++s) {
        int32_t r0 = tok_off[s], n = tok_off[s + 1] - tok_off[s];
        if (pos[s] < 0 || n <= 0 || n > max_new || r0 < 0 || tok_off[s + 1] > total_rows)
            continue;
        for (int32_t b = 0; b < n; ++b) {
            int64_t r = (int64_t)r0 + b;
            float* qo = q_out + r * qs;
            float* ko = kn + r * ks;
            float* vo = vn + r * ks;
            const float* vsrc = v ? v + r * ks : k + r * ks;
            for (int64_t h = 0; h < num_heads; ++h)
                pkvo_rms_norm(q + r * qs + h * D, q_norm_w, qo + h * D, D);
            for (int64_t h = 0; h < num_kv_heads; ++h) {
                pkvo_rms_norm(k + r * ks + h * D, k_norm_w, ko + h * D, D);
                pkvo_rms_norm_noscale(vsrc + h * D, vo + h * D, D);
            }
            pkvo_apply_rope_qk(qo, ko, num_heads, num_kv_heads, D, (int64_t)pos[s] + b,
                               is_global);
        }
    }
    int64_t nall = (int64_t)(total_rows > 0 ? total_rows : 0) * ks;
    if (dtype == PKVO_BF16) {
        pkvo_f32_to_bf16_array(kn, (uint16_t*)kc, nall);
        pkvo_f32_to_bf16_array(vn, (uint16_t*)vc, nall);
    } else {
        memcpy(kc, kn, (size_t)nall * 4);
        memcpy(vc, vn, (size_t)nall * 4);
    }
    if (ring_size > 0)
        pkvo_ring_append(dtype, (int32_t)ks, ring_size, num_blocks, k_pool, v_pool, tables,
                         table_stride, pos, tok_off, max_new, kc, vc, total_rows, batch, status);
    else
        pkvo_append(dtype, (int32_t)ks, block_size, k_pool, v_pool, tables, table_stride,
                    table_lens, free_list, free_count, pos, tok_off, max_new, kc, vc, total_rows,
                    batch, status);
    free(kn);
    free(vn);
    free(kc);
    free(vc);
}

/* ------------------------------------------- float64 producer step
 * pkvo_append_qkv's processed rows in float64: rms_norm / rms_norm_noscale and the
 * rotation evaluated exactly (double) from the reference's fp32 angles
 * theta_i = (float)pos / powf(base, 2i / rope_dim). Writes q_out / k_out / v_out
 * (double, input row layout) for every sequence with a usable token range.       */
void pkvo_append_qkv_f64(int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                         int is_global, const int32_t* pos, const int32_t* tok_off,
                         int32_t max_new, const float* q, const float* k, const float* v,
                         const float* q_norm_w, const float* k_norm_w, int32_t total_rows,
                         int32_t batch, double* q_out, double* k_out, double* v_out) {
    int64_t D = head_dim, half = D / 2;
    int64_t rotary_half = is_global ? (half < 64 ? half : 64) : half;
    float base = is_global ? 1000000.0f : 10000.0f;
    float rope_dim = is_global ? 512.0f : 256.0f;
    for (int32_t s = 0; s < batch; ++s) {
        int32_t r0 = tok_off[s], n = tok_off[s + 1] - tok_off[s];
        if (pos[s] < 0 || n <= 0 || n > max_new || r0 < 0 || tok_off[s + 1] > total_rows)
            continue;
        for (int32_t b = 0; b < n; ++b) {
            int64_t r = (int64_t)r0 + b;
            float pos_f = (float)((int64_t)pos[s] + b);
            double c[256], sn[256];
            for (int64_t i = 0; i < rotary_half; ++i) {
                float theta = pos_f / powf(base, (float)(2 * i) / rope_dim);
                c[i] = cos((double)theta);
                sn[i] = sin((double)theta);
            }
            for (int kind = 0; kind < 3; ++kind) {
                int64_t heads = kind == 0 ? num_heads : num_kv_heads;
                const float* src = kind == 0 ? q : (kind == 1 || !v ? k : v);
                const float* w = kind == 0 ? q_norm_w : (kind == 1 ? k_norm_w : NULL);
                double* dst = kind == 0 ? q_out : (kind == 1 ? k_out : v_out);
                for (int64_t h = 0; h < heads; ++h) {
                    const float* x = src + (r * heads + h) * D;
                    double* y = dst + (r * heads + h) * D;
                    double ss = 0.0;
                    for (int64_t d = 0; d < D; ++d) ss += (double)x[d] * (double)x[d];
                    double inv = 1.0 / sqrt(ss / (double)D + (double)1e-6f);
                    for (int64_t d = 0; d < D; ++d) y[d] = (double)x[d] * inv * (w ? (double)w[d] : 1.0);
                    if (kind == 2) continue;
                    for (int64_t i = 0; i < rotary_half; ++i) {
                        double a = y[i], bb = y[half + i];
                        y[i] = a * c[i] - bb * sn[i];
                        y[half + i] = bb * c[i] + a * sn[i];
                    }
                }
            }
        }
    }
}

/* ------------------------------------------------- lsa_core.mojo:630-680
 * Sparse paged attention over the key positions selected[0 .. n_sel): rows from the
 * block table, then the dispatch of paged_attention_layer (head pairs on `nthreads`
 * threads when n_sel >= 64) over the same _eval_head_range. n_sel == 0 gives zeros.  */
void pkvo_lsa_sparse_paged_attention(const float* q, const void* k_pool, const void* v_pool,
                                     int dtype, const int64_t* block_table, int64_t block_size,
                                     const int64_t* selected, int64_t n_sel, int64_t num_heads,
                                     int64_t num_kv_heads, int64_t head_dim, float* scores,
                                     int64_t* rows, float* out, int nthreads) {
    if (n_sel == 0) {
        for (int64_t i = 0; i < num_heads * head_dim; ++i) out[i] = 0.0f;
        return;
    }
    int64_t kv_stride = num_kv_heads * head_dim;
    int64_t ratio = num_heads / num_kv_heads;
    for (int64_t idx = 0; idx < n_sel; ++idx) {
        int64_t t = selected[idx];
        rows[idx] = (block_table[t / block_size] * block_size + t % block_size) * kv_stride;
    }
    if (n_sel >= 64 && num_heads >= 4 && (num_heads % 2 == 0) && (ratio % 2 == 0)) {
#pragma omp parallel for num_threads(nthreads > 0 ? nthreads : 1) schedule(static, 1) if (nthreads > 1)
        for (int64_t t = 0; t < num_heads / 2; ++t) {
            int64_t h_start = t * 2;
            eval_head_range(q, k_pool, v_pool, dtype, rows, scores, out, n_sel,
                            (h_start / ratio) * head_dim, h_start, h_start + 2, head_dim);
        }
    } else {
        for (int64_t g = 0; g < num_kv_heads; ++g)
            eval_head_range(q, k_pool, v_pool, dtype, rows, scores, out, n_sel, g * head_dim,
                            g * ratio, g * ratio + ratio, head_dim);
    }
}

/* ------------------------------------------------- lsa_core.mojo:573-604
 * Expands picked buckets into the key list: members of each picked bucket (in order) that
 * lie in [sink_size, window_start), stopping at top_k of them; then the window
 * [window_start, pos] with window_start = max(0, pos + 1 - window_size); then the sinks
 * [0, min(sink_size, window_start, pos + 1)). members is [bucket][bucket_cap]. Returns
 * the count written to out (at most top_k + window_size + sink_size entries).        */
int64_t pkvo_lsa_expand_buckets(const int64_t* picked, int64_t n_picked, const int64_t* sizes,
                                const int64_t* members, int64_t bucket_cap, int64_t pos,
                                int64_t top_k, int64_t sink_size, int64_t window_size,
                                int64_t* out) {
    int64_t window_start = pos + 1 - window_size;
    if (window_start < 0) window_start = 0;
    int64_t n = 0;
    for (int64_t bi = 0; bi < n_picked; ++bi) {
        int64_t b = picked[bi];
        for (int64_t m = 0; m < sizes[b]; ++m) {
            int64_t tok = members[b * bucket_cap + m];
            if (tok >= sink_size && tok < window_start) {
                out[n++] = tok;
                if (n >= top_k) break;
            }
        }
        if (n >= top_k) break;
    }
    for (int64_t t = window_start; t <= pos; ++t) out[n++] = t;
    int64_t sink_limit = sink_size < window_start ? sink_size : window_start;
    if (pos + 1 < sink_limit) sink_limit = pos + 1;
    for (int64_t t = 0; t < sink_limit; ++t) out[n++] = t;
    return n;
}

/* ------------------------------------------------ lsa_core.mojo:281-303
 * LSALayerIndex.reset and rollback_to on the index's integer state: the number of closed
 * 512-token cluster blocks, the tokens appended, and the member count of each bucket (32
 * buckets per block). rollback_to keeps min(target, max_capacity) tokens and reopens every
 * closed block from that count / 512 on, emptying its buckets; members and centroids are
 * left in place. (The reference asserts that at most one block reopens, :294-298, a
 * debug_assert; its loop handles any number, and so does this one.)                   */
void pkvo_lsa_reset(int64_t max_buckets, int64_t* closed_blocks, int64_t* total_tokens,
                    int64_t* sizes) {
    *closed_blocks = 0;
    *total_tokens = 0;
    for (int64_t i = 0; i < max_buckets; ++i) sizes[i] = 0;
}

void pkvo_lsa_rollback_to(int64_t max_capacity, int64_t max_buckets, int64_t* closed_blocks,
                          int64_t* total_tokens, int64_t* sizes, int64_t target_tokens) {
    if (target_tokens <= 0) {
        pkvo_lsa_reset(max_buckets, closed_blocks, total_tokens, sizes);
        return;
    }
    const int64_t clamped = target_tokens < max_capacity ? target_tokens : max_capacity;
    *total_tokens = clamped;
    const int64_t valid_closed = clamped / 512;
    while (*closed_blocks > valid_closed) {
        *closed_blocks -= 1;
        const int64_t base = *closed_blocks * 32;
        for (int64_t i = 0; i < 32; ++i) sizes[base + i] = 0;
    }
}

/* ------------------------------------------------ batched sparse attention
 * Sequence s attends the key positions keys[key_off[s] .. key_off[s+1]) through its
 * table (one lsa_sparse_paged_attention call); q / out are [batch][num_heads][head_dim].
 * q_scale multiplies q first (a power of two, exact). par: as pkvo_attend (0: head-pair
 * tasks on nthreads threads; 1: sequences spread over the threads).                  */
void pkvo_attend_sparse(int dtype, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                        int32_t block_size, float q_scale, const float* q, const void* k_pool,
                        const void* v_pool, const int32_t* tables, int32_t table_stride,
                        const int32_t* keys, const int32_t* key_off, int32_t batch, float* out,
                        int nthreads, int par) {
    int64_t hd = (int64_t)num_heads * head_dim;
    int64_t max_n = 1;
    for (int32_t s = 0; s < batch; ++s)
        if (key_off[s + 1] - key_off[s] > max_n) max_n = key_off[s + 1] - key_off[s];
    int outer = (par >= 1 && nthreads > 1) ? nthreads : 1;
    int inner = par >= 1 ? 1 : nthreads;
#pragma omp parallel num_threads(outer) if (outer > 1)
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)(num_heads * max_n));
        int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * (size_t)max_n);
        int64_t* sel = (int64_t*)malloc(sizeof(int64_t) * (size_t)max_n);
        int64_t* tab = (int64_t*)malloc(sizeof(int64_t) * (size_t)(table_stride > 0 ? table_stride : 1));
        float* qs = (float*)malloc(sizeof(float) * (size_t)hd);
#pragma omp for schedule(dynamic, 1)
        for (int32_t s = 0; s < batch; ++s) {
            int64_t n = key_off[s + 1] - key_off[s];
            for (int32_t i = 0; i < table_stride; ++i) tab[i] = tables[(int64_t)s * table_stride + i];
            for (int64_t i = 0; i < n; ++i) sel[i] = keys[key_off[s] + i];
            for (int64_t i = 0; i < hd; ++i) qs[i] = q[s * hd + i] * q_scale;
            pkvo_lsa_sparse_paged_attention(qs, k_pool, v_pool, dtype, tab, block_size, sel, n,
                                            num_heads, num_kv_heads, head_dim, scores, rows,
                                            out + s * hd, inner);
        }
        free(scores);
        free(rows);
        free(sel);
        free(tab);
        free(qs);
    }
}

/* The same in float64 (test_attention.mojo:123-163's naive oracle over the listed keys,
 * read through a one-row-per-block table). n = 0 gives zeros.                      */
void pkvo_attend_sparse_f64(int dtype, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                            int32_t block_size, float q_scale, const float* q,
                            const void* k_pool, const void* v_pool, const int32_t* tables,
                            int32_t table_stride, const int32_t* keys, const int32_t* key_off,
                            int32_t batch, double* out) {
    int64_t hd = (int64_t)num_heads * head_dim;
    float* qs = (float*)malloc(sizeof(float) * (size_t)hd);
    for (int32_t s = 0; s < batch; ++s) {
        int64_t n = key_off[s + 1] - key_off[s];
        if (n <= 0) {
            for (int64_t i = 0; i < hd; ++i) out[s * hd + i] = 0.0;
            continue;
        }
        int64_t* tab = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
        for (int64_t i = 0; i < n; ++i) {
            int64_t t = keys[key_off[s] + i];
            tab[i] = (int64_t)tables[(int64_t)s * table_stride + t / block_size] * block_size +
                     t % block_size;
        }
        for (int64_t i = 0; i < hd; ++i) qs[i] = q[s * hd + i] * q_scale;
        pkvo_attention_f64(qs, k_pool, v_pool, dtype, tab, 1, n - 1, 0, num_heads, num_kv_heads,
                           head_dim, out + s * hd);
        free(tab);
    }
    free(qs);
}

/* ----------------------------------------------------- moe_kernels.mojo:7-57
 * Q4_0 block-32: per block of 32 values, scale = max(max|v| / 7, 1e-5); q = clamp(round(v /
 * scale), -8, 7) + 8; byte j of the block's 16 holds element 2j in its low nibble and
 * element 2j + 1 in its high nibble. round() is restated as roundf (halves away from
 * zero); the rounding of exact halves is not pinned to Mojo's.                       */
void pkvo_quantize_q4_0(const float* src, uint8_t* packed, float* scales, int64_t n) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* v = src + b * 32;
        float max_abs = 0.0f;
        for (int i = 0; i < 32; ++i) {
            float a = fabsf(v[i]);
            if (a > max_abs) max_abs = a;
        }
        float scale = max_abs / 7.0f;
        if (scale < 1e-5f) scale = 1e-5f;
        scales[b] = scale;
        float inv = 1.0f / scale;
        for (int j = 0; j < 16; ++j) {
            float q0 = roundf(v[2 * j] * inv), q1 = roundf(v[2 * j + 1] * inv);
            q0 = q0 < -8.0f ? -8.0f : (q0 > 7.0f ? 7.0f : q0);
            q1 = q1 < -8.0f ? -8.0f : (q1 > 7.0f ? 7.0f : q1);
            packed[b * 16 + j] = (uint8_t)((uint8_t)(q0 + 8.0f) | ((uint8_t)(q1 + 8.0f) << 4));
        }
    }
}

/* SIMD[f32, 16].reduce_add as a halving tree. */
static inline float reduce_add16(const float* a) {
    float h[8];
    for (int j = 0; j < 8; ++j) h[j] = a[j] + a[j + 8];
    return reduce_add8(h);
}

/* ---------------------------------------------------- moe_kernels.mojo:59-163
 * out[r] = sum over blocks b of the dequantized row times x: x is split into its even and
 * odd elements per block ("dual-space deinterleave"); per block and lane j < 16,
 * acc[j] = fma(we[j], xe[j], fma(wo[j], xo[j], acc[j])) with we / wo = (nibble - 8) * scale;
 * finally out[r] = reduce_add(acc). The reference's 2-row and 1-row loops do the same per
 * row.                                                                              */
void pkvo_q4_matmul_vec(const uint8_t* w_packed, const float* scales, const float* x, float* out,
                        int64_t c_in, int64_t c_out) {
    int64_t cp = c_in / 2, nb = c_in / 32;
    for (int64_t r = 0; r < c_out; ++r) {
        float acc[16] = {0};
        for (int64_t b = 0; b < nb; ++b) {
            float sc = scales[r * nb + b];
            const uint8_t* bytes = w_packed + r * cp + b * 16;
            for (int j = 0; j < 16; ++j) {
                float we = (float)((int)(bytes[j] & 15) - 8) * sc;
                float wo = (float)((int)(bytes[j] >> 4) - 8) * sc;
                float xe = x[b * 32 + 2 * j], xo = x[b * 32 + 2 * j + 1];
                acc[j] = fmaf(we, xe, fmaf(wo, xo, acc[j]));
            }
        }
        out[r] = reduce_add16(acc);
    }
}

/* -------------------------------------------- test_q4_4row_tiling.mojo:14-34
 * Independent scalar dequantizing oracle: per block, sum w_lo * x[2j] + w_hi * x[2j+1]
 * over the 16 bytes, times the scale, accumulated over blocks.                       */
void pkvo_scalar_q4(const uint8_t* w_packed, const float* scales, const float* x, float* out,
                    int64_t c_in, int64_t c_out) {
    int64_t cp = c_in / 2, nb = c_in / 32;
    for (int64_t r = 0; r < c_out; ++r) {
        float row_sum = 0.0f;
        for (int64_t b = 0; b < nb; ++b) {
            float sc = scales[r * nb + b];
            float blk = 0.0f;
            for (int j = 0; j < 16; ++j) {
                int byte = w_packed[r * cp + b * 16 + j];
                float w_lo = (float)((byte & 15) - 8), w_hi = (float)((byte >> 4) - 8);
                blk = blk + (w_lo * x[b * 32 + 2 * j] + w_hi * x[b * 32 + 2 * j + 1]);
            }
            row_sum = row_sum + blk * sc;
        }
        out[r] = row_sum;
    }
}

/* The dequantized product in float64 (the exact value both fp32 forms approximate).  */
void pkvo_q4_matmul_f64(const uint8_t* w_packed, const float* scales, const float* x,
                        double* out, int64_t c_in, int64_t c_out) {
    int64_t cp = c_in / 2, nb = c_in / 32;
    for (int64_t r = 0; r < c_out; ++r) {
        double sum = 0.0;
        for (int64_t b = 0; b < nb; ++b) {
            double sc = scales[r * nb + b];
            for (int j = 0; j < 16; ++j) {
                int byte = w_packed[r * cp + b * 16 + j];
                sum += ((double)((byte & 15) - 8) * sc) * (double)x[b * 32 + 2 * j] +
                       ((double)((byte >> 4) - 8) * sc) * (double)x[b * 32 + 2 * j + 1];
            }
        }
        out[r] = sum;
    }
}

/* ------------------------------------------------------- rollback / retire
 * For each sequence s in index order with new_len[s] >= 0: keep
 * ceil(new_len / bs) blocks (never more than it holds) and free the rest in
 * ascending logical order, pushing each on the back of the free list. Retire
 * is new_len = 0 (the engine frees table[0..len) ascending, :3627-3628).
 * new_len[s] < 0 leaves sequence s untouched. Pool rows are not modified.   */
void pkvo_rollback(int32_t block_size, int32_t* tables, int32_t table_stride, int32_t* table_lens,
                   int32_t* free_list, int32_t* free_count, const int32_t* new_len, int32_t batch) {
    for (int32_t s = 0; s < batch; ++s) {
        if (new_len[s] < 0) continue;
        int32_t keep = (new_len[s] + block_size - 1) / block_size;
        if (keep > table_lens[s]) keep = table_lens[s];
        int32_t* table = tables + (int64_t)s * table_stride;
        for (int32_t j = keep; j < table_lens[s]; ++j) pkvo_bm_free(free_list, free_count, table[j]);
        table_lens[s] = keep;
    }
}

/* ---------------------------------------------------- batched attention
 * q:   [batch][q_len][num_heads][head_dim] fp32
 * out: [batch][q_len][num_heads][head_dim] fp32
 * Query j of sequence s sits at position pos[s] + j and attends
 * [window_start(pos[s] + j), pos[s] + j] through the sequence's table, one
 * paged_attention_layer call per query (the verify loop calls it per draft
 * token, :3090-3123). pos[s] < 0 gives zeros (n <= 0, attention.mojo:180-185).
 * q_scale multiplies q before the call (1.0 = the reference; a power of two is
 * exact, so a softmax scale of 2^-k is emulated without rounding).
 * par: 0 = serial over sequences, head-pair tasks on `nthreads` threads
 *      (reference-faithful); 1 = sequences spread over `nthreads` threads;
 *      2 = (sequence, query) pairs spread over `nthreads` threads (the calls are
 *      independent once the keys are in the pool; used for long prefill chunks);
 *      3 = every core on (sequence, query, head pair) items: the batched CPU mode, whose
 *      items are the reference's head-pair tasks of every call at once (a call below
 *      the head-pair condition of attention.mojo:276 is one item). Every mode computes
 *      each head with the same arithmetic, so all give the same bits.
 * ring_size > 0: ring pools; tables[s * table_stride] is sequence s's ring slot and
 * the call passes ring_base = slot * ring_size (…batched.mojo:648). Returns -1 when a
 * query's window exceeds the ring (the reference aborts, attention.mojo:265-266). */
/* pkvo_attend's par = 3: items (s, j, pair) over all threads. Item (s, j, t) computes the
 * key rows of query j of sequence s, then head pair t as paged_attention_layer's task t
 * does; when the call takes the serial path (attention.mojo:283-287) item t = 0 runs it
 * and the others do nothing. */
static int attend_pairs(int dtype, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                        int32_t block_size, int32_t window, float q_scale, const float* q,
                        const void* k_pool, const void* v_pool, const int32_t* tables,
                        int32_t table_stride, const int32_t* table_lens, const int32_t* pos,
                        int32_t q_len, int32_t batch, float* out, int nthreads, int32_t ring_size,
                        int64_t max_n) {
    const int64_t hd = (int64_t)num_heads * head_dim;
    const int64_t ratio = num_heads / num_kv_heads;
    const int64_t kv_stride = (int64_t)num_kv_heads * head_dim;
    const int64_t pairs = num_heads / 2 > 0 ? num_heads / 2 : 1;
    const int64_t items = (int64_t)batch * q_len * pairs;
    int err = 0;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1) if (nthreads > 1)
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)(num_heads * (max_n + 1)));
        int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * (size_t)(max_n + 1));
        int64_t* tab = (int64_t*)malloc(sizeof(int64_t) * (size_t)(table_stride > 0 ? table_stride : 1));
        float* qs = (float*)malloc(sizeof(float) * (size_t)hd);
#pragma omp for schedule(dynamic, 1)
        for (int64_t it = 0; it < items; ++it) {
            const int32_t s = (int32_t)(it / ((int64_t)q_len * pairs));
            const int32_t j = (int32_t)((it / pairs) % q_len);
            const int64_t t = it % pairs;
            const float* qj = q + ((int64_t)s * q_len + j) * hd;
            float* oj = out + ((int64_t)s * q_len + j) * hd;
            if (pos[s] < 0) {
                if (t == 0)
                    for (int64_t i = 0; i < hd; ++i) oj[i] = 0.0f;
                continue;
            }
            for (int32_t i = 0; i < table_stride; ++i) tab[i] = tables[(int64_t)s * table_stride + i];
            for (int64_t i = 0; i < hd; ++i) qs[i] = qj[i] * q_scale;
            const int64_t ring_base = ring_size > 0 ? tab[0] * ring_size : 0;
            const int64_t n = pal_rows(tab, ring_size > 0 ? 0 : table_lens[s], block_size,
                                       (int64_t)pos[s] + j, kv_stride, window, rows, ring_size,
                                       ring_base);
            if (n < 0) {
#pragma omp atomic write
                err = (int)n;
                continue;
            }
            if (pal_pairs(n, num_heads, ratio)) {
                const int64_t h_start = t * 2;
                eval_head_range(qs, k_pool, v_pool, dtype, rows, scores, oj, n,
                                (h_start / ratio) * head_dim, h_start, h_start + 2, head_dim);
            } else if (t == 0) {
                for (int64_t g = 0; g < num_kv_heads; ++g)
                    eval_head_range(qs, k_pool, v_pool, dtype, rows, scores, oj, n, g * head_dim,
                                    g * ratio, g * ratio + ratio, head_dim);
            }
        }
        free(scores);
        free(rows);
        free(tab);
        free(qs);
    }
    return err;
}

int pkvo_attend(int dtype, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                int32_t block_size, int32_t window, float q_scale, const float* q,
                const void* k_pool, const void* v_pool, const int32_t* tables,
                int32_t table_stride, const int32_t* table_lens, const int32_t* pos,
                int32_t q_len, int32_t batch, float* out, int nthreads, int par,
                int32_t ring_size) {
    int64_t max_n = 0;
    for (int32_t s = 0; s < batch; ++s) {
        int64_t p = (int64_t)pos[s] + q_len;
        if (p > max_n) max_n = p;
    }
    int64_t hd = (int64_t)num_heads * head_dim;
    int err = 0;
    if (par == 3)
        return attend_pairs(dtype, num_heads, num_kv_heads, head_dim, block_size, window, q_scale,
                            q, k_pool, v_pool, tables, table_stride, table_lens, pos, q_len,
                            batch, out, nthreads, ring_size, max_n);
    int outer = (par >= 1 && nthreads > 1) ? nthreads : 1;
    int inner = (par >= 1) ? 1 : nthreads;
    /* par 2: one work item per (sequence, query); otherwise one per sequence. */
    int64_t items = par == 2 ? (int64_t)batch * q_len : batch;
    int32_t per_item = par == 2 ? 1 : q_len;
#pragma omp parallel num_threads(outer) if (outer > 1)
    {
        float* scores = (float*)malloc(sizeof(float) * (size_t)(num_heads * (max_n + 1)));
        int64_t* rows = (int64_t*)malloc(sizeof(int64_t) * (size_t)(max_n + 1));
        int64_t* tab = (int64_t*)malloc(sizeof(int64_t) * (size_t)(table_stride > 0 ? table_stride : 1));
        float* qs = (float*)malloc(sizeof(float) * (size_t)hd);
#pragma omp for schedule(dynamic, 1)
        for (int64_t it = 0; it < items; ++it) {
            const int32_t s = (int32_t)(par == 2 ? it / q_len : it);
            const int32_t j0 = (int32_t)(par == 2 ? it % q_len : 0);
            for (int32_t i = 0; i < table_stride; ++i) tab[i] = tables[(int64_t)s * table_stride + i];
            for (int32_t j = j0; j < j0 + per_item; ++j) {
                const float* qj = q + ((int64_t)s * q_len + j) * hd;
                float* oj = out + ((int64_t)s * q_len + j) * hd;
                if (pos[s] < 0) {
                    for (int64_t i = 0; i < hd; ++i) oj[i] = 0.0f;
                    continue;
                }
                for (int64_t i = 0; i < hd; ++i) qs[i] = qj[i] * q_scale;
                int64_t ring_base = ring_size > 0 ? tab[0] * ring_size : 0;
                int rc = pkvo_paged_attention_layer(
                    qs, k_pool, v_pool, dtype, tab, ring_size > 0 ? 0 : table_lens[s], block_size,
                    (int64_t)pos[s] + j, num_heads, num_kv_heads, head_dim, window, scores, rows,
                    oj, ring_size, ring_base, inner);
                if (rc != 0) {
#pragma omp atomic write
                    err = rc;
                }
            }
        }
        free(scores);
        free(rows);
        free(tab);
        free(qs);
    }
    return err;
}

int pkvo_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------- batched float64 attention
 * pkvo_attend's layout and query positions, evaluated with the float64 naive
 * oracle (test_attention.mojo:123-163): the exact attention that both fp32
 * paths approximate. q_scale multiplies q in double. pos[s] < 0 gives zeros.
 * ring_size > 0 (ring pools, tables[s * table_stride] = ring slot): the float64
 * oracle reads the ring through a one-row-per-block table, tab[t] = ring row of t. */
int pkvo_attend_f64(int dtype, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                    int32_t block_size, int32_t window, float q_scale, const float* q,
                    const void* k_pool, const void* v_pool, const int32_t* tables,
                    int32_t table_stride, const int32_t* pos, int32_t q_len, int32_t batch,
                    double* out, int nthreads, int32_t ring_size) {
    int64_t hd = (int64_t)num_heads * head_dim;
    int64_t tab_len = table_stride > 0 ? table_stride : 1;
    if (ring_size > 0)
        for (int32_t s = 0; s < batch; ++s)
            if ((int64_t)pos[s] + q_len > tab_len) tab_len = (int64_t)pos[s] + q_len;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1) if (nthreads > 1)
    {
        int64_t* tab = (int64_t*)malloc(sizeof(int64_t) * (size_t)tab_len);
        float* qs = (float*)malloc(sizeof(float) * (size_t)hd);
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (int32_t s = 0; s < batch; ++s) {
            for (int32_t j = 0; j < q_len; ++j) {
                const float* qj = q + ((int64_t)s * q_len + j) * hd;
                double* oj = out + ((int64_t)s * q_len + j) * hd;
                if (pos[s] < 0) {
                    for (int64_t i = 0; i < hd; ++i) oj[i] = 0.0;
                    continue;
                }
                int64_t p = (int64_t)pos[s] + j;
                int64_t bsz = block_size;
                if (ring_size > 0) {
                    int64_t slot = tables[(int64_t)s * table_stride];
                    for (int64_t t = 0; t <= p; ++t) tab[t] = pkvo_ring_row(slot, ring_size, t);
                    bsz = 1;
                } else {
                    for (int32_t i = 0; i < table_stride; ++i)
                        tab[i] = tables[(int64_t)s * table_stride + i];
                }
                /* q_scale is a power of two in every use, so the fp32 product is exact. */
                for (int64_t i = 0; i < hd; ++i) qs[i] = qj[i] * q_scale;
                pkvo_attention_f64(qs, k_pool, v_pool, dtype, tab, bsz, p,
                                   pkvo_window_start(p, window), num_heads, num_kv_heads,
                                   head_dim, oj);
            }
        }
        free(tab);
        free(qs);
    }
    return 0;
}
