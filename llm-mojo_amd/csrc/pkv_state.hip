// K1 (block allocation + K/V scatter) and K5 (rollback / retire).
//
// Block-manager state lives in caller-owned device memory: tables [batch][stride],
// table_lens [batch], the LIFO free list [num_blocks] and its count. The reference
// keeps the same state on the host (BlockManager / Sequence,
// model_speculative_moe_batched.mojo:789-845) and mutates it one sequence at a time;
// here every sequence's blocks are derived from an ordered prefix sum over the batch,
// which yields exactly the serial order's result, and the per-block work (table
// entries, free-list pushes) is spread over all threads of the workgroup.
//
// pkv_append = two launches on the caller's stream:
//   alloc_kernel   (1 workgroup)  pops the blocks every sequence needs, writes the new
//                                 table entries, table_lens, free_count and status;
//   scatter_kernel (tokens x seq) copies each token's K and V rows to
//                                 table[p / bs] * bs + p % bs for sequences whose
//                                 status is OK.
// The launch boundary orders the table writes before the scatter's reads, so neither
// kernel needs a device-scope fence.
//
// Ring pools (ring_size > 0) take no blocks: the scatter alone writes token p of a
// sequence with ring slot `slot` to row slot * ring_size + p % ring_size
// (ring_row, attention.mojo:144-148, as at the engine's write sites
// model_speculative_moe_batched.mojo:1996, :2625, :3111).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pkv_internal.h"

namespace pkv {
namespace {

constexpr int kNT = kBlockThreads;
constexpr int kMaxBatch = 4096;  // per-sequence plan kept in LDS

// Block-wide exclusive scan of one int per thread; writes the block total to *total.
__device__ int block_exclusive_scan(int v, int* tmp, int* total) {
    const int tid = threadIdx.x;
    tmp[tid] = v;
    __syncthreads();
    for (int off = 1; off < kNT; off <<= 1) {
        int add = tid >= off ? tmp[tid - off] : 0;
        __syncthreads();
        tmp[tid] += add;
        __syncthreads();
    }
    int incl = tmp[tid];
    *total = tmp[kNT - 1];
    __syncthreads();
    return incl - v;
}

// Sequence s with pref[s] <= e < pref[s + 1] (pref non-decreasing, pref[0] = 0).
__device__ inline int find_seq(const int* pref, int batch, int e) {
    int lo = 0, hi = batch - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (pref[mid] <= e) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Fills pref[0..batch] with the exclusive prefix sum of cnt[0..batch) (both in LDS)
// and returns the total.
__device__ int lds_prefix(const int* cnt, int* pref, int batch, int* tmp) {
    const int seg = (batch + kNT - 1) / kNT;
    const int b0 = threadIdx.x * seg, b1 = min(batch, b0 + seg);
    int sum = 0;
    for (int s = b0; s < b1; ++s) sum += cnt[s];
    int total;
    int run = block_exclusive_scan(sum, tmp, &total);
    for (int s = b0; s < b1; ++s) {
        pref[s] = run;
        run += cnt[s];
    }
    if (threadIdx.x == 0) pref[batch] = total;
    __syncthreads();
    return total;
}

struct AppendArgs {
    char* k_pool;
    char* v_pool;
    int32_t* tables;
    int32_t table_stride;
    int32_t* table_lens;
    const int32_t* free_list;
    int32_t* free_count;
    const int32_t* pos;
    const int32_t* tok_off;  // [batch + 1] rows of k_new / v_new per sequence
    int32_t max_new;
    int32_t total_rows;
    const char* k_new;
    const char* v_new;
    int32_t batch;
    int32_t* status;
    int32_t bs;
    int32_t num_blocks;  // ring mode: ring slots in the pool
    int32_t ring_size;   // > 0: ring pools; tables[s * table_stride] is s's ring slot
    int32_t row_bytes;  // num_kv_heads * head_dim * element size (multiple of 16)
    int32_t tok_per_wg;
};

// Ring mode: PKV_SEQ_OK or the reason sequence s writes nothing.
__device__ inline int ring_append_status(const AppendArgs& a, int s) {
    const int p = a.pos[s];
    const int r0 = a.tok_off[s], r1 = a.tok_off[s + 1];
    const int n = r1 - r0;
    if (p < 0 || n <= 0) return PKV_SEQ_OK;
    if (n > a.max_new || r0 < 0 || r1 > a.total_rows) return PKV_SEQ_BAD_ARGS;
    const int slot = a.tables[(size_t)s * a.table_stride];
    if (slot < 0 || slot >= a.num_blocks) return PKV_SEQ_BAD_BLOCK;
    return PKV_SEQ_OK;
}

// Blocks sequence s needs (>= 0), or a negative PKV_SEQ_* code.
__device__ inline int append_need(const AppendArgs& a, int s, int len) {
    return append_blocks_needed(a.pos[s], a.tok_off[s], a.tok_off[s + 1], a.max_new,
                                a.total_rows, a.bs, a.table_stride, len);
}

// One workgroup. Sequence s (index order) takes the free-list entries
// free_list[fc - 1 - pref[s] - j], j < granted[s]: the LIFO pops of a serial pass.
// A sequence that runs the list dry keeps what it popped (status OUT_OF_BLOCKS).
// This kernel writes every sequence's final status: a block the append touches whose
// table entry (held, or just popped) lies outside the pool gives BAD_BLOCK, as does a
// free count outside [0, num_blocks] for a sequence that needs blocks. The row copies
// after it only read status, so no two workgroups of a launch share a status word.
__global__ __launch_bounds__(kNT) void alloc_kernel(AppendArgs a) {
    __shared__ int s_tmp[kNT];
    __shared__ int s_len[kMaxBatch];
    __shared__ int s_need[kMaxBatch];
    __shared__ int s_code[kMaxBatch];
    __shared__ int s_pref[kMaxBatch + 1];
    __shared__ int s_tp[kMaxBatch + 1];
    const int tid = threadIdx.x;
    int fc = *a.free_count;
    const bool fc_bad = fc < 0 || fc > a.num_blocks;
    if (fc_bad) fc = 0;
    for (int s = tid; s < a.batch; s += kNT) {
        const int len = a.table_lens[s];
        const int need = append_need(a, s, len);
        s_len[s] = len;
        s_need[s] = need > 0 ? need : 0;
        s_code[s] = need < 0 ? need : PKV_SEQ_OK;
    }
    __syncthreads();
    const int total = lds_prefix(s_need, s_pref, a.batch, s_tmp);
    const int popped = total < fc ? total : fc;
    // Table entries, flattened over every popped block.
    for (int e = tid; e < popped; e += kNT) {
        const int s = find_seq(s_pref, a.batch, e);
        const int j = e - s_pref[s];
        a.tables[(size_t)s * a.table_stride + s_len[s] + j] = a.free_list[fc - 1 - e];
    }
    // Status after the pops; s_need then counts the blocks each sequence's rows land in.
    for (int s = tid; s < a.batch; s += kNT) {
        const int need = s_need[s];
        const int granted = append_granted(need, fc, s_pref[s]);
        if (granted > 0) a.table_lens[s] = s_len[s] + granted;
        const int code = append_pop_status(s_code[s], need, granted, fc_bad);
        const int p = a.pos[s];
        const int n = a.tok_off[s + 1] - a.tok_off[s];
        s_code[s] = code;
        s_need[s] = code == PKV_SEQ_OK && p >= 0 && n > 0
                        ? (int)(((long long)p + n - 1) / a.bs) - p / a.bs + 1 : 0;
    }
    __syncthreads();
    const int checks = lds_prefix(s_need, s_tp, a.batch, s_tmp);
    // Every block the rows land in, flattened over the batch so the entry reads are all in
    // flight together: held entries from the table, new ones from the free list (the entries
    // the loop above writes, read at their source). One outside the pool: BAD_BLOCK.
    for (int e = tid; e < checks; e += kNT) {
        const int s = find_seq(s_tp, a.batch, e);
        const int blk = a.pos[s] / a.bs + (e - s_tp[s]);
        const int need = s_pref[s + 1] - s_pref[s];
        const int ent = append_block_entry(a.tables + (size_t)s * a.table_stride, a.free_list,
                                           s_len[s], append_granted(need, fc, s_pref[s]), fc,
                                           s_pref[s], blk);
        if (ent < 0 || ent >= a.num_blocks) s_code[s] = PKV_SEQ_BAD_BLOCK;
    }
    __syncthreads();
    for (int s = tid; s < a.batch; s += kNT) a.status[s] = s_code[s];
    if (tid == 0 && !fc_bad) *a.free_count = fc - popped;
}

// Paged pools: whether the rows of sequence s with status `st` (from alloc_kernel) are
// copied -- OK, or BAD_BLOCK where each row is then written only if its block is held
// (index < table_lens[s], a length within [0, table_stride]) and its entry lies in the
// pool.
__device__ inline bool paged_rows_written(int st) {
    return st == PKV_SEQ_OK || st == PKV_SEQ_BAD_BLOCK;
}

// grid = (ceil(max_new / tok_per_wg), batch). Copies this workgroup's tokens of one
// sequence; a table entry outside the pool is skipped and reported as BAD_BLOCK.
// Ring mode: every workgroup of sequence s derives its status itself (the one with
// blockIdx.x == 0 stores it), and of n > ring_size new tokens only the last ring_size
// are written -- the rows a serial pass leaves behind, since each earlier token's row
// is overwritten within the same call.
__global__ __launch_bounds__(kNT) void scatter_kernel(AppendArgs a) {
    const int s = blockIdx.y;
    const int tid = threadIdx.x;
    const bool ring = a.ring_size > 0;
    if (ring) {
        const int st = ring_append_status(a, s);
        if (blockIdx.x == 0 && tid == 0) a.status[s] = st;
        if (st != PKV_SEQ_OK) return;
    } else if (!paged_rows_written(a.status[s])) {
        return;
    }
    const int p0 = a.pos[s];
    const int row0 = a.tok_off[s];
    const int n = a.tok_off[s + 1] - row0;
    if (p0 < 0 || n <= 0) return;
    const int tok_first = ring && n > a.ring_size ? n - a.ring_size : 0;
    const int tok_begin = max(tok_first, (int)blockIdx.x * a.tok_per_wg);
    const int tok_end = min(n, (int)blockIdx.x * a.tok_per_wg + a.tok_per_wg);
    const int vec_per_row = a.row_bytes / 16;
    const int32_t* table = a.tables + (size_t)s * a.table_stride;
    const int held = ring ? 0 : a.table_lens[s];
    if (!ring && held > a.table_stride) return;  // a length outside the table: BAD_BLOCK
    for (int b = tok_begin; b < tok_end; ++b) {
        const int p = p0 + b;
        size_t row;
        if (ring) {
            row = (size_t)table[0] * a.ring_size + (size_t)(p % a.ring_size);
        } else {
            const int blk = p / a.bs;
            const int phys = blk < held ? table[blk] : -1;
            if (phys < 0 || phys >= a.num_blocks) continue;  // reported by alloc_kernel
            row = (size_t)phys * a.bs + (size_t)(p % a.bs);
        }
        const uint4* ks = reinterpret_cast<const uint4*>(a.k_new + ((size_t)row0 + b) * a.row_bytes);
        const uint4* vs = reinterpret_cast<const uint4*>(a.v_new + ((size_t)row0 + b) * a.row_bytes);
        uint4* kd = reinterpret_cast<uint4*>(a.k_pool + row * a.row_bytes);
        uint4* vd = reinterpret_cast<uint4*>(a.v_pool + row * a.row_bytes);
        for (int i = tid; i < vec_per_row; i += kNT) {
            const uint4 kv = ks[i];
            const uint4 vv = vs[i];
            kd[i] = kv;
            vd[i] = vv;
        }
    }
}

// ---- fused producer step + append (pkv_append_qkv) --------------------------------
//
// A workgroup takes a few tokens of one sequence. Each token's RoPE angles are computed
// once into LDS; then each wave takes whole heads: a lane holds elements [l*E, l*E+E) of the first
// half of the head and the same of the second half, so the pair (i, i + D/2) that RoPE
// rotates sits in one lane and the only cross-lane step is the sum of squares.
//   Q head:  rms_norm (q_norm weight), RoPE          -> q_out row (fp32 or bf16)
//   K head:  rms_norm (k_norm weight), RoPE          -> pool row
//   V head:  rms_norm_noscale (input V, or K as read)  -> pool row
// Angles: theta_i = pos / base^(2i / rope_dim) in fp32, as the reference computes them.
// base^(2i / rope_dim) is computed on the host in double and rounded once to fp32, the
// correctly rounded value (on every exponent the engine uses it equals the C library's
// powf), and passed in the kernel arguments.
// Arithmetic: the rotation runs in double -- x * weight (exact in double) times cos / sin
// of the fp32 angle -- and each output is rounded once. Where a rotation cancels, the
// reference's fp32 evaluation is several ulps of its terms away from exact, more than the
// parity bound's 1e-3 floor absorbs; this one stays within an ulp of the result. The
// RMS factor (sum of squares and 1/sqrt in fp32) scales a whole head, so its rounding
// stays a relative error of ~1e-7 of each output.
struct QkvArgs {
    AppendArgs ap;
    const float* q;    // [total_rows][Hq][D]
    const float* k;    // [total_rows][Hkv][D]
    const float* v;    // [total_rows][Hkv][D], or null: V := K
    const float* q_w;  // [D]
    const float* k_w;  // [D]
    void* q_out;       // [total_rows][Hq][D], fp32 or bf16
    int32_t q_out_bf16;
    int32_t kv_bf16;
    int32_t Hq;
    int32_t Hkv;
    int32_t rotary_half;
    float inv_freq[256];  // base^(2i / rope_dim), i < rotary_half, correctly rounded fp32
};

// Two fp32 values as packed bf16 bits, rounded to nearest even (v_cvt_pk_bf16_f32).
__device__ inline uint32_t pack_bf16x2(float x0, float x1) {
    const __bf16 h0 = (__bf16)x0, h1 = (__bf16)x1;
    return (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
}

// E values of a pool row or of q_out, as non-temporal stores (written once by this step).
template <int E>
__device__ inline void store_row(void* base, size_t elem, bool bf16, const float (&x)[E]) {
    typedef uint32_t u2v __attribute__((ext_vector_type(2)));
    typedef float f2v __attribute__((ext_vector_type(2)));
    typedef float f4v __attribute__((ext_vector_type(4)));
    if (bf16) {
        uint16_t* d = static_cast<uint16_t*>(base) + elem;
        if constexpr (E == 2) {
            __builtin_nontemporal_store(pack_bf16x2(x[0], x[1]), reinterpret_cast<uint32_t*>(d));
        } else {
            __builtin_nontemporal_store(u2v{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])}, reinterpret_cast<u2v*>(d));
        }
    } else {
        float* d = static_cast<float*>(base) + elem;
        if constexpr (E == 2) {
            __builtin_nontemporal_store(f2v{x[0], x[1]}, reinterpret_cast<f2v*>(d));
        } else {
            __builtin_nontemporal_store(f4v{x[0], x[1], x[2], x[3]}, reinterpret_cast<f4v*>(d));
        }
    }
}

// E fp32 values; NT: a non-temporal load (the projections of a token are read once).
template <int E, bool NT = false>
__device__ inline void load_vec(const float* p, float (&x)[E]) {
    typedef float f2v __attribute__((ext_vector_type(2)));
    typedef float f4v __attribute__((ext_vector_type(4)));
    if constexpr (E == 2) {
        f2v v;
        if constexpr (NT) v = __builtin_nontemporal_load(reinterpret_cast<const f2v*>(p));
        else v = *reinterpret_cast<const f2v*>(p);
        x[0] = v.x;
        x[1] = v.y;
    } else {
        f4v v;
        if constexpr (NT) v = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
        else v = *reinterpret_cast<const f4v*>(p);
        x[0] = v.x;
        x[1] = v.y;
        x[2] = v.z;
        x[3] = v.w;
    }
}

// A workgroup of kQkvWaves waves takes one token. A wave processes HS heads at once
// (HS = 2 for head_dim 256 when no pair of heads would mix Q, K and V: lanes 0-31 one
// head, 32-63 the next; else HS = 1), so a lane holds EL = D * HS / 128 elements of each
// half of its head (4 for head_dim 512 and for paired 256: 16-byte loads), with the RoPE
// pair (i, i + D/2) in one lane. Slots of HS heads go round-robin to the waves,
// kQkvHeads / HS at a time per wave; every slot of a batch is loaded before any is
// processed (the first batch before the angle table is built). Per batch, the heads'
// 1 / sqrt(mean + eps) runs once for all of them (lane j + 32 sub takes slot j's head
// sub). The per-element path reads the token's rotation table with the norm weights folded
// in (dims past the rotary range hold cos 1, sin 0), so it has neither branch nor select:
// 4 x 2048 tokens 92.0-93.6 -> 81.0-82.4 us per call, kernel 81.0 -> 72.0 us in the trace.
constexpr int kQkvWaves = 8;
constexpr int kQkvHeads = 4;  // heads per wave and batch: 32 heads (16 q + 8 k + 8 v) in one

// Sum over the 64 lanes, in every lane, without LDS: lane l ^ 32 and l ^ 16 by the
// permlane swaps (each returns both halves, so a + b pairs every lane with its partner),
// then l ^ 8 and the 4-lane classes by row rotations, then l ^ 2 and l ^ 1 by quad
// permutes.
__device__ inline float wave_sum(float x) {
    const uint32_t u = __float_as_uint(x);
    auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    x = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
    const uint32_t u16 = __float_as_uint(x);
    auto r16 = __builtin_amdgcn_permlane16_swap(u16, u16, false, false);
    x = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));  // row_ror:8
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xf, 0xf, false));  // row_ror:4
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));   // l ^ 2
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));   // l ^ 1
    return x;
}

// The same over each half of the wave (lanes 0-31 and 32-63 separately).
__device__ inline float half_wave_sum(float x) {
    const uint32_t u16 = __float_as_uint(x);
    auto r16 = __builtin_amdgcn_permlane16_swap(u16, u16, false, false);
    x = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));  // row_ror:8
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xf, 0xf, false));  // row_ror:4
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));   // l ^ 2
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));   // l ^ 1
    return x;
}
template <int D, int HS>
__global__ __launch_bounds__(kQkvWaves * kWave) void qkv_append_kernel(QkvArgs a) {
    constexpr int HALF = D / 2;
    constexpr int LPH = kWave / HS;   // lanes per head
    constexpr int EL = HALF / LPH;    // elements per lane per half
    static_assert((EL == 2 || EL == 4) && (HS == 1 || HS == 2), "8- or 16-byte lane slices");
    constexpr int NT = kQkvWaves * kWave;
    constexpr int IPW = kQkvHeads / HS;  // slots per wave and batch
    static_assert(IPW <= kWave / 2, "one lane per slot and head");
    // Per dim i < HALF and kind (q, k), with c, s = cos, sin of the token's angle (1, 0 past
    // the rotary dims) and w1, w2 = the norm weights of dims i and HALF + i:
    // [0] w1 c, [1] w2 s, [2] w2 c, [3] w1 s, so r1 = x1 (w1 c) - x2 (w2 s) and
    // r2 = x2 (w2 c) + x1 (w1 s) in double, with no select on the rotary range.
    __shared__ double s_rot[2][4][HALF];
    __shared__ long long s_prow;  // pool row of the token's K / V, or -1
    const AppendArgs& ap = a.ap;
    const int s = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int sub = lane / LPH, hl = lane % LPH;  // head of the slot, lane within the head
    const bool ring = ap.ring_size > 0;
    // independent loads first, so they are in flight together
    const int p0 = ap.pos[s];
    const int row0 = ap.tok_off[s];
    const int n = ap.tok_off[s + 1] - row0;
    int st = ring ? PKV_SEQ_OK : ap.status[s];  // paged: written by alloc_kernel
    if (ring) {
        st = ring_append_status(ap, s);
        if (blockIdx.x == 0 && tid == 0) ap.status[s] = st;
    }
    if (st == PKV_SEQ_BAD_ARGS) return;  // token range unusable: nothing is read
    const int b = blockIdx.x;             // this workgroup's token
    if (p0 < 0 || n <= 0 || b >= n) return;
    const int p = p0 + b;
    const size_t r = (size_t)row0 + b;    // its row in q / k / v

    // Slot it holds heads HS * it .. HS * it + HS - 1: Q, then K, then V (V := K without
    // v). Hq and Hkv are multiples of HS, so a slot never mixes kinds.
    const int heads = a.Hq + 2 * a.Hkv;
    const int slots = heads / HS;
    auto src_of = [&](int hh) -> const float* {
        if (hh < a.Hq) return a.q + (r * a.Hq + hh) * D;
        if (hh < a.Hq + a.Hkv) return a.k + (r * a.Hkv + (hh - a.Hq)) * D;
        return (a.v ? a.v : a.k) + (r * a.Hkv + (hh - a.Hq - a.Hkv)) * D;
    };
    float f1[IPW][EL], f2[IPW][EL];
    auto load_batch = [&](int first) {
#pragma unroll
        for (int j = 0; j < IPW; ++j) {
            const int it = first + j * kQkvWaves;
            if (it < slots) {
                const float* src = src_of(it * HS + sub);
                load_vec<EL, true>(src + hl * EL, f1[j]);
                load_vec<EL, true>(src + HALF + hl * EL, f2[j]);
            }
        }
    };
    load_batch(wave);

    for (int i = tid; i < HALF; i += NT) {
        const double q1 = a.q_w[i], q2 = a.q_w[HALF + i], k1 = a.k_w[i], k2 = a.k_w[HALF + i];
        double sn = 0.0, c = 1.0;
        if (i < a.rotary_half) {
            const float theta = (float)p / a.inv_freq[i];
            sincos((double)theta, &sn, &c);
        }
        s_rot[0][0][i] = q1 * c;
        s_rot[0][1][i] = q2 * sn;
        s_rot[0][2][i] = q2 * c;
        s_rot[0][3][i] = q1 * sn;
        s_rot[1][0][i] = k1 * c;
        s_rot[1][1][i] = k2 * sn;
        s_rot[1][2][i] = k2 * c;
        s_rot[1][3][i] = k1 * sn;
    }
    // K / V rows are written only by an OK sequence, and in ring mode only by the last
    // ring_size tokens of the call (earlier ones would be overwritten within it).
    if (tid == 0) {
        long long prow = -1;
        const bool write = ring ? st == PKV_SEQ_OK && b >= n - ap.ring_size : paged_rows_written(st);
        if (write) {
            const int32_t* table = ap.tables + (size_t)s * ap.table_stride;
            if (ring) {
                prow = (long long)table[0] * ap.ring_size + p % ap.ring_size;
            } else {
                // a block outside the pool or not held skips the row (alloc_kernel reported it)
                const int blk = p / ap.bs;
                const int held = ap.table_lens[s];
                const int phys = blk < held && held <= ap.table_stride ? table[blk] : -1;
                if (phys >= 0 && phys < ap.num_blocks) prow = (long long)phys * ap.bs + p % ap.bs;
            }
        }
        s_prow = prow;
    }
    __syncthreads();
    const long long prow = s_prow;

    const size_t kv_row_elems = (size_t)a.Hkv * D;
    for (int first = wave; first < slots; first += kQkvWaves * IPW) {
        if (first != wave) load_batch(first);
        // sums of squares of the batch's heads, reduced together (independent chains)
        float ss[IPW];
#pragma unroll
        for (int j = 0; j < IPW; ++j) {
            ss[j] = 0.f;
#pragma unroll
            for (int e = 0; e < EL; ++e) ss[j] += f1[j][e] * f1[j][e] + f2[j][e] * f2[j][e];
        }
#pragma unroll
        for (int j = 0; j < IPW; ++j) ss[j] = HS == 2 ? half_wave_sum(ss[j]) : wave_sum(ss[j]);
        // 1 / sqrt(mean + eps) of slot j's head `sub` on lane j + 32 sub, then each lane
        // takes its own head's value
        float ssl = ss[0];
#pragma unroll
        for (int j = 1; j < IPW; ++j) ssl = (lane & 31) == j ? ss[j] : ssl;
        const float inv_l = 1.0f / sqrtf(ssl / (float)D + 1e-6f);
#pragma unroll
        for (int j = 0; j < IPW; ++j) {
            const int it = first + j * kQkvWaves;
            if (it >= slots) break;
            const int hh0 = it * HS;  // the slot's first head; the kind is the slot's
            const int kind = hh0 < a.Hq ? 0 : (hh0 < a.Hq + a.Hkv ? 1 : 2);  // q, k, v
            if (kind != 0 && prow < 0) continue;
            const int hh = hh0 + sub;
            const int h = kind == 0 ? hh : (kind == 1 ? hh - a.Hq : hh - a.Hq - a.Hkv);
            const int inv_lo = __builtin_amdgcn_readlane(__builtin_bit_cast(int, inv_l), j);
            const int inv_hi = __builtin_amdgcn_readlane(__builtin_bit_cast(int, inv_l), 32 + j);
            const float inv_rms = __builtin_bit_cast(float, sub ? inv_hi : inv_lo);
            float o1[EL], o2[EL];
            if (kind < 2) {
                const double* t = s_rot[kind][0];
#pragma unroll
                for (int e = 0; e < EL; ++e) {
                    const int i = hl * EL + e;
                    const double x1 = f1[j][e], x2 = f2[j][e];
                    const double r1 = fma(x1, t[i], -(x2 * t[HALF + i]));
                    const double r2 = fma(x2, t[2 * HALF + i], x1 * t[3 * HALF + i]);
                    o1[e] = (float)(r1 * (double)inv_rms);
                    o2[e] = (float)(r2 * (double)inv_rms);
                }
            } else {
#pragma unroll
                for (int e = 0; e < EL; ++e) {
                    o1[e] = f1[j][e] * inv_rms;
                    o2[e] = f2[j][e] * inv_rms;
                }
            }
            if (kind == 0) {
                const size_t off = (r * a.Hq + h) * D;
                store_row<EL>(a.q_out, off + hl * EL, a.q_out_bf16, o1);
                store_row<EL>(a.q_out, off + HALF + hl * EL, a.q_out_bf16, o2);
            } else {
                void* pool = kind == 1 ? (void*)ap.k_pool : (void*)ap.v_pool;
                const size_t off = (size_t)prow * kv_row_elems + (size_t)h * D;
                store_row<EL>(pool, off + hl * EL, a.kv_bf16, o1);
                store_row<EL>(pool, off + HALF + hl * EL, a.kv_bf16, o2);
            }
        }
    }
}

struct RollbackArgs {
    int32_t* tables;
    int32_t table_stride;
    int32_t* table_lens;
    int32_t* free_list;
    int32_t* free_count;
    const int32_t* new_len;
    int32_t batch;
    int32_t* status;  // may be null
    int32_t bs;
    int32_t num_blocks;
};

// One workgroup: ordered prefix over the freed counts; freed entry e (sequence s's tail
// blocks in ascending logical order, sequences in index order) goes to
// free_list[fc + e]. Any inconsistency (a length or entry outside its range, or a
// free list that would overflow) rejects the whole call and changes nothing.
__global__ __launch_bounds__(kNT) void rollback_kernel(RollbackArgs a) {
    __shared__ int s_tmp[kNT];
    __shared__ int s_keep[kMaxBatch];
    __shared__ int s_cnt[kMaxBatch];
    __shared__ int s_pref[kMaxBatch + 1];
    __shared__ int s_bad;
    const int tid = threadIdx.x;
    if (tid == 0) s_bad = 0;
    __syncthreads();
    const int fc = *a.free_count;
    for (int s = tid; s < a.batch; s += kNT) {
        const int len = a.table_lens[s];
        const bool len_ok = len >= 0 && len <= a.table_stride;
        int keep = len_ok ? len : 0;
        if (len_ok && a.new_len[s] >= 0) {
            const long long k = ((long long)a.new_len[s] + a.bs - 1) / a.bs;
            keep = k < len ? (int)k : len;
        }
        if (!len_ok) s_bad = 1;
        s_keep[s] = keep;
        s_cnt[s] = len_ok ? len - keep : 0;
    }
    __syncthreads();
    const int total = lds_prefix(s_cnt, s_pref, a.batch, s_tmp);
    for (int e = tid; e < total; e += kNT) {  // every freed entry must name a pool block
        const int s = find_seq(s_pref, a.batch, e);
        const int blk = a.tables[(size_t)s * a.table_stride + s_keep[s] + (e - s_pref[s])];
        if (blk < 0 || blk >= a.num_blocks) s_bad = 1;
    }
    __syncthreads();
    const bool reject = s_bad || fc < 0 || (long long)fc + total > a.num_blocks;
    if (reject) {
        if (a.status)
            for (int s = tid; s < a.batch; s += kNT) {
                const int len = a.table_lens[s];
                const bool len_ok = len >= 0 && len <= a.table_stride;
                a.status[s] = !len_ok ? PKV_SEQ_BAD_BLOCK
                              : (s_cnt[s] > 0 ? (s_bad ? PKV_SEQ_BAD_BLOCK : PKV_SEQ_FREE_OVERFLOW)
                                              : PKV_SEQ_OK);
            }
        return;
    }
    for (int e = tid; e < total; e += kNT) {
        const int s = find_seq(s_pref, a.batch, e);
        a.free_list[fc + e] = a.tables[(size_t)s * a.table_stride + s_keep[s] + (e - s_pref[s])];
    }
    for (int s = tid; s < a.batch; s += kNT) {
        if (s_cnt[s] > 0) a.table_lens[s] = s_keep[s];
        if (a.status) a.status[s] = PKV_SEQ_OK;
    }
    if (tid == 0) *a.free_count = fc + total;
}

}  // namespace

int32_t append_validate(const pkv_params* p, void* k_pool, void* v_pool, int32_t* block_tables,
                        int32_t table_stride, int32_t* table_lens, int32_t* free_list,
                        int32_t* free_count, const int32_t* pos, const int32_t* tok_off,
                        int32_t max_new, const void* k_new, const void* v_new,
                        int32_t total_rows, int32_t batch, int32_t* status) {
    int32_t rc = validate_params(p);
    if (rc != PKV_OK) return rc;
    if (batch <= 0 || max_new <= 0 || table_stride <= 0 || total_rows <= 0)
        return fail(PKV_ERR_INVALID,
                    "batch, max_new, total_rows and table_stride must be positive");
    if (batch > kMaxBatch) return fail(PKV_ERR_UNSUPPORTED, "batch must be <= 4096");
    const bool ring = p->ring_size > 0;  // ring pools use no block-manager state
    if (!k_pool || !v_pool || !block_tables || !pos || !tok_off || !k_new || !v_new ||
        !status || (!ring && (!table_lens || !free_list || !free_count)))
        return fail(PKV_ERR_INVALID, "null device pointer");
    return PKV_OK;
}

int32_t append_launch(hipStream_t st, const pkv_params* p, void* k_pool, void* v_pool,
                      int32_t* block_tables, int32_t table_stride, int32_t* table_lens,
                      int32_t* free_list, int32_t* free_count, const int32_t* pos,
                      const int32_t* tok_off, int32_t max_new, const void* k_new,
                      const void* v_new, int32_t total_rows, int32_t batch, int32_t* status,
                      bool scatter) {
    const int32_t rc = append_validate(p, k_pool, v_pool, block_tables, table_stride, table_lens,
                                       free_list, free_count, pos, tok_off, max_new, k_new,
                                       v_new, total_rows, batch, status);
    if (rc != PKV_OK) return rc;
    const bool ring = p->ring_size > 0;  // ring pools use no block-manager state
    AppendArgs a{};
    a.k_pool = static_cast<char*>(k_pool);
    a.v_pool = static_cast<char*>(v_pool);
    a.tables = block_tables;
    a.table_stride = table_stride;
    a.table_lens = table_lens;
    a.free_list = free_list;
    a.free_count = free_count;
    a.pos = pos;
    a.tok_off = tok_off;
    a.max_new = max_new;
    a.total_rows = total_rows;
    a.k_new = static_cast<const char*>(k_new);
    a.v_new = static_cast<const char*>(v_new);
    a.batch = batch;
    a.status = status;
    a.bs = p->block_size;
    a.num_blocks = p->num_blocks;
    a.ring_size = p->ring_size;
    a.row_bytes = (int32_t)((size_t)p->num_kv_heads * p->head_dim * kv_elt_bytes(p->kv_dtype));
    // Tokens per scatter workgroup: ~64 KiB of K+V copies each (4 tokens at 8 x 256 fp32).
    const int tpw = (64 * 1024) / (2 * a.row_bytes);
    a.tok_per_wg = tpw < 1 ? 1 : tpw;
    if (!ring) hipLaunchKernelGGL(alloc_kernel, dim3(1), dim3(kNT), 0, st, a);
    if (scatter) {
        dim3 grid((max_new + a.tok_per_wg - 1) / a.tok_per_wg, batch);
        hipLaunchKernelGGL(scatter_kernel, grid, dim3(kNT), 0, st, a);
    }
    return check_launch("pkv_append");
}

}  // namespace pkv

extern "C" {

int32_t pkv_append(void* stream, const pkv_params* p, void* k_pool, void* v_pool,
                   int32_t* block_tables, int32_t table_stride, int32_t* table_lens,
                   int32_t* free_list, int32_t* free_count, const int32_t* pos,
                   const int32_t* tok_off, int32_t max_new, const void* k_new,
                   const void* v_new, int32_t total_rows, int32_t batch, int32_t* status) {
    pkv::clear_error();
    return pkv::append_launch(static_cast<hipStream_t>(stream), p, k_pool, v_pool, block_tables,
                              table_stride, table_lens, free_list, free_count, pos, tok_off,
                              max_new, k_new, v_new, total_rows, batch, status, true);
}

int32_t pkv_append_qkv(void* stream, const pkv_params* p, int32_t is_global, void* k_pool,
                       void* v_pool, int32_t* block_tables, int32_t table_stride,
                       int32_t* table_lens, int32_t* free_list, int32_t* free_count,
                       const int32_t* pos, const int32_t* tok_off, int32_t max_new,
                       const float* q, const float* k, const float* v,
                       const float* q_norm_weight, const float* k_norm_weight, void* q_out,
                       int32_t q_out_dtype, int32_t total_rows, int32_t batch,
                       int32_t* status) {
    using namespace pkv;
    clear_error();
    int32_t rc = validate_params(p);
    if (rc != PKV_OK) return rc;
    if (p->head_dim != 256 && p->head_dim != 512)
        return fail(PKV_ERR_UNSUPPORTED, "pkv_append_qkv: head_dim 256 or 512");
    if (batch <= 0 || max_new <= 0 || table_stride <= 0 || total_rows <= 0)
        return fail(PKV_ERR_INVALID,
                    "batch, max_new, total_rows and table_stride must be positive");
    if (batch > kMaxBatch) return fail(PKV_ERR_UNSUPPORTED, "batch must be <= 4096");
    if (q_out_dtype != PKV_DTYPE_F32 && q_out_dtype != PKV_DTYPE_BF16)
        return fail(PKV_ERR_INVALID, "q_out_dtype must be PKV_DTYPE_F32 or PKV_DTYPE_BF16");
    const bool ring = p->ring_size > 0;
    if (!k_pool || !v_pool || !block_tables || !pos || !tok_off || !q || !k ||
        !q_norm_weight || !k_norm_weight || !q_out || !status ||
        (!ring && (!table_lens || !free_list || !free_count)))
        return fail(PKV_ERR_INVALID, "null device pointer");
    QkvArgs a{};
    AppendArgs& ap = a.ap;
    ap.k_pool = static_cast<char*>(k_pool);
    ap.v_pool = static_cast<char*>(v_pool);
    ap.tables = block_tables;
    ap.table_stride = table_stride;
    ap.table_lens = table_lens;
    ap.free_list = free_list;
    ap.free_count = free_count;
    ap.pos = pos;
    ap.tok_off = tok_off;
    ap.max_new = max_new;
    ap.total_rows = total_rows;
    ap.batch = batch;
    ap.status = status;
    ap.bs = p->block_size;
    ap.num_blocks = p->num_blocks;
    ap.ring_size = p->ring_size;
    ap.row_bytes = (int32_t)((size_t)p->num_kv_heads * p->head_dim * kv_elt_bytes(p->kv_dtype));
    a.q = q;
    a.k = k;
    a.v = v;
    a.q_w = q_norm_weight;
    a.k_w = k_norm_weight;
    a.q_out = q_out;
    a.q_out_bf16 = q_out_dtype == PKV_DTYPE_BF16;
    a.kv_bf16 = p->kv_dtype == PKV_DTYPE_BF16;
    a.Hq = p->num_heads;
    a.Hkv = p->num_kv_heads;
    // apply_rope_qk's constants (attention.mojo:78-82): global layers rotate the first
    // min(64, D/2) pairs with base 1e6 over 512 dims, sliding layers all D/2 pairs with
    // base 1e4 over 256 dims.
    const int half = p->head_dim / 2;
    a.rotary_half = is_global ? (half < 64 ? half : 64) : half;
    const double base = is_global ? 1000000.0 : 10000.0;
    const float rope_dim = is_global ? 512.0f : 256.0f;
    for (int i = 0; i < a.rotary_half; ++i)
        a.inv_freq[i] = (float)pow(base, (double)((float)(2 * i) / rope_dim));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (!ring) hipLaunchKernelGGL(alloc_kernel, dim3(1), dim3(kNT), 0, st, ap);
    dim3 grid(max_new, batch);
    const dim3 block(kQkvWaves * kWave);
    // head_dim 256 pairs heads within a wave when no slot would mix Q, K and V heads
    if (p->head_dim == 512) hipLaunchKernelGGL((qkv_append_kernel<512, 1>), grid, block, 0, st, a);
    else if (p->num_heads % 2 == 0 && p->num_kv_heads % 2 == 0)
        hipLaunchKernelGGL((qkv_append_kernel<256, 2>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((qkv_append_kernel<256, 1>), grid, block, 0, st, a);
    return check_launch("pkv_append_qkv");
}

int32_t pkv_rollback(void* stream, const pkv_params* p, int32_t* block_tables,
                     int32_t table_stride, int32_t* table_lens, int32_t* free_list,
                     int32_t* free_count, const int32_t* new_len, int32_t batch,
                     int32_t* status) {
    using namespace pkv;
    clear_error();
    int32_t rc = validate_params(p);
    if (rc != PKV_OK) return rc;
    if (batch <= 0 || table_stride <= 0)
        return fail(PKV_ERR_INVALID, "batch and table_stride must be positive");
    if (p->ring_size > 0)
        return fail(PKV_ERR_INVALID,
                    "pkv_rollback acts on block tables: pass paged params (ring_size 0)");
    if (batch > kMaxBatch) return fail(PKV_ERR_UNSUPPORTED, "batch must be <= 4096");
    if (!block_tables || !table_lens || !free_list || !free_count || !new_len)
        return fail(PKV_ERR_INVALID, "null device pointer");
    RollbackArgs a{};
    a.tables = block_tables;
    a.table_stride = table_stride;
    a.table_lens = table_lens;
    a.free_list = free_list;
    a.free_count = free_count;
    a.new_len = new_len;
    a.batch = batch;
    a.status = status;
    a.bs = p->block_size;
    a.num_blocks = p->num_blocks;
    hipLaunchKernelGGL(rollback_kernel, dim3(1), dim3(kNT), 0, static_cast<hipStream_t>(stream),
                       a);
    return check_launch("pkv_rollback");
}

}  // extern "C"
