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
    const int p = a.pos[s];
    const int r0 = a.tok_off[s], r1 = a.tok_off[s + 1];
    const int n = r1 - r0;
    if (p < 0 || n <= 0) return 0;
    if (n > a.max_new || r0 < 0 || r1 > a.total_rows) return PKV_SEQ_BAD_ARGS;
    const long long last_blk = ((long long)p + n - 1) / a.bs;
    if (last_blk >= a.table_stride) return PKV_SEQ_TABLE_FULL;
    if (len < 0 || len > a.table_stride) return PKV_SEQ_BAD_BLOCK;
    const long long need = last_blk + 1 - len;
    return need > 0 ? (int)need : 0;
}

// One workgroup. Sequence s (index order) takes the free-list entries
// free_list[fc - 1 - pref[s] - j], j < granted[s]: the LIFO pops of a serial pass.
// A sequence that runs the list dry keeps what it popped (status OUT_OF_BLOCKS).
__global__ __launch_bounds__(kNT) void alloc_kernel(AppendArgs a) {
    __shared__ int s_tmp[kNT];
    __shared__ int s_len[kMaxBatch];
    __shared__ int s_need[kMaxBatch];
    __shared__ int s_pref[kMaxBatch + 1];
    const int tid = threadIdx.x;
    int fc = *a.free_count;
    const bool fc_bad = fc < 0 || fc > a.num_blocks;
    if (fc_bad) fc = 0;
    for (int s = tid; s < a.batch; s += kNT) {
        const int len = a.table_lens[s];
        const int need = append_need(a, s, len);
        s_len[s] = len;
        s_need[s] = need > 0 ? need : 0;
        a.status[s] = need < 0 ? need : PKV_SEQ_OK;
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
    for (int s = tid; s < a.batch; s += kNT) {
        const int need = s_need[s];
        if (need == 0) continue;
        const int avail = fc - s_pref[s];
        const int granted = avail <= 0 ? 0 : (avail < need ? avail : need);
        if (granted > 0) a.table_lens[s] = s_len[s] + granted;
        if (granted < need) a.status[s] = fc_bad ? PKV_SEQ_BAD_BLOCK : PKV_SEQ_OUT_OF_BLOCKS;
    }
    if (tid == 0 && !fc_bad) *a.free_count = fc - popped;
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
    } else if (a.status[s] != PKV_SEQ_OK) {
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
    for (int b = tok_begin; b < tok_end; ++b) {
        const int p = p0 + b;
        size_t row;
        if (ring) {
            row = (size_t)table[0] * a.ring_size + (size_t)(p % a.ring_size);
        } else {
            const int phys = table[p / a.bs];
            if (phys < 0 || phys >= a.num_blocks) {
                if (tid == 0) a.status[s] = PKV_SEQ_BAD_BLOCK;
                continue;
            }
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
}  // namespace pkv

extern "C" {

int32_t pkv_append(void* stream, const pkv_params* p, void* k_pool, void* v_pool,
                   int32_t* block_tables, int32_t table_stride, int32_t* table_lens,
                   int32_t* free_list, int32_t* free_count, const int32_t* pos,
                   const int32_t* tok_off, int32_t max_new, const void* k_new,
                   const void* v_new, int32_t total_rows, int32_t batch, int32_t* status) {
    using namespace pkv;
    clear_error();
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
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (!ring) hipLaunchKernelGGL(alloc_kernel, dim3(1), dim3(kNT), 0, st, a);
    dim3 grid((max_new + a.tok_per_wg - 1) / a.tok_per_wg, batch);
    hipLaunchKernelGGL(scatter_kernel, grid, dim3(kNT), 0, st, a);
    return check_launch("pkv_append");
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
