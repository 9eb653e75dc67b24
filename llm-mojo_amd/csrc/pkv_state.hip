// K1 (fused block allocation + K/V scatter) and K5 (rollback / retire).
//
// Block-manager state lives in caller-owned device memory: tables [batch][stride],
// table_lens [batch], the LIFO free list [num_blocks] and its count. The reference
// keeps the same state on the host (BlockManager / Sequence,
// model_speculative_moe_batched.mojo:789-845) and mutates it one sequence at a time;
// here every sequence's allocation is derived from an ordered prefix sum over the
// batch, which yields exactly the serial order's result.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pkv_internal.h"

namespace pkv {
namespace {

constexpr int kNT = kBlockThreads;

// Block-wide exclusive scan of one int per thread; returns the exclusive prefix and
// writes the block total to *total. `tmp` holds kNT ints of LDS.
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

struct AppendArgs {
    char* k_pool;
    char* v_pool;
    int32_t* tables;
    int32_t table_stride;
    int32_t* table_lens;
    const int32_t* free_list;
    int32_t* free_count;
    const int32_t* pos;
    const int32_t* n_new;
    int32_t max_new;
    const char* k_new;
    const char* v_new;
    int32_t batch;
    int32_t* status;
    int32_t bs;
    int32_t num_blocks;
    int32_t row_bytes;  // num_kv_heads * head_dim * element size (multiple of 16)
    int32_t tok_per_wg;
    int32_t* ticket;
    int32_t num_wg;
};

// Blocks sequence s still needs, or a negative PKV_SEQ_* code. Reads only state that
// no workgroup writes before the commit.
__device__ inline int append_need(const AppendArgs& a, int s, int* len_out) {
    int len = a.table_lens[s];
    *len_out = len;
    int p = a.pos[s], n = a.n_new[s];
    if (p < 0 || n <= 0) return 0;
    if (n > a.max_new) return PKV_SEQ_BAD_ARGS;
    long long last = (long long)p + n - 1;
    long long last_blk = last / a.bs;
    if (last_blk >= a.table_stride) return PKV_SEQ_TABLE_FULL;
    if (len < 0 || len > a.table_stride) return PKV_SEQ_BAD_BLOCK;
    long long need = last_blk + 1 - len;
    return need > 0 ? (int)need : 0;
}

// grid = (ceil(max_new / tok_per_wg), batch); 256 threads.
// Every workgroup recomputes the ordered allocation plan from the pre-call state and
// scatters its tokens' rows; the last workgroup to finish (atomic ticket) commits
// tables, table_lens, free_count and status, so no workgroup ever reads state that
// another has already changed.
__global__ __launch_bounds__(kNT) void append_kernel(AppendArgs a) {
    __shared__ int s_tmp[kNT];
    __shared__ int s_info[4];  // my prefix, my granted, my len, fc
    __shared__ int s_last;
    const int tid = threadIdx.x;
    const int s_me = blockIdx.y;
    const int tile = blockIdx.x;

    int fc = *a.free_count;
    bool fc_bad = fc < 0 || fc > a.num_blocks;
    if (fc_bad) fc = 0;

    // Pass 1: segment sums of `need` over the batch (thread-contiguous segments keep
    // the prefix in sequence order).
    const int seg = (a.batch + kNT - 1) / kNT;
    const int s_begin = tid * seg;
    const int s_end = min(a.batch, s_begin + seg);
    int seg_sum = 0;
    for (int s = s_begin; s < s_end; ++s) {
        int len;
        int need = append_need(a, s, &len);
        if (need > 0) seg_sum += need;
    }
    int total;
    int seg_prefix = block_exclusive_scan(seg_sum, s_tmp, &total);
    // Pass 2: the owner of s_me publishes its prefix.
    if (s_me >= s_begin && s_me < s_end) {
        int run = seg_prefix;
        for (int s = s_begin; s < s_end; ++s) {
            int len;
            int need = append_need(a, s, &len);
            if (s == s_me) {
                int granted = 0;
                int code = need < 0 ? need : 0;
                if (need > 0) {
                    int avail = fc - run;
                    granted = avail <= 0 ? 0 : (avail < need ? avail : need);
                    if (granted < need) code = fc_bad ? PKV_SEQ_BAD_BLOCK : PKV_SEQ_OUT_OF_BLOCKS;
                }
                s_info[0] = run;
                s_info[1] = code;  // 0 = proceed
                s_info[2] = len;
                s_info[3] = granted;
            }
            if (need > 0) run += need;
        }
    }
    __syncthreads();

    // Scatter this workgroup's tokens (only when the whole sequence's allocation holds).
    const int my_prefix = s_info[0];
    const int my_code = s_info[1];
    const int my_len = s_info[2];
    const int p0 = a.pos[s_me];
    const int n = a.n_new[s_me];
    if (my_code == 0 && p0 >= 0 && n > 0) {
        const int tok_begin = tile * a.tok_per_wg;
        const int tok_end = min(n, tok_begin + a.tok_per_wg);
        const int vec_per_row = a.row_bytes / 16;
        for (int b = tok_begin; b < tok_end; ++b) {
            const int p = p0 + b;
            const int lb = p / a.bs;
            int phys;
            if (lb < my_len) {
                phys = a.tables[(size_t)s_me * a.table_stride + lb];
            } else {
                int idx = fc - 1 - my_prefix - (lb - my_len);
                phys = (idx >= 0 && idx < a.num_blocks) ? a.free_list[idx] : -1;
            }
            if (phys < 0 || phys >= a.num_blocks) continue;  // reported by the commit
            const size_t row = (size_t)phys * a.bs + (size_t)(p % a.bs);
            const uint4* ks = reinterpret_cast<const uint4*>(
                a.k_new + ((size_t)s_me * a.max_new + b) * a.row_bytes);
            const uint4* vs = reinterpret_cast<const uint4*>(
                a.v_new + ((size_t)s_me * a.max_new + b) * a.row_bytes);
            uint4* kd = reinterpret_cast<uint4*>(a.k_pool + row * a.row_bytes);
            uint4* vd = reinterpret_cast<uint4*>(a.v_pool + row * a.row_bytes);
            for (int i = tid; i < vec_per_row; i += kNT) {
                uint4 kv = ks[i];
                uint4 vv = vs[i];
                kd[i] = kv;
                vd[i] = vv;
            }
        }
    }

    // Ticket: the last workgroup commits the state.
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        int t = atomicAdd(a.ticket, 1);
        s_last = (t == a.num_wg - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    int run = seg_prefix;
    int popped = 0;
    for (int s = s_begin; s < s_end; ++s) {
        int len;
        int need = append_need(a, s, &len);
        int code = need < 0 ? need : 0;
        int granted = 0;
        if (need > 0) {
            int avail = fc - run;
            granted = avail <= 0 ? 0 : (avail < need ? avail : need);
            if (granted < need) code = fc_bad ? PKV_SEQ_BAD_BLOCK : PKV_SEQ_OUT_OF_BLOCKS;
            run += need;
        }
        int32_t* table = a.tables + (size_t)s * a.table_stride;
        int prefix_s = run - (need > 0 ? need : 0);
        for (int j = 0; j < granted; ++j) {
            int blk = a.free_list[fc - 1 - prefix_s - j];
            if (blk < 0 || blk >= a.num_blocks) code = PKV_SEQ_BAD_BLOCK;
            table[len + j] = blk;
        }
        if (code == 0 && a.pos[s] >= 0 && a.n_new[s] > 0) {
            // Pre-existing entries covering the appended positions must be valid.
            int lb0 = a.pos[s] / a.bs;
            int lb1 = min(len, (a.pos[s] + a.n_new[s] - 1) / a.bs + 1);
            for (int lb = lb0; lb < lb1; ++lb) {
                int blk = table[lb];
                if (blk < 0 || blk >= a.num_blocks) code = PKV_SEQ_BAD_BLOCK;
            }
        }
        if (granted > 0) a.table_lens[s] = len + granted;
        a.status[s] = code;
        popped += granted;
    }
    // free_count -= popped (block-wide sum of per-thread pops).
    int all_popped;
    block_exclusive_scan(popped, s_tmp, &all_popped);
    if (tid == 0) {
        if (!fc_bad) *a.free_count = fc - all_popped;
        *a.ticket = 0;
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

__device__ inline int rollback_keep(const RollbackArgs& a, int s, int len) {
    int nl = a.new_len[s];
    if (nl < 0) return len;
    int keep = (int)(((long long)nl + a.bs - 1) / a.bs);
    return keep < len ? keep : len;
}

// One workgroup: ordered prefix over the freed counts, then each sequence pushes its
// tail blocks (ascending logical order) at free_list[fc + prefix + j].
__global__ __launch_bounds__(kNT) void rollback_kernel(RollbackArgs a) {
    __shared__ int s_tmp[kNT];
    __shared__ int s_bad;
    const int tid = threadIdx.x;
    if (tid == 0) s_bad = 0;
    __syncthreads();
    const int fc = *a.free_count;
    const int seg = (a.batch + kNT - 1) / kNT;
    const int s_begin = tid * seg;
    const int s_end = min(a.batch, s_begin + seg);

    int seg_sum = 0;
    for (int s = s_begin; s < s_end; ++s) {
        int len = a.table_lens[s];
        if (len < 0 || len > a.table_stride) {
            s_bad = 1;
            continue;
        }
        int keep = rollback_keep(a, s, len);
        const int32_t* table = a.tables + (size_t)s * a.table_stride;
        for (int j = keep; j < len; ++j)
            if (table[j] < 0 || table[j] >= a.num_blocks) s_bad = 1;
        seg_sum += len - keep;
    }
    int total;
    int run = block_exclusive_scan(seg_sum, s_tmp, &total);
    const bool reject = s_bad || fc < 0 || (long long)fc + total > a.num_blocks;
    for (int s = s_begin; s < s_end; ++s) {
        int len = a.table_lens[s];
        bool len_ok = len >= 0 && len <= a.table_stride;
        int keep = len_ok ? rollback_keep(a, s, len) : 0;
        int freed = len_ok ? len - keep : 0;
        if (reject) {
            if (a.status) {
                int code = PKV_SEQ_OK;
                if (!len_ok) code = PKV_SEQ_BAD_BLOCK;
                else if (freed > 0) code = s_bad ? PKV_SEQ_BAD_BLOCK : PKV_SEQ_FREE_OVERFLOW;
                a.status[s] = code;
            }
            continue;
        }
        const int32_t* table = a.tables + (size_t)s * a.table_stride;
        for (int j = 0; j < freed; ++j) a.free_list[fc + run + j] = table[keep + j];
        a.table_lens[s] = keep;
        if (a.status) a.status[s] = PKV_SEQ_OK;
        run += freed;
    }
    __syncthreads();
    if (tid == 0 && !reject) *a.free_count = fc + total;
}

}  // namespace
}  // namespace pkv

extern "C" {

int32_t pkv_append(void* stream, const pkv_params* p, void* k_pool, void* v_pool,
                   int32_t* block_tables, int32_t table_stride, int32_t* table_lens,
                   int32_t* free_list, int32_t* free_count, const int32_t* pos,
                   const int32_t* n_new, int32_t max_new, const void* k_new, const void* v_new,
                   int32_t batch, int32_t* status, void* workspace, size_t workspace_bytes) {
    using namespace pkv;
    clear_error();
    int32_t rc = validate_params(p);
    if (rc != PKV_OK) return rc;
    if (batch <= 0 || max_new <= 0 || table_stride <= 0)
        return fail(PKV_ERR_INVALID, "batch, max_new and table_stride must be positive");
    if (!k_pool || !v_pool || !block_tables || !table_lens || !free_list || !free_count ||
        !pos || !n_new || !k_new || !v_new || !status || !workspace)
        return fail(PKV_ERR_INVALID, "null device pointer");
    if (workspace_bytes < kTicketBytes)
        return fail(PKV_ERR_WORKSPACE, "workspace smaller than the append ticket");
    AppendArgs a{};
    a.k_pool = static_cast<char*>(k_pool);
    a.v_pool = static_cast<char*>(v_pool);
    a.tables = block_tables;
    a.table_stride = table_stride;
    a.table_lens = table_lens;
    a.free_list = free_list;
    a.free_count = free_count;
    a.pos = pos;
    a.n_new = n_new;
    a.max_new = max_new;
    a.k_new = static_cast<const char*>(k_new);
    a.v_new = static_cast<const char*>(v_new);
    a.batch = batch;
    a.status = status;
    a.bs = p->block_size;
    a.num_blocks = p->num_blocks;
    a.row_bytes = (int32_t)((size_t)p->num_kv_heads * p->head_dim * kv_elt_bytes(p->kv_dtype));
    // Tokens per workgroup: one row pair is row_bytes*2 (8 or 16 KiB at 8 x 256);
    // aim for ~64 KiB of copies per workgroup.
    int tpw = (64 * 1024) / (2 * a.row_bytes);
    a.tok_per_wg = tpw < 1 ? 1 : tpw;
    a.ticket = static_cast<int32_t*>(workspace);
    dim3 grid((max_new + a.tok_per_wg - 1) / a.tok_per_wg, batch);
    if ((long long)grid.x * grid.y > 0x7fffffffLL) return fail(PKV_ERR_INVALID, "grid too large");
    a.num_wg = (int32_t)(grid.x * grid.y);
    hipLaunchKernelGGL(append_kernel, grid, dim3(kNT), 0, static_cast<hipStream_t>(stream), a);
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
