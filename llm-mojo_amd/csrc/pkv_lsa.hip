// LSA bucket cache on the device: expand_buckets and rollback_to for a batch.
//
// The reference keeps one LSALayerIndex per (kv slot, global-layer group)
// (model_speculative_moe_batched.mojo:1885-1888, :632) on the host. Its bucket cache --
// per bucket a member count and up to 32 token positions (lsa_core.mojo:222-233) -- is what
// expand_buckets (lsa_core.mojo:568-604) turns into the key list of the sparse attention,
// and what rollback_to (lsa_core.mojo:287-303) trims after rejected drafts. Here the cache
// lives in HBM beside the pools, so the key lists are built where pkv_attend_sparse reads
// them: index instance i owns sizes[i][max_buckets], members[i][max_buckets][32],
// closed_blocks[i] and total_tokens[i]. Building buckets when a 512-token block closes
// (Ward clustering) and picking them (select_top_p) stay with the index on the host.
//
// pkv_lsa_expand is two launches. lsa_gather_kernel gives each sequence one wave: the
// picked ids and sizes of up to 64 buckets come in one load per lane, then every member row
// of those buckets in one round trip into LDS, and the filter walks them in order (one
// ballot per bucket keeps the members' order) into a fixed-stride staging area of the
// workspace. lsa_compact_kernel, one workgroup, scans the lengths into key_off and copies
// the lists end to end (CSR). lsa_rollback_kernel: one workgroup applying the entries in
// order, so repeated index ids behave like repeated calls.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pkv_internal.h"

namespace pkv {
namespace {

constexpr int kLsaBucketCap = 32;       // LSA_BUCKET_CAP (lsa_core.mojo:27)
constexpr int kLsaBlockBuckets = 32;    // LSA_BLOCK_BUCKET_COUNT (lsa_core.mojo:28)
constexpr int kLsaClusterBlock = 512;   // LSA_CLUSTER_BLOCK_SIZE (lsa_core.mojo:26)
constexpr int kLsaCompactThreads = 1024;
constexpr int kLsaCompactWaves = kLsaCompactThreads / 64;
constexpr int kLsaMaxBatch = kLsaCompactThreads;  // one scan element per thread
constexpr int kLsaChunk = 64;                     // picked buckets staged per round

struct LsaExpandArgs {
    const int32_t* index_ids;  // [batch]
    const int32_t* picked;     // [batch][picked_stride]
    const int32_t* n_picked;   // [batch]
    const int32_t* pos;        // [batch]
    const int32_t* sizes;      // [num_indices][max_buckets]
    const int32_t* members;    // [num_indices][max_buckets][32]
    int32_t* keys;
    int32_t* key_off;  // [batch + 1]
    int32_t* status;   // [batch]
    int32_t* stage;    // workspace: [batch][per] lists, then [batch] lengths
    int32_t* len;
    int32_t per;       // longest list (pkv_lsa_max_keys)
    int32_t picked_stride;
    int32_t top_k;
    int32_t sink;
    int32_t window;
    int32_t batch;
    int32_t num_indices;
    int32_t max_buckets;
};

// One wave per sequence s = blockIdx.x.
__global__ __launch_bounds__(64) void lsa_gather_kernel(LsaExpandArgs a) {
    __shared__ int s_b[kLsaChunk], s_size[kLsaChunk];
    __shared__ int s_tok[kLsaChunk][kLsaBucketCap];
    const int s = blockIdx.x, lane = threadIdx.x;
    int32_t* out = a.stage + (size_t)s * a.per;
    const int p = a.pos[s];
    const int ws = max(0, p + 1 - a.window);  // window start (lsa_core.mojo:577)
    const int idx = a.index_ids[s];
    bool bad = false;
    int n = 0;
    if (idx >= 0 && idx < a.num_indices) {
        int np = a.n_picked[s];
        if (np < 0 || np > a.picked_stride) {
            bad = true;
            np = max(0, min(np, a.picked_stride));
        }
        const int32_t* sz = a.sizes + (size_t)idx * a.max_buckets;
        const int32_t* mem = a.members + (size_t)idx * a.max_buckets * kLsaBucketCap;
        // 1. members of the picked buckets, in order, within [sink, window start). As in the
        // reference, the count is tested after each append (so a bucket adds at least one
        // kept member) and after each bucket (so top_k <= 0 stops after the first).
        bool stop = false;
        for (int j0 = 0; j0 < np && !stop; j0 += kLsaChunk) {
            const int cnt = min(kLsaChunk, np - j0);
            int b = -1, size = 0;
            if (lane < cnt) b = a.picked[(size_t)s * a.picked_stride + j0 + lane];
            if (lane < cnt && b >= 0 && b < a.max_buckets) size = min(max(sz[b], 0), kLsaBucketCap);
            s_b[lane] = b;
            s_size[lane] = size;
            __syncthreads();
            for (int t = lane; t < cnt * kLsaBucketCap; t += 64) {
                const int j = t / kLsaBucketCap, m = t % kLsaBucketCap;
                s_tok[j][m] = m < s_size[j] ? mem[(size_t)s_b[j] * kLsaBucketCap + m] : 0;
            }
            __syncthreads();
            for (int j = 0; j < cnt; ++j) {
                if (j0 + j > 0 && n >= a.top_k) {
                    stop = true;
                    break;
                }
                const int bj = s_b[j];
                if (bj < 0 || bj >= a.max_buckets) {
                    bad = true;
                    continue;
                }
                int tok = 0;
                bool keep = false;
                if (lane < s_size[j]) {
                    tok = s_tok[j][lane];
                    keep = tok >= a.sink && tok < ws;
                }
                const uint64_t mask = __ballot(keep);
                const int rank = __popcll(mask & ((1ull << lane) - 1ull));
                const int take = min(__popcll(mask), max(a.top_k - n, 1));
                if (keep && rank < take) out[n + rank] = tok;
                n += take;
            }
            __syncthreads();  // the next chunk overwrites the staged rows
        }
    } else {
        bad = true;
    }
    // 2. the window [ws, p]
    const int wcnt = max(0, p - ws + 1);
    for (int t = lane; t < wcnt; t += 64) out[n + t] = ws + t;
    n += wcnt;
    // 3. the sinks [0, min(sink, ws, p + 1))
    const int scnt = max(0, min(min(a.sink, ws), p + 1));
    for (int t = lane; t < scnt; t += 64) out[n + t] = t;
    if (lane == 0) {
        a.len[s] = n + scnt;
        a.status[s] = bad ? PKV_SEQ_BAD_INDEX : PKV_SEQ_OK;
    }
}

// Scan of the lengths into key_off, then the lists end to end into keys.
__global__ __launch_bounds__(kLsaCompactThreads) void lsa_compact_kernel(LsaExpandArgs a) {
    __shared__ int s_off[kLsaMaxBatch];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    s_off[tid] = tid < a.batch ? a.len[tid] : 0;
    __syncthreads();
    for (int d = 1; d < kLsaMaxBatch; d <<= 1) {  // inclusive Hillis-Steele scan
        const int t = tid >= d ? s_off[tid - d] : 0;
        __syncthreads();
        s_off[tid] += t;
        __syncthreads();
    }
    if (tid < a.batch) a.key_off[tid + 1] = s_off[tid];
    if (tid == 0) a.key_off[0] = 0;
    for (int s = wave; s < a.batch; s += kLsaCompactWaves) {
        const int base = s == 0 ? 0 : s_off[s - 1];
        const int n = s_off[s] - base;
        const int32_t* src = a.stage + (size_t)s * a.per;
        for (int t0 = 0; t0 < n; t0 += 4 * 64) {  // four loads in flight per lane
            int v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int t = t0 + u * 64 + lane;
                v[u] = t < n ? src[t] : 0;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int t = t0 + u * 64 + lane;
                if (t < n) a.keys[base + t] = v[u];
            }
        }
    }
}

struct LsaRollbackArgs {
    const int32_t* index_ids;  // [count]
    const int32_t* target;     // [count]
    int32_t* closed_blocks;    // [num_indices]
    int32_t* total_tokens;     // [num_indices]
    int32_t* sizes;            // [num_indices][max_buckets]
    int32_t count;
    int32_t num_indices;
    int32_t max_capacity;
    int32_t max_buckets;
};

// rollback_to (lsa_core.mojo:287-303), with reset (:281-285) for targets <= 0: entry by
// entry, the buckets of every cluster block that reopens get size 0.
__global__ __launch_bounds__(256) void lsa_rollback_kernel(LsaRollbackArgs a) {
    const int tid = threadIdx.x;
    for (int k = 0; k < a.count; ++k) {
        const int idx = a.index_ids[k];
        if (idx < 0 || idx >= a.num_indices) continue;  // uniform: the same k for all
        const int t = a.target[k];
        const int closed = a.closed_blocks[idx];
        int32_t* sizes = a.sizes + (size_t)idx * a.max_buckets;
        int lo, hi, new_closed, new_total;
        if (t <= 0) {
            lo = 0, hi = a.max_buckets, new_closed = 0, new_total = 0;
        } else {
            new_total = min(t, a.max_capacity);
            const int valid = new_total / kLsaClusterBlock;
            new_closed = min(closed, valid);
            lo = new_closed * kLsaBlockBuckets;
            hi = min(closed, a.max_buckets / kLsaBlockBuckets) * kLsaBlockBuckets;
        }
        for (int i = lo + tid; i < hi; i += 256) sizes[i] = 0;
        __syncthreads();  // every thread has read closed_blocks[idx]
        if (tid == 0) {
            a.closed_blocks[idx] = new_closed;
            a.total_tokens[idx] = new_total;
        }
        __syncthreads();  // the next entry may name the same index
    }
}

}  // namespace
}  // namespace pkv

extern "C" {

int32_t pkv_lsa_max_keys(int32_t top_k, int32_t sink_size, int32_t window_size) {
    const int64_t n = (int64_t)(top_k > 1 ? top_k : 1) + (window_size > 0 ? window_size : 0) +
                      (sink_size > 0 ? sink_size : 0);
    return n > INT32_MAX ? -1 : (int32_t)n;
}

size_t pkv_lsa_expand_workspace_size(int32_t batch, int32_t top_k, int32_t sink_size,
                                     int32_t window_size) {
    const int32_t per = pkv_lsa_max_keys(top_k, sink_size, window_size);
    if (batch <= 0 || per < 0) return 0;
    return ((size_t)batch * per + batch) * sizeof(int32_t);
}

int32_t pkv_lsa_expand(void* stream, const int32_t* index_ids, const int32_t* picked,
                       int32_t picked_stride, const int32_t* n_picked, const int32_t* pos,
                       int32_t top_k, int32_t sink_size, int32_t window_size, int32_t batch,
                       const int32_t* sizes, const int32_t* members, int32_t num_indices,
                       int32_t max_buckets, int32_t* keys, int32_t* key_off,
                       int64_t keys_capacity, int32_t* status, void* workspace,
                       size_t workspace_bytes) {
    using namespace pkv;
    clear_error();
    if (batch <= 0) return fail(PKV_ERR_INVALID, "pkv_lsa_expand: batch must be positive");
    if (batch > kLsaMaxBatch) return fail(PKV_ERR_UNSUPPORTED, "pkv_lsa_expand: batch must be <= 1024");
    if (!index_ids || !n_picked || !pos || !sizes || !members || !keys || !key_off || !status ||
        !workspace || (!picked && picked_stride > 0))
        return fail(PKV_ERR_INVALID, "pkv_lsa_expand: null device pointer");
    if (picked_stride < 0 || num_indices <= 0 || max_buckets <= 0)
        return fail(PKV_ERR_INVALID, "pkv_lsa_expand: picked_stride, num_indices, max_buckets");
    if (sink_size < 0 || window_size < 0)
        return fail(PKV_ERR_INVALID, "pkv_lsa_expand: sink_size and window_size must be >= 0");
    const int32_t per = pkv_lsa_max_keys(top_k, sink_size, window_size);
    if (per < 0) return fail(PKV_ERR_INVALID, "pkv_lsa_expand: list bound overflows int32");
    if (keys_capacity < (int64_t)batch * per || (int64_t)batch * per > INT32_MAX)
        return fail(PKV_ERR_WORKSPACE, "pkv_lsa_expand: keys smaller than batch * pkv_lsa_max_keys()");
    if (workspace_bytes < pkv_lsa_expand_workspace_size(batch, top_k, sink_size, window_size))
        return fail(PKV_ERR_WORKSPACE, "workspace smaller than pkv_lsa_expand_workspace_size()");
    LsaExpandArgs a{};
    a.index_ids = index_ids;
    a.picked = picked;
    a.n_picked = n_picked;
    a.pos = pos;
    a.sizes = sizes;
    a.members = members;
    a.keys = keys;
    a.key_off = key_off;
    a.status = status;
    a.stage = static_cast<int32_t*>(workspace);
    a.len = a.stage + (size_t)batch * per;
    a.per = per;
    a.picked_stride = picked_stride;
    a.top_k = top_k;
    a.sink = sink_size;
    a.window = window_size;
    a.batch = batch;
    a.num_indices = num_indices;
    a.max_buckets = max_buckets;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(lsa_gather_kernel, dim3(batch), dim3(64), 0, st, a);
    hipLaunchKernelGGL(lsa_compact_kernel, dim3(1), dim3(kLsaCompactThreads), 0, st, a);
    return check_launch("pkv_lsa_expand");
}

int32_t pkv_lsa_rollback(void* stream, const int32_t* index_ids, const int32_t* target_tokens,
                         int32_t count, int32_t num_indices, int32_t max_capacity,
                         int32_t max_buckets, int32_t* closed_blocks, int32_t* total_tokens,
                         int32_t* sizes) {
    using namespace pkv;
    clear_error();
    if (count < 0 || num_indices <= 0 || max_capacity <= 0)
        return fail(PKV_ERR_INVALID, "pkv_lsa_rollback: count, num_indices, max_capacity");
    if ((int64_t)max_buckets !=
        ((int64_t)max_capacity + kLsaClusterBlock - 1) / kLsaClusterBlock * kLsaBlockBuckets)
        return fail(PKV_ERR_INVALID, "pkv_lsa_rollback: max_buckets must be ceil(max_capacity / 512) * 32");
    if (count == 0) return PKV_OK;
    if (!index_ids || !target_tokens || !closed_blocks || !total_tokens || !sizes)
        return fail(PKV_ERR_INVALID, "pkv_lsa_rollback: null device pointer");
    LsaRollbackArgs a{};
    a.index_ids = index_ids;
    a.target = target_tokens;
    a.closed_blocks = closed_blocks;
    a.total_tokens = total_tokens;
    a.sizes = sizes;
    a.count = count;
    a.num_indices = num_indices;
    a.max_capacity = max_capacity;
    a.max_buckets = max_buckets;
    hipLaunchKernelGGL(lsa_rollback_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), a);
    return check_launch("pkv_lsa_rollback");
}

}  // extern "C"
