// Internal helpers shared by the libpkv HIP sources (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "pkv.h"

namespace pkv {

constexpr int kWave = 64;          // CDNA wavefront width
constexpr int kBlockThreads = 256; // 4 waves per workgroup for every kernel here
// Cache-policy operand of __builtin_amdgcn_global_load_lds that sets the NT (non-temporal)
// bit on gfx950: data read once is kept at the bottom of the L2's replacement order, so a
// stream of K/V pages or weights does not push out what is reused. Decode over fp32 pages
// streams ~9% faster with it (config 2: 0.68 -> 0.75 of HBM, same box).
constexpr int kCpolNT = 2;

// Lazy reference max of the online softmax (decode, verify, sparse and chunk attention): a
// row's reference m moves only when a batch's max exceeds it by more than kLazyMove
// (natural-log units), so the weights exp(s - m) stay below e^20 (~4.9e8, far inside float
// and double range) and the result does not change (softmax does not depend on the
// reference; the 1e-10 of the denominator shifts by at most a relative 1e-10, as l >= 1
// whenever a key is live). The rescale of the accumulators and its exponential then run on
// the few batches that move it, not on every batch whose max grows a little.
constexpr float kLazyMove = 20.f;

// Thread-local message behind pkv_last_error().
void set_error(const std::string& msg);
void clear_error();
int32_t fail(int32_t code, const std::string& msg);
int32_t check_launch(const char* what);

// Workgroups of `threads` threads and `lds` bytes of dynamic LDS of kernel `fn` that are
// resident on the current device at once (CUs x occupancy), at most `cap`; -1 if the
// runtime query fails. Cached per (kernel, device, shape).
int device_fill_workgroups(const void* fn, int threads, size_t lds, int cap);
// Lets kernel fn use up to `bytes` of dynamic LDS on the current device (above 64 KiB a
// kernel must opt in). The attribute is set once per kernel and device; false on failure.
bool reserve_lds(const void* fn, int bytes);

// Validates the geometry shared by every entry point. Returns PKV_OK or an error code
// (message set).
int32_t validate_params(const pkv_params* p);

inline size_t kv_elt_bytes(int32_t dtype) { return dtype == PKV_DTYPE_BF16 ? 2 : 4; }

// Workspace layout (bytes from the base; every region 256-byte aligned):
//   part_ml                     2 accumulators per (row, chunk): chunk max m, sum l
//   then part_o                 head_dim accumulators per (row, chunk)
// (accumulators are double for fp32 pools, float for bf16; sized for double)
struct AttendLayout {
    int32_t chunk;       // keys per split
    int32_t max_chunks;  // grid.x
    size_t ml_off;
    size_t o_off;
    size_t total;
};
AttendLayout attend_layout(const pkv_params* p, int32_t batch, int32_t q_len, int32_t max_pos);

// Stream-K attention (pkv_stream.hip): workspace layout and entry.
//   plan   int32 [4 batch + 5]     the key split (per_pair, even), the key prefix of every
//                                  sequence [batch + 1], then
//                                  for a fused append the allocation plan: the free count
//                                  as read, table lengths [batch], prefix of the blocks
//                                  needed [batch + 1], status before the pops [batch]
//   part_ml                        double (m, l) per (slot, row)
//   part_o                         double [head_dim] per (slot, row)
// slots = min(nwg_cap, kStreamMaxSlots) + batch, rows = num_heads * q_len: piece (w, s) of
// workgroup w < nwg <= nwg_cap and sequence s uses slot w + s.
constexpr int kStreamMaxSlots = 1024;  // workgroups along the keys, at most
// LDS of one CU; the stream kernels keep 5 ints per sequence there (8 with a fused append),
// so a launch takes at most kStreamMaxBatch sequences.
constexpr size_t kStreamLdsMax = 160 * 1024;
constexpr int kStreamMaxBatch = 8191;
struct StreamLayout {
    size_t plan_off;
    size_t ml_off;
    size_t o_off;
    size_t total;
};
StreamLayout stream_layout(const pkv_params* p, int32_t batch, int32_t q_len,
                           int32_t nwg_cap = kStreamMaxSlots);
// True when the stream kernel covers this geometry: head_dim 256 or 512 with
// G = num_heads / num_kv_heads <= 8 (any number of queries: launched in groups).
bool stream_eligible(const pkv_params* p, int32_t G);
// The appended rows of a fused append + attention (pkv_append_attend), with the block
// manager's state. The attention launch computes the block allocation from the state as
// it stands before the call (every workgroup the same result), copies row r of sequence s
// (tok_off[s] <= r < tok_off[s + 1], position pos[s] + r - tok_off[s]) into the pool
// with scatter_kernel's checks, and reads those positions from k_new / v_new instead of
// the pool; the merge launch after it writes the new table entries, table_lens,
// free_count and status. So no word of the state is written in the launch that reads it.
// k_new == NULL: no appended rows.
struct NewRows {
    const char* k_new;
    const char* v_new;
    const int32_t* tok_off;     // [batch + 1]
    char* k_dst;                // the pools, written
    char* v_dst;
    int32_t* tables;            // block tables [batch][table_stride]
    int32_t* table_lens;
    const int32_t* free_list;
    int32_t* free_count;
    int32_t* status;
    int32_t max_new;
    int32_t total_rows;
};
// Largest batch whose allocation plan the fused launch keeps in LDS.
constexpr int kFuseMaxBatch = 1024;
// True when stream_attend takes the appended rows itself for q_len queries: paged pools,
// one launch on the vector kernel and batch <= kFuseMaxBatch.
bool stream_takes_new_rows(const pkv_params* p, int32_t q_len, int32_t batch);
// Checks the arguments of a paged or ring append (pkv_state.hip); PKV_OK or an error code.
int32_t append_validate(const pkv_params* p, void* k_pool, void* v_pool, int32_t* block_tables,
                        int32_t table_stride, int32_t* table_lens, int32_t* free_list,
                        int32_t* free_count, const int32_t* pos, const int32_t* tok_off,
                        int32_t max_new, const void* k_new, const void* v_new,
                        int32_t total_rows, int32_t batch, int32_t* status);
// Validates a paged or ring append and launches it (pkv_state.hip): the block allocation,
// then, with scatter, the row copies.
int32_t append_launch(hipStream_t st, const pkv_params* p, void* k_pool, void* v_pool,
                      int32_t* block_tables, int32_t table_stride, int32_t* table_lens,
                      int32_t* free_list, int32_t* free_count, const int32_t* pos,
                      const int32_t* tok_off, int32_t max_new, const void* k_new,
                      const void* v_new, int32_t total_rows, int32_t batch, int32_t* status,
                      bool scatter);

// ---- block allocation of an append (BlockManager, model_speculative_moe_batched.mojo:
// 789-807): sequence s, in index order, pops the blocks it lacks from the top of the free
// list, free_list[fc - 1 - pref[s] - j] for its j-th new block (pref = exclusive prefix
// of the needs); one that runs the list dry keeps what it popped (OUT_OF_BLOCKS).
// Shared by alloc_kernel and the fused append + attention launch.

// Blocks an append of rows [r0, r1) of the new-row arrays at position p needs beyond the
// len its table holds (>= 0), or a negative PKV_SEQ_* code.
__device__ inline int append_blocks_needed(int p, int r0, int r1, int max_new,
                                           int total_rows, int bs, int table_stride,
                                           int len) {
    const int n = r1 - r0;
    if (p < 0 || n <= 0) return 0;
    if (n > max_new || r0 < 0 || r1 > total_rows) return PKV_SEQ_BAD_ARGS;
    const long long last_blk = ((long long)p + n - 1) / bs;
    if (last_blk >= table_stride) return PKV_SEQ_TABLE_FULL;
    if (len < 0 || len > table_stride) return PKV_SEQ_BAD_BLOCK;
    const long long need = last_blk + 1 - len;
    return need > 0 ? (int)need : 0;
}
// Blocks granted to a sequence that needs `need` and whose pops start pref entries below
// the top of a free list of fc entries.
__device__ inline int append_granted(int need, int fc, int pref) {
    const int avail = fc - pref;
    return need == 0 || avail <= 0 ? 0 : (avail < need ? avail : need);
}
// Status after the pops (before the check of the touched table entries): code0 is
// PKV_SEQ_OK or the code append_blocks_needed returned; fc_bad: a free count outside
// [0, num_blocks], read as an empty list.
__device__ inline int append_pop_status(int code0, int need, int granted, bool fc_bad) {
    if (granted < need) return fc_bad ? PKV_SEQ_BAD_BLOCK : PKV_SEQ_OUT_OF_BLOCKS;
    return code0;
}
// Table entry of block index blk after the pops: held entries from the table, new ones
// from the free list (where the allocation takes them), -1 past the granted blocks.
__device__ inline int append_block_entry(const int32_t* table, const int32_t* free_list,
                                         int len, int granted, int fc, int pref, int blk) {
    if (blk < 0) return -1;
    if (blk < len) return table[blk];
    if (blk < len + granted) return free_list[fc - 1 - pref - (blk - len)];
    return -1;
}

// pos == NULL: one sequence at pos_scalar; in ring mode its ring starts at row
// ring_base (otherwise ring slot block_tables[s * table_stride] starts at row
// slot * ring_size). keys != NULL: sparse mode, sequence s attends the key positions
// keys[key_off[s] .. key_off[s+1]) (q_len 1, at most max_keys each). q_lens != NULL:
// sequence s has q_lens[s] <= q_len queries; its other rows of out are not written.
int32_t stream_attend(const pkv_params* p, const float* q, const void* k_pool,
                      const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                      const int32_t* pos, int32_t pos_scalar, int64_t ring_base, int32_t q_len,
                      const int32_t* q_lens, int32_t batch, int32_t max_pos, const int32_t* keys,
                      const int32_t* key_off, int32_t max_keys, float* out, void* workspace,
                      hipStream_t st, const NewRows* nr = nullptr,
                      int32_t nwg_cap = kStreamMaxSlots);

__host__ __device__ inline int32_t window_start(int32_t pos, int32_t window) {
    if (window <= 0) return 0;
    int32_t s = pos - window + 1;
    return s > 0 ? s : 0;
}

// Ring mode (ring_size > 0, attention.mojo:144-148, :264-269): key t of a sequence whose
// ring starts at row `base` lives at row base + t % ring_size. The keys of one call span
// at most ring_size positions, so from the row r0 = t0 % ring_size of the first key t0
// every later key t is one subtraction away.
__host__ __device__ inline int64_t ring_key_row(int64_t base, int32_t r0, int32_t t_minus_t0,
                                                int32_t ring_size) {
    int32_t r = r0 + t_minus_t0;
    if (r >= ring_size) r -= ring_size;
    return base + r;
}

// bf16 (stored as uint16) -> fp32, exact.
__device__ inline float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even (NaN stays a quiet NaN).
__device__ inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

}  // namespace pkv
