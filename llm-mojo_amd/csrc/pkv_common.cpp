// Host-side plumbing of libpkv: error reporting, parameter validation, workspace
// layout, and the single-sequence paged_attention_layer drop-in.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <utility>

#include "pkv_internal.h"

namespace pkv {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int32_t fail(int32_t code, const std::string& msg) {
    set_error(msg);
    return code;
}

int32_t check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(PKV_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return PKV_OK;
}

namespace {
struct Occ {
    std::mutex mu;
    std::map<std::tuple<const void*, int, int, size_t>, int> blocks;  // -> workgroups
    std::map<std::pair<const void*, int>, int> lds_limit;           // (kernel, device) -> bytes set
};
Occ& occ() {
    static Occ o;
    return o;
}
}  // namespace

bool reserve_lds(const void* fn, int bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    Occ& o = occ();
    std::lock_guard<std::mutex> lk(o.mu);
    const auto key = std::make_pair(fn, dev);
    const auto it = o.lds_limit.find(key);
    if (it != o.lds_limit.end() && it->second >= bytes) return true;
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
        return false;
    o.lds_limit[key] = bytes;
    return true;
}

int device_fill_workgroups(const void* fn, int threads, size_t lds, int cap) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    Occ& o = occ();
    std::lock_guard<std::mutex> lk(o.mu);
    auto key = std::make_tuple(fn, dev, threads, lds);
    auto it = o.blocks.find(key);
    int p = 0;
    if (it != o.blocks.end()) {
        p = it->second;
    } else {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return -1;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds) != hipSuccess)
            return -1;
        p = cus * (per_cu > 0 ? per_cu : 1);
        o.blocks.emplace(key, p);
    }
    return p > cap ? cap : p;
}

int32_t validate_params(const pkv_params* p) {
    if (!p) return fail(PKV_ERR_INVALID, "params is NULL");
    if (p->num_heads <= 0 || p->num_kv_heads <= 0 || p->num_heads % p->num_kv_heads != 0)
        return fail(PKV_ERR_INVALID, "num_kv_heads must be positive and divide num_heads");
    if (p->head_dim != 64 && p->head_dim != 256 && p->head_dim != 512)
        return fail(PKV_ERR_UNSUPPORTED, "head_dim must be 64, 256 or 512");
    if (p->block_size <= 0 || p->block_size > 256 || (p->block_size & (p->block_size - 1)))
        return fail(PKV_ERR_INVALID, "block_size must be a power of two in [1, 256]");
    if (p->num_blocks <= 0) return fail(PKV_ERR_INVALID, "num_blocks must be positive");
    if (p->kv_dtype != PKV_DTYPE_F32 && p->kv_dtype != PKV_DTYPE_BF16)
        return fail(PKV_ERR_INVALID, "kv_dtype must be PKV_DTYPE_F32 or PKV_DTYPE_BF16");
    if (p->ring_size < 0) return fail(PKV_ERR_INVALID, "ring_size must be >= 0");
    if (p->reserved != 0) return fail(PKV_ERR_INVALID, "reserved must be 0");
    // Row offsets are computed in 64-bit; the element index of a pool must still fit
    // the int64 range comfortably, which any real pool does.
    return PKV_OK;
}

AttendLayout attend_layout(const pkv_params* p, int32_t batch, int32_t q_len, int32_t max_pos) {
    AttendLayout L{};
    // Keys per split: 256 rounded down to a whole number of blocks (at least one block).
    int32_t bs = p->block_size;
    int32_t chunk = (256 / bs) * bs;
    if (chunk <= 0) chunk = bs;
    L.chunk = chunk;
    // Key range of one sequence: [window_start(pos0), pos0 + q_len - 1], pos0 + q_len - 1
    // <= max_pos. Chunks are aligned to multiples of `chunk` in absolute positions.
    int64_t full = (int64_t)max_pos / chunk + 1;
    int64_t mc = full;
    if (p->window > 0) {
        int64_t span = (int64_t)p->window + q_len - 1;  // keys touched by the queries
        int64_t win = (span + chunk - 1) / chunk + 1;
        if (win < mc) mc = win;
    }
    if (p->ring_size > 0) {  // a ring call never spans more than ring_size keys
        int64_t ring = ((int64_t)p->ring_size + chunk - 1) / chunk + 1;
        if (ring < mc) mc = ring;
    }
    if (mc < 1) mc = 1;
    L.max_chunks = (int32_t)mc;
    auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
    size_t rows = (size_t)batch * q_len * p->num_heads;
    L.ml_off = 0;
    // Partials are kept in the accumulation type (double for fp32 pools).
    size_t ml_bytes = align(rows * L.max_chunks * 2 * sizeof(double));
    L.o_off = L.ml_off + ml_bytes;
    size_t o_bytes = align(rows * L.max_chunks * (size_t)p->head_dim * sizeof(double));
    L.total = L.o_off + o_bytes;
    return L;
}

}  // namespace pkv

extern "C" {

size_t pkv_workspace_size(const pkv_params* p, int32_t batch, int32_t q_len, int32_t max_pos) {
    if (pkv::validate_params(p) != PKV_OK) return 0;
    if (batch <= 0 || q_len <= 0 || max_pos < 0) return 0;
    const size_t chunked = pkv::attend_layout(p, batch, q_len, max_pos).total;
    const size_t stream = pkv::stream_layout(p, batch, q_len).total;
    return chunked > stream ? chunked : stream;
}

const char* pkv_last_error(void) { return pkv::g_last_error.c_str(); }

int32_t pkv_version(void) { return (1 << 16) | 0; }

}  // extern "C"
