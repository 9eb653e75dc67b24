// pkv_attend_noalloc -- pkv_attend without a workspace argument, for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc).
//
// The split-K partials and the merge plan live in `scratch`, a file-scope device array of
// kScratchBytes that every GPU holds from the first call on it until the process ends.
// Host code never passes the array's name to a kernel: on the host that name is only a
// stand-in, so the device address is taken once per device with hipGetSymbolAddress
// (with that device current) and kept; every launch gets that address. Nothing here
// allocates: no hipMalloc, hipFree or allocating library call.
//
// Nothing in the scratch must start at zero: the attention launch writes the plan and
// every piece's partials before the merge launch reads them, so the previous call's
// contents are never read. Calls that overlap on one GPU (two streams, or two host
// threads) share the array and race; order them on one stream.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>

#include "pkv_internal.h"

namespace pkv {

constexpr size_t kScratchBytes = PKV_NOALLOC_SCRATCH_BYTES;  // 64 MiB per GPU

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up on the first call there.
int32_t scratch_address(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess)
        return fail(PKV_ERR_HIP, "pkv_attend_noalloc: hipGetDevice failed");
    if (dev < 0 || dev >= kMaxDevices)
        return fail(PKV_ERR_UNSUPPORTED, "pkv_attend_noalloc: device index beyond 63");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(PKV_ERR_HIP, std::string("pkv_attend_noalloc: hipGetSymbolAddress: ") +
                                         hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return PKV_OK;
}

}  // namespace
}  // namespace pkv

extern "C" {

int32_t pkv_attend_noalloc(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                           const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                           const int32_t* pos, int32_t q_len, int32_t batch, int32_t max_pos,
                           float* out) {
    using namespace pkv;
    clear_error();
    int32_t rc = validate_params(p);
    if (rc != PKV_OK) return rc;
    if (batch <= 0 || batch > 4096 || q_len <= 0 || table_stride <= 0 || max_pos < 0)
        return fail(PKV_ERR_INVALID, "batch in [1, 4096], q_len and table_stride positive, "
                                     "max_pos >= 0");
    if (!q || !k_pool || !v_pool || !block_tables || !pos || !out)
        return fail(PKV_ERR_INVALID, "null device pointer");
    const int G = p->num_heads / p->num_kv_heads;
    if (!stream_eligible(p, G))
        return fail(PKV_ERR_UNSUPPORTED, "pkv_attend_noalloc: head_dim 256 or 512 with "
                                         "num_heads / num_kv_heads <= 8");
    // Workgroups along the keys the scratch holds partials for: the largest cap whose
    // layout (the plan, then (m, l) and o[D] in double per (slot, row), slots = cap +
    // batch) fits. The layout grows by per_slot bytes (plus alignment) per slot.
    const size_t rows = (size_t)p->num_heads * q_len;
    const size_t per_slot = rows * (2 + (size_t)p->head_dim) * sizeof(double);
    const size_t base = stream_layout(p, batch, q_len, 0).total;  // batch slots, no cap
    int32_t cap = base < kScratchBytes
                      ? (int32_t)std::min<size_t>((kScratchBytes - base) / per_slot, kStreamMaxSlots)
                      : 0;
    while (cap > 0 && stream_layout(p, batch, q_len, cap).total > kScratchBytes) --cap;
    if (cap < 1)
        return fail(PKV_ERR_WORKSPACE, "pkv_attend_noalloc: the call's split-K partials exceed "
                                       "the 64 MiB scratch (use pkv_attend with a workspace)");
    void* ws = nullptr;
    rc = scratch_address(&ws);
    if (rc != PKV_OK) return rc;
    rc = stream_attend(p, q, k_pool, v_pool, block_tables, table_stride, pos, 0, 0, q_len,
                       nullptr, batch, max_pos, nullptr, nullptr, 0, out, ws,
                       static_cast<hipStream_t>(stream), nullptr, cap);
    if (rc != PKV_OK) return rc;
    return check_launch("pkv_attend_noalloc");
}

}  // extern "C"
