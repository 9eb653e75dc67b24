// Synthetic-data generator for the benchmark and test workloads (libpkv_synth.so).
// Not part of the paged-KV ABI: it fills device buffers with seeded N(0, 1) values so
// that multi-GB pools are generated in milliseconds instead of minutes on the host.
//
// Value i of stream `seed` is a Box-Muller normal built from a counter hash:
//   h = splitmix64(seed * 0x9E3779B97F4A7C15 + i), u1 = (top 24 bits + 1) / 2^24 in (0, 1],
//   u2 = next 24 bits / 2^24, z = sqrt(-2 ln u1) * cos(2 pi u2), computed in double and
//   rounded once to fp32 (or further to bf16, round-to-nearest-even).
// The result depends only on (seed, i), so any slice can be regenerated independently.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__device__ inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

__device__ inline float normal_at(uint64_t seed, uint64_t i) {
    uint64_t h = splitmix64(seed * 0x9E3779B97F4A7C15ULL + i);
    double u1 = (double)((h >> 40) + 1) * (1.0 / 16777216.0);
    double u2 = (double)((h >> 16) & 0xFFFFFFULL) * (1.0 / 16777216.0);
    return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

__device__ inline uint16_t to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__global__ void fill_normal_f32(float* dst, uint64_t n, uint64_t seed, uint64_t offset) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = normal_at(seed, offset + i);
}

__global__ void fill_normal_bf16(uint16_t* dst, uint64_t n, uint64_t seed, uint64_t offset) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = to_bf16_rne(normal_at(seed, offset + i));
}

}  // namespace

extern "C" {

// Fills dst[0..n) with values offset .. offset+n-1 of normal stream `seed`.
// dtype 0 = fp32, 1 = bf16 (bits). Returns 0 or the HIP error code.
int32_t pkv_synth_normal(void* stream, void* dst, uint64_t n, uint64_t seed, uint64_t offset,
                         int32_t dtype) {
    if (!dst || n == 0) return 0;
    const unsigned threads = 256;
    uint64_t want = (n + threads - 1) / threads;
    unsigned blocks = (unsigned)(want < 65536 ? want : 65536);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (dtype == 1)
        hipLaunchKernelGGL(fill_normal_bf16, dim3(blocks), dim3(threads), 0, st,
                           static_cast<uint16_t*>(dst), n, seed, offset);
    else
        hipLaunchKernelGGL(fill_normal_f32, dim3(blocks), dim3(threads), 0, st,
                           static_cast<float*>(dst), n, seed, offset);
    return (int32_t)hipGetLastError();
}

}  // extern "C"
