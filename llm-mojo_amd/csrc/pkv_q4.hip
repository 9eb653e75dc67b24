// Wo projection after attention: batched Q4_0 matrix-vector products with bf16 MFMA.
//
// Replaces q4_matmul_vec (moe_kernels.mojo:59-163) as the engine calls it on attn_out
// (model_speculative_moe_batched.mojo:2011-2051): out[s][r] = sum_k W[r][k] * x[s][k] for
// every sequence s of the batch, W in Q4_0 block-32 form (moe_kernels.mojo:7-57): per row
// and block of 32 inputs a fp32 scale and 16 bytes, byte j holding element 2j in its low
// nibble and 2j + 1 in its high one, value (nibble - 8) * scale.
//
// At decode batches this is a skinny GEMM (M = c_out rows, N = batch, K = c_in) whose
// weights are read once, so it is HBM-bound on the weights; fp32 FMAs on the vector units
// would take several times the weight-read time, so it runs on the matrix cores:
//   - one v_mfma_f32_16x16x32_bf16 covers exactly one Q4 block: A = 16 rows x 32 weights
//     (nibble - 8 is exact in bf16), B = 32 inputs x 16 sequences;
//   - x is split into three bf16 parts (hi + mid + lo = x exactly: 3 x 8 bits cover fp32's
//     24-bit significand), so every product is exact and only fp32 accumulation rounds;
//   - the block's fp32 partial is scaled and accumulated in fp32.
// Work split: a workgroup owns 128 rows and a split of KB blocks of K. It stages its
// fp32 x slice in LDS once, in B-operand order; its 8 waves are 2 row halves x 4 K
// quarters, so each wave takes 64 rows (4 A tiles) over KB / 4 blocks and a B operand,
// read from LDS and split into parts in registers, feeds 4 A tiles. The K quarters are
// summed through LDS in a fixed order, (q0 + q1) + (q2 + q3), and the workgroup writes
// its split's partial; q4_reduce_kernel adds the splits in order (deterministic). A
// single split writes out directly. Workgroups of one split are placed on one XCD
// (dispatch is round-robin over the 8 XCDs), so each XCD's L2 holds one slice of x.
//
// MFMA lane layouts (v_mfma_f32_16x16x32_bf16):
//   A[i][k]: lane i + 16*(k/8), element k%8;   B[k][j]: lane j + 16*(k/8), element k%8;
//   C[i][j]: lane j + 16*(i/4), register i%4.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pkv_internal.h"

namespace pkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kQ4WR = 2;                       // row halves per workgroup
constexpr int kQ4WK = 4;                       // K quarters per workgroup
constexpr int kQ4Waves = kQ4WR * kQ4WK;
constexpr int kQ4ATiles = 4;                   // 16-row A tiles per wave
constexpr int kQ4Rows = kQ4WR * kQ4ATiles * 16;  // output rows per workgroup
constexpr int kQ4KB = 8;                       // Q4 blocks per split
constexpr int kQ4MaxBatch = 64;                // four column tiles of 16
constexpr int kQ4Parts = 3;                    // bf16 parts of each input

struct Q4Args {
    const uint8_t* w;     // [c_out][c_in / 2]
    const float* scales;  // [c_out][c_in / 32]
    const float* x;       // [batch][c_in]
    float* out;           // [batch][c_out]
    float* part;          // [splits][batch][c_out] (splits > 1)
    int32_t c_in;
    int32_t c_out;
    int32_t batch;
    int32_t nb;      // blocks per row
    int32_t groups;  // row groups of kQ4Rows
    int32_t splits;
};


__device__ inline bf16x8 as_bf16x8(uint4 v) {
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// 8 weights (nibbles of w, low first) minus 8, as bf16 bits: small integers, exact.
__device__ inline bf16x8 weights_bf16(uint32_t w) {
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float a = (float)((int)((w >> (8 * e)) & 15u) - 8);
        const float b = (float)((int)((w >> (8 * e + 4)) & 15u) - 8);
        h[e] = (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
    }
    return as_bf16x8(make_uint4(h[0], h[1], h[2], h[3]));
}

// TILES = column tiles of 16 sequences, KB = blocks per split; both compile-time, so the
// whole body is one basic block: every MFMA result is read by VALU code in the MFMA's own
// block. (With a runtime tile count a chain ended in a branch and the first register of
// its result was read in the target block without the MFMA's wait states: a wrong,
// varying value in every fourth row.)
// Up to two column tiles the kernel fits 80 VGPRs, which keeps three workgroups per CU
// resident (six waves per SIMD): the 704 workgroups of an 8192 -> 2816 call then run in
// one round instead of two.
template <int TILES, int KB>
__global__ __launch_bounds__(kQ4Waves * 64, TILES <= 2 ? 6 : 1) void q4_matmul_kernel(Q4Args a) {
    constexpr int NT = kQ4Waves * 64;
    constexpr int BPW = KB / kQ4WK;  // blocks per wave
    // x slice in B-operand order: slot ((ct * KB + b) * 2 + h) * 64 + lane holds inputs
    // 8 (lane >> 4) + 4h .. +3 of block b of sequence 16 ct + (lane & 15), so a wave's
    // operand read is 64 consecutive 16-byte slots. Reused for the K-quarter sums.
    constexpr int kSlots = TILES * KB * 2 * 64;
    constexpr int kRed = kQ4WR * 2 * kQ4ATiles * TILES * 64;  // f32x4 per pair of quarters
    static_assert(kRed * 16 <= kSlots * 16, "quarter sums fit the x slice");
    __shared__ uint4 s_x[kSlots];
    __shared__ uint4 s_w[kQ4Rows * KB];                                  // weights, see below
    __shared__ __attribute__((aligned(16))) float s_sc[KB][kQ4Rows];     // scales [block][row]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave / kQ4WK, wk = wave % kQ4WK;
    const int g = lane >> 4;

    // Work item: workgroups of one split are consecutive within an XCD.
    int q = blockIdx.x;
    const int total = a.groups * a.splits;
    if (total % 8 == 0) q = (q % 8) * (total / 8) + q / 8;
    const int split = q / a.groups;
    const int grow0 = (q % a.groups) * kQ4Rows;  // the workgroup's first row
    const int row0 = grow0 + wr * kQ4ATiles * 16;  // this wave's first row
    const int kb0 = wk * BPW;                      // this wave's first block in the split
    const int blk0 = split * KB;

    // Requests first: x staging, weights (straight to LDS), scales.
    constexpr int kStage = TILES * 16 * KB * 8 / NT;  // float4 per thread
    static_assert(kStage * NT == TILES * 16 * KB * 8, "whole float4 per thread");
    float4 xs[kStage];
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
        const int e = tid + i * NT;
        const int m = e & 7, col = (e >> 3) % (TILES * 16), b = (e >> 3) / (TILES * 16);
        xs[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (col < a.batch && blk0 + b < a.nb)
            xs[i] = *reinterpret_cast<const float4*>(a.x + (size_t)col * a.c_in + (size_t)(blk0 + b) * 32 + 4 * m);
    }
    // Weights: the workgroup's rows x KB blocks (each row's KB * 16 contiguous bytes) go
    // straight into LDS, 16 bytes per lane; row r's block b sits at position b ^ (r % 8)
    // of its LDS row, so the 4-byte A-operand reads of 16 rows spread over the banks. Rows
    // and blocks outside the matrix load a valid chunk and are replaced by zero weights
    // when read.
    constexpr int kWChunks = kQ4Rows * KB / (kQ4Waves * 64);  // DMA instructions per wave
    static_assert(kWChunks * kQ4Waves * 64 == kQ4Rows * KB && KB == 8, "whole chunks per wave");
#pragma unroll
    for (int j = 0; j < kWChunks; ++j) {
        const int pos = (wave * kWChunks + j) * 64 + lane;
        const int r = pos / KB, b = (pos % KB) ^ (r & 7);
        const bool in = grow0 + r < a.c_out && blk0 + b < a.nb;
        const uint8_t* src = in ? a.w + (size_t)(grow0 + r) * (a.c_in / 2) + (size_t)(blk0 + b) * 16 : a.w;
        __builtin_amdgcn_global_load_lds(src, (lds_void*)(s_w + (wave * kWChunks + j) * 64), 16, 0, 0);
    }
    // Scales: eight lanes read a row's KB consecutive scales; stored [block][row].
    constexpr int kScPer = kQ4Rows * KB / NT;
    float sc[kScPer];
#pragma unroll
    for (int i = 0; i < kScPer; ++i) {
        const int e = tid + i * NT, r = e / KB, b = e % KB;
        sc[i] = (grow0 + r < a.c_out && blk0 + b < a.nb) ? a.scales[(size_t)(grow0 + r) * a.nb + blk0 + b] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
        const int e = tid + i * NT;
        const int m = e & 7, col = (e >> 3) % (TILES * 16), b = (e >> 3) / (TILES * 16);
        const int ct = col >> 4, l = (col & 15) + 16 * (m >> 1), h = m & 1;
        s_x[((ct * KB + b) * 2 + h) * 64 + l] = *reinterpret_cast<const uint4*>(&xs[i]);
    }
#pragma unroll
    for (int i = 0; i < kScPer; ++i) {
        const int e = tid + i * NT;
        s_sc[e % KB][e / KB] = sc[i];
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's weight chunks have landed
    __syncthreads();
    uint32_t wv[kQ4ATiles][BPW];
#pragma unroll
    for (int t = 0; t < kQ4ATiles; ++t) {
        const int r = wr * kQ4ATiles * 16 + 16 * t + (lane & 15);  // row in the workgroup
#pragma unroll
        for (int bb = 0; bb < BPW; ++bb) {
            const int b = kb0 + bb;
            const uint32_t v = reinterpret_cast<const uint32_t*>(s_w)[(r * KB + (b ^ (r & 7))) * 4 + g];
            // zeros after the offset outside the matrix
            wv[t][bb] = (grow0 + r < a.c_out && blk0 + b < a.nb) ? v : 0x88888888u;
        }
    }

    f32x4 acc[kQ4ATiles][TILES];
#pragma unroll
    for (int t = 0; t < kQ4ATiles; ++t)
#pragma unroll
        for (int ct = 0; ct < TILES; ++ct) acc[t][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int bb = 0; bb < BPW; ++bb) {
        bf16x8 B[TILES][kQ4Parts];  // peel one bf16 part at a time; each residual is exact
#pragma unroll
        for (int ct = 0; ct < TILES; ++ct) {
            const uint4 u0 = s_x[((ct * KB + kb0 + bb) * 2 + 0) * 64 + lane];
            const uint4 u1 = s_x[((ct * KB + kb0 + bb) * 2 + 1) * 64 + lane];
            float r[8] = {__uint_as_float(u0.x), __uint_as_float(u0.y), __uint_as_float(u0.z),
                          __uint_as_float(u0.w), __uint_as_float(u1.x), __uint_as_float(u1.y),
                          __uint_as_float(u1.z), __uint_as_float(u1.w)};
#pragma unroll
            for (int p = 0; p < kQ4Parts; ++p) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    B[ct][p][e] = (__bf16)r[e];
                    r[e] -= (float)B[ct][p][e];
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kQ4ATiles; ++t) {
            const bf16x8 A = weights_bf16(wv[t][bb]);
            const f32x4 s4 =
                *reinterpret_cast<const f32x4*>(&s_sc[kb0 + bb][wr * kQ4ATiles * 16 + 16 * t + 4 * g]);
#pragma unroll
            for (int ct = 0; ct < TILES; ++ct) {
                f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int p = kQ4Parts - 1; p >= 0; --p)  // smallest part first
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B[ct][p], c, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[t][ct][r] = fmaf(s4[r], c[r], acc[t][ct][r]);
            }
        }
    }

    // Quarter sums: pair slot (wr, wk >> 1); odd quarters write, even ones add and store
    // back, then every thread adds the two pair sums of its outputs.
    f32x4* red = reinterpret_cast<f32x4*>(s_x);
    auto rslot = [&](int pair, int t, int ct) -> f32x4& {
        return red[(((wr * 2 + pair) * kQ4ATiles + t) * TILES + ct) * 64 + lane];
    };
    // Pin the last scaled accumulations here, in the MFMAs' basic block: left free, the
    // compiler may sink them past the branches below.
#pragma unroll
    for (int t = 0; t < kQ4ATiles; ++t)
#pragma unroll
        for (int ct = 0; ct < TILES; ++ct)
#pragma unroll
            for (int r = 0; r < 4; ++r) asm volatile("" : "+v"(acc[t][ct][r]));
    __syncthreads();  // every wave is done with the x slice
    if (wk & 1) {
#pragma unroll
        for (int t = 0; t < kQ4ATiles; ++t)
#pragma unroll
            for (int ct = 0; ct < TILES; ++ct) rslot(wk >> 1, t, ct) = acc[t][ct];
    }
    __syncthreads();
    if (!(wk & 1)) {
#pragma unroll
        for (int t = 0; t < kQ4ATiles; ++t)
#pragma unroll
            for (int ct = 0; ct < TILES; ++ct) {
                f32x4& r = rslot(wk >> 1, t, ct);
                r = acc[t][ct] + r;
            }
    }
    __syncthreads();

    // Consecutive threads take consecutive rows of one sequence.
    const float* redf = reinterpret_cast<const float*>(red);
    constexpr int kPairFloats = kQ4ATiles * TILES * 64 * 4;
#pragma unroll
    for (int i = 0; i < kQ4Rows * 16 * TILES / NT; ++i) {
        const int e = tid + i * NT;
        const int row = e % kQ4Rows, col = e / kQ4Rows;
        const int h = row / (kQ4ATiles * 16), rw = row % (kQ4ATiles * 16);
        const int t = rw >> 4, rg = (rw >> 2) & 3, r = rw & 3;
        const int l = (col & 15) + 16 * rg, ct = col >> 4;
        const int idx = (h * 2 * kPairFloats) + ((t * TILES + ct) * 64 + l) * 4 + r;
        const float sum = redf[idx] + redf[idx + kPairFloats];
        if (col < a.batch && grow0 + row < a.c_out) {
            if (a.splits == 1) a.out[(size_t)col * a.c_out + grow0 + row] = sum;
            else a.part[((size_t)split * a.batch + col) * a.c_out + grow0 + row] = sum;
        }
    }
}

// out[col][row] = sum over splits in order of the partials (loads 16 splits at a time).
__global__ __launch_bounds__(256) void q4_reduce_kernel(Q4Args a) {
    const size_t n = (size_t)a.batch * a.c_out;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        float sum = 0.f;
        for (int s0 = 0; s0 < a.splits; s0 += 16) {
            float v[16];
#pragma unroll
            for (int s = 0; s < 16; ++s) v[s] = s0 + s < a.splits ? a.part[(size_t)(s0 + s) * n + i] : 0.f;
#pragma unroll
            for (int s = 0; s < 16; ++s) sum += v[s];
        }
        a.out[i] = sum;
    }
}

// Splits of kQ4KB blocks. Eight blocks keep a workgroup at <= 68 KiB of LDS (two per CU)
// and give the Wo shapes >= 352 workgroups; sixteen measured slower (fewer, LDS-bound
// workgroups) despite half the partials.
int32_t q4_splits(int32_t c_in) { return (c_in / 32 + kQ4KB - 1) / kQ4KB; }

}  // namespace
}  // namespace pkv

extern "C" {

size_t pkv_q4_matmul_workspace_size(int32_t c_in, int32_t c_out, int32_t batch) {
    if (c_in <= 0 || c_in % 32 || c_out <= 0 || batch <= 0 || batch > pkv::kQ4MaxBatch) return 0;
    const int32_t splits = pkv::q4_splits(c_in);
    const size_t bytes = splits > 1 ? (size_t)splits * batch * c_out * sizeof(float) : 0;
    return bytes > 0 ? bytes : 256;
}

int32_t pkv_q4_matmul(void* stream, const uint8_t* w_packed, const float* scales, const float* x,
                      int32_t c_in, int32_t c_out, int32_t batch, float* out, void* workspace,
                      size_t workspace_bytes) {
    using namespace pkv;
    clear_error();
    if (c_in <= 0 || c_in % 32 != 0)
        return fail(PKV_ERR_INVALID, "pkv_q4_matmul: c_in must be a positive multiple of 32");
    if (c_out <= 0 || batch <= 0)
        return fail(PKV_ERR_INVALID, "pkv_q4_matmul: c_out and batch must be positive");
    if (batch > kQ4MaxBatch) return fail(PKV_ERR_UNSUPPORTED, "pkv_q4_matmul: batch must be <= 64");
    if (!w_packed || !scales || !x || !out || !workspace)
        return fail(PKV_ERR_INVALID, "pkv_q4_matmul: null device pointer");
    if ((reinterpret_cast<uintptr_t>(w_packed) & 15) || (reinterpret_cast<uintptr_t>(x) & 15) ||
        (reinterpret_cast<uintptr_t>(scales) & 3))
        return fail(PKV_ERR_INVALID, "pkv_q4_matmul: w_packed and x need 16-byte, scales 4-byte alignment");
    if (workspace_bytes < pkv_q4_matmul_workspace_size(c_in, c_out, batch))
        return fail(PKV_ERR_WORKSPACE, "workspace smaller than pkv_q4_matmul_workspace_size()");
    Q4Args a{};
    a.w = w_packed;
    a.scales = scales;
    a.x = x;
    a.out = out;
    a.part = static_cast<float*>(workspace);
    a.c_in = c_in;
    a.c_out = c_out;
    a.batch = batch;
    a.nb = c_in / 32;
    a.groups = (c_out + kQ4Rows - 1) / kQ4Rows;
    a.splits = q4_splits(c_in);
    const int tiles = (batch + 15) / 16;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(a.groups * a.splits), block(kQ4Waves * 64);
    switch (tiles) {
        case 1: hipLaunchKernelGGL((q4_matmul_kernel<1, kQ4KB>), grid, block, 0, st, a); break;
        case 2: hipLaunchKernelGGL((q4_matmul_kernel<2, kQ4KB>), grid, block, 0, st, a); break;
        case 3: hipLaunchKernelGGL((q4_matmul_kernel<3, kQ4KB>), grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL((q4_matmul_kernel<4, kQ4KB>), grid, block, 0, st, a); break;
    }
    if (a.splits > 1) {
        const size_t n = (size_t)batch * c_out;
        const int blocks = (int)((n + 255) / 256 < 2048 ? (n + 255) / 256 : 2048);
        hipLaunchKernelGGL(q4_reduce_kernel, dim3(blocks), dim3(256), 0, st, a);
    }
    return check_launch("pkv_q4_matmul");
}

}  // extern "C"
