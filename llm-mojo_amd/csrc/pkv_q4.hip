// Wo projection after attention: batched Q4_0 matrix-vector products with bf16 MFMA.
//
// Replaces q4_matmul_vec (moe_kernels.mojo:59-163) as the engine calls it on attn_out
// (model_speculative_moe_batched.mojo:2011-2051): out[s][r] = sum_k W[r][k] * x[s][k] for
// every sequence s of the batch, W in Q4_0 block-32 form (moe_kernels.mojo:7-57): per row
// and block of 32 inputs a fp32 scale and 16 bytes, byte j holding element 2j in its low
// nibble and 2j + 1 in its high one, value (nibble - 8) * scale.
//
// At decode batches this is a skinny GEMM (M = c_out rows, N = batch, K = c_in) whose
// weights are read once, so it is HBM-bound on the weights; it runs on the matrix cores:
//   - one v_mfma_f32_16x16x32_bf16 covers exactly one Q4 block: A = 32 inputs of 16
//     sequences, B = 16 rows x 32 weights (nibble - 8 is exact in bf16);
//   - x is split into three bf16 parts (hi + mid + lo = x exactly: each part takes the
//     next 8 significant bits of the 24-bit fp32 significand), so every product is exact
//     and only the fp32 accumulation rounds;
//   - the block's fp32 sum is scaled by the row's block scale and accumulated in fp32.
//
// Work split: row groups of 64 rows, each split into `splits` runs of `per` consecutive
// blocks, one workgroup per run, as many runs as keep every workgroup resident (two
// 8-wave workgroups per CU). Per workgroup:
//   - its rows' weights and scales go straight into LDS (global_load_lds over
//     consecutive memory: a row's blocks are contiguous, so whole cache lines are read),
//     in passes of 8 blocks that are computed as they land;
//   - the eight waves take the blocks in turn (wave v: blocks v, v + 8, ...); a wave
//     splits the inputs of its block into three exact bf16 operands once and feeds them
//     to every row tile of the group;
//   - the waves' sums are added through LDS in a fixed order. With one run per group the
//     workgroup writes out directly. Otherwise it writes its partial sums and counts
//     itself in the group's arrival counter; the last to arrive adds the group's
//     partials in run order (deterministic) and writes out. The partials are written and
//     read at system scope (through and past the L2 caches), so no cache write-back or
//     invalidation is needed; device-scope fences here cost more than the whole product
//     on this 8-XCD part.
//
// MFMA lane layouts (v_mfma_f32_16x16x32_bf16):
//   A[i][k]: lane i + 16*(k/8), element k%8;   B[k][j]: lane j + 16*(k/8), element k%8;
//   C[i][j]: lane j + 16*(i/4), register i%4.
// A block's element e of quarter g (K index 8g + e) is nibble e of dword g of the block
// (byte 4g + e/2, low nibble for even e), so both operands use the block's own K order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pkv_internal.h"

namespace pkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kQ4Waves = 8;               // waves per workgroup (blocks taken in turn)
constexpr int kQ4NT = kQ4Waves * 64;
constexpr int kQ4MaxBatch = 64;           // four column tiles of 16
constexpr int kQ4MaxWg = 1024;            // workgroups, at most

struct Q4Args {
    const uint8_t* w;     // [c_out][c_in / 2]
    const float* scales;  // [c_out][c_in / 32]
    const float* x;       // [batch][c_in]
    float* out;           // [batch][c_out]
    float* part;          // [workgroups][rows of a group][16 TILES sequence slots] (split groups)
    int32_t* arrived;     // [groups]: workgroups of the row group done (zero between calls)
    int32_t c_in;
    int32_t c_out;
    int32_t batch;
    int32_t nb;      // blocks per row
    int32_t groups;  // row groups
    int32_t splits;  // workgroups per row group (each takes `per` consecutive blocks)
    int32_t per;
};

__device__ inline bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint4 v = make_uint4(a, b, c, d);
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

// The upper halves of two fp32 words as one bf16 pair (lo first).
__device__ inline uint32_t hi_pair(uint32_t lo, uint32_t hi) {
    return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
}

// 8 weights of one dword (element e = nibble e, value nibble - 8) as bf16 values of
// (nibble - 8) / 16, exactly. v_cvt_off_f32_i4 converts bits [3:0] of its operand, read
// as a signed 4-bit integer, to that integer / 16; with SDWA it reads one byte, so the
// low nibbles come from the bytes of w ^ 0x88888888 (nibble ^ 8 as a signed 4-bit field
// is nibble - 8) and the high ones from the same word shifted right by 4. The 1/16 is
// folded into the block scale (a power of two: the scaled sums round as before).
template <int BYTE>
__device__ inline float cvt_off_byte(uint32_t v) {
    float r;
    if constexpr (BYTE == 0)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(v));
    else if constexpr (BYTE == 1)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(v));
    else if constexpr (BYTE == 2)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(v));
    else
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(v));
    return r;
}
__device__ inline bf16x8 unpack_q4(uint32_t w) {
    const uint32_t lo = w ^ 0x88888888u, hi = lo >> 4;
    return as_bf16x8(hi_pair(__float_as_uint(cvt_off_byte<0>(lo)), __float_as_uint(cvt_off_byte<0>(hi))),
                     hi_pair(__float_as_uint(cvt_off_byte<1>(lo)), __float_as_uint(cvt_off_byte<1>(hi))),
                     hi_pair(__float_as_uint(cvt_off_byte<2>(lo)), __float_as_uint(cvt_off_byte<2>(hi))),
                     hi_pair(__float_as_uint(cvt_off_byte<3>(lo)), __float_as_uint(cvt_off_byte<3>(hi))));
}
constexpr float kQ4Unpack = 16.0f;  // unpack_q4 gives (nibble - 8) / 16

// x = hi + mid + lo exactly: hi is x truncated to bf16; the remainder (at most 16
// significant bits) is exact in fp32 and is truncated again; the last remainder has at
// most 8 significant bits and is a bf16 value.
__device__ inline void split3(const float (&v)[8], bf16x8& hi, bf16x8& mid, bf16x8& lo) {
    uint32_t h[4], m[4], l[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t u[2], r[2], s[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            u[e] = __float_as_uint(v[2 * k + e]);
            const float r1 = v[2 * k + e] - __uint_as_float(u[e] & 0xffff0000u);
            r[e] = __float_as_uint(r1);
            s[e] = __float_as_uint(r1 - __uint_as_float(r[e] & 0xffff0000u));
        }
        h[k] = hi_pair(u[0], u[1]);
        m[k] = hi_pair(r[0], r[1]);
        l[k] = hi_pair(s[0], s[1]);
    }
    hi = as_bf16x8(h[0], h[1], h[2], h[3]);
    mid = as_bf16x8(m[0], m[1], m[2], m[3]);
    lo = as_bf16x8(l[0], l[1], l[2], l[3]);
}

typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_barrier without the fence of __syncthreads (which waits for every load in flight).
__device__ inline void pass_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

constexpr int kQ4Lds = 128 * 1024;
constexpr int kQ4MaxPass = 3;  // passes of 8 blocks staged at once (one block per wave each)

// One LDS dword read the compiler does not track: it would otherwise wait for every
// direct-to-LDS copy in flight (vmcnt 0) before it, since it cannot tell which LDS words
// a copy writes. The caller waits (lgkmcnt) before using the value (read_tile).
// base: an LDS byte address; OFF: a constant byte offset (< 65536).
template <int OFF>
__device__ inline uint32_t lds_read_u32(uint32_t base) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(base), "i"(OFF));
    return v;
}
__device__ inline uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const lds_void*)p;
}

// The inputs of one block for this wave's column tiles: per column tile, 8 of one sequence
// per lane (lane j + 16q: sequence 16ct + j, inputs 32b + 8q .. + 7). The sequence is
// clamped into the batch, so both loads are always issued: those of a sequence past the
// batch only reach outputs that are not stored.
template <int TILES>
struct XPass {
    f32x4 v[TILES][2];
};
template <int TILES>
__device__ inline XPass<TILES> load_x(const Q4Args& a, int b, int j, int lane) {
    XPass<TILES> r;
#pragma unroll
    for (int ct = 0; ct < TILES; ++ct) {
        const int seq = min(16 * ct + j, a.batch - 1);
        const f32x4* xp = reinterpret_cast<const f32x4*>(a.x + (size_t)seq * a.c_in + 32 * b + 8 * (lane >> 4));
        r.v[ct][0] = xp[0];
        r.v[ct][1] = xp[1];
    }
    return r;
}

// Pass i's weights ([row][8 blocks] 16-byte chunks; a row's blocks are contiguous in
// memory, so whole cache lines are read) and scales ([row][8 blocks]) straight into LDS:
// RH copy instructions of each kind per wave. Block bb of row r sits at chunk
// r * 8 + (bb ^ (r & 7)), so the 16 rows of a weight read fall on different banks. Rows
// past c_out read the last row and blocks past the run read the pass's first block (the
// run's last, for a pass wholly past the run); none of them is used.
template <int RH, int PASS_W, int PASS_S>
__device__ inline void copy_pass(const Q4Args& a, char* smem, int g, int c_lo, int b_hi, int v,
                                 int lane, int i) {
    constexpr int RG = 64 * RH;
    const int p0 = c_lo + 8 * i, pn = min(8, b_hi - p0), pf = min(p0, b_hi - 1);
    char* s_w = smem + i * (PASS_W + PASS_S);
    char* s_s = s_w + PASS_W;
#pragma unroll
    for (int n = 0; n < RH; ++n) {
        const int k = v + kQ4Waves * n;  // copy instruction of this pass
        const int e = 64 * k + lane, r = e >> 3, bb = (e & 7) ^ (r & 7);
        const int row = min(g * RG + r, a.c_out - 1);
        __builtin_amdgcn_global_load_lds(
            a.w + (size_t)row * (a.c_in / 2) + (size_t)(bb < pn ? p0 + bb : pf) * 16,
            (lds_void*)(s_w + 1024 * k), 16, 0, 0);
    }
#pragma unroll
    for (int n = 0; n < RH; ++n) {
        const int k = v + kQ4Waves * n;
        const int e = 64 * k + lane, r = e >> 3, bb = e & 7;
        const int row = min(g * RG + r, a.c_out - 1);
        __builtin_amdgcn_global_load_lds(a.scales + (size_t)row * a.nb + (bb < pn ? p0 + bb : pf),
                                         (lds_void*)(s_s + 256 * k), 4, 0, 0);
    }
}

// Row tile T's weight dword and block scale in pass I (row r = 16T + j of the group:
// weights at pass + ((r 8 + (v ^ (r & 7))) 4 + lane / 16) 4, the scale at
// pass + PASS_W + (r 8 + v) 4, i.e. the lane's base plus a constant), both complete on
// return: the values are tied to the lgkmcnt wait, so no use can be scheduled above it.
template <int I, int T, int PASS, int PASS_W>
__device__ inline void read_tile(uint32_t w_base, uint32_t s_base, uint32_t& wd, uint32_t& sc) {
    wd = lds_read_u32<I * PASS + T * 2048>(w_base);
    sc = lds_read_u32<I * PASS + PASS_W + T * 512>(s_base);
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(wd), "+v"(sc));
}

// One block of pass I: the wave splits its inputs into three exact bf16 operands once and
// feeds them to every row tile of the group.
template <int I, int TILES, int RT, int PASS, int PASS_W>
__device__ inline void compute_pass(const XPass<TILES>& xr, uint32_t w_base, uint32_t s_base,
                                    f32x4 (&acc)[RT][TILES]) {
    static_assert(RT == 4, "row tiles of a 64-row group");
    bf16x8 X[TILES][3];
#pragma unroll
    for (int ct = 0; ct < TILES; ++ct) {
        const float xv[8] = {xr.v[ct][0].x, xr.v[ct][0].y, xr.v[ct][0].z, xr.v[ct][0].w,
                             xr.v[ct][1].x, xr.v[ct][1].y, xr.v[ct][1].z, xr.v[ct][1].w};
        split3(xv, X[ct][0], X[ct][1], X[ct][2]);
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        uint32_t wd, scb;
        if (t == 0) read_tile<I, 0, PASS, PASS_W>(w_base, s_base, wd, scb);
        else if (t == 1) read_tile<I, 1, PASS, PASS_W>(w_base, s_base, wd, scb);
        else if (t == 2) read_tile<I, 2, PASS, PASS_W>(w_base, s_base, wd, scb);
        else read_tile<I, 3, PASS, PASS_W>(w_base, s_base, wd, scb);
        const float sc = __uint_as_float(scb) * kQ4Unpack;
        const bf16x8 W = unpack_q4(wd);
#pragma unroll
        for (int ct = 0; ct < TILES; ++ct) {
            f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(X[ct][2], W, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(X[ct][1], W, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(X[ct][0], W, c, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[t][ct][e] = fmaf(sc, c[e], acc[t][ct][e]);
        }
    }
}

// 16 bytes stored and loaded at system scope (written through, read past the L2 caches).
// The loads are not tracked by the compiler; wait_loads completes them (the values are
// tied to the wait, so no use can be scheduled above it).
__device__ inline void store16_system(float* p, f32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ inline f32x4 load16_system(const float* p) {
    f32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off sc0 sc1" : "=v"(v) : "v"(p) : "memory");
    return v;
}
constexpr int kQ4RedLoads = 12;  // partials requested at once per thread (the 11 splits of the engine shapes: one round trip)
__device__ inline void wait_loads(f32x4 (&v)[kQ4RedLoads]) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < kQ4RedLoads; ++i) asm volatile("" : "+v"(v[i]));
}

// TILES column tiles of 16 sequences; RH row halves of 64 rows (row group = 64 RH rows);
// PASSES passes of 8 blocks per chunk. All three are compile-time, so every MFMA result is
// read in the MFMA's own basic block (with a runtime count a chain could end in a branch
// whose target read the first result register without the MFMA's wait states), and every
// chunk issues the same loads (exact vmcnt waits).
//
// Workgroup = (row group g, split k): blocks [k per, (k + 1) per) of the group's rows.
// Operand roles: A = the inputs (16 sequences x 32), B = the weights (32 x 16 rows), so
// C[seq][row] puts one row in each lane (lane j + 16q: row j of the tile, sequences
// 4q .. 4q + 3) and each lane scales its four sums by one block scale.
// Staging, per chunk: each pass's inputs (registers, block v of the pass for wave v) and
// weights and scales (LDS, copied by the whole workgroup) are requested up front, and pass
// i is computed as soon as its own loads have landed, the later passes' still streaming in.
template <int TILES, int RH, int PASSES>
__global__ __launch_bounds__(kQ4NT) __attribute__((amdgpu_waves_per_eu(RH == 1 && TILES <= 2 ? 4 : 2)))
void q4_matmul_kernel(Q4Args a) {
    static_assert(PASSES >= 1 && PASSES <= kQ4MaxPass, "passes");
    constexpr int RT = 4 * RH;        // row tiles of the group
    constexpr int RG = 64 * RH;       // rows of the group
    constexpr int kPassW = RG * 8 * 16;  // bytes of weights per pass
    constexpr int kPassS = RG * 8 * 4;   // bytes of scales per pass
    constexpr int kXLoads = 2 * TILES;  // input load instructions per wave and pass
    static_assert(kXLoads + 4 * RH < 64, "vmcnt");
    constexpr int kLds = kQ4Waves * RT * TILES * 64 * 16 > kQ4MaxPass * (kPassW + kPassS)
                             ? kQ4Waves * RT * TILES * 64 * 16 : kQ4MaxPass * (kPassW + kPassS);
    static_assert(kLds <= kQ4Lds, "LDS");
    static_assert(kPassW / 1024 == kQ4Waves * RH && kPassS / 256 == kQ4Waves * RH,
                  "RH copy instructions of each kind per wave and pass");
    __shared__ __attribute__((aligned(16))) char smem[kLds];
    f32x4* s_red = reinterpret_cast<f32x4*>(smem);  // [wave][RT][TILES][64], after the passes
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int v = tid >> 6;
    const int j = lane & 15;
    const int g = blockIdx.x / a.splits;
    const int b_lo = (blockIdx.x % a.splits) * a.per;
    const int b_hi = min(a.nb, b_lo + a.per);

    f32x4 acc[RT][TILES];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int ct = 0; ct < TILES; ++ct) acc[t][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t w_base = lds_addr(smem) + ((j * 8 + (v ^ (j & 7))) * 4 + (lane >> 4)) * 4;
    const uint32_t s_base = lds_addr(smem) + (j * 8 + v) * 4;
    for (int c_lo = b_lo; c_lo < b_hi; c_lo += 8 * PASSES) {
        // 1. Loads, in this issue order: inputs of pass 0, weights and scales of pass 0,
        // inputs of pass 1, weights and scales of passes 1 and 2; the inputs of pass 2
        // follow once pass 0 is computed (in the registers pass 0 frees). Every chunk
        // issues all PASSES passes (a pass past the run reads in-range blocks it does not
        // use), so no branch separates a load from its use and each wait below counts
        // exactly the instructions issued after the pass it waits for. Compiler barriers
        // keep the groups in this order.
        XPass<TILES> x0, x1, x2;
        x0 = load_x<TILES>(a, min(c_lo + v, b_hi - 1), j, lane);
        copy_pass<RH, kPassW, kPassS>(a, smem, g, c_lo, b_hi, v, lane, 0);
        asm volatile("" ::: "memory");
        if constexpr (PASSES > 1) {
            x1 = load_x<TILES>(a, min(c_lo + 8 + v, b_hi - 1), j, lane);
            copy_pass<RH, kPassW, kPassS>(a, smem, g, c_lo, b_hi, v, lane, 1);
            asm volatile("" ::: "memory");
        }
        if constexpr (PASSES > 2) {
            copy_pass<RH, kPassW, kPassS>(a, smem, g, c_lo, b_hi, v, lane, 2);
            asm volatile("" ::: "memory");
        }
        // 2. Pass i once its loads have landed, the later passes' still in flight. The
        // barrier carries no fence: a fence would wait for every outstanding copy (vmcnt
        // 0), and so would the compiler before any LDS read it sees after a direct-to-LDS
        // copy; the wave's own vmcnt wait covers its share of pass i, the barrier the
        // others', and the pass's LDS words are read by read_tile.
        wait_vm<PASSES == 3 ? kXLoads + 4 * RH : PASSES == 2 ? kXLoads + 2 * RH : 0>();
        pass_barrier();
        if (c_lo + v < b_hi) compute_pass<0, TILES, RT, kPassW + kPassS, kPassW>(x0, w_base, s_base, acc);
        if constexpr (PASSES > 2) {
            asm volatile("" ::: "memory");
            x2 = load_x<TILES>(a, min(c_lo + 16 + v, b_hi - 1), j, lane);
            asm volatile("" ::: "memory");
        }
        if constexpr (PASSES > 1) {
            wait_vm<PASSES == 3 ? kXLoads + 2 * RH : 0>();  // w2, x2 pending
            pass_barrier();
            if (c_lo + 8 + v < b_hi) compute_pass<1, TILES, RT, kPassW + kPassS, kPassW>(x1, w_base, s_base, acc);
        }
        if constexpr (PASSES > 2) {
            wait_vm<0>();
            pass_barrier();
            if (c_lo + 16 + v < b_hi) compute_pass<2, TILES, RT, kPassW + kPassS, kPassW>(x2, w_base, s_base, acc);
        }
        __syncthreads();  // every wave is done with this chunk's LDS
    }
    // Pin the last scaled accumulations here, in the MFMAs' basic block: left free, the
    // compiler may sink them past the branches below.
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int ct = 0; ct < TILES; ++ct)
#pragma unroll
            for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(acc[t][ct][e]));
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int ct = 0; ct < TILES; ++ct) s_red[((v * RT + t) * TILES + ct) * 64 + lane] = acc[t][ct];
    __syncthreads();
    // Thread unit = one row and four sequences (one lane's f32x4). Consecutive threads take
    // a row's sequence quads, then the next row: a wave's partial stores (and the last
    // workgroup's loads) cover contiguous memory.
    const bool single = a.splits == 1;
    constexpr int kUnits = RG * 4 * TILES;
    constexpr int SW = 16 * TILES;  // sequence slots of a partial row
#pragma unroll
    for (int k = 0; k < (kUnits + kQ4NT - 1) / kQ4NT; ++k) {
        const int u = tid + k * kQ4NT;
        if (u < kUnits) {
            const int qq = u % 4, ct = (u / 4) % TILES, r = u / (4 * TILES);
            const int t = r >> 4, ln = (r & 15) + 16 * qq;
            f32x4 sum = s_red[(t * TILES + ct) * 64 + ln];
#pragma unroll
            for (int w = 1; w < kQ4Waves; ++w) sum += s_red[((w * RT + t) * TILES + ct) * 64 + ln];
            const int row = g * RG + r;
            if (single) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int seq = 16 * ct + 4 * qq + e;
                    if (seq < a.batch && row < a.c_out) a.out[(size_t)seq * a.c_out + row] = sum[e];
                }
            } else {  // the four sequences' sums in one store, written through (see below)
                store16_system(a.part + ((size_t)blockIdx.x * RG + r) * SW + 16 * ct + 4 * qq, sum);
            }
        }
    }
    if (single) return;
    // The row group's last workgroup to finish adds the partials of all of them, in
    // workgroup order (deterministic), and writes out. The partials are stored and loaded
    // at system scope, i.e. written through and read past the L2 caches: once a
    // workgroup's stores are acknowledged (vmcnt 0) they are in memory, where the last
    // workgroup reads them, so no L2 write-back or invalidation is needed (those cost
    // more than the whole product on this 8-XCD part).
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const int done = __hip_atomic_fetch_add(&a.arrived[g], 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
        s_last = done == a.splits - 1;
        if (s_last) __hip_atomic_store(&a.arrived[g], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    // Per unit, the partials of kQ4RedLoads workgroups are requested together (a group past
    // the last workgroup re-reads the last one and is not added), then added in workgroup
    // order.
    const float* p0 = a.part + (size_t)g * a.splits * RG * SW;
    for (int u = tid; u < kUnits; u += kQ4NT) {
        const int qq = u % 4, ct = (u / 4) % TILES, r = u / (4 * TILES);
        const float* pu = p0 + (size_t)r * SW + 16 * ct + 4 * qq;
        f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int k0 = 0; k0 < a.splits; k0 += kQ4RedLoads) {
            f32x4 vals[kQ4RedLoads];
#pragma unroll
            for (int k = 0; k < kQ4RedLoads; ++k)
                vals[k] = load16_system(pu + (size_t)min(k0 + k, a.splits - 1) * RG * SW);
            wait_loads(vals);
#pragma unroll
            for (int k = 0; k < kQ4RedLoads; ++k)
                if (k0 + k < a.splits) sum += vals[k];
        }
        const int row = g * RG + r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int seq = 16 * ct + 4 * qq + e;
            if (seq < a.batch && row < a.c_out) a.out[(size_t)seq * a.c_out + row] = sum[e];
        }
    }
}

// Rows of a group in halves of 64: one. 64-row groups need at most 128 VGPRs up to two
// column tiles, so two 8-wave workgroups share a CU (four waves per SIMD); 128-row groups
// (two halves) measured slower at one workgroup per CU.
int q4_rh(int32_t) { return 1; }

}  // namespace
}  // namespace pkv

extern "C" {

size_t pkv_q4_matmul_workspace_size(int32_t c_in, int32_t c_out, int32_t batch) {
    if (c_in <= 0 || c_in % 32 || c_out <= 0 || batch <= 0 || batch > pkv::kQ4MaxBatch) return 0;
    const size_t rg = 64 * (size_t)pkv::q4_rh(batch);
    const size_t groups = ((size_t)c_out + rg - 1) / rg;
    // the row groups' arrival counts, then partials of at most kQ4MaxWg workgroups (or
    // one per row group): [workgroup][row of the group][16 x column tiles sequence slots]
    const size_t counts = (groups * sizeof(int32_t) + 255) & ~(size_t)255;
    const size_t wgs = groups > (size_t)pkv::kQ4MaxWg ? groups : (size_t)pkv::kQ4MaxWg;
    const size_t slots = 16 * (((size_t)batch + 15) / 16);
    return counts + wgs * rg * slots * sizeof(float);
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
        (reinterpret_cast<uintptr_t>(scales) & 3) || (reinterpret_cast<uintptr_t>(workspace) & 15))
        return fail(PKV_ERR_INVALID, "pkv_q4_matmul: w_packed, x and workspace need 16-byte, "
                                     "scales 4-byte alignment");
    if (workspace_bytes < pkv_q4_matmul_workspace_size(c_in, c_out, batch))
        return fail(PKV_ERR_WORKSPACE, "workspace smaller than pkv_q4_matmul_workspace_size()");
    if ((int64_t)c_out * (c_in / 2) > ((int64_t)1 << 40))
        return fail(PKV_ERR_UNSUPPORTED, "pkv_q4_matmul: matrix too large");
    const int tiles = (batch + 15) / 16;
    const int rh = q4_rh(batch);
    // Kernel instance per (column tiles, passes of a chunk); every instance has the same
    // register cap and LDS, so the occupancy query takes the three-pass one.
    using Kern = void (*)(Q4Args);
    static const Kern kKerns[4][kQ4MaxPass] = {
        {q4_matmul_kernel<1, 1, 1>, q4_matmul_kernel<1, 1, 2>, q4_matmul_kernel<1, 1, 3>},
        {q4_matmul_kernel<2, 1, 1>, q4_matmul_kernel<2, 1, 2>, q4_matmul_kernel<2, 1, 3>},
        {q4_matmul_kernel<3, 1, 1>, q4_matmul_kernel<3, 1, 2>, q4_matmul_kernel<3, 1, 3>},
        {q4_matmul_kernel<4, 1, 1>, q4_matmul_kernel<4, 1, 2>, q4_matmul_kernel<4, 1, 3>}};
    const void* fn = reinterpret_cast<const void*>(kKerns[tiles - 1][kQ4MaxPass - 1]);
    Q4Args a{};
    a.w = w_packed;
    a.scales = scales;
    a.x = x;
    a.out = out;
    a.c_in = c_in;
    a.c_out = c_out;
    a.batch = batch;
    a.nb = c_in / 32;
    a.groups = (c_out + 64 * rh - 1) / (64 * rh);
    a.arrived = static_cast<int32_t*>(workspace);
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                      (((size_t)a.groups * sizeof(int32_t) + 255) & ~(size_t)255));
    const int fill = device_fill_workgroups(fn, kQ4NT, 0, kQ4MaxWg);
    if (fill <= 0) return fail(PKV_ERR_HIP, "pkv_q4_matmul: occupancy query failed");
    // Splits per row group: as many as keep every workgroup resident in one round.
    int splits = fill / a.groups;
    if (splits < 1) splits = 1;
    if (splits > a.nb) splits = a.nb;
    a.per = (a.nb + splits - 1) / splits;
    a.splits = (a.nb + a.per - 1) / a.per;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // passes of 8 blocks per chunk: a run of `per` blocks in chunks of up to kQ4MaxPass
    const int passes = a.per >= 8 * kQ4MaxPass ? kQ4MaxPass : (a.per + 7) / 8;
    const dim3 grid(a.groups * a.splits), block(kQ4NT);
    hipLaunchKernelGGL(kKerns[tiles - 1][passes - 1], grid, block, 0, st, a);
    return check_launch("pkv_q4_matmul");
}

}  // extern "C"
