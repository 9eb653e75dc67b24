// K3 -- chunked-prefill attention over paged bf16 K/V with bf16 MFMA (gfx950).
//
// Replaces the engine's per-token prefill loop, which appends one token and calls
// paged_attention_layer for it before the next (model_speculative_moe_batched.mojo
// :2600-2637 chunked, :2767-2833 CPU), i.e. causal attention of every chunk query over
// the cached prefix plus the chunk itself. The chunk's K/V rows are appended first
// (pkv_append); this kernel then attends all chunk queries in one launch.
//
// Workgroup = (tile of 128/G queries, kv head g, sequence), eight waves, two per SIMD
// (waves w and w + 4 share one); wave w owns 16 rows: query block w / G (16 consecutive
// queries) of q head g*G + w % G. All waves share the K/V tiles of 64 keys staged in LDS.
// The two waves of a SIMD run half a tile apart (scores and softmax of one tile beside
// the other's PV of the tile before). Per key tile (v_mfma_f32_16x16x32_bf16 throughout):
//   S^T = K Q^T (A = K rows from LDS, B = Q from registers): row j of the wave lands in
//     lanes j, j+16, j+32, j+48, each holding 4 of every 16 keys, so the online softmax
//     needs two cross-lane steps (permlane16 / permlane32 swaps);
//   P = exp2(S * scale * log2 e - m), split P = P_hi + P_lo (both bf16; the residual of a
//     single bf16 rounding would break the 2e-2 output bound near zero);
//   O^T += V^T P^T (A = V^T, B = P_hi then P_lo straight from the S^T registers): the keys
//     of a 32-key step are taken in the order the S^T registers hold them, four
//     consecutive keys at a time, which is what one ds_read_b64_tr_b16 gathers from V
//     kept in its natural [key][dim] layout (two such reads per operand).
// Accumulation is fp32 throughout; the output is O / (l + 1e-10) (the reference's
// softmax denominator, attention.mojo:151-162).
//
// MFMA lane layouts (v_mfma_f32_16x16x32_bf16, checked on the device):
//   A[i][k]: lane i + 16*(k/8), element k%8;   B[k][j]: lane j + 16*(k/8), element k%8;
//   C[i][j]: lane j + 16*(i/4), register i%4.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "pkv_internal.h"

namespace pkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 256;             // head_dim of this kernel
constexpr int kKT = 64;             // keys per tile
constexpr int kNT = 512;            // eight waves
constexpr float kLog2e = 1.4426950408889634f;
// LDS tiles, double-buffered (bf16 elements), both filled straight from global memory
// (global_load_lds), rows of 512 B:
//   K: [key][256]; its 16-byte chunk c sits at chunk c ^ (key & 15): the 16 keys of an
//     operand read land on distinct banks.
//   V: [key][256]; its 32-byte chunk c (dims 16c .. 16c+15) sits at chunk c ^ (key & 15):
//     a transposed read takes the same 32-byte chunk of 16 keys, which then lands on
//     distinct banks.
constexpr int kKTile = kKT * kD;    // elements per K buffer (32 KiB)
constexpr int kVTile = kKT * kD;    // elements per V buffer (32 KiB)
constexpr int kVAhead = 6;          // PV operands requested ahead of the matrix cores
constexpr int kKAhead = 2;          // QK^T steps whose K operands are requested ahead
static_assert(2 * kVAhead < 16 && 4 * kKAhead < 16, "LDS reads in flight fit lgkmcnt");

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

struct PrefillArgs {
    const uint16_t* q;  // bf16 [rows][Hq][D]
    const uint16_t* k_pool;
    const uint16_t* v_pool;
    const int32_t* tables;
    int32_t table_stride;
    const int32_t* pos;    // [batch]: position of each sequence's first query
    const int32_t* q_off;  // [batch + 1]: query rows of sequence s
    int32_t Hq;
    int32_t Hkv;
    int32_t bs_shift;
    int32_t num_blocks;
    int32_t window;
    float scale_log2;  // softmax scale * log2(e)
    int32_t max_q;
    int32_t max_pos;
    int32_t qtiles;
    float* out;  // fp32 [rows][Hq][D]
};


__device__ inline float swap32_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float swap32_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float swap16_max(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float swap16_sum(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from global memory straight into LDS at dst + 16 * lane (dst uniform).
__device__ inline void copy16_to_lds(const uint16_t* src, uint16_t* dst) {
    __builtin_amdgcn_global_load_lds(src, (lds_void*)dst, 16, 0, 0);
}

// LDS reads the compiler does not track. It cannot tell which LDS words a direct-to-LDS
// copy in flight writes, so before any read it can see it waits for every copy (vmcnt),
// including the ones just issued for a later tile. The caller waits for these reads with
// lgkm_wait, which ties the values, so no use is scheduled above the wait.
// addr: an LDS byte address; OFF: a constant byte offset (< 65536).
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
__device__ inline uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_void*)p; }
template <int OFF>
__device__ inline i32x4 lds_read_b128(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    i32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
// ds_read_b64_tr_b16 (checked on the device): inside each 16-lane group, output lane j
// element e is element j % 4 of what input lane 4e + j / 4 addressed.
template <int OFF>
__device__ inline i32x2 lds_read_tr16(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    i32x2 v;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
// s_waitcnt lgkmcnt(N): at most N of this wave's LDS reads still in flight (they complete
// in order), so every read issued before the last N has landed.
template <int N>
__device__ inline void lgkm_wait(i32x4& a) {
    static_assert(N >= 0 && N < 16, "lgkmcnt");
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(a) : "i"(N));
}
template <int N>
__device__ inline void lgkm_wait(i32x4& a, i32x4& b, i32x4& c, i32x4& d) {
    static_assert(N >= 0 && N < 16, "lgkmcnt");
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "i"(N));
}

template <int P>
using Par = std::integral_constant<int, P>;

// f(Par<I>{}), f(Par<I + 1>{}), ..., f(Par<N - 1>{}): constant indices for template offsets.
template <int I, int N, typename F>
__device__ inline void static_for(F&& f) {
    if constexpr (I < N) {
        f(Par<I>{});
        static_for<I + 1, N>(f);
    }
}

template <int G>
__global__ __launch_bounds__(kNT) void prefill_kernel(PrefillArgs a) {
    constexpr int QB = 128 / G;  // queries per workgroup
    // Static arrays indexed by constant buffer numbers, so the compiler can tell a
    // direct-to-LDS copy into one buffer from reads of another and does not wait for the
    // copy before those reads.
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][kKTile];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][kVTile];
    __shared__ int s_bad[kNT / 64];  // per wave: a table entry of the range is outside the pool

    // Workgroup order. The hardware hands out workgroup ids in increasing order, round-robin
    // over the eight XCDs (id mod 8), and each XCD gives its next id to whichever of its CUs
    // frees first. Ids run over (sequence, tile from the last to the first, kv head) with the
    // kv head fastest, so every XCD receives the same run of tile lengths, long to short
    // within a sequence: a CU that finished a short tile takes the next sequence's long one,
    // and the CUs' total work evens out (with the tiles of one kv head spread over the XCDs
    // instead, the CUs' sums differed by ~30%). The head turns by one every eight tiles, so
    // with 8 kv heads each XCD takes neighbouring tiles of one head one after another: they
    // start together and read the same K/V rows at about the same time, from its L2 (turned
    // every tile, the L2 misses doubled). Every kv head still visits every XCD.
    const int lin = blockIdx.x;
    const int pair = lin / a.Hkv;  // (sequence, tile)
    const int g = (lin - pair * a.Hkv + (pair >> 3)) % a.Hkv;
    const int s = pair / a.qtiles;
    const int tile = a.qtiles - 1 - (pair - s * a.qtiles);  // long (late) tiles first
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int grp = lane >> 4;  // 16-lane group
    const int l16 = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = a.q_off[s];
    const int n_q = a.q_off[s + 1] - row0;
    const int q0 = tile * QB;
    const int head = g * G + wave % G;
    const int qi = q0 + (wave / G) * 16 + l16;  // this lane's query
    const bool live = qi < n_q;
    const int pos0 = a.pos[s];
    auto out_at = [&](int query, int h) -> float* {
        return a.out + ((size_t)(row0 + query) * a.Hq + h) * kD;
    };

    // Contract violations: the rows this workgroup owns get NaN (or zeros when the
    // sequence is inactive); queries beyond the grid (n_q > max_q) get NaN from tile 0.
    const int hi_all = pos0 + n_q - 1;
    const bool inactive = pos0 < 0;
    const bool bad_seq = !inactive && n_q > 0 &&
                         (hi_all > a.max_pos || (hi_all >> a.bs_shift) >= a.table_stride ||
                          n_q > a.max_q);
    if (tile == 0 && n_q > a.qtiles * QB && !inactive) {
        for (int i = tid; i < (n_q - a.qtiles * QB) * G * kD; i += kNT) {
            const int r = i / (G * kD), h = (i / kD) % G, d = i % kD;
            out_at(a.qtiles * QB + r, g * G + h)[d] = __builtin_nanf("");
        }
    }
    if (q0 >= n_q) return;
    if (inactive || bad_seq) {
        const float fill = inactive ? 0.f : __builtin_nanf("");
        for (int i = tid; i < QB * G * kD; i += kNT) {
            const int r = i / (G * kD), h = (i / kD) % G, d = i % kD;
            if (q0 + r < n_q) out_at(q0 + r, g * G + h)[d] = fill;
        }
        return;
    }

    const int q_last = min(n_q, q0 + QB) - 1;
    const int k_lo = window_start(pos0 + q0, a.window);
    const int k_hi = pos0 + q_last;
    const int qpos = pos0 + qi;
    const int ws_row = window_start(qpos, a.window);
    const int min_qpos = pos0 + q0;                   // tiles inside every row's range
    const int max_ws = window_start(k_hi, a.window);  // need no mask
    const int kb0 = k_lo & ~(kKT - 1);
    const int ntiles = (k_hi - kb0) / kKT + 1;
    const int32_t* trow = a.tables + (size_t)s * a.table_stride;
    const int bs_mask = (1 << a.bs_shift) - 1;

    // Tile copies. Wave w copies keys 8w .. 8w+7 of a tile, which lie in one block
    // (block_size >= 8): instruction j (of four) fills key rows 8w + 2j (lanes 0-31) and
    // 8w + 2j + 1 (lanes 32-63), 1 KiB straight from global memory into LDS. The block's
    // table entry is one load per wave and tile (the same address in every lane), made a
    // step before the copies that use it; a copy's address is that block's first row
    // (scalar) plus a per-lane offset that is the same for every tile. Keys outside
    // [k_lo, k_hi] (and tiles past the last) read rows of a valid block and are masked or
    // never read; a bad entry reads block 0 (the whole range was checked up front).
    // K: lane i loads the global chunk that belongs at 16-byte position i % 32 of its row,
    // i.e. chunk (i % 32) ^ (key & 15). V: LDS position p of key row k holds global chunk
    // 2 * ((p / 2) ^ (k & 15)) + p % 2 (the 32-byte chunk swizzle).
    const uint32_t row_bytes = (uint32_t)a.Hkv * kD * 2;
    uint32_t k_voff[4], v_voff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int kk = (8 * wave + 2 * j + (lane >> 5)) & 15, p16 = lane & 31;
        const uint32_t r = (uint32_t)(2 * j + (lane >> 5)) * row_bytes;
        k_voff[j] = r + 16 * (p16 ^ kk);
        v_voff[j] = r + 16 * ((((p16 >> 1) ^ kk) << 1) | (p16 & 1));
    }
    auto blk_ptr = [&](int t) {
        return trow + (min(max(kb0 + t * kKT + 8 * wave, k_lo), k_hi) >> a.bs_shift);
    };
    // Byte offset of the first row this wave copies in tile t, from its block's entry e.
    auto tile_off = [&](int t, int e) -> uint64_t {
        e = __builtin_amdgcn_readfirstlane(e);
        const int b = (uint32_t)e < (uint32_t)a.num_blocks ? e : 0;
        const uint32_t row = ((uint32_t)b << a.bs_shift) | ((kb0 + t * kKT + 8 * wave) & bs_mask);
        return (uint64_t)row * row_bytes + (uint64_t)g * (kD * 2);
    };
    // The entry load untracked by the compiler (its waits would cover every copy issued
    // after it): it completes with the step's barrier wait, which ties its value.
    auto load_blk_async = [&](int t, int& e) {
        asm volatile("global_load_dword %0, %1, off" : "=v"(e) : "v"(blk_ptr(t)));
    };
    auto issue_k = [&](auto PAR, int t, int e) {
        const char* base = reinterpret_cast<const char*>(a.k_pool) + tile_off(t, e);
        uint16_t* dst = sK[decltype(PAR)::value] + 8 * wave * kD;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            copy16_to_lds(reinterpret_cast<const uint16_t*>(base + k_voff[j]), dst + 2 * j * kD);
    };
    auto issue_v = [&](auto PAR, int t, int e) {
        const char* base = reinterpret_cast<const char*>(a.v_pool) + tile_off(t, e);
        uint16_t* dst = sV[decltype(PAR)::value] + 8 * wave * kD;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            copy16_to_lds(reinterpret_cast<const uint16_t*>(base + v_voff[j]), dst + 2 * j * kD);
    };

    // Q as the B operand of S^T: lane holds Q[row][32c + 8*grp .. +7] for c = 0..7.
    bf16x8 qreg[8];
    {
        const uint16_t* qp = a.q + ((size_t)(row0 + (live ? qi : 0)) * a.Hq + head) * kD + 8 * grp;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint4 v = live ? *reinterpret_cast<const uint4*>(qp + 32 * c) : make_uint4(0, 0, 0, 0);
            qreg[c] = __builtin_bit_cast(bf16x8, v);
        }
    }

    f32x4 o[16];  // O^T: d-tile u holds dims 16u + 4grp + r of this lane's row
#pragma unroll
    for (int u = 0; u < 16; ++u) o[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY;  // reference max (log2 domain) of this lane's row
    float l = 0.f;        // this lane's share of the running sum (its 16 of every 64 keys)
    bf16x8 ph[2], pl[2];  // P = P_hi + P_lo of the last scored tile, as PV's B operands

    // S^T = K Q^T for tile t, then the online softmax and the P split.
    auto score = [&](auto PAR, int t) {
        constexpr int par = decltype(PAR)::value;
        const int kb = kb0 + t * kKT;
        // Four 16-key sub-tiles (independent accumulators). The K operand of sub-tile u,
        // 32-dim step c is row 16u + l16, chunk (4c + grp) ^ l16, i.e. byte
        // 8192u + 512 l16 + 16 (grp ^ (l16 & 3)) + 64 ((c & 3) ^ (l16 >> 2)) + 256 (c >> 2):
        // four per-lane bases (c & 3) and constant offsets. The operands of step c + 2 are
        // requested while step c runs on the matrix cores.
        f32x4 st[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) st[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        const uint32_t k_lane = lds_addr(sK[0]) + 512 * l16 + 16 * (grp ^ (l16 & 3));
        uint32_t k_addr[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) k_addr[q] = k_lane + 64 * (q ^ (l16 >> 2));
        i32x4 ka[kKAhead + 1][4];
        auto kread = [&](auto C) {
            constexpr int c = decltype(C)::value;
            static_for<0, 4>([&](auto U) {
                constexpr int u = decltype(U)::value;
                ka[c % (kKAhead + 1)][u] =
                    lds_read_b128<par * 2 * kKTile + 8192 * u + 256 * (c >> 2)>(k_addr[c & 3]);
            });
        };
        // Wave priorities order the two waves of a SIMD: S^T first (2), then the other wave's
        // PV (1), the softmax's vector work last (0), so the scores of a step are ready early
        // and the matrix cores stay fed while the vector ALUs run the softmax
        // (config 4: 766 -> 737 us per launch).
        __builtin_amdgcn_s_setprio(2);
        static_for<0, kKAhead>(kread);
        static_for<0, 8>([&](auto C) {
            constexpr int c = decltype(C)::value, slot = c % (kKAhead + 1);
            if constexpr (c + kKAhead < 8) kread(Par<c + kKAhead>{});
            constexpr int later = 4 * (7 - c < kKAhead ? 7 - c : kKAhead);  // reads issued after step c's
            lgkm_wait<later>(ka[slot][0], ka[slot][1], ka[slot][2], ka[slot][3]);
#pragma unroll
            for (int u = 0; u < 4; ++u)
                st[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[slot][u]),
                                                               qreg[c], st[u], 0, 0, 0);
        });
        __builtin_amdgcn_s_setprio(0);
        // Tiles that straddle a row's causal edge or window start get -inf outside
        // [window_start(qpos), qpos]; st[u][r] is key kb + 16u + 4grp + r. Rows past the
        // chunk are never written, so they need no mask.
        if (!(kb >= max_ws && kb + kKT - 1 <= min_qpos)) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int kpos = kb + 16 * u + 4 * grp + r;
                    st[u][r] = (kpos <= qpos && kpos >= ws_row) ? st[u][r] : -INFINITY;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[u][r]);
        mx = swap32_max(swap16_max(mx)) * a.scale_log2;  // scale > 0: the max commutes
        // The reference max m moves only when the tile max exceeds it by more than 8
        // (log2 units): p = exp2(s - m) <= 256 stays exact enough in fp32, the result is
        // unchanged (softmax does not depend on the reference), and the accumulators are
        // rescaled only on the rare tiles that move it.
        const bool move = mx > m + 8.f;
        const float m_new = move ? mx : m;
        const float alpha = move ? __builtin_amdgcn_exp2f(m - m_new) : 1.f;  // m = -inf: 0
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        // v_exp_f32 directly: results below 2^-126 flush to zero, immaterial next to the
        // row sum. P = P_hi + P_lo, both bf16, packed as the B operand of each 32-key step:
        // element e of step ks is sub-tile 2ks + e/4, register e % 4. P_hi is p truncated
        // to bf16 (its top 16 bits, so two of them pack with one permute) and P_lo the exact
        // remainder p - P_hi rounded to nearest: |p - P_hi - P_lo| <= 2^-16 p.
        float lsum[2] = {0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const float p0 = __builtin_amdgcn_exp2f(fmaf(st[2 * ks + (e >> 2)][e & 3], a.scale_log2, -m_use));
                const float p1 =
                    __builtin_amdgcn_exp2f(fmaf(st[2 * ks + (e >> 2)][(e & 3) + 1], a.scale_log2, -m_use));
                lsum[0] += p0;
                lsum[1] += p1;
                const uint32_t u0 = __float_as_uint(p0), u1 = __float_as_uint(p1);
                const uint32_t hp = (u0 >> 16) | (u1 & 0xffff0000u);
                ph[ks][e] = __builtin_bit_cast(__bf16, (uint16_t)hp);
                ph[ks][e + 1] = __builtin_bit_cast(__bf16, (uint16_t)(hp >> 16));
                pl[ks][e] = (__bf16)(p0 - __uint_as_float(u0 & 0xffff0000u));
                pl[ks][e + 1] = (__bf16)(p1 - __uint_as_float(u1 & 0xffff0000u));
            }
        l = l * alpha + (lsum[0] + lsum[1]);
        m = m_new;
        if (__any(move)) {
#pragma unroll
            for (int u = 0; u < 16; ++u) o[u] *= alpha;
        }
    };

    // O^T += V^T P^T for tile t: 16 d-tiles x 2 steps of 32 keys, hi then lo; the V operand
    // of (step ks, d-tile u) is dims 16u + l16 of keys 32ks + 4grp + 0..3 and
    // 32ks + 16 + 4grp + 0..3 (elements 0..3 and 4..7), two transposed reads. The 32
    // (step, d-tile) operands run as one pipeline, kVAhead operands requested ahead of the
    // matrix cores (across the step boundary too).
    auto accumulate = [&](auto PAR) {
        constexpr int par = decltype(PAR)::value;
        // Operand (ks, u): with z = 4 grp + l16 / 4 (the key this lane addresses, mod 16),
        // byte 512 (32 ks + z) + 32 (u ^ z) + 8 (l16 & 3), and 16 keys (8192 bytes) further
        // for its second half.
        const int z = 4 * grp + (l16 >> 2);
        const uint32_t v_lane = lds_addr(sV[0]) + 512 * z + 8 * (l16 & 3);
        auto vread = [&](auto I) -> i32x4 {
            constexpr int i = decltype(I)::value, ks = i / 16, u = i % 16;
            constexpr int off = par * 2 * kVTile + 16384 * ks;
            const uint32_t ad = v_lane + ((u ^ z) << 5);
            const i32x2 lo = lds_read_tr16<off>(ad);
            const i32x2 hi = lds_read_tr16<off + 8192>(ad);
            return i32x4{lo.x, lo.y, hi.x, hi.y};
        };
        __builtin_amdgcn_s_setprio(1);  // below the other wave's S^T, above its softmax
        i32x4 va[kVAhead];
        static_for<0, kVAhead>([&](auto I) { va[decltype(I)::value] = vread(I); });
        static_for<0, 32>([&](auto I) {
            constexpr int i = decltype(I)::value, ks = i / 16, u = i % 16;
            i32x4 cur = va[i % kVAhead];
            if constexpr (i + kVAhead < 32) va[i % kVAhead] = vread(Par<i + kVAhead>{});
            constexpr int later = 2 * (31 - i < kVAhead ? 31 - i : kVAhead);  // reads issued after
            lgkm_wait<later>(cur);
            const bf16x8 vb = __builtin_bit_cast(bf16x8, cur);
            o[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vb, ph[ks], o[u], 0, 0, 0);
            o[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vb, pl[ks], o[u], 0, 0, 0);
        });
    };

    // Prologue: Q, the table entries of tiles 0 and 1, the check of every table entry of
    // the range (one load per thread per 512 blocks), tile 0's K and V.
    int blk[2];  // table entry of this wave's block in tiles t (blk[t % 2]) and t + 1
    blk[0] = *blk_ptr(0);
    blk[1] = *blk_ptr(1);
    int bad_local = 0;
    {
        const int b_lo = k_lo >> a.bs_shift, nblk = (k_hi >> a.bs_shift) - b_lo + 1;
        for (int i = tid; i < nblk; i += kNT) {
            const int e = trow[b_lo + i];
            bad_local |= (e < 0 || e >= a.num_blocks);
        }
    }
    issue_k(Par<0>{}, 0, blk[0]);
    issue_v(Par<0>{}, 0, blk[0]);
    const int bad_wave = __any(bad_local);
    if (lane == 0) s_bad[wave] = bad_wave;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    bool bad = false;
#pragma unroll
    for (int w = 0; w < kNT / 64; ++w) bad |= s_bad[w] != 0;

    // Ping-pong over the two waves of each SIMD (waves w and w + 4). The workgroup's
    // barriers split time into steps; per tile t the lead waves (0-3) score tile t in step
    // 2t and accumulate it in step 2t + 1, the trailing waves (4-7) one step later. So
    // while one wave of a SIMD runs its softmax on the vector ALUs, the other's PV keeps
    // the matrix cores busy. Copies (every wave copies its eight keys of each):
    //   step 2t:     K of tile t + 1 -> sK[(t + 1) % 2] (its old tile t - 1 was last
    //                scored in step 2t - 1);
    //   step 2t + 1: the table entries of tile t + 2, then V of tile t + 1
    //                -> sV[(t + 1) % 2] (tile t - 1 was last accumulated in step 2t).
    // Before the barrier that ends a step, each wave waits for its copies of the step
    // before (vmcnt 4: the four copies just issued stay in flight), so every tile is in
    // LDS one step before its first reader. Copies past the last tile re-read valid rows
    // into buffers nobody reads again. The barriers carry no fence (a fence would wait for
    // the copies just issued).
    auto step_barrier = [&]() {
        asm volatile("s_waitcnt vmcnt(4)"
                     : "+v"(blk[0]), "+v"(blk[1])
                     :
                     : "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    constexpr int kLead = 4;
    if (wave < kLead) {
        auto lead = [&](auto PAR, int t) {
            constexpr int par = decltype(PAR)::value;
            issue_k(Par<par ^ 1>{}, t + 1, blk[par ^ 1]);  // step 2t
            score(PAR, t);
            step_barrier();
            load_blk_async(t + 2, blk[par]);  // step 2t + 1
            issue_v(Par<par ^ 1>{}, t + 1, blk[par ^ 1]);
            accumulate(PAR);
            step_barrier();
        };
        for (int t = 0; t < ntiles; t += 2) {
            lead(Par<0>{}, t);
            if (t + 1 < ntiles) lead(Par<1>{}, t + 1);
        }
    } else {
        issue_k(Par<1>{}, 1, blk[1]);  // step 0
        step_barrier();
        auto trail = [&](auto PAR, int t) {
            constexpr int par = decltype(PAR)::value;
            load_blk_async(t + 2, blk[par]);  // step 2t + 1
            issue_v(Par<par ^ 1>{}, t + 1, blk[par ^ 1]);
            score(PAR, t);
            step_barrier();
            issue_k(PAR, t + 2, blk[par]);  // step 2t + 2
            accumulate(PAR);
            if (t + 1 < ntiles) step_barrier();
        };
        for (int t = 0; t < ntiles; t += 2) {
            trail(Par<0>{}, t);
            if (t + 1 < ntiles) trail(Par<1>{}, t + 1);
        }
    }
    // No copy may still be writing LDS when the workgroup's last wave ends.
    __builtin_amdgcn_s_waitcnt(0);

    const float l_row = swap32_sum(swap16_sum(l));
    const float inv = 1.f / (l_row + 1e-10f);
    if (live) {
        float* op = out_at(qi, head) + 4 * grp;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            float4 v;
            v.x = bad ? __builtin_nanf("") : o[u][0] * inv;
            v.y = bad ? __builtin_nanf("") : o[u][1] * inv;
            v.z = bad ? __builtin_nanf("") : o[u][2] * inv;
            v.w = bad ? __builtin_nanf("") : o[u][3] * inv;
            *reinterpret_cast<float4*>(op + 16 * u) = v;
        }
    }
}

}  // namespace
}  // namespace pkv

extern "C" {

int32_t pkv_prefill(void* stream, const pkv_params* p, const void* q, const void* k_pool,
                    const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                    const int32_t* pos, const int32_t* q_off, int32_t max_q, int32_t batch,
                    int32_t max_pos, float* out) {
    using namespace pkv;
    clear_error();
    int32_t rc = validate_params(p);
    if (rc != PKV_OK) return rc;
    if (p->kv_dtype != PKV_DTYPE_BF16)
        return fail(PKV_ERR_UNSUPPORTED, "pkv_prefill: the MFMA path needs bf16 pools");
    // A chunk appended whole into a ring would overwrite keys its own earlier queries
    // attend; ring layers prefill through pkv_attend in chunks of at most
    // ring_size - window + 1 queries.
    if (p->ring_size > 0)
        return fail(PKV_ERR_UNSUPPORTED, "pkv_prefill: paged pools only (ring_size 0)");
    if (p->head_dim != kD) return fail(PKV_ERR_UNSUPPORTED, "pkv_prefill: head_dim 256 only");
    if (p->block_size < 8)
        return fail(PKV_ERR_UNSUPPORTED, "pkv_prefill: block_size must be at least 8");
    const int G = p->num_heads / p->num_kv_heads;
    if (G != 1 && G != 2 && G != 4)
        return fail(PKV_ERR_UNSUPPORTED, "pkv_prefill: num_heads / num_kv_heads must be 1, 2 or 4");
    if (!(p->scale > 0.f) || !(p->scale < INFINITY))
        return fail(PKV_ERR_INVALID, "pkv_prefill: scale must be positive and finite");
    if (batch <= 0 || batch > 65535 || max_q <= 0 || table_stride <= 0 || max_pos < 0 ||
        p->num_kv_heads > 65535)
        return fail(PKV_ERR_INVALID, "pkv_prefill: batch, max_q, table_stride must be positive");
    if (!q || !k_pool || !v_pool || !block_tables || !pos || !q_off || !out)
        return fail(PKV_ERR_INVALID, "pkv_prefill: null device pointer");
    if ((int64_t)p->num_blocks << __builtin_ctz((unsigned)p->block_size) > INT32_MAX)
        return fail(PKV_ERR_UNSUPPORTED, "pkv_prefill: pool rows must fit in int32");
    PrefillArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.k_pool = static_cast<const uint16_t*>(k_pool);
    a.v_pool = static_cast<const uint16_t*>(v_pool);
    a.tables = block_tables;
    a.table_stride = table_stride;
    a.pos = pos;
    a.q_off = q_off;
    a.Hq = p->num_heads;
    a.Hkv = p->num_kv_heads;
    a.bs_shift = __builtin_ctz((unsigned)p->block_size);
    a.num_blocks = p->num_blocks;
    a.window = p->window;
    a.scale_log2 = p->scale * kLog2e;
    a.max_q = max_q;
    a.max_pos = max_pos;
    a.out = out;
    const int qb = 128 / G;
    a.qtiles = (max_q + qb - 1) / qb;
    // one workgroup id per (sequence, tile, kv head); the launch's work-items must fit in 32 bits
    const int64_t wgs = (int64_t)a.qtiles * p->num_kv_heads * batch;
    if (wgs > (int64_t)(UINT32_MAX / kNT))
        return fail(PKV_ERR_UNSUPPORTED, "pkv_prefill: too many (sequence, query tile, kv head) workgroups");
    const dim3 grid((uint32_t)wgs);
    hipStream_t st = static_cast<hipStream_t>(stream);
    // The kernel's four 32 KiB K/V buffers are static LDS (128 KiB of the CU's 160 KiB).
    if (G == 1) hipLaunchKernelGGL(prefill_kernel<1>, grid, dim3(kNT), 0, st, a);
    else if (G == 2) hipLaunchKernelGGL(prefill_kernel<2>, grid, dim3(kNT), 0, st, a);
    else hipLaunchKernelGGL(prefill_kernel<4>, grid, dim3(kNT), 0, st, a);
    return check_launch("pkv_prefill");
}

}  // extern "C"
