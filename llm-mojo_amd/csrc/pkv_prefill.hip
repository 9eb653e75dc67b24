// K3 -- chunked-prefill attention over paged bf16 K/V with bf16 MFMA (gfx950).
//
// Replaces the engine's per-token prefill loop, which appends one token and calls
// paged_attention_layer for it before the next (model_speculative_moe_batched.mojo
// :2600-2637 chunked, :2767-2833 CPU), i.e. causal attention of every chunk query over
// the cached prefix plus the chunk itself. The chunk's K/V rows are appended first
// (pkv_append); this kernel then attends all chunk queries in one launch.
//
// Workgroup = (tile of 128/G queries, kv head g, sequence), eight waves (two per SIMD, so
// one wave's softmax overlaps the other's matrix work); wave w owns 16 rows: query block
// w / G (16 consecutive queries) of q head g*G + w % G. All waves share the K/V tiles of
// 64 keys staged in LDS. Per key tile (v_mfma_f32_16x16x32_bf16 throughout):
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
// __builtin_amdgcn_sched_group_barrier instruction classes
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

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

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

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
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16 (checked on the device): inside each 16-lane group, output lane j
// element e is element j % 4 of what input lane 4e + j / 4 addressed. With input lane a
// addressing dims 4(a % 4) .. +3 of key k0 + a / 4, output lane j holds dim j of keys
// k0 .. k0 + 3.
__device__ inline s16x4 read_tr(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

template <int G>
__global__ __launch_bounds__(kNT) void prefill_kernel(PrefillArgs a) {
    constexpr int QB = 128 / G;  // queries per workgroup
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    uint16_t* sK = smem;                    // [2][kKTile]
    uint16_t* sV = smem + 2 * kKTile;       // [2][kVTile]
    // element offset of each key's head slice in the pools, per staged tile
    int64_t* s_off = reinterpret_cast<int64_t*>(smem + 2 * kKTile + 2 * kVTile);  // [4][kKT]
    int* s_bad = reinterpret_cast<int*>(s_off + 4 * kKT);

    const int s = blockIdx.z;
    const int g = blockIdx.y;
    const int tile = a.qtiles - 1 - (int)blockIdx.x;  // long (late) tiles first
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
    const size_t head_off = (size_t)g * kD;
    const size_t row_elems = (size_t)a.Hkv * kD;
    const int bs_mask = (1 << a.bs_shift) - 1;

    // Pool offsets of the keys of tile t -> s_off[t % 4] (threads 0..63). Keys outside
    // [k_lo, k_hi] re-read a valid row and are masked.
    auto stage_rows = [&](int t) {
        if (tid < kKT && t < ntiles) {
            const int kpos = min(max(kb0 + t * kKT + tid, k_lo), k_hi);
            int b = trow[kpos >> a.bs_shift];
            if (b < 0 || b >= a.num_blocks) {
                *s_bad = 1;
                b = 0;
            }
            const int row = (b << a.bs_shift) | (kpos & bs_mask);
            s_off[(t & 3) * kKT + tid] = (int64_t)row * (int64_t)row_elems + (int64_t)head_off;
        }
    };
    // K and V tiles t -> sK[t % 2], sV[t % 2] straight from global memory into LDS: each
    // wave instruction fills two key rows (1 KiB), eight waves x 4 instructions = 64 rows.
    // The wave's four key offsets are read from s_off once, for K and V both. Lane i loads
    // the global chunk that belongs at 16-byte position i % 32 of its row: for K that is
    // chunk (i % 32) ^ (key & 15); for V, LDS position p of key row k holds global chunk
    // 2 * ((p / 2) ^ (k & 15)) + p % 2 (the 32-byte chunk swizzle).
    auto issue_kv = [&](int t) {
        uint16_t* kdst = sK + (t & 1) * kKTile;
        uint16_t* vdst = sV + (t & 1) * kVTile;
        const int64_t* offs = s_off + (t & 3) * kKT;
        int64_t ko[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) ko[j] = offs[wave * 8 + 2 * j + (lane >> 5)];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int key = wave * 8 + 2 * j + (lane >> 5);
            const int c = (lane & 31) ^ (key & 15);
            __builtin_amdgcn_global_load_lds(a.k_pool + ko[j] + 8 * c,
                                             (lds_void*)(kdst + (wave * 8 + 2 * j) * kD), 16, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int key = wave * 8 + 2 * j + (lane >> 5);
            const int p16 = lane & 31;
            const int c = ((((p16 >> 1) ^ (key & 15)) << 1) | (p16 & 1));
            __builtin_amdgcn_global_load_lds(a.v_pool + ko[j] + 8 * c,
                                             (lds_void*)(vdst + (wave * 8 + 2 * j) * kD), 16, 0, 0);
        }
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

    // prologue: tile 0 staged, tile 1's and 2's offsets known
    if (tid == 0) *s_bad = 0;
    stage_rows(0);
    stage_rows(1);
    stage_rows(2);
    __syncthreads();
    issue_kv(0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
        const int kb = kb0 + t * kKT;
        if (t + 1 < ntiles) issue_kv(t + 1);
        const uint16_t* cK = sK + (t & 1) * kKTile;
        const uint16_t* cV = sV + (t & 1) * kVTile;

        // S^T = K Q^T: four 16-key sub-tiles (independent accumulators). The K operands of
        // 32-dim step c + 2 are requested while step c runs on the matrix cores; the
        // scheduling groups below keep that order (the compiler otherwise waits for each
        // read right after issuing it).
        f32x4 st[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) st[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto kop = [&](int u, int c) -> bf16x8 {
            const int key = 16 * u + l16;
            const int ch = (4 * c + grp) ^ (key & 15);
            return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(&cK[key * kD + 8 * ch]));
        };
        bf16x8 ka[3][4];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int u = 0; u < 4; ++u) ka[c][u] = kop(u, c);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            if (c + 2 < 8) {
#pragma unroll
                for (int u = 0; u < 4; ++u) ka[(c + 2) % 3][u] = kop(u, c + 2);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
                st[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[c % 3][u], qreg[c], st[u], 0, 0, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8, 0);
#pragma unroll
        for (int c = 0; c < 6; ++c) {
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 8, 0);
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
        bf16x8 ph[2], pl[2];
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
        // O^T += V^T P^T: 16 d-tiles x 2 steps of 32 keys, hi then lo; the V operand of
        // (step ks, d-tile u) is dims 16u + l16 of keys 32ks + 4grp + 0..3 and
        // 32ks + 16 + 4grp + 0..3 (elements 0..3 and 4..7), two transposed reads.
        auto vop = [&](int ks, int u) -> bf16x8 {
            const int kr = 32 * ks + 4 * grp + (l16 >> 2);  // key this lane addresses
            const int dq = 4 * (l16 & 3);                    // its dims within the 16-dim tile
            const s16x4 lo = read_tr(&cV[kr * kD + ((u ^ (kr & 15)) << 4) + dq]);
            const int kr2 = kr + 16;
            const s16x4 hi = read_tr(&cV[kr2 * kD + ((u ^ (kr2 & 15)) << 4) + dq]);
            const s16x8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            return __builtin_bit_cast(bf16x8, v);
        };
        // The 32 (step, d-tile) operands run as one pipeline, kVAhead operands requested
        // ahead of the matrix cores (across the step boundary too), and the scheduling
        // groups interleave each operand's two reads with two MFMAs.
        {
            bf16x8 va[kVAhead];
#pragma unroll
            for (int i = 0; i < kVAhead; ++i) va[i] = vop(i / 16, i % 16);
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                const int ks = i / 16, u = i % 16;
                const bf16x8 cur = va[i % kVAhead];
                if (i + kVAhead < 32) va[i % kVAhead] = vop((i + kVAhead) / 16, (i + kVAhead) % 16);
                o[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur, ph[ks], o[u], 0, 0, 0);
                o[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur, pl[ks], o[u], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * kVAhead, 1);
#pragma unroll
            for (int i = 0; i < 32 - kVAhead; ++i) {
                __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 1);
                __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 1);
            }
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2 * kVAhead, 1);
        }
        stage_rows(t + 3);
        __builtin_amdgcn_s_waitcnt(0);  // tile t+1's direct-to-LDS K loads have landed
        __syncthreads();
    }
    const bool bad = *s_bad != 0;
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

// Dynamic LDS of prefill_kernel: two K and two V^T tiles, four key-offset tables, a flag.
constexpr size_t kPrefillLds = (size_t)(2 * kKTile + 2 * kVTile) * 2 + 4 * kKT * 8 + 16;

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
    dim3 grid(a.qtiles, p->num_kv_heads, batch);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const void* fn = G == 1 ? reinterpret_cast<const void*>(&prefill_kernel<1>)
                   : G == 2 ? reinterpret_cast<const void*>(&prefill_kernel<2>)
                            : reinterpret_cast<const void*>(&prefill_kernel<4>);
    // Above 64 KiB of dynamic LDS the kernel must opt in (once per kernel and device).
    static_assert(kPrefillLds <= 160 * 1024, "LDS budget of one CU");
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPrefillLds) !=
        hipSuccess)
        return fail(PKV_ERR_HIP, "pkv_prefill: could not reserve the kernel's LDS");
    if (G == 1) hipLaunchKernelGGL(prefill_kernel<1>, grid, dim3(kNT), kPrefillLds, st, a);
    else if (G == 2) hipLaunchKernelGGL(prefill_kernel<2>, grid, dim3(kNT), kPrefillLds, st, a);
    else hipLaunchKernelGGL(prefill_kernel<4>, grid, dim3(kNT), kPrefillLds, st, a);
    return check_launch("pkv_prefill");
}

}  // extern "C"
