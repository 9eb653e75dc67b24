// K2 -- split-K paged attention for decode and multi-token verify (fp32 / bf16 pools).
//
// Replaces the reference's three-pass CPU loop (attention.mojo:151-294). Two launches:
//
// attend_chunk_kernel -- one workgroup per (key chunk, kv head, sequence). All query rows
// that share the KV head (GQA group x verify queries, <= 16 rows) are evaluated together,
// so every K/V byte of the chunk is read from HBM exactly once. Each wave owns a
// contiguous quarter of the chunk and runs an online softmax over batches of U tokens:
//   1. K and V rows of the batch are loaded together, unconditionally, with 16-byte
//      loads (one fp32 row of a D=256 head = 64 lanes x 16 B; a lane past the range
//      re-reads a valid row that is masked), so all of the batch's loads are in flight.
//   2. Scores: per-lane partial dots for U tokens x R rows, reduced across the row's
//      lanes with a halving exchange (each step sends half of the values, so U*R dots
//      cost ~U*R shuffles instead of U*R*log2(lanes)); afterwards lane group idx holds
//      dot idx, so each lane evaluates one exponential per batch.
//   3. Running max / sum per row; the accumulators are rescaled only when a row's max
//      moves; p is broadcast lane to lane and PV is accumulated in registers.
//   4. The four waves' (m, l, acc) are merged through LDS. A single-chunk sequence writes
//      o / (l + 1e-10); otherwise the chunk writes its (m, l, o) to the workspace.
// attend_merge_kernel -- one workgroup per (kv head, sequence) with several chunks:
//   out = sum_c o_c e^(m_c - M) / (sum_c l_c e^(m_c - M) + 1e-10), M = max_c m_c,
// which is the reference's softmax(x)_i = e^(x_i - max) / (sum + 1e-10). The launch
// boundary orders the partials: a fused "last workgroup merges" variant needs a
// device-scope release/acquire per workgroup, which on this 8-XCD part writes back and
// invalidates L2 and cost more than the whole merge.
//
// Arithmetic: fp32 pools accumulate in double (scores, exponentials, PV sums, merge),
// so the output is the exact attention rounded once to fp32; the fp32 reference path
// carries ~1e-7 absolute error of its own, and the parity bound (1e-4 relative with a
// 1e-3 floor) leaves no room for a second fp32 error of that size. On CDNA a non-packed
// double FMA issues at the fp32 rate, and the kernel is HBM-bound. bf16 pools (2e-2
// bound, twice the tokens per byte) accumulate in fp32.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "pkv_internal.h"

namespace pkv {
namespace {

constexpr int kNT = kBlockThreads;
constexpr int kNW = kNT / kWave;  // waves per workgroup
constexpr int kMaxChunk = 256;    // keys per chunk (compile-time LDS bound)
constexpr int kMaxPages = 257;    // pages one chunk can touch (block_size >= 1)

template <typename KV>
struct KVT;
template <>
struct KVT<float> {
    static constexpr int VE = 4;  // elements per 16-byte vector
    using Acc = double;
};
template <>
struct KVT<uint16_t> {  // bf16 bits
    static constexpr int VE = 8;
    using Acc = float;
};

template <int D, typename KV>
struct Lay {
    static constexpr int VE = KVT<KV>::VE;
    static constexpr int VPR = D / VE;                     // 16-byte vectors per head row
    static constexpr int LPR = VPR < kWave ? VPR : kWave;  // lanes sharing one token row
    static constexpr int NLD = VPR / LPR;                  // 16-byte loads per lane per row
    static constexpr int TPW = kWave / LPR;                // tokens per wave per load step
    static constexpr int EPL = NLD * VE;                   // row elements held per lane
    static_assert(VPR % LPR == 0, "row must split evenly over lanes");
};

// Unpack one 16-byte vector into VE values.
template <typename A>
__device__ inline void unpack(const uint4& v, A* out, float) {
    out[0] = (A)__uint_as_float(v.x);
    out[1] = (A)__uint_as_float(v.y);
    out[2] = (A)__uint_as_float(v.z);
    out[3] = (A)__uint_as_float(v.w);
}
template <typename A>
__device__ inline void unpack(const uint4& v, A* out, uint16_t) {
    out[0] = (A)bf16_lo(v.x);
    out[1] = (A)bf16_hi(v.x);
    out[2] = (A)bf16_lo(v.y);
    out[3] = (A)bf16_hi(v.y);
    out[4] = (A)bf16_lo(v.z);
    out[5] = (A)bf16_hi(v.z);
    out[6] = (A)bf16_lo(v.w);
    out[7] = (A)bf16_hi(v.w);
}

__device__ inline double exp_acc(double x) { return exp(x); }
__device__ inline float exp_acc(float x) { return expf(x); }

// Sum of N values per lane across each aligned group of W lanes (W a power of two).
// Halving exchange: at offset O a lane keeps one half of its values (upper half if
// lane & O) and receives the partner's copy of that half. When it returns, lane `l`
// holds F = max(1, N / W) totals, those of value indices base(l) .. base(l) + F - 1.
template <int N, int O, typename T>
struct XRed {
    static __device__ inline void run(T* v, int lane) {
        if constexpr (O == 0) {
            return;
        } else if constexpr (N == 1) {
            v[0] += __shfl_xor(v[0], O);
            XRed<1, O / 2, T>::run(v, lane);
        } else {
            const bool upper = (lane & O) != 0;
#pragma unroll
            for (int i = 0; i < N / 2; ++i) {
                T send = upper ? v[i] : v[i + N / 2];
                T keep = upper ? v[i + N / 2] : v[i];
                v[i] = keep + __shfl_xor(send, O);
            }
            XRed<N / 2, O / 2, T>::run(v, lane);
        }
    }
};

template <int N, int W>
__device__ inline int xred_base(int lane) {
    int base = 0, n = N;
#pragma unroll
    for (int o = W / 2; o >= 1; o >>= 1) {
        if (n > 1) {
            if (lane & o) base += n / 2;
            n /= 2;
        }
    }
    return base;
}

template <typename T>
__device__ inline T wave_max(T v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmax(v, __shfl_xor(v, off));
    return v;
}
template <typename T>
__device__ inline T wave_sum(T v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

struct AttendArgs {
    const float* q;
    const char* k_pool;
    const char* v_pool;
    const int32_t* tables;
    int32_t table_stride;
    const int32_t* pos;  // null -> pos_scalar (single sequence)
    int32_t pos_scalar;
    int32_t q_len;
    int32_t Hq;
    int32_t Hkv;
    int32_t G;  // num_heads / num_kv_heads
    int32_t bs;
    int32_t num_blocks;
    int32_t window;
    float scale;
    int32_t ring_size;  // > 0: ring pools (tables hold one ring slot per sequence)
    int64_t ring_base;  // ring mode, pos == null: first row of the sequence's ring
    const int32_t* keys;     // sparse mode (non-null): key positions, ragged by key_off
    const int32_t* key_off;  // [batch + 1]
    int32_t max_keys;        // sparse mode: the longest list the caller sized for
    int32_t chunk;
    int32_t max_chunks;
    void* part_ml;  // Acc pairs (m, l) per (row, chunk)
    void* part_o;   // Acc [D] per (row, chunk)
    float* out;
};

// Whether sequence s's keys [lo, hi] can be addressed: within its block table, or in
// ring mode within the ring (the reference aborts otherwise, attention.mojo:265-266)
// with a ring slot inside the pool. `rbase` receives the first row of the ring.
__device__ inline bool keys_addressable(const AttendArgs& a, int s, int lo, int hi,
                                        int64_t* rbase) {
    if (a.ring_size <= 0) return hi / a.bs < a.table_stride;
    if (hi - lo + 1 > a.ring_size) return false;
    if (!a.pos) {
        *rbase = a.ring_base;
        return true;
    }
    const int slot = a.tables[(size_t)s * a.table_stride];
    *rbase = (int64_t)slot * a.ring_size;
    return slot >= 0 && slot < a.num_blocks;
}

// The keys sequence s attends, as a range [lo, hi] of chunk coordinates: key positions
// (dense / ring modes: [window_start(pos), pos + q_len - 1]) or, in sparse mode, indices
// into the sequence's key list. state: 0 = active, 1 = no keys (zero output), 2 = the
// call's contract is violated (NaN output).
struct SeqKeys {
    int lo, hi, c_lo, nch, state, kbeg, pos0;
    int64_t rbase;
};
__device__ inline SeqKeys seq_keys(const AttendArgs& a, int s) {
    SeqKeys k{};
    const int C = a.chunk;
    if (a.keys) {
        k.kbeg = a.key_off[s];
        const int n = a.key_off[s + 1] - k.kbeg;
        k.lo = 0;
        k.hi = n - 1;
        k.nch = (n + C - 1) / C;
        k.state = n == 0 ? 1 : ((n < 0 || n > a.max_keys || k.kbeg < 0) ? 2 : 0);
        return k;
    }
    k.pos0 = a.pos ? a.pos[s] : a.pos_scalar;
    if (k.pos0 < 0) {  // inactive sequence: n <= 0 gives zeros (attention.mojo:180-185)
        k.state = 1;
        return k;
    }
    k.hi = k.pos0 + a.q_len - 1;
    k.lo = window_start(k.pos0, a.window);
    k.c_lo = k.lo / C;
    k.nch = k.hi / C - k.c_lo + 1;
    k.state = (!keys_addressable(a, s, k.lo, k.hi, &k.rbase) || k.nch > a.max_chunks) ? 2 : 0;
    return k;
}

// Output row r of this workgroup: query j = r / G, head h = g * G + r % G.
__device__ inline size_t out_index(const AttendArgs& a, int s, int g, int r, int d, int D) {
    int j = r / a.G;
    int h = g * a.G + r % a.G;
    return (((size_t)s * a.q_len + j) * a.Hq + h) * (size_t)D + d;
}

// Broadcast of a lane value; `src` must be the same for every lane of the wave.
__device__ inline double lane_bcast(double v, int src) {
    int lo = __builtin_amdgcn_readlane(__double2loint(v), src);
    int hi = __builtin_amdgcn_readlane(__double2hiint(v), src);
    return __hiloint2double(hi, lo);
}
__device__ inline float lane_bcast(float v, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}

template <int D, typename KV, int R>
__global__ __launch_bounds__(kNT) void attend_chunk_kernel(AttendArgs a) {
    using L = Lay<D, KV>;
    using Acc = typename KVT<KV>::Acc;
    constexpr int EPL = L::EPL;
    constexpr int NLD = L::NLD;
    constexpr int LPR = L::LPR;
    constexpr int TPW = L::TPW;
    constexpr int VE = L::VE;
    constexpr int AW = sizeof(Acc) / 4;  // 32-bit registers per accumulator
    static_assert(R <= LPR, "query rows per kv head must not exceed the lanes of a row");
    // Tokens per batch per token slot: every one of the U*R dots of a batch must land in
    // its own lane group after the halving reduction (U*R <= LPR); K and V of the batch
    // are in flight together, which bounds U by register pressure.
    constexpr int UREG = (R * EPL * AW <= 16) ? 8 : ((R * EPL * AW <= 32) ? 4 : 2);
    constexpr int U = UREG < LPR / R ? UREG : LPR / R;
    constexpr int NV = U * R;
    constexpr int REP = LPR / NV;  // lanes holding the same reduced dot

    __shared__ int s_page[kMaxPages];
    __shared__ Acc s_wm[kNW][R], s_wl[kNW][R];
    __shared__ Acc red[R * D];
    __shared__ Acc s_M[R], s_L[R];
    __shared__ int s_flag;

    const int c = blockIdx.x;
    const int g = blockIdx.y;
    const int s = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int sub = lane / LPR;  // token slot within a wave step
    const int rl = lane % LPR;   // lane within the row
    const int rows = a.G * a.q_len;

    const SeqKeys K = seq_keys(a, s);
    if (K.state != 0) {  // no keys: zeros; contract violated: NaN
        if (c == 0) {
            const float fill = K.state == 1 ? 0.f : __builtin_nanf("");
            for (int i = tid; i < rows * D; i += kNT) a.out[out_index(a, s, g, i / D, i % D, D)] = fill;
        }
        return;
    }
    const int pos0 = K.pos0, lo = K.lo, hi = K.hi, c_lo = K.c_lo, nch = K.nch;
    const int64_t rbase = K.rbase;
    const int C = a.chunk;
    const bool sparse = a.keys != nullptr;
    if (c >= nch) return;
    const int t0 = max(lo, (c_lo + c) * C);
    const int t1 = min(hi, (c_lo + c) * C + C - 1);
    const int ntok = t1 - t0 + 1;

    // Pages of this chunk -> LDS (bounds-checked against the pool); in sparse mode the
    // pool row of each of the chunk's keys instead.
    const int pg0 = t0 / a.bs;
    const int npg = sparse ? ntok : (a.ring_size > 0 ? 0 : t1 / a.bs - pg0 + 1);
    const int r_t0 = a.ring_size > 0 ? t0 % a.ring_size : 0;  // ring row of key t0
    const int32_t* trow = a.tables + (size_t)s * a.table_stride;
    if (tid == 0) s_flag = 0;
    __syncthreads();
    for (int i = tid; i < npg; i += kNT) {
        int b = 0;
        if (sparse) {
            const int key = a.keys[K.kbeg + t0 + i];
            const int blk = key < 0 ? -1 : key / a.bs;
            const int phys = (blk >= 0 && blk < a.table_stride) ? trow[blk] : -1;
            if (phys < 0 || phys >= a.num_blocks) s_flag = 1;
            else b = phys * a.bs + key % a.bs;
        } else {
            b = trow[pg0 + i];
            if (b < 0 || b >= a.num_blocks) {
                s_flag = 1;
                b = 0;
            }
        }
        s_page[i] = b;
    }

    // Q rows -> registers (scaled). Rows beyond `rows` stay zero.
    Acc qr[R][EPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (r < rows) {
            const float* qp = a.q + out_index(a, s, g, r, 0, D);
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                const int d0 = (i * LPR + rl) * VE;
#pragma unroll
                for (int e = 0; e < VE; e += 4) {
                    float4 v = *reinterpret_cast<const float4*>(qp + d0 + e);
                    qr[r][i * VE + e + 0] = (Acc)v.x * (Acc)a.scale;
                    qr[r][i * VE + e + 1] = (Acc)v.y * (Acc)a.scale;
                    qr[r][i * VE + e + 2] = (Acc)v.z * (Acc)a.scale;
                    qr[r][i * VE + e + 3] = (Acc)v.w * (Acc)a.scale;
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < EPL; ++e) qr[r][e] = (Acc)0;
        }
    }
    __syncthreads();

    const size_t head_off = (size_t)g * D;  // element offset of this kv head in a row
    const size_t row_elems = (size_t)a.Hkv * D;
    const int bs_shift = __builtin_ctz(a.bs);  // block_size is a power of two
    const int bs_mask = a.bs - 1;
    auto row_off = [&](int tok) -> size_t {  // byte offset of token `tok`'s head slice
        const int t = t0 + tok;
        size_t row;
        if (sparse) {
            row = (size_t)s_page[tok];
        } else if (a.ring_size > 0) {
            row = (size_t)ring_key_row(rbase, r_t0, tok, a.ring_size);
        } else {
            const int page = s_page[(t >> bs_shift) - pg0];
            row = ((size_t)page << bs_shift) + (size_t)(t & bs_mask);
        }
        return (row * row_elems + head_off) * sizeof(KV);
    };

    // This wave's contiguous token range of the chunk.
    const int per_wave = (((ntok + kNW - 1) / kNW) + TPW - 1) / TPW * TPW;
    const int wt0 = wave * per_wave;
    const int wt1 = min(ntok, wt0 + per_wave);

    // After the halving reduction lane `rl` holds dot idx = rl / REP, i.e. (u, r) =
    // (idx / R, idx % R); the lanes of row r are closed under xor of the u bits.
    const int idx_own = rl / REP;
    const int r_own = idx_own % R;
    const int u_own = idx_own / R;
    // query position of my row and its first key (sparse mode: every listed key)
    const int pq_own = sparse ? INT32_MAX : pos0 + r_own / a.G;
    const int ws_own = sparse ? 0 : window_start(pq_own, a.window);
    const bool row_live = r_own < rows;

    Acc m_own = (Acc)-INFINITY;  // running max of my row over this wave's tokens
    Acc l_own = (Acc)0;          // running sum of exp(s - m_own)
    Acc acc[R][EPL];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[r][e] = (Acc)0;

    for (int b0 = wt0; b0 < wt1; b0 += U * TPW) {
        // Every lane loads unconditionally (a token past the wave's range re-reads the
        // range's last row and is masked below), so the 2*U*NLD loads of the batch are
        // all in flight together instead of each waiting inside a branch.
        uint4 kv[U][NLD], vv[U][NLD];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int tok = min(b0 + u * TPW + sub, wt1 - 1);
            const size_t off = row_off(tok);
            const uint4* kp = reinterpret_cast<const uint4*>(a.k_pool + off);
            const uint4* vp = reinterpret_cast<const uint4*>(a.v_pool + off);
#pragma unroll
            for (int i = 0; i < NLD; ++i) {
                kv[u][i] = kp[i * LPR + rl];
                vv[u][i] = vp[i * LPR + rl];
            }
        }
        // scores: per-lane partial dots, then the halving reduction over the row's lanes
        Acc dots[NV];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            Acc kf[EPL];
#pragma unroll
            for (int i = 0; i < NLD; ++i) unpack<Acc>(kv[u][i], kf + i * VE, KV());
#pragma unroll
            for (int r = 0; r < R; ++r) {
                Acc d = (Acc)0;
#pragma unroll
                for (int e = 0; e < EPL; ++e) d = fma(qr[r][e], kf[e], d);
                dots[u * R + r] = d;
            }
        }
        XRed<NV, LPR / 2, Acc>::run(dots, rl);
        const int tok_own = b0 + u_own * TPW + sub;
        const int t_own = t0 + tok_own;
        const bool ok = row_live && tok_own < wt1 && t_own <= pq_own && t_own >= ws_own;
        const Acc sc_own = ok ? dots[0] : (Acc)-INFINITY;
        // batch max / sum of my row: xor over the u lane bits and the token-slot bits
        Acc mb = sc_own;
#pragma unroll
        for (int o = REP * R; o < LPR; o <<= 1) mb = fmax(mb, __shfl_xor(mb, o));
#pragma unroll
        for (int o = LPR; o < kWave; o <<= 1) mb = fmax(mb, __shfl_xor(mb, o));
        const bool moved = mb > m_own + (Acc)kLazyMove;  // lazy reference max; -inf: any live key
        const Acc m_new = moved ? mb : m_own;
        const Acc p_own = ok ? exp_acc(sc_own - m_new) : (Acc)0;
        Acc lb = p_own;
#pragma unroll
        for (int o = REP * R; o < LPR; o <<= 1) lb += __shfl_xor(lb, o);
#pragma unroll
        for (int o = LPR; o < kWave; o <<= 1) lb += __shfl_xor(lb, o);
        Acc scl = (Acc)1;
        if (moved) scl = exp_acc(m_own - m_new);  // m_own = -inf gives 0
        l_own = l_own * scl + lb;
        m_own = m_new;
        if (__any(moved)) {  // rescale every row's accumulators (row r's factor: lane r*REP)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const Acc f = lane_bcast(scl, r * REP);
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[r][e] *= f;
            }
        }
        // PV: p of (u, r) lives in lane sub*LPR + (u*R + r)*REP
#pragma unroll
        for (int u = 0; u < U; ++u) {
            Acc vf[EPL];
#pragma unroll
            for (int i = 0; i < NLD; ++i) unpack<Acc>(vv[u][i], vf + i * VE, KV());
#pragma unroll
            for (int r = 0; r < R; ++r) {
                Acc p;
                if constexpr (TPW == 1) p = lane_bcast(p_own, (u * R + r) * REP);
                else p = __shfl(p_own, sub * LPR + (u * R + r) * REP);
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[r][e] = fma(p, vf[e], acc[r][e]);
            }
        }
    }
    // Token slots of one wave hold the same d range and share (m, l): fold them.
#pragma unroll
    for (int o = LPR; o < kWave; o <<= 1)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[r][e] += __shfl_xor(acc[r][e], o);
    if (lane < NV * REP && (lane % REP) == 0 && idx_own < R) {
        s_wm[wave][r_own] = m_own;
        s_wl[wave][r_own] = l_own;
    }
    __syncthreads();

    // ---- merge the waves: M = max_w m_w, factor e^(m_w - M), L = sum_w l_w e^(m_w - M)
    Acc fw[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        Acc M = s_wm[0][r];
#pragma unroll
        for (int w = 1; w < kNW; ++w) M = fmax(M, s_wm[w][r]);
        const Acc mw = s_wm[wave][r];
        fw[r] = (mw == (Acc)-INFINITY) ? (Acc)0 : exp_acc(mw - M);
    }
    for (int w = 0; w < kNW; ++w) {
        if (wave == w && sub == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (r < rows) {
#pragma unroll
                    for (int i = 0; i < NLD; ++i) {
                        const int d0 = (i * LPR + rl) * VE;
                        Acc* dst = red + r * D + d0;
#pragma unroll
                        for (int e = 0; e < VE; ++e)
                            dst[e] = (w == 0 ? (Acc)0 : dst[e]) + acc[r][i * VE + e] * fw[r];
                    }
                }
            }
        }
        __syncthreads();
    }
    if (tid < rows) {
        const int r = tid;
        Acc M = s_wm[0][r];
        for (int w = 1; w < kNW; ++w) M = fmax(M, s_wm[w][r]);
        Acc Ls = (Acc)0;
        for (int w = 0; w < kNW; ++w)
            if (s_wm[w][r] != (Acc)-INFINITY) Ls += s_wl[w][r] * exp_acc(s_wm[w][r] - M);
        s_M[r] = M;
        s_L[r] = Ls;
    }
    __syncthreads();

    const bool bad = s_flag != 0;
    if (nch == 1) {
        for (int idx = tid; idx < rows * D; idx += kNT) {
            const int r = idx / D, d = idx % D;
            Acc res = red[r * D + d] / (s_L[r] + (Acc)1e-10);
            a.out[out_index(a, s, g, r, d, D)] = bad ? __builtin_nanf("") : (float)res;
        }
        return;
    }

    // Partial (m, l, o) of this chunk for each row; attend_merge_kernel combines them.
    Acc* part_o = static_cast<Acc*>(a.part_o);
    Acc* part_ml = static_cast<Acc*>(a.part_ml);
    const size_t row_base = ((size_t)s * a.q_len) * a.Hq;  // first row of sequence s
    auto prow_of = [&](int r) -> size_t {
        const int j = r / a.G, h = g * a.G + r % a.G;
        return row_base + (size_t)j * a.Hq + h;
    };
    for (int idx = tid; idx < rows * D; idx += kNT) {
        const int r = idx / D, d = idx % D;
        part_o[(prow_of(r) * a.max_chunks + c) * D + d] = red[r * D + d];
    }
    if (tid < rows) {
        const size_t pr = prow_of(tid);
        part_ml[(pr * a.max_chunks + c) * 2 + 0] = bad ? (Acc)__builtin_nan("") : s_M[tid];
        part_ml[(pr * a.max_chunks + c) * 2 + 1] = s_L[tid];
    }
}

// Cross-chunk merge, one workgroup per (kv head, sequence) with more than one chunk:
//   out = sum_c o_c w_c / (sum_c l_c w_c + 1e-10),  w_c = e^(m_c - M),  M = max_c m_c.
// A separate launch: the kernel boundary orders the partials written by the chunk
// kernel's workgroups (on any XCD) before these reads, with no fence inside either
// kernel. A NaN m_c marks a chunk that met a table entry outside the pool.
template <int D, typename Acc>
__global__ __launch_bounds__(kNT) void attend_merge_kernel(AttendArgs a) {
    constexpr int kRowsMax = 16;
    constexpr int kWT = 64;  // chunk weights staged per round
    __shared__ Acc s_M[kRowsMax], s_invL[kRowsMax];
    __shared__ Acc s_w[kRowsMax][kWT];
    const int g = blockIdx.x;
    const int s = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int rows = a.G * a.q_len;
    const SeqKeys K = seq_keys(a, s);
    const int nch = K.nch;
    if (K.state != 0 || nch == 1) return;

    const Acc* part_o = static_cast<const Acc*>(a.part_o);
    const Acc* part_ml = static_cast<const Acc*>(a.part_ml);
    const size_t row_base = ((size_t)s * a.q_len) * a.Hq;
    auto prow_of = [&](int r) -> size_t {
        const int j = r / a.G, h = g * a.G + r % a.G;
        return row_base + (size_t)j * a.Hq + h;
    };
    for (int r = wave; r < rows; r += kNW) {
        const Acc* ml = part_ml + prow_of(r) * a.max_chunks * 2;
        Acc M = (Acc)-INFINITY;
        int nan = 0;
        for (int cc = lane; cc < nch; cc += kWave) {
            const Acc m = ml[cc * 2];
            nan |= (m != m);
            M = fmax(M, m);
        }
        M = wave_max(M);
        nan = __any(nan);
        Acc Ls = (Acc)0;
        for (int cc = lane; cc < nch; cc += kWave) {
            const Acc m = ml[cc * 2];
            if (m != (Acc)-INFINITY) Ls += ml[cc * 2 + 1] * exp_acc(m - M);
        }
        Ls = wave_sum(Ls);
        if (lane == 0) {
            s_M[r] = M;
            s_invL[r] = nan ? (Acc)__builtin_nan("") : (Acc)1 / (Ls + (Acc)1e-10);
        }
    }
    __syncthreads();
    constexpr int kOut = (kRowsMax * D + kNT - 1) / kNT;  // outputs per thread, at most
    Acc oacc[kOut];
#pragma unroll
    for (int k = 0; k < kOut; ++k) oacc[k] = (Acc)0;
    for (int ct = 0; ct < nch; ct += kWT) {
        const int cn = min(kWT, nch - ct);
        for (int i = tid; i < rows * cn; i += kNT) {
            const int r = i / cn, cc = i % cn;
            const Acc m = part_ml[(prow_of(r) * a.max_chunks + ct + cc) * 2];
            s_w[r][cc] = (m == (Acc)-INFINITY || s_M[r] == (Acc)-INFINITY) ? (Acc)0
                                                                             : exp_acc(m - s_M[r]);
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kOut; ++k) {
            const int idx = tid + k * kNT;
            if (idx < rows * D) {
                const int r = idx / D, d = idx % D;
                const Acc* po = part_o + (prow_of(r) * a.max_chunks + ct) * D + d;
                Acc o[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) o[q] = (Acc)0;
                int cc = 0;
                for (; cc + 8 <= cn; cc += 8) {  // eight independent loads in flight
#pragma unroll
                    for (int q = 0; q < 8; ++q)
                        o[q] = fma(s_w[r][cc + q], po[(size_t)(cc + q) * D], o[q]);
                }
                for (; cc < cn; ++cc) o[0] = fma(s_w[r][cc], po[(size_t)cc * D], o[0]);
                oacc[k] += ((o[0] + o[1]) + (o[2] + o[3])) + ((o[4] + o[5]) + (o[6] + o[7]));
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < kOut; ++k) {
        const int idx = tid + k * kNT;
        if (idx < rows * D) {
            const int r = idx / D, d = idx % D;
            a.out[out_index(a, s, g, r, d, D)] = (float)(oacc[k] * s_invL[r]);
        }
    }
}

template <int D, typename KV, int R>
void launch(const AttendArgs& a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((attend_chunk_kernel<D, KV, R>), grid, dim3(kNT), 0, st, a);
    if (a.max_chunks > 1)
        hipLaunchKernelGGL((attend_merge_kernel<D, typename KVT<KV>::Acc>), dim3(grid.y, grid.z),
                           dim3(kNT), 0, st, a);
}

template <int D, typename KV>
int32_t dispatch_rows(const AttendArgs& a, int rows, dim3 grid, hipStream_t st) {
    if (rows <= 1) launch<D, KV, 1>(a, grid, st);
    else if (rows <= 2) launch<D, KV, 2>(a, grid, st);
    else if (rows <= 4) launch<D, KV, 4>(a, grid, st);
    else if (rows <= 8) launch<D, KV, 8>(a, grid, st);
    else if constexpr (D <= 256 && Lay<D, KV>::LPR >= 16) launch<D, KV, 16>(a, grid, st);
    else return fail(PKV_ERR_UNSUPPORTED, "at most 8 query rows per kv head for this head_dim / dtype");
    return PKV_OK;
}

// Rows per kv head the chunk kernel takes: 8, or 16 where a row's lanes number 16 or more
// (head_dim 64 fp32, head_dim 256).
bool chunk_rows_ok(const pkv_params* p, int rows) {
    if (rows <= 8) return true;
    if (rows > 16) return false;
    const int ve = p->kv_dtype == PKV_DTYPE_BF16 ? 8 : 4;
    const int vpr = p->head_dim / ve;
    const int lpr = vpr < kWave ? vpr : kWave;
    return p->head_dim <= 256 && lpr >= 16;
}

// Every check pkv_attend / pkv_verify make, and the kernel they take: *use_stream for the
// stream kernel, else the chunk kernel with layout *lay. Launches nothing.
int32_t attend_check(const pkv_params* p, const float* q, const void* k_pool,
                     const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                     const int32_t* pos, int32_t q_len, const int32_t* q_lens, int32_t batch,
                     int32_t max_pos, const float* out, const void* workspace,
                     size_t workspace_bytes, bool* use_stream, AttendLayout* lay) {
    int32_t rc = validate_params(p);
    if (rc != PKV_OK) return rc;
    if (batch <= 0 || q_len <= 0 || table_stride <= 0 || max_pos < 0)
        return fail(PKV_ERR_INVALID, "batch, q_len, table_stride must be positive, max_pos >= 0");
    const bool tables_read = !(p->ring_size > 0 && !pos);
    if (!q || !k_pool || !v_pool || (tables_read && !block_tables) || !out || !workspace)
        return fail(PKV_ERR_INVALID, "null device pointer");
    const int G = p->num_heads / p->num_kv_heads;
    const int rows = G * q_len;
    if (batch > 4096) return fail(PKV_ERR_INVALID, "batch must be <= 4096");
    if (stream_eligible(p, G) && workspace_bytes >= stream_layout(p, batch, q_len).total) {
        *use_stream = true;
        return PKV_OK;
    }
    *use_stream = false;
    if (q_lens) {
        if (!stream_eligible(p, G))
            return fail(PKV_ERR_UNSUPPORTED, "per-sequence query counts need head_dim 256 or 512 "
                                             "and num_heads / num_kv_heads <= 8");
        return fail(PKV_ERR_WORKSPACE, "workspace smaller than pkv_workspace_size()");
    }
    if (!chunk_rows_ok(p, rows))
        return fail(PKV_ERR_UNSUPPORTED, "this geometry allows at most 16 query rows "
                                         "(q_len * num_heads / num_kv_heads) per kv head, 8 at "
                                         "head_dim 512 or bf16 head_dim 64");
    *lay = attend_layout(p, batch, q_len, max_pos);
    if (lay->chunk > kMaxChunk) return fail(PKV_ERR_UNSUPPORTED, "chunk larger than the kernel's LDS bound");
    if (workspace_bytes < lay->total)
        return fail(PKV_ERR_WORKSPACE, "workspace smaller than pkv_workspace_size()");
    if (batch > 65535 || p->num_kv_heads > 65535)
        return fail(PKV_ERR_INVALID, "batch and num_kv_heads must be <= 65535");
    return PKV_OK;
}

// pos == NULL: one sequence at pos_scalar (whose ring, in ring mode, starts at row
// ring_base; block_tables is then not read and may be NULL). q_lens != NULL: sequence s
// has q_lens[s] <= q_len queries (stream path only).
int32_t attend_impl(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                    const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                    const int32_t* pos, int32_t pos_scalar, int64_t ring_base, int32_t q_len,
                    const int32_t* q_lens, int32_t batch, int32_t max_pos, float* out,
                    void* workspace, size_t workspace_bytes, const NewRows* nr = nullptr) {
    bool use_stream = false;
    AttendLayout lay{};
    int32_t rc = attend_check(p, q, k_pool, v_pool, block_tables, table_stride, pos, q_len,
                              q_lens, batch, max_pos, out, workspace, workspace_bytes,
                              &use_stream, &lay);
    if (rc != PKV_OK) return rc;
    const int G = p->num_heads / p->num_kv_heads;
    const int rows = G * q_len;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (nr && !use_stream) return fail(PKV_ERR_UNSUPPORTED, "appended rows need the stream path");
    if (use_stream) {
        rc = stream_attend(p, q, k_pool, v_pool, block_tables, table_stride, pos, pos_scalar,
                           ring_base, q_len, q_lens, batch, max_pos, nullptr, nullptr, 0, out,
                           workspace, st, nr);
        if (rc != PKV_OK) return rc;
        return check_launch("pkv_attend");
    }
    AttendArgs a{};
    char* ws = static_cast<char*>(workspace);
    a.q = q;
    a.k_pool = static_cast<const char*>(k_pool);
    a.v_pool = static_cast<const char*>(v_pool);
    a.tables = block_tables;
    a.table_stride = table_stride;
    a.pos = pos;
    a.pos_scalar = pos_scalar;
    a.q_len = q_len;
    a.Hq = p->num_heads;
    a.Hkv = p->num_kv_heads;
    a.G = G;
    a.bs = p->block_size;
    a.num_blocks = p->num_blocks;
    a.window = p->window;
    a.scale = p->scale;
    a.ring_size = p->ring_size;
    a.ring_base = ring_base;
    a.chunk = lay.chunk;
    a.max_chunks = lay.max_chunks;
    a.part_ml = ws + lay.ml_off;
    a.part_o = ws + lay.o_off;
    a.out = out;
    dim3 grid(lay.max_chunks, p->num_kv_heads, batch);
    const bool bf16 = p->kv_dtype == PKV_DTYPE_BF16;
    switch (p->head_dim) {
        case 64: rc = bf16 ? dispatch_rows<64, uint16_t>(a, rows, grid, st)
                           : dispatch_rows<64, float>(a, rows, grid, st); break;
        case 256: rc = bf16 ? dispatch_rows<256, uint16_t>(a, rows, grid, st)
                            : dispatch_rows<256, float>(a, rows, grid, st); break;
        case 512: rc = bf16 ? dispatch_rows<512, uint16_t>(a, rows, grid, st)
                            : dispatch_rows<512, float>(a, rows, grid, st); break;
        default: return fail(PKV_ERR_UNSUPPORTED, "head_dim");
    }
    if (rc != PKV_OK) return rc;
    return check_launch("pkv_attend");
}

// Layout of the sparse mode's workspace: the chunk kernel's partials for key lists of up
// to max_keys entries (window and ring do not bound a key list). Chunks index the list,
// so they need not align with blocks: the largest of 256 / 128 / 64 / 32 keys that still
// gives two workgroups per CU of the 256 (LSA lists are a few hundred keys).
AttendLayout sparse_layout(const pkv_params* p, int32_t batch, int32_t max_keys) {
    AttendLayout L{};
    int chunk = 256;
    while (chunk > 32 &&
           (int64_t)batch * p->num_kv_heads * ((max_keys + chunk - 1) / chunk) < 512)
        chunk /= 2;
    L.chunk = chunk;
    L.max_chunks = (max_keys + chunk - 1) / chunk;
    auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t rows = (size_t)batch * p->num_heads;
    L.ml_off = 0;
    L.o_off = align(rows * L.max_chunks * 2 * sizeof(double));
    L.total = L.o_off + align(rows * L.max_chunks * (size_t)p->head_dim * sizeof(double));
    return L;
}

}  // namespace
}  // namespace pkv

extern "C" {

size_t pkv_sparse_workspace_size(const pkv_params* p, int32_t batch, int32_t max_keys) {
    if (pkv::validate_params(p) != PKV_OK) return 0;
    if (batch <= 0 || max_keys <= 0) return 0;
    const size_t chunked = pkv::sparse_layout(p, batch, max_keys).total;
    const size_t stream = pkv::stream_layout(p, batch, 1).total;
    return chunked > stream ? chunked : stream;
}

int32_t pkv_attend_sparse(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                          const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                          const int32_t* keys, const int32_t* key_off, int32_t max_keys,
                          int32_t batch, float* out, void* workspace, size_t workspace_bytes) {
    using namespace pkv;
    clear_error();
    int32_t rc = validate_params(p);
    if (rc != PKV_OK) return rc;
    if (p->ring_size > 0)
        return fail(PKV_ERR_UNSUPPORTED, "pkv_attend_sparse: paged pools only (ring_size 0)");
    if (batch <= 0 || batch > 65535 || max_keys <= 0 || table_stride <= 0 ||
        p->num_kv_heads > 65535)
        return fail(PKV_ERR_INVALID, "batch, max_keys and table_stride must be positive");
    if (!q || !k_pool || !v_pool || !block_tables || !keys || !key_off || !out || !workspace)
        return fail(PKV_ERR_INVALID, "null device pointer");
    const int G = p->num_heads / p->num_kv_heads;
    if (G > 16) return fail(PKV_ERR_UNSUPPORTED, "num_heads / num_kv_heads must be <= 16");
    if ((int64_t)p->num_blocks * p->block_size > INT32_MAX)
        return fail(PKV_ERR_UNSUPPORTED, "pool rows must fit in int32");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // Lists of more than kStreamMaxBatch sequences take the chunk kernel (the stream
    // kernels keep a per-sequence plan in LDS).
    if (stream_eligible(p, G) && batch <= kStreamMaxBatch &&
        workspace_bytes >= stream_layout(p, batch, 1).total) {
        rc = stream_attend(p, q, k_pool, v_pool, block_tables, table_stride, nullptr, 0, 0, 1,
                           nullptr, batch, 0, keys, key_off, max_keys, out, workspace, st);
        if (rc != PKV_OK) return rc;
        return check_launch("pkv_attend_sparse");
    }
    AttendLayout lay = sparse_layout(p, batch, max_keys);
    if (lay.chunk > kMaxChunk) return fail(PKV_ERR_UNSUPPORTED, "chunk larger than the kernel's LDS bound");
    if (workspace_bytes < lay.total)
        return fail(PKV_ERR_WORKSPACE, "workspace smaller than pkv_sparse_workspace_size()");
    AttendArgs a{};
    char* ws = static_cast<char*>(workspace);
    a.q = q;
    a.k_pool = static_cast<const char*>(k_pool);
    a.v_pool = static_cast<const char*>(v_pool);
    a.tables = block_tables;
    a.table_stride = table_stride;
    a.q_len = 1;
    a.Hq = p->num_heads;
    a.Hkv = p->num_kv_heads;
    a.G = G;
    a.bs = p->block_size;
    a.num_blocks = p->num_blocks;
    a.scale = p->scale;
    a.keys = keys;
    a.key_off = key_off;
    a.max_keys = max_keys;
    a.chunk = lay.chunk;
    a.max_chunks = lay.max_chunks;
    a.part_ml = ws + lay.ml_off;
    a.part_o = ws + lay.o_off;
    a.out = out;
    dim3 grid(lay.max_chunks, p->num_kv_heads, batch);
    const bool bf16 = p->kv_dtype == PKV_DTYPE_BF16;
    switch (p->head_dim) {
        case 64: rc = bf16 ? dispatch_rows<64, uint16_t>(a, G, grid, st)
                           : dispatch_rows<64, float>(a, G, grid, st); break;
        case 256: rc = bf16 ? dispatch_rows<256, uint16_t>(a, G, grid, st)
                            : dispatch_rows<256, float>(a, G, grid, st); break;
        case 512: rc = bf16 ? dispatch_rows<512, uint16_t>(a, G, grid, st)
                            : dispatch_rows<512, float>(a, G, grid, st); break;
        default: return fail(PKV_ERR_UNSUPPORTED, "head_dim");
    }
    if (rc != PKV_OK) return rc;
    return check_launch("pkv_attend_sparse");
}

int32_t pkv_attend(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                   const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                   const int32_t* pos, int32_t q_len, int32_t batch, int32_t max_pos,
                   float* out, void* workspace, size_t workspace_bytes) {
    pkv::clear_error();
    if (!pos) return pkv::fail(PKV_ERR_INVALID, "pos is NULL");
    return pkv::attend_impl(stream, p, q, k_pool, v_pool, block_tables, table_stride, pos, 0, 0,
                            q_len, nullptr, batch, max_pos, out, workspace, workspace_bytes);
}

int32_t pkv_append_attend(void* stream, const pkv_params* p, void* k_pool, void* v_pool,
                          int32_t* block_tables, int32_t table_stride, int32_t* table_lens,
                          int32_t* free_list, int32_t* free_count, const int32_t* pos,
                          const int32_t* tok_off, int32_t max_new, const void* k_new,
                          const void* v_new, int32_t total_rows, int32_t* status, const float* q,
                          int32_t q_len, int32_t batch, int32_t max_pos, float* out,
                          void* workspace, size_t workspace_bytes) {
    using namespace pkv;
    clear_error();
    int32_t rc = validate_params(p);
    if (rc != PKV_OK) return rc;
    // Every check of the attention runs before the append launches anything, so a call
    // that returns an error has changed no table, free list or pool.
    if (!pos) return fail(PKV_ERR_INVALID, "null device pointer");
    bool use_stream = false;
    AttendLayout lay{};
    rc = attend_check(p, q, k_pool, v_pool, block_tables, table_stride, pos, q_len, nullptr,
                      batch, max_pos, out, workspace, workspace_bytes, &use_stream, &lay);
    if (rc != PKV_OK) return rc;
    if (workspace_bytes < pkv_workspace_size(p, batch, q_len, max_pos))
        return fail(PKV_ERR_WORKSPACE, "workspace smaller than pkv_workspace_size()");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // When one vector-kernel launch covers the call, the stream kernel does the append
    // itself (allocation, row copies) and its merge launch writes the state; otherwise the
    // append runs whole first.
    const bool fuse = stream_takes_new_rows(p, q_len, batch) &&
                      workspace_bytes >= stream_layout(p, batch, q_len).total;
    if (fuse) {
        rc = append_validate(p, k_pool, v_pool, block_tables, table_stride, table_lens, free_list,
                             free_count, pos, tok_off, max_new, k_new, v_new, total_rows, batch,
                             status);
        if (rc != PKV_OK) return rc;
        NewRows nr{};
        nr.k_new = static_cast<const char*>(k_new);
        nr.v_new = static_cast<const char*>(v_new);
        nr.tok_off = tok_off;
        nr.k_dst = static_cast<char*>(k_pool);
        nr.v_dst = static_cast<char*>(v_pool);
        nr.tables = block_tables;
        nr.table_lens = table_lens;
        nr.free_list = free_list;
        nr.free_count = free_count;
        nr.status = status;
        nr.max_new = max_new;
        nr.total_rows = total_rows;
        return attend_impl(stream, p, q, k_pool, v_pool, block_tables, table_stride, pos, 0, 0,
                           q_len, nullptr, batch, max_pos, out, workspace, workspace_bytes, &nr);
    }
    rc = append_launch(st, p, k_pool, v_pool, block_tables, table_stride, table_lens, free_list,
                       free_count, pos, tok_off, max_new, k_new, v_new, total_rows, batch, status,
                       true);
    if (rc != PKV_OK) return rc;
    return attend_impl(stream, p, q, k_pool, v_pool, block_tables, table_stride, pos, 0, 0, q_len,
                       nullptr, batch, max_pos, out, workspace, workspace_bytes);
}

int32_t pkv_verify(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                   const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                   const int32_t* pos, const int32_t* q_lens, int32_t max_q_len, int32_t batch,
                   int32_t max_pos, float* out, void* workspace, size_t workspace_bytes) {
    pkv::clear_error();
    if (!pos || !q_lens) return pkv::fail(PKV_ERR_INVALID, "pos or q_lens is NULL");
    return pkv::attend_impl(stream, p, q, k_pool, v_pool, block_tables, table_stride, pos, 0, 0,
                            max_q_len, q_lens, batch, max_pos, out, workspace, workspace_bytes);
}

int32_t pkv_decode(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                   const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                   const int32_t* pos, int32_t batch, int32_t max_pos, float* out,
                   void* workspace, size_t workspace_bytes) {
    return pkv_attend(stream, p, q, k_pool, v_pool, block_tables, table_stride, pos, 1, batch,
                      max_pos, out, workspace, workspace_bytes);
}

int32_t pkv_paged_attention_layer(void* stream, const float* q, const void* k_pool,
                                  const void* v_pool, const int32_t* block_table,
                                  int32_t block_size, int32_t pos, int32_t num_heads,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t window,
                                  float* attn_out, int32_t ring_size, int32_t ring_base,
                                  int32_t num_blocks, int32_t kv_dtype, void* workspace,
                                  size_t workspace_bytes) {
    pkv::clear_error();
    pkv_params p{};
    p.num_heads = num_heads;
    p.num_kv_heads = num_kv_heads;
    p.head_dim = head_dim;
    p.block_size = block_size;
    p.num_blocks = num_blocks;
    p.window = window;
    p.scale = 1.0f;
    p.kv_dtype = kv_dtype;
    p.ring_size = ring_size;
    if (pos < 0) pos = -1;
    if (ring_size > 0) {
        // Ring rows ring_base .. ring_base + ring_size - 1 must lie in the pool of
        // num_blocks rings, and the attended keys must fit the ring (the reference aborts
        // otherwise, attention.mojo:265-266). block_table is not read.
        const int64_t n = pos < 0 ? 0 : (int64_t)pos + 1 - pkv::window_start(pos, window);
        if (ring_base < 0 || (int64_t)ring_base + ring_size > (int64_t)num_blocks * ring_size)
            return pkv::fail(PKV_ERR_INVALID, "ring_base outside the pool of num_blocks rings");
        if (n > ring_size)
            return pkv::fail(PKV_ERR_INVALID, "ring_size smaller than the attended window");
        return pkv::attend_impl(stream, &p, q, k_pool, v_pool, nullptr, 1, nullptr, pos,
                                ring_base, 1, nullptr, 1, pos < 0 ? 0 : pos, attn_out, workspace,
                                workspace_bytes);
    }
    // The table must cover pos (attention.mojo:271); the kernel checks against the
    // stride, so the stride is exactly the entries needed.
    int32_t stride = (pos < 0 ? 0 : pos / (block_size > 0 ? block_size : 1)) + 1;
    return pkv::attend_impl(stream, &p, q, k_pool, v_pool, block_table, stride, nullptr, pos, 0,
                            1, nullptr, 1, pos < 0 ? 0 : pos, attn_out, workspace, workspace_bytes);
}

}  // extern "C"
