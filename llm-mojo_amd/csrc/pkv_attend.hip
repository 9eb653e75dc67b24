// K2 -- split-K paged attention for decode and multi-token verify (fp32 / bf16 pools).
//
// Replaces the reference's three-pass CPU loop (attention.mojo:151-294). Work unit:
// one workgroup per (key chunk, kv head, sequence). All query rows that share the KV
// head (GQA group x verify queries, <= 16 rows) are evaluated together, so every K/V
// byte of the chunk is read from HBM exactly once:
//   1. Q rows -> registers (each lane holds the slice of D it multiplies).
//   2. Scores: each wave streams K rows of its tokens with 16-byte loads (one fp32 row of
//      a D=256 head = 64 lanes x 16 B), forms per-lane partial dots for U tokens x R rows
//      and reduces all of them across the row's lanes with a halving exchange (each
//      step sends half of the values, so U*R dots cost ~U*R shuffles instead of
//      U*R*log2(lanes)). Masked scores go to LDS.
//   3. Chunk softmax statistics: m = max, p = exp(s - m), l = sum p (in LDS).
//   4. PV: each wave streams V rows and accumulates p * v in registers; the per-wave
//      sums are added in LDS one wave after another.
//   5. A single-chunk sequence writes o / (l + 1e-10) directly. Otherwise the chunk
//      writes (m, l, o) to the workspace and the last chunk of (sequence, kv head) to
//      finish (atomic counter) merges all chunks:
//      out = sum_c o_c e^(m_c - M) / (sum_c l_c e^(m_c - M) + 1e-10), M = max_c m_c,
//      which is the reference's softmax(x)_i = e^(x_i - max) / (sum + 1e-10).
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
    int32_t chunk;
    int32_t max_chunks;
    void* part_ml;  // Acc pairs (m, l) per (row, chunk)
    void* part_o;   // Acc [D] per (row, chunk)
    int32_t* counters;
    float* out;
};

// Output row r of this workgroup: query j = r / G, head h = g * G + r % G.
__device__ inline size_t out_index(const AttendArgs& a, int s, int g, int r, int d, int D) {
    int j = r / a.G;
    int h = g * a.G + r % a.G;
    return (((size_t)s * a.q_len + j) * a.Hq + h) * (size_t)D + d;
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
    // Token steps kept in flight per wave, bounded by register pressure.
    constexpr int U = (R * EPL * AW <= 16) ? 8 : ((R * EPL * AW <= 32) ? 4 : 2);
    constexpr int NV = U * R;  // dots reduced together
    constexpr int F = NV >= LPR ? NV / LPR : 1;
    constexpr int SMEM_SCORES = R * kMaxChunk;
    constexpr int SMEM_RED = R * D;
    constexpr int SMEM = SMEM_SCORES > SMEM_RED ? SMEM_SCORES : SMEM_RED;

    __shared__ Acc smem[SMEM];
    __shared__ int s_page[kMaxPages];
    __shared__ Acc s_m[R], s_l[R];
    __shared__ int s_flag, s_last;

    const int c = blockIdx.x;
    const int g = blockIdx.y;
    const int s = blockIdx.z;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int sub = lane / LPR;  // token slot within a wave step
    const int rl = lane % LPR;   // lane within the row
    const int rows = a.G * a.q_len;

    const int pos0 = a.pos ? a.pos[s] : a.pos_scalar;
    if (pos0 < 0) {  // inactive sequence: n <= 0 gives zeros (attention.mojo:180-185)
        if (c == 0)
            for (int i = tid; i < rows * D; i += kNT) a.out[out_index(a, s, g, i / D, i % D, D)] = 0.f;
        return;
    }
    const int hi = pos0 + a.q_len - 1;
    const int lo = window_start(pos0, a.window);
    const int C = a.chunk;
    const int c_lo = lo / C;
    const int nch = hi / C - c_lo + 1;
    if (hi / a.bs >= a.table_stride || nch > a.max_chunks) {  // contract violated
        if (c == 0)
            for (int i = tid; i < rows * D; i += kNT)
                a.out[out_index(a, s, g, i / D, i % D, D)] = __builtin_nanf("");
        return;
    }
    if (c >= nch) return;
    const int t0 = max(lo, (c_lo + c) * C);
    const int t1 = min(hi, (c_lo + c) * C + C - 1);
    const int ntok = t1 - t0 + 1;

    // Pages of this chunk -> LDS (bounds-checked against the pool).
    const int pg0 = t0 / a.bs;
    const int npg = t1 / a.bs - pg0 + 1;
    if (tid == 0) s_flag = 0;
    __syncthreads();
    for (int i = tid; i < npg; i += kNT) {
        int b = a.tables[(size_t)s * a.table_stride + pg0 + i];
        if (b < 0 || b >= a.num_blocks) {
            s_flag = 1;
            b = 0;
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
    auto row_ptr = [&](const char* pool, int tok) -> const uint4* {
        const int t = t0 + tok;
        const int page = s_page[t / a.bs - pg0];
        const size_t row = (size_t)page * a.bs + (size_t)(t % a.bs);
        return reinterpret_cast<const uint4*>(pool + (row * row_elems + head_off) * sizeof(KV));
    };

    Acc* s_sc = smem;  // [R][kMaxChunk] scores, then probabilities
    const int step = kNW * TPW;
    const int base_idx = xred_base<NV, LPR>(rl);
    constexpr int kPlainMask = NV >= LPR ? 0 : (LPR / NV) - 1;

    // ---- scores
    for (int base = wave * TPW; base < ntok; base += step * U) {
        uint4 kv[U][NLD];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int tok = base + u * step + sub;
            if (tok < ntok) {
                const uint4* rp = row_ptr(a.k_pool, tok);
#pragma unroll
                for (int i = 0; i < NLD; ++i) kv[u][i] = rp[i * LPR + rl];
            } else {
#pragma unroll
                for (int i = 0; i < NLD; ++i) kv[u][i] = make_uint4(0, 0, 0, 0);
            }
        }
        Acc dots[NV];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            Acc kf[EPL];
#pragma unroll
            for (int i = 0; i < NLD; ++i) unpack<Acc>(kv[u][i], kf + i * VE, KV());
#pragma unroll
            for (int r = 0; r < R; ++r) {
                Acc acc = (Acc)0;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc = fma(qr[r][e], kf[e], acc);
                dots[u * R + r] = acc;
            }
        }
        XRed<NV, LPR / 2, Acc>::run(dots, rl);
        if ((rl & kPlainMask) == 0) {
#pragma unroll
            for (int f = 0; f < F; ++f) {
                const int idx = base_idx + f;
                const int u = idx / R, r = idx % R;
                const int tok = base + u * step + sub;
                if (r < rows && tok < ntok) {
                    const int t = t0 + tok;
                    const int pq = pos0 + r / a.G;  // this row's query position
                    const bool ok = t <= pq && t >= window_start(pq, a.window);
                    s_sc[r * kMaxChunk + tok] = ok ? dots[f] : (Acc)-INFINITY;
                }
            }
        }
    }
    __syncthreads();

    // ---- chunk softmax statistics (one wave per row)
    for (int r = wave; r < rows; r += kNW) {
        Acc m = (Acc)-INFINITY;
        for (int i = lane; i < ntok; i += kWave) m = fmax(m, s_sc[r * kMaxChunk + i]);
        m = wave_max(m);
        Acc l = (Acc)0;
        for (int i = lane; i < ntok; i += kWave) {
            Acc sc = s_sc[r * kMaxChunk + i];
            Acc p = (m == (Acc)-INFINITY) ? (Acc)0 : exp_acc(sc - m);
            s_sc[r * kMaxChunk + i] = p;
            l += p;
        }
        l = wave_sum(l);
        if (lane == 0) {
            s_m[r] = m;
            s_l[r] = l;
        }
    }
    __syncthreads();

    // ---- PV
    Acc acc[R][EPL];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[r][e] = (Acc)0;
    for (int base = wave * TPW; base < ntok; base += step * U) {
        uint4 vv[U][NLD];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int tok = base + u * step + sub;
            if (tok < ntok) {
                const uint4* rp = row_ptr(a.v_pool, tok);
#pragma unroll
                for (int i = 0; i < NLD; ++i) vv[u][i] = rp[i * LPR + rl];
            } else {
#pragma unroll
                for (int i = 0; i < NLD; ++i) vv[u][i] = make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int tok = base + u * step + sub;
            if (tok < ntok) {
                Acc vf[EPL];
#pragma unroll
                for (int i = 0; i < NLD; ++i) unpack<Acc>(vv[u][i], vf + i * VE, KV());
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const Acc p = r < rows ? s_sc[r * kMaxChunk + tok] : (Acc)0;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[r][e] = fma(p, vf[e], acc[r][e]);
                }
            }
        }
    }
    // Token slots of one wave hold the same d range: fold them first.
#pragma unroll
    for (int o = LPR; o < kWave; o <<= 1)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[r][e] += __shfl_xor(acc[r][e], o);
    __syncthreads();  // all waves done reading probabilities: smem becomes red[R][D]

    // ---- waves add their sums into red[R][D] one after another
    Acc* red = smem;
    for (int w = 0; w < kNW; ++w) {
        if (wave == w && sub == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (r < rows) {
#pragma unroll
                    for (int i = 0; i < NLD; ++i) {
                        const int d0 = (i * LPR + rl) * VE;
                        Acc* dst = red + (size_t)r * D + d0;
#pragma unroll
                        for (int e = 0; e < VE; ++e)
                            dst[e] = (w == 0 ? (Acc)0 : dst[e]) + acc[r][i * VE + e];
                    }
                }
            }
        }
        __syncthreads();
    }

    const bool bad = s_flag != 0;
    if (nch == 1) {
        for (int idx = tid; idx < rows * D; idx += kNT) {
            const int r = idx / D, d = idx % D;
            Acc res = red[(size_t)r * D + d] / (s_l[r] + (Acc)1e-10);
            a.out[out_index(a, s, g, r, d, D)] = bad ? __builtin_nanf("") : (float)res;
        }
        return;
    }

    // Partial (m, l, o) of this chunk for each row.
    Acc* part_o = static_cast<Acc*>(a.part_o);
    Acc* part_ml = static_cast<Acc*>(a.part_ml);
    const size_t row_base = ((size_t)s * a.q_len) * a.Hq;  // first row of sequence s
    for (int idx = tid; idx < rows * D; idx += kNT) {
        const int r = idx / D, d = idx % D;
        const int j = r / a.G, h = g * a.G + r % a.G;
        const size_t prow = row_base + (size_t)j * a.Hq + h;
        part_o[(prow * a.max_chunks + c) * D + d] = red[(size_t)r * D + d];
    }
    if (tid < rows) {
        const int r = tid;
        const int j = r / a.G, h = g * a.G + r % a.G;
        const size_t prow = row_base + (size_t)j * a.Hq + h;
        part_ml[(prow * a.max_chunks + c) * 2 + 0] = bad ? (Acc)__builtin_nan("") : s_m[r];
        part_ml[(prow * a.max_chunks + c) * 2 + 1] = s_l[r];
    }

    // Last chunk of (s, g) merges.
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        int prev = atomicAdd(&a.counters[(size_t)s * a.Hkv + g], 1);
        s_last = (prev == nch - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    // Per row: global max M, any-NaN flag and 1 / (L + 1e-10); then the weighted sum of
    // the chunk outputs, with the weights e^(m_c - M) staged in LDS kWTile at a time.
    constexpr int kWTile = 256;
    static_assert(SMEM >= kWTile, "weight tile must fit the shared buffer");
    constexpr int DPT = (D + kNT - 1) / kNT;
    Acc* s_w = smem;
    for (int r = 0; r < rows; ++r) {
        const int j = r / a.G, h = g * a.G + r % a.G;
        const size_t prow = row_base + (size_t)j * a.Hq + h;
        const Acc* ml = part_ml + prow * a.max_chunks * 2;
        if (wave == 0) {
            Acc M = (Acc)-INFINITY;
            int nan = 0;
            for (int cc = lane; cc < nch; cc += kWave) {
                Acc m = ml[cc * 2];
                if (m != m) nan = 1;
                M = fmax(M, m);
            }
            M = wave_max(M);
            nan = __any(nan);
            Acc Ls = (Acc)0;
            for (int cc = lane; cc < nch; cc += kWave) {
                Acc m = ml[cc * 2];
                Acc w = (M == (Acc)-INFINITY || m == (Acc)-INFINITY) ? (Acc)0 : exp_acc(m - M);
                Ls += ml[cc * 2 + 1] * w;
            }
            Ls = wave_sum(Ls);
            if (lane == 0) {
                s_m[0] = nan ? (Acc)__builtin_nan("") : (Acc)1 / (Ls + (Acc)1e-10);
                s_l[0] = M;
            }
        }
        __syncthreads();
        const Acc M = s_l[0];
        const Acc invL = s_m[0];
        const Acc* po = part_o + prow * a.max_chunks * D;
        Acc oacc[DPT];
#pragma unroll
        for (int k = 0; k < DPT; ++k) oacc[k] = (Acc)0;
        for (int ct = 0; ct < nch; ct += kWTile) {
            const int cn = min(kWTile, nch - ct);
            for (int cc = tid; cc < cn; cc += kNT) {
                Acc m = ml[(ct + cc) * 2];
                s_w[cc] = (M == (Acc)-INFINITY || m == (Acc)-INFINITY) ? (Acc)0 : exp_acc(m - M);
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < DPT; ++k) {
                const int d = tid + k * kNT;
                if (d < D)
                    for (int cc = 0; cc < cn; ++cc)
                        oacc[k] = fma(s_w[cc], po[(size_t)(ct + cc) * D + d], oacc[k]);
            }
            __syncthreads();
        }
#pragma unroll
        for (int k = 0; k < DPT; ++k) {
            const int d = tid + k * kNT;
            if (d < D) a.out[out_index(a, s, g, r, d, D)] = (float)(oacc[k] * invL);
        }
        __syncthreads();
    }
    if (tid == 0) a.counters[(size_t)s * a.Hkv + g] = 0;
}


template <int D, typename KV, int R>
void launch(const AttendArgs& a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((attend_chunk_kernel<D, KV, R>), grid, dim3(kNT), 0, st, a);
}

template <int D, typename KV>
int32_t dispatch_rows(const AttendArgs& a, int rows, dim3 grid, hipStream_t st) {
    if (rows <= 1) launch<D, KV, 1>(a, grid, st);
    else if (rows <= 2) launch<D, KV, 2>(a, grid, st);
    else if (rows <= 4) launch<D, KV, 4>(a, grid, st);
    else if (rows <= 8) launch<D, KV, 8>(a, grid, st);
    else if constexpr (D <= 256) launch<D, KV, 16>(a, grid, st);
    else return fail(PKV_ERR_UNSUPPORTED, "head_dim 512 supports at most 8 query rows per kv head");
    return PKV_OK;
}

int32_t attend_impl(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                    const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                    const int32_t* pos, int32_t pos_scalar, int32_t q_len, int32_t batch,
                    int32_t max_pos, float* out, void* workspace, size_t workspace_bytes) {
    int32_t rc = validate_params(p);
    if (rc != PKV_OK) return rc;
    if (batch <= 0 || q_len <= 0 || table_stride <= 0 || max_pos < 0)
        return fail(PKV_ERR_INVALID, "batch, q_len, table_stride must be positive, max_pos >= 0");
    if (!q || !k_pool || !v_pool || !block_tables || !out || !workspace)
        return fail(PKV_ERR_INVALID, "null device pointer");
    const int G = p->num_heads / p->num_kv_heads;
    const int rows = G * q_len;
    if (rows > 16) return fail(PKV_ERR_UNSUPPORTED, "q_len * (num_heads / num_kv_heads) must be <= 16");
    AttendLayout lay = attend_layout(p, batch, q_len, max_pos);
    if (lay.chunk > kMaxChunk) return fail(PKV_ERR_UNSUPPORTED, "chunk larger than the kernel's LDS bound");
    if (workspace_bytes < lay.total)
        return fail(PKV_ERR_WORKSPACE, "workspace smaller than pkv_workspace_size()");
    if (batch > 65535 || p->num_kv_heads > 65535)
        return fail(PKV_ERR_INVALID, "batch and num_kv_heads must be <= 65535");
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
    a.chunk = lay.chunk;
    a.max_chunks = lay.max_chunks;
    a.counters = reinterpret_cast<int32_t*>(ws + lay.counters_off);
    a.part_ml = ws + lay.ml_off;
    a.part_o = ws + lay.o_off;
    a.out = out;
    dim3 grid(lay.max_chunks, p->num_kv_heads, batch);
    hipStream_t st = static_cast<hipStream_t>(stream);
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

}  // namespace
}  // namespace pkv

extern "C" {

int32_t pkv_attend(void* stream, const pkv_params* p, const float* q, const void* k_pool,
                   const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                   const int32_t* pos, int32_t q_len, int32_t batch, int32_t max_pos,
                   float* out, void* workspace, size_t workspace_bytes) {
    pkv::clear_error();
    if (!pos) return pkv::fail(PKV_ERR_INVALID, "pos is NULL");
    return pkv::attend_impl(stream, p, q, k_pool, v_pool, block_tables, table_stride, pos, 0,
                            q_len, batch, max_pos, out, workspace, workspace_bytes);
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
    (void)ring_base;
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
    // The table must cover pos (attention.mojo:271); the kernel checks against the
    // stride, so the stride is exactly the entries needed.
    int32_t stride = (pos < 0 ? 0 : pos / (block_size > 0 ? block_size : 1)) + 1;
    return pkv::attend_impl(stream, &p, q, k_pool, v_pool, block_table, stride, nullptr, pos, 1,
                            1, pos < 0 ? 0 : pos, attn_out, workspace, workspace_bytes);
}

}  // extern "C"
