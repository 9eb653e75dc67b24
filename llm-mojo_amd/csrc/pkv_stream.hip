// K2 hot path -- stream-K paged attention over whole pages (decode and verify).
//
// Replaces the reference's three-pass CPU loop (attention.mojo:151-294) for head_dim
// 256 or 512 with up to 8 query rows per KV head per launch (decode: G = Hq / Hkv rows;
// verify: G x the launch's queries; the host splits longer verifies into query groups).
// Keys come from block tables, rings (attention.mojo:264-269) or, for LSA, explicit key
// lists (lsa_core.mojo:630-680).
//
// Work split. The keys every sequence attends ([window_start(pos), pos + q_len - 1])
// are laid end to end, sequence after sequence, and cut into P consecutive runs, one per
// workgroup (P even, sized to fill the chip once), so every workgroup streams about the
// same number of bytes whatever the mix of context lengths. The runs go in pairs: pair
// (2p, 2p + 1) covers ceil(2 total / P) keys, the even workgroup 530/1024 of them.
// Workgroup w runs on XCD w % 8 (round-robin dispatch, read back from XCC_ID), and
// per-workgroup timestamps on config 2 show the odd XCDs streaming ~10% slower than the
// even ones at equal shares; the uneven split brings the two halves closer to finishing
// together (+1% on the decode and verify launches). A workgroup has one wave per KV head (up to 8): the waves walk the
// same tokens together, so the workgroup reads whole 16-token pages -- 16 rows of
// Hkv*D*elt contiguous bytes (128 KiB for fp32, 8 heads, D=256) -- instead of 1 KiB
// slices scattered over the pool. Where a run crosses a sequence boundary the wave
// finishes one sequence's piece and starts the next. Sequences covered by a single
// piece write their output directly; the others write (m, l, o) partials, combined by
// stream_merge_kernel (a second launch, so no device-scope fences are needed).
// Piece (w, s) of workgroup w and sequence s is stored at slot w + s: the pieces are
// ordered by both w and s, so w + s is unique and below P + batch.
//
// Per wave and batch of U tokens (one token per load instruction: 64 lanes x D/64
// elements, 16-byte loads for fp32, 8-byte for bf16):
//   1. the K and V rows of all U tokens are loaded first (addresses are wave-uniform:
//      page id by readlane from a register holding the piece's page ids, offsets in
//      scalar registers), so 2U loads are in flight together;
//   2. partial dots of U tokens x R rows reduced across the 64 lanes by a halving
//      exchange: permlane32/permlane16 swaps for the two wide levels, DPP inside rows
//      for the rest (no LDS traffic); afterwards lane l holds dot l / REP;
//   3. online softmax per row: batch max / sum over the lanes of a row by DPP
//      rotations and permlane swaps, one exponential per lane, the accumulators
//      rescaled only when a row's max moves;
//   4. PV: p broadcast by readlane, accumulated in registers.
// fp32 pools accumulate in double (scores, exponentials, PV, partials, merge) so the
// output is the exact attention rounded once to fp32 -- the reference fp32 path carries
// ~1e-7 absolute error of its own and the parity bound leaves no room for a second
// error of that size. On CDNA3/4 a non-packed double FMA issues at the fp32 rate.
// bf16 pools accumulate in fp32.
// fp32 pools with 5..8 query rows per KV head (verify) run stream_mfma_kernel instead:
// the same plan, pieces and partials, with QK^T and PV on the fp64 4x4x4 MFMA.
//
// Fused append (pkv_append_attend, vector kernel): every workgroup computes the block
// allocation of the call from the state as it stands (a prefix over the batch in LDS),
// copies its share of the appended rows into the pool and takes the new positions from
// k_new / v_new; the merge launch writes the new table entries, lengths, free count and
// status. The whole decode step of a layer is these two launches.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "pkv_internal.h"

namespace pkv {
namespace {

#ifndef PKV_STREAM_WAVES
#define PKV_STREAM_WAVES 8
#endif
#ifndef PKV_STREAM_PER_MIN
#define PKV_STREAM_PER_MIN 16
#endif

constexpr int kSW = 64;                          // wavefront
constexpr int kMaxWaves = PKV_STREAM_WAVES;      // KV heads handled by one workgroup
// merge kernel threads: one per element of a row (head_dim 256 or 512)
template <int D>
constexpr int merge_threads() { return D; }
constexpr int kPerMin = PKV_STREAM_PER_MIN;      // fewest keys per workgroup
#ifndef PKV_STREAM_EVEN_W
#define PKV_STREAM_EVEN_W 530
#endif
// Lead-in: every sequence's run in the key concatenation starts with this many keys that
// no piece reads, so a workgroup whose run crosses into a sequence is charged for that
// piece's start (its page-id and Q round trip before the first batch lands, and its
// partials) and takes that many fewer keys. Per kernel, in keys of its own batch rate:
// config 5's verify 125.5 -> 121.5 us (fp64), 72.9 -> 68.4 us (bf16); LSA 41.6 -> 39.6 us;
// config 2 unchanged. Larger values up to twice these measured the same. The interleaved
// fp64 layout (eight waves on one kv head, a cross-wave exchange at each piece's end) pays
// more per piece: config 5's verify 121.5 (16) / 118.2 (48) / 116.4-117.5 (96) /
// 116.3 (128) / 118.8 (192) / 122.3 us (256), four traced runs each; the interleaved bf16
// kernel (16-token batches) 71.5 (32) / 69.6 (64) / 68.8 (128) / 65.6-65.8 (256) /
// 64.7 (384) / 66.4 (512) / 67.7 us (768), three each.
#ifndef PKV_LEAD_VEC
#define PKV_LEAD_VEC 16
#endif
#ifndef PKV_LEAD_MFMA
#define PKV_LEAD_MFMA 16
#endif
#ifndef PKV_LEAD_BF16
#define PKV_LEAD_BF16 32
#endif
#ifndef PKV_LEAD_IW
#define PKV_LEAD_IW 128
#endif
#ifndef PKV_LEAD_VEC_IW
#define PKV_LEAD_VEC_IW 16
#endif
#ifndef PKV_LEAD_BF16_IW
#define PKV_LEAD_BF16_IW 384
#endif
constexpr int kEvenW = PKV_STREAM_EVEN_W;        // even workgroup's share of a pair, / 1024

template <typename KV>
struct SKV;
template <>
struct SKV<float> {
    using Acc = double;
    static constexpr int kElt = 4;
};
template <>
struct SKV<uint16_t> {  // bf16 bits
    using Acc = float;
    static constexpr int kElt = 2;
};

// Tokens per batch for R query rows (register budget: 2U loads in flight).
#ifndef PKV_STREAM_U32
#define PKV_STREAM_U32 8
#endif
#ifndef PKV_STREAM_U16
#define PKV_STREAM_U16 16
#endif
template <int D, typename KV, int R, bool SPARSE>
constexpr int batch_tokens() {
    constexpr int u0 = sizeof(KV) == 4 ? PKV_STREAM_U32 : PKV_STREAM_U16;  // D 256, R <= 2
    // D 512: the same bytes in flight per wave, except for fp32 key lists (LSA), whose
    // pieces are a few dozen keys: twice the tokens per batch halves their chain of
    // dependent loads (measured 41.4 -> 40.5 us at the LSA sizes).
    constexpr int u = D == 512 ? ((SPARSE && sizeof(KV) == 4) ? u0 : u0 / 2) : u0;
    return R <= 2 ? u : (R == 4 ? u / 2 : u / 4);
}

// Where a sequence's keys live: pages through its block table, its ring, or the pool
// rows of an explicit key list (sparse attention, no causal mask).
constexpr int kAddrPaged = 0;
constexpr int kAddrRing = 1;
constexpr int kAddrSparse = 2;

// ---- cross-lane primitives (wave64) -------------------------------------------------

template <int CTRL>
__device__ inline uint32_t dpp32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ inline float dpp(float v) {
    return __uint_as_float(dpp32<CTRL>(__float_as_uint(v)));
}
template <int CTRL>
__device__ inline double dpp(double v) {
    const uint32_t lo = dpp32<CTRL>((uint32_t)__double2loint(v));
    const uint32_t hi = dpp32<CTRL>((uint32_t)__double2hiint(v));
    return __hiloint2double((int)hi, (int)lo);
}

// DPP controls (within rows of 16 lanes).
constexpr int kRor8 = 0x128;        // l -> l ^ 8
constexpr int kHalfMirror = 0x141;  // l -> l ^ 7 (within 8)
constexpr int kQuadX2 = 0x4E;       // quad_perm [2,3,0,1]: l -> l ^ 2
constexpr int kQuadX1 = 0xB1;       // quad_perm [1,0,3,2]: l -> l ^ 1
template <int O>
constexpr int ror_ctrl() { return 0x120 + O; }  // row_ror:O

// v_permlane{32,16}_swap: lanes 32-63 (odd 16-lane rows) of `a` swap places with
// lanes 0-31 (even rows) of `b`. Afterwards a + b holds, in the lower lanes, a summed
// with its partner lane l ^ O and, in the upper lanes, b summed likewise.
template <int O>
__device__ inline void swap_u32(uint32_t& a, uint32_t& b) {
    if constexpr (O == 32) {
        auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
        a = r[0];
        b = r[1];
    } else {
        static_assert(O == 16, "swap levels are 32 and 16");
        auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
        a = r[0];
        b = r[1];
    }
}
template <int O>
__device__ inline void swap_halves(float& a, float& b) {
    uint32_t x = __float_as_uint(a), y = __float_as_uint(b);
    swap_u32<O>(x, y);
    a = __uint_as_float(x);
    b = __uint_as_float(y);
}
template <int O>
__device__ inline void swap_halves(double& a, double& b) {
    uint32_t al = (uint32_t)__double2loint(a), ah = (uint32_t)__double2hiint(a);
    uint32_t bl = (uint32_t)__double2loint(b), bh = (uint32_t)__double2hiint(b);
    swap_u32<O>(al, bl);
    swap_u32<O>(ah, bh);
    a = __hiloint2double((int)ah, (int)al);
    b = __hiloint2double((int)bh, (int)bl);
}

// Partner of lane l at level O of the halving exchange (O <= 8). At O = 4 the partner
// is l ^ 7, which also flips bits 0-1; the exchange stays correct because levels 2 and
// 1 afterwards sum over those bits completely.
template <int O, typename T>
__device__ inline T xpartner(T v) {
    if constexpr (O == 8) return dpp<kRor8>(v);
    else if constexpr (O == 4) return dpp<kHalfMirror>(v);
    else if constexpr (O == 2) return dpp<kQuadX2>(v);
    else return dpp<kQuadX1>(v);
}

// Sum of N values per lane over all 64 lanes by halving exchange. On return lane l
// holds the total of value index l / (64 / N) (N a power of two <= 64).
template <int N, int O, typename T>
__device__ inline void xred(T* v, int lane) {
    if constexpr (O == 0) {
        return;
    } else if constexpr (N == 1) {
        if constexpr (O >= 16) {
            T a = v[0], b = v[0];
            swap_halves<O>(a, b);
            v[0] = a + b;
        } else {
            v[0] += xpartner<O>(v[0]);
        }
        xred<1, O / 2>(v, lane);
    } else {
        constexpr int H = N / 2;
        if constexpr (O >= 16) {
#pragma unroll
            for (int i = 0; i < H; ++i) {
                T a = v[i], b = v[i + H];
                swap_halves<O>(a, b);
                v[i] = a + b;
            }
        } else {
            const bool upper = (lane & O) != 0;
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const T send = upper ? v[i] : v[i + H];
                const T keep = upper ? v[i + H] : v[i];
                v[i] = keep + xpartner<O>(send);
            }
        }
        xred<H, O / 2>(v, lane);
    }
}

// All-reduce over lane bits [log2(O0), 6) (the lanes that differ only in those bits):
// rotations inside 16-lane rows for the bits below 4, then the two swaps.
struct OpMax {
    template <typename T>
    __device__ T operator()(T a, T b) const { return fmax(a, b); }
};
struct OpSum {
    template <typename T>
    __device__ T operator()(T a, T b) const { return a + b; }
};
template <int O, int O0, typename T, typename Op>
__device__ inline T allreduce_rows(T x, Op op) {
    if constexpr (O > 8) {
        return x;
    } else {
        if constexpr (O >= O0) x = op(x, dpp<ror_ctrl<O>()>(x));
        return allreduce_rows<O * 2, O0>(x, op);
    }
}
template <int O0, typename T, typename Op>
__device__ inline T allreduce_hi(T x, Op op) {
    static_assert(O0 >= 1 && O0 <= 64, "offset");
    if constexpr (O0 < 64) {
        if constexpr (O0 <= 8) x = allreduce_rows<1, O0>(x, op);
        if constexpr (O0 <= 16) {
            T a = x, b = x;
            swap_halves<16>(a, b);
            x = op(a, b);
        }
        T a = x, b = x;
        swap_halves<32>(a, b);
        x = op(a, b);
    }
    return x;
}

__device__ inline double bcast(double v, int src) {
    const int lo = __builtin_amdgcn_readlane(__double2loint(v), src);
    const int hi = __builtin_amdgcn_readlane(__double2hiint(v), src);
    return __hiloint2double(hi, lo);
}
__device__ inline float bcast(float v, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}
__device__ inline int ufirst(int v) { return __builtin_amdgcn_readfirstlane(v); }
// Global-memory (address space 1) pointers for the device pass; the host pass only
// parses the kernels and keeps generic pointers.
#if defined(__HIP_DEVICE_COMPILE__)
#define PKV_GLOBAL __attribute__((address_space(1)))
#else
#define PKV_GLOBAL
#endif
typedef const PKV_GLOBAL char gchar;
// A wave-uniform address held in scalar registers, so a load adds only the 32-bit lane
// offset (global_load ... v_off, s[base]) instead of a 64-bit vector add per load.
__device__ inline gchar* uniform_ptr(const char* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<gchar*>(((uint64_t)hi << 32) | lo);
}

__device__ inline double exp_acc(double x) { return exp(x); }
__device__ inline float exp_acc(float x) { return expf(x); }


// ---- loads ------------------------------------------------------------------------

// NW 32-bit words per lane from a lane-contiguous run. NT: non-temporal loads (NT bit),
// for rows that one wave alone reads; rows that several waves of a head read in turn
// (WPH > 1) must stay in the L2 for the later waves (NT loads there doubled the LSA
// launch's time).
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
template <bool NT, typename T>
__device__ inline T ld(const PKV_GLOBAL T* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}
template <int NW, bool NT>
__device__ inline void load_words(gchar* p, uint32_t (&w)[NW]) {
    typedef const PKV_GLOBAL u32x4v g4;
    typedef const PKV_GLOBAL u32x2v g2;
    typedef const PKV_GLOBAL uint32_t g1;
    if constexpr (NW % 4 == 0) {
#pragma unroll
        for (int i = 0; i < NW / 4; ++i) {
            const u32x4v v = ld<NT>(reinterpret_cast<g4*>(p) + i);
            w[4 * i + 0] = v.x;
            w[4 * i + 1] = v.y;
            w[4 * i + 2] = v.z;
            w[4 * i + 3] = v.w;
        }
    } else if constexpr (NW == 2) {
        const u32x2v v = ld<NT>(reinterpret_cast<g2*>(p));
        w[0] = v.x;
        w[1] = v.y;
    } else {
        static_assert(NW == 1, "words per lane");
        w[0] = ld<NT>(reinterpret_cast<g1*>(p));
    }
}

template <typename A, int NW>
__device__ inline void unpack_words(const uint32_t (&w)[NW], A* out, float) {
#pragma unroll
    for (int i = 0; i < NW; ++i) out[i] = (A)__uint_as_float(w[i]);
}
template <typename A, int NW>
__device__ inline void unpack_words(const uint32_t (&w)[NW], A* out, uint16_t) {
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        out[2 * i] = (A)bf16_lo(w[i]);
        out[2 * i + 1] = (A)bf16_hi(w[i]);
    }
}

// ---- kernels ----------------------------------------------------------------------

struct StreamArgs {
    const float* q;
    const char* k_pool;
    const char* v_pool;
    const int32_t* tables;
    int32_t table_stride;
    const int32_t* pos;  // null -> pos_scalar (single sequence)
    int32_t pos_scalar;
    int32_t q_len;       // queries per sequence in q / out (their layout)
    const int32_t* q_lens;  // queries of each sequence (<= q_len), or null: q_len for all
    int32_t j0;          // first query of this launch
    int32_t q_cnt;       // queries of this launch
    const int32_t* keys;     // sparse: key positions, ragged by key_off [batch + 1]
    const int32_t* key_off;
    int32_t max_keys;
    int32_t Hq;
    int32_t Hkv;
    int32_t G;
    int32_t bs_shift;
    int32_t num_blocks;
    int32_t window;
    float scale;
    int32_t ring_size;  // > 0: ring pools (tables hold one ring slot per sequence)
    int64_t ring_base;  // ring mode, pos == null: first row of the sequence's ring
    int32_t max_pos;   // last query position the caller sized for
    int32_t batch;
    int32_t nwg;       // P: workgroups along the keys
    int32_t nwg_cap;   // at most this many (the workspace holds nwg_cap + batch slots)
    int32_t lead;      // keys of split work charged to each sequence's start (set by the launcher)
    int32_t rows_seq;  // Hq * q_cnt: workspace rows per sequence
    int32_t* plan;     // [0] per_pair, [1] even, [2 + s] key prefix of sequence s (s <= batch)
    void* part_ml;     // Acc (m, l) per (slot, row)
    void* part_o;      // Acc [D] per (slot, row)
    float* out;
    NewRows nr;        // fused append (paged, vector kernel); nr.k_new == NULL: none
};

// Queries of sequence s in this launch (the rest of its rows are left untouched).
__device__ inline int seq_queries(const StreamArgs& a, int s) {
    return a.q_lens ? min(max(a.q_lens[s] - a.j0, 0), a.q_cnt) : a.q_cnt;
}

__device__ inline size_t out_row(const StreamArgs& a, int s, int g, int r) {
    const int j = a.j0 + r / a.G, h = g * a.G + r % a.G;
    return ((size_t)s * a.q_len + j) * a.Hq + h;
}

// Fused append: the launch computes the block allocation itself from the state as it
// stands before the call. Its plan, in LDS and (from workgroup (0, 0)) in the workspace
// after the key plan, holds [0] the free count as read, [1, 1 + B) the table lengths,
// [1 + B, 2 + 2B) the exclusive prefix of the blocks each sequence needs (total last),
// [2 + 2B, 2 + 3B) the status before the pops.
__device__ inline int alloc_plan_ints(int batch) { return 3 * batch + 2; }
// Ints of a stream kernel's per-sequence LDS before the allocation plan: s_pre [batch + 1],
// s_lo [batch], s_meta [3 batch + 1].
__host__ __device__ constexpr int stream_seq_ints(int batch) { return 5 * batch + 2; }
__device__ inline bool fused_append(const StreamArgs& a) { return a.nr.k_new && a.j0 == 0; }

struct SeqAlloc {
    int len;      // blocks held before the call
    int granted;  // blocks popped for it
    int fc;       // free count (0 if the count read lies outside [0, num_blocks])
    int pref;     // its first pop: free_list[fc - 1 - pref]
    int code;     // status after the pops
};
__device__ inline SeqAlloc seq_alloc(const int* al, int batch, int num_blocks, int s) {
    const int fc_raw = al[0];
    const bool fc_bad = fc_raw < 0 || fc_raw > num_blocks;
    SeqAlloc r;
    r.fc = fc_bad ? 0 : fc_raw;
    r.len = al[1 + s];
    r.pref = al[1 + batch + s];
    const int need = al[2 + batch + s] - r.pref;
    r.granted = append_granted(need, r.fc, r.pref);
    r.code = append_pop_status(al[2 + 2 * batch + s], need, r.granted, fc_bad);
    return r;
}
// Whether the rows of a sequence with this status are copied (as scatter_kernel): OK, or
// BAD_BLOCK where each row is written only if its table entry lies in the pool.
__device__ inline bool new_rows_written(int code) {
    return code == PKV_SEQ_OK || code == PKV_SEQ_BAD_BLOCK;
}

// Key split: workgroups in pairs (2p, 2p + 1); pair p takes per_pair consecutive keys
// of the concatenation (each sequence's run preceded by its lead-in), its even workgroup
// the first `even` of them. The launchers make
// the workgroup count even (or 1, which takes every key).
struct KeySplit {
    int per_pair;
    int even;
    __device__ int start(int w) const { return (w >> 1) * per_pair + (w & 1) * even; }
    __device__ int owner(int k) const {  // the workgroup holding key k
        const int p = k / per_pair;
        return 2 * p + (k - p * per_pair >= even ? 1 : 0);
    }
};
__device__ inline KeySplit key_split(int total, int nwg) {
    KeySplit sp;
    if (nwg <= 1) {
        sp.per_pair = sp.even = max(total, 1);
        return sp;
    }
    const int pairs = nwg >> 1;
    sp.per_pair = max(2 * kPerMin, (total + pairs - 1) / pairs);
    sp.even = (int)(((long long)sp.per_pair * kEvenW + 1023) >> 10);
    return sp;
}

// Exclusive scan of the key counts in s_pre[0..batch) (in place, one wave), total in
// s_pre[batch].
__device__ inline void wave_scan_counts(int* s_pre, int batch, int lane) {
    int carry = 0;
    for (int base = 0; base < batch; base += kSW) {
        const int i = base + lane;
        const int v = i < batch ? s_pre[i] : 0;
        int incl = v;
#pragma unroll
        for (int o = 1; o < kSW; o <<= 1) {
            const int t = __shfl_up(incl, o);
            if (lane >= o) incl += t;
        }
        if (i < batch) s_pre[i] = carry + incl - v;
        carry += __shfl(incl, kSW - 1);
    }
    if (lane == 0) s_pre[batch] = carry;
}

// Key ranges of the launch, laid end to end: s_pre[s] = start of sequence s's run in the
// concatenation (its lead-in, then its keys; an empty sequence has neither; s_pre[batch] =
// total), s_lo[s] = its first key position, or -1
// (inactive: zeros), -2 (contract violation: NaN rows), -3 (no query of it in this
// launch). Workgroup (0, 0) also writes the merge plan and fills the rows of inactive and
// invalid sequences. Returns the key split.
// s_meta (meta_ints(batch) ints) keeps what the pieces need of each sequence, so a piece
// reads none of it from global memory: [s] its position (sparse: its list's first index),
// [batch + s] its query count in this launch, and with a fused append [2 batch + s] its
// first appended row (tok_off[s]; [3 batch] = tok_off[batch]).
// With a fused append, s_al (alloc_plan_ints(batch) ints) receives the allocation plan.
template <int D, int ADDR>
__device__ inline KeySplit stream_setup(const StreamArgs& a, int* s_pre, int* s_lo, int* s_meta,
                                        int* s_al) {
    constexpr bool RING = ADDR == kAddrRing;
    constexpr bool SPARSE = ADDR == kAddrSparse;
    const int tid = threadIdx.x;
    const int lane = tid & (kSW - 1);
    const int wave = ufirst(tid / kSW);
    const int nthr = blockDim.x;
    const int w = blockIdx.y;
    const int B = a.batch;
    const bool fused = fused_append(a);
    for (int i = tid; i < B; i += nthr) {
        int n = 0, lo = -1;
        if constexpr (SPARSE) {  // the list's indices; an empty list gives zeros
            const int kb = a.key_off[i], cnt = a.key_off[i + 1] - kb;
            if (cnt < 0 || cnt > a.max_keys || kb < 0) lo = -2;
            else if (cnt > 0) lo = 0, n = cnt;
            s_pre[i] = n > 0 ? n + a.lead : 0;
            s_lo[i] = lo;
            s_meta[i] = kb;
            s_meta[B + i] = seq_queries(a, i);
            continue;
        }
        const int p0 = a.pos ? a.pos[i] : a.pos_scalar;
        const int qlen = a.q_lens ? a.q_lens[i] : a.q_len;
        const int qc = seq_queries(a, i);
        s_meta[i] = p0;
        s_meta[B + i] = qc;
        if (qlen < 0 || qlen > a.q_len) {
            lo = -2;  // a query count outside the layout: NaN rows
        } else if (qc == 0) {
            lo = -3;  // no query of this sequence in this launch: nothing to do
        } else if (p0 >= 0) {
            const int hi = p0 + a.j0 + qc - 1;
            const int w0 = window_start(p0 + a.j0, a.window);
            bool ok = hi <= a.max_pos;
            if constexpr (RING) {
                // Every key of the call must still be in the ring (the reference aborts,
                // attention.mojo:265-266) -- the call's later queries have already written
                // theirs -- and the ring slot must lie in the pool.
                ok = ok && (p0 + qlen - 1) - w0 + 1 <= a.ring_size;
                if (a.pos) {
                    const int slot = a.tables[(size_t)i * a.table_stride];
                    ok = ok && slot >= 0 && slot < a.num_blocks;
                }
            } else {
                ok = ok && (hi >> a.bs_shift) < a.table_stride;
            }
            if (ok) {
                lo = w0;
                n = hi - lo + 1;
            } else {
                lo = -2;
            }
        }
        s_pre[i] = n > 0 ? n + a.lead : 0;
        s_lo[i] = lo;
        if (ADDR == kAddrPaged && fused) {
            const int len = a.nr.table_lens[i];
            const int need = append_blocks_needed(p0, a.nr.tok_off[i], a.nr.tok_off[i + 1],
                                                  a.nr.max_new, a.nr.total_rows,
                                                  1 << a.bs_shift, a.table_stride, len);
            s_al[1 + i] = len;
            s_al[1 + B + i] = need > 0 ? need : 0;
            s_al[2 + 2 * B + i] = need < 0 ? need : PKV_SEQ_OK;
            s_meta[2 * B + i] = a.nr.tok_off[i];
            if (i == B - 1) s_meta[3 * B] = a.nr.tok_off[B];
        }
    }
    if (ADDR == kAddrPaged && fused && tid == 0) s_al[0] = *a.nr.free_count;
    __syncthreads();
    if (wave == 0) {
        wave_scan_counts(s_pre, B, lane);
        if (ADDR == kAddrPaged && fused) wave_scan_counts(s_al + 1 + B, B, lane);
    }
    __syncthreads();

    const int total = ufirst(s_pre[B]);
    const KeySplit sp = key_split(total, a.nwg);
    if (w == 0 && blockIdx.x == 0) {
        // Plan for the merge launch; inactive sequences get zeros, contract violations NaN.
        if (tid == 0) {
            a.plan[0] = sp.per_pair;
            a.plan[1] = sp.even;
        }
        for (int i = tid; i <= B; i += nthr) a.plan[2 + i] = s_pre[i];
        if (ADDR == kAddrPaged && fused)  // for the state writes of the merge launch
            for (int i = tid; i < alloc_plan_ints(B); i += nthr) a.plan[B + 3 + i] = s_al[i];
        for (int s = 0; s < B; ++s) {
            const int lo = s_lo[s];
            if (lo >= 0 || lo == -3) continue;
            const float fill = lo == -1 ? 0.f : __builtin_nanf("");
            // rows of the sequence's queries; an invalid query count marks the whole group
            const bool qbad = a.q_lens && (a.q_lens[s] < 0 || a.q_lens[s] > a.q_len);
            const int nrow = (qbad ? a.q_cnt : seq_queries(a, s)) * a.Hq;
            float* o = a.out + ((size_t)s * a.q_len + a.j0) * a.Hq * D;
            for (int i = tid; i < nrow * D; i += nthr) o[i] = fill;
        }
    }
    return sp;
}

// Fused append: the appended rows (NewRows) of sequences w, w + nwg, ... go into the pool
// from workgroup w, the first wave of each kv head copying that head's slice, with the
// checks of scatter_kernel (pkv_state.hip): a sequence is copied when its allocation
// gives OK or BAD_BLOCK, and a row whose block is neither held nor granted, or whose
// table entry lies outside the pool, is skipped. The block of a row comes from the plan
// (held: the table, granted: the free list), so this launch reads no state it writes.
template <int D, typename KV, int WPH>
__device__ inline void copy_new_rows(const StreamArgs& a, const int* s_meta, const int* s_al,
                                     int g_first, int wave, int lane, int w) {
    constexpr int kElt = SKV<KV>::kElt;
    constexpr int kVec = D * kElt / 16;  // 16-byte vectors per head slice
    const int g = g_first + wave / WPH;
    if (wave % WPH != 0 || g >= a.Hkv) return;
    const size_t row_bytes = (size_t)a.Hkv * D * kElt;
    const size_t head_off = (size_t)g * D * kElt;
    const int bs_mask = (1 << a.bs_shift) - 1;
    const int B = a.batch;
    for (int s = w; s < B; s += a.nwg) {
        const int p0 = s_meta[s];
        const int r0 = s_meta[2 * B + s];
        const int n = s_meta[2 * B + s + 1] - r0;
        const SeqAlloc al = seq_alloc(s_al, B, a.num_blocks, s);
        if (!new_rows_written(al.code) || p0 < 0 || n <= 0) continue;
        if (al.len > a.table_stride) continue;  // a length outside the table: BAD_BLOCK
        const int32_t* table = a.tables + (size_t)s * a.table_stride;
        for (int b = 0; b < n; ++b) {
            const int p = p0 + b;
            const int blk = p >> a.bs_shift;
            // the row's values are requested with its block's table entry (one round trip)
            const size_t src = ((size_t)r0 + b) * row_bytes + head_off;
            const uint4* ks = reinterpret_cast<const uint4*>(a.nr.k_new + src);
            const uint4* vs = reinterpret_cast<const uint4*>(a.nr.v_new + src);
            uint4 kv[(kVec + kSW - 1) / kSW], vv[(kVec + kSW - 1) / kSW];
#pragma unroll
            for (int j = 0; j < (kVec + kSW - 1) / kSW; ++j) {
                const int i = min(lane + j * kSW, kVec - 1);
                kv[j] = ks[i];
                vv[j] = vs[i];
            }
            const int phys = append_block_entry(table, a.nr.free_list, al.len, al.granted,
                                                al.fc, al.pref, blk);
            if (phys < 0 || phys >= a.num_blocks) continue;
            const size_t dst = (((size_t)phys << a.bs_shift) | (size_t)(p & bs_mask)) * row_bytes + head_off;
            uint4* kd = reinterpret_cast<uint4*>(a.nr.k_dst + dst);
            uint4* vd = reinterpret_cast<uint4*>(a.nr.v_dst + dst);
#pragma unroll
            for (int j = 0; j < (kVec + kSW - 1) / kSW; ++j) {
                const int i = lane + j * kSW;
                if (i < kVec) {
                    kd[i] = kv[j];
                    vd[i] = vv[j];
                }
            }
        }
    }
}

// R query rows per wave; WPH waves per KV head split the head's rows (WPH = 2 gives two
// waves of R rows each, reading the same K/V: the second read of a row slice hits the cache).
// ADDR: kAddrPaged, kAddrRing (key t at row ring_base + t % ring_size) or kAddrSparse.
// Vector kernel, interleaved waves: the exchange area after the per-sequence ints (and a
// fused append's plan): m [8 waves][4 rows], 8 bad flags, then four regions of a wave's
// accumulators (at most 4 rows x 4 doubles per lane) and its rows' l.
constexpr int kVecRedM = 8 * 4 * 8;
constexpr int kVecRedO = kVecRedM + 64;
constexpr int kVecRedRegion = 4 * 4 * 8 * 64 + 64;
__host__ __device__ constexpr size_t vec_red_offset(int batch, bool fused) {
    return ((size_t)(stream_seq_ints(batch) + (fused ? 3 * batch + 2 : 0)) * sizeof(int) + 15) & ~(size_t)15;
}
__host__ __device__ constexpr size_t vec_red_bytes() { return kVecRedO + 4 * (size_t)kVecRedRegion; }

// IW (interleaved waves; head_dim 256, one wave per kv head, paged or ring keys): grid
// (nwg, Hkv), the eight waves of a workgroup take the batches of one kv head's pieces in
// turn and combine their (m, l, acc) through LDS at each piece's end, as the fp64 MFMA
// kernel's interleaved form does; a piece then leaves one partial per kv head. The
// accumulators are a few KiB per wave, so the exchange runs right after the piece's last
// batch. Against one wave per kv head (same box): config 2 209.3-211.0 -> 205.9 us per
// launch (sliding layer 81.5 -> 78.7, global 322.9 -> 318.6 us in the trace), config 3
// 355.8-356.6 -> 346.1-347.4 us, config 5's step 1.098-1.100 -> 1.073-1.080 ms (its MTP
// reads); lead-in 16 / 64 / 128 / 256 keys on config 2: 205.9 / 205.8-205.9 / 206.1-206.4 /
// 209.7 us.
template <int D, typename KV, int R, int WPH, int ADDR, bool IW = false>
__global__ __launch_bounds__(kMaxWaves * kSW) void stream_attend_kernel(StreamArgs a) {
    using Acc = typename SKV<KV>::Acc;
    constexpr int kElt = SKV<KV>::kElt;
    constexpr int EPL = D / kSW;                // elements per lane per token
    constexpr int NWD = EPL * kElt / 4;         // 32-bit words per lane per token
    constexpr int U = batch_tokens<D, KV, R, ADDR == kAddrSparse>();  // tokens per batch
    constexpr bool RING = ADDR == kAddrRing;
    constexpr bool SPARSE = ADDR == kAddrSparse;
    constexpr int NV = U * R;                   // dots per batch
    static_assert(NV <= kSW && (NV & (NV - 1)) == 0, "dots per batch: power of two <= 64");
    constexpr int REP = kSW / NV;               // lanes holding the same reduced dot
    constexpr int ROWB = R * REP;               // lane offset of the first token bit

    extern __shared__ int smem[];
    int* s_pre = smem;                  // [batch + 1]
    int* s_lo = smem + a.batch + 1;     // [batch]: window start, -1 inactive, -2 bad
    int* s_meta = smem + 2 * a.batch + 1;             // [3 batch + 1] (stream_setup)
    int* s_al = smem + stream_seq_ints(a.batch);      // fused append: the allocation plan

    const int tid = threadIdx.x;
    const int lane = tid & (kSW - 1);
    const int wave = ufirst(tid / kSW);
    const int w = IW ? blockIdx.x : blockIdx.y;  // the workgroup's key range
    const int B = a.batch;
    constexpr bool PAGED = ADDR == kAddrPaged;
    static_assert(!IW || (WPH == 1 && D == 256 && ADDR != kAddrSparse), "interleaved waves");

    const KeySplit sp = stream_setup<D, ADDR>(a, s_pre, s_lo, s_meta, s_al);
    const bool fused = PAGED && fused_append(a);
    if (fused) {
        if constexpr (IW) copy_new_rows<D, KV, kMaxWaves>(a, s_meta, s_al, blockIdx.y, wave, lane, w);
        else copy_new_rows<D, KV, WPH>(a, s_meta, s_al, blockIdx.x * (kMaxWaves / WPH), wave, lane, w);
    }
    const int total = ufirst(s_pre[B]);
    const int k0 = sp.start(w);
    if (k0 >= total) return;
    const int k1 = min(total, sp.start(w + 1));
    // this wave's KV head (IW: the workgroup's, whose pieces wave 0 stores)
    const int g = IW ? (int)blockIdx.y : blockIdx.x * (kMaxWaves / WPH) + wave / WPH;
    const int rb = IW ? 0 : (wave % WPH) * R;  // first of this wave's rows of the head
    if (g >= a.Hkv) return;
    // IW: the waves' exchange area, after the per-sequence ints (and the allocation plan)
    char* const red = reinterpret_cast<char*>(smem) + vec_red_offset(B, fused);

    const int rows = a.G * a.q_cnt;
    const size_t row_bytes = (size_t)a.Hkv * D * kElt;
    const char* kbase = a.k_pool + (size_t)g * D * kElt;  // wave-uniform
    const char* vbase = a.v_pool + (size_t)g * D * kElt;
    const uint32_t lane_off = (uint32_t)lane * EPL * kElt;
    const int bs_mask = (1 << a.bs_shift) - 1;

    // lane -> (token u_own, row r_own) of the reduced dot it holds
    const int idx_own = lane / REP;
    const int r_own = idx_own % R;
    const int u_own = idx_own / R;
    const bool row_live = rb + r_own < rows;

    // first sequence with s_pre[s] <= k0 < s_pre[s + 1]
    int s = 0;
    {
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (ufirst(s_pre[mid]) <= k0) lo = mid;
            else hi = mid - 1;
        }
        s = lo;
    }
    int pre_s = -1, pre_raw = 0;  // paged: the next piece's first page ids (pre_s: its sequence)
    for (; s < B; ++s) {
        const int ps = ufirst(s_pre[s]);
        const int pe = ufirst(s_pre[s + 1]);
        if (ps >= k1) break;
        if (pe == ps) continue;
        const int psr = ps + a.lead;  // the sequence's first key after its lead-in
        if (psr >= k1) break;
        const int lo_key = ufirst(s_lo[s]);
        const int ta = lo_key + max(k0, psr) - psr;  // first key of the piece
        const int tb = lo_key + min(k1, pe) - psr;   // one past the last
        const bool single = sp.owner(psr) == sp.owner(pe - 1);
        const int32_t* trow = a.tables + (size_t)s * a.table_stride;
        const int last_page = (tb - 1) >> a.bs_shift;
        // the sequence's position (sparse: its list's first index) and query count, from
        // the setup's LDS copy
        const int kbeg = SPARSE ? ufirst(s_meta[s]) : 0;
        const int pos0 = SPARSE ? 0 : ufirst(s_meta[s]);
        const int rows_s = a.G * ufirst(s_meta[B + s]);  // this sequence's live rows
        const bool live_own = row_live && rb + r_own < rows_s;
        int pgbase = -kSW;  // page index (sparse: list index) held by lane 0 of vpg
        int vpg = 0;
        // NaN rows: a table entry outside the pool, or (fused append) a sequence whose append
        // fails -- OUT_OF_BLOCKS, TABLE_FULL, BAD_ARGS, BAD_BLOCK from a free count out of
        // range. The engine skips the attention of such a sequence
        // (model_speculative_moe_batched.mojo:1989-1992); its pieces still run, so the key
        // split of the others is that of the separate calls.
        bool bad = false;
        // Fused append: table indices [g_lo, g_hi) are the blocks granted in this call, whose
        // entries the merge launch writes: their ids come from the free list (g_top - index).
        int g_lo = INT32_MAX, g_hi = INT32_MIN, g_top = 0;
        if (fused) {
            const SeqAlloc al = seq_alloc(s_al, B, a.num_blocks, s);
            g_lo = ufirst(al.len);
            g_hi = g_lo + ufirst(al.granted);
            g_top = ufirst(al.fc) - 1 - ufirst(al.pref) + g_lo;
            bad = ufirst(al.code) != PKV_SEQ_OK;  // a failed append: NaN rows (see below)
        }
        // Pool rows of the 64 keys from t on: sparse, lane l reads listed key t + l and its
        // block's table entry; paged, lane l reads the page id of page (t >> bs_shift) + l.
        auto load_pages = [&](int t) {
            if constexpr (SPARSE) {
                pgbase = t;
                int row = 0;
                if (t + lane < tb) {
                    const int key = a.keys[kbeg + t + lane];
                    const int blk = key >> a.bs_shift;
                    const int phys = (key >= 0 && blk < a.table_stride) ? trow[blk] : -1;
                    if (phys < 0 || phys >= a.num_blocks) bad = true;
                    else row = (phys << a.bs_shift) | (key & bs_mask);
                }
                vpg = row;
            } else if constexpr (ADDR == kAddrPaged) {
                pgbase = t >> a.bs_shift;
                int b = 0;
                if (pgbase + lane <= last_page) {
                    const int pg = pgbase + lane;
                    b = (pg >= g_lo && pg < g_hi) ? a.nr.free_list[g_top - pg] : trow[pg];
                    if (b < 0 || b >= a.num_blocks) {
                        bad = true;
                        b = 0;
                    }
                }
                vpg = b;
            }
        };

        // The piece's first loads are all requested before any of them is used, so they
        // share one round trip: the first 64 page ids (sparse: listed keys) and the query
        // rows. Every load is issued (indices clamped into range; the values of lanes past
        // the piece or of rows past `rows` are not used), so no branch separates a load from
        // its use.
        int first_raw = 0;
        if constexpr (SPARSE) {
            pgbase = ta;
            first_raw = a.keys[kbeg + min(ta + lane, tb - 1)];
        } else if constexpr (ADDR == kAddrPaged) {
            pgbase = ta >> a.bs_shift;
            const int pg = min(pgbase + lane, last_page);
            const int32_t* src = (pg >= g_lo && pg < g_hi) ? a.nr.free_list + (g_top - pg) : trow + pg;
            first_raw = pre_s == s ? pre_raw : *src;
        }
        asm volatile("" ::: "memory");  // issued before the query rows
        float qraw[R][EPL];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float* qp = a.q + out_row(a, s, g, min(rb + r, rows - 1)) * D + lane * EPL;
#pragma unroll
            for (int e = 0; e < EPL; e += 2) {
                const float2 v = *reinterpret_cast<const float2*>(qp + e);
                qraw[r][e] = v.x;
                qraw[r][e + 1] = v.y;
            }
        }
        // Paged: the next sequence's first 64 page ids, for its piece after this one (a piece
        // starts at its sequence's first key), requested with this piece's first loads.
        if (ADDR == kAddrPaged && s + 1 < B && ufirst(s_pre[s + 1]) + a.lead < k1 &&
            ufirst(s_pre[s + 2]) > ufirst(s_pre[s + 1])) {
            const int lo_n = ufirst(s_lo[s + 1]);
            const int tb_n = lo_n + min(k1, ufirst(s_pre[s + 2])) - ufirst(s_pre[s + 1]) - a.lead;
            const int pg = min((lo_n >> a.bs_shift) + lane, (tb_n - 1) >> a.bs_shift);
            const int32_t* src = a.tables + (size_t)(s + 1) * a.table_stride + pg;
            if (fused) {  // the blocks granted to it come from the free list
                const SeqAlloc al = seq_alloc(s_al, B, a.num_blocks, s + 1);
                const int n_lo = ufirst(al.len), n_hi = n_lo + ufirst(al.granted);
                const int n_top = ufirst(al.fc) - 1 - ufirst(al.pref) + n_lo;
                if (pg >= n_lo && pg < n_hi) src = a.nr.free_list + (n_top - pg);
            }
            pre_raw = *src;
            pre_s = s + 1;
        }
        asm volatile("" ::: "memory");  // the query rows go out before the table lookup
        // (branch-free from here on, so the compiler does not move a load into a branch)
        if constexpr (SPARSE) {  // the listed keys' table entries (one more round trip)
            const int key = first_raw;
            const int blk = key >> a.bs_shift;
            const bool in_table = key >= 0 && blk < a.table_stride;
            const int ent = trow[in_table ? blk : 0];
            const int phys = in_table ? ent : -1;
            const bool lane_ok = ta + lane < tb;
            const bool id_ok = phys >= 0 && phys < a.num_blocks;
            bad = bad || (lane_ok && !id_ok);
            vpg = lane_ok && id_ok ? (phys << a.bs_shift) | (key & bs_mask) : 0;
        } else if constexpr (ADDR == kAddrPaged) {
            const bool lane_ok = pgbase + lane <= last_page;
            const bool id_ok = first_raw >= 0 && first_raw < a.num_blocks;
            bad = bad || (lane_ok && !id_ok);
            vpg = lane_ok && id_ok ? first_raw : 0;
        }
        // Query rows -> registers (scaled); rows beyond `rows` are scaled by zero (a product,
        // not a select: the compiler would move the load into a branch for the select).
        Acc qr[R][EPL];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const Acc sc = rb + r < rows ? (Acc)a.scale : (Acc)0;
#pragma unroll
            for (int e = 0; e < EPL; ++e) qr[r][e] = (Acc)qraw[r][e] * sc;
        }
        // query position of my row and its first key (sparse: every listed key)
        const int pq_own = SPARSE ? INT32_MAX : pos0 + a.j0 + (rb + r_own) / a.G;
        const int ws_own = SPARSE ? 0 : window_start(pq_own, a.window);

        Acc m_own = (Acc)-INFINITY, l_own = (Acc)0;
        Acc acc[R][EPL];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[r][e] = (Acc)0;

        int64_t rbase = 0;  // ring mode: first row of the sequence's ring
        int r0 = 0;         // ring mode: ring row of key ta
        if constexpr (RING) {
            rbase = a.pos ? (int64_t)ufirst(trow[0]) * a.ring_size : a.ring_base;
            r0 = ta % a.ring_size;
        }
        // Fused append: positions [pn_lo, pn_hi) come from k_new / v_new (row r0 + t - pos).
        int pn_lo = INT32_MAX, pn_hi = INT32_MIN, nr0 = 0;
        if (fused) {
            const int r0 = ufirst(s_meta[2 * B + s]);
            const int n = ufirst(s_meta[2 * B + s + 1]) - r0;
            const SeqAlloc al = seq_alloc(s_al, B, a.num_blocks, s);
            if (new_rows_written(ufirst(al.code)) && pos0 >= 0 && n > 0) {
                pn_lo = pos0;
                pn_hi = pos0 + n;
                nr0 = r0;
            }
        }

        constexpr int kStepT = IW ? kMaxWaves * U : U;  // from one of a wave's batches to the next
        for (int t = IW ? ta + U * wave : ta; t < tb; t += kStepT) {
            const int tl = min(t + U - 1, tb - 1);
            if (SPARSE && tl - pgbase >= kSW) load_pages(t);  // the next 64 listed keys
            if (ADDR == kAddrPaged && (tl >> a.bs_shift) - pgbase >= kSW) load_pages(t);  // next 64 pages
            // K and V rows of the batch, all in flight together (tokens past the piece
            // re-read its last row and are masked).
            uint32_t kw[U][NWD], vw[U][NWD];
            auto row_off = [&](int tt) -> size_t {
                if constexpr (RING) {
                    return (size_t)ring_key_row(rbase, r0, tt - ta, a.ring_size) * row_bytes;
                } else if constexpr (SPARSE) {
                    return (size_t)(uint32_t)__builtin_amdgcn_readlane(vpg, tt - pgbase) * row_bytes;
                } else {
                    const int page = __builtin_amdgcn_readlane(vpg, (tt >> a.bs_shift) - pgbase);
                    return (((size_t)page << a.bs_shift) | (size_t)(tt & bs_mask)) * row_bytes;
                }
            };
            if (ADDR == kAddrPaged && t + U > pn_lo && t < pn_hi) {
                // the batch holding appended rows (fused append): those come from k_new / v_new
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int tt = min(t + u, tb - 1);
                    const bool fresh = tt >= pn_lo && tt < pn_hi;
                    const size_t off = fresh ? (size_t)(nr0 + (tt - pn_lo)) * row_bytes : row_off(tt);
                    const char* kb = fresh ? a.nr.k_new + (size_t)g * D * kElt : kbase;
                    const char* vb = fresh ? a.nr.v_new + (size_t)g * D * kElt : vbase;
                    load_words<NWD, WPH == 1>(uniform_ptr(kb + off) + lane_off, kw[u]);
                    load_words<NWD, WPH == 1>(uniform_ptr(vb + off) + lane_off, vw[u]);
                }
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const size_t off = row_off(min(t + u, tb - 1));
                    load_words<NWD, WPH == 1>(uniform_ptr(kbase + off) + lane_off, kw[u]);
                    load_words<NWD, WPH == 1>(uniform_ptr(vbase + off) + lane_off, vw[u]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);  // keep all 2U loads ahead of the math
            // scores
            Acc dots[NV];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                Acc kf[EPL];
                unpack_words<Acc, NWD>(kw[u], kf, KV());
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    Acc d = (Acc)0;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) d = fma(qr[r][e], kf[e], d);
                    dots[u * R + r] = d;
                }
            }
            xred<NV, kSW / 2>(dots, lane);
            const int t_own = t + u_own;
            const bool ok = live_own && t_own < tb && t_own <= pq_own && t_own >= ws_own;
            const Acc sc = ok ? dots[0] : (Acc)-INFINITY;
            const Acc mb = allreduce_hi<ROWB>(sc, OpMax());
            const bool moved = mb > m_own + (Acc)kLazyMove;  // m_own = -inf: any live key
            const Acc m_new = moved ? mb : m_own;
            const Acc p_own = ok ? exp_acc(sc - m_new) : (Acc)0;
            const Acc lb = allreduce_hi<ROWB>(p_own, OpSum());
            Acc scl = (Acc)1;
            if (moved) scl = exp_acc(m_own - m_new);  // m_own = -inf gives 0
            l_own = l_own * scl + lb;
            m_own = m_new;
            if (__any(moved)) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const Acc f = bcast(scl, r * REP);
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[r][e] *= f;
                }
            }
            // PV
#pragma unroll
            for (int u = 0; u < U; ++u) {
                Acc vf[EPL];
                unpack_words<Acc, NWD>(vw[u], vf, KV());
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const Acc p = bcast(p_own, (u * R + r) * REP);
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[r][e] = fma(p, vf[e], acc[r][e]);
                }
            }
        }
        bad = __any(bad);

        if constexpr (IW) {
            // The waves' rows into wave 0's: the rows' common max, then the rescaled acc and l
            // summed in three rounds (waves 4-7 into 0-3, 2-3 into 0-1, 1 into 0). The branches
            // are uniform over the workgroup, so every wave meets the same barriers.
            const int nb = (tb - ta + U - 1) / U;  // batches of the piece
            if (nb > 1) {
                Acc* rm = reinterpret_cast<Acc*>(red);                      // m of [wave][row]
                int* rbad = reinterpret_cast<int*>(red + kVecRedM);         // [wave]
                if (lane == r_own * REP && u_own == 0) rm[wave * 4 + r_own] = m_own;
                if (lane == 0) rbad[wave] = bad ? 1 : 0;
                __syncthreads();
                bool any_bad = false;
                Acc M = (Acc)-INFINITY;
#pragma unroll
                for (int v = 0; v < kMaxWaves; ++v) {
                    any_bad = any_bad || rbad[v] != 0;
                    M = fmax(M, rm[v * 4 + r_own]);
                }
                bad = any_bad;
                const Acc f_own = m_own == (Acc)-INFINITY ? (Acc)0 : exp_acc(m_own - M);
                l_own *= f_own;
                m_own = M;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const Acc f = bcast(f_own, r * REP);
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[r][e] *= f;
                }
                // Region: element (r, e) of lane L at Acc index (r EPL + e) 64 + L, then l [row]
                auto region = [&](int i) { return reinterpret_cast<Acc*>(red + kVecRedO + (size_t)i * kVecRedRegion); };
                auto put = [&](int i) {
                    Acc* ro = region(i);
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int e = 0; e < EPL; ++e) ro[(r * EPL + e) * kSW + lane] = acc[r][e];
                    if (lane == r_own * REP && u_own == 0) ro[R * EPL * kSW + r_own] = l_own;
                };
                auto add = [&](int i) {
                    const Acc* ro = region(i);
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int e = 0; e < EPL; ++e) acc[r][e] += ro[(r * EPL + e) * kSW + lane];
                    l_own += ro[R * EPL * kSW + r_own];
                };
                if (nb > 4) {  // waves 4-7 into 0-3 (regions 0-3)
                    if (wave >= 4) put(wave - 4);
                    __syncthreads();
                    if (wave < 4) add(wave);
                }
                if (nb > 2) {  // waves 2, 3 into 0, 1 (regions 2, 3, which only they read before)
                    if (wave == 2 || wave == 3) put(wave);
                    __syncthreads();
                    if (wave < 2) add(wave + 2);
                }
                if (wave == 1) put(1);  // wave 1 into 0 (region 1, which only wave 1 read before)
                __syncthreads();
                if (wave == 0) add(1);
            }
        }
        if (IW && wave != 0) {
            // every wave but 0 has handed its rows over
        } else if (single) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (rb + r < rows_s) {
                    const Acc inv = (Acc)1 / (bcast(l_own, r * REP) + (Acc)1e-10);
                    float* op = a.out + out_row(a, s, g, rb + r) * D + lane * EPL;
#pragma unroll
                    for (int e = 0; e < EPL; e += 2) {
                        float2 v;
                        v.x = bad ? __builtin_nanf("") : (float)(acc[r][e] * inv);
                        v.y = bad ? __builtin_nanf("") : (float)(acc[r][e + 1] * inv);
                        *reinterpret_cast<float2*>(op + e) = v;
                    }
                }
            }
        } else {
            const size_t slot = (size_t)(w + s) * a.rows_seq;
            Acc* po = static_cast<Acc*>(a.part_o);
            Acc* pml = static_cast<Acc*>(a.part_ml);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (rb + r < rows) {
                    const int row = ((rb + r) / a.G) * a.Hq + g * a.G + (rb + r) % a.G;
                    Acc* dst = po + (slot + row) * D + lane * EPL;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) dst[e] = acc[r][e];
                    if (lane == r * REP) {
                        pml[(slot + row) * 2 + 0] = bad ? (Acc)__builtin_nan("") : m_own;
                        pml[(slot + row) * 2 + 1] = l_own;
                    }
                }
            }
        }
    }
}

// ---- fp64 MFMA path: fp32 pools, head_dim 256 or 512, 5..8 query rows per KV head --------
//
// v_mfma_f64_4x4x4_4b computes four independent 4x4x4 double products per instruction
// at the full fp64 rate. Lane l = 4b + x + 16y holds block b's elements (b = lane bits
// 2-3); inside a block (layouts checked on the device) A[i][k] sits at x = i, y = k,
// B[k][j] at x = j, y = k, and C[i][j] at x = j, y = i. WPH waves per KV head split its
// rows; each wave's rows form RG groups of 4 (row rb + 4rg + x of lane x). head_dim 256:
// one wave of 8 rows (RG 2); head_dim 512 (the engine's 16q/2kv global layers): two waves
// of 4 rows (RG 1), which keeps the accumulators of a wave at 32 doubles per lane.
//   S^T = K Q^T for each group of 4 tokens tg and row group rg: A = K (x = token, y = d
//     slot), B = Q (x = row, y = d slot). Over the steps (q, e) block b contracts
//     d = 64q + 16b + 4y + e, so the four blocks hold partial sums over disjoint d, added
//     by two DPP rotations. Lane (b, x, y) then holds S[row 4rg + x][token 4tg + y] --
//     the B operand of PV as it stands.
//   O^T += V^T P^T: A = V (x = d slot, y = token), B = P; tile (rg, q, e) of lane
//     (b, x, y) accumulates O[4rg + x][64q + 16b + 4y + e].
// Each load moves 16 bytes per lane of one token's row slice (64 lanes: 1 KiB), so a
// head_dim-512 slice takes two. Products of fp32 values are exact in double and every
// sum is a double sum, as in the vector path; the matrix cores take the 2 x rows x D
// multiply-adds per token off the vector ALUs, and the dot products need no cross-lane
// reduction beyond the block sum.
// Fused append (pkv_append_attend): as the vector kernel -- the allocation plan from the
// state as it stands, the appended rows copied into the pool by the launch and read from
// k_new / v_new, the state written by the merge launch.
typedef __attribute__((address_space(3))) void lds_void;
// s_waitcnt with only lgkmcnt = 0 (vmcnt and expcnt at their maxima).
constexpr int kLgkm0 = 0xC07F;
// LDS of the MFMA kernel: s_pre / s_lo / s_meta (and the allocation plan of a fused
// append), then one staging area per wave.
__host__ __device__ constexpr size_t mfma_stage_offset(int batch, bool fused) {
    return ((size_t)(stream_seq_ints(batch) + (fused ? 3 * batch + 2 : 0)) * sizeof(int) + 15) &
           ~(size_t)15;
}
// One token's row slice plus 16 bytes of bank padding.
__host__ __device__ constexpr int mfma_slot(int D) { return D * 4 + 16; }
__host__ __device__ constexpr size_t mfma_stage_bytes(int D, int tg) {
    return (size_t)tg * 8 * mfma_slot(D);
}

__device__ inline double mfma4(double a, double b, double c) {
    return __builtin_amdgcn_mfma_f64_4x4x4f64(a, b, c, 0, 0, 0);
}
// Sum over the four blocks (lane bits 2-3) in every lane.
__device__ inline double block_sum(double v) {
    v += dpp<ror_ctrl<4>()>(v);
    return v + dpp<ror_ctrl<8>()>(v);
}

// LDS reads the compiler does not track. It cannot tell which LDS words a direct-to-LDS
// copy in flight writes, so before any LDS read it sees it waits for every copy
// (vmcnt(0)) -- including the next batch's, which must stay in flight. These reads are
// inline assembly, and lgkm_tie0 ties their values to an explicit s_waitcnt lgkmcnt(0),
// so no use is scheduled above it.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ inline uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_void*)p; }
template <int OFF>
__device__ inline i32x4 lds_b128(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    i32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
template <int OFF>
__device__ inline double lds_r64(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    double v;
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
template <int OFF>
__device__ inline int lds_r32(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    int v;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
// Untracked LDS writes (as the reads above; ordered with them by the wave's LDS queue).
__device__ inline void lds_w128(uint32_t addr, i32x4 v) {
    asm volatile("ds_write_b128 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ inline void lds_w64(uint32_t addr, double v) {
    asm volatile("ds_write_b64 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ inline void lds_w32(uint32_t addr, int v) {
    asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
typedef double f64x2 __attribute__((ext_vector_type(2)));
template <int N>
__device__ inline void lgkm_tie0(i32x4 (&k)[N], i32x4 (&v)[N]) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(k[0]), "+v"(v[0]));
#pragma unroll
    for (int i = 1; i < N; ++i) asm volatile("" : "+v"(k[i]), "+v"(v[i]));
}
// s_waitcnt vmcnt(N), the other counters at their maxima.
template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
template <int I, int N, typename F>
__device__ inline void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Interleaved waves (IW; head_dim 256, paged or ring pools). Grid (nwg, Hkv): a workgroup
// is one kv head over one key range, and its eight waves take the batches of each piece
// in turn (wave v: batches v, v + 8, ...). At the end of a piece the waves' (m, l, o) are
// combined through LDS: a common row max, then the scaled o and l summed in three rounds
// (waves 4-7 into 0-3, 2-3 into 0-1, 1 into 0), and wave 0 writes the piece; this runs
// once the next piece's first batch has been requested. So a piece leaves one partial per
// kv head where one wave per kv head over an eighth of the keys left eight: config 5's
// verify writes 5.9 instead of 35.6 MB of double partials, and its merge takes 6.2
// instead of 9.7 us (verify launch 122.1 -> 116.1 us in the trace). Every kv head's
// workgroups take the same key split, and column w of every head runs on XCD w mod 8, so
// the heads of a token row are read at about the same time.
constexpr int kRedRegion = 2048 * 8 + 128;  // o of one wave (8 rows x 256 doubles), then l
constexpr int kRedO = 512 + 64;             // m [8 waves][8 rows] (doubles), 8 bad flags, pad
__host__ __device__ constexpr size_t iw_red_bytes() { return kRedO + 4 * (size_t)kRedRegion; }

// FUSED: the launch of a fused append (paged pools); a separate instance, so the scalar
// state of the appended rows costs the other launches nothing.
template <int D, int RG, int TG, int WPH, int ADDR, bool FUSED, bool IW = false>
__global__ __launch_bounds__(kMaxWaves * kSW) void stream_mfma_kernel(StreamArgs a) {
    constexpr int NQ = D / 64;  // 64-d chunks of a row
    constexpr int kSlot = mfma_slot(D);
    constexpr int U = 4 * TG;  // tokens per batch
    constexpr bool RING = ADDR == kAddrRing;
    constexpr bool SPARSE = ADDR == kAddrSparse;
    constexpr bool PAGED = ADDR == kAddrPaged;
    // Every chunk of a row slice is copied by one wave only (WPH > 1: the waves of a head
    // share the staging), so the rows are loaded with the NT bit: a launch streams ~1 GB
    // once, which would otherwise displace what is reused (partials, tables, Q). Head_dim
    // 512, 2 kv heads, B = 32: 215.8 -> 207.6 us per launch (same box).
    constexpr int kCpol = kCpolNT;
    extern __shared__ int smem[];
    int* s_pre = smem;               // [batch + 1]
    int* s_lo = smem + a.batch + 1;  // [batch]
    int* s_meta = smem + 2 * a.batch + 1;         // [3 batch + 1] (stream_setup)
    int* s_al = smem + stream_seq_ints(a.batch);  // fused append: the allocation plan

    const int tid = threadIdx.x;
    const int lane = tid & (kSW - 1);
    const int wave = ufirst(tid / kSW);
    const int w = IW ? blockIdx.x : blockIdx.y;  // the workgroup's key range
    const int B = a.batch;

    static_assert(!FUSED || PAGED, "appended rows: paged pools only");
    static_assert(!IW || (WPH == 1 && RG == 2 && TG == 1 && D == 256 && !SPARSE), "interleaved waves");
    const KeySplit sp = stream_setup<D, ADDR>(a, s_pre, s_lo, s_meta, s_al);
    constexpr bool fused = FUSED;  // the launcher passes the rows exactly when FUSED
    const int hpw = ufirst((int)(blockDim.x / kSW) / WPH);  // kv heads per workgroup
    if (fused) {
        if constexpr (IW) copy_new_rows<D, float, kMaxWaves>(a, s_meta, s_al, blockIdx.y, wave, lane, w);
        else copy_new_rows<D, float, WPH>(a, s_meta, s_al, blockIdx.x * hpw, wave, lane, w);
    }
    const int total = ufirst(s_pre[B]);
    const int k0 = sp.start(w);
    if (k0 >= total) return;
    const int k1 = min(total, sp.start(w + 1));
    // this wave's KV head. With WPH > 1 the waves of a head share its staging and meet at
    // barriers, so a wave past the last head (a head group with fewer heads) does the work of
    // the last head and stores nothing, instead of leaving. IW: the workgroup's head, whose
    // pieces wave 0 stores.
    const int g_raw = IW ? (int)blockIdx.y : blockIdx.x * hpw + wave / WPH;
    if (WPH == 1 && g_raw >= a.Hkv) return;
    const bool idle = IW ? wave != 0 : g_raw >= a.Hkv;
    const int g = g_raw >= a.Hkv ? a.Hkv - 1 : g_raw;
    const int rb = IW ? 0 : (wave % WPH) * 4 * RG;  // first of this wave's rows of the head

    const int rows = a.G * a.q_cnt;
    const size_t row_bytes = (size_t)a.Hkv * D * 4;
    const char* kbase = a.k_pool + (size_t)g * D * 4;
    const char* vbase = a.v_pool + (size_t)g * D * 4;
    const int x = lane & 3, b = (lane >> 2) & 3, y = lane >> 4;
    const int kdo = 64 * b + 16 * y;  // bytes of d = 16b + 4y in a 64-d chunk (K operand)
    const int vdo = 64 * b + 16 * x;  // bytes of d = 16b + 4x (V operand)
    const int bs_mask = (1 << a.bs_shift) - 1;
    // Staging. WPH 1: one buffer per wave, loaded and read by that wave (two buffers, with
    // the reads untracked, measured no faster: 129.5-130.9 against 128.0-128.4 us for the
    // config 5 verify launch). WPH > 1: two buffers per head (batches i and i + 1 in flight
    // together), each wave of the head copying its share of the batch's 1 KiB row chunks.
    constexpr int CPT = D / 256;  // 1 KiB chunks per row slice
    // copy i = j * CPT + c (token j, chunk c) of a batch is made by wave i % WPH of the head
    static_assert((4 * TG * CPT) % WPH == 0, "copies split evenly over a head's waves");
    char* stage = reinterpret_cast<char*>(smem) + mfma_stage_offset(B, fused) +
                  (WPH == 1 ? (size_t)wave * mfma_stage_bytes(D, TG)
                            : (size_t)(wave / WPH) * 2 * mfma_stage_bytes(D, TG));
    const int hw = WPH == 1 ? 0 : wave % WPH;  // this wave's share of the copies
    // IW: the waves' exchange area for the end of a piece, after the eight staging buffers
    char* const red = reinterpret_cast<char*>(smem) + mfma_stage_offset(B, fused) +
                      (size_t)kMaxWaves * mfma_stage_bytes(D, TG);
    // Waves w and w + 4 of an 8-wave workgroup share a SIMD, whose issue slots bound the
    // batch loop; the arbiter favours the older wave, which left the other one alone for
    // the last ~15% of a piece. Alternating their priorities every batch keeps the two in
    // step.
    const bool toggle = blockDim.x == kMaxWaves * kSW;

    int s = 0;
    {
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (ufirst(s_pre[mid]) <= k0) lo = mid;
            else hi = mid - 1;
        }
        s = lo;
    }
    // The piece's (m, l, o) per row. IW: a piece is finished (the waves' exchange, then
    // wave 0's stores) once the next piece's first batch has been requested, so that batch's
    // latency covers the exchange and the waves' wait for the slowest of them.
    double m[RG], l[RG], o[RG][NQ][4];
    int pend_s = -1, pend_rows = 0, pend_nb = 0;  // IW: the piece still to finish
    bool pend_single = false, pend_bad = false;
    // nb: the piece's batches (IW: waves past its last batch hold (-inf, 0, 0)).
    auto finish = [&](int fs, bool fsingle, int frows, int nb, bool fbad) {
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            // keep the last accumulations ahead of the stores' branches
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(o[rg][q][e]));
        }
        if constexpr (IW) {
            // The waves' (m, l, o) into wave 0's: the rows' common max, then the rescaled
            // o and l summed in three rounds. The branches are uniform over the workgroup, so
            // every wave meets the same barriers. The next piece's copies into the staging
            // buffers are in flight: the exchange area's LDS accesses are untracked by the
            // compiler (it would wait for the copies before each of them), and the barriers
            // wait only for LDS (lgkmcnt), with no fence.
            if (nb > 1) {
                // per-lane offsets through an opaque copy, so the addresses below are formed
                // here rather than kept in registers for the whole kernel
                uint32_t lo = lane;
                asm volatile("" : "+v"(lo));
                const uint32_t rm = lds_addr(red);  // m of [wave][rg][x] (doubles)
                const uint32_t rbad = rm + 512;     // [wave] (ints)
                const uint32_t xo = lo & 3;
                auto sync = [&]() {
                    __builtin_amdgcn_s_waitcnt(kLgkm0);
                    __builtin_amdgcn_s_barrier();
                    asm volatile("" ::: "memory");
                };
                if (lane < 4) {  // x = lane (b = y = 0)
                    lds_w64(rm + 64 * wave + 8 * lo, m[0]);
                    lds_w64(rm + 64 * wave + 8 * lo + 32, m[1]);
                }
                if (lane == 0) lds_w32(rbad + 4 * wave, fbad ? 1 : 0);
                sync();
                double mv[2][kMaxWaves];
                int bv[kMaxWaves];
                static_for<0, kMaxWaves>([&](auto V) {
                    constexpr int v = decltype(V)::value;
                    mv[0][v] = lds_r64<64 * v>(rm + 8 * xo);
                    mv[1][v] = lds_r64<64 * v + 32>(rm + 8 * xo);
                    bv[v] = lds_r32<4 * v>(rbad + 0 * lo);
                });
                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(mv[0][0]));
#pragma unroll
                for (int v = 0; v < kMaxWaves; ++v) asm volatile("" : "+v"(mv[0][v]), "+v"(mv[1][v]), "+v"(bv[v]));
                bool any_bad = false;
#pragma unroll
                for (int v = 0; v < kMaxWaves; ++v) any_bad = any_bad || bv[v] != 0;
                fbad = any_bad;
#pragma unroll
                for (int rg = 0; rg < RG; ++rg) {
                    double M = -INFINITY;
#pragma unroll
                    for (int v = 0; v < kMaxWaves; ++v) M = fmax(M, mv[rg][v]);
                    const double f = m[rg] == -INFINITY ? 0.0 : exp_acc(m[rg] - M);
                    l[rg] *= f;
#pragma unroll
                    for (int q = 0; q < NQ; ++q)
#pragma unroll
                        for (int e = 0; e < 4; ++e) o[rg][q][e] *= f;
                    m[rg] = M;
                }
                // Region r: element pair k of o (k = 8 rg + 2 q + e / 2) of lane L at byte
                // 16 (64 k + L) (16-byte accesses, consecutive over the lanes), then l [rg][x].
                const uint32_t reg0 = lds_addr(red + kRedO);
                auto put = [&](int r) {
                    const uint32_t rs = reg0 + r * kRedRegion;  // uniform
                    const uint32_t ro = rs + 16 * lo;
#pragma unroll
                    for (int k = 0; k < 16; ++k) {
                        const int rg = k >> 3, q = (k >> 1) & 3, e = 2 * (k & 1);
                        lds_w128(ro + 1024 * k, __builtin_bit_cast(i32x4, f64x2{o[rg][q][e], o[rg][q][e + 1]}));
                    }
                    if (lane < 4) {
                        const uint32_t rl = rs + 16384 + 8 * lo;
                        lds_w64(rl, l[0]);
                        lds_w64(rl + 32, l[1]);
                    }
                };
                auto add = [&](int r) {  // in two halves of eight reads
                    const uint32_t rs = reg0 + r * kRedRegion;  // uniform
                    const uint32_t ro = rs + 16 * lo;
                    static_for<0, 2>([&](auto H) {
                        constexpr int h = decltype(H)::value;
                        i32x4 v[8];
                        static_for<0, 8>([&](auto K) {
                            constexpr int k = decltype(K)::value;
                            v[k] = lds_b128<1024 * (8 * h + k)>(ro);
                        });
                        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]));
#pragma unroll
                        for (int k = 0; k < 8; ++k) {
                            asm volatile("" : "+v"(v[k]));
                            const f64x2 d = __builtin_bit_cast(f64x2, v[k]);
                            const int q = k >> 1, e = 2 * (k & 1);
                            o[h][q][e] += d.x;
                            o[h][q][e + 1] += d.y;
                        }
                    });
                    const uint32_t rl = rs + 16384 + 8 * xo;
                    double l0 = lds_r64<0>(rl), l1 = lds_r64<32>(rl);
                    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(l0), "+v"(l1));
                    l[0] += l0;
                    l[1] += l1;
                };
                if (nb > 4) {  // waves 4-7 into 0-3 (regions 0-3)
                    if (wave >= 4) put(wave - 4);
                    sync();
                    if (wave < 4) add(wave);
                }
                if (nb > 2) {  // waves 2, 3 into 0, 1 (regions 2, 3, which only they read before)
                    if (wave == 2 || wave == 3) put(wave);
                    sync();
                    if (wave < 2) add(wave + 2);
                }
                if (wave == 1) put(1);  // wave 1 into 0 (region 1, which only wave 1 read before)
                sync();
                if (wave == 0) add(1);
            }
        }
        if (idle) {
            // a wave past the last head (IW: every wave but 0): nothing to store
        } else if (fsingle) {
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                const int r = rb + 4 * rg + x;
                if (r < frows) {
                    const double inv = 1.0 / (l[rg] + 1e-10);
                    float* op = a.out + out_row(a, fs, g, r) * D + 16 * b + 4 * y;
#pragma unroll
                    for (int q = 0; q < NQ; ++q) {
                        float4 v;
                        v.x = fbad ? __builtin_nanf("") : (float)(o[rg][q][0] * inv);
                        v.y = fbad ? __builtin_nanf("") : (float)(o[rg][q][1] * inv);
                        v.z = fbad ? __builtin_nanf("") : (float)(o[rg][q][2] * inv);
                        v.w = fbad ? __builtin_nanf("") : (float)(o[rg][q][3] * inv);
                        *reinterpret_cast<float4*>(op + 64 * q) = v;
                    }
                }
            }
        } else {
            const size_t slot = (size_t)(w + fs) * a.rows_seq;
            double* po = static_cast<double*>(a.part_o);
            double* pml = static_cast<double*>(a.part_ml);
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                const int r = rb + 4 * rg + x;
                if (r < rows) {
                    const int row = (r / a.G) * a.Hq + g * a.G + r % a.G;
                    double* dst = po + (slot + row) * D + 16 * b + 4 * y;
#pragma unroll
                    for (int q = 0; q < NQ; ++q) {
                        double2* d2 = reinterpret_cast<double2*>(dst + 64 * q);
                        d2[0] = make_double2(o[rg][q][0], o[rg][q][1]);
                        d2[1] = make_double2(o[rg][q][2], o[rg][q][3]);
                    }
                    if (b == 0 && y == 0) {
                        pml[(slot + row) * 2 + 0] = fbad ? __builtin_nan("") : m[rg];
                        pml[(slot + row) * 2 + 1] = l[rg];
                    }
                }
            }
        }
    };

    int pre_s = -1, pre_raw = 0;  // the next piece's first page ids (pre_s: its sequence)
    for (; s < B; ++s) {
        const int ps = ufirst(s_pre[s]);
        const int pe = ufirst(s_pre[s + 1]);
        if (ps >= k1) break;
        if (pe == ps) continue;
        const int psr = ps + a.lead;  // the sequence's first key after its lead-in
        if (psr >= k1) break;
        const int lo_key = ufirst(s_lo[s]);
        const int ta = lo_key + max(k0, psr) - psr;  // first key of the piece
        const int tb = lo_key + min(k1, pe) - psr;   // one past the last
        const bool single = sp.owner(psr) == sp.owner(pe - 1);
        // the sequence's position (sparse: its list's first index) and query count, from
        // the setup's LDS copy
        const int kbeg = SPARSE ? ufirst(s_meta[s]) : 0;
        const int pos0 = SPARSE ? 0 : ufirst(s_meta[s]);
        const int rows_s = a.G * ufirst(s_meta[B + s]);
        const int32_t* trow = a.tables + (size_t)s * a.table_stride;
        const int last_page = (tb - 1) >> a.bs_shift;
        // Fused append: table indices [g_lo, g_hi) are the blocks granted in this call,
        // whose ids come from the free list (g_top - index); positions [pn_lo, pn_hi) are
        // read from k_new / v_new (row nr0 + t - pn_lo).
        int g_lo = INT32_MAX, g_hi = INT32_MIN, g_top = 0;
        int pn_lo = INT32_MAX, pn_hi = INT32_MIN, nr0 = 0;
        bool failed = false;  // a failed append: NaN rows, as in the vector kernel
        if (fused) {
            const SeqAlloc al = seq_alloc(s_al, B, a.num_blocks, s);
            failed = ufirst(al.code) != PKV_SEQ_OK;
            g_lo = ufirst(al.len);
            g_hi = g_lo + ufirst(al.granted);
            g_top = ufirst(al.fc) - 1 - ufirst(al.pref) + g_lo;
            const int r0 = ufirst(s_meta[2 * B + s]);
            const int n = ufirst(s_meta[2 * B + s + 1]) - r0;
            if (new_rows_written(ufirst(al.code)) && pos0 >= 0 && n > 0) {
                pn_lo = pos0;
                pn_hi = pos0 + n;
                nr0 = r0;
            }
        }

        // The piece's first loads are all requested before any of them is used (one round
        // trip): the first 64 page ids (sparse: listed keys) and the query rows. Each is
        // issued (indices clamped into range; values past the piece or of rows past `rows`
        // are not used), so no branch separates a load from its use.
        int first_raw = 0;
        if constexpr (SPARSE) {
            first_raw = a.keys[kbeg + min(ta + lane, tb - 1)];
        } else if constexpr (PAGED) {
            const int pg = min((ta >> a.bs_shift) + lane, last_page);
            const int32_t* src = trow + pg;
            if constexpr (FUSED) src = (pg >= g_lo && pg < g_hi) ? a.nr.free_list + (g_top - pg) : src;
            first_raw = (!FUSED && pre_s == s) ? pre_raw : *src;
        }
        asm volatile("" ::: "memory");  // issued before the query rows
        // this lane's rows rb + 4rg + x: Q slice (B operand), query position, first key
        float4 qf[RG][NQ];  // fp32: converted at each use, which saves registers
        int pq[RG], wsr[RG];
        bool live[RG];
        // IW: requested after the piece before is finished (fewer registers live there)
        auto load_q = [&]() {
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                const int r = rb + 4 * rg + x;
                const float* qp = a.q + out_row(a, s, g, min(r, rows - 1)) * D + 16 * b + 4 * y;
#pragma unroll
                for (int q = 0; q < NQ; ++q) qf[rg][q] = *reinterpret_cast<const float4*>(qp + 64 * q);
            }
        };
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            const int r = rb + 4 * rg + x;
            live[rg] = r < rows_s;
            pq[rg] = SPARSE ? INT32_MAX : pos0 + a.j0 + r / a.G;
            wsr[rg] = SPARSE ? 0 : window_start(pq[rg], a.window);
        }
        if constexpr (!IW) load_q();
        // The next sequence's first 64 page ids, for its piece after this one (a piece starts
        // at its sequence's first key).
        if (PAGED && !FUSED && s + 1 < B && ufirst(s_pre[s + 1]) + a.lead < k1 &&
            ufirst(s_pre[s + 2]) > ufirst(s_pre[s + 1])) {
            const int lo_n = ufirst(s_lo[s + 1]);
            const int tb_n = lo_n + min(k1, ufirst(s_pre[s + 2])) - ufirst(s_pre[s + 1]) - a.lead;
            pre_raw = a.tables[(size_t)(s + 1) * a.table_stride +
                               min((lo_n >> a.bs_shift) + lane, (tb_n - 1) >> a.bs_shift)];
            pre_s = s + 1;
        }
        auto zero_q = [&]() {
#pragma unroll
            for (int rg = 0; rg < RG; ++rg)
#pragma unroll
                for (int q = 0; q < NQ; ++q)
                    if (rb + 4 * rg + x >= rows) qf[rg][q] = make_float4(0.f, 0.f, 0.f, 0.f);
        };
        if constexpr (!IW) zero_q();
        int64_t rbase = 0;  // ring mode: first row of the sequence's ring
        int r0 = 0;         // ring mode: ring row of key ta
        if constexpr (RING) {
            rbase = a.pos ? (int64_t)ufirst(trow[0]) * a.ring_size : a.ring_base;
            r0 = ta % a.ring_size;
        }
        int pgbase = -kSW;  // page index (sparse: list index) held by lane 0 of vpg
        int vpg = 0;
        bool bad = failed;
        asm volatile("" ::: "memory");  // the query rows go out before the table lookup
        // (branch-free, so the compiler does not move a load into a branch)
        if constexpr (SPARSE) {  // the first listed keys' table entries (one more round trip)
            pgbase = ta;
            const int key = first_raw;
            const int blk = key >> a.bs_shift;
            const bool in_table = key >= 0 && blk < a.table_stride;
            const int ent = trow[in_table ? blk : 0];
            const int phys = in_table ? ent : -1;
            const bool lane_ok = ta + lane < tb;
            const bool id_ok = phys >= 0 && phys < a.num_blocks;
            bad = bad || (lane_ok && !id_ok);
            vpg = lane_ok && id_ok ? (phys << a.bs_shift) | (key & bs_mask) : 0;
        } else if constexpr (PAGED) {
            pgbase = ta >> a.bs_shift;
            const bool lane_ok = pgbase + lane <= last_page;
            const bool id_ok = first_raw >= 0 && first_raw < a.num_blocks;
            bad = bad || (lane_ok && !id_ok);
            vpg = lane_ok && id_ok ? first_raw : 0;
        }

        // Batch staging: each token's K and V slices go from global memory straight into
        // this wave's LDS slots (one row slice per slot, slots kSlot bytes apart), so the
        // next batch's loads are in flight while the current one is computed from registers.
        // The operand reads take 16 bytes of token 4tg + x (K) or 4tg + y (V); the 16-byte
        // slot padding puts the 16 lanes of each read phase on distinct banks.
        auto issue = [&](int t, char* buf) {
            const int tl = min(t + U - 1, tb - 1);
            if (SPARSE && tl - pgbase >= kSW) {  // pool rows of the next 64 listed keys
                pgbase = t;
                int row = 0;
                if (t + lane < tb) {
                    const int key = a.keys[kbeg + t + lane];
                    const int blk = key >> a.bs_shift;
                    const int phys = (key >= 0 && blk < a.table_stride) ? trow[blk] : -1;
                    if (phys < 0 || phys >= a.num_blocks) bad = true;
                    else row = (phys << a.bs_shift) | (key & bs_mask);
                }
                vpg = row;
            }
            if (PAGED && (tl >> a.bs_shift) - pgbase >= kSW) {  // next 64 page ids
                pgbase = t >> a.bs_shift;
                int pg = 0;
                if (pgbase + lane <= last_page) {
                    const int pi = pgbase + lane;
                    if constexpr (FUSED) pg = (pi >= g_lo && pi < g_hi) ? a.nr.free_list[g_top - pi] : trow[pi];
                    else pg = trow[pi];
                    if (pg < 0 || pg >= a.num_blocks) {
                        bad = true;
                        pg = 0;
                    }
                }
                vpg = pg;
            }
            // Copy k of this wave: 1 KiB chunk c of token j's row slice (64 lanes x 16 bytes,
            // contiguous), i = j * CPT + c = k * WPH + hw. The address is wave-uniform: page id by
            // readlane, offsets in scalar registers.
#pragma unroll
            for (int k = 0; k < U * CPT / WPH; ++k) {
                const int i = k * WPH + hw;
                const int j = i / CPT, c = i % CPT;
                const int tt = min(t + j, tb - 1);  // tokens past the piece re-read its last row
                size_t off;
                const char* kb = kbase;
                const char* vb = vbase;
                if constexpr (RING) {
                    off = (size_t)ring_key_row(rbase, r0, tt - ta, a.ring_size) * row_bytes;
                } else if constexpr (SPARSE) {
                    off = (size_t)(uint32_t)__builtin_amdgcn_readlane(vpg, tt - pgbase) * row_bytes;
                } else {
                    const int pg = __builtin_amdgcn_readlane(vpg, (tt >> a.bs_shift) - pgbase);
                    off = (((size_t)pg << a.bs_shift) | (size_t)(tt & bs_mask)) * row_bytes;
                    if (FUSED && tt >= pn_lo && tt < pn_hi) {  // an appended row: from k_new / v_new
                        off = (size_t)(nr0 + (tt - pn_lo)) * row_bytes;
                        kb = a.nr.k_new + (size_t)g * D * 4;
                        vb = a.nr.v_new + (size_t)g * D * 4;
                    }
                }
                __builtin_amdgcn_global_load_lds(uniform_ptr(kb + off + 1024 * c) + 16 * lane,
                                                 (lds_void*)(buf + (2 * j) * kSlot + 1024 * c), 16, 0,
                                                 kCpol);
                __builtin_amdgcn_global_load_lds(uniform_ptr(vb + off + 1024 * c) + 16 * lane,
                                                 (lds_void*)(buf + (2 * j + 1) * kSlot + 1024 * c), 16,
                                                 0, kCpol);
            }
        };

        constexpr int kBufBytes = (int)mfma_stage_bytes(D, TG);
        constexpr int kStepT = IW ? kMaxWaves * U : U;  // tokens from one of a wave's batches to the next
        const int t1 = IW ? ta + U * wave : ta;          // this wave's first batch
        if (t1 < tb) issue(t1, stage);
        if (WPH > 1 && ta + U < tb) issue(ta + U, stage + kBufBytes);
        if constexpr (IW) {  // the piece before, while this one's first batch is on its way
            if (pend_s >= 0) finish(pend_s, pend_single, pend_rows, pend_nb, pend_bad);
            load_q();
            zero_q();
        }
#pragma unroll
        for (int rg = 0; rg < RG; ++rg) {
            m[rg] = -INFINITY;
            l[rg] = 0.0;
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) o[rg][q][e] = 0.0;
        }
        int it = 0;  // this wave's batch index in the piece (WPH > 1: buffer it % 2)
        for (int t = t1; t < tb; t += kStepT, ++it) {
            float4 kw[TG][NQ], vw[TG][NQ];
            if constexpr (WPH == 1) {
                if (toggle) {
                    if ((it + (wave >> 2)) & 1) __builtin_amdgcn_s_setprio(1);
                    else __builtin_amdgcn_s_setprio(0);
                }
                __builtin_amdgcn_s_waitcnt(0);  // this batch's slices are in LDS
#pragma unroll
                for (int tg = 0; tg < TG; ++tg)
#pragma unroll
                    for (int q = 0; q < NQ; ++q) {
                        kw[tg][q] = *reinterpret_cast<const float4*>(stage + (2 * (4 * tg + x)) * kSlot + kdo + 256 * q);
                        vw[tg][q] = *reinterpret_cast<const float4*>(stage + (2 * (4 * tg + y) + 1) * kSlot + vdo + 256 * q);
                    }
                __builtin_amdgcn_s_waitcnt(kLgkm0);  // read out before the slots are refilled
                if (t + kStepT < tb) issue(t + kStepT, stage);
            } else {
                // This wave's copies of batch it have landed (those of batch it + 1, if issued,
                // stay in flight); the barrier then covers the other waves' copies. It carries no
                // fence, which would wait for the copies in flight.
                constexpr int kCopies = U * 2 * CPT / WPH;  // copies per batch and wave
                if (t + U < tb) wait_vm<kCopies>();
                else wait_vm<0>();
                __builtin_amdgcn_s_barrier();
                char* buf = stage + (it & 1) * kBufBytes;
                const uint32_t ka = lds_addr(buf) + (2 * x) * kSlot + kdo;
                const uint32_t va = lds_addr(buf) + (2 * y + 1) * kSlot + vdo;
                static_assert(TG == 1, "one 4-token group per batch");
                i32x4 kr[NQ], vr[NQ];
                static_for<0, NQ>([&](auto Q) {
                    constexpr int q = decltype(Q)::value;
                    kr[q] = lds_b128<256 * q>(ka);
                    vr[q] = lds_b128<256 * q>(va);
                });
                lgkm_tie0(kr, vr);
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    kw[0][q] = __builtin_bit_cast(float4, kr[q]);
                    vw[0][q] = __builtin_bit_cast(float4, vr[q]);
                }
                // every wave of the head has read the buffer: refill it with batch it + 2
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                if (t + 2 * U < tb) issue(t + 2 * U, buf);
            }

            // S^T, then the block sums
            double sc[TG][RG];
#pragma unroll
            for (int tg = 0; tg < TG; ++tg)
#pragma unroll
                for (int rg = 0; rg < RG; ++rg) sc[tg][rg] = 0.0;
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    double qd[RG];
#pragma unroll
                    for (int rg = 0; rg < RG; ++rg)
                        qd[rg] = (double)reinterpret_cast<const float*>(&qf[rg][q])[e];
#pragma unroll
                    for (int tg = 0; tg < TG; ++tg) {
                        const double kd = (double)reinterpret_cast<const float*>(&kw[tg][q])[e];
#pragma unroll
                        for (int rg = 0; rg < RG; ++rg) sc[tg][rg] = mfma4(kd, qd[rg], sc[tg][rg]);
                    }
                }
            // online softmax per row; p holds the weights, the B operand of PV
            double p[TG][RG], scl[RG], m_new[RG];
            bool ok[TG][RG];
            bool moved_any = false;
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                double mb = -INFINITY;
#pragma unroll
                for (int tg = 0; tg < TG; ++tg) {
                    const int tok = t + 4 * tg + y;
                    ok[tg][rg] = live[rg] && tok < tb && tok <= pq[rg] && tok >= wsr[rg];
                    const double v = block_sum(sc[tg][rg]) * (double)a.scale;
                    p[tg][rg] = v;
                    if (ok[tg][rg]) mb = fmax(mb, v);
                }
                mb = allreduce_hi<16>(mb, OpMax());
                m_new[rg] = mb > m[rg] + (double)kLazyMove ? mb : m[rg];  // lazy reference max
            }
            // Every block holds the same scores. With two row groups, blocks of even index
            // take row group 0's exponentials and odd ones row group 1's, and a rotation by
            // one block (4 lanes, the opposite parity) hands each lane the other half.
#pragma unroll
            for (int tg = 0; tg < TG; ++tg) {
                if constexpr (RG == 2) {
                    const bool odd = b & 1;
                    const double e = (odd ? ok[tg][1] : ok[tg][0])
                                         ? exp_acc(odd ? p[tg][1] - m_new[1] : p[tg][0] - m_new[0])
                                         : 0.0;
                    const double other = dpp<ror_ctrl<4>()>(e);
                    p[tg][0] = odd ? other : e;
                    p[tg][1] = odd ? e : other;
                } else {
#pragma unroll
                    for (int rg = 0; rg < RG; ++rg)
                        p[tg][rg] = ok[tg][rg] ? exp_acc(p[tg][rg] - m_new[rg]) : 0.0;
                }
            }
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                double lb = 0.0;
#pragma unroll
                for (int tg = 0; tg < TG; ++tg) lb += p[tg][rg];
                lb = allreduce_hi<16>(lb, OpSum());
                const bool moved = m_new[rg] != m[rg];
                double f = 1.0;
                if (moved) f = exp_acc(m[rg] - m_new[rg]);  // m = -inf gives 0
                scl[rg] = f;
                l[rg] = l[rg] * f + lb;
                m[rg] = m_new[rg];
                moved_any = moved_any || moved;
            }
            if (__any(moved_any)) {
#pragma unroll
                for (int rg = 0; rg < RG; ++rg)
#pragma unroll
                    for (int q = 0; q < NQ; ++q)
#pragma unroll
                        for (int e = 0; e < 4; ++e) o[rg][q][e] *= scl[rg];
            }
            // PV
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int tg = 0; tg < TG; ++tg) {
                        const double vd = (double)reinterpret_cast<const float*>(&vw[tg][q])[e];
#pragma unroll
                        for (int rg = 0; rg < RG; ++rg) o[rg][q][e] = mfma4(vd, p[tg][rg], o[rg][q][e]);
                    }
        }
        bad = __any(bad);
        if constexpr (IW) {
            pend_s = s;
            pend_single = single;
            pend_rows = rows_s;
            pend_nb = (tb - ta + U - 1) / U;
            pend_bad = bad;
        } else {
            finish(s, single, rows_s, 1, bad);
        }
    }
    if constexpr (IW) {
        if (pend_s >= 0) finish(pend_s, pend_single, pend_rows, pend_nb, pend_bad);
    }
}

// ---- bf16 MFMA path: bf16 pools, head_dim 256, 5..8 query rows per KV head -------------
//
// One wave per KV head, up to 8 query rows (a 4-token verify at G = 2), batches of 16
// tokens staged in LDS, all products on v_mfma_f32_16x16x32_bf16 (QK^T) and
// v_mfma_f32_16x16x16_bf16 (PV) with fp32 accumulation. Q is fp32, so it enters as
// Q = Q_hi + Q_lo (both bf16, |q - Q_hi - Q_lo| <= 2^-16 |q|), and so does P (P_hi = p
// truncated to bf16, P_lo = the remainder rounded to nearest, |p - P_hi - P_lo| <= 2^-16
// p): a single bf16 rounding of either would break the 2e-2 output bound near zero. The
// 8 rows use half of the MFMA's 16 columns; the other half carries the low parts, so one
// instruction forms both: column j < 8 holds row j's hi part, column j + 8 its lo part.
// Lane layouts (v_mfma_f32_16x16x32_bf16, checked on the device; the x16 form is its
// K = 16 counterpart): A[i][k] lane i + 16 (k / 8) element k % 8 (x16: lane i + 16 (k / 4)
// element k % 4); B[k][j] likewise with j for i; C[i][j] lane j + 16 (i / 4) register i % 4.
//   S^T[token][col] = K Q^T: A = K (16 tokens x 32 dims per step), B = Q^T. Lane L then
//     holds tokens 4 (L / 16) + r of column L % 16; the hi and lo halves are added by one
//     DPP rotation (lane L ^ 8), after which lanes L and L ^ 8 hold S of row L % 8.
//   O^T[d][col] += V^T P^T (16 dims x 16 tokens per d-tile): B = P^T is exactly what lane
//     L holds (tokens 4 (L / 16) + r): P_hi in the columns below 8, P_lo above; A = V^T
//     comes from one ds_read_b64_tr_b16 per d-tile (input lane a addresses dims
//     4 (a % 4) .. + 3 of token 4 (L / 16) + a / 4; inside each 16-lane group output lane j
//     element e is element j % 4 of what input lane 4e + j / 4 addressed). The hi and lo
//     columns are added once, at the end.
// LDS per wave: K and V of 16 tokens, rows of 512 bytes; K's 16-byte chunk c of token r
// sits at c ^ r and V's 32-byte chunk c at c ^ r, so the operand reads land on distinct
// banks. A copy instruction moves two tokens (1 KiB): the batches start on even positions
// (a piece starting on an odd key also copies the key before it, masked), so a pair lies
// in one block and its address is one scalar base plus a per-lane offset. The row after a
// sequence's last key may be copied (never used): its V row is zeroed in LDS, so a
// non-finite value there cannot reach PV through a zero weight.
constexpr int kBfTok = 16;                       // tokens per batch
constexpr int kBfRow = 512;                      // bytes per token row slice (256 bf16)
constexpr size_t kBfStage = 2 * kBfTok * kBfRow; // K and V of a batch, per wave
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
template <int OFF>
__device__ inline i32x2 lds_tr16(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    i32x2 v;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
__device__ inline uint16_t bf16_rne_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
__device__ inline float bf16_bits_to_float(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Interleaved waves (IW), as in the fp64 kernel: grid (nwg, Hkv), the eight waves of a
// workgroup take the 16-token batches of one kv head's pieces in turn and combine their
// (m, l, o) through LDS (fp32, after the hi/lo fold) once the next piece's first batch is
// requested. The eight staging buffers leave room for three 8 KiB exchange regions, so the
// sum takes four rounds: waves 4-6 into 0-2, 7 into 3, 2-3 into 0-1, 1 into 0. Config 5's
// bf16 verify: 60.4 + 6.7 -> 59.7 + 4.9 us (stream + merge in the trace), traffic 1.149 ->
// 1.025 x algorithmic. Every wave then holds the same rows, so the hi / lo split of Q is
// shared: wave v splits step v and the eight steps go round through LDS (64.6 -> 63.1 us).
constexpr int kBfRedRegion = 8192 + 32;  // o of the 32 hi-column lanes (8 rows x 256), then l
constexpr int kBfRedO = 256 + 32;        // m [8 waves][8 rows] (floats), 8 bad flags
__host__ __device__ constexpr size_t bf_iw_red_bytes() { return kBfRedO + 3 * (size_t)kBfRedRegion; }

template <int ADDR, bool IW = false>
__global__ __launch_bounds__(kMaxWaves * kSW) void stream_bf16_mfma_kernel(StreamArgs a) {
    constexpr int D = 256;
    static_assert(ADDR == kAddrPaged, "paged pools");
    constexpr float kLog2e = 1.4426950408889634f;
    constexpr float kLn2 = 0.6931471805599453f;
    extern __shared__ int smem[];
    int* s_pre = smem;               // [batch + 1]
    int* s_lo = smem + a.batch + 1;  // [batch]
    int* s_meta = smem + 2 * a.batch + 1;  // [3 batch + 1] (stream_setup)

    const int tid = threadIdx.x;
    const int lane = tid & (kSW - 1);
    const int wave = ufirst(tid / kSW);
    const int w = IW ? blockIdx.x : blockIdx.y;  // the workgroup's key range
    const int B = a.batch;
    const KeySplit sp = stream_setup<D, ADDR>(a, s_pre, s_lo, s_meta, nullptr);  // no fused append
    const int total = ufirst(s_pre[B]);
    const int k0 = sp.start(w);
    if (k0 >= total) return;
    const int k1 = min(total, sp.start(w + 1));
    const int g = IW ? (int)blockIdx.y : blockIdx.x * kMaxWaves + wave;  // this wave's KV head
    if (g >= a.Hkv) return;

    const int rows = a.G * a.q_cnt;
    const uint32_t row_bytes = (uint32_t)a.Hkv * D * 2;
    const char* kbase = a.k_pool + (size_t)g * D * 2;
    const char* vbase = a.v_pool + (size_t)g * D * 2;
    const int grp = lane >> 4, l16 = lane & 15;
    const int rr = l16 & 7;           // the row of this lane's column
    const bool hi_col = l16 < 8;      // column holds the row's hi part (else its lo part)
    const int bs_mask = (1 << a.bs_shift) - 1;
    const float sl2 = a.scale * kLog2e;
    char* sK = reinterpret_cast<char*>(smem) + mfma_stage_offset(B, false) + (size_t)wave * kBfStage;
    char* sV = sK + kBfTok * kBfRow;
    // IW: the waves' exchange area, after the eight staging buffers
    char* const red = reinterpret_cast<char*>(smem) + mfma_stage_offset(B, false) + (size_t)kMaxWaves * kBfStage;

    // Copy offsets: instruction j moves tokens 2j, 2j + 1 of the batch (lanes 0-31, 32-63);
    // lane p of a row loads the global chunk that belongs at its LDS position.
    uint32_t k_off[8], v_off[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int r = 2 * j + (lane >> 5), p16 = lane & 31;
        const uint32_t hb = (uint32_t)(lane >> 5) * row_bytes;
        k_off[j] = hb + 16u * (uint32_t)(p16 ^ r);
        v_off[j] = hb + 16u * (uint32_t)((((p16 >> 1) ^ r) << 1) | (p16 & 1));
    }
    // LDS operand addresses. K, 32-dim step c: token l16, 16-byte chunk (4c + grp) ^ l16 =
    // byte 512 l16 + 16 (grp ^ (l16 & 3)) + 64 ((c & 3) ^ (l16 >> 2)) + 256 (c >> 2).
    const uint32_t k_lane = lds_addr(sK) + 512u * l16 + 16u * (grp ^ (l16 & 3));
    uint32_t k_addr[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) k_addr[q] = k_lane + 64u * (q ^ (l16 >> 2));
    // V, d-tile u: token z = 4 grp + l16 / 4, byte 512 z + 32 (u ^ z) + 8 (l16 & 3).
    const int z = 4 * grp + (l16 >> 2);
    const uint32_t v_lane = lds_addr(sV) + 512u * z + 8u * (l16 & 3);

    int s = 0;
    {
        int lo = 0, hi = B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (ufirst(s_pre[mid]) <= k0) lo = mid;
            else hi = mid - 1;
        }
        s = lo;
    }
    // The piece's row max (log2 units), this lane's share of the row sum, O^T. IW: a piece
    // is finished (the waves' exchange, then wave 0's stores) once the next piece's first
    // batch has been requested, so that batch's latency covers the exchange.
    float m = -INFINITY;
    float l = 0.f;
    f32x4 o[16];  // O^T: d-tile u holds dims 16u + 4 grp + r of column l16
    int pend_s = -1, pend_rows = 0, pend_nb = 0;  // IW: the piece still to finish
    bool pend_single = false, pend_bad = false;
    const bool idle = IW && wave != 0;
    // nb: the piece's batches (IW: waves past its last batch hold (-inf, 0, 0)).
    auto finish = [&](int fs, bool fsingle, int frows, int nb, bool fbad) {
        // O^T hi + lo columns; the row sum over the four lane groups
        l = allreduce_hi<16>(l, OpSum());
#pragma unroll
        for (int u = 0; u < 16; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[u][r] += dpp<kRor8>(o[u][r]);
        if constexpr (IW) {
            // The waves' rows into wave 0's: the rows' common max, then the rescaled o (the
            // 32 hi-column lanes, which hold the rows after the fold) and l summed. Uniform
            // branches: every wave meets the same barriers. The next piece's copies are in
            // flight, so the LDS accesses are untracked and the barriers wait for LDS only.
            if (nb > 1) {
                uint32_t lo = lane;  // opaque: the addresses are formed here
                asm volatile("" : "+v"(lo));
                const uint32_t rm = lds_addr(red);  // m of [wave][row] (floats)
                const uint32_t rbad = rm + 256;     // [wave] (ints)
                const uint32_t rro = lo & 7;        // this lane's row
                auto sync = [&]() {
                    __builtin_amdgcn_s_waitcnt(kLgkm0);
                    __builtin_amdgcn_s_barrier();
                    asm volatile("" ::: "memory");
                };
                if (lane < 8) lds_w32(rm + 32 * wave + 4 * lo, __float_as_int(m));  // row = lane
                if (lane == 0) lds_w32(rbad + 4 * wave, fbad ? 1 : 0);
                sync();
                int mv[kMaxWaves], bv[kMaxWaves];
                static_for<0, kMaxWaves>([&](auto V) {
                    constexpr int v = decltype(V)::value;
                    mv[v] = lds_r32<32 * v>(rm + 4 * rro);
                    bv[v] = lds_r32<4 * v>(rbad + 0 * lo);
                });
                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(mv[0]));
#pragma unroll
                for (int v = 0; v < kMaxWaves; ++v) asm volatile("" : "+v"(mv[v]), "+v"(bv[v]));
                bool any_bad = false;
                float M = -INFINITY;
#pragma unroll
                for (int v = 0; v < kMaxWaves; ++v) {
                    any_bad = any_bad || bv[v] != 0;
                    M = fmaxf(M, __int_as_float(mv[v]));
                }
                fbad = any_bad;
                const float f = m == -INFINITY ? 0.f : exp2f(m - M);
                l *= f;
#pragma unroll
                for (int u = 0; u < 16; ++u) o[u] *= f;
                m = M;
                // Region r: d-tile u of hi-column lane j = 8 grp + l16 at byte 16 (32 u + j),
                // then l [row].
                const uint32_t reg0 = lds_addr(red + kBfRedO);
                const uint32_t jo = 16 * ((lo >> 4) * 8 + (lo & 7));
                auto put = [&](int r) {
                    const uint32_t rs = reg0 + r * kBfRedRegion;  // uniform
                    if (hi_col) {
#pragma unroll
                        for (int u = 0; u < 16; ++u) lds_w128(rs + jo + 512 * u, __builtin_bit_cast(i32x4, o[u]));
                    }
                    if (lane < 8) lds_w32(rs + 8192 + 4 * lo, __float_as_int(l));
                };
                auto add = [&](int r) {  // in two halves of eight reads
                    const uint32_t rs = reg0 + r * kBfRedRegion;  // uniform
                    if (hi_col) {
                        static_for<0, 2>([&](auto H) {
                            constexpr int h = decltype(H)::value;
                            i32x4 v[8];
                            static_for<0, 8>([&](auto U) {
                                constexpr int u = decltype(U)::value;
                                v[u] = lds_b128<512 * (8 * h + u)>(rs + jo);
                            });
                            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v[0]));
#pragma unroll
                            for (int u = 0; u < 8; ++u) {
                                asm volatile("" : "+v"(v[u]));
                                o[8 * h + u] += __builtin_bit_cast(f32x4, v[u]);
                            }
                        });
                    }
                    int lv = lds_r32<8192>(rs + 4 * rro);
                    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(lv));
                    l += __int_as_float(lv);
                };
                if (nb > 4) {  // waves 4-6 into 0-2 (regions 0-2), then every region read
                    if (wave >= 4 && wave < 7) put(wave - 4);
                    sync();
                    if (wave < 3) add(wave);
                    sync();
                }
                if (nb > 7) {  // wave 7 into 3 (region 0)
                    if (wave == 7) put(0);
                    sync();
                    if (wave == 3) add(0);
                }
                if (nb > 2) {  // waves 2, 3 into 0, 1 (regions 2, 1; region 0 may still be read)
                    if (wave == 2) put(2);
                    if (wave == 3) put(1);
                    sync();
                    if (wave == 0) add(2);
                    if (wave == 1) add(1);
                }
                if (wave == 1) put(1);  // wave 1 into 0 (region 1, which wave 1 read last)
                sync();
                if (wave == 0) add(1);
            }
        }
        if (idle) {
            // IW: every wave but 0 has handed its rows over
        } else if (fsingle) {
            int gofs = 4 * grp;
            if constexpr (IW) asm volatile("" : "+v"(gofs));
            if (hi_col && rr < frows) {
                const float inv = 1.f / (l + 1e-10f);
                float* op = a.out + out_row(a, fs, g, rr) * D + gofs;
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    float4 v;
                    v.x = fbad ? __builtin_nanf("") : o[u][0] * inv;
                    v.y = fbad ? __builtin_nanf("") : o[u][1] * inv;
                    v.z = fbad ? __builtin_nanf("") : o[u][2] * inv;
                    v.w = fbad ? __builtin_nanf("") : o[u][3] * inv;
                    *reinterpret_cast<float4*>(op + 16 * u) = v;
                }
            }
        } else {
            // IW: the lane's offset from an opaque copy (formed here, not kept in registers
            // across the kernel)
            int gofs = 4 * grp;
            if constexpr (IW) asm volatile("" : "+v"(gofs));
            const size_t slot = (size_t)(w + fs) * a.rows_seq;
            float* po = static_cast<float*>(a.part_o);
            float* pml = static_cast<float*>(a.part_ml);
            if (hi_col && rr < rows) {
                const int row = (rr / a.G) * a.Hq + g * a.G + rr % a.G;
                float* dst = po + (slot + row) * D + gofs;
#pragma unroll
                for (int u = 0; u < 16; ++u)
                    *reinterpret_cast<float4*>(dst + 16 * u) = make_float4(o[u][0], o[u][1], o[u][2], o[u][3]);
                if (grp == 0) {  // the merge takes natural-log units
                    pml[(slot + row) * 2 + 0] = fbad ? __builtin_nanf("") : m * kLn2;
                    pml[(slot + row) * 2 + 1] = l;
                }
            }
        }
    };

    int pre_s = -1, pre_raw = 0;  // the next piece's first page ids (pre_s: its sequence)
    for (; s < B; ++s) {
        const int ps = ufirst(s_pre[s]);
        const int pe = ufirst(s_pre[s + 1]);
        if (ps >= k1) break;
        if (pe == ps) continue;
        const int psr = ps + a.lead;  // the sequence's first key after its lead-in
        if (psr >= k1) break;
        const int lo_key = ufirst(s_lo[s]);
        const int ta = lo_key + max(k0, psr) - psr;  // first key of the piece
        const int tb = lo_key + min(k1, pe) - psr;   // one past the last
        const bool single = sp.owner(psr) == sp.owner(pe - 1);
        const int pos0 = ufirst(s_meta[s]);
        const int rows_s = a.G * ufirst(s_meta[B + s]);
        const int32_t* trow = a.tables + (size_t)s * a.table_stride;
        const int t0 = ta & ~1;  // batches start on even positions
        const int last_page = (tb - 1) >> a.bs_shift;

        // The first 64 page ids (requested while the previous piece ran, if there was one)
        // and the query rows, requested together; the first batch's copies go out before
        // the query rows are split, which waits for them.
        const int first_raw =
            pre_s == s ? pre_raw : trow[min((t0 >> a.bs_shift) + lane, last_page)];
        asm volatile("" ::: "memory");
        float4 qraw[8][2];
        // IW: wave v requests only step v of every lane's Q (its share of the hi / lo split
        // below); the other steps come through LDS.
        float4 qstep[2];
        if constexpr (IW) {
            const float* qp = a.q + out_row(a, s, g, min(rr, rows - 1)) * D + 8 * grp + 32 * wave;
            qstep[0] = *reinterpret_cast<const float4*>(qp);
            qstep[1] = *reinterpret_cast<const float4*>(qp + 4);
        } else {
            const float* qp = a.q + out_row(a, s, g, min(rr, rows - 1)) * D + 8 * grp;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                qraw[c][0] = *reinterpret_cast<const float4*>(qp + 32 * c);
                qraw[c][1] = *reinterpret_cast<const float4*>(qp + 32 * c + 4);
            }
        }
        asm volatile("" ::: "memory");
        // The next sequence's first 64 page ids, for its piece after this one (a piece
        // starts at its sequence's first key).
        if (s + 1 < B && ufirst(s_pre[s + 1]) + a.lead < k1 &&
            ufirst(s_pre[s + 2]) > ufirst(s_pre[s + 1])) {
            const int lo_n = ufirst(s_lo[s + 1]);
            const int t0_n = lo_n & ~1;
            const int tb_n = lo_n + min(k1, ufirst(s_pre[s + 2])) - ufirst(s_pre[s + 1]) - a.lead;
            pre_raw = a.tables[(size_t)(s + 1) * a.table_stride +
                               min((t0_n >> a.bs_shift) + lane, (tb_n - 1) >> a.bs_shift)];
            pre_s = s + 1;
        }
        const int pq = pos0 + a.j0 + rr / a.G;  // query position of this lane's row
        const int wsr = window_start(pq, a.window);
        const bool row_live = rr < rows_s;
        int pgbase = t0 >> a.bs_shift;
        bool bad = false;
        int vpg;
        {
            const bool lane_ok = pgbase + lane <= last_page;
            const bool id_ok = first_raw >= 0 && first_raw < a.num_blocks;
            bad = bad || (lane_ok && !id_ok);
            vpg = lane_ok && id_ok ? first_raw : 0;
        }
        auto issue = [&](int t) {
            const int tl = min(t + kBfTok - 1, tb - 1);
            if ((tl >> a.bs_shift) - pgbase >= kSW) {  // next 64 page ids
                pgbase = t >> a.bs_shift;
                int pg = 0;
                if (pgbase + lane <= last_page) {
                    pg = trow[pgbase + lane];
                    if (pg < 0 || pg >= a.num_blocks) {
                        bad = true;
                        pg = 0;
                    }
                }
                vpg = pg;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // pairs past the piece re-read its last pair (masked)
                const int tt = min(t + 2 * j, (tb - 1) & ~1);
                const int pg = __builtin_amdgcn_readlane(vpg, (tt >> a.bs_shift) - pgbase);
                const size_t off = (((size_t)pg << a.bs_shift) | (size_t)(tt & bs_mask)) * row_bytes;
                __builtin_amdgcn_global_load_lds(uniform_ptr(kbase + off) + k_off[j],
                                                 (lds_void*)(sK + 2 * j * kBfRow), 16, 0, kCpolNT);
                __builtin_amdgcn_global_load_lds(uniform_ptr(vbase + off) + v_off[j],
                                                 (lds_void*)(sV + 2 * j * kBfRow), 16, 0, kCpolNT);
            }
        };

        constexpr int kStepT = IW ? kMaxWaves * kBfTok : kBfTok;  // from one of a wave's batches to the next
        const int t1 = IW ? t0 + kBfTok * wave : t0;               // this wave's first batch
        if (t1 < tb) issue(t1);
        if constexpr (IW) {  // the piece before, while this one's first batch is on its way
            if (pend_s >= 0) finish(pend_s, pend_single, pend_rows, pend_nb, pend_bad);
        }
        m = -INFINITY;
        l = 0.f;
#pragma unroll
        for (int u = 0; u < 16; ++u) o[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        // Q^T as the B operand of step c: column l16 = row rr, dims 32c + 8 grp + e; its hi
        // (column < 8) or lo part, zero for rows past `rows`.
        bf16x8 qreg[8];
        const bool qlive = rr < rows;
        auto split = [&](const float4& q0, const float4& q1) {
            const float xv[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            bf16x8 r;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = qlive ? xv[e] : 0.f;
                const uint16_t h = bf16_rne_bits(x);
                const uint16_t b16 = hi_col ? h : bf16_rne_bits(x - bf16_bits_to_float(h));
                r[e] = __builtin_bit_cast(__bf16, b16);
            }
            return r;
        };
        if constexpr (IW) {
            // Every wave holds the same rows: wave v splits step v into LDS (exchange region 0,
            // which no finish uses between this barrier and the next piece's first one) and
            // reads the eight steps back. The LDS accesses are untracked (copies in flight).
            uint32_t lo = lane;
            asm volatile("" : "+v"(lo));
            const uint32_t qst = lds_addr(red + kBfRedO) + 16 * lo;
            lds_w128(qst + 1024 * wave, __builtin_bit_cast(i32x4, split(qstep[0], qstep[1])));
            __builtin_amdgcn_s_waitcnt(kLgkm0);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            i32x4 qv[8];
            static_for<0, 8>([&](auto C) {
                constexpr int c = decltype(C)::value;
                qv[c] = lds_b128<1024 * c>(qst);
            });
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(qv[0]));
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                asm volatile("" : "+v"(qv[c]));
                qreg[c] = __builtin_bit_cast(bf16x8, qv[c]);
            }
        } else {
#pragma unroll
            for (int c = 0; c < 8; ++c) qreg[c] = split(qraw[c][0], qraw[c][1]);
        }
        int it = 0;  // this wave's batch index in the piece
        for (int t = t1; t < tb; t += kStepT, ++it) {
            __builtin_amdgcn_s_waitcnt(0);  // this batch is in LDS
            if (t + kBfTok > tb - 1 && (tb & 1)) {
                // the batch holds the row after the sequence's last key: zero its V rows
                const int r_bad = tb - t;  // first LDS row past the piece
                for (int r = r_bad; r < kBfTok; r += 2) {  // r_bad is odd: its pair's second row
                    if (lane >= 32) *reinterpret_cast<uint4*>(sV + r * kBfRow + 16 * (lane - 32)) = make_uint4(0, 0, 0, 0);
                }
                __builtin_amdgcn_s_waitcnt(kLgkm0);
            }
            i32x4 kr[8];
            i32x2 vr[16];
            static_for<0, 8>([&](auto C) {
                constexpr int c = decltype(C)::value;
                kr[c] = lds_b128<256 * (c >> 2)>(k_addr[c & 3]);
            });
            static_for<0, 16>([&](auto U) {
                constexpr int u = decltype(U)::value;
                vr[u] = lds_tr16<0>(v_lane + ((uint32_t)(u ^ z) << 5));
            });
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kr[0]), "+v"(kr[1]), "+v"(kr[2]), "+v"(kr[3]));
#pragma unroll
            for (int i = 4; i < 8; ++i) asm volatile("" : "+v"(kr[i]));
#pragma unroll
            for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(vr[i]));
            if (t + kStepT < tb) issue(t + kStepT);

            // S^T over the 8 steps of 32 dims, then hi + lo
            // The two waves of a SIMD (w, w + 4) take turns at the higher priority, batch by
            // batch, so one runs ahead on the matrix cores while the other computes its softmax.
            if ((it + (wave >> 2)) & 1) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
            f32x4 st = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 8; ++c)
                st = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[c]), qreg[c], st, 0, 0, 0);
            float sv[4];
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float full = st[r] + dpp<kRor8>(st[r]);
                const int tok = t + 4 * grp + r;
                const bool ok = row_live && tok >= ta && tok < tb && tok <= pq && tok >= wsr;
                sv[r] = ok ? full * sl2 : -INFINITY;
                mx = fmaxf(mx, sv[r]);
            }
            mx = allreduce_hi<16>(mx, OpMax());
            // lazy reference max (log2 units): p = exp2(s - m) <= 256
            const bool move = mx > m + 8.f;
            const float m_new = move ? mx : m;
            const float alpha = move ? exp2f(m - m_new) : 1.f;  // m = -inf gives 0
            const float m_use = m_new == -INFINITY ? 0.f : m_new;
            float p[4];
            s16x4 pb;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                p[r] = exp2f(sv[r] - m_use);  // masked: exp2(-inf) = 0
                const uint32_t u = __float_as_uint(p[r]);
                const uint16_t h = (uint16_t)(u >> 16);  // P_hi: p truncated to bf16
                pb[r] = (short)(hi_col ? h : bf16_rne_bits(p[r] - __uint_as_float(u & 0xffff0000u)));
            }
            l = l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
            m = m_new;
            if (__any(move)) {
#pragma unroll
                for (int u = 0; u < 16; ++u) o[u] *= alpha;
            }
#pragma unroll
            for (int u = 0; u < 16; ++u)
                o[u] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, vr[u]), pb, o[u], 0, 0, 0);
        }
        bad = __any(bad);
        if constexpr (IW) {
            pend_s = s;
            pend_single = single;
            pend_rows = rows_s;
            pend_nb = (tb - t0 + kBfTok - 1) / kBfTok;
            pend_bad = bad;
        } else {
            finish(s, single, rows_s, 1, bad);
        }
    }
    if constexpr (IW) {
        if (pend_s >= 0) finish(pend_s, pend_single, pend_rows, pend_nb, pend_bad);
    }
}

// Combines the pieces of every sequence that spans more than one workgroup:
//   out = sum_c o_c e^(m_c - M) / (sum_c l_c e^(m_c - M) + 1e-10),  M = max_c m_c,
// the reference's softmax(x)_i = e^(x_i - max) / (sum + 1e-10). One workgroup per
// (row, sequence). A NaN m_c marks a piece that met a table entry outside the pool.
// After the plan, every piece's (m, l) and the o rows of the first kMergeRegs pieces are
// requested together, so a typical sequence costs two memory round trips.
// Fused append: the block-manager state after the call, from the allocation plan the
// attention launch left in the workspace (the launch boundary orders its reads of the old
// state before these writes). As alloc_kernel (pkv_state.hip): the granted table entries,
// table_lens, free_count and every sequence's final status, BAD_BLOCK where a block the
// rows land in has an entry outside the pool.
__device__ inline void write_alloc_state(const StreamArgs& a) {
    const int B = a.batch;
    const int* al = a.plan + B + 3;
    const int fc_raw = al[0];
    const bool fc_bad = fc_raw < 0 || fc_raw > a.num_blocks;
    for (int s = threadIdx.x; s < B; s += blockDim.x) {
        const SeqAlloc r = seq_alloc(al, B, a.num_blocks, s);
        int32_t* table = a.nr.tables + (size_t)s * a.table_stride;
        for (int j = 0; j < r.granted; ++j) table[r.len + j] = a.nr.free_list[r.fc - 1 - r.pref - j];
        if (r.granted > 0) a.nr.table_lens[s] = r.len + r.granted;
        int code = r.code;
        const int p = a.pos[s];
        const int n = a.nr.tok_off[s + 1] - a.nr.tok_off[s];
        if (code == PKV_SEQ_OK && p >= 0 && n > 0) {
            const int b1 = (int)(((long long)p + n - 1) >> a.bs_shift);
            for (int blk = p >> a.bs_shift; blk <= b1; ++blk) {
                const int e = append_block_entry(table, a.nr.free_list, r.len, r.granted, r.fc,
                                                 r.pref, blk);
                if (e < 0 || e >= a.num_blocks) {
                    code = PKV_SEQ_BAD_BLOCK;
                    break;
                }
            }
        }
        a.nr.status[s] = code;
    }
    if (threadIdx.x == 0 && !fc_bad) {
        const int total = al[1 + 2 * B];
        *a.nr.free_count = fc_raw - (total < fc_raw ? total : fc_raw);
    }
}

// grid (rows_seq, batch), plus one row of workgroups (blockIdx.y == batch) with a fused
// append, whose first workgroup writes the state.
template <int D, typename Acc>
__global__ __launch_bounds__(merge_threads<D>()) void stream_merge_kernel(StreamArgs a) {
    constexpr int kMergeNT = merge_threads<D>();
    constexpr int kMaxPieces = 1024;
    // Pieces whose o rows are held in registers, requested with the (m, l) loads. At head_dim
    // 256 a 16-sequence verify or MTP read splits each sequence into ~17 pieces, so 32 keep
    // them in one round trip (config 5's step: 1.134 -> 1.121 ms); at head_dim 512 (the LSA
    // shape's ~9 pieces) 32 measured slower than 16.
    constexpr int kMergeRegs = D == 256 ? 32 : 16;
    constexpr int DPT = D / kMergeNT;       // elements per thread
    static_assert(DPT * kMergeNT == D, "head_dim a multiple of the merge width");
    __shared__ Acc s_w[kMaxPieces];
    __shared__ Acc s_part[kMergeNT / kSW];
    __shared__ int s_nan;
    const int row = blockIdx.x;
    const int s = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & (kSW - 1);
    const int wave = tid / kSW;
    if (s == a.batch) {  // fused append
        if (row == 0) write_alloc_state(a);
        return;
    }
    if (row / a.Hq >= seq_queries(a, s)) return;  // a row past the sequence's queries
    KeySplit sp;
    sp.per_pair = a.plan[0];
    sp.even = a.plan[1];
    const int ps = a.plan[2 + s], pe = a.plan[3 + s];
    if (pe == ps) return;
    const int wf = sp.owner(ps + a.lead), wl = sp.owner(pe - 1);
    if (wf == wl) return;
    const int cnt = wl - wf + 1;  // <= nwg <= kMaxPieces
    const Acc* pml = static_cast<const Acc*>(a.part_ml);
    const Acc* po = static_cast<const Acc*>(a.part_o);
    auto slot_row = [&](int c) -> size_t { return (size_t)(wf + c + s) * a.rows_seq + row; };

    // Requests: (m, l) of this thread's pieces, o of the first kMergeRegs pieces.
    Acc m0 = (Acc)-INFINITY, l0 = (Acc)0;
    if (tid < cnt) {
        m0 = pml[slot_row(tid) * 2];
        l0 = pml[slot_row(tid) * 2 + 1];
    }
    Acc oreg[kMergeRegs][DPT];
#pragma unroll
    for (int c = 0; c < kMergeRegs; ++c)
#pragma unroll
        for (int e = 0; e < DPT; ++e)
            oreg[c][e] = c < cnt ? po[slot_row(c) * D + tid + e * kMergeNT] : (Acc)0;

    if (tid == 0) s_nan = 0;
    __syncthreads();
    Acc M = (Acc)-INFINITY;
    if (tid < cnt) {
        if (m0 != m0) s_nan = 1;
        M = m0;
        s_w[tid] = m0;
    }
    for (int c = tid + kMergeNT; c < cnt; c += kMergeNT) {
        const Acc m = pml[slot_row(c) * 2];
        if (m != m) s_nan = 1;
        M = fmax(M, m);
        s_w[c] = m;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmax(M, __shfl_xor(M, o));
    if (lane == 0) s_part[wave] = M;
    __syncthreads();
    M = s_part[0];
#pragma unroll
    for (int i = 1; i < kMergeNT / kSW; ++i) M = fmax(M, s_part[i]);
    __syncthreads();
    Acc L = (Acc)0;
    if (tid < cnt) {
        const Acc wgt = (m0 == (Acc)-INFINITY) ? (Acc)0 : exp_acc(m0 - M);
        s_w[tid] = wgt;
        L = l0 * wgt;
    }
    for (int c = tid + kMergeNT; c < cnt; c += kMergeNT) {
        const Acc m = s_w[c];
        const Acc wgt = (m == (Acc)-INFINITY) ? (Acc)0 : exp_acc(m - M);
        s_w[c] = wgt;
        L += pml[slot_row(c) * 2 + 1] * wgt;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) L += __shfl_xor(L, o);
    if (lane == 0) s_part[wave] = L;
    __syncthreads();
    L = (Acc)0;
#pragma unroll
    for (int i = 0; i < kMergeNT / kSW; ++i) L += s_part[i];
    const Acc inv = (Acc)1 / (L + (Acc)1e-10);
    const bool nan = s_nan != 0;
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
        const int d = tid + e * kMergeNT;
        Acc o8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o8[i] = (Acc)0;
#pragma unroll
        for (int c = 0; c < kMergeRegs; ++c)  // pieces past cnt hold weight-free zeros
            if (c < cnt) o8[c % 8] = fma(s_w[c], oreg[c][e], o8[c % 8]);
        int c = kMergeRegs;
        for (; c + 8 <= cnt; c += 8) {  // eight independent loads in flight
#pragma unroll
            for (int i = 0; i < 8; ++i) o8[i] = fma(s_w[c + i], po[slot_row(c + i) * D + d], o8[i]);
        }
        for (; c < cnt; ++c) o8[0] = fma(s_w[c], po[slot_row(c) * D + d], o8[0]);
        const Acc o = ((o8[0] + o8[1]) + (o8[2] + o8[3])) + ((o8[4] + o8[5]) + (o8[6] + o8[7]));
        a.out[(((size_t)s * a.q_len + a.j0) * a.Hq + row) * D + d] =
            nan ? __builtin_nanf("") : (float)(o * inv);
    }
}

// ---- host -------------------------------------------------------------------------

constexpr int kMaxSlots = kStreamMaxSlots;  // workgroups along the keys, at most (merge LDS bound)

// Dynamic LDS of the vector stream kernel: the per-sequence ints, plus the allocation plan
// of a fused append.
size_t stream_vector_lds(int batch, bool fused) {
    return (size_t)(stream_seq_ints(batch) + (fused ? 3 * batch + 2 : 0)) * sizeof(int);
}

// Workgroups that fill the device once (all resident together), capped at kMaxSlots.
int fill_workgroups(const void* fn, int threads, size_t lds) {
    return device_fill_workgroups(fn, threads, lds, kMaxSlots);
}

template <int D, typename KV, int R, int WPH, int ADDR>
int32_t launch_addr(StreamArgs a, hipStream_t st) {
    using Acc = typename SKV<KV>::Acc;
    const int waves = a.Hkv * WPH < kMaxWaves ? a.Hkv * WPH : kMaxWaves;
    const int threads = waves * kSW;
    const bool fused = ADDR == kAddrPaged && a.nr.k_new && a.j0 == 0;
    const size_t lds = stream_vector_lds(a.batch, fused);
    if constexpr (D == 256 && WPH == 1 && ADDR != kAddrSparse) {
        // Interleaved waves: grid (nwg, Hkv), eight waves per kv head.
        const size_t lds_iw = vec_red_offset(a.batch, fused) + vec_red_bytes();
        if (lds_iw <= kStreamLdsMax) {
            const void* fn = reinterpret_cast<const void*>(&stream_attend_kernel<D, KV, R, WPH, ADDR, true>);
            if (lds_iw > 64 * 1024 && !reserve_lds(fn, (int)kStreamLdsMax))
                return fail(PKV_ERR_HIP, "pkv_attend: could not reserve the kernel's LDS");
            const int slots = fill_workgroups(fn, kMaxWaves * kSW, lds_iw);
            if (slots <= 0) return fail(PKV_ERR_HIP, "pkv_attend: occupancy query failed");
            a.nwg = slots / a.Hkv > 0 ? slots / a.Hkv : 1;
            if (a.nwg > a.nwg_cap) a.nwg = a.nwg_cap;
            if (a.nwg > 1) a.nwg &= ~1;  // whole pairs (key_split)
            a.lead = PKV_LEAD_VEC_IW;
            hipLaunchKernelGGL((stream_attend_kernel<D, KV, R, WPH, ADDR, true>), dim3(a.nwg, a.Hkv),
                               dim3(kMaxWaves * kSW), lds_iw, st, a);
            if (hipGetLastError() != hipSuccess)
                return fail(PKV_ERR_HIP, "pkv_attend: the attention launch failed");
            hipLaunchKernelGGL((stream_merge_kernel<D, Acc>), dim3(a.rows_seq, a.batch + (fused ? 1 : 0)),
                               dim3(merge_threads<D>()), 0, st, a);
            return PKV_OK;
        }
    }
    const void* fn = reinterpret_cast<const void*>(&stream_attend_kernel<D, KV, R, WPH, ADDR>);
    if (lds > kStreamLdsMax)  // stream_attend refuses such batches before any launch
        return fail(PKV_ERR_UNSUPPORTED, "pkv_attend: batch too large for the kernel's LDS");
    // Above 64 KiB of dynamic LDS a kernel must opt in (once per kernel and device).
    if (lds > 64 * 1024 &&
        !reserve_lds(fn, (int)kStreamLdsMax))
        return fail(PKV_ERR_HIP, "pkv_attend: could not reserve the kernel's LDS");
    const int slots = fill_workgroups(fn, threads, lds);
    if (slots <= 0) return fail(PKV_ERR_HIP, "pkv_attend: occupancy query failed");
    // Resident workgroups only: the head groups share the slots, and each workgroup
    // covers ceil(total / nwg) keys.
    const int groups = (a.Hkv * WPH + kMaxWaves - 1) / kMaxWaves;
    a.nwg = slots / groups > 0 ? slots / groups : 1;
    if (a.nwg > a.nwg_cap) a.nwg = a.nwg_cap;
    if (a.nwg > 1) a.nwg &= ~1;  // whole pairs (key_split)
    a.lead = PKV_LEAD_VEC;
    dim3 grid(groups, a.nwg);
    hipLaunchKernelGGL((stream_attend_kernel<D, KV, R, WPH, ADDR>), grid, dim3(threads), lds, st,
                       a);
    // the merge reads the plan this launch writes
    if (hipGetLastError() != hipSuccess)
        return fail(PKV_ERR_HIP, "pkv_attend: the attention launch failed");
    hipLaunchKernelGGL((stream_merge_kernel<D, Acc>), dim3(a.rows_seq, a.batch + (fused ? 1 : 0)),
                       dim3(merge_threads<D>()), 0, st, a);
    return PKV_OK;
}

template <int D, typename KV, int R, int WPH = 1>
int32_t launch_r(StreamArgs a, hipStream_t st);
constexpr size_t kMfmaLdsMax = kStreamLdsMax;

#ifndef PKV_MFMA_HEADS_PER_WG
#define PKV_MFMA_HEADS_PER_WG 2
#endif
// Interleaved waves (head_dim 256, paged or ring pools): grid (nwg, Hkv), eight waves per
// kv head. False when the batch's LDS does not fit it (the caller then takes the launch
// below).
template <int ADDR>
bool launch_mfma_iw(StreamArgs& a, hipStream_t st, int32_t* rc) {
    constexpr int D = 256, RG = 2, TG = 1;
    const bool fused = ADDR == kAddrPaged && a.nr.k_new && a.j0 == 0;
    const size_t lds = mfma_stage_offset(a.batch, fused) + (size_t)kMaxWaves * mfma_stage_bytes(D, TG) +
                       iw_red_bytes();
    if (lds > kMfmaLdsMax) return false;
    constexpr bool kFusable = ADDR == kAddrPaged;
    const void* fn = fused ? reinterpret_cast<const void*>(&stream_mfma_kernel<D, RG, TG, 1, ADDR, kFusable, true>)
                           : reinterpret_cast<const void*>(&stream_mfma_kernel<D, RG, TG, 1, ADDR, false, true>);
    if (!reserve_lds(fn, (int)kMfmaLdsMax)) {
        *rc = fail(PKV_ERR_HIP, "pkv_attend: could not reserve the kernel's LDS");
        return true;
    }
    const int slots = fill_workgroups(fn, kMaxWaves * kSW, lds);
    if (slots <= 0) {
        *rc = fail(PKV_ERR_HIP, "pkv_attend: occupancy query failed");
        return true;
    }
    // every kv head's workgroups take the same key split; nwg even keeps column w on XCD w mod 8
    a.nwg = slots / a.Hkv > 0 ? slots / a.Hkv : 1;
    if (a.nwg > a.nwg_cap) a.nwg = a.nwg_cap;
    if (a.nwg > 1) a.nwg &= ~1;  // whole pairs (key_split)
    a.lead = PKV_LEAD_IW;
    const dim3 grid(a.nwg, a.Hkv);
    if (fused)
        hipLaunchKernelGGL((stream_mfma_kernel<D, RG, TG, 1, ADDR, kFusable, true>), grid, dim3(kMaxWaves * kSW), lds, st, a);
    else
        hipLaunchKernelGGL((stream_mfma_kernel<D, RG, TG, 1, ADDR, false, true>), grid, dim3(kMaxWaves * kSW), lds, st, a);
    if (hipGetLastError() != hipSuccess) {
        *rc = fail(PKV_ERR_HIP, "pkv_attend: the attention launch failed");
        return true;
    }
    hipLaunchKernelGGL((stream_merge_kernel<D, double>), dim3(a.rows_seq, a.batch + (fused ? 1 : 0)),
                       dim3(merge_threads<D>()), 0, st, a);
    *rc = PKV_OK;
    return true;
}

template <int D, int RG, int TG, int WPH, int ADDR>
int32_t launch_mfma_addr(StreamArgs a, hipStream_t st) {
    if constexpr (D == 256 && WPH == 1 && RG == 2 && TG == 1 && ADDR != kAddrSparse) {
        int32_t rc = PKV_OK;
        if (launch_mfma_iw<ADDR>(a, st, &rc)) return rc;
    }
    // WPH > 1: the waves of a head meet at a barrier every batch, so a workgroup holds few
    // heads (a barrier waits for every wave of the workgroup).
    constexpr int kHeadsMax = WPH == 1 ? kMaxWaves : PKV_MFMA_HEADS_PER_WG;
    const int waves = (a.Hkv < kHeadsMax ? a.Hkv : kHeadsMax) * WPH;
    const int threads = waves * kSW;
    const bool fused = ADDR == kAddrPaged && a.nr.k_new && a.j0 == 0;
    const size_t lds = mfma_stage_offset(a.batch, fused) + (size_t)waves * mfma_stage_bytes(D, TG);
    if (lds > kMfmaLdsMax) {  // very large batches: the vector kernel
        if constexpr (D == 256) return launch_r<256, float, 4, 2>(a, st);
        else return launch_r<512, float, 2, 4>(a, st);
    }
    constexpr bool kFusable = ADDR == kAddrPaged;
    const void* fn = fused ? reinterpret_cast<const void*>(&stream_mfma_kernel<D, RG, TG, WPH, ADDR, kFusable>)
                           : reinterpret_cast<const void*>(&stream_mfma_kernel<D, RG, TG, WPH, ADDR, false>);
    // Above 64 KiB of dynamic LDS a kernel must opt in (once per kernel and device).
    if (!reserve_lds(fn, (int)kMfmaLdsMax))
        return fail(PKV_ERR_HIP, "pkv_attend: could not reserve the kernel's LDS");
    const int slots = fill_workgroups(fn, threads, lds);
    if (slots <= 0) return fail(PKV_ERR_HIP, "pkv_attend: occupancy query failed");
    const int groups = (a.Hkv * WPH + waves - 1) / waves;
    a.nwg = slots / groups > 0 ? slots / groups : 1;
    if (a.nwg > a.nwg_cap) a.nwg = a.nwg_cap;
    if (a.nwg > 1) a.nwg &= ~1;  // whole pairs (key_split)
    a.lead = PKV_LEAD_MFMA;
    dim3 grid(groups, a.nwg);
    if (fused)
        hipLaunchKernelGGL((stream_mfma_kernel<D, RG, TG, WPH, ADDR, kFusable>), grid, dim3(threads), lds, st, a);
    else
        hipLaunchKernelGGL((stream_mfma_kernel<D, RG, TG, WPH, ADDR, false>), grid, dim3(threads), lds, st, a);
    if (hipGetLastError() != hipSuccess)
        return fail(PKV_ERR_HIP, "pkv_attend: the attention launch failed");
    hipLaunchKernelGGL((stream_merge_kernel<D, double>), dim3(a.rows_seq, a.batch + (fused ? 1 : 0)),
                       dim3(merge_threads<D>()), 0, st, a);
    return PKV_OK;
}

#ifndef PKV_MFMA_TG
#define PKV_MFMA_TG 1
#endif
// head_dim 256: one wave of 8 rows per kv head. (Two waves of 4 rows sharing the staging,
// two 8-wave workgroups per CU at 128 registers, spilled 24 registers and ran the config 5
// verify launch at 176 against 126 us.) head_dim 512: two waves of 4 rows.
template <int D>
int32_t launch_mfma(StreamArgs a, hipStream_t st) {
    constexpr int WPH = D == 256 ? 1 : 2;
    constexpr int RG = 2 / WPH;  // 8 rows per head over WPH waves
    if constexpr (D == 256) {
        if (a.keys) return launch_mfma_addr<D, RG, PKV_MFMA_TG, WPH, kAddrSparse>(a, st);
    }
    return a.ring_size > 0 ? launch_mfma_addr<D, RG, PKV_MFMA_TG, WPH, kAddrRing>(a, st)
                           : launch_mfma_addr<D, RG, PKV_MFMA_TG, WPH, kAddrPaged>(a, st);
}

// bf16 pools, head_dim 256, 5..8 rows per kv head: the bf16 matrix cores (paged pools,
// block_size >= 2: a copy pair lies in one block); else two vector waves of 4 rows.
int32_t launch_bf16_mfma(StreamArgs a, hipStream_t st) {
    const int waves = a.Hkv < kMaxWaves ? a.Hkv : kMaxWaves;
    const int threads = waves * kSW;
    const size_t lds = mfma_stage_offset(a.batch, false) + (size_t)waves * kBfStage;
    if (lds > kMfmaLdsMax || a.keys || a.ring_size > 0 || a.bs_shift < 1 || a.nr.k_new)
        return launch_r<256, uint16_t, 4, 2>(a, st);
    // Interleaved waves (grid (nwg, Hkv), eight waves per kv head) where the batch's LDS fits.
    const size_t lds_iw = mfma_stage_offset(a.batch, false) + (size_t)kMaxWaves * kBfStage + bf_iw_red_bytes();
    if (lds_iw <= kMfmaLdsMax) {
        const void* fn = reinterpret_cast<const void*>(&stream_bf16_mfma_kernel<kAddrPaged, true>);
        if (!reserve_lds(fn, (int)kMfmaLdsMax))
            return fail(PKV_ERR_HIP, "pkv_attend: could not reserve the kernel's LDS");
        const int slots = fill_workgroups(fn, kMaxWaves * kSW, lds_iw);
        if (slots <= 0) return fail(PKV_ERR_HIP, "pkv_attend: occupancy query failed");
        a.nwg = slots / a.Hkv > 0 ? slots / a.Hkv : 1;
        if (a.nwg > a.nwg_cap) a.nwg = a.nwg_cap;
        if (a.nwg > 1) a.nwg &= ~1;  // whole pairs (key_split)
        a.lead = PKV_LEAD_BF16_IW;
        hipLaunchKernelGGL((stream_bf16_mfma_kernel<kAddrPaged, true>), dim3(a.nwg, a.Hkv), dim3(kMaxWaves * kSW),
                           lds_iw, st, a);
        if (hipGetLastError() != hipSuccess)
            return fail(PKV_ERR_HIP, "pkv_attend: the attention launch failed");
        hipLaunchKernelGGL((stream_merge_kernel<256, float>), dim3(a.rows_seq, a.batch), dim3(merge_threads<256>()), 0,
                           st, a);
        return PKV_OK;
    }
    const void* fn = reinterpret_cast<const void*>(&stream_bf16_mfma_kernel<kAddrPaged>);
    if (!reserve_lds(fn, (int)kMfmaLdsMax))
        return fail(PKV_ERR_HIP, "pkv_attend: could not reserve the kernel's LDS");
    const int slots = fill_workgroups(fn, threads, lds);
    if (slots <= 0) return fail(PKV_ERR_HIP, "pkv_attend: occupancy query failed");
    const int groups = (a.Hkv + kMaxWaves - 1) / kMaxWaves;
    a.nwg = slots / groups > 0 ? slots / groups : 1;
    if (a.nwg > a.nwg_cap) a.nwg = a.nwg_cap;
    if (a.nwg > 1) a.nwg &= ~1;  // whole pairs (key_split)
    a.lead = PKV_LEAD_BF16;
    hipLaunchKernelGGL((stream_bf16_mfma_kernel<kAddrPaged>), dim3(groups, a.nwg), dim3(threads), lds,
                       st, a);
    if (hipGetLastError() != hipSuccess)
        return fail(PKV_ERR_HIP, "pkv_attend: the attention launch failed");
    hipLaunchKernelGGL((stream_merge_kernel<256, float>), dim3(a.rows_seq, a.batch), dim3(merge_threads<256>()), 0,
                       st, a);
    return PKV_OK;
}

template <int D, typename KV, int R, int WPH>
int32_t launch_r(StreamArgs a, hipStream_t st) {
    if (a.keys) return launch_addr<D, KV, R, WPH, kAddrSparse>(a, st);
    return a.ring_size > 0 ? launch_addr<D, KV, R, WPH, kAddrRing>(a, st)
                           : launch_addr<D, KV, R, WPH, kAddrPaged>(a, st);
}

// One launch (attention + merge) for `rows` <= 8 query rows per kv head. head_dim 256:
// one wave holds up to 4 rows (bf16 pools: two waves of 4 for 5..8); head_dim 512: waves of
// 2 rows. fp32 pools with 5..8 rows run on the fp64 matrix cores.
template <typename KV>
int32_t launch_rows(StreamArgs a, int D, int rows, hipStream_t st) {
    if (D == 256) {
        if (rows <= 1) return launch_r<256, KV, 1>(a, st);
        if (rows <= 2) return launch_r<256, KV, 2>(a, st);
        if (rows > 4) {  // fp32 pools: the fp64 matrix cores; bf16 pools: the bf16 ones
            if constexpr (sizeof(KV) == 4) return launch_mfma<256>(a, st);
            else return launch_bf16_mfma(a, st);
        }
        return launch_r<256, KV, 4>(a, st);
    }
    if (rows <= 1) return launch_r<512, KV, 1>(a, st);
    if (rows <= 2) return launch_r<512, KV, 2>(a, st);
    if constexpr (sizeof(KV) == 4) {
        // Key lists (LSA) are a few hundred keys per sequence, pieces of a few dozen keys:
        // there the vector kernel's shorter start wins (LSA shape 40 against 51 us).
        if (rows > 4 && !a.keys) return launch_mfma<512>(a, st);
    }
    if (rows <= 4) return launch_r<512, KV, 2, 2>(a, st);
    return launch_r<512, KV, 2, 4>(a, st);
}

}  // namespace

StreamLayout stream_layout(const pkv_params* p, int32_t batch, int32_t q_len, int32_t nwg_cap) {
    StreamLayout L{};
    auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t rows = (size_t)p->num_heads * q_len;
    const size_t slots = (size_t)(nwg_cap < kMaxSlots ? nwg_cap : kMaxSlots) + batch;
    L.plan_off = 0;
    L.ml_off = align((size_t)(4 * (size_t)batch + 5) * sizeof(int32_t));
    L.o_off = L.ml_off + align(slots * rows * 2 * sizeof(double));
    L.total = L.o_off + align(slots * rows * (size_t)p->head_dim * sizeof(double));
    return L;
}

bool stream_eligible(const pkv_params* p, int32_t G) {
    return (p->head_dim == 256 || p->head_dim == 512) && G >= 1 && G <= 8;
}

bool stream_takes_new_rows(const pkv_params* p, int32_t q_len, int32_t batch) {
    const int G = p->num_heads / p->num_kv_heads;
    if (p->ring_size > 0 || !stream_eligible(p, G) || batch > kFuseMaxBatch) return false;
    const int rows = G * q_len;
    if (rows > 8) return false;  // one launch (no query groups)
    const bool bf16 = p->kv_dtype == PKV_DTYPE_BF16;
    if (!bf16 && rows > 4) return true;  // the fp64 MFMA kernel (any number of head groups)
    // vector kernel: one head group, every kv head's waves in one workgroup
    int wph = 1;
    if (p->head_dim == 256) wph = rows <= 4 ? 1 : 2;
    else wph = rows <= 2 ? 1 : (rows <= 4 ? 2 : 4);
    return p->num_kv_heads * wph <= kMaxWaves;
}

int32_t stream_attend(const pkv_params* p, const float* q, const void* k_pool,
                      const void* v_pool, const int32_t* block_tables, int32_t table_stride,
                      const int32_t* pos, int32_t pos_scalar, int64_t ring_base, int32_t q_len,
                      const int32_t* q_lens, int32_t batch, int32_t max_pos, const int32_t* keys,
                      const int32_t* key_off, int32_t max_keys, float* out, void* workspace,
                      hipStream_t st, const NewRows* nr, int32_t nwg_cap) {
    const int G = p->num_heads / p->num_kv_heads;
    if (!stream_eligible(p, G)) return fail(PKV_ERR_UNSUPPORTED, "stream path: geometry");
    if (nwg_cap < 1) return fail(PKV_ERR_WORKSPACE, "stream path: no room for one workgroup's partials");
    StreamLayout lay = stream_layout(p, batch, q_len, nwg_cap);
    StreamArgs a{};
    char* ws = static_cast<char*>(workspace);
    a.q = q;
    a.k_pool = static_cast<const char*>(k_pool);
    a.v_pool = static_cast<const char*>(v_pool);
    a.tables = block_tables;
    a.table_stride = table_stride;
    a.pos = pos;
    a.pos_scalar = pos_scalar;
    a.q_len = q_len;
    a.q_lens = q_lens;
    a.keys = keys;
    a.key_off = key_off;
    a.max_keys = max_keys;
    a.Hq = p->num_heads;
    a.Hkv = p->num_kv_heads;
    a.G = G;
    a.bs_shift = __builtin_ctz((unsigned)p->block_size);
    a.num_blocks = p->num_blocks;
    a.window = p->window;
    a.scale = p->scale;
    a.ring_size = p->ring_size;
    a.ring_base = ring_base;
    a.max_pos = max_pos;
    a.batch = batch;
    a.nwg_cap = nwg_cap < kMaxSlots ? nwg_cap : kMaxSlots;
    a.plan = reinterpret_cast<int32_t*>(ws + lay.plan_off);
    a.part_ml = ws + lay.ml_off;
    a.part_o = ws + lay.o_off;
    a.out = out;
    if (nr) {
        if (!stream_takes_new_rows(p, q_len, batch))
            return fail(PKV_ERR_UNSUPPORTED, "stream path: appended rows need one launch");
        a.nr = *nr;
    }
    // Every launch below fits the CU's LDS if the first (the largest) does: refuse before
    // any launch otherwise.
    if (stream_vector_lds(batch, nr != nullptr) > kStreamLdsMax)
        return fail(PKV_ERR_UNSUPPORTED, "stream path: batch too large for the kernel's LDS");
    const bool bf16 = p->kv_dtype == PKV_DTYPE_BF16;
    // Queries in groups of at most 8 query rows per kv head, one launch pair each; the
    // launches share the workspace in stream order.
    const int per_launch = 8 / G;
    for (int j0 = 0; j0 < q_len; j0 += per_launch) {
        a.j0 = j0;
        a.q_cnt = q_len - j0 < per_launch ? q_len - j0 : per_launch;
        a.rows_seq = p->num_heads * a.q_cnt;
        const int rows = G * a.q_cnt;
        const int32_t rc = bf16 ? launch_rows<uint16_t>(a, p->head_dim, rows, st)
                                : launch_rows<float>(a, p->head_dim, rows, st);
        if (rc != PKV_OK) return rc;
    }
    return PKV_OK;
}

}  // namespace pkv
