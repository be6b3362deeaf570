// sampler_kernels.hip - gfx950 (CDNA4) kernels of the token sampler and the C ABI of include/ferro_sampler.h.
//
// One kernel per call on the caller's stream (two when a row is shorter than one 4096-logit tile).
//
// segment_kernel (one 512-thread workgroup per (row, segment) item, two per CU): a row of V fp32 logits is split
// into nseg segments of seg_tiles tiles (TILE = 4096 logits); the items are dealt to the 8 XCDs so that a row's
// segments share one XCD and its L2. A segment is streamed from HBM with PF tiles in flight (16-byte buffer
// loads, the only pass over the logits). Per tile:
//   - penalty pass on the fly (reference src/sampler.cpp:11-18, plus the frequency/presence extension):
//     repetition only - an exact bitmap of the window's ids in the segment; with counts - the window ids that fall
//     in the tile are counted in a 16-bit LDS table; each thread patches the few penalised logits it holds;
//   - greedy rows (temperature <= 0 or top_k == 1, sampler.cpp:19): each lane keeps its first maximum;
//   - top-k rows: every logit is compared with a running fp32 bound tf (a lower bound of the row's k-th key) in a
//     wave ballot; the few that pass are appended to an LDS buffer as 64-bit composites (key << 32 | ~id: integer
//     order = ferro's candidate order, value desc then id asc, sampler.cpp:30).
// The bound starts from tile 0's histogram and is raised from a per-row histogram of counted logits shared by the
// row's segments (L2 atomics): any k counted logits at or above a bin make its lower edge a valid bound. The
// buffer is compacted (entries below the bound dropped, else the exact k-th composite kept) when it could
// overflow. Each segment publishes its candidates at or above its final bound.
//
// The merge (a role of the same grid: one workgroup per row after the segments, on the row's XCD; a separate
// merge_kernel launch when rows are shorter than one tile): waits for the row's segment count in the L2, gathers
// the segments' lists, L = max of the segments' bounds bounds the
// row's k-th key from below, a histogram over [L, max] gives a tight T1, the ~k candidates >= T1 are sorted in
// LDS (ferro's cand_, sampler.cpp:25-35; rank sort or a counting sort), then the double-precision softmax at
// temperature, min-p, top-p and the draw r = u * tot (sampler.cpp:37-49), with scans in place of the sequential
// sums. Rows with k > 2048 are sampled here by whole-row passes. Verify windows (server.cpp:627-637): the last
// row of a stream to finish (agent-scope sc1 stores, a vmcnt drain and an agent-scope counter, no L2 write-back)
// computes the accepted prefix.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <new>
#include <random>
#include <vector>

#include "../../include/ferro_sampler.h"

#if !defined(__gfx950__) && defined(__HIP_DEVICE_COMPILE__)
#error "ferro sampler kernels are written for gfx950 only"
#endif

namespace fs {

constexpr int BLOCK = 512;                // threads per workgroup: 8 wave64s, two workgroups per CU
constexpr int WAVE = 64;
constexpr int NWAVES = BLOCK / WAVE;
constexpr int TPT = 8;                    // logits per thread per tile
constexpr int NV = TPT / 4;               // float4 loads per thread per tile
constexpr int TILE = BLOCK * TPT;         // 4096 logits per tile
constexpr int PF = 2;                     // tiles in flight per workgroup
constexpr int KMAX = 2048;                // largest k on the fused select path
constexpr int KPT = KMAX / BLOCK;         // candidates per thread in the softmax / draw phase
constexpr int CAP = KMAX + TILE;          // candidate buffer (LDS), per-segment list in the workspace, merge gather
constexpr int HBITS = 11;
constexpr int NBINS = 1 << HBITS;         // threshold histograms
constexpr int SMALL = 512;                // rank-sort capacity of the merge
constexpr int MAX_SEGS = 1024;            // segments per row
constexpr int SPEC = 2;                   // merge gather: loads in flight per thread per round
constexpr int FAST_SEGS = 64;             // merge fast path: a wave reads every list's bound and count
static_assert(SPEC * BLOCK + SMALL + 2 * WAVE + 4 * 2 * WAVE / 2 <= CAP, "merge fast path: list, ranks and finish buffers fit");
constexpr int RBITS = 12;                 // row histogram: bins of the top key bits, shared by a row's segments
constexpr int RBINS = 1 << RBITS;
constexpr int RSHIFT = 32 - RBITS;
constexpr int XCDS = 8;                   // MI355X: 8 XCDs, workgroups dealt round-robin by index
constexpr int WIDS = 2048;                // penalty-window ids of one segment kept in LDS (longer: rescanned per tile)

enum Mode : int { MODE_SAMPLE = 0, MODE_ARGMAX = 1, MODE_VERIFY = 2 };

struct Args {
    const float* logits;
    int64_t ld;
    int B;            // rows
    int V;
    const int32_t* hist;
    const int64_t* hist_off;
    const fs_row_params* params;   // NULL: no penalties (argmax mode only)
    const double* u;
    int32_t* tok;
    int kcap;
    int32_t* cand_ids;
    double* cand_probs;
    int32_t* keep;
    const int32_t* rows;           // verify: tokens fed per row
    const int64_t* row_off;        // verify: stream -> rows
    int n_streams;
    int eos;
    int32_t* accepted;
    int mode;
    int nseg;                      // segments per row (the default layout)
    int balance;                   // nonzero: each XCD splits its workgroups among its rows by the rows' cost
    int seg_tiles;                 // tiles per segment
    uint64_t* cand;                // [B*nseg][CAP]
    uint32_t* meta;                // [B*nseg][2]: lower bound of the k-th key, count
    uint32_t* rhist;               // [B][RBINS] row histograms of the segments' candidates, left at 0
    uint64_t* rmass;               // [B][4096] fixed-point mass histograms of large rows' candidates, left at 0
    uint32_t* stream_cnt;          // [n_streams] verify completion counters, left at 0
    int32_t* err;                  // device error bits
    int32_t* dirty;                // nonzero: a merge gave up waiting; the row histograms and counters may be stale
    uint32_t merge_spins;          // bounded wait of the merge role (polls); 0: give up without waiting
    uint64_t* trace;               // FS_TRACE builds: per-workgroup phase timestamps (NULL: none)
    // one-launch decode step (fs_decode_step): the draws come from device streams (row r = stream r) instead of u,
    // and each row's token is appended to its stream's history, out of place
    uint64_t* dmt;                 // [B][312] mt19937_64 states (NULL: draws from u)
    int32_t* didx;                 // [B] their next indices
    int32_t* out_hist;             // the histories with the tokens appended (NULL: no append)
    int64_t* out_hist_off;         // [B + 1]
    int64_t out_cap;               // ids out_hist holds
};

constexpr int MT_N = 312, MT_M = 156;
constexpr uint64_t MT_A = 0xB5026F5AA96619E9ull, MT_UPPER = 0xFFFFFFFF80000000ull, MT_LOWER = 0x7FFFFFFFull;

__device__ __forceinline__ uint64_t mt_temper(uint64_t y) {
    y ^= (y >> 29) & 0x5555555555555555ull;
    y ^= (y << 17) & 0x71D67FFFEDA60000ull;
    y ^= (y << 37) & 0xFFF7EEE000000000ull;
    y ^= y >> 43;
    return y;
}
__device__ __forceinline__ uint64_t mt_twist_one(uint64_t cur, uint64_t next, uint64_t far) {
    const uint64_t x = (cur & MT_UPPER) | (next & MT_LOWER);
    return far ^ (x >> 1) ^ ((x & 1ull) ? MT_A : 0ull);
}
__device__ void mt_twist(uint64_t* mt) {
    for (int k = 0; k < MT_N; ++k) mt[k] = mt_twist_one(mt[k], mt[(k + 1) % MT_N], mt[(k + MT_M) % MT_N]);
}
__device__ __forceinline__ double mt_canonical(uint64_t x) {
    const double r = __ull2double_rn(x) * 0x1p-64;
    return r < 1.0 ? r : 0x1.fffffffffffffp-1;
}
__device__ __forceinline__ bool samples(const fs_row_params& p) { return p.temperature > 0.0f && p.top_k != 1; }

// The draw of row `row` (sampler.cpp:45-46): u from the caller, or, in a decode step, the next value of the row's
// device stream, read without advancing it (the row's merge commits it after every reader is done).
__device__ __forceinline__ double row_u(const Args& a, int row) {
    if (a.dmt) {
        const uint64_t* mt = a.dmt + (int64_t)row * MT_N;
        const int idx = a.didx[row];
        const uint64_t y = idx < MT_N ? mt[idx] : mt_twist_one(mt[0], mt[1], mt[MT_M]);
        return mt_canonical(mt_temper(y));
    }
    return a.u ? a.u[row] : 0.0;
}

// Phase timestamps (FS_TRACE builds only; the product library compiles these to nothing): thread 0 of a workgroup
// keeps the constant 100 MHz clock (s_memrealtime) of phase i in LDS (no memory store, so no wait on the memory
// counter in the middle of the kernel) and writes them to trace[blockIdx * TRACE_W + i] at its end; slots 13-15 hold
// the role (1 segment, 2 merge), the row and the segment.
[[maybe_unused]] constexpr int TRACE_W = 16;
#ifdef FS_TRACE
#define FS_MARK(i)                                                                                        \
    do {                                                                                                  \
        if (threadIdx.x == 0) s.trace_t[(i)] = __builtin_amdgcn_s_memrealtime();                          \
    } while (0)
#define FS_TAG(i, v)                                                                                      \
    do {                                                                                                  \
        if (threadIdx.x == 0) s.trace_t[(i)] = (uint64_t)(v);                                            \
    } while (0)
// the latest of the workgroup's waves to reach phase i (lane 0 of each wave)
#define FS_MARKW(i)                                                                                       \
    do {                                                                                                  \
        if (lane_id() == 0) atomicMax((unsigned long long*)&s.trace_t[(i)],                               \
                                      (unsigned long long)__builtin_amdgcn_s_memrealtime());              \
    } while (0)
#define FS_FLUSH()                                                                                        \
    do {                                                                                                  \
        if (threadIdx.x == 0 && a.trace)                                                                  \
            for (int i_ = 0; i_ < TRACE_W; ++i_) a.trace[(int64_t)blockIdx.x * TRACE_W + i_] = s.trace_t[i_]; \
    } while (0)
#else
#define FS_MARK(i) do {} while (0)
#define FS_TAG(i, v) do {} while (0)
#define FS_MARKW(i) do {} while (0)
#define FS_FLUSH() do {} while (0)
#endif

// ------------------------------------------------------------------------------------------------ keys
// Order-preserving map fp32 -> u32: larger float -> larger key; -0 and +0 share a key (sampler.cpp:30 compares
// with == and >, under which they are equal); NaN maps below every number.
__device__ __forceinline__ uint32_t key_of(float x) {
    uint32_t u = __float_as_uint(x);
    if (x != x) return 0u;
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float val_of(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}
// Composite: ordered like ferro's candidate order (value desc, id asc) when compared as integers, descending.
__device__ __forceinline__ uint64_t comp_of(uint32_t key, uint32_t id) {
    return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - id);
}
__device__ __forceinline__ uint32_t comp_id(uint64_t c) { return 0xFFFFFFFFu - (uint32_t)c; }
__device__ __forceinline__ uint32_t comp_key(uint64_t c) { return (uint32_t)(c >> 32); }

// ------------------------------------------------------------------------------------------------ hand-off I/O
// Agent-scope relaxed accesses compile to sc1 loads/stores: coherent across the XCDs' L2s without a write-back.
__device__ __forceinline__ void st_agent(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(int32_t* p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_agent(const int32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this wave's vector memory operations (the sc1 stores above) have completed.
__device__ __forceinline__ void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Invalidate the CU's L1 (vector cache): later loads are served by the XCD's L2, which holds what other workgroups
// of this XCD stored or added (stores write through the L1; atomics execute in the L2).
__device__ __forceinline__ void l1_invalidate() { asm volatile("buffer_inv sc0" ::: "memory"); }

// ------------------------------------------------------------------------------------------------ wave/block
__device__ __forceinline__ int lane_id() { return __lane_id(); }
__device__ __forceinline__ uint32_t mbcnt(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Cross-lane moves for whole waves (every call site runs with all 64 lanes active). DPP moves and lane reads stay
// in the VALU; the LDS permute path (__shfl*) costs an LDS round trip per step.
template <int CTRL, int ROWMASK = 0xF>
__device__ __forceinline__ uint32_t dpp32(uint32_t v) {        // lanes without a source read 0
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWMASK, 0xF, false);
}
template <int CTRL, class T>
__device__ __forceinline__ T dpp_move(T v) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit lanes");
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, dpp32<CTRL>(__builtin_bit_cast(uint32_t, v)));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint64_t lo = dpp32<CTRL>((uint32_t)u), hi = dpp32<CTRL>((uint32_t)(u >> 32));
        return __builtin_bit_cast(T, (hi << 32) | lo);
    }
}
template <class T>
__device__ __forceinline__ T read_lane(T v, int lane) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
        const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
        return __builtin_bit_cast(T, (hi << 32) | lo);
    }
}
// op over the wave, result uniform: butterflies within each row of 16 lanes (quad swaps, half-row and row
// mirrors), then the four rows' lane 0
template <class T, class Op>
__device__ __forceinline__ T wave_allreduce(T v, Op op) {
    v = op(v, dpp_move<0xB1>(v));     // quad_perm [1,0,3,2]
    v = op(v, dpp_move<0x4E>(v));     // quad_perm [2,3,0,1]
    v = op(v, dpp_move<0x141>(v));    // row_half_mirror
    v = op(v, dpp_move<0x140>(v));    // row_mirror
    return op(op(read_lane(v, 0), read_lane(v, 16)), op(read_lane(v, 32), read_lane(v, 48)));
}
template <class T>
__device__ __forceinline__ T wave_max(T v) {
    return wave_allreduce(v, [](T x, T y) { return y > x ? y : x; });
}
template <class T>
__device__ __forceinline__ T wave_min(T v) {
    return wave_allreduce(v, [](T x, T y) { return y < x ? y : x; });
}
// The verification rule (server.cpp:627-637) over a stream's m >= 1 tokens, read by the whole wave at once (agent
// scope: the stream's rows ran on several XCDs): 1 + the leading rows whose token equals the next row's draft, the
// walk ending after an eos token. Uniform over the wave.
__device__ __forceinline__ int accepted_prefix(const int32_t* tok, const int32_t* rows, int64_t r0, int m, int eos) {
    for (int c0 = 0; c0 < m; c0 += WAVE) {
        const int r = c0 + lane_id();
        bool stop = false;
        if (r < m) {
            const int t = ld_agent(&tok[r0 + r]);
            stop = (eos >= 0 && t == eos) || r + 1 >= m || t != rows[r0 + r + 1];
        }
        const uint64_t b = __ballot(stop);
        if (b) return c0 + __ffsll((unsigned long long)b);    // 1-based: the row that ends the walk, plus one
    }
    return m;
}
// inclusive sum over lanes 0..lane (32-bit integers): row shifts 1, 2, 4, 8, then row broadcasts 15 and 31
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t x) {
    x += dpp32<0x111>(x);
    x += dpp32<0x112>(x);
    x += dpp32<0x114>(x);
    x += dpp32<0x118>(x);
    x += dpp32<0x142, 0xA>(x);
    x += dpp32<0x143, 0xC>(x);
    return x;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Small shared scratch for block-wide reductions and broadcasts.
struct Red {
    uint64_t u64[NWAVES];
    uint64_t u64b[NWAVES];
    double f64[NWAVES];
    int i32[NWAVES];
    uint32_t u32[NWAVES];
    uint32_t misc[8];
    double dmisc[4];
};

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, Red& r) {
    v = wave_max(v);
    if (lane_id() == 0) r.u64[threadIdx.x / WAVE] = v;
    __syncthreads();
    uint64_t m = r.u64[0];
#pragma unroll
    for (int w = 1; w < NWAVES; ++w) m = r.u64[w] > m ? r.u64[w] : m;
    __syncthreads();
    return m;
}
__device__ __forceinline__ uint64_t block_min_u64(uint64_t v, Red& r) {
    v = wave_min(v);
    if (lane_id() == 0) r.u64[threadIdx.x / WAVE] = v;
    __syncthreads();
    uint64_t m = r.u64[0];
#pragma unroll
    for (int w = 1; w < NWAVES; ++w) m = r.u64[w] < m ? r.u64[w] : m;
    __syncthreads();
    return m;
}
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, Red& r) {
    v = wave_max(v);
    if (lane_id() == 0) r.u32[threadIdx.x / WAVE] = v;
    __syncthreads();
    uint32_t m = r.u32[0];
#pragma unroll
    for (int w = 1; w < NWAVES; ++w) m = r.u32[w] > m ? r.u32[w] : m;
    __syncthreads();
    return m;
}
// max and min in one round
__device__ __forceinline__ void block_minmax_u32(uint32_t& mn, uint32_t& mx, Red& r) {
    uint32_t a = wave_max(mx), b = wave_min(mn);
    if (lane_id() == 0) { r.u32[threadIdx.x / WAVE] = a; r.i32[threadIdx.x / WAVE] = (int)b; }
    __syncthreads();
    a = r.u32[0];
    b = (uint32_t)r.i32[0];
#pragma unroll
    for (int w = 1; w < NWAVES; ++w) {
        a = r.u32[w] > a ? r.u32[w] : a;
        b = (uint32_t)r.i32[w] < b ? (uint32_t)r.i32[w] : b;
    }
    __syncthreads();
    mx = a;
    mn = b;
}
__device__ __forceinline__ int block_min_i32(int v, Red& r) {
    v = wave_min(v);
    if (lane_id() == 0) r.i32[threadIdx.x / WAVE] = v;
    __syncthreads();
    int m = r.i32[0];
#pragma unroll
    for (int w = 1; w < NWAVES; ++w) m = r.i32[w] < m ? r.i32[w] : m;
    __syncthreads();
    return m;
}
__device__ __forceinline__ int block_max_i32(int v, Red& r) {
    v = wave_max(v);
    if (lane_id() == 0) r.i32[threadIdx.x / WAVE] = v;
    __syncthreads();
    int m = r.i32[0];
#pragma unroll
    for (int w = 1; w < NWAVES; ++w) m = r.i32[w] > m ? r.i32[w] : m;
    __syncthreads();
    return m;
}
// Deterministic double sum: fixed butterfly in each wave, waves added in order.
__device__ __forceinline__ double block_sum_f64(double v, Red& r) {
    v = wave_sum_f64(v);
    if (lane_id() == 0) r.f64[threadIdx.x / WAVE] = v;
    __syncthreads();
    double s = r.f64[0];
#pragma unroll
    for (int w = 1; w < NWAVES; ++w) s += r.f64[w];
    __syncthreads();
    return s;
}
// DPP moves of a double (two 32-bit halves); lanes without a source read 0 (bound_ctrl off, old = 0).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROWMASK, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROWMASK, 0xF, false);
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint64_t)(uint32_t)lo));
}
// Inclusive wave scan: row_shr 1, 2, 4, 8 inside each 16-lane row, then row_bcast 15 / 31 across rows.
__device__ __forceinline__ double wave_scan_f64(double v) {
    v += dpp_f64<0x111, 0xF>(v);
    v += dpp_f64<0x112, 0xF>(v);
    v += dpp_f64<0x114, 0xF>(v);
    v += dpp_f64<0x118, 0xF>(v);
    v += dpp_f64<0x142, 0xA>(v);
    v += dpp_f64<0x143, 0xC>(v);
    return v;
}
// Exclusive prefix over threads (thread order), deterministic; *total = the sum over the block.
template <class T>
__device__ __forceinline__ T block_excl_scan(T v, T* wsum /*NWAVES*/, T* total) {
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    T x, ex;
    if constexpr (sizeof(T) == 4 && T(-1) > T(0)) {            // 32-bit unsigned: DPP scan (exact in any order)
        x = wave_incl_scan_u32(v);
        ex = x - v;
    } else if constexpr (sizeof(T) == 8 && T(0.5) > T(0)) {    // double: DPP scan, then wave_shr:1 (lane 0 reads 0)
        x = wave_scan_f64(v);
        ex = dpp_f64<0x138, 0xF>(x);
    } else {                                                   // the fixed shuffle order of the sums
        x = v;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
            const T y = __shfl_up(x, o);
            if (lane >= o) x += y;
        }
        ex = __shfl_up(x, 1);
        if (lane == 0) ex = T(0);
    }
    if (lane == WAVE - 1) wsum[w] = x;
    __syncthreads();
    T off = T(0), tot = T(0);
#pragma unroll
    for (int q = 0; q < NWAVES; ++q) {
        if (q < w) off += wsum[q];
        tot += wsum[q];
    }
    __syncthreads();
    *total = tot;
    return off + ex;
}

// Append `pred` lanes' values to an LDS list (one LDS atomic per wave); entries past cap are counted, not stored.
__device__ __forceinline__ void wave_append(bool pred, uint64_t v, uint64_t* list, uint32_t* count, uint32_t cap) {
    const uint64_t m = __ballot(pred);
    if (m == 0) return;
    uint32_t base = 0;
    const int leader = __ffsll((unsigned long long)m) - 1;
    if (lane_id() == leader) base = atomicAdd(count, (uint32_t)__popcll(m));
    base = (uint32_t)__builtin_amdgcn_readlane((int)base, leader);   // a scalar read, no LDS round trip
    if (pred) {
        const uint32_t pos = base + mbcnt(m);
        if (pos < cap) list[pos] = v;
    }
}

// wave_append for a register element: the 64-bit composite is formed only when some lane of the wave appends.
__device__ __forceinline__ void wave_append_kv(bool pred, uint32_t key, uint32_t id, uint64_t* list, uint32_t* count,
                                               uint32_t cap) {
    const uint64_t m = __ballot(pred);
    if (m == 0) return;
    uint32_t base = 0;
    const int leader = __ffsll((unsigned long long)m) - 1;
    if (lane_id() == leader) base = atomicAdd(count, (uint32_t)__popcll(m));
    base = (uint32_t)__builtin_amdgcn_readlane((int)base, leader);   // a scalar read, no LDS round trip
    if (pred) {
        const uint32_t pos = base + mbcnt(m);
        if (pos < cap) list[pos] = comp_of(key, id);
    }
}

// Histogram helpers over keys in [base, base + (NBINS << shift)): bin = (key - base) >> shift.
__device__ __forceinline__ int range_shift(uint32_t lo, uint32_t hi) {
    const uint32_t span = hi - lo;                       // keys lo..hi map to bins 0..span>>shift < NBINS
    int s = 0;
    while ((span >> s) >= (uint32_t)NBINS) ++s;
    return s;
}
// From a filled histogram, the bin b holding the kk-th largest entry: count(bins > b) < kk <= count(bins >= b).
// *above = count(bins > b), *atb = count(bins >= b). Requires 1 <= kk <= total.
__device__ __forceinline__ int hist_locate(const uint32_t* bins, int kk, uint32_t* above_out, uint32_t* atb_out, uint32_t* wsum,
                           Red& r) {
    constexpr int BPT = NBINS / BLOCK;
    const int tid = threadIdx.x;
    uint32_t mine = 0;
#pragma unroll
    for (int i = 0; i < BPT; ++i) mine += bins[NBINS - 1 - (tid * BPT + i)];
    uint32_t tot;
    const uint32_t above = block_excl_scan<uint32_t>(mine, wsum, &tot);
    if (above < (uint32_t)kk && above + mine >= (uint32_t)kk) {
        uint32_t c = above;
        for (int i = 0; i < BPT; ++i) {
            const int bin = NBINS - 1 - (tid * BPT + i);
            const uint32_t nb = bins[bin];
            if (c + nb >= (uint32_t)kk) { r.misc[4] = (uint32_t)bin; r.misc[5] = c; r.misc[6] = c + nb; break; }
            c += nb;
        }
    }
    __syncthreads();
    const int b = (int)r.misc[4];
    *above_out = r.misc[5];
    *atb_out = r.misc[6];
    __syncthreads();
    return b;
}

// From a filled histogram: the largest bin b such that count(bins >= b) >= k. Returns T = base + (b << shift) and
// *cnt = count(bins >= b); T = 0 and *cnt = total when the histogram holds fewer than k entries.
__device__ __forceinline__ uint32_t hist_threshold(const uint32_t* bins, uint32_t base, int shift, int k, uint32_t* cnt,
                                   uint32_t* wsum, Red& r) {
    constexpr int BPT = NBINS / BLOCK;
    const int tid = threadIdx.x;
    uint32_t mine = 0;
#pragma unroll
    for (int i = 0; i < BPT; ++i) mine += bins[NBINS - 1 - (tid * BPT + i)];
    uint32_t tot;
    const uint32_t above = block_excl_scan<uint32_t>(mine, wsum, &tot);
    if (tid == 0) { r.misc[4] = 0u; r.misc[5] = tot; }
    __syncthreads();
    if (tot >= (uint32_t)k && above < (uint32_t)k && above + mine >= (uint32_t)k) {
        uint32_t c = above;
        for (int i = 0; i < BPT; ++i) {
            const int bin = NBINS - 1 - (tid * BPT + i);
            c += bins[bin];
            if (c >= (uint32_t)k) { r.misc[4] = base + ((uint32_t)bin << shift); r.misc[5] = c; break; }
        }
    }
    __syncthreads();
    *cnt = r.misc[5];
    const uint32_t T = r.misc[4];
    __syncthreads();
    return T;
}

// Exact k-th largest composite among the candidates a visitor yields (all distinct, 0 = absent; 1 <= k <= count).
// Radix select from the top byte: 8 passes of a 256-bin LDS histogram. each(f) calls f(c) for every candidate the
// calling thread holds. With last_shift = 32 it stops after the key bytes: the result is the k-th largest key (low
// word 0), which at least k candidates reach.
template <class Each>
__device__ __forceinline__ uint64_t radix_kth(Each each, int k, uint32_t* hist256, uint32_t* wsum, Red& r,
                                              int last_shift = 0) {
    uint64_t prefix = 0, mask = 0;
    int kk = k;
    const int tid = threadIdx.x;
    for (int shift = 56; shift >= last_shift; shift -= 8) {
        if (tid < 256) hist256[tid] = 0;
        __syncthreads();
        each([&](uint64_t c) {
            if (c != 0 && (c & mask) == prefix) atomicAdd(&hist256[(c >> shift) & 255], 1u);
        });
        __syncthreads();
        const uint32_t cnt = tid < 256 ? hist256[255 - tid] : 0u;   // thread t owns bin 255 - t: scan from the top
        uint32_t tot;
        const uint32_t above = block_excl_scan<uint32_t>(cnt, wsum, &tot);
        if (tid < 256 && above < (uint32_t)kk && above + cnt >= (uint32_t)kk) {
            r.misc[0] = 255 - tid;
            r.misc[1] = above;
        }
        __syncthreads();
        const uint64_t d = r.misc[0];
        kk -= (int)r.misc[1];
        prefix |= d << shift;
        mask |= (uint64_t)255 << shift;
        __syncthreads();
    }
    return prefix;
}

// Descending bitonic sort of n (a power of two, n <= 4 * BLOCK) composites in LDS, whole block. The stages of the
// network are taken two at a time: for a pair of strides 2^p1, 2^p2 thread t loads the four entries whose indices
// are t with zero bits inserted at p1 and p2, plus 0/1 in those bits, applies both stages in registers and stores
// them back. While both bits are below 8 the four entries lie in the 256-entry block of the thread's wave
// (index bits 8.. = wave id), and a wave's LDS accesses complete in order, so such rounds need no barrier; a
// barrier is placed only on each side of a round that crosses blocks.
__device__ __forceinline__ void bitonic_desc(uint64_t* a, int n) {
    static_assert(4 * BLOCK >= KMAX && 4 * WAVE == 256, "four entries per thread; a wave spans 256 entries");
    const int tid = threadIdx.x;
    if (n < 4) {
        if (n == 2 && tid == 0) {
            const uint64_t x = a[0], y = a[1];
            if (x < y) { a[0] = y; a[1] = x; }
        }
        __syncthreads();
        return;
    }
    int lg = 0;
    while ((1 << lg) < n) ++lg;
    const bool act = tid < (n >> 2);
    int m = 1, p = 0;                               // next stage: merge size 2^m, stride 2^p
    bool prev_cross = false;
    while (m <= lg) {
        // this round: the stage (m, p), the next one, and a third while its stride is one of the two
        int sm[3], sp[3], ns = 0;
        int b0 = p, b1 = -1;
        while (m <= lg && ns < 3) {
            if (p != b0 && p != b1) {
                if (b1 >= 0) break;
                b1 = p;
            }
            sm[ns] = m; sp[ns] = p; ++ns;
            if (p == 0) { ++m; p = m - 1; } else { --p; }
        }
        if (b1 < 0) b1 = b0 == 0 ? 1 : 0;           // a lone last stage: any second bit
        const int hi = b0 > b1 ? b0 : b1, lo = b0 > b1 ? b1 : b0;
        const bool cross = hi >= 8;
        if (cross || prev_cross) __syncthreads();
        prev_cross = cross;
        if (act) {
            const int t = tid;
            const int base = (t & ((1 << lo) - 1)) | (((t >> lo) & ((1 << (hi - lo - 1)) - 1)) << (lo + 1)) |
                             ((t >> (hi - 1)) << (hi + 1));
            const int ix[4] = {base, base + (1 << lo), base + (1 << hi), base + (1 << hi) + (1 << lo)};
            uint64_t e[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) e[j] = a[ix[j]];
            auto cx = [](uint64_t& x, uint64_t& y, bool desc) {
                const uint64_t lo_v = x < y ? x : y, hi_v = x < y ? y : x;
                x = desc ? hi_v : lo_v;
                y = desc ? lo_v : hi_v;
            };
#pragma unroll
            for (int q = 0; q < 3; ++q) {
                if (q >= ns) break;
                const int sh = sm[q];
                if (sp[q] == hi) {                      // partners two registers apart
                    cx(e[0], e[2], ((ix[0] >> sh) & 1) == 0);
                    cx(e[1], e[3], ((ix[1] >> sh) & 1) == 0);
                } else {
                    cx(e[0], e[1], ((ix[0] >> sh) & 1) == 0);
                    cx(e[2], e[3], ((ix[2] >> sh) & 1) == 0);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) a[ix[j]] = e[j];
        }
    }
    __syncthreads();
}

// Rank sort of n <= SMALL distinct composites: out[rank] = in[i] for ranks < k.
__device__ __forceinline__ void rank_sort(const uint64_t* in, int n, uint64_t* out, int k) {
    for (int i = threadIdx.x; i < n; i += BLOCK) {
        const uint64_t c = in[i];
        int rank = 0;
        for (int m = 0; m < n; ++m) rank += in[m] > c ? 1 : 0;
        if (rank < k) out[rank] = c;
    }
    __syncthreads();
}

__device__ __forceinline__ int64_t window_begin(int64_t len, const fs_row_params& p) {
    int64_t b = (p.repeat_last_n > 0 && (int64_t)p.repeat_last_n < len) ? len - (int64_t)p.repeat_last_n : 0;
    if (p.penalty_from > 0 && (int64_t)p.penalty_from > b) b = p.penalty_from;
    return b;
}

// ------------------------------------------------------------------------------------------------ kernel
struct Shared {
    uint64_t cand[CAP];                // candidate buffer / merge gather
    uint32_t scr[TILE / 2 + NBINS];    // per-tile 16-bit penalty counts, then histograms; or a 64-bit stage
    uint32_t off[MAX_SEGS + 1];        // merge: flat offsets of the segment lists
    int32_t ids[WIDS];                 // the penalty window's ids that fall in the current segment
    uint32_t wsum[NWAVES];
    uint32_t count;
    uint32_t tmax;                     // segment kernel: the largest key of tile 0
    uint32_t rc64[WAVE];               // segment kernel: tile-0 counts in the 64 coarse bins up to tmax's
    uint32_t nids;
    uint32_t nfast;                    // large-row segment: the cut's survivors written to the slot
    uint32_t wcnt[NWAVES];             // large-row segment: each wave's part of the cut's LDS list
    uint32_t tmx[2][NWAVES];           // large-row segment: the waves' tile maxima (keys), alternating tiles
    uint32_t misc_alone;               // merge role: the row is computed from its logits alone
#ifdef FS_TRACE
    uint64_t trace_t[16];              // this workgroup's phase timestamps (written to a.trace at its end)
#endif
    Red red;
    __device__ __forceinline__ uint32_t* cnt() { return scr; }
    __device__ __forceinline__ uint32_t* bins() { return scr + TILE / 2; }
    __device__ __forceinline__ uint64_t* stage() { return reinterpret_cast<uint64_t*>(scr); }   // KMAX entries
};

// Descending sort of m <= KMAX distinct composites a[0, m), in place (whole block; returns after a barrier). A
// counting sort: NB bins span [min, max] of the composites (bin 0 = the largest); each entry takes a slot in its
// bin with an LDS atomic (cnt) and is scattered to tmp[bin start + slot]; then each entry counts the larger entries
// of its own bin and lands at bin start + that count. Bins of a smooth tail hold a few entries each (equal keys
// spread over the id bits); when one holds more than BIN_SORT_MAX the bitonic network sorts instead (a must then
// hold the next power of two >= m entries). cnt and start hold NB counters each; tmp holds m entries.
constexpr int BIN_SORT_MAX = 48;
template <int NB>
__device__ __forceinline__ uint32_t bin_sort_desc(uint64_t* a, int m, uint64_t* tmp, uint32_t* cnt, uint32_t* start,
                                                  Red& red, uint32_t* wsum) {
    constexpr int EPT = KMAX / BLOCK;            // entries per thread
    constexpr int BPT = NB / BLOCK;              // bins per thread
    static_assert(BPT >= 1 && NB == BPT * BLOCK, "whole bins per thread");
    const int tid = threadIdx.x;
    uint64_t v[EPT];
    uint64_t cmn = ~0ull, cmx = 0ull;
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
        const int i = q * BLOCK + tid;
        v[q] = i < m ? a[i] : 0ull;
        if (i < m) {
            cmn = v[q] < cmn ? v[q] : cmn;
            cmx = v[q] > cmx ? v[q] : cmx;
        }
    }
#pragma unroll
    for (int q = 0; q < BPT; ++q) cnt[q * BLOCK + tid] = 0u;
    cmn = block_min_u64(cmn, red);               // its barriers also order the zeroed counts
    cmx = block_max_u64(cmx, red);
    if (m <= 1) return 0u;
    int sh = 0;                                  // composites cmn..cmx map to bins NB-1..0
    while (((cmx - cmn) >> sh) >= (uint64_t)NB) ++sh;
    uint32_t bin[EPT], slot[EPT];
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
        bin[q] = 0u;
        slot[q] = 0u;
        if (q * BLOCK + tid < m) {
            bin[q] = (uint32_t)(NB - 1) - (uint32_t)((v[q] - cmn) >> sh);
            slot[q] = atomicAdd(&cnt[bin[q]], 1u);
        }
    }
    __syncthreads();
    uint32_t c[BPT], sum = 0u, big = 0u;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
        c[j] = cnt[BPT * tid + j];
        sum += c[j];
        big = c[j] > big ? c[j] : big;
    }
    uint32_t tot;
    uint32_t off = block_excl_scan<uint32_t>(sum, wsum, &tot);
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
        start[BPT * tid + j] = off;
        off += c[j];
    }
    big = block_max_u32(big, red);               // its barriers also publish the starts
    if (big > (uint32_t)BIN_SORT_MAX) {
        int np = 1;
        while (np < m) np <<= 1;
        for (int i = m + tid; i < np; i += BLOCK) a[i] = 0ull;
        __syncthreads();
        bitonic_desc(a, np);
        return big;
    }
#pragma unroll
    for (int q = 0; q < EPT; ++q)
        if (q * BLOCK + tid < m) tmp[start[bin[q]] + slot[q]] = v[q];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
        if (q * BLOCK + tid < m) {
            const uint32_t b0 = start[bin[q]], n = cnt[bin[q]];
            uint32_t r = 0u, j = 0u;
            for (; j + 4u <= n; j += 4u) {              // four LDS reads in flight per step
                const uint64_t t0 = tmp[b0 + j], t1 = tmp[b0 + j + 1], t2 = tmp[b0 + j + 2], t3 = tmp[b0 + j + 3];
                r += (t0 > v[q] ? 1u : 0u) + (t1 > v[q] ? 1u : 0u) + (t2 > v[q] ? 1u : 0u) + (t3 > v[q] ? 1u : 0u);
            }
            for (; j < n; ++j) r += tmp[b0 + j] > v[q] ? 1u : 0u;
            a[b0 + r] = v[q];
        }
    }
    __syncthreads();
    return big;                                  // the largest bin (> BIN_SORT_MAX: the bitonic network sorted)
}
// The candidate buffer's first m <= KMAX entries, with the second KMAX entries as the scatter area.
__device__ __forceinline__ uint32_t bin_sort_desc(int m, Shared& s) {
    static_assert(TILE / 2 >= NBINS && 2 * KMAX <= CAP, "counts in cnt(), starts in bins(), scatter after the input");
    return bin_sort_desc<NBINS>(s.cand, m, s.cand + KMAX, s.cnt(), s.bins(), s.red, s.wsum);
}
static_assert((TILE / 2 + NBINS) / 2 >= KMAX, "the stage holds a compacted top k");

// Per-row view of the arguments: params, greedy/k, and the two history segments (a verify row sees its stream's
// base history followed by the drafts fed before it).
struct RowCtx {
    int row, pidx;
    fs_row_params p;
    bool greedy, large, pen, rep_on, fp_on, capped;
    int k;
    int64_t hA0, lenA, lenB, b, len;     // window [b, len) over the concatenated history
    const int32_t* segB;
    // the row's segments: nseg of st tiles each (the last may be shorter); segment s publishes in list slot
    // lx + XCDS * (lbase + s) (the index of the segment workgroup that streams it)
    int nseg, st, lbase, lx;
};
__device__ __forceinline__ int64_t slot_of(const RowCtx& rc, int seg) {
    return (int64_t)rc.lx + (int64_t)XCDS * (int64_t)(rc.lbase + seg);
}

// Inputs that no kernel writes (params, history offsets, verify row offsets) are read through the constant address
// space, so uniform indices become scalar loads (lgkmcnt) and never wait behind the vector loads in flight.
template <class T>
__device__ __forceinline__ T ld_const(const T* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *(const __attribute__((address_space(4))) T*)(p);
#else
    return *p;                                  // the host pass never runs device code
#endif
}

__device__ __forceinline__ RowCtx row_ctx(const Args& a, int row) {
    RowCtx rc;
    rc.row = row;
    rc.pidx = row;
    rc.nseg = a.nseg;
    rc.st = a.seg_tiles;
    rc.lx = row % XCDS;
    rc.lbase = (row / XCDS) * a.nseg;
    rc.hA0 = 0; rc.lenA = 0; rc.lenB = 0;
    rc.segB = nullptr;
    if (a.mode == MODE_VERIFY) {
        int s0 = 0, s1 = a.n_streams;           // largest s with row_off[s] <= row
        while (s1 - s0 > 1) {
            const int m = (s0 + s1) >> 1;
            if (ld_const(a.row_off + m) <= row) s0 = m; else s1 = m;
        }
        rc.pidx = s0;
        const int64_t r0 = ld_const(a.row_off + s0);
        rc.segB = a.rows + r0 + 1;
        rc.lenB = row - r0;
    }
    if (a.hist_off && a.hist) {
        rc.hA0 = ld_const(a.hist_off + rc.pidx);
        rc.lenA = ld_const(a.hist_off + rc.pidx + 1) - rc.hA0;
    }
    if (a.params) {                           // dword by dword: scalar loads (a struct copy becomes vector loads)
        static_assert(sizeof(fs_row_params) % 4 == 0, "fs_row_params is a sequence of dwords");
        uint32_t w[sizeof(fs_row_params) / 4];
        const uint32_t* src = reinterpret_cast<const uint32_t*>(a.params + rc.pidx);
#pragma unroll
        for (int i = 0; i < (int)(sizeof(fs_row_params) / 4); ++i) w[i] = ld_const(src + i);
        __builtin_memcpy(&rc.p, w, sizeof(fs_row_params));
    } else {
        rc.p.temperature = 0.f; rc.p.top_k = 1; rc.p.top_p = 1.f; rc.p.min_p = 0.f; rc.p.repetition_penalty = 1.f;
        rc.p.frequency_penalty = 0.f; rc.p.presence_penalty = 0.f; rc.p.repeat_last_n = 0; rc.p.penalty_from = 0;
        rc.p.softcap = 0.f;
    }
    const int V = a.V;
    rc.greedy = a.mode == MODE_ARGMAX || rc.p.temperature <= 0.0f || rc.p.top_k == 1;
    rc.k = rc.greedy ? 1 : ((rc.p.top_k > 0 && rc.p.top_k < V) ? rc.p.top_k : V);
    rc.large = rc.k > KMAX;                 // not on the segment path: sampled by large_row in the merge kernel
    rc.capped = rc.p.softcap > 0.0f;
    rc.rep_on = rc.p.repetition_penalty != 1.0f;
    rc.fp_on = rc.p.frequency_penalty != 0.0f || rc.p.presence_penalty != 0.0f;
    rc.len = rc.lenA + rc.lenB;
    rc.pen = (rc.rep_on || rc.fp_on) && rc.p.repeat_last_n != 0 && rc.len > 0;
    rc.b = rc.pen ? window_begin(rc.len, rc.p) : rc.len;
    if (rc.b >= rc.len) rc.pen = false;
    return rc;
}

__device__ __forceinline__ int hist_at(const Args& a, const RowCtx& rc, int64_t i) {
    return i < rc.lenA ? a.hist[rc.hA0 + i] : rc.segB[i - rc.lenA];
}

// Issue the loads of one tile (TPT logits per thread: float4 j at element lo + (j*BLOCK + t)*4) without waiting.
// Lanes past the row's end read a clamped in-bounds address and are zeroed. The float4 holding element V-1 may
// extend up to 12 bytes past it, inside the same 16-byte-aligned block (never into another page); masked too.
// The segment kernel only streams full tiles (a row's partial last tile is handled by the merge kernel).
__device__ __forceinline__ void load_tile(float (&x)[TPT], const float* rowp, int lo) {
    const float4* p = reinterpret_cast<const float4*>(rowp + lo) + threadIdx.x;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const float4 t = p[j * BLOCK];
        x[4 * j + 0] = t.x; x[4 * j + 1] = t.y; x[4 * j + 2] = t.z; x[4 * j + 3] = t.w;
    }
}
// Tile t of a segment through its buffer resource: a tile past the segment's end reads zeros without a memory
// access, so the tile loop requests its next tiles unconditionally (straight-line loads keep the compiler's
// memory-counter waits exact: consuming a tile waits for that tile only).
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ f32x4 raw_buffer_load_f32x4(__amdgpu_buffer_rsrc_t rs, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.load.v4f32");
template <int AUX = 0>
__device__ __forceinline__ void load_seg_tile(float (&x)[TPT], __amdgpu_buffer_rsrc_t rs, int t) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const f32x4 v = raw_buffer_load_f32x4(rs, (j * BLOCK + (int)threadIdx.x) * 16, t * TILE * 4, AUX);
        x[4 * j + 0] = v.x; x[4 * j + 1] = v.y; x[4 * j + 2] = v.z; x[4 * j + 3] = v.w;
    }
}
// tanhf as the host C library computes it where ferro runs (glibc's float tanh, which follows Sun's fdlibm
// s_tanh.c / s_expm1.c in single precision): tanh(x) = -e/(e+2) with e = expm1(-2|x|) for |x| < 1,
// 1 - 2/(expm1(2|x|)+2) for 1 <= |x| < 22, +-1 beyond; expm1 reduces x = k ln2 + r (ln2 split into a 24-bit-exact
// hi part and a lo part), approximates expm1(r) by fdlibm's rational scheme (the degree-5 polynomial in r^2/2 with
// fdlibm's Q1..Q5 rounded to float) and rescales by 2^k. Every operation is a separately rounded IEEE fp32 add,
// multiply or divide (no contraction), so the result is bit-identical to the host's: the GPU test checks all 2^32
// inputs against the C library.
__device__ __forceinline__ float f_of(uint32_t u) { return __uint_as_float(u); }
// Straight-line form (every case computed, the result selected): no branches, so the eight-wide unrolled reads
// that call it stay one basic block each. Selecting between separately computed IEEE results changes none of them.
__device__ __forceinline__ float host_tanhf(float x) {
    const float ln2_hi = f_of(0x3f317180u), ln2_lo = f_of(0x3717f7d1u), invln2 = f_of(0x3fb8aa3bu);
    const float Q1 = f_of(0xbd088889u), Q2 = f_of(0x3ad00d01u), Q3 = f_of(0xb8a670cdu), Q4 = f_of(0x36867e54u),
                Q5 = f_of(0xb457edbbu);
    const uint32_t jx = __float_as_uint(x), ix = jx & 0x7fffffffu;
    const bool neg = (jx >> 31) != 0u;
    const float ax = __uint_as_float(ix);
    const bool big = ix >= 0x3f800000u;                     // |x| >= 1: tanh = 1 - 2/(expm1(2|x|)+2)
    const float y = big ? __fmul_rn(2.0f, ax) : __fmul_rn(-2.0f, ax);   // expm1's argument, in (-2, 44) for |x| < 22
    const uint32_t hy = __float_as_uint(y) & 0x7fffffffu;
    const bool yneg = !big;
    // expm1(y): y = k ln2 + r (|y| > ln2 / 2; k = +-1 below 1.5 ln2)
    const bool red = hy > 0x3eb17218u;
    const bool near = hy < 0x3F851592u;
    const float hiA = yneg ? __fadd_rn(y, ln2_hi) : __fsub_rn(y, ln2_hi);
    const float loA = yneg ? -ln2_lo : ln2_lo;
    const int kB = (int)__fadd_rn(__fmul_rn(invln2, y), yneg ? -0.5f : 0.5f);   // truncation toward zero
    const float tB = (float)kB;
    const float hiB = __fsub_rn(y, __fmul_rn(tB, ln2_hi));   // tB * ln2_hi is exact
    const float loB = __fmul_rn(tB, ln2_lo);
    const int k = red ? (near ? (yneg ? -1 : 1) : kB) : 0;
    const float hi = near ? hiA : hiB, lo = near ? loA : loB;
    const float xr = red ? __fsub_rn(hi, lo) : y;
    const float c = red ? __fsub_rn(__fsub_rn(hi, xr), lo) : 0.0f;
    const float hfx = __fmul_rn(0.5f, xr);
    const float hxs = __fmul_rn(xr, hfx);
    const float r1 = __fadd_rn(1.0f, __fmul_rn(hxs, __fadd_rn(Q1, __fmul_rn(hxs, __fadd_rn(Q2, __fmul_rn(hxs,
                     __fadd_rn(Q3, __fmul_rn(hxs, __fadd_rn(Q4, __fmul_rn(hxs, Q5))))))))));
    const float t = __fsub_rn(3.0f, __fmul_rn(r1, hfx));
    const float e = __fmul_rn(hxs, __fdiv_rn(__fsub_rn(r1, t), __fsub_rn(6.0f, __fmul_rn(xr, t))));
    const float R0 = __fsub_rn(xr, __fsub_rn(__fmul_rn(xr, e), hxs));                       // k = 0
    const float e2 = __fsub_rn(__fsub_rn(__fmul_rn(xr, __fsub_rn(e, c)), c), hxs);
    const float Rm1 = __fsub_rn(__fmul_rn(0.5f, __fsub_rn(xr, e2)), 0.5f);                 // k = -1
    const float R1 = xr < -0.25f ? __fmul_rn(-2.0f, __fsub_rn(e2, __fadd_rn(xr, 0.5f)))    // k = 1
                                 : __fadd_rn(1.0f, __fmul_rn(2.0f, __fsub_rn(xr, e2)));
    const int kc = k < -126 ? -126 : (k > 127 ? 127 : k);
    const float twopk = f_of(0x3f800000u + ((uint32_t)kc << 23));
    const float RL = __fsub_rn(__fmul_rn(__fsub_rn(1.0f, __fsub_rn(e2, xr)), twopk), 1.0f);  // k <= -2 or k > 56
    const int ks = k < 0 ? 0 : (k > 31 ? 31 : k);
    const float RS = __fmul_rn(__fsub_rn(f_of(0x3f800000u - (0x1000000u >> ks)), __fsub_rn(e2, xr)), twopk);   // 1 - 2^-k
    const int kt = k < 0 ? 0 : (k > 126 ? 126 : k);
    const float RB = __fmul_rn(__fadd_rn(__fsub_rn(xr, __fadd_rn(e2, f_of((uint32_t)(0x7f - kt) << 23))), 1.0f), twopk);
    float em = k == 0 ? R0 : k == -1 ? Rm1 : k == 1 ? R1 : (k <= -2 || k > 56) ? RL : k < 23 ? RS : RB;
    const float huge = 1.0e+30f;
    if (hy < 0x33000000u) em = __fsub_rn(y, __fsub_rn(__fadd_rn(huge, y), __fadd_rn(huge, y)));   // |y| < 2^-25
    // tanh from expm1
    float z = big ? __fsub_rn(1.0f, __fdiv_rn(2.0f, __fadd_rn(em, 2.0f))) : __fdiv_rn(-em, __fadd_rn(em, 2.0f));
    if (ix >= 0x41b00000u) z = __fsub_rn(1.0f, 1.0e-30f);      // |x| >= 22: +-1 (inexact)
    float r = neg ? -z : z;
    if (ix < 0x24000000u) r = __fmul_rn(x, __fadd_rn(1.0f, x));  // |x| < 2^-55
    if (ix >= 0x7f800000u)                                       // +-inf, NaN
        r = neg ? __fsub_rn(__fdiv_rn(1.0f, x), 1.0f) : __fadd_rn(__fdiv_rn(1.0f, x), 1.0f);
    return r;
}
// The model's final-logit softcap, moved into the read: l = cap * tanhf(l / cap) (model_gemma4_gpu.cpp:282-283:
// fp32 divide, the host C library's tanhf, fp32 multiply), before the penalties as in ferro, where the model caps
// the row first. Bit-identical to the host loop.
__device__ __forceinline__ float softcap_one(float l, float cap) { return __fmul_rn(cap, host_tanhf(__fdiv_rn(l, cap))); }
// Unrolled, for the streaming loop of the segment path (its three call sites): a rolled loop there changes the
// allocation of the tile registers and slows every row, capped or not.
template <int N>
__device__ __forceinline__ void softcap_vals_unrolled(float (&x)[N], float cap) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = softcap_one(x[i], cap);
}
// A rolled loop: one copy of the cap per call site (there are dozens, all unrolled eight-wide otherwise), for capped
// rows only; the element is picked and put back by index.
template <int N>
__device__ __forceinline__ void softcap_vals(float (&x)[N], float cap) {
#pragma unroll 1
    for (int i = 0; i < N; ++i) {
        float v = x[0];
#pragma unroll
        for (int j = 1; j < N; ++j) v = i == j ? x[j] : v;
        v = softcap_one(v, cap);
#pragma unroll
        for (int j = 0; j < N; ++j) x[j] = i == j ? v : x[j];
    }
}
// element id of this thread's i-th logit of the tile starting at lo
__device__ __forceinline__ int elem_id(int lo, int i) { return lo + ((i >> 2) * BLOCK + (int)threadIdx.x) * 4 + (i & 3); }

// Penalty pass on one tile in registers (sampler.cpp:11-18; frequency/presence extension): the window's ids that
// fall in [lo, lo + TILE) are counted in a 16-bit LDS table, then each thread patches its counted logits.
// Entry: the table may still be read by the previous tile's patching, so the caller has passed a barrier.
__device__ __forceinline__ void apply_penalties(float (&x)[TPT], const Args& a, const RowCtx& rc, int lo, Shared& s) {
    const int tid = threadIdx.x;
    for (int i = tid; i < TILE / 8; i += BLOCK) reinterpret_cast<uint4*>(s.cnt())[i] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();
    bool ovf = false;
    auto count_id = [&](int id) {
        const uint32_t rel = (uint32_t)(id - lo);
        if (rel < (uint32_t)TILE) {
            const uint32_t sh = (rel & 1u) * 16u;
            const uint32_t old = atomicAdd(&s.cnt()[rel >> 1], 1u << sh);
            ovf |= ((old >> sh) & 0xFFFFu) == 0xFFFFu;
        }
    };
    const int nids = (int)s.nids;
    if (nids <= WIDS)                                 // the segment's window ids, gathered in LDS
        for (int i = tid; i < nids; i += BLOCK) count_id(s.ids[i]);
    else                                              // a longer window: the whole window again, from memory
        for (int64_t i = rc.b + tid; i < rc.len; i += BLOCK) {
            const int id = hist_at(a, rc, i);
            if (id >= 0 && id < a.V) count_id(id);
        }
    if (ovf) atomicOr(a.err, FS_DEVERR_COUNT_OVERFLOW);
    __syncthreads();
    const float rp = rc.p.repetition_penalty, fq = rc.p.frequency_penalty, pr = rc.p.presence_penalty;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int local = (j * BLOCK + tid) * 4;
        const uint2 c2 = *reinterpret_cast<const uint2*>(&s.cnt()[local >> 1]);
        if ((c2.x | c2.y) != 0u) {
            const uint32_t cc[4] = {c2.x & 0xFFFFu, c2.x >> 16, c2.y & 0xFFFFu, c2.y >> 16};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (cc[q] != 0u) {
                    float l = x[4 * j + q];
                    if (rc.rep_on) l = l > 0.0f ? __fdiv_rn(l, rp) : __fmul_rn(l, rp);
                    if (rc.fp_on) l = __fsub_rn(l, __fadd_rn(__fmul_rn((float)cc[q], fq), pr));
                    x[4 * j + q] = l;
                }
            }
        }
    }
}

// The segment's window ids s.ids[0, nids) (nids <= WIDS, gathered by gather_window) reordered by tile, a counting
// sort: the ids of the segment's tile t are s.ids[t > 0 ? s.off[t - 1] : 0, s.off[t]) (s.off holds the bucket ends;
// ntiles <= 2 * BLOCK). Ends with a barrier.
__device__ __forceinline__ void bucket_window(int seg_lo, int ntiles, Shared& s) {
    const int tid = threadIdx.x;
    const int n = (int)s.nids;
    constexpr int Q = WIDS / BLOCK;
    int id[Q], tl[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int i = tid + q * BLOCK;
        id[q] = i < n ? s.ids[i] : 0;
        tl[q] = i < n ? (id[q] - seg_lo) / TILE : -1;
    }
    for (int t = tid; t < ntiles; t += BLOCK) s.off[t] = 0u;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < Q; ++q)
        if (tl[q] >= 0) atomicAdd(&s.off[tl[q]], 1u);
    __syncthreads();
    const uint32_t c0 = 2 * tid < ntiles ? s.off[2 * tid] : 0u;
    const uint32_t c1 = 2 * tid + 1 < ntiles ? s.off[2 * tid + 1] : 0u;
    uint32_t tot;
    const uint32_t base = block_excl_scan<uint32_t>(c0 + c1, s.wsum, &tot);   // its barriers end the reads above
    if (2 * tid < ntiles) s.off[2 * tid] = base;                              // bucket starts
    if (2 * tid + 1 < ntiles) s.off[2 * tid + 1] = base + c0;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < Q; ++q)
        if (tl[q] >= 0) s.ids[atomicAdd(&s.off[tl[q]], 1u)] = id[q];         // the starts advance to the ends
    __syncthreads();
}

// Penalty pass on one tile (the tt-th of the segment, starting at lo) in registers, wave by wave: the ids of the
// tile's bucket (bucket_window) that fall on this wave's logits are counted in the wave's own 16-bit table, then
// each lane patches its counted logits. Element lo + e belongs to wave (e % (4 * BLOCK)) / (4 * WAVE), at index
// (e / (4 * BLOCK)) * 4 * WAVE + e % (4 * WAVE) of its table (lane l's four logits of float4 j sit at
// j * 4 * WAVE + 4 * l). A wave's LDS accesses complete in order, so no barrier is needed; tiles holding no window
// id skip the pass. Same arithmetic as apply_penalties.
__device__ __forceinline__ void wave_penalties(float (&x)[TPT], const RowCtx& rc, int lo, int tt, Shared& s) {
    static_assert(NV * 4 * WAVE * NWAVES == TILE, "a tile is the waves' float4 columns");
    static_assert(WIDS < 0xFFFF, "16-bit counts");
    const int b0 = tt > 0 ? (int)s.off[tt - 1] : 0, b1 = (int)s.off[tt];
    if (b0 == b1) return;                                // uniform: no window id in this tile
    const int lane = lane_id();
    const uint32_t w = threadIdx.x / WAVE;
    uint32_t* tb = s.cnt() + w * (NV * 4 * WAVE / 2);    // NV * 4 * WAVE 16-bit counts (all waves: TILE / 2 words)
    // Every table access is a 32-bit access of tb, with compiler barriers between the clear, the counts and the
    // reads: the hardware keeps a wave's LDS accesses in order, but vector-typed accesses are not ordered by the
    // compiler against the 32-bit atomics (no barrier here does it).
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        tb[2 * (j * WAVE + lane)] = 0u;
        tb[2 * (j * WAVE + lane) + 1] = 0u;
    }
    __asm__ volatile("" ::: "memory");
    // at most WIDS ids in the segment: a 16-bit count cannot overflow
    for (int i = b0 + lane; i < b1; i += WAVE) {
        const uint32_t e = (uint32_t)(s.ids[i] - lo);   // < TILE
        if ((e % (4u * BLOCK)) / (4u * WAVE) == w) {
            const uint32_t idx = (e / (4u * BLOCK)) * (4u * WAVE) + e % (4u * WAVE);
            atomicAdd(&tb[idx >> 1], 1u << ((idx & 1u) * 16u));
        }
    }
    __asm__ volatile("" ::: "memory");
    const float rp = rc.p.repetition_penalty, fq = rc.p.frequency_penalty, pr = rc.p.presence_penalty;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint2 c2 = make_uint2(tb[2 * (j * WAVE + lane)], tb[2 * (j * WAVE + lane) + 1]);
        if ((c2.x | c2.y) != 0u) {
            const uint32_t cc[4] = {c2.x & 0xFFFFu, c2.x >> 16, c2.y & 0xFFFFu, c2.y >> 16};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (cc[q] != 0u) {
                    float l = x[4 * j + q];
                    if (rc.rep_on) l = l > 0.0f ? __fdiv_rn(l, rp) : __fmul_rn(l, rp);
                    if (rc.fp_on) l = __fsub_rn(l, __fadd_rn(__fmul_rn((float)cc[q], fq), pr));
                    x[4 * j + q] = l;
                }
            }
        }
    }
}

// The penalty window's ids in [seg_lo, seg_hi) into s.ids (s.nids counts past WIDS). Called with the segment's
// first tiles in flight; ends with a barrier.
__device__ __forceinline__ void gather_window(const Args& a, const RowCtx& rc, int seg_lo, int seg_hi, Shared& s) {
    const int tid = threadIdx.x;
    if (tid == 0) s.nids = 0u;
    __syncthreads();
    auto take = [&](int id) {
        const bool in = id >= seg_lo && id < seg_hi;
        const uint64_t m = __ballot(in);
        if (m != 0ull) {
            uint32_t base = 0u;
            if (lane_id() == 0) base = atomicAdd(&s.nids, (uint32_t)__popcll(m));
            base = (uint32_t)__builtin_amdgcn_readlane((int)base, 0);
            const uint32_t pos = base + mbcnt(m);
            if (in && pos < (uint32_t)WIDS) s.ids[pos] = id;
        }
    };
    // the first GW * BLOCK ids requested together (one round trip), the rest round by round
    constexpr int GW = 4;
    int idq[GW];
#pragma unroll
    for (int q = 0; q < GW; ++q) {
        const int64_t i = rc.b + q * BLOCK + tid;
        idq[q] = i < rc.len ? hist_at(a, rc, i) : -1;
    }
#pragma unroll
    for (int q = 0; q < GW; ++q) take(idq[q]);
    for (int64_t i0 = rc.b + GW * BLOCK; i0 < rc.len; i0 += BLOCK) {
        const int64_t i = i0 + tid;
        take(i < rc.len ? hist_at(a, rc, i) : -1);
    }
    __syncthreads();
}

// Narrow [rlo, rhi] onto the kk-th largest value among the entries a visitor yields (32-bit values, entries
// outside [rlo, rhi] ignored; count(value > rhi) == *above < kk <= count(value >= rlo) on entry). On return
// rlo == rhi is that value, *above = count(value > it), *at = count(value >= it).
template <class Each>
__device__ __forceinline__ void narrow32(Each each, int kk, uint32_t& rlo, uint32_t& rhi, uint32_t* above, uint32_t* at, Shared& s) {
    const int tid = threadIdx.x;
    for (int level = 0; level < 4 && rlo != rhi; ++level) {
        const int sh = range_shift(rlo, rhi);
        for (int i = tid; i < NBINS; i += BLOCK) s.bins()[i] = 0u;
        __syncthreads();
        const uint32_t lo = rlo, hi = rhi;
        each([&](uint32_t v) { if (v >= lo && v <= hi) atomicAdd(&s.bins()[(v - lo) >> sh], 1u); });
        __syncthreads();
        uint32_t ab, atb;
        const int bsel = hist_locate(s.bins(), kk - (int)*above, &ab, &atb, s.wsum, s.red);
        const uint64_t nlo = (uint64_t)rlo + ((uint64_t)bsel << sh);
        const uint64_t nhi = (uint64_t)rlo + (((uint64_t)bsel + 1) << sh) - 1;
        rlo = (uint32_t)nlo;
        rhi = nhi < rhi ? (uint32_t)nhi : rhi;
        *above += ab;
        *at = *above + (atb - ab);
    }
}

// Keeps the entries >= X of the n in s.cand (at the front, through the stage) and returns their count; when more
// than KMAX would remain, changes nothing and returns -1. Whole block; returns after a barrier.
__device__ __forceinline__ int keep_from(int n, uint64_t X, Shared& s) {
    const int tid = threadIdx.x;
    uint32_t mine = 0u;
    for (int i = tid; i < n; i += BLOCK) mine += s.cand[i] >= X ? 1u : 0u;
    uint32_t tot;
    uint32_t pos = block_excl_scan<uint32_t>(mine, s.wsum, &tot);
    if (tot > (uint32_t)KMAX) return -1;
    uint64_t* st = s.stage();
    for (int i = tid; i < n; i += BLOCK) {
        const uint64_t c = s.cand[i];
        if (c >= X) st[pos++] = c;
    }
    __syncthreads();
    for (uint32_t i = tid; i < tot; i += BLOCK) s.cand[i] = st[i];
    if (tid == 0) s.count = tot;
    __syncthreads();
    return (int)tot;
}

// Exact k-th largest composite X among the n > k candidates in s.cand, then keep exactly the k entries >= X.
// Returns X. Keys first (histogram levels over [min, max]), then, if the k-th key is tied, the ids among the ties.
__device__ __forceinline__ uint64_t compact_exact(int n, int k, Shared& s) {
    const int tid = threadIdx.x;
    uint32_t kmn = 0xFFFFFFFFu, kmx = 0u;
    for (int i = tid; i < n; i += BLOCK) {
        const uint32_t kk = comp_key(s.cand[i]);
        kmn = kk < kmn ? kk : kmn;
        kmx = kk > kmx ? kk : kmx;
    }
    block_minmax_u32(kmn, kmx, s.red);
    uint32_t rlo = kmn, rhi = kmx, above = 0u, at = (uint32_t)n;
    narrow32([&](auto&& f) { for (int i = tid; i < n; i += BLOCK) f(comp_key(s.cand[i])); }, k, rlo, rhi, &above, &at,
             s);
    const uint32_t t = rlo;                                   // the k-th key
    const uint32_t need = (uint32_t)k - above;                // ties at t that belong to the top k
    uint64_t X = (uint64_t)t << 32;
    if (at - above != need) {
        // the need-th largest low word (the need-th smallest id) among the entries with key t
        uint32_t lmn = 0xFFFFFFFFu, lmx = 0u;
        for (int i = tid; i < n; i += BLOCK) {
            const uint64_t c = s.cand[i];
            if (comp_key(c) == t) {
                const uint32_t lw = (uint32_t)c;
                lmn = lw < lmn ? lw : lmn;
                lmx = lw > lmx ? lw : lmx;
            }
        }
        block_minmax_u32(lmn, lmx, s.red);
        uint32_t ab2 = 0u, at2 = 0u;
        narrow32(
            [&](auto&& f) {
                for (int i = tid; i < n; i += BLOCK) {
                    const uint64_t c = s.cand[i];
                    if (comp_key(c) == t) f((uint32_t)c);
                }
            },
            (int)need, lmn, lmx, &ab2, &at2, s);
        X |= lmn;
    }
    (void)keep_from(n, X, s);                                 // exactly k entries are >= X
    return X;
}

// The merge of one row: gathers the segments' candidates, selects and sorts the row's top k, then softmax / min-p / top-p / draw (sampler.cpp:25-49).
// ------------------------------------------------------------------------------------------------ large k
// Rows that sample with k > KMAX candidates (top_k = 0 or > 2048; ferro's k = n / top_k, sampler.cpp:26) are handled
// by one workgroup with several streaming passes over the row (it stays in L2 / MALL after the first):
//   1. the max / min composite and the count of ordered (non-NaN) logits;
//   2. the k-th composite Xk (key histograms, then ids among ties), unless every logit is a candidate;
//   3. S = sum of exp((double)(float)(v - mx) / T) over the candidates (sampler.cpp:37-41);
//   4. min-p: pr = e / S is monotone in the logit, so the kept keys are found by a binary search over keys;
//   5. top-p and the draw: the first candidate (candidate order) whose cumulative mass reaches a target, by a
//      descent over fp64 mass histograms of the keys, then the j-th smallest id among the ties at the final key.
// Sums run in a different order than ferro's sequential loop (probabilities agree to ~1e-15 relative).
constexpr int LPF = 2;                    // tiles in flight per large-row pass
constexpr int MB = 256;                   // mass histogram bins

// One pass over the whole row, LPF tiles in flight, penalties applied (the window ids are in s.ids): g(x, lo) per
// tile, called by every thread (g may use barriers). Element i of a thread is elem_id(lo, i) when < V. The tiles are
// read through a buffer resource over the row (rounded up to whole float4s, which stay inside the row's ld-strided
// allocation): loads past it return zeros without a memory access, so every tile's successor is requested
// unconditionally and the compiler's memory-counter waits stay exact (consuming a tile waits for that tile only).
template <class G>
__device__ __forceinline__ void row_tiles(const Args& a, const RowCtx& rc, Shared& s, G g) {
    const int V = a.V;
    const float* rowp = a.logits + (int64_t)rc.row * a.ld;
    const int ntile = (V + TILE - 1) / TILE;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(rowp), (short)0,
                                                                        ((V + 3) & ~3) * 4, 0x00020000);
    float buf[LPF][TPT];
#pragma unroll
    for (int p = 0; p < LPF; ++p) load_seg_tile(buf[p], rs, p);
    for (int t0 = 0; t0 < ntile; t0 += LPF) {
#pragma unroll
        for (int p = 0; p < LPF; ++p) {
            const int t = t0 + p;
            float x[TPT];
#pragma unroll
            for (int i = 0; i < TPT; ++i) x[i] = buf[p][i];
            load_seg_tile(buf[p], rs, t + LPF);
            if (t < ntile) {
                if (rc.capped) softcap_vals(x, rc.p.softcap);
                if (rc.pen) {
                    __syncthreads();                 // the previous tile's table reads are done
                    apply_penalties(x, a, rc, t * TILE, s);
                }
                g(x, t * TILE);
            }
        }
    }
    __syncthreads();
}

// Per ordered element (non-NaN, id < V): f(x, key, composite).
template <class F>
__device__ __forceinline__ void row_elems(const Args& a, const RowCtx& rc, Shared& s, F f) {
    const int V = a.V;
    row_tiles(a, rc, s, [&](const float (&x)[TPT], int lo) {
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            const int e = elem_id(lo, i);
            if (e < V && x[i] == x[i]) {
                const uint32_t kq = key_of(x[i]);
                f(x[i], kq, comp_of(kq, (uint32_t)e));
            }
        }
    });
}

__device__ __forceinline__ double mass_of(float x, float mx, double Td) {
    const float d = x - mx;                    // fp32 subtraction, as ferro
    return exp((double)d / Td);
}

// The kk-th largest composite among the ordered elements with composite in [lo_c, hi_c) (1 <= kk <= their count;
// keys of that set span [klo, khi]).
__device__ __forceinline__ uint64_t large_kth(const Args& a, const RowCtx& rc, Shared& s, int kk, uint64_t lo_c, uint64_t hi_c,
                              uint32_t klo, uint32_t khi) {
    uint32_t rlo = klo, rhi = khi, above = 0u, at = 0u;
    narrow32([&](auto&& f) {
                 row_elems(a, rc, s, [&](float, uint32_t kq, uint64_t c) { if (c >= lo_c && c < hi_c) f(kq); });
             },
             kk, rlo, rhi, &above, &at, s);
    const uint32_t t = rlo;
    const uint32_t need = (uint32_t)kk - above;
    uint32_t lmn = 0xFFFFFFFFu - (uint32_t)(a.V - 1), lmx = 0xFFFFFFFFu;
    uint32_t ab2 = 0u, at2 = 0u;
    narrow32([&](auto&& f) {
                 row_elems(a, rc, s, [&](float, uint32_t kq, uint64_t c) {
                     if (kq == t && c >= lo_c && c < hi_c) f((uint32_t)c);
                 });
             },
             (int)need, lmn, lmx, &ab2, &at2, s);
    return ((uint64_t)t << 32) | lmn;
}

// The j-th smallest id among the ordered elements with key t and composite >= lo_c (their largest id if fewer
// than j): one id-ordered pass. Returns its composite (0: none).
__device__ __forceinline__ uint64_t large_pick(const Args& a, const RowCtx& rc, Shared& s, uint32_t t, uint64_t lo_c, uint32_t j) {
    const int tid = threadIdx.x;
    const int V = a.V;
    uint32_t running = 0u;                     // flagged elements in earlier tiles (uniform)
    uint64_t found = 0ull, last = ~0ull;
    row_tiles(a, rc, s, [&](const float (&x)[TPT], int lo) {
        bool f[TPT];
        uint32_t c0 = 0u, c1 = 0u;
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            const int e = elem_id(lo, i);
            f[i] = e < V && x[i] == x[i] && key_of(x[i]) == t && comp_of(t, (uint32_t)e) >= lo_c;
            if (f[i]) {
                if (i < 4) ++c0; else ++c1;
                const uint64_t c = comp_of(t, (uint32_t)e);
                last = c < last ? c : last;
            }
        }
        uint32_t tot;                          // ids in a tile: float4 0 of every thread, then float4 1
        const uint32_t pre = block_excl_scan<uint32_t>(c0 | (c1 << 16), s.wsum, &tot);
        uint32_t r0 = running + (pre & 0xFFFFu);
        uint32_t r1 = running + (tot & 0xFFFFu) + (pre >> 16);
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            if (f[i]) {
                const uint32_t rank = i < 4 ? r0++ : r1++;
                if (rank + 1u == j) found = comp_of(t, (uint32_t)elem_id(lo, i));
            }
        }
        running += (tot & 0xFFFFu) + (tot >> 16);
    });
    found = block_max_u64(found, s.red);
    last = block_min_u64(last, s.red);
    (void)tid;
    return found != 0ull ? found : (last != ~0ull ? last : 0ull);
}

// The first candidate, in candidate order among the ordered elements with composite >= lo_c, at which the
// cumulative mass reaches target (0: the total stays below it). Keys of that set span [klo, khi].
__device__ __forceinline__ uint64_t large_mass_select(const Args& a, const RowCtx& rc, Shared& s, double target, uint64_t lo_c,
                                      uint32_t klo, uint32_t khi, float mx, double Td) {
    const int tid = threadIdx.x;
    const int w = tid / WAVE;
    double* hd = reinterpret_cast<double*>(s.cand);          // [NWAVES][MB] per-wave masses
    uint32_t* hc = s.bins();                                  // [MB] counts
    double above = 0.0;
    while (klo != khi) {
        int sh = 0;
        while (((khi - klo) >> sh) >= (uint32_t)MB) ++sh;
        for (int i = tid; i < NWAVES * MB; i += BLOCK) hd[i] = 0.0;
        for (int i = tid; i < MB; i += BLOCK) hc[i] = 0u;
        __syncthreads();
        const uint32_t lo = klo, hi = khi;
        row_elems(a, rc, s, [&](float x, uint32_t kq, uint64_t c) {
            if (c >= lo_c && kq >= lo && kq <= hi) {
                const uint32_t b = (kq - lo) >> sh;
                atomicAdd(&hd[w * MB + b], mass_of(x, mx, Td));
                atomicAdd(&hc[b], 1u);
            }
        });
        // thread t < MB owns bin MB-1-t: cumulative from the top in a fixed order
        double m = 0.0;
        uint32_t cnt = 0u;
        if (tid < MB) {
            const int b = MB - 1 - tid;
#pragma unroll
            for (int q = 0; q < NWAVES; ++q) m += hd[q * MB + b];
            cnt = hc[b];
        }
        double tot;
        const double ex = block_excl_scan<double>(m, s.red.f64, &tot);
        const int hit = (tid < MB && cnt != 0u && above + ex + m >= target) ? tid : 0x7fffffff;
        const int first = block_min_i32(hit, s.red);
        if (first == 0x7fffffff) return 0ull;
        if (tid == first) s.red.dmisc[1] = ex;
        __syncthreads();
        above += s.red.dmisc[1];
        __syncthreads();
        const uint32_t b = (uint32_t)(MB - 1 - first);
        const uint64_t nlo = (uint64_t)klo + ((uint64_t)b << sh);
        const uint64_t nhi = (uint64_t)klo + (((uint64_t)b + 1) << sh) - 1;
        klo = (uint32_t)nlo;
        khi = nhi < khi ? (uint32_t)nhi : khi;
    }
    const double et = mass_of(val_of(klo), mx, Td);
    double jd = et > 0.0 ? ceil((target - above) / et) : 1.0;
    if (!(jd >= 1.0)) jd = 1.0;
    const uint32_t j = jd > 4294967295.0 ? 0xFFFFFFFFu : (uint32_t)jd;
    return large_pick(a, rc, s, klo, lo_c, j);
}

// The exact multi-pass selection (narrowing histograms over the keys; about 15 passes over the row): the fallback
// of large_row when a coarse-bin step does not apply. Sets the token and the kept count.
__device__ __forceinline__ void large_row_exact(const Args& a, const RowCtx& rc, Shared& s, int& tok_out, int& keep_out) {
    const int tid = threadIdx.x;
    const int row = rc.row;
    const fs_row_params& p = rc.p;
    // 1. extremes and count of the ordered elements
    uint64_t cmax = 0ull, cmin = ~0ull;
    uint32_t nv = 0u;
    row_elems(a, rc, s, [&](float, uint32_t, uint64_t c) {
        cmax = c > cmax ? c : cmax;
        cmin = c < cmin ? c : cmin;
        ++nv;
    });
    cmax = block_max_u64(cmax, s.red);
    cmin = block_min_u64(cmin, s.red);
    uint32_t ntot;
    (void)block_excl_scan<uint32_t>(nv, s.wsum, &ntot);
    if (ntot == 0u) {                         // every logit NaN: no order to sample from
        tok_out = 0;
        keep_out = 0;
        return;
    }
    const uint32_t kmax = comp_key(cmax);
    const float mx = val_of(kmax);
    const double Td = (double)p.temperature;
    // 2. the candidates: composites >= Xk
    const int keff = (uint32_t)rc.k < ntot ? rc.k : (int)ntot;
    const uint64_t Xk = (uint32_t)keff == ntot ? cmin : large_kth(a, rc, s, keff, 1ull, ~0ull, comp_key(cmin), kmax);
    const uint32_t kk = comp_key(Xk);
    // 3. the softmax denominator
    double part = 0.0;
    row_elems(a, rc, s, [&](float x, uint32_t, uint64_t c) { if (c >= Xk) part += mass_of(x, mx, Td); });
    const double S = block_sum_f64(part, s.red);
    if (S != S) {                             // an infinite maximum: every mass NaN, nothing cut, the draw falls
        tok_out = (int)comp_id(Xk);           // through to the last candidate (sampler.cpp:43-49)
        keep_out = keff;
        return;
    }
    // 4. min-p: the smallest key whose pr reaches pr[0] * min_p (pr[0] = 1 / S)
    uint64_t Xkeep = Xk;
    if (p.min_p > 0.0f) {
        const double thr = (1.0 / S) * (double)p.min_p;
        auto ok = [&](uint32_t key) { return mass_of(val_of(key), mx, Td) / S >= thr; };
        uint64_t Xm;
        if (!ok(kmax)) {
            Xm = cmax;                                  // keep >= 1
        } else {
            uint32_t lo = kk, hi = kmax;
            while (lo < hi) {
                const uint32_t mid = lo + ((hi - lo) >> 1);
                if (ok(mid)) hi = mid; else lo = mid + 1u;
            }
            Xm = (uint64_t)lo << 32;
        }
        Xkeep = Xm > Xkeep ? Xm : Xkeep;
    }
    // 5. top-p: the crossing candidate is the last one kept (sampler.cpp:44)
    if (p.top_p < 1.0f) {
        const uint64_t Xc = large_mass_select(a, rc, s, (double)p.top_p * S, Xk, kk, kmax, mx, Td);
        if (Xc != 0ull) Xkeep = Xc > Xkeep ? Xc : Xkeep;
    }
    // tot over the kept prefix, its size and its last candidate
    double tpart = 0.0;
    uint32_t kc = 0u;
    uint64_t clast = ~0ull;
    row_elems(a, rc, s, [&](float x, uint32_t, uint64_t c) {
        if (c >= Xkeep) {
            tpart += mass_of(x, mx, Td);
            ++kc;
            clast = c < clast ? c : clast;
        }
    });
    const double tot = block_sum_f64(tpart, s.red);
    uint32_t keep;
    (void)block_excl_scan<uint32_t>(kc, s.wsum, &keep);
    clast = block_min_u64(clast, s.red);
    // 6. the draw r = u * tot (sampler.cpp:45-49), in mass units
    const double u = row_u(a, row);
    uint64_t pick = large_mass_select(a, rc, s, u * tot + 0.0, Xkeep, comp_key(Xkeep), kmax, mx, Td);
    if (pick == 0ull) pick = clast;
    tok_out = (int)comp_id(pick);
    keep_out = (int)keep;
    (void)tid;
}

// Optional outputs of a large row: the first min(k, kcap) candidates in candidate order, KMAX at a time.
__device__ __forceinline__ void large_outputs(const Args& a, const RowCtx& rc, Shared& s, int keff, uint64_t Xk, uint32_t kk,
                                              uint32_t kmax, float mx, double Td, double S) {
    const int tid = threadIdx.x;
    const int row = rc.row;
    if (a.mode != MODE_VERIFY && a.kcap > 0 && (a.cand_ids || a.cand_probs)) {
        const int mtot = keff < a.kcap ? keff : a.kcap;
        uint64_t hi_c = ~0ull;                          // this chunk: composites in [Xc, hi_c)
        for (int done = 0; done < mtot;) {
            const int m = mtot - done < KMAX ? mtot - done : KMAX;
            const uint32_t khi = hi_c == ~0ull ? kmax : comp_key(hi_c - 1ull);
            const uint64_t Xc = done + m == keff ? Xk : large_kth(a, rc, s, m, Xk, hi_c, kk, khi);
            if (tid == 0) s.count = 0u;
            __syncthreads();
            const int V = a.V;
            row_tiles(a, rc, s, [&](const float (&x)[TPT], int lo) {
#pragma unroll
                for (int i = 0; i < TPT; ++i) {
                    const int e = elem_id(lo, i);
                    const bool in = e < V && x[i] == x[i] && comp_of(key_of(x[i]), (uint32_t)e) >= Xc &&
                                    comp_of(key_of(x[i]), (uint32_t)e) < hi_c;
                    wave_append(in, in ? comp_of(key_of(x[i]), (uint32_t)e) : 0ull, s.cand, &s.count, CAP);
                }
            });
            bin_sort_desc(m, s);
            for (int i = tid; i < m; i += BLOCK) {
                const uint64_t c = s.cand[i];
                const int64_t o = (int64_t)row * a.kcap + done + i;
                if (a.cand_ids) a.cand_ids[o] = (int32_t)comp_id(c);
                if (a.cand_probs) a.cand_probs[o] = mass_of(val_of(comp_key(c)), mx, Td) / S;
            }
            __syncthreads();
            done += m;
            hi_c = Xc;
        }
    }
}


// ---- large k through coarse key bins: a few passes instead of ~15
// Pass 1: extremes and a count histogram over LB coarse bins (key >> LB_SHIFT). Xk (the k-th composite, k < the
// count) is narrowed inside its coarse bin. Pass 2: S (a deterministic fp64 block sum, as the exact path) and a
// fixed-point mass histogram over the same bins (integer sums: deterministic, within 2^-44 per element). The bins'
// masses stay in registers (thread t: descending positions PT*t ..). The top-p and draw targets each pick a coarse
// bin from them; one pass gathers that bin's candidates into LDS, a counting sort orders them and the exact fp64
// masses are walked in candidate order from the bin's fixed-point "above" mass. A target that does not fall inside
// its bin's exact masses (a rounding step at the bin edge), or a bin of more than KMAX candidates, takes the exact
// multi-pass selection instead.
constexpr int LB = 4096;                    // coarse key bins of the large-k path
constexpr int LB_SHIFT = 32 - 12;
constexpr int LPT = LB / BLOCK;             // coarse bins per thread
constexpr double FXS = 17592186044416.0;    // 2^44: fixed-point mass scale (an element's mass is <= 1)
static_assert(LB * 8 <= CAP * 8, "the fixed-point mass histogram fits the candidate buffer");

// Smallest descending position d (bin LB-1-d) at which the running total from the top reaches target, given each
// thread's LPT values at positions LPT*t + j; *above = the total of the positions before d. -1: never reached.
template <class T>
__device__ __forceinline__ int desc_locate(const T (&v)[LPT], T target, T* above, T* wsum, Shared& s) {
    const int tid = threadIdx.x;
    T sum = T(0);
#pragma unroll
    for (int j = 0; j < LPT; ++j) sum += v[j];
    T tot;
    T run = block_excl_scan<T>(sum, wsum, &tot);
    int hit = 0x7fffffff;
    T ab = T(0);
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
        if (hit == 0x7fffffff && v[j] != T(0) && run + v[j] >= target) {
            hit = LPT * tid + j;
            ab = run;
        }
        run += v[j];
    }
    const int d = block_min_i32(hit, s.red);
    if (d == 0x7fffffff) return -1;
    if (hit == d) s.red.u64b[0] = (uint64_t)ab;
    __syncthreads();
    *above = (T)s.red.u64b[0];
    __syncthreads();
    return d;
}
// Gathers the candidates (composite >= lo_c) of coarse bin b into s.cand[0, n) and sorts them; returns n, or -1
// when more than KMAX (the caller falls back). Extra per-element work f(x, key, composite) for every candidate.
template <class F>
__device__ __forceinline__ int large_gather_bin(const Args& a, const RowCtx& rc, Shared& s, uint32_t b, uint64_t lo_c, F f) {
    const int V = a.V;
    if (threadIdx.x == 0) s.count = 0u;
    __syncthreads();
    row_tiles(a, rc, s, [&](const float (&x)[TPT], int lo) {
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            const int e = elem_id(lo, i);
            const bool ok = e < V && x[i] == x[i];
            const uint32_t kq = key_of(x[i]);
            const uint64_t c = comp_of(kq, (uint32_t)e);
            const bool cand = ok && c >= lo_c;
            if (cand) f(x[i], kq, c);
            const bool in = cand && (kq >> LB_SHIFT) == b;
            wave_append(in, c, s.cand, &s.count, KMAX);
        }
    });
    const int n = (int)s.count;                       // row_tiles ends with a barrier
    if (n > KMAX) return -1;
    bin_sort_desc(n, s);
    return n;
}

// The first of the n sorted entries s.cand[0, n) with composite >= lo_c at which above + the running exact mass
// reaches target: its index, and the running mass there in *cum. -1: above >= target (the crossing lies in a higher
// bin); -2: the bin's masses end below target.
__device__ __forceinline__ int large_walk(Shared& s, int n, uint64_t lo_c, double above, double target, float mx, double Td,
                                          double* cum) {
    const int i0 = (int)threadIdx.x * KPT;
    if (!(above < target)) return -1;
    double e[KPT], run = 0.0;
#pragma unroll
    for (int q = 0; q < KPT; ++q) {
        const int i = i0 + q;
        e[q] = (i < n && s.cand[i] >= lo_c) ? mass_of(val_of(comp_key(s.cand[i])), mx, Td) : 0.0;
        run += e[q];
    }
    double tot;
    const double off = block_excl_scan<double>(run, s.red.f64, &tot);
    double c = above + off;
    int hit = 0x7fffffff;
    double ch = 0.0;
#pragma unroll
    for (int q = 0; q < KPT; ++q) {
        c += e[q];
        if (hit == 0x7fffffff && i0 + q < n && e[q] > 0.0 && c >= target) { hit = i0 + q; ch = c; }
    }
    const int first = block_min_i32(hit, s.red);
    if (first == 0x7fffffff) return -2;
    if (hit == first) s.red.dmisc[2] = ch;
    __syncthreads();
    *cum = s.red.dmisc[2];
    __syncthreads();
    return first;
}

// What a large row's optional candidate outputs need (large_outputs), left by large_row or large_segment.
struct LargeOut {
    bool valid;
    int keff;
    uint64_t Xk;
    uint32_t kmax;
    double S;
};

// The whole large-k sample of one row: token and kept count; lo describes the candidates for the optional outputs.
__device__ __forceinline__ void large_row(const Args& a, const RowCtx& rc, Shared& s, int& tok_out, int& keep_out,
                                          LargeOut& lo) {
    lo.valid = false;
    const int tid = threadIdx.x;
    const int row = rc.row;
    const fs_row_params& p = rc.p;
    if (rc.pen) gather_window(a, rc, 0, a.V, s);
    // 1. extremes, count of the ordered elements, their coarse-bin counts (only needed to find the k-th when k < V:
    //    k >= V takes every ordered logit)
    uint32_t* hc = reinterpret_cast<uint32_t*>(s.cand);
    const bool need_kth = rc.k < a.V;
    for (int i = tid; i < LB; i += BLOCK) hc[i] = 0u;
    __syncthreads();
    uint64_t cmax = 0ull, cmin = ~0ull;
    uint32_t nv = 0u;
    row_elems(a, rc, s, [&](float, uint32_t kq, uint64_t c) {
        cmax = c > cmax ? c : cmax;
        cmin = c < cmin ? c : cmin;
        ++nv;
        if (need_kth) atomicAdd(&hc[kq >> LB_SHIFT], 1u);
    });
    cmax = block_max_u64(cmax, s.red);
    cmin = block_min_u64(cmin, s.red);
    uint32_t ntot;
    (void)block_excl_scan<uint32_t>(nv, s.wsum, &ntot);
    if (ntot == 0u) {                         // every logit NaN: no order to sample from
        tok_out = 0;
        keep_out = rc.greedy ? 1 : 0;
        return;
    }
    const uint32_t kmax = comp_key(cmax);
    const float mx = val_of(kmax);
    if (rc.greedy) {                          // ferro's scan (sampler.cpp:19-23): the first maximum above -inf,
        tok_out = mx > -__builtin_huge_valf() ? (int)comp_id(cmax) : 0;       // never moving off a NaN at index 0
        if (ld_const(a.logits + (int64_t)row * a.ld) != ld_const(a.logits + (int64_t)row * a.ld)) tok_out = 0;
        keep_out = 1;
        if (tid == 0 && a.mode != MODE_VERIFY && a.kcap > 0) {
            if (a.cand_ids) a.cand_ids[(int64_t)row * a.kcap] = tok_out;
            if (a.cand_probs) a.cand_probs[(int64_t)row * a.kcap] = 1.0;
        }
        return;
    }
    const double Td = (double)p.temperature;
    const int keff = (uint32_t)rc.k < ntot ? rc.k : (int)ntot;
    uint64_t Xk = cmin;
    if ((uint32_t)keff < ntot) {                          // the k-th composite, inside its coarse bin
        uint32_t cv[LPT];
#pragma unroll
        for (int j = 0; j < LPT; ++j) cv[j] = hc[LB - 1 - (LPT * tid + j)];
        uint32_t abk = 0u;
        const int dk = desc_locate<uint32_t>(cv, (uint32_t)keff, &abk, s.wsum, s);
        const uint32_t bk = (uint32_t)(LB - 1 - dk);
        const uint32_t blo = bk << LB_SHIFT, bhi = blo | ((1u << LB_SHIFT) - 1u);
        Xk = large_kth(a, rc, s, keff - (int)abk, 1ull, ~0ull, blo, bhi);
    }
    const uint32_t kk = comp_key(Xk);
    // 2. S and the fixed-point mass histogram of the candidates
    uint64_t* hm = reinterpret_cast<uint64_t*>(s.cand);
    for (int i = tid; i < LB; i += BLOCK) hm[i] = 0ull;
    __syncthreads();
    double part = 0.0;
    row_elems(a, rc, s, [&](float x, uint32_t kq, uint64_t c) {
        if (c >= Xk) {
            const double m = mass_of(x, mx, Td);
            part += m;
            atomicAdd(reinterpret_cast<unsigned long long*>(&hm[kq >> LB_SHIFT]), (unsigned long long)(m * FXS + 0.5));
        }
    });
    const double S = block_sum_f64(part, s.red);          // its barriers also complete the histogram
    if (S != S) {                                         // an infinite maximum: every mass NaN, nothing cut, the
        lo.valid = true; lo.keff = keff; lo.Xk = Xk; lo.kmax = kmax; lo.S = S;   // draw falls through to the last
        tok_out = (int)comp_id(Xk);                       // candidate (sampler.cpp:43-49)
        keep_out = keff;
        return;
    }
    uint64_t mv[LPT];
#pragma unroll
    for (int j = 0; j < LPT; ++j) mv[j] = hm[LB - 1 - (LPT * tid + j)];
    __syncthreads();                                      // the candidate buffer is reused below
    // 3. min-p: the smallest key whose pr reaches pr[0] * min_p (pr[0] = 1 / S)
    bool ok_fast = true;
    uint64_t Xm = 0ull;
    uint32_t km = 0xFFFFFFFFu;
    if (p.min_p > 0.0f) {
        const double thr = (1.0 / S) * (double)p.min_p;
        auto ok = [&](uint32_t key) { return mass_of(val_of(key), mx, Td) / S >= thr; };
        if (!ok(kmax)) {
            Xm = cmax;                                    // keep >= 1
        } else {
            uint32_t lo = kk, hi = kmax;
            while (lo < hi) {
                const uint32_t mid = lo + ((hi - lo) >> 1);
                if (ok(mid)) hi = mid; else lo = mid + 1u;
            }
            km = lo;
            Xm = (uint64_t)lo << 32;
        }
    }
    // 4. top-p's crossing bin, gathered with the min-p counts and masses
    uint64_t Xc = 0ull;
    uint32_t keep_c = 0u;
    double tot_c = 0.0;
    int nc = -1;                                          // top-p's bin, sorted in s.cand (-1: none)
    uint32_t bc = 0u;
    double above_c = 0.0;
    uint32_t cnt_m = 0u, ca_c = 0u;
    double sum_m = 0.0;
    uint64_t cl_m = ~0ull;
    const bool need_m = p.min_p > 0.0f && Xm != cmax;
    if (p.top_p < 1.0f || need_m) {
        const double tgt = (double)p.top_p * S;
        uint64_t abfx = 0ull;
        int dc = -1;
        if (p.top_p < 1.0f) {
            dc = desc_locate<uint64_t>(mv, (uint64_t)(tgt * FXS), &abfx, s.red.u64b, s);
            if (dc < 0) dc = LB - 1 - (int)(kk >> LB_SHIFT);     // the total rounds below the target: last bin
            bc = (uint32_t)(LB - 1 - dc);
            above_c = (double)abfx / FXS;
        }
        const uint32_t bsel = p.top_p < 1.0f ? bc : 0xFFFFFFFFu;
        uint32_t my_ca = 0u, my_cm = 0u;
        double my_sm = 0.0;
        uint64_t my_cl = ~0ull;
        nc = large_gather_bin(a, rc, s, bsel, Xk, [&](float x, uint32_t kq, uint64_t c) {
            if ((kq >> LB_SHIFT) > bsel && bsel != 0xFFFFFFFFu) ++my_ca;
            if (need_m && kq >= km) {
                ++my_cm;
                my_sm += mass_of(x, mx, Td);
                my_cl = c < my_cl ? c : my_cl;
            }
        });
        (void)block_excl_scan<uint32_t>(my_ca, s.wsum, &ca_c);
        if (need_m) {
            (void)block_excl_scan<uint32_t>(my_cm, s.wsum, &cnt_m);
            sum_m = block_sum_f64(my_sm, s.red);
            cl_m = block_min_u64(my_cl, s.red);
        }
        if (p.top_p < 1.0f) {
            if (nc < 0) {
                ok_fast = false;
            } else {
                double cum = 0.0;
                const int ic = large_walk(s, nc, Xk, above_c, tgt, mx, Td, &cum);
                if (ic < 0) {
                    ok_fast = false;
                } else {
                    Xc = s.cand[ic];
                    keep_c = ca_c + (uint32_t)ic + 1u;
                    tot_c = cum;
                }
            }
        }
    }
    lo.valid = true; lo.keff = keff; lo.Xk = Xk; lo.kmax = kmax; lo.S = S;
    if (!ok_fast) {
        large_row_exact(a, rc, s, tok_out, keep_out);
        return;
    }
    // the kept prefix: the largest of the three thresholds (sampler.cpp:43-44)
    uint64_t Xkeep = Xk, clast = Xk;
    uint32_t keep = (uint32_t)keff;
    double tot = S;
    if (p.min_p > 0.0f && Xm > Xkeep) {
        Xkeep = Xm;
        if (Xm == cmax) { keep = 1u; tot = 1.0; clast = cmax; }   // mass_of(mx) = exp(0)
        else { keep = cnt_m; tot = sum_m; clast = cl_m; }
    }
    if (p.top_p < 1.0f && Xc > Xkeep) {
        Xkeep = Xc;
        keep = keep_c;
        tot = tot_c;
        clast = Xc;
    }
    // 5. the draw r = u * tot (sampler.cpp:45-49), in mass units
    const double u = row_u(a, row);
    const double r = u * tot + 0.0;
    uint64_t abd = 0ull;
    int dd = desc_locate<uint64_t>(mv, (uint64_t)(r * FXS), &abd, s.red.u64b, s);
    uint64_t pick = 0ull;
    bool drawn = false;
    if (dd >= 0) {
        const uint32_t bd = (uint32_t)(LB - 1 - dd);
        int nd = -1;
        if (nc >= 0 && bd == bc && p.top_p < 1.0f) {
            nd = nc;                                          // the same bin is in LDS already
        } else {
            nd = large_gather_bin(a, rc, s, bd, Xkeep, [&](float, uint32_t, uint64_t) {});
        }
        if (nd >= 0) {
            double cum = 0.0;
            const int id = large_walk(s, nd, Xkeep, (double)abd / FXS, r, mx, Td, &cum);
            if (id >= 0) {
                pick = s.cand[id];
                drawn = true;
            } else if (id == -2 && comp_key(Xkeep) >> LB_SHIFT == bd) {
                drawn = true;                                 // past the last kept candidate: clast
            }
        }
    }
    if (!drawn) pick = large_mass_select(a, rc, s, r, Xkeep, comp_key(Xkeep), kmax, mx, Td);
    if (pick == 0ull) pick = clast;
    tok_out = (int)comp_id(pick);
    keep_out = (int)keep;
}

// Large rows sampled by their segments together (large_segment, below): the list slot's scalars and the row barrier.
// Slot layout: each phase's scalars in a 128-byte line of their own, then three gather regions of whole lines. A
// segment reads another segment's line only after the barrier that follows its writing, and never earlier in the
// call, so no line it reads can be stale in its L1.
constexpr int LLINE = 16;                      // composites per 128-byte line
constexpr int LSC = 5 * LLINE;                 // scalar lines at the head of a large-row segment's list slot
constexpr int LLR = ((CAP - LSC) / 3) / LLINE * LLINE;   // capacity of each of its three gather regions
enum LargeSlot : int {
    LS_MAX = 0, LS_MIN, LS_NV,                                   // P1: largest / smallest composite, ordered count
    LS_FN, LS_FC, LS_FT,                                         // P1, every token a candidate: the cut's list count,
                                                                 // its fp64 mass and the rest's (both relative to LS_MAX)
    LS_SHI = LLINE, LS_NBK,                                      // P2: fp64 mass of the candidates above bk; bin bk's count
    LS_NBC = 2 * LLINE, LS_CA, LS_CNTM, LS_SUMM, LS_CLM,         // P3: bin bc's count, candidates above bc, min-p's
    LS_NBD = 3 * LLINE,                                          // P4: bin bd's count
    LS_TOK = 4 * LLINE, LS_XK, LS_S, LS_KEFF, LS_STATUS          // segment 0: token | keep << 32, Xk, S, keff | kmax << 32, 1 = done
};
static_assert(LS_STATUS < LSC, "the scalars fit the slot head");
static_assert(LSC + 3 * LLR <= CAP, "three gather regions after the scalars");

// The row barrier counter: the row histogram's bin RBINS - 2, above every ordered key (bins <= 4088) like the
// completion counter. Low 15 bits: arrivals; bit 15: the row is abandoned.
__device__ __forceinline__ uint32_t* row_sync_ctr(const Args& a, int row) {
    return a.rhist + (int64_t)row * RBINS + (RBINS - 2);
}
constexpr uint32_t ROW_ABANDONED = 0x8000u;
__device__ __forceinline__ void row_abandon(const Args& a, int row) {
    if (threadIdx.x == 0) __hip_atomic_fetch_or(row_sync_ctr(a, row), ROW_ABANDONED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// ------------------------------------------------------------------------------------------------ one-wave finish
// For k <= 64 once the block has narrowed the row to c1 <= 128 candidates (composites, all distinct, containing the
// top k) and ranked them (block_ranks): wave 0 places them (lane i = candidate i in ferro's order) and runs the
// softmax / min-p / top-p / draw of sampler.cpp:37-49, the sums as DPP wave scans in candidate order. LDS accesses
// of one wave are ordered, so no further block barrier is needed: the other waves go straight to the epilogue.

__device__ __forceinline__ double lane_f64(double v, int lane) {   // lane: wave-uniform
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Ranks of the c1 <= 128 candidates in[0, c1) (whole block, one barrier): thread t compares candidate t % 128
// with a quarter of the list; rk[q*128 + e] is candidate e's count of larger entries in quarter q. Pads in[c1, 128)
// with 0 first. Returns after a barrier.
__device__ __forceinline__ void block_ranks(uint64_t* in, int c1, uint32_t* rk) {
    const int tid = threadIdx.x;
    if (tid >= c1 && tid < 2 * WAVE) in[tid] = 0ull;
    __syncthreads();
    const int e = tid & (2 * WAVE - 1), q = tid / (2 * WAVE);
    const uint64_t me = in[e];
    int r = 0;
#pragma unroll
    for (int j = 0; j < 2 * WAVE / 4; ++j) r += in[q * (2 * WAVE / 4) + j] > me ? 1 : 0;
    rk[q * 2 * WAVE + e] = (uint32_t)r;
    __syncthreads();
}
static_assert(BLOCK == 4 * 2 * WAVE, "block_ranks splits 128 candidates into four quarters");

__device__ __forceinline__ void wave_finish(const Args& a, const RowCtx& rc, const uint64_t* in, const uint32_t* rk,
                                            int k, double u, double* wbuf, int& tok_out, int& keep_out) {
    const int lane = lane_id();
    const int row = rc.row;
    // lane holds candidates lane and lane + 64 (0 = none) with their ranks from block_ranks
    const uint64_t m0 = in[lane], m1 = in[lane + WAVE];
    int r0 = 0, r1 = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        r0 += (int)rk[q * 2 * WAVE + lane];
        r1 += (int)rk[q * 2 * WAVE + lane + WAVE];
    }
    uint64_t* sorted = reinterpret_cast<uint64_t*>(wbuf) + WAVE;     // [WAVE] after the [WAVE] doubles
    if (m0 != 0ull && r0 < k) sorted[r0] = m0;
    if (m1 != 0ull && r1 < k) sorted[r1] = m1;
    const uint64_t v = lane < k ? sorted[lane] : 0ull;               // candidate `lane` in ferro's order
    // softmax at temperature, min-p, top-p, draw (sampler.cpp:37-49)
    const fs_row_params& p = rc.p;
    const float mx = val_of(comp_key(sorted[0]));
    const double Td = (double)p.temperature;
    double e = 0.0;
    if (lane < k) {
        const float d = val_of(comp_key(v)) - mx;        // fp32 subtraction, as ferro
        e = exp((double)d / Td);
    }
    const double sum = lane_f64(wave_scan_f64(e), WAVE - 1);   // lanes >= k hold 0
    const double pr = e / sum;
    const double cum = wave_scan_f64(pr);                 // ferro's running c (sampler.cpp:44,47)
    int keep_m = k;
    if (p.min_p > 0.0f) {                                 // keep = 1 + the last index not below pr[0]*min_p (NaN masses stay)
        const double thr = lane_f64(pr, 0) * (double)p.min_p;
        const uint64_t mm = __ballot(lane < k && !(pr < thr));
        keep_m = mm ? 64 - __clzll((long long)mm) : 1;
    }
    int keep = keep_m;
    if (p.top_p < 1.0f) {
        const uint64_t mm = __ballot(lane < keep_m && cum >= (double)p.top_p);
        if (mm) {
            const int first = __ffsll((unsigned long long)mm) - 1;
            keep = first + 1 < keep_m ? first + 1 : keep_m;
        }
    }
    const double tot = lane_f64(cum, keep - 1);
    const double rr = u * tot + 0.0;
    const uint64_t hm = __ballot(lane < keep && rr <= cum);
    const int at = hm ? __ffsll((unsigned long long)hm) - 1 : keep - 1;
    tok_out = (int)comp_id(sorted[at]);
    keep_out = keep;
    if (a.mode != MODE_VERIFY) {
        const int m = k < a.kcap ? k : a.kcap;
        if (lane < m) {
            if (a.cand_ids) a.cand_ids[(int64_t)row * a.kcap + lane] = (int32_t)comp_id(v);
            if (a.cand_probs) a.cand_probs[(int64_t)row * a.kcap + lane] = pr;
        }
    }
}

// The segment lists of a row, loaded at the merge kernel's entry (before the row's parameters, whose latency they
// overlap): tps threads per list, each holding the list's meta and SPEC entries r_me, r_me + tps, ... (entries past
// the list's count are stale and masked once the counts are known).
struct Pre {
    int tps, c_me, r_me;
    bool act;
    uint32_t t0m, cnm;
    uint64_t v[SPEC];
    double u;                              // the row's draw (requested with the lists)
    float l0;                              // the row's first logit (a NaN there is ferro's greedy answer)
};

__device__ __forceinline__ void prefetch_lists(const Args& a, const RowCtx& rc, Pre& pre) {
    const int row = rc.row;
    const int nseg = rc.nseg;
    const int tid = threadIdx.x;
    pre.tps = nseg > 0 ? BLOCK / nseg : 0;    // >= 1: the host keeps nseg < BLOCK
    pre.c_me = nseg > 0 ? tid % nseg : 0;
    pre.r_me = nseg > 0 ? tid / nseg : 0;
    pre.act = nseg > 0 && pre.r_me < pre.tps;
    const int64_t slot = slot_of(rc, pre.c_me);
    const uint64_t* lst = a.cand + slot * CAP;
    pre.u = row_u(a, row);
    pre.l0 = ld_const(a.logits + (int64_t)row * a.ld);
    pre.t0m = 0u;
    pre.cnm = 0u;
    if (nseg > 0) {
        pre.t0m = a.meta[2 * slot];
        pre.cnm = a.meta[2 * slot + 1];
    }
#pragma unroll
    for (int q = 0; q < SPEC; ++q) pre.v[q] = nseg > 0 ? lst[pre.act ? pre.r_me + q * pre.tps : 0] : 0ull;
}

// Softmax at temperature, min-p, top-p and the draw (sampler.cpp:37-49) over k <= WAVE candidates held by one wave:
// lane i holds candidate i in ferro's order (0 past k). Sums are DPP wave scans in candidate order. Writes the
// optional candidate outputs; returns the token and the kept count.
__device__ __forceinline__ void wave_softmax(const Args& a, const RowCtx& rc, uint64_t v, int k, double u, int& tok_out,
                                             int& keep_out) {
    const int lane = lane_id();
    const int row = rc.row;
    const fs_row_params& p = rc.p;
    const float mx = val_of(comp_key(read_lane(v, 0)));
    const double Td = (double)p.temperature;
    double e = 0.0;
    if (lane < k) {
        const float d = val_of(comp_key(v)) - mx;        // fp32 subtraction, as ferro
        e = exp((double)d / Td);
    }
    const double sum = lane_f64(wave_scan_f64(e), WAVE - 1);   // lanes >= k hold 0
    const double pr = e / sum;
    const double cum = wave_scan_f64(pr);                 // ferro's running c (sampler.cpp:44,47)
    int keep_m = k;
    if (p.min_p > 0.0f) {                                 // keep = 1 + the last index not below pr[0]*min_p (NaN masses stay)
        const double thr = lane_f64(pr, 0) * (double)p.min_p;
        const uint64_t mm = __ballot(lane < k && !(pr < thr));
        keep_m = mm ? 64 - __clzll((long long)mm) : 1;
    }
    int keep = keep_m;
    if (p.top_p < 1.0f) {
        const uint64_t mm = __ballot(lane < keep_m && cum >= (double)p.top_p);
        if (mm) {
            const int first = __ffsll((unsigned long long)mm) - 1;
            keep = first + 1 < keep_m ? first + 1 : keep_m;
        }
    }
    const double tot = lane_f64(cum, keep - 1);
    const double rr = u * tot + 0.0;
    const uint64_t hm = __ballot(lane < keep && rr <= cum);
    const int at = hm ? __ffsll((unsigned long long)hm) - 1 : keep - 1;
    tok_out = (int)comp_id(read_lane(v, at));
    keep_out = keep;
    if (a.mode != MODE_VERIFY) {
        const int m = k < a.kcap ? k : a.kcap;
        if (lane < m) {
            if (a.cand_ids) a.cand_ids[(int64_t)row * a.kcap + lane] = (int32_t)comp_id(v);
            if (a.cand_probs) a.cand_probs[(int64_t)row * a.kcap + lane] = pr;
        }
    }
}

// The short merge: rows with no partial tail tile whose segment lists lie inside the prefetched windows.
//   - greedy rows: the largest of the segments' maxima (wave 0; lanes < nseg hold entry 0 of every list);
//   - k <= WAVE: the candidates at or above L (the largest of the lists' bounds; at least k of the row's logits reach
//     every bound) go into LDS (one LDS atomic per wave); when there are at most 2 * BLOCK / 4 of them the block ranks
//     them (P threads per candidate, each comparing with 1/P of the list), places the first k by rank, and wave 0
//     finishes the row.
// Returns false, after a barrier and with nothing written, when the row does not fit (the general merge then runs).
constexpr int FRANK = BLOCK / 2;          // largest candidate count the short merge ranks
__device__ __forceinline__ bool merge_fast(const Args& a, const RowCtx& rc, Shared& s, const Pre& pre, int& tok,
                                           int& keep) {
    const int tid = threadIdx.x;
    const int k = rc.k;
    if (rc.nseg > FAST_SEGS) return false;
    const uint32_t cmax = wave_max(pre.cnm);
    if (cmax > (uint32_t)(SPEC * pre.tps)) return false;        // uniform: every wave holds every list's meta
    if (rc.greedy) {
        if (tid < WAVE) {
            uint64_t best = (pre.act && pre.r_me == 0) ? pre.v[0] : 0ull;   // each segment's best (entry 0)
            best = wave_max(best);
            tok = best != 0ull ? (int)comp_id(best) : 0;      // nothing above -inf / NaN: ferro's scan stays at 0
            if (pre.l0 != pre.l0) tok = 0;                    // ferro's scan never moves off a NaN at index 0
            keep = 1;
            if (tid == 0 && a.mode != MODE_VERIFY) {
                if (a.cand_ids && a.kcap > 0) a.cand_ids[(int64_t)rc.row * a.kcap] = tok;
                if (a.cand_probs && a.kcap > 0) a.cand_probs[(int64_t)rc.row * a.kcap] = 1.0;
            }
        }
        return true;
    }
    if (k > WAVE) return false;
    const uint32_t L = wave_max(pre.t0m);
    // the candidates >= L into LDS: one atomic per wave for all of a thread's entries
    {
        uint64_t bal[SPEC];
        uint32_t tot = 0u;
#pragma unroll
        for (int q = 0; q < SPEC; ++q) {
            const uint64_t w = pre.v[q];
            const bool in = pre.act && (uint32_t)(pre.r_me + q * pre.tps) < pre.cnm && w != 0ull && comp_key(w) >= L;
            bal[q] = __ballot(in);
            tot += (uint32_t)__popcll(bal[q]);
        }
        if (tid == 0) s.count = 0u;
        __syncthreads();
        if (tot != 0u) {
            uint32_t base = 0u;
            if (lane_id() == 0) base = atomicAdd(&s.count, tot);
            base = (uint32_t)__builtin_amdgcn_readlane((int)base, 0);
#pragma unroll
            for (int q = 0; q < SPEC; ++q) {
                if ((bal[q] >> lane_id()) & 1ull) s.cand[base + mbcnt(bal[q])] = pre.v[q];
                base += (uint32_t)__popcll(bal[q]);
            }
        }
    }
    __syncthreads();
    FS_MARK(2);
    const int n = (int)s.count;
    if (n < k || n > FRANK) {                                    // uniform
        __syncthreads();
        return false;
    }
    // ranks: P threads per candidate (c = tid % per), part q compares candidate c with entries [q*span, (q+1)*span)
    const int P = n <= BLOCK / 4 ? 4 : 2;
    const int per = BLOCK / P;
    const int span = (n + P - 1) / P;
    const int c = tid % per, q = tid / per;
    uint32_t* rk = reinterpret_cast<uint32_t*>(s.cand + FRANK);            // [BLOCK]
    uint64_t* sorted = s.cand + FRANK + BLOCK / 2;                        // [WAVE]
    if (c < n) {
        const uint64_t me = s.cand[c];
        const int j0 = q * span, j1 = j0 + span < n ? j0 + span : n;
        uint32_t r = 0u;
        int j = j0;
        for (; j + 4 <= j1; j += 4) {                  // four LDS reads in flight per step
            const uint64_t e0 = s.cand[j], e1 = s.cand[j + 1], e2 = s.cand[j + 2], e3 = s.cand[j + 3];
            r += (e0 > me ? 1u : 0u) + (e1 > me ? 1u : 0u) + (e2 > me ? 1u : 0u) + (e3 > me ? 1u : 0u);
        }
        for (; j < j1; ++j) r += s.cand[j] > me ? 1u : 0u;
        rk[q * per + c] = r;
    }
    __syncthreads();
    if (tid < n) {
        uint32_t r = 0u;
        for (int qq = 0; qq < P; ++qq) r += rk[qq * per + tid];
        if (r < (uint32_t)k) sorted[r] = s.cand[tid];
    }
    __syncthreads();
    FS_MARK(3);
    if (tid < WAVE) wave_softmax(a, rc, tid < k ? sorted[tid] : 0ull, k, pre.u, tok, keep);
    return true;
}

// ------------------------------------------------------------------------------------------------ decode step
// fs_decode_step's two additions to a row's merge (server.cpp:603-606, then gen_token's hist.push_back,
// server.cpp:342): its stream's history copied to the new histories (while the merge waits for its segments) and
// the token appended after it; and the row's draw committed (its stream advanced) once every reader is done.
// Stream s = row s; the new histories start at 0 and each stream gains one id (fs_hist_append's layout).
__device__ __forceinline__ void decode_hist_copy(const Args& a, int row) {
    if (!a.out_hist_off) return;
    const int64_t h0 = a.hist_off ? a.hist_off[0] : 0, b = a.hist_off ? a.hist_off[row] : 0;
    const int64_t e = a.hist_off ? a.hist_off[row + 1] : 0;
    const int64_t nb = b - h0 + row;
    for (int64_t i = threadIdx.x; i < e - b; i += BLOCK)
        if (nb + i < a.out_cap) a.out_hist[nb + i] = a.hist[b + i];
    if (threadIdx.x == 0) {
        a.out_hist_off[row] = nb;
        if (row == a.B - 1) a.out_hist_off[a.B] = e - h0 + a.B;
        if (nb + (e - b) + 1 > a.out_cap) atomicOr(a.err, FS_DEVERR_HIST_APPEND);
    }
}
__device__ __forceinline__ void decode_commit(const Args& a, const RowCtx& rc, Shared& s, int tok) {
    const int row = rc.row, t = threadIdx.x;
    if (a.out_hist_off && t == 0) {
        const int64_t h0 = a.hist_off ? a.hist_off[0] : 0, b = a.hist_off ? a.hist_off[row] : 0;
        const int64_t e = a.hist_off ? a.hist_off[row + 1] : 0;
        const int64_t at = b - h0 + row + (e - b);
        if (at < a.out_cap) a.out_hist[at] = tok;
    }
    if (!a.dmt || !samples(rc.p)) return;                // uniform; greedy rows draw nothing (sampler.cpp:19-23)
    uint64_t* mt = a.dmt + (int64_t)row * MT_N;
    const int idx = a.didx[row];
    if (idx < MT_N) {
        if (t == 0) a.didx[row] = idx + 1;
        return;
    }
    // the state's twist (the draw was its first value), in LDS: entries k < N - M need old values only, the others
    // the new ones below N - M and their own old neighbour (entry N - 1: the new entry 0)
    uint64_t* w = s.cand;
    __syncthreads();
    if (t < MT_N) w[t] = mt[t];
    __syncthreads();
    uint64_t nv = 0ull;
    if (t < MT_N - MT_M) nv = mt_twist_one(w[t], w[t + 1], w[t + MT_M]);
    __syncthreads();
    if (t < MT_N - MT_M) w[t] = nv;
    __syncthreads();
    if (t >= MT_N - MT_M && t < MT_N) nv = mt_twist_one(w[t], w[(t + 1) % MT_N], w[t - (MT_N - MT_M)]);
    __syncthreads();
    if (t >= MT_N - MT_M && t < MT_N) w[t] = nv;
    __syncthreads();
    if (t < MT_N) mt[t] = w[t];
    if (t == 0) a.didx[row] = 1;
}

__device__ __forceinline__ void merge_row(const Args& a, const RowCtx& rc, Shared& s, const Pre& pre, bool alone = false) {
    const int tid = threadIdx.x;
    const int row = rc.row;
    const int V = a.V;
    const int nseg = rc.nseg;
    const int tail_lo = (V / TILE) * TILE;            // the segment kernel streamed [0, tail_lo)
    const int ntail = V - tail_lo;                    // < TILE logits left for this kernel
    int k = rc.k;
    (void)nseg;
    int tok = 0, keep = 1;

    bool fast = false;
    LargeOut lo;
    lo.valid = false;
    bool whole = rc.large || alone;                   // sampled as a whole row: by the segments together or here
    bool from_segs = false;
    bool cut_done = false;                            // sampled by large_cut: the histograms were never touched
    if (rc.large && !alone && nseg > 0) {
        // the row's segments sampled it together (large_segment): segment 0's slot holds the result unless the row
        // was abandoned (then it is sampled here alone, exactly)
        const uint64_t* s0 = a.cand + slot_of(rc, 0) * CAP;
        const uint32_t sc = *reinterpret_cast<volatile const uint32_t*>(row_sync_ctr(a, row));   // not read before
        if (!(sc & ROW_ABANDONED) && s0[LS_STATUS] != 0ull) {
            cut_done = s0[LS_STATUS] == 2ull;
            const uint64_t tk = s0[LS_TOK];
            tok = (int)(uint32_t)tk;
            keep = (int)(tk >> 32);
            const uint64_t kw = s0[LS_KEFF];
            lo.valid = keep > 0;
            lo.keff = (int)(uint32_t)kw;
            lo.Xk = s0[LS_XK];
            lo.kmax = (uint32_t)(kw >> 32);
            lo.S = __longlong_as_double((long long)s0[LS_S]);
            from_segs = true;
        }
    }
    if (whole) {
        if (!from_segs) large_row(a, rc, s, tok, keep, lo);          // from the logits alone
        if (lo.valid && a.mode != MODE_VERIFY && a.kcap > 0 && (a.cand_ids || a.cand_probs)) {
            if (rc.pen && from_segs) gather_window(a, rc, 0, a.V, s);   // the output passes apply the penalties
            large_outputs(a, rc, s, lo.keff, lo.Xk, comp_key(lo.Xk), lo.kmax, val_of(lo.kmax),
                          (double)rc.p.temperature, lo.S);
        }
    } else if (ntail == 0 && (fast = merge_fast(a, rc, s, pre, tok, keep))) {
        // the short merge wrote the row's outputs
    } else {
    // ---- the row's tail: loads first, then its penalty pass (the same arithmetic as the segment kernel)
    constexpr int TT = TILE / BLOCK;                  // tail logits per thread: element tail_lo + r*BLOCK + tid
    float tx[TT];
    const float* rowp = a.logits + (int64_t)row * a.ld;
#pragma unroll
    for (int r = 0; r < TT; ++r) {
        const int e = tail_lo + r * BLOCK + tid;
        tx[r] = e < V ? rowp[e] : 0.f;
    }
    if (ntail > 0 && rc.capped) softcap_vals(tx, rc.p.softcap);
    if (ntail > 0 && rc.pen) {
        for (int i = tid; i < TILE / 8; i += BLOCK) reinterpret_cast<uint4*>(s.cnt())[i] = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();
        bool ovf = false;
        for (int64_t i = rc.b + tid; i < rc.len; i += BLOCK) {
            const int id = hist_at(a, rc, i);
            const uint32_t rel = (uint32_t)(id - tail_lo);
            if (id >= 0 && id < V && rel < (uint32_t)TILE) {
                const uint32_t sh = (rel & 1u) * 16u;
                const uint32_t old = atomicAdd(&s.cnt()[rel >> 1], 1u << sh);
                ovf |= ((old >> sh) & 0xFFFFu) == 0xFFFFu;
            }
        }
        if (ovf) atomicOr(a.err, FS_DEVERR_COUNT_OVERFLOW);
        __syncthreads();
        const float rp = rc.p.repetition_penalty, fq = rc.p.frequency_penalty, pr = rc.p.presence_penalty;
#pragma unroll
        for (int r = 0; r < TT; ++r) {
            const int rel = r * BLOCK + tid;
            const uint32_t cc = (s.cnt()[rel >> 1] >> ((rel & 1) * 16)) & 0xFFFFu;
            if (cc != 0u && tail_lo + rel < V) {
                float l = tx[r];
                if (rc.rep_on) l = l > 0.0f ? __fdiv_rn(l, rp) : __fmul_rn(l, rp);
                if (rc.fp_on) l = __fsub_rn(l, __fadd_rn(__fmul_rn((float)cc, fq), pr));
                tx[r] = l;
            }
        }
        __syncthreads();
    }

    if (rc.greedy) {
        uint64_t best = (pre.act && pre.r_me == 0) ? pre.v[0] : 0ull;    // each segment's best (entry 0)
#pragma unroll
        for (int r = 0; r < TT; ++r) {                // > -inf, as the segment kernel's IEEE compare from -inf:
            const int e = tail_lo + r * BLOCK + tid;  // NaN and -inf are never taken
            if (e < V && tx[r] > -__builtin_huge_valf()) {
                const uint64_t c = comp_of(key_of(tx[r]), (uint32_t)e);
                best = c > best ? c : best;
            }
        }
        best = block_max_u64(best, s.red);
        tok = best != 0 ? (int)comp_id(best) : 0;      // nothing above -inf / NaN: ferro's scan stays at 0
        const float l0 = rowp[0];
        if (l0 != l0) tok = 0;                         // ferro's scan never moves off a NaN at index 0
        if (tid == 0 && a.mode != MODE_VERIFY) {
            if (a.cand_ids && a.kcap > 0) a.cand_ids[(int64_t)row * a.kcap] = tok;
            if (a.cand_probs && a.kcap > 0) a.cand_probs[(int64_t)row * a.kcap] = 1.0;
        }
    } else {
        // ---- fast path: no tail, every list inside its prefetched window, k <= 64. L (the largest list bound)
        // comes from a wave reduction over the lists' bounds; T1 from a histogram of the prefetched registers over
        // [L, max]; the <= 128 candidates reaching T1 are ranked and finished by wave 0. Any other shape (or more
        // than 128 candidates at T1) takes the general path below.
        bool fast_done = false;
        if (ntail == 0 && k <= WAVE && nseg <= FAST_SEGS) {
            // every wave holds every list's (bound, count) pair (lane l: list l % nseg): no barrier
            const uint32_t L = wave_max(pre.t0m);
            const uint32_t cmax = wave_max(pre.cnm);
            if (cmax <= (uint32_t)(SPEC * pre.tps)) {
                for (int i = tid; i < NBINS; i += BLOCK) s.bins()[i] = 0u;
                if (tid == 0) { s.count = 0u; s.nids = 0u; }
                __syncthreads();
                // every candidate >= L into the candidate buffer (<= SPEC * BLOCK of them), tracking the max key
                uint32_t kmax = L;
#pragma unroll
                for (int q = 0; q < SPEC; ++q) {
                    const uint64_t w = pre.v[q];
                    const bool in = pre.act && (uint32_t)(pre.r_me + q * pre.tps) < pre.cnm && w != 0 && comp_key(w) >= L;
                    if (in) kmax = comp_key(w) > kmax ? comp_key(w) : kmax;
                    wave_append(in, w, s.cand, &s.count, CAP);
                }
                kmax = block_max_u32(kmax, s.red);            // its barrier also completes the appends
                const uint32_t n = s.count;
                uint64_t* list = s.cand;
                uint32_t c1 = n;
                if (n > (uint32_t)(2 * WAVE)) {
                    // more than 128: T1 from a histogram of the list over [L, kmax], then the <= 128 >= T1
                    const int sh = range_shift(L, kmax);
                    for (uint32_t i = tid; i < n; i += BLOCK) atomicAdd(&s.bins()[(comp_key(s.cand[i]) - L) >> sh], 1u);
                    __syncthreads();
                    const uint32_t T1 = hist_threshold(s.bins(), L, sh, k, &c1, s.wsum, s.red);
                    if (c1 >= (uint32_t)k && c1 <= (uint32_t)(2 * WAVE)) {
                        list = s.cand + SPEC * BLOCK;         // past the full list
                        for (uint32_t i0 = 0; i0 < n; i0 += BLOCK) {
                            const uint32_t i = i0 + tid;
                            const uint64_t c = i < n ? s.cand[i] : 0ull;
                            wave_append(c != 0 && comp_key(c) >= T1, c, list, &s.nids, 2 * WAVE);
                        }
                        __syncthreads();
                    }
                }
                if (c1 >= (uint32_t)k && c1 <= (uint32_t)(2 * WAVE)) {
                    uint64_t* small_out = list + SMALL;
                    uint32_t* rk = reinterpret_cast<uint32_t*>(small_out + 2 * WAVE);   // past wave_finish's buffers
                    block_ranks(list, (int)c1, rk);
                    if (tid < WAVE) wave_finish(a, rc, list, rk, k, pre.u, reinterpret_cast<double*>(small_out), tok, keep);
                    fast_done = true;
                }
            }
        }
        if (!fast_done) {
        // ---- the tail's own top k becomes one more list, kept in LDS at the top of the candidate buffer
        // (tl[0, nt); ttkey bounds the k-th key if the tail holds at least k candidates); the gather below then
        // fills at most gcap entries
        uint64_t* tl = s.cand + (CAP - KMAX);
        const uint32_t gcap = ntail > 0 ? (uint32_t)(CAP - KMAX) : (uint32_t)CAP;
        int nt = 0;
        uint32_t ttkey = 0u;
        if (ntail > 0) {
            if (tid == 0) s.count = 0u;
            __syncthreads();
#pragma unroll
            for (int r = 0; r < TT; ++r) {
                const int e = tail_lo + r * BLOCK + tid;
                const bool in = e < V && tx[r] == tx[r];
                wave_append(in, in ? comp_of(key_of(tx[r]), (uint32_t)e) : 0ull, s.cand, &s.count, CAP);
            }
            __syncthreads();
            nt = (int)s.count;
            if (nt > k) {
                ttkey = comp_key(compact_exact(nt, k, s));
                nt = k;
            }
            for (int i = tid; i < nt; i += BLOCK) tl[i] = s.cand[i];   // nt <= KMAX: no overlap
            __syncthreads();
        }
        // The segment lists (prefetched at kernel entry) and the tail list: L = the largest of their k-th key
        // bounds bounds the row's k-th key from below.
        const int tps = pre.tps, c_me = pre.c_me, r_me = pre.r_me;
        const bool act = pre.act;
        const uint32_t cnm = pre.cnm;
        const uint64_t* lst = a.cand + slot_of(rc, c_me) * CAP;
        if (act && r_me == 0) s.off[c_me] = cnm;
        if (tid == 0) s.count = 0u;
        // one reduction: L (bit 63 set when a list is longer than its prefetched window, or the lists' total may
        // overflow LDS: then the flat offsets below are needed)
        const bool longl = act && r_me == 0 && cnm > (uint32_t)(SPEC * tps);
        const uint64_t red = block_max_u64(((uint64_t)(longl ? 1u : 0u) << 63) | (act ? pre.t0m : 0u), s.red);
        uint32_t L = (uint32_t)red;
        L = ttkey > L ? ttkey : L;
        const bool need_off = (red >> 63) != 0ull || (uint32_t)nseg * (uint32_t)(SPEC * tps) + (uint32_t)nt > (uint32_t)CAP;
        // flat offsets of the segment lists (used when the candidates >= L overflow LDS)
        uint32_t total = 0u;
        if (need_off) {
            const uint32_t mine = tid < nseg ? s.off[tid] : 0u;
            const uint32_t o = block_excl_scan<uint32_t>(mine, s.wsum, &total);
            if (tid < nseg) s.off[tid] = o;
            if (tid == 0) s.off[nseg] = total;
            __syncthreads();
        }
        auto fetch = [&](uint32_t f) -> uint64_t {          // flat index -> candidate (0 past the end)
            const uint32_t g = f < total ? f : total - 1u;  // branch-free: the load is always issued in bounds
            int c0 = 0, c1 = nseg;                           // largest c with off[c] <= g
            while (c1 - c0 > 1) {
                const int m = (c0 + c1) >> 1;
                if (s.off[m] <= g) c0 = m; else c1 = m;
            }
            const uint64_t w = a.cand[slot_of(rc, c0) * CAP + (g - s.off[c0])];
            return f < total ? w : 0ull;
        };
        // gather the candidates >= L into LDS (counted past CAP), tracking their max key
        uint32_t kmax = L;
        for (int i0 = 0; i0 < nt; i0 += BLOCK) {
            const int i = i0 + tid;
            const uint64_t w = i < nt ? tl[i] : 0ull;
            const bool in = w != 0 && comp_key(w) >= L;
            if (in) kmax = comp_key(w) > kmax ? comp_key(w) : kmax;
            wave_append(in, w, s.cand, &s.count, gcap);
        }
        {                                           // the prefetched entries: one LDS atomic per wave
            uint64_t bal[SPEC];
            uint32_t tot = 0u;
#pragma unroll
            for (int q = 0; q < SPEC; ++q) {
                const uint64_t w = pre.v[q];
                const bool in = act && (uint32_t)(r_me + q * tps) < cnm && w != 0 && comp_key(w) >= L;
                if (in) kmax = comp_key(w) > kmax ? comp_key(w) : kmax;
                bal[q] = __ballot(in);
                tot += (uint32_t)__popcll(bal[q]);
            }
            if (tot != 0u) {
                uint32_t base = 0u;
                if (lane_id() == 0) base = atomicAdd(&s.count, tot);
                base = (uint32_t)__builtin_amdgcn_readlane((int)base, 0);
#pragma unroll
                for (int q = 0; q < SPEC; ++q) {
                    if ((bal[q] >> lane_id()) & 1ull) {
                        const uint32_t pos = base + mbcnt(bal[q]);
                        if (pos < gcap) s.cand[pos] = pre.v[q];
                    }
                    base += (uint32_t)__popcll(bal[q]);
                }
            }
        }
        // long lists: the entries past the prefetched window, LL loads in flight per thread and round (a list of
        // k ~ 2048 entries then costs one or two L2 round trips instead of one per tps entries)
        constexpr int LL = 8;
        for (uint32_t i0 = (uint32_t)(r_me + SPEC * tps); act && i0 < cnm; i0 += (uint32_t)(LL * tps)) {
            uint64_t w[LL];
#pragma unroll
            for (int q = 0; q < LL; ++q) {
                const uint32_t i = i0 + (uint32_t)(q * tps);
                w[q] = i < cnm ? lst[i] : 0ull;
            }
#pragma unroll
            for (int q = 0; q < LL; ++q) {
                const bool in = w[q] != 0 && comp_key(w[q]) >= L;
                if (in) kmax = comp_key(w[q]) > kmax ? comp_key(w[q]) : kmax;
                wave_append(in, w[q], s.cand, &s.count, gcap);
            }
        }
        for (int i = tid; i < NBINS; i += BLOCK) s.bins()[i] = 0u;
        uint32_t kmin = L;
        block_minmax_u32(kmin, kmax, s.red);
        FS_MARK(5);                                 // general merge: candidates >= L gathered
        const uint32_t n = s.count;
        const bool in_lds = n <= gcap;
        // T1: tight threshold from a histogram of the candidates' keys over [L, kmax]
        const int sh = range_shift(L, kmax);
        if (in_lds) {
            for (uint32_t i = tid; i < n; i += BLOCK) atomicAdd(&s.bins()[(comp_key(s.cand[i]) - L) >> sh], 1u);
        } else {
            for (uint32_t f = tid; f < total; f += BLOCK) {
                const uint64_t c = fetch(f);
                if (c != 0 && comp_key(c) >= L) atomicAdd(&s.bins()[(comp_key(c) - L) >> sh], 1u);
            }
            for (int i = tid; i < nt; i += BLOCK) {
                const uint64_t c = tl[i];
                if (comp_key(c) >= L) atomicAdd(&s.bins()[(comp_key(c) - L) >> sh], 1u);
            }
        }
        __syncthreads();
        uint32_t c1;
        const uint32_t T1 = hist_threshold(s.bins(), L, sh, k, &c1, s.wsum, s.red);
        FS_MARK(6);                                 // T1 known
        FS_TAG(9, c1); FS_TAG(10, n); FS_TAG(11, in_lds ? 1 : 0);
        if (c1 < (uint32_t)k) {
            // Fewer than k candidates: with L = 0 (no bound above NaN's key) every number of the row is a candidate,
            // so the row holds fewer than k numbers and samples over them (NaN is never a candidate); with L > 0 the
            // bounds promised k, an invariant failure. Never read past the list.
            if (tid == 0 && L != 0u) atomicOr(a.err, FS_DEVERR_INTERNAL);
            k = (int)c1;
        }
        // the c1 >= k candidates with key >= T1 contain the top k: sort them
        uint64_t* top;
        bool wave_done = false;                   // wave 0 finished the row (k <= 64, c1 <= 128)
        uint64_t* small_in = reinterpret_cast<uint64_t*>(s.bins());
        uint64_t* small_out = small_in + SMALL;
        if (tid == 0) s.count = 0u;
        __syncthreads();
        if (c1 <= (uint32_t)SMALL) {
            if (in_lds) {
                for (uint32_t i0 = 0; i0 < n; i0 += BLOCK) {
                    const uint32_t i = i0 + tid;
                    const uint64_t c = i < n ? s.cand[i] : 0ull;
                    wave_append(c != 0 && comp_key(c) >= T1, c, small_in, &s.count, SMALL);
                }
            } else {
                for (uint32_t f0 = 0; f0 < total; f0 += BLOCK) {
                    const uint64_t c = fetch(f0 + tid);
                    wave_append(c != 0 && comp_key(c) >= T1, c, small_in, &s.count, SMALL);
                }
                for (int i0 = 0; i0 < nt; i0 += BLOCK) {
                    const uint64_t c = i0 + tid < nt ? tl[i0 + tid] : 0ull;
                    wave_append(c != 0 && comp_key(c) >= T1, c, small_in, &s.count, SMALL);
                }
            }
            __syncthreads();
            if (c1 <= (uint32_t)(2 * WAVE) && k <= WAVE && k > 0) {
                uint32_t* rk = reinterpret_cast<uint32_t*>(small_out + 2 * WAVE);   // past wave_finish's buffers
                block_ranks(small_in, (int)c1, rk);
                if (tid < WAVE) wave_finish(a, rc, small_in, rk, k, pre.u, reinterpret_cast<double*>(small_out), tok, keep);
                wave_done = true;
            } else if (c1 <= (uint32_t)(4 * WAVE)) {
                rank_sort(small_in, (int)c1, small_out, k);
            } else {
                // the gathered list is spent: its buffer takes the scatter; counts and starts in cnt()
                static_assert(2 * (NBINS / 2) <= TILE / 2, "two half-size bin arrays in cnt()");
                bin_sort_desc<NBINS / 2>(small_in, (int)c1, s.cand, s.cnt(), s.cnt() + NBINS / 2, s.red, s.wsum);
            }
            top = !wave_done && c1 > (uint32_t)(4 * WAVE) ? small_in : small_out;   // binned sort: in place
        } else {
            // more than SMALL candidates reach T1: reduce to exactly the k >= X in LDS, then sort those
            int m = (int)n;
            if (!in_lds) {
                uint64_t X = 0;                         // threshold for a gather of <= CAP entries
                if (c1 > gcap) {
                    X = radix_kth(
                        [&](auto&& f) {
                            for (uint32_t f0 = tid; f0 < total; f0 += BLOCK) {
                                const uint64_t c = fetch(f0);
                                f(c != 0 && comp_key(c) >= L ? c : 0ull);
                            }
                            for (int i = tid; i < nt; i += BLOCK) f(comp_key(tl[i]) >= L ? tl[i] : 0ull);
                        },
                        k, s.bins(), s.wsum, s.red);
                }
                if (tid == 0) s.count = 0u;
                __syncthreads();
                for (uint32_t f0 = 0; f0 < total; f0 += BLOCK) {
                    const uint64_t c = fetch(f0 + tid);
                    wave_append(c != 0 && comp_key(c) >= T1 && c >= X, c, s.cand, &s.count, gcap);
                }
                for (int i0 = 0; i0 < nt; i0 += BLOCK) {
                    const uint64_t c = i0 + tid < nt ? tl[i0 + tid] : 0ull;
                    wave_append(c != 0 && comp_key(c) >= T1 && c >= X, c, s.cand, &s.count, gcap);
                }
                __syncthreads();
                m = (int)s.count;
            }
            if (in_lds) {                               // the c1 >= k entries at or above T1 hold the top k
                const int mt = keep_from(m, (uint64_t)T1 << 32, s);
                if (mt >= 0) m = mt;
            }
            if (m > KMAX) {                             // else the counting sort orders all m; the first k are used
                compact_exact(m, k, s);
                m = k;
            }
            const uint32_t big = bin_sort_desc(m, s);
            FS_TAG(12, big);
            (void)big;
            top = s.cand;
            c1 = (uint32_t)m;
        }
        FS_MARK(7);                                 // the top candidates sorted
        if (!wave_done) {
            if (c1 < (uint32_t)k) {                       // c1 >= k after the clamp above; never read past the list
                if (tid == 0) atomicOr(a.err, FS_DEVERR_INTERNAL);
                k = (int)c1;
            }
            if (k == 0) {                                 // every logit NaN: token 0, nothing kept
                tok = 0;
                keep = 0;
            } else {

            // ---- softmax at temperature, min-p, top-p, draw (sampler.cpp:37-49), k <= KMAX
            const fs_row_params& p = rc.p;
            const int i0 = tid * KPT;
            const float mx = val_of(comp_key(top[0]));
            const double Td = (double)p.temperature;
            double e[KPT];
            double part = 0.0;
#pragma unroll
            for (int q = 0; q < KPT; ++q) {
                const int i = i0 + q;
                e[q] = 0.0;
                if (i < k) {
                    const float d = val_of(comp_key(top[i])) - mx;   // fp32 subtraction, as ferro
                    e[q] = exp((double)d / Td);
                    part += e[q];
                }
            }
            const double sum = block_sum_f64(part, s.red);
            FS_MARK(8);                                 // exp and their sum
            double pr[KPT];
#pragma unroll
            for (int q = 0; q < KPT; ++q) pr[q] = e[q] / sum;
            // min-p: keep = 1 + the last index not below pr[0]*min_p (NaN masses stay) (at least 1)
            int keep_m = k;
            if (p.min_p > 0.0f) {
                const double thr = (1.0 / sum) * (double)p.min_p;
                int last = -1;
#pragma unroll
                for (int q = 0; q < KPT; ++q)
                    if (i0 + q < k && !(pr[q] < thr)) last = i0 + q;
                last = block_max_i32(last, s.red);
                keep_m = last + 1 > 1 ? last + 1 : 1;
            }
            // inclusive prefix of pr in candidate order
            double c[KPT];
            double run = 0.0;
#pragma unroll
            for (int q = 0; q < KPT; ++q) { run += pr[q]; c[q] = run; }
            double tot_all;
            const double off = block_excl_scan<double>(run, s.red.f64, &tot_all);
#pragma unroll
            for (int q = 0; q < KPT; ++q) c[q] += off;
            keep = keep_m;
            if (p.top_p < 1.0f) {
                int first = 0x7fffffff;
#pragma unroll
                for (int q = 0; q < KPT; ++q)
                    if (i0 + q < keep_m && c[q] >= (double)p.top_p && first == 0x7fffffff) first = i0 + q;
                first = block_min_i32(first, s.red);
                if (first != 0x7fffffff) keep = first + 1 < keep_m ? first + 1 : keep_m;
                if (keep < 1) keep = 1;
            }
            // tot = sum of the kept prefix; r = u * tot; the first i with r <= c_i
#pragma unroll
            for (int q = 0; q < KPT; ++q)
                if (i0 + q == keep - 1) s.red.dmisc[0] = c[q];
            __syncthreads();
            const double tot = s.red.dmisc[0];
            const double u = pre.u;
            const double rr = u * tot + 0.0;
            int hit = 0x7fffffff;
#pragma unroll
            for (int q = 0; q < KPT; ++q)
                if (i0 + q < keep && rr <= c[q] && hit == 0x7fffffff) hit = i0 + q;
            hit = block_min_i32(hit, s.red);
            const int pos = hit == 0x7fffffff ? keep - 1 : hit;
            tok = (int)comp_id(top[pos]);
            if (a.mode != MODE_VERIFY) {
                const int m = k < a.kcap ? k : a.kcap;
                if (a.cand_ids)
                    for (int i = tid; i < m; i += BLOCK) a.cand_ids[(int64_t)row * a.kcap + i] = (int32_t)comp_id(top[i]);
                if (a.cand_probs) {
#pragma unroll
                    for (int q = 0; q < KPT; ++q)
                        if (i0 + q < m) a.cand_probs[(int64_t)row * a.kcap + i0 + q] = pr[q];
                }
            }
            }                                             // k > 0
        }
        }                                             // general path
    }
    }
    if (!rc.greedy && nseg > 0 && !alone) {           // the segments' row histogram is spent: leave it at 0
        uint4* rz = reinterpret_cast<uint4*>(a.rhist + (int64_t)row * RBINS);
        for (int i = cut_done ? RBINS / 4 - 1 + tid : tid; i < RBINS / 4; i += BLOCK)   // (large_cut: the counters)
            rz[i] = make_uint4(0u, 0u, 0u, 0u);
        if (rc.large && !cut_done) {                   // and a large row's mass histogram
            uint4* mz = reinterpret_cast<uint4*>(a.rmass + (int64_t)row * LB);
            for (int i = tid; i < LB / 2; i += BLOCK) mz[i] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    if (a.out_hist_off || a.dmt) decode_commit(a, rc, s, tok);   // uniform (a decode step)
    if (a.mode != MODE_VERIFY) {
        if (tid == 0) {
            a.tok[row] = tok;
            if (a.keep) a.keep[row] = keep;
        }
    } else if (tid < WAVE) {
        // verify: the last row of a stream to finish computes the accepted prefix (server.cpp:627-637), wave 0.
        // Streams of up to 32 rows: one 64-bit atomic per row (the count of rows done, and a bit for each row that
        // ends the walk), the last row's fetched value gives the prefix; longer ones: tokens at agent scope, a row
        // counter after the 64-bit words, and the walk.
        const int st = rc.pidx;
        const int64_t r0 = a.row_off[st];
        const int m = (int)(a.row_off[st + 1] - r0);
        if (m <= 32) {
            if (tid == 0) {
                a.tok[row] = tok;
                const int rr = row - (int)r0;
                const bool stop = (a.eos >= 0 && tok == a.eos) || rr + 1 >= m || tok != a.rows[row + 1];
                const uint64_t mine = stop ? (1ull << rr) : 0ull;
                uint64_t* cnt = reinterpret_cast<uint64_t*>(a.stream_cnt) + st;
                const uint64_t old = __hip_atomic_fetch_add(cnt, (1ull << 32) | mine, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT);
                if ((uint32_t)(old >> 32) == (uint32_t)m - 1u) {
                    __hip_atomic_store(cnt, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    a.accepted[st] = __ffs((int)((uint32_t)old | (uint32_t)mine));
                }
            }
        } else {
            uint32_t* cnt32 = a.stream_cnt + 2 * (int64_t)a.n_streams + st;
            uint32_t old = 0u;
            if (tid == 0) {
                st_agent(&a.tok[row], (int32_t)tok);
                vm_drain();
                old = __hip_atomic_fetch_add(cnt32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (read_lane(old, 0) == (uint32_t)m - 1u) {
                if (tid == 0) st_agent(cnt32, 0u);
                const int acc = accepted_prefix(a.tok, a.rows, r0, m, a.eos);
                if (tid == 0) a.accepted[st] = acc;
            }
        }
    }
    __syncthreads();                                   // LDS is reused by the caller's next chunk
}

// A wave's snapshot of its row's histogram: lane l holds the counts of bins b0 + 4 (63 - l) + j, j = 0..3, where
// b0 is the wave's current bound's bin rounded down to a multiple of 4: the 256 bins (32 binades) from the bound
// up, in lane order = descending bins; counts above the window are left out (fewer counts: the bound stays
// valid).
// The row histogram lives in the L2 of the XCD that runs the row's segments (the grid places them there): counts
// are L2 atomics and snapshots are group-scope loads, served by that L2 or by a line the CU's L1 still holds from
// an earlier snapshot (older counts). Every access is an increment of zeroed memory or a read, so a read returns
// at most the row's true counts - stale, or with a segment on another XCD missing - and every bound stays valid.
struct RowSnap {
    uint64_t w[2];
    uint32_t b0;
};
// Through a buffer resource over the row histogram. With 0 records the load returns zeros without a memory access,
// so the tile loop can request it unconditionally (straight-line loads keep the compiler's memory-counter waits
// exact).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ u32x4 raw_buffer_load_u32x4(__amdgpu_buffer_rsrc_t rs, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.load.v4i32");
__device__ uint32_t raw_buffer_load_u32(__amdgpu_buffer_rsrc_t rs, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.ptr.buffer.load.i32");
constexpr int AUX_SC0 = 1;               // cache policy sc0: group scope (the CU's L1, else the XCD's L2)
__device__ __forceinline__ RowSnap row_snap(__amdgpu_buffer_rsrc_t rs, uint32_t tkey) {
    RowSnap r;
    r.b0 = (tkey >> RSHIFT) & ~3u;
    const uint32_t first = r.b0 + 4u * (uint32_t)(WAVE - 1 - lane_id());
    const uint32_t f = first <= (uint32_t)RBINS - 4u ? first : (uint32_t)RBINS - 4u;   // past the top: ignored
    const u32x4 v = raw_buffer_load_u32x4(rs, (int)(f * 4u), 0, AUX_SC0);
    r.w[0] = (uint64_t)v.x | ((uint64_t)v.y << 32);
    r.w[1] = (uint64_t)v.z | ((uint64_t)v.w << 32);
    return r;
}
// From a snapshot: the lower edge of the highest bin with at least k counted logits in it and the bins above. At
// least k logits of the row reach it, so it bounds the row's k-th key from below (0: the snapshot holds fewer than
// k). No barrier: each wave takes its own snapshot, and any snapshot gives a valid bound.
__device__ __forceinline__ uint32_t row_bound(const RowSnap& r, int k) {
    const int lane = lane_id();
    const uint32_t first = r.b0 + 4u * (uint32_t)(WAVE - 1 - lane);
    const bool valid = first <= (uint32_t)RBINS - 4u;
    const uint32_t c0 = valid ? (uint32_t)r.w[0] : 0u, c1 = valid ? (uint32_t)(r.w[0] >> 32) : 0u;
    const uint32_t c2 = valid ? (uint32_t)r.w[1] : 0u, c3 = valid ? (uint32_t)(r.w[1] >> 32) : 0u;
    const uint32_t mine = c0 + c1 + c2 + c3;
    const uint32_t cum = wave_incl_scan_u32(mine);
    const uint32_t ex = cum - mine;
    const bool hit = ex < (uint32_t)k && cum >= (uint32_t)k;
    const uint32_t a3 = ex + c3, a2 = a3 + c2, a1 = a2 + c1;
    const uint32_t bin = first + (a3 >= (uint32_t)k ? 3u : a2 >= (uint32_t)k ? 2u : a1 >= (uint32_t)k ? 1u : 0u);
    const uint64_t hb = __ballot(hit);
    if (hb == 0ull) return 0u;
    return (uint32_t)__builtin_amdgcn_readlane((int)bin, __ffsll((unsigned long long)hb) - 1) << RSHIFT;
}

// The first PF tiles of a segment, requested from the kernel arguments alone (before the row's parameters arrive).
struct SegStart {
    int seg_lo, ntiles;
    const float* rowp;
    __amdgpu_buffer_rsrc_t rs;   // [seg_lo, seg_lo + ntiles * TILE) of the row
};
// spec: the balanced layout may still move this workgroup, and its loads are then overwritten before use. They are
// marked volatile (aux bit 31) so that the compiler keeps them at kernel entry instead of sinking them past the layout.
template <bool SPEC = false>
__device__ __forceinline__ SegStart seg_start(const Args& a, int row, int seg, int st, float (&buf)[PF][TPT]) {
    SegStart g;
    g.seg_lo = seg * st * TILE;
    const int left = a.V / TILE - seg * st;                         // full tiles left in the row
    g.ntiles = left < st ? left : st;                               // >= 1
    g.rowp = a.logits + (int64_t)row * a.ld;
    g.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g.rowp + g.seg_lo), (short)0, g.ntiles * TILE * 4,
                                             0x00020000);
#pragma unroll
    for (int p = 0; p < PF; ++p) load_seg_tile<SPEC ? (int)0x80000000 : 0>(buf[p], g.rs, p);
    return g;
}

// One (row, segment) item: stream the segment's full tiles with PF tiles in flight, apply the penalties, and keep
// the running candidates.
//   - greedy rows: each lane's first maximum;
//   - top-k rows: every logit with key >= tkey, a lower bound of the row's k-th key (at least k logits of the row
//     reach it). tkey starts from tile 0 (the highest coarse bin with >= k of the tile's lane maxima at or above
//     it) and is raised from the row histogram (a.rhist): the segments add counts of real logits to their row's
//     coarse bins (tile 0's lane maxima, then the buffered logits of tiles 1-4), and every wave snapshots the
//     counts and takes the highest bin with >= k counted logits at or above it. Counts only grow, so any snapshot
//     gives a valid bound, and the bound combines the whole row's evidence instead of one segment's.
// The segment publishes its candidates with key >= the final tkey (plain stores; the merge kernel runs after this
// kernel). They include every logit of the row's top k that lies in this segment.
__device__ __forceinline__ void process_segment(const Args& a, const RowCtx& rc, int seg, Shared& s,
                                                float (&buf)[PF][TPT], const SegStart& g) {
    const int tid = threadIdx.x;
    const int seg_lo = g.seg_lo;
    const int ntiles = g.ntiles;

    // the window ids (their loads return after the first tiles': the bitmap below waits for those anyway)
    constexpr int WPF = 2;
    int wid[WPF];
#pragma unroll
    for (int q = 0; q < WPF; ++q) {
        const int64_t i = rc.b + q * BLOCK + tid;
        wid[q] = (rc.pen && i < rc.len) ? hist_at(a, rc, i) : -1;
    }
    // Tile 0 is staged in the candidate buffer's tail (tile 0's own appends, at most one tile, stay below it) and
    // tile PF requested in its registers as soon as tile 0 arrives: tile 0's bound computation (two barriers) and
    // appends then run with PF tiles in flight. (Staging it before the penalty set-up, so that tile PF is requested
    // earlier still, measured slower: +1.1 us on a B=64 x V=262144 top-k 64 batch, +1.5 us on a mixed B=256 one.)
    float4* const stage0 = reinterpret_cast<float4*>(s.cand + (CAP - TILE / 2));
    static_assert(TILE + TILE / 2 <= CAP, "tile 0's appends stay below its stage");
    auto stage_tile0 = [&]() {
#pragma unroll
        for (int j = 0; j < NV; ++j)
            stage0[j * BLOCK + tid] = make_float4(buf[0][4 * j], buf[0][4 * j + 1], buf[0][4 * j + 2], buf[0][4 * j + 3]);
        load_seg_tile(buf[0], g.rs, PF);
    };
    // Penalties. With a repetition penalty alone (sampler.cpp:11-18) only membership in the window matters: an
    // exact bitmap of the segment's window ids (bmp, in the merge's offset array, unused by this kernel) is built
    // once, and a thread's four consecutive logits share one bitmap word, so each tile costs two LDS reads and no
    // barrier. Frequency / presence penalties need counts: the segment's window ids bucketed by tile once, then
    // counted wave by wave (wave_penalties; segments of >= 4 tiles), else a per-tile count table (apply_penalties).
    const int seg_hi = seg_lo + ntiles * TILE;
    const bool fastpen = rc.pen && rc.rep_on && !rc.fp_on && seg_hi - seg_lo <= 32 * (MAX_SEGS + 1);
    const bool slowpen = rc.pen && !fastpen;
    uint32_t* bmp = s.off;
    const float rp = rc.p.repetition_penalty;
    if (slowpen) gather_window(a, rc, seg_lo, seg_hi, s);
    // counts (frequency / presence): the window's ids bucketed by tile once, then counted per wave (no barriers);
    // a window with more than WIDS ids in the segment keeps the per-tile table (apply_penalties)
    const bool wavepen = slowpen && s.nids <= (uint32_t)WIDS && ntiles >= 4 && ntiles <= 2 * BLOCK;
    const bool tablepen = slowpen && !wavepen;
    if (wavepen) bucket_window(seg_lo, ntiles, s);
    if (fastpen) {
        for (int i = tid; i <= MAX_SEGS; i += BLOCK) bmp[i] = 0u;
        __syncthreads();
        auto mark = [&](int id) {
            const uint32_t rel = (uint32_t)(id - seg_lo);
            if (id >= seg_lo && id < seg_hi) atomicOr(&bmp[rel >> 5], 1u << (rel & 31u));
        };
#pragma unroll
        for (int q = 0; q < WPF; ++q) mark(wid[q]);
        for (int64_t i = rc.b + WPF * BLOCK + tid; i < rc.len; i += BLOCK) mark(hist_at(a, rc, i));
        __syncthreads();
    }
    auto bitmap_pen = [&](float (&x)[TPT], int lo) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint32_t rel = (uint32_t)(lo - seg_lo) + (uint32_t)(j * BLOCK + tid) * 4u;
            const uint32_t nib = (bmp[rel >> 5] >> (rel & 31u)) & 0xFu;
            if (nib != 0u) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float l = x[4 * j + q];
                    if ((nib >> q) & 1u) x[4 * j + q] = l > 0.0f ? __fdiv_rn(l, rp) : __fmul_rn(l, rp);
                }
            }
        }
    };

    const int k = rc.k;
    const bool topk = !rc.greedy;      // large rows never reach this function
    float bv = -__builtin_huge_valf(); // greedy: this lane's first maximum (IEEE >: NaN never taken, -0 == +0)
    int bs = -1;                       //         and its slot tile*TPT + i (-1: none)
    uint32_t tkey = 0u;                // top-k: candidates are the logits with key >= tkey
    float tf = -__builtin_huge_valf(); //         in fp32: x >= tf (NaN never passes)
    uint32_t* rh = a.rhist + (int64_t)rc.row * RBINS;
    const __amdgpu_buffer_rsrc_t rsr = __builtin_amdgcn_make_buffer_rsrc(rh, (short)0, RBINS * 4, 0x00020000);
    // Row bounds from the row histogram. Segments of >= 3 tiles: each wave snapshots it after tile 0 and takes the
    // bound before appending tile 1; segments of >= 5 tiles snapshot again at tile 3 and take at tile 4, within one
    // iteration of the tile loop (no load outstanding across its back edge).
    // Shorter segments: one block-wide read at tile 0 (thread t holds bin b0 + BLOCK-1-t), taken after the loop.
    uint32_t scnt = 0u, sb0 = 0u;
    uint32_t rc0 = 0u;                 // lowest coarse bin of the tile-0 counts
    bool spending = false;
    if (tid == 0) { s.count = 0u; s.tmax = 0u; }
    if (tid < WAVE) s.rc64[tid] = 0u;
    __syncthreads();

    auto raise_key = [&](uint32_t kq) {
        if (kq > tkey) {
            tkey = kq;
            tf = kq > 0x007FFFFFu ? val_of(kq) : -__builtin_huge_valf();   // keys below -inf's are NaN patterns
        }
    };
    auto row_read = [&](uint32_t b0) -> uint32_t {
        const uint32_t b = b0 + (uint32_t)(BLOCK - 1 - tid);
        return raw_buffer_load_u32(rsr, (int)(4u * (b < (uint32_t)RBINS ? b : (uint32_t)RBINS - 1u)), 0, AUX_SC0);
    };
    // the highest bin b (>= rb0) with at least k counted logits in bins [b, rb0 + BLOCK - 1]: a row-wide bound
    auto row_take = [&](uint32_t rb0, uint32_t rcnt) {
        const uint32_t c = rb0 + (uint32_t)(BLOCK - 1 - tid) < (uint32_t)RBINS ? rcnt : 0u;
        uint32_t tot;
        const uint32_t above = block_excl_scan<uint32_t>(c, s.wsum, &tot);   // thread order = descending bins
        const int hit = (c != 0u && above + c >= (uint32_t)k) ? tid : BLOCK;
        const int first = block_min_i32(hit, s.red);
        if (first < BLOCK) raise_key((rb0 + (uint32_t)(BLOCK - 1 - first)) << RSHIFT);
    };
    // Top-k buffer discipline: after tile 0 the buffer is checked (barrier) every R tiles, R sized so the expected
    // appends fill at most half the headroom, and rows with k > 64 also at every iteration's first tile, where their
    // new entries are counted into the row histogram (the other segments' bounds tighten sooner: fewer appends row
    // wide); an overflow (appends past CAP are dropped) is detected at the next check and the segment is streamed
    // again in safe mode (a check after every tile).
    auto greedy_update = [&](const float (&x)[TPT], int tt) {
        const int sb = tt * TPT;
#pragma unroll
        for (int i = 0; i < TPT; ++i)
            if (x[i] > bv) { bv = x[i]; bs = sb + i; }
    };
    // appends of one tile: one fp32 compare per logit folded into a wave ballot; composites, LDS slots and row
    // counts are formed only where some lane passed
    auto topk_append = [&](const float (&x)[TPT], int lo) {
        uint64_t bal[TPT];
        uint64_t any = 0ull;
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            bal[i] = __ballot(x[i] >= tf);
            any |= bal[i];
        }
        if (any == 0ull) return;                     // wave-uniform
        const int lane = lane_id();
        uint32_t tot = 0u;
#pragma unroll
        for (int i = 0; i < TPT; ++i) tot += (uint32_t)__popcll(bal[i]);
        uint32_t base = 0u;
        if (lane == 0) base = atomicAdd(&s.count, tot);
        base = (uint32_t)__builtin_amdgcn_readlane((int)base, 0);
#pragma unroll
        for (int i = 0; i < TPT; ++i) {
            if (bal[i] != 0ull) {
                if ((bal[i] >> lane) & 1ull) {
                    const uint32_t kq = key_of(x[i]);
                    const uint32_t pos = base + mbcnt(bal[i]);
                    if (pos < (uint32_t)CAP) s.cand[pos] = comp_of(kq, (uint32_t)elem_id(lo, i));
                }
                base += (uint32_t)__popcll(bal[i]);
            }
        }
    };
    int counted = 0;                   // buffer entries [0, counted) are in the row histogram or never will be
    // Adds the buffered logits [from, count) of tiles >= 1 with key >= tkey to the row histogram, at their coarse
    // bins from tkey's (higher ones at the 64th: fewer counts, bounds stay valid). Tile 0 is counted already. The
    // waves' tkeys can differ (each wave takes its own row bounds), so each wave histograms the entries it reads
    // relative to its own tkey in its own 64 bins (in bins(), free between checks) and adds them to the row at
    // that base; a wave's LDS accesses complete in order, so no barrier is needed.
    // Entry: nb = the buffer's count, read by every wave after a barrier that followed the last append and before
    // any wave appends again; the next check's barrier ends the bins' use.
    auto count_row = [&](int from, int nb) {
        const uint32_t rb = tkey >> RSHIFT;
        uint32_t* wb = s.bins() + (tid / WAVE) * WAVE;
        wb[lane_id()] = 0u;
        if (nb <= CAP) {
            for (int i = from + tid; i < nb; i += BLOCK) {
                const uint64_t c = s.cand[i];
                if (comp_id(c) >= (uint32_t)(seg_lo + TILE) && comp_key(c) >= tkey) {
                    const uint32_t d = (comp_key(c) >> RSHIFT) - rb;
                    atomicAdd(&wb[d < (uint32_t)WAVE ? d : (uint32_t)WAVE - 1u], 1u);
                }
            }
        }
        const uint32_t c = wb[lane_id()];
        if (c != 0u && rb + (uint32_t)lane_id() < (uint32_t)RBINS)
            __hip_atomic_fetch_add(rh + rb + lane_id(), c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);   // an L2 atomic
        counted = nb;
    };
    // barrier + count; returns it (> CAP: overflowed). Compacts when the headroom gets short: for k <= 256, in safe
    // mode and at the end (the published list then holds at most max(k, CAP - TILE)), when another whole tile could
    // overflow; otherwise when less than 3 tiles' worth at the observed append rate (at least 341) is left - an
    // overflow past that is caught at the next check and the segment streamed again in safe mode. A compaction
    // first drops the entries below the row bound (the largest of the waves' tkeys: one pass); only if that leaves
    // the headroom short (or more than KMAX entries) it keeps exactly the segment's k largest.
    int lastn = 0;
    const bool dyncount = topk && k > WAVE;      // k > 64: the buffered entries are counted at checks
    // last: the segment's final check, after which nothing is appended (its count needs no second barrier)
    auto check = [&](int tiles, bool strict, bool last = false) -> int {
        __syncthreads();
        int n = (int)s.count;
        if (!last) __syncthreads();                    // every wave holds the same count before any appends again
        int rate = (n - lastn) / (tiles > 0 ? tiles : 1);
        rate = rate > 341 ? rate : 341;
        auto short_room = [&](int m) {
            return m > k && (strict || k <= 4 * WAVE ? m > CAP - TILE : CAP - m < 3 * rate);
        };
        if (n <= CAP && short_room(n)) {
            if (dyncount && !strict) count_row(counted, n);   // before the order changes (not in safe mode)
            raise_key(block_max_u32(tkey, s.red));          // its barriers also end count_row's use of bins()
            const int m = keep_from(n, (uint64_t)tkey << 32, s);
            if (m >= 0) {
                n = m;
                counted = m;
            }
            if (m < 0 || short_room(n)) {
                // the entries at or above the k-th largest key (a radix select over the key bytes: 4 passes of an
                // 8-bit LDS histogram); if ties at that key leave too little room, exactly the k largest composites
                int nn = n;
                auto each = [&](auto&& f) { for (int i = tid; i < nn; i += BLOCK) f(s.cand[i]); };
                uint64_t X = radix_kth(each, k, s.bins(), s.wsum, s.red, 32);
                const int m2 = keep_from(nn, X, s);
                if (m2 >= 0) nn = m2;
                if (m2 < 0 || short_room(nn)) {
                    X = radix_kth(each, k, s.bins(), s.wsum, s.red);
                    (void)keep_from(nn, X, s);   // exactly k (composites are distinct)
                    nn = k;
                }
                raise_key(comp_key(X));
                n = nn;
                counted = n;               // the survivors are left uncounted (fewer counts: bounds stay valid)
            }
        }
        lastn = n;
        return n;
    };
    static_assert(PF == 2, "the row read is issued and taken within one iteration of the tile loop");
    RowSnap snap1;                     // the row histogram after tile 0 (segments of >= 3 tiles)
    for (int pass = 0; pass < 2; ++pass) {
        const bool safe = pass == 1;
        // k <= 64: tile 0's candidates are appended at tile 1, after the first row bound (its penalised logits wait in
        // the candidate buffer's tail; each thread reads back its own). Rows with the per-tile count table, and rows
        // with larger k (whose tile-0 bound lets through half a tile or more), append at once.
        const bool defer0 = topk && !safe && ntiles >= 2 && !tablepen && k <= WAVE;
        bool overflow = false;
        int R = 1;
        // ---- tile 0 (peeled: the initial threshold is computed here), through its stage
        {
            float x[TPT];
            const int lo = seg_lo;
            {
                stage_tile0();
                if (!safe) { FS_MARK(1); }
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    const float4 v = stage0[j * BLOCK + tid];
                    x[4 * j] = v.x; x[4 * j + 1] = v.y; x[4 * j + 2] = v.z; x[4 * j + 3] = v.w;
                }
            }
            if (rc.capped) softcap_vals_unrolled(x, rc.p.softcap);
            if (tablepen) apply_penalties(x, a, rc, lo, s);
            if (wavepen) wave_penalties(x, rc, lo, 0, s);
            if (fastpen) bitmap_pen(x, lo);
            if (rc.greedy) {
                greedy_update(x, 0);
            } else {
                if (!safe) {
                    // T0 and the row counts from the tile's lane maxima (all 8 logits of a lane when k > 64): a
                    // histogram over the 64 coarse bins up to the tile's largest key (rc0 = its lowest), in LDS.
                    // Its bins go to the row histogram at once, and T0 = the lower edge of the highest bin with at
                    // least k counted logits at or above it. Logits below the 64 bins are not counted (fewer
                    // counts: every bound read from them stays valid).
                    uint32_t kq[TPT];
                    uint32_t m1 = 0u;
                    if (k > WAVE) {
#pragma unroll
                        for (int i = 0; i < TPT; ++i) {
                            kq[i] = key_of(x[i]);
                            m1 = kq[i] > m1 ? kq[i] : m1;
                        }
                    } else {                             // the lane's largest logit (fmaxf passes over NaN)
                        float fm = x[0];
#pragma unroll
                        for (int i = 1; i < TPT; ++i) fm = fmaxf(fm, x[i]);
                        m1 = key_of(fm);
                    }
                    const uint32_t wm = wave_max(m1);
                    if (lane_id() == 0) atomicMax(&s.tmax, wm);
                    __syncthreads();
                    const uint32_t topb = s.tmax >> RSHIFT;
                    rc0 = topb >= (uint32_t)(WAVE - 1) ? topb - (uint32_t)(WAVE - 1) : 0u;
                    if (k > WAVE) {
#pragma unroll
                        for (int i = 0; i < TPT; ++i) {
                            const uint32_t d = (kq[i] >> RSHIFT) - rc0;
                            if (d < (uint32_t)WAVE) atomicAdd(&s.rc64[d], 1u);
                        }
                    } else {
                        const uint32_t d = (m1 >> RSHIFT) - rc0;
                        if (d < (uint32_t)WAVE) atomicAdd(&s.rc64[d], 1u);
                    }
                    __syncthreads();
                    const uint32_t cb = s.rc64[WAVE - 1 - lane_id()];   // lane order = descending bins
                    const uint64_t hb = __ballot(wave_incl_scan_u32(cb) >= (uint32_t)k);
                    if (hb != 0ull)
                        raise_key((rc0 + (uint32_t)(WAVE - 1) - (uint32_t)(__ffsll((unsigned long long)hb) - 1)) << RSHIFT);
                    if (tid < WAVE) {
                        const uint32_t c = s.rc64[tid];
                        if (c != 0u) __hip_atomic_fetch_add(rh + rc0 + tid, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    }
                }
                if (defer0) {                            // the penalised tile waits in its stage for tile 1
#pragma unroll
                    for (int j = 0; j < NV; ++j)
                        stage0[j * BLOCK + tid] = make_float4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]);
                } else {
                    topk_append(x, lo);
                }
            }
            if (topk) {
                lastn = 0;
                // with tile 0's appends deferred the buffer is still empty: no check (two barriers) is needed
                const int n = defer0 ? 0 : check(1, safe);
                overflow = n > CAP;
                if (!safe && ntiles >= 3) snap1 = row_snap(rsr, tkey);
                const int per_tile = n > 32 ? n : 32;
                R = safe ? 1 : (CAP - n) / (2 * per_tile);
                if (R < 1) R = 1;
                if (!safe && ntiles < 3) {               // short segments: read once, taken at the end
                    sb0 = tkey >> RSHIFT;
                    scnt = row_read(sb0);
                    spending = true;
                }
            } else if (tablepen) {
                __syncthreads();                         // penalty-table reads of this tile are done
            }
            if (!safe) { FS_MARK(2); FS_MARKW(5); }
        }
        // ---- tiles 1.. (PF in flight; tile t is in buf[t % 2]). Iterations start at odd tiles, so the order in
        // which the two buffers were requested is the same on entry and around the back edge.
        int since = 0;
        // k > 64: a snapshot requested at every iteration's first tile (after its check and row count, before its
        // successor's loads), read at the next iteration's first tile: waiting for that tile covers it. Other rows
        // request it from an empty resource (no memory access).
        const bool dynrow = topk && !safe && k > WAVE;
        const __amdgpu_buffer_rsrc_t rsh = __builtin_amdgcn_make_buffer_rsrc(rh, (short)0, dynrow ? RBINS * 4 : 0,
                                                                             0x00020000);
        RowSnap snapd;
        bool dpend = false;
        for (int t0 = 1; t0 < ntiles && !overflow; t0 += PF) {
            const bool take1 = topk && !safe && t0 == 1 && ntiles >= 3;   // bound before tile 1
            const bool snap = topk && !safe && (t0 == 3 || t0 == 5) && t0 + 1 < ntiles;   // snapshot at 3/5, bound at 4/6
            const bool count2 = topk && !safe && t0 == 3 && ntiles >= 7 && k <= WAVE;   // tiles 1-4 at tile 4
            RowSnap snap2;
#pragma unroll
            for (int p = 0; p < PF; ++p) {
                const int tt = t0 + p;
                float (&x)[TPT] = buf[(p + 1) & 1];
                const bool live = tt < ntiles && !overflow;
                if (live) {
                    const int lo = seg_lo + tt * TILE;
                    if (rc.capped) softcap_vals_unrolled(x, rc.p.softcap);
                    if (tablepen) apply_penalties(x, a, rc, lo, s);
                    if (wavepen) wave_penalties(x, rc, lo, tt, s);
                    if (fastpen) bitmap_pen(x, lo);
                    if (p == 0 && take1) raise_key(row_bound(snap1, k));
                    if (p == 0 && dpend) raise_key(row_bound(snapd, k));
                    if (p == 1 && snap) raise_key(row_bound(snap2, k));
                    if (rc.greedy) {
                        greedy_update(x, tt);
                    } else {
                        if (p == 0 && defer0 && t0 == 1) {
                            float x0[TPT];
#pragma unroll
                            for (int j = 0; j < NV; ++j) {
                                const float4 v = stage0[j * BLOCK + tid];
                                x0[4 * j] = v.x; x0[4 * j + 1] = v.y; x0[4 * j + 2] = v.z; x0[4 * j + 3] = v.w;
                            }
                            topk_append(x0, seg_lo);
                        }
                        topk_append(x, lo);
                    }
                }
                // past the end: zeros, no memory access. The first tile of an iteration requests its successor
                // after the check and the row snapshot: the snapshot is then taken at the next tile with that
                // tile's successor still in flight (waits on the memory counter complete in request order).
                if (p == 1) load_seg_tile(x, g.rs, tt + PF);
                if (live) {
                    if (topk) {
                        bool checked = false;
                        if (++since >= R || tablepen || (dynrow && p == 0)) {
                            overflow = check(since, safe) > CAP;   // uniform: every thread read the same count
                            since = 0;
                            checked = true;
                        }
                        if (p == 0 && checked && dynrow && !overflow && t0 + PF < ntiles) count_row(counted, lastn);
                        if (p == 0) dpend = dynrow && !overflow && t0 + PF < ntiles;
                        if (p == 0 && snap) snap2 = row_snap(rsr, tkey);
                        if (p == 1 && count2 && !overflow) {
                            // second count: the buffered logits of tiles 1-4
                            __syncthreads();
                            const int nb = (int)s.count;
                            __syncthreads();
                            count_row(0, nb);
                        }
                    } else if (tablepen) {
                        __syncthreads();                 // penalty-table reads of this tile are done
                    }
                }
                if (p == 0) {
                    snapd = row_snap(rsh, tkey);
                    load_seg_tile(x, g.rs, tt + PF);
                }
                if (!safe && tt < 8) FS_MARKW(5 + tt);
            }
        }

        if (!topk) break;
        if (!overflow) overflow = check(since, true, true) > CAP;
        if (!overflow) break;
        // overflow: the buffer lost candidates. tkey is still a valid bound; stream the segment again in safe mode
        // (its logits are already counted in the row histogram).
        __syncthreads();
        if (tid == 0) s.count = 0u;
        spending = false;
#pragma unroll
        for (int p = 0; p < PF; ++p) load_seg_tile(buf[p], g.rs, p);
        __syncthreads();
    }
    if (topk && spending) row_take(sb0, scnt);
    FS_MARK(3);

    // ---- publish this segment's candidates (read by the merge kernel after this kernel completes)
    const int64_t slot = slot_of(rc, seg);
    uint64_t* gout = a.cand + (int64_t)slot * CAP;
    if (rc.greedy) {
        uint64_t best = 0ull;
        if (bs >= 0) best = comp_of(key_of(bv), (uint32_t)elem_id(seg_lo + (bs / TPT) * TILE, bs % TPT));
        best = block_max_u64(best, s.red);
        if (tid == 0) {
            gout[0] = best;
            a.meta[2 * slot] = comp_key(best);
            a.meta[2 * slot + 1] = 1u;
        }
    } else {
        // the buffered candidates with key >= tkey, in buffer order (thread t: entries t, t + BLOCK, ...)
        const int n = (int)s.count;              // <= CAP: no overflow past the checks above
        uint32_t mine = 0u;
        for (int i = tid; i < n; i += BLOCK)
            if (comp_key(s.cand[i]) >= tkey) ++mine;
        uint32_t tot;
        uint32_t pos = block_excl_scan<uint32_t>(mine, s.wsum, &tot);
        for (int i = tid; i < n; i += BLOCK) {
            const uint64_t c = s.cand[i];
            if (comp_key(c) >= tkey) gout[pos++] = c;
        }
        if (tid == 0) {
            a.meta[2 * slot] = tkey;              // at least k of the row's logits reach it
            a.meta[2 * slot + 1] = tot;
        }

    }
    __syncthreads();                               // LDS is reused by the next item
}

// ------------------------------------------------------------------------------------------------ large k, split
// Rows sampled with k > KMAX (top_k = 0 included: ferro's k = n, sampler.cpp:26) are sampled by the row's segment
// workgroups together: the passes of large_row (the one-workgroup version, kept as the fallback) each run over
// every segment at once, and the segments meet at row barriers between them. After each barrier every segment reads
// the others' published partial results and computes the same row-wide decision (the same inputs in the same
// order), so no workgroup waits for a coordinator:
//   P1 extremes, ordered count and (k < V) coarse-bin counts (added to the row histogram) -> the k-th's coarse bin bk;
//   P2 the masses exp((v - mx) / T) of the candidates above bk (fp64 partial sums, fixed-point mass histogram added
//      to the row's in the workspace) and bin bk's elements gathered -> the exact k-th Xk, S and the mass histogram;
//   P3 top-p's crossing bin bc gathered, with min-p's counts and masses -> the kept prefix and its total;
//   P4 the draw's bin bd gathered, unless it is bc (already sorted in LDS) -> the token.
// Segment 0 publishes the token and what the merge needs for the optional candidate outputs. A bin too large for
// one sort, a target outside its bin's exact masses, or a barrier that waits too long abandons the row (a flag on
// the barrier counter); the merging workgroup then samples it alone with large_row (exact).
// Arrive and wait until `target` arrivals (every segment of the row at this barrier). This workgroup's stores and
// atomics complete first (vmcnt(0)). No cache maintenance follows: what the others published lies in lines that no
// workgroup of the row reads before this barrier (their own lines per phase, see the slot layout), so this CU's L1
// holds no copy of them and the loads are served by the XCD's L2. (An agent-scope invalidate, buffer_inv sc1, cost
// about 10 us per barrier here.) The poll is an atomic that is not idempotent (it executes in the L2). Bounded: past
// a.merge_spins polls the row is abandoned. Returns false when the row is abandoned.
__device__ __forceinline__ bool row_sync(const Args& a, int row, uint32_t target, Shared& s) {
    vm_drain();
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t* c = row_sync_ctr(a, row);
        __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        uint32_t ok = 1u, spins = 0u;
        for (;;) {
            const uint32_t v = __hip_atomic_fetch_add(c, 0x10000u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (v & ROW_ABANDONED) { ok = 0u; break; }
            if ((v & 0x7FFFu) >= target && a.merge_spins != 0u) break;
            if (++spins >= a.merge_spins) {
                __hip_atomic_fetch_or(c, ROW_ABANDONED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                ok = 0u;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        s.red.misc[4] = ok;
    }
    __syncthreads();
    const bool ok = s.red.misc[4] != 0u;
    __syncthreads();                                     // misc[4] is reused by the next barrier
    return ok;
}

// One pass over a large-row segment's tiles [lo0, hi) (the last segment also takes the row's partial tile), two
// tiles in flight, softcap and penalties applied: f(x, key, composite) per ordered element. Ends with a barrier.
// bmp: a repetition penalty alone, from a bitmap of the window's ids over the segment (bit i = id lo0 + i; a
// thread's four consecutive logits share a word), else the per-tile count table (s.ids holds the window's ids).
// g(x): a per-tile hook, called on each tile's (softcapped, penalised) logits before f sees them.
template <class F, class G>
__device__ __forceinline__ void seg_elems_g(const Args& a, const RowCtx& rc, Shared& s, int lo0, int hi, bool bmp, F f, G g) {
    const float* rowp = a.logits + (int64_t)rc.row * a.ld;
    const int nt = (hi - lo0 + TILE - 1) / TILE;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(rowp + lo0), (short)0,
                                                                        ((hi - lo0 + 3) & ~3) * 4, 0x00020000);
    float buf[LPF][TPT];
#pragma unroll
    for (int p = 0; p < LPF; ++p) load_seg_tile(buf[p], rs, p);
    for (int t0 = 0; t0 < nt; t0 += LPF) {
#pragma unroll
        for (int p = 0; p < LPF; ++p) {
            const int t = t0 + p;
            float x[TPT];
#pragma unroll
            for (int i = 0; i < TPT; ++i) x[i] = buf[p][i];
            load_seg_tile(buf[p], rs, t + LPF);
            if (t < nt) {
                const int lo = lo0 + t * TILE;
                if (rc.capped) softcap_vals(x, rc.p.softcap);
                if (rc.pen && bmp) {
                    const uint32_t* bm = reinterpret_cast<const uint32_t*>(s.ids);
                    const float rp = rc.p.repetition_penalty;
#pragma unroll
                    for (int j = 0; j < NV; ++j) {
                        const uint32_t rel = (uint32_t)(lo - lo0) + (uint32_t)(j * BLOCK + (int)threadIdx.x) * 4u;
                        const uint32_t nib = (bm[rel >> 5] >> (rel & 31u)) & 0xFu;
                        if (nib != 0u) {
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const float l = x[4 * j + q];
                                if ((nib >> q) & 1u) x[4 * j + q] = l > 0.0f ? __fdiv_rn(l, rp) : __fmul_rn(l, rp);
                            }
                        }
                    }
                } else if (rc.pen) {
                    __syncthreads();                     // the previous tile's table reads are done
                    apply_penalties(x, a, rc, lo, s);
                }
                g(x, lo);
#pragma unroll
                for (int i = 0; i < TPT; ++i) {
                    const int e = elem_id(lo, i);
                    const bool ok = e < hi && x[i] == x[i];
                    const uint32_t kq = key_of(x[i]);
                    f(ok, x[i], kq, comp_of(kq, (uint32_t)e));
                }
            }
        }
    }
    __syncthreads();
}

template <class F>
__device__ __forceinline__ void seg_elems(const Args& a, const RowCtx& rc, Shared& s, int lo0, int hi, bool bmp, F f) {
    seg_elems_g(a, rc, s, lo0, hi, bmp, f, [](const float (&)[TPT], int) {});
}

// The gathered lists of one region of every segment of the row, concatenated into s.cand[0, n) and sorted in
// candidate order (descending composites). Returns n, or -1 when a list overflowed or they exceed KMAX together.
// Called after a row barrier (the lists are in the L2; this workgroup's L1 is invalidated).
__device__ __forceinline__ int load_lists(const Args& a, const RowCtx& rc, int region, int cnt_slot, Shared& s) {
    const int tid = threadIdx.x, nseg = rc.nseg;
    uint32_t mine = 0u;
    bool over = false;
    for (int j = tid; j < nseg; j += BLOCK) {
        const uint64_t c = a.cand[slot_of(rc, j) * CAP + cnt_slot];
        over |= c > (uint64_t)LLR;
    }
    // offsets: thread j < nseg holds list j's count (nseg < BLOCK, kept so by the host)
    if (tid < nseg) {
        const uint64_t c = a.cand[slot_of(rc, tid) * CAP + cnt_slot];
        mine = c > (uint64_t)LLR ? 0u : (uint32_t)c;
    }
    uint32_t tot;
    const uint32_t off = block_excl_scan<uint32_t>(mine, s.wsum, &tot);
    const bool any_over = block_max_u32(over ? 1u : 0u, s.red) != 0u;
    if (any_over || tot > (uint32_t)KMAX) return -1;    // uniform
    if (tid < nseg) s.off[tid] = off;
    if (tid == 0) s.off[nseg] = tot;
    __syncthreads();
    for (uint32_t f = tid; f < tot; f += BLOCK) {        // flat index -> (list, position)
        int c0 = 0, c1 = nseg;
        while (c1 - c0 > 1) {
            const int m = (c0 + c1) >> 1;
            if (s.off[m] <= f) c0 = m; else c1 = m;
        }
        s.cand[f] = a.cand[slot_of(rc, c0) * CAP + LSC + region * LLR + (f - s.off[c0])];
    }
    __syncthreads();
    bin_sort_desc((int)tot, s);
    return (int)tot;
}

// A row-wide sum over the segments' published scalar (fp64 bits at cnt_slot), in a fixed order (deterministic).
__device__ __forceinline__ double sum_slots_f64(const Args& a, const RowCtx& rc, int sl, Shared& s) {
    double v = 0.0;
    for (int j = threadIdx.x; j < rc.nseg; j += BLOCK) v += __longlong_as_double((long long)a.cand[slot_of(rc, j) * CAP + sl]);
    return block_sum_f64(v, s.red);
}
__device__ __forceinline__ uint64_t sum_slots_u64(const Args& a, const RowCtx& rc, int sl, Shared& s) {
    uint64_t v = 0ull;
    for (int j = threadIdx.x; j < rc.nseg; j += BLOCK) v += a.cand[slot_of(rc, j) * CAP + sl];
    uint64_t tot;
    (void)block_excl_scan<uint64_t>(v, s.red.u64b, &tot);
    return tot;
}

// Rows where every token is a candidate (k >= V) sampled from the logits within CUT_C * T of the row's maximum,
// when the rest provably holds neither top-p's crossing, min-p's boundary nor the draw: after the first row barrier
// every segment decides the same way from the published scalars (same inputs, same order); segment 0 then gathers the
// lists (at most KMAX logits), sorts them, and runs sampler.cpp:37-49 over them in double precision, the rest's mass
// (every element below e^-CUT_C of the maximum) added to S. Returns true when the row is done (or given to the merge:
// a target that still lands in the rest abandons the row to the exact path); false: the segments go on with the
// passes of the general large-row path.
constexpr float CUT_C = 16.0f;
constexpr double CFXS = 1125899906842624.0;      // 2^50: fixed-point scale of the lists' masses (each <= 1, <= CAP)

template <bool DESC>
__device__ __forceinline__ uint64_t sort64(uint64_t v);

// large_cut's finish when the lists hold at most 64 logits and the row has at most 64 segments: one wave, the
// logits in lanes (sampler.cpp:28-49 as in the block version below, with wave scans in candidate order).
// Returns false when a target lands in the rest (the caller abandons the row).
__device__ __forceinline__ bool wave_cut_finish(const Args& a, const RowCtx& rc, uint64_t* my, float mx, float cut,
                                                double Td, double st, uint32_t ntot, int keff, uint32_t kmax,
                                                uint64_t cmin, double u, bool min_in, uint32_t cnt) {
    const int lane = lane_id(), nseg = rc.nseg;
    const fs_row_params& p = rc.p;
    // the lists' offsets (lane j: list j's count cnt), then lane f takes flat entry f
    const uint32_t inc = wave_incl_scan_u32(cnt);
    const uint32_t off = inc - cnt;
    const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
    int j = 0;
    for (int q = 1; q < nseg; ++q)
        if ((uint32_t)lane >= (uint32_t)__builtin_amdgcn_readlane((int)off, q)) j = q;
    const uint32_t my_off = (uint32_t)__builtin_amdgcn_ds_bpermute(j << 2, (int)off);
    uint64_t c = 0ull;
    if ((uint32_t)lane < tot) c = a.cand[slot_of(rc, j) * CAP + LSC + ((uint32_t)lane - my_off)];
    const float x = val_of(comp_key(c));
    const bool in = (uint32_t)lane < tot && x >= mx - cut;
    const uint64_t dm = ((uint32_t)lane < tot && !in) ? (uint64_t)(mass_of(x, mx, Td) * CFXS + 0.5) : 0ull;
    const uint64_t dfx = wave_allreduce(dm, [](uint64_t p_, uint64_t q_) { return p_ + q_; });
    const uint64_t v = sort64<true>(in ? c : 0ull);      // ferro's order; lanes >= n hold 0
    const int n = __popcll(__ballot(in));
    const double rest = st + (double)dfx / CFXS;
    double e = 0.0;
    if (lane < n) e = mass_of(val_of(comp_key(v)), mx, Td);
    const double S = lane_f64(wave_scan_f64(e), WAVE - 1) + rest;
    const double pr = e / S;
    const double cum = wave_scan_f64(pr);
    int keep_m = n;
    bool m_beyond = (uint32_t)n < ntot;
    if (p.min_p > 0.0f) {
        const double thr = (1.0 / S) * (double)p.min_p;
        const uint64_t mm = __ballot(lane < n && !(pr < thr));
        keep_m = mm ? 64 - __clzll((long long)mm) : 1;
        m_beyond = keep_m == n && (uint32_t)n < ntot && !min_in;
    }
    int keep = keep_m;
    bool beyond = m_beyond;
    if (p.top_p < 1.0f) {
        const uint64_t mm = __ballot(lane < keep_m && cum >= (double)p.top_p);
        if (mm) {
            const int first = __ffsll((unsigned long long)mm) - 1;
            keep = first + 1 < keep_m ? first + 1 : keep_m;
            beyond = false;
        } else if (m_beyond) {
            return false;                                // top-p's crossing lies in the rest
        }
    } else if (m_beyond && p.min_p > 0.0f) {
        return false;                                    // min-p's boundary lies in the rest
    }
    const double totk = beyond ? lane_f64(cum, n - 1) + rest / S : lane_f64(cum, keep - 1);
    const double rr = u * totk + 0.0;
    const int lim = beyond ? n : keep;
    const uint64_t hm = __ballot(lane < lim && rr <= cum);
    int at;
    if (hm) at = __ffsll((unsigned long long)hm) - 1;
    else if (beyond) return false;                       // the draw lies in the rest
    else at = keep - 1;
    const uint64_t pick = read_lane(v, at);
    if (lane == 0) {
        const uint32_t kp = beyond ? ntot : (uint32_t)keep;
        my[LS_TOK] = (uint64_t)comp_id(pick) | ((uint64_t)kp << 32);
        my[LS_XK] = cmin;
        my[LS_S] = (uint64_t)__double_as_longlong(S);
        my[LS_KEFF] = (uint64_t)(uint32_t)keff | ((uint64_t)kmax << 32);
        my[LS_STATUS] = 2ull;
    }
    return true;
}

// The cut's decision from the row's published sums: sc / st the listed logits' / the rest's mass relative to the
// row's maximum, nft the lists' total. True when the rest provably holds neither top-p's crossing, min-p's boundary
// nor the draw (estimates within 1e-5; the exact walk still checks).
__device__ __forceinline__ bool cut_decide(const fs_row_params& p, double sc, double st, uint64_t nft, bool ovf,
                                           double u, bool& min_in) {
    const double S_est = sc + st;
    const double e_c = exp(-(double)CUT_C);
    const double sc_lo = sc - (double)nft * e_c;          // the row's cut moves at most e^-CUT_C per listed logit
    const double mrg = 1.0 + 1e-5;
    min_in = p.min_p > 0.0f && (double)p.min_p >= e_c * 1.01;   // min-p keeps only listed logits
    bool within = min_in;
    if (p.top_p < 1.0f) within = within || (double)p.top_p * S_est * mrg < sc_lo;
    if (!(p.top_p < 1.0f) && !(p.min_p > 0.0f)) within = u * S_est * mrg < sc_lo;
    return !ovf && nft >= 1u && nft <= (uint64_t)KMAX && within;
}

// large_cut's finish by the whole block (the lists hold more than 64 logits, or the row more than 64 segments).
__device__ __forceinline__ void cut_finish_block(const Args& a, const RowCtx& rc, Shared& s, uint64_t* my, float mx,
                                                 uint32_t kmax, uint64_t cmin, uint32_t ntot, int keff, double st,
                                                 double u, bool min_in) {
    const int tid = threadIdx.x, nseg = rc.nseg, row = rc.row;
    const fs_row_params& p = rc.p;
    const double Td = (double)p.temperature;
    const float cut = CUT_C * p.temperature;
    // ---- segment 0: the lists above mx - cut, sorted (sampler.cpp:28-35)
    uint32_t mine = 0u;
    if (tid < nseg) mine = (uint32_t)a.cand[slot_of(rc, tid) * CAP + LS_FN];
    uint32_t tot;
    const uint32_t off = block_excl_scan<uint32_t>(mine, s.wsum, &tot);
    if (tid < nseg) s.off[tid] = off;
    if (tid == 0) { s.off[nseg] = tot; s.count = 0u; }
    __syncthreads();
    uint64_t drop = 0ull;                                // fixed point: the lists' order is not fixed
    for (uint32_t b0 = 0u; b0 < tot; b0 += BLOCK) {
        const uint32_t f = b0 + (uint32_t)tid;
        uint64_t c = 0ull;
        if (f < tot) {
            int c0 = 0, c1 = nseg;
            while (c1 - c0 > 1) {
                const int m = (c0 + c1) >> 1;
                if (s.off[m] <= f) c0 = m; else c1 = m;
            }
            c = a.cand[slot_of(rc, c0) * CAP + LSC + (f - s.off[c0])];
        }
        const float x = val_of(comp_key(c));
        const bool in = f < tot && x >= mx - cut;
        if (f < tot && !in) drop += (uint64_t)(mass_of(x, mx, Td) * CFXS + 0.5);
        wave_append(in, c, s.cand, &s.count, (uint32_t)CAP);
    }
    uint64_t dfx;
    (void)block_excl_scan<uint64_t>(drop, s.red.u64b, &dfx);   // its barriers also complete the appends
    const int n = (int)s.count;
    FS_MARK(7);                                          // lists gathered
    __syncthreads();
    bin_sort_desc(n, s);
    FS_MARK(2);                                          // sorted
    // ---- softmax over the list plus the rest's mass, min-p, top-p, draw (sampler.cpp:37-49)
    const int i0 = tid * KPT;
    double e[KPT];
    double part = 0.0;
#pragma unroll
    for (int q = 0; q < KPT; ++q) {
        e[q] = i0 + q < n ? mass_of(val_of(comp_key(s.cand[i0 + q])), mx, Td) : 0.0;
        part += e[q];
    }
    const double rest = st + (double)dfx / CFXS;
    const double S = block_sum_f64(part, s.red) + rest;
    FS_MARK(3);                                          // S
    double pr[KPT];
#pragma unroll
    for (int q = 0; q < KPT; ++q) pr[q] = e[q] / S;
    int keep_m = n;
    bool m_beyond = (uint32_t)n < ntot;                  // every listed logit kept so far and the rest after them
    if (p.min_p > 0.0f) {
        const double thr = (1.0 / S) * (double)p.min_p;
        int last = -1;
#pragma unroll
        for (int q = 0; q < KPT; ++q)
            if (i0 + q < n && !(pr[q] < thr)) last = i0 + q;
        last = block_max_i32(last, s.red);
        keep_m = last + 1 > 1 ? last + 1 : 1;
        m_beyond = keep_m == n && (uint32_t)n < ntot && !min_in;
    }
    double c[KPT];
    double run = 0.0;
#pragma unroll
    for (int q = 0; q < KPT; ++q) { run += pr[q]; c[q] = run; }
    double tot_all;
    const double coff = block_excl_scan<double>(run, s.red.f64, &tot_all);
#pragma unroll
    for (int q = 0; q < KPT; ++q) c[q] += coff;
    int keep = keep_m;
    bool beyond = m_beyond;
    bool fail = false;
    if (p.top_p < 1.0f) {
        int first = 0x7fffffff;
#pragma unroll
        for (int q = 0; q < KPT; ++q)
            if (i0 + q < keep_m && c[q] >= (double)p.top_p && first == 0x7fffffff) first = i0 + q;
        first = block_min_i32(first, s.red);
        if (first != 0x7fffffff) {
            keep = first + 1 < keep_m ? first + 1 : keep_m;
            beyond = false;
        } else if (m_beyond) {
            fail = true;                                 // top-p's crossing lies in the rest
        }
    } else if (m_beyond && p.min_p > 0.0f) {
        fail = true;                                     // min-p's boundary lies in the rest
    }
    // tot = the kept prefix's sum; r = u * tot; the first i with r <= c_i
    double totk = 0.0;
    if (!beyond) {
#pragma unroll
        for (int q = 0; q < KPT; ++q)
            if (i0 + q == keep - 1) s.red.dmisc[0] = c[q];
        __syncthreads();
        totk = s.red.dmisc[0];
    } else {
        totk = tot_all + rest / S;
    }
    const double rr = u * totk + 0.0;
    const int lim = beyond ? n : keep;
    int hit = 0x7fffffff;
#pragma unroll
    for (int q = 0; q < KPT; ++q)
        if (i0 + q < lim && rr <= c[q] && hit == 0x7fffffff) hit = i0 + q;
    hit = block_min_i32(hit, s.red);
    if (hit == 0x7fffffff) {
        if (beyond) fail = true;                         // the draw lies in the rest
        else hit = keep - 1;
    }
    FS_MARK(8);                                          // walked
    if (fail) {
        row_abandon(a, row);
        return;
    }
    if (tid == 0) {
        const uint32_t kp = beyond ? ntot : (uint32_t)keep;
        my[LS_TOK] = (uint64_t)comp_id(s.cand[hit]) | ((uint64_t)kp << 32);
        my[LS_XK] = cmin;
        my[LS_S] = (uint64_t)__double_as_longlong(S);
        my[LS_KEFF] = (uint64_t)(uint32_t)keff | ((uint64_t)kmax << 32);
        my[LS_STATUS] = 2ull;
    }
}

__device__ __forceinline__ bool large_cut(const Args& a, const RowCtx& rc, Shared& s, int seg, uint64_t* my, float mx,
                                          uint32_t kmax, uint64_t cmin, uint32_t ntot, int keff) {
    const int tid = threadIdx.x, nseg = rc.nseg, row = rc.row;
    const fs_row_params& p = rc.p;
    if (!(mx > -__builtin_huge_valf() && mx < __builtin_huge_valf())) return false;   // uniform
    const double Td = (double)p.temperature;
    // row-wide: the lists' total, their masses and the rest's, relative to mx
    uint32_t nf = 0u, ovf = 0u;
    double sc = 0.0, st = 0.0;
    for (int j = tid; j < nseg; j += BLOCK) {
        const uint64_t* sl = a.cand + slot_of(rc, j) * CAP;
        const uint64_t n = sl[LS_FN];
        if (n > (uint64_t)LLR) ovf = 1u; else nf += (uint32_t)n;
        if (sl[LS_NV] != 0ull) {
            const double F = exp(((double)val_of(comp_key(sl[LS_MAX])) - (double)mx) / Td);
            sc += F * __longlong_as_double((long long)sl[LS_FC]);
            st += F * __longlong_as_double((long long)sl[LS_FT]);
        }
    }
    uint32_t nft;
    (void)block_excl_scan<uint32_t>(nf, s.wsum, &nft);
    ovf = block_max_u32(ovf, s.red);
    sc = block_sum_f64(sc, s.red);
    st = block_sum_f64(st, s.red);
    const double u = row_u(a, row);
    bool min_in;
    if (!cut_decide(p, sc, st, nft, ovf != 0u, u, min_in)) return false;   // uniform
    if (seg != 0) return true;
    cut_finish_block(a, rc, s, my, mx, kmax, cmin, ntot, keff, st, u, min_in);
    return true;
}

// A crowded coarse bin (more candidates than the gather regions hold, e.g. the middle of a flat row): the element
// at which the cumulative mass in ferro's order, from the row's top, reaches `target` inside bin b, through one
// level of finer bins (the next FSB key bits). above_b is the mass of the candidates above bin b. All segments run
// it together (uniform arguments, row barriers from nsync on):
//   1. the row's fine histogram is cleared (rmass: fixed-point masses, rhist: counts; neither is read any more)
//   2. each segment streams its tiles: masses and counts of its candidates in bin b by fine bin, added to the row's
//   3. every segment locates the fine bin of the target (the same sums, the same decision) and gathers it
//   4. the gathered lists, sorted, are walked in exact fp64 masses (large_walk)
// Returns false (the row is then abandoned) when the fine bin still overflows or the walk leaves it; otherwise the
// element, the cumulative mass through it and the number of candidates in bin b before it.
constexpr int FSB = 11;                                    // fine bins: 2048 (row histogram bins below its counters)
constexpr int FBN = 1 << FSB;
constexpr int FSH = LB_SHIFT - FSB;
static_assert(FBN <= RBINS - 2 && FBN <= LB && FSH >= 0, "fine bins fit the row histograms");
__device__ __forceinline__ bool refine_bin(const Args& a, const RowCtx& rc, Shared& s, int seg_i, uint64_t* my, int lo0, int hi,
                                        bool bmpen, uint32_t b, uint64_t Xlo, double above_b, double target, float mx,
                                        double Td, uint32_t& nsync, uint64_t& pick, double& cum, uint32_t& before) {
    const int tid = threadIdx.x, row = rc.row, nseg = rc.nseg;
    uint64_t* rm = a.rmass + (int64_t)row * LB;
    uint32_t* rh = a.rhist + (int64_t)row * RBINS;
    // 1. clear this segment's slice of the row's fine histogram
    const int per = (FBN + nseg - 1) / nseg;
    for (int i = seg_i * per + tid; i < (seg_i + 1) * per && i < FBN; i += BLOCK) { rm[i] = 0ull; rh[i] = 0u; }
    ++nsync;
    if (!row_sync(a, row, nsync * (uint32_t)nseg, s)) return false;
    // 2. this segment's candidates in bin b, by fine bin (LDS: masses in s.cand[0, FBN), counts after them)
    uint64_t* fm = s.cand;
    uint32_t* fc = reinterpret_cast<uint32_t*>(s.cand + FBN);
    for (int i = tid; i < FBN; i += BLOCK) { fm[i] = 0ull; fc[i] = 0u; }
    __syncthreads();
    seg_elems(a, rc, s, lo0, hi, bmpen, [&](bool ok, float x, uint32_t kq, uint64_t c) {
        if (ok && c >= Xlo && (kq >> LB_SHIFT) == b) {
            const uint32_t f = (kq >> FSH) & (uint32_t)(FBN - 1);
            atomicAdd(reinterpret_cast<unsigned long long*>(&fm[f]), (unsigned long long)(mass_of(x, mx, Td) * FXS + 0.5));
            atomicAdd(&fc[f], 1u);
        }
    });
    for (int i = tid; i < FBN; i += BLOCK) {
        if (fm[i] != 0ull) __hip_atomic_fetch_add(rm + i, fm[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (fc[i] != 0u) __hip_atomic_fetch_add(rh + i, fc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    ++nsync;
    if (!row_sync(a, row, nsync * (uint32_t)nseg, s)) return false;
    l1_invalidate();                                     // lines this call read before may be stale in the L1
    // 3. the fine bin holding the target (thread t: fine bins FBN-1-t*FPT .. descending), then its candidates
    constexpr int FPT = FBN / BLOCK;
    uint64_t v[LPT] = {};
    uint32_t cnt_v[FPT];
#pragma unroll
    for (int j = 0; j < FPT; ++j) {
        const int f = FBN - 1 - (FPT * tid + j);
        v[j] = __hip_atomic_load(rm + f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        cnt_v[j] = __hip_atomic_load(rh + f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    const double rest = target - above_b;
    uint64_t abf = 0ull;
    const uint64_t tfx = rest > 0.0 ? (uint64_t)(rest * FXS) : 0ull;
    // desc_locate over the FBN fine bins (LPT slots per thread, the first FPT used)
    int d;
    {
        uint64_t sum = 0ull;
#pragma unroll
        for (int j = 0; j < FPT; ++j) sum += v[j];
        uint64_t tot;
        uint64_t run = block_excl_scan<uint64_t>(sum, s.red.u64b, &tot);
        int hit = 0x7fffffff;
        uint64_t ab = 0ull;
#pragma unroll
        for (int j = 0; j < FPT; ++j) {
            if (hit == 0x7fffffff && v[j] != 0ull && run + v[j] >= tfx) { hit = FPT * tid + j; ab = run; }
            run += v[j];
        }
        d = block_min_i32(hit, s.red);
        if (d == 0x7fffffff) d = -1;
        if (d >= 0 && hit == d) s.red.u64b[0] = ab;
        __syncthreads();
        abf = d >= 0 ? s.red.u64b[0] : 0ull;
        __syncthreads();
    }
    if (d < 0) return false;                             // uniform
    const uint32_t fb = (uint32_t)(FBN - 1 - d);
    uint32_t cab = 0u;                                   // candidates in the fine bins above fb
#pragma unroll
    for (int j = 0; j < FPT; ++j) cab += (FPT * tid + j) < d ? cnt_v[j] : 0u;
    uint32_t cabt;
    (void)block_excl_scan<uint32_t>(cab, s.wsum, &cabt);
    if (tid == 0) s.count = 0u;
    __syncthreads();
    uint64_t* regC = my + LSC + 2 * LLR;
    seg_elems(a, rc, s, lo0, hi, bmpen, [&](bool ok, float, uint32_t kq, uint64_t c) {
        const bool in = ok && c >= Xlo && (kq >> LB_SHIFT) == b && ((kq >> FSH) & (uint32_t)(FBN - 1)) == fb;
        wave_append(in, c, regC, &s.count, (uint32_t)LLR);
    });
    if (tid == 0) my[LS_NBD] = s.count;
    ++nsync;
    if (!row_sync(a, row, nsync * (uint32_t)nseg, s)) return false;
    l1_invalidate();                                     // lines this call read before may be stale in the L1
    // 4. the walk inside the fine bin
    const int n = load_lists(a, rc, 2, LS_NBD, s);
    if (n < 0) return false;
    const int ic = large_walk(s, n, Xlo, above_b + (double)abf / FXS, target, mx, Td, &cum);
    if (ic < 0) return false;
    pick = s.cand[ic];
    before = cabt + (uint32_t)ic;
    return true;
}

// This segment's part of a large row (see above).
__device__ __forceinline__ void large_segment(const Args& a, const RowCtx& rc, int seg, Shared& s, const SegStart& g) {
    const int tid = threadIdx.x;
    const int row = rc.row, nseg = rc.nseg;
    const fs_row_params& p = rc.p;
    const int lo0 = g.seg_lo;
    const int hi = seg == nseg - 1 ? a.V : lo0 + g.ntiles * TILE;      // the last segment takes the partial tile
    uint64_t* my = a.cand + slot_of(rc, seg) * CAP;
    if (ld_agent(a.dirty) != 0) return;                 // a dirty context: the merge samples the row alone
    if (seg == 0 && tid == 0) my[LS_STATUS] = 0ull;
    // Penalties: a repetition penalty alone as an exact bitmap of the window's ids over this segment (in s.ids, built
    // once for every pass), frequency / presence with the per-tile count table over the gathered window.
    const bool bmpen = rc.pen && rc.rep_on && !rc.fp_on && ((hi - lo0 + TILE - 1) / TILE) * TILE <= 32 * WIDS;
    if (bmpen) {
        uint32_t* bm = reinterpret_cast<uint32_t*>(s.ids);
        for (int i = tid; i < WIDS; i += BLOCK) bm[i] = 0u;
        __syncthreads();
        for (int64_t i = rc.b + tid; i < rc.len; i += BLOCK) {
            const int id = hist_at(a, rc, i);
            if (id >= lo0 && id < hi) atomicOr(&bm[(uint32_t)(id - lo0) >> 5], 1u << ((uint32_t)(id - lo0) & 31u));
        }
        __syncthreads();
    } else if (rc.pen) {
        gather_window(a, rc, lo0, hi, s);
    }
    // ---- P1: extremes, ordered count, coarse-bin counts of the k-th's search (k < V)
    const bool need_kth = rc.k < a.V;
    uint32_t* hc = reinterpret_cast<uint32_t*>(s.cand);  // [LB]
    if (need_kth) {
        for (int i = tid; i < LB; i += BLOCK) hc[i] = 0u;
        __syncthreads();
    }
    uint64_t cmax = 0ull, cmin = ~0ull;
    uint32_t nv = 0u;
    // Every token a candidate (k >= V): the logits within cut = CUT_C * T of the workgroup's running maximum (over its
    // tiles so far, the current one included) go to an LDS list; the others (masses below e^-CUT_C of the row's, since
    // the running maximum never exceeds the row's) are summed in single precision relative to that maximum, rescaled
    // when it rises. Both depend only on the data (a barrier per tile), so the sums are deterministic.
    const bool fastc = !need_kth;
    const float cut = CUT_C * p.temperature;
    const float inv_tl2 = 1.4426950408889634f / p.temperature;   // log2(e) / T: the rest's masses as powers of 2
    float ref = -__builtin_huge_valf();
    float tacc = 0.0f;
    constexpr uint32_t WREG = CAP / NWAVES;              // each wave's own part of the LDS list: no atomics
    uint64_t* const wl = s.cand + (tid / WAVE) * WREG;
    uint32_t wcnt = 0u;                                  // wave-uniform
    // (fastc: the extremes tracked as floats with their first / last index, as the composite order ranks ties)
    float bmax = -__builtin_huge_valf(), bmin = __builtin_huge_valf();
    int bmax_id = -1, bmin_id = -1;
    if (!fastc) {
        seg_elems(a, rc, s, lo0, hi, bmpen, [&](bool ok, float, uint32_t kq, uint64_t c) {
            if (ok) {
                cmax = c > cmax ? c : cmax;
                cmin = c < cmin ? c : cmin;
                ++nv;
                if (need_kth) atomicAdd(&hc[kq >> LB_SHIFT], 1u);
            }
        });
    } else {
        seg_elems_g(a, rc, s, lo0, hi, bmpen, [](bool, float, uint32_t, uint64_t) {}, [&](const float (&x)[TPT], int lo) {
            const bool full = lo + TILE <= hi;
            bool valid[TPT];
            float tm = -__builtin_huge_valf();
#pragma unroll
            for (int i = 0; i < TPT; ++i) {
                valid[i] = (full || elem_id(lo, i) < hi) && x[i] == x[i];
                tm = valid[i] && x[i] > tm ? x[i] : tm;
                nv += valid[i] ? 1u : 0u;
                if (valid[i] && x[i] <= bmin) { bmin = x[i]; bmin_id = elem_id(lo, i); }
                if (valid[i] && (x[i] > bmax || bmax_id < 0)) { bmax = x[i]; bmax_id = elem_id(lo, i); }
            }
            // the running maximum of the workgroup's tiles so far (this one included), behind a barrier
            uint32_t mk = wave_max(key_of(tm));
            uint32_t* tmw = s.tmx[((lo - lo0) / TILE) & 1];
            if (lane_id() == 0) tmw[tid / WAVE] = mk;
            __syncthreads();
#pragma unroll
            for (int w = 0; w < NWAVES; ++w) mk = tmw[w] > mk ? tmw[w] : mk;
            const float nr = mk > key_of(-__builtin_huge_valf()) ? val_of(mk) : -__builtin_huge_valf();
            if (nr > ref) {
                if (tacc != 0.0f) tacc *= __builtin_amdgcn_exp2f((ref - nr) * inv_tl2);
                ref = nr;
            }
            const float thr = ref - cut;
            uint32_t cm = 0u;
#pragma unroll
            for (int i = 0; i < TPT; ++i) {
                const bool cand = valid[i] && x[i] >= thr;
                cm |= cand ? 1u << i : 0u;
                const float t = __builtin_amdgcn_exp2f((x[i] - ref) * inv_tl2);
                tacc += (valid[i] && !cand) ? t : 0.0f;
            }
            if (__ballot(cm != 0u) != 0ull) {
#pragma unroll
                for (int i = 0; i < TPT; ++i) {
                    const bool cand = (cm >> i) & 1u;
                    const uint64_t m = __ballot(cand);
                    if (m != 0ull) {
                        const uint32_t pos = wcnt + mbcnt(m);
                        if (cand && pos < WREG) wl[pos] = comp_of(key_of(x[i]), (uint32_t)elem_id(lo, i));
                        wcnt += (uint32_t)__popcll(m);
                    }
                }
            }
        });
    }
    if (fastc) {
        cmax = bmax_id >= 0 ? comp_of(key_of(bmax), (uint32_t)bmax_id) : 0ull;
        cmin = bmin_id >= 0 ? comp_of(key_of(bmin), (uint32_t)bmin_id) : ~0ull;
    }
    FS_MARK(1);                                          // P1 streamed
    if (fastc && lane_id() == 0) s.wcnt[tid / WAVE] = wcnt;
    cmax = block_max_u64(cmax, s.red);
    cmin = block_min_u64(cmin, s.red);
    uint32_t nseg_v;
    (void)block_excl_scan<uint32_t>(nv, s.wsum, &nseg_v);
    if (fastc) {
        // the list cut again at this segment's maximum; its survivors to gather region 0 of the slot, their exact
        // masses and the rest's summed relative to that maximum
        // (the list's order depends on the waves' timing: its masses are summed in fixed point, order-free)
        uint32_t n0 = 0u, wofs[NWAVES];                   // (the reductions above end with barriers)
        bool wovf = false;
#pragma unroll
        for (int w = 0; w < NWAVES; ++w) {
            wofs[w] = n0;
            wovf |= s.wcnt[w] > WREG;
            n0 += s.wcnt[w];
        }
        const float smax = nseg_v > 0u ? val_of(comp_key(cmax)) : -__builtin_huge_valf();
        const double Td = (double)p.temperature;
        double tsum = 0.0;
        if (tacc != 0.0f) tsum = (double)tacc * exp((double)(ref - smax) / Td);
        uint64_t cfx = 0ull, tfx = 0ull;
        if (tid == 0) s.nfast = 0u;
        __syncthreads();
        if (!wovf && smax > -__builtin_huge_valf() && smax < __builtin_huge_valf()) {
            for (uint32_t b0 = 0u; b0 < n0; b0 += BLOCK) {
                const uint32_t i = b0 + (uint32_t)tid;
                int w = 0;
#pragma unroll
                for (int v = 1; v < NWAVES; ++v) w = i >= wofs[v] ? v : w;
                const uint64_t c = i < n0 ? s.cand[w * WREG + (i - wofs[w])] : 0ull;
                const float x = val_of(comp_key(c));
                const bool keep = i < n0 && x >= smax - cut;
                if (i < n0) {
                    const uint64_t m = (uint64_t)(mass_of(x, smax, Td) * CFXS + 0.5);
                    if (keep) cfx += m; else tfx += m;
                }
                wave_append(keep, c, my + LSC, &s.nfast, (uint32_t)LLR);
            }
        }
        uint64_t t_;
        (void)block_excl_scan<uint64_t>(cfx, s.red.u64b, &t_);
        const double csum = (double)t_ / CFXS;
        (void)block_excl_scan<uint64_t>(tfx, s.red.u64b, &t_);
        tsum = block_sum_f64(tsum, s.red) + (double)t_ / CFXS;
        if (tid == 0) {
            const bool ok = !wovf && s.nfast <= (uint32_t)LLR;
            my[LS_FN] = ok ? s.nfast : 0xFFFFFFFFull;
            my[LS_FC] = (uint64_t)__double_as_longlong(csum);
            my[LS_FT] = (uint64_t)__double_as_longlong(tsum);
        }
    }
    uint32_t* rh = a.rhist + (int64_t)row * RBINS;
    if (need_kth)
        for (int i = tid; i < LB; i += BLOCK)
            if (hc[i] != 0u) __hip_atomic_fetch_add(rh + i, hc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (tid == 0) { my[LS_MAX] = cmax; my[LS_MIN] = cmin; my[LS_NV] = nseg_v; }
    if (!row_sync(a, row, (uint32_t)nseg, s)) return;
    FS_MARK(5);                                          // past the first barrier
    if (fastc && nseg <= WAVE) {
        // wave 0 reads every segment's published line once: the row's extremes and count, and the cut's decision
        // (large_cut below, in wave reductions); segment 0's wave 0 then samples a short list at once
        if (tid < WAVE) {
            const int lane = tid;
            uint64_t smx = 0ull, smn = ~0ull, snv = 0ull, sfn = 0ull;
            double sfc = 0.0, sft = 0.0;
            if (lane < nseg) {
                const uint64_t* sl = a.cand + slot_of(rc, lane) * CAP;
                smx = sl[LS_MAX]; smn = sl[LS_MIN]; snv = sl[LS_NV]; sfn = sl[LS_FN];
                sfc = __longlong_as_double((long long)sl[LS_FC]);
                sft = __longlong_as_double((long long)sl[LS_FT]);
            }
            auto add_u = [](uint64_t x_, uint64_t y_) { return x_ + y_; };
            auto add_d = [](double x_, double y_) { return x_ + y_; };
            const uint64_t rmx = wave_max(smx), rmn = wave_min(smn), rnv = wave_allreduce(snv, add_u);
            const float mxf = val_of(comp_key(rmx));
            const bool fin = rnv != 0ull && mxf > -__builtin_huge_valf() && mxf < __builtin_huge_valf();
            const double Td = (double)p.temperature;
            const double F = fin && lane < nseg && snv != 0ull
                                 ? exp(((double)val_of(comp_key(smx)) - (double)mxf) / Td) : 0.0;
            const double sc = wave_allreduce(F * sfc, add_d), st = wave_allreduce(F * sft, add_d);
            const bool ovf = wave_max(sfn > (uint64_t)LLR ? 1u : 0u) != 0u;
            const uint64_t nft = wave_allreduce(sfn > (uint64_t)LLR ? 0ull : sfn, add_u);
            const double u = row_u(a, row);
            bool min_in = false;
            const bool fast = fin && cut_decide(p, sc, st, nft, ovf, u, min_in);
            bool done = false;
            if (fast && seg == 0 && nft <= (uint64_t)WAVE) {
                FS_MARK(6);
                if (!wave_cut_finish(a, rc, my, mxf, CUT_C * p.temperature, Td, st, (uint32_t)rnv, (int)rnv,
                                     comp_key(rmx), rmn, u, min_in, (uint32_t)sfn))
                    row_abandon(a, row);
                FS_MARK(8);
                done = true;
            }
            if (lane == 0) {
                s.red.u64[0] = rmx; s.red.u64b[0] = rmn; s.red.misc[0] = (uint32_t)rnv;
                s.red.misc[1] = (fast ? 1u : 0u) | (done ? 2u : 0u) | (min_in ? 4u : 0u);
                s.red.dmisc[0] = st; s.red.dmisc[1] = u;
            }
        }
        __syncthreads();
        cmax = s.red.u64[0]; cmin = s.red.u64b[0]; nv = s.red.misc[0];
        const uint32_t fl = s.red.misc[1];
        const double st = s.red.dmisc[0], u = s.red.dmisc[1];
        __syncthreads();                                 // Red is reused below
        if (fl & 1u) {
            if (seg == 0 && !(fl & 2u))
                cut_finish_block(a, rc, s, my, val_of(comp_key(cmax)), comp_key(cmax), cmin, nv, (int)nv, st, u,
                                 (fl & 4u) != 0u);
            return;
        }
    } else {
    // row-wide: extremes, count; the k-th's coarse bin from the row histogram
        uint64_t mx_ = 0ull, mn_ = ~0ull, nv_ = 0ull;
        for (int j = tid; j < nseg; j += BLOCK) {
            const uint64_t* sl = a.cand + slot_of(rc, j) * CAP;
            mx_ = sl[LS_MAX] > mx_ ? sl[LS_MAX] : mx_;
            mn_ = sl[LS_MIN] < mn_ ? sl[LS_MIN] : mn_;
            nv_ += sl[LS_NV];
        }
        cmax = block_max_u64(mx_, s.red);
        cmin = block_min_u64(mn_, s.red);
        uint64_t t_;
        (void)block_excl_scan<uint64_t>(nv_, s.red.u64b, &t_);
        nv = (uint32_t)t_;
    }
    const uint32_t ntot = nv;
    if (ntot == 0u) {                                    // every logit NaN: no order to sample from
        if (seg == 0 && tid == 0) { my[LS_TOK] = 0ull; my[LS_STATUS] = 1ull; }
        return;
    }
    const uint32_t kmax = comp_key(cmax);
    const float mx = val_of(kmax);
    const double Td = (double)p.temperature;
    const int keff = (uint32_t)rc.k < ntot ? rc.k : (int)ntot;
    if (fastc && nseg > WAVE && large_cut(a, rc, s, seg, my, mx, kmax, cmin, ntot, keff)) return;
    uint32_t bk = 0xFFFFFFFFu, abk = 0u;                 // the k-th's coarse bin (none: every element a candidate)
    if ((uint32_t)keff < ntot) {
        uint32_t cv[LPT];
#pragma unroll
        for (int j = 0; j < LPT; ++j) {
            const int b = LB - 1 - (LPT * tid + j);
            cv[j] = b <= (int)(0xFF800000u >> LB_SHIFT) ? rh[b] : 0u;   // the counters above the keys are not counts
        }
        const int dk = desc_locate<uint32_t>(cv, (uint32_t)keff, &abk, s.wsum, s);
        if (dk < 0) { row_abandon(a, row); return; }    // uniform (the counts disagree with ntot: never expected)
        bk = (uint32_t)(LB - 1 - dk);
    }
    // ---- P2: candidate masses above bk, bin bk gathered
    FS_MARK(6);                                          // P2 starts
    uint64_t* hm = reinterpret_cast<uint64_t*>(s.cand);  // [LB] fixed-point masses
    for (int i = tid; i < LB; i += BLOCK) hm[i] = 0ull;
    if (tid == 0) s.count = 0u;
    __syncthreads();
    // An element whose mass exp((v - mx) / T) is below e^-32 (1.3e-14) adds 0 to the fixed-point histogram (2^-44
    // units) and at most 262144 * 1.3e-14 to S (>= 1) altogether: it takes a single-precision exp (relative error
    // ~1e-7 of a negligible term) instead of the fp64 one, so S stays within ~1e-14 relative of the exact sum.
    double part = 0.0;
    float part_tiny = 0.0f;
    const float inv_tf = 1.0f / p.temperature;
    uint64_t* regA = my + LSC;
    seg_elems(a, rc, s, lo0, hi, bmpen, [&](bool ok, float x, uint32_t kq, uint64_t c) {
        const uint32_t b = kq >> LB_SHIFT;
        if (ok && (bk == 0xFFFFFFFFu || b > bk)) {
            const float d = x - mx;                      // fp32 subtraction, as ferro
            const float zf = d * inv_tf;
            if (!(zf < -32.0f)) {                    // (NaN, from inf - inf, stays on the exact path)
                const double m = exp((double)d / Td);
                part += m;
                atomicAdd(reinterpret_cast<unsigned long long*>(&hm[b]), (unsigned long long)(m * FXS + 0.5));
            } else {
                part_tiny += __expf(zf);
            }
        }
        wave_append(ok && b == bk, c, regA, &s.count, (uint32_t)LLR);
    });
    part += (double)part_tiny;
    FS_MARK(2);                                          // P2 streamed
    const double shi = block_sum_f64(part, s.red);      // its barriers also complete the LDS histogram
    uint64_t* rm = a.rmass + (int64_t)row * LB;
    for (int i = tid; i < LB; i += BLOCK)
        if (hm[i] != 0ull) __hip_atomic_fetch_add(rm + i, hm[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (tid == 0) {
        my[LS_SHI] = (uint64_t)__double_as_longlong(shi);
        my[LS_NBK] = s.count;
    }
    if (!row_sync(a, row, 2u * (uint32_t)nseg, s)) return;
    FS_MARK(7);                                          // past the second barrier
    double S = sum_slots_f64(a, rc, LS_SHI, s);
    uint64_t Xk = cmin;
    uint64_t fx_bk = 0ull;                               // fixed-point mass of bin bk's candidates
    if (bk != 0xFFFFFFFFu) {
        const int n = load_lists(a, rc, 0, LS_NBK, s);
        const int need = keff - (int)abk;                // >= 1: the k-th lies in bin bk
        if (n < need || need < 1) { row_abandon(a, row); return; }   // uniform
        Xk = s.cand[need - 1];
        double sb = 0.0;
        uint64_t fb = 0ull;
        for (int i = tid; i < need; i += BLOCK) {
            const double m = mass_of(val_of(comp_key(s.cand[i])), mx, Td);
            sb += m;
            fb += (uint64_t)(m * FXS + 0.5);
        }
        S += block_sum_f64(sb, s.red);
        uint64_t t_;
        (void)block_excl_scan<uint64_t>(fb, s.red.u64b, &t_);
        fx_bk = t_;
    }
    FS_MARK(3);                                          // past the second barrier: S and Xk known
    if (S != S) {                                        // an infinite maximum: every mass NaN, nothing cut, the
        if (seg == 0 && tid == 0) {                      // draw falls through to the last candidate (sampler.cpp:43-49)
            my[LS_TOK] = (uint64_t)comp_id(Xk) | ((uint64_t)(uint32_t)keff << 32);
            my[LS_XK] = Xk;
            my[LS_S] = (uint64_t)__double_as_longlong(S);
            my[LS_KEFF] = (uint64_t)keff | ((uint64_t)kmax << 32);
            my[LS_STATUS] = 1ull;
        }
        return;
    }
    const uint32_t kk = comp_key(Xk);
    uint64_t mv[LPT];                                    // the candidates' mass histogram, descending positions
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
        const int b = LB - 1 - (LPT * tid + j);
        mv[j] = rm[b] + ((uint32_t)b == bk ? fx_bk : 0ull);
    }
    // min-p: the smallest key whose pr reaches pr[0] * min_p (pr[0] = 1 / S): a search over keys, no pass
    uint64_t Xm = 0ull;
    uint32_t km = 0xFFFFFFFFu;
    if (p.min_p > 0.0f) {
        const double thr = (1.0 / S) * (double)p.min_p;
        auto okm = [&](uint32_t key) { return mass_of(val_of(key), mx, Td) / S >= thr; };
        if (!okm(kmax)) {
            Xm = cmax;
        } else {
            uint32_t lo = kk, h = kmax;
            while (lo < h) {
                const uint32_t mid = lo + ((h - lo) >> 1);
                if (okm(mid)) h = mid; else lo = mid + 1u;
            }
            km = lo;
            Xm = (uint64_t)lo << 32;
        }
    }
    const bool need_m = p.min_p > 0.0f && Xm != cmax;
    // ---- P3: top-p's crossing bin gathered, with min-p's counts and masses
    uint64_t Xc = 0ull;
    uint32_t keep_c = 0u, cnt_m = 0u;
    double tot_c = 0.0, sum_m = 0.0;
    uint64_t cl_m = ~0ull;
    int nc = -1;
    uint32_t bc = 0xFFFFFFFFu;
    uint32_t bd_pred = 0xFFFFFFFFu;                      // the draw's bin, when P3 can gather it too
    bool refined_c = false;                              // top-p's crossing bin was refined (gather region 2 in use)
    uint32_t nsync = 2u;
    if (p.top_p < 1.0f || need_m) {
        const double tgt = (double)p.top_p * S;
        double above_c = 0.0;
        if (p.top_p < 1.0f) {
            uint64_t abfx = 0ull;
            int dc = desc_locate<uint64_t>(mv, (uint64_t)(tgt * FXS), &abfx, s.red.u64b, s);
            if (dc < 0) dc = LB - 1 - (int)(kk >> LB_SHIFT);   // the total rounds below the target: the last bin
            bc = (uint32_t)(LB - 1 - dc);
            above_c = (double)abfx / FXS;
            if (p.min_p <= 0.0f) {
                // Without min-p the kept total lies in [tgt, min(S, tgt + the largest mass in bin bc)] (top-p keeps
                // through the crossing candidate, sampler.cpp:44). When the draw u * tot falls in one coarse bin over
                // that whole range, this pass gathers that bin too and no draw pass is needed.
                const uint32_t top_key = ((bc << LB_SHIFT) | ((1u << LB_SHIFT) - 1u)) < kmax
                                             ? ((bc << LB_SHIFT) | ((1u << LB_SHIFT) - 1u)) : kmax;
                const double mhi = mass_of(val_of(top_key), mx, Td);
                const double thi = tgt + mhi < S ? tgt + mhi : S;
                const double u0 = row_u(a, rc.row);
                uint64_t ab_;
                const int d0 = desc_locate<uint64_t>(mv, (uint64_t)(u0 * tgt * (1.0 - 1e-12) * FXS), &ab_, s.red.u64b, s);
                const int d1 = desc_locate<uint64_t>(mv, (uint64_t)(u0 * thi * (1.0 + 1e-12) * FXS), &ab_, s.red.u64b, s);
                if (d0 >= 0 && d0 == d1 && (uint32_t)(LB - 1 - d0) != bc) bd_pred = (uint32_t)(LB - 1 - d0);
            }
        }
        uint32_t my_ca = 0u, my_cm = 0u;
        double my_sm = 0.0;
        uint64_t my_cl = ~0ull;
        if (tid == 0) { s.count = 0u; s.tmax = 0u; }
        __syncthreads();
        uint64_t* regB = my + LSC + LLR;
        uint64_t* regC = my + LSC + 2 * LLR;
        seg_elems(a, rc, s, lo0, hi, bmpen, [&](bool ok, float x, uint32_t kq, uint64_t c) {
            const bool cand = ok && c >= Xk;
            if (cand && bc != 0xFFFFFFFFu && (kq >> LB_SHIFT) > bc) ++my_ca;
            if (cand && need_m && kq >= km) {
                ++my_cm;
                my_sm += mass_of(x, mx, Td);
                my_cl = c < my_cl ? c : my_cl;
            }
            wave_append(cand && (kq >> LB_SHIFT) == bc, c, regB, &s.count, (uint32_t)LLR);
            wave_append(cand && (kq >> LB_SHIFT) == bd_pred, c, regC, &s.tmax, (uint32_t)LLR);
        });
        uint32_t ca_t, cm_t;
        (void)block_excl_scan<uint32_t>(my_ca, s.wsum, &ca_t);
        (void)block_excl_scan<uint32_t>(my_cm, s.wsum, &cm_t);
        const double sm_t = block_sum_f64(my_sm, s.red);
        const uint64_t cl_t = block_min_u64(my_cl, s.red);
        if (tid == 0) {
            my[LS_NBC] = s.count;
            my[LS_CA] = ca_t;
            my[LS_CNTM] = cm_t;
            my[LS_SUMM] = (uint64_t)__double_as_longlong(sm_t);
            my[LS_CLM] = cl_t;
            my[LS_NBD] = s.tmax;
        }
        FS_MARK(8);                                      // P3 streamed
        nsync = 3u;
        if (!row_sync(a, row, 3u * (uint32_t)nseg, s)) return;
        FS_MARK(9);                                      // past the third barrier
        const uint32_t ca_c = (uint32_t)sum_slots_u64(a, rc, LS_CA, s);
        if (need_m) {
            cnt_m = (uint32_t)sum_slots_u64(a, rc, LS_CNTM, s);
            sum_m = sum_slots_f64(a, rc, LS_SUMM, s);
            uint64_t c_ = ~0ull;
            for (int j = tid; j < nseg; j += BLOCK) {
                const uint64_t v = a.cand[slot_of(rc, j) * CAP + LS_CLM];
                c_ = v < c_ ? v : c_;
            }
            cl_m = block_min_u64(c_, s.red);
        }
        if (p.top_p < 1.0f) {
            nc = load_lists(a, rc, 1, LS_NBC, s);
            if (nc < 0) {
                // a crowded crossing bin: one level of finer bins (its gather region is spent, and the draw's
                // pre-gathered bin is overwritten)
                uint64_t pk = 0ull;
                double cm = 0.0;
                uint32_t bf = 0u;
                if (!refine_bin(a, rc, s, seg, my, lo0, hi, bmpen, bc, Xk, above_c, tgt, mx, Td, nsync, pk, cm, bf)) {
                    row_abandon(a, row);
                    return;
                }
                Xc = pk;
                keep_c = ca_c + bf + 1u;
                tot_c = cm;
                bd_pred = 0xFFFFFFFFu;
                refined_c = true;
            } else {
                double cum = 0.0;
                const int ic = large_walk(s, nc, Xk, above_c, tgt, mx, Td, &cum);
                if (ic < 0) { row_abandon(a, row); return; }   // outside the bin's exact masses: the exact path
                Xc = s.cand[ic];
                keep_c = ca_c + (uint32_t)ic + 1u;
                tot_c = cum;
            }
        }
    }
    // the kept prefix: the largest of the three thresholds (sampler.cpp:43-44)
    uint64_t Xkeep = Xk, clast = Xk;
    uint32_t keep = (uint32_t)keff;
    double tot = S;
    if (p.min_p > 0.0f && Xm > Xkeep) {
        Xkeep = Xm;
        if (Xm == cmax) { keep = 1u; tot = 1.0; clast = cmax; }
        else { keep = cnt_m; tot = sum_m; clast = cl_m; }
    }
    if (p.top_p < 1.0f && Xc > Xkeep) {
        Xkeep = Xc;
        keep = keep_c;
        tot = tot_c;
        clast = Xc;
    }
    // ---- P4: the draw r = u * tot (sampler.cpp:45-49) in its coarse bin
    const double u = row_u(a, rc.row);
    const double r = u * tot + 0.0;
    if (!(r > 0.0)) {                                    // r = 0: ferro's first candidate (r <= pr[0], sampler.cpp:48)
        if (seg == 0 && tid == 0) {
            my[LS_TOK] = (uint64_t)comp_id(cmax) | ((uint64_t)keep << 32);
            my[LS_XK] = Xk;
            my[LS_S] = (uint64_t)__double_as_longlong(S);
            my[LS_KEFF] = (uint64_t)keff | ((uint64_t)kmax << 32);
            my[LS_STATUS] = 1ull;
        }
        return;
    }
    uint64_t abd = 0ull;
    const int dd = desc_locate<uint64_t>(mv, (uint64_t)(r * FXS), &abd, s.red.u64b, s);
    if (dd < 0) { row_abandon(a, row); return; }
    const uint32_t bd = (uint32_t)(LB - 1 - dd);
    int nd;
    if (nc >= 0 && bd == bc) {
        nd = nc;                                         // the same bin is sorted in LDS already
    } else if (bd == bd_pred) {
        nd = load_lists(a, rc, 2, LS_NBD, s);           // gathered by P3
    } else {
        // after a refinement of top-p's bin the other segments may still read gather region 2: region 1 instead
        // (its lists were never read), read through an invalidated L1 (its counts were)
        const int rg = refined_c ? 1 : 2;
        const int rs = refined_c ? LS_NBC : LS_NBD;
        if (tid == 0) s.count = 0u;
        __syncthreads();
        uint64_t* regC = my + LSC + rg * LLR;
        seg_elems(a, rc, s, lo0, hi, bmpen, [&](bool ok, float, uint32_t kq, uint64_t c) {
            wave_append(ok && c >= Xkeep && (kq >> LB_SHIFT) == bd, c, regC, &s.count, (uint32_t)LLR);
        });
        if (tid == 0) my[rs] = s.count;
        FS_MARK(10);                                     // P4 streamed
        ++nsync;
        if (!row_sync(a, row, nsync * (uint32_t)nseg, s)) return;
        FS_MARK(11);                                     // past the last barrier
        if (refined_c) l1_invalidate();
        nd = load_lists(a, rc, rg, rs, s);
    }
    uint64_t pick = 0ull;
    if (nd < 0) {                                        // a crowded draw bin: one level of finer bins
        double cm = 0.0;
        uint32_t bf = 0u;
        if (!refine_bin(a, rc, s, seg, my, lo0, hi, bmpen, bd, Xkeep, (double)abd / FXS, r, mx, Td, nsync, pick, cm,
                        bf)) {
            row_abandon(a, row);
            return;
        }
    } else {
        double cum = 0.0;
        const int id = large_walk(s, nd, Xkeep, (double)abd / FXS, r, mx, Td, &cum);
        if (id >= 0) {
            pick = s.cand[id];
        } else if (!(id == -2 && comp_key(Xkeep) >> LB_SHIFT == bd)) {
            row_abandon(a, row);                         // a rounding step at the bin edge: the exact path
            return;
        }
    }
    if (pick == 0ull) pick = clast;                      // past the last kept candidate
    if (seg == 0 && tid == 0) {
        my[LS_TOK] = (uint64_t)comp_id(pick) | ((uint64_t)keep << 32);
        my[LS_XK] = Xk;
        my[LS_S] = (uint64_t)__double_as_longlong(S);
        my[LS_KEFF] = (uint64_t)keff | ((uint64_t)kmax << 32);
        my[LS_STATUS] = 1ull;
    }
}

// ------------------------------------------------------------------------------------------------ row layout
// By default every row has nseg segments of seg_tiles tiles. With a.balance, each XCD splits its W workgroups among
// its R rows (x, x + XCDS, ...) by the rows' cost per tile, so that rows with a large k, which cost up to three
// times a greedy row per tile, get more segments and a mixed batch's rows finish together. Every workgroup of the
// XCD computes the same split from the same parameters with integer arithmetic. Costs (per tile, relative to a
// greedy row = 100; measured on MI355X on uniform B=256 x V=262144 batches): k = 64 119, k = 256 158, k = 2048
// 292, whole-row sampling (k > 2048) about 400; frequency/presence penalties x1.25, a repetition penalty x1.05.
// What the cost needs of a row's parameters: two 16-byte buffer loads (temperature, top_k, top_p, min_p; repetition,
// frequency, presence, repeat_last_n). A segment workgroup requests them before its first tiles, behind a scheduling
// barrier, so that waiting for them (vector loads complete in order) does not wait for the tiles.
struct CostIn {
    float t, rep, fq, pr;
    int tk;
};
__device__ __forceinline__ CostIn cost_in(const Args& a, int row) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<fs_row_params*>(a.params), (short)0,
                                                                        a.B * (int)sizeof(fs_row_params), 0x00020000);
    const u32x4 lo = raw_buffer_load_u32x4(rs, row * (int)sizeof(fs_row_params), 0, 0);
    const u32x4 hi = raw_buffer_load_u32x4(rs, row * (int)sizeof(fs_row_params) + 16, 0, 0);
    CostIn c;
    c.t = __uint_as_float(lo.x); c.tk = (int)lo.y;
    c.rep = __uint_as_float(hi.x); c.fq = __uint_as_float(hi.y); c.pr = __uint_as_float(hi.z);
    return c;
}
__device__ __forceinline__ uint32_t row_cost(const Args& a, const CostIn& in) {
    const float t = in.t, rep = in.rep, fq = in.fq, pr = in.pr;
    const int tk = in.tk;
    if (t <= 0.0f || tk == 1) return 100u;
    const int k = (tk > 0 && tk < a.V) ? tk : a.V;
    float c;
    if (k > KMAX) {
        c = 400.0f;
    } else {
        const float l = __log2f((float)k);
        c = k <= 64 ? 100.0f + 3.0f * l : (k <= 256 ? 119.0f + 19.5f * (l - 6.0f) : 158.0f + 44.7f * (l - 8.0f));
    }
    if (fq != 0.0f || pr != 0.0f) c *= 1.25f;
    else if (rep != 1.0f) c *= 1.05f;
    return (uint32_t)c;
}
// Lane r < R: row x + XCDS * r gets n segments (at most its tiles), its first workgroup being base among the XCD's W.
// in: lane r's row parameters (cost_in of row x + XCDS * r, or of row x past R).
__device__ __forceinline__ CostIn xcd_cost_in(const Args& a, int x) {
    const int R = (a.B - x + XCDS - 1) / XCDS;
    return cost_in(a, x + XCDS * (lane_id() < R ? lane_id() : 0));
}
__device__ __forceinline__ void xcd_layout(const Args& a, int x, const CostIn& in, uint32_t& n, uint32_t& base) {
    const int lane = lane_id();
    const int R = (a.B - x + XCDS - 1) / XCDS;          // rows on this XCD (1 <= R <= WAVE: the host checks B)
    const uint32_t W = (uint32_t)(a.nseg * ((a.B + XCDS - 1) / XCDS));
    const uint32_t tiles_row = (uint32_t)(a.V / TILE);
    const uint32_t w = lane < R ? row_cost(a, in) : 0u;  // lane r: row x + XCDS r's cost
    const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_scan_u32(w), WAVE - 1);
    const uint32_t spare = W - (uint32_t)R;
    const uint32_t num = spare * w;
    const uint32_t tq = tot > 0u ? tot : 1u;            // >= 100 per row
    const uint32_t f = num / tq, rem = num % tq;
    n = lane < R ? 1u + f : 0u;
    const uint32_t left = W - (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_scan_u32(n), WAVE - 1);
    uint32_t rank = 0u;                                  // the largest remainders get the leftover workgroups
    for (int s2 = 0; s2 < R; ++s2) {
        const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)rem, s2);
        rank += (r2 > rem || (r2 == rem && s2 < lane)) ? 1u : 0u;
    }
    if (lane < R && rank < left) n += 1u;
    const uint32_t cap = tiles_row < (uint32_t)(BLOCK - 1) ? tiles_row : (uint32_t)(BLOCK - 1);
    if (n > cap) n = cap;                                // workgroups past a row's tiles stay idle
    base = wave_incl_scan_u32(n) - n;
}
// The layout of row x + XCDS * q into rc (merging workgroups): its lane q of xcd_layout.
__device__ __forceinline__ void row_layout(const Args& a, RowCtx& rc) {
    if (!a.balance || rc.nseg == 0) return;
    uint32_t n, base;
    xcd_layout(a, rc.lx, xcd_cost_in(a, rc.lx), n, base);
    const int q = rc.row / XCDS;
    const uint32_t nq = (uint32_t)__builtin_amdgcn_readlane((int)n, q);
    const uint32_t st = ((uint32_t)(a.V / TILE) + nq - 1u) / nq;
    rc.st = (int)st;
    rc.nseg = (int)(((uint32_t)(a.V / TILE) + st - 1u) / st);
    rc.lbase = __builtin_amdgcn_readlane((int)base, q);
}

// The row's completion counter: the row histogram's last bin, which no ordered key reaches (keys of non-NaN values
// are at most +inf's, bin 4088). Segments add 1 (an L2 atomic); the merge role polls it.
__device__ __forceinline__ uint32_t* row_counter(const Args& a, int row) {
    return a.rhist + (int64_t)row * RBINS + (RBINS - 1);
}
static_assert(((0xFF800000u >> RSHIFT) < (uint32_t)(RBINS - 1)), "the counter bin lies above every ordered key");
constexpr uint32_t MERGE_SPINS = 1u << 20;   // bounded wait of the merge role (far above any segment's time)

// Merge role of the segment grid: one workgroup per row, placed after the segments on the row's XCD (slot x of
// the last XCDS * ceil(B / XCDS) workgroups merges rows x, x + XCDS, ...). Workgroups are dispatched in index
// order, so the row's segments are running or done when it starts: it waits for their count (an atomic that
// is not idempotent, so it executes in the L2 and is never folded into an L1-served load), invalidates its L1
// and reads the lists from the L2. The wait is bounded (a.merge_spins polls): past it FS_DEVERR_INTERNAL is
// raised, the context is marked dirty and the row is computed from its logits alone (exact, one workgroup); a
// dirty context computes every row that way until fs_device_error clears the workspace.
__device__ __forceinline__ void merge_role(const Args& a, int mi, Shared& s) {
    const int row = mi % XCDS + XCDS * (mi / XCDS);
    if (row >= a.B) return;
    FS_TAG(13, 2); FS_TAG(14, row); FS_TAG(15, 0);
    RowCtx rc = row_ctx(a, row);                     // the row's inputs are read while the segments run
    row_layout(a, rc);
    decode_hist_copy(a, row);                        // a decode step: while the segments run
    uint32_t* ctr = row_counter(a, row);
    if (threadIdx.x == 0) {
        // A context left dirty by an earlier give-up: its row histograms and counters may hold a late segment's
        // additions, so no segment output is trusted and the row is computed from its logits alone. Otherwise a
        // bounded wait for the row's segments; past it the context is marked dirty (a segment that finishes later
        // still adds to this row's counter and histogram) and this row, too, is computed alone.
        uint32_t alone = ld_agent(a.dirty) != 0 ? 1u : 0u;
        uint32_t spins = 0u;
        while (!alone && (a.merge_spins == 0u ||
                          (__hip_atomic_fetch_add(ctr, 0x10000u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) &
                           0xFFFFu) < (uint32_t)rc.nseg)) {
            if (++spins >= a.merge_spins) {
                atomicOr(a.err, FS_DEVERR_INTERNAL);
                __hip_atomic_store(a.dirty, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                // err[2..3]: the address of a host-mapped flag that the next call reads on the host (or 0)
                int32_t* hf = (int32_t*)ld_agent(reinterpret_cast<const uint64_t*>(a.err + 2));
                if (hf) __hip_atomic_store(hf, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                alone = 1u;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        s.misc_alone = alone;
    }
    FS_MARK(1);
    __syncthreads();
    const bool alone = s.misc_alone != 0u;
    Pre pre = {};
    if (!alone) {
        l1_invalidate();
        prefetch_lists(a, rc, pre);
        if (threadIdx.x == 0) *ctr = 0u;             // the bin is left at 0 with the rest of the row histogram
    }
    merge_row(a, rc, s, pre, alone);                 // one call site: the merge code is inlined once
}

// Segment kernel: one (row, segment) item per workgroup (rows sampled with k > KMAX only count themselves done),
// then the merge role.
// The fields a workgroup needs first come as separate leading parameters: gfx950 preloads those into SGPRs at
// wave launch (build flag -amdgpu-kernarg-preload-count), so the first tile loads wait for no argument load.
__global__ __launch_bounds__(BLOCK, 4) void segment_kernel(const float* logits, int64_t ld, int B, int V, int nseg,
                                                           int seg_tiles, const fs_row_params* params,
                                                           const int64_t* hist_off, Args a) {
    static_assert(KMAX + TILE <= CAP, "a compacted buffer plus one tile must fit the candidate buffer");
    __shared__ __align__(16) Shared s;
    a.logits = logits; a.ld = ld; a.B = B; a.V = V; a.nseg = nseg; a.seg_tiles = seg_tiles; a.params = params;
    a.hist_off = hist_off;
    // One (row, segment) item per workgroup. Workgroup i runs on XCD i % XCDS (round-robin dispatch): slot
    // x = i % XCDS takes the rows x, x + XCDS, ..., all segments of a row in consecutive rounds, so a row's segments
    // share one XCD and its L2 (the row histogram). Slots past the last row return at once.
    const unsigned seg_grid = (unsigned)(XCDS * a.nseg * ((a.B + XCDS - 1) / XCDS));
    FS_MARK(0);
    for (int i_ = 1; i_ < 13; ++i_) FS_TAG(i_, 0);
    FS_TAG(13, 0);
    if (blockIdx.x >= seg_grid) {
        merge_role(a, (int)(blockIdx.x - seg_grid), s);
        FS_MARK(4);
        FS_FLUSH();
        return;
    }
    const int x = (int)(blockIdx.x % (unsigned)XCDS);
    const int j = (int)(blockIdx.x / (unsigned)XCDS);
    int q = __builtin_amdgcn_readfirstlane(j / a.nseg);          // uniform: lets the compiler use scalar loads
    int seg = j - q * a.nseg;
    int row = x + XCDS * q;
    if (row >= a.B && !a.balance) return;
    float buf[PF][TPT];
    // the layout's parameter loads come first, then the default layout's tiles, then the row's parameters; a balanced
    // layout that moves this workgroup requests its own tiles and parameters
    CostIn cin = {};
    if (a.balance) cin = xcd_cost_in(a, x);
    __builtin_amdgcn_sched_barrier(0);
    SegStart g = a.balance ? seg_start<true>(a, row < a.B ? row : a.B - 1, seg, a.seg_tiles, buf)
                           : seg_start<false>(a, row < a.B ? row : a.B - 1, seg, a.seg_tiles, buf);
    RowCtx rc = row_ctx(a, row < a.B ? row : a.B - 1);
    int st = a.seg_tiles, nsr = a.nseg, lbase = q * a.nseg;
    if (a.balance) {
        uint32_t n, base;
        xcd_layout(a, x, cin, n, base);
        const uint64_t mine = __ballot((uint32_t)j >= base && (uint32_t)j < base + n);
        if (mine == 0ull) return;                        // past the XCD's rows (or a capped row's tiles): idle
        const int r = __ffsll((unsigned long long)mine) - 1;
        const uint32_t nr = (uint32_t)__builtin_amdgcn_readlane((int)n, r);
        lbase = __builtin_amdgcn_readlane((int)base, r);
        st = (int)(((uint32_t)(a.V / TILE) + nr - 1u) / nr);
        nsr = (a.V / TILE + st - 1) / st;
        const int nseg_r = __builtin_amdgcn_readfirstlane(j - lbase);
        if (nseg_r >= nsr) return;                       // the row's tiles are covered by its first nsr workgroups
        if (r != q || nseg_r != seg || st != a.seg_tiles) {
            const bool moved_row = r != q || row >= a.B;
            q = r;
            seg = nseg_r;
            row = x + XCDS * q;
            g = seg_start(a, row, seg, st, buf);
            if (moved_row) rc = row_ctx(a, row);
        }
    }
    FS_TAG(13, 1); FS_TAG(14, row); FS_TAG(15, seg);
    rc.st = st;
    rc.nseg = nsr;
    rc.lbase = lbase;
    if (!rc.large) process_segment(a, rc, seg, s, buf, g);
    else large_segment(a, rc, seg, s, g);           // the row's segments sample it together
    vm_drain();                                      // the list and meta stores are in the L2
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(row_counter(a, row), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    FS_MARK(4);
    FS_FLUSH();
}

// Merge kernel: one workgroup per row, for rows shorter than one tile (no segments; the segment lists are requested
// first, so their latency overlaps the row's parameter loads), or, with `alone`, every row sampled from its logits by
// one workgroup (a device whose XCD layout the segment grid's hand-off cannot rely on).
__global__ __launch_bounds__(BLOCK) void merge_kernel(int nseg, uint64_t* cand, uint32_t* meta, uint32_t* rhist,
                                                      const fs_row_params* params, int alone, Args a) {
    static_assert(2 * SMALL * 8 <= NBINS * 4, "rank-sort buffers alias the histogram");
    __shared__ __align__(16) Shared s;
    a.nseg = nseg; a.cand = cand; a.meta = meta; a.rhist = rhist; a.params = params;
    const int row = __builtin_amdgcn_readfirstlane((int)blockIdx.x);
    Pre pre = {};
    const RowCtx rc = row_ctx(a, row);
    if (!alone) prefetch_lists(a, rc, pre);
    decode_hist_copy(a, row);
    merge_row(a, rc, s, pre, alone != 0);
}

// fs_softcap_batch: the sampler's fused final-logit cap as a standalone elementwise pass.
__global__ __launch_bounds__(256) void softcap_kernel(const float* in, float* out, int64_t n, float cap) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        out[i] = softcap_one(in[i], cap);
}

// In-place penalty pass (fs_penalize_batch): ferro's sample() leaves its host row penalised (sampler.cpp:11-18),
// and a caller that reads the row back afterwards (lm_cli.cpp:353) sees those values. One workgroup per
// (row, 8192-id chunk): the window's ids that fall in the chunk are counted in a 16-bit LDS table, then every
// counted logit is rewritten once with the same arithmetic as the sampling kernels.
constexpr int PEN_BLOCK = 256;
constexpr int PEN_CHUNK = 8192;

__global__ __launch_bounds__(PEN_BLOCK) void penalize_kernel(float* logits, int64_t ld, int V, const int32_t* hist,
                                                            const int64_t* hist_off, const fs_row_params* params,
                                                            int nchunk, int32_t* err) {
    __shared__ uint32_t cnt[PEN_CHUNK / 2];
    const int tid = threadIdx.x;
    const int row = (int)blockIdx.x / nchunk;
    const int lo = ((int)blockIdx.x - row * nchunk) * PEN_CHUNK;
    const fs_row_params p = ld_const(params + row);
    const bool rep_on = p.repetition_penalty != 1.0f;
    const bool fp_on = p.frequency_penalty != 0.0f || p.presence_penalty != 0.0f;
    if (!(rep_on || fp_on) || p.repeat_last_n == 0 || !hist || !hist_off) return;
    const int64_t h0 = ld_const(hist_off + row);
    const int64_t len = ld_const(hist_off + row + 1) - h0;
    const int64_t b = window_begin(len, p);
    if (b >= len) return;
    for (int i = tid; i < PEN_CHUNK / 2; i += PEN_BLOCK) cnt[i] = 0u;
    __syncthreads();
    bool ovf = false;
    for (int64_t i = b + tid; i < len; i += PEN_BLOCK) {
        const int id = hist[h0 + i];
        const uint32_t rel = (uint32_t)(id - lo);
        if (id >= 0 && id < V && rel < (uint32_t)PEN_CHUNK) {
            const uint32_t sh = (rel & 1u) * 16u;
            const uint32_t old = atomicAdd(&cnt[rel >> 1], 1u << sh);
            ovf |= ((old >> sh) & 0xFFFFu) == 0xFFFFu;
        }
    }
    if (ovf) atomicOr(err, FS_DEVERR_COUNT_OVERFLOW);
    __syncthreads();
    float* rowp = logits + (int64_t)row * ld + lo;
    for (int i = tid; i < PEN_CHUNK / 2; i += PEN_BLOCK) {
        const uint32_t c2 = cnt[i];
        if (c2 == 0u) continue;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint32_t c = (c2 >> (16 * q)) & 0xFFFFu;
            if (c != 0u) {                                  // a counted id is < V
                float l = rowp[2 * i + q];
                if (rep_on) l = l > 0.0f ? __fdiv_rn(l, p.repetition_penalty) : __fmul_rn(l, p.repetition_penalty);
                if (fp_on) l = __fsub_rn(l, __fadd_rn(__fmul_rn((float)c, p.frequency_penalty), p.presence_penalty));
                rowp[2 * i + q] = l;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------ prompt lookup
// Prompt-lookup drafting (server.cpp:552-564), one workgroup per stream: for n = min(4, L-1) down to min_n, every
// thread tests its positions p for h[p, p+n) == the history's last n tokens with a non-eos token after the match
// (the reference skips a match whose continuation is empty); the largest such p (the most recent occurrence) wins,
// and the tokens after it, up to kmax and stopping before eos, are the draft.
constexpr int LD_BLOCK = 256;

// History append (the per-stream hist.push_back of each consumed token, server.cpp:342, as the decode loop at
// server.cpp:603-606 and the verify window at server.cpp:627-637 feed them), on CSR histories and out of place: stream
// s keeps its old ids and gains tok[row_off[s] + i], i < n_s, where n_s is count[s] (NULL: 1) clamped to its rows
// [0, row_off[s+1] - row_off[s]]. The new offsets are old (rebased to 0) + the exclusive prefix of the n_s.
__device__ __forceinline__ int64_t app_n(const int64_t* row_off, const int32_t* count, int s, bool* bad) {
    const int64_t r0 = row_off ? row_off[s] : (int64_t)s;
    const int64_t nr = row_off ? row_off[s + 1] - r0 : 1;
    int64_t n = count ? (int64_t)count[s] : 1;
    if (n < 0 || n > nr) {
        *bad = true;
        n = n < 0 ? 0 : nr;
    }
    return n;
}

// One workgroup: the new offsets, streams in chunks of BLOCK (carry in int64).
__global__ __launch_bounds__(BLOCK) void hist_offsets_kernel(int S, const int64_t* hist_off, const int64_t* row_off,
                                                             const int32_t* count, int64_t* out_off, int64_t out_cap,
                                                             int32_t* err) {
    __shared__ uint32_t wsum[NWAVES];
    const int tid = threadIdx.x;
    const int64_t h0 = hist_off[0];
    int64_t carry = 0;
    bool bad = false;
    for (int c0 = 0; c0 < S; c0 += BLOCK) {
        const int s = c0 + tid;
        const uint32_t n = s < S ? (uint32_t)app_n(row_off, count, s, &bad) : 0u;
        uint32_t tot;
        const uint32_t ex = block_excl_scan<uint32_t>(n, wsum, &tot);
        if (s < S) out_off[s] = hist_off[s] - h0 + carry + ex;
        carry += tot;
        __syncthreads();                                 // wsum is reused by the next chunk
    }
    if (tid == 0) {
        const int64_t end = hist_off[S] - h0 + carry;
        out_off[S] = end;
        if (end > out_cap) atomicOr(err, FS_DEVERR_HIST_APPEND);
    }
    if (bad) atomicOr(err, FS_DEVERR_HIST_APPEND);
}

// One workgroup per stream: its old ids, then its appended tokens (positions >= out_cap are not written).
__global__ __launch_bounds__(LD_BLOCK) void hist_append_kernel(const int32_t* hist, const int64_t* hist_off,
                                                               const int32_t* tok, const int64_t* row_off,
                                                               const int32_t* count, const int64_t* out_off,
                                                               int32_t* out, int64_t out_cap) {
    const int s = (int)blockIdx.x;
    bool bad = false;
    const int64_t n = app_n(row_off, count, s, &bad);
    const int64_t a = hist_off[s], L = hist_off[s + 1] - a;
    const int64_t o = out_off[s];
    const int64_t r0 = row_off ? row_off[s] : (int64_t)s;
    for (int64_t i = threadIdx.x; i < L + n; i += LD_BLOCK) {
        const int64_t d = o + i;
        if (d < out_cap) out[d] = i < L ? hist[a + i] : tok[r0 + (i - L)];
    }
}

__global__ __launch_bounds__(LD_BLOCK) void lookup_draft_kernel(const int32_t* hist, const int64_t* hist_off,
                                                                const int32_t* kmax_arr, const int32_t* min_n_arr,
                                                                int eos, int32_t* draft, int draft_ld,
                                                                int32_t* ndraft) {
    __shared__ int64_t wbest[LD_BLOCK / WAVE];
    const int st = (int)blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t h0 = hist_off[st];
    const int64_t L = hist_off[st + 1] - h0;
    const int32_t* h = hist + h0;
    int kmax = kmax_arr ? kmax_arr[st] : draft_ld;
    kmax = kmax < draft_ld ? kmax : draft_ld;
    const int min_n = min_n_arr ? min_n_arr[st] : 2;
    int d = 0;
    for (int64_t n = (L - 1 < 4 ? L - 1 : 4); n >= min_n && kmax > 0; --n) {
        int32_t t[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) t[q] = q < n ? h[L - n + q] : 0;
        int64_t best = -1;
        for (int64_t p = tid; p <= L - n - 1; p += LD_BLOCK) {
            bool eq = true;
#pragma unroll
            for (int q = 0; q < 4; ++q) eq = eq && (q >= n || h[p + q] == t[q]);
            if (eq && h[p + n] != eos) best = p;               // p grows: the last hit is this thread's largest
        }
        best = wave_max(best);
        if (lane_id() == 0) wbest[tid / WAVE] = best;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < LD_BLOCK / WAVE; ++w) best = wbest[w] > best ? wbest[w] : best;
        __syncthreads();
        if (best >= 0) {
            if (tid == 0)
                for (int64_t k = best + n; k < L && d < kmax; ++k) {
                    if (h[k] == eos) break;
                    draft[(int64_t)st * draft_ld + d++] = h[k];
                }
            break;
        }
    }
    if (tid == 0) ndraft[st] = d;
}

// ------------------------------------------------------------------------------------------------ draw streams
// std::mt19937_64 (the standard's parameters: n = 312, m = 156, r = 31, a = 0xB5026F5AA96619E9, tempering
// u = 29 / d = 0x5555555555555555, s = 17 / b = 0x71D67FFFEDA60000, t = 37 / c = 0xFFF7EEE000000000, l = 43) per
// stream, and libstdc++'s generate_canonical<double, 53> of one 64-bit output: (double)x / 2^64, kept below 1.
// This is ferro::Sampler's draw (sampler.h:25,32; sampler.cpp:45-46) moved next to the sampler.

// One thread per stream. Stream s owns rows row_off[s] .. row_off[s+1]-1 (row_off NULL: row s alone); each row
// whose stream samples takes one draw, in row order; greedy streams take none and get u = 0. peek != 0 leaves the
// state unchanged (the draws are computed from it: at most MT_M draws past a twist).
__global__ __launch_bounds__(64) void drng_draw_kernel(uint64_t* mts, int32_t* idxs, int n_streams,
                                                       const int64_t* row_off, const fs_row_params* params,
                                                       double* u, int peek, int32_t* err) {
    const int sidx = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (sidx >= n_streams) return;
    uint64_t* mt = mts + (int64_t)sidx * MT_N;
    int idx = idxs[sidx];
    const int64_t r0 = row_off ? row_off[sidx] : sidx;
    const int64_t r1 = row_off ? row_off[sidx + 1] : sidx + 1;
    const bool smp = samples(params[sidx]);
    for (int64_t r = r0; r < r1; ++r) {
        if (!smp) { u[r] = 0.0; continue; }
        uint64_t y;
        if (!peek) {
            if (idx >= MT_N) { mt_twist(mt); idx = 0; }
            y = mt[idx++];
        } else {
            if (idx < MT_N) {
                y = mt[idx++];
            } else {
                const int k = idx - MT_N;                    // the k-th value of the next twist, from the old state
                if (k >= MT_M) { atomicOr(err, FS_DEVERR_INTERNAL); u[r] = 0.0; continue; }
                y = mt_twist_one(mt[k], mt[k + 1], mt[k + MT_M]);
                ++idx;
            }
        }
        u[r] = mt_canonical(mt_temper(y));
    }
    if (!peek) idxs[sidx] = idx;
}

// Advance stream s by counts[s] draws, or, for a stream that does not sample, by none.
__global__ __launch_bounds__(64) void drng_skip_kernel(uint64_t* mts, int32_t* idxs, int n_streams,
                                                       const int32_t* counts, const fs_row_params* params) {
    const int sidx = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (sidx >= n_streams || !samples(params[sidx])) return;
    uint64_t* mt = mts + (int64_t)sidx * MT_N;
    int idx = idxs[sidx];
    for (int32_t c = counts[sidx]; c > 0;) {
        if (idx >= MT_N) { mt_twist(mt); idx = 0; }
        const int take = MT_N - idx < c ? MT_N - idx : c;
        idx += take;
        c -= take;
    }
    idxs[sidx] = idx;
}

// ------------------------------------------------------------------------------------------------ small-k kernel
// A separate kernel for batches whose every row is greedy or samples from k <= SK_K candidates with at most a
// repetition penalty (no frequency / presence counts) - the serving batches of ferro's decode loop (server.cpp:603-606:
// top-k 40-64 on every row). The host picks it from a host copy of the parameters (fs_sample_batch_hp). It has its own
// register budget (it shares no code path with the fused kernel above), which lets it stream a row differently:
//   - one workgroup of SK_LT threads per (row, segment): every load of the segment (NL float4 per thread) is issued at
//     once, so the whole batch is requested at the start. The memory system serves the requests roughly in dispatch
//     order, so a row's segments (consecutive workgroups) receive their data together, and rows finish one after
//     another: the merge of an early row overlaps the streaming of later rows;
//   - per group of four logits only a maximum and, later, one compare: the bound is the ceil(k / waves)-th largest
//     lane maximum of each wave, the smallest over the waves (each lane maximum is a distinct logit of the segment, so
//     at least k logits of the segment reach it). Groups whose maximum reaches it are written to LDS, expanded to the
//     candidates at or above it (about 1.5 k per segment on heavy-tailed rows), and sorted exactly into the segment's
//     top k by a bitonic network in registers (DPP and permlane moves: no LDS round trips);
//   - the last segment of a row to finish (an L2 ticket) merges the row's sorted lists by a tree of bitonic merges and
//     finishes the row in one wave (softmax at temperature, min-p, top-p, draw: the merge path's wave_softmax).
// A segment with more than SK_CAP candidates (ties at its bound) selects its exact top k by a radix select over the
// composites held in registers instead (slow, exact).
constexpr int SK_LT = 256;                 // threads per segment workgroup
constexpr int SK_NW = SK_LT / WAVE;
constexpr int SK_K = 64;                   // largest k (one candidate per lane of the finishing wave)
constexpr int SK_GCAP = 128;               // groups of four a wave can hand to the expansion
constexpr int SK_CAP = 512;                // candidates a segment ranks in LDS
constexpr int SK_MAX_SEGS = 64;            // segments per row

struct SkArgs {
    const float* logits;
    int64_t ld;
    int B, V, nseg;
    const int32_t* hist;
    const int64_t* hist_off;
    const fs_row_params* params;
    const double* u;
    int32_t* tok;
    int kcap;
    int32_t* cand_ids;
    double* cand_probs;
    int32_t* keep;
    uint64_t* lists;                       // [B * nseg][SK_K]: each segment's top k, sorted, 0-padded
    uint32_t* ticket;                      // [B]: segments finished (left at 0)
    int32_t* err;
    uint64_t* trace;                       // FS_TRACE builds: per-workgroup phase timestamps (NULL: none)
    // verification windows (mode MODE_VERIFY; the host sends only windows without an active penalty here)
    int mode;
    const int32_t* rows;                   // token fed at each row
    const int64_t* row_off;                // stream -> rows
    int n_streams, eos;
    int32_t* accepted;
    uint32_t* stream_cnt;                  // [3 n_streams]: 64-bit counts + stop bits, 32-bit counts (left at 0)
    // a decode step (fs_decode_step_hp; NULL otherwise): draw streams and the histories with the tokens appended
    uint64_t* dmt;
    int32_t* didx;
    int32_t* out_hist;
    int64_t* out_hist_off;
    int64_t out_cap;
};

// lane ^ D over the wave, in the VALU: DPP for D < 16 (both shifts in full exec, then an arithmetic select: a branch
// would run each DPP move on half the lanes), permlane swaps for 16 and 32 (gfx950)
template <int D>
__device__ __forceinline__ uint32_t xor_lane32(uint32_t v) {
    if constexpr (D == 1) {
        return dpp32<0xB1>(v);                                  // quad_perm [1,0,3,2]
    } else if constexpr (D == 2) {
        return dpp32<0x4E>(v);                                  // quad_perm [2,3,0,1]
    } else if constexpr (D == 4 || D == 8) {
        const uint32_t up = dpp32<0x100 + D>(v), dn = dpp32<0x110 + D>(v);   // row_shl: lane + D; row_shr: lane - D
        const uint32_t m = 0u - (((uint32_t)lane_id() / D) & 1u);
        return up ^ ((up ^ dn) & m);
    } else if constexpr (D == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane_id() & 16) ? r[0] : r[1];
    } else {
        static_assert(D == 32, "xor distances 1..32");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane_id() & 32) ? r[0] : r[1];
    }
}
template <int D>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v) {
    return ((uint64_t)xor_lane32<D>((uint32_t)(v >> 32)) << 32) | (uint64_t)xor_lane32<D>((uint32_t)v);
}
// Bitonic compare-exchange at distance D: the lane keeps the larger of its pair iff (its bit D is clear) == up.
template <int D>
__device__ __forceinline__ uint64_t bcx(uint64_t v, bool up) {
    const uint64_t o = xor_lane64<D>(v);
    const bool keep_max = ((lane_id() & D) == 0) == up;
    return keep_max ? (v > o ? v : o) : (v < o ? v : o);
}
// 32-bit compare-exchange and descending sort of the wave's 64 values (lane 0 the largest), VALU only.
template <int D>
__device__ __forceinline__ uint32_t bcx32(uint32_t v, bool up) {
    const uint32_t o = xor_lane32<D>(v);
    const bool keep_max = ((lane_id() & D) == 0) == up;
    const uint32_t hi = v > o ? v : o, lo = v > o ? o : v;
    return keep_max ? hi : lo;
}
__device__ __forceinline__ uint32_t sort64_desc_u32(uint32_t v) {
    const int lane = lane_id();
    { const bool up = (lane & 2) == 0; v = bcx32<1>(v, up); }
    { const bool up = (lane & 4) == 0; v = bcx32<2>(v, up); v = bcx32<1>(v, up); }
    { const bool up = (lane & 8) == 0; v = bcx32<4>(v, up); v = bcx32<2>(v, up); v = bcx32<1>(v, up); }
    { const bool up = (lane & 16) == 0;
      v = bcx32<8>(v, up); v = bcx32<4>(v, up); v = bcx32<2>(v, up); v = bcx32<1>(v, up); }
    { const bool up = (lane & 32) == 0;
      v = bcx32<16>(v, up); v = bcx32<8>(v, up); v = bcx32<4>(v, up); v = bcx32<2>(v, up); v = bcx32<1>(v, up); }
    v = bcx32<32>(v, true); v = bcx32<16>(v, true); v = bcx32<8>(v, true); v = bcx32<4>(v, true);
    v = bcx32<2>(v, true);
    return bcx32<1>(v, true);
}

// The wave's 64 values sorted, descending (lane 0 the largest) or ascending.
template <bool DESC>
__device__ __forceinline__ uint64_t sort64(uint64_t v) {
    const int lane = lane_id();
    { const bool up = ((lane & 2) == 0) == DESC; v = bcx<1>(v, up); }
    { const bool up = ((lane & 4) == 0) == DESC; v = bcx<2>(v, up); v = bcx<1>(v, up); }
    { const bool up = ((lane & 8) == 0) == DESC; v = bcx<4>(v, up); v = bcx<2>(v, up); v = bcx<1>(v, up); }
    { const bool up = ((lane & 16) == 0) == DESC;
      v = bcx<8>(v, up); v = bcx<4>(v, up); v = bcx<2>(v, up); v = bcx<1>(v, up); }
    { const bool up = ((lane & 32) == 0) == DESC;
      v = bcx<16>(v, up); v = bcx<8>(v, up); v = bcx<4>(v, up); v = bcx<2>(v, up); v = bcx<1>(v, up); }
    v = bcx<32>(v, DESC); v = bcx<16>(v, DESC); v = bcx<8>(v, DESC); v = bcx<4>(v, DESC); v = bcx<2>(v, DESC);
    return bcx<1>(v, DESC);
}
// The top 64 of a (sorted descending) and b (sorted ascending), sorted descending (DESC) or ascending: the lane-wise
// maximum is a bitonic sequence holding them, then a bitonic merge.
template <bool DESC = true>
__device__ __forceinline__ uint64_t merge_top64(uint64_t a_desc, uint64_t b_asc) {
    uint64_t v = a_desc > b_asc ? a_desc : b_asc;
    v = bcx<32>(v, DESC); v = bcx<16>(v, DESC); v = bcx<8>(v, DESC); v = bcx<4>(v, DESC); v = bcx<2>(v, DESC);
    return bcx<1>(v, DESC);
}

// fs_decode_step_hp on the small-k kernel (the fused kernel's decode_hist_copy / row_u / decode_commit for this
// kernel's merging workgroup): the stream's history copied to the new histories by the whole workgroup before the
// merge; the draw read from the stream without advancing it; after the token, wave 0 appends it and advances the
// stream (greedy rows draw nothing).
__device__ __forceinline__ void sk_hist_copy(const SkArgs& a, int row) {
    const int64_t h0 = a.hist_off ? a.hist_off[0] : 0, b = a.hist_off ? a.hist_off[row] : 0;
    const int64_t e = a.hist_off ? a.hist_off[row + 1] : 0;
    const int64_t nb = b - h0 + row;
    for (int64_t i = threadIdx.x; i < e - b; i += SK_LT)
        if (nb + i < a.out_cap) a.out_hist[nb + i] = a.hist[b + i];
    if (threadIdx.x == 0) {
        a.out_hist_off[row] = nb;
        if (row == a.B - 1) a.out_hist_off[a.B] = e - h0 + a.B;
        if (nb + (e - b) + 1 > a.out_cap) atomicOr(a.err, FS_DEVERR_HIST_APPEND);
    }
}
__device__ __forceinline__ double sk_row_u(const SkArgs& a, int row) {
    if (a.dmt) {
        const uint64_t* mt = a.dmt + (int64_t)row * MT_N;
        const int idx = a.didx[row];
        const uint64_t y = idx < MT_N ? mt[idx] : mt_twist_one(mt[0], mt[1], mt[MT_M]);
        return mt_canonical(mt_temper(y));
    }
    return a.u ? ld_const(a.u + row) : 0.0;
}
// Wave 0 alone: w is LDS scratch of MT_N entries. The twist in three passes, each reading every value it needs
// before it writes: entries below N - M from old values only (all computed, then written); the rest in ascending
// chunks of one wave (each reads its own and the next old entry and a new one below N - M; entry N - 1 the new
// entry 0), so no entry is overwritten before it is read.
__device__ __forceinline__ void sk_decode_commit(const SkArgs& a, int row, bool sampled, int tok, uint64_t* w) {
    const int lane = lane_id();
    if (a.out_hist_off && lane == 0) {
        const int64_t h0 = a.hist_off ? a.hist_off[0] : 0, b = a.hist_off ? a.hist_off[row] : 0;
        const int64_t e = a.hist_off ? a.hist_off[row + 1] : 0;
        const int64_t at = b - h0 + row + (e - b);
        if (at < a.out_cap) a.out_hist[at] = tok;
    }
    if (!a.dmt || !sampled) return;
    uint64_t* mt = a.dmt + (int64_t)row * MT_N;
    const int idx = a.didx[row];
    if (idx < MT_N) {
        if (lane == 0) a.didx[row] = idx + 1;
        return;
    }
    auto wave_sync = []() {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    };
    for (int t = lane; t < MT_N; t += WAVE) w[t] = mt[t];
    wave_sync();
    constexpr int LO = MT_N - MT_M, NLO = (LO + WAVE - 1) / WAVE;
    uint64_t nv[NLO];
#pragma unroll
    for (int c = 0; c < NLO; ++c) {
        const int t = c * WAVE + lane;
        nv[c] = t < LO ? mt_twist_one(w[t], w[t + 1], w[t + MT_M]) : 0ull;
    }
    wave_sync();
#pragma unroll
    for (int c = 0; c < NLO; ++c) {
        const int t = c * WAVE + lane;
        if (t < LO) w[t] = nv[c];
    }
    wave_sync();
    for (int t0 = LO; t0 < MT_N; t0 += WAVE) {
        const int t = t0 + lane;
        uint64_t v = 0ull;
        if (t < MT_N) v = mt_twist_one(w[t], w[(t + 1) % MT_N], w[t - LO]);
        wave_sync();
        if (t < MT_N) w[t] = v;
        wave_sync();
    }
    for (int t = lane; t < MT_N; t += WAVE) mt[t] = w[t];
    if (lane == 0) a.didx[row] = 1;
}

struct SkShared {
    float4 gval[SK_NW][SK_GCAP + 1];       // groups of four whose maximum reaches the bound (+ a dummy slot)
    int32_t gidx[SK_NW][SK_GCAP + 1];      //   and the segment offset of their first logit
    uint64_t cand[SK_CAP];                 // the segment's candidates (composites)
    uint64_t wl[SK_NW][SK_K];              // per-wave sorted lists (segment sort, row merge)
    uint32_t bmp[SK_LT * 16 * 4 / 32];     // repetition window ids in the segment (largest segment: NL = 16)
    uint32_t hist[16];                     // radix select digits (exact fallback)
    uint32_t wb[SK_NW];
    uint32_t wcnt[SK_NW];
    uint32_t tscan[SK_NW];
    uint32_t misc[4];
#ifdef FS_TRACE
    uint64_t trace_t[16];
#endif
};
static_assert(offsetof(SkShared, cand) % 16 == 0, "the rank loops read the candidates in 16-byte pairs");
// Phase timestamps of the small-k kernel (FS_TRACE builds only; thread 0, after the barrier that closes a phase):
// 0 start, 11 the segment's logits in and transformed, 12 lane maxima sorted, 2 bound, 3 groups handed over,
// 4 candidates expanded, 5 list ranked and published, 6 ticket taken; merging workgroup: 7 lists folded, 8 row
// finished (greedy rows set only 0, 5-8). Slots 9-10: candidates and groups of the segment; 13-15: role (3 segment,
// 4 segment + merge), row, segment. ferro_amd/trace_phases.py --route host reads them.
#ifdef FS_TRACE
#define SK_MARK(i) do { if (threadIdx.x == 0) s.trace_t[(i)] = __builtin_amdgcn_s_memrealtime(); } while (0)
#define SK_TAG(i, v) do { if (threadIdx.x == 0) s.trace_t[(i)] = (uint64_t)(v); } while (0)
#define SK_FLUSH() do { if (threadIdx.x == 0 && a.trace) \
    for (int i_ = 0; i_ < TRACE_W; ++i_) a.trace[(int64_t)blockIdx.x * TRACE_W + i_] = s.trace_t[i_]; } while (0)
#else
#define SK_MARK(i) do {} while (0)
#define SK_TAG(i, v) do {} while (0)
#define SK_FLUSH() do {} while (0)
#endif

// The exact path, for segments whose candidates at the bound overflow SK_CAP (ties at the bound): the segment's
// logits are re-read from memory (the L2 holds them by then) in batches of SK_EB per thread, sixteen loads in flight,
// and transformed again (softcap, then the repetition penalty from the segment's bitmap; past n: NaN).
constexpr int SK_EB = 16;
template <bool CAP, class F>
__device__ __forceinline__ void sk_each(const float* segp, int n, int nseg_elems, float cap, bool pen, float rep,
                                        const uint32_t* bmp, F f) {
    const int tid = threadIdx.x;
#pragma unroll 1
    for (int i0 = 0; i0 < nseg_elems; i0 += SK_LT * SK_EB) {
        float x[SK_EB];
#pragma unroll
        for (int j = 0; j < SK_EB; ++j) {
            const int i = i0 + j * SK_LT + tid;
            x[j] = i < n ? segp[i] : 0.0f;
        }
        if (CAP && cap > 0.0f) softcap_vals(x, cap);
#pragma unroll
        for (int j = 0; j < SK_EB; ++j) {
            const int i = i0 + j * SK_LT + tid;
            float l = x[j];
            if (pen && i < n && ((bmp[i >> 5] >> (i & 31)) & 1u)) l = l > 0.0f ? __fdiv_rn(l, rep) : __fmul_rn(l, rep);
            f(i, i < n ? key_of(l) : 0u);
        }
    }
}
// The exact k-th largest composite of the segment (every composite is distinct: the id is part of it), by a radix
// select over 4-bit digits. Slow, and rare.
template <bool CAP>
__device__ __forceinline__ uint64_t sk_kth_exact(const float* segp, int seg_lo, int n, int nseg_elems, float cap,
                                                 bool pen, float rep, int k, SkShared& s) {
    const int tid = threadIdx.x;
    uint64_t prefix = 0ull;
    int need = k;
#pragma unroll 1
    for (int sh = 60; sh >= 0; sh -= 4) {
        if (tid < 16) s.hist[tid] = 0u;
        __syncthreads();
        const uint64_t hi_mask = sh + 4 >= 64 ? 0ull : (~0ull << (sh + 4));
        sk_each<CAP>(segp, n, nseg_elems, cap, pen, rep, s.bmp, [&](int i, uint32_t key) {
            const uint64_t cm = comp_of(key, (uint32_t)(seg_lo + i));
            if (key != 0u && (cm & hi_mask) == prefix) atomicAdd(&s.hist[(uint32_t)(cm >> sh) & 15u], 1u);
        });
        __syncthreads();
        if (tid == 0) {
            int d = 15;
            for (; d > 0; --d) {
                const int c = (int)s.hist[d];
                if (c >= need) break;
                need -= c;
            }
            s.misc[2] = (uint32_t)d;
            s.misc[3] = (uint32_t)need;
        }
        __syncthreads();
        prefix |= (uint64_t)s.misc[2] << sh;
        need = (int)s.misc[3];
        __syncthreads();
    }
    return prefix;
}

// CAP: some row of the batch has a softcap (the cap's code is left out of batches without one).
struct Ids16 {
    int32_t v[16];
};

// small_k_kernel's argument list as a struct: the argument segment follows the same layout rules
struct SkKernargs {
    const float* logits;
    int64_t ld;
    int B, V, nseg, may_pen;
    const fs_row_params* params;
    const int64_t* hist_off;
    const int32_t* hist;
    SkArgs a;
};
constexpr size_t SK_ARGS_OFF = offsetof(SkKernargs, a);

// Dynamic LDS a launch requests beyond SkShared (unused): with it a CU holds 4 workgroups (≈35 KB each of its 160 KB),
// as the kernel's 96 VGPRs would otherwise allow 5. Measured on MI355X with this instantiation: a 272-row call of 1088
// workgroups 21.3 -> 20.6 us with the limit, the headline's 1024 workgroups unchanged. (All-greedy batches run the
// greedy-only instantiation without it.)
constexpr unsigned SK_PAD_LDS = 16384;

// GREEDY: every row of the batch is greedy (the selection code is left out: fewer registers, more workgroups per CU).
template <int NL, bool CAP, bool GREEDY>
__global__ __launch_bounds__(SK_LT) void small_k_kernel(const float* logits, int64_t ld, int B, int V, int nseg,
                                                        int may_pen, const fs_row_params* params,
                                                        const int64_t* hist_off, const int32_t* hist, SkArgs a_) {
    // The leading arguments arrive in SGPRs at wave launch (kernel-argument preloading), so the logits are requested
    // before any scalar memory round trip. A call with a repetition window (may_pen, set by the host from its copy of
    // the parameters) then reads the row's window bounds and requests its ids behind the logits.
    constexpr int SEG = SK_LT * NL * 4;
    static_assert(NL <= 16, "the repetition bitmap covers NL <= 16");
    __shared__ __align__(16) SkShared s;
    const int tid = threadIdx.x, lane = lane_id(), w = tid / WAVE;
    // workgroup i: XCD slot i % XCDS takes rows x, x + XCDS, ...: a row's segments are consecutive workgroups of one
    // index class mod XCDS, so they share an XCD and its L2 (the ticket and the lists)
    const int x = (int)(blockIdx.x % (unsigned)XCDS);
    const int j = (int)(blockIdx.x / (unsigned)XCDS);
    const int q_row = __builtin_amdgcn_readfirstlane(j / nseg);
    const int seg = j - q_row * nseg;
    const int row = x + XCDS * q_row;
    if (row >= B) return;
    SK_MARK(0);
    for (int i_ = 1; i_ < 13; ++i_) SK_TAG(i_, 0);
    SK_TAG(13, 3); SK_TAG(14, row); SK_TAG(15, seg);
    const int seg_lo = seg * SEG;
    const int n_in = V - seg_lo < SEG ? V - seg_lo : SEG;             // logits of this segment (>= 1)

    // every load of the segment at once; past the row's end (rounded up to four, inside ld) reads are zeros, masked
    const float* rowp = logits + (int64_t)row * ld;
    const int nrec = ((n_in + 3) & ~3) * 4;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(rowp + seg_lo), (short)0, nrec, 0x00020000);
    float4 v[NL];
#pragma unroll
    for (int q = 0; q < NL; ++q) {
        const f32x4 t = raw_buffer_load_f32x4(rs, (q * SK_LT + tid) * 16, 0, 2);    // nontemporal: read once
        v[q] = make_float4(t.x, t.y, t.z, t.w);
    }
    __builtin_amdgcn_sched_barrier(0);

    // the repetition window [wb0, len) over the row's history (sampling rows only: verification windows reach this
    // kernel only without an active penalty); its first 512 ids are requested behind the logits, two per thread
    bool pen = false, cnt_on = false;
    float rep = 1.0f, fq = 0.0f, pres = 0.0f;
    int64_t h0 = 0, len = 0, wb0 = 0;
    int wid[2] = {-1, -1};
    if (may_pen) {
        const fs_row_params* pr = params + row;
        rep = ld_const(&pr->repetition_penalty);
        fq = ld_const(&pr->frequency_penalty);
        pres = ld_const(&pr->presence_penalty);
        fs_row_params pw;
        pw.repeat_last_n = ld_const(&pr->repeat_last_n);
        pw.penalty_from = ld_const(&pr->penalty_from);
        h0 = ld_const(hist_off + row);
        len = ld_const(hist_off + row + 1) - h0;
        // frequency / presence penalties (greedy rows only, segments of 4096 logits: the host checks both) need
        // each window id's count in the segment
        cnt_on = NL == 4 && (fq != 0.0f || pres != 0.0f);
        pen = (rep != 1.0f || cnt_on) && pw.repeat_last_n != 0 && len > 0;
        wb0 = window_begin(len, pw);                           // unconditionally: all five loads in one round trip
        if (!pen || wb0 >= len) { pen = false; wb0 = len; }
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int64_t i = wb0 + r * SK_LT + tid;
            wid[r] = (pen && i < len) ? hist[h0 + i] : -1;
        }
    }
    // The remaining arguments are read from here on, through a pointer the compiler cannot trace back to the argument
    // segment: otherwise it loads some of them early and, short of scalar registers, spills them to vector lanes,
    // which waits for those loads before the logits are requested.
    const __attribute__((address_space(4))) char* kseg =
        (const __attribute__((address_space(4))) char*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(kseg) : : "memory");
    const SkArgs& a = *(const SkArgs*)(kseg + SK_ARGS_OFF);
    (void)a_;

    // verification: the row's stream (its parameters); sampling: the row's own
    int pidx = row;
    if (a.mode == MODE_VERIFY) {
        int s0 = 0, s1 = a.n_streams;                          // the largest s with row_off[s] <= row
        while (s1 - s0 > 1) {
            const int m = (s0 + s1) >> 1;
            if (ld_const(a.row_off + m) <= row) s0 = m; else s1 = m;
        }
        pidx = s0;
    }
    const fs_row_params* pp = params + pidx;
    const float temp = ld_const(&pp->temperature);
    const int top_k = ld_const(&pp->top_k);
    const float cap = CAP ? ld_const(&pp->softcap) : 0.0f;
    const bool greedy = GREEDY || temp <= 0.0f || top_k == 1;
    const int k = greedy ? 1 : ((top_k > 0 && top_k < V) ? top_k : V);

    // repetition penalty: an exact bitmap of the window's ids in this segment (each distinct id once: sampler.cpp:14-17).
    // rep >= 1 never raises a logit (l > 0: l / rep <= l; l <= 0: l * rep <= l), so the bound is taken over the raw
    // logits, the bitmap is filled while the bound is sorted (the ids arrive right behind the logits), and the penalty
    // is applied to the handed-over logits only; the bound then needs a check (below). rep < 1 raises the flagged
    // logits: they are penalised before the bound (the bitmap first).
    // greedy rows take the penalty before their maximum (no bound to protect), with its counts when cnt_on
    const bool pen_late = pen && rep >= 1.0f && !greedy;
    const bool pen_early = pen && !pen_late;
    cnt_on = cnt_on && pen;
    // cnt_on: 16-bit counts of the window's ids per logit of the segment, in the group buffer (unused on this path)
    uint32_t* cnt = reinterpret_cast<uint32_t*>(&s.gval[0][0]);
    static_assert(sizeof(SkShared::gval) >= SK_LT * 4 * 4 / 2 * sizeof(uint32_t),
                  "a 4096-logit segment's 16-bit counts fit the group buffer");
    bool ovf = false;
    auto mark = [&](int id) {
        const uint32_t rel = (uint32_t)(id - seg_lo);
        if (id >= 0 && id < V && rel < (uint32_t)SEG) {
            atomicOr(&s.bmp[rel >> 5], 1u << (rel & 31u));
            if (cnt_on) {
                const uint32_t sh = (rel & 1u) * 16u;
                const uint32_t old = atomicAdd(&cnt[rel >> 1], 1u << sh);
                ovf |= ((old >> sh) & 0xFFFFu) == 0xFFFFu;
            }
        }
    };
    auto mark_window = [&]() {
        // the ids arrive behind the logits: an empty asm keeps the compiler from hoisting their first use (and the
        // wait for every load it needs) above the branch that calls this
        int i0 = wid[0], i1 = wid[1];
        asm volatile("" : "+v"(i0), "+v"(i1));
        mark(i0);
        mark(i1);
        for (int64_t i = wb0 + 2 * SK_LT + tid; i < len; i += SK_LT) mark(a.hist[h0 + i]);
    };
    if (pen) {
        for (int i = tid; i < SEG / 32; i += SK_LT) s.bmp[i] = 0u;
        if (cnt_on)
            for (int i = tid; i < SEG / 2; i += SK_LT) cnt[i] = 0u;
        __syncthreads();
    }
    uint64_t pm = 0ull;                        // rep < 1 or greedy: 4 bits per group of this thread
    if (pen_early) {
        mark_window();
        if (ovf) atomicOr(a.err, FS_DEVERR_COUNT_OVERFLOW);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < NL; ++q) {
            const uint32_t rel = (uint32_t)(q * SK_LT + tid) * 4u;
            pm |= (uint64_t)((s.bmp[rel >> 5] >> (rel & 31u)) & 0xFu) << (4 * q);
        }
    }
    const bool wpen = __ballot(pm != 0ull) != 0ull;
    const bool tail = n_in < SEG;

    // the logits as ferro's sampler sees them (softcap; rep < 1: the penalty; past the row's end: NaN, never a
    // candidate) and the lane maximum (NaN-free: fmaxf drops NaN; NaN when every logit of the lane is NaN)
    float lm = __builtin_nanf("");
#pragma unroll
    for (int q = 0; q < NL; ++q) {
        float e[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
        if (CAP && cap > 0.0f) softcap_vals(e, cap);       // a rolled loop: one copy of the cap per group
        if (wpen) {
            const uint32_t nib = (uint32_t)(pm >> (4 * q)) & 0xFu;
            if (__ballot(nib != 0u)) {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if ((nib >> c) & 1u) {
                        float l = e[c] > 0.0f ? __fdiv_rn(e[c], rep) : __fmul_rn(e[c], rep);
                        if (cnt_on) {                      // l - (count * frequency + presence), as the fused kernel
                            const uint32_t rel = (uint32_t)(q * SK_LT + tid) * 4u + (uint32_t)c;
                            const float cc = (float)((cnt[rel >> 1] >> ((rel & 1u) * 16u)) & 0xFFFFu);
                            l = __fsub_rn(l, __fadd_rn(__fmul_rn(cc, fq), pres));
                        }
                        e[c] = l;
                    }
            }
        }
        if (tail) {
            const int e0 = (q * SK_LT + tid) * 4;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (e0 + c >= n_in) e[c] = __builtin_nanf("");
        }
        v[q] = make_float4(e[0], e[1], e[2], e[3]);
        lm = fmaxf(lm, fmaxf(fmaxf(e[0], e[1]), fmaxf(e[2], e[3])));
    }
    // Greedy rows (their penalties already applied above): the segment's list is its first maximum alone (ferro's
    // scan, sampler.cpp:19-23, takes a larger logit only: the lowest index among equal maxima; NaN never), so the
    // bound, the candidates and their ranks are skipped: a lane's first index holding its maximum, then the largest
    // composite of the workgroup (value first, then the lower id). The rest of the list is zeros, which every merge
    // reads as empty.
    uint64_t* myl = a.lists + ((int64_t)row * a.nseg + seg) * SK_K;
    const bool gfast = greedy;
    if (gfast) {
        uint64_t best = 0ull;
        if (lm == lm) {                                        // NaN: every logit of the lane is NaN
            uint32_t first = 0u;
#pragma unroll
            for (int q = NL - 1; q >= 0; --q) {
                const uint32_t e0 = (uint32_t)(seg_lo + (q * SK_LT + tid) * 4);
                first = v[q].w == lm ? e0 + 3u : first;
                first = v[q].z == lm ? e0 + 2u : first;
                first = v[q].y == lm ? e0 + 1u : first;
                first = v[q].x == lm ? e0 : first;
            }
            best = comp_of(key_of(lm), first);
        }
        best = wave_max(best);
        if (lane == 0) s.wl[w][0] = best;
        __syncthreads();
        if (w == 0) {
            const uint64_t m = wave_max(lane < SK_NW ? s.wl[lane][0] : 0ull);
            myl[lane] = lane == 0 ? m : 0ull;
        }
    } else {
        // the bound: each wave sorts its lane maxima in registers (no scalar round trips per step); lane kq - 1 holds
        // its kq-th largest, and the smallest over the waves counts SK_NW kq >= k distinct logits (one lane more per
        // wave when the penalty comes later: the raw logits counted may be among the penalised ones)
        const uint32_t kq = (uint32_t)((k + SK_NW - 1) / SK_NW) + (pen_late ? 1u : 0u);
        SK_MARK(11);
        {
            const uint32_t srt = sort64_desc_u32(key_of(lm));
            if (lane == (int)kq - 1) s.wb[w] = srt;
        }
        if (pen_late) mark_window();                               // completed by the barrier below
        SK_MARK(12);
        __syncthreads();
        SK_MARK(2);
        uint32_t tau = s.wb[0];
#pragma unroll
        for (int q = 1; q < SK_NW; ++q) tau = s.wb[q] < tau ? s.wb[q] : tau;
        if (tau == 0u) tau = 1u;                                   // NaN (key 0) is never a candidate
        const float tf = tau > 0x007FFFFFu ? val_of(tau) : -__builtin_huge_valf();
        // groups whose maximum reaches the bound: this wave's region of the group buffer, in lane order
        uint32_t gmask = 0u;
#pragma unroll
        for (int q = 0; q < NL; ++q)                     // the group's raw maximum (recomputed: no register array)
            gmask |= (fmaxf(fmaxf(v[q].x, v[q].y), fmaxf(v[q].z, v[q].w)) >= tf ? 1u : 0u) << q;
        const uint32_t gn = (uint32_t)__popc(gmask);
        const uint32_t gincl = wave_incl_scan_u32(gn);
        const uint32_t wtot = (uint32_t)__builtin_amdgcn_readlane((int)gincl, WAVE - 1);
        uint32_t go = gincl - gn;
        // the groups any lane of the wave hands over (one scalar mask); per such group every lane writes, those without
        // it into the region's dummy slot, so no per-lane branch waits on a compare
        const uint32_t wmask = (uint32_t)__builtin_amdgcn_readfirstlane(
            (int)wave_allreduce(gmask, [](uint32_t x, uint32_t y) { return x | y; }));
#pragma unroll
        for (int q = 0; q < NL; ++q) {
            if ((wmask >> q) & 1u) {
                const bool mine = ((gmask >> q) & 1u) != 0u && go < (uint32_t)SK_GCAP;
                const uint32_t slot = mine ? go : (uint32_t)SK_GCAP;
                s.gval[w][slot] = v[q];
                s.gidx[w][slot] = (int32_t)((uint32_t)(q * SK_LT + tid) * 4u);
                go += (gmask >> q) & 1u;
            }
        }
        if (lane == 0) s.wcnt[w] = wtot;
        __syncthreads();
        SK_MARK(3);
        // expansion: thread t takes group t of the concatenated regions, its logits at or above the bound become
        // candidates
        uint32_t goff[SK_NW + 1];
        goff[0] = 0u;
        bool gover = false;
#pragma unroll
        for (int q = 0; q < SK_NW; ++q) {
            const uint32_t c = s.wcnt[q];
            gover |= c > (uint32_t)SK_GCAP;
            goff[q + 1] = goff[q] + (c < (uint32_t)SK_GCAP ? c : (uint32_t)SK_GCAP);
        }
        const uint32_t G = goff[SK_NW];
        uint64_t cm[4] = {0ull, 0ull, 0ull, 0ull};
        bool cp[4] = {false, false, false, false};
        uint32_t nc = 0u;
        if (!gover && (uint32_t)tid < G) {
            int r = 0;
            uint32_t gb = 0u;
#pragma unroll
            for (int q = 1; q < SK_NW; ++q) {
                const bool past = (uint32_t)tid >= goff[q];
                r += past ? 1 : 0;
                gb = past ? goff[q] : gb;
            }
            const uint32_t gi = (uint32_t)tid - gb;
            const float4 gv = s.gval[r][gi];
            const uint32_t gw = (uint32_t)s.gidx[r][gi];
            const int e0 = (int)gw;
            // rep >= 1: the group's penalised logits, from the bitmap (its 4 bits share a word: e0 % 4 == 0)
            float e[4] = {gv.x, gv.y, gv.z, gv.w};
            if (pen_late) {
                const uint32_t nib = (s.bmp[(uint32_t)e0 >> 5] >> ((uint32_t)e0 & 31u)) & 0xFu;
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if ((nib >> c) & 1u) e[c] = e[c] > 0.0f ? __fdiv_rn(e[c], rep) : __fmul_rn(e[c], rep);
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                cp[c] = e[c] >= tf;
                cm[c] = comp_of(key_of(e[c]), (uint32_t)(seg_lo + e0 + c));
                nc += cp[c] ? 1u : 0u;
            }
        }
        if (G > (uint32_t)SK_LT) gover = true;                     // more groups than threads: the exact path
        // block exclusive scan of the candidate counts
        const uint32_t cincl = wave_incl_scan_u32(nc);
        if (lane == WAVE - 1) s.tscan[w] = cincl;
        __syncthreads();
        SK_MARK(4);
        uint32_t cbase = 0u, ntot = 0u;
#pragma unroll
        for (int q = 0; q < SK_NW; ++q) {
            const uint32_t t = s.tscan[q];
            cbase += q < w ? t : 0u;
            ntot += t;
        }
        // With the penalty applied after the bound, fewer than k logits may stay at or above it: the segment's top k
        // may then hold a logit below the bound, which was not handed over (never expected with the spare lane per
        // wave)
        const bool short_k = pen_late && ntot < (uint32_t)k && tf > -__builtin_huge_valf();
        const bool exact = gover || short_k || ntot > (uint32_t)SK_CAP;   // uniform
        if (!exact) {
            uint32_t pos = cbase + cincl - nc;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (cp[c]) s.cand[pos++] = cm[c];
        }
        if (exact) {
            // ties at the bound: the exact k-th composite of the segment, then the (exactly k) composites at or above
            // it
            const float* segp = rowp + seg_lo;
            const uint64_t kth = sk_kth_exact<CAP>(segp, seg_lo, n_in, SEG, cap, pen, rep, k, s);
            if (tid == 0) s.misc[0] = 0u;
            __syncthreads();
            sk_each<CAP>(segp, n_in, SEG, cap, pen, rep, s.bmp, [&](int i, uint32_t key) {
                const uint64_t c64 = comp_of(key, (uint32_t)(seg_lo + i));
                if (key != 0u && c64 >= kth) {
                    const uint32_t p = atomicAdd(&s.misc[0], 1u);
                    if (p < (uint32_t)SK_K) s.cand[p] = c64;
                }
            });
            __syncthreads();
            ntot = s.misc[0] < (uint32_t)SK_K ? s.misc[0] : (uint32_t)SK_K;
        }
        __syncthreads();
        // the segment's top k, sorted by rank: P threads per candidate each count the larger entries in 1/P of the list
        // (LDS reads of one address per wave: broadcasts), the partial counts are summed and the first k placed by rank
        uint64_t* sorted = &s.wl[0][0];
        uint32_t* rk = reinterpret_cast<uint32_t*>(&s.wl[1][0]);    // [P][per] partial ranks (SK_LT words)
        {
            const int n = (int)ntot;
            if (n <= SK_LT) {
                const int P = n <= SK_LT / 4 ? 4 : (n <= SK_LT / 2 ? 2 : 1);
                const int per = SK_LT / P;
                const int c = tid % per, qq = tid / per;
                const int span = (((n + P - 1) / P) + 1) & ~1;     // even: every part starts on a 16-byte pair
                if (c < n) {
                    const uint64_t me = s.cand[c];
                    const int j0 = qq * span, j1 = j0 + span < n ? j0 + span : n;
                    uint32_t r = 0u;
                    int jj = j0;
                    const ulonglong2* c2 = reinterpret_cast<const ulonglong2*>(s.cand);
                    for (; jj + 8 <= j1; jj += 8) {                // eight entries per step: four 16-byte LDS reads
                        const ulonglong2 e0 = c2[jj >> 1], e1 = c2[(jj >> 1) + 1], e2 = c2[(jj >> 1) + 2],
                                         e3 = c2[(jj >> 1) + 3];
                        r += (e0.x > me ? 1u : 0u) + (e0.y > me ? 1u : 0u) + (e1.x > me ? 1u : 0u) +
                             (e1.y > me ? 1u : 0u) + (e2.x > me ? 1u : 0u) + (e2.y > me ? 1u : 0u) +
                             (e3.x > me ? 1u : 0u) + (e3.y > me ? 1u : 0u);
                    }
                    for (; jj < j1; ++jj) r += s.cand[jj] > me ? 1u : 0u;
                    rk[qq * per + c] = r;
                }
                __syncthreads();
                if (tid < n) {                                     // placed straight into the published list
                    uint32_t r = 0u;
                    for (int p2 = 0; p2 < P; ++p2) r += rk[p2 * per + tid];
                    if (r < (uint32_t)k) myl[r] = s.cand[tid];
                }
            } else {                                               // 256 < n <= SK_CAP: two candidates per thread
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int c = tid + h * SK_LT;
                    if (c < n) {
                        const uint64_t me = s.cand[c];
                        uint32_t r = 0u;
                        int jj = 0;
                        const ulonglong2* c2 = reinterpret_cast<const ulonglong2*>(s.cand);
                        for (; jj + 8 <= n; jj += 8) {
                            const ulonglong2 e0 = c2[jj >> 1], e1 = c2[(jj >> 1) + 1], e2 = c2[(jj >> 1) + 2],
                                             e3 = c2[(jj >> 1) + 3];
                            r += (e0.x > me ? 1u : 0u) + (e0.y > me ? 1u : 0u) + (e1.x > me ? 1u : 0u) +
                                 (e1.y > me ? 1u : 0u) + (e2.x > me ? 1u : 0u) + (e2.y > me ? 1u : 0u) +
                                 (e3.x > me ? 1u : 0u) + (e3.y > me ? 1u : 0u);
                        }
                        for (; jj < n; ++jj) r += s.cand[jj] > me ? 1u : 0u;
                        if (r < (uint32_t)k) myl[r] = me;
                    }
                }
            }
            if (tid >= (n < k ? n : k) && tid < SK_K) myl[tid] = 0ull;   // slots past the segment's top k
        }
        (void)sorted;
        SK_TAG(9, ntot);
        SK_TAG(10, G);
    }
    vm_drain();                                                // the list is in the L2
    __syncthreads();
    SK_MARK(5);
    if (tid == 0) {
        const uint32_t t = __hip_atomic_fetch_add(a.ticket + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        s.misc[1] = t == (uint32_t)a.nseg - 1u ? 1u : 0u;
    }
    __syncthreads();
    SK_MARK(6);
    if (s.misc[1] == 0u) {
        SK_FLUSH();
        return;
    }
    SK_TAG(13, 4);
    if (a.out_hist_off) sk_hist_copy(a, row);                  // a decode step: every thread, before the merge
    // ---- the row's merge (the last of its segments): wave w folds lists w, w + SK_NW, ... (the first as stored,
    // the rest reversed: ascending), then wave 0 folds the waves' lists
    const uint64_t* rl = a.lists + (int64_t)row * a.nseg * SK_K;
    uint64_t acc = 0ull;
    if (greedy) {
        // k = 1: every list holds its segment's top composite first; wave 0 takes the largest of the nseg heads
        if (w != 0) return;
        SK_MARK(7);
        if (tid == 0) a.ticket[row] = 0u;                     // all segments have counted: reset for the next call
        acc = wave_max(lane < a.nseg ? rl[lane * SK_K] : 0ull);
    } else {
        for (int L0 = w; L0 < a.nseg; L0 += 4 * SK_NW) {
            // four lists per wave, requested together: lists 0 and 2 as stored (descending), 1 and 3 reversed
            uint64_t b[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int L = L0 + r * SK_NW;
                b[r] = L < a.nseg ? rl[L * SK_K + ((r & 1) ? WAVE - 1 - lane : lane)] : 0ull;
            }
            // two independent merges (their latencies overlap), then one
            const uint64_t m01 = merge_top64<true>(b[0], b[1]);
            const uint64_t m23 = merge_top64<false>(b[2], b[3]);
            if (L0 == w) acc = merge_top64<true>(m01, m23);
            else acc = merge_top64<true>(acc, merge_top64<false>(m01, m23));
        }
        // across the waves: waves 0 and 2 fold 1 and 3 (in parallel), then wave 0 folds wave 2's
        s.wl[w][lane] = acc;
        __syncthreads();
        if (w == 0 || w == 2) acc = merge_top64(acc, s.wl[w + 1][WAVE - 1 - lane]);
        if (w == 2) s.wl[2][lane] = acc;
        __syncthreads();
        if (w != 0) return;
        SK_MARK(7);
        if (tid == 0) a.ticket[row] = 0u;                     // all segments have counted: reset for the next call
        acc = merge_top64(acc, s.wl[2][WAVE - 1 - lane]);
    }
    // the row's candidates: lane i holds the i-th in ferro's order (value desc, id asc); NaN never is one
    const int kk = __popcll(__ballot(lane < k && acc != 0ull));
    Args fa = {};
    fa.mode = MODE_SAMPLE; fa.kcap = a.kcap; fa.cand_ids = a.cand_ids; fa.cand_probs = a.cand_probs;
    RowCtx rc = {};
    rc.row = row;
    rc.p.temperature = temp; rc.p.top_k = top_k;
    rc.p.top_p = ld_const(&pp->top_p); rc.p.min_p = ld_const(&pp->min_p);
    int tok = 0, keep = 1;
    if (greedy) {
        // ferro's scan (sampler.cpp:19-23) keeps index 0 when its logit is NaN; otherwise the first maximum
        float l0 = ld_const(rowp);
        if (CAP && cap > 0.0f) l0 = softcap_one(l0, cap);
        tok = (l0 != l0 || kk == 0) ? 0 : (int)comp_id(read_lane(acc, 0));
        if (lane == 0 && a.kcap > 0) {
            if (a.cand_ids) a.cand_ids[(int64_t)row * a.kcap] = tok;
            if (a.cand_probs) a.cand_probs[(int64_t)row * a.kcap] = 1.0;
        }
    } else if (kk == 0) {
        tok = 0; keep = 0;                                     // every logit NaN: token 0, nothing kept
    } else {
        wave_softmax(fa, rc, lane < kk ? acc : 0ull, kk, sk_row_u(a, row), tok, keep);
    }
    if (a.mode != MODE_VERIFY) {
        if (lane == 0) {
            a.tok[row] = tok;
            if (a.keep) a.keep[row] = keep;
        }
        if (a.out_hist_off || a.dmt) sk_decode_commit(a, row, !greedy, tok, &s.cand[0]);
    } else {
        // the last row of a stream to finish computes its accepted prefix (server.cpp:627-637): the stream's rows
        // run on several XCDs, so the exchange is agent-scope.
        const int64_t r0 = ld_const(a.row_off + pidx);
        const int m = (int)(ld_const(a.row_off + pidx + 1) - r0);
        if (m <= 32) {
            // Streams of up to 32 rows: one 64-bit atomic per row carries everything - the count of rows done in its
            // high word, in its low word a bit for each row that ends the walk (an eos token, the last row, or a
            // token other than the next row's draft). The last row's fetched value holds every other row's bit, so
            // its accepted prefix is the lowest set bit + 1, with no token exchanged and no wait for stores.
            if (lane == 0) {
                a.tok[row] = tok;
                const int rr = row - (int)r0;
                const bool stop = (a.eos >= 0 && tok == a.eos) || rr + 1 >= m || tok != ld_const(a.rows + row + 1);
                const uint64_t mine = stop ? (1ull << rr) : 0ull;
                uint64_t* cnt = reinterpret_cast<uint64_t*>(a.stream_cnt) + pidx;
                const uint64_t old = __hip_atomic_fetch_add(cnt, (1ull << 32) | mine, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT);
                if ((uint32_t)(old >> 32) == (uint32_t)m - 1u) {
                    __hip_atomic_store(cnt, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    a.accepted[pidx] = __ffs((int)((uint32_t)old | (uint32_t)mine));
                }
            }
            SK_MARK(8);
            SK_FLUSH();
            return;
        }
        // longer streams: the token at agent scope, a row counter (after the 64-bit words), the last row walks
        uint32_t* cnt32 = a.stream_cnt + 2 * (int64_t)a.n_streams + pidx;
        uint32_t old = 0u;
        if (lane == 0) {
            st_agent(&a.tok[row], (int32_t)tok);
            vm_drain();
            old = __hip_atomic_fetch_add(cnt32, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (read_lane(old, 0) == (uint32_t)m - 1u) {
            if (lane == 0) st_agent(cnt32, 0u);
            const int acc = accepted_prefix(a.tok, a.rows, r0, m, a.eos);
            if (lane == 0) a.accepted[pidx] = acc;
        }
    }
    SK_MARK(8);
    SK_FLUSH();
}

}  // namespace fs

// ================================================================================================ host side
struct fs_context {
    std::mutex mu;
    int device = -1;
    int cus = 0;               // compute units of the device
    int xccs = 0;              // XCDs of the device (hipDeviceAttributeNumberOfXccs)
    bool seg_layout = true;    // the segment grid's hand-off holds on this device (XCDS % xccs == 0)
    int32_t* hflag = nullptr;  // host-mapped: a merge of an earlier call gave up (set by the kernel, read here)
    int32_t* hflag_dev = nullptr;
    bool captured = false;     // a call was recorded into a graph: workspaces are retired, never freed, on growth
    std::vector<void*> retired;
    uint64_t* sk_lists = nullptr;   // small-k kernel: [slots][SK_K] sorted segment lists
    size_t sk_slots = 0;
    uint32_t* sk_ticket = nullptr;  // small-k kernel: [rows] segment tickets, left at 0
    size_t sk_rows = 0;
    uint64_t* cand = nullptr;
    size_t cand_slots = 0;     // chunk slots of CAP entries
    uint32_t* meta = nullptr;
    uint32_t* rhist = nullptr;  // [row_cap][RBINS]
    uint64_t* rmass = nullptr;  // [row_cap][LB]
    size_t row_cap = 0;
    uint32_t* stream_cnt = nullptr;
    size_t stream_cap = 0;
    int32_t* err = nullptr;        // [0]: error bits; [1]: dirty (a merge gave up; see fs_device_error); [2..3]: hflag_dev
    uint32_t merge_spins = fs::MERGE_SPINS;
    int static_dev = -1;       // device whose static workspace fs_sample_batch_static used with this context
    uint64_t* trace = nullptr; // FS_TRACE builds: phase timestamps, trace_cap entries (fs_trace_set)
    int64_t trace_cap = 0;
    fs_row_params* greedy = nullptr;      // fs_argmax_batch without parameters: [greedy_cap] greedy records
    size_t greedy_cap = 0;
    std::vector<fs_row_params> h_greedy;  //   and their host copy (the small-k kernel's greedy path)
};

namespace fs {
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0u;
}
// n parameter records of a greedy row without penalties (fs_argmax_batch without parameters)
__global__ __launch_bounds__(256) void greedy_params_kernel(fs_row_params* p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        fs_row_params r;
        r.temperature = 0.0f; r.top_k = 1; r.top_p = 1.0f; r.min_p = 0.0f; r.repetition_penalty = 1.0f;
        r.frequency_penalty = 0.0f; r.presence_penalty = 0.0f; r.repeat_last_n = 0; r.penalty_from = 0;
        r.softcap = 0.0f;
        p[i] = r;
    }
}
}  // namespace fs

namespace {

// Zero n words on st with a fill kernel (no hipMemsetAsync: the call may be recorded into a graph).
void clear_words(hipStream_t st, void* p, int64_t n) {
    if (!p || n <= 0) return;
    const int64_t blocks = std::min<int64_t>(1024, (n + 255) / 256);
    hipLaunchKernelGGL(fs::zero_words_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (uint32_t*)p, n);
}

// A workspace buffer that is replaced: freed, or, once a call of the context has been recorded into a HIP graph
// (whose replays keep using the old addresses), kept until fs_destroy.
void release(fs_context* c, void* p) {
    if (!p) return;
    if (c->captured) c->retired.push_back(p);
    else (void)hipFree(p);
}

int grow(fs_context* c, size_t slots, size_t rows, size_t streams) {
    if (slots > c->cand_slots) {
        release(c, c->cand);
        release(c, c->meta);
        c->cand = nullptr; c->meta = nullptr; c->cand_slots = 0;
        if (hipMalloc(&c->cand, slots * fs::CAP * sizeof(uint64_t)) != hipSuccess) return FS_E_NOMEM;
        if (hipMalloc(&c->meta, slots * 2 * sizeof(uint32_t)) != hipSuccess) return FS_E_NOMEM;
        c->cand_slots = slots;
    }
    if (rows > c->row_cap) {
        release(c, c->rhist);
        release(c, c->rmass);
        c->rhist = nullptr; c->rmass = nullptr; c->row_cap = 0;
        if (hipMalloc(&c->rhist, rows * fs::RBINS * sizeof(uint32_t)) != hipSuccess) return FS_E_NOMEM;
        if (hipMemset(c->rhist, 0, rows * fs::RBINS * sizeof(uint32_t)) != hipSuccess) return FS_E_HIP;
        if (hipMalloc(&c->rmass, rows * fs::LB * sizeof(uint64_t)) != hipSuccess) return FS_E_NOMEM;
        if (hipMemset(c->rmass, 0, rows * fs::LB * sizeof(uint64_t)) != hipSuccess) return FS_E_HIP;
        c->row_cap = rows;
    }
    if (streams > c->stream_cap) {
        release(c, c->stream_cnt);
        c->stream_cnt = nullptr; c->stream_cap = 0;
        if (hipMalloc(&c->stream_cnt, streams * sizeof(uint32_t)) != hipSuccess) return FS_E_NOMEM;
        if (hipMemset(c->stream_cnt, 0, streams * sizeof(uint32_t)) != hipSuccess) return FS_E_HIP;
        c->stream_cap = streams;
    }
    if (!c->hflag) {
        if (hipHostMalloc((void**)&c->hflag, sizeof(int32_t), hipHostMallocMapped) != hipSuccess) return FS_E_NOMEM;
        *(volatile int32_t*)c->hflag = 0;
        if (hipHostGetDevicePointer((void**)&c->hflag_dev, c->hflag, 0) != hipSuccess) return FS_E_HIP;
    }
    if (!c->err) {
        // error bits, dirty flag, then the device address of the host-mapped give-up flag (read by a give-up only)
        int32_t h[4] = {0, 0, 0, 0};
        const uint64_t fa = (uint64_t)(uintptr_t)c->hflag_dev;
        memcpy(h + 2, &fa, sizeof(fa));
        if (hipMalloc(&c->err, sizeof(h)) != hipSuccess) return FS_E_NOMEM;
        if (hipMemcpy(c->err, h, sizeof(h), hipMemcpyHostToDevice) != hipSuccess) return FS_E_HIP;
    }
    return FS_OK;
}

// Segments: at most two per CU over the whole batch (all resident at once: a second round of a few workgroups
// would double the time), at least one per row; a segment streams >= 1 full tile of 4096 logits. The merge
// handles each row's partial last tile (all of a row shorter than one tile). Sets a.nseg / a.seg_tiles and the
// workspace the call needs (items = (row, segment) slots).
// max_slots > 0 caps the workspace slots (XCDS * nseg * ceil(rows / XCDS)) by taking fewer segments per row; one
// segment per row always fits rows <= max_slots.
int plan(int cus, fs::Args& a, int64_t rows, int64_t& items, int64_t& seg_grid, int64_t max_slots = 0,
         int per_cu = 2) {
    const int64_t tiles_row = a.V / fs::TILE;
    const int64_t per_slot = (rows + fs::XCDS - 1) / fs::XCDS;
    a.nseg = 0;
    a.seg_tiles = 1;
    if (tiles_row > 0) {
        int64_t want = ((int64_t)per_cu * (int64_t)cus) / rows;
        if (want < 1) want = 1;
        if (want > tiles_row) want = tiles_row;
        if (want > fs::BLOCK - 1) want = fs::BLOCK - 1;   // the merge gives each list (segments + tail) a thread
        for (;;) {
            a.seg_tiles = (int)((tiles_row + want - 1) / want);
            a.nseg = (int)((tiles_row + a.seg_tiles - 1) / a.seg_tiles);
            if (max_slots <= 0 || want <= 1 || (int64_t)fs::XCDS * a.nseg * per_slot <= max_slots) break;
            --want;
        }
    }
    if (a.nseg > fs::MAX_SEGS) return FS_E_INVALID;
    items = rows * a.nseg;
    if (items > 0x7fffffff) return FS_E_INVALID;
    // one workgroup per (row, segment), the rows dealt to XCDS slots (segment_kernel); each segment workgroup's
    // list slot is its index, so the workspace holds seg_grid slots
    seg_grid = items > 0 ? (int64_t)fs::XCDS * a.nseg * ((rows + fs::XCDS - 1) / fs::XCDS) : 0;
    if (seg_grid > 0x7fffffff) return FS_E_INVALID;
    items = seg_grid;
    // balanced layouts (sampling, >= 2 segments per row, >= 2 rows on some XCD, <= WAVE rows per XCD)
    // Balanced layouts: sampling, >= 2 segments per row, 16 to WAVE rows per XCD. Computing the layout delays every
    // workgroup by about 2 us, which pays on large mixed batches (B=256 x V=262144 with k from 1 to 2048: -20 us)
    // but not on small ones.
    a.balance = (a.mode == fs::MODE_SAMPLE && a.nseg >= 2 && (rows + fs::XCDS - 1) / fs::XCDS >= 16 &&
                 (rows + fs::XCDS - 1) / fs::XCDS <= fs::WAVE) ? 1 : 0;
    return FS_OK;
}

// Launches the sampling grid on a bound workspace (a.cand / meta / rhist / stream_cnt / err / dirty).
int launch_planned(const fs::Args& a, int64_t rows, int64_t seg_grid, hipStream_t st) {
    if (seg_grid > 0) {                            // the segments, then one merging workgroup per row (same grid)
        const int64_t grid = seg_grid + (int64_t)fs::XCDS * ((rows + fs::XCDS - 1) / fs::XCDS);
        if (grid > 0x7fffffff) return FS_E_INVALID;
        hipLaunchKernelGGL(fs::segment_kernel, dim3((unsigned)grid), dim3(fs::BLOCK), 0, st, a.logits, a.ld, a.B, a.V,
                           a.nseg, a.seg_tiles, a.params, a.hist_off, a);
        return hipGetLastError() == hipSuccess ? FS_OK : FS_E_HIP;
    }
    hipLaunchKernelGGL(fs::merge_kernel, dim3((unsigned)rows), dim3(fs::BLOCK), 0, st, a.nseg, a.cand, a.meta, a.rhist,
                       a.params, 0, a);
    return hipGetLastError() == hipSuccess ? FS_OK : FS_E_HIP;
}

// Every row sampled alone by one workgroup from its logits (a device whose XCD layout the segment grid's hand-off
// does not fit).
int launch_alone(fs::Args a, int64_t rows, hipStream_t st) {
    a.nseg = 0;
    a.balance = 0;
    hipLaunchKernelGGL(fs::merge_kernel, dim3((unsigned)rows), dim3(fs::BLOCK), 0, st, 0, a.cand, a.meta, a.rhist,
                       a.params, 1, a);
    return hipGetLastError() == hipSuccess ? FS_OK : FS_E_HIP;
}

// The segment grid places a row's segments and its merging workgroup on workgroups of one index class mod XCDS, so
// that they share an XCD (and its L2) under round-robin dispatch over the device's XCDs: that holds when the XCD
// count divides XCDS (8, 4, 2 or 1: every MI355X partition mode). On other devices every row is sampled alone.
bool layout_fits(int xccs) { return xccs >= 1 && fs::XCDS % xccs == 0; }

int device_of(fs_context* ctx) {
    if (ctx->device < 0) {
        int dev = -1;
        if (hipGetDevice(&dev) != hipSuccess) return FS_E_HIP;
        if (hipDeviceGetAttribute(&ctx->cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return FS_E_HIP;
        int x = 0;
        if (hipDeviceGetAttribute(&x, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess) return FS_E_HIP;
        ctx->xccs = x;
        ctx->seg_layout = layout_fits(x);
        ctx->device = dev;
    }
    return FS_OK;
}

// Whether an earlier call's merge gave up waiting for its segments (the kernel sets the host-mapped flag). The
// caller then enqueues, ahead of its own launch, fill kernels that clear what the late segments may have left (they
// have finished once the stream reaches the fills), so the call runs normally instead of computing every row alone;
// it returns FS_W_RECOVERED. The error bits stay for fs_device_error.
bool gave_up(int32_t* flag) {
    if (!flag || *(volatile int32_t*)flag == 0) return false;
    *(volatile int32_t*)flag = 0;
    return true;
}

bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// ---- small-k kernel (fs_sample_batch_hp)
// Whether every row of the batch fits the small-k kernel: greedy, or k = min(top_k or V, V) <= SK_K, with no
// frequency / presence penalty (h: the host copy of the parameters).
// A batch whose rows cost very differently: rows sampled with 64 < k <= KMAX beside greedy or k <= 64 rows, none on
// the whole-row path (k > KMAX), 16 to 64 rows per XCD (the balanced layout). The host copy of the parameters shows
// the mix, and such batches take about four segments per CU instead of two, which gives the balanced layout finer
// shares to apportion (B=256 x V=262144 with k from 1 to 2048: 119.7 -> 116.6-117.4 us). Uniform batches lose with
// more segments (more lists to merge, a second round of workgroups).
bool mixed_merges(const fs_row_params* h, int64_t B, int32_t V) {
    const int64_t per_x = (B + fs::XCDS - 1) / fs::XCDS;
    if (per_x < 16 || per_x > fs::WAVE) return false;
    bool heavy = false, light = false;
    for (int64_t b = 0; b < B; ++b) {
        const fs_row_params& p = h[b];
        const bool greedy = !(p.temperature > 0.0f && p.top_k != 1);
        const int64_t k = greedy ? 1 : ((p.top_k > 0 && p.top_k < V) ? p.top_k : V);
        if (k > fs::KMAX) return false;
        if (k > 64) heavy = true;
        else light = true;
    }
    return heavy && light;
}

bool small_k_batch(const fs_row_params* h, int64_t B, int32_t V) {
    for (int64_t b = 0; b < B; ++b) {
        const fs_row_params& p = h[b];
        const bool greedy = p.temperature <= 0.0f || p.top_k == 1;
        if (!greedy && (p.frequency_penalty != 0.0f || p.presence_penalty != 0.0f)) return false;
        const int64_t k = (p.top_k > 0 && p.top_k < V) ? p.top_k : V;
        if (!greedy && k > fs::SK_K) return false;
    }
    return true;
}

// Logits per thread (NL float4 loads) and segments per row: the largest segments that still give every CU four
// workgroups, else the smallest (most workgroups) whose row fits SK_MAX_SEGS lists; 0 when none does.
int small_k_plan(int cus, int64_t B, int32_t V, int& nl, int& nseg) {
    nl = 0;
    nseg = 0;
    const int nls[3] = {16, 8, 4};
    for (int i = 0; i < 3; ++i) {
        const int64_t seg = (int64_t)fs::SK_LT * nls[i] * 4;
        const int64_t n = ((int64_t)V + seg - 1) / seg;
        if (n > fs::SK_MAX_SEGS) break;
        nl = nls[i];
        nseg = (int)n;
        if (B * n >= 4 * (int64_t)cus) break;
    }
    return nl > 0 ? FS_OK : FS_E_INVALID;
}

int grow_small(fs_context* c, size_t slots, size_t rows) {
    if (slots > c->sk_slots) {
        release(c, c->sk_lists);
        c->sk_lists = nullptr; c->sk_slots = 0;
        if (hipMalloc(&c->sk_lists, slots * fs::SK_K * sizeof(uint64_t)) != hipSuccess) return FS_E_NOMEM;
        c->sk_slots = slots;
    }
    if (rows > c->sk_rows) {
        release(c, c->sk_ticket);
        c->sk_ticket = nullptr; c->sk_rows = 0;
        if (hipMalloc(&c->sk_ticket, rows * sizeof(uint32_t)) != hipSuccess) return FS_E_NOMEM;
        if (hipMemset(c->sk_ticket, 0, rows * sizeof(uint32_t)) != hipSuccess) return FS_E_HIP;
        c->sk_rows = rows;
    }
    return FS_OK;
}

// Verification windows fit the small-k kernel when every stream does and none has an active penalty (a row's
// history would then include the drafts fed before it).
bool small_k_windows(const fs_row_params* h, int64_t S, int32_t V) {
    if (!small_k_batch(h, S, V)) return false;
    for (int64_t s = 0; s < S; ++s)
        if ((h[s].repetition_penalty != 1.0f || h[s].frequency_penalty != 0.0f || h[s].presence_penalty != 0.0f) &&
            h[s].repeat_last_n != 0)
            return false;
    return true;
}

// B greedy parameter records without penalties on the device (filled by a kernel on st, no memset: the call may be
// captured) and on the host. The caller holds ctx->mu.
int greedy_params(fs_context* ctx, int64_t B, hipStream_t st) {
    if ((size_t)B <= ctx->greedy_cap) return FS_OK;
    const size_t cap = std::max<size_t>((size_t)B, 2 * ctx->greedy_cap);
    release(ctx, ctx->greedy);
    ctx->greedy = nullptr;
    ctx->greedy_cap = 0;
    if (hipMalloc(&ctx->greedy, cap * sizeof(fs_row_params)) != hipSuccess) return FS_E_NOMEM;
    const int64_t blocks = std::min<int64_t>(1024, ((int64_t)cap + 255) / 256);
    hipLaunchKernelGGL(fs::greedy_params_kernel, dim3((unsigned)blocks), dim3(256), 0, st, ctx->greedy, (int64_t)cap);
    if (hipGetLastError() != hipSuccess) return FS_E_HIP;
    fs_row_params r = {};
    r.temperature = 0.0f; r.top_k = 1; r.top_p = 1.0f; r.repetition_penalty = 1.0f;
    ctx->h_greedy.assign(cap, r);
    ctx->greedy_cap = cap;
    return FS_OK;
}

// The small-k kernel's plan for n host parameter records (B rows, or n_streams windows with `verify`): false when
// the batch does not fit it (the fused kernel runs). nl / nseg: its segments; all_greedy: the greedy-only form;
// capped: some row has a softcap; may_pen: some row has an active penalty window.
struct SmallKChoice {
    int nl = 0, nseg = 0;
    bool all_greedy = true, capped = false, may_pen = false;
};
bool small_k_choice(int cus, const fs_row_params* h, int64_t n, int64_t B, int32_t V, bool verify, SmallKChoice& c) {
    if (verify ? !small_k_windows(h, n, V) : !small_k_batch(h, n, V)) return false;
    if (small_k_plan(cus, B, V, c.nl, c.nseg) != FS_OK) return false;
    if ((int64_t)fs::XCDS * c.nseg * ((B + fs::XCDS - 1) / fs::XCDS) > 0x7fffffff) return false;
    bool counts = false;
    for (int64_t b = 0; b < n; ++b) {
        const fs_row_params& p = h[b];
        const bool fp = p.frequency_penalty != 0.0f || p.presence_penalty != 0.0f;
        c.all_greedy = c.all_greedy && !(p.temperature > 0.0f && p.top_k != 1);
        c.capped |= p.softcap > 0.0f;
        c.may_pen |= (p.repetition_penalty != 1.0f || fp) && p.repeat_last_n != 0;
        counts |= fp && p.repeat_last_n != 0;
    }
    return !(counts && c.nl != 4);               // count tables fit segments of 4096 logits only: the fused kernel
}

// Launches the small-k kernel when the batch fits it; *used = false (nothing launched) otherwise. a.mode selects
// sampling (h_params: B records) or verification windows (h_params: n_streams records).
// h_params NULL: every row greedy without penalties (fs_argmax_batch without parameters): the context's greedy
// records stand for the parameters, on the device and the host.
int launch_small(fs_context* ctx, const fs::Args& a_in, const fs_row_params* h_params, hipStream_t st, bool& used) {
    used = false;
    std::lock_guard<std::mutex> g(ctx->mu);
    int rc = device_of(ctx);
    if (rc != FS_OK) return rc;
    fs::Args a = a_in;
    if (!h_params) {
        rc = greedy_params(ctx, a.B, st);
        if (rc != FS_OK) return rc;
        h_params = ctx->h_greedy.data();
        a.params = ctx->greedy;
    }
    const bool verify = a.mode == fs::MODE_VERIFY;
    if (!ctx->seg_layout) return FS_OK;
    SmallKChoice ch;
    if (!small_k_choice(ctx->cus, h_params, verify ? (int64_t)a.n_streams : (int64_t)a.B, a.B, a.V, verify, ch))
        return FS_OK;
    const int nl = ch.nl, nseg = ch.nseg;
    const int64_t per_x = ((int64_t)a.B + fs::XCDS - 1) / fs::XCDS;
    const int64_t grid = (int64_t)fs::XCDS * nseg * per_x;
    // the error word and the verify stream counters: a 64-bit word per stream, then the 32-bit counters of streams
    // longer than 32 rows
    rc = grow(ctx, 0, 0, verify ? 3 * (size_t)a.n_streams : 0);
    if (rc != FS_OK) return rc;
    rc = grow_small(ctx, (size_t)a.B * nseg, (size_t)a.B);
    if (rc != FS_OK) return rc;
    if (capturing(st)) ctx->captured = true;
    fs::SkArgs k = {};
    k.logits = a.logits; k.ld = a.ld; k.B = a.B; k.V = a.V; k.nseg = nseg;
    k.hist = a.hist; k.hist_off = a.hist_off; k.params = a.params; k.u = a.u; k.tok = a.tok; k.kcap = a.kcap;
    k.cand_ids = a.cand_ids; k.cand_probs = a.cand_probs; k.keep = a.keep;
    k.lists = ctx->sk_lists; k.ticket = ctx->sk_ticket; k.err = ctx->err;
    k.mode = a.mode; k.rows = a.rows; k.row_off = a.row_off; k.n_streams = a.n_streams; k.eos = a.eos;
    k.accepted = a.accepted; k.stream_cnt = ctx->stream_cnt;
    k.dmt = a.dmt; k.didx = a.didx; k.out_hist = a.out_hist; k.out_hist_off = a.out_hist_off; k.out_cap = a.out_cap;
    k.trace = nullptr;
#ifdef FS_TRACE
    if (ctx->trace && grid * fs::TRACE_W <= ctx->trace_cap) k.trace = ctx->trace;
#endif
    const bool capped = ch.capped, all_greedy = ch.all_greedy;
    bool may_pen = ch.may_pen;
    // a verification window reaches this kernel only without an active penalty (small_k_windows)
    may_pen = may_pen && !verify && a.hist && a.hist_off;
    const dim3 gd((unsigned)grid), bd(fs::SK_LT);
    // all-greedy batches: the greedy-only kernel, without the LDS pad (its registers allow more workgroups per CU)
    auto go = [&](auto kern, unsigned pad) {
        hipLaunchKernelGGL(kern, gd, bd, pad, st, a.logits, a.ld, a.B, a.V, nseg, may_pen ? 1 : 0, a.params,
                           a.hist_off, a.hist, k);
    };
    const unsigned pad = fs::SK_PAD_LDS;
    if (all_greedy) {
        if (capped) {
            if (nl == 16) go(fs::small_k_kernel<16, true, true>, 0u);
            else if (nl == 8) go(fs::small_k_kernel<8, true, true>, 0u);
            else go(fs::small_k_kernel<4, true, true>, 0u);
        } else {
            if (nl == 16) go(fs::small_k_kernel<16, false, true>, 0u);
            else if (nl == 8) go(fs::small_k_kernel<8, false, true>, 0u);
            else go(fs::small_k_kernel<4, false, true>, 0u);
        }
    } else if (capped) {
        if (nl == 16) go(fs::small_k_kernel<16, true, false>, pad);
        else if (nl == 8) go(fs::small_k_kernel<8, true, false>, pad);
        else go(fs::small_k_kernel<4, true, false>, pad);
    } else {
        if (nl == 16) go(fs::small_k_kernel<16, false, false>, pad);
        else if (nl == 8) go(fs::small_k_kernel<8, false, false>, pad);
        else go(fs::small_k_kernel<4, false, false>, pad);
    }
    if (hipGetLastError() != hipSuccess) return FS_E_HIP;
    used = true;
    return FS_OK;
}

int launch(fs_context* ctx, fs::Args a, int64_t rows, int64_t streams, hipStream_t st, int per_cu = 2) {
    std::lock_guard<std::mutex> g(ctx->mu);
    int rc = device_of(ctx);
    if (rc != FS_OK) return rc;
    int64_t items = 0, seg_grid = 0;
    rc = plan(ctx->cus, a, rows, items, seg_grid, 0, per_cu);
    if (rc != FS_OK) return rc;
    // verify: a 64-bit word per stream, then the 32-bit counters of streams longer than 32 rows
    rc = grow(ctx, (size_t)(items > 0 ? items : 1), (size_t)rows, (size_t)(streams > 0 ? 3 * streams : 1));
    if (rc != FS_OK) return rc;
    if (capturing(st)) ctx->captured = true;
    a.cand = ctx->cand; a.meta = ctx->meta; a.rhist = ctx->rhist; a.rmass = ctx->rmass;
    a.stream_cnt = ctx->stream_cnt; a.err = ctx->err; a.dirty = ctx->err + 1; a.merge_spins = ctx->merge_spins;
    a.trace = nullptr;
    int done = FS_OK;
    if (gave_up(ctx->hflag)) {
        clear_words(st, ctx->rhist, (int64_t)(ctx->row_cap * fs::RBINS));
        clear_words(st, ctx->rmass, (int64_t)(ctx->row_cap * fs::LB * 2));
        clear_words(st, ctx->stream_cnt, (int64_t)ctx->stream_cap);
        clear_words(st, ctx->err + 1, 1);
        if (hipGetLastError() != hipSuccess) return FS_E_HIP;
        done = FS_W_RECOVERED;
    }
    if (!ctx->seg_layout) {
        rc = launch_alone(a, rows, st);
        return rc != FS_OK ? rc : done;
    }
#ifdef FS_TRACE
    {
        const int64_t grid = seg_grid > 0 ? seg_grid + (int64_t)fs::XCDS * ((rows + fs::XCDS - 1) / fs::XCDS) : rows;
        if (ctx->trace && grid * fs::TRACE_W <= ctx->trace_cap) a.trace = ctx->trace;   // else: untraced
    }
#endif
    rc = launch_planned(a, rows, seg_grid, st);
    return rc != FS_OK ? rc : done;
}

}  // namespace

// ------------------------------------------------------------------------------------------------ static workspace
// fs_sample_batch_static's workspace: one file-scope device array per GPU, held until the process ends, so the
// call allocates nothing. Layout (bytes): error word and dirty flag | meta [ST_SLOTS][2] | row histograms
// [ST_ROWS][RBINS] | large rows' mass histograms [ST_ROWS][LB] | candidate lists [ST_SLOTS][CAP]. The row and mass
// histograms (counters included) must be zero when a call starts; the kernels leave them so, and the first call on a
// device clears them with a fill kernel (no hipMemsetAsync: the call may be recorded into a graph).
constexpr int64_t ST_ROWS = 512;                                  // rows per call
constexpr int64_t ST_SLOTS = 512;                                 // (row, segment) slots per call
constexpr size_t ST_ERR_OFF = 0;                                  // int32 [2]: error bits, dirty
constexpr size_t ST_META_OFF = 256;
constexpr size_t ST_RHIST_OFF = ST_META_OFF + ((ST_SLOTS * 2 * sizeof(uint32_t) + 255) / 256) * 256;
constexpr size_t ST_RMASS_OFF = ST_RHIST_OFF + (size_t)ST_ROWS * fs::RBINS * sizeof(uint32_t);
constexpr size_t ST_CAND_OFF = ST_RMASS_OFF + (size_t)ST_ROWS * fs::LB * sizeof(uint64_t);
constexpr size_t ST_BYTES = ST_CAND_OFF + (size_t)ST_SLOTS * fs::CAP * sizeof(uint64_t);   // 50,336,000 B

static __device__ __align__(256) unsigned char scratch[ST_BYTES];


namespace {

constexpr int ST_MAX_DEVICES = 64;
std::mutex g_static_mu;
unsigned char* g_static_ptr[ST_MAX_DEVICES] = {};   // the device address of `scratch` on each device
int32_t* g_static_flag[ST_MAX_DEVICES] = {};        // host-mapped give-up flag of each device's static workspace

__global__ void store_u64_kernel(uint64_t* p, uint64_t v) { *p = v; }

// The static workspace of the current device: its address from hipGetSymbolAddress (the array's name is not a
// device address in host code), once per device; the first call also zeroes the error words and row histograms
// on `st`, ahead of its own launch.
int static_workspace(int dev, hipStream_t st, unsigned char** out) {
    if (dev < 0 || dev >= ST_MAX_DEVICES) return FS_E_INVALID;
    std::lock_guard<std::mutex> g(g_static_mu);
    if (!g_static_ptr[dev]) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return FS_E_HIP;
        unsigned char* base = (unsigned char*)ptr;
        int32_t* flag = nullptr;
        int32_t* flag_dev = nullptr;
        if (hipHostMalloc((void**)&flag, sizeof(int32_t), hipHostMallocMapped) != hipSuccess) return FS_E_NOMEM;
        *(volatile int32_t*)flag = 0;
        if (hipHostGetDevicePointer((void**)&flag_dev, flag, 0) != hipSuccess) return FS_E_HIP;
        hipLaunchKernelGGL(fs::zero_words_kernel, dim3(1), dim3(256), 0, st, (uint32_t*)(base + ST_ERR_OFF),
                           (int64_t)(ST_META_OFF / 4));
        // error word 2..3: the give-up flag's device address (a kernel store: the call may be under graph capture)
        hipLaunchKernelGGL(store_u64_kernel, dim3(1), dim3(1), 0, st, (uint64_t*)(base + ST_ERR_OFF + 8),
                           (uint64_t)(uintptr_t)flag_dev);
        g_static_flag[dev] = flag;
        hipLaunchKernelGGL(fs::zero_words_kernel, dim3(1024), dim3(256), 0, st, (uint32_t*)(base + ST_RHIST_OFF),
                           (int64_t)((ST_CAND_OFF - ST_RHIST_OFF) / 4));   // row and mass histograms
        if (hipGetLastError() != hipSuccess) return FS_E_HIP;
        g_static_ptr[dev] = base;
    }
    *out = g_static_ptr[dev];
    return FS_OK;
}

}  // namespace

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_rows(const float* d_logits, int64_t ld, int32_t B, int32_t V) {
    if (!d_logits || B < 0 || V < 1 || V > FS_MAX_VOCAB || ld < V || (ld & 3) != 0 || !aligned16(d_logits))
        return FS_E_INVALID;
    return FS_OK;
}

}  // namespace

extern "C" {

int fs_create(fs_context** out) {
    if (!out) return FS_E_INVALID;
    *out = new (std::nothrow) fs_context();
    return *out ? FS_OK : FS_E_NOMEM;
}

int fs_destroy(fs_context* c) {
    if (!c) return FS_E_INVALID;
    (void)hipFree(c->sk_lists);
    (void)hipFree(c->sk_ticket);
    (void)hipFree(c->cand);
    (void)hipFree(c->meta);
    (void)hipFree(c->rhist);
    (void)hipFree(c->rmass);
    (void)hipFree(c->stream_cnt);
    (void)hipFree(c->err);
    (void)hipFree(c->greedy);
    for (void* p : c->retired) (void)hipFree(p);
    if (c->hflag) (void)hipHostFree(c->hflag);
    delete c;
    return FS_OK;
}

int fs_sample_batch(fs_context* ctx, const float* d_logits, int64_t ld, int32_t B, int32_t V, const int32_t* d_hist,
                    const int64_t* d_hist_off, const fs_row_params* d_params, const double* d_u, int32_t* d_tok,
                    int32_t kcap, int32_t* d_cand_ids, double* d_cand_probs, int32_t* d_keep, void* stream) {
    if (!ctx || !d_params || !d_tok || kcap < 0 || ((d_cand_ids || d_cand_probs) && kcap == 0)) return FS_E_INVALID;
    int rc = check_rows(d_logits, ld, B, V);
    if (rc != FS_OK) return rc;
    if (B == 0) return FS_OK;
    fs::Args a = {};
    a.logits = d_logits; a.ld = ld; a.B = B; a.V = V; a.hist = d_hist; a.hist_off = d_hist_off; a.params = d_params;
    a.u = d_u; a.tok = d_tok; a.kcap = kcap; a.cand_ids = d_cand_ids; a.cand_probs = d_cand_probs; a.keep = d_keep;
    a.mode = fs::MODE_SAMPLE; a.eos = -1;
    return launch(ctx, a, B, 0, (hipStream_t)stream);
}

int fs_sample_batch_hp(fs_context* ctx, const float* d_logits, int64_t ld, int32_t B, int32_t V,
                       const int32_t* d_hist, const int64_t* d_hist_off, const fs_row_params* d_params,
                       const fs_row_params* h_params, const double* d_u, int32_t* d_tok, int32_t kcap,
                       int32_t* d_cand_ids, double* d_cand_probs, int32_t* d_keep, void* stream) {
    if (!ctx || !d_params || !d_tok || kcap < 0 || ((d_cand_ids || d_cand_probs) && kcap == 0)) return FS_E_INVALID;
    int rc = check_rows(d_logits, ld, B, V);
    if (rc != FS_OK) return rc;
    if (B == 0) return FS_OK;
    fs::Args a = {};
    a.logits = d_logits; a.ld = ld; a.B = B; a.V = V; a.hist = d_hist; a.hist_off = d_hist_off; a.params = d_params;
    a.u = d_u; a.tok = d_tok; a.kcap = kcap; a.cand_ids = d_cand_ids; a.cand_probs = d_cand_probs; a.keep = d_keep;
    a.mode = fs::MODE_SAMPLE; a.eos = -1;
    if (h_params) {
        bool used = false;
        rc = launch_small(ctx, a, h_params, (hipStream_t)stream, used);
        if (rc != FS_OK || used) return rc;
        if (mixed_merges(h_params, B, V)) return launch(ctx, a, B, 0, (hipStream_t)stream, 4);
    }
    return launch(ctx, a, B, 0, (hipStream_t)stream);
}

int fs_verify_hp(fs_context* ctx, const float* d_logits, int64_t ld, int32_t n_streams, int32_t total_rows, int32_t V,
                 const int32_t* d_rows, const int64_t* d_row_off, const int32_t* d_hist, const int64_t* d_hist_off,
                 const fs_row_params* d_params, const fs_row_params* h_params, const double* d_u, int32_t eos_id,
                 int32_t* d_tok, int32_t* d_accepted, void* stream) {
    if (!ctx || !d_rows || !d_row_off || !d_params || !d_tok || !d_accepted || n_streams < 0 || total_rows < 0)
        return FS_E_INVALID;
    int rc = check_rows(d_logits, ld, total_rows, V);
    if (rc != FS_OK) return rc;
    if (total_rows == 0 || n_streams == 0) return FS_OK;
    fs::Args a = {};
    a.logits = d_logits; a.ld = ld; a.B = total_rows; a.V = V; a.hist = d_hist; a.hist_off = d_hist_off;
    a.params = d_params; a.u = d_u; a.tok = d_tok; a.rows = d_rows; a.row_off = d_row_off; a.n_streams = n_streams;
    a.eos = eos_id; a.accepted = d_accepted; a.mode = fs::MODE_VERIFY;
    if (h_params) {
        bool used = false;
        rc = launch_small(ctx, a, h_params, (hipStream_t)stream, used);
        if (rc != FS_OK || used) return rc;
    }
    return launch(ctx, a, total_rows, n_streams, (hipStream_t)stream);
}

int fs_small_k_plan(int32_t cus, int32_t B, int32_t V, int32_t* nl, int32_t* nseg) {
    if (cus < 1 || B < 1 || V < 1 || V > FS_MAX_VOCAB || !nl || !nseg) return FS_E_INVALID;
    int l = 0, n = 0;
    const int rc = small_k_plan(cus, B, V, l, n);
    *nl = l;
    *nseg = n;
    return rc == FS_OK ? FS_OK : FS_E_LIMIT;
}

int fs_route_plan(int32_t cus, const fs_row_params* h_params, int32_t n, int32_t total_rows, int32_t V,
                  int32_t verify, int32_t* kernel, int32_t* nl, int32_t* nseg, int32_t* per_cu) {
    if (cus < 1 || !h_params || n < 1 || total_rows < 1 || V < 1 || V > FS_MAX_VOCAB || !kernel || !nl || !nseg ||
        !per_cu)
        return FS_E_INVALID;
    if (!verify && total_rows != n) return FS_E_INVALID;
    SmallKChoice ch;
    *nl = 0;
    if (small_k_choice(cus, h_params, n, total_rows, V, verify != 0, ch)) {
        *kernel = ch.all_greedy ? 2 : 1;
        *nl = ch.nl;
        *nseg = ch.nseg;
        *per_cu = 0;
        return FS_OK;
    }
    fs::Args a = {};
    a.V = V;
    a.mode = verify ? fs::MODE_VERIFY : fs::MODE_SAMPLE;
    *per_cu = (!verify && mixed_merges(h_params, n, V)) ? 4 : 2;
    int64_t items = 0, seg_grid = 0;
    const int rc = plan(cus, a, total_rows, items, seg_grid, 0, *per_cu);
    if (rc != FS_OK) return rc;
    *kernel = 0;
    *nseg = a.nseg;
    return FS_OK;
}

int fs_sample_batch_static(fs_context* ctx, const float* d_logits, int64_t ld, int32_t B, int32_t V,
                           const int32_t* d_hist, const int64_t* d_hist_off, const fs_row_params* d_params,
                           const double* d_u, int32_t* d_tok, int32_t kcap, int32_t* d_cand_ids, double* d_cand_probs,
                           int32_t* d_keep, void* stream) {
    if (!ctx || !d_params || !d_tok || kcap < 0 || ((d_cand_ids || d_cand_probs) && kcap == 0)) return FS_E_INVALID;
    int rc = check_rows(d_logits, ld, B, V);
    if (rc != FS_OK) return rc;
    if (B == 0) return FS_OK;
    if (B > ST_ROWS) return FS_E_LIMIT;
    fs::Args a = {};
    a.logits = d_logits; a.ld = ld; a.B = B; a.V = V; a.hist = d_hist; a.hist_off = d_hist_off; a.params = d_params;
    a.u = d_u; a.tok = d_tok; a.kcap = kcap; a.cand_ids = d_cand_ids; a.cand_probs = d_cand_probs; a.keep = d_keep;
    a.mode = fs::MODE_SAMPLE; a.eos = -1;
    const hipStream_t st = (hipStream_t)stream;
    std::lock_guard<std::mutex> g(ctx->mu);
    rc = device_of(ctx);
    if (rc != FS_OK) return rc;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return FS_E_HIP;
    if (ctx->static_dev >= 0 && ctx->static_dev != dev) return FS_E_INVALID;   // a context stays on one device
    int64_t items = 0, seg_grid = 0;
    rc = plan(ctx->cus, a, B, items, seg_grid, ST_SLOTS);        // fewer segments per row where the slots run out
    if (rc != FS_OK) return rc;
    if (items > ST_SLOTS) return FS_E_LIMIT;
    unsigned char* base = nullptr;
    rc = static_workspace(dev, st, &base);
    if (rc != FS_OK) return rc;
    ctx->static_dev = dev;
    a.err = (int32_t*)(base + ST_ERR_OFF); a.dirty = a.err + 1;
    a.meta = (uint32_t*)(base + ST_META_OFF);
    a.rhist = (uint32_t*)(base + ST_RHIST_OFF);
    a.rmass = (uint64_t*)(base + ST_RMASS_OFF);
    a.cand = (uint64_t*)(base + ST_CAND_OFF);
    a.stream_cnt = nullptr;                          // sampling mode has no verify streams
    a.merge_spins = ctx->merge_spins;
    int done = FS_OK;
    int32_t* sflag = nullptr;
    {
        std::lock_guard<std::mutex> gs(g_static_mu);
        sflag = g_static_flag[dev];
    }
    if (gave_up(sflag)) {                            // an earlier call on the device gave up: clear what it left
        clear_words(st, base + ST_RHIST_OFF, (int64_t)((ST_CAND_OFF - ST_RHIST_OFF) / 4));
        clear_words(st, a.dirty, 1);
        if (hipGetLastError() != hipSuccess) return FS_E_HIP;
        done = FS_W_RECOVERED;
    }
    rc = ctx->seg_layout ? launch_planned(a, B, seg_grid, st) : launch_alone(a, B, st);
    return rc != FS_OK ? rc : done;
}

int fs_argmax_batch(fs_context* ctx, const float* d_logits, int64_t ld, int32_t B, int32_t V, const int32_t* d_hist,
                    const int64_t* d_hist_off, const fs_row_params* d_params, int32_t* d_tok, void* stream) {
    if (!ctx || !d_tok) return FS_E_INVALID;
    int rc = check_rows(d_logits, ld, B, V);
    if (rc != FS_OK) return rc;
    if (B == 0) return FS_OK;
    fs::Args a = {};
    a.logits = d_logits; a.ld = ld; a.B = B; a.V = V; a.hist = d_hist; a.hist_off = d_params ? d_hist_off : nullptr;
    a.params = d_params; a.tok = d_tok; a.mode = fs::MODE_ARGMAX; a.eos = -1;
    if (!d_params) {
        // no penalties: every row greedy, so the small-k kernel's greedy path takes the batch (its parameters are
        // greedy records the context keeps on the device and the host)
        fs::Args g = a;
        g.mode = fs::MODE_SAMPLE;
        g.hist = nullptr;
        bool used = false;
        rc = launch_small(ctx, g, nullptr, (hipStream_t)stream, used);
        if (rc != FS_OK || used) return rc;
    }
    return launch(ctx, a, B, 0, (hipStream_t)stream);
}

int fs_verify(fs_context* ctx, const float* d_logits, int64_t ld, int32_t n_streams, int32_t total_rows, int32_t V,
              const int32_t* d_rows, const int64_t* d_row_off, const int32_t* d_hist, const int64_t* d_hist_off,
              const fs_row_params* d_params, const double* d_u, int32_t eos_id, int32_t* d_tok, int32_t* d_accepted,
              void* stream) {
    if (!ctx || !d_rows || !d_row_off || !d_params || !d_tok || !d_accepted || n_streams < 0 || total_rows < 0)
        return FS_E_INVALID;
    int rc = check_rows(d_logits, ld, total_rows, V);
    if (rc != FS_OK) return rc;
    if (total_rows == 0 || n_streams == 0) return FS_OK;
    fs::Args a = {};
    a.logits = d_logits; a.ld = ld; a.B = total_rows; a.V = V; a.hist = d_hist; a.hist_off = d_hist_off;
    a.params = d_params; a.u = d_u; a.tok = d_tok; a.rows = d_rows; a.row_off = d_row_off; a.n_streams = n_streams;
    a.eos = eos_id; a.accepted = d_accepted; a.mode = fs::MODE_VERIFY;
    return launch(ctx, a, total_rows, n_streams, (hipStream_t)stream);
}

int fs_penalize_batch(fs_context* ctx, float* d_logits, int64_t ld, int32_t B, int32_t V, const int32_t* d_hist,
                      const int64_t* d_hist_off, const fs_row_params* d_params, void* stream) {
    if (!ctx || !d_params) return FS_E_INVALID;
    int rc = check_rows(d_logits, ld, B, V);
    if (rc != FS_OK) return rc;
    if (B == 0 || !d_hist || !d_hist_off) return FS_OK;
    const int64_t nchunk = ((int64_t)V + fs::PEN_CHUNK - 1) / fs::PEN_CHUNK;
    if ((int64_t)B * nchunk > 0x7fffffff) return FS_E_INVALID;
    {
        std::lock_guard<std::mutex> g(ctx->mu);
        rc = grow(ctx, 0, 0, 0);
        if (rc != FS_OK) return rc;
    }
    hipLaunchKernelGGL(fs::penalize_kernel, dim3((unsigned)(B * nchunk)), dim3(fs::PEN_BLOCK), 0, (hipStream_t)stream,
                       d_logits, ld, V, d_hist, d_hist_off, d_params, (int)nchunk, ctx->err);
    return hipGetLastError() == hipSuccess ? FS_OK : FS_E_HIP;
}

int fs_softcap_batch(const float* d_in, float* d_out, int64_t n, float cap, void* stream) {
    if (n < 0 || (n > 0 && (!d_in || !d_out)) || !(cap > 0.0f)) return FS_E_INVALID;
    if (n == 0) return FS_OK;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fs::softcap_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, d_in, d_out, n,
                       cap);
    return hipGetLastError() == hipSuccess ? FS_OK : FS_E_HIP;
}

int fs_lookup_draft(fs_context* ctx, int32_t n_streams, const int32_t* d_hist, const int64_t* d_hist_off,
                    const int32_t* d_kmax, const int32_t* d_min_n, int32_t eos_id, int32_t* d_draft, int32_t draft_ld,
                    int32_t* d_ndraft, void* stream) {
    if (!ctx || n_streams < 0 || !d_hist_off || !d_draft || !d_ndraft || draft_ld < 1) return FS_E_INVALID;
    if (n_streams == 0) return FS_OK;
    hipLaunchKernelGGL(fs::lookup_draft_kernel, dim3((unsigned)n_streams), dim3(fs::LD_BLOCK), 0, (hipStream_t)stream,
                       d_hist, d_hist_off, d_kmax, d_min_n, eos_id, d_draft, draft_ld, d_ndraft);
    return hipGetLastError() == hipSuccess ? FS_OK : FS_E_HIP;
}

int fs_hist_append(fs_context* ctx, int32_t n_streams, const int32_t* d_hist, const int64_t* d_hist_off,
                   const int32_t* d_tok, const int64_t* d_row_off, const int32_t* d_count, int32_t* d_out_hist,
                   int64_t out_cap, int64_t* d_out_hist_off, void* stream) {
    if (!ctx || n_streams < 0 || !d_hist_off || !d_out_hist_off || out_cap < 0) return FS_E_INVALID;
    if (n_streams > 0 && (!d_tok || !d_hist)) return FS_E_INVALID;
    if (out_cap > 0 && !d_out_hist) return FS_E_INVALID;
    if (d_out_hist_off == d_hist_off || (d_out_hist && d_out_hist == d_hist)) return FS_E_INVALID;   // out of place
    {
        std::lock_guard<std::mutex> g(ctx->mu);
        const int rc = grow(ctx, 1, 1, 1);               // the device error word
        if (rc != FS_OK) return rc;
    }
    const hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(fs::hist_offsets_kernel, dim3(1), dim3(fs::BLOCK), 0, st, (int)n_streams, d_hist_off,
                       d_row_off, d_count, d_out_hist_off, out_cap, ctx->err);
    if (hipGetLastError() != hipSuccess) return FS_E_HIP;
    if (n_streams == 0) return FS_OK;
    hipLaunchKernelGGL(fs::hist_append_kernel, dim3((unsigned)n_streams), dim3(fs::LD_BLOCK), 0, st, d_hist,
                       d_hist_off, d_tok, d_row_off, d_count, d_out_hist_off, d_out_hist, out_cap);
    return hipGetLastError() == hipSuccess ? FS_OK : FS_E_HIP;
}

int fs_device_error(fs_context* ctx, void* stream, int32_t* bits) {
    if (!ctx || !bits) return FS_E_INVALID;
    *bits = 0;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (!ctx->err && ctx->static_dev < 0) return FS_OK;
    if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) return FS_E_HIP;
    if (ctx->err) {
        int32_t h[2] = {0, 0};
        if (hipMemcpy(h, ctx->err, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) return FS_E_HIP;
        *bits |= h[0];
        if (h[1] != 0) {
            // a merge gave up: the segments it did not wait for have finished by now (the stream is idle), so the
            // row histograms and counters are cleared and the context leaves its compute-alone mode
            if (ctx->rhist && hipMemset(ctx->rhist, 0, ctx->row_cap * fs::RBINS * sizeof(uint32_t)) != hipSuccess)
                return FS_E_HIP;
            if (ctx->rmass && hipMemset(ctx->rmass, 0, ctx->row_cap * fs::LB * sizeof(uint64_t)) != hipSuccess)
                return FS_E_HIP;
            if (ctx->stream_cnt && hipMemset(ctx->stream_cnt, 0, ctx->stream_cap * sizeof(uint32_t)) != hipSuccess)
                return FS_E_HIP;
        }
        if (hipMemset(ctx->err, 0, sizeof(h)) != hipSuccess) return FS_E_HIP;
    }
    if (ctx->static_dev >= 0) {
        // the device's static workspace (fs_sample_batch_static), shared by every context on the device
        unsigned char* base = nullptr;
        {
            std::lock_guard<std::mutex> gs(g_static_mu);
            base = g_static_ptr[ctx->static_dev];
        }
        if (base) {
            int32_t h[2] = {0, 0};
            if (hipMemcpy(h, base + ST_ERR_OFF, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) return FS_E_HIP;
            *bits |= h[0];
            if (h[1] != 0 && hipMemset(base + ST_RHIST_OFF, 0, ST_CAND_OFF - ST_RHIST_OFF) != hipSuccess)
                return FS_E_HIP;
            if (hipMemset(base + ST_ERR_OFF, 0, sizeof(h)) != hipSuccess) return FS_E_HIP;
        }
    }
    return FS_OK;
}

int fs_plan_layout(int32_t cus, int32_t xccs, int32_t B, int32_t V, int32_t static_ws, int32_t* nseg,
                   int32_t* seg_tiles, int64_t* slots) {
    if (cus < 1 || xccs < 0 || B < 1 || V < 1 || V > FS_MAX_VOCAB || !nseg || !seg_tiles || !slots) return FS_E_INVALID;
    if (static_ws && B > ST_ROWS) return FS_E_LIMIT;
    *nseg = 0; *seg_tiles = 0; *slots = 0;
    if (!layout_fits(xccs)) return FS_OK;                 // every row sampled alone by one workgroup
    fs::Args a = {};
    a.B = B; a.V = V; a.mode = fs::MODE_SAMPLE;
    int64_t items = 0, seg_grid = 0;
    const int rc = plan(cus, a, B, items, seg_grid, static_ws ? ST_SLOTS : 0);
    if (rc != FS_OK) return rc;
    if (static_ws && items > ST_SLOTS) return FS_E_LIMIT;
    *nseg = a.nseg; *seg_tiles = a.seg_tiles; *slots = items;
    return FS_OK;
}

int fs_error_word(fs_context* ctx, const int32_t** d_bits) {
    if (!ctx || !d_bits) return FS_E_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    const int rc = grow(ctx, 0, 0, 0);
    if (rc != FS_OK) return rc;
    *d_bits = ctx->err;
    return FS_OK;
}

int fs_set_wait_limit(fs_context* ctx, uint32_t polls) {
    if (!ctx) return FS_E_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    ctx->merge_spins = polls == FS_WAIT_GIVE_UP ? 0u : (polls ? polls : fs::MERGE_SPINS);
    return FS_OK;
}

// Per-stream draw source of ferro::Sampler (sampler.h:25,32 and the draw at sampler.cpp:45-46): the same libstdc++
// engine and canonical mapping, so u * tot equals uniform_real_distribution<double>(0, tot)(rng) bit for bit.
struct fs_rng {
    std::mt19937_64 eng;
};

int fs_rng_create(uint64_t seed, fs_rng** out) {
    if (!out) return FS_E_INVALID;
    *out = new (std::nothrow) fs_rng();
    if (!*out) return FS_E_NOMEM;
    (*out)->eng.seed(seed ? seed : (uint64_t)std::random_device{}());
    return FS_OK;
}

int fs_rng_destroy(fs_rng* r) {
    if (!r) return FS_E_INVALID;
    delete r;
    return FS_OK;
}

int fs_rng_next_u(fs_rng* r, double* u, int32_t n) {
    if (!r || !u || n < 0) return FS_E_INVALID;
    for (int32_t i = 0; i < n; ++i) u[i] = std::generate_canonical<double, 53>(r->eng);
    return FS_OK;
}

int fs_rng_copy(const fs_rng* src, fs_rng* dst) {
    if (!src || !dst) return FS_E_INVALID;
    dst->eng = src->eng;
    return FS_OK;
}

// Device draw streams (see fs::drng_draw_kernel): the engines' states live in device memory; seeding follows the
// standard's seed sequence for mt19937_64 (x0 = seed, x_i = 6364136223846793005 * (x_{i-1} ^ (x_{i-1} >> 62)) + i),
// so stream s reproduces std::mt19937_64(seed_s) and ferro::Sampler's draws.
struct fs_drng {
    int device = -1;
    int n = 0;
    uint64_t* mt = nullptr;     // [n][312]
    int32_t* idx = nullptr;     // [n]
    int32_t* err = nullptr;
};

// fs_decode_step: fs_sample_batch with the draws taken from the device streams r (row s = stream s) and each row's
// token appended to its stream's history out of place, in the sampling grid itself (one launch).
int fs_decode_step_hp(fs_context* ctx, fs_drng* r, const float* d_logits, int64_t ld, int32_t B, int32_t V,
                      const int32_t* d_hist, const int64_t* d_hist_off, const fs_row_params* d_params,
                      const fs_row_params* h_params, int32_t* d_tok, int32_t* d_keep, int32_t* d_out_hist,
                      int64_t* d_out_hist_off, int64_t out_cap, void* stream) {
    if (!ctx || !r || !d_params || !d_tok || !d_out_hist_off || out_cap < 0 || (out_cap > 0 && !d_out_hist) ||
        (d_hist == nullptr) != (d_hist_off == nullptr) || B > r->n)
        return FS_E_INVALID;
    int rc = check_rows(d_logits, ld, B, V);
    if (rc != FS_OK) return rc;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return FS_E_HIP;
    if (dev != r->device) return FS_E_INVALID;
    if (B == 0) return FS_OK;
    fs::Args a = {};
    a.logits = d_logits; a.ld = ld; a.B = B; a.V = V; a.hist = d_hist; a.hist_off = d_hist_off; a.params = d_params;
    a.u = nullptr; a.tok = d_tok; a.kcap = 0; a.keep = d_keep;
    a.mode = fs::MODE_SAMPLE; a.eos = -1;
    a.dmt = r->mt; a.didx = r->idx; a.out_hist = d_out_hist; a.out_hist_off = d_out_hist_off; a.out_cap = out_cap;
    if (h_params) {
        bool used = false;
        rc = launch_small(ctx, a, h_params, (hipStream_t)stream, used);
        if (rc != FS_OK || used) return rc;
    }
    return launch(ctx, a, B, 0, (hipStream_t)stream);
}

int fs_decode_step(fs_context* ctx, fs_drng* r, const float* d_logits, int64_t ld, int32_t B, int32_t V,
                   const int32_t* d_hist, const int64_t* d_hist_off, const fs_row_params* d_params, int32_t* d_tok,
                   int32_t* d_keep, int32_t* d_out_hist, int64_t* d_out_hist_off, int64_t out_cap, void* stream) {
    return fs_decode_step_hp(ctx, r, d_logits, ld, B, V, d_hist, d_hist_off, d_params, nullptr, d_tok, d_keep,
                             d_out_hist, d_out_hist_off, out_cap, stream);
}

int fs_drng_create(int32_t n_streams, const uint64_t* seeds, void* stream, fs_drng** out) {
    if (!out || n_streams < 1 || !seeds) return FS_E_INVALID;
    *out = nullptr;
    fs_drng* r = new (std::nothrow) fs_drng();
    if (!r) return FS_E_NOMEM;
    std::vector<uint64_t> mt((size_t)n_streams * fs::MT_N);
    std::vector<int32_t> idx((size_t)n_streams, fs::MT_N);
    std::random_device rd;
    for (int32_t s = 0; s < n_streams; ++s) {
        uint64_t* x = mt.data() + (size_t)s * fs::MT_N;
        x[0] = seeds[s] ? seeds[s] : (uint64_t)rd();                     // seed 0 = random, as ferro
        for (int i = 1; i < fs::MT_N; ++i) x[i] = 6364136223846793005ull * (x[i - 1] ^ (x[i - 1] >> 62)) + (uint64_t)i;
    }
    r->n = n_streams;
    int rc = FS_OK;
    if (hipGetDevice(&r->device) != hipSuccess) rc = FS_E_HIP;
    if (rc == FS_OK && (hipMalloc(&r->mt, mt.size() * sizeof(uint64_t)) != hipSuccess ||
                        hipMalloc(&r->idx, idx.size() * sizeof(int32_t)) != hipSuccess ||
                        hipMalloc(&r->err, sizeof(int32_t)) != hipSuccess))
        rc = FS_E_NOMEM;
    hipStream_t st = (hipStream_t)stream;
    if (rc == FS_OK && (hipMemcpyAsync(r->mt, mt.data(), mt.size() * sizeof(uint64_t), hipMemcpyHostToDevice, st) != hipSuccess ||
                        hipMemcpyAsync(r->idx, idx.data(), idx.size() * sizeof(int32_t), hipMemcpyHostToDevice, st) != hipSuccess ||
                        hipMemsetAsync(r->err, 0, sizeof(int32_t), st) != hipSuccess ||
                        hipStreamSynchronize(st) != hipSuccess))
        rc = FS_E_HIP;
    if (rc != FS_OK) { fs_drng_destroy(r); return rc; }
    *out = r;
    return FS_OK;
}

int fs_drng_destroy(fs_drng* r) {
    if (!r) return FS_E_INVALID;
    (void)hipFree(r->mt);
    (void)hipFree(r->idx);
    (void)hipFree(r->err);
    delete r;
    return FS_OK;
}

int fs_drng_draw(fs_drng* r, const int64_t* d_row_off, const fs_row_params* d_params, double* d_u, int32_t peek,
                 void* stream) {
    if (!r || !d_params || !d_u) return FS_E_INVALID;
    hipLaunchKernelGGL(fs::drng_draw_kernel, dim3((unsigned)((r->n + 63) / 64)), dim3(64), 0, (hipStream_t)stream,
                       r->mt, r->idx, r->n, d_row_off, d_params, d_u, peek ? 1 : 0, r->err);
    return hipGetLastError() == hipSuccess ? FS_OK : FS_E_HIP;
}

int fs_drng_skip(fs_drng* r, const int32_t* d_counts, const fs_row_params* d_params, void* stream) {
    if (!r || !d_counts || !d_params) return FS_E_INVALID;
    hipLaunchKernelGGL(fs::drng_skip_kernel, dim3((unsigned)((r->n + 63) / 64)), dim3(64), 0, (hipStream_t)stream,
                       r->mt, r->idx, r->n, d_counts, d_params);
    return hipGetLastError() == hipSuccess ? FS_OK : FS_E_HIP;
}

int fs_drng_error(fs_drng* r, void* stream, int32_t* bits) {
    if (!r || !bits) return FS_E_INVALID;
    if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) return FS_E_HIP;
    if (hipMemcpy(bits, r->err, sizeof(int32_t), hipMemcpyDeviceToHost) != hipSuccess) return FS_E_HIP;
    if (hipMemset(r->err, 0, sizeof(int32_t)) != hipSuccess) return FS_E_HIP;
    return FS_OK;
}

#ifdef FS_TRACE
// Trace builds only (not in the product library): phase timestamps of the next sampling grids into d_buf (cap
// entries, TRACE_W per workgroup); a grid larger than the buffer runs untraced.
int fs_trace_set(fs_context* ctx, uint64_t* d_buf, int64_t cap) {
    if (!ctx || cap < 0) return FS_E_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    ctx->trace = d_buf;
    ctx->trace_cap = d_buf ? cap : 0;
    return FS_OK;
}
#endif

const char* fs_strerror(int code) {
    switch (code) {
        case FS_OK: return "ok";
        case FS_E_INVALID: return "invalid argument";
        case FS_E_HIP: return "HIP runtime error";
        case FS_E_NOMEM: return "device allocation failed";
        case FS_E_DEVICE: return "device-side error";
        case FS_E_LIMIT: return "batch exceeds the static workspace of fs_sample_batch_static";
        case FS_W_RECOVERED: return "ok; an earlier call's merge gave up waiting and this call cleared its workspace";
        default: return "unknown error";
    }
}

}  // extern "C"
