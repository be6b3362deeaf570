// sampler_kernels.hip - gfx950 (CDNA4) kernels of the token sampler and the C ABI of include/ferro_sampler.h.
//
// One fused kernel per call. A row of V fp32 logits is split into chunks of BLOCK*EPT elements, one 512-thread
// workgroup per chunk (grid = B * nchunks, rows in order so early rows merge while later rows stream).
// Each chunk workgroup:
//   1. issues all of its 16-byte loads first (EPT/4 per thread, the chunk's only pass over HBM);
//   2. applies the penalty pass on the fly: the row's history window is scattered into an LDS table of 16-bit
//      counts over the chunk's ids and each thread patches the few penalised elements it holds
//      (reference src/sampler.cpp:11-18, plus the frequency/presence extension);
//   3. maps each logit to an order-preserving 32-bit key (-0 folded onto +0); for a top-k row it histograms the
//      maxima of >= 2k disjoint groups of its elements over their [min, max] key range and takes the floor T0 of
//      the bin where the count from the top reaches k - at least k of the chunk's elements reach T0;
//   4. compacts the elements with key >= T0 (a little over k) into LDS with wave ballots and publishes them as
//      64-bit composites (key << 32 | ~id: larger = earlier in ferro's candidate order, sampler.cpp:30); a chunk
//      with too many ties at T0 falls back to an exact radix select over its registers.
// Hand-off without an L2 write-back: the lists are written with agent-scope (sc1, write-through) stores, each wave
// drains its stores (s_waitcnt vmcnt(0)), then one agent-scope counter add per workgroup; the last workgroup of a
// row reads the lists with agent-scope loads and merges: L = max T0 bounds the row's k-th key from below, a
// histogram of the candidates >= L over [L, max] gives a tight T1, the ~k candidates >= T1 are rank-sorted in LDS,
// and the first k feed the double-precision softmax / min-p / top-p / draw (sampler.cpp:37-49), with block scans
// in place of the sequential sums. Greedy rows (temperature <= 0 or top_k == 1, sampler.cpp:19) publish one
// (key, lowest id) maximum per chunk.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <new>
#include <random>

#include "../../include/ferro_sampler.h"

#if !defined(__gfx950__) && defined(__HIP_DEVICE_COMPILE__)
#error "ferro sampler kernels are written for gfx950 only"
#endif

namespace fs {

constexpr int BLOCK = 512;                // threads per workgroup: 8 wave64s, two workgroups per CU
constexpr int WAVE = 64;
constexpr int NWAVES = BLOCK / WAVE;
constexpr int KMAX = 2048;                // largest k on the fused select path
constexpr int KPT = KMAX / BLOCK;         // candidates per thread in the softmax / draw phase
constexpr int CAP = 8192;                 // candidates per chunk in the workspace; merge gather capacity in LDS
constexpr int HBITS = 11;
constexpr int NBINS = 1 << HBITS;         // threshold histograms
constexpr int SMALL = 512;                // rank-sort capacity of the merge
constexpr int MAX_CHUNKS = 1024;
constexpr int SPEC = 4;                   // merge gather: loads in flight per thread per round

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
    int nchunks;
    uint64_t* cand;                // [B*nchunks][CAP]
    uint32_t* meta;                // [B*nchunks][2]: T0, count
    uint32_t* row_cnt;             // [B] chunk completion counters, left at 0
    uint32_t* stream_cnt;          // [n_streams] verify completion counters, left at 0
    int32_t* err;                  // device error bits
};

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

// ------------------------------------------------------------------------------------------------ wave/block
__device__ __forceinline__ int lane_id() { return __lane_id(); }
__device__ __forceinline__ uint32_t mbcnt(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

template <class T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) { const T w = __shfl_xor(v, o); v = w > v ? w : v; }
    return v;
}
template <class T>
__device__ __forceinline__ T wave_min(T v) {
#pragma unroll
    for (int o = WAVE / 2; o > 0; o >>= 1) { const T w = __shfl_xor(v, o); v = w < v ? w : v; }
    return v;
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
// Exclusive prefix over threads (thread order), deterministic; *total = the sum over the block.
template <class T>
__device__ __forceinline__ T block_excl_scan(T v, T* wsum /*NWAVES*/, T* total) {
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    T x = v;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
        const T y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    T ex = __shfl_up(x, 1);
    if (lane == 0) ex = T(0);
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
    base = __shfl(base, leader);
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
    base = __shfl(base, leader);
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
__device__ int hist_locate(const uint32_t* bins, int kk, uint32_t* above_out, uint32_t* atb_out, uint32_t* wsum,
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
__device__ uint32_t hist_threshold(const uint32_t* bins, uint32_t base, int shift, int k, uint32_t* cnt,
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
// calling thread holds.
template <class Each>
__device__ uint64_t radix_kth(Each each, int k, uint32_t* hist256, uint32_t* wsum, Red& r) {
    uint64_t prefix = 0, mask = 0;
    int kk = k;
    const int tid = threadIdx.x;
    for (int shift = 56; shift >= 0; shift -= 8) {
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

// Descending bitonic sort of n (power of two) composites in LDS.
__device__ void bitonic_desc(uint64_t* a, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < n / 2; t += BLOCK) {
                const int i = 2 * t - (t & (stride - 1));
                const int j = i + stride;
                const bool desc = (i & size) == 0;
                const uint64_t x = a[i], y = a[j];
                if ((x < y) == desc) { a[i] = y; a[j] = x; }
            }
            __syncthreads();
        }
    }
}

// Rank sort of n <= SMALL distinct composites: out[rank] = in[i] for ranks < k.
__device__ void rank_sort(const uint64_t* in, int n, uint64_t* out, int k) {
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
template <int EPT>
__global__ __launch_bounds__(BLOCK, 4) void sample_kernel(Args a) {
    constexpr int NV = EPT / 4;                 // float4 loads per thread
    constexpr int CHUNK = BLOCK * EPT;
    static_assert(CHUNK * 2 <= CAP * 8, "the 16-bit count table must fit the candidate storage");
    static_assert(2 * SMALL * 8 <= NBINS * 4, "rank-sort buffers alias the histogram");

    __shared__ __align__(16) uint64_t s_big[CAP];    // counts (chunk phase) / chunk candidates / merge gather
    __shared__ __align__(16) uint32_t s_bins[NBINS]; // histograms; merge: rank-sort input and output
    __shared__ uint32_t s_off[MAX_CHUNKS + 1];       // merge: flat offsets of the chunk lists
    __shared__ uint32_t s_wsum[NWAVES];
    __shared__ uint32_t s_count;
    __shared__ Red red;

    const int tid = threadIdx.x;
    const int row = blockIdx.x / a.nchunks;
    const int chunk = blockIdx.x - row * a.nchunks;
    const int V = a.V;
    const int lo = chunk * CHUNK;
    const float* rowp = a.logits + (int64_t)row * a.ld;

    // ---- 1. stream the chunk: every load is issued before anything waits
    float x[NV][4];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lo + (j * BLOCK + tid) * 4;
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        if (e + 4 <= V) t = *reinterpret_cast<const float4*>(rowp + e);
        else if (e < V) {                            // row tail: never read past element V-1
            t.x = rowp[e];
            if (e + 1 < V) t.y = rowp[e + 1];
            if (e + 2 < V) t.z = rowp[e + 2];
        }
        x[j][0] = t.x; x[j][1] = t.y; x[j][2] = t.z; x[j][3] = t.w;
    }

    // ---- 2. row descriptor: params, history segments (verify rows see base history + earlier drafts)
    int pidx = row;
    int64_t hA0 = 0, lenA = 0, lenB = 0;
    const int32_t* segB = nullptr;
    if (a.mode == MODE_VERIFY) {
        int s0 = 0, s1 = a.n_streams;           // largest s with row_off[s] <= row
        while (s1 - s0 > 1) {
            const int m = (s0 + s1) >> 1;
            if (a.row_off[m] <= row) s0 = m; else s1 = m;
        }
        pidx = s0;
        const int64_t r0 = a.row_off[s0];
        segB = a.rows + r0 + 1;
        lenB = row - r0;
    }
    if (a.hist_off && a.hist) {
        hA0 = a.hist_off[pidx];
        lenA = a.hist_off[pidx + 1] - hA0;
    }
    fs_row_params p;
    if (a.params) p = a.params[pidx];
    else {
        p.temperature = 0.f; p.top_k = 1; p.top_p = 1.f; p.min_p = 0.f; p.repetition_penalty = 1.f;
        p.frequency_penalty = 0.f; p.presence_penalty = 0.f; p.repeat_last_n = 0; p.penalty_from = 0;
        p.reserved = 0;
    }
    const bool greedy = a.mode == MODE_ARGMAX || p.temperature <= 0.0f || p.top_k == 1;
    int k = greedy ? 1 : ((p.top_k > 0 && p.top_k < V) ? p.top_k : V);
    const bool large = k > KMAX;                 // not on the fused select path: reported, token -1

    // ---- 3. penalties (sampler.cpp:11-18; frequency/presence extension)
    const bool rep_on = p.repetition_penalty != 1.0f;
    const bool fp_on = p.frequency_penalty != 0.0f || p.presence_penalty != 0.0f;
    const int64_t len = lenA + lenB;
    const bool pen = !large && (rep_on || fp_on) && p.repeat_last_n != 0 && len > 0;
    if (pen) {
        uint32_t* cnt = reinterpret_cast<uint32_t*>(s_big);   // CHUNK 16-bit counters, two per word
        for (int i = tid; i < CHUNK / 8; i += BLOCK) reinterpret_cast<uint4*>(cnt)[i] = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();
        const int64_t b = window_begin(len, p);
        bool ovf = false;
        for (int64_t i = b + tid; i < len; i += BLOCK) {
            const int id = i < lenA ? a.hist[hA0 + i] : segB[i - lenA];
            const uint32_t rel = (uint32_t)(id - lo);
            if (id >= 0 && id < V && rel < (uint32_t)CHUNK) {
                const uint32_t sh = (rel & 1u) * 16u;
                const uint32_t old = atomicAdd(&cnt[rel >> 1], 1u << sh);
                ovf |= ((old >> sh) & 0xFFFFu) == 0xFFFFu;
            }
        }
        if (ovf) atomicOr(a.err, FS_DEVERR_COUNT_OVERFLOW);
        __syncthreads();
        const float rp = p.repetition_penalty, fq = p.frequency_penalty, pr = p.presence_penalty;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int local = (j * BLOCK + tid) * 4;
            const uint2 c2 = *reinterpret_cast<const uint2*>(&cnt[local >> 1]);
            if ((c2.x | c2.y) != 0u) {
                const uint32_t cc[4] = {c2.x & 0xFFFFu, c2.x >> 16, c2.y & 0xFFFFu, c2.y >> 16};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (cc[q] != 0u) {
                        float l = x[j][q];
                        if (rep_on) l = l > 0.0f ? __fdiv_rn(l, rp) : __fmul_rn(l, rp);
                        if (fp_on) l = __fsub_rn(l, __fadd_rn(__fmul_rn((float)cc[q], fq), pr));
                        x[j][q] = l;
                    }
                }
            }
        }
        __syncthreads();                                     // the count table's storage is reused below
    }

    // ---- 4. keys (0 marks an element past V)
    uint32_t key[NV][4];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = lo + (j * BLOCK + tid) * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) key[j][q] = e + q < V ? key_of(x[j][q]) : 0u;
    }
    auto comp_at = [&](int j, int q) -> uint64_t {
        const int e = lo + (j * BLOCK + tid) * 4 + q;
        return e < V ? comp_of(key[j][q], (uint32_t)e) : 0ull;
    };

    // ---- 5. chunk selection, published with agent-scope stores
    const int slot = row * a.nchunks + chunk;
    uint64_t* gout = a.cand + (int64_t)slot * CAP;
    if (large) {
        if (tid == 0) { st_agent(&a.meta[2 * slot], 0u); st_agent(&a.meta[2 * slot + 1], 0u); }
    } else if (greedy) {
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) { const uint64_t c = comp_at(j, q); best = c > best ? c : best; }
        best = block_max_u64(best, red);
        if (tid == 0) {
            st_agent(gout, best);
            st_agent(&a.meta[2 * slot], comp_key(best));
            st_agent(&a.meta[2 * slot + 1], 1u);
        }
    } else {
        const int nvalid = min(CHUNK, V - lo);
        uint32_t T0 = 0;
        if (k < nvalid) {
            // maxima of G groups per thread, BLOCK*G >= 2k groups in all (G <= EPT)
            int G = 1;
            while (G * BLOCK < 2 * k && G < EPT) G <<= 1;
            const int per = EPT / G;                 // elements per group, in thread-local order j*4+q
            uint32_t gmin = 0xFFFFFFFFu, gmax = 0u;
            {
                uint32_t gm = 0;
                bool any = false;
#pragma unroll
                for (int j = 0; j < NV; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (lo + (j * BLOCK + tid) * 4 + q < V) { gm = key[j][q] > gm ? key[j][q] : gm; any = true; }
                        if ((j * 4 + q + 1) % per == 0) {
                            if (any) { gmin = gm < gmin ? gm : gmin; gmax = gm > gmax ? gm : gmax; }
                            gm = 0;
                            any = false;
                        }
                    }
            }
            for (int i = tid; i < NBINS; i += BLOCK) s_bins[i] = 0u;
            block_minmax_u32(gmin, gmax, red);
            const int sh = range_shift(gmin, gmax);
            {
                uint32_t gm = 0;
                bool any = false;
#pragma unroll
                for (int j = 0; j < NV; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (lo + (j * BLOCK + tid) * 4 + q < V) { gm = key[j][q] > gm ? key[j][q] : gm; any = true; }
                        if ((j * 4 + q + 1) % per == 0) {
                            if (any) atomicAdd(&s_bins[(gm - gmin) >> sh], 1u);
                            gm = 0;
                            any = false;
                        }
                    }
            }
            __syncthreads();
            uint32_t c0;
            T0 = hist_threshold(s_bins, gmin, sh, k, &c0, s_wsum, red);   // 0: groups could not certify k
        }
        // compaction of keys >= T0
        if (tid == 0) s_count = 0u;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e = lo + (j * BLOCK + tid) * 4 + q;
                wave_append_kv(e < V && key[j][q] >= T0, key[j][q], (uint32_t)e, s_big, &s_count, CAP);
            }
        __syncthreads();
        uint32_t n = s_count;
        if (n > (uint32_t)CAP) {
            // Too many keys >= T0 (a flat distribution or ties): narrow [rlo, rhi] onto the exact k-th key with
            // histogram levels over the registers (2048x per level, 4 levels reach a single key value).
            // Invariant: count(key > rhi) == above < k <= count(key >= rlo).
            uint32_t rlo = T0, rhi = 0u, above = 0u, cnt_ge = n;
#pragma unroll
            for (int j = 0; j < NV; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) rhi = key[j][q] > rhi ? key[j][q] : rhi;   // invalid keys are 0
            {
                uint32_t dummy = 0u;
                block_minmax_u32(dummy, rhi, red);
            }
            for (int level = 0; level < 4 && cnt_ge > (uint32_t)CAP && rlo != rhi; ++level) {
                const int sh = range_shift(rlo, rhi);
                for (int i = tid; i < NBINS; i += BLOCK) s_bins[i] = 0u;
                __syncthreads();
#pragma unroll
                for (int j = 0; j < NV; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t kq = key[j][q];
                        if (lo + (j * BLOCK + tid) * 4 + q < V && kq >= rlo && kq <= rhi)
                            atomicAdd(&s_bins[(kq - rlo) >> sh], 1u);
                    }
                __syncthreads();
                uint32_t ab, atb;
                const int bsel = hist_locate(s_bins, k - (int)above, &ab, &atb, s_wsum, red);
                const uint64_t nlo = (uint64_t)rlo + ((uint64_t)bsel << sh);
                const uint64_t nhi = (uint64_t)rlo + (((uint64_t)bsel + 1) << sh) - 1;
                rlo = (uint32_t)nlo;
                rhi = nhi < rhi ? (uint32_t)nhi : rhi;
                above += ab;
                cnt_ge = above + atb;
            }
            if (tid == 0) s_count = 0u;
            __syncthreads();
            if (cnt_ge <= (uint32_t)CAP) {
#pragma unroll
                for (int j = 0; j < NV; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int e = lo + (j * BLOCK + tid) * 4 + q;
                        wave_append_kv(e < V && key[j][q] >= rlo, key[j][q], (uint32_t)e, s_big, &s_count, CAP);
                    }
            } else {
                // rlo == rhi is the k-th key t and it is tied: keep every key > t and the (k - above) lowest ids
                // with key == t; ids run in (j, thread, q) order, so one block scan per j ranks the ties
                const uint32_t t = rlo;
                const uint32_t need = (uint32_t)k - above;
                uint32_t run = 0u;
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    uint32_t mine = 0u;
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        mine += (lo + (j * BLOCK + tid) * 4 + q < V && key[j][q] == t) ? 1u : 0u;
                    uint32_t tot;
                    uint32_t pos = run + block_excl_scan<uint32_t>(mine, s_wsum, &tot);
                    run += tot;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int e = lo + (j * BLOCK + tid) * 4 + q;
                        const bool valid = e < V;
                        const bool tie = valid && key[j][q] == t;
                        const bool take = (valid && key[j][q] > t) || (tie && pos < need);
                        pos += tie ? 1u : 0u;
                        wave_append_kv(take, key[j][q], (uint32_t)e, s_big, &s_count, CAP);
                    }
                }
            }
            __syncthreads();
            n = s_count;
            T0 = rlo;
        }
        for (uint32_t i = tid; i < n; i += BLOCK) st_agent(gout + i, s_big[i]);
        if (tid == 0) {
            st_agent(&a.meta[2 * slot], T0);
            st_agent(&a.meta[2 * slot + 1], n);
        }
    }

    // ---- 6. hand-off: drain this wave's stores, then one agent-scope count per chunk; the last one merges
    vm_drain();
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&a.row_cnt[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        red.misc[3] = (old == (uint32_t)a.nchunks - 1u) ? 1u : 0u;
    }
    __syncthreads();
    if (red.misc[3] == 0u) return;
    if (tid == 0) st_agent(&a.row_cnt[row], 0u);

    // ---- 7. merge
    const int nch = a.nchunks;
    const int slot0 = row * nch;
    int tok = 0, keep = 1;
    if (large) {
        tok = -1;
        keep = 0;
        if (tid == 0) atomicOr(a.err, FS_DEVERR_LARGE_K);
    } else if (greedy) {
        uint64_t best = 0;
        for (int c = tid; c < nch; c += BLOCK) {
            const uint64_t v = ld_agent(a.cand + (int64_t)(slot0 + c) * CAP);
            best = v > best ? v : best;
        }
        best = block_max_u64(best, red);
        tok = (int)comp_id(best);
        const float l0 = rowp[0];
        if (l0 != l0) tok = 0;                         // ferro's scan never moves off a NaN at index 0
        if (tid == 0 && a.mode != MODE_VERIFY) {
            if (a.cand_ids && a.kcap > 0) a.cand_ids[(int64_t)row * a.kcap] = tok;
            if (a.cand_probs && a.kcap > 0) a.cand_probs[(int64_t)row * a.kcap] = 1.0;
        }
    } else {
        // metas: L = max T0 (a lower bound of the row's k-th key), flat offsets of the chunk lists
        uint32_t Lloc = 0, nmine = 0;
        for (int c = 2 * tid; c < 2 * tid + 2 && c < nch; ++c) {
            const uint32_t t0 = ld_agent(&a.meta[2 * (slot0 + c)]);
            const uint32_t cn = ld_agent(&a.meta[2 * (slot0 + c) + 1]);
            Lloc = t0 > Lloc ? t0 : Lloc;
            s_off[c] = cn;
            nmine += cn;
        }
        const uint32_t L = (uint32_t)block_max_u64(Lloc, red);
        uint32_t total;
        uint32_t o = block_excl_scan<uint32_t>(nmine, s_wsum, &total);
        for (int c = 2 * tid; c < 2 * tid + 2 && c < nch; ++c) { const uint32_t cn = s_off[c]; s_off[c] = o; o += cn; }
        if (tid == 0) { s_off[nch] = total; s_count = 0u; }
        __syncthreads();
        auto fetch = [&](uint32_t f) -> uint64_t {          // flat index -> candidate (0 past the end)
            if (f >= total) return 0ull;
            int c0 = 0, c1 = nch;                            // largest c with s_off[c] <= f
            while (c1 - c0 > 1) {
                const int m = (c0 + c1) >> 1;
                if (s_off[m] <= f) c0 = m; else c1 = m;
            }
            return ld_agent(a.cand + (int64_t)(slot0 + c0) * CAP + (f - s_off[c0]));
        };
        // gather the candidates >= L into LDS (counted past CAP), tracking their max key
        uint32_t kmax = L;
        for (uint32_t f0 = 0; f0 < total; f0 += BLOCK * SPEC) {
            uint64_t v[SPEC];
#pragma unroll
            for (int q = 0; q < SPEC; ++q) v[q] = fetch(f0 + q * BLOCK + tid);
#pragma unroll
            for (int q = 0; q < SPEC; ++q) {
                const bool in = v[q] != 0 && comp_key(v[q]) >= L;
                if (in) kmax = comp_key(v[q]) > kmax ? comp_key(v[q]) : kmax;
                wave_append(in, v[q], s_big, &s_count, CAP);
            }
        }
        for (int i = tid; i < NBINS; i += BLOCK) s_bins[i] = 0u;
        uint32_t kmin = L;
        block_minmax_u32(kmin, kmax, red);
        const uint32_t n = s_count;
        const bool in_lds = n <= (uint32_t)CAP;
        // T1: tight threshold from a histogram of the candidates' keys over [L, kmax]
        const int sh = range_shift(L, kmax);
        if (in_lds) {
            for (uint32_t i = tid; i < n; i += BLOCK) atomicAdd(&s_bins[(comp_key(s_big[i]) - L) >> sh], 1u);
        } else {
            for (uint32_t f = tid; f < total; f += BLOCK) {
                const uint64_t c = fetch(f);
                if (c != 0 && comp_key(c) >= L) atomicAdd(&s_bins[(comp_key(c) - L) >> sh], 1u);
            }
        }
        __syncthreads();
        uint32_t c1;
        const uint32_t T1 = hist_threshold(s_bins, L, sh, k, &c1, s_wsum, red);
        // the c1 >= k candidates with key >= T1 contain the top k: sort them
        uint64_t* top;
        uint64_t* small_in = reinterpret_cast<uint64_t*>(s_bins);
        uint64_t* small_out = small_in + SMALL;
        if (tid == 0) s_count = 0u;
        __syncthreads();
        if (c1 <= (uint32_t)SMALL) {
            if (in_lds) {
                for (uint32_t i0 = 0; i0 < n; i0 += BLOCK) {
                    const uint32_t i = i0 + tid;
                    const uint64_t c = i < n ? s_big[i] : 0ull;
                    wave_append(c != 0 && comp_key(c) >= T1, c, small_in, &s_count, SMALL);
                }
            } else {
                for (uint32_t f0 = 0; f0 < total; f0 += BLOCK) {
                    const uint64_t c = fetch(f0 + tid);
                    wave_append(c != 0 && comp_key(c) >= T1, c, small_in, &s_count, SMALL);
                }
            }
            __syncthreads();
            rank_sort(small_in, (int)c1, small_out, k);
            top = small_out;
        } else if (in_lds) {
            int np = 1;
            while (np < (int)n) np <<= 1;
            for (int i = (int)n + tid; i < np; i += BLOCK) s_big[i] = 0ull;
            __syncthreads();
            bitonic_desc(s_big, np);
            top = s_big;
        } else {
            uint64_t X = 0;                             // threshold for an exact gather of <= CAP entries
            if (c1 > (uint32_t)CAP) {
                X = radix_kth(
                    [&](auto&& f) {
                        for (uint32_t f0 = tid; f0 < total; f0 += BLOCK) {
                            const uint64_t c = fetch(f0);
                            f(c != 0 && comp_key(c) >= L ? c : 0ull);
                        }
                    },
                    k, s_bins, s_wsum, red);
            }
            if (tid == 0) s_count = 0u;
            __syncthreads();
            for (uint32_t f0 = 0; f0 < total; f0 += BLOCK) {
                const uint64_t c = fetch(f0 + tid);
                wave_append(c != 0 && comp_key(c) >= T1 && c >= X, c, s_big, &s_count, CAP);
            }
            __syncthreads();
            const int m = (int)s_count;
            int np = 1;
            while (np < m) np <<= 1;
            for (int i = m + tid; i < np; i += BLOCK) s_big[i] = 0ull;
            __syncthreads();
            bitonic_desc(s_big, np);
            top = s_big;
        }
        if (c1 < (uint32_t)k) {                       // impossible by construction; never read past the list
            if (tid == 0) atomicOr(a.err, FS_DEVERR_INTERNAL);
            k = (int)c1;
        }

        // ---- softmax at temperature, min-p, top-p, draw (sampler.cpp:37-49), k <= KMAX
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
        const double sum = block_sum_f64(part, red);
        double pr[KPT];
#pragma unroll
        for (int q = 0; q < KPT; ++q) pr[q] = e[q] / sum;
        // min-p: keep = 1 + the last index with pr >= pr[0]*min_p (at least 1)
        int keep_m = k;
        if (p.min_p > 0.0f) {
            const double thr = (1.0 / sum) * (double)p.min_p;
            int last = -1;
#pragma unroll
            for (int q = 0; q < KPT; ++q)
                if (i0 + q < k && pr[q] >= thr) last = i0 + q;
            last = block_max_i32(last, red);
            keep_m = last + 1 > 1 ? last + 1 : 1;
        }
        // inclusive prefix of pr in candidate order
        double c[KPT];
        double run = 0.0;
#pragma unroll
        for (int q = 0; q < KPT; ++q) { run += pr[q]; c[q] = run; }
        double tot_all;
        const double off = block_excl_scan<double>(run, red.f64, &tot_all);
#pragma unroll
        for (int q = 0; q < KPT; ++q) c[q] += off;
        keep = keep_m;
        if (p.top_p < 1.0f) {
            int first = 0x7fffffff;
#pragma unroll
            for (int q = 0; q < KPT; ++q)
                if (i0 + q < keep_m && c[q] >= (double)p.top_p && first == 0x7fffffff) first = i0 + q;
            first = block_min_i32(first, red);
            if (first != 0x7fffffff) keep = first + 1 < keep_m ? first + 1 : keep_m;
            if (keep < 1) keep = 1;
        }
        // tot = sum of the kept prefix; r = u * tot; the first i with r <= c_i
#pragma unroll
        for (int q = 0; q < KPT; ++q)
            if (i0 + q == keep - 1) red.dmisc[0] = c[q];
        __syncthreads();
        const double tot = red.dmisc[0];
        const double u = a.u ? a.u[row] : 0.0;
        const double rr = u * tot + 0.0;
        int hit = 0x7fffffff;
#pragma unroll
        for (int q = 0; q < KPT; ++q)
            if (i0 + q < keep && rr <= c[q] && hit == 0x7fffffff) hit = i0 + q;
        hit = block_min_i32(hit, red);
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
    }
    if (a.mode != MODE_VERIFY) {
        if (tid == 0) {
            a.tok[row] = tok;
            if (a.keep) a.keep[row] = keep;
        }
        return;
    }

    // ---- verify: the last row of a stream to finish computes the accepted prefix (server.cpp:627-637)
    if (tid == 0) {
        st_agent(&a.tok[row], (int32_t)tok);
        vm_drain();
        const int s = pidx;
        const int64_t r0 = a.row_off[s];
        const int m = (int)(a.row_off[s + 1] - r0);
        const uint32_t old = __hip_atomic_fetch_add(&a.stream_cnt[s], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == (uint32_t)m - 1u) {
            st_agent(&a.stream_cnt[s], 0u);
            int acc = 0;
            for (int r = 0; r < m; ++r) {
                const int t = ld_agent(&a.tok[r0 + r]);
                acc = r + 1;
                if (a.eos >= 0 && t == a.eos) break;
                if (r + 1 < m && t == a.rows[r0 + r + 1]) continue;
                break;
            }
            a.accepted[s] = acc;
        }
    }
}

}  // namespace fs

// ================================================================================================ host side
struct fs_context {
    std::mutex mu;
    int device = -1;
    uint64_t* cand = nullptr;
    size_t cand_slots = 0;     // chunk slots of CAP entries
    uint32_t* meta = nullptr;
    uint32_t* row_cnt = nullptr;
    size_t row_cap = 0;
    uint32_t* stream_cnt = nullptr;
    size_t stream_cap = 0;
    int32_t* err = nullptr;
};

namespace {

int grow(fs_context* c, size_t slots, size_t rows, size_t streams) {
    if (slots > c->cand_slots) {
        if (c->cand) (void)hipFree(c->cand);
        if (c->meta) (void)hipFree(c->meta);
        c->cand = nullptr; c->meta = nullptr; c->cand_slots = 0;
        if (hipMalloc(&c->cand, slots * fs::CAP * sizeof(uint64_t)) != hipSuccess) return FS_E_NOMEM;
        if (hipMalloc(&c->meta, slots * 2 * sizeof(uint32_t)) != hipSuccess) return FS_E_NOMEM;
        c->cand_slots = slots;
    }
    if (rows > c->row_cap) {
        if (c->row_cnt) (void)hipFree(c->row_cnt);
        c->row_cnt = nullptr; c->row_cap = 0;
        if (hipMalloc(&c->row_cnt, rows * sizeof(uint32_t)) != hipSuccess) return FS_E_NOMEM;
        if (hipMemset(c->row_cnt, 0, rows * sizeof(uint32_t)) != hipSuccess) return FS_E_HIP;
        c->row_cap = rows;
    }
    if (streams > c->stream_cap) {
        if (c->stream_cnt) (void)hipFree(c->stream_cnt);
        c->stream_cnt = nullptr; c->stream_cap = 0;
        if (hipMalloc(&c->stream_cnt, streams * sizeof(uint32_t)) != hipSuccess) return FS_E_NOMEM;
        if (hipMemset(c->stream_cnt, 0, streams * sizeof(uint32_t)) != hipSuccess) return FS_E_HIP;
        c->stream_cap = streams;
    }
    if (!c->err) {
        if (hipMalloc(&c->err, sizeof(int32_t)) != hipSuccess) return FS_E_NOMEM;
        if (hipMemset(c->err, 0, sizeof(int32_t)) != hipSuccess) return FS_E_HIP;
    }
    return FS_OK;
}

// Chunk size: the largest of 16384 / 8192 / 2048 elements per workgroup that still puts >= 256 workgroups on the
// chip (one per CU); fewer, longer chunks mean fewer candidates to merge per row.
int choose_ept(int64_t rows, int V) {
    for (int ept : {32, 16}) {
        const int64_t nch = (V + fs::BLOCK * ept - 1) / (fs::BLOCK * ept);
        if (rows * nch >= 256) return ept;
    }
    return 4;
}

int launch(fs_context* ctx, fs::Args a, int64_t rows, int64_t streams, hipStream_t st) {
    int ept = choose_ept(rows, a.V);
    while (ept < 32 && (a.V + fs::BLOCK * ept - 1) / (fs::BLOCK * ept) > fs::MAX_CHUNKS) ept *= 4;
    const int chunk = fs::BLOCK * ept;
    a.nchunks = (a.V + chunk - 1) / chunk;
    if (a.nchunks > fs::MAX_CHUNKS) return FS_E_INVALID;
    const int64_t grid = rows * a.nchunks;
    if (grid > 0x7fffffff) return FS_E_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (ctx->device < 0) { if (hipGetDevice(&ctx->device) != hipSuccess) return FS_E_HIP; }
    int rc = grow(ctx, (size_t)grid, (size_t)rows, (size_t)(streams > 0 ? streams : 1));
    if (rc != FS_OK) return rc;
    a.cand = ctx->cand; a.meta = ctx->meta; a.row_cnt = ctx->row_cnt; a.stream_cnt = ctx->stream_cnt; a.err = ctx->err;
    if (ept == 32) hipLaunchKernelGGL(fs::sample_kernel<32>, dim3((unsigned)grid), dim3(fs::BLOCK), 0, st, a);
    else if (ept == 16) hipLaunchKernelGGL(fs::sample_kernel<16>, dim3((unsigned)grid), dim3(fs::BLOCK), 0, st, a);
    else hipLaunchKernelGGL(fs::sample_kernel<4>, dim3((unsigned)grid), dim3(fs::BLOCK), 0, st, a);
    return hipGetLastError() == hipSuccess ? FS_OK : FS_E_HIP;
}

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
    (void)hipFree(c->cand);
    (void)hipFree(c->meta);
    (void)hipFree(c->row_cnt);
    (void)hipFree(c->stream_cnt);
    (void)hipFree(c->err);
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

int fs_argmax_batch(fs_context* ctx, const float* d_logits, int64_t ld, int32_t B, int32_t V, const int32_t* d_hist,
                    const int64_t* d_hist_off, const fs_row_params* d_params, int32_t* d_tok, void* stream) {
    if (!ctx || !d_tok) return FS_E_INVALID;
    int rc = check_rows(d_logits, ld, B, V);
    if (rc != FS_OK) return rc;
    if (B == 0) return FS_OK;
    fs::Args a = {};
    a.logits = d_logits; a.ld = ld; a.B = B; a.V = V; a.hist = d_hist; a.hist_off = d_params ? d_hist_off : nullptr;
    a.params = d_params; a.tok = d_tok; a.mode = fs::MODE_ARGMAX; a.eos = -1;
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

int fs_device_error(fs_context* ctx, void* stream, int32_t* bits) {
    if (!ctx || !bits) return FS_E_INVALID;
    *bits = 0;
    if (!ctx->err) return FS_OK;
    if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) return FS_E_HIP;
    if (hipMemcpy(bits, ctx->err, sizeof(int32_t), hipMemcpyDeviceToHost) != hipSuccess) return FS_E_HIP;
    if (hipMemset(ctx->err, 0, sizeof(int32_t)) != hipSuccess) return FS_E_HIP;
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

const char* fs_strerror(int code) {
    switch (code) {
        case FS_OK: return "ok";
        case FS_E_INVALID: return "invalid argument";
        case FS_E_HIP: return "HIP runtime error";
        case FS_E_NOMEM: return "device allocation failed";
        case FS_E_DEVICE: return "device-side error";
        default: return "unknown error";
    }
}

}  // extern "C"
