/* sampler_oracle.c - CPU restatement of ferro::Sampler::sample. TEST INFRASTRUCTURE ONLY: the parity checker for
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg. The product library never links or calls it.
 *
 * Pinned by: the reference known-answer test (tests/test_kernels.cpp:348-358, five penalty window/scope cases),
 * golden vectors written by the compiled reference (tests/golden/), brute-force full sorts on tiny rows, and the
 * closed forms of the softmax / top-p / draw steps (tests/test_oracle.py).
 *
 * Built with the reference's own flags (-O3 -std=c11 -fno-math-errno, no -ffast-math, no FMA contraction) so the
 * float/double arithmetic below rounds exactly as sampler.cpp does on x86-64.
 */
#include "sampler_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ penalty: sampler.cpp:11-18 */
static int cmp_i32(const void* a, const void* b) {
    const int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

/* Window start b: sampler.cpp:13-14. */
static int64_t window_begin(int64_t hlen, const fso_params* p) {
    int64_t b = (p->repeat_last_n > 0 && (int64_t)p->repeat_last_n < hlen) ? hlen - (int64_t)p->repeat_last_n : 0;
    if (p->penalty_from > 0 && (int64_t)p->penalty_from > b) b = p->penalty_from;
    return b;
}

int fso_penalize(float* row, int n, const int32_t* hist, int64_t hlen, const fso_params* p) {
    const int rep_on = p->repetition_penalty != 1.0f;
    const int fp_on = p->frequency_penalty != 0.0f || p->presence_penalty != 0.0f;
    if (!(rep_on || fp_on) || p->repeat_last_n == 0 || hlen <= 0) return 0;   /* sampler.cpp:11 */
    const int64_t b = window_begin(hlen, p);
    if (b >= hlen) return 0;
    const int64_t w = hlen - b;
    int32_t* ids = (int32_t*)malloc((size_t)w * sizeof(int32_t));
    memcpy(ids, hist + b, (size_t)w * sizeof(int32_t));
    qsort(ids, (size_t)w, sizeof(int32_t), cmp_i32);            /* distinct ids with their counts */
    int changed = 0;
    for (int64_t i = 0; i < w;) {
        int64_t j = i;
        while (j < w && ids[j] == ids[i]) ++j;
        const int32_t id = ids[i];
        const int32_t cnt = (int32_t)(j - i);
        if (id >= 0 && id < n) {                                 /* sampler.cpp:16 */
            float l = row[id];
            if (rep_on) l = l > 0 ? l / p->repetition_penalty : l * p->repetition_penalty;   /* sampler.cpp:17 */
            if (fp_on) {                                         /* extension, llama.cpp convention */
                const float t = (float)cnt * p->frequency_penalty;
                const float s = t + p->presence_penalty;        /* cnt > 0 here */
                l = l - s;
            }
            row[id] = l;
            ++changed;
        }
        i = j;
    }
    free(ids);
    return changed;
}

/* ------------------------------------------------------------------ candidate order: sampler.cpp:30 */
typedef struct { float v; int32_t id; } cand_t;

/* a precedes b: larger logit first, equal logits (-0 == +0) by lower id. NaN: ferro's comparator (sampler.cpp:30)
 * is not a strict weak order with a NaN in the row, so std::partial_sort's result is unspecified there; this build
 * ranks NaN below every number (NaNs by lower id) and never makes it a candidate (see fso_sample). Rows without a
 * NaN are unaffected. */
static int better(const cand_t* a, const cand_t* b) {
    const int an = a->v != a->v, bn = b->v != b->v;
    if (an || bn) return an && bn ? a->id < b->id : bn;
    return a->v > b->v || (a->v == b->v && a->id < b->id);
}
static int cmp_cand(const void* pa, const void* pb) {
    const cand_t* a = (const cand_t*)pa;
    const cand_t* b = (const cand_t*)pb;
    return better(a, b) ? -1 : (better(b, a) ? 1 : 0);
}

/* Heap whose root is the worst kept candidate. */
static void sift_down(cand_t* h, int k, int i) {
    for (;;) {
        int l = 2 * i + 1, r = l + 1, w = i;
        if (l < k && better(&h[w], &h[l])) w = l;
        if (r < k && better(&h[w], &h[r])) w = r;
        if (w == i) return;
        cand_t t = h[i]; h[i] = h[w]; h[w] = t;
        i = w;
    }
}

/* First k of the row under the total order (the set and order std::partial_sort / std::sort produce:
 * sampler.cpp:25-35). Returns a malloc'd sorted array of k candidates. */
static cand_t* top_k_sorted(const float* row, int n, int k) {
    cand_t* c = (cand_t*)malloc((size_t)k * sizeof(cand_t));
    for (int i = 0; i < k; ++i) { c[i].v = row[i]; c[i].id = i; }
    if (k < n) {
        for (int i = k / 2 - 1; i >= 0; --i) sift_down(c, k, i);
        for (int i = k; i < n; ++i) {
            cand_t x = { row[i], i };
            if (better(&x, &c[0])) { c[0] = x; sift_down(c, k, 0); }
        }
    }
    qsort(c, (size_t)k, sizeof(cand_t), cmp_cand);
    return c;
}

/* ------------------------------------------------------------------ sample: sampler.cpp:10-50 */
int fso_sample(float* row, int n, const int32_t* hist, int64_t hlen, const fso_params* p, double u,
               int32_t* cand_ids, double* cand_probs, int kcap, int32_t* keep_out, int32_t* ncand_out) {
    if (p->softcap > 0.0f)                                     /* the model's final-logit softcap, applied to the */
        for (int i = 0; i < n; ++i)                            /* row before sample() (model_gemma4_gpu.cpp:282-283) */
            row[i] = p->softcap * tanhf(row[i] / p->softcap);
    fso_penalize(row, n, hist, hlen, p);
    if (p->temperature <= 0.0f || p->top_k == 1) {            /* greedy: sampler.cpp:19-23 */
        int best = 0;
        for (int i = 1; i < n; ++i) if (row[i] > row[best]) best = i;
        if (cand_ids && kcap > 0) cand_ids[0] = best;
        if (cand_probs && kcap > 0) cand_probs[0] = 1.0;
        if (keep_out) *keep_out = 1;
        if (ncand_out) *ncand_out = 1;
        return best;
    }
    int k = (p->top_k > 0 && p->top_k < n) ? p->top_k : n;   /* sampler.cpp:26 */
    int nnum = 0;                                              /* NaN policy: candidates are numbers only */
    for (int i = 0; i < n; ++i) nnum += row[i] == row[i];
    if (nnum == 0) {                                           /* every logit NaN: token 0, nothing kept */
        if (keep_out) *keep_out = 0;
        if (ncand_out) *ncand_out = 0;
        return 0;
    }
    if (k > nnum) k = nnum;
    cand_t* c = top_k_sorted(row, n, k);
    /* softmax at temperature: the difference is a float op, then double divide and exp (sampler.cpp:37-41) */
    const float mx = c[0].v;
    double sum = 0;
    double* pr = (double*)malloc((size_t)k * sizeof(double));
    for (int i = 0; i < k; ++i) {
        const float d = c[i].v - mx;
        pr[i] = exp((double)d / (double)p->temperature);
        sum += pr[i];
    }
    for (int i = 0; i < k; ++i) pr[i] /= sum;
    int keep = k;
    if (p->min_p > 0.0f) {                                     /* sampler.cpp:43 */
        const double thr = pr[0] * (double)p->min_p;
        while (keep > 1 && pr[keep - 1] < thr) --keep;
    }
    if (p->top_p < 1.0f) {                                     /* sampler.cpp:44 */
        double cs = 0;
        int i = 0;
        for (; i < keep; ++i) { cs += pr[i]; if (cs >= (double)p->top_p) { ++i; break; } }
        keep = keep < i ? keep : i;
        if (keep < 1) keep = 1;
    }
    double tot = 0;                                            /* sampler.cpp:45-49 */
    for (int i = 0; i < keep; ++i) tot += pr[i];
    const double r = u * tot + 0.0;
    int tok = c[keep - 1].id;
    double cs = 0;
    for (int i = 0; i < keep; ++i) { cs += pr[i]; if (r <= cs) { tok = c[i].id; break; } }
    const int m = k < kcap ? k : kcap;
    if (cand_ids) for (int i = 0; i < m; ++i) cand_ids[i] = c[i].id;
    if (cand_probs) for (int i = 0; i < m; ++i) cand_probs[i] = pr[i];
    if (keep_out) *keep_out = keep;
    if (ncand_out) *ncand_out = k;
    free(pr);
    free(c);
    return tok;
}

/* ------------------------------------------------------------------ batch (CPU baseline over host threads) */
typedef struct {
    float* logits; int64_t ld; int B, n; const int32_t* hist; const int64_t* hist_off; const fso_params* params;
    const double* u; int32_t* tok; int32_t* cand_ids; double* cand_probs; int kcap; int32_t* keep; int32_t* ncand;
    int t, nt;
} batch_job;

static void* batch_worker(void* arg) {
    const batch_job* j = (const batch_job*)arg;
    for (int b = j->t; b < j->B; b += j->nt) {
        const int64_t h0 = j->hist_off ? j->hist_off[b] : 0, h1 = j->hist_off ? j->hist_off[b + 1] : 0;
        j->tok[b] = fso_sample(j->logits + (int64_t)b * j->ld, j->n, j->hist + h0, h1 - h0, &j->params[b],
                               j->u ? j->u[b] : 0.0,
                               j->cand_ids ? j->cand_ids + (int64_t)b * j->kcap : 0,
                               j->cand_probs ? j->cand_probs + (int64_t)b * j->kcap : 0, j->kcap,
                               j->keep ? j->keep + b : 0, j->ncand ? j->ncand + b : 0);
    }
    return 0;
}

void fso_sample_batch(float* logits, int64_t ld, int B, int n, const int32_t* hist, const int64_t* hist_off,
                      const fso_params* params, const double* u, int32_t* tok, int32_t* cand_ids,
                      double* cand_probs, int kcap, int32_t* keep, int32_t* ncand, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > B) nthreads = B > 0 ? B : 1;
    batch_job* jobs = (batch_job*)malloc((size_t)nthreads * sizeof(batch_job));
    pthread_t* th = (pthread_t*)malloc((size_t)nthreads * sizeof(pthread_t));
    for (int t = 0; t < nthreads; ++t) {
        batch_job j = { logits, ld, B, n, hist, hist_off, params, u, tok, cand_ids, cand_probs, kcap, keep, ncand,
                        t, nthreads };
        jobs[t] = j;
    }
    if (nthreads == 1) batch_worker(&jobs[0]);
    else {
        for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], 0, batch_worker, &jobs[t]);
        for (int t = 0; t < nthreads; ++t) pthread_join(th[t], 0);
    }
    free(th);
    free(jobs);
}

/* ------------------------------------------------------------------ verification: server.cpp:627-637 */
void fso_verify(float* logits, int64_t ld, int n_streams, int n, const int32_t* rows, const int64_t* row_off,
                const int32_t* hist, const int64_t* hist_off, const fso_params* params, const double* u,
                int32_t eos_id, int32_t* tok, int32_t* accepted) {
    for (int s = 0; s < n_streams; ++s) {
        const int64_t r0 = row_off[s], m = row_off[s + 1] - row_off[s];
        const int64_t h0 = hist_off[s], hb = hist_off[s + 1] - hist_off[s];
        int32_t* h = (int32_t*)malloc((size_t)(hb + (m > 0 ? m : 1)) * sizeof(int32_t));
        memcpy(h, hist + h0, (size_t)hb * sizeof(int32_t));
        for (int64_t r = 0; r < m; ++r) {
            /* row r sees the base history plus the drafts fed before it: rows[1..r] */
            for (int64_t q = 1; q <= r; ++q) h[hb + q - 1] = rows[r0 + q];
            tok[r0 + r] = fso_sample(logits + (r0 + r) * ld, n, h, hb + r, &params[s], u ? u[r0 + r] : 0.0,
                                     0, 0, 0, 0, 0);
        }
        int acc = 0;
        for (int64_t r = 0; r < m; ++r) {
            acc = (int)r + 1;
            if (eos_id >= 0 && tok[r0 + r] == eos_id) break;
            if (r + 1 < m && tok[r0 + r] == rows[r0 + r + 1]) continue;
            break;
        }
        accepted[s] = acc;
        free(h);
    }
}

/* ------------------------------------------------------------------ mt19937_64 + generate_canonical */
void fso_mt64_seed(fso_mt64* s, uint64_t seed) {
    s->mt[0] = seed;
    for (int i = 1; i < 312; ++i)
        s->mt[i] = 6364136223846793005ULL * (s->mt[i - 1] ^ (s->mt[i - 1] >> 62)) + (uint64_t)i;
    s->mti = 312;
}

uint64_t fso_mt64_next(fso_mt64* s) {
    static const uint64_t UM = 0xFFFFFFFF80000000ULL, LM = 0x7FFFFFFFULL, A = 0xB5026F5AA96619E9ULL;
    if (s->mti >= 312) {
        int i;
        for (i = 0; i < 312; ++i) {
            const uint64_t x = (s->mt[i] & UM) | (s->mt[(i + 1) % 312] & LM);
            s->mt[i] = s->mt[(i + 156) % 312] ^ (x >> 1) ^ ((x & 1ULL) ? A : 0ULL);
        }
        s->mti = 0;
    }
    uint64_t x = s->mt[s->mti++];
    x ^= (x >> 29) & 0x5555555555555555ULL;
    x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
    x ^= (x << 37) & 0xFFF7EEE000000000ULL;
    x ^= x >> 43;
    return x;
}

/* One 64-bit draw / 2^64, clamped below 1 (what generate_canonical<double,53> does with a 64-bit engine). */
double fso_canonical(uint64_t x) {
    double r = (double)x / 18446744073709551616.0;
    if (r >= 1.0) r = nextafter(1.0, 0.0);
    return r;
}

/* ------------------------------------------------------------------ prompt-lookup drafting: server.cpp:552-564 */
/* The tokens that followed the most recent earlier occurrence of the history's last n tokens, for n = min(4, L-1)
 * down to min_n; at most kmax of them, stopping before an eos token; a match whose continuation is empty (its next
 * token is eos) is passed over. Writes the draft to out and returns its length (0: none). */
int fso_lookup_draft(const int32_t* h, int64_t L, int kmax, int32_t eos, int min_n, int32_t* out) {
    int64_t n;
    for (n = (L - 1 < 4 ? L - 1 : 4); n >= min_n; --n) {
        int64_t p;
        for (p = L - n - 1; p >= 0; --p) {
            int eq = 1;
            for (int64_t k = 0; k < n; ++k)
                if (h[p + k] != h[L - n + k]) { eq = 0; break; }
            if (!eq) continue;
            int d = 0;
            for (int64_t k = p + n; k < L && d < kmax; ++k) {
                if (h[k] == eos) break;
                out[d++] = h[k];
            }
            if (d > 0) return d;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ Gemma 4 softcap: model_gemma4_gpu.cpp:282-283 */
/* out[i] = cap * tanhf(in[i] / cap), the model's host loop verbatim in arithmetic (the C library's tanhf), over
 * nthreads threads. */
typedef struct { const float* in; float* out; int64_t lo, hi; float cap; } cap_job;
static void* cap_worker(void* p) {
    const cap_job* j = (const cap_job*)p;
    for (int64_t i = j->lo; i < j->hi; ++i) j->out[i] = j->cap * tanhf(j->in[i] / j->cap);
    return 0;
}
void fso_softcap(const float* in, float* out, int64_t n, float cap, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    cap_job jobs[64];
    pthread_t th[64];
    for (int t = 0; t < nthreads; ++t) {
        cap_job j = { in, out, n * t / nthreads, n * (t + 1) / nthreads, cap };
        jobs[t] = j;
    }
    for (int t = 1; t < nthreads; ++t) pthread_create(&th[t], 0, cap_worker, &jobs[t]);
    cap_worker(&jobs[0]);
    for (int t = 1; t < nthreads; ++t) pthread_join(th[t], 0);
}
