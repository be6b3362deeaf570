/* sampler_oracle.h - CPU restatement of ferro's token sampler, used ONLY as the test checker and the
 * timed CPU baseline (never linked into or called by the product library under ferro_amd/).
 *
 * Follows /root/reference/src/sampler.h:12-34 and /root/reference/src/sampler.cpp:10-50 step by step:
 * repetition penalty -> greedy | top-k -> softmax at temperature (double) -> min-p -> top-p -> draw.
 * Two deliberate differences from ferro::Sampler::sample:
 *   - the draw takes a caller-supplied u in [0,1) and forms r = u * tot. libstdc++'s
 *     uniform_real_distribution<double>(0, tot) computes exactly generate_canonical(rng) * tot + 0.0, and
 *     fso_canonical() restates generate_canonical<double,53> for mt19937_64 (one 64-bit draw / 2^64).
 *   - frequency / presence penalties (not in ferro) follow the llama.cpp convention,
 *     l -= cnt * freq + (cnt > 0) * pres, applied after the repetition step over the same window; with
 *     freq = pres = 0 the row is unchanged bit for bit.
 * One policy where ferro's result is unspecified: with a NaN logit in a sampled row, ferro's candidate
 * comparator (sampler.cpp:30) is no strict weak order. Here NaN ranks below every number and is never a
 * candidate: k becomes min(k, the row's count of numbers); a row of NaNs only gives token 0 and keeps 0. Rows
 * without a NaN are unaffected. Parity on NaN rows is therefore pinned to this policy, not to ferro.
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same field order and meaning as fs_row_params in include/ferro_sampler.h. */
typedef struct fso_params {
    float temperature;        /* <= 0: greedy */
    int32_t top_k;            /* 0 = off (all tokens); 1 = greedy */
    float top_p;              /* 1 = off */
    float min_p;              /* 0 = off */
    float repetition_penalty; /* 1 = off */
    float frequency_penalty;  /* 0 = off (extension) */
    float presence_penalty;   /* 0 = off (extension) */
    int32_t repeat_last_n;    /* -1 whole history, 0 off, N last tokens */
    int32_t penalty_from;     /* history positions before this are never penalised */
    float softcap;            /* > 0: l = softcap * tanhf(l / softcap) first (model_gemma4_gpu.cpp:282-283) */
} fso_params;

/* Penalty stage in place (sampler.cpp:11-18 + extension). Returns the number of distinct ids changed. */
int fso_penalize(float* row, int n, const int32_t* hist, int64_t hlen, const fso_params* p);

/* One full sample() call on a row (the row is penalised in place, as the reference does).
 * Optional outputs (any may be NULL): cand_ids / cand_probs receive the first min(ncand, kcap) candidates in
 * candidate order with their normalised probabilities pr[i]; *keep_out the kept prefix length after min-p/top-p;
 * *ncand_out the candidate count k. For a greedy row: ncand = keep = 1, cand = {argmax}, prob = 1.0. */
int fso_sample(float* row, int n, const int32_t* hist, int64_t hlen, const fso_params* p, double u,
               int32_t* cand_ids, double* cand_probs, int kcap, int32_t* keep_out, int32_t* ncand_out);

/* Batch over rows (row b = logits + b*ld, history CSR hist[hist_off[b] .. hist_off[b+1])), rows spread over
 * nthreads POSIX threads. Per-row outputs as fso_sample with leading dimension kcap. Rows are penalised in place. */
/* The model's final-logit softcap (model_gemma4_gpu.cpp:282-283): out[i] = cap * tanhf(in[i] / cap). */
void fso_softcap(const float* in, float* out, int64_t n, float cap, int nthreads);

void fso_sample_batch(float* logits, int64_t ld, int B, int n, const int32_t* hist, const int64_t* hist_off,
                      const fso_params* params, const double* u, int32_t* tok, int32_t* cand_ids,
                      double* cand_probs, int kcap, int32_t* keep, int32_t* ncand, int nthreads);

/* Speculative verification window (server.cpp:627-637). Stream s owns rows row_off[s]..row_off[s+1]-1; rows[r]
 * is the token fed at row r (rows[row_off[s]] = the last sampled token, the rest drafts). Row r's history is the
 * stream's base history followed by rows[row_off[s]+1 .. row_off[s]+r]. Every row is sampled (tok[]), then
 * accepted[s] = 1 + the number of leading rows r < m-1 whose token equals rows[row_off[s]+r+1]; a row whose token
 * is eos_id (>= 0) ends the window there. Rows are penalised in place. */
void fso_verify(float* logits, int64_t ld, int n_streams, int n, const int32_t* rows, const int64_t* row_off,
                const int32_t* hist, const int64_t* hist_off, const fso_params* params, const double* u,
                int32_t eos_id, int32_t* tok, int32_t* accepted);

/* Prompt-lookup drafting (server.cpp:552-564): the tokens that followed the most recent earlier occurrence of the
 * last n tokens of h[0, L), n = min(4, L-1) down to min_n; at most kmax, stopping before eos. Returns the length. */
int fso_lookup_draft(const int32_t* h, int64_t L, int kmax, int32_t eos, int min_n, int32_t* out);

/* mt19937_64 (Matsumoto & Nishimura 2004 parameters, as std::mt19937_64) and the libstdc++ canonical mapping. */
typedef struct fso_mt64 { uint64_t mt[312]; int mti; } fso_mt64;
void fso_mt64_seed(fso_mt64* s, uint64_t seed);
uint64_t fso_mt64_next(fso_mt64* s);
double fso_canonical(uint64_t x);

#ifdef __cplusplus
}
#endif
