/* ferro_sampler.h - C ABI of the MI355X (gfx950) token sampler.
 *
 * Drop-in device replacement for ferro's host sampler, ferro::Sampler (reference src/sampler.h:23-34,
 * src/sampler.cpp:10-50): repetition penalty -> greedy | top-k -> softmax at temperature -> min-p -> top-p ->
 * multinomial draw, plus the speculative-draft verification rule of the server (src/server.cpp:627-637).
 *
 * Conventions (all entry points):
 *   - every pointer named d_* is device memory owned by the caller; nothing is retained after the call returns;
 *   - work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the default stream);
 *   - the return value is FS_OK or a negative FS_E_* code; nothing throws across the ABI;
 *   - a context may be used from any thread, but calls on one context must not overlap in time (they share its
 *     device workspace): serialise them on one stream, or use one context per stream;
 *   - logits rows are fp32, row b starts at d_logits + b*ld, ld >= V, ld % 4 == 0, d_logits 16-byte aligned;
 *     only elements [0, V) of each row are read. Logits are read only: the penalty is applied on the fly and
 *     never written back (ferro's sample() penalises its host row in place).
 *   - per-row draws d_u are doubles in [0,1): r = u * tot replaces ferro's uniform_real_distribution(0, tot)
 *     draw from its mt19937_64 (libstdc++ computes exactly generate_canonical * tot). Greedy rows ignore u.
 */
#ifndef FERRO_SAMPLER_H
#define FERRO_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FS_OK 0
#define FS_E_INVALID (-1)   /* bad argument: null pointer, size out of range, misalignment */
#define FS_E_HIP (-2)       /* a HIP runtime call failed */
#define FS_E_NOMEM (-3)     /* workspace allocation failed */
#define FS_E_DEVICE (-4)    /* a kernel reported a row it could not process (see fs_device_error) */
#define FS_E_LIMIT (-5)     /* fs_sample_batch_static: the batch exceeds its static workspace */
#define FS_W_RECOVERED 1    /* success; an earlier call's merge had given up waiting for its segments
                               (FS_DEVERR_INTERNAL, kept for fs_device_error) and this call cleared the workspace
                               that call left, so the context does not stay in its compute-alone mode */

/* Device-side error bits (fs_device_error). */
#define FS_DEVERR_COUNT_OVERFLOW 1   /* one token occurs > 65535 times in a penalty window */
#define FS_DEVERR_INTERNAL 2         /* an internal invariant failed, or a row's merge gave up waiting for its
                                        segments (workgroups not dispatched round-robin over the XCDs by index, or
                                        a wait limit below the segments' time). The row was then computed alone from
                                        its logits (the token is exact). The next sampling call on the context (or
                                        fs_device_error) clears the workspace; that call returns FS_W_RECOVERED */
#define FS_DEVERR_HIST_APPEND 4      /* fs_hist_append: the new histories exceed out_cap (ids past it are not
                                        written), or a count lies outside [0, its stream's rows] (clamped) */

/* Limits. A row is read through one buffer resource (32-bit byte range): V * 4 < 2^31. */
#define FS_MAX_VOCAB (1 << 28)

/* Per-row sampling parameters. Fields 1-5 and 8-9 are ferro's SamplerParams (src/sampler.h:12-21) with the
 * same meaning and defaults; the seed is replaced by the per-row draw u. frequency_penalty / presence_penalty
 * extend ferro (llama.cpp convention: l -= cnt*freq + (cnt>0)*pres over the penalty window, after the
 * repetition step); 0 leaves a row bit-identical to ferro. softcap moves the model's final-logit transform into
 * the sampler's read (the logits stay as produced); fs_penalize_batch ignores it. */
typedef struct fs_row_params {
    float temperature;        /* <= 0: greedy (argmax after penalties)        sampler.h:13 */
    int32_t top_k;            /* 0 = all tokens; 1 = greedy                   sampler.h:14 */
    float top_p;              /* 1 = off                                      sampler.h:15 */
    float min_p;              /* 0 = off                                      sampler.h:16 */
    float repetition_penalty; /* 1 = off                                      sampler.h:17 */
    float frequency_penalty;  /* 0 = off (extension) */
    float presence_penalty;   /* 0 = off (extension) */
    int32_t repeat_last_n;    /* -1 whole history, 0 off, N last tokens       sampler.h:18 */
    int32_t penalty_from;     /* history positions before this never count    sampler.h:19 */
    float softcap;            /* > 0: logits become softcap * tanhf(l / softcap) before the penalties (Gemma 4's
                                 final-logit softcap, model_gemma4_gpu.cpp:282-283, fused into the read); 0 = off */
} fs_row_params;

typedef struct fs_context fs_context;

/* Create / destroy a context (owns a device workspace that grows on demand). Replaces constructing one
 * ferro::Sampler per stream (src/sampler.h:25); the per-stream RNG lives with the caller (u). */
int fs_create(fs_context** out);
int fs_destroy(fs_context* ctx);

/* Batched sample(): one token per row. Replaces the per-row loop
 *   for i: tok = sampler->sample(S.lg.data() + i*V, V, hist)          (src/server.cpp:603-606, sampler.cpp:10)
 * Row b's history is d_hist[d_hist_off[b] .. d_hist_off[b+1]) (d_hist_off has B+1 entries; d_hist may be NULL
 * when every row's history is empty). Outputs: d_tok[B]. Optional (NULL to skip): d_cand_ids / d_cand_probs
 * [B][kcap] receive the first min(k, kcap) candidates in ferro's candidate order (logit desc, id asc) and their
 * normalised probabilities pr[i] (sampler.cpp:37-41); d_keep[B] the kept prefix length after min-p / top-p.
 * Greedy rows report k = keep = 1 with probability 1. */
int fs_sample_batch(fs_context* ctx, const float* d_logits, int64_t ld, int32_t B, int32_t V,
                    const int32_t* d_hist, const int64_t* d_hist_off, const fs_row_params* d_params,
                    const double* d_u, int32_t* d_tok, int32_t kcap, int32_t* d_cand_ids, double* d_cand_probs,
                    int32_t* d_keep, void* stream);

/* fs_sample_batch with the parameters also in host memory: h_params holds the same B records as d_params (the
 * caller fills both; ferro's call sites hold SamplerParams on the host, sampler.h:25, server.cpp:603-606). With the
 * host copy the library picks the kernel for the batch without reading device memory: batches whose every row is
 * greedy (frequency / presence penalties only where rows split into segments of 4096 logits) or samples from at
 * most 64 candidates (k = top_k, or V when top_k is 0) with no frequency / presence penalty run on a kernel made for
 * them (every segment's loads issued at once, bitonic sorts in registers; all-greedy batches a greedy-only form);
 * batches mixing rows of 64 < k <= 2048 with cheaper rows run fs_sample_batch's kernel with about twice its segments;
 * other batches, and h_params = NULL, run fs_sample_batch. fs_route_plan reports the choice. Same outputs as
 * fs_sample_batch. h_params is read before the call returns. */
int fs_sample_batch_hp(fs_context* ctx, const float* d_logits, int64_t ld, int32_t B, int32_t V,
                       const int32_t* d_hist, const int64_t* d_hist_off, const fs_row_params* d_params,
                       const fs_row_params* h_params, const double* d_u, int32_t* d_tok, int32_t kcap,
                       int32_t* d_cand_ids, double* d_cand_probs, int32_t* d_keep, void* stream);

/* Host-only: the small-k kernel's layout for B rows of V logits on a device with `cus` compute units: *nl float4
 * loads per thread (segments of 1024 * nl logits) and *nseg segments per row; FS_E_LIMIT when V needs more than 64
 * segments (fs_sample_batch_hp then runs fs_sample_batch). No counterpart in the reference (a planner check). */
int fs_small_k_plan(int32_t cus, int32_t B, int32_t V, int32_t* nl, int32_t* nseg);

/* Host-only: the kernel fs_sample_batch_hp (verify = 0: n = total_rows = B row records) or fs_verify_hp (verify != 0:
 * n stream records over total_rows rows) launches for these host parameters, on a device with `cus` compute units
 * whose XCD count divides 8: *kernel 0 the fused kernel (*nseg segments per row, *per_cu segments per CU of its
 * layout), 1 the small-k kernel, 2 its greedy-only form (*nl float4 loads per thread, *nseg segments per row). No
 * counterpart in the reference (a routing check for callers and tests). */
int fs_route_plan(int32_t cus, const fs_row_params* h_params, int32_t n, int32_t total_rows, int32_t V,
                  int32_t verify, int32_t* kernel, int32_t* nl, int32_t* nseg, int32_t* per_cu);

/* fs_sample_batch without any allocation. No counterpart in the reference: it is for callers that cannot allocate
 * device memory during a call - code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * Same arguments, semantics and outputs as fs_sample_batch; ctx only carries settings (fs_set_wait_limit) and
 * error reporting (fs_device_error reads and clears this workspace's error bits too). The workspace is one static
 * device array per GPU (50.3 MB; it is part of the library's code object, so it is reserved on every device where
 * the library's module is loaded, held until the process ends, whether or not this entry point is ever called),
 * shared by every context on that GPU: calls that
 * overlap in time on one GPU race (serialise them on one stream). Limits: B <= 512 rows (beyond: FS_E_LIMIT, nothing
 * launched); every B <= 512 fits its 512 (row, segment) slots, taking fewer segments per row than fs_sample_batch
 * where the slots would run out (B = 17..23 at V = 262144, for example). The first call on a device also enqueues a clear of the workspace on `stream`. */
int fs_sample_batch_static(fs_context* ctx, const float* d_logits, int64_t ld, int32_t B, int32_t V,
                           const int32_t* d_hist, const int64_t* d_hist_off, const fs_row_params* d_params,
                           const double* d_u, int32_t* d_tok, int32_t kcap, int32_t* d_cand_ids, double* d_cand_probs,
                           int32_t* d_keep, void* stream);

/* Greedy batch: argmax after penalties, lowest index on ties (sampler.cpp:19-23). d_params may be NULL (no
 * penalties: the context keeps greedy parameter records of its own, on the device and the host, for the small-k
 * kernel); otherwise only the penalty fields are read and every row is treated as greedy. */
int fs_argmax_batch(fs_context* ctx, const float* d_logits, int64_t ld, int32_t B, int32_t V,
                    const int32_t* d_hist, const int64_t* d_hist_off, const fs_row_params* d_params,
                    int32_t* d_tok, void* stream);

/* Speculative verification window (src/server.cpp:613-651). Stream s owns logits rows
 * d_row_off[s] .. d_row_off[s+1]-1 (d_row_off has n_streams+1 entries, total rows = d_row_off[n_streams]);
 * d_rows[r] is the token fed at row r: d_rows[d_row_off[s]] is the stream's last sampled token, the rest are its
 * drafts. Row r of stream s is sampled with history = d_hist[d_hist_off[s] .. d_hist_off[s+1]) followed by the
 * drafts fed before it (d_rows[d_row_off[s]+1 .. d_row_off[s]+r]), with params d_params[s] and draw d_u[row].
 * Outputs: d_tok[row] for every row, and d_accepted[s] = 1 + the number of leading rows r < m-1 whose token
 * equals the next draft; a row whose token is eos_id (>= 0; -1 = none) ends the window at that row. */
int fs_verify(fs_context* ctx, const float* d_logits, int64_t ld, int32_t n_streams, int32_t total_rows,
              int32_t V, const int32_t* d_rows, const int64_t* d_row_off, const int32_t* d_hist,
              const int64_t* d_hist_off, const fs_row_params* d_params, const double* d_u, int32_t eos_id,
              int32_t* d_tok, int32_t* d_accepted, void* stream);

/* fs_verify with the stream parameters also in host memory (h_params: the same n_streams records as d_params). Windows
 * whose every stream is greedy or samples from at most 64 candidates, with no active penalty (repetition 1, or
 * repeat_last_n 0, and no frequency / presence penalty: a row's history then does not matter), run on the small-k
 * kernel of fs_sample_batch_hp; other windows, and h_params = NULL, run fs_verify. Same outputs as fs_verify. */
int fs_verify_hp(fs_context* ctx, const float* d_logits, int64_t ld, int32_t n_streams, int32_t total_rows,
                 int32_t V, const int32_t* d_rows, const int64_t* d_row_off, const int32_t* d_hist,
                 const int64_t* d_hist_off, const fs_row_params* d_params, const fs_row_params* h_params,
                 const double* d_u, int32_t eos_id, int32_t* d_tok, int32_t* d_accepted, void* stream);

/* Host draw source matching ferro::Sampler's std::mt19937_64 stream (src/sampler.h:25,32; sampler.cpp:45-46):
 * fs_rng_next_u returns generate_canonical<double,53> values, so u * tot is ferro's draw r. seed 0 = random.
 * A sampled (non-greedy) row consumes one u; greedy rows consume none (sampler.cpp:19-23). fs_rng_copy lets a
 * verifier draw a window's u ahead and commit only the accepted count (fs_rng_next_u on the original). */
typedef struct fs_rng fs_rng;
int fs_rng_create(uint64_t seed, fs_rng** out);
int fs_rng_destroy(fs_rng* r);
int fs_rng_next_u(fs_rng* r, double* u, int32_t n);
int fs_rng_copy(const fs_rng* src, fs_rng* dst);

/* Prompt-lookup drafting (src/server.cpp:552-564, src/lm_cli.cpp:145): for stream s with history
 * d_hist[d_hist_off[s] .. d_hist_off[s+1]) (L tokens), the tokens that followed the most recent earlier
 * occurrence of its last n tokens, trying n = min(4, L-1) down to d_min_n[s] (NULL: 2), at most d_kmax[s] (NULL:
 * draft_ld; clamped to draft_ld), stopping before eos_id (-1: none); a match followed directly by eos is passed
 * over. Writes d_draft[s*draft_ld + i] and d_ndraft[s] (0: no draft): the drafts that fs_verify then checks. */
int fs_lookup_draft(fs_context* ctx, int32_t n_streams, const int32_t* d_hist, const int64_t* d_hist_off,
                    const int32_t* d_kmax, const int32_t* d_min_n, int32_t eos_id, int32_t* d_draft, int32_t draft_ld,
                    int32_t* d_ndraft, void* stream);

/* History append: the per-stream hist.push_back of each consumed token (src/server.cpp:342, in gen_token; fed one
 * token per stream by the decode loop, server.cpp:603-606, and the accepted prefix by the verify window,
 * server.cpp:627-637), on device CSR histories, out of place. Stream s keeps d_hist[d_hist_off[s] ..
 * d_hist_off[s+1]) and gains d_tok[d_row_off[s] + i] for i < d_count[s] (d_row_off NULL: row s; d_count NULL: 1
 * per stream; fs_verify's d_tok / d_row_off / d_accepted fit as they are). Writes d_out_hist_off[0 .. n_streams]
 * (rebased to start at 0) and d_out_hist (capacity out_cap ids); an overflow or a count outside [0, the stream's
 * rows] sets FS_DEVERR_HIST_APPEND. The outputs must not alias the inputs; d_hist and d_tok may be NULL
 * only with no streams. Token rewrites the host applies after sampling (gen_token's think-budget close, server.cpp:339) must be
 * applied to d_tok first. */
int fs_hist_append(fs_context* ctx, int32_t n_streams, const int32_t* d_hist, const int64_t* d_hist_off,
                   const int32_t* d_tok, const int64_t* d_row_off, const int32_t* d_count, int32_t* d_out_hist,
                   int64_t out_cap, int64_t* d_out_hist_off, void* stream);

/* Device draw streams: n_streams std::mt19937_64 engines held in device memory (seeds[s] from the host; 0 =
 * random, as ferro), drawing libstdc++ generate_canonical<double,53> values - ferro::Sampler's draw stream
 * (sampler.h:25,32; sampler.cpp:45-46) without a host round trip. Stream s owns rows d_row_off[s] ..
 * d_row_off[s+1]-1 (d_row_off NULL: one row per stream, row s); d_params[s] are its sampling parameters.
 * fs_drng_draw writes d_u[row]: one draw per row of a sampling stream (temperature > 0 and top_k != 1), in row
 * order, as ferro's sequential sample() calls; rows of greedy streams get 0 and consume nothing. peek != 0 computes
 * the draws without consuming them (at most 156 draws past the engine's next twist; more sets FS_DEVERR_INTERNAL):
 * a verify window peeks its rows' draws, then fs_drng_skip consumes d_counts[s] draws per sampling stream (e.g.
 * fs_verify's d_accepted). The draws equal fs_rng_next_u on the same seeds. Calls on one fs_drng must be ordered
 * (one stream). */
typedef struct fs_drng fs_drng;
int fs_drng_create(int32_t n_streams, const uint64_t* seeds, void* stream, fs_drng** out);
int fs_drng_destroy(fs_drng* r);
int fs_drng_draw(fs_drng* r, const int64_t* d_row_off, const fs_row_params* d_params, double* d_u, int32_t peek,
                 void* stream);
int fs_drng_skip(fs_drng* r, const int32_t* d_counts, const fs_row_params* d_params, void* stream);
/* Waits for `stream`, then returns and clears the stream set's error bits. */
int fs_drng_error(fs_drng* r, void* stream, int32_t* bits);

/* One decode step in one launch: the loop body of server.cpp:603-606 (each stream's draw and sample()) followed by
 * gen_token's hist.push_back (server.cpp:342), for B streams with one row each (row s = stream s of r, B <= its
 * stream count). Equivalent to fs_drng_draw (d_row_off NULL) + fs_sample_batch (kcap 0) + fs_hist_append (one
 * token per stream) on the same arguments, in the sampling grid: each row's merge copies its stream's history to
 * the new histories while its segments run, reads its draw from the stream without advancing it, and after the
 * row is sampled appends the token and advances the stream (greedy rows draw nothing). d_out_hist / d_out_hist_off
 * are laid out as fs_hist_append's (offsets rebased to 0, out_cap ids; overflow sets FS_DEVERR_HIST_APPEND, read
 * with fs_device_error) and must not alias the inputs. d_keep may be NULL. No counterpart call in the reference: it
 * fuses three of its steps for a device-resident decode loop. */
int fs_decode_step(fs_context* ctx, fs_drng* r, const float* d_logits, int64_t ld, int32_t B, int32_t V,
                   const int32_t* d_hist, const int64_t* d_hist_off, const fs_row_params* d_params, int32_t* d_tok,
                   int32_t* d_keep, int32_t* d_out_hist, int64_t* d_out_hist_off, int64_t out_cap, void* stream);

/* fs_decode_step with a host copy of the parameters too (h_params: B records, as fs_sample_batch_hp): batches the
 * small-k kernel fits run on it, with the same three additions in each row's merge; others run fs_decode_step.
 * Same outputs and stream semantics. No counterpart call in the reference (the server holds its SamplerParams on
 * the host, server.cpp:603-606). */
int fs_decode_step_hp(fs_context* ctx, fs_drng* r, const float* d_logits, int64_t ld, int32_t B, int32_t V,
                      const int32_t* d_hist, const int64_t* d_hist_off, const fs_row_params* d_params,
                      const fs_row_params* h_params, int32_t* d_tok, int32_t* d_keep, int32_t* d_out_hist,
                      int64_t* d_out_hist_off, int64_t out_cap, void* stream);

/* The penalty stage alone, in place: row b of d_logits is left exactly as ferro's sample() leaves its host row
 * (sampler.cpp:11-18: each distinct window id in [0, V) once, l > 0 ? l/rep : l*rep, then the frequency/presence
 * extension). For callers that read the penalised row back (lm_cli.cpp:353); fs_sample_batch does not need it (it
 * penalises on the fly). Rows without an active penalty, and every row when d_hist or d_hist_off is NULL, are
 * left untouched. Same row layout rules as fs_sample_batch. */
int fs_penalize_batch(fs_context* ctx, float* d_logits, int64_t ld, int32_t B, int32_t V, const int32_t* d_hist,
                      const int64_t* d_hist_off, const fs_row_params* d_params, void* stream);

/* Gemma 4's final-logit softcap as the sampler applies it (fs_row_params.softcap): d_out[i] = cap * tanhf(d_in[i] /
 * cap), the host loop of model_gemma4_gpu.cpp:282-283, bit-identical to it on a glibc host (its float tanh is
 * restated on the device). For callers that need the capped logits themselves (log-probabilities); sampling does
 * not (the cap is fused into its read). In place when d_out == d_in; cap > 0. */
int fs_softcap_batch(const float* d_in, float* d_out, int64_t n, float cap, void* stream);

/* Waits for `stream`, then returns and clears the device error bits (FS_DEVERR_*) kernels of this context set; after
 * FS_DEVERR_INTERNAL it also clears the context's workspace (row histograms and counters). A context that has
 * called fs_sample_batch_static also reports and clears the bits of its device's static workspace. */
int fs_device_error(fs_context* ctx, void* stream, int32_t* bits);

/* The device address of the context's error bits (the word fs_device_error reads and clears). A caller that samples
 * in a loop can copy it asynchronously on its stream together with its outputs, and call fs_device_error (which
 * synchronizes, then clears) only when a bit is set. No counterpart in the reference (ferro's sample cannot fail). */
int fs_error_word(fs_context* ctx, const int32_t** d_bits);

/* The merge's bounded wait for a row's segments, in polls (0 = the default, 2^20: far above any segment's time).
 * A smaller limit makes merges give up (FS_DEVERR_INTERNAL) and compute their rows alone; FS_WAIT_GIVE_UP makes
 * every merge give up without polling: tests of that path. */
#define FS_WAIT_GIVE_UP 0xFFFFFFFFu
int fs_set_wait_limit(fs_context* ctx, uint32_t polls);

/* Host-only: the layout fs_sample_batch (static_ws = 0) or fs_sample_batch_static (static_ws != 0) launches for B
 * rows of V logits on a device with `cus` compute units and `xccs` XCDs: *nseg segments of *seg_tiles 4096-logit
 * tiles per row and *slots workspace slots. *nseg = 0 with V >= 4096: every row is sampled alone by one workgroup
 * (an XCD count that does not divide 8, where the segment grid's hand-off would not hold). Returns FS_E_LIMIT where
 * fs_sample_batch_static would. No counterpart in the reference; it lets tests check the planner without a GPU. */
int fs_plan_layout(int32_t cus, int32_t xccs, int32_t B, int32_t V, int32_t static_ws, int32_t* nseg,
                   int32_t* seg_tiles, int64_t* slots);

/* Static description of the error code. */
const char* fs_strerror(int code);

#ifdef __cplusplus
}
#endif

#endif /* FERRO_SAMPLER_H */
