// ref_harness.cpp - C entry points over the REFERENCE ferro::Sampler (compiled from
// /root/reference/src/sampler.cpp where it lies; nothing of it is copied here). Test infrastructure only:
// it writes the golden vectors under tests/golden/ and is the "reference" CPU baseline of bench.py.
#include <cstdint>
#include <thread>
#include <vector>

#include "sampler.h"   // /root/reference/src/sampler.h

namespace {
// Reference fields of SamplerParams (src/sampler.h:12-21); frequency/presence do not exist there.
struct RefParams {
    float temperature; int32_t top_k; float top_p; float min_p; float repetition_penalty;
    float frequency_penalty; float presence_penalty; int32_t repeat_last_n; int32_t penalty_from; int32_t reserved;
};
ferro::SamplerParams to_sp(const RefParams* p, uint64_t seed) {
    ferro::SamplerParams sp;
    sp.temperature = p->temperature; sp.top_k = p->top_k; sp.top_p = p->top_p; sp.min_p = p->min_p;
    sp.repetition_penalty = p->repetition_penalty; sp.repeat_last_n = p->repeat_last_n;
    sp.penalty_from = p->penalty_from; sp.seed = seed;
    return sp;
}
}  // namespace

extern "C" {

// A stateful reference Sampler (one per stream, as ferro's server keeps one per request: server.cpp:170,545).
void* ref_sampler_new(const RefParams* p, uint64_t seed) { return new ferro::Sampler(to_sp(p, seed)); }
void ref_sampler_free(void* s) { delete static_cast<ferro::Sampler*>(s); }
int ref_sampler_sample(void* s, float* logits, int n, const int32_t* hist, int64_t hlen) {
    std::vector<int> h(hist, hist + hlen);
    return static_cast<ferro::Sampler*>(s)->sample(logits, n, h);
}

// Row b sampled by a fresh Sampler(seed[b]) on logits + b*ld (penalised in place), rows spread over nthreads.
void ref_sample_batch(float* logits, int64_t ld, int B, int n, const int32_t* hist, const int64_t* hist_off,
                      const RefParams* params, const uint64_t* seeds, int32_t* tok, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    auto work = [&](int t) {
        for (int b = t; b < B; b += nthreads) {
            ferro::Sampler s(to_sp(&params[b], seeds[b]));
            std::vector<int> h(hist + hist_off[b], hist + hist_off[b + 1]);
            tok[b] = s.sample(logits + (int64_t)b * ld, n, h);
        }
    };
    if (nthreads == 1) { work(0); return; }
    std::vector<std::thread> th;
    for (int t = 0; t < nthreads; ++t) th.emplace_back(work, t);
    for (auto& x : th) x.join();
}

}  // extern "C"
