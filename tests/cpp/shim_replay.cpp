// Replays sampling streams through ferro_amd::Sampler (include/ferro_sampler.hpp), the C++ drop-in for
// ferro::Sampler, the way ferro's callers use it (src/lm_cli.cpp:129-130: sample a host row, append the token).
//
// usage: shim_replay IN OUT
//   IN : int64 S, then per stream: fs_row_params (40 B), uint64 seed, int64 V, int64 steps, int64 h0len,
//        int32 h0[h0len], float rows[steps][V]
//   OUT: per stream: int32 tok[steps], float rows[steps][V] as left by sample() (penalised in place)
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "ferro_sampler.hpp"

template <class T>
static void rd(FILE* f, T* p, size_t n) {
    if (n && fread(p, sizeof(T), n, f) != n) { fprintf(stderr, "short read\n"); exit(2); }
}

int main(int argc, char** argv) {
    if (argc != 3) { fprintf(stderr, "usage: %s IN OUT\n", argv[0]); return 2; }
    FILE* in = fopen(argv[1], "rb");
    FILE* out = fopen(argv[2], "wb");
    if (!in || !out) { fprintf(stderr, "cannot open files\n"); return 2; }
    int64_t S = 0;
    rd(in, &S, 1);
    for (int64_t s = 0; s < S; ++s) {
        fs_row_params r;
        uint64_t seed;
        int64_t V, steps, h0;
        rd(in, &r, 1); rd(in, &seed, 1); rd(in, &V, 1); rd(in, &steps, 1); rd(in, &h0, 1);
        std::vector<int> hist((size_t)h0);
        std::vector<int32_t> tmp((size_t)h0);
        rd(in, tmp.data(), (size_t)h0);
        for (int64_t i = 0; i < h0; ++i) hist[(size_t)i] = tmp[(size_t)i];
        std::vector<float> rows((size_t)(steps * V));
        rd(in, rows.data(), rows.size());
        ferro_amd::SamplerParams p;
        p.temperature = r.temperature; p.top_k = r.top_k; p.top_p = r.top_p; p.min_p = r.min_p;
        p.repetition_penalty = r.repetition_penalty; p.frequency_penalty = r.frequency_penalty;
        p.presence_penalty = r.presence_penalty; p.repeat_last_n = r.repeat_last_n; p.penalty_from = r.penalty_from;
        p.seed = seed;
        ferro_amd::Sampler smp(p);
        std::vector<int32_t> toks((size_t)steps);
        for (int64_t i = 0; i < steps; ++i) {
            const int t = smp.sample(rows.data() + i * V, (int)V, hist);
            toks[(size_t)i] = t;
            hist.push_back(t);
        }
        fwrite(toks.data(), sizeof(int32_t), toks.size(), out);
        fwrite(rows.data(), sizeof(float), rows.size(), out);
    }
    fclose(out);
    fclose(in);
    return 0;
}
