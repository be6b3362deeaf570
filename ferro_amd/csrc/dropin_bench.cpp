// Per-call cost of the C++ drop-in ferro_amd::Sampler (include/ferro_sampler.hpp), used the way ferro's single-row
// call sites use ferro::Sampler: src/server.cpp:546 (a request's first token) and src/lm_cli.cpp:129,324 (one row per
// generated token). Config 1's row: V = 65536 fp32, N(0, 2) plus 8 spikes at +12, repetition 1.1 over a 64-token
// history, temperature 0.7, top-k 40, top-p 0.95. Each call samples one row and appends the token to the history.
//
// usage: dropin_bench [calls]   ->  one JSON object on stdout, microseconds per call (wall clock, host timer):
//   host_row:            sample(host row): the row copied host -> device, the call, the token back (the server)
//   host_row_writeback:  the same leaving the host row penalised in place, as ferro's sample does (lm_cli.cpp:353)
//   device_row:          sample_device(row already on the device): no copy of the logits
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "ferro_sampler.hpp"

int main(int argc, char** argv) {
    const int calls = argc > 1 ? atoi(argv[1]) : 2000;
    const int V = 65536;
    std::mt19937_64 g(1);
    std::normal_distribution<float> nd(0.0f, 2.0f);
    std::vector<float> row(V);
    for (auto& x : row) x = nd(g);
    for (int i = 0; i < 8; ++i) row[g() % V] = 12.0f;
    std::vector<int> hist0(64);
    for (auto& h : hist0) h = (int)(g() % V);
    ferro_amd::SamplerParams p;
    p.temperature = 0.7f; p.top_k = 40; p.top_p = 0.95f; p.repetition_penalty = 1.1f; p.seed = 5489;
    float* d_row = nullptr;
    if (hipMalloc(&d_row, V * sizeof(float)) != hipSuccess) return 1;
    if (hipMemcpy(d_row, row.data(), V * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) return 1;
    auto timed = [&](int mode) {
        ferro_amd::Sampler s(p, nullptr, mode == 1);
        std::vector<int> hist = hist0;
        std::vector<float> work = row;
        auto one = [&]() {
            int t;
            if (mode == 2) t = s.sample_device(d_row, V, hist);
            else {
                if (mode == 1) work = row;                        // sample() left the row penalised
                t = s.sample(work.data(), V, hist);
            }
            hist.push_back(t);
            if (hist.size() > 512) hist.erase(hist.begin(), hist.begin() + 448);
        };
        for (int i = 0; i < 50; ++i) one();
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < calls; ++i) one();
        const auto t1 = std::chrono::steady_clock::now();
        return std::chrono::duration<double, std::micro>(t1 - t0).count() / calls;
    };
    const double host = timed(0), host_wb = timed(1), dev = timed(2);
    printf("{\"calls\": %d, \"V\": %d, \"host_row_us\": %.2f, \"host_row_writeback_us\": %.2f, \"device_row_us\": %.2f}\n",
           calls, V, host, host_wb, dev);
    (void)hipFree(d_row);
    return 0;
}
