// ferro_sampler.hpp - header-only C++ drop-in for ferro::Sampler (reference src/sampler.h:23-34) over the C ABI of
// ferro_sampler.h. Replace `ferro::Sampler` with `ferro_amd::Sampler` at the call sites
// (src/server.cpp:546,605,631; src/lm_cli.cpp:129,324,344); link libferro_sampler.so and libamdhip64.
//
//   ferro_amd::Sampler s(params);                    // params: ferro's SamplerParams fields (+ freq/presence)
//   int tok = s.sample(host_row, n_vocab, history);  // as ferro: the host row is left penalised in place
//   int tok = s.sample_device(d_row, n_vocab, history);  // device-resident row (no PCIe copy of the logits)
//
// Semantics match ferro::Sampler::sample token for token: the same std::mt19937_64 seeded the same way
// (sampler.h:25), one generate_canonical draw per sampled (non-greedy) call and none for greedy calls
// (sampler.cpp:19-23,45-46). Unlike ferro, failures of the device path throw std::runtime_error (ferro's
// sample cannot fail). One instance per stream and caller thread, as ferro's.
//
// Per call (besides the row's own copy in sample()): the window offsets, the draw and the history are written to
// pinned, device-mapped host memory that the kernel reads directly, and the kernel writes the token there too (no
// copy commands for them); one kernel (fs_sample_batch_hp: the parameters are on the host, so the library picks its
// kernel without reading them back); one device->host copy of the error bits into mapped memory, whose arrival the
// host polls for (it follows the kernel on the stream) instead of synchronizing the stream.
#pragma once

#include <hip/hip_runtime.h>

#include <chrono>
#include <climits>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "ferro_sampler.h"

static_assert(sizeof(int) == sizeof(int32_t), "history ids are copied as int32");

namespace ferro_amd {

// ferro::SamplerParams (src/sampler.h:12-21), same defaults, plus the frequency/presence extension (0 = off).
struct SamplerParams {
    float temperature = 0.05f;
    int top_k = 50;
    float top_p = 1.0f;
    float min_p = 0.0f;
    float repetition_penalty = 1.05f;
    int repeat_last_n = -1;
    int penalty_from = 0;
    uint64_t seed = 0;
    float frequency_penalty = 0.0f;
    float presence_penalty = 0.0f;
    float softcap = 0.0f;             // > 0: Gemma 4's final-logit softcap fused into the read (0 = off). For
                                      // sample_device on the model's raw output; a host row from ferro's model
                                      // code is already capped (model_gemma4_gpu.cpp:282-283): leave it 0 there.
};

class Sampler {
public:
    // write_back = true leaves the host row penalised like ferro's (one extra device->host copy of the row when
    // a penalty is active); false skips it (the token is the same).
    explicit Sampler(const SamplerParams& p, hipStream_t stream = nullptr, bool write_back = true)
        : p_(p), stream_(stream), write_back_(write_back) {
        check(fs_create(&ctx_), "fs_create");
        check(fs_rng_create(p.seed, &rng_), "fs_rng_create");
        rec_.temperature = p.temperature;
        rec_.top_k = p.top_k;
        rec_.top_p = p.top_p;
        rec_.min_p = p.min_p;
        rec_.repetition_penalty = p.repetition_penalty;
        rec_.frequency_penalty = p.frequency_penalty;
        rec_.presence_penalty = p.presence_penalty;
        rec_.repeat_last_n = p.repeat_last_n;
        rec_.penalty_from = p.penalty_from;
        rec_.softcap = p.softcap;
        hip(hipMalloc(&d_rec_, sizeof(rec_)), "hipMalloc");
        hip(hipMemcpy(d_rec_, &rec_, sizeof(rec_), hipMemcpyHostToDevice), "hipMemcpy");
        hip(hipHostMalloc((void**)&h_out_, 2 * sizeof(int32_t), hipHostMallocMapped), "hipHostMalloc");
        hip(hipHostGetDevicePointer((void**)&d_tok_, h_out_, 0), "hipHostGetDevicePointer");
        check(fs_error_word(ctx_, &d_err_), "fs_error_word");
        reserve(0);
    }
    ~Sampler() {
        (void)hipFree(d_row_);
        (void)hipFree(d_rec_);
        (void)hipHostFree(h_io_);
        (void)hipHostFree(h_out_);
        fs_rng_destroy(rng_);
        fs_destroy(ctx_);
    }
    Sampler(const Sampler&) = delete;
    Sampler& operator=(const Sampler&) = delete;

    // ferro::Sampler::sample (sampler.cpp:10): host row, penalised in place (when write_back).
    int sample(float* logits, int n_vocab, const std::vector<int>& history) {
        if (!logits || n_vocab < 1) throw std::runtime_error("ferro_amd::Sampler: bad row");
        const int64_t ld = ((int64_t)n_vocab + 3) & ~(int64_t)3;
        if (ld > row_cap_) {
            (void)hipFree(d_row_);
            d_row_ = nullptr;
            row_cap_ = 0;
            hip(hipMalloc(&d_row_, (size_t)ld * sizeof(float)), "hipMalloc");
            row_cap_ = ld;
        }
        hip(hipMemcpyAsync(d_row_, logits, (size_t)n_vocab * sizeof(float), hipMemcpyHostToDevice, stream_),
            "hipMemcpyAsync");
        const int tok = run(d_row_, n_vocab, history);
        if (write_back_ && penalised_) {
            check(fs_penalize_batch(ctx_, d_row_, ld, 1, n_vocab, hist_dev(), off_dev(), d_rec_, stream_),
                  "fs_penalize_batch");
            hip(hipMemcpyAsync(logits, d_row_, (size_t)n_vocab * sizeof(float), hipMemcpyDeviceToHost, stream_),
                "hipMemcpyAsync");
            hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
        }
        return tok;
    }

    // Device-resident row (16-byte aligned): read only; use fs_penalize_batch where the penalised row is wanted.
    int sample_device(const float* d_logits, int n_vocab, const std::vector<int>& history) {
        return run(d_logits, n_vocab, history);
    }

    const SamplerParams& params() const { return p_; }

private:
    // the per-call upload, packed: the window offsets {0, h}, the draw, then the history ids
    static constexpr size_t kHead = 2 * sizeof(int64_t) + sizeof(double);
    int64_t* off_dev() const { return reinterpret_cast<int64_t*>(d_io_); }
    double* u_dev() const { return reinterpret_cast<double*>(d_io_ + 2 * sizeof(int64_t)); }
    int32_t* hist_dev() const { return reinterpret_cast<int32_t*>(d_io_ + kHead); }

    void reserve(int64_t h) {
        if (h <= hist_cap_ && d_io_) return;
        const int64_t cap = h > 2 * hist_cap_ ? h : 2 * hist_cap_ + 64;
        if (h_io_) hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");   // no kernel still reads it
        (void)hipHostFree(h_io_);
        d_io_ = nullptr;
        h_io_ = nullptr;
        hist_cap_ = 0;
        hip(hipHostMalloc((void**)&h_io_, kHead + (size_t)cap * sizeof(int32_t), hipHostMallocMapped), "hipHostMalloc");
        hip(hipHostGetDevicePointer((void**)&d_io_, h_io_, 0), "hipHostGetDevicePointer");
        hist_cap_ = cap;
    }

    // The call's last command is the copy of the error bits into h_out_[1]: both mapped words leave kPending only
    // after the kernel (which wrote the token) has finished. Polling them returns about 5 us sooner than a stream
    // synchronization; a call still pending after kSpinUs falls back to the synchronization.
    static constexpr int32_t kPending = INT32_MIN;
    static constexpr double kSpinUs = 100000.0;
    void wait_done() {
        volatile const int32_t* out = h_out_;
        const auto t0 = std::chrono::steady_clock::now();
        for (unsigned i = 1;; ++i) {
            if (out[1] != kPending && out[0] != kPending) return;
            if ((i & 1023u) == 0u &&
                std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() > kSpinUs)
                break;
        }
        hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
        if (out[1] == kPending || out[0] == kPending)
            throw std::runtime_error("ferro_amd::Sampler: the call finished without writing its token");
    }

    static void check(int rc, const char* what) {
        if (rc != FS_OK) throw std::runtime_error(std::string("ferro_amd::Sampler: ") + what + ": " + fs_strerror(rc));
    }
    static void hip(hipError_t e, const char* what) {
        if (e != hipSuccess)
            throw std::runtime_error(std::string("ferro_amd::Sampler: ") + what + ": " + hipGetErrorString(e));
    }

    int run(const float* d_logits, int n_vocab, const std::vector<int>& history) {
        const bool greedy = p_.temperature <= 0.0f || p_.top_k == 1;      // sampler.cpp:19: no draw
        double u = 0.0;
        if (!greedy) check(fs_rng_next_u(rng_, &u, 1), "fs_rng_next_u");
        const int64_t h = (int64_t)history.size();
        reserve(h);
        // {0, h}, u and the history in the mapped staging buffer, which the kernel reads over the bus (the previous
        // call's kernel has finished with it: each call ends with a synchronization)
        const int64_t off[2] = {0, h};
        memcpy(h_io_, off, sizeof(off));
        memcpy(h_io_ + 2 * sizeof(int64_t), &u, sizeof(u));
        if (h) memcpy(h_io_ + kHead, history.data(), (size_t)h * sizeof(int32_t));   // int is int32_t here
        const int64_t ld = ((int64_t)n_vocab + 3) & ~(int64_t)3;
        volatile int32_t* out = h_out_;
        out[0] = kPending;
        out[1] = kPending;
        const int rc = fs_sample_batch_hp(ctx_, d_logits, ld, 1, n_vocab, h ? hist_dev() : nullptr, off_dev(), d_rec_,
                                          &rec_, u_dev(), d_tok_, 0, nullptr, nullptr, nullptr, stream_);
        if (rc < 0) check(rc, "fs_sample_batch_hp");               // FS_W_RECOVERED: the call ran normally
        // the token lands in h_out_[0] from the kernel; the error bits are copied into h_out_[1] behind it
        hip(hipMemcpyAsync(&h_out_[1], d_err_, sizeof(int32_t), hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync");
        wait_done();
        if (h_out_[1] != 0) {
            int32_t bits = 0;
            check(fs_device_error(ctx_, stream_, &bits), "fs_device_error");     // clears them
            throw std::runtime_error("ferro_amd::Sampler: device error bits " + std::to_string(bits));
        }
        penalised_ = h > 0 && p_.repeat_last_n != 0 &&
                     (p_.repetition_penalty != 1.0f || p_.frequency_penalty != 0.0f || p_.presence_penalty != 0.0f);
        return h_out_[0];
    }

    SamplerParams p_;
    hipStream_t stream_;
    bool write_back_;
    bool penalised_ = false;
    fs_context* ctx_ = nullptr;
    fs_rng* rng_ = nullptr;
    fs_row_params rec_{};
    fs_row_params* d_rec_ = nullptr;
    int32_t* d_tok_ = nullptr;
    const int32_t* d_err_ = nullptr;
    int32_t* h_out_ = nullptr;       // pinned, device-mapped: token (written by the kernel), error bits
    unsigned char* h_io_ = nullptr;  // pinned, device-mapped: offsets, draw, history
    unsigned char* d_io_ = nullptr;  // its device address
    float* d_row_ = nullptr;
    int64_t row_cap_ = 0;
    int64_t hist_cap_ = 0;
};

}  // namespace ferro_amd
