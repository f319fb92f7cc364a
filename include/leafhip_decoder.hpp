// leaf::runtime::Decoder on one MI355X, over the leafhip C ABI.
//
// Same class name, constructor arguments, methods and error behaviour as the
// reference CPU runtime (engine/include/leaf/runtime/decoder.h:15-50), so host
// code written against that header compiles against this one and links
// libleafhip instead of decoder.cpp.  Header-only: the only thing crossing into
// the library is the C ABI of leafhip.h.
//
//  * threads / force_scalar / worker_cpus are accepted and validated as the CPU
//    runtime validates them (thread count 1..64, host_support.h:119; CPU list
//    checks, worker_affinity.h) but the GPU grid replaces the thread pool.
//  * errors are std::runtime_error("Leaf decoder: ...") (decoder.cpp:86-88).
//  * forward_into resizes the caller's vector and writes into it; capacity is
//    reused (decoder.h:27-32).  The device argmax of the last row is kept and
//    available through last_argmax() (main_decoder.cpp:102 semantics).
#pragma once

#include <cstdint>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

#include "leafhip.h"

namespace leaf::runtime {

enum class FP32Math { Fast, Accurate };

class Decoder {
public:
    Decoder(const std::string& artifact, unsigned threads = 1, bool force_scalar = false,
            unsigned activation_bits = 32, const std::vector<unsigned>& worker_cpus = {},
            FP32Math fp32_math = FP32Math::Fast)
        : activation_bits_(activation_bits), accurate_(fp32_math == FP32Math::Accurate) {
        (void)force_scalar;
        if (threads < 1 || threads > 64) throw std::runtime_error("Leaf decoder: thread count must be 1..64");
        if (!worker_cpus.empty() && worker_cpus.size() != threads)
            throw std::runtime_error("Leaf decoder: worker CPU count must match thread count");
        for (std::size_t i = 0; i < worker_cpus.size(); ++i)
            for (std::size_t j = i + 1; j < worker_cpus.size(); ++j)
                if (worker_cpus[i] == worker_cpus[j]) throw std::runtime_error("Leaf decoder: duplicate worker CPU");
        int device = 0;
        if (const char* d = std::getenv("LEAF_HIP_DEVICE")) device = std::atoi(d);
        check(lh_context_create(device, &context_));
        try {
            check(lh_model_load_file(context_, artifact.c_str(), activation_bits, accurate_ ? 1u : 0u, &model_));
            lh_session_options options{0, 0};
            if (const char* c = std::getenv("LEAF_HIP_MAX_CONTEXT")) options.max_context = unsigned(std::atoi(c));
            check(lh_session_create(model_, &options, &session_));
            check(lh_model_get_info(model_, &info_));
            std::size_t count = 0;
            check(lh_model_eos_tokens(model_, nullptr, 0, &count));
            eos_.resize(count);
            if (count) check(lh_model_eos_tokens(model_, eos_.data(), eos_.size(), &count));
        } catch (...) {
            release();
            throw;
        }
    }
    ~Decoder() { release(); }
    Decoder(const Decoder&) = delete;
    Decoder& operator=(const Decoder&) = delete;

    void reset() { check(lh_reset(session_)); }

    std::vector<float> forward(const std::vector<std::uint32_t>& tokens, bool all_logits = false) {
        std::vector<float> logits;
        forward_into(tokens, logits, all_logits);
        return logits;
    }

    void forward_into(const std::vector<std::uint32_t>& tokens, std::vector<float>& logits, bool all_logits = false) {
        // Validation happens in the library before anything changes, so the
        // buffer is only resized for a call that will run.
        if (tokens.empty()) throw std::runtime_error("Leaf decoder: input tokens are empty");
        logits.resize((all_logits ? tokens.size() : 1) * std::size_t(info_.vocab));
        check(lh_forward(session_, tokens.data(), tokens.size(), all_logits ? 1 : 0, logits.data(), logits.size(),
                         &last_argmax_));
    }

    // Forward without copying logits to the host: only the device argmax of
    // the last row comes back (the greedy loop's need, main_decoder.cpp:95-113).
    std::uint32_t forward_argmax(const std::vector<std::uint32_t>& tokens) {
        check(lh_forward(session_, tokens.data(), tokens.size(), 0, nullptr, 0, &last_argmax_));
        return last_argmax_;
    }

    std::uint32_t last_argmax() const { return last_argmax_; }
    std::uint32_t vocabulary_size() const { return info_.vocab; }
    std::uint32_t eos_token() const { return info_.eos; }
    bool is_eos_token(std::uint32_t token) const {
        for (auto e : eos_)
            if (e == token) return true;
        return false;
    }
    std::size_t cache_tokens() const {
        std::size_t n = 0;
        check(lh_cache_tokens(session_, &n));
        return n;
    }
    std::uint64_t weight_bytes() const { return info_.artifact_bytes; }
    std::uint64_t device_weight_bytes() const { return info_.device_bytes; }
    // CPU-dispatch introspection of the reference (decoder.h:38-46).  None of
    // the AVX2 / VNNI / vector-SiLU CPU kernels run here.
    bool uses_avx2() const { return false; }
    bool uses_optimized_fp32() const { return false; }
    bool uses_accurate_fp32() const { return accurate_; }
    bool uses_vector_silu_gate() const { return false; }
    std::size_t silu_gate_vector_calls() const { return 0; }
    std::size_t source_bf16_tensors() const { return info_.source_bf16_tensors; }
    std::size_t source_bf16_linear_calls() const { return 0; }
    bool uses_vnni() const { return false; }
    unsigned activation_bits() const { return activation_bits_; }
    lh_session* session() const { return session_; }

private:
    static void check(lh_status status) {
        if (status != LH_OK) {
            const char* message = lh_last_error();
            throw std::runtime_error(message && *message ? message : "Leaf decoder: device call failed");
        }
    }
    void release() {
        if (session_) lh_session_destroy(session_);
        if (model_) lh_model_destroy(model_);
        if (context_) lh_context_destroy(context_);
        session_ = nullptr;
        model_ = nullptr;
        context_ = nullptr;
    }
    lh_context* context_ = nullptr;
    lh_model* model_ = nullptr;
    lh_session* session_ = nullptr;
    lh_model_info info_{};
    std::vector<std::uint32_t> eos_;
    std::uint32_t last_argmax_ = 0;
    unsigned activation_bits_ = 32;
    bool accurate_ = false;
};

}  // namespace leaf::runtime
