// Test-only harness around the reference Leaf decoder kernels.
//
// oracle/Makefile compiles this file together with the reference's own
// engine/src/decoder.cpp (included below by the path the Makefile passes in
// LEAF_REFERENCE_DECODER_CPP), with the reference's own flags
// (-std=c++17 -O3 -DNDEBUG -pthread, no -march: leaf/cli.py:66-67).
// Including the translation unit puts the anonymous-namespace kernels in scope,
// so the golden vectors come from the real reference arithmetic, not from a
// restatement.  The output goes to oracle/_ref/ only and is never shipped.
//
// Every wrapper below reproduces the dispatch of Decoder::Impl::linear
// (engine/src/decoder.cpp:994-1233) for one weight matrix, on the Linux build
// (LEAF_OPTIMIZED_FP32 == 0, decoder_config.h:69-78).
#include LEAF_REFERENCE_DECODER_CPP

#include <cstdint>
#include <cstdio>
#include <cstring>

using leaf::runtime::Weight;

namespace {
Weight make_weight(unsigned bits, std::size_t rows, std::size_t cols, std::size_t group,
                   const void* data, const float* scales) {
    Weight w;
    w.rows = rows; w.cols = cols; w.bits = bits;
    w.group = (bits == 8 || bits == 4) ? group : 0;
    w.data = static_cast<const std::uint8_t*>(data);
    w.scales = scales;
    return w;
}
bool have_avx() { return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"); }
bool have_vnni() {
#if LEAF_DECODER_VNNI
    return have_avx() && __builtin_cpu_supports("avxvnni");
#else
    return false;
#endif
}
}  // namespace

extern "C" {

// bit 0: AVX2+FMA dispatch active; bit 1: AVX-VNNI dispatch active.
int ref_cpu_features() { return (have_avx() ? 1 : 0) | (have_vnni() ? 2 : 0); }

// Per-token activation quantization exactly as decoder.cpp:1028-1043 (AVX2
// branch, quantize_input_avx :618-627).  q is int16 [M,K], scales [M].
void ref_quantize_rows(const float* x, std::size_t M, std::size_t K, std::int16_t* q, float* scales) {
    for (std::size_t t = 0; t < M; ++t) {
        const float* values = x + t * K;
        float maximum = 0;
        for (std::size_t col = 0; col < K; ++col) maximum = std::max(maximum, std::abs(values[col]));
        scales[t] = std::max(maximum / 127.0f, 1e-12f);
        leaf::runtime::quantize_input_avx(values, q + t * K, K, 1.0f / scales[t]);
    }
}

// W8A8 / W4A8 linear: decoder.cpp:1020-1044 then the integer dispatch
// :1183-1231.  mode 0 = what the reference would pick on this CPU,
// 1 = force quant_tile_avx + quant_dot_avx (no VNNI), 2 = force quant_dot_avx only.
int ref_linear_int(unsigned bits, std::size_t rows, std::size_t cols, std::size_t group,
                   const void* data, const float* scales, const float* bias,
                   const float* x, std::size_t M, int mode, float* out) {
    if (!have_avx()) return -1;
    Weight w = make_weight(bits, rows, cols, group, data, scales);
    std::vector<float> qs(M);
    const bool vnni = mode == 0 && have_vnni() && M > 1 && bits == 8 && group <= 65536;
    std::vector<std::int16_t> q16(M * cols);
#if LEAF_DECODER_VNNI
    std::vector<std::uint8_t> qb;
    if (vnni) {
        qb.resize(M * cols);
        for (std::size_t t = 0; t < M; ++t) {
            const float* values = x + t * cols;
            float maximum = 0;
            for (std::size_t col = 0; col < cols; ++col) maximum = std::max(maximum, std::abs(values[col]));
            qs[t] = std::max(maximum / 127.0f, 1e-12f);
            leaf::runtime::quantize_input_bytes(values, qb.data() + t * cols, cols, 1.0f / qs[t]);
        }
        leaf::runtime::prepare_signed_sums(w);
        constexpr std::size_t tile_rows = 2, tile_tokens = 4;
        float result[tile_rows * tile_tokens];
        for (std::size_t row = 0; row < rows; row += tile_rows) {
            const auto live = std::min(tile_rows, rows - row);
            for (std::size_t token = 0; token < M; token += tile_tokens) {
                const auto count = std::min(tile_tokens, M - token);
                leaf::runtime::quant_vnni_tile(w, row, live, qb.data() + token * cols, count, qs.data() + token, result);
                for (std::size_t r = 0; r < live; ++r)
                    for (std::size_t t = 0; t < count; ++t)
                        out[(token + t) * rows + row + r] = result[r * tile_tokens + t] + (bias ? bias[row + r] : 0);
            }
        }
        return 2;
    }
#endif
    ref_quantize_rows(x, M, cols, q16.data(), qs.data());
    std::size_t row = 0;
    if (mode != 2 && M > 1) {
        float result[8];
        for (; row + 4 <= rows; row += 4) {
            for (std::size_t token = 0; token < M; token += 2) {
                const auto count = std::min<std::size_t>(2, M - token);
                leaf::runtime::quant_tile_avx(w, row, q16.data() + token * cols, count, qs.data() + token, result);
                for (std::size_t r = 0; r < 4; ++r)
                    for (std::size_t t = 0; t < count; ++t)
                        out[(token + t) * rows + row + r] = result[r * 2 + t] + (bias ? bias[row + r] : 0);
            }
        }
    }
    float result[4];
    for (; row < rows; ++row) {
        for (std::size_t token = 0; token < M; token += 4) {
            const auto count = std::min<std::size_t>(4, M - token);
            leaf::runtime::quant_dot_avx(w, row, q16.data() + token * cols, count, qs.data() + token, result);
            for (std::size_t t = 0; t < count; ++t)
                out[(token + t) * rows + row] = result[t] + (bias ? bias[row] : 0);
        }
    }
    return 1;
}

// FP32 / BF16-source / weight-only INT8 and INT4 linear: decoder.cpp:1146-1231
// with dot = dot_avx (:355-391) and BF16 through dot_source_bf16_avx (:392-420).
int ref_linear_fp(unsigned bits, std::size_t rows, std::size_t cols, std::size_t group,
                  const void* data, const float* scales, const float* bias,
                  const float* x, std::size_t M, float* out) {
    if (!have_avx()) return -1;
    Weight w = make_weight(bits, rows, cols, group, data, scales);
    float result[4];
    for (std::size_t row = 0; row < rows; ++row) {
        for (std::size_t token = 0; token < M; token += 4) {
            const auto count = std::min<std::size_t>(4, M - token);
            if (bits == 16) leaf::runtime::dot_source_bf16_avx(w, row, x + token * cols, count, result);
            else leaf::runtime::dot_avx(w, row, x + token * cols, count, result);
            for (std::size_t t = 0; t < count; ++t)
                out[(token + t) * rows + row] = result[t] + (bias ? bias[row] : 0.0f);
        }
    }
    return 0;
}

// Accurate-mode FP32/BF16 prefill GEMM (tokens >= 8): decoder.cpp:1045-1145,
// accurate_fp32.h:140-166 via token-panel packing (token_panel.h:58-105).
int ref_linear_accurate(unsigned bits, std::size_t rows, std::size_t cols,
                        const void* data, const float* bias, const float* x, std::size_t M, float* out) {
    if (!have_avx()) return -1;
    leaf::kernels::TokenPanelsF32 panels;
    panels.pack(x, M, cols, cols, false);
    std::vector<float> expanded;
    for (std::size_t begin = 0; begin < rows; begin += 6) {
        const auto live = std::min<std::size_t>(6, rows - begin);
        const float* panel_weights;
        if (bits == 16) {
            expanded.resize(live * cols);
            leaf::kernels::expand_source_bf16(static_cast<const std::uint16_t*>(data) + begin * cols,
                                              expanded.data(), live * cols, true);
            panel_weights = expanded.data();
        } else {
            panel_weights = static_cast<const float*>(data) + begin * cols;
        }
        leaf::kernels::gemm_token_panels_f32_accurate(panel_weights, live, cols, cols, panels,
                                                      out + begin, rows, bias ? bias + begin : nullptr, true);
    }
    return 0;
}

// RMSNorm / LayerNorm exactly as norm() (decoder.cpp:706-727).
void ref_norm(const float* x, std::size_t M, std::size_t width, const float* gamma, const float* beta,
              float epsilon, unsigned kind, int accurate, float* out) {
    std::vector<float> input(x, x + M * width), output;
    Weight g = make_weight(32, 1, width, 0, gamma, nullptr);
    Weight b = make_weight(32, 1, width, 0, beta, nullptr);
    leaf::runtime::norm(input, g, beta ? &b : nullptr, epsilon, kind, output, width, accurate != 0);
    std::memcpy(out, output.data(), M * width * sizeof(float));
}

// The real Decoder's greedy continuation, as generate_continuation runs it
// (engine/src/main_decoder.cpp:95-113): forward_into(prompt) without
// all-token logits, the first maximal index, then one forward per token, up
// to `limit` tokens or an EOS token.  Writes the tokens and, for each forward
// index listed in `keep` (0 = the prompt, i = the i-th single-token step), its
// logits into logits[k * vocab].  Returns the number of tokens, or -1 with the
// error text.
int ref_decoder_greedy(const char* artifact, unsigned threads, unsigned activation_bits, int accurate,
                       const std::uint32_t* prompt, std::size_t count, unsigned limit, std::uint32_t* tokens,
                       const unsigned* keep, std::size_t keep_count, float* logits, char* error,
                       std::size_t error_size) {
    try {
        leaf::runtime::Decoder decoder(artifact, threads, false, activation_bits, {},
                                       accurate ? leaf::runtime::FP32Math::Accurate : leaf::runtime::FP32Math::Fast);
        const std::size_t vocab = decoder.vocabulary_size();
        std::vector<float> out;
        std::vector<std::uint32_t> ids(prompt, prompt + count);
        auto record = [&](unsigned forward) {
            for (std::size_t k = 0; k < keep_count; ++k)
                if (keep[k] == forward) std::memcpy(logits + k * vocab, out.data(), vocab * sizeof(float));
        };
        decoder.forward_into(ids, out);
        record(0);
        int produced = 0;
        for (unsigned token = 0; token < limit; ++token) {
            const auto id = static_cast<std::uint32_t>(std::max_element(out.begin(), out.end()) - out.begin());
            tokens[produced++] = id;
            if (decoder.is_eos_token(id)) break;
            if (token + 1 < limit) {
                decoder.forward_into({id}, out);
                record(token + 1);
            }
        }
        return produced;
    } catch (const std::exception& e) {
        std::snprintf(error, error_size, "%s", e.what());
        return -1;
    }
}

}  // extern "C"
