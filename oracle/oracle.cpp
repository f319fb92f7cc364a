// CPU oracle for Leaf's decoder hot path.  TEST INFRASTRUCTURE ONLY: loaded
// by tests/, the smoke check and bench.py's CPU-baseline leg as the checker.
//
// Restates the reference Linux dispatch (engine/src/decoder.cpp with
// LEAF_OPTIMIZED_FP32 == 0 and AVX2+FMA present; decoder_config.h:55-88) in
// plain scalar C++.  Vector lanes of the reference are spelled as arrays of
// eight floats, its fused multiply-adds as fmaf(), and everything else as
// separately rounded operations (this file is built with -ffp-contract=off).
// libm calls (expf, sinf, cosf, powf, erff, tanhf) are the same glibc calls
// the reference makes, so on one machine they return the same bits.
//
// Pinning, per function (tests/test_oracle_golden.py runs every check):
//  * oracle_quantize_rows, oracle_linear_int(_q): bit-exact against golden
//    vectors written by the real quantize_input_avx / quant_dot_avx /
//    quant_tile_avx / quant_vnni_tile (tests/golden/make_golden.py); int32
//    accumulators are exact integer sums (closed form, brute-force checked).
//  * oracle_linear_fp / oracle_linear_accurate: bit-exact against golden
//    vectors of dot_avx, dot_source_bf16_avx and the accurate token-panel
//    GEMM; plus the FP64 bound 2e-5(1+|e|) of tests/native/test_decode_gemv.cpp:36-42.
//  * oracle_norm: bit-exact against the real norm() (decoder.cpp:706-727).
//  * oracle_attention, oracle_rope_*, oracle_activate, the decoder: bit-exact
//    logits and identical greedy tokens against the real leaf_decoder binary
//    (verify / generate modes) on reduced synthetic models of all families;
//    GQA-by-index equals materialized repeat (tests/native/test_kernels.cpp:253-327).
//  * oracle_quantize_weights: equals the numpy exporter restatement
//    (tools/export_decoder.py:91-105) and the zero-row/both-signs example of
//    tests/unit/test_decoder_plan.py:83-96.
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace {

// ---------------------------------------------------------------- weights --
struct Matrix {
    size_t rows = 0, cols = 0, bits = 0, group = 0;
    const uint8_t* data = nullptr;
    const float* scales = nullptr;

    // Weight::value (decoder.cpp:236-251)
    float value(size_t row, size_t col) const {
        const size_t index = row * cols + col;
        if (bits == 32) return reinterpret_cast<const float*>(data)[index];
        if (bits == 16) {
            const uint32_t b = uint32_t(reinterpret_cast<const uint16_t*>(data)[index]) << 16;
            float f; std::memcpy(&f, &b, 4); return f;
        }
        return float(qvalue(index)) * scales[row * (cols / group) + col / group];
    }
    // Stored integer at a flat index (bits 8: int8; bits 4: low nibble = even column).
    int qvalue(size_t index) const {
        if (bits == 8) return reinterpret_cast<const int8_t*>(data)[index];
        int v = (data[index / 2] >> ((index % 2) * 4)) & 15;
        return v >= 8 ? v - 16 : v;
    }
    // The unscaled lane value the vector kernels load (weight8, decoder.cpp:299-320).
    float lane(size_t row, size_t col) const {
        const size_t index = row * cols + col;
        if (bits == 32) return reinterpret_cast<const float*>(data)[index];
        return float(qvalue(index));
    }
};

Matrix make_matrix(unsigned bits, size_t rows, size_t cols, size_t group, const void* data, const float* scales) {
    Matrix m;
    m.rows = rows; m.cols = cols; m.bits = bits;
    m.group = (bits == 8 || bits == 4) ? group : 0;
    m.data = static_cast<const uint8_t*>(data);
    m.scales = scales;
    return m;
}

// Horizontal sum of eight lanes in the reference's order (decoder.cpp:294-298):
// (l0+l4, l1+l5, l2+l6, l3+l7) -> (p0 = h0+h2, p1 = h1+h3) -> p0 + p1.
inline float reduce8(const float* v) {
    const float h0 = v[0] + v[4], h1 = v[1] + v[5], h2 = v[2] + v[6], h3 = v[3] + v[7];
    const float p0 = h0 + h2, p1 = h1 + h3;
    return p0 + p1;
}

// ------------------------------------------------------------- R5: FP dot --
// dot_avx (decoder.cpp:355-391) for bits 32/8/4, tokens 1..4.  Scalar tails and
// the per-group scale use the fused form the reference build emits
// (GCC contracts `a += b * c` inside its avx2,fma target functions).
void dot_fp(const Matrix& w, size_t row, const float* x, size_t tokens, float* result) {
    for (size_t t = 0; t < tokens; ++t) result[t] = 0.0f;
    const size_t group = w.bits == 32 ? w.cols : w.group;
    const size_t groups = w.cols / group;
    for (size_t g = 0; g < groups; ++g) {
        float acc[4][8] = {};
        size_t col = g * group;
        const size_t end = col + group;
        if (tokens == 1) {
            float b[8] = {}, c[8] = {}, d[8] = {};
            for (; col + 32 <= end; col += 32)
                for (int l = 0; l < 8; ++l) {
                    acc[0][l] = std::fmaf(w.lane(row, col + l), x[col + l], acc[0][l]);
                    b[l] = std::fmaf(w.lane(row, col + 8 + l), x[col + 8 + l], b[l]);
                    c[l] = std::fmaf(w.lane(row, col + 16 + l), x[col + 16 + l], c[l]);
                    d[l] = std::fmaf(w.lane(row, col + 24 + l), x[col + 24 + l], d[l]);
                }
            for (int l = 0; l < 8; ++l) acc[0][l] = (acc[0][l] + b[l]) + (c[l] + d[l]);
        }
        for (; col + 8 <= end; col += 8)
            for (size_t t = 0; t < tokens; ++t)
                for (int l = 0; l < 8; ++l)
                    acc[t][l] = std::fmaf(w.lane(row, col + l), x[t * w.cols + col + l], acc[t][l]);
        float partial[4];
        for (size_t t = 0; t < 4; ++t) partial[t] = reduce8(acc[t]);
        const float scale = w.bits == 32 ? 1.0f : w.scales[row * groups + g];
        for (; col < end; ++col) {
            const float value = w.value(row, col) / scale;
            for (size_t t = 0; t < tokens; ++t) partial[t] = std::fmaf(value, x[t * w.cols + col], partial[t]);
        }
        for (size_t t = 0; t < tokens; ++t) result[t] = std::fmaf(partial[t], scale, result[t]);
    }
}

// dot_source_bf16_avx (decoder.cpp:392-420): one group over the whole row.
void dot_bf16(const Matrix& w, size_t row, const float* x, size_t tokens, float* result) {
    float acc[4][8] = {};
    size_t col = 0;
    if (tokens == 1) {
        float b[8] = {}, c[8] = {}, d[8] = {};
        for (; col + 32 <= w.cols; col += 32)
            for (int l = 0; l < 8; ++l) {
                acc[0][l] = std::fmaf(w.value(row, col + l), x[col + l], acc[0][l]);
                b[l] = std::fmaf(w.value(row, col + 8 + l), x[col + 8 + l], b[l]);
                c[l] = std::fmaf(w.value(row, col + 16 + l), x[col + 16 + l], c[l]);
                d[l] = std::fmaf(w.value(row, col + 24 + l), x[col + 24 + l], d[l]);
            }
        for (int l = 0; l < 8; ++l) acc[0][l] = (acc[0][l] + b[l]) + (c[l] + d[l]);
    }
    for (; col + 8 <= w.cols; col += 8)
        for (size_t t = 0; t < tokens; ++t)
            for (int l = 0; l < 8; ++l)
                acc[t][l] = std::fmaf(w.value(row, col + l), x[t * w.cols + col + l], acc[t][l]);
    float partial[4];
    for (size_t t = 0; t < 4; ++t) partial[t] = reduce8(acc[t]);
    for (; col < w.cols; ++col) {
        const float value = w.value(row, col);
        for (size_t t = 0; t < tokens; ++t) partial[t] = std::fmaf(value, x[t * w.cols + col], partial[t]);
    }
    for (size_t t = 0; t < tokens; ++t) result[t] = 0.0f + partial[t];
}

// ---------------------------------------------------- R2-R4: W8A8 / W4A8 --
// Per-token quantization (decoder.cpp:1028-1043 with quantize_input_avx :618-627):
// s = max(max|x| / 127, 1e-12); q = round-half-even(x * (1/s)), within +-127.
void quantize_rows(const float* x, size_t M, size_t K, int8_t* q, float* scales) {
    for (size_t t = 0; t < M; ++t) {
        const float* v = x + t * K;
        float maximum = 0;
        for (size_t c = 0; c < K; ++c) maximum = std::max(maximum, std::fabs(v[c]));
        scales[t] = std::max(maximum / 127.0f, 1e-12f);
        const float multiplier = 1.0f / scales[t];
        for (size_t c = 0; c < K; ++c) {
            const float r = std::nearbyint(v[c] * multiplier);
            q[t * K + c] = static_cast<int8_t>(std::max(-127.0f, std::min(127.0f, r)));
        }
    }
}

// quant_dot_avx / quant_tile_avx / quant_vnni_tile (decoder.cpp:536-702): exact
// int32 per group, then res += ((float)acc * s_x) * s_w[row, g].  quant_dot_avx
// and quant_tile_avx are avx2,fma target functions, so the reference build
// fuses that accumulate; quant_vnni_tile's target (avx2,avxvnni) has no FMA and
// rounds the product first.  With one group per row both forms agree
// (fma(a, b, 0) == a * b); with several groups they differ, which makes the
// reference's grouped W8A8 prefill depend on whether its host has AVX-VNNI.
// `vnni` selects the unfused form.
void quant_row(const Matrix& w, size_t row, const int8_t* q, const float* qscale, size_t tokens, float* result,
               bool vnni = false) {
    const size_t groups = w.cols / w.group;
    for (size_t t = 0; t < tokens; ++t) result[t] = 0.0f;
    for (size_t g = 0; g < groups; ++g) {
        const float sw = w.scales[row * groups + g];
        for (size_t t = 0; t < tokens; ++t) {
            int32_t acc = 0;
            for (size_t c = g * w.group; c < (g + 1) * w.group; ++c)
                acc += w.qvalue(row * w.cols + c) * int32_t(q[t * w.cols + c]);
            const float term = float(acc) * qscale[t];
            result[t] = vnni ? result[t] + term * sw : std::fmaf(term, sw, result[t]);
        }
    }
}

// ------------------------------------------------ R7: accurate FP32 GEMM --
// gemm_token_panels_f32_accurate with AVX2 (accurate_fp32.h:18-84): per output,
// sequential fused sums over 256-column K blocks, combined by binary carries.
float accurate_dot(const Matrix& w, size_t row, const float* x) {
    float levels[64];
    float part = 0.0f;
    size_t blocks = 0;
    unsigned depth = 0;
    for (size_t first = 0; first < w.cols;) {
        const size_t width = std::min<size_t>(256, w.cols - first);
        part = 0.0f;
        for (size_t c = first; c < first + width; ++c) part = std::fmaf(w.value(row, c), x[c], part);
        size_t occupied = blocks;
        unsigned level = 0;
        for (; occupied & 1; occupied >>= 1, ++level) part = levels[level] + part;
        levels[level] = part;
        depth = std::max(depth, level + 1);
        ++blocks;
        first += width;
    }
    bool initialized = false;
    for (unsigned level = depth; level-- > 0;) {
        if (!(blocks & (size_t(1) << level))) continue;
        float value = levels[level];
        if (initialized) value = part + value;
        part = value;
        initialized = true;
    }
    return part;
}

// ------------------------------------------------------------------ R9 -----
// 0: the reference's sequential square sum; 1: pairwise (tree) sums, the order
// a parallel reduction uses.  The second exists only to measure how far W8A8
// logits move when nothing but the summation order changes.
int g_norm_order = 0;

float square_sum(const float* in, size_t width, float mean) {
    float square = 0;
    if (g_norm_order == 0) {
        for (size_t c = 0; c < width; ++c) { const float v = in[c] - mean; square += v * v; }
        return square;
    }
    std::vector<float> t(width);
    for (size_t c = 0; c < width; ++c) { const float v = in[c] - mean; t[c] = v * v; }
    for (size_t n = width; n > 1;) {
        const size_t half = (n + 1) / 2;
        for (size_t i = 0; i + half < n; ++i) t[i] = t[i] + t[i + half];
        n = half;
    }
    return width ? t[0] : 0.0f;
}

void norm_rows(const float* x, size_t M, size_t width, const float* gamma, const float* beta,
               float epsilon, unsigned kind, bool accurate, float* y) {
    for (size_t r = 0; r < M; ++r) {
        const float* in = x + r * width;
        float* out = y + r * width;
        float mean = 0, square = 0;
        if (kind == 1) {
            for (size_t c = 0; c < width; ++c) mean += in[c];
            mean /= static_cast<float>(width);
        }
        if (kind == 0 && accurate) {
            // accurate_rms_square_sum (accurate_fp32.h:6-13)
            double total = 0.0;
            for (size_t c = 0; c < width; ++c) { const float s = in[c] * in[c]; total += s; }
            square = static_cast<float>(total);
        } else {
            square = square_sum(in, width, mean);
        }
        const float scale = 1.0f / std::sqrt(square / static_cast<float>(width) + epsilon);
        for (size_t c = 0; c < width; ++c) {
            const float v = in[c] - mean;
            out[c] = v * scale * gamma[c] + (beta ? beta[c] : 0.0f);
        }
    }
}

// ----------------------------------------------------------------- R11 -----
// attention_impl with the scalar dot of the portable build (transformer.cpp:69-146).
void attention(const float* q, const float* keys, const float* values, const float* mask, float* out,
               size_t heads, size_t kv_heads, size_t tokens, size_t total, size_t stride, size_t dim,
               float scale) {
    std::vector<float> scores(total);
    for (size_t h = 0; h < heads; ++h) {
        const size_t kvh = h / (heads / kv_heads);
        for (size_t t = 0; t < tokens; ++t) {
            const float* qrow = q + (h * tokens + t) * dim;
            float* orow = out + (t * heads + h) * dim;
            std::fill(orow, orow + dim, 0.0f);
            float maximum = -std::numeric_limits<float>::infinity();
            for (size_t k = 0; k < total; ++k) {
                if (mask[t * total + k] == 0.0f) {
                    scores[k] = -std::numeric_limits<float>::infinity();
                } else {
                    const float* krow = keys + (kvh * stride + k) * dim;
                    float sum = 0.0f;
                    for (size_t d = 0; d < dim; ++d) sum += qrow[d] * krow[d];
                    scores[k] = sum * scale * scale;
                    maximum = std::max(maximum, scores[k]);
                }
            }
            if (!std::isfinite(maximum)) continue;
            float denominator = 0.0f;
            for (size_t k = 0; k < total; ++k) {
                scores[k] = std::exp(scores[k] - maximum);
                denominator += scores[k];
            }
            for (size_t k = 0; k < total; ++k) {
                const float p = scores[k] / denominator;
                const float* vrow = values + (kvh * stride + k) * dim;
                for (size_t d = 0; d < dim; ++d) orow[d] += p * vrow[d];
            }
        }
    }
}

// ----------------------------------------------------------------- R12 -----
// Decoder::Impl::activate (decoder.cpp:982-987)
float activate(unsigned activation, float x) {
    if (activation == 0) return x / (1.0f + std::exp(-x));
    if (activation == 1) return 0.5f * x * (1.0f + std::erf(x * 0.7071067811865475f));
    if (activation == 2) return 0.5f * x * (1.0f + std::tanh(0.7978845608028654f * (x + 0.044715f * x * x * x)));
    return std::max(x, 0.0f);
}

// --------------------------------------------------------- linear (R6) -----
enum class Path { Fp, Bf16, Int, Accurate };

// Which integer epilogue the reference would run for a W8A8 call with these
// shapes: its VNNI tile serves INT8 prefill (tokens > 1) when the host has
// AVX-VNNI (decoder.cpp:782, 1022); -1 asks this CPU, 0/1 force it.
int g_vnni_policy = 0;
bool vnni_epilogue(const Matrix& w, size_t M) {
    bool host = false;
    if (g_vnni_policy < 0) host = __builtin_cpu_supports("avxvnni");
    else host = g_vnni_policy != 0;
    return host && M > 1 && w.bits == 8 && w.group <= 65536;
}

void linear_rows(const Matrix& w, const float* bias, const float* x, size_t M, Path path, float* y,
                 const int8_t* q = nullptr, const float* qscale = nullptr) {
    const bool vnni = path == Path::Int && vnni_epilogue(w, M);
    if (path == Path::Accurate) {
#pragma omp parallel for schedule(static)
        for (long r = 0; r < long(w.rows); ++r)
            for (size_t t = 0; t < M; ++t)
                y[t * w.rows + r] = accurate_dot(w, r, x + t * w.cols) + (bias ? bias[r] : 0.0f);
        return;
    }
#pragma omp parallel for schedule(static)
    for (long r = 0; r < long(w.rows); ++r) {
        float result[4];
        for (size_t token = 0; token < M; token += 4) {
            const size_t count = std::min<size_t>(4, M - token);
            if (path == Path::Int) quant_row(w, r, q + token * w.cols, qscale + token, count, result, vnni);
            else if (path == Path::Bf16) dot_bf16(w, r, x + token * w.cols, count, result);
            else dot_fp(w, r, x + token * w.cols, count, result);
            for (size_t t = 0; t < count; ++t)
                y[(token + t) * w.rows + r] = result[t] + (bias ? bias[r] : 0.0f);
        }
    }
}

// ------------------------------------------------------------- decoder -----
struct Fail : std::runtime_error { using std::runtime_error::runtime_error; };
void check(bool ok, const std::string& message) { if (!ok) throw Fail("Leaf decoder: " + message); }

struct Cache {
    size_t kv_heads, dim, length = 0, capacity = 0;
    std::vector<float> keys, values;
    void append(const float* k, const float* v, size_t n) {
        const size_t need = length + n;
        if (need > capacity) {
            size_t next = std::max<size_t>(8, capacity);
            while (next < need) next *= 2;
            std::vector<float> nk(kv_heads * next * dim), nv(nk.size());
            for (size_t p = 0; p < kv_heads; ++p) {
                std::copy_n(keys.data() + p * capacity * dim, length * dim, nk.data() + p * next * dim);
                std::copy_n(values.data() + p * capacity * dim, length * dim, nv.data() + p * next * dim);
            }
            keys.swap(nk); values.swap(nv); capacity = next;
        }
        for (size_t p = 0; p < kv_heads; ++p) {
            std::copy_n(k + p * n * dim, n * dim, keys.data() + (p * capacity + length) * dim);
            std::copy_n(v + p * n * dim, n * dim, values.data() + (p * capacity + length) * dim);
        }
        length = need;
    }
};

}  // namespace

struct oracle_decoder {
    const uint8_t* map = nullptr;
    size_t size = 0;
    unsigned h, f, heads, kv_heads, layers, vocab, max_positions, eos, dim, window;
    float theta, epsilon, embedding_scale;
    unsigned norm_kind, activation, position_kind, gated, parallel, rotary_dim, position_offset, final_norm;
    unsigned qk_norm = 0, activation_bits = 32;
    bool accurate = false, fp32_artifact = false;
    std::vector<uint32_t> eos_tokens;
    std::map<std::string, Matrix> tensors;
    std::vector<float> freq, cosines, sines;
    std::vector<Cache> caches;

    ~oracle_decoder() { if (map) munmap(const_cast<uint8_t*>(map), size); }

    const Matrix& at(const std::string& name) const {
        auto it = tensors.find(name);
        check(it != tensors.end(), "missing tensor " + name);
        return it->second;
    }
    const Matrix* find(const std::string& name) const {
        auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }

    void open(const char* path) {
        const int fd = ::open(path, O_RDONLY);
        check(fd >= 0, std::string("cannot open artifact ") + path);
        struct stat st;
        if (fstat(fd, &st) || st.st_size <= 0) { ::close(fd); check(false, "invalid decoder artifact size"); }
        size = size_t(st.st_size);
        void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        check(m != MAP_FAILED, "cannot map decoder artifact");
        map = static_cast<const uint8_t*>(m);
        size_t pos = 0;
        auto need = [&](size_t n) { check(pos <= size && n <= size - pos, "truncated artifact metadata"); };
        auto u32 = [&]() { need(4); uint32_t v; std::memcpy(&v, map + pos, 4); pos += 4; return v; };
        auto u64 = [&]() { const uint64_t lo = u32(); return lo | (uint64_t(u32()) << 32); };
        auto f32 = [&]() { const uint32_t b = u32(); float v; std::memcpy(&v, &b, 4); return v; };
        need(8);
        const std::string magic(reinterpret_cast<const char*>(map), 8);
        check(magic.compare(0, 7, "LEAFDC0") == 0 && magic[7] >= '2' && magic[7] <= '7', "unsupported artifact magic");
        const unsigned version = unsigned(magic[7] - '0');
        pos = 8;
        check(u32() == version, "unsupported decoder artifact version");
        const uint32_t count = u32();
        const uint64_t base = u64();
        h = u32(); f = u32(); heads = u32(); kv_heads = u32(); layers = u32(); vocab = u32();
        max_positions = u32(); eos = u32(); dim = u32(); window = u32();
        theta = f32(); epsilon = f32();
        norm_kind = u32(); activation = u32(); position_kind = u32(); gated = u32(); parallel = u32();
        rotary_dim = u32(); position_offset = u32(); final_norm = u32(); embedding_scale = f32();
        check(h && f && heads && kv_heads && layers && vocab && dim && max_positions && heads % kv_heads == 0,
              "invalid decoder configuration");
        if (version == 7) {
            const uint32_t storage = u32(); qk_norm = u32(); const uint32_t n = u32();
            (void)storage;
            for (uint32_t i = 0; i < n; ++i) freq.push_back(f32());
        }
        if (version >= 4) {
            const uint32_t n = u32();
            for (uint32_t i = 0; i < n; ++i) eos_tokens.push_back(u32());
        } else if (eos < vocab) {
            eos_tokens.push_back(eos);
        }
        for (uint32_t i = 0; i < count; ++i) {
            const uint32_t length = u32();
            need(length);
            std::string name(reinterpret_cast<const char*>(map + pos), length);
            pos += length;
            const uint32_t rank = u32();
            Matrix w;
            w.rows = u32(); w.cols = u32(); w.bits = u32(); w.group = u32();
            const uint64_t offset = u64(), bytes = u64(), scale_offset = u64(), scale_count = u64();
            check(rank == 2 && offset % 64 == 0 && base + offset + bytes <= size, "invalid tensor " + name);
            w.data = map + base + offset;
            if (w.bits == 8 || w.bits == 4) {
                check(base + scale_offset + scale_count * 4 <= size, "invalid quantization metadata " + name);
                w.scales = reinterpret_cast<const float*>(map + base + scale_offset);
            } else {
                w.group = 0;
            }
            tensors[name] = w;
        }
        if (position_kind == 0 && freq.empty()) {
            freq.resize(rotary_dim / 2);
            oracle_rope_frequencies(theta, rotary_dim, freq.data());
        }
        for (unsigned l = 0; l < layers; ++l) caches.push_back(Cache{kv_heads, dim});
        fp32_artifact = activation_bits == 32;
        for (auto& item : tensors) fp32_artifact = fp32_artifact && (item.second.bits == 32 || item.second.bits == 16);
        check(!accurate || fp32_artifact, "accurate FP32 math requires FP32 compute and unquantized weights");
    }

    // Decoder::Impl::linear (decoder.cpp:994-1233), Linux dispatch.
    void linear(const float* input, size_t tokens, const std::string& name, std::vector<float>& out) {
        const Matrix& w = at(name + ".weight");
        const Matrix* b = find(name + ".bias");
        const float* bias = b ? reinterpret_cast<const float*>(b->data) : nullptr;
        std::vector<float> transformed;
        if (const Matrix* s = find(name + ".input_scale")) {
            const float* factors = reinterpret_cast<const float*>(s->data);
            transformed.resize(tokens * w.cols);
            for (size_t t = 0; t < tokens; ++t)
                for (size_t c = 0; c < w.cols; ++c)
                    transformed[t * w.cols + c] = input[t * w.cols + c] * factors[c];
            input = transformed.data();
        }
        out.assign(tokens * w.rows, 0.0f);
        const bool integer = (w.bits == 4 || w.bits == 8) && activation_bits == 8;
        if (integer) {
            std::vector<int8_t> q(tokens * w.cols);
            std::vector<float> qs(tokens);
            quantize_rows(input, tokens, w.cols, q.data(), qs.data());
            linear_rows(w, bias, input, tokens, Path::Int, out.data(), q.data(), qs.data());
            return;
        }
        const bool packed = accurate && (w.bits == 32 || w.bits == 16) && tokens >= 8 && (!b || b->bits == 32);
        const Path path = packed ? Path::Accurate : w.bits == 16 ? Path::Bf16 : Path::Fp;
        linear_rows(w, bias, input, tokens, path, out.data());
    }

    void normalize(const std::vector<float>& in, const std::string& name, std::vector<float>& out) {
        const Matrix& g = at(name + ".weight");
        const Matrix* b = find(name + ".bias");
        out.resize(in.size());
        norm_rows(in.data(), in.size() / h, h, reinterpret_cast<const float*>(g.data),
                  b ? reinterpret_cast<const float*>(b->data) : nullptr, epsilon, norm_kind, accurate, out.data());
    }

    // rotary() (decoder.cpp:1259-1281): [tokens, n, dim] -> [n, tokens, dim] plus rotate-half.
    void rotary(const std::vector<float>& values, std::vector<float>& out, size_t n, size_t tokens) {
        out.resize(values.size());
        const size_t half = rotary_dim / 2;
        for (size_t t = 0; t < tokens; ++t)
            for (size_t hd = 0; hd < n; ++hd) {
                for (size_t i = 0; i < dim; ++i) out[(hd * tokens + t) * dim + i] = values[(t * n + hd) * dim + i];
                if (position_kind != 0) continue;
                for (size_t i = 0; i < half; ++i) {
                    const float c = cosines[t * half + i], s = sines[t * half + i];
                    const size_t from = (t * n + hd) * dim + i, to = (hd * tokens + t) * dim + i;
                    const float a = values[from], b = values[from + half];
                    out[to] = a * c - b * s;
                    out[to + half] = b * c + a * s;
                }
            }
    }

    // Decoder::Impl::forward_into (decoder.cpp:1282-1444).
    void forward(const std::vector<uint32_t>& ids, bool all_logits, std::vector<float>& logits) {
        check(!ids.empty(), "input tokens are empty");
        const size_t tokens = ids.size(), position = caches[0].length;
        check(position <= max_positions && tokens <= max_positions - position, "context length exceeds artifact limit");
        for (auto id : ids) check(id < vocab, "token id exceeds vocabulary");
        if (position_kind == 0) {
            const size_t half = rotary_dim / 2;
            cosines.resize(tokens * half); sines.resize(tokens * half);
            oracle_rope_tables(freq.data(), rotary_dim, position, tokens, cosines.data(), sines.data());
        }
        std::vector<float> hidden(tokens * h), normalized, q, k, v, qh, kh, vh, att, attn_proj, up, gate, proj;
        const Matrix& embedding = at("model.embed_tokens.weight");
        const Matrix* positions = position_kind == 1 ? &at("model.position_embeddings.weight") : nullptr;
        for (size_t t = 0; t < tokens; ++t)
            for (size_t c = 0; c < h; ++c) {
                hidden[t * h + c] = embedding.value(ids[t], c) * embedding_scale;
                if (positions) hidden[t * h + c] += positions->value(position + t + position_offset, c);
            }
        const size_t total = position + tokens;
        std::vector<float> mask(tokens * total, 0.0f);
        for (size_t t = 0; t < tokens; ++t) {
            const size_t end = position + t + 1;
            const size_t begin = window && end > window ? end - window : 0;
            std::fill_n(mask.data() + t * total + begin, end - begin, 1.0f);
        }
        const float scale = 1.0f / std::sqrt(std::sqrt(static_cast<float>(dim)));
        for (size_t layer = 0; layer < layers; ++layer) {
            const std::string p = "model.layers." + std::to_string(layer) + ".";
            normalize(hidden, p + "input_layernorm", normalized);
            linear(normalized.data(), tokens, p + "self_attn.q_proj", q);
            linear(normalized.data(), tokens, p + "self_attn.k_proj", k);
            linear(normalized.data(), tokens, p + "self_attn.v_proj", v);
            if (qk_norm) {
                std::vector<float> tmp(q.size());
                norm_rows(q.data(), q.size() / dim, dim, reinterpret_cast<const float*>(at(p + "self_attn.q_norm.weight").data),
                          nullptr, epsilon, 0, accurate, tmp.data());
                q.swap(tmp);
                tmp.resize(k.size());
                norm_rows(k.data(), k.size() / dim, dim, reinterpret_cast<const float*>(at(p + "self_attn.k_norm.weight").data),
                          nullptr, epsilon, 0, accurate, tmp.data());
                k.swap(tmp);
            }
            rotary(q, qh, heads, tokens);
            rotary(k, kh, kv_heads, tokens);
            vh.resize(v.size());
            for (size_t hd = 0; hd < kv_heads; ++hd)
                for (size_t t = 0; t < tokens; ++t)
                    std::copy_n(v.data() + (t * kv_heads + hd) * dim, dim, vh.data() + (hd * tokens + t) * dim);
            Cache& cache = caches[layer];
            cache.append(kh.data(), vh.data(), tokens);
            att.assign(tokens * heads * dim, 0.0f);
            attention(qh.data(), cache.keys.data(), cache.values.data(), mask.data(), att.data(), heads, kv_heads,
                      tokens, cache.length, cache.capacity, dim, scale);
            linear(att.data(), tokens, p + "self_attn.o_proj", attn_proj);
            size_t mlp_tokens = tokens;
            if (layer + 1 == layers && !all_logits && fp32_artifact && tokens >= 32) {
                // Only the last row reaches the head; keep 16..31 trailing rows
                // (decoder.cpp:1375-1387), which fixes the 4-token grouping.
                const size_t first = ((tokens - 16) / 16) * 16;
                hidden.erase(hidden.begin(), hidden.begin() + first * h);
                attn_proj.erase(attn_proj.begin(), attn_proj.begin() + first * h);
                mlp_tokens -= first;
            }
            if (!parallel)
                for (size_t j = 0; j < hidden.size(); ++j) hidden[j] += attn_proj[j];
            normalize(hidden, p + "post_attention_layernorm", normalized);
            linear(normalized.data(), mlp_tokens, p + "mlp.up_proj", up);
            if (gated) {
                linear(normalized.data(), mlp_tokens, p + "mlp.gate_proj", gate);
                for (size_t j = 0; j < gate.size(); ++j) up[j] *= activate(activation, gate[j]);
            } else {
                for (auto& value : up) value = activate(activation, value);
            }
            linear(up.data(), mlp_tokens, p + "mlp.down_proj", proj);
            for (size_t j = 0; j < hidden.size(); ++j) hidden[j] += proj[j] + (parallel ? attn_proj[j] : 0.0f);
        }
        if (final_norm) normalize(hidden, "model.norm", normalized);
        else normalized = hidden;
        linear(normalized.data() + (all_logits ? 0 : normalized.size() - h), all_logits ? tokens : 1, "lm_head", logits);
    }
};

extern "C" {

void oracle_set_vnni_policy(int policy) { g_vnni_policy = policy; }
void oracle_set_norm_order(int order) { g_norm_order = order; }

void oracle_quantize_rows(const float* x, size_t M, size_t K, int8_t* q, float* scales) {
    quantize_rows(x, M, K, q, scales);
}

void oracle_int_accumulators(unsigned bits, size_t rows, size_t cols, size_t group, const void* data,
                             const int8_t* q, size_t M, int32_t* acc) {
    const Matrix w = make_matrix(bits, rows, cols, group, data, nullptr);
    const size_t groups = cols / group;
    for (size_t t = 0; t < M; ++t)
        for (size_t r = 0; r < rows; ++r)
            for (size_t g = 0; g < groups; ++g) {
                int32_t sum = 0;
                for (size_t c = g * group; c < (g + 1) * group; ++c) sum += w.qvalue(r * cols + c) * int32_t(q[t * cols + c]);
                acc[(t * rows + r) * groups + g] = sum;
            }
}

void oracle_linear_int(unsigned bits, size_t rows, size_t cols, size_t group, const void* data,
                       const float* scales, const float* bias, const float* x, size_t M, float* y) {
    std::vector<int8_t> q(M * cols);
    std::vector<float> qs(M);
    quantize_rows(x, M, cols, q.data(), qs.data());
    linear_rows(make_matrix(bits, rows, cols, group, data, scales), bias, x, M, Path::Int, y, q.data(), qs.data());
}

void oracle_linear_int_q(unsigned bits, size_t rows, size_t cols, size_t group, const void* data,
                         const float* scales, const float* bias, const int8_t* q, const float* qscale,
                         size_t M, float* y) {
    linear_rows(make_matrix(bits, rows, cols, group, data, scales), bias, nullptr, M, Path::Int, y, q, qscale);
}

void oracle_linear_fp(unsigned bits, size_t rows, size_t cols, size_t group, const void* data,
                      const float* scales, const float* bias, const float* x, size_t M, float* y) {
    linear_rows(make_matrix(bits, rows, cols, group, data, scales), bias, x, M, bits == 16 ? Path::Bf16 : Path::Fp, y);
}

void oracle_linear_accurate(unsigned bits, size_t rows, size_t cols, const void* data, const float* bias,
                            const float* x, size_t M, float* y) {
    linear_rows(make_matrix(bits, rows, cols, 0, data, nullptr), bias, x, M, Path::Accurate, y);
}

void oracle_norm(const float* x, size_t M, size_t width, const float* gamma, const float* beta,
                 float epsilon, unsigned kind, int accurate, float* y) {
    norm_rows(x, M, width, gamma, beta, epsilon, kind, accurate != 0, y);
}

// Decoder::Impl::Impl frequencies (decoder.cpp:929-933).
void oracle_rope_frequencies(float theta, unsigned rotary_dim, float* freq) {
    for (unsigned i = 0; i < rotary_dim / 2; ++i)
        freq[i] = 1.0f / std::pow(theta, static_cast<float>(2 * i) / static_cast<float>(rotary_dim));
}

// prepare_rotary_tables (decoder.cpp:1234-1258).
void oracle_rope_tables(const float* freq, unsigned rotary_dim, size_t position, size_t tokens,
                        float* cosines, float* sines) {
    const size_t half = rotary_dim / 2;
    for (size_t t = 0; t < tokens; ++t)
        for (size_t i = 0; i < half; ++i) {
            const float angle = static_cast<float>(position + t) * freq[i];
            cosines[t * half + i] = std::cos(angle);
            sines[t * half + i] = std::sin(angle);
        }
}

void oracle_attention(const float* q_heads, const float* keys, const float* values, const float* mask, float* out,
                      size_t heads, size_t kv_heads, size_t tokens, size_t total, size_t stride, size_t dim,
                      float scale) {
    attention(q_heads, keys, values, mask, out, heads, kv_heads, tokens, total, stride, dim, scale);
}

float oracle_activate(unsigned activation_code, float x) { return activate(activation_code, x); }

void oracle_activation(const float* gate_up, size_t tokens, size_t width, int gated, unsigned activation_code,
                       float* act) {
    for (size_t t = 0; t < tokens; ++t)
        for (size_t j = 0; j < width; ++j) {
            if (gated) {
                float up = gate_up[t * 2 * width + width + j];
                up *= activate(activation_code, gate_up[t * 2 * width + j]);
                act[t * width + j] = up;
            } else {
                act[t * width + j] = activate(activation_code, gate_up[t * width + j]);
            }
        }
}

void oracle_expf(const float* x, size_t count, float* y) {
#pragma omp parallel for schedule(static)
    for (long i = 0; i < long(count); ++i) y[i] = std::exp(x[i]);
}

// export_decoder.quantize (tools/export_decoder.py:91-105) in float32.
void oracle_quantize_weights(const float* w, size_t rows, size_t cols, unsigned bits, size_t group,
                             uint8_t* packed, float* scales) {
    const int limit = (1 << (bits - 1)) - 1;
    const size_t groups = cols / group;
    std::vector<int8_t> values(cols);
    for (size_t r = 0; r < rows; ++r) {
        for (size_t g = 0; g < groups; ++g) {
            float m = 0;
            for (size_t c = g * group; c < (g + 1) * group; ++c) m = std::max(m, std::fabs(w[r * cols + c]));
            const float s = std::max(m / static_cast<float>(limit), 1e-12f);
            scales[r * groups + g] = s;
            for (size_t c = g * group; c < (g + 1) * group; ++c) {
                const float v = std::nearbyint(w[r * cols + c] / s);
                values[c] = static_cast<int8_t>(std::max(float(-limit), std::min(float(limit), v)));
            }
        }
        if (bits == 8) {
            std::memcpy(packed + r * cols, values.data(), cols);
        } else {
            for (size_t c = 0; c < cols; c += 2)
                packed[r * (cols / 2) + c / 2] = uint8_t((values[c] & 15) | ((values[c + 1] & 15) << 4));
        }
    }
}

oracle_decoder* oracle_decoder_open(const char* path, unsigned activation_bits, int accurate,
                                    char* error, size_t error_size) {
    auto* d = new oracle_decoder();
    d->activation_bits = activation_bits;
    d->accurate = accurate != 0;
    try {
        d->open(path);
        return d;
    } catch (const std::exception& e) {
        if (error && error_size) std::snprintf(error, error_size, "%s", e.what());
        delete d;
        return nullptr;
    }
}

void oracle_decoder_close(oracle_decoder* d) { delete d; }
void oracle_decoder_reset(oracle_decoder* d) { for (auto& c : d->caches) c.length = 0; }
size_t oracle_decoder_cache_tokens(const oracle_decoder* d) { return d->caches[0].length; }
uint32_t oracle_decoder_vocab(const oracle_decoder* d) { return d->vocab; }
int oracle_decoder_is_eos(const oracle_decoder* d, uint32_t token) {
    return std::find(d->eos_tokens.begin(), d->eos_tokens.end(), token) != d->eos_tokens.end();
}

int oracle_decoder_forward(oracle_decoder* d, const uint32_t* ids, size_t count, int all_logits, float* logits,
                           char* error, size_t error_size) {
    try {
        std::vector<float> out;
        d->forward(std::vector<uint32_t>(ids, ids + count), all_logits != 0, out);
        std::memcpy(logits, out.data(), out.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        if (error && error_size) std::snprintf(error, error_size, "%s", e.what());
        return -1;
    }
}

// generate_continuation (main_decoder.cpp:95-113): greedy, first maximal index.
int oracle_decoder_generate(oracle_decoder* d, const uint32_t* prompt, size_t count, unsigned limit,
                            uint32_t* tokens, size_t* produced, char* error, size_t error_size) {
    try {
        std::vector<float> logits;
        d->forward(std::vector<uint32_t>(prompt, prompt + count), false, logits);
        size_t n = 0;
        for (unsigned i = 0; i < limit; ++i) {
            const auto id = static_cast<uint32_t>(std::max_element(logits.begin(), logits.end()) - logits.begin());
            tokens[n++] = id;
            if (oracle_decoder_is_eos(d, id)) break;
            if (i + 1 < limit) d->forward({id}, false, logits);
        }
        *produced = n;
        return 0;
    } catch (const std::exception& e) {
        if (error && error_size) std::snprintf(error, error_size, "%s", e.what());
        return -1;
    }
}

}  // extern "C"
