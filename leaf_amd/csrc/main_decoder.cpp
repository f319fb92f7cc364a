// leaf_decoder for MI355X: the process protocol of Leaf's native decoder
// (engine/src/main_decoder.cpp:116-363) over leaf::runtime::Decoder from
// include/leafhip_decoder.hpp, so `LEAF_DECODER_BIN=<this binary> leaf run`
// drives the GPU path unchanged.
//
//   leaf_decoder --runtime-info
//   leaf_decoder artifact tokens.bin logits.bin metrics.json
//                verify|chunked|bench|generate|bench-generate
//                [threads=1] [runs=3] [warmup=1] [generate=16] [scalar=0] [chunk=1]
//                [activation-bits=32] [worker-cpus] [--fp32-math=fast|accurate]
//
// tokens.bin: u32 request count, then per request u32 length + u32 ids
// (little endian).  verify / chunked write all-token logits to logits.bin;
// generate prints "TOKEN <id>" per greedy token; metrics.json carries the
// keys leaf run and the validation tools read.  Errors: "Leaf decoder: <what>"
// on stderr and exit status 1.
#include <sys/resource.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <fstream>
#include <iostream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "leafhip_decoder.hpp"

namespace {

using Clock = std::chrono::steady_clock;
using leaf::runtime::Decoder;

double ms_since(Clock::time_point t) {
    return std::chrono::duration<double, std::milli>(Clock::now() - t).count();
}

std::uint32_t read_le32(std::istream& in) {
    unsigned char b[4];
    if (!in.read(reinterpret_cast<char*>(b), 4)) throw std::runtime_error("truncated token request");
    return std::uint32_t(b[0]) | std::uint32_t(b[1]) << 8 | std::uint32_t(b[2]) << 16 | std::uint32_t(b[3]) << 24;
}

std::vector<std::vector<std::uint32_t>> read_requests(const char* path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw std::runtime_error("cannot open token request");
    const std::uint32_t count = read_le32(in);
    if (count == 0 || count > 100000) throw std::runtime_error("invalid request count");
    std::vector<std::vector<std::uint32_t>> requests(count);
    for (auto& ids : requests) {
        const std::uint32_t length = read_le32(in);
        if (length == 0 || length > 1048576) throw std::runtime_error("invalid token count");
        ids.resize(length);
        for (auto& id : ids) id = read_le32(in);
    }
    if (in.peek() != std::char_traits<char>::eof()) throw std::runtime_error("trailing token request bytes");
    return requests;
}

std::vector<unsigned> parse_cpus(const std::string& text) {
    std::vector<unsigned> cpus;
    std::stringstream stream(text);
    std::string item;
    while (std::getline(stream, item, ',')) {
        if (item.empty() || item.find_first_not_of("0123456789") != std::string::npos)
            throw std::runtime_error("worker CPUs must be comma-separated unsigned indices");
        const unsigned long long v = std::stoull(item);
        if (v > std::numeric_limits<unsigned>::max()) throw std::runtime_error("worker CPU index is too large");
        cpus.push_back(unsigned(v));
    }
    if (text.empty() || text.back() == ',') throw std::runtime_error("worker CPUs must be comma-separated unsigned indices");
    return cpus;
}

double median(std::vector<double> v) {
    if (v.empty()) return 0;
    std::sort(v.begin(), v.end());
    const std::size_t m = v.size() / 2;
    return v.size() % 2 ? v[m] : 0.5 * (v[m - 1] + v[m]);
}

template <typename T>
std::string json_list(const std::vector<T>& v) {
    std::ostringstream out;
    out.precision(10);
    out << '[';
    for (std::size_t i = 0; i < v.size(); ++i) out << (i ? "," : "") << v[i];
    out << ']';
    return out.str();
}

std::uint64_t peak_rss_bytes() {
    struct rusage usage {};
    return getrusage(RUSAGE_SELF, &usage) ? 0 : std::uint64_t(usage.ru_maxrss) * 1024;
}

// Greedy continuation (main_decoder.cpp:95-113): the first maximal logit wins,
// EOS stops, `limit` tokens come from limit - 1 single-token forwards.  The
// argmax is taken on the device; only token ids cross to the host.
double continue_greedily(Decoder& decoder, const std::vector<std::uint32_t>& prompt, unsigned limit, bool stream,
                         std::vector<std::uint32_t>& tokens, std::vector<double>& steps) {
    auto start = Clock::now();
    std::uint32_t id = decoder.forward_argmax(prompt);
    const double prefill = ms_since(start);
    for (unsigned i = 0; i < limit; ++i) {
        tokens.push_back(id);
        if (stream) std::cout << "TOKEN " << id << '\n' << std::flush;
        if (decoder.is_eos_token(id)) break;
        if (i + 1 < limit) {
            start = Clock::now();
            id = decoder.forward_argmax({id});
            steps.push_back(ms_since(start));
        }
    }
    return prefill;
}

void runtime_info() {
    std::cout << "{\"runtime\":\"leaf_decoder\",\"artifact_versions\":[2,3,4,5,6,7]"
                 ",\"source_bf16_head_supported\":true,\"source_bf16_matrices_supported\":true"
                 ",\"benchmark_power_guard\":false,\"worker_affinity_supported\":false,\"worker_spin_limit_us\":0"
                 ",\"fp32_math_modes\":[\"fast\",\"accurate\"],\"fp32_math_default\":\"fast\""
                 ",\"reusable_logits_supported\":true,\"generation_benchmark_supported\":true"
                 ",\"benchmark_counters_supported\":false,\"benchmark_counter_version\":1"
                 ",\"device\":\"MI355X (gfx950)\",\"backend\":\""
              << lh_version() << "\"}\n";
}

int run(int argc, char** argv) {
    const std::string mode = argv[5];
    const bool bench_generate = mode == "bench-generate";
    if (mode != "verify" && mode != "chunked" && mode != "bench" && mode != "generate" && !bench_generate)
        throw std::runtime_error("unknown decoder mode");
    auto arg = [&](int i, unsigned fallback) { return argc > i ? unsigned(std::stoul(argv[i])) : fallback; };
    const unsigned threads = arg(6, 1), runs = arg(7, 3), warmup = arg(8, 1), generate = arg(9, 16);
    const bool scalar = argc > 10 && std::stoi(argv[10]) != 0;
    const unsigned chunk = arg(11, 1), activation_bits = arg(12, 32);
    std::vector<unsigned> cpus;
    auto math = leaf::runtime::FP32Math::Fast;
    bool math_seen = false, cpus_seen = false, counters = false;
    for (int i = 13; i < argc; ++i) {
        const std::string v = argv[i];
        if (v.rfind("--fp32-math=", 0) == 0) {
            if (math_seen) throw std::runtime_error("duplicate FP32 math policy");
            math_seen = true;
            const std::string policy = v.substr(12);
            if (policy == "accurate") math = leaf::runtime::FP32Math::Accurate;
            else if (policy != "fast") throw std::runtime_error("FP32 math must be fast or accurate");
        } else if (v == "--benchmark-counters") {
            if (counters) throw std::runtime_error("duplicate benchmark counters flag");
            counters = true;
        } else {
            if (v.rfind("--", 0) == 0) throw std::runtime_error("unknown decoder option: " + v);
            if (cpus_seen || math_seen || counters)
                throw std::runtime_error("worker CPU list must precede named decoder options");
            cpus_seen = true;
            cpus = parse_cpus(v);
        }
    }
    if (counters && mode != "bench") throw std::runtime_error("benchmark counters require bench mode");
    if (counters) throw std::runtime_error("requested benchmark counters require Windows");
    if (!runs || !chunk) throw std::runtime_error("runs and chunk must be positive");
    const auto requests = read_requests(argv[2]);
    if (bench_generate && (requests.size() != 1 || generate == 0 ||
                           warmup > std::numeric_limits<unsigned>::max() - runs))
        throw std::runtime_error(
            "generation benchmark requires one prompt, a positive generation limit and valid iteration counts");

    const auto load_start = Clock::now();
    Decoder decoder(argv[1], threads, scalar, activation_bits, cpus, math);
    const double load_ms = ms_since(load_start);
    std::ofstream logits_out(argv[3], std::ios::binary);
    if (!logits_out) throw std::runtime_error("cannot open logits output");

    std::vector<double> prefills, decodes, generations;
    std::vector<std::vector<double>> steps_by_generation;
    std::vector<std::uint32_t> generated;
    std::vector<float> logits;
    for (const auto& ids : requests) {
        decoder.reset();
        if (mode == "verify" || mode == "chunked") {
            const std::size_t step = mode == "verify" ? ids.size() : std::size_t(chunk);
            for (std::size_t pos = 0; pos < ids.size(); pos += step) {
                const std::vector<std::uint32_t> part(ids.begin() + pos, ids.begin() + std::min(ids.size(), pos + step));
                decoder.forward_into(part, logits, true);
                logits_out.write(reinterpret_cast<const char*>(logits.data()), std::streamsize(logits.size() * 4));
            }
        } else if (mode == "bench") {
            if (ids.size() < 2) throw std::runtime_error("benchmark requires a prefix and final token");
            const std::vector<std::uint32_t> prefix(ids.begin(), ids.end() - 1), last{ids.back()};
            for (unsigned it = 0; it < runs + warmup; ++it) {
                decoder.reset();
                auto t = Clock::now();
                decoder.forward_into(prefix, logits);
                const double p = ms_since(t);
                t = Clock::now();
                decoder.forward_into(last, logits);
                const double d = ms_since(t);
                if (it >= warmup) { prefills.push_back(p); decodes.push_back(d); }
            }
        } else if (bench_generate) {
            for (unsigned it = 0; it < runs + warmup; ++it) {
                std::vector<std::uint32_t> tokens;
                std::vector<double> steps;
                decoder.reset();
                const auto t = Clock::now();
                const double p = continue_greedily(decoder, ids, generate, false, tokens, steps);
                const double total = ms_since(t);
                if (it == 0) generated = tokens;
                if (tokens != generated) throw std::runtime_error("greedy generation differed between benchmark iterations");
                if (it >= warmup) {
                    prefills.push_back(p);
                    decodes.insert(decodes.end(), steps.begin(), steps.end());
                    generations.push_back(total);
                    steps_by_generation.push_back(steps);
                }
            }
        } else {
            prefills.push_back(continue_greedily(decoder, ids, generate, true, generated, decodes));
        }
    }
    if (!logits_out) throw std::runtime_error("failed to write logits");
    std::ofstream metrics(argv[4]);
    if (!metrics) throw std::runtime_error("cannot write metrics");
    metrics.precision(10);
    metrics << "{\"avx2\":false,\"device\":\"MI355X (gfx950)\",\"vector_silu_gate_calls\":0"
            << ",\"source_bf16_tensors\":" << decoder.source_bf16_tensors()
            << ",\"benchmark_ac_checked\":false,\"source_bf16_linear_calls\":0"
            << ",\"vector_silu_gate_enabled\":false,\"optimized_fp32_active\":false"
            << ",\"fp32_math\":\"" << (decoder.uses_accurate_fp32() ? "accurate" : "fast") << '"'
            << ",\"reusable_logits\":true,\"vnni\":false,\"activation_bits\":" << decoder.activation_bits()
            << ",\"threads\":" << threads << ",\"artifact_bytes\":" << decoder.weight_bytes()
            << ",\"device_weight_bytes\":" << decoder.device_weight_bytes()
            << ",\"peak_rss_bytes\":" << peak_rss_bytes() << ",\"load_ms\":" << load_ms
            << ",\"prefill_p50_ms\":" << median(prefills) << ",\"decode_p50_ms\":" << median(decodes)
            << ",\"prefill_samples_ms\":" << json_list(prefills) << ",\"decode_samples_ms\":" << json_list(decodes)
            << ",\"worker_cpus\":" << json_list(cpus) << ",\"worker_spin_us\":0"
            << ",\"generated_tokens\":" << json_list(generated);
    if (bench_generate) {
        metrics << ",\"generation_samples_ms\":" << json_list(generations) << ",\"decode_steps_by_generation_ms\":[";
        for (std::size_t i = 0; i < steps_by_generation.size(); ++i)
            metrics << (i ? "," : "") << json_list(steps_by_generation[i]);
        metrics << ']';
    }
    metrics << "}\n";
    std::cout << "Leaf decoder completed; device=MI355X, peak RSS=" << peak_rss_bytes() << '\n';
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc == 2 && std::string(argv[1]) == "--runtime-info") {
        runtime_info();
        return 0;
    }
    if (argc < 6 || argc > 16) {
        std::cerr << "Usage: leaf_decoder artifact.leaf tokens.bin logits.bin metrics.json mode "
                     "(verify|chunked|bench|generate|bench-generate) [threads=1] [runs=3] [warmup=1] [generate=16] "
                     "[scalar=0] [chunk=1] [activation-bits=32] [worker-cpus=comma-list] "
                     "[--fp32-math=fast|accurate] [--benchmark-counters]\n";
        return 1;
    }
    try {
        return run(argc, argv);
    } catch (const std::exception& error) {
        std::string message = error.what();
        const std::string prefix = "Leaf decoder: ";
        if (message.compare(0, prefix.size(), prefix) == 0) message = message.substr(prefix.size());
        std::cerr << prefix << message << '\n';
        return 1;
    }
}
