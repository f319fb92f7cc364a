// Decoding session: device KV cache, workspaces and RoPE tables planned once,
// and the forward pass of Decoder::Impl::forward_into (decoder.cpp:1282-1444).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <limits>
#include <string>
#include <vector>

#include "runtime.h"

namespace leafhip {

namespace {
template <typename T>
void grow(DeviceBuffer& b, size_t count) {
    if (b.bytes < count * sizeof(T)) b.allocate(count * sizeof(T));
}
}  // namespace

const char* Profiler::name(int kind) {
    static const char* names[] = {"gemv_w8a8", "gemv_fp", "gemm_w8a8", "gemm_fp", "attention", "other",
                                  "decode_step"};
    return names[kind];
}

hipEvent_t Profiler::next_event() {
    if (used_ == events_.size()) {
        hipEvent_t e;
        hip_check(hipEventCreate(&e), "hipEventCreate");
        events_.push_back(e);
    }
    return events_[used_++];
}

void Profiler::begin(hipStream_t stream) {
    hip_check(hipEventRecord(next_event(), stream), "hipEventRecord");
}

void Profiler::end(hipStream_t stream, int kind, double bytes, double operations) {
    const size_t start = used_ - 1;
    hip_check(hipEventRecord(next_event(), stream), "hipEventRecord");
    pending_.push_back({kind, bytes, operations, start});
}

void Profiler::collect() {
    for (const auto& p : pending_) {
        float ms = 0;
        hip_check(hipEventElapsedTime(&ms, events_[p.event], events_[p.event + 1]), "hipEventElapsedTime");
        Total& t = totals[p.kind];
        ++t.launches;
        t.ms += ms;
        t.bytes += p.bytes;
        t.ops += p.ops;
    }
    pending_.clear();
    used_ = 0;
}

Profiler::~Profiler() {
    for (auto e : events_) (void)hipEventDestroy(e);
}

NumericsMode resolve_numerics(uint32_t numerics, bool integer_activations) {
    if (numerics == LH_NUMERICS_DEFAULT) {
        const char* env = std::getenv("LEAF_GPU_NUMERICS");
        const std::string name = env ? env : "";
        numerics = name == "reference" ? LH_NUMERICS_REFERENCE
                 : name == "reference-avx2" ? LH_NUMERICS_REFERENCE_AVX2
                 : name == "reference-vnni" ? LH_NUMERICS_REFERENCE_VNNI
                 : name == "fast" ? LH_NUMERICS_FAST
                 : integer_activations ? LH_NUMERICS_REFERENCE : LH_NUMERICS_FAST;
    }
    NumericsMode mode;
    switch (numerics) {
    case LH_NUMERICS_FAST: break;
    case LH_NUMERICS_REFERENCE: {
        mode.reference = true;
        const char* disabled = std::getenv("LEAF_DISABLE_VNNI");
#ifndef __HIP_DEVICE_COMPILE__   // x86 feature bits exist in the host pass only
        __builtin_cpu_init();
        mode.vnni = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
                    __builtin_cpu_supports("avxvnni") && !(disabled && disabled[0]);
#endif
        break;
    }
    case LH_NUMERICS_REFERENCE_AVX2: mode.reference = true; break;
    case LH_NUMERICS_REFERENCE_VNNI: mode.reference = mode.vnni = true; break;
    default: throw Error(LH_ERROR_INVALID_ARGUMENT, "Leaf decoder: unknown numerics mode");
    }
    return mode;
}

Session::Session(Model& m, uint32_t max_context, uint32_t max_prefill, uint32_t numerics) : model(m) {
    const Config& c = m.config;
    capacity = max_context ? std::min(max_context, c.max_positions) : c.max_positions;
    check(capacity > 0, "session capacity must be positive", LH_ERROR_INVALID_ARGUMENT);
    const NumericsMode mode = resolve_numerics(numerics, m.activation_bits == 8);
    reference_ = mode.reference;
    reference_vnni_ = mode.vnni && m.activation_bits == 8;
    if (reference_) {
        // The accurate FP32 policy sums its GEMMs in 256-column blocks
        // (accurate_fp32.h); the reference-order kernels follow dot_avx only.
        check(!m.accurate, "reference-order numerics do not support accurate FP32 math", LH_ERROR_UNSUPPORTED);
        check(c.hidden <= uint32_t(kReferenceOrderMaxWidth) && c.head_dim <= 256,
              "reference-order numerics: hidden or head width too large", LH_ERROR_UNSUPPORTED);
        // One query's keys sit in LDS in the reference-order attention.  A
        // session asked for more visible keys is refused here, not at the
        // token that would pass the limit; without a requested size the
        // capacity stops at the limit.
        reference_keys_ = reference_order_attention_keys();
        const uint32_t limit = uint32_t(reference_keys_);
        if (std::min(capacity, c.sliding_window ? c.sliding_window : capacity) > limit) {
            check(max_context == 0,
                  "reference-order numerics hold at most " + std::to_string(limit) +
                      " visible keys per query; ask for a smaller context",
                  LH_ERROR_UNSUPPORTED);
            capacity = limit;
        }
    }
    // KV cache for the whole context, [layers][k|v][kv_heads][capacity][dim].
    kv_.allocate(size_t(c.layers) * 2 * c.kv_heads * capacity * c.head_dim * sizeof(float));
    // RoPE tables for every position the cache can hold, from the same float
    // expressions and libm calls as prepare_rotary_tables (decoder.cpp:1247-1256),
    // so they equal the CPU's tables bit for bit.
    if (c.position_kind == 0) {
        const size_t half = c.rotary_dim / 2;
        std::vector<float> cosines(size_t(capacity) * half), sines(cosines.size());
        for (size_t pos = 0; pos < capacity; ++pos)
            for (size_t i = 0; i < half; ++i) {
                const float angle = static_cast<float>(pos) * c.rope_frequencies[i];
                cosines[pos * half + i] = std::cos(angle);
                sines[pos * half + i] = std::sin(angle);
            }
        rope_cos_.allocate(cosines.size() * sizeof(float));
        rope_sin_.allocate(sines.size() * sizeof(float));
        hip_check(hipMemcpy(rope_cos_.ptr, cosines.data(), cosines.size() * 4, hipMemcpyHostToDevice), "rope upload");
        hip_check(hipMemcpy(rope_sin_.ptr, sines.data(), sines.size() * 4, hipMemcpyHostToDevice), "rope upload");
    }
    // Split-K decode attention scratch: (max, sum, out[dim]) per head per key
    // span (spans are >= 16 keys).
    const size_t splits = (capacity + 15) / 16;
    partial_.allocate(splits * c.heads * (c.head_dim + 2) * sizeof(float));
    counters_.allocate(size_t(c.kv_heads) * sizeof(unsigned));
    hip_check(hipMemset(counters_.ptr, 0, counters_.bytes), "hipMemset");
    grow<uint32_t>(argmax_, 1);
    argmax_scratch_.allocate(size_t(argmax_scratch_floats()) * sizeof(float));
    hip_check(hipMemset(argmax_scratch_.ptr, 0, argmax_scratch_.bytes), "hipMemset");
    hip_check(hipHostMalloc((void**)&host_argmax_, sizeof(uint32_t), hipHostMallocMapped), "hipHostMalloc");
    hip_check(hipHostGetDevicePointer((void**)&mapped_argmax_, host_argmax_, 0), "hipHostGetDevicePointer");
    hip_check(hipHostMalloc((void**)&host_position_, sizeof(int)), "hipHostMalloc");
    position_.allocate(sizeof(int));
    const char* graphs = std::getenv("LEAF_DECODE_GRAPH");
    graphs_enabled_ = !(graphs && std::string(graphs) == "0");
    plan(max_prefill ? max_prefill : 512, false);
    const char* fuse = std::getenv("LEAF_PREFILL_FUSE");
    fuse_quantize_ = !(fuse && std::string(fuse) == "0");
    const char* step = std::getenv("LEAF_DECODE_STEP");
    step_enabled_ = !(step && std::string(step) == "0");
    // LEAF_DECODE_STEP_COOPERATIVE=0: launch the step as a plain grid (for
    // profilers that fail at process exit after cooperative launches).
    const char* coop = std::getenv("LEAF_DECODE_STEP_COOPERATIVE");
    step_cooperative_ = !(coop && std::string(coop) == "0");
    if (step_enabled_) step_prepare();
}

Session::~Session() {
    drop_graphs();
    if (step_host_abort_) (void)hipHostFree(step_host_abort_);
    if (host_ids_) (void)hipHostFree(host_ids_);
    if (host_argmax_) (void)hipHostFree(host_argmax_);
    if (host_position_) (void)hipHostFree(host_position_);
}

// Workspaces for `tokens` rows; kept at their high-water mark like the CPU
// runtime's vectors (decoder.cpp:755-765), so steady-state decode allocates nothing.
void Session::plan(uint32_t tokens, bool all_logits) {
    const Config& c = model.config;
    if (tokens > planned || (all_logits ? tokens : 1) > logits_rows_) drop_graphs();   // captured pointers move
    if (tokens > planned) {
        const size_t P = tokens;
        const size_t qkv_width = size_t(c.qwidth()) + 2 * c.kvwidth();
        const size_t widest = std::max<size_t>({c.hidden, c.qwidth(), c.intermediate});
        grow<float>(hidden_, P * c.hidden);
        grow<float>(normed_, P * c.hidden);
        grow<float>(qkv_, P * qkv_width);
        grow<float>(q_heads_, P * c.qwidth());
        grow<float>(attn_, P * c.qwidth());
        grow<float>(attn_proj_, P * c.hidden);
        grow<float>(gate_up_, P * 2 * c.intermediate);
        grow<float>(act_, P * c.intermediate);
        grow<float>(proj_, P * c.hidden);
        grow<int8_t>(xq_, P * widest);
        grow<float>(xs_, P);
        grow<float>(scaled_, P * widest);
        // split-K sums of the W8A8 prefill GEMM: up to 8 splits of a
        // hidden-wide output (wider outputs split less or not at all)
        if (model.activation_bits == 8 && tokens > 4) grow<int32_t>(split_, P * 8 * c.hidden);
        grow<uint32_t>(ids_, P);
        if (host_ids_) (void)hipHostFree(host_ids_);
        hip_check(hipHostMalloc((void**)&host_ids_, P * sizeof(uint32_t)), "hipHostMalloc");
        planned = tokens;
    }
    const uint32_t rows = all_logits ? tokens : 1;
    if (rows > logits_rows_) {
        logits_.allocate(size_t(rows) * c.vocab * sizeof(float));
        logits_rows_ = rows;
    }
}

LinearCall Session::make_call(const Linear& l, const float* x, int tokens, float* y, int epilogue,
                              const NormView* fuse_norm) {
    LinearCall call;
    call.w = l.view;
    call.tokens = tokens;
    call.y = y;
    call.epilogue = epilogue;
    call.integer_activations = model.integer_linear(l);
    call.x = l.input_scale ? nullptr : x;
    if (fuse_norm) call.norm = *fuse_norm;
    return call;
}

bool Session::prequantizes(const Linear& l, int tokens) const {
    return fuse_quantize_ && !reference_ && tokens > 1 && model.integer_linear(l) && !l.input_scale;
}

// Reference order: an integer linear after an RMSNorm takes its input from
// the column-order norm kernel's own quantization (one launch, no FP32 rows).
bool Session::reference_prequantizes(const Linear& l, int tokens, const NormView& n, int width) const {
    return fuse_quantize_ && reference_ && tokens > 1 && model.integer_linear(l) && !l.input_scale && n.kind == 0 &&
           !n.accurate && width <= kReferenceOrderQuantizeMaxWidth;
}

// Reference order: the gated activation before an integer down projection
// quantized in the same launch (reference-order activation, exact maximum).
bool Session::reference_prequantizes_down(const Layer& L, int rows) const {
    const Config& c = model.config;
    return fuse_quantize_ && reference_ && rows > 1 && c.gated && model.integer_linear(L.down) &&
           !L.down.input_scale && c.intermediate <= 8 * 1024;
}

void Session::norm_prequantize(const float* x, int rows, int width, const NormView& n) {
    timed(Profiler::Other, 0, 0, [&] {
        if (reference_)
            check(launch_norm_quantize_reference_order(x, rows, width, n, xq_.as<int8_t>(), xs_.as<float>(), stream()),
                  "reference-order norm rejected", LH_ERROR_UNSUPPORTED);
        else
            launch_norm_quantize(x, rows, width, n, xq_.as<int8_t>(), xs_.as<float>(), stream());
    });
}

void Session::norm(const float* x, int rows, int width, const NormView& n, float* y, int rows_per_group,
                   size_t group_stride) {
    if (reference_) {
        check(launch_norm_reference_order(x, rows, width, n, y, stream(), rows_per_group, group_stride),
              "reference-order norm rejected", LH_ERROR_UNSUPPORTED);
    } else {
        launch_norm(x, rows, width, n, y, stream(), rows_per_group, group_stride);
    }
}

void Session::activation(const float* gate_up, int rows, int width, int gated, float* act) {
    const int code = int(model.config.activation);
    if (reference_) launch_activation_reference_order(gate_up, rows, width, gated, code, act, stream());
    else launch_activation(gate_up, rows, width, gated, code, act, stream());
}

void Session::run_linear(const Linear& l, const float* x, int tokens, float* y, int epilogue,
                         const NormView* fuse_norm, const PairEpilogue* pair, bool prequantized) {
    LinearCall call;
    call.w = l.view;
    call.tokens = tokens;
    call.y = y;
    call.epilogue = epilogue;
    call.integer_activations = model.integer_linear(l);
    call.xq_scratch = xq_.as<int8_t>();
    call.xs_scratch = xs_.as<float>();
    call.norm_scratch = normed_.as<float>();
    call.split_scratch = split_.as<int32_t>();
    call.split_capacity = split_.bytes / sizeof(int32_t);
    call.unfused_group_sum = reference_vnni_ && l.view.bits == 8 && l.view.group <= 65536;
    if (l.input_scale) {
        // SmoothQuant input factors (decoder.cpp:1008-1019) before quantization.
        launch_scale_columns(x, tokens, l.view.cols, l.input_scale, scaled_.as<float>(), stream());
        x = scaled_.as<float>();
    }
    call.x = x;
    if (prequantized) {
        // xq_ / xs_ already hold this input quantized per token
        call.x = nullptr;
        call.xq = xq_.as<int8_t>();
        call.xs = xs_.as<float>();
    }
    if (fuse_norm) call.norm = *fuse_norm;
    if (pair) call.pair = *pair;
    // Algorithmic traffic: weights, scales, activations (int8 when quantized),
    // outputs: N*K*b_w + 4*N*(K/g) + K*M*b_x + 4*M*N.
    const WeightView& w = l.view;
    const double groups = (w.bits == 8 || w.bits == 4) ? double(w.cols) / w.group : 0.0;
    const double bytes = double(w.rows) * w.cols * w.bits / 8 + 4.0 * w.rows * groups +
                         double(w.cols) * tokens * (call.integer_activations ? 1 : 4) + 4.0 * tokens * w.rows;
    const double ops = 2.0 * tokens * double(w.rows) * w.cols;
    const int kind = tokens <= 4 ? (call.integer_activations ? Profiler::GemvW8A8 : Profiler::GemvFp)
                                 : (call.integer_activations ? Profiler::GemmW8A8 : Profiler::GemmFp);
    int path = 0;
    if (reference_ && !call.integer_activations) {
        // dot_avx order (the integer path is exact in every mode)
        check(!pair && !fuse_norm && !prequantized, "reference-order linear cannot fuse", LH_ERROR_UNSUPPORTED);
        timed(kind, bytes, ops, [&] {
            path = launch_linear_fp_reference_order(w, x, tokens, y, epilogue, stream()) ? 1 : -1;
        });
    } else {
        timed(kind, bytes, ops, [&] { path = launch_linear(call, stream()); });
    }
    check(path > 0, "linear launch rejected", LH_ERROR_UNSUPPORTED);
}

void Session::validate(const uint32_t* ids, size_t count, bool all_logits, float* host_logits,
                       size_t host_capacity) const {
    const Config& c = model.config;
    // Input validation before any mutation (decoder.cpp:1286-1289).
    check(count > 0, "input tokens are empty", LH_ERROR_INVALID_ARGUMENT);
    const size_t position = length;
    check(position <= c.max_positions && count <= c.max_positions - position, "context length exceeds artifact limit",
          LH_ERROR_STATE);
    for (size_t i = 0; i < count; ++i) check(ids[i] < c.vocab, "token id exceeds vocabulary", LH_ERROR_INVALID_ARGUMENT);
    check(position + count <= capacity, "context length exceeds session capacity", LH_ERROR_STATE);
    check(count <= uint32_t(std::numeric_limits<int32_t>::max()), "too many tokens", LH_ERROR_INVALID_ARGUMENT);
    const size_t out_rows = all_logits ? count : 1;
    check(!host_logits || host_capacity >= out_rows * c.vocab, "logits buffer too small", LH_ERROR_INVALID_ARGUMENT);
}

void Session::forward(const uint32_t* ids, size_t count, bool all_logits, float* host_logits, size_t host_capacity,
                      uint32_t* argmax) {
    validate(ids, count, all_logits, host_logits, host_capacity);
    plan(uint32_t(count), all_logits);
    hipStream_t s = stream();
    if (count == 1 && !all_logits && step_usable()) {
        decode_step(ids[0], host_logits, argmax);
        return;
    }
    step_token_valid_ = false;
    if (count == 1 && !all_logits && graph_decode_ok()) {
        decode_graphed(ids[0], true, host_logits, argmax);
        return;
    }
    std::memcpy(host_ids_, ids, count * sizeof(uint32_t));
    hip_check(hipMemcpyAsync(ids_.ptr, host_ids_, count * sizeof(uint32_t), hipMemcpyHostToDevice, s), "ids upload");
    launch(int(count), length, all_logits, nullptr, 0);
    const int head_rows = all_logits ? int(count) : 1;
    float* logits = logits_.as<float>();
    launch_argmax_row(logits + size_t(head_rows - 1) * model.config.vocab, int(model.config.vocab),
                      argmax_.as<uint32_t>(), argmax_scratch_.as<float>(), s);
    hip_check(hipMemcpyAsync(host_argmax_, argmax_.ptr, sizeof(uint32_t), hipMemcpyDeviceToHost, s), "argmax copy");
    if (host_logits)
        hip_check(hipMemcpyAsync(host_logits, logits, size_t(head_rows) * model.config.vocab * sizeof(float),
                                 hipMemcpyDeviceToHost, s), "logits copy");
    hip_check(hipStreamSynchronize(s), "forward");
    if (profiler.enabled) profiler.collect();
    if (argmax) *argmax = *host_argmax_;
    logits_device = logits;
    logits_count = size_t(head_rows) * model.config.vocab;
    length += count;
    device_position_valid_ = false;
}

// Single-token decode replayed from a captured graph.  Kernels read the
// position from device memory; the graph ends with the device argmax, which
// writes the next input id (for generate_continuation, main_decoder.cpp:95-113),
// the host-visible argmax and the advanced position.
bool Session::graph_decode_ok() const {
    if (profiler.enabled || !graphs_enabled_) return false;
    const Config& c = model.config;
    return attention_decode_supported(int(c.heads), int(c.kv_heads), int(c.head_dim));
}

void Session::decode_graphed(uint32_t id, bool upload_id, float* host_logits, uint32_t* argmax) {
    const Config& c = model.config;
    hipStream_t s = stream();
    const int needed = attention_decode_spans(int(length) + 1, int(c.head_dim));
    const int most = attention_decode_spans(int(capacity), int(c.head_dim));
    // Span buckets of 1, 2, 4, 8, ... spans, one captured graph each: a context
    // of one span runs its attention without the merge launch.
    int bucket = 1;
    while (bucket < needed) bucket *= 2;
    bucket = std::min(bucket, most);
    if (!device_position_valid_) {
        *host_position_ = int(length);
        hip_check(hipMemcpyAsync(position_.ptr, host_position_, sizeof(int), hipMemcpyHostToDevice, s), "position");
        device_position_valid_ = true;
    }
    if (upload_id) {
        *host_ids_ = id;
        hip_check(hipMemcpyAsync(ids_.ptr, host_ids_, sizeof(uint32_t), hipMemcpyHostToDevice, s), "ids upload");
    }
    hipGraphExec_t& exec = graphs_[bucket];
    if (!exec) {
        hipGraph_t graph;
        hip_check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            launch(1, length, false, position_.as<int>(), bucket);
            launch_argmax_advance(logits_.as<float>(), int(c.vocab), ids_.as<uint32_t>(), mapped_argmax_,
                                  position_.as<int>(), argmax_scratch_.as<float>(), s);
        } catch (...) {
            (void)hipStreamEndCapture(s, &graph);
            throw;
        }
        hip_check(hipStreamEndCapture(s, &graph), "hipStreamEndCapture");
        const hipError_t st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        hip_check(st, "hipGraphInstantiate");
    }
    hip_check(hipGraphLaunch(exec, s), "hipGraphLaunch");
    if (host_logits)
        hip_check(hipMemcpyAsync(host_logits, logits_.ptr, size_t(c.vocab) * sizeof(float), hipMemcpyDeviceToHost, s),
                  "logits copy");
    hip_check(hipStreamSynchronize(s), "decode");
    if (argmax) *argmax = *host_argmax_;
    logits_device = logits_.as<float>();
    logits_count = c.vocab;
    length += 1;
}

// ---------------------------------------------------------------------------
// Persistent decode step.  Used for single-token forwards of W8A8 decoders with
// per-row int8 matrices, RMSNorm, RoPE, a SiLU/GELU/ReLU-gated MLP, head dim 64
// and an FP32 head -- the TinyLlama shape -- when the geometry fits one block
// per CU (decode_step_fits).  Everything else takes the graph-replayed path.
void Session::step_prepare() {
    const Model& m = model;
    const Config& c = m.config;
    if (m.activation_bits != 8 || m.accurate || c.norm_kind != 0 || !c.gated || c.position_kind != 0 || c.qk_norm ||
        c.parallel || !c.final_norm || c.head_dim != kStepDim || c.rotary_dim > c.head_dim ||
        c.layers > uint32_t(kStepMaxLayers))
        return;
    if (m.final_norm.beta || m.head.view.bits != 32 || m.head.input_scale) return;
    if (reference_ && !decode_step_fits_reference(int(c.hidden), int(c.activation))) return;
    if (!(m.embedding.bits == 32 || (m.embedding.bits == 8 && m.embedding.group == m.embedding.cols))) return;
    auto per_row_int8 = [](const Linear& l) {
        return l.present && l.view.bits == 8 && l.view.group == l.view.cols && !l.input_scale && l.view.bias;
    };
    for (const Layer& L : m.layers) {
        if (!L.stacked_qkv || !L.stacked_gate_up || !per_row_int8(L.qkv) || !per_row_int8(L.o) ||
            !per_row_int8(L.gate_up) || !per_row_int8(L.down) || L.input_norm.beta || L.post_norm.beta ||
            !L.input_norm.gamma || !L.post_norm.gamma)
            return;
    }
    if (reference_) {
        // In reference order the step quantizes each layer's two normalized
        // inputs speculatively from x * gamma and confirms against the exact
        // norm; its error bound holds for |gamma| up to 1e20.
        std::vector<float> g(c.hidden);
        for (const Layer& L : m.layers)
            for (const float* gamma : {L.input_norm.gamma, L.post_norm.gamma}) {
                hip_check(hipMemcpy(g.data(), gamma, g.size() * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
                for (float v : g)
                    if (!(std::fabs(v) <= 1e20f)) return;
            }
    }
    const int blocks = decode_step_blocks(m.context.device);
    if (!decode_step_fits(int(c.hidden), int(c.intermediate), int(c.heads), int(c.kv_heads), int(c.head_dim),
                          int(c.vocab), blocks))
        return;
    std::vector<StepLayer> layers(c.layers);
    for (uint32_t i = 0; i < c.layers; ++i) {
        const Layer& L = m.layers[i];
        layers[i].qkv = L.qkv.view;
        layers[i].o = L.o.view;
        layers[i].gate_up = L.gate_up.view;
        layers[i].down = L.down.view;
        layers[i].input_gamma = L.input_norm.gamma;
        layers[i].post_gamma = L.post_norm.gamma;
    }
    step_layers_.allocate(layers.size() * sizeof(StepLayer));
    hip_check(hipMemcpy(step_layers_.ptr, layers.data(), step_layers_.bytes, hipMemcpyHostToDevice), "step upload");
    // Exchange words, per-head counters and the abort flag, zeroed once.
    const size_t group = c.heads / c.kv_heads;
    const size_t qkv = size_t(c.qwidth()) + 2 * c.kvwidth();
    const size_t part = size_t(c.kv_heads) * kStepMaxSpans * group * (c.head_dim + 2);
    // The kernel polls each vector in fixed per-lane blocks, so every vector
    // is padded to its largest width plus kStepPadWords.
    const size_t hidden_words = size_t(kStepMaxHidden) + kStepPadWords;
    const size_t qkv_words = qkv + kStepPadWords, ffn_words = size_t(kStepMaxFfn) + kStepPadWords;
    const size_t words = 3 * hidden_words + qkv_words + ffn_words + part + 2 * size_t(blocks);
    step_exchange_.allocate(words * 8 + (c.kv_heads + 1) * sizeof(unsigned));
    hip_check(hipMemset(step_exchange_.ptr, 0, step_exchange_.bytes), "hipMemset");
    auto* w = step_exchange_.as<unsigned long long>();
    StepParams& p = step_;
    p.x_hidden = w; w += hidden_words;
    p.x_mid = w; w += hidden_words;
    p.x_qkv = w; w += qkv_words;
    p.x_attn = w; w += hidden_words;
    p.x_act = w; w += ffn_words;
    p.x_part = w; w += part;
    p.x_best = w; w += 2 * size_t(blocks);
    // XCD-local copy of the span partials (plain device memory); see
    // StepParams::x_part_local.  LEAF_DECODE_STEP_LOCAL_MERGE=0 turns it off.
    const char* local = std::getenv("LEAF_DECODE_STEP_LOCAL_MERGE");
    if (!(local && std::string(local) == "0")) {
        step_part_local_.allocate(part * 8);
        hip_check(hipMemset(step_part_local_.ptr, 0, step_part_local_.bytes), "hipMemset");
        p.x_part_local = step_part_local_.as<unsigned long long>();
        // and the q rows of each head slice, read by that slice's items
        // (LEAF_DECODE_STEP_LOCAL_Q=0 turns this part off)
        const char* local_q = std::getenv("LEAF_DECODE_STEP_LOCAL_Q");
        if (!(local_q && std::string(local_q) == "0")) {
            step_q_local_.allocate(qkv_words * 8);
            hip_check(hipMemset(step_q_local_.ptr, 0, step_q_local_.bytes), "hipMemset");
            p.x_q_local = step_q_local_.as<unsigned long long>();
        }
        // LEAF_DECODE_STEP_FORCE_XCD_MISMATCH=1 (tests): the last block's XCD
        // check fails and it leaves at once, so the step aborts and the
        // fallback to the memory-based merge runs.
        if (const char* flip = std::getenv("LEAF_DECODE_STEP_FORCE_XCD_MISMATCH")) p.xcd_check_flip = std::atoi(flip) ? 1 : 0;
    }
    p.counters = reinterpret_cast<unsigned*>(w);
    p.abort_flag = p.counters + c.kv_heads;
    hip_check(hipHostMalloc((void**)&step_host_abort_, sizeof(unsigned), hipHostMallocMapped), "hipHostMalloc");
    *step_host_abort_ = 0;
    hip_check(hipHostGetDevicePointer((void**)&p.host_abort, step_host_abort_, 0), "hipHostGetDevicePointer");
    p.layers = int(c.layers);
    p.hidden = int(c.hidden);
    p.ffn = int(c.intermediate);
    p.heads = int(c.heads);
    p.kv_heads = int(c.kv_heads);
    p.rotary = int(c.rotary_dim);
    p.vocab = int(c.vocab);
    p.window = int(c.sliding_window);
    p.capacity = int(capacity);
    p.activation = int(c.activation);
    p.reference = reference_ ? 1 : 0;
    p.epsilon = c.epsilon;
    p.embedding_scale = c.embedding_scale;
    p.attention_scale = 1.0f / std::sqrt(std::sqrt(static_cast<float>(c.head_dim)));
    p.layer = static_cast<const StepLayer*>(step_layers_.ptr);
    p.embedding = m.embedding;
    p.head = m.head.view;
    p.final_gamma = m.final_norm.gamma;
    p.cosines = rope_cos_.as<float>();
    p.sines = rope_sin_.as<float>();
    p.kv = kv_.as<float>();
    // Algorithmic bytes: int8 weights, f32 row scales and biases of every
    // layer, the FP32 head, plus K and V of every visible key (added per step).
    double bytes = 0;
    for (const Layer& L : m.layers)
        for (const Linear* l : {&L.qkv, &L.o, &L.gate_up, &L.down})
            bytes += double(l->view.rows) * l->view.cols + 8.0 * l->view.rows;
    bytes += 4.0 * double(m.head.view.rows) * m.head.view.cols;
    step_bytes_ = bytes;
    step_kv_bytes_ = 2.0 * 4.0 * c.layers * c.kv_heads * c.head_dim;
    step_blocks_ = blocks;
    // LEAF_DECODE_STEP_ITEM_HEADS=<n>: at least n query heads per exchange
    // wave in each attention item (wider items, fewer blocks; for tests).
    if (const char* heads = std::getenv("LEAF_DECODE_STEP_ITEM_HEADS")) p.item_heads = std::max(1, std::atoi(heads));
    // LEAF_DECODE_STEP_CAPTURE=<file>: run the kernel's capture variant and
    // append every step's integer stages to the file: "LHSC", u32 layers,
    // u32 max_ffn, then x f32 [layers][4][max_ffn], q i8 [layers][4][max_ffn],
    // sx f32 [layers][4], acc i32 [layers][4][2 max_ffn] (StepCapture).
    if (const char* capture = std::getenv("LEAF_DECODE_STEP_CAPTURE")) {
        step_capture_path_ = capture;
        const size_t vec = size_t(c.layers) * 4 * kStepMaxFfn;
        step_capture_.allocate(vec * 4 + vec + size_t(c.layers) * 4 * 4 + 2 * vec * 4);
        hip_check(hipMemset(step_capture_.ptr, 0, step_capture_.bytes), "hipMemset");
        auto* base = static_cast<uint8_t*>(step_capture_.ptr);
        p.capture.x = reinterpret_cast<float*>(base);
        p.capture.q = reinterpret_cast<int8_t*>(base + vec * 4);
        p.capture.sx = reinterpret_cast<float*>(base + vec * 5);
        p.capture.acc = reinterpret_cast<int32_t*>(base + vec * 5 + size_t(c.layers) * 16);
    }
    // LEAF_DECODE_STEP_TRACE=<file>: append every step's phase timeline
    // (blocks x kStepTracePoints u64 stamps of the 100 MHz device clock).
    if (const char* trace = std::getenv("LEAF_DECODE_STEP_TRACE")) {
        step_trace_path_ = trace;
        step_trace_.allocate(size_t(blocks) * kStepTracePoints * 8);
        hip_check(hipMemset(step_trace_.ptr, 0, step_trace_.bytes), "hipMemset");
    }
}

bool Session::step_usable() const {
    if (!step_blocks_ || !step_enabled_) return false;
    const Config& c = model.config;
    const size_t end = length + 1;
    const size_t begin = (c.sliding_window && end > c.sliding_window) ? end - c.sliding_window : 0;
    const int spans = decode_step_spans(int(end - begin));
    if (reference_ && end - begin > size_t(decode_step_reference_keys())) return false;
    return spans <= kStepMaxSpans && size_t(spans) * c.kv_heads <= size_t(step_blocks_);
}

void Session::decode_step(uint32_t id, float* host_logits, uint32_t* argmax) {
    const Config& c = model.config;
    hipStream_t s = stream();
    if (!step_token_valid_ || step_token_ != id) {
        *host_ids_ = id;
        hip_check(hipMemcpyAsync(ids_.ptr, host_ids_, sizeof(uint32_t), hipMemcpyHostToDevice, s), "ids upload");
    }
    if (++step_launch_ >= (1u << 20)) {
        // Epoch tags would repeat: start the exchange words from zero again.
        hip_check(hipMemsetAsync(step_exchange_.ptr, 0, step_exchange_.bytes, s), "hipMemsetAsync");
        if (step_part_local_.ptr)
            hip_check(hipMemsetAsync(step_part_local_.ptr, 0, step_part_local_.bytes, s), "hipMemsetAsync");
        if (step_q_local_.ptr) hip_check(hipMemsetAsync(step_q_local_.ptr, 0, step_q_local_.bytes, s), "hipMemsetAsync");
        step_launch_ = 1;
    }
    StepParams p = step_;
    p.position = int(length);
    p.epoch = step_launch_ << 12;
    p.token = ids_.as<uint32_t>();
    p.host_token = mapped_argmax_;
    p.logits = logits_.as<float>();
    p.trace = step_trace_.as<unsigned long long>();
    *step_host_abort_ = 0;
    const double bytes = step_bytes_ + step_kv_bytes_ * double(length + 1);
    hipError_t launched = hipSuccess;
    timed(Profiler::DecodeStep, bytes, 0, [&] { launched = launch_decode_step(p, step_blocks_, s, step_cooperative_); });
    hip_check(launched, "decode step launch");
    if (host_logits)
        hip_check(hipMemcpyAsync(host_logits, logits_.ptr, size_t(c.vocab) * sizeof(float), hipMemcpyDeviceToHost, s),
                  "logits copy");
    hip_check(hipStreamSynchronize(s), "decode step");
    if (profiler.enabled) profiler.collect();
    if (*step_host_abort_) {
        // A wait timed out: counters and exchange words may be mid-round.
        // Start the next step from zeroed state.
        const unsigned why = *step_host_abort_;
        *step_host_abort_ = 0;
        hip_check(hipMemset(step_exchange_.ptr, 0, step_exchange_.bytes), "hipMemset");
        if (step_part_local_.ptr) hip_check(hipMemset(step_part_local_.ptr, 0, step_part_local_.bytes), "hipMemset");
        if (step_q_local_.ptr) hip_check(hipMemset(step_q_local_.ptr, 0, step_q_local_.bytes), "hipMemset");
        step_token_valid_ = false;
        if (why == 2 && step_.x_part_local) {
            // A block ran off XCD blockIdx % 8: the step (which wrote nothing
            // but its own layers' KV rows for this position) runs again with
            // the XCD-local merge off.  After four such steps in a row it
            // stays off for the session.
            void* part_local = step_.x_part_local;
            void* q_local = step_.x_q_local;
            step_.x_part_local = nullptr;
            step_.x_q_local = nullptr;
            const bool retry_local = ++step_xcd_misses_ < 4;
            ++step_reruns_;
            decode_step(id, host_logits, argmax);
            if (retry_local) {
                step_.x_part_local = static_cast<decltype(step_.x_part_local)>(part_local);
                step_.x_q_local = static_cast<decltype(step_.x_q_local)>(q_local);
            }
            return;
        }
        check(false, "decode step timed out waiting for another block", LH_ERROR_DEVICE);
    }
    if (!step_capture_path_.empty()) {
        std::vector<uint8_t> bytes(step_capture_.bytes);
        hip_check(hipMemcpy(bytes.data(), step_capture_.ptr, bytes.size(), hipMemcpyDeviceToHost), "capture copy");
        if (FILE* f = std::fopen(step_capture_path_.c_str(), "ab")) {
            const uint32_t head[3] = {0x4353484cu, uint32_t(c.layers), uint32_t(kStepMaxFfn)};   // "LHSC"
            std::fwrite(head, 4, 3, f);
            std::fwrite(bytes.data(), 1, bytes.size(), f);
            std::fclose(f);
        }
    }
    if (!step_trace_path_.empty()) {
        std::vector<unsigned long long> stamps(step_trace_.bytes / 8);
        hip_check(hipMemcpy(stamps.data(), step_trace_.ptr, step_trace_.bytes, hipMemcpyDeviceToHost), "trace copy");
        if (FILE* f = std::fopen(step_trace_path_.c_str(), "ab")) {
            std::fwrite(stamps.data(), 8, stamps.size(), f);
            std::fclose(f);
        }
    }
    if (p.x_part_local) step_xcd_misses_ = 0;
    ++step_tokens_;
    const uint32_t next = *host_argmax_;
    if (argmax) *argmax = next;
    step_token_ = next;
    step_token_valid_ = true;
    logits_device = logits_.as<float>();
    logits_count = c.vocab;
    length += 1;
    device_position_valid_ = false;
}

void Session::drop_graphs() {
    for (auto& g : graphs_)
        if (g.second) (void)hipGraphExecDestroy(g.second);
    graphs_.clear();
}

// All kernels of one forward up to the logits.  With position_ptr set (graph
// capture) every position-dependent kernel reads the position from device
// memory and the decode attention runs a fixed number of key spans.
void Session::launch(int M, size_t position, bool all_logits, const int* position_ptr, int spans) {
    const Config& c = model.config;
    hipStream_t s = stream();
    const int h = int(c.hidden), dim = int(c.head_dim);
    const int qw = int(c.qwidth()), kvw = int(c.kvwidth());
    const int qkv_width = qw + 2 * kvw;
    float* hidden = hidden_.as<float>();
    float* normed = normed_.as<float>();
    launch_embedding(model.embedding, model.has_positions ? &model.positions : nullptr, ids_.as<uint32_t>(), M,
                     int((position_ptr ? 0 : position) + c.position_offset), c.embedding_scale, hidden, s,
                     position_ptr);
    const float scale = 1.0f / std::sqrt(std::sqrt(static_cast<float>(c.head_dim)));
    const size_t plane = size_t(c.kv_heads) * capacity * dim;

    for (uint32_t layer = 0; layer < c.layers; ++layer) {
        const Layer& L = model.layers[layer];
        const bool last = layer + 1 == c.layers;
        // ---- attention block
        float* qkv = qkv_.as<float>();
        float* keys = kv_.as<float>() + size_t(layer) * 2 * plane;
        float* values = keys + plane;
        // Single-token q|k|v: the GEMV normalizes its input itself (integer or
        // FP weights; FP only with the fast kernels).  In reference order the
        // fused integer GEMV sums the norm in column order (and the RoPE pair
        // epilogue is the rope kernel's arithmetic).
        const bool fuse_in = M == 1 && L.stacked_qkv && !L.qkv.input_scale &&
                             (model.integer_linear(L.qkv) || !reference_);
        NormView input_norm = L.input_norm;
        input_norm.sequential = reference_ ? 1 : 0;
        // Single-token W8A8: one launch normalizes, quantizes, projects q|k|v,
        // rotates and appends k, v to the cache.
        PairEpilogue rope;
        rope.mode = kPairRopeKv;
        rope.heads = int(c.heads); rope.kv_heads = int(c.kv_heads); rope.dim = dim;
        rope.rotary = c.position_kind == 0 ? int(c.rotary_dim) : 0; rope.position = int(position);
        rope.capacity = int(capacity); rope.cosines = rope_cos_.as<float>(); rope.sines = rope_sin_.as<float>();
        rope.q_heads = q_heads_.as<float>(); rope.keys = keys; rope.values = values;
        rope.position_ptr = position_ptr;
        const bool fuse_rope = fuse_in && !c.qk_norm && dim % 2 == 0 &&
                               linear_fuses([&] { LinearCall t = make_call(L.qkv, hidden, M, qkv, kStore, &input_norm);
                                                  t.pair = rope; return t; }());
        if (fuse_rope) {
            run_linear(L.qkv, hidden, M, qkv, kStore, &input_norm, &rope);
        } else if (fuse_in) {
            run_linear(L.qkv, hidden, M, qkv, kStore, &input_norm);
        } else if (L.stacked_qkv &&
                   (prequantizes(L.qkv, M) || reference_prequantizes(L.qkv, M, L.input_norm, h))) {
            // norm + per-token quantization in one launch, then the GEMM
            norm_prequantize(hidden, M, h, L.input_norm);
            run_linear(L.qkv, nullptr, M, qkv, kStore, nullptr, nullptr, true);
        } else {
            norm(hidden, M, h, L.input_norm, normed);
            if (L.stacked_qkv) {
                run_linear(L.qkv, normed, M, qkv, kStore, nullptr);
            } else {
                // separate projections into a [M, q|k|v] staging layout
                float* q = q_heads_.as<float>();   // reuse as [M, qw] staging
                float* k = attn_.as<float>();      // [M, kvw]
                float* v = attn_proj_.as<float>(); // [M, kvw]
                run_linear(L.qkv, normed, M, q, kStore, nullptr);
                run_linear(L.k, normed, M, k, kStore, nullptr);
                run_linear(L.v, normed, M, v, kStore, nullptr);
                // one strided copy per matrix into the [M, q|k|v] rows
                const size_t pitch = size_t(qkv_width) * 4;
                hip_check(hipMemcpy2DAsync(qkv, pitch, q, size_t(qw) * 4, size_t(qw) * 4, M,
                                           hipMemcpyDeviceToDevice, s), "qkv staging");
                hip_check(hipMemcpy2DAsync(qkv + qw, pitch, k, size_t(kvw) * 4, size_t(kvw) * 4, M,
                                           hipMemcpyDeviceToDevice, s), "qkv staging");
                hip_check(hipMemcpy2DAsync(qkv + qw + kvw, pitch, v, size_t(kvw) * 4, size_t(kvw) * 4, M,
                                           hipMemcpyDeviceToDevice, s), "qkv staging");
            }
        }
        if (c.qk_norm) {
            // Q/K RMSNorm over each head's dim values (decoder.cpp:1327-1331).
            NormView qn{L.q_norm, nullptr, c.epsilon, 0, model.accurate ? 1 : 0};
            NormView kn{L.k_norm, nullptr, c.epsilon, 0, model.accurate ? 1 : 0};
            // every token's heads in one launch per tensor: rows of `dim`
            // values, `heads` of them per token, tokens qkv_width apart
            norm(qkv, M * int(c.heads), dim, qn, qkv, int(c.heads), size_t(qkv_width));
            norm(qkv + qw, M * int(c.kv_heads), dim, kn, qkv + qw, int(c.kv_heads), size_t(qkv_width));
        }
        RopeKvCall rk;
        rk.qkv = qkv; rk.ld = qkv_width; rk.q_offset = 0; rk.k_offset = qw; rk.v_offset = qw + kvw;
        rk.tokens = M; rk.heads = int(c.heads); rk.kv_heads = int(c.kv_heads); rk.dim = dim;
        rk.rotary = c.position_kind == 0 ? int(c.rotary_dim) : 0;
        rk.position = int(position);
        rk.position_ptr = position_ptr;
        rk.cosines = rope_cos_.as<float>(); rk.sines = rope_sin_.as<float>();
        rk.q_heads = q_heads_.as<float>(); rk.keys = keys; rk.values = values; rk.capacity = int(capacity);
        if (!fuse_rope) timed(Profiler::Other, 0, 0, [&] { launch_rope_kv(rk, s); });

        // After the last layer's KV append only the final row reaches the
        // head (decoder.cpp:1375-1387 trims the MLP the same way; here the
        // attention output, projections and MLP of earlier rows are skipped too:
        // rows are independent, so the last row's values do not change).
        // In reference order the kept rows are the last group of four, so an
        // FP linear sees the token groups the CPU's linear forms (decoder.cpp:1217-1228).
        const bool trim = last && !all_logits && M > 1;
        const int first_row = trim ? (reference_ ? 4 * ((M - 1) / 4) : M - 1) : 0;
        const int rows = M - first_row;
        AttentionCall at;
        at.q_heads = q_heads_.as<float>(); at.keys = keys; at.values = values; at.out = attn_.as<float>();
        at.heads = int(c.heads); at.kv_heads = int(c.kv_heads); at.tokens = M; at.position = int(position);
        at.dim = dim; at.capacity = int(capacity); at.window = int(c.sliding_window); at.scale = scale;
        at.partial = partial_.as<float>(); at.partial_capacity = int(partial_.bytes / sizeof(float));
        at.counters = counters_.as<unsigned>();
        at.position_ptr = position_ptr;
        at.spans = spans;
        {
            // KV bytes read: keys and values of every visible position, per query row.
            const double kv_bytes = 2.0 * 4.0 * c.kv_heads * dim * double(position + M) * (M == 1 ? 1 : 0.5 * M);
            // Operations: q.k and p.v (2 flops each per dimension) over the keys
            // each query row sees (position + t + 1, at most the window).
            double visible = 0.0;
            for (int t = 0; t < M; ++t) {
                double keys = double(position) + t + 1;
                if (c.sliding_window) keys = std::min(keys, double(c.sliding_window));
                visible += keys;
            }
            const double attention_ops = 4.0 * c.heads * dim * visible;
            if (reference_) {
                int keys = position_ptr ? int(capacity) : int(position) + M;
                if (c.sliding_window) keys = std::min(keys, int(c.sliding_window));
                check(keys <= reference_keys_, "reference-order attention: too many keys for one query",
                      LH_ERROR_UNSUPPORTED);
                timed(Profiler::Attention, kv_bytes, attention_ops, [&] {
                    check(launch_attention_reference_order(at, keys, s), "attention launch rejected",
                          LH_ERROR_UNSUPPORTED);
                });
            } else {
                timed(Profiler::Attention, kv_bytes, attention_ops,
                      [&] { check(launch_attention(at, s), "attention launch rejected", LH_ERROR_UNSUPPORTED); });
            }
        }
        const float* attn_rows = attn_.as<float>() + size_t(first_row) * qw;
        float* hid = hidden + size_t(first_row) * h;
        float* attn_proj = attn_proj_.as<float>();
        if (!c.parallel) {
            run_linear(L.o, attn_rows, rows, hid, kAccumulate, nullptr);       // hidden += o(attn) + b
        } else {
            run_linear(L.o, attn_rows, rows, attn_proj, kStore, nullptr);
        }
        // ---- MLP block
        float* gate_up = gate_up_.as<float>();
        float* act = act_.as<float>();
        const int f = int(c.intermediate);
        if (c.gated) {
            const bool fuse_post = rows == 1 && L.stacked_gate_up && !L.gate_up.input_scale &&
                                   (model.integer_linear(L.gate_up) || !reference_);
            NormView post_norm = L.post_norm;
            post_norm.sequential = reference_ ? 1 : 0;
            PairEpilogue gated;
            gated.mode = kPairGated;
            gated.width = f;
            gated.activation = int(c.activation);
            gated.act = act;
            gated.reference = reference_ ? 1 : 0;
            const bool fuse_act = fuse_post &&
                                  linear_fuses([&] { LinearCall t = make_call(L.gate_up, hid, rows, gate_up, kStore,
                                                                              &post_norm);
                                                     t.pair = gated; return t; }());
            if (fuse_act) {
                run_linear(L.gate_up, hid, rows, gate_up, kStore, &post_norm, &gated);
            } else if (fuse_post) {
                run_linear(L.gate_up, hid, rows, gate_up, kStore, &post_norm);
            } else if (L.stacked_gate_up &&
                       (prequantizes(L.gate_up, rows) || reference_prequantizes(L.gate_up, rows, L.post_norm, h))) {
                norm_prequantize(hid, rows, h, L.post_norm);
                run_linear(L.gate_up, nullptr, rows, gate_up, kStore, nullptr, nullptr, true);
            } else {
                norm(hid, rows, h, L.post_norm, normed);
                if (L.stacked_gate_up) {
                    run_linear(L.gate_up, normed, rows, gate_up, kStore, nullptr);
                } else {
                    float* g = proj_.as<float>();
                    run_linear(L.gate_up, normed, rows, act, kStore, nullptr);   // gate -> act (staging)
                    run_linear(L.up, normed, rows, g, kStore, nullptr);          // up -> proj (staging)
                    const size_t pitch = size_t(2 * f) * 4, width = size_t(f) * 4;
                    hip_check(hipMemcpy2DAsync(gate_up, pitch, act, width, width, rows, hipMemcpyDeviceToDevice, s),
                              "gate staging");
                    hip_check(hipMemcpy2DAsync(gate_up + f, pitch, g, width, width, rows, hipMemcpyDeviceToDevice, s),
                              "up staging");
                }
            }
            if (!fuse_act && !prequantizes(L.down, rows) && !reference_prequantizes_down(L, rows))
                timed(Profiler::Other, 0, 0, [&] { activation(gate_up, rows, f, 1, act); });
        } else {
            // ungated MLP: a single-token FP up projection normalizes its input
            // itself and stores activate(value) straight into act
            PairEpilogue activated;
            activated.mode = kPairActivation;
            activated.activation = int(c.activation);
            const bool fuse_up = rows == 1 && !reference_ && !model.integer_linear(L.up) &&
                                 linear_fuses([&] { LinearCall t = make_call(L.up, hid, rows, act, kStore,
                                                                             &L.post_norm);
                                                    t.pair = activated; return t; }());
            if (fuse_up) {
                run_linear(L.up, hid, rows, act, kStore, &L.post_norm, &activated);
            } else {
                norm(hid, rows, h, L.post_norm, normed);
                run_linear(L.up, normed, rows, gate_up, kStore, nullptr);
                activation(gate_up, rows, f, 0, act);
            }
        }
        const bool down_q = c.gated && prequantizes(L.down, rows) &&
                            !(rows == 1 && model.integer_linear(L.gate_up) && L.stacked_gate_up);
        const bool ref_down_q = reference_prequantizes_down(L, rows);
        if (down_q) {
            // the gated activation and its quantization in one launch
            timed(Profiler::Other, 0, 0, [&] {
                launch_activation_quantize(gate_up, rows, f, 1, int(c.activation), xq_.as<int8_t>(), xs_.as<float>(), s);
            });
        } else if (ref_down_q) {
            timed(Profiler::Other, 0, 0, [&] {
                check(launch_activation_quantize_reference_order(gate_up, rows, f, 1, int(c.activation),
                                                                 xq_.as<int8_t>(), xs_.as<float>(), s),
                      "reference-order activation rejected", LH_ERROR_UNSUPPORTED);
            });
        }
        if (!c.parallel) {
            run_linear(L.down, act, rows, hid, kAccumulate, nullptr, nullptr, down_q || ref_down_q);   // hidden += down(act) + b
        } else {
            float* proj = proj_.as<float>();
            run_linear(L.down, act, rows, proj, kStore, nullptr, nullptr, down_q || ref_down_q);
            launch_residual(hid, proj, attn_proj, rows * h, s);              // hidden += proj + attn_proj
        }
        if (trim) hidden = hid + size_t(rows - 1) * h;   // the final norm and head see only the last row
    }
    const int head_rows = all_logits ? M : 1;
    // `hidden` now points at the rows the head reads: all rows, or the last one.
    const float* x = hidden;
    // a single-row FP head normalizes its input itself (fast kernels)
    const bool fuse_head = c.final_norm && head_rows == 1 && !reference_ && !model.integer_linear(model.head) &&
                           linear_fuses(make_call(model.head, hidden, 1, logits_.as<float>(), kStore,
                                                  &model.final_norm));
    if (fuse_head) {
        run_linear(model.head, hidden, 1, logits_.as<float>(), kStore, &model.final_norm);
        return;
    }
    if (c.final_norm) {
        norm(hidden, head_rows, h, model.final_norm, normed);
        x = normed;
    }
    run_linear(model.head, x, head_rows, logits_.as<float>(), kStore, nullptr);
}

}  // namespace leafhip
