// Host runtime of the MI355X decoder: artifact validation, device memory plan,
// decoding sessions.  Internal to libleafhip; the public surface is include/leafhip.h.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/leafhip.h"
#include "decode_step.h"
#include "kernels.h"

namespace leafhip {

// An error carrying the C ABI status code.
struct Error : std::runtime_error {
    lh_status code;
    Error(lh_status c, const std::string& message) : std::runtime_error(message), code(c) {}
};

// Reference-style check (decoder.cpp:86-88): "Leaf decoder: <message>".
inline void check(bool ok, const std::string& message, lh_status code = LH_ERROR_ARTIFACT) {
    if (!ok) throw Error(code, "Leaf decoder: " + message);
}
void hip_check(hipError_t status, const char* what);

// A numerics mode (LH_NUMERICS_*) resolved: whether the kernels follow the CPU
// path's order, and whether grouped INT8 sums take quant_vnni_tile's form.
// DEFAULT reads LEAF_GPU_NUMERICS ("fast", "reference", "reference-avx2",
// "reference-vnni"); unset, it is REFERENCE for a decoder with int8
// activations (a one-ulp change upstream of an int8 quantization moves the
// whole bin, so only the CPU's order reproduces its tokens) and FAST
// otherwise.  REFERENCE asks this host what the CPU path would (AVX2, FMA and
// AVX-VNNI present, LEAF_DISABLE_VNNI unset or empty: decoder.cpp:773,
// 780-782).  Throws on an unknown mode.
struct NumericsMode {
    bool reference = false;
    bool vnni = false;
};
NumericsMode resolve_numerics(uint32_t numerics, bool integer_activations = false);

struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t n) { allocate(n); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    ~DeviceBuffer() { release(); }
    void allocate(size_t n);
    void release();
    template <typename T> T* as() const { return static_cast<T*>(ptr); }
};

// Device memory that bypasses the L2 caches (hipDeviceMallocUncached), for
// words that blocks on different XCDs exchange within one kernel: a cached
// poll can keep reading a stale L2 line long after another XCD stored the
// word.  Allocations are pooled per device and never returned to HIP, since
// memory of this kind must stay allocated once a kernel has read it.
struct UncachedBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    int device = -1;
    UncachedBuffer() = default;
    UncachedBuffer(const UncachedBuffer&) = delete;
    UncachedBuffer& operator=(const UncachedBuffer&) = delete;
    ~UncachedBuffer() { release(); }
    void allocate(size_t n);   // on the current device, from the pool when it can
    void release();            // back to the pool
    template <typename T> T* as() const { return static_cast<T*>(ptr); }
};

struct Context {
    int device = 0;
    hipStream_t stream = nullptr;
    ~Context();
};

// One tensor of the artifact's table (decoder.cpp:858-904).
struct TensorRecord {
    std::string name;
    uint32_t rows = 0, cols = 0, bits = 0, group = 0;
    const uint8_t* data = nullptr;
    const float* scales = nullptr;
    uint64_t size = 0, scale_count = 0;
};

// Header semantics (Appendix A layout; decoder.cpp:795-857).
struct Config {
    uint32_t version = 0, hidden = 0, intermediate = 0, heads = 0, kv_heads = 0, layers = 0, vocab = 0;
    uint32_t max_positions = 0, eos = 0, head_dim = 0, sliding_window = 0;
    float theta = 0, epsilon = 0, embedding_scale = 1;
    uint32_t norm_kind = 0, activation = 0, position_kind = 0, gated = 0, parallel = 0, rotary_dim = 0;
    uint32_t position_offset = 0, final_norm = 0, qk_norm = 0;
    std::vector<float> rope_frequencies;
    std::vector<uint32_t> eos_tokens;
    uint32_t qwidth() const { return heads * head_dim; }
    uint32_t kvwidth() const { return kv_heads * head_dim; }
};

// A linear layer on the device: possibly several artifact matrices stacked
// along rows (q|k|v, gate|up) so one launch streams them all.
struct Linear {
    WeightView view;
    const float* input_scale = nullptr;   // SmoothQuant factors (decoder.cpp:1008-1019), device
    bool present = false;
};

struct Layer {
    NormView input_norm, post_norm;
    Linear qkv;                 // [q | k | v] when stackable, else q only
    Linear k, v;                // used when q, k, v could not be stacked
    bool stacked_qkv = false;
    Linear o, gate_up, up, down;
    bool stacked_gate_up = false;
    const float* q_norm = nullptr;
    const float* k_norm = nullptr;
};

class Model {
public:
    static std::unique_ptr<Model> load(Context& context, const uint8_t* data, size_t size, uint32_t activation_bits,
                                       uint32_t fp32_math);
    Context& context;
    Config config;
    uint32_t activation_bits = 32;
    bool accurate = false;
    uint64_t artifact_bytes = 0;
    uint32_t source_bf16_tensors = 0, quantized_tensors = 0;
    DeviceBuffer weights;
    std::vector<Layer> layers;
    WeightView embedding, positions;
    Linear head;
    NormView final_norm;
    bool has_positions = false;

    explicit Model(Context& c) : context(c) {}
    bool integer_linear(const Linear& l) const {
        return activation_bits == 8 && (l.view.bits == 8 || l.view.bits == 4);
    }
};

// Per-kernel-class device timing (HIP events on the session stream).
class Profiler {
public:
    enum Kind { GemvW8A8, GemvFp, GemmW8A8, GemmFp, Attention, Other, DecodeStep, Count };
    static const char* name(int kind);
    bool enabled = false;
    void begin(hipStream_t stream);
    void end(hipStream_t stream, int kind, double bytes, double operations);
    void collect();          // after the stream synchronized
    struct Total { uint64_t launches = 0; double ms = 0, bytes = 0, ops = 0; };
    Total totals[Count];
    ~Profiler();
private:
    struct Pending { int kind; double bytes, ops; size_t event; };
    std::vector<hipEvent_t> events_;
    std::vector<Pending> pending_;
    size_t used_ = 0;
    hipEvent_t next_event();
};

class Session {
public:
    Profiler profiler;
    // numerics: LH_NUMERICS_* (DEFAULT reads LEAF_GPU_NUMERICS).
    Session(Model& model, uint32_t max_context, uint32_t max_prefill, uint32_t numerics = LH_NUMERICS_DEFAULT);
    // Whether the kernels follow the CPU reference's floating-point order.
    bool reference_order() const { return reference_; }
    void reset() {
        length = 0;
        device_position_valid_ = false;
        step_token_valid_ = false;
    }
    size_t cache_tokens() const { return length; }
    // Tokens produced by the persistent decode step since the session began;
    // of those, steps run a second time on the memory exchange path after a
    // block ran off its XCD; whether the XCD-local exchange is still on.
    uint64_t step_tokens() const { return step_tokens_; }
    uint64_t step_reruns() const { return step_reruns_; }
    bool step_xcd_local() const { return step_.x_part_local != nullptr; }
    // Decoder::forward_into (decoder.cpp:1282-1444)
    void forward(const uint32_t* ids, size_t count, bool all_logits, float* host_logits, size_t capacity,
                 uint32_t* argmax);
    Model& model;
    size_t length = 0;
    uint32_t capacity = 0;
    uint32_t planned = 0;
    const float* logits_device = nullptr;
    size_t logits_count = 0;

private:
    void plan(uint32_t tokens, bool all_logits);
    void validate(const uint32_t* ids, size_t count, bool all_logits, float* host_logits, size_t host_capacity) const;
    void launch(int M, size_t position, bool all_logits, const int* position_ptr, int spans);
    bool graph_decode_ok() const;
    void decode_graphed(uint32_t id, bool upload_id, float* host_logits, uint32_t* argmax);
    // Persistent single-token step (decode_step.hip) for W8A8 decoders it fits.
    void step_prepare();
    bool step_usable() const;
    void decode_step(uint32_t id, float* host_logits, uint32_t* argmax);
    int step_blocks_ = 0;
    bool step_enabled_ = true;
    bool step_cooperative_ = true;   // LEAF_DECODE_STEP_COOPERATIVE=0: plain launch
    bool step_token_valid_ = false;   // ids_[0] holds the previous step's argmax
    uint32_t step_token_ = 0;
    unsigned step_launch_ = 0;
    int step_xcd_misses_ = 0;        // consecutive steps re-run after an XCD mapping mismatch
    uint64_t step_tokens_ = 0;       // tokens the persistent step produced
    uint64_t step_reruns_ = 0;       // of those, steps run again on the memory exchange path
    double step_bytes_ = 0;          // algorithmic bytes of one step, without KV
    double step_kv_bytes_ = 0;       // KV bytes per visible key
    StepParams step_;
    DeviceBuffer step_layers_, step_trace_, step_part_local_, step_q_local_, step_capture_;
    std::string step_capture_path_;
    UncachedBuffer step_exchange_;
    std::string step_trace_path_;
    unsigned* step_host_abort_ = nullptr;
    void drop_graphs();
    std::map<int, hipGraphExec_t> graphs_;
    bool graphs_enabled_ = true;
    bool device_position_valid_ = false;
    DeviceBuffer position_;
    int* host_position_ = nullptr;
    uint32_t* mapped_argmax_ = nullptr;
    LinearCall make_call(const Linear& l, const float* x, int tokens, float* y, int epilogue,
                         const NormView* fuse_norm);
    void run_linear(const Linear& l, const float* x, int tokens, float* y, int epilogue, const NormView* fuse_norm,
                    const PairEpilogue* pair = nullptr, bool prequantized = false);
    // Whether a multi-token integer linear can take its input quantized by a
    // fused norm or activation kernel (into xq_ / xs_).
    bool prequantizes(const Linear& l, int tokens) const;
    bool reference_prequantizes(const Linear& l, int tokens, const NormView& n, int width) const;
    void norm_prequantize(const float* x, int rows, int width, const NormView& n);
    bool reference_prequantizes_down(const Layer& L, int rows) const;
    bool fuse_quantize_ = true;   // LEAF_PREFILL_FUSE=0 turns the fused norm / activation quantization off
    bool reference_ = false;      // reference-order numerics (LH_NUMERICS_REFERENCE)
    bool reference_vnni_ = false; // grouped INT8 sums as quant_vnni_tile (two roundings)
    int reference_keys_ = 0;      // most keys one query may see in reference order
    // rows_per_group > 0: rows come in groups that many long, group_stride
    // floats apart (Q/K norm over the heads of every token's q|k|v row)
    void norm(const float* x, int rows, int width, const NormView& n, float* y, int rows_per_group = 0,
              size_t group_stride = 0);
    void activation(const float* gate_up, int rows, int width, int gated, float* act);
    template <typename F> void timed(int kind, double bytes, double ops, F&& launch) {
        if (profiler.enabled) profiler.begin(stream());
        launch();
        if (profiler.enabled) profiler.end(stream(), kind, bytes, ops);
    }
    hipStream_t stream() const { return model.context.stream; }
    DeviceBuffer kv_, rope_cos_, rope_sin_;
    DeviceBuffer hidden_, normed_, qkv_, q_heads_, attn_, attn_proj_, gate_up_, act_, proj_, logits_, xq_, xs_;
    DeviceBuffer ids_, argmax_, argmax_scratch_, partial_, scaled_, counters_, split_;
    uint32_t logits_rows_ = 0;
    uint32_t* host_ids_ = nullptr;   // pinned staging for token ids
    uint32_t* host_argmax_ = nullptr;
public:
    ~Session();
};

}  // namespace leafhip
