// Host runtime: LEAFDC validation and upload, session memory plan, forward.
//
// Validation mirrors Decoder::Impl::Impl (engine/src/decoder.cpp:767-972) check
// for check, with the same messages, so an artifact the CPU runtime rejects is
// rejected here too, before anything reaches the device.
#include "runtime.h"

#include <mutex>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <mutex>

namespace leafhip {

void hip_check(hipError_t status, const char* what) {
    if (status != hipSuccess) {
        const lh_status code = status == hipErrorOutOfMemory ? LH_ERROR_OUT_OF_MEMORY : LH_ERROR_DEVICE;
        throw Error(code, std::string("Leaf decoder: HIP error in ") + what + ": " + hipGetErrorString(status));
    }
}

void DeviceBuffer::allocate(size_t n) {
    release();
    if (n == 0) return;
    hip_check(hipMalloc(&ptr, n), "hipMalloc");
    bytes = n;
}

void DeviceBuffer::release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
}

namespace {
struct UncachedBlock {
    int device;
    void* ptr;
    size_t bytes;
};
std::mutex uncached_mutex;
std::vector<UncachedBlock> uncached_free;   // released blocks, kept for reuse
}  // namespace

void UncachedBuffer::allocate(size_t n) {
    release();
    if (n == 0) return;
    n = (n + 65535) / 65536 * 65536;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    {
        std::lock_guard<std::mutex> lock(uncached_mutex);
        size_t best = uncached_free.size();
        for (size_t i = 0; i < uncached_free.size(); ++i) {
            const UncachedBlock& f = uncached_free[i];
            if (f.device == device && f.bytes >= n && (best == uncached_free.size() || f.bytes < uncached_free[best].bytes))
                best = i;
        }
        if (best < uncached_free.size()) {
            ptr = uncached_free[best].ptr;
            bytes = uncached_free[best].bytes;
            uncached_free.erase(uncached_free.begin() + best);
            return;
        }
    }
    hip_check(hipExtMallocWithFlags(&ptr, n, hipDeviceMallocUncached), "hipExtMallocWithFlags(uncached)");
    bytes = n;
}

void UncachedBuffer::release() {
    if (!ptr) return;
    std::lock_guard<std::mutex> lock(uncached_mutex);
    uncached_free.push_back({device, ptr, bytes});
    ptr = nullptr;
    bytes = 0;
}

Context::~Context() {
    if (stream) (void)hipStreamDestroy(stream);
}

namespace {

// Little-endian reader over the artifact bytes (host_support.h:94-114).
struct Reader {
    const uint8_t* data;
    size_t size;
    size_t position = 0;
    void require(size_t length) const {
        if (!(position <= size && length <= size - position))
            throw Error(LH_ERROR_ARTIFACT, "Leaf runtime: truncated artifact metadata");
    }
    uint32_t u32() {
        require(4);
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) v |= uint32_t(data[position++]) << (8 * i);
        return v;
    }
    uint64_t u64() {
        const uint64_t low = u32();
        return low | (uint64_t(u32()) << 32);
    }
    float f32() {
        const uint32_t bits = u32();
        float v;
        std::memcpy(&v, &bits, 4);
        return v;
    }
    std::string string() {
        const uint32_t length = u32();
        require(length);
        std::string v(reinterpret_cast<const char*>(data + position), length);
        position += length;
        return v;
    }
};

// Tensor roles v6 may store as BF16 (decoder.cpp:93-115).
bool bf16_matrix_role(const std::string& name, uint32_t rows, uint32_t layers) {
    if (rows <= 1) return false;
    if (name == "lm_head.weight" || name == "model.embed_tokens.weight" || name == "model.position_embeddings.weight")
        return true;
    const std::string prefix = "model.layers.";
    if (name.compare(0, prefix.size(), prefix) != 0) return false;
    const size_t end = name.find('.', prefix.size());
    if (end == std::string::npos || end == prefix.size() || (end > prefix.size() + 1 && name[prefix.size()] == '0'))
        return false;
    uint64_t layer = 0;
    for (size_t i = prefix.size(); i < end; ++i) {
        if (name[i] < '0' || name[i] > '9') return false;
        layer = layer * 10 + uint64_t(name[i] - '0');
        if (layer > std::numeric_limits<uint32_t>::max()) return false;
    }
    if (layer >= layers) return false;
    static const char* roles[] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                                  "self_attn.o_proj.weight", "mlp.up_proj.weight", "mlp.gate_proj.weight",
                                  "mlp.down_proj.weight"};
    const std::string role = name.substr(end + 1);
    for (const char* r : roles)
        if (role == r) return true;
    return false;
}

// Device memory plan: host segments laid out in one allocation.
struct Plan {
    struct Segment { const void* source; size_t bytes; size_t offset; };
    std::vector<Segment> segments;
    size_t total = 0;
    size_t add(const void* source, size_t bytes, size_t align = 256) {
        total = (total + align - 1) / align * align;
        segments.push_back({source, bytes, total});
        total += bytes;
        return total - bytes;
    }
};

}  // namespace

std::unique_ptr<Model> Model::load(Context& context, const uint8_t* data, size_t size, uint32_t activation_bits,
                                   uint32_t fp32_math) {
    check(activation_bits == 8 || activation_bits == 32, "activation bits must be 8 or 32", LH_ERROR_INVALID_ARGUMENT);
    check(fp32_math <= 1, "invalid FP32 math policy", LH_ERROR_INVALID_ARGUMENT);
    auto model = std::make_unique<Model>(context);
    Model& m = *model;
    Config& c = m.config;
    m.activation_bits = activation_bits;
    m.artifact_bytes = size;
    Reader reader{data, size};
    reader.require(8);
    char magic[9] = {};
    std::memcpy(magic, data, 8);
    const bool window_format = std::memcmp(magic, "LEAFDC03", 8) == 0;
    const bool multi_eos_format = std::memcmp(magic, "LEAFDC04", 8) == 0;
    bool bf16_io_format = std::memcmp(magic, "LEAFDC05", 8) == 0;
    bool bf16_matrix_format = std::memcmp(magic, "LEAFDC06", 8) == 0;
    const bool operator_format = std::memcmp(magic, "LEAFDC07", 8) == 0;
    check(operator_format || bf16_io_format || bf16_matrix_format || multi_eos_format || window_format ||
              std::memcmp(magic, "LEAFDC02", 8) == 0,
          "unsupported artifact magic");
    reader.position = 8;
    c.version = reader.u32();
    const uint32_t expected = operator_format ? 7 : bf16_matrix_format ? 6 : bf16_io_format ? 5 : multi_eos_format ? 4
                              : window_format ? 3 : 2;
    check(c.version == expected, "unsupported decoder artifact version");
    const uint32_t count = reader.u32();
    const uint64_t base = reader.u64();
    c.hidden = reader.u32(); c.intermediate = reader.u32(); c.heads = reader.u32(); c.kv_heads = reader.u32();
    c.layers = reader.u32(); c.vocab = reader.u32(); c.max_positions = reader.u32(); c.eos = reader.u32();
    c.head_dim = reader.u32(); c.sliding_window = reader.u32();
    check(operator_format || bf16_io_format || bf16_matrix_format || multi_eos_format ||
              (window_format ? c.sliding_window > 0 : c.sliding_window == 0),
          "invalid sliding-window artifact configuration");
    c.theta = reader.f32(); c.epsilon = reader.f32();
    c.norm_kind = reader.u32(); c.activation = reader.u32(); c.position_kind = reader.u32();
    c.gated = reader.u32(); c.parallel = reader.u32(); c.rotary_dim = reader.u32();
    c.position_offset = reader.u32(); c.final_norm = reader.u32(); c.embedding_scale = reader.f32();
    check(c.hidden && c.intermediate && c.heads && c.kv_heads && c.layers && c.vocab && c.head_dim && c.max_positions &&
              c.heads % c.kv_heads == 0 && uint64_t(c.heads) * c.head_dim <= std::numeric_limits<uint32_t>::max() &&
              c.norm_kind <= 1 && c.activation <= 3 && c.position_kind <= 2 && c.gated <= 1 && c.parallel <= 1 &&
              c.rotary_dim <= c.head_dim && c.rotary_dim % 2 == 0 && (c.position_kind != 0 || c.rotary_dim > 0) &&
              c.final_norm <= 1 && std::isfinite(c.embedding_scale) && c.embedding_scale > 0 &&
              std::isfinite(c.theta) && c.theta > 0 && std::isfinite(c.epsilon) && c.epsilon > 0,
          "invalid decoder configuration");
    const uint64_t qwidth = uint64_t(c.heads) * c.head_dim;
    const uint64_t widest = std::max<uint64_t>({c.hidden, qwidth, c.intermediate, c.vocab, c.max_positions});
    check(c.max_positions <= std::numeric_limits<size_t>::max() - c.position_offset &&
              c.max_positions <= std::numeric_limits<size_t>::max() / sizeof(float) / widest,
          "decoder workspace dimensions overflow address space");
    check(base % 64 == 0 && base <= size && count <= size / 56, "invalid tensor table");
    check(c.eos < c.vocab || c.eos == 0xffffffffu, "invalid EOS token");
    if (operator_format) {
        check(reader.position <= base && base - reader.position >= 12, "truncated decoder operator metadata");
        const uint32_t storage = reader.u32(), qk = reader.u32(), frequencies = reader.u32();
        check(storage == 0 || storage == 5 || storage == 6, "invalid decoder storage policy");
        check((qk || frequencies) && qk <= 1 && c.position_kind == 0 && (!qk || c.norm_kind == 0) &&
                  (!frequencies || frequencies == c.rotary_dim / 2) && frequencies <= (base - reader.position) / 4,
              "invalid decoder operator metadata");
        bf16_io_format = storage == 5;
        bf16_matrix_format = storage == 6;
        c.qk_norm = qk;
        for (uint32_t i = 0; i < frequencies; ++i) {
            const float f = reader.f32();
            check(std::isfinite(f) && f > 0 && f <= 1, "invalid static RoPE frequency");
            c.rope_frequencies.push_back(f);
        }
    }
    check(c.qk_norm || qwidth == c.hidden, "invalid decoder head geometry");
    check(c.head_dim <= 256, "head dimensions above 256 are not supported on this device path", LH_ERROR_UNSUPPORTED);
    const bool bf16_format = bf16_io_format || bf16_matrix_format;
    check(!bf16_format || activation_bits == 32, "source BF16 storage requires FP32 activations",
          LH_ERROR_INVALID_ARGUMENT);
    if (multi_eos_format || bf16_format || operator_format) {
        check(reader.position <= base && base - reader.position >= 4, "truncated EOS metadata");
        const uint32_t eos_count = reader.u32();
        check((bf16_format || operator_format || eos_count >= 2) && eos_count <= 1024 && eos_count <= c.vocab &&
                  reader.position <= base && eos_count <= (base - reader.position) / 4,
              "invalid multi-EOS token count");
        for (uint32_t i = 0; i < eos_count; ++i) {
            const uint32_t token = reader.u32();
            check(token < c.vocab && std::find(c.eos_tokens.begin(), c.eos_tokens.end(), token) == c.eos_tokens.end(),
                  "invalid or duplicate EOS token");
            c.eos_tokens.push_back(token);
        }
        check(c.eos_tokens.empty() ? c.eos == 0xffffffffu : c.eos == c.eos_tokens.front(),
              "multi-EOS primary token mismatch");
    } else if (c.eos < c.vocab) {
        c.eos_tokens.push_back(c.eos);
    }

    std::unordered_map<std::string, TensorRecord> tensors;
    for (uint32_t i = 0; i < count; ++i) {
        TensorRecord t;
        t.name = reader.string();
        const uint32_t rank = reader.u32();
        t.rows = reader.u32(); t.cols = reader.u32(); t.bits = reader.u32(); t.group = reader.u32();
        const uint64_t offset = reader.u64();
        t.size = reader.u64();
        const uint64_t scale_offset = reader.u64();
        t.scale_count = reader.u64();
        check(rank == 2 && t.rows && t.cols &&
                  (t.bits == 32 || t.bits == 8 || t.bits == 4 ||
                   (bf16_format && t.bits == 16 &&
                    (bf16_matrix_format ? bf16_matrix_role(t.name, t.rows, c.layers)
                                        : t.name == "lm_head.weight" || t.name == "model.embed_tokens.weight"))),
              "invalid tensor " + t.name);
        if (bf16_format) check(t.bits == 32 || t.bits == 16, "source BF16 storage cannot mix quantized weights");
        if (bf16_matrix_format)
            check(t.scale_count == 0 && t.group == 0, "source BF16 matrix storage cannot contain quantization metadata");
        if (t.bits == 16) ++m.source_bf16_tensors;
        const uint64_t elements = uint64_t(t.rows) * t.cols;
        check(elements <= std::numeric_limits<size_t>::max() / 4 && (t.bits != 4 || t.cols % 2 == 0) &&
                  t.size == elements * t.bits / 8 && offset % 64 == 0 && offset <= size - base &&
                  t.size <= size - base - offset,
              "invalid tensor data range " + t.name);
        if (t.bits == 8 || t.bits == 4) {
            check(t.group && t.cols % t.group == 0 && (t.bits != 4 || t.group % 2 == 0) &&
                      t.scale_count == uint64_t(t.rows) * (t.cols / t.group) && scale_offset % 64 == 0 &&
                      scale_offset <= size - base && t.scale_count <= (size - base - scale_offset) / 4,
                  "invalid quantization metadata " + t.name);
            t.scales = reinterpret_cast<const float*>(data + base + scale_offset);
            for (uint64_t j = 0; j < t.scale_count; ++j) {
                float s;
                std::memcpy(&s, data + base + scale_offset + 4 * j, 4);
                check(std::isfinite(s) && s > 0, "invalid quantization scale");
            }
            ++m.quantized_tensors;
        } else {
            check(t.scale_count == 0 && t.group == 0, "unexpected FP32 quantization metadata");
        }
        t.data = data + base + offset;
        if (t.name.size() >= 12 && t.name.compare(t.name.size() - 12, 12, ".input_scale") == 0) {
            check(!bf16_matrix_format, "source BF16 matrix storage cannot contain calibrated input scales");
            check(t.bits == 32 && t.rows == 1, "invalid calibrated input scale tensor");
            for (uint32_t j = 0; j < t.cols; ++j) {
                float f;
                std::memcpy(&f, t.data + 4 * j, 4);
                check(std::isfinite(f) && f > 0, "invalid calibrated input scale value");
            }
        }
        check(tensors.emplace(t.name, t).second, "duplicate tensor " + t.name);
    }
    check(reader.position <= base, "metadata overlaps tensor payload");
    check(!bf16_format || m.source_bf16_tensors, "source BF16 artifact contains no BF16 tensors");

    auto require = [&](const std::string& name, uint32_t rows, uint32_t cols) -> const TensorRecord& {
        auto it = tensors.find(name);
        check(it != tensors.end() && it->second.rows == rows && it->second.cols == cols,
              "missing or incompatible tensor " + name);
        return it->second;
    };
    auto find = [&](const std::string& name) -> const TensorRecord* {
        auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    };
    require("model.embed_tokens.weight", c.vocab, c.hidden);
    require("lm_head.weight", c.vocab, c.hidden);
    if (c.final_norm) require("model.norm.weight", 1, c.hidden);
    if (c.position_kind == 1) require("model.position_embeddings.weight", c.max_positions + c.position_offset, c.hidden);
    for (uint32_t i = 0; i < c.layers; ++i) {
        const std::string p = "model.layers." + std::to_string(i) + ".";
        require(p + "input_layernorm.weight", 1, c.hidden);
        require(p + "post_attention_layernorm.weight", 1, c.hidden);
        require(p + "self_attn.q_proj.weight", c.qwidth(), c.hidden);
        require(p + "self_attn.k_proj.weight", c.kvwidth(), c.hidden);
        require(p + "self_attn.v_proj.weight", c.kvwidth(), c.hidden);
        require(p + "self_attn.o_proj.weight", c.hidden, c.qwidth());
        if (c.qk_norm)
            check(require(p + "self_attn.q_norm.weight", 1, c.head_dim).bits == 32 &&
                      require(p + "self_attn.k_norm.weight", 1, c.head_dim).bits == 32,
                  "Q/K normalization weights must use FP32 storage");
        if (c.gated) require(p + "mlp.gate_proj.weight", c.intermediate, c.hidden);
        require(p + "mlp.up_proj.weight", c.intermediate, c.hidden);
        require(p + "mlp.down_proj.weight", c.hidden, c.intermediate);
    }
    if (c.position_kind == 0 && c.rope_frequencies.empty()) {
        c.rope_frequencies.resize(c.rotary_dim / 2);
        for (uint32_t i = 0; i < c.rotary_dim / 2; ++i)
            c.rope_frequencies[i] = 1.0f / std::pow(c.theta, static_cast<float>(2 * i) / static_cast<float>(c.rotary_dim));
    }
    bool fp32_artifact = activation_bits == 32;
    for (auto& item : tensors) fp32_artifact = fp32_artifact && (item.second.bits == 32 || item.second.bits == 16);
    m.accurate = fp32_math == 1;
    check(!m.accurate || fp32_artifact, "accurate FP32 math requires FP32 compute and unquantized weights",
          LH_ERROR_INVALID_ARGUMENT);

    // ---- device memory plan -------------------------------------------------
    // Matrices that share an input and storage are stacked row-wise (q|k|v,
    // gate|up) so one launch streams them.  Every linear gets a bias vector,
    // zeros where the artifact has none: adding 0.0f is what the CPU path does
    // (decoder.cpp:1229), so results do not change.
    Plan plan;
    std::vector<std::vector<float>> zero_biases;   // host zeros kept alive until upload
    struct Pending { WeightView* view; size_t data, scales, bias; bool has_scales; };
    std::vector<Pending> pending;
    struct NormPending { const float** gamma; const float** beta; size_t g, b; bool has_beta; };
    std::vector<NormPending> norm_pending;
    struct PtrPending { const float** ptr; size_t offset; };
    std::vector<PtrPending> ptr_pending;

    auto linear_check = [&](const std::string& name, const TensorRecord& w) {
        if (const TensorRecord* b = find(name + ".bias"))
            check(b->rows == 1 && b->cols == w.rows && b->bits == 32, "incompatible linear bias");
        if (const TensorRecord* s = find(name + ".input_scale"))
            check(s->bits == 32 && s->rows == 1 && s->cols == w.cols, "incompatible calibrated input scale");
        if ((w.bits == 4 || w.bits == 8) && activation_bits == 8)
            check(w.group <= 131000, "integer accumulation exceeds safe input width");
    };
    auto add_linear = [&](Linear& out, const std::vector<std::string>& names) {
        std::vector<const TensorRecord*> parts;
        for (auto& n : names) {
            const TensorRecord& w = *find(n + ".weight");
            linear_check(n, w);
            parts.push_back(&w);
        }
        const TensorRecord& first = *parts[0];
        uint32_t rows = 0;
        for (auto* p : parts) rows += p->rows;
        size_t data_at = 0, scales_at = 0, bias_at = 0;
        for (size_t i = 0; i < parts.size(); ++i) {
            const size_t at = plan.add(parts[i]->data, parts[i]->size, i == 0 ? 256 : 1);
            if (i == 0) data_at = at;
        }
        const bool has_scales = first.bits == 8 || first.bits == 4;
        if (has_scales)
            for (size_t i = 0; i < parts.size(); ++i) {
                const size_t at = plan.add(parts[i]->scales, parts[i]->scale_count * 4, i == 0 ? 256 : 1);
                if (i == 0) scales_at = at;
            }
        for (size_t i = 0; i < parts.size(); ++i) {
            const TensorRecord* b = find(names[i] + ".bias");
            const void* src;
            if (b) {
                src = b->data;
            } else {
                zero_biases.emplace_back(parts[i]->rows, 0.0f);
                src = zero_biases.back().data();
            }
            const size_t at = plan.add(src, size_t(parts[i]->rows) * 4, i == 0 ? 256 : 1);
            if (i == 0) bias_at = at;
        }
        out.view.rows = rows;
        out.view.cols = first.cols;
        out.view.bits = first.bits;
        out.view.group = first.group;
        out.present = true;
        pending.push_back({&out.view, data_at, scales_at, bias_at, has_scales});
        if (names.size() == 1)
            if (const TensorRecord* s = find(names[0] + ".input_scale"))
                ptr_pending.push_back({&out.input_scale, plan.add(s->data, size_t(s->cols) * 4)});
    };
    auto stackable = [&](const std::vector<std::string>& names) {
        const TensorRecord& a = *find(names[0] + ".weight");
        for (auto& n : names) {
            const TensorRecord& w = *find(n + ".weight");
            if (w.bits != a.bits || w.cols != a.cols || w.group != a.group || find(n + ".input_scale")) return false;
        }
        return true;
    };
    auto add_norm = [&](NormView& out, const std::string& name) {
        const TensorRecord& g = *find(name + ".weight");
        const TensorRecord* b = find(name + ".bias");
        if (b) check(b->rows == 1 && b->cols == c.hidden && b->bits == 32, "incompatible normalization bias");
        out.kind = int(c.norm_kind);
        out.epsilon = c.epsilon;
        out.accurate = m.accurate ? 1 : 0;
        const size_t ga = plan.add(g.data, size_t(g.cols) * 4);
        const size_t ba = b ? plan.add(b->data, size_t(b->cols) * 4) : 0;
        norm_pending.push_back({&out.gamma, &out.beta, ga, ba, b != nullptr});
    };
    auto add_matrix = [&](WeightView& out, const std::string& name) {
        const TensorRecord& w = *find(name);
        out.rows = w.rows; out.cols = w.cols; out.bits = w.bits; out.group = w.group;
        const size_t d = plan.add(w.data, w.size);
        const size_t s = (w.bits == 8 || w.bits == 4) ? plan.add(w.scales, w.scale_count * 4) : 0;
        pending.push_back({&out, d, s, size_t(-1), w.bits == 8 || w.bits == 4});
    };

    m.layers.resize(c.layers);
    for (uint32_t i = 0; i < c.layers; ++i) {
        Layer& L = m.layers[i];
        const std::string p = "model.layers." + std::to_string(i) + ".";
        add_norm(L.input_norm, p + "input_layernorm");
        add_norm(L.post_norm, p + "post_attention_layernorm");
        const std::vector<std::string> qkv = {p + "self_attn.q_proj", p + "self_attn.k_proj", p + "self_attn.v_proj"};
        L.stacked_qkv = stackable(qkv);
        if (L.stacked_qkv) {
            add_linear(L.qkv, qkv);
        } else {
            add_linear(L.qkv, {qkv[0]});
            add_linear(L.k, {qkv[1]});
            add_linear(L.v, {qkv[2]});
        }
        add_linear(L.o, {p + "self_attn.o_proj"});
        if (c.gated) {
            const std::vector<std::string> gu = {p + "mlp.gate_proj", p + "mlp.up_proj"};
            L.stacked_gate_up = stackable(gu);
            if (L.stacked_gate_up) {
                add_linear(L.gate_up, gu);
            } else {
                add_linear(L.gate_up, {gu[0]});
                add_linear(L.up, {gu[1]});
            }
        } else {
            add_linear(L.up, {p + "mlp.up_proj"});
        }
        add_linear(L.down, {p + "mlp.down_proj"});
        if (c.qk_norm) {
            ptr_pending.push_back({&L.q_norm, plan.add(find(p + "self_attn.q_norm.weight")->data, c.head_dim * 4)});
            ptr_pending.push_back({&L.k_norm, plan.add(find(p + "self_attn.k_norm.weight")->data, c.head_dim * 4)});
        }
    }
    add_matrix(m.embedding, "model.embed_tokens.weight");
    if (c.position_kind == 1) {
        add_matrix(m.positions, "model.position_embeddings.weight");
        m.has_positions = true;
    }
    add_linear(m.head, {"lm_head"});
    if (c.final_norm) add_norm(m.final_norm, "model.norm");

    m.weights.allocate(plan.total);
    auto* dev = m.weights.as<uint8_t>();
    for (auto& s : plan.segments)
        hip_check(hipMemcpy(dev + s.offset, s.source, s.bytes, hipMemcpyHostToDevice), "weight upload");
    for (auto& p2 : pending) {
        p2.view->data = dev + p2.data;
        p2.view->scales = p2.has_scales ? reinterpret_cast<const float*>(dev + p2.scales) : nullptr;
        p2.view->bias = p2.bias == size_t(-1) ? nullptr : reinterpret_cast<const float*>(dev + p2.bias);
    }
    for (auto& n : norm_pending) {
        *n.gamma = reinterpret_cast<const float*>(dev + n.g);
        *n.beta = n.has_beta ? reinterpret_cast<const float*>(dev + n.b) : nullptr;
    }
    for (auto& q : ptr_pending) *q.ptr = reinterpret_cast<const float*>(dev + q.offset);
    return model;
}

}  // namespace leafhip
