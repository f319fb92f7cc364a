// Host runtime: LEAFDC validation and upload, session memory plan, forward.
//
// Validation is artifact_format.cpp's: an artifact the CPU runtime rejects is
// rejected here too, with its message, before anything reaches the device.
#include "runtime.h"

#include "artifact_format.h"

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
    ArtifactContents artifact = read_artifact(data, size, activation_bits, fp32_math);
    // The loader's size rule computes rows·cols·bits/8 in 64 bits, as the
    // reference's does, so a shape of 2^59 elements or more can wrap to the
    // stored byte count.  Kernels index by shape: recheck without wrapping.
    for (const auto& [name, t] : artifact.tensors) {
        const unsigned __int128 bits = static_cast<unsigned __int128>(uint64_t(t.rows) * t.cols) * t.bits;
        if (bits != static_cast<unsigned __int128>(t.size) * 8)
            throw Error(LH_ERROR_ARTIFACT, "Leaf decoder: invalid tensor data range " + name);
    }
    auto model = std::make_unique<Model>(context);
    Model& m = *model;
    m.config = artifact.config;
    Config& c = m.config;
    m.activation_bits = activation_bits;
    m.artifact_bytes = size;
    m.accurate = artifact.accurate;
    m.source_bf16_tensors = artifact.source_bf16_tensors;
    m.quantized_tensors = artifact.quantized_tensors;
    auto find = [&](const std::string& name) { return artifact.find(name); };

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

    auto add_linear = [&](Linear& out, const std::vector<std::string>& names) {
        std::vector<const TensorRecord*> parts;
        for (auto& n : names) {
            parts.push_back(find(n + ".weight"));
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
