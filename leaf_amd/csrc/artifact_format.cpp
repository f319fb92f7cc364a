// LEAFDC artifact validation (see artifact_format.h for the layout).
//
// The artifact is decoded front to back.  Each stage decodes one region and
// then enforces an ordered list of named rules over what it decoded; a rule
// that fails raises its message.  Rules that share a message are split into
// single-purpose predicates, evaluated in list order.  A region that runs
// past the end of the file raises "truncated artifact metadata" at the point
// where it is decoded, after the rules of the regions before it.
#include "artifact_format.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <vector>

namespace leafhip {
namespace {

static_assert(sizeof(float) == 4 && sizeof(uint32_t) == 4, "LEAFDC scalars are 32 and 64 bits");

[[noreturn]] void reject(const std::string& message, lh_status code = LH_ERROR_ARTIFACT) {
    throw Error(code, "Leaf decoder: " + message);
}

constexpr uint32_t kNoEos = 0xffffffffu;

// ------------------------------------------------------------ byte stream --
class ByteStream {
public:
    ByteStream(const uint8_t* data, size_t size) : data_(data), size_(size) {}
    size_t offset() const { return at_; }
    void seek(size_t at) { at_ = at; }
    void need(size_t bytes) const {
        if (!(at_ <= size_ && bytes <= size_ - at_))
            throw Error(LH_ERROR_ARTIFACT, "Leaf runtime: truncated artifact metadata");
    }
    // Little-endian scalars, assembled byte by byte.
    uint64_t unsigned_le(int bytes) {
        need(size_t(bytes));
        uint64_t v = 0;
        for (int i = 0; i < bytes; ++i) v |= uint64_t(data_[at_ + i]) << (8 * i);
        at_ += size_t(bytes);
        return v;
    }
    uint32_t u32() { return uint32_t(unsigned_le(4)); }
    uint64_t u64() { return unsigned_le(8); }
    float f32() {
        const uint32_t bits = u32();
        float v;
        std::memcpy(&v, &bits, 4);
        return v;
    }
    std::string text() {
        const uint32_t length = u32();
        need(length);
        std::string v(reinterpret_cast<const char*>(data_ + at_), length);
        at_ += length;
        return v;
    }

private:
    const uint8_t* data_;
    size_t size_;
    size_t at_ = 0;
};

float f32_at(const uint8_t* p) {
    float v;
    std::memcpy(&v, p, 4);
    return v;
}

// ---------------------------------------------------------------- rules ----
template <class T>
struct Rule {
    bool (*holds)(const T&);
    const char* message;
};

template <class T, size_t N>
void enforce(const T& subject, const Rule<T> (&rules)[N], const std::string& suffix = "") {
    for (const Rule<T>& r : rules)
        if (!r.holds(subject)) reject(std::string(r.message) + suffix);
}

// -------------------------------------------------------------- versions --
// What each magic implies.  `window`: -1 the sliding window must be 0,
// +1 it must be positive, 0 either.  `storage`: 0 FP32 / integer, 5 BF16
// embedding and head only, 6 BF16 matrices (v7 reads it from its metadata).
struct Edition {
    char magic[9];
    uint32_t version;
    int window;
    bool eos_list;
    uint32_t storage;
    bool operator_metadata;
};
constexpr Edition kEditions[] = {
    {"LEAFDC02", 2, -1, false, 0, false}, {"LEAFDC03", 3, +1, false, 0, false},
    {"LEAFDC04", 4, 0, true, 0, false},   {"LEAFDC05", 5, 0, true, 5, false},
    {"LEAFDC06", 6, 0, true, 6, false},   {"LEAFDC07", 7, 0, true, 0, true},
};

// ---------------------------------------------------------------- header --
struct Header {
    const Edition* edition = nullptr;
    size_t file_bytes = 0;
    uint32_t count = 0;
    uint64_t base = 0;
    Config c;
};

bool dimensions_positive(const Header& h) {
    const Config& c = h.c;
    return c.hidden && c.intermediate && c.heads && c.kv_heads && c.layers && c.vocab && c.head_dim &&
           c.max_positions;
}
bool heads_group_evenly(const Header& h) { return h.c.heads % h.c.kv_heads == 0; }
bool query_width_fits(const Header& h) {
    return uint64_t(h.c.heads) * h.c.head_dim <= std::numeric_limits<uint32_t>::max();
}
bool operator_codes_known(const Header& h) {
    const Config& c = h.c;
    return c.norm_kind <= 1 && c.activation <= 3 && c.position_kind <= 2 && c.gated <= 1 && c.parallel <= 1 &&
           c.final_norm <= 1;
}
bool rotary_width_fits(const Header& h) {
    const Config& c = h.c;
    return c.rotary_dim <= c.head_dim && c.rotary_dim % 2 == 0 && (c.position_kind != 0 || c.rotary_dim > 0);
}
bool positive_finite(float v) { return std::isfinite(v) && v > 0; }
bool scalars_positive(const Header& h) {
    return positive_finite(h.c.embedding_scale) && positive_finite(h.c.theta) && positive_finite(h.c.epsilon);
}
constexpr Rule<Header> kConfiguration[] = {
    {dimensions_positive, "invalid decoder configuration"}, {heads_group_evenly, "invalid decoder configuration"},
    {query_width_fits, "invalid decoder configuration"},    {operator_codes_known, "invalid decoder configuration"},
    {rotary_width_fits, "invalid decoder configuration"},   {scalars_positive, "invalid decoder configuration"},
};

bool workspaces_addressable(const Header& h) {
    const Config& c = h.c;
    const uint64_t widest =
        std::max<uint64_t>({c.hidden, uint64_t(c.heads) * c.head_dim, c.intermediate, c.vocab, c.max_positions});
    const size_t limit = std::numeric_limits<size_t>::max();
    return c.max_positions <= limit - c.position_offset && c.max_positions <= limit / sizeof(float) / widest;
}
bool table_in_file(const Header& h) {
    // a descriptor is at least 56 bytes, so the count is bounded by the file
    return h.base % 64 == 0 && h.base <= h.file_bytes && h.count <= h.file_bytes / 56;
}
bool eos_in_vocabulary(const Header& h) { return h.c.eos < h.c.vocab || h.c.eos == kNoEos; }
constexpr Rule<Header> kLayout[] = {
    {workspaces_addressable, "decoder workspace dimensions overflow address space"},
    {table_in_file, "invalid tensor table"},
    {eos_in_vocabulary, "invalid EOS token"},
};

// The sliding-window field must agree with the edition (v2: none, v3: some).
void check_window(const Header& h) {
    const int rule = h.edition->window;
    if ((rule < 0 && h.c.sliding_window != 0) || (rule > 0 && h.c.sliding_window == 0))
        reject("invalid sliding-window artifact configuration");
}

Header decode_header(ByteStream& in, size_t file_bytes) {
    Header h;
    h.file_bytes = file_bytes;
    in.need(8);
    in.seek(0);
    char magic[8];
    for (char& ch : magic) ch = char(in.unsigned_le(1));
    for (const Edition& e : kEditions)
        if (std::memcmp(magic, e.magic, 8) == 0) h.edition = &e;
    if (!h.edition) reject("unsupported artifact magic");
    Config& c = h.c;
    c.version = in.u32();
    if (c.version != h.edition->version) reject("unsupported decoder artifact version");
    h.count = in.u32();
    h.base = in.u64();
    for (uint32_t* field : {&c.hidden, &c.intermediate, &c.heads, &c.kv_heads, &c.layers, &c.vocab, &c.max_positions,
                            &c.eos, &c.head_dim, &c.sliding_window})
        *field = in.u32();
    check_window(h);
    c.theta = in.f32();
    c.epsilon = in.f32();
    for (uint32_t* field : {&c.norm_kind, &c.activation, &c.position_kind, &c.gated, &c.parallel, &c.rotary_dim,
                            &c.position_offset, &c.final_norm})
        *field = in.u32();
    c.embedding_scale = in.f32();
    enforce(h, kConfiguration);
    enforce(h, kLayout);
    return h;
}

// ------------------------------------------------ v7 operator metadata ----
struct OperatorMetadata {
    const Header* h = nullptr;
    uint32_t storage = 0, qk_norm = 0, frequencies = 0;
    uint64_t room = 0;   // bytes between the frequencies and the data base
};
bool asks_for_something(const OperatorMetadata& m) { return m.qk_norm || m.frequencies; }
bool qk_flag_known(const OperatorMetadata& m) { return m.qk_norm <= 1; }
bool with_rotary_positions(const OperatorMetadata& m) { return m.h->c.position_kind == 0; }
bool qk_norm_is_rms(const OperatorMetadata& m) { return !m.qk_norm || m.h->c.norm_kind == 0; }
bool one_frequency_per_pair(const OperatorMetadata& m) {
    return !m.frequencies || m.frequencies == m.h->c.rotary_dim / 2;
}
bool frequencies_before_data(const OperatorMetadata& m) { return m.frequencies <= m.room / 4; }
constexpr Rule<OperatorMetadata> kOperatorMetadata[] = {
    {asks_for_something, "invalid decoder operator metadata"},
    {qk_flag_known, "invalid decoder operator metadata"},
    {with_rotary_positions, "invalid decoder operator metadata"},
    {qk_norm_is_rms, "invalid decoder operator metadata"},
    {one_frequency_per_pair, "invalid decoder operator metadata"},
    {frequencies_before_data, "invalid decoder operator metadata"},
};

// Space left for metadata before the data base, or none when past it.
bool room_before(const ByteStream& in, uint64_t base, uint64_t bytes) {
    return in.offset() <= base && base - in.offset() >= bytes;
}

uint32_t decode_operator_metadata(ByteStream& in, Header& h) {
    if (!room_before(in, h.base, 12)) reject("truncated decoder operator metadata");
    OperatorMetadata m;
    m.h = &h;
    m.storage = in.u32();
    m.qk_norm = in.u32();
    m.frequencies = in.u32();
    if (m.storage != 0 && m.storage != 5 && m.storage != 6) reject("invalid decoder storage policy");
    m.room = h.base - in.offset();
    enforce(m, kOperatorMetadata);
    h.c.qk_norm = m.qk_norm;
    for (uint32_t i = 0; i < m.frequencies; ++i) {
        const float f = in.f32();
        if (!(std::isfinite(f) && f > 0 && f <= 1)) reject("invalid static RoPE frequency");
        h.c.rope_frequencies.push_back(f);
    }
    return m.storage;
}

// ------------------------------------------------------------ EOS list ----
void decode_eos(ByteStream& in, Header& h, bool bf16_storage) {
    Config& c = h.c;
    if (!h.edition->eos_list) {
        if (c.eos < c.vocab) c.eos_tokens.push_back(c.eos);
        return;
    }
    if (!room_before(in, h.base, 4)) reject("truncated EOS metadata");
    const uint32_t n = in.u32();
    // v4 exists to carry several EOS tokens; later editions may carry none
    const bool enough = bf16_storage || h.edition->operator_metadata || n >= 2;
    if (!(enough && n <= 1024 && n <= c.vocab && in.offset() <= h.base && n <= (h.base - in.offset()) / 4))
        reject("invalid multi-EOS token count");
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t token = in.u32();
        const bool seen = std::find(c.eos_tokens.begin(), c.eos_tokens.end(), token) != c.eos_tokens.end();
        if (token >= c.vocab || seen) reject("invalid or duplicate EOS token");
        c.eos_tokens.push_back(token);
    }
    const uint32_t primary = c.eos_tokens.empty() ? kNoEos : c.eos_tokens.front();
    if (c.eos != primary) reject("multi-EOS primary token mismatch");
}

// ----------------------------------------------------- tensor descriptors --
// Matrices v6 may store as BF16: the embeddings, the head and the seven
// projection roles of layers below the layer count (decoder.cpp:93-115).
bool bf16_matrix_name(const std::string& name, uint32_t rows, uint32_t layers) {
    if (rows <= 1) return false;
    static const char* whole[] = {"lm_head.weight", "model.embed_tokens.weight", "model.position_embeddings.weight"};
    for (const char* n : whole)
        if (name == n) return true;
    static const std::string prefix = "model.layers.";
    if (name.rfind(prefix, 0) != 0) return false;
    const size_t digits_end = name.find('.', prefix.size());
    if (digits_end == std::string::npos) return false;
    const std::string digits = name.substr(prefix.size(), digits_end - prefix.size());
    // a canonical decimal index: no sign, no leading zero, within the layer count
    if (digits.empty() || (digits.size() > 1 && digits[0] == '0') || digits.size() > 20) return false;
    uint64_t layer = 0;
    for (char d : digits) {
        if (d < '0' || d > '9') return false;
        if (layer > (std::numeric_limits<uint64_t>::max() - uint64_t(d - '0')) / 10) return false;
        layer = layer * 10 + uint64_t(d - '0');
    }
    if (layer >= layers) return false;
    static const char* roles[] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                                  "self_attn.o_proj.weight", "mlp.up_proj.weight",      "mlp.gate_proj.weight",
                                  "mlp.down_proj.weight"};
    const std::string role = name.substr(digits_end + 1);
    return std::any_of(std::begin(roles), std::end(roles), [&](const char* r) { return role == r; });
}

struct Descriptor {
    std::string name;
    uint32_t rank = 0, rows = 0, cols = 0, bits = 0, group = 0;
    uint64_t offset = 0, bytes = 0, scale_offset = 0, scale_count = 0;
    // context
    uint32_t storage = 0, layers = 0;
    uint64_t payload = 0;   // file bytes after the data base
};

bool storage_allowed(const Descriptor& d) {
    if (d.bits == 32 || d.bits == 8 || d.bits == 4) return true;
    if (d.bits != 16 || d.storage == 0) return false;
    if (d.storage == 6) return bf16_matrix_name(d.name, d.rows, d.layers);
    return d.name == "lm_head.weight" || d.name == "model.embed_tokens.weight";
}
bool matrix_shaped(const Descriptor& d) { return d.rank == 2 && d.rows && d.cols; }
constexpr Rule<Descriptor> kTensorKind[] = {
    {matrix_shaped, "invalid tensor "},
    {storage_allowed, "invalid tensor "},
};

uint64_t elements(const Descriptor& d) { return uint64_t(d.rows) * d.cols; }
bool addressable(const Descriptor& d) { return elements(d) <= std::numeric_limits<size_t>::max() / 4; }
bool nibbles_pair_up(const Descriptor& d) { return d.bits != 4 || d.cols % 2 == 0; }
bool payload_size_matches(const Descriptor& d) { return d.bytes == elements(d) * d.bits / 8; }
bool payload_aligned(const Descriptor& d) { return d.offset % 64 == 0; }
bool payload_in_file(const Descriptor& d) { return d.offset <= d.payload && d.bytes <= d.payload - d.offset; }
constexpr Rule<Descriptor> kTensorData[] = {
    {addressable, "invalid tensor data range "},       {nibbles_pair_up, "invalid tensor data range "},
    {payload_size_matches, "invalid tensor data range "}, {payload_aligned, "invalid tensor data range "},
    {payload_in_file, "invalid tensor data range "},
};

bool group_divides_row(const Descriptor& d) { return d.group && d.cols % d.group == 0; }
bool nibble_groups_even(const Descriptor& d) { return d.bits != 4 || d.group % 2 == 0; }
bool one_scale_per_group(const Descriptor& d) { return d.scale_count == uint64_t(d.rows) * (d.cols / d.group); }
bool scales_aligned(const Descriptor& d) { return d.scale_offset % 64 == 0; }
bool scales_in_file(const Descriptor& d) {
    return d.scale_offset <= d.payload && d.scale_count <= (d.payload - d.scale_offset) / 4;
}
constexpr Rule<Descriptor> kQuantizationMetadata[] = {
    {group_divides_row, "invalid quantization metadata "}, {nibble_groups_even, "invalid quantization metadata "},
    {one_scale_per_group, "invalid quantization metadata "}, {scales_aligned, "invalid quantization metadata "},
    {scales_in_file, "invalid quantization metadata "},
};

bool ends_with(const std::string& s, const char* suffix) {
    const size_t n = std::strlen(suffix);
    return s.size() >= n && s.compare(s.size() - n, n, suffix) == 0;
}

Descriptor decode_descriptor(ByteStream& in, const Header& h, uint32_t storage) {
    Descriptor d;
    d.name = in.text();
    for (uint32_t* field : {&d.rank, &d.rows, &d.cols, &d.bits, &d.group}) *field = in.u32();
    for (uint64_t* field : {&d.offset, &d.bytes, &d.scale_offset, &d.scale_count}) *field = in.u64();
    d.storage = storage;
    d.layers = h.c.layers;
    d.payload = h.file_bytes - h.base;
    return d;
}

void validate_tensor(const Descriptor& d, const uint8_t* data, const Header& h, ArtifactContents& out) {
    enforce(d, kTensorKind, d.name);
    if (d.storage != 0 && d.bits != 32 && d.bits != 16) reject("source BF16 storage cannot mix quantized weights");
    if (d.storage == 6 && (d.scale_count || d.group))
        reject("source BF16 matrix storage cannot contain quantization metadata");
    if (d.bits == 16) ++out.source_bf16_tensors;
    enforce(d, kTensorData, d.name);
    TensorRecord t;
    t.name = d.name;
    t.rows = d.rows;
    t.cols = d.cols;
    t.bits = d.bits;
    t.group = d.group;
    t.size = d.bytes;
    t.scale_count = d.scale_count;
    t.data = data + h.base + d.offset;
    if (d.bits == 8 || d.bits == 4) {
        enforce(d, kQuantizationMetadata, d.name);
        const uint8_t* scales = data + h.base + d.scale_offset;
        for (uint64_t j = 0; j < d.scale_count; ++j)
            if (!positive_finite(f32_at(scales + 4 * j))) reject("invalid quantization scale");
        t.scales = reinterpret_cast<const float*>(scales);
        ++out.quantized_tensors;
    } else if (d.scale_count || d.group) {
        reject("unexpected FP32 quantization metadata");
    }
    if (ends_with(d.name, ".input_scale")) {
        if (d.storage == 6) reject("source BF16 matrix storage cannot contain calibrated input scales");
        if (d.bits != 32 || d.rows != 1) reject("invalid calibrated input scale tensor");
        for (uint32_t j = 0; j < d.cols; ++j)
            if (!positive_finite(f32_at(t.data + 4 * j))) reject("invalid calibrated input scale value");
    }
    if (!out.tensors.emplace(d.name, t).second) reject("duplicate tensor " + d.name);
}

// ------------------------------------------------------- required tensors --
struct Requirement {
    std::string name;
    uint32_t rows, cols;
    bool fp32;   // Q/K norm weights: FP32 storage required (checked as soon as the tensor is found)
};

// Calls `each` for every required tensor in the reference's order, stopping
// at the first call that throws (a layer count from a corrupt header must not
// be materialized).
template <class Each>
void for_each_requirement(const Config& c, Each&& each) {
    struct Sink {
        Each& each;
        void push_back(const Requirement& r) { each(r); }
    } r{each};
    r.push_back({"model.embed_tokens.weight", c.vocab, c.hidden, false});
    r.push_back({"lm_head.weight", c.vocab, c.hidden, false});
    if (c.final_norm) r.push_back({"model.norm.weight", 1, c.hidden, false});
    if (c.position_kind == 1)
        r.push_back({"model.position_embeddings.weight", c.max_positions + c.position_offset, c.hidden, false});
    for (uint32_t i = 0; i < c.layers; ++i) {
        const std::string p = "model.layers." + std::to_string(i) + ".";
        const std::pair<const char*, std::pair<uint32_t, uint32_t>> projections[] = {
            {"input_layernorm.weight", {1, c.hidden}},
            {"post_attention_layernorm.weight", {1, c.hidden}},
            {"self_attn.q_proj.weight", {c.qwidth(), c.hidden}},
            {"self_attn.k_proj.weight", {c.kvwidth(), c.hidden}},
            {"self_attn.v_proj.weight", {c.kvwidth(), c.hidden}},
            {"self_attn.o_proj.weight", {c.hidden, c.qwidth()}},
        };
        for (const auto& pr : projections) r.push_back({p + pr.first, pr.second.first, pr.second.second, false});
        if (c.qk_norm) {
            r.push_back({p + "self_attn.q_norm.weight", 1, c.head_dim, true});
            r.push_back({p + "self_attn.k_norm.weight", 1, c.head_dim, true});
        }
        if (c.gated) r.push_back({p + "mlp.gate_proj.weight", c.intermediate, c.hidden, false});
        r.push_back({p + "mlp.up_proj.weight", c.intermediate, c.hidden, false});
        r.push_back({p + "mlp.down_proj.weight", c.hidden, c.intermediate, false});
    }
}

// What the reference checks when a tensor is first used in a forward
// (decoder.cpp:975-981, 994-1024), in forward order, checked here at load.
void check_uses(const ArtifactContents& a, uint32_t activation_bits) {
    const Config& c = a.config;
    auto norm = [&](const std::string& name) {
        if (const TensorRecord* b = a.find(name + ".bias"))
            if (!(b->rows == 1 && b->cols == c.hidden)) reject("incompatible normalization bias");
    };
    auto linear = [&](const std::string& name) {
        const TensorRecord* w = a.find(name + ".weight");
        if (!w) return;
        if (const TensorRecord* b = a.find(name + ".bias"))
            if (!(b->rows == 1 && b->cols == w->rows)) reject("incompatible linear bias");
        if (const TensorRecord* s = a.find(name + ".input_scale"))
            if (!(s->bits == 32 && s->rows == 1 && s->cols == w->cols)) reject("incompatible calibrated input scale");
        if ((w->bits == 8 || w->bits == 4) && activation_bits == 8 && w->group > 131000)
            reject("integer accumulation exceeds safe input width");
    };
    for (uint32_t i = 0; i < c.layers; ++i) {
        const std::string p = "model.layers." + std::to_string(i) + ".";
        norm(p + "input_layernorm");
        for (const char* n : {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj"})
            linear(p + n);
        norm(p + "post_attention_layernorm");
        linear(p + "mlp.up_proj");
        if (c.gated) linear(p + "mlp.gate_proj");
        linear(p + "mlp.down_proj");
    }
    if (c.final_norm) norm("model.norm");
    linear("lm_head");
}

// Device limits of this build (no reference counterpart): biases and
// normalization vectors are read as f32.
void check_device_storage(const ArtifactContents& a) {
    for (const auto& item : a.tensors) {
        const std::string& n = item.first;
        const bool vector = ends_with(n, ".bias") || ends_with(n, "layernorm.weight") || n == "model.norm.weight" ||
                            ends_with(n, "_norm.weight");
        if (vector && item.second.bits != 32)
            reject("normalization weights and biases must use FP32 storage on this device path", LH_ERROR_UNSUPPORTED);
    }
}

}  // namespace

ArtifactContents read_artifact(const uint8_t* data, size_t size, uint32_t activation_bits, uint32_t fp32_math) {
    if (activation_bits != 8 && activation_bits != 32)
        reject("activation bits must be 8 or 32", LH_ERROR_INVALID_ARGUMENT);
    if (fp32_math > 1) reject("invalid FP32 math policy", LH_ERROR_INVALID_ARGUMENT);
    ArtifactContents out;
    ByteStream in(data, size);
    Header h = decode_header(in, size);
    uint32_t storage = h.edition->storage;
    if (h.edition->operator_metadata) storage = decode_operator_metadata(in, h);
    Config& c = h.c;
    if (!(c.qk_norm || uint64_t(c.heads) * c.head_dim == c.hidden)) reject("invalid decoder head geometry");
    if (c.head_dim > 256) reject("head dimensions above 256 are not supported on this device path", LH_ERROR_UNSUPPORTED);
    const bool bf16_storage = storage == 5 || storage == 6;
    if (bf16_storage && activation_bits != 32)
        reject("source BF16 storage requires FP32 activations", LH_ERROR_INVALID_ARGUMENT);
    decode_eos(in, h, bf16_storage);
    for (uint32_t i = 0; i < h.count; ++i) validate_tensor(decode_descriptor(in, h, storage), data, h, out);
    if (in.offset() > h.base) reject("metadata overlaps tensor payload");
    if (bf16_storage && !out.source_bf16_tensors) reject("source BF16 artifact contains no BF16 tensors");
    out.config = c;
    for_each_requirement(c, [&](const Requirement& r) {
        const TensorRecord* t = out.find(r.name);
        if (!t || t->rows != r.rows || t->cols != r.cols) reject("missing or incompatible tensor " + r.name);
        if (r.fp32 && t->bits != 32) reject("Q/K normalization weights must use FP32 storage");
    });
    if (c.position_kind == 0 && c.rope_frequencies.empty()) {
        // RoPE frequencies the reference derives: 1 / theta^(2i / rotary_dim) in f32 (decoder.cpp:929-933)
        for (uint32_t i = 0; i < c.rotary_dim / 2; ++i)
            out.config.rope_frequencies.push_back(
                1.0f / std::pow(c.theta, static_cast<float>(2 * i) / static_cast<float>(c.rotary_dim)));
    }
    const bool unquantized = std::all_of(out.tensors.begin(), out.tensors.end(), [](const auto& item) {
        return item.second.bits == 32 || item.second.bits == 16;
    });
    out.accurate = fp32_math == 1;
    if (out.accurate && !(activation_bits == 32 && unquantized))
        reject("accurate FP32 math requires FP32 compute and unquantized weights", LH_ERROR_INVALID_ARGUMENT);
    check_uses(out, activation_bits);
    check_device_storage(out);
    return out;
}

}  // namespace leafhip
