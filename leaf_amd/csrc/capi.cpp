// extern "C" surface of libleafhip (include/leafhip.h).  Every entry point
// converts exceptions into a status code plus a thread-local message; nothing
// throws across the ABI.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "artifact_format.h"
#include "runtime.h"

struct lh_context { leafhip::Context impl; };
struct lh_model { std::unique_ptr<leafhip::Model> impl; };
struct lh_session { std::unique_ptr<leafhip::Session> impl; };
struct lh_timer { hipEvent_t start, stop; };
struct lh_graph { hipGraphExec_t exec; };

namespace {

thread_local std::string g_error;

template <typename F>
lh_status guarded(F&& body) {
    try {
        body();
        g_error.clear();
        return LH_OK;
    } catch (const leafhip::Error& e) {
        g_error = e.what();
        return e.code;
    } catch (const std::bad_alloc&) {
        g_error = "Leaf decoder: out of host memory";
        return LH_ERROR_OUT_OF_MEMORY;
    } catch (const std::exception& e) {
        g_error = e.what();
        return LH_ERROR_DEVICE;
    }
}

void require_arg(bool ok, const char* what) {
    if (!ok) throw leafhip::Error(LH_ERROR_INVALID_ARGUMENT, std::string("Leaf decoder: ") + what);
}

hipStream_t as_stream(lh_stream s) { return static_cast<hipStream_t>(s); }

// Device scratch of the kernel-level entry points (quantized inputs, split-K
// sums, attention partials), one set per (device, stream): calls on different
// streams never share memory.  A buffer that must grow is replaced and the old
// one is kept with the stream's set, so work already queued on it, or a graph
// captured with it, stays valid without any synchronization.  Growth while
// the stream is capturing is refused: run the call once before capturing it.
// lh_stream_destroy waits for the stream and frees its sets, unless the
// stream has been captured: a graph captured from it may be launched later on
// another stream, so such a set is kept until the process ends.  Nothing is
// freed by static destructors, which run after the HIP runtime and a
// profiler may have shut down.
struct StreamScratch {
    leafhip::DeviceBuffer* work = nullptr;       // grown on demand
    leafhip::DeviceBuffer* counters = nullptr;   // zeroed once; the attention kernel resets what it uses
    std::vector<leafhip::DeviceBuffer*> retired;  // outgrown work buffers
    bool captured = false;                        // a graph may hold these buffers
};
std::mutex g_scratch_lock;
auto* g_scratch = new std::map<std::pair<int, hipStream_t>, StreamScratch>();

StreamScratch& scratch_of(hipStream_t stream) {
    int dev = 0;
    leafhip::hip_check(hipGetDevice(&dev), "hipGetDevice");
    return (*g_scratch)[{dev, stream}];
}

// Called with the stream idle and about to be destroyed.
void release_stream_scratch(hipStream_t stream) {
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    for (auto it = g_scratch->begin(); it != g_scratch->end();) {
        if (it->first.second != stream) {
            ++it;
            continue;
        }
        StreamScratch& sc = it->second;
        if (!sc.captured) {
            delete sc.work;
            delete sc.counters;
            for (leafhip::DeviceBuffer* b : sc.retired) delete b;
        }
        it = g_scratch->erase(it);
    }
}

void mark_stream_captured(hipStream_t stream) {
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    for (auto& [key, sc] : *g_scratch)
        if (key.second == stream) sc.captured = true;
}

bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    leafhip::hip_check(hipStreamIsCapturing(stream, &status), "hipStreamIsCapturing");
    return status != hipStreamCaptureStatusNone;
}

void* scratch_bytes(size_t bytes, hipStream_t stream) {
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    StreamScratch& sc = scratch_of(stream);
    if (!sc.work || sc.work->bytes < bytes) {
        if (capturing(stream))
            throw leafhip::Error(LH_ERROR_STATE, "Leaf decoder: kernel scratch must grow outside stream capture "
                                                 "(run the call once before capturing it)");
        auto* grown = new leafhip::DeviceBuffer(std::max(bytes, sc.work ? 2 * sc.work->bytes : size_t(1) << 20));
        if (sc.work) sc.retired.push_back(sc.work);
        sc.work = grown;
    }
    return sc.work->ptr;
}

// Zero-initialized span counters of the decode attention kernel (it resets
// them itself), one set per (device, stream).
unsigned* attention_counters(hipStream_t stream) {
    std::lock_guard<std::mutex> guard(g_scratch_lock);
    StreamScratch& sc = scratch_of(stream);
    if (!sc.counters) {
        if (capturing(stream))
            throw leafhip::Error(LH_ERROR_STATE, "Leaf decoder: attention counters must be set up outside stream "
                                                 "capture (run the call once before capturing it)");
        auto* b = new leafhip::DeviceBuffer(1024 * sizeof(unsigned));
        leafhip::hip_check(hipMemsetAsync(b->ptr, 0, b->bytes, stream), "hipMemsetAsync");
        sc.counters = b;
    }
    return sc.counters->as<unsigned>();
}

// Numerics of this thread's kernel-level calls (lh_set_kernel_numerics).
thread_local bool t_reference_order = false;
thread_local bool t_reference_vnni = false;   // grouped INT8 sums as quant_vnni_tile

// Scratch of lh_linear_noalloc: a device array that exists from module load
// to process end, one copy per GPU, so that entry point allocates nothing.
// Host code never uses the array's name as an address: its per-device
// address comes from hipGetSymbolAddress, resolved once per device with that
// device current (at lh_context_create, or at the entry point's first call on
// the device) and kept in g_noalloc_address.
static __device__ __align__(256) uint8_t scratch[LH_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_lock;
void* g_noalloc_address[kMaxDevices] = {};

// The current device's copy of `scratch`.
void* noalloc_scratch() {
    int dev = 0;
    leafhip::hip_check(hipGetDevice(&dev), "hipGetDevice");
    require_arg(dev >= 0 && dev < kMaxDevices, "device index out of range");
    std::lock_guard<std::mutex> guard(g_noalloc_lock);
    if (!g_noalloc_address[dev]) {
        void* address = nullptr;
        leafhip::hip_check(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)), "hipGetSymbolAddress");
        g_noalloc_address[dev] = address;
    }
    return g_noalloc_address[dev];
}

leafhip::WeightView view_of(const lh_weight* w) {
    require_arg(w && w->data && w->rows && w->cols, "weight descriptor is empty");
    require_arg(w->bits == 32 || w->bits == 16 || w->bits == 8 || w->bits == 4, "weight bits must be 32, 16, 8 or 4");
    if (w->bits == 8 || w->bits == 4) {
        require_arg(w->scales && w->group && w->cols % w->group == 0, "quantized weight needs scales and a group dividing cols");
        require_arg(w->bits != 4 || (w->cols % 2 == 0 && w->group % 2 == 0), "INT4 weight needs even cols and group");
    }
    require_arg(w->rows <= 0x7fffffffu && w->cols <= 0x7fffffffu, "weight is too large");
    leafhip::WeightView v;
    v.data = w->data;
    v.scales = w->scales;
    v.bias = w->bias;
    v.rows = int(w->rows);
    v.cols = int(w->cols);
    v.bits = int(w->bits);
    v.group = (w->bits == 8 || w->bits == 4) ? int(w->group) : 0;
    return v;
}

lh_status linear_impl(const lh_weight* weight, const float* x, const int8_t* q, const float* qs, size_t tokens,
                      uint32_t activation_bits, float* y, int32_t* acc, lh_stream stream, int force_path,
                      unsigned required_bits, bool no_alloc = false) {
    return guarded([&] {
        leafhip::LinearCall c;
        c.w = view_of(weight);
        require_arg(!required_bits || weight->bits == required_bits, "weight storage does not match the entry point");
        require_arg(tokens > 0 && tokens <= 0x7fffffff && y, "tokens and output are required");
        require_arg(activation_bits == 8 || activation_bits == 32, "activation bits must be 8 or 32");
        c.integer_activations = activation_bits == 8;
        require_arg(!c.integer_activations || c.w.bits == 8 || c.w.bits == 4,
                    "integer activations need INT8 or INT4 weights");
        require_arg(!c.integer_activations || c.w.group <= 131000, "integer accumulation exceeds safe input width");
        require_arg(x || (q && qs), "input is required");
        c.x = x;
        c.xq = q;
        c.xs = qs;
        c.tokens = int(tokens);
        c.y = y;
        c.acc_out = acc;
        c.force_path = force_path;
        c.unfused_group_sum = t_reference_vnni && c.integer_activations && c.w.bits == 8 && c.w.group <= 65536;
        if (c.integer_activations) {
            // quantized copy of x (when the kernel does not quantize in registers),
            // then room for 8 split-K partial sums of the output (prefill GEMM)
            const size_t q_bytes = q ? 0 : ((tokens * c.w.cols + 255) / 256) * 256;
            const size_t s_bytes = q ? 0 : ((tokens * 4 + 255) / 256) * 256;
            size_t split = tokens > 4 ? 8 * tokens * c.w.rows : 0;
            uint8_t* base = nullptr;
            if (no_alloc) {
                // the fixed array: the quantized input must fit; split-K uses
                // what is left (the GEMM splits less when it has less room,
                // with identical integer sums)
                require_arg(q_bytes + s_bytes <= LH_NOALLOC_SCRATCH_BYTES,
                            "input too large for the allocation-free scratch (tokens * (cols + 4) bytes)");
                base = static_cast<uint8_t*>(noalloc_scratch());
                split = std::min(split, (LH_NOALLOC_SCRATCH_BYTES - q_bytes - s_bytes) / sizeof(int32_t));
            } else {
                base = static_cast<uint8_t*>(
                    scratch_bytes(q_bytes + s_bytes + split * sizeof(int32_t) + 256, as_stream(stream)));
            }
            if (!q) {
                c.xq_scratch = reinterpret_cast<int8_t*>(base);
                c.xs_scratch = reinterpret_cast<float*>(base + q_bytes);
            }
            c.split_scratch = split ? reinterpret_cast<int32_t*>(base + q_bytes + s_bytes) : nullptr;
            c.split_capacity = split;
        }
        if (t_reference_order && !c.integer_activations) {
            // dot_avx order; the integer path is exact in every mode
            require_arg(x != nullptr, "input is required");
            if (!leafhip::launch_linear_fp_reference_order(c.w, x, int(tokens), y, leafhip::kStore, as_stream(stream)))
                throw leafhip::Error(LH_ERROR_UNSUPPORTED, "Leaf decoder: unsupported linear configuration");
            leafhip::hip_check(hipGetLastError(), "linear launch");
            return;
        }
        const int path = leafhip::launch_linear(c, as_stream(stream));
        if (path < 0) throw leafhip::Error(LH_ERROR_UNSUPPORTED, "Leaf decoder: unsupported linear configuration");
        leafhip::hip_check(hipGetLastError(), "linear launch");
    });
}

}  // namespace

extern "C" {

const char* lh_last_error(void) { return g_error.c_str(); }
const char* lh_version(void) { return "leafhip 0.1 (gfx950)"; }

lh_status lh_context_create(int device, lh_context** out) {
    return guarded([&] {
        require_arg(out != nullptr, "output pointer is null");
        int count = 0;
        leafhip::hip_check(hipGetDeviceCount(&count), "hipGetDeviceCount");
        require_arg(device >= 0 && device < count, "no such GPU");
        leafhip::hip_check(hipSetDevice(device), "hipSetDevice");
        (void)noalloc_scratch();   // lh_linear_noalloc's array on this device
        auto* c = new lh_context();
        c->impl.device = device;
        const hipError_t st = hipStreamCreateWithFlags(&c->impl.stream, hipStreamNonBlocking);
        if (st != hipSuccess) {
            delete c;
            leafhip::hip_check(st, "hipStreamCreate");
        }
        *out = c;
    });
}

lh_status lh_context_destroy(lh_context* context) {
    return guarded([&] { delete context; });
}

lh_status lh_model_load(lh_context* context, const void* artifact, size_t bytes, uint32_t activation_bits,
                        uint32_t fp32_math, lh_model** out) {
    return guarded([&] {
        require_arg(context && artifact && out, "context, artifact and output are required");
        leafhip::hip_check(hipSetDevice(context->impl.device), "hipSetDevice");
        auto model = leafhip::Model::load(context->impl, static_cast<const uint8_t*>(artifact), bytes, activation_bits,
                                          fp32_math);
        *out = new lh_model{std::move(model)};
    });
}

lh_status lh_model_load_file(lh_context* context, const char* path, uint32_t activation_bits, uint32_t fp32_math,
                             lh_model** out) {
    return guarded([&] {
        require_arg(context && path && out, "context, path and output are required");
        // Mapping (host_support.h:37-92): read-only private map of the artifact.
        const int fd = ::open(path, O_RDONLY);
        if (fd < 0) throw leafhip::Error(LH_ERROR_ARTIFACT, std::string("Leaf runtime: cannot open artifact ") + path);
        struct stat info;
        if (fstat(fd, &info) || info.st_size <= 0) {
            ::close(fd);
            throw leafhip::Error(LH_ERROR_ARTIFACT, "invalid decoder artifact size");
        }
        const size_t size = size_t(info.st_size);
        void* mapped = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (mapped == MAP_FAILED) throw leafhip::Error(LH_ERROR_ARTIFACT, "cannot map decoder artifact");
        try {
            leafhip::hip_check(hipSetDevice(context->impl.device), "hipSetDevice");
            auto model = leafhip::Model::load(context->impl, static_cast<const uint8_t*>(mapped), size,
                                              activation_bits, fp32_math);
            *out = new lh_model{std::move(model)};
        } catch (...) {
            munmap(mapped, size);
            throw;
        }
        // Weights now live on the device; the host mapping is no longer needed.
        munmap(mapped, size);
    });
}

lh_status lh_artifact_check(const void* artifact, size_t bytes, uint32_t activation_bits, uint32_t fp32_math) {
    return guarded([&] {
        require_arg(artifact != nullptr, "artifact bytes are required");
        (void)leafhip::read_artifact(static_cast<const uint8_t*>(artifact), bytes, activation_bits, fp32_math);
    });
}

lh_status lh_model_get_info(const lh_model* model, lh_model_info* out) {
    return guarded([&] {
        require_arg(model && out, "model and output are required");
        const auto& m = *model->impl;
        const auto& c = m.config;
        lh_model_info i{};
        i.version = c.version; i.hidden = c.hidden; i.intermediate = c.intermediate; i.heads = c.heads;
        i.kv_heads = c.kv_heads; i.layers = c.layers; i.vocab = c.vocab; i.max_positions = c.max_positions;
        i.eos = c.eos; i.head_dim = c.head_dim; i.sliding_window = c.sliding_window; i.theta = c.theta;
        i.epsilon = c.epsilon; i.norm_kind = c.norm_kind; i.activation = c.activation; i.position_kind = c.position_kind;
        i.gated = c.gated; i.parallel_residual = c.parallel; i.rotary_dim = c.rotary_dim;
        i.position_offset = c.position_offset; i.final_norm = c.final_norm; i.embedding_scale = c.embedding_scale;
        i.qk_norm = c.qk_norm; i.eos_count = uint32_t(c.eos_tokens.size());
        i.source_bf16_tensors = m.source_bf16_tensors; i.quantized_tensors = m.quantized_tensors;
        i.artifact_bytes = m.artifact_bytes; i.device_bytes = m.weights.bytes;
        *out = i;
    });
}

lh_status lh_model_eos_tokens(const lh_model* model, uint32_t* out, size_t capacity, size_t* count) {
    return guarded([&] {
        require_arg(model && count, "model and count are required");
        const auto& e = model->impl->config.eos_tokens;
        *count = e.size();
        if (out) {
            require_arg(capacity >= e.size(), "EOS buffer too small");
            std::copy(e.begin(), e.end(), out);
        }
    });
}

lh_status lh_model_destroy(lh_model* model) {
    return guarded([&] { delete model; });
}

lh_status lh_session_create(lh_model* model, const lh_session_options* options, lh_session** out) {
    return guarded([&] {
        require_arg(model && out, "model and output are required");
        leafhip::hip_check(hipSetDevice(model->impl->context.device), "hipSetDevice");
        const uint32_t context = options ? options->max_context : 0;
        const uint32_t prefill = options ? options->max_prefill : 0;
        const uint32_t numerics = options ? options->numerics : LH_NUMERICS_DEFAULT;
        *out = new lh_session{std::make_unique<leafhip::Session>(*model->impl, context, prefill, numerics)};
    });
}

lh_status lh_session_destroy(lh_session* session) {
    return guarded([&] { delete session; });
}

lh_status lh_reset(lh_session* session) {
    return guarded([&] {
        require_arg(session, "session is required");
        session->impl->reset();
    });
}

lh_status lh_cache_tokens(const lh_session* session, size_t* out) {
    return guarded([&] {
        require_arg(session && out, "session and output are required");
        *out = session->impl->cache_tokens();
    });
}

lh_status lh_forward(lh_session* session, const uint32_t* ids, size_t count, int all_logits, float* logits,
                     size_t logits_capacity, uint32_t* argmax) {
    return guarded([&] {
        require_arg(session && (ids || count == 0), "session and ids are required");
        leafhip::hip_check(hipSetDevice(session->impl->model.context.device), "hipSetDevice");
        session->impl->forward(ids, count, all_logits != 0, logits, logits_capacity, argmax);
    });
}

lh_status lh_generate(lh_session* session, const uint32_t* prompt, size_t count, uint32_t limit, uint32_t* tokens,
                      size_t* produced, double* prefill_ms, double* decode_ms) {
    return guarded([&] {
        require_arg(session && tokens && produced, "session, token buffer and count are required");
        auto& s = *session->impl;
        leafhip::hip_check(hipSetDevice(s.model.context.device), "hipSetDevice");
        using Clock = std::chrono::steady_clock;
        const auto& eos = s.model.config.eos_tokens;
        auto start = Clock::now();
        uint32_t id = 0;
        s.forward(prompt, count, false, nullptr, 0, &id);
        if (prefill_ms) *prefill_ms = std::chrono::duration<double, std::milli>(Clock::now() - start).count();
        size_t n = 0;
        for (uint32_t i = 0; i < limit; ++i) {
            tokens[n++] = id;
            if (std::find(eos.begin(), eos.end(), id) != eos.end()) break;
            if (i + 1 < limit) {
                start = Clock::now();
                const uint32_t next = id;
                s.forward(&next, 1, false, nullptr, 0, &id);
                if (decode_ms) decode_ms[i] = std::chrono::duration<double, std::milli>(Clock::now() - start).count();
            }
        }
        *produced = n;
    });
}

lh_status lh_session_set_profiling(lh_session* session, int enable) {
    return guarded([&] {
        require_arg(session, "session is required");
        session->impl->profiler.enabled = enable != 0;
    });
}

lh_status lh_session_profile(lh_session* session, lh_profile_entry* out, size_t capacity, size_t* count) {
    return guarded([&] {
        require_arg(session && count, "session and count are required");
        auto& p = session->impl->profiler;
        size_t n = 0;
        for (int k = 0; k < leafhip::Profiler::Count; ++k) {
            const auto& t = p.totals[k];
            if (!t.launches) continue;
            if (out && n < capacity) {
                lh_profile_entry e{};
                std::snprintf(e.name, sizeof(e.name), "%s", leafhip::Profiler::name(k));
                e.launches = t.launches;
                e.milliseconds = t.ms;
                e.bytes = t.bytes;
                e.operations = t.ops;
                out[n] = e;
            }
            ++n;
        }
        *count = n;
        if (out)
            for (auto& t : p.totals) t = leafhip::Profiler::Total();
    });
}

lh_status lh_session_status(const lh_session* session, int* reference_order, uint64_t* step_tokens,
                            uint64_t* step_memory_reruns, int* xcd_local) {
    return guarded([&] {
        require_arg(session && reference_order && step_tokens && step_memory_reruns && xcd_local,
                    "session and outputs are required");
        *reference_order = session->impl->reference_order() ? 1 : 0;
        *step_tokens = session->impl->step_tokens();
        *step_memory_reruns = session->impl->step_reruns();
        *xcd_local = session->impl->step_xcd_local() ? 1 : 0;
    });
}

lh_status lh_session_logits_device(const lh_session* session, const float** logits, size_t* count) {
    return guarded([&] {
        require_arg(session && logits && count, "session and outputs are required");
        *logits = session->impl->logits_device;
        *count = session->impl->logits_count;
    });
}

lh_status lh_device_alloc(size_t bytes, void** out) {
    return guarded([&] {
        require_arg(out, "output pointer is null");
        leafhip::hip_check(hipMalloc(out, bytes ? bytes : 1), "hipMalloc");
    });
}
lh_status lh_device_free(void* pointer) {
    return guarded([&] { leafhip::hip_check(hipFree(pointer), "hipFree"); });
}
lh_status lh_copy_to_device(void* dst, const void* src, size_t bytes) {
    return guarded([&] { leafhip::hip_check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy"); });
}
lh_status lh_copy_to_host(void* dst, const void* src, size_t bytes) {
    return guarded([&] { leafhip::hip_check(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy"); });
}
lh_status lh_memset_device(void* dst, int value, size_t bytes) {
    return guarded([&] { leafhip::hip_check(hipMemset(dst, value, bytes), "hipMemset"); });
}
lh_status lh_synchronize(void) {
    return guarded([&] { leafhip::hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize"); });
}
lh_status lh_stream_create(lh_stream* out) {
    return guarded([&] {
        require_arg(out, "output pointer is null");
        hipStream_t s;
        leafhip::hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
        *out = s;
    });
}
lh_status lh_stream_destroy(lh_stream stream) {
    return guarded([&] {
        require_arg(stream, "only a created stream can be destroyed");
        leafhip::hip_check(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
        release_stream_scratch(as_stream(stream));
        leafhip::hip_check(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
    });
}
lh_status lh_stream_synchronize(lh_stream stream) {
    return guarded([&] { leafhip::hip_check(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize"); });
}
lh_status lh_stream_begin_capture(lh_stream stream) {
    return guarded([&] {
        require_arg(stream, "capture needs a created stream");
        mark_stream_captured(as_stream(stream));
        leafhip::hip_check(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal),
                           "hipStreamBeginCapture");
    });
}
lh_status lh_stream_end_capture(lh_stream stream, lh_graph** out) {
    return guarded([&] {
        require_arg(stream && out, "stream and output are required");
        hipGraph_t graph;
        leafhip::hip_check(hipStreamEndCapture(as_stream(stream), &graph), "hipStreamEndCapture");
        hipGraphExec_t exec;
        const hipError_t st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        leafhip::hip_check(st, "hipGraphInstantiate");
        *out = new lh_graph{exec};
    });
}
lh_status lh_graph_launch(lh_graph* graph, lh_stream stream) {
    return guarded([&] {
        require_arg(graph, "graph is null");
        leafhip::hip_check(hipGraphLaunch(graph->exec, as_stream(stream)), "hipGraphLaunch");
    });
}
lh_status lh_graph_destroy(lh_graph* graph) {
    return guarded([&] {
        if (graph) (void)hipGraphExecDestroy(graph->exec);
        delete graph;
    });
}
lh_status lh_timer_start(lh_stream stream, lh_timer** out) {
    return guarded([&] {
        require_arg(out, "output pointer is null");
        auto* t = new lh_timer();
        leafhip::hip_check(hipEventCreate(&t->start), "hipEventCreate");
        leafhip::hip_check(hipEventCreate(&t->stop), "hipEventCreate");
        leafhip::hip_check(hipEventRecord(t->start, as_stream(stream)), "hipEventRecord");
        *out = t;
    });
}
lh_status lh_timer_stop(lh_timer* timer, lh_stream stream, double* milliseconds) {
    return guarded([&] {
        require_arg(timer, "timer is null");
        float ms = 0;
        leafhip::hip_check(hipEventRecord(timer->stop, as_stream(stream)), "hipEventRecord");
        leafhip::hip_check(hipEventSynchronize(timer->stop), "hipEventSynchronize");
        leafhip::hip_check(hipEventElapsedTime(&ms, timer->start, timer->stop), "hipEventElapsedTime");
        (void)hipEventDestroy(timer->start);
        (void)hipEventDestroy(timer->stop);
        delete timer;
        if (milliseconds) *milliseconds = ms;
    });
}

lh_status lh_set_kernel_numerics(uint32_t numerics) {
    return guarded([&] {
        require_arg(numerics != LH_NUMERICS_DEFAULT, "unknown numerics mode");
        const leafhip::NumericsMode mode = leafhip::resolve_numerics(numerics);
        t_reference_order = mode.reference;
        t_reference_vnni = mode.vnni;
    });
}

lh_status lh_expf(const float* x, size_t count, float* y, lh_stream stream) {
    return guarded([&] {
        require_arg(x && y, "input and output are required");
        if (!count) return;
        leafhip::launch_libm_expf(x, count, y, as_stream(stream));
        leafhip::hip_check(hipGetLastError(), "expf launch");
    });
}

lh_status lh_sequential_sum(const float* x, size_t n, size_t count, float* sums, int64_t* cycles, uint32_t method,
                            lh_stream stream) {
    return guarded([&] {
        require_arg(x && sums && n >= 1 && n <= size_t(leafhip::kSequentialSumMax) && count >= 1 &&
                        count <= 0x7fffffff && method <= 2,
                    "invalid sequential sum call");
        leafhip::launch_sequential_sum(x, int(n), int(count), sums, reinterpret_cast<long long*>(cycles),
                                       int(method), as_stream(stream));
        leafhip::hip_check(hipGetLastError(), "sequential sum launch");
    });
}

lh_status lh_quantize_rows_i8(const float* x, size_t rows, size_t cols, int8_t* q, float* scales, lh_stream stream) {
    return guarded([&] {
        require_arg(x && q && scales && rows && cols && rows <= 0x7fffffff && cols <= 0x7fffffff, "invalid quantization call");
        leafhip::launch_quantize(x, int(rows), int(cols), q, scales, as_stream(stream));
        leafhip::hip_check(hipGetLastError(), "quantize launch");
    });
}

lh_status lh_linear(const lh_weight* weight, const float* x, size_t tokens, uint32_t activation_bits, float* y,
                    int32_t* acc, lh_stream stream) {
    return linear_impl(weight, x, nullptr, nullptr, tokens, activation_bits, y, acc, stream, 0, 0);
}
lh_status lh_linear_noalloc(const lh_weight* weight, const float* x, size_t tokens, uint32_t activation_bits, float* y,
                            int32_t* acc, lh_stream stream) {
    return linear_impl(weight, x, nullptr, nullptr, tokens, activation_bits, y, acc, stream, 0, 0, true);
}
lh_status lh_linear_q(const lh_weight* weight, const int8_t* q, const float* scales, size_t tokens, float* y,
                      int32_t* acc, lh_stream stream) {
    if (!q || !scales) { g_error = "Leaf decoder: quantized input and scales are required"; return LH_ERROR_INVALID_ARGUMENT; }
    return linear_impl(weight, nullptr, q, scales, tokens, 8, y, acc, stream, 0, 0);
}
lh_status lh_gemv_f32(const lh_weight* w, const float* x, size_t tokens, float* y, lh_stream s) {
    return linear_impl(w, x, nullptr, nullptr, tokens, 32, y, nullptr, s, 0, 32);
}
lh_status lh_gemv_bf16(const lh_weight* w, const float* x, size_t tokens, float* y, lh_stream s) {
    return linear_impl(w, x, nullptr, nullptr, tokens, 32, y, nullptr, s, 0, 16);
}
lh_status lh_gemv_w8a32(const lh_weight* w, const float* x, size_t tokens, float* y, lh_stream s) {
    return linear_impl(w, x, nullptr, nullptr, tokens, 32, y, nullptr, s, 0, 8);
}
lh_status lh_gemv_w4a32(const lh_weight* w, const float* x, size_t tokens, float* y, lh_stream s) {
    return linear_impl(w, x, nullptr, nullptr, tokens, 32, y, nullptr, s, 0, 4);
}
lh_status lh_gemv_w8a8(const lh_weight* w, const float* x, size_t tokens, float* y, int32_t* acc, lh_stream s) {
    return linear_impl(w, x, nullptr, nullptr, tokens, 8, y, acc, s, 0, 8);
}
lh_status lh_gemv_w4a8(const lh_weight* w, const float* x, size_t tokens, float* y, int32_t* acc, lh_stream s) {
    return linear_impl(w, x, nullptr, nullptr, tokens, 8, y, acc, s, 0, 4);
}
lh_status lh_gemm_w8a8(const lh_weight* w, const float* x, size_t tokens, float* y, int32_t* acc, lh_stream s) {
    return linear_impl(w, x, nullptr, nullptr, tokens, 8, y, acc, s, 3, 8);
}
lh_status lh_gemm_f32(const lh_weight* w, const float* x, size_t tokens, float* y, lh_stream s) {
    return linear_impl(w, x, nullptr, nullptr, tokens, 32, y, nullptr, s, 3, 0);
}

lh_status lh_rmsnorm(const float* x, size_t rows, size_t width, const float* gamma, float epsilon, int accurate,
                     float* y, lh_stream stream) {
    return guarded([&] {
        require_arg(x && gamma && y && rows && width && rows <= 0x7fffffff && width <= 0x7fffffff, "invalid norm call");
        leafhip::NormView n{gamma, nullptr, epsilon, 0, accurate ? 1 : 0};
        if (t_reference_order) {
            require_arg(leafhip::launch_norm_reference_order(x, int(rows), int(width), n, y, as_stream(stream)),
                        "reference-order norm rows are at most 16384 wide");
        } else {
            leafhip::launch_norm(x, int(rows), int(width), n, y, as_stream(stream));
        }
        leafhip::hip_check(hipGetLastError(), "norm launch");
    });
}
lh_status lh_layernorm(const float* x, size_t rows, size_t width, const float* gamma, const float* beta, float epsilon,
                       float* y, lh_stream stream) {
    return guarded([&] {
        require_arg(x && gamma && y && rows && width && rows <= 0x7fffffff && width <= 0x7fffffff, "invalid norm call");
        leafhip::NormView n{gamma, beta, epsilon, 1, 0};
        if (t_reference_order) {
            require_arg(leafhip::launch_norm_reference_order(x, int(rows), int(width), n, y, as_stream(stream)),
                        "reference-order norm rows are at most 16384 wide");
        } else {
            leafhip::launch_norm(x, int(rows), int(width), n, y, as_stream(stream));
        }
        leafhip::hip_check(hipGetLastError(), "norm launch");
    });
}
lh_status lh_rope_kv(const float* qkv, size_t tokens, uint32_t heads, uint32_t kv_heads, uint32_t dim,
                     uint32_t rotary_dim, size_t position, const float* cosines, const float* sines, float* q_heads,
                     float* keys, float* values, size_t capacity, lh_stream stream) {
    return guarded([&] {
        require_arg(qkv && q_heads && keys && values && tokens && heads && kv_heads && dim && heads % kv_heads == 0,
                    "invalid rope call");
        require_arg(rotary_dim <= dim && rotary_dim % 2 == 0 && (!rotary_dim || (cosines && sines)), "invalid rotary dim");
        require_arg(position + tokens <= capacity && capacity <= 0x7fffffff, "KV append exceeds capacity");
        leafhip::RopeKvCall r;
        r.qkv = qkv; r.ld = int((heads + 2 * kv_heads) * dim); r.q_offset = 0; r.k_offset = int(heads * dim);
        r.v_offset = int((heads + kv_heads) * dim); r.tokens = int(tokens); r.heads = int(heads);
        r.kv_heads = int(kv_heads); r.dim = int(dim); r.rotary = int(rotary_dim); r.position = int(position);
        r.cosines = cosines; r.sines = sines; r.q_heads = q_heads; r.keys = keys; r.values = values;
        r.capacity = int(capacity);
        leafhip::launch_rope_kv(r, as_stream(stream));
        leafhip::hip_check(hipGetLastError(), "rope launch");
    });
}
lh_status lh_attention(const float* q_heads, const float* keys, const float* values, size_t capacity, uint32_t heads,
                       uint32_t kv_heads, uint32_t dim, size_t tokens, size_t position, uint32_t window, float* out,
                       lh_stream stream) {
    return guarded([&] {
        require_arg(q_heads && keys && values && out && heads && kv_heads && heads % kv_heads == 0 && tokens,
                    "invalid attention call");
        require_arg(dim > 0 && dim <= 256, "head dim must be 1..256");
        require_arg(position + tokens <= capacity && capacity <= 0x7fffffff, "attention span exceeds the cache");
        leafhip::AttentionCall a;
        a.q_heads = q_heads; a.keys = keys; a.values = values; a.out = out; a.heads = int(heads);
        a.kv_heads = int(kv_heads); a.tokens = int(tokens); a.position = int(position); a.dim = int(dim);
        a.capacity = int(capacity); a.window = int(window);
        a.scale = 1.0f / std::sqrt(std::sqrt(static_cast<float>(dim)));
        if (t_reference_order) {
            size_t keys = position + tokens;
            if (window) keys = std::min<size_t>(keys, window);
            require_arg(keys <= size_t(leafhip::reference_order_attention_keys()),
                        "too many keys for one query in reference order");
            leafhip::check(leafhip::launch_attention_reference_order(a, int(keys), as_stream(stream)),
                           "attention launch rejected", LH_ERROR_UNSUPPORTED);
            leafhip::hip_check(hipGetLastError(), "attention launch");
            return;
        }
        if (tokens == 1 && kv_heads <= 1024) {
            const size_t floats = ((position + tokens + 15) / 16) * heads * (dim + 2);
            a.partial = static_cast<float*>(scratch_bytes(floats * sizeof(float), as_stream(stream)));
            a.partial_capacity = int(floats);
            a.counters = attention_counters(as_stream(stream));
        }
        leafhip::check(leafhip::launch_attention(a, as_stream(stream)), "attention launch rejected", LH_ERROR_UNSUPPORTED);
        leafhip::hip_check(hipGetLastError(), "attention launch");
    });
}
lh_status lh_silu_gate(const float* gate_up, size_t tokens, size_t width, float* out, lh_stream stream) {
    return guarded([&] {
        require_arg(gate_up && out && tokens && width && tokens * width <= 0x7fffffff, "invalid SiLU call");
        if (t_reference_order)
            leafhip::launch_activation_reference_order(gate_up, int(tokens), int(width), 1, 0, out, as_stream(stream));
        else
            leafhip::launch_activation(gate_up, int(tokens), int(width), 1, 0, out, as_stream(stream));
        leafhip::hip_check(hipGetLastError(), "activation launch");
    });
}
lh_status lh_activation(const float* x, size_t count, uint32_t activation, float* out, lh_stream stream) {
    return guarded([&] {
        require_arg(x && out && count && count <= 0x7fffffff && activation <= 3, "invalid activation call");
        if (t_reference_order)
            leafhip::launch_activation_reference_order(x, 1, int(count), 0, int(activation), out, as_stream(stream));
        else
            leafhip::launch_activation(x, 1, int(count), 0, int(activation), out, as_stream(stream));
        leafhip::hip_check(hipGetLastError(), "activation launch");
    });
}
lh_status lh_argmax(const float* logits, size_t rows, size_t width, uint32_t* out, lh_stream stream) {
    return guarded([&] {
        require_arg(logits && out && rows && width && rows <= 0x7fffffff && width <= 0x7fffffff, "invalid argmax call");
        leafhip::launch_argmax(logits, int(rows), int(width), out, as_stream(stream));
        leafhip::hip_check(hipGetLastError(), "argmax launch");
    });
}

}  // extern "C"
