/*
 * leafhip: C ABI of the MI355X (gfx950) decoder path.
 *
 * Drop-in boundary for Leaf's native decoder runtime.  The reference exposes
 * the C++ class leaf::runtime::Decoder (engine/include/leaf/runtime/decoder.h:15-50)
 * and the leaf_decoder process protocol (engine/src/main_decoder.cpp:116-363);
 * this header is what a C++ Decoder wrapper (include/leafhip_decoder.hpp),
 * the leaf_decoder-compatible executable and any FFI binding call instead.
 *
 * Conventions:
 *  - every function returns lh_status (LH_OK == 0) and never throws;
 *    lh_last_error() holds a thread-local message for the last failure,
 *    formatted like the reference's errors ("Leaf decoder: <what>").
 *  - pointers documented as "device" are HIP device pointers; lh_stream is a
 *    hipStream_t (NULL selects the default stream); sizes are element counts.
 *  - no allocation, type or exception crosses the ABI.
 */
#ifndef LEAFHIP_H
#define LEAFHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t lh_status;
#define LH_OK 0
#define LH_ERROR_INVALID_ARGUMENT 1 /* bad shapes, ids, sizes (reference: invalid_argument / check()) */
#define LH_ERROR_ARTIFACT 2         /* artifact rejected by validation (decoder.cpp:787-933) */
#define LH_ERROR_DEVICE 3           /* a HIP runtime error */
#define LH_ERROR_OUT_OF_MEMORY 4
#define LH_ERROR_STATE 5            /* e.g. context length exceeded (decoder.cpp:1288) */
#define LH_ERROR_UNSUPPORTED 6

typedef struct lh_context lh_context;
typedef struct lh_model lh_model;
typedef struct lh_session lh_session;
typedef void* lh_stream;

/* Thread-local text of the last failure on this thread ("" when none). */
const char* lh_last_error(void);
/* Library version string. */
const char* lh_version(void);

/* ---------------------------------------------------------------- context */
/* Selects a GPU and creates the library's stream on it.  No reference
 * counterpart: the CPU reference has no device. */
lh_status lh_context_create(int device, lh_context** out);
lh_status lh_context_destroy(lh_context* context);

/* ------------------------------------------------------------------ model */
typedef struct lh_model_info {
    uint32_t version;          /* LEAFDC0v */
    uint32_t hidden, intermediate, heads, kv_heads, layers, vocab, max_positions;
    uint32_t eos;              /* 0xffffffff = none */
    uint32_t head_dim, sliding_window;
    float theta, epsilon;
    uint32_t norm_kind, activation, position_kind, gated, parallel_residual;
    uint32_t rotary_dim, position_offset, final_norm;
    float embedding_scale;
    uint32_t qk_norm;
    uint32_t eos_count;
    uint32_t source_bf16_tensors;  /* Decoder::source_bf16_tensors (decoder.h:43) */
    uint32_t quantized_tensors;    /* INT8 / INT4 tensors */
    uint64_t artifact_bytes;       /* Decoder::weight_bytes (decoder.h:37) */
    uint64_t device_bytes;         /* device memory holding the weights */
} lh_model_info;

/* Validates a LEAFDC02..07 artifact exactly as Decoder::Impl::Impl does
 * (engine/src/decoder.cpp:787-933, same messages) and uploads every tensor
 * once into device memory.  `activation_bits` (8 or 32) and `fp32_math`
 * (0 fast, 1 accurate) are the reference constructor's policy arguments
 * (decoder.h:17-19); they are checked here because some artifacts reject
 * them (source BF16 requires 32; accurate requires unquantized weights). */
lh_status lh_model_load_file(lh_context* context, const char* path, uint32_t activation_bits,
                             uint32_t fp32_math, lh_model** out);
/* Same from a caller-mapped artifact (the caller keeps the bytes alive only
 * for the duration of the call). */
lh_status lh_model_load(lh_context* context, const void* artifact, size_t bytes, uint32_t activation_bits,
                        uint32_t fp32_math, lh_model** out);
/* The artifact validation of lh_model_load alone, on the host (no device):
 * LH_OK when the CPU reference's loader accepts the artifact (decoder.cpp:787-933)
 * and its first use of each tensor would pass (decoder.cpp:975-1024), else
 * the status and, in lh_last_error, the reference's message for the first
 * problem.  No reference counterpart as a separate call. */
lh_status lh_artifact_check(const void* artifact, size_t bytes, uint32_t activation_bits, uint32_t fp32_math);
lh_status lh_model_get_info(const lh_model* model, lh_model_info* out);
/* EOS token set (decoder.cpp:842-857; Decoder::is_eos_token, decoder.h:35). */
lh_status lh_model_eos_tokens(const lh_model* model, uint32_t* out, size_t capacity, size_t* count);
lh_status lh_model_destroy(lh_model* model);

/* ---------------------------------------------------------------- session */
/* Floating-point order of a session's kernels.
 *  FAST: parallel reductions (per-lane partials, wave trees, key spans merged
 *    by log-sum-exp) and the device's libm.  Integer stages stay bit-exact;
 *    FP32 logits stay within 1e-3 of the CPU path, W8A8 ones within a few
 *    percent (a one-ulp change upstream of a quantization can move an int8 bin).
 *  REFERENCE: the CPU path's summation orders (sequential norm and softmax
 *    sums, dot_avx's lane chains) and glibc's expf, so logits equal the CPU
 *    reference's bit for bit, hence identical greedy tokens, for decoders with
 *    SiLU or ReLU activations and fast FP32 math (GELU uses the device's
 *    erff / tanhf; accurate FP32 math is rejected).  Slower.
 *    The CPU path sums the groups of a grouped INT8 linear over several
 *    tokens in two ways, chosen by its host: fused multiply-adds
 *    (quant_tile_avx, decoder.cpp:571-617) or, on AVX-VNNI hosts unless
 *    LEAF_DISABLE_VNNI is set, a multiply and an add (quant_vnni_tile,
 *    :661-702; selection at :780-782, 1022).  REFERENCE follows this host as
 *    the CPU path would; REFERENCE_AVX2 / REFERENCE_VNNI pin either form.
 *    A REFERENCE session holds at most 32,448 visible keys per query (one
 *    query's scores sit in LDS); a larger requested max_context is refused
 *    with LH_ERROR_UNSUPPORTED, and max_context 0 stops there.
 *  DEFAULT: REFERENCE for a model loaded with 8-bit activations (W8A8),
 *    FAST otherwise, unless the environment variable LEAF_GPU_NUMERICS names
 *    a mode: fast, reference, reference-avx2 or reference-vnni. */
#define LH_NUMERICS_DEFAULT 0
#define LH_NUMERICS_FAST 1
#define LH_NUMERICS_REFERENCE 2
#define LH_NUMERICS_REFERENCE_AVX2 3
#define LH_NUMERICS_REFERENCE_VNNI 4

typedef struct lh_session_options {
    uint32_t max_context;  /* KV capacity in tokens; 0 = the artifact's max_positions */
    uint32_t max_prefill;  /* tokens per forward the workspaces are planned for; 0 = 512 (grown on demand) */
    uint32_t numerics;     /* LH_NUMERICS_*; no reference counterpart (the CPU has one order) */
} lh_session_options;

/* A decoding session: preallocated device KV cache for max_context tokens,
 * device workspaces and RoPE tables (one memory plan, reused by every
 * forward).  The reference equivalent is the per-instance state of
 * Decoder (KV caches and workspaces, decoder.cpp:730-765). */
lh_status lh_session_create(lh_model* model, const lh_session_options* options, lh_session** out);
lh_status lh_session_destroy(lh_session* session);
/* Decoder::reset (decoder.h:23): logical length to zero, capacity kept. */
lh_status lh_reset(lh_session* session);
/* Decoder::cache_tokens (decoder.h:36). */
lh_status lh_cache_tokens(const lh_session* session, size_t* out);
/* Decoder::forward_into (decoder.h:31-32): appends `count` tokens; writes
 * [vocab] logits of the last token, or [count, vocab] when all_logits, into
 * host memory `logits` (capacity in floats; may be NULL to skip the copy).
 * `argmax` (may be NULL) receives the first maximal index of the last row,
 * computed on the device (main_decoder.cpp:102).  Inputs are validated
 * before any state changes (decoder.cpp:1286-1289). */
lh_status lh_forward(lh_session* session, const uint32_t* ids, size_t count, int all_logits, float* logits,
                     size_t logits_capacity, uint32_t* argmax);
/* generate_continuation (main_decoder.cpp:95-113): prefill, then greedy
 * decode until `limit` tokens or an EOS token.  Per-step wall times in ms
 * (decode_ms has room for limit entries; either may be NULL). */
lh_status lh_generate(lh_session* session, const uint32_t* prompt, size_t count, uint32_t limit, uint32_t* tokens,
                      size_t* produced, double* prefill_ms, double* decode_ms);
/* Device-side phase profile, the GPU counterpart of LEAF_DECODER_PROFILE
 * (decoder.cpp:119-230): when enabled, every launch of a forward is bracketed
 * by HIP events on the session's stream and accumulated per kernel class,
 * with the algorithmic bytes it had to move.  Classes: "gemv_w8a8",
 * "gemv_fp", "gemm_w8a8", "gemm_fp", "attention", "other". */
typedef struct lh_profile_entry {
    char name[24];
    uint64_t launches;
    double milliseconds;
    double bytes;          /* algorithmic HBM bytes (weights, scales, inputs, outputs) */
    double operations;     /* multiply-adds x 2 */
} lh_profile_entry;
lh_status lh_session_set_profiling(lh_session* session, int enable);
/* Copies the accumulated entries and clears them. */
lh_status lh_session_profile(lh_session* session, lh_profile_entry* out, size_t capacity, size_t* count);
/* The session's numerics and the persistent decode step's record since the
 * session began (no counterpart in the reference; for benchmarks and
 * monitoring): whether the kernels follow the CPU engine's float order
 * (LH_NUMERICS_DEFAULT resolved); tokens the persistent step produced; how
 * many of those steps ran a second time on the memory exchange path because a
 * block found itself off the XCD its index names; and whether the XCD-local
 * exchange is still on (it is switched off for the session after four such
 * steps in a row, or when the session never had it). */
lh_status lh_session_status(const lh_session* session, int* reference_order, uint64_t* step_tokens,
                            uint64_t* step_memory_reruns, int* xcd_local);
/* Device pointer of the last forward's logits (valid until the next call). */
lh_status lh_session_logits_device(const lh_session* session, const float** logits, size_t* count);

/* ------------------------------------------------- device memory helpers */
lh_status lh_device_alloc(size_t bytes, void** out);
lh_status lh_device_free(void* pointer);
lh_status lh_copy_to_device(void* device_dst, const void* host_src, size_t bytes);
lh_status lh_copy_to_host(void* host_dst, const void* device_src, size_t bytes);
lh_status lh_memset_device(void* device_dst, int value, size_t bytes);
lh_status lh_synchronize(void);
/* The kernel-level entry points keep their device scratch per (device, stream
 * handle), at least 1 MiB per stream once used.  lh_stream_destroy waits for
 * the stream and frees that scratch; the scratch of a stream that was ever
 * captured stays allocated until the process ends, since a graph captured
 * from it may still be launched. */
lh_status lh_stream_create(lh_stream* out);
lh_status lh_stream_destroy(lh_stream stream);
lh_status lh_stream_synchronize(lh_stream stream);
/* Capture the work submitted to `stream` into a replayable graph (HIP graph).
 * Only kernel-level entry points may be called on the stream while capturing. */
typedef struct lh_graph lh_graph;
lh_status lh_stream_begin_capture(lh_stream stream);
lh_status lh_stream_end_capture(lh_stream stream, lh_graph** out);
lh_status lh_graph_launch(lh_graph* graph, lh_stream stream);
lh_status lh_graph_destroy(lh_graph* graph);
/* Device-side timing of work submitted to `stream` (HIP events). */
typedef struct lh_timer lh_timer;
lh_status lh_timer_start(lh_stream stream, lh_timer** out);
lh_status lh_timer_stop(lh_timer* timer, lh_stream stream, double* milliseconds); /* destroys the timer */

/* ------------------------------------------------- kernel-level entry points
 * Numerics of this thread's later kernel-level calls (LH_NUMERICS_FAST or
 * one of the LH_NUMERICS_REFERENCE modes, as for sessions): lh_rmsnorm,
 * lh_layernorm, lh_attention, lh_silu_gate, lh_activation and the FP paths
 * of lh_linear, lh_gemv_{f32,bf16,w8a32,w4a32} and lh_gemm_f32 follow it;
 * integer accumulators are exact in every mode, and grouped INT8 sums over
 * several tokens take the mode's CPU form.  No reference counterpart. */
lh_status lh_set_kernel_numerics(uint32_t numerics);
/* y[i] = expf(x[i]) with the result glibc 2.35's expf returns on x86-64 with
 * FMA (the exp of the CPU path's softmax and SiLU, transformer.cpp:134,
 * decoder.cpp:983), for every float input (a NaN input gives a NaN, its
 * payload unspecified). */
lh_status lh_expf(const float* x, size_t count, float* y, lh_stream stream);
/* sums[i] = (...((0 + x[i][0]) + x[i][1]) + ...) + x[i][n - 1] in float, the
 * order in which norm() sums its squares and attention_impl its softmax
 * denominator (decoder.cpp:716-718, transformer.cpp:127-130), for count rows
 * of n <= 8192 values.  Method 0 forms that sum in parallel on one wave and
 * method 2 on two waves (the reference-order decode step's ways;
 * bit-identical); method 1 adds one by one.  Rows with a negative value take
 * method 1.  cycles (may be NULL): the GPU clock cycles each row's sum took.
 * No reference counterpart: a diagnostic of this build. */
lh_status lh_sequential_sum(const float* x, size_t n, size_t count, float* sums, int64_t* cycles,
                            uint32_t method, lh_stream stream);

/* One weight matrix as stored in a LEAFDC artifact (Weight, decoder.cpp:236-251):
 * bits 32 = f32, 16 = BF16 bits, 8 = int8, 4 = signed nibbles (low = even column);
 * scales[row * (cols / group) + col / group] for bits 8 and 4; bias may be NULL.
 * All pointers are device pointers. */
typedef struct lh_weight {
    const void* data;
    const float* scales;
    const float* bias;
    uint32_t rows, cols, bits, group;
} lh_weight;

/* Per-token activation quantization (decoder.cpp:1020-1044, quantize_input_avx :618-627):
 * scales[r] = max(max|x[r,:]| / 127, 1e-12); q = round-half-even(x / scale), +-127. */
lh_status lh_quantize_rows_i8(const float* x, size_t rows, size_t cols, int8_t* q, float* scales, lh_stream stream);

/* Decoder::Impl::linear (decoder.cpp:994-1233) for one matrix: y[tokens, rows] = x W^T + b.
 * activation_bits 8 quantizes x per token (W8A8 / W4A8, bits 8/4 only);
 * 32 computes in FP32 (FP32, BF16-source, W8A32, W4A32).  acc (may be NULL)
 * receives the exact int32 group accumulators [tokens][rows][cols/group]
 * of the integer path.  Decode-sized calls (tokens <= 4) run the GEMV kernels,
 * larger ones the MFMA GEMMs. */
lh_status lh_linear(const lh_weight* weight, const float* x, size_t tokens, uint32_t activation_bits, float* y,
                    int32_t* acc, lh_stream stream);
/* lh_linear without any allocation.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The integer path's
 * scratch -- the quantized input, its per-token scales and split-K sums -- is
 * a fixed device array of LH_NOALLOC_SCRATCH_BYTES per GPU, present from
 * library load until the process ends; nothing in it has to start at zero.
 * A call whose quantized input and scales need more than the array
 * (about tokens * (cols + 4) bytes) fails with LH_ERROR_INVALID_ARGUMENT;
 * the split-K sums use what is left.  Every call on one GPU shares the
 * array: calls that overlap (other streams, other threads) race.  Results
 * equal lh_linear's bit for bit. */
#define LH_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
lh_status lh_linear_noalloc(const lh_weight* weight, const float* x, size_t tokens, uint32_t activation_bits,
                            float* y, int32_t* acc, lh_stream stream);
/* The integer path from already-quantized activations (q [tokens, cols], scales [tokens]). */
lh_status lh_linear_q(const lh_weight* weight, const int8_t* q, const float* scales, size_t tokens, float* y,
                      int32_t* acc, lh_stream stream);
/* Typed entry points; each checks the storage it names, then runs lh_linear.
 * Decode GEMVs: dot_avx / dot_source_bf16_avx / quant_dot_avx (decoder.cpp:355-420, 536-570). */
lh_status lh_gemv_f32(const lh_weight* weight, const float* x, size_t tokens, float* y, lh_stream stream);
lh_status lh_gemv_bf16(const lh_weight* weight, const float* x, size_t tokens, float* y, lh_stream stream);
lh_status lh_gemv_w8a32(const lh_weight* weight, const float* x, size_t tokens, float* y, lh_stream stream);
lh_status lh_gemv_w4a32(const lh_weight* weight, const float* x, size_t tokens, float* y, lh_stream stream);
lh_status lh_gemv_w8a8(const lh_weight* weight, const float* x, size_t tokens, float* y, int32_t* acc,
                       lh_stream stream);
lh_status lh_gemv_w4a8(const lh_weight* weight, const float* x, size_t tokens, float* y, int32_t* acc,
                       lh_stream stream);
/* Prefill GEMMs: quant_tile_avx / quant_vnni_tile (decoder.cpp:571-702) and the
 * FP32 token-panel GEMMs (token_panel.h:290-336, accurate_fp32.h:140-166). */
lh_status lh_gemm_w8a8(const lh_weight* weight, const float* x, size_t tokens, float* y, int32_t* acc,
                       lh_stream stream);
lh_status lh_gemm_f32(const lh_weight* weight, const float* x, size_t tokens, float* y, lh_stream stream);

/* norm() (decoder.cpp:706-727): RMSNorm (accurate = FP64 square sum,
 * accurate_fp32.h:6-13) and LayerNorm with optional beta. */
lh_status lh_rmsnorm(const float* x, size_t rows, size_t width, const float* gamma, float epsilon, int accurate,
                     float* y, lh_stream stream);
lh_status lh_layernorm(const float* x, size_t rows, size_t width, const float* gamma, const float* beta,
                       float epsilon, float* y, lh_stream stream);
/* rotary() + KV append (decoder.cpp:1259-1281, 1332-1343) for `tokens` rows of
 * qkv [tokens, (heads + 2 kv_heads) * dim] at `position`: q -> q_heads
 * [heads, tokens, dim]; k, v -> caches [kv_heads, capacity, dim].
 * cosines/sines are [positions, rotary/2] tables (prepare_rotary_tables, :1234-1258). */
lh_status lh_rope_kv(const float* qkv, size_t tokens, uint32_t heads, uint32_t kv_heads, uint32_t dim,
                     uint32_t rotary_dim, size_t position, const float* cosines, const float* sines,
                     float* q_heads, float* keys, float* values, size_t capacity, lh_stream stream);
/* Causal GQA attention over a KV cache (KVCache::attend, kv_cache.cpp:65-84;
 * attention_impl, transformer.cpp:94-146): queries at positions
 * [position, position + tokens), keys [0, position + tokens), optional
 * sliding window; scores (q.k * scale) * scale with scale = 1/sqrt(sqrt(dim)). */
lh_status lh_attention(const float* q_heads, const float* keys, const float* values, size_t capacity,
                       uint32_t heads, uint32_t kv_heads, uint32_t dim, size_t tokens, size_t position,
                       uint32_t window, float* out, lh_stream stream);
/* SiLU gate (decoder.cpp:1414): out = up * silu(gate); gate_up = [tokens, 2 * width] = [gate | up]. */
lh_status lh_silu_gate(const float* gate_up, size_t tokens, size_t width, float* out, lh_stream stream);
/* activate() (decoder.cpp:982-987) for activation codes 1 (erf GELU) / 2 (tanh GELU) / 3 (ReLU), elementwise. */
lh_status lh_activation(const float* x, size_t count, uint32_t activation, float* out, lh_stream stream);
/* First maximal index per row (main_decoder.cpp:102). */
lh_status lh_argmax(const float* logits, size_t rows, size_t width, uint32_t* out, lh_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* LEAFHIP_H */
