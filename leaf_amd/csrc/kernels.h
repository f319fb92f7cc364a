// Host-visible launch interface of the decoder kernels (gfx950).
//
// Each launcher validates nothing: callers (the C ABI and the decoder) check
// shapes first.  All pointers are device pointers; `stream` is a hipStream_t.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace leafhip {

// One weight matrix [rows, cols] as stored in a LEAFDC artifact (decoder.cpp:236-251):
// bits 32 = f32, 16 = BF16 bits, 8 = int8, 4 = two signed nibbles per byte
// (low nibble = even column); scales[row * (cols / group) + col / group] for 8/4.
struct WeightView {
    const void* data = nullptr;
    const float* scales = nullptr;
    const float* bias = nullptr;    // null adds 0.0f, as the CPU path does without a bias
    int rows = 0, cols = 0, bits = 32, group = 0;
};

// Optional normalization applied to the input rows of a linear (decoder.cpp:706-727).
struct NormView {
    const float* gamma = nullptr;
    const float* beta = nullptr;
    float epsilon = 0.0f;
    int kind = -1;                  // -1 none, 0 RMS, 1 LayerNorm
    int accurate = 0;               // RMS square sum in double (accurate_fp32.h:6-13)
    int sequential = 0;             // mean and square sums in column order (decoder.cpp:706-727)
};

enum Epilogue : int {
    kStore = 0,     // y = acc + bias
    kAccumulate = 1 // y = y + (acc + bias)      (residual add, decoder.cpp:1390)
};

// Token-major activations use row stride == width unless stated.
void launch_embedding(const WeightView& table, const WeightView* positions, const uint32_t* ids, int tokens,
                      int position_base, float scale, float* hidden, hipStream_t stream,
                      const int* position_ptr = nullptr);
// Rows are contiguous, or (rows_per_group > 0) in groups of rows_per_group
// contiguous rows, group_stride floats from one group's start to the next.
void launch_norm(const float* x, int rows, int width, const NormView& norm, float* y, hipStream_t stream,
                 int rows_per_group = 0, size_t group_stride = 0);
void launch_quantize(const float* x, int rows, int width, int8_t* q, float* scales, hipStream_t stream);
// norm_kernel + quantize_kernel in one launch (same q and scales, no f32 row in between)
void launch_norm_quantize(const float* x, int rows, int width, const NormView& norm, int8_t* q, float* scales,
                          hipStream_t stream);
// activation_kernel + quantize_kernel in one launch
void launch_activation_quantize(const float* gate_up, int tokens, int width, int gated, int activation, int8_t* q,
                                float* scales, hipStream_t stream);
void launch_scale_columns(const float* x, int rows, int width, const float* factors, float* y,
                          hipStream_t stream);

// Epilogues over pairs of output rows computed by one wave (single token):
//  kPairRopeKv: rows are a stacked [q | k | v] projection; rotate-half pairs
//    (i, i + rotary/2) of q and k heads with the host-built tables, write q to
//    q_heads [heads, 1, dim] and k, v into the caches at `position`
//    (rotary() and KVCache::append, decoder.cpp:1259-1281, 1332-1343);
//  kPairGated: rows are a stacked [gate | up] projection; act[j] =
//    up[j] * activate(gate[j]) (decoder.cpp:1396-1414);
//  kPairActivation (single-token FP linears only): not a pair, each row's
//    output is stored as activate(value) (an ungated MLP's up projection).
enum PairMode : int { kPairNone = 0, kPairRopeKv = 1, kPairGated = 2, kPairActivation = 3 };
struct PairEpilogue {
    int mode = kPairNone;
    int heads = 0, kv_heads = 0, dim = 0, rotary = 0, position = 0, capacity = 0;
    const int* position_ptr = nullptr;  // when set, the position is read from device memory
    const float* cosines = nullptr;
    const float* sines = nullptr;
    float* q_heads = nullptr;
    float* keys = nullptr;
    float* values = nullptr;
    int width = 0, activation = 0;
    float* act = nullptr;
    int reference = 0;              // gated: SiLU with the CPU's libm expf (libm_expf.h)
};

// y[t, row] for t < tokens.  integer_activations selects W8A8/W4A8 (bits 8/4):
// then either x (f32, quantized per token inside the kernel) or xq/xs (given).
// acc_out, when not null, receives the exact int32 group accumulators
// [tokens][rows][cols/group] (integer path only).
struct LinearCall {
    WeightView w;
    const float* x = nullptr;
    const int8_t* xq = nullptr;
    const float* xs = nullptr;
    NormView norm;                  // applied to x first (integer path, tokens == 1 only)
    int tokens = 1;
    bool integer_activations = false;
    float* y = nullptr;
    int epilogue = kStore;
    int32_t* acc_out = nullptr;
    int8_t* xq_scratch = nullptr;   // [tokens, cols] when the GEMM path quantizes
    float* xs_scratch = nullptr;    // [tokens]
    float* norm_scratch = nullptr;  // [tokens, cols] when `norm` cannot be fused into the kernel
    int force_path = 0;             // 0 auto, 1 GEMV, 2 generic, 3 GEMM
    int32_t* split_scratch = nullptr;   // split-K int32 sums for the W8A8 GEMM; may be null
    size_t split_capacity = 0;          // int32 elements available in split_scratch
    PairEpilogue pair;              // single-token paired epilogue (y unused when set)
    // Integer path, tokens > 1: sum the groups as quant_vnni_tile does,
    // res + ((float)acc * s_x) * s_w with two roundings, instead of fused.
    bool unfused_group_sum = false;
};
// W8A8 prefill GEMM on int8 MFMA (gemm_w8a8.hip) for per-row weight scales:
// y[t, n] = ((float)sum_k xq[t, k] W[n, k] * xs[t]) * w_scales[n] + bias[n]
// (kStore) or y += that (kAccumulate).  K % 128 == 0.  Blocks own
// tiles.rows weight rows x tiles.tokens tokens; with partial set the K range
// is split tiles.splits ways and the exact int32 sums go to
// partial[split][t][n] instead of y (acc_out and the epilogue are then the
// split epilogue's).
struct GemmTiles {
    int rows = 64, tokens = 64, splits = 1;
};
bool gemm_w8a8_mfma_supported(int K);
// The tile shape and K split for an M x N x K product; splits > 1 only when
// 2 * splits * M * N int32 sums fit in split_capacity.
GemmTiles gemm_w8a8_tiles(int M, int N, int K, size_t split_capacity);
void launch_gemm_w8a8_mfma(const int8_t* W, const float* w_scales, const float* bias, const int8_t* xq,
                           const float* xs, int M, int N, int K, float* y, int epilogue, int32_t* acc_out,
                           const GemmTiles& tiles, int32_t* partial, hipStream_t stream);

// Returns the path used (1 GEMV, 2 generic, 3 GEMM) or a negative value when
// the call cannot run (missing scratch for the GEMM quantization).
// FP32-math prefill GEMM on f32 MFMA with LDS-staged tiles (gemm_f32.hip):
// K % 32 == 0, 16-byte aligned input and weights, quantized groups % 16 == 0.
bool gemm_f32_lds_supported(const WeightView& w, const float* x);
void launch_gemm_f32_lds(const WeightView& w, const float* x, int tokens, float* y, int epilogue,
                         hipStream_t stream);

int launch_linear(const LinearCall& call, hipStream_t stream);
// True when launch_linear runs the single-token integer GEMV that normalizes,
// quantizes and applies paired epilogues inside the kernel.
bool linear_fuses(const LinearCall& call);

// RoPE + head-major reorder + KV append for `tokens` new tokens at `position`.
// qkv is [tokens, qwidth + 2 * kvwidth]; q_heads gets [heads, tokens, dim];
// key/value caches are [kv_heads, capacity, dim].
struct RopeKvCall {
    const float* qkv = nullptr;
    int ld = 0;                     // row stride of qkv
    int q_offset = 0, k_offset = 0, v_offset = 0;
    int tokens = 0, heads = 0, kv_heads = 0, dim = 0, rotary = 0;
    int position = 0;
    const int* position_ptr = nullptr;  // when set, the position is read from device memory
    const float* cosines = nullptr; // [positions, rotary/2] tables built on the host
    const float* sines = nullptr;
    float* q_heads = nullptr;
    float* keys = nullptr;
    float* values = nullptr;
    int capacity = 0;
};
void launch_rope_kv(const RopeKvCall& call, hipStream_t stream);

// Causal (optionally sliding-window) GQA attention of `tokens` queries at
// positions [position, position+tokens) over keys [0, position+tokens).
struct AttentionCall {
    const float* q_heads = nullptr; // [heads, tokens, dim]
    const float* keys = nullptr;    // [kv_heads, capacity, dim]
    const float* values = nullptr;
    float* out = nullptr;           // [tokens, heads * dim]
    int heads = 0, kv_heads = 0, tokens = 0, position = 0, dim = 0, capacity = 0, window = 0;
    const int* position_ptr = nullptr;  // decode only: position read from device memory
    int spans = 0;                  // decode only: fixed number of key spans (0 = from position)
    float scale = 1.0f;             // applied twice: (q.k * scale) * scale (decoder.cpp:1348)
    float* partial = nullptr;       // split-K scratch (decode); may be null
    int partial_capacity = 0;       // floats available in partial
    unsigned* counters = nullptr;   // kv_heads zero-initialized counters (decode); reset by the kernel
};
// Returns false when the call cannot run: a device-resident position
// (position_ptr) is only supported by the single-token decode kernels.
bool launch_attention(const AttentionCall& call, hipStream_t stream);

// act = up * activate(gate) for gated MLPs, act = activate(up) otherwise.
// gate_up holds [tokens, 2 * width] = [gate | up] when gated, [tokens, width] otherwise.
void launch_activation(const float* gate_up, int tokens, int width, int gated, int activation, float* act,
                       hipStream_t stream);
// hidden = hidden + (a + (b ? b : 0))   (decoder.cpp:1434)
void launch_residual(float* hidden, const float* a, const float* b, int count, hipStream_t stream);
// index of the first maximum of each row (std::max_element, main_decoder.cpp:102)
void launch_argmax(const float* logits, int rows, int width, uint32_t* out, hipStream_t stream);
// Greedy step on the device: argmax of one row into next_id[0] and host_out[0]
// (mapped host memory, may be null), then position[0] += 1.  Many blocks take
// a part of the row each, a second launch combines their results; scratch
// holds argmax_scratch_floats() floats.
void launch_argmax_advance(const float* logits, int width, uint32_t* next_id, uint32_t* host_out, int* position,
                           float* scratch, hipStream_t stream);
// The same for one row without the greedy step.
void launch_argmax_row(const float* logits, int width, uint32_t* out, float* scratch, hipStream_t stream);
int argmax_scratch_floats();
// Number of key spans the decode attention uses for `keys` visible keys.
int attention_decode_spans(int keys, int dim);
// Whether single-token attention runs the span kernels (graph-capturable).
bool attention_decode_supported(int heads, int kv_heads, int dim);

// ---- reference-order kernels (reference_order.hip): the CPU path's
// summation orders and libm results, so logits match it bit for bit.
constexpr int kReferenceOrderMaxWidth = 16384;   // norm rows staged in LDS
// norm() with sequential sums; false when width exceeds kReferenceOrderMaxWidth.
bool launch_norm_reference_order(const float* x, int rows, int width, const NormView& norm, float* y,
                                 hipStream_t stream, int rows_per_group = 0, size_t group_stride = 0);
// The same RMSNorm rows (kind 0, not accurate, width up to
// kReferenceOrderQuantizeMaxWidth) quantized per row as quantize_rows does:
// int8 values into q, the per-row scale into scales (no FP32 output).
constexpr int kReferenceOrderQuantizeMaxWidth = 2048;
bool launch_norm_quantize_reference_order(const float* x, int rows, int width, const NormView& norm, int8_t* q,
                                          float* scales, hipStream_t stream);
// Most visible keys one query of the reference-order attention can score (LDS).
int reference_order_attention_keys();
// attention_impl order; `max_keys` bounds the visible keys of every query
// (the LDS it sizes).  False when max_keys or the head dim is too large.
bool launch_attention_reference_order(const AttentionCall& call, int max_keys, hipStream_t stream);
// activate() with glibc's expf for SiLU (GELU codes use the device's erff / tanhf).
void launch_activation_reference_order(const float* gate_up, int tokens, int width, int gated, int activation,
                                       float* act, hipStream_t stream);
// launch_activation_reference_order's values quantized per row as
// quantize_rows does (int8 values into q, scales per row), in one launch;
// false past 8192 columns.
bool launch_activation_quantize_reference_order(const float* gate_up, int tokens, int width, int gated,
                                                int activation, int8_t* q, float* scales, hipStream_t stream);
// y[i] = expf(x[i]) as glibc computes it.
void launch_libm_expf(const float* x, size_t count, float* y, hipStream_t stream);
// sums[i] = the column-order f32 sum of row i of x [count, n] (norm()'s and
// the softmax denominator's order), by wave_sequential_sum (method 0) or by
// one lane's plain chain (method 1); cycles[i] (may be null) = the clock
// cycles the sum took.  False when n or method is out of range.
constexpr int kSequentialSumMax = 8192;
inline int seq_per_lane_host(int n) { return (n + 255) / 256 * 4; }
bool launch_sequential_sum(const float* x, int n, int count, float* sums, long long* cycles, int method,
                           hipStream_t stream);
// dot_avx / dot_source_bf16_avx order for FP32, BF16, INT8 and INT4 weights with
// FP32 activations, tokens in groups of four; y = result + bias (kStore) or
// y += result + bias (kAccumulate).  False for other storage.
bool launch_linear_fp_reference_order(const WeightView& w, const float* x, int tokens, float* y, int epilogue,
                                      hipStream_t stream);

}  // namespace leafhip
