// CPU oracle for Leaf's decoder hot path.  TEST INFRASTRUCTURE ONLY.
//
// A restatement, in this repository's own code, of the arithmetic of the
// reference CPU decoder on its Linux dispatch (engine/src/decoder.cpp with
// LEAF_OPTIMIZED_FP32 == 0, AVX2+FMA present).  Only tests/, the smoke check
// and bench.py's CPU-baseline leg may load it, and only as the checker: the
// GPU library never calls into it.
//
// Pinning (what makes these functions trustworthy) is recorded per function
// in oracle.cpp.  Integer parts are exact; floating-point parts reproduce the
// reference's operation order, fused multiply-adds included, so they match the
// real reference build bit for bit on the golden vectors.
#pragma once
#include <cstddef>
#include <cstdint>

extern "C" {

// Grouped INT8 W8A8 prefill epilogue: 0 = fused (quant_tile_avx, the default and
// what the GPU computes), 1 = unfused (quant_vnni_tile), -1 = what this CPU's
// reference build would pick.
void oracle_set_vnni_policy(int policy);
// RMSNorm / LayerNorm square sum: 0 = the reference's sequential order (default),
// 1 = pairwise.  Only for measuring the order sensitivity of W8A8 logits.
void oracle_set_norm_order(int order);
// R2: per-token activation quantization, q in [-127,127] stored as int8.
void oracle_quantize_rows(const float* x, size_t M, size_t K, int8_t* q, float* scales);
// R3 integer part: acc[t][row][g] = exact sum_{col in group g} w[row,col] * q[t,col].
void oracle_int_accumulators(unsigned bits, size_t rows, size_t cols, size_t group,
                             const void* data, const int8_t* q, size_t M, int32_t* acc);
// R2-R4: W8A8 / W4A8 linear, y[M,rows] (activation quantization included).
void oracle_linear_int(unsigned bits, size_t rows, size_t cols, size_t group, const void* data,
                       const float* scales, const float* bias, const float* x, size_t M, float* y);
// Same epilogue from precomputed quantized input and scales.
void oracle_linear_int_q(unsigned bits, size_t rows, size_t cols, size_t group, const void* data,
                         const float* scales, const float* bias, const int8_t* q,
                         const float* qscale, size_t M, float* y);
// R5: FP32 / BF16-source / weight-only INT8 / INT4 linear in 4-token groups.
void oracle_linear_fp(unsigned bits, size_t rows, size_t cols, size_t group, const void* data,
                      const float* scales, const float* bias, const float* x, size_t M, float* y);
// R7: accurate-mode FP32/BF16 token-panel GEMM (tokens >= 8).
void oracle_linear_accurate(unsigned bits, size_t rows, size_t cols, const void* data,
                            const float* bias, const float* x, size_t M, float* y);
// R9: RMSNorm (kind 0) / LayerNorm (kind 1); accurate widens the RMS sum.
void oracle_norm(const float* x, size_t M, size_t width, const float* gamma, const float* beta,
                 float epsilon, unsigned kind, int accurate, float* y);
// R8: rotary coefficient tables for positions [position, position+tokens).
void oracle_rope_frequencies(float theta, unsigned rotary_dim, float* freq);
void oracle_rope_tables(const float* freq, unsigned rotary_dim, size_t position, size_t tokens,
                        float* cosines, float* sines);
// R11: masked GQA attention over a strided cache, reference operation order.
void oracle_attention(const float* q_heads, const float* keys, const float* values,
                      const float* mask, float* out, size_t heads, size_t kv_heads,
                      size_t tokens, size_t total, size_t stride, size_t dim, float scale);
// R12: activation function by header code.
float oracle_activate(unsigned activation, float x);
// R12 over rows: gated, act[t,j] = up[t,j] * activate(gate[t,j]) with
// gate_up = [tokens, 2 width] = [gate | up] (decoder.cpp:1414); otherwise
// act = activate(x) over [tokens, width].
void oracle_activation(const float* gate_up, size_t tokens, size_t width, int gated, unsigned activation,
                       float* act);
// The libm expf the reference's softmax and SiLU call (std::exp on float).
void oracle_expf(const float* x, size_t count, float* y);
// R16: weight quantization (export side); packed is int8 [rows,cols] or nibble-packed.
void oracle_quantize_weights(const float* w, size_t rows, size_t cols, unsigned bits, size_t group,
                             uint8_t* packed, float* scales);

// R13-R15: whole decoder over a LEAFDC artifact.
typedef struct oracle_decoder oracle_decoder;
oracle_decoder* oracle_decoder_open(const char* path, unsigned activation_bits, int accurate,
                                    char* error, size_t error_size);
void oracle_decoder_close(oracle_decoder*);
void oracle_decoder_reset(oracle_decoder*);
// logits: vocab floats (or tokens*vocab when all_logits).  Returns 0, or -1 with error text.
int oracle_decoder_forward(oracle_decoder*, const uint32_t* ids, size_t count, int all_logits,
                           float* logits, char* error, size_t error_size);
size_t oracle_decoder_cache_tokens(const oracle_decoder*);
uint32_t oracle_decoder_vocab(const oracle_decoder*);
int oracle_decoder_is_eos(const oracle_decoder*, uint32_t token);
// Greedy loop (main_decoder.cpp:95-113): prefill, then argmax / forward.
int oracle_decoder_generate(oracle_decoder*, const uint32_t* prompt, size_t count, unsigned limit,
                            uint32_t* tokens, size_t* produced, char* error, size_t error_size);
}
