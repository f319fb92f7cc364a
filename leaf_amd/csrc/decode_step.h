// Persistent single-token decode step for W8A8 decoders (gfx950).
//
// One cooperative launch runs a whole decode token: embedding, every layer
// (RMSNorm + q|k|v + RoPE + KV append, GQA attention, o_proj + residual,
// RMSNorm + gate|up + SiLU gate, down_proj + residual), the final norm, the
// LM head and the greedy argmax.  One block per CU; phases hand their outputs
// to each other through epoch-tagged exchange buffers, and every wave issues
// the weight loads of its next phase before computing the current one, so the
// weight stream runs ahead of the dependency chain.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace leafhip {

constexpr int kStepThreads = 512;      // threads per block (8 waves)
constexpr int kStepMaxHidden = 2048;   // hidden widths up to this
constexpr int kStepMaxFfn = 6144;      // intermediate widths up to this
constexpr int kStepDim = 64;           // head dim
constexpr int kStepMaxGroup = 16;      // query heads per KV head
constexpr int kStepSpanKeys = 64;      // keys per attention span
constexpr int kStepMaxSpans = 64;      // spans per KV head
constexpr int kStepMaxLayers = 64;
constexpr int kStepPadWords = 1024;    // slack after each exchange vector for block-wise polls
constexpr int kStepTracePoints = 64 * kStepMaxLayers + 16;   // timeline stamps per block

struct StepLayer {
    WeightView qkv, o, gate_up, down;  // int8, one scale per row, bias vector present
    const float* input_gamma = nullptr;
    const float* post_gamma = nullptr;
};

// Diagnostics: the integer stages of one step, recorded by a separately
// compiled variant of the kernel (null pointers: off).  Per layer, phase p of
// 0 q|k|v, 1 o_proj, 2 gate|up, 3 down_proj: the f32 vector the phase
// quantizes (block 0's copy: the normalized layer input, the attention
// output, the normalized mid vector, the gated activation), its int8 values
// and per-token scale, and the exact int32 dot of every output row.
struct StepCapture {
    float* x = nullptr;        // [layers][4][kStepMaxFfn]
    int8_t* q = nullptr;       // [layers][4][kStepMaxFfn]
    float* sx = nullptr;       // [layers][4]
    int32_t* acc = nullptr;    // [layers][4][2 * kStepMaxFfn] (q|k|v rows, o rows, gate then up rows, down rows)
};

struct StepParams {
    int layers = 0, hidden = 0, ffn = 0, heads = 0, kv_heads = 0, rotary = 0, vocab = 0;
    int window = 0, capacity = 0, activation = 0;
    int item_heads = 1;                 // least query heads per exchange wave in an attention item (1, 2, 4 or 8)
    // Nonzero: every floating-point step in the CPU reference's order and rounding (sequential norm and
    // softmax sums, key-order p.v, glibc expf in the softmax and SiLU, dot_avx order in the FP32 head),
    // so logits equal the reference's bit for bit.  Needs SiLU or ReLU and a hidden width that is a
    // multiple of 32 (decode_step_fits_reference).
    int reference = 0;
    float epsilon = 0, embedding_scale = 1, attention_scale = 1;
    const StepLayer* layer = nullptr;   // device array [layers]
    WeightView embedding;               // int8 per row or f32
    WeightView head;                    // f32 [vocab, hidden] with bias
    const float* final_gamma = nullptr;
    const float* cosines = nullptr;     // [capacity, rotary / 2]
    const float* sines = nullptr;
    float* kv = nullptr;                // [layers][K|V][kv_heads][capacity][dim]
    // exchange buffers: (epoch << 32 | f32 bits) words
    unsigned long long* x_hidden = nullptr;     // layer input (after down_proj)   [hidden]
    unsigned long long* x_mid = nullptr;        // after o_proj                    [hidden]
    unsigned long long* x_qkv = nullptr;        // q|k|v after RoPE                [q + 2 kv]
    unsigned long long* x_attn = nullptr;       // merged attention output        [q]
    unsigned long long* x_act = nullptr;        // SiLU-gated MLP activation       [ffn]
    unsigned long long* x_part = nullptr;       // attention span partials [kv][spans][group][dim + 2]
    // The same partials in plain device memory, for the XCD-local merge (null: off).  Items and
    // merge waves of a head pair then sit on one XCD (block b runs on XCD b % 8), the items write
    // with plain stores that stay in that XCD's L2 and the merge waves read them from there.
    unsigned long long* x_part_local = nullptr;
    int xcd_check_flip = 0;                     // tests: nonzero fails the last block's XCD check (forces the fallback)
    // The q rows of each head slice, in plain device memory, for XCD-local q (null: off): the
    // rows of a slice are computed on its XCD and its items read them from that XCD's L2.
    unsigned long long* x_q_local = nullptr;
    unsigned long long* x_best = nullptr;       // per-block argmax candidates [blocks][2]
    unsigned* counters = nullptr;               // [kv_heads] span arrivals (zero between uses)
    unsigned* abort_flag = nullptr;             // set when a wait times out (device copy, polled by blocks)
    unsigned* host_abort = nullptr;             // mapped host copy of the abort flag (may be null)
    float* logits = nullptr;                    // [vocab]
    uint32_t* token = nullptr;                  // in: this step's id; out: the argmax
    uint32_t* host_token = nullptr;             // mapped host copy of the argmax (may be null)
    unsigned long long* trace = nullptr;        // [blocks][kStepTracePoints] clock stamps, or null
    int position = 0;                           // index of this token in the cache
    unsigned epoch = 0;                         // launch tag (launch number << 12)
    StepCapture capture;                        // diagnostics, off unless set
};

// Whether a decoder of this geometry runs on the persistent step kernel.
bool decode_step_fits(int hidden, int ffn, int heads, int kv_heads, int dim, int vocab, int blocks);
// ... and, in addition, in reference order (StepParams::reference).
bool decode_step_fits_reference(int hidden, int activation);
// Most visible keys a step takes in reference order (longer contexts decode on the graph path).
int decode_step_reference_keys();
// Attention spans for `keys` visible keys.
int decode_step_spans(int keys);
// Blocks the step runs on (one per CU), or 0 when one block per CU cannot be resident.
int decode_step_blocks(int device);
// Launches one decode step (`blocks` = CUs), as a cooperative launch, which
// guarantees every block is resident, or as a plain one of the same grid
// (profilers that fail at process exit after cooperative launches).
// Returns the HIP status.
hipError_t launch_decode_step(const StepParams& params, int blocks, hipStream_t stream, bool cooperative = true);

}  // namespace leafhip
