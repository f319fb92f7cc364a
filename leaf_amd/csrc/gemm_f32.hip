// FP32-math prefill GEMM on f32 MFMA with LDS-staged tiles.
//
//   Y[t, n] = sum_k X[t, k] W[n, k] (+ bias[n], or added to Y)
//
// for weights stored as f32, BF16, or int8 / int4 with group scales
// (decoder.cpp:236-251's storage; a quantized weight enters as
// (float)q * scale, one rounding, as the FP linears of the CPU path
// dequantize it).  Tokens are the MFMA's A operand and weight rows its B
// operand of v_mfma_f32_16x16x4_f32.  Lane l supplies row l % 16 of its
// operand at the four K values 16 g + 4 (l / 16) + j of K-group g, one per
// MFMA j = 0..3, and every accumulator takes the K-groups in ascending
// order: the same products in the same order as gemm_f32_kernel, which
// streams its operands from global memory, so both give identical outputs.
//
// Tiling.  A block of four waves (2 x 2) owns 32 WTM tokens x 32 WTN weight
// rows; each wave a WTM x WTN grid of 16 x 16 accumulators.  K advances 32
// values (128 bytes of f32) per stage, two stages alternate in LDS.
//
// Staging.  Both operands sit in LDS as f32 rows of 128 bytes: 16-byte
// segment c of row r in slot c ^ (r % 8), so the 16 rows one operand read
// touches spread over all banks.  Activations (and f32 weights) move from
// global memory straight into LDS (global_load_lds_dwordx4: one wave
// instruction fills 8 rows x 128 bytes, lane l fetching row l / 8, segment
// (l % 8) ^ (l / 8)).  BF16 / int8 / int4 weights are loaded into registers
// one stage ahead, widened or dequantized, and written to their slots.
#include <cstdlib>
#include <cstring>

#include "device_common.h"
#include "kernels.h"

namespace leafhip {
namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kThreads = 256;
constexpr int kStageK = 32;                      // K values per stage (128 bytes of f32)
constexpr int kRowBytes = kStageK * 4;

// s_waitcnt immediate (gfx9 encoding) for vmcnt <= 0 with lgkmcnt and expcnt free.
constexpr int kVmcnt0 = (7 << 4) | (15 << 8);

template <int BITS, int WTM, int WTN>
__global__ __launch_bounds__(kThreads) void gemm_f32_lds_kernel(WeightView w, const float* __restrict__ x, int tokens,
                                                               float* __restrict__ y, int epilogue) {
    constexpr int BM = 32 * WTM, BN = 32 * WTN;            // tokens, weight rows per block
    constexpr int kStageA = BM * kRowBytes, kStageB = BN * kRowBytes;
    constexpr int kStage = kStageA + kStageB;
    constexpr int kChunksA = BM / 8, kChunksB = BN / 8;    // 1 KiB chunks: 8 rows x 128 bytes
    static_assert(kChunksA % 4 == 0 && kChunksB % 4 == 0, "chunks divide among four waves");
    // Non-f32 weights: each thread widens `kVals` consecutive values of one row.
    constexpr int kThreadsPerRow = kThreads / BN;
    constexpr int kVals = kStageK / kThreadsPerRow;        // 16 (BN 128) or 8 (BN 64)
    constexpr int kRawBytes = kVals * BITS / 8;
    static_assert(BITS == 32 || (kRawBytes % 4 == 0 && kRawBytes <= 32), "raw weight slice of whole words");
    constexpr int kRawWords = BITS == 32 ? 1 : kRawBytes / 4;
    __shared__ __align__(1024) uint8_t lds[2 * kStage];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = w.cols, N = w.rows;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int ns = K / kStageK;

    // ---- direct-to-LDS sources (at stage 0) of this wave's chunks
    const int seg_l = (lane & 7) ^ (lane >> 3);
    const float* a_src[kChunksA / 4];
#pragma unroll
    for (int j = 0; j < kChunksA / 4; ++j) {
        const int row = (j * 4 + wave) * 8 + (lane >> 3);
        const int t = min(m0 + row, tokens - 1);
        a_src[j] = x + (size_t)t * K + seg_l * 4;
    }
    const float* b_src[BITS == 32 ? kChunksB / 4 : 1];
    if constexpr (BITS == 32) {
#pragma unroll
        for (int j = 0; j < kChunksB / 4; ++j) {
            const int row = (j * 4 + wave) * 8 + (lane >> 3);
            const int n = min(n0 + row, N - 1);
            b_src[j] = (const float*)w.data + (size_t)n * K + seg_l * 4;
        }
    }
    // ---- register path of non-f32 weights: row b_row, values b_col .. b_col + kVals
    const int b_row = threadIdx.x / kThreadsPerRow, b_col = (threadIdx.x % kThreadsPerRow) * kVals;
    const int b_n = min(n0 + b_row, N - 1);
    const int groups = (BITS == 8 || BITS == 4) ? K / w.group : 1;
    uint32_t raw[kRawWords];
    float raw_scale = 1.0f;
    auto load_raw = [&](int s) {
        if constexpr (BITS != 32) {
            const int k = s * kStageK + b_col;
            const uint8_t* p = (const uint8_t*)w.data + ((size_t)b_n * K + k) * BITS / 8;
#pragma unroll
            for (int q = 0; q < kRawWords; q += 4) {
                if (q + 4 <= kRawWords) {
                    const uint4 v = *(const uint4*)(p + 4 * q);
                    raw[q] = v.x; raw[q + 1] = v.y; raw[q + 2] = v.z; raw[q + 3] = v.w;
                } else if (q + 2 <= kRawWords) {
                    const uint2 v = *(const uint2*)(p + 4 * q);
                    raw[q] = v.x; raw[q + 1] = v.y;
                } else {
                    raw[q] = *(const uint32_t*)(p + 4 * q);
                }
            }
            if constexpr (BITS == 8 || BITS == 4) raw_scale = w.scales[(size_t)b_n * groups + k / w.group];
        }
    };
    // widened values of the thread's slice, written to their swizzled slots
    auto store_raw = [&](int buffer) {
        if constexpr (BITS != 32) {
            float f[kVals];
#pragma unroll
            for (int e = 0; e < kVals; ++e) {
                if constexpr (BITS == 16) f[e] = bf16_to_f32((raw[e / 2] >> (16 * (e & 1))) & 0xFFFFu);
                else if constexpr (BITS == 8) f[e] = (float)(int)(int8_t)((raw[e / 4] >> (8 * (e & 3))) & 0xFFu) * raw_scale;
                else f[e] = (float)nibble((raw[e / 8] >> (8 * ((e & 7) / 2))) & 0xFFu, e & 1) * raw_scale;
            }
            uint8_t* rowp = lds + buffer * kStage + kStageA + b_row * kRowBytes;
#pragma unroll
            for (int q = 0; q < kVals / 4; ++q) {
                const int seg = b_col / 4 + q;
                *(v4f*)(rowp + ((seg ^ (b_row & 7)) * 16)) = v4f{f[4 * q], f[4 * q + 1], f[4 * q + 2], f[4 * q + 3]};
            }
        }
    };
    auto issue_dma = [&](int s, int buffer) {
        uint8_t* base = lds + buffer * kStage;
#pragma unroll
        for (int j = 0; j < kChunksA / 4; ++j)
            __builtin_amdgcn_global_load_lds((void*)(a_src[j] + s * kStageK),
                                             (lds_ptr_t)(base + (j * 4 + wave) * 1024 + lane * 16), 16, 0, 0);
        if constexpr (BITS == 32) {
#pragma unroll
            for (int j = 0; j < kChunksB / 4; ++j)
                __builtin_amdgcn_global_load_lds((void*)(b_src[j] + s * kStageK),
                                                 (lds_ptr_t)(base + kStageA + (j * 4 + wave) * 1024 + lane * 16), 16,
                                                 0, 0);
        }
    };

    v4f acc[WTM][WTN];
#pragma unroll
    for (int i = 0; i < WTM; ++i)
#pragma unroll
        for (int n = 0; n < WTN; ++n) acc[i][n] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    const int wm = (wave >> 1) * 16 * WTM, wn = (wave & 1) * 16 * WTN;
    const int li = lane & 15, kk = lane >> 4;

    issue_dma(0, 0);
    load_raw(0);
    store_raw(0);
    __builtin_amdgcn_s_waitcnt(kVmcnt0);
    __syncthreads();
    for (int s = 0; s < ns; ++s) {
        const int buffer = s & 1;
        const bool more = s + 1 < ns;
        if (more) {
            issue_dma(s + 1, buffer ^ 1);
            load_raw(s + 1);
        }
        const uint8_t* base = lds + buffer * kStage;
#pragma unroll
        for (int g = 0; g < kStageK / 16; ++g) {
            const int seg = 4 * g + kk;
            v4f a[WTM], b[WTN];
#pragma unroll
            for (int i = 0; i < WTM; ++i) {
                const int row = wm + 16 * i + li;
                a[i] = *(const v4f*)(base + row * kRowBytes + ((seg ^ (row & 7)) * 16));
            }
#pragma unroll
            for (int n = 0; n < WTN; ++n) {
                const int row = wn + 16 * n + li;
                b[n] = *(const v4f*)(base + kStageA + row * kRowBytes + ((seg ^ (row & 7)) * 16));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < WTM; ++i)
#pragma unroll
                    for (int n = 0; n < WTN; ++n)
                        acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][j], b[n][j], acc[i][n], 0, 0, 0);
        }
        if (more) store_raw(buffer ^ 1);
        __builtin_amdgcn_s_waitcnt(kVmcnt0);
        __syncthreads();
    }

    // ---- epilogue: lane holds tokens wm + 16 i + 4 kk + r of weight row wn + 16 n + li
#pragma unroll
    for (int n = 0; n < WTN; ++n) {
        const int row = n0 + wn + 16 * n + li;
        if (row >= N) continue;
        const float bias = w.bias ? w.bias[row] : 0.0f;
#pragma unroll
        for (int i = 0; i < WTM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = m0 + wm + 16 * i + 4 * kk + r;
                if (t >= tokens) continue;
                float* out = y + (size_t)t * N + row;
                const float v = acc[i][n][r] + bias;
                *out = epilogue == kAccumulate ? *out + v : v;
            }
    }
}

template <int BITS, int WTM, int WTN>
void launch_tiles(const WeightView& w, const float* x, int tokens, float* y, int epilogue, hipStream_t stream) {
    const dim3 grid((w.rows + 32 * WTN - 1) / (32 * WTN), (tokens + 32 * WTM - 1) / (32 * WTM));
    gemm_f32_lds_kernel<BITS, WTM, WTN><<<grid, kThreads, 0, stream>>>(w, x, tokens, y, epilogue);
}

// LEAF_F32_GEMM_TILE=128x64|64x128|128x128|64x64 (tokens x rows) forces a
// tile (tests compare them); any other value, or none, lets the cost decide.
int forced_tile() {
    const char* v = getenv("LEAF_F32_GEMM_TILE");
    if (!v) return -1;
    const char* names[4] = {"128x64", "64x128", "128x128", "64x64"};
    for (int i = 0; i < 4; ++i)
        if (strcmp(v, names[i]) == 0) return i;
    return -1;
}

template <int BITS>
void launch_bits(const WeightView& w, const float* x, int tokens, float* y, int epilogue, hipStream_t stream) {
    // Tile by the work of the busiest CU: ceil(blocks / 256 CUs) tiles of
    // bm x bn, 64 x 64 tiles charged 10% for their lower MFMA density; ties
    // go to the earlier tile.  (Measured at the Qwen / SmolLM2 prefill shapes:
    // within 15% of the best of the four tiles, and 128 x 128 alone lost up
    // to 1.8x where its grid covered the CUs 1.1 or 2.5 times.)
    const int tiles[4][2] = {{128, 64}, {64, 128}, {128, 128}, {64, 64}};
    int best = 0;
    double best_cost = 0.0;
    for (int i = 0; i < 4; ++i) {
        const int bm = tiles[i][0], bn = tiles[i][1];
        const long blocks = (long)((tokens + bm - 1) / bm) * ((w.rows + bn - 1) / bn);
        const double cost = (double)((blocks + 255) / 256) * bm * bn * (i == 3 ? 1.1 : 1.0);
        if (i == 0 || cost < best_cost) {
            best = i;
            best_cost = cost;
        }
    }
    const int forced = forced_tile();
    if (forced >= 0) best = forced;
    switch (best) {
    case 0: launch_tiles<BITS, 4, 2>(w, x, tokens, y, epilogue, stream); break;
    case 1: launch_tiles<BITS, 2, 4>(w, x, tokens, y, epilogue, stream); break;
    case 2: launch_tiles<BITS, 4, 4>(w, x, tokens, y, epilogue, stream); break;
    default: launch_tiles<BITS, 2, 2>(w, x, tokens, y, epilogue, stream); break;
    }
}

}  // namespace

bool gemm_f32_lds_supported(const WeightView& w, const float* x) {
    auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (w.cols % kStageK != 0 || w.cols <= 0 || !aligned(x) || !aligned(w.data)) return false;
    // a thread's slice (8 or 16 values) of a quantized row shares one scale
    if ((w.bits == 8 || w.bits == 4) && (w.group <= 0 || w.group % 16 != 0 || w.cols % w.group != 0)) return false;
    return w.bits == 32 || w.bits == 16 || w.bits == 8 || w.bits == 4;
}

void launch_gemm_f32_lds(const WeightView& w, const float* x, int tokens, float* y, int epilogue,
                         hipStream_t stream) {
    switch (w.bits) {
    case 32: launch_bits<32>(w, x, tokens, y, epilogue, stream); break;
    case 16: launch_bits<16>(w, x, tokens, y, epilogue, stream); break;
    case 8: launch_bits<8>(w, x, tokens, y, epilogue, stream); break;
    default: launch_bits<4>(w, x, tokens, y, epilogue, stream); break;
    }
}

}  // namespace leafhip
