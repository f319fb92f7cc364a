// W8A8 prefill GEMM on gfx950's int8 matrix cores.
//
//   Y[t, n] = ((float)sum_k Xq[t, k] W[n, k] * s_x[t]) * s_w[n] + b[n]
//
// for per-row weight scales (group = K, the export default; decoder.cpp:571-617
// quant_tile_avx and :661-702 quant_vnni_tile compute the same sums) and
// K % 128 == 0.  The integer sums are exact and the epilogue is the CPU
// path's expression, so every output is bit-identical to it.
//
// Tiling.  A block owns BM tokens x 128 weight rows; each of its waves owns a
// 64 x 64 sub-tile as 2 x 2 v_mfma_i32_32x32x32_i8 accumulators (4
// independent chains per wave keep the matrix pipe issuing back to back).
// K advances 128 bytes per pipeline stage.
//
// Operand staging.  global_load_lds_dwordx4 moves each lane's 16 bytes from
// global memory straight into LDS (no register round trip), NSTAGE - 1
// stages in flight while one is consumed.  One wave instruction fills one
// 1 KiB chunk: 8 rows x 128 K bytes, every row a whole 128-byte line, lane l
// fetching row l / 8, segment (l % 8) ^ (l / 8), written at chunk + 16 l.  So
// segment c of row r sits in slot c ^ (r % 8) of its 128-byte LDS row (XOR
// swizzle).  An MFMA operand (32 rows x 32 K bytes; lane l holds row l % 32,
// segment 2 step + l / 32) then reads eight different slots across any eight
// consecutive rows: no LDS bank conflicts.  A stage is [A rows | B rows].
//
// Issue order.  Per stage a wave issues 16 MFMAs, 16 operand reads and its
// share of the next stage's loads; sched_barrier fences pin an order in which
// consecutive MFMAs use different accumulators and the loads and later reads
// sit between MFMA pairs, so the matrix pipe does not wait for issue bursts.
//
// Waiting.  Loads retire in order per wave, and every iteration issues one
// stage, so "stage s landed" is vmcnt <= (NSTAGE - 2) stages of loads; each
// wave waits for its own share, then a barrier publishes every wave's share.
// The buffer refilled after that barrier was consumed in the previous
// iteration by every wave.
//
// Work mapping.  Items are (token tile, weight tile, K split).  The token
// tiles of one (weight tile, split) pair share that pair's weight rows, so
// they are dealt to blocks b with the same b % 8 (blocks are dispatched to
// the eight XCDs round robin): the second and later reads of those rows hit
// the XCD's L2.  Placement only affects speed, never results.
//
// Split K.  With `partial` set, a block stores its exact int32 sums to
// partial[split][t][n]; gemm_w8a8_split_epilogue adds them in split order.
#include "device_common.h"
#include "kernels.h"

#include <type_traits>

namespace leafhip {
namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kTileN = 128;     // weight rows per block
constexpr int kStageK = 128;    // K bytes per pipeline stage
constexpr int kChunkBytes = 1024;

// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt <= n and leaves
// lgkmcnt and expcnt unconstrained.
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(N));
}

// Compiler and hardware barrier for the waves of a block: LDS operations
// complete, then s_barrier; global loads in flight stay in flight.
__device__ __forceinline__ void block_barrier_lds() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((0) << 8 | (7 << 4) | 15 | (3 << 14));   // lgkmcnt(0), vmcnt/expcnt free
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int BM, int NSTAGE>
__global__ __launch_bounds__(BM / 64 * 2 * 64) void gemm_w8a8_mfma_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ w_scales, const float* __restrict__ bias,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, int M, int N, int K, float* __restrict__ y,
    int epilogue, int32_t* __restrict__ acc_out, int splits, int32_t* __restrict__ partial) {
    constexpr int kWaves = BM / 64 * 2;
    constexpr int kChunksA = BM / 8;                        // 8 rows x 128 K bytes per chunk
    constexpr int kChunks = kChunksA + kTileN / 8;
    constexpr int kLoads = kChunks / kWaves;                 // 16-byte loads per lane per stage
    constexpr int kStageBytes = kChunks * kChunkBytes;
    static_assert(kChunks % kWaves == 0, "chunks must divide among the waves");
    __shared__ __align__(1024) int8_t lds[NSTAGE * kStageBytes];

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    // ---- work item
    const int mt = (M + BM - 1) / BM;
    const int nt = (N + kTileN - 1) / kTileN;
    const int units = nt * splits;
    int m_tile, unit;
    {
        const int b = blockIdx.x;
        if (units % 8 == 0) {
            const int x = b & 7, i = b >> 3;
            m_tile = i % mt;
            unit = (i / mt) * 8 + x;
        } else {
            m_tile = b % mt;
            unit = b / mt;
        }
    }
    const int n_tile = unit / splits, split = unit % splits;
    const int m0 = m_tile * BM, n0 = n_tile * kTileN;
    const int total_stages = K / kStageK;
    const int s_begin = split * total_stages / splits, s_end = (split + 1) * total_stages / splits;
    const int ns = s_end - s_begin;

    // ---- per-lane sources of this wave's chunk loads (at the split's first K byte)
    const int8_t* src[kLoads];
    int dst[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int c = j * kWaves + wave;
        const bool is_a = c < kChunksA;
        const int cc = is_a ? c : c - kChunksA;
        const int row = cc * 8 + (lane >> 3);
        const int koff = ((lane & 7) ^ (lane >> 3)) * 16 + s_begin * kStageK;   // swizzled 16-byte segment
        if (is_a) {
            const int t = m0 + row < M ? m0 + row : M - 1;   // rows past the end are never stored
            src[j] = xq + (size_t)t * K + koff;
        } else {
            const int n = n0 + row < N ? n0 + row : N - 1;
            src[j] = W + (size_t)n * K + koff;
        }
        dst[j] = c * kChunkBytes;
    }

    // ---- accumulators: wave sub-tile rows wm.., cols wn..
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    // Operand read offsets within a stage buffer.  Lane l reads row l % 32 of
    // a 32-row operand, 16-byte K segment 2 step + l / 32, stored at slot
    // segment ^ (row % 8) of its 128-byte LDS row.
    const int row_off = ((lane & 31) >> 3) * kChunkBytes + (lane & 7) * 128;
    int seg_off[4];
#pragma unroll
    for (int step = 0; step < 4; ++step) seg_off[step] = ((2 * step + (lane >> 5)) ^ (lane & 7)) * 16;
    int a_off[2], b_off[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        a_off[i] = (wm + 32 * i) * 128 + row_off;
        b_off[i] = kChunksA * kChunkBytes + (wn + 32 * i) * 128 + row_off;
    }
    {
        // Stages past the split's end load the first 16 bytes of the
        // activations (an L1 hit) into a buffer nobody reads again, so every
        // iteration issues exactly one stage.
        auto issue = [&](int stage, int buffer) {
            const bool real = stage < ns;
#pragma unroll
            for (int j = 0; j < kLoads; ++j)
                __builtin_amdgcn_global_load_lds((void*)(real ? src[j] + stage * kStageK : xq),
                                                 (lds_ptr_t)(lds + buffer * kStageBytes + dst[j]), 16, 0, 0);
        };
        auto issue_one = [&](int j, int stage, int buffer) {
            __builtin_amdgcn_global_load_lds((void*)(stage < ns ? src[j] + stage * kStageK : xq),
                                             (lds_ptr_t)(lds + buffer * kStageBytes + dst[j]), 16, 0, 0);
        };
        for (int s = 0; s < NSTAGE - 1; ++s) issue(s, s);
        for (int s = 0; s < ns; ++s) {
            wait_vmcnt<(NSTAGE - 2) * kLoads>();
            block_barrier_lds();
            const int8_t* base = lds + (s % NSTAGE) * kStageBytes;
            const int next = s + NSTAGE - 1, next_buffer = next % NSTAGE;
            v4i fa[4][2], fb[4][2];
            auto read = [&](int step, int i) {
                const int koff = seg_off[step];
                fa[step][i] = *(const v4i*)(base + a_off[i] + koff);
                fb[step][i] = *(const v4i*)(base + b_off[i] + koff);
            };
            // The first two k-steps' operands, then eight MFMA pairs, each
            // followed by a share of the next stage's loads and (first four)
            // the last two k-steps' operands.
#pragma unroll
            for (int step = 0; step < 2; ++step)
#pragma unroll
                for (int i = 0; i < 2; ++i) read(step, i);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                const int step = g >> 1, i = g & 1;
                acc[i][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[step][i], fb[step][0], acc[i][0], 0, 0, 0);
                acc[i][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[step][i], fb[step][1], acc[i][1], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = g * kLoads / 8; j < (g + 1) * kLoads / 8; ++j) issue_one(j, next, next_buffer);
                if (g < 4) read(2 + (g >> 1), g & 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        wait_vmcnt<0>();
    }

    // ---- epilogue: lane holds column n = .. + lane % 32 and rows 8 (r/4) + 4 (lane/32) + r % 4.
    if (m0 + BM <= M && n0 + kTileN <= N) {
        // whole tile in range: straight-line stores, every operand load issued first
        const int tb = m0 + wm + 4 * (lane >> 5);
        const int nb = n0 + wn + (lane & 31);
        if (partial) {
            int32_t* out = partial + (size_t)split * M * N + nb;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    int32_t* row = out + (size_t)(tb + 32 * i + 8 * (r >> 2) + (r & 3)) * N;
                    row[0] = acc[i][0][r];
                    row[32] = acc[i][1][r];
                }
            return;
        }
        const float sw0 = w_scales[nb], sw1 = w_scales[nb + 32];
        const float b0 = bias ? bias[nb] : 0.0f, b1 = bias ? bias[nb + 32] : 0.0f;
        float* yb = y + nb;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float sx[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) sx[r] = xs[tb + 32 * i + 8 * (r >> 2) + (r & 3)];
            if (acc_out) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    int32_t* row = acc_out + (size_t)(tb + 32 * i + 8 * (r >> 2) + (r & 3)) * N + nb;
                    row[0] = acc[i][0][r];
                    row[32] = acc[i][1][r];
                }
            }
            if (epilogue == kAccumulate) {
                float prev[16][2];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float* row = yb + (size_t)(tb + 32 * i + 8 * (r >> 2) + (r & 3)) * N;
                    prev[r][0] = row[0];
                    prev[r][1] = row[32];
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float* row = yb + (size_t)(tb + 32 * i + 8 * (r >> 2) + (r & 3)) * N;
                    row[0] = prev[r][0] + (fmaf((float)acc[i][0][r] * sx[r], sw0, 0.0f) + b0);
                    row[32] = prev[r][1] + (fmaf((float)acc[i][1][r] * sx[r], sw1, 0.0f) + b1);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float* row = yb + (size_t)(tb + 32 * i + 8 * (r >> 2) + (r & 3)) * N;
                    row[0] = fmaf((float)acc[i][0][r] * sx[r], sw0, 0.0f) + b0;
                    row[32] = fmaf((float)acc[i][1][r] * sx[r], sw1, 0.0f) + b1;
                }
            }
        }
        return;
    }
    // edge tile: per-element bounds
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn + 32 * j + (lane & 31);
        if (n >= N) continue;
        const float sw = partial ? 0.0f : w_scales[n];
        const float b = (partial || !bias) ? 0.0f : bias[n];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (t >= M) continue;
                const int a = acc[i][j][r];
                const size_t o = (size_t)t * N + n;
                if (partial) {
                    partial[(size_t)split * M * N + o] = a;
                } else {
                    if (acc_out) acc_out[o] = a;
                    const float v = fmaf((float)a * xs[t], sw, 0.0f) + b;
                    y[o] = epilogue == kAccumulate ? y[o] + v : v;
                }
            }
    }
}

}  // namespace

bool gemm_w8a8_mfma_supported(int K) { return K % kStageK == 0 && K > 0; }

void launch_gemm_w8a8_mfma(const int8_t* W, const float* w_scales, const float* bias, const int8_t* xq,
                           const float* xs, int M, int N, int K, float* y, int epilogue, int32_t* acc_out,
                           int tile_m, int splits, int32_t* partial, hipStream_t stream) {
    const int nt = (N + kTileN - 1) / kTileN;
    if (tile_m == 64) {
        const dim3 grid(((M + 63) / 64) * nt * splits);
        gemm_w8a8_mfma_kernel<64, 6><<<grid, 128, 0, stream>>>(W, w_scales, bias, xq, xs, M, N, K, y, epilogue,
                                                                acc_out, splits, partial);
    } else {
        const dim3 grid(((M + 127) / 128) * nt * splits);
        gemm_w8a8_mfma_kernel<128, 4><<<grid, 256, 0, stream>>>(W, w_scales, bias, xq, xs, M, N, K, y, epilogue,
                                                                 acc_out, splits, partial);
    }
}

}  // namespace leafhip
