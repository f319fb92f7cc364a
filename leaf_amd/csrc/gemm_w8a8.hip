// W8A8 prefill GEMM on gfx950's int8 matrix cores.
//
//   Y[t, n] = ((float)sum_k Xq[t, k] W[n, k] * s_x[t]) * s_w[n] + b[n]
//
// for per-row weight scales (group = K, the export default; decoder.cpp:571-617
// quant_tile_avx and :661-702 quant_vnni_tile compute the same sums) and
// K % 128 == 0.  The integer sums are exact and the epilogue is the CPU
// path's expression, so every output is bit-identical to it.
//
// Tiling.  A block of WR x WC waves owns 32 WR TM weight rows x 32 WC TN
// tokens; each wave a TM x TN grid of v_mfma_i32_32x32x32_i8 tiles.  The
// weight rows are the MFMA's A operand and the tokens its B operand, so a
// lane of an output tile holds one token and, per group of four results,
// four consecutive weight rows: the epilogue writes 16-byte vectors (with
// the tokens as A it would write single words, and a wave may keep only 63
// memory instructions in flight, which made the output drain, not the
// matrix cores, the limit).  Tiles with fewer than four MFMA tiles per wave
// keep two accumulator sets, alternate k-steps between them and add them at
// the end (exact integer sums), so consecutive MFMAs never depend on each
// other.  K advances 128 bytes per pipeline stage.
//
// Operand staging.  global_load_lds_dwordx4 moves each lane's 16 bytes from
// global memory straight into LDS (no register round trip), NSTAGE - 1
// stages in flight while one is consumed.  One wave instruction fills one
// 1 KiB chunk: 8 rows x 128 K bytes, every row a whole 128-byte line, lane l
// fetching row l / 8, segment (l % 8) ^ (l / 8), written at chunk + 16 l.  So
// segment c of row r sits in slot c ^ (r % 8) of its 128-byte LDS row (XOR
// swizzle).  An MFMA operand (32 rows x 32 K bytes; lane l holds row l % 32,
// segment 2 step + l / 32) then reads eight different slots across any eight
// consecutive rows: no LDS bank conflicts.  A stage is [weight rows | tokens].
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

namespace leafhip {
namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

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

// One output element: the CPU path's epilogue, stored or added to y.
__device__ __forceinline__ float dequant(int acc, float sx, float sw, float b) {
    return fmaf((float)acc * sx, sw, 0.0f) + b;
}

template <int TM, int TN, int NSTAGE, int WR = 2, int WC = 2>
__global__ __launch_bounds__(64 * WR * WC) void gemm_w8a8_mfma_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ w_scales, const float* __restrict__ bias,
    const int8_t* __restrict__ xq, const float* __restrict__ xs, int M, int N, int K, float* __restrict__ y,
    int epilogue, int32_t* __restrict__ acc_out, int splits, int32_t* __restrict__ partial, bool vec) {
    constexpr int kWaves = WR * WC;                           // WR x WC waves (weight rows x tokens)
    constexpr int BN = 32 * WR * TM, BM = 32 * WC * TN;       // weight rows, tokens per block
    constexpr int kChunksW = BN / 8;                          // 8 rows x 128 K bytes per chunk
    constexpr int kChunks = kChunksW + BM / 8;
    constexpr int kLoads = kChunks / kWaves;                  // 16-byte loads per lane per stage
    constexpr int kStageBytes = kChunks * kChunkBytes;
    constexpr int kSets = TM * TN >= 4 ? 1 : 2;               // accumulator sets (alternating k-steps)
    static_assert(kChunks % kWaves == 0, "chunks must divide among the waves");
    static_assert((NSTAGE - 2) * kLoads < 64, "vmcnt holds at most 63");
    __shared__ __align__(1024) int8_t lds[NSTAGE * kStageBytes];

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    // ---- work item
    const int mt = (M + BM - 1) / BM;
    const int nt = (N + BN - 1) / BN;
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
    const int m0 = m_tile * BM, n0 = n_tile * BN;
    const int total_stages = K / kStageK;
    const int s_begin = split * total_stages / splits, s_end = (split + 1) * total_stages / splits;
    const int ns = s_end - s_begin;

    // ---- per-lane sources of this wave's chunk loads (at the split's first K byte)
    const int8_t* src[kLoads];
    int dst[kLoads];
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        const int c = j * kWaves + wave;
        const bool is_w = c < kChunksW;
        const int cc = is_w ? c : c - kChunksW;
        const int row = cc * 8 + (lane >> 3);
        const int koff = ((lane & 7) ^ (lane >> 3)) * 16 + s_begin * kStageK;   // swizzled 16-byte segment
        if (is_w) {
            const int n = n0 + row < N ? n0 + row : N - 1;    // rows past the end are never stored
            src[j] = W + (size_t)n * K + koff;
        } else {
            const int t = m0 + row < M ? m0 + row : M - 1;
            src[j] = xq + (size_t)t * K + koff;
        }
        dst[j] = c * kChunkBytes;
    }

    // ---- accumulators: wave sub-tile rows wn.., tokens wm..
    const int wn = (wave / WC) * 32 * TM, wm = (wave % WC) * 32 * TN;
    v16i acc[kSets][TM][TN];
#pragma unroll
    for (int q = 0; q < kSets; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[q][i][j][r] = 0;

    // Operand read offsets within a stage buffer.  Lane l reads row l % 32 of
    // a 32-row operand (row r of the stage sits at r * 128), 16-byte K
    // segment 2 step + l / 32, stored at slot segment ^ (row % 8).
    const int row_off = (lane & 31) * 128;
    int seg_off[4];
#pragma unroll
    for (int step = 0; step < 4; ++step) seg_off[step] = ((2 * step + (lane >> 5)) ^ (lane & 7)) * 16;
    {
        // Stages past the split's end load the first 16 bytes of the
        // activations (an L1 hit) into a buffer nobody reads again, so every
        // iteration issues exactly one stage.
        auto issue_one = [&](int j, int stage, int buffer) {
            __builtin_amdgcn_global_load_lds((void*)(stage < ns ? src[j] + stage * kStageK : xq),
                                             (lds_ptr_t)(lds + buffer * kStageBytes + dst[j]), 16, 0, 0);
        };
        for (int s = 0; s < NSTAGE - 1; ++s)
#pragma unroll
            for (int j = 0; j < kLoads; ++j) issue_one(j, s, s);
        for (int s = 0; s < ns; ++s) {
            wait_vmcnt<(NSTAGE - 2) * kLoads>();
            block_barrier_lds();
            const int8_t* base = lds + (s % NSTAGE) * kStageBytes;
            const int next = s + NSTAGE - 1, next_buffer = next % NSTAGE;
            // Per k-step: TM weight and TN token operand reads, TM x TN MFMAs,
            // then a quarter of the next stage's loads.
#pragma unroll
            for (int step = 0; step < 4; ++step) {
                v4i fw[TM], fx[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i) fw[i] = *(const v4i*)(base + (wn + 32 * i) * 128 + row_off + seg_off[step]);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    fx[j] = *(const v4i*)(base + kChunksW * kChunkBytes + (wm + 32 * j) * 128 + row_off + seg_off[step]);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[step % kSets][i][j] =
                            __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[i], fx[j], acc[step % kSets][i][j], 0, 0, 0);
#pragma unroll
                for (int j = step * kLoads / 4; j < (step + 1) * kLoads / 4; ++j) issue_one(j, next, next_buffer);
            }
        }
        wait_vmcnt<0>();
    }
    if (kSets == 2) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[0][i][j] += acc[kSets - 1][i][j];
    }

    // ---- epilogue.  Output tile (i, j): lane holds token m0 + wm + 32 j +
    // lane % 32 and, for g = 0..3, rows n0 + wn + 32 i + 8 g + 4 (lane / 32)
    // + 0..3 in acc[.][4 g + 0..3].  `vec`: N % 4 == 0 and every output,
    // scale and bias pointer 16-byte aligned, so four rows move as one vector.
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int t = m0 + wm + 32 * j + (lane & 31);
        if (t >= M) continue;
        const float sx = partial ? 0.0f : xs[t];
        const size_t row_base = (size_t)t * N;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n0 + wn + 32 * i + 8 * g + 4 * (lane >> 5);
                const v4i a = v4i{acc[0][i][j][4 * g], acc[0][i][j][4 * g + 1], acc[0][i][j][4 * g + 2],
                                  acc[0][i][j][4 * g + 3]};
                if (vec && n + 3 < N) {
                    if (partial) {
                        *(v4i*)(partial + (size_t)split * M * N + row_base + n) = a;
                        continue;
                    }
                    if (acc_out) *(v4i*)(acc_out + row_base + n) = a;
                    const v4f sw = *(const v4f*)(w_scales + n);
                    const v4f b = bias ? *(const v4f*)(bias + n) : v4f{0.0f, 0.0f, 0.0f, 0.0f};
                    v4f o;
#pragma unroll
                    for (int q = 0; q < 4; ++q) o[q] = dequant(a[q], sx, sw[q], b[q]);
                    float* out = y + row_base + n;
                    if (epilogue == kAccumulate) {
                        const v4f prev = *(const v4f*)out;
#pragma unroll
                        for (int q = 0; q < 4; ++q) o[q] = prev[q] + o[q];
                    }
                    *(v4f*)out = o;
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (n + q >= N) continue;
                        const size_t o = row_base + n + q;
                        if (partial) {
                            partial[(size_t)split * M * N + o] = a[q];
                            continue;
                        }
                        if (acc_out) acc_out[o] = a[q];
                        const float v = dequant(a[q], sx, w_scales[n + q], bias ? bias[n + q] : 0.0f);
                        y[o] = epilogue == kAccumulate ? y[o] + v : v;
                    }
                }
            }
    }
}

template <int TM, int TN, int NSTAGE, int WR = 2, int WC = 2>
void launch_tiles(const int8_t* W, const float* w_scales, const float* bias, const int8_t* xq, const float* xs,
                  int M, int N, int K, float* y, int epilogue, int32_t* acc_out, int splits, int32_t* partial,
                  hipStream_t stream) {
    auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool vec = N % 4 == 0 && aligned(w_scales) && aligned(bias) && aligned(y) && aligned(acc_out) &&
                     aligned(partial);
    constexpr int BN = 32 * WR * TM, BM = 32 * WC * TN;
    const dim3 grid(((M + BM - 1) / BM) * ((N + BN - 1) / BN) * splits);
    gemm_w8a8_mfma_kernel<TM, TN, NSTAGE, WR, WC><<<grid, 64 * WR * WC, 0, stream>>>(W, w_scales, bias, xq, xs, M, N, K, y, epilogue,
                                                                     acc_out, splits, partial, vec);
}

}  // namespace

bool gemm_w8a8_mfma_supported(int K) { return K % kStageK == 0 && K > 0; }

GemmTiles gemm_w8a8_tiles(int M, int N, int K, size_t split_capacity) {
    // Large outputs (the stacked gate|up projection of a 512-token prefill)
    // take 128 weight rows x 256 tokens per block, eight waves of 64 x 64
    // (two waves per SIMD: one issues MFMAs while the other waits on a
    // barrier or its operands; 25 against 29 us with four waves of 64 x 128
    // for 512 x 11264 x 2048); everything else 64 x 64 with four waves (two
    // blocks fit a CU), which puts the most blocks on the CUs.  A grid still short of 128
    // blocks (few tokens) splits K, each split at least four 128-byte stages,
    // when the workspace holds the int32 sums.
    GemmTiles g;
    auto count = [&](int bn, int bm) { return ((N + bn - 1) / bn) * ((M + bm - 1) / bm); };
    if (M >= 256 && count(128, 256) >= 128) {
        g.rows = 128;
        g.tokens = 256;
    } else {
        g.rows = 64;
        g.tokens = 64;
    }
    const int tiles = count(g.rows, g.tokens);
    const int stages = K / kStageK;
    g.splits = 1;
    while (tiles * g.splits < 128 && stages >= 8 * g.splits &&
           (size_t)(2 * g.splits) * M * N <= split_capacity)
        g.splits *= 2;
    return g;
}

void launch_gemm_w8a8_mfma(const int8_t* W, const float* w_scales, const float* bias, const int8_t* xq,
                           const float* xs, int M, int N, int K, float* y, int epilogue, int32_t* acc_out,
                           const GemmTiles& tiles, int32_t* partial, hipStream_t stream) {
    const int splits = partial ? tiles.splits : 1;
    if (tiles.rows == 128 && tiles.tokens == 256)   // eight waves (two per SIMD), each 64 rows x 64 tokens
        launch_tiles<2, 2, 3, 2, 4>(W, w_scales, bias, xq, xs, M, N, K, y, epilogue, acc_out, splits, partial, stream);
    else
        launch_tiles<1, 1, 4>(W, w_scales, bias, xq, xs, M, N, K, y, epilogue, acc_out, splits, partial, stream);
}

}  // namespace leafhip
