// Reference-order kernels (gfx950): floating-point work in the order and
// rounding of Leaf's CPU path, so that a decoder's logits equal the CPU's bit
// for bit.
//
// The fast kernels reduce in parallel orders (per-lane partials, DPP trees,
// span partials merged by log-sum-exp).  That moves W8A8 logits by a few
// percent, because a one-ulp change upstream of a quantization can move an
// int8 bin.  These kernels instead follow the reference's sequential sums:
//   * norm() (engine/src/decoder.cpp:706-727): one lane sums the row's
//     squares (or values, for LayerNorm's mean) in column order;
//     accurate_rms_square_sum (accurate_fp32.h:6-13) sums the float squares
//     in double, in column order.
//   * attention_impl (engine/src/kernels/transformer.cpp:94-146): per query,
//     scores (q.k * scale) * scale with the scalar dot of the Linux build
//     (:69-73), the maximum, exp(s - max) with glibc's expf (libm_expf.h), a
//     sequential denominator, p = e / denominator, then output[d] += p * v[d]
//     in key order, one lane per d.
//   * activate (decoder.cpp:982-987): SiLU g / (1 + expf(-g)) with glibc's
//     expf and ReLU as std::max(x, 0.0f).  GELU uses the device's erff /
//     tanhf, which are not glibc's: GELU decoders are not bit-exact here.
//   * dot_avx / dot_source_bf16_avx (decoder.cpp:355-420): FP32, BF16-source
//     and weight-only INT8 / INT4 rows.  One token: four 8-lane FMA chains over
//     32-column blocks, (a + b) + (c + d), 8-column blocks, the 8-lane
//     horizontal sum ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)), a scalar fused
//     tail of (value / scale) * x, then result += partial * scale per group
//     (fused).  Two to four tokens: one 8-lane chain per token.  The linear
//     runs tokens in groups of four (decoder.cpp:1217-1228).
// The W8A8 integer path needs none of this: its quantization, int32 sums and
// epilogue already match the CPU exactly in the fast kernels.
//
// All files are compiled with -ffp-contract=off, so every product and sum
// below rounds separately unless it is spelled fmaf().
#include "device_common.h"
#include "kernels.h"
#include "libm_expf.h"
#include "sequential_sum.h"

#include <math.h>

#include <algorithm>

namespace leafhip {
namespace {

constexpr int kRoBlock = 256;

// ------------------------------------------------------------------ norm ---
// One block per row.  The row is staged in LDS, every thread forms its
// columns' squares (the same rounded products the CPU forms), and thread 0
// adds them in column order.
__global__ __launch_bounds__(kRoBlock) void ro_norm_kernel(const float* x, int width, NormView norm, float* y,
                                                           int rows_per_group, size_t group_stride) {
    extern __shared__ float row[];        // [width] values, then [width] squares
    float* sq = row + width;
    __shared__ float stat[2];
    const size_t at = rows_per_group > 0 ? (size_t)(blockIdx.x / rows_per_group) * group_stride +
                                               (size_t)(blockIdx.x % rows_per_group) * width
                                         : (size_t)blockIdx.x * width;
    const float* in = x + at;
    float* out = y + at;
    for (int c = threadIdx.x; c < width; c += blockDim.x) row[c] = in[c];
    __syncthreads();
    float mean = 0.0f;
    if (norm.kind == 1) {
        if (threadIdx.x == 0) stat[0] = sequential_sum(row, width) / (float)width;
        __syncthreads();
        mean = stat[0];
    }
    const bool accurate = norm.kind == 0 && norm.accurate;
    for (int c = threadIdx.x; c < width; c += blockDim.x) {
        const float v = accurate ? row[c] : row[c] - mean;
        sq[c] = v * v;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const float square = accurate ? (float)sequential_sum_f64(sq, width) : sequential_sum(sq, width);
        stat[1] = 1.0f / sqrtf(square / (float)width + norm.epsilon);
    }
    __syncthreads();
    const float scale = stat[1];
    for (int c = threadIdx.x; c < width; c += blockDim.x)
        out[c] = (row[c] - mean) * scale * norm.gamma[c] + (norm.beta ? norm.beta[c] : 0.0f);
}

// RMSNorm (mean 0, the non-accurate policy) with the column-order square sum
// formed by the block's two waves in parallel (wave_pair_sequential_sum:
// the chain's bits in a fraction of its time; the squares are never
// negative), one block per row.  Rows up to kSeqSumMaxPerLane * 64 wide.
// With q set, the normalized row is quantized as quantize_rows_kernel does
// (its maximum, exact in any order; the scale and int8 values into q and
// scales) instead of stored.
__global__ __launch_bounds__(2 * kWave) void ro_rms_norm_kernel(const float* x, int width, NormView norm, float* y,
                                                               int rows_per_group, size_t group_stride,
                                                               int8_t* q = nullptr, float* scales = nullptr) {
    // thread t owns columns t + 128 k; every load of the row and its gamma is
    // issued before the first use
    constexpr int kThreads = 2 * kWave, kPer = kSeqSumMaxPerLane * kWave / kThreads;
    extern __shared__ float lds[];
    float4* area0 = reinterpret_cast<float4*>(lds);
    float4* area1 = area0 + kSeqSumArea;
    float4* xchg = area1 + kSeqSumArea;
    float4* comp = xchg + kSeqPairXchg;
    float* v = reinterpret_cast<float*>(comp + 2 * kSeqPairComp);   // the squares, in SeqLayout
    const SeqLayout lay(width);
    const size_t at = rows_per_group > 0 ? (size_t)(blockIdx.x / rows_per_group) * group_stride +
                                               (size_t)(blockIdx.x % rows_per_group) * width
                                         : (size_t)blockIdx.x * width;
    const float* in = x + at;
    float value[kPer], gamma[kPer], beta[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = threadIdx.x + k * kThreads;
        value[k] = c < width ? in[c] : 0.0f;
        gamma[k] = c < width ? norm.gamma[c] : 0.0f;
        beta[k] = c < width && norm.beta ? norm.beta[c] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = threadIdx.x + k * kThreads;
        const float d = value[k] - 0.0f;
        if (c < width) v[lay.at(c)] = d * d;
    }
    seq_zero_tail(v, width, threadIdx.x, blockDim.x);
    __syncthreads();
    const int w = threadIdx.x / kWave;
    float square;
    wave_pair_sequential_sum(v, width, area0, area1, xchg, comp + w * kSeqPairComp, w,
                             [] { __syncthreads(); return true; }, square);
    const float scale = 1.0f / sqrtf(square / (float)width + norm.epsilon);
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        value[k] = (value[k] - 0.0f) * scale * gamma[k] + beta[k];
        m = fmaxf(m, fabsf(value[k]));   // columns past the row hold 0
    }
    if (!q) {
        float* out = y + at;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int c = threadIdx.x + k * kThreads;
            if (c < width) out[c] = value[k];
        }
        return;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    __shared__ float wave_max[2];
    if ((threadIdx.x & (kWave - 1)) == 0) wave_max[w] = m;
    __syncthreads();
    const float sx = fmaxf(fmaxf(wave_max[0], wave_max[1]) / 127.0f, 1e-12f);
    const float multiplier = 1.0f / sx;
    if (threadIdx.x == 0) scales[blockIdx.x] = sx;
    int8_t* qr = q + (size_t)blockIdx.x * width;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = threadIdx.x + k * kThreads;
        if (c < width) qr[c] = (int8_t)quantize_one(value[k], multiplier);
    }
}

// ------------------------------------------------------------- attention ---
// One block per (query head, query token).  LDS holds q and the scores of the
// visible keys; thread 0 sums the denominator; thread d < dim accumulates
// output element d over the keys in order.
__global__ __launch_bounds__(kRoBlock) void ro_attention_kernel(AttentionCall p) {
    extern __shared__ float lds[];
    float* qs = lds;                       // [dim]
    float* sc = lds + p.dim;               // [visible keys]
    __shared__ float red[kRoBlock / kWave];
    __shared__ float den_shared;
    const int h = blockIdx.x, t = blockIdx.y;
    const int position = p.position_ptr ? *p.position_ptr : p.position;
    const int end = position + t + 1;
    const int begin = (p.window && end > p.window) ? end - p.window : 0;
    const int n = end - begin;
    const int dim = p.dim;
    const int kvh = h / (p.heads / p.kv_heads);
    const float* q = p.q_heads + ((size_t)h * p.tokens + t) * dim;
    const float* K = p.keys + (size_t)kvh * p.capacity * dim;
    const float* V = p.values + (size_t)kvh * p.capacity * dim;
    float* o = p.out + ((size_t)t * p.heads + h) * dim;
    for (int d = threadIdx.x; d < dim; d += blockDim.x) qs[d] = q[d];
    __syncthreads();
    // scores and their maximum (NaN scores never become the maximum, as with
    // std::max(maximum, score))
    float m = -INFINITY;
    for (int k = threadIdx.x; k < n; k += blockDim.x) {
        const float* kr = K + (size_t)(begin + k) * dim;
        float s = 0.0f;
        for (int d = 0; d < dim; ++d) s += qs[d] * kr[d];
        s = s * p.scale * p.scale;
        sc[k] = s;
        m = m < s ? s : m;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float other = __shfl_xor(m, off, kWave);
        m = m < other ? other : m;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float maximum = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) maximum = maximum < red[w] ? red[w] : maximum;
    if (!isfinite(maximum)) {
        // fully masked (or infinite) row: the CPU leaves the zero-filled output
        for (int d = threadIdx.x; d < dim; d += blockDim.x) o[d] = 0.0f;
        return;
    }
    for (int k = threadIdx.x; k < n; k += blockDim.x) sc[k] = libm_expf(sc[k] - maximum);
    __syncthreads();
    // masked keys add exp(-inf) = 0, which leaves the sum unchanged
    if (threadIdx.x == 0) den_shared = sequential_sum(sc, n);
    __syncthreads();
    const float den = den_shared;
    for (int k = threadIdx.x; k < n; k += blockDim.x) sc[k] = sc[k] / den;
    __syncthreads();
    // output[d] += p * v[d] in key order; masked keys add p * v = +-0, which
    // leaves a sum that started at +0 unchanged
    for (int d = threadIdx.x; d < dim; d += blockDim.x) {
        float acc = 0.0f;
        const float* vr = V + (size_t)begin * dim + d;
        int k = 0;
        for (; k + 4 <= n; k += 4) {
            const float v0 = vr[(size_t)(k + 0) * dim], v1 = vr[(size_t)(k + 1) * dim];
            const float v2 = vr[(size_t)(k + 2) * dim], v3 = vr[(size_t)(k + 3) * dim];
            acc += sc[k + 0] * v0;
            acc += sc[k + 1] * v1;
            acc += sc[k + 2] * v2;
            acc += sc[k + 3] * v3;
        }
        for (; k < n; ++k) acc += sc[k] * vr[(size_t)k * dim];
        o[d] = acc;
    }
}

// The same arithmetic for head dim 64, one block per (query token, KV head)
// with one wave per HPW query heads of the group: the lanes are the keys for
// the scores (q in scalar registers; the group's K rows of 64 keys staged in
// LDS once by coalesced loads, then each lane's row read back) and the output
// elements for p.v, so no lane idles through a dependent sum and many rows
// share each SIMD.  A wave's HPW heads run their dependent sums side by side
// (independent chains interleaved; one K row read and one V load serve all
// of them).  The denominator is the plain in-order chain, every lane forming
// it alike.  Blocks run from the last token down: the longest rows start
// first.
constexpr int kRoWaveDim = 64;
constexpr int kRoWaveKeys = 12;    // keys per chunk of the p.v chain (three float4 of p)
constexpr int kRoWaveDepth = 2;    // chunks of V in flight
constexpr int kRoKPitch = kRoWaveDim + 4;   // floats per staged K row: lanes' 16-byte reads meet distinct banks
constexpr int kRoMaxGroup = 16;    // query heads per KV head
// Floats of a row's scores: its keys rounded up to whole groups of chunks,
// plus the chunk the chain reads ahead.
__host__ __device__ constexpr int ro_wave_row_floats(int keys) {
    return (keys + kRoWaveKeys * kRoWaveDepth - 1) / (kRoWaveKeys * kRoWaveDepth) * (kRoWaveKeys * kRoWaveDepth) +
           kRoWaveKeys * kRoWaveDepth + kRoWaveKeys;
}
// PER: 16-byte K loads per thread per 64 keys (64 * 16 / blockDim.x, rounded up
// to a power of two); the next keys' loads are in flight while these are scored.
// HPW: query heads per wave (it divides the group); head i of wave w is w + i * (group / HPW).
template <int PER, int HPW>
__global__ __launch_bounds__(kRoMaxGroup / HPW * kWave) void ro_attention_wave_kernel(AttentionCall p, int row_floats) {
    extern __shared__ float lds[];
    constexpr int dim = kRoWaveDim;
    constexpr int kRowBytes = dim * (int)sizeof(float);
    const int group = p.heads / p.kv_heads, waves = group / HPW;
    const int lane = threadIdx.x & (kWave - 1), w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = p.tokens - 1 - (int)blockIdx.x / p.kv_heads, kvh = (int)blockIdx.x % p.kv_heads;
    const int position = p.position_ptr ? *p.position_ptr : p.position;
    const int end = position + t + 1;
    const int begin = (p.window && end > p.window) ? end - p.window : 0;
    const int n = end - begin;
    float* kt = lds;                                       // [kWave][kRoKPitch]: 64 keys' rows
    float* sc[HPW];                                        // each head's scores, then exp, then p
    // expf's table after the group's rows (stored here, read after the first barrier below)
    uint64_t* exp2 = reinterpret_cast<uint64_t*>(lds + kWave * kRoKPitch + group * row_floats);
    if (threadIdx.x < 32) exp2[threadIdx.x] = kExp2Table32[threadIdx.x];
    float qs[HPW][dim];
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
        const int gh = w + i * waves, h = kvh * group + gh;
        sc[i] = lds + kWave * kRoKPitch + gh * row_floats;
        const float* q = p.q_heads + ((size_t)h * p.tokens + t) * dim;
#pragma unroll
        for (int d = 0; d < dim; ++d) qs[i][d] = q[d];
    }
    float* K = const_cast<float*>(p.keys) + ((size_t)kvh * p.capacity + begin) * dim;
    float* V = const_cast<float*>(p.values) + ((size_t)kvh * p.capacity + begin) * dim;
    // bounds-checked views of the n visible rows: rows past them read as 0
    const __amdgpu_buffer_rsrc_t kbuf = __builtin_amdgcn_make_buffer_rsrc(K, (short)0, n * kRowBytes, kRawBufferWord3);
    const __amdgpu_buffer_rsrc_t vbuf = __builtin_amdgcn_make_buffer_rsrc(V, (short)0, n * kRowBytes, kRawBufferWord3);
    // scores (s += q[d] * k[d] in column order, then * scale * scale) and
    // their maxima (NaN scores never become one, as with std::max)
    float m[HPW];
#pragma unroll
    for (int i = 0; i < HPW; ++i) m[i] = -INFINITY;
    v4u pre[PER];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = threadIdx.x + i * (int)blockDim.x;   // past 64 * 16: a row past the keys (reads 0)
            pre[i] = __builtin_amdgcn_raw_buffer_load_b128(kbuf, (k0 + f / (dim / 4)) * kRowBytes + 16 * (f % (dim / 4)),
                                                           0, 0);
        }
    };
    fetch(0);
    for (int k0 = 0; k0 < n; k0 += kWave) {
        __syncthreads();   // every wave is done with the previous keys' rows
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = threadIdx.x + i * (int)blockDim.x;
            if (f < kWave * dim / 4) *reinterpret_cast<v4u*>(kt + f / (dim / 4) * kRoKPitch + 4 * (f % (dim / 4))) = pre[i];
        }
        __syncthreads();
        if (k0 + kWave < n) fetch(k0 + kWave);
        // the row in two halves: 32 registers for it instead of 64
        float s[HPW];
#pragma unroll
        for (int i = 0; i < HPW; ++i) s[i] = 0.0f;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            v4f kr[dim / 8];
#pragma unroll
            for (int j = 0; j < dim / 8; ++j)
                kr[j] = *reinterpret_cast<const v4f*>(kt + lane * kRoKPitch + 4 * (j + half * dim / 8));
#pragma unroll
            for (int d = 0; d < dim / 2; ++d)
#pragma unroll
                for (int i = 0; i < HPW; ++i) s[i] = s[i] + qs[i][d + half * dim / 2] * kr[d / 4][d % 4];
        }
        const int key = k0 + lane;
#pragma unroll
        for (int i = 0; i < HPW; ++i) {
            s[i] = s[i] * p.scale * p.scale;
            if (key < n) {
                sc[i][key] = s[i];
                m[i] = m[i] < s[i] ? s[i] : m[i];
            }
        }
    }
    // from here on each wave works alone (no block barrier)
    float maximum[HPW];
    bool live[HPW];   // a fully masked (or infinite) row: the CPU leaves the zero-filled output
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float other = __shfl_xor(m[i], off, kWave);
            m[i] = m[i] < other ? other : m[i];
        }
        maximum[i] = m[i];
        live[i] = isfinite(maximum[i]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // exp(s - max) with glibc's expf (its table in LDS), eight per lane at a time
#pragma unroll
    for (int i = 0; i < HPW; ++i)
        for (int k0 = 0; k0 < n; k0 += 8 * kWave) {
            float e[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int k = k0 + u * kWave + lane;
                e[u] = (k < n ? sc[i][k] : 0.0f) - maximum[i];
            }
            libm_expf_batch(e, [exp2](uint32_t k) { return exp2[k]; });
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int k = k0 + u * kWave + lane;
                if (k < n) sc[i][k] = e[u];
            }
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the denominators in key order: one chain per wave (with two heads,
    // lanes 0-31 form the first head's and lanes 32-63 the second's, each
    // lane alike within its half); groups of eight terms are read
    // kRoDenAhead groups ahead of their adds, so the chain does not wait for
    // LDS (the scores' registers are free by now)
    static_assert(HPW <= 2, "one denominator chain per half-wave");
    float den[HPW];
    {
        constexpr int kRoDenAhead = 3;
        const int groups8 = n / 8;
        const float* src = HPW == 2 && lane >= 32 ? sc[HPW - 1] : sc[0];
        v4f ring[kRoDenAhead][2];
        auto read8 = [&](v4f (&r)[2], int g) {
            const int at = 8 * min(g, max(groups8 - 1, 0));   // past the last group: read again, unused
            r[0] = *reinterpret_cast<const v4f*>(src + at);
            r[1] = *reinterpret_cast<const v4f*>(src + at + 4);
        };
        float chain = 0.0f;
        auto add8 = [&](const v4f (&r)[2]) {
#pragma unroll
            for (int j = 0; j < 8; ++j) chain = chain + r[j / 4][j % 4];
        };
#pragma unroll
        for (int u = 0; u < kRoDenAhead; ++u) read8(ring[u], u);
        int g = 0;
        for (; g + kRoDenAhead <= groups8; g += kRoDenAhead) {
#pragma unroll
            for (int u = 0; u < kRoDenAhead; ++u) {
                const v4f cur[2] = {ring[u][0], ring[u][1]};
                read8(ring[u], g + u + kRoDenAhead);
                add8(cur);
            }
        }
        // the last groups (fewer than kRoDenAhead) are already in the ring
#pragma unroll
        for (int u = 0; u < kRoDenAhead; ++u)
            if (g + u < groups8) add8(ring[u]);
        for (int k = 8 * groups8; k < n; ++k) chain = chain + src[k];
#pragma unroll
        for (int i = 0; i < HPW; ++i)
            den[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, chain), 32 * i));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // p = e / den; the slots past n hold +0, so the chain's reads past the
    // keys add p * v = +0 * 0, which leaves a sum that started at +0 unchanged
    const int slots = ro_wave_row_floats(n);
#pragma unroll
    for (int i = 0; i < HPW; ++i)
        for (int k = lane; k < slots; k += kWave) sc[i][k] = k < n ? sc[i][k] / den[i] : 0.0f;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // output[d] += p * v[d] in key order, lane d, one chain per head;
    // kRoWaveDepth chunks of V in flight, each chunk's p read one chunk ahead
    const int chunks = (n + kRoWaveKeys - 1) / kRoWaveKeys;
    const int groups = (chunks + kRoWaveDepth - 1) / kRoWaveDepth;
    float ring[kRoWaveDepth][kRoWaveKeys];
    auto load = [&](float (&r)[kRoWaveKeys], int c) {
        const int at = lane * (int)sizeof(float) + c * kRoWaveKeys * kRowBytes;
#pragma unroll
        for (int j = 0; j < kRoWaveKeys; ++j)
            r[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(vbuf, at + j * kRowBytes, 0, 0));
    };
    v4f pp[2][HPW][kRoWaveKeys / 4];
    auto read_p = [&](v4f (&pr)[HPW][kRoWaveKeys / 4], int c) {
#pragma unroll
        for (int i = 0; i < HPW; ++i)
#pragma unroll
            for (int j = 0; j < kRoWaveKeys / 4; ++j)
                pr[i][j] = *reinterpret_cast<const v4f*>(sc[i] + c * kRoWaveKeys + 4 * j);
    };
#pragma unroll
    for (int u = 0; u < kRoWaveDepth; ++u) load(ring[u], u);
    read_p(pp[0], 0);
    float acc[HPW];
#pragma unroll
    for (int i = 0; i < HPW; ++i) acc[i] = 0.0f;
    static_assert(kRoWaveDepth % 2 == 0 && kRoWaveKeys == 12, "p pairs alternate; the wait names twelve values");
    for (int g = 0; g < groups; ++g) {
#pragma unroll
        for (int u = 0; u < kRoWaveDepth; ++u) {
            const int c = g * kRoWaveDepth + u;
            read_p(pp[(u + 1) & 1], c + 1);
            float (&r)[kRoWaveKeys] = ring[u];
            // one wait for the whole chunk
            asm volatile("" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]),
                              "+v"(r[7]), "+v"(r[8]), "+v"(r[9]), "+v"(r[10]), "+v"(r[11]));
#pragma unroll
            for (int i = 0; i < HPW; ++i) asm volatile("" : "+v"(pp[u & 1][i][0]), "+v"(pp[u & 1][i][1]), "+v"(pp[u & 1][i][2]));
#pragma unroll
            for (int j = 0; j < kRoWaveKeys; ++j)
#pragma unroll
                for (int i = 0; i < HPW; ++i) acc[i] = acc[i] + pp[u & 1][i][j / 4][j % 4] * ring[u][j];
            load(ring[u], c + kRoWaveDepth);
        }
    }
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
        const int h = kvh * group + w + i * waves;
        p.out[((size_t)t * p.heads + h) * dim + lane] = live[i] ? acc[i] : 0.0f;
    }
}

// Single-token attention at head dim 64 (decode): the same arithmetic as
// ro_attention_kernel, arranged so that no dependent sum waits on memory.
//   * Scores: thread k takes keys k, k + 512, ...; the next key's row loads
//     into registers while the current one is summed (q . k in column order,
//     q read from LDS).
//   * Exponentials: four independent keys per thread at a time.
//   * Output: output[d] = (...(p_0 v_0[d]) + p_1 v_1[d]) + ...) in key order.
//     The products are independent of the running sum.  The V rows of up to
//     kRoRound keys are loaded into registers (all threads, coalesced) while
//     the denominator is formed; then, chunk by chunk,
//     all threads write p_k * v_k[d] into an LDS buffer and wave 0 adds a
//     chunk's products in key order (lane d, output element d); the next
//     chunk's products are written once wave 0 is done with the buffer (the
//     barrier at the top of each chunk), so one buffer serves every chunk.
constexpr int kRoChunk = 128;                                          // keys per product buffer
constexpr int kRoDecodeDim = 64;
constexpr int kRoDecodeBlock = 512;                                  // threads of the decode kernel
constexpr int kRoChunkF4 = kRoChunk * kRoDecodeDim / 4 / kRoDecodeBlock;    // float4 per thread per chunk (4)
constexpr int kRoRoundChunks = 5;
constexpr int kRoRound = kRoChunk * kRoRoundChunks;                    // keys whose V rows sit in registers

__global__ __launch_bounds__(kRoDecodeBlock) void ro_attention_decode_kernel(AttentionCall p) {
    constexpr int D = kRoDecodeDim;
    extern __shared__ float lds[];
    float* qs = lds;                          // [D]
    float* prod = lds + D;                    // [kRoChunk][D] products p_k * v_k[d]
    float* sc = prod + kRoChunk * D;          // [visible keys]: scores, then e, then p
    __shared__ float red[kRoDecodeBlock / kWave];
    __shared__ float den_shared;
    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    const int position = p.position_ptr ? *p.position_ptr : p.position;
    const int end = position + 1;
    const int begin = (p.window && end > p.window) ? end - p.window : 0;
    const int n = end - begin;
    const int kvh = h / (p.heads / p.kv_heads);
    const float* q = p.q_heads + (size_t)h * D;
    const float* K = p.keys + ((size_t)kvh * p.capacity + begin) * D;
    const float* V = p.values + ((size_t)kvh * p.capacity + begin) * D;
    float* o = p.out + (size_t)h * D;
    if (tid < D) qs[tid] = q[tid];
    __syncthreads();

    // ---- scores (q . k) * scale * scale and their maximum
    float m = -INFINITY;
    {
        v4f cur[D / 4], nxt[D / 4];
        auto load_row = [&](v4f (&dst)[D / 4], int k) {
            const v4f* src = reinterpret_cast<const v4f*>(K + (size_t)k * D);
#pragma unroll
            for (int j = 0; j < D / 4; ++j) dst[j] = src[j];
        };
        if (tid < n) load_row(cur, tid);
        for (int k = tid; k < n; k += kRoDecodeBlock) {
            if (k + kRoDecodeBlock < n) load_row(nxt, k + kRoDecodeBlock);
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < D / 4; ++j) {
                const v4f q4 = *reinterpret_cast<const v4f*>(qs + 4 * j);
                s += q4[0] * cur[j][0];
                s += q4[1] * cur[j][1];
                s += q4[2] * cur[j][2];
                s += q4[3] * cur[j][3];
            }
            s = s * p.scale * p.scale;
            sc[k] = s;
            m = m < s ? s : m;   // NaN never becomes the maximum (std::max)
#pragma unroll
            for (int j = 0; j < D / 4; ++j) cur[j] = nxt[j];
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float other = __shfl_xor(m, off, kWave);
        m = m < other ? other : m;
    }
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    float maximum = red[0];
    for (int w = 1; w < kRoDecodeBlock / kWave; ++w) maximum = maximum < red[w] ? red[w] : maximum;
    if (!isfinite(maximum)) {
        // fully masked (or infinite) row: the CPU leaves the zero-filled output
        if (tid < D) o[tid] = 0.0f;
        return;
    }

    // ---- V rows of a round: thread t holds float4 f = t + kRoDecodeBlock i (key
    // r0 + f / 16, columns 4 (f % 16) ..); chunk c of the round is
    // vv[kRoChunkF4 c .. kRoChunkF4 (c + 1))
    v4f vv[kRoRoundChunks * kRoChunkF4];
    auto load_round = [&](int r0) {
#pragma unroll
        for (int i = 0; i < kRoRoundChunks * kRoChunkF4; ++i) {
            const int f = tid + kRoDecodeBlock * i, key = r0 + f / (D / 4);
            vv[i] = key < n ? *reinterpret_cast<const v4f*>(V + (size_t)key * D + 4 * (f % (D / 4)))
                            : v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    // exponentials, four keys per thread at a time (their table reads overlap)
    for (int k0 = 0; k0 < n; k0 += 4 * kRoDecodeBlock) {
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = sc[min(k0 + tid + kRoDecodeBlock * i, n - 1)];
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = libm_expf(e[i] - maximum);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = k0 + tid + kRoDecodeBlock * i;
            if (k < n) sc[k] = e[i];
        }
    }
    __syncthreads();   // every e is written
    // The first round of V lands while the denominator is summed.  (Issued
    // before the exponentials, it would make each table read wait for it:
    // loads complete in order.)
    load_round(0);
    // masked keys add exp(-inf) = 0, which leaves the sum unchanged
    if (tid == 0) den_shared = sequential_sum(sc, n);
    __syncthreads();
    const float den = den_shared;
    for (int k = tid; k < n; k += kRoDecodeBlock) sc[k] = sc[k] / den;

    float acc = 0.0f;
    for (int r0 = 0; r0 < n; r0 += kRoRound) {
        if (r0 > 0) load_round(r0);
#pragma unroll
        for (int c = 0; c < kRoRoundChunks; ++c) {
            const int k0 = r0 + c * kRoChunk;
            if (k0 >= n) break;
            __syncthreads();   // wave 0 is done with this buffer (and, first time, every p is written)
            float* dst = prod;
            // every p of this thread's keys first: a read between the stores
            // below would wait out its latency once per key
            float pks[kRoChunkF4];
#pragma unroll
            for (int i = 0; i < kRoChunkF4; ++i) {
                const int key = k0 + (tid + kRoDecodeBlock * i) / (D / 4);
                pks[i] = key < n ? sc[key] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < kRoChunkF4; ++i) {
                const int f = tid + kRoDecodeBlock * i;
                const float pk = pks[i];
                const v4f v = vv[kRoChunkF4 * c + i];
                v4f r;
                r[0] = pk * v[0];
                r[1] = pk * v[1];
                r[2] = pk * v[2];
                r[3] = pk * v[3];
                // Four 4-byte stores (16-byte LDS accesses of 64 lanes ran
                // several times slower per byte here).  Element d of key kl
                // sits at kl * D + (d ^ (kl % 4)): the 64 lanes of a store
                // (keys 4 j .. 4 j + 3, one e) meet 64 different banks.
                const int swz = (f / (D / 4)) & 3;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    asm volatile("" ::: "memory");
                    dst[4 * f + (e ^ swz)] = r[e];
                }
            }
            __syncthreads();   // the chunk's products are written
            if (tid < D) {
                // output[d] += p * v[d] in key order (16 products at a time
                // into registers); key kl's element d at kl * D + (d ^ (kl % 4))
                const int rows = min(kRoChunk, n - k0);
                int k = 0;
                for (; k + 16 <= rows; k += 16) {
                    float t[16];
#pragma unroll
                    for (int j = 0; j < 16; ++j) t[j] = dst[(k + j) * D + (tid ^ (j & 3))];
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc += t[j];
                }
                for (; k < rows; ++k) acc += dst[k * D + (tid ^ (k & 3))];
            }
        }
    }
    if (tid < D) o[tid] = acc;
}

// ------------------------------------------------------------ activation ---
__device__ __forceinline__ float ro_activate(int activation, float x) {
    if (activation == 0) return x / (1.0f + libm_expf(-x));
    if (activation == 1) return 0.5f * x * (1.0f + erff(x * 0.7071067811865475f));
    if (activation == 2) return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
    return x < 0.0f ? 0.0f : x;   // std::max(x, 0.0f)
}

__global__ void ro_activation_kernel(const float* gate_up, int tokens, int width, int gated, int activation,
                                     float* act) {
    const size_t count = (size_t)tokens * width;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count; i += (size_t)gridDim.x * blockDim.x) {
        const size_t t = i / width, j = i % width;
        if (gated) {
            const float g = gate_up[t * 2 * width + j], u = gate_up[t * 2 * width + width + j];
            act[i] = u * ro_activate(activation, g);
        } else {
            act[i] = ro_activate(activation, gate_up[i]);
        }
    }
}

// ro_activation_kernel's values quantized per row as quantize_rows_kernel
// does (an exact maximum, then the int8 values), one block per row: the
// activation and its quantization in one launch, no FP32 rows.  Thread t
// owns columns t + k * blockDim.x (k < K).
template <int K>
__global__ __launch_bounds__(1024) void ro_activation_quantize_kernel(const float* gate_up, int width, int gated,
                                                                      int activation, int8_t* q, float* scales) {
    __shared__ float wave_max[1024 / kWave];
    const float* in = gate_up + (size_t)blockIdx.x * width * (gated ? 2 : 1);
    float a[K];
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int j = threadIdx.x + k * (int)blockDim.x;
        float v = 0.0f;
        if (j < width) v = gated ? in[width + j] * ro_activate(activation, in[j]) : ro_activate(activation, in[j]);
        a[k] = v;
        m = fmaxf(m, fabsf(v));
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
    const int waves = (int)blockDim.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) wave_max[threadIdx.x / kWave] = m;
    __syncthreads();
    m = 0.0f;
    for (int i = 0; i < waves; ++i) m = fmaxf(m, wave_max[i]);
    const float sx = fmaxf(m / 127.0f, 1e-12f);
    const float multiplier = 1.0f / sx;
    if (threadIdx.x == 0) scales[blockIdx.x] = sx;
    int8_t* out = q + (size_t)blockIdx.x * width;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int j = threadIdx.x + k * (int)blockDim.x;
        if (j < width) out[j] = (int8_t)quantize_one(a[k], multiplier);
    }
}

// One block per vector: the vector staged in LDS in wave_sequential_sum's
// layout, then its column-order sum by that function (method 0, one wave),
// by the plain chain (method 1) or by wave_pair_sequential_sum (method 2, two
// waves), with the clock cycles the sum took.
__global__ __launch_bounds__(2 * kWave) void ro_sequential_sum_kernel(const float* x, int n, float* sums,
                                                                      long long* cycles, int method) {
    extern __shared__ float lds[];
    float4* area0 = reinterpret_cast<float4*>(lds);
    float4* area1 = area0 + kSeqSumArea;
    float4* xchg = area1 + kSeqSumArea;
    float4* comp = xchg + kSeqPairXchg;
    float* v = reinterpret_cast<float*>(comp + 2 * kSeqPairComp);
    const float* row = x + (size_t)blockIdx.x * n;
    const SeqLayout lay(n);
    const int w = threadIdx.x / kWave;
    for (int j = threadIdx.x; j < n; j += blockDim.x) v[lay.at(j)] = row[j];
    seq_zero_tail(v, n, threadIdx.x, blockDim.x);
    // the sums take non-negative terms; a row with a negative one (not a
    // norm's squares or a softmax's exponentials) takes the chain
    bool negative = false;
    for (int j = threadIdx.x; j < n; j += blockDim.x) negative |= __float_as_uint(row[j]) > 0x80000000u;
    const bool parallel = method != 1 && !__syncthreads_or(negative);
    const long long t0 = clock64();
    float s;
    if (!parallel)
        s = seq_chain(v, n, lay.E);
    else if (method == 0)
        s = wave_sequential_sum(v, n, area0);
    else
        wave_pair_sequential_sum(v, n, area0, area1, xchg, comp + w * kSeqPairComp, w,
                                 [] { __syncthreads(); return true; }, s);
    const long long t1 = clock64();
    // method 2: both waves formed the sum; they must agree bit for bit
    __shared__ unsigned second;
    if (threadIdx.x == kWave) second = __float_as_uint(s);
    __syncthreads();
    if (threadIdx.x == 0) {
        sums[blockIdx.x] = method == 2 && second != __float_as_uint(s) ? __uint_as_float(0x7fc0deadu) : s;
        if (cycles) cycles[blockIdx.x] = t1 - t0;
    }
}

// Eight inputs per thread through libm_expf_batch (the decode step's softmax
// form), so that lh_expf checks that form.
__global__ void ro_expf_kernel(const float* x, size_t count, float* y) {
    const size_t stride = (size_t)gridDim.x * blockDim.x * 8;
    for (size_t i0 = (blockIdx.x * (size_t)blockDim.x + threadIdx.x) * 8; i0 < count; i0 += stride) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = i0 + k < count ? x[i0 + k] : 0.0f;
        libm_expf_batch(v, [](uint32_t k) { return kExp2Table32[k]; });
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (i0 + k < count) y[i0 + k] = v[k];
    }
}

// ------------------------------------------------------------------ dot ----
// The unscaled value a vector lane of dot_avx loads (f32 as stored, INT8 and
// INT4 as integers; decoder.cpp:299-320), and Weight::value (:236-251).
template <int BITS>
__device__ __forceinline__ float lane_value(const WeightView& w, size_t index) {
    if constexpr (BITS == 32) return ((const float*)w.data)[index];
    else if constexpr (BITS == 16) return bf16_to_f32(((const uint16_t*)w.data)[index]);
    else if constexpr (BITS == 8) return (float)((const int8_t*)w.data)[index];
    else return (float)nibble(((const uint8_t*)w.data)[index / 2], (int)(index & 1));
}

// Horizontal sum of the eight lanes of an aligned 8-lane group in the CPU's
// order: (l0+l4, l1+l5, l2+l6, l3+l7) -> (h0+h2, h1+h3) -> p0 + p1.  Every
// lane of the group ends with the total (IEEE addition is commutative, so
// which operand comes first does not matter).
__device__ __forceinline__ float reduce8(float v) {
    const int wl = threadIdx.x & 63, base = wl & ~7, l = wl & 7;
    const float h = v + __shfl(v, base + ((l + 4) & 7), kWave);      // lanes 0-3: h_l = v_l + v_{l+4}
    const float pp = h + __shfl(h, base + ((l + 2) & 3), kWave);     // lanes 0, 1: p_l = h_l + h_{l+2}
    return __shfl(pp, base, kWave) + __shfl(pp, base + 1, kWave);
}

// y[t, row] for one (row, group of up to four tokens) per 32-lane worker.
template <int BITS>
__global__ __launch_bounds__(kRoBlock) void ro_gemv_kernel(WeightView w, const float* __restrict__ x, int tokens,
                                                           float* y, int epilogue) {
    const int lane = threadIdx.x & 31;
    const int worker = (int)((blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 5);
    const int token_groups = (tokens + 3) / 4;
    const bool live = worker < w.rows * token_groups;
    const int row = live ? worker / token_groups : 0;
    const int t0 = live ? (worker % token_groups) * 4 : 0;
    const int count = min(4, tokens - t0);
    const int K = w.cols;
    const int group = (BITS == 32 || BITS == 16) ? K : w.group;
    const int groups = K / group;
    const size_t base = (size_t)row * K;
    // token of this lane in the multi-token chains (lanes 8 tt .. 8 tt + 7)
    const int tt = lane >> 3, l = lane & 7;
    const bool chain = tt < count;
    const float* xt = x + (size_t)(t0 + (count == 1 ? 0 : min(tt, count - 1))) * K;
    float result = 0.0f;   // lanes 8 tt: the result of token tt
    for (int g = 0; g < groups; ++g) {
        int col = g * group;
        const int end = col + group;
        float acc = 0.0f;
        if (count == 1) {
            // lane c * 8 + l runs lane l of chain c (a, b, c, d)
            for (; col + 32 <= end; col += 32) acc = fmaf(lane_value<BITS>(w, base + col + lane), xt[col + lane], acc);
            const int half = threadIdx.x & 32;
            const float b = __shfl(acc, half + l + 8, kWave);
            const float c = __shfl(acc, half + l + 16, kWave);
            const float d = __shfl(acc, half + l + 24, kWave);
            acc = (acc + b) + (c + d);                  // lanes 0-7 of the worker: the combined chains
        }
        for (; col + 8 <= end; col += 8)
            acc = fmaf(lane_value<BITS>(w, base + col + l), xt[col + l], acc);
        float partial = reduce8(acc);
        float scale = 1.0f;
        if constexpr (BITS == 8 || BITS == 4) scale = w.scales[(size_t)row * groups + g];
        for (; col < end; ++col) {
            float value = lane_value<BITS>(w, base + col);
            if constexpr (BITS == 8 || BITS == 4) value = (value * scale) / scale;   // Weight::value / scale
            else if constexpr (BITS == 32) value = value / scale;
            partial = fmaf(value, xt[col], partial);
        }
        if constexpr (BITS == 16) result = 0.0f + partial;                 // one group
        else result = fmaf(partial, scale, result);
    }
    if (live && chain && l == 0) {
        const size_t index = (size_t)(t0 + tt) * w.rows + row;
        const float v = result + (w.bias ? w.bias[row] : 0.0f);
        y[index] = epilogue == kAccumulate ? y[index] + v : v;
    }
}

// One token, FP32 rows whose width is a multiple of 32: ro_gemv_kernel's
// single-token order with eight lanes per row, eight rows per wave.  Lane j
// of a row loads columns 32 s + 4 j .. + 3 with one 16-byte load and runs
// their four chain lanes (lanes 4 (j % 2) .. + 3 of chain j / 2 of the four
// 8-lane chains a, b, c, d), so a wave's load covers eight whole 128-byte row
// segments; the chains are then combined, (a + b) + (c + d), and reduced as
// reduce8 does.
__global__ __launch_bounds__(kRoBlock) void ro_gemv_f32_rows_kernel(WeightView w, const float* __restrict__ x,
                                                                    float* y, int epilogue) {
    const int lane = threadIdx.x & 63, j = lane & 7;
    const int row = (int)((blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 3);
    const bool live = row < w.rows;
    const int K = w.cols;
    const v4f* wr = reinterpret_cast<const v4f*>(static_cast<const float*>(w.data) + (size_t)(live ? row : 0) * K) + j;
    const v4f* xr = reinterpret_cast<const v4f*>(x) + j;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int steps = K / 32;
    constexpr int kU = 16;  // steps in flight
    int s = 0;
    for (; s + kU <= steps; s += kU) {
        v4f wv[kU], xv[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            wv[u] = __builtin_nontemporal_load(wr + (size_t)(s + u) * 8);
            xv[u] = xr[(s + u) * 8];
        }
#pragma unroll
        for (int u = 0; u < kU; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = fmaf(wv[u][i], xv[u][i], acc[i]);
    }
    for (; s < steps; ++s) {
        const v4f wv = __builtin_nontemporal_load(wr + (size_t)s * 8), xv = xr[s * 8];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(wv[i], xv[i], acc[i]);
    }
    // lanes j = 0, 1 (chain a) combine chain lane 4 j + i with b, c, d:
    // (a + b) + (c + d)
    const int base = lane & ~7;
    float c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float b = __shfl(acc[i], base + (j & 1) + 2, kWave);
        const float cc = __shfl(acc[i], base + (j & 1) + 4, kWave);
        const float d = __shfl(acc[i], base + (j & 1) + 6, kWave);
        c[i] = (acc[i] + b) + (cc + d);
    }
    // reduce8 over the combined lanes 0-7 (lane 0 of the row holds 0-3,
    // lane 1 holds 4-7): (l0 + l4, l1 + l5, l2 + l6, l3 + l7) -> (h0 + h2,
    // h1 + h3) -> p0 + p1
    float h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) h[i] = c[i] + __shfl(c[i], base + 1, kWave);
    const float partial = (h[0] + h[2]) + (h[1] + h[3]);
    const float result = fmaf(partial, 1.0f, 0.0f);
    if (live && j == 0) {
        const float v = result + (w.bias ? w.bias[row] : 0.0f);
        y[row] = epilogue == kAccumulate ? y[row] + v : v;
    }
}

// Full groups of four tokens (every group but a ragged last one), TG groups
// per 32-lane worker: lane 8 tt + l runs lane l of token tt's chain in each
// group, so one load of a weight element serves all 4 TG tokens.  The order
// per token is that of ro_gemv_kernel's multi-token case.
template <int BITS, int TG>
__global__ __launch_bounds__(kRoBlock) void ro_gemm_kernel(WeightView w, const float* __restrict__ x, int groups,
                                                           float* y, int epilogue) {
    const int lane = threadIdx.x & 31;
    const int worker = (int)((blockIdx.x * (size_t)blockDim.x + threadIdx.x) >> 5);
    const int per_row = (groups + TG - 1) / TG;
    const bool live = worker < w.rows * per_row;
    const int row = live ? worker / per_row : 0;
    const int g0 = live ? (worker % per_row) * TG : 0;
    const int K = w.cols;
    const int group = (BITS == 32 || BITS == 16) ? K : w.group;
    const int sgroups = K / group;
    const size_t base = (size_t)row * K;
    const int tt = lane >> 3, l = lane & 7;
    const float* xt[TG];
#pragma unroll
    for (int j = 0; j < TG; ++j) xt[j] = x + (size_t)(4 * min(g0 + j, groups - 1) + tt) * K;
    float result[TG];
#pragma unroll
    for (int j = 0; j < TG; ++j) result[j] = 0.0f;
    for (int g = 0; g < sgroups; ++g) {
        int col = g * group;
        const int end = col + group;
        float acc[TG];
#pragma unroll
        for (int j = 0; j < TG; ++j) acc[j] = 0.0f;
        for (; col + 8 <= end; col += 8) {
            const float wv = lane_value<BITS>(w, base + col + l);
#pragma unroll
            for (int j = 0; j < TG; ++j) acc[j] = fmaf(wv, xt[j][col + l], acc[j]);
        }
        float scale = 1.0f;
        if constexpr (BITS == 8 || BITS == 4) scale = w.scales[(size_t)row * sgroups + g];
        float partial[TG];
#pragma unroll
        for (int j = 0; j < TG; ++j) partial[j] = reduce8(acc[j]);
        for (; col < end; ++col) {
            float value = lane_value<BITS>(w, base + col);
            if constexpr (BITS == 8 || BITS == 4) value = (value * scale) / scale;
            else if constexpr (BITS == 32) value = value / scale;
#pragma unroll
            for (int j = 0; j < TG; ++j) partial[j] = fmaf(value, xt[j][col], partial[j]);
        }
#pragma unroll
        for (int j = 0; j < TG; ++j) {
            if constexpr (BITS == 16) result[j] = 0.0f + partial[j];
            else result[j] = fmaf(partial[j], scale, result[j]);
        }
    }
    if (live && l == 0) {
        const float b = w.bias ? w.bias[row] : 0.0f;
#pragma unroll
        for (int j = 0; j < TG; ++j)
            if (g0 + j < groups) {
                const size_t index = (size_t)(4 * (g0 + j) + tt) * w.rows + row;
                const float v = result[j] + b;
                y[index] = epilogue == kAccumulate ? y[index] + v : v;
            }
    }
}

// Dynamic LDS beyond the default 64 KiB must be allowed per kernel first
// (up to the 160 KiB of a CU less the kernel's static arrays); false when the
// runtime refuses the size.
template <typename K>
bool allow_lds(K kernel, size_t bytes, int& allowed) {
    if (bytes <= 65536 || (int)bytes <= allowed) return true;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)bytes) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    allowed = (int)bytes;
    return true;
}
int g_norm_lds = 0, g_rms_norm_lds = 0, g_attention_lds = 0, g_attention_decode_lds = 0, g_attention_wave_lds[7] = {};

}  // namespace

// --------------------------------------------------------------- launchers ---
bool launch_norm_quantize_reference_order(const float* x, int rows, int width, const NormView& norm, int8_t* q,
                                          float* scales, hipStream_t stream) {
    static_assert(kReferenceOrderQuantizeMaxWidth == kSeqSumMaxPerLane * kWave, "the pair sum's width");
    if (norm.kind != 0 || norm.accurate || width < 1 || width > kReferenceOrderQuantizeMaxWidth || rows < 1)
        return false;
    const size_t lds = (size_t)(2 * kSeqSumArea + kSeqPairXchg + 2 * kSeqPairComp) * sizeof(float4) +
                       (size_t)seq_per_lane_host(width) * kWave * sizeof(float);
    if (!allow_lds(ro_rms_norm_kernel, lds, g_rms_norm_lds)) return false;
    ro_rms_norm_kernel<<<rows, 2 * kWave, lds, stream>>>(x, width, norm, nullptr, 0, 0, q, scales);
    return true;
}

bool launch_norm_reference_order(const float* x, int rows, int width, const NormView& norm, float* y,
                                 hipStream_t stream, int rows_per_group, size_t group_stride) {
    if (width > kReferenceOrderMaxWidth) return false;
    if (norm.kind == 0 && !norm.accurate && width <= kSeqSumMaxPerLane * kWave) {
        const size_t lds = (size_t)(2 * kSeqSumArea + kSeqPairXchg + 2 * kSeqPairComp) * sizeof(float4) +
                           (size_t)seq_per_lane_host(width) * kWave * sizeof(float);
        if (allow_lds(ro_rms_norm_kernel, lds, g_rms_norm_lds)) {
            ro_rms_norm_kernel<<<rows, 2 * kWave, lds, stream>>>(x, width, norm, y, rows_per_group, group_stride);
            return true;
        }
    }
    const size_t lds = 2 * (size_t)width * sizeof(float);
    if (!allow_lds(ro_norm_kernel, lds, g_norm_lds)) return false;
    ro_norm_kernel<<<rows, kRoBlock, lds, stream>>>(x, width, norm, y, rows_per_group, group_stride);
    return true;
}

// LDS of the decode kernel (the larger one): q, the product buffer, the
// scores; 1 KiB stays for the static arrays.
int reference_order_attention_keys() { return (160 * 1024 - 1024) / 4 - kRoDecodeDim - kRoChunk * kRoDecodeDim; }

namespace {
// One block per (query head, query token), any head width.
bool launch_attention_rows(const AttentionCall& p, int max_keys, hipStream_t stream) {
    const size_t lds = ((size_t)p.dim + max_keys) * sizeof(float);
    if (!allow_lds(ro_attention_kernel, lds, g_attention_lds)) return false;
    dim3 grid(p.heads, p.tokens);
    ro_attention_kernel<<<grid, kRoBlock, lds, stream>>>(p);
    return true;
}
}  // namespace

bool launch_attention_reference_order(const AttentionCall& p, int max_keys, hipStream_t stream) {
    if (max_keys > reference_order_attention_keys() || p.dim > 256) return false;
    if (p.tokens == 1 && p.dim == kRoDecodeDim) {
        const size_t lds = ((size_t)kRoDecodeDim + kRoChunk * kRoDecodeDim + max_keys) * sizeof(float);
        if (!allow_lds(ro_attention_decode_kernel, lds, g_attention_decode_lds)) return false;
        ro_attention_decode_kernel<<<p.heads, kRoDecodeBlock, lds, stream>>>(p);
        return true;
    }
    const int group = p.heads / p.kv_heads;
    if (p.dim == kRoWaveDim && group <= kRoMaxGroup) {
        const int row_floats = ro_wave_row_floats(max_keys);
        const size_t lds = ((size_t)kWave * kRoKPitch + (size_t)group * row_floats) * sizeof(float) +
                           32 * sizeof(uint64_t);   // expf's table
        // two heads per wave when the group pairs up (their chains interleave),
        // with at least two waves per block
        const int hpw = group % 2 == 0 && group >= 4 ? 2 : 1;
        const int threads = group / hpw * kWave, per = (kWave * kRoWaveDim / 4 + threads - 1) / threads;
        auto run = [&](auto kernel, int& allowed) {
            if (!allow_lds(kernel, lds, allowed)) return launch_attention_rows(p, max_keys, stream);
            kernel<<<p.kv_heads * p.tokens, threads, lds, stream>>>(p, row_floats);
            return true;
        };
        if (hpw == 2) {
            if (per <= 2) return run(ro_attention_wave_kernel<2, 2>, g_attention_wave_lds[4]);
            if (per <= 4) return run(ro_attention_wave_kernel<4, 2>, g_attention_wave_lds[5]);
            return run(ro_attention_wave_kernel<8, 2>, g_attention_wave_lds[6]);   // 128 threads or more
        }
        if (per <= 2) return run(ro_attention_wave_kernel<2, 1>, g_attention_wave_lds[0]);
        if (per <= 4) return run(ro_attention_wave_kernel<4, 1>, g_attention_wave_lds[1]);
        if (per <= 8) return run(ro_attention_wave_kernel<8, 1>, g_attention_wave_lds[2]);
        return run(ro_attention_wave_kernel<16, 1>, g_attention_wave_lds[3]);
    }
    return launch_attention_rows(p, max_keys, stream);
}

bool launch_activation_quantize_reference_order(const float* gate_up, int tokens, int width, int gated,
                                                int activation, int8_t* q, float* scales, hipStream_t stream) {
    if (tokens < 1 || width < 1 || width > 8 * 1024) return false;
    const int k = (width + 1023) / 1024;
    if (k <= 2) ro_activation_quantize_kernel<2><<<tokens, 1024, 0, stream>>>(gate_up, width, gated, activation, q, scales);
    else if (k <= 4) ro_activation_quantize_kernel<4><<<tokens, 1024, 0, stream>>>(gate_up, width, gated, activation, q, scales);
    else if (k <= 6) ro_activation_quantize_kernel<6><<<tokens, 1024, 0, stream>>>(gate_up, width, gated, activation, q, scales);
    else ro_activation_quantize_kernel<8><<<tokens, 1024, 0, stream>>>(gate_up, width, gated, activation, q, scales);
    return true;
}

void launch_activation_reference_order(const float* gate_up, int tokens, int width, int gated, int activation,
                                       float* act, hipStream_t stream) {
    const size_t count = (size_t)tokens * width;
    const int grid = (int)std::min<size_t>((count + kRoBlock - 1) / kRoBlock, 4096);
    ro_activation_kernel<<<grid, kRoBlock, 0, stream>>>(gate_up, tokens, width, gated, activation, act);
}

bool launch_sequential_sum(const float* x, int n, int count, float* sums, long long* cycles, int method,
                           hipStream_t stream) {
    if (n < 1 || n > kSequentialSumMax || count < 1 || method < 0 || method > 2) return false;
    const size_t lds = (size_t)(2 * kSeqSumArea + kSeqPairXchg + 2 * kSeqPairComp) * sizeof(float4) +
                       (size_t)seq_per_lane_host(n) * kWave * sizeof(float);
    ro_sequential_sum_kernel<<<count, method == 2 ? 2 * kWave : kWave, lds, stream>>>(x, n, sums, cycles, method);
    return true;
}

void launch_libm_expf(const float* x, size_t count, float* y, hipStream_t stream) {
    const int grid = (int)std::min<size_t>((count + kRoBlock - 1) / kRoBlock, 8192);
    ro_expf_kernel<<<grid ? grid : 1, kRoBlock, 0, stream>>>(x, count, y);
}

namespace {
template <int BITS>
void launch_ro_linear(const WeightView& w, const float* x, int tokens, float* y, int epilogue, hipStream_t stream) {
    constexpr int TG = 16;
    // Full groups of four while more than 4 TG tokens remain, then the rest
    // (up to 4 TG tokens, the ragged group among them) one group per worker.
    const int batched = tokens > 4 * TG ? tokens / 4 : 0;   // whole groups; a ragged one stays in the rest
    if (batched) {
        const size_t workers = (size_t)w.rows * ((batched + TG - 1) / TG);
        const int grid = (int)((workers * 32 + kRoBlock - 1) / kRoBlock);
        ro_gemm_kernel<BITS, TG><<<grid, kRoBlock, 0, stream>>>(w, x, batched, y, epilogue);
    }
    const int rest = tokens - 4 * batched;
    if constexpr (BITS == 32) {
        if (tokens == 1 && w.cols % 32 == 0) {
            const int grid = (int)(((size_t)w.rows * 8 + kRoBlock - 1) / kRoBlock);
            ro_gemv_f32_rows_kernel<<<grid, kRoBlock, 0, stream>>>(w, x, y, epilogue);
            return;
        }
    }
    if (rest > 0) {
        const size_t workers = (size_t)w.rows * ((rest + 3) / 4);
        const int grid = (int)((workers * 32 + kRoBlock - 1) / kRoBlock);
        ro_gemv_kernel<BITS><<<grid, kRoBlock, 0, stream>>>(w, x + (size_t)4 * batched * w.cols, rest,
                                                            y + (size_t)4 * batched * w.rows, epilogue);
    }
}
}  // namespace

bool launch_linear_fp_reference_order(const WeightView& w, const float* x, int tokens, float* y, int epilogue,
                                      hipStream_t stream) {
    switch (w.bits) {
    case 32: launch_ro_linear<32>(w, x, tokens, y, epilogue, stream); return true;
    case 16: launch_ro_linear<16>(w, x, tokens, y, epilogue, stream); return true;
    case 8: launch_ro_linear<8>(w, x, tokens, y, epilogue, stream); return true;
    case 4: launch_ro_linear<4>(w, x, tokens, y, epilogue, stream); return true;
    default: return false;
    }
}

}  // namespace leafhip
