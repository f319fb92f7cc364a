// Decoder kernels for MI355X (gfx950, CDNA4, wave64).
//
// Layout conventions (all device-resident, row-major):
//   weights   [rows, cols] in their artifact storage (f32 / BF16 bits / int8 /
//             signed nibbles), rows 16-byte aligned so a lane streams one
//             128-bit chunk per load;
//   hidden    [tokens, width] f32;
//   KV cache  [kv_heads, capacity, dim] f32 per layer.
// Decode GEMVs are HBM-bound: a wave owns whole rows, lanes stride over
// 128-bit chunks of them (coalesced 1 KiB per wave load), and the dot product
// is reduced across the wave with butterfly shuffles.  Prefill linears run on
// MFMA (int8 for W8A8, f32 otherwise).
#include "device_common.h"
#include "kernels.h"
#include "libm_expf.h"

#include <math.h>

namespace leafhip {
namespace {

constexpr int kBlock = 256;
constexpr int kWideRow = 1024;   // threads of the per-token row kernels (norm, quantize)

__device__ __forceinline__ float weight_value(const WeightView& w, int row, int col) {
    const size_t index = (size_t)row * w.cols + col;
    if (w.bits == 32) return ((const float*)w.data)[index];
    if (w.bits == 16) return bf16_to_f32(((const uint16_t*)w.data)[index]);
    int q;
    if (w.bits == 8) q = ((const int8_t*)w.data)[index];
    else q = nibble(((const uint8_t*)w.data)[index / 2], (int)(index & 1));
    return (float)q * w.scales[(size_t)row * (w.cols / w.group) + col / w.group];
}

__device__ __forceinline__ float bias_at(const WeightView& w, int row) {
    return w.bias ? w.bias[row] : 0.0f;
}

__device__ __forceinline__ int weight_int(const WeightView& w, int row, int col) {
    const size_t index = (size_t)row * w.cols + col;
    if (w.bits == 8) return ((const int8_t*)w.data)[index];
    return nibble(((const uint8_t*)w.data)[index / 2], (int)(index & 1));
}

// ------------------------------------------------------------ embedding ---
__global__ void embedding_kernel(WeightView table, WeightView positions, int use_positions, const uint32_t* ids,
                                 int position_base, float scale, float* hidden, const int* position_ptr) {
    const int t = blockIdx.x;
    if (position_ptr) position_base += *position_ptr;
    const int id = (int)ids[t];
    const int h = table.cols;
    for (int c = threadIdx.x; c < h; c += blockDim.x) {
        float v = weight_value(table, id, c) * scale;
        if (use_positions) v = v + weight_value(positions, position_base + t, c);
        hidden[(size_t)t * h + c] = v;
    }
}

// ----------------------------------------------------------------- norm ---
// Per-row statistics of a normalization over `width` values (decoder.cpp:706-727).
// The sums are tree reductions (the CPU path sums left to right).
struct NormStats { float mean, scale; };

__device__ NormStats block_norm_stats(const float* in, int width, const NormView& norm, float* scratch) {
    float mean = 0.0f;
    if (norm.kind == 1) {
        float s = 0.0f;
        for (int c = threadIdx.x; c < width; c += blockDim.x) s += in[c];
        s = block_reduce<float>(s, scratch, [](float a, float b) { return a + b; }, wave_sum_f32);
        mean = s / (float)width;
    }
    float square;
    if (norm.kind == 0 && norm.accurate) {
        double s = 0.0;
        for (int c = threadIdx.x; c < width; c += blockDim.x) { const float v = in[c] * in[c]; s += (double)v; }
        __shared__ double dscratch[16];
        s = block_reduce<double>(s, dscratch, [](double a, double b) { return a + b; }, wave_sum_f64);
        square = (float)s;
    } else {
        float s = 0.0f;
        for (int c = threadIdx.x; c < width; c += blockDim.x) { const float v = in[c] - mean; s += v * v; }
        square = block_reduce<float>(s, scratch, [](float a, float b) { return a + b; }, wave_sum_f32);
    }
    NormStats st;
    st.mean = mean;
    st.scale = 1.0f / sqrtf(square / (float)width + norm.epsilon);
    return st;
}

__device__ __forceinline__ float apply_norm(float x, int c, const NormStats& st, const NormView& norm) {
    return (x - st.mean) * st.scale * norm.gamma[c] + (norm.beta ? norm.beta[c] : 0.0f);
}

// Offset of row `row`: contiguous rows, or groups of rows_per_group rows
// group_stride floats apart.
__device__ __forceinline__ size_t row_offset(int row, int width, int rows_per_group, size_t group_stride) {
    if (rows_per_group <= 0) return (size_t)row * width;
    return (size_t)(row / rows_per_group) * group_stride + (size_t)(row % rows_per_group) * width;
}

__global__ __launch_bounds__(kWideRow) void norm_kernel(const float* x, int width, NormView norm, float* y,
                                                        int rows_per_group, size_t group_stride) {
    __shared__ float scratch[16];
    const size_t at = row_offset(blockIdx.x, width, rows_per_group, group_stride);
    const float* in = x + at;
    float* out = y + at;
    const NormStats st = block_norm_stats(in, width, norm, scratch);
    for (int c = threadIdx.x; c < width; c += blockDim.x) out[c] = apply_norm(in[c], c, st, norm);
}

// ------------------------------------------------------------- quantize ---
// Per-token symmetric int8 quantization (decoder.cpp:1028-1043).
__global__ __launch_bounds__(kBlock) void quantize_kernel(const float* x, int width, int8_t* q, float* scales) {
    __shared__ float scratch[16];
    const float* in = x + (size_t)blockIdx.x * width;
    float m = 0.0f;
    for (int c = threadIdx.x; c < width; c += blockDim.x) m = fmaxf(m, fabsf(in[c]));
    m = block_reduce<float>(m, scratch, [](float a, float b) { return fmaxf(a, b); }, wave_max_f32);
    const float s = fmaxf(m / 127.0f, 1e-12f);
    const float multiplier = 1.0f / s;
    if (threadIdx.x == 0) scales[blockIdx.x] = s;
    int8_t* out = q + (size_t)blockIdx.x * width;
    for (int c = threadIdx.x; c < width; c += blockDim.x) out[c] = (int8_t)quantize_one(in[c], multiplier);
}

// A row's norm and its per-token int8 quantization in one pass over the
// block: the statistics of norm_kernel, then the absmax of the normalized
// values and their quantization as quantize_kernel does them (recomputing
// each normalized value with the same expression), so q and the scale are
// bit-identical to the two kernels in sequence without the f32 round trip.
__global__ __launch_bounds__(kWideRow) void norm_quantize_kernel(const float* x, int width, NormView norm, int8_t* q,
                                                              float* scales) {
    __shared__ float scratch[16];
    const float* in = x + (size_t)blockIdx.x * width;
    const NormStats st = block_norm_stats(in, width, norm, scratch);
    float m = 0.0f;
    for (int c = threadIdx.x; c < width; c += blockDim.x) m = fmaxf(m, fabsf(apply_norm(in[c], c, st, norm)));
    m = block_reduce<float>(m, scratch, [](float a, float b) { return fmaxf(a, b); }, wave_max_f32);
    const float s = fmaxf(m / 127.0f, 1e-12f);
    const float multiplier = 1.0f / s;
    if (threadIdx.x == 0) scales[blockIdx.x] = s;
    int8_t* out = q + (size_t)blockIdx.x * width;
    for (int c = threadIdx.x; c < width; c += blockDim.x)
        out[c] = (int8_t)quantize_one(apply_norm(in[c], c, st, norm), multiplier);
}

// The same row norm + quantization with the row held in registers: thread t
// owns columns t + k * kWideRow (k < K), so every load of the row is issued
// up front instead of once per pass.  Each thread sums its columns in the
// same order as block_norm_stats over kWideRow threads and the reductions are
// the same, so q and the scale are bit-identical to norm_quantize_kernel.
template <int K>
__global__ __launch_bounds__(kWideRow) void norm_quantize_rows_kernel(const float* x, int width, NormView norm,
                                                                   int8_t* q, float* scales) {
    __shared__ float scratch[16];
    const float* in = x + (size_t)blockIdx.x * width;
    float v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int c = threadIdx.x + k * kWideRow;
        v[k] = c < width ? in[c] : 0.0f;
    }
    float mean = 0.0f;
    if (norm.kind == 1) {
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) if (threadIdx.x + k * kWideRow < width) s += v[k];
        s = block_reduce<float>(s, scratch, [](float a, float b) { return a + b; }, wave_sum_f32);
        mean = s / (float)width;
    }
    float square;
    if (norm.kind == 0 && norm.accurate) {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (threadIdx.x + k * kWideRow < width) { const float w = v[k] * v[k]; s += (double)w; }
        __shared__ double dscratch[16];
        s = block_reduce<double>(s, dscratch, [](double a, double b) { return a + b; }, wave_sum_f64);
        square = (float)s;
    } else {
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (threadIdx.x + k * kWideRow < width) { const float w = v[k] - mean; s += w * w; }
        square = block_reduce<float>(s, scratch, [](float a, float b) { return a + b; }, wave_sum_f32);
    }
    NormStats st;
    st.mean = mean;
    st.scale = 1.0f / sqrtf(square / (float)width + norm.epsilon);
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int c = threadIdx.x + k * kWideRow;
        if (c < width) { v[k] = apply_norm(v[k], c, st, norm); m = fmaxf(m, fabsf(v[k])); }
    }
    m = block_reduce<float>(m, scratch, [](float a, float b) { return fmaxf(a, b); }, wave_max_f32);
    const float sc = fmaxf(m / 127.0f, 1e-12f);
    const float multiplier = 1.0f / sc;
    if (threadIdx.x == 0) scales[blockIdx.x] = sc;
    int8_t* out = q + (size_t)blockIdx.x * width;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int c = threadIdx.x + k * kWideRow;
        if (c < width) out[c] = (int8_t)quantize_one(v[k], multiplier);
    }
}

// Columns per thread for the 1024-thread register-row kernels (0: the row
// does not fit).
int wide_row_registers(int width) {
    const int k = (width + kWideRow - 1) / kWideRow;
    for (int c : {1, 2, 3, 4, 6, 8})
        if (k <= c) return c;
    return 0;
}

// quantize_kernel with the row in registers (thread t of T holds columns
// t + k * T): one load pass.  The absmax is exact in any order, so q and the
// scale are bit-identical whatever T is.
template <int K, int T>
__global__ __launch_bounds__(T) void quantize_rows_kernel(const float* x, int width, int8_t* q, float* scales) {
    __shared__ float scratch[16];
    const float* in = x + (size_t)blockIdx.x * width;
    float v[K];
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int c = threadIdx.x + k * T;
        v[k] = c < width ? in[c] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < K; ++k) m = fmaxf(m, fabsf(v[k]));
    m = block_reduce<float>(m, scratch, [](float a, float b) { return fmaxf(a, b); }, wave_max_f32);
    const float s = fmaxf(m / 127.0f, 1e-12f);
    const float multiplier = 1.0f / s;
    if (threadIdx.x == 0) scales[blockIdx.x] = s;
    int8_t* out = q + (size_t)blockIdx.x * width;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int c = threadIdx.x + k * T;
        if (c < width) out[c] = (int8_t)quantize_one(v[k], multiplier);
    }
}

__global__ void scale_columns_kernel(const float* x, int width, size_t count, const float* factors, float* y) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count; i += (size_t)gridDim.x * blockDim.x)
        y[i] = x[i] * factors[i % width];
}

// --------------------------------------------------------- GEMV helpers ---
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 255) | ((uint32_t)(b & 255) << 8) | ((uint32_t)(c & 255) << 16) | ((uint32_t)(d & 255) << 24);
}
// Even / odd columns of eight consecutive int8 values held in two words, so a
// word of INT4 weights widened with widen_nibbles_lo/hi lines up with them.
__device__ __forceinline__ uint32_t even_bytes(uint32_t w0, uint32_t w1) {
    return (w0 & 0x000000FFu) | ((w0 >> 8) & 0x0000FF00u) | ((w1 << 16) & 0x00FF0000u) | ((w1 << 8) & 0xFF000000u);
}
__device__ __forceinline__ uint32_t odd_bytes(uint32_t w0, uint32_t w1) {
    return ((w0 >> 8) & 0x000000FFu) | ((w0 >> 16) & 0x0000FF00u) | ((w1 << 8) & 0x00FF0000u) | (w1 & 0xFF000000u);
}

// Exact W8A8 epilogue for one group per row: ((float)acc * s_x) * s_w, then
// + bias (decoder.cpp:568, 1229).  Separate roundings, as in the CPU path.
__device__ __forceinline__ float int_epilogue(int acc, float sx, float sw) {
    const float term = (float)acc * sx;
    return term * sw;
}

__device__ __forceinline__ void store_out(float* y, size_t index, float value, float bias, int epilogue) {
    const float v = value + bias;
    if (epilogue == kAccumulate) y[index] = y[index] + v;
    else y[index] = v;
}

// Integer dot of one 16-byte weight chunk with the matching activation words.
template <int BITS>
__device__ __forceinline__ int chunk_dot(const uint4 wv, const uint32_t* xw, int acc) {
    if constexpr (BITS == 8) {
        acc = dot4((int)wv.x, (int)xw[0], acc);
        acc = dot4((int)wv.y, (int)xw[1], acc);
        acc = dot4((int)wv.z, (int)xw[2], acc);
        acc = dot4((int)wv.w, (int)xw[3], acc);
    } else {
        const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            acc = dot4(widen_nibbles_lo(words[k]), (int)xw[2 * k], acc);
            acc = dot4(widen_nibbles_hi(words[k]), (int)xw[2 * k + 1], acc);
        }
    }
    return acc;
}

// ------------------------------------------ W8A8/W4A8 decode GEMV (fused) ---
// One token.  Each block first normalizes (optionally) and quantizes the input
// row cooperatively -- float4 loads, block reductions, int8 row into LDS -- so
// no separate quantization launch or grid-wide barrier is needed; the row is
// L2-resident and re-read once per block.  Weight chunks for all of a wave's
// rows are requested before the prologue starts, so the HBM latency of the
// stream overlaps it.  One scale group per row.
constexpr int kFusedMaxK = 6144;                 // 6 float4 per thread
constexpr int kFusedMaxV = kFusedMaxK / (4 * kBlock);

// The activation row as this thread sees it: V float4 per thread (and the
// matching norm gamma / beta), loaded before any weight so that waiting for
// them never waits for the weight stream.
template <int V>
struct RowSlice {
    float4 x[V], g[V], b[V];
    // Branch-free: out-of-range slots load a valid address (issue) and are
    // zeroed later (finish), so no consumer sits between these loads and the
    // weight stream and the compiler can count outstanding loads exactly.
    __device__ __forceinline__ void issue(const float* __restrict__ xp, int K, const NormView& norm) {
        const int tid = threadIdx.x;
        const bool normed = norm.kind >= 0;
        const float* gp = normed ? norm.gamma : xp;
        const float* bp = (normed && norm.beta) ? norm.beta : xp;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const int e = 4 * (tid + kBlock * i);
            const int ec = e < K ? e : K - 4;
            x[i] = *(const float4*)(xp + ec);
            g[i] = *(const float4*)(gp + ec);
            b[i] = *(const float4*)(bp + ec);
        }
    }
};

// The row slice of this thread, normalized when norm.kind >= 0 (in v; in[i]
// marks float4 slots inside the row, the others are zero).  The block
// reductions run in a fixed order (decoder.cpp:706-727).
//
// With `seq` (a K-float LDS buffer) and norm.sequential, the mean and square
// sums are those of the CPU's norm(): every thread writes its columns' terms
// to seq and one lane adds them in column order.
template <int V>
__device__ __forceinline__ void block_norm(RowSlice<V>& r, int K, const NormView& norm, float* red, double* dred, float* seq,
                           float4 (&v)[V], bool (&in)[V]) {
    const int tid = threadIdx.x;
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < V; ++i) {
        in[i] = 4 * (tid + kBlock * i) < K;
        v[i] = in[i] ? r.x[i] : zero;
    }
    if (norm.kind >= 0 && seq && norm.sequential) {
        // terms into seq, one lane's sum in column order, broadcast through red
        auto column_sum = [&](auto term, bool in_double) {
#pragma unroll
            for (int i = 0; i < V; ++i)
                if (in[i]) *(float4*)(seq + 4 * (tid + kBlock * i)) = term(v[i]);
            __syncthreads();
            if (tid == 0) red[0] = in_double ? (float)sequential_sum_f64(seq, K) : sequential_sum(seq, K);
            __syncthreads();
            const float total = red[0];
            __syncthreads();   // seq and red are free again
            return total;
        };
        float mean = 0.0f;
        if (norm.kind == 1) mean = column_sum([](float4 x) { return x; }, false) / (float)K;
        const bool accurate = norm.kind == 0 && norm.accurate;
        const float square = column_sum(
            [&](float4 x) {
                if (!accurate) x = make_float4(x.x - mean, x.y - mean, x.z - mean, x.w - mean);
                return make_float4(x.x * x.x, x.y * x.y, x.z * x.z, x.w * x.w);
            },
            accurate);
        const float scale = 1.0f / sqrtf(square / (float)K + norm.epsilon);
        const bool use_beta = norm.beta != nullptr;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const float4 g = r.g[i], b = use_beta ? r.b[i] : zero;
            v[i].x = (v[i].x - mean) * scale * g.x + b.x;
            v[i].y = (v[i].y - mean) * scale * g.y + b.y;
            v[i].z = (v[i].z - mean) * scale * g.z + b.z;
            v[i].w = (v[i].w - mean) * scale * g.w + b.w;
            if (!in[i]) v[i] = zero;
        }
    } else if (norm.kind >= 0) {
        float mean = 0.0f;
        if (norm.kind == 1) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < V; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
            s = block_reduce<float>(s, red, [](float a, float b) { return a + b; }, wave_sum_f32);
            mean = s / (float)K;
        }
        float square;
        if (norm.kind == 0 && norm.accurate) {
            double s = 0.0;
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const float a = v[i].x * v[i].x, b = v[i].y * v[i].y, c = v[i].z * v[i].z, d = v[i].w * v[i].w;
                s += ((double)a + (double)b) + ((double)c + (double)d);
            }
            square = (float)block_reduce<double>(s, dred, [](double a, double b) { return a + b; }, wave_sum_f64);
        } else {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < V; ++i) {
                const float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
                const float t = (a * a + b * b) + (c * c + d * d);
                s += in[i] ? t : 0.0f;
            }
            square = block_reduce<float>(s, red, [](float a, float b) { return a + b; }, wave_sum_f32);
        }
        const float scale = 1.0f / sqrtf(square / (float)K + norm.epsilon);
        const bool use_beta = norm.beta != nullptr;
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const float4 g = r.g[i], b = use_beta ? r.b[i] : zero;
            v[i].x = (v[i].x - mean) * scale * g.x + b.x;
            v[i].y = (v[i].y - mean) * scale * g.y + b.y;
            v[i].z = (v[i].z - mean) * scale * g.z + b.z;
            v[i].w = (v[i].w - mean) * scale * g.w + b.w;
            if (!in[i]) v[i] = zero;
        }
    }
}

// Normalize (optionally) and quantize the row into lds_q; returns the
// per-token activation scale (decoder.cpp:706-727, 1028-1043).
template <int V>
__device__ float block_norm_quantize(RowSlice<V>& r, int K, const NormView& norm, int8_t* lds_q, float* red,
                                     double* dred, float* seq = nullptr) {
    const int tid = threadIdx.x;
    float4 v[V];
    bool in[V];
    block_norm<V>(r, K, norm, red, dred, seq, v, in);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i)
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    amax = block_reduce<float>(amax, red, [](float a, float b) { return fmaxf(a, b); }, wave_max_f32);
    const float sx = fmaxf(amax / 127.0f, 1e-12f);
    const float multiplier = 1.0f / sx;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int e = 4 * (tid + kBlock * i);
        if (in[i])
            *(uint32_t*)(lds_q + e) = pack4(quantize_one(v[i].x, multiplier), quantize_one(v[i].y, multiplier),
                                            quantize_one(v[i].z, multiplier), quantize_one(v[i].w, multiplier));
    }
    __syncthreads();
    return sx;
}

// Activation words of chunk c (E values) from the int8 row in LDS, arranged to
// line up with chunk_dot<BITS>'s weight words.
template <int BITS>
__device__ __forceinline__ void chunk_x(const int8_t* lds_q, int c, uint32_t* xw) {
    if constexpr (BITS == 8) {
        const uint4 v = *(const uint4*)(lds_q + c * 16);
        xw[0] = v.x; xw[1] = v.y; xw[2] = v.z; xw[3] = v.w;
    } else {
        const uint4 a = *(const uint4*)(lds_q + c * 32), b = *(const uint4*)(lds_q + c * 32 + 16);
        const uint32_t words[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            xw[2 * k] = even_bytes(words[2 * k], words[2 * k + 1]);
            xw[2 * k + 1] = odd_bytes(words[2 * k], words[2 * k + 1]);
        }
    }
}

// Rows handled together by wave `p` of a paired epilogue.
__device__ __forceinline__ void pair_rows(const PairEpilogue& e, int p, int& r0, int& r1) {
    if (e.mode == kPairGated) {
        r0 = p;
        r1 = e.width + p;
        return;
    }
    const int per_head = e.dim / 2, half = e.rotary / 2;
    const int hb = p / per_head, j = p % per_head;
    const bool rotated_head = hb < e.heads + e.kv_heads;
    if (rotated_head && j < half) {
        r0 = hb * e.dim + j;
        r1 = r0 + half;
    } else {
        const int base = rotated_head ? e.rotary : 0;
        r0 = hb * e.dim + base + 2 * (rotated_head ? j - half : j);
        r1 = r0 + 1;
    }
}

__device__ __forceinline__ float activate_value(int activation, float x) {
    // Decoder::Impl::activate (decoder.cpp:982-987)
    if (activation == 0) return x / (1.0f + expf(-x));
    if (activation == 1) return 0.5f * x * (1.0f + erff(x * 0.7071067811865475f));
    if (activation == 2) return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
    return x < 0.0f ? 0.0f : x;
}

// The activation with the CPU's libm expf in the SiLU (bit-equal to the CPU's).
__device__ __forceinline__ float activate_value_reference(int activation, float x) {
    if (activation == 0) return x / (1.0f + libm_expf(-x));
    return activate_value(activation, x);
}

// Final values (bias included) of rows r0 and r1 of a paired epilogue.
__device__ __forceinline__ void pair_store(const PairEpilogue& e, int r0, float v0, int r1, float v1) {
    if (e.mode == kPairGated) {
        e.act[r0] = v1 * (e.reference ? activate_value_reference(e.activation, v0) : activate_value(e.activation, v0));
        return;
    }
    const int position = e.position_ptr ? *e.position_ptr : e.position;
    const int hb = r0 / e.dim, i0 = r0 % e.dim, i1 = r1 % e.dim;
    const int half = e.rotary / 2;
    float* dst;
    if (hb < e.heads) dst = e.q_heads + (size_t)hb * e.dim;
    else if (hb < e.heads + e.kv_heads) dst = e.keys + ((size_t)(hb - e.heads) * e.capacity + position) * e.dim;
    else dst = e.values + ((size_t)(hb - e.heads - e.kv_heads) * e.capacity + position) * e.dim;
    if (hb < e.heads + e.kv_heads && i0 < half) {
        const float c = e.cosines[(size_t)position * half + i0], s = e.sines[(size_t)position * half + i0];
        dst[i0] = v0 * c - v1 * s;
        dst[i1] = v1 * c + v0 * s;
    } else {
        dst[i0] = v0;
        dst[i1] = v1;
    }
}

template <int BITS, int RPW, int MAXJ, int EPI, bool SEQ = false>
__global__ __launch_bounds__(kBlock) void gemv_int_fused_kernel(WeightView w, const float* __restrict__ x, NormView norm,
                                                               float* __restrict__ y, int epilogue,
                                                               int32_t* __restrict__ acc_out, PairEpilogue pe) {
    static_assert(EPI == kPairNone || RPW % 2 == 0, "paired epilogues compute pairs of rows");
    constexpr int E = BITS == 8 ? 16 : 32;          // weight values per 16-byte chunk
    __shared__ __align__(16) int8_t lds_q[kFusedMaxK];
    // the row's terms for sequential sums (K <= MAXJ * 64 * E columns)
    __shared__ __align__(16) float lds_seq[SEQ ? (MAXJ * kWave * E < kFusedMaxK ? MAXJ * kWave * E : kFusedMaxK) : 4];
    __shared__ float red[16];
    __shared__ double dred[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = w.cols, nch = K / E;
    const int wave_index = blockIdx.x * (kBlock / kWave) + wave;
    const int row_first = wave_index * RPW;
    int rows_of[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) rows_of[r] = row_first + r;
    if constexpr (EPI != kPairNone) {
        // RPW / 2 pairs per wave; pair i's rows go to rows_of[2i], rows_of[2i + 1]
        // (a pair past the last one keeps rows past w.rows: nothing is stored)
#pragma unroll
        for (int i = 0; i < RPW / 2; ++i)
            if (row_first + 2 * i < w.rows) pair_rows(pe, wave_index * (RPW / 2) + i, rows_of[2 * i], rows_of[2 * i + 1]);
    }

    // Small L2-resident operands first (row slice, norm parameters, this
    // wave's scales and biases), then the HBM weight stream: the prologue's
    // waits then never wait for weights.
    constexpr int V = MAXJ * E / 16;                 // float4 of the row per thread
    RowSlice<V> slice;
    slice.issue(x, K, norm);
    float sw[RPW], bw[RPW], yw[RPW];
    const float* bias_src = w.bias ? w.bias : w.scales;
    // residual epilogue: the hidden values this wave adds to (rows owned by this wave)
    const float* y_src = (EPI == kPairNone && epilogue == kAccumulate) ? y : w.scales;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = min(rows_of[r], w.rows - 1);
        sw[r] = w.scales[row];
        bw[r] = bias_src[row];
        yw[r] = y_src[row];
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 wv[RPW][MAXJ];
    const uint8_t* base = (const uint8_t*)w.data;
    const size_t row_bytes = (size_t)K * BITS / 8;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = min(rows_of[r], w.rows - 1);
        const uint4* rp = (const uint4*)(base + (size_t)row * row_bytes);
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) wv[r][j] = load_stream16(rp + min(lane + kWave * j, nch - 1));
    }
    __builtin_amdgcn_sched_barrier(0);
    // Chunks past the row end carry zero activations (below), so the clamped
    // duplicate weights they loaded add nothing.
    const float sx = block_norm_quantize<V>(slice, K, norm, lds_q, red, dred, SEQ ? lds_seq : nullptr);
    if (row_first >= w.rows) return;
    uint32_t xq[MAXJ][E / 4];
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int c = lane + kWave * j;
        if (c < nch) chunk_x<BITS>(lds_q, c, xq[j]);
        else
#pragma unroll
            for (int k = 0; k < E / 4; ++k) xq[j][k] = 0;
    }
    float vals[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        int acc = 0;
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) acc = chunk_dot<BITS>(wv[r][j], xq[j], acc);
        acc = wave_sum_i32(acc);
        const int row = rows_of[r];
        if (row < w.rows) {
            if (acc_out && lane == 0) acc_out[row] = acc;
            vals[r] = int_epilogue(acc, sx, sw[r]);
            if (!w.bias) bw[r] = 0.0f;
            if constexpr (EPI == kPairNone) {
                const float v = vals[r] + bw[r];
                if (lane == 0) y[row] = epilogue == kAccumulate ? yw[r] + v : v;
            }
        }
    }
    if constexpr (EPI != kPairNone) {
#pragma unroll
        for (int i = 0; i < RPW / 2; ++i)
            if (lane == 0 && row_first + 2 * i < w.rows)
                pair_store(pe, rows_of[2 * i], vals[2 * i] + bw[2 * i], rows_of[2 * i + 1], vals[2 * i + 1] + bw[2 * i + 1]);
    }
}

// --------------------------------------- W8A8/W4A8 GEMV, given int8 input ---
// Up to four tokens with activations already quantized (xq [T, K], xs [T]).
template <int BITS, int T, int RPW>
__global__ __launch_bounds__(kBlock) void gemv_int_kernel(WeightView w, const int8_t* __restrict__ xq,
                                                         const float* __restrict__ xs, float* __restrict__ y,
                                                         int epilogue, int32_t* __restrict__ acc_out) {
    constexpr int E = BITS == 8 ? 16 : 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = w.cols, nch = K / E;
    const int row_first = (blockIdx.x * (kBlock / kWave) + wave) * RPW;
    if (row_first >= w.rows) return;
    const uint8_t* base = (const uint8_t*)w.data;
    const size_t row_bytes = (size_t)K * BITS / 8;
    int acc[RPW][T];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[r][t] = 0;
    for (int c = lane; c < nch; c += kWave) {
        uint32_t xw[T][E / 4];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const uint4* xp = (const uint4*)(xq + (size_t)t * K + (size_t)c * E);
            if constexpr (BITS == 8) {
                const uint4 v = xp[0];
                xw[t][0] = v.x; xw[t][1] = v.y; xw[t][2] = v.z; xw[t][3] = v.w;
            } else {
                const uint4 a = xp[0], b = xp[1];
                const uint32_t words[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    xw[t][2 * k] = even_bytes(words[2 * k], words[2 * k + 1]);
                    xw[t][2 * k + 1] = odd_bytes(words[2 * k], words[2 * k + 1]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = min(row_first + r, w.rows - 1);
            const uint4 wv = load_stream16((const uint4*)(base + (size_t)row * row_bytes) + c);
#pragma unroll
            for (int t = 0; t < T; ++t) acc[r][t] = chunk_dot<BITS>(wv, xw[t], acc[r][t]);
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row_first + r;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int a = wave_sum_i32(acc[r][t]);
            if (lane == 0 && row < w.rows) {
                if (acc_out) acc_out[(size_t)t * w.rows + row] = a;
                store_out(y, (size_t)t * w.rows + row, int_epilogue(a, xs[t], w.scales[row]), bias_at(w, row), epilogue);
            }
        }
    }
}

// ------------------------------------------------ FP decode GEMV family ---
// FP32, BF16-source and weight-only INT8 / INT4 (W8A32, W4A32) for up to four
// tokens.  Quantized weights accumulate q * x per scale group and apply the
// group scale once per group, as the CPU kernels do; the summation order is
// the wave's, not the CPU's, so results agree to rounding.
template <int BITS, int T, int RPW>
__global__ __launch_bounds__(kBlock) void gemv_fp_kernel(WeightView w, const float* __restrict__ x,
                                                        float* __restrict__ y, int epilogue) {
    constexpr int E = 128 / BITS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = w.cols, nch = K / E;
    const int row_first = (blockIdx.x * (kBlock / kWave) + wave) * RPW;
    if (row_first >= w.rows) return;
    const uint8_t* base = (const uint8_t*)w.data;
    const size_t row_bytes = (size_t)K * BITS / 8;
    const int groups = (BITS == 8 || BITS == 4) ? K / w.group : 1;
    // Values of one chunk that share a scale: the whole chunk, or group-sized pieces.
    const int piece = (BITS == 8 || BITS == 4) ? min(E, w.group) : E;
    float acc[RPW][T];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[r][t] = 0.0f;
    for (int c = lane; c < nch; c += kWave) {
        float xv[T][E];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float4* xp = (const float4*)(x + (size_t)t * K + (size_t)c * E);
#pragma unroll
            for (int k = 0; k < E / 4; ++k) {
                const float4 v = xp[k];
                xv[t][4 * k] = v.x; xv[t][4 * k + 1] = v.y; xv[t][4 * k + 2] = v.z; xv[t][4 * k + 3] = v.w;
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = min(row_first + r, w.rows - 1);
            const uint4 wv = load_stream16((const uint4*)(base + (size_t)row * row_bytes) + c);
            const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
            // int4: value / 16 (the group scale is taken times 16 below)
            float wf[E];
            if constexpr (BITS == 4) {
#pragma unroll
                for (int q = 0; q < 4; ++q) int4_sixteenths(words[q], *(float(*)[8])(wf + 8 * q));
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    if constexpr (BITS == 32) wf[e] = __uint_as_float(words[e]);
                    else if constexpr (BITS == 16) wf[e] = bf16_to_f32((words[e / 2] >> (16 * (e & 1))) & 0xFFFFu);
                    else wf[e] = (float)(int)(int8_t)((words[e / 4] >> (8 * (e & 3))) & 0xFFu);
                }
            }
            constexpr float kScaleOf = BITS == 4 ? 16.0f : 1.0f;
            if constexpr (BITS == 32 || BITS == 16) {
#pragma unroll
                for (int t = 0; t < T; ++t)
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[r][t] = fmaf(wf[e], xv[t][e], acc[r][t]);
            } else if (piece == E) {
                // one scale group covers the chunk: unrolled, the same sums
                const float s = w.scales[(size_t)row * groups + (c * E) / w.group] * kScaleOf;
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    float part = 0.0f;
#pragma unroll
                    for (int e = 0; e < E; ++e) part = fmaf(wf[e], xv[t][e], part);
                    acc[r][t] = fmaf(part, s, acc[r][t]);
                }
            } else {
                for (int p0 = 0; p0 < E; p0 += piece) {
                    const float s = w.scales[(size_t)row * groups + (c * E + p0) / w.group] * kScaleOf;
#pragma unroll
                    for (int t = 0; t < T; ++t) {
                        float part = 0.0f;
                        for (int e = p0; e < p0 + piece; ++e) part = fmaf(wf[e], xv[t][e], part);
                        acc[r][t] = fmaf(part, s, acc[r][t]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row_first + r;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float a = wave_sum_f32(acc[r][t]);
            if (lane == 0 && row < w.rows) store_out(y, (size_t)t * w.rows + row, a, bias_at(w, row), epilogue);
        }
    }
}

// ---------------------------------- FP decode GEMV with the norm fused in ---
// One token of an FP32 / BF16 / weight-only INT8 / INT4 linear whose input is
// normalized first (the q|k|v and gate|up inputs): every block normalizes the
// row itself (block_norm, the fused integer GEMV's order) into LDS, so no
// separate norm launch or round trip through memory is needed; the weight
// chunks of the wave's rows are requested before the norm starts.  Per row
// the sums are gemv_fp_kernel's (lane-strided chunks, groups summed then
// scaled), then one wave sum.  Paired epilogues fuse RoPE with the KV append
// (q|k|v) or the gated activation (gate|up), as in the integer GEMV; a wave
// takes RPW / 2 consecutive pairs.  Each chunk's activations are read from
// LDS once and serve all of the wave's rows.
// Quantized weights need scale groups of whole 16-byte chunks.
template <int BITS, int RPW, int MAXJ, int EPI>
__global__ __launch_bounds__(kBlock) void gemv_fp_fused_kernel(WeightView w, const float* __restrict__ x,
                                                              NormView norm, float* __restrict__ y, int epilogue,
                                                              PairEpilogue pe) {
    constexpr bool kPaired = EPI == kPairRopeKv || EPI == kPairGated;
    static_assert(!kPaired || RPW % 2 == 0, "paired epilogues compute whole pairs");
    constexpr int E = 128 / BITS;                    // weight values per 16-byte chunk
    // float4 of the row per thread: enough for the widest row this MAXJ takes
    // (64 MAXJ chunks of E values), so short rows do not hold registers for
    // the longest
    constexpr int V = (MAXJ * E + 15) / 16 < kFusedMaxV ? (MAXJ * E + 15) / 16 : kFusedMaxV;
    __shared__ __align__(16) float lds_x[kFusedMaxK];
    __shared__ float red[16];
    __shared__ double dred[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = w.cols, nch = K / E;
    const int wave_index = blockIdx.x * (kBlock / kWave) + wave;
    const int row_first = wave_index * RPW;
    int rows_of[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) rows_of[r] = row_first + r;
    if constexpr (kPaired) {
        // pair q = wave_index * RPW / 2 + i exists while 2 q < rows
#pragma unroll
        for (int i = 0; i < RPW / 2; ++i)
            if (row_first + 2 * i < w.rows) pair_rows(pe, wave_index * (RPW / 2) + i, rows_of[2 * i], rows_of[2 * i + 1]);
    }
    RowSlice<V> slice;
    slice.issue(x, K, norm);
    const int groups = (BITS == 8 || BITS == 4) ? K / w.group : 1;
    uint4 wv[RPW][MAXJ];
    float ws[RPW][MAXJ];
    const uint8_t* base = (const uint8_t*)w.data;
    const size_t row_bytes = (size_t)K * BITS / 8;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = min(rows_of[r], w.rows - 1);
        const uint4* rp = (const uint4*)(base + (size_t)row * row_bytes);
#pragma unroll
        for (int j = 0; j < MAXJ; ++j) {
            const int c = min(lane + kWave * j, nch - 1);
            wv[r][j] = load_stream16(rp + c);
            // int4 sums run on value / 16: the scale is taken times 16
            if constexpr (BITS == 8 || BITS == 4)
                ws[r][j] = w.scales[(size_t)row * groups + (c * E) / w.group] * (BITS == 4 ? 16.0f : 1.0f);
        }
    }
    float4 v[V];
    bool in[V];
    block_norm<V>(slice, K, norm, red, dred, nullptr, v, in);
#pragma unroll
    for (int i = 0; i < V; ++i)
        if (in[i]) *(float4*)(lds_x + 4 * (threadIdx.x + kBlock * i)) = v[i];
    __syncthreads();
    if (row_first >= w.rows) return;
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int c = lane + kWave * j;
        if (c >= nch) continue;
        float xv[E];
#pragma unroll
        for (int k = 0; k < E / 4; ++k) {
            const float4 q = *(const float4*)(lds_x + c * E + 4 * k);
            xv[4 * k] = q.x; xv[4 * k + 1] = q.y; xv[4 * k + 2] = q.z; xv[4 * k + 3] = q.w;
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const uint32_t words[4] = {wv[r][j].x, wv[r][j].y, wv[r][j].z, wv[r][j].w};
            float wf[E];
            if constexpr (BITS == 4) {
#pragma unroll
                for (int q = 0; q < 4; ++q) int4_sixteenths(words[q], *(float(*)[8])(wf + 8 * q));
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    if constexpr (BITS == 32) wf[e] = __uint_as_float(words[e]);
                    else if constexpr (BITS == 16) wf[e] = bf16_to_f32((words[e / 2] >> (16 * (e & 1))) & 0xFFFFu);
                    else wf[e] = (float)(int)(int8_t)((words[e / 4] >> (8 * (e & 3))) & 0xFFu);
                }
            }
            float part = 0.0f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                if constexpr (BITS == 32 || BITS == 16) acc[r] = fmaf(wf[e], xv[e], acc[r]);
                else part = fmaf(wf[e], xv[e], part);
            }
            if constexpr (BITS == 8 || BITS == 4) acc[r] = fmaf(part, ws[r][j], acc[r]);
        }
    }
    float vals[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = rows_of[r];
        const float a = wave_sum_f32(acc[r]);
        vals[r] = row < w.rows ? a + bias_at(w, row) : 0.0f;
        if constexpr (EPI == kPairNone) {
            if (lane == 0 && row < w.rows) {
                const float prev = epilogue == kAccumulate ? y[row] : 0.0f;
                y[row] = epilogue == kAccumulate ? prev + vals[r] : vals[r];
            }
        } else if constexpr (EPI == kPairActivation) {
            if (lane == 0 && row < w.rows) y[row] = activate_value(pe.activation, vals[r]);
        }
    }
    if constexpr (kPaired) {
#pragma unroll
        for (int i = 0; i < RPW / 2; ++i)
            if (lane == 0 && row_first + 2 * i < w.rows)
                pair_store(pe, rows_of[2 * i], vals[2 * i], rows_of[2 * i + 1], vals[2 * i + 1]);
    }
}

// ------------------------------------------------------ generic linear ---
// res += ((float)acc * s_x) * s_w for one group: fused as quant_dot_avx and
// quant_tile_avx compile it (target avx2,fma; decoder.cpp:568, 614), or two
// roundings as in quant_vnni_tile (target avx2,avxvnni has no FMA; :699).
__device__ __forceinline__ float group_term(int acc, float sx, float sw, float res, int unfused) {
    const float term = (float)acc * sx;
    return unfused ? __fadd_rn(res, __fmul_rn(term, sw)) : fmaf(term, sw, res);
}

// Any shape and storage: one thread per (token, row), sequential over columns.
// Integer activations reproduce the CPU epilogue exactly, groups in order.
__global__ __launch_bounds__(kBlock) void linear_generic_kernel(WeightView w, const float* x, const int8_t* xq,
                                                               const float* xs, int tokens, int integer,
                                                               float* y, int epilogue, int32_t* acc_out,
                                                               int unfused) {
    const size_t index = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (index >= (size_t)tokens * w.rows) return;
    const int t = (int)(index / w.rows), row = (int)(index % w.rows);
    const int K = w.cols;
    float result = 0.0f;
    if (integer) {
        const int groups = K / w.group;
        for (int g = 0; g < groups; ++g) {
            int acc = 0;
            for (int c = g * w.group; c < (g + 1) * w.group; ++c) acc += weight_int(w, row, c) * (int)xq[(size_t)t * K + c];
            if (acc_out) acc_out[((size_t)t * w.rows + row) * groups + g] = acc;
            result = group_term(acc, xs[t], w.scales[(size_t)row * groups + g], result, unfused);
        }
    } else {
        for (int c = 0; c < K; ++c) result = fmaf(weight_value(w, row, c), x[(size_t)t * K + c], result);
    }
    store_out(y, (size_t)t * w.rows + row, result, bias_at(w, row), epilogue);
}

// ------------------------------------------------ W8A8 prefill: int8 MFMA ---
// Y[t, n] = sum_k Xq[t, k] W[n, k] with v_mfma_i32_16x16x64_i8.  A 64x64 block
// tile, four waves of 32x32 (2x2 MFMA tiles).  Lane l feeds row/column (l & 15)
// with 16 consecutive K bytes at offset 16 * (l >> 4) of each 64-wide K step,
// for both operands, so the exact integer sum does not depend on how the
// hardware orders K inside the instruction.  Accumulators are exact; the
// epilogue is the CPU path's per group (group_term).
__global__ __launch_bounds__(kBlock) void gemm_int8_kernel(WeightView w, const int8_t* __restrict__ xq,
                                                          const float* __restrict__ xs, int tokens,
                                                          float* __restrict__ y, int epilogue,
                                                          int32_t* __restrict__ acc_out, int unfused) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = w.cols, N = w.rows;
    const int tile_m = blockIdx.y * 64 + (wave >> 1) * 32;   // tokens
    const int tile_n = blockIdx.x * 64 + (wave & 1) * 32;    // weight rows
    const int li = lane & 15, lk = (lane >> 4) * 16;
    const int groups = K / w.group;
    const int steps_per_group = w.group / 64;
    v4i acc[2][2];
    float res[2][2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            acc[a][b] = v4i{0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) res[a][b][i] = 0.0f;
        }
    const int8_t* wbase = (const int8_t*)w.data;
    const int steps = K / 64;
    for (int s = 0; s < steps; ++s) {
        const int k = s * 64 + lk;
        v4i av[2], bv[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            const int t = tile_m + a * 16 + li;
            av[a] = t < tokens ? *(const v4i*)(xq + (size_t)t * K + k) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int n = tile_n + b * 16 + li;
            bv[b] = n < N ? __builtin_nontemporal_load((const v4i*)(wbase + (size_t)n * K + k)) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[a], bv[b], acc[a][b], 0, 0, 0);
        if ((s + 1) % steps_per_group == 0) {
            const int g = (s + 1) / steps_per_group - 1;
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const int n = tile_n + b * 16 + li;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int t = tile_m + a * 16 + (lane >> 4) * 4 + i;
                        if (t < tokens && n < N) {
                            if (acc_out) acc_out[((size_t)t * N + n) * groups + g] = acc[a][b][i];
                            res[a][b][i] = group_term(acc[a][b][i], xs[t], w.scales[(size_t)n * groups + g],
                                                      res[a][b][i], unfused);
                        }
                    }
                    acc[a][b] = v4i{0, 0, 0, 0};
                }
        }
    }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int n = tile_n + b * 16 + li;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = tile_m + a * 16 + (lane >> 4) * 4 + i;
                if (t < tokens && n < N) store_out(y, (size_t)t * N + n, res[a][b][i], bias_at(w, n), epilogue);
            }
        }
}

// ---------------------- W8A8 prefill, per-row scales: split-K epilogue ---
// The MFMA GEMM (gemm_w8a8.hip) stores each K split's exact int32 sums to
// partial[split][t][n]; this adds them in split order and applies the CPU
// path's epilogue, so results are bit-identical to an unsplit run.
__global__ __launch_bounds__(kBlock) void gemm_w8a8_split_epilogue(WeightView w, const float* __restrict__ xs,
                                                                  int tokens, const int32_t* __restrict__ partial,
                                                                  int splits, float* __restrict__ y, int epilogue,
                                                                  int32_t* __restrict__ acc_out) {
    const int N = w.rows;
    const size_t count = (size_t)tokens * N;
    for (size_t i = blockIdx.x * (size_t)kBlock + threadIdx.x; i < count; i += (size_t)gridDim.x * kBlock) {
        int acc = 0;
        for (int s = 0; s < splits; ++s) acc += partial[s * count + i];
        const int t = (int)(i / N), n = (int)(i % N);
        if (acc_out) acc_out[i] = acc;
        const float res = fmaf((float)acc * xs[t], w.scales[n], 0.0f);
        store_out(y, i, res, bias_at(w, n), epilogue);
    }
}

// gemm_w8a8_split_epilogue four outputs per thread (N % 4 == 0): 128-bit
// loads of each split's sums and of y.  Exact integer sums, the same
// epilogue per output: identical results.
__global__ __launch_bounds__(kBlock) void gemm_w8a8_split_epilogue4(WeightView w, const float* __restrict__ xs,
                                                                   int tokens, const int32_t* __restrict__ partial,
                                                                   int splits, float* __restrict__ y, int epilogue,
                                                                   int32_t* __restrict__ acc_out) {
    const int N = w.rows;
    const size_t count = (size_t)tokens * N;
    for (size_t i = 4 * (blockIdx.x * (size_t)kBlock + threadIdx.x); i < count; i += 4 * (size_t)gridDim.x * kBlock) {
        v4i acc = *(const v4i*)(partial + i);
        for (int s = 1; s < splits; ++s) acc += *(const v4i*)(partial + s * count + i);
        const int t = (int)(i / N), n = (int)(i % N);
        if (acc_out) *(v4i*)(acc_out + i) = acc;
        const float sx = xs[t];
        v4f prev = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        if (epilogue == kAccumulate) prev = *(const v4f*)(y + i);
        v4f out;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float v = fmaf((float)acc[j] * sx, w.scales[n + j], 0.0f) + bias_at(w, n + j);
            out[j] = epilogue == kAccumulate ? prev[j] + v : v;
        }
        *(v4f*)(y + i) = out;
    }
}

// ------------------------------------------------ FP prefill: f32 MFMA ---
// Y[t, n] = sum_k X[t, k] W[n, k] with v_mfma_f32_16x16x4_f32; weights of any
// storage are widened (BF16) or dequantized (INT8 / INT4) as they are loaded.
// Each lane loads four consecutive K values of its row and column and feeds
// them to four MFMAs, so operand K positions always agree between A and B.
template <int BITS>
__device__ __forceinline__ float4 load_w4(const WeightView& w, int n, int k) {
    // four consecutive values W[n, k..k+3], k a multiple of 4
    if constexpr (BITS == 32) {
        return *(const float4*)((const float*)w.data + (size_t)n * w.cols + k);
    } else if constexpr (BITS == 16) {
        const uint2 v = *(const uint2*)((const uint16_t*)w.data + (size_t)n * w.cols + k);
        return make_float4(bf16_to_f32(v.x & 0xFFFFu), bf16_to_f32(v.x >> 16), bf16_to_f32(v.y & 0xFFFFu),
                           bf16_to_f32(v.y >> 16));
    } else {
        float f[4];
        const int groups = w.cols / w.group;
        if constexpr (BITS == 8) {
            const uint32_t v = *(const uint32_t*)((const int8_t*)w.data + (size_t)n * w.cols + k);
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = (float)(int)(int8_t)((v >> (8 * e)) & 0xFFu);
        } else {
            const uint16_t v = *(const uint16_t*)((const uint8_t*)w.data + ((size_t)n * w.cols + k) / 2);
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = (float)nibble((v >> (8 * (e / 2))) & 0xFFu, e & 1);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = f[e] * w.scales[(size_t)n * groups + (k + e) / w.group];
        return make_float4(f[0], f[1], f[2], f[3]);
    }
}

template <int BITS>
__global__ __launch_bounds__(kBlock) void gemm_f32_kernel(WeightView w, const float* __restrict__ x, int tokens,
                                                         float* __restrict__ y, int epilogue) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = w.cols, N = w.rows;
    const int tile_m = blockIdx.y * 64 + (wave >> 1) * 32;
    const int tile_n = blockIdx.x * 64 + (wave & 1) * 32;
    const int li = lane & 15, lk = (lane >> 4) * 4;
    v4f acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < K; k0 += 16) {
        const int k = k0 + lk;
        float4 av[2], bv[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            const int t = tile_m + a * 16 + li;
            av[a] = (t < tokens && k < K) ? *(const float4*)(x + (size_t)t * K + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int n = tile_n + b * 16 + li;
            bv[b] = (n < N && k < K) ? load_w4<BITS>(w, n, k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a].x, bv[b].x, acc[a][b], 0, 0, 0);
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a].y, bv[b].y, acc[a][b], 0, 0, 0);
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a].z, bv[b].z, acc[a][b], 0, 0, 0);
                acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[a].w, bv[b].w, acc[a][b], 0, 0, 0);
            }
    }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int n = tile_n + b * 16 + li;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = tile_m + a * 16 + (lane >> 4) * 4 + i;
                if (t < tokens && n < N) store_out(y, (size_t)t * N + n, acc[a][b][i], bias_at(w, n), epilogue);
            }
        }
}

// --------------------------------------------------------- RoPE + KV ---
// rotary() + KV append (decoder.cpp:1259-1281, 1332-1343): head-major reorder,
// rotate-half of the first `rotary` values with host-built cos/sin tables,
// a*c - b*s and b*c + a*s rounded separately as on the CPU.
__global__ void rope_kv_kernel(RopeKvCall p) {
    const int t = blockIdx.y;
    const int total_heads = p.heads + 2 * p.kv_heads;
    const int item = blockIdx.x * blockDim.x + threadIdx.x;   // over total_heads * dim
    if (item >= total_heads * p.dim) return;
    const int hh = item / p.dim, i = item % p.dim;
    const int half = p.rotary / 2;
    const float* row = p.qkv + (size_t)t * p.ld;
    const int pos = (p.position_ptr ? *p.position_ptr : p.position) + t;
    float* dst;
    const float* src;
    if (hh < p.heads) {
        src = row + p.q_offset + hh * p.dim;
        dst = p.q_heads + ((size_t)hh * p.tokens + t) * p.dim;
    } else if (hh < p.heads + p.kv_heads) {
        const int kh = hh - p.heads;
        src = row + p.k_offset + kh * p.dim;
        dst = p.keys + ((size_t)kh * p.capacity + pos) * p.dim;
    } else {
        const int vh = hh - p.heads - p.kv_heads;
        dst = p.values + ((size_t)vh * p.capacity + pos) * p.dim;
        dst[i] = row[p.v_offset + vh * p.dim + i];
        return;
    }
    if (i < half) {
        const float c = p.cosines[(size_t)pos * half + i], s = p.sines[(size_t)pos * half + i];
        const float a = src[i], b = src[i + half];
        dst[i] = a * c - b * s;
        dst[i + half] = b * c + a * s;
    } else if (i >= p.rotary) {
        dst[i] = src[i];
    }
}

// ------------------------------------------------------------ attention ---
// Online-softmax GQA attention (kv head = h / (heads / kv_heads), by index;
// transformer.cpp:94-146).  Scores use the CPU's sequential dot order and
// (dot * scale) * scale; the softmax is rescaled per key block, so results
// agree with the CPU's max / exp / sum / divide to rounding.
// Grid: (heads, tokens, splits).  With splits > 1 (decode) each block writes
// (max, sum, o[dim]) for its key range to `partial`, merged by attention_merge.
constexpr int kKeysPerPass = 256;

__global__ __launch_bounds__(kBlock) void attention_kernel(AttentionCall p, int keys_per_split) {
    __shared__ float q_s[256];
    __shared__ float scores[kKeysPerPass];
    __shared__ float o_s[4][256];
    __shared__ float red[16];
    const int h = blockIdx.x, t = blockIdx.y, split = blockIdx.z;
    const int kvh = h / (p.heads / p.kv_heads);
    const int dim = p.dim;
    const int qpos = p.position + t;
    int begin = 0;
    const int end = qpos + 1;
    if (p.window && end > p.window) begin = end - p.window;
    const int s_begin = max(begin, split * keys_per_split);
    const int s_end = min(end, (split + 1) * keys_per_split);
    for (int d = threadIdx.x; d < dim; d += blockDim.x) q_s[d] = p.q_heads[((size_t)h * p.tokens + t) * dim + d];
    __syncthreads();
    const float* K = p.keys + (size_t)kvh * p.capacity * dim;
    const float* V = p.values + (size_t)kvh * p.capacity * dim;
    float m = -INFINITY, l = 0.0f;
    // thread owns output dims d = tid % 64 (+64, ...) for key lane kl = tid / 64
    const int dl = threadIdx.x & 63, kl = threadIdx.x >> 6;
    float o[4] = {0.f, 0.f, 0.f, 0.f};   // dims dl, dl+64, dl+128, dl+192
    for (int k0 = s_begin; k0 < s_end; k0 += kKeysPerPass) {
        const int n = min(kKeysPerPass, s_end - k0);
        float local_max = -INFINITY;
        if (threadIdx.x < n) {
            const float* krow = K + (size_t)(k0 + threadIdx.x) * dim;
            float sum = 0.0f;
            for (int d = 0; d < dim; ++d) sum = sum + q_s[d] * krow[d];
            const float sc = sum * p.scale * p.scale;
            scores[threadIdx.x] = sc;
            local_max = sc;
        }
        const float block_max = block_reduce<float>(local_max, red, [](float a, float b) { return fmaxf(a, b); },
                                                    wave_max_f32);
        const float m_new = fmaxf(m, block_max);
        const float alpha = m == -INFINITY ? 0.0f : expf(m - m_new);
        __syncthreads();
        float e = 0.0f;
        if (threadIdx.x < n) {
            e = expf(scores[threadIdx.x] - m_new);
            scores[threadIdx.x] = e;
        }
        const float block_sum = block_reduce<float>(e, red, [](float a, float b) { return a + b; }, wave_sum_f32);
        __syncthreads();
        l = l * alpha + block_sum;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] *= alpha;
        for (int kk = kl; kk < n; kk += 4) {
            const float pk = scores[kk];
            const float* vrow = V + (size_t)(k0 + kk) * dim;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = dl + 64 * j;
                if (d < dim) o[j] = fmaf(pk, vrow[d], o[j]);
            }
        }
        m = m_new;
        __syncthreads();
    }
    // combine the four key lanes
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int d = dl + 64 * j;
        if (d < dim) o_s[kl][d] = o[j];
    }
    __syncthreads();
    if (gridDim.z == 1) {
        float* out = p.out + ((size_t)t * p.heads + h) * dim;
        for (int d = threadIdx.x; d < dim; d += blockDim.x) {
            const float v = (o_s[0][d] + o_s[1][d]) + (o_s[2][d] + o_s[3][d]);
            out[d] = l > 0.0f ? v / l : 0.0f;
        }
    } else {
        float* part = p.partial + (((size_t)t * p.heads + h) * gridDim.z + split) * (dim + 2);
        if (threadIdx.x == 0) { part[0] = m; part[1] = l; }
        for (int d = threadIdx.x; d < dim; d += blockDim.x)
            part[2 + d] = (o_s[0][d] + o_s[1][d]) + (o_s[2][d] + o_s[3][d]);
    }
}

// ----------------------------------------- prefill attention: f32 MFMA ---
// Flash attention for head dim 64 (every supported decoder family).  A work
// item is one query head and 32 tokens; waves w + 2 s (w < 2, s <
// kPrefillSlices) own tokens t0 + 16w .. +15, wave w + 2 s the 16-key slices
// s, s + kPrefillSlices, ... of each key tile, each with its own online
// softmax; the states merge at the end (several waves per SIMD, so one's
// MFMAs overlap another's softmax).  Items are numbered token-tile-major, and
// block b runs item b, then item n - 1 - b: a causal prefill's short and long
// key ranges pair up, so every block does about the same work.  Key
// tiles of 64 keys are staged in LDS (K and V, rows padded to 68 floats: the
// MFMA operand reads then hit every bank twice, the minimum for 64 lanes),
// the next tile waiting in registers while this one is used.
//
// Per 16 keys a wave computes S^T = K Q^T with v_mfma_f32_16x16x4_f32 (lane l
// feeds key row l % 16 and query column l % 16 at dims 4c + l / 16), which
// leaves lane l with the scores of query l % 16 for keys 4 (l / 16) + r,
// r < 4: exactly the B operand of O^T += V^T P^T when that product takes the
// keys {4j + r} as its K dimension.  So P never leaves registers.  Softmax is
// online per query (max and sum exchanged between the four lanes of a query),
// scores are (q.k * scale) * scale and masked keys are -inf, as in
// transformer.cpp:112-143; the output is divided by the sum at the end.
constexpr int kPrefillQ = 32;        // tokens per work item
constexpr int kPrefillGroups = kPrefillQ / 16;
constexpr int kPrefillKeys = 64;     // keys per LDS tile
constexpr int kPrefillStride = 68;   // padded row of a K or V tile
constexpr int kPrefillSlices = 4;    // waves per 16-token group
constexpr int kPrefillThreads = kPrefillGroups * kWave * kPrefillSlices;
constexpr int kPrefillLoads = 1024 / kPrefillThreads;   // float4 of a 64 x 64 tile per thread
constexpr int kPrefillMerge = 18;    // merge record per lane: O^T (16), max, sum
constexpr int kPrefillLds = 2 * kPrefillKeys * kPrefillStride > (kPrefillSlices - 1) * kPrefillGroups * kWave * kPrefillMerge
                                ? 2 * kPrefillKeys * kPrefillStride
                                : (kPrefillSlices - 1) * kPrefillGroups * kWave * kPrefillMerge;

// One thread's share of a 64 x 64 K (and V) tile: float4 i, i + kPrefillThreads, ...
// Rows at or past `end` were never written (they may hold NaN, and a masked
// key still multiplies its V row by 0): they load row 0 and are stored as
// zeros.  (The loaded values are not touched until the store, so the loads
// stay in flight while the current tile is used.)
__device__ __forceinline__ void prefill_tile_load(const float* K, const float* V, int k0, int end,
                                                  v4f (&kr)[kPrefillLoads], v4f (&vr)[kPrefillLoads]) {
#pragma unroll
    for (int j = 0; j < kPrefillLoads; ++j) {
        const int f = threadIdx.x + kPrefillThreads * j, row = f / 16, col = 4 * (f % 16);
        const int key = k0 + row;
        const size_t at = (size_t)(key < end ? key : 0) * 64 + col;
        kr[j] = *(const v4f*)(K + at);
        vr[j] = *(const v4f*)(V + at);
    }
}
__device__ __forceinline__ void prefill_tile_store(float* ks, float* vs, const v4f (&kr)[kPrefillLoads],
                                                   const v4f (&vr)[kPrefillLoads], int k0, int end) {
#pragma unroll
    for (int j = 0; j < kPrefillLoads; ++j) {
        const int f = threadIdx.x + kPrefillThreads * j, row = f / 16, col = 4 * (f % 16);
        const bool ok = k0 + row < end;
        const v4f zero = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        *(v4f*)(ks + row * kPrefillStride + col) = ok ? kr[j] : zero;
        *(v4f*)(vs + row * kPrefillStride + col) = ok ? vr[j] : zero;
    }
}

// One work item: query head h, tokens t0 .. t0 + kPrefillQ - 1.  Starts and
// ends with a barrier, so items can follow each other on the same LDS.
__device__ __forceinline__ void attention_prefill_item(const AttentionCall& p, int h, int t0, float* lds) {
    float* ks = lds;
    float* vs = lds + kPrefillKeys * kPrefillStride;
    constexpr int dim = 64;
    constexpr int kMerge = kPrefillMerge;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int group = wave % kPrefillGroups, slice = wave / kPrefillGroups;   // token group, key slice
    const int li = lane & 15, lj = lane >> 4;
    const int kvh = h / (p.heads / p.kv_heads);
    const int tw = t0 + 16 * group;                   // this wave's first token
    const int q_tok = tw + li;                        // this lane's query (score columns)
    const int q_pos = p.position + q_tok;
    const bool q_live = q_tok < p.tokens;
    // Q^T operand: dims 4c + lj of query q_tok
    float qv[16];
#pragma unroll
    for (int c = 0; c < 16; ++c)
        qv[c] = q_live ? p.q_heads[((size_t)h * p.tokens + q_tok) * dim + 4 * c + lj] : 0.0f;
    // keys the block needs: [first, end)
    const int last_tok = min(t0 + kPrefillQ, p.tokens) - 1;
    const int end = p.position + last_tok + 1;
    int first = 0;
    if (p.window) first = max(0, p.position + t0 + 1 - p.window);
    first &= ~(kPrefillKeys - 1);
    const float* K = p.keys + (size_t)kvh * p.capacity * dim;
    const float* V = p.values + (size_t)kvh * p.capacity * dim;
    v4f kr[kPrefillLoads], vr[kPrefillLoads];
    prefill_tile_load(K, V, first, end, kr, vr);
    v4f o[4];   // O^T: dims 16 dc + 4 lj + i, query li
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) o[dc] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    const float scale = p.scale;
    for (int k0 = first; k0 < end; k0 += kPrefillKeys) {
        lds_barrier();     // the previous tile is no longer read (the next one's loads stay in flight)
        prefill_tile_store(ks, vs, kr, vr, k0, end);
        lds_barrier();
        if (k0 + kPrefillKeys < end) prefill_tile_load(K, V, k0 + kPrefillKeys, end, kr, vr);
        // the keys this wave can see in this tile
        const int wave_end = min(end, p.position + min(tw + 16, p.tokens));
        for (int sub = 16 * slice; sub < kPrefillKeys && k0 + sub < wave_end; sub += 16 * kPrefillSlices) {
            v4f sc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            const float* krow = ks + (sub + li) * kPrefillStride + lj;
            float kv[16];   // all of the chain's K operands first: one LDS wait, not eight
#pragma unroll
            for (int c = 0; c < 16; ++c) kv[c] = krow[4 * c];
            __builtin_amdgcn_sched_barrier(0);   // keep the reads batched ahead of the chain
#pragma unroll
            for (int c = 0; c < 16; ++c) sc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[c], qv[c], sc, 0, 0, 0);
            // the V operands of O^T += V^T P^T below, read while the softmax runs
            float vv[4][4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int dc = 0; dc < 4; ++dc) vv[r][dc] = vs[(sub + 4 * lj + r) * kPrefillStride + li + 16 * dc];
            __builtin_amdgcn_sched_barrier(0);
            // lane: query q_tok, keys k0 + sub + 4 lj + r
            float e[4];
            float tile_max = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = k0 + sub + 4 * lj + r;
                const bool ok = q_live && key <= q_pos && (p.window == 0 || key > q_pos - p.window);
                e[r] = ok ? sc[r] * scale * scale : -INFINITY;
                tile_max = fmaxf(tile_max, e[r]);
            }
            tile_max = max_xor16(tile_max);
            tile_max = max_xor32(tile_max);
            const float m_new = fmaxf(m, tile_max);
            const float alpha = m_new == -INFINITY ? 1.0f : expf(m - m_new);
            float tile_sum = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                e[r] = m_new == -INFINITY ? 0.0f : expf(e[r] - m_new);
                tile_sum += e[r];
            }
            tile_sum = add_xor16(tile_sum);
            tile_sum = add_xor32(tile_sum);
            l = l * alpha + tile_sum;
            m = m_new;
#pragma unroll
            for (int dc = 0; dc < 4; ++dc) o[dc] = o[dc] * alpha;
            // O^T += V^T P^T over keys {4 j + r}: lane supplies V[4 lj + r][16 dc + li]
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int dc = 0; dc < 4; ++dc)
                    o[dc] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[r][dc], e[r], o[dc], 0, 0, 0);
        }
    }
    // merge the other slices' states into slice 0's wave of the same tokens
    __syncthreads();             // the last tile is no longer read
    if (slice > 0) {
        float* dst = lds + (((slice - 1) * kPrefillGroups + group) * kWave + lane) * kMerge;
#pragma unroll
        for (int dc = 0; dc < 4; ++dc)
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[4 * dc + i] = o[dc][i];
        dst[16] = m;
        dst[17] = l;
    }
    __syncthreads();
    if (slice == 0) {
        float mt = m;
#pragma unroll
        for (int z = 1; z < kPrefillSlices; ++z)
            mt = fmaxf(mt, lds[(((z - 1) * kPrefillGroups + group) * kWave + lane) * kMerge + 16]);
        const float a0 = m == -INFINITY ? 0.0f : expf(m - mt);
        l = l * a0;
#pragma unroll
        for (int dc = 0; dc < 4; ++dc) o[dc] = o[dc] * a0;
#pragma unroll
        for (int z = 1; z < kPrefillSlices; ++z) {
            const float* src = lds + (((z - 1) * kPrefillGroups + group) * kWave + lane) * kMerge;
            const float a = src[16] == -INFINITY ? 0.0f : expf(src[16] - mt);
            l = l + src[17] * a;
#pragma unroll
            for (int dc = 0; dc < 4; ++dc)
#pragma unroll
                for (int i = 0; i < 4; ++i) o[dc][i] = o[dc][i] + src[4 * dc + i] * a;
        }
    }
    if (slice == 0 && q_live) {
        float* out = p.out + ((size_t)q_tok * p.heads + h) * dim;
#pragma unroll
        for (int dc = 0; dc < 4; ++dc) {
            const v4f v = l > 0.0f ? v4f{o[dc][0] / l, o[dc][1] / l, o[dc][2] / l, o[dc][3] / l}
                                   : v4f{0.0f, 0.0f, 0.0f, 0.0f};
            *(v4f*)(out + 16 * dc + 4 * lj) = v;
        }
    }
    __syncthreads();   // the merge records are read before the next item's tile lands
}

__global__ __launch_bounds__(kPrefillThreads) void attention_prefill_kernel(AttentionCall p, int items) {
    __shared__ float lds[kPrefillLds];
    const int first = blockIdx.x, second = items - 1 - (int)blockIdx.x;
    attention_prefill_item(p, first % p.heads, (first / p.heads) * kPrefillQ, lds);
    if (second > first) attention_prefill_item(p, second % p.heads, (second / p.heads) * kPrefillQ, lds);
}

__global__ void attention_merge_kernel(AttentionCall p, int splits) {
    const int h = blockIdx.x, t = blockIdx.y;
    const float* part = p.partial + ((size_t)t * p.heads + h) * splits * (p.dim + 2);
    float m = -INFINITY;
    for (int s = 0; s < splits; ++s) m = fmaxf(m, part[s * (p.dim + 2)]);
    float l = 0.0f;
    for (int s = 0; s < splits; ++s) {
        const float ms = part[s * (p.dim + 2)];
        if (ms != -INFINITY) l += part[s * (p.dim + 2) + 1] * expf(ms - m);
    }
    float* out = p.out + ((size_t)t * p.heads + h) * p.dim;
    for (int d = threadIdx.x; d < p.dim; d += blockDim.x) {
        float v = 0.0f;
        for (int s = 0; s < splits; ++s) {
            const float ms = part[s * (p.dim + 2)];
            if (ms != -INFINITY) v = fmaf(part[s * (p.dim + 2) + 2 + d], expf(ms - m), v);
        }
        out[d] = l > 0.0f ? v / l : 0.0f;
    }
}

// ------------------------------------------------- decode attention (GQA) ---
// One query token.  A block owns one KV head and a span of keys: it stages the
// K and V tiles of that span in LDS once (K rows padded by one float so lanes
// walking keys hit distinct banks) and serves every query head of the group
// from them (GQA by index, no repeat).  Each score is two interleaved fused
// chains over the head's dims, added at the end (the reference-order kernels
// keep the CPU's single sequential chain).  Each block writes its
// (max, sum, out[dim]) per head; the last block
// of a KV head to finish (device-scope counter, reset by that block) merges
// the spans of its heads, so no second launch is needed.
constexpr int kTileFloats = 4096;                // K (or V) tile: keys * dim floats
constexpr int kDecodeKeys = 64;                  // keys per decode block (<= one wave)

// Merge of the spans of head h (partials at part, `splits` entries).
__device__ __forceinline__ void merge_head_spans(const float* part, int splits, int dim, float* out, int lane) {
    const size_t stride = (size_t)dim + 2;
    float m = -INFINITY;
    for (int s2 = lane; s2 < splits; s2 += kWave) m = fmaxf(m, part[s2 * stride]);
    m = wave_max_f32(m);
    float l = 0.0f;
    for (int s2 = lane; s2 < splits; s2 += kWave) {
        const float ms = part[s2 * stride];
        l += ms == -INFINITY ? 0.0f : part[s2 * stride + 1] * expf(ms - m);
    }
    l = wave_sum_f32(l);
    for (int d = lane; d < dim; d += kWave) {
        float v = 0.0f;
#pragma unroll 8
        for (int s2 = 0; s2 < splits; ++s2) {
            const float ms = part[s2 * stride];
            const float w = ms == -INFINITY ? 0.0f : expf(ms - m);
            v = fmaf(part[s2 * stride + 2 + d], w, v);
        }
        out[d] = l > 0.0f ? v / l : 0.0f;
    }
}

// Decode attention: block = (KV head, span of <= 64 keys).  K and V tiles are
// staged in LDS once (K rows padded to dim + 4 floats) and serve every query
// head of the group (GQA by index).  Scores: lane = key, float4 reads, one
// accumulator per head; outputs: lane = dim, two heads per thread.  Each
// block writes (max, sum, out[dim]) per head; with `counters` the last span
// of a KV head merges in place, otherwise attention_merge_kernel does.
__global__ __launch_bounds__(kBlock) void attention_decode_kernel(AttentionCall p, int keys_per_split,
                                                                 unsigned* counters, bool direct) {
    __shared__ __align__(16) float k_s[kDecodeKeys * (256 + 4)];
    __shared__ __align__(16) float v_s[kTileFloats];
    __shared__ __align__(16) float q_s[16 * 256];
    __shared__ float e_s[16 * kDecodeKeys];
    __shared__ float m_s[16], l_s[16];
    __shared__ int last_s;
    const int kvh = blockIdx.x, split = blockIdx.y, splits = gridDim.y;
    const int group = p.heads / p.kv_heads;
    const int dim = p.dim, kstride = dim + 4;
    const int end = (p.position_ptr ? *p.position_ptr : p.position) + 1;
    const int begin = (p.window && end > p.window) ? end - p.window : 0;
    const int k0 = max(begin, split * keys_per_split);
    const int k1 = min(end, (split + 1) * keys_per_split);
    const int n = max(0, k1 - k0);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = 4 * threadIdx.x; i < group * dim; i += 4 * blockDim.x)
        *(float4*)(q_s + i) = *(const float4*)(p.q_heads + (size_t)(kvh * group) * dim + i);
    const float* K = p.keys + ((size_t)kvh * p.capacity + k0) * dim;
    const float* V = p.values + ((size_t)kvh * p.capacity + k0) * dim;
    const int floats = n * dim;
    if (n > 0) {
        // all loads first, then the LDS stores: no load waits on a store
        constexpr int kStage = kTileFloats / (4 * kBlock);
        float4 kr[kStage], vr[kStage];
#pragma unroll
        for (int j = 0; j < kStage; ++j) {
            const int i = min(4 * (threadIdx.x + kBlock * j), floats - 4);
            kr[j] = *(const float4*)(K + i);
            vr[j] = *(const float4*)(V + i);
        }
#pragma unroll
        for (int j = 0; j < kStage; ++j) {
            const int i = 4 * (threadIdx.x + kBlock * j);
            if (i < floats) {
                *(float4*)(k_s + (i / dim) * kstride + i % dim) = kr[j];
                *(float4*)(v_s + i) = vr[j];
            }
        }
    }
    __syncthreads();
    // scores: wave w scores heads g = w, w+4, ...; lane = key
    if (lane < n) {
        const float* kr = k_s + lane * kstride;
        for (int g = wave; g < group; g += kBlock / kWave) {
            const float* qr = q_s + g * dim;
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll 4
            for (int d = 0; d < dim; d += 8) {
                const float4 k4 = *(const float4*)(kr + d), q4 = *(const float4*)(qr + d);
                const float4 k5 = *(const float4*)(kr + d + 4), q5 = *(const float4*)(qr + d + 4);
                a0 = fmaf(q4.x, k4.x, a0); a0 = fmaf(q4.y, k4.y, a0); a0 = fmaf(q4.z, k4.z, a0); a0 = fmaf(q4.w, k4.w, a0);
                a1 = fmaf(q5.x, k5.x, a1); a1 = fmaf(q5.y, k5.y, a1); a1 = fmaf(q5.z, k5.z, a1); a1 = fmaf(q5.w, k5.w, a1);
            }
            e_s[g * kDecodeKeys + lane] = (a0 + a1) * p.scale * p.scale;
        }
    }
    __syncthreads();
    for (int g = wave; g < group; g += kBlock / kWave) {
        const float sc = lane < n ? e_s[g * kDecodeKeys + lane] : -INFINITY;
        const float m = wave_max_f32(sc);
        const float e = lane < n ? expf(sc - m) : 0.0f;
        if (lane < n) e_s[g * kDecodeKeys + lane] = e;
        const float l = wave_sum_f32(e);
        if (lane == 0) { m_s[g] = n ? m : -INFINITY; l_s[g] = l; }
    }
    __syncthreads();
    const size_t stride = (size_t)dim + 2;
    for (int d = lane; d < dim; d += kWave) {
        for (int g = wave; g < group; g += 2 * (kBlock / kWave)) {
            const int g2 = g + kBlock / kWave;
            const bool two = g2 < group;
            const float* e0 = e_s + g * kDecodeKeys;
            const float* e1 = e_s + (two ? g2 : g) * kDecodeKeys;
            float o0 = 0.0f, o1 = 0.0f;
#pragma unroll 4
            for (int k = 0; k < n; ++k) {
                const float v = v_s[k * dim + d];
                o0 = fmaf(e0[k], v, o0);
                o1 = fmaf(e1[k], v, o1);
            }
            if (direct) {
                // a single span: the merge would weigh it by exp(0) = 1, so
                // its output is o / l, written here
                const float l0 = l_s[g];
                p.out[(size_t)(kvh * group + g) * dim + d] = l0 > 0.0f ? o0 / l0 : 0.0f;
                if (two) {
                    const float l1 = l_s[g2];
                    p.out[(size_t)(kvh * group + g2) * dim + d] = l1 > 0.0f ? o1 / l1 : 0.0f;
                }
                continue;
            }
            float* part = p.partial + ((size_t)(kvh * group + g) * splits + split) * stride;
            part[2 + d] = o0;
            if (d == 0) { part[0] = m_s[g]; part[1] = l_s[g]; }
            if (two) {
                float* part2 = p.partial + ((size_t)(kvh * group + g2) * splits + split) * stride;
                part2[2 + d] = o1;
                if (d == 0) { part2[0] = m_s[g2]; part2[1] = l_s[g2]; }
            }
        }
    }
    if (!counters) return;
    // Publish this span, count it; the last span of this KV head merges.
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned done = __hip_atomic_fetch_add(counters + kvh, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last_s = done == (unsigned)(splits - 1);
        if (last_s) __hip_atomic_store(counters + kvh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last_s) return;
    __threadfence();
    for (int g = wave; g < group; g += kBlock / kWave) {
        const int h = kvh * group + g;
        merge_head_spans(p.partial + (size_t)h * splits * stride, splits, dim, p.out + (size_t)h * dim, lane);
    }
}

// Merge for decode spans written without in-kernel merging: one wave per head.
// Merge of one query head's span partials (max, sum, unnormalized output)
// by a block of 256 threads: the spans' weights exp(m_s - m) once per span
// into LDS, then 256 / dim groups of dim threads each sum every group-th
// span's outputs (many loads in flight per thread, not one chain of loads
// per output element), combined at the end.
constexpr int kMergeThreads = 256;
__global__ __launch_bounds__(kMergeThreads) void attention_merge_spans_kernel(AttentionCall p, int splits) {
    extern __shared__ float w_s[];                 // [splits]
    __shared__ float red[kMergeThreads / kWave];
    __shared__ float o_s[kMergeThreads];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int dim = p.dim;
    const size_t stride = (size_t)dim + 2;
    const float* part = p.partial + (size_t)h * splits * stride;
    float m = -INFINITY;
    for (int s2 = tid; s2 < splits; s2 += kMergeThreads) m = fmaxf(m, part[s2 * stride]);
    m = block_reduce<float>(m, red, [](float a, float b) { return fmaxf(a, b); }, wave_max_f32);
    float l = 0.0f;
    for (int s2 = tid; s2 < splits; s2 += kMergeThreads) {
        const float ms = part[s2 * stride];
        const float w = ms == -INFINITY ? 0.0f : expf(ms - m);
        w_s[s2] = w;
        l += part[s2 * stride + 1] * w;
    }
    l = block_reduce<float>(l, red, [](float a, float b) { return a + b; }, wave_sum_f32);
    __syncthreads();   // every weight is in LDS
    const int groups = dim <= kMergeThreads ? kMergeThreads / dim : 1;
    const int g = tid / dim, d = tid % dim;
    float v = 0.0f;
    if (g < groups) {
#pragma unroll 8
        for (int s2 = g; s2 < splits; s2 += groups) v = fmaf(part[s2 * stride + 2 + d], w_s[s2], v);
        o_s[tid] = v;
    }
    __syncthreads();
    for (int e = tid; e < dim; e += kMergeThreads) {
        float total = 0.0f;
        for (int k = 0; k < groups; ++k) total += o_s[k * dim + e];
        p.out[(size_t)h * dim + e] = l > 0.0f ? total / l : 0.0f;
    }
}

// ----------------------------------------------------- small elementwise ---
__device__ __forceinline__ float activate(int activation, float x) {
    // Decoder::Impl::activate (decoder.cpp:982-987)
    if (activation == 0) return x / (1.0f + expf(-x));
    if (activation == 1) return 0.5f * x * (1.0f + erff(x * 0.7071067811865475f));
    if (activation == 2) return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
    return x < 0.0f ? 0.0f : x;
}

__global__ void activation_kernel(const float* gate_up, int tokens, int width, int gated, int activation, float* act) {
    const size_t count = (size_t)tokens * width;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < count; i += (size_t)gridDim.x * blockDim.x) {
        const size_t t = i / width, j = i % width;
        if (gated) {
            const float g = gate_up[t * 2 * width + j], u = gate_up[t * 2 * width + width + j];
            act[i] = u * activate(activation, g);
        } else {
            act[i] = activate(activation, gate_up[i]);
        }
    }
}

// The MLP activation of a token row (as activation_kernel computes it) and
// its per-token int8 quantization (as quantize_kernel does it) in one pass.
__global__ __launch_bounds__(kBlock) void activation_quantize_kernel(const float* gate_up, int width, int gated,
                                                                    int activation, int8_t* q, float* scales) {
    __shared__ float scratch[16];
    const float* in = gate_up + (size_t)blockIdx.x * width * (gated ? 2 : 1);
    auto value = [&](int j) { return gated ? in[width + j] * activate(activation, in[j]) : activate(activation, in[j]); };
    float m = 0.0f;
    for (int j = threadIdx.x; j < width; j += blockDim.x) m = fmaxf(m, fabsf(value(j)));
    m = block_reduce<float>(m, scratch, [](float a, float b) { return fmaxf(a, b); }, wave_max_f32);
    const float s = fmaxf(m / 127.0f, 1e-12f);
    const float multiplier = 1.0f / s;
    if (threadIdx.x == 0) scales[blockIdx.x] = s;
    int8_t* out = q + (size_t)blockIdx.x * width;
    for (int j = threadIdx.x; j < width; j += blockDim.x) out[j] = (int8_t)quantize_one(value(j), multiplier);
}

// activation_quantize_kernel with the row held in registers (thread t of T
// owns columns t + k * T); each activation is computed once.  Elementwise
// values and an exact absmax: q and the scale are bit-identical whatever T is.
template <int K, int T>
__global__ __launch_bounds__(T) void activation_quantize_rows_kernel(const float* gate_up, int width, int gated,
                                                                         int activation, int8_t* q, float* scales) {
    __shared__ float scratch[16];
    const float* in = gate_up + (size_t)blockIdx.x * width * (gated ? 2 : 1);
    float a[K];
    if (gated) {
        float u[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int j = threadIdx.x + k * T;
            a[k] = j < width ? in[j] : 0.0f;
            u[k] = j < width ? in[width + j] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < K; ++k) a[k] = u[k] * activate(activation, a[k]);
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int j = threadIdx.x + k * T;
            a[k] = j < width ? in[j] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < K; ++k) a[k] = activate(activation, a[k]);
    }
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k)
        if (threadIdx.x + k * T < width) m = fmaxf(m, fabsf(a[k]));
    m = block_reduce<float>(m, scratch, [](float x, float y) { return fmaxf(x, y); }, wave_max_f32);
    const float s = fmaxf(m / 127.0f, 1e-12f);
    const float multiplier = 1.0f / s;
    if (threadIdx.x == 0) scales[blockIdx.x] = s;
    int8_t* out = q + (size_t)blockIdx.x * width;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int j = threadIdx.x + k * T;
        if (j < width) out[j] = (int8_t)quantize_one(a[k], multiplier);
    }
}

__global__ void residual_kernel(float* hidden, const float* a, const float* b, int count) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x)
        hidden[i] = hidden[i] + (a[i] + (b ? b[i] : 0.0f));
}

constexpr int kArgmaxThreads = 1024;
constexpr int kArgmaxMaxBlocks = 256;
__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* logits, int width, uint32_t* out,
                                                                uint32_t* host_out, int* position) {
    __shared__ float bv[kArgmaxThreads / kWave];
    __shared__ int bi[kArgmaxThreads / kWave];
    const float* row = logits + (size_t)blockIdx.x * width;
    float best = -INFINITY;
    int index = width;
    // ties resolve to the lowest index (std::max_element keeps the first maximum)
    auto take = [&](float v, int c) {
        if (index == width || v > best || (v == best && c < index)) { best = v; index = c; }
    };
    const bool vec = (width % 4 == 0) && ((reinterpret_cast<uintptr_t>(row) & 15) == 0);
    if (vec) {
        for (int c = 4 * threadIdx.x; c < width; c += 4 * blockDim.x) {
            const float4 v = *(const float4*)(row + c);
            take(v.x, c); take(v.y, c + 1); take(v.z, c + 2); take(v.w, c + 3);
        }
    } else {
        for (int c = threadIdx.x; c < width; c += blockDim.x) take(row[c], c);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, kWave);
        const int oi = __shfl_xor(index, o, kWave);
        if (oi != width && (index == width || ov > best || (ov == best && oi < index))) { best = ov; index = oi; }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { bv[wave] = best; bi[wave] = index; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w2 = 1; w2 < (int)(blockDim.x >> 6); ++w2)
            if (bi[w2] != width && (index == width || bv[w2] > best || (bv[w2] == best && bi[w2] < index))) {
                best = bv[w2];
                index = bi[w2];
            }
        out[blockIdx.x] = (uint32_t)index;
        if (host_out) host_out[blockIdx.x] = (uint32_t)index;
        if (position) *position += 1;
    }
}

// One row's argmax over many blocks: block b takes columns [b chunk,
// (b + 1) chunk) with argmax_kernel's rule (greater, or equal at a lower
// index) and stores its (value, index) in scratch[2 b], then one wave of
// argmax_combine_kernel combines the blocks' results in block order with the
// same rule, so the index is the first maximum as with one block.  (Two
// launches: a last-block combine needs agent-scope fences, which cost more.)
constexpr int kArgmaxChunkThreads = 256;
struct ArgmaxBest {
    float best = -INFINITY;
    int index;
    __device__ explicit ArgmaxBest(int width) : index(width) {}
    __device__ __forceinline__ void take(float v, int c, int width) {
        if (c != width && (index == width || v > best || (v == best && c < index))) { best = v; index = c; }
    }
};
__global__ __launch_bounds__(kArgmaxChunkThreads) void argmax_chunks_kernel(const float* logits, int width, int chunk,
                                                                           float* scratch) {
    __shared__ float bv[kArgmaxChunkThreads / kWave];
    __shared__ int bi[kArgmaxChunkThreads / kWave];
    const int c0 = blockIdx.x * chunk, c1 = min(width, c0 + chunk);
    ArgmaxBest r(width);
    for (int c = c0 + threadIdx.x; c < c1; c += kArgmaxChunkThreads) r.take(logits[c], c, width);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) r.take(__shfl_xor(r.best, o, kWave), __shfl_xor(r.index, o, kWave), width);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { bv[wave] = r.best; bi[wave] = r.index; }
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int w2 = 1; w2 < kArgmaxChunkThreads / kWave; ++w2) r.take(bv[w2], bi[w2], width);
    scratch[2 * blockIdx.x] = r.best;
    scratch[2 * blockIdx.x + 1] = __int_as_float(r.index);
}
__global__ __launch_bounds__(kWave) void argmax_combine_kernel(const float* scratch, int blocks, int width,
                                                             uint32_t* out, uint32_t* host_out, int* position) {
    // lane l takes blocks l, l + 64, ... in order, then the lanes combine in
    // lane order: every candidate meets the rule in block order
    ArgmaxBest r(width);
    for (int b = threadIdx.x; b < blocks; b += kWave) r.take(scratch[2 * b], __float_as_int(scratch[2 * b + 1]), width);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) r.take(__shfl_xor(r.best, o, kWave), __shfl_xor(r.index, o, kWave), width);
    if (threadIdx.x != 0) return;
    out[0] = (uint32_t)r.index;
    if (host_out) host_out[0] = (uint32_t)r.index;
    if (position) *position += 1;
}

int ceil_div(size_t a, size_t b) { return (int)((a + b - 1) / b); }

template <int BITS, int RPW, int EPI, bool SEQ>
void launch_fused_int_seq(const LinearCall& c, int jn, hipStream_t stream) {
    const int grid = ceil_div(c.w.rows, (kBlock / kWave) * RPW);
#define LEAF_FUSED(J) gemv_int_fused_kernel<BITS, RPW, J, EPI, SEQ><<<grid, kBlock, 0, stream>>>(c.w, c.x, c.norm, \
        c.y, c.epilogue, c.acc_out, c.pair)
    if (jn <= 1) LEAF_FUSED(1);
    else if (jn <= 2) LEAF_FUSED(2);
    else if (jn <= 4) LEAF_FUSED(4);
    else LEAF_FUSED(6);
#undef LEAF_FUSED
}

template <int BITS, int RPW, int EPI>
void launch_fused_int_rpw(const LinearCall& c, int jn, hipStream_t stream) {
    if (c.norm.kind >= 0 && c.norm.sequential) launch_fused_int_seq<BITS, RPW, EPI, true>(c, jn, stream);
    else launch_fused_int_seq<BITS, RPW, EPI, false>(c, jn, stream);
}

template <int BITS>
void launch_fused_int(const LinearCall& c, hipStream_t stream) {
    constexpr int E = BITS == 8 ? 16 : 32;
    const int nch = c.w.cols / E;
    const int jn = (nch + kWave - 1) / kWave;
    if (c.pair.mode == kPairRopeKv) return launch_fused_int_rpw<BITS, 2, kPairRopeKv>(c, jn, stream);
    if (c.pair.mode == kPairGated) {
        // A column-order norm sum is a long chain in every block: two pairs
        // per wave halve the blocks, so that a tall gate|up matrix runs in
        // one round of resident blocks.
        if (c.norm.kind >= 0 && c.norm.sequential && c.w.rows >= 8192 && jn <= 2)
            return launch_fused_int_seq<BITS, 4, kPairGated, true>(c, jn, stream);
        return launch_fused_int_rpw<BITS, 2, kPairGated>(c, jn, stream);
    }
    // Enough blocks to cover the CUs, and more rows per wave for tall matrices
    // so the per-block prologue is amortized.
    if (c.w.rows >= 8192 && jn <= 2) launch_fused_int_rpw<BITS, 4, kPairNone>(c, jn, stream);
    else if (c.w.rows >= 2048) launch_fused_int_rpw<BITS, 2, kPairNone>(c, jn, stream);
    else launch_fused_int_rpw<BITS, 1, kPairNone>(c, jn, stream);
}

template <int BITS, int RPW, int EPI>
void launch_fused_fp_rpw(const LinearCall& c, int jn, hipStream_t stream) {
    const int grid = ceil_div(c.w.rows, (kBlock / kWave) * RPW);
#define LEAF_FUSED_FP(J) gemv_fp_fused_kernel<BITS, RPW, J, EPI><<<grid, kBlock, 0, stream>>>(c.w, c.x, c.norm, c.y, \
        c.epilogue, c.pair)
    if (jn <= 1) LEAF_FUSED_FP(1);
    else if (jn <= 2) LEAF_FUSED_FP(2);
    else if (jn <= 4) LEAF_FUSED_FP(4);
    else if (jn <= 8) LEAF_FUSED_FP(8);
    else {
        if constexpr (RPW == 1) LEAF_FUSED_FP(16);   // long rows: one row per wave (launch_fused_fp)
    }
#undef LEAF_FUSED_FP
}

template <int BITS>
void launch_fused_fp(const LinearCall& c, hipStream_t stream) {
    constexpr int E = 128 / BITS;
    const int jn = (c.w.cols / E + kWave - 1) / kWave;
    // rows of 9-16 chunks per lane (fp_fuses: no pair epilogue): one per wave
    if (jn > 8) return launch_fused_fp_rpw<BITS, 1, kPairNone>(c, jn, stream);
    if (c.pair.mode == kPairRopeKv) return launch_fused_fp_rpw<BITS, 2, kPairRopeKv>(c, jn, stream);
    if (c.pair.mode == kPairActivation) return launch_fused_fp_rpw<BITS, 2, kPairActivation>(c, jn, stream);
    if (c.pair.mode == kPairGated) {
        // Tall int8 / int4 gate|up stacks (rows of few bytes): several pairs
        // per wave, so fewer blocks repeat the norm prologue, while the grid
        // still covers the CUs (>= 256 blocks) and the wave's weight chunks
        // fit its registers.  FP32 / BF16 rows keep one pair per wave: more
        // blocks keep more of their bytes in flight.
        if constexpr (BITS <= 8) {
            if (jn <= 2 && c.w.rows >= 8 * 4 * 256) return launch_fused_fp_rpw<BITS, 8, kPairGated>(c, jn, stream);
            if (jn <= 4 && c.w.rows >= 4 * 4 * 256) return launch_fused_fp_rpw<BITS, 4, kPairGated>(c, jn, stream);
        }
        return launch_fused_fp_rpw<BITS, 2, kPairGated>(c, jn, stream);
    }
    // tall int8 / int4 matrices: four or eight rows per wave (the row staged
    // in LDS by every block serves more weight bytes), when the grid still
    // covers the CUs and the chunks fit the wave's registers
    if constexpr (BITS == 8 || BITS == 4) {
        if (jn <= 2 && c.w.rows >= 8 * 4 * 2048) return launch_fused_fp_rpw<BITS, 8, kPairNone>(c, jn, stream);
        if (c.w.rows >= 4 * 4096) return launch_fused_fp_rpw<BITS, 4, kPairNone>(c, jn, stream);
    }
    launch_fused_fp_rpw<BITS, 2, kPairNone>(c, jn, stream);
}

template <int BITS, int T>
void launch_gemv_int_t(const LinearCall& c, const int8_t* xq, const float* xs, hipStream_t stream) {
    constexpr int RPW = 2;
    const int grid = ceil_div(c.w.rows, (kBlock / kWave) * RPW);
    gemv_int_kernel<BITS, T, RPW><<<grid, kBlock, 0, stream>>>(c.w, xq, xs, c.y, c.epilogue, c.acc_out);
}

template <int BITS>
void launch_gemv_int(const LinearCall& c, const int8_t* xq, const float* xs, hipStream_t stream) {
    switch (c.tokens) {
    case 1: launch_gemv_int_t<BITS, 1>(c, xq, xs, stream); break;
    case 2: launch_gemv_int_t<BITS, 2>(c, xq, xs, stream); break;
    case 3: launch_gemv_int_t<BITS, 3>(c, xq, xs, stream); break;
    default: launch_gemv_int_t<BITS, 4>(c, xq, xs, stream); break;
    }
}

template <int BITS, int T>
void launch_gemv_fp_t(const LinearCall& c, hipStream_t stream) {
    // A wave reads the whole activation row from L1 / L2 for its rows: int4 /
    // int8 rows are 4-8x shorter in bytes than the row they multiply, so a
    // wave takes four of them when the grid still covers the CUs.
    constexpr int RPW = (BITS <= 8) ? 4 : 2;
    const int rpw = (RPW == 4 && c.w.rows < 4 * 4096) ? 2 : RPW;
    const int grid = ceil_div(c.w.rows, (kBlock / kWave) * rpw);
    if (rpw == 4) gemv_fp_kernel<BITS, T, 4><<<grid, kBlock, 0, stream>>>(c.w, c.x, c.y, c.epilogue);
    else gemv_fp_kernel<BITS, T, 2><<<grid, kBlock, 0, stream>>>(c.w, c.x, c.y, c.epilogue);
}

template <int BITS>
void launch_gemv_fp(const LinearCall& c, hipStream_t stream) {
    switch (c.tokens) {
    case 1: launch_gemv_fp_t<BITS, 1>(c, stream); break;
    case 2: launch_gemv_fp_t<BITS, 2>(c, stream); break;
    case 3: launch_gemv_fp_t<BITS, 3>(c, stream); break;
    default: launch_gemv_fp_t<BITS, 4>(c, stream); break;
    }
}

}  // namespace

// --------------------------------------------------------------- launchers ---
void launch_embedding(const WeightView& table, const WeightView* positions, const uint32_t* ids, int tokens,
                      int position_base, float scale, float* hidden, hipStream_t stream, const int* position_ptr) {
    WeightView none;
    embedding_kernel<<<tokens, kBlock, 0, stream>>>(table, positions ? *positions : none, positions != nullptr, ids,
                                                    position_base, scale, hidden, position_ptr);
}

void launch_norm(const float* x, int rows, int width, const NormView& norm, float* y, hipStream_t stream,
                 int rows_per_group, size_t group_stride) {
    norm_kernel<<<rows, kWideRow, 0, stream>>>(x, width, norm, y, rows_per_group, group_stride);
}

void launch_quantize(const float* x, int rows, int width, int8_t* q, float* scales, hipStream_t stream) {
    switch (wide_row_registers(width)) {
#define LEAF_ROWS(K) case K: quantize_rows_kernel<K, kWideRow><<<rows, kWideRow, 0, stream>>>(x, width, q, scales); break;
        LEAF_ROWS(1) LEAF_ROWS(2) LEAF_ROWS(3) LEAF_ROWS(4) LEAF_ROWS(6) LEAF_ROWS(8)
#undef LEAF_ROWS
        default: quantize_kernel<<<rows, kBlock, 0, stream>>>(x, width, q, scales);
    }
}

void launch_norm_quantize(const float* x, int rows, int width, const NormView& norm, int8_t* q, float* scales,
                          hipStream_t stream) {
    switch (wide_row_registers(width)) {
#define LEAF_ROWS(K) case K: norm_quantize_rows_kernel<K><<<rows, kWideRow, 0, stream>>>(x, width, norm, q, scales); break;
        LEAF_ROWS(1) LEAF_ROWS(2) LEAF_ROWS(3) LEAF_ROWS(4) LEAF_ROWS(6) LEAF_ROWS(8)
#undef LEAF_ROWS
        default: norm_quantize_kernel<<<rows, kWideRow, 0, stream>>>(x, width, norm, q, scales);
    }
}

void launch_activation_quantize(const float* gate_up, int tokens, int width, int gated, int activation, int8_t* q,
                                float* scales, hipStream_t stream) {
    switch (wide_row_registers(width)) {
#define LEAF_ROWS(K)                                                                                               \
    case K:                                                                                                        \
        activation_quantize_rows_kernel<K, kWideRow><<<tokens, kWideRow, 0, stream>>>(gate_up, width, gated,       \
                                                                                     activation, q, scales);       \
        break;
        LEAF_ROWS(1) LEAF_ROWS(2) LEAF_ROWS(3) LEAF_ROWS(4) LEAF_ROWS(6) LEAF_ROWS(8)
#undef LEAF_ROWS
        default: activation_quantize_kernel<<<tokens, kBlock, 0, stream>>>(gate_up, width, gated, activation, q, scales);
    }
}

void launch_scale_columns(const float* x, int rows, int width, const float* factors, float* y, hipStream_t stream) {
    const size_t count = (size_t)rows * width;
    scale_columns_kernel<<<std::min(ceil_div(count, kBlock), 4096), kBlock, 0, stream>>>(x, width, count, factors, y);
}

// The single-token FP GEMV with the norm (and a paired epilogue) fused in:
// whole 16-byte chunks, at most 8 per lane (16 without a pair epilogue),
// scale groups of whole chunks.
bool fp_fuses(const LinearCall& c) {
    const WeightView& w = c.w;
    if (c.integer_activations || c.tokens != 1 || !c.x || c.xq) return false;
    if (w.bits != 32 && w.bits != 16 && w.bits != 8 && w.bits != 4) return false;
    const int E = 128 / w.bits;
    const bool quantized = w.bits == 8 || w.bits == 4;
    const int max_chunks = (c.pair.mode == kPairNone ? 16 : 8) * kWave;
    return w.cols % E == 0 && w.cols <= kFusedMaxK && w.cols / E <= max_chunks && (!quantized || w.group % E == 0) &&
           (c.force_path == 0 || c.force_path == 1) && (reinterpret_cast<uintptr_t>(c.x) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(w.data) & 15) == 0 &&
           (c.pair.mode == kPairNone || c.pair.mode == kPairActivation || w.rows % 2 == 0);
}

bool linear_fuses(const LinearCall& c) {
    const WeightView& w = c.w;
    const int E8 = w.bits == 8 ? 16 : 32;
    if (!c.integer_activations) return fp_fuses(c);
    return (w.bits == 8 || w.bits == 4) && c.tokens == 1 && c.x && !c.xq && c.pair.mode != kPairActivation &&
           w.group == w.cols && w.cols % E8 == 0 && w.cols <= kFusedMaxK &&
           (c.force_path == 0 || c.force_path == 1) && (reinterpret_cast<uintptr_t>(c.x) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(w.data) & 15) == 0 && (c.pair.mode == kPairNone || w.rows % 2 == 0);
}

int launch_linear(const LinearCall& call, hipStream_t stream) {
    LinearCall c = call;
    const WeightView& w = c.w;
    if (c.pair.mode != kPairNone && !linear_fuses(c)) return -1;
    if (c.norm.kind >= 0) {
        // Only the single-token integer GEMV normalizes inside the kernel;
        // everywhere else the rows are normalized first into norm_scratch.
        const bool fusable = linear_fuses(c);
        if (!fusable) {
            if (!c.norm_scratch || !c.x) return -1;
            if (c.norm.sequential) {
                if (!launch_norm_reference_order(c.x, c.tokens, w.cols, c.norm, c.norm_scratch, stream)) return -1;
            } else {
                launch_norm(c.x, c.tokens, w.cols, c.norm, c.norm_scratch, stream);
            }
            c.x = c.norm_scratch;
            c.norm = NormView();
        }
    }
    const int K = w.cols;
    const bool quantized = w.bits == 8 || w.bits == 4;
    const int E = 128 / w.bits;
    // 128-bit loads need 16-byte aligned rows and inputs; anything else runs generic.
    auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool chunked = K % E == 0 && aligned(w.data) && (!c.x || aligned(c.x)) && (!c.xq || aligned(c.xq));
    if (c.integer_activations) {
        const bool per_row = w.group == K;
        const bool fast = per_row && chunked;
        int path = c.force_path;
        if (!path) path = (fast && c.tokens <= 4) ? 1 : (w.bits == 8 && c.tokens > 4 && K % 64 == 0 && w.group % 64 == 0) ? 3 : 2;
        if (path == 1 && !(fast && c.tokens <= 4)) path = 2;
        if (path == 3 && !(w.bits == 8 && K % 64 == 0 && w.group % 64 == 0 && aligned(w.data))) path = 2;
        const int E8 = w.bits == 8 ? 16 : 32;
        if (path == 1 && c.tokens == 1 && c.x && !c.xq && K <= kFusedMaxK) {
            if (w.bits == 8) launch_fused_int<8>(c, stream); else launch_fused_int<4>(c, stream);
            return 1;
        }
        const int8_t* xq = c.xq;
        const float* xs = c.xs;
        if (!xq) {
            if (!c.xq_scratch || !c.xs_scratch || !c.x) return -1;
            const float* src = c.x;
            if (c.norm.kind >= 0) return -1;   // callers normalize beforehand on this path
            launch_quantize(src, c.tokens, K, c.xq_scratch, c.xs_scratch, stream);
            xq = c.xq_scratch;
            xs = c.xs_scratch;
        }
        if (path == 1) {
            if (w.bits == 8) launch_gemv_int<8>(c, xq, xs, stream); else launch_gemv_int<4>(c, xq, xs, stream);
            return 1;
        }
        if (path == 3 && w.group == K && gemm_w8a8_mfma_supported(K)) {
            const GemmTiles tiles = gemm_w8a8_tiles(c.tokens, w.rows, K, c.split_scratch ? c.split_capacity : 0);
            int32_t* partial = tiles.splits > 1 ? c.split_scratch : nullptr;
            const int splits = tiles.splits;
            launch_gemm_w8a8_mfma((const int8_t*)w.data, w.scales, w.bias, xq, xs, c.tokens, w.rows, K, c.y,
                                  c.epilogue, c.acc_out, tiles, partial, stream);
            if (partial) {
                const bool vec = w.rows % 4 == 0 && (reinterpret_cast<uintptr_t>(c.y) & 15) == 0 &&
                                 (reinterpret_cast<uintptr_t>(partial) & 15) == 0 &&
                                 (reinterpret_cast<uintptr_t>(c.acc_out) & 15) == 0;
                if (vec)
                    gemm_w8a8_split_epilogue4<<<std::min(ceil_div((size_t)c.tokens * w.rows / 4, kBlock), 4096), kBlock,
                                                0, stream>>>(w, xs, c.tokens, partial, splits, c.y, c.epilogue,
                                                             c.acc_out);
                else
                    gemm_w8a8_split_epilogue<<<std::min(ceil_div((size_t)c.tokens * w.rows, kBlock), 4096), kBlock, 0,
                                               stream>>>(w, xs, c.tokens, partial, splits, c.y, c.epilogue,
                                                         c.acc_out);
            }
            return 3;
        }
        if (path == 3) {
            dim3 grid(ceil_div(w.rows, 64), ceil_div(c.tokens, 64));
            gemm_int8_kernel<<<grid, kBlock, 0, stream>>>(w, xq, xs, c.tokens, c.y, c.epilogue, c.acc_out,
                                                          c.unfused_group_sum && c.tokens > 1);
            return 3;
        }
        linear_generic_kernel<<<ceil_div((size_t)c.tokens * w.rows, kBlock), kBlock, 0, stream>>>(
            w, nullptr, xq, xs, c.tokens, 1, c.y, c.epilogue, c.acc_out, c.unfused_group_sum && c.tokens > 1);
        return 2;
    }
    if (fp_fuses(c)) {
        // every single-token FP GEMV it handles: all of a wave's weight chunks
        // in flight at once, the input row read once per block
        switch (w.bits) {
        case 32: launch_fused_fp<32>(c, stream); break;
        case 16: launch_fused_fp<16>(c, stream); break;
        case 8: launch_fused_fp<8>(c, stream); break;
        default: launch_fused_fp<4>(c, stream); break;
        }
        return 1;
    }
    if (c.norm.kind >= 0) return -1;
    const bool group_ok = !quantized || (w.group % E == 0) || (E % w.group == 0);
    int path = c.force_path;
    if (!path) path = (chunked && group_ok && c.tokens <= 4) ? 1 : (c.tokens > 4 && K % 4 == 0 && (!quantized || w.group % 4 == 0)) ? 3 : 2;
    if (path == 1 && !(chunked && group_ok && c.tokens <= 4)) path = 2;
    if (path == 3 && !(K % 4 == 0 && (!quantized || w.group % 4 == 0) && aligned(w.data) && aligned(c.x))) path = 2;
    if (path == 1) {
        switch (w.bits) {
        case 32: launch_gemv_fp<32>(c, stream); break;
        case 16: launch_gemv_fp<16>(c, stream); break;
        case 8: launch_gemv_fp<8>(c, stream); break;
        default: launch_gemv_fp<4>(c, stream); break;
        }
        return 1;
    }
    if (path == 3 && !c.force_path && gemm_f32_lds_supported(w, c.x)) {
        launch_gemm_f32_lds(w, c.x, c.tokens, c.y, c.epilogue, stream);
        return 3;
    }
    if (path == 3) {
        dim3 grid(ceil_div(w.rows, 64), ceil_div(c.tokens, 64));
        switch (w.bits) {
        case 32: gemm_f32_kernel<32><<<grid, kBlock, 0, stream>>>(w, c.x, c.tokens, c.y, c.epilogue); break;
        case 16: gemm_f32_kernel<16><<<grid, kBlock, 0, stream>>>(w, c.x, c.tokens, c.y, c.epilogue); break;
        case 8: gemm_f32_kernel<8><<<grid, kBlock, 0, stream>>>(w, c.x, c.tokens, c.y, c.epilogue); break;
        default: gemm_f32_kernel<4><<<grid, kBlock, 0, stream>>>(w, c.x, c.tokens, c.y, c.epilogue); break;
        }
        return 3;
    }
    linear_generic_kernel<<<ceil_div((size_t)c.tokens * w.rows, kBlock), kBlock, 0, stream>>>(
        w, c.x, nullptr, nullptr, c.tokens, 0, c.y, c.epilogue, nullptr, 0);
    return 2;
}

void launch_rope_kv(const RopeKvCall& call, hipStream_t stream) {
    const int items = (call.heads + 2 * call.kv_heads) * call.dim;
    dim3 grid(ceil_div(items, kBlock), call.tokens);
    rope_kv_kernel<<<grid, kBlock, 0, stream>>>(call);
}

bool launch_attention(const AttentionCall& call, hipStream_t stream) {
    const int total = call.position + call.tokens;
    const int group = call.heads / call.kv_heads;
    if (call.tokens == 1 && call.partial && attention_decode_supported(call.heads, call.kv_heads, call.dim)) {
        // decode: GQA-grouped tiles of keys per KV head, merged by the last tile
        const int per_split = std::min(kDecodeKeys, kTileFloats / call.dim);
        const int splits = call.spans ? call.spans : (total + per_split - 1) / per_split;
        if ((size_t)splits * call.heads * (call.dim + 2) <= (size_t)call.partial_capacity) {
            // A separate merge launch is cheaper here than merging in the last
            // block: that needs device-scope release/acquire fences, which
            // write back and invalidate L2 on every block (measured ~5 us/layer).
            // One span (a short context) writes the output itself.
            const bool direct = splits == 1;
            attention_decode_kernel<<<dim3(call.kv_heads, splits), kBlock, 0, stream>>>(call, per_split, nullptr,
                                                                                   direct);
            if (!direct)
                attention_merge_spans_kernel<<<call.heads, kMergeThreads, splits * sizeof(float), stream>>>(call,
                                                                                                        splits);
            return true;
        }
    }
    if (call.position_ptr) return false;
    int splits = 1, per_split = total;
    if (call.tokens == 1 && call.partial) {
        per_split = 256;
        splits = (total + per_split - 1) / per_split;
        while (splits > 1 && (size_t)splits * call.heads * (call.dim + 2) > (size_t)call.partial_capacity) {
            per_split *= 2;
            splits = (total + per_split - 1) / per_split;
        }
        if (splits == 1) per_split = total;
    }
    if (splits == 1 && call.tokens > 1 && call.dim == 64) {
        const int items = call.heads * ((call.tokens + kPrefillQ - 1) / kPrefillQ);
        attention_prefill_kernel<<<(items + 1) / 2, kPrefillThreads, 0, stream>>>(call, items);
        return true;
    }
    dim3 grid(call.heads, call.tokens, splits);
    attention_kernel<<<grid, kBlock, 0, stream>>>(call, per_split);
    if (splits > 1) attention_merge_kernel<<<dim3(call.heads, call.tokens), 64, 0, stream>>>(call, splits);
    return true;
}

void launch_activation(const float* gate_up, int tokens, int width, int gated, int activation, float* act,
                       hipStream_t stream) {
    const size_t count = (size_t)tokens * width;
    activation_kernel<<<std::min(ceil_div(count, kBlock), 8192), kBlock, 0, stream>>>(gate_up, tokens, width, gated,
                                                                                    activation, act);
}

void launch_residual(float* hidden, const float* a, const float* b, int count, hipStream_t stream) {
    residual_kernel<<<std::min(ceil_div(count, kBlock), 8192), kBlock, 0, stream>>>(hidden, a, b, count);
}

int argmax_scratch_floats() { return 2 * kArgmaxMaxBlocks; }

// Blocks of at least 1024 columns, at most kArgmaxMaxBlocks of them.
static void launch_argmax_chunks(const float* logits, int width, uint32_t* out, uint32_t* host_out, int* position,
                                 float* scratch, hipStream_t stream) {
    const int blocks = std::max(1, std::min(kArgmaxMaxBlocks, ceil_div(width, 1024)));
    const int chunk = ceil_div(width, blocks);
    argmax_chunks_kernel<<<blocks, kArgmaxChunkThreads, 0, stream>>>(logits, width, chunk, scratch);
    argmax_combine_kernel<<<1, kWave, 0, stream>>>(scratch, blocks, width, out, host_out, position);
}

void launch_argmax_advance(const float* logits, int width, uint32_t* next_id, uint32_t* host_out, int* position,
                           float* scratch, hipStream_t stream) {
    launch_argmax_chunks(logits, width, next_id, host_out, position, scratch, stream);
}

void launch_argmax_row(const float* logits, int width, uint32_t* out, float* scratch, hipStream_t stream) {
    launch_argmax_chunks(logits, width, out, nullptr, nullptr, scratch, stream);
}

bool attention_decode_supported(int heads, int kv_heads, int dim) {
    return kv_heads > 0 && heads % kv_heads == 0 && heads / kv_heads <= 16 && dim <= 256 && dim % 8 == 0;
}

int attention_decode_spans(int keys, int dim) {
    const int per_split = std::min(kDecodeKeys, kTileFloats / std::max(dim, 1));
    return (keys + per_split - 1) / per_split;
}

void launch_argmax(const float* logits, int rows, int width, uint32_t* out, hipStream_t stream) {
    argmax_kernel<<<rows, kArgmaxThreads, 0, stream>>>(logits, width, out, nullptr, nullptr);
}

}  // namespace leafhip
