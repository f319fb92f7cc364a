// mfma_peak: the matrix-core issue rate this device reaches.
//
//   mfma_peak [iterations]
//
// Every CU runs 16 waves; each wave issues `iterations` rounds of independent
// accumulator chains of one MFMA instruction (sixteen for the 16x16 shapes,
// eight for the 32x32 ones: fewer 16x16 chains leave the pipe waiting on each
// result, 8 chains measured 2.5 against 4.4 POPS for int8), operands held in
// registers, so nothing but the matrix cores limits the rate.  Prints one line
// per instruction: dense operations per second (2 m n k per instruction).
// The prefill GEMMs' utilisation is reported against these measured rates
// beside MI355X's datasheet peaks (int8 5.0 POPS, bf16 2.5 PFLOPS, f32
// 157.3 TFLOPS).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kChains = 16;

__global__ __launch_bounds__(256) void mfma_i8_kernel(int iterations, int* sink) {
    const v4i a = {(int)threadIdx.x, 1, 2, 3}, b = {3, 2, 1, (int)threadIdx.x};
    v4i acc[kChains] = {};
    for (int i = 0; i < iterations; ++i)
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[c], 0, 0, 0);
    int s = 0;
#pragma unroll
    for (int c = 0; c < kChains; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    if (s == 0x1234567) sink[0] = s;   // keeps the chains live
}

__global__ __launch_bounds__(256) void mfma_f32_kernel(int iterations, float* sink) {
    const float a = 1.0f + threadIdx.x * 1e-7f, b = 1.0f - threadIdx.x * 1e-7f;
    v4f acc[kChains] = {};
    for (int i = 0; i < iterations; ++i)
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[c], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChains; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    if (s == 1.2345f) sink[0] = s;
}

__global__ __launch_bounds__(256) void mfma_bf16_kernel(int iterations, float* sink) {
    v8bf a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = (__bf16)(1.0f + j * 0.125f);
        b[j] = (__bf16)(1.0f - threadIdx.x * 1e-3f);
    }
    v4f acc[kChains] = {};
    for (int i = 0; i < iterations; ++i)
#pragma unroll
        for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChains; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    if (s == 1.2345f) sink[0] = s;
}

typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void mfma_i8_32_kernel(int iterations, int* sink) {
    const v4i a = {(int)threadIdx.x, 1, 2, 3}, b = {3, 2, 1, (int)threadIdx.x};
    v16i acc[kChains / 2] = {};
    for (int i = 0; i < iterations; ++i)
#pragma unroll
        for (int c = 0; c < kChains / 2; ++c) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
    int s = 0;
#pragma unroll
    for (int c = 0; c < kChains / 2; ++c) s += acc[c][0] + acc[c][15];
    if (s == 0x1234567) sink[0] = s;
}

__global__ __launch_bounds__(256) void mfma_bf16_32_kernel(int iterations, float* sink) {
    v8bf a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = (__bf16)(1.0f + j * 0.125f);
        b[j] = (__bf16)(1.0f - threadIdx.x * 1e-3f);
    }
    v16f acc[kChains / 2] = {};
    for (int i = 0; i < iterations; ++i)
#pragma unroll
        for (int c = 0; c < kChains / 2; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kChains / 2; ++c) s += acc[c][0] + acc[c][15];
    if (s == 1.2345f) sink[0] = s;
}

bool ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    std::fprintf(stderr, "mfma_peak: %s: %s\n", what, hipGetErrorString(e));
    return false;
}

template <typename Launch>
bool measure(const char* name, double ops_per_instruction, int iterations, int blocks, Launch launch) {
    hipEvent_t start, stop;
    if (!ok(hipEventCreate(&start), "event") || !ok(hipEventCreate(&stop), "event")) return false;
    launch(iterations / 10);   // warm up
    if (!ok(hipGetLastError(), "launch") || !ok(hipDeviceSynchronize(), "sync")) return false;
    if (!ok(hipEventRecord(start, 0), "record")) return false;
    launch(iterations);
    if (!ok(hipGetLastError(), "launch") || !ok(hipEventRecord(stop, 0), "record") ||
        !ok(hipEventSynchronize(stop), "sync"))
        return false;
    float ms = 0;
    if (!ok(hipEventElapsedTime(&ms, start, stop), "elapsed")) return false;
    const double waves = double(blocks) * 4;
    const double ops = waves * iterations * kChains * ops_per_instruction;   // 32x32 kernels: half the chains, twice the ops
    std::printf("mfma_peak: %s %.1f T/s (%d blocks x 4 waves, %d x %d instructions per wave, %.3f ms)\n", name,
                ops / ms / 1e9, blocks, iterations, kChains, ms);
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    return true;
}

}  // namespace

int main(int argc, char** argv) {
    const int iterations = argc > 1 ? std::atoi(argv[1]) : 20000;
    if (iterations < 10 || iterations > 10000000) {
        std::fprintf(stderr, "usage: mfma_peak [iterations 10..10000000]\n");
        return 2;
    }
    int cus = 0;
    if (!ok(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0), "attribute")) return 1;
    const int blocks = cus * 4;   // 16 waves per CU, 4 per SIMD
    void* sink = nullptr;
    if (!ok(hipMalloc(&sink, 64), "hipMalloc")) return 1;
    bool good = measure("int8 v_mfma_i32_16x16x64_i8", 2.0 * 16 * 16 * 64, iterations, blocks, [&](int n) {
        mfma_i8_kernel<<<blocks, 256>>>(n, static_cast<int*>(sink));
    });
    good = good && measure("int8 v_mfma_i32_32x32x32_i8", 2.0 * 32 * 32 * 32 / 2, iterations, blocks, [&](int n) {
        mfma_i8_32_kernel<<<blocks, 256>>>(n, static_cast<int*>(sink));
    });
    good = good && measure("bf16 v_mfma_f32_32x32x16_bf16", 2.0 * 32 * 32 * 16 / 2, iterations, blocks, [&](int n) {
        mfma_bf16_32_kernel<<<blocks, 256>>>(n, static_cast<float*>(sink));
    });
    good = good && measure("bf16 v_mfma_f32_16x16x32_bf16", 2.0 * 16 * 16 * 32, iterations, blocks, [&](int n) {
        mfma_bf16_kernel<<<blocks, 256>>>(n, static_cast<float*>(sink));
    });
    good = good && measure("f32 v_mfma_f32_16x16x4_f32", 2.0 * 16 * 16 * 4, iterations, blocks, [&](int n) {
        mfma_f32_kernel<<<blocks, 256>>>(n, static_cast<float*>(sink));
    });
    (void)hipFree(sink);
    return good ? 0 : 1;
}
