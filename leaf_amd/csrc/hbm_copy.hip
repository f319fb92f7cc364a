// hbm_copy: a plain device-to-device copy of a known size.
//
//   hbm_copy [MiB] [repeats]
//
// It is the reference kernel for the hardware byte counters: a copy of B
// bytes reads B and writes B, so rocprofv3's FETCH_SIZE / WRITE_SIZE of
// hbm_copy_kernel give the factor that turns those counters into bytes for
// any other kernel profiled the same way.  It also prints the copy rate
// (read + write bytes per second) and, from a second kernel, the rate of
// reading the same buffer without writing: the streaming bandwidths this
// device reaches.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void hbm_copy_kernel(const v4u* __restrict__ src, v4u* __restrict__ dst,
                                                      size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// Streaming read: every 16-byte word once, folded into one word per thread
// (written only if it matches an impossible value, so the loads stay live).
__global__ __launch_bounds__(256) void hbm_read_kernel(const v4u* __restrict__ src, size_t n, v4u* sink) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    v4u acc = {0u, 0u, 0u, 0u};
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        acc ^= __builtin_nontemporal_load(src + i);
    if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u) sink[0] = acc;
}

bool ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    std::fprintf(stderr, "hbm_copy: %s: %s\n", what, hipGetErrorString(e));
    return false;
}

}  // namespace

int main(int argc, char** argv) {
    const long mib = argc > 1 ? std::atol(argv[1]) : 1024;
    const int repeats = argc > 2 ? std::atoi(argv[2]) : 5;
    if (mib <= 0 || mib > 65536 || repeats <= 0 || repeats > 1000) {
        std::fprintf(stderr, "usage: hbm_copy [MiB 1..65536] [repeats 1..1000]\n");
        return 2;
    }
    const size_t bytes = size_t(mib) << 20, n = bytes / sizeof(v4u);
    void *src = nullptr, *dst = nullptr;
    if (!ok(hipMalloc(&src, bytes), "hipMalloc") || !ok(hipMalloc(&dst, bytes), "hipMalloc")) return 1;
    if (!ok(hipMemset(src, 1, bytes), "hipMemset") || !ok(hipMemset(dst, 0, bytes), "hipMemset")) return 1;
    int cus = 0;
    if (!ok(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0), "attribute")) return 1;
    const dim3 grid(unsigned(cus) * 8), block(256);
    hipEvent_t start, stop;
    if (!ok(hipEventCreate(&start), "event") || !ok(hipEventCreate(&stop), "event")) return 1;
    hbm_copy_kernel<<<grid, block>>>(static_cast<const v4u*>(src), static_cast<v4u*>(dst), n);   // warm
    if (!ok(hipGetLastError(), "launch") || !ok(hipDeviceSynchronize(), "sync")) return 1;
    if (!ok(hipEventRecord(start, 0), "record")) return 1;
    for (int r = 0; r < repeats; ++r)
        hbm_copy_kernel<<<grid, block>>>(static_cast<const v4u*>(src), static_cast<v4u*>(dst), n);
    if (!ok(hipGetLastError(), "launch") || !ok(hipEventRecord(stop, 0), "record") ||
        !ok(hipEventSynchronize(stop), "sync"))
        return 1;
    float ms = 0;
    if (!ok(hipEventElapsedTime(&ms, start, stop), "elapsed")) return 1;
    const double per = ms / repeats;
    std::printf("hbm_copy: %zu bytes per launch (read %zu + write %zu), %d launches, %.3f ms each, %.1f GB/s\n",
                2 * bytes, bytes, bytes, repeats + 1, per, 2.0 * bytes / per / 1e6);
    // the same buffer read without writes: the bound of read-dominated kernels
    hbm_read_kernel<<<grid, block>>>(static_cast<const v4u*>(src), n, static_cast<v4u*>(dst));
    if (!ok(hipGetLastError(), "launch") || !ok(hipDeviceSynchronize(), "sync")) return 1;
    if (!ok(hipEventRecord(start, 0), "record")) return 1;
    for (int r = 0; r < repeats; ++r)
        hbm_read_kernel<<<grid, block>>>(static_cast<const v4u*>(src), n, static_cast<v4u*>(dst));
    if (!ok(hipGetLastError(), "launch") || !ok(hipEventRecord(stop, 0), "record") ||
        !ok(hipEventSynchronize(stop), "sync"))
        return 1;
    if (!ok(hipEventElapsedTime(&ms, start, stop), "elapsed")) return 1;
    std::printf("hbm_read: %zu bytes per launch, %d launches, %.3f ms each, %.1f GB/s\n", bytes, repeats + 1,
                ms / repeats, double(bytes) / (ms / repeats) / 1e6);
    (void)hipFree(src);
    (void)hipFree(dst);
    return 0;
}
