// Device-side helpers shared by the decoder kernels (gfx950, wave64).
//
// The library is compiled with -ffp-contract=off: every fused multiply-add in
// these kernels is spelled with fmaf(), so operation order is explicit wherever
// results must match Leaf's CPU arithmetic bit for bit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace leafhip {

constexpr int kWave = 64;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));

typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// Descriptor word 3 of a raw (untyped) buffer resource on gfx9: loads through
// it are bounds-checked against the resource's size (reads past it return 0).
constexpr int kRawBufferWord3 = 0x00020000;

// 128-bit streaming load (non-temporal: weights are read once per forward).
__device__ __forceinline__ uint4 load_stream16(const void* p) {
    const v4u v = __builtin_nontemporal_load(static_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// The eight two's-complement nibbles of `word` (nibble e = bits 4e..4e+3, the
// low nibble first) as value / 16, exactly.  v_cvt_off_f32_i4 converts the
// low four bits of its operand to value / 16; byte selects of `word` reach the
// even nibbles and byte selects of `word >> 4` the odd ones, so a word costs
// one shift and eight converts.  (The empty asm keeps the compiler from
// folding the shift into bit-field extracts, which would drop the selects.)
// A product with value / 16, and every sum of such products, is the one with
// value scaled by exactly 2^-4 (outside the subnormal range), so a group
// scale taken times 16 gives the same results as dequantizing to value.
__device__ __forceinline__ void int4_sixteenths(uint32_t word, float (&f)[8]) {
    uint32_t odd = word >> 4;
    asm("" : "+v"(odd));
    f[0] = __builtin_amdgcn_cvt_off_f32_i4(word);
    f[2] = __builtin_amdgcn_cvt_off_f32_i4((word >> 8) & 0xFFu);
    f[4] = __builtin_amdgcn_cvt_off_f32_i4((word >> 16) & 0xFFu);
    f[6] = __builtin_amdgcn_cvt_off_f32_i4(word >> 24);
    f[1] = __builtin_amdgcn_cvt_off_f32_i4(odd);
    f[3] = __builtin_amdgcn_cvt_off_f32_i4((odd >> 8) & 0xFFu);
    f[5] = __builtin_amdgcn_cvt_off_f32_i4((odd >> 16) & 0xFFu);
    f[7] = __builtin_amdgcn_cvt_off_f32_i4(odd >> 24);
}

// Barrier for LDS hand-offs between the waves of a block: waits for this
// wave's LDS operations only (lgkmcnt(0)), so global loads into registers
// stay in flight across it (__syncthreads also waits for those).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((7 << 4) | 15 | (3 << 14));   // lgkmcnt(0); vmcnt, expcnt unconstrained
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// op(own, partner) for the partner lane l ^ 16 or l ^ 32, in registers
// (gfx950 v_permlane16_swap / v_permlane32_swap instead of an LDS
// permute).  Swapping a value with itself leaves each lane holding its own
// value and its partner's, in one order or the other: max and + commute, so
// every lane gets exactly op(own, partner).
__device__ __forceinline__ float max_xor16(float x) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float add_xor16(float x) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Butterfly reductions across the 64 lanes of a wave; every lane gets the result.
__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Block-wide reductions for blockDim.x a multiple of 64 (<= 1024).
template <typename T, typename Op>
__device__ __forceinline__ T block_reduce(T v, T* scratch, Op op, T (*wave_op)(T)) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    v = wave_op(v);
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    T r = scratch[0];
    for (int w = 1; w < waves; ++w) r = op(r, scratch[w]);
    return r;
}

// Symmetric int8 activation quantization of one value (decoder.cpp:618-627):
// round half to even of x * multiplier, saturated to +-127.
__device__ __forceinline__ int quantize_one(float x, float multiplier) {
    float r = __builtin_rintf(x * multiplier);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int)r;
}

// Signed nibble (low nibble = even column) -> int.
__device__ __forceinline__ int nibble(uint32_t byte, int high) {
    int v = (byte >> (high * 4)) & 15;
    return v >= 8 ? v - 16 : v;
}

// Four signed int8 packed in a 32-bit word, from eight signed nibbles'
// low (even columns) or high (odd columns) halves of four bytes: used to widen
// INT4 weights to the int8 lanes of v_dot4_i32_i8.
__device__ __forceinline__ int widen_nibbles_lo(uint32_t w) {   // nibbles 0,2,4,6 -> bytes 0..3? (see callers)
    uint32_t n = w & 0x0F0F0F0Fu;                                // low nibble of each byte
    uint32_t s = (n & 0x08080808u) * 0x1Eu;                      // 0x08 -> 0xF0 sign extension
    return (int)(n | s);
}
__device__ __forceinline__ int widen_nibbles_hi(uint32_t w) {
    uint32_t n = (w >> 4) & 0x0F0F0F0Fu;
    uint32_t s = (n & 0x08080808u) * 0x1Eu;
    return (int)(n | s);
}

__device__ __forceinline__ int dot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Sum of v[0..n) in index order, one rounding per addition (a CPU's scalar
// loop).  Values are read 64 at a time into registers before they are
// added: a read inside the dependent chain would add an LDS round trip to
// every step.
__device__ __forceinline__ float sequential_sum(const float* v, int n) {
    float s = 0.0f;
    int k = 0;
    for (; k + 64 <= n; k += 64) {
        float e[64];
#pragma unroll
        for (int j = 0; j < 64; ++j) e[j] = v[k + j];
#pragma unroll
        for (int j = 0; j < 64; ++j) s += e[j];
    }
    for (; k < n; ++k) s += v[k];
    return s;
}

// The same in double (the accurate RMS square sum).
__device__ __forceinline__ double sequential_sum_f64(const float* v, int n) {
    double s = 0.0;
    int k = 0;
    for (; k + 64 <= n; k += 64) {
        float e[64];
#pragma unroll
        for (int j = 0; j < 64; ++j) e[j] = v[k + j];
#pragma unroll
        for (int j = 0; j < 64; ++j) s += (double)e[j];
    }
    for (; k < n; ++k) s += (double)v[k];
    return s;
}

}  // namespace leafhip
