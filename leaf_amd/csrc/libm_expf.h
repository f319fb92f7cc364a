// The single-precision exponential of the CPU reference's libm, restated.
//
// Leaf's CPU path calls std::exp(float) -> glibc expf in its softmax
// (engine/src/kernels/transformer.cpp:134) and its SiLU
// (engine/src/decoder.cpp:983).  glibc is a third-party dependency of the
// reference, not part of it: glibc 2.35 (the version of this image) computes
// expf with the published double-precision algorithm of
// sysdeps/ieee754/flt-32/e_expf.c (from Arm's optimized-routines):
//
//   x * 32/ln2 = k + r, |r| <= 1/2, k an integer (round to nearest even);
//   exp(x) = 2^(k/32) * 2^(r/32),  2^(k/32) = 2^(k div 32) * T[k mod 32],
//   2^(r/32) ~ 1 + C2 r + C1 r^2 + C0 r^3           (evaluated in double),
//   result = (float)(s * p)
//
// with T[i] the double nearest 2^(i/32), stored less (i << 47) so that adding
// k << 47 to its bits scales it by 2^(k div 32).  On x86-64 CPUs with FMA,
// glibc's ifunc selects the build of this file compiled with -mfma, in which
// GCC fuses every product whose uses are all additions: the polynomial steps,
// and z = x * 32/ln2, which both k (z + shift) and r (z - k) then take
// unrounded.  The kernels here follow that build; with z rounded first, two
// inputs (0x4202422f, 0xc27c65d9) come out one ulp apart from it.
//
// Special cases (|x| >= 88 or NaN): -inf -> 0; +inf and NaN -> x + x;
// x > 0x1.62e42ep6 (overflow) -> +inf; x < -0x1.9fe368p6 (underflow) -> 0.
//
// The result equals this machine's expf bit for bit for every one of the
// 2^32 float inputs: tests/native/expf_exhaustive.cpp checks all of them.
#pragma once
#include <stdint.h>

#if defined(__HIP__)
#define LEAF_HOST_DEVICE __host__ __device__
#else
#define LEAF_HOST_DEVICE
#endif

namespace leafhip {

// T[i] = bits(nearest double to 2^(i/32)) - (i << 47).  The values follow from
// the definition alone: tests/test_libm_expf.py::
// test_exp2_table_follows_from_its_definition recomputes them in decimal
// arithmetic.
#if defined(__HIP__)
__device__ __constant__
#endif
static const uint64_t kExp2Table32[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// table(i) returns kExp2Table32[i]: kernels that call expf often pass a copy
// in LDS, since the per-lane index makes every read of the constant table a
// memory round trip.
template <typename Table>
LEAF_HOST_DEVICE inline float libm_expf_from(float x, const Table& table) {
    const uint32_t ux = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                              // |x| >= 88 or x is NaN
        if (ux == 0xff800000u) return 0.0f;             // -inf
        if (abstop >= 0x7f8) return x + x;              // +inf, NaN
        if (x > 0x1.62e42ep6f) return __builtin_inff(); // exp(x) > 2^128
        if (x < -0x1.9fe368p6f) return 0.0f;            // exp(x) < 2^-150
    }
    const double inv_ln2_n = 0x1.71547652b82fep+5;      // 32 / ln 2
    const double shift = 0x1.8p+52;                     // rounds z to an integer in its low bits
    const double c0 = 0x1.c6af84b912394p-20;            // polynomial of 2^(r/32), r in [-1/2, 1/2]
    const double c1 = 0x1.ebfce50fac4f3p-13;
    const double c2 = 0x1.62e42ff0c52d6p-6;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);    // z + shift, z = x * 32/ln2 unrounded
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd); // z - k
    uint64_t t = table((uint32_t)(ki % 32));
    t += ki << 47;
    const double s = __builtin_bit_cast(double, t);
    const double p = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    y = y * s;
    return (float)y;
}

#if defined(__HIP__)
// N evaluations of libm_expf_from at once, for kernels: in phases (every
// table read issued before any is used) and without branches (the special
// cases selected afterwards), so the evaluations interleave.  Equal to N
// separate calls bit for bit, except that a NaN input gives a NaN of another
// payload.
template <int N, typename Table>
__device__ inline void libm_expf_batch(float (&x)[N], const Table& table) {
    const double inv_ln2_n = 0x1.71547652b82fep+5;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-20;
    const double c1 = 0x1.ebfce50fac4f3p-13;
    const double c2 = 0x1.62e42ff0c52d6p-6;
    double r[N];
    uint64_t ki[N], t[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const double xd = (double)x[i];
        double kd = __builtin_fma(inv_ln2_n, xd, shift);
        ki[i] = __builtin_bit_cast(uint64_t, kd);
        kd -= shift;
        r[i] = __builtin_fma(inv_ln2_n, xd, -kd);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) t[i] = table((uint32_t)(ki[i] % 32));
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const double s = __builtin_bit_cast(double, t[i] + (ki[i] << 47));
        const double p = __builtin_fma(c0, r[i], c1);
        const double r2 = r[i] * r[i];
        double y = __builtin_fma(c2, r[i], 1.0);
        y = __builtin_fma(p, r2, y);
        y = y * s;
        float result = (float)y;                                      // NaN stays NaN
        result = x[i] < -0x1.9fe368p6f ? 0.0f : result;              // exp(x) < 2^-150, and -inf
        result = x[i] > 0x1.62e42ep6f ? __builtin_inff() : result;   // exp(x) > 2^128, and +inf
        x[i] = result;
    }
}
#endif

LEAF_HOST_DEVICE inline float libm_expf(float x) {
    return libm_expf_from(x, [](uint32_t i) { return kExp2Table32[i]; });
}

}  // namespace leafhip
