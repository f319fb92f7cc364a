// The sum  float s = 0; for (j = 0; j < n; ++j) s += v[j];  of n non-negative
// floats, bit for bit, by one wave in a fraction of the time of the 2048-step
// dependent chain (decoder.cpp:716-718 sums a norm's squares this way,
// transformer.cpp:127-130 a softmax denominator).
//
// Why it can be split.  While the running sum s and the exact sum s + a of a
// step lie in one binade [2^e, 2^(e+1)), s is a multiple of the binade's unit
// g = 2^(e-23) and the step rounds to nearest on that grid, so
//     fl(s + a) = s + g * rint(a / g)
// whenever a / g is not a tie: the step's increment does not depend on s.  The
// increments of such "safe" steps are multiples of g that stay below 2^(e+1),
// so any order of adding them is exact.  Only the other steps need the true s:
// those where the sum enters the next binade (about log2(n) of them), those
// whose binade is not certain, and ties, which round to the even neighbour.
//
// How.  Lane l takes elements [l E, (l + 1) E), E = 4 ceil(n / 256).
//   1. An approximate exclusive prefix P of every element (lane totals in
//      f32, a scan over the lanes, running sums in the lane).
//   2. The true running sum s_j differs from P_j by less than
//      (j + 2E + 8) 2^-24 P_j (each of the j earlier steps rounds by at most
//      2^-24 of the sum so far; P has at most 2E + 8 roundings on its path;
//      sums in the subnormal range round not at all);
//      with d a little wider than that, a step is safe when P_j (1 - d) and
//      (P_j + a_j) (1 + d) lie in one binade 2^e, a_j / g is not a tie and g
//      is at least 2^-27 of the total (so the increments' f64 prefix sums are
//      exact).  The increment is (2^e + a_j) - 2^e: 2^e has an even
//      significand, so the addition rounds a_j to the grid with ties to even,
//      and the subtraction is exact; a tie is |a_j - increment| == g / 2.
//      Safe increments are added in f64 per lane and scanned over the lanes:
//      I_j, the exact sum of the safe increments before element j.
//   3. Every other step (at most kSeqSumCap per lane) is recorded with its
//      I_j and a_j, compacted in element order, and walked: between two such
//      steps the sum grows by exactly I_q - I_p (a multiple of that run's g,
//      so exact in f32 too); at each one, s = fl(s + a) is the real step.
// Lane 0's chunk, where the binade changes at almost every doubling, is summed
// one by one instead (its in-order total).  A lane with more than kSeqSumCap
// unsafe steps, or a total that is not below 2^126 (infinite or NaN terms
// make it so), falls back to the plain chain.  Terms must not be negative;
// -0 and subnormal terms are fine.
//
// The values sit in LDS in the transposed layout of SeqLayout: element j of
// lane l's chunk at row j - l E, column l, so the lanes' reads of their chunks
// meet different banks.  Every lane returns the sum.
#pragma once

#include <type_traits>

#include "device_common.h"

namespace leafhip {

constexpr int kSeqSumCap = 12;                    // unsafe steps one lane records
constexpr int kSeqSumArea = kWave * (kSeqSumCap + 1);   // float4 of LDS scratch per wave (one spare per lane)

// Elements per lane: a multiple of four, so that the lanes' chunks load and
// step in whole groups of four.
__host__ __device__ constexpr int seq_per_lane(int n) { return (n + 4 * kWave - 1) / (4 * kWave) * 4; }

// Where element j of an n-element vector lives (E = seq_per_lane(n)):
// (j mod E) * 64 + j / E.  The quotient comes from a float reciprocal and one
// correction (exact for j < 2^24), not a 32-bit integer division.
struct SeqLayout {
    int E;
    float inv;
    __device__ explicit SeqLayout(int n) : E(seq_per_lane(n)), inv(1.0f / (float)E) {}
    __device__ __forceinline__ int at(int j) const {
        int q = (int)((float)j * inv);
        int r = j - q * E;
        if (r >= E) { ++q; r -= E; }
        if (r < 0) { --q; r += E; }
        return r * kWave + q;
    }
};

// The layout's slots past the n values ([n, 64 E)) set to +0, as the sums
// below require; `first`, `stride`: this thread's share of them.
__device__ __forceinline__ void seq_zero_tail(float* v, int n, int first, int stride) {
    const SeqLayout lay(n);
    for (int e = n + first; e < kWave * lay.E; e += stride) v[lay.at(e)] = 0.0f;
}

// Elements [0, m) in order (lane by lane, a lane's chunk top to bottom), 8
// LDS reads in flight at a time.  The fallback of the parallel sums below:
// one call site each, small code.
__device__ __forceinline__ float seq_chain(const float* v, int m, int E) {
    float s = 0.0f;
    for (int l = 0; l * E < m; ++l) {
        const int end = min(E, m - l * E);
        for (int i0 = 0; i0 < end; i0 += 8) {
            float e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = v[min(i0 + i, end - 1) * kWave + l];
#pragma unroll
            for (int i = 0; i < 8; ++i) s = s + (i0 + i < end ? e[i] : 0.0f);   // + 0 leaves s unchanged
        }
    }
    return s;
}

// Inclusive prefix sums over the wave's lanes on DPP lane moves: shifts by
// 1, 2, 4 and 8 inside each 16-lane row, then the row totals broadcast to the
// rows above (row_bcast:15 to rows 1 and 3, row_bcast:31 to rows 2 and 3).
// Lanes a move does not reach add 0.  Exact for integers and for floating
// values whose partial sums are all representable.
constexpr int kDppRowShr = 0x110;
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;
constexpr int kDppWaveShr1 = 0x138;      // lane i reads lane i - 1 (lane 0: 0)
template <int Ctrl, int RowMask = 0xF>
__device__ __forceinline__ unsigned dpp_move(unsigned v) {
    if constexpr (RowMask == 0xF && Ctrl != kDppWaveShr1)   // row shifts: bound_ctrl reads 0 past the row
        return (unsigned)__builtin_amdgcn_mov_dpp((int)v, Ctrl, RowMask, 0xF, true);
    else
        return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, Ctrl, RowMask, 0xF, false);
}
template <int Ctrl, int RowMask = 0xF>
__device__ __forceinline__ double dpp_move(double v) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = dpp_move<Ctrl, RowMask>((unsigned)b), hi = dpp_move<Ctrl, RowMask>((unsigned)(b >> 32));
    return __longlong_as_double((long long)((unsigned long long)lo | ((unsigned long long)hi << 32)));
}
template <int Ctrl, int RowMask = 0xF>
__device__ __forceinline__ float dpp_move(float v) {
    return __uint_as_float(dpp_move<Ctrl, RowMask>(__float_as_uint(v)));
}
template <int Ctrl, int RowMask = 0xF>
__device__ __forceinline__ int dpp_move(int v) {
    return (int)dpp_move<Ctrl, RowMask>((unsigned)v);
}
template <typename T>
__device__ __forceinline__ T wave_inclusive_sum(T x) {
    x = x + dpp_move<kDppRowShr + 1>(x);
    x = x + dpp_move<kDppRowShr + 2>(x);
    x = x + dpp_move<kDppRowShr + 4>(x);
    x = x + dpp_move<kDppRowShr + 8>(x);
    x = x + dpp_move<kDppRowBcast15, 0xA>(x);
    x = x + dpp_move<kDppRowBcast31, 0xC>(x);
    return x;
}
__device__ __forceinline__ float lane_value(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double lane_value(double v, int l) {
    const unsigned long long b = (unsigned long long)__double_as_longlong(v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    return __longlong_as_double((long long)((unsigned long long)lo | ((unsigned long long)hi << 32)));
}

// Building blocks of the column-order sum (below).  The passes over a lane's
// chunk are loops over groups of four elements read from LDS (the next
// group's loads go out before the current group's work): one group's code
// instead of a fully unrolled chunk keeps the decode step's instruction
// working set inside the instruction cache.

// Elements g .. g + 3 of this lane's chunk.
__device__ __forceinline__ void seq_group(const float* v, int g, int lane, float (&a)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = v[(g + i) * kWave + lane];
}

// The in-order sum of this lane's elements [i0, i1) added to t (i0, i1
// multiples of 4; slots past n hold +0 and add nothing).
__device__ __forceinline__ float seq_total(const float* v, int lane, int i0, int i1, float t) {
    if (i0 >= i1) return t;
    float cur[4], nxt[4];
    seq_group(v, i0, lane, cur);
    for (int g = i0; g < i1; g += 4) {
        seq_group(v, min(g + 4, i1 - 4), lane, nxt);   // the last round reloads its own group
#pragma unroll
        for (int i = 0; i < 4; ++i) t = t + cur[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
    }
    return t;
}

// What the steps of one lane's elements [i0, i1) need to know: the margins of
// the binade test for this lane and the finest grid that is safe.
struct SeqBounds {
    float clo, chi;
    unsigned thr;
    __device__ SeqBounds(float S, int j0, int E) {
        const unsigned ebS = __float_as_uint(S) >> 23;
        thr = (ebS > 51u ? ebS - 27u : 24u) << 23;   // finer grids are unsafe
        const float d = (float)(j0 + 3 * E + 16) * 0x1.1p-24f;
        clo = 1.0f - d;
        chi = 1.0f + d;
    }
};

// Steps over this lane's elements [i0, i1) from the approximate prefix P:
// safe increments into J (f64), unsafe steps recorded (J before the step, the
// term) in the lane's slots [first, first + kSeqSumCap) of area, the slot
// after them a spare that absorbs the stores of safe steps and of records
// past the cap.  Returns the number of records (more than kSeqSumCap: too
// many).
__device__ __forceinline__ int seq_steps(const float* v, int lane, int i0, int i1, float P, const SeqBounds& b,
                                         float4* area, int first, double& J) {
    char* const base = reinterpret_cast<char*>(area);
    const unsigned spare_at = (unsigned)(first + kSeqSumCap) * sizeof(float4);   // byte offsets into area
    unsigned at = (unsigned)first * sizeof(float4);
    J = 0.0;
    if (i0 < i1) {
        float cur[4], nxt[4];
        seq_group(v, i0, lane, cur);
        for (int g = i0; g < i1; g += 4) {
            seq_group(v, min(g + 4, i1 - 4), lane, nxt);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a = cur[i];
                const float Pn = P + a;
                const unsigned lo = __float_as_uint(P * b.clo), hi = __float_as_uint(Pn * b.chi);
                const unsigned mb = hi & 0x7f800000u;
                const float M = __uint_as_float(mb);
                const float inc = (M + a) - M;                       // g rint(a / g), ties to even
                const float h = __uint_as_float(mb - (24u << 23));   // g / 2
                const bool safe = (lo ^ hi) < 0x00800000u && hi >= b.thr && fabsf(a - inc) != h;
                char* const rec = base + min(at, spare_at);
                *reinterpret_cast<double*>(rec) = J;
                *reinterpret_cast<float*>(rec + 8) = a;
                at += safe ? 0u : (unsigned)sizeof(float4);
                float add = safe ? inc : 0.0f;
                asm volatile("" : "+v"(add));   // select in f32, convert once
                J += (double)add;
                P = Pn;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
        }
    }
    return (int)(at / sizeof(float4)) - first;
}

__device__ __forceinline__ double seq_record_j(const float4& e) {
    return __longlong_as_double((long long)((unsigned long long)__float_as_uint(e.x) |
                                            ((unsigned long long)__float_as_uint(e.y) << 32)));
}
__device__ __forceinline__ float4 seq_record(double I, float a) {
    const unsigned long long ib = (unsigned long long)__double_as_longlong(I);
    return make_float4(__uint_as_float((unsigned)ib), __uint_as_float((unsigned)(ib >> 32)), a, 0.0f);
}

// Moves this lane's records src[first + k], k < cnt, to dst[off + k] with
// I = base + (their J); lanes past their count write dst[spare].  All reads
// complete before any write, so src and dst may be the same.
__device__ __forceinline__ void seq_compact(const float4* src, int first, int cnt, double base, float4* dst, int off,
                                            int spare) {
    auto move = [&](auto width) {
        constexpr int kR = decltype(width)::value;
        float4 mine[kR];
#pragma unroll
        for (int k = 0; k < kR; ++k) mine[k] = src[first + k];
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int k = 0; k < kR; ++k)
            dst[k < cnt ? off + k : spare] = seq_record(base + seq_record_j(mine[k]), mine[k].z);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };
    if (!__any(cnt > 0)) return;
    if (!__any(cnt > 4))
        move(std::integral_constant<int, 4>());
    else
        move(std::integral_constant<int, kSeqSumCap>());
}

// The same from src into a distinct dst, one record per round (rounds: while
// any lane has one left).
__device__ __forceinline__ void seq_copy_records(const float4* src, int first, int cnt, double base, float4* dst,
                                                 int off, int spare) {
    for (int k = 0; __any(k < cnt); ++k) {
        const float4 e = src[first + k];
        dst[k < cnt ? off + k : spare] = seq_record(base + seq_record_j(e), e.z);
    }
}

// The walk over the K compacted records rec[0, K), lane i taking recorded
// step i: the running sum moves one lane up per step (wave_shr:1), lane i
// adds its exact jump R_i to the step and then the step's term,
// fl(fl(s + R_i) + a_i).  Lane 0 of a batch starts from the sum so far
// (folded into its jump, exactly).  s starts at the head's total; Itot is the
// exact sum of every safe increment.
__device__ __forceinline__ float seq_walk(const float4* rec, int K, float s, double Itot, int lane) {
    double prev = 0.0;
    for (int b = 0; b < K; b += kWave) {
        const float4 e = rec[min(b + lane, K - 1)];
        const double I = seq_record_j(e);
        const double up = dpp_move<kDppWaveShr1>(I);
        float R = (float)(I - (lane == 0 ? prev : up));   // exact jump to this step
        if (lane == 0) R = s + R;                         // exact: the sum just before step b
        const int m = __builtin_amdgcn_readfirstlane(min(kWave, K - b));
        // after step i lanes 0..i hold their final values, which further
        // steps recompute unchanged: m rounds up to whole groups of four
        float t = 0.0f;
        for (int i = 0; i < m; i += 4) {
#pragma unroll
            for (int u = 0; u < 4; ++u) t = (dpp_move<kDppWaveShr1>(t) + R) + e.z;
        }
        s = lane_value(t, m - 1);
        prev = lane_value(I, m - 1);
    }
    return s + (float)(Itot - prev);
}

// v: n >= 1 non-negative floats in the transposed layout, its slots past n
// holding +0 (seq_zero_tail); area: this wave's kSeqSumArea float4 of LDS
// scratch.  n <= kSeqSumMaxPerLane * 64 = 2048; longer vectors take the chain.
constexpr int kSeqSumMaxPerLane = 32;
// The parallel form; false where the chain must be taken.
__device__ __forceinline__ bool seq_parallel(const float* v, int n, int E, int lane, float4* area, float& sum) {
    // 1. this lane's in-order total, the lanes' prefixes
    const float T = seq_total(v, lane, 0, E, 0.0f);
    const float incl = wave_inclusive_sum(T);
    const float S = lane_value(incl, kWave - 1);
    const float P = dpp_move<kDppWaveShr1>(incl);   // the exclusive prefix (lane 0: 0)
    if (!(S < 0x1p126f)) return false;
    if (S == 0.0f) {   // all terms zero: the chain stays +0
        sum = 0.0f;
        return true;
    }
    const float head = lane_value(T, 0);            // lane 0's chunk: its in-order total
    // 2. safe increments and recorded steps
    const int first = lane * (kSeqSumCap + 1);
    double J;
    int cnt = seq_steps(v, lane, 0, E, P, SeqBounds(S, lane * E, E), area, first, J);
    if (lane == 0) {   // the head took lane 0's chunk
        cnt = 0;
        J = 0.0;
    }
    if (__any(cnt > kSeqSumCap)) return false;
    // 3. scans: the lanes' safe totals (exact in f64) and record counts; the
    // records compacted in element order with I = (safe increments before)
    const double Jincl = wave_inclusive_sum(J);
    const int cincl = wave_inclusive_sum(cnt);
    const double Itot = lane_value(Jincl, kWave - 1);
    const int K = __builtin_amdgcn_readlane(cincl, kWave - 1);
    seq_compact(area, first, cnt, Jincl - J, area, cincl - cnt,
                kWave * kSeqSumCap + lane);   // past every record: K <= 63 kSeqSumCap
    // 4. the walk
    sum = seq_walk(area, K, head, Itot, lane);
    return true;
}

__device__ __forceinline__ float wave_sequential_sum(const float* v, int n, float4* area) {
    // A fresh lane index per call: callers inside long loops would otherwise
    // have the lane-dependent constants below hoisted and held in registers.
    int lane = threadIdx.x & (kWave - 1);
    asm volatile("" : "+v"(lane));
    const int E = seq_per_lane(n);
    float sum;
    if (!(E <= kSeqSumMaxPerLane && seq_parallel(v, n, E, lane, area, sum))) sum = seq_chain(v, n, E);
    return sum;
}

// The same sum formed by the two waves of a pair, each stepping half of every
// lane's chunk.  h: this wave (0 or 1); area0, area1: each wave's
// kSeqSumArea float4; xchg: 2 * 64 float4 both waves see; comp: this wave's 128 float4.
// trade(): the pair's barrier (false: leave, the sum is not formed).  Both
// waves get the same bits.  Up to 64 recorded steps in all; more take the
// plain chain (both waves).
constexpr int kSeqPairRecords = kWave;
constexpr int kSeqPairXchg = 2 * kWave;      // float4
constexpr int kSeqPairComp = 2 * kWave;      // float4 per wave
// The pair's parallel form: 0 done, 1 the chain must be taken, 2 the trade
// failed.
template <typename Trade>
__device__ __forceinline__ int seq_pair_parallel(const float* v, int n, int E, int lane, float4* area0,
                                                 float4* area1, float4* xchg, float4* comp, int h, Trade&& trade,
                                                 float& sum) {
    // 1. as above, with the in-order total of the chunk's first part
    const int half = E / 8 * 4;   // wave 0 steps [0, half), wave 1 [half, E)
    const float Th = seq_total(v, lane, 0, half, 0.0f);
    const float T = seq_total(v, lane, half, E, Th);
    const float incl = wave_inclusive_sum(T);
    const float S = lane_value(incl, kWave - 1);
    const float P = dpp_move<kDppWaveShr1>(incl);
    if (!(S < 0x1p126f)) return 1;
    if (S == 0.0f) {
        sum = 0.0f;
        return 0;
    }
    const float head = lane_value(T, 0);
    // 2. this wave's part of every chunk (from P + Th: a few more roundings
    // on the prefix's path, within the margin)
    const int first = lane * (kSeqSumCap + 1);
    double J;
    int cnt = seq_steps(v, lane, h == 0 ? 0 : half, h == 0 ? half : E, h == 0 ? P : P + Th,
                        SeqBounds(S, lane * E, E), h == 0 ? area0 : area1, first, J);
    if (lane == 0) {
        cnt = 0;
        J = 0.0;
    }
    xchg[h * kWave + lane] = seq_record(J, __int_as_float(cnt));
    if (!trade()) return 2;
    const float4 other = xchg[(h ^ 1) * kWave + lane];
    const double J0 = h == 0 ? J : seq_record_j(other), J1 = h == 0 ? seq_record_j(other) : J;
    const int c0 = h == 0 ? cnt : __float_as_int(other.z), c1 = h == 0 ? __float_as_int(other.z) : cnt;
    // 3. both waves: the same scans, the records copied into their own
    // list, the walk
    const double Jl = J0 + J1;   // exact
    const int cl = c0 + c1;
    const double Jincl = wave_inclusive_sum(Jl);
    const int cincl = wave_inclusive_sum(cl);
    const int K = __builtin_amdgcn_readlane(cincl, kWave - 1);
    if (__any(c0 > kSeqSumCap || c1 > kSeqSumCap) || K > kSeqPairRecords) return 1;
    const double Ibase = Jincl - Jl;
    const int off = cincl - cl, spare = kSeqPairRecords + lane;
    seq_copy_records(area0, first, c0, Ibase, comp, off, spare);
    seq_copy_records(area1, first, c1, Ibase + J0, comp, off + c0, spare);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    sum = seq_walk(comp, K, head, lane_value(Jincl, kWave - 1), lane);
    return 0;
}

template <typename Trade>
__device__ __forceinline__ bool wave_pair_sequential_sum(const float* v, int n, float4* area0, float4* area1,
                                                         float4* xchg, float4* comp, int h, Trade&& trade,
                                                         float& sum) {
    int lane = threadIdx.x & (kWave - 1);
    asm volatile("" : "+v"(lane));
    const int E = seq_per_lane(n);
    const int state = E <= kSeqSumMaxPerLane ? seq_pair_parallel(v, n, E, lane, area0, area1, xchg, comp, h, trade, sum)
                                             : 1;
    if (state == 2) return false;
    if (state == 1) sum = seq_chain(v, n, E);
    return true;
}

}  // namespace leafhip
