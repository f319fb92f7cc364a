// Persistent single-token decode step for W8A8 decoders on MI355X (gfx950).
//
// Why one launch per token: a TinyLlama-shape layer streams 44 MB of int8
// weights (5.5 us at 8 TB/s), but as seven separate launches it costs ~36 us,
// because each launch pays wave start-up, a cold HBM round trip and its
// reductions in series.  Here one block of 512 threads per CU stays resident
// for the whole token, and its waves split into two roles:
//
//   * 2 exchange waves move the activation vectors between blocks.  Phases
//     hand vectors to each other through exchange buffers of 64-bit words
//     (epoch << 32 | f32 bits), written and read with agent-scope relaxed
//     atomics: a reader spins on the data itself until every word carries the
//     epoch of the phase it waits for -- no fences, no barrier counters (one
//     round trip against ~8 us for fenced barriers, measured).  The words live
//     in uncached device memory and each wave reads them coalesced.  Every
//     block normalizes and quantizes the whole input vector itself (the
//     per-token absmax of the W8A8 quantization is global) and posts the int8
//     vector in LDS.  These waves also run attention: (KV head, span of 64
//     keys) items whose cached keys are fetched during the RMSNorm, and merge
//     waves (one per query head, in the last blocks) that combine the spans.
//   * 6 weight waves own whole rows of every matrix of a layer and keep them
//     in registers.  After computing a phase they load the same phase of the
//     next layer, so the weight stream runs a full layer ahead of the
//     dependency chain.  They wait for their input on an LDS flag, which
//     counts on lgkmcnt: the loads in flight (vmcnt) never delay that wait,
//     the way they would delay an exchange poll issued behind them.
//
// Arithmetic per output is that of the multi-launch path: exact int32 dot,
// ((float)acc * s_x) * s_w + bias, residual adds as y + v, RoPE a*c - b*s /
// b*c + a*s with the host-built tables, SiLU gate up * silu(gate).  Every spin
// is bounded: on timeout a block raises the abort flag, which every other
// block observes, and all blocks leave the kernel.
#include "decode_step.h"

#include <math.h>

#include <type_traits>

#include "device_common.h"
#include "libm_expf.h"
#include "sequential_sum.h"

namespace leafhip {
namespace {

typedef unsigned long long u64;

// Global-address-space views of generic pointers: the loads and atomics then
// compile to global_* instructions, which count only on vmcnt, so waiting for
// LDS never waits for the weight stream in flight.
#define LEAF_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ T ldg(const T* p) {
    return *(const LEAF_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ void stg(T* p, T v) {
    *(LEAF_GLOBAL T*)p = v;
}
__device__ __forceinline__ v4u ldg_stream(const void* p) {
    return __builtin_nontemporal_load((const LEAF_GLOBAL v4u*)p);
}

constexpr int kT = kStepThreads;                             // 512
constexpr int kWaves = kT / kWave;                           // 8: two per SIMD, 256 VGPRs each
constexpr int kA = 2;                                        // exchange waves
constexpr int kAT = kA * kWave;                              // exchange lanes
constexpr int kB = kWaves - kA;                              // weight waves
static_assert(kA == 2, "the exchange waves work as a pair");
constexpr int kKCH = kStepMaxHidden / 16 / kWave;            // 16-byte chunks per lane, hidden-wide int8 row
constexpr int kKCF = kStepMaxFfn / 16 / kWave;               // ... ffn-wide int8 row
constexpr int kNH = (kStepMaxHidden + kAT - 1) / kAT;        // hidden values per exchange lane
constexpr int kNF = (kStepMaxFfn + kAT - 1) / kAT;           // ffn values per exchange lane
constexpr int kSpanF4 = kStepSpanKeys * kStepDim / 4;        // float4 of a K (or V) span
constexpr int kNQ = (kStepMaxGroup * kStepDim + kAT - 1) / kAT + 1;   // q values (+ new k or v) per exchange lane
constexpr int kNK = kSpanF4 / kAT;                           // float4 of a K (or V) span per exchange lane
static_assert(kNK * kAT == kSpanF4, "exchange lanes cover a span exactly");
constexpr int kQP = 1;                                       // q|k|v pairs per weight wave
constexpr int kOR = 2;                                       // o / down rows per weight wave
constexpr int kGP = 4;                                       // gate|up pairs per weight wave
constexpr int kHeadsA = (kStepMaxGroup + kA - 1) / kA;       // query heads per exchange wave
constexpr int kKStride = kStepDim + 4;                       // padded K row in LDS
constexpr int kMergeBatch = 16;                              // span partials polled together
constexpr unsigned kSpinLimit = 1u << 20;                    // about a second of polling

static_assert(sizeof(StepLayer) % 16 == 0, "layer descriptors are copied as 16-byte words");

struct __align__(16) Shared {
    // Layer descriptors, copied once: read from LDS they are not vector loads,
    // which would wait (in order) behind every weight prefetch in flight.
    unsigned char layer_bytes[kStepMaxLayers * sizeof(StepLayer)];
    int8_t xq[2][kStepMaxFfn];      // quantized input, double-buffered by phase
    float h_in[kStepMaxHidden];     // layer input (residual of o_proj)
    float h_mid[kStepMaxHidden];    // after o_proj (residual of down_proj)
    float xf[kStepMaxHidden];       // normalized FP32 input of the head
    float gamma_in[kNH * kAT];      // gamma of the next input (or final) RMSNorm, as exchange-lane runs
    float k[kStepSpanKeys * kKStride];
    float v[kStepSpanKeys * kStepDim];
    float q[kStepMaxGroup * kStepDim];
    float e[kStepMaxGroup * kStepSpanKeys];
    float sx[2];                    // activation scale per xq buffer
    u64 pair[kA][2];                // a_trade words: [wave][sequence parity]
    float best_v[kWaves];
    int best_i[kWaves];
    int ready[kA];                  // last phase whose input each exchange wave posted
    int received[kA];               // last phase whose input vector each exchange wave has read
    int published;                  // phase outputs this block's weight waves published (kB per phase)
    int abort;
};

// Where element e of a staged product vector (SharedRef::xg) sits.
__device__ __forceinline__ int xg_at(int e) { return e + 4 * (e >> 4); }

// Reference order adds each chain wave's softmax terms of one query head
// (scores, then exp(score - max), then the probabilities) in the transposed
// layout of wave_sequential_sum, and per exchange wave the scratch of that
// sum, which the p.v chain then uses to stage its V rows.
constexpr int kRefMaxKeys = 2048;   // softmax terms one chain wave holds (kSeqSumMaxPerLane per lane)
static_assert(kRefMaxKeys == kWave * kSeqSumMaxPerLane, "the denominator's terms fit one register chunk per lane");
// Visible keys of the reference-order step: the p.v chain reads its last
// group's p (fewer than 64 past the keys) inside the wave's kRefMaxKeys floats.
constexpr int kRefStepKeys = kRefMaxKeys - kWave;
static_assert(kA * kRefMaxKeys <= kStepSpanKeys * kStepDim, "s.v holds each chain wave's probabilities in key order");
struct __align__(16) SharedRef : Shared {
    float pe[kA][kRefMaxKeys];
    float4 area[kA][kSeqSumArea];
    uint64_t exp2[32];   // expf's table (libm_expf.h), read per lane
    // The RMSNorms before q|k|v and gate|up (wave_speculate, wave_confirm):
    // the products x * gamma (element e at xg_at(e): 16-element chunks 20
    // floats apart, so a lane's 16-byte reads of its chunks meet no bank
    // conflict), the gamma of the norm before gate|up (natural element order;
    // the input norm's waits in gamma_in), the column-order square sums, and
    // the last phase whose vectors each exchange wave has stored.
    float xg[kStepMaxHidden / 16 * 20];
    float gamma_mid[kNH * kAT];
    float sq[2];
    int staged[kA];
    // pe and area, both free then, stage the gated activation while its
    // maximum is traded (quantize_into)
    __device__ float* stage() { return &pe[0][0]; }
    // the RMSNorm's pair sum: the waves' trade and compaction space in pe
    __device__ float4* seq_xchg() { return reinterpret_cast<float4*>(&pe[0][0]); }
    __device__ float4* seq_comp(int w) { return seq_xchg() + kSeqPairXchg + w * kSeqPairComp; }
};
static_assert(kA == 2 && (kSeqPairXchg + kA * kSeqPairComp) * 4 <= kA * kRefMaxKeys, "pe holds the pair sum's space");
static_assert(sizeof(float) * kA * kRefMaxKeys + sizeof(float4) * kA * kSeqSumArea >= sizeof(float) * kNF * kAT,
              "pe and area hold an ffn-wide vector's runs");
static_assert(sizeof(SharedRef) <= 160 * 1024, "one block per CU holds the reference-order LDS");

// Wave reductions on DPP lane moves instead of LDS-crossbar shuffles: xor 1
// and xor 2 (quad permutes), then the half-row and row mirrors (once lanes of
// a quad, then of a half-row, agree, these pair each lane with the other
// half), then the four row totals read out and combined in a fixed order, so
// every lane gets the same bits.
constexpr int kDppXor1 = 0xB1;         // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror
constexpr int kDppRor8 = 0x128;        // row_ror:8 (lane i of a 16-lane row reads lane (i + 8) mod 16)
template <int Ctrl>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, Ctrl, 0xF, 0xF, false);
}
template <int Ctrl>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(dpp<Ctrl>(__float_as_int(v)));
}
__device__ __forceinline__ float rows_f32(float v, int row) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * row));
}
__device__ __forceinline__ float dpp_sum_f32(float v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    return (rows_f32(v, 0) + rows_f32(v, 1)) + (rows_f32(v, 2) + rows_f32(v, 3));
}
__device__ __forceinline__ float dpp_max_f32(float v) {
    v = fmaxf(v, dpp<kDppXor1>(v));
    v = fmaxf(v, dpp<kDppXor2>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppMirror>(v));
    return fmaxf(fmaxf(rows_f32(v, 0), rows_f32(v, 1)), fmaxf(rows_f32(v, 2), rows_f32(v, 3)));
}
__device__ __forceinline__ int dpp_sum_i32(int v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    v += dpp<kDppMirror>(v);
    return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
           (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
}

// Makes every LDS read of a step complete before any of its arithmetic: the
// register-pressure-driven scheduler otherwise interleaves each read with its
// use, paying one LDS round trip per read instead of one per step.
__device__ __forceinline__ void all_loaded(const v4f& a, const v4f (&b)[8]) {
    asm volatile("" ::"v"(a), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "v"(b[4]), "v"(b[5]), "v"(b[6]), "v"(b[7]));
}
__device__ __forceinline__ void all_loaded(const v4f& a, const v4f (&b)[4]) {
    asm volatile("" ::"v"(a), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]));
}
__device__ __forceinline__ void all_loaded(const v4f& a, const v4f (&b)[2]) {
    asm volatile("" ::"v"(a), "v"(b[0]), "v"(b[1]));
}
__device__ __forceinline__ void all_loaded(const v4f& a, const v4f (&b)[1]) {
    asm volatile("" ::"v"(a), "v"(b[0]));
}

__device__ __forceinline__ const StepLayer& layer_at(const Shared& s, int L) {
    return reinterpret_cast<const StepLayer*>(s.layer_bytes)[L];
}

__device__ __forceinline__ u64 tagged(unsigned epoch, float v) {
    return (u64(epoch) << 32) | __float_as_uint(v);
}
__device__ __forceinline__ void publish(u64* p, unsigned epoch, float v) {
    __hip_atomic_store((LEAF_GLOBAL u64*)p, tagged(epoch, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 fetch(const u64* p) {
    return __hip_atomic_load((const LEAF_GLOBAL u64*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool aborted(const unsigned* flag) {
    return __hip_atomic_load((const LEAF_GLOBAL unsigned*)flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
// The first code raised stands: a wave that gives up only because another
// block aborted must not overwrite the reason the host acts on (a mismatched
// XCD, which makes the host run the step again, against a timeout).  Only the
// block that raised first writes the host copy.
__device__ __forceinline__ void raise_abort(const StepParams& P, unsigned why = 1u) {
    unsigned expected = 0u;
    if (__hip_atomic_compare_exchange_strong((LEAF_GLOBAL unsigned*)P.abort_flag, &expected, why, __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &&
        P.host_abort)
        *P.host_abort = why;
}
// Abort code: a block did not run on XCD blockIdx.x % 8, so the XCD-local
// merge cannot work (the host turns it off and runs the step again).
constexpr unsigned kAbortXcdMapping = 2u;
__device__ __forceinline__ int xcc_id() {
    return __builtin_amdgcn_s_getreg((20) | (0 << 6) | (15 << 11)) & 15;   // hwreg(HW_REG_XCC_ID, 0, 16)
}
__device__ __forceinline__ int lds_load(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Completes this wave's LDS accesses and keeps the compiler from moving
// memory operations across (no vmcnt wait: loads in flight stay in flight).
__device__ __forceinline__ void lds_done() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Waits until src[index(i)] carries `epoch` for every i < N whose index is
// not negative (absent elements read as 0); the values land in out[].  All
// loads are issued together and only missing words are polled again; indices
// are recomputed per poll rather than held in registers.  Returns false (after
// raising the abort flag) on timeout or when another block aborted.
template <int N, typename Index>
__device__ __forceinline__ bool await(const u64* src, Index index, unsigned epoch, float (&out)[N],
                                      const StepParams& P) {
    // Branch-free: absent elements load word 0 and are replaced by a tagged
    // zero; a lane that is still missing a word re-polls its whole set.
    u64 w[N];
    auto poll = [&] {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int k = index(i);
            const u64 v = fetch(src + (k >= 0 ? k : 0));
            w[i] = k >= 0 ? v : tagged(epoch, 0.0f);
        }
    };
    poll();
    for (unsigned spin = 0;; ++spin) {
        bool ready = true;
#pragma unroll
        for (int i = 0; i < N; ++i) ready = ready && unsigned(w[i] >> 32) == epoch;
        if (ready) break;
        if (spin >= kSpinLimit || ((spin & 255u) == 255u && aborted(P.abort_flag))) {
            raise_abort(P);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
        poll();
    }
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __uint_as_float(unsigned(w[i]));
    return true;
}

// Exchange-lane ownership of a vector: lane a holds x[kRun g + j] = element
// kRun (g kAT + a) + j.  A run of two elements is one 16-byte load of two
// tagged words, and a wave's load instruction reads 1 KiB of consecutive
// memory: the exchange words live in uncached memory, where a wave
// instruction whose lanes are not contiguous turns into many small
// transactions (runs of four, read as two 16-byte halves 32 bytes apart,
// measured 2.7 us for 24 KiB per block).  Vectors handled this way have
// n % kRun == 0 and buffers of at least kAT * N words.
constexpr int kRun = 2;
__device__ __forceinline__ int run_of(int g, int a) { return g * kAT + a; }

// A raw buffer resource over exchange words: its loads take a per-lane
// 32-bit offset plus a wave-uniform SGPR offset, so a lane's runs need one
// address register rather than one 64-bit address per word.  Loads use sc1
// (coherent at agent scope), like the atomic loads of fetch().
constexpr int kLoadSc1 = 16;                  // cache-policy bit sc1
__device__ __forceinline__ __amdgpu_buffer_rsrc_t exchange_view(const u64* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<u64*>(base), (short)0, 0x7fffffff, kRawBufferWord3);
}

// Spins until *p carries `epoch`; false (abort raised) on timeout or abort.
__device__ __forceinline__ bool spin_until(const u64* p, unsigned epoch, unsigned& spin, const StepParams& P) {
    while (unsigned(fetch(p) >> 32) != epoch) {
        if (++spin >= kSpinLimit || ((spin & 255u) == 255u && aborted(P.abort_flag))) {
            raise_abort(P);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}

// This lane's runs of the n-element vector src once they all carry
// `epoch`.  Runs past n are not waited for and hold whatever the buffer holds
// there (callers mask them out or never read them).  A lane first watches one
// word it needs, then reads all of them; a word still missing is watched alone
// before the next full read (a full re-read per spin from every lane of every
// block would crowd the memory pipeline the weight waves use).  G0 > 0 takes
// the lane's runs G0 .. G0 + N/kRun - 1 only (a long vector in parts, so
// fewer 64-bit words are held at once); Watch false skips the first watched
// word (the caller knows the vector is landing).
template <int N, int G0 = 0, bool Watch = true>
__device__ __forceinline__ bool await_runs(const u64* src, int n, unsigned epoch, float* out, int a,
                                           const StepParams& P) {
    static_assert(N % kRun == 0, "whole runs");
    constexpr int G = N / kRun;
    src += kRun * kAT * G0;
    const int live = n / kRun - a - kAT * G0;   // run g (from G0) is inside the vector when g * kAT < live
    const u64* mine = src + kRun * a;
    unsigned spin = 0;
    if (Watch && live > 0 &&
        !spin_until(mine + kRun * kAT * min(G - 1, (live - 1) / kAT) + kRun - 1, epoch, spin, P))
        return false;
    const __amdgpu_buffer_rsrc_t view = exchange_view(src);
    u64 w[N];
    for (;;) {
        asm volatile("" ::: "memory");   // a fresh read each time round
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const v2u v = __builtin_amdgcn_raw_buffer_load_b64(view, 8 * kRun * a + 8 * (i % kRun),
                                                              8 * kRun * kAT * (i / kRun), kLoadSc1);
            w[i] = (u64(v.y) << 32) | v.x;
        }
        int missing = -1;
#pragma unroll
        for (int i = N - 1; i >= 0; --i)
            missing = ((i / kRun) * kAT < live && unsigned(w[i] >> 32) != epoch) ? i : missing;
        if (missing < 0) break;
        if (!spin_until(mine + kRun * kAT * (missing / kRun) + missing % kRun, epoch, spin, P)) return false;
    }
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __uint_as_float(unsigned(w[i]));
    return true;
}

// One word once it carries `epoch` (wanted false: 0 without waiting).
__device__ __forceinline__ bool await_one(const u64* p, bool wanted, unsigned epoch, float& out, const StepParams& P) {
    unsigned spin = 0;
    out = 0.0f;
    if (!wanted) return true;
    if (!spin_until(p, epoch, spin, P)) return false;
    out = __uint_as_float(unsigned(fetch(p)));
    return true;
}

// Span partials of one query head (span j at base + j * stride words: max,
// sum, then the dim outputs).  Once they all carry `epoch`: ml = (max, sum)
// of span `lane` (lanes < spans), os[j] = output element `lane` of span
// s0 + j (j < spans - s0).  One buffer read takes all of them and repeats
// until every word is there: only the merge waves (one per query head) poll
// this way, and a full re-read costs less than watching a single word first,
// which adds a round trip.  Words of spans past the last are read from the
// last span and ignored.
template <int NB>
__device__ __forceinline__ bool await_partials(const u64* base, int stride, int spans, int s0, int lane,
                                               unsigned epoch, v2f& ml, float (&os)[NB], const StepParams& P) {
    const __amdgpu_buffer_rsrc_t view = exchange_view(base);
    const int own = min(lane, spans - 1);
    unsigned spin = 0;
    for (;;) {
        asm volatile("" ::: "memory");
        const v4u m = __builtin_amdgcn_raw_buffer_load_b128(view, 8 * own * stride, 0, kLoadSc1);
        u64 w[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const v2u v = __builtin_amdgcn_raw_buffer_load_b64(view, 8 * (2 + lane),
                                                              8 * stride * min(s0 + j, spans - 1), kLoadSc1);
            w[j] = (u64(v.y) << 32) | v.x;
        }
        bool ready = lane >= spans || (m.y == epoch && m.w == epoch);
#pragma unroll
        for (int j = 0; j < NB; ++j) ready = ready && (s0 + j >= spans || unsigned(w[j] >> 32) == epoch);
        if (__all(ready)) {
            ml = v2f{__uint_as_float(m.x), __uint_as_float(m.z)};
#pragma unroll
            for (int j = 0; j < NB; ++j) os[j] = __uint_as_float(unsigned(w[j]));
            return true;
        }
        if (++spin >= kSpinLimit || ((spin & 255u) == 255u && aborted(P.abort_flag))) {
            raise_abort(P);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// ------------------------------------------------------ exchange waves ---
// The two exchange waves trade one value: each posts it, tagged with the
// call's sequence number, in its own LDS word and reads the other's.  A wave
// that arrives first waits only for that word (no shared counter, no
// arrival count to poll), and both combine the two values themselves.  Each
// wave's earlier LDS writes are complete before its word is posted, so this
// is also the pair's barrier.  Returns false (abort flag raised in LDS) on
// timeout or when the block is being abandoned.
__device__ __forceinline__ bool a_trade(float mine, float& theirs, Shared& s, int& round) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    ++round;
    lds_done();
    if ((threadIdx.x & 63) == 0)
        __hip_atomic_store(&s.pair[w][round & 1], tagged(unsigned(round), mine), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
    const u64* other = &s.pair[w ^ 1][round & 1];
    // A tight poll (one LDS round trip per try): the other wave usually
    // posts within a few hundred cycles.  The abort flag is checked every
    // 64 tries only.
    for (unsigned spin = 0;; ++spin) {
        const u64 v = __hip_atomic_load(other, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (unsigned(v >> 32) == unsigned(round)) {
            theirs = __uint_as_float(unsigned(v));
            break;
        }
        if ((spin & 63u) == 63u && (spin > 16 * kSpinLimit || lds_load(&s.abort))) {
            lds_store(&s.abort, 1);
            return false;
        }
    }
    asm volatile("" ::: "memory");
    return true;
}

__device__ __forceinline__ bool a_sync(Shared& s, int& round) {
    float unused;
    return a_trade(0.0f, unused, s, round);
}

// Every exchange wave has `ok`; otherwise this wave leaves the kernel with the
// block's abort flag raised (the other exchange wave and the weight waves see
// it in their next wait, other blocks see the device flag).
__device__ __forceinline__ bool a_check(bool ok, Shared& s, const StepParams& P) {
    if (__all(ok)) return true;
    lds_store(&s.abort, 1);
    raise_abort(P);
    return false;
}

// Sums (or maxes) over the exchange lanes; both exchange waves get the same
// bits (IEEE addition and fmaxf are commutative).
__device__ __forceinline__ bool a_sum(float& v, Shared& s, int& round) {
    v = dpp_sum_f32(v);
    float other;
    if (!a_trade(v, other, s, round)) return false;
    v += other;
    return true;
}
__device__ __forceinline__ bool a_max(float& v, Shared& s, int& round) {
    v = dpp_max_f32(v);
    float other;
    if (!a_trade(v, other, s, round)) return false;
    v = fmaxf(v, other);
    return true;
}

// Waits until this block's weight waves issued their stores of `phases`
// phases (kB each).  Blocks publish within about a microsecond of each other,
// so this is when the exchange waves start reading a vector: the first full
// read then usually finds every word, one round trip sooner than watching a
// remote word first.  Missing words are still watched and read again.
__device__ __forceinline__ bool wait_published(Shared& s, int phases) {
    for (unsigned spin = 0; lds_load(&s.published) < kB * phases; ++spin) {
        if (spin > kSpinLimit || lds_load(&s.abort)) return false;
        __builtin_amdgcn_s_sleep(0);
    }
    return true;
}

// Notes that this exchange wave has read the input vector of `phase`.
__device__ __forceinline__ void note_received(Shared& s, int phase) {
    if ((threadIdx.x & 63) == 0) lds_store(&s.received[threadIdx.x >> 6], phase);
}

// Posts phase `phase` for this exchange wave: it has finished writing its
// part of the phase's input.  The weight waves start once both posted.
__device__ __forceinline__ void post(Shared& s, int phase) {
    lds_done();
    if ((threadIdx.x & 63) == 0) lds_store(&s.ready[threadIdx.x >> 6], phase);
}

// Reference order: stores this exchange wave's runs of x * gamma (the
// products the weight waves quantize speculatively, wave_speculate) and notes
// that its part of the vector that phase `phase` normalizes, and of its
// gamma, is in LDS; the exchange waves then form the column-order square sum.
template <int N>
__device__ __forceinline__ void stage_products(SharedRef& r, const float (&x)[N], const float (&gamma)[N], int a,
                                               int phase) {
    static_assert(N % kRun == 0 && kRun == 2, "runs of two");
#pragma unroll
    for (int g = 0; g < N / kRun; ++g) {
        const int e = kRun * run_of(g, a);   // even: both elements of a run share a 16-element chunk
        *reinterpret_cast<v2f*>(r.xg + xg_at(e)) = v2f{x[kRun * g] * gamma[kRun * g], x[kRun * g + 1] * gamma[kRun * g + 1]};
    }
    lds_done();
    if ((threadIdx.x & 63) == 0) lds_store(&r.staged[threadIdx.x >> 6], phase);
}

// RMSNorm scale of a square sum, norm()'s expression (decoder.cpp:719-721).
__device__ __forceinline__ float rms_scale(float sq, int n, float eps) { return 1.0f / sqrtf(sq / (float)n + eps); }

// The squares of the n values held as runs, summed in column order as
// norm() sums them (decoder.cpp:716-718): every lane stores its runs' squares
// (s.xf is free until the head) in the layout of wave_sequential_sum, and the
// two exchange waves form the column-order sum together
// (wave_pair_sequential_sum: each steps half of every chunk, one trade
// between them); both get the same bits.
template <int N>
__device__ __forceinline__ bool ref_square_sum(const float (&x)[N], int n, int a, Shared& s, int& round, float& sq) {
    const int live = n / kRun - a;
    const SeqLayout lay(n);
    // A run's two elements are consecutive rows of one column; when E
    // divides the kRun * kAT elements between a lane's runs, run g sits
    // kRun * kAT / E columns past run 0.
    const int at0 = lay.at(kRun * a);
    const int step = (kRun * kAT) % lay.E == 0 ? kRun * kAT / lay.E : -1;
#pragma unroll
    for (int g = 0; g < N / kRun; ++g)
        if (g * kAT < live) {
            const int at = step >= 0 ? at0 + step * g : lay.at(kRun * run_of(g, a));
            const float x0 = x[kRun * g] - 0.0f, x1 = x[kRun * g + 1] - 0.0f;
            s.xf[at] = x0 * x0;
            s.xf[at + kWave] = x1 * x1;
        }
    seq_zero_tail(s.xf, n, a, kAT);
    if (!a_sync(s, round)) return false;   // both waves' squares are in place
    // each exchange wave steps half of every lane's chunk
    SharedRef& r = static_cast<SharedRef&>(s);
    const int w = __builtin_amdgcn_readfirstlane(a >> 6);
    return wave_pair_sequential_sum(s.xf, n, r.area[0], r.area[1], r.seq_xchg(), r.seq_comp(w), w,
                                    [&] { return a_sync(s, round); }, sq);
}

// RMSNorm of the n values held as runs (decoder.cpp:706-727).  In reference
// order the squares are summed in column order (ref_square_sum) and the
// normalized value is (x - 0) * scale * gamma + 0, norm()'s expression with
// mean 0 and no beta.
template <bool REF, int N>
__device__ __forceinline__ bool rms_normalize(float (&x)[N], int n, const float (&gamma)[N], float eps, int a,
                                              Shared& s, int& round) {
    const int live = n / kRun - a;
    float sq = 0.0f;
    if constexpr (REF) {
        if (!ref_square_sum(x, n, a, s, round, sq)) return false;
        const float scale = rms_scale(sq, n, eps);
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = (x[i] - 0.0f) * scale * gamma[i] + 0.0f;
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) sq += (i / kRun) * kAT < live ? x[i] * x[i] : 0.0f;
        if (!a_sum(sq, s, round)) return false;
        const float scale = rms_scale(sq, n, eps);
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = x[i] * scale * gamma[i];
    }
    return true;
}

// This lane's runs into dst (natural element order; dst holds kAT * N floats).
template <int N>
__device__ __forceinline__ void store_runs(float* dst, const float (&x)[N], int a) {
    static_assert(N % kRun == 0 && kRun == 2, "runs of two");
#pragma unroll
    for (int g = 0; g < N / kRun; ++g)
        *reinterpret_cast<v2f*>(dst + kRun * run_of(g, a)) = v2f{x[kRun * g], x[kRun * g + 1]};
}

// This lane's runs out of src (natural element order), as store_runs wrote them.
template <int N>
__device__ __forceinline__ void load_runs(float (&x)[N], const float* src, int a) {
    static_assert(N % kRun == 0 && kRun == 2, "runs of two");
#pragma unroll
    for (int g = 0; g < N / kRun; ++g) {
        const v2f v = *reinterpret_cast<const v2f*>(src + kRun * run_of(g, a));
        x[kRun * g] = v[0];
        x[kRun * g + 1] = v[1];
    }
}

// Per-token symmetric int8 quantization into s.xq[buf] (decoder.cpp:1028-1043).
// Runs past n land in the buffer's tail, which no reader uses.  With `stage`
// the values wait in LDS (this lane's runs) while the maximum is traded, so
// they hold no registers across the wait.
template <int N>
__device__ __forceinline__ bool quantize_into(float (&x)[N], int n, int buf, int a, Shared& s, int& round,
                                              float* stage = nullptr) {
    static_assert(N % kRun == 0 && kRun == 2, "runs of two");
    const int live = n / kRun - a;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < N; ++i) amax = fmaxf(amax, (i / kRun) * kAT < live ? fabsf(x[i]) : 0.0f);
    if (stage) store_runs(stage, x, a);
    if (!a_max(amax, s, round)) return false;
    if (stage) load_runs(x, stage, a);
    const float sx = fmaxf(amax / 127.0f, 1e-12f);
    const float multiplier = 1.0f / sx;
#pragma unroll
    for (int g = 0; g < N / kRun; ++g) {
        const float* v = x + kRun * g;
        *reinterpret_cast<uint16_t*>(s.xq[buf] + kRun * run_of(g, a)) =
            (uint16_t)((quantize_one(v[0], multiplier) & 255) | ((quantize_one(v[1], multiplier) & 255) << 8));
    }
    if (a == 0) s.sx[buf] = sx;
    return true;
}

// Reference order streams the gated activation through LDS instead (its 48
// values per lane and the 64-bit words they arrive in would not fit the
// exchange waves' registers beside the rest): runs G0 .. G0 + N/kRun - 1 of
// the vector, once they carry `epoch`, go to `stage` (natural element order)
// and into the running maximum of |x|.
template <int N, int G0>
__device__ __forceinline__ bool await_staged(const u64* src, int n, unsigned epoch, float* stage, float& amax, int a,
                                             const StepParams& P) {
    float x[N];
    if (!await_runs<N, G0, false>(src, n, epoch, x, a, P)) return false;
    const int live = n / kRun - a - kAT * G0;
#pragma unroll
    for (int g = 0; g < N / kRun; ++g) {
        if (g * kAT < live) amax = fmaxf(amax, fmaxf(fabsf(x[kRun * g]), fabsf(x[kRun * g + 1])));
        *reinterpret_cast<v2f*>(stage + kRun * run_of(G0 + g, a)) = v2f{x[kRun * g], x[kRun * g + 1]};
    }
    return true;
}
// quantize_into for a vector staged by await_staged (amax: this lane's part).
template <int N>
__device__ __forceinline__ bool quantize_staged(const float* stage, int n, int buf, float amax, int a, Shared& s,
                                                int& round) {
    static_assert(N % kRun == 0 && kRun == 2, "runs of two");
    if (!a_max(amax, s, round)) return false;
    const float sx = fmaxf(amax / 127.0f, 1e-12f);
    const float multiplier = 1.0f / sx;
#pragma unroll
    for (int g = 0; g < N / kRun; ++g) {
        const v2f v = *reinterpret_cast<const v2f*>(stage + kRun * run_of(g, a));
        *reinterpret_cast<uint16_t*>(s.xq[buf] + kRun * run_of(g, a)) =
            (uint16_t)((quantize_one(v[0], multiplier) & 255) | ((quantize_one(v[1], multiplier) & 255) << 8));
    }
    if (a == 0) s.sx[buf] = sx;
    return true;
}

// gamma for this lane's runs; runs past n read the last one (their x are 0).
template <int N>
__device__ __forceinline__ void fetch_gamma(float (&g)[N], const float* gamma, int n, int a) {
    static_assert(N % kRun == 0 && kRun == 2, "runs of two");
#pragma unroll
    for (int q = 0; q < N / kRun; ++q) {
        const v2f v = ldg(reinterpret_cast<const v2f*>(gamma + kRun * min(run_of(q, a), n / kRun - 1)));
        g[kRun * q] = v[0];
        g[kRun * q + 1] = v[1];
    }
}

// -------------------------------------------------------- weight waves ---
// A row no wave of this block reads for real (not owned, or past the last
// layer) is still loaded, so that every phase issues the same loads on every
// path: that keeps the compiler's in-order wait counts exact across the
// layer loop (with a path that skips loads it must assume the worst and waits
// for every load in flight, next-layer prefetches included).  Such loads read
// one 16-byte chunk of row blockIdx.x, so the blocks spread them over
// different lines and memory channels.
__device__ __forceinline__ int spare_row(const WeightView& m) {
    return min((int)blockIdx.x, m.rows - 1);
}

// One int8 row of `m` into registers: lane holds chunks lane + 64 j.  Slots
// past the row end reload its last chunk (same cache line as a neighbour's
// load, so no extra traffic); row_dot ignores them.  Branch-free, so every
// load of a phase is in flight at once.
template <int KC>
__device__ __forceinline__ void load_row(v4u (&w)[KC], const WeightView& m, int row, int lane, bool live) {
    const int last = m.cols / 16 - 1;
    const uint8_t* base = static_cast<const uint8_t*>(m.data) + (size_t)(live ? row : spare_row(m)) * m.cols;
#pragma unroll
    for (int j = 0; j < KC; ++j) w[j] = ldg_stream(base + 16 * (live ? min(lane + kWave * j, last) : 0));
}

// Exact int32 dot of a register-held row with the int8 input in LDS, summed over the wave.
template <int KC>
__device__ __forceinline__ int row_dot(const v4u (&w)[KC], const int8_t* xq, int chunks, int lane) {
    int acc = 0;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
        const int c = lane + kWave * j;
        const v4u x = *reinterpret_cast<const v4u*>(xq + 16 * min(c, chunks - 1));
        int a = dot4((int)w[j].x, (int)x.x, 0);
        a = dot4((int)w[j].y, (int)x.y, a);
        a = dot4((int)w[j].z, (int)x.z, a);
        a = dot4((int)w[j].w, (int)x.w, a);
        acc += c < chunks ? a : 0;
    }
    return dpp_sum_i32(acc);
}

// This lane's part of the exact int32 dot of a register-held row with the
// int8 input chunks xc (chunk lane + 64 j of the input, read once per phase).
template <int KC>
__device__ __forceinline__ int row_part(const v4u (&w)[KC], const v4u (&xc)[KC], int chunks, int lane) {
    int acc = 0;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
        int a = dot4((int)w[j].x, (int)xc[j].x, 0);
        a = dot4((int)w[j].y, (int)xc[j].y, a);
        a = dot4((int)w[j].z, (int)xc[j].z, a);
        a = dot4((int)w[j].w, (int)xc[j].w, a);
        acc += lane + kWave * j < chunks ? a : 0;
    }
    return acc;
}

// Totals of eight rows' lane parts v[0..7], transposed: every lane of the
// 8-lane group l / 8 ends with the total of v[l / 8].  The rows fold pairwise
// across the wave halves (v[j] with v[j + 4], permlane32 swap), then across
// 16-lane rows (permlane16 swap), then within each 16-lane row (row_ror 8 with
// lane selects), then within the 8-lane groups (half-row mirror and quad
// permutes): 22 lane moves and adds instead of a full reduction per row.
// Integer sums, so the totals are exact whatever the order.
__device__ __forceinline__ int sum8_transposed(const int (&v)[8], int lane) {
    int u[4], w[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const auto p = __builtin_amdgcn_permlane32_swap((unsigned)v[j], (unsigned)v[j + 4], false, false);
        u[j] = (int)p[0] + (int)p[1];   // lanes 0-31: v[j] folded; lanes 32-63: v[j + 4] folded
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const auto p = __builtin_amdgcn_permlane16_swap((unsigned)u[j], (unsigned)u[j + 2], false, false);
        w[j] = (int)p[0] + (int)p[1];   // 16-lane rows 0..3: v[j], v[j + 2], v[j + 4], v[j + 6]
    }
    const bool high = (lane & 8) != 0;
    int g = (high ? w[1] : w[0]) + dpp<kDppRor8>(high ? w[0] : w[1]);   // 8-lane group k: v[k]
    g += dpp<kDppHalfMirror>(g);
    g += dpp<kDppXor2>(g);
    g += dpp<kDppXor1>(g);
    return g;
}

// Totals of two rows' lane parts: lanes 0-31 end with the total of v0,
// lanes 32-63 with that of v1 (permlane32 and permlane16 swaps, then four
// DPP steps within each 16-lane row).  Exact integer sums.
__device__ __forceinline__ int sum2_transposed(int v0, int v1) {
    const auto p = __builtin_amdgcn_permlane32_swap((unsigned)v0, (unsigned)v1, false, false);
    const int u = (int)p[0] + (int)p[1];
    const auto q = __builtin_amdgcn_permlane16_swap((unsigned)u, (unsigned)u, false, false);
    int g = (int)q[0] + (int)q[1];   // 16-lane rows 0, 1: v0 folded to 16 lanes; rows 2, 3: v1
    g += dpp<kDppRor8>(g);
    g += dpp<kDppHalfMirror>(g);
    g += dpp<kDppXor2>(g);
    g += dpp<kDppXor1>(g);
    return g;
}

// ---- Reference order: each weight wave quantizes the normalized input itself ---
// The exchange waves form only the column-order square sum of the RMSNorms
// before q|k|v and gate|up (ref_square_sum), the one step whose order the
// result depends on.  Meanwhile every weight wave quantizes the whole vector
// speculatively itself, lane l taking the 16-element chunks l + 64 j of its
// dots, and takes its int8 dots with those values; when the exact sum lands
// it confirms them.  The values (decoder.cpp:706-727, 1028-1043):
//   y = ((x - 0) * s) * g + 0,   t = y * (1 / max(max|y| / 127, 1e-12)),   q = rint(t) in [-127, 127].
// The int8 values do not depend on the RMSNorm scale s but through
// roundings: the speculation quantizes y~ = x * g instead (wave_speculate).
// Every y is y~ * s up to three roundings and so is max|y| (against max|y~|),
// so t/t~ lies within 12 units of roundoff (2^-24) of 1: |t| <= 127 moves by
// less than 1e-4.  An element more than kQuantMargin from a rounding boundary
// (a half-integer) therefore keeps its int8 value; the few nearer ones are
// quantized again with the exact scale (wave_confirm), and the exact maximum,
// which sets the per-token scale, is the largest |y| among the candidates
// |y~| >= max|y~| * kCandidate (no other element can reach it).  A changed
// value, two candidates in one lane, a maximum near the 1e-12 floor or a
// value that is not finite: the wave quantizes again with the exact scale
// (wave_quantize) and takes its dots again.  (Products x * s below the
// normal range would void the bound; they can only occur for elements whose
// t is below 1e-6, as long as no |gamma| exceeds 1e20, which the host checks
// before it runs this step.)
constexpr float kQuantMargin = 4e-4f;
constexpr float kCandidate = 1.0f - 1e-6f;

struct WaveQuant {
    float multiplier;    // 1 / the speculative per-token scale (wave-uniform)
    float amax;          // max |y~| over the vector (wave-uniform)
    float top, second;   // this lane's two largest |y~|
    int top_e;           // element of `top`
    unsigned near;       // this lane's elements near a rounding boundary (bit 16 j + i: chunk j, element i)
    bool odd;            // this lane holds a value that is not finite
};

// Four staged products of this lane's chunk j, elements 4 q .. 4 q + 3 (zero past the vector).
__device__ __forceinline__ v4f products4(const float* xg, int n, int lane, int j, int q) {
    const int c = lane + kWave * j;
    const bool live = c < n / 16;
    const v4f v = *reinterpret_cast<const v4f*>(xg + 20 * (live ? c : 0) + 4 * q);
    return live ? v : v4f{0.0f, 0.0f, 0.0f, 0.0f};
}

// The speculative int8 values of this lane's chunks (row_part's layout) from
// the staged products, and what wave_confirm needs.  The products are read
// twice (for the maximum, then for the quantization) rather than held in
// registers; the loops stay rolled for the same reason.
template <int KC>
__device__ __forceinline__ void wave_speculate(const float* xg, int n, int lane, v4u (&xc)[KC], WaveQuant& st) {
    float top = 0.0f, second = 0.0f;
    int top_e = 0;
    bool odd = false;
#pragma unroll 1
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const v4f y = products4(xg, n, lane, j, q);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float m = fabsf(y[k]);
                odd |= __builtin_amdgcn_class(y[k], 0x207);   // NaN, infinities
                const bool first = m > top;
                second = first ? top : fmaxf(second, m);
                top_e = first ? 16 * (lane + kWave * j) + 4 * q + k : top_e;
                top = first ? m : top;
            }
        }
    }
    const float amax = dpp_max_f32(top);
    const float multiplier = 1.0f / fmaxf(amax / 127.0f, 1e-12f);
    unsigned near = 0;
    v4u words[KC] = {};
#pragma unroll 1
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const v4f y = products4(xg, n, lane, j, q);
            unsigned word = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                // quantize_one, with the distance of t from the nearest integer
                const float t = y[k] * multiplier;
                const float r = __builtin_rintf(t);
                word |= (unsigned)((int)fminf(fmaxf(r, -127.0f), 127.0f) & 255) << (8 * k);
                near |= fabsf(t - r) > 0.5f - kQuantMargin ? 1u << (16 * j + 4 * q + k) : 0u;
            }
            words[j] = v4u{words[j][1], words[j][2], words[j][3], word};   // word q ends in slot q
        }
    }
#pragma unroll
    for (int j = 0; j < KC; ++j) xc[j] = words[j];
    st = WaveQuant{multiplier, amax, top, second, top_e, near, odd};
}

// Four normalized values of this lane's chunk j, elements 4 q .. 4 q + 3 (zero past the vector).
__device__ __forceinline__ v4f normalized4(const float* x, const float* gamma, int n, float scale, int lane, int j,
                                           int q) {
    const int c = lane + kWave * j;
    const bool live = c < n / 16;
    const int at = 16 * (live ? c : 0) + 4 * q;
    const v4f xv = *reinterpret_cast<const v4f*>(x + at);
    const v4f gv = *reinterpret_cast<const v4f*>(gamma + at);
    v4f y;
#pragma unroll
    for (int k = 0; k < 4; ++k) y[k] = live ? (xv[k] - 0.0f) * scale * gv[k] + 0.0f : 0.0f;
    return y;
}

// The exact int8 values of this lane's chunks (x and gamma in natural
// element order, `scale` the RMSNorm scale); returns the per-token scale.
template <int KC>
__device__ __forceinline__ float wave_quantize(const float* x, const float* gamma, int n, float scale, int lane,
                                               v4u (&xc)[KC]) {
    float top = 0.0f;
#pragma unroll 1
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const v4f y = normalized4(x, gamma, n, scale, lane, j, q);
#pragma unroll
            for (int k = 0; k < 4; ++k) top = fmaxf(top, fabsf(y[k]));
        }
    }
    const float sx = fmaxf(dpp_max_f32(top) / 127.0f, 1e-12f);
    const float multiplier = 1.0f / sx;
    v4u words[KC] = {};
#pragma unroll 1
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const v4f y = normalized4(x, gamma, n, scale, lane, j, q);
            unsigned word = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) word |= (unsigned)(quantize_one(y[k], multiplier) & 255) << (8 * k);
            words[j] = v4u{words[j][1], words[j][2], words[j][3], word};
        }
    }
#pragma unroll
    for (int j = 0; j < KC; ++j) xc[j] = words[j];
    return sx;
}

// Whether the int8 values wave_speculate formed are the ones the exact
// RMSNorm `scale` gives; sets sx, the vector's exact per-token scale.
__device__ __forceinline__ bool wave_confirm(const float* x, const float* gamma, const float* xg, float scale,
                                             const WaveQuant& st, int lane, float& sx) {
    const float bound = st.amax * kCandidate;
    const bool candidate = st.top >= bound;
    bool bad = st.odd || (candidate && st.second >= bound);
    float ye = 0.0f;
    if (candidate) {
        const int e = st.top_e;
        ye = fabsf((x[e] - 0.0f) * scale * gamma[e] + 0.0f);
    }
    const float amax = dpp_max_f32(ye);
    sx = fmaxf(amax / 127.0f, 1e-12f);
    const float multiplier = 1.0f / sx;
    for (unsigned m = st.near; m != 0; m &= m - 1) {
        const int i = __builtin_ctz(m);
        const int e = 16 * (lane + kWave * (i >> 4)) + (i & 15);
        bad |= quantize_one((x[e] - 0.0f) * scale * gamma[e] + 0.0f, multiplier) !=
               quantize_one(xg[xg_at(e)], st.multiplier);
    }
    // both maxima clear of the 1e-12 floor (NaN fails), the exact one finite
    const bool range = st.amax / 127.0f > 1e-11f && amax / 127.0f > 1e-11f && amax <= 3.0e38f;
    return range && __builtin_amdgcn_ballot_w64(bad) == 0;
}

// ((float)acc * s_x) * s_w + b  (decoder.cpp:568, 1229), separate roundings.
__device__ __forceinline__ float dequant(int acc, float sx, float sw, float bias) {
    const float term = (float)acc * sx;
    return term * sw + bias;
}

// Per-row scale and bias, fetched a layer ahead like the rows.
struct RowScale {
    float scale = 0.0f, bias = 0.0f;
    __device__ __forceinline__ void fetch(const WeightView& m, int r, bool live) {
        scale = ldg(m.scales + (live ? r : spare_row(m)));
        bias = ldg(m.bias + (live ? r : spare_row(m)));
    }
};

// Rows of rotate-half pair p of a stacked [q | k | v] projection: (i, i + rotary/2)
// in rotated heads, neighbouring rows elsewhere.
__device__ __forceinline__ void rope_rows(int p, int heads, int kv_heads, int rotary, int& r0, int& r1) {
    const int per_head = kStepDim / 2, half = rotary / 2;
    const int hb = p / per_head, j = p % per_head;
    const bool rotated = hb < heads + kv_heads;
    if (rotated && j < half) {
        r0 = hb * kStepDim + j;
        r1 = r0 + half;
    } else {
        const int base = rotated ? rotary : 0;
        r0 = hb * kStepDim + base + 2 * (rotated ? j - half : j);
        r1 = r0 + 1;
    }
}

__device__ __forceinline__ float activate(int activation, float x) {
    // Decoder::Impl::activate (decoder.cpp:982-987)
    if (activation == 0) return x / (1.0f + expf(-x));
    if (activation == 1) return 0.5f * x * (1.0f + erff(x * 0.7071067811865475f));
    if (activation == 2) return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
    return x < 0.0f ? 0.0f : x;
}

// glibc's expf with its table in LDS.
__device__ __forceinline__ float lds_expf(float x, const uint64_t* table) {
    return libm_expf_from(x, [table](uint32_t i) { return table[i]; });
}

// Decoder::Impl::activate in reference order: SiLU with glibc's expf, ReLU
// as std::max(x, 0.0f).  (The step runs reference order only for these two.)
__device__ __forceinline__ float ref_activate(int activation, float x, const uint64_t* exp2) {
    if (activation == 0) return x / (1.0f + lds_expf(-x, exp2));
    return x < 0.0f ? 0.0f : x;
}

__device__ __forceinline__ float embed_value(const WeightView& w, uint32_t id, int c) {
    const size_t index = (size_t)id * w.cols + c;
    if (w.bits == 32) return ldg(static_cast<const float*>(w.data) + index);
    return (float)ldg(static_cast<const int8_t*>(w.data) + index) * ldg(w.scales + id);
}

// A weight wave has issued the stores of its current phase.
__device__ __forceinline__ void note_published(Shared& s) {
    asm volatile("" ::: "memory");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(&s.published, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Waits (weight waves) until both exchange waves' flags reach `phase`.
__device__ __forceinline__ bool wait_flags(Shared& s, const int (&flag)[kA], int phase) {
    for (unsigned spin = 0;; ++spin) {
        if (min(lds_load(&flag[0]), lds_load(&flag[1])) >= phase) break;
        if (lds_load(&s.abort) || spin > 64 * kSpinLimit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");
    return true;
}
// ... until the exchange waves posted the int8 input of `phase`.
__device__ __forceinline__ bool wait_ready(Shared& s, int phase) { return wait_flags(s, s.ready, phase); }
// ... until they have read the input vector of `phase` (its hop is over).
// The weight waves issue a phase's next-layer loads only then: a burst of
// weight loads in flight slows the exchange reads of a hop down, while the
// norm and quantization that follow the hop need no memory.
__device__ __forceinline__ bool wait_received(Shared& s, int phase) { return wait_flags(s, s.received, phase); }

// Phase timeline: the first thread of each role stamps the 100 MHz device
// clock at phase boundaries into trace[block][point]: points 64 * layer + k
// (k < 8 exchange wave 0, 8 + 8 * w + j weight wave w, 56, 57, 60 inside
// attention, 58, 59, 61, 63 exchange wave 1's arrivals of x_attn, x_mid,
// the layer input and x_act), then the head's.  Off (null) outside
// diagnostics.
__device__ __forceinline__ void stamp(unsigned long long* trace, int block, int point, int thread = 0) {
    if (trace && threadIdx.x == thread)
        stg(trace + (size_t)block * kStepTracePoints + point, (unsigned long long)__builtin_amdgcn_s_memrealtime());
}

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// Where the rows of one block sit: q|k|v rotate-half pairs, o/down rows and
// gate|up pairs are split into contiguous ranges per block.
struct Ownership {
    int q_first, q_end, r_first, r_end, g_first, g_end;
    __device__ Ownership(const StepParams& P, int b, int G) {
        const int nq = (P.heads + 2 * P.kv_heads) * kStepDim / 2;
        q_first = (int)((long long)b * nq / G);
        q_end = (int)((long long)(b + 1) * nq / G);
        r_first = (int)((long long)b * P.hidden / G);
        r_end = (int)((long long)(b + 1) * P.hidden / G);
        g_first = (int)((long long)b * P.ffn / G);
        g_end = (int)((long long)(b + 1) * P.ffn / G);
    }
};

// Attention over this block's span of keys (K rows in s.k, V rows in s.v,
// q of the group's heads in s.q) for the wave's query heads h0 + aw,
// h0 + aw + kA, ... below h_end (HPW of them; heads past h_end repeat the
// last one, branch-free, so all heads' LDS reads overlap).  Fewer heads per
// wave leave registers for more LDS reads in flight: the loops are unrolled
// 8 / HPW times.  Publishes per head: max score, sum of
// exp(score - max), and the unnormalized output sum_k exp(s_k - max) v_k.
// Every staged row is finite: rows past the span hold key 0's values and get
// weight 0.
template <int HPW>
__device__ __forceinline__ void attention_item(const StepParams& P, Shared& s, int lane, int aw, int h0, int h_end,
                                               int keys, u64* parts, unsigned epoch, bool local,
                                               float* keep = nullptr) {
    // plain stores (they stay in this XCD's L2) for the XCD-local merge
    auto put = [&](u64* p, float v) {
        if (local) __hip_atomic_store((LEAF_GLOBAL u64*)p, tagged(epoch, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
        else publish(p, epoch, v);
    };
    constexpr int dim = kStepDim;
    // scores: lane = key, four dims of its K row at a time
    float sum[HPW];
#pragma unroll
    for (int h = 0; h < HPW; ++h) sum[h] = 0.0f;
#pragma unroll(8 / HPW)
    for (int d4 = 0; d4 < dim / 4; ++d4) {
        const v4f kv = *reinterpret_cast<const v4f*>(s.k + lane * kKStride + 4 * d4);
        v4f qv[HPW];
#pragma unroll
        for (int h = 0; h < HPW; ++h)
            qv[h] = *reinterpret_cast<const v4f*>(s.q + min(h0 + aw + kA * h, h_end - 1) * dim + 4 * d4);
        all_loaded(kv, qv);
#pragma unroll
        for (int h = 0; h < HPW; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) sum[h] = fmaf(qv[h][j], kv[j], sum[h]);
    }
    float m[HPW], l[HPW];
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
        const int gh = h0 + aw + kA * h;
        m[h] = -INFINITY;
        l[h] = 0.0f;
        if (gh < h_end) {
            const float sc = lane < keys ? sum[h] * P.attention_scale * P.attention_scale : -INFINITY;
            m[h] = dpp_max_f32(sc);
            const float e = lane < keys ? expf(sc - m[h]) : 0.0f;
            l[h] = dpp_sum_f32(e);
            s.e[gh * kStepSpanKeys + lane] = e;
        }
    }
    lds_done();   // each wave reads back only its own heads' weights
    // e . V: lane = dim, keys in order, V rows shared by the wave's heads
    float o[HPW];
#pragma unroll
    for (int h = 0; h < HPW; ++h) o[h] = 0.0f;
    const int keys4 = (keys + 3) & ~3;
#pragma unroll(8 / HPW)
    for (int kk = 0; kk < keys4; kk += 4) {
        v4f v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = s.v[(kk + j) * dim + lane];
        v4f e4[HPW];
#pragma unroll
        for (int h = 0; h < HPW; ++h)
            e4[h] = *reinterpret_cast<const v4f*>(s.e + min(h0 + aw + kA * h, h_end - 1) * kStepSpanKeys + kk);
        all_loaded(v, e4);
#pragma unroll
        for (int h = 0; h < HPW; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j) o[h] = fmaf(e4[h][j], v[j], o[h]);
    }
    if (keep) {
        // the caller folds the new key in and publishes (one head per wave)
        keep[0] = m[0];
        keep[1] = l[0];
        keep[2] = o[0];
        return;
    }
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
        const int gh = h0 + aw + kA * h;
        if (gh < h_end) {
            u64* part = parts + (size_t)gh * (dim + 2);
            put(part + 2 + lane, o[h]);
            if (lane == 0) {
                put(part, m[h]);
                put(part + 1, l[h]);
            }
        }
    }
}

// Reference order (attention_impl, transformer.cpp:112-143): an item only
// scores its span's keys for the wave's query heads, (q . k) * scale * scale
// with the dot summed over the dims in order and separate roundings
// (scalar_dot, :69-73), and publishes the raw scores in the span-partial
// layout: word 2 + key of each head's slot (lanes past the span's keys
// publish -inf), words 0 and 1 only the epoch.  The head's chain wave takes
// the maximum, the exponentials, the sequential denominator and the key-order
// output.  Rows of s.k past the span hold finite values that no score uses.
template <int HPW>
__device__ __forceinline__ void ref_score_item(const StepParams& P, Shared& s, int lane, int aw, int h0, int h_end,
                                               int keys, u64* parts, unsigned epoch, bool local) {
    auto put = [&](u64* p, float v) {
        if (local) __hip_atomic_store((LEAF_GLOBAL u64*)p, tagged(epoch, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
        else publish(p, epoch, v);
    };
    constexpr int dim = kStepDim;
    float sum[HPW];
#pragma unroll
    for (int h = 0; h < HPW; ++h) sum[h] = 0.0f;
    if constexpr (HPW <= 2) {
        // the next step's reads in flight while one is summed
        v4f kc, qc[HPW], kn, qn[HPW];
        auto read = [&](int d4, v4f& k, v4f (&q)[HPW]) {
            k = *reinterpret_cast<const v4f*>(s.k + lane * kKStride + 4 * d4);
#pragma unroll
            for (int h = 0; h < HPW; ++h)
                q[h] = *reinterpret_cast<const v4f*>(s.q + min(h0 + aw + kA * h, h_end - 1) * dim + 4 * d4);
        };
        read(0, kc, qc);
#pragma unroll 2
        for (int d4 = 0; d4 < dim / 4; ++d4) {
            read(min(d4 + 1, dim / 4 - 1), kn, qn);   // the last step reads its own again
            all_loaded(kc, qc);
#pragma unroll
            for (int h = 0; h < HPW; ++h)
#pragma unroll
                for (int j = 0; j < 4; ++j) sum[h] = sum[h] + qc[h][j] * kc[j];
            kc = kn;
#pragma unroll
            for (int h = 0; h < HPW; ++h) qc[h] = qn[h];
        }
    } else {
#pragma unroll(8 / HPW)
        for (int d4 = 0; d4 < dim / 4; ++d4) {
            const v4f kv = *reinterpret_cast<const v4f*>(s.k + lane * kKStride + 4 * d4);
            v4f qv[HPW];
#pragma unroll
            for (int h = 0; h < HPW; ++h)
                qv[h] = *reinterpret_cast<const v4f*>(s.q + min(h0 + aw + kA * h, h_end - 1) * dim + 4 * d4);
            all_loaded(kv, qv);
#pragma unroll
            for (int h = 0; h < HPW; ++h)
#pragma unroll
                for (int j = 0; j < 4; ++j) sum[h] = sum[h] + qv[h][j] * kv[j];
        }
    }
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
        const int gh = h0 + aw + kA * h;
        if (gh < h_end) {
            u64* part = parts + (size_t)gh * (dim + 2);
            put(part + 2 + lane, lane < keys ? sum[h] * P.attention_scale * P.attention_scale : -INFINITY);
            if (lane == 0) {
                put(part, 0.0f);
                put(part + 1, 0.0f);
            }
        }
    }
}

// Reference order, the rest of one query head's attention (attention_impl,
// transformer.cpp:122-143), by both exchange waves of its merge block (h: this
// wave): the scores of its n visible keys (pe[0], in the column-order sum's
// layout; m: this wave's maximum of those it gathered) -> the maximum (NaN
// scores never become it, as with std::max) -> exp(s - max) with glibc's
// expf, row blocks split between the waves -> the denominator summed in key
// order by the pair (wave_pair_sequential_sum) -> p = e / denominator, row
// groups split -> output[d] += p * v[d] in key order, lane d of wave 0.  Lane
// d loads column d of the cached V rows itself (one coalesced 256-byte row
// per load), kChainDepth chunks of kChainKeys keys in flight; the new key's
// row comes from the exchange words of q|k|v.  A fully masked or infinite row
// leaves the zero output, like the CPU.  Returns false (abort raised) when a
// wait failed; o is lane d's output element in wave 0.
constexpr int kChainKeys = 12;                                      // keys per chunk: three float4 of p
constexpr int kChainDepth = 4;                                      // chunks in flight (48 loads)
__device__ __forceinline__ bool ref_merge(const StepParams& P, SharedRef& r, int& round, int h, int n, float m,
                                          const float* V, const u64* vnew_word, unsigned vnew_epoch, int lane,
                                          float& o) {
    constexpr int dim = kStepDim;
    constexpr int kRowBytes = dim * (int)sizeof(float);
    o = 0.0f;
    float maximum = m;
    if (!a_max(maximum, r, round)) return false;
    if (!isfinite(maximum)) return true;
    float* pe = r.pe[0];
    float* pnat = r.v;   // p in key order
    const uint64_t* exp2 = r.exp2;
    const int E = seq_per_lane(n);
    const int valid = min(max(n - lane * E, 0), E);
    const int cached = n - 1;   // the new key is the last visible one
    const int chunks = (cached + kChainKeys - 1) / kChainKeys;
    const int groups = (chunks + kChainDepth - 1) / kChainDepth;
    // V rows through a bounds-checked buffer view of the cached rows: rows
    // past them read as 0, so the loads need no clamping.
    const __amdgpu_buffer_rsrc_t vbuf = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(V), (short)0, cached * kRowBytes, kRawBufferWord3);
    float ring[kChainDepth][kChainKeys];
    auto load = [&](float (&rr)[kChainKeys], int c) {
        const int at = lane * (int)sizeof(float) + c * kChainKeys * kRowBytes;
#pragma unroll
        for (int j = 0; j < kChainKeys; ++j)
            rr[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(vbuf, at + j * kRowBytes, 0, 0));
    };
    // exp(s - max) of this lane's keys (lane * E + i, at row i of column
    // lane): blocks of eight rows, the last one four (E is a multiple of 4),
    // alternating between the waves
    {
        auto exps = [&](auto width, int i0) {
            constexpr int W = decltype(width)::value;
            float e[W];
#pragma unroll
            for (int i = 0; i < W; ++i) e[i] = pe[(i0 + i) * kWave + lane] - maximum;
            libm_expf_batch(e, [exp2](uint32_t k) { return exp2[k]; });
            // every lane forms all of them (a select per key, no branch
            // around an evaluation)
#pragma unroll
            for (int i = 0; i < W; ++i) asm volatile("" : "+v"(e[i]));
#pragma unroll
            for (int i = 0; i < W; ++i) pe[(i0 + i) * kWave + lane] = i0 + i < valid ? e[i] : 0.0f;
        };
        int i0 = 8 * h;
        for (; i0 + 8 <= E; i0 += 16) exps(std::integral_constant<int, 8>(), i0);
        if (i0 < E) exps(std::integral_constant<int, 4>(), i0);
    }
    if (!a_sync(r, round)) return false;
    // wave 0: the first chunks' V columns load while the denominator is formed
    if (h == 0) {
#pragma unroll
        for (int u = 0; u < kChainDepth; ++u) load(ring[u], u);
    }
    float den;
    float4* xchg = reinterpret_cast<float4*>(&r.pe[1][0]);   // the pair's trade and compaction space
    if (!wave_pair_sequential_sum(pe, n, r.area[0], r.area[1], xchg, xchg + kSeqPairXchg + h * kSeqPairComp, h,
                                  [&] { return a_sync(r, round); }, den))
        return false;
    // p = e / den in key order (pnat), groups of four rows alternating between
    // the waves; the padding rows (e = +0) give p = +0 for keys [n, 64 E), and
    // the keys the last group of the chain runs past that (fewer than
    // kChainDepth * kChainKeys) +0 too
    for (int i0 = 4 * h; i0 < E; i0 += 8) {
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = pe[(i0 + i) * kWave + lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) pnat[lane * E + i0 + i] = e[i] / den;
    }
    if (h == 0 && kWave * E + lane < kRefMaxKeys) pnat[kWave * E + lane] = 0.0f;
    if (!a_sync(r, round)) return false;
    if (h != 0) return true;
    // Whole groups of kChainDepth chunks, one straight-line body per group:
    // a chunk's loads are replaced by those kChainDepth chunks on as soon as
    // it is added, and its p come from LDS two chunks ahead.  Keys from the
    // new one on add p * (+0) with p finite: their rows lie past the buffer
    // view's cached rows and read as 0, which leaves the sum unchanged (it
    // starts at +0 and is never -0).
    static_assert(kChainKeys % 4 == 0, "p loads are float4");
    static_assert((kChainDepth + 1) * kChainKeys <= kWave, "the zeroed p past 64 E cover what the last group reads");
    v4f pp[kChainDepth][kChainKeys / 4];
    auto read_p = [&](v4f (&pr)[kChainKeys / 4], int c) {
        const float* at = pnat + c * kChainKeys;   // < kRefMaxKeys: n <= kRefStepKeys
#pragma unroll
        for (int j = 0; j < kChainKeys / 4; ++j) pr[j] = *reinterpret_cast<const v4f*>(at + 4 * j);
    };
    read_p(pp[0], 0);
    read_p(pp[1], 1);
    for (int g = 0; g < groups; ++g) {
#pragma unroll
        for (int u = 0; u < kChainDepth; ++u) {
            const int c = g * kChainDepth + u;
            read_p(pp[(u + 2) % kChainDepth], c + 2);
            // one wait for the whole chunk: every product below reads the
            // values through this statement, which needs all of them loaded
            static_assert(kChainKeys == 12, "the statement names twelve values");
            float (&rr)[kChainKeys] = ring[u];
            v4f (&q)[kChainKeys / 4] = pp[u];
            asm volatile("" : "+v"(rr[0]), "+v"(rr[1]), "+v"(rr[2]), "+v"(rr[3]), "+v"(rr[4]), "+v"(rr[5]),
                              "+v"(rr[6]), "+v"(rr[7]), "+v"(rr[8]), "+v"(rr[9]), "+v"(rr[10]), "+v"(rr[11]),
                              "+v"(q[0]), "+v"(q[1]), "+v"(q[2]));
#pragma unroll
            for (int j = 0; j < kChainKeys; ++j) o = o + pp[u][j / 4][j % 4] * ring[u][j];
            load(ring[u], c + kChainDepth);
        }
    }
    lds_done();
    float vnew;
    if (!await_one(vnew_word, true, vnew_epoch, vnew, P)) return false;
    o = o + pnat[cached] * vnew;
    return true;
}

// How a step lays out its attention (both roles compute the same plan).
// Items are (KV head, span of keys, slice of the group's query heads);
// slices are as narrow as the grid allows (hpw heads per exchange wave).
// Local mode deals the head slices to the XCDs round robin (slice sigma to
// XCD sigma % 8): its span items and its merge block run there and the span
// partials go through that XCD's L2.  Local q also computes a slice's q rows
// on its XCD (each block of XCD x owns `qkv_per_block` consecutive entries of
// the list: q pairs of slices x, x + 8, ..., then 1/8 of the k|v pairs), so
// the items read q from L2 as well; the new key's k and v still travel
// through memory, and an item folds that key in after its cached keys.
struct AttnPlan {
    int begin, end, spans, hpw, slices, S, per;
    bool local, local_q;
    int qkv_per_xcd, qkv_per_block;
};
__device__ __forceinline__ AttnPlan attn_plan(const StepParams& P, int G) {
    AttnPlan a;
    const int group = P.heads / P.kv_heads;
    a.end = P.position + 1;
    a.begin = (P.window > 0 && a.end > P.window) ? a.end - P.window : 0;
    a.spans = (a.end - a.begin + kStepSpanKeys - 1) / kStepSpanKeys;
    a.hpw = 1;
    while (a.hpw < kHeadsA && a.hpw < P.item_heads) a.hpw *= 2;
    while (a.hpw < kHeadsA && P.kv_heads * a.spans * ((group + kA * a.hpw - 1) / (kA * a.hpw)) > G) a.hpw *= 2;
    a.slices = (group + kA * a.hpw - 1) / (kA * a.hpw);
    a.S = P.kv_heads * a.slices;
    a.per = a.S / 8;
    a.local = P.x_part_local && a.hpw == 1 && G % 8 == 0 && a.S % 8 == 0 && a.per * a.spans <= G / 8;
    constexpr int pairs_per_head = kStepDim / 2;
    a.qkv_per_xcd = a.per * kA * pairs_per_head + 2 * P.kv_heads * pairs_per_head / 8;
    a.qkv_per_block = G >= 8 ? (a.qkv_per_xcd + G / 8 - 1) / (G / 8) : 0;
    a.local_q = a.local && P.x_q_local && group % kA == 0 && a.qkv_per_block <= kQP * kB;
    return a;
}

// Rotate-half pair `i` (of the plan's qkv_per_block) of block b in local-q
// mode, or -1 past the block's share.
__device__ __forceinline__ int local_qkv_pair(const AttnPlan& a, const StepParams& P, int b, int i) {
    constexpr int pairs_per_head = kStepDim / 2;
    const int group = P.heads / P.kv_heads;
    const int x = b & 7, e = (b >> 3) * a.qkv_per_block + i;
    if (i >= a.qkv_per_block || e >= a.qkv_per_xcd) return -1;
    const int qpairs = a.per * kA * pairs_per_head;
    if (e < qpairs) {
        const int sigma = x + 8 * (e / (kA * pairs_per_head)), w = e % (kA * pairs_per_head);
        const int head = sigma / a.slices * group + sigma % a.slices * kA + w / pairs_per_head;
        return head * pairs_per_head + w % pairs_per_head;
    }
    return P.heads * pairs_per_head + x * (2 * P.kv_heads * pairs_per_head / 8) + (e - qpairs);
}

// ======================================================= exchange role ===
// Diagnostics (CAP): block 0 records phase `phase` of layer L -- this lane's
// runs of the f32 vector it quantized, their int8 values (read back from the
// LDS runs this lane wrote) and the scale.
template <bool CAP, int N>
__device__ __forceinline__ void capture_input(const StepParams& P, const Shared& s, const float (&x)[N], int n,
                                              int buf, int L, int phase, int a) {
    if constexpr (CAP) {
        if (blockIdx.x != 0) return;
        const size_t at = ((size_t)L * 4 + phase) * kStepMaxFfn;
#pragma unroll
        for (int g = 0; g < N / kRun; ++g)
#pragma unroll
            for (int j = 0; j < kRun; ++j) {
                const int e = kRun * run_of(g, a) + j;
                if (e < n) {
                    P.capture.x[at + e] = x[kRun * g + j];
                    P.capture.q[at + e] = s.xq[buf][e];
                }
            }
        if (a == 0) P.capture.sx[L * 4 + phase] = s.sx[buf];
    }
}

// Block 0's record of a weight wave's normalized input (reference order):
// the values from the exact scale, the int8 values its dots used and the
// per-token scale (CAP only).
template <bool CAP, int KC>
__device__ __forceinline__ void capture_wave_input(const StepParams& P, const float* x, const float* gamma, int n,
                                                   float scale, const v4u (&xc)[KC], float sx, int L, int phase,
                                                   int lane) {
    if constexpr (CAP) {
        if (blockIdx.x != 0) return;
        const size_t at = ((size_t)L * 4 + phase) * kStepMaxFfn;
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const int c = lane + kWave * j;
            if (c >= n / 16) continue;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int e = 16 * c + i;
                P.capture.x[at + e] = (x[e] - 0.0f) * scale * gamma[e] + 0.0f;
                P.capture.q[at + e] = (int8_t)(xc[j][i / 4] >> (8 * (i % 4)));
            }
        }
        if (lane == 0) P.capture.sx[L * 4 + phase] = sx;
    }
}

// The exact int32 dot of output row `row` of phase `phase` (CAP only).
template <bool CAP>
__device__ __forceinline__ void capture_acc(const StepParams& P, int L, int phase, int row, int acc) {
    if constexpr (CAP) P.capture.acc[((size_t)L * 4 + phase) * (2 * kStepMaxFfn) + row] = acc;
}

// Returns false when the kernel is abandoned (abort).
template <bool CAP, bool REF>
__device__ __forceinline__ bool exchange_role(const StepParams& P, Shared& s) {
    int a = threadIdx.x;                     // 0 .. kAT - 1
    const int G = gridDim.x, b = blockIdx.x;
    const int H = P.hidden, F = P.ffn, dim = kStepDim;
    const int qw = P.heads * dim, kvw = P.kv_heads * dim;
    const int group = P.heads / P.kv_heads;
    const int pos = P.position;
    int round = 0;
    auto epoch = [&](int layer, int phase) { return P.epoch + (unsigned)(layer * 8 + phase); };

    // this block's attention item: (KV head, span of keys, slice of the
    // group's query heads).  Slices are as narrow as the grid allows (hpw
    // heads per exchange wave): an item's time grows with its heads.
    const AttnPlan plan = attn_plan(P, G);
    const int end = plan.end, begin = plan.begin, spans = plan.spans, hpw = plan.hpw, slices = plan.slices;
    const int per = plan.per;
    const bool local = plan.local;
    int sigma = -1, merge_sigma = -1;      // this block's item slice and merge slice (local mode)
    bool has_item;
    int item_g, item_s, item_h0;
    if (local) {
        const int x = b & 7, k = b >> 3;
        has_item = k < per * spans;
        sigma = has_item ? x + 8 * (k / spans) : 0;
        item_g = sigma / slices;
        item_s = has_item ? k % spans : 0;
        item_h0 = sigma % slices * kA;
        if (k >= G / 8 - per) merge_sigma = x + 8 * (G / 8 - 1 - k);
    } else {
        has_item = b < P.kv_heads * spans * slices;
        item_g = has_item ? b / (spans * slices) : 0;
        item_s = has_item ? b / slices % spans : 0;
        item_h0 = has_item ? b % slices * kA * hpw : 0;
    }
    const int item_h1 = min(group, item_h0 + kA * hpw);
    const int k0 = begin + item_s * kStepSpanKeys, k1 = min(end, k0 + kStepSpanKeys);
    const int cached_end = min(k1, pos), keys = k1 - k0;
    const bool new_key = pos >= k0 && pos < k1;
    // merge blocks: the last ceil(heads / kA) blocks, one query head per wave
    // (local mode: the last `per` blocks of each XCD, one head slice each)
    const bool merge_block = local ? merge_sigma >= 0 : (G - 1 - b) * kA < P.heads;
    // reference order: the last `heads` blocks merge one query head each, with
    // both exchange waves (local mode: the last per * kA blocks of each XCD,
    // one head of the XCD's slices each)
    int ref_mh = -1;
    if (REF) {
        if (local) {
            const int idx = G / 8 - 1 - (b >> 3);
            if (idx >= 0 && idx < per * kA) {
                const int sl = (b & 7) + 8 * (idx / kA), hs = idx % kA;
                if (sl % slices * kA + hs < group) ref_mh = sl / slices * group + sl % slices * kA + hs;
            }
        } else if (G - 1 - b < P.heads) {
            ref_mh = G - 1 - b;
        }
    }
    u64* const part_base = local ? P.x_part_local : P.x_part;

    float x[kNH];
    {
        // The input norm's gamma waits in LDS (each lane reads back its own
        // runs): a cold read of it after the layer input lands would add a
        // memory round trip to every layer.
        float gamma[kNH];
        fetch_gamma(gamma, layer_at(s, 0).input_gamma, H, a);
        store_runs(s.gamma_in, gamma, a);
    }
    {
        const uint32_t id = ldg(P.token);
#pragma unroll
        for (int i = 0; i < kNH; ++i) {
            const int e = kRun * run_of(i / kRun, a) + i % kRun;
            x[i] = e < H ? embed_value(P.embedding, id, e) * P.embedding_scale : 0.0f;
        }
    }
    for (int L = 0; L < P.layers; ++L) {
        // A fresh copy of the lane index per layer keeps per-lane address
        // arithmetic inside the loop instead of hoisting dozens of 64-bit
        // addresses into registers for the whole kernel.
        asm volatile("" : "+v"(a));
        const int lane = a & 63, aw = __builtin_amdgcn_readfirstlane(a >> 6);   // aw: wave-uniform
        const StepLayer& Ly = layer_at(s, L);
        const float* Kc = P.kv + (size_t)L * 2 * P.kv_heads * P.capacity * dim;
        const float* Vc = Kc + (size_t)P.kv_heads * P.capacity * dim;
        float gamma[kNH];
        load_runs(gamma, s.gamma_in, a);

        // ---- layer input (x, polled at the end of the previous layer) -> RMSNorm -> int8 for q|k|v
        stamp(P.trace, b, 64 * L + 1);
        stamp(P.trace, b, 64 * L + 61, kWave);
        // cached keys and values of this block's span (rows past the cached
        // ones load key 0 again; they are overwritten or never read)
        v4u kv_pre[2 * kNK] = {};
        if (has_item) {
#pragma unroll
            for (int j = 0; j < kNK; ++j) {
                const int f = a + kAT * j, key = k0 + f / 16, part = f % 16;   // 16 float4 per 64-float row
                const size_t at = ((size_t)item_g * P.capacity + (key < cached_end ? key : 0)) * dim + 4 * part;
                kv_pre[j] = ldg(reinterpret_cast<const v4u*>(Kc + at));
                kv_pre[kNK + j] = ldg(reinterpret_cast<const v4u*>(Vc + at));
            }
        }
        store_runs(s.h_in, x, a);
        if constexpr (REF) {
            // the weight waves normalize and quantize; this is the exact sum for them
            SharedRef& r = static_cast<SharedRef&>(s);
            stage_products(r, x, gamma, a, 4 * L + 0);
            float sq;
            if (!ref_square_sum(x, H, a, s, round, sq)) return false;
            if (a == 0) r.sq[0] = sq;
        } else {
            if (!rms_normalize<REF>(x, H, gamma, P.epsilon, a, s, round) || !quantize_into(x, H, 0, a, s, round))
                return false;
            capture_input<CAP>(P, s, x, H, 0, L, 0, a);
        }
        post(s, 4 * L + 0);
        stamp(P.trace, b, 64 * L + 2);
        if (has_item) {
            // the cached keys and values, loaded during the norm, into LDS
#pragma unroll
            for (int j = 0; j < kNK; ++j) {
                const int f = a + kAT * j, kl = f / 16, part = f % 16;
                *reinterpret_cast<v4u*>(s.k + kl * kKStride + 4 * part) = kv_pre[j];
                *reinterpret_cast<v4u*>(s.v + kl * dim + 4 * part) = kv_pre[kNK + j];
            }
        }

        // ---- attention, flash-decoding style: item blocks score one KV
        // head's span of keys for all heads of its group and publish (max,
        // sum, unnormalized output) per head; merge waves (one per query head,
        // in the last blocks) combine the spans as soon as they land.
        if (has_item && plan.local_q) {
            // q of this item's kA heads from this XCD's L2; the span's
            // cached keys first, then (last span) the new key folded in
            const int kv_word = a < dim ? qw + item_g * dim + a : qw + kvw + item_g * dim + (a - dim);
            float got2[2];
            const bool ok_q = wait_published(s, 4 * L + 1) &&
                              await_runs<2, 0, false>(P.x_q_local + (item_g * group + item_h0) * dim, kA * dim,
                                                      epoch(L, 1), got2, a, P);
            if (!a_check(ok_q, s, P)) return false;
            stamp(P.trace, b, 64 * L + 3);
            if (a < kA * dim / 2) *reinterpret_cast<v2f*>(s.q + item_h0 * dim + 2 * a) = v2f{got2[0], got2[1]};
            if constexpr (REF) {
                // the new key's k joins the staged rows before the scores
                float kv_got;
                if (!a_check(await_one(P.x_qkv + kv_word, new_key && a < dim, epoch(L, 1), kv_got, P), s, P))
                    return false;
                if (new_key && a < dim) s.k[(pos - k0) * kKStride + a] = kv_got;
                if (!a_sync(s, round)) return false;
                stamp(P.trace, b, 64 * L + 56);
                u64* parts = part_base + (size_t)(item_g * spans + item_s) * group * (dim + 2);
                ref_score_item<1>(P, s, lane, aw, item_h0, item_h1, keys, parts, epoch(L, 2), true);
                stamp(P.trace, b, 64 * L + 57);
            } else {
                if (!a_sync(s, round)) return false;
                stamp(P.trace, b, 64 * L + 56);
                float keep[3];
                attention_item<1>(P, s, lane, aw, item_h0, item_h1, keys - (new_key ? 1 : 0), nullptr, epoch(L, 2),
                                  true, keep);
                float m = keep[0], l = keep[1], o = keep[2];
                if (new_key) {
                    float kv_got;
                    if (!a_check(await_one(P.x_qkv + kv_word, a < 2 * dim, epoch(L, 1), kv_got, P), s, P)) return false;
                    if (!a_sync(s, round)) return false;   // both waves are done with the cached rows
                    const int nl = pos - k0;
                    if (a < dim) s.k[nl * kKStride + a] = kv_got;
                    else s.v[nl * dim + (a - dim)] = kv_got;
                    if (!a_sync(s, round)) return false;
                    // fold key nl in: rescale the cached keys' partials to the new max
                    const int gh = min(item_h0 + aw, item_h1 - 1);
                    const float qd = s.q[gh * dim + lane], kd = s.k[nl * kKStride + lane], vd = s.v[nl * dim + lane];
                    const float sn = dpp_sum_f32(qd * kd) * P.attention_scale * P.attention_scale;
                    const float mn = fmaxf(m, sn);
                    const float alpha = expf(m - mn), beta = expf(sn - mn);
                    l = l * alpha + beta;
                    o = fmaf(o, alpha, beta * vd);
                    m = mn;
                }
                const int gh = item_h0 + aw;
                if (gh < item_h1) {
                    u64* part = part_base + ((size_t)(item_g * spans + item_s) * group + gh) * (dim + 2);
                    const unsigned e2 = epoch(L, 2);
                    __hip_atomic_store((LEAF_GLOBAL u64*)(part + 2 + lane), tagged(e2, o), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_WAVEFRONT);
                    if (lane == 0) {
                        __hip_atomic_store((LEAF_GLOBAL u64*)part, tagged(e2, m), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WAVEFRONT);
                        __hip_atomic_store((LEAF_GLOBAL u64*)(part + 1), tagged(e2, l), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WAVEFRONT);
                    }
                }
                stamp(P.trace, b, 64 * L + 57);
            }
        } else if (has_item) {
            // q of the group's heads, and the new key's k (lanes < dim) or v
            // (the q|k|v buffer is padded so a lane's runs stay inside it)
            float got[kNQ - 1], kv_got;
            const int q_base = item_g * group * dim;
            const int kv_word = a < dim ? qw + item_g * dim + a : qw + kvw + item_g * dim + (a - dim);
            const bool has_kv = new_key && a < 2 * dim;
            const bool ok_q = wait_published(s, 4 * L + 1) &&
                              await_runs<kNQ - 1, 0, false>(P.x_qkv + q_base, group * dim, epoch(L, 1), got, a, P);
            const bool ok_kv = ok_q && await_one(P.x_qkv + kv_word, has_kv, epoch(L, 1), kv_got, P);
            if (!a_check(ok_kv, s, P)) return false;
            stamp(P.trace, b, 64 * L + 3);
            store_runs(s.q, got, a);
            if (has_kv) {
                const int nl = pos - k0;
                if (a < dim) s.k[nl * kKStride + a] = kv_got;
                else s.v[nl * dim + (a - dim)] = kv_got;
            }
            if (!a_sync(s, round)) return false;
            stamp(P.trace, b, 64 * L + 56);
            u64* parts = part_base + (size_t)(item_g * spans + item_s) * group * (dim + 2);
            if constexpr (REF) {
                if (hpw == 1) ref_score_item<1>(P, s, lane, aw, item_h0, item_h1, keys, parts, epoch(L, 2), local);
                else if (hpw == 2) ref_score_item<2>(P, s, lane, aw, item_h0, item_h1, keys, parts, epoch(L, 2), false);
                else if (hpw == 4) ref_score_item<4>(P, s, lane, aw, item_h0, item_h1, keys, parts, epoch(L, 2), false);
                else ref_score_item<kHeadsA>(P, s, lane, aw, item_h0, item_h1, keys, parts, epoch(L, 2), false);
            } else {
                if (hpw == 1) attention_item<1>(P, s, lane, aw, item_h0, item_h1, keys, parts, epoch(L, 2), local);
                else if (hpw == 2) attention_item<2>(P, s, lane, aw, item_h0, item_h1, keys, parts, epoch(L, 2), false);
                else if (hpw == 4) attention_item<4>(P, s, lane, aw, item_h0, item_h1, keys, parts, epoch(L, 2), false);
                else attention_item<kHeadsA>(P, s, lane, aw, item_h0, item_h1, keys, parts, epoch(L, 2), false);
            }
            stamp(P.trace, b, 64 * L + 57);
        }
        if (REF && ref_mh >= 0) {
            // reference order: both exchange waves on query head ref_mh
            bool ok = true;
            const int g = ref_mh / group, gh = ref_mh % group;
            const size_t stride = (size_t)group * (dim + 2);
            const u64* base = part_base + ((size_t)g * spans * group + gh) * (dim + 2);
            SharedRef& r = static_cast<SharedRef&>(s);
            float* pe = r.pe[0];
            const int n = end - begin;
            float m = -INFINITY;
            v2f ml;
            float os[kMergeBatch];
            const SeqLayout lay(n);
            // the waves gather alternate batches of spans
            for (int s0 = aw * kMergeBatch; s0 < spans && ok; s0 += kA * kMergeBatch) {
                ok = await_partials(base, (int)stride, spans, s0, lane, epoch(L, 2), ml, os, P);
#pragma unroll
                for (int j = 0; j < kMergeBatch; ++j) {
                    const int k = (s0 + j) * kStepSpanKeys + lane;
                    if (ok && k < n) {
                        pe[lay.at(k)] = os[j];
                        m = m < os[j] ? os[j] : m;
                    }
                }
            }
            if (!a_check(ok, s, P)) return false;
            float o = 0.0f;
            ok = ref_merge(P, r, round, aw, n, m, Vc + ((size_t)g * P.capacity + begin) * dim,
                           P.x_qkv + qw + kvw + g * dim + lane, epoch(L, 1), lane, o);
            if (ok && aw == 0) publish(P.x_attn + ref_mh * dim + lane, epoch(L, 3), o);
            if (!a_check(ok, s, P)) return false;
            stamp(P.trace, b, 64 * L + 60);
        } else if (!REF && merge_block) {
            // this wave's query head mh: combine its spans (lane s holds span
            // s's max and sum; lane d accumulates output element d)
            bool ok = true;
            const int mh = local ? merge_sigma / slices * group + merge_sigma % slices * kA + aw : (G - 1 - b) * kA + aw;
            const bool mine = local ? merge_sigma % slices * kA + aw < group : mh < P.heads;
            if (mine) {
                const int g = mh / group, gh = mh % group;
                const size_t stride = (size_t)group * (dim + 2);
                const u64* base = part_base + ((size_t)g * spans * group + gh) * (dim + 2);
                // One read takes every (max, sum) pair and the first
                // kMergeBatch spans' outputs; later batches are read as needed.
                v2f ml;
                float os[kMergeBatch];
                ok = await_partials(base, (int)stride, spans, 0, lane, epoch(L, 2), ml, os, P);
                const float ms = lane < spans ? ml[0] : -INFINITY;
                const float mx = dpp_max_f32(ms);
                const float weight = lane < spans ? expf(ms - mx) : 0.0f;
                const float total = dpp_sum_f32(lane < spans ? ml[1] * weight : 0.0f);
                float acc = 0.0f;
                for (int s0 = 0; s0 < spans && ok; s0 += kMergeBatch) {
                    if (s0 > 0) ok = await_partials(base, (int)stride, spans, s0, lane, epoch(L, 2), ml, os, P);
#pragma unroll
                    for (int j = 0; j < kMergeBatch; ++j) {
                        const float wj = __builtin_bit_cast(
                            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, weight), (s0 + j) & 63));
                        acc = s0 + j < spans ? fmaf(os[j], wj, acc) : acc;
                    }
                }
                if (ok) publish(P.x_attn + mh * dim + lane, epoch(L, 3), total > 0.0f ? acc / total : 0.0f);
            }
            if (!a_check(ok, s, P)) return false;
            stamp(P.trace, b, 64 * L + 60);
        }
        stamp(P.trace, b, 64 * L + 4);

        // ---- attention output -> int8 for o_proj
        {
            float xa[kNH];
            if (!a_check(await_runs<kNH>(P.x_attn, qw, epoch(L, 3), xa, a, P), s, P)) return false;
            note_received(s, 4 * L + 1);
            stamp(P.trace, b, 64 * L + 5);
            stamp(P.trace, b, 64 * L + 58, kWave);
            if (!quantize_into(xa, qw, 1, a, s, round)) return false;
            capture_input<CAP>(P, s, xa, qw, 1, L, 1, a);
            post(s, 4 * L + 1);
        }
        // ---- after o_proj -> RMSNorm -> int8 for gate|up
        fetch_gamma(gamma, Ly.post_gamma, H, a);
        {
            // the next norm's gamma (the next layer's input norm, or the final one)
            float next[kNH];
            fetch_gamma(next, L + 1 < P.layers ? layer_at(s, L + 1).input_gamma : P.final_gamma, H, a);
            if (!a_check(wait_published(s, 4 * L + 2) && await_runs<kNH, 0, false>(P.x_mid, H, epoch(L, 4), x, a, P), s, P))
                return false;
            note_received(s, 4 * L + 2);
            store_runs(s.gamma_in, next, a);
        }
        stamp(P.trace, b, 64 * L + 6);
        stamp(P.trace, b, 64 * L + 59, kWave);
        store_runs(s.h_mid, x, a);
        if constexpr (REF) {
            SharedRef& r = static_cast<SharedRef&>(s);
            store_runs(r.gamma_mid, gamma, a);
            stage_products(r, x, gamma, a, 4 * L + 2);
            float sq;
            if (!ref_square_sum(x, H, a, s, round, sq)) return false;
            if (a == 0) r.sq[1] = sq;
        } else {
            if (!rms_normalize<REF>(x, H, gamma, P.epsilon, a, s, round) || !quantize_into(x, H, 0, a, s, round))
                return false;
            capture_input<CAP>(P, s, x, H, 0, L, 2, a);
        }
        post(s, 4 * L + 2);
        // ---- SiLU-gated activation -> int8 for down_proj
        {
            bool ok = wait_published(s, 4 * L + 3);
            if constexpr (REF) {
                float* st = static_cast<SharedRef&>(s).stage();
                float amax = 0.0f;
                ok = ok && await_staged<kNF / 4, 0>(P.x_act, F, epoch(L, 5), st, amax, a, P);
                ok = ok && await_staged<kNF / 4, kNF / 4 / kRun>(P.x_act, F, epoch(L, 5), st, amax, a, P);
                ok = ok && await_staged<kNF / 4, kNF / 2 / kRun>(P.x_act, F, epoch(L, 5), st, amax, a, P);
                ok = ok && await_staged<kNF / 4, 3 * kNF / 4 / kRun>(P.x_act, F, epoch(L, 5), st, amax, a, P);
                stamp(P.trace, b, 64 * L + 63, kWave);
                if (!a_check(ok, s, P)) return false;
                note_received(s, 4 * L + 3);
                stamp(P.trace, b, 64 * L + 7);
                if (!quantize_staged<kNF>(st, F, 1, amax, a, s, round)) return false;
                if constexpr (CAP) {
                    float xd[kNF];
                    load_runs(xd, st, a);
                    capture_input<CAP>(P, s, xd, F, 1, L, 3, a);
                }
            } else {
                float xd[kNF];
                ok = ok && await_runs<kNF, 0, false>(P.x_act, F, epoch(L, 5), xd, a, P);
                stamp(P.trace, b, 64 * L + 63, kWave);
                if (!a_check(ok, s, P)) return false;
                note_received(s, 4 * L + 3);
                stamp(P.trace, b, 64 * L + 7);
                if (!quantize_into(xd, F, 1, a, s, round)) return false;
                capture_input<CAP>(P, s, xd, F, 1, L, 3, a);
            }
            post(s, 4 * L + 3);
        }
        // ---- the next layer's input (the last layer's feeds the head below)
        if (L + 1 < P.layers) {
            stamp(P.trace, b, 64 * (L + 1) + 0);
            if (!a_check(wait_published(s, 4 * L + 4) && await_runs<kNH, 0, false>(P.x_hidden, H, epoch(L, 6), x, a, P), s, P))
                return false;
            note_received(s, 4 * L + 4);
        }
    }
    // ---- final RMSNorm -> FP32 input of the head
    {
        float gamma[kNH];
        load_runs(gamma, s.gamma_in, a);
        stamp(P.trace, b, 64 * P.layers + 0);
        if (!a_check(wait_published(s, 4 * P.layers) &&
                         await_runs<kNH, 0, false>(P.x_hidden, H, epoch(P.layers - 1, 6), x, a, P), s, P))
            return false;
        note_received(s, 4 * P.layers);
        stamp(P.trace, b, 64 * P.layers + 1);
        if (!rms_normalize<REF>(x, H, gamma, P.epsilon, a, s, round)) return false;
        // (reference order: the other wave may still be reading its squares from s.xf)
        if (REF && !a_sync(s, round)) return false;
        store_runs(s.xf, x, a);
        post(s, 4 * P.layers);
    }
    return true;
}

// ========================================================= weight role ===
struct LayerRows {
    v4u q[kQP][2][kKCH];
    v4u o[kOR][kKCH];
    v4u g[kGP][2][kKCH];
    v4u d[kOR][kKCF];
    RowScale qs[kQP][2];
    RowScale os, ds;   // per lane: o / down row k = lane / 32 of this wave
    RowScale gs;   // per lane: the gate|up row whose total this lane's 8-lane group holds
};

template <bool CAP, bool REF>
__device__ __forceinline__ bool weight_role(const StepParams& P, Shared& s) {
    const int t = threadIdx.x, lane = t & 63;
    const int bw = __builtin_amdgcn_readfirstlane((t >> 6) - kA);   // 0 .. kB - 1, wave-uniform
    const int G = gridDim.x, b = blockIdx.x;
    const int H = P.hidden, F = P.ffn, dim = kStepDim;
    const int pos = P.position;
    auto epoch = [&](int layer, int phase) { return P.epoch + (unsigned)(layer * 8 + phase); };
    const Ownership own(P, b, G);

    const AttnPlan plan = attn_plan(P, G);
    int qr[kQP][2];
    bool has_q[kQP], has_r[kOR], has_g[kGP];
    float rope_c[kQP], rope_s[kQP];
#pragma unroll
    for (int k = 0; k < kQP; ++k) {
        const int p = plan.local_q ? local_qkv_pair(plan, P, b, bw + kB * k) : own.q_first + bw + kB * k;
        has_q[k] = plan.local_q ? p >= 0 : p < own.q_end;
        qr[k][0] = qr[k][1] = 0;
        rope_c[k] = 1.0f;
        rope_s[k] = 0.0f;
        if (has_q[k]) {
            rope_rows(p, P.heads, P.kv_heads, P.rotary, qr[k][0], qr[k][1]);
            const int half = P.rotary / 2, i0 = qr[k][0] % dim;
            if (qr[k][0] / dim < P.heads + P.kv_heads && i0 < half) {
                rope_c[k] = ldg(P.cosines + (size_t)pos * half + i0);
                rope_s[k] = ldg(P.sines + (size_t)pos * half + i0);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < kOR; ++k) has_r[k] = own.r_first + bw + kB * k < own.r_end;
#pragma unroll
    for (int k = 0; k < kGP; ++k) has_g[k] = own.g_first + bw + kB * k < own.g_end;
    static_assert(kGP == 4, "gate|up totals are reduced eight rows at a time");
    static_assert(kOR == 2, "o and down totals are reduced two rows at a time");
    // This lane's o / down row after sum2_transposed: lanes 0-31 hold row 0
    // of the wave, lanes 32-63 row 1.
    const int r_row = own.r_first + bw + kB * (lane >> 5);
    const bool r_live = r_row < own.r_end;
    // This lane's gate|up row after sum8_transposed: 8-lane groups 0-3 hold
    // the gate rows of pairs 0-3, groups 4-7 their up rows.
    const int g_pair = own.g_first + bw + kB * ((lane >> 3) & 3);
    const bool g_live = g_pair < own.g_end;
    const int g_row = (lane < 32 ? 0 : F) + g_pair;

    LayerRows w;
    // Loads of one phase's rows; `more` false loads nothing useful (the last
    // layer has no successor) but keeps the load count of every path equal.
    auto load_qkv = [&](const StepLayer& Ly, bool more) {
#pragma unroll
        for (int k = 0; k < kQP; ++k)
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                load_row(w.q[k][r], Ly.qkv, qr[k][r], lane, has_q[k] && more);
                w.qs[k][r].fetch(Ly.qkv, qr[k][r], has_q[k] && more);
            }
    };
    auto load_o = [&](const StepLayer& Ly, bool more) {
#pragma unroll
        for (int k = 0; k < kOR; ++k) {
            const int row = own.r_first + bw + kB * k;
            load_row(w.o[k], Ly.o, row, lane, has_r[k] && more);
        }
        w.os.fetch(Ly.o, r_row, r_live && more);
    };
    auto load_gate_up = [&](const StepLayer& Ly, bool more, int k0 = 0, int k1 = kGP) {
#pragma unroll
        for (int k = 0; k < kGP; ++k) {
            if (k < k0 || k >= k1) continue;
            const int p = own.g_first + bw + kB * k;
            load_row(w.g[k][0], Ly.gate_up, p, lane, has_g[k] && more);
            load_row(w.g[k][1], Ly.gate_up, F + p, lane, has_g[k] && more);
        }
        if (k0 == 0) w.gs.fetch(Ly.gate_up, g_row, g_live && more);
    };
    auto load_down = [&](const StepLayer& Ly, bool more, int k0 = 0, int k1 = kOR) {
#pragma unroll
        for (int k = 0; k < kOR; ++k) {
            if (k < k0 || k >= k1) continue;
            const int row = own.r_first + bw + kB * k;
            load_row(w.d[k], Ly.down, row, lane, has_r[k] && more);
        }
        if (k0 == 0) w.ds.fetch(Ly.down, r_row, r_live && more);
    };
    load_qkv(layer_at(s, 0), true);
    load_o(layer_at(s, 0), true);
    load_gate_up(layer_at(s, 0), true);

    // Reference order, a normalized phase (the input of q|k|v or gate|up, in
    // LDS at x with its gamma): this wave's own quantization of it, and its
    // dots (`dots(xc)`) taken on the speculative values, again only when the
    // exact sum (sq[slot]) rejects them.  Sets sx, the per-token scale.
    auto ref_quantize = [&](const float* x, const float* gamma, int phase, int slot, int L, float& sx,
                            auto&& dots) {
        SharedRef& r = static_cast<SharedRef&>(s);
        if (!wait_flags(s, r.staged, phase)) return false;
        // a fresh copy of the lane index keeps the per-lane LDS addresses
        // here instead of hoisted into registers across the layer loop
        int ln = lane;
        asm volatile("" : "+v"(ln));
        v4u xc[kKCH];
        WaveQuant st;
        wave_speculate<kKCH>(r.xg, H, ln, xc, st);
        dots(xc);
        if (!wait_ready(s, phase)) return false;
        stamp(P.trace, b, 64 * L + 8 + 2 * (phase % 4) + 8 * bw, kAT + kWave * bw);
        asm volatile("" : "+v"(ln));
        const float scale = rms_scale(r.sq[slot], H, P.epsilon);
        if (!wave_confirm(x, gamma, r.xg, scale, st, ln, sx)) {
            sx = wave_quantize<kKCH>(x, gamma, H, scale, ln, xc);
            dots(xc);
        }
        if (bw == 0) capture_wave_input<CAP>(P, x, gamma, H, scale, xc, sx, L, phase % 4, ln);
        return true;
    };

    for (int L = 0; L < P.layers; ++L) {
        float* Kc = P.kv + (size_t)L * 2 * P.kv_heads * P.capacity * dim;
        float* Vc = Kc + (size_t)P.kv_heads * P.capacity * dim;
        const bool more = L + 1 < P.layers;
        const StepLayer& next = layer_at(s, more ? L + 1 : L);
        // ---- q|k|v, RoPE, KV append
        {
            float sx;
            int tot[kQP][2];
            if constexpr (REF) {
                auto dots = [&](const v4u (&xc)[kKCH]) {
#pragma unroll
                    for (int k = 0; k < kQP; ++k)
#pragma unroll
                        for (int r = 0; r < 2; ++r)
                            tot[k][r] = has_q[k] ? dpp_sum_i32(row_part(w.q[k][r], xc, H / 16, lane)) : 0;
                };
                if (!ref_quantize(s.h_in, s.gamma_in, 4 * L + 0, 0, L, sx, dots)) return false;
            } else {
                if (!wait_ready(s, 4 * L + 0)) return false;
                stamp(P.trace, b, 64 * L + 8 + 8 * bw, kAT + kWave * bw);
                sx = s.sx[0];
#pragma unroll
                for (int k = 0; k < kQP; ++k)
#pragma unroll
                    for (int r = 0; r < 2; ++r) tot[k][r] = has_q[k] ? row_dot(w.q[k][r], s.xq[0], H / 16, lane) : 0;
            }
#pragma unroll
            for (int k = 0; k < kQP; ++k)
                if (has_q[k]) {
                    const int a0 = tot[k][0], a1 = tot[k][1];
                    if (lane == 0) {
                        const int r0 = qr[k][0], r1 = qr[k][1];
                        capture_acc<CAP>(P, L, 0, r0, a0);
                        capture_acc<CAP>(P, L, 0, r1, a1);
                        float v0 = dequant(a0, sx, w.qs[k][0].scale, w.qs[k][0].bias);
                        float v1 = dequant(a1, sx, w.qs[k][1].scale, w.qs[k][1].bias);
                        const int hb = r0 / dim, i0 = r0 % dim, i1 = r1 % dim, half = P.rotary / 2;
                        if (hb < P.heads + P.kv_heads && i0 < half) {
                            const float c = rope_c[k], sn = rope_s[k];
                            const float x0 = v0 * c - v1 * sn;
                            const float x1 = v1 * c + v0 * sn;
                            v0 = x0;
                            v1 = x1;
                        }
                        if (plan.local_q && hb < P.heads) {
                            // a q row of this XCD's head slices: plain stores, read from L2
                            __hip_atomic_store((LEAF_GLOBAL u64*)(P.x_q_local + r0), tagged(epoch(L, 1), v0),
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                            __hip_atomic_store((LEAF_GLOBAL u64*)(P.x_q_local + r1), tagged(epoch(L, 1), v1),
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                        } else {
                            publish(P.x_qkv + r0, epoch(L, 1), v0);
                            publish(P.x_qkv + r1, epoch(L, 1), v1);
                        }
                        if (hb >= P.heads) {
                            float* dst = hb < P.heads + P.kv_heads
                                             ? Kc + ((size_t)(hb - P.heads) * P.capacity + pos) * dim
                                             : Vc + ((size_t)(hb - P.heads - P.kv_heads) * P.capacity + pos) * dim;
                            stg(dst + i0, v0);
                            stg(dst + i1, v1);
                        }
                    }
                }
        }
        note_published(s);
        stamp(P.trace, b, 64 * L + 9 + 8 * bw, kAT + kWave * bw);
        if (!wait_received(s, 4 * L + 1)) return false;
        load_qkv(next, more);
        // ---- o_proj + residual
        if (!wait_ready(s, 4 * L + 1)) return false;
        stamp(P.trace, b, 64 * L + 10 + 8 * bw, kAT + kWave * bw);
        {
            // both rows' dots against one read of the input, one joint
            // reduction; lane 32 k publishes row k
            const float sx = s.sx[1];
            const int chunks = P.heads * dim / 16;
            v4u xc[kKCH];
#pragma unroll
            for (int j = 0; j < kKCH; ++j)
                xc[j] = *reinterpret_cast<const v4u*>(s.xq[1] + 16 * min(lane + kWave * j, chunks - 1));
            const int p0 = has_r[0] ? row_part(w.o[0], xc, chunks, lane) : 0;
            const int p1 = has_r[1] ? row_part(w.o[1], xc, chunks, lane) : 0;
            const int acc = sum2_transposed(p0, p1);
            if ((lane & 31) == 0 && r_live) capture_acc<CAP>(P, L, 1, r_row, acc);
            if ((lane & 31) == 0 && r_live)
                publish(P.x_mid + r_row, epoch(L, 4), s.h_in[r_row] + dequant(acc, sx, w.os.scale, w.os.bias));
        }
        note_published(s);
        stamp(P.trace, b, 64 * L + 11 + 8 * bw, kAT + kWave * bw);
        if (!wait_received(s, 4 * L + 2)) return false;
        load_o(next, more);
        // this layer's down rows (free since the last layer's down phase):
        // with the attention's reads and stores now in XCD-local L2, a load
        // burst in the attention window slowed the items down (640 against
        // 635 us per token with them here)
        load_down(layer_at(s, L), true);
        // ---- gate|up + SiLU gate
        {
            // Eight row dots against one read of the input, one transposed
            // reduction, then every pair's epilogue at once: lane 8 k (k < 4)
            // combines pair k's gate with its up (brought over from lane 8 k + 32).
            // Pairs this wave does not own are skipped (a wave-uniform test).
            const int chunks = H / 16;
            int total;
            auto dots = [&](const v4u (&xc)[kKCH]) {
                int part[2 * kGP];
#pragma unroll
                for (int k = 0; k < kGP; ++k) {
                    part[k] = has_g[k] ? row_part(w.g[k][0], xc, chunks, lane) : 0;
                    part[kGP + k] = has_g[k] ? row_part(w.g[k][1], xc, chunks, lane) : 0;
                }
                total = sum8_transposed(part, lane);
            };
            float sx;
            if constexpr (REF) {
                if (!ref_quantize(s.h_mid, static_cast<SharedRef&>(s).gamma_mid, 4 * L + 2, 1, L, sx, dots))
                    return false;
            } else {
                if (!wait_ready(s, 4 * L + 2)) return false;
                stamp(P.trace, b, 64 * L + 12 + 8 * bw, kAT + kWave * bw);
                sx = s.sx[0];
                v4u xc[kKCH];
#pragma unroll
                for (int j = 0; j < kKCH; ++j)
                    xc[j] = *reinterpret_cast<const v4u*>(s.xq[0] + 16 * min(lane + kWave * j, chunks - 1));
                dots(xc);
            }
            if ((lane & 7) == 0 && g_live) capture_acc<CAP>(P, L, 2, g_row, total);
            const float mine = dequant(total, sx, w.gs.scale, w.gs.bias);
            const float up = __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(mine),
                                                                             __float_as_uint(mine), false, false)[1]);
            if (lane < 32 && (lane & 7) == 0 && g_live) {
                float act;
                if constexpr (REF)
                    act = ref_activate(P.activation, mine, static_cast<SharedRef&>(s).exp2);
                else
                    act = activate(P.activation, mine);
                publish(P.x_act + g_pair, epoch(L, 5), up * act);
            }
        }
        note_published(s);
        stamp(P.trace, b, 64 * L + 13 + 8 * bw, kAT + kWave * bw);
        if (!wait_received(s, 4 * L + 3)) return false;
        // The next layer's gate|up rows go out in two halves: pairs 0-1 now
        // (the activation has been read), pairs 2-3 after the down publish.
        // One burst of all four here kept the weight waves issuing loads
        // when the down phase became ready (690 against 664 us per token).
        load_gate_up(next, more, 0, 2);
        // ---- down_proj + residual
        if (!wait_ready(s, 4 * L + 3)) return false;
        stamp(P.trace, b, 64 * L + 14 + 8 * bw, kAT + kWave * bw);
        {
            const float sx = s.sx[1];
            const int chunks = F / 16;
            v4u xc[kKCF];
#pragma unroll
            for (int j = 0; j < kKCF; ++j)
                xc[j] = *reinterpret_cast<const v4u*>(s.xq[1] + 16 * min(lane + kWave * j, chunks - 1));
            const int p0 = has_r[0] ? row_part(w.d[0], xc, chunks, lane) : 0;
            const int p1 = has_r[1] ? row_part(w.d[1], xc, chunks, lane) : 0;
            const int acc = sum2_transposed(p0, p1);
            if ((lane & 31) == 0 && r_live) capture_acc<CAP>(P, L, 3, r_row, acc);
            if ((lane & 31) == 0 && r_live)
                publish(P.x_hidden + r_row, epoch(L, 6), s.h_mid[r_row] + dequant(acc, sx, w.ds.scale, w.ds.bias));
        }
        note_published(s);
        stamp(P.trace, b, 64 * L + 15 + 8 * bw, kAT + kWave * bw);
        load_gate_up(next, more, 2, kGP);
    }
    return wait_ready(s, 4 * P.layers);
}

template <bool CAP, bool REF>
__global__ __launch_bounds__(kT, 1) void decode_step_kernel(StepParams P) {
    __shared__ typename std::conditional<REF, SharedRef, Shared>::type s;
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int G = gridDim.x, b = blockIdx.x;
    const int H = P.hidden;
    if (t == 0) {
        s.ready[0] = s.ready[1] = -1;
        s.received[0] = s.received[1] = -1;
        s.published = 0;
        s.abort = 0;
        s.pair[0][0] = s.pair[0][1] = s.pair[1][0] = s.pair[1][1] = 0;
    }
    if constexpr (REF) {
        if (t < 32) s.exp2[t] = kExp2Table32[t];
        if (t == 0) s.staged[0] = s.staged[1] = -1;
    }
    {
        const int words = P.layers * (int)(sizeof(StepLayer) / 16);
        const v4u* src = reinterpret_cast<const v4u*>(P.layer);
        v4u* dst = reinterpret_cast<v4u*>(s.layer_bytes);
        for (int i = t; i < words; i += kT) dst[i] = ldg(src + i);
    }
    __syncthreads();
    // Tests force a failed check on the last block, which then leaves at once:
    // the other blocks find its outputs missing and leave through their
    // bounded waits, and the host must still see the mismatch code.
    const bool forced = P.x_part_local && P.xcd_check_flip && b == G - 1;
    if (P.x_part_local && t == 0 && (forced || xcc_id() != (b & 7))) raise_abort(P, kAbortXcdMapping);
    if (forced) return;
    const bool ok = wave < kA ? exchange_role<CAP, REF>(P, s) : weight_role<CAP, REF>(P, s);
    if (__syncthreads_or(!ok)) return;          // every wave leaves when one gave up (abort flags raised)

    // ---------------- FP32 LM head and greedy argmax (all waves)
    const int V = P.vocab;
    const int v_first = (int)((long long)b * V / G), v_end = (int)((long long)(b + 1) * V / G);
    const int chunks = H / 4;                                  // float4 per row
    float best = -INFINITY;
    int best_i = V;
    const float* head = static_cast<const float*>(P.head.data);
    constexpr int kPerLane = kStepMaxHidden / 4 / kWave;       // float4 per lane of a row
    if constexpr (REF) {
        // dot_avx order (decoder.cpp:355-391; one token, one scale group):
        // chains a, b, c, d of 8 lanes run over the row's 32-column blocks,
        // lane l of chain c summing fmaf(w, x) over columns 32 j + 8 c + l;
        // then (a + b) + (c + d) per lane, the horizontal sum
        // ((l0 + l4) + (l2 + l6)) + ((l1 + l5) + (l3 + l7)), fmaf(sum, 1, 0)
        // for the group scale, and the bias.  Eight rows per wave: lane
        // 8 r + 2 c + h holds lanes 4 h .. 4 h + 3 of chain c of row r, so each
        // load is one 16-byte piece of a 32-column block.  Every lane of a
        // row's eight ends with the same total (IEEE addition commutes).
        const int r8 = lane >> 3, col = 8 * ((lane >> 1) & 3) + 4 * (lane & 1);
        constexpr int kBatch = 8;                              // 32-column blocks per batch of loads
        const int blocks32 = H / 32;
        for (int r0 = v_first + 8 * wave; r0 < v_end; r0 += 8 * kWaves) {
            const int r = min(r0 + r8, v_end - 1);
            const LEAF_GLOBAL v4f* wr = (const LEAF_GLOBAL v4f*)(head + (size_t)r * H + col);
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            v4f wa[kBatch], wb[kBatch];
            auto load = [&](v4f (&w)[kBatch], int j0) {
#pragma unroll
                for (int j = 0; j < kBatch; ++j) w[j] = __builtin_nontemporal_load(wr + 8 * min(j0 + j, blocks32 - 1));
            };
            auto fold = [&](const v4f (&w)[kBatch], int j0) {
#pragma unroll
                for (int j = 0; j < kBatch; ++j)
                    if (j0 + j < blocks32) {
                        const v4f xv = *reinterpret_cast<const v4f*>(s.xf + 32 * (j0 + j) + col);
                        acc[0] = fmaf(w[j].x, xv.x, acc[0]);
                        acc[1] = fmaf(w[j].y, xv.y, acc[1]);
                        acc[2] = fmaf(w[j].z, xv.z, acc[2]);
                        acc[3] = fmaf(w[j].w, xv.w, acc[3]);
                    }
            };
            load(wa, 0);
            for (int j0 = 0; j0 < blocks32; j0 += 2 * kBatch) {
                if (j0 + kBatch < blocks32) load(wb, j0 + kBatch);
                fold(wa, j0);
                if (j0 + kBatch >= blocks32) break;
                if (j0 + 2 * kBatch < blocks32) load(wa, j0 + 2 * kBatch);
                fold(wb, j0 + kBatch);
            }
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float t2 = acc[i] + __shfl_xor(acc[i], 2, kWave);   // a + b, c + d
                v[i] = t2 + __shfl_xor(t2, 4, kWave);                     // (a + b) + (c + d)
            }
            float h4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) h4[i] = v[i] + __shfl_xor(v[i], 1, kWave);   // l + (l + 4)
            const float total = (h4[0] + h4[2]) + (h4[1] + h4[3]);
            const float logit = fmaf(total, 1.0f, 0.0f) + ldg(P.head.bias + r);
            if (r0 + r8 < v_end) {
                if ((lane & 7) == 0) stg(P.logits + r, logit);
                if (better(logit, r, best, best_i)) { best = logit; best_i = r; }
            }
        }
#pragma unroll
        for (int o = 8; o < kWave; o <<= 1) {
            const float ov = __shfl_xor(best, o, kWave);
            const int oi = __shfl_xor(best_i, o, kWave);
            if (better(ov, oi, best, best_i)) { best = ov; best_i = oi; }
        }
    }
    for (int r = v_first + wave; !REF && r < v_end; r += 2 * kWaves) {
        const int r2 = r + kWaves;
        const bool two = r2 < v_end;
        v4f wa[kPerLane], wb[kPerLane];
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const int c = min(lane + kWave * j, chunks - 1);
            wa[j] = __builtin_nontemporal_load((const LEAF_GLOBAL v4f*)(head + (size_t)r * H) + c);
            wb[j] = __builtin_nontemporal_load((const LEAF_GLOBAL v4f*)(head + (size_t)(two ? r2 : r) * H) + c);
        }
        float aa = 0.0f, ab = 0.0f;
#pragma unroll
        for (int j = 0; j < kPerLane; ++j) {
            const int c = lane + kWave * j;
            if (c < chunks) {
                const v4f xv = *reinterpret_cast<const v4f*>(s.xf + 4 * c);
                aa = fmaf(wa[j].x, xv.x, aa); aa = fmaf(wa[j].y, xv.y, aa);
                aa = fmaf(wa[j].z, xv.z, aa); aa = fmaf(wa[j].w, xv.w, aa);
                ab = fmaf(wb[j].x, xv.x, ab); ab = fmaf(wb[j].y, xv.y, ab);
                ab = fmaf(wb[j].z, xv.z, ab); ab = fmaf(wb[j].w, xv.w, ab);
            }
        }
        aa = dpp_sum_f32(aa);
        const float la = aa + ldg(P.head.bias + r);
        if (lane == 0) stg(P.logits + r, la);
        if (better(la, r, best, best_i)) { best = la; best_i = r; }
        if (two) {
            ab = dpp_sum_f32(ab);
            const float lb = ab + ldg(P.head.bias + r2);
            if (lane == 0) stg(P.logits + r2, lb);
            if (better(lb, r2, best, best_i)) { best = lb; best_i = r2; }
        }
    }
    if (lane == 0) {
        s.best_v[wave] = best;
        s.best_i[wave] = best_i;
    }
    __syncthreads();
    stamp(P.trace, b, 64 * P.layers + 2);
    const unsigned final_epoch = P.epoch + (unsigned)(P.layers * 8 + 1);
    if (t == 0) {
        float bv = s.best_v[0];
        int bi = s.best_i[0];
        for (int w = 1; w < kWaves; ++w)
            if (better(s.best_v[w], s.best_i[w], bv, bi)) { bv = s.best_v[w]; bi = s.best_i[w]; }
        publish(P.x_best + 2 * b, final_epoch, bv);
        publish(P.x_best + 2 * b + 1, final_epoch, __int_as_float(bi));
    }
    if (b != 0) return;
    // Block 0: the first maximal logit over all blocks (std::max_element).
    float cand[2];
    {
        auto best_index = [&](int i) { return t < G ? 2 * t + i : -1; };
        const bool done = await(P.x_best, best_index, final_epoch, cand, P);
        if (!__syncthreads_and(done)) return;
    }
    float bv = t < G ? cand[0] : -INFINITY;
    int bi = t < G ? __float_as_int(cand[1]) : V;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, kWave);
        const int oi = __shfl_xor(bi, o, kWave);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) {
        s.best_v[wave] = bv;
        s.best_i[wave] = bi;
    }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < kWaves; ++w)
            if (better(s.best_v[w], s.best_i[w], bv, bi)) { bv = s.best_v[w]; bi = s.best_i[w]; }
        stg(P.token, (uint32_t)bi);
        if (P.host_token) *P.host_token = (uint32_t)bi;
        stamp(P.trace, b, 64 * P.layers + 3);
    }
}

}  // namespace

int decode_step_spans(int keys) { return (keys + kStepSpanKeys - 1) / kStepSpanKeys; }

int decode_step_blocks(int device) {
    int cus = 0, resident = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
    for (const void* kernel : {reinterpret_cast<const void*>(decode_step_kernel<false, false>),
                               reinterpret_cast<const void*>(decode_step_kernel<true, false>),
                               reinterpret_cast<const void*>(decode_step_kernel<false, true>),
                               reinterpret_cast<const void*>(decode_step_kernel<true, true>)}) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, kernel, kT, 0) != hipSuccess || resident < 1)
            return 0;
    }
    return cus;
}

bool decode_step_fits(int hidden, int ffn, int heads, int kv_heads, int dim, int vocab, int blocks) {
    if (dim != kStepDim || kv_heads <= 0 || heads % kv_heads || heads / kv_heads > kStepMaxGroup) return false;
    if (hidden <= 0 || hidden > kStepMaxHidden || hidden % 16 || heads * dim != hidden) return false;
    if (ffn <= 0 || ffn > kStepMaxFfn || ffn % 16 || vocab <= 0 || blocks <= 0 || blocks > kT) return false;
    const int pairs = (heads + 2 * kv_heads) * dim / 2;
    // rows per weight wave: kQP q|k|v pairs, kOR o/down rows, kGP gate|up pairs
    return (pairs + blocks - 1) / blocks <= kQP * kB && (hidden + blocks - 1) / blocks <= kOR * kB &&
           (ffn + blocks - 1) / blocks <= kGP * kB;
}

int decode_step_reference_keys() { return kRefStepKeys; }

bool decode_step_fits_reference(int hidden, int activation) {
    // the head's dot_avx chains cover the row in whole 32-column blocks;
    // GELU needs glibc's erff / tanhf, which the device does not restate
    return hidden % 32 == 0 && (activation == 0 || activation == 3);
}

hipError_t launch_decode_step(const StepParams& params, int blocks, hipStream_t stream, bool cooperative) {
    StepParams p = params;
    void* args[] = {&p};
    const void* kernel = p.reference ? (p.capture.x ? reinterpret_cast<const void*>(decode_step_kernel<true, true>)
                                                    : reinterpret_cast<const void*>(decode_step_kernel<false, true>))
                                     : (p.capture.x ? reinterpret_cast<const void*>(decode_step_kernel<true, false>)
                                                    : reinterpret_cast<const void*>(decode_step_kernel<false, false>));
    if (cooperative) return hipLaunchCooperativeKernel(kernel, dim3(blocks), dim3(kT), args, 0, stream);
    // A plain launch of the same grid: one block per CU fits (decode_step_blocks
    // checked the occupancy), so on an otherwise idle device every block is
    // resident at once; if one were not, the others' bounded waits would
    // abort the step with an error rather than hang.
    return hipLaunchKernel(kernel, dim3(blocks), dim3(kT), args, 0, stream);
}

}  // namespace leafhip
