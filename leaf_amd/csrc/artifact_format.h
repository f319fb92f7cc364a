// LEAFDC decoder artifacts (versions 2-7): parsing and validation on the host.
//
// The format, little-endian throughout:
//   header   magic "LEAFDC0v", u32 version, u32 tensor count, u64 data base
//            (a multiple of 64), ten u32 geometry fields (hidden, intermediate,
//            heads, kv heads, layers, vocab, max positions, eos, head dim,
//            sliding window), f32 theta, f32 epsilon, eight u32 operator codes
//            (norm kind, activation, position kind, gated, parallel residual,
//            rotary dim, position offset, final norm), f32 embedding scale;
//   v7       u32 storage (0 / 5 / 6), u32 Q/K norm, u32 n, f32 frequency[n];
//   v4-v7    u32 EOS count, u32 EOS token[count];
//   tensors  count x (u32 name length, name, u32 rank, rows, cols, bits,
//            group, u64 offset, size, scale offset, scale count), offsets
//            relative to the data base;
//   data     payloads and f32 scales at 64-byte aligned offsets.
// The reference reads it in Decoder::Impl::Impl (engine/src/decoder.cpp:787-933)
// and writes it in tools/export_decoder.py:213-420.
//
// read_artifact() accepts exactly the artifacts the reference accepts and
// rejects the others with the reference's message for the first problem it
// meets (callers and tests match on those messages).  It also applies, at
// load time, the consistency checks the reference makes on first use of a
// tensor (linear and norm biases, calibrated input scales; decoder.cpp:994-1024,
// 975-981), and one device limit of its own (head dims above 256).
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>

#include "runtime.h"

namespace leafhip {

struct ArtifactContents {
    Config config;
    std::unordered_map<std::string, TensorRecord> tensors;   // data / scales point into the caller's bytes
    uint32_t source_bf16_tensors = 0, quantized_tensors = 0;
    bool accurate = false;                                   // FP32Math::Accurate accepted
    const TensorRecord* find(const std::string& name) const {
        const auto it = tensors.find(name);
        return it == tensors.end() ? nullptr : &it->second;
    }
};

// Throws Error (LH_ERROR_ARTIFACT, or LH_ERROR_INVALID_ARGUMENT /
// LH_ERROR_UNSUPPORTED for policy and device limits) on the first problem.
ArtifactContents read_artifact(const uint8_t* data, size_t size, uint32_t activation_bits, uint32_t fp32_math);

}  // namespace leafhip
