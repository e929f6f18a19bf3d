// kvexp-amd: BF16 field helpers and the container size model.
// Same names and meaning as the reference's include/kvexp/bf16.hpp:12-49.
#pragma once

#include <cstdint>
#include <cstring>

namespace kvexp {

// Default tokens per encoded block and the largest supported head dimension.
inline constexpr int kEncodeBlock = 128;
inline constexpr int kMaxHeadDim = 256;

// BF16 is the upper half of an IEEE binary32: sign 1 | exponent 8 | mantissa 7.
inline float bf16_to_fp32(uint16_t bits) {
    const uint32_t u = uint32_t(bits) << 16;
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
}

inline uint8_t bf16_exponent(uint16_t bits) { return uint8_t(bits >> 7); }

// Sign in bit 7, mantissa in bits 6:0 (the exponent is coded separately).
inline uint8_t bf16_sm(uint16_t bits) { return uint8_t(((bits >> 8) & 0x80u) | (bits & 0x7Fu)); }

inline uint16_t bf16_from_parts(uint8_t exponent, uint8_t sm) {
    return uint16_t(((sm & 0x80u) << 8) | (uint32_t(exponent) << 7) | (sm & 0x7Fu));
}

// The exponent is base + delta modulo 256.
inline uint16_t bf16_from_delta(uint8_t base, uint8_t delta, uint8_t sm) {
    return bf16_from_parts(uint8_t(base + delta), sm);
}

inline int exp_payload_bytes(int n_tokens, int dim, int bits) { return (n_tokens * dim * bits + 7) / 8; }

inline int coded_block_bytes(int n_tokens, int dim, int bits, int n_escape) {
    return 8 + dim + n_tokens * dim + exp_payload_bytes(n_tokens, dim, bits) + 2 * n_escape;
}

inline int raw_block_bytes(int n_tokens, int dim) { return 8 + 2 * n_tokens * dim; }

} // namespace kvexp
