// kvexp-amd: the XKV container codec, run on the GPU.
// Same interface as the reference's include/kvexp/codec.hpp:38-48; the
// container bytes are identical to the reference encoder's.
#pragma once

#include "kvexp/bf16.hpp"

#include <cstddef>
#include <cstdint>
#include <vector>

namespace kvexp {

// Blocks of up to block_tokens tokens; per block an 8-byte header
// (mode, n_tokens, n_escape, head_dim, reserved), then raw BF16 rows or
// base[dim], sign/mantissa bytes, 2- or 4-bit exponent residuals and u16
// escape words in scan order.
struct EncodedTensor {
    std::vector<uint8_t> bytes;
    int seq_len = 0;
    int head_dim = 0;
    int block_tokens = kEncodeBlock;
};

// Host buffers in and out; the work runs on device 0 (or the device set with
// set_device). Throws std::invalid_argument / std::runtime_error /
// std::logic_error with the reference's messages.
EncodedTensor encode_bf16(const uint16_t *kv, int seq_len, int head_dim, int block_tokens = kEncodeBlock);

void decode_bf16(const uint8_t *blob, size_t bytes, int seq_len, int head_dim, uint16_t *out);

// Device used by the host-pointer entry points of this header and
// attention.hpp (default 0).
void set_device(int device);

} // namespace kvexp
