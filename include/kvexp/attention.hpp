// kvexp-amd: decode attention over raw BF16 or XKV containers.
// Same interface as the reference's include/kvexp/attention.hpp:10-61, with
// two GPU entries in the backend table.
#pragma once

#include "kvexp/bf16.hpp"

#include <cstddef>
#include <cstdint>

namespace kvexp {

enum class Backend {
    Scalar,      // reference CPU backends: not part of this library
    Avx2,
    Avx512Bf16,
    Hip,         // MI355X, score order of Scalar/Avx2 (bit-identical outputs)
    HipDpbf16,   // MI355X, score order of Avx512Bf16 (bit-identical outputs)
};

struct CpuFeatures {
    bool avx2 = false;
    bool avx512_bf16 = false;
};

CpuFeatures detect_cpu();

// One decode step over `seq` keys for `n_q` queries sharing one KV head; Q, K,
// V BF16, output FP32 [n_q, dim]. Exactly one of (k_raw, k_xkv) is non-null,
// and the same for V. The sequence is split on `split_tokens` tiles into
// min(n_threads, tiles) parts (token_bounds), each folded in token order with
//   m' = max(m, s); alpha = exp(m - m'); e = exp(s - m'); l = fma(l, alpha, e);
//   acc = fma(e, v, acc * alpha)
// and the parts merged left to right; out = acc * (1/l). For the same split
// the Hip backends return the reference backends' bits, and XKV and raw
// inputs return the same bits. Host pointers; the call synchronises.
void attention_decode(Backend backend, const uint16_t *q, const uint16_t *k_raw, const uint16_t *v_raw,
                      const uint8_t *k_xkv, size_t k_bytes, const uint8_t *v_xkv, size_t v_bytes, float *out,
                      int n_q, int dim, int seq, int n_threads, int split_tokens = kEncodeBlock);

} // namespace kvexp
