/* TEST INFRASTRUCTURE ONLY — the CPU oracle for kvexp's fused decode path.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker. The product (libkvexp_hip.so)
 * never links, loads or calls it.
 *
 * Status codes mirror the reference's exception classes:
 *   0 ok, 1 std::invalid_argument, 2 std::runtime_error, 3 std::logic_error,
 *   5 output buffer too small. The message text equals the reference's
 *   what() string; read it with oracle_last_error().
 */
#ifndef KVEXP_ORACLE_H
#define KVEXP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char *oracle_last_error(void);

/* Size model (include/kvexp/bf16.hpp:39-49). */
int oracle_exp_payload_bytes(int n_tokens, int dim, int bits);
int oracle_coded_block_bytes(int n_tokens, int dim, int bits, int n_escape);
int oracle_raw_block_bytes(int n_tokens, int dim);
/* Upper bound of any container of [seq, dim] at `block` tokens per block:
 * every block raw. The encoder never emits more. */
size_t oracle_encode_bound(int seq, int dim, int block);

/* encode_bf16 (src/codec.cpp:39-164). */
int oracle_encode(const uint16_t *kv, int seq, int dim, int block, uint8_t *out, size_t cap,
                  size_t *out_bytes);
/* encode_bf16 with a choice of coded modes (bit m set: mode m may be
 * chosen; raw always may). ORACLE_MODES_REFERENCE (2- and 4-bit) is
 * encode_bf16; adding bit 3 gives the 3-bit format extension (mode byte 3,
 * codes 0..6 over the window [base, base + 6], 7 the escape sentinel, element
 * i at bits [3i, 3i + 3) of the code bytes, head_dim a multiple of 8), sized
 * and chosen as the reference's python/analyze_exponents.py:104-157 sizes it
 * (its kernels and readers do not implement it). */
#define ORACLE_MODES_REFERENCE 0x14u
#define ORACLE_MODE_3BIT 0x08u
int oracle_encode_modes(const uint16_t *kv, int seq, int dim, int block, unsigned modes, uint8_t *out,
                        size_t cap, size_t *out_bytes);
/* decode_bf16 (src/codec.cpp:166-174, scan.hpp:79-165); also reads mode 3. */
int oracle_decode(const uint8_t *blob, size_t bytes, int seq, int dim, uint16_t *out);

/* Block walk: byte offset and first token of every block the decode-side
 * readers touch when `seq` tokens are consumed (scan.hpp:94-123,176-189),
 * plus one terminal entry (offset of the next byte, total tokens).
 * Arrays need room for max_blocks + 1 entries. */
int oracle_block_index(const uint8_t *blob, size_t bytes, int dim, int seq, int64_t *offsets,
                       int32_t *first_token, int max_blocks, int *n_blocks);

/* Per-block statistics of a container: mode histogram and escape count. */
int oracle_container_stats(const uint8_t *blob, size_t bytes, int dim, int64_t *n_raw,
                           int64_t *n_2bit, int64_t *n_4bit, int64_t *n_escapes);

/* Blocks per mode byte: counts[m] for m in 0..4. */
int oracle_container_mode_counts(const uint8_t *blob, size_t bytes, int dim, int64_t *counts);

/* attention_decode (src/dispatch.cpp:27-104). backend: 0 scalar, 1 avx2
 * (bit-identical to scalar, attention.hpp:30-39), 2 avx512-bf16 score order
 * (attention_avx512.cpp:114-138), emulated in portable C.
 * lse (nullable): m + logf(l) per query row after the merge — an extension
 * that the reference does not output. */
int oracle_attention(int backend, const uint16_t *q, const uint16_t *k_raw, const uint16_t *v_raw,
                     const uint8_t *k_xkv, size_t k_bytes, const uint8_t *v_xkv, size_t v_bytes,
                     float *out, float *lse, int n_q, int dim, int seq, int n_threads,
                     int split_tokens);

/* Many independent KV heads (OpenMP over heads, each head as above).
 * Head h uses q + h*n_q*dim, out + h*n_q*dim, lse + h*n_q, and either
 * k_raw[h]/v_raw[h] or k_xkv[h]/v_xkv[h] with byte counts; seq[h], splits[h]. */
int oracle_attention_heads(int backend, int n_heads, const uint16_t *q,
                           const uint16_t *const *k_raw, const uint16_t *const *v_raw,
                           const uint8_t *const *k_xkv, const uint64_t *k_bytes,
                           const uint8_t *const *v_xkv, const uint64_t *v_bytes, float *out,
                           float *lse, int n_q, int dim, const int32_t *seq,
                           const int32_t *n_threads, int split_tokens, int *status_per_head);

/* Scalar score for one (q row, k row): the 8-lane strided FMA order and tree
 * (attention_scalar.cpp:13-29), and the VDPBF16PS order (attention_avx512.cpp). */
float oracle_score_scalar(const uint16_t *q, const uint16_t *k, int dim);
float oracle_score_dpbf16(const uint16_t *q, const uint16_t *k, int dim);

/* Element-wise glibc expf and logf (the reference's std::exp(float)). */
void oracle_expf_array(const float *x, float *y, size_t n);
/* Compares y[i] with expf(x[i]) bit for bit (NaN matches NaN); returns the
 * number of mismatches and the first mismatching index in *first (or -1). */
size_t oracle_expf_compare(const float *x, const float *y, size_t n, int64_t *first);
/* Same over every float whose bit pattern is in [lo, hi) with y indexed from 0. */
size_t oracle_expf_compare_range(uint32_t lo, uint32_t hi, const float *y, int64_t *first);

#ifdef __cplusplus
}
#endif
#endif
