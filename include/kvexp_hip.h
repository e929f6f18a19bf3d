/* kvexp-amd: C ABI of the MI355X (gfx950) backend for kvexp's fused
 * compressed-KV decode attention.
 *
 * Plain pointers and sizes only; no HIP or torch types cross this boundary
 * (streams are passed as `void *` holding a hipStream_t, NULL = default
 * stream). Every entry point returns a status code (0 = success) and never
 * lets a C++ exception escape; kvexp_hip_last_error() returns the calling
 * thread's message for the last failure, worded like the reference's
 * exception text where the reference defines one.
 *
 * Device pointers are marked d_*. The caller owns every buffer. Entry points
 * that take a stream are stream-ordered and do not synchronise unless stated.
 *
 * Reference interfaces each entry point replaces (paths in the reference):
 *   kvexp_hip_attention_decode_host  kvexp::attention_decode
 *                                    include/kvexp/attention.hpp:58-61,
 *                                    src/dispatch.cpp:27-104 (Backend::Hip case)
 *   kvexp_hip_attention_run          the per-thread range plugin
 *                                    detail::range_<isa> (src/detail.hpp:9-19)
 *                                    plus merge_state/finalize_state
 *                                    (src/softmax.hpp:16-41), batched over heads
 *   kvexp_hip_encode                 kvexp::encode_bf16 (include/kvexp/codec.hpp:45-46,
 *                                    src/codec.cpp:39-164)
 *   kvexp_hip_append(_batch)         kvexp::encode_bf16 of the grown sequence
 *                                    (src/codec.cpp:39-164), done incrementally
 *   kvexp_hip_decode                 kvexp::decode_bf16 (include/kvexp/codec.hpp:48,
 *                                    src/codec.cpp:166-174)
 *   kvexp_hip_build_index            the header walk of XkvReader::seek / open_xkv
 *                                    (include/kvexp/scan.hpp:94-123,192-218)
 *   kvexp_hip_*_block_bytes          include/kvexp/bf16.hpp:39-49
 */
#ifndef KVEXP_HIP_H
#define KVEXP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------- status ---- */
enum {
    KVEXP_HIP_OK = 0,
    KVEXP_HIP_INVALID_ARGUMENT = 1, /* reference: std::invalid_argument */
    KVEXP_HIP_FORMAT_ERROR = 2,     /* reference: std::runtime_error (container, split) */
    KVEXP_HIP_LOGIC_ERROR = 3,      /* reference: std::logic_error */
    KVEXP_HIP_UNSUPPORTED = 4,      /* shape or option this build does not run */
    KVEXP_HIP_DEVICE_ERROR = 5,     /* a HIP runtime call failed */
    KVEXP_HIP_CAPACITY = 6          /* an output buffer is too small */
};

const char *kvexp_hip_status_string(int status);
/* Message of the calling thread's last failure ("" after a success). */
const char *kvexp_hip_last_error(void);
/* Library version string and the gfx target it was built for. */
const char *kvexp_hip_version(void);

/* ------------------------------------------------------------ context ---- */
/* A context binds one device and owns the encoders' scratch memory, their
 * status word and a non-blocking stream for the host-pointer entry
 * (kvexp_hip_attention_decode_host). Contexts are independent: calls on
 * different contexts may run concurrently from different host threads and
 * share no mutable state. One context may be used from one host thread at a
 * time; its encoders order their scratch reuse across streams themselves
 * (a later call on another stream waits on the GPU for the earlier one). */
typedef struct kvexp_hip_ctx kvexp_hip_ctx;

int kvexp_hip_ctx_create(int device, kvexp_hip_ctx **out);
int kvexp_hip_ctx_destroy(kvexp_hip_ctx *ctx);

/* --------------------------------------------------------- size model ---- */
/* include/kvexp/bf16.hpp:39-49 */
int kvexp_hip_exp_payload_bytes(int n_tokens, int dim, int bits);
int kvexp_hip_coded_block_bytes(int n_tokens, int dim, int bits, int n_escape);
int kvexp_hip_raw_block_bytes(int n_tokens, int dim);
/* Largest container encode_bf16 can emit for [seq, dim] (every block raw). */
int64_t kvexp_hip_encode_bound(int seq, int dim, int block_tokens);
int kvexp_hip_block_count(int seq, int block_tokens);

/* ------------------------------------------------------- block index ---- */
/* Host walk of a host-resident container: byte offset and first token of
 * each block that a reader consuming `seq` tokens touches, plus one terminal
 * entry (next byte offset, token count). Arrays hold capacity + 1 entries.
 * Validation and messages follow parse_block (scan.hpp:28-66), including the
 * eager parse of the header after the last block used (scan.hpp:144-151). */
int kvexp_hip_build_index(const uint8_t *blob, size_t bytes, int dim, int seq, int64_t *offsets,
                          int32_t *first_token, int capacity, int *n_blocks);

/* ------------------------------------------------------------- codec ---- */
/* Coded block modes the context's encoders (kvexp_hip_encode,
 * kvexp_hip_append, kvexp_hip_append_batch) may choose; raw blocks always
 * may be chosen. The default, KVEXP_HIP_MODES_REFERENCE, gives encode_bf16's
 * containers (codec.cpp:84-104). KVEXP_HIP_MODE_3BIT adds this library's
 * format extension: mode byte 3, 3-bit codes over a 7-exponent window per
 * channel (code 7 is the escape sentinel), element i of the block in bits
 * [3i, 3i + 3) of the little-endian code bytes, taken only when head_dim is
 * a multiple of 8; a block then takes the smallest of raw, 2-, 3- and 4-bit
 * with ties to raw, fewer escapes, fewer bits (the 3-bit sizing of the
 * reference's python/analyze_exponents.py:104-157, which its kernels do not
 * implement). Every reader in this library (decode, index, plans, the
 * attention kernels) accepts mode 3 blocks; the reference's readers reject
 * them. Appends to a container should use the setting it was encoded with,
 * or its blocks differ from a fresh encode. No counterpart in the reference. */
#define KVEXP_HIP_MODE_2BIT 4u
#define KVEXP_HIP_MODE_3BIT 8u
#define KVEXP_HIP_MODE_4BIT 16u
#define KVEXP_HIP_MODES_REFERENCE (KVEXP_HIP_MODE_2BIT | KVEXP_HIP_MODE_4BIT)
int kvexp_hip_set_encoder_modes(kvexp_hip_ctx *ctx, unsigned modes);
/* The context's encoder modes (-1 for a null context). */
int kvexp_hip_get_encoder_modes(kvexp_hip_ctx *ctx);

/* Encodes d_kv [seq, dim] BF16 (token-major) into d_out, byte-identical to
 * encode_bf16 (with the default encoder modes). d_out needs kvexp_hip_encode_bound() bytes. Writes the block
 * index (n_blocks + 1 entries each) to d_offsets / d_first_token when they
 * are non-NULL. The container size is written to *bytes_out (host) after a
 * synchronisation of `stream` when bytes_out is non-NULL; it is also
 * d_offsets[n_blocks] when d_offsets is given. */
int kvexp_hip_encode(kvexp_hip_ctx *ctx, const uint16_t *d_kv, int seq, int dim, int block_tokens,
                     uint8_t *d_out, size_t capacity, int64_t *d_offsets, int32_t *d_first_token,
                     size_t *bytes_out, void *stream);

/* kvexp_hip_encode for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. It allocates nothing and does not
 * synchronise: its scratch is a static device array of
 * KVEXP_HIP_NOALLOC_SCRATCH_BYTES per GPU (looked up when a context is
 * created on that GPU), which must hold 256 + 8 * n_blocks bytes (rounded up
 * to 256) plus 256 where the one-pass encoder runs (head_dim % 8 == 0,
 * block_tokens * dim <= 16384, d_kv 16-byte aligned: about 520,000 blocks),
 * else n_blocks * (16 + 3 * dim) bytes (each part rounded up to 256) plus
 * 256 (about 20,000 blocks at head_dim 64); larger inputs are refused with
 * KVEXP_HIP_CAPACITY. The block index is an output here: d_offsets and
 * d_first_token (n_blocks + 1 entries) are required; the container size is
 * d_offsets[n_blocks]. When d_status is not NULL, a nonzero value is OR-ed
 * into it if the encoder's size model drifted (it is never cleared). All
 * calls on one GPU share the scratch, which keeps the last call's contents:
 * calls that overlap on one GPU (any contexts, any streams) race. Each call
 * clears the look-back state it uses with a kernel launched ahead of the
 * encoder (no memset), so a call captured in a graph may be replayed over
 * new inputs. Output is byte-identical to kvexp_hip_encode's. */
#define KVEXP_HIP_NOALLOC_SCRATCH_BYTES 4194304
int kvexp_hip_encode_noalloc(kvexp_hip_ctx *ctx, const uint16_t *d_kv, int seq, int dim, int block_tokens,
                             uint8_t *d_out, size_t capacity, int64_t *d_offsets, int32_t *d_first_token,
                             uint32_t *d_status, void *stream);

/* Appends n_new tokens (d_new [n_new, dim] BF16) to a device container that
 * holds the first n_tokens tokens of a sequence, so that afterwards it is
 * byte-identical to encode_bf16 of all n_tokens + n_new tokens (blocks are
 * encoded independently, so only the trailing partial block is encoded
 * again, followed by the new blocks). d_blob (capacity bytes, at least
 * kvexp_hip_encode_bound(n_tokens + n_new, ...)) and its block index
 * d_offsets / d_first_token (index_capacity entries, at least
 * kvexp_hip_block_count(n_tokens + n_new, ...) + 1) are updated in place.
 * d_tail [block_tokens, dim] BF16 holds the raw tokens of the trailing
 * partial block (the last n_tokens % block_tokens tokens) and is updated;
 * a caller starting from a container made by kvexp_hip_encode fills it with
 * those tokens. n_tokens = 0 starts a new container (n_new = 0 then writes
 * the empty index). The new container size goes to *bytes_out after a
 * synchronisation of `stream` when bytes_out is non-NULL. Scratch memory
 * comes from the context (grown on demand, like kvexp_hip_encode's), so
 * calls on one context must not overlap. */
int kvexp_hip_append(kvexp_hip_ctx *ctx, const uint16_t *d_new, int n_new, int n_tokens, int dim,
                     int block_tokens, uint16_t *d_tail, uint8_t *d_blob, size_t capacity, int64_t *d_offsets,
                     int32_t *d_first_token, int index_capacity, size_t *bytes_out, void *stream);

/* One container of a batched append: the arguments of kvexp_hip_append. */
typedef struct kvexp_hip_append_job {
    const uint16_t *d_new;      /* [n_new, dim] BF16 */
    int32_t n_new;
    int32_t n_tokens;           /* tokens already in the container */
    uint16_t *d_tail;           /* [block_tokens, dim] BF16, raw trailing partial block */
    uint8_t *d_blob;
    uint64_t capacity;
    int64_t *d_offsets;
    int32_t *d_first_token;
    int32_t index_capacity;
    int32_t reserved;
} kvexp_hip_append_job;

/* kvexp_hip_append for n_jobs containers of one shape in one set of
 * launches (a decode step appends one token to every K and V tensor). No
 * synchronisation unless `check` is non-zero, which then reports an encoder
 * size-model error. */
int kvexp_hip_append_batch(kvexp_hip_ctx *ctx, const kvexp_hip_append_job *jobs, int n_jobs, int dim,
                           int block_tokens, int check, void *stream);

/* Decodes seq tokens of a device container into d_out [seq, dim] BF16,
 * bit-identical to decode_bf16. d_offsets / d_first_token is the block index
 * (n_blocks + 1 entries) of that container. Synchronises `stream` and
 * reports container format errors (bad header, escape overrun) when
 * `check` is non-zero. */
int kvexp_hip_decode(kvexp_hip_ctx *ctx, const uint8_t *d_blob, size_t bytes, const int64_t *d_offsets,
                     const int32_t *d_first_token, int n_blocks, int seq, int dim, uint16_t *d_out,
                     int check, void *stream);

/* --------------------------------------------------------- attention ---- */
/* Score order of the QK dot product (bit-for-bit with one reference backend):
 *   KVEXP_HIP_ORDER_SCALAR: 8 strided FMA lanes then ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)),
 *                           as attention_scalar.cpp and attention_avx2.cpp;
 *   KVEXP_HIP_ORDER_DPBF16: VDPBF16PS pairs (odd element first, DAZ/FTZ) over 32-element
 *                           steps and a 16-lane pairwise tree, as attention_avx512.cpp. */
enum { KVEXP_HIP_ORDER_SCALAR = 0, KVEXP_HIP_ORDER_DPBF16 = 1 };

/* One KV head: either XKV containers with their device block indexes, or raw
 * [seq, dim] BF16 arrays (exactly one of the two, for K and V alike). */
typedef struct kvexp_hip_head {
    const uint8_t *k_xkv, *v_xkv;             /* device containers, or NULL */
    uint64_t k_bytes, v_bytes;
    const int64_t *k_offsets, *v_offsets;     /* device block index (n_blocks + 1) */
    const int32_t *k_first_token, *v_first_token;
    int32_t k_n_blocks, v_n_blocks;
    const uint16_t *k_raw, *v_raw;            /* device [seq, dim] BF16, or NULL */
    int32_t seq;                              /* tokens attended (> 0) */
    int32_t n_splits;                         /* sequence splits, as attention_decode's n_threads */
} kvexp_hip_head;

/* A plan fixes the heads, the split of each head and the kernel choice; it
 * owns the device-side descriptors and its own status word, so running it
 * launches kernels and copies nothing from the host. Splits follow
 * token_bounds (dispatch.cpp:17-23) over `split_tokens`-token tiles with
 * min(max(1, n_splits), tiles) parts; XKV split starts must fall on block
 * starts of both K and V (else "token split is not aligned to an encoded
 * block"). Creating a plan is ordered on `stream` (the stream whose encodes
 * or appends wrote the containers): it reads the block indexes and checks
 * every block header after the work queued there, and synchronises only
 * that stream. Plans of one context may be created from one thread at a
 * time (they share its pinned staging buffer). */
typedef struct kvexp_hip_plan kvexp_hip_plan;

int kvexp_hip_plan_create(kvexp_hip_ctx *ctx, const kvexp_hip_head *heads, int n_heads, int n_q, int dim,
                          int split_tokens, int order, void *stream, kvexp_hip_plan **out);
int kvexp_hip_plan_destroy(kvexp_hip_plan *plan);
/* Re-targets a plan at its heads after their containers grew
 * (kvexp_hip_append): `heads` as at creation (same buffers, n_splits and
 * order of heads) with the new seq, bytes (the buffer capacity will do) and
 * n_blocks. While no head gains a block or a split tile, only the last
 * block of each container is read again (its descriptor and escape
 * positions are rewritten on the GPU) and the device heads and work items
 * are uploaded: stream-ordered on `stream` (the stream the plan runs on), no
 * synchronisation, no allocation; an index that does not cover seq is then
 * reported by the next checked run. Otherwise a new plan is built aside as
 * by kvexp_hip_plan_create (ordered on `stream`, after the runs queued
 * there) and replaces the old one only when complete. If an update fails
 * after argument checks (a damaged container, a misaligned split, a device
 * error), the plan refuses to run (KVEXP_HIP_FORMAT_ERROR naming the
 * failure) until a later update succeeds; its memory stays valid. No
 * counterpart in the reference, which has no plans. */
int kvexp_hip_plan_update(kvexp_hip_plan *plan, const kvexp_hip_head *heads, int n_heads, void *stream);
/* Suggested n_splits for a head of `seq` tokens so that a plan over
 * `n_heads` such heads fills the device (one wave group per split). */
int kvexp_hip_suggest_splits(kvexp_hip_ctx *ctx, int n_heads, int seq, int split_tokens);
/* The same for a given head_dim, query rows per head and score order (the
 * resident waves per SIMD depend on them); kvexp_hip_suggest_splits is this
 * at head_dim 64, 7 query rows, scalar order. */
int kvexp_hip_suggest_splits_for(kvexp_hip_ctx *ctx, int n_heads, int seq, int split_tokens, int dim, int n_q,
                                 int order);
/* One n_splits for a batch of heads of different lengths (seqs[n_heads];
 * heads of length 0 are skipped): the largest count whose longest split is
 * no longer than the mean split of one round of resident waves. Equal
 * lengths give kvexp_hip_suggest_splits_for's count. No counterpart in the
 * reference, where n_threads is the caller's choice. */
int kvexp_hip_suggest_splits_batch(kvexp_hip_ctx *ctx, int n_heads, const int *seqs, int split_tokens, int dim,
                                   int n_q, int order);

/* Runs a plan: d_q is [n_heads, n_q, dim] BF16; d_out [n_heads, n_q, dim]
 * FP32 is fully overwritten; d_lse (nullable) [n_heads, n_q] receives
 * m + log(l) per query row. With `check` non-zero the call synchronises
 * `stream` and reports container format errors found by the kernels. */
int kvexp_hip_attention_run(kvexp_hip_plan *plan, const uint16_t *d_q, float *d_out, float *d_lse, int check,
                            void *stream);
/* Reads and clears the plan's status word (synchronises `stream`). */
int kvexp_hip_plan_status(kvexp_hip_plan *plan, void *stream);

/* Split-kernel timing. No counterpart in the reference (its bench times the
 * whole call); it lets a benchmark time the dominant kernel alone. With
 * `enable` non-zero every later run records a HIP event pair around its
 * split-kernel launches on the run's stream; kvexp_hip_plan_kernel_time
 * waits for the recorded pairs, returns their summed time in ms and the
 * number of runs, and clears the record. */
int kvexp_hip_plan_timing(kvexp_hip_plan *plan, int enable);
int kvexp_hip_plan_kernel_time(kvexp_hip_plan *plan, double *ms, int *runs);

/* The Backend::Hip case of attention_decode: the reference argument list
 * with host pointers. Copies the inputs to the device, builds indexes and a
 * plan with n_splits = n_threads, runs it and copies `out` back, all on the
 * context's own stream (synchronised before returning). Reentrant across
 * contexts: the reference's attention_decode holds no shared state and its
 * bench calls it from an OpenMP parallel for (bench.cpp:715-728); callers
 * doing the same give each thread its own context. */
int kvexp_hip_attention_decode_host(kvexp_hip_ctx *ctx, int order, const uint16_t *q, const uint16_t *k_raw,
                                    const uint16_t *v_raw, const uint8_t *k_xkv, size_t k_bytes,
                                    const uint8_t *v_xkv, size_t v_bytes, float *out, int n_q, int dim, int seq,
                                    int n_threads, int split_tokens);

/* ------------------------------------------------------------ numerics ---- */
/* d_y[i] = exp(d_x[i]) with the kernels' exp, which returns the bits of the
 * reference's std::exp(float) (glibc 2.35 expf). No reference counterpart:
 * it lets a caller check that function on its own. */
int kvexp_hip_expf(kvexp_hip_ctx *ctx, const float *d_x, float *d_y, size_t n, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* KVEXP_HIP_H */
