/* TEST INFRASTRUCTURE ONLY — CPU oracle for kvexp's fused decode path.
 *
 * A plain-C restatement of the reference algorithm, used by tests/ (and by
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg) as the checker of
 * the HIP product path. The product never links or calls it.
 *
 * Each function cites the reference file:line it restates (paths relative to
 * the reference repository root). Pinning, per function:
 *   - codec (encode/decode/parse/index): bit-exact against golden containers
 *     written by the compiled reference (tests/golden), against the compiled
 *     reference itself (oracle/_ref) on random inputs, and against closed
 *     forms (clean 4-bit block = 12360 B, clean 2-bit block = 10312 B,
 *     decode(encode(x)) == x).
 *   - scalar / avx2 attention: bit-exact against golden outputs and
 *     oracle/_ref; identity-token known answer; FP64 brute force within a
 *     tolerance on small inputs.
 *   - avx512 attention (VDPBF16PS score order, emulated here in portable C
 *     with DAZ on inputs and FTZ on outputs of each fused step): bit-exact
 *     against golden outputs from an AVX512_BF16 host and oracle/_ref.
 *   - expf/logf: glibc's own (the reference's std::exp(float)); the device
 *     restatement is compared with it exhaustively.
 *   - lse (m + logf(l)): no reference output exists; parity unpinned beyond
 *     its definition (tests check it against an FP64 log-sum-exp).
 *
 * Numeric flags: built with -ffp-contract=off -fno-fast-math like the
 * reference (CMakeLists.txt:48); every call runs with MXCSR FTZ and DAZ
 * cleared, which is the Linux x86-64 default the reference observes.
 */
#include "kvexp_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <xmmintrin.h>

#define KVEXP_MAX_DIM 256

enum { ST_OK = 0, ST_INVALID = 1, ST_RUNTIME = 2, ST_LOGIC = 3, ST_CAPACITY = 5 };

static __thread char g_err[256];

static int fail(int code, const char *msg) {
    snprintf(g_err, sizeof g_err, "%s", msg);
    return code;
}

const char *oracle_last_error(void) { return g_err; }

/* MXCSR with FTZ (bit 15) and DAZ (bit 6) cleared for the duration of a call. */
static unsigned ieee_enter(void) {
    unsigned old = _mm_getcsr();
    _mm_setcsr(old & ~((1u << 15) | (1u << 6)));
    return old;
}
static void ieee_leave(unsigned old) { _mm_setcsr(old); }

/* ---------------------------------------------------------------- BF16 ---- */
/* bf16.hpp:15-37 */
static inline float bf16_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline unsigned bf16_exponent(uint16_t b) { return (b >> 7) & 0xFFu; }
static inline unsigned bf16_signmant(uint16_t b) { return ((b >> 8) & 0x80u) | (b & 0x7Fu); }
/* exponent wraps modulo 256 (bf16.hpp:35-37: uint8_t(base + delta)). */
static inline uint16_t bf16_join(unsigned exponent, unsigned sm) {
    return (uint16_t)(((sm & 0x80u) << 8) | ((exponent & 0xFFu) << 7) | (sm & 0x7Fu));
}
static inline unsigned rd_u16(const uint8_t *p) { return (unsigned)p[0] | ((unsigned)p[1] << 8); }
static inline void wr_u16(uint8_t *p, unsigned v) {
    p[0] = (uint8_t)(v & 0xFF);
    p[1] = (uint8_t)(v >> 8);
}

/* bf16.hpp:39-49 */
int oracle_exp_payload_bytes(int n_tokens, int dim, int bits) { return (n_tokens * dim * bits + 7) / 8; }
int oracle_coded_block_bytes(int n_tokens, int dim, int bits, int n_escape) {
    return 8 + dim + n_tokens * dim + oracle_exp_payload_bytes(n_tokens, dim, bits) + 2 * n_escape;
}
int oracle_raw_block_bytes(int n_tokens, int dim) { return 8 + 2 * n_tokens * dim; }

size_t oracle_encode_bound(int seq, int dim, int block) {
    if (seq <= 0 || dim <= 0 || block <= 0) return 0;
    size_t nb = ((size_t)seq + (size_t)block - 1) / (size_t)block;
    return nb * 8u + 2u * (size_t)seq * (size_t)dim;
}

/* ------------------------------------------------------------- encoder ---- */
/* best_base (codec.cpp:18-35): the smallest base b in [0, 256-width] whose
 * window [b, b+width) holds the most exponents. Sliding-window count; the
 * strict comparison keeps the first (smallest) maximiser. */
static int window_base(const int *hist, int width, int *covered) {
    int c = 0;
    for (int e = 0; e < width; ++e) c += hist[e];
    int best = c, base = 0;
    for (int b = 1; b <= 256 - width; ++b) {
        c += hist[b + width - 1] - hist[b - 1];
        if (c > best) {
            best = c;
            base = b;
        }
    }
    *covered = best;
    return base;
}

/* Mode choice (codec.cpp:75-103): raw first, then 2-bit, then 4-bit; a
 * candidate replaces the current best when strictly smaller, or on a size tie
 * when the best is not raw and it has fewer escapes (or equal escapes and
 * fewer bits). With the 3-bit extension allowed (bit 3 of `modes`, head_dim
 * a multiple of 8) it competes between them, which gives the order of the
 * reference's sizer (analyze_exponents.py:117-143: smallest container, then
 * raw, then fewer escapes, then narrower codes). */
typedef struct {
    int mode, bytes, escapes;
} mode_choice;

static mode_choice choose_mode(const int *hist, int n, int dim, unsigned modes) {
    mode_choice best = {0, oracle_raw_block_bytes(n, dim), 0};
    for (int bits = 2; bits <= 4; ++bits) {
        if (!(modes & (1u << bits)) || (bits == 3 && dim % 8 != 0)) continue;
        const int width = (1 << bits) - 1;
        int esc = 0;
        for (int d = 0; d < dim; ++d) {
            int cov = 0;
            (void)window_base(hist + (size_t)d * 256, width, &cov);
            esc += n - cov;
        }
        mode_choice c = {bits, oracle_coded_block_bytes(n, dim, bits, esc), esc};
        int smaller = c.bytes < best.bytes;
        int tie_win = c.bytes == best.bytes && best.mode != 0 &&
                      (c.escapes < best.escapes || (c.escapes == best.escapes && c.mode < best.mode));
        if (smaller || tie_win) best = c;
    }
    return best;
}

/* Code `code` of element i at bits [bits i, bits i + bits) of the code bytes,
 * least significant bit first (codec.hpp:27-31 for 4 and 2 bits; the same
 * rule for the 3-bit extension, whose codes may straddle two bytes). */
static inline void put_code(uint8_t *codes, int i, int bits, int code) {
    const int bit = i * bits;
    codes[bit >> 3] |= (uint8_t)(code << (bit & 7));
    if ((bit & 7) + bits > 8) codes[(bit >> 3) + 1] |= (uint8_t)(code >> (8 - (bit & 7)));
}

/* encode_bf16 (codec.cpp:39-164), container layout codec.hpp:12-36. */
int oracle_encode(const uint16_t *kv, int seq, int dim, int block, uint8_t *out, size_t cap,
                  size_t *out_bytes) {
    return oracle_encode_modes(kv, seq, dim, block, ORACLE_MODES_REFERENCE, out, cap, out_bytes);
}

int oracle_encode_modes(const uint16_t *kv, int seq, int dim, int block, unsigned modes, uint8_t *out,
                        size_t cap, size_t *out_bytes) {
    if (kv == NULL || seq <= 0 || dim <= 0 || block <= 0)
        return fail(ST_INVALID, "encode_bf16: empty input");
    if (dim % 4 != 0 || dim > KVEXP_MAX_DIM)
        return fail(ST_INVALID, "encode_bf16: head_dim must be a multiple of 4 and at most 256");
    if (block > 255) return fail(ST_INVALID, "encode_bf16: block_tokens must fit in a byte");
    if ((int64_t)block * dim > 65535)
        return fail(ST_INVALID, "encode_bf16: block escape count would not fit in u16");

    int *hist = (int *)malloc(sizeof(int) * 256 * (size_t)dim);
    if (!hist) return fail(ST_LOGIC, "oracle: out of memory");
    size_t pos = 0;
    int overflow = 0;
    for (int t0 = 0; t0 < seq; t0 += block) {
        const int n = (seq - t0 < block) ? seq - t0 : block;
        const uint16_t *src = kv + (size_t)t0 * (size_t)dim;
        memset(hist, 0, sizeof(int) * 256 * (size_t)dim);
        for (int t = 0; t < n; ++t)
            for (int d = 0; d < dim; ++d) ++hist[(size_t)d * 256 + bf16_exponent(src[(size_t)t * dim + d])];
        const mode_choice mc = choose_mode(hist, n, dim, modes);
        if (pos + (size_t)mc.bytes > cap) {
            overflow = 1;
            pos += (size_t)mc.bytes;
            continue;
        }
        uint8_t *blk = out + pos;
        blk[0] = (uint8_t)mc.mode;
        blk[1] = (uint8_t)n;
        wr_u16(blk + 2, mc.mode == 0 ? 0u : (unsigned)mc.escapes);
        wr_u16(blk + 4, (unsigned)dim);
        wr_u16(blk + 6, 0u);
        uint8_t *p = blk + 8;
        if (mc.mode == 0) {
            for (int i = 0; i < n * dim; ++i) wr_u16(p + 2 * i, src[i]);
            pos += (size_t)mc.bytes;
            continue;
        }
        const int bits = mc.mode;
        const int width = (1 << bits) - 1; /* codes 0..width-1; width is the sentinel */
        uint8_t *basep = p, *smp = p + dim, *codes = smp + (size_t)n * dim;
        const int payload = oracle_exp_payload_bytes(n, dim, bits);
        uint8_t *escp = codes + payload;
        memset(codes, 0, (size_t)payload);
        for (int d = 0; d < dim; ++d) {
            int cov;
            basep[d] = (uint8_t)window_base(hist + (size_t)d * 256, width, &cov);
        }
        int n_esc = 0;
        for (int i = 0; i < n * dim; ++i) {
            const uint16_t h = src[i];
            smp[i] = (uint8_t)bf16_signmant(h);
            const int delta = (int)bf16_exponent(h) - (int)basep[i % dim];
            int code = width;
            if (delta >= 0 && delta < width) {
                code = delta;
            } else {
                wr_u16(escp + 2 * n_esc, h);
                ++n_esc;
            }
            put_code(codes, i, bits, code);
        }
        if (n_esc != mc.escapes) {
            free(hist);
            return fail(ST_LOGIC, "escape count drifted from the size model");
        }
        pos += (size_t)mc.bytes;
    }
    free(hist);
    *out_bytes = pos;
    if (overflow) return fail(ST_CAPACITY, "oracle_encode: output capacity too small");
    return ST_OK;
}

/* ------------------------------------------------------ block parsing ---- */
typedef struct {
    int mode, n_tokens, n_escape;
    const uint8_t *base, *sm, *codes, *esc, *raw, *next;
} block_view;

/* parse_block (scan.hpp:28-66). */
static int parse_block(const uint8_t *p, const uint8_t *end, int dim, block_view *b) {
    if (end - p < 8) return fail(ST_RUNTIME, "truncated xkv block header");
    memset(b, 0, sizeof *b);
    b->mode = p[0];
    b->n_tokens = p[1];
    b->n_escape = (int)rd_u16(p + 2);
    const int hdim = (int)rd_u16(p + 4);
    if (hdim != dim || b->n_tokens <= 0) return fail(ST_RUNTIME, "xkv block dimension or length mismatch");
    p += 8;
    if (b->mode == 0) {
        const size_t nbytes = (size_t)b->n_tokens * (size_t)dim * 2u;
        if ((size_t)(end - p) < nbytes) return fail(ST_RUNTIME, "truncated raw xkv block");
        b->raw = p;
        b->next = p + nbytes;
        return ST_OK;
    }
    /* mode 3: the 3-bit extension (head_dim a multiple of 8) */
    if (b->mode != 2 && b->mode != 4 && !(b->mode == 3 && dim % 8 == 0))
        return fail(ST_RUNTIME, "unknown xkv block mode");
    const size_t sm_bytes = (size_t)b->n_tokens * (size_t)dim;
    const size_t code_bytes = (size_t)oracle_exp_payload_bytes(b->n_tokens, dim, b->mode);
    const size_t esc_bytes = (size_t)b->n_escape * 2u;
    const size_t need = (size_t)dim + sm_bytes + code_bytes + esc_bytes;
    if ((size_t)(end - p) < need) return fail(ST_RUNTIME, "truncated coded xkv block");
    b->base = p;
    b->sm = p + dim;
    b->codes = b->sm + sm_bytes;
    b->esc = b->codes + code_bytes;
    b->next = b->esc + esc_bytes;
    return ST_OK;
}

/* residual_code (scan.hpp:68-75); 3-bit codes as put_code writes them. */
static inline int residual(const uint8_t *codes, int index, int bits) {
    if (bits == 4) {
        const uint8_t byte = codes[index >> 1];
        return (index & 1) ? (byte >> 4) : (byte & 0x0F);
    }
    if (bits == 3) {
        const int bit = index * 3, sh = bit & 7;
        unsigned w = codes[bit >> 3];
        if (sh > 5) w |= (unsigned)codes[(bit >> 3) + 1] << 8;
        return (int)((w >> sh) & 7u);
    }
    return (codes[index >> 2] >> ((index & 3) * 2)) & 0x03;
}

/* Row cursor over a container: the readers XkvReader (scan.hpp:79-165) and
 * XkvPos/open_xkv (scan.hpp:168-218) consume whole rows from a block-aligned
 * token and parse the next header as soon as a block's last element is read. */
typedef struct {
    block_view blk;
    const uint8_t *end;
    int dim, local, esc_i, done;
} row_cursor;

/* seek / open_xkv (scan.hpp:94-123, 192-218). */
static int cursor_open(row_cursor *c, const uint8_t *data, size_t size, int dim, int token) {
    c->end = data + size;
    c->dim = dim;
    c->local = 0;
    c->esc_i = 0;
    c->done = 1;
    const uint8_t *p = data;
    int at = 0;
    if (token < 0) return fail(ST_RUNTIME, "negative token");
    while (at < token) {
        if (p >= c->end) return fail(ST_RUNTIME, "xkv seek past end");
        block_view b;
        int rc = parse_block(p, c->end, dim, &b);
        if (rc) return rc;
        if (at + b.n_tokens > token) return fail(ST_RUNTIME, "token split is not aligned to an encoded block");
        at += b.n_tokens;
        p = b.next;
    }
    if (p >= c->end) return ST_OK;
    int rc = parse_block(p, c->end, dim, &c->blk);
    if (rc) return rc;
    c->done = 0;
    return ST_OK;
}

/* Decodes the cursor's current row into dst[dim] (read_next, scan.hpp:125-155;
 * load_token, attention_avx2.cpp:87-108), then advances with the eager header
 * parse (advance_token, scan.hpp:176-189). The escape stream is bounds-checked:
 * a block with more sentinels than n_escape is reported, not read past. */
static int cursor_row(row_cursor *c, uint16_t *dst) {
    const block_view *b = &c->blk;
    const int dim = c->dim;
    const int row0 = c->local * dim;
    if (b->mode == 0) {
        for (int d = 0; d < dim; ++d) dst[d] = (uint16_t)rd_u16(b->raw + 2 * (size_t)(row0 + d));
    } else {
        const int sentinel = (1 << b->mode) - 1;
        for (int d = 0; d < dim; ++d) {
            const int idx = row0 + d;
            const int code = residual(b->codes, idx, b->mode);
            if (code == sentinel) {
                if (c->esc_i >= b->n_escape) return fail(ST_RUNTIME, "xkv escape stream overrun");
                dst[d] = (uint16_t)rd_u16(b->esc + 2 * (size_t)c->esc_i);
                ++c->esc_i;
            } else {
                dst[d] = bf16_join(b->base[d] + (unsigned)code, b->sm[idx]);
            }
        }
    }
    ++c->local;
    if (c->local < b->n_tokens) return ST_OK;
    if (b->next >= c->end) {
        c->done = 1;
        return ST_OK;
    }
    const uint8_t *nx = b->next;
    int rc = parse_block(nx, c->end, dim, &c->blk);
    if (rc) return rc;
    c->local = 0;
    c->esc_i = 0;
    return ST_OK;
}

/* decode_bf16 (codec.cpp:166-174): element-sequential read of seq*dim values. */
int oracle_decode(const uint8_t *blob, size_t bytes, int seq, int dim, uint16_t *out) {
    row_cursor c;
    int rc = cursor_open(&c, blob, bytes, dim, 0);
    if (rc) return rc;
    for (int t = 0; t < seq; ++t) {
        if (c.done) return fail(ST_RUNTIME, "xkv decode ran out of blocks");
        rc = cursor_row(&c, out + (size_t)t * (size_t)dim);
        if (rc) return rc;
    }
    return ST_OK;
}

int oracle_block_index(const uint8_t *blob, size_t bytes, int dim, int seq, int64_t *offsets,
                       int32_t *first_token, int max_blocks, int *n_blocks) {
    const uint8_t *p = blob, *end = blob + bytes;
    int nb = 0, tok = 0;
    /* Blocks covering [0, seq), then one eager header parse (scan.hpp:144-151). */
    while (p < end) {
        block_view b;
        int rc = parse_block(p, end, dim, &b);
        if (rc) return rc;
        if (tok >= seq) break; /* the eager parse of the block after the last one used */
        if (nb >= max_blocks) return fail(ST_CAPACITY, "oracle_block_index: too many blocks");
        offsets[nb] = (int64_t)(p - blob);
        first_token[nb] = tok;
        ++nb;
        tok += b.n_tokens;
        p = b.next;
    }
    offsets[nb] = (int64_t)(p - blob);
    first_token[nb] = tok;
    *n_blocks = nb;
    return ST_OK;
}

int oracle_container_stats(const uint8_t *blob, size_t bytes, int dim, int64_t *n_raw,
                           int64_t *n_2bit, int64_t *n_4bit, int64_t *n_escapes) {
    const uint8_t *p = blob, *end = blob + bytes;
    *n_raw = *n_2bit = *n_4bit = *n_escapes = 0;
    while (p < end) {
        block_view b;
        int rc = parse_block(p, end, dim, &b);
        if (rc) return rc;
        if (b.mode == 0) ++*n_raw;
        if (b.mode == 2) ++*n_2bit;
        if (b.mode == 4) ++*n_4bit;
        if (b.mode != 0) *n_escapes += b.n_escape;
        p = b.next;
    }
    return ST_OK;
}

int oracle_container_mode_counts(const uint8_t *blob, size_t bytes, int dim, int64_t *counts) {
    const uint8_t *p = blob, *end = blob + bytes;
    for (int i = 0; i < 5; ++i) counts[i] = 0;
    while (p < end) {
        block_view b;
        int rc = parse_block(p, end, dim, &b);
        if (rc) return rc;
        ++counts[b.mode];
        p = b.next;
    }
    return ST_OK;
}

/* ------------------------------------------------------------ softmax ---- */
/* std::max(a, b) is (a < b) ? b : a. */
static inline float ref_max(float a, float b) { return (a < b) ? b : a; }

/* softmax_coeff (src/softmax.hpp:8-14). */
static inline void softmax_coeff(float *m, float *l, float s, float *alpha, float *e) {
    const float m2 = ref_max(*m, s);
    *alpha = expf(*m - m2);
    *e = expf(s - m2);
    *l = fmaf(*l, *alpha, *e);
    *m = m2;
}

/* merge_state (src/softmax.hpp:16-30). */
static void merge_state(float *m, float *l, float *acc, const float *mb, const float *lb,
                        const float *accb, int n_q, int dim) {
    for (int g = 0; g < n_q; ++g) {
        const float mm = ref_max(m[g], mb[g]);
        const float e1 = expf(m[g] - mm);
        const float e2 = expf(mb[g] - mm);
        l[g] = fmaf(l[g], e1, lb[g] * e2);
        float *a = acc + (size_t)g * dim;
        const float *b = accb + (size_t)g * dim;
        for (int d = 0; d < dim; ++d) a[d] = fmaf(a[d], e1, b[d] * e2);
        m[g] = mm;
    }
}

/* finalize_state (src/softmax.hpp:32-41): out = acc * (1/l). */
static void finalize_state(const float *l, const float *acc, float *out, int n_q, int dim) {
    for (int g = 0; g < n_q; ++g) {
        const float inv = 1.0f / l[g];
        for (int d = 0; d < dim; ++d) out[(size_t)g * dim + d] = acc[(size_t)g * dim + d] * inv;
    }
}

/* -------------------------------------------------------------- scores ---- */
/* hsum8 + apply_token score loop (attention_scalar.cpp:13-29): 8 strided FMA
 * lanes over d, then ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)). AVX2 computes the
 * same bits (hsum256, attention_avx2.cpp:15-22,112-120). */
static inline float score_scalar_f(const float *qf, const uint16_t *k, int dim) {
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int d = 0; d < dim; d += 8)
        for (int j = 0; j < 8; ++j) lane[j] = fmaf(qf[d + j], bf16_f32(k[d + j]), lane[j]);
    const float a = (lane[0] + lane[4]) + (lane[1] + lane[5]);
    const float b = (lane[2] + lane[6]) + (lane[3] + lane[7]);
    return a + b;
}

/* DAZ on inputs / FTZ on outputs as VDPBF16PS applies them. */
static inline float flush_denorm(float x) {
    return (fpclassify(x) == FP_SUBNORMAL) ? copysignf(0.0f, x) : x;
}

/* VDPBF16PS lane step (Intel SDM): acc += k[2j+1]*q[2j+1], then acc +=
 * k[2j]*q[2j], each a single-rounding FMA (RNE) with DAZ inputs and FTZ output. */
static inline float dpbf16_step(float acc, uint16_t k_even, uint16_t k_odd, uint16_t q_even,
                                uint16_t q_odd) {
    acc = flush_denorm(fmaf(flush_denorm(bf16_f32(k_odd)), flush_denorm(bf16_f32(q_odd)), flush_denorm(acc)));
    acc = flush_denorm(fmaf(flush_denorm(bf16_f32(k_even)), flush_denorm(bf16_f32(q_even)), flush_denorm(acc)));
    return acc;
}

/* apply512 score loop + hsum512 (attention_avx512.cpp:21-30,116-124): 16 lanes,
 * lane j takes elements 32i+2j and 32i+2j+1 of every 32-element step, then a
 * pairwise tree over the 16 lanes. */
static inline float score_dpbf16(const uint16_t *q, const uint16_t *k, int dim) {
    float t[16];
    for (int j = 0; j < 16; ++j) t[j] = 0.0f;
    for (int c = 0; c < dim; c += 32)
        for (int j = 0; j < 16; ++j)
            t[j] = dpbf16_step(t[j], k[c + 2 * j], k[c + 2 * j + 1], q[c + 2 * j], q[c + 2 * j + 1]);
    const float a0 = (t[0] + t[1]) + (t[2] + t[3]);
    const float a1 = (t[4] + t[5]) + (t[6] + t[7]);
    const float a2 = (t[8] + t[9]) + (t[10] + t[11]);
    const float a3 = (t[12] + t[13]) + (t[14] + t[15]);
    return (a0 + a1) + (a2 + a3);
}

float oracle_score_scalar(const uint16_t *q, const uint16_t *k, int dim) {
    unsigned old = ieee_enter();
    float qf[KVEXP_MAX_DIM];
    for (int d = 0; d < dim; ++d) qf[d] = bf16_f32(q[d]);
    float s = score_scalar_f(qf, k, dim);
    ieee_leave(old);
    return s;
}

float oracle_score_dpbf16(const uint16_t *q, const uint16_t *k, int dim) {
    unsigned old = ieee_enter();
    float s = score_dpbf16(q, k, dim);
    ieee_leave(old);
    return s;
}

/* --------------------------------------------------------- range kernel ---- */
/* One token of apply_token (attention_scalar.cpp:19-42) / apply_regs
 * (attention_avx2.cpp:110-134) / apply512 (attention_avx512.cpp:114-138). */
static void apply_token(int backend, const uint16_t *q, const float *qf, const uint16_t *k,
                        const uint16_t *v, int n_q, int dim, float *m, float *l, float *acc,
                        float *score, float *alpha, float *e) {
    for (int g = 0; g < n_q; ++g)
        score[g] = (backend == 2) ? score_dpbf16(q + (size_t)g * dim, k, dim)
                                  : score_scalar_f(qf + (size_t)g * dim, k, dim);
    for (int g = 0; g < n_q; ++g) softmax_coeff(&m[g], &l[g], score[g], &alpha[g], &e[g]);
    for (int g = 0; g < n_q; ++g) {
        float *ag = acc + (size_t)g * dim;
        for (int d = 0; d < dim; ++d) ag[d] = fmaf(e[g], bf16_f32(v[d]), ag[d] * alpha[g]);
    }
}

static const char *ran_out_msg(int backend) {
    if (backend == 1) return "avx2 xkv ran out of tokens";
    if (backend == 2) return "avx512 xkv ran out of tokens";
    return "xkv ran out of tokens"; /* the scalar reader does not check (undefined there) */
}

/* range_scalar / range_avx2 / range_avx512 (attention_scalar.cpp:46-85,
 * attention_avx2.cpp:138-185, attention_avx512.cpp:153-196) over [t0, t1). */
static int range_tokens(int backend, const uint16_t *q, const uint16_t *k_raw, const uint16_t *v_raw,
                        const uint8_t *k_xkv, size_t k_bytes, const uint8_t *v_xkv, size_t v_bytes,
                        int n_q, int dim, int t0, int t1, float *m, float *l, float *acc) {
    if (backend == 2) {
        if (dim % 32 != 0 || dim <= 0 || dim > KVEXP_MAX_DIM || n_q <= 0)
            return fail(ST_INVALID, "avx512 attention: head_dim must be a multiple of 32");
    } else if (dim % 8 != 0 || dim <= 0 || dim > KVEXP_MAX_DIM || n_q <= 0) {
        return fail(ST_INVALID, backend == 1 ? "avx2 attention: bad shape" : "scalar attention: bad shape");
    }
    if (t0 >= t1) return ST_OK;
    float *qf = (float *)malloc(sizeof(float) * ((size_t)n_q * dim + 3u * (size_t)n_q));
    float *score = qf + (size_t)n_q * dim, *alpha = score + n_q, *e = alpha + n_q;
    uint16_t kt[KVEXP_MAX_DIM], vt[KVEXP_MAX_DIM];
    for (int i = 0; i < n_q * dim; ++i) qf[i] = bf16_f32(q[i]);
    int rc = ST_OK;
    if (k_raw != NULL) {
        for (int t = t0; t < t1; ++t)
            apply_token(backend, q, qf, k_raw + (size_t)t * dim, v_raw + (size_t)t * dim, n_q, dim, m, l, acc,
                        score, alpha, e);
        free(qf);
        return ST_OK;
    }
    row_cursor kc, vc;
    rc = cursor_open(&kc, k_xkv, k_bytes, dim, t0);
    if (!rc) rc = cursor_open(&vc, v_xkv, v_bytes, dim, t0);
    for (int t = t0; t < t1 && !rc; ++t) {
        if (kc.done || vc.done) {
            rc = fail(ST_RUNTIME, ran_out_msg(backend));
            break;
        }
        rc = cursor_row(&kc, kt);
        if (!rc) rc = cursor_row(&vc, vt);
        if (!rc) apply_token(backend, q, qf, kt, vt, n_q, dim, m, l, acc, score, alpha, e);
    }
    free(qf);
    return rc;
}

/* token_bounds (dispatch.cpp:17-23). */
static void token_bounds(int seq, int tile, int tid, int nthreads, int *a, int *b) {
    const int ntiles = (seq + tile - 1) / tile;
    const int b0 = (int)((long long)tid * ntiles / nthreads);
    const int b1 = (int)((long long)(tid + 1) * ntiles / nthreads);
    *a = (seq < b0 * tile) ? seq : b0 * tile;
    *b = (seq < b1 * tile) ? seq : b1 * tile;
}

/* attention_decode (dispatch.cpp:27-104). */
static int attention_one(int backend, const uint16_t *q, const uint16_t *k_raw, const uint16_t *v_raw,
                         const uint8_t *k_xkv, size_t k_bytes, const uint8_t *v_xkv, size_t v_bytes,
                         float *out, float *lse, int n_q, int dim, int seq, int n_threads,
                         int split_tokens) {
    if (q == NULL || out == NULL || n_q <= 0 || dim <= 0 || seq <= 0 || split_tokens <= 0)
        return fail(ST_INVALID, "attention_decode: bad argument");
    const int raw = k_raw != NULL, xkv = k_xkv != NULL;
    if (raw == xkv || (v_raw != NULL) != raw || (v_xkv != NULL) != xkv)
        return fail(ST_INVALID, "attention_decode: pass raw K and V or xkv K and V, not both");
    if (backend < 0 || backend > 2) return fail(ST_INVALID, "oracle: unknown backend");
    const int ntiles = (seq + split_tokens - 1) / split_tokens;
    int threads = n_threads < 1 ? 1 : n_threads;
    if (threads > ntiles) threads = ntiles;

    const size_t ns = (size_t)n_q, na = (size_t)n_q * (size_t)dim;
    float *m = (float *)malloc(sizeof(float) * ns * threads);
    float *l = (float *)malloc(sizeof(float) * ns * threads);
    float *acc = (float *)calloc(na * threads, sizeof(float));
    for (size_t i = 0; i < ns * threads; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
    }
    int rc = ST_OK;
    for (int tid = 0; tid < threads && !rc; ++tid) {
        int a, b;
        token_bounds(seq, split_tokens, tid, threads, &a, &b);
        if (a < b)
            rc = range_tokens(backend, q, k_raw, v_raw, k_xkv, k_bytes, v_xkv, v_bytes, n_q, dim, a, b,
                              m + ns * tid, l + ns * tid, acc + na * tid);
    }
    if (!rc) {
        for (int t = 1; t < threads; ++t)
            merge_state(m, l, acc, m + ns * t, l + ns * t, acc + na * t, n_q, dim);
        finalize_state(l, acc, out, n_q, dim);
        if (lse)
            for (int g = 0; g < n_q; ++g) lse[g] = m[g] + logf(l[g]);
    }
    free(m);
    free(l);
    free(acc);
    return rc;
}

int oracle_attention(int backend, const uint16_t *q, const uint16_t *k_raw, const uint16_t *v_raw,
                     const uint8_t *k_xkv, size_t k_bytes, const uint8_t *v_xkv, size_t v_bytes,
                     float *out, float *lse, int n_q, int dim, int seq, int n_threads,
                     int split_tokens) {
    unsigned old = ieee_enter();
    int rc = attention_one(backend, q, k_raw, v_raw, k_xkv, k_bytes, v_xkv, v_bytes, out, lse, n_q,
                           dim, seq, n_threads, split_tokens);
    ieee_leave(old);
    return rc;
}

int oracle_attention_heads(int backend, int n_heads, const uint16_t *q,
                           const uint16_t *const *k_raw, const uint16_t *const *v_raw,
                           const uint8_t *const *k_xkv, const uint64_t *k_bytes,
                           const uint8_t *const *v_xkv, const uint64_t *v_bytes, float *out,
                           float *lse, int n_q, int dim, const int32_t *seq,
                           const int32_t *n_threads, int split_tokens, int *status_per_head) {
    int first_bad = -1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int h = 0; h < n_heads; ++h) {
        unsigned old = ieee_enter();
        const size_t qo = (size_t)h * n_q * dim;
        int rc = attention_one(backend, q + qo, k_raw ? k_raw[h] : NULL, v_raw ? v_raw[h] : NULL,
                               k_xkv ? k_xkv[h] : NULL, k_bytes ? (size_t)k_bytes[h] : 0,
                               v_xkv ? v_xkv[h] : NULL, v_bytes ? (size_t)v_bytes[h] : 0, out + qo,
                               lse ? lse + (size_t)h * n_q : NULL, n_q, dim, seq[h], n_threads[h],
                               split_tokens);
        ieee_leave(old);
        status_per_head[h] = rc;
        if (rc) {
#pragma omp critical
            if (first_bad < 0 || h < first_bad) first_bad = h;
        }
    }
    return first_bad < 0 ? ST_OK : status_per_head[first_bad];
}

/* ------------------------------------------------------------- expf ---- */
void oracle_expf_array(const float *x, float *y, size_t n) {
    unsigned old = ieee_enter();
    for (size_t i = 0; i < n; ++i) y[i] = expf(x[i]);
    ieee_leave(old);
}

static inline int same_float(float a, float b) {
    if (isnan(a) && isnan(b)) return 1;
    uint32_t ua, ub;
    memcpy(&ua, &a, 4);
    memcpy(&ub, &b, 4);
    return ua == ub;
}

size_t oracle_expf_compare(const float *x, const float *y, size_t n, int64_t *first) {
    unsigned old = ieee_enter();
    size_t bad = 0;
    *first = -1;
    for (size_t i = 0; i < n; ++i) {
        if (!same_float(expf(x[i]), y[i])) {
            if (*first < 0) *first = (int64_t)i;
            ++bad;
        }
    }
    ieee_leave(old);
    return bad;
}

size_t oracle_expf_compare_range(uint32_t lo, uint32_t hi, const float *y, int64_t *first) {
    unsigned old = ieee_enter();
    size_t bad = 0;
    *first = -1;
    for (uint64_t u = lo; u < hi; ++u) {
        uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        if (!same_float(expf(x), y[u - lo])) {
            if (*first < 0) *first = (int64_t)(u - lo);
            ++bad;
        }
    }
    ieee_leave(old);
    return bad;
}
