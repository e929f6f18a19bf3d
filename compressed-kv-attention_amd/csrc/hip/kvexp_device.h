// Device helpers shared by the gfx950 kernels: container header checks, byte
// loads at any alignment, BF16 field assembly and wave64 scans (DPP).
//
// Container format (reference include/kvexp/codec.hpp:12-36): blocks of
//   u8 mode (0 raw, 2, 4) | u8 n_tokens | u16 n_escape | u16 head_dim | u16 0
// then raw BF16 rows, or base[dim], sm[n*dim], packed codes, u16 escapes.
// Mode 3 is this library's format extension (3-bit codes, sentinel 7,
// element i in bits [3i, 3i + 3) of the little-endian code bytes, head_dim a
// multiple of 8 so that rows start on a byte); the reference's readers
// reject it, and the encoders write it only when asked to.
#pragma once

#include <hip/hip_runtime.h>
#include <limits.h>
#include <stdint.h>

#include "kvexp_expf.h"
#include "kvexp_types.h"

namespace kvexp_dev {

constexpr int kMaxDim = 256;
constexpr int kWave = 64;

__device__ __forceinline__ uint32_t f32_bits(float x) { return __float_as_uint(x); }
__device__ __forceinline__ float bits_f32(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ float bf16_f32(uint32_t b) { return __uint_as_float(b << 16); }

// BF16 from an exponent (wrapping modulo 256, bf16.hpp:35-37) and a
// sign/mantissa byte (sign in bit 7).
__device__ __forceinline__ uint32_t bf16_join(uint32_t exponent, uint32_t sm) {
    return ((sm & 0x80u) << 8) | ((exponent & 0xFFu) << 7) | (sm & 0x7Fu);
}

// The four bytes [p, p+4) at any alignment, little-endian. Reads only the
// aligned dwords that hold those bytes, so a caller whose four bytes lie
// inside a buffer never touches a page outside it.
__device__ __forceinline__ uint32_t load_u32_any(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t sh = uint32_t(a & 3u);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
    const uint32_t lo = w[0];
    if (sh == 0) return lo;
    const uint32_t hi = w[1];
    return uint32_t(((uint64_t(hi) << 32) | lo) >> (sh * 8u));
}

__device__ __forceinline__ uint32_t load_u8(const uint8_t *p) { return *p; }
__device__ __forceinline__ uint32_t load_u16_any(const uint8_t *p) {
    return uint32_t(p[0]) | (uint32_t(p[1]) << 8);
}

struct BlockHdr {
    int mode, n_tokens, n_escape, dim;
};

__device__ __forceinline__ BlockHdr read_hdr(const uint8_t *p) {
    BlockHdr h;
    h.mode = p[0];
    h.n_tokens = p[1];
    h.n_escape = int(load_u16_any(p + 2));
    h.dim = int(load_u16_any(p + 4));
    return h;
}

__host__ __device__ __forceinline__ int exp_payload_bytes(int n, int dim, int bits) {
    return (n * dim * bits + 7) / 8;
}

// Byte size of a block from its header, or -1 when the mode is unknown.
__host__ __device__ __forceinline__ int64_t block_bytes(int mode, int n, int n_escape, int dim) {
    if (mode == 0) return 8 + 2 * int64_t(n) * dim;
    if (mode != 2 && mode != 4 && !(mode == 3 && dim % 8 == 0)) return -1;
    return 8 + int64_t(dim) + int64_t(n) * dim + exp_payload_bytes(n, dim, mode) + 2 * int64_t(n_escape);
}

// Status bits for the block at byte `off` of a container of `bytes` bytes
// that should hold `want_tokens` tokens of `dim` channels (0 = valid).
__device__ __forceinline__ uint32_t check_block(const uint8_t *blob, uint64_t bytes, int64_t off, int dim,
                                                int want_tokens, BlockHdr *out) {
    if (off < 0 || uint64_t(off) + 8u > bytes) return kStHeader;
    const BlockHdr h = read_hdr(blob + off);
    *out = h;
    if (h.dim != dim || h.n_tokens <= 0) return kStHeader;
    if (h.n_tokens != want_tokens) return kStIndex;
    const int64_t sz = block_bytes(h.mode, h.n_tokens, h.n_escape, dim);
    if (sz < 0) return kStMode;
    if (uint64_t(off) + uint64_t(sz) > bytes) return kStTruncated;
    return 0u;
}

// ------------------------------------------------------------- DPP scans --
// dpp_ctrl encodings (GFX9): row_shr:n = 0x110 + n, wave_shr:1 = 0x138,
// row_bcast:15 = 0x142, row_bcast:31 = 0x143.
template <int CTRL, int ROW_MASK = 0xf, bool BOUND_CTRL = false>
__device__ __forceinline__ float dpp_f32(float old, float src) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(src), CTRL, ROW_MASK,
                                                      0xf, BOUND_CTRL));
}
template <int CTRL, int ROW_MASK = 0xf, bool BOUND_CTRL = false>
__device__ __forceinline__ int dpp_i32(int old, int src) {
    return __builtin_amdgcn_update_dpp(old, src, CTRL, ROW_MASK, 0xf, BOUND_CTRL);
}

// Inclusive prefix maximum over the 64 lanes (IEEE maxNum: NaN lanes are
// ignored, as `(m < s) ? s : m` ignores a NaN score).
__device__ __forceinline__ float wave_scan_max(float x) {
    const float ninf = -__builtin_inff();
    x = fmaxf(x, dpp_f32<0x111>(ninf, x));
    x = fmaxf(x, dpp_f32<0x112>(ninf, x));
    x = fmaxf(x, dpp_f32<0x114>(ninf, x));
    x = fmaxf(x, dpp_f32<0x118>(ninf, x));
    x = fmaxf(x, dpp_f32<0x142, 0xa>(ninf, x));
    x = fmaxf(x, dpp_f32<0x143, 0xc>(ninf, x));
    return x;
}

// wave_scan_max of G values at once with the maximum fused into the DPP
// read (v_max_f32_dpp, one instruction per step and value), as one asm block
// so that its DPP hazards are under its own control: s_nop 1 before the
// first step (the inputs were written by the compiler's code just before) and
// after the last (a DPP read of a result may follow), and between steps when
// fewer than three values separate a write from the next read of the same
// VGPR (gfx9 needs two wait states between a VALU write and a DPP read).
// The inputs must not be signalling NaNs (they are arithmetic results or
// -inf), so the plain v_max_f32 needs no quieting. Lanes without a source
// lane keep their value, which is max(x, -inf).
#define KVEXP_DPPMAX(i, C) "v_max_f32_dpp %" #i ", %" #i ", %" #i " " C "\n"
#define KVEXP_DPPMAX_ROW1(C) KVEXP_DPPMAX(0, C)
#define KVEXP_DPPMAX_ROW2(C) KVEXP_DPPMAX_ROW1(C) KVEXP_DPPMAX(1, C)
#define KVEXP_DPPMAX_ROW3(C) KVEXP_DPPMAX_ROW2(C) KVEXP_DPPMAX(2, C)
#define KVEXP_DPPMAX_ROW4(C) KVEXP_DPPMAX_ROW3(C) KVEXP_DPPMAX(3, C)
#define KVEXP_DPPMAX_ROW5(C) KVEXP_DPPMAX_ROW4(C) KVEXP_DPPMAX(4, C)
#define KVEXP_DPPMAX_ROW6(C) KVEXP_DPPMAX_ROW5(C) KVEXP_DPPMAX(5, C)
#define KVEXP_DPPMAX_ROW7(C) KVEXP_DPPMAX_ROW6(C) KVEXP_DPPMAX(6, C)
#define KVEXP_DPPMAX_ROW8(C) KVEXP_DPPMAX_ROW7(C) KVEXP_DPPMAX(7, C)
#define KVEXP_DPPMAX_SCAN(N, PAD)                                                             \
    "s_nop 1\n" KVEXP_DPPMAX_ROW##N("row_shr:1 row_mask:0xf bank_mask:0xf") PAD            \
        KVEXP_DPPMAX_ROW##N("row_shr:2 row_mask:0xf bank_mask:0xf") PAD                     \
        KVEXP_DPPMAX_ROW##N("row_shr:4 row_mask:0xf bank_mask:0xf") PAD                     \
        KVEXP_DPPMAX_ROW##N("row_shr:8 row_mask:0xf bank_mask:0xf") PAD                     \
        KVEXP_DPPMAX_ROW##N("row_bcast:15 row_mask:0xa bank_mask:0xf") PAD                  \
        KVEXP_DPPMAX_ROW##N("row_bcast:31 row_mask:0xc bank_mask:0xf") "s_nop 1\n"

template <int G>
__device__ __forceinline__ void wave_scan_max_rows(float (&x)[G]);
template <>
__device__ __forceinline__ void wave_scan_max_rows<1>(float (&x)[1]) {
    asm volatile(KVEXP_DPPMAX_SCAN(1, "s_nop 1\n") : "+v"(x[0]));
}
template <>
__device__ __forceinline__ void wave_scan_max_rows<2>(float (&x)[2]) {
    asm volatile(KVEXP_DPPMAX_SCAN(2, "s_nop 0\n") : "+v"(x[0]), "+v"(x[1]));
}
template <>
__device__ __forceinline__ void wave_scan_max_rows<3>(float (&x)[3]) {
    asm volatile(KVEXP_DPPMAX_SCAN(3, "") : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]));
}
template <>
__device__ __forceinline__ void wave_scan_max_rows<4>(float (&x)[4]) {
    asm volatile(KVEXP_DPPMAX_SCAN(4, "") : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]));
}
template <>
__device__ __forceinline__ void wave_scan_max_rows<5>(float (&x)[5]) {
    asm volatile(KVEXP_DPPMAX_SCAN(5, "") : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]));
}
template <>
__device__ __forceinline__ void wave_scan_max_rows<6>(float (&x)[6]) {
    asm volatile(KVEXP_DPPMAX_SCAN(6, "")
                 : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]));
}
template <>
__device__ __forceinline__ void wave_scan_max_rows<7>(float (&x)[7]) {
    asm volatile(KVEXP_DPPMAX_SCAN(7, "")
                 : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]));
}
template <>
__device__ __forceinline__ void wave_scan_max_rows<8>(float (&x)[8]) {
    asm volatile(KVEXP_DPPMAX_SCAN(8, "")
                 : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]),
                   "+v"(x[7]));
}

// Value of lane - 1 (lane 0 gets `first`).
__device__ __forceinline__ float wave_shift_up(float x, float first) { return dpp_f32<0x138>(first, x); }

// Inclusive prefix sum of ints over the 64 lanes.
__device__ __forceinline__ int wave_scan_add(int x) {
    x += dpp_i32<0x111>(0, x);
    x += dpp_i32<0x112>(0, x);
    x += dpp_i32<0x114>(0, x);
    x += dpp_i32<0x118>(0, x);
    x += dpp_i32<0x142, 0xa>(0, x);
    x += dpp_i32<0x143, 0xc>(0, x);
    return x;
}

// Minimum, maximum and sum over the 64 lanes, returned to every lane (the
// scan pattern of wave_scan_add with the operation's identity shifted in,
// then lane 63's value).
__device__ __forceinline__ int wave_min_i32(int x) {
    x = min(x, dpp_i32<0x111>(INT_MAX, x));
    x = min(x, dpp_i32<0x112>(INT_MAX, x));
    x = min(x, dpp_i32<0x114>(INT_MAX, x));
    x = min(x, dpp_i32<0x118>(INT_MAX, x));
    x = min(x, dpp_i32<0x142, 0xa>(INT_MAX, x));
    x = min(x, dpp_i32<0x143, 0xc>(INT_MAX, x));
    return __builtin_amdgcn_readlane(x, 63);
}
__device__ __forceinline__ int wave_max_i32(int x) {
    x = max(x, dpp_i32<0x111>(INT_MIN, x));
    x = max(x, dpp_i32<0x112>(INT_MIN, x));
    x = max(x, dpp_i32<0x114>(INT_MIN, x));
    x = max(x, dpp_i32<0x118>(INT_MIN, x));
    x = max(x, dpp_i32<0x142, 0xa>(INT_MIN, x));
    x = max(x, dpp_i32<0x143, 0xc>(INT_MIN, x));
    return __builtin_amdgcn_readlane(x, 63);
}
__device__ __forceinline__ int wave_sum_i32(int x) { return __builtin_amdgcn_readlane(wave_scan_add(x), 63); }

__device__ __forceinline__ int lane_id() { return int(__lane_id()); }

__device__ __forceinline__ float readlane_f32(float x, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Exclusive prefix sum over a workgroup of NW waves. `tmp` holds NW ints in
// LDS. Returns the prefix and writes the workgroup total to *total. Every
// thread of the workgroup must call it.
template <int NW>
__device__ __forceinline__ int block_excl_scan(int v, int *tmp, int *total) {
    const int incl = wave_scan_add(v);
    const int lane = lane_id();
    const int wave = int(threadIdx.x) >> 6;
    if (lane == kWave - 1) tmp[wave] = incl;
    __syncthreads();
    int base = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const int t = tmp[w];
        base += (w < wave) ? t : 0;
        tot += t;
    }
    __syncthreads();
    *total = tot;
    return base + incl - v;
}

// Number of 4-bit codes equal to 15 (sentinels) in a dword of 8 codes.
__device__ __forceinline__ int sentinels4(uint32_t x) {
    uint32_t a = x & (x >> 1);
    a = a & (a >> 2);
    return __builtin_popcount(a & 0x11111111u);
}
// Number of 2-bit codes equal to 3 (sentinels) in a dword of 16 codes.
__device__ __forceinline__ int sentinels2(uint32_t x) {
    return __builtin_popcount(x & (x >> 1) & 0x55555555u);
}
// Number of 3-bit codes equal to 7 (sentinels) in the low 24 bits (8 codes).
__device__ __forceinline__ int sentinels3(uint32_t x) {
    return __builtin_popcount(x & (x >> 1) & (x >> 2) & 0x249249u);
}

// Code units of a coded block: the codes of elements [U u, U u + U), with
// U = 4 for 2- and 4-bit codes (one byte or two) and 8 for 3-bit codes
// (three bytes); code k of a unit is bits [mode k, mode k + mode).
__device__ __forceinline__ int code_unit(int mode) { return mode == 3 ? 8 : 4; }
__device__ __forceinline__ uint32_t load_codes(const uint8_t *codes, int mode, int u) {
    if (mode == 4) return load_u16_any(codes + 2 * size_t(u));
    if (mode == 2) return codes[u];
    const uint8_t *p = codes + 3 * size_t(u);
    return uint32_t(p[0]) | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16);
}
__device__ __forceinline__ int unit_sentinels(uint32_t cw, int mode) {
    return mode == 4 ? sentinels4(cw) : (mode == 2 ? sentinels2(cw) : sentinels3(cw));
}
__device__ __forceinline__ uint32_t unit_code(uint32_t cw, int mode, int k) {
    return (cw >> (mode * k)) & ((1u << mode) - 1u);
}

} // namespace kvexp_dev
