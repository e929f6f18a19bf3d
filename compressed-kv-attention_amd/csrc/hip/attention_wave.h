// The one-wave split kernel and its merge (templates), shared by the
// translation units that instantiate them: attention_wave.hip (head_dim 64
// and 128, the merges, the entry points) and attention_wave256.hip (head_dim
// 256), compiled in parallel.
#pragma once
// gfx950 fused decode attention, head_dim 64, 128 or 256, scalar/AVX2 and
// AVX-512 BF16 score orders: one wave64 per split, no workgroup barriers on
// the hot path.
//
// A split [tok_begin, tok_end) of one KV head is processed in chunks of up to
// 64 tokens that never cross a K or V block; the order below is the loop's,
// except that the softmax (4) runs before the V decode (3), so that the
// scores are no longer live while V is decoded. Per chunk the wave:
//   1. decodes the chunk's K rows from registers loaded one chunk ahead (16-
//      channel pieces, consecutive lanes on consecutive bytes, so every load
//      instruction reads a few whole cache lines) into a BF16 tile in its own
//      LDS slice (row t: token t): a coded element is
//      (sm & 0x80) << 8 | (base + code) << 7 | (sm & 0x7F), built two at a
//      time with v_perm_b32 / v_lshl_add_u32 / v_bfi_b32 on packed pairs;
//      escape words are then written over their elements from the plan's
//      escape records (position and word in one dword; a cursor per tensor:
//      the window of 256 (2,048 at head_dim 256) loaded with the rows starts at the chunk's first
//      escape, and a chunk is cut short where its escapes would not fit);
//      raw blocks are copied in chunks of at most 48 rows (the registers of
//      64 coded rows). Every lane issues the same loads on every path, so
//      the compiler's waits for the K rows leave the V rows in flight. At
//      head_dim 64 (lane = row in the decode as in the scores), a 4- or
//      2-bit chunk without escapes (and, in the AVX-512 order, without a
//      possible flush) skips the tile: its pairs are decoded straight into
//      the score products (scores_coded, scores_dp_of);
//   2. computes the G scores of each token in the reference order: 8 strided
//      FMA chains over the head's channels, then the
//      ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)) tree. Every fmaf of the chains is
//      done on the matrix cores as a rank-1 product
//      (v_mfma_f32_4x4x1_16b_f32, one IEEE fused multiply-add per element, the
//      same bits as fmaf): four query rows (A, the block-broadcast operand)
//      times the lane's token (B), one instruction per channel and row group;
//   3. decodes the V rows into the same tile (tokens past the chunk's end get
//      -0, which the fold adds as an exact no-op);
//   4. turns scores into e = exp(s - m) and, for the query rows where some
//      token moves the running maximum, alpha = exp(m_prev - m), with an
//      exact DPP prefix maximum seeded by the maxima held in scalar registers
//      and the glibc-identical expf; e and alpha go to LDS by query row;
//   5. folds the chunk's tokens in order (lane = channel; at head_dim 128
//      each lane holds channels lane and lane + 64), unrolled (at head_dim
//      256 a group of 16 tokens that moves a maximum runs as a loop, to keep
//      the code within the instruction cache):
//      acc = fma(e, v, acc) as one rank-1 product per token and row group
//      (e of four rows in A, picked per token by the block broadcast; the
//      token's V row in B), with acc scaled by alpha first only on the tokens
//      that move a maximum (a uniform branch; alpha == 1 elsewhere, so
//      skipping the multiply is exact), and l = fma(l, alpha, e) on lane g.
// A head cut into several splits leaves one partial state (m, l, acc) per
// split; wave_merge_kernel, launched after the split kernels, folds them left
// to right (merge_state order) and finalizes out = acc * (1/l).
//
// Every float operation is the reference's (attention_scalar.cpp:19-85,
// softmax.hpp:8-41, dispatch.cpp:98-103), so outputs equal the reference's
// bits for the same split, and the raw instantiation equals the XKV one.
#include "kvexp_device.h"
#include "kvexp_types.h"

namespace kvexp_dev {
namespace wave {

// Phase trace (builds with KVEXP_PHASE_TRACE only: build.py --trace, read
// by bench.py --phase-trace): per wave of the scalar-order XKV kernel, the
// cycles spent in each phase of the chunk loop, summed over its chunks. A wait is measured
// by a timestamp taken after an empty asm that reads the loaded register.
#if defined(KVEXP_PHASE_TRACE)
constexpr int kTracePhases = 12;
constexpr int kTraceWaves = 8192, kTraceWords = kTracePhases + 3; // start, end, the phases, CU id | head << 16 | split << 40
static __device__ unsigned long long g_phase_trace[kTraceWaves * kTraceWords];
#define KVEXP_TRACE_ON(X, O) ((X) && (O) == 0)
#else
#define KVEXP_TRACE_ON(X, O) false
#endif

constexpr int kChunk = 64;      // tokens per chunk (one per lane)
// Escape records a chunk can patch, loaded with its rows: four per lane per
// 16-byte load, one load at head_dim 64 and 128, eight at 256 (where escape-
// dense blocks would otherwise cut chunks short: c5's 4-bit K blocks hold
// about 1,300 escapes per 64 rows).
template <int D>
constexpr int kEscLoads = D == 256 ? 8 : 1;
template <int D>
constexpr int kEscWindow = 256 * kEscLoads<D>;
constexpr int kRawRows = 48;    // rows of a raw block per chunk: 64 lanes x 3D/2 bytes = 48 rows of 2D bytes
constexpr uint16_t kNegZeroBf16 = 0x8000u; // V of a token past the chunk's end: fma(0, -0, acc) == acc exactly
constexpr int kSlotQ = 8;       // partial-state slot: m[8], l[8], acc[8][head_dim]

// How a chunk's coded rows are loaded (see Rows): whole rows (lane = row) at
// head_dim 64, where a row's 64 sign/mantissa and 32 code bytes take six
// 16-byte loads per lane; 16-channel pieces at 128 and 256, where whole rows
// would put every load instruction on 64 different cache lines. Measured on
// c2 (head_dim 64), whole rows: 93.7 us per step against 97.7 for pieces; on
// c4 (head_dim 128), pieces: 2,726 against 3,323 for whole rows.
template <int D>
constexpr bool kWholeRows = D == 64;
// Whether K rows of a chunk without escapes may skip the tile (whole rows:
// lane = row = token in both the decode and the scores; in the AVX-512 BF16
// order only where the chunk needs no flush).
template <int D, int ORDER>
constexpr bool kDirectK = kWholeRows<D>;

// The kernel's sizes for head_dim D (64, 128 or 256).
template <int D>
struct Shape {
    static constexpr int kTileStride = 2 * D + 16;  // bytes per tile row: D BF16 + 16 (conflict-free 16-byte rows)
    static constexpr int kSlotFloats = kSlotQ * (D + 2);
    static constexpr int kPieces = D / 16;          // 16-channel pieces per row, and pieces per lane per chunk
    static constexpr int kPieceRows = kChunk / kPieces; // chunk rows between a lane's consecutive pieces
    static constexpr int kSmRegs = D / 16;          // whole rows: 16-byte registers of a row's sign/mantissa bytes
    static constexpr int kRowRegs = kSmRegs + D / 32; // + its 4-bit codes: what a coded row needs
    static constexpr int kHalves = D / 64;          // channels per lane in the fold (lane, lane + 64, ...)
    static constexpr int kWaves = D == 64 ? 4 : (D == 128 ? 2 : 1); // waves per workgroup (LDS: see WaveLds)
    // splits per merge batch (one per lane; their rows in flight together)
    static constexpr int kMergeBatch = D == 256 ? 32 : 64;
};

// Per-wave LDS. The tile holds the chunk's K rows (row t: the D BF16 of
// token t) and then its V rows, read by channel in the fold.
// eT / aT hold e and alpha by query row (row g: the chunk's 64 tokens), so a
// lane reads four tokens of its row in one access. At D = 64 and G <= 7 a
// wave takes 13,152 bytes and a workgroup of four waves with the shared table
// 52,864 bytes, which leaves room for three workgroups per CU (the limit lies
// between 53,760 and 54,016 bytes per workgroup). At D = 128 and G = 4 a wave
// takes 19,840 bytes; workgroups of two waves, four per CU.
constexpr int kRowPad = kChunk + 4; // floats per eT / aT row: 16 spare bytes keep the rows' reads conflict-free

template <int G, int D>
struct alignas(16) WaveLds {
    uint8_t tile[kChunk * Shape<D>::kTileStride];
    float eT[G][kRowPad]; // e of token t, row g (0 past the chunk's end)
    float aT[G][kRowPad]; // alpha of token t, row g (1 where no running maximum moves)
    uint32_t bp[kWholeRows<D> ? D / 2 : 1]; // whole rows: base pair words of the block being decoded
};

template <int G, int D>
struct alignas(16) WgLds {
    uint64_t exptab[32];
    WaveLds<G, D> w[Shape<D>::kWaves];
};

// Global-memory loads (address space 1, so they are issued as global_load_*
// and counted on the vector-memory counter only). Addresses need only 2-byte
// alignment: gfx950 under ROCm runs in unaligned-access mode.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4), aligned(2)));
typedef const __attribute__((address_space(1))) u32x4 g_u32x4;
typedef unsigned int u32x2 __attribute__((ext_vector_type(2), aligned(2)));
typedef const __attribute__((address_space(1))) u32x2 g_u32x2;
typedef const __attribute__((address_space(1))) uint16_t g_u16;
typedef const __attribute__((address_space(1))) uint32_t g_u32 __attribute__((aligned(2)));

// A copy of *p read through the constant address space (4): uniform loads
// from it are scalar loads. For descriptors written by earlier launches only
// (the scalar cache is coherent across launches). The host pass of this file
// only needs the declaration to compile.
template <class T>
__device__ __forceinline__ T load_scalar(const T *p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *(const __attribute__((address_space(4))) T *)(p);
#else
    return *p;
#endif
}

// Constant address space (4): uniform loads from it are scalar loads.
typedef float f8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(4))) f8 c_f8;
// An LDS float (address space 3), for pointers that pass through inline asm
// and must still be read with ds_read.
typedef const __attribute__((address_space(3))) float lds_f32;
typedef float f4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(3))) f4 lds_f4;

__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
    const u32x4 v = *(g_u32x4 *)(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8(const uint8_t *p) {
    const u32x2 v = *(g_u32x2 *)(p);
    return make_uint2(v.x, v.y);
}

// The lane index as an opaque value: the addresses derived from it are then
// recomputed where they are used (a few instructions) instead of being
// hoisted out of the chunk loop and held in registers across it.
__device__ __forceinline__ int lane_here() {
    int l = int(__lane_id());
    asm volatile("" : "+v"(l));
    return l;
}

// Position of one tensor inside its XKV container. The scalar fields are
// wave-uniform; erec holds the block's next escape records (component j of
// erec[i] at lane l: escape ecur + 256 i + 4 l + j, meaningful below
// n_escape; kEscLoads of them are loaded); basew holds base exponents of
// the block: whole rows, lane p < D / 2: base[2p], base[2p + 1]; pieces,
// bytes 4j .. 4j + 3 of channel column c (channels 16 c .. 16 c + 15, see
// Rows) at lane c + (D / 16) j, j < 4 (lanes past 4 D / 16 repeat them).
struct Cursor {
    const BlockDesc *d;  // descriptor of the current block (the next one follows it)
    const uint8_t *blk;  // current block's header
    const uint32_t *esc; // its escape records
    int t0, t1;          // its token range
    uint32_t meta;       // mode | n_tokens << 8 | n_escape << 16
    int ecur;            // first escape of the block not yet written into a tile
    int lrows;           // rows requested by the last load_rows (the raw piece layout depends on it)
    uint4 erec[8];
    uint32_t basew;
    __device__ int mode() const { return int(meta & 0xFFu); }
    __device__ int ntok() const { return int((meta >> 8) & 0xFFu); }
    __device__ int nesc() const { return int(meta >> 16); }
};

// Enters the block of descriptor d, whose first token is t0: one scalar load
// of the descriptor (checked against the container when the plan was built).
// Scalar state only; block_vectors loads the per-lane data.
__device__ __forceinline__ void enter_block(Cursor &c, const BlockDesc *d, int t0) {
    const u32x8 w = *(const __attribute__((address_space(4))) u32x8 *)(d);
    c.d = d;
    c.blk = reinterpret_cast<const uint8_t *>((uint64_t(w.s1) << 32) | w.s0);
    c.esc = reinterpret_cast<const uint32_t *>((uint64_t(w.s3) << 32) | w.s2);
    c.meta = w.s4;
    c.t0 = t0;
    c.t1 = t0 + c.ntok();
    c.ecur = 0;
}

// The block's base exponents (see Cursor: one 4-byte load) and its next
// kEscWindow escape records (four per lane per 16-byte load). The call is
// made on every chunk whether or not the block changed, and each load
// instruction is issued whatever the path (lane 0 always loads, from an
// always valid address: a records array ends with kEscPad spare records),
// so the number of loads in flight never depends on the path taken: the
// compiler's wait counts then stay exact, and a wait for the K rows leaves
// the V rows in flight. Lanes whose four records all lie at or past
// n_escape do not load (their bytes would be masked where used): a block
// holds about two dozen escapes on c2, so the window's load reads one or two
// cache lines instead of sixteen.
template <int D>
__device__ __forceinline__ void block_vectors(Cursor &c) {
    const int lane = lane_here();
    constexpr int NP = Shape<D>::kPieces;
    if constexpr (kWholeRows<D>) c.basew = *(g_u16 *)(c.blk + 8 + 2 * (lane & (D / 2 - 1)));
    else c.basew = *(g_u32 *)(c.blk + 8 + 16 * (lane % NP) + 4 * ((lane / NP) & 3));
    const int left = c.nesc() - c.ecur; // records of the block not yet written
#pragma unroll
    for (int i = 0; i < kEscLoads<D>; ++i) {
        const int first = 256 * i + 4 * lane;
        u32x4 r = {0u, 0u, 0u, 0u};
        if (first < left || lane == 0) r = *(g_u32x4 *)(c.esc + c.ecur + first);
        c.erec[i] = make_uint4(r.x, r.y, r.z, r.w);
    }
}

// Rows of the cursor's block from row r0 on that the next chunk may take so
// that its escapes all lie in the loaded window: when more than kEscWindow
// escapes remain, the rows before the one holding the window's last record (its
// position, read from lane 63). A row holds at most D <= 256 escapes, so the
// answer is at least 1 (a row of 256 escapes fills the window alone).
template <int D>
__device__ __forceinline__ int escape_rows(const Cursor &c, int r0) {
    if (c.nesc() - c.ecur <= kEscWindow<D>) return kChunk;
    const uint32_t last = __builtin_amdgcn_readlane(c.erec[kEscLoads<D> - 1].w, kWave - 1) & 0xFFFFu;
    return max(1, int(last / D) - r0);
}

// A chunk's rows in registers. Whole rows (head_dim 64): lane = row, r[0 ..
// D/16) its D sign/mantissa bytes, then its D/2 (4-bit), 3D/8 (3-bit: the
// second code register holds bytes 8 .. 23) or D/4 (2-bit, the register
// repeated) code bytes; a raw block (at most kRawRows rows) as 16-byte pieces
// (piece p: column p % (D / 8) of row p / (D / 8)), kRowRegs consecutive ones
// per lane from raw_start.
// Pieces (head_dim 128, 256): one piece per lane per register pair. Coded
// block: piece p of the chunk is channels 16 (p % (D / 16)) .. + 16 of its
// row p / (D / 16), and lane l holds pieces l + 64 k (k < D / 16): one
// channel column c = l % (D / 16) in rows kPieceRows k + l / (D / 16). s[k]
// holds the piece's 16 sign/mantissa bytes, c[k] the 8 bytes that end with
// its last code byte (4-bit: its 8 code bytes; 3-bit: 2 bytes before its 6;
// 2-bit: 4 bytes before its 4; so no load reaches past the block, and one
// that starts before its first code byte still lies in the block's
// sign/mantissa bytes). Consecutive lanes read consecutive bytes: each load
// covers a few whole cache lines instead of one line per lane. Raw block (at
// most kRawRows rows): s[k] holds bytes 1024 k + 16 l of the chunk's rows,
// c[k] bytes 64 D + 512 k + 8 l (rows 32 .. 47), clamped to the last piece of
// the rows loaded.
template <int D, bool W = kWholeRows<D>>
struct Rows {
    uint4 s[Shape<D>::kPieces];
    uint2 c[Shape<D>::kPieces];
};
template <int D>
struct Rows<D, true> {
    uint4 r[Shape<D>::kRowRegs];
};

// Whole rows: the first raw piece held by the lane, the last lanes' starts
// clamped so that every lane's pieces lie inside the rows (lanes past the end
// repeat the last kRowRegs).
template <int D>
__device__ __forceinline__ int raw_start(int rows) {
    constexpr int RR = Shape<D>::kRowRegs;
    const int np = max(1, min(rows, kRawRows)) * (D / 8); // >= RR
    return min(RR * lane_here(), np - RR);
}

// Whole rows: loads rows r0 .. r0 + rows of the cursor's block into R
// (lanes past the rows load the last row again). Every load is
// unconditional, at the block's (uniform) address plus one of two per-lane
// 32-bit offsets picked by uniform selects.
template <int D>
__device__ __forceinline__ void load_whole_rows(Cursor &c, int r0, int rows, Rows<D, true> &R) {
    constexpr int SM = Shape<D>::kSmRegs, RR = Shape<D>::kRowRegs;
    const int mode = c.mode();
    const bool raw = mode == 0;
    c.lrows = rows;
    // (rows <= 0 only past a plan's zero-token sentinel block: row r0 then)
    const int r = r0 + max(0, min(lane_here(), rows - 1));
    const int cbytes = mode * (D / 8); // code bytes per coded row
    const uint8_t *b = c.blk + 8;
    // sign/mantissa bytes of the row, then its codes; raw: the lane's pieces
    const uint32_t oa = raw ? uint32_t(r0 * (2 * D) + 16 * raw_start<D>(rows)) : uint32_t(D + r * D);
    const uint32_t ob = raw ? oa + 16 * SM : uint32_t(D + c.ntok() * D + r * cbytes);
#pragma unroll
    for (int i = 0; i < SM; ++i) R.r[i] = ld16(b + oa + 16 * i);
#pragma unroll
    for (int i = SM; i < RR; ++i) R.r[i] = ld16(b + ob + (raw ? 16 * (i - SM) : min(16 * (i - SM), cbytes - 16)));
}

// Pieces: loads rows r0 .. r0 + rows of the cursor's block into R. Both
// register streams (s and c) are runs of equal pieces: register k of
// lane l reads from x0 + step k + w l (bytes from the block's data), clamped
// to the stream's last piece e, which lanes whose piece lies past `rows`
// read again, so no load leaves the rows asked for. The stream parameters
// are picked once (coded or raw); per register the uniform part
// min(x0 + step k, e) goes to the load's scalar base and the lane's part is
// one v_min against e minus it (never negative, so the load takes a 32-bit
// vector offset). Every load is unconditional, so the registers need no
// merge before their use.
template <int D>
__device__ __forceinline__ void load_pieces(Cursor &c, int r0, int rows, Rows<D, false> &R) {
    constexpr int NP = Shape<D>::kPieces;
    const int mode = c.mode();
    const bool raw = mode == 0;
    c.lrows = rows;
    rows = max(rows, 1); // (rows <= 0 only past a plan's zero-token sentinel block: row r0 then)
    const int lane = lane_here();
    const uint8_t *b = c.blk + 8;
    // sign/mantissa stream: 16 bytes per lane, 1,024 per register
    int s0, se;
    // code stream: w bytes per lane (8 bytes loaded, ending with the piece's codes), cs per register
    int c0, ce, cw;
    if (!raw) {
        const int cbytes = mode * (D / 8); // code bytes per coded row
        s0 = D + r0 * D;
        se = s0 + rows * D - 16;
        cw = 2 * mode;
        c0 = D + c.ntok() * D + r0 * cbytes + cw - 8;
        ce = c0 + (rows * NP - 1) * cw;
    } else {
        const int rn = 2 * D * min(rows, kRawRows); // raw bytes loaded: rows [0, 32) in s, [32, 48) in c
        s0 = r0 * (2 * D);
        se = s0 + rn - 16;
        cw = 8;
        c0 = s0 + 64 * D;
        ce = s0 + rn - 8;
    }
    const int cs = 64 * cw;
    const uint32_t ls = uint32_t(16 * lane), lc = uint32_t(cw * lane);
#pragma unroll
    for (int k = 0; k < NP; ++k) {
        const int bs = min(s0 + 1024 * k, se), bc = min(c0 + cs * k, ce);
        R.s[k] = ld16(b + bs + min(ls, uint32_t(se - bs)));
        R.c[k] = ld8(b + bc + min(lc, uint32_t(ce - bc)));
    }
}

template <int D>
__device__ __forceinline__ void load_rows(Cursor &c, int r0, int rows, Rows<D> &R) {
    if constexpr (kWholeRows<D>) load_whole_rows<D>(c, r0, rows, R);
    else load_pieces<D>(c, r0, rows, R);
}

// A word that arrives with the last load of load_rows.
template <int D>
__device__ __forceinline__ uint32_t last_loaded(const Rows<D> &R) {
    if constexpr (kWholeRows<D>) return R.r[Shape<D>::kRowRegs - 1].w;
    else return R.c[Shape<D>::kPieces - 1].y;
}

__device__ __forceinline__ uint32_t comp(const uint4 &v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Whole rows: base pair words of the cursor's block into LDS, word p =
// base[2p] << 7 | base[2p+1] << 23 (lane p < D / 2 builds word p from the
// bytes loaded with the block).
template <int D>
__device__ __forceinline__ void base_pairs(const Cursor &c, uint32_t *bp) {
    const int lane = lane_id();
    if (lane < D / 2) bp[lane] = ((c.basew & 0xFFu) << 7) | ((c.basew >> 8) << 23);
}

// The sign/mantissa bit mask of a BF16 pair, 0x807F807F, in a vector
// register (made once per chunk): as the mask operand of v_bitop3_b32 from a
// vector register it keeps that instruction at the fast issue rate, where a
// scalar operand or v_bfi_b32 would take the slow one.
__device__ __forceinline__ uint32_t sm_mask_vgpr() {
    uint32_t m = 0x807F807Fu;
    asm volatile("" : "+v"(m));
    return m;
}

// One BF16 pair from two sign/mantissa bytes (positions lb, lb+1 of sw), two
// codes (byte p of lo and hi) and the channel pair's base word (bases at bits
// 14:7 and 30:23); smm is sm_mask_vgpr(). The sign and mantissa bits come from
// the spread bytes, the exponents from base + code (bitop3 0xE4: S2 ? S0 : S1).
__device__ __forceinline__ uint32_t pair4(uint32_t sw, int lb, uint32_t lo, uint32_t hi, int p, uint32_t bpw,
                                          uint32_t smm) {
    const uint32_t code16 = __builtin_amdgcn_perm(hi, lo, 0x0c000c00u | (uint32_t(4 + p) << 16) | uint32_t(p));
    const uint32_t t = (code16 << 7) + bpw; // exponent pair at bits 14:7 / 30:23
    const uint32_t hb = uint32_t(lb + 1);
    const uint32_t s = __builtin_amdgcn_perm(sw, sw, (hb << 24) | (hb << 16) | (uint32_t(lb) << 8) | uint32_t(lb));
    return __builtin_amdgcn_bitop3_b32(s, t, smm, 0xE4);
}

// Octet o (channels 8o .. 8o + 7 of the piece) as four BF16 pairs: the
// piece's sign/mantissa bytes sm, its codes split into lo (byte p: code 2p of
// the octet) and hi (byte p: code 2p + 1), and the column's base pair words.
__device__ __forceinline__ uint4 octet(const uint4 &sm, int o, uint32_t lo, uint32_t hi, const uint32_t (&bp)[8],
                                       uint32_t smm) {
    const uint32_t s0 = comp(sm, 2 * o), s1 = comp(sm, 2 * o + 1);
    uint4 r;
    r.x = pair4(s0, 0, lo, hi, 0, bp[4 * o], smm);
    r.y = pair4(s0, 2, lo, hi, 1, bp[4 * o + 1], smm);
    r.z = pair4(s1, 0, lo, hi, 2, bp[4 * o + 2], smm);
    r.w = pair4(s1, 2, lo, hi, 3, bp[4 * o + 3], smm);
    return r;
}

// Whole rows: octet dg (channels 8dg .. 8dg + 7) of a coded row, four BF16
// pairs from the row's sign/mantissa bytes in R.r[0 .. D/16), its codes split
// into lo (byte p: code 2p) and hi (byte p: code 2p + 1), and the channel
// pairs' base words in LDS.
template <int D>
__device__ __forceinline__ uint4 octet_row(const Rows<D, true> &R, int dg, uint32_t lo, uint32_t hi,
                                           const uint32_t *bp, uint32_t smm) {
    const uint32_t s0 = comp(R.r[dg >> 1], (dg & 1) * 2);
    const uint32_t s1 = comp(R.r[dg >> 1], (dg & 1) * 2 + 1);
    const uint4 b4 = *reinterpret_cast<const uint4 *>(bp + 4 * dg);
    uint4 o;
    o.x = pair4(s0, 0, lo, hi, 0, b4.x, smm);
    o.y = pair4(s0, 2, lo, hi, 1, b4.y, smm);
    o.z = pair4(s1, 0, lo, hi, 2, b4.z, smm);
    o.w = pair4(s1, 2, lo, hi, 3, b4.w, smm);
    return o;
}

// Whole rows: dword i of a 3-bit coded row's code bytes as load_whole_rows
// placed them.
template <int D>
__device__ __forceinline__ uint32_t code_dword3(const Rows<D, true> &R, int i) {
    constexpr int SM = Shape<D>::kSmRegs;
    if (D == 64 && i >= 4) return comp(R.r[SM + 1], i - 2); // bytes 16..23 are dwords 2, 3 of the register at byte 8
    return comp(R.r[SM + (i >> 2)], i & 3);
}

// -0 in every channel of the lane's tile row (a token past the chunk's end).
template <int D>
__device__ __forceinline__ void fill_negzero(uint8_t *row) {
    const uint32_t z = uint32_t(kNegZeroBf16) * 0x10001u;
#pragma unroll
    for (int i = 0; i < D / 8; ++i) reinterpret_cast<uint4 *>(row)[i] = make_uint4(z, z, z, z);
}

// Whole rows: the codes of octet dg (channels 8dg .. 8dg + 7) of the lane's
// coded row for a block of mode MODE (4, 3 or 2 bits per code), as lo (byte
// p: code 2p) and hi (byte p: code 2p + 1).
template <int D, int MODE>
__device__ __forceinline__ void octet_codes(const Rows<D, true> &R, int dg, uint32_t &lo, uint32_t &hi) {
    constexpr int SM = Shape<D>::kSmRegs;
    if constexpr (MODE == 4) {
        const uint32_t cw = comp(R.r[SM + (dg >> 2)], dg & 3);
        lo = cw & 0x0F0F0F0Fu;
        hi = (cw >> 4) & 0x0F0F0F0Fu;
    } else if constexpr (MODE == 2) {
        // 16 two-bit codes per dword; octet dg uses 16 bits
        const uint32_t cw = comp(R.r[SM + (dg >> 3)], (dg >> 1) & 3) >> (16 * (dg & 1));
        lo = (cw & 3u) | (((cw >> 4) & 3u) << 8) | (((cw >> 8) & 3u) << 16) | (((cw >> 12) & 3u) << 24);
        hi = ((cw >> 2) & 3u) | (((cw >> 6) & 3u) << 8) | (((cw >> 10) & 3u) << 16) | (((cw >> 14) & 3u) << 24);
    } else {
        // 3-bit codes: octet dg's 24 bits are bytes [3dg, 3dg + 3) of the
        // row's codes; groups of two codes (6 bits) are spread to bytes first
        const int q = (3 * dg) >> 2, b = (3 * dg) & 3;
        const uint32_t w = __builtin_amdgcn_alignbyte(code_dword3<D>(R, q + (b > 1 ? 1 : 0)), code_dword3<D>(R, q),
                                                      uint32_t(b));
        const uint32_t x = (w & 0x3Fu) | ((w << 2) & 0x3F00u) | ((w << 4) & 0x3F0000u) | ((w << 6) & 0x3F000000u);
        lo = x & 0x07070707u;
        hi = (x >> 3) & 0x07070707u;
    }
}

// Whole rows: octet dg of the lane's coded row as four BF16 pairs (mode
// MODE), with the channel pairs' base words in bp (base_pairs).
template <int D, int MODE>
__device__ __forceinline__ uint4 coded_octet(const Rows<D, true> &R, int dg, const uint32_t *bp, uint32_t smm) {
    uint32_t lo, hi;
    octet_codes<D, MODE>(R, dg, lo, hi);
    return octet_row<D>(R, dg, lo, hi, bp, smm);
}

// Whole rows: pair P (channels 8dg + 2P, 8dg + 2P + 1) of octet dg, as
// octet_row builds it, from the octet's codes and the pair's base word.
template <int D>
__device__ __forceinline__ uint32_t coded_pair(const Rows<D, true> &R, int dg, int P, uint32_t lo, uint32_t hi,
                                               uint32_t bpw, uint32_t smm) {
    const uint32_t sw = comp(R.r[dg >> 1], (dg & 1) * 2 + (P >> 1));
    return pair4(sw, 2 * (P & 1), lo, hi, P, bpw, smm);
}

// Whole rows: decodes the rows held in R into the tile, a coded row into the
// lane's tile row with the base pair words in bp (base_pairs), raw pieces to
// their rows. One uniform branch on the mode, then a straight-line body per
// mode; lanes >= rows then store -0 in every channel of their row.
template <int D>
__device__ __forceinline__ void decode_whole_rows(const Cursor &c, const Rows<D, true> &R, const uint32_t *bp,
                                                  uint8_t *tile, int rows, uint32_t smm) {
    constexpr int RR = Shape<D>::kRowRegs;
    const int lane = lane_here();
    uint4 *dst = reinterpret_cast<uint4 *>(tile + lane * Shape<D>::kTileStride);
    const int mode = c.mode();
    if (mode == 4) {
#pragma unroll
        for (int dg = 0; dg < D / 8; ++dg) dst[dg] = coded_octet<D, 4>(R, dg, bp, smm);
    } else if (mode == 2) {
#pragma unroll
        for (int dg = 0; dg < D / 8; ++dg) dst[dg] = coded_octet<D, 2>(R, dg, bp, smm);
    } else if (mode == 3) {
#pragma unroll
        for (int dg = 0; dg < D / 8; ++dg) dst[dg] = coded_octet<D, 3>(R, dg, bp, smm);
    } else {
        // raw rows: register i holds piece raw_start + i of the rows loaded
        // (c.lrows >= rows); pieces of rows >= rows are overwritten below
        const int p0 = raw_start<D>(c.lrows);
#pragma unroll
        for (int i = 0; i < RR; ++i) {
            const int p = p0 + i;
            *reinterpret_cast<uint4 *>(tile + (p / (D / 8)) * Shape<D>::kTileStride + (p % (D / 8)) * 16) = R.r[i];
        }
    }
    if (rows < kChunk && lane >= rows) fill_negzero<D>(tile + lane * Shape<D>::kTileStride);
}

// Pieces: decodes the rows held in R (cursor's block mode; layout: Rows) into the
// tile: each coded piece to its 32 bytes of its tile row (a coded element is
// (sm & 0x80) << 8 | (base + code) << 7 | (sm & 0x7F)), raw pieces to their
// rows. One uniform branch on the mode, then a straight-line body per mode.
// Lanes >= rows (past the chunk's end) then store -0 in every channel of
// their row (wanted for V; harmless for K).
template <int D>
__device__ __forceinline__ void decode_pieces(const Cursor &c, Rows<D, false> &R, uint8_t *tile, int rows,
                                              uint32_t smm) {
    constexpr int NP = Shape<D>::kPieces, RS = Shape<D>::kPieceRows, TS = Shape<D>::kTileStride;
    // At head_dim 256 the coded pieces go in two passes of eight, the last
    // eight registers moved into the first eight in between: one copy of each
    // mode's body instead of two keeps the chunk loop within the instruction
    // cache (64 KiB; the kernel's code, 149 KiB fully unrolled, is now 63 KiB
    // at eight query rows). Four passes of four cost more in register moves
    // than they save (c5: 1,992 against 1,936 us per step).
    constexpr int NPASS = D == 256 ? 2 : 1, PP = NP / NPASS;
    const int mode = c.mode();
    const int lane = lane_here();
    if (mode != 0) {
        // the column's base pair words: pair j (channels 2j, 2j + 1 of the
        // column) at bits 14:7 and 30:23, from the four lanes that hold its
        // base exponents
        uint32_t bp[8];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t w = uint32_t(__builtin_amdgcn_ds_bpermute(4 * (lane % NP + NP * m), int(c.basew)));
            bp[2 * m] = __builtin_amdgcn_perm(w, w, 0x0c010c00u) << 7;
            bp[2 * m + 1] = __builtin_amdgcn_perm(w, w, 0x0c030c02u) << 7;
        }
        uint8_t *dst = tile + (lane / NP) * TS + 32 * (lane % NP); // piece 0's place; piece k is RS k rows below
#pragma unroll 1
        for (int pass = 0; pass < NPASS; ++pass) {
            if (mode == 4) {
#pragma unroll
                for (int k = 0; k < PP; ++k) {
                    const uint32_t c0 = R.c[k].x, c1 = R.c[k].y;
                    uint4 *o = reinterpret_cast<uint4 *>(dst + RS * k * TS);
                    o[0] = octet(R.s[k], 0, c0 & 0x0F0F0F0Fu, (c0 >> 4) & 0x0F0F0F0Fu, bp, smm);
                    o[1] = octet(R.s[k], 1, c1 & 0x0F0F0F0Fu, (c1 >> 4) & 0x0F0F0F0Fu, bp, smm);
                }
            } else if (mode == 2) {
#pragma unroll
                for (int k = 0; k < PP; ++k) {
                    uint4 *o = reinterpret_cast<uint4 *>(dst + RS * k * TS);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        // the octet's 16 bits: byte p of lo / hi holds codes 2p / 2p + 1
                        const uint32_t cw = R.c[k].y >> (16 * h);
                        const uint32_t lo = (cw & 3u) | (((cw >> 4) & 3u) << 8) | (((cw >> 8) & 3u) << 16) |
                                            (((cw >> 12) & 3u) << 24);
                        const uint32_t hi = ((cw >> 2) & 3u) | (((cw >> 6) & 3u) << 8) | (((cw >> 10) & 3u) << 16) |
                                            (((cw >> 14) & 3u) << 24);
                        o[h] = octet(R.s[k], h, lo, hi, bp, smm);
                    }
                }
            } else {
                // 3-bit codes: octet h's 24 bits are bytes 2 + 3h .. 4 + 3h of
                // c[k]; groups of two codes (6 bits) are spread to bytes first
#pragma unroll
                for (int k = 0; k < PP; ++k) {
                    uint4 *o = reinterpret_cast<uint4 *>(dst + RS * k * TS);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t w =
                            h == 0 ? __builtin_amdgcn_alignbyte(R.c[k].y, R.c[k].x, 2u) : R.c[k].y >> 8;
                        const uint32_t x =
                            (w & 0x3Fu) | ((w << 2) & 0x3F00u) | ((w << 4) & 0x3F0000u) | ((w << 6) & 0x3F000000u);
                        o[h] = octet(R.s[k], h, x & 0x07070707u, (x >> 3) & 0x07070707u, bp, smm);
                    }
                }
            }
            if constexpr (NPASS > 1) {
#pragma unroll
                for (int k = 0; k < NP - PP; ++k) {
                    R.s[k] = R.s[k + PP];
                    R.c[k] = R.c[k + PP];
                }
                dst += PP * RS * TS;
            }
        }
    } else {
        // raw rows: the pieces loaded (c.lrows >= rows; clamped pieces repeat
        // the last one), to their rows; pieces of rows >= rows are overwritten below
        const int rn = 2 * D * max(1, min(c.lrows, kRawRows));
#pragma unroll
        for (int k = 0; k < NP; ++k) {
            const int os = min(1024 * k + 16 * lane, rn - 16), oc = min(64 * D + 512 * k + 8 * lane, rn - 8);
            *reinterpret_cast<uint4 *>(tile + (os / (2 * D)) * TS + os % (2 * D)) = R.s[k];
            *reinterpret_cast<uint2 *>(tile + (oc / (2 * D)) * TS + oc % (2 * D)) = R.c[k];
        }
    }
    if (rows < kChunk && lane >= rows) fill_negzero<D>(tile + lane * TS);
}

// The chunk's rows into the tile in the layout of head_dim D; bp: the base
// pair words that base_pairs wrote (whole rows only).
template <int D>
__device__ __forceinline__ void decode_rows(const Cursor &c, Rows<D> &R, const uint32_t *bp, uint8_t *tile,
                                            int rows, uint32_t smm) {
    if constexpr (kWholeRows<D>) decode_whole_rows<D>(c, R, bp, tile, rows, smm);
    else decode_pieces<D>(c, R, tile, rows, smm);
}

// ---- AVX-512 BF16 order ------------------------------------------------------
// VDPBF16PS (attention_avx512.cpp:21-30) reads denormal inputs as zero and
// flushes denormal results. The matrix-core products keep denormals, so the
// fast score path runs only on chunks where no flush can happen: every
// product k * q of nonzero BF16 values (8-bit significands) is an integer
// multiple of 2^(e_k + e_q - 14) (unbiased exponents), every partial sum of
// such products rounded to FP32 stays a multiple of the smallest of these
// powers, and a nonzero multiple of 2^-126 is a normal number. So with
// biased exponents E_k + E_q >= 142 for every nonzero K element and query
// element of the head (denormal queries read as zero beforehand), no input,
// chain value or sum is denormal, and the flushes are the identity. A chunk
// with a smaller K exponent (or a raw block, which is not checked element by
// element) takes the vector path that applies the flushes.

// Whether BF16 x is nonzero with exponent field below T, for
// low = (T << 7) - 1 (T >= 1): (x & 0x7FFF) - 1 wraps to 2^32 - 1 for a zero.
__device__ __forceinline__ bool low_bf16(uint32_t x, uint32_t low) { return (x & 0x7FFFu) - 1u < low; }

// Denormal to signed zero (VDPBF16PS's DAZ on inputs and FTZ on results).
__device__ __forceinline__ float flush_tiny(float x) {
    return fabsf(x) < 1.17549435e-38f ? copysignf(0.0f, x) : x;
}

// Writes the escape words of rows [r0, r0 + n) of the cursor's block over
// their elements in the tile and advances the cursor's escape index past
// them. Positions ascend within a block and every escape before ecur lies in
// an earlier chunk, so the chunk's escapes are the next ones from ecur whose
// positions are below (r0 + n) * D, all inside the window of records loaded
// with the chunk's rows (the chunk's length was cut to escape_rows). No
// loads here. With CHK, returns whether any of the words written is a
// nonzero value whose exponent field lies below the threshold that `low`
// encodes (see low_bf16).
template <int D, bool CHK = false>
__device__ __forceinline__ bool patch_escapes(Cursor &c, int r0, int n, uint8_t *tile, uint32_t low = 0) {
    constexpr int TS = Shape<D>::kTileStride;
    const int nesc = c.nesc();
    if (c.ecur >= nesc) return false;
    const int lane = lane_id();
    const uint32_t hi = uint32_t((r0 + n) * D);
    bool bad = false;
    int got = 0;
#pragma unroll
    for (int ij = 0; ij < 4 * kEscLoads<D>; ++ij) {
        const int i = ij >> 2, j = ij & 3;
        if (kEscLoads<D> > 1 && j == 0 && c.ecur + 256 * i >= nesc) break; // the block's records end before load i
        const uint32_t rj = comp(c.erec[i], j);
        const uint32_t pos = rj & 0xFFFFu, word = rj >> 16;
        const bool mine = c.ecur + 256 * i + 4 * lane + j < nesc && pos < hi;
        if (mine) {
            const uint32_t row = pos / D - uint32_t(r0), col = pos % D;
            *reinterpret_cast<uint16_t *>(tile + row * TS + col * 2) = uint16_t(word);
        }
        if (CHK) bad |= __ballot(mine && low_bf16(word, low)) != 0;
        got += __popcll(__ballot(mine));
    }
    c.ecur += got;
    return bad;
}

// Phase boundary inside one wave. The LDS performs one wave's operations in
// issue order, so a lane reads what other lanes of its wave wrote before
// without any wait; this only keeps the compiler from moving LDS accesses
// across the boundary.
__device__ __forceinline__ void wave_sync() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_wave_barrier();
}

// max(a, b) as one v_max_f32 (IEEE maxNum: a NaN operand gives the other).
// The inputs are arithmetic results, DPP maxima of them or -inf, never
// signalling NaNs, so fmaxf's quieting of each operand is not needed.
__device__ __forceinline__ float max_f32(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// a in the lanes whose bit of m is set, b in the others: v_cndmask_b32 with
// the lane mask in a scalar register pair. The compiler's own selects take
// one condition in VCC, and that form (VOP2, reading VCC) issues at about a
// quarter of the rate of this one on gfx950.
__device__ __forceinline__ float lane_select(uint64_t m, float a, float b) {
    float r;
    asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(b), "v"(a), "s"(m));
    return r;
}
// lane_select(m, a, 0) and lane_select(m, a, 1), the constant inline
__device__ __forceinline__ float lane_select_or0(uint64_t m, float a) {
    float r;
    asm("v_cndmask_b32_e64 %0, 0, %1, %2" : "=v"(r) : "v"(a), "s"(m));
    return r;
}
__device__ __forceinline__ float lane_select_or1(uint64_t m, float a) {
    float r;
    asm("v_cndmask_b32_e64 %0, 1.0, %1, %2" : "=v"(r) : "v"(a), "s"(m));
    return r;
}

__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Rank-1 update on the matrix cores: v_mfma_f32_4x4x1_16b_f32 with A taken
// from block ABID for all 16 blocks (CBSZ 4), so that
//   D[r] at lane l = A[lane 4 * ABID + r] * B[lane l] + C[r] at lane l.
// Each element is one IEEE fused multiply-add with round-to-nearest-even and
// denormals kept, the same bits as fmaf; the query rows (r) go in A and the
// tokens or channels (l) in B, so one instruction performs four query rows'
// fmaf of one channel for 64 tokens (scores), or of one token for 64
// channels (the V fold).
template <int ABID>
__device__ __forceinline__ f4 mfma_rank1(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, ABID, 0);
}

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Query rows in 4-row groups (rg): query row g is register g % 4 of group g / 4.
template <int G>
constexpr int kGroups = (G + 3) / 4;

// Scores of the lane's K row (lane = token) for G query rows in the
// scalar/AVX2 order of attention_scalar.cpp:23-29: chain j (j = 0..7) takes
// channels j, j + 8, ..., j + D - 8 in order, lane[j] = fmaf(q, k, lane[j]),
// then hsum8's ((l0 + l4) + (l1 + l5)) + ((l2 + l6) + (l3 + l7)). Channel d
// is one rank-1 product per row group into chain d % 8. qa[rg][d / 16] holds
// q[4 rg + r][d] at lane 4 (d % 16) + r. octet(dg) gives channels 8dg ..
// 8dg + 7 of the row as four BF16 pairs (from the tile, or decoded from the
// coded row in registers).
template <int G, int D, class Octet>
__device__ __forceinline__ void scores_of(Octet &&octet, const float (&qa)[kGroups<G>][D / 16], float (&s)[G]) {
    constexpr int NG = kGroups<G>;
    f4 ch[NG][8];
#pragma unroll
    for (int rg = 0; rg < NG; ++rg)
#pragma unroll
        for (int j = 0; j < 8; ++j) ch[rg][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    static_for<0, D / 8>([&](auto DG) {
        const uint4 kb = octet(int(decltype(DG)::value));
        const float k[8] = {lo_f32(kb.x), hi_f32(kb.x), lo_f32(kb.y), hi_f32(kb.y),
                            lo_f32(kb.z), hi_f32(kb.z), lo_f32(kb.w), hi_f32(kb.w)};
        static_for<0, 8>([&](auto J) {
            constexpr int d = 8 * decltype(DG)::value + decltype(J)::value;
#pragma unroll
            for (int rg = 0; rg < NG; ++rg) ch[rg][J] = mfma_rank1<d % 16>(qa[rg][d / 16], k[J], ch[rg][J]);
        });
        // the octet's eight widenings, then its products in one run: a
        // product that reads a register the vector ALU has just written
        // waits, and single products between vector instructions stall the
        // SIMD more than one run of them
        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 8 * NG, 0);
    });
#pragma unroll
    for (int rg = 0; rg < NG; ++rg) {
        const f4 a = (ch[rg][0] + ch[rg][4]) + (ch[rg][1] + ch[rg][5]);
        const f4 b = (ch[rg][2] + ch[rg][6]) + (ch[rg][3] + ch[rg][7]);
        const f4 t = a + b;
        if (4 * rg + 0 < G) s[(4 * rg + 0) % G] = t.x;
        if (4 * rg + 1 < G) s[(4 * rg + 1) % G] = t.y;
        if (4 * rg + 2 < G) s[(4 * rg + 2) % G] = t.z;
        if (4 * rg + 3 < G) s[(4 * rg + 3) % G] = t.w;
    }
}

// Scores of the lane's tile row (scores_of).
template <int G, int D>
__device__ __forceinline__ void scores(const uint8_t *row, const float (&qa)[kGroups<G>][D / 16], float (&s)[G]) {
    scores_of<G, D>([&](int dg) { return *reinterpret_cast<const uint4 *>(row + 16 * dg); }, qa, s);
}

// Scores (scores_of's order) of the lane's coded row held in R (whole rows,
// a block of mode MODE without escapes in the chunk), decoded pair by pair
// into the products instead of through the tile. Two passes over the row's
// octets, each over four of the eight chains: chains 0, 1, 4, 5 (pairs 0
// and 2 of every octet), then 2, 3, 6, 7 (pairs 1 and 3); every chain still
// takes its channels in order, and hsum8's tree splits into the two passes'
// sums (l0 + l4) + (l1 + l5) and (l2 + l6) + (l3 + l7). Half the chains are
// live at a time, which leaves room for the coded row.
template <int G, int D, int MODE>
__device__ __forceinline__ void scores_coded(const Rows<D, true> &R, const uint32_t *bp, uint32_t smm,
                                             const float (&qa)[kGroups<G>][D / 16], float (&s)[G]) {
    constexpr int NG = kGroups<G>;
    f4 half[2][NG];
    static_for<0, 2>([&](auto H) {
        constexpr int h = decltype(H)::value;
        // ch[rg][c]: chains 2h, 2h + 1, 4 + 2h, 5 + 2h
        f4 ch[NG][4];
#pragma unroll
        for (int rg = 0; rg < NG; ++rg)
#pragma unroll
            for (int c = 0; c < 4; ++c) ch[rg][c] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        static_for<0, D / 8>([&](auto DG) {
            constexpr int dg = decltype(DG)::value;
            uint32_t lo, hi;
            octet_codes<D, MODE>(R, dg, lo, hi);
            const uint32_t p0 = coded_pair<D>(R, dg, h, lo, hi, bp[4 * dg + h], smm);
            const uint32_t p1 = coded_pair<D>(R, dg, 2 + h, lo, hi, bp[4 * dg + 2 + h], smm);
            const float k[4] = {lo_f32(p0), hi_f32(p0), lo_f32(p1), hi_f32(p1)};
            static_for<0, 4>([&](auto C) {
                constexpr int c = decltype(C)::value;
                constexpr int d = 8 * dg + (c < 2 ? 2 * h + c : 4 + 2 * h + (c - 2));
#pragma unroll
                for (int rg = 0; rg < NG; ++rg) ch[rg][c] = mfma_rank1<d % 16>(qa[rg][d / 16], k[c], ch[rg][c]);
            });
            // the octet's decode and widenings, then its products: the
            // scheduler would otherwise decode octets ahead and hold more
            // registers than three waves per SIMD have (G 5 to 7 spilled)
            __builtin_amdgcn_sched_group_barrier(0x002, 14, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4 * NG, 0);
        });
#pragma unroll
        for (int rg = 0; rg < NG; ++rg) half[h][rg] = (ch[rg][0] + ch[rg][2]) + (ch[rg][1] + ch[rg][3]);
    });
#pragma unroll
    for (int rg = 0; rg < NG; ++rg) {
        const f4 t = half[0][rg] + half[1][rg];
        if (4 * rg + 0 < G) s[(4 * rg + 0) % G] = t.x;
        if (4 * rg + 1 < G) s[(4 * rg + 1) % G] = t.y;
        if (4 * rg + 2 < G) s[(4 * rg + 2) % G] = t.z;
        if (4 * rg + 3 < G) s[(4 * rg + 3) % G] = t.w;
    }
}

// Whether rows [r0, r0 + n) of the cursor's block hold an escape: the
// block's next escape not yet written (record ecur, the first of lane 0's
// window) lies before their end.
template <int D>
__device__ __forceinline__ bool rows_have_escapes(const Cursor &c, int r0, int n) {
    if (c.ecur >= c.nesc()) return false;
    const uint32_t pos = __builtin_amdgcn_readfirstlane(c.erec[0].x) & 0xFFFFu;
    return pos < uint32_t((r0 + n) * D);
}

// Scores in the AVX-512 BF16 order (attention_avx512.cpp:21-30,116-124) for a
// chunk where no flush can happen (see low_bf16): 16 chains; per 32-channel
// step c, chain j takes k[c + 2j + 1] * q[c + 2j + 1] and then
// k[c + 2j] * q[c + 2j] (VDPBF16PS's order, one rounding each); then the
// pairwise tree over the 16 chains, ((a0 + a1) + (a2 + a3)) with
// a_i = (t_4i + t_4i+1) + (t_4i+2 + t_4i+3). The chains run in quads
// (chains 4Q .. 4Q + 3 read octets Q, Q + 4, ...), R quads at a time: two
// for one row group (eight independent products between dependent ones),
// one for two row groups (the same, and fewer registers live); each run is
// reduced to its a_i before the next starts. octet(dg) gives channels 8dg ..
// 8dg + 7 of the lane's K row as four BF16 pairs (from the tile, or decoded
// from the coded row in registers); each octet is taken once.
template <int G, int D, class Octet>
__device__ __forceinline__ void scores_dp_of(Octet &&octet, const float (&qa)[kGroups<G>][D / 16], float (&s)[G]) {
    constexpr int NG = kGroups<G>;
    // One quad of chains at a time for every row group: at most 4 NG chains
    // live beside the partial sums.
    f4 a01[NG], a2[NG];
    static_for<0, 4>([&](auto RUN) {
        constexpr int Q0 = decltype(RUN)::value;
        __builtin_amdgcn_sched_barrier(0);
        f4 ch[NG][4];
#pragma unroll
        for (int rg = 0; rg < NG; ++rg)
#pragma unroll
            for (int j = 0; j < 4; ++j) ch[rg][j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        static_for<0, D / 32>([&](auto S) {
            constexpr int DG0 = 4 * decltype(S)::value + Q0; // octet of this step
            const uint4 kb = octet(DG0);
            const uint32_t w[4] = {kb.x, kb.y, kb.z, kb.w};
            static_for<0, 4>([&](auto J) { // odd channel of pair J first
                constexpr int d = 8 * DG0 + 2 * decltype(J)::value + 1;
                const float k = hi_f32(w[J]);
#pragma unroll
                for (int rg = 0; rg < NG; ++rg) ch[rg][J] = mfma_rank1<d % 16>(qa[rg][d / 16], k, ch[rg][J]);
            });
            static_for<0, 4>([&](auto J) {
                constexpr int d = 8 * DG0 + 2 * decltype(J)::value;
                const float k = lo_f32(w[J]);
#pragma unroll
                for (int rg = 0; rg < NG; ++rg) ch[rg][J] = mfma_rank1<d % 16>(qa[rg][d / 16], k, ch[rg][J]);
            });
        });
#pragma unroll
        for (int rg = 0; rg < NG; ++rg) {
            const f4 a = (ch[rg][0] + ch[rg][1]) + (ch[rg][2] + ch[rg][3]); // a_Q0
            // (the empty asm keeps each quad's sum here: sunk to the last
            // quad, every quad's chains would stay live until then)
            if constexpr (Q0 == 0) {
                a01[rg] = a;
                asm volatile("" : "+v"(a01[rg]));
            } else if constexpr (Q0 == 1) {
                a01[rg] = a01[rg] + a;
                asm volatile("" : "+v"(a01[rg]));
            } else if constexpr (Q0 == 2) {
                a2[rg] = a;
                asm volatile("" : "+v"(a2[rg]));
            } else {
                const f4 t = a01[rg] + (a2[rg] + a);
                if (4 * rg + 0 < G) s[(4 * rg + 0) % G] = t.x;
                if (4 * rg + 1 < G) s[(4 * rg + 1) % G] = t.y;
                if (4 * rg + 2 < G) s[(4 * rg + 2) % G] = t.z;
                if (4 * rg + 3 < G) s[(4 * rg + 3) % G] = t.w;
            }
        }
    });
}

// Scores of the lane's tile row in the AVX-512 BF16 order (scores_dp_of).
template <int G, int D>
__device__ __forceinline__ void scores_dp(const uint8_t *row, const float (&qa)[kGroups<G>][D / 16], float (&s)[G]) {
    scores_dp_of<G, D>([&](int dg) { return *reinterpret_cast<const uint4 *>(row + 16 * dg); }, qa, s);
}

// The same order on the vector ALU with every flush applied, for chunks the
// fast path cannot take: q from the head's BF16 rows in global memory, one
// query row and one quad of chains at a time (few registers live; the chains
// are independent, and each keeps its order), the score staged in `st`
// (row g at st + g * kRowPad).
template <int G, int D>
__device__ __forceinline__ void scores_dp_flush(const uint8_t *row, const uint16_t *q, float *st) {
    const int lane = lane_id();
#pragma unroll 1
    for (int g = 0; g < G; ++g) {
        float a01 = 0.0f, a2 = 0.0f, res = 0.0f;
#pragma unroll 1
        for (int Q = 0; Q < 4; ++Q) {
            float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < D; c += 32) {
                // pairs 4Q .. 4Q + 3 of the step: elements c + 8Q .. c + 8Q + 7
                const uint4 kb = *reinterpret_cast<const uint4 *>(row + 2 * (c + 8 * Q));
                const uint4 qb = *reinterpret_cast<const uint4 *>(q + size_t(g) * D + c + 8 * Q);
                const uint32_t kw[4] = {kb.x, kb.y, kb.z, kb.w}, qw[4] = {qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    t[p] = flush_tiny(fmaf(flush_tiny(hi_f32(kw[p])), flush_tiny(hi_f32(qw[p])), t[p]));
                    t[p] = flush_tiny(fmaf(flush_tiny(lo_f32(kw[p])), flush_tiny(lo_f32(qw[p])), t[p]));
                }
            }
            const float a = (t[0] + t[1]) + (t[2] + t[3]);
            if (Q == 0) a01 = a;
            else if (Q == 1) a01 = a01 + a;
            else if (Q == 2) a2 = a;
            else res = a01 + (a2 + a);
        }
        st[g * kRowPad + lane] = res;
    }
}

// Transposed read of four tokens' V for the fold (ds_read_b64_tr_b16): in
// each group of 16 lanes, lane 16 g + 4 k + i points at the 8 bytes of
// channels 16 g + 4 i .. + 3 of token T0 + k, and every lane c then receives
// V[T0 + k][c] as 16-bit element k of its result (a 4 x 4 transpose of
// 16-bit elements within the group). One LDS read per four tokens and
// channel half instead of four.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// The lane's byte offset in the tile for load_tr (token T0 = 0, channels 0 .. 63).
template <int D>
__device__ __forceinline__ uint32_t tr_lane_offset(int lane) {
    const int s = lane & 15;
    return uint32_t((s >> 2) * Shape<D>::kTileStride + 32 * (lane >> 4) + 8 * (s & 3));
}

__device__ __forceinline__ uint2 load_tr(const uint8_t *p) {
    const s16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(p));
    return __builtin_bit_cast(uint2, r);
}

// Token k (0 .. 3) of a load_tr quad as FP32.
template <int K>
__device__ __forceinline__ float quad_f32(const uint2 &q) {
    if constexpr (K == 0) return lo_f32(q.x);
    else if constexpr (K == 1) return hi_f32(q.x);
    else if constexpr (K == 2) return lo_f32(q.y);
    else return hi_f32(q.y);
}

// Operands of the fold in flight: V of the lane's channels (lane + 64 h) for
// the next quads of four tokens (quad Q in vq[Q % 3], requested two quads
// ahead) and e of four tokens (lane g < G: its row; the next quad's).
template <int H>
struct FoldIn {
    uint2 vq[3][H];
    f4 e4[2];
};

// Token T of the ordered fold (attention_scalar.cpp:33-40), lane = channel
// (channels lane + 64 h, h < D / 64). Tokens past the chunk's end carry
// e = 0, alpha = 1 and V = -0, which leave acc and l exactly as they are. A
// token that moves no running maximum (alpha == 1 for every row, exactly)
// takes acc = fma(e, v, acc); a token that moves one scales by alpha first:
// acc = fma(e, v, acc * alpha) (MOVE: the caller found a move among this
// token's group of 16 and tests the token's own bit; otherwise no test).
// acc[rg] register r is row 4 rg + r (acc[rg][h]: channel lane + 64 h); the
// fma of every row of a group is one rank-1 product per h whose A operand is
// ea[rg][T / 16] (e[4 rg + r][T] at lane 4 (T % 16) + r). Lane g < G carries
// l of row g: l = fma(l, alpha, e), which is l + e exactly where every
// alpha of the group is 1 (so only groups with a move read alpha, a quad at a
// time). V arrives by quads (load_tr) two quads ahead, e a quad ahead.
template <int G, int D, int T, bool MOVE>
__device__ __forceinline__ void fold_token(const WaveLds<G, D> &S, lds_f32 *eb, lds_f32 *ab, const uint8_t *trb,
                                           const uint32_t (&am)[2], const float (&ea)[kGroups<G>][4], FoldIn<D / 64> &in,
                                           f4 &a4, f4 (&acc)[kGroups<G>][D / 64], float &lvec) {
    constexpr int NG = kGroups<G>, H = D / 64, TS = Shape<D>::kTileStride, Q = T / 4;
    if constexpr (T % 4 == 0) {
        if constexpr (4 * (Q + 2) < kChunk) {
#pragma unroll
            for (int h = 0; h < H; ++h) in.vq[(Q + 2) % 3][h] = load_tr(trb + 4 * (Q + 2) * TS + 128 * h);
        }
        if constexpr (4 * (Q + 1) < kChunk) in.e4[(Q + 1) & 1] = *reinterpret_cast<lds_f4 *>(eb + 4 * (Q + 1));
        if constexpr (MOVE) a4 = *reinterpret_cast<lds_f4 *>(ab + 4 * Q);
    }
    float v[H];
#pragma unroll
    for (int h = 0; h < H; ++h) v[h] = quad_f32<T % 4>(in.vq[Q % 3][h]);
    const f4 e4 = in.e4[Q & 1];
    const float el = (T % 4 == 0) ? e4.x : (T % 4 == 1) ? e4.y : (T % 4 == 2) ? e4.z : e4.w;
    if constexpr (MOVE) {
        const uint32_t mw = am[T / 32];
        if ((mw & (1u << (T % 32))) != 0) {
            float av[G];
#pragma unroll
            for (int g = 0; g < G; ++g) av[g] = S.aT[g][T];
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int h = 0; h < H; ++h) acc[g / 4][h][g % 4] *= av[g];
        }
        const float al = (T % 4 == 0) ? a4.x : (T % 4 == 1) ? a4.y : (T % 4 == 2) ? a4.z : a4.w;
        lvec = fmaf(lvec, al, el);
    } else {
        lvec = lvec + el;
    }
    // keeps the l chain in token order (otherwise it may be sunk to the
    // end of the unrolled fold with every token's operands held live)
    asm volatile("" : "+v"(lvec));
#pragma unroll
    for (int rg = 0; rg < NG; ++rg)
#pragma unroll
        for (int h = 0; h < H; ++h) acc[rg][h] = mfma_rank1<T % 16>(ea[rg][T / 16], v[h], acc[rg][h]);
}

// The chunk's fold in groups of 16 tokens: one uniform test of the group's
// 16 bits of amask (tokens that move some running maximum) picks the straight
// path or the one that tests each token. On the straight path each run of
// four tokens issues its vector work (V widening, the l chain) and then its
// eight products: a product right after a vector instruction, or the reverse,
// stalls the SIMD, so few switches between the two pay.
// Group J (tokens 16 J .. 16 J + 15) of the fold with a runtime quad index,
// for a group where some token moves a running maximum at head_dim 256: there
// the unrolled form (32 accumulator scalings per token, through the matrix
// registers) would put the chunk loop far beyond the instruction cache. The
// same operations in the same order as fold_token, four tokens per pass:
// V of the quad by load_tr, e and alpha of the quad as 16-byte reads, every
// row's alpha of a token that moves a maximum read one token ahead, and the
// quad's A operands (e of the group's rows, lanes 16 q .. 16 q + 15 of
// ea[rg][J]) moved to lanes 0 .. 15 by one ds_bpermute, so that token u of
// the quad is block u. Then the next group's operands are requested as the
// unrolled fold would have left them.
template <int G, int D, int J>
__device__ __forceinline__ void fold_group_dyn(const WaveLds<G, D> &S, lds_f32 *eb, lds_f32 *ab,
                                               const uint8_t *trb, const uint32_t (&am)[2],
                                               const float (&ea)[kGroups<G>][4], FoldIn<D / 64> &in,
                                               f4 (&acc)[kGroups<G>][D / 64], float &lvec) {
    constexpr int NG = kGroups<G>, H = D / 64, TS = Shape<D>::kTileStride;
    const int lane = lane_id();
    const uint32_t mw = am[J / 2];
#pragma unroll 1
    for (int q = 0; q < 4; ++q) {
        const int T0 = 16 * J + 4 * q;
        uint2 vq[H];
#pragma unroll
        for (int h = 0; h < H; ++h) vq[h] = load_tr(trb + T0 * TS + 128 * h);
        const f4 e4 = *reinterpret_cast<lds_f4 *>(eb + T0);
        const f4 a4 = *reinterpret_cast<lds_f4 *>(ab + T0);
        float a[NG];
#pragma unroll
        for (int rg = 0; rg < NG; ++rg)
            a[rg] = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (lane + 16 * q), __float_as_int(ea[rg][J])));
        const uint32_t qb = (mw >> (T0 % 32)) & 15u; // the quad's tokens that move a maximum
        // every row's alpha of the token (read one token ahead)
        float an[G];
        if (qb & 1u) {
#pragma unroll
            for (int g = 0; g < G; ++g) an[g] = S.aT[g][T0];
        }
        static_for<0, 4>([&](auto U) {
            constexpr int u = decltype(U)::value;
            float av[G];
#pragma unroll
            for (int g = 0; g < G; ++g) av[g] = an[g];
            if constexpr (u < 3) {
                if ((qb >> (u + 1)) & 1u) {
#pragma unroll
                    for (int g = 0; g < G; ++g) an[g] = S.aT[g][T0 + u + 1];
                }
            }
            float v[H];
#pragma unroll
            for (int h = 0; h < H; ++h) v[h] = quad_f32<u>(vq[h]);
            if ((qb >> u) & 1u) {
#pragma unroll
                for (int g = 0; g < G; ++g)
#pragma unroll
                    for (int h = 0; h < H; ++h) acc[g / 4][h][g % 4] *= av[g];
            }
            lvec = fmaf(lvec, a4[u], e4[u]);
            asm volatile("" : "+v"(lvec));
#pragma unroll
            for (int rg = 0; rg < NG; ++rg)
#pragma unroll
                for (int h = 0; h < H; ++h) acc[rg][h] = mfma_rank1<u>(a[rg], v[h], acc[rg][h]);
        });
    }
    constexpr int Q0 = 4 * (J + 1); // the next group's first quad
    if constexpr (4 * Q0 < kChunk) {
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
            for (int h = 0; h < H; ++h) in.vq[(Q0 + k) % 3][h] = load_tr(trb + 4 * (Q0 + k) * TS + 128 * h);
        in.e4[Q0 & 1] = *reinterpret_cast<lds_f4 *>(eb + 4 * Q0);
    }
}

template <int G, int D, int T>
__device__ __forceinline__ void fold(const WaveLds<G, D> &S, lds_f32 *eb, lds_f32 *ab, const uint16_t *vb,
                                     const uint8_t *trb, const uint32_t (&am)[2], const float (&ea)[kGroups<G>][4],
                                     FoldIn<D / 64> &in, f4 (&acc)[kGroups<G>][D / 64], float &lvec) {
    constexpr int GS = 16, NG = kGroups<G>, H = D / 64;
    if constexpr (T < kChunk) {
        const uint32_t mw = am[T / 32];
        constexpr uint32_t gm = uint32_t(((1ull << GS) - 1ull) << (T % 32));
        f4 a4;
        if ((mw & gm) == 0) {
            static_for<0, GS>([&](auto K) {
                fold_token<G, D, T + decltype(K)::value, false>(S, eb, ab, trb, am, ea, in, a4, acc, lvec);
            });
            static_for<0, GS / 4>([&](auto) {
                __builtin_amdgcn_sched_group_barrier(0x002, 4 * (H + 1), 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 4 * NG * H, 0);
            });
        } else if constexpr (D == 256) {
            fold_group_dyn<G, D, T / GS>(S, eb, ab, trb, am, ea, in, acc, lvec);
        } else {
            static_for<0, GS>([&](auto K) {
                fold_token<G, D, T + decltype(K)::value, true>(S, eb, ab, trb, am, ea, in, a4, acc, lvec);
            });
        }
        fold<G, D, T + GS>(S, eb, ab, vb, trb, am, ea, in, acc, lvec);
    }
}


// Rows of the plain BF16 kernel: register j of lane l holds bytes
// [1024 j + 16 l, + 16) of the chunk's rows from token t (row
// (1024 j + 16 l) / 2D), so every load reads one contiguous run; rows past
// `avail` repeat the last one.
template <int D>
__device__ __forceinline__ void load_raw(const uint16_t *base, int t, int avail, uint4 (&R)[D / 8]) {
    const uint8_t *b = reinterpret_cast<const uint8_t *>(base + size_t(t) * D);
    const int lane = lane_here();
#pragma unroll
    for (int j = 0; j < D / 8; ++j) {
        const int off = 1024 * j + 16 * lane;
        R[j] = ld16(b + uint32_t(min(off / (2 * D), avail - 1) * (2 * D) + off % (2 * D)));
    }
}

template <int D>
__device__ __forceinline__ void store_raw(const uint4 (&R)[D / 8], uint8_t *tile) {
    const int lane = lane_here();
#pragma unroll
    for (int j = 0; j < D / 8; ++j) {
        const int off = 1024 * j + 16 * lane;
        *reinterpret_cast<uint4 *>(tile + (off / (2 * D)) * Shape<D>::kTileStride + off % (2 * D)) = R[j];
    }
}

template <bool XKV, int D> struct RegsOf { typedef Rows<D> T; };
template <int D> struct RegsOf<false, D> { typedef uint4 T[D / 8]; };

// At D = 64 the XKV instantiations with up to seven query rows are held to
// three waves per SIMD (168 VGPRs), and LDS allows three workgroups of four
// waves per CU; at D = 128 (the rows in flight take twice the registers) and
// at eight query rows two waves per SIMD; at D = 256 a wave's tile of 64
// full rows (33,792 bytes) leaves room for four one-wave workgroups per CU,
// one wave per SIMD, which may then take all 512 registers.
// ORDER 0: scalar/AVX2 score order; ORDER 1: AVX-512 BF16 order.
template <int G, int D, bool XKV, int ORDER>
constexpr int kWaveOcc = D == 256 ? 1 : (D == 64 && XKV && G < 8 ? 3 : 2);

template <int G, int D, bool XKV, int ORDER>
__global__ __launch_bounds__(Shape<D>::kWaves * 64) __attribute__((amdgpu_waves_per_eu(kWaveOcc<G, D, XKV, ORDER>)))
void attn_wave_kernel(const HeadDev *__restrict__ heads, const WorkItem *__restrict__ items, int n_items,
                      int wpg, const BlockDesc *__restrict__ desc,
                      const uint16_t *__restrict__ q_all, float *__restrict__ out_all, float *__restrict__ lse_all,
                      float *__restrict__ ws) {
    constexpr int TS = Shape<D>::kTileStride, H = D / 64;
    __shared__ WgLds<G, D> L;
    if (threadIdx.x < 64) kvexp_exp_table_to_lds(L.exptab);
    __syncthreads();

    const int lane = lane_id();
    const int w = int(threadIdx.x) >> 6;
    const int item = __builtin_amdgcn_readfirstlane(int(blockIdx.x) * wpg + w);
    if (item >= n_items) return;
    WaveLds<G, D> &S = L.w[w];
    const uint64_t *tab = L.exptab;
    const WorkItem wi = load_scalar(items + item);
    const HeadDev hd = load_scalar(heads + wi.head);
    // The head's query rows widened to FP32 as the A operands of the score
    // products: qa[rg][j] at lane 4b + r holds q[4 rg + r][16 j + b] (0 for
    // rows past G).
    constexpr int NG = kGroups<G>;
    float qa[NG][D / 16];
    {
        const int r = lane & 3, b = lane >> 2;
#pragma unroll
        for (int rg = 0; rg < NG; ++rg) {
            const int g = min(4 * rg + r, G - 1);
#pragma unroll
            for (int j = 0; j < D / 16; ++j) {
                float qv = __uint_as_float(uint32_t(q_all[(size_t(hd.q_row) + g) * D + 16 * j + b]) << 16);
                if constexpr (ORDER == 1) qv = flush_tiny(qv);
                qa[rg][j] = 4 * rg + r < G ? qv : 0.0f;
            }
        }
    }
    // ORDER 1: the K exponent bound of the fast score path, as low_bf16's
    // argument (T = 142 - the smallest exponent field of a nonzero query
    // element, at least 1), and T itself.
    uint32_t klow = 0, kmin = 0;
    if constexpr (ORDER == 1) {
        int qe = 255;
#pragma unroll
        for (int rg = 0; rg < NG; ++rg)
#pragma unroll
            for (int j = 0; j < D / 16; ++j) {
                const uint32_t b = __float_as_uint(qa[rg][j]);
                if ((b & 0x7FFFFFFFu) != 0) qe = min(qe, int((b >> 23) & 0xFFu));
            }
#pragma unroll
        for (int m = 1; m < kWave; m *= 2) qe = min(qe, __shfl_xor(qe, m));
        kmin = uint32_t(max(1, 142 - __builtin_amdgcn_readfirstlane(qe)));
        klow = (kmin << 7) - 1u;
    }

    f4 acc[NG][H];
#pragma unroll
    for (int rg = 0; rg < NG; ++rg)
#pragma unroll
        for (int h = 0; h < H; ++h) acc[rg][h] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float msc[G]; // running maximum of each query row (wave-uniform)
#pragma unroll
    for (int g = 0; g < G; ++g) msc[g] = -__builtin_inff();
    float lvec = 0.0f; // lane g < G holds l of query row g

    Cursor kc{}, vc{};
    typename RegsOf<XKV, D>::T RK, RV;
    int t = wi.tok_begin;
    if constexpr (XKV) {
        enter_block(kc, desc + wi.kdi, t);
        enter_block(vc, desc + wi.vdi, t);
        block_vectors<D>(kc);
        load_rows<D>(kc, 0, min(kChunk, min(kc.t1, wi.tok_end) - t), RK);
        block_vectors<D>(vc);
        load_rows<D>(vc, 0, min(kChunk, min(vc.t1, wi.tok_end) - t), RV);
    } else {
        // unconditional loads (rows past the split repeat its last row)
        load_raw<D>(hd.kraw, t, min(kChunk, wi.tok_end - t), RK);
        load_raw<D>(hd.vraw, t, min(kChunk, wi.tok_end - t), RV);
    }

    // Issue priority by progress: a SIMD issues from its oldest wave first, so
    // the first workgroup placed on a CU would race ahead and the last finish
    // alone at the end of the launch, with few loads in flight. Each wave
    // instead lowers its priority as it gets through its split (3 for the
    // first quarter of its tokens, then 2, 1, 0): the waves that are behind
    // win the issue slots and all of a CU's waves finish at about the same
    // time.
    constexpr bool TR = KVEXP_TRACE_ON(XKV, ORDER);
    unsigned long long ph[12] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const unsigned long long tw0 = TR ? __builtin_readcyclecounter() : 0ull;
    unsigned long long tprev = tw0;
    auto stamp = [&](int i) {
        if constexpr (TR) {
            const unsigned long long tn_ = __builtin_readcyclecounter();
            ph[i] += tn_ - tprev;
            tprev = tn_;
        }
    };
    auto after = [&](uint32_t x) {
        if constexpr (TR) asm volatile("" ::"v"(x));
    };
    (void)stamp;
    (void)after;

    __builtin_amdgcn_s_setprio(3);
    int prio = 3;
    const int span = wi.tok_end - wi.tok_begin;
    while (t < wi.tok_end) {
        const int ln = lane_here(); // this chunk's lane index (see lane_here)
        {
            const int want = 3 - min(3, ((t - wi.tok_begin) * 4) / max(span, 1));
            if (want != prio) {
                if (want == 2) __builtin_amdgcn_s_setprio(2);
                else if (want == 1) __builtin_amdgcn_s_setprio(1);
                else __builtin_amdgcn_s_setprio(0);
                prio = want;
            }
        }
        int n = min(kChunk, wi.tok_end - t);
        if constexpr (XKV) {
            // within both blocks; raw rows as loaded; escapes inside the windows
            n = min(n, min(kc.t1 - t, vc.t1 - t));
            if (kc.mode() == 0 || vc.mode() == 0) n = min(n, kRawRows);
            n = min(n, min(escape_rows<D>(kc, t - kc.t0), escape_rows<D>(vc, t - vc.t0)));
        }
        if (n <= 0) break; // unreachable with plan-checked descriptors (n_tokens > 0)
        const int tn = t + n;

        if constexpr (XKV) after(last_loaded<D>(RK)); // K rows arrived
        stamp(0);
        // 1. K rows -> tile (ORDER 1: and whether the chunk needs the flushing
        // score path)
        bool flush = false, kdirect = false;
        if constexpr (XKV) {
            if (kc.mode() != 0) {
                if constexpr (ORDER == 1) {
                    // coded exponents are base + code with code < 2^bits: all
                    // >= kmin when no base is below it or wraps (whole rows:
                    // every lane two bases, pieces: four, together every
                    // channel); bytes as 16-bit halves
                    const uint32_t w = kc.basew;
                    const u16x2 e = __builtin_bit_cast(u16x2, w & 0x00FF00FFu);
                    const u16x2 o = __builtin_bit_cast(u16x2, (w >> 8) & 0x00FF00FFu);
                    u16x2 bmin = __builtin_elementwise_min(e, o), bmax = __builtin_elementwise_max(e, o);
                    if constexpr (kWholeRows<D>) bmin.y = bmin.x, bmax.y = bmax.x; // the upper halves hold no base
                    const uint32_t top = 256u - (1u << kc.mode());
                    flush = __ballot(uint32_t(min(bmin.x, bmin.y)) < kmin || uint32_t(max(bmax.x, bmax.y)) > top) != 0;
                }
                if constexpr (kWholeRows<D>) {
                    base_pairs<D>(kc, S.bp);
                    wave_sync();
                }
            } else {
                flush = ORDER == 1;
            }
            // whole rows: a 4- or 2-bit chunk without escapes (and, in the
            // AVX-512 order, without a possible flush) is decoded octet by
            // octet into the score products below, not into the tile
            if constexpr (kDirectK<D, ORDER>)
                kdirect = (kc.mode() == 4 || kc.mode() == 2) && !flush && !rows_have_escapes<D>(kc, t - kc.t0, n);
            if (!kdirect) {
                decode_rows<D>(kc, RK, S.bp, S.tile, n, sm_mask_vgpr());
                wave_sync();
                flush |= patch_escapes<D, ORDER == 1>(kc, t - kc.t0, n, S.tile, klow);
            }
        } else {
            store_raw<D>(RK, S.tile);
            if constexpr (ORDER == 1) {
                // any element of the chunk's rows (pieces of rows < n) below the bound
                u16x2 lo = {0xFFFFu, 0xFFFFu};
#pragma unroll
                for (int j = 0; j < D / 8; ++j) {
                    if ((1024 * j + 16 * ln) / (2 * D) >= n) continue;
                    const uint32_t c4[4] = {RK[j].x, RK[j].y, RK[j].z, RK[j].w};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        lo = __builtin_elementwise_min(lo, (__builtin_bit_cast(u16x2, c4[k]) & uint16_t(0x7FFF)) -
                                                               uint16_t(1));
                }
                flush = __ballot(uint32_t(min(lo.x, lo.y)) < klow) != 0;
            }
        }
        wave_sync();

        stamp(1); // K decoded
        // 2. scores, lane = token
        float s[G];
        if constexpr (ORDER == 0) {
            if constexpr (XKV && kDirectK<D, ORDER>) {
                if (kdirect) {
                    const uint32_t smm = sm_mask_vgpr();
                    if (kc.mode() == 4) scores_coded<G, D, 4>(RK, S.bp, smm, qa, s);
                    else scores_coded<G, D, 2>(RK, S.bp, smm, qa, s);
                } else {
                    scores<G, D>(S.tile + ln * TS, qa, s);
                }
            } else {
                scores<G, D>(S.tile + ln * TS, qa, s);
            }
        } else if (!flush) {
            if constexpr (XKV && kDirectK<D, ORDER>) {
                if (kdirect) {
                    const uint32_t smm = sm_mask_vgpr();
                    if (kc.mode() == 4)
                        scores_dp_of<G, D>([&](int dg) { return coded_octet<D, 4>(RK, dg, S.bp, smm); }, qa, s);
                    else
                        scores_dp_of<G, D>([&](int dg) { return coded_octet<D, 2>(RK, dg, S.bp, smm); }, qa, s);
                } else {
                    scores_dp<G, D>(S.tile + ln * TS, qa, s);
                }
            } else {
                scores_dp<G, D>(S.tile + ln * TS, qa, s);
            }
        } else {
            scores_dp_flush<G, D>(S.tile + ln * TS, q_all + size_t(hd.q_row) * D, &S.eT[0][0]);
            wave_sync();
#pragma unroll
            for (int g = 0; g < G; ++g) s[g] = S.eT[g][ln];
        }
        wave_sync();

        after(__float_as_uint(s[0]));
        stamp(2); // scores done
        // 3. softmax coefficients, lane = token: the running maxima by an exact
        // DPP prefix maximum (seeded with each row's maximum so far, held in
        // scalar registers), then e = exp(s - m) and alpha = exp(m_prev - m)
        // for every token and row (softmax.hpp:8-14). A token moves its row's
        // maximum exactly when it scores above the maximum before it (a NaN
        // score never does), and then m = s, so its e is exp(0); a token that
        // does not has m_prev = m, so its alpha is exp(0) (NaN where the
        // maximum is infinite, as in the reference): one exponential per
        // token and row gives both, with no branch on the rows. Tokens past
        // the chunk's end get e = 0 and alpha = 1. The exponentials run in
        // batches of up to four rows: every row's reduction and table read,
        // then every row's polynomial, so that the table reads are in flight
        // together.
        const uint64_t nmask = n >= kChunk ? ~0ull : ((1ull << n) - 1ull);
        float mi[G];
        uint64_t amask = 0;
#pragma unroll
        for (int g = 0; g < G; ++g) mi[g] = s[g];
        wave_scan_max_rows<G>(mi);
#pragma unroll
        for (int g0 = 0; g0 < G; g0 += 4) {
            constexpr int B = 4;
            float m[B], mp[B], x[B];
            double kd[B], rr[B];
            uint64_t tb[B];
#pragma unroll
            for (int b = 0; b < B; ++b) {
                if (g0 + b >= G) break;
                const int g = g0 + b;
                m[b] = max_f32(mi[g], msc[g]);
                // the maximum before this token; the token moves it exactly
                // when it scores above it, and then m = s
                mp[b] = wave_shift_up(m[b], msc[g]);
                // one exponential per token: alpha's argument where the token
                // moves the maximum (its e is exp(0)), e's elsewhere (its
                // alpha is exp(0), or NaN where m_prev - m is)
                x[b] = lane_select(__ballot(s[g] > mp[b]), mp[b] - s[g], s[g] - m[b]);
                kvexp_expf_reduce(x[b], kd[b], rr[b]);
                tb[b] = tab[uint32_t(__double_as_longlong(kd[b])) & 31u];
            }
#pragma unroll
            for (int b = 0; b < B; ++b) {
                if (g0 + b >= G) break;
                const int g = g0 + b;
                float y = kvexp_expf_finish(kd[b], rr[b], tb[b]);
                // glibc's expf gives +0 below -0x1.9fe368p6 (the core does not)
                y = lane_select_or0(__ballot(!(x[b] < -0x1.9fe368p6f)), y);
                const float dg = mp[b] - m[b];
                // alpha != 1 exactly when m_prev - m is not zero (NaN included)
                amask |= __ballot(!(dg == 0.0f)) & nmask;
                // a moving token: e = exp(s - m) with s = m, that is exp(0)
                // = 1, or NaN where s is infinite (s - m + 1 gives both);
                // elsewhere alpha = exp(dg) with dg 0 or NaN (dg + 1)
                const uint64_t mv = __ballot(s[g] > mp[b]); // the lanes whose token moves the maximum
                const float e = lane_select(mv, (s[g] - m[b]) + 1.0f, y);
                const float al = lane_select(mv, y, dg + 1.0f);
                S.eT[g][ln] = lane_select_or0(nmask, e); // lanes ln < n
                S.aT[g][ln] = lane_select_or1(nmask, al);
                msc[g] = readlane_f32(m[b], n - 1);
            }
        }
        wave_sync();

        stamp(3); // softmax coefficients in LDS
        if constexpr (XKV) after(last_loaded<D>(RV)); // V rows arrived
        stamp(4);
        // 4. V rows -> tile (the scores are then no longer live); request the
        // next chunk's K and V rows (RK and RV are then not live across the
        // score and decode registers)
        if constexpr (XKV) {
            // the loads are issued on every chunk (the last one re-reads its
            // own final row), the next K rows before the next V rows: the K
            // decode can then wait for its loads while the V loads stay in
            // flight. At head_dim 64 and 128 the K rows are requested before
            // this chunk's V decode (which waits only for the older V rows;
            // c2 and c4 about 1 % faster), at 256 after it (no gain measured
            // there, where one wave per SIMD has registers to spare).
            const int tp = min(tn, wi.tok_end - 1);
            auto request_k = [&]() {
                if (tp >= kc.t1) enter_block(kc, kc.d + 1, kc.t1);
                stamp(7); // next K block entered
                block_vectors<D>(kc);
                load_rows<D>(kc, tp - kc.t0, min(kChunk, min(kc.t1, wi.tok_end) - tp), RK);
                stamp(8); // next K rows requested
            };
            if constexpr (D <= 128) request_k();
            if constexpr (kWholeRows<D>) {
                if (vc.mode() != 0) {
                    base_pairs<D>(vc, S.bp);
                    wave_sync();
                }
            }
            decode_rows<D>(vc, RV, S.bp, S.tile, n, sm_mask_vgpr());
            wave_sync();
            stamp(5); // V rows decoded
            patch_escapes<D>(vc, t - vc.t0, n, S.tile);
            stamp(6); // V escapes written
            if constexpr (D > 128) request_k();
            if (tp >= vc.t1) enter_block(vc, vc.d + 1, vc.t1);
            stamp(9); // next V block entered
            block_vectors<D>(vc);
            load_rows<D>(vc, tp - vc.t0, min(kChunk, min(vc.t1, wi.tok_end) - tp), RV);
        } else {
            store_raw<D>(RV, S.tile);
            if (n < kChunk && ln >= n) fill_negzero<D>(S.tile + ln * TS);
            {
                // issued on every chunk (the last one re-reads its final row), K first
                const int tp = min(tn, wi.tok_end - 1);
                load_raw<D>(hd.kraw, tp, min(kChunk, wi.tok_end - tp), RK);
                load_raw<D>(hd.vraw, tp, min(kChunk, wi.tok_end - tp), RV);
            }
        }

        stamp(10); // next V rows requested
        // 5. ordered fold, lane = channel, fully unrolled over the chunk
        {
            // e as the A operands: ea[rg][j] at lane 4b + r holds e[4 rg + r][16 j + b]
            // (rows past G repeat row G - 1; their results are not used)
            // (the lane index passes through an empty asm so that these LDS
            // addresses are made here, not kept live across the loop)
            int lq = ln;
            asm volatile("" : "+v"(lq));
            float ea[NG][4];
#pragma unroll
            for (int rg = 0; rg < NG; ++rg) {
                const int g = min(4 * rg + (lq & 3), G - 1);
#pragma unroll
                for (int j = 0; j < 4; ++j) ea[rg][j] = S.eT[g][16 * j + (ln >> 2)];
            }
            const int gl = min(ln & 7, G - 1); // lanes >= G read a row they do not use
            lds_f32 *eb = (lds_f32 *)&S.eT[gl][0];
            lds_f32 *ab = (lds_f32 *)&S.aT[gl][0];
            FoldIn<H> in;
            const uint16_t *vb = reinterpret_cast<const uint16_t *>(S.tile) + ln; // channel lane of token 0
            const uint8_t *trb = S.tile + tr_lane_offset<D>(ln);                   // the lane's load_tr address
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int h = 0; h < H; ++h) in.vq[k][h] = load_tr(trb + 4 * k * TS + 128 * h);
            in.e4[0] = *reinterpret_cast<lds_f4 *>(eb);
            // amask as two words behind an empty asm: the group tests stay
            // 32-bit scalar compares (not a 64-bit vector compare against a
            // constant held in registers)
            uint32_t am[2] = {uint32_t(amask), uint32_t(amask >> 32)};
            asm volatile("" : "+s"(am[0]), "+s"(am[1]));
            fold<G, D, 0>(S, eb, ab, vb, trb, am, ea, in, acc, lvec);
        }
        wave_sync();
        after(__float_as_uint(acc[0][0].x));
        stamp(11); // fold done
        t = tn;
    }
#if defined(KVEXP_PHASE_TRACE)
    if constexpr (TR) {
        if (lane == 0 && item < kTraceWaves) {
            unsigned long long *o = g_phase_trace + size_t(item) * kTraceWords;
            o[0] = tw0;
            o[1] = __builtin_readcyclecounter();
            for (int i = 0; i < kTracePhases; ++i) o[2 + i] = ph[i];
            // the CU, then the split's device head and split number
            o[kTracePhases + 2] = (unsigned long long)__smid() | ((unsigned long long)wi.head << 16) |
                                  ((unsigned long long)wi.split << 40);
        }
    }
#endif

    // ---- epilogue --------------------------------------------------------------
    float mv = msc[0]; // lane g < G: running maximum of row g
#pragma unroll
    for (int g = 1; g < G; ++g) mv = lane == g ? msc[g] : mv;
    if (hd.n_splits == 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float l = readlane_f32(lvec, g);
#pragma unroll
            for (int h = 0; h < H; ++h)
                out_all[(size_t(hd.q_row) + g) * D + 64 * h + lane] = acc[g / 4][h][g % 4] * (1.0f / l);
        }
        if (lse_all != nullptr && lane < G) lse_all[hd.q_row + lane] = mv + logf(lvec);
        return;
    }
    float *slot = ws + size_t(hd.ws_base + wi.split) * Shape<D>::kSlotFloats;
    if (lane < G) {
        slot[lane] = mv;
        slot[kSlotQ + lane] = lvec;
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int h = 0; h < H; ++h) slot[2 * kSlotQ + g * D + 64 * h + lane] = acc[g / 4][h][g % 4];
}

// Waves (merge items) per workgroup of the merge kernel: one, so that a
// launch's few hundred items spread over every CU (c2: 336 items; 4.97 us
// per launch against 5.25 with four waves per workgroup on 84 CUs).
constexpr int kMergeWaves = 1;

// Ordered merge of a head's split states (softmax.hpp:16-30 merge_state,
// left to right in split order; dispatch.cpp:98-103), then out = acc * (1/l)
// and lse = m + log l. One wave per merge item (device head, query row): lane
// = channel (channels lane + 64 h) for the accumulators. A separate launch,
// so the slots written by the split kernel are visible without fences.
//
// Splits go in batches of kMergeBatch. In a batch, lane j first loads m and
// l of split s0 + j, then every lane its channels of the batch's
// accumulator rows (all loads in flight together). While the rows arrive,
// lane j computes the running maximum after split s0 + j (a wave scan; the
// maximum is exact in any grouping), the two exponentials of its merge step
// (e1 scales the running state, e2 the split) and l_j * e2 (the same product
// merge_state forms), and stages the three in LDS. The ordered chains then
// read them four splits at a time (one broadcast LDS read per operand) and
// take one fused multiply-add per split and channel, as merge_state does.
// The first batch starts from split 0's state, as dispatch.cpp does.
template <int D>
__global__ __launch_bounds__(kMergeWaves * 64) void wave_merge_kernel(
    const MergeItem *__restrict__ mitems, int n_mitems, MergeItem uni, float *__restrict__ out_all,
    float *__restrict__ lse_all, const float *__restrict__ ws) {
    constexpr int H = D / 64, B = Shape<D>::kMergeBatch, SF = Shape<D>::kSlotFloats;
    static_assert(B % 4 == 0 && B <= kWave, "one split per lane, read four at a time");
    __shared__ uint64_t tab[32];
    __shared__ float stage[kMergeWaves][3][B]; // per wave: e1, e2 and l * e2 of the batch's splits
    if (threadIdx.x < 64) kvexp_exp_table_to_lds(tab);
    __syncthreads();
    const int lane = lane_id();
    const int w = int(threadIdx.x) >> 6;
    const int mi = __builtin_amdgcn_readfirstlane(int(blockIdx.x) * kMergeWaves + w);
    if (mi >= n_mitems) return;
    // uni.g > 0: item i is (uni.ws_base + k uni.n_splits, uni.n_splits,
    // uni.q_row + k uni.g, i - k uni.g) with k = i / uni.g, so the slots'
    // loads need not wait for the item's
    MergeItem it;
    if (uni.g > 0) {
        const int k = mi / uni.g;
        it = MergeItem{uni.ws_base + k * uni.n_splits, uni.n_splits, uni.q_row + k * uni.g, mi - k * uni.g};
    } else {
        it = load_scalar(mitems + mi);
    }
    const int g = it.g;
    const float *slots = ws + size_t(it.ws_base) * SF;
    const int n = it.n_splits;
    lds_f32 *st = (lds_f32 *)&stage[w][0][0];
    float a[H] = {};
    float mf = 0.0f, lf = 0.0f;
    for (int s0 = 0; s0 < n; s0 += B) {
        const int cnt = min(B, n - s0);
        const float *ls = slots + size_t(s0 + min(lane, cnt - 1)) * SF;
        const float ms = lane < cnt ? ls[g] : -__builtin_inff();
        const float lb = ls[kSlotQ + g];
        float ab[B][H];
#pragma unroll
        for (int j = 0; j < B; ++j)
#pragma unroll
            for (int c = 0; c < H; ++c)
                ab[j][c] = slots[size_t(s0 + min(j, cnt - 1)) * SF + 2 * kSlotQ + g * D + 64 * c + lane];
        const int j0 = s0 == 0 ? 1 : 0; // split 0 is the starting state
        if (s0 == 0) mf = readlane_f32(ms, 0);
        const float mm = fmaxf(wave_scan_max(ms), mf);
        const float mprev = wave_shift_up(mm, mf);
        const float e1 = kvexp_expf_nonpos_nb(mprev - mm, tab); // scale of the running state
        const float e2 = kvexp_expf_nonpos_nb(ms - mm, tab);    // scale of split s0 + lane
        if (lane < B) {
            stage[w][0][lane] = e1;
            stage[w][1][lane] = e2;
            stage[w][2][lane] = lb * e2;
        }
        mf = readlane_f32(mm, cnt - 1);
        wave_sync();
        if (s0 == 0) {
            lf = readlane_f32(lb, 0);
#pragma unroll
            for (int c = 0; c < H; ++c) a[c] = ab[0][c];
        }
#pragma unroll
        for (int jq = 0; jq < B; jq += 4) {
            if (jq >= cnt) continue;
            const f4 x1 = *reinterpret_cast<lds_f4 *>(st + jq);
            const f4 x2 = *reinterpret_cast<lds_f4 *>(st + B + jq);
            const f4 pl = *reinterpret_cast<lds_f4 *>(st + 2 * B + jq);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (jq + k >= j0 && jq + k < cnt) {
#pragma unroll
                    for (int c = 0; c < H; ++c) a[c] = fmaf(a[c], x1[k], ab[jq + k][c] * x2[k]);
                    lf = fmaf(lf, x1[k], pl[k]);
                }
            }
        }
        wave_sync(); // the next batch overwrites the stage
    }
#pragma unroll
    for (int c = 0; c < H; ++c) out_all[(size_t(it.q_row) + g) * D + 64 * c + lane] = a[c] * (1.0f / lf);
    if (lse_all != nullptr && lane == 0) lse_all[it.q_row + g] = mf + logf(lf);
}

} // namespace wave
} // namespace kvexp_dev

namespace kvexp_launch {
using namespace kvexp_dev;

template <int G, int D, bool XKV, int ORDER>
static hipError_t launch_wave_g(const HeadDev *heads, const WorkItem *items, int n_items, int wpg,
                                const BlockDesc *desc, const uint16_t *q, float *out, float *lse, float *ws,
                                hipStream_t s) {
    // wpg waves (work items) per workgroup: the kernel's count, or fewer
    // (1) where a launch has no more items than CUs, so they spread over as
    // many CUs
    const int W = wpg >= 1 && wpg <= wave::Shape<D>::kWaves ? wpg : wave::Shape<D>::kWaves;
    const int grid = (n_items + W - 1) / W;
    hipLaunchKernelGGL((wave::attn_wave_kernel<G, D, XKV, ORDER>), dim3(grid), dim3(W * 64), 0, s, heads, items,
                       n_items, W, desc, q, out, lse, ws);
    return hipGetLastError();
}

template <int D, bool XKV, int ORDER>
static hipError_t launch_wave_x(int G, const HeadDev *heads, const WorkItem *items, int n_items, int wpg,
                                const BlockDesc *desc, const uint16_t *q, float *out, float *lse, float *ws,
                                hipStream_t s) {
    switch (G) {
    case 1: return launch_wave_g<1, D, XKV, ORDER>(heads, items, n_items, wpg, desc, q, out, lse, ws, s);
    case 2: return launch_wave_g<2, D, XKV, ORDER>(heads, items, n_items, wpg, desc, q, out, lse, ws, s);
    case 3: return launch_wave_g<3, D, XKV, ORDER>(heads, items, n_items, wpg, desc, q, out, lse, ws, s);
    case 4: return launch_wave_g<4, D, XKV, ORDER>(heads, items, n_items, wpg, desc, q, out, lse, ws, s);
    case 5: return launch_wave_g<5, D, XKV, ORDER>(heads, items, n_items, wpg, desc, q, out, lse, ws, s);
    case 6: return launch_wave_g<6, D, XKV, ORDER>(heads, items, n_items, wpg, desc, q, out, lse, ws, s);
    case 7: return launch_wave_g<7, D, XKV, ORDER>(heads, items, n_items, wpg, desc, q, out, lse, ws, s);
    case 8: return launch_wave_g<8, D, XKV, ORDER>(heads, items, n_items, wpg, desc, q, out, lse, ws, s);
    default: return hipErrorInvalidValue;
    }
}

// The split kernels of one head_dim D and score order O (both the XKV and the
// plain BF16 instantiation, every query-row count), launched by G. Each
// (D, O) pair is instantiated in a translation unit of its own
// (attention_wave_d<D>_o<O>.hip), so that they compile in parallel.
// In a phase-trace build each unit also exports a reader of its own copy of
// the trace array (a file-scope device array exists once per unit).
#if defined(KVEXP_PHASE_TRACE)
#define KVEXP_WAVE_TRACE_READER(D, O)                                                                                \
    hipError_t attention_wave_d##D##_o##O##_trace_read(unsigned long long *host, size_t n) {                       \
        return hipMemcpyFromSymbol(host, HIP_SYMBOL(kvexp_dev::wave::g_phase_trace), n * 8);                        \
    }
#else
#define KVEXP_WAVE_TRACE_READER(D, O)
#endif
#define KVEXP_WAVE_UNIT(D, O)                                                                                        \
    hipError_t attention_wave_d##D##_o##O(bool xkv, int G, const HeadDev *heads, const WorkItem *items,             \
                                         int n_items, int wpg, const BlockDesc *desc, const uint16_t *q,           \
                                         float *out, float *lse, float *ws, hipStream_t s) {                       \
        return xkv ? launch_wave_x<D, true, O>(G, heads, items, n_items, wpg, desc, q, out, lse, ws, s)             \
                   : launch_wave_x<D, false, O>(G, heads, items, n_items, wpg, desc, q, out, lse, ws, s);           \
    }                                                                                                                \
    KVEXP_WAVE_TRACE_READER(D, O)

} // namespace kvexp_launch
