// Descriptors shared by the host planner and the gfx950 kernels.
#pragma once

#include <stdint.h>

namespace kvexp_dev {

// Status bits a kernel raises in the context's status word.
enum : uint32_t {
    kStHeader = 1u << 0,    // header past the end, dim mismatch or n_tokens == 0
    kStMode = 1u << 1,      // mode not in {0, 2, 4}
    kStTruncated = 1u << 2, // payload past the end of the container
    kStEscape = 1u << 3,    // more sentinels than n_escape
    kStIndex = 1u << 4,     // block index disagrees with the headers
};


// One KV head as the attention kernels see it (device copy, built by a plan).
struct HeadDev {
    const uint8_t *kx, *vx;      // containers (XKV heads)
    uint64_t kbytes, vbytes;
    const int64_t *koff, *voff;  // block byte offsets (n_blocks + 1)
    const int32_t *kfirst, *vfirst; // block first tokens (n_blocks + 1)
    const uint16_t *kraw, *vraw; // [seq, dim] BF16 (raw heads)
    // Escape-position index (plan-owned, XKV heads of the wave kernel):
    // block b's escape words are entries [esc0[b], esc0[b+1]) and escpos[k]
    // is the element index (row * dim + channel) of entry k inside its block.
    const int32_t *kesc0, *vesc0;
    const uint16_t *kescpos, *vescpos;
    int32_t seq;
    int32_t n_splits;            // work items of this head, in merge order
    int32_t ws_base;             // first partial-state slot of this head
    int32_t q_row;               // first query row of this head in d_q / d_out
    int32_t n_q;                 // query rows of this head (<= 8)
    int32_t pad;
};

// One tensor (container + block index) for the escape-position index builders.
struct EscJob {
    const uint8_t *blob;
    uint64_t bytes;
    const int64_t *offs;
    int32_t *esc0;      // out: n_blocks + 1 entries
    uint16_t *pos;      // out: esc0[n_blocks] entries
    int32_t n_blocks;
    int32_t dim;
};

// One split: tokens [tok_begin, tok_end) of a head; for XKV the blocks that
// hold tok_begin in K and V.
struct WorkItem {
    int32_t head;
    int32_t split;
    int32_t tok_begin, tok_end;
    int32_t kblk, vblk;
};

// Per-block result of the encoder's statistics pass.
struct EncBlockMeta {
    int64_t bytes;
    int32_t mode;
    int32_t n_escape;
};

} // namespace kvexp_dev
