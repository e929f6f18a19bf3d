// Descriptors shared by the host planner and the gfx950 kernels.
#pragma once

#include <stdint.h>

namespace kvexp_dev {

// Status bits a kernel raises in the context's status word.
enum : uint32_t {
    kStHeader = 1u << 0,    // header past the end, dim mismatch or n_tokens == 0
    kStMode = 1u << 1,      // mode not in {0, 2, 4} (nor 3 with head_dim % 8 == 0)
    kStTruncated = 1u << 2, // payload past the end of the container
    kStEscape = 1u << 3,    // more sentinels than n_escape
    kStIndex = 1u << 4,     // block index disagrees with the headers
    kStLookback = 1u << 5,  // the fused encoder's wait for an earlier block's size ran out
};


// One KV head as the attention kernels see it (device copy, built by a plan).
struct HeadDev {
    const uint8_t *kx, *vx;      // containers (XKV heads)
    uint64_t kbytes, vbytes;
    const int64_t *koff, *voff;  // block byte offsets (n_blocks + 1)
    const int32_t *kfirst, *vfirst; // block first tokens (n_blocks + 1)
    const uint16_t *kraw, *vraw; // [seq, dim] BF16 (raw heads)
    // Plan-owned, XKV heads of the wave kernel: validated block descriptors
    // and the escape records (block b's escapes are records
    // [desc[b].esc, desc[b].esc + n_escape), in scan order; format at kEscPad).
    const struct BlockDesc *kdesc, *vdesc;
    const uint32_t *kesc, *vesc;
    int32_t seq;
    int32_t n_splits;            // work items of this head, in merge order
    int32_t ws_base;             // first partial-state slot of this head
    int32_t q_row;               // first query row of this head in d_q / d_out
    int32_t n_q;                 // query rows of this head (<= 8)
    int32_t pad;
};

// An escape record: the escape's element index inside its block (row * dim
// + channel) in bits 0..15 and its BF16 word in bits 16..31. The plan copies
// each block's escape words out of the container next to their positions, so
// the wave kernel reads a window of escapes with 16-byte loads per lane (up
// to 2,048 records). Every records array ends with kEscPad spare records, so
// such a window read from any escape of any block stays inside the
// allocation.
constexpr int kEscPad = 2052;

// One block of a container as the wave kernel reads it, built and checked
// against the block index once per plan (esc_start_kernel). 32 bytes, so a
// scalar load of one descriptor reads exactly one.
struct BlockDesc {
    const uint8_t *data; // the block's header
    const uint32_t *esc; // its escape records
    uint32_t meta;       // mode | n_tokens << 8 | n_escape << 16 (n_escape 0 for raw blocks)
    uint32_t pad[3];
};

// One tensor (container + block index) for the plan-time builders.
struct EscJob {
    const uint8_t *blob;
    uint64_t bytes;
    const int64_t *offs;
    const int32_t *first; // block first tokens (n_blocks + 1)
    int32_t *esc0;        // out: n_blocks + 1 entries
    uint32_t *pos;        // out: esc0[n_blocks] escape records
    BlockDesc *desc;      // out: n_blocks entries (nullable)
    int32_t n_blocks;
    int32_t dim;
    int32_t pos_cap;      // records of `pos` (the tensor's escapes plus room for its last block to grow)
    int32_t seq;          // tokens a plan update attends (esc_tail_kernel checks the index covers them)
};

// One split: tokens [tok_begin, tok_end) of a head; for XKV the blocks that
// hold tok_begin in K and V, as block indexes of the head's tensors and (one-
// wave kernel plans) as indexes into the plan's descriptor array (-1
// otherwise), so that the split's first descriptors load without waiting for
// the head. 32 bytes: one scalar load.
struct WorkItem {
    int32_t head;
    int32_t split;
    int32_t tok_begin, tok_end;
    int32_t kblk, vblk;
    int32_t kdi, vdi;
};

// One (device head, query row) of the one-wave kernel's merge: the head's
// first partial-state slot, its split count and output row, and the row.
struct MergeItem {
    int32_t ws_base;
    int32_t n_splits;
    int32_t q_row;
    int32_t g;
};

// Per-block result of the encoder's statistics pass.
// Size of the no-allocation encoder's device scratch (per GPU): block
// metadata and base-exponent candidates of up to about 20,000 blocks at
// head_dim 64 (2.6M tokens of 128-token blocks) or 5,300 at head_dim 256.
constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;

struct EncBlockMeta {
    int64_t bytes;
    int32_t mode;
    int32_t n_escape;
};

// Look-back state of the fused encoder: one entry per block of a launch
// (`words`), one ticket counter per job (`tickets`, an array of its own, left
// at 0 by every launch), the launch's epoch (1..65535), and how many entries
// and counters to clear before the launch (all of them when an array is new,
// the entries when the epoch wrapped, else 0).
struct EncLookback {
    uint64_t *words;
    uint32_t *tickets;
    uint32_t epoch;
    size_t clear_words;
    size_t clear_tickets;
};

// The fused encoder holds a block in registers: at most this many elements.
constexpr int kFusedMaxElems = 16384;

// Job of a batched append, as the kernels read it (built by the host API).
struct AppendJobDev {
    uint16_t *tail;        // raw trailing partial block [bt, dim] (read, then rewritten)
    const uint16_t *src;   // new tokens [n_new, dim]
    int64_t *offs;         // the container's index from its trailing block on
    int32_t *first;
    uint8_t *out;          // the container
    int32_t tail_n;        // raw tokens in `tail` (n_tokens % bt)
    int32_t seq;           // tokens encoded: tail_n + n_new
    int32_t tok0;          // first token of the trailing block
    int32_t blk0;          // first block of this job in the launch
    int32_t nb;            // blocks encoded
    int32_t rebase;        // the container is not empty (its trailing block starts at offs[0])
    int32_t copy_from;     // new-token row that starts the raw rows kept for the next append
    int32_t copy_to;       // their first row in `tail`
    int32_t copy_rows;
    int32_t pad;
};

} // namespace kvexp_dev
