// The host side of the container walk: parse_block (scan.hpp:28-66) and the
// block index a reader of `seq` tokens touches (scan.hpp:144-151, 176-189),
// token_bounds (dispatch.cpp:17-23), and the failure type the C ABI turns
// into status codes. Plain C++ (no HIP), so the same code also builds into
// the sanitizer check (tests/csrc/sanitize_walk.cpp, oracle/Makefile).
#pragma once

#include "kvexp_hip.h"

#include <algorithm>
#include <climits>
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace kvexp_host {

struct KvexpFail {
    int code;
    std::string msg;
};

[[noreturn]] inline void fail(int code, const std::string &msg) { throw KvexpFail{code, msg}; }

struct HostBlock {
    int mode, n_tokens, n_escape;
    size_t next;
};

inline unsigned rd16(const uint8_t *p) { return unsigned(p[0]) | (unsigned(p[1]) << 8); }

// parse_block (scan.hpp:28-66): validation order and messages. Mode 3
// (3-bit codes, head_dim a multiple of 8) is this library's extension.
inline HostBlock parse_block_host(const uint8_t *blob, size_t bytes, size_t at, int dim) {
    if (bytes - at < 8) fail(KVEXP_HIP_FORMAT_ERROR, "truncated xkv block header");
    const uint8_t *p = blob + at;
    HostBlock b{p[0], p[1], int(rd16(p + 2)), 0};
    const int hdim = int(rd16(p + 4));
    if (hdim != dim || b.n_tokens <= 0) fail(KVEXP_HIP_FORMAT_ERROR, "xkv block dimension or length mismatch");
    const size_t body = at + 8;
    if (b.mode == 0) {
        const size_t nb = size_t(b.n_tokens) * size_t(dim) * 2u;
        if (bytes - body < nb) fail(KVEXP_HIP_FORMAT_ERROR, "truncated raw xkv block");
        b.next = body + nb;
        return b;
    }
    if (b.mode != 2 && b.mode != 4 && !(b.mode == 3 && dim % 8 == 0))
        fail(KVEXP_HIP_FORMAT_ERROR, "unknown xkv block mode");
    const size_t need = size_t(dim) + size_t(b.n_tokens) * size_t(dim) +
                        size_t((b.n_tokens * dim * b.mode + 7) / 8) + size_t(b.n_escape) * 2u;
    if (bytes - body < need) fail(KVEXP_HIP_FORMAT_ERROR, "truncated coded xkv block");
    b.next = body + need;
    return b;
}

// Blocks that a reader consuming `seq` tokens touches, then the eager parse of
// the following header (scan.hpp:144-151, 176-189).
inline void walk_index(const uint8_t *blob, size_t bytes, int dim, int seq, std::vector<int64_t> &off,
                std::vector<int32_t> &first) {
    off.clear();
    first.clear();
    size_t at = 0;
    int64_t tok = 0;
    while (at < bytes) {
        const HostBlock b = parse_block_host(blob, bytes, at, dim);
        if (tok >= seq) break;
        off.push_back(int64_t(at));
        first.push_back(int32_t(tok));
        tok += b.n_tokens;
        at = b.next;
    }
    off.push_back(int64_t(at));
    first.push_back(int32_t(std::min<int64_t>(tok, INT32_MAX)));
}

// token_bounds (dispatch.cpp:17-23).
inline void token_bounds(int seq, int tile, int tid, int n, int &a, int &b) {
    const int ntiles = (seq + tile - 1) / tile;
    const int b0 = int((long long)tid * ntiles / n);
    const int b1 = int((long long)(tid + 1) * ntiles / n);
    a = std::min(seq, b0 * tile);
    b = std::min(seq, b1 * tile);
}

} // namespace kvexp_host
