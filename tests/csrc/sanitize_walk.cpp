// CPU sanitizer check of the host container walk that libkvexp_hip.so runs
// before any launch (compressed-kv-attention_amd/csrc/host/host_walk.hpp:
// parse_block_host, walk_index, token_bounds) and of the C oracle
// (oracle/kvexp_oracle.c), both compiled with
// -fsanitize=address,undefined -fno-sanitize-recover=all by
// `make -C oracle sanitize` (gcc/g++ only, no GPU code) and run by
// tests/test_sanitize.py.
//
//  1. containers of many shapes (head_dim 4..256, 1..1000 tokens, 1..255
//     tokens per block, the reference's 2/4-bit policy and the 3-bit
//     extension), each held in a heap buffer of exactly its size: the decode
//     round trip is exact, and the host walk's block index equals the
//     oracle's for readers of several lengths;
//  2. the same containers cut at and inside the headers (every header of
//     a container of up to 24 blocks, 24 spread over a longer one, and the
//     last) and at random points, and with header fields and random bytes
//     changed: the walk and the oracle's index agree on the status, the
//     message and the index, and the oracle's decode either succeeds or
//     reports a format error;
//  3. token_bounds splits [0, seq) into ordered, contiguous, tile-aligned
//     ranges for every (seq, tile, n) in a grid;
//  4. small oracle attention runs of every backend over raw and XKV inputs
//     at the same splits are equal bit for bit (the container is lossless).
//
// A sanitizer report aborts the program; a mismatch is printed and the
// program exits with status 1 after the summary line.
#include "host_walk.hpp"
#include "kvexp_oracle.h"

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

namespace {

int g_bad = 0;

#define CHECK(cond, ...)                                                                                    \
    do {                                                                                                    \
        if (!(cond)) {                                                                                      \
            if (g_bad++ < 20) {                                                                             \
                std::fprintf(stderr, "%s:%d: ", __FILE__, __LINE__);                                        \
                std::fprintf(stderr, __VA_ARGS__);                                                          \
                std::fputc('\n', stderr);                                                                   \
            }                                                                                               \
        }                                                                                                   \
    } while (0)

struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
    uint64_t next() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return s;
    }
    int below(int n) { return int(next() % uint64_t(n)); }
    bool chance(double p) { return double(next() >> 11) * (1.0 / 9007199254740992.0) < p; }
};

// BF16 rows whose exponents stay within a few binades of a per-row centre,
// with planted outliers (escapes), an occasional wide block (4-bit or raw),
// and special values (zeros, subnormals, infinities, NaN).
std::vector<uint16_t> make_kv(Rng &r, int seq, int dim, int spread, double p_out, double p_special) {
    std::vector<uint16_t> kv(size_t(seq) * dim);
    for (int t = 0; t < seq; ++t) {
        const int centre = 110 + r.below(20);
        const int row_spread = r.chance(0.05) ? 12 : spread;
        for (int d = 0; d < dim; ++d) {
            int e = centre + r.below(row_spread + 1);
            if (r.chance(p_out)) e = r.below(254) + 1;
            uint16_t v = uint16_t((r.below(2) << 15) | (e << 7) | r.below(128));
            if (r.chance(p_special)) {
                static const uint16_t special[] = {0x0000, 0x8000, 0x0001, 0x807F, 0x7F80, 0xFF80, 0x7FC0, 0x7F81};
                v = special[r.below(8)];
            }
            kv[size_t(t) * dim + d] = v;
        }
    }
    return kv;
}

std::unique_ptr<uint8_t[]> exact_copy(const uint8_t *src, size_t n) {
    std::unique_ptr<uint8_t[]> p(new uint8_t[n]);
    if (n) std::memcpy(p.get(), src, n);
    return p;
}

struct Walk {
    int status = 0;
    std::string msg;
    std::vector<int64_t> off;
    std::vector<int32_t> first;
};

Walk host_walk(const uint8_t *blob, size_t bytes, int dim, int seq) {
    Walk w;
    try {
        kvexp_host::walk_index(blob, bytes, dim, seq, w.off, w.first);
    } catch (const kvexp_host::KvexpFail &e) {
        w.status = e.code;
        w.msg = e.msg;
        w.off.clear();
        w.first.clear();
    }
    return w;
}

Walk oracle_walk(const uint8_t *blob, size_t bytes, int dim, int seq) {
    Walk w;
    const int cap = int(bytes / 8) + (seq > 0 ? seq : 0) + 2;
    std::vector<int64_t> off(size_t(cap) + 1);
    std::vector<int32_t> first(size_t(cap) + 1);
    int nb = 0;
    w.status = oracle_block_index(blob, bytes, dim, seq, off.data(), first.data(), cap, &nb);
    if (w.status) {
        w.msg = oracle_last_error();
        return w;
    }
    w.off.assign(off.begin(), off.begin() + nb + 1);
    w.first.assign(first.begin(), first.begin() + nb + 1);
    return w;
}

// Walk and oracle index over one buffer, for readers of the given lengths;
// the oracle's decode of the same lengths must not crash and must either
// succeed or report a runtime (format) error.
void compare_walks(const uint8_t *blob, size_t bytes, int dim, const std::vector<int> &seqs, const char *what,
                   int *n_fail) {
    for (int seq : seqs) {
        const Walk a = host_walk(blob, bytes, dim, seq);
        const Walk b = oracle_walk(blob, bytes, dim, seq);
        CHECK(a.status == b.status && a.msg == b.msg, "%s seq %d: walk status %d '%s', oracle %d '%s'", what, seq,
              a.status, a.msg.c_str(), b.status, b.msg.c_str());
        CHECK(a.off == b.off && a.first == b.first, "%s seq %d: block index differs (%zu vs %zu entries)", what,
              seq, a.off.size(), b.off.size());
        if (a.status) ++*n_fail;
        if (seq > 0) {
            std::vector<uint16_t> out(size_t(seq) * dim);
            const int rc = oracle_decode(blob, bytes, seq, dim, out.data());
            CHECK(rc == 0 || rc == 2, "%s seq %d: oracle_decode status %d", what, seq, rc);
        }
    }
}

struct Container {
    int seq, dim, block;
    unsigned modes;
    std::vector<uint16_t> kv;
    std::vector<uint8_t> blob;
};

int g_containers = 0, g_cuts = 0, g_edits = 0, g_edit_failures = 0, g_attn = 0;

void check_container(Rng &r, const Container &c) {
    ++g_containers;
    const size_t bytes = c.blob.size();
    auto blob = exact_copy(c.blob.data(), bytes);
    char what[128];
    std::snprintf(what, sizeof what, "seq %d dim %d block %d modes %#x", c.seq, c.dim, c.block, c.modes);

    // 1. round trip and index agreement on the intact container
    std::vector<uint16_t> back(size_t(c.seq) * c.dim);
    CHECK(oracle_decode(blob.get(), bytes, c.seq, c.dim, back.data()) == 0, "%s: decode failed: %s", what,
          oracle_last_error());
    CHECK(back == c.kv, "%s: decode round trip differs", what);
    const std::vector<int> seqs = {1, (c.seq + 1) / 2, c.seq, c.seq + 7};
    int fails = 0;
    compare_walks(blob.get(), bytes, c.dim, seqs, what, &fails);
    CHECK(fails == 0, "%s: the intact container did not walk", what);
    const Walk w = host_walk(blob.get(), bytes, c.dim, c.seq + 7);
    CHECK(!w.off.empty() && size_t(w.off.back()) == bytes && w.first.back() == c.seq,
          "%s: the full walk does not end at the container's end", what);

    // 2a. cuts at and inside every header, and at random points
    std::vector<size_t> cuts;
    const size_t nblk = w.off.size() - 1, stride = nblk > 24 ? nblk / 24 : 1;
    for (size_t i = 0; i < nblk; i += stride)
        for (size_t k = 0; k <= 9; ++k) cuts.push_back(size_t(w.off[i]) + k);
    for (size_t k = 0; k <= 9; ++k) cuts.push_back(size_t(w.off[nblk - 1]) + k);
    for (int i = 0; i < 12; ++i) cuts.push_back(size_t(r.next() % (bytes + 1)));
    for (size_t cut : cuts) {
        if (cut > bytes) continue;
        ++g_cuts;
        auto part = exact_copy(blob.get(), cut);
        int f = 0;
        compare_walks(part.get(), cut, c.dim, {1, c.seq, c.seq + 7}, what, &f);
    }

    // 2b. header fields and random bytes changed
    for (int i = 0; i < 24; ++i) {
        ++g_edits;
        auto ed = exact_copy(blob.get(), bytes);
        if (i % 2 == 0 && w.off.size() > 1) {
            const size_t at = size_t(w.off[size_t(r.below(int(w.off.size()) - 1))]);
            const int field = r.below(6);
            ed[at + field] = uint8_t(r.chance(0.5) ? r.below(6) : r.below(256));
        } else {
            for (int k = 1 + r.below(3); k > 0; --k) ed[size_t(r.next() % bytes)] = uint8_t(r.below(256));
        }
        int f = 0;
        compare_walks(ed.get(), bytes, c.dim, {1, (c.seq + 1) / 2, c.seq}, what, &f);
        g_edit_failures += f != 0;
    }
}

// 3. token_bounds partitions [0, seq) into ordered, contiguous, tile-aligned ranges.
void check_token_bounds() {
    for (int seq = 1; seq <= 600; seq += 37)
        for (int tile : {1, 7, 64, 128, 255})
            for (int n : {1, 2, 3, 8, 64}) {
                int prev = 0;
                for (int tid = 0; tid < n; ++tid) {
                    int a = -1, b = -1;
                    kvexp_host::token_bounds(seq, tile, tid, n, a, b);
                    CHECK(a == prev && a <= b && b <= seq && (a == seq || a % tile == 0),
                          "token_bounds(%d, %d, %d, %d) = [%d, %d) after %d", seq, tile, tid, n, a, b, prev);
                    prev = b;
                }
                CHECK(prev == seq, "token_bounds(%d, %d, *, %d) ends at %d", seq, tile, n, prev);
            }
}

// 4. oracle attention over raw and XKV inputs at the same splits.
void check_attention(Rng &r) {
    struct Shape {
        int n_q, dim, seq, block, threads;
    };
    const Shape shapes[] = {{1, 64, 1, 128, 1}, {7, 64, 300, 128, 3}, {4, 128, 257, 64, 4},
                            {2, 256, 130, 128, 2}, {3, 32, 45, 8, 5}};
    for (const Shape &s : shapes) {
        const auto k = make_kv(r, s.seq, s.dim, 2, 0.003, 0.0);
        const auto v = make_kv(r, s.seq, s.dim, 2, 0.003, 0.0);
        auto q = make_kv(r, s.n_q, s.dim, 3, 0.0, 0.0);
        std::vector<uint8_t> kx(oracle_encode_bound(s.seq, s.dim, s.block));
        std::vector<uint8_t> vx(kx.size());
        size_t kb = 0, vb = 0;
        CHECK(oracle_encode(k.data(), s.seq, s.dim, s.block, kx.data(), kx.size(), &kb) == 0, "encode K");
        CHECK(oracle_encode(v.data(), s.seq, s.dim, s.block, vx.data(), vx.size(), &vb) == 0, "encode V");
        auto kxe = exact_copy(kx.data(), kb), vxe = exact_copy(vx.data(), vb);
        for (int backend = 0; backend < 3; ++backend) {
            ++g_attn;
            const size_t na = size_t(s.n_q) * s.dim;
            std::vector<float> o_raw(na), o_xkv(na), l_raw(s.n_q), l_xkv(s.n_q);
            const int rc1 = oracle_attention(backend, q.data(), k.data(), v.data(), nullptr, 0, nullptr, 0,
                                             o_raw.data(), l_raw.data(), s.n_q, s.dim, s.seq, s.threads, s.block);
            const int rc2 = oracle_attention(backend, q.data(), nullptr, nullptr, kxe.get(), kb, vxe.get(), vb,
                                             o_xkv.data(), l_xkv.data(), s.n_q, s.dim, s.seq, s.threads, s.block);
            CHECK(rc1 == 0 && rc2 == 0, "attention backend %d dim %d: status %d %d (%s)", backend, s.dim, rc1,
                  rc2, oracle_last_error());
            CHECK(std::memcmp(o_raw.data(), o_xkv.data(), na * sizeof(float)) == 0 &&
                      std::memcmp(l_raw.data(), l_xkv.data(), s.n_q * sizeof(float)) == 0,
                  "attention backend %d dim %d seq %d: raw and XKV outputs differ", backend, s.dim, s.seq);
        }
    }
}

} // namespace

int main() {
    Rng r(20260);
    const int dims[] = {4, 8, 12, 64, 128, 256};
    const int seqs[] = {1, 5, 128, 129, 1000};
    const int blocks[] = {1, 3, 100, 128, 255};
    for (int dim : dims)
        for (int seq : seqs)
            for (int block : blocks) {
                if (dim == 256 && seq == 1000 && block < 100) continue; // size only, same code paths
                for (unsigned modes : {unsigned(ORACLE_MODES_REFERENCE), unsigned(ORACLE_MODES_REFERENCE | ORACLE_MODE_3BIT)}) {
                    if ((modes & ORACLE_MODE_3BIT) && dim % 8 != 0) continue;
                    Container c{seq, dim, block, modes, {}, {}};
                    c.kv = make_kv(r, seq, dim, r.below(2) ? 2 : 5, 0.004, 0.002);
                    c.blob.resize(oracle_encode_bound(seq, dim, block));
                    size_t bytes = 0;
                    const int rc = oracle_encode_modes(c.kv.data(), seq, dim, block, modes, c.blob.data(),
                                                       c.blob.size(), &bytes);
                    CHECK(rc == 0, "encode seq %d dim %d block %d: %s", seq, dim, block, oracle_last_error());
                    if (rc) continue;
                    c.blob.resize(bytes);
                    check_container(r, c);
                }
            }
    check_token_bounds();
    check_attention(r);
    std::printf("sanitize_walk: %d containers, %d cuts, %d edits (%d refused), %d attention runs: %s\n",
                g_containers, g_cuts, g_edits, g_edit_failures, g_attn, g_bad ? "MISMATCH" : "ok");
    return g_bad ? 1 : 0;
}
