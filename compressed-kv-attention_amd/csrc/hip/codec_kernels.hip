// gfx950 kernels for the XKV container: block decode and the encoder.
//
// Decode (reference src/codec.cpp:166-174 via XkvReader::read_next,
// include/kvexp/scan.hpp:125-155): one workgroup per block. A coded element
// is bf16_from_delta(base[d], code, sm) unless its code is the all-ones
// sentinel, in which case it is the next escape word of the block in scan
// order; the escape rank of each element comes from a workgroup prefix sum
// of per-thread sentinel counts.
//
// Encode (reference src/codec.cpp:18-164), three launches:
//   1. per block: exponent histogram per channel, the smallest base that
//      covers the most exponents for 2- and 4-bit windows, escape counts,
//      and the mode choice with the reference's tie rules;
//   2. one workgroup: prefix sum of block sizes -> block byte offsets and
//      first tokens (the block index the attention kernels read);
//   3. per block: header, base, sign/mantissa bytes, packed codes, escapes.
// Appends run the same three steps over a batch of containers (one job per
// container: its trailing partial block and the new blocks), reading each
// block's rows from the job's raw tail and new tokens in place, then store
// the new trailing partial block's raw tokens for the next append.
#include "kvexp_device.h"
#include <algorithm>
#include <mutex>
#include "kvexp_types.h"

namespace kvexp_dev {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// ----------------------------------------------------------------- decode --
__global__ __launch_bounds__(kThreads) void decode_blocks_kernel(const uint8_t *__restrict__ blob, uint64_t bytes,
                                                                const int64_t *__restrict__ offs,
                                                                const int32_t *__restrict__ first, int seq, int dim,
                                                                uint16_t *__restrict__ out,
                                                                uint32_t *__restrict__ status) {
    __shared__ int scan_tmp[kWaves];
    const int b = int(blockIdx.x);
    const int t0 = first[b];
    const int want = first[b + 1] - t0;
    const int64_t off = offs[b];
    BlockHdr h;
    const uint32_t st = check_block(blob, bytes, off, dim, want, &h);
    if (st != 0u) {
        if (threadIdx.x == 0) atomicOr(status, st);
        return;
    }
    const int rows = min(want, seq - t0);
    if (rows <= 0) return;
    const uint8_t *p = blob + off + 8;
    uint16_t *o = out + size_t(t0) * size_t(dim);
    const int total = rows * dim;
    if (h.mode == 0) {
        for (int i = int(threadIdx.x); i < total; i += kThreads) o[i] = uint16_t(load_u16_any(p + 2 * i));
        return;
    }
    const int mode = h.mode;
    const int U = code_unit(mode);
    const uint32_t sentinel = (1u << mode) - 1u;
    const uint8_t *base = p;
    const uint8_t *sm = p + dim;
    const uint8_t *codes = sm + size_t(h.n_tokens) * size_t(dim);
    const uint8_t *esc = codes + exp_payload_bytes(h.n_tokens, dim, mode);
    const int units = total / U; // dim % 4 == 0 (dim % 8 == 0 for 3-bit codes)
    int carry = 0;
    uint32_t bad = 0;
    for (int r = 0; r < units; r += kThreads) {
        const int u = r + int(threadIdx.x);
        const bool act = u < units;
        uint32_t cw = 0;
        int cnt = 0;
        if (act) {
            cw = load_codes(codes, mode, u);
            cnt = unit_sentinels(cw, mode);
        }
        int rank = carry;
        if (h.n_escape > 0) {
            int tot = 0;
            rank += block_excl_scan<kWaves>(cnt, scan_tmp, &tot);
            carry += tot;
        }
        if (act) {
            const int e0 = U * u;
            const int d0 = e0 % dim;
            uint32_t v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (k >= U) break;
                const uint32_t code = unit_code(cw, mode, k);
                if (code == sentinel) {
                    if (rank < h.n_escape) {
                        v[k] = load_u16_any(esc + 2 * size_t(rank));
                    } else {
                        v[k] = 0;
                        bad = kStEscape;
                    }
                    ++rank;
                } else {
                    v[k] = bf16_join(uint32_t(base[d0 + k]) + code, load_u8(sm + e0 + k));
                }
            }
            for (int k = 0; k < U; k += 4) {
                uint2 w;
                w.x = v[k] | (v[k + 1] << 16);
                w.y = v[k + 2] | (v[k + 3] << 16);
                *reinterpret_cast<uint2 *>(o + e0 + k) = w;
            }
        }
    }
    if (bad) atomicOr(status, bad);
}

// The elements of one block to encode, token-major: elements [0, split) at
// a, the rest at b (an append's first block starts with the raw tokens of
// the container's trailing partial block, then the new tokens).
struct EncRows {
    const uint16_t *a, *b;
    int split;
    __device__ __forceinline__ uint32_t at(int i) const { return i < split ? a[i] : b[i - split]; }
};

// The job holding launch block g (jobs sorted by blk0; wave-uniform).
__device__ __forceinline__ int find_job(const AppendJobDev *jobs, int n_jobs, int g) {
    int lo = 0, hi = n_jobs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (jobs[mid].blk0 <= g) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Rows of local block b of an append job: block 0 starts with the job's raw
// tail (tail_n rows), every block then reads new tokens.
__device__ __forceinline__ EncRows job_rows(const AppendJobDev &j, int b, int bt, int dim) {
    const int t0 = b * bt;
    const int na = b == 0 ? j.tail_n : 0;
    EncRows r;
    r.a = j.tail;
    r.b = j.src + size_t(t0 + na - j.tail_n) * size_t(dim);
    r.split = na * dim;
    return r;
}

// ------------------------------------------------------------ encode: stats --
// bases: [n_blocks][3][dim] (2-, 3- and 4-bit window bases). `modes` has bit
// m set for each coded mode m that may be chosen (raw always may): bits 2
// and 4 give the reference's encoder; bit 3 adds the 3-bit extension, taken
// only when dim % 8 == 0.
// A channel's exponents are counted in a column of LDS byte counters (four
// bins per dword; a block has at most 255 tokens, so a byte cannot overflow
// into its neighbour) with fire-and-forget LDS adds by the threads of every
// row slice; one thread per column then slides
// each code window over the bins between its smallest and largest exponent
// (windows outside them cover nothing) to find best_base: the most covered
// exponents, then the smallest base (codec.cpp:18-35).
constexpr int kHistStride = 65; // dwords per channel column (64 + 1: columns start on different banks)

// LDS of the statistics: stats_cols(dim) channel columns, the per-wave
// escape sums (3 per wave), each column's smallest and largest exponent.
// The stats kernels run kThreads threads: 4 row slices at head_dim <= 64,
// 2 above.
__host__ __device__ constexpr int stats_cols(int dim) { return dim > 64 ? 128 : 64; }
__host__ __device__ constexpr size_t stats_lds_bytes(int dim) {
    return size_t(stats_cols(dim)) * kHistStride * sizeof(uint32_t) +
           (3 * kWaves + 2 * stats_cols(dim)) * sizeof(int);
}

__device__ __forceinline__ void encode_stats_block(uint32_t *hist, int *esc_part, const EncRows src, int n, int dim,
                                                   EncBlockMeta *__restrict__ meta, uint8_t *__restrict__ bases,
                                                   int modes) {
    const int tid = int(threadIdx.x);
    // Channel columns: thread `own` of each row slice counts channels own,
    // own + nthr, ... of rows slice, slice + nslices, ... into the column of
    // `own` (LDS adds, so the slices share it); after a barrier the threads
    // of slice 0 slide the windows. blockDim.x is a multiple of nthr.
    const int nthr = min(int(blockDim.x), stats_cols(dim));
    const int own = tid % nthr, slice = tid / nthr, nslices = int(blockDim.x) / nthr;
    uint32_t *h = hist + own * kHistStride;
    int *lohi = esc_part + 3 * kWaves; // [2][nthr]: smallest and largest exponent of each column
    int esc[3] = {0, 0, 0}; // escapes of the 2-, 3- and 4-bit codes
    const int nwin = (modes & 8) && dim % 8 == 0 ? 3 : 2; // windows computed (the 3-bit one only when allowed)
    const int na = min(n, src.split / dim);
    for (int d0 = 0; d0 < dim; d0 += nthr) {
        const int d = d0 + own;
        const bool has = d < dim;
        if (slice == 0 && has) {
#pragma unroll 16
            for (int k = 0; k < 64; ++k) h[k] = 0u;
            lohi[own] = 255;
            lohi[nthr + own] = 0;
        }
        __syncthreads();
        if (has) {
            int e_lo = 255, e_hi = 0;
            // this slice's rows, 32 loads in flight before their adds; rows
            // [0, na) come from src.a, the rest from src.b
            for (int r0 = slice; r0 < n; r0 += 32 * nslices) {
                uint32_t x[32];
#pragma unroll
                for (int k = 0; k < 32; ++k) {
                    const int r = r0 + k * nslices;
                    x[k] = r < n ? uint32_t(r < na ? src.a[r * dim + d] : src.b[(r - na) * dim + d]) : 0xFFFFFFFFu;
                }
#pragma unroll
                for (int k = 0; k < 32; ++k) {
                    if (x[k] == 0xFFFFFFFFu) break;
                    const uint32_t e = (x[k] >> 7) & 0xFFu;
                    atomicAdd(&h[e >> 2], 1u << (8 * (e & 3u)));
                    e_lo = min(e_lo, int(e));
                    e_hi = max(e_hi, int(e));
                }
            }
            atomicMin(&lohi[own], e_lo);
            atomicMax(&lohi[nthr + own], e_hi);
        }
        __syncthreads();
        if (slice == 0 && has) {
            const int e_lo = lohi[own], e_hi = lohi[nthr + own];
            auto count = [&](int b) { return int((h[b >> 2] >> (8 * (b & 3))) & 0xFFu); };
            for (int wi = 0; wi < nwin; ++wi) {
                const int bi = wi == 0 ? 0 : (wi == 1 && nwin == 2 ? 2 : wi); // 2-, (3-,) 4-bit
                const int width = (4 << bi) - 1; // codes 0..2^bits-2
                const int lo = min(max(0, e_lo - width + 1), 256 - width);
                const int hi = min(e_hi, 256 - width);
                int cov = 0;
                for (int b = lo; b < lo + width; ++b) cov += count(b);
                int best = cov, best_base = lo;
                for (int b = lo + 1; b <= hi; ++b) {
                    cov += count(b + width - 1) - count(b - 1);
                    if (cov > best) {
                        best = cov;
                        best_base = b;
                    }
                }
                bases[size_t(bi) * size_t(dim) + size_t(d)] = uint8_t(best_base);
                esc[bi] += n - best;
            }
        }
        __syncthreads(); // the columns are cleared again for the next channels
    }
    // escape counts of the whole block
    for (int o = 32; o > 0; o >>= 1) {
#pragma unroll
        for (int bi = 0; bi < 3; ++bi) esc[bi] += __shfl_xor(esc[bi], o);
    }
    const int w = tid >> 6, nw = int(blockDim.x) >> 6;
    if ((tid & 63) == 0) {
#pragma unroll
        for (int bi = 0; bi < 3; ++bi) esc_part[3 * w + bi] = esc[bi];
    }
    __syncthreads();
    if (tid == 0) {
        int cand_esc[3] = {0, 0, 0};
        for (int i = 0; i < nw; ++i) {
#pragma unroll
            for (int bi = 0; bi < 3; ++bi) cand_esc[bi] += esc_part[3 * i + bi];
        }
        // codec.cpp:94-103: raw, then the coded modes by width; replace when
        // smaller, or on a tie when the best is not raw and has more escapes
        // (or equal escapes and more bits). With the 3-bit mode this is the
        // order of the reference's sizer (analyze_exponents.py:142-143:
        // smaller, then raw, then fewer escapes, then narrower codes).
        int best_mode = 0, best_esc = 0;
        int64_t best_bytes = block_bytes(0, n, 0, dim);
#pragma unroll
        for (int bi = 0; bi < 3; ++bi) {
            const int mode = bi + 2;
            if (!(modes & (1 << mode)) || (mode == 3 && nwin < 3)) continue;
            const int64_t by = block_bytes(mode, n, cand_esc[bi], dim);
            const bool smaller = by < best_bytes;
            const bool tie_win = by == best_bytes && best_mode != 0 &&
                                 (cand_esc[bi] < best_esc || (cand_esc[bi] == best_esc && mode < best_mode));
            if (smaller || tie_win) {
                best_mode = mode;
                best_bytes = by;
                best_esc = cand_esc[bi];
            }
        }
        EncBlockMeta m;
        m.bytes = best_bytes;
        m.mode = best_mode;
        m.n_escape = best_esc;
        *meta = m;
    }
}



__global__ __launch_bounds__(kThreads) void encode_stats_kernel(const uint16_t *__restrict__ kv, int seq, int dim,
                                                               int bt, EncBlockMeta *__restrict__ meta,
                                                               uint8_t *__restrict__ bases, int modes) {
    const int b = int(blockIdx.x);
    const int t0 = b * bt;
    const EncRows src{kv + size_t(t0) * size_t(dim), kv + size_t(t0) * size_t(dim), 0};
    extern __shared__ uint32_t stats_lds[];
    encode_stats_block(stats_lds, reinterpret_cast<int *>(stats_lds + stats_cols(dim) * kHistStride), src,
                       min(bt, seq - t0), dim, meta + b, bases + size_t(b) * 3 * size_t(dim), modes);
}

__global__ __launch_bounds__(kThreads) void append_stats_kernel(const AppendJobDev *__restrict__ jobs, int n_jobs,
                                                               int dim, int bt, EncBlockMeta *__restrict__ meta,
                                                               uint8_t *__restrict__ bases, int modes) {
    const int g = int(blockIdx.x);
    const AppendJobDev j = jobs[find_job(jobs, n_jobs, g)];
    const int b = g - j.blk0;
    extern __shared__ uint32_t stats_lds[];
    encode_stats_block(stats_lds, reinterpret_cast<int *>(stats_lds + stats_cols(dim) * kHistStride),
                       job_rows(j, b, bt, dim), min(bt, j.seq - b * bt), dim, meta + g,
                       bases + size_t(g) * 3 * size_t(dim), modes);
}

// ------------------------------------------------------------- encode: scan --
// offs[i] = base + sum of block sizes before block i (n_blocks + 1 entries);
// first[i] = tok0 + i * bt, first[n_blocks] = tok0 + seq. base is offs[0] as
// found on entry when `rebase` is set (an append continues the container at
// its trailing block), else 0.
struct ScanLds {
    long long wave_tot[16];
    long long carry;
};

__device__ __forceinline__ void encode_scan_body(ScanLds &L, const EncBlockMeta *__restrict__ meta, int n_blocks,
                                                 int bt, int seq, int64_t *__restrict__ offs,
                                                 int32_t *__restrict__ first, int rebase, int tok0) {
    auto &wave_tot = L.wave_tot;
    auto &carry_s = L.carry;
    const int tid = int(threadIdx.x);
    const int lane = lane_id();
    const int w = tid >> 6;
    if (tid == 0) carry_s = rebase ? offs[0] : 0;
    __syncthreads();
    for (int r = 0; r < n_blocks; r += 1024) {
        const int i = r + tid;
        long long v = i < n_blocks ? meta[i].bytes : 0;
        long long incl = v;
        for (int o = 1; o < kWave; o <<= 1) {
            const long long y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
        }
        if (lane == kWave - 1) wave_tot[w] = incl;
        __syncthreads();
        long long base = carry_s;
        long long tot = 0;
        for (int k = 0; k < 16; ++k) {
            base += (k < w) ? wave_tot[k] : 0;
            tot += wave_tot[k];
        }
        if (i < n_blocks) {
            offs[i] = base + incl - v;
            first[i] = tok0 + i * bt;
        }
        __syncthreads();
        if (tid == 0) carry_s += tot;
        __syncthreads();
    }
    if (tid == 0) {
        offs[n_blocks] = carry_s;
        first[n_blocks] = tok0 + seq;
    }
}

__global__ __launch_bounds__(1024) void encode_scan_kernel(const EncBlockMeta *__restrict__ meta, int n_blocks,
                                                          int bt, int seq, int64_t *__restrict__ offs,
                                                          int32_t *__restrict__ first, int rebase, int tok0) {
    __shared__ ScanLds L;
    encode_scan_body(L, meta, n_blocks, bt, seq, offs, first, rebase, tok0);
}

// One workgroup per append job.
__global__ __launch_bounds__(1024) void append_scan_kernel(const AppendJobDev *__restrict__ jobs,
                                                          const EncBlockMeta *__restrict__ meta, int bt) {
    const AppendJobDev j = jobs[blockIdx.x];
    __shared__ ScanLds L;
    encode_scan_body(L, meta + j.blk0, j.nb, bt, j.seq, j.offs, j.first, j.rebase, j.tok0);
}

// ------------------------------------------------------------ encode: write --
// One block: `p` is its place in the container, `bases3` its window bases
// [3][dim] (2-, 3-, 4-bit).
__device__ __forceinline__ void encode_write_block(int *scan_tmp, const EncRows src, int n, int dim,
                                                   const EncBlockMeta m, const uint8_t *__restrict__ bases3,
                                                   uint8_t *__restrict__ p, uint32_t *__restrict__ status) {
    const int total = n * dim;
    if (threadIdx.x == 0) {
        p[0] = uint8_t(m.mode);
        p[1] = uint8_t(n);
        const int ne = m.mode == 0 ? 0 : m.n_escape;
        p[2] = uint8_t(ne & 0xFF);
        p[3] = uint8_t(ne >> 8);
        p[4] = uint8_t(dim & 0xFF);
        p[5] = uint8_t(dim >> 8);
        p[6] = 0;
        p[7] = 0;
    }
    p += 8;
    if (m.mode == 0) {
        for (int i = int(threadIdx.x); i < total; i += kThreads) {
            const uint32_t h = src.at(i);
            p[2 * i] = uint8_t(h & 0xFF);
            p[2 * i + 1] = uint8_t(h >> 8);
        }
        return;
    }
    const int mode = m.mode;
    const int U = code_unit(mode); // elements per thread and step: 4, or 8 for 3-bit codes (3 bytes)
    const int width = (1 << mode) - 1;
    const uint8_t *bsrc = bases3 + size_t(mode - 2) * size_t(dim);
    for (int d = int(threadIdx.x); d < dim; d += kThreads) p[d] = bsrc[d];
    uint8_t *sm = p + dim;
    uint8_t *codes = sm + size_t(total);
    uint8_t *esc = codes + exp_payload_bytes(n, dim, mode);
    const int units = total / U;
    int carry = 0;
    for (int r = 0; r < units; r += kThreads) {
        const int u = r + int(threadIdx.x);
        const bool act = u < units;
        uint32_t cw = 0;
        int cnt = 0;
        if (act) {
            const int e0 = U * u;
            const int d0 = e0 % dim;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (k >= U) break;
                const uint32_t h = src.at(e0 + k);
                sm[e0 + k] = uint8_t(((h >> 8) & 0x80u) | (h & 0x7Fu));
                const int delta = int((h >> 7) & 0xFFu) - int(bsrc[d0 + k]);
                uint32_t c = uint32_t(width);
                if (delta >= 0 && delta < width) c = uint32_t(delta);
                else ++cnt;
                cw |= c << (mode * k);
            }
            if (mode == 4) {
                codes[2 * u] = uint8_t(cw);
                codes[2 * u + 1] = uint8_t(cw >> 8);
            } else if (mode == 2) {
                codes[u] = uint8_t(cw);
            } else {
                codes[3 * u] = uint8_t(cw);
                codes[3 * u + 1] = uint8_t(cw >> 8);
                codes[3 * u + 2] = uint8_t(cw >> 16);
            }
        }
        int tot = 0;
        int rank = carry + block_excl_scan<kWaves>(cnt, scan_tmp, &tot);
        carry += tot;
        if (act && cnt) {
            const int e0 = U * u;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (k >= U) break;
                if (unit_code(cw, mode, k) == uint32_t(width)) {
                    const uint32_t h = src.at(e0 + k);
                    if (rank < m.n_escape) {
                        esc[2 * rank] = uint8_t(h & 0xFF);
                        esc[2 * rank + 1] = uint8_t(h >> 8);
                    }
                    ++rank;
                }
            }
        }
    }
    if (threadIdx.x == 0 && carry != m.n_escape) atomicOr(status, kStEscape);
}

__global__ __launch_bounds__(kThreads) void encode_write_kernel(const uint16_t *__restrict__ kv, int seq, int dim,
                                                               int bt, const EncBlockMeta *__restrict__ meta,
                                                               const uint8_t *__restrict__ bases,
                                                               const int64_t *__restrict__ offs,
                                                               uint8_t *__restrict__ out,
                                                               uint32_t *__restrict__ status) {
    const int b = int(blockIdx.x);
    const int t0 = b * bt;
    const EncRows src{kv + size_t(t0) * size_t(dim), kv + size_t(t0) * size_t(dim), 0};
    __shared__ int scan_tmp[kWaves];
    encode_write_block(scan_tmp, src, min(bt, seq - t0), dim, meta[b], bases + size_t(b) * 3 * size_t(dim),
                       out + offs[b], status);
}

__global__ __launch_bounds__(kThreads) void append_write_kernel(const AppendJobDev *__restrict__ jobs, int n_jobs,
                                                               int dim, int bt, const EncBlockMeta *__restrict__ meta,
                                                               const uint8_t *__restrict__ bases,
                                                               uint32_t *__restrict__ status) {
    const int g = int(blockIdx.x);
    const AppendJobDev j = jobs[find_job(jobs, n_jobs, g)];
    const int b = g - j.blk0;
    __shared__ int scan_tmp[kWaves];
    encode_write_block(scan_tmp, job_rows(j, b, bt, dim), min(bt, j.seq - b * bt), dim, meta[g],
                       bases + size_t(g) * 3 * size_t(dim), j.out + j.offs[b], status);
}

// The raw rows of each job's new trailing partial block that are not in
// its tail buffer yet, copied there (after the write kernel has read it).
__global__ __launch_bounds__(kThreads) void append_tail_kernel(const AppendJobDev *__restrict__ jobs, int dim) {
    const AppendJobDev j = jobs[blockIdx.x];
    const int total = j.copy_rows * dim;
    const uint16_t *from = j.src + size_t(j.copy_from) * size_t(dim);
    uint16_t *to = j.tail + size_t(j.copy_to) * size_t(dim);
    for (int i = int(threadIdx.x); i < total; i += kThreads) to[i] = from[i];
}

// Append jobs that encode one block each (a decode step: the trailing block
// plus one token never exceeds a block), fused in one launch: one workgroup
// (kThreads) per job computes the block's statistics, its place (the
// container's trailing-block offset, which no other job touches), writes it
// and the index entries around it, then stores the raw rows kept for the
// next append (rows the block did not read from the tail).
__global__ __launch_bounds__(kThreads) void append_one_kernel(const AppendJobDev *__restrict__ jobs, int dim,
                                                             int bt, uint32_t *__restrict__ status, int modes) {
    extern __shared__ uint32_t one_lds[]; // stats columns, escape sums, then the three window bases
    __shared__ EncBlockMeta meta_s;
    __shared__ int scan_tmp[kWaves];
    const AppendJobDev j = jobs[blockIdx.x];
    int *esc_part = reinterpret_cast<int *>(one_lds + stats_cols(dim) * kHistStride);
    uint8_t *bases_s = reinterpret_cast<uint8_t *>(esc_part + 3 * kWaves + 2 * stats_cols(dim));
    const int64_t base = j.rebase ? j.offs[0] : 0;
    if (j.nb == 0) { // an empty container: its terminal index entry
        if (threadIdx.x == 0) {
            j.offs[0] = base;
            j.first[0] = j.tok0;
        }
        return;
    }
    const EncRows rows = job_rows(j, 0, bt, dim);
    encode_stats_block(one_lds, esc_part, rows, j.seq, dim, &meta_s, bases_s, modes);
    __syncthreads();
    const EncBlockMeta m = meta_s;
    if (threadIdx.x == 0) {
        j.offs[0] = base;
        j.offs[1] = base + m.bytes;
        j.first[0] = j.tok0;
        j.first[1] = j.tok0 + j.seq;
    }
    encode_write_block(scan_tmp, rows, j.seq, dim, m, bases_s, j.out + base, status);
    __syncthreads();
    const int total = j.copy_rows * dim;
    const uint16_t *from = j.src + size_t(j.copy_from) * size_t(dim);
    uint16_t *to = j.tail + size_t(j.copy_to) * size_t(dim);
    for (int i = int(threadIdx.x); i < total; i += kThreads) to[i] = from[i];
}

// ------------------------------------------------------------ escape records --
// The escape record (element index | word << 16, kvexp_types.h) of every
// escape of a coded block (mode 2, 3 or 4) whose `total` codes start at
// `codes`, written to rec[0 .. n_escape): the i-th sentinel in scan order
// takes the i-th escape word, which the format stores after the codes; a
// sentinel count other than n_escape raises kStEscape. All threads of the
// workgroup call it.
__device__ __forceinline__ void escape_positions(const uint8_t *codes, int mode, int total, int n_escape,
                                                 uint32_t *__restrict__ pos, int *scan_tmp,
                                                 uint32_t *__restrict__ status) {
    const uint8_t *words = codes + (total * mode + 7) / 8;
    const int U = code_unit(mode);
    const uint32_t sentinel = (1u << mode) - 1u;
    const int units = total / U;
    int carry = 0;
    for (int r = 0; r < units; r += kThreads) {
        const int u = r + int(threadIdx.x);
        const bool act = u < units;
        uint32_t cw = 0;
        int cnt = 0;
        if (act) {
            cw = load_codes(codes, mode, u);
            cnt = unit_sentinels(cw, mode);
        }
        int tot = 0;
        int rank = carry + block_excl_scan<kWaves>(cnt, scan_tmp, &tot);
        carry += tot;
        if (act && cnt) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (k >= U) break;
                if (unit_code(cw, mode, k) == sentinel) {
                    if (rank < n_escape) {
                        const uint32_t w = uint32_t(words[2 * rank]) | (uint32_t(words[2 * rank + 1]) << 8);
                        pos[rank] = uint32_t(U * u + k) | (w << 16);
                    }
                    ++rank;
                }
            }
        }
    }
    if (threadIdx.x == 0 && carry != n_escape) atomicOr(status, kStEscape);
}

// esc0[b] = escape words in blocks before b (raw blocks count 0), one
// workgroup per tensor. With j.first set, every block is also checked against
// the index (header inside the container, head_dim, n_tokens equal to the
// index's token count, known mode, payload inside the container); with
// j.desc set (and j.pos allocated), its descriptor is written.
__global__ __launch_bounds__(kThreads) void esc_start_kernel(const EscJob *__restrict__ jobs,
                                                            uint32_t *__restrict__ status) {
    __shared__ int scan_tmp[kWaves];
    const EscJob j = jobs[blockIdx.x];
    int carry = 0;
    for (int r = 0; r < j.n_blocks; r += kThreads) {
        const int b = r + int(threadIdx.x);
        int ne = 0;
        BlockHdr h{};
        uint32_t st = 0;
        int64_t off = 0;
        if (b < j.n_blocks) {
            off = j.offs[b];
            if (j.first != nullptr) {
                st = check_block(j.blob, j.bytes, off, j.dim, j.first[b + 1] - j.first[b], &h);
            } else if (off >= 0 && uint64_t(off) + 8u <= j.bytes) {
                h = read_hdr(j.blob + off);
            } else {
                st = kStHeader;
            }
            if (st != 0u) atomicOr(status, st);
            else ne = h.mode == 0 ? 0 : h.n_escape;
        }
        int tot = 0;
        const int excl = block_excl_scan<kWaves>(ne, scan_tmp, &tot);
        if (b < j.n_blocks) {
            j.esc0[b] = carry + excl;
            if (j.desc != nullptr) {
                BlockDesc d{};
                d.data = j.blob + off;
                d.esc = j.pos + (carry + excl);
                d.meta = st != 0u ? 0u : uint32_t(h.mode) | (uint32_t(h.n_tokens) << 8) | (uint32_t(ne) << 16);
                j.desc[b] = d;
            }
        }
        carry += tot;
    }
    if (threadIdx.x == 0) j.esc0[j.n_blocks] = carry;
}

// Element index of every escape of one block (one workgroup per block;
// `blocks` lists (job, block) pairs).
__global__ __launch_bounds__(kThreads) void esc_pos_kernel(const EscJob *__restrict__ jobs,
                                                          const int2 *__restrict__ blocks,
                                                          uint32_t *__restrict__ status) {
    __shared__ int scan_tmp[kWaves];
    const int2 jb = blocks[blockIdx.x];
    const EscJob j = jobs[jb.x];
    const int b = jb.y;
    const int dim = j.dim;
    const int64_t off = j.offs[b];
    if (off < 0 || uint64_t(off) + 8u > j.bytes) return;
    const BlockHdr h = read_hdr(j.blob + off);
    if (h.mode == 0 || h.n_escape == 0) return;
    const int64_t sz = block_bytes(h.mode, h.n_tokens, h.n_escape, dim);
    if (sz < 0 || h.dim != dim || uint64_t(off) + uint64_t(sz) > j.bytes) {
        if (threadIdx.x == 0) atomicOr(status, kStTruncated);
        return;
    }
    const uint8_t *codes = j.blob + off + 8 + dim + size_t(h.n_tokens) * size_t(dim);
    escape_positions(codes, h.mode, h.n_tokens * dim, h.n_escape, j.pos + j.esc0[b], scan_tmp, status);
}

// Plan update after appends. Workgroups [0, n_jobs), one per tensor: the
// last block is checked against the index again and its descriptor and
// escape records are rewritten (blocks before it are unchanged by an
// append); the entry after it becomes a zero-token sentinel (a split kernel
// that reached it would stop there), and an index that ends before the
// attended tokens raises kStIndex. The workgroups after them set each device
// head's length and byte counts and the end of each head's last split from
// the jobs (tensors 2h and 2h + 1 are the K and V of head h, which owns
// device heads [h * per_head, (h + 1) * per_head)).
__global__ __launch_bounds__(kThreads) void plan_refresh_kernel(const EscJob *__restrict__ jobs, int n_jobs,
                                                               HeadDev *__restrict__ heads, int n_dev_heads,
                                                               WorkItem *__restrict__ items, int n_items,
                                                               int per_head, uint32_t *__restrict__ status) {
    __shared__ int scan_tmp[kWaves];
    __shared__ int ok_s;
    if (int(blockIdx.x) >= n_jobs) {
        const int i = (int(blockIdx.x) - n_jobs) * kThreads + int(threadIdx.x);
        if (i < n_dev_heads) {
            const int h = i / per_head;
            heads[i].seq = jobs[2 * h].seq;
            heads[i].kbytes = jobs[2 * h].bytes;
            heads[i].vbytes = jobs[2 * h + 1].bytes;
        }
        if (i < n_items) {
            WorkItem &w = items[i];
            const int h = w.head / per_head;
            if (w.split == heads[w.head].n_splits - 1) w.tok_end = jobs[2 * h].seq;
        }
        return;
    }
    const EscJob j = jobs[blockIdx.x];
    const int b = j.n_blocks - 1;
    const int dim = j.dim;
    const int64_t off = j.offs[b];
    const int e0 = j.esc0[b];
    if (threadIdx.x == 0) {
        BlockHdr h{};
        uint32_t st = check_block(j.blob, j.bytes, off, dim, j.first[b + 1] - j.first[b], &h);
        const int ne = st != 0u || h.mode == 0 ? 0 : h.n_escape;
        if (st == 0u && e0 + ne > j.pos_cap) st = kStEscape;
        if (j.first[j.n_blocks] < j.seq) st |= kStIndex;
        BlockDesc d{};
        d.data = j.blob + off;
        d.esc = j.pos + e0;
        d.meta = st != 0u ? 0u : uint32_t(h.mode) | (uint32_t(h.n_tokens) << 8) | (uint32_t(ne) << 16);
        j.desc[b] = d;
        BlockDesc z{};
        z.data = j.blob;
        z.esc = j.pos;
        j.desc[b + 1] = z;
        j.esc0[b + 1] = e0 + ne;
        if (st != 0u) atomicOr(status, st);
        ok_s = st == 0u && ne > 0;
    }
    __syncthreads();
    if (!ok_s) return;
    const BlockHdr h = read_hdr(j.blob + off);
    const uint8_t *codes = j.blob + off + 8 + dim + size_t(h.n_tokens) * size_t(dim);
    escape_positions(codes, h.mode, h.n_tokens * dim, h.n_escape, j.pos + e0, scan_tmp, status);
}

// y = expf(x) in the forms the attention kernels evaluate it (all must equal
// glibc): thread % 3 == 0 the branching special cases with the constant-memory
// table, 1 the branch-free form with the table copied to LDS, 2 the
// non-positive form for x <= 0, +0 and NaN (the branch-free form otherwise).
__global__ __launch_bounds__(256) void expf_kernel(const float *__restrict__ x, float *__restrict__ y, size_t n) {
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 32) tab[threadIdx.x] = kvexp_exp2_32_table[threadIdx.x];
    __syncthreads();
    const size_t i = size_t(blockIdx.x) * 256u + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    const uint32_t b = __float_as_uint(v);
    const int form = int(threadIdx.x % 3u);
    if (form == 0) y[i] = kvexp_expf(v);
    else if (form == 2 && ((b >> 31) != 0u || b == 0u || v != v)) y[i] = kvexp_expf_nonpos_nb(v, tab);
    else y[i] = kvexp_expf_tab_nb(v, tab);
}

} // namespace kvexp_dev

// ---------------------------------------------------------------- launchers --
namespace kvexp_launch {
using namespace kvexp_dev;

hipError_t decode(const uint8_t *blob, uint64_t bytes, const int64_t *offs, const int32_t *first, int n_blocks,
                  int seq, int dim, uint16_t *out, uint32_t *status, hipStream_t s) {
    if (n_blocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(decode_blocks_kernel, dim3(n_blocks), dim3(kThreads), 0, s, blob, bytes, offs, first, seq,
                       dim, out, status);
    return hipGetLastError();
}

hipError_t encode(const uint16_t *kv, int seq, int dim, int bt, int n_blocks, EncBlockMeta *meta, uint8_t *bases,
                  int64_t *offs, int32_t *first, uint8_t *out, uint32_t *status, hipStream_t s, bool rebase,
                  int tok0, int modes) {
    hipLaunchKernelGGL(encode_stats_kernel, dim3(n_blocks), dim3(kThreads), stats_lds_bytes(dim), s, kv, seq,
                       dim, bt, meta, bases, modes);
    hipLaunchKernelGGL(encode_scan_kernel, dim3(1), dim3(1024), 0, s, meta, n_blocks, bt, seq, offs, first,
                       rebase ? 1 : 0, tok0);
    hipLaunchKernelGGL(encode_write_kernel, dim3(n_blocks), dim3(kThreads), 0, s, kv, seq, dim, bt, meta, bases,
                       offs, out, status);
    return hipGetLastError();
}

hipError_t append(const AppendJobDev *jobs, int n_jobs, int total_blocks, int dim, int bt, EncBlockMeta *meta,
                  uint8_t *bases, uint32_t *status, hipStream_t s, bool one_block, int modes) {
    if (n_jobs <= 0) return hipSuccess;
    if (one_block) {
        const size_t lds = stats_lds_bytes(dim) + 3 * size_t(dim);
        hipLaunchKernelGGL(append_one_kernel, dim3(n_jobs), dim3(kThreads), lds, s, jobs, dim, bt, status, modes);
        return hipGetLastError();
    }
    if (total_blocks > 0)
        hipLaunchKernelGGL(append_stats_kernel, dim3(total_blocks), dim3(kThreads), stats_lds_bytes(dim), s,
                           jobs, n_jobs, dim, bt, meta, bases, modes);
    hipLaunchKernelGGL(append_scan_kernel, dim3(n_jobs), dim3(1024), 0, s, jobs, meta, bt);
    if (total_blocks > 0)
        hipLaunchKernelGGL(append_write_kernel, dim3(total_blocks), dim3(kThreads), 0, s, jobs, n_jobs, dim, bt, meta,
                           bases, status);
    hipLaunchKernelGGL(append_tail_kernel, dim3(n_jobs), dim3(kThreads), 0, s, jobs, dim);
    return hipGetLastError();
}

hipError_t esc_start(const EscJob *jobs, int n_jobs, uint32_t *status, hipStream_t s) {
    if (n_jobs <= 0) return hipSuccess;
    hipLaunchKernelGGL(esc_start_kernel, dim3(n_jobs), dim3(kThreads), 0, s, jobs, status);
    return hipGetLastError();
}

hipError_t plan_refresh(const EscJob *jobs, int n_jobs, HeadDev *heads, int n_dev_heads, WorkItem *items,
                        int n_items, int per_head, uint32_t *status, hipStream_t s) {
    const int extra = (std::max(n_dev_heads, n_items) + kThreads - 1) / kThreads;
    if (n_jobs + extra <= 0) return hipSuccess;
    hipLaunchKernelGGL(plan_refresh_kernel, dim3(n_jobs + extra), dim3(kThreads), 0, s, jobs, n_jobs, heads,
                       n_dev_heads, items, n_items, per_head, status);
    return hipGetLastError();
}

hipError_t esc_pos(const EscJob *jobs, const int2 *blocks, int n_blocks, uint32_t *status, hipStream_t s) {
    if (n_blocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(esc_pos_kernel, dim3(n_blocks), dim3(kThreads), 0, s, jobs, blocks, status);
    return hipGetLastError();
}

// ---------------------------------------------------- no-alloc scratch --
// Device scratch of the no-allocation encoder entry point: a file-scope array
// (each GPU the library runs on holds its own copy until the process ends),
// addressed from the host only through the per-device pointer that
// hipGetSymbolAddress returns (the array's name in host code is not a device
// address). Calls that overlap on one GPU share it and race.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxScratchDevices] = {};
} // namespace

// Looks the array up on `device` (which must be current) once; later calls
// return the stored pointer.
hipError_t noalloc_scratch_setup(int device, void **ptr) {
    *ptr = nullptr;
    if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[device] == nullptr) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[device] = p;
    }
    *ptr = g_scratch_ptr[device];
    return hipSuccess;
}

void *noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxScratchDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return g_scratch_ptr[device];
}

hipError_t expf(const float *x, float *y, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(expf_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, x, y, n);
    return hipGetLastError();
}

} // namespace kvexp_launch
