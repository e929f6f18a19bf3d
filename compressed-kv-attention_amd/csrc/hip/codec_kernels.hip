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

// The block's mode from the escape counts of the 2-, 3- and 4-bit windows
// (codec.cpp:94-103): raw, then the coded modes by width; replace when
// smaller, or on a tie when the best is not raw and has more escapes (or
// equal escapes and more bits). With the 3-bit mode this is the order of the
// reference's sizer (analyze_exponents.py:142-143: smaller, then raw, then
// fewer escapes, then narrower codes).
__device__ __forceinline__ EncBlockMeta choose_mode(const int (&cand_esc)[3], int n, int dim, int modes, int nwin) {
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
    return m;
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
        *meta = choose_mode(cand_esc, n, dim, modes, nwin);
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
// With `terminal` set (after the fused encoder, which writes the index of
// the jobs with blocks), also the index entry of an empty container.
__global__ __launch_bounds__(kThreads) void append_tail_kernel(const AppendJobDev *__restrict__ jobs, int dim,
                                                              int terminal) {
    const AppendJobDev j = jobs[blockIdx.x];
    if (terminal && j.nb == 0 && threadIdx.x == 0) {
        j.offs[0] = j.rebase ? j.offs[0] : 0;
        j.first[0] = j.tok0;
    }
    const int total = j.copy_rows * dim;
    const uint16_t *from = j.src + size_t(j.copy_from) * size_t(dim);
    uint16_t *to = j.tail + size_t(j.copy_to) * size_t(dim);
    for (int i = int(threadIdx.x); i < total; i += kThreads) to[i] = from[i];
}

// ------------------------------------------------ encode: one fused pass --
// Statistics, place and bytes of every block in one launch, reading the
// tokens once (the three launches above read them twice). The grid is
// [P] x [jobs], P workgroups per job, as many as stay resident together (at
// most the longest job's block count); a workgroup takes its job's
// (blockIdx.y) blocks one at a time from the job's ticket counter, so every
// earlier block of the job has already been taken by a running workgroup
// (which finishes its current block first and then that one). It draws its
// next ticket as soon as it starts a block and, once the ticket is back
// (after the histograms), issues the next block's token loads, so that
// neither round trip stands on a block's path but the first one's. It stops
// at its first ticket past the job's blocks (the one that draws the job's
// last ticket, number n_blocks + P - 1, resets the counter). A block: it
// holds the block's tokens in
// registers (chunks of 8 elements of one row, 16 bytes, NL chunks per
// thread), counts each channel's exponents into LDS byte counters, slides the
// code windows (one (window, channel) pair per thread, so that every wave
// works), chooses the mode, and finds its place in the container by a
// decoupled look-back over the sizes of its job's earlier blocks: each block
// publishes its own size as soon as its mode is known, and the job-relative
// end of its bytes once its place is known; wave 0 reads up to 64 earlier
// entries at a time and sums back to the nearest end, after the block's codes
// and escape ranks are computed (so that the earlier blocks have had that
// long to publish). Then the block is written from the registers.
// head_dim % 8 == 0, at most kFusedMaxElems elements per block, sources
// 16-byte aligned (the host checks; otherwise it uses the three launches).
//
// Look-back state: one ticket counter per job (reset to 0 by the workgroup
// that takes the job's last ticket) and, in an array of its own, one entry
// per block of the launch (the job's first block at jobs[i].blk0): bits
// 63..48 the launch's epoch (1..65535, so entries of earlier launches never
// match), 47..46 the kind (1: the block's size, 2: the job-relative end of
// the block), 45..0 the value. The host clears the entries when the epoch
// wraps and when the array is new, and the counters when their array is new.
constexpr uint32_t kLookbackPolls = 1u << 20; // ~1 s of polling, then kStLookback

// Phase trace of the one-pass encoder (builds with KVEXP_PHASE_TRACE only;
// build.py --trace, read by bench.py --phase-trace): per block of a launch, wave 0's
// clock at the start, after the ticket, the job, the tokens' arrival, the
// histograms, the mode, the escape ranks, the look-back and the end; then
// the look-back's polls, the CU that ran it and the workgroup's blockIdx.x.
#if defined(KVEXP_PHASE_TRACE)
constexpr int kEncTraceBlocks = 32768, kEncTraceWords = 12;
__device__ unsigned long long g_enc_trace[kEncTraceBlocks * kEncTraceWords];
#define KVEXP_ENC_MARK(i) (enc_tr[i] = __builtin_readcyclecounter())
#else
#define KVEXP_ENC_MARK(i) ((void)0)
#endif
constexpr uint64_t kLbValueMask = (uint64_t(1) << 46) - 1u;

__device__ __forceinline__ uint64_t lb_word(uint32_t epoch, uint32_t kind, uint64_t value) {
    return (uint64_t(epoch) << 48) | (uint64_t(kind) << 46) | (value & kLbValueMask);
}

__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4_t g_cu32x4; // 16-byte global loads

// Exclusive prefix over the workgroup, in chunk order (chunk k * kThreads +
// thread), of the sentinel counts packed two to a 32-bit word (16 bits
// each: at most 8 per chunk, 2048 per chunk row of the workgroup, so no
// field carries into the next). tmp: [kWaves][NP] words in LDS. Leaves in
// excl[q] the thread's exclusive prefix within each chunk row and in
// total[q] the rows' totals (field k % 2 of word k / 2 for chunk row k);
// EscRanks::rank gives a chunk's first rank.
template <int NL>
struct EscRanks {
    static constexpr int NP = (NL + 1) / 2;
    uint32_t excl[NP], total[NP];
    __device__ __forceinline__ int field(const uint32_t (&a)[NP], int k) const {
        return int((a[k / 2] >> (16 * (k % 2))) & 0xFFFFu);
    }
    __device__ __forceinline__ int rank(int k) const {
        int carry = 0;
#pragma unroll
        for (int i = 0; i < NL; ++i)
            if (i < k) carry += field(total, i);
        return carry + field(excl, k);
    }
    __device__ __forceinline__ int sum() const {
        int t = 0;
#pragma unroll
        for (int i = 0; i < NL; ++i) t += field(total, i);
        return t;
    }
};

template <int NL>
__device__ __forceinline__ EscRanks<NL> fused_escape_ranks(const uint32_t (&v)[EscRanks<NL>::NP], uint32_t *tmp) {
    constexpr int NP = EscRanks<NL>::NP;
    const int lane = lane_id(), w = int(threadIdx.x) >> 6;
    EscRanks<NL> r;
    uint32_t incl[NP];
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        incl[q] = uint32_t(wave_scan_add(int(v[q])));
        if (lane == kWave - 1) tmp[w * NP + q] = incl[q];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NP; ++q) {
        uint32_t before = 0, total = 0;
#pragma unroll
        for (int x = 0; x < kWaves; ++x) {
            const uint32_t t = tmp[x * NP + q];
            before += x < w ? t : 0;
            total += t;
        }
        r.excl[q] = before + incl[q] - v[q];
        r.total[q] = total;
    }
    return r;
}

// Waves per SIMD the one-pass encoder is compiled for (its registers fit
// 512 / waves without spilling): 8 with up to four chunk rows per thread.
template <int NL>
constexpr int kFusedWaves = NL <= 4 ? 8 : 4;
// Fewest waves per SIMD the compiler may plan for. Up to two chunk rows per
// thread, one block's tokens fit in registers beside the next block's (NL
// 16-byte loads each) at eight waves; at four rows the next block's tokens
// are loaded only once this block's are dead (kFusedNextEarly), which keeps
// the kernel at 64 registers and eight waves (eight workgroups per CU: the
// c2 prefill 2.6 % faster than six with both sets in registers). At NL 8 the
// budget stays at four (128 registers): three would let a head_dim-128
// tensor's 1,024 blocks fill only 768 workgroups at once.
template <int NL>
constexpr int kFusedWavesMin = NL <= 4 ? 8 : 4;
// Whether the next block's tokens are loaded right after the histograms
// (beside this block's) or only once this block's bytes are staged.
template <int NL>
constexpr bool kFusedNextEarly = NL <= 2;

// Dynamic LDS of the one-pass encoder: the histogram columns, or the
// largest block (raw: header + 2 bytes per element) staged for its copy,
// whichever is larger. At most 66,560 bytes (head_dim 256, 64-token blocks).
__host__ __device__ constexpr size_t fused_lds_bytes(int dim, int bt) {
    const size_t hist = size_t(dim) * kHistStride * sizeof(uint32_t);
    const size_t raw = (8u + 2u * size_t(bt) * size_t(dim) + 15u) & ~size_t(15);
    return hist > raw ? hist : raw;
}

// JOBS: the jobs are in device memory (appends); else the one job is a
// kernel argument (an encode), read from the argument segment.
template <int NL, bool JOBS>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kFusedWavesMin<NL>, kFusedWaves<NL>))) void
encode_fused_kernel(const AppendJobDev *__restrict__ jobs, AppendJobDev one, int dim, int bt, int modes,
                    uint64_t *__restrict__ state, uint32_t *__restrict__ tickets, uint32_t epoch,
                    uint32_t *__restrict__ status) {
    // dynamic LDS: the exponent byte counters [dim][kHistStride], then the
    // block's bytes staged for the copy to the container (fused_lds_bytes)
    extern __shared__ __align__(16) uint32_t fz_lds[];
    uint32_t *fz_hist = fz_lds;
    uint8_t *stage = reinterpret_cast<uint8_t *>(fz_lds);
    __shared__ uint32_t s_ticket, s_next;
    __shared__ int s_lo[kWaves], s_hi[kWaves], s_esc[kWaves][3];
    __shared__ __align__(16) uint8_t s_base[3][kMaxDim]; // window bases of the 2-, 3- and 4-bit codes
    __shared__ uint16_t s_key[3 * kMaxDim];               // best (coverage, base) of the upper half of each range
    __shared__ uint32_t s_scan[kWaves * EscRanks<NL>::NP];
    __shared__ long long s_excl;
    const int tid = int(threadIdx.x), lane = lane_id(), w = tid >> 6;
    const int jx = int(blockIdx.y);
    uint32_t polls = 0; // look-back reads that found a nearer block unpublished
#if defined(KVEXP_PHASE_TRACE)
    unsigned long long enc_tr[9];
#endif

    // ---- first ticket while the job loads; every workgroup of the job's
    // grid row draws tickets until one lies past the job's blocks, so the
    // job's draws number n_blocks + P, and the one that draws the last
    // resets the counter
    const AppendJobDev j = JOBS ? jobs[jx] : one;
    // a job with no more blocks than workgroups: one ticket each, no
    // prefetch (the job's draws number P)
    const bool one_shot = gridDim.x >= uint32_t(j.nb);
    const uint32_t last_draw = (one_shot ? 0u : uint32_t(j.nb)) + gridDim.x - 1u;
    if (tid == 0) {
        const uint32_t t = atomicAdd(tickets + jx, 1u);
        if (t == last_draw) atomicExch(tickets + jx, 0u);
        s_ticket = t;
    }
    // first channel of chunk c (8 * (c mod dim / 8); the float quotient is
    // exact to far below its distance from an integer, c < 4096)
    const int cpr = dim / 8;
    const float inv_cpr = __builtin_amdgcn_rcpf(float(cpr));
    auto chunk_d0 = [&](int c) {
        const int row = int((float(c) + 0.5f) * inv_cpr);
        return 8 * (c - row * cpr);
    };
    // the tokens of block bb into registers: chunks of 8 elements of one
    // row, NL per thread, all loads in flight together (chunks past the
    // block read chunk 0)
    auto load_tokens = [&](int bb, u32x4_t (&dst)[NL]) {
        const EncRows sr = job_rows(j, bb, bt, dim);
        const int nch = min(bt, j.seq - bb * bt) * dim / 8, spl = sr.split / 8;
#pragma unroll
        for (int k = 0; k < NL; ++k) {
            const int c = k * kThreads + tid < nch ? k * kThreads + tid : 0;
            const uint16_t *p = c < spl ? sr.a + 8 * size_t(c) : sr.b + 8 * size_t(c - spl);
            dst[k] = *(g_cu32x4 *)(p);
        }
    };
    __syncthreads();
    u32x4_t x[NL], xn[NL];
    int b = int(s_ticket);
    if (b < j.nb) load_tokens(b, x);
#pragma unroll 1
    while (true) {
        // the thread index through an empty asm, so that the addresses made
        // from it are made again in each block rather than hoisted out of the
        // loop and held in registers across it
        const int tid = [] {
            int t = int(threadIdx.x);
            asm volatile("" : "+v"(t));
            return t;
        }();
        const int lane = tid & (kWave - 1), w = tid >> 6;
        if (b >= j.nb) { // past the job's blocks (or a counter not left at 0: then nothing of the job runs)
            if (tid == 0 && uint32_t(b) > last_draw) atomicOr(status, kStLookback);
            return;
        }
        KVEXP_ENC_MARK(0);
        // the next ticket, consumed after the histograms
        uint32_t tn = uint32_t(j.nb);
        if (tid == 0 && !one_shot) tn = atomicAdd(tickets + jx, 1u);
        // (dim * kHistStride is a multiple of 8: 16-byte stores)
#pragma unroll 1
        for (int i = 4 * tid; i < dim * kHistStride; i += 4 * kThreads)
            *reinterpret_cast<uint4 *>(fz_hist + i) = make_uint4(0u, 0u, 0u, 0u);
        __syncthreads();
        polls = 0;
        const int g = j.blk0 + b; // look-back entry of the block
        KVEXP_ENC_MARK(1);
        const int n = min(bt, j.seq - b * bt);
#if defined(KVEXP_PHASE_TRACE)
        asm volatile("" ::"v"(n));
#endif
        KVEXP_ENC_MARK(2);
        const int chunks = n * dim / 8;

        // ---- channel histograms of the block's tokens (in registers)
        // exponent fields (bits 14..7 of each BF16) of the thread's elements,
        // smallest and largest, both halves at once (v_pk_min_u16 /
        // v_pk_max_u16); 0xFFFF: no element
        typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
        u16x2_t lo2 = {0xFFFF, 0xFFFF}, hi2 = {0, 0};
#if defined(KVEXP_PHASE_TRACE)
        asm volatile("" ::"v"(x[NL - 1][0]), "v"(x[0][0]));
#endif
        KVEXP_ENC_MARK(3);
        // Lanes that share a chunk column (the rows of one chunk position) count
        // their 8 elements in an order rotated by the row (step h takes element
        // (h + row) % 8), so that the 64 lanes of an LDS add hit different
        // channel columns rather than 8 lanes one counter.
#pragma unroll
        for (int k = 0; k < NL; ++k) {
            const int c = k * kThreads + tid;
            if (c < chunks) {
                const int row = int((float(c) + 0.5f) * inv_cpr);
                const int rot = row & 7;
                uint32_t *col = fz_hist + 8 * (c - row * cpr) * kHistStride;
                // the chunk rotated right by 16 * rot bits: element h of v is element (h + rot) % 8
                u32x4_t v = x[k];
                if (rot & 4) v = u32x4_t{v[2], v[3], v[0], v[1]};
                if (rot & 2) v = u32x4_t{v[1], v[2], v[3], v[0]};
                if (rot & 1)
                    v = u32x4_t{__builtin_amdgcn_alignbit(v[1], v[0], 16), __builtin_amdgcn_alignbit(v[2], v[1], 16),
                                __builtin_amdgcn_alignbit(v[3], v[2], 16), __builtin_amdgcn_alignbit(v[0], v[3], 16)};
#pragma unroll
                for (int h = 0; h < 8; ++h) {
                    const uint32_t e = (v[h >> 1] >> (16 * (h & 1) + 7)) & 0xFFu;
                    atomicAdd(col + ((h + rot) & 7) * kHistStride + int(e >> 2), 1u << (8u * (e & 3u)));
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const u16x2_t ef = __builtin_bit_cast(u16x2_t, x[k][i] & 0x7F807F80u);
                    lo2 = __builtin_elementwise_min(lo2, ef);
                    hi2 = __builtin_elementwise_max(hi2, ef);
                }
            }
        }
        const uint32_t pk_lo = min(uint32_t(lo2.x), uint32_t(lo2.y)), pk_hi = max(uint32_t(hi2.x), uint32_t(hi2.y));
        const int e_lo = wave_min_i32(pk_lo == 0xFFFFu ? 255 : int(pk_lo >> 7));
        const int e_hi = wave_max_i32(int(pk_hi >> 7));
        if (lane == 0) {
            s_lo[w] = e_lo;
            s_hi[w] = e_hi;
        }
        if (tid == 0) {
            if (!one_shot && tn == last_draw) atomicExch(tickets + jx, 0u);
            s_next = tn;
        }
        __syncthreads();
        KVEXP_ENC_MARK(4);
        int blk_lo = 255, blk_hi = 0;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) {
            blk_lo = min(blk_lo, s_lo[i]);
            blk_hi = max(blk_hi, s_hi[i]);
        }
        // the next block's tokens, in flight while this block is encoded (at
        // NL 8 once this block's are dead, before the look-back: two sets
        // would not fit the 128 registers of four waves per SIMD)
        const int bn = int(s_next);
        if constexpr (kFusedNextEarly<NL>) {
            if (bn < j.nb) load_tokens(bn, xn);
        }

        // ---- best_base of each (window, channel) (codec.cpp:18-35): the most
        // covered exponents, then the smallest base; bases outside
        // [blk_lo - width + 1, blk_hi] cover nothing. Each range is split in two
        // halves taken by different waves (tasks [0, pairs) the lower halves,
        // [pairs, 2 pairs) the upper); a half's best is the key
        // coverage * 256 + 255 - base, so the larger key is the better base.
        const int nwin = (modes & 8) ? 3 : 2;
        const int pairs = nwin * dim;
        int key_lo[3] = {0, 0, 0}; // this thread's lower-half results (tasks tid, tid + 256, tid + 512)
#pragma unroll
        for (int r = 0; r < 6; ++r) {
            const int t = tid + r * kThreads;
            if (t >= 2 * pairs) break;
            const int half = int(t >= pairs);
            const int pt = t - half * pairs;
            const int wi = int(pt >= dim) + int(pt >= 2 * dim);
            const int d = pt - wi * dim;
            const int bi = wi == 0 ? 0 : (nwin == 2 ? 2 : wi);
            const int width = (4 << bi) - 1;
            const int lo0 = min(max(0, blk_lo - width + 1), 256 - width);
            const int hi0 = min(blk_hi, 256 - width);
            const int mid = (lo0 + hi0 + 1) >> 1;
            const int lo = half ? mid : lo0, hi = half ? hi0 : mid - 1;
            int key = 0;
            if (lo <= hi) {
                const uint8_t *hb = reinterpret_cast<const uint8_t *>(fz_hist + d * kHistStride);
                // the first window's coverage: the byte counters of bins [lo,
                // lo + width) summed a word (four bins) at a time with
                // v_sad_u8, the bins outside masked off (lo is the same in
                // every lane of the wave, so is the loop)
                int cov = 0;
                {
                    const uint32_t *hw = fz_hist + d * kHistStride;
                    const int w0 = lo >> 2, w1 = (lo + width - 1) >> 2;
                    const uint32_t m0 = 0xFFFFFFFFu << (8 * (lo & 3));
                    const uint32_t m1 = 0xFFFFFFFFu >> (8 * (3 - ((lo + width - 1) & 3)));
                    uint32_t acc = 0;
                    for (int wi = w0; wi <= w1; ++wi) {
                        uint32_t m = 0xFFFFFFFFu;
                        if (wi == w0) m &= m0;
                        if (wi == w1) m &= m1;
                        acc = __builtin_amdgcn_sad_u8(hw[wi] & m, 0u, acc);
                    }
                    cov = int(acc);
                }
                int best = cov, best_b = lo;
#pragma unroll 4
                for (int base = lo + 1; base <= hi; ++base) {
                    cov += int(hb[base + width - 1]) - int(hb[base - 1]);
                    if (cov > best) {
                        best = cov;
                        best_b = base;
                    }
                }
                key = best * 256 + 255 - best_b;
            }
            if (half) s_key[pt] = uint16_t(key);
            else if (r < 3) key_lo[r] = key;
        }
        __syncthreads();
        int esc[3] = {0, 0, 0};
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            const int pt = tid + r * kThreads;
            if (pt >= pairs) break;
            const int wi = int(pt >= dim) + int(pt >= 2 * dim);
            const int d = pt - wi * dim;
            const int bi = wi == 0 ? 0 : (nwin == 2 ? 2 : wi);
            const int key = max(key_lo[r], int(s_key[pt]));
            s_base[bi][d] = uint8_t(255 - (key & 255));
            esc[bi] += n - (key >> 8);
        }
#pragma unroll
        for (int bi = 0; bi < 3; ++bi) esc[bi] = wave_sum_i32(esc[bi]);
        if (lane == 0) {
#pragma unroll
            for (int bi = 0; bi < 3; ++bi) s_esc[w][bi] = esc[bi];
        }
        __syncthreads();
        int cand[3] = {0, 0, 0};
#pragma unroll
        for (int i = 0; i < kWaves; ++i) {
#pragma unroll
            for (int bi = 0; bi < 3; ++bi) cand[bi] += s_esc[i][bi];
        }
        const EncBlockMeta m = choose_mode(cand, n, dim, modes, nwin);
        KVEXP_ENC_MARK(5);

        // ---- publish the size
        if (tid == 0)
            __hip_atomic_store(state + g, lb_word(epoch, b == 0 ? 2u : 1u, uint64_t(m.bytes)), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);

        // ---- codes and sentinel counts
        const int mode = m.mode;
        const uint32_t width = (1u << mode) - 1u;
        uint32_t cw[NL];
        uint32_t cnt_pk[EscRanks<NL>::NP] = {}; // sentinels per chunk, 16 bits each
#pragma unroll
        for (int k = 0; k < NL; ++k) {
            cw[k] = 0u;
            if (mode != 0 && k * kThreads + tid < chunks) {
                int cnt = 0;
                const uint2 bb = *reinterpret_cast<const uint2 *>(&s_base[mode - 2][chunk_d0(k * kThreads + tid)]);
#pragma unroll
                for (int h = 0; h < 8; ++h) {
                    const uint32_t e = (x[k][h >> 1] >> (16 * (h & 1) + 7)) & 0xFFu;
                    const uint32_t base = ((h < 4 ? bb.x : bb.y) >> (8 * (h & 3))) & 0xFFu;
                    const uint32_t delta = e - base; // wraps when e < base
                    const bool hit = delta < width;
                    cw[k] |= (hit ? delta : width) << (mode * h);
                    cnt += hit ? 0 : 1;
                }
                cnt_pk[k / 2] |= uint32_t(cnt) << (16 * (k % 2));
            }
        }
        // the escape ranks; the barrier in it also ends every read of the
        // histograms, whose LDS now takes the staged block
        const EscRanks<NL> er = fused_escape_ranks<NL>(cnt_pk, s_scan);
        KVEXP_ENC_MARK(6);

        // ---- the block's bytes, staged in LDS in their final order
        if (tid < 8) {
            const int ne = mode == 0 ? 0 : m.n_escape;
            const uint32_t hdr[8] = {uint32_t(mode), uint32_t(n), uint32_t(ne & 0xFF), uint32_t(ne >> 8),
                                     uint32_t(dim & 0xFF), uint32_t(dim >> 8), 0u, 0u};
            stage[tid] = uint8_t(hdr[tid]);
        }
        uint8_t *body = stage + 8;
        if (mode == 0) {
#pragma unroll
            for (int k = 0; k < NL; ++k) {
                const int c = k * kThreads + tid;
                typedef u32x4_t __attribute__((aligned(8))) u32x4_a8;
                if (c < chunks) *reinterpret_cast<u32x4_a8 *>(body + 16 * c) = x[k]; // 8 + 16c: 8-byte aligned
            }
        } else {
            if (2 * tid < dim) // dim <= 256 = kThreads: one pair of bases per thread
                *reinterpret_cast<uint16_t *>(body + 2 * tid) =
                    *reinterpret_cast<const uint16_t *>(&s_base[mode - 2][2 * tid]);
            uint8_t *sm = body + dim;
            uint8_t *codes = sm + n * dim;
            uint8_t *escw = codes + exp_payload_bytes(n, dim, mode);
#pragma unroll
            for (int k = 0; k < NL; ++k) {
                const int c = k * kThreads + tid;
                if (c >= chunks) continue;
                // sign and mantissa bytes of the 8 elements: (h >> 8 & 0x80) | (h & 0x7F)
                uint32_t s4[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t mm = x[k][i] & 0x807F807Fu;
                    s4[i] = mm | (mm >> 8); // bytes 0 and 2 hold the two elements' sm bytes
                }
                u32x2_t smv;
                smv.x = __builtin_amdgcn_perm(s4[1], s4[0], 0x06040200u);
                smv.y = __builtin_amdgcn_perm(s4[3], s4[2], 0x06040200u);
                *reinterpret_cast<u32x2_t *>(sm + 8 * c) = smv; // 8 + dim + 8c: 8-byte aligned
                if (mode == 4) {
                    *reinterpret_cast<uint32_t *>(codes + 4 * c) = cw[k];
                } else if (mode == 2) {
                    *reinterpret_cast<uint16_t *>(codes + 2 * c) = uint16_t(cw[k]);
                } else {
                    uint8_t *q = codes + 3 * c;
                    q[0] = uint8_t(cw[k]);
                    q[1] = uint8_t(cw[k] >> 8);
                    q[2] = uint8_t(cw[k] >> 16);
                }
                if (((cnt_pk[k / 2] >> (16 * (k % 2))) & 0xFFFFu) != 0) {
                    int r = er.rank(k);
#pragma unroll
                    for (int h = 0; h < 8; ++h) {
                        if (((cw[k] >> (mode * h)) & width) == width) {
                            if (r < m.n_escape) { // escape words may sit at odd offsets (3-bit codes): bytes
                                const uint32_t v = x[k][h >> 1] >> (16 * (h & 1));
                                escw[2 * r] = uint8_t(v);
                                escw[2 * r + 1] = uint8_t(v >> 8);
                            }
                            ++r;
                        }
                    }
                }
            }
        }

        if constexpr (!kFusedNextEarly<NL>) {
            if (bn < j.nb) load_tokens(bn, x);
        }

        // ---- wave 0 finds the block's place while the others wait at the barrier
        if (w == 0) {
            int64_t excl = 0;
            if (b > 0) {
                int pos = g - 1;
                auto lb_read = [&]() -> uint64_t {
                    const int idx = pos - lane;
                    return idx >= j.blk0 ? __hip_atomic_load(state + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                         : 0u;
                };
                uint64_t wv = lb_read();
                while (true) {
                    const bool in = pos - lane >= j.blk0;
                    const uint32_t kind = in && uint32_t(wv >> 48) == epoch ? uint32_t(wv >> 46) & 3u : 0u;
                    const uint64_t ends = __ballot(in && kind == 2u);
                    const uint64_t open = __ballot(in && kind == 0u);
                    const int fe = ends ? __ffsll((unsigned long long)ends) - 1 : kWave;
                    const int fo = open ? __ffsll((unsigned long long)open) - 1 : kWave;
                    if (fo < fe) { // a nearer block has not published its size yet
                        if (++polls > kLookbackPolls) {
                            if (lane == 0) atomicOr(status, kStLookback);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(2);
                        wv = lb_read();
                        continue;
                    }
                    excl += wave_sum_i64(in && lane <= fe ? int64_t(wv & kLbValueMask) : 0);
                    if (fe < kWave) break;
                    pos -= kWave;
                    wv = lb_read();
                }
                if (lane == 0)
                    __hip_atomic_store(state + g, lb_word(epoch, 2u, uint64_t(excl + m.bytes)), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
            if (lane == 0) s_excl = excl;
        }
        __syncthreads();
        KVEXP_ENC_MARK(7);

        // ---- the staged bytes to the container: 16-byte aligned stores, the
        // bytes before the first aligned address and after the last one alone
        const int64_t off = (j.rebase ? j.offs[0] : 0) + s_excl;
        uint8_t *p = j.out + off;
        const int nbytes = int(m.bytes);
        const int head = min(nbytes, int((16u - (uint32_t(reinterpret_cast<uintptr_t>(p)) & 15u)) & 15u));
        const int n16 = (nbytes - head) >> 4;
        const int tail0 = head + 16 * n16;
        for (int i = tid; i < n16; i += kThreads) {
            typedef const u32x4_t __attribute__((aligned(1))) u32x4_a1;
            *(__attribute__((address_space(1))) u32x4_t *)(p + head + 16 * i) =
                *reinterpret_cast<u32x4_a1 *>(stage + head + 16 * i);
        }
        if (tid < head) p[tid] = stage[tid];
        else if (tid >= 16 && tid - 16 < nbytes - tail0) p[tail0 + tid - 16] = stage[tail0 + tid - 16];
        if (tid == 0) {
            j.offs[b] = off;
            j.first[b] = j.tok0 + b * bt;
            if (b == j.nb - 1) {
                j.offs[b + 1] = off + m.bytes;
                j.first[b + 1] = j.tok0 + j.seq;
            }
            if (er.sum() != (mode == 0 ? 0 : m.n_escape)) atomicOr(status, kStEscape);
        }
#if defined(KVEXP_PHASE_TRACE)
        KVEXP_ENC_MARK(8);
        if (w == 0 && lane == 0 && g < kEncTraceBlocks) {
            unsigned long long *o = g_enc_trace + size_t(g) * kEncTraceWords;
            for (int i = 0; i < 9; ++i) o[i] = enc_tr[i];
            o[9] = polls;
            o[10] = (unsigned long long)__smid();
            o[11] = (unsigned long long)blockIdx.x; // the workgroup that encoded the block
        }
#endif
        if (one_shot) return;
        // the next block; the barrier at its start also ends every read of this
        // block's staged bytes before the histograms reuse their LDS
        b = bn;
        if constexpr (kFusedNextEarly<NL>) {
#pragma unroll
            for (int k = 0; k < NL; ++k) x[k] = xn[k];
        }
        __syncthreads();
    }
}

#if defined(KVEXP_PHASE_TRACE)
} // namespace kvexp_dev
extern "C" int kvexp_hip_encode_trace_read(unsigned long long *host, size_t n) {
    return int(hipMemcpyFromSymbol(host, HIP_SYMBOL(kvexp_dev::g_enc_trace), n * 8));
}
namespace kvexp_dev {
#endif

// Clears the first nw look-back entries and nt ticket counters of the fused
// encoder in one launch (a kernel, not a memset, so that a captured graph
// replays it).
__global__ __launch_bounds__(256) void clear_lookback_kernel(uint64_t *__restrict__ words, size_t nw,
                                                             uint32_t *__restrict__ tickets, size_t nt) {
    const size_t i = size_t(blockIdx.x) * 256u + threadIdx.x;
    if (i < nw) words[i] = 0u;
    if (i < nt) tickets[i] = 0u;
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
// table, 1 the branch-free form with the table copied to LDS (as the wave
// kernels copy it: from immediates), 2 the non-positive form for x <= 0, +0
// and NaN (the branch-free form otherwise).
__global__ __launch_bounds__(256) void expf_kernel(const float *__restrict__ x, float *__restrict__ y, size_t n) {
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 64) kvexp_exp_table_to_lds(tab);
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

bool encode_fused_supported(int dim, int bt) {
    return dim >= 8 && dim % 8 == 0 && dim <= kMaxDim && bt >= 1 && int64_t(bt) * dim <= kFusedMaxElems;
}

namespace {
template <int NL, bool JOBS>
hipError_t launch_fused_j(const AppendJobDev *jobs, int n_jobs, const AppendJobDev &one, int max_job_blocks, int dim,
                          int bt, int modes, const EncLookback &lb, uint32_t *status, hipStream_t s) {
    // head_dim 256 needs 66,560 bytes of histogram columns, past the default
    // 64 KiB of dynamic LDS (set once per instantiation)
    static const hipError_t configured =
        hipFuncSetAttribute(reinterpret_cast<const void *>(encode_fused_kernel<NL, JOBS>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, int(fused_lds_bytes(kMaxDim, 64)));
    if (configured != hipSuccess) return configured;
    const size_t lds = fused_lds_bytes(dim, bt);
    // P workgroups per job: as many as are resident together over all jobs
    // (each loops over its job's blocks), at most the longest job's blocks
    int dev = 0, cus = 0, per_cu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void *>(encode_fused_kernel<NL, JOBS>), kThreads, lds);
    if (e != hipSuccess) return e;
    const int64_t resident = std::max<int64_t>(1, int64_t(cus) * std::max(per_cu, 1));
    const int per_job = int(std::max<int64_t>(1, std::min<int64_t>(max_job_blocks, resident / std::max(n_jobs, 1))));
    hipLaunchKernelGGL((encode_fused_kernel<NL, JOBS>), dim3(unsigned(per_job), unsigned(n_jobs)),
                       dim3(kThreads), lds, s, jobs, one, dim, bt, modes, lb.words, lb.tickets, lb.epoch, status);
    return hipGetLastError();
}

template <int NL>
hipError_t launch_fused(const AppendJobDev *jobs, int n_jobs, const AppendJobDev &one, int max_job_blocks, int dim,
                        int bt, int modes, const EncLookback &lb, uint32_t *status, hipStream_t s) {
    return jobs != nullptr
               ? launch_fused_j<NL, true>(jobs, n_jobs, one, max_job_blocks, dim, bt, modes, lb, status, s)
               : launch_fused_j<NL, false>(jobs, n_jobs, one, max_job_blocks, dim, bt, modes, lb, status, s);
}

// The fused encoder over the blocks of `jobs` (device; n_jobs of them, the
// longest with max_job_blocks blocks), or of the one job `one` when jobs is
// null (n_jobs 1).
hipError_t encode_fused(const AppendJobDev *jobs, int n_jobs, const AppendJobDev &one, int max_job_blocks, int dim,
                        int bt, int modes, const EncLookback &lb, uint32_t *status, hipStream_t s) {
    const size_t nclear = std::max(lb.clear_words, lb.clear_tickets);
    if (nclear > 0)
        hipLaunchKernelGGL(clear_lookback_kernel, dim3(unsigned((nclear + 255) / 256)), dim3(256), 0, s, lb.words,
                           lb.clear_words, lb.tickets, lb.clear_tickets);
    const int chunks = (bt * dim) / 8;
    if (chunks <= kThreads) return launch_fused<1>(jobs, n_jobs, one, max_job_blocks, dim, bt, modes, lb, status, s);
    if (chunks <= 2 * kThreads)
        return launch_fused<2>(jobs, n_jobs, one, max_job_blocks, dim, bt, modes, lb, status, s);
    if (chunks <= 4 * kThreads)
        return launch_fused<4>(jobs, n_jobs, one, max_job_blocks, dim, bt, modes, lb, status, s);
    return launch_fused<8>(jobs, n_jobs, one, max_job_blocks, dim, bt, modes, lb, status, s);
}
} // namespace

hipError_t encode(const uint16_t *kv, int seq, int dim, int bt, int n_blocks, EncBlockMeta *meta, uint8_t *bases,
                  int64_t *offs, int32_t *first, uint8_t *out, uint32_t *status, hipStream_t s, bool rebase,
                  int tok0, int modes, const EncLookback *lb) {
    if (lb != nullptr) { // one pass (the caller checked encode_fused_supported and the alignment)
        AppendJobDev one{};
        one.src = kv;
        one.offs = offs;
        one.first = first;
        one.out = out;
        one.seq = seq;
        one.tok0 = tok0;
        one.nb = n_blocks;
        one.rebase = rebase ? 1 : 0;
        return encode_fused(nullptr, 1, one, n_blocks, dim, bt, modes, *lb, status, s);
    }
    hipLaunchKernelGGL(encode_stats_kernel, dim3(n_blocks), dim3(kThreads), stats_lds_bytes(dim), s, kv, seq,
                       dim, bt, meta, bases, modes);
    hipLaunchKernelGGL(encode_scan_kernel, dim3(1), dim3(1024), 0, s, meta, n_blocks, bt, seq, offs, first,
                       rebase ? 1 : 0, tok0);
    hipLaunchKernelGGL(encode_write_kernel, dim3(n_blocks), dim3(kThreads), 0, s, kv, seq, dim, bt, meta, bases,
                       offs, out, status);
    return hipGetLastError();
}

hipError_t append(const AppendJobDev *jobs, int n_jobs, int total_blocks, int dim, int bt, EncBlockMeta *meta,
                  uint8_t *bases, uint32_t *status, hipStream_t s, bool one_block, int modes, const EncLookback *lb,
                  int max_job_blocks) {
    if (n_jobs <= 0) return hipSuccess;
    if (one_block) {
        const size_t lds = stats_lds_bytes(dim) + 3 * size_t(dim);
        hipLaunchKernelGGL(append_one_kernel, dim3(n_jobs), dim3(kThreads), lds, s, jobs, dim, bt, status, modes);
        return hipGetLastError();
    }
    if (lb != nullptr) { // one pass, then the tails (and the index of empty containers)
        if (total_blocks > 0) {
            const hipError_t e =
                encode_fused(jobs, n_jobs, AppendJobDev{}, max_job_blocks, dim, bt, modes, *lb, status, s);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(append_tail_kernel, dim3(n_jobs), dim3(kThreads), 0, s, jobs, dim, 1);
        return hipGetLastError();
    }
    if (total_blocks > 0)
        hipLaunchKernelGGL(append_stats_kernel, dim3(total_blocks), dim3(kThreads), stats_lds_bytes(dim), s,
                           jobs, n_jobs, dim, bt, meta, bases, modes);
    hipLaunchKernelGGL(append_scan_kernel, dim3(n_jobs), dim3(1024), 0, s, jobs, meta, bt);
    if (total_blocks > 0)
        hipLaunchKernelGGL(append_write_kernel, dim3(total_blocks), dim3(kThreads), 0, s, jobs, n_jobs, dim, bt, meta,
                           bases, status);
    hipLaunchKernelGGL(append_tail_kernel, dim3(n_jobs), dim3(kThreads), 0, s, jobs, dim, 0);
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
