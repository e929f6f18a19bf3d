// gfx950 fused decode attention over raw BF16 or XKV containers.
//
// One workgroup (4 wave64) per work item = one split [tok_begin, tok_end) of
// one KV head, processed in chunks of up to 64 tokens that never cross a K or
// V block boundary. Per chunk:
//   1. the four waves decode the chunk's K and V rows into FP32 LDS tiles
//      (XKV: sign/mantissa + base + residual code, escapes ranked by a
//      workgroup prefix sum; raw: BF16 widened). These tiles are the only
//      place decoded values exist; HBM holds only the container bytes.
//   2. wave w owns query rows g = w and g = w + 4. With lane = token it
//      computes the scores in the reference order, the running maximum (a
//      DPP prefix max, exact), alpha = exp(m_prev - m) and e = exp(s - m)
//      with the glibc-identical expf.
//   3. with lane = channel it folds the chunk's tokens in order into
//      acc = fma(e, v, acc * alpha) and l = fma(l, alpha, e).
// The per-split (m, l, acc) is written to the workspace (or finalised
// directly when the head has one split); merge_kernel folds the splits of a
// head left to right exactly as dispatch.cpp:98-103 and finalises
// out = acc * (1/l).
//
// The arithmetic of every query row is the reference's per-thread range
// (attention_scalar.cpp:19-85 / attention_avx512.cpp:114-196, softmax.hpp:8-41)
// operation for operation, so for the same split the output equals the
// reference's bit for bit, and the raw and XKV instantiations (which differ
// only in how the LDS tiles are filled) equal each other bit for bit.
#include "kvexp_device.h"
#include "kvexp_types.h"

namespace kvexp_dev {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = 4;
constexpr int kChunk = 64;
constexpr int kMaxQ = 8; // query rows per head in one launch (more are split into heads of <= 8)

// LDS layout of one workgroup (floats). Row stride DM + 4 keeps the per-lane
// 16-byte row reads of phase 2 free of bank conflicts.
template <int DPL>
struct AttnLds {
    static constexpr int DM = DPL * 64;
    static constexpr int RS = DM + 4;
    float k[kChunk * RS];
    float v[kChunk * RS];
    float q[kMaxQ * DM];
    float e[kMaxQ][kChunk];
    float a[kMaxQ][kChunk];
    int scan_tmp[kAttnWaves];
};

// ----------------------------------------------------- chunk decode to LDS --
// Rows [r0, r0 + n) of the block at `blk` (XKV) into tile rows 0..n-1.
// `esc_carry` is the number of escape words of this block consumed by rows
// before r0; it is advanced by this chunk's sentinels. Called by all threads.
template <int DPL>
__device__ __forceinline__ void xkv_rows_to_lds(const uint8_t *blk, const BlockHdr &h, int dim, int r0, int n,
                                                float *tile, int *esc_carry, int *scan_tmp, uint32_t *bad) {
    constexpr int RS = AttnLds<DPL>::RS;
    const uint8_t *p = blk + 8;
    const int octets = (n * dim) >> 3; // dim % 8 == 0
    if (h.mode == 0) {
        const uint8_t *raw = p + 2 * size_t(r0) * size_t(dim);
        for (int o = int(threadIdx.x); o < octets; o += kAttnThreads) {
            const int e = o * 8;
            const int row = e / dim, col = e - row * dim;
            float *dst = tile + row * RS + col;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t w = load_u32_any(raw + 2 * size_t(e) + 4 * k);
                dst[2 * k] = bits_f32(w << 16);
                dst[2 * k + 1] = bits_f32(w & 0xFFFF0000u);
            }
        }
        return;
    }
    const int mode = h.mode; // 2, 3 or 4 code bits
    const uint32_t sentinel = (1u << mode) - 1u;
    const uint8_t *base = p;
    const uint8_t *sm = p + dim;
    const uint8_t *codes = sm + size_t(h.n_tokens) * size_t(dim);
    const uint8_t *escp = codes + exp_payload_bytes(h.n_tokens, dim, h.mode);
    const size_t e_first = size_t(r0) * size_t(dim);
    int carry = *esc_carry;
    for (int r = 0; r < octets; r += kAttnThreads) {
        const int o = r + int(threadIdx.x);
        const bool act = o < octets;
        uint32_t s0 = 0, s1 = 0, cw = 0;
        int cnt = 0;
        const size_t e = e_first + size_t(o) * 8u;
        if (act) {
            s0 = load_u32_any(sm + e);
            s1 = load_u32_any(sm + e + 4);
            // the octet's codes: 4, 3 or 2 bytes
            cw = mode == 4 ? load_u32_any(codes + (e >> 1))
                           : (mode == 2 ? load_u16_any(codes + (e >> 2)) : load_codes(codes, 3, int(e >> 3)));
            cnt = mode == 4 ? sentinels4(cw) : (mode == 2 ? sentinels2(cw) : sentinels3(cw));
        }
        int rank = carry;
        if (h.n_escape > 0) {
            int tot = 0;
            rank += block_excl_scan<kAttnWaves>(cnt, scan_tmp, &tot);
            carry += tot;
        }
        if (act) {
            const int le = o * 8;
            const int row = le / dim, col = le - row * dim;
            const uint32_t b0 = load_u32_any(base + col), b1 = load_u32_any(base + col + 4);
            float f[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t code = unit_code(cw, mode, k);
                const uint32_t smk = ((k < 4 ? s0 : s1) >> (8 * (k & 3))) & 0xFFu;
                const uint32_t bk = ((k < 4 ? b0 : b1) >> (8 * (k & 3))) & 0xFFu;
                uint32_t bf;
                if (code == sentinel) {
                    if (rank < h.n_escape) {
                        bf = load_u16_any(escp + 2 * size_t(rank));
                    } else {
                        bf = 0;
                        *bad |= kStEscape;
                    }
                    ++rank;
                } else {
                    bf = bf16_join(bk + code, smk);
                }
                f[k] = bf16_f32(bf);
            }
            float4 *dst = reinterpret_cast<float4 *>(tile + row * RS + col);
            dst[0] = make_float4(f[0], f[1], f[2], f[3]);
            dst[1] = make_float4(f[4], f[5], f[6], f[7]);
        }
    }
    *esc_carry = carry;
}

// Raw [seq, dim] rows [t, t + n) into tile rows 0..n-1.
template <int DPL>
__device__ __forceinline__ void raw_rows_to_lds(const uint16_t *src, int dim, int t, int n, float *tile) {
    constexpr int RS = AttnLds<DPL>::RS;
    const uint8_t *raw = reinterpret_cast<const uint8_t *>(src + size_t(t) * size_t(dim));
    const int octets = (n * dim) >> 3;
    for (int o = int(threadIdx.x); o < octets; o += kAttnThreads) {
        const int e = o * 8;
        const int row = e / dim, col = e - row * dim;
        float *dst = tile + row * RS + col;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t w = load_u32_any(raw + 2 * size_t(e) + 4 * k);
            dst[2 * k] = bits_f32(w << 16);
            dst[2 * k + 1] = bits_f32(w & 0xFFFF0000u);
        }
    }
}

// ------------------------------------------------------------------ scores --
// attention_scalar.cpp:13-29: lane[j] = fma(q[d+j], k[d+j], lane[j]) for
// d = 0, 8, ..., then ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)).
__device__ __forceinline__ float tree8(const float *c) {
    const float a = (c[0] + c[4]) + (c[1] + c[5]);
    const float b = (c[2] + c[6]) + (c[3] + c[7]);
    return a + b;
}

// VDPBF16PS treats denormal inputs as zero and flushes denormal results.
__device__ __forceinline__ float daz(float x) {
    return (fabsf(x) < 1.17549435e-38f) ? copysignf(0.0f, x) : x;
}

// attention_avx512.cpp:21-30,116-124 with the SDM's VDPBF16PS step: per
// 32-element step, lane j (0..15) does acc += k[2j+1]*q[2j+1] then
// acc += k[2j]*q[2j], each one rounding (RNE), inputs DAZ, result FTZ; then
// a pairwise tree over the 16 lanes. q here is already DAZ-flushed.
__device__ __forceinline__ float tree16(const float *t) {
    const float a0 = (t[0] + t[1]) + (t[2] + t[3]);
    const float a1 = (t[4] + t[5]) + (t[6] + t[7]);
    const float a2 = (t[8] + t[9]) + (t[10] + t[11]);
    const float a3 = (t[12] + t[13]) + (t[14] + t[15]);
    return (a0 + a1) + (a2 + a3);
}

template <int ORDER, bool TWO>
__device__ __forceinline__ void chunk_scores(const float *krow, const float *q0, const float *q1, int dim, float *s0,
                                             float *s1) {
    if (ORDER == 0) {
        float c0[8], c1[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) c0[j] = c1[j] = 0.0f;
        for (int d = 0; d < dim; d += 8) {
            const float4 ka = *reinterpret_cast<const float4 *>(krow + d);
            const float4 kb = *reinterpret_cast<const float4 *>(krow + d + 4);
            const float k8[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) c0[j] = fmaf(q0[d + j], k8[j], c0[j]);
            if (TWO) {
#pragma unroll
                for (int j = 0; j < 8; ++j) c1[j] = fmaf(q1[d + j], k8[j], c1[j]);
            }
        }
        *s0 = tree8(c0);
        if (TWO) *s1 = tree8(c1);
    } else {
        float t0[16], t1[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) t0[j] = t1[j] = 0.0f;
        for (int d = 0; d < dim; d += 32) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float ke = daz(krow[d + 2 * j]), ko = daz(krow[d + 2 * j + 1]);
                t0[j] = daz(fmaf(ko, q0[d + 2 * j + 1], daz(t0[j])));
                t0[j] = daz(fmaf(ke, q0[d + 2 * j], t0[j]));
                if (TWO) {
                    t1[j] = daz(fmaf(ko, q1[d + 2 * j + 1], daz(t1[j])));
                    t1[j] = daz(fmaf(ke, q1[d + 2 * j], t1[j]));
                }
            }
        }
        *s0 = tree16(t0);
        if (TWO) *s1 = tree16(t1);
    }
}

// softmax_coeff (softmax.hpp:8-14) for the 64 tokens of a chunk at once:
// m_t = max(m_{t-1}, s_t) as an exact prefix maximum, alpha_t = exp(m_{t-1} - m_t),
// e_t = exp(s_t - m_t). Returns whether any valid token has alpha != 1.
__device__ __forceinline__ bool chunk_softmax(float s, int n, float *m_run, float *e_out, float *a_out) {
    const int lane = lane_id();
    const float mi = fmaxf(wave_scan_max(s), *m_run);
    const float mp = wave_shift_up(mi, *m_run);
    const float alpha = kvexp_expf(mp - mi);
    const float e = kvexp_expf(s - mi);
    e_out[lane] = e;
    a_out[lane] = alpha;
    *m_run = readlane_f32(mi, n - 1);
    return __ballot(lane < n && !(alpha == 1.0f)) != 0;
}

// Partial-state slot of one split: m[8], l[8], acc[8][dim] floats.
__host__ __device__ __forceinline__ size_t slot_floats(int dim) { return size_t(kMaxQ) * size_t(dim + 2); }

// Finalises one query row (head with a single split: out = acc * (1/l),
// finalize_state, softmax.hpp:32-41) or stores its partial state in the
// head's slot for this split.
template <int DPL>
__device__ __forceinline__ void store_row(const HeadDev &hd, const WorkItem &wi, int g, float m, float l,
                                          const float (&acc)[DPL], int dim, int lane, float *out_all,
                                          float *lse_all, float *ws) {
    if (hd.n_splits == 1) {
        float *o = out_all + (size_t(hd.q_row) + size_t(g)) * size_t(dim);
        const float inv = 1.0f / l;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
            const int d = lane + 64 * j;
            if (d < dim) o[d] = acc[j] * inv;
        }
        if (lse_all != nullptr && lane == 0) lse_all[hd.q_row + g] = m + logf(l);
        return;
    }
    float *slot = ws + size_t(hd.ws_base + wi.split) * slot_floats(dim);
    if (lane == 0) {
        slot[g] = m;
        slot[kMaxQ + g] = l;
    }
    float *a = slot + 2 * kMaxQ + g * dim;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
        const int d = lane + 64 * j;
        if (d < dim) a[d] = acc[j];
    }
}

// --------------------------------------------------------------- the kernel --
template <int DPL, bool XKV, int ORDER>
__global__ __launch_bounds__(kAttnThreads) void attn_split_kernel(
    const HeadDev *__restrict__ heads, const WorkItem *__restrict__ items, const uint16_t *__restrict__ q_all,
    float *__restrict__ out_all, float *__restrict__ lse_all, float *__restrict__ ws, int dim,
    uint32_t *__restrict__ status) {
    using L = AttnLds<DPL>;
    constexpr int DM = L::DM;
    constexpr int RS = L::RS;
    extern __shared__ __align__(16) unsigned char lds_raw[];
    L &lds = *reinterpret_cast<L *>(lds_raw);

    const WorkItem wi = items[blockIdx.x];
    const HeadDev hd = heads[wi.head];
    const int G = hd.n_q;
    const int lane = lane_id();
    const int w = int(threadIdx.x) >> 6;

    // q rows as FP32 (DAZ-flushed for the VDPBF16PS order).
    const uint16_t *qh = q_all + size_t(hd.q_row) * size_t(dim);
    for (int i = int(threadIdx.x); i < G * dim; i += kAttnThreads) {
        const int g = i / dim, d = i - g * dim;
        const float qf = bf16_f32(qh[i]);
        lds.q[g * DM + d] = ORDER == 1 ? daz(qf) : qf;
    }

    const int g0 = w, g1 = w + kAttnWaves;
    const bool own0 = g0 < G, own1 = g1 < G;
    float m0 = -__builtin_inff(), m1 = -__builtin_inff();
    float l0 = 0.0f, l1 = 0.0f;
    float acc0[DPL], acc1[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc0[j] = acc1[j] = 0.0f;

    // `bad` holds header/index problems: every thread computes the same value,
    // so the chunk loop below stays uniform. `bad_esc` (escape overrun) is
    // per thread and only reported.
    uint32_t bad = 0, bad_esc = 0;
    // XKV cursors: current block, its first token and header, escape carry.
    int kb = wi.kblk, vb = wi.vblk;
    int kb_t0 = 0, kb_t1 = 0, vb_t0 = 0, vb_t1 = 0;
    int kesc = 0, vesc = 0;
    BlockHdr kh{}, vh{};
    const uint8_t *kblkp = nullptr, *vblkp = nullptr;
    if (XKV) {
        kb_t0 = hd.kfirst[kb];
        kb_t1 = hd.kfirst[kb + 1];
        vb_t0 = hd.vfirst[vb];
        vb_t1 = hd.vfirst[vb + 1];
        bad |= check_block(hd.kx, hd.kbytes, hd.koff[kb], dim, kb_t1 - kb_t0, &kh);
        bad |= check_block(hd.vx, hd.vbytes, hd.voff[vb], dim, vb_t1 - vb_t0, &vh);
        kblkp = hd.kx + hd.koff[kb];
        vblkp = hd.vx + hd.voff[vb];
        if (kb_t0 != wi.tok_begin || vb_t0 != wi.tok_begin) bad |= kStIndex;
    }
    __syncthreads();

    for (int t = wi.tok_begin; t < wi.tok_end && bad == 0u;) {
        if (XKV) {
            if (t >= kb_t1) {
                ++kb;
                kb_t0 = kb_t1;
                kb_t1 = hd.kfirst[kb + 1];
                bad |= check_block(hd.kx, hd.kbytes, hd.koff[kb], dim, kb_t1 - kb_t0, &kh);
                kblkp = hd.kx + hd.koff[kb];
                kesc = 0;
            }
            if (t >= vb_t1) {
                ++vb;
                vb_t0 = vb_t1;
                vb_t1 = hd.vfirst[vb + 1];
                bad |= check_block(hd.vx, hd.vbytes, hd.voff[vb], dim, vb_t1 - vb_t0, &vh);
                vblkp = hd.vx + hd.voff[vb];
                vesc = 0;
            }
            if (bad) break;
        }
        int n = min(kChunk, wi.tok_end - t);
        if (XKV) n = min(n, min(kb_t1 - t, vb_t1 - t));

        // 1. decode the chunk's K and V rows into LDS
        if (XKV) {
            xkv_rows_to_lds<DPL>(kblkp, kh, dim, t - kb_t0, n, lds.k, &kesc, lds.scan_tmp, &bad_esc);
            xkv_rows_to_lds<DPL>(vblkp, vh, dim, t - vb_t0, n, lds.v, &vesc, lds.scan_tmp, &bad_esc);
        } else {
            raw_rows_to_lds<DPL>(hd.kraw, dim, t, n, lds.k);
            raw_rows_to_lds<DPL>(hd.vraw, dim, t, n, lds.v);
        }
        __syncthreads();

        // 2. scores and softmax coefficients, lane = token
        bool resc0 = false, resc1 = false;
        if (own0) {
            const float *krow = lds.k + lane * RS;
            float s0 = 0.0f, s1 = 0.0f;
            if (own1)
                chunk_scores<ORDER, true>(krow, lds.q + g0 * DM, lds.q + g1 * DM, dim, &s0, &s1);
            else
                chunk_scores<ORDER, false>(krow, lds.q + g0 * DM, lds.q + g0 * DM, dim, &s0, &s1);
            resc0 = chunk_softmax(s0, n, &m0, lds.e[g0], lds.a[g0]);
            if (own1) resc1 = chunk_softmax(s1, n, &m1, lds.e[g1], lds.a[g1]);
        }
        __syncthreads();

        // 3. ordered fold of the chunk, lane = channel
        if (own0) {
            for (int tok = 0; tok < n; ++tok) {
                float v[DPL];
#pragma unroll
                for (int j = 0; j < DPL; ++j) v[j] = lds.v[tok * RS + lane + 64 * j];
                const float e0 = lds.e[g0][tok], a0 = lds.a[g0][tok];
                if (resc0) {
#pragma unroll
                    for (int j = 0; j < DPL; ++j) acc0[j] = fmaf(e0, v[j], acc0[j] * a0);
                } else {
#pragma unroll
                    for (int j = 0; j < DPL; ++j) acc0[j] = fmaf(e0, v[j], acc0[j]);
                }
                l0 = fmaf(l0, a0, e0);
                if (own1) {
                    const float e1 = lds.e[g1][tok], a1 = lds.a[g1][tok];
                    if (resc1) {
#pragma unroll
                        for (int j = 0; j < DPL; ++j) acc1[j] = fmaf(e1, v[j], acc1[j] * a1);
                    } else {
#pragma unroll
                        for (int j = 0; j < DPL; ++j) acc1[j] = fmaf(e1, v[j], acc1[j]);
                    }
                    l1 = fmaf(l1, a1, e1);
                }
            }
        }
        __syncthreads();
        t += n;
    }
    bad |= bad_esc;
    if (bad) atomicOr(status, bad);

    // epilogue: finalise (single split) or store the partial state
    if (own0) store_row<DPL>(hd, wi, g0, m0, l0, acc0, dim, lane, out_all, lse_all, ws);
    if (own1) store_row<DPL>(hd, wi, g1, m1, l1, acc1, dim, lane, out_all, lse_all, ws);
}

// merge_state in split order, then finalize_state (softmax.hpp:16-41).
__global__ __launch_bounds__(256) void merge_kernel(const HeadDev *__restrict__ heads, const int32_t *__restrict__ ids,
                                                   const float *__restrict__ ws, float *__restrict__ out_all,
                                                   float *__restrict__ lse_all, int dim) {
    const HeadDev hd = heads[ids[blockIdx.x]];
    const int G = hd.n_q;
    const size_t stride = slot_floats(dim);
    const float *slots = ws + size_t(hd.ws_base) * stride;
    for (int i = int(threadIdx.x); i < G * dim; i += 256) {
        const int g = i / dim, d = i - g * dim;
        float m = slots[g], l = slots[kMaxQ + g], a = slots[2 * kMaxQ + i];
        for (int s = 1; s < hd.n_splits; ++s) {
            const float *sl = slots + size_t(s) * stride;
            const float mb = sl[g], lb = sl[kMaxQ + g], ab = sl[2 * kMaxQ + i];
            const float mm = (m < mb) ? mb : m;
            const float e1 = kvexp_expf(m - mm);
            const float e2 = kvexp_expf(mb - mm);
            l = fmaf(l, e1, lb * e2);
            a = fmaf(a, e1, ab * e2);
            m = mm;
        }
        const float inv = 1.0f / l;
        out_all[(size_t(hd.q_row) + g) * size_t(dim) + d] = a * inv;
        if (lse_all != nullptr && d == 0) lse_all[hd.q_row + g] = m + logf(l);
    }
}

} // namespace kvexp_dev

// ---------------------------------------------------------------- launchers --
namespace kvexp_launch {
using namespace kvexp_dev;

template <int DPL, bool XKV, int ORDER>
static hipError_t launch_attn(const HeadDev *heads, const WorkItem *items, int n_items, const uint16_t *q, float *out,
                              float *lse, float *ws, int dim, uint32_t *status, hipStream_t s) {
    auto kern = attn_split_kernel<DPL, XKV, ORDER>;
    const size_t lds = sizeof(AttnLds<DPL>);
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
        if (e != hipSuccess) return e;
        configured = true;
    }
    hipLaunchKernelGGL(kern, dim3(n_items), dim3(kAttnThreads), lds, s, heads, items, q, out, lse, ws, dim, status);
    return hipGetLastError();
}

template <int DPL>
static hipError_t attn_dpl(bool xkv, int order, const HeadDev *heads, const WorkItem *items, int n_items,
                           const uint16_t *q, float *out, float *lse, float *ws, int dim, uint32_t *status,
                           hipStream_t s) {
    if (xkv)
        return order == 0 ? launch_attn<DPL, true, 0>(heads, items, n_items, q, out, lse, ws, dim, status, s)
                          : launch_attn<DPL, true, 1>(heads, items, n_items, q, out, lse, ws, dim, status, s);
    return order == 0 ? launch_attn<DPL, false, 0>(heads, items, n_items, q, out, lse, ws, dim, status, s)
                      : launch_attn<DPL, false, 1>(heads, items, n_items, q, out, lse, ws, dim, status, s);
}

hipError_t attention(bool xkv, int order, const HeadDev *heads, const WorkItem *items, int n_items,
                     const int32_t *merge_ids, int n_merge, const uint16_t *q, float *out, float *lse, float *ws,
                     int dim, uint32_t *status, hipStream_t s) {
    hipError_t e;
    if (dim <= 64)
        e = attn_dpl<1>(xkv, order, heads, items, n_items, q, out, lse, ws, dim, status, s);
    else if (dim <= 128)
        e = attn_dpl<2>(xkv, order, heads, items, n_items, q, out, lse, ws, dim, status, s);
    else
        e = attn_dpl<4>(xkv, order, heads, items, n_items, q, out, lse, ws, dim, status, s);
    if (e != hipSuccess) return e;
    if (n_merge > 0) {
        hipLaunchKernelGGL(merge_kernel, dim3(n_merge), dim3(256), 0, s, heads, merge_ids, ws, out, lse, dim);
        e = hipGetLastError();
    }
    return e;
}

size_t attention_lds_bytes(int dim) {
    if (dim <= 64) return sizeof(AttnLds<1>);
    if (dim <= 128) return sizeof(AttnLds<2>);
    return sizeof(AttnLds<4>);
}

} // namespace kvexp_launch
