// C ABI of the gfx950 backend (include/kvexp_hip.h).
//
// Host-side responsibilities: argument validation with the reference's
// exception classes and messages, the host walk of block headers, split
// planning (token_bounds, dispatch.cpp:17-23, with the block-alignment rule
// of scan.hpp:107-109), device descriptors and workspace, and mapping the
// kernels' status word back to errors. All arithmetic runs in the kernels.
#include "kvexp_hip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../hip/kvexp_types.h"
#include "host_walk.hpp"

using kvexp_dev::AppendJobDev;
using kvexp_dev::EncBlockMeta;
using kvexp_dev::HeadDev;
using kvexp_dev::WorkItem;

namespace kvexp_launch {
hipError_t decode(const uint8_t *blob, uint64_t bytes, const int64_t *offs, const int32_t *first, int n_blocks,
                  int seq, int dim, uint16_t *out, uint32_t *status, hipStream_t s);
bool encode_fused_supported(int dim, int bt);
hipError_t encode(const uint16_t *kv, int seq, int dim, int bt, int n_blocks, EncBlockMeta *meta, uint8_t *bases,
                  int64_t *offs, int32_t *first, uint8_t *out, uint32_t *status, hipStream_t s, bool rebase,
                  int tok0, int modes, const kvexp_dev::EncLookback *lb);
hipError_t append(const kvexp_dev::AppendJobDev *jobs, int n_jobs, int total_blocks, int dim, int bt,
                  EncBlockMeta *meta, uint8_t *bases, uint32_t *status, hipStream_t s, bool one_block, int modes,
                  const kvexp_dev::EncLookback *lb, int max_job_blocks);
hipError_t attention(bool xkv, int order, const HeadDev *heads, const WorkItem *items, int n_items,
                     const int32_t *merge_ids, int n_merge, const uint16_t *q, float *out, float *lse, float *ws,
                     int dim, uint32_t *status, hipStream_t s);
size_t attention_lds_bytes(int dim);
hipError_t expf(const float *x, float *y, size_t n, hipStream_t s);
hipError_t esc_start(const kvexp_dev::EscJob *jobs, int n_jobs, uint32_t *status, hipStream_t s);
hipError_t esc_pos(const kvexp_dev::EscJob *jobs, const int2 *blocks, int n_blocks, uint32_t *status, hipStream_t s);
hipError_t plan_refresh(const kvexp_dev::EscJob *jobs, int n_jobs, HeadDev *heads, int n_dev_heads, WorkItem *items,
                        int n_items, int per_head, uint32_t *status, hipStream_t s);
bool wave_supports(int dim);
hipError_t attention_wave(bool xkv, int order, int G, int dim, const HeadDev *heads, const WorkItem *items,
                          int n_items, int wpg, const kvexp_dev::BlockDesc *desc, const uint16_t *q, float *out,
                          float *lse, float *ws, hipStream_t s);
hipError_t wave_merge(int dim, const kvexp_dev::MergeItem *mitems, int n_mitems, const kvexp_dev::MergeItem &uni,
                      float *out, float *lse, const float *ws, hipStream_t s);
int wave_waves_per_wg(int dim);
hipError_t noalloc_scratch_setup(int device, void **ptr);
void *noalloc_scratch(int device);
} // namespace kvexp_launch

namespace {

using namespace kvexp_host; // KvexpFail, fail, the host walk, token_bounds

constexpr int kMaxQPerLaunch = 8;
constexpr int kMaxDim = 256;

thread_local std::string g_error;

int set_error(int code, const std::string &msg) {
    g_error = msg;
    return code;
}
int ok() {
    g_error.clear();
    return KVEXP_HIP_OK;
}

struct HipFail {
    hipError_t err;
    const char *what;
};

#define HIPX(call)                                                                                                    \
    do {                                                                                                              \
        hipError_t e_ = (call);                                                                                       \
        if (e_ != hipSuccess) throw HipFail{e_, #call};                                                               \
    } while (0)



template <class F> int guarded(F &&fn) {
    try {
        fn();
        return ok();
    } catch (const KvexpFail &f) {
        return set_error(f.code, f.msg);
    } catch (const HipFail &h) {
        return set_error(KVEXP_HIP_DEVICE_ERROR, std::string(h.what) + ": " + hipGetErrorString(h.err));
    } catch (const std::bad_alloc &) {
        return set_error(KVEXP_HIP_DEVICE_ERROR, "host allocation failed");
    } catch (const std::exception &e) {
        return set_error(KVEXP_HIP_LOGIC_ERROR, e.what());
    }
}

// Device buffers kept for reuse by a context: hipFree synchronises the whole
// device, so a call path that allocated and freed on every call would wait
// for every other caller's work. Blocks are kept by size class (four classes
// per power of two), at most kMaxHeld bytes in all, and returned to the
// device when the context is destroyed. Only buffers whose last use is known
// to be finished when they are released go back to a pool.
class DevPool {
  public:
    static size_t size_class(size_t n) {
        size_t c = 256;
        while (c < n) c *= 2;
        if (c <= 256) return c;
        const size_t q = c / 8; // c/2 + q, c/2 + 2q, c/2 + 3q, c
        for (size_t k = 5; k <= 8; ++k)
            if (q * k >= n) return q * k;
        return c;
    }
    void *get(size_t n, size_t &cap) {
        cap = size_class(n);
        {
            std::lock_guard<std::mutex> lock(mu_);
            for (size_t i = 0; i < free_.size(); ++i)
                if (free_[i].first == cap) {
                    void *p = free_[i].second;
                    free_[i] = free_.back();
                    free_.pop_back();
                    held_ -= cap;
                    return p;
                }
        }
        void *p = nullptr;
        HIPX(hipMalloc(&p, cap));
        return p;
    }
    void put(void *p, size_t cap) {
        {
            std::lock_guard<std::mutex> lock(mu_);
            if (held_ + cap <= kMaxHeld) {
                free_.emplace_back(cap, p);
                held_ += cap;
                return;
            }
        }
        (void)hipFree(p);
    }
    ~DevPool() {
        for (auto &f : free_) (void)hipFree(f.second);
    }

  private:
    static constexpr size_t kMaxHeld = size_t(1) << 30;
    std::mutex mu_;
    std::vector<std::pair<size_t, void *>> free_;
    size_t held_ = 0;
};

// Device allocation released on scope exit unless kept: back to its pool
// when it came from one, else to the device.
struct DevBuf {
    void *p = nullptr;
    DevPool *pool = nullptr;
    size_t cap = 0;
    DevBuf() = default;
    explicit DevBuf(size_t n) {
        if (n) HIPX(hipMalloc(&p, n));
    }
    DevBuf(DevPool *from, size_t n) {
        if (from == nullptr) {
            if (n) HIPX(hipMalloc(&p, n));
        } else if (n) {
            p = from->get(n, cap);
            pool = from;
        }
    }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    DevBuf(DevBuf &&o) noexcept : p(o.p), pool(o.pool), cap(o.cap) { o.p = nullptr; }
    DevBuf &operator=(DevBuf &&o) noexcept {
        std::swap(p, o.p);
        std::swap(pool, o.pool);
        std::swap(cap, o.cap);
        return *this;
    }
    ~DevBuf() {
        if (p == nullptr) return;
        if (pool) pool->put(p, cap);
        else (void)hipFree(p);
    }
    template <class T> T *as() const { return static_cast<T *>(p); }
};

std::string status_message(uint32_t st) {
    using namespace kvexp_dev;
    if (st & kStHeader) return "xkv block dimension or length mismatch";
    if (st & kStMode) return "unknown xkv block mode";
    if (st & kStTruncated) return "truncated coded xkv block";
    if (st & kStIndex) return "xkv block index does not match the container";
    if (st & kStEscape) return "xkv escape stream overrun";
    return "xkv container error";
}

// The encoders' status word as an error message.
std::string encoder_status_message(uint32_t st) {
    if (st & kvexp_dev::kStLookback) return "one-pass encoder: an earlier block's size never arrived";
    return "escape count drifted from the size model";
}

} // namespace

// ================================================================ context ==
struct kvexp_hip_ctx {
    int device = 0;
    // buffers of the host-pointer entry and of the plans it builds (declared
    // first: destroyed after everything that may return buffers to it)
    DevPool pool;
    DevBuf status; // uint32 status word of the encoders and the decoder
    // encoder scratch, grown on demand; `scratch_done` is recorded on the
    // stream of the last launch that used it, so growing it never frees
    // memory that a kernel still in flight reads
    DevBuf enc_meta, enc_bases, enc_off, enc_first, app_jobs;
    size_t enc_meta_cap = 0, enc_bases_cap = 0, enc_index_cap = 0, app_jobs_cap = 0;
    // look-back entries and ticket counters of the one-pass encoder, the
    // epoch of its last launch, and whether a launch reported a broken
    // look-back (the next one then clears both arrays)
    DevBuf enc_lb, enc_tk;
    size_t enc_lb_cap = 0, enc_tk_cap = 0;
    uint32_t enc_epoch = 0;
    bool enc_lb_dirty = false;
    hipEvent_t scratch_done = nullptr;
    // stream of the host-pointer entry (kvexp_hip_attention_decode_host): its
    // copies and kernels wait for nothing outside this context
    hipStream_t stream = nullptr;
    int cu_count = 0;
    int enc_modes = int(KVEXP_HIP_MODES_REFERENCE); // coded modes the encoders may choose
    // pinned host staging for the plan builder's reads of block indexes
    void *pinned = nullptr;
    size_t pinned_cap = 0;
    ~kvexp_hip_ctx() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (scratch_done) (void)hipEventSynchronize(scratch_done);
        if (pinned) (void)hipHostFree(pinned);
        if (scratch_done) (void)hipEventDestroy(scratch_done);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

struct kvexp_hip_plan {
    kvexp_hip_ctx *ctx = nullptr;
    // buffers from the context's pool (plans of the host-pointer entry, which
    // synchronises its stream before destroying them); others are freed
    bool pooled = false;
    DevBuf alloc(size_t n) const { return DevBuf(pooled ? &ctx->pool : nullptr, n); }
    int n_heads = 0, n_q = 0, dim = 0, order = 0, split_tokens = 0;
    // set when kvexp_hip_plan_update failed after the containers changed: the
    // plan's descriptors no longer describe them, so runs are refused until
    // an update succeeds
    bool invalid = false;
    std::string invalid_msg;
    // ---- everything below is made by plan_build (swapped in whole by updates)
    bool xkv = false;
    // what kvexp_hip_plan_update needs: the heads as given and the per-tensor
    // escape-index jobs (host copy and device copy)
    std::vector<kvexp_hip_head> src;
    std::vector<kvexp_dev::EscJob> jobs;
    std::vector<int32_t> esc_prefix; // per tensor (jobs order): escapes before each block, n_blocks + 1 entries
    std::vector<size_t> esc_prefix_at;
    DevBuf djobs;
    bool wave = false; // one-wave-per-split kernel (dim 64 or 128)
    DevBuf heads, items, merge_ids, ws, status;
    // wave kernel: merge work (head, row), escape records, block descriptors
    DevBuf mitems, esc0, escpos, desc;
    int n_mitems = 0;
    // the merge items as a pattern when they follow one (g > 0; see
    // wave_merge_kernel), else g = 0
    kvexp_dev::MergeItem merge_uni{};
    int n_dev_heads = 0, n_items = 0, n_merge = 0;
    // wave kernel: items sorted by query-row count G; group_start[G] .. group_start[G+1]
    int group_start[10] = {0};
    // ---- end of plan_build's part
    // split-kernel timing: one event pair per run while enabled
    bool timing = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> events;
    void clear_events() {
        for (auto &e : events) {
            (void)hipEventDestroy(e.first);
            (void)hipEventDestroy(e.second);
        }
        events.clear();
    }
    ~kvexp_hip_plan() { clear_events(); }
};

namespace {
struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        HIPX(hipGetDevice(&prev));
        if (prev != dev) HIPX(hipSetDevice(dev));
    }
    ~DeviceGuard() {
        int cur = -1;
        if (hipGetDevice(&cur) == hipSuccess && cur != prev && prev >= 0) (void)hipSetDevice(prev);
    }
};

// Grows one of the context's scratch buffers. The old buffer may still be
// read by the last launch that used it (on any stream): wait for it first.
void grow(kvexp_hip_ctx *ctx, DevBuf &buf, size_t &cap, size_t need) {
    if (need <= cap) return;
    if (ctx->scratch_done) HIPX(hipEventSynchronize(ctx->scratch_done));
    DevBuf nb(need);
    buf = std::move(nb);
    cap = need;
}

// The one-pass encoder's look-back state for a launch of `blocks` blocks
// over `jobs` containers (an entry per block, a ticket counter per job):
// grown on demand; the entries cleared (by the launcher, with a kernel) when
// new and when the launch epoch wraps, so that no entry left by an earlier
// launch carries the epoch of a later one; the counters when new (each
// launch leaves them at 0) and after a launch reported a broken look-back.
kvexp_dev::EncLookback lookback_for(kvexp_hip_ctx *ctx, int jobs, int blocks) {
    size_t clear = 0, clear_tk = 0;
    if (size_t(blocks) * sizeof(uint64_t) > ctx->enc_lb_cap) {
        grow(ctx, ctx->enc_lb, ctx->enc_lb_cap, size_t(blocks) * sizeof(uint64_t));
        clear = ctx->enc_lb_cap / sizeof(uint64_t);
    }
    if (size_t(jobs) * sizeof(uint32_t) > ctx->enc_tk_cap) {
        grow(ctx, ctx->enc_tk, ctx->enc_tk_cap, size_t(jobs) * sizeof(uint32_t));
        clear_tk = ctx->enc_tk_cap / sizeof(uint32_t);
    }
    if (++ctx->enc_epoch > 0xFFFFu || ctx->enc_lb_dirty) {
        ctx->enc_epoch = 1;
        clear = ctx->enc_lb_cap / sizeof(uint64_t);
        if (ctx->enc_lb_dirty) clear_tk = ctx->enc_tk_cap / sizeof(uint32_t);
        ctx->enc_lb_dirty = false;
    }
    return kvexp_dev::EncLookback{ctx->enc_lb.as<uint64_t>(), ctx->enc_tk.as<uint32_t>(), ctx->enc_epoch, clear,
                                  clear_tk};
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Orders work about to be queued on `s` that writes the context's scratch
// after the last work that used it (which may be on another stream).
void scratch_acquire(kvexp_hip_ctx *ctx, hipStream_t s) {
    if (ctx->scratch_done) HIPX(hipStreamWaitEvent(s, ctx->scratch_done, 0));
}

// Marks the context's scratch as in use by the work just queued on `s`.
void scratch_used(kvexp_hip_ctx *ctx, hipStream_t s) {
    if (ctx->scratch_done == nullptr) HIPX(hipEventCreateWithFlags(&ctx->scratch_done, hipEventDisableTiming));
    HIPX(hipEventRecord(ctx->scratch_done, s));
}

void check_status_word(uint32_t *d_status, hipStream_t s) {
    uint32_t st = 0;
    HIPX(hipMemcpyAsync(&st, d_status, sizeof st, hipMemcpyDeviceToHost, s));
    HIPX(hipStreamSynchronize(s));
    if (st != 0u) {
        HIPX(hipMemsetAsync(d_status, 0, sizeof(uint32_t), s));
        HIPX(hipStreamSynchronize(s));
        fail(KVEXP_HIP_FORMAT_ERROR, status_message(st));
    }
}
// Block descriptors and escape records of every XKV tensor of a plan:
// per block its address, first escape index and header fields (checked
// against the block index; a mismatch fails the plan with the matching
// format error), and per escape its element index inside the block. Built on
// the device from the containers, once per plan; the device heads of one
// user head share it.
void build_escape_index(kvexp_hip_plan &p, const kvexp_hip_head *heads, int n_heads, int n_q, int dim,
                        std::vector<HeadDev> &hv, hipStream_t s) {
    std::vector<kvexp_dev::EscJob> jobs;
    std::vector<size_t> e0_at;
    size_t e0_total = 0;
    for (int h = 0; h < n_heads; ++h) {
        for (int kv = 0; kv < 2; ++kv) {
            kvexp_dev::EscJob j{};
            j.blob = kv ? heads[h].v_xkv : heads[h].k_xkv;
            j.bytes = kv ? heads[h].v_bytes : heads[h].k_bytes;
            j.offs = kv ? heads[h].v_offsets : heads[h].k_offsets;
            j.first = kv ? heads[h].v_first_token : heads[h].k_first_token;
            j.n_blocks = kv ? heads[h].v_n_blocks : heads[h].k_n_blocks;
            j.dim = dim;
            e0_at.push_back(e0_total);
            e0_total += size_t(j.n_blocks) + 1;
            jobs.push_back(j);
        }
    }
    p.esc0 = p.alloc(e0_total * sizeof(int32_t));
    p.desc = p.alloc(e0_total * sizeof(kvexp_dev::BlockDesc));
    // HIP memory is not zeroed: the entry after each tensor's last block is
    // the zero-token sentinel until a plan update writes it again
    HIPX(hipMemsetAsync(p.desc.p, 0, e0_total * sizeof(kvexp_dev::BlockDesc), s));
    for (size_t i = 0; i < jobs.size(); ++i) {
        jobs[i].esc0 = p.esc0.as<int32_t>() + e0_at[i];
        jobs[i].desc = p.desc.as<kvexp_dev::BlockDesc>() + e0_at[i];
    }
    DevBuf djobs = p.alloc(jobs.size() * sizeof(kvexp_dev::EscJob));
    uint32_t *st = p.status.as<uint32_t>(); // the plan's own status word
    // pass 1: block checks and escape counts (descriptors need the position array)
    std::vector<kvexp_dev::EscJob> jobs1 = jobs;
    for (auto &j : jobs1) j.desc = nullptr;
    HIPX(hipMemcpyAsync(djobs.p, jobs1.data(), jobs1.size() * sizeof(kvexp_dev::EscJob), hipMemcpyHostToDevice, s));
    HIPX(kvexp_launch::esc_start(djobs.as<kvexp_dev::EscJob>(), int(jobs.size()), st, s));
    check_status_word(st, s);
    std::vector<int32_t> e0(e0_total);
    HIPX(hipMemcpyAsync(e0.data(), p.esc0.p, e0_total * sizeof(int32_t), hipMemcpyDeviceToHost, s));
    HIPX(hipStreamSynchronize(s));
    p.esc_prefix = e0;
    p.esc_prefix_at = e0_at;
    // each tensor's positions, then room for its last block to grow to the
    // largest block the format allows (255 tokens) after appends
    size_t pos_total = 0;
    std::vector<size_t> pos_at;
    std::vector<int2> blocks;
    for (size_t i = 0; i < jobs.size(); ++i) {
        pos_at.push_back(pos_total);
        const size_t own = size_t(e0[e0_at[i] + size_t(jobs[i].n_blocks)]);
        jobs[i].pos_cap = int32_t(own + size_t(255) * size_t(dim));
        pos_total += size_t(jobs[i].pos_cap);
        for (int b = 0; b < jobs[i].n_blocks; ++b) blocks.push_back(make_int2(int(i), b));
    }
    // escape records, then kEscPad spare ones: a kernel's window of records
    // read from any escape stays inside the allocation (zeroed, never used)
    p.escpos = p.alloc((pos_total + size_t(kvexp_dev::kEscPad)) * sizeof(uint32_t));
    HIPX(hipMemsetAsync(p.escpos.as<uint32_t>() + pos_total, 0, size_t(kvexp_dev::kEscPad) * sizeof(uint32_t), s));
    for (size_t i = 0; i < jobs.size(); ++i) jobs[i].pos = p.escpos.as<uint32_t>() + pos_at[i];
    HIPX(hipMemcpyAsync(djobs.p, jobs.data(), jobs.size() * sizeof(kvexp_dev::EscJob), hipMemcpyHostToDevice, s));
    // pass 2: descriptors (with the escape-record pointers)
    HIPX(kvexp_launch::esc_start(djobs.as<kvexp_dev::EscJob>(), int(jobs.size()), st, s));
    DevBuf dblocks = p.alloc(std::max<size_t>(blocks.size(), 1) * sizeof(int2));
    HIPX(hipMemcpyAsync(dblocks.p, blocks.data(), blocks.size() * sizeof(int2), hipMemcpyHostToDevice, s));
    HIPX(kvexp_launch::esc_pos(djobs.as<kvexp_dev::EscJob>(), dblocks.as<int2>(), int(blocks.size()), st, s));
    check_status_word(st, s); // synchronises s: the host vectors above may go
    p.jobs = jobs;
    p.djobs = std::move(djobs);
    const int per_head = (n_q + kMaxQPerLaunch - 1) / kMaxQPerLaunch;
    for (int h = 0; h < n_heads; ++h) {
        for (int c = 0; c < per_head; ++c) {
            HeadDev &d = hv[size_t(h * per_head + c)];
            d.kdesc = jobs[size_t(2 * h)].desc;
            d.kesc = jobs[size_t(2 * h)].pos;
            d.vdesc = jobs[size_t(2 * h + 1)].desc;
            d.vesc = jobs[size_t(2 * h + 1)].pos;
        }
    }
}

} // namespace

extern "C" {

const char *kvexp_hip_status_string(int status) {
    switch (status) {
    case KVEXP_HIP_OK: return "ok";
    case KVEXP_HIP_INVALID_ARGUMENT: return "invalid argument";
    case KVEXP_HIP_FORMAT_ERROR: return "container or split format error";
    case KVEXP_HIP_LOGIC_ERROR: return "internal consistency error";
    case KVEXP_HIP_UNSUPPORTED: return "unsupported shape or option";
    case KVEXP_HIP_DEVICE_ERROR: return "HIP runtime error";
    case KVEXP_HIP_CAPACITY: return "output buffer too small";
    default: return "unknown status";
    }
}

const char *kvexp_hip_last_error(void) { return g_error.c_str(); }

const char *kvexp_hip_version(void) { return "kvexp-amd 0.1 (gfx950)"; }

int kvexp_hip_ctx_create(int device, kvexp_hip_ctx **out) {
    return guarded([&] {
        if (out == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_ctx_create: null output");
        *out = nullptr;
        int n = 0;
        HIPX(hipGetDeviceCount(&n));
        if (device < 0 || device >= n) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_ctx_create: no such device");
        DeviceGuard g(device);
        hipDeviceProp_t prop;
        HIPX(hipGetDeviceProperties(&prop, device));
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            fail(KVEXP_HIP_UNSUPPORTED, std::string("kvexp-amd is built for gfx950, device is ") + prop.gcnArchName);
        auto *c = new kvexp_hip_ctx();
        c->device = device;
        c->cu_count = prop.multiProcessorCount;
        try {
            c->status = DevBuf(sizeof(uint32_t));
            HIPX(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
            // the no-allocation encoder's scratch on this device (looked up once per device)
            void *scratch = nullptr;
            HIPX(kvexp_launch::noalloc_scratch_setup(device, &scratch));
            HIPX(hipMemsetAsync(c->status.p, 0, sizeof(uint32_t), c->stream));
            HIPX(hipStreamSynchronize(c->stream));
        } catch (...) {
            delete c;
            throw;
        }
        *out = c;
    });
}

int kvexp_hip_ctx_destroy(kvexp_hip_ctx *ctx) {
    return guarded([&] {
        if (ctx == nullptr) return;
        DeviceGuard g(ctx->device);
        delete ctx;
    });
}

int kvexp_hip_set_encoder_modes(kvexp_hip_ctx *ctx, unsigned modes) {
    return guarded([&] {
        if (ctx == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_set_encoder_modes: null context");
        const unsigned known = KVEXP_HIP_MODE_2BIT | KVEXP_HIP_MODE_3BIT | KVEXP_HIP_MODE_4BIT;
        if (modes & ~known) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_set_encoder_modes: unknown mode bits");
        ctx->enc_modes = int(modes);
    });
}

int kvexp_hip_get_encoder_modes(kvexp_hip_ctx *ctx) {
    return ctx == nullptr ? -1 : ctx->enc_modes;
}

// ============================================================ size model ==
int kvexp_hip_exp_payload_bytes(int n, int dim, int bits) { return (n * dim * bits + 7) / 8; }
int kvexp_hip_coded_block_bytes(int n, int dim, int bits, int esc) {
    return 8 + dim + n * dim + kvexp_hip_exp_payload_bytes(n, dim, bits) + 2 * esc;
}
int kvexp_hip_raw_block_bytes(int n, int dim) { return 8 + 2 * n * dim; }
int kvexp_hip_block_count(int seq, int bt) {
    if (seq <= 0 || bt <= 0) return 0;
    return (seq + bt - 1) / bt;
}
int64_t kvexp_hip_encode_bound(int seq, int dim, int bt) {
    if (seq <= 0 || dim <= 0 || bt <= 0) return 0;
    return int64_t(kvexp_hip_block_count(seq, bt)) * 8 + 2 * int64_t(seq) * dim;
}

// ================================================================= index ==
int kvexp_hip_build_index(const uint8_t *blob, size_t bytes, int dim, int seq, int64_t *offsets,
                          int32_t *first_token, int capacity, int *n_blocks) {
    return guarded([&] {
        if ((blob == nullptr && bytes) || offsets == nullptr || first_token == nullptr || n_blocks == nullptr)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_build_index: null argument");
        std::vector<int64_t> off;
        std::vector<int32_t> first;
        walk_index(blob, bytes, dim, seq, off, first);
        const int nb = int(off.size()) - 1;
        *n_blocks = nb;
        if (nb > capacity) fail(KVEXP_HIP_CAPACITY, "kvexp_hip_build_index: capacity below the block count");
        std::memcpy(offsets, off.data(), off.size() * sizeof(int64_t));
        std::memcpy(first_token, first.data(), first.size() * sizeof(int32_t));
    });
}

// ================================================================= codec ==
int kvexp_hip_encode(kvexp_hip_ctx *ctx, const uint16_t *d_kv, int seq, int dim, int bt, uint8_t *d_out,
                     size_t capacity, int64_t *d_offsets, int32_t *d_first_token, size_t *bytes_out, void *stream) {
    return guarded([&] {
        if (ctx == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_encode: null context");
        // codec.cpp:40-52
        if (d_kv == nullptr || seq <= 0 || dim <= 0 || bt <= 0)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: empty input");
        if (dim % 4 != 0 || dim > kMaxDim)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: head_dim must be a multiple of 4 and at most 256");
        if (bt > 255) fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: block_tokens must fit in a byte");
        if (int64_t(bt) * dim > 65535)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: block escape count would not fit in u16");
        if (d_out == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_encode: null output");
        if (int64_t(capacity) < kvexp_hip_encode_bound(seq, dim, bt))
            fail(KVEXP_HIP_CAPACITY, "kvexp_hip_encode: capacity below kvexp_hip_encode_bound");
        DeviceGuard g(ctx->device);
        hipStream_t s = static_cast<hipStream_t>(stream);
        const int nb = kvexp_hip_block_count(seq, bt);
        const bool fused = kvexp_launch::encode_fused_supported(dim, bt) && aligned16(d_kv);
        if (!fused) {
            grow(ctx, ctx->enc_meta, ctx->enc_meta_cap, size_t(nb) * sizeof(EncBlockMeta));
            grow(ctx, ctx->enc_bases, ctx->enc_bases_cap, size_t(nb) * 3u * size_t(dim));
        }
        int64_t *offs = d_offsets;
        int32_t *first = d_first_token;
        if (offs == nullptr || first == nullptr) {
            const size_t need = size_t(nb + 1) * (sizeof(int64_t) + sizeof(int32_t));
            if (need > ctx->enc_index_cap) {
                if (ctx->scratch_done) HIPX(hipEventSynchronize(ctx->scratch_done));
                ctx->enc_off = DevBuf(size_t(nb + 1) * sizeof(int64_t));
                ctx->enc_first = DevBuf(size_t(nb + 1) * sizeof(int32_t));
                ctx->enc_index_cap = need;
            }
            if (offs == nullptr) offs = ctx->enc_off.as<int64_t>();
            if (first == nullptr) first = ctx->enc_first.as<int32_t>();
        }
        kvexp_dev::EncLookback lb{};
        if (fused) lb = lookback_for(ctx, 1, nb);
        scratch_acquire(ctx, s);
        HIPX(kvexp_launch::encode(d_kv, seq, dim, bt, nb, ctx->enc_meta.as<EncBlockMeta>(),
                                  ctx->enc_bases.as<uint8_t>(), offs, first, d_out, ctx->status.as<uint32_t>(), s,
                                  false, 0, ctx->enc_modes, fused ? &lb : nullptr));
        scratch_used(ctx, s);
        if (bytes_out != nullptr) {
            int64_t total = 0;
            uint32_t st = 0;
            HIPX(hipMemcpyAsync(&total, offs + nb, sizeof total, hipMemcpyDeviceToHost, s));
            HIPX(hipMemcpyAsync(&st, ctx->status.p, sizeof st, hipMemcpyDeviceToHost, s));
            HIPX(hipStreamSynchronize(s));
            if (st != 0u) {
                HIPX(hipMemsetAsync(ctx->status.p, 0, sizeof(uint32_t), s));
                HIPX(hipStreamSynchronize(s));
                if (st & kvexp_dev::kStLookback) ctx->enc_lb_dirty = true;
        fail(KVEXP_HIP_LOGIC_ERROR, encoder_status_message(st));
            }
            *bytes_out = size_t(total);
        }
    });
}

// Look-back state of a no-allocation one-pass call in the per-device static
// array: the ticket counter in the first 256 bytes, then one entry per block.
// Every call clears its own entries and the ticket with a kernel queued
// before the encoder, and every call uses epoch 1: a call (or a replay of a
// captured graph that holds one) then never takes an entry that an earlier
// call left behind for a published one, whatever the earlier call's input
// was. The cost is one small launch (8 bytes per block).
namespace {
kvexp_dev::EncLookback noalloc_lookback(uint8_t *scratch, int blocks) {
    return kvexp_dev::EncLookback{reinterpret_cast<uint64_t *>(scratch + 256), reinterpret_cast<uint32_t *>(scratch),
                                  1u, size_t(blocks), 1u};
}
} // namespace

// kvexp_hip_encode with its scratch (block metadata and base-exponent
// candidates) in the library's per-device static array instead of context
// buffers grown with hipMalloc: no allocation, no synchronisation, and the
// index is an output the caller provides. Rejects inputs whose scratch would
// not fit the array.
int kvexp_hip_encode_noalloc(kvexp_hip_ctx *ctx, const uint16_t *d_kv, int seq, int dim, int bt, uint8_t *d_out,
                             size_t capacity, int64_t *d_offsets, int32_t *d_first_token, uint32_t *d_status,
                             void *stream) {
    return guarded([&] {
        if (ctx == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_encode_noalloc: null context");
        // codec.cpp:40-52, as kvexp_hip_encode
        if (d_kv == nullptr || seq <= 0 || dim <= 0 || bt <= 0)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: empty input");
        if (dim % 4 != 0 || dim > kMaxDim)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: head_dim must be a multiple of 4 and at most 256");
        if (bt > 255) fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: block_tokens must fit in a byte");
        if (int64_t(bt) * dim > 65535)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: block escape count would not fit in u16");
        if (d_out == nullptr || d_offsets == nullptr || d_first_token == nullptr)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_encode_noalloc: null output or block index");
        if (int64_t(capacity) < kvexp_hip_encode_bound(seq, dim, bt))
            fail(KVEXP_HIP_CAPACITY, "kvexp_hip_encode_noalloc: capacity below kvexp_hip_encode_bound");
        const int nb = kvexp_hip_block_count(seq, bt);
        auto up = [](size_t n) { return (n + 255u) & ~size_t(255); };
        // one pass: a look-back word per block and the ticket; else block
        // metadata and base-exponent candidates
        const bool fused = kvexp_launch::encode_fused_supported(dim, bt) && aligned16(d_kv);
        const size_t meta_bytes = fused ? 256u + up(size_t(nb) * sizeof(uint64_t)) : up(size_t(nb) * sizeof(EncBlockMeta));
        const size_t base_bytes = fused ? 0 : up(size_t(nb) * 3u * size_t(dim));
        const size_t need = meta_bytes + base_bytes + 256u; // + a status word when d_status is NULL
        if (need > kvexp_dev::kNoAllocScratchBytes)
            fail(KVEXP_HIP_CAPACITY, "kvexp_hip_encode_noalloc: " + std::to_string(nb) + " blocks of head_dim " +
                                         std::to_string(dim) + " need " + std::to_string(need) +
                                         " bytes of scratch, more than its " +
                                         std::to_string(kvexp_dev::kNoAllocScratchBytes));
        auto *sp = static_cast<uint8_t *>(kvexp_launch::noalloc_scratch(ctx->device));
        if (sp == nullptr) fail(KVEXP_HIP_LOGIC_ERROR, "kvexp_hip_encode_noalloc: scratch not set up on this device");
        DeviceGuard g(ctx->device);
        uint32_t *st = d_status != nullptr ? d_status : reinterpret_cast<uint32_t *>(sp + meta_bytes + base_bytes);
        kvexp_dev::EncLookback lb{};
        if (fused) lb = noalloc_lookback(sp, nb);
        HIPX(kvexp_launch::encode(d_kv, seq, dim, bt, nb, reinterpret_cast<EncBlockMeta *>(sp), sp + meta_bytes,
                                  d_offsets, d_first_token, d_out, st, static_cast<hipStream_t>(stream), false, 0,
                                  ctx->enc_modes, fused ? &lb : nullptr));
    });
}

// Blocks are encoded independently (codec.cpp:54-160 walks t0 = 0, bt, 2bt,
// ... and each block's bytes depend only on its own tokens), so appending
// tokens changes only the trailing partial block and adds blocks after it:
// each job encodes its container's raw tail followed by the new tokens at
// the tail block's offset (offsets[n_tokens / bt], which is the container's
// size when there is no partial block) and rewrites the index from that
// block on; then the raw rows of the new partial block go to the tail.
namespace {

void check_append_shape(int dim, int bt) {
    if (dim <= 0 || bt <= 0) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_append: bad shape");
    if (dim % 4 != 0 || dim > kMaxDim)
        fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: head_dim must be a multiple of 4 and at most 256");
    if (bt > 255) fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: block_tokens must fit in a byte");
    if (int64_t(bt) * dim > 65535)
        fail(KVEXP_HIP_INVALID_ARGUMENT, "encode_bf16: block escape count would not fit in u16");
}

// Validates one job and appends its device form (none for a no-op);
// returns the blocks it encodes.
int add_append_job(const kvexp_hip_append_job &a, int dim, int bt, int blk0, std::vector<AppendJobDev> &out) {
    if (a.n_new < 0 || a.n_tokens < 0) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_append: bad shape");
    if (a.d_tail == nullptr || a.d_blob == nullptr || a.d_offsets == nullptr || a.d_first_token == nullptr ||
        (a.n_new > 0 && a.d_new == nullptr))
        fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_append: null argument");
    const int64_t total = int64_t(a.n_tokens) + a.n_new;
    if (total > INT32_MAX) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_append: too many tokens");
    if (int64_t(a.capacity) < kvexp_hip_encode_bound(int(total), dim, bt))
        fail(KVEXP_HIP_CAPACITY, "kvexp_hip_append: capacity below kvexp_hip_encode_bound");
    if (a.index_capacity < kvexp_hip_block_count(int(total), bt) + 1)
        fail(KVEXP_HIP_CAPACITY, "kvexp_hip_append: index capacity below n_blocks + 1");
    if (a.n_new == 0 && a.n_tokens > 0) return 0;
    const int tail_n = a.n_tokens % bt, tail_blk = a.n_tokens / bt;
    AppendJobDev j{};
    j.tail = a.d_tail;
    j.src = a.d_new;
    j.offs = a.d_offsets + tail_blk;
    j.first = a.d_first_token + tail_blk;
    j.out = a.d_blob;
    j.tail_n = tail_n;
    j.seq = tail_n + a.n_new;
    j.tok0 = tail_blk * bt;
    j.blk0 = blk0;
    j.nb = kvexp_hip_block_count(j.seq, bt);
    j.rebase = a.n_tokens > 0 ? 1 : 0;
    const int rest = int(total % bt);
    if (rest > 0) {
        const int start = int(total - rest) - j.tok0; // first local row of the new partial block
        const int from = std::max(start, tail_n);      // rows before tail_n are in the tail already
        j.copy_from = from - tail_n;
        j.copy_to = from - start;
        j.copy_rows = start + rest - from;
    }
    out.push_back(j);
    return j.nb;
}

void run_append(kvexp_hip_ctx *ctx, const kvexp_hip_append_job *jobs, int n_jobs, int dim, int bt, hipStream_t s) {
    std::vector<AppendJobDev> dj;
    dj.reserve(size_t(n_jobs));
    int blocks = 0;
    for (int i = 0; i < n_jobs; ++i) blocks += add_append_job(jobs[i], dim, bt, blocks, dj);
    if (dj.empty()) return;
    // every job encodes at most one block (a decode step): one fused launch
    const bool one_block = std::all_of(dj.begin(), dj.end(), [](const AppendJobDev &j) { return j.nb <= 1; });
    // several blocks: one pass when the shape fits it and every source is
    // 16-byte aligned (the tails are allocated so; the new tokens' rows are
    // then aligned too, since dim % 8 == 0)
    int max_nb = 0;
    for (const AppendJobDev &j : dj) max_nb = std::max(max_nb, j.nb);
    const bool fused = !one_block && kvexp_launch::encode_fused_supported(dim, bt) && dj.size() <= 65535u &&
                       std::all_of(dj.begin(), dj.end(), [](const AppendJobDev &j) {
                           return aligned16(j.src) && aligned16(j.tail);
                       });
    if (!fused) {
        grow(ctx, ctx->enc_meta, ctx->enc_meta_cap, size_t(std::max(blocks, 1)) * sizeof(EncBlockMeta));
        grow(ctx, ctx->enc_bases, ctx->enc_bases_cap, size_t(std::max(blocks, 1)) * 3u * size_t(dim));
    }
    grow(ctx, ctx->app_jobs, ctx->app_jobs_cap, dj.size() * sizeof(AppendJobDev));
    kvexp_dev::EncLookback lb{};
    if (fused) lb = lookback_for(ctx, int(dj.size()), blocks);
    scratch_acquire(ctx, s);
    // pageable source: the runtime has consumed it when the call returns (a
    // copy from pinned memory measured slower in the stream: 433 against
    // 342 us per c2 prefill call)
    HIPX(hipMemcpyAsync(ctx->app_jobs.p, dj.data(), dj.size() * sizeof(AppendJobDev), hipMemcpyHostToDevice, s));
    HIPX(kvexp_launch::append(ctx->app_jobs.as<AppendJobDev>(), int(dj.size()), blocks, dim, bt,
                              ctx->enc_meta.as<EncBlockMeta>(), ctx->enc_bases.as<uint8_t>(),
                              ctx->status.as<uint32_t>(), s, one_block, ctx->enc_modes, fused ? &lb : nullptr,
                              max_nb));
    scratch_used(ctx, s);
}

void check_encoder_status(kvexp_hip_ctx *ctx, hipStream_t s) {
    uint32_t st = 0;
    HIPX(hipMemcpyAsync(&st, ctx->status.p, sizeof st, hipMemcpyDeviceToHost, s));
    HIPX(hipStreamSynchronize(s));
    if (st != 0u) {
        HIPX(hipMemsetAsync(ctx->status.p, 0, sizeof(uint32_t), s));
        HIPX(hipStreamSynchronize(s));
        if (st & kvexp_dev::kStLookback) ctx->enc_lb_dirty = true;
        fail(KVEXP_HIP_LOGIC_ERROR, encoder_status_message(st));
    }
}

} // namespace

int kvexp_hip_append(kvexp_hip_ctx *ctx, const uint16_t *d_new, int n_new, int n_tokens, int dim, int bt,
                     uint16_t *d_tail, uint8_t *d_blob, size_t capacity, int64_t *d_offsets,
                     int32_t *d_first_token, int index_capacity, size_t *bytes_out, void *stream) {
    return guarded([&] {
        if (ctx == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_append: null context");
        check_append_shape(dim, bt);
        kvexp_hip_append_job a{};
        a.d_new = d_new;
        a.n_new = n_new;
        a.n_tokens = n_tokens;
        a.d_tail = d_tail;
        a.d_blob = d_blob;
        a.capacity = capacity;
        a.d_offsets = d_offsets;
        a.d_first_token = d_first_token;
        a.index_capacity = index_capacity;
        DeviceGuard g(ctx->device);
        hipStream_t s = static_cast<hipStream_t>(stream);
        run_append(ctx, &a, 1, dim, bt, s);
        if (bytes_out != nullptr) {
            const int nb_all = kvexp_hip_block_count(n_tokens + n_new, bt);
            int64_t bytes = 0;
            HIPX(hipMemcpyAsync(&bytes, d_offsets + nb_all, sizeof bytes, hipMemcpyDeviceToHost, s));
            check_encoder_status(ctx, s);
            *bytes_out = size_t(bytes);
        }
    });
}

int kvexp_hip_append_batch(kvexp_hip_ctx *ctx, const kvexp_hip_append_job *jobs, int n_jobs, int dim, int bt,
                           int check, void *stream) {
    return guarded([&] {
        if (ctx == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_append: null context");
        if (n_jobs < 0 || (n_jobs > 0 && jobs == nullptr))
            fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_append: null argument");
        check_append_shape(dim, bt);
        DeviceGuard g(ctx->device);
        hipStream_t s = static_cast<hipStream_t>(stream);
        run_append(ctx, jobs, n_jobs, dim, bt, s);
        if (check) check_encoder_status(ctx, s);
    });
}

int kvexp_hip_decode(kvexp_hip_ctx *ctx, const uint8_t *d_blob, size_t bytes, const int64_t *d_offsets,
                     const int32_t *d_first_token, int n_blocks, int seq, int dim, uint16_t *d_out, int check,
                     void *stream) {
    return guarded([&] {
        if (ctx == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_decode: null context");
        if (seq < 0 || dim <= 0 || n_blocks < 0) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_decode: bad shape");
        if (dim % 4 != 0 || dim > kMaxDim)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_decode: head_dim must be a multiple of 4 and at most 256");
        if (seq == 0) return;
        if (d_blob == nullptr || d_offsets == nullptr || d_first_token == nullptr || d_out == nullptr)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_decode: null argument");
        DeviceGuard g(ctx->device);
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (check) {
            int32_t have = 0;
            HIPX(hipMemcpyAsync(&have, d_first_token + n_blocks, sizeof have, hipMemcpyDeviceToHost, s));
            HIPX(hipStreamSynchronize(s));
            if (have < seq) fail(KVEXP_HIP_FORMAT_ERROR, "xkv decode ran out of blocks");
        }
        scratch_acquire(ctx, s); // the status word is shared with the encoders
        HIPX(kvexp_launch::decode(d_blob, bytes, d_offsets, d_first_token, n_blocks, seq, dim, d_out,
                                  ctx->status.as<uint32_t>(), s));
        scratch_used(ctx, s);
        if (check) check_status_word(ctx->status.as<uint32_t>(), s);
    });
}

// ============================================================= attention ==
int kvexp_hip_suggest_splits(kvexp_hip_ctx *ctx, int n_heads, int seq, int split_tokens) {
    return kvexp_hip_suggest_splits_for(ctx, n_heads, seq, split_tokens, 64, 7, KVEXP_HIP_ORDER_SCALAR);
}

namespace {

// One round of the split kernel's resident waves: three single-wave splits
// per SIMD at head_dim 64 (two for 8 query rows, and for the AVX-512 order
// with 6 or more), two at head_dim 128. The uniform count is the largest one
// whose longest split is no longer than the mean split of one round
// (total tokens / resident waves): for equal lengths that is one full round,
// with no second, partly filled one; for ragged lengths the long heads are
// cut finer, and the shorter splits that come with it are dealt out by the
// dispatcher as waves retire.
int suggest_core(const kvexp_hip_ctx *ctx, int64_t total_tokens, int max_seq, int split_tokens, int dim, int n_q,
                 int order) {
    if (ctx == nullptr || total_tokens <= 0 || max_seq <= 0 || split_tokens <= 0) return 1;
    const int tiles = (max_seq + split_tokens - 1) / split_tokens;
    const int g = std::min(std::max(1, n_q), kMaxQPerLaunch);
    const int per_simd = dim == 256 ? 1 : (dim == 64 && g < 8 ? 3 : 2); // the wave kernel's occupancy (kWaveOcc)
    (void)order;
    const int64_t groups = (std::max(1, n_q) + kMaxQPerLaunch - 1) / kMaxQPerLaunch; // device heads per head
    const int64_t slots = int64_t(4) * per_simd * std::max(1, ctx->cu_count);
    const int64_t target = std::max<int64_t>(1, int64_t(max_seq) * slots / (total_tokens * groups));
    return int(std::max<int64_t>(1, std::min<int64_t>(tiles, target)));
}

} // namespace

int kvexp_hip_suggest_splits_for(kvexp_hip_ctx *ctx, int n_heads, int seq, int split_tokens, int dim, int n_q,
                                 int order) {
    if (n_heads <= 0 || seq <= 0) return 1;
    return suggest_core(ctx, int64_t(n_heads) * seq, seq, split_tokens, dim, n_q, order);
}

int kvexp_hip_suggest_splits_batch(kvexp_hip_ctx *ctx, int n_heads, const int *seqs, int split_tokens, int dim,
                                   int n_q, int order) {
    if (n_heads <= 0 || seqs == nullptr) return 1;
    int64_t total = 0;
    int max_seq = 0;
    for (int i = 0; i < n_heads; ++i) {
        if (seqs[i] <= 0) continue;
        total += seqs[i];
        max_seq = std::max(max_seq, seqs[i]);
    }
    return suggest_core(ctx, total, max_seq, split_tokens, dim, n_q, order);
}

namespace {

// Orders each query-row group's work items so that the waves sharing a SIMD
// carry similar work. The dispatcher places workgroup g on XCD g % 8 and the
// workgroups g, g + C, g + 2C, ... (C = CU count) on the same CU, one wave
// of each on every SIMD, and a SIMD issues its oldest wave first, so a SIMD
// is busy for the sum of its waves' work and the launch ends with the
// busiest SIMD. Cost of a split: its tokens plus its K and V escape words
// (about 1/15 token each, measured on c2: an escape costs ~5.7 SIMD cycles,
// a token ~85; plain BF16 heads: their tokens). Items are sorted by cost,
// cut into workgroup-sized groups,
// and the groups are dealt to the workgroup slots tier by tier, in forward
// order on even tiers and reversed on odd ones, so that each CU receives a
// mix of heavy and light groups. The merge follows split numbers, not item
// order, so the results do not depend on it.
void balance_items(kvexp_hip_plan &p, std::vector<WorkItem> &items, bool xkv, const int32_t *first_all,
                   const std::vector<size_t> &first_at, int n_q, int dim) {
    const int per_head = (n_q + kMaxQPerLaunch - 1) / kMaxQPerLaunch;
    const int wpw = kvexp_launch::wave_waves_per_wg(dim);
    const int C = std::max(1, p.ctx->cu_count);
    auto cost = [&](const WorkItem &w) {
        const int h = w.head / per_head;
        double c = double(w.tok_end - w.tok_begin);
        for (int kv = 0; kv < (xkv ? 2 : 0); ++kv) {
            const size_t t = size_t(2 * h + kv);
            const int32_t *f0 = first_all + first_at[t];
            const int nb = p.jobs[t].n_blocks;
            const int b0 = kv ? w.vblk : w.kblk;
            const int b1 = int(std::lower_bound(f0, f0 + nb, w.tok_end) - f0);
            const int32_t *e = p.esc_prefix.data() + p.esc_prefix_at[t];
            c += double(e[b1] - e[b0]) / 15.0;
        }
        return c;
    };
    for (int G = 1; G <= 8; ++G) {
        const int b = p.group_start[G], e = p.group_start[G + 1];
        const int n = e - b;
        if (n <= wpw || n % wpw != 0) continue; // whole workgroups only
        std::vector<std::pair<double, int>> order(static_cast<size_t>(n));
        for (int i = 0; i < n; ++i) order[size_t(i)] = {cost(items[size_t(b + i)]), i};
        std::stable_sort(order.begin(), order.end(), [](const auto &x, const auto &y) { return x.first > y.first; });
        const int n_groups = (n + wpw - 1) / wpw;
        std::vector<int> slot_of_group(static_cast<size_t>(n_groups));
        for (int t0 = 0; t0 < n_groups; t0 += C) {
            const int cnt = std::min(C, n_groups - t0);
            const bool rev = (t0 / C) % 2 == 1;
            for (int k = 0; k < cnt; ++k) slot_of_group[size_t(t0 + k)] = t0 + (rev ? cnt - 1 - k : k);
        }
        std::vector<WorkItem> out(static_cast<size_t>(n));
        std::vector<int> fill(size_t(n_groups), 0);
        for (int r = 0; r < n; ++r) {
            const int gq = r / wpw;
            const int slot = slot_of_group[size_t(gq)];
            out[size_t(slot * wpw + fill[size_t(slot)]++)] = items[size_t(b + order[size_t(r)].second)];
        }
        std::copy(out.begin(), out.end(), items.begin() + b);
    }
}

// Builds every device-side part of a fresh plan from its heads: work items
// (token_bounds splits, split starts checked against the block index), device
// heads, merge work, and for the one-wave kernel the block descriptors and
// escape records. Stream-ordered on `s`: it first waits for the work
// already queued there (the encodes or appends that wrote the containers and
// indexes it reads) and synchronises only `s`. Status words: the plan's own.
void plan_build(kvexp_hip_plan *p, const kvexp_hip_head *heads, int n_heads, hipStream_t s) {
    kvexp_hip_ctx *ctx = p->ctx;
    p->status = p->alloc(sizeof(uint32_t));
    HIPX(hipMemsetAsync(p->status.p, 0, sizeof(uint32_t), s));
    const int n_q = p->n_q, dim = p->dim, split_tokens = p->split_tokens;
    const bool xkv = heads[0].k_xkv != nullptr;
    std::vector<HeadDev> hv;
    std::vector<WorkItem> items;
    std::vector<int32_t> merge;
    int ws_slots = 0;
    // every XKV head's block first tokens, read with one synchronisation
    std::vector<size_t> first_at(size_t(n_heads) * 2, 0);
    std::vector<int32_t> firsts;
    const int32_t *first_all = nullptr;
    if (xkv) {
        size_t total = 0;
        for (int h = 0; h < n_heads; ++h) {
            const kvexp_hip_head &H = heads[h];
            if (H.k_xkv == nullptr || H.k_offsets == nullptr || H.v_offsets == nullptr ||
                H.k_first_token == nullptr || H.v_first_token == nullptr || H.k_n_blocks <= 0 || H.v_n_blocks <= 0)
                break; // reported below, head by head
            first_at[size_t(2 * h)] = total;
            total += size_t(H.k_n_blocks) + 1;
            first_at[size_t(2 * h + 1)] = total;
            total += size_t(H.v_n_blocks) + 1;
        }
        if (total * 4 > ctx->pinned_cap) {
            if (ctx->pinned) HIPX(hipHostFree(ctx->pinned));
            ctx->pinned = nullptr;
            ctx->pinned_cap = 0;
            HIPX(hipHostMalloc(&ctx->pinned, total * 4, hipHostMallocDefault));
            ctx->pinned_cap = total * 4;
        }
        int32_t *host = static_cast<int32_t *>(ctx->pinned);
        for (int h = 0; h < n_heads; ++h) {
            const kvexp_hip_head &H = heads[h];
            if (H.k_xkv == nullptr || H.k_offsets == nullptr || H.v_offsets == nullptr ||
                H.k_first_token == nullptr || H.v_first_token == nullptr || H.k_n_blocks <= 0 || H.v_n_blocks <= 0)
                break;
            HIPX(hipMemcpyAsync(host + first_at[size_t(2 * h)], H.k_first_token, (size_t(H.k_n_blocks) + 1) * 4,
                                hipMemcpyDeviceToHost, s));
            HIPX(hipMemcpyAsync(host + first_at[size_t(2 * h + 1)], H.v_first_token, (size_t(H.v_n_blocks) + 1) * 4,
                                hipMemcpyDeviceToHost, s));
        }
        HIPX(hipStreamSynchronize(s));
        firsts.assign(host, host + total);
        first_all = firsts.data();
    }
    for (int h = 0; h < n_heads; ++h) {
        const kvexp_hip_head &H = heads[h];
        const bool raw = H.k_raw != nullptr, x = H.k_xkv != nullptr;
        if (H.seq <= 0) fail(KVEXP_HIP_INVALID_ARGUMENT, "attention_decode: bad argument");
        if (raw == x || (H.v_raw != nullptr) != raw || (H.v_xkv != nullptr) != x)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "attention_decode: pass raw K and V or xkv K and V, not both");
        if (x != xkv) fail(KVEXP_HIP_UNSUPPORTED, "kvexp_hip_plan_create: one plan holds raw or XKV heads, not both");
        const int ntiles = (H.seq + split_tokens - 1) / split_tokens;
        const int n_splits = std::min(std::max(1, H.n_splits), ntiles);
        if (x) {
            if (H.k_offsets == nullptr || H.v_offsets == nullptr || H.k_first_token == nullptr ||
                H.v_first_token == nullptr || H.k_n_blocks <= 0 || H.v_n_blocks <= 0)
                fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_plan_create: XKV head without a block index");
        }
        const int32_t *kf0 = x ? first_all + first_at[size_t(2 * h)] : nullptr;
        const int32_t *vf0 = x ? first_all + first_at[size_t(2 * h + 1)] : nullptr;
        const int32_t *kf1 = x ? kf0 + H.k_n_blocks : nullptr; // last entry: tokens covered
        const int32_t *vf1 = x ? vf0 + H.v_n_blocks : nullptr;
        if (x && (*kf1 < H.seq || *vf1 < H.seq)) fail(KVEXP_HIP_FORMAT_ERROR, "xkv ran out of tokens");
        // query rows in groups of <= 8 per device head, same splits
        for (int q0 = 0; q0 < n_q; q0 += kMaxQPerLaunch) {
            HeadDev d{};
            d.kx = H.k_xkv;
            d.vx = H.v_xkv;
            d.kbytes = H.k_bytes;
            d.vbytes = H.v_bytes;
            d.koff = H.k_offsets;
            d.voff = H.v_offsets;
            d.kfirst = H.k_first_token;
            d.vfirst = H.v_first_token;
            d.kraw = H.k_raw;
            d.vraw = H.v_raw;
            d.seq = H.seq;
            d.n_splits = n_splits;
            d.ws_base = ws_slots;
            d.q_row = h * n_q + q0;
            d.n_q = std::min(kMaxQPerLaunch, n_q - q0);
            const int dh = int(hv.size());
            for (int sp = 0; sp < n_splits; ++sp) {
                WorkItem wi{};
                wi.head = dh;
                wi.split = sp;
                token_bounds(H.seq, split_tokens, sp, n_splits, wi.tok_begin, wi.tok_end);
                wi.kblk = wi.vblk = -1;
                wi.kdi = wi.vdi = -1;
                if (x) {
                    const int32_t *kit = std::lower_bound(kf0, kf1, wi.tok_begin);
                    const int32_t *vit = std::lower_bound(vf0, vf1, wi.tok_begin);
                    if (kit == kf1 || *kit != wi.tok_begin || vit == vf1 || *vit != wi.tok_begin)
                        fail(KVEXP_HIP_FORMAT_ERROR, "token split is not aligned to an encoded block");
                    wi.kblk = int(kit - kf0);
                    wi.vblk = int(vit - vf0);
                }
                items.push_back(wi);
            }
            if (n_splits > 1) {
                merge.push_back(dh);
                ws_slots += n_splits;
            }
            hv.push_back(d);
        }
    }
    p->xkv = xkv;
    p->wave = kvexp_launch::wave_supports(dim);
    p->n_dev_heads = int(hv.size());
    p->n_items = int(items.size());
    p->n_merge = int(merge.size());
    if (p->wave) {
        // items grouped by G (one launch per distinct G)
        std::stable_sort(items.begin(), items.end(), [&](const WorkItem &a, const WorkItem &b) {
            return hv[size_t(a.head)].n_q < hv[size_t(b.head)].n_q;
        });
        for (int G = 0; G <= 8; ++G)
            p->group_start[G + 1] =
                int(std::count_if(items.begin(), items.end(),
                                  [&](const WorkItem &w) { return hv[size_t(w.head)].n_q <= G; }));
        std::vector<kvexp_dev::MergeItem> mi;
        for (int32_t dh : merge) {
            const HeadDev &d = hv[size_t(dh)];
            for (int g = 0; g < d.n_q; ++g) mi.push_back(kvexp_dev::MergeItem{d.ws_base, d.n_splits, d.q_row, g});
        }
        p->n_mitems = int(mi.size());
        // every merged device head with the same query rows and splits, its
        // slots and output rows one after another: the kernel then builds
        // item i from i instead of loading it
        p->merge_uni = kvexp_dev::MergeItem{};
        if (!mi.empty()) {
            const kvexp_dev::MergeItem f = mi[0];
            const int G = hv[size_t(merge[0])].n_q;
            bool uni = true;
            for (size_t i = 0; i < mi.size() && uni; ++i) {
                const int32_t k = int32_t(i) / G;
                uni = mi[i].ws_base == f.ws_base + k * f.n_splits && mi[i].n_splits == f.n_splits &&
                      mi[i].q_row == f.q_row + k * G && mi[i].g == int32_t(i) % G;
            }
            if (uni) p->merge_uni = kvexp_dev::MergeItem{f.ws_base, f.n_splits, f.q_row, G};
        }
        p->mitems = p->alloc(std::max<size_t>(1, mi.size()) * sizeof(kvexp_dev::MergeItem));
        if (!mi.empty())
            HIPX(hipMemcpyAsync(p->mitems.p, mi.data(), mi.size() * sizeof(kvexp_dev::MergeItem),
                                hipMemcpyHostToDevice, s));
        if (xkv) {
            build_escape_index(*p, heads, n_heads, n_q, dim, hv, s);
            balance_items(*p, items, true, first_all, first_at, n_q, dim);
            // the split's first descriptors as indexes into the plan's array
            // (device head dh belongs to user head dh / per_head)
            const int per_head = (n_q + kMaxQPerLaunch - 1) / kMaxQPerLaunch;
            for (WorkItem &w : items) {
                const int h = w.head / per_head;
                w.kdi = int(p->esc_prefix_at[size_t(2 * h)]) + w.kblk;
                w.vdi = int(p->esc_prefix_at[size_t(2 * h + 1)]) + w.vblk;
            }
        } else {
            balance_items(*p, items, false, nullptr, std::vector<size_t>(), n_q, dim);
        }
    }
    p->heads = p->alloc(hv.size() * sizeof(HeadDev));
    p->items = p->alloc(items.size() * sizeof(WorkItem));
    p->merge_ids = p->alloc(std::max<size_t>(1, merge.size()) * sizeof(int32_t));
    const size_t slot_floats = size_t(kMaxQPerLaunch) * size_t(dim + 2);
    p->ws = p->alloc(std::max<size_t>(1, size_t(ws_slots)) * slot_floats * sizeof(float));
    HIPX(hipMemcpyAsync(p->heads.p, hv.data(), hv.size() * sizeof(HeadDev), hipMemcpyHostToDevice, s));
    HIPX(hipMemcpyAsync(p->items.p, items.data(), items.size() * sizeof(WorkItem), hipMemcpyHostToDevice, s));
    if (!merge.empty())
        HIPX(hipMemcpyAsync(p->merge_ids.p, merge.data(), merge.size() * sizeof(int32_t), hipMemcpyHostToDevice, s));
    if (!xkv) { // the job table kvexp_hip_plan_update sends lengths through
        p->jobs.assign(size_t(2 * n_heads), kvexp_dev::EscJob{});
        p->djobs = p->alloc(p->jobs.size() * sizeof(kvexp_dev::EscJob));
    }
    p->src.assign(heads, heads + n_heads);
    HIPX(hipStreamSynchronize(s)); // the host vectors above are the copies' sources
}

// Moves a freshly built plan's device state into `dst` (an update that
// succeeded); the old state goes to `src` and is freed with it.
void swap_built(kvexp_hip_plan &dst, kvexp_hip_plan &src) {
    using std::swap;
    swap(dst.xkv, src.xkv);
    swap(dst.src, src.src);
    swap(dst.jobs, src.jobs);
    swap(dst.esc_prefix, src.esc_prefix);
    swap(dst.esc_prefix_at, src.esc_prefix_at);
    swap(dst.djobs, src.djobs);
    swap(dst.wave, src.wave);
    swap(dst.heads, src.heads);
    swap(dst.items, src.items);
    swap(dst.merge_ids, src.merge_ids);
    swap(dst.ws, src.ws);
    swap(dst.status, src.status);
    swap(dst.mitems, src.mitems);
    swap(dst.esc0, src.esc0);
    swap(dst.escpos, src.escpos);
    swap(dst.desc, src.desc);
    swap(dst.n_mitems, src.n_mitems);
    swap(dst.merge_uni, src.merge_uni);
    swap(dst.n_dev_heads, src.n_dev_heads);
    swap(dst.n_items, src.n_items);
    swap(dst.n_merge, src.n_merge);
    for (int i = 0; i < 10; ++i) swap(dst.group_start[i], src.group_start[i]);
}

} // namespace

namespace {
// kvexp_hip_plan_create's checks and build (throws); `pooled`: the plan's
// buffers come from and return to the context's pool.
kvexp_hip_plan *plan_create(kvexp_hip_ctx *ctx, const kvexp_hip_head *heads, int n_heads, int n_q, int dim,
                            int split_tokens, int order, hipStream_t stream, bool pooled) {
    if (ctx == nullptr || heads == nullptr || n_heads <= 0 || n_q <= 0 || dim <= 0 || split_tokens <= 0)
        fail(KVEXP_HIP_INVALID_ARGUMENT, "attention_decode: bad argument");
    if (order != KVEXP_HIP_ORDER_SCALAR && order != KVEXP_HIP_ORDER_DPBF16)
        fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_plan_create: unknown score order");
    // attention_scalar.cpp:47-49 / attention_avx512.cpp:155-157
    if (order == KVEXP_HIP_ORDER_SCALAR && (dim % 8 != 0 || dim > kMaxDim))
        fail(KVEXP_HIP_INVALID_ARGUMENT, "scalar attention: bad shape");
    if (order == KVEXP_HIP_ORDER_DPBF16 && (dim % 32 != 0 || dim > kMaxDim))
        fail(KVEXP_HIP_INVALID_ARGUMENT, "avx512 attention: head_dim must be a multiple of 32");
    DeviceGuard g(ctx->device);
    auto *p = new kvexp_hip_plan();
    try {
        p->ctx = ctx;
        p->pooled = pooled;
        p->n_heads = n_heads;
        p->n_q = n_q;
        p->dim = dim;
        p->order = order;
        p->split_tokens = split_tokens;
        plan_build(p, heads, n_heads, stream);
    } catch (...) {
        delete p;
        throw;
    }
    return p;
}
} // namespace

int kvexp_hip_plan_create(kvexp_hip_ctx *ctx, const kvexp_hip_head *heads, int n_heads, int n_q, int dim,
                          int split_tokens, int order, void *stream, kvexp_hip_plan **out) {
    return guarded([&] {
        if (out == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_plan_create: null output");
        *out = nullptr;
        *out = plan_create(ctx, heads, n_heads, n_q, dim, split_tokens, order, static_cast<hipStream_t>(stream),
                           false);
    });
}

// After appends: the same heads with new lengths. The split partition is
// unchanged unless a head gains a split tile or a block; then (every
// block_tokens tokens of a decode loop) the plan is built again. Otherwise
// only the last split of each head ends later, and only the last block of
// each container changed (kvexp_hip_append rewrites nothing before it): its
// descriptor and escape records are rewritten on the GPU, the device heads
// and work items are uploaded again, all on `stream`.
int kvexp_hip_plan_update(kvexp_hip_plan *plan, const kvexp_hip_head *heads, int n_heads, void *stream) {
    return guarded([&] {
        if (plan == nullptr || heads == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "attention_decode: bad argument");
        if (n_heads != plan->n_heads)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_plan_update: the heads of the plan, with new lengths");
        DeviceGuard g(plan->ctx->device);
        hipStream_t s = static_cast<hipStream_t>(stream);
        const int st = plan->split_tokens;
        bool fast = plan->wave || !plan->xkv;
        for (int h = 0; h < n_heads; ++h) {
            const kvexp_hip_head &a = heads[h], &b = plan->src[size_t(h)];
            if (a.k_xkv != b.k_xkv || a.v_xkv != b.v_xkv || a.k_raw != b.k_raw || a.v_raw != b.v_raw ||
                a.k_offsets != b.k_offsets || a.v_offsets != b.v_offsets || a.k_first_token != b.k_first_token ||
                a.v_first_token != b.v_first_token || a.n_splits != b.n_splits)
                fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_plan_update: the heads of the plan, with new lengths");
            if (a.seq <= 0) fail(KVEXP_HIP_INVALID_ARGUMENT, "attention_decode: bad argument");
            if ((a.seq + st - 1) / st != (b.seq + st - 1) / st || a.k_n_blocks != b.k_n_blocks ||
                a.v_n_blocks != b.v_n_blocks)
                fast = false;
        }
        // From here on the containers have changed under the plan: a failure
        // leaves the plan refusing runs until an update succeeds.
        try {
            if (!fast) {
                // a new plan is built aside (its build first waits for the work
                // queued on s, runs included, which still read the old buffers)
                // and swapped in only when it is complete
                kvexp_hip_plan np;
                np.ctx = plan->ctx;
                np.pooled = plan->pooled;
                np.n_heads = plan->n_heads;
                np.n_q = plan->n_q;
                np.dim = plan->dim;
                np.order = plan->order;
                np.split_tokens = plan->split_tokens;
                plan_build(&np, heads, n_heads, s);
                swap_built(*plan, np);
                plan->invalid = false;
                plan->invalid_msg.clear();
                return;
            }
            // the device heads' lengths and byte counts and the last splits' ends
            // are set on the GPU from the jobs, with the last blocks' descriptors
            const int per_head = (plan->n_q + kMaxQPerLaunch - 1) / kMaxQPerLaunch;
            for (int h = 0; h < n_heads; ++h)
                for (int kv = 0; kv < 2; ++kv) {
                    kvexp_dev::EscJob &j = plan->jobs[size_t(2 * h + kv)];
                    j.bytes = kv ? heads[h].v_bytes : heads[h].k_bytes;
                    j.seq = heads[h].seq;
                }
            HIPX(hipMemcpyAsync(plan->djobs.p, plan->jobs.data(), plan->jobs.size() * sizeof(kvexp_dev::EscJob),
                                hipMemcpyHostToDevice, s));
            HIPX(kvexp_launch::plan_refresh(plan->djobs.as<kvexp_dev::EscJob>(),
                                            plan->xkv ? int(plan->jobs.size()) : 0, plan->heads.as<HeadDev>(),
                                            plan->n_dev_heads, plan->items.as<WorkItem>(), plan->n_items, per_head,
                                            plan->status.as<uint32_t>(), s));
            plan->src.assign(heads, heads + n_heads);
            plan->invalid = false;
            plan->invalid_msg.clear();
        } catch (const KvexpFail &f) {
            plan->invalid = true;
            plan->invalid_msg = f.msg;
            throw;
        } catch (const HipFail &h) {
            plan->invalid = true;
            plan->invalid_msg = std::string(h.what) + ": " + hipGetErrorString(h.err);
            throw;
        } catch (...) {
            plan->invalid = true;
            plan->invalid_msg = "update failed";
            throw;
        }
    });
}

int kvexp_hip_plan_destroy(kvexp_hip_plan *plan) {
    return guarded([&] {
        if (plan == nullptr) return;
        DeviceGuard g(plan->ctx->device);
        delete plan;
    });
}

int kvexp_hip_attention_run(kvexp_hip_plan *plan, const uint16_t *d_q, float *d_out, float *d_lse, int check,
                            void *stream) {
    return guarded([&] {
        if (plan == nullptr || d_q == nullptr || d_out == nullptr)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "attention_decode: bad argument");
        if (plan->invalid)
            fail(KVEXP_HIP_FORMAT_ERROR, "plan is stale after a failed kvexp_hip_plan_update (" + plan->invalid_msg +
                                             "); update it again before running");
        DeviceGuard g(plan->ctx->device);
        hipStream_t s = static_cast<hipStream_t>(stream);
        hipEvent_t ev0 = nullptr, ev1 = nullptr;
        if (plan->timing) {
            HIPX(hipEventCreate(&ev0));
            if (hipEventCreate(&ev1) != hipSuccess) {
                (void)hipEventDestroy(ev0);
                fail(KVEXP_HIP_DEVICE_ERROR, "hipEventCreate failed");
            }
            plan->events.emplace_back(ev0, ev1);
        }
        if (plan->wave) {
            if (ev0) HIPX(hipEventRecord(ev0, s));
            for (int G = 1; G <= 8; ++G) {
                const int b = plan->group_start[G], e = plan->group_start[G + 1];
                if (e > b)
                    // a group with no more items than CUs: one wave per
                    // workgroup, up to twice as many: two, so that its items
                    // spread over every CU (else the kernel's own count)
                    HIPX(kvexp_launch::attention_wave(plan->xkv, plan->order, G, plan->dim, plan->heads.as<HeadDev>(),
                                                      plan->items.as<WorkItem>() + b, e - b,
                                                      e - b <= plan->ctx->cu_count ? 1
                                                      : e - b <= 2 * plan->ctx->cu_count ? 2 : 0,
                                                      plan->desc.as<kvexp_dev::BlockDesc>(), d_q, d_out, d_lse,
                                                      plan->ws.as<float>(), s));
            }
            if (ev1) HIPX(hipEventRecord(ev1, s));
            HIPX(kvexp_launch::wave_merge(plan->dim, plan->mitems.as<kvexp_dev::MergeItem>(), plan->n_mitems,
                                          plan->merge_uni, d_out,
                                          d_lse, plan->ws.as<float>(), s));
        } else {
            if (ev0) HIPX(hipEventRecord(ev0, s));
            HIPX(kvexp_launch::attention(plan->xkv, plan->order, plan->heads.as<HeadDev>(),
                                         plan->items.as<WorkItem>(), plan->n_items, plan->merge_ids.as<int32_t>(),
                                         plan->n_merge, d_q, d_out, d_lse, plan->ws.as<float>(), plan->dim,
                                         plan->status.as<uint32_t>(), s));
            if (ev1) HIPX(hipEventRecord(ev1, s));
        }
        if (check) check_status_word(plan->status.as<uint32_t>(), s);
    });
}

int kvexp_hip_plan_timing(kvexp_hip_plan *plan, int enable) {
    return guarded([&] {
        if (plan == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_plan_timing: null plan");
        DeviceGuard g(plan->ctx->device);
        plan->timing = enable != 0;
    });
}

int kvexp_hip_plan_kernel_time(kvexp_hip_plan *plan, double *ms, int *runs) {
    return guarded([&] {
        if (plan == nullptr || ms == nullptr || runs == nullptr)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_plan_kernel_time: bad argument");
        DeviceGuard g(plan->ctx->device);
        double total = 0.0;
        for (auto &e : plan->events) {
            HIPX(hipEventSynchronize(e.second));
            float t = 0.0f;
            HIPX(hipEventElapsedTime(&t, e.first, e.second));
            total += double(t);
        }
        *ms = total;
        *runs = int(plan->events.size());
        plan->clear_events();
    });
}

int kvexp_hip_plan_status(kvexp_hip_plan *plan, void *stream) {
    return guarded([&] {
        if (plan == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_plan_status: null plan");
        DeviceGuard g(plan->ctx->device);
        check_status_word(plan->status.as<uint32_t>(), static_cast<hipStream_t>(stream));
    });
}

int kvexp_hip_attention_decode_host(kvexp_hip_ctx *ctx, int order, const uint16_t *q, const uint16_t *k_raw,
                                    const uint16_t *v_raw, const uint8_t *k_xkv, size_t k_bytes,
                                    const uint8_t *v_xkv, size_t v_bytes, float *out, int n_q, int dim, int seq,
                                    int n_threads, int split_tokens) {
    return guarded([&] {
        // dispatch.cpp:31-38
        if (q == nullptr || out == nullptr || n_q <= 0 || dim <= 0 || seq <= 0 || split_tokens <= 0)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "attention_decode: bad argument");
        const bool raw = k_raw != nullptr, x = k_xkv != nullptr;
        if (raw == x || (v_raw != nullptr) != raw || (v_xkv != nullptr) != x)
            fail(KVEXP_HIP_INVALID_ARGUMENT, "attention_decode: pass raw K and V or xkv K and V, not both");
        if (ctx == nullptr) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_attention_decode_host: null context");
        if (order == KVEXP_HIP_ORDER_SCALAR && (dim % 8 != 0 || dim > kMaxDim))
            fail(KVEXP_HIP_INVALID_ARGUMENT, "scalar attention: bad shape");
        if (order == KVEXP_HIP_ORDER_DPBF16 && (dim % 32 != 0 || dim > kMaxDim))
            fail(KVEXP_HIP_INVALID_ARGUMENT, "avx512 attention: head_dim must be a multiple of 32");
        DeviceGuard g(ctx->device);
        // everything on the context's own stream: concurrent calls on other
        // contexts neither wait for this one nor see its status words. Device
        // buffers (staging and the plan's) come from the context's pool and go
        // back to it once the stream is synchronised: after the first calls of
        // a shape no call allocates or frees device memory.
        hipStream_t s = ctx->stream;
        DevPool *pool = &ctx->pool;
        const size_t qn = size_t(n_q) * size_t(dim);
        DevBuf dq(pool, qn * 2), dout(pool, qn * 4);
        HIPX(hipMemcpyAsync(dq.p, q, qn * 2, hipMemcpyHostToDevice, s));
        kvexp_hip_head H{};
        H.seq = seq;
        H.n_splits = n_threads;
        DevBuf dk, dv, kio, kif, vio, vif;
        // declared after the buffers, so destroyed first: on an early failure
        // the copies and kernels queued with them finish before they are
        // released (and the plan is destroyed before the buffers it reads)
        struct SyncOnExit {
            hipStream_t s;
            ~SyncOnExit() { (void)hipStreamSynchronize(s); }
        } sync_on_exit{s};
        if (raw) {
            const size_t nb = size_t(seq) * size_t(dim) * 2u;
            dk = DevBuf(pool, nb);
            dv = DevBuf(pool, nb);
            HIPX(hipMemcpyAsync(dk.p, k_raw, nb, hipMemcpyHostToDevice, s));
            HIPX(hipMemcpyAsync(dv.p, v_raw, nb, hipMemcpyHostToDevice, s));
            H.k_raw = dk.as<uint16_t>();
            H.v_raw = dv.as<uint16_t>();
        } else {
            std::vector<int64_t> ko, vo;
            std::vector<int32_t> kf, vf;
            walk_index(k_xkv, k_bytes, dim, seq, ko, kf);
            walk_index(v_xkv, v_bytes, dim, seq, vo, vf);
            if (kf.back() < seq || vf.back() < seq)
                fail(KVEXP_HIP_FORMAT_ERROR, "xkv ran out of tokens");
            dk = DevBuf(pool, std::max<size_t>(k_bytes, 4));
            dv = DevBuf(pool, std::max<size_t>(v_bytes, 4));
            HIPX(hipMemcpyAsync(dk.p, k_xkv, k_bytes, hipMemcpyHostToDevice, s));
            HIPX(hipMemcpyAsync(dv.p, v_xkv, v_bytes, hipMemcpyHostToDevice, s));
            kio = DevBuf(pool, ko.size() * 8);
            kif = DevBuf(pool, kf.size() * 4);
            vio = DevBuf(pool, vo.size() * 8);
            vif = DevBuf(pool, vf.size() * 4);
            HIPX(hipMemcpyAsync(kio.p, ko.data(), ko.size() * 8, hipMemcpyHostToDevice, s));
            HIPX(hipMemcpyAsync(kif.p, kf.data(), kf.size() * 4, hipMemcpyHostToDevice, s));
            HIPX(hipMemcpyAsync(vio.p, vo.data(), vo.size() * 8, hipMemcpyHostToDevice, s));
            HIPX(hipMemcpyAsync(vif.p, vf.data(), vf.size() * 4, hipMemcpyHostToDevice, s));
            H.k_xkv = dk.as<uint8_t>();
            H.v_xkv = dv.as<uint8_t>();
            H.k_bytes = k_bytes;
            H.v_bytes = v_bytes;
            H.k_offsets = kio.as<int64_t>();
            H.v_offsets = vio.as<int64_t>();
            H.k_first_token = kif.as<int32_t>();
            H.v_first_token = vif.as<int32_t>();
            H.k_n_blocks = int(ko.size()) - 1;
            H.v_n_blocks = int(vo.size()) - 1;
        }
        struct PlanOnExit {
            kvexp_hip_plan *p = nullptr;
            hipStream_t s;
            ~PlanOnExit() {
                if (p == nullptr) return;
                (void)hipStreamSynchronize(s); // its runs are finished before its buffers go back
                delete p;
            }
        } plan{nullptr, s};
        plan.p = plan_create(ctx, &H, 1, n_q, dim, split_tokens, order, s, true);
        const int rc = kvexp_hip_attention_run(plan.p, dq.as<uint16_t>(), dout.as<float>(), nullptr, 1, s);
        if (rc) fail(rc, g_error);
        HIPX(hipMemcpyAsync(out, dout.p, qn * 4, hipMemcpyDeviceToHost, s));
        HIPX(hipStreamSynchronize(s));
    });
}

int kvexp_hip_expf(kvexp_hip_ctx *ctx, const float *d_x, float *d_y, size_t n, void *stream) {
    return guarded([&] {
        if (ctx == nullptr || (n && (d_x == nullptr || d_y == nullptr)))
            fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_expf: null argument");
        if (n > (size_t(1) << 40)) fail(KVEXP_HIP_INVALID_ARGUMENT, "kvexp_hip_expf: n too large");
        DeviceGuard g(ctx->device);
        HIPX(kvexp_launch::expf(d_x, d_y, n, static_cast<hipStream_t>(stream)));
    });
}

} // extern "C"
