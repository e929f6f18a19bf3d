// The kvexp C++ API (include/kvexp/*.hpp) over the C ABI, built as its own
// library (libkvexp_hip_cxx.so) so that libkvexp_hip.so exports C symbols
// only and links beside the reference library without a clash.
//
// Host buffers in and out; C ABI status codes become the reference's
// exception classes again. Like the reference's attention_decode and
// encode_bf16 (src/dispatch.cpp:27-104, src/codec.cpp:39-164), every entry
// is reentrant: a call leases a context (device workspace, status words and
// a non-blocking stream) from a per-device pool for its whole duration, so
// concurrent calls never share mutable device state, and every copy and
// launch of a call is ordered on its lease's stream alone (no device-wide
// synchronisation). The pool grows to the largest number of concurrent
// calls and keeps its contexts until the process ends.
#include "kvexp/attention.hpp"
#include "kvexp/codec.hpp"
#include "kvexp_hip.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace kvexp {
namespace {

std::atomic<int> g_device{0};

[[noreturn]] void raise(int rc) {
    const std::string msg = kvexp_hip_last_error();
    switch (rc) {
    case KVEXP_HIP_INVALID_ARGUMENT: throw std::invalid_argument(msg);
    case KVEXP_HIP_LOGIC_ERROR: throw std::logic_error(msg);
    default: throw std::runtime_error(msg);
    }
}

void check(int rc) {
    if (rc != KVEXP_HIP_OK) raise(rc);
}

void hip(hipError_t e) {
    if (e != hipSuccess) throw std::runtime_error(std::string("HIP: ") + hipGetErrorString(e));
}

struct Slot {
    kvexp_hip_ctx *ctx = nullptr;
    hipStream_t stream = nullptr; // copies and codec launches of the lease holder
};

// Idle contexts per device. Contexts are created outside the lock; a slot is
// owned by exactly one call between acquire and release.
class Pool {
  public:
    Slot acquire(int dev) {
        {
            std::lock_guard<std::mutex> lock(mu_);
            if (size_t(dev) < idle_.size() && !idle_[size_t(dev)].empty()) {
                Slot s = idle_[size_t(dev)].back();
                idle_[size_t(dev)].pop_back();
                return s;
            }
        }
        Slot s;
        check(kvexp_hip_ctx_create(dev, &s.ctx));
        int prev = 0;
        hip(hipGetDevice(&prev));
        hip(hipSetDevice(dev));
        const hipError_t e = hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking);
        (void)hipSetDevice(prev);
        if (e != hipSuccess) {
            (void)kvexp_hip_ctx_destroy(s.ctx);
            hip(e);
        }
        return s;
    }
    void release(int dev, Slot s) {
        std::lock_guard<std::mutex> lock(mu_);
        if (size_t(dev) >= idle_.size()) idle_.resize(size_t(dev) + 1);
        idle_[size_t(dev)].push_back(s);
    }

  private:
    std::mutex mu_;
    std::vector<std::vector<Slot>> idle_;
};

Pool &pool() {
    static Pool *p = new Pool(); // never destroyed: callers may run during exit
    return *p;
}

// A context for the duration of one call, on the caller's device choice.
struct Lease {
    int dev;
    int prev = 0;
    Slot slot;
    Lease() : dev(g_device.load()) {
        slot = pool().acquire(dev);
        if (hipGetDevice(&prev) != hipSuccess || hipSetDevice(dev) != hipSuccess) {
            pool().release(dev, slot);
            throw std::runtime_error("HIP: cannot select the device");
        }
    }
    ~Lease() {
        // the lease's work is finished before the slot is handed on
        (void)hipStreamSynchronize(slot.stream);
        (void)hipSetDevice(prev);
        pool().release(dev, slot);
    }
    Lease(const Lease &) = delete;
    Lease &operator=(const Lease &) = delete;
};

// Device allocation of one call; the lease's stream is synchronised before
// it is freed (declared after the Lease, so destroyed first, and every
// early exit syncs explicitly).
struct Dev {
    void *p = nullptr;
    hipStream_t s;
    Dev(size_t n, hipStream_t stream) : s(stream) { hip(hipMalloc(&p, n ? n : 4)); }
    ~Dev() {
        (void)hipStreamSynchronize(s);
        (void)hipFree(p);
    }
    Dev(const Dev &) = delete;
    Dev &operator=(const Dev &) = delete;
};

} // namespace

void set_device(int device) { g_device.store(device); }

CpuFeatures detect_cpu() {
    CpuFeatures f;
#if defined(__x86_64__)
    __builtin_cpu_init();
    f.avx2 = __builtin_cpu_supports("avx2");
    f.avx512_bf16 = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                    __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512bf16");
#endif
    return f;
}

EncodedTensor encode_bf16(const uint16_t *kv, int seq_len, int head_dim, int block_tokens) {
    Lease L;
    const hipStream_t s = L.slot.stream;
    const int64_t bound = kvexp_hip_encode_bound(seq_len, head_dim, block_tokens);
    const size_t in_bytes = (seq_len > 0 && head_dim > 0) ? size_t(seq_len) * size_t(head_dim) * 2u : 0u;
    Dev din(in_bytes, s), dout(size_t(bound > 0 ? bound : 0), s);
    if (kv != nullptr && in_bytes) hip(hipMemcpyAsync(din.p, kv, in_bytes, hipMemcpyHostToDevice, s));
    size_t n = 0;
    check(kvexp_hip_encode(L.slot.ctx, kv ? static_cast<const uint16_t *>(din.p) : nullptr, seq_len, head_dim,
                           block_tokens, static_cast<uint8_t *>(dout.p), size_t(bound > 0 ? bound : 0), nullptr,
                           nullptr, &n, s));
    EncodedTensor e;
    e.seq_len = seq_len;
    e.head_dim = head_dim;
    e.block_tokens = block_tokens;
    e.bytes.resize(n);
    if (n) hip(hipMemcpyAsync(e.bytes.data(), dout.p, n, hipMemcpyDeviceToHost, s));
    hip(hipStreamSynchronize(s));
    return e;
}

void decode_bf16(const uint8_t *blob, size_t bytes, int seq_len, int head_dim, uint16_t *out) {
    const int cap = int(bytes / 8 + 2);
    std::vector<int64_t> off(size_t(cap) + 1);
    std::vector<int32_t> first(size_t(cap) + 1);
    int nb = 0;
    check(kvexp_hip_build_index(blob, bytes, head_dim, seq_len, off.data(), first.data(), cap, &nb));
    if (first[size_t(nb)] < seq_len) throw std::runtime_error("xkv decode ran out of blocks");
    if (seq_len <= 0) return;
    Lease L;
    const hipStream_t s = L.slot.stream;
    const size_t out_bytes = size_t(seq_len) * size_t(head_dim) * 2u;
    Dev db(bytes, s), doff(size_t(nb + 1) * 8, s), dfirst(size_t(nb + 1) * 4, s), dout(out_bytes, s);
    hip(hipMemcpyAsync(db.p, blob, bytes, hipMemcpyHostToDevice, s));
    hip(hipMemcpyAsync(doff.p, off.data(), size_t(nb + 1) * 8, hipMemcpyHostToDevice, s));
    hip(hipMemcpyAsync(dfirst.p, first.data(), size_t(nb + 1) * 4, hipMemcpyHostToDevice, s));
    check(kvexp_hip_decode(L.slot.ctx, static_cast<const uint8_t *>(db.p), bytes,
                           static_cast<const int64_t *>(doff.p), static_cast<const int32_t *>(dfirst.p), nb, seq_len,
                           head_dim, static_cast<uint16_t *>(dout.p), 1, s));
    hip(hipMemcpyAsync(out, dout.p, out_bytes, hipMemcpyDeviceToHost, s));
    hip(hipStreamSynchronize(s));
}

void attention_decode(Backend backend, const uint16_t *q, const uint16_t *k_raw, const uint16_t *v_raw,
                      const uint8_t *k_xkv, size_t k_bytes, const uint8_t *v_xkv, size_t v_bytes, float *out,
                      int n_q, int dim, int seq, int n_threads, int split_tokens) {
    // dispatch.cpp:31-38: the argument checks come first, for every backend
    if (q == nullptr || out == nullptr || n_q <= 0 || dim <= 0 || seq <= 0 || split_tokens <= 0)
        throw std::invalid_argument("attention_decode: bad argument");
    if ((k_raw != nullptr) == (k_xkv != nullptr) || (v_raw != nullptr) != (k_raw != nullptr) ||
        (v_xkv != nullptr) != (k_xkv != nullptr))
        throw std::invalid_argument("attention_decode: pass raw K and V or xkv K and V, not both");
    // an unavailable backend is a runtime_error in the reference (dispatch.cpp:39-45)
    if (backend != Backend::Hip && backend != Backend::HipDpbf16)
        throw std::runtime_error("CPU backend requested but not available in libkvexp_hip_cxx (the reference "
                                 "library with its Backend::Hip dispatch case runs all backends)");
    const int order = backend == Backend::Hip ? KVEXP_HIP_ORDER_SCALAR : KVEXP_HIP_ORDER_DPBF16;
    Lease L;
    check(kvexp_hip_attention_decode_host(L.slot.ctx, order, q, k_raw, v_raw, k_xkv, k_bytes, v_xkv, v_bytes, out,
                                          n_q, dim, seq, n_threads, split_tokens));
}

} // namespace kvexp
