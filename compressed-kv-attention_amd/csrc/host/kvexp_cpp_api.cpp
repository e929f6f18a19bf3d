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
// launch of a call is ordered on its lease's stream alone. Device memory is
// grow-only (the lease's staging buffers here; the context's buffer pool in
// the attention entry): after the first calls of a shape no call allocates
// or frees device memory, so none waits on the implicit device-wide
// synchronisation of hipFree. The pool grows to the largest number of
// concurrent calls and keeps its contexts until the process ends.
#include "kvexp/attention.hpp"
#include "kvexp/codec.hpp"
#include "kvexp_hip.h"

#include <hip/hip_runtime.h>

#include <atomic>
#if defined(__x86_64__)
#include <cpuid.h>
#endif
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

// A grow-only device buffer of a slot: reallocated only when a call needs
// more than it holds (the slot's stream is then idle: a lease synchronises
// it before the slot is handed on), so after warm-up no call allocates or
// frees device memory.
struct Stage {
    void *p = nullptr;
    size_t cap = 0;
    void *get(size_t n) {
        n = n ? n : 4;
        if (n > cap) {
            if (p) hip(hipFree(p));
            p = nullptr;
            cap = 0;
            hip(hipMalloc(&p, n));
            cap = n;
        }
        return p;
    }
};

struct Slot {
    kvexp_hip_ctx *ctx = nullptr;
    hipStream_t stream = nullptr; // copies and codec launches of the lease holder
    Stage *stage = nullptr;       // four staging buffers of the codec calls
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
        s.stage = new Stage[4]; // kept with the slot until the process ends
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


} // namespace

void set_device(int device) { g_device.store(device); }

// The host's features with the reference's gates (src/cpu.cpp:35-61), which
// follow the Intel SDM: the OS must save the vector state (CPUID.1:ECX
// OSXSAVE and AVX, then XCR0 from xgetbv: bits 1-2 for YMM, and 5-7 as well
// for ZMM), and the instruction sets are CPUID.(7,0):EBX bit 5 (AVX2), bits
// 16, 30, 31 (AVX-512 F, BW, VL) and CPUID.(7,1):EAX bit 5 (AVX512_BF16).
// The GPU backends do not depend on it; it reports what the reference's
// CPU backends would accept on this host.
namespace {
struct CpuidBit {
    unsigned leaf, sub;
    int reg; // 0 eax, 1 ebx, 2 ecx, 3 edx
    unsigned bit;
};

#if defined(__x86_64__)
bool cpuid_has(const CpuidBit &b) {
    unsigned r[4] = {0, 0, 0, 0};
    if (__get_cpuid_max(0, nullptr) < b.leaf) return false;
    __cpuid_count(b.leaf, b.sub, r[0], r[1], r[2], r[3]);
    return (r[b.reg] >> b.bit) & 1u;
}

unsigned long long xcr0() {
    unsigned lo = 0, hi = 0;
    __asm__ volatile("xgetbv" : "=a"(lo), "=d"(hi) : "c"(0));
    return (static_cast<unsigned long long>(hi) << 32) | lo;
}
#endif
} // namespace

CpuFeatures detect_cpu() {
    CpuFeatures f;
#if defined(__x86_64__)
    if (!cpuid_has({1, 0, 2, 27}) || !cpuid_has({1, 0, 2, 28})) return f; // OSXSAVE, AVX
    const unsigned long long x = xcr0();
    const bool ymm_state = (x & 0x06u) == 0x06u;
    const bool zmm_state = (x & 0xE6u) == 0xE6u;
    f.avx2 = ymm_state && cpuid_has({7, 0, 1, 5});
    f.avx512_bf16 = zmm_state && cpuid_has({7, 0, 1, 16}) && cpuid_has({7, 0, 1, 30}) && cpuid_has({7, 0, 1, 31}) &&
                    cpuid_has({7, 1, 0, 5});
#endif
    return f;
}

EncodedTensor encode_bf16(const uint16_t *kv, int seq_len, int head_dim, int block_tokens) {
    Lease L;
    const hipStream_t s = L.slot.stream;
    const int64_t bound = kvexp_hip_encode_bound(seq_len, head_dim, block_tokens);
    const size_t in_bytes = (seq_len > 0 && head_dim > 0) ? size_t(seq_len) * size_t(head_dim) * 2u : 0u;
    void *din = L.slot.stage[0].get(in_bytes), *dout = L.slot.stage[1].get(size_t(bound > 0 ? bound : 0));
    if (kv != nullptr && in_bytes) hip(hipMemcpyAsync(din, kv, in_bytes, hipMemcpyHostToDevice, s));
    size_t n = 0;
    check(kvexp_hip_encode(L.slot.ctx, kv ? static_cast<const uint16_t *>(din) : nullptr, seq_len, head_dim,
                           block_tokens, static_cast<uint8_t *>(dout), size_t(bound > 0 ? bound : 0), nullptr,
                           nullptr, &n, s));
    EncodedTensor e;
    e.seq_len = seq_len;
    e.head_dim = head_dim;
    e.block_tokens = block_tokens;
    e.bytes.resize(n);
    if (n) hip(hipMemcpyAsync(e.bytes.data(), dout, n, hipMemcpyDeviceToHost, s));
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
    void *db = L.slot.stage[0].get(bytes), *doff = L.slot.stage[1].get(size_t(nb + 1) * 8),
         *dfirst = L.slot.stage[2].get(size_t(nb + 1) * 4), *dout = L.slot.stage[3].get(out_bytes);
    hip(hipMemcpyAsync(db, blob, bytes, hipMemcpyHostToDevice, s));
    hip(hipMemcpyAsync(doff, off.data(), size_t(nb + 1) * 8, hipMemcpyHostToDevice, s));
    hip(hipMemcpyAsync(dfirst, first.data(), size_t(nb + 1) * 4, hipMemcpyHostToDevice, s));
    check(kvexp_hip_decode(L.slot.ctx, static_cast<const uint8_t *>(db), bytes, static_cast<const int64_t *>(doff),
                           static_cast<const int32_t *>(dfirst), nb, seq_len, head_dim, static_cast<uint16_t *>(dout),
                           1, s));
    hip(hipMemcpyAsync(out, dout, out_bytes, hipMemcpyDeviceToHost, s));
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
