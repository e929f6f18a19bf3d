// The kvexp C++ API (include/kvexp/*.hpp) over the C ABI: host buffers in and
// out, one lazily created context per device, C ABI status codes turned back
// into the reference's exception classes.
#include "kvexp/attention.hpp"
#include "kvexp/codec.hpp"
#include "kvexp_hip.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <memory>
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

// One context per device for the process lifetime.
kvexp_hip_ctx *context() {
    static std::mutex mu;
    static std::vector<kvexp_hip_ctx *> ctxs;
    const int dev = g_device.load();
    std::lock_guard<std::mutex> lock(mu);
    if (size_t(dev) >= ctxs.size()) ctxs.resize(size_t(dev) + 1, nullptr);
    if (ctxs[size_t(dev)] == nullptr) check(kvexp_hip_ctx_create(dev, &ctxs[size_t(dev)]));
    return ctxs[size_t(dev)];
}

struct Dev {
    void *p = nullptr;
    explicit Dev(size_t n) {
        if (hipMalloc(&p, n ? n : 4) != hipSuccess) throw std::runtime_error("hipMalloc failed");
    }
    ~Dev() { (void)hipFree(p); }
    Dev(const Dev &) = delete;
    Dev &operator=(const Dev &) = delete;
};

void hip(hipError_t e) {
    if (e != hipSuccess) throw std::runtime_error(std::string("HIP: ") + hipGetErrorString(e));
}

struct DevScope {
    int prev = 0;
    explicit DevScope(int d) {
        hip(hipGetDevice(&prev));
        hip(hipSetDevice(d));
    }
    ~DevScope() { (void)hipSetDevice(prev); }
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
    kvexp_hip_ctx *ctx = context();
    DevScope scope(g_device.load());
    const int64_t bound = kvexp_hip_encode_bound(seq_len, head_dim, block_tokens);
    const size_t in_bytes = (seq_len > 0 && head_dim > 0) ? size_t(seq_len) * size_t(head_dim) * 2u : 0u;
    Dev din(in_bytes), dout(size_t(bound > 0 ? bound : 0));
    if (kv != nullptr && in_bytes) hip(hipMemcpy(din.p, kv, in_bytes, hipMemcpyHostToDevice));
    size_t n = 0;
    check(kvexp_hip_encode(ctx, kv ? static_cast<const uint16_t *>(din.p) : nullptr, seq_len, head_dim,
                           block_tokens, static_cast<uint8_t *>(dout.p), size_t(bound > 0 ? bound : 0), nullptr,
                           nullptr, &n, nullptr));
    EncodedTensor e;
    e.seq_len = seq_len;
    e.head_dim = head_dim;
    e.block_tokens = block_tokens;
    e.bytes.resize(n);
    if (n) hip(hipMemcpy(e.bytes.data(), dout.p, n, hipMemcpyDeviceToHost));
    return e;
}

void decode_bf16(const uint8_t *blob, size_t bytes, int seq_len, int head_dim, uint16_t *out) {
    kvexp_hip_ctx *ctx = context();
    DevScope scope(g_device.load());
    const int cap = int(bytes / 8 + 2);
    std::vector<int64_t> off(size_t(cap) + 1);
    std::vector<int32_t> first(size_t(cap) + 1);
    int nb = 0;
    check(kvexp_hip_build_index(blob, bytes, head_dim, seq_len, off.data(), first.data(), cap, &nb));
    if (first[size_t(nb)] < seq_len) throw std::runtime_error("xkv decode ran out of blocks");
    if (seq_len <= 0) return;
    const size_t out_bytes = size_t(seq_len) * size_t(head_dim) * 2u;
    Dev db(bytes), doff(size_t(nb + 1) * 8), dfirst(size_t(nb + 1) * 4), dout(out_bytes);
    hip(hipMemcpy(db.p, blob, bytes, hipMemcpyHostToDevice));
    hip(hipMemcpy(doff.p, off.data(), size_t(nb + 1) * 8, hipMemcpyHostToDevice));
    hip(hipMemcpy(dfirst.p, first.data(), size_t(nb + 1) * 4, hipMemcpyHostToDevice));
    check(kvexp_hip_decode(ctx, static_cast<const uint8_t *>(db.p), bytes, static_cast<const int64_t *>(doff.p),
                           static_cast<const int32_t *>(dfirst.p), nb, seq_len, head_dim,
                           static_cast<uint16_t *>(dout.p), 1, nullptr));
    hip(hipMemcpy(out, dout.p, out_bytes, hipMemcpyDeviceToHost));
}

void attention_decode(Backend backend, const uint16_t *q, const uint16_t *k_raw, const uint16_t *v_raw,
                      const uint8_t *k_xkv, size_t k_bytes, const uint8_t *v_xkv, size_t v_bytes, float *out,
                      int n_q, int dim, int seq, int n_threads, int split_tokens) {
    if (backend != Backend::Hip && backend != Backend::HipDpbf16)
        throw std::runtime_error("kvexp-amd runs Backend::Hip and Backend::HipDpbf16; the CPU backends are in the "
                                 "reference library");
    const int order = backend == Backend::Hip ? KVEXP_HIP_ORDER_SCALAR : KVEXP_HIP_ORDER_DPBF16;
    check(kvexp_hip_attention_decode_host(context(), order, q, k_raw, v_raw, k_xkv, k_bytes, v_xkv, v_bytes, out,
                                          n_q, dim, seq, n_threads, split_tokens));
}

} // namespace kvexp
