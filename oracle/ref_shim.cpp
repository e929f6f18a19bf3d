// TEST INFRASTRUCTURE ONLY. Never linked into the product library.
//
// extern "C" shim over the reference kvexp public API so that Python tests can
// call the compiled reference (oracle/_ref/libkvexp_ref.so, built by
// oracle/Makefile from the sources under /root/reference, which are never
// copied here). Exceptions are mapped to status codes:
//   1 = std::invalid_argument, 2 = std::runtime_error, 3 = std::logic_error,
//   4 = other. The message is kept per thread and read with kvexp_ref_last_error().
//
// Wrapped interfaces:
//   kvexp::encode_bf16 / decode_bf16   include/kvexp/codec.hpp:45-48
//   kvexp::attention_decode            include/kvexp/attention.hpp:58-61
//   kvexp::detect_cpu                  include/kvexp/attention.hpp:16-21

#include "kvexp/attention.hpp"
#include "kvexp/codec.hpp"

#include <cstring>
#include <omp.h>
#include <stdexcept>
#include <string>

namespace {
thread_local std::string g_msg;

template <class F> int guarded(F &&fn) {
    try {
        fn();
        g_msg.clear();
        return 0;
    } catch (const std::invalid_argument &e) {
        g_msg = e.what();
        return 1;
    } catch (const std::logic_error &e) {
        g_msg = e.what();
        return 3;
    } catch (const std::runtime_error &e) {
        g_msg = e.what();
        return 2;
    } catch (const std::exception &e) {
        g_msg = e.what();
        return 4;
    }
}
} // namespace

extern "C" {

const char *kvexp_ref_last_error(void) { return g_msg.c_str(); }

int kvexp_ref_detect_cpu(int *avx2, int *avx512_bf16) {
    const kvexp::CpuFeatures f = kvexp::detect_cpu();
    *avx2 = f.avx2 ? 1 : 0;
    *avx512_bf16 = f.avx512_bf16 ? 1 : 0;
    return 0;
}

// Encodes into `out` (capacity `cap`); writes the container size to *out_bytes.
// Returns 5 when the container does not fit (size still reported).
int kvexp_ref_encode(const uint16_t *kv, int seq, int dim, int block, uint8_t *out, size_t cap,
                     size_t *out_bytes) {
    int rc = guarded([&] {
        kvexp::EncodedTensor e = kvexp::encode_bf16(kv, seq, dim, block);
        *out_bytes = e.bytes.size();
        if (e.bytes.size() > cap) {
            throw std::length_error("capacity");
        }
        if (!e.bytes.empty()) {
            std::memcpy(out, e.bytes.data(), e.bytes.size());
        }
    });
    if (rc == 3 && g_msg == "capacity") {
        return 5;
    }
    return rc;
}

int kvexp_ref_decode(const uint8_t *blob, size_t bytes, int seq, int dim, uint16_t *out) {
    return guarded([&] { kvexp::decode_bf16(blob, bytes, seq, dim, out); });
}

// backend: 0 = Scalar, 1 = Avx2, 2 = Avx512Bf16 (attention.hpp:10-14).
int kvexp_ref_attention(int backend, const uint16_t *q, const uint16_t *k_raw, const uint16_t *v_raw,
                        const uint8_t *k_xkv, size_t k_bytes, const uint8_t *v_xkv, size_t v_bytes,
                        float *out, int n_q, int dim, int seq, int n_threads, int split_tokens) {
    return guarded([&] {
        kvexp::Backend be = kvexp::Backend::Scalar;
        if (backend == 1) {
            be = kvexp::Backend::Avx2;
        } else if (backend == 2) {
            be = kvexp::Backend::Avx512Bf16;
        } else if (backend != 0) {
            throw std::invalid_argument("kvexp_ref_attention: unknown backend");
        }
        kvexp::attention_decode(be, q, k_raw, v_raw, k_xkv, k_bytes, v_xkv, v_bytes, out, n_q, dim,
                                seq, n_threads, split_tokens);
    });
}

// The reference bench's `model_heads` scope (src/bench.cpp:711-728): OpenMP over
// independent KV heads, each head attention_decode with one thread. Head h
// reads q + h*n_q*dim and writes out + h*n_q*dim; XKV inputs when k_xkv is set.
int kvexp_ref_attention_heads(int backend, int n_heads, int omp_threads, const uint16_t *q,
                              const uint16_t *const *k_raw, const uint16_t *const *v_raw,
                              const uint8_t *const *k_xkv, const uint64_t *k_bytes,
                              const uint8_t *const *v_xkv, const uint64_t *v_bytes, float *out, int n_q,
                              int dim, int seq, int split_tokens) {
    return guarded([&] {
        kvexp::Backend be = backend == 2 ? kvexp::Backend::Avx512Bf16
                                         : (backend == 1 ? kvexp::Backend::Avx2 : kvexp::Backend::Scalar);
        int failed = 0;
        omp_set_dynamic(0);
#pragma omp parallel for schedule(static) num_threads(omp_threads)
        for (int h = 0; h < n_heads; ++h) {
            const size_t qo = size_t(h) * size_t(n_q) * size_t(dim);
            try {
                if (k_xkv != nullptr) {
                    kvexp::attention_decode(be, q + qo, nullptr, nullptr, k_xkv[h], k_bytes[h], v_xkv[h],
                                            v_bytes[h], out + qo, n_q, dim, seq, 1, split_tokens);
                } else {
                    kvexp::attention_decode(be, q + qo, k_raw[h], v_raw[h], nullptr, 0, nullptr, 0, out + qo,
                                            n_q, dim, seq, 1, split_tokens);
                }
            } catch (...) {
#pragma omp atomic write
                failed = 1;
            }
        }
        if (failed) {
            throw std::runtime_error("kvexp_ref_attention_heads: a head failed");
        }
    });
}

} // extern "C"
