// Entry points of the one-wave split kernel (attention_wave.h) and its
// merges; the split kernels themselves are instantiated per head_dim and
// score order in attention_wave_d<D>_o<O>.hip.
#include "attention_wave.h"

namespace kvexp_launch {
using namespace kvexp_dev;

#define KVEXP_WAVE_DECL(D, O)                                                                                        \
    hipError_t attention_wave_d##D##_o##O(bool xkv, int G, const HeadDev *heads, const WorkItem *items,             \
                                         int n_items, int wpg, const BlockDesc *desc, const uint16_t *q,           \
                                         float *out, float *lse, float *ws, hipStream_t s);
KVEXP_WAVE_DECL(64, 0)
KVEXP_WAVE_DECL(64, 1)
KVEXP_WAVE_DECL(128, 0)
KVEXP_WAVE_DECL(128, 1)
KVEXP_WAVE_DECL(256, 0)
KVEXP_WAVE_DECL(256, 1)

// head_dim 64, 128 and 256, both score orders (the host sends other sizes
// to the general kernel).
bool wave_supports(int dim) { return dim == 64 || dim == 128 || dim == 256; }

// Waves per workgroup of the split kernel (consecutive work items share a
// workgroup).
int wave_waves_per_wg(int dim) {
    return dim == 64 ? wave::Shape<64>::kWaves : (dim == 128 ? wave::Shape<128>::kWaves : wave::Shape<256>::kWaves);
}

hipError_t wave_merge(int dim, const MergeItem *mitems, int n_mitems, const MergeItem &uni, float *out, float *lse,
                      const float *ws, hipStream_t s) {
    if (n_mitems <= 0) return hipSuccess;
    const int grid = (n_mitems + wave::kMergeWaves - 1) / wave::kMergeWaves;
    if (dim == 64)
        hipLaunchKernelGGL(wave::wave_merge_kernel<64>, dim3(grid), dim3(wave::kMergeWaves * 64), 0, s, mitems, n_mitems, uni, out,
                           lse, ws);
    else if (dim == 128)
        hipLaunchKernelGGL(wave::wave_merge_kernel<128>, dim3(grid), dim3(wave::kMergeWaves * 64), 0, s, mitems, n_mitems, uni, out,
                           lse, ws);
    else if (dim == 256)
        hipLaunchKernelGGL(wave::wave_merge_kernel<256>, dim3(grid), dim3(wave::kMergeWaves * 64), 0, s, mitems, n_mitems, uni, out,
                           lse, ws);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t attention_wave(bool xkv, int order, int G, int dim, const HeadDev *heads, const WorkItem *items,
                          int n_items, int wpg, const BlockDesc *desc, const uint16_t *q, float *out, float *lse,
                          float *ws, hipStream_t s) {
    if (n_items <= 0) return hipSuccess;
    if (order != 0 && order != 1) return hipErrorInvalidValue;
#define KVEXP_WAVE_CASE(D)                                                                                           \
    if (dim == D)                                                                                                    \
        return order == 0 ? attention_wave_d##D##_o0(xkv, G, heads, items, n_items, wpg, desc, q, out, lse, ws, s)   \
                          : attention_wave_d##D##_o1(xkv, G, heads, items, n_items, wpg, desc, q, out, lse, ws, s);
    KVEXP_WAVE_CASE(64)
    KVEXP_WAVE_CASE(128)
    KVEXP_WAVE_CASE(256)
#undef KVEXP_WAVE_CASE
    return hipErrorInvalidValue;
}

} // namespace kvexp_launch

#if defined(KVEXP_PHASE_TRACE)
namespace kvexp_launch {
hipError_t attention_wave_d64_o0_trace_read(unsigned long long *host, size_t n);
hipError_t attention_wave_d128_o0_trace_read(unsigned long long *host, size_t n);
hipError_t attention_wave_d256_o0_trace_read(unsigned long long *host, size_t n);
} // namespace kvexp_launch
// Copies the phase trace of the last traced launch at head_dim `dim` (n
// words) to the host (trace builds only).
extern "C" int kvexp_hip_phase_trace_read(unsigned long long *host, size_t n, int dim) {
    using namespace kvexp_launch;
    if (dim == 64) return int(attention_wave_d64_o0_trace_read(host, n));
    if (dim == 128) return int(attention_wave_d128_o0_trace_read(host, n));
    if (dim == 256) return int(attention_wave_d256_o0_trace_read(host, n));
    return int(hipErrorInvalidValue);
}
#endif
