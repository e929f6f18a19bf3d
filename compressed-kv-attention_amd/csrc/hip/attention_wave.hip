// Entry points of the one-wave split kernel (attention_wave.h): head_dim 64
// and 128 instantiated here, 256 in attention_wave256.hip; the merges.
#include "attention_wave.h"

namespace kvexp_launch {
using namespace kvexp_dev;

hipError_t attention_wave_256(bool xkv, int order, int G, const HeadDev *heads, const WorkItem *items, int n_items,
                              const BlockDesc *desc, const uint16_t *q, float *out, float *lse, float *ws,
                              hipStream_t s);

// head_dim 64, 128 and 256, both score orders (the host sends other sizes
// to the general kernel).
bool wave_supports(int dim) { return dim == 64 || dim == 128 || dim == 256; }

// Waves per workgroup of the split kernel (consecutive work items share a
// workgroup).
int wave_waves_per_wg(int dim) {
    return dim == 64 ? wave::Shape<64>::kWaves : (dim == 128 ? wave::Shape<128>::kWaves : wave::Shape<256>::kWaves);
}

hipError_t wave_merge(int dim, const MergeItem *mitems, int n_mitems, float *out, float *lse, const float *ws,
                      hipStream_t s) {
    if (n_mitems <= 0) return hipSuccess;
    const int grid = (n_mitems + 3) / 4;
    if (dim == 64)
        hipLaunchKernelGGL(wave::wave_merge_kernel<64>, dim3(grid), dim3(4 * 64), 0, s, mitems, n_mitems, out, lse,
                           ws);
    else if (dim == 128)
        hipLaunchKernelGGL(wave::wave_merge_kernel<128>, dim3(grid), dim3(4 * 64), 0, s, mitems, n_mitems, out, lse,
                           ws);
    else if (dim == 256)
        hipLaunchKernelGGL(wave::wave_merge_kernel<256>, dim3(grid), dim3(4 * 64), 0, s, mitems, n_mitems, out, lse,
                           ws);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t attention_wave(bool xkv, int order, int G, int dim, const HeadDev *heads, const WorkItem *items,
                          int n_items, const BlockDesc *desc, const uint16_t *q, float *out, float *lse, float *ws,
                          hipStream_t s) {
    if (n_items <= 0) return hipSuccess;
    if (dim == 64) return launch_wave_d<64>(xkv, order, G, heads, items, n_items, desc, q, out, lse, ws, s);
    if (dim == 128) return launch_wave_d<128>(xkv, order, G, heads, items, n_items, desc, q, out, lse, ws, s);
    if (dim == 256) return attention_wave_256(xkv, order, G, heads, items, n_items, desc, q, out, lse, ws, s);
    return hipErrorInvalidValue;
}

} // namespace kvexp_launch

#if defined(KVEXP_PHASE_TRACE)
// Copies the phase trace of the last traced launch (n words) to the host.
extern "C" int kvexp_hip_phase_trace_read(unsigned long long *host, size_t n) {
    return int(hipMemcpyFromSymbol(host, HIP_SYMBOL(kvexp_dev::wave::g_phase_trace), n * 8));
}
#endif
