// head_dim 256 instantiations of the one-wave split kernel
// (attention_wave.h), in a translation unit of their own so that they
// compile beside the others.
#include "attention_wave.h"

namespace kvexp_launch {

hipError_t attention_wave_256(bool xkv, int order, int G, const HeadDev *heads, const WorkItem *items, int n_items,
                              const BlockDesc *desc, const uint16_t *q, float *out, float *lse, float *ws,
                              hipStream_t s) {
    return launch_wave_d<256>(xkv, order, G, heads, items, n_items, desc, q, out, lse, ws, s);
}

} // namespace kvexp_launch
