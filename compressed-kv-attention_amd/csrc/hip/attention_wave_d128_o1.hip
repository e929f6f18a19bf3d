// The one-wave split kernel (attention_wave.h) at head_dim 128, AVX-512 BF16 score order:
// XKV and plain BF16 instantiations for every query-row count.
#include "attention_wave.h"

namespace kvexp_launch {
KVEXP_WAVE_UNIT(128, 1)
} // namespace kvexp_launch
