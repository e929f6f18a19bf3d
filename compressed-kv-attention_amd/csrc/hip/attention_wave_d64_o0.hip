// The one-wave split kernel (attention_wave.h) at head_dim 64, scalar/AVX2 score order:
// XKV and plain BF16 instantiations for every query-row count.
#include "attention_wave.h"

namespace kvexp_launch {
KVEXP_WAVE_UNIT(64, 0)
} // namespace kvexp_launch
