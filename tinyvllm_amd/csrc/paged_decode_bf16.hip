// Paged-decode kernel instantiations for element type __bf16.
#include "paged_decode_inst.h"

namespace tv {
TV_DECODE_DEFINE(__bf16)
}  // namespace tv
