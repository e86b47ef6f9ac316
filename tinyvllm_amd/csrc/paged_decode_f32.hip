// Paged-decode kernel instantiations for element type float.
#include "paged_decode_inst.h"

namespace tv {
TV_DECODE_DEFINE(float)
}  // namespace tv
