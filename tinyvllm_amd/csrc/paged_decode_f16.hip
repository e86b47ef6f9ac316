// Paged-decode kernel instantiations for element type _Float16.
#include "paged_decode_inst.h"

namespace tv {
TV_DECODE_DEFINE(_Float16)
}  // namespace tv
