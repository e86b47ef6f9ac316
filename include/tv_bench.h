/*
 * Measurement helper of libtvattn.so (no counterpart in the reference, whose
 * hot path has no native code): the HBM streaming-read ceiling that the
 * HBM-bound kernels' bandwidth is compared with.
 */
#ifndef TV_BENCH_H
#define TV_BENCH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Reads every 16-byte vector of src[0, bytes) once, with ordinary
 * (nontemporal = 0) or non-temporal 16-byte loads, loads_in_flight (4 or 8)
 * of them issued per lane before the first is used, on work_groups
 * work-groups of 256 lanes: interleaved over the whole grid (contiguous = 0)
 * or one contiguous range per work-group (contiguous = 1).  src is 16-byte aligned and
 * bytes a positive multiple of 16; sink holds work_groups words and is written
 * only if the xor of the data equals a fixed constant (it keeps the loads
 * live).  Returns TV_OK, TV_EINVAL or TV_EHIP (codes of tv_attn.h).
 */
int tv_stream_read(const void* src, int64_t bytes, int nontemporal, int loads_in_flight,
                   int work_groups, int contiguous, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TV_BENCH_H */
