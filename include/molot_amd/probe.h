/*
 * molot_amd measurement probes (no reference counterpart).
 *
 * Plain streaming kernels of known traffic, used by bench.py to measure the
 * achievable HBM bandwidth of the box it runs on and to calibrate rocprofv3's
 * FETCH_SIZE / WRITE_SIZE counters (bytes counted per byte moved).  They are
 * not on the decode path.
 */
#ifndef MOLOT_AMD_PROBE_H_
#define MOLOT_AMD_PROBE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Read `bytes` (multiple of 16, 16-byte aligned) from src with 16-byte loads;
 * writes one float per workgroup into sink[grid] so the loads stay live. */
int molot_probe_read(const void* src, int64_t bytes, float* sink, int64_t sink_len,
                     void* stream);

/* Copy `bytes` (multiple of 16, both 16-byte aligned) from src to dst. */
int molot_probe_copy(void* dst, const void* src, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOLOT_AMD_PROBE_H_ */
