/* Streaming probes of bench.py (libesep_probe.so, built beside this file by build.py). They are
 * measurement kernels, not part of the product library or its ABI (include/esep_body.h). */
#ifndef ESEP_PROBE_H
#define ESEP_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ESEP_PROBE_ONESHOT 0 /* the grid covers the data once, u chunks per stream per lane */
#define ESEP_PROBE_STRIDED 1 /* `blocks` blocks step through the data, next step issued early */

/* Grid the probe launches for these arguments (one-shot: ceil(bytes / (u * threads * 16))). */
int esep_probe_grid(int mode, int u, int threads, int64_t bytes, int blocks);

/* out = a (+ b when b is not NULL) over `bytes` bytes (a multiple of 16, below 4 GiB), all three
 * 16-byte aligned; u in {1, 2, 4, 8} chunks of 16 bytes per stream per lane; threads 256 or 512.
 * Returns 0, a negative argument error (nothing launched) or a positive hipError_t. */
int esep_probe_stream(int mode, int u, int threads, int blocks, const void* a, const void* b,
                      void* out, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif
