/* sbx_probe.h -- measurement interface of the probe build of the library
 * (lib/libsbx_probe.so, the same sources compiled with SBX_PROBE; the product
 * library lib/libsbx.so exports none of this).  Not part of the drop-in C ABI
 * (include/sbx.h): it serves bench.py --probe, which reads the clock and the
 * busy cycles of every dispatch of a back-to-back timed loop.
 *
 * The GEMM kernels (the MFMA tile kernel and the small-problem kernel) store,
 * for each workgroup b < blocks of batch entry 0, SBX_PROBE_POINTS pairs
 * (s_memtime core-cycle counter, s_memrealtime constant-rate counter) at
 * buf[((d % ring) * blocks + b) * SBX_PROBE_POINTS * 2 + 2 * point + {0, 1}],
 * where d counts the GEMM dispatches since the last sbx_probe_set.  Points:
 * tile kernel 0 = entry, 1 = end of the k loop; small-problem kernel 0 =
 * entry, 1 = first loads issued, 2 = MFMAs issued, 3 = C stores issued.
 * Unused points are left as they were. */
#ifndef SBX_PROBE_H
#define SBX_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SBX_PROBE_POINTS 4

/* Device buffer of ring * blocks * SBX_PROBE_POINTS * 2 uint64 (null: stop
 * recording); resets the dispatch count.  Returns SBX_OK or
 * SBX_INVALID_ARGUMENT. */
int sbx_probe_set(void* buf, int64_t blocks, int64_t ring);

/* GEMM dispatches recorded since the last sbx_probe_set. */
int64_t sbx_probe_dispatches(void);

/* Rate of the s_memrealtime counter of the current device, in kHz (0 if the
 * runtime cannot say). */
int64_t sbx_probe_wall_clock_khz(void);

#ifdef __cplusplus
}
#endif

#endif /* SBX_PROBE_H */
