/*
 * rxmet_prof.h — launch timing of the library's own kernels with HIP events.
 *
 * No counterpart in the reference: this is measurement support for benchmarks that
 * must time one kernel inside an entry point that launches several.  When enabled,
 * every instrumented launch is bracketed by a pair of hipEvents recorded on the
 * stream the kernel is launched on; rxmet_prof_query resolves the pending pairs
 * (waiting for them) and reports the accumulated time per kernel name.  Disabled by
 * default; when disabled the instrumentation costs one branch per launch.
 */
#ifndef RXMET_PROF_H_
#define RXMET_PROF_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Turn event timing on (non-zero) or off. Returns 0. */
int rxmet_prof_enable(int32_t on);
/* Time only the launches whose name is in the comma-separated list `names` (null or empty:
 * every instrumented launch).  Each timed launch adds two event records to its stream, so a
 * benchmark can keep the perturbation of its timed region to the kernels it reports. */
int rxmet_prof_filter(const char *names);
/* Drop every accumulated figure and pending event pair. Returns 0. */
int rxmet_prof_reset(void);
/* Total milliseconds and launch count recorded for `name` since the last reset
 * (waits for pending events of that name).  Unknown names give 0 and 0. */
int rxmet_prof_query(const char *name, double *total_ms, int64_t *launches);
/* Comma-separated names seen since the last reset, written into buf (NUL-terminated,
 * truncated to len-1 bytes).  Returns the length needed without the NUL. */
int64_t rxmet_prof_names(char *buf, int64_t len);

#ifdef __cplusplus
}
#endif

#endif /* RXMET_PROF_H_ */
