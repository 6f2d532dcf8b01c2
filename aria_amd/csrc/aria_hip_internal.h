/*
 * aria_hip_internal.h - internal: runtime helpers shared by the C host files of the
 * backend (aria_hip.c, aria_hip_dit.c). Hidden from the library's exported ABI.
 */
#ifndef ARIA_HIP_INTERNAL_H
#define ARIA_HIP_INTERNAL_H

#include <hip/hip_runtime_api.h>

#define ARIA_HIDDEN __attribute__((visibility("hidden")))

/* select the library device on this thread; 0 or ARIA_HIP_ENODEV (error text set) */
ARIA_HIDDEN int aria_hip_ensure(void);
/* record (and print) a failed HIP call; returns the error code as int */
ARIA_HIDDEN int aria_hip_fail(hipError_t e, const char *what);
/* set the per-thread error text */
ARIA_HIDDEN void aria_hip_set_error(const char *fmt, ...);
/* the stream to use for a caller's void* (NULL = library stream) */
ARIA_HIDDEN hipStream_t aria_hip_stream(void *stream);
/* the allocation-free GEMM's per-device set-up (k_noalloc.hip) for the current device, run at
 * library init so that a first call under stream capture finds it done; 0 or an error code */
ARIA_HIDDEN int aria_noalloc_setup(void);

#endif /* ARIA_HIP_INTERNAL_H */
