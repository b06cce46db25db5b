// ghip_internal.h -- entry points shared between the host library's sources
// (not part of the C ABI).
#ifndef GHIP_INTERNAL_H
#define GHIP_INTERNAL_H
#include "../../include/ghip.h"

// ghip_mul_mat with a caller-fixed workspace [scratch, scratch + bytes): no
// allocation; a call that needs more fails with GHIP_STATUS_ALLOC_FAILED.
ghip_status ghip_mul_mat_fixed_scratch(ghip_context *ctx, const ghip_tensor *src0, const ghip_tensor *src1,
                                       const ghip_tensor *dst, void *scratch, size_t bytes, void *stream);
int ghip_context_device(const ghip_context *ctx);
// Copy n host bytes to device memory dst on stream through the context's
// pinned staging buffers; returns when the copy has completed.
ghip_status ghip_context_upload(ghip_context *ctx, void *dst, const void *src, size_t n, void *stream);
ghip_status ghip_context_fail(ghip_context *ctx, ghip_status st, const char *msg);

// ghip_noalloc.hip: resolve the device address of the fixed scratch array on
// `device` (which must be current); called once per device from ghip_init.
ghip_status ghip_noalloc_setup(int device, const char **why);
#endif
