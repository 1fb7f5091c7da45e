/*
 * wkv7_noalloc.h -- wkv7_run without a caller-provided workspace, in its own library, librwkv7_noalloc.so, which
 * links librwkv7_hip.so (the C ABI of wkv7.h).  Only a process that loads librwkv7_noalloc.so holds its static device
 * scratch array; librwkv7_hip.so alone allocates nothing at load time.
 */
#ifndef RWKV_NEXT_AMD_WKV7_NOALLOC_H
#define RWKV_NEXT_AMD_WKV7_NOALLOC_H

#include "wkv7.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Size of the device scratch array behind wkv7_run_noalloc: per GPU, held from the library's load to process exit. */
#define WKV7_NOALLOC_SCRATCH_BYTES (128u << 20)

/* wkv7_run without a caller-provided workspace.  It has no counterpart in the reference; it is for callers that
 * cannot allocate device memory (code under HIP graph capture that must not allocate, tight serving loops, harnesses
 * that forbid hipMalloc).  args->workspace and args->workspace_bytes are ignored: the scratch is a static device
 * array of WKV7_NOALLOC_SCRATCH_BYTES per GPU, whose flag region starts zero and is left zero by every call.  The
 * first call on a device looks up the array's device address (hipGetSymbolAddress): make one eager call on a device
 * before capturing calls into a HIP graph there.
 * A call whose wkv7_workspace_size exceeds that returns WKV7_ERR_SCRATCH_LIMIT before launching anything.  Calls no
 * hipMalloc/hipFree.  All calls on one GPU share its array: calls whose kernels overlap on one device (other streams,
 * other threads) race; calls in stream order on one stream do not. */
int wkv7_run_noalloc(const wkv7_args *args, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV_NEXT_AMD_WKV7_NOALLOC_H */
