// wkv7_noalloc.hip -- wkv7_run_noalloc: wkv7_run for callers that cannot allocate device memory (code under HIP
// graph capture that must not touch an allocator, tight serving loops, harnesses that forbid hipMalloc).
//
// The only scratch memory wkv7_run uses is the chunked paths' workspace (hand-off flags, exchange entries, records).
// Here it comes from `scratch`, a file-scope device array of WKV7_NOALLOC_SCRATCH_BYTES that every GPU the library
// runs on holds from module load until the process ends.  It is built as its own library, librwkv7_noalloc.so, on
// top of librwkv7_hip.so (it calls only wkv7_workspace_size and wkv7_run), so processes that never load it hold no
// such array.  Calls needing more are refused with WKV7_ERR_SCRATCH_LIMIT before anything is launched.  The
// segmented kernel's flag region (the first
// WKV7_SEG_FLAG_BYTES) must be zero before a call: the array starts zeroed and every call that completes leaves it
// zero; everything else is written before it is read within each call, so no clearing is needed between calls.  (A
// call that reports WKV7_STATUS_SEGMENT_WAIT -- a bounded hand-off wait that expired -- can leave flags set; later
// segmented calls through this entry are then unreliable until the process restarts.)
//
// All calls on one GPU share that GPU's array: two calls whose kernels overlap on one device (different streams,
// or different host threads) race on it.  Calls in stream order on one stream are safe.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "wkv7_noalloc.h"

namespace {

static __device__ __align__(256) unsigned char scratch[WKV7_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device.  In host code the array's name is only a host-side stand-in
// for the symbol; the device address comes from hipGetSymbolAddress, looked up once per device with that device
// current, and that address is what the kernels receive.
int scratch_on_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return static_cast<int>(e);
    if (dev < 0 || dev >= kMaxDevices) return WKV7_ERR_ARG;
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return static_cast<int>(e);
        if (!p) return WKV7_ERR_NULL;
        g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return WKV7_OK;
}

}  // namespace

extern "C" int wkv7_run_noalloc(const wkv7_args* args, void* stream) {
    if (!args) return WKV7_ERR_NULL;
    size_t need = 0;
    int rc = wkv7_workspace_size(args, &need);  // validates the arguments
    if (rc != WKV7_OK) return rc;
    if (need > (size_t)WKV7_NOALLOC_SCRATCH_BYTES) return WKV7_ERR_SCRATCH_LIMIT;
    wkv7_args a = *args;
    a.workspace = nullptr;
    a.workspace_bytes = 0;
    if (need > 0) {
        void* p = nullptr;
        rc = scratch_on_current_device(&p);
        if (rc != WKV7_OK) return rc;
        a.workspace = p;
        a.workspace_bytes = WKV7_NOALLOC_SCRATCH_BYTES;
    }
    return wkv7_run(&a, stream);
}
