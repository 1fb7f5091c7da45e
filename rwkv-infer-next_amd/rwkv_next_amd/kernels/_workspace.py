"""Per-stream device workspaces whose leading region holds counters or flags that must be zero when a call starts.

Both the W6A16 split-K kernels (arrival counters, include/w6a16.h) and the segmented WKV7 prefill (hand-off flags,
include/wkv7.h) keep such a region: every completed call leaves it zero, so the calls of one stream, which run in
order, share one workspace, and calls on different streams, which may overlap, never do.
"""
from __future__ import annotations

import ctypes

import torch

_HIP = None
_RETIRED: list = []


def capture_id(stream: int) -> int:
    """The id of the HIP graph capture in progress on `stream` (hipStreamGetCaptureInfo)."""
    global _HIP
    if _HIP is None:
        hip = ctypes.CDLL("libamdhip64.so")
        hip.hipStreamGetCaptureInfo.restype = ctypes.c_int
        hip.hipStreamGetCaptureInfo.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int),
                                                ctypes.POINTER(ctypes.c_ulonglong)]
        _HIP = hip
    status, cid = ctypes.c_int(0), ctypes.c_ulonglong(0)
    rc = _HIP.hipStreamGetCaptureInfo(ctypes.c_void_p(stream), ctypes.byref(status), ctypes.byref(cid))
    if rc != 0:
        raise RuntimeError(f"hipStreamGetCaptureInfo failed ({rc})")
    return int(cid.value)


def stream_workspace(cache: dict, device, nbytes: int, zero_bytes: int):
    """The workspace of the current stream on `device` from `cache`, at least `nbytes` long, whose first `zero_bytes`
    are zero in stream order when the call that requested it runs.

    Only that leading region is ever cleared.  A workspace created eagerly is cleared there.  A capture on a stream
    without a workspace first takes over a large-enough one that another stream of the device has cleared eagerly
    (torch synchronises the device before a capture begins, so the clear is complete; that stream gets a new one at
    its next call), so a graph captured after an eager warm-up records no clearing.  Otherwise the new workspace is
    cleared by a node of that graph, and until an eager call has cleared it in stream order, every further capture
    that uses it starts with a clear of its leading region (a graph may be replayed before the one that created the
    buffer).  A larger request replaces the buffer; the old one is kept alive, since a captured graph may still
    address it."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(idx).cuda_stream
    capturing = torch.cuda.is_current_stream_capturing()
    key = (idx, stream)
    entry = cache.get(key)
    if entry is None and capturing:
        for other, e in list(cache.items()):
            if other[0] == idx and e[1] and e[0].numel() >= nbytes:
                entry = cache.pop(other)
                entry[2] = capture_id(stream)
                cache[key] = entry
                break
    if entry is None or entry[0].numel() < nbytes:
        if entry is not None:
            _RETIRED.append(entry[0])
        ws = torch.empty(max(nbytes, 2 * zero_bytes), dtype=torch.uint8, device=torch.device("cuda", idx))
        ws[:zero_bytes].zero_()
        entry = [ws, not capturing, capture_id(stream) if capturing else None]
        cache[key] = entry
    if not entry[1]:
        if capturing:
            cid = capture_id(stream)
            if entry[2] != cid:
                entry[0][:zero_bytes].zero_()
                entry[2] = cid
        else:
            entry[0][:zero_bytes].zero_()
            entry[1] = True
    return entry[0]
