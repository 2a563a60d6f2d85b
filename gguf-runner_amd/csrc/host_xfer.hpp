// Host <-> device row transfers of the run-state entry points.
//
// The run-state calls take the reference's pageable host rows.  A pageable
// hipMemcpyAsync stages them through the runtime's own pinned buffers with a
// single host thread per copy (about 20 GB/s host to device and far less device
// to host on the target machines).  HostXfer instead keeps a ring of pinned
// slots per run state: the host side of each slot is filled or drained by a
// small pool of copy threads while the DMA engine moves the neighbouring slot,
// so the host copy and the PCIe transfer overlap.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace gr {

struct HostXfer {
    static constexpr int kSlots = 3;
    static constexpr size_t kSlotBytes = size_t(8) << 20;
    // Copies below this size keep the runtime's pageable path (one small
    // staging copy costs less than a pool hand-off).
    static constexpr size_t kMinStaged = size_t(1) << 20;

    char* ring = nullptr;  // kSlots x kSlotBytes of pinned host memory
    hipEvent_t done[kSlots] = {};
    bool pending[kSlots] = {};  // done[i] recorded after the last DMA of slot i
    int next = 0;
};

// Asynchronous on `st` with respect to the device; `src` may be reused as soon
// as the call returns (every byte has been copied out of it).
hipError_t xfer_h2d(HostXfer& x, hipStream_t st, void* dst, const void* src, size_t bytes);

// Enqueues the copy on `st` after the work already there and returns once
// `dst` holds the bytes (and `st` has drained up to the copy).
hipError_t xfer_d2h(HostXfer& x, hipStream_t st, void* dst, const void* src, size_t bytes);

// Releases the ring (after the caller synchronised `st`).
void xfer_release(HostXfer& x);

}  // namespace gr
