// Host <-> device row transfers of the run-state entry points.
//
// The run-state calls take the reference's pageable host rows.  A pageable
// hipMemcpyAsync stages them through the runtime's own pinned buffers with a
// single host thread per copy (about 20 GB/s host to device and far less device
// to host on the target machines).  HostXfer instead keeps a ring of pinned
// slots per run state: the host side of each slot is filled or drained by a
// small pool of copy threads while the DMA engine moves the neighbouring slot,
// so the host copy and the PCIe transfer overlap.  Large calls whose rows can be
// processed in pieces (XferPipe) also overlap the uploads of one piece, the
// kernels of the one before and the downloads of the one before that.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <functional>
#include <vector>

namespace gr {

struct HostXfer {
    static constexpr int kSlots = 3;
    static constexpr size_t kSlotBytes = size_t(16) << 20;
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

// Host memcpy, split over the process-wide copy threads from 1 MB on (below
// that, waking the threads costs more than the copy on the calling thread).
void host_copy(void* dst, const void* src, size_t bytes);

// One contiguous host <-> device range of a piece.
struct XferRange {
    char* dev;
    char* host;
    size_t bytes;
    int piece;
};

// Streams, events and the download ring of the pipelined transfers; created on
// first use and kept with the run state.
struct XferPipe {
    static constexpr int kMaxPieces = 8;
    hipStream_t up = nullptr, down = nullptr;
    hipEvent_t uploaded[kMaxPieces] = {};
    hipEvent_t computed[kMaxPieces] = {};
    HostXfer dn;  // download ring (the upload ring is the state's own HostXfer)
    bool ready = false;
};

// Runs n_pieces pieces: piece p's uploads (ranges tagged p, in order) go on
// pipe.up through `up_ring` (consecutive ranges of a piece whose device ends
// meet, or are at most 4 KB apart, share one ring slot and one DMA; the gap is
// written with whatever the slot holds), then `work` waits for them and enqueue(p) adds
// the piece's kernels to `work`, then pipe.down waits for those and the
// piece's downloads come back through the download ring.  One host thread
// drives all three, polling: it stages the next upload slot, issues downloads
// of finished pieces and drains finished download slots as each becomes
// possible.  Returns after every download is in host memory (and so every
// upload and kernel before it has finished).  A nonzero enqueue status stops
// the pipeline: the work already issued is waited for and the status is
// returned in *status.
hipError_t xfer_pipeline(HostXfer& up_ring, XferPipe& pipe, hipStream_t work, int n_pieces,
                         const std::vector<XferRange>& ups, const std::vector<XferRange>& downs,
                         const std::function<int(int)>& enqueue, int* status);

// Allocates what xfer_pipeline needs (both rings, the streams, the events) if it
// is not there yet; false when that fails (no pinned memory), and the caller
// then moves its pieces one after another with xfer_h2d / xfer_d2h.
bool xfer_pipe_prepare(HostXfer& up_ring, XferPipe& pipe);

// Destroys the pipe's streams, events and ring (after its work has finished).
void xfer_pipe_release(XferPipe& pipe);

}  // namespace gr
