// Pinned-ring host <-> device transfers with a pool of host copy threads.
#include "host_xfer.hpp"

#include <emmintrin.h>
#include <unistd.h>

#include <algorithm>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <deque>
#include <mutex>
#include <thread>
#include <utility>
#include <vector>

namespace gr {
namespace {

// Process-wide memcpy pool.  copy() splits the bytes into equal parts, one per
// thread, the calling thread taking part 0; concurrent callers take turns.  In
// a forked child (no worker threads there) copies run on the caller alone.
class CopyPool {
public:
    static CopyPool& get() {
        static CopyPool* pool = new CopyPool();  // never destroyed: idle workers stay parked
        return *pool;
    }

    void copy(void* dst, const void* src, size_t n) {
        const size_t want = std::max<size_t>(1, n / kMinPart);
        const int parts = getpid() == pid_ ? (int)std::min<size_t>(workers_ + 1, want) : 1;
        if (parts <= 1) {
            std::memcpy(dst, src, n);
            return;
        }
        // (parts >= 2: at least kMinPart bytes, large enough for streaming stores)
        std::lock_guard<std::mutex> call(call_mu_);
        {
            std::lock_guard<std::mutex> lk(mu_);
            dst_ = (char*)dst;
            src_ = (const char*)src;
            n_ = n;
            parts_ = parts;
            left_ = parts - 1;
            ++gen_;
        }
        cv_.notify_all();
        copy_part(0, (char*)dst, (const char*)src, n, parts);
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [this] { return left_ == 0; });
    }

private:
    static constexpr size_t kMinPart = size_t(512) << 10;

    CopyPool() : pid_(getpid()) {
        const unsigned hw = std::thread::hardware_concurrency();
        workers_ = (int)std::min(8u, std::max(hw, 1u)) - 1;
        for (int i = 0; i < workers_; i++) std::thread([this, i] { loop(i + 1); }).detach();
    }

    static void copy_part(int id, char* dst, const char* src, size_t n, int parts) {
        const size_t per = (n / parts + 4095) & ~size_t(4095);
        const size_t lo = std::min(n, per * id), hi = std::min(n, lo + per);
        if (hi > lo) stream_copy(dst + lo, src + lo, hi - lo);
    }

    // memcpy with non-temporal 16-byte stores: the bytes are not read again
    // soon by this thread (a DMA or the caller reads them), and streaming
    // stores skip the read of each destination line that ordinary stores
    // make, a third of the host memory traffic of the copy.
    static void stream_copy(char* d, const char* s, size_t n) {
        const size_t head = std::min(n, (size_t)((16 - ((uintptr_t)d & 15)) & 15));
        std::memcpy(d, s, head);
        d += head;
        s += head;
        n -= head;
        const size_t body = n & ~size_t(63);
        for (size_t i = 0; i < body; i += 64) {
            const __m128i a = _mm_loadu_si128((const __m128i*)(s + i));
            const __m128i b = _mm_loadu_si128((const __m128i*)(s + i + 16));
            const __m128i c = _mm_loadu_si128((const __m128i*)(s + i + 32));
            const __m128i e = _mm_loadu_si128((const __m128i*)(s + i + 48));
            _mm_stream_si128((__m128i*)(d + i), a);
            _mm_stream_si128((__m128i*)(d + i + 16), b);
            _mm_stream_si128((__m128i*)(d + i + 32), c);
            _mm_stream_si128((__m128i*)(d + i + 48), e);
        }
        std::memcpy(d + body, s + body, n - body);
        _mm_sfence();  // the streamed stores are globally visible before the part is reported done
    }

    void loop(int id) {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            cv_.wait(lk, [&] { return gen_ != seen; });
            seen = gen_;
            if (id >= parts_) continue;
            char* d = dst_;
            const char* s = src_;
            const size_t n = n_;
            const int parts = parts_;
            lk.unlock();
            copy_part(id, d, s, n, parts);
            lk.lock();
            if (--left_ == 0) done_cv_.notify_one();
        }
    }

    const pid_t pid_;
    int workers_ = 0;
    std::mutex call_mu_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    uint64_t gen_ = 0;
    char* dst_ = nullptr;
    const char* src_ = nullptr;
    size_t n_ = 0;
    int parts_ = 0;
    int left_ = 0;
};

// The ring is allocated on first use; false when pinned memory is unavailable
// (the caller then keeps the runtime's pageable copy).
bool ensure_ring(HostXfer& x) {
    if (x.ring) return true;
    void* p = nullptr;
    if (hipHostMalloc(&p, HostXfer::kSlots * HostXfer::kSlotBytes, hipHostMallocDefault) != hipSuccess) return false;
    for (int i = 0; i < HostXfer::kSlots; i++) {
        if (hipEventCreateWithFlags(&x.done[i], hipEventDisableTiming) != hipSuccess) {
            for (int j = 0; j < i; j++) (void)hipEventDestroy(x.done[j]);
            (void)hipHostFree(p);
            return false;
        }
        x.pending[i] = false;
    }
    x.ring = (char*)p;
    x.next = 0;
    return true;
}

bool pipe_init(XferPipe& p) {
    if (p.ready) return true;
    bool ok = hipStreamCreateWithFlags(&p.up, hipStreamNonBlocking) == hipSuccess &&
              hipStreamCreateWithFlags(&p.down, hipStreamNonBlocking) == hipSuccess;
    for (int i = 0; ok && i < XferPipe::kMaxPieces; i++)
        ok = hipEventCreateWithFlags(&p.uploaded[i], hipEventDisableTiming) == hipSuccess &&
             hipEventCreateWithFlags(&p.computed[i], hipEventDisableTiming) == hipSuccess;
    if (ok) ok = ensure_ring(p.dn);
    if (!ok) {
        xfer_pipe_release(p);
        return false;
    }
    p.ready = true;
    return true;
}

// The ranges cut into pieces of at most one ring slot.
std::vector<XferRange> slot_chunks(const std::vector<XferRange>& rs) {
    std::vector<XferRange> out;
    for (const XferRange& r : rs)
        for (size_t off = 0; off < r.bytes; off += HostXfer::kSlotBytes)
            out.push_back({r.dev + off, r.host + off, std::min(HostXfer::kSlotBytes, r.bytes - off), r.piece});
    return out;
}

// One upload DMA: device bytes [dev, dev + bytes) from one ring slot, filled
// from parts[first .. first + count) (host range, offset in the slot).
struct SlotLoad {
    char* dev;
    size_t bytes;
    int piece;
    size_t first, count;
};

constexpr size_t kMaxPadBytes = 4096;

void pack_loads(const std::vector<XferRange>& chunks, std::vector<SlotLoad>& loads,
                std::vector<std::pair<XferRange, size_t>>& parts) {
    for (const XferRange& c : chunks) {
        if (!loads.empty()) {
            SlotLoad& l = loads.back();
            const char* end = l.dev + l.bytes;
            if (c.piece == l.piece && c.dev >= end && (size_t)(c.dev - end) <= kMaxPadBytes &&
                (size_t)(c.dev + c.bytes - l.dev) <= HostXfer::kSlotBytes) {
                parts.emplace_back(c, (size_t)(c.dev - l.dev));
                l.bytes = (size_t)(c.dev + c.bytes - l.dev);
                l.count++;
                continue;
            }
        }
        loads.push_back({c.dev, c.bytes, c.piece, parts.size(), 1});
        parts.emplace_back(c, 0);
    }
}

}  // namespace

void host_copy(void* dst, const void* src, size_t bytes) { CopyPool::get().copy(dst, src, bytes); }

hipError_t xfer_h2d(HostXfer& x, hipStream_t st, void* dst, const void* src, size_t bytes) {
    if (!bytes) return hipSuccess;
    if (bytes < HostXfer::kMinStaged || !ensure_ring(x))
        return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
    for (size_t off = 0; off < bytes; off += HostXfer::kSlotBytes) {
        const size_t n = std::min(HostXfer::kSlotBytes, bytes - off);
        const int i = x.next;
        x.next = (x.next + 1) % HostXfer::kSlots;
        if (x.pending[i]) {  // the slot's previous DMA must have read it
            hipError_t e = hipEventSynchronize(x.done[i]);
            if (e != hipSuccess) return e;
            x.pending[i] = false;
        }
        char* slot = x.ring + (size_t)i * HostXfer::kSlotBytes;
        CopyPool::get().copy(slot, (const char*)src + off, n);
        hipError_t e = hipMemcpyAsync((char*)dst + off, slot, n, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipEventRecord(x.done[i], st);
        if (e != hipSuccess) return e;
        x.pending[i] = true;
    }
    return hipSuccess;
}

hipError_t xfer_d2h(HostXfer& x, hipStream_t st, void* dst, const void* src, size_t bytes) {
    hipError_t e = hipSuccess;
    if (bytes < HostXfer::kMinStaged || !ensure_ring(x)) {
        if (bytes) e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st);
        return e == hipSuccess ? hipStreamSynchronize(st) : e;
    }
    // Chunk c lands in slot (base + c) % kSlots; up to kSlots chunks are in
    // flight while the host drains the oldest one.  A slot's earlier DMA on the
    // same stream precedes the new one, so no wait is needed before reuse.
    const size_t S = HostXfer::kSlotBytes;
    const size_t nch = (bytes + S - 1) / S;
    const int base = x.next;
    auto slot_of = [&](size_t c) { return (int)((base + c) % HostXfer::kSlots); };
    auto issue = [&](size_t c) {
        const int i = slot_of(c);
        const size_t n = std::min(S, bytes - c * S);
        hipError_t r = hipMemcpyAsync(x.ring + (size_t)i * S, (const char*)src + c * S, n, hipMemcpyDeviceToHost, st);
        if (r == hipSuccess) r = hipEventRecord(x.done[i], st);
        if (r == hipSuccess) x.pending[i] = true;
        return r;
    };
    for (size_t c = 0; c < nch && c < (size_t)HostXfer::kSlots; c++)
        if ((e = issue(c)) != hipSuccess) return e;
    for (size_t c = 0; c < nch; c++) {
        const int i = slot_of(c);
        if ((e = hipEventSynchronize(x.done[i])) != hipSuccess) return e;
        x.pending[i] = false;
        CopyPool::get().copy((char*)dst + c * S, x.ring + (size_t)i * S, std::min(S, bytes - c * S));
        if (c + HostXfer::kSlots < nch && (e = issue(c + HostXfer::kSlots)) != hipSuccess) return e;
    }
    x.next = slot_of(nch);
    return hipSuccess;
}

void xfer_release(HostXfer& x) {
    if (!x.ring) return;
    for (int i = 0; i < HostXfer::kSlots; i++) (void)hipEventDestroy(x.done[i]);
    (void)hipHostFree(x.ring);
    x.ring = nullptr;
}

bool xfer_pipe_prepare(HostXfer& upr, XferPipe& pp) { return ensure_ring(upr) && pipe_init(pp); }

hipError_t xfer_pipeline(HostXfer& upr, XferPipe& pp, hipStream_t work, int n_pieces,
                         const std::vector<XferRange>& ups, const std::vector<XferRange>& downs,
                         const std::function<int(int)>& enqueue, int* status) {
    *status = 0;
    if (n_pieces < 1 || n_pieces > XferPipe::kMaxPieces) return hipErrorInvalidValue;
    if (!ensure_ring(upr) || !pipe_init(pp)) return hipErrorOutOfMemory;
    const std::vector<XferRange> D = slot_chunks(downs);
    std::vector<SlotLoad> U;
    std::vector<std::pair<XferRange, size_t>> parts;
    pack_loads(slot_chunks(ups), U, parts);
    const size_t S = HostXfer::kSlotBytes;
    size_t iu = 0, idn = 0;
    int pe = 0;                                // pieces whose kernels are enqueued
    std::deque<std::pair<size_t, int>> held;  // downloads in flight or undrained: (chunk, slot)
    hipError_t err = hipSuccess;
    // One host thread, polling: the host copies (the pool's threads share the
    // host's memory bandwidth with both DMA directions) run one at a time.
    for (;;) {
        bool moved = false;
        // the next upload, once its ring slot's previous DMA has read the slot
        if (iu < U.size()) {
            const int i = upr.next;
            const hipError_t q = upr.pending[i] ? hipEventQuery(upr.done[i]) : hipSuccess;
            if (q == hipSuccess) {
                upr.pending[i] = false;
                char* slot = upr.ring + (size_t)i * S;
                for (size_t j = U[iu].first; j < U[iu].first + U[iu].count; j++)
                    CopyPool::get().copy(slot + parts[j].second, parts[j].first.host, parts[j].first.bytes);
                err = hipMemcpyAsync(U[iu].dev, slot, U[iu].bytes, hipMemcpyHostToDevice, pp.up);
                if (err == hipSuccess) err = hipEventRecord(upr.done[i], pp.up);
                if (err != hipSuccess) break;
                upr.pending[i] = true;
                upr.next = (i + 1) % HostXfer::kSlots;
                iu++;
                moved = true;
            } else if (q != hipErrorNotReady) {
                err = q;
                break;
            }
        }
        // kernels of every piece whose uploads are all issued
        while (pe < n_pieces && (iu == U.size() || U[iu].piece > pe)) {
            if ((err = hipEventRecord(pp.uploaded[pe], pp.up)) != hipSuccess ||
                (err = hipStreamWaitEvent(work, pp.uploaded[pe], 0)) != hipSuccess)
                break;
            if ((*status = enqueue(pe)) != 0) break;
            if ((err = hipEventRecord(pp.computed[pe], work)) != hipSuccess ||
                (err = hipStreamWaitEvent(pp.down, pp.computed[pe], 0)) != hipSuccess)
                break;
            pe++;
            moved = true;
        }
        if (err != hipSuccess || *status) break;
        // downloads of enqueued pieces into free slots (slots are taken in order,
        // so the next one is free while fewer than kSlots are held)
        while (idn < D.size() && D[idn].piece < pe && held.size() < (size_t)HostXfer::kSlots) {
            const int i = pp.dn.next;
            err = hipMemcpyAsync(pp.dn.ring + (size_t)i * S, D[idn].dev, D[idn].bytes, hipMemcpyDeviceToHost, pp.down);
            if (err == hipSuccess) err = hipEventRecord(pp.dn.done[i], pp.down);
            if (err != hipSuccess) break;
            pp.dn.next = (i + 1) % HostXfer::kSlots;
            held.emplace_back(idn, i);
            idn++;
            moved = true;
        }
        if (err != hipSuccess) break;
        // drain the oldest download once it has landed
        if (!held.empty()) {
            const size_t c = held.front().first;
            const int i = held.front().second;
            const hipError_t q = hipEventQuery(pp.dn.done[i]);
            if (q == hipSuccess) {
                CopyPool::get().copy(D[c].host, pp.dn.ring + (size_t)i * S, D[c].bytes);
                held.pop_front();
                moved = true;
            } else if (q != hipErrorNotReady) {
                err = q;
                break;
            }
        }
        if (iu == U.size() && pe == n_pieces && idn == D.size() && held.empty()) break;
        if (!moved) std::this_thread::yield();
    }
    if (err != hipSuccess || *status) {
        // let what was issued finish before the rings and buffers are reused
        (void)hipStreamSynchronize(pp.up);
        (void)hipStreamSynchronize(work);
        (void)hipStreamSynchronize(pp.down);
    }
    return err;
}

void xfer_pipe_release(XferPipe& p) {
    for (int i = 0; i < XferPipe::kMaxPieces; i++) {
        if (p.uploaded[i]) (void)hipEventDestroy(p.uploaded[i]);
        if (p.computed[i]) (void)hipEventDestroy(p.computed[i]);
        p.uploaded[i] = p.computed[i] = nullptr;
    }
    if (p.up) (void)hipStreamDestroy(p.up);
    if (p.down) (void)hipStreamDestroy(p.down);
    p.up = p.down = nullptr;
    xfer_release(p.dn);
    p.ready = false;
}

}  // namespace gr
