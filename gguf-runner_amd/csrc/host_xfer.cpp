// Pinned-ring host <-> device transfers with a pool of host copy threads.
#include "host_xfer.hpp"

#include <unistd.h>

#include <algorithm>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <thread>
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
        if (hi > lo) std::memcpy(dst + lo, src + lo, hi - lo);
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

}  // namespace

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

}  // namespace gr
