// Stream schedule of the split-K decode kernels (DecodeLaunch::stream_sched).
//
// The (sequence, column, key) space is flattened: with E_s = L_s + P for a
// non-empty sequence (0 for an empty one; L_s = kv_end - kv_start, P =
// stream_seg_cost virtual keys that stand for what starting a segment costs a
// workgroup), pair (s, c) occupies [off_s + c E_s, off_s + (c + 1) E_s), off_s
// = n_cols * sum_{s' < s} E_s', and its keys are the last L_s of that interval.
// Workgroup b takes [b Q, (b + 1) Q), Q = max(stream_min_keys, ceil(total /
// #workgroups)) rounded up to 32, and writes one partial per pair it meets, in
// slot b - first_key(s, c) / Q of that pair.  Workgroup 0 publishes off_s and Q
// in stream_sched[0 .. n_seq] for the combine kernels.
#pragma once

#include "gr_internal.hpp"

namespace gr {

// Keys of sequence i on the schedule: kv_end - kv_start, at least 0 and at most
// what the partial slots cover ((n_splits - 1) * stream_min_keys >= max_kv_len),
// so that a length above the max_kv_len the caller declared cannot push the
// flattened offsets past the range the host checked (its keys past the slots
// are dropped, as on the fixed grid).
__device__ __forceinline__ int stream_len(const DecodeLaunch& p, int i) {
    return min(max(0, p.kv_end[i] - p.kv_start[i]), (p.n_splits - 1) * p.stream_min_keys);
}

// Per-workgroup cursor over the workgroup's key range.  The per-sequence
// lengths and offsets live in LDS (len, off: kStreamMaxSeq entries each).
template <int kThreads>
struct StreamCursor {
    static constexpr int kWaves = kThreads / 64;
    int* len;
    int* off;
    int q = 0, pos = 0, hi = 0;  // range size, cursor, end of the workgroup's range
    int s = 0, col = 0;          // current (sequence, column) pair
    int n_cols = 1, cost = 0;

    __device__ int ext(int i) const { return len[i] > 0 ? len[i] + cost : 0; }

    // Block-wide scan of the flattened lengths (consecutive sequences per
    // thread), then the pair holding the range's first key.  Every thread of
    // the workgroup calls it; returns false (for the whole workgroup) when the
    // range starts past the last key.  first / wsum: LDS scratch.
    __device__ bool init(const DecodeLaunch& p, int n_cols_, int* len_, int* off_, int* first, int* wsum) {
        len = len_;
        off = off_;
        n_cols = n_cols_;
        cost = p.stream_seg_cost;
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int n = p.n_seq;
        constexpr int C = kStreamMaxSeq / kThreads;
        int loc[C];
        int tsum = 0;
#pragma unroll
        for (int c = 0; c < C; c++) {
            const int i = tid * C + c;
            const int l = i < n ? stream_len(p, i) : 0;
            loc[c] = tsum;
            tsum += (l > 0 ? l + cost : 0) * n_cols;
            if (i < n) len[i] = l;
        }
        int incl = tsum;  // inclusive scan over the wave
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int y = __shfl_up(incl, d, 64);
            if (lane >= d) incl += y;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        int base = 0, total = 0;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            base += w < wave ? wsum[w] : 0;
            total += wsum[w];
        }
        const int excl = base + incl - tsum;
        q = max(p.stream_min_keys, (total + (int)gridDim.x - 1) / (int)gridDim.x);
        q = (q + 31) / 32 * 32;
        const int lo = (int)blockIdx.x * q;
#pragma unroll
        for (int c = 0; c < C; c++) {
            const int i = tid * C + c;
            if (i < n) {
                const int o = excl + loc[c];
                off[i] = o;
                if (blockIdx.x == 0) p.stream_sched[i] = o;
                const int l = len[i];
                if (lo >= o && lo < o + (l > 0 ? l + cost : 0) * n_cols) *first = i;
            }
        }
        if (blockIdx.x == 0 && tid == 0) p.stream_sched[n] = q;
        if (lo >= total) return false;
        __syncthreads();
        pos = lo;
        hi = min(total, lo + q);
        s = *first;
        col = (lo - off[s]) / ext(s);
        return true;
    }

    // The current pair's part of the range: keys [t_begin, t_stop) of sequence
    // s (cache positions) and the partial slot.  False when the range ends
    // inside the pair's virtual keys (nothing left for this workgroup).
    __device__ bool segment(const DecodeLaunch& p, int& t_begin, int& t_stop, int& split) {
        const int l = len[s];
        const int o = off[s] + col * ext(s) + cost;  // the pair's first key
        const int beg = max(pos, o);
        const int end = min(hi, o + l);
        pos = max(pos, end);
        if (beg >= end) return false;
        split = (int)blockIdx.x - o / q;
        t_begin = p.kv_start[s] + (beg - o);
        t_stop = p.kv_start[s] + (end - o);
        return true;
    }

    // Move to the next pair; false when the range is exhausted.  A range that
    // continues past a pair always reaches a later non-empty sequence.
    __device__ bool advance() {
        if (pos >= hi) return false;
        if (++col == n_cols) {
            col = 0;
            do {
                s++;
            } while (len[s] == 0);
        }
        return true;
    }
};

// Partials the split kernel wrote for pair (s, col), from the offsets and range
// size workgroup 0 published.
__device__ __forceinline__ int stream_partials(const DecodeLaunch& p, int s, int col) {
    const int len = stream_len(p, s);
    if (len <= 0) return 0;
    const int q = p.stream_sched[p.n_seq];
    const int o = p.stream_sched[s] + col * (len + p.stream_seg_cost) + p.stream_seg_cost;
    return min(p.n_splits, (o + len - 1) / q - o / q + 1);
}

}  // namespace gr
