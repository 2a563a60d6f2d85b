"""CPU replay of the split-K decode stream schedule (csrc/stream_sched.hpp: StreamCursor
init / segment / advance, stream_partials; the host plan in csrc/api.cpp plan_decode).

The replay restates the schedule's integer arithmetic line by line and checks what the
split and combine kernels rely on, for the shape of the Turbo d256 decode test
(test_turbo_decode_head_dims_and_groups[256-16-1]) and for random ragged batches:
  - the segments of all workgroups cover every key of every (sequence, column) pair
    exactly once, inside the pair's [kv_start, kv_end);
  - each segment's partial slot is in [0, n_splits), and the slots of one pair are
    0 .. n - 1 with n = stream_partials(pair), the count the combine kernels read;
  - partial indices stay inside the workspace the host plan sizes.
No GPU is involved.
"""
from __future__ import annotations

import numpy as np
import pytest

STREAM_MAX_SEQ = 1024


def stream_len(starts, ends, i, n_splits, min_keys):
    return min(max(0, ends[i] - starts[i]), (n_splits - 1) * min_keys)


def plan(max_len, min_keys):
    """plan_decode's stream branch: n_splits."""
    return (max_len + min_keys - 1) // min_keys + 1


def replay(starts, ends, n_cols, grid, min_keys, cost, max_len):
    """Segments (wg, s, col, t_begin, t_stop, split) of every workgroup."""
    n = len(starts)
    n_splits = plan(max_len, min_keys)
    lens = [stream_len(starts, ends, i, n_splits, min_keys) for i in range(n)]
    ext = [(l + cost if l > 0 else 0) for l in lens]
    off = np.concatenate([[0], np.cumsum([e * n_cols for e in ext])]).astype(int).tolist()
    total = off[n]
    q = max(min_keys, -(-total // grid))
    q = -(-q // 32) * 32
    segs = []
    for b in range(grid):
        lo = b * q
        if lo >= total:
            continue
        s = next(i for i in range(n) if off[i] <= lo < off[i] + ext[i] * n_cols)
        pos, hi = lo, min(total, lo + q)
        col = (lo - off[s]) // ext[s]
        while True:
            o = off[s] + col * ext[s] + cost
            beg, end = max(pos, o), min(hi, o + lens[s])
            pos = max(pos, end)
            if beg >= end:
                break
            split = b - o // q
            segs.append((b, s, col, starts[s] + beg - o, starts[s] + end - o, split))
            if pos >= hi:
                break
            col += 1
            if col == n_cols:
                col = 0
                s += 1
                while lens[s] == 0:
                    s += 1
    return segs, lens, off, q, n_splits


def partials(lens, off, q, s, col, cost, n_splits):
    """stream_partials: partial slots the split kernel wrote for pair (s, col)."""
    if lens[s] <= 0:
        return 0
    o = off[s] + col * (lens[s] + cost) + cost
    return min(n_splits, (o + lens[s] - 1) // q - o // q + 1)


def check(starts, ends, n_cols, grid, min_keys, cost, n_heads_per_col=16):
    max_len = max(1, max(e - b for b, e in zip(starts, ends)))
    segs, lens, off, q, n_splits = replay(starts, ends, n_cols, grid, min_keys, cost, max_len)
    for s in range(len(starts)):
        for c in range(n_cols):
            mine = sorted((t0, t1, sp) for (_, ss, cc, t0, t1, sp) in segs if ss == s and cc == c)
            covered = [t for t0, t1, _ in mine for t in range(t0, t1)]
            assert covered == list(range(starts[s], starts[s] + lens[s])), (s, c)
            slots = [sp for _, _, sp in mine]
            assert slots == list(range(len(slots))), (s, c, slots)
            assert len(slots) == partials(lens, off, q, s, c, cost, n_splits), (s, c)
            assert all(0 <= sp < n_splits for sp in slots)
    # partial index ((s * n_heads + head) * n_splits + split) inside n_seq * n_heads * n_splits
    n_heads = n_cols * n_heads_per_col
    for (_, s, c, _, _, sp) in segs:
        for h in range(c * n_heads_per_col, (c + 1) * n_heads_per_col):
            assert (s * n_heads + h) * n_splits + sp < len(starts) * n_heads * n_splits
    return segs


def test_turbo_d256_group16_shape():
    """The test_turbo_decode_head_dims_and_groups[256-16-1] batch on the Turbo schedule
    (ranges >= 1024 keys, 512 virtual keys per pair, 256 resident workgroups): workgroup 0
    takes sequence 0, workgroup 1 sequences 1 and 2 in two segments, all in slot 0."""
    segs = check([0, 2, 400], [1, 33, 700], n_cols=1, grid=256, min_keys=1024, cost=512)
    assert [(b, s, t0, t1, sp) for (b, s, _, t0, t1, sp) in segs] == [
        (0, 0, 0, 1, 0), (1, 1, 2, 33, 0), (1, 2, 400, 700, 0)]


@pytest.mark.parametrize("seed", range(40))
def test_random_ragged_batches(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 40))
    lens = rng.integers(0, 5000, n)
    lens[rng.random(n) < 0.2] = 0
    if lens.max() == 0:
        lens[0] = 1
    starts = rng.integers(0, 300, n)
    ends = (starts + lens).tolist()
    turbo = seed % 2 == 0
    check(starts.tolist(), ends, n_cols=int(rng.integers(1, 5)), grid=int(rng.choice([16, 256, 512])),
          min_keys=1024 if turbo else 256, cost=512)


def test_max_sequences():
    """kStreamMaxSeq sequences of one key each."""
    check([0] * STREAM_MAX_SEQ, [1] * STREAM_MAX_SEQ, n_cols=2, grid=256, min_keys=256, cost=512)
