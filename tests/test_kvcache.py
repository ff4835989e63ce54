"""KVCache bookkeeping on the CPU against the reference's own fixture (native/live/tests/fixtures/ring.json,
copied to tests/golden/ring.json): the ring slots each commit writes, with a sink, multi-shot pins and resets."""

import json
from pathlib import Path

import torch

GOLDEN = Path(__file__).parent / "golden"


def test_ring_commits_match_reference_fixture():
    from wdl.kvcache import KVCache

    fx = json.loads((GOLDEN / "ring.json").read_text())
    per, chunk, window, sink = fx["tokens_per_frame"], fx["chunk"], fx["window"], fx["sink"]
    n = chunk * per
    cache = KVCache((window - chunk) * per, sink * per, chunk=chunk)
    cache.allocate(torch.zeros(1, n, 1, 4))
    steps, pin_next = [], False
    for op in fx["script"]:
        if op == "shot":
            pin_next = True
        elif op == "new":
            cache.reset()
            cache.last_slots = None
            pin_next = False
        else:
            at = cache.saved
            cache.commit()
            if pin_next:
                cache.pin_last()
            pin_next = False
            slots = None if cache.last_slots is None else cache.last_slots.tolist()
            steps.append(dict(at=at, saved=cache.saved, slots=slots))
    assert steps == fx["commits"]


def test_commit_copies_rows_into_evicted_slots():
    from wdl.kvcache import KVCache

    per, chunk = 2, 1
    cache = KVCache(4 * per, 0, chunk=chunk)
    cache.allocate(torch.zeros(1, per, 1, 8))
    for c in range(6):
        at = cache.saved
        val = torch.full((1, per, 1, 8), float(c + 1))
        cache.k[:, at:at + per] = val.to(torch.float8_e4m3fn)
        cache.commit()
    # window of 4 frames: chunks 3..6 survive (values 3, 4, 5, 6 at some rows)
    kept = sorted(set(cache.k[0, :8, 0, 0].float().tolist()))
    assert kept == [3.0, 4.0, 5.0, 6.0]


def test_a_pinned_chunk_larger_than_the_free_ring_is_evicted_last():
    """A ring of 6 slots (3 frames of 2 tokens) whose two oldest frames are a pinned shot chunk: a 4-token commit
    takes the one unpinned frame and then the oldest pinned slots (the reference ranks pinned tokens after all
    others, causal.py:329-337) instead of failing."""
    from wdl.kvcache import _FrameQueue

    q = _FrameQueue()
    q.append(0, 2, [0, 1, 2, 3], [0, 1, 2, 3])      # frames 0, 1 in slots 0..3
    q.append(2, 2, [0, 1], [4, 5])                  # frame 2 in slots 4, 5
    q.pinned = frozenset([0, 1, 2, 3])              # the shot's first chunk
    assert q.take_oldest(4) == [4, 5, 0, 1]         # the unpinned frame first, then the oldest pinned
    assert q.frames == [[1, [2, 3]]]
    q.append(3, 2, [0, 1, 2, 3], [4, 5, 0, 1])
    assert q.take_oldest(2) == [4, 5]               # slot 0 and 1 stay pinned with their new tokens
