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


def test_anchor_rows_are_the_newest_frame_in_topk_order():
    """Forcing-KV's anchor (causal.py:243-248): the ring tokens with the largest (frame, place) order, as torch.topk
    ranks them (largest first), after the sink. Checked against an independent per-slot bookkeeping of the frame and
    place of every ring token over 9 commits (the window fills, then evicts the oldest frames)."""
    from wdl.kvcache import KVCache

    per, chunk, window, sink = 3, 2, 10, 2
    n = chunk * per
    cache = KVCache((window - chunk) * per, sink * per, chunk=chunk)
    cache.allocate(torch.zeros(1, n, 1, 4))
    ring = (window - chunk - sink) * per
    frame_of = torch.full((ring,), -1, dtype=torch.long)  # -1: no token yet (never the newest)
    place = torch.zeros(ring, dtype=torch.long)
    for c in range(9):
        frames_before = cache.frames
        cache.commit()
        if cache.last_slots is not None:
            # the chunk's tokens past the sink, in token order (the tail of the chunk when part of it is sink)
            i = torch.arange(n - len(cache.last_slots), n)
            frame_of[cache.last_slots] = frames_before + i // per
            place[cache.last_slots] = i % per
        order = torch.where(frame_of >= 0, frame_of * per + place, torch.full_like(frame_of, -1))
        if int((frame_of >= 0).sum()) >= per:
            want = (sink * per + torch.topk(order, per).indices).tolist()
            assert cache.anchor_rows() == want, (c, cache.anchor_rows(), want)


def test_evicted_and_copy_have_the_reference_signatures():
    """KVCache.evicted(n) names the ring slots the next commit takes (oldest frames first, causal.py:329-337) without
    changing the cache, and KVCache.copy(to, at, n) moves rows [at, at + n) of all four buffers, FP8 as bytes
    (causal.py:339-343): a full-window commit equals copy(sink + evicted(n), at, n) by hand."""
    from wdl.kvcache import KVCache

    per, chunk, window, sink = 2, 2, 8, 2
    n = chunk * per
    g = torch.Generator().manual_seed(4)
    a = KVCache((window - chunk) * per, sink * per, chunk=chunk)
    b = KVCache((window - chunk) * per, sink * per, chunk=chunk)
    for c in (a, b):
        c.allocate(torch.zeros(1, n, 1, 4))
    for _ in range(5):  # past a full window
        at = a.saved
        rows = torch.randn(1, n, 1, 4, generator=g) * 50
        for c in (a, b):
            c.k[:, at:at + n] = rows.clamp(-448, 448).to(torch.float8_e4m3fn)
            c.v[:, at:at + n] = (-rows).clamp(-448, 448).to(torch.float8_e4m3fn)
            c.ks[:, at:at + n] = rows.abs().amax(-1, keepdim=True)
            c.vs[:, at:at + n] = rows.abs().amin(-1, keepdim=True)
        if a.full():
            slots = a.evicted(n)
            assert torch.equal(a.evicted(n), slots)  # asking twice changes nothing
            b.copy(sink * per + slots, at, n)
            a.commit()
            assert a.last_slots.tolist() == slots.tolist()
            for x, y in ((a.k, b.k), (a.v, b.v)):
                assert torch.equal(x[:, :at].view(torch.uint8), y[:, :at].view(torch.uint8))
            assert torch.equal(a.ks[:, :at], b.ks[:, :at]) and torch.equal(a.vs[:, :at], b.vs[:, :at])
            b.saved, b.frames = a.saved, a.frames
            b.queue.frames = [[f, list(s)] for f, s in a.queue.frames]
        else:
            a.commit()
            b.commit()
