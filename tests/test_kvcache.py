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
