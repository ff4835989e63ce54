"""KVCache of one block on MI355X: the FP8 keys/values of the finished frames in one device buffer allocated once, the
hot-path subset of src/wan_dit_lab/generation/causal.py:48-343 (KVCache).

Device side. One buffer [1, max_tokens + n, H, D] in e4m3 per K and V with fp32 scales per (token, head)
([1, max_tokens + n, H, 1]). Rows [0, sink_tokens) are the sink, never evicted; rows [sink_tokens, max_tokens) are
the ring; the last n rows take the chunk once the ring is full. attend() writes the chunk (wdl_kv_append_fp8) at
row `saved` and attends over rows [0, saved) and the chunk (wdl::sage_kv_attend), the sage + fp8 branch of
KVCache.attend (causal.py:193-210).

Column statistics. The Sage preparation needs the K column means and |V| column maxima over every key it attends
to. Those of rows [0, saved) change only when those rows do (a commit, a reset, a new `saved`), while a chunk runs
its denoising levels and write pass over the same rows; so the cache keeps them (`stats`, fp32 [2, H, 128]: K sums
and |V| maxima, wdl_sage_cache_stats), refreshes them eagerly at a commit and lazily at the next attend after
`saved` is set, and attend's preparation reads only the chunk's own tokens beside them. A caller that writes rows
[0, saved) itself calls invalidate_stats() afterwards. A HIP graph captured over attend reads `stats` in place, so
its replays stay correct across commits.

Host side. Which ring slot holds which token is bookkeeping on the host (`_FrameQueue`): the ring's frames in the
order they were committed, each with the slots of its tokens in token order. Attention does not depend on where a
key sits, only the eviction order does, and the reference defines it as "the oldest unpinned tokens of the video
first" (causal.py:329-337); walking the queue from its head, skipping pinned slots, yields exactly that order
without sorting. The slot numbers a commit produces are pinned by the reference's own fixture
(native/live/tests/fixtures/ring.json, in tests/golden/).

Forcing-KV head split (set_heads, causal.py:98-104, 222-248): once the window is full, the dynamic heads attend over
the whole window and the static heads over the sink and the newest finished frame only (anchor_tokens: the sink's
rows, then the newest frame's rows in decreasing token order, as the reference's topk gives them, refreshed at every
commit); both read the one cache through the heads / tokens maps of the Sage preparation, nothing copied.

Positions-in-window turns, Echo-Forcing decay and Participative Compression are not on this hot path and are not
implemented here.
"""

from __future__ import annotations

import math

import torch

from wdl.cache_fp8 import store_kv_fp8

FP8 = torch.float8_e4m3fn
CHUNK = 3
CONTEXT = 21


class _FrameQueue:
    """The ring's frames, oldest first: entries [frame number, [slot of each remaining token, in token order]].
    A frame loses tokens from its front when they are evicted; an empty frame leaves the queue."""

    def __init__(self):
        self.frames: list[list] = []
        self.pinned: frozenset = frozenset()

    def clear(self):
        self.frames = []
        self.pinned = frozenset()

    def append(self, first_frame: int, per_frame: int, tokens: list[int], slots: list[int]):
        """Chunk tokens `tokens` (indices within the chunk, increasing) now live in `slots`."""
        for i, s in zip(tokens, slots):
            f = first_frame + i // per_frame
            if not self.frames or self.frames[-1][0] != f:
                self.frames.append([f, []])
            self.frames[-1][1].append(s)

    def take_oldest(self, n: int) -> list[int]:
        """Removes and returns the n oldest unpinned slots (in token order of the video). When fewer than n are
        unpinned, the oldest pinned slots follow: the reference ranks pinned tokens after every other one
        (causal.py:329-337, the pinned order masked to the largest value) and leaves the order among them to
        torch.topk; here it is the video's. A slot stays pinned when a new token takes it, as the reference's
        per-slot mask does."""
        out = self._take(n, lambda s: s not in self.pinned)
        if len(out) < n:
            out += self._take(n - len(out), lambda s: True)
        if len(out) < n:
            raise RuntimeError(f"the ring has {len(out)} tokens, the chunk needs {n}")
        return out

    def _take(self, n: int, eligible) -> list[int]:
        out: list[int] = []
        for entry in self.frames:
            keep = []
            for s in entry[1]:
                if len(out) < n and eligible(s):
                    out.append(s)
                else:
                    keep.append(s)
            entry[1] = keep
            if len(out) == n:
                break
        self.frames = [e for e in self.frames if e[1]]
        return out


class KVCache:
    def __init__(self, max_tokens: int, sink_tokens: int = 0, chunk: int = CHUNK, entropy_ratio=None):
        self.max_tokens, self.sink_tokens, self.chunk = max_tokens, sink_tokens, chunk
        self.entropy_ratio = entropy_ratio
        self.fp8 = True
        self.k = self.v = None
        self.queue = _FrameQueue()
        self.static_heads = None  # Forcing-KV: the heads that see only the sink and the newest frame (set_heads)
        self._groups = None
        self.stats = None
        self._stats_at = -1  # rows [0, _stats_at) are what `stats` describes; -1: stale
        self.reset()

    @property
    def saved(self) -> int:
        """Rows [0, saved) hold the committed tokens."""
        return self._saved

    @saved.setter
    def saved(self, value: int):
        self._saved = value
        self._stats_at = -1

    def invalidate_stats(self):
        """To call after writing rows [0, saved) other than through attend / commit."""
        self._stats_at = -1

    def _refresh_stats(self):
        from wdl.ops import sage_cache_stats_launch

        if self.k is None or not self.k.is_cuda:  # the statistics live beside device buffers only
            return
        self.stats = sage_cache_stats_launch(self.k.view(torch.uint8), self.ks, self.v.view(torch.uint8), self.vs,
                                             self.saved, out=self.stats)
        self._stats_at = self.saved

    def reset(self):
        """Empties the cache; the buffers stay (causal.py:104-114)."""
        self.saved = 0
        self.frames = 0
        self.last_slots = None
        self.queue.clear()

    def set_heads(self, static, heads: int):
        """static: the head numbers (of `heads`) that attend to the sink, the newest finished frame and the chunk
        once the cache is full; None or empty: every head sees the whole window (causal.py:98-104)."""
        self.static_heads = sorted(static) if static else None
        self.dynamic_heads = [h for h in range(heads) if h not in (static or ())]
        self._groups = None
        self.__dict__.pop("anchor_tokens", None)

    def full(self) -> bool:
        return self.k is not None and self.saved == self.max_tokens

    def scale(self, keys: int, head_dim: int):
        """None (1/sqrt(d)) or the entropy-preserving sqrt(log_T N / d), T = keys * ratio (causal.py:138-142)."""
        if self.entropy_ratio is None:
            return None
        return math.sqrt(math.log(keys) / math.log(keys * self.entropy_ratio) / head_dim)

    def allocate(self, like: torch.Tensor):
        """Buffers for chunks shaped like `like` [1, n, H, D] (causal.py:149-175)."""
        B, n, H, D = like.shape
        dev = like.device
        self.n, self.per_frame = n, n // self.chunk
        rows = self.max_tokens + n
        self.k = torch.zeros(B, rows, H, D, dtype=FP8, device=dev)
        self.v = torch.zeros_like(self.k)
        self.ks = torch.ones(B, rows, H, 1, device=dev)
        self.vs = torch.ones_like(self.ks)
        self.stats = torch.zeros(2, H, D, device=dev) if like.is_cuda else None
        self._stats_at = -1
        self.last_slots = None
        self.queue.clear()

    def store(self, at: int, K: torch.Tensor, V: torch.Tensor):
        store_kv_fp8(K, V, self.k, self.ks, self.v, self.vs, at)

    def attend(self, Q, K, V):
        """softmax(Q K^T / sqrt(d)) V over the saved frames and the chunk; [1, tokens, H, D] (causal.py:193-220)."""
        from wdl.sage_kv import attend

        if self.k is None:
            self.allocate(V)
        n, at = K.shape[1], self.saved
        if self.static_heads is not None and self.full():
            self.store(at, K, V)
            return self.attend_split(Q, K, V, at, n)
        if self._stats_at != at:
            self._refresh_stats()
        # the store of the chunk (rows at .. at + n, the bytes and scales store() writes) runs inside the
        # preparation pass of the attention, which reads the chunk anyway
        return attend(Q, self.k, self.ks, self.v, self.vs, at, K, V, sm_scale=self.scale(at + n, Q.shape[-1]),
                      cache_stats=self.stats, append=True)

    def _head_groups(self, dev):
        """[(cache heads int32, as index, cache rows int32 or None)] of the two Forcing-KV groups, made once per
        set_heads: the dynamic heads read rows [0, at), the static ones anchor_tokens (the sink's rows, then the
        newest finished frame's, which commit rewrites in place)."""
        if self._groups is None:
            self.anchor_tokens = torch.zeros(self.sink_tokens + self.per_frame, device=dev, dtype=torch.int32)
            self.anchor_tokens[:self.sink_tokens] = torch.arange(self.sink_tokens, device=dev, dtype=torch.int32)
            self.place_anchor()
            groups = []
            for heads, rows in ((self.dynamic_heads, None), (self.static_heads, self.anchor_tokens)):
                if heads:
                    idx = torch.tensor(heads, device=dev, dtype=torch.int32)
                    groups.append((idx, idx.long(), rows))
            self._groups = groups
        return self._groups

    def attend_split(self, Q, K, V, at: int, n: int):
        """Forcing-KV over the FP8 cache (causal.py:222-241): each head group attends with its own heads' columns
        of Q, K, V over the one cache, read through the head map and, for the static heads, the row map (nothing
        of the cache copied); [1, n, H, D] bf16."""
        from wdl.sage_kv import attend

        A = torch.empty(Q.shape, device=Q.device, dtype=torch.bfloat16)
        for idx, cols, rows in self._head_groups(Q.device):
            length = at if rows is None else rows.numel()
            A[:, :, cols] = attend(Q[:, :, cols].contiguous(), self.k, self.ks, self.v, self.vs, length,
                                   K[:, :, cols].contiguous(), V[:, :, cols].contiguous(),
                                   sm_scale=self.scale(length + n, Q.shape[-1]), heads=idx, tokens=rows)
        return A

    def anchor_rows(self) -> list[int]:
        """The cache rows of the newest finished frame, in decreasing token order (the largest frame and place of
        the ring first, as torch.topk ranks them in the reference, causal.py:243-248)."""
        newest = self.queue.frames[-1][1] if self.queue.frames else []
        return [self.sink_tokens + s for s in reversed(newest)]

    def place_anchor(self):
        """The newest finished frame's rows into anchor_tokens after the sink, in place (a captured graph reads
        them)."""
        rows = self.anchor_rows()
        if len(rows) != self.per_frame:
            raise RuntimeError(f"the newest frame holds {len(rows)} ring tokens, a frame has {self.per_frame}")
        self.anchor_tokens[self.sink_tokens:] = torch.tensor(rows, dtype=torch.int32).to(self.anchor_tokens.device)

    def commit(self):
        """Keeps the chunk that attend last wrote at row `saved` (causal.py:297-327, without turns, decay or
        compression). While the ring has room the chunk stays where it is; once full it moves into the slots of
        the oldest unpinned tokens. last_slots: the ring slots its tokens took (None when the window is the chunk
        alone)."""
        n, at, sink = self.n, self.saved, self.sink_tokens
        if at + n <= self.max_tokens:
            first = max(at, sink)  # rows of the chunk in the sink stay there; the rest enter the ring in place
            tokens = list(range(first - at, n))
            slots = [at + i - sink for i in tokens]
            self.saved = at + n
        elif self.max_tokens > sink:
            tokens = list(range(n))
            slots = self.queue.take_oldest(n)
            self.copy([sink + s for s in slots], at, n)
        else:
            tokens = slots = None
        if slots is not None:
            self.queue.append(self.frames, self.per_frame, tokens, slots)
            self.last_slots = torch.tensor(slots, dtype=torch.long)
        else:
            self.last_slots = None
        self.frames += self.chunk
        if self._groups is not None and self.max_tokens > sink and self.full():  # anchors are read when full
            self.place_anchor()
        self._refresh_stats()  # rows [0, saved) changed

    def evicted(self, n: int) -> torch.Tensor:
        """Ring indices (long) of the n tokens the next chunk replaces once the window is full, oldest first: the
        oldest unpinned tokens in video order, then pinned ones (causal.py:329-337). The cache is not changed."""
        probe = _FrameQueue()
        probe.frames = [[f, list(slots)] for f, slots in self.queue.frames]
        probe.pinned = self.queue.pinned
        return torch.tensor(probe.take_oldest(n), dtype=torch.long)

    def copy(self, to, at: int, n: int):
        """Rows [at, at + n) of the four buffers to the buffer rows `to` (n indices), one row per token in order;
        FP8 rows move as bytes (causal.py:339-343)."""
        dev = self.k.device
        dst = torch.as_tensor(to, dtype=torch.long).to(dev)
        if dst.numel() != n:
            raise ValueError(f"copy: {dst.numel()} destination rows for {n} tokens")
        for buf in (self.k, self.v, self.ks, self.vs):
            rows = buf[0].view(torch.uint8) if buf.dtype == FP8 else buf[0]
            rows.index_copy_(0, dst, rows[at:at + n].clone())

    def pin_last(self):
        """The chunk just committed (a new shot's first chunk) stays in the ring until the next pin; the one pinned
        before becomes evictable (causal.py:126-133)."""
        pins = [] if self.last_slots is None else self.last_slots.tolist()
        if len(pins) >= self.max_tokens - self.sink_tokens:
            raise ValueError("a pinned chunk must leave room in the ring for the next one")
        self.queue.pinned = frozenset(pins)

    def fill_for_benchmark(self, generator=None):
        """A full window of random FP8 keys/values (scales 1/448-ish), as after max_tokens / per_frame committed
        frames: saved = max_tokens and the ring's frames in order."""
        rows = self.max_tokens
        g = generator
        for buf, sc in ((self.k, self.ks), (self.v, self.vs)):
            x = torch.randn(buf.shape[0], rows, *buf.shape[2:], generator=g, device=buf.device)
            buf[:, :rows] = (x * 100).clamp(-448, 448).to(FP8)
            sc[:, :rows] = 0.01
        self.saved = rows
        self.queue.clear()
        ring = self.max_tokens - self.sink_tokens
        first = self.sink_tokens // self.per_frame
        self.queue.append(first, self.per_frame, list(range(ring)), list(range(ring)))
        self.frames = rows // self.per_frame
        self._refresh_stats()
