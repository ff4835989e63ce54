"""KVCache of one block on MI355X: the FP8 keys/values of the finished frames in one buffer allocated once, the
hot-path subset of src/wan_dit_lab/generation/causal.py:48-343 (KVCache).

Buffer [1, max_tokens + n, H, D] in e4m3 with fp32 scales per (token, head) ([1, max_tokens + n, H, 1]). The first
sink_tokens are the sink, never evicted; the rest of max_tokens is the ring. While the ring fills, a chunk is
written right after the saved tokens and committing it moves a counter; once full, the chunk goes into the last n
rows and committing copies it over the tokens of the oldest unpinned frames (causal.py:297-337). pin_last keeps
the last committed chunk (a new shot's first chunk) in the ring until the next pin (causal.py:126-133).

attend writes the chunk (wdl_kv_append_fp8) and attends over the saved tokens and the chunk (wdl::sage_kv_attend:
cache tokens from FP8, the chunk's own K, V in bf16), as KVCache.attend's sage + fp8 branch (causal.py:193-210).
Positions-in-window turns, Echo-Forcing decay, Participative Compression and Forcing-KV head splits are not on
this hot path and are not implemented here.
"""

from __future__ import annotations

import math

import torch

from wdl.cache_fp8 import store_kv_fp8

FP8 = torch.float8_e4m3fn
CHUNK = 3
CONTEXT = 21


class KVCache:
    def __init__(self, max_tokens: int, sink_tokens: int = 0, chunk: int = CHUNK, entropy_ratio=None):
        self.max_tokens, self.sink_tokens, self.chunk = max_tokens, sink_tokens, chunk
        self.entropy_ratio = entropy_ratio
        self.fp8 = True
        self.k = self.v = None
        self.pinned = None
        self.reset()

    def reset(self):
        """Empties the cache; the buffers stay (causal.py:104-114)."""
        self.saved = 0
        self.frames = 0
        self.last_slots = None
        if self.pinned is not None:
            self.pinned.zero_()

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
        ring = self.max_tokens - self.sink_tokens
        self.frame_of = torch.zeros(ring, dtype=torch.long, device=dev)
        self.place_in_frame = torch.zeros_like(self.frame_of)
        self.pinned = torch.zeros(ring, dtype=torch.bool, device=dev)
        self.last_slots = None

    def store(self, at: int, K: torch.Tensor, V: torch.Tensor):
        store_kv_fp8(K, V, self.k, self.ks, self.v, self.vs, at)

    def attend(self, Q, K, V):
        """softmax(Q K^T / sqrt(d)) V over the saved frames and the chunk; [1, tokens, H, D] (causal.py:193-220)."""
        from wdl.sage_kv import attend

        if self.k is None:
            self.allocate(V)
        n, at = K.shape[1], self.saved
        self.store(at, K, V)
        return attend(Q, self.k, self.ks, self.v, self.vs, at, K, V, sm_scale=self.scale(at + n, Q.shape[-1]))

    def commit(self):
        """Keeps the chunk last written by attend (causal.py:297-327, without turns, decay or compression)."""
        n, at, per, sink = self.n, self.saved, self.per_frame, self.sink_tokens
        dev = self.frame_of.device
        i = torch.arange(n, device=dev)
        slots = None
        if at + n <= self.max_tokens:
            self.saved += n
            o = torch.arange(max(at, sink), max(at + n, sink), device=dev)
            slots, i = o - sink, o - at
        elif self.max_tokens > sink:
            slots = self.evicted(n)
            self.copy(sink + slots, at, n)
        self.last_slots = slots
        if slots is not None and len(slots):
            self.frame_of[slots] = self.frames + i // per
            self.place_in_frame[slots] = i % per
        self.frames += self.chunk

    def evicted(self, n: int) -> torch.Tensor:
        """Ring indices of the n tokens a chunk replaces: the oldest unpinned (causal.py:329-337)."""
        order = self.frame_of * self.per_frame + self.place_in_frame
        order = order.masked_fill(self.pinned, torch.iinfo(order.dtype).max)
        return torch.topk(order, n, largest=False).indices

    def copy(self, to: torch.Tensor, at: int, n: int):
        """Rows [at, at + n) of the four buffers to rows `to`, as bytes (causal.py:339-343)."""
        for buf in (self.k, self.v, self.ks, self.vs):
            raw = buf.view(torch.uint8) if buf.dtype == FP8 else buf
            raw[:, to] = raw[:, at:at + n].clone()

    def pin_last(self):
        """The chunk just committed stays in the ring until the next pin (causal.py:126-133)."""
        self.pinned.zero_()
        if self.last_slots is not None:
            assert int(self.last_slots.numel()) < len(self.pinned), "the ring must hold more than the pinned chunk"
            self.pinned[self.last_slots] = True

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
        ring = self.max_tokens - self.sink_tokens
        idx = torch.arange(ring, device=self.frame_of.device)
        self.frame_of.copy_(self.sink_tokens // self.per_frame + idx // self.per_frame)
        self.place_in_frame.copy_(idx % self.per_frame)
        self.frames = rows // self.per_frame
