"""The DiT step on latents and the DMD chunk loop, around the quantized blocks, on MI355X.

WanModel.forward (src/wan_dit_lab/models/model.py:32-84) with QuantizedWanBlock blocks:
  tokens = patch embedding of the latent (Conv3d, kernel = stride = (1, 2, 2), model.py:13, 36): one GEMM
           [f h w, in_dim * 4] x [in_dim * 4, dim] over the 2 x 2 patches, channel-major (ic, dy, dx) as the
           convolution weight [dim, in_dim, 1, 2, 2] flattens;
  t_emb  = time_embedding([cos(t omega), sin(t omega)]), omega = 10000^(-i / 128) in fp64 (model.py:38-40);
  e0     = time_projection(t_emb) as [6, dim] (41), each block's e = e0 + its modulation;
  flow   = Head (models/head.py:13-18): linear(LN(X) (1 + scale) + shift), (shift, scale) = modulation + t_emb,
           unpatchified to [out_dim, f, 2h, 2w] (model.py:82-84).
The edges are plain bf16 GEMMs and small normalisations, as the reference runs them under bf16 autocast
(causal.py:388-390): the linears take bf16 operands and return bf16, LayerNorm and the modulation run in fp32. They
go through torch (hipBLASLt for the GEMMs); the blocks run the wdl kernels.

ChunkStream.next_chunk restates Stream.next_chunk's DMD sampler (generation/causal.py:680-740) for the default
"video" positions: at each level sigma (causal.py:41-45) x0 = x - sigma flow, renoised to the next level with fresh
noise; then the write pass at t = 0 puts the final keys and values in the caches, which commit. With sampler "unipc"
the chunk is denoised by the UniPC sampler instead (causal.py:620-636, LongLive 2.0's; wdl.unipc): the model at the
sampler's integer timesteps, each input x_0 - C[k] . flows of the plan, the clean latents its last row. Not restated:
prompt blending, re-anchoring, shots and context noise.

ChunkStream.switch_resolution changes the latent size mid-stream (a mode of this build; the reference's Stream has a
fixed size, causal.py:471-472, and its recache, causal.py:662-678, re-encodes the window at the same size): the
clean latents of the chunks the caches hold are resampled to the new size (resample_latents), every block gets a
cache of the same window in frames at the new tokens per frame, and the resampled chunks are written into it by
the write pass (t = 0) at their original frame positions, oldest first, as recache does. The RoPE grid follows
from each call's latent size.
"""

from __future__ import annotations

from collections import deque

import torch
import torch.nn.functional as F

from wdl import unipc

SHIFT = 5.0                    # timestep_shift of the distilled model (causal.py:35)
STEPS = (1000, 750, 500, 250)  # its four timesteps before the shift (causal.py:36)
FREQ_DIM = 256                 # cos and sin of 128 frequencies


def sigmas(shift: float = SHIFT, steps=STEPS) -> list:
    """The DMD noise levels (causal.py:41-45): sigma = shift u / (1 + (shift - 1) u), u = t / 1000, in fp64."""
    u = torch.tensor(steps, dtype=torch.float64) / 1000
    return (shift * u / (1 + (shift - 1) * u)).tolist()


_OMEGA: dict = {}


def time_features(t: torch.Tensor) -> torch.Tensor:
    """[cos(t omega), sin(t omega)] in fp64, omega = 10000^(-i / 128), i < 128 (model.py:38-40) -> fp32 [B, 256]
    (omega made once per device)."""
    omega = _OMEGA.get(t.device)
    if omega is None:
        omega = _OMEGA[t.device] = 10000 ** (-torch.arange(128, dtype=torch.float64, device=t.device) / 128)
    theta = t.double()[:, None] * omega[None, :]
    return torch.cat([torch.cos(theta), torch.sin(theta)], dim=1).float()


def patch_matrix(x: torch.Tensor) -> torch.Tensor:
    """Latent [C, f, H, W] -> its 2 x 2 patches [f (H/2) (W/2), C 4], tokens in (f, i, j) order, features in the
    convolution weight's (ic, dy, dx) order."""
    C, f, H, W = x.shape
    if H % 2 or W % 2:
        raise ValueError(f"latent height and width must be even, got {H} x {W}")
    return x.reshape(C, f, H // 2, 2, W // 2, 2).permute(1, 2, 4, 0, 3, 5).reshape(f * (H // 2) * (W // 2), C * 4)


def resample_latents(x: torch.Tensor, height: int, width: int) -> torch.Tensor:
    """Latent frames [C, f, H, W] -> fp32 [C, f, height, width]: each frame and channel resampled bilinearly with
    half-pixel centres and, when shrinking, the triangle filter widened to the scale (F.interpolate, bilinear,
    align_corners=False, antialias=True)."""
    C, f, H, W = x.shape
    y = F.interpolate(x.float().permute(1, 0, 2, 3), size=(height, width), mode="bilinear", align_corners=False,
                      antialias=True)
    return y.permute(1, 0, 2, 3).contiguous()


class FrameHistory:
    """The clean latent frames the caches hold, as Stream.next_chunk keeps them (sink_latents / recent_latents,
    causal.py:535-536, 744-746): the first `sink` frames of the video stay; of the others the newest `ring` follow.
    Frames are (frame number, latents [C, H, W])."""

    def __init__(self, sink: int, ring: int):
        self.sink_frames, self.sink, self.recent = sink, [], deque(maxlen=max(ring, 0))

    def add(self, first_frame: int, x0: torch.Tensor):
        """The frames of a chunk x0 [C, f, H, W] starting at frame `first_frame`."""
        for f in range(x0.shape[1]):
            n = first_frame + f
            (self.sink if n < self.sink_frames else self.recent).append((n, x0[:, f]))

    def chunks(self, chunk: int) -> list:
        """[(first frame, latents [C, chunk, H, W])] of the kept frames, oldest first; ValueError unless they are
        whole chunks of consecutive frames (the reference's recache asserts the same, causal.py:672)."""
        frames = self.sink + list(self.recent)
        if len(frames) % chunk:
            raise ValueError(f"{len(frames)} kept frames are not whole chunks of {chunk}")
        out = []
        for g in range(0, len(frames), chunk):
            group = frames[g:g + chunk]
            first = group[0][0]
            if [n for n, _ in group] != list(range(first, first + chunk)):
                raise ValueError("the kept frames do not form whole chunks of consecutive frames")
            out.append((first, torch.stack([x for _, x in group], dim=1)))
        return out


def unpatchify(y: torch.Tensor, grid, out_dim: int) -> torch.Tensor:
    """Head output [f h w, 4 out_dim] ((1, 2, 2, out_dim) per token) -> [out_dim, f, 2h, 2w] (model.py:82-84)."""
    f, h, w = grid
    return y.view(f, h, w, 1, 2, 2, out_dim).permute(6, 0, 3, 1, 4, 2, 5).reshape(out_dim, f, h * 2, w * 2)


class ModelEdges:
    """P: patch_w [dim, in_dim, 1, 2, 2], patch_b [dim]; t1_w [dim, 256], t1_b, t2_w [dim, dim], t2_b
    (time_embedding); proj_w [6 dim, dim], proj_b (time_projection); head_w [4 out_dim, dim], head_b [4 out_dim],
    head_mod [2, dim] (Head.modulation). Stored bf16 (head_mod fp32) on `device`."""

    def __init__(self, P: dict, device, eps: float = 1e-6):
        bf = lambda t: t.to(device=device, dtype=torch.bfloat16).contiguous()
        self.dim, self.in_dim = P["patch_w"].shape[:2]
        self.out_dim = P["head_w"].shape[0] // 4
        self.eps = eps
        self.patch_w, self.patch_b = bf(P["patch_w"].reshape(self.dim, self.in_dim * 4)), bf(P["patch_b"])
        self.t1_w, self.t1_b, self.t2_w, self.t2_b = bf(P["t1_w"]), bf(P["t1_b"]), bf(P["t2_w"]), bf(P["t2_b"])
        self.proj_w, self.proj_b = bf(P["proj_w"]), bf(P["proj_b"])
        self.head_w, self.head_b = bf(P["head_w"]), bf(P["head_b"])
        self.head_mod = P["head_mod"].to(device=device, dtype=torch.float32).reshape(2, self.dim)

    def patchify(self, x: torch.Tensor) -> torch.Tensor:
        """Latent [in_dim, f, H, W] -> tokens bf16 [f (H/2) (W/2), dim]."""
        if x.shape[0] != self.in_dim:
            raise ValueError(f"latent has {x.shape[0]} channels, the patch embedding {self.in_dim}")
        return F.linear(patch_matrix(x.to(torch.bfloat16)), self.patch_w, self.patch_b)

    def time(self, t: torch.Tensor):
        """t [1] -> (t_emb bf16 [dim], e0 fp32 [6, dim])."""
        h = F.linear(time_features(t).to(torch.bfloat16), self.t1_w, self.t1_b)
        # one row: matrix-vector products (the 113 MB modulation projection streams its weights faster through
        # addmv than through a 1-row GEMM; step -0.04 ms)
        t_emb = torch.addmv(self.t2_b, self.t2_w, F.silu(h)[0])
        e0 = torch.addmv(self.proj_b, self.proj_w, F.silu(t_emb))
        return t_emb, e0.float().view(6, self.dim)

    def head(self, X: torch.Tensor, t_emb: torch.Tensor, grid, ln_partials=None) -> torch.Tensor:
        """Tokens bf16 [f h w, dim] -> flow bf16 [out_dim, f, 2h, 2w]. ln_partials: the LayerNorm chunk partials of X
        (as the last block's residual GEMM wrote them); with them the LayerNorm and modulation run as one launch of
        the activation quantizer's LayerNorm path (its bf16 copy of the modulated rows), the statistics in the
        partials' order; without them, through torch."""
        shift, scale = self.head_mod + t_emb.float()[None, :]
        if ln_partials is not None:
            from wdl import ops

            if not hasattr(self, "_ones"):
                self._ones = torch.ones(self.dim, device=X.device, dtype=torch.bfloat16)
            y = torch.empty_like(X)
            ops.act_quant_launch(X, self._ones, None, ln=dict(shift=shift.contiguous(), scale=scale.contiguous(),
                                                             weight=None, bias=None, eps=self.eps,
                                                             partials=ln_partials), v_out=y)
        else:
            y = (F.layer_norm(X.float(), (self.dim,), eps=self.eps) * (1 + scale) + shift).to(torch.bfloat16)
        return unpatchify(F.linear(y, self.head_w, self.head_b), grid, self.out_dim)


def random_edges(dim: int, in_dim: int, out_dim: int, generator: torch.Generator, std: float = 0.02) -> dict:
    """Random-init edge weights of the architecture (linears and the patch convolution N(0, std^2), biases 0,
    head modulation N(0, 1) / sqrt(dim) as Head initialises it), on the generator's device."""
    g, dev = generator, generator.device
    n = lambda *s: torch.randn(*s, generator=g, device=dev) * std
    z = lambda *s: torch.zeros(*s, device=dev)
    return dict(patch_w=n(dim, in_dim, 1, 2, 2), patch_b=z(dim), t1_w=n(dim, FREQ_DIM), t1_b=z(dim),
                t2_w=n(dim, dim), t2_b=z(dim), proj_w=n(6 * dim, dim), proj_b=z(6 * dim),
                head_w=n(4 * out_dim, dim), head_b=z(4 * out_dim),
                head_mod=torch.randn(2, dim, generator=g, device=dev) / dim ** 0.5)


class DiTModel:
    """The step of WanModel.forward on one chunk: edges + QuantizedWanBlocks, one KVCache and one prepared context
    per block (the prompt's cross-attention keys and values, computed once, as causal.Stream.cross does)."""

    def __init__(self, edges: ModelEdges, blocks: list, caches: list, context: torch.Tensor, freq: torch.Tensor):
        self.edges, self.blocks, self.caches, self.freq = edges, blocks, caches, freq
        self.ctx = [b.prepare_context(context) for b in blocks]
        self.modulation = torch.stack([b.p["modulation"] for b in blocks])  # [blocks, 6, dim]

    def forward(self, x: torch.Tensor, t: torch.Tensor, start_frame: int) -> torch.Tensor:
        """Latent [in_dim, f, H, W], t [1] -> flow bf16 [out_dim, f, H, W]; each block attends over its cache and
        writes the chunk's keys and values at its write offset."""
        _, f, H, W = x.shape
        grid = (f, H // 2, W // 2)
        X = self.edges.patchify(x)
        t_emb, e0 = self.edges.time(t)
        e_all = e0 + self.modulation
        # each block's feed-forward residual GEMM writes the LayerNorm chunk partials of X for the next block's first
        # LayerNorm (two buffers in turn); block 0 forms its own
        lnb = torch.empty(2, X.shape[0], X.shape[1] // 32, 2, device=X.device, dtype=torch.float32)
        ln_in = None
        for i, (blk, cache, ctx, e) in enumerate(zip(self.blocks, self.caches, self.ctx, e_all)):
            blk.forward(X, e, grid, self.freq, start_frame, cache, ctx, ln_in=ln_in, ln_out=lnb[i % 2])
            ln_in = lnb[i % 2]
        return self.edges.head(X, t_emb, grid, ln_partials=ln_in)


class ChunkStream:
    """Stream.next_chunk's loop (causal.py:680-740, positions "video", no context noise) over a DiTModel: chunks of
    `shape` [in_dim, chunk, H, W] latents, one after another. sampler "dmd" (Self-Forcing's, at `levels`) or "unipc"
    (`steps` of LongLive 2.0's sampler, 4 by default as the reference's; its live preset runs 2); `steps` only with
    "unipc" (causal.py:525-528)."""

    def __init__(self, model: DiTModel, shape, generator: torch.Generator, levels=None, write_pass: bool = True,
                 sampler: str = "dmd", steps: int | None = None, shift: float = SHIFT):
        if sampler not in ("dmd", "unipc"):
            raise ValueError(f"unknown sampler {sampler!r}")
        if steps is not None and sampler != "unipc":
            raise ValueError("the dmd sampler has the fixed timesteps of its levels")
        self.model, self.shape, self.generator = model, tuple(shape), generator
        self.levels = sigmas(shift) if levels is None else list(levels)
        self.write_pass, self.start, self.sampler = write_pass, 0, sampler
        self.history = None  # FrameHistory of the clean frames the caches hold (made at the first chunk)
        if sampler == "unipc":
            timesteps, C = unipc.plan(steps or len(STEPS), shift)
            self.timesteps, self.plan = timesteps, C.tolist()

    @torch.no_grad()
    def next_chunk(self, noise: torch.Tensor | None = None) -> torch.Tensor:
        """Latents fp32 [in_dim, chunk, H, W] of the next chunk, from `noise` of that shape or fresh noise."""
        dev = self.model.freq.device
        x = torch.randn(self.shape, generator=self.generator, device=dev) if noise is None else noise.float()
        x0 = x
        if self.sampler == "unipc":
            x0 = self._unipc(x)
        for i, sigma in enumerate(self.levels if self.sampler == "dmd" else ()):
            t = torch.full((1,), 1000 * sigma, device=dev)
            flow = self.model.forward(x, t, self.start).float()
            x0 = x - sigma * flow  # x_t = (1 - sigma) x0 + sigma noise, flow = noise - x0
            if i + 1 < len(self.levels):
                fresh = torch.randn(x0.shape, generator=self.generator, device=dev)
                x = (1 - self.levels[i + 1]) * x0 + self.levels[i + 1] * fresh
        if self.write_pass:  # the final latents' keys and values into the caches (t = 0)
            self.model.forward(x0, torch.zeros(1, device=dev), self.start)
        for cache in self.model.caches:
            cache.commit()
        self._keep(self.start, x0)
        self.start += self.shape[1]
        return x0

    def _window(self):
        """(frames the caches hold, of which sink) at the current latent size."""
        c = self.model.caches[0]
        per_frame = (self.shape[2] // 2) * (self.shape[3] // 2)
        return c.max_tokens // per_frame, c.sink_tokens // per_frame

    def _window_split(self):
        frames, sink = self._window()
        return sink, frames - sink

    def _keep(self, first_frame: int, x0: torch.Tensor):
        if self.history is None:
            self.history = FrameHistory(*self._window_split())
        self.history.add(first_frame, x0)

    @property
    def kept(self) -> list:
        """(first frame, clean latents [C, chunk, H, W]) of the chunks the caches hold, oldest first."""
        return [] if self.history is None else self.history.chunks(self.shape[1])

    @kept.setter
    def kept(self, chunks):
        self.history = FrameHistory(*self._window_split())
        for first, x0 in chunks:
            self.history.add(first, x0)

    @torch.no_grad()
    def switch_resolution(self, height: int, width: int):
        """Continue the stream at latents of height x width: the kept chunks resampled, each block's cache rebuilt
        for the same window in frames at the new tokens per frame and refilled by the write pass over them (t = 0,
        their original frame positions, oldest first; the caches commit after each, as recache does)."""
        from wdl.kvcache import KVCache

        if height % 2 or width % 2 or height <= 0 or width <= 0:
            raise ValueError(f"latent height and width must be positive and even, got {height} x {width}")
        frames, sink = self._window()
        chunk = self.shape[1]
        if sink % chunk or (frames - sink) % chunk:
            raise ValueError("the resolution switch re-encodes whole chunks: the window and its sink must hold "
                             f"whole chunks of {chunk} frames (window {frames}, sink {sink})")
        kept = self.kept  # raises before anything changes if the kept frames are not whole chunks
        per_frame = (height // 2) * (width // 2)
        self.model.caches[:] = [KVCache(frames * per_frame, sink * per_frame, chunk=chunk,
                                        entropy_ratio=c.entropy_ratio) for c in self.model.caches]
        self.shape = (self.shape[0], chunk, height, width)
        self.history = FrameHistory(*self._window_split())
        dev = self.model.freq.device
        for first, x0 in kept:
            x = resample_latents(x0, height, width)
            self.model.forward(x, torch.zeros(1, device=dev), first)
            for cache in self.model.caches:
                cache.commit()
            self._keep(first, x)

    def _unipc(self, noise: torch.Tensor) -> torch.Tensor:
        """The UniPC steps from `noise`: the model at each timestep on x_0 - C[k] . flows; the clean latents."""
        flows, x = [], noise
        for k, t in enumerate(self.timesteps):
            flows.append(self.model.forward(x, torch.full((1,), float(t), device=noise.device), self.start).float())
            x = noise
            for c, f in zip(self.plan[k + 1], flows):
                x = x - c * f
        return x
