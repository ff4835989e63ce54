"""The model edges and the DMD chunk loop on the CPU — test infrastructure, a restatement of
src/wan_dit_lab/models/model.py:32-84, models/head.py:13-18 and generation/causal.py:41-45, 680-740 around
oracle.block.block_forward. Only tests/ may import it.

Arithmetic as the reference runs it under bf16 autocast (causal.py:388-390): a linear or the patch convolution
takes bf16 operands, accumulates exactly enough to round once (fp64 here) and returns bf16; SiLU on bf16; the
Head's LayerNorm (no affine, eps 1e-6) and modulation in fp32, then the bf16 linear; the sinusoid in fp64.

Pinned by: the noise levels against the reference's own fixture (tests/test_causal_schedule.py:14:
[1, 0.9375, 5/6, 0.625]); the patch embedding as torch.nn.functional.conv3d (a textbook routine) of the same
weights; unpatchify as the exact inverse of the patch order (an index identity); the time features against
their closed form at t = 0 (cos 1, sin 0) and t with omega_0 = 1.

The mid-stream resolution switch has no reference counterpart (the reference's stream keeps its size,
causal.py:471-472; its recache, causal.py:662-678, re-encodes the window at the same size): resample() states
the build's latent resampling, separable, Pillow's antialiased bilinear (the triangle filter max(0, 1 - |t|)
widened to the scale when shrinking, half-pixel centres, weights normalised over the taps inside the frame), in
float64; reencode() writes resampled chunks into fresh caches by the write pass at their frame positions. Pinned
by (tests/test_switch.py): torch's antialiased bilinear interpolation (a library routine) on random frames,
the identity at the same size, and constant frames staying constant.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import block as oblock
from oracle import unipc as ounipc

BF = torch.bfloat16


def sigmas(shift: float = 5.0, steps=(1000, 750, 500, 250)) -> list:
    """causal.py:41-45 in fp64 scalars (no torch): sigma = shift u / (1 + (shift - 1) u), u = t / 1000."""
    out = []
    for t in steps:
        u = t / 1000.0
        out.append(shift * u / (1.0 + (shift - 1.0) * u))
    return out


def linear_bf16(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None) -> torch.Tensor:
    """A bf16 linear: bf16 operands, the sum in fp64, one rounding of (sum + bias) to bf16."""
    y = x.to(BF).double() @ w.to(BF).double().t()
    if b is not None:
        y = y + b.to(BF).double()
    return y.to(BF)


def linear_f32(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None) -> torch.Tensor:
    """An fp32 linear: the sum in fp64 of the fp32 operands, one rounding to fp32."""
    y = x.float().double() @ w.float().double().t()
    if b is not None:
        y = y + b.float().double()
    return y.float()


def _linear(dtype):
    return linear_bf16 if dtype == BF else linear_f32


def patch_embed(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, dtype=BF) -> torch.Tensor:
    """Conv3d(in_dim, dim, (1, 2, 2), (1, 2, 2)) of the latent [C, f, H, W] (model.py:13, 36), through
    torch's conv3d in fp64 on operands rounded to `dtype`, rounded to `dtype`: tokens [f h w, dim] in (f, i, j)
    order."""
    y = F.conv3d(x.to(dtype).double()[None], w.to(dtype).double(), b.to(dtype).double(), stride=(1, 2, 2))[0]
    return y.flatten(1).t().contiguous().to(dtype)


def time_embed(t: torch.Tensor, P: dict, dtype=BF):
    """model.py:38-41: (t_emb [dim], e0 [6, dim]) in `dtype` (bf16: the autocast step; fp32: the float model)."""
    lin = _linear(dtype)
    omega = 10000 ** (-torch.arange(128, dtype=torch.float64) / 128)
    theta = t.double()[:, None] * omega[None, :]
    feats = torch.cat([torch.cos(theta), torch.sin(theta)], dim=1).float()
    h = lin(feats, P["t1_w"], P["t1_b"])
    t_emb = lin(F.silu(h.float()).to(dtype), P["t2_w"], P["t2_b"])
    e0 = lin(F.silu(t_emb.float()).to(dtype), P["proj_w"], P["proj_b"])
    return t_emb[0], e0.reshape(6, -1)


def head(X: torch.Tensor, t_emb: torch.Tensor, P: dict, grid, eps: float = 1e-6, dtype=BF) -> torch.Tensor:
    """Head.forward (head.py:13-18) and unpatchify (model.py:82-84): tokens [f h w, dim] -> [out, f, 2h, 2w] in
    `dtype`."""
    dim = X.shape[1]
    shift, scale = P["head_mod"].float().reshape(2, dim) + t_emb.float()[None, :]
    y = F.layer_norm(X.float(), (dim,), eps=eps) * (1 + scale) + shift
    o = _linear(dtype)(y, P["head_w"], P["head_b"])
    out_dim = P["head_w"].shape[0] // 4
    f, h, w = grid
    return o.view(f, h, w, 1, 2, 2, out_dim).permute(6, 0, 3, 1, 4, 2, 5).reshape(out_dim, f, 2 * h, 2 * w)


def _model(x: torch.Tensor, t: torch.Tensor, E: dict, blocks, dtype) -> torch.Tensor:
    """WanModel.forward (model.py:32-84) on one chunk: patch embedding, time embedding, blocks(X, e0, grid), head
    and unpatchify."""
    _, f, H, W = x.shape
    grid = (f, H // 2, W // 2)
    X = patch_embed(x, E["patch_w"], E["patch_b"], dtype)
    t_emb, e0 = time_embed(t, E, dtype)
    return head(blocks(X, e0, grid), t_emb, E, grid, dtype=dtype)


def model_forward(x: torch.Tensor, t: torch.Tensor, E: dict, blocks: list, caches: list, ctx_kvs: list, freq,
                  start_frame: int, heads: int) -> torch.Tensor:
    """WanModel.forward on one chunk (model.py:32-84) with oracle blocks: latent [C, f, H, W] -> flow bf16. Each
    block's cache dict (k, ks, v, vs, at) receives the chunk's keys and values at `at`."""
    def run(X, e0, grid):
        for P, cache, kv in zip(blocks, caches, ctx_kvs):
            X = oblock.block_forward(X, e0.float(), P, grid, freq, start_frame, cache, kv, heads)
        return X

    return _model(x, t, E, run, BF)


def float_model_forward(x: torch.Tensor, t: torch.Tensor, E: dict, blocks: list, cache_kvs: list, ctxs: list, freq,
                        start_frame: int, heads: int) -> torch.Tensor:
    """The same model in fp32 with unquantized blocks (oracle.block.float_block_forward): latent -> flow fp32;
    cache_kvs[i] = (K, V) fp32 [Lc, D] the cached keys / values of block i, ctxs[i] its context fp32."""
    def run(X, e0, grid):
        for B, ckv, ctx in zip(blocks, cache_kvs, ctxs):
            X = oblock.float_block_forward(X, e0, B, grid, freq, start_frame, ckv, ctx, heads)
        return X

    return _model(x, t, E, run, torch.float32)


def next_chunk(noise: torch.Tensor, fresh: list, E: dict, blocks: list, caches: list, ctx_kvs: list, freq,
               start_frame: int, heads: int, levels=None, flow=None) -> torch.Tensor:
    """Stream.next_chunk's DMD loop (causal.py:680-740): x0 of one chunk from `noise`, renoising with the given
    `fresh` noises (one per level after the first), then the write pass at t = 0; the caches' write offsets `at`
    advance by the chunk's tokens (the commit of a cache that is not full). flow(x, t) replaces the oracle model
    (a model with a known exact flow, in the tests)."""
    levels = sigmas() if levels is None else levels
    run = flow if flow is not None else (
        lambda x, t: model_forward(x, t, E, blocks, caches, ctx_kvs, freq, start_frame, heads))
    x = noise.float()
    x0 = x
    for i, sigma in enumerate(levels):
        x0 = x - sigma * run(x, torch.full((1,), 1000 * sigma)).float()  # flow = noise - x0 (causal.py:716)
        if i + 1 < len(levels):
            x = (1 - levels[i + 1]) * x0 + levels[i + 1] * fresh[i]
    run(x0, torch.zeros(1))
    n = x0.shape[1] * (x0.shape[2] // 2) * (x0.shape[3] // 2)
    for cache in caches:
        cache["at"] += n
    return x0


def next_chunk_unipc(noise: torch.Tensor, E: dict, blocks: list, caches: list, ctx_kvs: list, freq, start_frame: int,
                     heads: int, steps: int = 2) -> torch.Tensor:
    """Stream.next_chunk with sampler "unipc" (causal.py:620-636, 709-710): oracle.unipc's sampler in float64 over
    the oracle model at the scheduler's integer timesteps, then the write pass at t = 0 and the commit."""
    def flow(x, t, k):
        f = model_forward(torch.from_numpy(x).float(), torch.full((1,), float(t)), E, blocks, caches, ctx_kvs, freq,
                          start_frame, heads)
        return f.double().numpy()

    x0 = torch.from_numpy(ounipc.sample(noise.double().numpy(), flow, steps)).float()
    model_forward(x0, torch.zeros(1), E, blocks, caches, ctx_kvs, freq, start_frame, heads)
    n = x0.shape[1] * (x0.shape[2] // 2) * (x0.shape[3] // 2)
    for cache in caches:
        cache["at"] += n
    return x0


def _taps(n_in: int, n_out: int):
    """Weights [n_out, n_in] of one axis of the antialiased bilinear resampling (float64)."""
    scale = n_in / n_out
    support = scale if scale >= 1 else 1.0
    inv = 1 / scale if scale >= 1 else 1.0
    W = np.zeros((n_out, n_in))
    for i in range(n_out):
        centre = scale * (i + 0.5)
        lo, hi = max(int(centre - support + 0.5), 0), min(int(centre + support + 0.5), n_in)
        w = np.array([max(0.0, 1 - abs((j - centre + 0.5) * inv)) for j in range(lo, hi)])
        W[i, lo:hi] = w / w.sum()
    return W


def resample(x: torch.Tensor, height: int, width: int) -> torch.Tensor:
    """Latent frames [C, f, H, W] -> fp32 [C, f, height, width], each frame through the row and column taps."""
    C, f, H, W = x.shape
    rows, cols = _taps(H, height), _taps(W, width)
    y = np.einsum("ih,cfhw,jw->cfij", rows, x.double().numpy(), cols)
    return torch.from_numpy(y).float()


def reencode(kept: list, E: dict, blocks: list, caches: list, ctx_kvs: list, freq, heads: int) -> None:
    """The write pass (t = 0) over the chunks `kept` [(first frame, latents at the new size)], oldest first, into
    `caches` (fresh, sized for the new tokens per frame); each cache's `at` advances by a chunk after each."""
    for first, x in kept:
        model_forward(x, torch.zeros(1), E, blocks, caches, ctx_kvs, freq, first, heads)
        n = x.shape[1] * (x.shape[2] // 2) * (x.shape[3] // 2)
        for cache in caches:
            cache["at"] += n
