"""3D (time, height, width) RoPE, CPU restatement of src/wan_dit_lab/models/rope.py and positions.py.

- rope(count, dim) (rope.py:4-10): cos/sin tables [2, count, dim/2] of angle pos * 10000^(-2i/dim), float64.
- freqs(dim, positions, dtype): the three axis tables concatenated: a head's 64 pairs split [22 time, 21 height,
  21 width] for d = 128 (rope.py:16-17; tests/test_kv_cache.py:12).
- rope_apply(X, grid, freq, start_frame) (rope.py:12-31): token i of a (f, h, w) grid has position
  (start_frame + i // (h w), (i // w) % h, i % w); pair (x1, x2) -> (x1 c - x2 s, x2 c + x1 s) in the promoted
  dtype of X and freq, result in X's dtype. Tokens past f h w are returned unchanged (the Triton op's padding rule,
  kernels/rope_triton.py:54-56).

Pinned by: the fp64 complex oracle of tests/test_rope_triton.py:21-45 (restated as rope_complex); norm
preservation, the relative-position identity and the chunk-offset identity (test_rope_triton.py:89-104); the axis
split [22, 21, 21] (Appendix-B known answer).
"""

from __future__ import annotations

import torch


def rope(pos_count: int, pos_dim: int) -> torch.Tensor:
    pairs = pos_dim // 2
    positions = torch.arange(pos_count)[:, None]
    idx = torch.arange(pairs, dtype=torch.float64)
    angles = positions * (10000 ** (-2 * idx / pos_dim))
    return torch.stack((torch.cos(angles), torch.sin(angles)))


def axis_split(dim: int):
    c = dim // 2
    return [c - 2 * (c // 3), c // 3, c // 3]


def freqs(dim: int = 128, positions: int = 1024, dtype=torch.float64) -> torch.Tensor:
    """[2, positions, dim/2]: the time, height and width tables side by side (tests/test_kv_cache.py:12)."""
    t, s, _ = axis_split(dim)
    return torch.cat([rope(positions, 2 * t), rope(positions, 2 * s), rope(positions, 2 * s)], dim=-1).to(dtype)


def positions(grid, start_frame: int = 0) -> torch.Tensor:
    """[f h w, 3] integer positions (time, height, width) of a grid."""
    f, h, w = grid
    i = torch.arange(f * h * w)
    return torch.stack([start_frame + i // (h * w), (i // w) % h, i % w], dim=1)


def rope_apply(X: torch.Tensor, grid, freq: torch.Tensor, start_frame: int = 0) -> torch.Tensor:
    """rope.py:12-31 for one grid (batch 1 or one shared grid), X [B, L, H, D]."""
    f, h, w = grid
    c = X.size(3) // 2
    sizes = axis_split(X.size(3))
    time, height, width = freq.split(sizes, dim=-1)
    C, S = torch.cat([
        time[:, start_frame:start_frame + f].view(2, f, 1, 1, -1).expand(2, f, h, w, -1),
        height[:, :h].view(2, 1, h, 1, -1).expand(2, f, h, w, -1),
        width[:, :w].view(2, 1, 1, w, -1).expand(2, f, h, w, -1),
    ], dim=-1).reshape(2, f * h * w, 1, c)
    n = f * h * w
    Xr = X[:, :n]
    X1, X2 = Xr[..., ::2], Xr[..., 1::2]
    out = torch.stack((X1 * C - X2 * S, X2 * C + X1 * S), dim=-1).flatten(-2).type_as(X)
    return torch.cat([out, X[:, n:]], dim=1) if n < X.shape[1] else out


def rope_complex(x: torch.Tensor, grid, freq: torch.Tensor, start: int = 0) -> torch.Tensor:
    """The fp64 complex-phase oracle of tests/test_rope_triton.py:21-45 (one grid)."""
    pairs = x.shape[-1] // 2
    t, s, _ = axis_split(x.shape[-1])
    time, height, width = torch.complex(*freq.double()).split((t, s, s), dim=-1)
    f, h, w = grid
    n = f * h * w
    phase = torch.cat((time[start:start + f, None, None].expand(f, h, w, -1),
                       height[None, :h, None].expand(f, h, w, -1),
                       width[None, None, :w].expand(f, h, w, -1)), dim=-1).reshape(n, 1, pairs)
    v = x[:, :n].double().reshape(x.shape[0], n, x.shape[2], pairs, 2)
    even, odd = v[..., 0], v[..., 1]
    rot = torch.stack((even * phase.real - odd * phase.imag, odd * phase.real + even * phase.imag), dim=-1)
    return torch.cat((rot.flatten(-2).to(x.dtype), x[:, n:]), dim=1)


def rope_rotate(x: torch.Tensor, grids, freq: torch.Tensor, start: int = 0, inverse: bool = False,
                out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """The rotation of wan_dit_lab::rope3d_rotate (kernels/rope_triton.py:14-63, 66-81), x [B, L, H, dim] (any
    strides), one (f, h, w) grid per sample. Pair p of token i rotates by the angle of its axis: time pairs (the
    first dim/2 - 2 (dim/2 // 3)) at start + i // (h w), height pairs at (i // w) % h, width pairs at i % w;
    (e, o) -> (e c - o s, o c + e s), with s negated when inverse. Arithmetic in fp64 when x or freq is fp64, else
    fp32, each product rounded (no fused multiply-add); results for fp16 / bf16 outputs pass through fp32 (torch's
    own fp64 -> half casts do); tokens i >= f h w are copied."""
    out_dtype = x.dtype if out_dtype is None else out_dtype
    ct = torch.float64 if torch.float64 in (x.dtype, freq.dtype) else torch.float32
    B, L, H, dim = x.shape
    pairs = dim // 2
    t, s, _ = axis_split(dim)
    out = torch.empty(B, L, H, dim, dtype=out_dtype)
    to_out = (lambda v: v.float().to(out_dtype)) if out_dtype in (torch.float16, torch.bfloat16) else \
        (lambda v: v.to(out_dtype))
    for b, (f, h, w) in enumerate(grids):
        n = f * h * w
        i = torch.arange(n)
        pos = torch.empty(n, pairs, dtype=torch.long)
        pos[:, :t] = (start + i // (h * w))[:, None]
        pos[:, t:t + s] = ((i // w) % h)[:, None]
        pos[:, t + s:] = (i % w)[:, None]
        cols = torch.arange(pairs).expand(n, pairs)
        c = freq[0][pos, cols].to(ct)[:, None, :]
        sn = freq[1][pos, cols].to(ct)[:, None, :]
        if inverse:
            sn = -sn
        e, o = x[b, :n, :, 0::2].to(ct), x[b, :n, :, 1::2].to(ct)
        rot = torch.stack((e * c - o * sn, o * c + e * sn), dim=-1).flatten(-2)
        out[b, :n] = to_out(rot)
        out[b, n:] = to_out(x[b, n:].to(ct))
    return out
