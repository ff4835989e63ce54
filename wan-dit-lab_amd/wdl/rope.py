"""3D RoPE and the Q/K RMSNorm in front of it on MI355X (one fused HIP kernel, wdl_qk_norm_rope).

rope / rope_at tables follow src/wan_dit_lab/models/rope.py:4-10 and positions.py:7-11 (float64, then cast);
norm_rope(q, k, ...) is RMSNorm over all heads (models/rms_norm.py:10-13) followed by rope_apply
(models/rope.py:12-31) for Q and K of one chunk, as FusedQKVAttention.forward does (quantization/w4a4.py:255-257).
"""

from __future__ import annotations

import torch

from wdl.ops import qk_norm_rope_launch


def rope(pos_count: int, pos_dim: int) -> torch.Tensor:
    pairs = pos_dim // 2
    angles = torch.arange(pos_count)[:, None] * (10000 ** (-2 * torch.arange(pairs, dtype=torch.float64) / pos_dim))
    return torch.stack((torch.cos(angles), torch.sin(angles)))


def rope_at(count: int, dim: int, scale: float) -> torch.Tensor:
    """rope at positions i * scale (positions.py:7-11)."""
    positions = torch.arange(count, dtype=torch.float64)[:, None] * scale
    angles = positions * 10000 ** (-2 * torch.arange(dim // 2, dtype=torch.float64) / dim)
    return torch.stack((torch.cos(angles), torch.sin(angles)))


def freqs(dim: int = 128, positions: int = 1024, device=None) -> torch.Tensor:
    """fp32 [2, positions, dim/2]: time, height, width tables side by side (split [22, 21, 21] for dim 128)."""
    c = dim // 2
    t, s = c - 2 * (c // 3), c // 3
    f = torch.cat([rope(positions, 2 * t), rope(positions, 2 * s), rope(positions, 2 * s)], dim=-1)
    return f.to(torch.float32).contiguous().to(device)


def _check_table(freq, grid, rows, start_frame):
    if freq.dtype not in (torch.float32, torch.float64) or not freq.is_contiguous() or freq.ndim != 3 \
            or freq.shape[0] != 2 or freq.shape[2] != 64:
        raise TypeError("freq must be a contiguous fp32 or fp64 [2, positions, 64] table")
    f, h, w = grid
    if f * h * w > rows or start_frame < 0 or start_frame + f > freq.shape[1] or max(h, w) > freq.shape[1]:
        raise ValueError("grid exceeds the rows or the frequency table")


def norm_rope(q, k, wq, wk, freq, grid, start_frame=0, eps=1e-6):
    """q, k bf16 [M, H*128] (row-strided views of the QKV output allowed) -> (Q, K) bf16 [M, H*128]:
    bf16(bf16(x * rstd) * w) then the 3D rotation of the first f*h*w rows."""
    _check_table(freq, grid, q.shape[0], start_frame)
    return qk_norm_rope_launch(q, k, wq, wk, freq, grid, start_frame, eps)


def rope_apply(X, grid_sizes, freq, start_frame=0):
    """rope.py:12-31 / wan_dit_lab::rope3d_rotate (rope_triton.py:66-81) on MI355X: X bf16 [B, L, H, 128] (one
    grid for the batch, grid_sizes[0] = (f, h, w)) -> a new bf16 tensor, tokens of the grid rotated in the table's
    precision, tokens past f h w copied. The table: fp32 or fp64 [2, positions, 64] (rope()'s layout)."""
    if X.dtype != torch.bfloat16 or X.dim() != 4 or X.shape[-1] != 128:
        raise TypeError("X must be bf16 [B, L, H, 128]")
    g = grid_sizes[0].tolist() if isinstance(grid_sizes, torch.Tensor) else grid_sizes[0]
    f, h, w = (int(v) for v in g)
    B, L, H, D = X.shape
    _check_table(freq, (f, h, w), L, start_frame)
    out = torch.empty(B, L, H, D, device=X.device, dtype=torch.bfloat16)
    for b in range(B):
        xb = X[b].reshape(L, H * D)
        if xb.stride(1) != 1:
            xb = xb.contiguous()
        qk_norm_rope_launch(xb, None, None, None, freq, (f, h, w), start_frame, q_out=out[b].view(L, H * D))
    return out
