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


def norm_rope(q, k, wq, wk, freq, grid, start_frame=0, eps=1e-6):
    """q, k bf16 [M, H*128] (row-strided views of the QKV output allowed) -> (Q, K) bf16 [M, H*128]:
    bf16(bf16(x * rstd) * w) then the 3D rotation of the first f*h*w rows."""
    if freq.dtype != torch.float32 or not freq.is_contiguous() or freq.ndim != 3 or freq.shape[0] != 2:
        raise TypeError("freq must be a contiguous fp32 [2, positions, 64] table")
    f, h, w = grid
    if f * h * w > q.shape[0] or start_frame < 0 or start_frame + f > freq.shape[1]:
        raise ValueError("grid exceeds the rows or the frequency table")
    return qk_norm_rope_launch(q, k, wq, wk, freq, grid, start_frame, eps)
