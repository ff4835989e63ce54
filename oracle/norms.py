"""LayerNorm + adaLN modulation and RMSNorm with a defined fp32 reduction order — CPU restatement of
src/wan_dit_lab/models/layer_norm.py:4-7, rms_norm.py:4-13 and the modulation of block.py:24-28.

The reference computes these in fp32 through torch (whose reduction order is its own); this oracle fixes one
order so the fused HIP kernels can be pinned bit-exactly to it:
- a row of K values is cut into chunks of 8 (chunk c = values 8c .. 8c+7); lane l of a 64-lane wave owns the
  chunks c = l, l + 64, l + 128, ... and adds their values into one fp32 running sum, chunk by chunk, value by
  value;
- the 64 lane sums are combined by the butterfly s[i] + s[i^32], then ^16, ^8, ^4, ^2, ^1 (fp32);
- mean = sum / K; var = sum((x - mean)^2) / K by the same order; rstd = 1 / sqrt(var + eps) (IEEE sqrt, IEEE div);
- LayerNorm: (x - mean) * rstd [* w + b]; modulation: n * (1 + scale) + shift in fp32; one bf16 rounding at the end
  (the bf16 activation the reference feeds its W4A4 linear, w4a4.py:230).
- RMSNorm: x * rstd with rstd from mean(x^2), the result rounded to the input type, then times the weight
  (rms_norm.py:12-13).

Pinned by the closed form: in float64 the same functions agree with torch.nn.functional.layer_norm / the RMSNorm
formula to fp32 rounding (tests/test_oracle_w4a4.py), and the reduction order is checked against an independent
scalar loop.
"""

from __future__ import annotations

import numpy as np
import torch

LANES = 64
VEC = 8


def _ordered_sum(x: np.ndarray) -> np.ndarray:
    """x float32 [M, K] (K a multiple of 8) -> float32 [M] in the order described above (a lane owning no chunk,
    or a chunk past the row, adds +0, which leaves a running sum started at +0 unchanged)."""
    M, K = x.shape
    pad = (-K) % (LANES * VEC)
    if pad:
        x = np.concatenate([x, np.zeros((M, pad), dtype=np.float32)], axis=1)
        K += pad
    x = x.reshape(M, K // (LANES * VEC), LANES, VEC)
    s = np.zeros((M, LANES), dtype=np.float32)
    for i in range(x.shape[1]):
        for j in range(VEC):
            s = (s + x[:, i, :, j]).astype(np.float32)
    for o in (32, 16, 8, 4, 2, 1):
        s = (s + s[:, np.arange(LANES) ^ o]).astype(np.float32)
    return s[:, 0]


def row_stats(x: torch.Tensor, eps: float, centered: bool = True):
    """mean (0 for RMS) and rstd per row, float32 numpy."""
    a = x.float().numpy().astype(np.float32)
    K = a.shape[1]
    Kf = np.float32(K)
    if centered:
        mean = (_ordered_sum(a) / Kf).astype(np.float32)
        d = (a - mean[:, None]).astype(np.float32)
    else:
        mean = np.zeros(a.shape[0], dtype=np.float32)
        d = a
    var = (_ordered_sum((d * d).astype(np.float32)) / Kf).astype(np.float32)
    rstd = (np.float32(1.0) / np.sqrt((var + np.float32(eps)).astype(np.float32))).astype(np.float32)
    return mean, rstd


def ln_mod(x: torch.Tensor, shift: torch.Tensor | None, scale: torch.Tensor | None, weight=None, bias=None,
           eps: float = 1e-6) -> torch.Tensor:
    """bf16(LayerNorm(x)[*w+b] * (1 + scale) + shift) in fp32 arithmetic; x [M, K]; shift/scale [K] (any float
    dtype, used in fp32); weight/bias [K] or None."""
    mean, rstd = row_stats(x, eps, centered=True)
    a = x.float().numpy().astype(np.float32)
    n = ((a - mean[:, None]).astype(np.float32) * rstd[:, None]).astype(np.float32)
    if weight is not None:
        n = (n * weight.float().numpy()[None, :]).astype(np.float32)
    if bias is not None:
        n = (n + bias.float().numpy()[None, :]).astype(np.float32)
    if scale is not None:
        one_plus = (np.float32(1.0) + scale.float().numpy()).astype(np.float32)
        n = (n * one_plus[None, :]).astype(np.float32)
    if shift is not None:
        n = (n + shift.float().numpy()[None, :]).astype(np.float32)
    return torch.from_numpy(n).to(torch.bfloat16)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """rms_norm.py:12-13: (x32 * rstd).type_as(x) * weight -> bf16 for bf16 x and weight."""
    _, rstd = row_stats(x, eps, centered=False)
    a = x.float().numpy().astype(np.float32)
    n = torch.from_numpy((a * rstd[:, None]).astype(np.float32)).to(x.dtype)
    return (n.float() * weight.float()).to(x.dtype) if x.dtype != torch.float32 else n * weight.float()
