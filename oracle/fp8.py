"""FP8 E4M3FN quantization, CPU restatement of src/wan_dit_lab/quantization/fp8.py.

- quantize (fp8.py:14-17): per-tensor, scale = clamp(max|X|, 1e-12) / 448, X_fp8 = e4m3(X / scale).
- quantize_rows (fp8.py:37-41): the same per last-dim row; the KV cache's rule (generation/causal.py:177-184).
- w8a8_linear_rows (fp8.py:58-62): unit-scale fp8 product, then y * (xs ⊗ ws) + b.
- w8a8_linear_tensor (fp8.py:32-33 / 60): per-tensor scales.
- w8a16_linear: the weight-only FP8 linear of the mixed-precision mode (no counterpart in the reference, whose FP8
  linears are W8A8): the weight quantized by quantize_rows (or quantize), the activation kept in bf16,
  y = bf16(scale * (x . w_fp8) + b) with the product in float64.

The e4m3 rounding is torch's CPU conversion (the reference's own rule). Pinned by:
- the reference's known answers (tests/test_cache_fp8.py:47-58, 150-158: 84.021 -> 88, never 80 through fp16;
  the 1.06251 / 1.06249 midpoints; the boundary row [0, -0, 1e-15, ..., 448, -448]);
- e4m3_nearest, an independent brute-force search over all 254 finite codes (nearest value, ties to the even
  code), checked against torch on random and on every midpoint between consecutive codes.
"""

from __future__ import annotations

import numpy as np
import torch

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0


def e4m3_bits(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> e4m3fn codes (uint8) by torch's CPU conversion."""
    return x.float().cpu().to(FP8).view(torch.uint8)


def e4m3_values() -> np.ndarray:
    """The fp32 value of each of the 256 codes (NaN for 0x7f and 0xff)."""
    codes = torch.arange(256, dtype=torch.uint8)
    return codes.view(FP8).float().numpy()


def e4m3_nearest(x: np.ndarray) -> np.ndarray:
    """Brute force: the code of the finite e4m3 value nearest to each x (ties to the code with even mantissa);
    magnitudes past 448 + half a step (464) go to NaN as torch does. Independent of torch's conversion."""
    x = np.asarray(x, dtype=np.float64).ravel()
    vals = e4m3_values().astype(np.float64)
    finite = np.where(np.isfinite(vals))[0]
    pos = [c for c in finite if c < 128]  # non-negative codes 0x00..0x7e
    pv = vals[pos]
    out = np.empty(x.shape, dtype=np.uint8)
    for i, v in enumerate(x):
        a = abs(v)
        sign = 0x80 if (v < 0 or (v == 0 and np.signbit(v))) else 0
        if np.isnan(v) or a > 464.0:  # past the midpoint of 448 and the missing 480: NaN
            out[i] = sign | 0x7F
            continue
        d = np.abs(pv - a)
        best = np.flatnonzero(d == d.min())
        if len(best) > 1:  # tie: the even mantissa (even code)
            best = [b for b in best if pos[b] % 2 == 0]
        out[i] = sign | pos[best[0]]
    return out


def quantize(X: torch.Tensor):
    """fp8.py:14-17 — X in FP8 and the scale it was divided by (per tensor)."""
    scale = X.abs().amax().float().clamp(min=1e-12) / FP8_MAX
    return (X / scale).to(FP8), scale


def quantize_rows(X: torch.Tensor):
    """fp8.py:37-41 — X [..., d] in FP8 with one fp32 scale per row."""
    scale = X.abs().amax(dim=-1, keepdim=True).float().clamp(min=1e-12) / FP8_MAX
    return (X / scale).to(FP8), scale


def w8a8_linear_rows(x: torch.Tensor, W: torch.Tensor, b: torch.Tensor | None):
    """fp8.py:57-62 (rows=True): per-token x scale, per-output-row W scale, the unit-scale fp8 product rounded to
    bf16 (_scaled_mm's out_dtype; exact products of fp8 values, fp64 sum here), then y * (xs ⊗ ws) in fp32, + b,
    output bf16."""
    (xq, xs), (wq, ws) = quantize_rows(x), quantize_rows(W)
    y = (xq.double() @ wq.double().t()).to(torch.bfloat16).float()
    y = y * (xs * ws.t())
    if b is not None:
        y = y + b.float()
    return y.to(torch.bfloat16), (xq, xs, wq, ws)


def w8a8_linear_tensor(x: torch.Tensor, W: torch.Tensor, b: torch.Tensor | None):
    """fp8.py:63-66 (rows=False) / Fp8Linear fp8.py:27-31: per-tensor scales; _scaled_mm's acc * (xs ws) + b in
    fp32, one bf16 rounding."""
    (xq, xs), (wq, ws) = quantize(x), quantize(W)
    y = (xq.double() @ wq.double().t()).float() * (xs * ws)
    if b is not None:
        y = y + b.float()
    return y.to(torch.bfloat16)


def w8a16_linear(x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, b: torch.Tensor | None):
    """The weight-only FP8 linear: x bf16 [M, K], e4m3 weight [N, K] with fp32 scales [N, 1] or a 0-d / [1] one ->
    bf16 [M, N] = bf16(scale_n * sum_k x_mk w_nk + b_n): the sum in float64 (its products are exact), the scale and
    the bias in fp32 as the kernel applies them."""
    y = (x.double() @ wq.double().t()).float()
    y = y * ws.reshape(1, -1).float()
    if b is not None:
        y = y + b.float()
    return y.to(torch.bfloat16)
