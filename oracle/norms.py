"""LayerNorm + adaLN modulation and RMSNorm with a defined fp32 reduction order — CPU restatement of
src/wan_dit_lab/models/layer_norm.py:4-7, rms_norm.py:4-13 and the modulation of block.py:24-28.

The reference computes these in fp32 through torch (whose reduction order is its own); this oracle fixes one
order so the fused HIP kernels can be pinned bit-exactly to it.

LayerNorm statistics come from per-chunk partials, so that any kernel holding a 32-value chunk of a row (the
residual GEMM epilogues that write the row, or a statistics kernel) can produce them:
- chunk c of a row = values 32c .. 32c+31, cut into 8 quads (quad k = values 4k .. 4k+3 of the chunk);
  t_k = ((x0 + x1) + x2) + x3; the chunk sum S_c = ((t0 + t1) + (t2 + t3)) + ((t4 + t5) + (t6 + t7)); its mean
  m_c = S_c / 32 (exact); M2_c = the same quad and tree sums of (x - m_c)^2 (each difference and square one fp32
  rounding);
- the C = K / 32 chunks are merged by 8 slots: slot j takes the chunk pairs p = j, j + 8, j + 16, ... (pair p =
  chunks 2p and 2p + 1, those below C; a lane loads a pair with one 16-byte load) and adds them into a running sum
  started at +0, in increasing chunk order; the 8 slot sums are combined as
  ((L0 + L1) + (L2 + L3)) + ((L4 + L5) + (L6 + L7)) (a butterfly over 8 lanes gives every lane this value);
- mean = sum over the chunks of S_c / K; M2 = the same merge of T_c = M2_c + 32 (m_c - mean)^2 (difference,
  square, the exact product by 32, then the sum, each one fp32 rounding); var = M2 / K; rstd = 1 / sqrt(var + eps)
  (IEEE sqrt, IEEE div) — the two-pass identity M2 = sum_c M2_c + sum_c 32 (m_c - mean)^2;
- LayerNorm: (x - mean) * rstd [* w + b]; modulation: n * (1 + scale) + shift in fp32; one bf16 rounding at the end
  (the bf16 activation the reference feeds its W4A4 linear, w4a4.py:230).

RMSNorm (rms_norm.py:12-13; the Q/K norms) keeps a wave's order: a row of K values is cut into chunks of 8 (chunk
c = values 8c .. 8c+7); lane l of a 64-lane wave owns the chunks c = l, l + 64, l + 128, ... and adds their values
into one fp32 running sum, chunk by chunk, value by value; the 64 lane sums are combined by the butterfly
s[i] + s[i^32], then ^16, ^8, ^4, ^2, ^1 (fp32); rstd from mean(x^2) as above; x * rstd rounded to the input type,
then times the weight.

Pinned by the closed form: in float64 the same functions agree with torch.nn.functional.layer_norm / the RMSNorm
formula to fp32 rounding (tests/test_oracle_w4a4.py), and both reduction orders are checked against independent
scalar loops.
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


CHUNK = 32  # values per LayerNorm partial
SLOTS = 8   # merge slots of a row's chunks


def _tree8(t: np.ndarray) -> np.ndarray:
    """((t0 + t1) + (t2 + t3)) + ((t4 + t5) + (t6 + t7)) over the last axis (length 8), fp32."""
    f = np.float32
    a = (t[..., 0] + t[..., 1]).astype(f)
    b = (t[..., 2] + t[..., 3]).astype(f)
    c = (t[..., 4] + t[..., 5]).astype(f)
    d = (t[..., 6] + t[..., 7]).astype(f)
    return ((a + b).astype(f) + (c + d).astype(f)).astype(f)


def _chunk_sum(v: np.ndarray) -> np.ndarray:
    """v float32 [..., 32] -> float32 [...]: the quads' sequential sums, then the tree of the 8 quads."""
    q = v.reshape(v.shape[:-1] + (8, 4))
    t = (((q[..., 0] + q[..., 1]).astype(np.float32) + q[..., 2]).astype(np.float32) + q[..., 3]).astype(np.float32)
    return _tree8(t)


def ln_chunk_partials(x) -> tuple[np.ndarray, np.ndarray]:
    """x bf16 / float [M, K] (K a multiple of 32) -> (S, M2) float32 [M, K / 32]: each 32-value chunk's sum and
    sum of squared deviations from its own mean, in the order of the module docstring."""
    a = (x.float().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)).astype(np.float32)
    M, K = a.shape
    v = a.reshape(M, K // CHUNK, CHUNK)
    S = _chunk_sum(v)
    mc = (S * np.float32(1.0 / CHUNK)).astype(np.float32)
    d = (v - mc[..., None]).astype(np.float32)
    M2 = _chunk_sum((d * d).astype(np.float32))
    return S, M2


def _slot_merge(v: np.ndarray) -> np.ndarray:
    """v float32 [M, C] -> float32 [M]: 8 slots, slot j the chunk pairs j, j + 8, j + 16, ... (pair p = chunks 2p
    and 2p + 1 below C) in increasing chunk order as a running sum from +0, then the tree."""
    M, C = v.shape
    slots = []
    for j in range(SLOTS):
        acc = np.zeros(M, dtype=np.float32)
        for p in range(j, (C + 1) // 2, SLOTS):
            for c in (2 * p, 2 * p + 1):
                if c < C:
                    acc = (acc + v[:, c]).astype(np.float32)
        slots.append(acc)
    return _tree8(np.stack(slots, axis=-1))


def ln_merge(S: np.ndarray, M2: np.ndarray, K: int, eps: float) -> tuple[np.ndarray, np.ndarray]:
    """Chunk partials [M, C] -> (mean, rstd) float32 [M] in the order of the module docstring."""
    f = np.float32
    mean = (_slot_merge(S) / f(K)).astype(f)
    d = ((S * f(1.0 / CHUNK)).astype(f) - mean[:, None]).astype(f)
    T = (M2 + (f(CHUNK) * (d * d).astype(f)).astype(f)).astype(f)
    var = (_slot_merge(T) / f(K)).astype(f)
    rstd = (f(1.0) / np.sqrt((var + f(eps)).astype(f))).astype(f)
    return mean, rstd


def ln_stats(x, eps: float) -> tuple[np.ndarray, np.ndarray]:
    """LayerNorm (mean, rstd) per row through the chunk partials."""
    S, M2 = ln_chunk_partials(x)
    return ln_merge(S, M2, S.shape[1] * CHUNK, eps)


def ln_mod(x: torch.Tensor, shift: torch.Tensor | None, scale: torch.Tensor | None, weight=None, bias=None,
           eps: float = 1e-6) -> torch.Tensor:
    """bf16(LayerNorm(x)[*w+b] * (1 + scale) + shift) in fp32 arithmetic; x [M, K]; shift/scale [K] (any float
    dtype, used in fp32); weight/bias [K] or None."""
    mean, rstd = ln_stats(x, eps)
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
