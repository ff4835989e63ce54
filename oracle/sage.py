"""Sage-2 style quantized attention over the FP8 KV cache, CPU restatement of src/wan_dit_lab/kernels/sage_kv.py.

Tokens [0, at) come from the FP8 cache (value * per-row scale, fp32), [at, at + n) from the chunk's own K/V
(bf16 -> fp32), tokens >= L = at + n are zero (sage_kv.py:28-40).

- colstats (sage_kv.py:43-56, 155-158, 165-168): k_mean = sum_t K / L, v_scale = max(max_t |V|, 1e-8) / 2.25.
  The reference sums with fp32 atomics in a nondeterministic order; this oracle sums in float64 and rounds once,
  and its tests allow the +-1 LSB of int8 K that the reference's own test allows (tests/test_sage_kv.py:81).
- quant_k (sage_kv.py:59-85): per 64-token block, group g = 0..3 owns tokens 8i + 2g and 8i + 2g + 1 (i = 0..7);
  scale = max|K - mean| / 127 + 1e-7; q = trunc(x / scale +- 0.5) (half away from zero); tokens >= L zero.
- quant_v (sage_kv.py:88-105): e4m3(V / v_scale[d]), rounded to nearest even straight from fp32 (the reference's
  Triton cast goes through fp16 first; its own test allows 0.1 % differing bytes against Sage, test_sage_kv.py:55).
  Values are returned token-major [B, L, H, D]; the layouts (the reference's 16-token permutation and wdl's
  64-token one) are separate index maps (sage_v_layout, wdl_v_layout).
- quant_q (sage_kv.py:112-124): per 32-token block, lane l = 0..7 owns tokens l, l+8, l+16, l+24 with one scale
  max|Q| / 127 + 1e-7; q = trunc(Q / scale +- 0.5).
- attention: O = softmax(sm_scale * q_scale * k_scale * (q_i8 . k_i8)) (v_fp8 * v_scale), exact softmax in float64
  on the quantized operands. The sm89 kernel's own P rounding and fp16 accumulation (sage_ops.cpp:16-17) are in
  absent code: parity unpinned at that step. The bars are cosine >= 0.999 against the exact-P emulation, and a
  relative error against exact attention within 1.2x + 1e-3 of an fp8-P emulation (P * 448 rounded to e4m3, the
  denominator the unrounded sum) — the reference's own bar, stated against sageattn, which also rounds P to fp8
  (tests/test_sage_kv.py:85-97). Any e4m3 rounding of P costs about 0.037 relative error at these shapes.

Pinned by: the identity softmax(q (k - mu)^T) = softmax(q k^T) (mean smoothing changes nothing exactly), exact
SDPA on the dequantized operands, and brute-force rounding checks of the three quantizers.
"""

from __future__ import annotations

import math

import torch

V_MAX = 2.25  # sage_kv.py:24
BLKQ, WARPQ, BLKK = 128, 32, 64  # sage_kv.py:25


def gather(cache: torch.Tensor, scale: torch.Tensor, chunk: torch.Tensor, at: int, heads=None,
           tokens=None) -> torch.Tensor:
    """fp32 [B, at + n, H, D]: the cached tokens times their scales, then the chunk (sage_kv.py:28-40). With the maps
    of sage_kv.attend (sage_kv.py:127-134): head h is cache head heads[h] (the cache keeps all of them), cached token
    i is buffer token tokens[i]; without them, cache tokens 0 .. at - 1 and heads 0 .. H - 1."""
    rows = torch.arange(at) if tokens is None else tokens[:at].long()
    cols = torch.arange(chunk.shape[2]) if heads is None else heads.long()
    c = cache[:, rows][:, :, cols].float() * scale[:, rows][:, :, cols].float()
    return torch.cat([c, chunk.float()], dim=1)


def colstats(K: torch.Tensor, V: torch.Tensor):
    """K, V fp32 [B, L, H, D] -> k_mean fp32 [B, H, D], v_scale fp32 [B, H, D]."""
    L = K.shape[1]
    k_mean = (K.double().sum(dim=1) / L).float()
    v_max = V.abs().amax(dim=1)
    v_scale = v_max.clamp(min=1e-8) / V_MAX
    return k_mean, v_scale


def _round_away(y: torch.Tensor) -> torch.Tensor:
    return (y + torch.where(y >= 0, torch.tensor(0.5), torch.tensor(-0.5))).trunc()


def quant_k(K: torch.Tensor, k_mean: torch.Tensor):
    """K fp32 [B, L, H, D], k_mean [B, H, D] -> k_int8 [B, L, H, D], k_scale fp32 [B, H, blocks * 4]."""
    B, L, H, D = K.shape
    blocks = -(-L // BLKK)
    Lp = blocks * BLKK
    x = torch.zeros(B, Lp, H, D)
    x[:, :L] = K - k_mean[:, None]
    # token = blk*64 + 8i + 2g + p  ->  [B, blk, i, g, p, H, D]
    xv = x.view(B, blocks, 8, 4, 2, H, D)
    scale = xv.abs().amax(dim=(2, 4, 6)) / 127.0 + 1e-7  # [B, blk, g, H]
    s = scale[:, :, None, :, None, :, None]
    q = _round_away(xv / s).to(torch.int8).view(B, Lp, H, D)[:, :L]
    return q.contiguous(), scale.permute(0, 3, 1, 2).reshape(B, H, blocks * 4).contiguous()


def quant_v(V: torch.Tensor, v_scale: torch.Tensor) -> torch.Tensor:
    """V fp32 [B, L, H, D] -> e4m3 [B, L, H, D] of V / v_scale (token-major; see the layout maps)."""
    return (V / v_scale[:, None]).to(torch.float8_e4m3fn)


def quant_q(Q: torch.Tensor):
    """Q [B, n, H, D] -> q int8 [B, n, H, D], q_scale fp32 [B, H, blocks * 8] (sage_kv.py:112-124)."""
    B, n, H, D = Q.shape
    blocks = -(-n // BLKQ) * (BLKQ // WARPQ)
    x = torch.nn.functional.pad(Q.float(), (0, 0, 0, 0, 0, blocks * WARPQ - n)).view(B, blocks, 4, 8, H, D)
    scale = x.abs().amax(dim=(2, 5), keepdim=True) / 127.0 + 1e-7
    q = _round_away(x / scale).to(torch.int8).view(B, blocks * WARPQ, H, D)[:, :n]
    return q.contiguous(), scale.view(B, blocks, 8, H).permute(0, 3, 1, 2).reshape(B, H, blocks * 8).contiguous()


def expand_q_scale(q_scale: torch.Tensor, n: int) -> torch.Tensor:
    """[B, H, blocks*8] -> per token [B, n, H]: token t has scale index (t // 32) * 8 + t % 8."""
    t = torch.arange(n)
    return q_scale[:, :, (t // 32) * 8 + t % 8].permute(0, 2, 1)


def expand_k_scale(k_scale: torch.Tensor, L: int) -> torch.Tensor:
    """[B, H, blocks*4] -> per token [B, L, H]: token t has index (t // 64) * 4 + (t % 8) // 2."""
    t = torch.arange(L)
    return k_scale[:, :, (t // 64) * 4 + (t % 8) // 2].permute(0, 2, 1)


def sage_v_layout(v_fp8: torch.Tensor) -> torch.Tensor:
    """[B, L, H, D] -> the reference's [B, D, H, Lpad] with the 16-token order
    [0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15] (sage_kv.py:92-105), zero padded."""
    B, L, H, D = v_fp8.shape
    Lp = -(-L // BLKK) * BLKK
    raw = torch.zeros(B, D, H, Lp, dtype=torch.uint8)
    i = torch.arange(L)
    j = i % 16
    pair = j // 2
    to = i - j + (pair % 4) * 4 + (pair // 4) * 2 + j % 2
    raw[:, :, :, to] = v_fp8.view(torch.uint8).permute(0, 3, 2, 1)
    return raw.view(torch.float8_e4m3fn)


def wdl_v_position(t: torch.Tensor) -> torch.Tensor:
    """wdl's V order within a 64-token block: position p holds token perm[p], where the first 32 positions
    are tokens 8a + r (a = 0..7, r = 0..3) and the last 32 are 8a + 4 + r — the token order of one lane half of the
    transposed QK^T MFMA tile, so P feeds the PV MFMA without a shuffle. Returns the position of token t."""
    r = t % 64
    half = (r % 8) // 4
    return t - r + half * 32 + (r // 8) * 4 + r % 4


def wdl_v_layout(v_fp8: torch.Tensor) -> torch.Tensor:
    """[B, L, H, D] -> [B, H, D, Lpad] (token positions by wdl_v_position), zero padded."""
    B, L, H, D = v_fp8.shape
    Lp = -(-L // BLKK) * BLKK
    raw = torch.zeros(B, H, D, Lp, dtype=torch.uint8)
    raw[:, :, :, wdl_v_position(torch.arange(L))] = v_fp8.view(torch.uint8).permute(0, 2, 3, 1)
    return raw.view(torch.float8_e4m3fn)


def prep(Q, cache_k, cache_ks, cache_v, cache_vs, at, K, V, heads=None, tokens=None):
    """All quantized operands of one attend call."""
    Kf = gather(cache_k, cache_ks, K, at, heads, tokens)
    Vf = gather(cache_v, cache_vs, V, at, heads, tokens)
    k_mean, v_scale = colstats(Kf, Vf)
    k_i8, k_scale = quant_k(Kf, k_mean)
    v_fp8 = quant_v(Vf, v_scale)
    q_i8, q_scale = quant_q(Q)
    return dict(q=q_i8, q_scale=q_scale, k=k_i8, k_scale=k_scale, v=v_fp8, v_scale=v_scale, k_mean=k_mean,
                K=Kf, V=Vf)


def frame_mask(n: int, L: int, frame: int) -> torch.Tensor:
    """bool [n, L]: the keys each of the n chunk queries sees under the block-causal mask per latent frame of
    `frame` tokens, the chunk being the last n of the L keys: query q sees keys k < L - n + (q // frame + 1) frame
    (all of them for frame 0)."""
    q, k = torch.arange(n)[:, None], torch.arange(L)[None, :]
    if not frame:
        return torch.ones(n, L, dtype=torch.bool)
    return k < torch.clamp(L - n + (q // frame + 1) * frame, max=L)


def attention_quantized(p: dict, sm_scale: float, p_fp8: bool = False, frame: int = 0) -> torch.Tensor:
    """Softmax (float64) over the quantized operands -> fp32 [B, n, H, D]. p_fp8: P = exp(s - rowmax) rounded to
    e4m3 after scaling by 448 (the PV operand of an fp8 PV kernel), the denominator the unrounded row sum; this
    is the baseline the reference measures its kernel against (sageattn also rounds P to fp8). frame: the
    block-causal per-frame mask of frame_mask (keys a query does not see get no weight)."""
    q, k = p["q"].double(), p["k"].double()
    B, n, H, D = q.shape
    L = k.shape[1]
    qs = expand_q_scale(p["q_scale"], n).double()  # [B, n, H]
    ks = expand_k_scale(p["k_scale"], L).double()  # [B, L, H]
    S = torch.einsum("bnhd,blhd->bhnl", q, k) * qs.permute(0, 2, 1)[..., None] * ks.permute(0, 2, 1)[:, :, None]
    S = (S * sm_scale).masked_fill(~frame_mask(n, L, frame), float("-inf"))
    if p_fp8:
        E = torch.exp(S - S.amax(-1, keepdim=True))
        P = (E.float() * 448.0).to(torch.float8_e4m3fn).double() / 448.0 / E.sum(-1, keepdim=True)
    else:
        P = torch.softmax(S, dim=-1)
    Vd = p["v"].double() * p["v_scale"].double()[:, None]
    return torch.einsum("bhnl,blhd->bnhd", P, Vd).float()


def attention_exact(Q, Kf, Vf, sm_scale=None, frame: int = 0) -> torch.Tensor:
    """fp64 softmax(Q K^T * scale) V -> fp32 [B, n, H, D] (frame: the mask of frame_mask)."""
    D = Q.shape[-1]
    sm_scale = D ** -0.5 if sm_scale is None else sm_scale
    S = torch.einsum("bnhd,blhd->bhnl", Q.double(), Kf.double()) * sm_scale
    S = S.masked_fill(~frame_mask(Q.shape[1], Kf.shape[1], frame), float("-inf"))
    return torch.einsum("bhnl,blhd->bnhd", torch.softmax(S, -1), Vf.double()).float()


def cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    return float((a @ b) / (a.norm() * b.norm()))


def rel_err(x: torch.Tensor, ref: torch.Tensor) -> float:
    return float((x.double() - ref.double()).norm() / ref.double().norm())


def entropy_scale(keys: int, head_dim: int, ratio):
    """KVCache.scale (generation/causal.py:138-142)."""
    if ratio is None:
        return None
    return math.sqrt(math.log(keys) / math.log(keys * ratio) / head_dim)


def attention_online(p: dict, sm_scale: float, block: int = 64, round_p: bool = True, splits: int = 2,
                     tau: float = 2.0) -> torch.Tensor:
    """The blockwise online-softmax restatement of the HIP kernel's arithmetic (fp32). In log2 units
    y = int dot * k_scale * c with c = q_scale * sm_scale * log2(e). The key blocks (a partial final block
    included) are split in `splits` contiguous parts (for two: the first ceil(blocks / 2), then the rest), each run
    as an online softmax with a lazy reference max m: per 64-key block with max mb, where
    mb > m + tau the reference moves, m' = mb, and O, l are rescaled by 2^(m - m'); elsewhere m stays.
    P448 = 2^(y - m + log2 448 - tau) (<= 448) is rounded to e4m3; O = O + P448_fp8 . V_fp8 and l = l + sum P448_fp8
    (fp32). The parts merge as O = sum_i O_i 2^(m_i - m), l = sum_i l_i 2^(m_i - m) with m = max_i m_i, and
    out = O / l * v_scale. Its exp2 is torch's, not the hardware's: P can differ by an ulp before rounding.
    round_p=False keeps P in fp32 (in O and l): then the result is the exact softmax of attention_quantized up to
    fp32 rounding, whatever tau (the check that pins the online rescaling and the merge)."""
    q, k = p["q"].float(), p["k"].float()
    B, n, H, D = q.shape
    L = k.shape[1]
    c = (expand_q_scale(p["q_scale"], n).float() * (sm_scale * 1.4426950408889634)).permute(0, 2, 1)  # [B, H, n]
    ks = expand_k_scale(p["k_scale"], L).float().permute(0, 2, 1)  # [B, H, L]
    vq = p["v"].float()  # fp8 codes as values [B, L, H, D]
    log2_448 = math.log2(448.0)
    nblk = -(-L // block)
    bounds = [0, -(-nblk // 2), nblk] if splits == 2 else [0, nblk]
    parts = []
    for s0, s1 in zip(bounds[:-1], bounds[1:]):
        m = torch.full((B, H, n), float("-inf"))
        l = torch.zeros(B, H, n)
        O = torch.zeros(B, H, n, D)
        for bi in range(s0, s1):
            b0, b1 = bi * block, min(L, (bi + 1) * block)
            I = torch.einsum("bnhd,blhd->bhnl", q.double(), k[:, b0:b1].double()).float()
            y = I * ks[:, :, None, b0:b1] * c[..., None]
            mb = y.amax(-1)
            mn = torch.where(mb > m + tau, mb, m)
            alpha = torch.exp2(m - mn)
            O, l, m = O * alpha[..., None], l * alpha, mn
            P = torch.exp2(y - m[..., None] + (log2_448 - tau))
            Pq = P.to(torch.float8_e4m3fn).float() if round_p else P
            O = O + torch.einsum("bhnl,blhd->bhnd", Pq.double(), vq[:, b0:b1].double()).float()
            l = l + Pq.sum(-1)
        parts.append((O, m, l))
    mt = parts[0][1]
    for _, mi, _ in parts[1:]:
        mt = torch.maximum(mt, mi)
    O = sum(Oi * torch.exp2(mi - mt)[..., None] for Oi, mi, _ in parts)
    l = sum(li * torch.exp2(mi - mt) for _, mi, li in parts)
    out = O / l[..., None] * p["v_scale"].float()[:, :, None, :]
    return out.permute(0, 2, 1, 3)
