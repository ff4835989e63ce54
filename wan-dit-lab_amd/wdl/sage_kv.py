"""Sage-2 style attention straight over the FP8 KV cache on MI355X — the API of src/wan_dit_lab/kernels/sage_kv.py.

Tokens [0, at) come from the FP8 cache (value * per-row scale), [at, at + n) from the chunk's own bf16 K, V; the
K mean, int8 K, fp8 V (wdl_sage_prep), int8 Q (wdl_quant_q) and the attention (wdl_sage_attn) are HIP kernels.
The head/token maps of the reference (Forcing-KV, sage_kv.py:127-134) select cache heads and rows in place.
"""

from __future__ import annotations

import torch

from wdl.ops import (quant_q_launch, sage_attn_launch, sage_kv_append_attend_cached, sage_kv_attend,
                     sage_kv_attend_cached, sage_prep_launch)

V_MAX = 2.25  # sage_kv.py:24
BLKQ, WARPQ, BLKK = 128, 32, 64

__all__ = ["V_MAX", "attend", "cache_stats", "quant_q", "prep"]


def _check(Q, cache_k, cache_ks, cache_v, cache_vs, at, K, V, heads=None, tokens=None):
    if Q.ndim != 4 or K.ndim != 4 or V.shape != K.shape or Q.shape[0] != 1 or Q.shape[-1] != 128:
        raise ValueError("Q, K, V must be [1, tokens, heads, 128]")
    if Q.shape[2] != K.shape[2] or (heads is None and cache_k.shape[2] != K.shape[2]):
        raise ValueError("head counts differ")
    for name, m, count, bound in (("heads", heads, K.shape[2], cache_k.shape[2]),
                                  ("tokens", tokens, at, cache_k.shape[1])):
        if m is None:
            continue
        if m.dtype != torch.int32 or m.ndim != 1 or m.shape[0] < count or m.device != cache_k.device:
            raise ValueError(f"{name} must be an int32 vector of at least {count} entries on the cache's device")
        if count and (int(m[:count].min()) < 0 or int(m[:count].max()) >= bound):
            raise ValueError(f"{name} maps outside the cache (0 .. {bound - 1})")
    if cache_k.dtype != torch.float8_e4m3fn or cache_v.dtype != torch.float8_e4m3fn:
        raise TypeError("cache values must be FP8 E4M3FN")
    if cache_ks.dtype != torch.float32 or cache_vs.dtype != torch.float32:
        raise TypeError("cache scales must be FP32")
    if Q.dtype != torch.bfloat16 or K.dtype != torch.bfloat16 or V.dtype != torch.bfloat16:
        raise TypeError("Q, K, V must be bf16")
    H = K.shape[2] if heads is None else cache_k.shape[2]
    if cache_k.ndim != 4 or cache_k.shape[0] != 1 or cache_k.shape[2:] != (H, 128) or cache_v.shape != cache_k.shape:
        raise ValueError("cache_k / cache_v must be [1, capacity, heads, 128] (batch 1)")
    if cache_ks.shape != (*cache_k.shape[:3], 1) or cache_vs.shape != cache_ks.shape:
        raise ValueError("cache_ks / cache_vs must be [1, capacity, heads, 1]: one scale per cache row")
    if any(not t.is_contiguous() for t in (cache_k, cache_ks, cache_v, cache_vs)):
        raise ValueError("cache buffers must be contiguous (the kernels index rows as (token * heads + head))")
    if not isinstance(at, int) or at < 0 or at > cache_k.shape[1]:
        raise ValueError("at outside the cache")
    if any(t.stride(-1) != 1 or t.stride(-2) != 128 for t in (Q, K, V)):
        raise ValueError("heads must be contiguous [.., heads, 128] rows")


def attend(Q, cache_k, cache_ks, cache_v, cache_vs, at, K, V, sm_scale=None, heads=None, tokens=None,
           frame_tokens=0, cache_stats=None, append=False):
    """softmax(Q K^T * sm_scale) V over the cached tokens and the chunk (sage_kv.py:127-134); [1, nq, H, 128] bf16
    (sm_scale defaults to 128^-0.5). heads (int32 [H]): head h of Q, K, V is cache head heads[h], the cache keeping
    all of them; tokens (int32 [at]): cached token i is cache row tokens[i] (KVCache.attend_split's static heads,
    causal.py:222-241). Neither copies the cache. The maps' ranges are checked on the host (one synchronisation).
    frame_tokens > 0 (not a mode of the reference, whose chunk attention sees the whole chunk): block-causal per
    latent frame of that many tokens, Q being the chunk (nq == n): chunk query q sees the cache and the chunk's
    frames up to its own, keys below at + (q // frame_tokens + 1) * frame_tokens. cache_stats (fp32 [2, H, 128],
    wdl.ops.sage_cache_stats_launch of rows [0, at), no maps): the K mean and V scale then read only the chunk's
    tokens beside them. append (with cache_stats, not with frame_tokens): K, V also go into cache rows at .. at + n
    (KVCache.store's store_kv_fp8, causal.py:177-181) inside the preparation pass; its requirements are checked
    first, and a broken one raises before anything is written."""
    _check(Q, cache_k, cache_ks, cache_v, cache_vs, at, K, V, heads, tokens)
    if append:
        from wdl.cache_fp8 import _refusal

        if cache_stats is None or frame_tokens:
            raise ValueError("append runs with the cache statistics and without frame_tokens")
        refused = _refusal(K, V, cache_k, cache_ks, cache_v, cache_vs, at)
        if refused is not None:
            kind, message = refused
            raise kind(message)
    if cache_stats is not None and (heads is not None or tokens is not None):
        raise ValueError("cache statistics are for the unmapped cache")
    if frame_tokens:
        if not isinstance(frame_tokens, int) or frame_tokens < 0 or Q.shape[1] != K.shape[1]:
            raise ValueError("frame_tokens: a positive int, with the chunk's own queries (nq == n)")
        from wdl import ops

        n, H = K.shape[1], K.shape[2]
        prep = ops.sage_prep_launch(cache_k.view(torch.uint8), cache_ks, cache_v.view(torch.uint8), cache_vs,
                                    K[0].flatten(1), V[0].flatten(1), at, heads=heads, tokens=tokens,
                                    cache_stats=cache_stats)
        sm = Q.shape[-1] ** -0.5 if sm_scale is None else float(sm_scale)
        return ops.sage_attn_q16_launch(Q[0].flatten(1), prep, at + n, sm, frame_tokens=frame_tokens).view(Q.shape)
    sm = Q.shape[-1] ** -0.5 if sm_scale is None else float(sm_scale)
    if cache_stats is not None:
        op = sage_kv_append_attend_cached if append else sage_kv_attend_cached
        return op(Q, cache_k.view(torch.uint8), cache_ks, cache_v.view(torch.uint8), cache_vs, K, V, at, sm,
                  cache_stats)
    return sage_kv_attend(Q, cache_k.view(torch.uint8), cache_ks, cache_v.view(torch.uint8), cache_vs, K, V, at, sm,
                          heads, tokens)


def quant_q(Q):
    """Sage's per-thread int8 Q (sage_kv.py:112-124): Q [1, n, H, 128] -> (q int8 [1, n, H, 128],
    q_scale fp32 [1, H, blocks * 8])."""
    q, qs = quant_q_launch(Q[0].flatten(1), Q.shape[2])
    return q[None], qs[None]


def prep(cache_k, cache_ks, cache_v, cache_vs, at, K, V, cache_stats=None):
    """The quantized K/V operands of one call in wdl's layouts (see wdl_sage_prep in include/wdl.h); cache_stats as
    in attend."""
    return sage_prep_launch(cache_k.view(torch.uint8), cache_ks, cache_v.view(torch.uint8), cache_vs,
                            K[0].flatten(1), V[0].flatten(1), at, want_stats=True, cache_stats=cache_stats)


def cache_stats(cache_k, cache_ks, cache_v, cache_vs, at):
    """fp32 [2, H, 128]: the K column sums and |V| column maxima of cache rows [0, at) (wdl_sage_cache_stats)."""
    from wdl.ops import sage_cache_stats_launch

    return sage_cache_stats_launch(cache_k.view(torch.uint8), cache_ks, cache_v.view(torch.uint8), cache_vs, at)
