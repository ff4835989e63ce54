"""FP8 E4M3 row quantization of K and V straight into the persistent KV cache, one HIP launch
(wdl_kv_append_fp8), drop-in for store_kv_fp8 of src/wan_dit_lab/kernels/cache_fp8.py:75-105.

Per (token, head) row: scale = max(max|x|, 1e-12) / 448, cache = e4m3(x / scale), rounded to nearest even directly
from fp32 (no fp16 step), bit-exact to quantize_rows (src/wan_dit_lab/quantization/fp8.py:37-41). Inputs may be
strided and of fp32/fp16/bf16 (K and V may differ); cache buffers are contiguous and caller-owned.
"""

from __future__ import annotations

import torch

from wdl.ops import store_kv_fp8_op

FLOATS = (torch.float16, torch.bfloat16, torch.float32)


def store_kv_fp8(k, v, cache_k, cache_ks, cache_v, cache_vs, at):
    """Store [B,N,H,D] in cache[:, at:at+N]; every contract violation raises before any write
    (the checks of src/wan_dit_lab/kernels/cache_fp8.py:82-104)."""
    tensors = (k, v, cache_k, cache_ks, cache_v, cache_vs)
    if k.ndim != 4 or v.shape != k.shape or k.shape[-1] < 1:
        raise ValueError("K and V must have matching [B,N,H,D] shapes")
    if k.device.type != "cuda" or any(t.device != k.device for t in tensors):
        raise ValueError("All buffers must be on the same GPU device")
    if any(t.requires_grad for t in tensors):
        raise ValueError("Cache store is inference-only")
    if k.dtype not in FLOATS or v.dtype not in FLOATS:
        raise TypeError("K and V must be FP16, BF16 or FP32")
    if cache_k.dtype != torch.float8_e4m3fn or cache_v.dtype != cache_k.dtype:
        raise TypeError("Cache values must be FP8 E4M3FN")
    if cache_ks.dtype != torch.float32 or cache_vs.dtype != torch.float32:
        raise TypeError("Cache scales must be FP32")
    b, n, h, d = k.shape
    if cache_k.ndim != 4 or cache_k.shape != cache_v.shape or (cache_k.shape[0], *cache_k.shape[2:]) != (b, h, d):
        raise ValueError("Cache dimensions must match inputs")
    if cache_ks.shape != (*cache_k.shape[:3], 1) or cache_vs.shape != cache_ks.shape:
        raise ValueError("One scale is required per cache row")
    if any(not t.is_contiguous() for t in tensors[2:]):
        raise ValueError("Cache buffers must be contiguous")
    if not isinstance(at, int) or at < 0 or at + n > cache_k.shape[1]:
        raise ValueError("Write exceeds cache bounds")
    if d > 1024:
        raise ValueError("head_dim above 1024 is not supported")
    store_kv_fp8_op(k, v, cache_k, cache_ks, cache_v, cache_vs, at)


def install_cache_store(cls=None):
    """KVCache.store through store_kv_fp8 for FP8 caches; returns the original method
    (src/wan_dit_lab/kernels/cache_fp8.py:108-121). cls: the cache class to patch (the reference's
    generation.causal.KVCache, or by default wdl.kvcache.KVCache); it must keep fp8, k, ks, v, vs as the
    reference's does (causal.py:159-163)."""
    if cls is None:
        from wdl.kvcache import KVCache as cls

    KVCache = cls
    original = KVCache.store

    def store(cache, at, k, v):
        if cache.fp8:
            store_kv_fp8(k, v, cache.k, cache.ks, cache.v, cache.vs, at)
        else:
            original(cache, at, k, v)

    KVCache.store = store
    return original
