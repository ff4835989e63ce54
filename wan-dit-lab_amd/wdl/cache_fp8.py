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
MAX_HEAD_DIM = 1024  # the kernel holds a row in one lane group's registers


def _refusal(k, v, cache_k, cache_ks, cache_v, cache_vs, at):
    """The first broken requirement of a cache store as (exception type, message), or None. The requirements are
    the reference's store contract (cache_fp8.py:82-104): data types are TypeErrors; shapes, devices, gradients,
    layout and bounds are ValueErrors."""
    inputs, cache = (k, v), (cache_k, cache_ks, cache_v, cache_vs)
    if k.ndim != 4 or v.shape != k.shape or k.shape[-1] < 1:
        return ValueError, f"k and v need one [B, N, H, D] shape, got {tuple(k.shape)} and {tuple(v.shape)}"
    devices = {t.device for t in inputs + cache}
    if k.device.type != "cuda" or len(devices) != 1:
        return ValueError, f"k, v and the cache buffers must share one GPU, got {sorted(map(str, devices))}"
    if any(t.requires_grad for t in inputs + cache):
        return ValueError, "the cache store does not record gradients (inference only)"
    if any(t.dtype not in FLOATS for t in inputs):
        return TypeError, f"k and v must be fp16, bf16 or fp32, got {k.dtype} and {v.dtype}"
    if {cache_k.dtype, cache_v.dtype} != {torch.float8_e4m3fn}:
        return TypeError, f"cache values are float8_e4m3fn, got {cache_k.dtype} and {cache_v.dtype}"
    if {cache_ks.dtype, cache_vs.dtype} != {torch.float32}:
        return TypeError, f"cache scales are float32, got {cache_ks.dtype} and {cache_vs.dtype}"
    B, N, H, D = k.shape
    if cache_k.ndim != 4 or cache_v.shape != cache_k.shape or \
            (cache_k.shape[0], cache_k.shape[2], cache_k.shape[3]) != (B, H, D):
        return ValueError, f"cache values must be [{B}, rows, {H}, {D}], got {tuple(cache_k.shape)}"
    if cache_ks.shape != (*cache_k.shape[:3], 1) or cache_vs.shape != cache_ks.shape:
        return ValueError, f"cache scales must be {(*cache_k.shape[:3], 1)}, one per row"
    if not all(t.is_contiguous() for t in cache):
        return ValueError, "the cache buffers must be contiguous"
    if not isinstance(at, int) or at < 0 or at + N > cache_k.shape[1]:
        return ValueError, f"rows {at} .. {at} + {N} do not fit a cache of {cache_k.shape[1]} rows"
    if D > MAX_HEAD_DIM:
        return ValueError, f"head_dim {D} above {MAX_HEAD_DIM}"
    return None


def store_kv_fp8(k, v, cache_k, cache_ks, cache_v, cache_vs, at):
    """Quantize k, v [B, N, H, D] into cache rows at .. at + N; a broken requirement (_refusal) raises before
    anything is written."""
    refused = _refusal(k, v, cache_k, cache_ks, cache_v, cache_vs, at)
    if refused is not None:
        kind, message = refused
        raise kind(message)
    store_kv_fp8_op(k, v, cache_k, cache_ks, cache_v, cache_vs, at)


def install_cache_store(cls=None):
    """KVCache.store through store_kv_fp8 for FP8 caches; returns the original method
    (src/wan_dit_lab/kernels/cache_fp8.py:108-121). cls: the cache class to patch (the reference's
    generation.causal.KVCache, or by default wdl.kvcache.KVCache); it must keep fp8, k, ks, v, vs as the
    reference's does (causal.py:159-163)."""
    if cls is None:
        from wdl.kvcache import KVCache as cls

    original = cls.store

    def store(cache, at, k, v):  # FP8 caches through the kernel, the others as before
        if not cache.fp8:
            return original(cache, at, k, v)
        return store_kv_fp8(k, v, cache.k, cache.ks, cache.v, cache.vs, at)

    cls.store = store
    return original
