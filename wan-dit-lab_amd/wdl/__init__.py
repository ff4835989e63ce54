"""wdl — MI355X-native (gfx950) quantized Wan DiT block hot path.

Python host code over the C ABI lib/libwdl.so (include/wdl.h): torch custom ops wdl::* (ops.py) and the module API
of the reference's hot path — PackedW4A4Linear / PackedW4A4GeluMLP / FusedQKVAttention (w4a4.py), FP8 linears
(fp8.py), the FP8 KV-cache append (cache_fp8.py), Sage-style attention over the FP8 cache (sage_kv.py), 3D RoPE
(rope.py), KVCache (kvcache.py) and the Wan block and step (block.py).
"""

__all__ = ["build"]


def build(force: bool = False):
    from wdl.build import build as _build

    return _build(force=force)
