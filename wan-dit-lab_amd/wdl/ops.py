"""The torch operators wdl::* over the C ABI of lib/libwdl.so.

Each operator is a `torch.library.custom_op` whose implementation hands raw device pointers, sizes and the current
HIP stream to one `wdl_*` launcher, and whose fake (Meta) implementation gives the output shapes, so torch.compile
and graph capture see one opaque op, as the reference's TORCH_LIBRARY ops live::* are
(native/ops/w4a4_ops.cpp:79-95; native/ops/sage_ops.cpp:28-35). Outputs and workspaces are allocated here, by
torch, on the current stream; the library allocates nothing.
"""

from __future__ import annotations

import torch

from wdl import _lib

DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------------------------------------ KV cache append

@torch.library.custom_op("wdl::store_kv_fp8", mutates_args=("cache_k", "cache_ks", "cache_v", "cache_vs"))
def store_kv_fp8_op(k: torch.Tensor, v: torch.Tensor, cache_k: torch.Tensor, cache_ks: torch.Tensor,
                    cache_v: torch.Tensor, cache_vs: torch.Tensor, at: int) -> None:
    b, n, h, d = k.shape
    if k.numel() == 0:
        return
    _lib.call("wdl_kv_append_fp8", ptr(k), DTYPE_CODE[k.dtype], _lib.i64s(k.stride()), ptr(v), DTYPE_CODE[v.dtype],
              _lib.i64s(v.stride()), b, n, h, d, ptr(cache_k), ptr(cache_ks), ptr(cache_v), ptr(cache_vs),
              cache_k.shape[1], at, stream_of(k))


@store_kv_fp8_op.register_fake
def _(k, v, cache_k, cache_ks, cache_v, cache_vs, at):
    return None
