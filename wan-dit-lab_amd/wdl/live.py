"""`live::` operator names over libwdl, for code written against the reference's native ops.

The reference registers `live::w4a4_linear` and `live::w4a4_gelu_mlp` from Nunchaku-based DLLs
(src/wan_dit_lab/kernels/operators.py:12-24; native/ops/w4a4_ops.cpp:79-95) and calls them as
`torch.ops.live.w4a4_linear(...)` (quantization/w4a4.py:212-213, 242-245). Importing this module registers the same
names and schemas over wdl's HIP kernels, so those call sites run unchanged on MI355X, given weights packed
by wdl.w4a4.quantize (wdl's layout; Nunchaku's tile order is not reproduced).

`live::sage_sm89` takes the reference's argument list over the operands the reference's sage_kv._attend builds
(kernels/sage_kv.py:141-176: int8 K [1, L, H, 128], fp8 V [1, 128, H, Lpad] in Sage's 16-token order, the scales),
copied into wdl's layouts on the device, or over wdl's own layouts (wdl.sage_kv.quant_q / prep). The faster swap
point is one level up, `sage_kv.attend` / `KVCache.attend` (kernels/sage_kv.py:127-134; generation/causal.py:193-220),
replaced by wdl.sage_kv.attend / wdl.kvcache.KVCache, whose preparation writes wdl's layouts directly.
"""

from __future__ import annotations

import torch

from wdl import ops

__all__ = ["load", "w4a4_linear", "w4a4_gelu_mlp", "sage_sm89"]


@torch.library.custom_op("live::w4a4_linear", mutates_args=())
def w4a4_linear(x: torch.Tensor, qweight: torch.Tensor, wscales: torch.Tensor, proj_down: torch.Tensor,
                proj_up: torch.Tensor, smooth: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """live::w4a4_linear (w4a4_ops.cpp:31-40, 79-80) on libwdl."""
    return ops.w4a4_linear(x, qweight, wscales, proj_down, proj_up, smooth, bias)


@w4a4_linear.register_fake
def _(x, qweight, wscales, proj_down, proj_up, smooth, bias):
    return x.new_empty(x.shape[0], ops.out_features(qweight), dtype=torch.bfloat16)


@torch.library.custom_op("live::w4a4_gelu_mlp", mutates_args=())
def w4a4_gelu_mlp(x: torch.Tensor, qweight1: torch.Tensor, wscales1: torch.Tensor, proj_down1: torch.Tensor,
                  proj_up1: torch.Tensor, smooth1: torch.Tensor, bias1: torch.Tensor, qweight2: torch.Tensor,
                  wscales2: torch.Tensor, proj_down2: torch.Tensor, proj_up2: torch.Tensor, smooth2: torch.Tensor,
                  bias2: torch.Tensor) -> torch.Tensor:
    """live::w4a4_gelu_mlp (w4a4_ops.cpp:44-63, 81-85) on libwdl."""
    return ops.w4a4_gelu_mlp(x, qweight1, wscales1, proj_down1, proj_up1, smooth1, bias1, qweight2, wscales2,
                             proj_down2, proj_up2, smooth2, bias2)


@w4a4_gelu_mlp.register_fake
def _(x, qweight1, wscales1, proj_down1, proj_up1, smooth1, bias1, qweight2, wscales2, proj_down2, proj_up2,
      smooth2, bias2):
    return x.new_empty(x.shape[0], ops.out_features(qweight2), dtype=torch.bfloat16)


@torch.library.custom_op("live::sage_sm89", mutates_args=())
def sage_sm89(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_scale: torch.Tensor, k_scale: torch.Tensor,
              v_scale: torch.Tensor, sm_scale: float) -> torch.Tensor:
    """live::sage_sm89 (sage_ops.cpp:12-19, 28-31) on libwdl (either layout, see the module docstring)."""
    return ops.sage_sm89(q, k, v, q_scale, k_scale, v_scale, sm_scale)


@sage_sm89.register_fake
def _(q, k, v, q_scale, k_scale, v_scale, sm_scale):
    return q.new_empty(q.shape, dtype=torch.bfloat16)


def load():
    """The counterpart of operators.load() (kernels/operators.py:19-24): checks that libwdl.so is built (raises
    FileNotFoundError otherwise, as the reference does for its DLLs) and returns torch.ops.live."""
    from wdl import _lib

    _lib.library()
    return torch.ops.live
