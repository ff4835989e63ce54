"""3D RoPE and the Q/K RMSNorm in front of it on MI355X (one fused HIP kernel, wdl_qk_norm_rope).

rope / rope_at tables follow src/wan_dit_lab/models/rope.py:4-10 and positions.py:7-11 (float64, then cast);
norm_rope(q, k, ...) is RMSNorm over all heads (models/rms_norm.py:10-13) followed by rope_apply
(models/rope.py:12-31) for Q and K of one chunk, as FusedQKVAttention.forward does (quantization/w4a4.py:255-257).
rope_apply / the wdl::rope3d_rotate operator are the reference's standalone rotation (kernels/rope_triton.py:66-139)
with its full contract: batches of per-sample grids, strides, fp16 / bf16 / fp32 / fp64, the inverse rotation as
its autograd backward.
"""

from __future__ import annotations

import torch

from wdl import _lib
from wdl.ops import DTYPE_CODE, qk_norm_rope_launch, stream_of


def rope(pos_count: int, pos_dim: int) -> torch.Tensor:
    pairs = pos_dim // 2
    angles = torch.arange(pos_count)[:, None] * (10000 ** (-2 * torch.arange(pairs, dtype=torch.float64) / pos_dim))
    return torch.stack((torch.cos(angles), torch.sin(angles)))


def rope_at(count: int, dim: int, scale: float) -> torch.Tensor:
    """rope at positions i * scale (positions.py:7-11)."""
    positions = torch.arange(count, dtype=torch.float64)[:, None] * scale
    angles = positions * 10000 ** (-2 * torch.arange(dim // 2, dtype=torch.float64) / dim)
    return torch.stack((torch.cos(angles), torch.sin(angles)))


def freqs(dim: int = 128, positions: int = 1024, device=None) -> torch.Tensor:
    """fp32 [2, positions, dim/2]: time, height, width tables side by side (split [22, 21, 21] for dim 128)."""
    c = dim // 2
    t, s = c - 2 * (c // 3), c // 3
    f = torch.cat([rope(positions, 2 * t), rope(positions, 2 * s), rope(positions, 2 * s)], dim=-1)
    return f.to(torch.float32).contiguous().to(device)


def _check_table(freq, grid, rows, start_frame):
    if freq.dtype not in (torch.float32, torch.float64) or not freq.is_contiguous() or freq.ndim != 3 \
            or freq.shape[0] != 2 or freq.shape[2] != 64:
        raise TypeError("freq must be a contiguous fp32 or fp64 [2, positions, 64] table")
    f, h, w = grid
    if f * h * w > rows or start_frame < 0 or start_frame + f > freq.shape[1] or max(h, w) > freq.shape[1]:
        raise ValueError("grid exceeds the rows or the frequency table")


def norm_rope(q, k, wq, wk, freq, grid, start_frame=0, eps=1e-6):
    """q, k bf16 [M, H*128] (row-strided views of the QKV output allowed) -> (Q, K) bf16 [M, H*128]:
    bf16(bf16(x * rstd) * w) then the 3D rotation of the first f*h*w rows."""
    _check_table(freq, grid, q.shape[0], start_frame)
    return qk_norm_rope_launch(q, k, wq, wk, freq, grid, start_frame, eps)


FLOATS = (torch.float16, torch.bfloat16, torch.float32, torch.float64)
MAX_BATCH = 64


@torch.library.custom_op("wdl::rope3d_rotate", mutates_args=())
def rope3d_rotate(x: torch.Tensor, freq: torch.Tensor, grid_key: str, start: int, inverse: bool,
                  output_dtype: torch.dtype) -> torch.Tensor:
    """wan_dit_lab::rope3d_rotate (kernels/rope_triton.py:66-81) on wdl_rope3d_rotate: x [B, L, H, dim] (any strides)
    turned by the 3D RoPE angles of the grids in grid_key ("f,h,w,f,h,w,..."), by -angle when inverse; a new
    contiguous tensor of output_dtype."""
    out = torch.empty(x.shape, device=x.device, dtype=output_dtype)
    if x.numel():
        grids = [int(v) for v in grid_key.split(",")]
        B, L, H, dim = x.shape
        _lib.call("wdl_rope3d_rotate", x.data_ptr(), DTYPE_CODE[x.dtype], _lib.i64s(x.stride()), freq.data_ptr(),
                  DTYPE_CODE[freq.dtype], _lib.i64s(freq.stride()), freq.shape[1], B, L, H, dim, _lib.i32s(grids),
                  int(start), int(bool(inverse)), out.data_ptr(), DTYPE_CODE[output_dtype], stream_of(x))
    return out


@rope3d_rotate.register_fake
def _(x, freq, grid_key, start, inverse, output_dtype):
    return x.new_empty(x.shape, dtype=output_dtype)


def _setup(ctx, inputs, output):
    x, freq, grid_key, start, inverse, _ = inputs
    ctx.save_for_backward(freq)
    ctx.grid_key, ctx.start, ctx.inverse, ctx.input_dtype = grid_key, start, inverse, x.dtype


def _backward(ctx, grad):
    (freq,) = ctx.saved_tensors
    # a rotation's Jacobian is its transpose: the gradient turns back by the same angles
    return rope3d_rotate(grad, freq, ctx.grid_key, ctx.start, not ctx.inverse, ctx.input_dtype), None, None, None, \
        None, None


rope3d_rotate.register_autograd(_backward, setup_context=_setup)


def rope_apply(x, grid_sizes, freq, start_frame=0, *, output_dtype=None):
    """rope_apply of kernels/rope_triton.py:84-139 on MI355X: x [B, L, H, dim] (fp16 / bf16 / fp32 / fp64, any
    strides), one grid (f, h, w) per sample (a list, or a CPU tensor), freq the real tables [2, positions, dim/2]
    (fp32 or fp64) -> a new tensor of output_dtype (x's by default); tokens past f h w copied. Every violated
    contract raises before a launch, with the reference's exception types."""
    if x.device.type != "cuda" or freq.device != x.device:
        raise ValueError("x and freq must be on the same GPU")
    if x.dtype not in FLOATS or freq.dtype not in (torch.float32, torch.float64):
        raise TypeError("x must be fp16 / bf16 / fp32 / fp64 and freq real fp32 / fp64")
    if x.ndim != 4 or x.shape[-1] < 2 or x.shape[-1] % 2:
        raise ValueError("x must be [batch, token, heads, even dim]")
    if freq.ndim != 3 or freq.shape[0] != 2 or freq.shape[2] != x.shape[-1] // 2:
        raise ValueError("freq must be [2, positions, dim / 2]")
    if freq.requires_grad:
        raise ValueError("the frequency tables are constants, not trainable")
    if isinstance(grid_sizes, torch.Tensor):
        if grid_sizes.device.type != "cpu":
            raise ValueError("grid sizes are host metadata, not device tensors")
        grid_sizes = grid_sizes.tolist()
    grids = [list(g) for g in grid_sizes]
    if not grids or len(grids) != x.shape[0]:
        raise ValueError("one grid per sample of a non-empty batch")
    if len(grids) > MAX_BATCH:
        raise ValueError(f"at most {MAX_BATCH} samples per call")
    if not isinstance(start_frame, int) or start_frame < 0:
        raise ValueError("start_frame must be a non-negative int")
    spatial = (x.shape[-1] // 2) // 3
    for g in grids:
        if len(g) != 3 or not all(isinstance(v, int) for v in g):
            raise ValueError("a grid is three ints (frames, height, width)")
        f, h, w = g
        if f < 0 or h <= 0 or w <= 0 or f * h * w > x.shape[1]:
            raise ValueError("a grid exceeds the sequence or has a non-positive extent")
        if start_frame + f > freq.shape[1] or (spatial and max(h, w) > freq.shape[1]):
            raise ValueError("the grid and offset exceed the frequency table")
    output_dtype = x.dtype if output_dtype is None else output_dtype
    if output_dtype not in FLOATS:
        raise TypeError("output_dtype must be a floating dtype")
    key = ",".join(str(v) for g in grids for v in g)
    return rope3d_rotate(x, freq, key, start_frame, False, output_dtype)
