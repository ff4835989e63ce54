"""FP8 (E4M3) linear layers on MI355X: the API of src/wan_dit_lab/quantization/fp8.py over wdl's HIP kernels.

W8A8: the weight in FP8 with one scale per tensor (Fp8Linear, PackedFp8Linear, DynamicFp8Linear rows=False) or one
per output row (DynamicFp8Linear rows=True), the activation quantized on every call by its own maximum (per tensor
or per token). wdl_fp8_quantize quantizes (fp8.py:14-17, 37-41); wdl_fp8_gemm multiplies on the fp8 MFMA with
_scaled_mm's epilogue (fp8.py:32-33, 57-66, 92-93). The GEMM tiles need out_features % 128 == 0 and
in_features % 64 == 0; other shapes raise ValueError.
"""

from __future__ import annotations

import torch

from wdl import _lib
from wdl.ops import ptr, stream_of, workspace

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0
ROWS_PAD = 128

__all__ = ["FP8", "FP8_MAX", "quantize", "quantize_rows", "Fp8Linear", "DynamicFp8Linear", "PackedFp8Linear",
           "to_fp8", "to_dynamic_fp8", "quantize_padded", "gemm", "weight_only_gemm", "Fp8WeightOnlyLinear",
           "to_fp8_weight_only"]


def _dtype_code(x):
    codes = {torch.bfloat16: 2, torch.float32: 0}
    if x.dtype not in codes:
        raise TypeError(f"fp8 quantization takes bf16 or fp32, got {x.dtype}")
    return codes[x.dtype]


def quantize_padded(x: torch.Tensor, rows: bool, pad: int = ROWS_PAD):
    """x [M, K] (bf16 / fp32, unit column stride) -> (q uint8 [Mp, K] e4m3 codes, rows >= M zero; scale fp32 [Mp]
    (rows) or [1] (tensor)), Mp = ceil(M / pad) * pad."""
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be a [M, K] matrix with contiguous rows")
    M, K = x.shape
    Mp = (M + pad - 1) // pad * pad
    q = torch.empty(Mp, K, device=x.device, dtype=torch.uint8)
    scale = torch.empty(Mp if rows else 1, device=x.device, dtype=torch.float32)
    ws = None
    if not rows:
        n = _lib.library().wdl_fp8_quantize_workspace_floats(M, K)
        ws = torch.empty(n, device=x.device, dtype=torch.float32)
    _lib.call("wdl_fp8_quantize", ptr(x), _dtype_code(x), x.stride(0), M, K, Mp, int(rows), ptr(q), ptr(scale),
              ptr(ws), stream_of(x))
    return q, scale


def quantize(X: torch.Tensor):
    """fp8.py:14-17: X in FP8 (same shape) and the 0-d fp32 scale it was divided by; the largest |X| goes to 448."""
    x = X.reshape(-1, X.shape[-1])
    q, scale = quantize_padded(x.contiguous(), rows=False, pad=1)
    return q.view(FP8).view(X.shape), scale.reshape(())


def quantize_rows(X: torch.Tensor):
    """fp8.py:37-41: X [..., d] in FP8 with one fp32 scale per row ([..., 1])."""
    x = X.reshape(-1, X.shape[-1])
    q, scale = quantize_padded(x.contiguous(), rows=True, pad=1)
    return q.view(FP8).view(X.shape), scale.view(*X.shape[:-1], 1)


_FP8_GEMM_WS: dict = {}  # stream-K partial sums, one buffer per device (wdl.ops.workspace)


def gemm(q: torch.Tensor, x_scale: torch.Tensor, M: int, w_codes: torch.Tensor, w_scale: torch.Tensor,
         bias: torch.Tensor | None, rows: bool, stream_k: bool = True) -> torch.Tensor:
    """The FP8 product of quantize_padded's output with an FP8 weight [N, K] -> bf16 [M, N]. stream_k: let long-K
    shapes that leave CUs idle split K over the CUs (fp32 partial sums in a per-device workspace; a different but
    fixed summation order); False: the one-pass launch."""
    Mp, K = q.shape
    N = w_codes.shape[0]
    if w_codes.shape[1] != K or N % 128 or K % 64:
        raise ValueError(f"fp8 GEMM needs [N, K] weights with N % 128 == 0 and K % 64 == 0, got {tuple(w_codes.shape)}")
    b = None if bias is None else bias.to(torch.bfloat16).contiguous()
    out = torch.empty(M, N, device=q.device, dtype=torch.bfloat16)
    nbytes = _lib.library().wdl_fp8_gemm_workspace_bytes(Mp, N, K) if stream_k else 0
    ws = workspace(_FP8_GEMM_WS, q.device, nbytes) if nbytes else None
    _lib.call("wdl_fp8_gemm", ptr(q), ptr(x_scale), ptr(w_codes.view(torch.uint8)), ptr(w_scale), ptr(b), M, Mp, N,
              K, int(rows), ptr(out), out.stride(0), ptr(ws), stream_of(q))
    return out


def weight_only_gemm(x: torch.Tensor, w_codes: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None,
                     out: torch.Tensor | None = None, gate: torch.Tensor | None = None) -> torch.Tensor:
    """The FP8 weight-only product: x bf16 [M, K] (row-strided, ldx % 8 == 0) times an e4m3 weight [N, K] with fp32
    scales [N] (per output row) or [1] -> bf16 [M, N] = w_scale * (x . w) + bias. With `gate` (fp32 [N]) the result
    is added into `out` as the gated residual out = bf16(out + bf16(y) * gate)."""
    M, K = x.shape
    N = w_codes.shape[0]
    if x.dtype != torch.bfloat16 or x.stride(1) != 1 or w_codes.shape[1] != K or N % 128 or K % 64:
        raise ValueError(f"weight-only FP8 GEMM: bf16 x [M, K] and an [N, K] weight, N % 128 == 0, K % 64 == 0; "
                         f"got {tuple(x.shape)} and {tuple(w_codes.shape)}")
    # the kernel reads the weight as dense rows of K codes: a transposed or sliced view would be read wrongly
    if w_codes.element_size() != 1 or not w_codes.is_contiguous():
        raise ValueError("weight-only FP8 GEMM: the weight must be a contiguous e4m3 [N, K] tensor")
    if w_scale.dtype != torch.float32 or w_scale.numel() not in (1, N) or not w_scale.is_contiguous():
        raise ValueError("w_scale: contiguous fp32 [N] or [1]")
    if bias is not None and bias.numel() != N:
        raise ValueError(f"bias: {N} values, got {bias.numel()}")
    tensors = [t for t in (x, w_codes, w_scale, bias, out, gate) if t is not None]
    if any(t.device != x.device for t in tensors):
        raise ValueError("weight-only FP8 GEMM: every tensor must be on x's device")
    b = None if bias is None else bias.to(torch.bfloat16).contiguous()
    if out is not None and (out.shape != (M, N) or out.dtype != torch.bfloat16 or out.stride(1) != 1):
        raise ValueError(f"out must be bf16 [{M}, {N}] with unit column stride")
    if gate is not None:
        if out is None:
            raise ValueError("the gated residual needs out bf16 [M, N]")
        if gate.numel() != N:
            raise ValueError(f"gate: {N} values, got {gate.numel()}")
        gate = gate.float().contiguous()
    elif out is None:
        out = torch.empty(M, N, device=x.device, dtype=torch.bfloat16)
    _lib.call("wdl_fp8wo_gemm", ptr(x), x.stride(0), ptr(w_codes.view(torch.uint8)), ptr(w_scale),
              int(w_scale.numel() == N and N > 1), ptr(b), M, N, K, ptr(out), out.stride(0), 0 if gate is None else 2,
              ptr(gate), stream_of(x))
    return out


class Fp8WeightOnlyLinear(torch.nn.Module):
    """A linear layer with its weight in FP8 (e4m3, one scale per output row, or per tensor with rows=False) and
    the activation kept in bf16: y = x (w * scale)^T + b. Not a mode of the reference, whose FP8 linears quantize
    the activation too (quantization/fp8.py:1-6); the attention projections of the mixed-precision benchmark mode."""

    def __init__(self, linear, rows=True):
        super().__init__()
        W = linear.weight.detach()
        if W.dtype not in (torch.bfloat16, torch.float32):  # the quantizer reads bf16 or fp32; fp32 holds any float
            W = W.float()
        wq, ws = quantize_padded(W.contiguous(), rows=rows, pad=1)
        self.register_buffer("weight", wq.view(FP8))
        self.register_buffer("scale", ws)
        self.register_buffer("bias", None if linear.bias is None else linear.bias.detach().to(torch.bfloat16))
        self.out_features = linear.out_features

    def forward(self, X):
        x = X.reshape(-1, X.shape[-1]).to(torch.bfloat16).contiguous()
        y = weight_only_gemm(x, self.weight, self.scale, self.bias)
        return y.reshape(*X.shape[:-1], self.out_features)


def to_fp8_weight_only(module, rows=True):
    """Every nn.Linear inside `module` replaced by an Fp8WeightOnlyLinear, in place (weights on the GPU)."""
    for name, child in module.named_children():
        if isinstance(child, torch.nn.Linear):
            setattr(module, name, Fp8WeightOnlyLinear(child, rows))
        else:
            to_fp8_weight_only(child, rows)
    return module


class Fp8Linear(torch.nn.Module):
    """fp8.py:20-34: nn.Linear with the weight in FP8 (one scale), x quantized on the fly; output bf16."""

    def __init__(self, linear):
        super().__init__()
        W = linear.weight.detach()
        wq, ws = quantize_padded(W.contiguous(), rows=False, pad=1)
        self.register_buffer("weight", wq.view(FP8))
        self.register_buffer("scale", ws)
        self.register_buffer("bias", None if linear.bias is None else linear.bias.detach().to(torch.bfloat16))
        self.out_features = linear.out_features

    def forward(self, X):
        x = X.reshape(-1, X.shape[-1]).contiguous()
        q, s = quantize_padded(x, rows=False)
        y = gemm(q, s, x.shape[0], self.weight, self.scale, self.bias, rows=False)
        return y.reshape(*X.shape[:-1], self.out_features)


class DynamicFp8Linear(torch.nn.Module):
    """fp8.py:44-67: W8A8 over an nn.Linear whose weight may change in place; the weight is quantized on every
    call. rows=False: one scale per tensor; rows=True: one per token of x and one per output row of W, applied to
    the bf16 product (y_ij = s_i t_j sum_k x_ik w_jk)."""

    def __init__(self, linear, rows=False):
        super().__init__()
        self.linear, self.rows = linear, rows

    def forward(self, X):
        W, b = self.linear.weight, self.linear.bias
        x = X.reshape(-1, X.shape[-1]).contiguous()
        q, s = quantize_padded(x, rows=self.rows)
        wq, ws = quantize_padded(W.detach().contiguous(), rows=self.rows, pad=1)
        y = gemm(q, s, x.shape[0], wq, ws, None if b is None else b.detach(), rows=self.rows)
        return y.reshape(*X.shape[:-1], W.shape[0])


def to_dynamic_fp8(module, rows=False):
    """fp8.py:70-77: every nn.Linear inside `module` wrapped by a DynamicFp8Linear, in place."""
    for name, child in module.named_children():
        if isinstance(child, torch.nn.Linear):
            setattr(module, name, DynamicFp8Linear(child, rows))
        else:
            to_dynamic_fp8(child, rows)
    return module


class PackedFp8Linear(torch.nn.Module):
    """fp8.py:80-94: a linear layer over an FP8 weight [out, in], its 0-d fp32 scale and a bf16 bias (views of a
    packed row of bytes); only the activation is quantized."""

    def __init__(self, weight, scale, bias):
        super().__init__()
        self.weight, self.scale, self.bias = weight, scale, bias
        self.out_features = weight.shape[0]

    def forward(self, X):
        x = X.reshape(-1, X.shape[-1]).contiguous()
        q, s = quantize_padded(x, rows=False)
        y = gemm(q, s, x.shape[0], self.weight, self.scale.reshape(1).float(), self.bias, rows=False)
        return y.reshape(*X.shape[:-1], self.out_features)


def to_fp8(module):
    """fp8.py:122-129: every nn.Linear inside `module` replaced by an Fp8Linear, in place (weights on the GPU)."""
    for name, child in module.named_children():
        if isinstance(child, torch.nn.Linear):
            setattr(module, name, Fp8Linear(child))
        else:
            to_fp8(child)
    return module
