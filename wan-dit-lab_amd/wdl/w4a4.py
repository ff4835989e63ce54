"""W4A4 linears of SVDQuant on MI355X: the module API of src/wan_dit_lab/quantization/w4a4.py over the wdl::* ops.

    y = x W^T + b = Q(x / s) Q(R)^T + (x proj_down) proj_up^T + b,      W diag(s) = up down + R     (w4a4.py:4-10)

Weights are quantized offline (quantize, w4a4.py:140-180) into wdl's own packed layout (the reference packs
into Nunchaku's MMA tile order, which lives outside its tree):
- qweight uint8 [N, K/2]: per 64-channel group, byte j holds k = j in the low nibble and k = j + 32 in the high
  nibble, two's complement int4 (pack_weight / unpack_weight);
- wscales bf16 (or fp16) [K/64, N] (group-major); proj_down bf16 [32, K] (the down factor divided by s, transposed);
  proj_up bf16 [N, 32]; smooth bf16 [K]; bias bf16 [N] (shift-corrected for the second GELU-MLP layer).
The integer values are those of int4_groups (w4a4.py:80-100) on the quantizer input R; the int4 parity of the
build is defined on R, since the SVD is not bit-portable between LAPACK and rocSOLVER.
"""

from __future__ import annotations

import torch

from wdl import ops
from wdl.ops import GELU_SHIFT, w4a4_gelu_mlp, w4a4_linear

GROUP = 64
PARTS = ("qweight", "wscales", "proj_down", "proj_up", "smooth", "bias")  # w4a4.py:207
MSE_STEPS = torch.linspace(0.5, 1.0, 26).tolist()

__all__ = ["GROUP", "GELU_SHIFT", "PARTS", "int4_groups", "gptq", "smoothing", "quantize", "pack_weight",
           "unpack_weight",
           "linear", "gelu_mlp", "w4a4_linear", "w4a4_gelu_mlp", "PackedW4A4Linear", "PackedW4A4GeluMLP",
           "FusedQKVAttention"]


@torch.no_grad()
def int4_groups(R: torch.Tensor, rule: str = "max"):
    """R [N, K] in symmetric INT4 groups of 64 input channels (w4a4.py:80-100): the integers [N, K] and the fp32
    scales [N, K/64]. "max": the largest |x| of a group maps to 7. "mse": of the scales MSE_STEPS times that one,
    the one with the least squared error of the group."""
    N, K = R.shape
    g = R.float().reshape(N, K // GROUP, GROUP)
    base = g.abs().amax(dim=-1).clamp(min=1e-8) / 7
    scale = base
    if rule == "mse":
        best = None
        for c in MSE_STEPS:
            s = base * c
            err = (g - torch.round(g / s[..., None]).clamp(-8, 7) * s[..., None]).square().sum(-1)
            if best is None:
                best, scale = err, s
            else:
                take = err < best
                best = torch.where(take, err, best)
                scale = torch.where(take, s, scale)
    elif rule != "max":
        raise ValueError(f"unknown rule {rule!r}")
    q = torch.round(g / scale[..., None]).clamp(-8, 7).to(torch.int32).reshape(N, K)
    return q, scale


@torch.no_grad()
def gptq(R: torch.Tensor, H: torch.Tensor, damp: float = 0.01):
    """GPTQ rounding (Frantar et al., "GPTQ: Accurate Post-Training Quantization for Generative Pre-trained
    Transformers", ICLR 2023) of R [N, K] into symmetric int4 groups of 64 input channels, minimising
    ||X R^T - X Q(R)^T|| for inputs with H = X^T X [K, K] (w4a4.py:103-137 states the same method).

    Channels that never carry input (H[k, k] = 0) are zeroed and given a unit diagonal; the diagonal is damped by
    damp * its mean. U is the upper Cholesky factor of H^-1. Columns are rounded in order, one 64-column group at a
    time: the group's scale is amax / 7 of its columns as the earlier groups' updates left them; inside the group
    each column's rounding error e = (w - q s) / U[c, c] is pushed onto the group's later columns at once (e
    U[c, later]); at the end of the group its errors E update every later column in one product (E U[group,
    later]). Returns the integers int32 [N, K] and the fp32 scales [N, K / 64]."""
    W = R.float().clone()
    N, K = W.shape
    if K % GROUP:
        raise ValueError(f"K = {K} is not a multiple of {GROUP}")
    Hd = H.float().clone().to(W.device)
    diag = Hd.diagonal()
    dead = diag == 0
    diag[dead] = 1.0
    W[:, dead] = 0.0
    diag += damp * diag.mean()
    U = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(Hd)), upper=True)
    q = torch.empty(N, K, dtype=torch.int32, device=W.device)
    scales = torch.empty(N, K // GROUP, device=W.device)
    for g0 in range(0, K, GROUP):
        g1 = g0 + GROUP
        s = W[:, g0:g1].abs().amax(dim=1).clamp(min=1e-8) / 7
        scales[:, g0 // GROUP] = s
        E = torch.empty(N, GROUP, device=W.device)
        for j in range(GROUP):
            c = g0 + j
            w = W[:, c]
            qc = torch.round(w / s).clamp(-8, 7)
            q[:, c] = qc.to(torch.int32)
            e = (w - qc * s) / U[c, c]
            E[:, j] = e
            if c + 1 < g1:
                W[:, c + 1:g1] -= e[:, None] * U[c, c + 1:g1][None, :]
        if g1 < K:
            W[:, g1:] -= E @ U[g0:g1, g1:]
    return q, scales


def smoothing(act_amax: torch.Tensor, weight: torch.Tensor, alpha: float = 0.5) -> torch.Tensor:
    """SmoothQuant's per-input-channel s = max|x|^alpha / max|W|^(1-alpha), clamped to [1e-2, 1e2]
    (w4a4.py:183-186)."""
    wmax = weight.float().abs().amax(dim=0).clamp(min=1e-5)
    amax = act_amax.float().to(wmax.device).clamp(min=1e-5)
    return (amax ** alpha / wmax ** (1 - alpha)).clamp(min=1e-2, max=1e2)


def pack_weight(q: torch.Tensor) -> torch.Tensor:
    """int4 values [N, K] -> uint8 [N, K/2] in wdl's layout (module docstring)."""
    N, K = q.shape
    u = (q.to(torch.int32) & 0xF).to(torch.uint8).reshape(N, K // GROUP, 2, GROUP // 2)
    return (u[:, :, 0] | (u[:, :, 1] << 4)).reshape(N, K // 2).contiguous()


def unpack_weight(p: torch.Tensor) -> torch.Tensor:
    """uint8 [N, K/2] -> int32 [N, K] (inverse of pack_weight)."""
    N, H = p.shape
    b = p.reshape(N, H // 32, 32).to(torch.int32)
    lo, hi = b & 0xF, b >> 4
    v = torch.stack([lo, hi], dim=2).reshape(N, H * 2)
    return torch.where(v >= 8, v - 16, v)


@torch.no_grad()
def quantize(weight, bias=None, smooth=None, rank: int = 32, shift: float = 0.0, rule: str = "max", R=None,
             hessian=None, scale_dtype=torch.bfloat16):
    """The tensors of a W4A4 layer for y = x W^T + b (w4a4.py:140-180) in wdl's packed layout.
    weight [N, K]; smooth [K] (ones when None); shift: the second GELU-MLP layer quantizes x + shift unsigned, so
    its bias takes off shift * (Q(R) / s) 1. R: the quantizer input, when given (parity tests). hessian [K, K]:
    X^T X of the inputs the int4 branch multiplies by R (x + shift for the GELU MLP's second layer, before
    smoothing): R is then rounded by gptq in the smoothed space (whose Hessian is diag(1/s) H diag(1/s)) instead
    of to the nearest. scale_dtype: the weight scales' type, bf16 (the reference's) or fp16."""
    if scale_dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("weight scales are bf16 or fp16")
    W = weight.float()
    N, K = W.shape
    dev = W.device
    s = torch.ones(K, device=dev) if smooth is None else smooth.float().to(dev)
    Ws = W * s[None, :]
    U, S, Vh = torch.linalg.svd(Ws, full_matrices=False)
    up, down = U[:, :rank] * S[:rank], Vh[:rank]
    if R is None:
        R = Ws - up @ down
    if hessian is None:
        q, scale = int4_groups(R.to(dev), rule)
    else:
        Hs = hessian.float().to(dev) / s[:, None] / s[None, :]
        q, scale = gptq(R.to(dev), Hs)
    b = torch.zeros(N, device=dev) if bias is None else bias.float().to(dev)
    if shift:
        deq = (q.reshape(N, K // GROUP, GROUP).float() * scale[..., None]).reshape(N, K)
        b = b - shift * (deq / s[None, :]).sum(dim=1)
    return dict(
        qweight=pack_weight(q),
        wscales=scale.to(scale_dtype).t().contiguous(),
        proj_down=(down / s[None, :]).to(torch.bfloat16).contiguous(),
        proj_up=up.to(torch.bfloat16).contiguous(),
        smooth=s.to(torch.bfloat16),
        bias=b.to(torch.bfloat16),
    )


def random_parts(N: int, K: int, device, generator=None, rank: int = 32, scale: float = 0.02, unsigned_input=False,
                 scale_dtype=torch.bfloat16):
    """A W4A4 layer of the right shapes and value ranges without an SVD (random-init weights of the architecture,
    for the step benchmark): int4 in [-7, 7], group scales of a N(0, scale^2) weight, small low-rank factors."""
    g = generator  # a generator on `device` (or None: the global one of that device)
    kw = dict(generator=g, device=device)
    q = torch.randint(-7, 8, (N, K), dtype=torch.int32, **kw)
    wsc = (torch.rand(K // GROUP, N, **kw) * 0.5 + 0.75) * (3 * scale / 7)
    return dict(
        qweight=pack_weight(q),
        wscales=wsc.to(scale_dtype),
        proj_down=(torch.randn(rank, K, **kw) * (1 / K ** 0.5)).to(torch.bfloat16),
        proj_up=(torch.randn(N, rank, **kw) * scale).to(torch.bfloat16),
        smooth=torch.ones(K, dtype=torch.bfloat16, device=device),
        bias=(torch.randn(N, **kw) * scale).to(torch.bfloat16),
    )


def linear(x: torch.Tensor, t: dict) -> torch.Tensor:
    """y = x W^T + b for x [M, K] bf16 and t the tensors of quantize (w4a4.py:189-192)."""
    return w4a4_linear(x, *(t[part] for part in PARTS))


def gelu_mlp(x: torch.Tensor, t1: dict, t2: dict) -> torch.Tensor:
    """GELU(x W1^T + b1) W2^T + b2, t2 made with shift=GELU_SHIFT (w4a4.py:198-204)."""
    return w4a4_gelu_mlp(x, *(t1[p] for p in PARTS), *(t2[p] for p in PARTS))


def _operand(parts: dict, name: str):
    """Module operands: packed weights on the GPU are expanded once to the GEMM's tile-blocked fp6 codes (e3m2 of 2w) of [N, K]."""
    t = parts[name]
    return ops.weight_codes(t) if name == "qweight" and t.is_cuda else t


class PackedW4A4Linear(torch.nn.Module):
    """A W4A4 linear layer over the parts of quantize (w4a4.py:220-231)."""

    def __init__(self, **parts):
        super().__init__()
        self.parts = [_operand(parts, name) for name in PARTS]
        self.out_features = parts["proj_up"].shape[0]

    def forward(self, X):
        y = w4a4_linear(X.reshape(-1, X.shape[-1]).to(torch.bfloat16).contiguous(), *self.parts)
        return y.reshape(*X.shape[:-1], self.out_features)


class PackedW4A4GeluMLP(torch.nn.Module):
    """Wan's feed forward (Linear, GELU tanh, Linear) in W4A4 as one gelu_mlp (w4a4.py:234-245)."""

    def __init__(self, fc1, fc2):
        super().__init__()
        self.parts = [_operand(fc1, name) for name in PARTS] + [_operand(fc2, name) for name in PARTS]
        self.out_features = fc2["proj_up"].shape[0]

    def forward(self, X):
        y = w4a4_gelu_mlp(X.reshape(-1, X.shape[-1]).to(torch.bfloat16).contiguous(), *self.parts)
        return y.reshape(*X.shape[:-1], self.out_features)


class FusedQKVAttention(torch.nn.Module):
    """Self-attention with q, k, v as one W4A4 layer qkv [3 dim, dim] (w4a4.py:246-262): X quantized once, one GEMM,
    then the fused Q/K RMSNorm + 3D RoPE kernel, the KVCache's Sage attention over the FP8 window (or, with no
    cache, the chunk attending to itself in bf16 with an exact fp32 softmax, as the reference's
    scaled_dot_product_attention does, w4a4.py:259-261) and the W4A4 o projection. qkv / o: PackedW4A4Linear;
    norm_q / norm_k: bf16 RMSNorm weights [dim]."""

    def __init__(self, dim, num_heads, eps=1e-6):
        super().__init__()
        self.dim, self.num_heads, self.head_dim, self.eps = dim, num_heads, dim // num_heads, eps
        self.qkv = self.o = None
        self.norm_q = self.norm_k = None

    def forward(self, X, grid_sizes=None, freq=None, context=None, start_frame=0, cache=None, context_kv=None):
        from wdl import rope

        assert context is None and context_kv is None, "q, k and v of one input: self-attention only"
        if self.head_dim != 128:
            raise ValueError("the MI355X kernels take heads of 128")
        B, L = X.shape[0], X.shape[-2]
        if B != 1:
            raise ValueError("batch 1 (one chunk of one stream)")
        qkv = self.qkv(X).reshape(L, 3 * self.dim)
        g = grid_sizes[0].tolist() if isinstance(grid_sizes, torch.Tensor) else grid_sizes[0]
        Q, K = rope.norm_rope(qkv[:, :self.dim], qkv[:, self.dim:2 * self.dim], self.norm_q, self.norm_k, freq,
                              tuple(int(v) for v in g), start_frame, self.eps)
        shape = (1, L, self.num_heads, self.head_dim)
        V = qkv[:, 2 * self.dim:]
        if cache is not None:
            A = cache.attend(Q.view(shape), K.view(shape), V.reshape(shape))
        else:  # SDPA over the chunk alone (w4a4.py:259-261): bf16 operands, exact softmax
            A = ops.attn_bf16_launch(Q, ops.attn_bf16_prep_launch(K, V), self.head_dim ** -0.5)
        return self.o(A.reshape(1, L, self.dim))


def pack_parts(logical: dict, device=None) -> dict:
    """Logical parts (q int [N, K], wscales [N, K/64], proj_down [K, r], proj_up [N, r], smooth [K], bias [N]) ->
    wdl's packed layout, on `device`. fp16 weight scales stay fp16, any other type becomes bf16."""
    return dict(
        qweight=pack_weight(logical["q"]).to(device),
        wscales=logical["wscales"].to(logical["wscales"].dtype if logical["wscales"].dtype == torch.float16
                                      else torch.bfloat16).t().contiguous().to(device),
        proj_down=logical["proj_down"].to(torch.bfloat16).t().contiguous().to(device),
        proj_up=logical["proj_up"].to(torch.bfloat16).contiguous().to(device),
        smooth=logical["smooth"].to(torch.bfloat16).to(device),
        bias=logical["bias"].to(torch.bfloat16).to(device),
    )


def unpack_parts(parts: dict) -> dict:
    """Inverse of pack_parts, on the CPU."""
    return dict(q=unpack_weight(parts["qweight"].cpu()), wscales=parts["wscales"].cpu().t().contiguous(),
                proj_down=parts["proj_down"].cpu().t().contiguous(), proj_up=parts["proj_up"].cpu(),
                smooth=parts["smooth"].cpu(), bias=parts["bias"].cpu())
