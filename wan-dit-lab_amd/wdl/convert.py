"""Whole-block conversion of a float Wan block to W4A4 with calibrated smoothing: the counterpart of
src/wan_dit_lab/quantization/w4a4.py:265-357 (layers, layer_parts, install, convert) over wdl's layout and modules,
and quantized_block(), the same parts as one QuantizedWanBlock (the fused hot path of the step).

A float block is any torch module with the names of the reference's WanBlock (models/block.py:11-20): self_attn /
cross_attn with q, k, v, o (nn.Linear) and norm_q, norm_k (RMSNorm, a .weight each), ffn = (Linear, GELU, Linear),
norm3 with an affine weight and bias, and modulation [1, 6, dim].

Calibration: amax maps "<block index>.<linear name>" to the largest |x| of each input channel of that linear
(input_amax records it with forward hooks while the caller runs the float model); a layer without an entry keeps
unit smoothing. Members of a fused layer share their input, so the first member's entry is used, as the reference
does (w4a4.py:327).
"""

from __future__ import annotations

import torch

from wdl import w4a4

QKV = ("self_attn.q", "self_attn.k", "self_attn.v")  # one input: one layer self_attn.qkv when fused
FFN = ("ffn.0", "ffn.2")  # Linear, GELU, Linear: one fused GELU MLP when fused
# the layers of a fused block -> the part names of QuantizedWanBlock
BLOCK_LINEARS = {"self_attn.qkv": "qkv", "self_attn.o": "o", "cross_attn.q": "cq", "cross_attn.k": "ck",
                 "cross_attn.v": "cv", "cross_attn.o": "co", "ffn.0": "ffn1", "ffn.2": "ffn2"}


def layers(block: torch.nn.Module, fused: bool = False, keep=()) -> dict:
    """The W4A4 layers of `block`: {layer name: [(linear name, nn.Linear), ...] stacked by output}; fused: q, k and v
    of self-attention as one layer self_attn.qkv; keep: names of linears left unquantized."""
    out: dict = {}
    for name, m in block.named_modules():
        if isinstance(m, torch.nn.Linear) and name not in keep:
            out.setdefault("self_attn.qkv" if fused and name in QKV else name, []).append((name, m))
    return out


@torch.no_grad()
def layer_parts(block: torch.nn.Module, index: int = 0, amax: dict | None = None, alpha: float = 0.5,
                rank: int = 32, fused: bool = False, keep=(), hessians: dict | None = None, rule: str = "max",
                scale_dtype=torch.bfloat16, device=None) -> dict:
    """{layer: the packed parts of wdl.w4a4.quantize} for every layer of `layers` (computed on `device`, by default
    the block's). Smoothing s = smoothing(amax + shift, W, alpha) from the calibration maxima; in a fused block the
    feed-forward's second layer is made for the fused GELU MLP, which quantizes GELU's output + GELU_SHIFT unsigned
    (so its maxima are taken of that shifted input). hessians {layer: X^T X of its input}: GPTQ rounding instead of
    to the nearest."""
    amax = amax or {}
    out = {}
    for g, members in layers(block, fused, keep).items():
        dev = device if device is not None else members[0][1].weight.device
        W = torch.cat([m.weight.detach().to(dev, torch.float32) for _, m in members])
        b = None
        if any(m.bias is not None for _, m in members):
            b = torch.cat([torch.zeros(m.out_features, device=dev) if m.bias is None else
                           m.bias.detach().to(dev, torch.float32) for _, m in members])
        shift = w4a4.GELU_SHIFT if fused and g == FFN[1] else 0.0
        a = amax.get(f"{index}.{members[0][0]}")
        s = None if a is None else w4a4.smoothing(a.to(dev).float() + shift, W, alpha)
        H = None if hessians is None else hessians.get(g)
        out[g] = w4a4.quantize(W, b, smooth=s, rank=rank, shift=shift, rule=rule, hessian=H,
                               scale_dtype=scale_dtype)
    return out


def install(block: torch.nn.Module, parts: dict, gelu_mlp: bool | None = None) -> torch.nn.Module:
    """`block` with its layers from `parts` ({layer: packed parts}, on the GPU) as wdl modules, in place:
    self_attn.qkv makes self_attn a FusedQKVAttention (its RMSNorm weights and o projection carried over), gelu_mlp
    (by default when self_attn.qkv is there) makes ffn a PackedW4A4GeluMLP, every other listed linear a
    PackedW4A4Linear; linears without parts stay as they are."""
    if gelu_mlp is None:
        gelu_mlp = "self_attn.qkv" in parts
    if "self_attn.qkv" in parts:
        old = block.self_attn
        fused = w4a4.FusedQKVAttention(old.dim, old.num_heads)
        fused.qkv = w4a4.PackedW4A4Linear(**parts["self_attn.qkv"])
        fused.o = (w4a4.PackedW4A4Linear(**parts["self_attn.o"]) if "self_attn.o" in parts else old.o)
        dev = parts["self_attn.qkv"]["bias"].device
        fused.norm_q = old.norm_q.weight.detach().to(dev, torch.bfloat16)
        fused.norm_k = old.norm_k.weight.detach().to(dev, torch.bfloat16)
        fused.eps = getattr(old.norm_q, "eps", fused.eps)
        block.self_attn = fused
    if gelu_mlp and FFN[0] in parts and FFN[1] in parts:
        block.ffn = w4a4.PackedW4A4GeluMLP(parts[FFN[0]], parts[FFN[1]])
    for name, child in list(block.named_modules()):
        if isinstance(child, torch.nn.Linear) and name in parts:
            parent, _, attr = name.rpartition(".")
            setattr(block.get_submodule(parent) if parent else block, attr, w4a4.PackedW4A4Linear(**parts[name]))
    return block


def convert(block: torch.nn.Module, index: int = 0, amax: dict | None = None, alpha: float = 0.5, rank: int = 32,
            fused: bool = False, keep=()) -> torch.nn.Module:
    """`block` (on the GPU) in W4A4, in place: the layers of layer_parts installed (w4a4.py:355-357)."""
    return install(block, layer_parts(block, index, amax, alpha, rank, fused, keep), gelu_mlp=fused)


def quantized_block(block: torch.nn.Module, heads: int, index: int = 0, amax: dict | None = None,
                    alpha: float = 0.5, rank: int = 32, hessians: dict | None = None, rule: str = "max",
                    scale_dtype=torch.bfloat16, device="cuda", parts: dict | None = None):
    """The fused QuantizedWanBlock of a float block: its eight W4A4 layers (layer_parts, fused; or `parts`, made by
    it before) plus the Q/K RMSNorm weights (bf16), norm3's affine (fp32) and the modulation (fp32 [6, dim])."""
    from wdl.block import QuantizedWanBlock

    if parts is None:
        parts = layer_parts(block, index, amax, alpha, rank, True, (), hessians, rule, scale_dtype, device)
    missing = set(BLOCK_LINEARS) - set(parts)
    if missing:
        raise ValueError(f"the block has no linears {sorted(missing)}")
    P = {BLOCK_LINEARS[name]: t for name, t in parts.items() if name in BLOCK_LINEARS}
    get = lambda t, dtype: t.detach().to(device, dtype).contiguous()
    P["wq"], P["wk"] = get(block.self_attn.norm_q.weight, torch.bfloat16), get(block.self_attn.norm_k.weight,
                                                                                torch.bfloat16)
    P["cwq"], P["cwk"] = get(block.cross_attn.norm_q.weight, torch.bfloat16), get(block.cross_attn.norm_k.weight,
                                                                                  torch.bfloat16)
    dim = P["wq"].shape[0]
    n3w, n3b = block.norm3.weight, block.norm3.bias
    P["n3w"] = get(n3w, torch.float32) if n3w is not None else torch.ones(dim, device=device)
    P["n3b"] = get(n3b, torch.float32) if n3b is not None else torch.zeros(dim, device=device)
    P["modulation"] = get(block.modulation, torch.float32).reshape(6, dim)
    return QuantizedWanBlock(P, dim, heads)


def input_amax(model: torch.nn.Module, run, prefix_of=None) -> dict:
    """The calibration maxima of every nn.Linear of `model` while run() executes: {"<block>.<linear>": fp32 [in]}
    (the largest |x| of each input channel over all calls). prefix_of(name) -> (block index, linear name within
    the block), by default blocks.<i>.<rest> -> (i, rest) and any other name -> (0, name)."""
    def split(name):
        parts = name.split(".")
        if len(parts) > 2 and parts[0] == "blocks" and parts[1].isdigit():
            return int(parts[1]), ".".join(parts[2:])
        return 0, name

    prefix_of = prefix_of or split
    seen: dict = {}
    hooks = []
    for name, m in model.named_modules():
        if isinstance(m, torch.nn.Linear):
            i, rest = prefix_of(name)
            key = f"{i}.{rest}"

            def hook(module, args, key=key):
                x = args[0].detach()
                a = x.reshape(-1, x.shape[-1]).abs().amax(0).float()
                seen[key] = a if key not in seen else torch.maximum(seen[key], a)

            hooks.append(m.register_forward_pre_hook(hook))
    try:
        with torch.no_grad():
            run()
    finally:
        for h in hooks:
            h.remove()
    return seen
