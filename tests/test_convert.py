"""Whole-block conversion (wdl.convert: layers, layer_parts, input_amax; quantization/w4a4.py:265-357) on the CPU:
the layer grouping of the reference (fused q|k|v stacked by output, the feed-forward pair, kept linears), each layer's
parts equal to wdl.w4a4.quantize of the stacked weight with the calibrated smoothing (the feed-forward's second
layer for GELU's shifted output), and the calibration maxima equal to the inputs' own."""

import torch

from oracle import block as oblock
from float_block import FloatWanBlock
from wdl import convert, w4a4


def _block(seed=0, dim=128, ffn=256, heads=1):
    g = torch.Generator().manual_seed(seed)
    return FloatWanBlock.from_random_block(oblock.random_block(dim, ffn, g), dim, ffn, heads), g


def test_layer_grouping():
    blk, _ = _block()
    plain = convert.layers(blk)
    assert sorted(plain) == sorted(["self_attn.q", "self_attn.k", "self_attn.v", "self_attn.o", "cross_attn.q",
                                    "cross_attn.k", "cross_attn.v", "cross_attn.o", "ffn.0", "ffn.2"])
    fused = convert.layers(blk, fused=True, keep=("cross_attn.k",))
    assert [n for n, _ in fused["self_attn.qkv"]] == list(convert.QKV)
    assert "cross_attn.k" not in fused and "self_attn.q" not in fused


def test_layer_parts_are_quantize_of_the_stacked_weights_with_calibrated_smoothing():
    blk, g = _block(1)
    dim = 128
    x = torch.randn(2, 24, dim, generator=g)
    amax = convert.input_amax(blk, lambda: blk.ffn(x))
    assert torch.equal(amax["0.ffn.0"], x.reshape(-1, dim).abs().amax(0))
    h = torch.nn.functional.gelu(blk.ffn[0](x), approximate="tanh")
    assert torch.allclose(amax["0.ffn.2"], h.reshape(-1, h.shape[-1]).abs().amax(0))
    amax["0.self_attn.q"] = torch.rand(dim, generator=g) * 5 + 0.1
    parts = convert.layer_parts(blk, 0, amax, fused=True)
    W = torch.cat([blk.self_attn.q.weight, blk.self_attn.k.weight, blk.self_attn.v.weight]).float()
    b = torch.cat([blk.self_attn.q.bias, blk.self_attn.k.bias, blk.self_attn.v.bias]).float()
    want = w4a4.quantize(W, b, smooth=w4a4.smoothing(amax["0.self_attn.q"], W))
    for p in w4a4.PARTS:
        assert torch.equal(parts["self_attn.qkv"][p], want[p]), p
    W2 = blk.ffn[2].weight.float()
    want2 = w4a4.quantize(W2, blk.ffn[2].bias.float(), smooth=w4a4.smoothing(amax["0.ffn.2"] + w4a4.GELU_SHIFT, W2),
                          shift=w4a4.GELU_SHIFT)
    for p in w4a4.PARTS:
        assert torch.equal(parts["ffn.2"][p], want2[p]), p
    assert torch.equal(parts["cross_attn.o"]["smooth"], torch.ones(dim, dtype=torch.bfloat16))  # no maxima: s = 1
