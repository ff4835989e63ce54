"""Whole-block conversion on the MI355X (wdl.convert.quantized_block / convert, quantization/w4a4.py:265-357): a float
block (dim 256, 2 heads, FFN 1024) with calibrated smoothing becomes
- a QuantizedWanBlock whose forward is bit-identical to build_block on the same layers' parts (the wiring of every
  layer, norm and the modulation into the fused block), and whose update stays within the reference's W4A4 contract
  of the float block (tests/test_w4a4.py:62-87: relative error below 0.21 with Sage attention);
- the float module itself with wdl's modules installed (FusedQKVAttention without a cache runs the bf16 attention,
  PackedW4A4Linear in cross-attention, PackedW4A4GeluMLP), its update within the same contract."""

import pytest
import torch

from float_block import FloatWanBlock
from oracle import block as oblock
from oracle import rope as orope

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def test_converted_block_matches_build_block_and_the_float_block(gpu):
    from wdl import convert, w4a4
    from wdl.block import LINEARS, build_block
    from wdl.kvcache import KVCache

    dim, heads, ffn, grid = 256, 2, 1024, (2, 4, 6)
    g = torch.Generator().manual_seed(4)
    B = oblock.random_block(dim, ffn, g, init="torch")
    fb = FloatWanBlock.from_random_block(B, dim, ffn, heads).cuda()
    M = grid[0] * grid[1] * grid[2]
    X = torch.randn(1, M, dim, generator=g).cuda()
    time_in = (torch.randn(1, 6, dim, generator=g) * 0.1).cuda()
    C = torch.randn(1, 16, dim, generator=g).cuda()
    freq = orope.freqs(128, 1024, torch.float64).float().cuda()
    with torch.no_grad():
        ref = fb(X, time_in, [grid], freq, context=C)
    amax = convert.input_amax(fb, lambda: fb(X, time_in, [grid], freq, context=C))
    assert "0.self_attn.q" in amax and "0.ffn.2" in amax
    parts = convert.layer_parts(fb, 0, amax, fused=True, device="cuda")
    qb = convert.quantized_block(fb, heads, parts={n: dict(t) for n, t in parts.items()})
    # the same layers through build_block: the logical parts of each packed layer, then packed again
    P = {convert.BLOCK_LINEARS[n]: w4a4.unpack_parts(t) for n, t in parts.items()}
    for k, src in (("wq", fb.self_attn.norm_q), ("wk", fb.self_attn.norm_k), ("cwq", fb.cross_attn.norm_q),
                   ("cwk", fb.cross_attn.norm_k)):
        P[k] = src.weight.detach().cpu().to(BF)
    P["n3w"], P["n3b"] = fb.norm3.weight.detach().cpu(), fb.norm3.bias.detach().cpu()
    P["modulation"] = fb.modulation.detach().cpu().reshape(6, dim)
    bb = build_block(P, dim, heads, torch.device("cuda"))
    Xb = X[0].to(BF)
    outs = []
    for blk in (qb, bb):
        cache = KVCache(0, 0, chunk=grid[0])
        e = (time_in[0] + blk.p["modulation"]).float()
        outs.append(blk.forward(Xb.clone(), e, grid, freq, 0, cache, blk.prepare_context(C[0].to(BF))).float())
    assert torch.equal(outs[0], outs[1])
    upd, rupd = outs[0] - X[0], ref[0].float() - X[0]
    err = float((upd - rupd).norm() / rupd.norm())
    print(f"quantized_block vs float block: update rel err {err:.3f}")
    assert err < 0.21
    # the float module with wdl's modules installed (no cache: bf16 attention over the chunk)
    convert.convert(fb, 0, amax, fused=True)
    assert isinstance(fb.self_attn, w4a4.FusedQKVAttention) and isinstance(fb.ffn, w4a4.PackedW4A4GeluMLP)
    assert isinstance(fb.cross_attn.q, w4a4.PackedW4A4Linear)
    with torch.no_grad():
        got = fb(X.to(BF), time_in, [grid], freq, context=C.to(BF))
    err2 = float(((got.float() - X) - (ref.float() - X)).norm() / (ref.float() - X).norm())
    print(f"converted module vs float block: update rel err {err2:.3f}")
    assert err2 < 0.21
