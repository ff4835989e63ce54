"""Blocks loaded from a weight pack (wdl.pack.load_blocks) run bit-identically to the blocks the pack was made from
(dim 256, 2 x 128 heads, FFN 1024, SVD-quantized, over an FP8 cache and a prompt)."""

import pytest
import torch

from oracle import block as oblock
from oracle import rope as orope

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def test_packed_blocks_run_bit_identically(gpu, tmp_path):
    from wdl import pack
    from wdl.block import build_block
    from wdl.kvcache import KVCache

    g = torch.Generator().manual_seed(5)
    dev = torch.device("cuda")
    blocks = [build_block(oblock.quantize_block(oblock.random_block(256, 1024, g)), 256, 2, dev) for _ in range(2)]
    pack.build_pack([b.p for b in blocks], tmp_path / "w.pack", source="seed 5")
    loaded = pack.load_blocks(tmp_path / "w.pack", 2, dev, source="seed 5", verify=True)
    grid, M = (2, 4, 6), 48
    X = torch.randn(M, 256, generator=g).to(BF).to(dev)
    C = torch.randn(16, 256, generator=g).to(BF).to(dev)
    freq = orope.freqs(128, 1024, torch.float64).float().to(dev)
    time_in = (torch.randn(6, 256, generator=g) * 0.1).to(dev)
    outs = []
    for chain in (blocks, loaded):
        x = X.clone()
        for b in chain:
            cache = KVCache(0, 0, chunk=grid[0])
            x = b.forward(x, time_in + b.p["modulation"], grid, freq, 0, cache, b.prepare_context(C))
        outs.append(x.cpu())
    assert torch.equal(outs[0], outs[1])


def test_packed_mixed_precision_blocks_run_bit_identically(gpu, tmp_path):
    """The mixed-precision mode (FP8 weight-only attention projections, W4A4 feed-forward) through
    block_mixed_v1_gfx950: the loaded blocks compute bit-identically to the blocks packed."""
    from wdl import pack
    from wdl.block import build_block
    from wdl.kvcache import KVCache

    g = torch.Generator().manual_seed(8)
    dev = torch.device("cuda")
    blocks = [build_block(oblock.mixed_precision_block(256, 1024, g), 256, 2, dev) for _ in range(2)]
    info = pack.build_pack([b.p for b in blocks], tmp_path / "m.pack", source="seed 8")
    assert info["format"] == pack.FORMAT_MIXED
    loaded = pack.load_blocks(tmp_path / "m.pack", 2, dev, source="seed 8", verify=True)
    assert all("fp8" in b.p["qkv"] and "wcodes" in b.p["ffn1"] for b in loaded)
    grid, M = (2, 4, 6), 48
    X = torch.randn(M, 256, generator=g).to(BF).to(dev)
    C = torch.randn(16, 256, generator=g).to(BF).to(dev)
    freq = orope.freqs(128, 1024, torch.float64).float().to(dev)
    time_in = (torch.randn(6, 256, generator=g) * 0.1).to(dev)
    outs = []
    for chain in (blocks, loaded):
        x = X.clone()
        for b in chain:
            cache = KVCache(0, 0, chunk=grid[0])
            x = b.forward(x, time_in + b.p["modulation"], grid, freq, 0, cache, b.prepare_context(C))
        outs.append(x.cpu())
    assert torch.equal(outs[0], outs[1])
