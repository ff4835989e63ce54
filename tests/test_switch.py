"""The mid-stream resolution switch on the CPU: the oracle's resampling pinned against torch's antialiased
bilinear interpolation (a library routine) and by its identities, the product's resample_latents against it, and
the window bookkeeping of the chunks a cache holds (the GPU test of the switch itself is in test_model_gpu.py)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import model as omodel


@pytest.mark.parametrize("H,W,h,w", [(44, 80, 32, 58), (32, 58, 44, 80), (8, 16, 12, 8), (10, 6, 5, 3)])
def test_oracle_resample_is_antialiased_bilinear(H, W, h, w):
    g = torch.Generator().manual_seed(H * W + h)
    x = torch.randn(3, 2, H, W, generator=g)
    want = F.interpolate(x.permute(1, 0, 2, 3), size=(h, w), mode="bilinear", align_corners=False,
                         antialias=True).permute(1, 0, 2, 3)
    got = omodel.resample(x, h, w)
    assert got.shape == (3, 2, h, w)
    assert float((got - want).abs().max()) <= 2e-5 * float(x.abs().max())


def test_oracle_resample_identities():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 3, 6, 10, generator=g)
    assert torch.equal(omodel.resample(x, 6, 10), x)  # same size: every row of taps is one 1
    c = torch.full((1, 1, 44, 80), -1.75)
    assert float((omodel.resample(c, 32, 58) + 1.75).abs().max()) < 1e-6  # taps sum to one
    # a planted mistake (taps not renormalised at the frame's edges) fails the torch check
    taps = omodel._taps

    def unnormalised(n_in, n_out):
        t = taps(n_in, n_out)
        t[0] *= 0.9
        return t

    omodel._taps = unnormalised
    try:
        bad = omodel.resample(x, 4, 7)
    finally:
        omodel._taps = taps
    want = F.interpolate(x.permute(1, 0, 2, 3), size=(4, 7), mode="bilinear", align_corners=False,
                         antialias=True).permute(1, 0, 2, 3)
    assert float((bad - want).abs().max()) > 1e-3


def test_product_resample_matches_the_oracle():
    from wdl.model import resample_latents

    g = torch.Generator().manual_seed(2)
    x = torch.randn(48, 3, 44, 80, generator=g)
    got = resample_latents(x, 32, 58)
    assert float((got - omodel.resample(x, 32, 58)).abs().max()) <= 2e-5 * float(x.abs().max())


def test_window_chunks_keeps_the_sink_and_the_newest():
    from wdl.model import window_chunks

    kept = [(3 * i, i) for i in range(10)]  # ten committed 3-frame chunks
    assert window_chunks(kept[:4], 3, 18, 0) == kept[:4]
    assert window_chunks(kept, 3, 18, 0) == kept[4:]
    assert window_chunks(kept, 3, 18, 6) == kept[:2] + kept[6:]
    assert window_chunks(kept, 3, 6, 6) == kept[:2]
    with pytest.raises(ValueError):
        window_chunks(kept, 3, 20, 0)
    with pytest.raises(ValueError):
        window_chunks(kept, 3, 18, 4)
