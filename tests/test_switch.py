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


def test_frame_history_keeps_the_sink_and_the_newest():
    """Stream.next_chunk's latent history (causal.py:535-536, 744-746): the first `sink` frames of the video stay,
    then the newest `ring` others; chunks() regroups them and refuses frames that are not whole chunks."""
    from wdl.model import FrameHistory

    def run(sink, ring, chunks):
        h = FrameHistory(sink, ring)
        for i in range(chunks):
            h.add(3 * i, torch.full((1, 3, 2, 2), float(i)).add(torch.arange(3.0).view(1, 3, 1, 1) / 10))
        return h

    h = run(0, 15, 10)
    assert [f for f, _ in h.chunks(3)] == [15, 18, 21, 24, 27]
    h = run(6, 9, 10)
    assert [f for f, _ in h.chunks(3)] == [0, 3, 21, 24, 27]
    first, x = h.chunks(3)[2]
    assert torch.equal(x[0, :, 0, 0], torch.tensor([7.0, 7.1, 7.2]))  # chunk 7, frames in order
    assert [f for f, _ in run(6, 0, 10).chunks(3)] == [0, 3]
    h = run(1, 17, 10)  # a sink of one frame: kept, but not whole chunks
    assert [n for n, _ in h.sink] == [0] and [n for n, _ in h.recent] == list(range(13, 30))
    with pytest.raises(ValueError):
        h.chunks(3)


class _Cache:
    def __init__(self, max_tokens, sink_tokens):
        self.max_tokens, self.sink_tokens, self.entropy_ratio, self.commits = max_tokens, sink_tokens, None, 0

    def commit(self):
        self.commits += 1


class _PointMass:
    """A model whose data distribution is the single latent x*: the exact flow of x = (1 - s) x* + s eps is
    eps - x* = (x - x*) / s; the noise a level was given is (x - (1 - s) x*) / s."""

    def __init__(self, x_star, caches):
        self.x_star, self.caches, self.freq, self.seen = x_star, caches, torch.zeros(1), []

    def forward(self, x, t, start_frame=0):
        s = float(t[0]) / 1000
        self.seen.append((s, x.clone(), start_frame))
        return torch.zeros_like(x) if s == 0 else (x - self.x_star) / s


def _check_point_mass(x0, seen, x_star, noises, levels):
    assert float((x0 - x_star).abs().max()) <= 1e-5
    assert [s for s, _, _ in seen] == pytest.approx(list(levels) + [0.0], abs=1e-6)  # t is fp32
    for (s, x, _), eps in zip(seen, noises):  # each level's input is x* noised with that level's noise
        assert float(((x - (1 - s) * x_star) / s - eps).abs().max()) <= 1e-5
    assert float((seen[-1][1] - x_star).abs().max()) <= 1e-5  # the write pass encodes the clean chunk


def test_dmd_loop_returns_the_point_mass():
    """The DMD loop (causal.py:711-718) on a point-mass model returns x* (x0 = x - sigma flow with sigma = t / 1000),
    feeds level 0 the given noise and level i its fresh noise at sigma_i, and writes x* at t = 0: the oracle's loop
    and wdl's ChunkStream. A renoising mistake (wrong level, wrong weight) fails the per-level noise check."""
    from oracle import model as omodel
    from wdl.model import ChunkStream, sigmas

    g = torch.Generator().manual_seed(4)
    shape = (4, 3, 4, 6)
    x_star, noise = torch.randn(shape, generator=g), torch.randn(shape, generator=g)
    fresh = [torch.randn(shape, generator=g) for _ in range(3)]
    levels = sigmas()
    pm = _PointMass(x_star, [])
    x0 = omodel.next_chunk(noise, fresh, None, [], [], [], None, 0, 2, flow=lambda x, t: pm.forward(x, t))
    _check_point_mass(x0, pm.seen, x_star, [noise] + fresh, levels)

    caches = [_Cache(18 * 6, 0), _Cache(18 * 6, 0)]
    pm = _PointMass(x_star, caches)
    stream = ChunkStream(pm, shape, torch.Generator().manual_seed(9))
    replay = torch.Generator().manual_seed(9)
    x0 = stream.next_chunk(noise)
    _check_point_mass(x0, pm.seen, x_star, [noise] + [torch.randn(shape, generator=replay) for _ in range(3)],
                      levels)
    assert [c.commits for c in caches] == [1, 1] and stream.start == 3


def test_chunk_stream_with_a_one_frame_sink():
    """Any sink the reference's Stream accepts (sink_frames <= window - 2 chunks, causal.py:481) streams; only the
    resolution switch, which re-encodes whole chunks, refuses a sink that is not one, before changing anything."""
    from wdl.model import ChunkStream

    shape = (4, 3, 4, 4)  # 4 tokens per frame
    caches = [_Cache(18 * 4, 1 * 4)]
    pm = _PointMass(torch.zeros(shape), caches)
    stream = ChunkStream(pm, shape, torch.Generator().manual_seed(1))
    for _ in range(8):
        stream.next_chunk()
    assert stream.start == 24 and caches[0].commits == 8
    assert [n for n, _ in stream.history.sink] == [0]
    assert [n for n, _ in stream.history.recent] == list(range(7, 24))
    with pytest.raises(ValueError):
        stream.switch_resolution(6, 6)
    assert stream.shape == shape and stream.model.caches[0] is caches[0]
