"""Pins of the RoPE oracle (oracle/rope.py) and of the attention scale rule, on the CPU.

- rope_apply (the real-arithmetic form of src/wan_dit_lab/models/rope.py:26-31) against the fp64 complex-phase
  oracle of tests/test_rope_triton.py:21-45, restated as rope_complex: a swapped sine sign, a transposed pair or a
  wrong axis split fails it;
- the identities of tests/test_rope_triton.py:89-104: norm preservation, chunk offsets (a grid split into frames
  with start_frame + i equals the whole grid), relative positions (shifting both start frames leaves q . k);
- the tables against the closed form angle = pos * 10000^(-2i/dim) evaluated with math.cos / math.sin;
- the axis split [22, 21, 21] of a 128-dim head (tests/test_kv_cache.py:12);
- tokens past f h w pass through unchanged (kernels/rope_triton.py:54-56);
- KVCache.scale's known answers (tests/test_resolution_adaptation.py:16-21) and rope_at's
  (tests/test_resolution_adaptation.py:36-40), the latter on wdl's host tables (wdl.rope).
"""

import math

import torch

from oracle import rope as orope
from oracle import sage as osage


def frequencies(dim=128, positions=64):
    return orope.freqs(dim, positions, torch.float64)


def test_axis_split_of_a_128_dim_head():
    assert orope.axis_split(128) == [22, 21, 21]
    assert orope.axis_split(12) == [2, 2, 2]
    assert orope.axis_split(6) == [1, 1, 1]


def test_tables_are_the_closed_form():
    t = orope.rope(50, 44)
    for pos in (0, 1, 7, 49):
        for i in (0, 5, 21):
            a = pos * 10000 ** (-2 * i / 44)
            assert math.isclose(float(t[0, pos, i]), math.cos(a), rel_tol=0, abs_tol=1e-15)
            assert math.isclose(float(t[1, pos, i]), math.sin(a), rel_tol=0, abs_tol=1e-15)


def test_real_form_equals_complex_phase_oracle():
    g = torch.Generator().manual_seed(3)
    for dim, grid, start in ((128, (2, 3, 5), 7), (12, (1, 3, 5), 11), (6, (3, 2, 2), 0)):
        x = torch.randn(1, grid[0] * grid[1] * grid[2] + 4, 3, dim, generator=g, dtype=torch.float64)
        freq = frequencies(dim)
        a = orope.rope_apply(x, grid, freq, start)
        b = orope.rope_complex(x, grid, freq, start)
        torch.testing.assert_close(a, b, rtol=0, atol=1e-15)
        n = grid[0] * grid[1] * grid[2]
        assert torch.equal(a[:, n:], x[:, n:])


def test_a_planted_sign_error_is_caught():
    """The complex oracle is independent enough: a rotation by -angle (sine sign flipped) does not pass."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, 30, 2, 12, generator=g, dtype=torch.float64)
    freq = frequencies(12)
    flipped = torch.stack((freq[0], -freq[1]))
    assert not torch.allclose(orope.rope_apply(x, (2, 3, 5), flipped, 1), orope.rope_complex(x, (2, 3, 5), freq, 1))


def test_norm_chunk_offset_and_relative_position_identities():
    g = torch.Generator().manual_seed(5)
    freq = frequencies(12)
    x = torch.randn(1, 12, 2, 12, generator=g, dtype=torch.float64)
    grid = (3, 2, 2)
    rotated = orope.rope_apply(x, grid, freq, 5)
    torch.testing.assert_close(rotated.square().sum(-1), x.square().sum(-1), rtol=2e-14, atol=2e-14)
    chunks = torch.cat([orope.rope_apply(x[:, i * 4:(i + 1) * 4], (1, 2, 2), freq, 5 + i) for i in range(3)], dim=1)
    torch.testing.assert_close(rotated, chunks, rtol=0, atol=0)
    q = torch.randn(x.shape, generator=g, dtype=torch.float64)
    dot = lambda a, b: (a * b).sum(-1)
    before = dot(orope.rope_apply(x, grid, freq, 2), orope.rope_apply(q, grid, freq, 7))
    after = dot(orope.rope_apply(x, grid, freq, 9), orope.rope_apply(q, grid, freq, 14))
    torch.testing.assert_close(before, after, rtol=2e-13, atol=2e-13)


def test_positions_follow_the_grid():
    p = orope.positions((2, 3, 4), start_frame=5)
    assert p.shape == (24, 3)
    assert p[0].tolist() == [5, 0, 0] and p[5].tolist() == [5, 1, 1] and p[23].tolist() == [6, 2, 3]


def test_attention_scale_known_answers():
    assert math.isclose(osage.entropy_scale(1000, 128, 1.0), 128 ** -0.5, rel_tol=1e-12)
    smaller, larger = osage.entropy_scale(12480, 128, 2.256), osage.entropy_scale(12480, 128, 0.5)
    assert smaller < 128 ** -0.5 < larger
    assert math.isclose(smaller * 128 ** 0.5, math.sqrt(math.log(12480) / math.log(12480 * 2.256)))
    assert osage.entropy_scale(400, 128, None) is None


def test_host_rope_tables_and_rope_at_known_answers():
    from wdl import rope as wrope

    assert torch.equal(wrope.rope(1024, 42), orope.rope(1024, 42))
    assert torch.equal(wrope.rope_at(1024, 42, 1.0), wrope.rope(1024, 42))
    assert torch.allclose(wrope.rope_at(64, 42, 1.5)[:, 2], wrope.rope(64, 42)[:, 3])
    assert torch.equal(wrope.freqs(128, 64), frequencies(128, 64).float())


def test_general_rotation_equals_the_complex_oracle_per_sample():
    """rope_rotate (the op's general form: per-sample grids, padding, any dim) against the fp64 complex-phase
    oracle of the reference's tests (test_rope_triton.py:21-45) on fp64 inputs: equal to the last bit, since both
    compute e c - o s, o c + e s in fp64."""
    g = torch.Generator().manual_seed(3)
    for dim in (2, 6, 12, 128):
        freq = orope.freqs(dim, 64)
        x = torch.randn(2, 33, 3, dim, generator=g, dtype=torch.float64)
        grids = ((2, 3, 5), (1, 2, 4))
        got = orope.rope_rotate(x, grids, freq, 3)
        for b, grid in enumerate(grids):
            assert torch.equal(got[b:b + 1], orope.rope_complex(x[b:b + 1], grid, freq, 3))


def test_inverse_undoes_the_rotation_and_half_outputs_round_through_fp32():
    g = torch.Generator().manual_seed(4)
    freq = orope.freqs(128, 64)
    x = torch.randn(1, 30, 2, 128, generator=g, dtype=torch.float64)
    back = orope.rope_rotate(orope.rope_rotate(x, ((2, 3, 5),), freq, 7), ((2, 3, 5),), freq, 7, inverse=True)
    assert float((back - x).abs().max()) < 1e-14
    fwd = orope.rope_rotate(x, ((2, 3, 5),), freq, 7)
    assert not torch.equal(orope.rope_rotate(x, ((2, 3, 5),), freq, 7, inverse=True), fwd)
    half = orope.rope_rotate(x, ((2, 3, 5),), freq, 7, out_dtype=torch.bfloat16)
    assert torch.equal(half, fwd.float().to(torch.bfloat16))
    # fp32 inputs with fp32 tables: fp32 products, each rounded
    x32, f32 = x.float(), freq.float()
    r32 = orope.rope_rotate(x32, ((2, 3, 5),), f32, 7)
    e, o = x32[0, :30, :, 0::2], x32[0, :30, :, 1::2]
    pos = orope.positions((2, 3, 5), 7)
    t, s, _ = orope.axis_split(128)
    col = torch.cat([pos[:, :1].expand(30, t), pos[:, 1:2].expand(30, s), pos[:, 2:3].expand(30, s)], 1)
    c = f32[0][col, torch.arange(64)][:, None]
    sn = f32[1][col, torch.arange(64)][:, None]
    assert torch.equal(r32[0, :, :, 0::2], e * c - o * sn) and torch.equal(r32[0, :, :, 1::2], o * c + e * sn)
