"""The Sage oracle on the CPU: the mean-smoothing identity, the V layout maps, the quantizers against brute force,
and the attention emulation against exact attention on dequantized operands."""

import torch

from oracle import sage as osage


def test_mean_smoothing_changes_nothing_exactly():
    """softmax(q (k - mu)^T) == softmax(q k^T): the identity that makes Sage's K smoothing exact (float64)."""
    g = torch.Generator().manual_seed(0)
    q, k = torch.randn(5, 16, dtype=torch.float64, generator=g), torch.randn(9, 16, dtype=torch.float64, generator=g)
    mu = k.mean(0)
    assert torch.allclose(torch.softmax(q @ k.t(), -1), torch.softmax(q @ (k - mu).t(), -1), atol=1e-14)


def test_v_layouts_are_permutations():
    pos = osage.wdl_v_position(torch.arange(64))
    assert sorted(pos.tolist()) == list(range(64))
    assert torch.equal(osage.wdl_v_position(torch.arange(64, 128)), pos + 64)
    # the reference's 16-token order [0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15] (sage_kv.py:93)
    v = torch.arange(16, dtype=torch.float32).reshape(1, 16, 1, 1).expand(1, 16, 1, 1) / 16
    codes = osage.sage_v_layout(v.to(torch.float8_e4m3fn))[0, 0, 0].float() * 16
    assert codes[:16].round().tolist() == [0, 1, 8, 9, 2, 3, 10, 11, 4, 5, 12, 13, 6, 7, 14, 15]


def test_quantizers_round_half_away_within_one_step():
    g = torch.Generator().manual_seed(1)
    Q = torch.randn(1, 70, 2, 128, generator=g) * 4
    q, qs = osage.quant_q(Q)
    s = osage.expand_q_scale(qs, 70)[..., None]
    y = Q / s
    assert torch.all((y - q.float()).abs() <= 0.5 + 1e-6)
    assert int(q.abs().max()) <= 127
    # every group of 4 tokens (l, l+8, l+16, l+24) of a 32-block holds a value of magnitude 127
    assert int(q[0, :64].abs().reshape(2, 4, 8, 2, 128).amax(dim=(1, 4)).min()) == 127
    K = torch.randn(1, 130, 2, 128, generator=g) + 2
    mean = K.mean(1)
    k, ks = osage.quant_k(K, mean)
    s = osage.expand_k_scale(ks, 130)[..., None]
    assert torch.all(((K - mean[:, None]) / s - k.float()).abs() <= 0.5 + 1e-5)


def test_attention_emulation_close_to_exact():
    g = torch.Generator().manual_seed(2)
    Q = torch.randn(1, 40, 2, 128, generator=g).to(torch.bfloat16)
    cache = (torch.randn(1, 90, 2, 128, generator=g) + 0.5).to(torch.float8_e4m3fn)
    V = torch.randn(1, 40, 2, 128, generator=g).to(torch.bfloat16)
    one = torch.ones(1, 90, 2, 1)
    p = osage.prep(Q, cache, one, cache, one, 50, Q, V)
    exact = osage.attention_exact(Q, p["K"], p["V"])
    assert osage.rel_err(osage.attention_quantized(p, 128 ** -0.5), exact) < 0.05
    assert osage.rel_err(osage.attention_quantized(p, 128 ** -0.5, p_fp8=True), exact) < 0.06


def test_online_softmax_restatement_equals_exact_softmax():
    """attention_online (the kernel's blockwise arithmetic) with P kept in fp32 equals the float64 softmax of the
    same quantized operands (fp32 rounding only), for a key count that is not a multiple of the 64-key block; with
    P rounded to e4m3 it sits at the fp8-P emulation's error against exact attention."""
    g = torch.Generator().manual_seed(3)
    Q = torch.randn(1, 48, 2, 128, generator=g).to(torch.bfloat16)
    cache = (torch.randn(1, 150, 2, 128, generator=g) * 2).to(torch.float8_e4m3fn)
    V = torch.randn(1, 48, 2, 128, generator=g).to(torch.bfloat16)
    one = torch.ones(1, 150, 2, 1) * 0.5
    p = osage.prep(Q, cache, one, cache, one, 102, Q * 0.7, V)
    ref = osage.attention_quantized(p, 128 ** -0.5)
    assert osage.rel_err(osage.attention_online(p, 128 ** -0.5, round_p=False), ref) < 1e-5
    exact = osage.attention_exact(Q, p["K"], p["V"])
    e_fp8 = osage.rel_err(osage.attention_quantized(p, 128 ** -0.5, p_fp8=True), exact)
    assert osage.rel_err(osage.attention_online(p, 128 ** -0.5), exact) <= 1.2 * e_fp8 + 1e-3


def test_exact_attention_and_cross_attention_are_sdpa():
    """attention_exact (and the block's cross-attention built on it) against torch's scaled_dot_product_attention in
    float64, an independent library routine; a transposed V or a missing scale would fail."""
    from oracle import block as oblock

    g = torch.Generator().manual_seed(4)
    Q = torch.randn(1, 21, 3, 128, generator=g).to(torch.bfloat16)
    K = torch.randn(1, 37, 3, 128, generator=g).to(torch.bfloat16)
    V = torch.randn(1, 37, 3, 128, generator=g).to(torch.bfloat16)
    want = torch.nn.functional.scaled_dot_product_attention(
        *(t.double().transpose(1, 2) for t in (Q, K, V))).transpose(1, 2)
    assert (osage.attention_exact(Q, K.float(), V.float()).double() - want).abs().max() < 1e-6
    got = oblock.cross_attention(Q.reshape(21, 384), K.reshape(37, 384), V.reshape(37, 384), 3)
    assert torch.equal(got, want.reshape(21, 384).float().to(torch.bfloat16))


def test_mapped_gather_is_the_explicit_index_loop():
    """gather with the heads / tokens maps of sage_kv.attend: output (t, h) is cache row tokens[t], head heads[h],
    times its scale, for t < at; then the chunk."""
    g = torch.Generator().manual_seed(5)
    cache = torch.randn(1, 12, 5, 4, generator=g).to(torch.float8_e4m3fn)
    scale = torch.rand(1, 12, 5, 1, generator=g)
    chunk = torch.randn(1, 3, 2, 4, generator=g)
    heads, tokens = torch.tensor([4, 1], dtype=torch.int32), torch.tensor([7, 0, 11, 2, 9], dtype=torch.int32)
    got = osage.gather(cache, scale, chunk, 4, heads, tokens)
    assert got.shape == (1, 7, 2, 4)
    for t in range(4):
        for h in range(2):
            r, c = int(tokens[t]), int(heads[h])
            assert torch.equal(got[0, t, h], cache[0, r, c].float() * scale[0, r, c, 0])
    assert torch.equal(got[0, 4:], chunk[0])


def test_lazy_reference_max_keeps_the_exact_softmax():
    """attention_online with P unrounded equals the exact softmax for every rescale threshold tau, on keys whose
    scores grow block after block (so the reference max has to move past the first block: the data is checked for
    that); with a dropped rescale or a wrong alpha the result would be off by far more than 1e-5."""
    g = torch.Generator().manual_seed(6)
    Q = torch.randn(1, 64, 1, 128, generator=g).to(torch.bfloat16)
    grow = torch.linspace(0.2, 3.0, 320).reshape(1, 320, 1, 1)
    K = (torch.randn(1, 320, 1, 128, generator=g) * grow + Q.float().mean(1, keepdim=True) * grow * 4)
    V = torch.randn(1, 320, 1, 128, generator=g).to(torch.bfloat16)
    z8 = torch.zeros(1, 1, 1, 128, dtype=torch.float8_e4m3fn)
    z = torch.ones(1, 1, 1, 1)
    p = osage.prep(Q, z8, z, z8, z, 0, K.to(torch.bfloat16), V)
    ref = osage.attention_quantized(p, 128 ** -0.5)
    y = torch.einsum("bnhd,blhd->bnl", Q.double(), K.double()) * 128 ** -0.5 * 1.4426950408889634
    bmax = y.reshape(1, 64, 5, 64).amax(-1)
    assert bool((bmax[..., 4] > bmax[..., 0] + 4).all())  # later blocks hold scores larger by more than 2^4
    for tau in (0.0, 2.0, 8.0):
        got = osage.attention_online(p, 128 ** -0.5, round_p=False, splits=1, tau=tau)
        assert osage.rel_err(got, ref) < 1e-5, tau
    # with P rounded to e4m3 the lazy max costs nothing measurable against exact attention
    exact = osage.attention_exact(Q, p["K"], p["V"])
    e0 = osage.rel_err(osage.attention_online(p, 128 ** -0.5, tau=0.0), exact)
    assert osage.rel_err(osage.attention_online(p, 128 ** -0.5, tau=2.0), exact) <= 1.2 * e0 + 1e-3


def test_frame_mask_is_each_query_over_its_own_keys():
    """The block-causal per-frame mask: each chunk query's output equals exact attention over the keys it sees
    (the cache and the chunk's frames up to its own), computed by slicing; frame 0 is no mask."""
    g = torch.Generator().manual_seed(7)
    n, at, F = 12, 10, 5  # a chunk of 12 queries in frames of 5 (the last frame partial) over 10 cached keys
    Q = torch.randn(1, n, 2, 128, generator=g, dtype=torch.float64)
    K = torch.randn(1, at + n, 2, 128, generator=g, dtype=torch.float64)
    V = torch.randn(1, at + n, 2, 128, generator=g, dtype=torch.float64)
    got = osage.attention_exact(Q, K, V, frame=F)
    for q in range(n):
        seen = min(at + (q // F + 1) * F, at + n)
        want = osage.attention_exact(Q[:, q:q + 1], K[:, :seen], V[:, :seen])
        assert torch.allclose(got[:, q:q + 1], want, atol=1e-6, rtol=0)
    assert torch.equal(osage.attention_exact(Q, K, V, frame=0), osage.attention_exact(Q, K, V))
    m = osage.frame_mask(n, at + n, F)
    assert m.sum(1).tolist() == [15] * 5 + [20] * 5 + [22] * 2
