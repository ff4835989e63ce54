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
