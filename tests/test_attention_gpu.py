"""Q/K RMSNorm + RoPE, Sage preparation and Sage-style attention on the HIP path against the oracle.

Bars: norm + RoPE — bit-exact bf16 (the oracle's ordered-sum RMSNorm and the reference's fp32 rotation); int8 Q —
bit-exact values and scales; int8 K — bit-exact given the kernel's own K mean (the quantizer), within 1 LSB of the
oracle's float64 mean (the reference's own bar, tests/test_sage_kv.py:81); V — bit-exact e4m3 codes and scales;
attention — cosine >= 0.999 against the oracle's exact softmax over the same quantized operands, and relative error
against exact fp64 attention within 1.2x that of the quantized oracle + 1e-3 (tests/test_sage_kv.py:97)."""

import pytest
import torch

from oracle import norms as onorms
from oracle import rope as orope
from oracle import sage as osage

pytestmark = pytest.mark.gpu


def setup(at=200, n=150, nq=None, H=3, seed=0, kbias=None):
    g = torch.Generator().manual_seed(seed)
    nq = n if nq is None else nq
    total = at + n + 64
    k = (torch.randn(1, total, H, 128, generator=g) + 0.5)
    if kbias is not None:
        k = k + kbias
    k = k.to(torch.float8_e4m3fn)
    v = (torch.randn(1, total, H, 128, generator=g) * 0.7).to(torch.float8_e4m3fn)
    ks = torch.ones(1, total, H, 1)
    vs = torch.ones(1, total, H, 1)
    K = torch.randn(1, n, H, 128, generator=g) + 0.5
    if kbias is not None:
        K = K + kbias
    K = K.to(torch.bfloat16)
    V = torch.randn(1, n, H, 128, generator=g).to(torch.bfloat16)
    Q = torch.randn(1, nq, H, 128, generator=g).to(torch.bfloat16)
    return Q, k, ks, v, vs, at, K, V


def cuda(*ts):
    return [t.cuda() for t in ts]


@pytest.mark.parametrize("n,H", [(7, 2), (150, 3), (1392, 24), (2640, 2)])
def test_quant_q_bit_exact(gpu, n, H):
    from wdl import sage_kv

    Q = torch.randn(1, n, H, 128, generator=torch.Generator().manual_seed(n)).to(torch.bfloat16) * 3
    q, qs = sage_kv.quant_q(Q.cuda())
    torch.cuda.synchronize()
    rq, rqs = osage.quant_q(Q)
    assert torch.equal(q.cpu(), rq)
    assert torch.equal(qs.cpu(), rqs)


@pytest.mark.parametrize("at,n,H", [(200, 150, 3), (0, 130, 2), (928, 464, 24), (6600, 2640, 2)])
def test_sage_prep_k_and_v(gpu, at, n, H):
    from wdl import sage_kv

    kbias = torch.randn(1, 1, H, 128, generator=torch.Generator().manual_seed(5)) * 3
    Q, k, ks, v, vs, at, K, V = setup(at, n, H=H, seed=at + n, kbias=kbias)
    ks = ks * 0.5 + torch.rand(ks.shape, generator=torch.Generator().manual_seed(1))  # non-unit cache scales
    p = sage_kv.prep(*cuda(k, ks, v, vs), at, *cuda(K, V))
    torch.cuda.synchronize()
    L = at + n
    Lp = (L + 63) // 64 * 64
    Kf = osage.gather(k, ks, K, at)
    Vf = osage.gather(v, vs, V, at)
    ref_mean, ref_vscale = osage.colstats(Kf, Vf)
    gpu_mean = p["k_mean"].cpu()[None]
    assert float((gpu_mean - ref_mean).abs().max()) <= 1e-5 * float(ref_mean.abs().max()) + 1e-6
    assert torch.equal(p["v_scale"].cpu()[None], ref_vscale)  # a max: exact
    # the K quantizer, given the kernel's mean: bit-exact values and scales
    qk, qks = osage.quant_k(Kf, gpu_mean)
    got_k = p["k"].cpu().permute(1, 0, 2)[:L][None]  # [1, L, H, 128]
    assert torch.equal(got_k, qk)
    assert torch.equal(p["k_scale"].cpu()[None], qks)
    assert torch.all(p["k"].cpu()[:, L:] == 0)
    # against the oracle's float64 mean: within 1 LSB (reference tests/test_sage_kv.py:81)
    qk64, qks64 = osage.quant_k(Kf, ref_mean)
    assert int((got_k.int() - qk64.int()).abs().max()) <= 1
    assert torch.allclose(p["k_scale"].cpu()[None], qks64, rtol=2e-2)
    # V: codes in this build's layout, bit-exact
    vq = osage.quant_v(Vf, p["v_scale"].cpu()[None])
    want = osage.wdl_v_layout(vq)[0].view(torch.uint8)  # [H, 128, Lpad]
    assert p["v"].shape == (H, 128, Lp)
    assert torch.equal(p["v"].cpu(), want)



@pytest.mark.parametrize("at,n,H", [(200, 150, 3), (0, 2640, 2), (6600, 2640, 2), (928, 464, 24)])
def test_attention_matches_quantized_oracle_and_exact(gpu, at, n, H):
    from wdl import sage_kv

    Q, k, ks, v, vs, at, K, V = setup(at, n, H=H, seed=3)
    out = sage_kv.attend(*cuda(Q, k, ks, v, vs), at, *cuda(K, V))
    torch.cuda.synchronize()
    out = out.cpu().float()
    p = osage.prep(Q, k, ks, v, vs, at, K, V)
    emul = osage.attention_quantized(p, 128 ** -0.5)
    emul8 = osage.attention_quantized(p, 128 ** -0.5, p_fp8=True)
    exact = osage.attention_exact(Q, p["K"], p["V"])
    cos = osage.cosine(out, emul)
    print(f"at {at} n {n}: cos vs emulation {cos:.6f}, err vs exact {osage.rel_err(out, exact):.4f} "
          f"(emulation exact P {osage.rel_err(emul, exact):.4f}, fp8 P {osage.rel_err(emul8, exact):.4f})")
    assert cos >= 0.999
    assert osage.rel_err(out, exact) < 1.2 * osage.rel_err(emul8, exact) + 1e-3


def test_attention_single_key_and_ragged_lengths(gpu):
    from wdl import sage_kv

    for at, n in ((0, 1), (1, 1), (63, 2), (64, 1), (127, 70)):
        Q, k, ks, v, vs, at, K, V = setup(at, n, nq=n, H=2, seed=at * 7 + n)
        out = sage_kv.attend(*cuda(Q, k, ks, v, vs), at, *cuda(K, V)).cpu().float()
        p = osage.prep(Q, k, ks, v, vs, at, K, V)
        emul = osage.attention_quantized(p, 128 ** -0.5)
        assert osage.cosine(out, emul) >= 0.999, (at, n)



@pytest.mark.parametrize("grid,start,M", [((1, 16, 29), 2, 464), ((3, 16, 29), 0, 1408), ((2, 3, 5), 7, 30)])
def test_qk_norm_rope_bit_exact(gpu, grid, start, M):
    from wdl import rope

    H = 24 if M >= 464 else 2
    g = torch.Generator().manual_seed(M)
    qkv = (torch.randn(M, 3 * H * 128, generator=g) * 2).to(torch.bfloat16)
    wq = (torch.rand(H * 128, generator=g) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(H * 128, generator=g) + 0.5).to(torch.bfloat16)
    freq = orope.freqs(128, 1024, torch.float64).float()
    d = qkv.cuda()
    C = H * 128
    Qo, Ko = rope.norm_rope(d[:, :C], d[:, C:2 * C], wq.cuda(), wk.cuda(), freq.cuda(), grid, start)
    torch.cuda.synchronize()
    for x, w, got in ((qkv[:, :C], wq, Qo), (qkv[:, C:2 * C], wk, Ko)):
        n = onorms.rms_norm(x.contiguous(), w).reshape(1, M, H, 128)
        want = orope.rope_apply(n, grid, freq, start)
        assert torch.equal(got.cpu().reshape(1, M, H, 128), want)


def test_rope_identities_on_gpu(gpu):
    """Chunk-offset identity (bit-exact) and norm preservation (tests/test_rope_triton.py:89-104) on the kernel."""
    from wdl import rope

    H, M = 2, 12
    g = torch.Generator().manual_seed(1)
    x = torch.randn(M, H * 128, generator=g).to(torch.bfloat16).cuda()
    ones = torch.ones(H * 128, dtype=torch.bfloat16).cuda()
    freq = orope.freqs(128, 64, torch.float64).float().cuda()
    whole, _ = rope.norm_rope(x, x, ones, ones, freq, (3, 2, 2), 5)
    parts = [rope.norm_rope(x[4 * i:4 * i + 4], x[4 * i:4 * i + 4], ones, ones, freq, (1, 2, 2), 5 + i)[0]
             for i in range(3)]
    assert torch.equal(whole, torch.cat(parts))
    plain, _ = rope.norm_rope(x, x, ones, ones, freq, (0, 2, 2), 0)  # f = 0: norm only
    a = whole.float().reshape(M, H, 64, 2).square().sum(-1)
    b = plain.float().reshape(M, H, 64, 2).square().sum(-1)
    assert torch.allclose(a, b, rtol=2 ** -6, atol=1e-3)
