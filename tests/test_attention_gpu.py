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


@pytest.mark.parametrize("cached", [False, True], ids=["whole", "cached-stats"])
@pytest.mark.parametrize("at,n,H", [(200, 150, 3), (0, 130, 2), (928, 464, 24), (6600, 2640, 2), (8352, 1392, 2),
                                    (1, 1, 2)])
def test_sage_prep_k_and_v(gpu, at, n, H, cached):
    """cached-stats: the preparation from the cached rows' statistics (wdl_sage_cache_stats) plus the chunk's
    tokens, held to the same bars."""
    from wdl import sage_kv

    kbias = torch.randn(1, 1, H, 128, generator=torch.Generator().manual_seed(5)) * 3
    Q, k, ks, v, vs, at, K, V = setup(at, n, H=H, seed=at + n, kbias=kbias)
    ks = ks * 0.5 + torch.rand(ks.shape, generator=torch.Generator().manual_seed(1))  # non-unit cache scales
    vs = vs * 0.25 + torch.rand(vs.shape, generator=torch.Generator().manual_seed(2))
    stats = sage_kv.cache_stats(*cuda(k, ks, v, vs), at) if cached else None
    p = sage_kv.prep(*cuda(k, ks, v, vs), at, *cuda(K, V), cache_stats=stats)
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
    # V: codes in wdl's layout, bit-exact
    vq = osage.quant_v(Vf, p["v_scale"].cpu()[None])
    want = osage.wdl_v_layout(vq)[0].view(torch.uint8)  # [H, 128, Lpad]
    assert p["v"].shape == (H, 128, Lp)
    assert torch.equal(p["v"].cpu(), want)


@pytest.mark.parametrize("at,n,H", [(200, 150, 3), (0, 130, 2), (64, 64, 2), (63, 1, 2), (8352, 1392, 24)])
def test_prep_with_append_is_store_then_prep(gpu, at, n, H):
    """wdl_sage_prep_cached_append (the chunk's cache store inside the preparation pass) against store_kv_fp8
    (wdl_kv_append_fp8) followed by the unfused preparation: every byte of the caches and their scales equal (rows
    at .. at + n written, the others untouched), and the Sage operands, K mean and V scales bit-equal."""
    from wdl import ops, sage_kv
    from wdl.cache_fp8 import store_kv_fp8

    Q, k, ks, v, vs, at, K, V = setup(at, n, H=H, seed=at + n + 7)
    ks = ks * 0.5 + torch.rand(ks.shape, generator=torch.Generator().manual_seed(3))
    vs = vs * 0.25 + torch.rand(vs.shape, generator=torch.Generator().manual_seed(4))
    k, ks, v, vs, K, V = cuda(k, ks, v, vs, K, V)
    stats = sage_kv.cache_stats(k, ks, v, vs, at)
    ka, ksa, va, vsa = (t.clone() for t in (k, ks, v, vs))
    store_kv_fp8(K, V, ka, ksa, va, vsa, at)
    pa = ops.sage_prep_launch(ka.view(torch.uint8), ksa, va.view(torch.uint8), vsa, K[0].flatten(1), V[0].flatten(1),
                              at, want_stats=True, cache_stats=stats)
    kb, ksb, vb, vsb = (t.clone() for t in (k, ks, v, vs))
    pb = ops.sage_prep_launch(kb.view(torch.uint8), ksb, vb.view(torch.uint8), vsb, K[0].flatten(1), V[0].flatten(1),
                              at, want_stats=True, cache_stats=stats, append=True)
    torch.cuda.synchronize()
    assert torch.equal(ka.view(torch.uint8), kb.view(torch.uint8)) and torch.equal(va.view(torch.uint8),
                                                                                      vb.view(torch.uint8))
    assert torch.equal(ksa, ksb) and torch.equal(vsa, vsb)
    assert not torch.equal(kb.view(torch.uint8)[:, at:at + n], k.view(torch.uint8)[:, at:at + n])
    for key in ("k", "k_scale", "v", "v_scale", "k_mean"):
        assert torch.equal(pa[key], pb[key]), key


def test_attend_with_append_refuses_before_writing(gpu):
    """sage_kv.attend(append=True) checks the store's requirements (rows past the cache here) before any launch."""
    from wdl import sage_kv

    Q, k, ks, v, vs, at, K, V = setup(100, 64, H=2, seed=11)
    Q, k, ks, v, vs, K, V = cuda(Q, k, ks, v, vs, K, V)
    stats = sage_kv.cache_stats(k, ks, v, vs, at)
    before = k.view(torch.uint8).clone()
    with pytest.raises(ValueError):
        sage_kv.attend(Q, k, ks, v, vs, k.shape[1] - 10, K, V, cache_stats=stats, append=True)
    torch.cuda.synchronize()
    assert torch.equal(k.view(torch.uint8), before)


@pytest.mark.parametrize("at,H", [(0, 2), (1, 3), (63, 2), (200, 3), (8352, 24)])
def test_cache_stats_against_float64_sums_and_exact_maxima(gpu, at, H):
    """wdl_sage_cache_stats: the K column sums within 1e-5 of the sum of |values| (a token dropped or counted twice
    moves a sum by ~1e-4 of it at 8352 tokens), the |V| maxima exact (fp32 products of e4m3 values and scales)."""
    from wdl import sage_kv

    g = torch.Generator().manual_seed(at + H)
    cap = at + 70
    k = (torch.randn(1, cap, H, 128, generator=g) * 2 + 1).to(torch.float8_e4m3fn)
    v = torch.randn(1, cap, H, 128, generator=g).to(torch.float8_e4m3fn)
    ks = torch.rand(1, cap, H, 1, generator=g) + 0.1
    vs = torch.rand(1, cap, H, 1, generator=g) + 0.1
    stats = sage_kv.cache_stats(*cuda(k, ks, v, vs), at).cpu()
    assert stats.shape == (2, H, 128)
    Kc = k[0, :at].float() * ks[0, :at]
    Vc = v[0, :at].float() * vs[0, :at]
    want = Kc.double().sum(0)
    bound = 1e-5 * Kc.double().abs().sum(0) + 1e-30
    assert bool(((stats[0].double() - want).abs() <= bound).all())
    assert torch.equal(stats[1], Vc.abs().amax(0) if at else torch.zeros(H, 128))



@pytest.mark.parametrize("at,n,H", [(200, 150, 3), (0, 2640, 2), (6600, 2640, 2), (928, 464, 24), (0, 1392, 24)])
def test_attention_matches_quantized_oracle_and_exact(gpu, at, n, H):
    """(0, 1392, 24): 11 x 24 = 264 tiles over 1392 keys (22 blocks, the last ragged): on 256 CUs the first 8
    workgroups run two whole tiles, one per group, each over all the key blocks and its own masked final block."""
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


@pytest.mark.parametrize("at,n,H,frame", [(100, 1392, 2, 464), (0, 1392, 24, 464), (200, 150, 3, 64),
                                         (928, 464, 2, 464), (37, 1000, 2, 300)])
def test_block_causal_per_frame_mask(gpu, at, n, H, frame):
    """The chunk attention with the block-causal mask per latent frame (query q of the chunk sees the cache and the
    chunk's frames up to its own): frames of 464 tokens put frame ends inside 128-query tiles (tiles 3 and 7), L is
    ragged (1492, 1392, 350, 1037 keys), (0, 1392, 24) runs the dual-tile launch (264 tiles over 22 blocks), and
    (37, 1000, 2, 300) a partial last frame. Against the masked oracle: cosine >= 0.999 with the quantized
    emulation, error against exact masked attention within 1.2x that of the fp8-P emulation + 1e-3, and the first
    frame's queries unchanged when the later frames' keys are replaced (they are not seen)."""
    from wdl import sage_kv

    Q, k, ks, v, vs, at, K, V = setup(at, n, H=H, seed=5)
    out = sage_kv.attend(*cuda(Q, k, ks, v, vs), at, *cuda(K, V), frame_tokens=frame).cpu().float()
    p = osage.prep(Q, k, ks, v, vs, at, K, V)
    emul = osage.attention_quantized(p, 128 ** -0.5, frame=frame)
    emul8 = osage.attention_quantized(p, 128 ** -0.5, p_fp8=True, frame=frame)
    exact = osage.attention_exact(Q, p["K"], p["V"], frame=frame)
    cos = osage.cosine(out, emul)
    print(f"at {at} n {n} frame {frame}: cos vs emulation {cos:.6f}, err vs exact {osage.rel_err(out, exact):.4f} "
          f"(fp8 P emulation {osage.rel_err(emul8, exact):.4f})")
    assert cos >= 0.999
    assert osage.rel_err(out, exact) < 1.2 * osage.rel_err(emul8, exact) + 1e-3
    # keys of frames after the first replaced: the first frame's outputs must not move (its K mean and V scale
    # statistics do, so compare with the oracle on the changed operands rather than bitwise)
    K2, V2 = K.clone(), V.clone()
    K2[:, frame:] = -K2[:, frame:]
    V2[:, frame:] = V2[:, frame:] * 2
    out2 = sage_kv.attend(*cuda(Q, k, ks, v, vs), at, *cuda(K2, V2), frame_tokens=frame).cpu().float()
    p2 = osage.prep(Q, k, ks, v, vs, at, K2, V2)
    ex2 = osage.attention_exact(Q, p2["K"], p2["V"], frame=frame)
    f0 = slice(0, min(frame, n))
    assert osage.rel_err(out2[:, f0], ex2[:, f0]) < 1.2 * osage.rel_err(emul8[:, f0], exact[:, f0]) + 2e-3
    assert osage.rel_err(ex2[:, f0], exact[:, f0]) < 1e-6  # the first frame does not see the changed keys


def test_attention_longest_window_with_k_bias(gpu):
    """The chunk-causal attention workload's longest case: 2640 queries over 18480 cached + 2640 chunk keys (21120),
    K with a per-channel bias N(0, 3^2) that the mean smoothing removes; one head (the oracle's CPU cost), at the
    bars of the test above."""
    from wdl import sage_kv

    H = 1
    kbias = torch.randn(1, 1, H, 128, generator=torch.Generator().manual_seed(8)) * 3
    Q, k, ks, v, vs, at, K, V = setup(18480, 2640, H=H, seed=21, kbias=kbias)
    out = sage_kv.attend(*cuda(Q, k, ks, v, vs), at, *cuda(K, V)).cpu().float()
    p = osage.prep(Q, k, ks, v, vs, at, K, V)
    emul = osage.attention_quantized(p, 128 ** -0.5)
    emul8 = osage.attention_quantized(p, 128 ** -0.5, p_fp8=True)
    exact = osage.attention_exact(Q, p["K"], p["V"])
    cos = osage.cosine(out, emul)
    print(f"21120 keys: cos vs emulation {cos:.6f}, err vs exact {osage.rel_err(out, exact):.4f}")
    assert cos >= 0.999
    assert osage.rel_err(out, exact) < 1.2 * osage.rel_err(emul8, exact) + 1e-3


def test_attention_split_tiles_merge_across_workgroups(gpu):
    """(128-query tile, head) pairs just above the CU count: every CU runs one whole tile and the key blocks of the
    remaining tiles (the last head's, with the ragged query tile) are split over all CUs, their partial softmax
    states merged by a second launch. Checked on the first head (whole tiles) and the last (split tiles) against the
    oracle with the bars of the test above; two calls are bit-identical (the merge order is fixed)."""
    from wdl import sage_kv

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    n, at = 1392, 8352                      # 11 query tiles, 9744 keys (153 key blocks, the last ragged)
    H = cus // 11 + 1                       # 11 H tiles: just above the CU count
    Q, k, ks, v, vs, at, K, V = setup(at, n, H=H, seed=11)
    args = (*cuda(Q, k, ks, v, vs), at, *cuda(K, V))
    out = sage_kv.attend(*args)
    torch.cuda.synchronize()
    again = sage_kv.attend(*args)
    torch.cuda.synchronize()
    assert torch.equal(out, again)
    out = out.cpu().float()
    for hh in (0, H - 1):
        sl = lambda t: t[:, :, hh:hh + 1].contiguous()
        p = osage.prep(sl(Q), sl(k), sl(ks), sl(v), sl(vs), at, sl(K), sl(V))
        emul = osage.attention_quantized(p, 128 ** -0.5)
        emul8 = osage.attention_quantized(p, 128 ** -0.5, p_fp8=True)
        exact = osage.attention_exact(sl(Q), p["K"], p["V"])
        got = out[:, :, hh:hh + 1]
        assert osage.cosine(got, emul) >= 0.999, hh
        assert osage.rel_err(got, exact) < 1.2 * osage.rel_err(emul8, exact) + 1e-3, hh


@pytest.mark.parametrize("at,n,H", [(200, 150, 3), (0, 1, 2), (127, 70, 2), (8352, 1392, 24)])
def test_attention_q16_is_quant_q_then_attention(gpu, at, n, H):
    """wdl_sage_attn_q16 (Q quantized inside the attention kernel) against wdl_quant_q + wdl_sage_attn on the same
    operands: bit-identical outputs, also for a row-strided Q (a column slice of a wider buffer), ragged query
    counts and the split-tile launch (11 x 24 tiles on 256 CUs)."""
    from wdl import ops

    Q, k, ks, v, vs, at, K, V = setup(at, n, nq=n, H=H, seed=5)
    Qc, k, ks, v, vs, K, V = cuda(Q, k, ks, v, vs, K, V)
    prep = ops.sage_prep_launch(k.view(torch.uint8), ks, v.view(torch.uint8), vs, K[0].flatten(1), V[0].flatten(1),
                                at)
    q2 = Qc[0].flatten(1)
    wide = torch.zeros(n, H * 128 + 64, device="cuda", dtype=torch.bfloat16)
    wide[:, 32:32 + H * 128] = q2
    for q in (q2, wide[:, 32:32 + H * 128]):
        q_i8, q_sc = ops.quant_q_launch(q2, H)
        ref = ops.sage_attn_launch(q_i8, q_sc, prep, at + n, 128 ** -0.5)
        got = ops.sage_attn_q16_launch(q, prep, at + n, 128 ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (at, n, H, q.stride(0))


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


@pytest.mark.parametrize("table", ["fp32", "fp64"])
def test_rope_apply_bit_exact_with_padding_and_batch(gpu, table):
    """wdl.rope.rope_apply (rope.py:12-31 / rope3d_rotate) against the oracle's rope_apply: bf16 X [2, L, H, 128]
    with L past the grid (padding rows copied), a chunk offset, an fp32 or an fp64 table (the fp64 products are
    rounded to fp32, then bf16, as torch converts double to bfloat16)."""
    from wdl import rope

    g = torch.Generator().manual_seed(21)
    grid, start, L, H = (2, 3, 5), 7, 34, 3
    X = (torch.randn(2, L, H, 128, generator=g) * 3).to(torch.bfloat16)
    freq = orope.freqs(128, 64, torch.float64)
    if table == "fp32":
        freq = freq.float()
    got = rope.rope_apply(X.cuda(), [grid, grid], freq.cuda(), start).cpu()  # one grid per sample
    for b in range(2):
        want = orope.rope_apply(X[b:b + 1], grid, freq, start)
        assert torch.equal(got[b:b + 1], want)
    assert torch.equal(got[:, 30:], X[:, 30:])
    with pytest.raises(ValueError):
        rope.rope_apply(X.cuda(), [(3, 3, 5)] * 2, freq.cuda(), start)


@pytest.mark.parametrize("cached", [False, True])
def test_fused_qkv_attention_module_matches_oracle(gpu, cached):
    """FusedQKVAttention (w4a4.py:246-262) on the HIP path, dim 256, 2 heads, grid (2, 4, 6), with and without an
    FP8 cache of 96 prior tokens:
    - wiring: bit-equal to the forward of the reference written out with the same wdl ops (with a cache, the
      KVCache's Sage attention, causal.py:193-210; without, the bf16 attention of the chunk over itself, the
      reference's scaled_dot_product_attention branch, w4a4.py:259-261);
    - the attention stage, fed the oracle's own Q, K, V: with a cache, cosine >= 0.99999 and relative L2 <= 2e-3
      against the oracle's blockwise Sage attention (the config-1 stage bar); without, relative L2 <= 2 * 2^-9 and
      cosine >= 0.99999 against the exact softmax on the bf16 operands (P's bf16 rounding, the bf16 attention's
      bar);
    - end to end against the oracle composition: relative L2 <= 2e-2 (the W4A4 o projection re-quantizes the
      attention output to int4, so its ~1e-3 differences flip codes: measured ~7e-3)."""
    from oracle import block as oblock
    from wdl import ops, rope, w4a4
    from wdl.kvcache import KVCache

    g = torch.Generator().manual_seed(5)
    dim, H, grid, start, prior = 256, 2, (2, 4, 6), 3, 96
    P = oblock.quantize_block(oblock.random_block(dim, 512, g))
    M = grid[0] * grid[1] * grid[2]
    X = torch.randn(1, M, dim, generator=g).to(torch.bfloat16)
    freq = orope.freqs(128, 64, torch.float64).float()
    dev = torch.device("cuda")
    m = w4a4.FusedQKVAttention(dim, H)
    m.qkv = w4a4.PackedW4A4Linear(**w4a4.pack_parts(P["qkv"], dev))
    m.o = w4a4.PackedW4A4Linear(**w4a4.pack_parts(P["o"], dev))
    m.norm_q, m.norm_k = P["wq"].to(torch.bfloat16).to(dev), P["wk"].to(torch.bfloat16).to(dev)
    ck = (torch.randn(1, prior + M, H, 128, generator=g) * 50).clamp(-448, 448).to(torch.float8_e4m3fn)
    cks = torch.rand(1, prior + M, H, 1, generator=g) * 0.02

    def new_cache():
        if not cached:
            return None
        c = KVCache(prior, 0, chunk=grid[0])
        c.allocate(torch.empty(1, M, H, 128, device=dev))
        c.k.copy_(ck.to(dev)), c.v.copy_(ck.to(dev)), c.ks.copy_(cks.to(dev)), c.vs.copy_(cks.to(dev))
        c.saved = prior
        return c

    got = m(X.to(dev), [grid], freq.to(dev), start_frame=start, cache=new_cache())
    # the reference's forward, written out with the same ops
    Xd = X.to(dev)
    q, k, v = m.qkv(Xd).split(dim, dim=-1)
    Qw, Kw = rope.norm_rope(q[0], k[0], m.norm_q, m.norm_k, freq.to(dev), grid, start)
    shape = (1, M, H, 128)
    c = new_cache()
    if c is not None:
        Aw = c.attend(Qw.view(shape), Kw.view(shape), v[0].reshape(shape))
    else:
        Aw = ops.attn_bf16_launch(Qw, ops.attn_bf16_prep_launch(Kw, v[0]), 128 ** -0.5)
    assert torch.equal(got, m.o(Aw.reshape(1, M, dim)))
    # the oracle
    qkv = oblock._lin(X[0], P["qkv"]).to(torch.bfloat16)
    Q = orope.rope_apply(oblock._rms(qkv[:, :dim], P["wq"]).reshape(1, M, H, 128), grid, freq, start)
    K = orope.rope_apply(oblock._rms(qkv[:, dim:2 * dim], P["wk"]).reshape(1, M, H, 128), grid, freq, start)
    V = qkv[:, 2 * dim:].contiguous()
    ocache = dict(k=ck, ks=cks, v=ck, vs=cks, at=prior) if cached else None
    # the cache rows [0, at) and the chunk's own bf16 K, V enter the attention (rows >= at are not read)
    A = oblock.attention(Q.reshape(M, dim), ocache, K.reshape(M, dim), V, H)
    c = new_cache()
    Qd, Kd, Vd = (t.reshape(shape).to(dev) for t in (Q, K, V))
    if c is not None:
        Ag = c.attend(Qd, Kd, Vd)
    else:
        Ag = ops.attn_bf16_launch(Qd.reshape(M, dim), ops.attn_bf16_prep_launch(Kd.reshape(M, dim),
                                                                                Vd.reshape(M, dim)), 128 ** -0.5)
    Ag = Ag.cpu().reshape(M, dim)
    rel = lambda a, b: float((a.float() - b.float()).norm() / b.float().norm())
    assert rel(Ag, A) <= (2e-3 if cached else 2 * 2 ** -9) and osage.cosine(Ag, A) >= 0.99999
    want = oblock._lin(A, P["o"]).to(torch.bfloat16)
    e2e = rel(got.cpu().reshape(M, dim), want)
    print(f"cached={cached}: attention stage rel {rel(Ag, A):.2e}, end to end rel-L2 {e2e:.2e}")
    assert e2e <= 2e-2


@pytest.mark.parametrize("n,L,H", [(1392, 512, 24), (464, 512, 24), (100, 77, 2), (300, 1000, 3), (1700, 512, 24),
                                   (2640, 512, 24)])
def test_bf16_attention_is_the_exact_softmax(gpu, n, L, H):
    """wdl_attn_bf16 (the cross-attention: bf16 operands, fp32 online softmax, P rounded to bf16 as flash attention
    does) against the exact softmax in float64 on the same bf16 values. On 256 CUs: 1392 x 512 x 24 heads is the
    step's cross-attention (160-query tiles, 216 workgroups in one round), 1700 queries take 192-query tiles, 2640
    queries 128-query tiles with two per workgroup on the first ones, 464 x 512 one 128-query tile per workgroup;
    L = 77 and 1000 end in a partial 64-key block. Bar: relative L2 <= 2 * 2^-9 and cosine >= 0.99999 (P's bf16 rounding is the
    only approximation: up to 2^-9 relative per weight; measured 2.2e-3 at the step's shape)."""
    from oracle import sage as osage
    from wdl import ops

    g = torch.Generator().manual_seed(n + L + H)
    Q = torch.randn(n, H * 128, generator=g).to(torch.bfloat16)
    K = (torch.randn(L, H * 128, generator=g) + torch.randn(1, H * 128, generator=g) * 2).to(torch.bfloat16)
    V = torch.randn(L, H * 128, generator=g).to(torch.bfloat16)
    sm = 128 ** -0.5
    prep = ops.attn_bf16_prep_launch(K.cuda(), V.cuda())
    out = ops.attn_bf16_launch(Q.cuda(), prep, sm).cpu()
    ref = osage.attention_exact(Q.view(1, n, H, 128), K.view(1, L, H, 128).float(), V.view(1, L, H, 128).float(), sm)
    rel, cos = osage.rel_err(out.view(1, n, H, 128), ref), osage.cosine(out, ref)
    print(f"bf16 attention n={n} L={L} H={H}: rel-L2 {rel:.2e}, cosine {cos:.7f}")
    assert rel <= 2 * 2 ** -9 and cos >= 0.99999
