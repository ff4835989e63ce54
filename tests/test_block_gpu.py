"""The quantized Wan block on the HIP path against the oracle block (oracle/block.py).

Bars:
- small blocks (dim 256, SVD-quantized): bf16 output within max-rel-err 1e-2 and 2^-8 relative L2 of the oracle;
- config 1 (dim 3072): max-rel-err 1e-2, and relative L2 within 1.5x of the oracle's own change under 50 one-ulp
  changes of its bf16 input (a random-weight W4A4 block without smoothing is chaotic at that level: one
  activation-int4 flip moves a whole quantization step; measured in the test);
- stage by stage at config 1, each HIP stage fed the oracle's own input: 1e-4 relative L2 (linears), 1e-3 (the
  fused GELU MLP, whose fp32 hidden layer meets GELU's last-bit differences before its int4 rounding), 2e-3 with
  cosine >= 0.99999 (attention);
- the reference's own contract (tests/test_w4a4.py:62-87): the W4A4 block's update against the float block's,
  within 5 % of the oracle's own error there and below 0.21 (the reference's 0.2 was stated for exact SDPA; the
  Sage attention adds about 0.003)."""

import pytest
import torch

from oracle import block as oblock
from oracle import rope as orope

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def run_pair(dim, heads, ffn, grid, start, prior, Lc, seed, svd=False, scale_dtype=None, weight_scale=0.02):
    from wdl.block import LINEARS, build_block
    from wdl.kvcache import KVCache

    g = torch.Generator().manual_seed(seed)
    P = (oblock.quantize_block(oblock.random_block(dim, ffn, g)) if svd
         else oblock.random_logical_block(dim, ffn, g, scale=weight_scale))
    if scale_dtype is not None:  # both sides take the weight scales in this type
        for name in LINEARS:
            P[name]["wscales"] = P[name]["wscales"].to(scale_dtype)
    M = grid[0] * grid[1] * grid[2]
    X = torch.randn(M, dim, generator=g)
    X[:, torch.randperm(dim, generator=g)[: max(1, dim // 100)]] *= 20
    X = X.to(BF)
    time_in = torch.randn(6, dim, generator=g) * 0.1
    C = torch.randn(Lc, dim, generator=g).to(BF)
    freq = orope.freqs(128, 1024, torch.float64).float()
    cap = prior + M
    ck = (torch.randn(1, cap, heads, 128, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    cv = (torch.randn(1, cap, heads, 128, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    cks = torch.rand(1, cap, heads, 1, generator=g) * 0.02
    cvs = torch.rand(1, cap, heads, 1, generator=g) * 0.02
    # oracle
    ocache = dict(k=ck.clone(), ks=cks.clone(), v=cv.clone(), vs=cvs.clone(), at=prior)
    ctx_kv = oblock.context_kv(C, P)
    ref = oblock.block_forward(X, time_in, P, grid, freq, start, ocache, ctx_kv, heads)
    # HIP path
    dev = torch.device("cuda")
    blk = build_block(P, dim, heads, dev)
    cache = KVCache(prior, 0, chunk=grid[0])
    cache.allocate(torch.empty(1, M, heads, 128, device=dev))
    cache.k.copy_(ck.to(dev))
    cache.v.copy_(cv.to(dev))
    cache.ks.copy_(cks.to(dev))
    cache.vs.copy_(cvs.to(dev))
    cache.saved = prior
    ctx = blk.prepare_context(C.to(dev))
    e = (time_in + P["modulation"]).float().to(dev)
    out = blk.forward(X.to(dev).clone(), e, grid, freq.to(dev), start, cache, ctx)
    torch.cuda.synchronize()
    inputs = dict(P=P, time_in=time_in, ctx_kv=ctx_kv, freq=freq, grid=grid, start=start, heads=heads,
                  cache=dict(k=ck, ks=cks, v=cv, vs=cvs, at=prior))
    return X, out.cpu(), ref, cache, ocache, inputs


def check(tag, out, ref):
    err = float((out.float() - ref.float()).abs().max()) / float(ref.float().abs().max())
    rel = float((out.float() - ref.float()).norm() / ref.float().norm())
    print(f"{tag}: max-rel-err {err:.2e}, rel-L2 {rel:.3e}")
    assert err <= 1e-2
    assert rel <= 2 ** -8


@pytest.mark.parametrize("seed", [0, 1])
def test_small_block_matches_oracle(gpu, seed):
    X, out, ref, cache, ocache, _ = run_pair(256, 2, 1024, (2, 4, 6), 2, 96, 16, seed, svd=True)
    check(f"seed {seed}", out, ref)
    # the chunk's K/V went into the cache rows at..at+M: fp8 bytes equal up to bf16 flips upstream
    at, M = ocache["at"], X.shape[0]
    same = (cache.k.cpu()[:, at:at + M].view(torch.uint8) == ocache["k"][:, at:at + M].view(torch.uint8))
    assert float(same.float().mean()) > 0.97


def test_small_block_with_fp16_weight_scales_matches_oracle(gpu):
    """The fp16 weight-scale mode (the benchmark configurations quantize with fp16 scales; the reference keeps bf16):
    the same bars as the bf16 block."""
    X, out, ref, cache, ocache, _ = run_pair(256, 2, 1024, (2, 4, 6), 2, 96, 16, 3, svd=True,
                                             scale_dtype=torch.float16)
    check("fp16 scales", out, ref)


def test_mixed_precision_block_matches_oracle(gpu):
    """The mixed-precision mode: attention projections FP8 weight-only (e4m3 rows, bf16 activations), the
    feed-forward W4A4, at dim 256 over an FP8 cache and a prompt, against the oracle block with the same parts: the
    block bars (max-rel-err 1e-2, relative L2 2^-8)."""
    from wdl.block import build_block
    from wdl.kvcache import KVCache

    g = torch.Generator().manual_seed(23)
    dim, heads, ffn, grid, start, prior, Lc = 256, 2, 1024, (2, 4, 8), 3, 192, 40
    P = oblock.mixed_precision_block(dim, ffn, g)
    M = grid[0] * grid[1] * grid[2]
    X = torch.randn(M, dim, generator=g).to(BF)
    time_in = torch.randn(6, dim, generator=g) * 0.1
    C = torch.randn(Lc, dim, generator=g).to(BF)
    freq = orope.freqs(128, 1024, torch.float64).float()
    ck = (torch.randn(1, prior + M, heads, 128, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    cks = torch.rand(1, prior + M, heads, 1, generator=g) * 0.02
    ocache = dict(k=ck.clone(), ks=cks.clone(), v=ck.clone(), vs=cks.clone(), at=prior)
    ref = oblock.block_forward(X, time_in, P, grid, freq, start, ocache, oblock.context_kv(C, P), heads)
    dev = torch.device("cuda")
    blk = build_block(P, dim, heads, dev)
    cache = KVCache(prior, 0, chunk=grid[0])
    cache.allocate(torch.empty(1, M, heads, 128, device=dev))
    for dst, src in ((cache.k, ck), (cache.v, ck), (cache.ks, cks), (cache.vs, cks)):
        dst.copy_(src.to(dev))
    cache.saved = prior
    e = (time_in + P["modulation"]).float().to(dev)
    out = blk.forward(X.to(dev).clone(), e, grid, freq.to(dev), start, cache, blk.prepare_context(C.to(dev))).cpu()
    check("mixed precision block", out, ref)


def test_full_width_block_on_one_frame_matches_oracle(gpu):
    """The full-width block on one frame: dim 3072, 24 x 128 heads, FFN 14336, 464-token frame (16 x 29) at start frame 2 over a
    928-token FP8 cache (two prior frames), 512 context tokens, random-init W4A4 weights."""
    X, out, ref, cache, ocache, inp = run_pair(3072, 24, 14336, (1, 16, 29), 2, 928, 512, 7)
    err = float((out.float() - ref.float()).abs().max()) / float(ref.float().abs().max())
    rel = float((out.float() - ref.float()).norm() / ref.float().norm())
    # the oracle against itself with 50 one-ulp input changes
    Xp = X.clone()
    flat = Xp.view(-1).view(torch.int16)
    flat[torch.randperm(flat.numel(), generator=torch.Generator().manual_seed(99))[:50]] += 1
    pert = oblock.block_forward(Xp, inp["time_in"], inp["P"], inp["grid"], inp["freq"], inp["start"],
                                dict(inp["cache"]), inp["ctx_kv"], inp["heads"])
    floor = float((pert.float() - ref.float()).norm() / ref.float().norm())
    print(f"config 1: max-rel-err {err:.2e}, rel-L2 {rel:.3e} (oracle under 50 one-ulp input changes: {floor:.3e})")
    assert err <= 1e-2
    assert rel <= 1.5 * floor


def test_w4a4_block_stays_close_to_the_float_block(gpu):
    """tests/test_w4a4.py:62-87: the fused W4A4 block within 0.2 relative error of the float block, the block's
    update compared (dim 256, 2 heads, FFN 1024, 2 x 8 x 16 tokens, X ~ N(0, 1), e ~ 0.1 N(0, 1), 16 context
    tokens, SVD-quantized weights of rank 32, no cache). Here the attention is also quantized (Sage: int8 QK, fp8
    PV), where the reference's test ran exact SDPA."""
    from wdl.block import build_block
    from wdl.kvcache import KVCache

    dim, heads, ffn, grid, Lc = 256, 2, 1024, (2, 8, 16), 16
    g = torch.Generator().manual_seed(1)
    B = oblock.random_block(dim, ffn, g, init="torch")
    P = oblock.quantize_block(B)
    M = 256
    X = torch.randn(M, dim, generator=g).to(BF)
    time_in = torch.randn(6, dim, generator=g) * 0.1
    C = torch.randn(Lc, dim, generator=g).to(BF)
    none = torch.zeros(0, dim)
    freq = orope.freqs(128, 1024, torch.float64).float()
    ref = oblock.float_block_forward(X, time_in, B, grid, freq, 0, (none, none), C.float(), heads)
    dev = torch.device("cuda")
    blk = build_block(P, dim, heads, dev)
    cache = KVCache(0, 0, chunk=grid[0])
    out = blk.forward(X.to(dev).clone(), (time_in + P["modulation"]).float().to(dev), grid, freq.to(dev), 0, cache,
                      blk.prepare_context(C.to(dev))).cpu()
    upd, rupd = out.float() - X.float(), ref - X.float()
    err = float((upd - rupd).norm() / rupd.norm())
    z8 = torch.zeros(1, M, heads, 128, dtype=torch.float8_e4m3fn)
    zs = torch.ones(1, M, heads, 1)
    oq = oblock.block_forward(X, time_in, P, grid, freq, 0, dict(k=z8, ks=zs, v=z8.clone(), vs=zs.clone(), at=0),
                              oblock.context_kv(C, P), heads)
    oerr = float(((oq.float() - X.float()) - rupd).norm() / rupd.norm())
    print(f"W4A4 block vs float block: update rel err {err:.3f} (oracle's own: {oerr:.3f})")
    # the W4A4 scheme itself sits at ~0.2 here (0.195-0.203 with exact attention); the Sage attention adds ~0.003
    assert err <= 1.05 * oerr and err < 0.21


@pytest.mark.parametrize("M,prior,grid,start", [(464, 928, (1, 16, 29), 2), (1392, 8352, (3, 16, 29), 18)])
def test_block_stages_given_identical_inputs(gpu, M, prior, grid, start):
    """Each stage of the full-width block on the HIP path, fed the oracle's own input for that stage: one frame over
    two cached frames (464 over 928 keys), and the step's chunk of three frames over the full window (1392 over
    8352 + 1392 keys)."""
    from oracle import norms as onorms
    from oracle import sage as osage
    from oracle import w4a4 as ow
    from wdl import ops, sage_kv
    from wdl.block import build_block

    dev = torch.device("cuda")
    dim, heads, ffn = 3072, 24, 14336
    g = torch.Generator().manual_seed(7)
    P = oblock.random_logical_block(dim, ffn, g)
    X = torch.randn(M, dim, generator=g).to(BF)
    e = (torch.randn(6, dim, generator=g) * 0.1 + P["modulation"]).float()
    C = torch.randn(512, dim, generator=g).to(BF)
    freq = orope.freqs(128, 1024, torch.float64).float()
    ck = (torch.randn(1, prior + M, heads, 128, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    cks = torch.rand(1, prior + M, heads, 1, generator=g) * 0.02
    blk = build_block(P, dim, heads, dev)
    rel = lambda a, b: float((a.float() - b.float()).norm() / b.float().norm())

    def gpu_lin(x, name, shift=0.0, unsigned=False, epi=0):
        t = blk.p[name]
        qa = ops.act_quant_launch(x.to(dev).contiguous(), t["smooth"], t["proj_down"], shift, unsigned)
        out = torch.empty(x.shape[0], ops.out_features(t["wcodes"]), device=dev, dtype=BF)
        ops.gemm_launch(*qa, t["wcodes"], t["wscales"], t["proj_up"], t["bias"], x.shape[0], out, epi)
        return out.cpu()

    x1 = onorms.ln_mod(X, e[0], e[1])
    qkv = oblock._lin(x1, P["qkv"]).to(BF)
    assert rel(gpu_lin(x1, "qkv"), qkv) <= 1e-4
    D = dim
    Q = orope.rope_apply(oblock._rms(qkv[:, :D], P["wq"]).reshape(1, -1, heads, 128), grid, freq, start)
    K = orope.rope_apply(oblock._rms(qkv[:, D:2 * D], P["wk"]).reshape(1, -1, heads, 128), grid, freq, start)
    V = qkv[:, 2 * D:].reshape(1, -1, heads, 128).contiguous()
    A = oblock.attention(Q.reshape(-1, D), dict(k=ck, ks=cks, v=ck, vs=cks, at=prior), K.reshape(-1, D),
                         V.reshape(-1, D), heads)
    Ag = sage_kv.attend(*(t.to(dev) for t in (Q, ck, cks, ck, cks)), prior, K.to(dev), V.to(dev)).cpu()
    # (128-query tile, head) pairs beyond the last whole multiple of the CU count (at 1392 queries, 264 on 256 CUs:
    # the last head's tiles 3 .. 10) run split over all workgroups in pieces of a few key blocks, each piece with its
    # own lazy reference max, which the oracle's two-part emulation does not follow: their P roundings differ (~1 %),
    # so they are held to the Sage bars (cosine 0.9999 with the emulation, error against exact attention within
    # 1.2x that of the fp8-P emulation + 1e-3), the whole tiles to cosine 0.99999 and 2e-3
    Ag, A4 = Ag.reshape(M, heads, 128), A.reshape(M, heads, 128)
    whole = torch.ones(M, heads, dtype=torch.bool)
    qt, cus = -(-M // 128), torch.cuda.get_device_properties(0).multi_processor_count
    T = qt * heads
    if T > cus and (T + cus - 1) // cus * cus * 85 > T * 100 and -(-(prior + M) // 64) >= 32:
        for tile in range(cus * (T // cus), T):
            whole[128 * (tile % qt):128 * (tile % qt + 1), tile // qt] = False
    print(f"attention stage: whole tiles rel {rel(Ag[whole], A4[whole]):.2e}"
          + (f", split tiles rel {rel(Ag[~whole], A4[~whole]):.2e}" if (~whole).any() else ""))
    assert rel(Ag[whole], A4[whole]) <= 2e-3 and osage.cosine(Ag[whole], A4[whole]) >= 0.99999
    if (~whole).any():
        assert osage.cosine(Ag[~whole], A4[~whole]) >= 0.9999
        hs = sorted({int(h) for h in (~whole).nonzero()[:, 1]})
        for h in hs:
            sl = lambda t: t[:, :, h:h + 1].contiguous()
            p = osage.prep(sl(Q), sl(ck), sl(cks), sl(ck), sl(cks), prior, sl(K), sl(V))
            exact = osage.attention_exact(sl(Q), p["K"], p["V"])[0, :, 0]
            emul8 = osage.attention_quantized(p, 128 ** -0.5, p_fp8=True)[0, :, 0]
            rows = ~whole[:, h]
            assert rel(Ag[rows, h], exact[rows]) <= 1.2 * rel(emul8[rows], exact[rows]) + 1e-3
    Ag = Ag.reshape(M, D)
    assert rel(gpu_lin(A, "o"), oblock._lin(A, P["o"]).to(BF)) <= 1e-4
    xc = onorms.ln_mod(X, None, None, P["n3w"], P["n3b"])
    assert rel(gpu_lin(xc, "cq"), oblock._lin(xc, P["cq"]).to(BF)) <= 1e-4
    assert rel(gpu_lin(C, "ck"), oblock._lin(C, P["ck"]).to(BF)) <= 1e-4
    # cross-attention: the oracle's exact softmax on bf16 operands (the reference's SDPA) against the bf16 kernel
    Qc = oblock._rms(oblock._lin(xc, P["cq"]).to(BF), P["cwq"])
    Kc, Vc = oblock.context_kv(C, P)
    Ac = oblock.cross_attention(Qc, Kc, Vc, heads)
    Acg = ops.attn_bf16_launch(Qc.to(dev), ops.attn_bf16_prep_launch(Kc.to(dev), Vc.to(dev)), 128 ** -0.5).cpu()
    assert rel(Acg, Ac) <= 2 * 2 ** -9 and osage.cosine(Acg, Ac) >= 0.99999  # P rounded to bf16: 2^-9 per weight
    # the fused GELU MLP: the oracle's hidden layer is fp32 (w4a4.py:198-204); the kernel's GELU differs from
    # torch's in the last bits, so a few int4 values of the hidden layer land one step apart (the epilogue test
    # bounds them): relative L2 1e-3 here
    x2 = onorms.ln_mod(X, e[3], e[4])
    y2 = ow.gelu_mlp(x2, P["ffn1"], P["ffn2"])
    t1, t2 = blk.p["ffn1"], blk.p["ffn2"]
    qa = ops.act_quant_launch(x2.to(dev).contiguous(), t1["smooth"], t1["proj_down"])
    hq = ops.gelu_quant_launch(*qa, t1["wcodes"], t1["wscales"], t1["proj_up"], t1["bias"], M, t2["smooth"],
                               t2["proj_down"])
    out = torch.empty(M, dim, device=dev, dtype=BF)
    ops.gemm_launch(*hq, t2["wcodes"], t2["wscales"], t2["proj_up"], t2["bias"], M, out)
    print(f"fused MLP stage: rel-L2 {rel(out.cpu(), y2):.2e}")
    assert rel(out.cpu(), y2) <= 1e-3
