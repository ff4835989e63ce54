"""W4A4 on the HIP path against the oracle.

Bars (written in each test): activation quantizer — bit-exact int4 values and bf16 scales (the fused LayerNorm +
modulation variant too, with its bf16 input bit-exact to the oracle's ordered-reduction LayerNorm); GEMM integer
accumulators — bit-exact (unit scales, fp32 output equals the exact integer product); full GEMM — within 2^-20
relative of the float64 oracle in fp32, one bf16 rounding step in bf16; module-level — the reference's own tolerance
contracts (tests/test_w4a4.py:7-59)."""

import pytest
import torch

from oracle import norms as onorms
from oracle import w4a4 as ow

pytestmark = pytest.mark.gpu


def codes_to_int(q):
    """Activation operand (tile-blocked fp6 codes [R/128, K/64, 128, 48]) -> the integer values [R, K]."""
    from wdl import ops

    return ops.decode_acts(q.cpu())


def data(M, K, seed=0, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if outliers:
        idx = torch.randperm(K, generator=g)[: max(1, K // 100)]
        x[:, idx] *= 20
    return x.to(torch.bfloat16), g


@pytest.mark.parametrize("M,K", [(7, 128), (300, 256), (464, 3072), (130, 14336)])
@pytest.mark.parametrize("unsigned", [False, True])
def test_act_quant_bit_exact(gpu, M, K, unsigned):
    from wdl import ops

    x, g = data(M, K, seed=M + K)
    if unsigned:
        x = torch.nn.functional.gelu(x.float(), approximate="tanh").to(torch.bfloat16)
    smooth = (torch.rand(K, generator=g) + 0.5).to(torch.bfloat16)
    pdt = (torch.randn(32, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    shift = ow.GELU_SHIFT if unsigned else 0.0
    q, asc, lora = ops.act_quant_launch(x.cuda(), smooth.cuda(), pdt.cuda(), shift, unsigned)
    torch.cuda.synchronize()
    rq, rs = ow.act_quant(x, smooth, shift, unsigned)
    Mp = asc.shape[1]
    assert Mp % 128 == 0 and Mp >= M
    assert torch.equal(codes_to_int(q)[:M], rq)  # bar: bit-exact int4 values
    assert torch.equal(codes_to_int(q)[M:], torch.zeros(Mp - M, K, dtype=torch.int32))
    assert torch.equal(asc.cpu()[:, :M].t(), rs)  # bar: bit-exact bf16 scales
    ref_lora = ow.lora_down(x, pdt.t())
    err = (lora.cpu()[:M] - ref_lora).abs().max()
    assert float(err) <= 1e-5 * float(ref_lora.abs().max()) + 1e-6  # fp32 sums of exact bf16 products
    assert torch.all(lora.cpu()[M:] == 0)


@pytest.mark.parametrize("affine", [False, True])
def test_fused_layernorm_modulation_quant_bit_exact(gpu, affine):
    from wdl import ops

    M, K = 200, 3072
    x, g = data(M, K, seed=11)
    shift = torch.randn(K, generator=g) * 0.1
    scale = torch.randn(K, generator=g) * 0.1
    w = (torch.rand(K, generator=g) + 0.5) if affine else None
    b = (torch.randn(K, generator=g) * 0.1) if affine else None
    smooth = torch.ones(K, dtype=torch.bfloat16)
    pdt = (torch.randn(32, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    v_out = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")
    ln = dict(shift=shift.cuda(), scale=scale.cuda(), weight=None if w is None else w.cuda(),
              bias=None if b is None else b.cuda(), eps=1e-6)
    q, asc, lora = ops.act_quant_launch(x.cuda(), smooth.cuda(), pdt.cuda(), ln=ln, v_out=v_out)
    torch.cuda.synchronize()
    v = onorms.ln_mod(x, shift, scale, w, b, eps=1e-6)
    assert torch.equal(v_out.cpu(), v)  # bar: bit-exact bf16 normalized, modulated input
    rq, rs = ow.act_quant(v, smooth)
    assert torch.equal(codes_to_int(q)[:M], rq)
    assert torch.equal(asc.cpu()[:, :M].t(), rs)


@pytest.mark.parametrize("Mp,M,N,K,stream_k", [(1408, 1392, 3072, 3072, True), (384, 300, 384, 256, False),
                                               (512, 464, 512, 14336, True)])
def test_layernorm_partials_of_the_residual_epilogue(gpu, Mp, M, N, K, stream_k):
    """The gated-residual epilogue's LayerNorm chunk partials of the rows it writes, bit-exact to the oracle's
    partials of those rows, through each launch that runs the residual: the balanced form with its 32 x 32 pieces
    (1392 x 3072, K 3072), the one-pass tile, stream-K + merge (K 14336). Then the LayerNorm-fused quantizer of the
    new rows from those partials equals the quantizer forming them itself (and the oracle), bit for bit."""
    from wdl import ops, w4a4

    g = torch.Generator().manual_seed(M + N)
    qa = torch.randint(-7, 8, (Mp, K), generator=g, dtype=torch.int32)
    qw = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int32)
    asc = (torch.rand(K // 64, Mp, generator=g) * 0.3 + 0.01).to(torch.bfloat16)
    wsc = (torch.rand(K // 64, N, generator=g) * 0.01 + 1e-4).to(torch.bfloat16)
    lora = torch.randn(Mp, 32, generator=g)
    pu = (torch.randn(N, 32, generator=g) * 0.05).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16)
    X = (torch.randn(M, N, generator=g) * 2 + 0.5).to(torch.bfloat16)
    gate = torch.randn(N, generator=g)
    out = X.cuda().clone()
    part = torch.full((M, N // 32, 2), float("nan"), device="cuda")
    codes = ops.encode_acts(qa).cuda()
    ops.gemm_launch(codes, asc.cuda(), lora.cuda(), ops.as_codes(w4a4.pack_weight(qw).cuda(), K), wsc.cuda(),
                    pu.cuda(), bias.cuda(), M, out, ops.EPI_RESIDUAL, gate.cuda(), stream_k, ln_out=part)
    torch.cuda.synchronize()
    S, M2 = onorms.ln_chunk_partials(out.cpu())
    got = part.cpu().numpy()
    assert (got[..., 0] == S).all() and (got[..., 1] == M2).all()
    if N % 64 == 0 and N <= 4096:
        shift, scale = torch.randn(N, generator=g) * 0.1, torch.randn(N, generator=g) * 0.1
        smooth = (torch.rand(N, generator=g) + 0.5).to(torch.bfloat16)
        pdt = (torch.randn(32, N, generator=g) / N ** 0.5).to(torch.bfloat16)
        ln = dict(shift=shift.cuda(), scale=scale.cuda(), eps=1e-6)
        v1, v2 = (torch.empty(M, N, device="cuda", dtype=torch.bfloat16) for _ in range(2))
        a = ops.act_quant_launch(out, smooth.cuda(), pdt.cuda(), ln=dict(ln, partials=part), v_out=v1)
        b = ops.act_quant_launch(out, smooth.cuda(), pdt.cuda(), ln=ln, v_out=v2)
        torch.cuda.synchronize()
        assert torch.equal(v1, v2) and all(torch.equal(x, y) for x, y in zip(a, b))
        assert torch.equal(v1.cpu(), onorms.ln_mod(out.cpu(), shift, scale, eps=1e-6))


def launch_gemm(qa_int, asc, qweight, wsc, lora=None, pu=None, bias=None, M=None, epi=1, out=None, gate=None,
                stream_k=True):
    from wdl import ops

    Mp, K = qa_int.shape
    codes = ops.encode_acts(qa_int).cuda()
    N = qweight.shape[0]
    M = Mp if M is None else M
    if out is None:
        out = torch.empty(M, N, device="cuda", dtype=torch.float32 if epi == 1 else torch.bfloat16)
    c = lambda t: None if t is None else t.cuda()
    return ops.gemm_launch(codes, c(asc), c(lora), ops.as_codes(qweight.cuda(), K), c(wsc), c(pu), c(bias), M, out,
                           epi, c(gate), stream_k)


@pytest.mark.parametrize("N,K", [(128, 64), (384, 3072), (256, 14336)])
def test_weight_codes_are_the_fp6_codes_of_the_packed_integers(gpu, N, K):
    """wdl_w4a4_weight_codes: packed nibbles [N, K/2] -> tile-blocked fp6 codes (e3m2 of 2w) of [N, K], bit-exact
    against the format's statement (ops.encode_weights, itself checked on the closed form of e3m2)."""
    from wdl import ops, w4a4

    q = torch.randint(-8, 8, (N, K), generator=torch.Generator().manual_seed(N + K), dtype=torch.int32)
    codes = ops.weight_codes(w4a4.pack_weight(q).cuda()).cpu()
    want = ops.encode_weights(q)
    assert codes.shape == (N // 128, K // 64, 128, 48)
    assert torch.equal(codes, want)
    assert torch.equal(ops.decode_weights(codes), q)


@pytest.mark.parametrize("M,N,K", [(128, 128, 64), (256, 384, 512), (128, 256, 3072), (128, 128, 14336),
                                   (1408, 3072, 3072), (1408, 3072, 8192), (128, 256, 14336)])
def test_gemm_integer_accumulation_is_exact(gpu, M, N, K):
    """Unit scales, no low-rank, fp32 out: y must equal the exact integer product (bar: bit-exact)."""
    from wdl import w4a4

    g = torch.Generator().manual_seed(M + N + K)
    qa = torch.randint(-8, 8, (M, K), generator=g, dtype=torch.int32)
    qa[: M // 2, : K // 2] = torch.randint(0, 16, (M // 2, K // 2), generator=g)  # unsigned codes 8..15 too
    qw = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int32)
    ones_a = torch.ones(K // 64, M, dtype=torch.bfloat16)
    ones_w = torch.ones(K // 64, N, dtype=torch.bfloat16)
    y = launch_gemm(qa, ones_a, w4a4.pack_weight(qw), ones_w)
    torch.cuda.synchronize()
    exact = ow.int_gemm(qa, qw)
    assert torch.equal(y.cpu().double(), exact.double())


def test_scale_pairs_are_exact_for_every_fp16_and_bf16_scale(gpu):
    """The weight-scale operand: every finite fp16 value (all 63488 bit patterns) and every finite bf16 value split
    into bf16 hi + lo equal to it exactly (hi the truncation, lo the remainder); bf16 scales give (s, 0)."""
    from wdl import ops

    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    for dt in (torch.float16, torch.bfloat16):
        v = bits.view(dt)
        v = v[torch.isfinite(v.float())]
        pairs = ops.scale_pairs(v.cuda()).cpu()
        hi = (pairs & 0xFFFF).to(torch.int16).view(torch.bfloat16).float()
        lo = ((pairs >> 16) & 0xFFFF).to(torch.int16).view(torch.bfloat16).float()
        assert torch.equal(hi + lo, v.float())  # both exact bf16 values, their fp32 sum exact
        if dt == torch.bfloat16:
            assert torch.equal(hi, v.float()) and torch.all(lo == 0)
        else:
            assert torch.equal(hi, (v.float().view(torch.int32) & -65536).view(torch.float32))


@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K,valid", [(128, 256, 512, 100), (256, 128, 3072, 256), (1408, 384, 3072, 1392),
                                         (2688, 384, 3072, 2640)])
def test_gemm_scaled_lowrank_bias_matches_oracle(gpu, M, N, K, valid, sdt):
    """bf16 and fp16 weight scales (the two modes; fp16 goes through the exact hi + lo pair)."""
    from wdl import w4a4

    g = torch.Generator().manual_seed(7 + M)
    qa = torch.randint(-7, 8, (M, K), generator=g, dtype=torch.int32)
    qw = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int32)
    asc = (torch.rand(K // 64, M, generator=g) * 0.3 + 0.01).to(torch.bfloat16)
    wsc = (torch.rand(K // 64, N, generator=g) * 0.01 + 1e-4).to(sdt)
    lora = torch.randn(M, 32, generator=g)
    pu = (torch.randn(N, 32, generator=g) * 0.05).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16)
    y = launch_gemm(qa, asc, w4a4.pack_weight(qw), wsc, lora, pu, bias, M=valid, epi=1)
    yb = launch_gemm(qa, asc, w4a4.pack_weight(qw), wsc, lora, pu, bias, M=valid, epi=0)
    torch.cuda.synchronize()
    ref = ow.group_gemm(qa[:valid], asc.t()[:valid].float(), qw, wsc.t().float())
    ref += lora[:valid].to(torch.bfloat16).double() @ pu.double().t() + bias.double()
    scale = float(ref.abs().max())
    # fp32 result: fp32 rounding of ~K/64 fused steps (bar: 2^-20 of the output scale)
    assert float((y.cpu().double() - ref).abs().max()) <= 2 ** -20 * scale * (K // 64)
    # bf16 result: one bf16 rounding of that
    diff = (yb.cpu().double() - ref).abs()
    assert torch.all(diff <= ref.abs() * 2 ** -8 + 2 ** -20 * scale * (K // 64))


@pytest.mark.parametrize("M,N,K,valid", [(1024, 3072, 8192, 1000), (512, 512, 14336, 464), (1408, 3072, 14336, 1392),
                                         (1408, 3072, 6144, 1392), (1408, 3072, 3072, 1392), (1408, 3072, 2048, 1300),
                                         (2048, 2048, 1024, 2000), (2048, 4096, 3072, 2047)])
def test_gemm_split_k_matches_one_pass_and_oracle(gpu, M, N, K, valid):
    """Shapes whose tiles leave CUs idle run split in K when the library asks for a workspace: stream-K + merge
    (the first two shapes), or the balanced form on 256 CUs (whole tiles in two K halves; 264 tiles: 8 left over in
    128 pieces of 32 x 32, at K = 14336 (FFN-down at 1392 tokens: each wave's 28 groups of a piece in 5 batches),
    6144 (2 batches), 3072 and 2048 (one batch); 256 and 512 tiles: none left over, one and two tiles per CU). The
    result is
    deterministic, within fp32 rounding of the one-pass launch, and meets the oracle bar of the one-pass test; gated
    residual epilogue in place, bf16 and GELU outputs one rounding from the fp32 one."""
    from wdl import _lib, ops, w4a4

    assert _lib.library().wdl_w4a4_gemm_workspace_bytes(M, N, K) > 0  # the split path is the one under test
    g = torch.Generator().manual_seed(11 + M)
    qa = torch.randint(-7, 8, (M, K), generator=g, dtype=torch.int32)
    qw = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int32)
    asc = (torch.rand(K // 64, M, generator=g) * 0.3 + 0.01).to(torch.bfloat16)
    wsc = (torch.rand(K // 64, N, generator=g) * 0.01 + 1e-4).to(torch.bfloat16)
    lora = torch.randn(M, 32, generator=g)
    pu = (torch.randn(N, 32, generator=g) * 0.05).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16)
    X = torch.randn(valid, N, generator=g).to(torch.bfloat16)
    gate = torch.randn(N, generator=g)
    wq = w4a4.pack_weight(qw)
    y1 = launch_gemm(qa, asc, wq, wsc, lora, pu, bias, M=valid, epi=1)
    y2 = launch_gemm(qa, asc, wq, wsc, lora, pu, bias, M=valid, epi=1)
    y0 = launch_gemm(qa, asc, wq, wsc, lora, pu, bias, M=valid, epi=1, stream_k=False)
    outs = X.cuda().clone()
    launch_gemm(qa, asc, wq, wsc, lora, pu, bias, M=valid, epi=2, out=outs, gate=gate)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)  # deterministic
    ref = ow.group_gemm(qa[:valid], asc.t()[:valid].float(), qw, wsc.t().float())
    ref += lora[:valid].to(torch.bfloat16).double() @ pu.double().t() + bias.double()
    scale = float(ref.abs().max())
    bar = 2 ** -20 * scale * (K // 64)  # fp32 rounding of ~K/64 fused steps, as in the one-pass test
    assert float((y1.cpu().double() - ref).abs().max()) <= bar
    assert float((y1 - y0).abs().max()) <= bar
    expect = (X.float() + y1.cpu().to(torch.bfloat16).float() * gate).to(torch.bfloat16)
    assert torch.equal(outs.cpu(), expect)  # the residual epilogue of the split: bf16(x + bf16(y) gate)
    yb = launch_gemm(qa, asc, wq, wsc, lora, pu, bias, M=valid, epi=0)
    yg = launch_gemm(qa, asc, wq, wsc, lora, pu, bias, M=valid, epi=3)
    torch.cuda.synchronize()
    assert torch.equal(yb, y1.to(torch.bfloat16))
    hg = torch.nn.functional.gelu(y1.double(), approximate="tanh")
    assert float((yg.double() - hg).abs().max()) <= 2 ** -7 * float(hg.abs().max()) + 1e-6


def test_gemm_residual_and_gelu_epilogues(gpu):
    from wdl import w4a4

    M, N, K = 256, 256, 512
    g = torch.Generator().manual_seed(9)
    qa = torch.randint(-7, 8, (M, K), generator=g, dtype=torch.int32)
    qw = torch.randint(-8, 8, (N, K), generator=g, dtype=torch.int32)
    asc = (torch.rand(K // 64, M, generator=g) * 0.1).to(torch.bfloat16)
    wsc = (torch.rand(K // 64, N, generator=g) * 0.01).to(torch.bfloat16)
    bias = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16)
    ref = ow.group_gemm(qa, asc.t().float(), qw, wsc.t().float()) + bias.double()
    X = torch.randn(M, N, generator=g).to(torch.bfloat16)
    gate = torch.randn(N, generator=g)
    out = X.cuda().clone()
    launch_gemm(qa, asc, w4a4.pack_weight(qw), wsc, bias=bias, epi=2, out=out, gate=gate)
    h = launch_gemm(qa, asc, w4a4.pack_weight(qw), wsc, bias=bias, epi=3)
    torch.cuda.synchronize()
    expect = (X.float() + ref.float().to(torch.bfloat16).float() * gate).to(torch.bfloat16)
    assert float((out.cpu().float() - expect.float()).abs().max()) <= 2 ** -7 * float(expect.float().abs().max())
    hg = torch.nn.functional.gelu(ref, approximate="tanh")
    assert float((h.cpu().double() - hg).abs().max()) <= 2 ** -7 * float(hg.abs().max()) + 1e-6


def test_low_rank_weight_is_exact_and_smoothing_helps(gpu):
    # reference tests/test_w4a4.py:7-29
    from wdl import w4a4

    torch.manual_seed(0)
    M, K, N = 512, 1024, 768
    x = torch.randn(M, K, device="cuda", dtype=torch.bfloat16)
    x[:, :8] *= 20
    b = torch.randn(N, device="cuda") * 0.1

    def err(W, t):
        ref = x.float() @ W.t() + b
        return float((w4a4.linear(x, t).float() - ref).norm() / ref.norm())

    low = (torch.randn(N, 32, device="cuda") @ torch.randn(32, K, device="cuda")) * 0.01
    s = torch.rand(K, device="cuda") + 0.5
    assert err(low, w4a4.quantize(low, b, smooth=s)) < 0.01
    W = torch.randn(N, K, device="cuda") * 0.02
    plain = err(W, w4a4.quantize(W, b))
    smooth = err(W, w4a4.quantize(W, b, smooth=w4a4.smoothing(x.abs().amax(dim=0), W)))
    assert smooth < plain < 0.25


def test_gelu_mlp_is_the_feed_forward_and_needs_the_shift(gpu):
    # reference tests/test_w4a4.py:32-59
    from wdl import w4a4

    torch.manual_seed(0)
    M, K, H, N = 300, 256, 1024, 256
    x = torch.randn(M, K, device="cuda", dtype=torch.bfloat16)
    x[:, :4] *= 10
    W1, b1 = torch.randn(H, K, device="cuda") * 0.08, torch.randn(H, device="cuda") * 0.1
    W2, b2 = torch.randn(N, H, device="cuda") * 0.05, torch.randn(N, device="cuda") * 0.1
    gelu = torch.nn.GELU(approximate="tanh")
    h = gelu(x.float() @ W1.t() + b1)
    ref = h @ W2.t() + b2
    err = lambda y: float((y.float() - ref).norm() / ref.norm())
    offset = lambda y: float((y.float() - ref).mean(dim=0).norm() / ref.mean(dim=0).norm())
    s1 = w4a4.smoothing(x.abs().amax(dim=0), W1)
    t1 = w4a4.quantize(W1, b1, smooth=s1)
    s2 = w4a4.smoothing(h.abs().amax(dim=0) + w4a4.GELU_SHIFT, W2)
    unfused = w4a4.linear(gelu(w4a4.linear(x, t1).float()).to(torch.bfloat16), w4a4.quantize(W2, b2, smooth=s2))
    fused = w4a4.gelu_mlp(x, t1, w4a4.quantize(W2, b2, smooth=s2, shift=w4a4.GELU_SHIFT))
    uncorrected = w4a4.gelu_mlp(x, t1, w4a4.quantize(W2, b2, smooth=s2))
    assert err(fused) < 0.2 and err(fused) < err(unfused)
    assert offset(fused) < 1.1 * offset(unfused) and offset(uncorrected) > 1.5 * offset(fused)


def test_linear_end_to_end_matches_oracle(gpu):
    from wdl import w4a4

    M, K, N = 300, 512, 384
    x, g = data(M, K, seed=21)
    W = torch.randn(N, K, generator=g) * 0.02
    b = torch.randn(N, generator=g) * 0.02
    s = w4a4.smoothing(x.float().abs().amax(0), W)
    host = w4a4.quantize(W, b, smooth=s)
    ref_t = ow.quantize_weight(W, b, smooth=s)
    y = w4a4.linear(x.cuda(), {k: v.cuda() for k, v in host.items()})
    torch.cuda.synchronize()
    ref = ow.linear_parts(x, ref_t)[0]
    diff = (y.cpu().double() - ref).abs()
    assert torch.all(diff <= ref.abs() * 2 ** -8 + 1e-4 * float(ref.abs().max()))


def test_live_names_module_and_bare_op_agree(gpu):
    """torch.ops.live.w4a4_linear (the reference's call site), PackedW4A4Linear (weights expanded once) and
    wdl::w4a4_linear on packed nibbles (expanded per call) give the same bits."""
    from wdl import w4a4
    import wdl.live  # noqa: F401

    g = torch.Generator(device="cuda").manual_seed(11)
    t = w4a4.random_parts(384, 512, "cuda", g)
    x = torch.randn(200, 512, device="cuda", generator=g).to(torch.bfloat16)
    a = torch.ops.live.w4a4_linear(x, *(t[p] for p in w4a4.PARTS))
    b = w4a4.PackedW4A4Linear(**t)(x)
    c = w4a4.linear(x, t)
    assert torch.equal(a, b) and torch.equal(a, c)


@pytest.mark.parametrize("M,K,N", [(300, 256, 1024), (1392, 3072, 14336)])
def test_fused_gelu_quant_epilogue_on_the_kernels_own_sums(gpu, M, K, N):
    """The fused GELU MLP's first GEMM (wdl_w4a4_gemm_gelu_quant) against the oracle's second-layer inputs computed
    from the same GEMM's fp32 result y (the plain launch with an fp32 output, identical sums): h = GELU_tanh(y) in
    fp32, u = (h + 0.171875) / s2, unsigned int4 per 64-group, lora2 = h . proj_down2. The kernel's GELU and
    torch's differ in the last bits (an exp-based tanh against tanhf), so a value on a rounding boundary may land
    one step apart: bar — scales bit-equal except at most 0.1 % of groups (those one bf16 ulp apart), codes equal
    where the scales are except at most 0.01 % of values (those one step apart); lora2 within 1e-5 relative L2 (h
    split into two bf16 parts: ~16 significant bits); padding rows zero. At 1392 x 3072 -> 14336 this is the
    step's FFN-up shape."""
    from wdl import ops

    g = torch.Generator().manual_seed(N + M)
    x, _ = data(M, K, seed=M)
    from oracle.block import random_logical

    t1 = random_logical(N, K, g)
    s2 = (torch.rand(N, generator=g) + 0.5).to(torch.bfloat16)
    pd2 = (torch.randn(N, 32, generator=g) / N ** 0.5).to(torch.bfloat16)
    from wdl import w4a4

    p1 = w4a4.pack_parts(t1, "cuda")
    wcodes = ops.weight_codes(p1["qweight"])
    qa = ops.act_quant_launch(x.cuda(), p1["smooth"], p1["proj_down"])
    y = torch.empty(M, N, device="cuda", dtype=torch.float32)
    ops.gemm_launch(*qa, wcodes, p1["wscales"], p1["proj_up"], p1["bias"], M, y, ops.EPI_F32, stream_k=False)
    q2, asc2, lora2 = ops.gelu_quant_launch(*qa, wcodes, p1["wscales"], p1["proj_up"], p1["bias"], M, s2.cuda(),
                                            pd2.t().contiguous().cuda())
    torch.cuda.synchronize()
    h = ow.gelu_tanh(y.cpu())
    rq, rs = ow.act_quant(h, s2, ow.GELU_SHIFT, True)
    rl = ow.lora_down(h, pd2)
    Mp = asc2.shape[1]
    q = codes_to_int(q2)
    sc = asc2.cpu().t()
    assert torch.all(q[M:] == 0) and torch.all(sc[M:].float() == 0) and torch.all(lora2.cpu()[M:] == 0)
    sb, rb = sc[:M].contiguous().view(torch.int16).int(), rs.view(torch.int16).int()
    scale_diff = (sb != rb)
    assert int((sb - rb).abs().max()) <= 1
    assert float(scale_diff.float().mean()) <= 1e-3
    same = ~scale_diff.repeat_interleave(64, dim=1)
    dq = (q[:M] - rq)[same]
    print(f"M={M} N={N}: scales differing {int(scale_diff.sum())} of {scale_diff.numel()}, codes differing "
          f"{int((dq != 0).sum())} of {dq.numel()}")
    assert int(dq.abs().max()) <= 1 and float((dq != 0).float().mean()) <= 1e-4
    assert float((lora2.cpu()[:M] - rl).norm() / rl.norm()) <= 1e-5


def test_fused_gelu_mlp_matches_oracle_at_the_block_shapes(gpu):
    """wdl::w4a4_gelu_mlp (fused epilogue, then the second GEMM) against the oracle's gelu_mlp (fp32 hidden layer)
    at 464 tokens, 3072 -> 14336 -> 3072, random-init parts with the shift-corrected second-layer bias: bar —
    max-rel-err 1e-2 and relative L2 1e-3 (the GELU last-bit differences of the epilogue test, propagated)."""
    from wdl import w4a4

    g = torch.Generator().manual_seed(31)
    x, _ = data(464, 3072, seed=31)
    from oracle.block import random_logical

    t1, t2 = random_logical(14336, 3072, g), random_logical(3072, 14336, g, shift=ow.GELU_SHIFT)
    ref = ow.gelu_mlp(x, t1, t2)
    y = w4a4.gelu_mlp(x.cuda(), w4a4.pack_parts(t1, "cuda"), w4a4.pack_parts(t2, "cuda")).cpu()
    err = float((y.float() - ref.float()).abs().max()) / float(ref.float().abs().max())
    rel = float((y.float() - ref.float()).norm() / ref.float().norm())
    print(f"fused GELU MLP vs oracle: max-rel-err {err:.2e}, rel-L2 {rel:.2e}")
    assert err <= 1e-2 and rel <= 1e-3
