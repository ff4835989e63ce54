"""The FP8 weight-only linear (wdl_fp8wo_gemm) on the GPU against oracle/fp8.w8a16_linear: the weight quantized to
e4m3 per output row (or per tensor), the activation bf16. The kernel sums the exact products in fp32 and the oracle
in float64, so a bf16 output can round to the neighbouring value where the fp32 sum lands next to a rounding
boundary, and where the sum cancels to near zero the fp32 error is large relative to it. Bar: every output within
its bf16 rounding (2^-8 relative) plus the rigorous fp32 summation bound gamma_K * scale * sum_k |x_k w_k| of the
float64 value, and at least 99.5 % of the outputs equal to the oracle's bf16. Shapes: the attention projections at
1392 and 2640 tokens (QKV 3072 -> 9216, o 3072 -> 3072), ragged M, one token, the gated residual epilogue."""

import pytest
import torch

from oracle import fp8 as ofp8

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def check(got: torch.Tensor, x: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor, b, want: torch.Tensor):
    """got within bf16 rounding + the fp32 summation bound of the float64 result; returns the equal fraction."""
    K = x.shape[1]
    s = ws.reshape(1, -1).double()
    y64 = (x.double() @ wq.double().t()) * s + (0 if b is None else b.double())
    terms = (x.double().abs() @ wq.double().abs().t()) * s
    gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    err = (got.double() - y64).abs()
    bound = 2.0 ** -8 * y64.abs() + gamma * terms + 1e-30
    assert bool((err <= bound).all()), float((err / bound).max())
    return float((got.view(torch.int16) == want.view(torch.int16)).float().mean())


@pytest.mark.parametrize("M,N,K,rows", [(1392, 9216, 3072, True), (2640, 3072, 3072, True), (130, 256, 192, True),
                                        (1, 128, 64, False), (700, 384, 1024, False)])
def test_weight_only_gemm_matches_oracle(gpu, M, N, K, rows):
    from wdl import fp8

    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=g).to(BF)
    W = torch.randn(N, K, generator=g) * 0.05
    b = (torch.randn(N, generator=g) * 0.1).to(BF)
    wq, ws = ofp8.quantize_rows(W) if rows else ofp8.quantize(W)
    want = ofp8.w8a16_linear(x, wq, ws, b)
    got = fp8.weight_only_gemm(x.cuda(), wq.cuda(), ws.reshape(-1).float().cuda(), b.cuda()).cpu()
    equal = check(got, x, wq, ws, b, want)
    print(f"{M}x{N}x{K} rows={rows}: {100 * equal:.3f} % equal to the oracle's bf16")
    assert equal >= 0.995


def test_weight_only_residual_epilogue_and_module(gpu):
    """The gated residual out = bf16(out + bf16(y) gate) in place, and Fp8WeightOnlyLinear on an nn.Linear (its own
    row quantizer gives the oracle's codes and scales)."""
    from wdl import fp8

    g = torch.Generator().manual_seed(11)
    M, N, K = 464, 3072, 3072
    x = torch.randn(M, K, generator=g).to(BF)
    lin = torch.nn.Linear(K, N)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        lin.bias.copy_(torch.randn(N, generator=g) * 0.1)
    wq, ws = ofp8.quantize_rows(lin.weight.detach())
    y = ofp8.w8a16_linear(x, wq, ws, lin.bias.detach().to(BF))
    res = torch.randn(M, N, generator=g).to(BF)
    gate = torch.rand(N, generator=g)
    want = (res.float() + y.float() * gate).to(BF)
    out = res.cuda()
    fp8.weight_only_gemm(x.cuda(), wq.cuda(), ws.reshape(-1).cuda(), lin.bias.detach().cuda(), out=out,
                         gate=gate.cuda())
    # the residual: y rounded to bf16, times the gate, added to the residual (each rounding at most half a step)
    assert float((out.cpu().float() - want.float()).abs().max()) <= float(2 ** -7 * (res.float().abs() +
                                                                                      y.float().abs()).max())
    assert float((out.cpu() == want).float().mean()) >= 0.99
    b = lin.bias.detach().to(BF).clone()
    mod = fp8.Fp8WeightOnlyLinear(lin.cuda())
    assert torch.equal(mod.weight.cpu().view(torch.uint8), wq.view(torch.uint8))
    got = mod(x.cuda()[None]).cpu()[0]
    assert check(got, x, wq, ws, b, y) >= 0.995
