"""FP8 linears (src/wan_dit_lab/quantization/fp8.py) on the HIP path.

Bars: the quantizers bit-exact against the oracle (fp8 bytes and fp32 scales), including the known answers of
tests/test_cache_fp8.py:150-158 on a row; the GEMM bit-exact where the fp32 accumulation is exact (small integer
values), within 2^-8 relative L2 and 1e-2 max-rel of the oracle otherwise (cuBLASLt's accumulation order is its
own: parity unpinned there); the reference's contract (tests/test_fp8.py:9-25): relative error < 0.06 against the
bf16 linear, and a weight changed in place is followed."""

import pytest
import torch

from oracle import fp8 as ofp8

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,K", [(1, 64), (37, 256), (1392, 3072), (130, 14336)])
def test_quantize_rows_bit_exact(gpu, dtype, M, K):
    from wdl import fp8

    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) * torch.rand(M, 1, generator=g) * 10).to(dtype)
    x[0, :8] = 0.0
    if M > 1:
        x[1] = 0.0  # an all-zero row: scale 1e-12 / 448
    q, s = fp8.quantize_rows(x.cuda())
    rq, rs = ofp8.quantize_rows(x)
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s.cpu(), rs)


def test_known_answer_row(gpu):
    """tests/test_cache_fp8.py:150-158: 84.021 -> 88 directly (never 80 through fp16), the 1.06251 / 1.06249
    midpoints, on an fp32 row whose maximum is 448 (scale 1)."""
    from wdl import fp8

    row = torch.tensor([[448.0, 84.021, -84.021, 1.06251, -1.06251, 1.06249, -1.06249, 0.0] * 2])
    q, s = fp8.quantize_rows(row.cuda())
    assert float(s) == 1.0
    assert torch.equal(q.cpu().view(torch.uint8), ofp8.quantize_rows(row)[0].view(torch.uint8))
    assert q.cpu().float()[0, 1] == 88.0


@pytest.mark.parametrize("M,K", [(5, 128), (1392, 3072)])
def test_quantize_tensor_bit_exact(gpu, M, K):
    from wdl import fp8

    g = torch.Generator().manual_seed(7)
    x = (torch.randn(M, K, generator=g) * 3).to(BF)
    q, s = fp8.quantize(x.cuda())
    rq, rs = ofp8.quantize(x)
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s.cpu(), rs)


@pytest.mark.parametrize("rows", [False, True])
@pytest.mark.parametrize("M,N", [(200, 256), (1392, 9216)])
def test_gemm_exact_on_integer_values(gpu, rows, M, N):
    """Operands whose fp8 values are small integers (scale 1: each row / the tensor holds 448): every fp32 sum is
    exact, so the result is the oracle's bit for bit whatever the accumulation order. (Only while the sums stay
    small: at K = 6144 with the 448 x 448 column the fp8 matrix cores' accumulation is off by a few units in
    ~2e5, which turns 0.5 % of the bf16 outputs by one ulp, in the one-pass launch as in stream-K.) 1392 x 9216
    runs the wide 256 x 128 tiles (396 of them), 200 x 256 the 128 x 128 ones."""
    from wdl import fp8

    g = torch.Generator().manual_seed(3)
    K = 512
    x = torch.randint(-3, 4, (M, K), generator=g).float()
    w = torch.randint(-3, 4, (N, K), generator=g).float()
    x[:, 0] = 448.0
    w[:, 0] = 448.0
    b = (torch.randn(N, generator=g) * 10).to(BF)
    q, s = fp8.quantize_padded(x.cuda(), rows)
    wq, ws = fp8.quantize_padded(w.cuda(), rows, pad=1)
    y = fp8.gemm(q, s, M, wq, ws, b.cuda(), rows).cpu()
    ref = (ofp8.w8a8_linear_rows if rows else ofp8.w8a8_linear_tensor)(x, w, b)
    ref = ref[0] if rows else ref
    assert torch.equal(y, ref)


@pytest.mark.parametrize("rows", [False, True])
@pytest.mark.parametrize("M,N,K", [(96, 512, 256), (1392, 3072, 3072), (1392, 9216, 1024), (1392, 3072, 14336)])
def test_gemm_matches_oracle(gpu, rows, M, N, K):
    """Against the oracle's W8A8 linear at the bars of the reference's FP8 tests, through the 128 x 128 tiles, the
    wide 256 x 128 tiles (1392 x 9216) and stream-K (FFN-down, K 14336), which must also agree with the one-pass
    launch to fp32 summation order."""
    from wdl import fp8

    g = torch.Generator().manual_seed(N)
    x = torch.randn(M, K, generator=g).to(BF)
    x[:, torch.randperm(K, generator=g)[:K // 100 + 1]] *= 20
    w = (torch.randn(N, K, generator=g) * 0.02).to(BF)
    b = (torch.randn(N, generator=g) * 0.02).to(BF)
    q, s = fp8.quantize_padded(x.cuda(), rows)
    wq, ws = fp8.quantize_padded(w.cuda(), rows, pad=1)
    y = fp8.gemm(q, s, M, wq, ws, b.cuda(), rows).cpu().float()
    ref = (ofp8.w8a8_linear_rows if rows else ofp8.w8a8_linear_tensor)(x, w, b)
    ref = (ref[0] if rows else ref).float()
    err = float((y - ref).abs().max()) / float(ref.abs().max())
    rel = float((y - ref).norm() / ref.norm())
    assert err <= 1e-2 and rel <= 2 ** -8, (err, rel)
    one = fp8.gemm(q, s, M, wq, ws, b.cuda(), rows, stream_k=False).cpu().float()
    # element by element: a bf16 ulp or two of fp32 summation order, nothing of a misplaced tile or piece
    assert bool(((y - one).abs() <= 2 ** -7 * one.abs() + 1e-3 * one.abs().max()).all())


@pytest.mark.parametrize("rows", [False, True])
def test_dynamic_linear_close_to_bf16_and_follows_the_weight(gpu, rows):
    """tests/test_fp8.py:9-25 on the HIP path: Linear(256, 512) in bf16, x [4, 96, 256]; relative error < 0.06,
    twice, the weight replaced in place in between."""
    from wdl.fp8 import DynamicFp8Linear

    torch.manual_seed(0)
    linear = torch.nn.Linear(256, 512, device="cuda", dtype=BF)
    layer = DynamicFp8Linear(linear, rows)
    x = torch.randn(4, 96, 256, device="cuda", dtype=BF)
    for _ in range(2):
        ref = linear(x).float()
        err = (layer(x).float() - ref).norm() / ref.norm()
        assert err < 0.06
        with torch.no_grad():
            linear.weight.copy_(torch.randn_like(linear.weight) * 0.05)


def test_fp8_packed_and_dynamic_tensor_modules_agree(gpu):
    """Fp8Linear (weight quantized once), PackedFp8Linear (over that FP8 weight, scale and bias) and
    DynamicFp8Linear(rows=False) compute the same bits; to_fp8 / to_dynamic_fp8 replace the linears in place."""
    from wdl import fp8

    torch.manual_seed(1)
    lin = torch.nn.Linear(384, 256, device="cuda", dtype=BF)
    x = torch.randn(2, 50, 384, device="cuda", dtype=BF)
    a = fp8.Fp8Linear(lin)(x)
    f = fp8.Fp8Linear(lin)
    b = fp8.PackedFp8Linear(f.weight, f.scale.reshape(()), f.bias)(x)
    c = fp8.DynamicFp8Linear(lin)(x)
    assert torch.equal(a, b) and torch.equal(a, c)
    seq = torch.nn.Sequential(torch.nn.Linear(128, 128, device="cuda", dtype=BF))
    fp8.to_fp8(seq)
    assert isinstance(seq[0], fp8.Fp8Linear)


def test_shapes_outside_the_tiles_are_rejected(gpu):
    from wdl import fp8

    lin = torch.nn.Linear(256, 100, device="cuda", dtype=BF)
    with pytest.raises(ValueError):
        fp8.DynamicFp8Linear(lin)(torch.randn(3, 256, device="cuda", dtype=BF))
