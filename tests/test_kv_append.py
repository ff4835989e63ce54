"""wdl_kv_append_fp8 against the oracle's quantize_rows: the reference's contract tests
(tests/test_cache_fp8.py:28-129, 150-158) on the HIP path. Bar: bit-exact fp8 bytes and fp32 scales."""

import pytest
import torch

from oracle.fp8 import quantize_rows

pytestmark = pytest.mark.gpu


def buffers(batch, tokens, heads, dim):
    shape = (batch, tokens, heads, dim)
    return (torch.full(shape, 2., device="cuda").to(torch.float8_e4m3fn),
            torch.full((batch, tokens, heads, 1), 7., device="cuda"),
            torch.full(shape, -2., device="cuda").to(torch.float8_e4m3fn),
            torch.full((batch, tokens, heads, 1), 9., device="cuda"))


def compare_bits(actual, expected):
    actual, expected = actual.cpu(), expected.cpu()
    if actual.dtype == torch.float8_e4m3fn:
        assert torch.equal(actual.view(torch.uint8), expected.view(torch.uint8))
    else:
        assert torch.equal(actual, expected)


def oracle_rows(x):
    return quantize_rows(x.cpu())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("batch,heads,dim", [(1, 2, 64), (2, 3, 128), (1, 1, 160), (1, 24, 128)])
def test_bitwise_values_scales_and_untouched_cache(gpu, dtype, batch, heads, dim):
    from wdl.cache_fp8 import store_kv_fp8

    torch.manual_seed(23)
    k = torch.randn(batch, 7, heads, dim, device="cuda", dtype=dtype)
    v = torch.randn_like(k) * 3
    actual = buffers(batch, 17, heads, dim)
    expected = [t.cpu().clone() for t in actual]
    for x, ci, si in ((k, 0, 1), (v, 2, 3)):
        q, s = oracle_rows(x)
        expected[ci][:, 5:12], expected[si][:, 5:12] = q, s
    before_k, before_v = k.clone(), v.clone()
    store_kv_fp8(k, v, *actual, 5)
    torch.cuda.synchronize()
    for left, right in zip(actual, expected):
        compare_bits(left, right)
    compare_bits(k, before_k)
    compare_bits(v, before_v)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_zero_tiny_large_and_fp8_rounding_boundaries(gpu, dtype):
    from wdl.cache_fp8 import store_kv_fp8

    values = torch.tensor([0., -0., 1e-15, -1e-15, .5, -.5, 1., -1., 3., -3., 448., -448.],
                          device="cuda").to(dtype)
    k = values.repeat(8).reshape(1, 1, 1, 96)
    v = torch.zeros_like(k)
    actual = buffers(1, 3, 1, 96)
    store_kv_fp8(k, v, *actual, 1)
    for x, cache, scales in ((k, actual[0], actual[1]), (v, actual[2], actual[3])):
        q, scale = oracle_rows(x)
        compare_bits(cache[:, 1:2], q)
        compare_bits(scales[:, 1:2], scale)


def test_fp32_values_around_fp8_midpoints_do_not_round_through_fp16(gpu):
    from wdl.cache_fp8 import store_kv_fp8

    k = torch.tensor([448., 84.021, -84.021, 1.06251, -1.06251, 1.06249, -1.06249, 0.],
                     device="cuda").reshape(1, 1, 1, 8)
    actual = buffers(1, 3, 1, 8)
    store_kv_fp8(k, k, *actual, 1)
    q, scale = oracle_rows(k)
    compare_bits(actual[0][:, 1:2], q)
    compare_bits(actual[1][:, 1:2], scale)
    assert actual[0][0, 1, 0, 1].float().item() == 88.0


def test_every_fp8_code_and_midpoint_bitwise(gpu):
    """All e4m3 magnitudes and all midpoints between them, scaled so the row max is exactly 448 (scale 1)."""
    from wdl.cache_fp8 import store_kv_fp8

    codes = torch.arange(0, 127, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    mids = (codes[1:] + codes[:-1]) / 2
    row = torch.cat([codes, -codes, mids, -mids, torch.tensor([448.])])
    pad = (-row.numel()) % 8
    row = torch.cat([row, torch.zeros(pad)]).reshape(1, 1, 1, -1).cuda()
    D = row.shape[-1]
    actual = buffers(1, 1, 1, D)
    store_kv_fp8(row, row, *actual, 0)
    q, s = oracle_rows(row)
    compare_bits(actual[0], q)
    compare_bits(actual[1], s)


def test_strided_inputs_mixed_dtypes_and_nondefault_stream(gpu):
    from wdl.cache_fp8 import store_kv_fp8

    k = torch.randn(2, 5, 3, 256, device="cuda", dtype=torch.float32)[..., ::2]
    v = torch.randn(2, 10, 3, 128, device="cuda", dtype=torch.bfloat16)[:, ::2]
    actual = buffers(2, 11, 3, 128)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        store_kv_fp8(k, v, *actual, 6)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for x, cache, scales in ((k, actual[0], actual[1]), (v, actual[2], actual[3])):
        q, scale = oracle_rows(x)
        compare_bits(cache[:, 6:], q)
        compare_bits(scales[:, 6:], scale)


def test_graph_capture_replays(gpu):
    from wdl.cache_fp8 import store_kv_fp8

    k = torch.randn(1, 7, 2, 128, device="cuda", dtype=torch.bfloat16)
    v, actual = torch.randn_like(k), buffers(1, 12, 2, 128)
    store_kv_fp8(k, v, *actual, 4)  # warm up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        store_kv_fp8(k, v, *actual, 4)
    for _ in range(3):
        k.copy_(torch.randn_like(k))
        v.copy_(torch.randn_like(v))
        graph.replay()
        torch.cuda.synchronize()
        for x, cache, scales in ((k, actual[0], actual[1]), (v, actual[2], actual[3])):
            q, scale = oracle_rows(x)
            compare_bits(cache[:, 4:11], q)
            compare_bits(scales[:, 4:11], scale)


@pytest.mark.parametrize("problem", ["negative", "overflow", "shape", "cache_dtype", "scale_dtype", "grad",
                                     "noncontiguous"])
def test_invalid_contract_rejected_before_write(gpu, problem):
    from wdl.cache_fp8 import store_kv_fp8

    k = torch.randn(1, 5, 2, 128, device="cuda")
    v, actual, offset = k.clone(), list(buffers(1, 8, 2, 128)), 1
    before = [t.clone() for t in actual]
    if problem == "negative":
        offset = -1
    elif problem == "overflow":
        offset = 4
    elif problem == "shape":
        v = v[:, :3]
    elif problem == "cache_dtype":
        actual[0] = actual[0].float()
    elif problem == "scale_dtype":
        actual[1] = actual[1].half()
    elif problem == "grad":
        k.requires_grad_()
    else:
        actual[1] = torch.full((1, 2, 8, 1), 7., device="cuda").transpose(1, 2)
    with pytest.raises((ValueError, TypeError)):
        store_kv_fp8(k, v, *actual, offset)
    torch.cuda.synchronize()
    for a, b in zip(actual, before):
        if a.dtype == b.dtype and a.shape == b.shape:
            compare_bits(a, b)
