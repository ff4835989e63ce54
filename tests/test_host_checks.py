"""Host-side argument checks that run before any launch (CPU tensors: nothing reaches the library)."""

import pytest
import torch

FP8 = torch.float8_e4m3fn


def _attend_args(H=2, cap=64, n=16):
    Q = torch.zeros(1, n, H, 128, dtype=torch.bfloat16)
    K = torch.zeros(1, n, H, 128, dtype=torch.bfloat16)
    V = torch.zeros(1, n, H, 128, dtype=torch.bfloat16)
    ck = torch.zeros(1, cap, H, 128, dtype=FP8)
    cs = torch.ones(1, cap, H, 1)
    return Q, ck, cs, ck.clone(), cs.clone(), K, V


def test_sage_attend_rejects_strided_or_misshaped_caches():
    from wdl.sage_kv import _check

    Q, ck, cks, cv, cvs, K, V = _attend_args()
    _check(Q, ck, cks, cv, cvs, 8, K, V)  # well formed
    wide = torch.zeros(1, 64, 4, 128, dtype=FP8)
    with pytest.raises(ValueError, match="contiguous"):  # a head slice of a wider cache: strided rows
        _check(Q, wide[:, :, :2], cks, wide[:, :, 2:], cvs, 8, K, V)
    with pytest.raises(ValueError, match="batch 1"):
        _check(Q, torch.zeros(2, 64, 2, 128, dtype=FP8), cks, torch.zeros(2, 64, 2, 128, dtype=FP8), cvs, 8, K, V)
    with pytest.raises(ValueError, match="one scale per cache row"):
        _check(Q, ck, torch.ones(1, 64, 2), cv, cvs, 8, K, V)
    with pytest.raises(ValueError, match="contiguous"):
        _check(Q, ck, torch.ones(1, 64, 2, 2)[..., :1], cv, cvs, 8, K, V)
    with pytest.raises(ValueError, match="at outside"):
        _check(Q, ck, cks, cv, cvs, 65, K, V)


def test_weight_only_gemm_refuses_views_and_mismatched_parts():
    """fp8.weight_only_gemm reads the weight as dense [N, K] rows: a transposed or sliced e4m3 weight, a bias or
    gate of the wrong length, a misshaped out and tensors on different devices are refused before any launch."""
    from wdl.fp8 import weight_only_gemm

    M, N, K = 16, 128, 64
    x = torch.zeros(M, K, dtype=torch.bfloat16)
    w = torch.zeros(N, K, dtype=FP8)
    s = torch.ones(N)
    b = torch.zeros(N, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="contiguous e4m3"):
        weight_only_gemm(x, torch.zeros(K, N, dtype=FP8).t(), s, b)
    with pytest.raises(ValueError, match="contiguous e4m3"):
        weight_only_gemm(x, torch.zeros(N, 2 * K, dtype=FP8)[:, :K], s, b)
    with pytest.raises(ValueError, match="bias"):
        weight_only_gemm(x, w, s, torch.zeros(N - 1, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="out must be"):
        weight_only_gemm(x, w, s, b, out=torch.zeros(M, N + 1, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="gate"):
        weight_only_gemm(x, w, s, b, out=torch.zeros(M, N, dtype=torch.bfloat16), gate=torch.ones(N - 1))
    with pytest.raises(ValueError, match="device"):
        weight_only_gemm(x, w, s.to("meta"), b)
