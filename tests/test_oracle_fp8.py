"""The oracle's FP8 rule against the reference's known answers (tests/test_cache_fp8.py:47-58, 150-158, kept as data in
tests/golden/fp8_known_answers.json) and an independent brute-force nearest-value search over the e4m3 codes."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import fp8

KNOWN = json.loads((Path(__file__).parent / "golden" / "fp8_known_answers.json").read_text())


def test_fp32_midpoints_known_answers():
    m = KNOWN["midpoint_row"]
    q, scale = fp8.quantize_rows(torch.tensor(m["values"]).reshape(1, 1, 1, -1))
    assert float(scale) == m["scale"]
    assert q.float().flatten().tolist() == m["expected"]
    assert float(torch.tensor(84.021).half().float().to(fp8.FP8).float()) == 80.0  # the fp16 path it avoids


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_boundary_row_known_answers(dtype):
    b = KNOWN["boundary_row"]
    q, scale = fp8.quantize_rows(torch.tensor(b["values"] * b["repeat"]).to(dtype).reshape(1, 1, 1, -1))
    assert float(scale) == b["scale"]
    assert q.view(torch.uint8).flatten()[:4].tolist() == b["bits_first4"]  # +0, -0, tiny -> signed zero
    assert q.float().flatten()[4:12].tolist() == b["values_4_to_12"]


def test_torch_conversion_equals_brute_force_nearest():
    vals = fp8.e4m3_values()
    finite = np.sort(vals[np.isfinite(vals) & (vals >= 0)])
    mids = (finite[1:] + finite[:-1]) / 2  # every tie point: must go to the even code
    rng = np.random.default_rng(0)
    samples = np.concatenate([
        mids, -mids, finite, -finite,
        rng.standard_normal(4000) * 50, rng.uniform(-470, 470, 2000), rng.uniform(-0.02, 0.02, 2000),
        np.array([449., 463.9, 464., 464.1, 479.9, 480., 1000., -464.1]),
    ]).astype(np.float32)
    torch_bits = fp8.e4m3_bits(torch.from_numpy(samples)).numpy()
    brute = fp8.e4m3_nearest(samples)
    nan_t = np.isnan(fp8.e4m3_values()[torch_bits])
    nan_b = np.isnan(fp8.e4m3_values()[brute])
    assert np.array_equal(nan_t, nan_b)
    assert np.array_equal(torch_bits[~nan_t], brute[~nan_b])


def test_rows_scale_is_amax_over_448_and_values_reconstruct():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 7, 3, 128, generator=g).to(torch.bfloat16)
    q, s = fp8.quantize_rows(x)
    assert torch.equal(s, (x.abs().amax(-1, keepdim=True).float() / 448))
    assert torch.equal(q.float().abs().amax(-1), torch.full((5, 7, 3), 448.))  # the row max lands on 448
    rel = ((q.float() * s) - x.float()).abs() / x.float().abs().clamp(min=1e-3)
    assert float(rel[x.float().abs() > s * 2 ** -6 * 448].max()) <= 2 ** -4  # e4m3: 3 mantissa bits, half-ulp


def test_weight_only_linear_known_answer():
    """w8a16_linear with x the identity: row k of the result is column k of the dequantized weight (times its row
    scale) plus the bias, so a transposed weight or a dropped scale fails."""
    from oracle import fp8 as ofp8

    g = torch.Generator().manual_seed(2)
    W = torch.randn(128, 64, generator=g)
    wq, ws = ofp8.quantize_rows(W)
    b = torch.randn(128, generator=g).to(torch.bfloat16)
    y = ofp8.w8a16_linear(torch.eye(64).to(torch.bfloat16), wq, ws, b)
    want = (wq.float() * ws).t() + b.float()
    assert torch.equal(y, want.to(torch.bfloat16))
    # the codes are the nearest e4m3 values of W / scale (the brute-force search)
    assert np.array_equal(wq.view(torch.uint8).numpy().ravel(), ofp8.e4m3_nearest((W / ws).numpy()))
