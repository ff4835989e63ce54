"""The W4A4 oracle and the host-side packing on the CPU: the reference's closed forms and tolerance contracts
(tests/test_w4a4.py:163-191) and brute-force nearest-grid checks of both quantizers."""

import numpy as np
import pytest
import torch

from oracle import norms as onorms
from oracle import w4a4 as ow


def test_int4_max_rule_is_the_reference_closed_form():
    # reference tests/test_w4a4.py:175-176
    torch.manual_seed(0)
    R = torch.distributions.StudentT(3.0).sample((128, 512))
    q, s = ow.int4_groups(R, "max")
    assert torch.equal(q, torch.round(R.view(128, -1, 64) / s[..., None]).clamp(-8, 7).to(torch.int32).view(128, 512))


def test_int4_values_are_the_nearest_grid_points():
    torch.manual_seed(1)
    R = torch.randn(64, 256) * torch.rand(64, 1) * 3
    q, s = ow.int4_groups(R)
    x = (R.view(64, -1, 64) / s[..., None]).view(64, 256).double()
    grid = torch.arange(-8, 8, dtype=torch.float64)
    d = (x[..., None] - grid).abs()
    best = d.min(-1).values
    assert torch.all((x - q.double()).abs() <= best + 1e-12)  # q is a nearest grid point
    assert q.min() >= -7 and q.max() <= 7  # the max rule never reaches -8


def test_mse_scales_fit_heavy_tails_better():
    # reference tests/test_w4a4.py:163-174
    torch.manual_seed(0)
    R = torch.distributions.StudentT(3.0).sample((128, 512))
    back = lambda q, s: (q.view(128, -1, 64).float() * s[..., None]).view(128, 512)
    err = lambda q, s: float(((R - back(q, s)) ** 2).sum())
    qm, sm = ow.int4_groups(R, "max")
    qe, se = ow.int4_groups(R, "mse")
    assert qe.min() >= -8 and qe.max() <= 7
    assert err(qe, se) < 0.9 * err(qm, sm)


@pytest.mark.parametrize("unsigned", [False, True])
def test_activation_quantizer_is_nearest_grid_with_bf16_scale(unsigned):
    g = torch.Generator().manual_seed(2)
    x = torch.randn(40, 256, generator=g)
    x[:, :3] *= 20
    if unsigned:
        x = torch.nn.functional.gelu(x, approximate="tanh")
    x = x.to(torch.bfloat16)
    smooth = (torch.rand(256, generator=g) + 0.5).to(torch.bfloat16)
    shift = ow.GELU_SHIFT if unsigned else 0.0
    q, sc = ow.act_quant(x, smooth, shift, unsigned)
    v = ((x.float() + shift) / smooth.float()).view(40, 4, 64)
    amax = v.abs().amax(-1)
    assert torch.equal(sc, (amax / (15. if unsigned else 7.)).to(torch.bfloat16))
    u = (v / sc.float()[..., None]).view(40, 256).double()
    lo, hi = (0, 15) if unsigned else (-8, 7)
    grid = torch.arange(lo, hi + 1, dtype=torch.float64)
    best = (u[..., None] - grid).abs().min(-1).values
    assert torch.all((u - q.double()).abs() <= best + 1e-12)
    assert q.min() >= lo and q.max() <= hi


def test_group_gemm_integer_part_is_exact():
    g = torch.Generator().manual_seed(3)
    qa = torch.randint(-8, 8, (33, 192), generator=g)
    qw = torch.randint(-8, 8, (40, 192), generator=g)
    ones_a, ones_w = torch.ones(33, 3), torch.ones(40, 3)
    y = ow.group_gemm(qa, ones_a, qw, ones_w)
    assert torch.equal(y.long(), ow.int_gemm(qa, qw))


def test_host_pack_roundtrip_and_quantize_matches_oracle():
    from wdl import w4a4

    g = torch.Generator().manual_seed(4)
    q = torch.randint(-8, 8, (48, 256), generator=g, dtype=torch.int32)
    p = w4a4.pack_weight(q)
    assert p.shape == (48, 128) and p.dtype == torch.uint8
    assert torch.equal(w4a4.unpack_weight(p), q)
    # byte j of group 0: low nibble k = j, high nibble k = j + 32
    assert int(p[0, 5]) == ((int(q[0, 5]) & 0xF) | ((int(q[0, 37]) & 0xF) << 4))
    W = torch.randn(96, 256, generator=g) * 0.02
    b = torch.randn(96, generator=g) * 0.1
    s = torch.rand(256, generator=g) + 0.5
    for rule in ("max", "mse"):
        host = w4a4.quantize(W, b, smooth=s, shift=ow.GELU_SHIFT, rule=rule)
        ref = ow.quantize_weight(W, b, smooth=s, shift=ow.GELU_SHIFT, rule=rule)
        assert torch.equal(w4a4.unpack_weight(host["qweight"]), ref["q"])
        assert torch.equal(host["wscales"].t(), ref["wscales"])
        assert torch.equal(host["bias"], ref["bias"])
        assert torch.equal(host["proj_down"].t(), ref["proj_down"])
        assert torch.equal(host["proj_up"], ref["proj_up"])


def test_int4_groups_host_equals_oracle():
    from wdl import w4a4

    torch.manual_seed(5)
    R = torch.distributions.StudentT(3.0).sample((64, 512))
    for rule in ("max", "mse"):
        assert torch.equal(w4a4.int4_groups(R, rule)[0], ow.int4_groups(R, rule)[0])


def test_ordered_row_sum_equals_scalar_loop():
    g = torch.Generator().manual_seed(6)
    x = (torch.randn(3, 1024, generator=g) * 10).numpy().astype(np.float32)
    got = onorms._ordered_sum(x)
    for r in range(3):
        lanes = []
        for lane in range(64):
            s = np.float32(0)
            for c in range(lane, 1024 // 8, 64):
                for j in range(8):
                    s = np.float32(s + x[r, 8 * c + j])
            lanes.append(s)
        for o in (32, 16, 8, 4, 2, 1):
            lanes = [np.float32(lanes[i] + lanes[i ^ o]) for i in range(64)]
        assert got[r] == lanes[0]


def test_ln_mod_and_rms_close_to_torch():
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(5, 3072, generator=g) * 2 + 0.3).to(torch.bfloat16)
    shift, scale = torch.randn(3072, generator=g) * 0.1, torch.randn(3072, generator=g) * 0.1
    got = onorms.ln_mod(x, shift, scale).float()
    ref = torch.nn.functional.layer_norm(x.float(), (3072,), eps=1e-6) * (1 + scale) + shift
    assert float((got - ref).abs().max()) <= 2 ** -7 * float(ref.abs().max())
    w = (torch.rand(3072, generator=g) + 0.5).to(torch.bfloat16)
    r = onorms.rms_norm(x, w).float()
    rref = x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
    assert float((r - rref).abs().max()) <= 2 ** -7 * float(rref.abs().max())
