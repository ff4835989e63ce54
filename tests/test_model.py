"""The model edges and the DMD schedule on the CPU (wdl/model.py against oracle/model.py and the closed forms).

Bars: the noise levels equal the reference's fixture (tests/test_causal_schedule.py:14) to 1e-15; the patch
embedding is the convolution (torch conv3d) to one bf16 rounding (the GEMM's fp32 sum against fp64); unpatchify
inverts the patch order exactly and equals an explicit index loop; the time features equal their closed form;
the time embedding and the Head match the oracle to one bf16 rounding per linear."""

import math

import torch

from oracle import model as omodel
from wdl import model as wmodel

BF = torch.bfloat16


def close_bf16(a, b, ulps=2):
    a, b = a.float(), b.float()
    assert torch.all((a - b).abs() <= ulps * 2 ** -8 * b.abs() + 1e-6), float((a - b).abs().max())


def test_sigmas_are_the_reference_fixture():
    want = [1.0, 0.9375, 5 / 6, 0.625]  # tests/test_causal_schedule.py:14
    for got in (wmodel.sigmas(), omodel.sigmas()):
        assert len(got) == 4
        assert all(abs(a - b) <= 1e-15 for a, b in zip(got, want))
    assert wmodel.sigmas(1.0) == [1.0, 0.75, 0.5, 0.25]  # shift 1: the identity schedule


def test_patch_embedding_is_the_convolution():
    g = torch.Generator().manual_seed(0)
    E = wmodel.random_edges(64, 48, 48, g)
    x = torch.randn(48, 2, 8, 12, generator=g)
    edges = wmodel.ModelEdges(E, "cpu")
    got = edges.patchify(x)
    want = omodel.patch_embed(x, E["patch_w"], E["patch_b"])
    assert got.shape == (2 * 4 * 6, 64)
    close_bf16(got, want)


def test_unpatchify_inverts_the_patch_order_and_is_the_index_map():
    g = torch.Generator().manual_seed(1)
    C, f, H, W = 5, 2, 6, 8
    x = torch.randn(C, f, H, W, generator=g)
    p = wmodel.patch_matrix(x)                                    # (ic, dy, dx) per token
    y = p.view(-1, C, 2, 2).permute(0, 2, 3, 1).reshape(-1, 4 * C)  # the head's (1, 2, 2, out) per token
    assert torch.equal(wmodel.unpatchify(y, (f, H // 2, W // 2), C), x)
    h, w = H // 2, W // 2
    out = torch.empty(C, f, H, W)
    for c in range(C):
        for ff in range(f):
            for i in range(h):
                for j in range(w):
                    for dy in range(2):
                        for dx in range(2):
                            out[c, ff, 2 * i + dy, 2 * j + dx] = y[(ff * h + i) * w + j, (dy * 2 + dx) * C + c]
    assert torch.equal(out, x)


def test_time_features_closed_form():
    f0 = wmodel.time_features(torch.zeros(1))
    assert torch.equal(f0[0, :128], torch.ones(128)) and torch.equal(f0[0, 128:], torch.zeros(128))
    t = 937.5
    f1 = wmodel.time_features(torch.tensor([t]))
    assert float(f1[0, 0]) == float(torch.tensor(math.cos(t), dtype=torch.float32))   # omega_0 = 1
    assert abs(float(f1[0, 128 + 127]) - math.sin(t * 10000 ** (-127 / 128))) < 1e-7


def test_time_embedding_and_head_match_the_oracle():
    g = torch.Generator().manual_seed(2)
    dim = 64
    E = wmodel.random_edges(dim, 48, 48, g, std=0.2)
    edges = wmodel.ModelEdges(E, "cpu")
    t = torch.tensor([812.5])
    t_emb, e0 = edges.time(t)
    ot, oe0 = omodel.time_embed(t, E)
    close_bf16(t_emb, ot, ulps=4)
    close_bf16(e0, oe0.float(), ulps=8)
    X = torch.randn(2 * 3 * 4, dim, generator=g).to(BF)
    flow = edges.head(X, ot, (2, 3, 4))
    want = omodel.head(X, ot, E, (2, 3, 4))
    assert flow.shape == (48, 2, 6, 8)
    close_bf16(flow, want, ulps=4)
