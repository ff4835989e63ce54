"""Seeded fp32 weights of a small Wan block and of the model's edges, in the oracle's dict layout, for the fixtures
of the reference's own WanBlock / Head / WanModel (tests/golden/make_block_fixtures.py writes them, tests/
test_oracle_block.py reads them). The fixture file holds the inputs, the outputs and a sha256 of these weights, so a
change of torch's generator shows up as a digest mismatch rather than as a wrong answer.

Weights are N(0, 1/fan_in) so that each sub-layer's update is of the order of its input (the fixtures then see a
wrong gate or a swapped shift / scale), RMSNorm and norm3 weights in [0.5, 1.5), norm3's bias N(0, 0.1^2), biases
N(0, 0.1^2), modulations N(0, 1) / sqrt(dim) as the reference initialises them (block.py:20, head.py:11).
"""

from __future__ import annotations

import hashlib

import torch

DIM, FFN, HEADS, IN_DIM, OUT_DIM, FREQ_DIM = 256, 512, 2, 8, 8, 256


def block_weights(seed: int, dim: int = DIM, ffn: int = FFN) -> dict:
    g = torch.Generator().manual_seed(seed)
    lin = lambda n, k: (torch.randn(n, k, generator=g) / k ** 0.5, torch.randn(n, generator=g) * 0.1)
    W = {name: lin(*shape) for name, shape in dict(
        q=(dim, dim), k=(dim, dim), v=(dim, dim), o=(dim, dim), cq=(dim, dim), ck=(dim, dim), cv=(dim, dim),
        co=(dim, dim), ffn1=(ffn, dim), ffn2=(dim, ffn)).items()}
    B = dict(W=W)
    for name in ("wq", "wk", "cwq", "cwk", "n3w"):
        B[name] = torch.rand(dim, generator=g) + 0.5
    B["n3b"] = torch.randn(dim, generator=g) * 0.1
    B["modulation"] = torch.randn(6, dim, generator=g) / dim ** 0.5
    return B


def edge_weights(seed: int, dim: int = DIM, in_dim: int = IN_DIM, out_dim: int = OUT_DIM) -> dict:
    g = torch.Generator().manual_seed(seed)
    n = lambda *s: torch.randn(*s, generator=g)
    return dict(patch_w=n(dim, in_dim, 1, 2, 2) / (4 * in_dim) ** 0.5, patch_b=n(dim) * 0.1,
                t1_w=n(dim, FREQ_DIM) / FREQ_DIM ** 0.5, t1_b=n(dim) * 0.1, t2_w=n(dim, dim) / dim ** 0.5,
                t2_b=n(dim) * 0.1, proj_w=n(6 * dim, dim) / dim ** 0.5, proj_b=n(6 * dim) * 0.1,
                head_w=n(4 * out_dim, dim) / dim ** 0.5, head_b=n(4 * out_dim) * 0.1,
                head_mod=n(2, dim) / dim ** 0.5)


def digest(*dicts) -> str:
    """sha256 over every tensor of the dicts (nested (weight, bias) pairs included), keys in sorted order."""
    h = hashlib.sha256()

    def feed(obj):
        if isinstance(obj, dict):
            for k in sorted(obj):
                h.update(k.encode())
                feed(obj[k])
        elif isinstance(obj, (tuple, list)):
            for t in obj:
                feed(t)
        else:
            h.update(obj.float().contiguous().numpy().tobytes())

    for d in dicts:
        feed(d)
    return h.hexdigest()
