"""The oracle's block and model composition against the reference's own fp32 modules (tests/golden/
block_fixtures.npz, written by tests/golden/make_block_fixtures.py from WanBlock, KVCache, Head and WanModel of
src/wan_dit_lab): oracle.block.float_block_forward (the composition the quantized oracle block shares, _compose),
oracle.model.float_model_forward, head and time_embed in fp32, and the RoPE table.

Bars: the fp32 update of each sub-layer chain within 5e-6 relative L2 and 1e-5 of its largest entry (the reference
sums in fp32 with its own orders, the oracle in fp64 where it can; measured 3-5e-7); the RoPE table bit-equal. Each planted
composition mistake (a swapped shift / scale, a swapped gate, a dropped norm3 affine, the RMSNorm weights of Q and K
exchanged, no RoPE on K) fails the block fixture by orders of magnitude more than the bar.
"""

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import block as oblock
from oracle import model as omodel
from oracle import rope as orope

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))

import block_recipe as R  # noqa: E402


@pytest.fixture(scope="module")
def fx():
    with np.load(GOLDEN / "block_fixtures.npz", allow_pickle=False) as z:
        d = {k: z[k] for k in z.files}
    B = R.block_weights(int(d["seeds"][0]))
    E = R.edge_weights(int(d["seeds"][1]))
    assert R.digest(B, E) == str(d["weights_sha256"]), "torch's generator no longer makes the fixture's weights"
    t = {k: torch.from_numpy(v) for k, v in d.items() if v.dtype.kind == "f"}
    return dict(t, B=B, E=E, grid=tuple(int(v) for v in d["grid"]), start=int(d["start"]),
                freq=orope.freqs(128, 1024, torch.float64))


def close(got, want, base, rel=5e-6, peak=1e-5):
    """got / want fp32 outputs; base the input they update (the bar is on the update)."""
    du, dw = (got.double() - base.double()), (want.double() - base.double())
    err = float((du - dw).norm() / dw.norm())
    mx = float((du - dw).abs().max() / dw.abs().max())
    return err <= rel and mx <= peak, (err, mx)


def test_rope_table_is_the_reference_table(fx):
    """orope.freqs equals the reference's table (rope() per axis, runtime/live_presets.py:52-61) bit for bit."""
    assert torch.equal(fx["freq"][:, :64], fx["freqs"])


def _block(fx, cached, ops_cls=oblock._FloatOps, e_perm=None):
    D = fx["X"].shape[1]
    none = torch.zeros(0, D)
    cache_kv = (fx["Kp"], fx["Vp"]) if cached else (none, none)
    e = fx["time_in"].float() + fx["B"]["modulation"].float()
    if e_perm is not None:
        e = e[list(e_perm)]
    ops = ops_cls(fx["B"], fx["grid"], fx["freq"], fx["start"], cache_kv, fx["C"])
    return oblock._compose(fx["X"].float(), e, fx["B"], ops, R.HEADS)


@pytest.mark.parametrize("cached", [False, True])
def test_float_block_is_the_reference_block(fx, cached):
    """WanBlock.forward with cache=None (SDPA over the chunk) and over a KVCache of 48 earlier tokens."""
    D = fx["X"].shape[1]
    none = torch.zeros(0, D)
    cache_kv = (fx["Kp"], fx["Vp"]) if cached else (none, none)
    got = oblock.float_block_forward(fx["X"], fx["time_in"], fx["B"], fx["grid"], fx["freq"], fx["start"], cache_kv,
                                     fx["C"], R.HEADS)
    ok, (err, mx) = close(got, fx["out_block_cached" if cached else "out_block_nocache"], fx["X"])
    print(f"block cached={cached}: update rel-L2 {err:.2e}, max {mx:.2e}")
    assert ok


class _SwapShiftScale(oblock._FloatOps):
    def norm_mod(self, X, shift, scale):
        return super().norm_mod(X, scale, shift)


class _NoAffine3(oblock._FloatOps):
    def norm_affine(self, X, w, b):
        return self._ln(X)


class _NoRopeOnK(oblock._FloatOps):
    def __init__(self, *a):
        super().__init__(*a)
        self.calls = 0

    def rope(self, X4):
        self.calls += 1
        return super().rope(X4) if self.calls % 2 == 1 else X4.float()


@pytest.mark.parametrize("plant", ["shift/scale", "gates", "norm3 affine", "norm_q/norm_k", "rope on K"])
def test_planted_composition_mistakes_fail_the_fixture(fx, plant):
    want = fx["out_block_nocache"]
    if plant == "shift/scale":
        got = _block(fx, False, _SwapShiftScale)
    elif plant == "gates":
        got = _block(fx, False, e_perm=(0, 1, 5, 3, 4, 2))
    elif plant == "norm3 affine":
        got = _block(fx, False, _NoAffine3)
    elif plant == "norm_q/norm_k":
        B = dict(fx["B"], wq=fx["B"]["wk"], wk=fx["B"]["wq"])
        got = _block(dict(fx, B=B), False)
    else:
        got = _block(fx, False, _NoRopeOnK)
    ok, (err, mx) = close(got, want, fx["X"])
    print(f"planted {plant}: update rel-L2 {err:.2e}")
    assert not ok and err > 1000 * 5e-6
    assert close(_block(fx, False), want, fx["X"])[0]  # the unplanted composition passes


def test_head_is_the_reference_head(fx):
    """Head.forward (head.py:13-18) on tokens and a time embedding, then unpatchify (the product's, itself pinned
    by an index loop in tests/test_model.py) to compare with the oracle's head, which unpatchifies."""
    from wdl.model import unpatchify

    got = omodel.head(fx["X"], fx["t_head"], fx["E"], fx["grid"], dtype=torch.float32)
    want = unpatchify(fx["out_head"], fx["grid"], R.OUT_DIM)
    zero = torch.zeros_like(want)
    ok, (err, mx) = close(got, want, zero)
    print(f"head: rel-L2 {err:.2e}")
    assert ok


def test_float_model_is_the_reference_model(fx):
    """WanModel.forward (model.py:32-84) with one block: patch embedding, the fp64 sinusoid at t = 700,
    time_embedding, time_projection (e0 into the block), the block over the context's keys / values, Head with the
    time embedding, unpatchify."""
    D = fx["X"].shape[1]
    none = torch.zeros(0, D)
    got = omodel.float_model_forward(fx["latent"], fx["t"], fx["E"], [fx["B"]], [(none, none)], [fx["C"]],
                                     fx["freq"], fx["start"], R.HEADS)
    want = fx["out_model"]
    ok, (err, mx) = close(got, want, torch.zeros_like(want))
    print(f"model: rel-L2 {err:.2e}, max {mx:.2e}")
    assert ok
    t_emb, e0 = omodel.time_embed(fx["t"], fx["E"], dtype=torch.float32)
    assert t_emb.shape == (D,) and e0.shape == (6, D)
