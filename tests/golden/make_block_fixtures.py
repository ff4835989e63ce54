"""Writes tests/golden/block_fixtures.npz from the reference's own fp32 modules (run in the build container, where
the reference's source tree is at /root/reference; nothing on the GPU side reads it):

- block_nocache: WanBlock.forward (src/wan_dit_lab/models/block.py:22-29) with cache=None and the context given,
  so MultiHeadAttention (models/multi_head_attention.py:21-44) runs keys_values on the context and SDPA over the
  chunk alone;
- block_cached: the same block over a causal.KVCache (generation/causal.py:48-260, fp32 buffers, no FP8 / Sage)
  holding 48 earlier tokens: attend stores the chunk after them and runs SDPA over both (attend_unpacked);
- head: Head.forward (models/head.py:13-18) on tokens and a time embedding;
- model: WanModel.forward (models/model.py:32-84) with one block on a latent, the context's per-block keys and
  values given (context_kvs), so patch embedding, the fp64 sinusoid, time_embedding, time_projection, the block,
  the Head and unpatchify all run;
- freqs: the RoPE table of runtime/live_presets.py:52-61 (rope() of models/rope.py per axis, 22/21/21 pairs),
  the first 64 positions.

The fixture holds the inputs, the outputs and the sha256 of the weights tests/golden/block_recipe.py makes from its
seeds. Usage: python tests/golden/make_block_fixtures.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REFERENCE_SRC = Path("/root/reference/src")
sys.path.insert(0, str(HERE))
sys.path.insert(0, str(REFERENCE_SRC))

import block_recipe as R  # noqa: E402
from wan_dit_lab.generation.causal import KVCache  # noqa: E402
from wan_dit_lab.models.block import WanBlock  # noqa: E402
from wan_dit_lab.models.head import Head  # noqa: E402
from wan_dit_lab.models.model import WanModel  # noqa: E402
from wan_dit_lab.models.rope import rope  # noqa: E402

BLOCK_SEED, EDGE_SEED, INPUT_SEED = 11, 12, 13
GRID, START, PRIOR, CONTEXT = (2, 4, 6), 1, 48, 16
POSITIONS = 64


def load_block(block: WanBlock, B: dict):
    W = B["W"]
    sd = {}
    for prefix, names in (("self_attn", dict(q="q", k="k", v="v", o="o")),
                          ("cross_attn", dict(q="cq", k="ck", v="cv", o="co"))):
        for layer, name in names.items():
            sd[f"{prefix}.{layer}.weight"], sd[f"{prefix}.{layer}.bias"] = W[name]
    sd["self_attn.norm_q.weight"], sd["self_attn.norm_k.weight"] = B["wq"], B["wk"]
    sd["cross_attn.norm_q.weight"], sd["cross_attn.norm_k.weight"] = B["cwq"], B["cwk"]
    sd["ffn.0.weight"], sd["ffn.0.bias"] = W["ffn1"]
    sd["ffn.2.weight"], sd["ffn.2.bias"] = W["ffn2"]
    sd["norm3.weight"], sd["norm3.bias"] = B["n3w"], B["n3b"]
    sd["modulation"] = B["modulation"].reshape(1, 6, -1)
    block.load_state_dict(sd, strict=True)


class _InOrder:
    """The block_offloader WanModel.forward asks for its blocks (model.py:44, 79): here they are all resident."""

    def __init__(self, blocks):
        self.blocks, self.i = list(blocks), 0

    def get_next(self):
        b = self.blocks[self.i % len(self.blocks)]
        self.i += 1
        return b

    def release(self, block):
        pass


@torch.no_grad()
def main():
    torch.set_num_threads(1)
    B = R.block_weights(BLOCK_SEED)
    E = R.edge_weights(EDGE_SEED)
    g = torch.Generator().manual_seed(INPUT_SEED)
    f, h, w = GRID
    M, D, H = f * h * w, R.DIM, R.HEADS
    X = torch.randn(1, M, D, generator=g)
    time_in = torch.randn(1, 6, D, generator=g) * 0.3
    C = torch.randn(1, CONTEXT, D, generator=g)
    Kp = torch.randn(1, PRIOR, H, D // H, generator=g)
    Vp = torch.randn(1, PRIOR, H, D // H, generator=g)
    latent = torch.randn(1, R.IN_DIM, f, 2 * h, 2 * w, generator=g)
    t = torch.tensor([700.0])
    t_head = torch.randn(1, D, generator=g)
    d = D // H
    freqs = torch.cat([rope(1024, d - 4 * (d // 6)), rope(1024, 2 * (d // 6)), rope(1024, 2 * (d // 6))], dim=-1)

    block = WanBlock(D, R.FFN, H, 1e-6)
    load_block(block, B)
    out_nocache = block(X, time_in, grid_sizes=[GRID], freqs=freqs, context=C, start_frame=START)

    cache = KVCache(PRIOR, 0, chunk=f)
    cache.allocate(torch.empty(1, M, H, d))
    cache.k[:, :PRIOR], cache.v[:, :PRIOR] = Kp, Vp
    cache.saved = PRIOR
    out_cached = block(X, time_in, grid_sizes=[GRID], freqs=freqs, context=C, start_frame=START, cache=cache)
    assert torch.equal(cache.k[:, :PRIOR], Kp)

    head = Head(D, R.OUT_DIM, 1e-6)
    head.load_state_dict({"head.weight": E["head_w"], "head.bias": E["head_b"],
                          "modulation": E["head_mod"].reshape(1, 2, D)}, strict=True)
    out_head = head(X, t_head)

    model = WanModel(D, 1e-6, R.FFN, R.FREQ_DIM, R.IN_DIM, H, 1, R.OUT_DIM, CONTEXT, text_dim=64)
    sd = {"patch_embedding.weight": E["patch_w"], "patch_embedding.bias": E["patch_b"],
          "time_embedding.0.weight": E["t1_w"], "time_embedding.0.bias": E["t1_b"],
          "time_embedding.2.weight": E["t2_w"], "time_embedding.2.bias": E["t2_b"],
          "time_projection.1.weight": E["proj_w"], "time_projection.1.bias": E["proj_b"],
          "head.head.weight": E["head_w"], "head.head.bias": E["head_b"],
          "head.modulation": E["head_mod"].reshape(1, 2, D)}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all(k.startswith(("blocks.", "text_embedding.")) for k in missing), missing
    load_block(model.blocks[0], B)
    model.block_offloader = _InOrder(model.blocks)
    kv = [model.blocks[0].cross_attn.keys_values(C)]
    out_model = model(latent, t, None, [GRID], freqs, start_frame=START, context_kvs=kv)

    np.savez_compressed(HERE / "block_fixtures.npz",
             weights_sha256=np.array(R.digest(B, E)),
             seeds=np.array([BLOCK_SEED, EDGE_SEED]),
             grid=np.array(GRID), start=np.array(START),
             X=X[0].numpy(), time_in=time_in[0].numpy(), C=C[0].numpy(),
             Kp=Kp[0].reshape(PRIOR, D).numpy(), Vp=Vp[0].reshape(PRIOR, D).numpy(),
             latent=latent[0].numpy(), t=t.numpy(), t_head=t_head[0].numpy(),
             freqs=freqs[:, :POSITIONS].numpy(),
             out_block_nocache=out_nocache[0].numpy(), out_block_cached=out_cached[0].numpy(),
             out_head=out_head[0].numpy(), out_model=out_model[0].numpy())
    print("wrote", HERE / "block_fixtures.npz")


if __name__ == "__main__":
    main()
