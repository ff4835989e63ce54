"""The DiT step on latents (wdl.model.DiTModel: edges + QuantizedWanBlocks) and the DMD chunk loop
(wdl.model.ChunkStream) against the oracle (oracle/model.py over oracle/block.py).

Small config: dim 256, 2 x 128 heads, FFN 1024, 2 SVD-quantized blocks, 48-channel latents of 2 frames x 8 x 16
(64 tokens), 16 context tokens. Bars: each edge stage within a few bf16 steps of the oracle on the same input; the
blocks + Head on the oracle's edge outputs within the block bar (max-rel-err 1e-2, 2^-8 relative L2); end to end
(one step, and x0 over two chunks of the loop) within 1.5x of the oracle's own change under 50 one-step input
changes (random-weight W4A4 blocks are chaotic at that level), and so the cached keys of the chunk loop; the
mid-stream resolution switch (the window re-encoded at a new latent size) at the same bars."""

import pytest
import torch

from oracle import block as oblock
from oracle import model as omodel
from oracle import rope as orope

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
DIM, HEADS, FFN, NB = 256, 2, 1024, 2
SHAPE = (48, 2, 8, 16)


def setup(seed):
    from wdl import model as wmodel
    from wdl.block import build_block
    from wdl.kvcache import KVCache

    g = torch.Generator().manual_seed(seed)
    Ps = [oblock.quantize_block(oblock.random_block(DIM, FFN, g)) for _ in range(NB)]
    E = wmodel.random_edges(DIM, 48, 48, g)
    C = torch.randn(16, DIM, generator=g).to(BF)
    freq = orope.freqs(128, 1024, torch.float64).float()
    dev = torch.device("cuda")
    n = SHAPE[1] * (SHAPE[2] // 2) * (SHAPE[3] // 2)
    caches = [KVCache(4 * n, 0, chunk=SHAPE[1]) for _ in range(NB)]
    model = wmodel.DiTModel(wmodel.ModelEdges(E, dev), [build_block(P, DIM, HEADS, dev) for P in Ps], caches,
                            C.to(dev), freq.to(dev))
    cap = 4 * n + n
    ocaches = [dict(k=torch.zeros(1, cap, HEADS, 128, dtype=torch.float8_e4m3fn), ks=torch.ones(1, cap, HEADS, 1),
                    v=torch.zeros(1, cap, HEADS, 128, dtype=torch.float8_e4m3fn), vs=torch.ones(1, cap, HEADS, 1),
                    at=0) for _ in range(NB)]
    octx = [oblock.context_kv(C, P) for P in Ps]
    return model, (E, Ps, ocaches, octx, freq), g, n


def perturbed(x, count, seed):
    """x with `count` entries moved by one bf16 step (2^-8 relative): the oracle's own sensitivity."""
    y = x.clone().view(-1)
    idx = torch.randperm(y.numel(), generator=torch.Generator().manual_seed(seed))[:count]
    y[idx] = y[idx] * (1 + 2 ** -7)
    return y.view(x.shape)


def test_model_step_matches_oracle(gpu):
    """Stage by stage, each fed the same input: patch tokens within 2 bf16 steps of the convolution (hipBLASLt's
    fp32 sum against fp64), t_emb / e0 within 4 / 8 steps; the two blocks + Head on the oracle's tokens and e0,
    and the whole step end to end, within 1.5x of the oracle's own relative-L2 change when 50 of its input entries
    move by one bf16 step (each block alone meets max-rel-err 1e-2 in test_block_gpu.py; a chain of random-weight
    W4A4 blocks is chaotic at the one-step level: an activation-int4 flip moves a whole quantization step)."""
    model, (E, Ps, ocaches, octx, freq), g, n = setup(3)
    x = torch.randn(SHAPE, generator=g)
    t = torch.tensor([937.5])
    dev = torch.device("cuda")
    tokens = model.edges.patchify(x.to(dev)).cpu()
    otokens = omodel.patch_embed(x, E["patch_w"], E["patch_b"])
    assert torch.all((tokens.float() - otokens.float()).abs() <= 2 * 2 ** -8 * otokens.float().abs() + 1e-6)
    t_emb, e0 = model.edges.time(t.to(dev))
    ot, oe0 = omodel.time_embed(t, E)
    assert torch.all((t_emb.cpu().float() - ot.float()).abs() <= 4 * 2 ** -8 * ot.float().abs() + 1e-6)
    assert torch.all((e0.cpu() - oe0.float()).abs() <= 8 * 2 ** -8 * oe0.float().abs() + 1e-6)
    # blocks + Head on the oracle's tokens and e0
    import copy
    c0 = copy.deepcopy(ocaches)
    X = otokens.to(dev)
    e_all = oe0.float().to(dev) + model.modulation
    for blk, cache, ctx, e in zip(model.blocks, model.caches, model.ctx, e_all):
        blk.forward(X, e, (SHAPE[1], SHAPE[2] // 2, SHAPE[3] // 2), model.freq, 0, cache, ctx)
    flow_b = model.edges.head(X, ot.to(dev), (SHAPE[1], SHAPE[2] // 2, SHAPE[3] // 2)).cpu()
    def oracle_blocks_head(X0, caches):
        Xo = X0
        for P, oc, kv in zip(Ps, caches, octx):
            Xo = oblock.block_forward(Xo, oe0.float(), P, (SHAPE[1], SHAPE[2] // 2, SHAPE[3] // 2), freq, 0, oc,
                                      kv, HEADS)
        return omodel.head(Xo, ot, E, (SHAPE[1], SHAPE[2] // 2, SHAPE[3] // 2))

    ref_b = oracle_blocks_head(otokens, c0)
    pert_b = oracle_blocks_head(perturbed(otokens.float(), 50, 5).to(BF), copy.deepcopy(ocaches))
    err = float((flow_b.float() - ref_b.float()).abs().max()) / float(ref_b.float().abs().max())
    rel = float((flow_b.float() - ref_b.float()).norm() / ref_b.float().norm())
    floor = float((pert_b.float() - ref_b.float()).norm() / ref_b.float().norm())
    print(f"blocks + head on the oracle's edge outputs: max-rel-err {err:.2e}, rel-L2 {rel:.3e} "
          f"(oracle under 50 one-step token changes: {floor:.3e})")
    assert rel <= 1.5 * max(floor, 2 ** -8)
    # end to end
    for c in model.caches:
        c.reset()
    flow = model.forward(x.to(dev), t.to(dev), 0).cpu()
    ref = omodel.model_forward(x, t, E, Ps, copy.deepcopy(ocaches), octx, freq, 0, HEADS)
    pert = omodel.model_forward(perturbed(x, 50, 9), t, E, Ps, copy.deepcopy(ocaches), octx, freq, 0, HEADS)
    assert flow.shape == ref.shape == SHAPE
    rel = float((flow.float() - ref.float()).norm() / ref.float().norm())
    floor = float((pert.float() - ref.float()).norm() / ref.float().norm())
    print(f"model step end to end: rel-L2 {rel:.3e} (oracle under 50 one-step latent changes: {floor:.3e})")
    assert rel <= 1.5 * max(floor, 2 ** -8)


def test_chunk_loop_matches_oracle(gpu):
    """Two chunks of the DMD loop from the same noises (and the same fresh noises): per chunk, x0's error relative
    to its change from the noise within 1.5x of the oracle's own under 50 one-step noise changes (floor 2 %),
    the caches' write offsets advance by a chunk, and the last chunk's cached keys (dequantized) within the same
    bar against the perturbed run's."""
    import copy

    from wdl import model as wmodel

    model, (E, Ps, ocaches, octx, freq), g, n = setup(4)
    gen = torch.Generator(device="cuda").manual_seed(11)
    stream = wmodel.ChunkStream(model, SHAPE, gen)
    ref_gen = torch.Generator(device="cuda").manual_seed(11)
    for chunk in range(2):
        noise = torch.randn(SHAPE, generator=g)
        x0 = stream.next_chunk(noise.cuda()).cpu()
        fresh = [torch.randn(SHAPE, generator=ref_gen, device="cuda").cpu() for _ in range(3)]
        pc = copy.deepcopy(ocaches)
        pert = omodel.next_chunk(perturbed(noise, 50, 20 + chunk), fresh, E, Ps, pc, octx, freq,
                                 chunk * SHAPE[1], HEADS)
        ref = omodel.next_chunk(noise, fresh, E, Ps, ocaches, octx, freq, chunk * SHAPE[1], HEADS)
        rel = float((x0 - ref).norm() / (ref - noise).norm())
        floor = float((pert - ref).norm() / (ref - noise).norm())
        print(f"chunk {chunk}: x0 error / x0 change {rel:.3e} (oracle under 50 one-step changes: {floor:.3e})")
        assert rel <= 1.5 * max(floor, 0.02)
        assert all(c.saved == (chunk + 1) * n for c in model.caches)
    # the last chunk's cached keys (written by its write pass), dequantized, against the oracle's, with the same
    # floor: the perturbed run's caches
    deq = lambda k, ks: k[:, n:2 * n].float() * ks[:, n:2 * n]
    for c, oc, po in zip(model.caches, ocaches, pc):
        ref_k = deq(oc["k"], oc["ks"])
        rel = float((deq(c.k.cpu(), c.ks.cpu()) - ref_k).norm() / ref_k.norm())
        floor = float((deq(po["k"], po["ks"]) - ref_k).norm() / ref_k.norm())
        print(f"cached keys: rel-L2 {rel:.3e} (oracle under 50 one-step changes: {floor:.3e})")
        assert rel <= 1.5 * max(floor, 0.02)


def test_unipc_chunk_loop_matches_oracle(gpu):
    """Two chunks of the "unipc" loop (2 steps at t = 999, 833, then the write pass) from the same noises: x0's
    error relative to its change from the noise within 1.5x of the oracle's own under 50 one-step noise changes
    (floor 2 %), and the caches' write offsets advance by a chunk."""
    import copy

    from wdl import model as wmodel

    model, (E, Ps, ocaches, octx, freq), g, n = setup(6)
    stream = wmodel.ChunkStream(model, SHAPE, torch.Generator(device="cuda"), sampler="unipc", steps=2)
    assert stream.timesteps == [999, 833]
    for chunk in range(2):
        noise = torch.randn(SHAPE, generator=g)
        x0 = stream.next_chunk(noise.cuda()).cpu()
        pert = omodel.next_chunk_unipc(perturbed(noise, 50, 40 + chunk), E, Ps, copy.deepcopy(ocaches), octx, freq,
                                       chunk * SHAPE[1], HEADS)
        ref = omodel.next_chunk_unipc(noise, E, Ps, ocaches, octx, freq, chunk * SHAPE[1], HEADS)
        rel = float((x0 - ref).norm() / (ref - noise).norm())
        floor = float((pert - ref).norm() / (ref - noise).norm())
        print(f"unipc chunk {chunk}: x0 error / x0 change {rel:.3e} (oracle under 50 one-step changes: {floor:.3e})")
        assert rel <= 1.5 * max(floor, 0.02)
        assert all(c.saved == (chunk + 1) * n for c in model.caches)


def test_resolution_switch_reencodes_the_window(gpu):
    """Two chunks at 8 x 16 latents (64 tokens per chunk), then the switch to 12 x 8 (48 per chunk, grid 2 x 6 x 4):
    the kept chunks' latents resampled as the oracle resamples them (within fp32 rounding); every block's cache
    rebuilt for the same 8-frame window at the new tokens per frame and refilled by the write pass, its keys
    (dequantized) against the oracle's write pass over the same resampled latents, and then one chunk at the new
    size against the oracle's chunk loop over those caches, both within the chunk-loop bar (1.5x the oracle's own
    change under 50 one-step input changes, floor 2 %)."""
    import copy

    from wdl import model as wmodel

    model, (E, Ps, _, octx, freq), g, n = setup(8)
    gen = torch.Generator(device="cuda").manual_seed(13)
    stream = wmodel.ChunkStream(model, SHAPE, gen)
    for _ in range(2):
        stream.next_chunk(torch.randn(SHAPE, generator=g).cuda())
    kept = [(f, x.cpu()) for f, x in stream.kept]
    assert [f for f, _ in kept] == [0, 2]
    H2, W2 = 12, 8
    stream.switch_resolution(H2, W2)
    n2 = SHAPE[1] * (H2 // 2) * (W2 // 2)
    assert stream.shape == (48, 2, H2, W2) and stream.start == 4
    assert all(c.max_tokens == 4 * n2 and c.saved == 2 * n2 for c in model.caches)
    resampled = [(f, x.cpu()) for f, x in stream.kept]
    for (f, x), (f2, y) in zip(kept, resampled):
        want = omodel.resample(x, H2, W2)
        assert f == f2 and float((y - want).abs().max()) <= 2e-5 * float(x.abs().max())
    cap = 5 * n2
    fresh_caches = lambda: [dict(k=torch.zeros(1, cap, HEADS, 128, dtype=torch.float8_e4m3fn),
                                 ks=torch.ones(1, cap, HEADS, 1),
                                 v=torch.zeros(1, cap, HEADS, 128, dtype=torch.float8_e4m3fn),
                                 vs=torch.ones(1, cap, HEADS, 1), at=0) for _ in range(NB)]
    oc, pc = fresh_caches(), fresh_caches()
    omodel.reencode(resampled, E, Ps, oc, octx, freq, HEADS)
    omodel.reencode([(f, perturbed(x, 50, 60 + f)) for f, x in resampled], E, Ps, pc, octx, freq, HEADS)
    deq = lambda k, ks: k[:, :2 * n2].float() * ks[:, :2 * n2]
    for c, o, p in zip(model.caches, oc, pc):
        ref_k = deq(o["k"], o["ks"])
        rel = float((deq(c.k.cpu(), c.ks.cpu()) - ref_k).norm() / ref_k.norm())
        floor = float((deq(p["k"], p["ks"]) - ref_k).norm() / ref_k.norm())
        print(f"re-encoded keys: rel-L2 {rel:.3e} (oracle under 50 one-step changes: {floor:.3e})")
        assert rel <= 1.5 * max(floor, 0.02)
    # one chunk at the new size from the re-encoded caches (the stream's renoising draws reproduced)
    ref_gen = torch.Generator(device="cuda").manual_seed(13)
    for _ in range(6):
        torch.randn(SHAPE, generator=ref_gen, device="cuda")
    shape2 = (48, 2, H2, W2)
    noise = torch.randn(shape2, generator=g)
    x0 = stream.next_chunk(noise.cuda()).cpu()
    fresh = [torch.randn(shape2, generator=ref_gen, device="cuda").cpu() for _ in range(3)]
    pert = omodel.next_chunk(perturbed(noise, 50, 70), fresh, E, Ps, copy.deepcopy(oc), octx, freq, 4, HEADS)
    ref = omodel.next_chunk(noise, fresh, E, Ps, oc, octx, freq, 4, HEADS)
    rel = float((x0 - ref).norm() / (ref - noise).norm())
    floor = float((pert - ref).norm() / (ref - noise).norm())
    print(f"chunk after the switch: x0 error / x0 change {rel:.3e} (oracle under 50 one-step changes: {floor:.3e})")
    assert rel <= 1.5 * max(floor, 0.02)
    assert all(c.saved == 3 * n2 for c in model.caches)
