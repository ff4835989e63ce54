"""The mixed-precision 704x1280 streaming workload with the mid-stream switch to 512x928 at its full size (30 blocks,
dim 3072, 24 x 128 heads, FFN 14336; attention projections FP8 weight-only, feed-forward W4A4; 3-frame chunks of
22 x 40 = 2640 tokens over a full 21-frame window of 15 840 cached FP8 tokens + the chunk = 18 480 keys; 512 prompt
tokens), as bench.py --mixed-704 runs it, held to properties (no oracle runs a 30-block stream):
- every chunk's latents are finite, and after every commit each cache holds a full window (saved = its capacity)
  and the stream keeps the window's clean frames;
- a HIP graph captured over the step at 704x1280 replays bit-equal to the eager step;
- the switch rebuilds each cache for the same 18 frames at 464 tokens per frame and re-encodes the window's 6 kept
  chunks: block 0's rows of each re-encoded chunk are bit-equal to block 0's write pass of that chunk's resampled
  latents at its own frame positions (block 0's keys depend only on its input, so this pins where each chunk went
  and the RoPE positions it was written at);
- one chunk at 512x928 after the switch is finite and keeps the window full.
Then one full-width mixed-precision block at the chunk size (2640 tokens over 880 cached FP8 keys and the prompt)
against the oracle block: max-rel-err 1e-2, relative L2 1e-2."""

import pytest
import torch

from oracle import block as oblock
from oracle import rope as orope

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
DIM, HEADS, FFN, BLOCKS, WINDOW, LATENT, CONTEXT = 3072, 24, 14336, 30, 21, 48, 512


def test_mixed_704x1280_stream_and_switch_at_full_size(gpu):
    from wdl.block import random_block
    from wdl.kvcache import KVCache
    from wdl.model import ChunkStream, DiTModel, ModelEdges, random_edges, resample_latents
    from wdl.rope import freqs

    dev = torch.device("cuda")
    grid = (3, 22, 40)
    tokens, per_frame = grid[0] * grid[1] * grid[2], grid[1] * grid[2]
    g = torch.Generator(device=dev).manual_seed(5)
    blocks = [random_block(DIM, FFN, HEADS, dev, g, mixed=True) for _ in range(BLOCKS)]
    assert "fp8" in blocks[0].p["qkv"] and "wcodes" in blocks[0].p["ffn1"]
    caches = []
    for _ in range(BLOCKS):
        c = KVCache((WINDOW - grid[0]) * per_frame, 0, chunk=grid[0])
        c.allocate(torch.empty(1, tokens, HEADS, 128, device=dev))
        c.fill_for_benchmark(g)
        caches.append(c)
    context = torch.randn(CONTEXT, DIM, generator=g, device=dev).to(BF)
    edges = ModelEdges(random_edges(DIM, LATENT, LATENT, g), dev)
    model = DiTModel(edges, blocks, caches, context, freqs(128, 1024, dev))
    shape = (LATENT, grid[0], 2 * grid[1], 2 * grid[2])
    stream = ChunkStream(model, shape, g)
    stream.start = WINDOW - grid[0]
    stream.kept = [(f, torch.randn(shape, generator=g, device=dev)) for f in range(0, stream.start, grid[0])]
    print("config 5: 30 mixed blocks at 704x1280 ready", flush=True)
    for _ in range(2):
        x0 = stream.next_chunk()
        torch.cuda.synchronize()
        assert torch.isfinite(x0).all()
        assert all(c.saved == c.max_tokens == 18 * per_frame for c in model.caches)
    assert [f for f, _ in stream.kept] == list(range(6, 24, 3))  # the window's 18 newest frames
    # the step captured at 704x1280 replays as the eager step
    x = torch.randn(shape, generator=g, device=dev)
    t = torch.tensor([750.0], device=dev)
    with torch.no_grad():
        eager = model.forward(x, t, stream.start).clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            model.forward(x, t, stream.start)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = model.forward(x, t, stream.start)
        for _ in range(2):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
    del graph
    print("config 5: two chunks and the captured step done", flush=True)
    kept = [(f, x.clone()) for f, x in stream.kept]
    stream.switch_resolution(32, 58)
    torch.cuda.synchronize()
    n2 = 3 * 16 * 29
    assert stream.shape == (LATENT, 3, 32, 58)
    assert all(c.max_tokens == 18 * 464 and c.saved == 6 * n2 for c in model.caches)
    # block 0's rows of each re-encoded chunk: its write pass of that chunk alone, at the chunk's frames
    blk, ctx0 = model.blocks[0], model.ctx[0]
    t_emb, e0 = model.edges.time(torch.zeros(1, device=dev))
    e = e0 + model.modulation[0]
    for j, (f, x) in enumerate(kept):
        y = resample_latents(x, 32, 58)
        fresh = KVCache(0, 0, chunk=3)
        blk.forward(model.edges.patchify(y), e, (3, 16, 29), model.freq, f, fresh, ctx0)
        rows = slice(j * n2, (j + 1) * n2)
        c0 = model.caches[0]
        assert torch.equal(c0.k[:, rows].view(torch.uint8), fresh.k[:, :n2].view(torch.uint8)), f"chunk {j} keys"
        assert torch.equal(c0.ks[:, rows], fresh.ks[:, :n2]) and torch.equal(c0.vs[:, rows], fresh.vs[:, :n2])
    x0 = stream.next_chunk()
    torch.cuda.synchronize()
    assert torch.isfinite(x0).all() and x0.shape == (LATENT, 3, 32, 58)
    assert all(c.saved == c.max_tokens for c in model.caches)
    print("config 5: switch and the chunk after it done", flush=True)


def test_full_width_mixed_precision_block_at_the_chunk_size(gpu):
    """One mixed-precision block (FP8 weight-only attention projections of N(0, 0.02^2) weights, W4A4 feed-forward
    of weight standard deviation 0.02) at 2640 tokens (3 frames of 22 x 40, start frame 1) over 880 cached FP8 keys
    and 512 prompt tokens, against the oracle block with the same parts."""
    from wdl.block import build_block
    from wdl.kvcache import KVCache

    g = torch.Generator().manual_seed(9)
    grid, prior, Lc = (3, 22, 40), 880, 512
    P = oblock.mixed_precision_block(DIM, FFN, g, scale=0.02 / 1.871)
    M = grid[0] * grid[1] * grid[2]
    X = torch.randn(M, DIM, generator=g)
    X[:, torch.randperm(DIM, generator=g)[:DIM // 100]] *= 20
    X = X.to(BF)
    time_in = torch.randn(6, DIM, generator=g) * 0.1
    C = torch.randn(Lc, DIM, generator=g).to(BF)
    freq = orope.freqs(128, 1024, torch.float64).float()
    cap = prior + M
    ck = (torch.randn(1, cap, HEADS, 128, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    cv = (torch.randn(1, cap, HEADS, 128, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    cks = torch.rand(1, cap, HEADS, 1, generator=g) * 0.02
    cvs = torch.rand(1, cap, HEADS, 1, generator=g) * 0.02
    ref = oblock.block_forward(X, time_in, P, grid, freq, 1, dict(k=ck.clone(), ks=cks.clone(), v=cv.clone(),
                                                                 vs=cvs.clone(), at=prior),
                               oblock.context_kv(C, P), HEADS)
    dev = torch.device("cuda")
    blk = build_block(P, DIM, HEADS, dev)
    cache = KVCache(prior, 0, chunk=grid[0])
    cache.allocate(torch.empty(1, M, HEADS, 128, device=dev))
    for dst, src in ((cache.k, ck), (cache.v, cv), (cache.ks, cks), (cache.vs, cvs)):
        dst.copy_(src.to(dev))
    cache.saved = prior
    e = (time_in + P["modulation"]).float().to(dev)
    out = blk.forward(X.to(dev).clone(), e, grid, freq.to(dev), 1, cache, blk.prepare_context(C.to(dev))).cpu()
    err = float((out.float() - ref.float()).abs().max()) / float(ref.float().abs().max())
    rel = float((out.float() - ref.float()).norm() / ref.float().norm())
    print(f"mixed block at 2640 tokens: max-rel-err {err:.2e}, rel-L2 {rel:.3e}")
    assert err <= 1e-2 and rel <= 1e-2
