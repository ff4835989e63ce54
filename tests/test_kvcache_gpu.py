"""The FP8 KV cache on the GPU over many chunks, well past a full window (tests/test_kv_cache.py:36-118 states the
window invariants for the reference's cache): after every commit the cache rows hold exactly the sink frames and
the newest frames of the window (the oldest evicted, the chunk's rows copied into their slots), as FP8 rows of the
keys and values that were written; attention over the window meets the Sage bars against the oracle emulation of
the cache as it stands: cosine >= 0.999, and an error against exact attention over the unquantized window within
1.2x (+ 1e-3) of the error the emulation itself carries (FP8 cache rows, int8 Q / K, fp8 P: the reference's
quantized baseline, tests/test_sage_kv.py:97)."""

import pytest
import torch

from oracle import fp8 as ofp8
from oracle import sage as osage

pytestmark = pytest.mark.gpu
T, H, CHUNK = 4, 2, 3  # tokens per latent frame, heads, frames per chunk


def rows_as_set(k: torch.Tensor) -> list:
    """The FP8 rows of a [n, H, 128] key block as a sorted list of byte strings (the ring's order is its own)."""
    b = k.view(torch.uint8).reshape(k.shape[0], -1)
    return sorted(bytes(r.tolist()) for r in b)


@pytest.mark.parametrize("window,sink", [(21, 0), (21, 3), (9, 3), (12, 4), (21, 10)])
def test_window_holds_sink_and_newest_frames_past_many_commits(gpu, window, sink):
    from wdl.kvcache import KVCache

    g = torch.Generator().manual_seed(window * 31 + sink)
    cache = KVCache((window - CHUNK) * T, sink * T, chunk=CHUNK)
    frames = []  # (K, V) bf16 [T, H, 128] of every committed frame, in video order
    worst = 0.0
    for c in range(12):
        Q, K, V = (torch.randn(1, CHUNK * T, H, 128, generator=g).to(torch.bfloat16) for _ in range(3))
        out = cache.attend(Q.cuda(), K.cuda(), V.cuda()).cpu()
        at = cache.saved
        ring = window - CHUNK - sink
        seen = frames if len(frames) <= window - CHUNK else frames[:sink] + frames[len(frames) - ring:]
        assert at == len(seen) * T
        # the cache rows before the chunk: exactly the FP8 rows of the seen frames' keys and values
        if seen:
            want_k = torch.cat([ofp8.quantize_rows(k)[0] for k, _ in seen])
            want_v = torch.cat([ofp8.quantize_rows(v)[0] for _, v in seen])
            assert rows_as_set(cache.k[0, :at].cpu()) == rows_as_set(want_k)
            assert rows_as_set(cache.v[0, :at].cpu()) == rows_as_set(want_v)
        # attention: the Sage bars against the oracle on the cache as it stands
        p = osage.prep(Q, cache.k[:, :max(at, 1)].cpu(), cache.ks[:, :max(at, 1)].cpu(), cache.v[:, :max(at, 1)].cpu(),
                       cache.vs[:, :max(at, 1)].cpu(), at, K, V)
        emul = osage.attention_quantized(p, 128 ** -0.5)
        assert osage.cosine(out, emul) >= 0.999
        # and against exact attention over the unquantized window, relative to the quantized emulation's own error
        Kw = torch.cat([k for k, _ in seen] + [K[0]]).float()[None]
        Vw = torch.cat([v for _, v in seen] + [V[0]]).float()[None]
        exact = osage.attention_exact(Q, Kw, Vw)
        base = osage.rel_err(osage.attention_quantized(p, 128 ** -0.5, p_fp8=True), exact)
        assert osage.rel_err(out, exact) < 1.2 * base + 1e-3
        worst = max(worst, osage.rel_err(out, exact))
        cache.commit()
        frames += [(K[0, f * T:(f + 1) * T], V[0, f * T:(f + 1) * T]) for f in range(CHUNK)]
    print(f"window {window}, sink {sink}: worst error against exact attention {worst:.4f}")
    assert cache.full()


def test_captured_attend_follows_commits_through_the_cached_statistics(gpu):
    """A HIP graph of KVCache.attend captured on a full window stays correct across commits: each commit rewrites
    the ring rows and refreshes the cached column statistics in place, so every replay equals an eager attend after
    the same commits bit for bit, and matches the preparation from all tokens (no cached statistics) to the Sage
    bar. Replays alternate with eager work and synchronisations."""
    from wdl import sage_kv
    from wdl.kvcache import KVCache

    g = torch.Generator().manual_seed(77)
    window = 9
    cache = KVCache((window - CHUNK) * T, 0, chunk=CHUNK)
    new = lambda: [torch.randn(1, CHUNK * T, H, 128, generator=g).to(torch.bfloat16).cuda() for _ in range(3)]
    for _ in range(4):  # past a full window
        cache.attend(*new())
        cache.commit()
    assert cache.full()
    Q, K, V = new()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        cache.attend(Q, K, V)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = cache.attend(Q, K, V)
    for _ in range(3):
        Qn, Kn, Vn = new()
        cache.attend(Qn, Kn, Vn)  # the next chunk, eager, then its commit (eviction and statistics)
        cache.commit()
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = cache.attend(Q, K, V)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)
        whole = sage_kv.attend(Q, cache.k, cache.ks, cache.v, cache.vs, cache.saved, K, V)
        assert osage.cosine(eager.cpu().float(), whole.cpu().float()) >= 0.9999


def test_rows_written_directly_need_invalidate_stats(gpu):
    """Rows [0, saved) written around commit (as a caller restoring a cache would) are seen once invalidate_stats()
    is called: the attention then equals the whole-window preparation's within the Sage bar; assigning `saved`
    invalidates by itself."""
    from wdl import sage_kv
    from wdl.kvcache import KVCache

    g = torch.Generator().manual_seed(5)
    cache = KVCache(6 * T, 0, chunk=CHUNK)
    Q, K, V = (torch.randn(1, CHUNK * T, H, 128, generator=g).to(torch.bfloat16).cuda() for _ in range(3))
    cache.attend(Q, K, V)
    cache.commit()
    rows = torch.randn(1, cache.saved, H, 128, generator=g).mul(50).clamp(-448, 448).to(torch.float8_e4m3fn)
    cache.k[:, :cache.saved] = rows.cuda()
    cache.invalidate_stats()
    out = cache.attend(Q, K, V)
    whole = sage_kv.attend(Q, cache.k, cache.ks, cache.v, cache.vs, cache.saved, K, V)
    assert osage.cosine(out.cpu().float(), whole.cpu().float()) >= 0.9999
    cache.v[:, :cache.saved] = rows.cuda()
    cache.saved = cache.saved  # assigning saved invalidates too
    out = cache.attend(Q, K, V)
    whole = sage_kv.attend(Q, cache.k, cache.ks, cache.v, cache.vs, cache.saved, K, V)
    assert osage.cosine(out.cpu().float(), whole.cpu().float()) >= 0.9999


@pytest.mark.parametrize("static", [(1, 3), (0,), (0, 1, 2, 3)])
def test_forcing_kv_head_split_on_a_full_window(gpu, static):
    """KVCache.set_heads (causal.py:98-104, 222-248): on a full window the static heads attend over the sink, the
    newest finished frame and the chunk only, the dynamic heads over the whole window. Each group's output equals a
    direct sage_kv.attend of its heads through the head and row maps bit for bit, and meets the Sage bars against
    the oracle emulation over the same rows and against exact attention over the unquantized keys and values of
    those frames. The anchor follows each commit (the rows of the frame just finished)."""
    from wdl import sage_kv
    from wdl.kvcache import KVCache

    heads, window, sink = 4, 12, 3
    g = torch.Generator().manual_seed(sum(static) + 10 * len(static))
    cache = KVCache((window - CHUNK) * T, sink * T, chunk=CHUNK)
    cache.set_heads(list(static), heads)
    dynamic = [h for h in range(heads) if h not in static]
    frames = []
    new = lambda: [torch.randn(1, CHUNK * T, heads, 128, generator=g).to(torch.bfloat16) for _ in range(3)]
    for c in range(7):
        Q, K, V = new()
        full = cache.full()
        out = cache.attend(Q.cuda(), K.cuda(), V.cuda())
        at = cache.saved
        if full:
            ring = window - CHUNK - sink
            seen = frames[:sink] + frames[len(frames) - ring:]
            rows = torch.tensor(list(range(sink * T)) + cache.anchor_rows(), dtype=torch.int32)
            assert torch.equal(cache.anchor_tokens.cpu(), rows)
            for group, tokens, length, keep in ((dynamic, None, at, seen), (list(static), rows, rows.numel(),
                                                                           frames[:sink] + frames[-1:])):
                if not group:
                    continue
                idx = torch.tensor(group, dtype=torch.int32)
                q, k, v = (t[:, :, idx.long()].contiguous() for t in (Q, K, V))
                direct = sage_kv.attend(q.cuda(), cache.k, cache.ks, cache.v, cache.vs, length, k.cuda(), v.cuda(),
                                        heads=idx.cuda(), tokens=None if tokens is None else tokens.cuda())
                mine = out[:, :, idx.long()].cpu()
                assert torch.equal(mine, direct.cpu()), f"heads {group}"
                p = osage.prep(q, cache.k.cpu(), cache.ks.cpu(), cache.v.cpu(), cache.vs.cpu(), length, k, v,
                               heads=idx, tokens=tokens)
                assert osage.cosine(mine, osage.attention_quantized(p, 128 ** -0.5)) >= 0.999, f"heads {group}"
                Kw = torch.cat([f[0][:, idx.long()] for f in keep] + [k[0]]).float()[None]
                Vw = torch.cat([f[1][:, idx.long()] for f in keep] + [v[0]]).float()[None]
                exact = osage.attention_exact(q, Kw, Vw)
                base = osage.rel_err(osage.attention_quantized(p, 128 ** -0.5, p_fp8=True), exact)
                assert osage.rel_err(mine, exact) < 1.2 * base + 1e-3, f"heads {group}"
        cache.commit()
        frames += [(K[0, f * T:(f + 1) * T], V[0, f * T:(f + 1) * T]) for f in range(CHUNK)]
    assert cache.full()
