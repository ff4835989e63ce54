"""DiT step benchmark on one MI355X: the Wan2.2-TI2V-5B-shaped, W4A4 + FP8-KV denoising step at 512x928.

Workload: 30 blocks (dim 3072, 24 heads x 128, FFN 14336) over one 3-latent-frame chunk of 16 x 29 tokens (1392),
with a full 21-frame rolling window (8352 cached FP8 tokens + the chunk = 9744 keys) and 512 cross-attention
tokens, random-init W4A4 weights of that architecture (synthetic data; no checkpoint). A step is
WanModel.forward (src/wan_dit_lab/models/model.py:32-84): patch embedding, time embedding and projection, the 30
blocks (each writing its chunk into its FP8 cache and attending over the window), head and unpatchify. The
timed loop replays one HIP graph of the whole step K times; the per-kernel durations (W4A4 GEMM, attention) come
from an instrumented eager step with HIP events on the launch stream. The cache's column statistics (K sums, |V|
maxima of the cached rows) are refreshed by the commit that changes those rows, not by the step; chunk_ms (the DMD
loop's 4 levels, write pass and commit) includes them.

Prints one JSON line (rank 0; one GPU).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "wan-dit-lab_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

DIM, HEADS, FFN, BLOCKS = 3072, 24, 14336, 30
GRID = (3, 16, 29)                 # 512x928: 3 latent frames of 16 x 29 tokens
TOKENS = GRID[0] * GRID[1] * GRID[2]  # 1392
PER_FRAME = GRID[1] * GRID[2]        # 464
WINDOW = 21                          # frames attention sees: 18 cached + the 3-frame chunk
CACHED = (WINDOW - GRID[0]) * PER_FRAME  # 8352
CONTEXT = 512
LATENT = 48
INT8_PEAK_TOPS = 5000.0   # MI355X dense int8 / fp8 MFMA
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Step:
    """One DiT step over resident weights and caches."""

    def __init__(self, device, seed=0):
        import torch

        from wdl.block import random_block
        from wdl.kvcache import KVCache
        from wdl.model import DiTModel, ModelEdges, random_edges
        from wdl.rope import freqs

        g = torch.Generator(device=device).manual_seed(seed)
        self.device = device
        self.blocks = []
        for i in range(BLOCKS):
            self.blocks.append(random_block(DIM, FFN, HEADS, device, g))
        log(f"bench: {BLOCKS} blocks of random W4A4 weights ready")
        self.caches = []
        for i in range(BLOCKS):
            c = KVCache(CACHED, 0, chunk=GRID[0])
            c.allocate(torch.empty(1, TOKENS, HEADS, 128, device=device))
            c.fill_for_benchmark(g)
            self.caches.append(c)
        context = torch.randn(CONTEXT, DIM, generator=g, device=device).to(torch.bfloat16)
        self.freq = freqs(128, 1024, device)
        # WanModel's step on one chunk: patch embedding, time embedding and projection, the blocks (each
        # attending over its full FP8 window and the prompt), Head and unpatchify (wdl.model, model.py:32-84)
        edges = ModelEdges(random_edges(DIM, LATENT, LATENT, g), device)
        self.model = DiTModel(edges, self.blocks, self.caches, context, self.freq)
        self.latent = torch.randn(LATENT, GRID[0], 2 * GRID[1], 2 * GRID[2], generator=g, device=device)
        self.t = torch.tensor([750.0], device=device)
        # the chunk sits after the window's cached frames: its first frame is frame 18
        self.start_frame = WINDOW - GRID[0]

    def __call__(self):
        return self.model.forward(self.latent, self.t, self.start_frame)


def mixed_stream_ms(chunks: int, device, switch: bool = False) -> dict:
    """The mixed-precision streaming workload at 704x1280: 30 blocks with FP8 weight-only attention projections and
    W4A4 feed-forward, 3-frame chunks of 22 x 40 = 2640 tokens over a full 21-frame window (15840 cached FP8 tokens +
    the chunk = 18480 keys) and 512 prompt tokens, `chunks` consecutive chunks of the DMD loop (4 levels, write pass,
    commit with eviction), eager, after one chunk of warm-up. Milliseconds per chunk and latent tokens/s. switch:
    then the mid-stream switch to 512x928 (the window's 6 chunks resampled and re-encoded, timed) and `chunks` more
    chunks at 16 x 29 = 1392 tokens over the 9744-key window. The window starts filled with random FP8 rows and
    random clean latents for its chunks (synthetic)."""
    import torch

    from wdl.block import random_block
    from wdl.kvcache import KVCache
    from wdl.model import ChunkStream, DiTModel, ModelEdges, random_edges
    from wdl.rope import freqs

    grid = (3, 22, 40)
    tokens, per_frame = grid[0] * grid[1] * grid[2], grid[1] * grid[2]
    g = torch.Generator(device=device).manual_seed(5)
    blocks = [random_block(DIM, FFN, HEADS, device, g, mixed=True) for _ in range(BLOCKS)]
    caches = []
    for _ in range(BLOCKS):
        c = KVCache((WINDOW - grid[0]) * per_frame, 0, chunk=grid[0])
        c.allocate(torch.empty(1, tokens, HEADS, 128, device=device))
        c.fill_for_benchmark(g)
        caches.append(c)
    context = torch.randn(CONTEXT, DIM, generator=g, device=device).to(torch.bfloat16)
    model = DiTModel(ModelEdges(random_edges(DIM, LATENT, LATENT, g), device), blocks, caches, context,
                     freqs(128, 1024, device))
    stream = ChunkStream(model, (LATENT, grid[0], 2 * grid[1], 2 * grid[2]), g)
    stream.start = WINDOW - grid[0]
    stream.kept = [(f, torch.randn(stream.shape, generator=g, device=device)) for f in range(0, stream.start, grid[0])]
    stream.next_chunk()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(chunks):
        stream.next_chunk()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / chunks
    log(f"bench: 704x1280 mixed precision: {ms:.2f} ms per chunk over {chunks} chunks (DMD loop, eager)")
    out = {"workload": "704x1280, 3-frame chunks of 22x40 = 2640 tokens, 21-frame window (18480 keys, FP8 KV), 512 "
                       "prompt tokens, attention projections FP8 weight-only, FFN W4A4, DMD loop (4 levels + write "
                       "pass + commit), eager", "chunks": chunks, "ms_per_chunk": ms,
           "latent_tokens_per_s": tokens / (ms * 1e-3)}
    if switch:
        e0.record()
        stream.switch_resolution(32, 58)
        e1.record()
        torch.cuda.synchronize()
        ms_switch = e0.elapsed_time(e1)
        stream.next_chunk()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(chunks):
            stream.next_chunk()
        e1.record()
        torch.cuda.synchronize()
        ms2 = e0.elapsed_time(e1) / chunks
        log(f"bench: switch to 512x928: {ms_switch:.2f} ms (6 chunks re-encoded); then {ms2:.2f} ms per chunk")
        out["switch_512x928"] = {"ms_switch": ms_switch, "reencoded_chunks": 6, "ms_per_chunk_after": ms2,
                                 "latent_tokens_per_s_after": 1392 / (ms2 * 1e-3)}
    return out


def chunk_ms(step, chunks: int) -> float:
    """Milliseconds per chunk of Stream.next_chunk's DMD loop over the step's model (generation/causal.py:680-740):
    four levels, the write pass and the commit of every block's full FP8 window (the oldest frames evicted), eager;
    one chunk of warm-up first."""
    import torch

    from wdl.model import ChunkStream

    gen = torch.Generator(device=step.latent.device).manual_seed(1)
    stream = ChunkStream(step.model, tuple(step.latent.shape), gen)
    stream.start = step.start_frame
    stream.next_chunk()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(chunks):
        stream.next_chunk()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / chunks
    log(f"bench: {ms:.2f} ms per chunk (DMD loop, eager)")
    return ms


def instrumented(step):
    """The step's W4A4 GEMM and attention launches, timed two ways on the launch stream: HIP events around every
    launch of one eager step (`events`), and each kind's launches of that step (the same calls on the same
    buffers) captured into a HIP graph of their own whose replays are timed as a whole (`ms`, kernel time without
    per-launch event records; the roofline's basis)."""
    import torch

    from wdl import ops

    rec = {"gemm": [], "attn": []}
    calls = {"gemm": [], "attn": []}
    orig_gemm, orig_attn, orig_attn16 = ops.gemm_launch, ops.sage_attn_launch, ops.sage_attn_q16_launch
    orig_gq, orig_bf16 = ops.gelu_quant_launch, ops.attn_bf16_launch

    def timed(kind, fn, flops, *a, **k):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        out = fn(*a, **k)
        e1.record()
        rec[kind].append((e0, e1, flops))
        calls[kind].append((fn, a, k))
        return out

    def gemm(q, ascales, lora, qweight, *a, **k):
        return timed("gemm", orig_gemm, 2.0 * a[3] * ops.out_features(qweight) * q.shape[1] * 64,
                     q, ascales, lora, qweight, *a, **k)

    def gelu_quant(q, ascales, lora, wcodes, *a, **k):  # (wscales, proj_up, bias, M, smooth2, proj_down2_t)
        return timed("gemm", orig_gq, 2.0 * a[3] * ops.out_features(wcodes) * q.shape[1] * 64,
                     q, ascales, lora, wcodes, *a, **k)

    def attn(q_i8, q_scale, prep, L, sm_scale, out=None):
        n, H, d = q_i8.shape
        return timed("attn", orig_attn, 4.0 * n * L * d * H, q_i8, q_scale, prep, L, sm_scale, out)

    def attn_bf16(Q, prep, sm_scale, out=None):
        return timed("attn", orig_bf16, 4.0 * Q.shape[0] * prep["L"] * Q.shape[1], Q, prep, sm_scale, out)

    def attn16(Q, prep, L, sm_scale, out=None):
        return timed("attn", orig_attn16, 4.0 * Q.shape[0] * L * Q.shape[1], Q, prep, L, sm_scale, out)

    ops.gemm_launch, ops.sage_attn_launch, ops.sage_attn_q16_launch = gemm, attn, attn16
    ops.gelu_quant_launch, ops.attn_bf16_launch = gelu_quant, attn_bf16
    # Keep the GPU behind the host while the step is enqueued, so that each start event is followed at once by its
    # (already queued) kernel and no host launch latency falls between the events: a spin kernel of ~0.5 s first.
    probe = 10_000_000
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record()
    torch.cuda._sleep(probe)
    s1.record()
    torch.cuda.synchronize()
    cycles_per_ms = probe / max(s0.elapsed_time(s1), 1e-3)
    try:
        torch.cuda._sleep(int(500 * cycles_per_ms))
        step()
        torch.cuda.synchronize()
    finally:
        ops.gemm_launch, ops.sage_attn_launch, ops.sage_attn_q16_launch = orig_gemm, orig_attn, orig_attn16
        ops.gelu_quant_launch, ops.attn_bf16_launch = orig_gq, orig_bf16
    out = {}
    for name, items in rec.items():
        ev = sum(a.elapsed_time(b) for a, b, _ in items)
        flops = sum(f for _, _, f in items)
        # the same launches as one graph, replayed: kernel time back to back (the launches rewrite their outputs,
        # the residual GEMMs their residual in place: the values change, the work does not)
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for fn, a, k in calls[name]:
                fn(*a, **k)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            for fn, a, k in calls[name]:
                fn(*a, **k)
        graph.replay()
        torch.cuda.synchronize()
        reps = 5
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        del graph
        out[name] = dict(launches=len(items), ms=ms, tops=flops / (ms * 1e-3) / 1e12 if ms else 0.0,
                         events_ms=ev, events_tops=flops / (ev * 1e-3) / 1e12 if ev else 0.0)
    return out


COUNTERS = ROOT / "profiles" / "w4a4_gemm_kernel_dit_step_512x928_counters.md"


def fp8_sweep(device) -> dict:
    """The FP8 W8A8 GEMMs of the W4A4 sweep's shapes (QKV, O, FFN-up, FFN-down at 1392 and 2640 tokens), e4m3
    activations with per-token scales and e4m3 weights with per-channel scales, as DynamicFp8Linear runs them: each
    shape's GEMM launches (stream-K and merge where the library splits K) replayed ten times from a HIP graph and
    timed with HIP events on the stream it runs on; tops = all shapes' 2 M N K over their summed times."""
    import torch

    from wdl import fp8

    g = torch.Generator(device=device).manual_seed(11)
    ops = us = 0.0
    per = {}
    for M in (1392, 2640):
        for name, N, K in (("qkv", 9216, 3072), ("o", 3072, 3072), ("ffn1", 14336, 3072), ("ffn2", 3072, 14336)):
            x = torch.randn(M, K, device=device, generator=g).to(torch.bfloat16)
            wq, ws = fp8.quantize_padded(torch.randn(N, K, device=device, generator=g) * 0.02, rows=True, pad=1)
            q, xs = fp8.quantize_padded(x, rows=True)
            fn = lambda: fp8.gemm(q, xs, M, wq, ws, None, rows=True)
            fn()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(10):
                    fn()
            graph.replay()
            stream = torch.cuda.current_stream()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            graph.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) / 10 * 1e3
            per[f"{name}_{M}"] = round(t, 1)
            ops += 2.0 * M * N * K
            us += t
            del graph
    return {"tops": ops / us / 1e6, "us_per_shape": per}


def gemm_traffic():
    """HBM bytes per W4A4 GEMM launch over the step: FETCH_SIZE and WRITE_SIZE averages of two rocprofv3 --pmc runs
    of this benchmark, each scaled by its reading for a copy of known size (the committed counter summary)."""
    import re

    if not COUNTERS.exists():
        return None
    m = re.search(r"w4a4_gemm_kernel, all launches: HBM bytes per launch \(calibrated\): (\d+)", COUNTERS.read_text())
    return int(m.group(1)) if m else None


class CpuBlock:
    """The quantized Wan block as a PyTorch program on the host CPU, in one floating dtype (bf16 or fp32): the
    reference's block (models/block.py:22-29) with its W4A4 linears computed as fake quantization (activations per
    token and 64-channel group to int4 with a bf16 scale, then dequantized; int4 weights dequantized once), the
    fused GELU MLP's hidden layer quantized unsigned after the 0.171875 shift, the FP8 cache dequantized, Q/K
    RMSNorm, 3D RoPE (fp32 table) and torch's scaled_dot_product_attention over the window and over the prompt.
    Random-init parts of the Wan2.2-TI2V-5B block shapes (int4 in [-7, 7], N(0, 0.02^2)-sized group scales)."""

    def __init__(self, dtype, seed=0, dim=DIM, ffn=FFN, heads=HEADS):
        import torch

        g = torch.Generator().manual_seed(seed)
        self.dt, self.dim, self.heads = dtype, dim, heads
        shapes = dict(qkv=(3 * dim, dim), o=(dim, dim), cq=(dim, dim), ck=(dim, dim), cv=(dim, dim), co=(dim, dim),
                      ffn1=(ffn, dim), ffn2=(dim, ffn))
        self.lin, self.logical = {}, {}
        for name, (n, k) in shapes.items():
            q = torch.randint(-7, 8, (n, k), generator=g)
            ws = ((torch.rand(n, k // 64, generator=g) * 0.5 + 0.75) * (3 * 0.02 / 7)).to(torch.bfloat16)
            pd = (torch.randn(k, 32, generator=g) / k ** 0.5).to(torch.bfloat16)
            pu = (torch.randn(n, 32, generator=g) * 0.02).to(torch.bfloat16)
            b = (torch.randn(n, generator=g) * 0.02).to(torch.bfloat16)
            self.lin[name] = dict(
                W=(q.float().view(n, k // 64, 64) * ws.float()[..., None]).view(n, k).to(dtype),
                pd=pd.to(dtype), pu=pu.to(dtype), b=b.to(dtype))
            # the same layer as the oracle's logical W4A4 parts (unit smoothing)
            self.logical[name] = dict(q=q.to(torch.int32), wscales=ws, proj_down=pd, proj_up=pu,
                                      smooth=torch.ones(k, dtype=torch.bfloat16), bias=b)
        self.mod = torch.randn(6, dim, generator=g) / dim ** 0.5
        from oracle import rope as orope

        self.freq = orope.freqs(128, 1024, torch.float64).float()

    def linear(self, x, name, shift=0.0, unsigned=False):
        import torch

        t = self.lin[name]
        M, K = x.shape
        u = (x.float() + shift).view(M, K // 64, 64)
        qmax = 15.0 if unsigned else 7.0
        s = (u.abs().amax(-1, keepdim=True) / qmax).to(torch.bfloat16).float()
        q = torch.round(u / torch.where(s > 0, s, torch.ones_like(s))).clamp(0.0 if unsigned else -8.0, qmax)
        xq = (q * s).view(M, K).to(self.dt)
        return xq @ t["W"].t() + (x.to(self.dt) @ t["pd"]) @ t["pu"].t() + t["b"]

    def attention(self, Q, K, V):
        import torch

        o = torch.nn.functional.scaled_dot_product_attention(Q.transpose(0, 1)[None], K.transpose(0, 1)[None],
                                                             V.transpose(0, 1)[None])
        return o[0].transpose(0, 1).reshape(Q.shape[0], -1)

    def oracle_parts(self) -> dict:
        """The block as the oracle's logical parts (oracle.block.block_forward): the linears, unit RMSNorm weights,
        no affine on norm3, the modulation."""
        import torch

        P = dict(self.logical)
        for name in ("wq", "wk", "cwq", "cwk"):
            P[name] = torch.ones(self.dim, dtype=torch.bfloat16)
        P["n3w"], P["n3b"] = torch.ones(self.dim), torch.zeros(self.dim)
        P["modulation"] = self.mod.float()
        return P

    def forward(self, X, time_in, cache_k, cache_v, ctx_k, ctx_v, grid, start):
        import torch
        from oracle import rope as orope

        dt, H, D = self.dt, self.heads, self.dim
        e = (time_in + self.mod).to(dt)
        M = X.shape[0]
        ln = lambda x: torch.nn.functional.layer_norm(x.float(), (D,), eps=1e-6).to(dt)
        rms = lambda x: (x.float() * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-6)).to(dt)
        qkv = self.linear(ln(X) * (1 + e[1]) + e[0], "qkv")
        Q = orope.rope_apply(rms(qkv[:, :D]).view(1, M, H, 128).float(), grid, self.freq, start)[0].to(dt)
        K = orope.rope_apply(rms(qkv[:, D:2 * D]).view(1, M, H, 128).float(), grid, self.freq, start)[0].to(dt)
        V = qkv[:, 2 * D:].reshape(M, H, 128)
        A = self.attention(Q, torch.cat([cache_k, K]), torch.cat([cache_v, V]))
        X = X + self.linear(A, "o") * e[2]
        qc = rms(self.linear(ln(X), "cq")).view(M, H, 128)
        X = X + self.linear(self.attention(qc, ctx_k, ctx_v), "co")
        h = torch.nn.functional.gelu(self.linear(ln(X) * (1 + e[4]) + e[3], "ffn1").float(), approximate="tanh")
        return X + self.linear(h, "ffn2", 0.171875, True) * e[5]


def cpu_baseline(runs=5, warmups=2):
    """The block on this host's CPU cores (CpuBlock, bf16 and fp32), on the step's own block workload: 1392 tokens
    (3 frames of 16 x 29) over a full window (8352 cached FP8 tokens + the chunk = 9744 keys) and 512 prompt tokens.
    Per dtype: `warmups` untimed runs, then the median of `runs` timed ones (time.perf_counter). Reported as latent
    tokens/s of a 30-block step (one block timed, x 30: the blocks of a step are alike)."""
    import torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(1)
    X = torch.randn(TOKENS, DIM, generator=g)
    time_in = torch.randn(6, DIM, generator=g) * 0.1
    fp8 = (torch.randn(CACHED, HEADS, 128, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    scales = torch.rand(CACHED, HEADS, 1, generator=g) * 0.02
    ctx = torch.randn(2, CONTEXT, HEADS, 128, generator=g)
    per = {}
    with torch.no_grad():
        for dt in (torch.bfloat16, torch.float32):
            blk = CpuBlock(dt)
            cache = (fp8.float() * scales).to(dt)  # the FP8 window dequantized, as the bf16 cache path reads it
            args = (X.to(dt), time_in, cache, cache, ctx[0].to(dt), ctx[1].to(dt), GRID, WINDOW - GRID[0])
            times = []
            for i in range(warmups + runs):
                t0 = time.perf_counter()
                blk.forward(*args)
                if i >= warmups:
                    times.append(time.perf_counter() - t0)
            per[str(dt).split(".")[-1]] = sorted(times)[len(times) // 2]
            log(f"bench: cpu block ({dt}): median {per[str(dt).split('.')[-1]]:.3f} s of {runs} after {warmups} "
                f"warm-ups")
            del blk
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    best = min(per, key=per.get)
    return dict(value=TOKENS / (BLOCKS * per[best]), unit="latent tokens/s", cores=cores, kind="port",
                dtype=best, seconds_per_block={k: round(v, 4) for k, v in per.items()},
                sample=f"one block of the step's workload ({TOKENS} tokens over {CACHED + TOKENS} keys + "
                       f"{CONTEXT} prompt tokens, dim {DIM}, FFN {FFN}) as a PyTorch fake-quant W4A4 block "
                       f"(bench.CpuBlock) in bf16 and fp32, {warmups} warm-ups then the median of {runs} runs each; "
                       f"value from the faster dtype ({best}) x {BLOCKS} blocks; CPU {cpu}, torch {torch.__version__}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of the HIP graph")
    ap.add_argument("--chunks", type=int, default=3, metavar="C",
                    help="also time C whole chunks of the DMD loop (4 levels + write pass + cache commit, eager) "
                         "after the step measurement, as chunk_ms")
    ap.add_argument("--mixed-704", type=int, default=0, metavar="C",
                    help="also stream C chunks of the mixed-precision 704x1280 workload (FP8 weight-only attention "
                         "projections, W4A4 FFN, 2640-token chunks over an 18480-key window), as mixed_704x1280")
    ap.add_argument("--switch", action="store_true",
                    help="with --mixed-704: then switch to 512x928 mid-stream (window re-encoded) and stream C more "
                         "chunks")
    ap.add_argument("--no-fp8-sweep", action="store_true",
                    help="skip the FP8 W8A8 GEMM sweep (fp8_gemm_tops), e.g. for a kernel trace of the step alone")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run a plain elementwise copy of MIB MiB (bitwise_not, uint8) three times: the "
                         "known-size kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the quantized Wan block hot path runs on a single MI355X, so --gpus "
              "above 1 is not supported", file=sys.stderr)
        sys.exit(2)
    import torch

    from wdl import _lib

    _lib.library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe:
        src = torch.randint(0, 256, (args.copy_probe << 20,), dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.bitwise_not(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
        log(f"bench: copy probe of {args.copy_probe} MiB done")
    step = Step(dev)
    with torch.no_grad():
        for _ in range(max(1, args.warmup)):
            step()
        torch.cuda.synchronize()
        log("bench: eager warmup done")
        kernels = instrumented(step)
        run = step
        if not args.eager:
            graph = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                step()
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            with torch.cuda.graph(graph):
                step()
            run = graph.replay
            for _ in range(args.warmup):
                run()
            torch.cuda.synchronize()
            log("bench: graph captured")
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            run()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
    log(f"bench: {ms:.3f} ms per step")
    g = kernels["gemm"]
    a = kernels["attn"]
    gemm_frac = g["tops"] / INT8_PEAK_TOPS
    result = {
        "metric": "DiT step ms + latent tokens/s at 512x928; W4A4 GEMM TOPS (% of int8 peak)",
        "value": TOKENS / (ms * 1e-3),
        "unit": "latent tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4",
        "data": "synthetic (random-init W4A4 weights of the Wan2.2-TI2V-5B block shapes, random latents, context "
                "and FP8 cache contents)",
        "config": {"workload": "Wan2.2-TI2V-5B-shaped DiT step at 512x928: 30 blocks, dim 3072, 24x128 heads, FFN "
                               "14336, 3-frame chunk of 16x29 = 1392 tokens, 21-frame window = 9744 keys (FP8 KV), "
                               "512 cross tokens, all block linears W4A4, HIP-graph replay",
                   "tokens": TOKENS, "keys": CACHED + TOKENS, "context": CONTEXT, "blocks": BLOCKS,
                   "graph": not args.eager,
                   "cache_statistics": "each block's Sage preparation reads the K column sums and |V| maxima of its "
                                       "8352 cached rows from the cache, which refreshes them at a commit (outside "
                                       "the step, as the commit's row copies are; once per chunk of 5 passes, "
                                       "included in chunk_ms), and sums only the chunk's 1392 tokens"},
        "gemm_tops": g["tops"],
        "gemm_pct_int8_peak": 100 * gemm_frac,
        "gemm_ms_per_step": g["ms"],
        "gemm_tops_eager_events": g["events_tops"],
        "attention_tops": a["tops"],
        "attention_pct_int8_peak": 100 * a["tops"] / INT8_PEAK_TOPS,
        "attention_ms_per_step": a["ms"],
        "roofline": {"bound": "mfma", "kernel": "w4a4_gemm_kernel", "achieved": g["tops"], "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": gemm_frac, "traffic": gemm_traffic(),
                     "basis": "2*M*N*K int ops per launch (M = 1392 tokens) summed over the step's "
                              f"{g['launches']} W4A4 GEMM launches / the HIP-event time of those launches replayed "
                              "back to back from a graph of their own (per-launch events around an eager step: "
                              "gemm_tops_eager_events); traffic = "
                              "calibrated HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE; peak = the "
                              "metric's dense int8 MFMA peak (the kernel issues fp6 MFMAs, dense peak 10.1 POP/s: "
                              "against that the fraction is half)"},
    }
    if not args.no_fp8_sweep:
        with torch.no_grad():
            f8 = fp8_sweep(dev)
        log(f"bench: FP8 W8A8 sweep {f8['tops']:.0f} TOP/s")
        result["fp8_gemm_tops"] = f8["tops"]
        result["fp8_gemm_pct_fp8_peak"] = 100 * f8["tops"] / INT8_PEAK_TOPS
        result["fp8_gemm_us"] = f8["us_per_shape"]
    if args.chunks > 0:
        result["chunk_ms"] = chunk_ms(step, args.chunks)
    if args.mixed_704 > 0:
        del step, run
        if not args.eager:
            del graph
        torch.cuda.empty_cache()
        with torch.no_grad():
            result["mixed_704x1280"] = mixed_stream_ms(args.mixed_704, dev, args.switch)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
