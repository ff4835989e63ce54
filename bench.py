"""DiT step benchmark on one MI355X: the Wan2.2-TI2V-5B-shaped, W4A4 + FP8-KV denoising step at 512x928.

Workload: 30 blocks (dim 3072, 24 heads x 128, FFN 14336) over one 3-latent-frame chunk of 16 x 29 tokens (1392),
with a full 21-frame rolling window (8352 cached FP8 tokens + the chunk = 9744 keys) and 512 cross-attention
tokens, random-init W4A4 weights of that architecture (synthetic data; no checkpoint). A step is
WanModel.forward (src/wan_dit_lab/models/model.py:32-84): patch embedding, time embedding and projection, the 30
blocks (each writing its chunk into its FP8 cache and attending over the window), head and unpatchify. The
timed loop replays one HIP graph of the whole step K times; the per-kernel durations (W4A4 GEMM, attention) come
from an instrumented eager step with HIP events on the launch stream.

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
    """One eager step with HIP events around every W4A4 GEMM and attention launch (on the launch stream)."""
    import torch

    from wdl import ops

    rec = {"gemm": [], "attn": []}
    orig_gemm, orig_attn, orig_attn16 = ops.gemm_launch, ops.sage_attn_launch, ops.sage_attn_q16_launch

    def gemm(q, ascales, lora, qweight, *a, **k):
        M = a[3]
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        out = orig_gemm(q, ascales, lora, qweight, *a, **k)
        e1.record()
        rec["gemm"].append((e0, e1, 2.0 * M * ops.out_features(qweight) * q.shape[1] * 64))
        return out

    def attn(q_i8, q_scale, prep, L, sm_scale, out=None):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        r = orig_attn(q_i8, q_scale, prep, L, sm_scale, out)
        e1.record()
        n, H, d = q_i8.shape
        rec["attn"].append((e0, e1, 4.0 * n * L * d * H))
        return r

    def attn16(Q, prep, L, sm_scale, out=None):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        r = orig_attn16(Q, prep, L, sm_scale, out)
        e1.record()
        rec["attn"].append((e0, e1, 4.0 * Q.shape[0] * L * Q.shape[1]))
        return r

    ops.gemm_launch, ops.sage_attn_launch, ops.sage_attn_q16_launch = gemm, attn, attn16
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
    out = {}
    for name, items in rec.items():
        ms = sum(a.elapsed_time(b) for a, b, _ in items)
        flops = sum(f for _, _, f in items)
        out[name] = dict(launches=len(items), ms=ms, tops=flops / (ms * 1e-3) / 1e12 if ms else 0.0)
    return out


COUNTERS = ROOT / "profiles" / "w4a4_gemm_kernel_dit_step_512x928_counters.md"


def gemm_traffic():
    """HBM bytes per W4A4 GEMM launch over the step: FETCH_SIZE and WRITE_SIZE averages of two rocprofv3 --pmc runs
    of this benchmark, each scaled by its reading for a copy of known size (the committed counter summary)."""
    import re

    if not COUNTERS.exists():
        return None
    m = re.search(r"w4a4_gemm_kernel, all launches: HBM bytes per launch \(calibrated\): (\d+)", COUNTERS.read_text())
    return int(m.group(1)) if m else None


def cpu_baseline():
    """The oracle block on the reference's CPU-sized workload (one 16 x 29 = 464-token frame over a 928-token FP8
    cache, 512 context tokens, dim 3072) timed on this host's cores; reported as latent tokens/s of a 30-block
    step."""
    import torch

    from oracle import block as oblock
    from oracle import rope as orope

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    P = oblock.random_logical_block(DIM, FFN, g)
    grid, M, prior = (1, 16, 29), 464, 928
    X = torch.randn(M, DIM, generator=g).to(torch.bfloat16)
    time_in = torch.randn(6, DIM, generator=g) * 0.1
    C = torch.randn(CONTEXT, DIM, generator=g).to(torch.bfloat16)
    freq = orope.freqs(128, 1024, torch.float64).float()
    ck = (torch.randn(1, prior + M, HEADS, 128, generator=g) * 100).clamp(-448, 448).to(torch.float8_e4m3fn)
    cks = torch.rand(1, prior + M, HEADS, 1, generator=g) * 0.02
    ctx = oblock.context_kv(C, P)
    runs = []
    for i in range(3):
        cache = dict(k=ck.clone(), ks=cks.clone(), v=ck.clone(), vs=cks.clone(), at=prior)
        t0 = time.perf_counter()
        oblock.block_forward(X, time_in, P, grid, freq, 2, cache, ctx, HEADS)
        runs.append(time.perf_counter() - t0)
        log(f"bench: cpu oracle block run {i}: {runs[-1]:.2f} s")
    t_block = sorted(runs)[len(runs) // 2]
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return dict(value=M / (BLOCKS * t_block), unit="latent tokens/s", cores=cores, kind="port",
                sample=f"oracle block (CPU restatement, torch {torch.__version__}, fp32/fp64 CPU arithmetic) of "
                       f"one 464-token frame over a 928-token FP8 cache + 512 context tokens, dim 3072; "
                       f"median of 3 runs = {t_block:.2f} s per block, scaled to a 30-block step; CPU {cpu}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of the HIP graph")
    ap.add_argument("--chunks", type=int, default=0, metavar="C",
                    help="also time C whole chunks of the DMD loop (4 levels + write pass + cache commit, eager) "
                         "after the step measurement, as chunk_ms")
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
                   "graph": not args.eager},
        "gemm_tops": g["tops"],
        "gemm_pct_int8_peak": 100 * gemm_frac,
        "gemm_ms_per_step": g["ms"],
        "attention_tops": a["tops"],
        "attention_pct_int8_peak": 100 * a["tops"] / INT8_PEAK_TOPS,
        "attention_ms_per_step": a["ms"],
        "roofline": {"bound": "mfma", "kernel": "w4a4_gemm_kernel", "achieved": g["tops"], "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": gemm_frac, "traffic": gemm_traffic(),
                     "basis": "2*M*N*K int ops per launch (M = 1392 tokens) summed over the step's "
                              f"{g['launches']} W4A4 GEMM launches / their summed HIP-event durations; traffic = "
                              "calibrated HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE; peak = the "
                              "metric's dense int8 MFMA peak (the kernel issues fp6 MFMAs, dense peak 10.1 POP/s: "
                              "against that the fraction is half)"},
    }
    if args.chunks > 0:
        result["chunk_ms"] = chunk_ms(step, args.chunks)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
