"""Kernel timings at the step's shapes, for profiling runs: `python kbench.py attention|cross|prep|gemm|quant
[lib]`.

attention: Sage prep + attention of 1280 and 1392 queries over a full 9744-key window (8352 cached FP8 tokens + the
chunk), 24 x 128 heads; prep: the Sage preparation (K mean and V maxima, int8 K and fp8 V of the whole window) of
the same two shapes; gemm: the W4A4 GEMMs of one block at 1392 tokens (QKV 3072 -> 9216, o 3072 -> 3072 with the
gated residual, FFN-up 3072 -> 14336 with GELU (bf16 out) and fused with the second layer's quantization, FFN-down 14336 -> 3072 with the gated residual), random weights; quant: the activation quantizer with its low-rank down projection at 1392 tokens
(K 3072 with the fused LayerNorm and modulation, its statistics formed in the launch or from chunk partials given,
K 3072 plain, K 14336 unsigned).
Each shape is captured into a HIP graph of 10 launches and replayed; one line per shape with microseconds per
launch (gemm: the launch the library picks and the one-pass launch, alternated three times, the best of each).
An optional library path replaces lib/libwdl.so (for comparing builds).
"""

from __future__ import annotations

import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "wan-dit-lab_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))


def _replay_us(fn, reps: int = 10) -> float:
    import torch

    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e3


def attention():
    import torch

    from wdl import ops

    dev, H = "cuda", 24
    g = torch.Generator(device=dev).manual_seed(0)
    for n, at in ((1280, 8464), (1392, 8352)):
        L = at + n
        ck = (torch.randn(1, at, H, 128, device=dev, generator=g) * 50).clamp(-448, 448).to(torch.float8_e4m3fn)
        cks = torch.rand(1, at, H, 1, device=dev, generator=g) * 0.02
        K, V, Q = (torch.randn(n, H * 128, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
        prep = ops.sage_prep_launch(ck.view(torch.uint8), cks, ck.view(torch.uint8), cks, K, V, at)
        out = torch.empty(n, H * 128, device=dev, dtype=torch.bfloat16)
        us = _replay_us(lambda: ops.sage_attn_q16_launch(Q, prep, L, 128 ** -0.5, out))
        print(f"attention n={n} L={L}: {us:.1f} us ({4 * n * L * 128 * H / us / 1e6:.0f} TOP/s)", flush=True)


def chunk():
    """The chunk-causal attention workload at 704x1280: 2640 queries (3 frames of 880) over 6600 / 15840 cached +
    the chunk's keys, 24 heads, without and with the block-causal mask per latent frame."""
    import torch

    from wdl import ops

    dev, H, n = "cuda", 24, 2640
    g = torch.Generator(device=dev).manual_seed(0)
    for at in (6600, 15840):
        L = at + n
        ck = (torch.randn(1, at, H, 128, device=dev, generator=g) * 50).clamp(-448, 448).to(torch.float8_e4m3fn)
        cks = torch.rand(1, at, H, 1, device=dev, generator=g) * 0.02
        K, V, Q = (torch.randn(n, H * 128, device=dev, generator=g).to(torch.bfloat16) for _ in range(3))
        prep = ops.sage_prep_launch(ck.view(torch.uint8), cks, ck.view(torch.uint8), cks, K, V, at)
        out = torch.empty(n, H * 128, device=dev, dtype=torch.bfloat16)
        for frame in (0, 880):
            us = _replay_us(lambda: ops.sage_attn_q16_launch(Q, prep, L, 128 ** -0.5, out, frame_tokens=frame))
            # the masked workload: each query's visible keys
            keys = n * L if not frame else sum(min(L, at + (q // frame + 1) * frame) for q in range(0, n, 16)) * 16
            print(f"chunk attention n={n} L={L} frame={frame}: {us:.1f} us ({4 * keys * 128 * H / us / 1e6:.0f} "
                  f"TOP/s over the visible keys)", flush=True)


def cross():
    """The cross-attention of the step (1392 queries over 512 prompt keys, 24 x 128 heads): bf16 attention (the
    reference's SDPA semantics) and Sage (int8 QK, fp8 PV), each over K / V laid out once."""
    import torch

    from wdl import ops

    dev, H, n, L = "cuda", 24, 1392, 512
    g = torch.Generator(device=dev).manual_seed(0)
    Q, K, V = (torch.randn(m, H * 128, device=dev, generator=g).to(torch.bfloat16) for m in (n, L, L))
    pb = ops.attn_bf16_prep_launch(K, V)
    out = torch.empty(n, H * 128, device=dev, dtype=torch.bfloat16)
    for m in (1280, n):  # 240 and 264 (query tile, head) pairs on 256 CUs
        us = _replay_us(lambda: ops.attn_bf16_launch(Q[:m], pb, 128 ** -0.5, out[:m]))
        print(f"cross bf16 n={m} L={L}: {us:.1f} us ({4 * m * L * 128 * H / us / 1e6:.0f} TFLOP/s)", flush=True)
    z8 = torch.zeros(1, 1, H, 128, device=dev, dtype=torch.uint8)
    one = torch.ones(1, 1, H, 1, device=dev)
    ps = ops.sage_prep_launch(z8, one, z8, one, K, V, 0)
    us = _replay_us(lambda: ops.sage_attn_q16_launch(Q, ps, L, 128 ** -0.5, out))
    print(f"cross sage n={n} L={L}: {us:.1f} us ({4 * n * L * 128 * H / us / 1e6:.0f} TOP/s)", flush=True)


def prep():
    import torch

    from wdl import ops

    dev, H = "cuda", 24
    g = torch.Generator(device=dev).manual_seed(0)
    for n, at in ((1280, 8464), (1392, 8352)):
        ck = (torch.randn(1, at, H, 128, device=dev, generator=g) * 50).clamp(-448, 448).to(torch.float8_e4m3fn)
        cks = torch.rand(1, at, H, 1, device=dev, generator=g) * 0.02
        K, V = (torch.randn(n, H * 128, device=dev, generator=g).to(torch.bfloat16) for _ in range(2))
        us = _replay_us(lambda: ops.sage_prep_launch(ck.view(torch.uint8), cks, ck.view(torch.uint8), cks, K, V, at))
        L = at + n
        moved = 2 * (2 * at * H * 132 + 2 * n * H * 256) + 2 * L * H * 128  # inputs read twice, outputs written once
        print(f"prep n={n} L={L}: {us:.1f} us ({moved / us / 1e3:.0f} GB/s)", flush=True)
        stats = ops.sage_cache_stats_launch(ck.view(torch.uint8), cks, ck.view(torch.uint8), cks, at)
        us_c = _replay_us(lambda: ops.sage_prep_launch(ck.view(torch.uint8), cks, ck.view(torch.uint8), cks, K, V, at,
                                                       cache_stats=stats))
        us_s = _replay_us(lambda: ops.sage_cache_stats_launch(ck.view(torch.uint8), cks, ck.view(torch.uint8), cks,
                                                              at, out=stats))
        print(f"prep n={n} L={L} from cached statistics: {us_c:.1f} us; the statistics of the {at} cached rows: "
              f"{us_s:.1f} us", flush=True)


def gemm():
    import torch

    from wdl import ops, w4a4

    dev, M = "cuda", 1392
    g = torch.Generator(device=dev).manual_seed(0)
    for name, N, K, epi in (("qkv", 9216, 3072, ops.EPI_BF16), ("o", 3072, 3072, ops.EPI_RESIDUAL),
                            ("ffn1", 14336, 3072, ops.EPI_GELU), ("ffn2", 3072, 14336, ops.EPI_RESIDUAL)):
        t = w4a4.random_parts(N, K, dev, g)
        wc = ops.as_codes(t["qweight"], K)
        wsp = ops.scale_pairs(t["wscales"])
        x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        q, asc, lora = ops.act_quant_launch(x, t["smooth"], t["proj_down"])
        out = torch.randn(M, N, device=dev, generator=g).to(torch.bfloat16)
        gate = torch.rand(N, device=dev) if epi == ops.EPI_RESIDUAL else None
        best = {}
        for split in (True, False) * 3:  # the launch the library picks / the one-pass launch, alternated
            us = _replay_us(lambda: ops.gemm_launch(q, asc, lora, wc, wsp, t["proj_up"], t["bias"], M, out, epi,
                                                    gate, stream_k=split))
            best[split] = min(us, best.get(split, us))
        for split, us in best.items():
            print(f"gemm {name} {M}x{N}x{K}{'' if split else ' one-pass'}: {us:.1f} us "
                  f"({2 * M * N * K / us / 1e6:.0f} TOP/s)", flush=True)
        if name == "ffn1":  # the fused GELU MLP's first GEMM (epilogue: GELU, second layer's int4 input, low rank)
            s2 = torch.ones(N, device=dev, dtype=torch.bfloat16)
            pd2 = (torch.randn(32, N, device=dev, generator=g) / N ** 0.5).to(torch.bfloat16)
            us = _replay_us(lambda: ops.gelu_quant_launch(q, asc, lora, wc, wsp, t["proj_up"], t["bias"],
                                                          M, s2, pd2))
            print(f"gemm ffn1 fused {M}x{N}x{K}: {us:.1f} us ({2 * M * N * K / us / 1e6:.0f} TOP/s, with the "
                  f"low-rank sum launch)", flush=True)


def fp8():
    """The FP8 W8A8 linears (fp8.py's DynamicFp8Linear rows / tensor: e4m3 activations quantized per token or per
    tensor on every call, e4m3 weights) on the W4A4 sweep's shapes at 1392 and 2640 tokens: the activation quantizer
    and the FP8 GEMM timed together and the GEMM alone."""
    import torch

    from wdl import fp8

    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0)
    for M in (1392, 2640):
        for name, N, K in (("qkv", 9216, 3072), ("o", 3072, 3072), ("ffn1", 14336, 3072), ("ffn2", 3072, 14336)):
            x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
            for rows in (True, False):
                wq, ws = fp8.quantize_padded(torch.randn(N, K, device=dev, generator=g) * 0.02, rows=rows, pad=1)
                q, s = fp8.quantize_padded(x, rows=rows)
                us_g = _replay_us(lambda: fp8.gemm(q, s, M, wq, ws, None, rows=rows))
                us = _replay_us(lambda: fp8.gemm(*fp8.quantize_padded(x, rows=rows), M, wq, ws, None, rows=rows))
                print(f"fp8 {'rows' if rows else 'tensor'} {name} {M}x{N}x{K}: GEMM {us_g:.1f} us "
                      f"({2 * M * N * K / us_g / 1e6:.0f} TOP/s), with the activation quantizer {us:.1f} us",
                      flush=True)


def fp8wo():
    """The FP8 weight-only attention projections (bf16 activations, e4m3 weights with row scales) at 1392 and 2640
    tokens: QKV 3072 -> 9216, o 3072 -> 3072."""
    import torch

    from wdl import fp8

    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0)
    for M in (1392, 2640):
        for name, N, K in (("qkv", 9216, 3072), ("o", 3072, 3072)):
            x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
            wq, ws = fp8.quantize_rows(torch.randn(N, K, device=dev, generator=g) * 0.02)
            out = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
            us = _replay_us(lambda: fp8.weight_only_gemm(x, wq, ws.reshape(-1), None, out=out))
            print(f"fp8 weight-only {name} {M}x{N}x{K}: {us:.1f} us ({2 * M * N * K / us / 1e6:.0f} TFLOP/s)",
                  flush=True)


def quant():
    import torch

    from wdl import ops, w4a4

    dev, M = "cuda", 1392
    g = torch.Generator(device=dev).manual_seed(0)
    for name, K, ln, unsigned in (("ln", 3072, True, False), ("ln from partials", 3072, True, False),
                                  ("plain", 3072, False, False), ("unsigned", 14336, False, True)):
        t = w4a4.random_parts(64, K, dev, g)
        x = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
        lnd = dict(shift=torch.randn(K, device=dev, generator=g) * 0.1, scale=torch.randn(K, device=dev,
                   generator=g) * 0.1, weight=None, bias=None, eps=1e-6) if ln else None
        if name == "ln from partials":  # the chunk partials a residual GEMM epilogue would have written
            xs = x.float().view(M, K // 32, 32)
            s = xs.sum(-1)
            lnd["partials"] = torch.stack((s, ((xs - (s / 32)[..., None]) ** 2).sum(-1)), -1).contiguous()
        us = _replay_us(lambda: ops.act_quant_launch(x, t["smooth"], t["proj_down"], 0.171875 if unsigned else 0.0,
                                                     unsigned, ln=lnd))
        print(f"quant {name} {M}x{K}: {us:.1f} us ({M * K * 2 / us / 1e3:.0f} GB/s of x)", flush=True)


def main(argv):
    if len(argv) < 2 or argv[1] not in ("attention", "chunk", "cross", "prep", "gemm", "quant", "fp8", "fp8wo"):
        raise SystemExit("usage: python kbench.py attention|chunk|cross|prep|gemm|quant|fp8|fp8wo [library path]")
    if len(argv) > 2:
        from wdl import _lib

        _lib.LIB_PATH = Path(argv[2])
    {"attention": attention, "chunk": chunk, "cross": cross, "prep": prep, "gemm": gemm, "quant": quant, "fp8": fp8,
     "fp8wo": fp8wo}[argv[1]]()


if __name__ == "__main__":
    main(sys.argv)
