"""CPU oracle of the quantized Wan DiT block hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU and in plain torch/numpy, the arithmetic of the reference's hot path
(TieBeTie/wan-dit-lab): FP8 row quantization, SVDQuant W4A4 linears, the per-token activation quantizer, 3D RoPE,
RMSNorm/LayerNorm/modulation, the Sage-2 preparation (K mean, int8 K/Q, fp8 V) and quantized attention, and the
Wan block. Every function cites the reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only to check results (or as the
timed CPU baseline). The product path (the wdl package and lib/libwdl.so) never imports or calls it.

Pinning (what checks each function beyond its own formula) is listed in each module's docstring; functions whose
result no known answer, closed form or invariant fixes say "parity unpinned" there.
"""
