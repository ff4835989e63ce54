"""The quantized Wan DiT block on the CPU, restating src/wan_dit_lab/models/block.py:22-29 with the W4A4 linears
(quantization/w4a4.py:248-262 FusedQKVAttention, 234-245 PackedW4A4GeluMLP), the FP8 KV cache and Sage attention
(generation/causal.py:177-210; kernels/sage_kv.py), in the arithmetic wdl defines for the fused kernels:

  e = time_in + modulation (fp32), chunks shift_a, scale_a, gate_a, shift_f, scale_f, gate_f   (block.py:24)
  x1  = bf16(LN(X) * (1 + scale_a) + shift_a)                     one rounding (norms.ln_mod)
  qkv = W4A4(x1) -> bf16;  Q, K = RoPE(RMSNorm(q)), RoPE(RMSNorm(k));  V = v                (w4a4.py:255-258)
  cache[at:at+n] = quantize_rows(K), quantize_rows(V);  A = Sage(Q; cache[:at] ++ (K, V))   (causal.py:193-210)
  X   = bf16(X + bf16(W4A4(A)) * gate_a)                                                     (block.py:25-26)
  Xc  = bf16(LN3_affine(X));  Qc = RMSNorm(W4A4(Xc));  X = bf16(X + bf16(W4A4(SDPA(Qc; Kc, Vc))))  (block.py:27)
  h   = GELU(W4A4(bf16(LN(X) * (1 + scale_f) + shift_f))) in fp32;  X = bf16(X + bf16(W4A4_u(h)) * gate_f)  (28)
with W4A4_u the second GELU-MLP layer: its INT4 branch quantizes (h + 0.171875) / s2 unsigned and its low-rank
branch reads h itself, the hidden layer never rounded to 16 bits (the fused GELU MLP, w4a4.py:198-204,
w4a4_ops.cpp:42-63; w4a4.gelu_mlp of this oracle). The attention is the blockwise online
softmax of the kernel (sage.attention_online); the cross-attention over the prompt is the exact softmax on
bf16 operands (the reference's SDPA). The reference applies the modulation in bf16 op by op and adds
the residual in bf16 after a bf16 product; the bar against it is the tolerance of tests/test_w4a4.py:62-87.
"""

from __future__ import annotations

import torch

from oracle import fp8 as ofp8
from oracle import norms as onorms
from oracle import rope as orope
from oracle import sage as osage
from oracle import w4a4 as ow

BF = torch.bfloat16


def _lin(x: torch.Tensor, t: dict, shift=0.0, unsigned=False) -> torch.Tensor:
    """A block linear: W4A4 parts (float64 result), or FP8 weight-only parts dict(fp8, fp8_scale, bias) of the
    mixed-precision mode (the bf16 result of w8a16_linear on the bf16 input)."""
    if "fp8" in t:
        return ofp8.w8a16_linear(x.to(BF), t["fp8"], t["fp8_scale"], t["bias"])
    return ow.linear_parts(x, t, shift, unsigned)[0]  # float64


def _rms(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return onorms.rms_norm(x.contiguous(), w)


def context_kv(C: torch.Tensor, P: dict):
    """keys_values (multi_head_attention.py:21-26) of the context C bf16 [Lc, D]: K = RMSNorm(k(C)), V = v(C)."""
    K = _rms(_lin(C, P["ck"]).to(BF), P["cwk"])
    V = _lin(C, P["cv"]).to(BF)
    return K, V


def cross_attention(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, heads: int) -> torch.Tensor:
    """The context attention as the reference computes it: scaled_dot_product_attention on the bf16 Qc, Kc, Vc
    (multi_head_attention.py:37-44; causal.py:418-420 keep SDPA for cross-attention), here the exact softmax in
    float64 -> bf16 [M, D]."""
    M, D = Q.shape
    Q4, K4, V4 = (t.reshape(1, -1, heads, 128) for t in (Q, K, V))
    return osage.attention_exact(Q4, K4.float(), V4.float()).reshape(M, D).to(BF)


def attention(Q: torch.Tensor, cache: dict | None, K: torch.Tensor, V: torch.Tensor, heads: int) -> torch.Tensor:
    """Q, K, V bf16 [M, D] -> bf16 [M, D]; cache = dict(k, ks, v, vs, at) (k fp8 [1, cap, H, 128]) or None."""
    M, D = Q.shape
    Q4, K4, V4 = (t.reshape(1, -1, heads, 128) for t in (Q, K, V))
    if cache is None:
        z8 = torch.zeros(1, 1, heads, 128, dtype=torch.float8_e4m3fn)
        z = torch.ones(1, 1, heads, 1)
        p = osage.prep(Q4, z8, z, z8, z, 0, K4, V4)
    else:
        p = osage.prep(Q4, cache["k"], cache["ks"], cache["v"], cache["vs"], cache["at"], K4, V4)
    return osage.attention_online(p, 128 ** -0.5).reshape(M, D).to(BF)


def block_forward(X: torch.Tensor, time_in: torch.Tensor, P: dict, grid, freq: torch.Tensor, start_frame: int,
                  cache: dict, ctx_kv, heads: int, eps: float = 1e-6):
    """X bf16 [M, D] -> X bf16 [M, D]; stores the chunk's K, V into cache (rows at .. at + M) in place."""
    e = time_in.float().reshape(6, -1) + P["modulation"].float().reshape(6, -1)
    sh_a, sc_a, g_a, sh_f, sc_f, g_f = e
    D = X.shape[1]
    x1 = onorms.ln_mod(X, sh_a, sc_a, eps=eps)
    qkv = _lin(x1, P["qkv"]).to(BF)
    Q = orope.rope_apply(_rms(qkv[:, :D], P["wq"]).reshape(1, -1, heads, 128), grid, freq, start_frame)
    K = orope.rope_apply(_rms(qkv[:, D:2 * D], P["wk"]).reshape(1, -1, heads, 128), grid, freq, start_frame)
    V = qkv[:, 2 * D:].reshape(1, -1, heads, 128)
    at, n = cache["at"], X.shape[0]
    A = attention(Q.reshape(-1, D), cache, K.reshape(-1, D), V.reshape(-1, D), heads)
    for src, cb, sb in ((K, "k", "ks"), (V, "v", "vs")):
        q8, s8 = ofp8.quantize_rows(src)
        cache[cb][:, at:at + n], cache[sb][:, at:at + n] = q8, s8
    y = _lin(A, P["o"]).to(BF)
    X = (X.float() + y.float() * g_a).to(BF)
    xc = onorms.ln_mod(X, None, None, P["n3w"], P["n3b"], eps=eps)
    Qc = _rms(_lin(xc, P["cq"]).to(BF), P["cwq"])
    Kc, Vc = ctx_kv
    Ac = cross_attention(Qc, Kc, Vc, heads)
    yc = _lin(Ac, P["co"]).to(BF)
    X = (X.float() + yc.float()).to(BF)
    x2 = onorms.ln_mod(X, sh_f, sc_f, eps=eps)
    y2 = ow.gelu_mlp(x2, P["ffn1"], P["ffn2"])  # the hidden layer in fp32 (w4a4.py:198-204)
    return (X.float() + y2.float() * g_f).to(BF)


def random_block(dim: int, ffn: int, generator: torch.Generator, rank: int = 32, init: str = "normal"):
    """Float weights of a Wan block: linears N(0, 0.02^2) (init "normal", the benchmark workloads) or torch.nn.Linear's
    default U(-1/sqrt(in), 1/sqrt(in)) (init "torch", the reference's test blocks); RMSNorm weights 1, LN3 affine
    (1, 0), modulation randn / sqrt(dim) (block.py:20)."""
    g = generator
    if init == "torch":
        lin = lambda n, k: ((torch.rand(n, k, generator=g) * 2 - 1) / k ** 0.5,
                            (torch.rand(n, generator=g) * 2 - 1) / k ** 0.5)
    else:
        lin = lambda n, k: (torch.randn(n, k, generator=g) * 0.02, torch.randn(n, generator=g) * 0.02)
    W = {name: lin(*shape) for name, shape in dict(
        q=(dim, dim), k=(dim, dim), v=(dim, dim), o=(dim, dim), cq=(dim, dim), ck=(dim, dim), cv=(dim, dim),
        co=(dim, dim), ffn1=(ffn, dim), ffn2=(dim, ffn)).items()}
    return dict(W=W, wq=torch.ones(dim), wk=torch.ones(dim), cwq=torch.ones(dim), cwk=torch.ones(dim),
                n3w=torch.ones(dim), n3b=torch.zeros(dim), modulation=torch.randn(6, dim, generator=g) / dim ** 0.5)


def quantize_block(B: dict, rank: int = 32) -> dict:
    """The logical W4A4 parts of every linear (q, k, v fused as qkv; ffn2 made for the unsigned shifted input)."""
    W = B["W"]
    P = {}
    qkv_w = torch.cat([W["q"][0], W["k"][0], W["v"][0]])
    qkv_b = torch.cat([W["q"][1], W["k"][1], W["v"][1]])
    P["qkv"] = ow.quantize_weight(qkv_w, qkv_b, rank=rank)
    for name in ("o", "cq", "ck", "cv", "co", "ffn1"):
        P[name] = ow.quantize_weight(*W[name], rank=rank)
    P["ffn2"] = ow.quantize_weight(*W["ffn2"], rank=rank, shift=ow.GELU_SHIFT)
    for name in ("wq", "wk", "cwq", "cwk"):
        P[name] = B[name].to(BF)
    P["n3w"], P["n3b"] = B["n3w"].float(), B["n3b"].float()
    P["modulation"] = B["modulation"].float()
    return P


def random_logical(N: int, K: int, g: torch.Generator, rank: int = 32, scale: float = 0.02, shift: float = 0.0):
    """Logical W4A4 parts of random-init weights without an SVD (int4 in [-7, 7], group scales of an
    N(0, scale^2) weight), for full-size block checks."""
    q = torch.randint(-7, 8, (N, K), generator=g, dtype=torch.int32)
    ws = ((torch.rand(N, K // 64, generator=g) * 0.5 + 0.75) * (3 * scale / 7)).to(BF)
    bias = torch.randn(N, generator=g) * scale
    if shift:
        bias = bias - shift * (q.view(N, K // 64, 64).float() * ws.float()[..., None]).view(N, K).sum(1)
    return dict(q=q, wscales=ws, proj_down=(torch.randn(K, rank, generator=g) / K ** 0.5).to(BF),
                proj_up=(torch.randn(N, rank, generator=g) * scale).to(BF), smooth=torch.ones(K, dtype=BF),
                bias=bias.to(BF))


def fp8_weight_only(N: int, K: int, g: torch.Generator, scale: float = 0.02) -> dict:
    """FP8 weight-only parts of a random-init N(0, scale^2) linear: e4m3 rows with their fp32 scales, bf16 bias."""
    wq, ws = ofp8.quantize_rows(torch.randn(N, K, generator=g) * scale)
    return dict(fp8=wq, fp8_scale=ws, bias=(torch.randn(N, generator=g) * scale).to(BF))


def mixed_precision_block(dim: int, ffn: int, g: torch.Generator) -> dict:
    """The mixed-precision mode's parts: the attention projections (qkv, o, cq, ck, cv, co) FP8 weight-only, the
    feed-forward W4A4 (random_logical)."""
    P = random_logical_block(dim, ffn, g)
    for name, (n, k) in dict(qkv=(3 * dim, dim), o=(dim, dim), cq=(dim, dim), ck=(dim, dim), cv=(dim, dim),
                             co=(dim, dim)).items():
        P[name] = fp8_weight_only(n, k, g)
    return P


def random_logical_block(dim: int, ffn: int, g: torch.Generator) -> dict:
    P = {name: random_logical(n, k, g) for name, (n, k) in dict(
        qkv=(3 * dim, dim), o=(dim, dim), cq=(dim, dim), ck=(dim, dim), cv=(dim, dim), co=(dim, dim),
        ffn1=(ffn, dim)).items()}
    P["ffn2"] = random_logical(dim, ffn, g, shift=ow.GELU_SHIFT)
    for name in ("wq", "wk", "cwq", "cwk"):
        P[name] = (torch.rand(dim, generator=g) * 0.5 + 0.75).to(BF)
    P["n3w"] = torch.rand(dim, generator=g) * 0.5 + 0.75
    P["n3b"] = torch.randn(dim, generator=g) * 0.02
    P["modulation"] = torch.randn(6, dim, generator=g) / dim ** 0.5
    return P


def float_block_forward(X: torch.Tensor, time_in: torch.Tensor, B: dict, grid, freq: torch.Tensor,
                        start_frame: int, cache_kv, ctx: torch.Tensor, heads: int, eps: float = 1e-6):
    """The unquantized block in fp32 (block.py:22-29, multi_head_attention.py:28-44): float linears, exact softmax
    over the cached keys/values cache_kv = (K, V) fp32 [Lc, D] and the chunk; ctx fp32 [Lc2, D] the context."""
    W = B["W"]
    D = X.shape[1]
    lin = lambda x, name: x @ W[name][0].t() + W[name][1]
    rms = lambda x, w: x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w
    e = time_in.float().reshape(6, -1) + B["modulation"].float().reshape(6, -1)
    X = X.float()
    ln = lambda x: torch.nn.functional.layer_norm(x, (D,), eps=eps)
    x1 = ln(X) * (1 + e[1]) + e[0]
    Q = orope.rope_apply(rms(lin(x1, "q"), B["wq"]).reshape(1, -1, heads, 128), grid, freq.double(), start_frame)
    K = orope.rope_apply(rms(lin(x1, "k"), B["wk"]).reshape(1, -1, heads, 128), grid, freq.double(), start_frame)
    V = lin(x1, "v").reshape(1, -1, heads, 128)
    Kc, Vc = cache_kv
    Kall = torch.cat([Kc.reshape(1, -1, heads, 128), K.float()], 1)
    Vall = torch.cat([Vc.reshape(1, -1, heads, 128), V], 1)
    A = osage.attention_exact(Q.float(), Kall, Vall).reshape(-1, D)
    X = X + lin(A, "o") * e[2]
    xc = ln(X) * B["n3w"] + B["n3b"]
    Qc = rms(lin(xc, "cq"), B["cwq"]).reshape(1, -1, heads, 128)
    Kx = rms(lin(ctx, "ck"), B["cwk"]).reshape(1, -1, heads, 128)
    Vx = lin(ctx, "cv").reshape(1, -1, heads, 128)
    X = X + lin(osage.attention_exact(Qc, Kx, Vx).reshape(-1, D), "co")
    x2 = ln(X) * (1 + e[4]) + e[3]
    return X + lin(ow.gelu_tanh(lin(x2, "ffn1")), "ffn2") * e[5]
