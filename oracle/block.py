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
softmax of the kernel (sage.attention_online); the cross-attention over the prompt, and the self-attention of a
chunk with no cache, is the exact softmax on bf16 operands (the reference's SDPA). The reference applies the
modulation in bf16 op by op and adds the residual in bf16 after a bf16 product; the bar against it is the
tolerance of tests/test_w4a4.py:62-87.

The composition (which chunk of the modulation goes where, the gates, norm3's affine, RMSNorm weights and RoPE) is
one function, _compose, shared by block_forward and float_block_forward (the unquantized fp32 block); the reference's
own fp32 WanBlock and WanModel pin it through tests/golden/block_fixtures.npz (tests/test_oracle_block.py).

Test infrastructure: only tests/, the smoke check and the benchmark's CPU baseline import this package.
"""

from __future__ import annotations

import torch

from oracle import fp8 as ofp8
from oracle import norms as onorms
from oracle import rope as orope
from oracle import sage as osage
from oracle import w4a4 as ow

BF = torch.bfloat16


def _lin(x: torch.Tensor, t: dict) -> torch.Tensor:
    """A block linear: W4A4 parts (float64 result), or FP8 weight-only parts dict(fp8, fp8_scale, bias) of the
    mixed-precision mode (the bf16 result of w8a16_linear on the bf16 input)."""
    if "fp8" in t:
        return ofp8.w8a16_linear(x.to(BF), t["fp8"], t["fp8_scale"], t["bias"])
    return ow.linear_parts(x, t)[0]  # float64


def _rms(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return onorms.rms_norm(x.contiguous(), w)


# ------------------------------------------------------------------------------------------------ composition
# WanBlock.forward (block.py:22-29) and MultiHeadAttention.forward (multi_head_attention.py:21-44) are stated once,
# here, over an `ops` object that supplies the arithmetic: _QuantOps (wdl's kernels' arithmetic) or _FloatOps (the
# unquantized fp32 block). Both oracle blocks run this one composition, so the golden fixtures of the reference's
# own fp32 WanBlock (tests/golden/block_fixtures.npz) pin the wiring of both: the order of the six modulation
# chunks, which gate goes where, the affine norm3, which RMSNorm weight goes with Q and K, RoPE on Q and K only.

def _compose(X: torch.Tensor, e: torch.Tensor, P: dict, ops, heads: int) -> torch.Tensor:
    """X [M, D] -> X [M, D] after the three residual sub-layers."""
    M, D = X.shape
    heads4 = lambda t: t.reshape(1, -1, heads, D // heads)
    shift_a, scale_a, gate_a, shift_f, scale_f, gate_f = e  # (time_in + modulation).chunk(6) (block.py:24)
    x = ops.norm_mod(X, shift_a, scale_a)  # norm1(X) * (1 + scale) + shift (block.py:25)
    q, k, v = ops.qkv(x)  # self.q, self.k, self.v (multi_head_attention.py:30-31)
    Q = ops.rope(heads4(ops.rms(q, P["wq"])))  # norm_q, then rope_apply (30, 33-34)
    K = ops.rope(heads4(ops.rms(k, P["wk"])))  # norm_k (24)
    A = ops.self_attend(Q, K, heads4(v))
    X = ops.add(X, ops.linear(A.reshape(M, D), "o"), gate_a)  # X + self_attn(...) * gate (block.py:25-26)
    xc = ops.norm_affine(X, P["n3w"], P["n3b"])  # norm3, elementwise_affine=True (block.py:18, 27)
    Qc = heads4(ops.rms(ops.linear(xc, "cq"), P["cwq"]))  # no RoPE on cross-attention (multi_head_attention.py:32)
    Kc, Vc = ops.context
    X = ops.add(X, ops.linear(ops.cross_attend(Qc, heads4(Kc), heads4(Vc)).reshape(M, D), "co"), None)  # (27)
    x2 = ops.norm_mod(X, shift_f, scale_f)
    return ops.add(X, ops.ffn(x2), gate_f)  # X + ffn(...) * gate (block.py:28)


def _context(C: torch.Tensor, P: dict, ops):
    """keys_values (multi_head_attention.py:21-26) of the context C [Lc, D]: K = norm_k(k(C)), V = v(C)."""
    return ops.rms(ops.linear(C, "ck"), P["cwk"]), ops.linear(C, "cv")


class _QuantOps:
    """The quantized block's arithmetic (wdl's fused kernels): LayerNorm + modulation with one bf16 rounding, W4A4
    (or FP8 weight-only) linears rounded to bf16, the fused q|k|v linear, Sage attention over the FP8 cache (whose
    rows at .. at + M receive the chunk's keys and values), the cross-attention as the exact softmax on bf16
    operands, the fused GELU MLP, residuals rounded once to bf16."""

    def __init__(self, P, grid=None, freq=None, start_frame=0, cache=None, ctx=None, eps=1e-6):
        self.P, self.grid, self.freq, self.start, self.cache, self.context, self.eps = \
            P, grid, freq, start_frame, cache, ctx, eps

    def norm_mod(self, X, shift, scale):
        return onorms.ln_mod(X, shift, scale, eps=self.eps)

    def norm_affine(self, X, w, b):
        return onorms.ln_mod(X, None, None, w, b, eps=self.eps)

    def linear(self, x, name):
        return _lin(x, self.P[name]).to(BF)

    def qkv(self, x):
        return self.linear(x, "qkv").chunk(3, dim=1)  # one fused linear [3 D, D] (w4a4.py:255)

    def rms(self, x, w):
        return _rms(x, w)

    def rope(self, X4):
        return orope.rope_apply(X4, self.grid, self.freq, self.start)

    def self_attend(self, Q, K, V):
        heads = Q.shape[2]
        A = attention(Q.reshape(Q.shape[1], -1), self.cache, K.reshape(K.shape[1], -1),
                      V.reshape(V.shape[1], -1), heads)
        if self.cache is not None:
            at, n = self.cache["at"], K.shape[1]
            for src, cb, sb in ((K, "k", "ks"), (V, "v", "vs")):
                q8, s8 = ofp8.quantize_rows(src)
                self.cache[cb][:, at:at + n], self.cache[sb][:, at:at + n] = q8, s8
        return A

    def cross_attend(self, Q, K, V):
        return cross_attention(Q.reshape(Q.shape[1], -1), K.reshape(K.shape[1], -1), V.reshape(V.shape[1], -1),
                               Q.shape[2])

    def add(self, X, y, gate):
        return (X.float() + (y.float() if gate is None else y.float() * gate)).to(BF)

    def ffn(self, x):
        return ow.gelu_mlp(x, self.P["ffn1"], self.P["ffn2"])  # the hidden layer in fp32 (w4a4.py:198-204)


class _FloatOps:
    """The unquantized block in fp32: float linears, exact softmax attention (over the cached keys and values and
    the chunk), torch's LayerNorm, the RMSNorm formula, GELU tanh."""

    def __init__(self, B, grid=None, freq=None, start_frame=0, cache_kv=None, ctx=None, eps=1e-6):
        self.W, self.grid, self.freq, self.start, self.cache_kv, self.eps = \
            B["W"], grid, freq, start_frame, cache_kv, eps
        self.context = None if ctx is None else _context(ctx.float(), B, self)

    def norm_mod(self, X, shift, scale):
        return self._ln(X) * (1 + scale) + shift

    def norm_affine(self, X, w, b):
        return self._ln(X) * w + b

    def _ln(self, X):
        return torch.nn.functional.layer_norm(X, (X.shape[1],), eps=self.eps)

    def linear(self, x, name):
        w, b = self.W[name]
        return x @ w.t() + b

    def qkv(self, x):
        return self.linear(x, "q"), self.linear(x, "k"), self.linear(x, "v")

    def rms(self, x, w):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps) * w.float()

    def rope(self, X4):
        return orope.rope_apply(X4, self.grid, self.freq.double(), self.start).float()

    def self_attend(self, Q, K, V):
        Kc, Vc = self.cache_kv
        heads = Q.shape[2]
        Kall = torch.cat([Kc.reshape(1, -1, heads, 128).float(), K.float()], 1)
        Vall = torch.cat([Vc.reshape(1, -1, heads, 128).float(), V.float()], 1)
        return osage.attention_exact(Q.float(), Kall, Vall)

    def cross_attend(self, Q, K, V):
        return osage.attention_exact(Q, K, V)

    def add(self, X, y, gate):
        return X + (y if gate is None else y * gate)

    def ffn(self, x):
        return self.linear(ow.gelu_tanh(self.linear(x, "ffn1")), "ffn2")


def context_kv(C: torch.Tensor, P: dict):
    """keys_values of the context C bf16 [Lc, D] in the quantized block's arithmetic: bf16 K = RMSNorm(k(C)),
    V = v(C), [Lc, D] each."""
    return _context(C, P, _QuantOps(P))


def cross_attention(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, heads: int) -> torch.Tensor:
    """The context attention as the reference computes it: scaled_dot_product_attention on the bf16 Qc, Kc, Vc
    (multi_head_attention.py:37-44; causal.py:418-420 keep SDPA for cross-attention), here the exact softmax in
    float64 -> bf16 [M, D]."""
    M, D = Q.shape
    Q4, K4, V4 = (t.reshape(1, -1, heads, 128) for t in (Q, K, V))
    return osage.attention_exact(Q4, K4.float(), V4.float()).reshape(M, D).to(BF)


def attention(Q: torch.Tensor, cache: dict | None, K: torch.Tensor, V: torch.Tensor, heads: int) -> torch.Tensor:
    """Q, K, V bf16 [M, D] -> bf16 [M, D]. cache = dict(k, ks, v, vs, at) (k fp8 [1, cap, H, 128]): Sage attention
    over the cache rows [0, at) and the chunk (KVCache.attend, causal.py:193-210; sage_kv.attend). cache None: the
    chunk attends to itself through scaled_dot_product_attention on the bf16 operands
    (multi_head_attention.py:37-44; quantization/w4a4.py:259-261), the exact softmax here."""
    M, D = Q.shape
    if cache is None:
        return cross_attention(Q, K, V, heads)
    Q4, K4, V4 = (t.reshape(1, -1, heads, 128) for t in (Q, K, V))
    p = osage.prep(Q4, cache["k"], cache["ks"], cache["v"], cache["vs"], cache["at"], K4, V4)
    return osage.attention_online(p, 128 ** -0.5).reshape(M, D).to(BF)


def block_forward(X: torch.Tensor, time_in: torch.Tensor, P: dict, grid, freq: torch.Tensor, start_frame: int,
                  cache: dict | None, ctx_kv, heads: int, eps: float = 1e-6):
    """X bf16 [M, D] -> X bf16 [M, D]; stores the chunk's K, V into cache (rows at .. at + M) in place. cache None:
    no cache, the chunk attends to itself in bf16 (the reference's SDPA branch)."""
    e = time_in.float().reshape(6, -1) + P["modulation"].float().reshape(6, -1)
    ops = _QuantOps(P, grid, freq, start_frame, cache, ctx_kv, eps)
    return _compose(X, e, P, ops, heads)


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


def mixed_precision_block(dim: int, ffn: int, g: torch.Generator, scale: float = 0.02) -> dict:
    """The mixed-precision mode's parts: the attention projections (qkv, o, cq, ck, cv, co) FP8 weight-only
    (N(0, 0.02^2) weights), the feed-forward W4A4 (random_logical at `scale`)."""
    P = random_logical_block(dim, ffn, g, scale=scale)
    for name, (n, k) in dict(qkv=(3 * dim, dim), o=(dim, dim), cq=(dim, dim), ck=(dim, dim), cv=(dim, dim),
                             co=(dim, dim)).items():
        P[name] = fp8_weight_only(n, k, g)
    return P


def random_logical_block(dim: int, ffn: int, g: torch.Generator, scale: float = 0.02) -> dict:
    """Logical W4A4 parts of every linear (random_logical at `scale`: int4 uniform in [-7, 7], so the weights' own
    standard deviation is about 1.85 scale), RMSNorm / LN3 weights near 1, modulation randn / sqrt(dim)."""
    P = {name: random_logical(n, k, g, scale=scale) for name, (n, k) in dict(
        qkv=(3 * dim, dim), o=(dim, dim), cq=(dim, dim), ck=(dim, dim), cv=(dim, dim), co=(dim, dim),
        ffn1=(ffn, dim)).items()}
    P["ffn2"] = random_logical(dim, ffn, g, scale=scale, shift=ow.GELU_SHIFT)
    for name in ("wq", "wk", "cwq", "cwk"):
        P[name] = (torch.rand(dim, generator=g) * 0.5 + 0.75).to(BF)
    P["n3w"] = torch.rand(dim, generator=g) * 0.5 + 0.75
    P["n3b"] = torch.randn(dim, generator=g) * 0.02
    P["modulation"] = torch.randn(6, dim, generator=g) / dim ** 0.5
    return P


def float_block_forward(X: torch.Tensor, time_in: torch.Tensor, B: dict, grid, freq: torch.Tensor,
                        start_frame: int, cache_kv, ctx: torch.Tensor, heads: int, eps: float = 1e-6):
    """The unquantized block in fp32 (block.py:22-29, multi_head_attention.py:21-44): float linears, exact softmax
    over the cached keys/values cache_kv = (K, V) fp32 [Lc, D] and the chunk; ctx fp32 [Lc2, D] the context."""
    e = time_in.float().reshape(6, -1) + B["modulation"].float().reshape(6, -1)
    ops = _FloatOps(B, grid, freq, start_frame, cache_kv, ctx, eps)
    return _compose(X.float(), e, B, ops, heads)
