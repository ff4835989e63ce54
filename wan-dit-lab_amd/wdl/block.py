"""The quantized Wan DiT block and the 30-block step on MI355X, over the wdl kernels.

WanBlock.forward (src/wan_dit_lab/models/block.py:22-29) with the W4A4 layers installed as the reference's fused
pack installs them (quantization/w4a4.py:336-352: self_attn.qkv FusedQKVAttention, ffn PackedW4A4GeluMLP, every
other linear PackedW4A4Linear) and the FP8 KV cache attended through Sage (generation/causal.py:193-210). The
kernel sequence of one block (about 19 launches, all on the current stream, capturable into one HIP graph):

  act_quant(X; LN + (1 + scale_a), + shift_a)  -> W4A4 qkv -> norm_rope(q, k) -> kv_append(K, V @ at)
  -> sage_prep(cache[:at] ++ K, V) -> sage_attn (int8 Q quantized in the kernel) -> act_quant(A) -> W4A4 o
  (X += gate_a * y, fused)
  act_quant(X; LN3 affine) -> W4A4 cross q -> RMSNorm -> bf16 attention over the context K/V (laid out once per
  prompt; exact fp32 softmax, as the reference's SDPA) -> act_quant -> W4A4 cross o (X += y, fused)
  act_quant(X; LN + (1 + scale_f), + shift_f) -> W4A4 ffn.0 (epilogue: GELU, (h + 0.171875) / s2 quantized
  unsigned, h . proj_down2 partials) -> low-rank sum -> W4A4 ffn.2 (X += gate_f * y, fused)

X is updated in place (a bf16 [M, dim] buffer owned by the caller).

Mixed precision (the benchmark plan's mode; not a mode of the reference, whose FP8 linears are W8A8): attention
projections given as FP8 weight-only parts dict(fp8, fp8_scale, bias) run on wdl_fp8wo_gemm with bf16 inputs (the
norm and modulation through the quantizer kernel's bf16 output), the feed-forward stays W4A4.
"""

from __future__ import annotations

import torch

from wdl import fp8, ops
from wdl.kvcache import KVCache
from wdl.ops import EPI_BF16, EPI_RESIDUAL

LINEARS = ("qkv", "o", "cq", "ck", "cv", "co", "ffn1", "ffn2")


class QuantizedWanBlock:
    """parts: {linear: packed W4A4 parts (w4a4.quantize / pack_parts)} for LINEARS, plus wq, wk, cwq, cwk (bf16
    RMSNorm weights [dim]), n3w, n3b (fp32 LayerNorm-3 affine [dim]) and modulation (fp32 [6, dim]). The caller's
    dicts are not changed: the block keeps shallow copies in which each linear's packed nibbles ([N, K/2], 0.5 B
    per weight) are replaced by the GEMM's tile-blocked fp6 codes (0.75 B per weight), so once the caller drops
    its parts the weights are held once (3.7 GB of fp6 codes for the 30 blocks of Wan 5B instead of that plus
    2.45 GB of nibbles); keep_packed keeps both."""

    def __init__(self, parts: dict, dim: int, heads: int, eps: float = 1e-6, cross_attention: str = "sdpa",
                 keep_packed: bool = False):
        """cross_attention: "sdpa" — bf16 attention with an exact fp32 softmax, what the reference runs for the
        context (scaled_dot_product_attention, causal.py:418-420); "sage" — int8 QK / fp8 PV Sage attention over
        the context too (an opt-in deviation: faster on long prompts, within Sage's error bars)."""
        if cross_attention not in ("sdpa", "sage"):
            raise ValueError(f"cross_attention must be 'sdpa' or 'sage', got {cross_attention!r}")
        parts = {name: dict(t) if name in LINEARS else t for name, t in parts.items()}
        self.p, self.dim, self.heads, self.eps = parts, dim, heads, eps
        self.cross_attention = cross_attention
        dev = parts["ffn1"]["qweight"].device
        for name in LINEARS:  # the GEMM operand: tile-blocked fp6 codes (e3m2 of 2w), expanded once from the nibbles
            if "fp8" in parts[name]:  # an FP8 weight-only attention projection (mixed precision)
                if name in ("ffn1", "ffn2"):
                    raise ValueError("the feed-forward is W4A4 in every mode")
                continue
            parts[name]["wcodes"] = ops.weight_codes(parts[name]["qweight"])
            parts[name]["wspairs"] = ops.scale_pairs(parts[name]["wscales"])  # bf16 or fp16 scales, exactly
            if not keep_packed:
                del parts[name]["qweight"]
        self.ones = torch.ones(dim, device=dev, dtype=torch.float32)
        self.ones_bf16 = torch.ones(dim, device=dev, dtype=torch.bfloat16)

    # --------------------------------------------------------------------------------------- pieces
    def _quant(self, x, name, ln=None, shift=0.0, unsigned=False):
        t = self.p[name]
        return ops.act_quant_launch(x, t["smooth"], t["proj_down"], shift, unsigned, ln=ln)

    def _gemm(self, qa, name, M, out, epilogue=EPI_BF16, gate=None, ln_out=None):
        t = self.p[name]
        q, asc, lora = qa
        return ops.gemm_launch(q, asc, lora, t["wcodes"], t["wspairs"], t["proj_up"], t["bias"], M, out, epilogue,
                               gate, ln_out=ln_out)

    def _apply(self, x, name, out, epilogue=EPI_BF16, gate=None, ln=None, ln_out=None):
        """out (or out += gate * y with EPI_RESIDUAL) for the linear `name` of x (normalized and modulated first
        when ln is given), W4A4 or FP8 weight-only. ln_out (residual): a buffer for the LayerNorm chunk partials of
        the updated rows; returns it when the W4A4 epilogue filled it, else None (the FP8 weight-only GEMM forms
        none)."""
        t = self.p[name]
        if "fp8" in t:
            if ln is not None:  # the quantizer kernel's bf16 copy of the normalized, modulated input
                v = torch.empty_like(x)
                ops.act_quant_launch(x, self.ones_bf16, None, ln=ln, v_out=v)
                x = v
            fp8.weight_only_gemm(x, t["fp8"], t["fp8_scale"], t["bias"], out=out,
                                 gate=gate if epilogue == EPI_RESIDUAL else None)
            return None
        self._gemm(self._quant(x, name, ln=ln), name, x.shape[0], out, epilogue, gate, ln_out=ln_out)
        return ln_out

    def out_features(self, name):
        t = self.p[name]
        return t["fp8"].shape[0] if "fp8" in t else ops.out_features(t["wcodes"])

    def linear(self, x, name):
        out = torch.empty(x.shape[0], self.out_features(name), device=x.device, dtype=torch.bfloat16)
        self._apply(x, name, out)
        return out

    def prepare_context(self, C: torch.Tensor) -> dict:
        """Cross-attention keys and values of a prompt, once per prompt (multi_head_attention.py:21-26;
        causal.Stream.cross, causal.py:557-568): K = RMSNorm(k(C)), V = v(C), laid out for the bf16 attention
        (or quantized to Sage's int8 K / fp8 V with cross_attention="sage")."""
        Kc = self.linear(C, "ck")
        Kn, _ = ops.qk_norm_rope_launch(Kc, None, self.p["cwk"], None, self._nofreq(C.device), (0, 1, 1), 0,
                                        self.eps)
        Vc = self.linear(C, "cv")
        if self.cross_attention == "sdpa":
            return ops.attn_bf16_prep_launch(Kn, Vc)
        H = self.heads
        z8 = torch.zeros(1, 1, H, 128, device=C.device, dtype=torch.uint8)
        z = torch.ones(1, 1, H, 1, device=C.device)
        prep = ops.sage_prep_launch(z8, z, z8, z, Kn, Vc, 0)
        prep["L"] = C.shape[0]
        return prep

    def _nofreq(self, device):
        if not hasattr(self, "_zero_freq"):
            self._zero_freq = torch.zeros(2, 1, 64, device=device)
        return self._zero_freq

    # --------------------------------------------------------------------------------------- forward
    def forward(self, X: torch.Tensor, e: torch.Tensor, grid, freq, start_frame: int, cache: KVCache, ctx: dict,
                ln_in=None, ln_out=None):
        """X bf16 [M, dim] (updated in place and returned); e fp32 [6, dim] = time_in + modulation.
        ln_in: the LayerNorm chunk partials of X (fp32 [M, dim / 32, 2], as the previous block's ln_out), or None;
        ln_out: a buffer of that shape that receives them for the returned X (the feed-forward's residual GEMM
        writes them), or None. Each LayerNorm-fused quantization of the block takes its partials from the residual
        GEMM that wrote X before it where that GEMM is W4A4, and forms them itself otherwise."""
        M, D = X.shape
        H = self.heads
        sh_a, sc_a, g_a, sh_f, sc_f, g_f = e
        dev = X.device
        lnp = torch.empty(2, M, D // 32, 2, device=dev, dtype=torch.float32)  # after o, after cross-o
        # self-attention
        qkv = torch.empty(M, 3 * D, device=dev, dtype=torch.bfloat16)
        self._apply(X, "qkv", qkv, ln=dict(shift=sh_a, scale=sc_a, eps=self.eps, partials=ln_in))
        Q, K = ops.qk_norm_rope_launch(qkv[:, :D], qkv[:, D:2 * D], self.p["wq"], self.p["wk"], freq, grid,
                                       start_frame, self.eps)
        V = qkv[:, 2 * D:]
        A = cache.attend(Q.view(1, M, H, 128), K.view(1, M, H, 128), V.view(1, M, H, 128))
        p_o = self._apply(A.view(M, D), "o", X, EPI_RESIDUAL, g_a, ln_out=lnp[0])
        # cross-attention over the prompt
        qc = torch.empty(M, D, device=dev, dtype=torch.bfloat16)
        n3 = dict(weight=self.p["n3w"], bias=self.p["n3b"], eps=self.eps, partials=p_o)
        self._apply(X, "cq", qc, ln=n3)
        Qc, _ = ops.qk_norm_rope_launch(qc, None, self.p["cwq"], None, self._nofreq(dev), (0, 1, 1), 0,
                                        self.eps)
        if "kp" in ctx:
            Ac = ops.attn_bf16_launch(Qc, ctx, 128 ** -0.5)
        else:
            Ac = ops.sage_attn_q16_launch(Qc, ctx, ctx["L"], 128 ** -0.5)
        p_co = self._apply(Ac, "co", X, EPI_RESIDUAL, self.ones, ln_out=lnp[1])
        # feed forward: the fused W4A4 GELU MLP (the hidden layer goes from the first GEMM's epilogue to the second
        # GEMM as int4 codes, scales and low-rank sums)
        q, asc, lora = self._quant(X, "ffn1", ln=dict(shift=sh_f, scale=sc_f, eps=self.eps, partials=p_co))
        t1, t2 = self.p["ffn1"], self.p["ffn2"]
        hq = ops.gelu_quant_launch(q, asc, lora, t1["wcodes"], t1["wspairs"], t1["proj_up"], t1["bias"], M,
                                   t2["smooth"], t2["proj_down"])
        self._gemm(hq, "ffn2", M, X, EPI_RESIDUAL, g_f, ln_out=ln_out)
        return X


def build_block(P_logical: dict, dim: int, heads: int, device, cross_attention: str = "sdpa") -> QuantizedWanBlock:
    """A QuantizedWanBlock from the logical parts of oracle-style quantization (tests) or of quantize_block."""
    from wdl.w4a4 import pack_parts

    parts = {name: (dict(fp8=P_logical[name]["fp8"].to(device), fp8_scale=P_logical[name]["fp8_scale"].reshape(-1)
                         .float().to(device), bias=P_logical[name]["bias"].to(torch.bfloat16).to(device))
                    if "fp8" in P_logical[name] else pack_parts(P_logical[name], device)) for name in LINEARS}
    for name in ("wq", "wk", "cwq", "cwk"):
        parts[name] = P_logical[name].to(torch.bfloat16).to(device)
    parts["n3w"] = P_logical["n3w"].float().to(device)
    parts["n3b"] = P_logical["n3b"].float().to(device)
    parts["modulation"] = P_logical["modulation"].float().to(device)
    return QuantizedWanBlock(parts, dim, heads, cross_attention=cross_attention)


def random_block(dim: int, ffn: int, heads: int, device, generator=None, mixed: bool = False) -> QuantizedWanBlock:
    """A block of random-init W4A4 weights of the Wan architecture (no SVD: random int4, group scales of an
    N(0, 0.02^2) weight, small low-rank factors), for the step benchmark. mixed: the attention projections FP8
    weight-only instead (an N(0, 0.02^2) weight quantized to e4m3 rows on the GPU), the feed-forward W4A4."""
    from wdl.w4a4 import random_parts

    g = generator
    shapes = dict(qkv=(3 * dim, dim), o=(dim, dim), cq=(dim, dim), ck=(dim, dim), cv=(dim, dim), co=(dim, dim),
                  ffn1=(ffn, dim), ffn2=(dim, ffn))
    parts = {}
    for name, (n, k) in shapes.items():
        if mixed and name not in ("ffn1", "ffn2"):
            wq, ws = fp8.quantize_rows(torch.randn(n, k, generator=g, device=device) * 0.02)
            parts[name] = dict(fp8=wq, fp8_scale=ws.reshape(-1),
                               bias=(torch.randn(n, generator=g, device=device) * 0.02).to(torch.bfloat16))
        else:
            parts[name] = random_parts(n, k, device, g)
    for name in ("wq", "wk", "cwq", "cwk"):
        parts[name] = torch.ones(dim, device=device, dtype=torch.bfloat16)
    parts["n3w"] = torch.ones(dim, device=device)
    parts["n3b"] = torch.zeros(dim, device=device)
    parts["modulation"] = torch.randn(6, dim, generator=g, device=device) / dim ** 0.5
    return QuantizedWanBlock(parts, dim, heads)
