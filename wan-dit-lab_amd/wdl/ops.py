"""The torch operators wdl::* over the C ABI of lib/libwdl.so.

Each operator is a `torch.library.custom_op` whose implementation hands raw device pointers, sizes and the current
HIP stream to one `wdl_*` launcher, and whose fake (Meta) implementation gives the output shapes, so torch.compile
and graph capture see one opaque op, as the reference's TORCH_LIBRARY ops live::* are
(native/ops/w4a4_ops.cpp:79-95; native/ops/sage_ops.cpp:28-35). Outputs and workspaces are allocated here, by
torch, on the current stream; the library allocates nothing.
"""

from __future__ import annotations

import weakref

import torch

from wdl import _lib

DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# ------------------------------------------------------------------------------------------------ KV cache append

@torch.library.custom_op("wdl::store_kv_fp8", mutates_args=("cache_k", "cache_ks", "cache_v", "cache_vs"))
def store_kv_fp8_op(k: torch.Tensor, v: torch.Tensor, cache_k: torch.Tensor, cache_ks: torch.Tensor,
                    cache_v: torch.Tensor, cache_vs: torch.Tensor, at: int) -> None:
    b, n, h, d = k.shape
    if k.numel() == 0:
        return
    _lib.call("wdl_kv_append_fp8", ptr(k), DTYPE_CODE[k.dtype], _lib.i64s(k.stride()), ptr(v), DTYPE_CODE[v.dtype],
              _lib.i64s(v.stride()), b, n, h, d, ptr(cache_k), ptr(cache_ks), ptr(cache_v), ptr(cache_vs),
              cache_k.shape[1], at, stream_of(k))


@store_kv_fp8_op.register_fake
def _(k, v, cache_k, cache_ks, cache_v, cache_vs, at):
    return None


# ------------------------------------------------------------------------------------------------ W4A4

ROWS_PAD = 128  # activation rows padded to a multiple (GEMM token tile)
RANK = 32


BLOCK = 128  # rows per tile of the GEMM's blocked operands
ROW6 = 48    # bytes of one row's 64-deep group of fp6 codes


def padded_rows(m: int) -> int:
    return (m + ROWS_PAD - 1) // ROWS_PAD * ROWS_PAD


EPI_BF16, EPI_F32, EPI_RESIDUAL, EPI_GELU = 0, 1, 2, 3


def act_quant_launch(x, smooth, proj_down_t, qshift=0.0, unsigned=False, *, ln=None, v_out=None):
    """x bf16 [M, K] (rows 16-byte aligned) -> (q fp6 codes of the int4 values, tile-blocked uint8
    [Mp/128, K/64, 128, 48] (decode_acts gives the [Mp, K] integers), ascales bf16 [K/64, Mp], lora fp32 [Mp, 32]
    or None).
    ln: dict(shift, scale, weight, bias, eps, partials) fuses LayerNorm + modulation; partials: the LayerNorm chunk
    partials of x (fp32 [M, K / 32, 2], as gemm_launch's ln_out writes them), or None to form them here."""
    M, K = x.shape
    Mp = padded_rows(M)
    q = torch.empty(Mp // BLOCK, K // 64, BLOCK, ROW6, device=x.device, dtype=torch.uint8)
    ascales = torch.empty(K // 64, Mp, device=x.device, dtype=torch.bfloat16)
    lora = None if proj_down_t is None else torch.empty(Mp, RANK, device=x.device, dtype=torch.float32)
    ln = ln or {}
    ws = torch.empty(_lib.library().wdl_act_quant_workspace_floats(Mp, K), device=x.device, dtype=torch.float32)
    _lib.call("wdl_act_quant_w4", ptr(x), x.stride(0), M, K, ptr(smooth), float(qshift), int(unsigned),
              ptr(proj_down_t), RANK, ptr(q), ptr(ascales), ptr(lora), Mp, ptr(ln.get("shift")), ptr(ln.get("scale")),
              ptr(ln.get("weight")), ptr(ln.get("bias")), int(bool(ln)), float(ln.get("eps", 1e-6)),
              ptr(ln.get("partials")), ptr(v_out), ptr(ws), stream_of(x))
    return q, ascales, lora


# ---- the GEMM's operand format (tile-blocked fp6 codes): weights w in [-8, 7] as e3m2 codes of 2w, activations
# q in [-8, 15] as e2m3 codes of q / 2, value k of a row's 64-deep group in half k // 32 at position k % 32, the 32
# codes of a half packed 6 bits each (24 bytes), a row's group stored as [half 0 bytes 0..15][half 1 bytes 0..15]
# [half 0 bytes 16..23][half 1 bytes 16..23] (48 bytes), a matrix [R, K] as [R/128, K/64, 128, 48]. These torch
# helpers state the format for callers that build or inspect operands; the product path writes it on the GPU.


def _e3m2_value(c: int) -> float:
    s, e, m = -1 if c & 32 else 1, (c >> 2) & 7, c & 3
    return s * (m / 16 if e == 0 else 2.0 ** (e - 3) * (1 + m / 4))


def _e2m3_value(c: int) -> float:
    s, e, m = -1 if c & 32 else 1, (c >> 3) & 3, c & 7
    return s * (m / 8 if e == 0 else 2.0 ** (e - 1) * (1 + m / 8))


def _code_tables():
    # value -> code for the integer range of each side, and code -> integer value (a code of no integer decodes
    # to -128)
    w_dec = torch.full((64,), -128, dtype=torch.int32)
    a_dec = torch.full((64,), -128, dtype=torch.int32)
    w_enc = torch.zeros(16, dtype=torch.int64)
    a_enc = torch.zeros(24, dtype=torch.int64)
    for c in range(64):
        wv, av = _e3m2_value(c) / 2, _e2m3_value(c) * 2
        if wv == int(wv) and -8 <= wv <= 7 and not (c == 32):
            w_dec[c] = int(wv)
            w_enc[int(wv) + 8] = c
        if av == int(av) and -8 <= av <= 15 and not (c == 32):
            a_dec[c] = int(av)
            a_enc[int(av) + 8] = c
    return w_enc, w_dec, a_enc, a_dec


_W_ENC, _W_DEC, _A_ENC, _A_DEC = _code_tables()


def _pack6(codes: torch.Tensor) -> torch.Tensor:
    R, K = codes.shape
    if R % BLOCK or K % 64:
        raise ValueError(f"tile-blocked operands need rows % {BLOCK} == 0 and K % 64 == 0, got {tuple(codes.shape)}")
    c = codes.to(torch.int64).reshape(R, K // 64, 2, 8, 4)  # row, group, half, quad, code
    v = c[..., 0] | (c[..., 1] << 6) | (c[..., 2] << 12) | (c[..., 3] << 18)
    b = torch.stack([v & 255, (v >> 8) & 255, v >> 16], -1).reshape(R, K // 64, 2, 24)
    rowg = torch.cat([b[:, :, 0, :16], b[:, :, 1, :16], b[:, :, 0, 16:], b[:, :, 1, 16:]], -1)  # [R, G, 48]
    return rowg.to(torch.uint8).reshape(R // BLOCK, BLOCK, K // 64, ROW6).permute(0, 2, 1, 3).contiguous()


def _unpack6(t: torch.Tensor) -> torch.Tensor:
    if t.dim() != 4 or t.shape[2] != BLOCK or t.shape[3] != ROW6:
        raise ValueError(f"tile-blocked fp6 operands have shape [R/128, K/64, 128, 48], got {tuple(t.shape)}")
    nr, ng = t.shape[0], t.shape[1]
    rowg = t.permute(0, 2, 1, 3).reshape(nr * BLOCK, ng, ROW6).to(torch.int64)
    halves = torch.stack([torch.cat([rowg[..., 0:16], rowg[..., 32:40]], -1),
                          torch.cat([rowg[..., 16:32], rowg[..., 40:48]], -1)], 2)  # [R, G, 2, 24]
    b = halves.reshape(nr * BLOCK, ng, 2, 8, 3)
    v = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16)
    c = torch.stack([(v >> (6 * i)) & 63 for i in range(4)], -1)
    return c.reshape(nr * BLOCK, ng * 64)


def encode_weights(w: torch.Tensor) -> torch.Tensor:
    """Integer weights [N, K] in [-8, 7] -> the GEMM's weight operand (tile-blocked fp6 codes)."""
    if int(w.min()) < -8 or int(w.max()) > 7:
        raise ValueError("int4 weights must lie in [-8, 7]")
    return _pack6(_W_ENC.to(w.device)[(w.to(torch.int64) + 8)])


def decode_weights(t: torch.Tensor) -> torch.Tensor:
    """The inverse of encode_weights: [N/128, K/64, 128, 48] -> int32 [N, K]."""
    return _W_DEC.to(t.device)[_unpack6(t)]


def encode_acts(q: torch.Tensor) -> torch.Tensor:
    """Integer activations [Mp, K] in [-8, 15] -> the GEMM's activation operand (tile-blocked fp6 codes)."""
    if int(q.min()) < -8 or int(q.max()) > 15:
        raise ValueError("int4 activations must lie in [-8, 15]")
    return _pack6(_A_ENC.to(q.device)[(q.to(torch.int64) + 8)])


def decode_acts(t: torch.Tensor) -> torch.Tensor:
    """The inverse of encode_acts: [Mp/128, K/64, 128, 48] -> int32 [Mp, K]."""
    return _A_DEC.to(t.device)[_unpack6(t)]


def weight_codes(qweight: torch.Tensor) -> torch.Tensor:
    """Packed int4 weights uint8 [N, K/2] -> the GEMM's weight operand, tile-blocked fp6 codes of the same integers,
    uint8 [N/128, K/64, 128, 48] (on the GPU)."""
    N, half = qweight.shape
    if N % BLOCK:
        raise ValueError(f"W4A4 weights need out_features % {BLOCK} == 0, got {N}")
    codes = torch.empty(N // BLOCK, 2 * half // 64, BLOCK, ROW6, device=qweight.device, dtype=torch.uint8)
    _lib.call("wdl_w4a4_weight_codes", ptr(qweight.contiguous()), N, 2 * half, ptr(codes), stream_of(qweight))
    return codes


def scale_pairs(wscales: torch.Tensor) -> torch.Tensor:
    """Weight scales bf16 or fp16 [K/64, N] -> the GEMM's scale operand, int32 [K/64, N] bf16 pairs hi | lo << 16
    with hi + lo = the scale exactly (on the GPU). Pairs pass through."""
    if wscales.dtype == torch.int32:
        return wscales
    if wscales.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"weight scales must be bf16 or fp16, got {wscales.dtype}")
    src = wscales.contiguous()
    pairs = torch.empty(src.shape, device=src.device, dtype=torch.int32)
    _lib.call("wdl_w4a4_scale_pairs", ptr(src), int(src.dtype == torch.float16), src.numel(), ptr(pairs),
              stream_of(src))
    return pairs


# scale pairs made for bf16 / fp16 weight-scale tensors passed to the bare ops, per tensor object and version:
# the reference-schema ops (w4a4_linear, w4a4_gelu_mlp) take the module's scales on every call, and converting them
# each time would cost an allocation and a launch per call
_PAIRS: dict[int, tuple] = {}


def cached_scale_pairs(wscales: torch.Tensor) -> torch.Tensor:
    """scale_pairs(wscales), made once per tensor (and again after an in-place change of it)."""
    if wscales.dtype == torch.int32:
        return wscales
    key = id(wscales)
    hit = _PAIRS.get(key)
    if hit is not None and hit[0]() is wscales and hit[1] == wscales._version:
        return hit[2]
    pairs = scale_pairs(wscales)
    _PAIRS[key] = (weakref.ref(wscales, lambda _, k=key: _PAIRS.pop(k, None)), wscales._version, pairs)
    return pairs


def as_codes(qweight: torch.Tensor, K: int) -> torch.Tensor:
    """The weight operand for input width K: tile-blocked fp6 codes [N/128, K/64, 128, 48] pass through, packed
    [N, K/2] nibbles are expanded (once per call)."""
    if qweight.dtype not in (torch.uint8, torch.int8) or qweight.dim() not in (2, 4):
        raise TypeError(f"qweight must be a uint8 tensor of 2 or 4 dims, got {qweight.dtype} {tuple(qweight.shape)}")
    if qweight.dim() == 4:
        if tuple(qweight.shape[1:]) != (K // 64, BLOCK, ROW6) or K % 64:
            raise ValueError(f"blocked weight codes {tuple(qweight.shape)} do not match input width {K}")
        return qweight.view(torch.uint8)
    if 2 * qweight.shape[1] == K:
        return weight_codes(qweight.view(torch.uint8))
    raise ValueError(f"qweight {tuple(qweight.shape)} fits neither blocked codes nor [N, {K // 2}] nibbles")


def gemm_launch(q, ascales, lora, wcodes, wscales, proj_up, bias, M, out, epilogue=EPI_BF16, gate=None,
                stream_k=True, ln_out=None):
    """W4A4 GEMM on the quantizer's outputs (q, ascales, lora) and tile-blocked fp6 weight codes (weight_codes);
    wscales: the scale pairs (scale_pairs), or bf16 / fp16 scales (converted once per tensor, cached_scale_pairs).
    stream_k=False runs the one-pass launch also for the shapes that the library splits in K. ln_out (with the
    gated residual): fp32 [M, N / 32, 2] receiving the LayerNorm chunk partials of the updated rows of out."""
    wscales = cached_scale_pairs(wscales)
    if q.dim() != 4 or wcodes.dim() != 4 or q.shape[2:] != (BLOCK, ROW6) or wcodes.shape[2:] != (BLOCK, ROW6):
        raise ValueError("the W4A4 GEMM takes tile-blocked fp6 operands [rows/128, K/64, 128, 48]")
    Mp, K = q.shape[0] * BLOCK, q.shape[1] * 64
    N = wcodes.shape[0] * BLOCK
    if wcodes.shape[1] != q.shape[1]:
        raise ValueError(f"weight codes {tuple(wcodes.shape)} do not match activations of width {K}")
    nbytes = _lib.library().wdl_w4a4_gemm_workspace_bytes(Mp, N, K) if stream_k else 0
    ws = workspace(_GEMM_WS, q.device, nbytes) if nbytes else None
    if ln_out is not None and (ln_out.dtype != torch.float32 or not ln_out.is_contiguous() or
                               ln_out.numel() < M * (N // 32) * 2 or out.shape[-1] != N):
        raise ValueError(f"ln_out: a contiguous fp32 [{M}, {N // 32}, 2] buffer for whole output rows of {N}")
    _lib.call("wdl_w4a4_gemm", ptr(q), ptr(ascales), ptr(wcodes), ptr(wscales), ptr(lora), ptr(proj_up), ptr(bias),
              M, Mp, N, K, RANK, ptr(out), out.stride(0), epilogue, ptr(gate), ptr(ln_out), ptr(ws), stream_of(q))
    return out


def gelu_quant_launch(q, ascales, lora, wcodes, wscales, proj_up, bias, M, smooth2, proj_down2_t):
    """The fused GELU MLP's first GEMM: the quantizer's outputs of x (q, ascales, lora) and the first layer's
    operands -> the second layer's inputs (q2 fp6 codes [Mp/128, N/64, 128, 48], ascales2 bf16 [N/64, Mp], lora2
    fp32 [Mp, 32]) for h = GELU(x W1^T + b1) quantized as (h + 0.171875) / smooth2, unsigned; h stays in
    registers. wscales: the scale pairs (scale_pairs), or bf16 / fp16 scales (cached_scale_pairs)."""
    wscales = cached_scale_pairs(wscales)
    if q.dim() != 4 or wcodes.dim() != 4 or q.shape[2:] != (BLOCK, ROW6) or wcodes.shape[2:] != (BLOCK, ROW6):
        raise ValueError("the W4A4 GEMM takes tile-blocked fp6 operands [rows/128, K/64, 128, 48]")
    Mp, K = q.shape[0] * BLOCK, q.shape[1] * 64
    N = wcodes.shape[0] * BLOCK
    if wcodes.shape[1] != q.shape[1]:
        raise ValueError(f"weight codes {tuple(wcodes.shape)} do not match activations of width {K}")
    if smooth2.shape != (N,) or proj_down2_t.shape != (RANK, N):
        raise ValueError(f"smooth2 must be [{N}] and proj_down2 [{RANK}, {N}] for a hidden layer of {N}")
    dev = q.device
    q2 = torch.empty(Mp // BLOCK, N // 64, BLOCK, ROW6, device=dev, dtype=torch.uint8)
    asc2 = torch.empty(N // 64, Mp, device=dev, dtype=torch.bfloat16)
    lora2 = torch.empty(Mp, RANK, device=dev, dtype=torch.float32)
    ws = torch.empty(_lib.library().wdl_w4a4_gemm_gelu_quant_workspace_floats(Mp, N), device=dev,
                     dtype=torch.float32)
    _lib.call("wdl_w4a4_gemm_gelu_quant", ptr(q), ptr(ascales), ptr(wcodes), ptr(wscales), ptr(lora), ptr(proj_up),
              ptr(bias), M, Mp, N, K, RANK, ptr(smooth2), ptr(proj_down2_t), ptr(q2), ptr(asc2), ptr(lora2), ptr(ws),
              stream_of(q))
    return q2, asc2, lora2


@torch.library.custom_op("wdl::act_quant_w4", mutates_args=())
def act_quant_w4(x: torch.Tensor, smooth: torch.Tensor, proj_down: torch.Tensor, qshift: float,
                 unsigned: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return act_quant_launch(x, smooth, proj_down, qshift, unsigned)


@act_quant_w4.register_fake
def _(x, smooth, proj_down, qshift, unsigned):
    M, K = x.shape
    Mp = padded_rows(M)
    return (x.new_empty(Mp // BLOCK, K // 64, BLOCK, ROW6, dtype=torch.uint8),
            x.new_empty(K // 64, Mp, dtype=torch.bfloat16), x.new_empty(Mp, RANK, dtype=torch.float32))


def out_features(qweight: torch.Tensor) -> int:
    """N of a weight operand: packed [N, K/2] nibbles or tile-blocked [N/128, K/64, 128, 48] codes."""
    return qweight.shape[0] * (BLOCK if qweight.dim() == 4 else 1)


@torch.library.custom_op("wdl::w4a4_gemm", mutates_args=())
def w4a4_gemm(q: torch.Tensor, ascales: torch.Tensor, lora: torch.Tensor, qweight: torch.Tensor,
              wscales: torch.Tensor, proj_up: torch.Tensor, bias: torch.Tensor, M: int, fp32_out: bool) -> torch.Tensor:
    out = torch.empty(M, out_features(qweight), device=q.device, dtype=torch.float32 if fp32_out else torch.bfloat16)
    return gemm_launch(q, ascales, lora, as_codes(qweight, q.shape[1] * 64), wscales, proj_up, bias, M, out,
                       EPI_F32 if fp32_out else EPI_BF16)


@w4a4_gemm.register_fake
def _(q, ascales, lora, qweight, wscales, proj_up, bias, M, fp32_out):
    return q.new_empty(M, out_features(qweight), dtype=torch.float32 if fp32_out else torch.bfloat16)


@torch.library.custom_op("wdl::w4a4_linear", mutates_args=())
def w4a4_linear(x: torch.Tensor, qweight: torch.Tensor, wscales: torch.Tensor, proj_down: torch.Tensor,
                proj_up: torch.Tensor, smooth: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """live::w4a4_linear (native/ops/w4a4_ops.cpp:31-40): activation quantizer + low-rank down projection, then
    the W4A4 GEMM with the low-rank up projection and the bias; x bf16 [M, K] -> bf16 [M, N]."""
    q, asc, lora = act_quant_launch(x, smooth, proj_down)
    out = torch.empty(x.shape[0], out_features(qweight), device=x.device, dtype=torch.bfloat16)
    return gemm_launch(q, asc, lora, as_codes(qweight, x.shape[1]), wscales, proj_up, bias, x.shape[0], out)


@w4a4_linear.register_fake
def _(x, qweight, wscales, proj_down, proj_up, smooth, bias):
    return x.new_empty(x.shape[0], out_features(qweight), dtype=torch.bfloat16)


GELU_SHIFT = 0.171875


@torch.library.custom_op("wdl::w4a4_gelu_mlp", mutates_args=())
def w4a4_gelu_mlp(x: torch.Tensor, qweight1: torch.Tensor, wscales1: torch.Tensor, proj_down1: torch.Tensor,
                  proj_up1: torch.Tensor, smooth1: torch.Tensor, bias1: torch.Tensor, qweight2: torch.Tensor,
                  wscales2: torch.Tensor, proj_down2: torch.Tensor, proj_up2: torch.Tensor, smooth2: torch.Tensor,
                  bias2: torch.Tensor) -> torch.Tensor:
    """live::w4a4_gelu_mlp (native/ops/w4a4_ops.cpp:44-63): the first GEMM applies GELU, quantizes
    (h + 0.171875) / smooth2 unsigned and forms the low-rank down projection of h in its epilogue (h in fp32, never
    in memory), then the second GEMM."""
    M = x.shape[0]
    q, asc, lora = act_quant_launch(x, smooth1, proj_down1)
    hidden = out_features(qweight1)
    q2, asc2, lora2 = gelu_quant_launch(q, asc, lora, as_codes(qweight1, x.shape[1]), wscales1, proj_up1, bias1, M,
                                        smooth2, proj_down2)
    out = torch.empty(M, out_features(qweight2), device=x.device, dtype=torch.bfloat16)
    return gemm_launch(q2, asc2, lora2, as_codes(qweight2, hidden), wscales2, proj_up2, bias2, M, out)


@w4a4_gelu_mlp.register_fake
def _(x, qweight1, wscales1, proj_down1, proj_up1, smooth1, bias1, qweight2, wscales2, proj_down2, proj_up2,
      smooth2, bias2):
    return x.new_empty(x.shape[0], out_features(qweight2), dtype=torch.bfloat16)


# ------------------------------------------------------------------------------------------------ Q/K norm + RoPE

def qk_norm_rope_launch(q, k, wq, wk, freq, grid, start_frame, eps=1e-6, q_out=None, k_out=None):
    """q, k bf16 [M, H*128] (row-strided views allowed) -> RMSNorm(all heads) + 3D RoPE, bf16 [M, H*128] each.
    wq / wk None: that input is only rotated; k None: q alone (returns (q_out, None)). freq: contiguous fp32 or
    fp64 [2, positions, 64]."""
    M, C = q.shape
    f, h, w = (int(v) for v in grid)
    q_out = torch.empty(M, C, device=q.device, dtype=torch.bfloat16) if q_out is None else q_out
    if k is not None and k_out is None:
        k_out = torch.empty(M, C, device=q.device, dtype=torch.bfloat16)
    code = {torch.float32: 0, torch.float64: 3}[freq.dtype]
    _lib.call("wdl_qk_norm_rope", ptr(q), q.stride(0), ptr(k), 0 if k is None else k.stride(0), ptr(wq), ptr(wk),
              ptr(freq), code, freq.shape[1], M, C // 128, f, h, w, int(start_frame), float(eps), ptr(q_out),
              ptr(k_out), q_out.stride(0), stream_of(q))
    return q_out, k_out


def quant_q_launch(x, heads):
    """x bf16 [n, heads*128] (row stride allowed) -> q int8 [n, heads, 128], q_scale fp32 [heads, blocks*8]."""
    n = x.shape[0]
    blocks8 = (n + 127) // 128 * 32
    q = torch.empty(n, heads, 128, device=x.device, dtype=torch.int8)
    qs = torch.empty(heads, blocks8, device=x.device, dtype=torch.float32)
    _lib.call("wdl_quant_q", ptr(x), x.stride(0), n, heads, ptr(q), ptr(qs), stream_of(x))
    return q, qs


# token splits of the Sage preparation's column statistics per head (workgroups of colstats_kernel, partials summed in
# order by finalize_kernel): 16 measured 0.02 ms per step faster than 8 or 32 and 0.14 ms faster than 64
SPLITS = 16


def sage_cache_stats_launch(cache_k, cache_ks, cache_v, cache_vs, at, out=None):
    """The statistics of cache rows [0, at) (fp8 as uint8 [1, cap, H, 128] + fp32 scales [1, cap, H, 1]) that
    sage_prep_launch(cache_stats=...) starts from: fp32 [2, H, 128], the K column sums and the |V| column maxima
    (written into `out` when given)."""
    H = cache_k.shape[2]
    dev = cache_k.device
    if not isinstance(at, int) or at < 0 or at > cache_k.shape[1]:
        raise ValueError("at outside the cache")
    if out is None:
        out = torch.empty(2, H, 128, device=dev, dtype=torch.float32)
    elif out.shape != (2, H, 128) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError(f"cache statistics must be contiguous fp32 [2, {H}, 128]")
    ws = torch.empty(_lib.library().wdl_sage_prep_workspace_floats(H, SPLITS), device=dev, dtype=torch.float32)
    _lib.call("wdl_sage_cache_stats", ptr(cache_k), ptr(cache_ks), ptr(cache_v), ptr(cache_vs), cache_k.shape[1], H,
              at, SPLITS, ptr(ws), ptr(out), stream_of(cache_k))
    return out


def sage_prep_launch(cache_k, cache_ks, cache_v, cache_vs, k, v, at, want_stats=False, heads=None, tokens=None,
                     cache_stats=None, append=False):
    """Cache (fp8 [1, cap, Hc, 128] + fp32 scales [1, cap, Hc, 1]) tokens [0, at) and the chunk k, v
    (bf16 [n, H*128] row-strided) -> k_int8 [H, Lpad, 128], k_scale [H, Lpad/16], v_fp8 [H, 128, Lpad],
    v_scale [H, 128] (and k_mean when want_stats). heads (int32 [H], device): head h reads cache head heads[h];
    tokens (int32 [>= at], device): cached token i is cache row tokens[i]; without them Hc = H and rows 0 .. at-1.
    cache_stats: sage_cache_stats_launch of the same cache rows [0, at) (no maps): only the chunk's tokens are then
    read for the K mean and V scale. append (with cache_stats): the pass also writes k, v into cache rows at .. at + n
    (wdl_sage_prep_cached_append: the bytes and scales of wdl_kv_append_fp8)."""
    n = k.shape[0]
    H = k.shape[1] // 128
    Hc = cache_k.shape[2]
    L = at + n
    Lp = (L + 63) // 64 * 64
    dev = k.device
    ws = torch.empty(_lib.library().wdl_sage_prep_workspace_floats(H, SPLITS), device=dev, dtype=torch.float32)
    k_i8 = torch.empty(H, Lp, 128, device=dev, dtype=torch.int8)
    k_sc = torch.empty(H, Lp // 16, device=dev, dtype=torch.float32)
    v_f8 = torch.empty(H, 128, Lp, device=dev, dtype=torch.uint8)
    k_mean = torch.empty(H, 128, device=dev, dtype=torch.float32)
    v_sc = torch.empty(H, 128, device=dev, dtype=torch.float32)
    if cache_stats is not None:
        if heads is not None or tokens is not None:
            raise ValueError("cache statistics are for the unmapped cache")
        if cache_stats.shape != (2, H, 128) or cache_stats.dtype != torch.float32 or not cache_stats.is_contiguous():
            raise ValueError(f"cache statistics must be contiguous fp32 [2, {H}, 128]")
        _lib.call("wdl_sage_prep_cached_append" if append else "wdl_sage_prep_cached", ptr(cache_k), ptr(cache_ks),
                  ptr(cache_v), ptr(cache_vs), cache_k.shape[1], ptr(k), k.stride(0), ptr(v), v.stride(0), H, at, n,
                  ptr(cache_stats), SPLITS, ptr(ws), ptr(k_i8), ptr(k_sc), ptr(v_f8), ptr(k_mean), ptr(v_sc),
                  stream_of(k))
    elif append:
        raise ValueError("append runs with the cache statistics")
    elif heads is None and tokens is None:
        _lib.call("wdl_sage_prep", ptr(cache_k), ptr(cache_ks), ptr(cache_v), ptr(cache_vs), cache_k.shape[1],
                  ptr(k), k.stride(0), ptr(v), v.stride(0), H, at, n, SPLITS, ptr(ws), ptr(k_i8), ptr(k_sc),
                  ptr(v_f8), ptr(k_mean), ptr(v_sc), stream_of(k))
    else:
        _lib.call("wdl_sage_prep_mapped", ptr(cache_k), ptr(cache_ks), ptr(cache_v), ptr(cache_vs),
                  cache_k.shape[1], Hc, ptr(heads), ptr(tokens), ptr(k), k.stride(0), ptr(v), v.stride(0), H, at, n,
                  SPLITS, ptr(ws), ptr(k_i8), ptr(k_sc), ptr(v_f8), ptr(k_mean), ptr(v_sc), stream_of(k))
    out = dict(k=k_i8, k_scale=k_sc, v=v_f8, v_scale=v_sc)
    if want_stats:
        out["k_mean"] = k_mean
    return out


_ATTN_WS: dict = {}
_GEMM_WS: dict = {}
# Buffers a larger request replaced. A HIP graph captured while one of them was current keeps its address in its
# kernel arguments, so none is ever freed: a replay after the growth still writes memory that is its own.
_RETIRED: list = []


def workspace(cache: dict, device: torch.device, nbytes: int) -> torch.Tensor | None:
    """A device's scratch buffer for one kind of call (partial results of split tiles); no initial contents are
    needed. One per device and kind: such calls on one device must not overlap (each launches on the current stream
    of its tensors). A request larger than the buffer replaces it (the old one is kept alive, see _RETIRED); during
    stream capture that raises instead, since the captured graph would hold an allocation made inside the capture:
    size the buffer first with reserve()."""
    if nbytes <= 0:
        return None
    key = device.index if device.index is not None else torch.cuda.current_device()
    ws = cache.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"workspace of {nbytes} bytes requested during graph capture (have "
                               f"{0 if ws is None else ws.numel()}): call wdl.ops.reserve() for the largest shape "
                               f"before capturing")
        if ws is not None:
            _RETIRED.append(ws)
        ws = torch.empty(max(nbytes, 1 << 20), device=device, dtype=torch.uint8)
        cache[key] = ws
    return ws


def reserve(device: torch.device, *, gemm: tuple | None = None, attn: tuple | None = None) -> None:
    """Sizes the scratch buffers up front for the largest shapes a caller will run (and capture): gemm = (Mp, N, K)
    of the largest W4A4 product, attn = (n, L, heads) of the largest attention."""
    lib = _lib.library()
    if gemm is not None:
        workspace(_GEMM_WS, device, lib.wdl_w4a4_gemm_workspace_bytes(*(int(v) for v in gemm)))
    if attn is not None:
        workspace(_ATTN_WS, device, lib.wdl_sage_attn_workspace_bytes(*(int(v) for v in attn)))


def sage_attn_launch(q_i8, q_scale, prep, L, sm_scale, out=None):
    """q_i8 [n, H, 128] -> bf16 [n, H*128] (or into `out`, a row-strided [n, H*128] view)."""
    n, H, _ = q_i8.shape
    if out is None:
        out = torch.empty(n, H * 128, device=q_i8.device, dtype=torch.bfloat16)
    ws = workspace(_ATTN_WS, q_i8.device, _lib.library().wdl_sage_attn_workspace_bytes(n, L, H))
    _lib.call("wdl_sage_attn", ptr(q_i8), H * 128, ptr(q_scale), ptr(prep["k"]), ptr(prep["k_scale"]),
              ptr(prep["v"]), ptr(prep["v_scale"]), n, L, H, float(sm_scale), ptr(out), out.stride(0), ptr(ws),
              stream_of(q_i8))
    return out


def sage_attn_q16_launch(Q, prep, L, sm_scale, out=None, frame_tokens=0):
    """Q bf16 [n, H*128] (row-strided) -> bf16 [n, H*128]: Sage attention with the int8 quantization of Q done in
    the kernel (bit-identical to quant_q_launch followed by sage_attn_launch). frame_tokens > 0: block-causal per
    latent frame, the n queries being the last n of the L keys (query q sees keys below L - n + (q // frame_tokens
    + 1) * frame_tokens)."""
    n = Q.shape[0]
    H = Q.shape[1] // 128
    if Q.dtype != torch.bfloat16 or Q.dim() != 2 or Q.shape[1] % 128 or Q.stride(1) != 1:
        raise ValueError("sage_attn_q16: Q must be bf16 [n, H*128] with unit column stride")
    if out is None:
        out = torch.empty(n, H * 128, device=Q.device, dtype=torch.bfloat16)
    if frame_tokens:
        if not isinstance(frame_tokens, int) or frame_tokens < 0 or n > L:
            raise ValueError("sage_attn_q16: frame_tokens must be a positive int and the queries among the keys")
        _lib.call("wdl_sage_attn_q16_framed", ptr(Q), Q.stride(0), ptr(prep["k"]), ptr(prep["k_scale"]),
                  ptr(prep["v"]), ptr(prep["v_scale"]), n, L, H, float(sm_scale), frame_tokens, ptr(out),
                  out.stride(0), 0, stream_of(Q))
        return out
    ws = workspace(_ATTN_WS, Q.device, _lib.library().wdl_sage_attn_workspace_bytes(n, L, H))
    _lib.call("wdl_sage_attn_q16", ptr(Q), Q.stride(0), ptr(prep["k"]), ptr(prep["k_scale"]), ptr(prep["v"]),
              ptr(prep["v_scale"]), n, L, H, float(sm_scale), ptr(out), out.stride(0), ptr(ws), stream_of(Q))
    return out


def attn_bf16_prep_launch(K, V):
    """The keys and values of a bf16 attention (the prompt's, for the cross-attention) in wdl_attn_bf16's layouts:
    K, V bf16 [L, H*128] (row-strided views allowed) -> dict(kp, vp, L, heads)."""
    L, C = K.shape
    if K.dtype != torch.bfloat16 or V.dtype != torch.bfloat16 or V.shape != K.shape or C % 128 or \
            K.stride(1) != 1 or V.stride(1) != 1:
        raise ValueError("attn_bf16_prep: K, V must be bf16 [L, heads*128] with unit column stride")
    H = C // 128
    n = _lib.library().wdl_attn_bf16_prep_elems(L, H)
    kp = torch.empty(n, device=K.device, dtype=torch.bfloat16)
    vp = torch.empty(n, device=K.device, dtype=torch.bfloat16)
    _lib.call("wdl_attn_bf16_prep", ptr(K), K.stride(0), ptr(V), V.stride(0), L, H, ptr(kp), ptr(vp), stream_of(K))
    return dict(kp=kp, vp=vp, L=L, heads=H)


def _attn_bf16_into(Q, kp, vp, L, H, sm_scale, out):
    _lib.call("wdl_attn_bf16", ptr(Q), Q.stride(0), ptr(kp), ptr(vp), Q.shape[0], L, H, float(sm_scale), ptr(out),
              out.stride(0), stream_of(Q))
    return out


@torch.library.custom_op("wdl::attn_bf16", mutates_args=())
def attn_bf16(q: torch.Tensor, kp: torch.Tensor, vp: torch.Tensor, keys: int, sm_scale: float) -> torch.Tensor:
    """softmax(q K^T sm_scale) V in bf16 with an fp32 softmax (the reference's SDPA on bf16 operands) for q bf16
    [n, H*128] over the `keys` keys laid out by attn_bf16_prep_launch (kp, vp) -> bf16 [n, H*128]."""
    out = torch.empty(q.shape, device=q.device, dtype=torch.bfloat16)
    return _attn_bf16_into(q, kp, vp, keys, q.shape[1] // 128, sm_scale, out)


@attn_bf16.register_fake
def _(q, kp, vp, keys, sm_scale):
    return q.new_empty(q.shape, dtype=torch.bfloat16)


def attn_bf16_launch(Q, prep, sm_scale, out=None):
    """Q bf16 [n, H*128] (row-strided) -> bf16 [n, H*128]: exact-softmax bf16 attention over prep's keys (into
    `out` when given: a row-strided [n, H*128] view)."""
    n, C = Q.shape
    H = prep["heads"]
    if Q.dtype != torch.bfloat16 or C != H * 128 or Q.stride(1) != 1:
        raise ValueError(f"attn_bf16: Q must be bf16 [n, {H * 128}] with unit column stride")
    if out is None:
        return attn_bf16(Q, prep["kp"], prep["vp"], prep["L"], float(sm_scale))
    return _attn_bf16_into(Q, prep["kp"], prep["vp"], prep["L"], H, sm_scale, out)


@torch.library.custom_op("wdl::sage_kv_attend", mutates_args=())
def sage_kv_attend(Q: torch.Tensor, cache_k: torch.Tensor, cache_ks: torch.Tensor, cache_v: torch.Tensor,
                   cache_vs: torch.Tensor, K: torch.Tensor, V: torch.Tensor, at: int, sm_scale: float,
                   heads: torch.Tensor | None = None, tokens: torch.Tensor | None = None) -> torch.Tensor:
    """wan_dit_lab::sage_kv_attend (src/wan_dit_lab/kernels/sage_kv.py:137-176): Q [1, nq, H, 128], K, V
    [1, n, H, 128] bf16 (row-strided token dim allowed), cache fp8 (as uint8) [1, cap, Hc, 128] with fp32 scales
    [1, cap, Hc, 1] -> [1, nq, H, 128] bf16. heads (int32 [H]): head h is cache head heads[h]; tokens (int32 [at]):
    cached token i is cache row tokens[i] (neither copies the cache)."""
    _, nq, H, D = Q.shape
    n = K.shape[1]
    prep = sage_prep_launch(cache_k, cache_ks, cache_v, cache_vs, K[0].reshape(n, H * D) if K.is_contiguous() else
                            K[0].flatten(1), V[0].flatten(1), at, heads=heads, tokens=tokens)
    return sage_attn_q16_launch(Q[0].flatten(1), prep, at + n, sm_scale).view(1, nq, H, D)


@sage_kv_attend.register_fake
def _(Q, cache_k, cache_ks, cache_v, cache_vs, K, V, at, sm_scale, heads=None, tokens=None):
    return Q.new_empty(Q.shape, dtype=torch.bfloat16)


@torch.library.custom_op("wdl::sage_kv_attend_cached", mutates_args=())
def sage_kv_attend_cached(Q: torch.Tensor, cache_k: torch.Tensor, cache_ks: torch.Tensor, cache_v: torch.Tensor,
                          cache_vs: torch.Tensor, K: torch.Tensor, V: torch.Tensor, at: int, sm_scale: float,
                          cache_stats: torch.Tensor) -> torch.Tensor:
    """sage_kv_attend over an unmapped cache whose rows [0, at) have the statistics cache_stats
    (sage_cache_stats_launch): the preparation reads only the chunk's tokens for the K mean and V scale."""
    _, nq, H, D = Q.shape
    n = K.shape[1]
    prep = sage_prep_launch(cache_k, cache_ks, cache_v, cache_vs, K[0].reshape(n, H * D) if K.is_contiguous() else
                            K[0].flatten(1), V[0].flatten(1), at, cache_stats=cache_stats)
    return sage_attn_q16_launch(Q[0].flatten(1), prep, at + n, sm_scale).view(1, nq, H, D)


@sage_kv_attend_cached.register_fake
def _(Q, cache_k, cache_ks, cache_v, cache_vs, K, V, at, sm_scale, cache_stats):
    return Q.new_empty(Q.shape, dtype=torch.bfloat16)


@torch.library.custom_op("wdl::sage_kv_append_attend_cached", mutates_args=("cache_k", "cache_ks", "cache_v", "cache_vs"))
def sage_kv_append_attend_cached(Q: torch.Tensor, cache_k: torch.Tensor, cache_ks: torch.Tensor, cache_v: torch.Tensor,
                                 cache_vs: torch.Tensor, K: torch.Tensor, V: torch.Tensor, at: int, sm_scale: float,
                                 cache_stats: torch.Tensor) -> torch.Tensor:
    """The cache store of the chunk (KVCache.store, causal.py:177-181: store_kv_fp8 into rows at .. at + n) and
    sage_kv_attend_cached over the cache and the chunk, with the store inside the preparation's quantization pass
    (one read of the chunk, no launch of its own): the cache receives the bytes and scales store_kv_fp8 writes."""
    _, nq, H, D = Q.shape
    n = K.shape[1]
    prep = sage_prep_launch(cache_k, cache_ks, cache_v, cache_vs, K[0].reshape(n, H * D) if K.is_contiguous() else
                            K[0].flatten(1), V[0].flatten(1), at, cache_stats=cache_stats, append=True)
    return sage_attn_q16_launch(Q[0].flatten(1), prep, at + n, sm_scale).view(1, nq, H, D)


@sage_kv_append_attend_cached.register_fake
def _(Q, cache_k, cache_ks, cache_v, cache_vs, K, V, at, sm_scale, cache_stats):
    return Q.new_empty(Q.shape, dtype=torch.bfloat16)


@torch.library.custom_op("wdl::sage_attn", mutates_args=())
def sage_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_scale: torch.Tensor, k_scale: torch.Tensor,
              v_scale: torch.Tensor, sm_scale: float, keys: int) -> torch.Tensor:
    """The Sage kernel alone, the counterpart of live::sage_sm89(q, k, v, q_scale, k_scale, v_scale, sm_scale)
    (native/ops/sage_ops.cpp:12-19, 28-31) on wdl's operand layouts: q int8 [1, n, H, 128] with q_scale fp32
    [1, H, ceil(n/128)*32] (wdl.sage_kv.quant_q), k int8 [H, Lpad, 128] with k_scale [H, Lpad/16], v fp8 (as uint8)
    [H, 128, Lpad], v_scale [H, 128] (wdl.sage_kv.prep); `keys` = L, the unpadded key count (wdl's K and V are
    padded to 64-key blocks) -> [1, n, H, 128] bf16."""
    _, n, H, D = q.shape
    prep = dict(k=k, k_scale=k_scale, v=v, v_scale=v_scale)
    return sage_attn_launch(q[0], q_scale[0], prep, keys, sm_scale).view(1, n, H, D)


@sage_attn.register_fake
def _(q, k, v, q_scale, k_scale, v_scale, sm_scale, keys):
    return q.new_empty(q.shape, dtype=torch.bfloat16)


@torch.library.custom_op("wdl::sage_sm89", mutates_args=())
def sage_sm89(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_scale: torch.Tensor, k_scale: torch.Tensor,
              v_scale: torch.Tensor, sm_scale: float) -> torch.Tensor:
    """live::sage_sm89 (native/ops/sage_ops.cpp:12-19, 28-31): q int8 [1, n, H, 128], q_scale fp32 [1, H,
    ceil(n/128)*32], v_scale fp32 [1, H, 128] -> bf16 [1, n, H, 128]. k and v in either of two layouts:
    - the reference's, as kernels/sage_kv.py:141-176 builds them: k int8 [1, L, H, 128], k_scale [1, H,
      ceil(L/64)*4], v fp8 [1, 128, H, Lpad] in Sage's 16-token order (Lpad = 64 ceil(L/64)); the op copies k and
      v into wdl's layouts on the device (wdl_sage_sm89_relayout: one pass over them) and runs wdl's kernel;
    - wdl's own: k the [H, L, 128] view of the padded int8 keys (k_int8[:, :L]) with k_scale [H, Lpad/16], v the
      [H, 128, L] view of the fp8 values (v_fp8[:, :, :L]), as wdl.sage_kv.prep makes them."""
    _, n, H, D = q.shape
    if k.dim() == 4:
        _, L, Hk, Dk = k.shape
        Lpad = (L + 63) // 64 * 64
        if (k.shape[0] != 1 or Hk != H or Dk != D or D != 128 or k.dtype != torch.int8 or k.stride(3) != 1
                or k.stride(2) != D or v.shape != (1, D, H, Lpad) or v.stride(3) != 1 or v.element_size() != 1
                or k_scale.shape[-1] != Lpad // 16 or v_scale.shape[-2:] != (H, D)):
            raise ValueError(f"sage_sm89: k must be int8 [1, L, {H}, 128] and v fp8 [1, 128, {H}, 64 ceil(L / 64)] "
                             "(the layouts of kernels/sage_kv.py:160-170)")
        kw = torch.empty(H, Lpad, D, device=k.device, dtype=torch.int8)
        vw = torch.empty(H, D, Lpad, device=k.device, dtype=torch.uint8)
        _lib.call("wdl_sage_sm89_relayout", ptr(k), k.stride(1), ptr(v), v.stride(1), v.stride(2), L, H, ptr(kw),
                  ptr(vw), stream_of(k))
        prep = dict(k=kw, k_scale=k_scale.reshape(H, -1), v=vw, v_scale=v_scale.reshape(H, D))
        return sage_attn_launch(q[0], q_scale.reshape(H, -1), prep, L, sm_scale).view(1, n, H, D)
    H, L, D = k.shape
    Lpad = (L + 63) // 64 * 64  # the kernel's row pitch for L keys: the views must come from buffers of that pitch
    if k.stride(1) != D or k.stride(2) != 1 or k.stride(0) != Lpad * D or v.stride(2) != 1 or v.stride(1) != Lpad \
            or v.shape != (H, D, L):
        raise ValueError("sage_sm89: k must be a [H, L, 128] view of wdl's [H, Lpad, 128] keys and v the matching "
                         "[H, 128, L] view of the [H, 128, Lpad] values")
    prep = dict(k=k, k_scale=k_scale, v=v, v_scale=v_scale)
    return sage_attn_launch(q[0], q_scale[0], prep, L, sm_scale).view(1, n, H, D)


@sage_sm89.register_fake
def _(q, k, v, q_scale, k_scale, v_scale, sm_scale):
    return q.new_empty(q.shape, dtype=torch.bfloat16)
