"""The torch operators of the drop-in boundary (wdl::*, the reference's wan_dit_lab:: / live:: schemas) under the
reference's calling contracts: the head / token maps of sage_kv_attend read exactly what a cache holding only those
heads and rows gives (tests/test_sage_kv.py:118-131 states the same contract), the Sage kernel alone as an operator,
and every operator through torch.compile(fullgraph=True) and HIP-graph capture, bit-equal to its eager form, the
cache append as exactly one kernel (tests/test_cache_fp8.py:75-95)."""

import pytest
import torch

pytestmark = pytest.mark.gpu
FP8 = torch.float8_e4m3fn


def kernels_of(fn):
    """Names of the device kernels one call of fn launches."""
    from torch.profiler import ProfilerActivity, profile

    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    return [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]


def cache_case(H=4, cap=320, n=150, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    r = lambda *s: torch.randn(*s, device="cuda", generator=g)
    k = (r(1, cap, H, 128) * 40 + 20).clamp(-448, 448).to(FP8)
    v = (r(1, cap, H, 128) * 30).clamp(-448, 448).to(FP8)
    ks = torch.rand(1, cap, H, 1, device="cuda", generator=g) * 0.02 + 0.005
    vs = torch.rand(1, cap, H, 1, device="cuda", generator=g) * 0.02 + 0.005
    K = (r(1, n, H, 128) + 0.5).to(torch.bfloat16)
    V = r(1, n, H, 128).to(torch.bfloat16)
    Q = r(1, n, H, 128).to(torch.bfloat16)
    return Q, k, ks, v, vs, K, V


def test_head_and_token_maps_equal_the_same_call_on_a_gathered_cache(gpu):
    from oracle import sage as osage
    from wdl import sage_kv

    Q, k, ks, v, vs, K, V = cache_case()
    heads = torch.tensor([3, 0], device="cuda", dtype=torch.int32)
    tokens = torch.tensor(list(range(17, 60)) + list(range(200, 290)), device="cuda", dtype=torch.int32)
    at = tokens.numel()
    pick = lambda x: x[:, tokens.long()][:, :, heads.long()].contiguous()
    sub = lambda x: x[:, :, heads.long()].contiguous()
    expected = sage_kv.attend(sub(Q), pick(k), pick(ks), pick(v), pick(vs), at, sub(K), sub(V))
    out = sage_kv.attend(sub(Q), k, ks, v, vs, at, sub(K), sub(V), heads=heads, tokens=tokens)
    assert torch.equal(out, expected)
    # and against the oracle's mapped gather: the Sage bars of the attention tests
    p = osage.prep(sub(Q).cpu(), k.cpu(), ks.cpu(), v.cpu(), vs.cpu(), at, sub(K).cpu(), sub(V).cpu(),
                   heads=heads.cpu(), tokens=tokens.cpu())
    ref = osage.attention_quantized(p, 128 ** -0.5)
    assert osage.cosine(out.cpu(), ref) >= 0.999
    # maps that leave the cache are rejected before any launch
    with pytest.raises(ValueError):
        sage_kv.attend(sub(Q), k, ks, v, vs, at, sub(K), sub(V), heads=heads + 3, tokens=tokens)
    with pytest.raises(ValueError):
        sage_kv.attend(sub(Q), k, ks, v, vs, at, sub(K), sub(V), heads=heads, tokens=tokens.long())


def test_sage_attn_operator_is_the_kernel_of_sage_kv_attend(gpu):
    """wdl::sage_attn (live::sage_sm89's counterpart on wdl's layouts) over wdl.sage_kv.quant_q and prep gives the
    bits of sage_kv.attend, whose kernel quantizes Q itself."""
    from wdl import sage_kv

    Q, k, ks, v, vs, K, V = cache_case(H=2)
    at = 200
    q, qs = sage_kv.quant_q(Q)
    p = sage_kv.prep(k, ks, v, vs, at, K, V)
    out = torch.ops.wdl.sage_attn(q, p["k"], p["v"], qs, p["k_scale"], p["v_scale"], 128 ** -0.5, at + K.shape[1])
    assert torch.equal(out, sage_kv.attend(Q, k, ks, v, vs, at, K, V))
    # the reference's schema (live::sage_sm89): the key count from the views' shapes
    import wdl.live  # noqa: F401

    L = at + K.shape[1]
    sm = torch.ops.live.sage_sm89(q, p["k"][:, :L], p["v"][:, :, :L], qs, p["k_scale"], p["v_scale"], 128 ** -0.5)
    assert torch.equal(sm, out)


@pytest.mark.parametrize("at,n,H", [(200, 150, 2), (128, 37, 3), (0, 64, 1)])
def test_sage_sm89_takes_the_reference_operands(gpu, at, n, H):
    """live::sage_sm89 on the operands the reference's sage_kv._attend hands it (kernels/sage_kv.py:141-176): int8 K
    [1, L, H, 128], k_scale [1, H, 4 ceil(L/64)], fp8 V [1, 128, H, Lpad] in Sage's 16-token order, q int8 [1, n, H,
    128] with q_scale [1, H, 32 ceil(n/128)], v_scale [1, H, 128], built by the oracle's restatement of those
    quantizers and layouts (sage_v_layout). The device relayout gives exactly wdl's layouts of the same operands
    (k [H, Lpad, 128], wdl_v_layout), the result is bit-equal to wdl::sage_attn on them, meets the Sage bars
    (cosine >= 0.999 against the exact-P emulation, error against exact attention within 1.2x + 1e-3 of the fp8-P
    emulation), and is bit-equal to eager under torch.compile and HIP-graph capture. L = 350 and 165 end in a
    partial 64-key block."""
    import wdl.live  # noqa: F401
    from oracle import sage as osage
    from wdl import ops

    Q, k, ks, v, vs, K, V = cache_case(H=H, n=n, seed=at + n)
    Qc, Kc, Vc = Q.cpu(), K.cpu(), V.cpu()
    p = osage.prep(Qc, k.cpu(), ks.cpu(), v.cpu(), vs.cpu(), at, Kc, Vc)
    L = at + n
    Lpad = (L + 63) // 64 * 64
    ref_ops = [t.cuda() for t in (p["q"], p["k"], osage.sage_v_layout(p["v"]), p["q_scale"], p["k_scale"],
                                  p["v_scale"])]
    assert ref_ops[1].shape == (1, L, H, 128) and ref_ops[2].shape == (1, 128, H, Lpad)
    # the relayout alone: wdl's layouts of the same operands
    kw = torch.empty(H, Lpad, 128, device="cuda", dtype=torch.int8)
    vw = torch.empty(H, 128, Lpad, device="cuda", dtype=torch.uint8)
    from wdl import _lib
    _lib.call("wdl_sage_sm89_relayout", ref_ops[1].data_ptr(), ref_ops[1].stride(1), ref_ops[2].data_ptr(),
              ref_ops[2].stride(1), ref_ops[2].stride(2), L, H, kw.data_ptr(), vw.data_ptr(),
              torch.cuda.current_stream().cuda_stream)
    want_k = torch.zeros(H, Lpad, 128, dtype=torch.int8)
    want_k[:, :L] = p["k"][0].permute(1, 0, 2)
    assert torch.equal(kw.cpu(), want_k)
    assert torch.equal(vw.cpu(), osage.wdl_v_layout(p["v"])[0].view(torch.uint8))
    sm = 128 ** -0.5
    out = torch.ops.live.sage_sm89(*ref_ops, sm)
    direct = torch.ops.wdl.sage_attn(ref_ops[0], kw, vw, ref_ops[3], ref_ops[4][0], ref_ops[5][0], sm, L)
    assert torch.equal(out, direct)
    emul = osage.attention_quantized(p, sm)
    emul8 = osage.attention_quantized(p, sm, p_fp8=True)
    exact = osage.attention_exact(Qc, p["K"], p["V"], sm)
    cos, err = osage.cosine(out.cpu(), emul), osage.rel_err(out.cpu(), exact)
    print(f"sage_sm89 reference operands at={at} n={n} H={H}: cos {cos:.6f}, err {err:.4f} "
          f"(fp8-P emulation {osage.rel_err(emul8, exact):.4f})")
    assert cos >= 0.999 and err < 1.2 * osage.rel_err(emul8, exact) + 1e-3
    _compiled_and_captured(lambda: torch.ops.live.sage_sm89(*ref_ops, sm), _equal)
    with pytest.raises(ValueError):  # V not padded to whole 64-key blocks
        torch.ops.live.sage_sm89(ref_ops[0], ref_ops[1], ref_ops[2][..., :Lpad - 16].contiguous(), *ref_ops[3:], sm)


def _compiled_and_captured(fn, check):
    """fn() eager, compiled (fullgraph) and replayed from a captured graph: `check` compares each to the eager
    result."""
    eager = fn()
    torch.cuda.synchronize()
    compiled = torch.compile(fn, fullgraph=True, dynamic=False)
    check(compiled(), eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        compiled()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = compiled()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        check(out, eager)
    return compiled


def _equal(a, b):
    assert torch.equal(a, b)


def test_store_kv_fp8_compiles_captures_and_is_one_kernel(gpu):
    from wdl.cache_fp8 import store_kv_fp8

    g = torch.Generator(device="cuda").manual_seed(3)
    k = torch.randn(1, 7, 2, 128, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(1, 7, 2, 128, device="cuda", generator=g).to(torch.bfloat16)
    bufs = [torch.zeros(1, 12, 2, 128, device="cuda", dtype=FP8), torch.zeros(1, 12, 2, 1, device="cuda"),
            torch.zeros(1, 12, 2, 128, device="cuda", dtype=FP8), torch.zeros(1, 12, 2, 1, device="cuda")]

    def run():
        store_kv_fp8(k, v, *bufs, 4)
        return torch.cat([bufs[0].view(torch.uint8).flatten().float(), bufs[1].flatten()])

    compiled = _compiled_and_captured(run, _equal)
    names = kernels_of(lambda: compiled())
    assert sum("kv_append" in n for n in names) == 1
    assert not any("kv_append" not in n and "cat" not in n.lower() and "copy" not in n.lower() and
                   "elementwise" not in n.lower() for n in names), names


def test_sage_ops_compile_and_capture(gpu):
    from wdl import sage_kv

    Q, k, ks, v, vs, K, V = cache_case(H=2)
    heads = torch.tensor([1, 0], device="cuda", dtype=torch.int32)
    tokens = torch.arange(100, 300, device="cuda", dtype=torch.int32)

    def attend():
        return torch.ops.wdl.sage_kv_attend(Q, k.view(torch.uint8), ks, v.view(torch.uint8), vs, K, V, 200,
                                            128 ** -0.5, heads, tokens)

    _compiled_and_captured(attend, _equal)
    assert torch.equal(attend(), sage_kv.attend(Q, k, ks, v, vs, 200, K, V, heads=heads, tokens=tokens))
    q, qs = sage_kv.quant_q(Q)
    p = sage_kv.prep(k, ks, v, vs, 200, K, V)
    _compiled_and_captured(lambda: torch.ops.wdl.sage_attn(q, p["k"], p["v"], qs, p["k_scale"], p["v_scale"],
                                                           128 ** -0.5, 200 + K.shape[1]), _equal)


def test_cached_statistics_op_compiles_and_captures(gpu):
    """wdl::sage_kv_attend_cached (KVCache.attend's op: the cached rows' column statistics beside the chunk's) under
    torch.compile(fullgraph) and graph capture, bit-equal to its eager form and to sage_kv.attend with the same
    statistics, and within the Sage bar of the whole-window preparation."""
    from oracle import sage as osage
    from wdl import sage_kv

    Q, k, ks, v, vs, K, V = cache_case(H=2)
    stats = sage_kv.cache_stats(k, ks, v, vs, 200)

    def attend():
        return torch.ops.wdl.sage_kv_attend_cached(Q, k.view(torch.uint8), ks, v.view(torch.uint8), vs, K, V, 200,
                                                   128 ** -0.5, stats)

    _compiled_and_captured(attend, _equal)
    out = attend()
    assert torch.equal(out, sage_kv.attend(Q, k, ks, v, vs, 200, K, V, cache_stats=stats))
    whole = sage_kv.attend(Q, k, ks, v, vs, 200, K, V)
    assert osage.cosine(out.cpu().float(), whole.cpu().float()) >= 0.9999


def test_w4a4_ops_compile_and_capture(gpu):
    from wdl import w4a4

    g = torch.Generator(device="cuda").manual_seed(7)
    t1 = w4a4.random_parts(512, 256, "cuda", g)
    t2 = w4a4.random_parts(256, 512, "cuda", g)
    x = torch.randn(300, 256, device="cuda", generator=g).to(torch.bfloat16)
    _compiled_and_captured(lambda: torch.ops.wdl.w4a4_linear(x, *(t1[p] for p in w4a4.PARTS)), _equal)
    _compiled_and_captured(lambda: torch.ops.wdl.w4a4_gelu_mlp(x, *(t1[p] for p in w4a4.PARTS),
                                                               *(t2[p] for p in w4a4.PARTS)), _equal)


def test_bf16_cross_attention_compiles_and_captures(gpu):
    from wdl import ops

    g = torch.Generator(device="cuda").manual_seed(8)
    K, V = (torch.randn(77, 256, device="cuda", generator=g).to(torch.bfloat16) for _ in range(2))
    Q = torch.randn(200, 256, device="cuda", generator=g).to(torch.bfloat16)
    prep = ops.attn_bf16_prep_launch(K, V)
    _compiled_and_captured(lambda: ops.attn_bf16_launch(Q, prep, 128 ** -0.5), _equal)
