"""wdl_act_quant_w4_static (the quantizer with its scratch in a static device array, no workspace argument) against
wdl_act_quant_w4 with a torch-allocated workspace, through the C ABI: bit-identical codes, scales and low-rank sums
on two calls in a row, the second smaller (the array keeps the first call's contents), with LayerNorm + modulation
and without, at K = 3072 (one column block per 4 groups) and K = 14336 (the wide shape, low-rank partials summed
by a second kernel). A shape above the static maximum is refused before any launch."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _call(static, x, smooth, pdt, M, Mp, unsigned, ln):
    from wdl import _lib, ops

    K = x.shape[1]
    dev = x.device
    q = torch.full((Mp // 128, K // 64, 128, 48), 0xAB, device=dev, dtype=torch.uint8)
    asc = torch.full((K // 64, Mp), 0x7F7F, device=dev, dtype=torch.int16).view(torch.bfloat16)
    lora = torch.full((Mp, 32), float("nan"), device=dev)
    ln = ln or {}
    common = [x.data_ptr(), x.stride(0), M, K, smooth.data_ptr(), ctypes.c_float(0.171875 if unsigned else 0.0),
              int(unsigned), pdt.data_ptr(), 32, q.data_ptr(), asc.data_ptr(), lora.data_ptr(), Mp,
              ops.ptr(ln.get("shift")), ops.ptr(ln.get("scale")), ops.ptr(ln.get("weight")), ops.ptr(ln.get("bias")),
              int(bool(ln)), ctypes.c_float(1e-6), None, None]  # eps, no LN partials (formed here), no v_out
    stream = torch.cuda.current_stream().cuda_stream
    if static:
        _lib.call("wdl_act_quant_w4_static", *common, stream)
    else:
        ws = torch.empty(_lib.library().wdl_act_quant_workspace_floats(Mp, K), device=dev)
        _lib.call("wdl_act_quant_w4", *common, ws.data_ptr(), stream)
    torch.cuda.synchronize()
    return q, asc, lora


@pytest.mark.parametrize("K", [3072, 14336])
def test_static_scratch_matches_workspace_entry_point_twice(gpu, K):
    g = torch.Generator(device="cuda").manual_seed(K)
    dev = torch.device("cuda")
    pdt = (torch.randn(32, K, device=dev, generator=g) / K ** 0.5).to(torch.bfloat16)
    smooth = (torch.rand(K, device=dev, generator=g) + 0.5).to(torch.bfloat16)
    ln = None if K > 4096 else dict(shift=torch.randn(K, device=dev, generator=g) * 0.1,
                                    scale=torch.randn(K, device=dev, generator=g) * 0.1,
                                    weight=torch.rand(K, device=dev, generator=g) + 0.5,
                                    bias=torch.randn(K, device=dev, generator=g) * 0.1)
    unsigned = K > 4096
    for M, Mp in ((1392, 1408), (300, 384)):  # second call smaller: stale scratch contents from the first
        x = torch.randn(M, K, device=dev, generator=g)
        x[:, :K // 100] *= 20
        if unsigned:
            x = torch.nn.functional.gelu(x, approximate="tanh")
        x = x.to(torch.bfloat16)
        print(f"static act quant: K={K} M={M} Mp={Mp}", flush=True)
        want = _call(False, x, smooth, pdt, M, Mp, unsigned, ln)
        got = _call(True, x, smooth, pdt, M, Mp, unsigned, ln)
        for a, b in zip(got, want):
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_static_scratch_refuses_shapes_above_its_maximum(gpu):
    from wdl import _lib

    lib = _lib.library()
    K, Mp = 14336, 8192
    assert lib.wdl_act_quant_workspace_floats(Mp, K) > (4 << 20)
    x = torch.zeros(1, K, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="static maximum"):
        _lib.call("wdl_act_quant_w4_static", x.data_ptr(), K, 1, K, x.data_ptr(), ctypes.c_float(0.0), 0, None, 32,
                  x.data_ptr(), x.data_ptr(), None, Mp, None, None, None, None, 0, ctypes.c_float(1e-6), None, None,
                  torch.cuda.current_stream().cuda_stream)
