"""wdl::rope3d_rotate / wdl.rope.rope_apply (the reference's standalone RoPE operator, kernels/rope_triton.py:14-139)
against the oracle's general rotation (oracle/rope.py rope_rotate, pinned to the reference's fp64 complex-phase
oracle): bit-exact results in every input / output dtype, per-sample grids, strides, padding, the inverse rotation
as the autograd backward, torch.compile and graph capture, one kernel per call, contract violations rejected."""

import pytest
import torch

from oracle import rope as orope

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16, torch.float32, torch.float64]


def table(dim=128, positions=64, dtype=torch.float64):
    return orope.freqs(dim, positions).to(dtype).cuda()


def same(a, b):
    assert a.dtype == b.dtype and a.shape == b.shape
    assert torch.equal(a.cpu(), b.cpu())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch", [1, 2, 4, 8])
def test_forward_and_backward_bit_exact(gpu, dtype, batch):
    from wdl.rope import rope_apply

    g = torch.Generator(device="cuda").manual_seed(12 + batch)
    grids = ((2, 3, 5),) * batch
    x = torch.randn(batch, 30, 3, 128, device="cuda", generator=g).to(dtype).requires_grad_()
    freq = table()
    y = rope_apply(x, grids, freq, 7)
    same(y.detach(), orope.rope_rotate(x.detach().cpu(), grids, freq.cpu(), 7))
    probe = torch.randn(batch, 30, 3, 256, device="cuda", generator=g).to(dtype)[..., ::2]  # strided upstream grad
    grad = torch.autograd.grad(y, x, probe)[0]
    same(grad, orope.rope_rotate(probe.cpu(), grids, freq.cpu(), 7, inverse=True))


@pytest.mark.parametrize("dtype", DTYPES[:3])
def test_strided_input_per_sample_grids_padding_untouched(gpu, dtype):
    from wdl.rope import rope_apply

    g = torch.Generator(device="cuda").manual_seed(5)
    grids = ((2, 3, 5), (1, 2, 4))
    x = torch.randn(2, 33, 2, 256, device="cuda", generator=g).to(dtype)[..., ::2]
    before = x.clone()
    y = rope_apply(x, torch.tensor(grids), table(), 3)
    same(y, orope.rope_rotate(x.cpu(), grids, table().cpu(), 3))
    same(x, before)
    for b, (f, h, w) in enumerate(grids):
        same(y[b, f * h * w:], x[b, f * h * w:].contiguous())
    assert y.data_ptr() != x.data_ptr() and y.is_contiguous()


@pytest.mark.parametrize("dim", [2, 6, 12, 64, 128])
def test_axis_splits_and_strided_tables(gpu, dim):
    from wdl.rope import rope_apply

    store = torch.zeros(2, 64, dim, device="cuda", dtype=torch.float64)
    store[..., ::2] = table(dim)
    freq = store[..., ::2]  # a non-contiguous table
    x = torch.randn(1, 15, 3, dim, device="cuda")
    same(rope_apply(x, ((1, 3, 5),), freq, 11), orope.rope_rotate(x.cpu(), ((1, 3, 5),), freq.cpu(), 11))


def test_rotation_invariants(gpu):
    """Norms are kept, a chunk rotated with its frame offset equals the same frames of a longer sequence, and
    q . k depends only on the relative position (test_rope_triton.py:89-104)."""
    from wdl.rope import rope_apply

    freq = table(12)
    x = torch.randn(1, 12, 2, 12, device="cuda", dtype=torch.float64)
    rot = rope_apply(x, ((3, 2, 2),), freq, 5)
    assert torch.allclose(rot.square().sum(-1), x.square().sum(-1), rtol=2e-14, atol=2e-14)
    parts = torch.cat([rope_apply(x[:, 4 * i:4 * i + 4], ((1, 2, 2),), freq, 5 + i) for i in range(3)], dim=1)
    same(rot, parts)
    q = torch.randn_like(x)
    dot = lambda a, b: (a * b).sum(-1)
    d0 = dot(rope_apply(x, ((3, 2, 2),), freq, 2), rope_apply(q, ((3, 2, 2),), freq, 7))
    d1 = dot(rope_apply(x, ((3, 2, 2),), freq, 9), rope_apply(q, ((3, 2, 2),), freq, 14))
    assert torch.allclose(d0, d1, rtol=2e-13, atol=2e-13)


def test_gradcheck_and_second_order(gpu):
    from wdl.rope import rope_apply

    x = torch.randn(1, 2, 1, 6, device="cuda", dtype=torch.float64, requires_grad=True)
    fn = lambda v: rope_apply(v, ((1, 1, 2),), table(6), 2)
    assert torch.autograd.gradcheck(fn, (x,), eps=1e-6, atol=1e-7, rtol=1e-5)
    assert torch.autograd.gradgradcheck(fn, (x,), eps=1e-6, atol=1e-7, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fp32_tables_and_fp32_output(gpu, dtype):
    """The live presets' fp32 tables (fp32 arithmetic, each product rounded) and the Wan adapter's fp32 output of a
    bf16 input (rope_triton.py:146-152)."""
    from wdl.rope import rope_apply

    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn(2, 30, 3, 128, device="cuda", generator=g).to(dtype)
    f32 = table(dtype=torch.float32)
    same(rope_apply(x, ((2, 3, 5),) * 2, f32, 4), orope.rope_rotate(x.cpu(), ((2, 3, 5),) * 2, f32.cpu(), 4))
    y = rope_apply(x, ((2, 3, 5),) * 2, table(), 4, output_dtype=torch.float32)
    same(y, orope.rope_rotate(x.cpu(), ((2, 3, 5),) * 2, table().cpu(), 4, out_dtype=torch.float32))


def test_compile_fullgraph_forward_and_backward(gpu):
    from wdl.rope import rope_apply

    compiled = torch.compile(rope_apply, fullgraph=True, dynamic=False)
    for batch, grids in [(1, ((2, 3, 5),)), (2, ((1, 3, 5), (2, 3, 5)))]:
        x = torch.randn(batch, 30, 2, 12, device="cuda", requires_grad=True)
        probe = torch.randn(batch, 30, 2, 12, device="cuda")
        eager = rope_apply(x, grids, table(12), 1)
        comp = compiled(x, grids, table(12), 1)
        same(comp.detach(), eager.detach())
        same(torch.autograd.grad(comp, x, probe)[0], torch.autograd.grad(eager, x, probe)[0])


def test_one_kernel_on_the_current_stream_and_graph_replay(gpu):
    from torch.profiler import ProfilerActivity, profile

    from wdl.rope import rope_apply

    x = torch.randn(1, 30, 2, 128, device="cuda", dtype=torch.bfloat16)
    freq = table()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with profile(activities=[ProfilerActivity.CUDA]) as prof, torch.cuda.stream(side):
        y = rope_apply(x, ((2, 3, 5),), freq, 0)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    kernels = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    assert sum("rope3d_kernel" in k for k in kernels) == 1, kernels
    graph = torch.cuda.CUDAGraph()
    out = None
    with torch.cuda.graph(graph):
        out = rope_apply(x, ((2, 3, 5),), freq, 0)
    for _ in range(3):
        x.copy_(torch.randn_like(x))
        graph.replay()
        torch.cuda.synchronize()
        same(out, rope_apply(x, ((2, 3, 5),), freq, 0))


def test_operator_schema_and_empty_input(gpu):
    from wdl.rope import rope3d_rotate, rope_apply

    schema = str(torch.ops.wdl.rope3d_rotate.default._schema)
    assert "Tensor x, Tensor freq, str grid_key, SymInt start, bool inverse, ScalarType output_dtype" in schema
    empty = torch.empty(1, 0, 2, 12, device="cuda")
    assert rope_apply(empty, ((0, 1, 1),), table(12), 0).shape == empty.shape
    assert rope3d_rotate(empty, table(12), "0,1,1", 0, False, torch.float16).dtype == torch.float16


BAD = {
    "cpu input": lambda a: a.update(x=a["x"].cpu()),
    "integer input": (lambda a: a.update(x=a["x"].long()), TypeError),
    "odd dim": lambda a: a.update(x=a["x"][..., :11]),
    "table shape": lambda a: a.update(freq=a["freq"][:, :, :5]),
    "trainable table": lambda a: a.update(freq=a["freq"].clone().requires_grad_()),
    "grid count": lambda a: a.update(grids=((2, 3, 5), (2, 3, 5))),
    "grid too long": lambda a: a.update(grids=((2, 4, 5),)),
    "negative start": lambda a: a.update(start=-1),
    "past the table": lambda a: a.update(start=63),
    "float grid": lambda a: a.update(grids=((2.0, 3, 5),)),
    "device grid": lambda a: a.update(grids=torch.tensor([[2, 3, 5]], device="cuda")),
    "output dtype": (lambda a: a.update(out=torch.int32), TypeError),
}


@pytest.mark.parametrize("problem", list(BAD))
def test_contract_violations_raise(gpu, problem):
    from wdl.rope import rope_apply

    change, exc = BAD[problem] if isinstance(BAD[problem], tuple) else (BAD[problem], ValueError)
    a = dict(x=torch.randn(1, 30, 2, 12, device="cuda"), grids=((2, 3, 5),), freq=table(12), start=0, out=None)
    change(a)
    with pytest.raises(exc):
        rope_apply(a["x"], a["grids"], a["freq"], a["start"], output_dtype=a["out"])
