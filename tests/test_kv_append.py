"""wdl_kv_append_fp8 (through wdl.cache_fp8.store_kv_fp8) against the oracle's quantize_rows, bit for bit: the
cache rows written, their fp32 scales, and every byte outside the written rows left as it was. The contract is the
reference's FP8 cache store (kernels/cache_fp8.py:75-105; its tests at tests/test_cache_fp8.py); the known-answer
rows are data in tests/golden/fp8_known_answers.json."""

import json
from pathlib import Path

import pytest
import torch

from oracle.fp8 import quantize_rows

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
KNOWN = json.loads((Path(__file__).parent / "golden" / "fp8_known_answers.json").read_text())
DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}


class Target:
    """A cache of `rows` rows (fp8 K / V and fp32 scales) filled with sentinels that no write produces here, and a
    CPU copy of what it must hold after writes."""

    def __init__(self, batch, rows, heads, dim):
        self.k = torch.full((batch, rows, heads, dim), 2.0, device="cuda").to(FP8)
        self.v = torch.full((batch, rows, heads, dim), -2.0, device="cuda").to(FP8)
        self.ks = torch.full((batch, rows, heads, 1), 7.0, device="cuda")
        self.vs = torch.full((batch, rows, heads, 1), 9.0, device="cuda")
        self.expect = [t.cpu().clone() for t in self.buffers()]

    def buffers(self):
        return self.k, self.ks, self.v, self.vs

    def write(self, k, v, at, stream=None):
        from wdl.cache_fp8 import store_kv_fp8

        n = k.shape[1]
        for x, (vi, si) in ((k, (0, 1)), (v, (2, 3))):
            q, s = quantize_rows(x.cpu())
            self.expect[vi][:, at:at + n], self.expect[si][:, at:at + n] = q, s
        store_kv_fp8(k, v, *self.buffers(), at)

    def check(self):
        torch.cuda.synchronize()
        for got, want in zip(self.buffers(), self.expect):
            got = got.cpu()
            if got.dtype == FP8:
                got, want = got.view(torch.uint8), want.view(torch.uint8)
            assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", list(DTYPES))
def test_known_answer_rows(gpu, dtype):
    b = KNOWN["boundary_row"]
    row = torch.tensor(b["values"] * b["repeat"]).to(DTYPES[dtype]).reshape(1, 1, 1, -1).cuda()
    t = Target(1, 3, 1, row.shape[-1])
    t.write(row, torch.zeros_like(row), 1)
    t.check()
    assert float(t.ks[0, 1, 0, 0]) == b["scale"]
    assert t.k[0, 1, 0, :4].view(torch.uint8).cpu().tolist() == b["bits_first4"]
    assert t.k[0, 1, 0, 4:12].float().cpu().tolist() == b["values_4_to_12"]
    m = KNOWN["midpoint_row"]
    row = torch.tensor(m["values"], dtype=DTYPES[m["dtype"]]).reshape(1, 1, 1, -1).cuda()
    t = Target(1, 3, 1, row.shape[-1])
    t.write(row, row, 1)
    t.check()
    assert t.k[0, 1, 0].float().cpu().tolist() == m["expected"] and float(t.ks[0, 1, 0, 0]) == m["scale"]


@pytest.mark.parametrize("dtype", list(DTYPES.values()))
@pytest.mark.parametrize("shape", [(1, 2, 64), (2, 3, 128), (1, 1, 160), (1, 24, 128)])
def test_random_rows_leave_the_rest_untouched(gpu, dtype, shape):
    batch, heads, dim = shape
    g = torch.Generator(device="cuda").manual_seed(23)
    k = torch.randn(batch, 7, heads, dim, device="cuda", generator=g).to(dtype)
    v = 3 * torch.randn(batch, 7, heads, dim, device="cuda", generator=g).to(dtype)
    k0, v0 = k.clone(), v.clone()
    t = Target(batch, 17, heads, dim)
    t.write(k, v, 5)
    t.check()
    assert torch.equal(k, k0) and torch.equal(v, v0)  # inputs are read only


def test_every_e4m3_magnitude_and_every_midpoint(gpu):
    """All 127 finite magnitudes and the midpoints between neighbours, both signs, with 448 in the row so the scale
    is exactly 1: the kernel's conversion must take every tie to the even code."""
    mags = torch.arange(127, dtype=torch.uint8).view(FP8).float()
    mids = 0.5 * (mags[1:] + mags[:-1])
    row = torch.cat([mags, -mags, mids, -mids, torch.tensor([448.0])])
    row = torch.nn.functional.pad(row, (0, (-row.numel()) % 8)).reshape(1, 1, 1, -1).cuda()
    t = Target(1, 1, 1, row.shape[-1])
    t.write(row, -row, 0)
    t.check()


def test_strided_mixed_dtype_inputs_on_a_side_stream(gpu):
    g = torch.Generator(device="cuda").manual_seed(4)
    k = torch.randn(2, 5, 3, 256, device="cuda", generator=g)[..., ::2]                       # fp32, stride 2
    v = torch.randn(2, 10, 3, 128, device="cuda", generator=g).to(torch.bfloat16)[:, ::2]     # bf16, token stride
    t = Target(2, 11, 3, 128)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        t.write(k, v, 6)
    torch.cuda.current_stream().wait_stream(side)
    t.check()


def test_replays_of_a_captured_append(gpu):
    g = torch.Generator(device="cuda").manual_seed(8)
    k = torch.randn(1, 7, 2, 128, device="cuda", generator=g).to(torch.bfloat16)
    v = torch.randn(1, 7, 2, 128, device="cuda", generator=g).to(torch.bfloat16)
    t = Target(1, 12, 2, 128)
    t.write(k, v, 4)  # eager once before capture
    t.check()
    from wdl.cache_fp8 import store_kv_fp8

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        store_kv_fp8(k, v, *t.buffers(), 4)
    for _ in range(3):
        k.copy_(torch.randn(k.shape, device="cuda", generator=g))
        v.copy_(torch.randn(v.shape, device="cuda", generator=g))
        graph.replay()
        for x, (vi, si) in ((k, (0, 1)), (v, (2, 3))):
            t.expect[vi][:, 4:11], t.expect[si][:, 4:11] = quantize_rows(x.cpu())
        t.check()


BAD = {
    "negative offset": lambda a: a.update(at=-1),
    "past the end": lambda a: a.update(at=4),
    "K / V shapes differ": lambda a: a.update(v=a["v"][:, :3]),
    "cache not fp8": lambda a: a["bufs"].__setitem__(0, a["bufs"][0].float()),
    "scales not fp32": lambda a: a["bufs"].__setitem__(1, a["bufs"][1].half()),
    "input needs grad": lambda a: a["k"].requires_grad_(),
    "strided scales": lambda a: a["bufs"].__setitem__(
        1, torch.full((1, 2, 8, 1), 7.0, device="cuda").transpose(1, 2)),
}


@pytest.mark.parametrize("problem", list(BAD))
def test_contract_violations_raise_before_any_write(gpu, problem):
    from wdl.cache_fp8 import store_kv_fp8

    t = Target(1, 8, 2, 128)
    k = torch.randn(1, 5, 2, 128, device="cuda")
    args = dict(k=k, v=k.clone(), bufs=list(t.buffers()), at=1)
    BAD[problem](args)
    with pytest.raises((ValueError, TypeError)):
        store_kv_fp8(args["k"], args["v"], *args["bufs"], args["at"])
    t.check()  # the original buffers hold their sentinels
