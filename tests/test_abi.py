"""The C ABI surface on the CPU: the library loads, and it exports exactly the entry points include/wdl.h declares
(no compute calls: there is no GPU here)."""

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def declared():
    text = (ROOT / "include" / "wdl.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(wdl_\w+)\(", text, re.M)))


def test_header_declares_entry_points():
    assert "wdl_kv_append_fp8" in declared()
    assert "wdl_last_error" in declared()


def test_library_loads_and_exports_every_declared_symbol():
    from wdl import _lib

    lib = _lib.library()
    for name in declared():
        assert hasattr(lib, name), name
    assert set(declared()) == set(_lib.SIGNATURES)
    assert lib.wdl_abi_version() == 14
    assert lib.wdl_last_error() == b""


def test_return_types_follow_the_header():
    """Every entry point the header declares as returning int64_t is bound with a 64-bit ctypes result (the c_int
    default would silently truncate a workspace size), and every other int entry point with c_int."""
    import ctypes

    from wdl import _lib

    text = (ROOT / "include" / "wdl.h").read_text()
    wide = set(re.findall(r"^\s*int64_t\s+(wdl_\w+)\(", text, re.M))
    narrow = set(re.findall(r"^\s*int\s+(wdl_\w+)\(", text, re.M))
    assert wide and narrow
    lib = _lib.library()
    for name in wide:
        assert _lib.RESTYPES.get(name) is ctypes.c_int64, name
        assert getattr(lib, name).restype is ctypes.c_int64, name
    for name in narrow:
        assert getattr(lib, name).restype is ctypes.c_int, name


def test_invalid_call_reports_error_without_launch():
    from wdl import _lib

    lib = _lib.library()
    strides = _lib.i64s([1, 1, 1, 1])
    # at + n beyond capacity: rejected on the host, before any launch (null pointers are never dereferenced)
    rc = lib.wdl_kv_append_fp8(None, 2, strides, None, 2, strides, 1, 4, 1, 8, None, None, None, None, 3, 0, None)
    assert rc == 1
    assert b"exceeds capacity" in lib.wdl_last_error()


def test_live_operator_names_carry_the_reference_schemas():
    """wdl.live registers live::w4a4_linear / live::w4a4_gelu_mlp with the argument lists of
    native/ops/w4a4_ops.cpp:79-85, and their fake kernels give the reference's output shapes."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode

    import wdl.live  # noqa: F401

    lin = str(torch.ops.live.w4a4_linear.default._schema)
    assert "x, Tensor qweight, Tensor wscales, Tensor proj_down, Tensor proj_up, Tensor smooth, Tensor bias" in lin
    mlp = str(torch.ops.live.w4a4_gelu_mlp.default._schema)
    assert "qweight1" in mlp and "bias2" in mlp
    with FakeTensorMode():
        x = torch.empty(10, 128, dtype=torch.bfloat16)
        q = torch.empty(64, 64, dtype=torch.uint8)
        y = torch.ops.live.w4a4_linear(x, q, torch.empty(2, 64), torch.empty(32, 128), torch.empty(64, 32),
                                       torch.empty(128), torch.empty(64))
        assert y.shape == (10, 64) and y.dtype == torch.bfloat16


def test_weight_operand_shapes_are_checked_before_any_launch():
    import pytest
    import torch

    from wdl import ops

    with pytest.raises(ValueError):
        ops.as_codes(torch.zeros(4, 48, dtype=torch.uint8), 128)
    with pytest.raises(TypeError):
        ops.as_codes(torch.zeros(4, 64, dtype=torch.float32), 128)
    codes = torch.zeros(1, 2, 128, 48, dtype=torch.uint8)
    assert ops.as_codes(codes, 128) is not None  # blocked fp6 codes pass through
    with pytest.raises(ValueError):
        ops.as_codes(torch.zeros(128, 128, dtype=torch.uint8), 128)  # one byte per value is not an operand
    with pytest.raises(ValueError):
        ops.as_codes(torch.zeros(1, 3, 128, 48, dtype=torch.uint8), 128)  # blocked codes of another width
    with pytest.raises(ValueError):
        ops.as_codes(torch.zeros(1, 2, 128, 64, dtype=torch.uint8), 128)  # 64-byte rows
    with pytest.raises(ValueError):
        ops.encode_weights(torch.zeros(100, 128, dtype=torch.int32))  # rows not a multiple of 128
    with pytest.raises(ValueError):
        ops.encode_weights(torch.full((128, 64), 8, dtype=torch.int32))  # not an int4 weight
    with pytest.raises(ValueError):
        ops.encode_acts(torch.full((128, 64), 16, dtype=torch.int32))  # not an int4 activation


def test_fp6_codes_are_the_formats_values():
    """Each code the format helpers write is the fp6 code of the stated value: weights e3m2(2w) (bias 3, 2 mantissa
    bits), activations e2m3(q / 2) (bias 1, 3 mantissa bits), checked on the closed forms of both formats for every
    int4 value, and decode inverts encode."""
    import torch

    from wdl import ops

    def e3m2(c):
        s, e, m = (-1 if c & 32 else 1), (c >> 2) & 7, c & 3
        return s * (m / 4 * 2.0 ** -2 if e == 0 else 2.0 ** (e - 3) * (1 + m / 4))

    def e2m3(c):
        s, e, m = (-1 if c & 32 else 1), (c >> 3) & 3, c & 7
        return s * (m / 8 if e == 0 else 2.0 ** (e - 1) * (1 + m / 8))

    w = torch.arange(-8, 8).repeat(128, 4)            # [128, 64]
    q = torch.arange(-8, 16).repeat(128, 3)[:, :64]   # [128, 64]
    cw = ops._unpack6(ops.encode_weights(w))
    ca = ops._unpack6(ops.encode_acts(q))
    assert all(e3m2(int(c)) == 2 * int(v) for c, v in zip(cw[0], w[0]))
    assert all(e2m3(int(c)) == int(v) / 2 for c, v in zip(ca[0], q[0]))
    assert torch.equal(cw, cw[:1].expand_as(cw)) and torch.equal(ca, ca[:1].expand_as(ca))
    assert int(cw[0, 9]) == 0b010000 and int(cw[0, 0]) == 0b111100  # w = 1: 2 = 1.0 * 2^1; w = -8: -16
    assert int(ca[0, 9]) == 0b000100 and int(ca[0, 23]) == 0b011111  # q = 1: subnormal 0.5; q = 15: 7.5
    assert torch.equal(ops.decode_weights(ops.encode_weights(w)), w.to(torch.int32))
    assert torch.equal(ops.decode_acts(ops.encode_acts(q)), q.to(torch.int32))


def test_tile_blocked_layout_offsets():
    """Code k of row r sits where the kernels put it: 128-row tiles of [K/64][128][48 bytes] (group g of row r at
    (r // 128) * (K / 64) * 6144 + g * 6144 + (r % 128) * 48), value k of the group in half h = k // 32 at bits
    6 (k % 32) of the half's 24 bytes, the half's bytes 0..15 at 16 h and bytes 16..23 at 32 + 8 h."""
    import torch

    from wdl import ops

    R, K = 256, 192
    g = torch.Generator().manual_seed(0)
    w = torch.randint(-8, 8, (R, K), generator=g, dtype=torch.int32)
    b = ops.encode_weights(w)
    assert b.shape == (2, 3, 128, 48) and b.is_contiguous()
    codes = ops._W_ENC[(w + 8).long()]
    flat = b.reshape(-1)

    def byte_at(r, grp, h, hb):
        base = (r // 128) * (K // 64) * 6144 + grp * 6144 + (r % 128) * 48
        return int(flat[base + (16 * h + hb if hb < 16 else 32 + 8 * h + hb - 16)])

    for r in [0, 5, 127, 128, 200, 255]:
        for k in range(K):
            grp, h, i = k // 64, (k % 64) // 32, k % 32
            bit = 6 * i
            lo = byte_at(r, grp, h, bit // 8)
            hi = byte_at(r, grp, h, bit // 8 + 1) if bit // 8 + 1 < 24 else 0
            assert ((lo | hi << 8) >> (bit % 8)) & 63 == int(codes[r, k]), (r, k)
    assert torch.equal(ops.decode_weights(b), w)


def test_static_scratch_size_is_one_value():
    """WDL_ACT_QUANT_STATIC_FLOATS (the no-workspace quantizer's static array) is stated once in the public header
    and once for the kernels: both must be the same 4 Mi floats."""
    public = (ROOT / "include" / "wdl.h").read_text()
    private = (ROOT / "wan-dit-lab_amd" / "csrc" / "wdl_common.h").read_text()
    assert "#define WDL_ACT_QUANT_STATIC_FLOATS ((int64_t)4 << 20)" in public
    assert "#define WDL_ACT_QUANT_STATIC_FLOATS (int64_t(4) << 20)" in private
