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
    assert lib.wdl_abi_version() == 4
    assert lib.wdl_last_error() == b""


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
    codes = torch.zeros(128, 128, dtype=torch.uint8)
    assert ops.as_codes(codes, 128).shape == (1, 2, 128, 64)  # [N, K] codes are blocked
    with pytest.raises(ValueError):
        ops.as_codes(torch.zeros(1, 3, 128, 64, dtype=torch.uint8), 128)  # blocked codes of another width
    with pytest.raises(ValueError):
        ops.block_rows(torch.zeros(100, 128, dtype=torch.uint8))  # rows not a multiple of 128


def test_tile_blocked_layout_round_trip_and_offsets():
    """block_rows / unblock_rows are inverse; element (r, k) of the blocked copy sits at the byte offset
    (r // 128) * 128 * K + (k // 64) * 8192 + (r % 128) * 64 + k % 64, the one the kernels use."""
    import torch

    from wdl import ops

    R, K = 256, 192
    t = torch.randint(0, 256, (R, K), generator=torch.Generator().manual_seed(0), dtype=torch.int32).to(torch.uint8)
    b = ops.block_rows(t)
    assert b.shape == (2, 3, 128, 64) and b.is_contiguous()
    assert torch.equal(ops.unblock_rows(b), t)
    flat = b.reshape(-1)
    for r, k in [(0, 0), (5, 70), (127, 191), (128, 0), (200, 100), (255, 191)]:
        off = (r // 128) * 128 * K + (k // 64) * 8192 + (r % 128) * 64 + k % 64
        assert int(flat[off]) == int(t[r, k])
