"""The on-disk weight pack (wdl/pack.py; the reference's block_w4a4_v2 rows + manifest, quantization/w4a4.py:279-436)
on the CPU: a round trip is bit-exact for every tensor, entries are 16-byte aligned, the manifest's sha256 is the
file's, and a pack that exists, is incomplete, has another format / source or a wrong digest is refused."""

import hashlib
import json

import pytest
import torch

from wdl import pack, w4a4


def parts_of(dim, ffn, seed):
    g = torch.Generator().manual_seed(seed)
    shapes = dict(qkv=(3 * dim, dim), o=(dim, dim), cq=(dim, dim), ck=(dim, dim), cv=(dim, dim), co=(dim, dim),
                  ffn1=(ffn, dim), ffn2=(dim, ffn))
    P = {k: w4a4.random_parts(n, kk, "cpu", g) for k, (n, kk) in shapes.items()}
    for k in ("wq", "wk", "cwq", "cwk"):
        P[k] = torch.randn(dim, generator=g).to(torch.bfloat16)
    P["n3w"], P["n3b"] = torch.randn(dim, generator=g), torch.randn(dim, generator=g)
    P["modulation"] = torch.randn(6, dim, generator=g)
    return P


def same(a, b):
    assert a.dtype == b.dtype and a.shape == b.shape
    assert torch.equal(a.view(torch.uint8) if a.dtype != torch.uint8 else a,
                       b.view(torch.uint8) if b.dtype != torch.uint8 else b)


def test_round_trip_is_bit_exact(tmp_path):
    blocks = [parts_of(256, 1024, s) for s in (0, 1)]
    path = tmp_path / "blocks.pack"
    info = pack.build_pack(blocks, path, source="test", calibrated=False)
    assert info["format"] == pack.FORMAT and info["blocks"] == 2 and info["calibrated"] is False
    rows, layout, meta = pack.mapped_pack(path, source="test", verify=True)
    assert rows.shape == (2, meta["bytes_per_block"]) and meta["bytes"] == path.stat().st_size
    assert all(e["offset"] % 16 == 0 for e in layout)
    assert hashlib.sha256(path.read_bytes()).hexdigest() == meta["sha256"]
    for i, parts in enumerate(blocks):
        got = pack.slot(rows[i], layout)
        for k in pack.LAYERS:
            for p in pack.PARTS:
                same(got[k][p], parts[k][p])
        for k in pack.OTHERS:
            same(got[k], parts[k])
    assert not path.with_suffix(".pack.tmp").exists()


def test_refusals(tmp_path):
    blocks = [parts_of(128, 256, 2)]
    path = tmp_path / "b.pack"
    pack.build_pack(blocks, path, source="a")
    with pytest.raises(FileExistsError):
        pack.build_pack(blocks, path, source="a")
    with pytest.raises(ValueError):
        pack.mapped_pack(path, source="b")
    data = bytearray(path.read_bytes())
    data[100] ^= 1
    path.write_bytes(bytes(data))
    pack.mapped_pack(path)  # the digest is only checked on request
    with pytest.raises(ValueError):
        pack.mapped_pack(path, verify=True)
    path.write_bytes(bytes(data[:-16]))
    with pytest.raises(ValueError):
        pack.mapped_pack(path)
    manifest = path.with_suffix(".pack.json")
    meta = json.loads(manifest.read_text())
    meta["format"] = "block_w4a4_v2"  # the reference's Nunchaku layout is another format
    manifest.write_text(json.dumps(meta))
    with pytest.raises(ValueError):
        pack.mapped_pack(path)
    with pytest.raises(ValueError):  # blocks of different shapes cannot share a pack
        pack.build_pack([parts_of(128, 256, 3), parts_of(128, 512, 4)], tmp_path / "c.pack")
    assert not (tmp_path / "c.pack").exists() and not (tmp_path / "c.pack.json").exists()


def test_blocks_holding_only_weight_codes_write_the_same_pack(tmp_path):
    """A QuantizedWanBlock keeps only the GEMM's fp6 weight codes; its parts write the nibbles they decode to, so
    the pack is byte-identical to the one written from the packed parts."""
    from wdl import ops

    P = parts_of(256, 1024, 3)
    codes_only = {k: (dict(v) if isinstance(v, dict) else v) for k, v in P.items()}
    for k, v in codes_only.items():
        if isinstance(v, dict):
            v["wcodes"] = ops.encode_weights(w4a4.unpack_weight(v.pop("qweight")))
    pack.build_pack([P], tmp_path / "a.pack")
    pack.build_pack([codes_only], tmp_path / "b.pack")
    assert (tmp_path / "a.pack").read_bytes() == (tmp_path / "b.pack").read_bytes()


def test_fp16_weight_scales_round_trip(tmp_path):
    P = parts_of(256, 1024, 4)
    for v in P.values():
        if isinstance(v, dict):
            v["wscales"] = v["wscales"].to(torch.float16)
    pack.build_pack([P], tmp_path / "h.pack")
    rows, layout, _ = pack.mapped_pack(tmp_path / "h.pack")
    back = pack.slot(rows[0], layout)
    for k, v in P.items():
        if isinstance(v, dict):
            assert back[k]["wscales"].dtype == torch.float16
            same(back[k]["wscales"], v["wscales"])


def mixed_parts_of(dim, ffn, seed):
    """Mixed-precision parts: the attention projections FP8 weight-only (e4m3 rows, fp32 scale per row, bf16 bias),
    the feed-forward W4A4."""
    g = torch.Generator().manual_seed(seed)
    P = parts_of(dim, ffn, seed)
    for k, (n, kk) in dict(qkv=(3 * dim, dim), o=(dim, dim), cq=(dim, dim), ck=(dim, dim), cv=(dim, dim),
                           co=(dim, dim)).items():
        w = torch.randn(n, kk, generator=g) * 0.02
        s = w.abs().amax(1) / 448
        P[k] = dict(fp8=(w / s[:, None]).to(torch.float8_e4m3fn), fp8_scale=s.float(),
                    bias=(torch.randn(n, generator=g) * 0.02).to(torch.bfloat16))
    return P


def test_mixed_precision_round_trip(tmp_path):
    """Blocks with FP8 weight-only attention projections pack under block_mixed_v1_gfx950: every entry (e4m3 codes,
    per-row scales, biases, the W4A4 feed-forward, norms) round-trips bit-exactly, 16-byte aligned, digest checked;
    an all-W4A4 pack keeps block_w4a4_v2_gfx950; an FP8 feed-forward is refused before anything is written."""
    blocks = [mixed_parts_of(256, 1024, s) for s in (5, 6)]
    path = tmp_path / "m.pack"
    info = pack.build_pack(blocks, path, source="mixed")
    assert info["format"] == pack.FORMAT_MIXED and "FP8" in info["quantization"]
    rows, layout, meta = pack.mapped_pack(path, source="mixed", verify=True)
    assert all(e["offset"] % 16 == 0 for e in layout)
    assert [e["name"] for e in layout][:3] == ["self_attn.qkv.fp8", "self_attn.qkv.fp8_scale", "self_attn.qkv.bias"]
    for i, parts in enumerate(blocks):
        got = pack.slot(rows[i], layout)
        for k in pack.LAYERS:
            for p in (pack.FP8_PARTS if "fp8" in parts[k] else pack.PARTS):
                same(got[k][p], parts[k][p])
        for k in pack.OTHERS:
            same(got[k], parts[k])
    assert pack.build_pack([parts_of(128, 256, 1)], tmp_path / "w.pack")["format"] == pack.FORMAT
    bad = mixed_parts_of(128, 256, 7)
    bad["ffn1"] = dict(bad["qkv"])
    with pytest.raises(ValueError, match="feed-forward"):
        pack.build_pack([bad], tmp_path / "bad.pack")
    assert not (tmp_path / "bad.pack").exists() and not (tmp_path / "bad.pack.json").exists()
