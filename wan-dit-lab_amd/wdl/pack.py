"""On-disk weight pack of quantized blocks in wdl's physical layout (block_w4a4_v2_gfx950; block_mixed_v1_gfx950 with FP8
weight-only attention projections).

The reference's block_w4a4_v2 pack (quantization/w4a4.py:279-313 pack_layout, 360-436 build_pack / mapped_pack;
weight_pack.py:84-171 for the FP8 sibling): one uint8 row per block, each tensor of the block at a 16-byte aligned
offset of the row, the rows back to back in one file, and a JSON manifest beside it (`<path>.json`) with the format,
the layout (name, dtype, shape, offset, bytes per entry), the bytes per block, the sha256 of the whole file and the
source identity. The file is written to `<path>.tmp` first and renamed when complete; an existing target raises
FileExistsError; any failure removes what was written.

The library's rows hold the QuantizedWanBlock parts in its own layouts (the reference's hold Nunchaku's): per W4A4
layer — fused self_attn.qkv, self_attn.o, cross_attn.q / k / v / o, ffn.0 and ffn.2 (the GELU MLP's second layer,
quantized for GELU's output + 0.171875) — qweight uint8 [N, K/2] (per 64-group byte j = k_j low nibble, k_{j+32}
high nibble), wscales bf16 or fp16 [K/64, N], proj_down bf16 [32, K], proj_up bf16 [N, 32], smooth bf16 [K], bias bf16
[N]; then the Q/K RMSNorm weights (bf16), norm3's affine (fp32) and the modulation (fp32 [6, dim]). The manifest
names that layout ("layout_notes"), so a reader never guesses it.

Blocks of the mixed-precision mode (attention projections FP8 weight-only, feed-forward W4A4) are packed the same
way under the format block_mixed_v1_gfx950: an FP8 layer's entries are fp8 (e4m3 codes [N, K]), fp8_scale (fp32 [N],
one per output row, or [1]) and bias (bf16 [N]), in the place of the W4A4 layer's six — the FP8 sibling of the
reference's block_fp8_v1 rows (weight_pack.py:84-171: e4m3 weights with fp32 scales, 16-byte aligned entries), with
this build's per-row scales.
"""

from __future__ import annotations

import hashlib
import json
import os
from pathlib import Path

import numpy as np
import torch

FORMAT = "block_w4a4_v2_gfx950"
FORMAT_MIXED = "block_mixed_v1_gfx950"
FORMATS = (FORMAT, FORMAT_MIXED)
FP8_PARTS = ("fp8", "fp8_scale", "bias")
ALIGN = 16
# wdl's part names -> the reference block's module names (models/block.py, multi_head_attention.py)
LAYERS = {"qkv": "self_attn.qkv", "o": "self_attn.o", "cq": "cross_attn.q", "ck": "cross_attn.k",
          "cv": "cross_attn.v", "co": "cross_attn.o", "ffn1": "ffn.0", "ffn2": "ffn.2"}
PARTS = ("qweight", "wscales", "proj_down", "proj_up", "smooth", "bias")
OTHERS = {"wq": "self_attn.norm_q.weight", "wk": "self_attn.norm_k.weight", "cwq": "cross_attn.norm_q.weight",
          "cwk": "cross_attn.norm_k.weight", "n3w": "norm3.weight", "n3b": "norm3.bias", "modulation": "modulation"}
DTYPES = {torch.uint8: "uint8", torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32",
          torch.float8_e4m3fn: "float8_e4m3fn"}
LAYOUT_NOTES = ("qweight uint8 [N, K/2]: per 64-group byte j holds k_j (low nibble) and k_{j+32} (high), int4 in "
                "two's complement; wscales bf16 or fp16 [K/64, N] group-major; proj_down bf16 [32, K] (transposed); proj_up "
                "bf16 [N, 32]; smooth bf16 [K]; bias bf16 [N]; ffn.2 quantized for the GELU output + 0.171875 "
                "(unsigned int4 activations); norm weights bf16; norm3 affine and modulation fp32")
LAYOUT_NOTES_MIXED = LAYOUT_NOTES + ("; FP8 weight-only layers: fp8 e4m3 [N, K] row-major, fp8_scale fp32 [N] (per "
                                     "output row) or [1], bias bf16 [N]; y = fp8_scale * (x . w) + bias with bf16 x")


def _entries(parts: dict):
    """(name, tensor) of a block's parts, in row order. A layer that holds only the GEMM's weight codes (a
    QuantizedWanBlock drops the packed nibbles once it has them) is written as the nibbles those codes decode to."""
    for key, name in LAYERS.items():
        if "fp8" in parts[key]:  # an FP8 weight-only layer (the mixed-precision mode)
            if key in ("ffn1", "ffn2"):
                raise ValueError(f"{key}: the feed-forward is W4A4 in every mode")
            t = parts[key]
            yield f"{name}.fp8", t["fp8"].contiguous()
            yield f"{name}.fp8_scale", t["fp8_scale"].reshape(-1).float()
            yield f"{name}.bias", t["bias"].to(torch.bfloat16)
            continue
        for p in PARTS:
            if p == "qweight" and p not in parts[key]:
                from wdl.ops import decode_weights
                from wdl.w4a4 import pack_weight

                yield f"{name}.{p}", pack_weight(decode_weights(parts[key]["wcodes"].cpu()))
                continue
            yield f"{name}.{p}", parts[key][p]
    for key, name in OTHERS.items():
        yield name, parts[key]


def pack_layout(parts: dict):
    """The row layout of a block's parts: [dict(name, dtype, shape, offset, bytes)], bytes per row."""
    layout, offset = [], 0
    for name, t in _entries(parts):
        if t.dtype not in DTYPES:
            raise TypeError(f"{name}: dtype {t.dtype} has no pack type")
        size = t.numel() * t.element_size()
        layout.append(dict(name=name, dtype=DTYPES[t.dtype], shape=list(t.shape), offset=offset, bytes=size))
        offset += -(-size // ALIGN) * ALIGN
    return layout, offset


class _StagedFile:
    """Writes `target` under a temporary name and publishes it by rename only when the whole body succeeded;
    on any exception the temporary, and a companion file written inside the body, are removed. The bytes written
    are hashed as they go."""

    def __init__(self, target: Path, companion: Path):
        self.target, self.companion = target, companion
        self.temp = target.with_name(target.name + ".tmp")
        self.sha = hashlib.sha256()
        self.written = 0

    def __enter__(self):
        for p in (self.target, self.companion, self.temp):
            if p.exists():
                raise FileExistsError(p)
        self.fd = os.open(self.temp, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o644)
        return self

    def write(self, data: bytes):
        self.sha.update(data)
        view = memoryview(data)
        while view:
            view = view[os.write(self.fd, view):]
        self.written += len(data)

    def __exit__(self, kind, value, tb):
        try:
            if kind is None:
                os.fsync(self.fd)
        finally:
            os.close(self.fd)
        if kind is None:
            os.replace(self.temp, self.target)
            return False
        for p in (self.temp, self.target, self.companion):
            if p.exists():
                p.unlink()
        return False


def _row_bytes(parts: dict, layout: list, size: int) -> bytes:
    """One block's row: every entry's raw bytes at its offset, zero padding between entries."""
    row = np.zeros(size, dtype=np.uint8)
    for e, (_, t) in zip(layout, _entries(parts)):
        raw = t.detach().cpu().contiguous().view(torch.uint8).reshape(-1).numpy()
        row[e["offset"]:e["offset"] + raw.size] = raw
    return row.tobytes()


def build_pack(blocks: list, path, source: str = "", **metadata) -> dict:
    """Writes the parts dicts of `blocks` (QuantizedWanBlock.p or build_block inputs; any device) as a pack at
    `path` with its manifest `<path>.json`; returns the manifest without the layout. Refuses an existing pack
    (FileExistsError) and blocks of differing layouts (ValueError) before writing anything."""
    path = Path(path)
    if not blocks:
        raise ValueError("a pack needs at least one block")
    layouts = [pack_layout(b) for b in blocks]
    if any(lay != layouts[0] for lay in layouts[1:]):
        raise ValueError("packed blocks must share one layout")
    layout, size = layouts[0]
    mixed = any(e["name"].endswith(".fp8") for e in layout)
    manifest = path.with_name(path.name + ".json")
    with _StagedFile(path, manifest) as out:
        for parts in blocks:
            out.write(_row_bytes(parts, layout, size))
        quantization = ("SVDQuant W4A4: int4 groups of 64, rank-32 low-rank branch in bf16, smoothing; q, k, v of "
                        "self-attention as one layer, the feed forward as the fused GELU MLP")
        if mixed:
            quantization += ("; the attention projections FP8 e4m3 weight-only (one fp32 scale per output row, bf16 "
                             "activations)")
        meta = dict(format=FORMAT_MIXED if mixed else FORMAT, blocks=len(blocks), layout=layout,
                    bytes_per_block=size, bytes=out.written, sha256=out.sha.hexdigest(), source=source,
                    layout_notes=LAYOUT_NOTES_MIXED if mixed else LAYOUT_NOTES, quantization=quantization,
                    **metadata)
        manifest.write_text(json.dumps(meta, indent=1), encoding="utf-8")
    return {k: v for k, v in meta.items() if k != "layout"}


def read_manifest(path) -> dict:
    path = Path(path)
    return json.loads(path.with_name(path.name + ".json").read_text(encoding="utf-8"))


def _file_sha256(path: Path) -> str:
    sha = hashlib.sha256()
    with open(path, "rb", buffering=0) as f:
        block = bytearray(1 << 24)
        while True:
            got = f.readinto(block)
            if not got:
                return sha.hexdigest()
            sha.update(memoryview(block)[:got])


def mapped_pack(path, source: str | None = None, verify: bool = False):
    """The pack at `path` mapped without reading it: (uint8 [blocks, bytes per block], layout, manifest). The map is
    copy-on-write, so nothing done to the tensor reaches the file. Raises ValueError for another format or source,
    a file whose size is not the manifest's, or (verify) a sha256 mismatch."""
    path = Path(path)
    meta = read_manifest(path)
    problems = []
    if meta.get("format") not in FORMATS:
        problems.append(f"format {meta.get('format')!r} is not one of {FORMATS}")
    if source is not None and meta.get("source") != source:
        problems.append(f"made from {meta.get('source')!r}, not {source!r}")
    rows, size = meta["blocks"], meta["bytes_per_block"]
    if path.stat().st_size != rows * size:
        problems.append(f"{path.stat().st_size} bytes on disk, {rows * size} in the manifest (incomplete)")
    if not problems and verify and _file_sha256(path) != meta["sha256"]:
        problems.append("sha256 differs from the manifest")
    if problems:
        raise ValueError(f"weight pack {path}: " + "; ".join(problems))
    table = np.memmap(path, dtype=np.uint8, mode="c", shape=(rows, size))
    return torch.from_numpy(table), meta["layout"], meta


def slot(row: torch.Tensor, layout: list, device=None) -> dict:
    """The parts dict of one row of a pack (copies on `device`), as QuantizedWanBlock takes it."""
    inv_layers = {v: k for k, v in LAYERS.items()}
    inv_others = {v: k for k, v in OTHERS.items()}
    types = {v: k for k, v in DTYPES.items()}
    parts = {k: {} for k in LAYERS}
    for e in layout:
        raw = row[e["offset"]:e["offset"] + e["bytes"]].clone()
        t = raw.view(types[e["dtype"]]).reshape(e["shape"])
        t = t.to(device) if device is not None else t
        name = e["name"]
        layer, _, part = name.rpartition(".")
        if layer in inv_layers and (part in PARTS or part in FP8_PARTS):
            parts[inv_layers[layer]][part] = t
        elif name in inv_others:
            parts[inv_others[name]] = t
        else:
            raise ValueError(f"unknown pack entry {name}")
    return parts


def load_blocks(path, heads: int, device, source: str | None = None, verify: bool = False) -> list:
    """The QuantizedWanBlocks of the pack at `path` on `device` (each expands its weight codes once)."""
    from wdl.block import QuantizedWanBlock

    rows, layout, _ = mapped_pack(path, source, verify)
    blocks = []
    for i in range(rows.shape[0]):
        parts = slot(rows[i], layout, device)
        blocks.append(QuantizedWanBlock(parts, parts["modulation"].shape[1], heads))
    return blocks
