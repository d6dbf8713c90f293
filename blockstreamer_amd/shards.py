"""Block shards whose MXFP4 expert weights are stored in the k-pair layout.

The format is the reference's (block_streamer/shards.py:44-200): one flat
file per streamed block holding its tensors back to back in sorted name
order, and a JSON manifest (``manifest.json``) listing each tensor's name,
dtype, shape, byte offset and byte count, so a staging buffer of the block's
bytes is turned into tensors by views alone (shards.py:57-60).  Two things
differ, for the k-pair kernels of this package:

* every tensor starts on a 16-byte boundary (the reference pads to 8,
  shards.py:164-165): the k-pair kernels move packed blocks in 16-byte
  pieces, and a staged view of an 8-byte aligned tensor would be refused;
* each expert ``*_proj_blocks`` tensor (uint8 ``[E, R, G, 16]`` with
  R % 16 == 0 and G even) is stored in the k-pair layout
  ``[E, R/16, G/2, 16, 2, 16]``: group g of row r at ``[e][r/16][g/2][r%16]
  [g%2]``.  The scales keep the checkpoint layout.

Both are recorded in a versioned top-level manifest field, ``LAYOUT_FIELD``:
``{"version": 1, "alignment": 16, "layouts": {"<block index>": {"<tensor
name>": "kpair"}}}``.  The reference's loader reads only the ``blocks``,
``resident`` and ``resident_filename`` keys (shards.py:102-124), so it still
reads such a manifest; a staged k-pair tensor then has the 6-D shape the
kernels recognise (``kernels.blocks_layout``).  ``load_manifest`` here checks
the field: an unknown version, a tagged tensor whose shape is not the k-pair
shape or a tensor off its alignment is refused.
"""

from __future__ import annotations

import json
from collections.abc import Iterator
from pathlib import Path

import torch
from torch import Tensor

MANIFEST_NAME = "manifest.json"
LAYOUT_FIELD = "blockstreamer_amd"
LAYOUT_VERSION = 1
ALIGN = 16
KPAIR = "kpair"

# dtype names of the reference's manifest (shards.py:22-33)
DTYPES: dict[str, torch.dtype] = {
    "float32": torch.float32,
    "float16": torch.float16,
    "bfloat16": torch.bfloat16,
    "float64": torch.float64,
    "uint8": torch.uint8,
    "int8": torch.int8,
    "int32": torch.int32,
    "int64": torch.int64,
    "bool": torch.bool,
}
_DTYPE_NAMES = {v: k for k, v in DTYPES.items()}


def kpair_pack(blocks: Tensor) -> Tensor:
    """Checkpoint-layout blocks ``[E, R, G, 16]`` in the k-pair layout
    ``[E, R/16, G/2, 16, 2, 16]`` (a copy; any device).  The GPU repack
    kernel (``kernels.to_kpair``) gives the same bytes."""
    if blocks.dim() != 4 or blocks.shape[-1] != 16 or blocks.dtype != torch.uint8:
        raise ValueError(f"expected uint8 blocks [E, R, G, 16], got {blocks.dtype} {tuple(blocks.shape)}")
    E, R, G, _ = blocks.shape
    if R % 16 or G % 2:
        raise ValueError(f"the k-pair layout needs R % 16 == 0 and an even G (R={R}, G={G})")
    return blocks.reshape(E, R // 16, 16, G // 2, 2, 16).permute(0, 1, 3, 2, 4, 5).contiguous()


def kpair_unpack(blocks: Tensor) -> Tensor:
    """The inverse of ``kpair_pack``."""
    if blocks.dim() != 6 or tuple(blocks.shape[3:]) != (16, 2, 16):
        raise ValueError(f"expected k-pair blocks [E, R/16, G/2, 16, 2, 16], got {tuple(blocks.shape)}")
    E, bands, pairs = blocks.shape[:3]
    return blocks.permute(0, 1, 3, 2, 4, 5).reshape(E, bands * 16, pairs * 2, 16).contiguous()


def _wants_kpair(name: str, t: Tensor) -> bool:
    return (name.endswith("_proj_blocks") and t.dtype == torch.uint8 and t.dim() == 4 and t.shape[-1] == 16
            and t.shape[1] % 16 == 0 and t.shape[2] % 2 == 0)


def plan_block(index: int, named: list[tuple[str, Tensor]], align: int = ALIGN) -> tuple[dict, int]:
    """Tensors back to back in the given order, each starting on an
    ``align``-byte boundary: the block's manifest entry and its byte count
    (block_streamer/shards.py:148-165 with a wider alignment)."""
    specs, offset = [], 0
    for name, t in named:
        if t.dtype not in _DTYPE_NAMES:
            raise ValueError(f"unsupported shard dtype {t.dtype} for {name}")
        nbytes = t.numel() * t.element_size()
        specs.append({"name": name, "dtype": _DTYPE_NAMES[t.dtype], "shape": list(t.shape), "offset": offset,
                      "nbytes": nbytes})
        offset += nbytes
        offset += -offset % align
    return {"index": index, "filename": f"block_{index:05d}.bin", "nbytes": offset, "tensors": specs}, offset


def write_block(path: Path, spec: dict, named: dict[str, Tensor]) -> None:
    """One contiguous shard file; the padding between tensors is zero."""
    buf = torch.zeros(spec["nbytes"], dtype=torch.uint8)
    for ts in spec["tensors"]:
        flat = named[ts["name"]].detach().contiguous().cpu().view(torch.uint8).reshape(-1)
        buf[ts["offset"]:ts["offset"] + ts["nbytes"]].copy_(flat)
    path.write_bytes(buf.numpy().tobytes())


def convert_modules(blocks: Iterator[tuple[int, dict[str, Tensor]]], out_dir: str | Path,
                    kpair: bool = True) -> dict:
    """Write one shard per ``(index, state)`` and the manifest
    (block_streamer/shards.py:178-200), the expert blocks in the k-pair
    layout when ``kpair`` (those whose shape allows it), every tensor
    16-byte aligned.  Consumes the iterator lazily, one block in memory at a
    time.  Returns the manifest as written."""
    root = Path(out_dir)
    root.mkdir(parents=True, exist_ok=True)
    entries, layouts = [], {}
    for index, state in blocks:
        state = dict(state)
        tagged = {}
        for name, t in list(state.items()):
            if kpair and _wants_kpair(name, t):
                state[name] = kpair_pack(t.detach().cpu())
                tagged[name] = KPAIR
        spec, _ = plan_block(index, sorted(state.items()))
        write_block(root / spec["filename"], spec, state)
        entries.append(spec)
        if tagged:
            layouts[str(index)] = tagged
    manifest = {
        "blocks": entries,
        "resident": [],
        "resident_filename": "resident.bin",
        LAYOUT_FIELD: {"version": LAYOUT_VERSION, "alignment": ALIGN, "layouts": layouts},
    }
    (root / MANIFEST_NAME).write_text(json.dumps(manifest, indent=1))
    return manifest


def load_manifest(root: str | Path) -> dict:
    """The manifest of a shard directory, with its layout field checked: a
    version newer than this reader's, a tensor tagged "kpair" whose shape is
    not ``[E, R/16, G/2, 16, 2, 16]``, or (with the field present) a tensor
    offset off the recorded alignment raises ``ValueError``.  A manifest
    without the field (the reference's own) is returned as is: its tensors
    are in the checkpoint layout, 8-byte aligned."""
    m = json.loads((Path(root) / MANIFEST_NAME).read_text())
    field = m.get(LAYOUT_FIELD)
    if field is None:
        return m
    if int(field.get("version", 0)) != LAYOUT_VERSION:
        raise ValueError(f"shard layout field version {field.get('version')} (this reader knows {LAYOUT_VERSION})")
    align = int(field.get("alignment", ALIGN))
    for b in m["blocks"]:
        tags = field.get("layouts", {}).get(str(b["index"]), {})
        names = {t["name"] for t in b["tensors"]}
        for name, layout in tags.items():
            if layout != KPAIR or name not in names:
                raise ValueError(f"block {b['index']}: unknown layout {layout!r} for {name!r}")
        for t in b["tensors"]:
            if t["offset"] % align:
                raise ValueError(f"block {b['index']}: {t['name']} at offset {t['offset']}, not {align}-aligned")
            if tags.get(t["name"]) == KPAIR and (len(t["shape"]) != 6 or t["shape"][3:] != [16, 2, 16]):
                raise ValueError(f"block {b['index']}: {t['name']} is tagged k-pair but has shape {t['shape']}")
    return m


def block_layouts(manifest: dict, index: int) -> dict[str, str]:
    """``{tensor name: layout}`` of the tagged tensors of block ``index``."""
    return dict(manifest.get(LAYOUT_FIELD, {}).get("layouts", {}).get(str(index), {}))


def read_block(root: str | Path, block: dict, out: Tensor) -> None:
    """A block's bytes into a flat uint8 host buffer (shards.py:126-140)."""
    if out.numel() < block["nbytes"]:
        raise ValueError(f"staging buffer holds {out.numel()} bytes; block {block['index']} needs {block['nbytes']}")
    with open(Path(root) / block["filename"], "rb", buffering=0) as fh:
        got = fh.readinto(memoryview(out[:block["nbytes"]].numpy()))
    if got != block["nbytes"]:
        raise OSError(f"short read on block {block['index']}: {got} of {block['nbytes']} bytes")


def materialize(block: dict, buffer: Tensor) -> dict[str, Tensor]:
    """Views of a staged block's tensors in a flat uint8 buffer (host or
    device), as the reference's ``TensorSpec.view`` makes them
    (shards.py:57-60)."""
    out = {}
    for t in block["tensors"]:
        window = buffer[t["offset"]:t["offset"] + t["nbytes"]]
        out[t["name"]] = window.view(DTYPES[t["dtype"]]).view(t["shape"])
    return out
