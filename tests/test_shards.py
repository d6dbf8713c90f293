"""The k-pair shard writer and reader (CPU): the reference's shard format
(block_streamer/shards.py:44-200) with 16-byte tensor alignment, the expert
blocks in the k-pair layout, and a versioned layout field in the manifest.

What must hold for the reference's own loader to still read these manifests
(shards.py:102-124 reads the "blocks", "resident" and "resident_filename"
keys and passes each tensor entry to ``TensorSpec(**entry)``): the tensor
entries carry exactly the keys name, dtype, shape, offset, nbytes, and the
layout tag lives in a top-level key of its own.
"""

from __future__ import annotations

import json

import pytest
import torch

import oracle
from blockstreamer_amd import shards, synthetic

EXPERTS = ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
           "down_proj_blocks", "down_proj_scales", "down_proj_bias")


def _block_state(seed: int) -> dict[str, torch.Tensor]:
    t = synthetic.moe_layer(synthetic.TINY, seed=seed, scale_lo=119, scale_hi=129)
    state = {f"mlp.experts.{n}": t[n] for n in EXPERTS}
    state["mlp.router.weight"] = t["router_weight"]
    state["mlp.router.bias"] = t["router_bias"]
    state["post_attention_layernorm.weight"] = torch.randn(256)
    state["odd"] = torch.arange(5, dtype=torch.uint8)   # 5 bytes: the next tensor must be re-aligned
    return state


def _write(tmp_path, kpair=True):
    states = {0: _block_state(1), 1: _block_state(2)}
    manifest = shards.convert_modules(iter(states.items()), tmp_path, kpair=kpair)
    return states, manifest


def test_manifest_keeps_the_reference_schema_and_aligns_to_16(tmp_path):
    _, manifest = _write(tmp_path)
    on_disk = json.loads((tmp_path / shards.MANIFEST_NAME).read_text())
    assert on_disk == json.loads(json.dumps(manifest))
    assert set(on_disk) == {"blocks", "resident", "resident_filename", shards.LAYOUT_FIELD}
    for b in on_disk["blocks"]:
        assert set(b) == {"index", "filename", "nbytes", "tensors"}
        names = [t["name"] for t in b["tensors"]]
        assert names == sorted(names)                         # sorted name order, as the reference writes
        end = 0
        for t in b["tensors"]:
            assert set(t) == {"name", "dtype", "shape", "offset", "nbytes"}
            assert t["offset"] % 16 == 0 and t["offset"] >= end
            end = t["offset"] + t["nbytes"]
        assert b["nbytes"] == end + (-end % 16)
        assert (tmp_path / b["filename"]).stat().st_size == b["nbytes"]
    field = on_disk[shards.LAYOUT_FIELD]
    assert field["version"] == shards.LAYOUT_VERSION and field["alignment"] == 16
    assert field["layouts"] == {str(i): {"mlp.experts.gate_up_proj_blocks": "kpair",
                                         "mlp.experts.down_proj_blocks": "kpair"} for i in (0, 1)}


def test_round_trip_through_a_staging_buffer(tmp_path):
    states, _ = _write(tmp_path)
    m = shards.load_manifest(tmp_path)
    for b in m["blocks"]:
        buf = torch.empty(b["nbytes"], dtype=torch.uint8)
        shards.read_block(tmp_path, b, buf)
        views = shards.materialize(b, buf)
        tags = shards.block_layouts(m, b["index"])
        for name, want in states[b["index"]].items():
            got = views[name]
            if tags.get(name) == shards.KPAIR:
                assert got.shape == (8, want.shape[1] // 16, want.shape[2] // 2, 16, 2, 16)
                assert torch.equal(got, oracle.to_kpair_ref(want))   # the layout's definition
                assert torch.equal(shards.kpair_unpack(got), want)
            else:
                assert got.dtype == want.dtype and torch.equal(got, want)


def test_without_kpair_the_blocks_keep_the_checkpoint_layout(tmp_path):
    states, manifest = _write(tmp_path, kpair=False)
    assert manifest[shards.LAYOUT_FIELD]["layouts"] == {}
    b = shards.load_manifest(tmp_path)["blocks"][0]
    buf = torch.empty(b["nbytes"], dtype=torch.uint8)
    shards.read_block(tmp_path, b, buf)
    views = shards.materialize(b, buf)
    assert torch.equal(views["mlp.experts.gate_up_proj_blocks"], states[0]["mlp.experts.gate_up_proj_blocks"])


def test_pack_matches_the_layout_definition_and_refuses_bad_shapes():
    blocks = torch.randint(0, 256, (3, 48, 6, 16), dtype=torch.uint8, generator=torch.Generator().manual_seed(5))
    packed = shards.kpair_pack(blocks)
    assert torch.equal(packed, oracle.to_kpair_ref(blocks))
    # element by element: group g of row r of expert e at [e][r/16][g/2][r%16][g%2]
    for e, r, g in [(0, 0, 0), (1, 17, 3), (2, 47, 5)]:
        assert torch.equal(packed[e, r // 16, g // 2, r % 16, g % 2], blocks[e, r, g])
    with pytest.raises(ValueError, match="R % 16"):
        shards.kpair_pack(torch.zeros(1, 40, 4, 16, dtype=torch.uint8))
    with pytest.raises(ValueError, match="even G"):
        shards.kpair_pack(torch.zeros(1, 32, 3, 16, dtype=torch.uint8))


def _tamper(tmp_path, fn):
    p = tmp_path / shards.MANIFEST_NAME
    m = json.loads(p.read_text())
    fn(m)
    p.write_text(json.dumps(m))


def test_reader_refuses_unknown_versions_and_inconsistent_tags(tmp_path):
    _write(tmp_path)
    _tamper(tmp_path, lambda m: m[shards.LAYOUT_FIELD].update(version=2))
    with pytest.raises(ValueError, match="version"):
        shards.load_manifest(tmp_path)
    _write(tmp_path)

    def flatten_shape(m):
        for t in m["blocks"][0]["tensors"]:
            if t["name"] == "mlp.experts.gate_up_proj_blocks":
                t["shape"] = [8, 512, 8, 16]
    _tamper(tmp_path, flatten_shape)
    with pytest.raises(ValueError, match="tagged k-pair"):
        shards.load_manifest(tmp_path)
    _write(tmp_path)

    def misalign(m):
        m["blocks"][1]["tensors"][-1]["offset"] += 8
    _tamper(tmp_path, misalign)
    with pytest.raises(ValueError, match="aligned"):
        shards.load_manifest(tmp_path)


def test_a_reference_manifest_without_the_field_loads_unchanged(tmp_path):
    """No layout field: the reference's own shards (checkpoint layout,
    8-byte alignment) read as they are."""
    _write(tmp_path, kpair=False)
    _tamper(tmp_path, lambda m: m.pop(shards.LAYOUT_FIELD))
    m = shards.load_manifest(tmp_path)
    assert shards.LAYOUT_FIELD not in m and shards.block_layouts(m, 0) == {}
