"""Safetensors admission (CPU): shard parsing, the reference's rejection
classes (crates/ferric-build/src/safetensors.rs:128-160: non-BF16 tensor,
shape/byte-range mismatch, duplicate tensor, unknown tensor, shard pin
mismatch) and a bit-exact upload stream into a recording runner."""

import json
import struct

import numpy as np
import pytest

from ferric_amd import _lib
from ferric_amd.checkpoint import (CheckpointError, expected_shape, file_sha256, load_safetensors,
                                   required_tensors, write_safetensors)

TINY = dict(layers=2, hidden=256, query_heads=8, kv_heads=8, head_dim=128, intermediate=512, vocabulary=384,
            tied_embedding=0, rope_theta=1_000_000, rms_epsilon=1e-6)

_GLOBAL_NAMES = {_lib.TOKEN_EMBEDDING: "model.embed_tokens.weight", _lib.FINAL_NORM: "model.norm.weight",
                 _lib.LANGUAGE_MODEL_HEAD: "lm_head.weight"}
_LAYER_NAMES = {_lib.INPUT_LAYER_NORM: "input_layernorm.weight",
                _lib.POST_ATTENTION_LAYER_NORM: "post_attention_layernorm.weight",
                _lib.QUERY_NORM: "self_attn.q_norm.weight", _lib.KEY_NORM: "self_attn.k_norm.weight",
                _lib.QUERY_PROJECTION: "self_attn.q_proj.weight", _lib.KEY_PROJECTION: "self_attn.k_proj.weight",
                _lib.VALUE_PROJECTION: "self_attn.v_proj.weight", _lib.OUTPUT_PROJECTION: "self_attn.o_proj.weight",
                _lib.GATE_PROJECTION: "mlp.gate_proj.weight", _lib.UP_PROJECTION: "mlp.up_proj.weight",
                _lib.DOWN_PROJECTION: "mlp.down_proj.weight"}


def tensor_name(kind, layer):
    return _GLOBAL_NAMES[kind] if kind in _GLOBAL_NAMES else f"model.layers.{layer}.{_LAYER_NAMES[kind]}"


def make_tensors(cfg, seed=5):
    r = np.random.default_rng(seed)
    return {tensor_name(k, l): r.integers(0, 1 << 16, expected_shape(cfg, k), dtype=np.uint16)
            for k, l in sorted(required_tensors(cfg))}


class Recorder:
    def __init__(self, cfg):
        self.model = cfg
        self.uploads = {}

    def upload_weight(self, kind, layer, data):
        assert data.dtype == np.uint16
        self.uploads[(kind, layer)] = np.array(data)


def write_two_shards(tmp_path, tensors):
    names = list(tensors)
    a, b = tmp_path / "model-00001-of-00002.safetensors", tmp_path / "model-00002-of-00002.safetensors"
    write_safetensors(str(a), {n: tensors[n] for n in names[::2]}, {"format": "pt"})
    write_safetensors(str(b), {n: tensors[n] for n in names[1::2]})
    return [str(a), str(b)]


def test_two_shards_upload_every_tensor_bit_exact(tmp_path):
    tensors = make_tensors(TINY)
    paths = write_two_shards(tmp_path, tensors)
    rec = Recorder(TINY)
    pins = {p.split("/")[-1]: file_sha256(p) for p in paths}
    info = load_safetensors(rec, paths, sha256=pins)
    assert info["tensors"] == len(tensors) == 3 + 11 * TINY["layers"]
    for (kind, layer), got in rec.uploads.items():
        assert np.array_equal(got, tensors[tensor_name(kind, layer)].reshape(-1))


def test_tied_embedding_has_no_head(tmp_path):
    cfg = dict(TINY, tied_embedding=1)
    tensors = make_tensors(cfg)
    assert "lm_head.weight" not in tensors
    rec = Recorder(cfg)
    load_safetensors(rec, write_two_shards(tmp_path, tensors))
    assert (_lib.LANGUAGE_MODEL_HEAD, 0) not in rec.uploads
    extra = dict(tensors, **{"lm_head.weight": np.zeros((384, 256), np.uint16)})
    with pytest.raises(CheckpointError, match="tied"):
        load_safetensors(Recorder(cfg), write_two_shards(tmp_path, extra))


def _raw_shard(path, header, payload=b""):
    text = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + payload)


@pytest.mark.parametrize("case,match", [
    ("dtype", "not BF16"),
    ("shape", "shape"),
    ("offsets", "byte range"),
    ("past_end", "byte range"),
    ("unknown", "unexpected tensor"),
    ("layer", "layer outside"),
    ("missing", "missing"),
])
def test_rejections(tmp_path, case, match):
    tensors = make_tensors(TINY)
    paths = write_two_shards(tmp_path, tensors)
    header_len = struct.unpack("<Q", open(paths[0], "rb").read(8))[0]
    header = json.loads(open(paths[0], "rb").read(8 + header_len)[8:])
    payload = open(paths[0], "rb").read()[8 + header_len:]
    name = "model.embed_tokens.weight" if "model.embed_tokens.weight" in header else next(
        n for n in header if n != "__metadata__")
    if case == "dtype":
        header[name]["dtype"] = "F16"
    elif case == "shape":
        header[name]["shape"] = list(reversed(header[name]["shape"])) + [1]
    elif case == "offsets":
        header[name]["data_offsets"][1] -= 2
    elif case == "past_end":
        payload = payload[:-2]
    elif case == "unknown":
        header["model.rotary_emb.inv_freq"] = dict(header[name])
    elif case == "layer":
        header["model.layers.2.input_layernorm.weight"] = dict(header[name])
    elif case == "missing":
        del header[name]
    _raw_shard(paths[0], header, payload)
    with pytest.raises(CheckpointError, match=match):
        load_safetensors(Recorder(TINY), paths)


def _read_shard(path):
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    return json.loads(raw[8:8 + n]), raw[8 + n:]


def _by_start(header):
    return sorted((n for n in header if n != "__metadata__"), key=lambda n: header[n]["data_offsets"][0])


@pytest.mark.parametrize("case,match", [
    ("gap", "offset gap"),
    ("overlap", "overlaps"),
    ("trailing", "trailing"),
])
def test_offset_coverage_rejections(tmp_path, case, match):
    # The reference's gaps_overlaps_invalid_ranges_and_reordering_are_rejected
    # (crates/ferric-build/src/safetensors.rs:1305): the first tensor moved two
    # bytes on (a gap at the start), the second tensor moved two bytes back (an
    # overlap with the first), and two bytes past the last tensor.
    paths = write_two_shards(tmp_path, make_tensors(TINY))
    header, payload = _read_shard(paths[0])
    first, second = _by_start(header)[:2]
    if case == "gap":
        header[first]["data_offsets"] = [o + 2 for o in header[first]["data_offsets"]]
    elif case == "overlap":
        header[second]["data_offsets"] = [o - 2 for o in header[second]["data_offsets"]]
    else:
        payload = payload + b"\0\0"
    _raw_shard(paths[0], header, payload)
    with pytest.raises(CheckpointError, match=match):
        load_safetensors(Recorder(TINY), paths)


def test_header_order_is_free(tmp_path):
    # Coverage is checked over the tensors sorted by offset, so a header that
    # lists them in another order admits the same bytes.
    tensors = make_tensors(TINY)
    paths = write_two_shards(tmp_path, tensors)
    header, payload = _read_shard(paths[0])
    _raw_shard(paths[0], dict(reversed(list(header.items()))), payload)
    rec = Recorder(TINY)
    load_safetensors(rec, paths)
    for (kind, layer), got in rec.uploads.items():
        assert np.array_equal(got, tensors[tensor_name(kind, layer)].reshape(-1))


def test_duplicate_tensor_across_shards(tmp_path):
    tensors = make_tensors(TINY)
    paths = write_two_shards(tmp_path, tensors)
    dup = tmp_path / "extra.safetensors"
    write_safetensors(str(dup), {"model.norm.weight": tensors["model.norm.weight"]})
    with pytest.raises(CheckpointError, match="appears in"):
        load_safetensors(Recorder(TINY), paths + [str(dup)])


def test_shard_pins(tmp_path):
    paths = write_two_shards(tmp_path, make_tensors(TINY))
    pins = {p.split("/")[-1]: file_sha256(p) for p in paths}
    bad = dict(pins)
    bad[paths[1].split("/")[-1]] = "0" * 64
    rec = Recorder(TINY)
    with pytest.raises(CheckpointError, match="SHA-256"):
        load_safetensors(rec, paths, sha256=bad)
    assert rec.uploads == {}  # nothing uploaded before the pins pass
    with pytest.raises(CheckpointError, match="not pinned"):
        load_safetensors(rec, paths, sha256={paths[0].split("/")[-1]: pins[paths[0].split("/")[-1]]})


def test_truncated_header(tmp_path):
    p = tmp_path / "bad.safetensors"
    p.write_bytes(struct.pack("<Q", 1 << 20) + b"{}")
    with pytest.raises(CheckpointError, match="header length"):
        load_safetensors(Recorder(TINY), [str(p)])
