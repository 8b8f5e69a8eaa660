"""Real-checkpoint path: Qwen3 safetensors shards into a TpBatchRunner.

Mirrors the reference's weight admission (crates/ferric-build/src/
safetensors.rs): a shard is an 8-byte little-endian header length, a JSON
header of {name: {dtype, shape, data_offsets}} (plus an optional
"__metadata__"), then the tensor bytes. Every tensor must be BF16
(safetensors.rs:642), its byte range must match its shape (:674-690) and lie
inside the shard, no tensor may appear twice across shards, and an unknown
tensor name is an error. Names follow the Hugging Face Qwen3 layout the
reference admits (model_layout.rs:605-615: "model.embed_tokens.weight",
"model.layers.{l}.self_attn.q_proj.weight", ...), and shapes the admitted
schema (crates/ferric-spec/src/qwen3.rs:70-230). Shards may be pinned by
SHA-256 like the reference's shard pins (safetensors.rs:20-63); the digest
is checked before any tensor is uploaded.

Tensors are memory-mapped and uploaded one by one through fh_upload_weight
(row-major [N][K] bf16; the library re-lays projections into MFMA tile order
on the device). With a tied embedding (Qwen3-0.6B) there is no lm_head.
"""

from __future__ import annotations

import hashlib
import json
import os
import re
import struct
from dataclasses import dataclass
from typing import Iterable, Mapping, Optional

import numpy as np

from . import _lib

_GLOBAL = {
    "model.embed_tokens.weight": _lib.TOKEN_EMBEDDING,
    "model.norm.weight": _lib.FINAL_NORM,
    "lm_head.weight": _lib.LANGUAGE_MODEL_HEAD,
}
_LAYER = {
    "input_layernorm.weight": _lib.INPUT_LAYER_NORM,
    "post_attention_layernorm.weight": _lib.POST_ATTENTION_LAYER_NORM,
    "self_attn.q_norm.weight": _lib.QUERY_NORM,
    "self_attn.k_norm.weight": _lib.KEY_NORM,
    "self_attn.q_proj.weight": _lib.QUERY_PROJECTION,
    "self_attn.k_proj.weight": _lib.KEY_PROJECTION,
    "self_attn.v_proj.weight": _lib.VALUE_PROJECTION,
    "self_attn.o_proj.weight": _lib.OUTPUT_PROJECTION,
    "mlp.gate_proj.weight": _lib.GATE_PROJECTION,
    "mlp.up_proj.weight": _lib.UP_PROJECTION,
    "mlp.down_proj.weight": _lib.DOWN_PROJECTION,
}
_LAYER_RE = re.compile(r"^model\.layers\.(\d+)\.(.+)$")
NO_LAYER = 0


class CheckpointError(ValueError):
    """A shard or tensor failed admission; nothing after the failing check was uploaded."""


@dataclass(frozen=True)
class TensorEntry:
    name: str
    kind: int
    layer: int
    shape: tuple
    path: str
    offset: int  # absolute byte offset of the tensor data in the shard
    nbytes: int


def tensor_coordinate(name: str, layers: int):
    """(kind, layer) of a Hugging Face Qwen3 tensor name; CheckpointError if unknown."""
    if name in _GLOBAL:
        return _GLOBAL[name], NO_LAYER
    m = _LAYER_RE.match(name)
    if m and m.group(2) in _LAYER:
        layer = int(m.group(1))
        if layer >= layers or str(layer) != m.group(1):
            raise CheckpointError(f"tensor {name!r}: layer outside the model")
        return _LAYER[m.group(2)], layer
    raise CheckpointError(f"unexpected tensor {name!r}")


def expected_shape(cfg: Mapping, kind: int) -> tuple:
    """Row-major shape of a tensor kind for a model description (qwen3.rs:70-230)."""
    h, qh, kvh, i, v = cfg["hidden"], cfg["query_heads"], cfg["kv_heads"], cfg["intermediate"], cfg["vocabulary"]
    d = cfg.get("head_dim", 128)
    return {
        _lib.LANGUAGE_MODEL_HEAD: (v, h),
        _lib.TOKEN_EMBEDDING: (v, h),
        _lib.FINAL_NORM: (h,),
        _lib.INPUT_LAYER_NORM: (h,),
        _lib.POST_ATTENTION_LAYER_NORM: (h,),
        _lib.QUERY_NORM: (d,),
        _lib.KEY_NORM: (d,),
        _lib.QUERY_PROJECTION: (qh * d, h),
        _lib.KEY_PROJECTION: (kvh * d, h),
        _lib.VALUE_PROJECTION: (kvh * d, h),
        _lib.OUTPUT_PROJECTION: (h, qh * d),
        _lib.GATE_PROJECTION: (i, h),
        _lib.UP_PROJECTION: (i, h),
        _lib.DOWN_PROJECTION: (h, i),
    }[kind]


def required_tensors(cfg: Mapping) -> set:
    """Every (kind, layer) a checkpoint of this model must hold."""
    need = {(_lib.TOKEN_EMBEDDING, NO_LAYER), (_lib.FINAL_NORM, NO_LAYER)}
    if not cfg["tied_embedding"]:
        need.add((_lib.LANGUAGE_MODEL_HEAD, NO_LAYER))
    for layer in range(cfg["layers"]):
        need.update((kind, layer) for kind in _LAYER.values())
    return need


def read_header(path: str) -> tuple:
    """(header dict, data section offset) of one shard."""
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise CheckpointError(f"{path}: truncated header length")
        (n,) = struct.unpack("<Q", raw)
        if n == 0 or 8 + n > size or n > 100 << 20:
            raise CheckpointError(f"{path}: header length {n} does not fit the file")
        text = f.read(n)
    try:
        header = json.loads(text.decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise CheckpointError(f"{path}: header is not JSON ({e})") from None
    if not isinstance(header, dict):
        raise CheckpointError(f"{path}: header is not an object")
    return header, 8 + n


def check_offset_coverage(path: str, ranges: list, data_bytes: int) -> None:
    """The tensors of one shard, sorted by start offset, must tile its data
    section exactly: no gap, no overlap, no trailing bytes (the reference's
    validate_offset_coverage, crates/ferric-build/src/safetensors.rs:626-627,
    762-790; header order itself is free)."""
    expected = 0
    for start, end, name in sorted(ranges):
        if start > expected:
            raise CheckpointError(f"{path}: offset gap before tensor {name!r} (expected {expected}, got {start})")
        if start < expected:
            raise CheckpointError(f"{path}: tensor {name!r} overlaps the previous one (expected {expected}, "
                                  f"got {start})")
        expected = end
    if expected != data_bytes:
        raise CheckpointError(f"{path}: tensors cover {expected} data bytes of {data_bytes} (trailing bytes)")


def index_shards(cfg: Mapping, paths: Iterable[str]) -> list:
    """Parses and checks every shard header; returns the tensors to upload."""
    entries, seen = [], {}
    for path in paths:
        header, data0 = read_header(path)
        size = os.path.getsize(path)
        ranges = []
        for name, spec in header.items():
            if name == "__metadata__":
                continue
            if name in seen:
                raise CheckpointError(f"tensor {name!r} appears in {seen[name]} and {path}")
            seen[name] = path
            if not isinstance(spec, dict) or spec.get("dtype") != "BF16":
                raise CheckpointError(f"tensor {name!r} is not BF16")
            kind, layer = tensor_coordinate(name, cfg["layers"])
            if kind == _lib.LANGUAGE_MODEL_HEAD and cfg["tied_embedding"]:
                raise CheckpointError("lm_head.weight present for a tied-embedding model")
            shape = tuple(int(x) for x in spec.get("shape", ()))
            if shape != expected_shape(cfg, kind):
                raise CheckpointError(f"tensor {name!r} has shape {shape}, expected {expected_shape(cfg, kind)}")
            offs = spec.get("data_offsets")
            if not (isinstance(offs, list) and len(offs) == 2 and all(isinstance(o, int) for o in offs)):
                raise CheckpointError(f"tensor {name!r}: malformed data_offsets")
            start, end = offs
            nbytes = 2 * int(np.prod(shape))
            if start < 0 or end - start != nbytes or data0 + end > size:
                raise CheckpointError(f"tensor {name!r}: byte range does not match its shape")
            ranges.append((start, end, name))
            entries.append(TensorEntry(name, kind, layer, shape, path, data0 + start, nbytes))
        check_offset_coverage(path, ranges, size - data0)
    have = {(e.kind, e.layer) for e in entries}
    missing = required_tensors(cfg) - have
    if missing:
        names = sorted(f"kind {k} layer {l}" for k, l in missing)
        raise CheckpointError(f"checkpoint is missing {len(missing)} tensors: {', '.join(names[:6])}")
    return entries


def file_sha256(path: str, chunk: int = 64 << 20) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            b = f.read(chunk)
            if not b:
                return h.hexdigest()
            h.update(b)


def load_safetensors(runner, paths: Iterable[str], sha256: Optional[Mapping[str, str]] = None) -> dict:
    """Admits the shards and uploads every tensor into `runner` (a TpBatchRunner, or
    anything with .model and .upload_weight(kind, layer, uint16 array)).

    sha256: optional {shard file name: hex digest}; every listed shard must match
    and every shard must be listed. Returns {"tensors": n, "bytes": total}."""
    paths = [str(p) for p in paths]
    cfg = runner.model
    if sha256 is not None:
        for p in paths:
            want = sha256.get(os.path.basename(p))
            if want is None:
                raise CheckpointError(f"shard {os.path.basename(p)!r} is not pinned")
            got = file_sha256(p)
            if got != want.lower():
                raise CheckpointError(f"shard {os.path.basename(p)!r} has SHA-256 {got}, expected {want}")
    entries = index_shards(cfg, paths)
    total = 0
    maps = {p: np.memmap(p, dtype=np.uint8, mode="r") for p in paths}
    for e in entries:
        raw = maps[e.path][e.offset:e.offset + e.nbytes]
        runner.upload_weight(e.kind, e.layer, raw.view("<u2"))
        total += e.nbytes
    del maps
    return {"tensors": len(entries), "bytes": total}


def write_safetensors(path: str, tensors: Mapping[str, np.ndarray], metadata: Optional[Mapping[str, str]] = None):
    """Writes bf16 tensors (uint16 arrays, row-major) as one safetensors shard."""
    header, offset, order = {}, 0, []
    if metadata:
        header["__metadata__"] = dict(metadata)
    for name, arr in tensors.items():
        arr = np.ascontiguousarray(arr, dtype=np.uint16)
        header[name] = {"dtype": "BF16", "shape": list(arr.shape), "data_offsets": [offset, offset + arr.nbytes]}
        offset += arr.nbytes
        order.append(arr)
    text = json.dumps(header, separators=(",", ":")).encode("utf-8")
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for arr in order:
            f.write(arr.astype("<u2", copy=False).tobytes())
