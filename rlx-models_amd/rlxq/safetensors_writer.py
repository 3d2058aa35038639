"""Writes safetensors files and MLX checkpoint directories (synthetic
checkpoints for the MLX loader's tests), from the published safetensors
layout: u64 little-endian header length n, n bytes of JSON
{name: {"dtype", "shape", "data_offsets": [begin, end]}, "__metadata__": {..}},
then the data (offsets relative to its start).  The library itself only
reads these files (rlxq_mlx_*)."""
from __future__ import annotations

import json
import struct

import numpy as np

# numpy dtype -> safetensors dtype name
_DT = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16", np.dtype(np.uint32): "U32",
       np.dtype(np.uint8): "U8", np.dtype(np.int8): "I8", np.dtype(np.int32): "I32",
       np.dtype(np.int64): "I64", np.dtype(np.float64): "F64", np.dtype(np.uint16): "U16"}


def safetensors_bytes(tensors: dict, metadata: dict | None = None, *, bf16: tuple = ()) -> bytes:
    """tensors: {name: numpy array}; names listed in `bf16` hold uint16 bf16
    bit patterns and are written with dtype BF16."""
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, arr in tensors.items():
        a = np.ascontiguousarray(arr)
        dt = "BF16" if name in bf16 else _DT[a.dtype]
        b = a.tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    return struct.pack("<Q", len(h)) + h + b"".join(blobs)


def write_safetensors(path, tensors: dict, metadata: dict | None = None, **kw) -> None:
    with open(path, "wb") as f:
        f.write(safetensors_bytes(tensors, metadata, **kw))


def write_mlx_dir(d, shards: list, quantization: dict | None, *, index: bool = False, **kw) -> None:
    """An mlx-community style directory: config.json (with `quantization` when
    given) and the shards [{name: array}] as model-0000i-of-0000n.safetensors
    (with model.safetensors.index.json when index=True), or model.safetensors
    for one shard."""
    from pathlib import Path

    d = Path(d)
    d.mkdir(parents=True, exist_ok=True)
    cfg = {"model_type": "qwen3"}
    if quantization is not None:
        cfg["quantization"] = quantization
    (d / "config.json").write_text(json.dumps(cfg))
    names = ["model.safetensors"] if len(shards) == 1 and not index else \
        [f"model-{i + 1:05d}-of-{len(shards):05d}.safetensors" for i in range(len(shards))]
    weight_map = {}
    for fn, tensors in zip(names, shards):
        write_safetensors(d / fn, tensors, {"format": "mlx"}, **kw)
        weight_map.update({t: fn for t in tensors})
    if index:
        (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
