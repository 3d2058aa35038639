"""Writes GGUF files (synthetic checkpoints for the reader's tests and the
upload benchmark), from the published GGUF layout (version 2/3,
little-endian):

    u32 magic "GGUF", u32 version, u64 tensor_count, u64 kv_count,
    kv_count x {string key, u32 value_type, value},
    tensor_count x {string name, u32 n_dims, u64 dims[n_dims] (innermost
                    first), u32 ggml_type, u64 offset from the data start},
    padding to general.alignment (default 32), tensor data.

Strings are u64 length + UTF-8 bytes; an array is u32 element type, u64 count
and the elements.  The library itself only reads GGUF (rlxq_gguf_*).
"""
import struct

VALUE_TYPES = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7, "str": 8,
               "arr": 9, "u64": 10, "i64": 11, "f64": 12}
_FMT = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}

# ggml type ids used by the tests
F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q6_K, Q5_K, BF16 = 0, 1, 2, 3, 8, 12, 14, 13, 30
Q2_K, Q3_K, Q8_K = 10, 11, 15


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    return _str(v) if t == 8 else struct.pack("<" + _FMT[t], v)


def gguf_bytes(meta, tensors, *, version: int = 3, alignment=None, magic: bytes = b"GGUF") -> tuple[bytes, dict]:
    """meta: [(key, type name, value)], an array value being (element type
    name, [values]); tensors: [(name, ggml type, dims innermost first, data
    bytes)].  Returns the file and {tensor name: absolute data offset}."""
    kv = list(meta)
    if alignment is not None:
        kv.append(("general.alignment", "u32", alignment))
    out = bytearray(magic) + struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, tn, v in kv:
        out += _str(key) + struct.pack("<I", VALUE_TYPES[tn])
        if tn == "arr":
            et, vals = v
            out += struct.pack("<IQ", VALUE_TYPES[et], len(vals)) + b"".join(_value(VALUE_TYPES[et], x) for x in vals)
        else:
            out += _value(VALUE_TYPES[tn], v)
    a = alignment or 32
    rel, offs = 0, []
    for _, _, _, data in tensors:
        offs.append(rel)
        rel = (rel + len(data) + a - 1) // a * a
    for (name, gt, dims, _), o in zip(tensors, offs):
        out += _str(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        out += struct.pack("<IQ", gt, o)
    start = (len(out) + a - 1) // a * a
    out += bytes(start - len(out))
    for (_, _, _, data), o in zip(tensors, offs):
        out += bytes(start + o - len(out)) + bytes(data)
    return bytes(out), {t[0]: start + o for t, o in zip(tensors, offs)}


def write_gguf(path, meta, tensors, **kw) -> dict:
    data, offsets = gguf_bytes(meta, tensors, **kw)
    with open(path, "wb") as f:
        f.write(data)
    return offsets
