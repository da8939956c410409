"""Minimal GGUF v3 writer for the loader tests (test infrastructure).

Writes the header, metadata key/values and tensor infos in the layout
gguf.rs:213-262 parses, then the tensor data aligned to 32 bytes.  Values
are given as (type, value) pairs using the GGUF metadata type ids.
"""
import struct

T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STRING, T_ARRAY, T_U64, T_I64, T_F64 = range(13)
_FMT = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
        T_BOOL: "<B", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(ty, v) -> bytes:
    if ty == T_STRING:
        return _str(v)
    if ty == T_ARRAY:
        elem, items = v
        out = struct.pack("<IQ", elem, len(items))
        return out + b"".join(_value(elem, x) for x in items)
    return struct.pack(_FMT[ty], v)


def write_gguf(path, kv, tensors, version=3, align=32, pad_between=True):
    """kv: list of (key, type, value); tensors: list of (name, ggml_dims,
    ggml_type, data bytes).  Tensor data is laid out in order, each padded
    to `align`."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, len(tensors), len(kv))
    for key, ty, v in kv:
        out += _str(key) + struct.pack("<I", ty) + _value(ty, v)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off += len(data)
        if pad_between:
            off = -(-off // align) * align
    for (name, dims, gtype, _), o in zip(tensors, offsets):
        out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", gtype, o)
    out += b"\0" * ((-len(out)) % align)
    base = len(out)
    for (_, _, _, data), o in zip(tensors, offsets):
        out += b"\0" * (base + o - len(out))
        out += data
    with open(path, "wb") as f:
        f.write(bytes(out))
