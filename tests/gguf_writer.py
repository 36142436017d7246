"""A GGUF v3 writer for tests: metadata and tensors laid out as the format
specifies (header, metadata, tensor table, data section aligned to
general.alignment), so the C++ reader (include/kraken/gguf.hpp) can be checked
on files whose every byte the test chose."""
import struct

import numpy as np

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}
GGML_F32, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 0, 12, 13, 14


def _string(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind, value):
    if kind == STRING:
        return _string(value)
    return struct.pack(_SCALAR[kind], value)


def metadata_entry(key, kind, value, array_kind=None):
    out = _string(key) + struct.pack("<I", kind)
    if kind == ARRAY:
        out += struct.pack("<IQ", array_kind, len(value))
        out += b"".join(_value(array_kind, v) for v in value)
    else:
        out += _value(kind, value)
    return out


def write(path, metadata, tensors, alignment=32, version=3):
    """metadata: list of (key, kind, value[, array_kind]).  tensors: list of
    (name, shape innermost-first, ggml type, bytes).  Returns the absolute
    offset of every tensor's data."""
    head = struct.pack("<IIQQ", MAGIC, version, len(tensors), len(metadata))
    head += b"".join(metadata_entry(*m) for m in metadata)
    blobs = [np.ascontiguousarray(data).tobytes() for _, _, _, data in tensors]
    table, offsets, cursor = b"", [], 0
    for (name, shape, ggml_type, _), blob in zip(tensors, blobs):
        cursor = -(-cursor // alignment) * alignment
        offsets.append(cursor)
        table += _string(name) + struct.pack("<I", len(shape))
        table += b"".join(struct.pack("<Q", d) for d in shape)
        table += struct.pack("<IQ", ggml_type, cursor)
        cursor += len(blob)
    tables = head + table
    data_start = -(-len(tables) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(tables)
        f.write(b"\0" * (data_start - len(tables)))
        pos = 0
        for blob, off in zip(blobs, offsets):
            f.write(b"\0" * (off - pos))
            f.write(blob)
            pos = off + len(blob)
    return [data_start + o for o in offsets]
