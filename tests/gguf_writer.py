"""GGUF v2/v3 writer for the reader's tests (test infrastructure), written
from the published format description: little-endian; u32 magic 'GGUF', u32
version, u64 tensor count, u64 metadata count; metadata entries (string key,
u32 value type, value; strings are u64 length + bytes; arrays are u32
element type + u64 count + elements); tensor entries (string name, u32
n_dims, u64 dims, u32 ggml type, u64 data offset); padding to
general.alignment (default 32); tensor data, each tensor starting at an
aligned offset."""
import struct

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
        BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


def gguf_string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def gguf_value(t: int, v) -> bytes:
    if t == STRING:
        return gguf_string(v)
    if t == ARRAY:
        et, vals = v
        return struct.pack("<IQ", et, len(vals)) + b"".join(gguf_value(et, x) for x in vals)
    return struct.pack(_FMT[t], v)


def gguf_bytes(kvs, tensors, alignment=None, version=3, offsets=None) -> bytes:
    """kvs: [(key, type, value)]; tensors: [(name, ggml type, ne list, data
    bytes)].  offsets overrides the tensor data offsets (for malformed files)."""
    kvs = list(kvs)
    if alignment is not None:
        kvs.append(("general.alignment", UINT32, alignment))
    align = alignment or 32
    out = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for key, t, v in kvs:
        out += gguf_string(key) + struct.pack("<I", t) + gguf_value(t, v)
    offs, pos = [], 0
    for _, _, _, data in tensors:
        offs.append(pos)
        pos += len(data)
        pos += (align - pos % align) % align
    if offsets is not None:
        offs = offsets
    for (name, gt, ne, _), off in zip(tensors, offs):
        out += gguf_string(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
        out += struct.pack("<IQ", gt, off)
    out += b"\0" * ((align - len(out) % align) % align)
    base = len(out)
    for (_, _, _, data), off in zip(tensors, offs):
        if base + off > len(out):
            out += b"\0" * (base + off - len(out))
        out = out[:base + off] + data + out[base + off + len(data):]
    return out


def write_gguf(path, kvs, tensors, alignment=None, version=3, offsets=None):
    with open(path, "wb") as f:
        f.write(gguf_bytes(kvs, tensors, alignment, version, offsets))
